"""CPU: the packed-sequence layout (sgsa_amd.varlen) that cu_seqlens calls go
through -- the padded batch it builds, its inverse, its gradients, the pads the
state update gets and the argument checks."""

import pytest
import torch

from sgsa_amd import varlen


def test_layout_round_trip_and_mask():
    cu = torch.tensor([0, 3, 3, 10, 12], dtype=torch.int32)   # lengths 3, 0, 7, 2
    x = torch.arange(12 * 2, dtype=torch.float64).view(1, 12, 2)
    lay = varlen.layout(cu, x)
    assert (lay.n, lay.max_len) == (4, 7)
    p = lay.pad(x, fill=-1.0)
    assert p.shape == (4, 7, 2)
    for n, (a, b) in enumerate([(0, 3), (3, 3), (3, 10), (10, 12)]):
        L = b - a
        assert torch.equal(p[n, :L], x[0, a:b])
        assert bool((p[n, L:] == -1.0).all())
        assert lay.mask[n, :L].all() and not lay.mask[n, L:].any()
    assert torch.equal(lay.unpad(p), x)
    rows = torch.randn(4, 3, 7, 5)   # [N,H,L,*]
    back = lay.unpad_rows(rows)
    assert back.shape == (1, 3, 12, 5)
    assert torch.equal(back[0, :, 3:10], rows[2, :, :7])


def test_layout_is_differentiable():
    cu = torch.tensor([0, 4, 9], dtype=torch.int64)
    x = torch.randn(1, 9, 3, dtype=torch.float64, requires_grad=True)
    lay = varlen.layout(cu, x)
    assert torch.autograd.gradcheck(lambda t: lay.unpad(lay.pad(t) * 2.0 + 1.0), (x,))


def test_state_inputs_pads_leave_the_state_alone():
    cu = torch.tensor([0, 2, 5], dtype=torch.int32)
    B, T, H, D = 1, 5, 2, 4
    q, k, v = (torch.randn(B, T, H, D) for _ in range(3))
    beta, gamma, alpha = torch.rand(B, T, H), torch.rand(B, T, H), torch.rand(B, T, H)
    lay = varlen.layout(cu, q)
    pq, pk, pv, pb, pg, psk, psv, pa = varlen.pad_state_inputs(lay, q, k, v, beta, gamma, k, v, alpha)
    pad = ~lay.mask
    assert bool((pb[pad] == 0).all()) and bool((pa[pad] == 0).all()) and bool((pg[pad] == 1).all())
    assert bool((pk[pad] == 0).all()) and bool((psv[pad] == 0).all())
    assert torch.equal(pg[lay.mask], gamma[0])


@pytest.mark.parametrize("cu,err", [([0, 3, 2], "not decrease"), ([1, 5], "start at 0"), ([0, 4], "end at"),
                                    ([0], "N\\+1")])
def test_layout_rejects_bad_offsets(cu, err):
    x = torch.zeros(1, 5, 2)
    with pytest.raises(ValueError, match=err):
        varlen.layout(torch.tensor(cu, dtype=torch.int32), x)


def test_layout_rejects_batches_and_float_offsets():
    with pytest.raises(ValueError, match="batch size must be 1"):
        varlen.layout(torch.tensor([0, 2]), torch.zeros(2, 2, 3))
    with pytest.raises(ValueError, match="int32 or int64"):
        varlen.layout(torch.tensor([0.0, 2.0]), torch.zeros(1, 2, 3))
    lay = varlen.layout(torch.tensor([0, 1, 2]), torch.zeros(1, 2, 3))
    with pytest.raises(ValueError, match="one state per sequence"):
        varlen.check_states(lay, torch.zeros(3, 1, 4, 4))
