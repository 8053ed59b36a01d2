"""CPU checks of the backward's recompute (sgsa_amd/backward.py).

chunk_sgsa_torch is the differentiable torch form of what the HIP forward
computes; the op backwards differentiate it (the reference's recompute
semantics, modelings/sgsa_ops/chunk_bwd.py:31-77).  Pinned three ways:

* its forward equals the token recurrence of the oracle (naive.py:34-57) in
  float64 -- with and without the sparse write, with an initial state, ragged T,
  several chunk sizes, and decays whose chunk prefix falls far below 1e-6;
* its gradients equal torch autograd through that oracle recurrence, a
  different algorithm (token loop instead of chunk solve), in float64;
* torch.autograd.gradcheck: finite differences against the analytic gradient.

The shapes follow the reference's own core tests (tests/test_sgsa_core.py:11-22:
B=2, T=9, H=3, D=5, chunk 4).
"""

import pytest
import torch

from oracle import sgsa_oracle as O
from sgsa_amd.backward import chunk_sgsa_torch, recompute_grads


def _inputs(B=2, T=9, H=3, D=5, seed=0, gamma_scale=None, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    x = dict(q=r(B, T, H, D), k=r(B, T, H, D), v=r(B, T, H, D),
             beta=torch.sigmoid(r(B, T, H)), gamma=torch.sigmoid(r(B, T, H)),
             sparse_k=r(B, T, H, D), sparse_v=r(B, T, H, D), alpha=0.25 * torch.sigmoid(r(B, T, H)),
             initial_state=0.3 * r(B, H, D, D))
    if gamma_scale is not None:   # chunk-local prefixes far below 1e-6
        x["gamma"] = gamma_scale * (1.0 + torch.rand(B, T, H, generator=g, dtype=dtype))
    return x


ORDER = ["q", "k", "v", "beta", "gamma", "sparse_k", "sparse_v", "alpha", "initial_state"]


def _select(x, sparse, init):
    y = dict(x)
    if not sparse:
        y["sparse_k"] = y["sparse_v"] = y["alpha"] = None
    if not init:
        y["initial_state"] = None
    return y


@pytest.mark.parametrize("sparse", [False, True])
@pytest.mark.parametrize("init", [False, True])
@pytest.mark.parametrize("chunk", [1, 4, 64])
def test_recompute_forward_equals_recurrence(sparse, init, chunk):
    x = _select(_inputs(), sparse, init)
    o, s = chunk_sgsa_torch(**x, chunk_size=chunk)
    o_ref, s_ref = O.naive_recurrent_sgsa(**x, output_final_state=True)
    torch.testing.assert_close(o, o_ref, atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(s, s_ref, atol=1e-10, rtol=1e-10)


def test_recompute_forward_tiny_decay_and_ragged():
    # gamma ~ 1e-3: a chunk prefix reaches 1e-12; T = 11 is ragged for chunk 4
    x = _inputs(T=11, gamma_scale=1e-3)
    o, s = chunk_sgsa_torch(**x, chunk_size=4)
    o_ref, s_ref = O.naive_recurrent_sgsa(**x, output_final_state=True)
    torch.testing.assert_close(o, o_ref, atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(s, s_ref, atol=1e-10, rtol=1e-10)


def test_recompute_forward_empty_sequence():
    x = _inputs(T=0)
    o, s = chunk_sgsa_torch(**x, chunk_size=4)
    assert o.shape == (2, 0, 3, 5)
    torch.testing.assert_close(s, x["initial_state"])


@pytest.mark.parametrize("sparse", [False, True])
@pytest.mark.parametrize("init", [False, True])
@pytest.mark.parametrize("with_dht", [False, True])
def test_recompute_grads_equal_recurrence_autograd(sparse, init, with_dht):
    x = _select(_inputs(T=10, seed=3), sparse, init)
    g = torch.Generator().manual_seed(7)
    do = torch.randn(2, 10, 3, 5, generator=g, dtype=torch.float64)
    dht = torch.randn(2, 3, 5, 5, generator=g, dtype=torch.float64) if with_dht else None
    inputs = [x[n] for n in ORDER]
    needs = [t is not None for t in inputs]
    got = recompute_grads(inputs, needs, do, dht)

    leaves = {n: (None if x[n] is None else x[n].clone().requires_grad_(True)) for n in ORDER}
    o, s = O.naive_recurrent_sgsa(**leaves, output_final_state=True)
    obj = (o * do).sum() + ((s * dht).sum() if dht is not None else 0.0)
    live = [n for n in ORDER if leaves[n] is not None]
    ref = dict(zip(live, torch.autograd.grad(obj, [leaves[n] for n in live])))
    for n, gr in zip(ORDER, got):
        if x[n] is None:
            assert gr is None, n
        else:
            torch.testing.assert_close(gr, ref[n], atol=1e-9, rtol=1e-9, msg=lambda m: f"{n}: {m}")


def test_recompute_grads_respects_needs_and_dtype():
    x = _inputs()
    inputs = [x[n].float() for n in ORDER]
    needs = [True, False, False, True, False, False, False, True, False]
    do = torch.ones(2, 9, 3, 5)
    got = recompute_grads(inputs, needs, do, None)
    for n, gr, need in zip(ORDER, got, needs):
        assert (gr is not None) == need, n
        if gr is not None:
            assert gr.dtype == torch.float32 and gr.shape == x[n].shape and torch.isfinite(gr).all()


def test_recompute_gradcheck():
    x = _inputs(B=1, T=6, H=2, D=3, seed=5)
    args = tuple(x[n].clone().requires_grad_(True) for n in ORDER)

    def f(*a):
        o, s = chunk_sgsa_torch(*a, chunk_size=4)
        return o, s

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6, rtol=1e-5)
