"""GPU: the split-row form of sgsa_sparse_gather (decode shapes: few rows, many
slots; each row's slots go to several waves whose partial sums are merged in a
fixed order) against the one-wave-per-row form of the same call, through the C
ABI.  Both forms compute the same sums in a different order: outputs agree
within 2e-5 (fp32) / 1e-2 (bf16 outputs), the weights and diagnostics within
1e-5, and each form is bitwise repeatable.
"""

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)
from sgsa_amd import _abi  # noqa: E402
from sgsa_amd.retrieval import score_topk  # noqa: E402


def _gather(dt, k, v, kn, idx, sc, top2, cnt, bud, Tc, split, mode):
    B, Tbuf, H, D = k.shape
    kk = idx.shape[-1]
    L = _abi.lib()
    dev = k.device
    if split:
        n = ctypes.c_size_t()
        _abi.check(L.sgsa_sparse_gather_workspace_size(B, 1, H, D, kk, ctypes.byref(n)))
        assert n.value > 256, "the split form must be available at this shape"
        nb = n.value
    else:
        nb = 256
    ws = torch.empty(nb, device=dev, dtype=torch.uint8)
    wk = torch.empty(B, 1, H, D, device=dev, dtype=dt)
    vh = torch.empty_like(wk)
    al = torch.empty(B, 1, H, device=dev)
    w = torch.empty(B, H, 1, kk, device=dev)
    dg = torch.empty(_abi.NDIAG, B, H, 1, device=dev)
    _abi.check(L.sgsa_sparse_gather(
        _abi.dtype_code(dt), B, 1, Tbuf, H, D, kk, Tc - 1, _abi.ptr(k), _abi.ptr(v), _abi.ptr(kn), _abi.ptr(idx),
        _abi.ptr(sc), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(bud), mode, 0.25, 0.1, 64, 8,
        _abi.ptr(wk if mode == 0 else None), _abi.ptr(vh), _abi.ptr(wk if mode == 1 else None), _abi.ptr(al),
        _abi.ptr(w), _abi.ptr(dg), _abi.ptr(ws), nb, _abi.stream_of(k)))
    torch.cuda.synchronize()
    return dict(wk=wk.float(), vh=vh.float(), al=al, w=w, dg=dg)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("online", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
def test_split_gather_matches_row_gather(dev, dt, online, mode):
    B, H, D, Tc, top_k = 2, 8, 128, 3000, 1000   # 16 rows, 8 partials of 128 slots each
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(B, Tc, H, D, device=dev, generator=g).to(dt)
    v = torch.randn(B, Tc, H, D, device=dev, generator=g).to(dt)
    q = torch.randn(B, 1, H, D, device=dev, generator=g).to(dt)
    kn = torch.randn(B, 1, H, D, device=dev, generator=g).to(dt)
    bud = torch.randn(B, 1, H, device=dev, generator=g)
    idx, sc, top2, cnt = score_topk(q, k, top_k, causal=True, q_offset=Tc - 1, sorted=False)
    if online:
        top2 = None
    a = _gather(dt, k, v, kn, idx, sc, top2, cnt, bud, Tc, False, mode)
    b = _gather(dt, k, v, kn, idx, sc, top2, cnt, bud, Tc, True, mode)
    b2 = _gather(dt, k, v, kn, idx, sc, top2, cnt, bud, Tc, True, mode)
    for name in b:
        assert torch.equal(b[name], b2[name]), f"{name}: split form not repeatable"
    tol = 2e-5 if dt == torch.float32 else 1e-2
    for name in ("wk", "vh"):
        torch.testing.assert_close(b[name], a[name], atol=tol, rtol=tol, msg=name)
    torch.testing.assert_close(b["al"], a["al"], atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(b["w"], a["w"], atol=1e-6, rtol=1e-4)
    torch.testing.assert_close(b["dg"], a["dg"], atol=1e-5, rtol=1e-4)
    assert math.isfinite(float(b["dg"].abs().max()))
