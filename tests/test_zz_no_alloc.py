"""GPU: sgsa_score_topk_noalloc (no workspace argument, no device allocation; its
scratch is a fixed per-GPU array) returns exactly what sgsa_score_topk returns
given sgsa_score_topk_fast_workspace_size() bytes of workspace, through the C ABI.

Two calls in a row on one GPU, the second with a smaller input (the scratch keeps
the first call's contents), for the decode-shaped few-row form and for the row
kernel (more query rows than the few-row form takes); then a request beyond the
scratch is refused with SGSA_ERR_WORKSPACE.
"""

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)
from sgsa_amd import _abi  # noqa: E402


def _inputs(B, Tq, Tk, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Tq, H, D, generator=g)
    k = torch.randn(B, Tk, H, D, generator=g)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    return q.to("cuda", dtype).contiguous(), k.to("cuda", dtype).contiguous()


def _outputs(B, Tq, H, kk, dev):
    return (torch.full((B, H, Tq, kk), -7, device=dev, dtype=torch.int32),
            torch.full((B, H, Tq, kk), 7.0, device=dev, dtype=torch.float32),
            torch.full((B, H, Tq, 2), 7.0, device=dev, dtype=torch.float32),
            torch.full((B, H, Tq), -7, device=dev, dtype=torch.int32),
            torch.full((B, H, Tq), -7, device=dev, dtype=torch.int32))


def _both(q, k, top_k, q_offset, sorted_):
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    kk = min(top_k, Tk)
    dev = q.device
    L = _abi.lib()
    dt = _abi.dtype_code(q.dtype)
    scale = math.sqrt(D)
    st = _abi.stream_of(q)
    P = _abi.ptr
    n = ctypes.c_size_t()
    _abi.check(L.sgsa_score_topk_fast_workspace_size(dt, B, Tq, Tk, H, D, ctypes.byref(n)))
    ws = torch.empty(n.value, device=dev, dtype=torch.uint8)
    ref = _outputs(B, Tq, H, kk, dev)
    got = _outputs(B, Tq, H, kk, dev)
    split_r = None if sorted_ else ref[4]
    split_g = None if sorted_ else got[4]
    _abi.check(L.sgsa_score_topk(dt, B, Tq, Tk, H, D, kk, 1, q_offset, scale, 0, P(q), P(k), P(ref[0]), P(ref[1]),
                                 P(ref[2]), P(ref[3]), P(split_r), int(sorted_), P(ws), n.value, st))
    _abi.check(L.sgsa_score_topk_noalloc(dt, B, Tq, Tk, H, D, kk, 1, q_offset, scale, 0, P(q), P(k), P(got[0]),
                                         P(got[1]), P(got[2]), P(got[3]), P(split_g), int(sorted_), st))
    torch.cuda.synchronize()
    for name, a, b in zip(("indices", "scores", "top2", "counts", "split"), got, ref):
        assert torch.equal(a, b), f"{name} differs from sgsa_score_topk (B={B} Tq={Tq} Tk={Tk} H={H} k={kk})"
    assert (ref[3] > 0).all()


@pytest.mark.parametrize("sorted_", [0, 1])
def test_noalloc_decode_shape_then_smaller(dev, sorted_):
    # few-row form: one query row per (b, h) at the end of the cache
    q, k = _inputs(8, 1, 16640, 16, 128, torch.bfloat16, 1)
    print("noalloc decode B=8 Tq=1 Tk=16640 H=16 k=2048", flush=True)
    _both(q, k, 2048, 16639, sorted_)
    q, k = _inputs(2, 1, 3000, 16, 128, torch.bfloat16, 2)
    print("noalloc decode B=2 Tq=1 Tk=3000 H=16 k=256", flush=True)
    _both(q, k, 256, 2999, sorted_)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_row_kernel_then_smaller(dev, dtype):
    # more rows per (b, h) than the few-row form takes: the row kernel on the scratch
    q, k = _inputs(1, 1024, 1024, 4, 64, dtype, 3)
    print(f"noalloc rows B=1 T=1024 H=4 D=64 k=64 {dtype}", flush=True)
    _both(q, k, 64, 0, 0)
    q, k = _inputs(1, 300, 300, 2, 64, dtype, 4)
    print(f"noalloc rows B=1 T=300 H=2 D=64 k=32 {dtype}", flush=True)
    _both(q, k, 32, 0, 0)


def test_noalloc_refuses_beyond_its_scratch(dev):
    # 16 heads x 8192 rows need 512 MiB of candidate lists: refused before any launch.  The
    # operands are real device buffers of the stated shape, so a guard that stopped refusing
    # would show as a wrong status, not as a kernel reading a bogus address.
    L = _abi.lib()
    B, T, H, D, kk = 1, 8192, 16, 128, 256
    q, k = _inputs(B, T, T, H, D, torch.bfloat16, 5)
    idx = torch.zeros(B, H, T, kk, device=dev, dtype=torch.int32)
    sc = torch.zeros(B, H, T, kk, device=dev, dtype=torch.float32)
    top2 = torch.zeros(B, H, T, 2, device=dev, dtype=torch.float32)
    cnt = torch.zeros(B, H, T, device=dev, dtype=torch.int32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    s = L.sgsa_score_topk_noalloc(1, B, T, T, H, D, kk, 1, 0, 11.3, 0, P(q), P(k), P(idx), P(sc), P(top2), P(cnt),
                                  None, 0, st)
    torch.cuda.synchronize()
    assert s == 4 and b"SGSA_NOALLOC_SCRATCH_BYTES" in L.sgsa_last_error()
    assert not cnt.any(), "a refused call wrote its outputs"
