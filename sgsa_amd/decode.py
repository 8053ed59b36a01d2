"""One SGSA decode step: the new token's retrieval over the KV cache, its write
key and gate, and the recurrent state update -- the token-by-token form of
SGSABlock.forward's attention half (modelings/modeling_sgsa.py:669-684) with
the recurrent backend (:570-582).

The caller appends the new token's key and value to the cache first; the
token sits at cache position Tc - 1 and retrieves over keys [0, Tc - 1]
(causal).  Three C-ABI calls on the current stream: sgsa_score_topk (one
query row, q_offset = Tc - 1), sgsa_sparse_gather (weights, k_hat / write
key, v_hat, alpha) and sgsa_recurrent_fwd (T = 1).

Top-k reuse (modelings/idea.md:395-401; config 4 recomputes every 4 decode
steps): a step given ``candidates`` -- the (indices, counts) an earlier step
returned -- skips the selection and re-scores those keys for the new query
(sgsa_score_at); the weights, gate and update then follow as usual, with the
row maximum and top-2 taken over the re-scored set.  Keys appended since the
candidates were selected are not among them.
"""

from __future__ import annotations

import ctypes
import functools
import math
from typing import Optional, Tuple

import torch

from . import _abi
from .recurrent import fused_recurrent_sgsa, recurrent_sgsa_fwd

Tensor = torch.Tensor

_WRITE_MODES = {"direct": 0, "residual": 1}


@functools.lru_cache(maxsize=256)
def _workspace_size(fn: str, *args: int) -> int:
    """Bytes from one of the library's workspace-size queries; they depend on the shapes only."""
    n = ctypes.c_size_t()
    _abi.check(getattr(_abi.lib(), fn)(*args, ctypes.byref(n)))
    return n.value


def sgsa_decode_step(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    q_ret: Tensor,
    beta: Tensor,
    gamma: Tensor,
    budget_logits: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    state: Tensor,
    top_k: int,
    write_mode: str = "direct",
    alpha_max: float = 0.25,
    tau_c: float = 0.1,
    candidates: Optional[Tuple[Tensor, Tensor]] = None,
    return_candidates: bool = False,
    length: Optional[int] = None,
):
    """q, k, v, q_ret [B,1,H,D]; beta, gamma, budget_logits [B,1,H];
    k_cache, v_cache [B,Tc,H,D] (ending with this token); state [B,H,D,D] fp32.
    candidates: (indices int32 [B,H,1,n], counts int32 [B,H,1]) to re-score
    instead of selecting (top-k reuse); indices must be < Tc.  length: the
    number of valid cache positions when k_cache / v_cache are a preallocated
    buffer longer than that (the token then sits at length - 1); the kernels
    address the buffer in place.

    Returns (o [B,1,H,D] in q.dtype, new state [B,H,D,D] fp32), and the step's
    candidates (selected or reused) as a third item when return_candidates.
    """
    if not q.is_cuda:
        raise ValueError("sgsa_decode_step: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, one, H, D = q.shape
    if one != 1:
        raise ValueError(f"sgsa_decode_step takes one token per sequence, got T={one}")
    Tbuf = k_cache.shape[1]
    if k_cache.shape != (B, Tbuf, H, D) or v_cache.shape != (B, Tbuf, H, D):
        raise ValueError("k_cache / v_cache must be [B, Tc, H, D] like q")
    Tc = Tbuf if length is None else int(length)
    if not 1 <= Tc <= Tbuf:
        raise ValueError(f"length={length} must be in [1, {Tbuf}]")
    if write_mode not in _WRITE_MODES:
        raise ValueError(f"write_mode must be one of {sorted(_WRITE_MODES)}")
    dt = q.dtype
    dev = q.device
    rc, kn = (t.to(dt).contiguous() for t in (q_ret, k))
    # a contiguous cache of q's dtype is addressed in place (rows >= Tc are never read: the
    # selection is causal and the indices are < Tc); anything else is copied first
    kc, vc = (t if (t.dtype == dt and t.is_contiguous()) else t.to(dt).contiguous() for t in (k_cache, v_cache))
    L = _abi.lib()
    if candidates is None:
        # 1. top-k of the new query over the cache (causal: position Tc - 1)
        kk = min(int(top_k), Tc)
        idx = torch.empty(B, H, 1, kk, device=dev, dtype=torch.int32)
        sc = torch.empty(B, H, 1, kk, device=dev, dtype=torch.float32)
        top2 = torch.empty(B, H, 1, 2, device=dev, dtype=torch.float32)
        cnt = torch.empty(B, H, 1, device=dev, dtype=torch.int32)
        nb = _workspace_size("sgsa_score_topk_fast_workspace_size", _abi.dtype_code(dt), B, 1, Tbuf, H, D)
        tws = torch.empty(nb, device=dev, dtype=torch.uint8)
        _abi.check(L.sgsa_score_topk(_abi.dtype_code(dt), B, 1, Tbuf, H, D, kk, 1, Tc - 1, math.sqrt(D), 0,
                                     _abi.ptr(rc), _abi.ptr(kc), _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(top2),
                                     _abi.ptr(cnt), None, 0, _abi.ptr(tws), nb, _abi.stream_of(rc)))
    else:
        # 1'. the reused candidates, re-scored for the new query; the gather tracks
        # the row maximum and top-2 itself (top2 = NULL)
        idx, cnt = candidates
        if idx.dim() != 4 or idx.shape[:3] != (B, H, 1) or idx.dtype != torch.int32 or cnt.shape != (B, H, 1) \
                or cnt.dtype != torch.int32:
            raise ValueError("candidates must be (int32 [B,H,1,n], int32 [B,H,1]) from an earlier step")
        idx, cnt = idx.contiguous(), cnt.contiguous()
        kk = idx.shape[-1]
        sc = torch.empty(B, H, 1, kk, device=dev, dtype=torch.float32)
        top2 = None
        _abi.check(L.sgsa_score_at(_abi.dtype_code(dt), B, 1, Tbuf, H, D, kk, math.sqrt(D), 0, _abi.ptr(rc),
                                   _abi.ptr(kc), _abi.ptr(idx), _abi.ptr(cnt), _abi.ptr(sc), _abi.stream_of(rc)))
    # 2. weights, k_hat / write key, v_hat and the gate for that row
    mode = _WRITE_MODES[write_mode]
    wk = torch.empty(B, 1, H, D, device=dev, dtype=dt)
    vh = torch.empty_like(wk)
    al = torch.empty(B, 1, H, device=dev, dtype=torch.float32)
    bud = budget_logits.float().contiguous()
    gn = _workspace_size("sgsa_sparse_gather_workspace_size", B, 1, H, D, kk)
    gws = torch.empty(gn, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_sparse_gather(
        _abi.dtype_code(dt), B, 1, Tbuf, H, D, kk, Tc - 1, _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(kn), _abi.ptr(idx),
        _abi.ptr(sc), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(bud), mode, float(alpha_max), float(tau_c), 64, 8,
        _abi.ptr(wk if mode == 0 else None), _abi.ptr(vh), _abi.ptr(wk if mode == 1 else None), _abi.ptr(al),
        None, None, _abi.ptr(gws), gn, _abi.stream_of(kc)))
    # 3. the recurrent update for this token (without autograd, the forward itself: the autograd
    # Function's dispatch costs more host time than the kernel)
    rec = fused_recurrent_sgsa if torch.is_grad_enabled() else recurrent_sgsa_fwd
    o, st = rec(q, k, v, beta, gamma, wk, vh, al, state, output_final_state=True)
    return (o, st, (idx, cnt)) if return_candidates else (o, st)
