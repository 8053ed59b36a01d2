"""Token top-k sparse retrieval on gfx950 (SparseRetriever, token_only mode).

``sparse_retrieve`` returns the dict of SparseRetriever.forward
(modelings/modeling_sgsa.py:407-474) computed by two HIP kernels: the score
GEMM + exact top-k (sgsa_score_topk) and the gather + weights + diagnostics
(sgsa_sparse_gather).  Indices are int64 as in the reference (:152); weights
are returned in the input dtype (:126-128); ties in the top-k are broken by
the lowest key index.
"""

from __future__ import annotations

import ctypes
import math
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import _abi

Tensor = torch.Tensor


def score_topk(q: Tensor, k: Tensor, top_k: int, causal: bool = True, q_offset: int = 0,
               scale: Optional[float] = None, scale_mode: int = 0, sorted: bool = True,
               return_split: bool = False, fast: bool = True):
    """Exact top-k over causal scores without materialising them.

    q [B,Tq,H,D], k [B,Tk,H,D].  Returns (indices int32 [B,H,Tq,kk],
    scores float32 [B,H,Tq,kk], top2 float32 [B,H,Tq,2], counts int32 [B,H,Tq])
    with kk = min(top_k, Tk); with ``return_split`` (unsorted output only) also
    the length of each row's first ascending run.  ``fast`` passes the workspace
    of sgsa_score_topk_fast_workspace_size, which lets decode-shaped calls (few
    query rows per head) use the few-row form; ``fast=False`` keeps the row kernel.
    """
    if not q.is_cuda:
        raise ValueError("score_topk: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    if k.shape != (B, Tk, H, D) or k.dtype != q.dtype:
        raise ValueError(f"k shape/dtype {tuple(k.shape)}/{k.dtype} does not match q {tuple(q.shape)}/{q.dtype}")
    kk = min(int(top_k), Tk)
    if scale is None:
        scale = math.sqrt(D) if scale_mode == 0 else 1.0 / math.sqrt(D)
    qc, kc = q.contiguous(), k.contiguous()
    dev = q.device
    idx = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.int32)
    sc = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.float32)
    top2 = torch.empty(B, H, Tq, 2, device=dev, dtype=torch.float32)
    cnt = torch.empty(B, H, Tq, device=dev, dtype=torch.int32)
    spl = torch.empty(B, H, Tq, device=dev, dtype=torch.int32) if return_split else None
    L = _abi.lib()
    nbytes = ctypes.c_size_t()
    if fast:
        _abi.check(L.sgsa_score_topk_fast_workspace_size(_abi.dtype_code(q.dtype), B, Tq, Tk, H, D,
                                                         ctypes.byref(nbytes)))
    else:
        _abi.check(L.sgsa_score_topk_workspace_size(B, Tq, H, ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_score_topk(
        _abi.dtype_code(q.dtype), B, Tq, Tk, H, D, kk, int(causal), int(q_offset), float(scale), int(scale_mode),
        _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(spl),
        int(sorted), _abi.ptr(ws), nbytes.value, _abi.stream_of(qc)))
    if return_split:
        return idx, sc, top2, cnt, spl
    return idx, sc, top2, cnt


def _mask_bytes(mask: Optional[Tensor], shape, name: str) -> Optional[Tensor]:
    if mask is None:
        return None
    if tuple(mask.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(mask.shape)}, expected {tuple(shape)}")
    return mask.to(torch.bool).to(torch.uint8).contiguous()


def score_topk_masked(q: Tensor, k: Tensor, top_k: int, key_mask: Optional[Tensor] = None,
                      query_mask: Optional[Tensor] = None, causal: bool = True, q_offset: int = 0,
                      scale: Optional[float] = None, scale_mode: int = 0, kq_rule: int = 0,
                      kv_layout: int = 0, sorted: bool = True):
    """``score_topk`` with padding masks (sgsa_score_topk_masked).

    q [B,Tq,H,D]; k [B,Tk,H,D] (kv_layout 0) or [B,H,Tk,D] (kv_layout 1);
    key_mask [B,Tk] and query_mask [B,Tq] (nonzero = valid) or None.
    kq_rule 0 gives each row min(top_k, max(1, largest valid count over the
    batch)) slots (SparseRetriever._masked_topk, modeling_sgsa.py:159-160);
    kq_rule 1 gives every row min(top_k, Tk) (TopKSparseKVReuseAttention,
    hybrid_dense_delta_topk.py:348).  Returns (indices int32, scores float32,
    slot_valid uint8, all [B,H,Tq,kk]; top2 [B,H,Tq,2]; counts int32 [B,H,Tq]
    of valid selected slots; fill int32 [B,H,Tq] of filled slots), kk = min(top_k, Tk).
    """
    if not q.is_cuda:
        raise ValueError("score_topk_masked: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, Tq, H, D = q.shape
    Tk = k.shape[2] if kv_layout == 1 else k.shape[1]
    want = (B, H, Tk, D) if kv_layout == 1 else (B, Tk, H, D)
    if tuple(k.shape) != want or k.dtype != q.dtype:
        raise ValueError(f"k shape/dtype {tuple(k.shape)}/{k.dtype} does not match {want}/{q.dtype}")
    km = _mask_bytes(key_mask, (B, Tk), "key_mask")
    qm = _mask_bytes(query_mask, (B, Tq), "query_mask")
    kk = min(int(top_k), Tk)
    if scale is None:
        scale = math.sqrt(D) if scale_mode == 0 else 1.0 / math.sqrt(D)
    qc, kc = q.contiguous(), k.contiguous()
    dev = q.device
    idx = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.int32)
    sc = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.float32)
    valid = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.uint8)
    top2 = torch.empty(B, H, Tq, 2, device=dev, dtype=torch.float32)
    cnt = torch.empty(B, H, Tq, device=dev, dtype=torch.int32)
    fill = torch.empty(B, H, Tq, device=dev, dtype=torch.int32)
    L = _abi.lib()
    nbytes = ctypes.c_size_t()
    _abi.check(L.sgsa_score_topk_masked_workspace_size(_abi.dtype_code(q.dtype), B, Tq, Tk, H, D, int(km is not None),
                                                       int(kv_layout), ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_score_topk_masked(
        _abi.dtype_code(q.dtype), B, Tq, Tk, H, D, kk, int(causal), int(q_offset), float(scale), int(scale_mode),
        int(kq_rule), int(kv_layout), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(km), _abi.ptr(qm), _abi.ptr(idx),
        _abi.ptr(sc), _abi.ptr(valid), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(fill), int(sorted), _abi.ptr(ws),
        nbytes.value, _abi.stream_of(qc)))
    return idx, sc, valid, top2, cnt, fill


def gather_masked(k: Optional[Tensor], v: Tensor, idx: Tensor, sc: Tensor, valid: Optional[Tensor], top2: Tensor,
                  fill: Tensor, q_offset: int = 0, kv_layout: int = 0, self_key: Optional[Tensor] = None,
                  budget_logits: Optional[Tensor] = None, write_mode: str = "direct", alpha_max: float = 0.25,
                  tau_c: float = 0.1, local_window: int = 64, sink_size: int = 8, return_weights: bool = False,
                  return_diagnostics: bool = False, return_stats: bool = False) -> Dict[str, Optional[Tensor]]:
    """sgsa_sparse_gather_masked over ``score_topk_masked`` output.

    k (None: V-only), v: [B,Tk,H,D] (kv_layout 0) or [B,H,Tk,D] (kv_layout 1).
    ``valid`` None: every filled slot takes its softmax weight (the hybrid's
    probabilities); else the retriever's softmax * valid / sum.  Returns a dict
    of k_hat / v_hat [B,Tq,H,D], write_key, alpha [B,Tq,H], weights
    [B,H,Tq,kk] float32, diag [NDIAG,B,H,Tq], stats [2,B,H,Tq] (largest weight;
    |write key| / |k_hat| in residual mode) (None where not requested).
    """
    B, H, Tq, kk = idx.shape
    Tk = v.shape[2] if kv_layout == 1 else v.shape[1]
    D = v.shape[-1]
    dev = v.device
    kc = k.contiguous() if k is not None else None
    vc = v.contiguous()
    skc = self_key.contiguous() if self_key is not None else None
    mode = {"direct": 0, "residual": 1}[write_mode]
    k_hat = torch.empty(B, Tq, H, D, device=dev, dtype=v.dtype) if k is not None else None
    v_hat = torch.empty(B, Tq, H, D, device=dev, dtype=v.dtype)
    bud = budget_logits.float().contiguous() if budget_logits is not None else None
    al = torch.empty(B, Tq, H, device=dev, dtype=torch.float32) if bud is not None else None
    wkey = torch.empty_like(k_hat) if (bud is not None and mode == 1) else None
    weights = torch.empty(B, H, Tq, kk, device=dev, dtype=torch.float32) if return_weights else None
    diag = torch.empty(_abi.NDIAG, B, H, Tq, device=dev, dtype=torch.float32) if return_diagnostics else None
    stats = torch.empty(2, B, H, Tq, device=dev, dtype=torch.float32) if return_stats else None
    L = _abi.lib()
    nbytes = ctypes.c_size_t()
    _abi.check(L.sgsa_sparse_gather_workspace_size(B, Tq, H, D, kk, ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_sparse_gather_masked(
        _abi.dtype_code(v.dtype), B, Tq, Tk, H, D, kk, int(q_offset), int(kv_layout), _abi.ptr(kc), _abi.ptr(vc),
        _abi.ptr(skc), _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(valid), _abi.ptr(top2), _abi.ptr(fill), _abi.ptr(bud),
        mode, float(alpha_max), float(tau_c), int(local_window), int(sink_size), _abi.ptr(k_hat), _abi.ptr(v_hat),
        _abi.ptr(wkey), _abi.ptr(al), _abi.ptr(weights), _abi.ptr(diag), _abi.ptr(stats), _abi.ptr(ws), nbytes.value,
        _abi.stream_of(vc)))
    return {"k_hat": k_hat, "v_hat": v_hat, "write_key": (wkey if mode == 1 else k_hat), "alpha": al,
            "weights": weights, "diag": diag, "stats": stats}


def masked_gather_gate(q_ret: Tensor, k: Tensor, v: Tensor, budget_logits: Tensor, top_k: int,
                       attention_mask: Tensor, causal: bool = True, write_mode: str = "direct",
                       alpha_max: float = 0.25, tau_c: float = 0.1,
                       stats: Optional[dict] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Retrieval half of the SGSA layer under a padding mask [B,T] (the
    retriever's valid = causal & key_valid & query_valid, modeling_sgsa.py:421-428):
    (write key, v_hat, alpha) for the chunked update.  ``stats`` (a dict) receives
    "row_stats" as sgsa_layer_fwd_stats writes them."""
    idx, sc, valid, top2, cnt, fill = score_topk_masked(q_ret, k, top_k, key_mask=attention_mask,
                                                        query_mask=attention_mask, causal=causal, sorted=False)
    r = gather_masked(k, v, idx, sc, valid, top2, fill, self_key=k, budget_logits=budget_logits,
                      write_mode=write_mode, alpha_max=alpha_max, tau_c=tau_c, return_stats=stats is not None)
    if stats is not None:
        stats["row_stats"] = r["stats"]
        stats["alpha"] = r["alpha"]
    return r["write_key"], r["v_hat"], r["alpha"]


def gather_gate(k: Tensor, v: Tensor, idx: Tensor, sc: Tensor, top2: Tensor, cnt: Tensor,
                budget_logits: Tensor, split: Optional[Tensor] = None, write_mode: str = "direct",
                alpha_max: float = 0.25, tau_c: float = 0.1):
    """K2 of the layer path on top of ``score_topk`` output: (write key, v_hat, alpha).

    With ``split`` (unsorted top-k output, bf16, D=128) the tiled kernel runs;
    without it, the direct row gather.  k, v: [B,T,H,D]; budget_logits [B,T,H].
    """
    B, T, H, D = k.shape
    kk = idx.shape[-1]
    mode = {"direct": 0, "residual": 1}[write_mode]
    kc, vc = k.contiguous(), v.contiguous()
    dev = k.device
    wk = torch.empty(B, T, H, D, device=dev, dtype=k.dtype)
    vh = torch.empty_like(wk)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    bud = budget_logits.float().contiguous()
    L = _abi.lib()
    khat = wk if mode == 0 else None
    wkey = wk if mode == 1 else None
    if split is not None:
        _abi.check(L.sgsa_sparse_gather_tiled(
            B, T, H, D, kk, _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(top2),
            _abi.ptr(cnt), _abi.ptr(split), _abi.ptr(bud), mode, float(alpha_max), float(tau_c),
            _abi.ptr(khat), _abi.ptr(vh), _abi.ptr(wkey), _abi.ptr(al), _abi.stream_of(kc)))
    else:
        _abi.check(L.sgsa_sparse_gather(
            _abi.dtype_code(k.dtype), B, T, T, H, D, kk, 0, _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(kc),
            _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(bud), mode, float(alpha_max),
            float(tau_c), 64, 8, _abi.ptr(khat), _abi.ptr(vh), _abi.ptr(wkey), _abi.ptr(al), None, None, None, 0,
            _abi.stream_of(kc)))
    return wk, vh, al


def score_topk_lists(q: Tensor, k: Tensor, top_k: int):
    """K1 of the fused layer: the causal top-k of q.k/sqrt(D) written as tile
    lists (see include/sgsa.h) instead of per-row index/score lists.

    q, k [B,T,H,D] bfloat16.  Returns (lists uint8 buffer, offsets int32,
    top2 float32 [B,H,T,2], counts int32 [B,H,T]).
    """
    if not q.is_cuda:
        raise ValueError("score_topk_lists: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or k.shape != q.shape:
        raise ValueError("score_topk_lists takes bfloat16 q and k of equal shape")
    B, T, H, D = q.shape
    qc, kc = q.contiguous(), k.contiguous()
    dev = q.device
    L = _abi.lib()
    lb, ob, wb = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    _abi.check(L.sgsa_topk_lists_size(B, T, H, int(top_k), ctypes.byref(lb), ctypes.byref(ob)))
    _abi.check(L.sgsa_score_topk_workspace_size(B, T, H, ctypes.byref(wb)))
    lists = torch.empty(lb.value, device=dev, dtype=torch.uint8)
    offs = torch.empty(ob.value // 4, device=dev, dtype=torch.int32)
    top2 = torch.empty(B, H, T, 2, device=dev, dtype=torch.float32)
    cnt = torch.empty(B, H, T, device=dev, dtype=torch.int32)
    ws = torch.empty(wb.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_score_topk_lists(B, T, H, D, int(top_k), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(lists),
                                       _abi.ptr(offs), _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(ws), wb.value,
                                       _abi.stream_of(qc)))
    return lists, offs, top2, cnt


def gather_lists(k: Tensor, v: Tensor, lists: Tensor, offs: Tensor, top2: Tensor, cnt: Tensor,
                 budget_logits: Tensor, top_k: int, write_mode: str = "direct", alpha_max: float = 0.25,
                 tau_c: float = 0.1):
    """K2 of the fused layer on ``score_topk_lists`` output: (write key, v_hat, alpha)."""
    B, T, H, D = k.shape
    mode = {"direct": 0, "residual": 1}[write_mode]
    kc, vc = k.contiguous(), v.contiguous()
    wk = torch.empty_like(kc)
    vh = torch.empty_like(kc)
    al = torch.empty(B, T, H, device=k.device, dtype=torch.float32)
    bud = budget_logits.float().contiguous()
    _abi.check(_abi.lib().sgsa_sparse_gather_lists(
        B, T, H, D, int(top_k), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(lists), _abi.ptr(offs), _abi.ptr(top2),
        _abi.ptr(cnt), _abi.ptr(bud), mode, float(alpha_max), float(tau_c), _abi.ptr(wk if mode == 0 else None),
        _abi.ptr(vh), _abi.ptr(wk if mode == 1 else None), _abi.ptr(al), _abi.stream_of(kc)))
    return wk, vh, al


def score_topk_thresholds(q: Tensor, k: Tensor, top_k: int):
    """K1 of the fused layer (bf16, D = 128): the causal top-k of q.k/sqrt(D)
    left as one exact cut per row (see include/sgsa.h).

    q, k [B,T,H,D] bfloat16.  Returns (thr int32 [B,H,T,2] holding {float32 bits
    of th, cut}, top2 float32 [B,H,T,2], counts int32 [B,H,T]): key j <= t is
    selected iff score > th, or score == th and j <= cut.
    """
    if not q.is_cuda:
        raise ValueError("score_topk_thresholds: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or k.shape != q.shape:
        raise ValueError("score_topk_thresholds takes bfloat16 q and k of equal shape")
    B, T, H, D = q.shape
    qc, kc = q.contiguous(), k.contiguous()
    dev = q.device
    L = _abi.lib()
    wb = ctypes.c_size_t()
    _abi.check(L.sgsa_score_topk_workspace_size(B, T, H, ctypes.byref(wb)))
    thr = torch.empty(B, H, T, 2, device=dev, dtype=torch.int32)
    top2 = torch.empty(B, H, T, 2, device=dev, dtype=torch.float32)
    cnt = torch.empty(B, H, T, device=dev, dtype=torch.int32)
    ws = torch.empty(wb.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_score_topk_thresholds(B, T, H, D, int(top_k), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(thr),
                                            _abi.ptr(top2), _abi.ptr(cnt), _abi.ptr(ws), wb.value,
                                            _abi.stream_of(qc)))
    return thr, top2, cnt


def gather_thresholds(q: Tensor, k: Tensor, v: Tensor, thr: Tensor, top2: Tensor, cnt: Tensor,
                      budget_logits: Tensor, top_k: int, write_mode: str = "direct", alpha_max: float = 0.25,
                      tau_c: float = 0.1):
    """K2 of the fused layer on ``score_topk_thresholds`` output: (write key, v_hat, alpha)."""
    B, T, H, D = k.shape
    mode = {"direct": 0, "residual": 1}[write_mode]
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    wk = torch.empty_like(kc)
    vh = torch.empty_like(kc)
    al = torch.empty(B, T, H, device=k.device, dtype=torch.float32)
    bud = budget_logits.float().contiguous()
    _abi.check(_abi.lib().sgsa_sparse_gather_thresholds(
        B, T, H, D, int(top_k), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(thr), _abi.ptr(top2),
        _abi.ptr(cnt), _abi.ptr(bud), mode, float(alpha_max), float(tau_c), _abi.ptr(wk if mode == 0 else None),
        _abi.ptr(vh), _abi.ptr(wk if mode == 1 else None), _abi.ptr(al), _abi.stream_of(kc)))
    return wk, vh, al


def gather_thresholds_selection(q: Tensor, k: Tensor, v: Tensor, thr: Tensor, top2: Tensor, cnt: Tensor,
                                top_k: int) -> Tensor:
    """The selection K2 applies to ``score_topk_thresholds`` output, summarised per
    row as int32 [B,H,T,3] = {count, sum of key indices, xor of index * 2654435761}
    (sgsa_gather_thresholds_selection; compare with ``selection_summary``)."""
    B, T, H, D = k.shape
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    out = torch.empty(B, H, T, 3, device=k.device, dtype=torch.int32)
    _abi.check(_abi.lib().sgsa_gather_thresholds_selection(
        B, T, H, D, int(top_k), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(thr), _abi.ptr(top2),
        _abi.ptr(cnt), _abi.ptr(out), _abi.stream_of(kc)))
    return out


def selection_summary(idx: Tensor, cnt: Tensor) -> Tensor:
    """{count, sum, xor of index * 2654435761} (mod 2^32, as int32) of the first
    cnt slots of each row of index lists [..., k] -- the summary
    ``gather_thresholds_selection`` reports."""
    k = idx.shape[-1]
    live = torch.arange(k, device=idx.device) < cnt[..., None]
    j = idx.long() & 0xFFFFFFFF
    s = torch.where(live, j, torch.zeros_like(j)).sum(-1) & 0xFFFFFFFF
    hsh = torch.where(live, (j * 2654435761) & 0xFFFFFFFF, torch.zeros_like(j))
    x = torch.zeros_like(hsh[..., 0])
    for bit in range(32):   # xor over the slots, bit by bit (parity of the set bits)
        x |= (((hsh >> bit) & 1).sum(-1) & 1) << bit
    to_i32 = lambda t: torch.where(t >= 2 ** 31, t - 2 ** 32, t).to(torch.int32)
    return torch.stack([cnt.to(torch.int32), to_i32(s), to_i32(x)], dim=-1)


def score_dump(q: Tensor, k: Tensor, row0: int, rows: int, causal: bool = True, q_offset: int = 0,
               scale: Optional[float] = None, scale_mode: int = 0) -> Tensor:
    """The exact fp32 scores score_topk selects on, for query rows [row0, row0+rows): [B,H,rows,Tk]."""
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    if scale is None:
        scale = math.sqrt(D) if scale_mode == 0 else 1.0 / math.sqrt(D)
    qc, kc = q.contiguous(), k.contiguous()
    out = torch.empty(B, H, rows, Tk, device=q.device, dtype=torch.float32)
    _abi.check(_abi.lib().sgsa_score_dump(
        _abi.dtype_code(q.dtype), B, Tq, Tk, H, D, int(causal), int(q_offset), float(scale), int(scale_mode),
        _abi.ptr(qc), _abi.ptr(kc), int(row0), int(rows), _abi.ptr(out), _abi.stream_of(qc)))
    return out


def sparse_retrieve(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    top_k: int,
    causal: bool = True,
    attention_mask: Optional[Tensor] = None,
    tau_c: float = 0.1,
    local_window: int = 64,
    sink_size: int = 8,
    sorted: bool = True,
    return_weights: bool = True,
    return_diagnostics: bool = True,
    cu_seqlens: Optional[Tensor] = None,
) -> Dict[str, object]:
    """Token-only retrieval; the dict of SparseRetriever.forward (modeling_sgsa.py:467-474).

    q,k,v: [B,T,H,D].  k_hat/v_hat are [B,T,H,D]; indices/weights [B,H,T,kk];
    diagnostics [B,H,T] each.  attention_mask [B,T] (nonzero = real token)
    masks padded keys and padded queries (:421-428); a row then keeps
    min(top_k, max(1, largest valid count of that row over the batch)) slots,
    its invalid ones pointing at its lowest-index invalid keys with weight 0
    and the rest index 0 (:144-165).  ``cu_seqlens`` [N+1]: N sequences packed
    along T of a batch of one, each retrieving from itself (sgsa_amd.varlen);
    outputs come back packed, indices relative to the sequence start.
    """
    if cu_seqlens is not None:
        from . import varlen
        if attention_mask is not None:
            raise ValueError("sparse_retrieve: pass either cu_seqlens or attention_mask, not both")
        lay = varlen.layout(cu_seqlens, q)
        r = sparse_retrieve(lay.pad(q), lay.pad(k), lay.pad(v), top_k, causal=causal, attention_mask=lay.mask,
                            tau_c=tau_c, local_window=local_window, sink_size=sink_size, sorted=sorted,
                            return_weights=return_weights, return_diagnostics=return_diagnostics)
        return varlen.unpad_retrieval(lay, r)
    B, T, H, D = q.shape
    if v.shape != k.shape or v.dtype != k.dtype:
        raise ValueError("v must match k in shape and dtype")
    if attention_mask is not None:
        idx, sc, valid, top2, cnt, fill = score_topk_masked(q, k, top_k, key_mask=attention_mask,
                                                            query_mask=attention_mask, causal=causal, sorted=sorted)
        r = gather_masked(k, v, idx, sc, valid, top2, fill, self_key=k, tau_c=tau_c, local_window=local_window,
                          sink_size=sink_size, return_weights=return_weights, return_diagnostics=return_diagnostics)
        diag = r["diag"]
        return {
            "indices": idx.long(),
            "block_indices": None,
            "weights": r["weights"].to(q.dtype) if r["weights"] is not None else None,
            "k_hat": r["k_hat"],
            "v_hat": r["v_hat"],
            "diagnostics": ({n: diag[i] for i, n in enumerate(_abi.DIAG_NAMES)} if diag is not None else {}),
            "scores": sc,
            "counts": cnt,
            "valid": valid.bool(),
        }
    idx, sc, top2, cnt = score_topk(q, k, top_k, causal=causal, sorted=sorted)
    kk = idx.shape[-1]
    kc, vc = k.contiguous(), v.contiguous()
    dev = q.device
    k_hat = torch.empty(B, T, H, D, device=dev, dtype=q.dtype)
    v_hat = torch.empty_like(k_hat)
    weights = torch.empty(B, H, T, kk, device=dev, dtype=torch.float32) if return_weights else None
    diag = torch.empty(_abi.NDIAG, B, H, T, device=dev, dtype=torch.float32) if return_diagnostics else None
    ws = torch.empty(256, device=dev, dtype=torch.uint8)
    _abi.check(_abi.lib().sgsa_sparse_gather(
        _abi.dtype_code(q.dtype), B, T, T, H, D, kk, 0,
        _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(kc), _abi.ptr(idx), _abi.ptr(sc), _abi.ptr(top2), _abi.ptr(cnt),
        None, 0, 0.0, float(tau_c), int(local_window), int(sink_size),
        _abi.ptr(k_hat), _abi.ptr(v_hat), None, None, _abi.ptr(weights), _abi.ptr(diag),
        _abi.ptr(ws), 256, _abi.stream_of(kc)))
    out = {
        "indices": idx.long(),
        "block_indices": None,
        "weights": weights.to(q.dtype) if weights is not None else None,
        "k_hat": k_hat,
        "v_hat": v_hat,
        "diagnostics": ({n: diag[i] for i, n in enumerate(_abi.DIAG_NAMES)} if diag is not None else {}),
        "scores": sc,
        "counts": cnt,
    }
    return out


BLOCK_MODES = {"block_only": 0, "block_token": 1}


def block_retrieve(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    top_k: int,
    block_size: int,
    top_blocks: int,
    mode: str = "block_token",
    causal: bool = True,
    attention_mask: Optional[Tensor] = None,
    tau_c: float = 0.1,
    local_window: int = 64,
    sink_size: int = 8,
    return_weights: bool = True,
    return_diagnostics: bool = True,
    return_block_scores: bool = False,
    cu_seqlens: Optional[Tensor] = None,
) -> Dict[str, object]:
    """Block retrieval; the dict of SparseRetriever.forward for ``retrieval_mode``
    "block_only" / "block_token" on the torch path (modelings/modeling_sgsa.py:444-474).

    q,k,v: [B,T,H,D].  k_hat/v_hat [B,T,H,D]; block_indices [B,H,T,min(top_blocks, nb)];
    block_token: indices and weights [B,H,T,min(top_k, T)]; block_only: indices None,
    weights [B,H,T,T], and the diagnostics without the distance statistics (:455-463).
    attention_mask [B,T] (nonzero = real token) masks keys and query rows alike, as
    the reference's valid mask does (:421-428): block scores, the rows' k_q over the
    valid blocks (:188-195, :159-160) and the candidates (:313-320) see only real
    tokens, and padded rows retrieve nothing (sgsa_block_retrieve_masked).
    ``cu_seqlens`` [N+1]: packed sequences in a batch of one (sgsa_amd.varlen);
    blocks start at each sequence's start, outputs come back packed (block_only's
    dense weights [1,H,total,L_max] over the row's own sequence).
    """
    if cu_seqlens is not None:
        from . import varlen
        if attention_mask is not None:
            raise ValueError("block_retrieve: pass either cu_seqlens or attention_mask, not both")
        lay = varlen.layout(cu_seqlens, q)
        r = block_retrieve(lay.pad(q), lay.pad(k), lay.pad(v), top_k, block_size, top_blocks, mode, causal=causal,
                           attention_mask=lay.mask, tau_c=tau_c, local_window=local_window, sink_size=sink_size,
                           return_weights=return_weights, return_diagnostics=return_diagnostics,
                           return_block_scores=return_block_scores)
        return varlen.unpad_retrieval(lay, r)
    if mode not in BLOCK_MODES:
        raise ValueError(f"mode must be one of {sorted(BLOCK_MODES)}, got {mode!r}")
    B, T, H, D = q.shape
    if k.shape != q.shape or v.shape != k.shape or k.dtype != q.dtype or v.dtype != k.dtype:
        raise ValueError("q, k and v must share shape and dtype")
    m = BLOCK_MODES[mode]
    dev = q.device
    nb = (T - 1) // block_size + 1 if T > 0 and block_size > 0 else 0
    eb = min(top_blocks, nb)
    kk = min(top_k, T)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    lib = _abi.lib()
    n = ctypes.c_size_t()
    _abi.check(lib.sgsa_block_retrieve_workspace_size(B, T, H, int(top_k), int(block_size), int(top_blocks), m,
                                                      ctypes.byref(n)))
    ws = torch.empty(max(n.value, 1), device=dev, dtype=torch.uint8)
    idx = torch.empty(B, H, T, kk, device=dev, dtype=torch.int32) if m == 1 else None
    bidx = torch.empty(B, H, T, eb, device=dev, dtype=torch.int32)
    bsc = torch.empty(B, H, T, nb, device=dev, dtype=torch.float32) if return_block_scores else None
    weights = None
    if return_weights:
        weights = torch.empty(B, H, T, kk if m == 1 else T, device=dev, dtype=torch.float32)
    k_hat = torch.empty(B, T, H, D, device=dev, dtype=q.dtype)
    v_hat = torch.empty_like(k_hat)
    diag = torch.empty(_abi.NDIAG, B, H, T, device=dev, dtype=torch.float32) if return_diagnostics else None
    if attention_mask is None:
        _abi.check(lib.sgsa_block_retrieve(
            _abi.dtype_code(q.dtype), B, T, H, D, int(top_k), int(block_size), int(top_blocks), m, int(causal),
            float(tau_c), int(local_window), int(sink_size), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(idx),
            _abi.ptr(bidx), _abi.ptr(bsc), _abi.ptr(weights), _abi.ptr(k_hat), _abi.ptr(v_hat), _abi.ptr(diag),
            _abi.ptr(ws), ws.numel(), _abi.stream_of(qc)))
    else:
        if tuple(attention_mask.shape) != (B, T):
            raise ValueError(f"attention_mask must have shape [batch, seq] = {(B, T)}, got {tuple(attention_mask.shape)}")
        am = (attention_mask.to(dev) != 0).to(torch.uint8).contiguous()
        _abi.check(lib.sgsa_block_retrieve_masked(
            _abi.dtype_code(q.dtype), B, T, H, D, int(top_k), int(block_size), int(top_blocks), m, int(causal),
            float(tau_c), int(local_window), int(sink_size), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(am),
            _abi.ptr(idx), _abi.ptr(bidx), _abi.ptr(bsc), _abi.ptr(weights), _abi.ptr(k_hat), _abi.ptr(v_hat),
            _abi.ptr(diag), _abi.ptr(ws), ws.numel(), _abi.stream_of(qc)))
    names = _abi.DIAG_NAMES if m == 1 else _abi.DIAG_NAMES[:6]
    out = {
        "indices": idx.long() if idx is not None else None,
        "block_indices": bidx.long(),
        "weights": weights.to(q.dtype) if weights is not None else None,
        "k_hat": k_hat,
        "v_hat": v_hat,
        "diagnostics": ({name: diag[i] for i, name in enumerate(names)} if diag is not None else {}),
    }
    if bsc is not None:
        out["block_scores"] = bsc
    return out


class SparseRetriever(nn.Module):
    """SparseRetriever (modelings/modeling_sgsa.py:90-474): ``retrieval_mode`` token_only,
    block_only or block_token, with the torch retrieval path's semantics (the flash_moba
    backend of :103-108 is a CUDA library this build does not have).

    Takes any config object with ``top_k``, ``tau_c``, ``local_window``,
    ``sink_size``, ``retrieval_mode`` and, for the block modes, ``block_size`` and
    ``top_blocks`` attributes (the reference's SGSAConfig).
    """

    def __init__(self, config) -> None:
        super().__init__()
        mode = getattr(config, "retrieval_mode", "token_only")
        if mode != "token_only" and mode not in BLOCK_MODES:
            raise ValueError(f"retrieval_mode={mode!r}: expected token_only, block_only or block_token")
        self.mode = mode
        self.block_size = getattr(config, "block_size", 32)
        self.top_blocks = getattr(config, "top_blocks", 2)
        self.top_k = config.top_k
        self.tau_c = getattr(config, "tau_c", 0.1)
        self.local_window = getattr(config, "local_window", 64)
        self.sink_size = getattr(config, "sink_size", 8)

    def forward(self, q: Tensor, k: Tensor, v: Tensor, causal: bool = True,
                attention_mask: Optional[Tensor] = None, cu_seqlens: Optional[Tensor] = None) -> Dict[str, object]:
        """The reference's forward (:407-474); ``cu_seqlens`` additionally takes packed
        sequences in a batch of one (the varlen layout of the reference's flash_moba calls)."""
        if self.mode != "token_only":
            r = block_retrieve(q, k, v, self.top_k, self.block_size, self.top_blocks, self.mode, causal=causal,
                               attention_mask=attention_mask, tau_c=self.tau_c, local_window=self.local_window,
                               sink_size=self.sink_size, cu_seqlens=cu_seqlens)
            return {key: r[key] for key in ("indices", "block_indices", "weights", "k_hat", "v_hat", "diagnostics")}
        r = sparse_retrieve(q, k, v, self.top_k, causal=causal, attention_mask=attention_mask, tau_c=self.tau_c,
                            local_window=self.local_window, sink_size=self.sink_size, cu_seqlens=cu_seqlens)
        return {key: r[key] for key in ("indices", "block_indices", "weights", "k_hat", "v_hat", "diagnostics")}
