"""Whole SGSA layer forward in one C-ABI call (sgsa_layer_fwd).

The attention half of SGSABlock.forward (modelings/modeling_sgsa.py:669-684)
with the projections taken as inputs: token top-k retrieval on (q_ret, k, v),
the write key and alpha gate of SGSAStateLayer (:546-552, :497-504) from the
budget logits, then the chunked state update (:584-596).
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _abi
from .ops import chunk_sgsa_fwd
from .retrieval import masked_gather_gate

Tensor = torch.Tensor

_WRITE_MODES = {"direct": 0, "residual": 1}


class LayerWorkspace:
    """Reusable device workspace for sgsa_layer_fwd, grown on demand."""

    def __init__(self) -> None:
        self.buf: Optional[Tensor] = None

    def get(self, nbytes: int, device) -> Tensor:
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.empty(nbytes, device=device, dtype=torch.uint8)
        return self.buf


def layer_workspace_bytes(dtype: torch.dtype, B: int, T: int, H: int, D: int, top_k: int) -> int:
    n = ctypes.c_size_t()
    _abi.check(_abi.lib().sgsa_layer_fwd_workspace_size(_abi.dtype_code(dtype), B, T, H, D, int(top_k),
                                                        ctypes.byref(n)))
    return n.value


def _masked_threshold_form(q: Tensor) -> bool:
    """A padded bf16 layer with d = 128 and T <= 65536 runs the threshold form on its
    valid-first keys (sgsa_layer_retrieve_masked); anything else the masked row path."""
    return q.dtype == torch.bfloat16 and q.shape[-1] == 128 and q.shape[1] <= 65536


def _retrieve_masked_thr(q_ret: Tensor, k: Tensor, v: Tensor, budget_logits: Tensor, top_k: int,
                         attention_mask: Tensor, write_mode: str, alpha_max: float, tau_c: float,
                         workspace: Optional["LayerWorkspace"], stats: Optional[dict]):
    B, T, H, D = q_ret.shape
    dev = q_ret.device
    if tuple(attention_mask.shape) != (B, T):
        raise ValueError(f"attention_mask must have shape [batch, seq] = {(B, T)}, got {tuple(attention_mask.shape)}")
    am = (attention_mask.to(dev) != 0).to(torch.uint8).contiguous()
    rc, kc, vc = (t.contiguous() for t in (q_ret, k, v))
    uc = budget_logits.float().contiguous()
    n = ctypes.c_size_t()
    _abi.check(_abi.lib().sgsa_layer_retrieve_masked_workspace_size(_abi.dtype_code(q_ret.dtype), B, T, H, D,
                                                                    int(top_k), ctypes.byref(n)))
    ws = (workspace or LayerWorkspace()).get(n.value, dev)
    wk = torch.empty_like(kc)
    vh = torch.empty_like(kc)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    rs = None
    if stats is not None:
        stats["alpha"] = al
        rs = stats["row_stats"] = torch.empty(2, B, H, T, device=dev, dtype=torch.float32)
    _abi.check(_abi.lib().sgsa_layer_retrieve_masked(
        _abi.dtype_code(q_ret.dtype), B, T, H, D, int(top_k), _abi.ptr(rc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(am),
        _abi.ptr(uc), _WRITE_MODES[write_mode], float(alpha_max), float(tau_c), _abi.ptr(wk), _abi.ptr(vh),
        _abi.ptr(al), _abi.ptr(rs), _abi.ptr(ws), ws.numel(), _abi.stream_of(rc)))
    return wk, vh, al


def sgsa_layer_forward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    q_ret: Tensor,
    beta: Tensor,
    gamma: Tensor,
    budget_logits: Tensor,
    top_k: int,
    initial_state: Optional[Tensor] = None,
    write_mode: str = "direct",
    alpha_max: float = 0.25,
    tau_c: float = 0.1,
    chunk_size: int = 64,
    output_final_state: bool = True,
    workspace: Optional[LayerWorkspace] = None,
    out: Optional[Tensor] = None,
    attention_mask: Optional[Tensor] = None,
    stats: Optional[dict] = None,
) -> Tuple[Tensor, Optional[Tensor]]:
    """q,k,v,q_ret [B,T,H,D] (float32 or bfloat16); beta,gamma,budget_logits [B,T,H].

    Returns (o [B,T,H,D] in q.dtype, final state [B,H,D,D] float32 or None).
    attention_mask [B,T] (nonzero = real token): the retrieval masks padded
    keys and queries (SparseRetriever.forward, modeling_sgsa.py:421-428); the
    state update itself takes no mask (:584-596).  The masked layer runs its
    retrieval on the threshold form over valid-first keys (bf16, d = 128,
    T <= 65536: sgsa_layer_retrieve_masked) or else as the masked select and
    gather, then the chunked update.
    ``stats`` (a dict) receives "alpha" [B,T,H] and "row_stats" [2,B,H,T]
    (sgsa_layer_fwd_stats: largest weight, write-key norm ratio per row).
    """
    if not q.is_cuda:
        raise ValueError("sgsa_layer_forward: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, T, H, D = q.shape
    for name, t in (("k", k), ("v", v), ("q_ret", q_ret)):
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError(f"{name} must match q in shape and dtype")
    for name, t in (("beta", beta), ("gamma", gamma), ("budget_logits", budget_logits)):
        if t.shape != (B, T, H):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {(B, T, H)}")
    if write_mode not in _WRITE_MODES:
        raise ValueError(f"write_mode must be one of {sorted(_WRITE_MODES)}")
    if attention_mask is not None:
        if _masked_threshold_form(q):
            wk, vh, al = _retrieve_masked_thr(q_ret, k, v, budget_logits, top_k, attention_mask, write_mode,
                                              alpha_max, tau_c, workspace, stats)
        else:
            wk, vh, al = masked_gather_gate(q_ret, k, v, budget_logits, top_k, attention_mask, write_mode=write_mode,
                                            alpha_max=alpha_max, tau_c=tau_c, stats=stats)
        o, ht = chunk_sgsa_fwd(q, k, v, beta, gamma, wk, vh, al, initial_state=initial_state,
                               chunk_size=chunk_size, output_final_state=output_final_state)
        if out is not None:
            out.copy_(o)
            o = out
        return o, ht
    dev = q.device
    qc, kc, vc, rc = (t.contiguous() for t in (q, k, v, q_ret))
    bc, gc, uc = (t.float().contiguous() for t in (beta, gamma, budget_logits))
    h0 = initial_state.float().contiguous() if initial_state is not None else None
    if out is None:
        out = torch.empty_like(qc)
    ht = torch.empty(B, H, D, D, device=dev, dtype=torch.float32) if output_final_state else None
    nbytes = layer_workspace_bytes(q.dtype, B, T, H, D, top_k)
    ws = (workspace or LayerWorkspace()).get(nbytes, dev)
    al = rs = None
    if stats is not None:
        al = stats["alpha"] = torch.empty(B, T, H, device=dev, dtype=torch.float32)
        rs = stats["row_stats"] = torch.empty(2, B, H, T, device=dev, dtype=torch.float32)
    _abi.check(_abi.lib().sgsa_layer_fwd_stats(
        _abi.dtype_code(q.dtype), B, T, H, D, int(top_k), int(chunk_size),
        _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(rc), _abi.ptr(bc), _abi.ptr(gc), _abi.ptr(uc),
        _abi.ptr(h0), _WRITE_MODES[write_mode], float(alpha_max), float(tau_c), _abi.ptr(out), _abi.ptr(ht),
        _abi.ptr(al), _abi.ptr(rs), _abi.ptr(ws), ws.numel(), _abi.stream_of(qc)))
    return out, ht


def sgsa_layer_retrieve(
    q_ret: Tensor,
    k: Tensor,
    v: Tensor,
    budget_logits: Tensor,
    top_k: int,
    write_mode: str = "direct",
    alpha_max: float = 0.25,
    tau_c: float = 0.1,
    workspace: Optional[LayerWorkspace] = None,
    attention_mask: Optional[Tensor] = None,
    stats: Optional[dict] = None,
) -> Tuple[Tensor, Tensor, Tensor]:
    """The retrieval half of ``sgsa_layer_forward`` (sgsa_layer_retrieve): the
    (write key, v_hat, alpha) that the layer feeds to the chunked update
    (with ``attention_mask`` [B,T], the masked select and gather).

    q_ret, k, v [B,T,H,D] (float32 or bfloat16); budget_logits [B,T,H].
    Returns write_key / v_hat [B,T,H,D] in the input dtype and alpha [B,T,H] float32.
    """
    if not q_ret.is_cuda:
        raise ValueError("sgsa_layer_retrieve: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, T, H, D = q_ret.shape
    for name, t in (("k", k), ("v", v)):
        if t.shape != q_ret.shape or t.dtype != q_ret.dtype:
            raise ValueError(f"{name} must match q_ret in shape and dtype")
    if budget_logits.shape != (B, T, H):
        raise ValueError(f"budget_logits has shape {tuple(budget_logits.shape)}, expected {(B, T, H)}")
    if write_mode not in _WRITE_MODES:
        raise ValueError(f"write_mode must be one of {sorted(_WRITE_MODES)}")
    if attention_mask is not None:
        if _masked_threshold_form(q_ret):
            return _retrieve_masked_thr(q_ret, k, v, budget_logits, top_k, attention_mask, write_mode, alpha_max,
                                        tau_c, workspace, stats)
        return masked_gather_gate(q_ret, k, v, budget_logits, top_k, attention_mask, write_mode=write_mode,
                                  alpha_max=alpha_max, tau_c=tau_c, stats=stats)
    dev = q_ret.device
    rc, kc, vc = (t.contiguous() for t in (q_ret, k, v))
    uc = budget_logits.float().contiguous()
    wk = torch.empty_like(kc)
    vh = torch.empty_like(kc)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    nbytes = layer_workspace_bytes(q_ret.dtype, B, T, H, D, top_k)
    ws = (workspace or LayerWorkspace()).get(nbytes, dev)
    rs = None
    if stats is not None:
        stats["alpha"] = al
        rs = stats["row_stats"] = torch.empty(2, B, H, T, device=dev, dtype=torch.float32)
    _abi.check(_abi.lib().sgsa_layer_retrieve_stats(
        _abi.dtype_code(q_ret.dtype), B, T, H, D, int(top_k), _abi.ptr(rc), _abi.ptr(kc), _abi.ptr(vc),
        _abi.ptr(uc), _WRITE_MODES[write_mode], float(alpha_max), float(tau_c), _abi.ptr(wk), _abi.ptr(vh),
        _abi.ptr(al), _abi.ptr(rs), _abi.ptr(ws), ws.numel(), _abi.stream_of(rc)))
    return wk, vh, al


_BLOCK_MODES = {"block_only": 0, "block_token": 1}


def sgsa_block_layer_retrieve(
    q_ret: Tensor,
    k: Tensor,
    v: Tensor,
    budget_logits: Tensor,
    top_k: int,
    block_size: int,
    top_blocks: int,
    mode: str = "block_token",
    write_mode: str = "direct",
    alpha_max: float = 0.25,
    tau_c: float = 0.1,
    workspace: Optional[LayerWorkspace] = None,
    attention_mask: Optional[Tensor] = None,
    stats: Optional[dict] = None,
) -> Tuple[Tensor, Tensor, Tensor]:
    """The retrieval half of SGSABlock.forward in the block modes (sgsa_block_layer_retrieve):
    SparseRetriever's block_only / block_token retrieval (modelings/modeling_sgsa.py:444-463,
    causal, with the optional padding mask of :421-428), then the write key and alpha gate
    of SGSAStateLayer (:543-552, :497-504).

    q_ret, k, v [B,T,H,D] (float32 or bfloat16); budget_logits [B,T,H].  Returns write_key /
    v_hat [B,T,H,D] in the input dtype and alpha [B,T,H] float32.  ``stats`` receives
    "alpha" and "row_stats" [2,B,H,T] (largest weight; |write key| / |k_hat| in residual mode).
    """
    if not q_ret.is_cuda:
        raise ValueError("sgsa_block_layer_retrieve: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    if mode not in _BLOCK_MODES:
        raise ValueError(f"mode must be one of {sorted(_BLOCK_MODES)}, got {mode!r}")
    if write_mode not in _WRITE_MODES:
        raise ValueError(f"write_mode must be one of {sorted(_WRITE_MODES)}")
    B, T, H, D = q_ret.shape
    for name, t in (("k", k), ("v", v)):
        if t.shape != q_ret.shape or t.dtype != q_ret.dtype:
            raise ValueError(f"{name} must match q_ret in shape and dtype")
    if budget_logits.shape != (B, T, H):
        raise ValueError(f"budget_logits has shape {tuple(budget_logits.shape)}, expected {(B, T, H)}")
    dev = q_ret.device
    m = _BLOCK_MODES[mode]
    rc, kc, vc = (t.contiguous() for t in (q_ret, k, v))
    uc = budget_logits.float().contiguous()
    am = None
    if attention_mask is not None:
        if tuple(attention_mask.shape) != (B, T):
            raise ValueError(f"attention_mask must have shape [batch, seq] = {(B, T)}, got "
                             f"{tuple(attention_mask.shape)}")
        am = (attention_mask.to(dev) != 0).to(torch.uint8).contiguous()
    n = ctypes.c_size_t()
    _abi.check(_abi.lib().sgsa_block_layer_retrieve_workspace_size(B, T, H, int(top_k), int(block_size),
                                                                   int(top_blocks), m, ctypes.byref(n)))
    ws = (workspace or LayerWorkspace()).get(max(n.value, 1), dev)
    wk = torch.empty_like(kc)
    vh = torch.empty_like(kc)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    rs = None
    if stats is not None:
        stats["alpha"] = al
        rs = stats["row_stats"] = torch.empty(2, B, H, T, device=dev, dtype=torch.float32)
    _abi.check(_abi.lib().sgsa_block_layer_retrieve(
        _abi.dtype_code(q_ret.dtype), B, T, H, D, int(top_k), int(block_size), int(top_blocks), m, float(tau_c),
        _abi.ptr(rc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(am), _abi.ptr(uc), _WRITE_MODES[write_mode],
        float(alpha_max), _abi.ptr(wk), _abi.ptr(vh), _abi.ptr(al), _abi.ptr(rs), _abi.ptr(ws), ws.numel(),
        _abi.stream_of(rc)))
    return wk, vh, al
