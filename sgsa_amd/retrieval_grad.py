"""Differentiable retrieval and write gate, for training the SGSA block.

The inference path (``sgsa_layer_forward`` / ``sgsa_layer_retrieve`` /
``sgsa_block_layer_retrieve``) selects, weighs and gathers inside HIP kernels
that have no backward.  Under autograd the block takes this form instead, which
keeps the reference's own structure (modelings/modeling_sgsa.py:113-142
``_token_only``, :296-345 ``_tokens_from_blocks``, :361-382 ``_diagnostics``,
:497-504 ``_compute_alpha``, :543-551 the write key):

* the selection runs on the GPU under ``no_grad`` with the forward's kernels and
  tie rules -- K1 (``score_topk`` / ``score_topk_masked``) for token_only, the
  block retrieval (``block_retrieve``) for the block modes: indices are
  constants of the step, as ``torch.topk``'s are for autograd in the reference;
* the scores of the selected keys, their softmax weights, k_hat and v_hat, the
  margin, concentration, novelty, the write key and alpha are then torch ops on
  the selected rows only ([B,H,T,n,D] gathers: the reference's expand+gather
  restricted to the n selected or candidate slots), so autograd reaches q_ret, k,
  v and the budget logits through every term, with no detach, as in the reference.

The selected rows cost B*H*T*n*D fp32 elements per tensor (K and V, plus their
gradients); calls above ``MAX_SELECTED_ELEMS`` raise instead of exhausting memory.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch
from torch import Tensor

from .retrieval import block_retrieve, score_topk, score_topk_masked

__all__ = ["retrieve_differentiable", "retrieve_block_differentiable", "MAX_SELECTED_ELEMS"]

MAX_SELECTED_ELEMS = 1 << 31   # B*H*T*n*D: 8 GB of fp32 per gathered tensor

_FMIN = torch.finfo(torch.float32).min


def _check(q_ret: Tensor, n: int, write_mode: str, who: str) -> None:
    if write_mode not in ("direct", "residual"):
        raise ValueError(f"write_mode must be 'direct' or 'residual', got {write_mode!r}")
    if not q_ret.is_cuda:
        raise ValueError(f"{who}: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, T, H, D = q_ret.shape
    if B * H * T * n * D > MAX_SELECTED_ELEMS:
        raise ValueError(f"{who}: B*H*T*n*D = {B * H * T * n * D} selected elements exceed {MAX_SELECTED_ELEMS}; "
                         "train on shorter sequences or fewer selected keys")


def _weigh(q_ret: Tensor, k: Tensor, v: Tensor, idx: Tensor, valid: Tensor, eps: float):
    """Scores, weights, k_hat, v_hat [B,H,T,*] of the slots ``idx`` [B,H,T,n] (key positions)
    whose ``valid`` flag is set: q.k / sqrt(D) in fp32 (finfo.min elsewhere), the softmax
    times the flags renormalised (modeling_sgsa.py:126-128), the weighted sums (:130-134);
    also the keys [B,H,T,D] in fp32 for the diagnostics."""
    B, T, H, D = q_ret.shape
    n = idx.shape[-1]
    with torch.no_grad():
        rows = (torch.arange(B * H, device=idx.device, dtype=torch.long).view(B, H, 1, 1) * T
                + idx.long().clamp(0, T - 1)).reshape(-1)
    qh = q_ret.float().transpose(1, 2).contiguous()            # [B,H,T,D]
    kh = k.float().transpose(1, 2).contiguous()
    vh = v.float().transpose(1, 2).contiguous()
    ksel = kh.reshape(B * H * T, D).index_select(0, rows).view(B, H, T, n, D)
    vsel = vh.reshape(B * H * T, D).index_select(0, rows).view(B, H, T, n, D)
    s = torch.matmul(ksel, qh.unsqueeze(-1)).squeeze(-1) * (1.0 / math.sqrt(D))
    s = torch.where(valid, s, torch.full_like(s, _FMIN))
    w = torch.softmax(s, dim=-1) * valid.to(s.dtype)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(eps)
    k_hat = torch.matmul(w.unsqueeze(-2), ksel).squeeze(-2)
    v_hat = torch.matmul(w.unsqueeze(-2), vsel).squeeze(-2)
    return s, w, k_hat, v_hat, kh


def _gate(k: Tensor, v: Tensor, kh: Tensor, w: Tensor, k_hat: Tensor, v_hat: Tensor, margin: Tensor,
          budget_logits: Tensor, write_mode: str, alpha_max: float, tau_c: float, eps: float):
    """_diagnostics' concentration and novelty (modeling_sgsa.py:368-381), the write key
    (:543-550) and alpha (:497-504); returns (write key, v_hat, alpha, stats) in the
    block's layouts."""
    conc = torch.sigmoid(margin / max(tau_c, eps))
    dot = (k_hat * kh).sum(dim=-1)
    self_norm = kh.norm(dim=-1).clamp_min(eps)
    kh_norm = k_hat.norm(dim=-1).clamp_min(eps)
    proj = dot / (self_norm * self_norm + eps)
    perp = k_hat - proj.unsqueeze(-1) * kh
    novelty = (perp.norm(dim=-1) / (kh_norm + eps)).clamp(0.0, 1.0)
    if write_mode == "residual":
        wkey = k_hat - (dot / (kh * kh).sum(dim=-1).clamp_min(eps)).unsqueeze(-1) * kh
        perp_ratio = (wkey.norm(dim=-1) / kh_norm).clamp(0.0, 10.0)
    else:
        wkey = k_hat
        perp_ratio = torch.zeros_like(dot)
    budget = torch.sigmoid(budget_logits.float().transpose(1, 2))    # [B,H,T]
    alpha = alpha_max * conc * novelty * budget
    prox = alpha * v_hat.norm(dim=-1) * wkey.norm(dim=-1)
    alpha = alpha * torch.clamp(1.0 / prox.clamp_min(1.0), max=1.0)
    alpha_bth = alpha.transpose(1, 2).contiguous()
    stats = {"alpha": alpha_bth.detach(),
             "row_stats": torch.stack([w.detach().max(dim=-1).values, perp_ratio.detach()])}
    return (wkey.transpose(1, 2).to(k.dtype).contiguous(), v_hat.transpose(1, 2).to(v.dtype).contiguous(),
            alpha_bth, stats)


def _top2_margin(s: Tensor, valid: Tensor) -> Tensor:
    """Best minus second-best valid score of each row (finfo.min stands in for a missing
    second, as the reference's padded slots do), 0 for rows of one slot."""
    if s.shape[-1] < 2:
        return torch.zeros_like(s[..., 0])
    t2 = torch.topk(torch.where(valid, s, torch.full_like(s, _FMIN)), 2, dim=-1).values
    return t2[..., 0] - t2[..., 1]


def retrieve_differentiable(q_ret: Tensor, k: Tensor, v: Tensor, budget_logits: Tensor, top_k: int,
                            write_mode: str = "direct", alpha_max: float = 0.25, tau_c: float = 0.1,
                            attention_mask: Optional[Tensor] = None, eps: float = 1e-6
                            ) -> Tuple[Tensor, Tensor, Tensor, Dict[str, Tensor]]:
    """token_only: (write_key [B,T,H,D] in k's dtype, v_hat [B,T,H,D] in v's dtype, alpha
    [B,T,H] fp32, stats) for q_ret, k, v [B,T,H,D] and budget logits [B,T,H],
    differentiable in all four.

    ``stats`` holds "alpha" and "row_stats" [2,B,H,T] (the largest weight; |write key| /
    |k_hat| in the residual mode, else 0), as the inference path reports them.  The
    causal top-k runs with ``attention_mask`` [B,T] (nonzero = real token) on keys and
    queries, and each row keeps min(top_k, max(1, largest valid count)) slots
    (modeling_sgsa.py:159-160).
    """
    B, T, H, D = q_ret.shape
    kk = min(int(top_k), T)
    _check(q_ret, kk, write_mode, "retrieve_differentiable")
    dev = q_ret.device
    with torch.no_grad():
        if attention_mask is None:
            idx, _, _, cnt = score_topk(q_ret.detach(), k.detach(), kk, causal=True, sorted=True)
            valid = torch.arange(kk, device=dev) < cnt[..., None].long()
        else:
            m = attention_mask.to(torch.bool)
            idx, _, vmask, _, _, _ = score_topk_masked(q_ret.detach(), k.detach(), kk, key_mask=m, query_mask=m,
                                                       causal=True, kq_rule=0, sorted=True)
            valid = vmask.to(torch.bool)
    with torch.autocast("cuda", enabled=False):   # fp32 arithmetic also inside an autocast region
        s, w, k_hat, v_hat, kh = _weigh(q_ret, k, v, idx, valid, eps)
        return _gate(k, v, kh, w, k_hat, v_hat, _top2_margin(s, valid), budget_logits, write_mode, alpha_max,
                     tau_c, eps)


def retrieve_block_differentiable(q_ret: Tensor, k: Tensor, v: Tensor, budget_logits: Tensor, top_k: int,
                                  block_size: int, top_blocks: int, mode: str = "block_token",
                                  write_mode: str = "direct", alpha_max: float = 0.25, tau_c: float = 0.1,
                                  attention_mask: Optional[Tensor] = None, eps: float = 1e-6
                                  ) -> Tuple[Tensor, Tensor, Tensor, Dict[str, Tensor]]:
    """The block modes (modeling_sgsa.py:432-463, ``_tokens_from_blocks`` :296-345) in the
    form of ``retrieve_differentiable``.

    block_token: the block retrieval's token slots, a slot counting as selected where its
    weight is positive (the unused ones weigh exactly 0; a used slot whose weight
    underflows to 0 contributes nothing either way), then the weights over them and a
    margin of the two best selected scores (:310-337).  block_only: every token of the
    row's selected blocks that is causal and unpadded, each block once (:339-345), and the
    reference's margin of the first two block indices (``"scores":
    top_block_indices.float()``, :341, :369-372), a constant.
    """
    if mode not in ("block_token", "block_only"):
        raise ValueError(f"mode must be 'block_token' or 'block_only', got {mode!r}")
    B, T, H, D = q_ret.shape
    dev = q_ret.device
    nb = (T - 1) // block_size + 1 if T > 0 else 0
    eb = min(int(top_blocks), nb)
    n = min(int(top_k), T) if mode == "block_token" else eb * block_size
    _check(q_ret, n, write_mode, "retrieve_block_differentiable")
    with torch.no_grad():
        r = block_retrieve(q_ret.detach(), k.detach(), v.detach(), top_k, block_size, top_blocks, mode,
                           attention_mask=attention_mask, return_weights=mode == "block_token",
                           return_diagnostics=False)
        bidx = r["block_indices"]                                    # [B,H,T,eb]
        if mode == "block_token":
            idx = r["indices"]
            valid = r["weights"] > 0
        else:
            idx = (bidx.unsqueeze(-1) * block_size + torch.arange(block_size, device=dev)).reshape(B, H, T, n)
            pos = torch.arange(T, device=dev).view(1, 1, T, 1)
            valid = (idx <= pos) & (idx < T)
            if attention_mask is not None:
                am = attention_mask.to(dev).to(torch.bool)
                valid &= torch.gather(am.view(B, 1, 1, T).expand(B, H, T, T), 3, idx.clamp(0, T - 1))
                valid &= am.view(B, 1, T, 1)
            # a block listed twice (the slot fill repeats block 0) counts once
            dup = torch.zeros_like(bidx, dtype=torch.bool)
            for i in range(1, eb):
                dup[..., i] = (bidx[..., :i] == bidx[..., i:i + 1]).any(dim=-1)
            valid &= ~dup.repeat_interleave(block_size, dim=-1)
    with torch.autocast("cuda", enabled=False):   # fp32 arithmetic also inside an autocast region
        s, w, k_hat, v_hat, kh = _weigh(q_ret, k, v, idx, valid, eps)
        if mode == "block_token":
            margin = _top2_margin(s, valid)
        else:
            margin = (bidx[..., 0] - bidx[..., 1]).float() if eb >= 2 else torch.zeros(B, H, T, device=dev)
        return _gate(k, v, kh, w, k_hat, v_hat, margin, budget_logits, write_mode, alpha_max, tau_c, eps)
