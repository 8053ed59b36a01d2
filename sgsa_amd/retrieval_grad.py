"""Differentiable token_only retrieval and write gate, for training the SGSA block.

The inference path (``sgsa_layer_forward`` / ``sgsa_layer_retrieve``) selects,
weighs and gathers inside HIP kernels that have no backward.  Under autograd the
block takes this form instead, which keeps the reference's own structure
(modelings/modeling_sgsa.py:113-142 ``_token_only``, :361-382 ``_diagnostics``,
:497-504 ``_compute_alpha``, :543-551 the write key):

* the top-k selection is K1 on the GPU (``score_topk`` / ``score_topk_masked``,
  the same kernels and tie rule as the forward path) under ``no_grad``: the
  indices are constants of the step, as ``torch.topk``'s are for autograd in the
  reference;
* the scores of the selected keys, their softmax weights, k_hat and v_hat, the
  margin, concentration, novelty, the write key and alpha are then torch ops on
  the selected rows only ([B,H,T,k,D] gathers, the reference's expand+gather
  restricted to the k slots), so autograd reaches q_ret, k, v and the budget
  logits through every term, with no detach, as in the reference.

The selected rows cost B*H*T*k*D fp32 elements per tensor (K and V, plus their
gradients); calls above ``MAX_SELECTED_ELEMS`` raise instead of exhausting memory.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch
from torch import Tensor

from .retrieval import score_topk, score_topk_masked

__all__ = ["retrieve_differentiable", "MAX_SELECTED_ELEMS"]

MAX_SELECTED_ELEMS = 1 << 31   # B*H*T*k*D: 8 GB of fp32 per gathered tensor


def retrieve_differentiable(q_ret: Tensor, k: Tensor, v: Tensor, budget_logits: Tensor, top_k: int,
                            write_mode: str = "direct", alpha_max: float = 0.25, tau_c: float = 0.1,
                            attention_mask: Optional[Tensor] = None, eps: float = 1e-6
                            ) -> Tuple[Tensor, Tensor, Tensor, Dict[str, Tensor]]:
    """(write_key [B,T,H,D] in k's dtype, v_hat [B,T,H,D] in v's dtype, alpha [B,T,H] fp32,
    stats) for q_ret, k, v [B,T,H,D] and budget logits [B,T,H], differentiable in all four.

    ``stats`` holds "alpha" and "row_stats" [2,B,H,T] (the largest weight; |write key| /
    |k_hat| in the residual mode, else 0), as the inference path reports them.  The
    causal top-k runs with ``attention_mask`` [B,T] (nonzero = real token) on keys and
    queries, and each row keeps min(top_k, max(1, largest valid count)) slots
    (modeling_sgsa.py:159-160).
    """
    if write_mode not in ("direct", "residual"):
        raise ValueError(f"write_mode must be 'direct' or 'residual', got {write_mode!r}")
    if not q_ret.is_cuda:
        raise ValueError("retrieve_differentiable: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, T, H, D = q_ret.shape
    kk = min(int(top_k), T)
    if B * H * T * kk * D > MAX_SELECTED_ELEMS:
        raise ValueError(f"retrieve_differentiable: B*H*T*k*D = {B * H * T * kk * D} selected elements exceed "
                         f"{MAX_SELECTED_ELEMS}; train on shorter sequences or a smaller top_k")
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
        rows = (torch.arange(B * H, device=dev, dtype=torch.long).view(B, H, 1, 1) * T + idx.long()).reshape(-1)
    qh = q_ret.float().transpose(1, 2).contiguous()            # [B,H,T,D]
    kh = k.float().transpose(1, 2).contiguous()
    vh = v.float().transpose(1, 2).contiguous()
    ksel = kh.reshape(B * H * T, D).index_select(0, rows).view(B, H, T, kk, D)
    vsel = vh.reshape(B * H * T, D).index_select(0, rows).view(B, H, T, kk, D)
    # scores of the selected keys, in slot order (descending by K1's scores)
    s = torch.matmul(ksel, qh.unsqueeze(-1)).squeeze(-1) * (1.0 / math.sqrt(D))      # [B,H,T,kk]
    fmin = torch.finfo(torch.float32).min
    s = torch.where(valid, s, torch.full_like(s, fmin))
    w = torch.softmax(s, dim=-1) * valid.to(s.dtype)
    w = w / w.sum(dim=-1, keepdim=True).clamp_min(eps)
    k_hat = torch.matmul(w.unsqueeze(-2), ksel).squeeze(-2)    # [B,H,T,D]
    v_hat = torch.matmul(w.unsqueeze(-2), vsel).squeeze(-2)
    # _diagnostics (modeling_sgsa.py:368-381): margin of the two best slots, novelty of k_hat
    margin = s[..., 0] - s[..., 1] if kk >= 2 else torch.zeros_like(s[..., 0])
    conc = torch.sigmoid(margin / max(tau_c, eps))
    dot = (k_hat * kh).sum(dim=-1)
    self_norm = kh.norm(dim=-1).clamp_min(eps)
    kh_norm = k_hat.norm(dim=-1).clamp_min(eps)
    proj = dot / (self_norm * self_norm + eps)
    perp = k_hat - proj.unsqueeze(-1) * kh
    novelty = (perp.norm(dim=-1) / (kh_norm + eps)).clamp(0.0, 1.0)
    # write key (modeling_sgsa.py:543-550) and alpha (:497-504)
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
