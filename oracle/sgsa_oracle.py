"""CPU restatement of the SGSA layer-forward hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker the HIP kernels are
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; nothing under
``sgsa_amd/`` may, and the product path never falls back to it.

Everything here is plain PyTorch on the CPU, written from the reference's
behaviour (FAndromedA/sgsa, paths relative to the repository root):

* ``naive_recurrent_sgsa``  -- modelings/sgsa_ops/naive.py:10-57
* ``chunk_sgsa_fwd``        -- modelings/sgsa_ops/chunk_fwd.py:12-131 (torch branch)
* ``masked_topk``           -- modelings/modeling_sgsa.py:144-165, with the
                               tie rule fixed to (score desc, index asc)
* ``token_topk_retrieval``  -- modelings/modeling_sgsa.py:407-474, token_only
                               mode :113-142, diagnostics :361-405
* ``write_key`` / ``compute_alpha`` -- modelings/modeling_sgsa.py:543-552, :497-504
* ``rms_norm`` / ``gated_mlp`` / ``sgsa_model_forward`` -- the causal LM around the
                               layer, modelings/modeling_sgsa.py:634-749 (RMSNorm and
                               GatedMLP as restated in hybrid_dense_delta_topk.py:94-117)
* ``topk_kv_reuse_attention`` -- modelings/hybrid_dense_delta_topk.py:330-358
                               (V-only gather, ``finfo.min`` masking, no valid mask)
* ``make_inputs``           -- the seeded synthetic inputs of the benchmark configs

How each function is pinned (tests/test_oracle.py):

* recurrence: T=1 and T=2 closed forms written out by hand, the GDN transition
  form ``S_t = g_t (I - b k k^T) S_{t-1} + b k v^T`` (an algebraically different
  statement), decay-only and exact-overwrite special cases, and a planted
  mistake (sparse residual read from the updated state) that must fail;
* chunk form: equality with the recurrence for several chunk sizes including
  a ragged tail (the reference's own 1e-5 test), and state continuation;
  ``carry_dtype`` (the reference's bf16 state between chunks): the run equals
  its chunks run one at a time with the state rounded in between, bit for bit;
* top-k: brute force with Python ``sorted`` on tiny rows with ties and -0.0,
  causality, the t<k row counts and the padded-slot convention;
* retrieval/diagnostics/gate: explicit Python loops on tiny inputs, sums of
  weights, k_hat parallel/orthogonal novelty limits, alpha range and clip;
* model: RMSNorm and the SwiGLU MLP against scalar loops; a model with no
  layers is lm_head(norm(embedding + position)); one layer with zeroed o_proj
  and MLP leaves the residual stream unchanged, and with zeroed MLP equals the
  stream plus o_proj of the layer oracle's output.
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

__all__ = [
    "naive_recurrent_sgsa",
    "chunk_sgsa_fwd",
    "topk_lowest_index",
    "masked_topk",
    "token_topk_retrieval",
    "write_key",
    "compute_alpha",
    "sgsa_layer_forward",
    "topk_kv_reuse_attention",
    "make_inputs",
    "CONFIGS",
]


# ---------------------------------------------------------------------------
# Recurrence (parity target)
# ---------------------------------------------------------------------------

def naive_recurrent_sgsa(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    beta: Tensor,
    gamma: Tensor,
    sparse_k: Optional[Tensor] = None,
    sparse_v: Optional[Tensor] = None,
    alpha: Optional[Tensor] = None,
    initial_state: Optional[Tensor] = None,
    output_final_state: bool = False,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Token-by-token SGSA recurrence (modelings/sgsa_ops/naive.py:34-57).

    Per token: ``base = gamma_t * S``; the local residual and the sparse
    residual both read ``base`` (naive.py:40-53); output ``o_t = S^T q_t``
    (naive.py:55).  Shapes: q,k,v,sparse_* [B,T,H,D]; beta,gamma,alpha [B,T,H];
    state [B,H,Dk,Dv].  Computes in the dtype of ``q``.
    """
    bsz, seq_len, heads, dk = q.shape
    dv = v.shape[-1]
    if initial_state is None:
        state = q.new_zeros(bsz, heads, dk, dv)
    else:
        state = initial_state.to(q.dtype).clone()
    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    outs = []
    for t in range(seq_len):
        base = gamma[:, t, :, None, None] * state
        k_t, v_t = k[:, t], v[:, t]
        pred = torch.einsum("bhde,bhd->bhe", base, k_t)
        state = base + k_t[..., :, None] * ((v_t - pred) * beta[:, t, :, None])[..., None, :]
        if has_sparse:
            sk, sv = sparse_k[:, t], sparse_v[:, t]
            pred_s = torch.einsum("bhde,bhd->bhe", base, sk)
            state = state + sk[..., :, None] * ((sv - pred_s) * alpha[:, t, :, None])[..., None, :]
        outs.append(torch.einsum("bhde,bhd->bhe", state, q[:, t]))
    out = torch.stack(outs, dim=1) if outs else q.new_zeros(bsz, 0, heads, dv)
    return out, (state if output_final_state else None)


def chunk_sgsa_fwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    beta: Tensor,
    gamma: Tensor,
    sparse_k: Optional[Tensor] = None,
    sparse_v: Optional[Tensor] = None,
    alpha: Optional[Tensor] = None,
    initial_state: Optional[Tensor] = None,
    chunk_size: int = 64,
    output_final_state: bool = False,
    carry_dtype: Optional[torch.dtype] = None,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Chunked SGSA forward, torch branch of modelings/sgsa_ops/chunk_fwd.py:12-131.

    Virtual samples interleave (local, sparse) per token (chunk_fwd.py:53-56);
    ``D`` is the inclusive chunk-local cumprod of ``gamma.clamp_min(1e-6)``
    (:46, :70-71); ``rhs = nu - D_tau * (kappa S0)`` (:73-74); the transition
    ``T_ij = 1[tau_j < tau_i] lam_j D_tau_i / max(D_tau_j, 1e-6) (kappa_i . kappa_j)``
    (:86-87) is solved with ``solve_triangular`` (:89); readout uses the
    ``tau_i <= t`` mask (:120); the final state is :109-115.

    By default the state is carried between chunks in the compute dtype (fp32
    for low-precision inputs), as the kernels carry it.  ``carry_dtype``
    rounds it to that dtype after every chunk, which is what the reference
    does with q.dtype (the zero start state made in it, :34; ``state =
    state_h.to(q.dtype)`` after each chunk, :129): pass the inputs' dtype
    (bfloat16) to get the reference's own roundings of the carried state.  An
    initial state is taken as given (:34, :48) and the returned final state
    is the rounded one, upcast to the compute dtype.
    """
    bsz, seq_len, heads, dk = q.shape
    dv = v.shape[-1]
    cdt = torch.float32 if q.dtype in (torch.float16, torch.bfloat16) else q.dtype
    state = (q.new_zeros(bsz, heads, dk, dv, dtype=cdt) if initial_state is None
             else initial_state.to(cdt))
    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    outs = []
    for start in range(0, seq_len, chunk_size):
        end = min(start + chunk_size, seq_len)
        n = end - start
        qc = q[:, start:end].to(cdt)
        kc = k[:, start:end].to(cdt)
        vc = v[:, start:end].to(cdt)
        bc = beta[:, start:end].to(cdt)
        gc = gamma[:, start:end].to(cdt).clamp_min(1e-6)
        if has_sparse:
            kap = torch.stack((kc, sparse_k[:, start:end].to(cdt)), 2).reshape(bsz, 2 * n, heads, dk)
            nu = torch.stack((vc, sparse_v[:, start:end].to(cdt)), 2).reshape(bsz, 2 * n, heads, dv)
            lam = torch.stack((bc, alpha[:, start:end].to(cdt)), 2).reshape(bsz, 2 * n, heads)
            tau = torch.arange(n).repeat_interleave(2)
        else:
            kap, nu, lam, tau = kc, vc, bc, torch.arange(n)
        kap = kap.transpose(1, 2)           # [B,H,M,Dk]
        nu = nu.transpose(1, 2)             # [B,H,M,Dv]
        lam = lam.transpose(1, 2)           # [B,H,M]
        qh = qc.transpose(1, 2)             # [B,H,n,Dk]
        prefix = torch.cumprod(gc.transpose(1, 2), dim=-1)   # [B,H,n]
        ptau = prefix[..., tau]                              # [B,H,M]
        rhs = nu - ptau[..., None] * torch.einsum("bhde,bhmd->bhme", state, kap)
        gram = kap @ kap.transpose(-1, -2)
        dep = (tau[None, :] < tau[:, None]).to(cdt)
        decay = ptau[..., :, None] / ptau[..., None, :].clamp_min(1e-6)
        trans = dep * lam[..., None, :] * decay * gram
        eye = torch.eye(kap.shape[2], dtype=cdt)
        resid = torch.linalg.solve_triangular(trans + eye, rhs, upper=False)
        # readout: o_t = D_t S0^T q_t + sum_{tau_i <= t} lam_i D_t / D_tau_i (q_t.kappa_i) R_i
        read_mask = (tau[None, :] <= torch.arange(n)[:, None]).to(cdt)          # [n,M]
        read_w = read_mask * lam[..., None, :] * (prefix[..., :, None] / ptau[..., None, :].clamp_min(1e-6))
        qk = qh @ kap.transpose(-1, -2)                                         # [B,H,n,M]
        o = prefix[..., None] * (qh @ state) + (qk * read_w) @ resid
        outs.append(o.transpose(1, 2).to(q.dtype))
        final = prefix[..., -1]
        tail = final[..., None] / ptau.clamp_min(1e-6)
        state = final[..., None, None] * state + kap.transpose(-1, -2) @ (resid * (lam * tail)[..., None])
        if carry_dtype is not None:
            state = state.to(carry_dtype).to(cdt)
    out = torch.cat(outs, dim=1) if outs else q.new_zeros(bsz, 0, heads, dv)
    return out, (state if output_final_state else None)


# ---------------------------------------------------------------------------
# Retrieval (token_only)
# ---------------------------------------------------------------------------

def topk_lowest_index(x: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    """Exact top-k of each row of a 2-D tensor, ordered (value desc, index asc).

    ``torch.topk`` is used only for the k-th value (which is tie-independent);
    membership then takes every element above it plus the lowest-index elements
    equal to it, and a stable descending sort orders the result.  -0.0 and +0.0
    compare equal, as IEEE comparison (and torch.topk) treat them.
    """
    rows, n = x.shape
    if k == 0 or rows == 0:
        return x.new_zeros(rows, k), torch.zeros(rows, k, dtype=torch.long)
    kth = torch.topk(x, k, dim=-1, largest=True, sorted=True).values[:, k - 1:k]
    above = x > kth
    eq = x == kth
    need = k - above.sum(-1, keepdim=True)
    eq_rank = torch.cumsum(eq.to(torch.int64), dim=-1) - 1
    sel = above | (eq & (eq_rank < need))
    idx = torch.nonzero(sel)[:, 1].reshape(rows, k)            # ascending per row
    vals = x.gather(1, idx)
    order = torch.sort(vals, dim=-1, descending=True, stable=True).indices
    return vals.gather(1, order), idx.gather(1, order)


def masked_topk(scores: Tensor, valid_mask: Tensor, topk: int) -> Tuple[Tensor, Tensor, Tensor]:
    """Fixed-size masked top-k (modelings/modeling_sgsa.py:144-165).

    Invalid entries are filled with ``finfo(dtype).min`` (:150, :158).  The row
    count ``k_q = min(topk, max(valid_count, 1))`` uses the maximum valid count
    over (B,H) (:159-160).  Slots >= k_q keep score=min, index=0, valid=False
    (:151-153).  Ties are broken by lowest index (the reference leaves this to
    torch.topk; the port fixes it).
    scores/valid_mask: [B,H,Q,K].  Returns scores [B,H,Q,topk], int64 indices,
    bool valid.
    """
    bsz, heads, qn, kn = scores.shape
    fmin = torch.finfo(scores.dtype).min
    masked = scores.masked_fill(~valid_mask, fmin)
    vc = valid_mask.sum(-1).amax(dim=(0, 1))                          # [Q]
    kq = torch.clamp(torch.clamp(vc, min=1), max=topk)                # [Q]
    vals, idx = topk_lowest_index(masked.reshape(-1, kn), topk)
    vals = vals.reshape(bsz, heads, qn, topk)
    idx = idx.reshape(bsz, heads, qn, topk)
    valid = valid_mask.gather(-1, idx)
    slot = torch.arange(topk)
    live = slot[None, None, None, :] < kq[None, None, :, None]
    vals = torch.where(live, vals, torch.full_like(vals, fmin))
    idx = torch.where(live, idx, torch.zeros_like(idx))
    valid = valid & live
    return vals, idx, valid


def token_topk_retrieval(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    top_k: int,
    causal: bool = True,
    attention_mask: Optional[Tensor] = None,
    tau_c: float = 0.1,
    local_window: int = 64,
    sink_size: int = 8,
    eps: float = 1e-6,
    block_rows: int = 256,
    rows: Optional[Tuple[int, int]] = None,
) -> Dict[str, object]:
    """Token top-k retrieval (SparseRetriever.forward, modelings/modeling_sgsa.py:407-474).

    Scores ``q k^T / sqrt(d)`` (:420) are computed query-block by query-block
    (the reference materialises [B,H,T,T]); valid mask is causal & key/query
    padding (:421-428); weights are ``softmax(fp32 scores) * valid`` renormalised
    with ``clamp_min(eps)`` (:126-128); k_hat/v_hat are weighted sums of the
    selected rows (:130-134).  Diagnostics follow :361-405 with
    ``self_key = k`` (:459).  Inputs [B,T,H,D]; k_hat/v_hat returned [B,T,H,D];
    everything else [B,H,T,*].  ``rows=(r0, r1)`` restricts the work to those
    query rows (used to time a bounded sample); outputs then cover only them.
    """
    bsz, seq_len, heads, dk = q.shape
    dtype = q.dtype
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    topk = min(top_k, seq_len)
    sc = math.sqrt(dk)
    out_scores = []
    out_idx = []
    out_w = []
    out_kh = []
    out_vh = []
    pos = torch.arange(seq_len)
    key_valid = attention_mask.to(torch.bool) if attention_mask is not None else None
    row_lo, row_hi = rows if rows is not None else (0, seq_len)
    for r0 in range(row_lo, row_hi, block_rows):
        r1 = min(row_hi, r0 + block_rows)
        scores = torch.matmul(qh[:, :, r0:r1], kh.transpose(-2, -1)) / sc
        if causal:
            valid = (pos[None, :] <= pos[r0:r1, None])[None, None].expand(bsz, heads, -1, -1)
        else:
            valid = torch.ones(bsz, heads, r1 - r0, seq_len, dtype=torch.bool)
        if key_valid is not None:
            valid = valid & key_valid[:, None, None, :] & key_valid[:, None, r0:r1, None]
        ts, ti, tv = masked_topk(scores, valid, topk)
        w = F.softmax(ts.float(), dim=-1).to(dtype)
        w = w * tv.to(dtype)
        w = w / w.sum(-1, keepdim=True).clamp_min(eps)
        gk = kh[:, :, None, :, :].expand(-1, -1, r1 - r0, -1, -1).gather(
            3, ti[..., None].expand(-1, -1, -1, -1, dk))
        gv = vh[:, :, None, :, :].expand(-1, -1, r1 - r0, -1, -1).gather(
            3, ti[..., None].expand(-1, -1, -1, -1, vh.shape[-1]))
        out_kh.append((w[..., None] * gk).sum(3))
        out_vh.append((w[..., None] * gv).sum(3))
        out_scores.append(ts)
        out_idx.append(ti)
        out_w.append(w)
    scores = torch.cat(out_scores, 2)
    idx = torch.cat(out_idx, 2)
    weights = torch.cat(out_w, 2)
    k_hat = torch.cat(out_kh, 2)                   # [B,H,T,D]
    v_hat = torch.cat(out_vh, 2)
    diag = retrieval_diagnostics(scores, weights, idx, k_hat, kh[:, :, row_lo:row_hi], tau_c, local_window,
                                 sink_size, eps, row_offset=row_lo)
    return {
        "indices": idx,
        "block_indices": None,
        "weights": weights,
        "scores": scores,
        "k_hat": k_hat.transpose(1, 2),
        "v_hat": v_hat.transpose(1, 2),
        "diagnostics": diag,
    }


def block_retrieval(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    top_k: int,
    block_size: int,
    top_blocks: int,
    mode: str = "block_token",
    causal: bool = True,
    tau_c: float = 0.1,
    local_window: int = 64,
    sink_size: int = 8,
    eps: float = 1e-6,
    attention_mask: Optional[Tensor] = None,
) -> Dict[str, object]:
    """Block retrieval modes of SparseRetriever.forward on its torch path (no flash_moba;
    modelings/modeling_sgsa.py:444-463), causal or not (:423-424), with an optional
    padding mask [B,T] folded into the valid mask for keys and queries (:425-428).

    Scores ``q k^T / sqrt(d)`` (:420).  Block b holds keys [b bs, (b+1) bs)
    (:167-170); its score is the max over its causal keys, finfo.min when it has
    none (:172-186); the row keeps the top ``top_blocks`` blocks through the masked
    top-k (:188-195, lowest index on ties).  Candidates are the causal keys of the
    kept blocks (:313-320).  ``block_token``: the masked top-k of the candidates,
    softmax weights times validity, renormalised (:322-344).  ``block_only``:
    softmax over every key of the row with non-candidates at finfo.min, times the
    candidate mask, renormalised, so k_hat / v_hat are dense products (:346-359);
    its diagnostics read the kept block indices as the selected scores and have no
    token indices (:360-361, :455-463).  Inputs [B,T,H,D]; returns the dict of
    token_topk_retrieval (k_hat / v_hat [B,T,H,D], the rest [B,H,T,*]).
    """
    if mode not in ("block_only", "block_token"):
        raise ValueError(f"mode must be block_only or block_token, got {mode!r}")
    B, T, H, D = q.shape
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    scores = torch.matmul(qh, kh.transpose(-2, -1)) / math.sqrt(D)
    pos = torch.arange(T)
    valid = (pos[None, :] <= pos[:, None]) if causal else torch.ones(T, T, dtype=torch.bool)
    valid = valid[None, None].expand(B, H, T, T)
    if attention_mask is not None:
        am = attention_mask.to(torch.bool)
        valid = valid & am[:, None, None, :] & am[:, None, :, None]
    fmin = torch.finfo(scores.dtype).min
    block_ids = pos // block_size
    nb = int(block_ids.max().item()) + 1
    bscores = scores.new_full((B, H, T, nb), fmin)
    for blk in range(nb):
        tm = block_ids == blk
        bscores[..., blk] = scores[..., tm].masked_fill(~valid[..., tm], fmin).max(dim=-1).values
    bvalid = bscores > fmin / 2
    _, bidx, _ = masked_topk(bscores, bvalid, min(top_blocks, nb))
    in_sel = (block_ids.view(1, 1, 1, T, 1) == bidx.unsqueeze(-2)).any(dim=-1)
    cmask = valid & in_sel
    cscores = scores.masked_fill(~cmask, fmin)
    if mode == "block_token":
        ts, ti, tv = masked_topk(cscores, cmask, min(top_k, T))
        w = F.softmax(ts.float(), dim=-1).to(scores.dtype) * tv.to(scores.dtype)
        w = w / w.sum(-1, keepdim=True).clamp_min(eps)
        gk = kh[:, :, None].expand(-1, -1, T, -1, -1).gather(3, ti[..., None].expand(-1, -1, -1, -1, D))
        gv = vh[:, :, None].expand(-1, -1, T, -1, -1).gather(3, ti[..., None].expand(-1, -1, -1, -1, vh.shape[-1]))
        k_hat, v_hat = (w[..., None] * gk).sum(3), (w[..., None] * gv).sum(3)
        diag = retrieval_diagnostics(ts, w, ti, k_hat, kh, tau_c, local_window, sink_size, eps)
        sel_scores, indices = ts, ti
    else:
        w = F.softmax(cscores.float(), dim=-1).to(scores.dtype) * cmask.to(scores.dtype)
        w = w / w.sum(-1, keepdim=True).clamp_min(eps)
        k_hat, v_hat = torch.matmul(w, kh), torch.matmul(w, vh)
        sel_scores, indices = bidx.float(), None
        diag = retrieval_diagnostics(sel_scores, w, torch.zeros(B, H, T, 1, dtype=torch.long), k_hat, kh, tau_c,
                                     local_window, sink_size, eps)
        for name in ("avg_distance", "local_ratio", "sink_ratio", "remote_ratio"):
            del diag[name]
    return {
        "indices": indices,
        "block_indices": bidx,
        "block_scores": bscores,
        "weights": w,
        "scores": sel_scores,
        "k_hat": k_hat.transpose(1, 2),
        "v_hat": v_hat.transpose(1, 2),
        "diagnostics": diag,
    }


def retrieval_diagnostics(
    scores: Tensor,
    weights: Tensor,
    indices: Tensor,
    k_hat: Tensor,
    self_key: Tensor,
    tau_c: float = 0.1,
    local_window: int = 64,
    sink_size: int = 8,
    eps: float = 1e-6,
    row_offset: int = 0,
) -> Dict[str, Tensor]:
    """SparseRetriever._diagnostics (modelings/modeling_sgsa.py:361-405).  [B,H,T,*] layout.

    ``row_offset`` is the query position of the first row (0 for a full pass).
    """
    if scores.shape[-1] >= 2:
        margin = scores[..., 0] - scores[..., 1]
    else:
        margin = torch.zeros_like(scores[..., 0])
    concentration = torch.sigmoid(margin / max(tau_c, eps))
    max_conf = weights.max(dim=-1).values
    dot = (k_hat * self_key).sum(-1)
    self_norm = self_key.norm(dim=-1).clamp_min(eps)
    kh_norm = k_hat.norm(dim=-1).clamp_min(eps)
    proj = dot / (self_norm * self_norm + eps)
    k_perp = k_hat - proj[..., None] * self_key
    novelty = (k_perp.norm(dim=-1) / (kh_norm + eps)).clamp(0.0, 1.0)
    conflict = (dot / (self_norm * kh_norm + eps)).clamp(-1.0, 1.0)
    wc = weights.clamp_min(eps)
    entropy = -(wc * wc.log()).sum(-1)
    out = {
        "score_margin": margin,
        "concentration": concentration,
        "max_confidence": max_conf,
        "novelty": novelty,
        "write_conflict": conflict,
        "entropy": entropy,
    }
    seq_len = int(indices.max().item()) + 1 if indices.numel() > 0 else 1
    qpos = torch.arange(row_offset, row_offset + indices.shape[2]).view(1, 1, -1, 1)
    dist = (qpos - indices).clamp_min(0)
    out["avg_distance"] = dist.float().mean(-1) / max(seq_len, 1)
    out["local_ratio"] = (dist <= local_window).float().mean(-1)
    out["sink_ratio"] = (indices < sink_size).float().mean(-1)
    out["remote_ratio"] = ((dist > local_window) & (indices >= sink_size)).float().mean(-1)
    return out


# ---------------------------------------------------------------------------
# Write gate (SGSAStateLayer)
# ---------------------------------------------------------------------------

def write_key(k_hat: Tensor, k: Tensor, mode: str = "direct", eps: float = 1e-6) -> Tensor:
    """Write key of SGSAStateLayer.forward (modelings/modeling_sgsa.py:546-551)."""
    if mode == "direct":
        return k_hat
    if mode == "residual":
        dot = (k_hat * k).sum(-1)
        nsq = (k * k).sum(-1).clamp_min(eps)
        return k_hat - (dot / nsq)[..., None] * k
    raise ValueError(f"unknown write mode {mode!r}")


def compute_alpha(
    concentration: Tensor,
    novelty: Tensor,
    budget_logits: Tensor,
    wkey: Tensor,
    v_hat: Tensor,
    alpha_max: float = 0.25,
) -> Tensor:
    """SGSAStateLayer._compute_alpha (modelings/modeling_sgsa.py:497-504).

    concentration/novelty [B,H,T]; budget_logits [B,T,H] (the output of
    ``budget_proj``, before the sigmoid); wkey/v_hat [B,T,H,D].  Returns [B,T,H].
    """
    c = concentration.transpose(1, 2)
    n = novelty.transpose(1, 2).clamp(0.0, 1.0)
    a = alpha_max * c * n * torch.sigmoid(budget_logits)
    proxy = a * v_hat.norm(dim=-1) * wkey.norm(dim=-1)
    clip = torch.clamp(1.0 / proxy.clamp_min(1.0), max=1.0)
    return a * clip


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
    use_chunk: bool = False,
    chunk_size: int = 64,
    block_rows: int = 256,
    attention_mask: Optional[Tensor] = None,
    retrieval_mode: str = "token_only",
    block_size: int = 32,
    top_blocks: int = 2,
) -> Dict[str, Tensor]:
    """Op-level SGSA layer forward: retrieval -> gate -> state update.

    Mirrors SGSABlock.forward's attention half (modelings/modeling_sgsa.py:669-684)
    with the projections taken as inputs: retrieval on (q_ret, k, v) under the
    optional padding mask [B,T] (:672-675 pass it to the retriever only) --
    ``retrieval_mode`` token_only (:430-431) or block_only / block_token
    (``block_retrieval``, :432-463) -- write key and alpha (:543-552), then the
    recurrent state update (naive.py, or the chunk form when ``use_chunk``).
    ``write_mode`` "none" keeps the write key k_hat for alpha (:546-550) and
    leaves the sparse write out of the update (:557-609).  Inputs are upcast to fp32.
    """
    f = lambda x: None if x is None else x.float()
    q, k, v, q_ret, beta, gamma, budget_logits = map(f, (q, k, v, q_ret, beta, gamma, budget_logits))
    if retrieval_mode == "token_only":
        ret = token_topk_retrieval(q_ret, k, v, top_k, tau_c=tau_c, block_rows=block_rows,
                                   attention_mask=attention_mask)
    else:
        ret = block_retrieval(q_ret, k, v, top_k, block_size, top_blocks, retrieval_mode, causal=True,
                              tau_c=tau_c, attention_mask=attention_mask)
    if write_mode not in ("none", "direct", "residual"):
        raise ValueError(f"unknown write mode {write_mode!r}")
    wk = write_key(ret["k_hat"], k, "residual" if write_mode == "residual" else "direct")
    alpha = compute_alpha(ret["diagnostics"]["concentration"], ret["diagnostics"]["novelty"],
                          budget_logits, wk, ret["v_hat"], alpha_max)
    sp = (wk, ret["v_hat"], alpha) if write_mode != "none" else (None, None, None)
    if use_chunk:
        o, st = chunk_sgsa_fwd(q, k, v, beta, gamma, *sp, f(initial_state), chunk_size, True)
    else:
        o, st = naive_recurrent_sgsa(q, k, v, beta, gamma, *sp, f(initial_state), True)
    return {"o": o, "final_state": st, "write_key": wk, "v_hat": ret["v_hat"],
            "alpha": alpha, "retrieval": ret}


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
    eps: float = 1e-6,
) -> Tuple[Tensor, Tensor, Tuple[Tensor, Tensor]]:
    """One generated token of the layer, with optional top-k reuse.

    The token's retrieval over the cache k_cache/v_cache [B,Tc,H,D] (ending with
    the token; causal, so every cached key is valid), its write key and gate,
    and one recurrent update, as ``sgsa_layer_forward`` does at that position
    (modelings/modeling_sgsa.py:669-684 with the recurrent backend).  Without
    ``candidates`` the keys are the exact top-k (lowest index on ties).  With
    candidates (indices [B,H,1,n], counts [B,H,1]) selected by an earlier step,
    those keys are re-scored for this query (modelings/idea.md:395-401) and
    ordered by score, ties by index, before the weights, the diagnostics and
    the gate.  Inputs are upcast to fp32.  Returns (o [B,1,H,D], state, the
    step's candidates).
    """
    f = lambda x: x.float()
    q, k, v, q_ret, beta, gamma, budget_logits, kc, vc, state = map(
        f, (q, k, v, q_ret, beta, gamma, budget_logits, k_cache, v_cache, state))
    B, Tc, H, D = kc.shape
    qh = q_ret.transpose(1, 2)                                     # [B,H,1,D]
    kh, vh = kc.transpose(1, 2), vc.transpose(1, 2)                # [B,H,Tc,D]
    scores = torch.matmul(qh, kh.transpose(-2, -1)) / math.sqrt(D)   # [B,H,1,Tc]
    if candidates is None:
        kk = min(top_k, Tc)
        ts, ti, _ = masked_topk(scores, torch.ones_like(scores, dtype=torch.bool), kk)
        cnt = torch.full((B, H, 1), kk, dtype=torch.int32)
        cand = (ti.to(torch.int32), cnt)
    else:
        cidx, cnt = candidates
        n = int(cnt.min().item())
        if int(cnt.max().item()) != n:
            raise ValueError("the oracle takes candidates with one count for every row")
        # in key-index order, so that ordering by (score desc, position asc) is (score desc, index asc)
        ci = torch.sort(cidx[..., :n].long(), dim=-1).values
        cs = scores.gather(-1, ci)
        vals, pos = topk_lowest_index(cs.reshape(-1, n), n)
        ts = vals.reshape(B, H, 1, n)
        ti = ci.reshape(-1, n).gather(1, pos).reshape(B, H, 1, n)
        cand = (cidx, cnt)
    w = F.softmax(ts, dim=-1)
    w = w / w.sum(-1, keepdim=True).clamp_min(eps)
    gk = kh.gather(2, ti[..., 0, :, None].expand(-1, -1, -1, D))       # [B,H,n,D]
    gv = vh.gather(2, ti[..., 0, :, None].expand(-1, -1, -1, D))
    k_hat = (w[..., 0, :, None] * gk).sum(2)[:, :, None]               # [B,H,1,D]
    v_hat = (w[..., 0, :, None] * gv).sum(2)[:, :, None]
    diag = retrieval_diagnostics(ts, w, ti, k_hat, k.transpose(1, 2), tau_c, eps=eps, row_offset=Tc - 1)
    kh_t, vh_t = k_hat.transpose(1, 2), v_hat.transpose(1, 2)          # [B,1,H,D]
    wk = write_key(kh_t, k, write_mode)
    alpha = compute_alpha(diag["concentration"], diag["novelty"], budget_logits, wk, vh_t, alpha_max)
    o, st = naive_recurrent_sgsa(q, k, v, beta, gamma, wk, vh_t, alpha, state, True)
    return o, st, cand


# ---------------------------------------------------------------------------
# The causal LM around the layer (SGSABlock / SGSAForCausalLM)
# ---------------------------------------------------------------------------

def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight: the fla-core RMSNorm that modeling_sgsa.py:40
    imports, as the reference restates it in modelings/hybrid_dense_delta_topk.py:94-103."""
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * weight


def gated_mlp(x: Tensor, w_gate: Tensor, w_up: Tensor, w_down: Tensor) -> Tensor:
    """down(silu(gate x) * up x): fla-core GatedMLP with SwiGLU (modeling_sgsa.py:651-657), as
    restated in modelings/hybrid_dense_delta_topk.py:106-117."""
    return (F.silu(x @ w_gate.T) * (x @ w_up.T)) @ w_down.T


def sgsa_model_forward(params: Dict[str, Tensor], input_ids: Tensor, *, num_layers: int, num_heads: int,
                       top_k: int, eps: float = 1e-6, write_mode: str = "direct", alpha_max: float = 0.25,
                       tau_c: float = 0.1, sparse_output_lambda: float = 0.0,
                       act_dtype: Optional[torch.dtype] = None, attention_mask: Optional[Tensor] = None,
                       return_metrics: bool = False, retrieval_mode: str = "token_only", block_size: int = 32,
                       top_blocks: int = 2):
    """Logits of SGSAForCausalLM.forward (modelings/modeling_sgsa.py:735-749) in fp32.

    ``params`` uses the parameter names of sgsa_amd.model.SGSAForCausalLM, which follow
    the reference's modules: embedding + learned position embedding (:739), per block
    (:669-709) RMSNorm, q/k/v/q_ret projections, the gates of SGSAStateLayer
    (beta = sigmoid(.).clamp_min(1e-4), gamma = sigmoid(.), budget logits; :584-585,
    :501), the retrieval in ``retrieval_mode`` (token_only, block_only, block_token with
    ``block_size`` / ``top_blocks``) and the state update (``sgsa_layer_forward``; every
    linear_backend of :554-609 computes this recurrence), o_proj,
    the optional sparse output (:689-692), the residual MLP (:695), then the final
    RMSNorm and lm_head (:746).

    ``act_dtype`` (e.g. bfloat16) rounds every activation a model in that dtype stores
    -- each projection, norm, MLP product and residual sum -- while the arithmetic
    stays fp32, so that a low-precision model is compared on the inputs it actually
    feeds each layer.

    ``attention_mask`` [B,T] zeroes the padded embeddings (:740-741) and goes to
    every layer's retrieval (:668-674).  ``return_metrics``: returns (logits,
    metrics) with the per-layer metrics of :697-708 / :744-752 --
    alpha_mean, k_hat_perp_ratio_mean ((|k_hat_perp| / max(|k_hat|, eps))
    clamped to [0, 10], residual mode only; :546-551, :614) and
    retrieval_confidence_mean (mean max weight, :374).
    """
    P = {k: v.float() for k, v in params.items()}
    r = (lambda x: x) if act_dtype is None else (lambda x: x.to(act_dtype).float())
    B, T = input_ids.shape
    h = r(P["embed_tokens.weight"][input_ids] + P["pos_embed.weight"][:T][None])
    if attention_mask is not None:
        h = h * attention_mask.to(torch.bool).float()[..., None]
    metrics = {}
    C = h.shape[-1]
    H, D = num_heads, C // num_heads
    for i in range(num_layers):
        w = lambda n: P[f"layers.{i}.{n}"]
        n = r(rms_norm(h, w("input_norm.weight"), eps))
        q = r(n @ w("q_proj.weight").T).view(B, T, H, D)
        k = r(n @ w("k_proj.weight").T).view(B, T, H, D)
        v = r(n @ w("v_proj.weight").T).view(B, T, H, D)
        q_ret = r(n @ w("q_ret_proj.weight").T).view(B, T, H, D)
        beta = torch.sigmoid(r(n @ w("beta_proj.weight").T + w("beta_proj.bias"))).clamp_min(1e-4)
        gamma = torch.sigmoid(r(n @ w("gamma_proj.weight").T + w("gamma_proj.bias")))
        budget = r(n @ w("budget_proj.weight").T + w("budget_proj.bias"))
        lay = sgsa_layer_forward(q, k, v, q_ret, beta, gamma, budget, top_k, write_mode=write_mode,
                                 alpha_max=alpha_max, tau_c=tau_c, attention_mask=attention_mask,
                                 retrieval_mode=retrieval_mode, block_size=block_size, top_blocks=top_blocks)
        kh = lay["retrieval"]["k_hat"]
        metrics[f"layer_{i}_alpha_mean"] = lay["alpha"].mean()
        metrics[f"layer_{i}_k_hat_perp_ratio_mean"] = (
            (lay["write_key"].norm(dim=-1) / kh.norm(dim=-1).clamp_min(1e-6)).clamp(0.0, 10.0).mean()
            if write_mode == "residual" else torch.zeros(()))
        metrics[f"layer_{i}_retrieval_confidence_mean"] = lay["retrieval"]["diagnostics"]["max_confidence"].mean()
        out = r(r(lay["o"]).reshape(B, T, C) @ w("o_proj.weight").T)
        if sparse_output_lambda > 0:
            sp = r(r(lay["v_hat"]).reshape(B, T, C) @ w("sparse_out_proj.weight").T)
            out = r(out + r(sparse_output_lambda * sp))
        h = r(h + out)
        m = r(rms_norm(h, w("post_attn_norm.weight"), eps))
        gate, up = r(m @ w("mlp.gate_proj.weight").T), r(m @ w("mlp.up_proj.weight").T)
        h = r(h + r(r(r(F.silu(gate)) * up) @ w("mlp.down_proj.weight").T))
    head = P.get("lm_head.weight", P["embed_tokens.weight"])
    logits = r(r(rms_norm(h, P["norm.weight"], eps)) @ head.T)
    return (logits, metrics) if return_metrics else logits


# ---------------------------------------------------------------------------
# Config 4: the hybrid decoder (SGSA blocks and dense GQA attention blocks)
# ---------------------------------------------------------------------------

def rope_apply(x: Tensor, pos: Tensor, theta: float = 10000.0, act_dtype=None) -> Tensor:
    """Rotary embedding of x [B, heads, T, D] at positions pos [T], in the rotate-half
    form of modelings/hybrid_dense_delta_topk.py:124-150 (fp32).  ``act_dtype``: a model
    in that dtype -- the cos / sin tables stored in it (:134-136) and each product and
    the sum rounded to it (:150)."""
    D = x.shape[-1]
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    f = torch.outer(pos.float(), inv_freq)
    emb = torch.cat((f, f), dim=-1)
    rot = torch.cat((-x[..., D // 2:], x[..., :D // 2]), dim=-1)
    if act_dtype is None:
        return x * emb.cos() + rot * emb.sin()
    r = lambda t: t.to(act_dtype).float()
    return r(r(x * r(emb.cos())) + r(rot * r(emb.sin())))


def dense_gqa_attention(q: Tensor, k: Tensor, v: Tensor, q_pos: Tensor, act_dtype=None) -> Tensor:
    """Causal softmax attention (:178-192) with grouped key/value heads: q [B, H, Tq, D]
    at positions q_pos [Tq]; k, v [B, Hkv, Tk, D] at positions 0 .. Tk-1; query head h
    reads key/value head h // (H / Hkv).  ``act_dtype``: the roundings of a model in that
    dtype -- the product q k^T and its scaling by 1/sqrt(D) each rounded (:186-187), the
    fp32 softmax's probabilities rounded (:190), the output rounded."""
    H, Hkv, D = q.shape[1], k.shape[1], q.shape[-1]
    r = (lambda x: x) if act_dtype is None else (lambda x: x.to(act_dtype).float())
    kk = k.repeat_interleave(H // Hkv, dim=1)
    vv = v.repeat_interleave(H // Hkv, dim=1)
    if act_dtype is None:
        s = torch.matmul(q, kk.transpose(-1, -2)) / math.sqrt(D)
    else:   # a low-precision tensor times a Python float: the product in fp32, rounded once
        s = r(r(torch.matmul(q, kk.transpose(-1, -2))) * (1.0 / math.sqrt(D)))
    s = s.masked_fill(torch.arange(k.shape[2])[None, :] > q_pos[:, None], float("-inf"))
    return r(torch.matmul(r(torch.softmax(s, dim=-1)), vv))


def hybrid_generate(params: Dict[str, Tensor], prompt_ids: Tensor, decode_ids: Tensor, *, num_layers: int,
                    num_heads: int, num_kv_heads: int, dense_every: int, top_k: int, recompute_every: int,
                    rope_theta: float = 10000.0, eps: float = 1e-6, write_mode: str = "direct",
                    alpha_max: float = 0.25, tau_c: float = 0.1,
                    act_dtype: Optional[torch.dtype] = None) -> Tuple[Tensor, Tensor]:
    """Logits of the config-4 hybrid decoder in fp32: the prompt [B, T] in one pass, then
    the tokens decode_ids [B, n] one at a time (token s at position T + s).

    Layer i is a dense GQA attention block when i % dense_every == 0
    (modelings/hybrid_dense_delta_topk.py:195-244, :394-437, dense every 4th at :398)
    and an SGSA block otherwise (SGSABlock, modelings/modeling_sgsa.py:669-709): the
    prompt through ``sgsa_layer_forward``, each decoded token through
    ``sgsa_decode_step``, which selects its top-k when s % recompute_every == 0 and
    re-scores the layer's kept candidates otherwise.  ``params`` uses the names of
    sgsa_amd.hybrid.HybridForCausalLM.  Returns (prompt logits [B, T, V], decode
    logits [B, n, V]).

    ``act_dtype`` (e.g. bfloat16) rounds every activation a model in that dtype
    stores -- embeddings, norms, projections, the rotary embedding, the attention's
    scores, probabilities and output, the SGSA layer's output, the MLP's products and
    each residual sum -- while the arithmetic stays fp32, as sgsa_model_forward does.
    """
    P = {k: v.float() for k, v in params.items()}
    r = (lambda x: x) if act_dtype is None else (lambda x: x.to(act_dtype).float())
    B, T = prompt_ids.shape
    C = P["embed_tokens.weight"].shape[1]
    H, Hkv = num_heads, num_kv_heads
    D = C // H
    head = P.get("lm_head.weight", P["embed_tokens.weight"])
    caches: List[dict] = [dict() for _ in range(num_layers)]

    def mlp(i, h):
        w = lambda n: P[f"layers.{i}.{n}"]
        m = r(rms_norm(h, w("post_attn_norm.weight"), eps))
        gate, up = r(m @ w("mlp.gate_proj.weight").T), r(m @ w("mlp.up_proj.weight").T)
        return r(h + r(r(r(F.silu(gate)) * up) @ w("mlp.down_proj.weight").T))

    def run(ids: Tensor, pos0: int, step: Optional[int]) -> Tensor:
        n_t = ids.shape[1]
        h = r(P["embed_tokens.weight"][ids])
        pos = torch.arange(pos0, pos0 + n_t)
        for i in range(num_layers):
            w = lambda n: P[f"layers.{i}.{n}"]
            c = caches[i]
            nrm = r(rms_norm(h, w("input_norm.weight"), eps))
            if i % dense_every == 0:
                q = rope_apply(r(nrm @ w("q_proj.weight").T).view(B, n_t, H, D).transpose(1, 2), pos, rope_theta,
                               act_dtype)
                k = rope_apply(r(nrm @ w("k_proj.weight").T).view(B, n_t, Hkv, D).transpose(1, 2), pos, rope_theta,
                               act_dtype)
                v = r(nrm @ w("v_proj.weight").T).view(B, n_t, Hkv, D).transpose(1, 2)
                c["k"] = k if step is None else torch.cat((c["k"], k), dim=2)
                c["v"] = v if step is None else torch.cat((c["v"], v), dim=2)
                att = dense_gqa_attention(q, c["k"], c["v"], pos, act_dtype)
                h = r(h + r(att.transpose(1, 2).reshape(B, n_t, C) @ w("o_proj.weight").T))
            else:
                q = r(nrm @ w("q_proj.weight").T).view(B, n_t, H, D)
                k = r(nrm @ w("k_proj.weight").T).view(B, n_t, H, D)
                v = r(nrm @ w("v_proj.weight").T).view(B, n_t, H, D)
                q_ret = r(nrm @ w("q_ret_proj.weight").T).view(B, n_t, H, D)
                beta = torch.sigmoid(r(nrm @ w("beta_proj.weight").T + w("beta_proj.bias"))).clamp_min(1e-4)
                gamma = torch.sigmoid(r(nrm @ w("gamma_proj.weight").T + w("gamma_proj.bias")))
                budget = r(nrm @ w("budget_proj.weight").T + w("budget_proj.bias"))
                if step is None:
                    lay = sgsa_layer_forward(q, k, v, q_ret, beta, gamma, budget, top_k, write_mode=write_mode,
                                             alpha_max=alpha_max, tau_c=tau_c)
                    o = lay["o"]
                    c["k"], c["v"], c["state"], c["cand"] = k, v, lay["final_state"], None
                else:
                    c["k"] = torch.cat((c["k"], k), dim=1)
                    c["v"] = torch.cat((c["v"], v), dim=1)
                    select = step % recompute_every == 0 or c["cand"] is None
                    o, c["state"], c["cand"] = sgsa_decode_step(
                        q, k, v, q_ret, beta, gamma, budget, c["k"], c["v"], c["state"], top_k, write_mode,
                        alpha_max, tau_c, candidates=None if select else c["cand"])
                h = r(h + r(r(o).reshape(B, n_t, C) @ w("o_proj.weight").T))
            h = mlp(i, h)
        return r(r(rms_norm(h, P["norm.weight"], eps)) @ head.T)

    prompt_logits = run(prompt_ids, 0, None)
    dec = [run(decode_ids[:, s:s + 1], T + s, s) for s in range(decode_ids.shape[1])]
    return prompt_logits, (torch.cat(dec, dim=1) if dec else prompt_logits[:, :0])


# ---------------------------------------------------------------------------
# Hybrid top-k KV reuse (V-only)
# ---------------------------------------------------------------------------

def topk_kv_reuse_attention(query: Tensor, key: Tensor, value: Tensor, top_k: int,
                            attention_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Core of TopKSparseKVReuseAttention.forward (modelings/hybrid_dense_delta_topk.py:343-356).

    query [B,H,Q,D] (RoPE already applied), key/value [B,H,K,D]; queries sit at
    positions K-Q .. K-1 (:153-156).  Scores are multiplied by 1/sqrt(d) (:343-344),
    masked with ``finfo.min`` (:346) and every row keeps ``min(top_k, K)`` slots
    (:348-349) with no valid mask; probabilities are a fp32 softmax (:350).
    Returns (attended [B,H,Q,D], indices [B,H,Q,k], probs [B,H,Q,k]).
    """
    bsz, heads, qn, d = query.shape
    kn = key.shape[-2]
    scale = 1.0 / math.sqrt(d)
    scores = torch.matmul(query, key.transpose(-2, -1)) * scale
    qpos = torch.arange(kn - qn, kn)[:, None]
    masked = torch.arange(kn)[None, :] > qpos
    masked = masked[None, None].expand(bsz, heads, -1, -1)
    if attention_mask is not None:
        masked = masked | ~attention_mask.to(torch.bool)[:, None, None, :]
    scores = scores.masked_fill(masked, torch.finfo(scores.dtype).min)
    kk = min(top_k, kn)
    vals, idx = topk_lowest_index(scores.reshape(-1, kn), kk)
    vals = vals.reshape(bsz, heads, qn, kk)
    idx = idx.reshape(bsz, heads, qn, kk)
    probs = F.softmax(vals.float(), dim=-1).to(query.dtype)
    gv = value[:, :, None].expand(-1, -1, qn, -1, -1).gather(3, idx[..., None].expand(-1, -1, -1, -1, d))
    return (probs[..., None] * gv).sum(3), idx, probs


# ---------------------------------------------------------------------------
# Synthetic inputs
# ---------------------------------------------------------------------------

CONFIGS = {
    0: dict(B=1, H=4, T=512, D=64, chunk=64, top_k=32, dtype=torch.float32),
    1: dict(B=4, H=16, T=8192, D=128, chunk=64, top_k=256, dtype=torch.bfloat16),
    "north_star": dict(B=1, H=16, T=32768, D=128, chunk=64, top_k=2048, dtype=torch.bfloat16),
    3: dict(B=1, H=16, T=65536, D=128, chunk=64, top_k=2048, dtype=torch.bfloat16, heavy_tail=True),
}


def make_inputs(B: int, T: int, H: int, D: int, dtype=torch.float32, seed: int = 0,
                heavy_tail: bool = False, with_budget: bool = True) -> Dict[str, Tensor]:
    """Seeded synthetic inputs, drawn in a fixed order on a CPU generator.

    q,k,v ~ N(0,1) [B,T,H,D]; beta = sigmoid(N(0,1)); g = logsigmoid(N(0,1)+4)
    and gamma = exp(g); budget logits ~ N(0,1); q and k are L2-normalised per
    head.  Low-precision configs round to ``dtype``; the returned fp32 copies
    (``*_f32``) are those rounded values upcast, so the oracle and the kernels
    see identical inputs.  With ``heavy_tail`` 1% of key positions per (b,h)
    (``randperm`` on the same generator) are scaled x8 in a separate
    retrieval-key tensor ``k_ret``; the state key stays unit-norm.
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    glog = F.logsigmoid(torch.randn(B, T, H, generator=g) + 4.0)
    gamma = torch.exp(glog)
    budget = torch.randn(B, T, H, generator=g) if with_budget else None
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    k_ret = k
    if heavy_tail:
        k_ret = k.clone()
        n = int(round(0.01 * T))
        for b in range(B):
            for h in range(H):
                sel = torch.randperm(T, generator=g)[:n]
                k_ret[b, sel, h] *= 8.0
    out = {"q": q, "k": k, "v": v, "beta": beta, "gamma": gamma, "g": glog, "budget": budget,
           "k_ret": k_ret}
    if dtype != torch.float32:
        for name in ("q", "k", "v", "k_ret"):
            out[name] = out[name].to(dtype)
    for name in ("q", "k", "v", "k_ret"):
        out[name + "_f32"] = out[name].float()
    return out
