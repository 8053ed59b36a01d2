"""Backward of the SGSA ops by recomputation under autograd.

The reference differentiates its ops by recomputing the forward in torch under
autograd and taking the gradient of <o, do> + <S_T, dS_T>
(modelings/sgsa_ops/chunk_bwd.py:31-77 for ``chunk_sgsa``,
modelings/sgsa_ops/recurrent.py:78-135 for ``fused_recurrent_sgsa``).  This
module restates that for the HIP forward: ``chunk_sgsa_torch`` is a
differentiable torch form of exactly what the HIP kernels compute -- the chunk
form with virtual samples (local, sparse) per token, the chunk-local inclusive
log-decay prefix l_t = sum_{p<=t} log max(gamma_p, 1e-6) and decay ratios
exp(l_a - l_b) -- and ``recompute_grads`` differentiates it.  It runs where the
tensors are (the GPU, after a HIP forward) in float32, or float64 for float64
inputs.  Per chunk (M virtual samples, tau_i the token of sample i):

    T_ij = 1[tau_j < tau_i] lam_j exp(l_tau_i - l_tau_j) (kappa_i . kappa_j)
    W = (I + T)^-1 diag(exp(l_tau)) kappa        U = (I + T)^-1 nu
    R = U - W S
    o_t = exp(l_t) S^T q_t + sum_{tau_i <= t} lam_i exp(l_t - l_tau_i) (q_t . kappa_i) R_i
    S' = exp(l_L) S + sum_i kappa_i lam_i exp(l_L - l_tau_i) R_i^T

(modelings/sgsa_ops/chunk_fwd.py:49-129 with the clamped prefix-product
ratios replaced by exponentials of prefix differences, which equal the
token recurrence of naive.py:34-57 also where a prefix falls below 1e-6).
Every exponent above is <= 0 for gamma <= 1.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def chunk_sgsa_torch(
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
) -> Tuple[Tensor, Tensor]:
    """Differentiable chunk-form SGSA forward.

    q, k, v, sparse_k, sparse_v [B,T,H,D]; beta, gamma, alpha [B,T,H];
    initial_state [B,H,Dk,Dv].  Returns (o [B,T,H,Dv], final state
    [B,H,Dk,Dv]), both in the compute dtype (float64 for float64 q, else
    float32).  The sparse write is used iff sparse_k, sparse_v and alpha are
    all given, as in modelings/sgsa_ops/chunk.py:123.
    """
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    dev = q.device
    cdt = torch.float64 if q.dtype == torch.float64 else torch.float32
    L = int(chunk_size)
    if L <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    NT = max(1, -(-T // L))
    Tp = NT * L

    def tokens(x: Tensor) -> Tensor:   # [B,T,H,D] -> [B,H,NT,L,D], zero-padded
        x = x.to(cdt).transpose(1, 2)
        if Tp != T:
            x = F.pad(x, (0, 0, 0, Tp - T))
        return x.reshape(B, H, NT, L, x.shape[-1])

    def gates(x: Tensor, pad: float) -> Tensor:   # [B,T,H] -> [B,H,NT,L]
        x = x.to(cdt).transpose(1, 2)
        if Tp != T:
            x = F.pad(x, (0, Tp - T), value=pad)
        return x.reshape(B, H, NT, L)

    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    qh, kh, vh = tokens(q), tokens(k), tokens(v)
    lb = gates(beta, 0.0)
    # padded tokens: gamma = 1 (no decay), beta = alpha = 0 (no write)
    ell = torch.cumsum(torch.log(gates(gamma, 1.0).clamp_min(1e-6)), dim=-1)   # [B,H,NT,L]
    if has_sparse:
        kap = torch.stack((kh, tokens(sparse_k)), dim=4).reshape(B, H, NT, 2 * L, Dk)
        nu = torch.stack((vh, tokens(sparse_v)), dim=4).reshape(B, H, NT, 2 * L, Dv)
        lam = torch.stack((lb, gates(alpha, 0.0)), dim=-1).reshape(B, H, NT, 2 * L)
        tau = torch.arange(L, device=dev).repeat_interleave(2)
    else:
        kap, nu, lam, tau = kh, vh, lb, torch.arange(L, device=dev)
    M = kap.shape[3]
    et = ell[..., tau]                                            # l at each sample's token [B,H,NT,M]

    dep = tau[None, :] < tau[:, None]                             # (i, j): tau_j < tau_i
    dexp = torch.exp(torch.where(dep, et[..., :, None] - et[..., None, :], torch.zeros((), dtype=cdt, device=dev)))
    trans = torch.where(dep, lam[..., None, :] * dexp, torch.zeros((), dtype=cdt, device=dev))
    trans = trans * (kap @ kap.transpose(-1, -2))
    ia = trans + torch.eye(M, dtype=cdt, device=dev)
    W = torch.linalg.solve_triangular(ia, torch.exp(et)[..., None] * kap, upper=False)   # [B,H,NT,M,Dk]
    U = torch.linalg.solve_triangular(ia, nu, upper=False)                               # [B,H,NT,M,Dv]

    S = (torch.zeros(B, H, Dk, Dv, dtype=cdt, device=dev) if initial_state is None
         else initial_state.to(cdt))
    dL = ell[..., -1]                                             # [B,H,NT]
    wdec = lam * torch.exp(dL[..., None] - et)                    # [B,H,NT,M]
    starts: List[Tensor] = []
    resids: List[Tensor] = []
    for c in range(NT):
        starts.append(S)
        R = U[:, :, c] - W[:, :, c] @ S
        resids.append(R)
        S = torch.exp(dL[:, :, c])[..., None, None] * S + kap[:, :, c].transpose(-1, -2) @ (wdec[:, :, c, :, None] * R)
    Sc = torch.stack(starts, dim=2)                               # chunk-start states [B,H,NT,Dk,Dv]
    Rc = torch.stack(resids, dim=2)                               # residuals [B,H,NT,M,Dv]

    t = torch.arange(L, device=dev)
    rmask = tau[None, :] <= t[:, None]                            # (t, i): tau_i <= t
    rexp = torch.exp(torch.where(rmask, ell[..., :, None] - et[..., None, :], torch.zeros((), dtype=cdt, device=dev)))
    P = torch.where(rmask, lam[..., None, :] * rexp, torch.zeros((), dtype=cdt, device=dev))
    P = P * (qh @ kap.transpose(-1, -2))                          # [B,H,NT,L,M]
    o = torch.exp(ell)[..., None] * (qh @ Sc) + P @ Rc            # [B,H,NT,L,Dv]
    o = o.reshape(B, H, Tp, Dv)[:, :, :T].transpose(1, 2)
    return o, S


def recompute_grads(
    inputs: Sequence[Optional[Tensor]],
    needs: Sequence[bool],
    do: Optional[Tensor],
    dht: Optional[Tensor],
) -> List[Optional[Tensor]]:
    """Gradients of <o, do> + <S_T, dht> w.r.t. (q, k, v, beta, gamma,
    sparse_k, sparse_v, alpha, initial_state), recomputing the forward with
    ``chunk_sgsa_torch`` under autograd (chunk_bwd.py:43-63).  ``inputs`` holds
    those nine tensors (None where absent); ``needs[i]`` says whether input i
    wants a gradient.  Returns nine entries, None where absent or not needed;
    each gradient has its input's dtype.
    """
    leaves = [None if x is None else x.detach().requires_grad_(bool(n)) for x, n in zip(inputs, needs)]
    with torch.enable_grad():
        o, ht = chunk_sgsa_torch(*leaves)
        objective = o.new_zeros(())
        if do is not None:
            objective = objective + (o * do.to(o.dtype)).sum()
        if dht is not None:
            objective = objective + (ht * dht.to(ht.dtype)).sum()
    want = [i for i, x in enumerate(leaves) if x is not None and x.requires_grad]
    grads: List[Optional[Tensor]] = [None] * len(leaves)
    if want and objective.requires_grad:
        got = torch.autograd.grad(objective, [leaves[i] for i in want], allow_unused=True)
        for i, g in zip(want, got):
            grads[i] = torch.zeros_like(leaves[i]) if g is None else g.to(inputs[i].dtype)
    else:
        for i in want:
            grads[i] = torch.zeros_like(leaves[i])
    return grads
