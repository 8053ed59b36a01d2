"""Drop-in ``fused_recurrent_sgsa`` backed by the gfx950 HIP recurrent kernel.

Same signature and return as modelings/sgsa_ops/recurrent.py:138-175 (the
function the layer's "recurrent" / "fused_recurrent" backends call,
modelings/modeling_sgsa.py:570-582), with the semantics of
naive_recurrent_sgsa (naive.py:34-57).  T = 1 is one decode step: pass the
previous final state as ``initial_state``.  The final state is float32, as on
the reference's Triton path (recurrent_fwd_triton.py:121-123); ``use_triton``
is accepted and ignored; unsupported input raises.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _abi
from .ops import chunk_sgsa_bwd
from .ops import _check_layout

Tensor = torch.Tensor


def recurrent_sgsa_fwd(
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
    """The HIP recurrent forward (sgsa_recurrent_fwd), no autograd.
    q, k, v [B,T,H,D]; beta, gamma [B,T,H]; state [B,H,D,D] (float32 out)."""
    if not q.is_cuda:
        raise ValueError("fused_recurrent_sgsa: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    B, T, H, D = q.shape
    dev = q.device
    for name, t in (("k", k), ("v", v)):
        _check_layout(name, t, (B, T, H, D), dev)
    for name, t in (("beta", beta), ("gamma", gamma)):
        _check_layout(name, t, (B, T, H), dev)
    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    if has_sparse:
        _check_layout("sparse_k", sparse_k, (B, T, H, D), dev)
        _check_layout("sparse_v", sparse_v, (B, T, H, D), dev)
        _check_layout("alpha", alpha, (B, T, H), dev)
    dt = q.dtype
    code = _abi.dtype_code(dt)
    cast = lambda t: t.to(dt).contiguous()
    qc, kc, vc = cast(q), cast(k), cast(v)
    bc = beta.float().contiguous()
    gc = gamma.float().contiguous()
    skc = cast(sparse_k) if has_sparse else None
    svc = cast(sparse_v) if has_sparse else None
    ac = alpha.float().contiguous() if has_sparse else None
    h0 = None
    if initial_state is not None:
        _check_layout("initial_state", initial_state, (B, H, D, D), dev)
        h0 = initial_state.float().contiguous()
    out = torch.empty_like(qc)
    ht = torch.empty(B, H, D, D, device=dev, dtype=torch.float32) if output_final_state else None
    _abi.check(_abi.lib().sgsa_recurrent_fwd(
        code, B, T, H, D, _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(bc), _abi.ptr(gc), _abi.ptr(skc),
        _abi.ptr(svc), _abi.ptr(ac), _abi.ptr(h0), _abi.ptr(out), _abi.ptr(ht), _abi.stream_of(qc)))
    return out, ht


class FusedRecurrentSGSAFunction(torch.autograd.Function):
    """Autograd wrapper of the recurrent op (modelings/sgsa_ops/recurrent.py:13-135).

    The forward runs the HIP recurrent kernel.  The backward is the native
    chunk-form backward (sgsa_chunk_bwd) of the same function: the recurrence
    and the chunk form are one map, so its gradient of <o, do> + <S_T, dS_T>
    is the recurrence's (the reference recomputes under autograd,
    recurrent.py:78-135).
    """

    @staticmethod
    def forward(ctx, q, k, v, beta, gamma, sparse_k, sparse_v, alpha, initial_state, has_sparse,
                has_initial_state, output_final_state):
        out, final = recurrent_sgsa_fwd(
            q, k, v, beta, gamma,
            sparse_k if has_sparse else None,
            sparse_v if has_sparse else None,
            alpha if has_sparse else None,
            initial_state if has_initial_state else None,
            output_final_state)
        ctx.save_for_backward(q, k, v, beta, gamma, sparse_k, sparse_v, alpha, initial_state)
        ctx.has_sparse, ctx.has_initial_state = has_sparse, has_initial_state
        return out, final

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, beta, gamma, sparse_k, sparse_v, alpha, initial_state = ctx.saved_tensors
        hs, hi = ctx.has_sparse, ctx.has_initial_state
        inputs = [q, k, v, beta, gamma, sparse_k if hs else None, sparse_v if hs else None, alpha if hs else None,
                  initial_state if hi else None]
        grads = chunk_sgsa_bwd(inputs, ctx.needs_input_grad[:9], do, dht)
        return (*grads, None, None, None)


def fused_recurrent_sgsa(
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
    use_triton: bool = True,
    cu_seqlens: Optional[Tensor] = None,
) -> Tuple[Tensor, Optional[Tensor]]:
    """q, k, v [B,T,H,D]; beta, gamma [B,T,H]; state [B,H,D,D] (float32 out).
    Differentiable: the backward is the native chunk-form backward (FusedRecurrentSGSAFunction).
    ``cu_seqlens`` [N+1]: packed sequences in a batch of one, states [N,H,D,D] (sgsa_amd.varlen)."""
    if not q.is_cuda:
        raise ValueError("fused_recurrent_sgsa: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    if cu_seqlens is not None:
        from . import varlen
        lay = varlen.layout(cu_seqlens, q)
        varlen.check_states(lay, initial_state)
        pq, pk, pv, pb, pg, psk, psv, pa = varlen.pad_state_inputs(lay, q, k, v, beta, gamma, sparse_k, sparse_v,
                                                                   alpha)
        o, ht = fused_recurrent_sgsa(pq, pk, pv, pb, pg, psk, psv, pa, initial_state, output_final_state, use_triton)
        return lay.unpad(o), ht
    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    has_init = initial_state is not None
    empty = torch.empty(0, device=q.device, dtype=q.dtype)
    return FusedRecurrentSGSAFunction.apply(
        q, k, v, beta, gamma,
        sparse_k if has_sparse else empty,
        sparse_v if has_sparse else empty,
        alpha if has_sparse else torch.empty(0, device=q.device, dtype=beta.dtype),
        initial_state if has_init else empty,
        has_sparse, has_init, output_final_state)
