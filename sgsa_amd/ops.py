"""Drop-in ``chunk_sgsa`` backed by the gfx950 HIP kernels.

Same signature and return as modelings/sgsa_ops/chunk.py:104-148, so callers
such as SGSAStateLayer.forward (modelings/modeling_sgsa.py:584-596) work by
swapping the import.  Differences, all deliberate:

* the state is carried between chunks in float32 and the final state is
  returned in float32 (the reference holds it in q.dtype between chunks and
  returns it so, chunk_fwd.py:34, :129: with bf16 inputs a rounding of the
  state after every chunk, worth about 1e-3 of o's largest magnitude at
  T = 32768);
* ``use_triton`` is accepted and ignored; ``chunk_size`` is accepted, the
  kernels always use 64-token chunks (the result depends on it only through
  rounding), and a value other than 64 draws a warning;
* decay ratios are exp(log-cumsum differences) rather than ratios of clamped
  prefix products (chunk_fwd.py:86, :110, :121), which follows the recurrent
  definition (naive.py:40) also where a chunk-local prefix falls below 1e-6;
* unsupported input (CPU tensors, float16, D > 128) raises instead of falling
  back to another implementation.

The backward is native too (sgsa_chunk_bwd, chunk_bwd.hip): the gradient of
the chunk form written out, where the reference recomputes the forward under
torch autograd (chunk_bwd.py:31-77).  ``backward.py`` keeps a differentiable
torch form of the same function, which the tests use as a second reference.
"""

from __future__ import annotations

import ctypes
import warnings
from typing import List, Optional, Sequence, Tuple

import torch

from . import _abi

Tensor = torch.Tensor


def _check_layout(name: str, t: Tensor, shape, device) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


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
    use_triton: bool = True,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Forward body (replaces modelings/sgsa_ops/chunk_fwd.py:12-131)."""
    if not q.is_cuda:
        raise ValueError("chunk_sgsa: the SGSA kernels run on a ROCm GPU; got CPU tensors")
    if chunk_size <= 0:
        raise ValueError(f"chunk_size={chunk_size} must be positive")
    if chunk_size != 64:
        warnings.warn(f"chunk_sgsa: chunk_size={chunk_size} is accepted for compatibility; the kernels use "
                      "64-token chunks, whose result differs from other chunkings only by rounding", stacklevel=3)
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
    L = _abi.lib()
    nbytes = ctypes.c_size_t()
    _abi.check(L.sgsa_chunk_fwd_workspace_size(B, T, H, D, int(has_sparse), ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_chunk_fwd(code, B, T, H, D, int(chunk_size), _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc),
                                _abi.ptr(bc), _abi.ptr(gc), _abi.ptr(skc), _abi.ptr(svc), _abi.ptr(ac),
                                _abi.ptr(h0), _abi.ptr(out), _abi.ptr(ht), _abi.ptr(ws), nbytes.value,
                                _abi.stream_of(qc)))
    return out, ht


def chunk_sgsa_bwd(
    inputs: Sequence[Optional[Tensor]],
    needs: Sequence[bool],
    do: Optional[Tensor],
    dht: Optional[Tensor],
) -> List[Optional[Tensor]]:
    """Native backward (sgsa_chunk_bwd): the gradients of <o, do> + <S_T, dht>
    w.r.t. (q, k, v, beta, gamma, sparse_k, sparse_v, alpha, initial_state) for
    the function the forward kernels compute -- the role of chunk_sgsa_bwd
    (modelings/sgsa_ops/chunk_bwd.py:12-77).  ``inputs`` holds those nine
    tensors (None where absent), ``needs[i]`` whether input i wants a gradient.
    Returns nine entries, None where absent or not needed; each gradient has its
    input's dtype (the kernels compute in fp32).
    """
    q, k, v, beta, gamma, sk, sv, alpha, h0 = inputs
    B, T, H, D = q.shape
    dev = q.device
    dt = q.dtype
    code = _abi.dtype_code(dt)
    has_sparse = sk is not None
    cast = lambda t: t.to(dt).contiguous()
    qc, kc, vc = cast(q), cast(k), cast(v)
    bc, gc = beta.float().contiguous(), gamma.float().contiguous()
    skc = cast(sk) if has_sparse else None
    svc = cast(sv) if has_sparse else None
    ac = alpha.float().contiguous() if has_sparse else None
    h0c = h0.float().contiguous() if h0 is not None else None
    doc = cast(do) if do is not None else torch.zeros_like(qc)
    dhtc = dht.float().contiguous() if dht is not None else None
    dq, dk, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
    dbeta = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    dgamma = torch.empty_like(dbeta)
    dsk = torch.empty_like(skc) if has_sparse else None
    dsv = torch.empty_like(svc) if has_sparse else None
    dalpha = torch.empty_like(dbeta) if has_sparse else None
    dh0 = torch.empty(B, H, D, D, device=dev, dtype=torch.float32) if h0 is not None else None
    L = _abi.lib()
    nbytes = ctypes.c_size_t()
    _abi.check(L.sgsa_chunk_bwd_workspace_size(B, T, H, D, int(has_sparse), ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_chunk_bwd(
        code, B, T, H, D, _abi.ptr(qc), _abi.ptr(kc), _abi.ptr(vc), _abi.ptr(bc), _abi.ptr(gc), _abi.ptr(skc),
        _abi.ptr(svc), _abi.ptr(ac), _abi.ptr(h0c), _abi.ptr(doc), _abi.ptr(dhtc), _abi.ptr(dq), _abi.ptr(dk),
        _abi.ptr(dv), _abi.ptr(dbeta), _abi.ptr(dgamma), _abi.ptr(dsk), _abi.ptr(dsv), _abi.ptr(dalpha),
        _abi.ptr(dh0), _abi.ptr(ws), nbytes.value, _abi.stream_of(qc)))
    grads = [dq, dk, dv, dbeta, dgamma, dsk, dsv, dalpha, dh0]
    out: List[Optional[Tensor]] = []
    for x, g, n in zip(inputs, grads, needs):
        out.append(g.to(x.dtype) if (x is not None and n and g is not None) else None)
    return out


class ChunkSGSAFunction(torch.autograd.Function):
    """Autograd wrapper with the reference's argument list (modelings/sgsa_ops/chunk.py:13-101).

    The forward runs the HIP kernels; so does the backward (``chunk_sgsa_bwd``,
    sgsa_chunk_bwd: the gradient of the chunk form, where the reference
    recomputes the forward under torch autograd, chunk.py:58-101 ->
    chunk_bwd.py:31-77).  It returns the 9 input gradients (None for absent
    optionals) and None for the 5 flags.
    """

    @staticmethod
    def forward(ctx, q, k, v, beta, gamma, sparse_k, sparse_v, alpha, initial_state, has_sparse,
                has_initial_state, chunk_size, output_final_state, use_triton):
        out, final = chunk_sgsa_fwd(
            q, k, v, beta, gamma,
            sparse_k if has_sparse else None,
            sparse_v if has_sparse else None,
            alpha if has_sparse else None,
            initial_state if has_initial_state else None,
            chunk_size, output_final_state, use_triton)
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
        return (*grads, None, None, None, None, None)


def chunk_sgsa(
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
    use_triton: bool = True,
    cu_seqlens: Optional[Tensor] = None,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Chunked Sparse-Guided State Attention core (modelings/sgsa_ops/chunk.py:104-148).

    q,k,v,sparse_k,sparse_v: [B,T,H,D]; beta,gamma,alpha: [B,T,H];
    initial_state: [B,H,D,D].  The sparse write is used iff sparse_k, sparse_v
    and alpha are all given (chunk.py:123).  Returns (o [B,T,H,D] in q.dtype,
    final state [B,H,D,D] float32 or None).

    ``cu_seqlens`` [N+1]: N sequences packed along T of a batch of one (the FLA
    varlen convention, sgsa_amd.varlen); initial and final states are then
    [N,H,D,D], one per sequence, and each sequence starts from its own state.
    """
    if cu_seqlens is not None:
        from . import varlen
        lay = varlen.layout(cu_seqlens, q)
        varlen.check_states(lay, initial_state)
        pq, pk, pv, pb, pg, psk, psv, pa = varlen.pad_state_inputs(lay, q, k, v, beta, gamma, sparse_k, sparse_v,
                                                                   alpha)
        o, ht = chunk_sgsa(pq, pk, pv, pb, pg, psk, psv, pa, initial_state, chunk_size, output_final_state,
                           use_triton)
        return lay.unpad(o), ht
    has_sparse = sparse_k is not None and sparse_v is not None and alpha is not None
    has_init = initial_state is not None
    empty = torch.empty(0, device=q.device, dtype=q.dtype)
    return ChunkSGSAFunction.apply(
        q, k, v, beta, gamma,
        sparse_k if sparse_k is not None else empty,
        sparse_v if sparse_v is not None else empty,
        alpha if alpha is not None else torch.empty(0, device=q.device, dtype=beta.dtype),
        initial_state if has_init else empty,
        has_sparse, has_init, chunk_size, output_final_state, use_triton)
