"""Config 4: a hybrid decoder of SGSA layers and dense GQA attention layers, with
prefill and greedy decode.

Layer i is dense full attention when i % dense_every == 0 and an SGSA block
otherwise: the 3:1 scheduling of the reference's hybrid stack
(modelings/hybrid_dense_delta_topk.py:394-437, dense every 4th layer at :398),
with the reference's SGSABlock (modelings/modeling_sgsa.py:634-709, here
sgsa_amd.model.SGSABlock on the HIP kernels) as the sparse layer.

* Dense layers: RMSNorm, q / k / v projections with num_kv_heads key/value heads
  (grouped-query attention: query head h reads key/value head h // (H / Hkv)),
  rotary embedding in the reference's rotate-half form (:124-150), causal
  softmax attention with scores in the activation dtype and the softmax in
  fp32 (:178-192), o_proj; then the SwiGLU MLP (:106-116).  PyTorch GEMMs.
* SGSA layers: prefill is sgsa_layer_forward over the prompt (K1, K2, K3-K5),
  keeping the layer's keys, values and final state; a decode step is
  sgsa_decode_step over the cache (K1 one row, K2, K6).  Each layer selects
  its top-k every ``topk_recompute_every`` decode steps and re-scores that
  candidate set in between (sgsa_score_at; modelings/idea.md:395-401).
* Caches are preallocated for prompt + decode steps: [B, Hkv, Tmax, D] keys
  (after RoPE) and values per dense layer, [B, Tmax, H, D] keys and values plus
  the fp32 [B, H, D, D] state and the candidate set per SGSA layer.

No right-hand operand of an attention product is a transposed view: scores
are Q K^T with K^T copied contiguous (prefill) or K Q^T with Q^T copied
contiguous (decode), and the values are a row-major slice of the cache.
The decoder (prefill, decode) is inference only; TopKSparseKVReuseAttention
also trains (its differentiable form under autograd).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .decode import sgsa_decode_step
from .layer import LayerWorkspace, sgsa_layer_forward
from . import _abi
from .model import GatedMLP, RMSNorm, SGSABlock, SGSAConfig, fused_linear, fused_linear_out, fused_weight, lin
from .retrieval import gather_masked, score_topk_masked
from .retrieval_grad import MAX_SELECTED_ELEMS

Tensor = torch.Tensor


@dataclass
class HybridConfig:
    """Config 4 defaults: 24 layers, hidden 2048, 16 query / 4 key-value heads of 128,
    SwiGLU 5632, vocab 32000, top-k 2048 recomputed every 4 decode steps."""

    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_kv_heads: int = 4
    dense_every: int = 4
    rope_theta: float = 10000.0
    layer_norm_eps: float = 1e-6
    top_k: int = 2048
    topk_recompute_every: int = 4
    sgsa_write_mode: str = "direct"
    alpha_max: float = 0.25
    tau_c: float = 0.1
    tie_word_embeddings: bool = True
    pad_token_id: int = 0

    @property
    def head_dim(self) -> int:
        if self.hidden_size % self.num_attention_heads != 0:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        return self.hidden_size // self.num_attention_heads

    def is_dense(self, i: int) -> bool:
        return i % self.dense_every == 0

    def sgsa_config(self) -> SGSAConfig:
        return SGSAConfig(vocab_size=self.vocab_size, hidden_size=self.hidden_size,
                          intermediate_size=self.intermediate_size, num_hidden_layers=1,
                          num_attention_heads=self.num_attention_heads, num_kv_heads=self.num_attention_heads,
                          layer_norm_eps=self.layer_norm_eps, top_k=self.top_k, retrieval_mode="token_only",
                          sgsa_write_mode=self.sgsa_write_mode, alpha_max=self.alpha_max, tau_c=self.tau_c)


def rope_tables(n: int, head_dim: int, theta: float, device) -> Tuple[Tensor, Tensor]:
    """cos, sin [n, head_dim] in fp32 (modelings/hybrid_dense_delta_topk.py:124-137)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    freqs = torch.outer(torch.arange(n, device=device, dtype=torch.float32), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """x [B, heads, T, D] at the positions of cos / sin [T, D] (:140-150), in x's dtype."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos.to(x.dtype) + rot * sin.to(x.dtype)


def gqa_attention(q: Tensor, k: Tensor, v: Tensor, pos0: int, block: int = 1024) -> Tensor:
    """Causal attention: q [B, H, Tq, D] at positions pos0 .., k / v [B, Hkv, Tk, D]
    with Tk >= pos0 + Tq.  Scores and their 1/sqrt(D) scaling in q's dtype, softmax in
    fp32, probabilities cast back (:178-192).  Query blocks of ``block`` rows read only the keys they may see.
    Long query blocks (prefill) form Q K^T with a contiguous copy of the block's K^T
    and a softmax over the last dimension; short ones (decode) form K Q^T, which
    reads the cache in place."""
    B, H, Tq, D = q.shape
    Hkv = k.shape[1]
    G = H // Hkv
    if Tq == 1 and _decode_attention_fits(q, k, v, pos0):
        return _decode_attention(q, k, v)
    if Tq > 1 and _dense_attention_fits(q, k, v, pos0):
        return _dense_attention(q, k, v, pos0)
    out = torch.empty_like(q)
    qg = q.reshape(B, Hkv, G, Tq, D)
    kpos = torch.arange(k.shape[2], device=q.device)
    if Tq >= 64:
        for r0 in range(0, Tq, block):
            r1 = min(Tq, r0 + block)
            n = r1 - r0
            kend = pos0 + r1
            qb = qg[:, :, :, r0:r1].reshape(B, Hkv, G * n, D)
            kt = k[:, :, :kend].transpose(-1, -2).contiguous()                                  # [B,Hkv,D,kend]
            s = (torch.matmul(qb, kt) * (1.0 / math.sqrt(D))).float()                           # [B,Hkv,G*n,kend]
            qpos = (pos0 + r0 + torch.arange(n, device=q.device)).repeat(G)
            s = s.masked_fill(kpos[None, :kend] > qpos[:, None], float("-inf"))
            p = torch.softmax(s, dim=-1).to(q.dtype)
            o = torch.matmul(p, v[:, :, :kend])   # a row-major slice of the cache, not a transposed view
            out[:, :, r0:r1] = o.view(B, Hkv, G, n, D).reshape(B, H, n, D)
        return out
    for r0 in range(0, Tq, block):
        r1 = min(Tq, r0 + block)
        n = r1 - r0
        kend = pos0 + r1
        qb = qg[:, :, :, r0:r1].reshape(B, Hkv, G * n, D).transpose(-1, -2).contiguous()   # [B,Hkv,D,G*n]
        s = (torch.matmul(k[:, :, :kend], qb) * (1.0 / math.sqrt(D))).float()             # [B,Hkv,kend,G*n]
        qpos = (pos0 + r0 + torch.arange(n, device=q.device)).repeat(G)                    # column -> position
        s = s.masked_fill(kpos[:kend, None] > qpos[None, :], float("-inf"))
        p = torch.softmax(s, dim=-2).to(q.dtype).transpose(-1, -2).contiguous()             # [B,Hkv,G*n,kend]
        o = torch.matmul(p, v[:, :, :kend])   # [B,Hkv,G*n,D]; a row-major slice, not a transposed view
        out[:, :, r0:r1] = o.view(B, Hkv, G, n, D).reshape(B, H, n, D)
    return out


def _cache_view_len(t: Tensor) -> int:
    """cache_len of a [B, Hkv, kend, D] view of a contiguous [B, Hkv, cache_len, D] cache, or 0."""
    B, Hkv, _, D = t.shape
    if t.stride(3) != 1 or t.stride(2) != D or t.stride(1) % D != 0:
        return 0
    n = t.stride(1) // D
    return n if t.stride(0) == Hkv * n * D and n >= t.shape[2] else 0


def _decode_attention_fits(q: Tensor, k: Tensor, v: Tensor, pos0: int) -> bool:
    """Whether sgsa_decode_attention takes this call: one query row per sequence at the
    last cached position, no autograd, D = 128, H / Hkv in {1, 2, 4, 8}, q contiguous and
    k / v views of contiguous caches of q's dtype."""
    B, H, _, D = q.shape
    Hkv = k.shape[1]
    return (not torch.is_grad_enabled() and q.is_cuda and q.dtype in (torch.float32, torch.bfloat16) and D == 128
            and H % Hkv == 0 and H // Hkv in (1, 2, 4, 8) and k.dtype == q.dtype and v.dtype == q.dtype
            and q.is_contiguous() and k.shape == v.shape and k.shape[2] == pos0 + 1
            and _cache_view_len(k) > 0 and _cache_view_len(k) == _cache_view_len(v))


def _decode_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """gqa_attention for one query row per sequence, in one HIP pass over the cache
    (sgsa_decode_attention): the same rounding points as the torch form."""
    B, H, _, D = q.shape
    Hkv, kend = k.shape[1], k.shape[2]
    code = _abi.dtype_code(q.dtype)
    nb = ctypes.c_size_t()
    L = _abi.lib()
    _abi.check(L.sgsa_decode_attention_workspace_size(code, B, H, kend, ctypes.byref(nb)))
    ws = torch.empty(nb.value, device=q.device, dtype=torch.uint8)
    out = torch.empty_like(q)
    _abi.check(L.sgsa_decode_attention(code, B, H, Hkv, D, _abi.ptr(q), _abi.ptr(k), _abi.ptr(v), _cache_view_len(k),
                                       kend, _abi.ptr(out), _abi.ptr(ws), nb.value, _abi.stream_of(q)))
    return out


def _dense_attention_fits(q: Tensor, k: Tensor, v: Tensor, pos0: int) -> bool:
    """Whether sgsa_dense_attention takes this call: bf16, no autograd, D = 128, q contiguous,
    k / v views of contiguous caches ending at the block's last position."""
    B, H, Tq, D = q.shape
    Hkv = k.shape[1]
    return (not torch.is_grad_enabled() and q.is_cuda and q.dtype == torch.bfloat16 and D == 128 and H % Hkv == 0
            and k.dtype == q.dtype and v.dtype == q.dtype and q.is_contiguous() and k.shape == v.shape
            and k.shape[2] == pos0 + Tq and _cache_view_len(k) > 0 and _cache_view_len(k) == _cache_view_len(v)
            and (pos0 + Tq) * 256 < 2 ** 31 - 1)


def _dense_attention(q: Tensor, k: Tensor, v: Tensor, pos0: int) -> Tensor:
    """gqa_attention for a block of query rows in two HIP passes over the cache
    (sgsa_dense_attention): each row's softmax maximum and sum, then p V with the
    probabilities rounded after normalisation, as the torch form does."""
    B, H, Tq, D = q.shape
    ws = torch.empty(B * H * Tq * 8, device=q.device, dtype=torch.uint8)
    out = torch.empty_like(q)
    _abi.check(_abi.lib().sgsa_dense_attention(_abi.dtype_code(q.dtype), B, H, k.shape[1], D, Tq, pos0, _abi.ptr(q),
                                               _abi.ptr(k), _abi.ptr(v), _cache_view_len(k), _abi.ptr(out),
                                               _abi.ptr(ws), ws.numel(), _abi.stream_of(q)))
    return out


class DenseGQABlock(nn.Module):
    """Dense full-attention block of the hybrid stack (:195-244, :407-437), with grouped key/value heads."""

    def __init__(self, config: HybridConfig) -> None:
        super().__init__()
        H, Hkv, D, C = config.num_attention_heads, config.num_kv_heads, config.head_dim, config.hidden_size
        if H % Hkv != 0:
            raise ValueError("num_attention_heads must be a multiple of num_kv_heads")
        self.H, self.Hkv, self.D = H, Hkv, D
        self.input_norm = RMSNorm(C, config.layer_norm_eps)
        self.post_attn_norm = RMSNorm(C, config.layer_norm_eps)
        self.q_proj = nn.Linear(C, H * D, bias=False)
        self.k_proj = nn.Linear(C, Hkv * D, bias=False)
        self.v_proj = nn.Linear(C, Hkv * D, bias=False)
        self.o_proj = nn.Linear(H * D, C, bias=False)
        self.mlp = GatedMLP(C, config.intermediate_size)

    def forward_cached(self, h: Tensor, pos0: int, cache: dict, rope: Tuple[Tensor, Tensor]) -> Tensor:
        """h [B, T, C] at positions pos0 ..; appends its keys and values to the cache."""
        B, T, C = h.shape
        n = self.input_norm(h)
        q, k, v = fused_linear(self, n, ("q_proj", "k_proj", "v_proj"))
        v = v.reshape(B, T, self.Hkv, self.D).transpose(1, 2)
        if torch.is_grad_enabled():
            q = q.reshape(B, T, self.H, self.D).transpose(1, 2)
            k = k.reshape(B, T, self.Hkv, self.D).transpose(1, 2)
            cos, sin = rope[0][pos0:pos0 + T], rope[1][pos0:pos0 + T]
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        else:
            # q and k are adjacent groups of one projection row: one launch rotates both into [B, heads, T, D]
            qs = q
            q = torch.empty(B, self.H, T, self.D, device=h.device, dtype=h.dtype)
            k = torch.empty(B, self.Hkv, T, self.D, device=h.device, dtype=h.dtype)
            cos_t, sin_t = rope[0].float().contiguous(), rope[1].float().contiguous()
            _abi.check(_abi.lib().sgsa_rope_qk(_abi.dtype_code(h.dtype), B, T, self.H, self.Hkv, self.D, pos0,
                                               cos_t.shape[0], _abi.ptr(qs), qs.stride(-2), _abi.ptr(cos_t),
                                               _abi.ptr(sin_t), _abi.ptr(q), _abi.ptr(k), _abi.stream_of(qs)))
        cache["k"][:, :, pos0:pos0 + T] = k
        cache["v"][:, :, pos0:pos0 + T] = v
        att = gqa_attention(q, cache["k"][:, :, :pos0 + T], cache["v"][:, :, :pos0 + T], pos0)
        h, n = self.post_attn_norm.add_forward(h, lin(self.o_proj, att.transpose(1, 2).reshape(B, T, self.H * self.D)))
        return h + self.mlp(n)


class SGSADecoderBlock(SGSABlock):
    """SGSABlock with a prefill that keeps its cache and a one-token decode step."""

    def _finish(self, h: Tensor, att: Tensor) -> Tensor:
        B, T, C = h.shape
        h, n = self.post_attn_norm.add_forward(h, lin(self.o_proj, att.reshape(B, T, C)))
        return h + self.mlp(n)

    def prefill(self, h: Tensor, cache: dict) -> Tensor:
        cfg = self.config
        T = h.shape[1]
        q, k, v, q_ret, beta, gamma, budget = self._project(h)
        att, st = sgsa_layer_forward(q, k, v, q_ret, beta, gamma, budget, cfg.top_k, write_mode=cfg.sgsa_write_mode,
                                     alpha_max=cfg.alpha_max, tau_c=cfg.tau_c, output_final_state=True,
                                     workspace=self._ws)
        cache["k"][:, :T] = k
        cache["v"][:, :T] = v
        cache["state"] = st
        cache["cand"] = None
        return self._finish(h, att)

    _PROJ = ("q_proj", "k_proj", "v_proj", "q_ret_proj", "beta_proj", "gamma_proj", "budget_proj")

    def _project_decode(self, h: Tensor, pos: int, cache: dict):
        """_project for one token per sequence, appending its k and v to the cache.  Without
        autograd, one launch (sgsa_decode_split) splits the fused projection row into
        contiguous q, k, v, q_ret, makes the gates and writes the cache row, in place of
        the strided copies the kernels would otherwise take."""
        kc, vc = cache["k"], cache["v"]
        if torch.is_grad_enabled() or kc.dtype != h.dtype or vc.dtype != h.dtype or not kc.is_contiguous() \
                or not vc.is_contiguous():
            q, k, v, q_ret, beta, gamma, budget = self._project(h)
            kc[:, pos:pos + 1] = k
            vc[:, pos:pos + 1] = v
            return q, k, v, q_ret, beta, gamma, budget
        B = h.shape[0]
        H, D = self.num_heads, self.head_dim
        y = fused_linear_out(self, self.input_norm(h), self._PROJ)   # [B, 1, 4HD + 3H], contiguous
        q, k, v, q_ret = (torch.empty(B, 1, H, D, device=h.device, dtype=h.dtype) for _ in range(4))
        beta, gamma, budget = (torch.empty(B, 1, H, device=h.device, dtype=torch.float32) for _ in range(3))
        _abi.check(_abi.lib().sgsa_decode_split(
            _abi.dtype_code(h.dtype), B, H, D, _abi.ptr(y), y.stride(0), _abi.ptr(q), _abi.ptr(k), _abi.ptr(v),
            _abi.ptr(q_ret), _abi.ptr(beta), _abi.ptr(gamma), _abi.ptr(budget), _abi.ptr(kc), _abi.ptr(vc),
            kc.shape[1], pos, _abi.stream_of(y)))
        return q, k, v, q_ret, beta, gamma, budget

    def decode(self, h: Tensor, pos: int, cache: dict, select: bool) -> Tensor:
        """h [B, 1, C] at position pos; select: recompute the top-k (else re-score the kept set)."""
        cfg = self.config
        q, k, v, q_ret, beta, gamma, budget = self._project_decode(h, pos, cache)
        cand = None if (select or cache["cand"] is None) else cache["cand"]
        att, st, cand = sgsa_decode_step(q, k, v, q_ret, beta, gamma, budget, cache["k"], cache["v"],
                                         cache["state"], cfg.top_k, write_mode=cfg.sgsa_write_mode,
                                         alpha_max=cfg.alpha_max, tau_c=cfg.tau_c, candidates=cand,
                                         return_candidates=True, length=pos + 1)
        cache["state"], cache["cand"] = st, cand
        return self._finish(h, att)


class HybridForCausalLM(nn.Module):
    """Embedding, the hybrid stack, final RMSNorm and (tied) LM head (:439-532)."""

    def __init__(self, config: HybridConfig) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, padding_idx=config.pad_token_id)
        scfg = config.sgsa_config()
        self.layers = nn.ModuleList([DenseGQABlock(config) if config.is_dense(i) else SGSADecoderBlock(scfg)
                                     for i in range(config.num_hidden_layers)])
        shared = LayerWorkspace()   # the SGSA layers run one at a time: one workspace serves them all
        for layer in self.layers:
            if isinstance(layer, SGSADecoderBlock):
                layer._ws = shared
        self.norm = RMSNorm(config.hidden_size, config.layer_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        # decode steps go through sgsa_decode_stack where it applies (False: always the per-layer path)
        self.decode_stack = True
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    def init_weights(self, std: float = 0.02, qk_std: Optional[float] = None, generator=None) -> None:
        """Normal(0, std) weights, zero biases, unit norms (:455-464).  qk_std replaces std for
        the SGSA layers' q / k / q_ret projections: at std 0.02 their keys leave the delta rule's
        stable range (|k|^2 ~ 0.0004 C D), as sgsa_amd.model.SGSAForCausalLM.init_weights explains."""
        with torch.no_grad():
            for name, p in self.named_parameters():
                if name.endswith("bias"):
                    p.zero_()
                elif p.dim() == 1:
                    p.fill_(1.0)
                else:
                    s = std
                    layer = int(name.split(".")[1]) if name.startswith("layers.") else -1
                    sgsa_qk = layer >= 0 and not self.config.is_dense(layer) and \
                        any(t in name for t in ("q_proj", "k_proj", "q_ret_proj"))
                    if qk_std is not None and sgsa_qk:
                        s = qk_std
                    p.copy_(torch.randn(p.shape, generator=generator, dtype=torch.float32) * s)

    def new_cache(self, B: int, T_max: int, device, dtype) -> List[dict]:
        cfg = self.config
        H, Hkv, D = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        caches = []
        for i in range(cfg.num_hidden_layers):
            if cfg.is_dense(i):
                caches.append({"k": torch.empty(B, Hkv, T_max, D, device=device, dtype=dtype),
                               "v": torch.empty(B, Hkv, T_max, D, device=device, dtype=dtype)})
            else:
                caches.append({"k": torch.empty(B, T_max, H, D, device=device, dtype=dtype),
                               "v": torch.empty(B, T_max, H, D, device=device, dtype=dtype),
                               "state": None, "cand": None})
        return caches

    def _head(self, h: Tensor) -> Tensor:
        return lin(self.lm_head, self.norm(h))

    @torch.no_grad()
    def prefill(self, input_ids: Tensor, caches: List[dict], rope: Tuple[Tensor, Tensor]) -> Tensor:
        """Runs the prompt [B, T]; fills the caches; returns logits [B, T, V]."""
        h = self.embed_tokens(input_ids)
        for layer, cache in zip(self.layers, caches):
            h = layer.forward_cached(h, 0, cache, rope) if isinstance(layer, DenseGQABlock) else layer.prefill(h, cache)
        return self._head(h)

    @torch.no_grad()
    def decode_step(self, tokens: Tensor, pos: int, step: int, caches: List[dict],
                    rope: Tuple[Tensor, Tensor]) -> Tensor:
        """tokens [B] at position pos, the step-th generated token; returns logits [B, V].
        SGSA layers select their top-k when step % topk_recompute_every == 0.

        Where the stack and its caches fit sgsa_decode_stack (bf16, head_dim 128, B <= 16,
        contiguous caches, top_k <= pos + 1), the whole layer loop is that one call: the
        same launches as the per-layer path below, without its Python dispatch, on copies
        of the weights tiled for the few-row products (made once per plan, about the size
        of the linears' weights; the same results bit for bit).  That call keeps its own
        candidate sets (it selects on its first step) and updates the SGSA states in place."""
        select = step % self.config.topk_recompute_every == 0
        h = self.embed_tokens(tokens[:, None])
        plan = self._stack_plan(caches, rope, h, pos)
        if plan is not None:
            B, C = h.shape[0], h.shape[-1]
            hb = h.view(B, C)
            _abi.check(_abi.lib().sgsa_decode_stack(
                ctypes.byref(plan["cfg"]), len(plan["layers"]), plan["layers"], _abi.ptr(hb), pos,
                int(select or not plan["primed"]), ctypes.c_void_p(plan["ws_ptr"]), plan["ws_bytes"],
                _abi.stream_of(hb)))
            plan["primed"] = True
            return self._head_tiled(h, plan)[:, 0]
        else:
            for layer, cache in zip(self.layers, caches):
                if isinstance(layer, DenseGQABlock):
                    h = layer.forward_cached(h, pos, cache, rope)
                else:
                    h = layer.decode(h, pos, cache, select)
        return self._head(h)[:, 0]

    def _stack_plan(self, caches: List[dict], rope: Tuple[Tensor, Tensor], h: Tensor, pos: int) -> Optional[dict]:
        """sgsa_decode_stack's arguments for these caches (built on first use and kept while the
        caches, states and parameters stay the same objects and versions), or None when the
        stack does not fit it and the per-layer path runs."""
        cfg = self.config
        B = h.shape[0]
        if not self.decode_stack or torch.is_grad_enabled() or not h.is_cuda or h.dtype != torch.bfloat16 or not h.is_contiguous() \
                or B > 16 or cfg.head_dim != 128 or pos + 1 < cfg.top_k:
            return None
        state_key = tuple(id(c.get("state")) for c in caches)
        pkey = tuple((id(p), p._version) for p in self.parameters())
        plan = self.__dict__.get("_decode_plan")
        if plan is not None and plan["caches"] is caches and plan["state_key"] == state_key \
                and plan["pkey"] == pkey and plan["rope"] is rope and plan["B"] == B:
            return plan
        self.__dict__["_decode_plan"] = None
        plan = self._build_stack_plan(caches, rope, B)
        if plan is not None:
            # a new plan selects on its first step; the per-layer path's candidate sets are
            # dropped, so that it also selects afresh should it take over later
            plan.update(caches=caches, state_key=state_key, pkey=pkey, rope=rope, B=B, primed=False)
            for c in caches:
                if "cand" in c:
                    c["cand"] = None
            self.__dict__["_decode_plan"] = plan
        return plan

    def _build_stack_plan(self, caches: List[dict], rope: Tuple[Tensor, Tensor], B: int) -> Optional[dict]:
        cfg = self.config
        C, H, Hkv, D, I = cfg.hidden_size, cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim, \
            cfg.intermediate_size
        if C % 32 or I % 32 or H % Hkv or H // Hkv not in (1, 2, 4, 8) or cfg.sgsa_write_mode not in ("direct", "residual"):
            return None
        bf = torch.bfloat16
        norms = [m.weight for l in self.layers for m in (l.input_norm, l.post_attn_norm)]
        if any(w.dtype != norms[0].dtype or not w.is_contiguous() for w in norms) or norms[0].dtype not in (bf, torch.float32):
            return None
        T_max = caches[0]["k"].shape[1] if not self.config.is_dense(0) else caches[0]["k"].shape[2]

        def ok(t, shape, dt=bf):
            return t is not None and t.is_cuda and t.dtype == dt and t.is_contiguous() and tuple(t.shape) == shape

        keep, layers = [], (_abi.SgsaDecodeLayer * len(self.layers))()
        for i, (layer, cache) in enumerate(zip(self.layers, caches)):
            dense = isinstance(layer, DenseGQABlock)
            names = ("q_proj", "k_proj", "v_proj") if dense else SGSADecoderBlock._PROJ
            w_in, b_in = fused_weight(layer, names)
            w_gu, b_gu = fused_weight(layer.mlp, ("gate_proj", "up_proj"))
            # gate and up rows interleaved in groups of 8 (the swiglu epilogue's layout)
            w_gu = torch.stack([w_gu[:I].view(I // 8, 8, C), w_gu[I:].view(I // 8, 8, C)], 1).reshape(2 * I, C)
            w_o, b_o, w_down = layer.o_proj.weight, layer.o_proj.bias, layer.mlp.down_proj.weight
            if b_gu is not None or layer.mlp.down_proj.bias is not None:
                return None
            n_in = (H + 2 * Hkv) * D if dense else 4 * H * D + 3 * H
            if not (ok(w_in, (n_in, C)) and ok(w_o, (C, H * D)) and ok(w_gu, (2 * I, C)) and ok(w_down, (C, I))
                    and (b_in is None or ok(b_in, (n_in,))) and (b_o is None or ok(b_o, (C,)))):
                return None
            L = layers[i]
            L.kind = 1 if dense else 0
            L.input_norm, L.post_norm = layer.input_norm.weight.data_ptr(), layer.post_attn_norm.weight.data_ptr()
            # the stack's linears read their weights tiled (one wave step's operand in one 1 KB piece)
            w_in, w_o, w_gu, w_down = (_tile_rows(w) for w in (w_in, w_o, w_gu, w_down))
            L.w_in, L.b_in = w_in.data_ptr(), (b_in.data_ptr() if b_in is not None else None)
            L.w_o, L.b_o = w_o.data_ptr(), (b_o.data_ptr() if b_o is not None else None)
            L.w_gu, L.w_down = w_gu.data_ptr(), w_down.data_ptr()
            keep += [w_in, b_in, w_o, b_o, w_gu, w_down]
            if dense:
                if not (ok(cache["k"], (B, Hkv, T_max, D)) and ok(cache["v"], (B, Hkv, T_max, D))):
                    return None
            else:
                st = cache.get("state")
                if not (ok(cache["k"], (B, T_max, H, D)) and ok(cache["v"], (B, T_max, H, D))
                        and ok(st, (B, H, D, D), torch.float32)):
                    return None
                idx = torch.zeros(B, H, cfg.top_k, device=st.device, dtype=torch.int32)
                cnt = torch.zeros(B, H, device=st.device, dtype=torch.int32)
                keep += [idx, cnt]
                L.state, L.cand_idx, L.cand_cnt = st.data_ptr(), idx.data_ptr(), cnt.data_ptr()
            L.k_cache, L.v_cache = cache["k"].data_ptr(), cache["v"].data_ptr()
        cos, sin = rope[0].float().contiguous(), rope[1].float().contiguous()
        keep += [cos, sin]
        lm_w, lm_b = self.lm_head.weight, self.lm_head.bias
        lm = None
        if ok(lm_w, (cfg.vocab_size, C)) and (lm_b is None or ok(lm_b, (cfg.vocab_size,))):
            lm = _tile_rows(lm_w)
        c = _abi.SgsaDecodeConfig(B=B, C=C, H=H, Hkv=Hkv, D=D, I=I, top_k=cfg.top_k,
                                  write_mode=0 if cfg.sgsa_write_mode == "direct" else 1, alpha_max=cfg.alpha_max,
                                  tau_c=cfg.tau_c, eps=self.layers[0].input_norm.eps,
                                  norm_w_f32=int(norms[0].dtype == torch.float32), cache_len=T_max,
                                  rope_cos=cos.data_ptr(), rope_sin=sin.data_ptr(), rope_len=cos.shape[0])
        nb = ctypes.c_size_t()
        _abi.check(_abi.lib().sgsa_decode_stack_workspace_size(ctypes.byref(c), ctypes.byref(nb)))
        ws = torch.empty(nb.value + 256, device=caches[0]["k"].device, dtype=torch.uint8)
        keep.append(ws)
        return {"cfg": c, "layers": layers, "keep": keep, "ws_ptr": (ws.data_ptr() + 255) // 256 * 256,
                "ws_bytes": nb.value, "lm": lm}

    def _head_tiled(self, h: Tensor, plan: dict) -> Tensor:
        """_head on the plan's tiled LM-head weight (sgsa_linear_rows_tiled: the same bits)."""
        if plan["lm"] is None:
            return self._head(h)
        n = self.norm(h)
        B, C = n.shape[0], n.shape[-1]
        V = self.lm_head.out_features
        y = torch.empty(B, 1, V, device=n.device, dtype=n.dtype)
        _abi.check(_abi.lib().sgsa_linear_rows_tiled(
            _abi.SGSA_BF16, B, V, C, _abi.ptr(n), C, _abi.ptr(plan["lm"]), _abi.ptr(self.lm_head.bias), _abi.ptr(y),
            V, _abi.stream_of(n)))
        return y


def _tile_rows(w: Tensor) -> Tensor:
    """w [N, K] bf16 in sgsa_linear_rows_tile's layout (16 ceil(N / 16) K elements)."""
    N, K = w.shape
    out = torch.empty(16 * ((N + 15) // 16) * K, device=w.device, dtype=w.dtype)
    _abi.check(_abi.lib().sgsa_linear_rows_tile(_abi.SGSA_BF16, N, K, _abi.ptr(w), _abi.ptr(out), _abi.stream_of(w)))
    return out


def expand_caches(caches: List[dict], B: int) -> List[dict]:
    """Caches of one sequence repeated for B sequences (prefill at B = 1, decode at B)."""
    out = []
    for c in caches:
        e = {}
        for name, t in c.items():
            e[name] = None if t is None else (t.expand(B, *t.shape[1:]).contiguous() if t.shape[0] == 1 else t)
        out.append(e)
    return out


@torch.no_grad()
def generate(model: HybridForCausalLM, prompt: Tensor, steps: int, batch: Optional[int] = None):
    """Greedy decoding: prefill ``prompt`` [Bp, T], then ``steps`` decode steps for ``batch``
    sequences (the prompt's caches repeated when Bp = 1).  Step s takes the previous
    greedy token (the prefill's for s = 0) at position T + s.  Returns (prefill logits
    [Bp, T, V], the tokens the decode steps produced [B, steps])."""
    cfg = model.config
    Bp, T = prompt.shape
    B = Bp if batch is None else batch
    if Bp != B and Bp != 1:
        raise ValueError("batch differs from the prompt batch, which must then be 1")
    dev, dt = prompt.device, model.embed_tokens.weight.dtype
    rope = rope_tables(T + steps, cfg.head_dim, cfg.rope_theta, dev)
    caches = model.new_cache(Bp, T + steps, dev, dt)
    logits = model.prefill(prompt, caches, rope)
    if B != Bp:
        caches = expand_caches(caches, B)
    tok = logits[:, -1].argmax(-1).expand(B).contiguous() if Bp == 1 else logits[:, -1].argmax(-1)
    out = torch.empty(B, steps, dtype=torch.long, device=dev)
    for s in range(steps):
        tok = model.decode_step(tok, T + s, s, caches, rope).argmax(-1)
        out[:, s] = tok
    return logits, out


def topk_kv_reuse_attention(query: Tensor, key: Tensor, value: Tensor, top_k: int,
                            attention_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Core of TopKSparseKVReuseAttention.forward (modelings/hybrid_dense_delta_topk.py:343-356)
    on the HIP kernels: the masked select (sgsa_score_topk_masked, kq_rule 1) and
    the V-only gather (sgsa_sparse_gather_masked), with no [B,H,Q,K] score matrix.

    query [B,Q,H,D] (RoPE applied); key, value [B,H,K,D], the dense layer's KV
    as the reference holds it; queries sit at key positions K-Q .. K-1 (:153-156);
    attention_mask [B,K] (nonzero = real token) or None.  Scores are
    q.k * 1/sqrt(D) (:343-344); future and padded keys are masked (:346,
    :166-175) and every row keeps min(top_k, K) slots (:348-349), the masked
    ones (score finfo.min, ties to the lowest index) with probability 0 unless
    a row has no unmasked key, whose slots then share it evenly, as the fp32
    softmax of equal scores does (:350).  Returns (attended [B,Q,H,D] in the
    value dtype, indices int64 [B,H,Q,k], probabilities float32 [B,H,Q,k]).
    """
    B, Q, H, D = query.shape
    K = key.shape[2]
    if key.shape != (B, H, K, D) or value.shape != key.shape:
        raise ValueError(f"key/value must be [B,H,K,D] = {(B, H, K, D)}; got {tuple(key.shape)} / {tuple(value.shape)}")
    if Q > K:
        raise ValueError(f"{Q} queries over {K} keys: the queries are the last Q positions of the KV")
    idx, sc, _, top2, _, fill = score_topk_masked(query, key, top_k, key_mask=attention_mask, causal=True,
                                                  q_offset=K - Q, scale_mode=1, kq_rule=1, kv_layout=1, sorted=True)
    r = gather_masked(None, value, idx, sc, None, top2, fill, q_offset=K - Q, kv_layout=1, return_weights=True)
    return r["v_hat"], idx.long(), r["weights"]


def topk_kv_reuse_attention_grad(query: Tensor, key: Tensor, value: Tensor, top_k: int,
                                 attention_mask: Optional[Tensor] = None, dropout_p: float = 0.0) -> Tensor:
    """``topk_kv_reuse_attention``'s attended [B,Q,H,D] in a form autograd differentiates
    in query, key and value: the masked select on the GPU under no_grad (the same kernel,
    slot rule and tie order; the indices are constants of the step, as torch.topk's are to
    autograd in the reference), then the selected slots' scores q.k / sqrt(D) (finfo.min on
    masked slots, :346), their fp32 softmax (:350) and the probability-weighted value rows
    (:351-356) as torch ops on the [B,H,Q,k,D] selected rows; ``dropout_p`` > 0 drops
    probabilities as training does (:351)."""
    B, Q, H, D = query.shape
    K = key.shape[2]
    if key.shape != (B, H, K, D) or value.shape != key.shape:
        raise ValueError(f"key/value must be [B,H,K,D] = {(B, H, K, D)}; got {tuple(key.shape)} / {tuple(value.shape)}")
    if Q > K:
        raise ValueError(f"{Q} queries over {K} keys: the queries are the last Q positions of the KV")
    n = B * H * Q * min(int(top_k), K) * D
    if n > MAX_SELECTED_ELEMS:
        raise ValueError(f"topk_kv_reuse_attention_grad: B*H*Q*k*D = {n} selected elements exceed "
                         f"{MAX_SELECTED_ELEMS}; train on shorter sequences or a smaller top_k")
    with torch.no_grad():
        idx, _, valid, _, _, _ = score_topk_masked(query.detach(), key.detach(), top_k, key_mask=attention_mask,
                                                   causal=True, q_offset=K - Q, scale_mode=1, kq_rule=1,
                                                   kv_layout=1, sorted=True)
        kk = idx.shape[-1]
        rows = (torch.arange(B * H, device=idx.device, dtype=torch.long).view(B, H, 1, 1) * K
                + idx.long()).reshape(-1)
        valid = valid.to(torch.bool)
    with torch.autocast("cuda", enabled=False):   # fp32 arithmetic also inside an autocast region
        qh = query.float().transpose(1, 2).contiguous()                       # [B,H,Q,D]
        ksel = key.float().reshape(B * H * K, D).index_select(0, rows).view(B, H, Q, kk, D)
        vsel = value.float().reshape(B * H * K, D).index_select(0, rows).view(B, H, Q, kk, D)
        sc = torch.matmul(ksel, qh.unsqueeze(-1)).squeeze(-1) * (1.0 / math.sqrt(D))
        sc = torch.where(valid, sc, torch.full_like(sc, torch.finfo(torch.float32).min))
        p = torch.softmax(sc, dim=-1)
        if dropout_p > 0:
            p = torch.nn.functional.dropout(p, p=dropout_p, training=True)
        out = torch.matmul(p.unsqueeze(-2), vsel).squeeze(-2)                 # [B,H,Q,D]
    return out.transpose(1, 2).to(value.dtype)


class TopKSparseKVReuseAttention(nn.Module):
    """Top-k sparse attention over the nearest previous dense layer's KV cache
    (modelings/hybrid_dense_delta_topk.py:317-358): q_proj, RoPE at offset
    K-Q, the masked top-k select and V-only gather of ``topk_kv_reuse_attention``,
    o_proj.  Same constructor config fields (num_attention_heads, head_dim or
    hidden_size, top_k, dropout) and forward signature.  Where autograd records
    it, the select stays on the GPU kernels and the softmax and the value sum
    take their differentiable form (``topk_kv_reuse_attention_grad``), so q_proj,
    o_proj, the hidden states and the dense KV get their gradients; in training
    mode with dropout > 0 the probabilities are dropped there as in the reference.
    """

    def __init__(self, config) -> None:
        super().__init__()
        self.config = config
        self.num_heads = config.num_attention_heads
        self.head_dim = config.head_dim
        self.top_k = config.top_k
        self.q_proj = nn.Linear(config.hidden_size, config.hidden_size, bias=False)
        self.o_proj = nn.Linear(config.hidden_size, config.hidden_size, bias=False)
        self.dropout_p = getattr(config, "dropout", 0.0)

    def forward(self, hidden_states: Tensor, dense_kv: Tuple[Tensor, Tensor], rope: Tuple[Tensor, Tensor],
                attention_mask: Optional[Tensor]) -> Tensor:
        B, Q, _ = hidden_states.shape
        key, value = dense_kv
        K = key.shape[-2]
        H, D = self.num_heads, self.head_dim
        if attention_mask is not None:
            if attention_mask.dim() != 2:
                raise ValueError("attention_mask must have shape [batch_size, kv_len]")
            if attention_mask.shape[-1] != K:
                raise ValueError("attention_mask length must match the current KV length")
        query = self.q_proj(hidden_states).view(B, Q, H, D)
        cos, sin = rope
        if cos.dim() == 4:   # the reference's [1, 1, S, D] tables
            cos, sin = cos[0, 0], sin[0, 0]
        off = K - Q
        c = cos[off:off + Q].to(query.dtype)[None, :, None, :]
        s = sin[off:off + Q].to(query.dtype)[None, :, None, :]
        half = D // 2
        query = query * c + torch.cat((-query[..., half:], query[..., :half]), dim=-1) * s
        grad = torch.is_grad_enabled() and (hidden_states.requires_grad or key.requires_grad or
                                            value.requires_grad or any(p.requires_grad for p in self.parameters()))
        drop = self.dropout_p if self.training else 0.0
        if grad or drop > 0:
            attended = topk_kv_reuse_attention_grad(query, key.to(query.dtype), value.to(query.dtype), self.top_k,
                                                    attention_mask, dropout_p=drop)
        else:
            attended, _, _ = topk_kv_reuse_attention(query.contiguous(), key.to(query.dtype), value.to(query.dtype),
                                                     self.top_k, attention_mask)
        return self.o_proj(attended.reshape(B, Q, H * D))
