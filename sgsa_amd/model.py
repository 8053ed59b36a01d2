"""The SGSA causal LM around the layer kernels: SGSABlock and SGSAForCausalLM.

Mirrors modelings/modeling_sgsa.py:634-767 (SGSABlock, SGSAForCausalLM) in every
retrieval mode (token_only, block_only, block_token) and state backend:

  h   = (embed(ids) + pos_embed(positions)) * attention_mask         (:739-743)
  per block (:669-709):
    n = RMSNorm(h);  q, k, v, q_ret = proj(n) as [B,T,H,D]
    beta  = sigmoid(beta_proj(n)).clamp_min(1e-4);  gamma = sigmoid(gamma_proj(n))   (:584-585)
    attended = SGSA layer(q, k, v, q_ret, beta, gamma, budget_proj(n))  -- K1, K2, K3-K5
    h = h + o_proj(attended) [+ lambda * sparse_out_proj(v_hat)]
    h = h + down(silu(gate(m)) * up(m)),  m = RMSNorm(h)
  logits = lm_head(RMSNorm(h))   (lm_head tied to the embedding by default)
  loss = cross_entropy(logits[:, :-1], labels[:, 1:], ignore_index=-100)  (:758-766)
  metrics: per layer alpha_mean, k_hat_perp_ratio_mean, retrieval_confidence_mean
           and the path flags (:697-708, :744-752)

The layer core runs in the HIP library: sgsa_layer_forward for token_only with
the chunked backend, else the retrieval half (sgsa_layer_retrieve or, in the
block modes, sgsa_block_layer_retrieve) followed by chunk_sgsa or
fused_recurrent_sgsa as ``linear_backend`` selects (:554-609).  The projections
and the MLP are GEMMs left to PyTorch (hipBLASLt); norms, gates and the MLP
activation are one HIP launch each.  RMSNorm and GatedMLP are the fla-core
modules the reference imports (modeling_sgsa.py:40-41); their arithmetic is the
in-tree restatement of modelings/hybrid_dense_delta_topk.py:94-117.

Training: under autograd the block selects on the GPU as above (K1, or the
block retrieval), then computes the weights, gathers, diagnostics and write
gate of the selected rows as differentiable torch ops (``retrieval_grad.py``,
the reference's own structure over the selected slots) and runs the state
update through chunk_sgsa / fused_recurrent_sgsa, whose backward is native;
every parameter gets its gradient, in every retrieval mode.
"""

from __future__ import annotations

from dataclasses import dataclass
import ctypes
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _abi

from .layer import LayerWorkspace, sgsa_block_layer_retrieve, sgsa_layer_forward, sgsa_layer_retrieve
from .ops import chunk_sgsa
from .recurrent import fused_recurrent_sgsa
from .retrieval_grad import retrieve_block_differentiable, retrieve_differentiable

Tensor = torch.Tensor


@dataclass
class SGSAConfig:
    """SGSAConfig of modelings/modeling_sgsa.py:47-78: the same fields and defaults."""

    vocab_size: int = 32000
    hidden_size: int = 256
    intermediate_size: int = 512
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_kv_heads: int = 4
    max_position_embeddings: int = 2048
    dropout: float = 0.0
    layer_norm_eps: float = 1e-6
    pad_token_id: int = 0
    top_k: int = 16
    block_size: int = 32
    top_blocks: int = 2
    retrieval_mode: str = "block_token"   # token_only | block_only | block_token
    sgsa_write_mode: str = "direct"       # none | direct | residual
    alpha_max: float = 0.25
    tau_c: float = 0.1
    local_window: int = 64
    sink_size: int = 8
    sparse_output_lambda: float = 0.0
    tie_word_embeddings: bool = True
    linear_backend: str = "auto"   # auto | python | torch_chunk | recurrent | triton_recurrent | fla_gdn
    retrieval_backend: str = "auto"   # auto | torch | flash_moba (flash_moba absent: the torch path's semantics)
    chunk_size: int = 64

    @property
    def head_dim(self) -> int:
        if self.hidden_size % self.num_attention_heads != 0:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        return self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight, evaluated in fp32 and stored in x's dtype, in one
    HIP launch (sgsa_rms_norm; hybrid_dense_delta_topk.py:94-103); under autograd, the same
    arithmetic as torch ops so that gradients flow."""

    def __init__(self, hidden_size: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        if not x.is_cuda:
            raise ValueError("RMSNorm: the SGSA model runs on a ROCm GPU; got a CPU tensor")
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad):
            # Under autograd: the same fp32 arithmetic as differentiable torch ops, so
            # gradients reach x and the norm weight (the HIP launch has no backward).
            xf = x.float()
            y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps) * self.weight.float()
            return y.to(x.dtype)
        xc = x.contiguous()
        C = xc.shape[-1]
        w = self.weight
        if w.dtype != x.dtype and w.dtype != torch.float32:
            w = w.float()
        w = w.contiguous()
        y = torch.empty_like(xc)
        _abi.check(_abi.lib().sgsa_rms_norm(_abi.dtype_code(x.dtype), int(w.dtype == torch.float32),
                                            xc.numel() // C, C, _abi.ptr(xc), _abi.ptr(w), float(self.eps),
                                            _abi.ptr(y), _abi.stream_of(xc)))
        return y

    def add_forward(self, a: Tensor, b: Tensor) -> Tuple[Tensor, Tensor]:
        """(a + b, self(a + b)): the residual add and this norm; without autograd in one
        launch (sgsa_add_rms_norm) with the same roundings as the two steps."""
        if torch.is_grad_enabled() or a.shape != b.shape or a.dtype != b.dtype or not a.is_cuda:
            h = a + b
            return h, self(h)
        ac, bc = a.contiguous(), b.contiguous()
        C = ac.shape[-1]
        w = self.weight
        if w.dtype != a.dtype and w.dtype != torch.float32:
            w = w.float()
        w = w.contiguous()
        h, y = torch.empty_like(ac), torch.empty_like(ac)
        _abi.check(_abi.lib().sgsa_add_rms_norm(_abi.dtype_code(a.dtype), int(w.dtype == torch.float32),
                                                ac.numel() // C, C, _abi.ptr(ac), _abi.ptr(bc), _abi.ptr(h),
                                                _abi.ptr(w), float(self.eps), _abi.ptr(y), _abi.stream_of(ac)))
        return h, y


def linear_rows(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """F.linear(x, weight, bias).  Without autograd, for bf16 x of at most 16 rows (a decode
    step's tokens), one sgsa_linear_rows launch: a library GEMM's host dispatch costs more
    than such a product."""
    shape = x.shape
    K = shape[-1]
    M = x.numel() // K if K else 0
    if M > 16 or M < 1 or K % 32 != 0 or x.dtype != _BF16 or weight.dtype != _BF16 or torch.is_grad_enabled() \
            or not x.is_cuda or not _weight_ok(weight, bias):
        return F.linear(x, weight, bias)
    x2 = x if x.dim() == 2 else x.reshape(M, K)
    xs = x2.stride(0) if M > 1 else K
    xp = x2.data_ptr()
    if x2.stride(-1) != 1 or xs % 8 != 0 or xp % 16 != 0:
        return F.linear(x, weight, bias)
    N = weight.shape[0]
    y = torch.empty(shape[:-1] + (N,), device=x.device, dtype=_BF16)
    _abi.check(_LINEAR_ROWS(_abi.SGSA_BF16, M, N, K, ctypes.c_void_p(xp), xs, ctypes.c_void_p(weight.data_ptr()),
                            _abi.ptr(bias), ctypes.c_void_p(y.data_ptr()), N, _abi.stream_of(x)))
    return y


_BF16 = torch.bfloat16
_LINEAR_ROWS = None
_WEIGHT_OK: dict = {}


def _weight_ok(weight: Tensor, bias: Optional[Tensor]) -> bool:
    """weight (and bias) fit sgsa_linear_rows: bf16, contiguous, 16-byte aligned; remembered per
    (address, version, shape, strides, dtype) of each, so that a strided view of a checked
    weight is checked on its own, and the library's entry point looked up once."""
    global _LINEAR_ROWS
    key = (weight.data_ptr(), weight._version, tuple(weight.shape), weight.stride(), weight.dtype,
           None if bias is None else (bias.data_ptr(), bias._version, tuple(bias.shape), bias.stride(), bias.dtype))
    ok = _WEIGHT_OK.get(key)
    if ok is None:
        ok = weight.is_contiguous() and weight.data_ptr() % 16 == 0 and \
            (bias is None or (bias.dtype == _BF16 and bias.is_contiguous()))
        if len(_WEIGHT_OK) > 4096:
            _WEIGHT_OK.clear()
        _WEIGHT_OK[key] = ok
        if _LINEAR_ROWS is None:
            _LINEAR_ROWS = _abi.lib().sgsa_linear_rows
    return ok


def lin(module: nn.Linear, x: Tensor) -> Tensor:
    """module(x) through linear_rows."""
    return linear_rows(x, module.weight, module.bias)


def fused_linear(module: nn.Module, x: Tensor, names) -> list:
    """The outputs of the nn.Linear children ``names`` of ``module`` on the same input x.

    Without autograd they come from one GEMM over the concatenated weights (views of
    its output, split along the last dimension); the concatenation is cached on the
    module and rebuilt when any weight or bias changes (storage or in-place version).
    With autograd on, each projection runs on its own so gradients reach its weight.
    """
    lins = [getattr(module, n) for n in names]
    if torch.is_grad_enabled():
        return [lin(x) for lin in lins]
    y = fused_linear_out(module, x, names)
    return list(torch.split(y, [l.out_features for l in lins], dim=-1))


def fused_weight(module: nn.Module, names) -> Tuple[Tensor, Optional[Tensor]]:
    """(weight, bias) of the nn.Linear children ``names`` of ``module`` concatenated along the
    output dimension (bias None when none has one; zeros for those without), cached on the
    module and rebuilt when any weight or bias changes (storage or in-place version)."""
    lins = [getattr(module, n) for n in names]
    key = tuple((l.weight.data_ptr(), l.weight._version,
                 None if l.bias is None else (l.bias.data_ptr(), l.bias._version)) for l in lins)
    cached = module.__dict__.get("_fused_" + "_".join(names))
    if cached is None or cached[0] != key:
        w = torch.cat([l.weight for l in lins], 0)
        b = None
        if any(l.bias is not None for l in lins):
            b = torch.cat([l.bias if l.bias is not None else l.weight.new_zeros(l.out_features) for l in lins])
        cached = (key, w, b)
        module.__dict__["_fused_" + "_".join(names)] = cached
    return cached[1], cached[2]


def fused_linear_out(module: nn.Module, x: Tensor, names) -> Tensor:
    """The one GEMM of fused_linear (no autograd): the outputs of the nn.Linear children
    ``names`` side by side along the last dimension of one contiguous tensor."""
    w, b = fused_weight(module, names)
    return linear_rows(x, w, b)


class GatedMLP(nn.Module):
    """down(silu(gate(x)) * up(x))."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        if torch.is_grad_enabled() or x.dtype not in (torch.float32, torch.bfloat16) or not x.is_cuda:
            gate, up = fused_linear(self, x, ("gate_proj", "up_proj"))
            return self.down_proj(F.silu(gate) * up)
        # one launch for silu(gate) * up on the fused projection (sgsa_silu_mul)
        gu = fused_linear_out(self, x, ("gate_proj", "up_proj"))
        I = self.gate_proj.out_features
        act = torch.empty(*gu.shape[:-1], I, device=gu.device, dtype=gu.dtype)
        _abi.check(_abi.lib().sgsa_silu_mul(_abi.dtype_code(gu.dtype), gu.numel() // (2 * I), I, _abi.ptr(gu),
                                            gu.stride(-2) if gu.dim() > 1 else 2 * I, _abi.ptr(act),
                                            _abi.stream_of(gu)))
        return lin(self.down_proj, act)


# linear_backend -> the state update SGSAStateLayer.forward runs (modeling_sgsa.py:554-609).  fla is
# not part of this build, so "fla_gdn" and "python" take the reference's last branch, the token
# recurrence naive_recurrent_sgsa, whose semantics the recurrent kernel computes.
_STATE_BACKENDS = {"auto": "chunk", "torch_chunk": "chunk", "recurrent": "recurrent",
                   "triton_recurrent": "recurrent", "fused_recurrent": "recurrent", "python": "naive",
                   "fla_gdn": "naive"}
_RETRIEVAL_MODES = ("token_only", "block_only", "block_token")


def needs_grad(module: nn.Module, *inputs: Tensor) -> bool:
    """Whether autograd records ``module`` on ``inputs``."""
    return torch.is_grad_enabled() and (any(t.requires_grad for t in inputs) or
                                        any(p.requires_grad for p in module.parameters()))


class SGSABlock(nn.Module):
    def __init__(self, config: SGSAConfig) -> None:
        super().__init__()
        if config.retrieval_mode not in _RETRIEVAL_MODES:
            raise ValueError(f"retrieval_mode must be one of {_RETRIEVAL_MODES}, got {config.retrieval_mode!r}")
        if config.num_kv_heads != config.num_attention_heads:
            raise ValueError("the SGSA block uses one key/value head per query head")
        if config.sgsa_write_mode not in ("none", "direct", "residual"):
            raise ValueError("sgsa_write_mode must be 'none', 'direct' or 'residual'")
        if config.linear_backend not in _STATE_BACKENDS:
            raise ValueError(f"linear_backend must be one of {sorted(_STATE_BACKENDS)}, got {config.linear_backend!r}")
        if config.retrieval_backend not in ("auto", "torch", "flash_moba"):
            raise ValueError(f"retrieval_backend must be auto, torch or flash_moba, got {config.retrieval_backend!r}")
        if not 0.0 <= config.dropout < 1.0:
            raise ValueError(f"dropout must be in [0, 1), got {config.dropout}")
        self.config = config
        H, D, C = config.num_attention_heads, config.head_dim, config.hidden_size
        self.num_heads, self.head_dim = H, D
        self.input_norm = RMSNorm(C, config.layer_norm_eps)
        self.post_attn_norm = RMSNorm(C, config.layer_norm_eps)
        self.q_proj = nn.Linear(C, H * D, bias=False)
        self.k_proj = nn.Linear(C, H * D, bias=False)
        self.v_proj = nn.Linear(C, H * D, bias=False)
        self.o_proj = nn.Linear(C, C, bias=False)
        self.q_ret_proj = nn.Linear(C, H * D, bias=False)
        self.sparse_out_proj = nn.Linear(C, C, bias=False)
        # SGSAStateLayer's gates (modeling_sgsa.py:480-482)
        self.beta_proj = nn.Linear(C, H, bias=True)
        self.gamma_proj = nn.Linear(C, H, bias=True)
        self.budget_proj = nn.Linear(C, H, bias=True)
        self.mlp = GatedMLP(C, config.intermediate_size)
        self._ws = LayerWorkspace()

    def _project(self, h: Tensor):
        """q, k, v, q_ret [B,T,H,D] and beta, gamma, budget [B,T,H] (fp32) of the block's input."""
        B, T, C = h.shape
        H, D = self.num_heads, self.head_dim
        n = self.input_norm(h)
        q, k, v, q_ret, bl, gl, ul = fused_linear(
            self, n, ("q_proj", "k_proj", "v_proj", "q_ret_proj", "beta_proj", "gamma_proj", "budget_proj"))
        if torch.is_grad_enabled():
            beta = torch.sigmoid(bl.float()).clamp_min(1e-4)
            gamma = torch.sigmoid(gl.float())
            budget = ul.float()
        else:
            # bl, gl, ul are consecutive H-wide groups of one projection row: one launch for all three
            beta, gamma, budget = (torch.empty(B, T, H, device=h.device, dtype=torch.float32) for _ in range(3))
            _abi.check(_abi.lib().sgsa_layer_gates(_abi.dtype_code(bl.dtype), B * T, H, _abi.ptr(bl), bl.stride(-2),
                                                   _abi.ptr(beta), _abi.ptr(gamma), _abi.ptr(budget),
                                                   _abi.stream_of(bl)))
        return (q.view(B, T, H, D), k.view(B, T, H, D), v.view(B, T, H, D), q_ret.view(B, T, H, D), beta, gamma,
                budget)

    def forward(self, h: Tensor, attention_mask: Optional[Tensor] = None) -> Tuple[Tensor, Dict[str, Tensor]]:
        """SGSABlock.forward (modeling_sgsa.py:660-709): (hidden states, metrics).

        attention_mask [B,T] (nonzero = real token) reaches the retrieval only
        (:668-674).  ``retrieval_mode`` picks the token or block retrieval
        (:430-463), ``sgsa_write_mode`` "none" drops the sparse write from the
        state update while alpha is still reported (:543-552, :557-609), and
        ``linear_backend`` the chunked or the token-recurrent update (:554-609).
        The metrics are the reference's: alpha_mean, k_hat_perp_ratio_mean
        (residual write mode, else 0), retrieval_confidence_mean (mean largest
        retrieval weight) and the path flags.

        Under autograd the retrieval and the write gate take their
        differentiable form (``retrieval_grad.py``: the selection on the GPU,
        then the weights, gathers and gate as torch ops on the selected rows)
        and the state update its native backward, so every projection gets its
        gradient, in every retrieval mode.
        """
        grad = needs_grad(self, h)
        cfg = self.config
        B, T, C = h.shape
        q, k, v, q_ret, beta, gamma, budget = self._project(h)
        stats: Dict[str, Tensor] = {}
        backend = _STATE_BACKENDS[cfg.linear_backend]
        sparse = cfg.sgsa_write_mode != "none"
        # with write_mode "none" the reference's write key is k_hat (:546-550): alpha as "direct"
        wm = "residual" if cfg.sgsa_write_mode == "residual" else "direct"
        vh = None
        if grad:
            if cfg.retrieval_mode == "token_only":
                wk, vh, al, stats = retrieve_differentiable(q_ret, k, v, budget, cfg.top_k, wm, cfg.alpha_max,
                                                            cfg.tau_c, attention_mask=attention_mask)
            else:
                wk, vh, al, stats = retrieve_block_differentiable(q_ret, k, v, budget, cfg.top_k, cfg.block_size,
                                                                  cfg.top_blocks, cfg.retrieval_mode, wm,
                                                                  cfg.alpha_max, cfg.tau_c,
                                                                  attention_mask=attention_mask)
            sk, sv, sa = (wk, vh, al) if sparse else (None, None, None)
            if backend == "chunk":
                att, _ = chunk_sgsa(q, k, v, beta, gamma, sk, sv, sa)
            else:
                att, _ = fused_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, sa)
        elif cfg.retrieval_mode == "token_only" and backend == "chunk" and sparse and cfg.sparse_output_lambda <= 0:
            att, _ = sgsa_layer_forward(q, k, v, q_ret, beta, gamma, budget, cfg.top_k, write_mode=wm,
                                        alpha_max=cfg.alpha_max, tau_c=cfg.tau_c, output_final_state=False,
                                        workspace=self._ws, attention_mask=attention_mask, stats=stats)
        else:
            if cfg.retrieval_mode == "token_only":
                wk, vh, al = sgsa_layer_retrieve(q_ret, k, v, budget, cfg.top_k, wm, cfg.alpha_max, cfg.tau_c,
                                                 workspace=self._ws, attention_mask=attention_mask, stats=stats)
            else:
                wk, vh, al = sgsa_block_layer_retrieve(q_ret, k, v, budget, cfg.top_k, cfg.block_size,
                                                       cfg.top_blocks, cfg.retrieval_mode, wm, cfg.alpha_max,
                                                       cfg.tau_c, workspace=self._ws, attention_mask=attention_mask,
                                                       stats=stats)
            sk, sv, sa = (wk, vh, al) if sparse else (None, None, None)
            if backend == "chunk":
                att, _ = chunk_sgsa(q, k, v, beta, gamma, sk, sv, sa)
            else:
                att, _ = fused_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, sa)
        out = self.o_proj(att.reshape(B, T, C))
        if cfg.sparse_output_lambda > 0:
            out = out + cfg.sparse_output_lambda * self.sparse_out_proj(vh.reshape(B, T, C))
        if self.training and cfg.dropout > 0:   # the residual branch's dropout (:651, :695)
            out = F.dropout(out, p=cfg.dropout, training=True)
        h, n = self.post_attn_norm.add_forward(h, out)
        h = h + self.mlp(n)
        rs = stats["row_stats"]
        zero = torch.zeros((), device=h.device)
        one = torch.ones((), device=h.device)
        metrics = {
            "alpha_mean": stats["alpha"].mean(),
            "k_hat_perp_ratio_mean": rs[1].mean() if cfg.sgsa_write_mode == "residual" else h.new_zeros(()),
            "retrieval_confidence_mean": rs[0].mean(),
            "used_fla_gdn": zero,
            "used_torch_chunk": one if backend == "chunk" else zero,
            "used_recurrent": one if backend == "recurrent" else zero,
        }
        return h, metrics


class SGSAForCausalLM(nn.Module):
    def __init__(self, config: SGSAConfig) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, padding_idx=config.pad_token_id)
        self.pos_embed = nn.Embedding(config.max_position_embeddings, config.hidden_size)
        self.layers = nn.ModuleList([SGSABlock(config) for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.layer_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    def init_weights(self, std: float = 0.02, qk_std: Optional[float] = None, generator=None) -> None:
        """Normal(0, std) for every Linear / Embedding weight, zero biases (modeling_sgsa.py:727-733).

        qk_std, if given, replaces std for q_proj, k_proj and q_ret_proj.  With the
        reference's std = 0.02 at hidden size C the keys have |k|^2 ~ 0.0004 C D, and
        the delta-rule transition 1 - beta |k|^2 leaves the unit disc once that exceeds
        ~4 (C = 1024, D = 128 gives ~52): the state then grows without bound, in the
        reference as here.  qk_std = 1 / sqrt(C D) keeps |k| ~ 1.
        """
        with torch.no_grad():
            for name, p in self.named_parameters():
                if name.endswith("bias"):
                    p.zero_()
                elif p.dim() == 1:   # norm weights
                    p.fill_(1.0)
                else:
                    s = std
                    if qk_std is not None and any(t in name for t in ("q_proj", "k_proj", "q_ret_proj")):
                        s = qk_std
                    p.copy_(torch.randn(p.shape, generator=generator, dtype=torch.float32) * s)

    def forward(self, input_ids: Tensor, attention_mask: Optional[Tensor] = None,
                labels: Optional[Tensor] = None) -> Dict[str, object]:
        """SGSAForCausalLM.forward (modeling_sgsa.py:733-767): {"logits", "metrics"}
        and, with labels, "loss" -- the next-token cross entropy with ignore_index
        -100 (:758-766).  attention_mask [B,T] zeroes the padded embeddings
        (:740-741) and masks padded keys and queries in every retrieval.  Trains
        (autograd through every layer) with retrieval_mode token_only."""
        B, T = input_ids.shape
        if T > self.config.max_position_embeddings:
            raise ValueError("sequence length exceeds max_position_embeddings")
        pos = torch.arange(T, device=input_ids.device)
        h = self.embed_tokens(input_ids) + self.pos_embed(pos)[None]
        if attention_mask is not None:
            h = h * attention_mask.unsqueeze(-1).to(h.dtype)
        metrics: Dict[str, Tensor] = {}
        for i, layer in enumerate(self.layers):
            h, m = layer(h, attention_mask=attention_mask)
            for name in ("alpha_mean", "k_hat_perp_ratio_mean", "retrieval_confidence_mean", "used_fla_gdn",
                         "used_torch_chunk", "used_recurrent"):
                metrics[f"layer_{i}_{name}"] = m[name]
        logits = self.lm_head(self.norm(h))
        out: Dict[str, object] = {"logits": logits, "metrics": metrics}
        if labels is not None:
            shift_logits = logits[:, :-1, :].contiguous()
            shift_labels = labels[:, 1:].contiguous()
            out["loss"] = F.cross_entropy(shift_logits.view(-1, shift_logits.size(-1)), shift_labels.view(-1),
                                          ignore_index=-100)
        return out
