"""SGSA layer forward on AMD MI355X (gfx950): HIP kernels behind a C ABI.

Public entry points mirror FAndromedA/sgsa:
  chunk_sgsa            -- modelings/sgsa_ops/chunk.py:104-148
  chunk_sgsa_bwd        -- its gradients, native (the reference recomputes in torch, chunk_bwd.py:12-77)
  SparseRetriever       -- modelings/modeling_sgsa.py:90-474 (token_only, block_only, block_token)
  sparse_retrieve       -- functional form of SparseRetriever.forward
  sgsa_layer_forward    -- retrieval + write gate + chunked state update in one call
  sgsa_layer_retrieve   -- its retrieval half: (write key, v_hat, alpha)
  sgsa_block_layer_retrieve -- the same in the block retrieval modes
  fused_recurrent_sgsa  -- token-by-token recurrence (decode step), recurrent.py:138-175
  sgsa_decode_step      -- one generated token: retrieval over the KV cache, gate, recurrent update
  SGSAForCausalLM       -- the causal LM around the layer, modeling_sgsa.py:634-767 (every retrieval mode, forward)
The compiled library (libsgsa_hip.so) is required; there is no fallback path.
"""

from .ops import ChunkSGSAFunction, chunk_sgsa, chunk_sgsa_bwd, chunk_sgsa_fwd
from .retrieval import (SparseRetriever, block_retrieve, gather_gate, gather_lists, gather_masked, gather_thresholds,
                        masked_gather_gate, score_dump, gather_thresholds_selection, selection_summary, score_topk, score_topk_lists, score_topk_masked,
                        score_topk_thresholds, sparse_retrieve)
from .layer import LayerWorkspace, sgsa_block_layer_retrieve, sgsa_layer_forward, sgsa_layer_retrieve
from .recurrent import fused_recurrent_sgsa
from .decode import sgsa_decode_step
from .model import SGSABlock, SGSAConfig, SGSAForCausalLM
from .hybrid import TopKSparseKVReuseAttention, topk_kv_reuse_attention

__all__ = [
    "ChunkSGSAFunction",
    "chunk_sgsa",
    "chunk_sgsa_fwd",
    "chunk_sgsa_bwd",
    "fused_recurrent_sgsa",
    "sgsa_decode_step",
    "SparseRetriever",
    "score_topk",
    "score_topk_masked",
    "gather_masked",
    "masked_gather_gate",
    "topk_kv_reuse_attention",
    "TopKSparseKVReuseAttention",
    "score_dump",
    "gather_gate",
    "gather_lists",
    "gather_thresholds",
    "score_topk_lists",
    "score_topk_thresholds",
    "sparse_retrieve",
    "block_retrieve",
    "sgsa_layer_forward",
    "sgsa_layer_retrieve",
    "sgsa_block_layer_retrieve",
    "LayerWorkspace",
    "SGSAConfig",
    "SGSABlock",
    "SGSAForCausalLM",
]
