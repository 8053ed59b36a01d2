"""ctypes binding of libsgsa_hip.so (the C ABI declared in include/sgsa.h).

The library is loaded from the package directory; if it is missing this
raises -- there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsgsa_hip.so")

SGSA_F32 = 0
SGSA_BF16 = 1
NDIAG = 10
DIAG_NAMES = (
    "score_margin",
    "concentration",
    "max_confidence",
    "novelty",
    "write_conflict",
    "entropy",
    "avg_distance",
    "local_ratio",
    "sink_ratio",
    "remote_ratio",
)

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "sgsa_abi_version": (_I, []),
    "sgsa_status_string": (ctypes.c_char_p, [_I]),
    "sgsa_last_error": (ctypes.c_char_p, []),
    "sgsa_chunk_fwd_workspace_size": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_chunk_fwd": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_chunk_bwd_workspace_size": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_chunk_bwd": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            _P, _P, _P, _P, _SZ, _P]),
    "sgsa_score_topk_workspace_size": (_I, [_I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_score_topk_fast_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_score_topk": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P,
                             _SZ, _P]),
    "sgsa_score_topk_noalloc": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _P, _P, _I,
                                     _P]),
    "sgsa_score_topk_masked_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_score_topk_masked": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P, _P, _P, _P, _P, _P,
                                    _P, _P, _P, _P, _I, _P, _SZ, _P]),
    "sgsa_sparse_gather_masked": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                       _I, _F, _F, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_layer_fwd_stats": (_I, [_I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P,
                                  _P, _P, _P, _SZ, _P]),
    "sgsa_layer_retrieve_stats": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _F, _F, _P, _P, _P, _P, _P,
                                       _SZ, _P]),
    "sgsa_sparse_gather_tiled": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P, _P,
                                      _P, _P]),
    "sgsa_score_dump": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _I, _I, _P, _P]),
    "sgsa_sparse_gather": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F,
                                _I, _I, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_sparse_gather_workspace_size": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_rms_norm": (_I, [_I, _I, ctypes.c_long, _I, _P, _P, _F, _P, _P]),
    "sgsa_add_rms_norm": (_I, [_I, _I, ctypes.c_long, _I, _P, _P, _P, _P, _F, _P, _P]),
    "sgsa_linear_rows": (_I, [_I, _I, _I, _I, _P, ctypes.c_long, _P, _P, _P, ctypes.c_long, _P]),
    "sgsa_linear_rows_tile": (_I, [_I, _I, _I, _P, _P, _P]),
    "sgsa_linear_rows_tiled": (_I, [_I, _I, _I, _I, _P, ctypes.c_long, _P, _P, _P, ctypes.c_long, _P]),
    "sgsa_silu_mul": (_I, [_I, ctypes.c_long, _I, _P, ctypes.c_long, _P, _P]),
    "sgsa_layer_gates": (_I, [_I, ctypes.c_long, _I, _P, ctypes.c_long, _P, _P, _P, _P]),
    "sgsa_rope_qk": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P, ctypes.c_long, _P, _P, _P, _P, _P]),
    "sgsa_dense_attention": (_I, [_I, _I, _I, _I, _I, _I, _I, _P, _P, _P, ctypes.c_long, _P, _P, ctypes.c_size_t, _P]),
    "sgsa_decode_attention_workspace_size": (_I, [_I, _I, _I, _I, ctypes.POINTER(ctypes.c_size_t)]),
    "sgsa_decode_attention": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, ctypes.c_long, _I, _P, _P, ctypes.c_size_t, _P]),
    "sgsa_decode_split": (_I, [_I, _I, _I, _I, _P, ctypes.c_long, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               ctypes.c_long, ctypes.c_long, _P]),
    "sgsa_score_at": (_I, [_I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _P]),
    "sgsa_block_retrieve_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_block_retrieve": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P, _P, _P, _P, _P,
                                 _P, _P, _P, _P, _SZ, _P]),
    "sgsa_block_retrieve_masked": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P, _P, _P, _P,
                                        _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_block_layer_retrieve_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_block_layer_retrieve": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _I, _F, _P,
                                       _P, _P, _P, _P, _SZ, _P]),
    "sgsa_layer_retrieve_masked_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_layer_retrieve_masked": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P, _P, _P,
                                        _P, _SZ, _P]),
    "sgsa_layer_fwd_workspace_size": (_I, [_I, _I, _I, _I, _I, _I, ctypes.POINTER(_SZ)]),
    "sgsa_layer_fwd": (_I, [_I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P,
                            _P, _SZ, _P]),
    "sgsa_recurrent_fwd": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sgsa_topk_lists_size": (_I, [_I, _I, _I, _I, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "sgsa_score_topk_lists": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_sparse_gather_lists": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P, _P,
                                      _P, _P]),
    "sgsa_score_topk_thresholds": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "sgsa_sparse_gather_thresholds": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _F, _F, _P, _P,
                                           _P, _P, _P]),
    "sgsa_gather_thresholds_selection": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sgsa_layer_retrieve": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _F, _F, _P, _P, _P, _P, _SZ, _P]),
}

class SgsaDecodeConfig(ctypes.Structure):
    """struct SgsaDecodeConfig of include/sgsa.h."""
    _fields_ = [("B", _I), ("C", _I), ("H", _I), ("Hkv", _I), ("D", _I), ("I", _I), ("top_k", _I),
                ("write_mode", _I), ("alpha_max", _F), ("tau_c", _F), ("eps", _F), ("norm_w_f32", _I),
                ("cache_len", ctypes.c_long), ("rope_cos", _P), ("rope_sin", _P), ("rope_len", _I)]


class SgsaDecodeLayer(ctypes.Structure):
    """struct SgsaDecodeLayer of include/sgsa.h."""
    _fields_ = [("kind", _I), ("input_norm", _P), ("post_norm", _P), ("w_in", _P), ("b_in", _P), ("w_o", _P),
                ("b_o", _P), ("w_gu", _P), ("w_down", _P), ("k_cache", _P), ("v_cache", _P), ("state", _P),
                ("cand_idx", _P), ("cand_cnt", _P)]


SIGNATURES["sgsa_decode_stack_workspace_size"] = (_I, [ctypes.POINTER(SgsaDecodeConfig), ctypes.POINTER(_SZ)])
SIGNATURES["sgsa_decode_stack"] = (_I, [ctypes.POINTER(SgsaDecodeConfig), _I, ctypes.POINTER(SgsaDecodeLayer), _P, _I,
                                        _I, _P, _SZ, _P])

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library with typed entry points."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m sgsa_amd.build`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class SGSAError(RuntimeError):
    pass


def check(status: int) -> None:
    if status == 0:
        return
    L = lib()
    msg = f"{L.sgsa_status_string(status).decode()}: {L.sgsa_last_error().decode()}"
    if status in (1, 2, 4):
        raise ValueError(msg)
    raise SGSAError(msg)


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current stream of t's device (torch's raw-stream query when present: the
    Stream object of torch.cuda.current_stream costs several microseconds per call)."""
    if t.is_cuda:
        if _raw_stream is not None:
            return ctypes.c_void_p(_raw_stream(t.device.index))
        return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
    return None


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return SGSA_F32
    if dt == torch.bfloat16:
        return SGSA_BF16
    raise ValueError(f"unsupported dtype {dt}: the SGSA kernels take float32 or bfloat16")
