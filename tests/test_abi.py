"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the GPU."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from sgsa_amd import _abi
    if not os.path.exists(_abi.LIB_PATH):
        pytest.fail("libsgsa_hip.so is not built (run `python -m sgsa_amd.build`)")
    return _abi, _abi.lib()


def _header_functions():
    text = open(os.path.join(ROOT, "include", "sgsa.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sgsa_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_header_symbol():
    abi, L = _lib()
    names = _header_functions()
    assert names, "no functions parsed from include/sgsa.h"
    for n in names:
        assert hasattr(L, n), f"{n} declared in sgsa.h but not exported"
    assert set(names) == set(abi.SIGNATURES), "ctypes signature table out of sync with sgsa.h"


def test_abi_version_and_status_strings():
    abi, L = _lib()
    assert L.sgsa_abi_version() == 1
    assert L.sgsa_status_string(0) == b"ok"
    assert L.sgsa_status_string(4) == b"workspace too small"


def test_workspace_size_queries():
    abi, L = _lib()
    n = ctypes.c_size_t()
    assert L.sgsa_chunk_fwd_workspace_size(1, 32768, 16, 128, 1, ctypes.byref(n)) == 0
    assert n.value > 16 * 512 * 128 * 128 * 4
    chunk = n.value
    assert L.sgsa_layer_fwd_workspace_size(1, 1, 32768, 16, 128, 2048, ctypes.byref(n)) == 0
    # bf16, D = 128 (threshold form): chunk workspace, K1's threshold-bin candidate
    # lists (512 x 8 B per row), the per-row cut (8 B), write key and v_hat
    rows = 16 * 32768
    assert n.value > chunk + rows * 512 * 8 + rows * 8 + 2 * rows * 128 * 2
    assert n.value < chunk + rows * 2048 * 8   # no per-row index/score lists
    assert L.sgsa_layer_fwd_workspace_size(0, 1, 4096, 4, 64, 256, ctypes.byref(n)) == 0
    assert n.value > 2 * 4 * 4096 * 256 * 4     # fp32: row lists (indices + scores)


@pytest.mark.parametrize("call,needle", [
    (lambda L, p: L.sgsa_chunk_fwd(7, 1, 8, 1, 64, 64, p, p, p, p, p, None, None, None, None, p, None, p, 1 << 30, None),
     "dtype"),
    (lambda L, p: L.sgsa_chunk_fwd(0, 1, 8, 1, 200, 64, p, p, p, p, p, None, None, None, None, p, None, p, 1 << 30, None),
     "D=200"),
    (lambda L, p: L.sgsa_chunk_fwd(0, 1, 8, 1, 64, 64, p, p, p, p, p, p, None, None, None, p, None, p, 1 << 30, None),
     "together"),
    (lambda L, p: L.sgsa_chunk_fwd(0, 1, 8, 1, 64, 64, p, p, p, p, p, None, None, None, None, p, None, p, 16, None),
     "workspace"),
    (lambda L, p: L.sgsa_chunk_fwd(0, 1, 0, 1, 64, 64, p, p, p, p, p, None, None, None, None, p, None, p, 1 << 30, None),
     "positive"),
    (lambda L, p: L.sgsa_score_topk(1, 1, 16, 16, 2, 64, 32, 1, 0, 8.0, 0, p, p, p, p, None, None, None, 0, p, 1 << 30, None),
     "exceeds"),
    (lambda L, p: L.sgsa_score_topk(1, 1, 16, 16, 2, 64, 4, 1, 0, 8.0, 2, p, p, p, p, None, None, None, 0, p, 1 << 30, None),
     "scale_mode"),
    (lambda L, p: L.sgsa_score_topk(1, 1, 16, 16, 2, 64, 4, 1, 0, 8.0, 0, p, None, p, p, None, None, None, 0, p, 1 << 30, None),
     "k must not be NULL"),
    (lambda L, p: L.sgsa_score_topk(1, 1, 16, 16, 2, 64, 4, 1, 0, 8.0, 0, p, p, p, p, None, None, None, 1, p, 1 << 30,
                                    None),
     "counts"),
    (lambda L, p: L.sgsa_score_topk(1, 1, 16, 16, 2, 64, 4, 1, 0, 8.0, 0, p, p, p, p, None, p, None, 0, p, 64, None),
     "workspace"),
    (lambda L, p: L.sgsa_score_dump(1, 1, 16, 16, 2, 64, 1, 0, 8.0, 0, p, p, 10, 10, p, None),
     "row range"),
    (lambda L, p: L.sgsa_sparse_gather(1, 1, 16, 16, 2, 64, 4, 0, p, p, None, p, p, p, p, None, 0, 0.25, 0.1, 64, 8,
                                       p, p, None, None, None, p, p, 256, None),
     "self_key"),
    (lambda L, p: L.sgsa_sparse_gather(1, 1, 16, 16, 2, 64, 4, 0, p, p, p, p, p, p, p, p, 1, 0.25, 0.1, 64, 8,
                                       p, p, None, p, None, None, None, 0, None),
     "write_key"),
    (lambda L, p: L.sgsa_layer_fwd(1, 1, 16, 2, 64, 4, 64, p, p, p, p, p, p, p, None, 3, 0.25, 0.1, p, None, p,
                                   1 << 30, None),
     "write_mode"),
    (lambda L, p: L.sgsa_recurrent_fwd(1, 1, 16, 2, 64, p, p, p, p, p, p, None, p, None, p, None, None),
     "together"),
    (lambda L, p: L.sgsa_recurrent_fwd(0, 1, 16, 2, 160, p, p, p, p, p, None, None, None, None, p, None, None),
     "D=160"),
    (lambda L, p: L.sgsa_sparse_gather_lists(1, 16, 2, 64, 4, p, p, p, p, p, p, None, 0, 0.25, 0.1, p, p, None, None,
                                             None),
     "D == 128"),
    (lambda L, p: L.sgsa_score_topk_lists(1, 16, 2, 64, 4, p, p, p, p, p, p, p, 16, None),
     "workspace"),
    (lambda L, p: L.sgsa_linear_rows_tile(1, 64, 48, p, p, None), "K=48"),
    (lambda L, p: L.sgsa_linear_rows_tile(0, 64, 64, p, p, None), "bf16"),
    (lambda L, p: L.sgsa_linear_rows_tile(1, 64, 64, ctypes.c_void_p(0x1008), p, None), "16-byte"),
    (lambda L, p: L.sgsa_linear_rows_tiled(1, 17, 64, 64, p, 64, p, None, p, 64, None), "M=17"),
    (lambda L, p: L.sgsa_linear_rows_tiled(1, 8, 64, 64, p, 60, p, None, p, 64, None), "x_row_stride"),
    (lambda L, p: L.sgsa_linear_rows_tiled(1, 8, 64, 64, p, 64, None, None, p, 64, None), "tiled must not be NULL"),
])
def test_argument_validation(call, needle):
    abi, L = _lib()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    st = call(L, fake)
    assert st != 0
    msg = L.sgsa_last_error().decode()
    assert needle in msg, msg


def test_python_wrappers_reject_cpu_tensors():
    import sgsa_amd
    x = torch.zeros(1, 8, 1, 64)
    g = torch.zeros(1, 8, 1)
    with pytest.raises(ValueError, match="ROCm GPU"):
        sgsa_amd.chunk_sgsa(x, x, x, g, g)
    with pytest.raises(ValueError, match="ROCm GPU"):
        sgsa_amd.score_topk(x, x, 4)
    with pytest.raises(ValueError, match="ROCm GPU"):
        sgsa_amd.sgsa_layer_forward(x, x, x, x, g, g, g, 4)


def test_dtype_code_rejects_fp16():
    from sgsa_amd import _abi
    with pytest.raises(ValueError, match="float16"):
        _abi.dtype_code(torch.float16)


def test_product_package_does_not_import_oracle():
    pkg = os.path.join(ROOT, "sgsa_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracle/", ""), f"{f} mentions the oracle"
