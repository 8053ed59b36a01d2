"""GPU: block retrieval modes (sgsa_block_retrieve through sgsa_amd.block_retrieve)
against the oracle's restatement of the reference's torch path
(oracle.block_retrieval; modelings/modeling_sgsa.py:167-195, :302-359, :444-463).

The oracle runs in float32 on the same (bf16-rounded) inputs, so -FLT_MAX
paddings and the margins they produce compare exactly.  Selections (block
indices, token indices, including the invalid slots' lowest-index keys) are
compared exactly; values within 2e-5 (fp32) or 2e-2 relative (bf16 outputs).
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)


def _qkv(B, T, H, D, dt, seed, dup=False):
    g = torch.Generator().manual_seed(seed)
    x = [torch.randn(B, T, H, D, generator=g) for _ in range(3)]
    if dup:   # every key equal: all scores of a row tie
        x[1] = x[1][:, :1].expand(B, T, H, D).contiguous()
    return [t.to(dt).float() for t in x]


def _check(dev, B, T, H, D, dt, top_k, bs, tb, mode, causal=True, seed=0, dup=False, am=None):
    q, k, v = _qkv(B, T, H, D, dt, seed, dup)
    ref = O.block_retrieval(q, k, v, top_k, bs, tb, mode=mode, causal=causal, attention_mask=am)
    got = sgsa_amd.block_retrieve(q.to(dev, dt), k.to(dev, dt), v.to(dev, dt), top_k, bs, tb, mode=mode,
                                  causal=causal, return_block_scores=True,
                                  attention_mask=None if am is None else am.to(dev))
    torch.cuda.synchronize()
    tol = dict(atol=2e-5, rtol=2e-5) if dt == torch.float32 else dict(atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(got["block_scores"].cpu(), ref["block_scores"], atol=1e-5, rtol=1e-5)
    assert torch.equal(got["block_indices"].cpu(), ref["block_indices"]), "block indices"
    if mode == "block_token":
        assert torch.equal(got["indices"].cpu(), ref["indices"]), "token indices"
    else:
        assert got["indices"] is None
    torch.testing.assert_close(got["weights"].float().cpu(), ref["weights"].float(), **tol)
    for name in ("k_hat", "v_hat"):
        torch.testing.assert_close(got[name].float().cpu(), ref[name].float(), **tol, msg=name)
    assert set(got["diagnostics"]) == set(ref["diagnostics"])
    for name, val in ref["diagnostics"].items():
        g = got["diagnostics"][name].cpu()
        if name == "score_margin":
            torch.testing.assert_close(g, val, atol=1e-4, rtol=1e-5, msg=name)
        else:
            torch.testing.assert_close(g, val, atol=2e-4 if dt == torch.float32 else 2e-2, rtol=1e-3, msg=name)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["block_token", "block_only"])
@pytest.mark.parametrize("T,bs,tb,top_k", [(150, 32, 2, 16), (97, 7, 3, 12), (64, 64, 2, 8), (40, 1, 5, 6),
                                           (33, 32, 4, 48), (300, 16, 3, 20), (260, 48, 2, 30)])
def test_block_modes_match_oracle(dev, dt, mode, T, bs, tb, top_k):
    _check(dev, 2, T, 3, 64, dt, top_k, bs, tb, mode, seed=T + bs)


@pytest.mark.parametrize("mode", ["block_token", "block_only"])
def test_block_modes_head_dim_128_and_odd(dev, mode):
    _check(dev, 1, 130, 2, 128, torch.bfloat16, 16, 32, 2, mode, seed=5)
    _check(dev, 1, 70, 2, 36, torch.float32, 16, 16, 2, mode, seed=6)


@pytest.mark.parametrize("mode", ["block_token", "block_only"])
def test_block_modes_non_causal(dev, mode):
    _check(dev, 1, 90, 2, 32, torch.float32, 10, 16, 2, mode, causal=False, seed=7)
    for bs in (16, 32, 64):   # the bf16 MFMA sweeps: wave-owned blocks (16, 32) and the LDS-tile form (64)
        _check(dev, 1, 290, 2, 64, torch.bfloat16, 12, bs, 2, mode, causal=False, seed=8 + bs)


@pytest.mark.parametrize("mode", ["block_token", "block_only"])
def test_block_modes_ties_take_lowest_index(dev, mode):
    _check(dev, 1, 80, 2, 16, torch.float32, 8, 8, 3, mode, seed=8, dup=True)


def test_block_token_unit_blocks_equal_token_retrieval(dev):
    # one key per block and every block kept: the token-only retrieval of the same inputs
    q, k, v = _qkv(2, 60, 2, 64, torch.bfloat16, 9)
    args = [t.to(dev, torch.bfloat16) for t in (q, k, v)]
    blk = sgsa_amd.block_retrieve(*args, 8, 1, 60, mode="block_token")
    tok = sgsa_amd.sparse_retrieve(*args, 8)
    torch.cuda.synchronize()
    assert torch.equal(blk["indices"], tok["indices"])
    for name in ("weights", "k_hat", "v_hat"):
        torch.testing.assert_close(blk[name].float(), tok[name].float(), atol=2e-2, rtol=2e-2, msg=name)


def test_block_only_all_blocks_is_causal_attention(dev):
    q, k, v = _qkv(1, 200, 2, 64, torch.float32, 10)
    got = sgsa_amd.block_retrieve(*(t.to(dev) for t in (q, k, v)), 4, 16, 100, mode="block_only")
    want = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                                            is_causal=True)
    torch.testing.assert_close(got["v_hat"].cpu(), want.transpose(1, 2), atol=2e-5, rtol=2e-5)


def test_retriever_modes(dev):
    class Cfg:
        top_k, block_size, top_blocks, tau_c, local_window, sink_size = 8, 16, 2, 0.1, 64, 8
        retrieval_mode = "block_token"
    q, k, v = _qkv(1, 50, 2, 32, torch.float32, 11)
    out = sgsa_amd.SparseRetriever(Cfg()).forward(*(t.to(dev) for t in (q, k, v)))
    ref = O.block_retrieval(q, k, v, 8, 16, 2)
    assert set(out) == {"indices", "block_indices", "weights", "k_hat", "v_hat", "diagnostics"}
    assert torch.equal(out["indices"].cpu(), ref["indices"])
    Cfg.retrieval_mode = "nope"
    with pytest.raises(ValueError):
        sgsa_amd.SparseRetriever(Cfg())


def test_block_retrieve_rejects_too_many_candidates(dev):
    q = torch.zeros(1, 4096, 1, 16, device=dev)
    with pytest.raises(ValueError, match="candidate keys"):
        sgsa_amd.block_retrieve(q, q, q, 8, 1024, 4, mode="block_only")


def _pad(B, T):
    """Batch 0 all real, batch 1 left-padded with a hole, batch 2 right-padded
    with every 5th token a pad (padded query rows and rows whose k_q exceeds
    their own valid count are both present)."""
    am = torch.ones(B, T, dtype=torch.bool)
    am[1, :min(19, T - 1)] = False
    am[1, T // 2:T // 2 + 3] = False
    if B > 2:
        am[2, T - T // 4:] = False
        am[2, ::5] = False
    return am


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["block_token", "block_only"])
@pytest.mark.parametrize("T,bs,tb,top_k", [(150, 32, 2, 16), (97, 7, 3, 12), (130, 16, 4, 24), (260, 48, 2, 30),
                                           (40, 1, 5, 6), (64, 64, 2, 8)])
def test_block_modes_with_padding_mask_match_oracle(dev, dt, mode, T, bs, tb, top_k):
    """sgsa_block_retrieve_masked against the oracle with the reference's valid
    mask (causal & real key & real query, modeling_sgsa.py:421-428): block scores,
    block and token selections (fills included) exactly, values within tolerance.
    bs 16 / 32 run the register sweep, 48 / 64 the LDS-tiled MFMA sweep, 7 and 1
    the key-by-key reduction (fp32: the fma sweep)."""
    print(f"masked block {mode} {dt} T={T} bs={bs} tb={tb} k={top_k}", flush=True)
    _check(dev, 3, T, 2, 64, dt, top_k, bs, tb, mode, seed=T + bs + 1, am=_pad(3, T))


@pytest.mark.parametrize("mode", ["block_token", "block_only"])
def test_block_modes_with_padding_mask_non_causal_and_d128(dev, mode):
    _check(dev, 3, 120, 2, 128, torch.bfloat16, 10, 16, 3, mode, causal=False, seed=5, am=_pad(3, 120))
    _check(dev, 3, 99, 1, 128, torch.bfloat16, 10, 32, 2, mode, causal=True, seed=6, am=_pad(3, 99))


def test_block_modes_all_real_mask_equals_unmasked(dev):
    q, k, v = (t.to(dev, torch.bfloat16) for t in _qkv(2, 200, 2, 64, torch.bfloat16, 9))
    am = torch.ones(2, 200, dtype=torch.bool, device=dev)
    for mode in ("block_token", "block_only"):
        a = sgsa_amd.block_retrieve(q, k, v, 12, 32, 3, mode=mode)
        b = sgsa_amd.block_retrieve(q, k, v, 12, 32, 3, mode=mode, attention_mask=am)
        torch.cuda.synchronize()
        for name in ("block_indices", "k_hat", "v_hat", "weights"):
            assert torch.equal(a[name], b[name]), (mode, name)
