"""CPU checks of the oracle's block retrieval modes (oracle.block_retrieval).

* block_token with one key per block and every block kept is token top-k
  retrieval (token_topk_retrieval, pinned elsewhere): same selection, weights,
  k_hat / v_hat and diagnostics;
* block_only with every block kept weights every causal key by softmax: k_hat /
  v_hat equal torch's causal scaled_dot_product_attention;
* block scores equal a loop over rows and blocks taking the max causal score.
"""

import math

import torch
import torch.nn.functional as F

from oracle import sgsa_oracle as O


def _qkv(B=2, T=40, H=2, D=8, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, T, H, D, generator=g, dtype=torch.float64).to(dtype) for _ in range(3))


def test_block_token_with_unit_blocks_is_token_topk():
    q, k, v = _qkv()
    T = q.shape[1]
    got = O.block_retrieval(q, k, v, top_k=6, block_size=1, top_blocks=T, mode="block_token")
    ref = O.token_topk_retrieval(q, k, v, 6)
    assert torch.equal(got["indices"], ref["indices"])
    for name in ("weights", "scores"):
        torch.testing.assert_close(got[name], ref[name])
    for name in ("k_hat", "v_hat"):
        torch.testing.assert_close(got[name], ref[name])
    for name, val in ref["diagnostics"].items():
        torch.testing.assert_close(got["diagnostics"][name], val, msg=name)


def test_block_only_with_every_block_is_causal_attention():
    q, k, v = _qkv(T=37)
    got = O.block_retrieval(q, k, v, top_k=4, block_size=5, top_blocks=100, mode="block_only")
    qh, kh, vh = (x.transpose(1, 2) for x in (q, k, v))
    torch.testing.assert_close(got["v_hat"], F.scaled_dot_product_attention(qh, kh, vh, is_causal=True).transpose(1, 2))
    torch.testing.assert_close(got["k_hat"], F.scaled_dot_product_attention(qh, kh, kh, is_causal=True).transpose(1, 2))
    assert "avg_distance" not in got["diagnostics"] and got["indices"] is None


def test_block_scores_are_the_causal_block_maxima():
    q, k, v = _qkv(B=1, T=23, H=1, D=4, seed=3)
    bs = 4
    got = O.block_retrieval(q, k, v, top_k=3, block_size=bs, top_blocks=2)["block_scores"]
    fmin = torch.finfo(torch.float64).min
    for t in range(23):
        for b in range(got.shape[-1]):
            keys = [j for j in range(b * bs, min((b + 1) * bs, 23)) if j <= t]
            want = max((float(q[0, t, 0] @ k[0, j, 0]) / math.sqrt(4) for j in keys), default=fmin)
            assert abs(float(got[0, 0, t, b]) - want) <= 1e-12 * max(1.0, abs(want)), (t, b)


# The masked checks run in float32: the reference's softmax(scores.float()) turns
# float64's finfo.min fills into -inf, and a padded row of them into NaN.
def _pad_mask(B, T):
    am = torch.ones(B, T, dtype=torch.bool)
    am[1, :7] = False          # left padding
    am[1, T - 3:] = False      # and right padding
    am[1, 15:19] = False       # and a hole
    return am


def test_masked_block_token_with_unit_blocks_is_masked_token_topk():
    q, k, v = _qkv(dtype=torch.float32)
    T = q.shape[1]
    am = _pad_mask(2, T)
    got = O.block_retrieval(q, k, v, top_k=6, block_size=1, top_blocks=T, mode="block_token", attention_mask=am)
    ref = O.token_topk_retrieval(q, k, v, 6, attention_mask=am)
    assert torch.equal(got["indices"], ref["indices"])
    for name in ("weights", "scores", "k_hat", "v_hat"):
        torch.testing.assert_close(got[name], ref[name], msg=name)
    for name, val in ref["diagnostics"].items():
        torch.testing.assert_close(got["diagnostics"][name], val, msg=name)


def test_masked_block_only_with_every_block_is_masked_causal_attention():
    q, k, v = _qkv(T=37, dtype=torch.float32)
    T = q.shape[1]
    am = _pad_mask(2, T)
    got = O.block_retrieval(q, k, v, top_k=4, block_size=5, top_blocks=100, mode="block_only", attention_mask=am)
    qh, kh, vh = (x.transpose(1, 2) for x in (q, k, v))
    pos = torch.arange(T)
    allowed = (pos[None, :] <= pos[:, None])[None, None] & am[:, None, None, :] & am[:, None, :, None]
    s = (qh @ kh.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    p = torch.softmax(s.masked_fill(~allowed, float("-inf")), dim=-1).nan_to_num(0.0)   # padded rows: all -inf
    torch.testing.assert_close(got["v_hat"], (p @ vh).transpose(1, 2))
    torch.testing.assert_close(got["k_hat"], (p @ kh).transpose(1, 2))
    assert got["v_hat"][~am].abs().max() == 0


def test_masked_block_scores_are_the_masked_block_maxima():
    q, k, v = _qkv(B=2, T=23, H=1, D=4, seed=3, dtype=torch.float32)
    bs = 4
    am = _pad_mask(2, 23)
    got = O.block_retrieval(q, k, v, top_k=3, block_size=bs, top_blocks=2, attention_mask=am)["block_scores"]
    fmin = torch.finfo(torch.float32).min
    for b in range(2):
        for t in range(23):
            for blk in range(got.shape[-1]):
                keys = [j for j in range(blk * bs, min((blk + 1) * bs, 23)) if j <= t and am[b, j] and am[b, t]]
                want = max((float(q[b, t, 0].double() @ k[b, j, 0].double()) / math.sqrt(4) for j in keys),
                           default=fmin)
                assert abs(float(got[b, 0, t, blk]) - want) <= 1e-6 * max(1.0, abs(want)), (b, t, blk)


def test_all_real_mask_equals_no_mask():
    q, k, v = _qkv(T=29)
    am = torch.ones(2, 29, dtype=torch.bool)
    for mode in ("block_token", "block_only"):
        a = O.block_retrieval(q, k, v, top_k=5, block_size=4, top_blocks=3, mode=mode)
        b = O.block_retrieval(q, k, v, top_k=5, block_size=4, top_blocks=3, mode=mode, attention_mask=am)
        for name in ("block_indices", "k_hat", "v_hat", "weights"):
            assert torch.equal(a[name], b[name]), (mode, name)
