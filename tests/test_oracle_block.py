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


def _qkv(B=2, T=40, H=2, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, T, H, D, generator=g, dtype=torch.float64) for _ in range(3))


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
