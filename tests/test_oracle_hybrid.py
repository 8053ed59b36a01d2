"""CPU checks of the oracle's config-4 hybrid decoder (oracle.hybrid_generate).

* dense_gqa_attention equals torch's scaled_dot_product_attention (causal, the
  key/value heads repeated for their query groups);
* rope_apply is multiplication by exp(i pos / theta^(2j/D)) of the complex pairs
  (x_j, x_{j+D/2}) -- the rotate-half form of
  modelings/hybrid_dense_delta_topk.py:140-150;
* decoding token by token with the top-k selected at every step reproduces one
  full pass over prompt + decoded tokens (dense KV caching, positions, SGSA
  decode steps against the full-sequence layer).
"""

import torch
import torch.nn.functional as F

from oracle import sgsa_oracle as O


def test_dense_gqa_attention_is_sdpa():
    g = torch.Generator().manual_seed(0)
    B, H, Hkv, T, D = 2, 6, 2, 37, 16
    q = torch.randn(B, H, T, D, generator=g)
    k = torch.randn(B, Hkv, T, D, generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g)
    got = O.dense_gqa_attention(q, k, v, torch.arange(T))
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1), is_causal=True)
    torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-5)
    # the last 5 queries alone (positions T-5 ..) against all keys
    got5 = O.dense_gqa_attention(q[:, :, -5:], k, v, torch.arange(T - 5, T))
    torch.testing.assert_close(got5, ref[:, :, -5:], atol=1e-5, rtol=1e-5)


def test_rope_is_a_complex_rotation():
    g = torch.Generator().manual_seed(1)
    B, H, T, D, theta = 1, 3, 11, 16, 10000.0
    x = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    pos = torch.arange(5, 5 + T)
    got = O.rope_apply(x.float(), pos, theta).double()
    ang = pos.double()[:, None] * (1.0 / theta ** (torch.arange(0, D, 2).double() / D))[None, :]
    z = torch.complex(x[..., :D // 2], x[..., D // 2:]) * torch.polar(torch.ones_like(ang), ang)
    ref = torch.cat((z.real, z.imag), dim=-1)
    torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-5)


def test_decode_steps_reproduce_the_full_pass():
    from sgsa_amd.hybrid import HybridConfig, HybridForCausalLM
    cfg = HybridConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=5,
                       num_attention_heads=2, num_kv_heads=1, top_k=16)
    m = HybridForCausalLM(cfg)
    g = torch.Generator().manual_seed(0)
    m.init_weights(0.02, qk_std=(cfg.hidden_size * cfg.head_dim) ** -0.5, generator=g)
    params = {k: v.detach().float() for k, v in m.state_dict().items()}
    B, T, n = 2, 60, 6
    prompt = torch.randint(0, 256, (B, T), generator=g)
    dec = torch.randint(0, 256, (B, n), generator=g)
    kw = dict(num_layers=5, num_heads=2, num_kv_heads=1, dense_every=4, top_k=16, recompute_every=1)
    pl, dl = O.hybrid_generate(params, prompt, dec, **kw)
    full, _ = O.hybrid_generate(params, torch.cat([prompt, dec], 1), dec[:, :0], **kw)
    torch.testing.assert_close(pl, full[:, :T], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dl, full[:, T:T + n], atol=1e-5, rtol=1e-5)


def test_activation_rounding_is_identity_in_fp32_and_small_in_bf16():
    # act_dtype=float32 rounds nothing: the unrounded decoder exactly; bfloat16 stays within a few
    # bf16 ulps of it on this 5-layer model
    from sgsa_amd.hybrid import HybridConfig, HybridForCausalLM
    cfg = HybridConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=5,
                       num_attention_heads=2, num_kv_heads=1, top_k=16)
    m = HybridForCausalLM(cfg)
    g = torch.Generator().manual_seed(2)
    m.init_weights(0.02, qk_std=(cfg.hidden_size * cfg.head_dim) ** -0.5, generator=g)
    params = {k: v.detach().float() for k, v in m.state_dict().items()}
    prompt = torch.randint(0, 256, (1, 40), generator=g)
    dec = torch.randint(0, 256, (1, 3), generator=g)
    kw = dict(num_layers=5, num_heads=2, num_kv_heads=1, dense_every=4, top_k=16, recompute_every=2)
    pl, dl = O.hybrid_generate(params, prompt, dec, **kw)
    p32, d32 = O.hybrid_generate(params, prompt, dec, act_dtype=torch.float32, **kw)
    assert torch.equal(pl, p32) and torch.equal(dl, d32)
    p16, d16 = O.hybrid_generate(params, prompt, dec, act_dtype=torch.bfloat16, **kw)
    assert ((p16 - pl).abs().max() / pl.abs().max()).item() < 3e-2
    assert not torch.equal(p16, pl)
