"""GPU: the config-4 hybrid decoder (sgsa_amd.hybrid) -- dense GQA attention every
4th layer, SGSA blocks between them on the HIP kernels, prefill then decode with
the SGSA layers' top-k recomputed every 4 steps and re-scored in between.

* fp32: prompt logits and 9 teacher-forced decode steps against the oracle's
  hybrid decoder (oracle.hybrid_generate) fed the same parameters and the same
  recompute schedule; relative to the largest logit, 1e-3 (five layers, each
  within the layer's 1e-4).
* bf16 greedy generation: a prompt prefilled at B = 1 and decoded for B = 3
  sequences gives finite logits, the same tokens in every sequence and the same
  tokens on a second run.
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)


def _model(dev, dtype, seed=0, top_k=32, heads=2):
    from sgsa_amd.hybrid import HybridConfig, HybridForCausalLM
    cfg = HybridConfig(vocab_size=512, hidden_size=128 * heads, intermediate_size=512, num_hidden_layers=5,
                       num_attention_heads=heads, num_kv_heads=heads // 2, top_k=top_k, topk_recompute_every=4)
    m = HybridForCausalLM(cfg)
    m.init_weights(0.02, qk_std=(cfg.hidden_size * cfg.head_dim) ** -0.5, generator=torch.Generator().manual_seed(seed))
    return cfg, m.to(dev, dtype).eval()


def _rel(got, ref, name):
    got, ref = got.float().cpu(), ref.float().cpu()
    assert torch.isfinite(got).all(), f"{name}: non-finite"
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-3, f"{name}: {err:.3e} from the oracle"


def test_hybrid_fp32_matches_the_oracle(dev):
    from sgsa_amd.hybrid import rope_tables
    cfg, m = _model(dev, torch.float32)
    g = torch.Generator().manual_seed(1)
    B, T, n = 2, 180, 9
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    dec = torch.randint(0, cfg.vocab_size, (B, n), generator=g)
    params = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    ref_p, ref_d = O.hybrid_generate(params, prompt, dec, num_layers=cfg.num_hidden_layers,
                                     num_heads=cfg.num_attention_heads, num_kv_heads=cfg.num_kv_heads,
                                     dense_every=cfg.dense_every, top_k=cfg.top_k,
                                     recompute_every=cfg.topk_recompute_every)
    rope = rope_tables(T + n, cfg.head_dim, cfg.rope_theta, dev)
    caches = m.new_cache(B, T + n, dev, torch.float32)
    logits = m.prefill(prompt.to(dev), caches, rope)
    _rel(logits, ref_p, "prompt logits")
    for s in range(n):
        out = m.decode_step(dec[:, s].to(dev), T + s, s, caches, rope)
        _rel(out, ref_d[:, s], f"decode step {s} ({'select' if s % 4 == 0 else 'reuse'})")


def test_hybrid_bf16_greedy_generation(dev):
    from sgsa_amd.hybrid import generate
    cfg, m = _model(dev, torch.bfloat16, seed=2)
    prompt = torch.randint(0, cfg.vocab_size, (1, 200), generator=torch.Generator().manual_seed(3)).to(dev)
    logits, toks = generate(m, prompt, steps=6, batch=3)
    logits2, toks2 = generate(m, prompt, steps=6, batch=3)
    torch.cuda.synchronize()
    assert torch.isfinite(logits.float()).all()
    assert toks.shape == (3, 6) and (toks == toks[0:1]).all(), "sequences with one prompt diverged"
    assert torch.equal(toks, toks2) and torch.equal(logits, logits2), "not deterministic"


@pytest.mark.parametrize("top_k,T,B,heads", [(32, 160, 3, 2), (320, 600, 3, 2), (320, 600, 16, 16)])
def test_decode_stack_equals_the_per_layer_path(dev, top_k, T, B, heads):
    # sgsa_decode_stack (one call per step) against the per-layer Python path on copies of
    # the same prefilled caches: logits equal bit for bit on selecting and re-scoring steps,
    # and so are the SGSA states and caches after the last step.  top_k 320 takes the
    # split-row gather (3 partials per row, the last one short), where the stack re-scores
    # the kept candidates inside the gather and merges the rows in the state update's
    # launch, and the per-layer path scores them first; at B * heads = 256 the state
    # update runs one workgroup per head (all columns) instead of four
    import sgsa_amd.hybrid as HY
    cfg, m = _model(dev, torch.bfloat16, seed=6, top_k=top_k, heads=heads)
    g = torch.Generator().manual_seed(7)
    n = 9
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=g).to(dev)
    toks = torch.randint(0, cfg.vocab_size, (B, n), generator=g).to(dev)
    rope = HY.rope_tables(T + n, cfg.head_dim, cfg.rope_theta, dev)
    with torch.no_grad():
        caches = m.new_cache(B, T + n, dev, torch.bfloat16)
        m.prefill(prompt, caches, rope)
        copy = [{k: (v.clone() if torch.is_tensor(v) else v) for k, v in c.items()} for c in caches]
        m.decode_stack = False
        ref = [m.decode_step(toks[:, s], T + s, s, caches, rope) for s in range(n)]
        assert m.__dict__.get("_decode_plan") is None
        m.decode_stack = True
        got = [m.decode_step(toks[:, s], T + s, s, copy, rope) for s in range(n)]
        assert m.__dict__.get("_decode_plan") is not None, "sgsa_decode_stack was not used"
    torch.cuda.synchronize()
    for s in range(n):
        assert torch.equal(got[s], ref[s]), f"step {s} ({'select' if s % 4 == 0 else 'reuse'}): logits differ"
    for i, (a, b) in enumerate(zip(copy, caches)):
        for name in ("k", "v", "state"):
            if name in a:
                assert torch.equal(a[name], b[name]), f"layer {i}: {name} differs"


def test_hybrid_bf16_prompt_logits_near_the_oracle(dev):
    # bf16 activations (dense scores scaled in bf16 as hybrid_dense_delta_topk.py:186-187
    # does) against the fp32 oracle on the same bf16 parameters: prompt and three
    # decode steps, relative to the largest logit.  Five stacked layers, each within
    # the layer's bf16 2e-2, and the bf16 rounding of every stored activation.
    from sgsa_amd.hybrid import rope_tables
    from tolerance import close
    cfg, m = _model(dev, torch.bfloat16, seed=4)
    g = torch.Generator().manual_seed(5)
    B, T, n = 2, 150, 3
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    dec = torch.randint(0, cfg.vocab_size, (B, n), generator=g)
    params = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    ref_p, ref_d = O.hybrid_generate(params, prompt, dec, num_layers=cfg.num_hidden_layers,
                                     num_heads=cfg.num_attention_heads, num_kv_heads=cfg.num_kv_heads,
                                     dense_every=cfg.dense_every, top_k=cfg.top_k,
                                     recompute_every=cfg.topk_recompute_every)
    rope = rope_tables(T + n, cfg.head_dim, cfg.rope_theta, dev)
    caches = m.new_cache(B, T + n, dev, torch.bfloat16)
    close(m.prefill(prompt.to(dev), caches, rope), ref_p, 2e-2, "bf16 prompt logits")
    for s in range(n):
        out = m.decode_step(dec[:, s].to(dev), T + s, s, caches, rope)
        close(out, ref_d[:, s], 2e-2, f"bf16 decode step {s}")


@pytest.mark.parametrize("dt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("kend", [1, 255, 257, 1000])
def test_decode_attention_equals_torch_form(dev, dt, tol, G, kend):
    # one query row per sequence over a cache view: the HIP pass (sgsa_decode_attention, taken by
    # gqa_attention at Tq = 1) against the torch form with the same rounding points (scores and
    # scaling in dtype, softmax in fp32, probabilities in dtype); relative to max |o|
    from sgsa_amd.hybrid import _decode_attention, _decode_attention_fits, gqa_attention
    import math
    B, Hkv, D, Tmax = 3, 2, 128, 1040
    H = G * Hkv
    g = torch.Generator().manual_seed(kend * 10 + G)
    q = torch.randn(B, H, 1, D, generator=g).to(dt).to(dev)
    kc = torch.randn(B, Hkv, Tmax, D, generator=g).to(dt).to(dev)
    vc = torch.randn(B, Hkv, Tmax, D, generator=g).to(dt).to(dev)
    k, v = kc[:, :, :kend], vc[:, :, :kend]
    with torch.no_grad():
        assert _decode_attention_fits(q, k, v, kend - 1)
        got = _decode_attention(q, k, v)
        via = gqa_attention(q, k, v, kend - 1)
    qg = q.reshape(B, Hkv, G, D)
    s = (torch.matmul(qg, k.transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(D))).float()   # [B,Hkv,G,kend]
    p = torch.softmax(s, dim=-1).to(dt)
    want = torch.matmul(p, v.contiguous()).reshape(B, H, 1, D)
    torch.cuda.synchronize()
    assert torch.equal(got, via)
    err = ((got.float() - want.float()).abs().max() / want.float().abs().max()).item()
    assert err <= tol, f"{err:.3e}"


@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("Tq,pos0", [(64, 0), (200, 0), (130, 57), (1000, 300)])
def test_dense_attention_equals_torch_form(dev, G, Tq, pos0):
    # a block of query rows at positions pos0 .. over a cache view: the two HIP passes
    # (sgsa_dense_attention, taken by gqa_attention in bf16) against the torch form with the same
    # rounding points (bf16 scores and scaling, fp32 softmax, bf16 probabilities); relative to max |o|
    from sgsa_amd.hybrid import _dense_attention, _dense_attention_fits, gqa_attention
    import math
    B, Hkv, D, L = 2, 2, 128, 1400
    H = G * Hkv
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(Tq + pos0 + G)
    q = torch.randn(B, H, Tq, D, generator=g).to(dt).to(dev)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(dt).to(dev)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(dt).to(dev)
    kend = pos0 + Tq
    k, v = kc[:, :, :kend], vc[:, :, :kend]
    with torch.no_grad():
        assert _dense_attention_fits(q, k, v, pos0)
        got = _dense_attention(q, k, v, pos0)
        via = gqa_attention(q, k, v, pos0)
    qg = q.reshape(B, Hkv, G * Tq, D)
    s = (torch.matmul(qg, k.transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(D))).float()   # [B,Hkv,G*Tq,kend]
    qpos = (pos0 + torch.arange(Tq, device=dev)).repeat(G)
    s = s.masked_fill(torch.arange(kend, device=dev)[None, :] > qpos[:, None], float("-inf"))
    p = torch.softmax(s, dim=-1).to(dt)
    want = torch.matmul(p, v.contiguous()).reshape(B, H, Tq, D)
    torch.cuda.synchronize()
    assert torch.equal(got, via)
    err = ((got.float() - want.float()).abs().max() / want.float().abs().max()).item()
    assert err <= 1e-2, f"{err:.3e}"
