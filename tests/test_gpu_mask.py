"""GPU parity of the padding-mask paths: SparseRetriever's attention_mask
(modelings/modeling_sgsa.py:421-428, :144-165) and TopKSparseKVReuseAttention's
merged mask (modelings/hybrid_dense_delta_topk.py:153-175, :343-356).

* Selection, bit for bit: sgsa_score_topk_masked against the oracle's
  masked_topk applied to the exact fp32 scores sgsa_score_dump returns, with
  the reference's valid mask built from the padding mask -- indices, scores,
  valid flags, counts and each row's k_q.
* Values: k_hat / v_hat / weights / diagnostics of the masked retrieval, the
  masked layer (write key, v_hat, alpha, output, final state) and the KV-reuse
  attention against the oracle within the stated tolerances; the KV-reuse
  module's gradients under autograd against autograd through the oracle.
* The threshold form under a mask (bf16, d = 128: the layer's keys compacted
  valid-first, per-row valid prefix and slot count in score_thr128_kernel, its
  radix fallback and gather_thr_kernel) against the oracle layer, bit-equal to
  the unmasked form under an all-ones mask, and on mass ties that send blocks to
  the fallback.

Masks: batch 0 all real tokens, batch 1 left-padded, batch 2 right-padded with
holes; padded query rows and rows with fewer valid keys than k_q are included.
"""

import math

import pytest
import torch

from oracle import sgsa_oracle as O
from tolerance import close

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)

FMIN = torch.finfo(torch.float32).min


def _mask(B, T, seed=0):
    am = torch.ones(B, T, dtype=torch.bool)
    if B > 1:
        am[1, :37 % T] = False
    if B > 2:
        am[2, T - 50:] = False
        am[2, ::7] = False
    return am


def _check_masked(got, dump, valid, kk, kq_rule=0, name=""):
    idx, sc, ok, top2, cnt, fill = (t.cpu() for t in got)
    if kq_rule == 0:
        ovals, oidx, ovalid = O.masked_topk(dump, valid, kk)
        vc = valid.sum(-1).amax(dim=(0, 1))
        kq = torch.clamp(torch.clamp(vc, min=1), max=kk)
    else:   # hybrid: every row keeps kk slots and there is no valid mask
        masked = dump.masked_fill(~valid, FMIN)
        B, H, R, Tk = dump.shape
        ovals, oidx = O.topk_lowest_index(masked.reshape(-1, Tk), kk)
        ovals, oidx = ovals.reshape(B, H, R, kk), oidx.reshape(B, H, R, kk)
        ovalid = valid.gather(-1, oidx)
        kq = torch.full((R,), kk)
    assert torch.equal(cnt, ovalid.sum(-1).int()), f"{name}: valid counts differ"
    assert torch.equal(fill, kq.int().view(1, 1, -1).expand_as(fill)), f"{name}: k_q differs"
    bad = (idx.long() != oidx)
    assert not bad.any(), f"{name}: indices differ in {int(bad.sum())} slots (first at {bad.nonzero()[0].tolist()})"
    assert torch.equal(sc, ovals.float()), f"{name}: scores differ"
    assert torch.equal(ok.bool(), ovalid), f"{name}: valid flags differ"
    assert torch.equal(top2[..., 0], torch.where(ovalid[..., 0], ovals[..., 0], torch.full_like(ovals[..., 0], FMIN)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 300, 2, 64, 32), (3, 257, 3, 128, 100), (2, 130, 1, 64, 200)])
@pytest.mark.parametrize("causal", [True, False])
def test_masked_select_bit_exact_on_dumped_scores(dev, dtype, shape, causal):
    B, T, H, D, k = shape
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, T, H, D, generator=g).to(dev, dtype)
    kk_ = torch.randn(B, T, H, D, generator=g).to(dev, dtype)
    am = _mask(B, T)
    kk = min(k, T)
    print(f"masked select B={B} T={T} H={H} D={D} k={k} {dtype} causal={causal}", flush=True)
    got = sgsa_amd.score_topk_masked(q, kk_, k, key_mask=am.to(dev), query_mask=am.to(dev), causal=causal)
    dump = sgsa_amd.score_dump(q, kk_, 0, T, causal=False)
    torch.cuda.synchronize()
    pos = torch.arange(T)
    valid = torch.ones(T, T, dtype=torch.bool) if not causal else pos[None, :] <= pos[:, None]
    valid = (valid[None, None] & am[:, None, None, :] & am[:, None, :, None]).expand(B, H, T, T)
    _check_masked(got, dump.cpu(), valid, kk, 0, "retriever")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Q,K,k", [(5, 300, 32), (64, 200, 48), (3, 40, 64)])
def test_kv_reuse_select_bit_exact_on_dumped_scores(dev, dtype, Q, K, k):
    B, H, D = 3, 2, 64
    g = torch.Generator().manual_seed(4)
    q = torch.randn(B, Q, H, D, generator=g).to(dev, dtype)
    key = torch.randn(B, H, K, D, generator=g).to(dev, dtype)   # the dense layer's [B,H,K,D]
    am = _mask(B, K)
    am[0, :K - Q + 1] = False     # batch 0: the first query sees only padding
    kk = min(k, K)
    print(f"kv-reuse select B={B} Q={Q} K={K} k={k} {dtype}", flush=True)
    got = sgsa_amd.score_topk_masked(q, key, k, key_mask=am.to(dev), causal=True, q_offset=K - Q, scale_mode=1,
                                     kq_rule=1, kv_layout=1)
    dump = sgsa_amd.score_dump(q, key.transpose(1, 2).contiguous(), 0, Q, causal=False, scale_mode=1,
                               scale=1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    qpos = torch.arange(K - Q, K)
    valid = (torch.arange(K)[None, :] <= qpos[:, None])[None, None] & am[:, None, None, :]
    _check_masked(got, dump.cpu(), valid.expand(B, H, Q, K), kk, 1, "kv-reuse")


def test_masked_select_without_masks_matches_plain_select(dev):
    B, T, H, D, k = 2, 400, 2, 128, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    kk_ = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    idx, sc, ok, top2, cnt, fill = sgsa_amd.score_topk_masked(q, kk_, k)
    i2, s2, t2, c2 = sgsa_amd.score_topk(q, kk_, k, sorted=True)
    torch.cuda.synchronize()
    assert torch.equal(idx, i2) and torch.equal(sc, s2) and torch.equal(cnt, c2) and torch.equal(top2, t2)
    assert torch.equal(ok.bool().sum(-1).int(), cnt)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_masked_retrieval_matches_oracle(dev, dtype, tol):
    B, T, H, D, k = 3, 384, 2, 64, 32
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=1)
    am = _mask(B, T)
    ret = O.token_topk_retrieval(x["q_f32"], x["k_f32"], x["v_f32"], k, attention_mask=am)
    got = sgsa_amd.sparse_retrieve(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), k, attention_mask=am.to(dev))
    torch.cuda.synchronize()
    gi = got["indices"].cpu()
    mism = (gi != ret["indices"]).any(-1).float().mean().item()
    assert mism < 0.01, f"{mism:.3%} of rows select a different key set"
    close(got["k_hat"], ret["k_hat"], tol, "k_hat")
    close(got["v_hat"], ret["v_hat"], tol, "v_hat")
    close(got["weights"], ret["weights"], tol, "weights")
    # padded query rows retrieve nothing
    pad = ~am
    assert got["k_hat"].cpu()[pad].abs().max() == 0 and got["v_hat"].cpu()[pad].abs().max() == 0
    for name in ("concentration", "max_confidence", "novelty", "write_conflict", "entropy",
                 "avg_distance", "local_ratio", "sink_ratio", "remote_ratio"):
        close(got["diagnostics"][name], ret["diagnostics"][name], max(tol, 1e-4), name)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_masked_layer_matches_oracle(dev, dtype, tol):
    B, T, H, D, k = 3, 320, 2, 64, 32
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=2)
    am = _mask(B, T)
    ref = O.sgsa_layer_forward(x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"],
                               x["budget"], k, attention_mask=am)
    g = {n: x[n].to(dev) for n in ("q", "k", "v", "beta", "gamma", "budget")}
    o, st = sgsa_amd.sgsa_layer_forward(g["q"], g["k"], g["v"], g["q"], g["beta"], g["gamma"], g["budget"], k,
                                        attention_mask=am.to(dev))
    wk, vh, al = sgsa_amd.sgsa_layer_retrieve(g["q"], g["k"], g["v"], g["budget"], k, attention_mask=am.to(dev))
    torch.cuda.synchronize()
    close(wk, ref["write_key"], tol, "write key")
    close(vh, ref["v_hat"], tol, "v_hat")
    close(al, ref["alpha"], tol, "alpha")
    close(o, ref["o"], tol, "o")
    close(st, ref["final_state"], tol, "final state")


@pytest.mark.parametrize("shape", [(3, 640, 2, 32), (2, 1500, 2, 300)])
def test_masked_threshold_layer_matches_oracle(dev, shape):
    # bf16, d = 128: the masked layer runs the threshold form (score_thr128_kernel and
    # gather_thr_kernel over keys compacted valid-first, per-row valid prefix and slots)
    B, T, H, k = shape
    D = 128
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=8)
    am = _mask(B, T)
    assert sgsa_amd.layer._masked_threshold_form(x["q"])
    print(f"masked threshold layer B={B} T={T} H={H} D={D} k={k}", flush=True)
    ref = O.sgsa_layer_forward(x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"],
                               x["budget"], k, attention_mask=am)
    g = {n: x[n].to(dev) for n in ("q", "k", "v", "beta", "gamma", "budget")}
    st_ = {}
    o, st = sgsa_amd.sgsa_layer_forward(g["q"], g["k"], g["v"], g["q"], g["beta"], g["gamma"], g["budget"], k,
                                        attention_mask=am.to(dev), stats=st_)
    wk, vh, al = sgsa_amd.sgsa_layer_retrieve(g["q"], g["k"], g["v"], g["budget"], k, attention_mask=am.to(dev))
    torch.cuda.synchronize()
    assert "row_stats" in st_, "the threshold form did not run"
    assert torch.equal(al, st_["alpha"])
    close(wk, ref["write_key"], 2e-2, "write key")
    close(vh, ref["v_hat"], 2e-2, "v_hat")
    close(al, ref["alpha"], 2e-2, "alpha")
    close(o, ref["o"], 2e-2, "o", elem_p99=2e-2)
    close(st, ref["final_state"], 2e-2, "final state", elem_p99=2e-2)
    pad = ~am.to(dev)
    assert vh[pad].abs().max() == 0 and al[pad].abs().max() == 0, "padded query rows retrieve nothing"


def test_masked_threshold_all_ones_mask_equals_unmasked(dev):
    B, T, H, D, k = 2, 1200, 2, 128, 256
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=9)
    g = {n: x[n].to(dev) for n in ("q", "k", "v", "budget")}
    am = torch.ones(B, T, dtype=torch.bool, device=dev)
    for mode in ("direct", "residual"):
        got = sgsa_amd.sgsa_layer_retrieve(g["q"], g["k"], g["v"], g["budget"], k, attention_mask=am,
                                           write_mode=mode)
        want = sgsa_amd.sgsa_layer_retrieve(g["q"], g["k"], g["v"], g["budget"], k, write_mode=mode)
        torch.cuda.synchronize()
        for name, a_, b_ in zip(("write key", "v_hat", "alpha"), got, want):
            assert torch.equal(a_, b_), f"{mode} {name}: an all-ones mask changes the threshold form"


def test_masked_threshold_ties_take_the_fallback(dev):
    # keys drawn from two rows: a row's threshold bin holds every valid key equal to its
    # better row, more than the collect capacity past ~1100 rows, so those blocks take the
    # masked radix fallback; ties resolve to the lowest-index valid keys, as in the oracle
    B, T, H, D, k = 3, 1600, 2, 128, 64
    gen = torch.Generator().manual_seed(10)
    base = torch.randn(2, H, D, generator=gen)
    kr = base[torch.randint(0, 2, (B, T), generator=gen)].to(torch.bfloat16)
    q = torch.randn(B, T, H, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, T, H, D, generator=gen).to(torch.bfloat16)
    bud = torch.randn(B, T, H, generator=gen)
    am = _mask(B, T)
    print(f"masked threshold ties B={B} T={T} H={H} k={k}", flush=True)
    ret = O.token_topk_retrieval(q.float(), kr.float(), v.float(), k, attention_mask=am)
    wk, vh, al = sgsa_amd.sgsa_layer_retrieve(q.to(dev), kr.to(dev), v.to(dev), bud.to(dev), k,
                                              attention_mask=am.to(dev))
    torch.cuda.synchronize()
    close(vh, ret["v_hat"], 2e-2, "v_hat")
    wko = O.write_key(ret["k_hat"], kr.float(), "direct")
    close(wk, wko, 2e-2, "write key")
    alo = O.compute_alpha(ret["diagnostics"]["concentration"], ret["diagnostics"]["novelty"], bud, wko, ret["v_hat"])
    close(al, alo, 2e-2, "alpha")


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_kv_reuse_attention_matches_oracle(dev, dtype, tol):
    B, H, D, Q, K, k = 3, 2, 64, 48, 300, 40
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, Q, H, D, generator=g).to(dtype)
    key = torch.randn(B, H, K, D, generator=g).to(dtype)
    val = torch.randn(B, H, K, D, generator=g).to(dtype)
    am = _mask(B, K)
    am[0, :K - Q + 2] = False   # the first two queries of batch 0 see only padding
    out, oidx, op = O.topk_kv_reuse_attention(q.float().transpose(1, 2), key.float(), val.float(), k, attention_mask=am)
    att, idx, p = sgsa_amd.topk_kv_reuse_attention(q.to(dev), key.to(dev), val.to(dev), k, attention_mask=am.to(dev))
    torch.cuda.synchronize()
    mism = (idx.cpu() != oidx).any(-1).float().mean().item()
    assert mism < 0.01, f"{mism:.3%} of rows select a different key set"
    assert torch.equal(idx.cpu()[0, :, 0], oidx[0, :, 0]), "an all-padding row keeps the lowest-index keys"
    close(p, op, tol, "probabilities")
    close(att, out.transpose(1, 2), tol, "attended")
    torch.testing.assert_close(p.cpu()[0, :, 0], torch.full((H, k), 1.0 / k), rtol=1e-6, atol=1e-7)


def test_kv_reuse_module_matches_reference_formula(dev):
    # the module: q_proj, RoPE at offset K-Q on the reference's [1,1,S,D] tables, core, o_proj
    from types import SimpleNamespace
    C, H, Q, K, k = 128, 2, 6, 90, 16
    D = C // H
    cfg = SimpleNamespace(num_attention_heads=H, head_dim=D, hidden_size=C, top_k=k, dropout=0.0)
    m = sgsa_amd.TopKSparseKVReuseAttention(cfg).to(dev)
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * C ** -0.5)
    hs = torch.randn(2, Q, C, generator=g).to(dev)
    key = torch.randn(2, H, K, D, generator=g).to(dev)
    val = torch.randn(2, H, K, D, generator=g).to(dev)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2).float() / D))
    emb = torch.cat([torch.outer(torch.arange(K).float(), inv)] * 2, dim=-1)
    rope = (emb.cos()[None, None].to(dev), emb.sin()[None, None].to(dev))
    am = torch.ones(2, K, dtype=torch.bool)
    am[1, :20] = False
    with torch.no_grad():
        y = m(hs, (key, val), rope, am.to(dev))
        qh = m.q_proj(hs).view(2, Q, H, D).transpose(1, 2).cpu()
        c, s = rope[0][:, :, K - Q:K].cpu(), rope[1][:, :, K - Q:K].cpu()
        qh = qh * c + torch.cat((-qh[..., D // 2:], qh[..., :D // 2]), dim=-1) * s
        att, _, _ = O.topk_kv_reuse_attention(qh, key.cpu(), val.cpu(), k, attention_mask=am)
        ref = m.o_proj(att.transpose(1, 2).reshape(2, Q, C).to(dev))
    torch.cuda.synchronize()
    close(y, ref, 1e-4, "module output")
    # under autograd: gradients of q_proj, o_proj, the hidden states and the dense KV
    # against torch autograd through the oracle's formula on the CPU (fp32)
    hs_g, key_g, val_g = (t.clone().requires_grad_(True) for t in (hs, key, val))
    wout = torch.randn(2, Q, C, generator=g)
    y = m(hs_g, (key_g, val_g), rope, am.to(dev))
    (y * wout.to(dev)).sum().backward()
    torch.cuda.synchronize()
    qw, ow = (m.q_proj.weight.detach().cpu().requires_grad_(True), m.o_proj.weight.detach().cpu().requires_grad_(True))
    hs_c, key_c, val_c = (t.detach().cpu().requires_grad_(True) for t in (hs, key, val))
    qh = (hs_c @ qw.T).view(2, Q, H, D).transpose(1, 2)
    qh = qh * c + torch.cat((-qh[..., D // 2:], qh[..., :D // 2]), dim=-1) * s
    att, _, _ = O.topk_kv_reuse_attention(qh, key_c, val_c, k, attention_mask=am)
    yr = att.transpose(1, 2).reshape(2, Q, C) @ ow.T
    close(y.detach(), yr.detach(), 1e-4, "module output under autograd")
    (yr * wout).sum().backward()
    for name, got, want in (("q_proj", m.q_proj.weight.grad, qw.grad), ("o_proj", m.o_proj.weight.grad, ow.grad),
                            ("hidden states", hs_g.grad, hs_c.grad), ("key", key_g.grad, key_c.grad),
                            ("value", val_g.grad, val_c.grad)):
        assert got is not None, f"{name}: no gradient"
        close(got, want, 1e-4, f"gradient of {name}")
    # dropout on the probabilities in training mode (hybrid_dense_delta_topk.py:351): eval
    # unchanged, training random but reproducible under a seed
    md = sgsa_amd.TopKSparseKVReuseAttention(SimpleNamespace(num_attention_heads=H, head_dim=D, hidden_size=C,
                                                             top_k=k, dropout=0.5)).to(dev)
    md.load_state_dict(m.state_dict())
    with torch.no_grad():
        assert torch.equal(md.eval()(hs, (key, val), rope, am.to(dev)), m(hs, (key, val), rope, am.to(dev)))
        md.train()
        ys = []
        for seed in (1, 1, 2):
            torch.manual_seed(seed)
            ys.append(md(hs, (key, val), rope, am.to(dev)))
    assert torch.isfinite(ys[0]).all() and torch.equal(ys[0], ys[1]) and not torch.equal(ys[0], ys[2])
