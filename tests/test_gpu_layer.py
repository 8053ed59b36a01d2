"""GPU parity of the retrieval (K1+K2) and of the whole layer forward.

Oracle: oracle/sgsa_oracle.py (fp32 CPU restatement of modeling_sgsa.py and
the recurrent core).  Inputs are the benchmark distributions (make_inputs);
bf16 runs feed the oracle the bf16-rounded values.
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)


def _close(got, ref, rel, name=""):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    scale = ref.abs().max().clamp_min(1e-12)
    err = (got - ref).abs().max() / scale
    assert torch.isfinite(got).all(), f"{name}: non-finite"
    assert err <= rel, f"{name}: max error {err:.3e} relative to max|ref| {scale:.3e} exceeds {rel:.1e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_retrieval_matches_oracle(dev, dtype, tol):
    B, T, H, D, k = 1, 512, 4, 64, 32
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=0)
    ret = O.token_topk_retrieval(x["q_f32"], x["k_f32"], x["v_f32"], k)
    got = sgsa_amd.sparse_retrieve(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), k)
    torch.cuda.synchronize()
    gi = got["indices"].cpu()
    mism = (gi != ret["indices"]).any(-1).float().mean().item()
    assert mism < 0.01, f"{mism:.3%} of rows select a different key set"
    _close(got["k_hat"], ret["k_hat"], tol, "k_hat")
    _close(got["v_hat"], ret["v_hat"], tol, "v_hat")
    _close(got["weights"], ret["weights"], tol, "weights")
    for name in ("concentration", "max_confidence", "novelty", "write_conflict", "entropy",
                 "avg_distance", "local_ratio", "sink_ratio", "remote_ratio"):
        _close(got["diagnostics"][name], ret["diagnostics"][name], max(tol, 1e-4), name)
    # margins: row 0 has a finfo.min second slot in both
    gm, rm = got["diagnostics"]["score_margin"].cpu(), ret["diagnostics"]["score_margin"]
    _close(gm[..., 1:], rm[..., 1:], max(tol, 1e-4), "score_margin")


def test_retrieval_causality_and_shapes(dev):
    # scripts/sgsa_sanity_checks.py:22-39
    B, T, H, D, k = 2, 12, 4, 24, 4
    g = torch.Generator().manual_seed(1)
    q, kk, v = (torch.randn(B, T, H, D, generator=g).to(dev) for _ in range(3))
    out = sgsa_amd.SparseRetriever(type("C", (), {"top_k": k, "retrieval_mode": "token_only"})())(q, kk, v)
    pos = torch.arange(T, device=dev).view(1, 1, T, 1)
    assert torch.all(out["indices"] <= pos)
    assert out["k_hat"].shape == (B, T, H, D) and out["v_hat"].shape == (B, T, H, D)
    assert out["diagnostics"]["score_margin"].shape == (B, H, T)
    assert out["indices"].dtype == torch.int64


@pytest.mark.parametrize("dtype,tol,dims", [
    (torch.float32, 1e-4, (1, 512, 4, 64, 32)),       # config 0
    (torch.bfloat16, 2e-2, (1, 1024, 2, 128, 256)),
])
@pytest.mark.parametrize("write_mode", ["direct", "residual"])
def test_layer_forward_matches_recurrent_oracle(dev, dtype, tol, dims, write_mode):
    B, T, H, D, k = dims
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=0)
    ref = O.sgsa_layer_forward(x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"],
                               x["budget"], k, write_mode=write_mode)
    o, st = sgsa_amd.sgsa_layer_forward(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), x["q"].to(dev),
                                        x["beta"].to(dev), x["gamma"].to(dev), x["budget"].to(dev), k,
                                        write_mode=write_mode)
    torch.cuda.synchronize()
    _close(o, ref["o"], tol, "o")
    _close(st, ref["final_state"], tol, "final_state")


def test_layer_forward_deterministic(dev):
    B, T, H, D, k = 1, 700, 2, 128, 64
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=3)
    args = [x[n].to(dev) for n in ("q", "k", "v", "q", "beta", "gamma", "budget")]
    o1, s1 = sgsa_amd.sgsa_layer_forward(*args, k)
    o2, s2 = sgsa_amd.sgsa_layer_forward(*args, k)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("write_mode", ["direct", "residual"])
@pytest.mark.parametrize("dims", [(1, 2100, 2, 128, 256), (2, 700, 3, 128, 64)])
def test_tiled_gather_matches_direct_gather(dev, write_mode, dims):
    # the LDS-tiled MFMA form of K2 against the row-gather form on the same top-k lists
    B, T, H, D, k = dims
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=5)
    q, kk, v, bud = x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), x["budget"].to(dev)
    idx, sc, top2, cnt, spl = sgsa_amd.score_topk(q, kk, k, sorted=False, return_split=True)
    wk_t, vh_t, al_t = sgsa_amd.gather_gate(kk, v, idx, sc, top2, cnt, bud, split=spl, write_mode=write_mode)
    wk_d, vh_d, al_d = sgsa_amd.gather_gate(kk, v, idx, sc, top2, cnt, bud, split=None, write_mode=write_mode)
    torch.cuda.synchronize()
    assert (spl <= cnt).all() and (spl >= 0).all()
    _close(wk_t, wk_d, 1e-2, "write_key")
    _close(vh_t, vh_d, 1e-2, "v_hat")
    _close(al_t, al_d, 1e-2, "alpha")


@pytest.mark.parametrize("dtype,tol,dims", [
    (torch.float32, 1e-4, (1, 512, 4, 64, 32)),        # direct gather
    (torch.bfloat16, 2e-2, (1, 1024, 2, 128, 256)),    # tile lists (D = 128)
    (torch.bfloat16, 2e-2, (2, 700, 3, 128, 64)),      # tile lists, ragged last row block
    (torch.bfloat16, 2e-2, (1, 300, 2, 64, 40)),       # direct gather, bf16
])
@pytest.mark.parametrize("write_mode", ["direct", "residual"])
def test_layer_retrieve_matches_oracle(dev, dtype, tol, dims, write_mode):
    # the (write key, v_hat, alpha) that the layer feeds to the chunked update
    B, T, H, D, k = dims
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=2)
    ref = O.sgsa_layer_forward(x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"],
                               x["budget"], k, write_mode=write_mode)
    wk, vh, al = sgsa_amd.sgsa_layer_retrieve(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), x["budget"].to(dev),
                                              k, write_mode=write_mode)
    torch.cuda.synchronize()
    _close(wk, ref["write_key"], tol, "write_key")
    _close(vh, ref["v_hat"], tol, "v_hat")
    _close(al, ref["alpha"], max(tol, 1e-4), "alpha")


def test_layer_forward_carries_the_sparse_write(dev):
    # the sparse write must be visible in o: closer to the full reference than
    # to the reference without it (budget -> -inf gives alpha = 0)
    B, T, H, D, k = 1, 512, 2, 128, 64
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=7)
    bud = torch.full_like(x["budget"], 6.0)   # sigmoid ~ 1: large gates
    args = (x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"])
    ref = O.sgsa_layer_forward(*args, bud, k, alpha_max=0.9)["o"]
    ref0 = O.sgsa_layer_forward(*args, torch.full_like(bud, -1e4), k, alpha_max=0.9)["o"]
    o, _ = sgsa_amd.sgsa_layer_forward(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), x["q"].to(dev),
                                       x["beta"].to(dev), x["gamma"].to(dev), bud.to(dev), k, alpha_max=0.9)
    torch.cuda.synchronize()
    o = o.float().cpu()
    gap = (ref - ref0).abs().max()
    assert gap > 0.05 * ref.abs().max(), "the sparse write is too small to test"
    assert (o - ref).abs().max() < 0.25 * gap


@pytest.mark.parametrize("dtype,tol,dims", [
    (torch.float32, 1e-4, (1, 512, 4, 64, 32)),        # direct gather
    (torch.bfloat16, 2e-2, (1, 1024, 2, 128, 256)),    # threshold form (D = 128)
])
@pytest.mark.parametrize("write_mode", ["direct", "residual"])
def test_layer_stats_match_oracle(dev, dtype, tol, dims, write_mode):
    # sgsa_layer_fwd_stats / sgsa_layer_retrieve_stats: alpha, each row's largest
    # weight (max_confidence, modeling_sgsa.py:374) and the write-key norm ratio (:614)
    B, T, H, D, k = dims
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=4)
    ref = O.sgsa_layer_forward(x["q_f32"], x["k_f32"], x["v_f32"], x["q_f32"], x["beta"], x["gamma"],
                               x["budget"], k, write_mode=write_mode)
    g = {n: x[n].to(dev) for n in ("q", "k", "v", "beta", "gamma", "budget")}
    s1, s2 = {}, {}
    sgsa_amd.sgsa_layer_forward(g["q"], g["k"], g["v"], g["q"], g["beta"], g["gamma"], g["budget"], k,
                                write_mode=write_mode, stats=s1)
    sgsa_amd.sgsa_layer_retrieve(g["q"], g["k"], g["v"], g["budget"], k, write_mode=write_mode, stats=s2)
    torch.cuda.synchronize()
    kh = ref["retrieval"]["k_hat"]
    ratio = (ref["write_key"].norm(dim=-1) / kh.norm(dim=-1).clamp_min(1e-6)).clamp(0, 10).transpose(1, 2)
    for s in (s1, s2):
        _close(s["alpha"], ref["alpha"], tol, "alpha")
        _close(s["row_stats"][0], ref["retrieval"]["diagnostics"]["max_confidence"], tol, "max_confidence")
        if write_mode == "residual":
            _close(s["row_stats"][1], ratio, tol, "k_hat_perp ratio")
        else:
            assert (s["row_stats"][1] == 0).all()
