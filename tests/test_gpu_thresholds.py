"""GPU parity of the threshold form of the layer path (what sgsa_layer_fwd runs
for bf16, D = 128): K1 leaves one exact cut per row, K2 recomputes the scores
and applies it.

* The cut selects exactly the rows of the row-list K1 (the lowest-index top-k
  of K1's own fp32 scores, checked against the oracle elsewhere), applied to
  the scores sgsa_score_dump returns -- on random, tied, mass-tied (radix
  fallback blocks), bursts of tied keys (the 128-row kernel's candidate
  staging overflows and the block goes to the fallback), score ties between
  different accumulators across the 128-row kernel's bin edges (it bins raw
  accumulators) and heavy-tailed inputs and a ragged shape.
* K2's selection, key for key: the known-answer variant of the threshold
  gather reports each row's {count, index sum, index hash xor} of the keys it
  weighs, which must equal those of the row lists exactly.
* K2 on the thresholds gives the outputs of K2 on the tile lists: the same
  selection, and weights that differ only in the rounding of the exponent's
  argument (one fused multiply-add on the raw accumulator instead of the
  rounded score), so within 1e-2 of the largest magnitude.
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)


def _inputs(case, dev, big=False):
    # big: the headline top-k (2048) at T = 8192 (ragged: T = 8100, B = 2, H = 3)
    B, T, H, D, k = (1, 8192, 2, 128, 2048) if big else (1, 2100, 2, 128, 256)
    g = torch.Generator().manual_seed(33)
    if case == "random":
        q, kk = torch.randn(B, T, H, D, generator=g), torch.randn(B, T, H, D, generator=g)
    elif case == "ties":   # five distinct key rows: exact score ties at every threshold
        base = torch.randn(5, H, D, generator=g)
        kk = base[torch.randint(0, 5, (T,), generator=g)][None]
        q = torch.randn(B, T, H, D, generator=g)
    elif case == "mass_ties":   # threshold bins beyond the candidate cap: radix fallback blocks
        base = torch.randn(2, H, D, generator=g)
        kk = base[torch.randint(0, 2, (T,), generator=g)][None]
        q = torch.randn(B, T, H, D, generator=g)
    elif case == "tile_burst":
        # Queries near one key vector A, which scores far above the rest and ties
        # exactly.  A fills key tile 1 and a quarter of every other tile, so a
        # row's threshold bin is A's (tie cut by index) and, in K1's 128-row
        # kernel, a lane stages a few candidates in tile 0 and then more in tile 1
        # than its staging column holds: the block goes to the radix fallback.
        B, T, k = 1, 500, 100
        A = torch.randn(H, D, generator=g)
        j = torch.arange(T)
        is_a = ((j >= 64) & (j < 128)) | (j % 16 < 4)
        kk = 0.05 * torch.randn(B, T, H, D, generator=g)
        kk[:, is_a] = A
        q = A + 0.01 * torch.randn(B, T, H, D, generator=g)
    elif case == "straddle":
        # Every query is (1, 1, 0, ..), every key (1.5, m 2^-23, 0, ..) with m < 256:
        # accumulators 1.5 + m 2^-23, consecutive fp32 values, which the score scale
        # 1/sqrt(128) maps two to one score about a third of the time.  Ties by score
        # then span different accumulators, and the bins (fitted to this narrow
        # range, about 1.5 accumulator steps wide) put edges between them.
        q = torch.zeros(B, T, H, D)
        q[..., 0] = 1.0
        q[..., 1] = 1.0
        kk = torch.zeros(B, T, H, D)
        kk[..., 0] = 1.5
        kk[..., 1] = torch.randint(0, 256, (B, T, H), generator=g).float() * 2.0 ** -23
    elif case == "heavy_tail":
        x = O.make_inputs(B, T, H, D, dtype=torch.float32, seed=12, heavy_tail=True, with_budget=False)
        q, kk = x["q"], x["k_ret"]
    else:   # ragged: T not a multiple of the 128-row gather block, B > 1
        B, T, H, D, k = (2, 8100, 3, 128, 2048) if big else (2, 700, 3, 128, 100)
        q, kk = torch.randn(B, T, H, D, generator=g), torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    bud = torch.randn(B, T, H, generator=g)
    cast = lambda t: t.to(dev, torch.bfloat16).contiguous()
    return cast(q), cast(kk), cast(v), bud.to(dev), k


CASES = ["random", "ties", "mass_ties", "tile_burst", "straddle", "heavy_tail", "ragged"]
# (case, big): every case at its own size, and all but tile_burst (a fixed T = 500
# construction) at top-k 2048 with T = 8192
SIZED = [(c, False) for c in CASES] + [(c, True) for c in CASES if c != "tile_burst"]
SIZE_IDS = [f"{c}-k2048" if big else c for c, big in SIZED]


@pytest.mark.parametrize("case,big", SIZED, ids=SIZE_IDS)
def test_thresholds_select_exactly_the_row_lists(dev, case, big):
    q, kk, v, _, k = _inputs(case, dev, big)
    print(f"thresholds vs row lists: case {case} shape {tuple(q.shape)} k={k}", flush=True)
    B, T, H, D = q.shape
    thr, t2t, ct = sgsa_amd.score_topk_thresholds(q, kk, k)
    idx, sc, t2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=False)
    dump = sgsa_amd.score_dump(q, kk, 0, T)
    torch.cuda.synchronize()
    assert torch.equal(ct.cpu(), cnt.cpu()), "counts differ"
    assert torch.equal(t2t.cpu(), t2.cpu()), "top2 differs"
    s = dump.cpu()                                              # [B,H,T,T] K1's fp32 scores
    th = thr[..., 0].cpu().contiguous().view(torch.float32)[..., None]
    cut = thr[..., 1].cpu().long()[..., None]
    j = torch.arange(T)
    causal = (j[None, :] <= j[:, None])[None, None]
    mask = causal & ((s > th) | ((s == th) & (j[None, None, None, :] <= cut)))
    kq = min(k, T)
    ref = torch.zeros(B, H, T, T, dtype=torch.bool)
    ic, cc = idx.cpu().long(), cnt.cpu()
    live = torch.arange(kq)[None, None, None, :] < cc[..., None]
    bi, hi, ri, si = live.nonzero(as_tuple=True)
    ref[bi, hi, ri, ic[bi, hi, ri, si]] = True
    assert torch.equal(mask, ref), f"selected sets differ in {(mask != ref).sum().item()} (row, key) pairs"
    if case in ("ties", "mass_ties", "tile_burst", "straddle"):
        assert (thr[..., 1] != 0x7fffffff).any(), "no row needed a tie cut"


@pytest.mark.parametrize("case,big", SIZED, ids=SIZE_IDS)
def test_threshold_gather_selects_key_for_key(dev, case, big):
    # K2 recomputes the scores and applies K1's cut: its selection, summarised
    # per row by the known-answer variant of the same kernel, equals the row
    # lists' exactly (count, index sum, index hash xor)
    q, kk, v, _, k = _inputs(case, dev, big)
    print(f"threshold gather selection: case {case} shape {tuple(q.shape)} k={k}", flush=True)
    thr, t2t, ct = sgsa_amd.score_topk_thresholds(q, kk, k)
    got = sgsa_amd.gather_thresholds_selection(q, kk, v, thr, t2t, ct, k)
    idx, sc, t2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=False)
    want = sgsa_amd.selection_summary(idx, cnt)
    torch.cuda.synchronize()
    bad = (got != want).any(-1)
    assert not bad.any(), f"{int(bad.sum())} rows select differently (first {bad.nonzero()[0].tolist()})"


@pytest.mark.parametrize("write_mode", ["direct", "residual"])
@pytest.mark.parametrize("case,big", SIZED, ids=SIZE_IDS)
def test_threshold_gather_equals_list_gather(dev, case, big, write_mode):
    q, kk, v, bud, k = _inputs(case, dev, big)
    print(f"threshold gather vs list gather: case {case} shape {tuple(q.shape)} k={k} {write_mode}", flush=True)
    thr, t2t, ct = sgsa_amd.score_topk_thresholds(q, kk, k)
    wk_t, vh_t, al_t = sgsa_amd.gather_thresholds(q, kk, v, thr, t2t, ct, bud, k, write_mode=write_mode)
    lists, offs, t2l, cl = sgsa_amd.score_topk_lists(q, kk, k)
    wk_l, vh_l, al_l = sgsa_amd.gather_lists(kk, v, lists, offs, t2l, cl, bud, k, write_mode=write_mode)
    torch.cuda.synchronize()
    for name, a, b in (("write key", wk_t, wk_l), ("v_hat", vh_t, vh_l), ("alpha", al_t, al_l)):
        a, b = a.float().cpu(), b.float().cpu()
        assert torch.isfinite(a).all(), f"{name}: non-finite"
        err = (a - b).abs().max() / b.abs().max().clamp_min(1e-12)
        assert err <= 1e-2, f"{name}: {err:.3e} from the tile-list gather"


def test_layer_path_is_the_threshold_form(dev):
    # sgsa_layer_retrieve (bf16, D = 128) returns what the threshold halves return
    q, kk, v, bud, k = _inputs("random", dev)
    wk, vh, al = sgsa_amd.sgsa_layer_retrieve(q, kk, v, bud, k)
    thr, t2t, ct = sgsa_amd.score_topk_thresholds(q, kk, k)
    wk_t, vh_t, al_t = sgsa_amd.gather_thresholds(q, kk, v, thr, t2t, ct, bud, k)
    torch.cuda.synchronize()
    assert torch.equal(wk, wk_t) and torch.equal(vh, vh_t) and torch.equal(al, al_t)
