"""GPU parity of the score GEMM + exact top-k (K1).

Bit-exactness is checked on identical fp32 scores: sgsa_score_dump returns the
scores K1 selects on, and the oracle's (score desc, index asc) top-k of those
scores must equal K1's indices exactly.
"""

import math

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)

FMIN = torch.finfo(torch.float32).min


def _oracle_on_dump(dump, top_k, causal=True, q_offset=0, row0=0):
    B, H, R, Tk = dump.shape
    pos = torch.arange(row0, row0 + R) + q_offset
    if causal:
        valid = (torch.arange(Tk)[None, :] <= pos[:, None])[None, None].expand(B, H, R, Tk)
    else:
        valid = torch.ones(B, H, R, Tk, dtype=torch.bool)
    return O.masked_topk(dump, valid, min(top_k, Tk))


def _check_rows(idx, sc, cnt, top2, dump, top_k, causal=True, q_offset=0, row0=0):
    ovals, oidx, ovalid = _oracle_on_dump(dump, top_k, causal, q_offset, row0)
    R = dump.shape[2]
    gi = idx[:, :, row0:row0 + R].long().cpu()
    gs = sc[:, :, row0:row0 + R].cpu()
    gc = cnt[:, :, row0:row0 + R].cpu()
    assert torch.equal(gc, ovalid.sum(-1).to(gc.dtype)), "valid slot counts differ"
    assert torch.equal(gi, oidx), f"indices differ in {(gi != oidx).sum().item()} slots"
    assert torch.equal(gs, ovals.float()), "selected scores differ"
    t2 = top2[:, :, row0:row0 + R].cpu()
    assert torch.equal(t2[..., 0], ovals[..., 0])
    if ovals.shape[-1] >= 2:
        assert torch.equal(t2[..., 1], ovals[..., 1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 700, 2, 128, 64), (2, 130, 3, 64, 16), (1, 257, 1, 5, 7)])
def test_topk_bit_exact_on_dumped_scores(dev, dtype, shape):
    B, T, H, D, k = shape
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, T, H, D, generator=g).to(dev, dtype)
    kk = torch.randn(B, T, H, D, generator=g).to(dev, dtype)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=True)
    dump = sgsa_amd.score_dump(q, kk, 0, T)
    torch.cuda.synchronize()
    _check_rows(idx, sc, cnt, top2, dump.cpu(), k)


def test_topk_ties_break_by_lowest_index(dev):
    # keys drawn from 5 distinct rows: every score is tied many times
    B, T, H, D, k = 1, 400, 2, 128, 37
    g = torch.Generator().manual_seed(1)
    base = torch.randn(5, H, D, generator=g)
    pick = torch.randint(0, 5, (T,), generator=g)
    kk = base[pick][None].to(dev, torch.bfloat16).contiguous()
    q = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=True)
    dump = sgsa_amd.score_dump(q, kk, 0, T)
    torch.cuda.synchronize()
    _check_rows(idx, sc, cnt, top2, dump.cpu(), k)


def test_topk_all_equal_scores(dev):
    B, T, H, D, k = 1, 300, 1, 64, 20
    q = torch.zeros(B, T, H, D, device=dev)
    kk = torch.randn(B, T, H, D, device=dev)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=True)
    torch.cuda.synchronize()
    for t in range(T):
        kq = min(k, t + 1)
        assert idx[0, 0, t, :kq].tolist() == list(range(kq))
        assert (sc[0, 0, t, :kq] == 0).all()


def test_topk_unsorted_same_set_and_deterministic(dev):
    B, T, H, D, k = 1, 1500, 2, 128, 50
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    kk = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    i1, s1, _, c1 = sgsa_amd.score_topk(q, kk, k, sorted=True)
    i0, s0, _, c0 = sgsa_amd.score_topk(q, kk, k, sorted=False)
    i2, s2, _, c2 = sgsa_amd.score_topk(q, kk, k, sorted=False)
    torch.cuda.synchronize()
    assert torch.equal(c0, c1) and torch.equal(i0, i2) and torch.equal(s0, s2)
    a = i0.cpu().sort(-1).values
    b = i1.cpu().sort(-1).values
    assert torch.equal(a, b)


def test_topk_mass_ties_take_the_radix_path(dev):
    # two distinct key rows: the threshold bin holds far more than 512 candidates
    B, T, H, D, k = 1, 3000, 2, 128, 100
    g = torch.Generator().manual_seed(9)
    base = torch.randn(2, H, D, generator=g)
    kk = base[torch.randint(0, 2, (T,), generator=g)][None].to(dev, torch.bfloat16).contiguous()
    q = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=True)
    dump = sgsa_amd.score_dump(q, kk, 0, T)
    torch.cuda.synchronize()
    _check_rows(idx, sc, cnt, top2, dump.cpu(), k)


def test_topk_heavy_tailed_keys(dev):
    # config-3 style: 1% of key rows scaled x8 (coarse first-pass bins)
    B, T, H, D, k = 1, 4096, 2, 128, 512
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=11, heavy_tail=True, with_budget=False)
    q, kk = x["q"].to(dev), x["k_ret"].to(dev)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=True)
    dump = sgsa_amd.score_dump(q, kk, 0, T)
    torch.cuda.synchronize()
    _check_rows(idx, sc, cnt, top2, dump.cpu(), k)


@pytest.mark.parametrize("q_offset", [0, 37])
def test_topk_noncausal_and_offset(dev, q_offset):
    # hybrid layout: Q queries at key positions Tk-Q.. (q_offset = Tk - Q), multiply scale
    B, Tq, H, D, k = 1, 40, 2, 64, 9
    Tk = Tq + q_offset
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, Tq, H, D, generator=g).to(dev)
    kk = torch.randn(B, Tk, H, D, generator=g).to(dev)
    for causal in (True, False):
        idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, causal=causal, q_offset=q_offset, scale_mode=1)
        dump = sgsa_amd.score_dump(q, kk, 0, Tq, causal=causal, q_offset=q_offset, scale_mode=1)
        torch.cuda.synchronize()
        _check_rows(idx, sc, cnt, top2, dump.cpu(), k, causal, q_offset)


def test_topk_large_rows_subset(dev):
    # north-star-like row length: bit-exact on the last 64 rows, structural checks on all
    B, T, H, D, k = 1, 8192, 2, 128, 2048
    x = O.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=4, with_budget=False)
    q, kk = x["q"].to(dev), x["k"].to(dev)
    idx, sc, top2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=False)
    dump = sgsa_amd.score_dump(q, kk, T - 64, 64)
    torch.cuda.synchronize()
    n = torch.clamp(torch.arange(T) + 1, max=k)
    assert torch.equal(cnt[0, 0].cpu(), n.to(torch.int32))
    ic = idx.cpu()
    pos = torch.arange(T)[None, None, :, None]
    slot = torch.arange(k)[None, None, None, :]
    live = slot < n[None, None, :, None]
    assert (ic[live.expand_as(ic)] <= pos.expand_as(ic)[live.expand_as(ic)]).all(), "causality"
    # bit-exact on the dumped rows (after sorting both to the same order)
    i_s, s_s, _, c_s = sgsa_amd.score_topk(q, kk, k, sorted=True)
    torch.cuda.synchronize()
    _check_rows(i_s, s_s, c_s, top2, dump.cpu(), k, row0=T - 64)


def _decode_tile_lists(lists, offs, B, T, H, top_k):
    """(mask [B*H,T,T] of selected (row, key), scores at those) from the layer-path tile lists."""
    nqb = ntm = (T + 63) // 64
    kk = min(top_k, T)
    cap = 16 * (kk + 512)
    R = B * H * nqb * 4
    ent = lists.view(torch.int32).view(R, cap, 2).cpu()
    off = offs.view(R, ntm + 1).cpu().long()
    mask = torch.zeros(B * H, T, T, dtype=torch.bool)
    smat = torch.zeros(B * H, T, T)
    for r in range(R):
        bh, qb, w = r // (nqb * 4), (r // 4) % nqb, r % 4
        ntile = (min(T, qb * 64 + 64) + 63) // 64
        n = int(off[r, ntile])
        if n == 0:
            continue
        e = ent[r, :n]
        tile = torch.searchsorted(off[r, 1:ntile + 1].contiguous(), torch.arange(n), right=True)
        key = tile * 64 + (e[:, 1] & 63).long()
        row = qb * 64 + 16 * w + (e[:, 1] >> 8).long()
        s = e[:, 0].contiguous().view(torch.float32)
        keep = s != float("-inf")
        assert not mask[bh, row[keep], key[keep]].any(), "a (row, key) appears twice"
        mask[bh, row[keep], key[keep]] = True
        smat[bh, row[keep], key[keep]] = s[keep]
    return mask, smat


@pytest.mark.parametrize("case", ["random", "ties", "mass_ties", "heavy_tail", "d64"])
def test_tile_lists_hold_the_exact_selection(dev, case):
    # the layer-path K1 (tile lists) selects exactly what the row-list K1 selects
    B, T, H, D, k = 1, 2100, 2, 128, 256
    g = torch.Generator().manual_seed(21)
    if case == "random":
        q, kk = torch.randn(B, T, H, D, generator=g), torch.randn(B, T, H, D, generator=g)
    elif case == "ties":
        base = torch.randn(5, H, D, generator=g)
        kk = base[torch.randint(0, 5, (T,), generator=g)][None]
        q = torch.randn(B, T, H, D, generator=g)
    elif case == "mass_ties":   # threshold bin beyond the candidate cap: radix fallback blocks
        base = torch.randn(2, H, D, generator=g)
        kk = base[torch.randint(0, 2, (T,), generator=g)][None]
        q = torch.randn(B, T, H, D, generator=g)
    elif case == "heavy_tail":
        x = O.make_inputs(B, T, H, D, dtype=torch.float32, seed=12, heavy_tail=True, with_budget=False)
        q, kk = x["q"], x["k_ret"]
    else:
        B, T, H, D, k = 2, 700, 3, 64, 100
        q, kk = torch.randn(B, T, H, D, generator=g), torch.randn(B, T, H, D, generator=g)
    q, kk = q.to(dev, torch.bfloat16).contiguous(), kk.to(dev, torch.bfloat16).contiguous()
    lists, offs, t2l, cl = sgsa_amd.score_topk_lists(q, kk, k)
    idx, sc, t2, cnt = sgsa_amd.score_topk(q, kk, k, sorted=False)
    torch.cuda.synchronize()
    assert torch.equal(cl.cpu(), cnt.cpu()), "counts differ"
    assert torch.equal(t2l.cpu(), t2.cpu()), "top2 differs"
    mask, smat = _decode_tile_lists(lists, offs, B, T, H, k)
    ref = torch.zeros_like(mask)
    rsc = torch.zeros_like(smat)
    kq = min(k, T)
    ic, sg, cc = idx.cpu().long().view(B * H, T, kq), sc.cpu().view(B * H, T, kq), cnt.cpu().view(B * H, T)
    live = torch.arange(kq)[None, None, :] < cc[..., None]
    bi, ri, si = live.nonzero(as_tuple=True)
    ref[bi, ri, ic[bi, ri, si]] = True
    rsc[bi, ri, ic[bi, ri, si]] = sg[bi, ri, si]
    assert torch.equal(mask, ref), f"selected sets differ in {(mask != ref).sum().item()} (row, key) pairs"
    assert torch.equal(smat[mask], rsc[mask]), "selected scores differ"
