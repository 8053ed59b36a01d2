"""Pins the CPU oracle (oracle/sgsa_oracle.py) before anything is compared with it.

Each check is chosen so that a plausible mistake in the oracle (a dropped term,
the sparse residual read from the wrong state, an off-by-one decay, a wrong tie
order) fails at least one of them.  The reference ships no golden vectors for
this path (its tests are the chunk==recurrent equalities of
tests/test_sgsa_core.py:25-50 and the causality checks of
scripts/sgsa_sanity_checks.py:22-39), so these are closed forms, algebraic
restatements, invariants and brute force.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import sgsa_oracle as O


def _inputs(seed=0, B=2, T=9, H=3, D=5, dtype=torch.float64):
    # Same draw shape as the reference's _random_inputs (tests/test_sgsa_core.py:11-22).
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    q, k, v, sk, sv = (r(B, T, H, D) for _ in range(5))
    beta = torch.sigmoid(r(B, T, H))
    gamma = torch.sigmoid(r(B, T, H))
    alpha = 0.25 * torch.sigmoid(r(B, T, H))
    return q, k, v, sk, sv, beta, gamma, alpha


# ---------------------------------------------------------------- recurrence

def _one_step_by_hand(S, q, k, v, sk, sv, b, g, a, sparse_reads_base=True):
    """Scalar loops, one token, one head: the recurrence written out element-wise."""
    d, e = len(k), len(v)
    base = [[g * S[i][j] for j in range(e)] for i in range(d)]
    pred = [sum(base[i][j] * k[i] for i in range(d)) for j in range(e)]
    new = [[base[i][j] + k[i] * b * (v[j] - pred[j]) for j in range(e)] for i in range(d)]
    src = base if sparse_reads_base else new
    pred_s = [sum(src[i][j] * sk[i] for i in range(d)) for j in range(e)]
    new = [[new[i][j] + sk[i] * a * (sv[j] - pred_s[j]) for j in range(e)] for i in range(d)]
    o = [sum(new[i][j] * q[i] for i in range(d)) for j in range(e)]
    return new, o


def test_recurrence_two_tokens_by_hand():
    q, k, v, sk, sv, beta, gamma, alpha = _inputs(B=1, T=2, H=1, D=3)
    S0 = torch.randn(1, 1, 3, 3, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    out, st = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, alpha, S0, True)
    S = S0[0, 0].tolist()
    outs = []
    for t in range(2):
        S, o = _one_step_by_hand(S, q[0, t, 0].tolist(), k[0, t, 0].tolist(), v[0, t, 0].tolist(),
                                 sk[0, t, 0].tolist(), sv[0, t, 0].tolist(), float(beta[0, t, 0]),
                                 float(gamma[0, t, 0]), float(alpha[0, t, 0]))
        outs.append(o)
    torch.testing.assert_close(out[0, :, 0], torch.tensor(outs, dtype=torch.float64), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(st[0, 0], torch.tensor(S, dtype=torch.float64), rtol=1e-12, atol=1e-12)
    # the planted mistake (sparse residual read from the updated state) must be detectable
    S_bad = S0[0, 0].tolist()
    S_bad, _ = _one_step_by_hand(S_bad, q[0, 0, 0].tolist(), k[0, 0, 0].tolist(), v[0, 0, 0].tolist(),
                                 sk[0, 0, 0].tolist(), sv[0, 0, 0].tolist(), float(beta[0, 0, 0]),
                                 float(gamma[0, 0, 0]), float(alpha[0, 0, 0]), sparse_reads_base=False)
    _, st1 = O.naive_recurrent_sgsa(q[:, :1], k[:, :1], v[:, :1], beta[:, :1], gamma[:, :1],
                                    sk[:, :1], sv[:, :1], alpha[:, :1], S0, True)
    assert (st1[0, 0] - torch.tensor(S_bad, dtype=torch.float64)).abs().max() > 1e-3


def test_recurrence_matches_transition_matrix_form():
    # S_t = g (I - b k k^T - a s s^T) S_{t-1} + b k v^T + a s w^T  (both residuals read g*S)
    q, k, v, sk, sv, beta, gamma, alpha = _inputs(seed=3, B=1, T=7, H=2, D=4)
    S0 = torch.randn(1, 2, 4, 4, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    out, st = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, alpha, S0, True)
    eye = torch.eye(4, dtype=torch.float64)
    for h in range(2):
        S = S0[0, h].clone()
        for t in range(7):
            kt, st_, vt, sv_t = k[0, t, h], sk[0, t, h], v[0, t, h], sv[0, t, h]
            b, g, a = beta[0, t, h], gamma[0, t, h], alpha[0, t, h]
            A = g * (eye - b * torch.outer(kt, kt) - a * torch.outer(st_, st_))
            S = A @ S + b * torch.outer(kt, vt) + a * torch.outer(st_, sv_t)
            torch.testing.assert_close(out[0, t, h], S.T @ q[0, t, h], rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(st[0, h], S, rtol=1e-10, atol=1e-10)


def test_recurrence_special_cases():
    q, k, v, sk, sv, beta, gamma, alpha = _inputs(seed=5, B=1, T=6, H=2, D=4)
    S0 = torch.randn(1, 2, 4, 4, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    zero = torch.zeros_like(beta)
    # decay only: o_t = c^(t+1) S0^T q_t
    c = 0.9
    out, _ = O.naive_recurrent_sgsa(q, k, v, zero, torch.full_like(gamma, c), sk, sv, zero, S0, False)
    for t in range(6):
        exp = (c ** (t + 1)) * torch.einsum("bhde,bhd->bhe", S0, q[:, t])
        torch.testing.assert_close(out[:, t], exp, rtol=1e-12, atol=1e-12)
    # exact overwrite: unit key, beta=1, gamma=1, no sparse write => S^T k = v after the step
    kk = k[:, :1] / k[:, :1].norm(dim=-1, keepdim=True)
    _, st = O.naive_recurrent_sgsa(q[:, :1], kk, v[:, :1], torch.ones_like(beta[:, :1]),
                                   torch.ones_like(gamma[:, :1]), None, None, None, S0, True)
    torch.testing.assert_close(torch.einsum("bhde,bhd->bhe", st, kk[:, 0]), v[:, 0], rtol=1e-12, atol=1e-12)
    # no sparse arguments == sparse write with alpha = 0
    o1, s1 = O.naive_recurrent_sgsa(q, k, v, beta, gamma, None, None, None, S0, True)
    o2, s2 = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, zero, S0, True)
    torch.testing.assert_close(o1, o2, rtol=0, atol=0)
    torch.testing.assert_close(s1, s2, rtol=0, atol=0)


def test_state_continuation():
    q, k, v, sk, sv, beta, gamma, alpha = _inputs(seed=9, T=10)
    full, sf = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, alpha, None, True)
    a, sa = O.naive_recurrent_sgsa(q[:, :4], k[:, :4], v[:, :4], beta[:, :4], gamma[:, :4],
                                   sk[:, :4], sv[:, :4], alpha[:, :4], None, True)
    b, sb = O.naive_recurrent_sgsa(q[:, 4:], k[:, 4:], v[:, 4:], beta[:, 4:], gamma[:, 4:],
                                   sk[:, 4:], sv[:, 4:], alpha[:, 4:], sa, True)
    torch.testing.assert_close(torch.cat([a, b], 1), full, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(sb, sf, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- chunk form

@pytest.mark.parametrize("chunk", [1, 2, 3, 4, 5, 16])
@pytest.mark.parametrize("sparse", [False, True])
def test_chunk_matches_recurrent_fp64(chunk, sparse):
    q, k, v, sk, sv, beta, gamma, alpha = _inputs(seed=chunk)
    S0 = torch.randn(2, 3, 5, 5, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    kw = dict(sparse_k=sk, sparse_v=sv, alpha=alpha) if sparse else {}
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, initial_state=S0, output_final_state=True, **kw)
    co, cs = O.chunk_sgsa_fwd(q, k, v, beta, gamma, initial_state=S0, chunk_size=chunk,
                              output_final_state=True, **kw)
    torch.testing.assert_close(co, ro, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(cs, rs, rtol=1e-10, atol=1e-10)


def test_chunk_matches_recurrent_fp32_reference_tolerance():
    # the reference's own check: chunk_size=4, T=9 (ragged), 1e-5 (tests/test_sgsa_core.py:34-50)
    q, k, v, sk, sv, beta, gamma, alpha = (x.float() for x in _inputs())
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, alpha, None, True)
    co, cs = O.chunk_sgsa_fwd(q, k, v, beta, gamma, sk, sv, alpha, None, 4, True)
    torch.testing.assert_close(co, ro, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(cs, rs, rtol=1e-5, atol=1e-5)


def test_chunk_carry_dtype_rounds_the_state_between_chunks_only():
    # chunk_fwd.py:129 holds the state in q.dtype between chunks; within a chunk everything
    # is fp32.  Restated piecewise: each chunk run alone from the previous chunk's final
    # state with no carry rounding, that state rounded to bf16 in between, must give the
    # carry_dtype run bit for bit (T=10, chunks of 4: a ragged last chunk).
    q, k, v, sk, sv, beta, gamma, alpha = (x.to(torch.bfloat16) for x in _inputs(seed=5, T=10, D=8))
    o, s = O.chunk_sgsa_fwd(q, k, v, beta, gamma, sk, sv, alpha, None, 4, True, carry_dtype=torch.bfloat16)
    pieces, st = [], None
    for a, b in ((0, 4), (4, 8), (8, 10)):
        sl = lambda x: x[:, a:b]
        oi, si = O.chunk_sgsa_fwd(*(sl(x) for x in (q, k, v, beta, gamma, sk, sv, alpha)), st, 4, True)
        pieces.append(oi)
        st = si.to(torch.bfloat16).float()
    assert torch.equal(torch.cat(pieces, 1), o)
    assert torch.equal(st, s)
    # the rounding changes the later chunks and leaves the first chunk's outputs alone
    o32, s32 = O.chunk_sgsa_fwd(q, k, v, beta, gamma, sk, sv, alpha, None, 4, True)
    assert torch.equal(o32[:, :4], o[:, :4])
    assert not torch.equal(o32[:, 4:], o[:, 4:]) and not torch.equal(s32, s)
    # carrying in the compute dtype is the default
    o2, s2 = O.chunk_sgsa_fwd(q, k, v, beta, gamma, sk, sv, alpha, None, 4, True, carry_dtype=torch.float32)
    assert torch.equal(o2, o32) and torch.equal(s2, s32)


# ---------------------------------------------------------------- top-k

def _brute_topk(row, k):
    order = sorted(range(len(row)), key=lambda j: (-row[j], j))[:k]
    return [row[j] for j in order], order


def test_topk_lowest_index_brute_force_with_ties():
    g = torch.Generator().manual_seed(0)
    for trial in range(40):
        n = int(torch.randint(1, 40, (1,), generator=g))
        k = int(torch.randint(1, n + 1, (1,), generator=g))
        # small integer values force many ties
        x = torch.randint(-3, 4, (3, n), generator=g).to(torch.float32) * 0.25
        vals, idx = O.topk_lowest_index(x, k)
        for r in range(3):
            bv, bi = _brute_topk(x[r].tolist(), k)
            assert idx[r].tolist() == bi
            assert vals[r].tolist() == bv


def test_topk_signed_zero_is_a_tie():
    x = torch.tensor([[0.0, -0.0, 0.0, -1.0, -0.0]])
    vals, idx = O.topk_lowest_index(x, 3)
    assert idx[0].tolist() == [0, 1, 2]


def test_masked_topk_causal_rows_and_padding():
    g = torch.Generator().manual_seed(1)
    B, H, T, k = 2, 3, 12, 5
    s = torch.randn(B, H, T, T, generator=g)
    pos = torch.arange(T)
    valid = (pos[None, :] <= pos[:, None])[None, None].expand(B, H, -1, -1)
    vals, idx, ok = O.masked_topk(s, valid, k)
    fmin = torch.finfo(torch.float32).min
    for t in range(T):
        kq = min(k, t + 1)
        assert ok[:, :, t, :kq].all() and not ok[:, :, t, kq:].any()
        assert (idx[:, :, t, kq:] == 0).all() and (vals[:, :, t, kq:] == fmin).all()
        assert (idx[:, :, t, :kq] <= t).all()
        for b in range(B):
            for h in range(H):
                bv, bi = _brute_topk(s[b, h, t, :t + 1].tolist(), kq)
                assert idx[b, h, t, :kq].tolist() == bi


# ---------------------------------------------------------------- retrieval, diagnostics, gate

def test_retrieval_by_explicit_loops():
    g = torch.Generator().manual_seed(2)
    B, T, H, D, k = 1, 7, 2, 4, 3
    q, kk, v = (torch.randn(B, T, H, D, generator=g, dtype=torch.float64) for _ in range(3))
    ret = O.token_topk_retrieval(q, kk, v, k, block_rows=3)
    for h in range(H):
        for t in range(T):
            s = [sum(q[0, t, h, d].item() * kk[0, j, h, d].item() for d in range(D)) / math.sqrt(D)
                 for j in range(t + 1)]
            kq = min(k, t + 1)
            bv, bi = _brute_topk(s, kq)
            m = max(bv)
            e = [math.exp(x - m) for x in bv]
            w = [x / sum(e) for x in e]
            assert ret["indices"][0, h, t, :kq].tolist() == bi
            torch.testing.assert_close(ret["weights"][0, h, t, :kq], torch.tensor(w, dtype=torch.float64))
            exp_k = sum(w[i] * kk[0, bi[i], h] for i in range(kq))
            exp_v = sum(w[i] * v[0, bi[i], h] for i in range(kq))
            torch.testing.assert_close(ret["k_hat"][0, t, h], exp_k)
            torch.testing.assert_close(ret["v_hat"][0, t, h], exp_v)
            margin = (bv[0] - bv[1]) if kq >= 2 else None
            if margin is not None:
                torch.testing.assert_close(ret["diagnostics"]["score_margin"][0, h, t],
                                           torch.tensor(margin, dtype=torch.float64))
    # row 0 with k >= 2: the second slot is finfo.min, so concentration saturates at 1
    assert torch.all(ret["diagnostics"]["concentration"][:, :, 0] == 1.0)


def test_diagnostics_novelty_limits():
    key = torch.tensor([[[[1.0, 2.0, 0.0]]]])
    par = 3.0 * key
    orth = torch.tensor([[[[2.0, -1.0, 5.0]]]])
    sc = torch.tensor([[[[1.0, 0.5]]]])
    w = torch.tensor([[[[0.6, 0.4]]]])
    idx = torch.zeros(1, 1, 1, 2, dtype=torch.long)
    d_par = O.retrieval_diagnostics(sc, w, idx, par, key)
    d_orth = O.retrieval_diagnostics(sc, w, idx, orth, key)
    assert float(d_par["novelty"]) < 1e-5
    assert abs(float(d_orth["novelty"]) - 1.0) < 1e-5
    assert abs(float(d_par["write_conflict"]) - 1.0) < 1e-5
    assert abs(float(d_orth["write_conflict"])) < 1e-5
    torch.testing.assert_close(d_par["concentration"], torch.sigmoid(torch.tensor([[[0.5 / 0.1]]])))
    torch.testing.assert_close(d_par["entropy"], torch.tensor([[[-(0.6 * math.log(0.6) + 0.4 * math.log(0.4))]]]))


def test_alpha_range_and_clip():
    g = torch.Generator().manual_seed(3)
    B, T, H, D = 2, 5, 3, 4
    conc = torch.rand(B, H, T, generator=g)
    nov = torch.rand(B, H, T, generator=g)
    budget = torch.randn(B, T, H, generator=g)
    wk = 10 * torch.randn(B, T, H, D, generator=g)
    vh = 10 * torch.randn(B, T, H, D, generator=g)
    a = O.compute_alpha(conc, nov, budget, wk, vh, 0.25)
    assert torch.all(a >= 0) and torch.all(a <= 0.25 + 1e-7)
    raw = 0.25 * conc.transpose(1, 2) * nov.transpose(1, 2) * torch.sigmoid(budget)
    prox = raw * vh.norm(dim=-1) * wk.norm(dim=-1)
    clipped = prox > 1
    assert clipped.any()
    torch.testing.assert_close((a * vh.norm(dim=-1) * wk.norm(dim=-1))[clipped],
                               torch.ones(int(clipped.sum())))
    torch.testing.assert_close(a[~clipped], raw[~clipped])


def test_residual_write_key_is_orthogonal():
    # scripts/sgsa_sanity_checks.py:72-76
    g = torch.Generator().manual_seed(4)
    kh, k = torch.randn(2, 6, 3, 8, generator=g), torch.randn(2, 6, 3, 8, generator=g)
    wk = O.write_key(kh, k, "residual")
    assert (wk * k).sum(-1).abs().mean() < 1e-5


def test_kv_reuse_causal_offset_and_probs():
    g = torch.Generator().manual_seed(5)
    B, H, Q, K, D = 1, 2, 3, 8, 4
    qh = torch.randn(B, H, Q, D, generator=g)
    kh = torch.randn(B, H, K, D, generator=g)
    vh = torch.randn(B, H, K, D, generator=g)
    out, idx, p = O.topk_kv_reuse_attention(qh, kh, vh, 4)
    for r in range(Q):
        pos = K - Q + r
        s = (qh[0, 0, r] @ kh[0, 0].T) * (1.0 / math.sqrt(D))
        s[pos + 1:] = torch.finfo(torch.float32).min
        _, bi = _brute_topk(s.tolist(), 4)
        assert idx[0, 0, r].tolist() == bi
    torch.testing.assert_close(p.sum(-1), torch.ones(B, H, Q))


# ---------------------------------------------------------------- padding masks

def _padding_mask(B, T):
    # batch 0 all real tokens, batch 1 left-padded, batch 2 right-padded with a hole
    am = torch.ones(B, T, dtype=torch.bool)
    am[1, :4] = False
    am[2, T - 4:] = False
    am[2, 3] = False
    return am


def test_masked_topk_padding_by_loops():
    # _masked_topk (modeling_sgsa.py:144-165) restated per row: invalid scores are
    # finfo.min, k_q = min(topk, max(valid count over (B,H), 1)), ties to the lowest index
    g = torch.Generator().manual_seed(11)
    B, H, T, k = 3, 2, 14, 5
    s = torch.randn(B, H, T, T, generator=g)
    am = _padding_mask(B, T)
    pos = torch.arange(T)
    valid = ((pos[None, :] <= pos[:, None])[None, None] & am[:, None, None, :] & am[:, None, :, None]).expand(B, H, T, T)
    vals, idx, ok = O.masked_topk(s, valid, k)
    fmin = torch.finfo(torch.float32).min
    for t in range(T):
        vc = max(sum(bool(valid[b, h, t, j]) for j in range(T)) for b in range(B) for h in range(H))
        kq = min(k, max(vc, 1))
        for b in range(B):
            for h in range(H):
                row = [s[b, h, t, j].item() if valid[b, h, t, j] else fmin for j in range(T)]
                bv, bi = _brute_topk(row, kq)
                assert idx[b, h, t, :kq].tolist() == bi
                assert vals[b, h, t, :kq].tolist() == bv
                assert ok[b, h, t, :kq].tolist() == [bool(valid[b, h, t, j]) for j in bi]
                assert idx[b, h, t, kq:].tolist() == [0] * (k - kq)
                assert vals[b, h, t, kq:].tolist() == [fmin] * (k - kq)
                assert not ok[b, h, t, kq:].any()
    # a padded query row has no valid slot; a row with fewer valid keys than
    # k_q fills the rest with its lowest-index invalid keys
    assert not ok[1, :, 2].any() and idx[1, 0, 2, :min(k, 3)].tolist() == list(range(min(k, 3)))


def test_retrieval_with_padding_by_loops():
    # float32 inputs: the reference's softmax(scores.float()) turns a float64
    # finfo.min into -inf, and a row of them into NaN weights
    g = torch.Generator().manual_seed(12)
    B, T, H, D, k = 3, 11, 2, 4, 3
    q, kk, v = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    am = _padding_mask(B, T)
    ret = O.token_topk_retrieval(q, kk, v, k, attention_mask=am, block_rows=4)
    fmin = torch.finfo(torch.float32).min
    for t in range(T):
        ok = lambda b, j: j <= t and bool(am[b, j]) and bool(am[b, t])
        kq = min(k, max(1, max(sum(ok(b, j) for j in range(T)) for b in range(B))))
        for b in range(B):
            for h in range(H):
                row = [sum(q[b, t, h, d].item() * kk[b, j, h, d].item() for d in range(D)) / math.sqrt(D)
                       if ok(b, j) else fmin for j in range(T)]
                bv, bi = _brute_topk(row, kq)
                assert ret["indices"][b, h, t, :kq].tolist() == bi
                m = max(bv)
                e = [math.exp(x - m) for x in bv]
                w = [e[i] / sum(e) * (1.0 if ok(b, bi[i]) else 0.0) for i in range(kq)]
                w = [x / max(sum(w), 1e-6) for x in w]
                torch.testing.assert_close(ret["weights"][b, h, t, :kq], torch.tensor(w, dtype=torch.float32))
                exp_k = sum(w[i] * kk[b, bi[i], h].double() for i in range(kq))
                torch.testing.assert_close(ret["k_hat"][b, t, h], exp_k.float())
                if not am[b, t]:
                    assert ret["k_hat"][b, t, h].abs().max() == 0 and ret["v_hat"][b, t, h].abs().max() == 0


def test_kv_reuse_padding_by_loops():
    # TopKSparseKVReuseAttention (hybrid_dense_delta_topk.py:343-356) with _merge_masks
    # (:153-175): a query whose visible keys are all padding averages the
    # lowest-index keys (equal finfo.min scores, fp32 softmax)
    g = torch.Generator().manual_seed(13)
    B, H, Q, K, D, k = 2, 2, 4, 9, 4, 3
    qh, kh, vh = (torch.randn(B, H, n, D, generator=g) for n in (Q, K, K))
    am = torch.ones(B, K, dtype=torch.bool)
    am[0, :6] = False   # query 0 of batch 0 sits at position 5: nothing visible
    am[1, 7] = False
    out, idx, p = O.topk_kv_reuse_attention(qh, kh, vh, k, attention_mask=am)
    fmin = torch.finfo(torch.float32).min
    for b in range(B):
        for h in range(H):
            for r in range(Q):
                pos = K - Q + r
                s = [(qh[b, h, r].double() @ kh[b, h, j].double()).item() / math.sqrt(D)
                     if (j <= pos and am[b, j]) else fmin for j in range(K)]
                bv, bi = _brute_topk(s, k)
                assert idx[b, h, r].tolist() == bi
                m = max(bv)
                e = [math.exp(x - m) for x in bv]
                pw = [x / sum(e) for x in e]
                torch.testing.assert_close(p[b, h, r], torch.tensor(pw, dtype=torch.float32))
                torch.testing.assert_close(out[b, h, r], sum(pw[i] * vh[b, h, bi[i]] for i in range(k)))
    assert idx[0, 0, 0].tolist() == [0, 1, 2]
    torch.testing.assert_close(p[0, 0, 0], torch.full((k,), 1.0 / k))


def test_diagnostics_by_explicit_loops():
    # _diagnostics (modeling_sgsa.py:361-405): max weight, entropy, and the distance
    # statistics over every slot, padded ones (index 0) included, with avg_distance
    # divided by the largest index + 1 over the whole tensor
    g = torch.Generator().manual_seed(14)
    B, H, T, k, D = 2, 2, 9, 4, 5
    lw, ss, eps = 2, 1, 1e-6
    sc = torch.randn(B, H, T, k, generator=g, dtype=torch.float64)
    idx = torch.randint(0, T, (B, H, T, k), generator=g)
    w = torch.rand(B, H, T, k, generator=g, dtype=torch.float64)
    w[0, 0, 3] = 0.0
    kh = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    key = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    d = O.retrieval_diagnostics(sc, w, idx, kh, key, local_window=lw, sink_size=ss, eps=eps)
    imax = int(idx.max())
    for b in range(B):
        for h in range(H):
            for t in range(T):
                ws = w[b, h, t].tolist()
                js = idx[b, h, t].tolist()
                dist = [max(t - j, 0) for j in js]
                assert d["max_confidence"][b, h, t].item() == max(ws)
                ent = -sum(max(x, eps) * math.log(max(x, eps)) for x in ws)
                assert abs(d["entropy"][b, h, t].item() - ent) < 1e-12
                # the reference takes these means in float32 (dist.float().mean)
                assert abs(d["avg_distance"][b, h, t].item() - sum(dist) / k / (imax + 1)) < 1e-7
                assert d["local_ratio"][b, h, t].item() == sum(x <= lw for x in dist) / k
                assert d["sink_ratio"][b, h, t].item() == sum(j < ss for j in js) / k
                assert d["remote_ratio"][b, h, t].item() == sum(x > lw and j >= ss for x, j in zip(dist, js)) / k
                assert abs(d["score_margin"][b, h, t].item() - (sc[b, h, t, 0] - sc[b, h, t, 1]).item()) < 1e-12


def test_make_inputs_shapes_and_rounding():
    x = O.make_inputs(1, 300, 2, 8, dtype=torch.bfloat16, heavy_tail=True)
    assert x["q"].dtype == torch.bfloat16 and x["q_f32"].dtype == torch.float32
    assert torch.equal(x["q"].float(), x["q_f32"])
    n = (x["k_ret_f32"].norm(dim=-1) > 4).sum()
    assert int(n) == 2 * round(0.01 * 300) and int(n) > 0


# --- the causal LM around the layer ------------------------------------------

def test_rms_norm_and_mlp_by_scalar_loops():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 5, generator=g, dtype=torch.float64)
    w = torch.randn(5, generator=g, dtype=torch.float64)
    y = O.rms_norm(x, w, 1e-6)
    for i in range(3):
        ms = sum(float(x[i, j]) ** 2 for j in range(5)) / 5
        for j in range(5):
            assert abs(float(y[i, j]) - float(x[i, j]) / math.sqrt(ms + 1e-6) * float(w[j])) < 1e-12
    wg, wu, wd = (torch.randn(s, generator=g, dtype=torch.float64) for s in ((4, 5), (4, 5), (5, 4)))
    m = O.gated_mlp(x, wg, wu, wd)
    for i in range(3):
        hid = []
        for r in range(4):
            a = sum(float(wg[r, j]) * float(x[i, j]) for j in range(5))
            b = sum(float(wu[r, j]) * float(x[i, j]) for j in range(5))
            hid.append(a / (1.0 + math.exp(-a)) * b)
        for c in range(5):
            assert abs(float(m[i, c]) - sum(float(wd[c, r]) * hid[r] for r in range(4))) < 1e-12


def _model_params(L, C, H, V, Tmax, I, g):
    P = {"embed_tokens.weight": torch.randn(V, C, generator=g) * 0.5,
         "pos_embed.weight": torch.randn(Tmax, C, generator=g) * 0.5,
         "norm.weight": 1.0 + 0.1 * torch.randn(C, generator=g)}
    for i in range(L):
        p = f"layers.{i}."
        for n in ("q_proj", "k_proj", "v_proj", "q_ret_proj"):
            P[p + n + ".weight"] = torch.randn(C, C, generator=g) / C
        P[p + "o_proj.weight"] = torch.randn(C, C, generator=g) / math.sqrt(C)
        P[p + "sparse_out_proj.weight"] = torch.randn(C, C, generator=g) / math.sqrt(C)
        for n in ("beta_proj", "gamma_proj", "budget_proj"):
            P[p + n + ".weight"] = torch.randn(H, C, generator=g) / math.sqrt(C)
            P[p + n + ".bias"] = torch.randn(H, generator=g)
        P[p + "input_norm.weight"] = 1.0 + 0.1 * torch.randn(C, generator=g)
        P[p + "post_attn_norm.weight"] = 1.0 + 0.1 * torch.randn(C, generator=g)
        P[p + "mlp.gate_proj.weight"] = torch.randn(I, C, generator=g) / math.sqrt(C)
        P[p + "mlp.up_proj.weight"] = torch.randn(I, C, generator=g) / math.sqrt(C)
        P[p + "mlp.down_proj.weight"] = torch.randn(C, I, generator=g) / math.sqrt(I)
    return P


def test_model_without_layers_is_head_of_embeddings():
    g = torch.Generator().manual_seed(7)
    P = _model_params(0, 8, 2, 11, 16, 12, g)
    ids = torch.randint(0, 11, (2, 5), generator=g)
    got = O.sgsa_model_forward(P, ids, num_layers=0, num_heads=2, top_k=3)
    for b in range(2):
        for t in range(5):
            h = P["embed_tokens.weight"][ids[b, t]] + P["pos_embed.weight"][t]
            want = O.rms_norm(h, P["norm.weight"], 1e-6) @ P["embed_tokens.weight"].T   # tied head
            torch.testing.assert_close(got[b, t], want)


def test_model_residual_structure():
    g = torch.Generator().manual_seed(8)
    P = _model_params(1, 8, 2, 11, 16, 12, g)
    ids = torch.randint(0, 11, (1, 7), generator=g)
    head = lambda h: O.rms_norm(h, P["norm.weight"], 1e-6) @ P["embed_tokens.weight"].T
    h0 = P["embed_tokens.weight"][ids] + P["pos_embed.weight"][:7][None]
    # o_proj and the MLP's down projection zeroed: the block is the identity
    Z = dict(P)
    Z["layers.0.o_proj.weight"] = torch.zeros(8, 8)
    Z["layers.0.mlp.down_proj.weight"] = torch.zeros(8, 12)
    torch.testing.assert_close(O.sgsa_model_forward(Z, ids, num_layers=1, num_heads=2, top_k=3), head(h0))
    # only the MLP zeroed: residual + o_proj(layer output) with the block's own projections
    Z = dict(P)
    Z["layers.0.mlp.down_proj.weight"] = torch.zeros(8, 12)
    n = O.rms_norm(h0, P["layers.0.input_norm.weight"], 1e-6)
    pr = lambda name: (n @ P[f"layers.0.{name}.weight"].T).view(1, 7, 2, 4)
    gate = lambda name: n @ P[f"layers.0.{name}.weight"].T + P[f"layers.0.{name}.bias"]
    lay = O.sgsa_layer_forward(pr("q_proj"), pr("k_proj"), pr("v_proj"), pr("q_ret_proj"),
                               torch.sigmoid(gate("beta_proj")).clamp_min(1e-4), torch.sigmoid(gate("gamma_proj")),
                               gate("budget_proj"), 3)
    h1 = h0 + lay["o"].reshape(1, 7, 8) @ P["layers.0.o_proj.weight"].T
    torch.testing.assert_close(O.sgsa_model_forward(Z, ids, num_layers=1, num_heads=2, top_k=3), head(h1))
    # a different q_ret projection changes the retrieval and so the output
    Z2 = dict(Z)
    Z2["layers.0.q_ret_proj.weight"] = P["layers.0.q_proj.weight"] * -1.0
    assert not torch.allclose(O.sgsa_model_forward(Z2, ids, num_layers=1, num_heads=2, top_k=3), head(h1))


def test_layer_block_modes_reduce_to_known_forms():
    # block_token with unit blocks, every block kept: the token_only layer (the same
    # candidates, the same masked top-k); block_only with every block kept: v_hat is causal
    # softmax attention (modeling_sgsa.py:346-359), and the write gate reads it
    g = torch.Generator().manual_seed(11)
    B, T, H, D, k = 2, 13, 2, 8, 4
    q, kk, v, qr = (torch.randn(B, T, H, D, generator=g) for _ in range(4))
    beta, gamma, bud = torch.rand(B, T, H, generator=g), torch.rand(B, T, H, generator=g), torch.randn(B, T, H, generator=g)
    args = (q, kk, v, qr, beta, gamma, bud, k)
    for wm in ("direct", "residual"):
        tok = O.sgsa_layer_forward(*args, write_mode=wm)
        blk = O.sgsa_layer_forward(*args, write_mode=wm, retrieval_mode="block_token", block_size=1, top_blocks=T)
        for name in ("o", "final_state", "write_key", "v_hat", "alpha"):
            torch.testing.assert_close(blk[name], tok[name], msg=name)
    only = O.sgsa_layer_forward(*args, retrieval_mode="block_only", block_size=4, top_blocks=4)
    sdpa = F.scaled_dot_product_attention(qr.transpose(1, 2), kk.transpose(1, 2), v.transpose(1, 2), is_causal=True)
    torch.testing.assert_close(only["v_hat"], sdpa.transpose(1, 2))
    ret = O.block_retrieval(qr, kk, v, k, 4, 4, "block_only")
    want_alpha = O.compute_alpha(ret["diagnostics"]["concentration"], ret["diagnostics"]["novelty"], bud,
                                 ret["k_hat"], ret["v_hat"])
    torch.testing.assert_close(only["alpha"], want_alpha)


def test_layer_write_mode_none_drops_the_sparse_write():
    # write_mode "none": the state update without the sparse write equals the direct mode
    # with alpha forced to 0; alpha itself is still the direct mode's (reported, not applied)
    g = torch.Generator().manual_seed(12)
    B, T, H, D, k = 1, 11, 2, 8, 3
    q, kk, v, qr = (torch.randn(B, T, H, D, generator=g) for _ in range(4))
    beta, gamma, bud = torch.rand(B, T, H, generator=g), torch.rand(B, T, H, generator=g), torch.randn(B, T, H, generator=g)
    none = O.sgsa_layer_forward(q, kk, v, qr, beta, gamma, bud, k, write_mode="none")
    direct = O.sgsa_layer_forward(q, kk, v, qr, beta, gamma, bud, k, write_mode="direct")
    zero = O.sgsa_layer_forward(q, kk, v, qr, beta, gamma, bud, k, write_mode="direct", alpha_max=0.0)
    torch.testing.assert_close(none["o"], zero["o"])
    torch.testing.assert_close(none["final_state"], zero["final_state"])
    torch.testing.assert_close(none["alpha"], direct["alpha"])
    assert (direct["alpha"] > 0).any() and not torch.allclose(none["o"], direct["o"])


def test_model_block_token_with_unit_blocks_is_token_only():
    g = torch.Generator().manual_seed(13)
    P = _model_params(2, 8, 2, 11, 16, 12, g)
    ids = torch.randint(0, 11, (2, 9), generator=g)
    tok = O.sgsa_model_forward(P, ids, num_layers=2, num_heads=2, top_k=3)
    blk = O.sgsa_model_forward(P, ids, num_layers=2, num_heads=2, top_k=3, retrieval_mode="block_token",
                               block_size=1, top_blocks=9)
    torch.testing.assert_close(blk, tok)
    other = O.sgsa_model_forward(P, ids, num_layers=2, num_heads=2, top_k=3, retrieval_mode="block_token",
                                 block_size=4, top_blocks=1)
    assert not torch.allclose(other, tok)
