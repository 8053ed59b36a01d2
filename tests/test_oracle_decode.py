"""CPU checks of the oracle's decode step with top-k reuse (oracle.sgsa_decode_step).

* Without candidates, decode steps reproduce the full-sequence layer oracle
  (sgsa_layer_forward: one blocked retrieval over all rows, then the token
  recurrence) at those positions, and chain to its final state.
* Re-scoring a step's own candidates reproduces the step exactly.
* Candidates selected at an earlier step give exactly the selecting step's
  result when they are still the exact top-k: the later steps retrieve with
  the same query, and the tokens appended since then have zero keys (score 0,
  below every row's k-th score), so the selection would not change.
"""

import torch

from oracle import sgsa_oracle as O


def _args(x, sl):
    return (x["q_f32"][:, sl], x["k_f32"][:, sl], x["v_f32"][:, sl], x["q_f32"][:, sl],
            x["beta"][:, sl], x["gamma"][:, sl], x["budget"][:, sl])


def test_decode_steps_reproduce_the_layer():
    B, T, H, D, k, n = 2, 120, 2, 16, 24, 6
    x = O.make_inputs(B, T, H, D, dtype=torch.float32, seed=8)
    full = O.sgsa_layer_forward(*_args(x, slice(0, T)), k)
    st = O.sgsa_layer_forward(*_args(x, slice(0, T - n)), k)["final_state"]
    for t in range(T - n, T):
        sl = slice(t, t + 1)
        o, st, _ = O.sgsa_decode_step(*_args(x, sl), x["k_f32"][:, :t + 1], x["v_f32"][:, :t + 1], st, k)
        torch.testing.assert_close(o, full["o"][:, sl], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(st, full["final_state"], atol=1e-5, rtol=1e-5)


def test_reusing_a_steps_own_candidates_is_the_step():
    B, T, H, D, k = 2, 90, 3, 16, 20
    x = O.make_inputs(B, T, H, D, dtype=torch.float32, seed=9)
    st0 = O.sgsa_layer_forward(*_args(x, slice(0, T - 1)), k)["final_state"]
    sl = slice(T - 1, T)
    o, st, cand = O.sgsa_decode_step(*_args(x, sl), x["k_f32"], x["v_f32"], st0, k, write_mode="residual")
    o2, st2, _ = O.sgsa_decode_step(*_args(x, sl), x["k_f32"], x["v_f32"], st0, k, write_mode="residual",
                                    candidates=cand)
    assert torch.equal(o, o2) and torch.equal(st, st2)


def test_earlier_candidates_that_are_still_the_top_k():
    B, T, H, D, k, n = 1, 100, 2, 16, 20, 3
    x = O.make_inputs(B, T, H, D, dtype=torch.float32, seed=10)
    for name in ("k", "k_f32"):   # the last n tokens write and are retrieved with zero keys
        x[name] = x[name].clone()
        x[name][:, T - n:] = 0.0
    st = O.sgsa_layer_forward(*_args(x, slice(0, T - n)), k)["final_state"]
    t0 = T - n - 1
    _, _, cand = O.sgsa_decode_step(*_args(x, slice(t0, t0 + 1)), x["k_f32"][:, :t0 + 1], x["v_f32"][:, :t0 + 1],
                                    O.sgsa_layer_forward(*_args(x, slice(0, t0)), k)["final_state"], k)
    q_ret = x["q_f32"][:, t0:t0 + 1]   # the selecting step's retrieval query
    qk = torch.einsum("bhd,bthd->bht", q_ret[:, 0], x["k_f32"][:, :t0 + 1])
    assert (torch.topk(qk, k, dim=-1).values[..., -1] > 0).all(), "k-th score must be above the new keys' 0"
    for t in range(T - n, T):
        sl = slice(t, t + 1)
        kc, vc = x["k_f32"][:, :t + 1], x["v_f32"][:, :t + 1]
        a = list(_args(x, sl))
        a[3] = q_ret
        o_sel, st_sel, _ = O.sgsa_decode_step(*a, kc, vc, st, k)
        o_re, st_re, _ = O.sgsa_decode_step(*a, kc, vc, st, k, candidates=cand)
        torch.testing.assert_close(o_re, o_sel, atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(st_re, st_sel, atol=1e-6, rtol=1e-6)
        st = st_sel
