"""GPU parity of the recurrent form (K6): fused_recurrent_sgsa / decode steps.

Oracle: oracle/sgsa_oracle.py naive_recurrent_sgsa (fp32 restatement of
modelings/sgsa_ops/naive.py:34-57).  bf16 runs feed the oracle the
bf16-rounded inputs.
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


def _inputs(B, T, H, D, seed, sparse=True, h0=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=g), dim=-1)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gamma = torch.exp(torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g) + 4.0))
    sk = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=g), dim=-1) if sparse else None
    sv = torch.randn(B, T, H, D, generator=g) if sparse else None
    al = 0.25 * torch.rand(B, T, H, generator=g) if sparse else None
    s0 = 0.1 * torch.randn(B, H, D, D, generator=g) if h0 else None
    return q, k, v, beta, gamma, sk, sv, al, s0


@pytest.mark.parametrize("dims,sparse,h0", [
    ((2, 37, 3, 64), True, True),
    ((1, 50, 2, 128), True, False),
    ((2, 23, 2, 40), False, True),
    ((1, 9, 3, 5), True, True),          # the reference's tiny ragged head dim
])
def test_recurrent_fp32_matches_oracle(dev, dims, sparse, h0):
    B, T, H, D = dims
    q, k, v, beta, gamma, sk, sv, al, s0 = _inputs(B, T, H, D, seed=1, sparse=sparse, h0=h0)
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, al, s0, True)
    d = lambda t: None if t is None else t.to(dev)
    o, st = sgsa_amd.fused_recurrent_sgsa(d(q), d(k), d(v), d(beta), d(gamma), d(sk), d(sv), d(al), d(s0),
                                          output_final_state=True)
    torch.cuda.synchronize()
    _close(o, ro, 1e-4, "o")
    _close(st, rs, 1e-4, "final_state")
    assert st.dtype == torch.float32


def test_recurrent_bf16_matches_oracle(dev):
    B, T, H, D = 2, 64, 4, 128
    q, k, v, beta, gamma, sk, sv, al, s0 = _inputs(B, T, H, D, seed=2)
    bf = lambda t: t.to(torch.bfloat16)
    q, k, v, sk, sv = map(bf, (q, k, v, sk, sv))
    f = lambda t: t.float()
    ro, rs = O.naive_recurrent_sgsa(f(q), f(k), f(v), beta, gamma, f(sk), f(sv), al, s0, True)
    d = lambda t: t.to(dev)
    o, st = sgsa_amd.fused_recurrent_sgsa(d(q), d(k), d(v), d(beta), d(gamma), d(sk), d(sv), d(al), d(s0),
                                          output_final_state=True)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16
    _close(o, ro, 2e-2, "o")
    _close(st, rs, 2e-2, "final_state")


def test_decode_steps_equal_one_pass(dev):
    # T single-token calls carrying the state give the one-pass result bit for bit
    B, T, H, D = 2, 20, 3, 128
    q, k, v, beta, gamma, sk, sv, al, s0 = (None if t is None else t.to(dev) for t in _inputs(B, T, H, D, seed=3))
    o1, s1 = sgsa_amd.fused_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, al, s0, output_final_state=True)
    st = s0
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, st = sgsa_amd.fused_recurrent_sgsa(q[:, sl], k[:, sl], v[:, sl], beta[:, sl], gamma[:, sl], sk[:, sl],
                                              sv[:, sl], al[:, sl], st, output_final_state=True)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(outs, 1), o1)
    assert torch.equal(st, s1)


def test_recurrent_agrees_with_chunk_form(dev):
    # the two kernel families compute the same recurrence
    B, T, H, D = 1, 200, 2, 128
    q, k, v, beta, gamma, sk, sv, al, s0 = (None if t is None else t.to(dev) for t in _inputs(B, T, H, D, seed=4))
    o1, s1 = sgsa_amd.fused_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, al, s0, output_final_state=True)
    o2, s2 = sgsa_amd.chunk_sgsa(q, k, v, beta, gamma, sk, sv, al, s0, output_final_state=True)
    torch.cuda.synchronize()
    _close(o1, o2, 1e-4, "o")
    _close(s1, s2, 1e-4, "final_state")


@pytest.mark.parametrize("dtype,tol,D", [(torch.float32, 1e-4, 64), (torch.bfloat16, 2e-2, 128)])
@pytest.mark.parametrize("write_mode", ["direct", "residual"])
def test_decode_steps_match_the_layer_oracle(dev, dtype, tol, D, write_mode):
    # the last 6 tokens generated one at a time (retrieval over the growing cache,
    # gate, recurrent update) reproduce the full-sequence layer at those positions
    B, T, H, k, n = 2, 200, 2, 32, 6
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=8)
    args = lambda sl: (x["q_f32"][:, sl], x["k_f32"][:, sl], x["v_f32"][:, sl], x["q_f32"][:, sl],
                       x["beta"][:, sl], x["gamma"][:, sl], x["budget"][:, sl])
    full = O.sgsa_layer_forward(*args(slice(0, T)), k, write_mode=write_mode)
    prev = O.sgsa_layer_forward(*args(slice(0, T - n)), k, write_mode=write_mode)
    st = prev["final_state"].to(dev)
    d = lambda t: t.to(dev)
    for t in range(T - n, T):
        sl = slice(t, t + 1)
        o, st = sgsa_amd.sgsa_decode_step(d(x["q"][:, sl]), d(x["k"][:, sl]), d(x["v"][:, sl]), d(x["q"][:, sl]),
                                          d(x["beta"][:, sl]), d(x["gamma"][:, sl]), d(x["budget"][:, sl]),
                                          d(x["k"][:, :t + 1]), d(x["v"][:, :t + 1]), st, k, write_mode=write_mode)
        torch.cuda.synchronize()
        _close(o, full["o"][:, sl], tol, f"o[{t}]")
    _close(st, full["final_state"], tol, "final_state")


@pytest.mark.parametrize("dtype,tol,D", [(torch.float32, 1e-4, 64), (torch.bfloat16, 2e-2, 128)])
def test_decode_with_topk_reuse_matches_the_oracle(dev, dtype, tol, D):
    # 8 generated tokens: steps 0 and 4 select their top-k over the cache, steps
    # 1-3 and 5-7 re-score the last selection (sgsa_score_at) -- against the
    # oracle's decode step on the same schedule
    B, T, H, k, n = 2, 200, 2, 32, 8
    x = O.make_inputs(B, T, H, D, dtype=dtype, seed=11)
    args = lambda sl: (x["q_f32"][:, sl], x["k_f32"][:, sl], x["v_f32"][:, sl], x["q_f32"][:, sl],
                       x["beta"][:, sl], x["gamma"][:, sl], x["budget"][:, sl])
    st_ref = O.sgsa_layer_forward(*args(slice(0, T - n)), k)["final_state"]
    st = st_ref.to(dev)
    d = lambda t: t.to(dev)
    cand = cand_ref = None
    for s, t in enumerate(range(T - n, T)):
        sl = slice(t, t + 1)
        reuse = s % 4 != 0
        o_ref, st_ref, c_ref = O.sgsa_decode_step(*args(sl), x["k_f32"][:, :t + 1], x["v_f32"][:, :t + 1], st_ref, k,
                                                  candidates=cand_ref if reuse else None)
        cand_ref = c_ref
        o, st, c = sgsa_amd.sgsa_decode_step(d(x["q"][:, sl]), d(x["k"][:, sl]), d(x["v"][:, sl]), d(x["q"][:, sl]),
                                             d(x["beta"][:, sl]), d(x["gamma"][:, sl]), d(x["budget"][:, sl]),
                                             d(x["k"][:, :t + 1]), d(x["v"][:, :t + 1]), st, k,
                                             candidates=cand if reuse else None, return_candidates=True)
        cand = c
        torch.cuda.synchronize()
        _close(o, o_ref, tol, f"o[{t}] ({'reuse' if reuse else 'select'})")
    _close(st, st_ref, tol, "final_state")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,n", [(96, 40), (128, 300)])
def test_score_at_is_the_dot_product(dev, dtype, D, n):
    # sgsa_score_at: q . k[idx] / sqrt(D) at given keys, slots past the count untouched
    # (bf16 at D = 128 takes the 16-byte-load path, 16 keys in flight per wave)
    B, Tq, Tk, H = 2, 3, 300, 2
    g = torch.Generator().manual_seed(12)
    q = torch.randn(B, Tq, H, D, generator=g).to(dtype)
    kk = torch.randn(B, Tk, H, D, generator=g).to(dtype)
    idx = torch.randint(0, Tk, (B, H, Tq, n), generator=g, dtype=torch.int32)
    cnt = torch.randint(1, n + 1, (B, H, Tq), generator=g, dtype=torch.int32)
    out = torch.full((B, H, Tq, n), 123.0, device=dev)
    from sgsa_amd import _abi
    qd, kd, idxd, cntd = q.to(dev).contiguous(), kk.to(dev).contiguous(), idx.to(dev), cnt.to(dev)   # kept alive
    _abi.check(_abi.lib().sgsa_score_at(_abi.dtype_code(dtype), B, Tq, Tk, H, D, n, float(D) ** 0.5, 0,
                                        _abi.ptr(qd), _abi.ptr(kd), _abi.ptr(idxd), _abi.ptr(cntd), _abi.ptr(out),
                                        _abi.stream_of(out)))
    torch.cuda.synchronize()
    qf, kf = q.double(), kk.double()
    ref = torch.einsum("bqhd,bhqnd->bhqn", qf, kf.permute(0, 2, 1, 3)[:, :, None].expand(-1, -1, Tq, -1, -1)
                       .gather(3, idx.long()[..., None].expand(-1, -1, -1, -1, D))) / D ** 0.5
    live = torch.arange(n)[None, None, None, :] < cnt[..., None]
    got = out.cpu().double()
    assert torch.allclose(got[live], ref[live], atol=1e-4, rtol=1e-4)
    assert (got[~live] == 123.0).all(), "slots past the count were written"
