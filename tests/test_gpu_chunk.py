"""GPU parity of chunk_sgsa (K3/K4/K5) against the fp32 recurrent oracle.

Tolerances: 1e-4 relative for fp32 inputs, 2e-2 relative
for bf16 inputs, on outputs and final states; "relative" is taken against the
largest magnitude of the reference tensor, elementwise.
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)


def _close(got, ref, rel):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    scale = ref.abs().max().clamp_min(1e-12)
    err = (got - ref).abs().max() / scale
    assert torch.isfinite(got).all(), "non-finite output"
    assert err <= rel, f"max error {err:.3e} (relative to max |ref| {scale:.3e}) exceeds {rel:.1e}"


def _raw_inputs(seed, B, T, H, D):
    # the distribution of the reference's own test (tests/test_sgsa_core.py:11-22)
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    q, k, v, sk, sv = (r(B, T, H, D) for _ in range(5))
    beta = torch.sigmoid(r(B, T, H))
    gamma = torch.sigmoid(r(B, T, H))
    alpha = 0.25 * torch.sigmoid(r(B, T, H))
    return q, k, v, sk, sv, beta, gamma, alpha


def _norm_inputs(seed, B, T, H, D):
    x = O.make_inputs(B, T, H, D, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    sk = torch.randn(B, T, H, D, generator=g)
    sk = sk / sk.norm(dim=-1, keepdim=True)
    sv = torch.randn(B, T, H, D, generator=g)
    alpha = 0.25 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    return x["q"], x["k"], x["v"], sk, sv, x["beta"], x["gamma"], alpha


def _run(dev, dtype, q, k, v, sk, sv, beta, gamma, alpha, h0, sparse):
    c = lambda t: None if t is None else t.to(dev, dtype)
    cf = lambda t: None if t is None else t.to(dev, torch.float32)
    kw = dict(sparse_k=c(sk), sparse_v=c(sv), alpha=cf(alpha)) if sparse else {}
    out, st = sgsa_amd.chunk_sgsa(c(q), c(k), c(v), cf(beta), cf(gamma), initial_state=cf(h0),
                                  output_final_state=True, **kw)
    torch.cuda.synchronize()
    return out, st


@pytest.mark.parametrize("sparse", [False, True])
def test_chunk_reference_shape_fp32(dev, sparse):
    # B=2 T=9 H=3 D=5: the reference test's ragged shape
    q, k, v, sk, sv, beta, gamma, alpha = _raw_inputs(0, 2, 9, 3, 5)
    kw = dict(sparse_k=sk, sparse_v=sv, alpha=alpha) if sparse else {}
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, output_final_state=True, **kw)
    out, st = _run(dev, torch.float32, q, k, v, sk, sv, beta, gamma, alpha, None, sparse)
    _close(out, ro, 1e-4)
    _close(st, rs, 1e-4)


@pytest.mark.parametrize("dims", [(1, 512, 4, 64), (2, 200, 2, 128), (1, 64, 1, 128), (1, 65, 2, 96)])
@pytest.mark.parametrize("sparse", [False, True])
def test_chunk_fp32_with_initial_state(dev, dims, sparse):
    B, T, H, D = dims
    q, k, v, sk, sv, beta, gamma, alpha = _norm_inputs(1, B, T, H, D)
    h0 = 0.1 * torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(5))
    kw = dict(sparse_k=sk, sparse_v=sv, alpha=alpha) if sparse else {}
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, initial_state=h0, output_final_state=True, **kw)
    out, st = _run(dev, torch.float32, q, k, v, sk, sv, beta, gamma, alpha, h0, sparse)
    _close(out, ro, 1e-4)
    _close(st, rs, 1e-4)


@pytest.mark.parametrize("dims", [(1, 1024, 2, 128), (2, 300, 3, 64)])
def test_chunk_bf16_matches_fp32_recurrent(dev, dims):
    B, T, H, D = dims
    q, k, v, sk, sv, beta, gamma, alpha = _norm_inputs(2, B, T, H, D)
    rb = lambda t: t.to(torch.bfloat16).float()
    q, k, v, sk, sv = map(rb, (q, k, v, sk, sv))
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, sk, sv, alpha, None, True)
    out, st = _run(dev, torch.bfloat16, q, k, v, sk, sv, beta, gamma, alpha, None, True)
    assert out.dtype == torch.bfloat16 and st.dtype == torch.float32
    _close(out, ro, 2e-2)
    _close(st, rs, 2e-2)


def test_chunk_state_continuation(dev):
    B, T, H, D = 1, 256, 2, 128
    q, k, v, sk, sv, beta, gamma, alpha = _norm_inputs(3, B, T, H, D)
    full_o, full_s = _run(dev, torch.float32, q, k, v, sk, sv, beta, gamma, alpha, None, True)
    s = 100   # split inside a chunk
    a_o, a_s = _run(dev, torch.float32, q[:, :s], k[:, :s], v[:, :s], sk[:, :s], sv[:, :s], beta[:, :s],
                    gamma[:, :s], alpha[:, :s], None, True)
    b_o, b_s = _run(dev, torch.float32, q[:, s:], k[:, s:], v[:, s:], sk[:, s:], sv[:, s:], beta[:, s:],
                    gamma[:, s:], alpha[:, s:], a_s.cpu(), True)
    _close(torch.cat([a_o, b_o], 1), full_o, 1e-4)
    _close(b_s, full_s, 1e-4)


def test_chunk_deterministic(dev):
    q, k, v, sk, sv, beta, gamma, alpha = _norm_inputs(4, 1, 300, 2, 128)
    o1, s1 = _run(dev, torch.bfloat16, q, k, v, sk, sv, beta, gamma, alpha, None, True)
    o2, s2 = _run(dev, torch.bfloat16, q, k, v, sk, sv, beta, gamma, alpha, None, True)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("dims", [(1, 333, 2, 128), (2, 130, 2, 96), (1, 64, 3, 40)])
@pytest.mark.parametrize("sparse", [False, True])
def test_chunk_bf16_initial_state_and_shapes(dev, dims, sparse):
    B, T, H, D = dims
    q, k, v, sk, sv, beta, gamma, alpha = _norm_inputs(6, B, T, H, D)
    rb = lambda t: t.to(torch.bfloat16).float()
    q, k, v, sk, sv = map(rb, (q, k, v, sk, sv))
    h0 = 0.1 * torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(8))
    kw = dict(sparse_k=sk, sparse_v=sv, alpha=alpha) if sparse else {}
    ro, rs = O.naive_recurrent_sgsa(q, k, v, beta, gamma, initial_state=h0, output_final_state=True, **kw)
    out, st = _run(dev, torch.bfloat16, q, k, v, sk, sv, beta, gamma, alpha, h0, sparse)
    _close(out, ro, 2e-2)
    _close(st, rs, 2e-2)
