"""GPU: the model shells' RMSNorm kernel (sgsa_rms_norm through sgsa_amd.model.RMSNorm)
against the torch fp32 form of the same expression, x * rsqrt(mean(x^2) + eps) * w,
stored in x's dtype (hybrid_dense_delta_topk.py:94-103 evaluated in fp32).  fp32
within 1e-5; bf16 within one bf16 rounding (2e-2 relative)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)
from sgsa_amd.model import RMSNorm  # noqa: E402


@pytest.mark.parametrize("dt,wdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                    (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("shape", [(8, 1, 2048), (3, 77, 1000), (1, 5, 37)])
def test_rms_norm_matches_torch(dev, dt, wdt, shape):
    g = torch.Generator().manual_seed(shape[-1])
    x = (3.0 * torch.randn(*shape, generator=g)).to(dt)
    norm = RMSNorm(shape[-1], 1e-6)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(shape[-1], generator=g))
    norm = norm.to(device=dev, dtype=wdt)
    with torch.no_grad():   # the HIP launch (under autograd the torch form runs)
        y = norm(x.to(dev))
    torch.cuda.synchronize()
    xf = x.float()
    want = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * norm.weight.detach().float().cpu()
    assert y.dtype == dt and y.shape == x.shape
    tol = 1e-5 if dt == torch.float32 else 2e-2
    torch.testing.assert_close(y.float().cpu(), want.to(dt).float(), atol=tol, rtol=tol)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_rms_norm_under_autograd(dev, dt):
    # gradients reach the input and the norm weight, and the forward equals the HIP launch
    g = torch.Generator().manual_seed(3)
    x = (2.0 * torch.randn(4, 9, 256, generator=g)).to(dev, dt).requires_grad_(True)
    norm = RMSNorm(256, 1e-6).to(dev)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(256, generator=g))
        y_hip = norm(x)
    y = norm(x)
    assert y.grad_fn is not None
    torch.testing.assert_close(y.float(), y_hip.float(), atol=1e-5 if dt == torch.float32 else 2e-2, rtol=1e-5)
    gy = torch.randn(y.shape, generator=g).to(dev, dt)
    y.backward(gy)
    assert norm.weight.grad is not None and x.grad is not None
    xr = x.detach().double().cpu().requires_grad_(True)
    wr = norm.weight.detach().double().cpu().requires_grad_(True)
    yr = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6) * wr
    yr.backward(gy.double().cpu())
    tol = 1e-4 if dt == torch.float32 else 3e-2
    torch.testing.assert_close(norm.weight.grad.double().cpu(), wr.grad, atol=tol * wr.grad.abs().max().item(), rtol=tol)
    torch.testing.assert_close(x.grad.double().cpu(), xr.grad, atol=tol * xr.grad.abs().max().item(), rtol=tol)


def test_rms_norm_rejects_cpu():
    with pytest.raises(ValueError):
        RMSNorm(16, 1e-6)(torch.ones(2, 16))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_layer_gates_match_torch(dev, dt):
    # logits laid out as a fused projection row: [other 40 | beta H | gamma H | budget H | 5 more]
    from sgsa_amd import _abi
    B, T, H = 3, 7, 16
    g = torch.Generator().manual_seed(4)
    y = (4.0 * torch.randn(B, T, 40 + 3 * H + 5, generator=g)).to(dt).to(dev)
    bl, gl, ul = y[..., 40:40 + H], y[..., 40 + H:40 + 2 * H], y[..., 40 + 2 * H:40 + 3 * H]
    out = [torch.empty(B, T, H, device=dev) for _ in range(3)]
    _abi.check(_abi.lib().sgsa_layer_gates(_abi.dtype_code(dt), B * T, H, _abi.ptr(bl), bl.stride(-2),
                                           *(_abi.ptr(o) for o in out), _abi.stream_of(y)))
    torch.cuda.synchronize()
    want = (torch.sigmoid(bl.float()).clamp_min(1e-4), torch.sigmoid(gl.float()), ul.float())
    for name, o, w in zip(("beta", "gamma", "budget"), out, want):
        torch.testing.assert_close(o, w, atol=1e-6, rtol=1e-5, msg=name)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,pos0", [(1, 40), (9, 0), (300, 17)])
def test_rope_qk_equals_torch_rope(dev, dt, T, pos0):
    # the fused projection row [q (Hq heads) | k (Hk heads) | v ...]; the kernel equals apply_rope bit for bit
    from sgsa_amd import _abi
    from sgsa_amd.hybrid import apply_rope, rope_tables
    B, Hq, Hk, D = 2, 8, 2, 64
    g = torch.Generator().manual_seed(T)
    y = torch.randn(B, T, (Hq + 2 * Hk) * D, generator=g).to(dt).to(dev)
    cos, sin = rope_tables(pos0 + T + 5, D, 10000.0, dev)
    q = torch.empty(B, Hq, T, D, device=dev, dtype=dt)
    k = torch.empty(B, Hk, T, D, device=dev, dtype=dt)
    _abi.check(_abi.lib().sgsa_rope_qk(_abi.dtype_code(dt), B, T, Hq, Hk, D, pos0, cos.shape[0], _abi.ptr(y),
                                       y.stride(-2), _abi.ptr(cos), _abi.ptr(sin), _abi.ptr(q), _abi.ptr(k),
                                       _abi.stream_of(y)))
    qr = y[..., :Hq * D].reshape(B, T, Hq, D).transpose(1, 2)
    kr = y[..., Hq * D:(Hq + Hk) * D].reshape(B, T, Hk, D).transpose(1, 2)
    c, s = cos[pos0:pos0 + T], sin[pos0:pos0 + T]
    torch.cuda.synchronize()
    assert torch.equal(q, apply_rope(qr, c, s)) and torch.equal(k, apply_rope(kr, c, s))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,D,pad", [(8, 4, 64, 0), (3, 5, 48, 7), (1, 2, 128, 0)])
def test_decode_split_equals_views_and_gates(dev, dt, B, H, D, pad):
    # one decode token per sequence: the fused projection row [q | k | v | q_ret | b | g | u | pad]
    # split into contiguous q, k, v, q_ret (bit for bit), the gates of sgsa_layer_gates' formula,
    # and k, v appended at cache row pos with every other cache row untouched
    from sgsa_amd import _abi
    HD = H * D
    X = 4 * HD + 3 * H + pad
    g = torch.Generator().manual_seed(B * 100 + H)
    y = (3.0 * torch.randn(B, 1, X, generator=g)).to(dt).to(dev)
    Tc, pos = 11, 6
    kc = torch.randn(B, Tc, H, D, generator=g).to(dt).to(dev)
    vc = torch.randn(B, Tc, H, D, generator=g).to(dt).to(dev)
    kc0, vc0 = kc.clone(), vc.clone()
    q, k, v, qr = (torch.empty(B, 1, H, D, device=dev, dtype=dt) for _ in range(4))
    beta, gamma, budget = (torch.empty(B, 1, H, device=dev) for _ in range(3))
    _abi.check(_abi.lib().sgsa_decode_split(
        _abi.dtype_code(dt), B, H, D, _abi.ptr(y), y.stride(0), _abi.ptr(q), _abi.ptr(k), _abi.ptr(v), _abi.ptr(qr),
        _abi.ptr(beta), _abi.ptr(gamma), _abi.ptr(budget), _abi.ptr(kc), _abi.ptr(vc), Tc, pos, _abi.stream_of(y)))
    torch.cuda.synchronize()
    parts = torch.split(y, [HD, HD, HD, HD, H, H, H, pad], dim=-1)
    for name, got, want in zip(("q", "k", "v", "q_ret"), (q, k, v, qr), parts[:4]):
        assert torch.equal(got, want.reshape(B, 1, H, D)), name
    want = (torch.sigmoid(parts[4].float()).clamp_min(1e-4), torch.sigmoid(parts[5].float()), parts[6].float())
    for name, o, w in zip(("beta", "gamma", "budget"), (beta, gamma, budget), want):
        torch.testing.assert_close(o, w, atol=1e-6, rtol=1e-5, msg=name)
    kw, vw = kc0.clone(), vc0.clone()
    kw[:, pos] = parts[1].reshape(B, H, D)
    vw[:, pos] = parts[2].reshape(B, H, D)
    assert torch.equal(kc, kw) and torch.equal(vc, vw)
    # without caches nothing else is written; a pos outside the cache is an error
    _abi.check(_abi.lib().sgsa_decode_split(
        _abi.dtype_code(dt), B, H, D, _abi.ptr(y), y.stride(0), _abi.ptr(q), _abi.ptr(k), _abi.ptr(v), _abi.ptr(qr),
        _abi.ptr(beta), _abi.ptr(gamma), _abi.ptr(budget), None, None, 0, 0, _abi.stream_of(y)))
    rc = _abi.lib().sgsa_decode_split(
        _abi.dtype_code(dt), B, H, D, _abi.ptr(y), y.stride(0), _abi.ptr(q), _abi.ptr(k), _abi.ptr(v), _abi.ptr(qr),
        _abi.ptr(beta), _abi.ptr(gamma), _abi.ptr(budget), _abi.ptr(kc), _abi.ptr(vc), Tc, Tc, _abi.stream_of(y))
    assert rc != 0
    torch.cuda.synchronize()
    assert torch.equal(kc, kw) and torch.equal(vc, vw)


@pytest.mark.parametrize("dt,wdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                    (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("shape", [(8, 1, 2048), (3, 77, 1000)])
def test_add_rms_norm_equals_the_two_steps(dev, dt, wdt, shape):
    # sgsa_add_rms_norm (RMSNorm.add_forward without autograd) = (a + b, RMSNorm(a + b)) bit for bit
    g = torch.Generator().manual_seed(shape[1])
    a = (2.0 * torch.randn(*shape, generator=g)).to(dt).to(dev)
    b = (2.0 * torch.randn(*shape, generator=g)).to(dt).to(dev)
    norm = RMSNorm(shape[-1], 1e-6)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(shape[-1], generator=g))
    norm = norm.to(device=dev, dtype=wdt)
    with torch.no_grad():
        h, y = norm.add_forward(a, b)
        h2 = a + b
        y2 = norm(h2)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(y, y2)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_gated_mlp_silu_mul_equals_torch(dev, dt):
    # GatedMLP without autograd (one sgsa_silu_mul launch on the fused gate | up projection)
    # against silu(gate) * up in torch on the same projection: within one rounding of dt
    from sgsa_amd.model import GatedMLP
    torch.manual_seed(3)
    mlp = GatedMLP(256, 640).to(device=dev, dtype=dt)
    x = torch.randn(4, 3, 256, device=dev).to(dt)
    with torch.no_grad():
        got = mlp(x)
        gate, up = mlp.gate_proj(x), mlp.up_proj(x)
        act = torch.nn.functional.silu(gate) * up
        want = mlp.down_proj(act)
    torch.cuda.synchronize()
    err = ((got.float() - want.float()).abs().max() / want.float().abs().max()).item()
    assert err <= (1e-5 if dt == torch.float32 else 1.6e-2), f"{err:.3e}"


@pytest.mark.parametrize("M", [1, 3, 8, 16])
@pytest.mark.parametrize("N,K,bias", [(16, 64, False), (100, 2048, True), (2096, 2048, False), (48, 5632, True)])
def test_linear_rows_equals_f_linear(dev, M, N, K, bias):
    # sgsa_linear_rows (model.linear_rows at <= 16 bf16 rows) against F.linear in fp32 on the same
    # bf16 operands: within one bf16 rounding of the largest output; x as a strided view of a wider row
    from sgsa_amd.model import linear_rows
    g = torch.Generator().manual_seed(M * 7 + N)
    xw = torch.randn(M, K + 32, generator=g).to(torch.bfloat16).to(dev)
    x = xw[:, 16:16 + K]
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(dev) if bias else None
    with torch.no_grad():
        got = linear_rows(x, w, b)
    want = torch.nn.functional.linear(x.float(), w.float(), None if b is None else b.float())
    torch.cuda.synchronize()
    assert got.shape == (M, N) and got.dtype == torch.bfloat16
    err = ((got.float() - want).abs().max() / want.abs().max()).item()
    assert err <= 8e-3, f"{err:.3e}"


@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N,K,bias", [(16, 64, False), (100, 2048, True), (2096, 2048, False), (2048, 5632, False),
                                      (40, 5632, True)])
def test_linear_rows_tiled_equals_linear_rows(dev, M, N, K, bias):
    # sgsa_linear_rows_tile's layout against a torch permutation of the zero-padded weight
    # ([tiles, 16 rows, K/32 steps, 4 pieces, 8] -> [tiles, steps, pieces, rows, 8]), and
    # sgsa_linear_rows_tiled against sgsa_linear_rows bit for bit
    from sgsa_amd import _abi
    from sgsa_amd.model import linear_rows
    g = torch.Generator().manual_seed(M * 13 + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(dev) if bias else None
    tiles = (N + 15) // 16
    tiled = torch.full((16 * tiles * K,), 7.0, device=dev, dtype=torch.bfloat16)
    lib = _abi.lib()
    _abi.check(lib.sgsa_linear_rows_tile(_abi.SGSA_BF16, N, K, _abi.ptr(w), _abi.ptr(tiled), _abi.stream_of(w)))
    wp = torch.zeros(16 * tiles, K, device=dev, dtype=torch.bfloat16)
    wp[:N] = w
    want_t = wp.view(tiles, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    y = torch.full((M, N), 3.0, device=dev, dtype=torch.bfloat16)
    _abi.check(lib.sgsa_linear_rows_tiled(_abi.SGSA_BF16, M, N, K, _abi.ptr(x), K, _abi.ptr(tiled), _abi.ptr(b),
                                          _abi.ptr(y), N, _abi.stream_of(x)))
    with torch.no_grad():
        want = linear_rows(x, w, b)
    torch.cuda.synchronize()
    assert torch.equal(tiled, want_t)
    assert torch.equal(y, want)
