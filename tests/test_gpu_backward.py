"""GPU: backward of chunk_sgsa and fused_recurrent_sgsa through their autograd
wrappers (HIP forward, native HIP backward sgsa_chunk_bwd in place of the
reference's recompute, modelings/sgsa_ops/chunk_bwd.py:31-77 and
recurrent.py:78-135), against torch autograd through the oracle's token
recurrence (naive.py:34-57) in float64 on the CPU.  float32 inputs: gradients
within 1e-4 of the largest magnitude; bfloat16 inputs: gradients come back in
bfloat16, within 2e-2.  The loss follows the reference's tests
(tests/test_sgsa_core.py:190, :261): out.square().mean() + state.square().mean().
At larger shapes the native backward is compared with the torch recompute of
the same function (sgsa_amd.backward.recompute_grads) on the GPU.
"""

import pytest
import torch

from oracle import sgsa_oracle as O

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)

ORDER = ["q", "k", "v", "beta", "gamma", "sparse_k", "sparse_v", "alpha", "initial_state"]


def _inputs(B, T, H, D, sparse, init, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    nk = lambda t: t / t.norm(dim=-1, keepdim=True)   # unit keys keep the delta rule contractive
    x = dict(q=r(B, T, H, D), k=nk(r(B, T, H, D)), v=r(B, T, H, D),
             beta=torch.sigmoid(r(B, T, H)), gamma=torch.sigmoid(r(B, T, H) + 3.0),
             sparse_k=nk(r(B, T, H, D)), sparse_v=r(B, T, H, D), alpha=0.25 * torch.sigmoid(r(B, T, H)),
             initial_state=0.1 * r(B, H, D, D))
    if not sparse:
        x["sparse_k"] = x["sparse_v"] = x["alpha"] = None
    if not init:
        x["initial_state"] = None
    return x


def _oracle_grads(x):
    leaves = {n: (None if x[n] is None else x[n].clone().requires_grad_(True)) for n in ORDER}
    o, s = O.naive_recurrent_sgsa(**leaves, output_final_state=True)
    (o.square().mean() + s.square().mean()).backward()
    return {n: leaves[n].grad for n in ORDER if leaves[n] is not None}


def _run(fn, x, dev, dt):
    leaves = {}
    for n in ORDER:
        if x[n] is None:
            leaves[n] = None
            continue
        t = x[n].to(dev)
        t = t.to(dt) if n in ("q", "k", "v", "sparse_k", "sparse_v") else t.float()
        leaves[n] = t.requires_grad_(True)
    out, state = fn(**leaves, output_final_state=True)
    (out.float().square().mean() + state.square().mean()).backward()
    return {n: leaves[n].grad for n in ORDER if leaves[n] is not None}


def _compare(got, ref, tol, dt):
    for n, gr in ref.items():
        g = got[n]
        assert g is not None, f"{n}: no gradient"
        want_dt = dt if n in ("q", "k", "v", "sparse_k", "sparse_v") else torch.float32
        assert g.dtype == want_dt, f"{n}: dtype {g.dtype}"
        g = g.double().cpu()
        assert torch.isfinite(g).all(), f"{n}: non-finite gradient"
        err = (g - gr).abs().max() / gr.abs().max().clamp_min(1e-12)
        assert err <= tol, f"{n}: {err:.3e} from the oracle recurrence's autograd"


@pytest.mark.parametrize("op", ["chunk", "recurrent"])
@pytest.mark.parametrize("sparse,init", [(True, True), (True, False), (False, True)])
def test_backward_fp32_matches_oracle_autograd(dev, op, sparse, init):
    x = _inputs(2, 150, 2, 64, sparse, init, seed=11)
    fn = sgsa_amd.chunk_sgsa if op == "chunk" else sgsa_amd.fused_recurrent_sgsa
    got = _run(fn, x, dev, torch.float32)
    _compare(got, _oracle_grads(x), 1e-4, torch.float32)


@pytest.mark.parametrize("op", ["chunk", "recurrent"])
def test_backward_bf16_matches_oracle_autograd(dev, op):
    x = _inputs(1, 200, 2, 128, True, True, seed=12)
    for n in ("q", "k", "v", "sparse_k", "sparse_v"):   # the oracle sees the bf16-rounded inputs
        x[n] = x[n].to(torch.bfloat16).double()
    fn = sgsa_amd.chunk_sgsa if op == "chunk" else sgsa_amd.fused_recurrent_sgsa
    got = _run(fn, x, dev, torch.bfloat16)
    _compare(got, _oracle_grads(x), 2e-2, torch.bfloat16)


def test_backward_only_some_inputs_and_no_final_state(dev):
    # grads only where requested; the output alone drives the objective (no final state)
    x = _inputs(1, 70, 2, 64, True, False, seed=13)
    q = x["q"].float().to(dev).requires_grad_(True)
    beta = x["beta"].float().to(dev).requires_grad_(True)
    rest = {n: x[n].float().to(dev) for n in ("k", "v", "gamma", "sparse_k", "sparse_v", "alpha")}
    out, st = sgsa_amd.chunk_sgsa(q, rest["k"], rest["v"], beta, rest["gamma"], rest["sparse_k"],
                                  rest["sparse_v"], rest["alpha"])
    assert st is None
    out.sum().backward()
    leaves = {n: (x[n].clone().requires_grad_(n in ("q", "beta")) if x[n] is not None else None) for n in ORDER}
    o, _ = O.naive_recurrent_sgsa(**leaves)
    o.sum().backward()
    for name, t in (("q", q), ("beta", beta)):
        ref = leaves[name].grad
        err = (t.grad.double().cpu() - ref).abs().max() / ref.abs().max()
        assert err <= 1e-4, f"{name}: {err:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("dims,sparse,init", [((1, 700, 3, 128), True, True), ((2, 333, 2, 40), False, True),
                                              ((1, 129, 2, 96), True, False)])
def test_native_backward_matches_torch_recompute(dev, dtype, tol, dims, sparse, init):
    from sgsa_amd.backward import recompute_grads
    from sgsa_amd.ops import chunk_sgsa_bwd
    B, T, H, D = dims
    x = _inputs(B, T, H, D, sparse, init, seed=21)
    inputs = []
    for n in ORDER:
        t = x[n]
        if t is not None:
            t = t.to(dev)
            t = t.to(dtype) if n in ("q", "k", "v", "sparse_k", "sparse_v") else t.float()
        inputs.append(t)
    g = torch.Generator().manual_seed(22)
    do = torch.randn(B, T, H, D, generator=g).to(dev, dtype)
    dht = torch.randn(B, H, D, D, generator=g).to(dev)
    print(f"native backward {dims} sparse={sparse} init={init} {dtype}", flush=True)
    needs = [t is not None for t in inputs]
    got = chunk_sgsa_bwd(inputs, needs, do, dht)
    f32 = [None if t is None else t.float() for t in inputs]
    want = recompute_grads(f32, needs, do.float(), dht)
    torch.cuda.synchronize()
    for n, a, b in zip(ORDER, got, want):
        if b is None:
            assert a is None, n
            continue
        a, b = a.double().cpu(), b.double().cpu()
        assert torch.isfinite(a).all(), f"{n}: non-finite"
        err = (a - b).abs().max() / b.abs().max().clamp_min(1e-12)
        assert err <= tol, f"{n}: {err:.3e} from the torch recompute"
