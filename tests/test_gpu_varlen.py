"""GPU: packed variable-length sequences (cu_seqlens) against the same calls
run on each sequence alone.

* chunk_sgsa and fused_recurrent_sgsa: outputs and per-sequence final states,
  with and without per-sequence initial states and the sparse write, and the
  gradients of every input through the packed call against the per-sequence
  calls' gradients.
* sparse_retrieve and block_retrieve (both modes): indices exactly, k_hat /
  v_hat / weights / diagnostics within tolerance.  A packed call is a padded
  batch under the reference's mask semantics, so what depends on the whole
  batch is left out: avg_distance (divided by the call's largest index); in
  block_token the slots past a row's own candidates (their count k_q is the
  largest over the batch, :159-160) and the distance ratios that count them; in
  block_only the entropy, whose zero weights span the padded row.

Sequence lengths 37, 130, 64 and 1 (ragged against the 64-token chunks and the
block sizes).
"""

import pytest
import torch

import sgsa_amd

pytestmark = pytest.mark.gpu

LENS = [37, 130, 64, 1]


def _cu(lens, dev):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32, device=dev)


def _state_inputs(total, H, D, dt, dev, sparse, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    nk = lambda t: t / t.norm(dim=-1, keepdim=True)
    x = dict(q=r(1, total, H, D), k=nk(r(1, total, H, D)), v=r(1, total, H, D),
             beta=torch.sigmoid(r(1, total, H)), gamma=torch.sigmoid(r(1, total, H) + 3.0))
    if sparse:
        x.update(sparse_k=nk(r(1, total, H, D)), sparse_v=r(1, total, H, D), alpha=0.25 * torch.sigmoid(r(1, total, H)))
    return {n: t.to(dev, dt if t.dim() == 4 else torch.float32) for n, t in x.items()}


@pytest.mark.parametrize("op", ["chunk", "recurrent"])
@pytest.mark.parametrize("dt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("sparse,init", [(True, True), (False, False)])
def test_packed_state_update_equals_per_sequence(dev, op, dt, tol, sparse, init):
    H, D = 2, 64
    fn = sgsa_amd.chunk_sgsa if op == "chunk" else sgsa_amd.fused_recurrent_sgsa
    total = sum(LENS)
    x = _state_inputs(total, H, D, dt, dev, sparse)
    h0 = 0.1 * torch.randn(len(LENS), H, D, D, device=dev) if init else None
    print(f"varlen {op} {dt} sparse={sparse} init={init}", flush=True)
    o, ht = fn(**x, initial_state=h0, output_final_state=True, cu_seqlens=_cu(LENS, dev))
    assert o.shape == (1, total, H, D) and ht.shape == (len(LENS), H, D, D)
    a = 0
    for n, L in enumerate(LENS):
        xs = {k: t[:, a:a + L] for k, t in x.items()}
        on, hn = fn(**xs, initial_state=None if h0 is None else h0[n:n + 1], output_final_state=True)
        ref = on.float()
        err = (o[:, a:a + L].float() - ref).abs().max() / ref.abs().max().clamp_min(1e-6)
        assert err <= tol, (n, float(err))
        herr = (ht[n].float() - hn[0].float()).abs().max() / hn.abs().max().clamp_min(1e-6)
        assert herr <= tol, (n, float(herr))
        a += L


def test_packed_backward_equals_per_sequence(dev):
    H, D = 2, 64
    total = sum(LENS)
    x = _state_inputs(total, H, D, torch.float32, dev, True, seed=3)
    h0 = 0.1 * torch.randn(len(LENS), H, D, D, device=dev)
    leaves = {k: t.clone().requires_grad_() for k, t in x.items()}
    h0p = h0.clone().requires_grad_()
    o, ht = sgsa_amd.chunk_sgsa(**leaves, initial_state=h0p, output_final_state=True, cu_seqlens=_cu(LENS, dev))
    (o.square().mean() * total + ht.square().sum()).backward()
    a = 0
    for n, L in enumerate(LENS):
        ls = {k: t[:, a:a + L].clone().requires_grad_() for k, t in x.items()}
        hs = h0[n:n + 1].clone().requires_grad_()
        on, hn = sgsa_amd.chunk_sgsa(**ls, initial_state=hs, output_final_state=True)
        (on.square().mean() * L + hn.square().sum()).backward()
        for k in x:
            g, ref = leaves[k].grad[:, a:a + L], ls[k].grad
            err = (g - ref).abs().max() / ref.abs().max().clamp_min(1e-6)
            assert err <= 1e-4, (n, k, float(err))
        err = (h0p.grad[n] - hs.grad[0]).abs().max() / hs.grad.abs().max().clamp_min(1e-6)
        assert err <= 1e-4, (n, "initial_state", float(err))
        a += L


def _qkv(total, H, D, dt, dev, seed=5):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(1, total, H, D, generator=g).to(dev, dt) for _ in range(3)]


def _compare_retrieval(got, ref, a, L, kk, tol, skip=(), slots=None):
    for name in ("k_hat", "v_hat"):
        g, r = got[name][:, a:a + L].float(), ref[name].float()
        assert (g - r).abs().max() <= tol * r.abs().max().clamp_min(1.0), name
    if got.get("indices") is not None:
        gi = got["indices"][:, :, a:a + L, :kk]
        if slots is None:
            assert torch.equal(gi, ref["indices"]), "indices"
        else:
            assert torch.equal(gi[slots], ref["indices"][slots]), "indices"
    for name, val in ref["diagnostics"].items():
        if name == "avg_distance" or name in skip:
            continue
        g = got["diagnostics"][name][:, :, a:a + L]
        assert (g.float() - val.float()).abs().max() <= max(tol, 1e-4) * val.float().abs().max().clamp_min(1.0), name


@pytest.mark.parametrize("dt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_packed_token_retrieval_equals_per_sequence(dev, dt, tol):
    H, D, k = 2, 64, 16
    lens = [37, 130, 64, 20]
    total = sum(lens)
    q, kk_, v = _qkv(total, H, D, dt, dev)
    got = sgsa_amd.sparse_retrieve(q, kk_, v, k, cu_seqlens=_cu(lens, dev))
    assert got["k_hat"].shape == (1, total, H, D) and got["indices"].shape[:3] == (1, H, total)
    a = 0
    for L in lens:
        ref = sgsa_amd.sparse_retrieve(q[:, a:a + L], kk_[:, a:a + L], v[:, a:a + L], k)
        _compare_retrieval(got, ref, a, L, ref["indices"].shape[-1], tol)
        w = got["weights"][:, :, a:a + L, :ref["weights"].shape[-1]].float()
        assert (w - ref["weights"].float()).abs().max() <= tol
        a += L


@pytest.mark.parametrize("mode", ["block_token", "block_only"])
@pytest.mark.parametrize("dt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_packed_block_retrieval_equals_per_sequence(dev, mode, dt, tol):
    H, D, k, bs, tb = 2, 64, 12, 16, 3
    lens = [37, 130, 64, 20]
    total = sum(lens)
    q, kk_, v = _qkv(total, H, D, dt, dev, seed=7)
    got = sgsa_amd.block_retrieve(q, kk_, v, k, bs, tb, mode=mode, cu_seqlens=_cu(lens, dev))
    a = 0
    for L in lens:
        ref = sgsa_amd.block_retrieve(q[:, a:a + L], kk_[:, a:a + L], v[:, a:a + L], k, bs, tb, mode=mode)
        eb = ref["block_indices"].shape[-1]
        assert torch.equal(got["block_indices"][:, :, a:a + L, :eb], ref["block_indices"]), "block indices"
        if mode == "block_token":
            _compare_retrieval(got, ref, a, L, ref["indices"].shape[-1], tol,
                               skip=("local_ratio", "sink_ratio", "remote_ratio"), slots=ref["weights"] > 0)
        else:
            _compare_retrieval(got, ref, a, L, 0, tol, skip=("entropy",))
        a += L
