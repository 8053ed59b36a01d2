"""GPU: the few-row form of sgsa_score_topk (decode shapes; rows_score_kernel +
rows_select_kernel) against the row kernel on the same call.  The scores come
from the same MFMA operand roles and score expression, so selections, scores,
top-2 and counts are compared exactly; the unsorted order of the few-row form
is one ascending run of key indices.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

import sgsa_amd  # noqa: E402  (pure Python; the HIP library loads on first call and raises if missing)
from sgsa_amd.retrieval import score_topk  # noqa: E402


def _inputs(dev, B, Tq, Tk, H, D, seed, dup=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, Tq, H, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Tk, H, D, device=dev, generator=g).to(torch.bfloat16)
    if dup:   # repeated keys: many exactly tied scores
        k = k[:, torch.arange(Tk, device=dev) % 37].contiguous()
    return q, k


@pytest.mark.parametrize("B,Tq,Tk,H,D,top_k,q_offset,causal,dup", [
    (8, 1, 16640, 16, 128, 2048, 16383, True, False),   # config-4 decode: 16384 valid of a 16640 buffer
    (3, 1, 4000, 16, 128, 300, 1000, True, True),        # 1001 valid keys (not a multiple of 16), ties
    (2, 1, 3001, 16, 128, 512, 0, False, False),         # not causal, Tk % 16 = 9
    (2, 1, 5000, 4, 64, 700, 4999, True, True),          # ties at the cut
    (1, 4, 3000, 2, 96, 512, 100, True, False),          # rows with fewer valid keys than top_k
    (2, 3, 2048, 2, 32, 64, 0, False, False),            # not causal
    (1, 1, 32768, 2, 128, 2048, 32767, True, False),     # the longest cache the form takes
])
def test_few_row_form_matches_row_kernel(dev, B, Tq, Tk, H, D, top_k, q_offset, causal, dup):
    q, k = _inputs(dev, B, Tq, Tk, H, D, seed=Tk + Tq, dup=dup)
    for srt in (True, False):
        ref = score_topk(q, k, top_k, causal=causal, q_offset=q_offset, sorted=srt, fast=False)
        got = score_topk(q, k, top_k, causal=causal, q_offset=q_offset, sorted=srt, fast=True,
                         **({} if srt else {"return_split": True}))
        torch.cuda.synchronize()
        for name, r, g in zip(("top2", "counts"), ref[2:4], got[2:4]):
            assert torch.equal(r, g), name
        cnt = ref[3]
        if srt:
            assert torch.equal(ref[0], got[0]), "sorted indices"
            assert torch.equal(ref[1], got[1]), "sorted scores"
        else:
            idx, sc, spl = got[0], got[1], got[4]
            assert torch.equal(spl, cnt), "one ascending run"
            slot = torch.arange(idx.shape[-1], device=dev)
            live = slot < cnt[..., None]
            d = idx[..., 1:] - idx[..., :-1]
            assert bool(((d > 0) | ~live[..., 1:]).all()), "ascending key order"
            assert bool((idx[~live] == 0).all()) and bool((sc[~live] == -torch.finfo(torch.float32).max).all())
            # same selected (index, score) pairs as the row kernel's unsorted output
            a = torch.sort(torch.where(live, ref[0], -1), dim=-1).values
            b = torch.sort(torch.where(live, idx, -1), dim=-1).values
            assert torch.equal(a, b), "selected key sets"
            ra = torch.gather(ref[1], -1, torch.argsort(torch.where(live, ref[0], 1 << 30), dim=-1))
            rb = torch.gather(sc, -1, torch.argsort(torch.where(live, idx, 1 << 30), dim=-1))
            assert torch.equal(torch.where(live, ra, 0.0), torch.where(live, rb, 0.0)), "scores of the selected keys"
