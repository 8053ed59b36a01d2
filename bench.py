#!/usr/bin/env python3
"""SGSA layer-forward benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-cpu-baseline] [--no-other-configs]
                    [--workload layer|model|hybrid|block|backward|train]

A step is one SGSA layer forward over the batch at the north-star shape
(B=1, H=16, T=32768, d=128, top-k=2048, chunk 64, bf16 inputs, fp32 state),
the kernels sgsa_layer_fwd runs:
  K1 sgsa_score_topk_thresholds   causal score GEMM + exact top-k, left as one
                        cut per row (threshold, tie index)
  K2 sgsa_sparse_gather_thresholds  the scores recomputed on MFMA against K/V
                        tiles loaded straight into LDS, the cut applied, top-k
                        weighted K/V sums + concentration/novelty + write gate
  K3-K5 sgsa_chunk_fwd  chunked gated-delta-rule update with the sparse write
--gather tiled times the tile-list form (K1 writes the selected entries, K2
reads them) and --gather direct the row-list form with per-row gathers; the
K1/K2 of one other form are timed once beside the step for comparison.
Inputs are synthetic (seed 0, the benchmark distribution) and resident in HBM
before timing.  Per-stage durations come from HIP events recorded on the
stream the kernels run on, inside the timed region.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "SGSA layer fwd tokens/s (bf16, T=32k, H=16, d=128); % MFMA / HBM roofline"
HBM_PEAK_GBS = 8000.0
NORTH_STAR = dict(B=1, T=32768, H=16, D=128, top_k=2048, chunk=64)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth_inputs(B, T, H, D, seed=0):
    """Benchmark distribution, drawn in a fixed order on a CPU generator:
    q,k,v ~ N(0,1) (q,k L2-normalised per head), beta = sigmoid(N(0,1)),
    gamma = exp(logsigmoid(N(0,1)+4)), budget logits ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gamma = torch.exp(torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g) + 4.0))
    budget = torch.randn(B, T, H, generator=g)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    return q, k, v, beta, gamma, budget


def heavy_tail_keys(k, seed=0, frac=0.01, mult=8.0):
    """Config 3's retrieval keys: for each (b, h), round(frac * T) key positions (randperm on a
    generator seeded ``seed``) scaled by ``mult``; the state update keeps the unit-norm keys."""
    B, T, H, _ = k.shape
    g = torch.Generator().manual_seed(seed + 1)
    kr = k.clone()
    n = int(round(frac * T))
    for b in range(B):
        for h in range(H):
            kr[b, torch.randperm(T, generator=g)[:n], h] *= mult
    return kr


def time_config(name, B, T, H, D, top_k, dtype, heavy=False, reps=3, cpu=False):
    """One BASELINE.json configuration through the layer path, outside the timed steps:
    K1 -> K2 -> chunk update as sgsa_layer_fwd runs them (bf16, d = 128: the threshold
    form, per stage; otherwise the whole sgsa_layer_fwd call).  Config 3 retrieves over
    the heavy-tailed keys and updates the state with the unit-norm ones.  Returns ms per
    layer forward (mean of ``reps`` after one warm-up), tokens/s and the stage split, and
    with ``cpu`` the CPU oracle's rate on a bounded sample of the same inputs."""
    import sgsa_amd
    from sgsa_amd import _abi
    dev = torch.device("cuda:0")
    q, k, v, beta, gamma, budget = synth_inputs(B, T, H, D)
    kr = heavy_tail_keys(k) if heavy else k
    qd, kd, vd, krd = (t.to(dev, dtype).contiguous() for t in (q, k, v, kr))
    bd, gd, ud = (t.to(dev).contiguous() for t in (beta, gamma, budget))
    cpu_in = (q.to(dtype), kr.to(dtype), v.to(dtype), beta, gamma, budget) if cpu else None
    del q, k, v, kr
    L, P = _abi.lib(), _abi.ptr
    stream = _abi.stream_of(qd)
    dc = _abi.dtype_code(dtype)
    kk = min(top_k, T)
    out = torch.empty_like(qd)
    ht = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    thr_form = dtype == torch.bfloat16 and D == 128
    if thr_form:
        n = ctypes.c_size_t()
        _abi.check(L.sgsa_score_topk_workspace_size(B, T, H, ctypes.byref(n)))
        tws = torch.empty(n.value, device=dev, dtype=torch.uint8)
        _abi.check(L.sgsa_chunk_fwd_workspace_size(B, T, H, D, 1, ctypes.byref(n)))
        cws = torch.empty(n.value, device=dev, dtype=torch.uint8)
        thr = torch.empty(B, H, T, 2, device=dev, dtype=torch.int32)
        top2 = torch.empty(B, H, T, 2, device=dev, dtype=torch.float32)
        cnt = torch.empty(B, H, T, device=dev, dtype=torch.int32)
        wk, vh = torch.empty_like(qd), torch.empty_like(qd)
        al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
        stages = (
            ("score_topk", lambda: _abi.check(L.sgsa_score_topk_thresholds(
                B, T, H, D, kk, P(qd), P(krd), P(thr), P(top2), P(cnt), P(tws), tws.numel(), stream))),
            ("gather_gate", lambda: _abi.check(L.sgsa_sparse_gather_thresholds(
                B, T, H, D, kk, P(qd), P(krd), P(vd), P(thr), P(top2), P(cnt), P(ud), 0, 0.25, 0.1, P(wk), P(vh),
                None, P(al), stream))),
            ("chunk", lambda: _abi.check(L.sgsa_chunk_fwd(
                dc, B, T, H, D, 64, P(qd), P(kd), P(vd), P(bd), P(gd), P(wk), P(vh), P(al), None, P(out), P(ht),
                P(cws), cws.numel(), stream))),
        )
    else:
        n = ctypes.c_size_t()
        _abi.check(L.sgsa_layer_fwd_workspace_size(dc, B, T, H, D, kk, ctypes.byref(n)))
        lws = torch.empty(n.value, device=dev, dtype=torch.uint8)
        stages = (("layer", lambda: _abi.check(L.sgsa_layer_fwd(
            dc, B, T, H, D, kk, 64, P(qd), P(kd), P(vd), P(qd), P(bd), P(gd), P(ud), None, 0, 0.25, 0.1, P(out),
            P(ht), P(lws), lws.numel(), stream))),)
    cur = torch.cuda.current_stream(dev)
    for _, fn in stages:
        fn()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(reps)]
    for r in range(reps):
        for i, (_, fn) in enumerate(stages):
            ev[r][i].record(cur)
            fn()
        ev[r][-1].record(cur)
    torch.cuda.synchronize()
    st = {nm: sum(ev[r][i].elapsed_time(ev[r][i + 1]) for r in range(reps)) / reps for i, (nm, _) in enumerate(stages)}
    ms = sum(st.values())
    ok = bool(torch.isfinite(out.float()).all() and torch.isfinite(ht).all())
    f_score = B * H * T * (T + 1) * D
    res = {"config": name, "B": B, "T": T, "H": H, "D": D, "top_k": top_k, "dtype": str(dtype).split(".")[-1],
           "heavy_tail_keys": heavy, "ms": round(ms, 3), "tokens_per_s": round(B * T / (ms / 1000.0), 1),
           "stage_ms": {nm: round(v, 3) for nm, v in st.items()}, "finite": ok}
    if "score_topk" in st:
        res["score_topk_mfma_frac"] = round(f_score / (st["score_topk"] / 1000.0) / 2.5e15, 4)
    if cpu_in is not None:
        res["cpu_baseline"] = cpu_baseline(*cpu_in, dict(B=B, T=T, H=H, D=D, top_k=top_k, chunk=64))
    log(f"{name}: {json.dumps(res)}")
    return res


def time_masked(B, T, H, D, top_k, pad, reps=3):
    """The layer under a padding mask (bf16, d = 128): the first ``pad`` positions of
    every sequence are padding.  sgsa_layer_retrieve_masked (per-row valid prefixes,
    keys and values compacted valid-first, the threshold K1 and K2 over them) then the
    chunk update, outside the timed steps.  Returns ms per layer forward (mean of
    ``reps`` after one warm-up) and the stage split."""
    from sgsa_amd import _abi
    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    q, k, v, beta, gamma, budget = synth_inputs(B, T, H, D)
    qd, kd, vd = (t.to(dev, dtype).contiguous() for t in (q, k, v))
    bd, gd, ud = (t.to(dev).contiguous() for t in (beta, gamma, budget))
    del q, k, v
    am = torch.ones(B, T, device=dev, dtype=torch.uint8)
    am[:, :pad] = 0
    L, P = _abi.lib(), _abi.ptr
    stream = _abi.stream_of(qd)
    kk = min(top_k, T)
    n = ctypes.c_size_t()
    _abi.check(L.sgsa_layer_retrieve_masked_workspace_size(1, B, T, H, D, kk, ctypes.byref(n)))
    rws = torch.empty(n.value, device=dev, dtype=torch.uint8)
    _abi.check(L.sgsa_chunk_fwd_workspace_size(B, T, H, D, 1, ctypes.byref(n)))
    cws = torch.empty(n.value, device=dev, dtype=torch.uint8)
    wk, vh, out = torch.empty_like(qd), torch.empty_like(qd), torch.empty_like(qd)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    ht = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    stages = (
        ("retrieve_masked", lambda: _abi.check(L.sgsa_layer_retrieve_masked(
            1, B, T, H, D, kk, P(qd), P(kd), P(vd), P(am), P(ud), 0, 0.25, 0.1, P(wk), P(vh), P(al), None,
            P(rws), rws.numel(), stream))),
        ("chunk", lambda: _abi.check(L.sgsa_chunk_fwd(
            1, B, T, H, D, 64, P(qd), P(kd), P(vd), P(bd), P(gd), P(wk), P(vh), P(al), None, P(out), P(ht),
            P(cws), cws.numel(), stream))),
    )
    cur = torch.cuda.current_stream(dev)
    for _, fn in stages:
        fn()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(reps)]
    for r in range(reps):
        for i, (_, fn) in enumerate(stages):
            ev[r][i].record(cur)
            fn()
        ev[r][-1].record(cur)
    torch.cuda.synchronize()
    st = {nm: sum(ev[r][i].elapsed_time(ev[r][i + 1]) for r in range(reps)) / reps for i, (nm, _) in enumerate(stages)}
    ms = sum(st.values())
    pad_rows = vh[:, :pad].float().abs().max().item() if pad > 0 else 0.0
    res = {"config": "north star, left-padded", "B": B, "T": T, "H": H, "D": D, "top_k": top_k, "pad": pad,
           "dtype": "bfloat16", "ms": round(ms, 3), "tokens_per_s": round(B * T / (ms / 1000.0), 1),
           "stage_ms": {nm: round(v, 3) for nm, v in st.items()},
           "finite": bool(torch.isfinite(out.float()).all() and torch.isfinite(ht).all()),
           "padded_rows_retrieve_nothing": pad_rows == 0.0}
    log(f"masked: {json.dumps(res)}")
    return res


def gather_bytes(B, H, T, D, k, elem=2):
    """Algorithmic bytes of the K/V gather: B*H*sum_t min(k, t+1) * 2 rows * D * elem."""
    rows = k * (T - k) + k * (k + 1) // 2 if T > k else T * (T + 1) // 2
    return B * H * rows * 2 * D * elem


def cpu_baseline(q, k, v, beta, gamma, budget, cfg, sample_rows=256, chunk_tokens=1024):
    """The CPU oracle (fp32 torch restatement) timed on a bounded, stratified sample
    of the same workload and extrapolated to the whole layer."""
    from oracle import sgsa_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, T, H, D, top_k = cfg["B"], cfg["T"], cfg["H"], cfg["D"], cfg["top_k"]
    qf, kf, vf = q.float(), k.float(), v.float()
    # retrieval: 16 blocks of sample_rows/16 rows spread evenly over the sequence
    nblk = 16
    per = max(1, sample_rows // nblk)
    starts = [min(T - per, (i * T) // nblk + (T // nblk) - per) for i in range(nblk)]
    t0 = time.perf_counter()
    for s in starts:
        O.token_topk_retrieval(qf, kf, vf, top_k, rows=(s, s + per), block_rows=per)
    t_ret = (time.perf_counter() - t0) * T / (nblk * per)
    log(f"cpu retrieval sample: {nblk * per} rows in {time.perf_counter() - t0:.1f}s")
    # chunked state update on the first chunk_tokens tokens (cost linear in T)
    n = min(T, chunk_tokens)
    g = torch.Generator().manual_seed(1)
    sk = kf[:, :n]
    sv = vf[:, :n]
    alpha = 0.25 * torch.rand(B, n, H, generator=g)
    t0 = time.perf_counter()
    O.chunk_sgsa_fwd(qf[:, :n], kf[:, :n], vf[:, :n], beta[:, :n], gamma[:, :n], sk, sv, alpha, None,
                     cfg["chunk"], True)
    t_chunk = (time.perf_counter() - t0) * T / n
    log(f"cpu chunk sample: {n} tokens in {time.perf_counter() - t0:.1f}s")
    total = t_ret + t_chunk
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": B * T / total,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "extrapolated": True,
        "sample": (f"fp32 torch oracle on {cores} threads ({cpu}); retrieval timed on {nblk}x{per} query rows "
                   f"spread evenly over T={T} (all {H} heads) and scaled by T/{nblk * per}; chunk update timed on "
                   f"the first {n} tokens and scaled by T/{n}; extrapolated layer time {total:.1f}s"),
    }


MODEL_METRIC = "SGSA 2-layer model fwd tokens/s (config 2: bf16, B=16, T=4096, hidden 1024, 8x128 heads, vocab 8192)"
HYBRID_METRIC = ("hybrid decoder decode tokens/s (config 4: bf16, 24 layers 3:1 SGSA:dense GQA, hidden 2048, "
                 "16q/4kv x 128, prefill 16384 at B=1, 256 greedy steps at B=8, top-k 2048 every 4 steps)")


def recall_batch(B: int, T: int, vocab: int, seed: int = 0) -> torch.Tensor:
    """Config 2's associative-recall sequences: 1024 (key, value) token pairs drawn
    without replacement from the lower / upper half of the vocabulary, then query
    pairs whose keys are resampled from the stored ones (each followed by its
    value), repeated until the sequence has T tokens."""
    g = torch.Generator().manual_seed(seed)
    half = vocab // 2
    seqs = []
    for _ in range(B):
        keys = torch.randperm(half - 1, generator=g)[:1024] + 1
        vals = torch.randperm(half, generator=g)[:1024] + half
        pairs = torch.stack([keys, vals], 1).reshape(-1)
        nq = (T - pairs.numel() + 1) // 2
        pick = torch.randint(0, 1024, (nq,), generator=g)
        queries = torch.stack([keys[pick], vals[pick]], 1).reshape(-1)
        seqs.append(torch.cat([pairs, queries])[:T])
    return torch.stack(seqs)


def run_model(args) -> int:
    """Config 2: the 2-layer SGSA causal LM forward (sgsa_amd.SGSAForCausalLM).  The value is the
    reference config's default retrieval (block_token, top-k 16, blocks of 32, 2 kept;
    modelings/modeling_sgsa.py:58-61); token_only at top-k 16 is timed beside it."""
    import sgsa_amd
    B, T = 16, 4096
    dev = torch.device("cuda:0")
    ids = recall_batch(B, T, 8192).to(dev)
    res = {}
    for mode in ("block_token", "token_only"):
        cfg = sgsa_amd.SGSAConfig(vocab_size=8192, hidden_size=1024, intermediate_size=2816, num_hidden_layers=2,
                                  num_attention_heads=8, num_kv_heads=8, max_position_embeddings=T, top_k=16,
                                  retrieval_mode=mode)
        model = sgsa_amd.SGSAForCausalLM(cfg)
        model.init_weights(std=0.02, qk_std=1.0 / math.sqrt(cfg.hidden_size * cfg.head_dim),
                           generator=torch.Generator().manual_seed(0))
        model = model.to(device=dev, dtype=torch.bfloat16).eval()
        log(f"model: config 2 ({mode}), B={B} T={T}, warmup {args.warmup}")
        with torch.no_grad():
            for _ in range(args.warmup):
                logits = model(ids)["logits"]
            torch.cuda.synchronize()
            cur = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cur)
            for _ in range(args.steps):
                logits = model(ids)["logits"]
            e1.record(cur)
            torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / max(args.steps, 1)
        if not torch.isfinite(logits).all():
            log("non-finite logits")
            return 1
        log(f"model ({mode}) ms/step {ms:.3f}")
        res[mode] = ms
        del model, logits
        torch.cuda.empty_cache()
    ms = res["block_token"]
    print(json.dumps({
        "metric": MODEL_METRIC, "value": round(B * T / (ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic associative-recall token ids, random-init weights",
        "config": {"workload": "sgsa_model_fwd", "B": B, "T": T, "hidden": 1024, "heads": 8, "head_dim": 128,
                   "vocab": 8192, "layers": 2, "intermediate": 2816, "top_k": 16, "retrieval_mode": "block_token",
                   "block_size": 32, "top_blocks": 2,
                   "init": "normal std 0.02; q/k/q_ret projections std 1/sqrt(hidden*head_dim)"},
        "token_only": {"ms_per_step": round(res["token_only"], 3),
                       "value": round(B * T / (res["token_only"] / 1000.0), 1)},
        "cpu_baseline": None,
    }), flush=True)
    return 0


TRAIN_METRIC = ("SGSA 2-layer model training tokens/s (config-2 shape: fp32, AdamW, B=16, T=4096, hidden 1024, "
                "8x128 heads, vocab 8192, block_token)")


def run_train(args) -> int:
    """Training steps of the config-2 model as the reference's experiment runs them
    (experiments/run_sgsa_synthetic_retrieval.py:100-117: fp32 parameters, AdamW, forward with
    labels, backward, optimizer step), with the reference config's default block_token
    retrieval: per step the forward, the backward through the retrieval's differentiable form
    and the native chunk backward, and the AdamW update."""
    import sgsa_amd
    B, T = 16, 4096
    dev = torch.device("cuda:0")
    ids = recall_batch(B, T, 8192).to(dev)
    cfg = sgsa_amd.SGSAConfig(vocab_size=8192, hidden_size=1024, intermediate_size=2816, num_hidden_layers=2,
                              num_attention_heads=8, num_kv_heads=8, max_position_embeddings=T, top_k=16,
                              retrieval_mode="block_token")
    model = sgsa_amd.SGSAForCausalLM(cfg)
    model.init_weights(std=0.02, qk_std=1.0 / math.sqrt(cfg.hidden_size * cfg.head_dim),
                       generator=torch.Generator().manual_seed(0))
    model = model.to(device=dev).train()
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)

    def step():
        loss = model(ids, labels=ids)["loss"]
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        return loss

    log(f"train: config-2 shape, fp32, B={B} T={T}, warmup {args.warmup}")
    for _ in range(args.warmup):
        loss = step()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(args.steps):
        loss = step()
    e1.record(cur)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / max(args.steps, 1)
    if not torch.isfinite(loss):
        log("non-finite loss")
        return 1
    log(f"train ms/step {ms:.3f} loss {loss.item():.4f}")
    peak = torch.cuda.max_memory_allocated() / 2**30
    # the same steps under bf16 autocast (fp32 parameters and optimizer; the projections, the
    # retrieval's selection and the state update in bf16)
    for _ in range(args.warmup):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids)["loss"]
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
    torch.cuda.synchronize()
    e0.record(cur)
    for _ in range(args.steps):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids)["loss"]
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
    e1.record(cur)
    torch.cuda.synchronize()
    ms_ac = e0.elapsed_time(e1) / max(args.steps, 1)
    if not torch.isfinite(loss):
        log("non-finite loss under autocast")
        return 1
    log(f"train (bf16 autocast) ms/step {ms_ac:.3f} loss {loss.item():.4f}")
    print(json.dumps({
        "metric": TRAIN_METRIC, "value": round(B * T / (ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic associative-recall token ids, random-init weights",
        "config": {"workload": "sgsa_model_train", "B": B, "T": T, "hidden": 1024, "heads": 8, "head_dim": 128,
                   "vocab": 8192, "layers": 2, "intermediate": 2816, "top_k": 16, "retrieval_mode": "block_token",
                   "block_size": 32, "top_blocks": 2, "optimizer": "AdamW lr 1e-4",
                   "peak_memory_gb": round(peak, 1)},
        "bf16_autocast": {"ms_per_step": round(ms_ac, 3), "value": round(B * T / (ms_ac / 1000.0), 1)},
        "cpu_baseline": None,
    }), flush=True)
    return 0


def run_hybrid(args) -> int:
    """Config 4: the 24-layer hybrid decoder (sgsa_amd.hybrid), prefill then greedy decode: a warm-up
    prefill, the timed prefill, 4 untimed decode steps (where the decode plan is built), then the 256
    timed decode steps."""
    from sgsa_amd.hybrid import HybridConfig, HybridForCausalLM, expand_caches, rope_tables
    T, B, steps = 16384, 8, 256
    wsteps = 4   # untimed decode steps first (one selecting, three re-scoring): the decode plan is built there
    cfg = HybridConfig()
    dev = torch.device("cuda:0")
    model = HybridForCausalLM(cfg)
    model.init_weights(std=0.02, qk_std=1.0 / math.sqrt(cfg.hidden_size * cfg.head_dim),
                       generator=torch.Generator().manual_seed(0))
    model = model.to(device=dev, dtype=torch.bfloat16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(1)).to(dev)
    rope = rope_tables(T + wsteps + steps, cfg.head_dim, cfg.rope_theta, dev)
    cur = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    log(f"hybrid: config 4, prefill T={T} at B=1, then {wsteps} untimed and {steps} timed decode steps at B={B}")
    with torch.no_grad():
        caches = model.new_cache(1, T + wsteps + steps, dev, torch.bfloat16)
        model.prefill(ids, caches, rope)   # warm-up: kernels, workspaces, GEMM plans
        torch.cuda.synchronize()
        ev[0].record(cur)
        logits = model.prefill(ids, caches, rope)
        ev[1].record(cur)
        torch.cuda.synchronize()
        log(f"prefill {ev[0].elapsed_time(ev[1]):.1f} ms")
        caches = expand_caches(caches, B)
        tok = logits[:, -1].argmax(-1).expand(B).contiguous()
        for s in range(wsteps):
            tok = model.decode_step(tok, T + s, s, caches, rope).argmax(-1)
        torch.cuda.synchronize()
        ev[2].record(cur)
        for s in range(wsteps, wsteps + steps):
            tok = model.decode_step(tok, T + s, s, caches, rope).argmax(-1)
            if (s + 1 - wsteps) % 64 == 0:
                log(f"decode step {s + 1 - wsteps}")
        ev[3].record(cur)
        torch.cuda.synchronize()
    pre_ms, dec_ms = ev[0].elapsed_time(ev[1]), ev[2].elapsed_time(ev[3])
    if not torch.isfinite(logits.float()).all():
        log("non-finite logits")
        return 1
    log(f"decode {dec_ms:.1f} ms for {steps} steps")
    print(json.dumps({
        "metric": HYBRID_METRIC, "value": round(B * steps / (dec_ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": wsteps, "ms_per_step": round(dec_ms / steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "uniform-random token ids, random-init weights",
        "prefill": {"T": T, "B": 1, "ms": round(pre_ms, 1), "tokens_per_s": round(T / (pre_ms / 1000.0), 1)},
        "config": {"workload": "hybrid_decoder", "layers": cfg.num_hidden_layers, "dense_every": cfg.dense_every,
                   "hidden": cfg.hidden_size, "heads": cfg.num_attention_heads, "kv_heads": cfg.num_kv_heads,
                   "head_dim": cfg.head_dim, "intermediate": cfg.intermediate_size, "vocab": cfg.vocab_size,
                   "top_k": cfg.top_k, "topk_recompute_every": cfg.topk_recompute_every, "decode_batch": B,
                   "init": "normal std 0.02; SGSA q/k/q_ret projections std 1/sqrt(hidden*head_dim)"},
        "cpu_baseline": None,
    }), flush=True)
    return 0


BLOCK_METRIC = ("SGSA block retrieval tokens/s (bf16, T=32k, H=16, d=128; retrieval_mode block_token with the "
                "reference config defaults top_k 16, block_size 32, top_blocks 2)")


def run_block(args) -> int:
    """Block retrieval modes of SparseRetriever (sgsa_amd.block_retrieve) at the north-star shape, with the
    reference config's defaults top_k 16, block_size 32, top_blocks 2 (modelings/modeling_sgsa.py:58-61).
    Times block_token (the value) and block_only; block_only's dense [B,H,T,T] weights are not requested."""
    import sgsa_amd
    B, T, H, D = NORTH_STAR["B"], args.T, NORTH_STAR["H"], NORTH_STAR["D"]
    top_k, bs, tb = 16, 32, 2
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(B, T, H, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    cur = torch.cuda.current_stream()
    out = {}
    for mode in ("block_token", "block_only"):
        call = lambda: sgsa_amd.block_retrieve(q, k, v, top_k, bs, tb, mode=mode, return_weights=(mode == "block_token"))
        for _ in range(args.warmup):
            r = call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        for _ in range(args.steps):
            r = call()
        e1.record(cur)
        torch.cuda.synchronize()
        out[mode] = e0.elapsed_time(e1) / max(args.steps, 1)
        if not torch.isfinite(r["v_hat"].float()).all():
            log(f"{mode}: non-finite output")
            return 1
        log(f"{mode} ms/call {out[mode]:.3f}")
    ms = out["block_token"]
    print(json.dumps({
        "metric": BLOCK_METRIC, "value": round(B * T / (ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic normal q/k/v",
        "block_only_ms": round(out["block_only"], 3),
        "config": {"workload": "sgsa_block_retrieval", "B": B, "T": T, "H": H, "D": D, "top_k": top_k,
                   "block_size": bs, "top_blocks": tb, "outputs": "k_hat, v_hat, indices, block_indices, "
                   "weights (block_token), diagnostics"},
        "cpu_baseline": None,
    }), flush=True)
    return 0


def run_backward(args) -> int:
    """The native backward of chunk_sgsa (sgsa_chunk_bwd through sgsa_amd.chunk_sgsa_bwd) at the north-star shape
    with the sparse write: every input gradient from dO, bf16 inputs, fp32 state.  A step is one backward call on
    resident inputs and output gradient.  --torch-recompute also times, once, the reference's method (the forward
    recomputed in torch under autograd, modelings/sgsa_ops/chunk_bwd.py:31-77) on the same inputs in fp32."""
    import sgsa_amd
    from sgsa_amd.ops import chunk_sgsa_bwd
    B, T, H, D = NORTH_STAR["B"], args.T, NORTH_STAR["H"], NORTH_STAR["D"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    r = lambda *s: torch.randn(*s, device=dev, generator=g)
    unit = lambda t: t / t.norm(dim=-1, keepdim=True)
    bf = torch.bfloat16
    q, k, v = unit(r(B, T, H, D)).to(bf), unit(r(B, T, H, D)).to(bf), r(B, T, H, D).to(bf)
    sk, sv = unit(r(B, T, H, D)).to(bf), r(B, T, H, D).to(bf)
    beta, gamma = torch.sigmoid(r(B, T, H)), torch.sigmoid(r(B, T, H) + 4.0)
    alpha = 0.25 * torch.sigmoid(r(B, T, H))
    do = r(B, T, H, D).to(bf)
    inputs = [q, k, v, beta, gamma, sk, sv, alpha, None]
    needs = [True] * 8 + [False]
    cur = torch.cuda.current_stream()
    for _ in range(args.warmup):
        grads = chunk_sgsa_bwd(inputs, needs, do, None)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(args.steps):
        grads = chunk_sgsa_bwd(inputs, needs, do, None)
    e1.record(cur)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / max(args.steps, 1)
    if not all(torch.isfinite(t.float()).all() for t in grads if t is not None):
        log("backward: non-finite gradient")
        return 1
    log(f"native backward ms/call {ms:.3f}")
    # fp32 MFMA multiply-adds per chunk-head (M = 2L samples with the sparse write, L tokens, d dims)
    M, L, d = 128, 64, 128
    mac = (3 * M * M * d + M ** 3 // 3                                    # intra: Gram, (I+T)^-1, W, U
           + 2 * d * d * M                                               # maps: Phi, Pm
           + 2 * d ** 3                                                  # the two scans, one step each
           + L * M * d + d * d * L + M * d * L + d * d * M               # pre: P, Q^T dO, P^T dO, W^T X1
           + 5 * M * d * d + 7 * M * M * d + 2 * M ** 3 + 4 * L * M * d + L * d * d)   # gradient kernel
    nchunks = B * H * ((T + 63) // 64)
    flops = 2.0 * mac * nchunks
    torch_ms = None
    if args.torch_recompute:
        from sgsa_amd.backward import recompute_grads
        f32 = [None if t is None else t.float() for t in inputs]
        recompute_grads(f32, needs, do.float(), None)
        torch.cuda.synchronize()
        t0 = time.time()
        recompute_grads(f32, needs, do.float(), None)
        torch.cuda.synchronize()
        torch_ms = (time.time() - t0) * 1e3
        log(f"torch recompute ms/call {torch_ms:.1f}")
    print(json.dumps({
        "metric": "chunk_sgsa backward tokens/s (bf16, T=32k, H=16, d=128, sparse write)",
        "value": round(B * T / (ms / 1000.0), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 (bf16 inputs and gradients)", "data": "synthetic",
        "config": {"workload": "chunk_sgsa_backward", "B": B, "T": T, "H": H, "D": D, "chunk": 64,
                   "sparse_write": True},
        "mfma_fp32": {"flops": flops, "achieved_tflops": round(flops / (ms / 1000.0) / 1e12, 2),
                      "peak_tflops": 157.3, "frac": round(flops / (ms / 1000.0) / 1e12 / 157.3, 4)},
        "torch_recompute_ms": round(torch_ms, 1) if torch_ms is not None else None,
        "cpu_baseline": None,
    }), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--T", type=int, default=NORTH_STAR["T"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip timing configs 0, 1 and 3 beside the headline (outside the timed steps)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one plain 256 MiB fp32 copy kernel (torch.neg) first; its PMC byte counters "
                         "give the scale factor for the traffic of the SGSA kernels")
    ap.add_argument("--traffic-from", default=os.path.join(ROOT, "profiles", "hbm_traffic_north_star_pmc.md"),
                    help="committed PMC summary whose 'hbm_bytes_per_launch <kernel>:' lines give the measured "
                         "L2-to-fabric bytes of one launch at the north-star shape")
    ap.add_argument("--gather", choices=("threshold", "tiled", "direct"), default="threshold",
                    help="timed step: the fused layer path (K1 row thresholds -> K2 recomputing the scores on "
                         "MFMA -> chunk, what sgsa_layer_fwd runs; default), the tile-list form (K1 tile lists -> "
                         "LDS-tiled MFMA K2 -> chunk) or K1 row lists -> per-row 16-byte gathers -> chunk")
    ap.add_argument("--torch-recompute", action="store_true",
                    help="with --workload backward: also time the torch recompute backward once")
    ap.add_argument("--workload", choices=("layer", "model", "hybrid", "block", "backward", "train"), default="layer",
                    help="layer: the north-star SGSA layer forward (the headline metric, default); model: "
                         "config 2, the 2-layer SGSA causal LM forward at B=16 T=4096; hybrid: config 4, the "
                         "24-layer SGSA / dense-GQA decoder, prefill of 16384 tokens then 256 decode steps at B=8; "
                         "block: the retriever's block_token / block_only modes at the north-star shape; "
                         "backward: the native backward of chunk_sgsa at the north-star shape; train: config 2's "
                         "model trained as the reference's experiment trains it (fp32, AdamW)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); the SGSA layer shards by head, "
              "and no multi-GPU path is part of this build", file=sys.stderr)
        return 2
    if args.workload == "model":
        return run_model(args)
    if args.workload == "hybrid":
        return run_hybrid(args)
    if args.workload == "block":
        return run_block(args)
    if args.workload == "backward":
        return run_backward(args)
    if args.workload == "train":
        return run_train(args)

    import sgsa_amd
    from sgsa_amd import _abi

    cfg = dict(NORTH_STAR)
    cfg["T"] = args.T
    B, T, H, D, top_k = cfg["B"], cfg["T"], cfg["H"], cfg["D"], cfg["top_k"]
    kk = min(top_k, T)
    dev = torch.device("cuda:0")
    log(f"generating inputs B={B} T={T} H={H} D={D} k={top_k}")
    q, k, v, beta, gamma, budget = synth_inputs(B, T, H, D)
    bf = torch.bfloat16
    qd, kd, vd = (t.to(dev, bf).contiguous() for t in (q, k, v))
    bd, gd, ud = (t.to(dev).contiguous() for t in (beta, gamma, budget))
    idx = torch.empty(B, H, T, kk, device=dev, dtype=torch.int32)
    sc = torch.empty(B, H, T, kk, device=dev, dtype=torch.float32)
    cnt = torch.empty(B, H, T, device=dev, dtype=torch.int32)
    top2 = torch.empty(B, H, T, 2, device=dev, dtype=torch.float32)
    wk = torch.empty(B, T, H, D, device=dev, dtype=bf)
    vh = torch.empty_like(wk)
    al = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    out = torch.empty_like(qd)
    ht = torch.empty(B, H, D, D, device=dev, dtype=torch.float32)
    nbytes = ctypes.c_size_t()
    L = _abi.lib()
    _abi.check(L.sgsa_chunk_fwd_workspace_size(B, T, H, D, 1, ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, device=dev, dtype=torch.uint8)
    tbytes = ctypes.c_size_t()
    _abi.check(L.sgsa_score_topk_workspace_size(B, T, H, ctypes.byref(tbytes)))
    tws = torch.empty(tbytes.value, device=dev, dtype=torch.uint8)
    lbytes, obytes = ctypes.c_size_t(), ctypes.c_size_t()
    _abi.check(L.sgsa_topk_lists_size(B, T, H, kk, ctypes.byref(lbytes), ctypes.byref(obytes)))
    tl = torch.empty(lbytes.value, device=dev, dtype=torch.uint8)
    toff = torch.empty(obytes.value // 4, device=dev, dtype=torch.int32)
    thr = torch.empty(B, H, T, 2, device=dev, dtype=torch.int32)
    P = _abi.ptr
    stream = _abi.stream_of(qd)
    scale = math.sqrt(D)

    def k1_rows():
        _abi.check(L.sgsa_score_topk(_abi.SGSA_BF16, B, T, T, H, D, kk, 1, 0, scale, 0, P(qd), P(kd), P(idx),
                                     P(sc), P(top2), P(cnt), None, 0, P(tws), tbytes.value, stream))

    def k1_lists():
        _abi.check(L.sgsa_score_topk_lists(B, T, H, D, kk, P(qd), P(kd), P(tl), P(toff), P(top2), P(cnt),
                                           P(tws), tbytes.value, stream))

    def k1_thr():
        _abi.check(L.sgsa_score_topk_thresholds(B, T, H, D, kk, P(qd), P(kd), P(thr), P(top2), P(cnt), P(tws),
                                                tbytes.value, stream))

    def k2_thr():
        _abi.check(L.sgsa_sparse_gather_thresholds(B, T, H, D, kk, P(qd), P(kd), P(vd), P(thr), P(top2), P(cnt),
                                                   P(ud), 0, 0.25, 0.1, P(wk), P(vh), None, P(al), stream))

    def k2_tiled():
        _abi.check(L.sgsa_sparse_gather_lists(B, T, H, D, kk, P(kd), P(vd), P(tl), P(toff), P(top2), P(cnt),
                                              P(ud), 0, 0.25, 0.1, P(wk), P(vh), None, P(al), stream))

    def k2_direct():
        _abi.check(L.sgsa_sparse_gather(_abi.SGSA_BF16, B, T, T, H, D, kk, 0, P(kd), P(vd), P(kd), P(idx), P(sc),
                                        P(top2), P(cnt), P(ud), 0, 0.25, 0.1, 64, 8, P(wk), P(vh), None, P(al),
                                        None, None, None, 0, stream))

    def k345():
        _abi.check(L.sgsa_chunk_fwd(_abi.SGSA_BF16, B, T, H, D, cfg["chunk"], P(qd), P(kd), P(vd), P(bd), P(gd),
                                    P(wk), P(vh), P(al), None, P(out), P(ht), P(ws), nbytes.value, stream))

    if args.gather == "threshold":
        stages = (("score_topk", k1_thr), ("gather_gate", k2_thr), ("chunk", k345))
        other = (k1_lists, k2_tiled)
    elif args.gather == "tiled":
        stages = (("score_topk", k1_lists), ("gather_gate", k2_tiled), ("chunk", k345))
        other = (k1_rows, k2_direct)
    else:
        stages = (("score_topk", k1_rows), ("gather_gate", k2_direct), ("chunk", k345))
        other = (k1_lists, k2_tiled)
    cur = torch.cuda.current_stream(dev)

    def step(events=None):
        for i, (_, fn) in enumerate(stages):
            if events is not None:
                events[i].record(cur)
            fn()
        if events is not None:
            events[-1].record(cur)

    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log("copy calibration: 268435456 bytes read, 268435456 bytes written (torch.neg)")
        del src, dst
    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(args.steps)]
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = 1000.0 * elapsed / args.steps
    stage_ms = {name: sum(evs[s][i].elapsed_time(evs[s][i + 1]) for s in range(args.steps)) / args.steps
                for i, (name, _) in enumerate(stages)}
    assert torch.isfinite(out.float()).all() and torch.isfinite(ht).all(), "non-finite layer output"
    log(f"ms/step {ms_step:.3f}  stages {json.dumps({n: round(v, 3) for n, v in stage_ms.items()})}")

    if args.gather == "threshold":
        # the timed step is exactly sgsa_layer_fwd: same kernels, same order, bit-identical result
        lbytes_ws = ctypes.c_size_t()
        _abi.check(L.sgsa_layer_fwd_workspace_size(_abi.SGSA_BF16, B, T, H, D, kk, ctypes.byref(lbytes_ws)))
        out_l, ht_l = torch.empty_like(out), torch.empty_like(ht)
        del ws
        lws = torch.empty(lbytes_ws.value, device=dev, dtype=torch.uint8)
        _abi.check(L.sgsa_layer_fwd(_abi.SGSA_BF16, B, T, H, D, kk, cfg["chunk"], P(qd), P(kd), P(vd), P(qd),
                                    P(bd), P(gd), P(ud), None, 0, 0.25, 0.1, P(out_l), P(ht_l), P(lws),
                                    lbytes_ws.value, stream))
        torch.cuda.synchronize()
        assert torch.equal(out, out_l) and torch.equal(ht, ht_l), "timed step differs from sgsa_layer_fwd"
        log("timed step reproduces sgsa_layer_fwd bit for bit")
        del lws, out_l, ht_l

    # the other K1/K2 form, for comparison (outside the timed steps)
    other_ms = None
    other_name = {"threshold": "tiled", "tiled": "direct", "direct": "tiled"}[args.gather]
    if args.steps > 0:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        other[0]()
        other[1]()
        ev[0].record(cur)
        for _ in range(3):
            other[0]()
        ev[1].record(cur)
        for _ in range(3):
            other[1]()
        ev[2].record(cur)
        torch.cuda.synchronize()
        other_ms = {"score_topk": round(ev[0].elapsed_time(ev[1]) / 3, 3),
                    "gather_gate": round(ev[1].elapsed_time(ev[2]) / 3, 3)}
        log(f"{other_name} form for comparison: {json.dumps(other_ms)} ms")

    # The north star's K2 is a gather of the selected K/V rows: time it beside the step (K1 row lists, then
    # the per-row 16-byte gather), outside the timed steps, for its HBM roofline.
    gather_form_ms = rows_k1_ms = None
    if args.steps > 0 and args.gather != "direct":
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        k1_rows()
        k2_direct()
        ev[0].record(cur)
        for _ in range(2):
            k1_rows()
        ev[1].record(cur)
        for _ in range(2):
            k2_direct()
        ev[2].record(cur)
        torch.cuda.synchronize()
        rows_k1_ms = ev[0].elapsed_time(ev[1]) / 2
        gather_form_ms = ev[1].elapsed_time(ev[2]) / 2
        log(f"row-list K1 {rows_k1_ms:.3f} ms; row gather K2 (sparse_gather_kernel) on its lists: "
            f"{gather_form_ms:.3f} ms")

    # HBM bytes per launch are not measured inside this run (that takes rocprofv3 --pmc): they are read
    # from the committed counter summary, which names the command that produced it, and labelled so.
    measured = {}
    traffic_source = None
    if args.traffic_from and os.path.exists(args.traffic_from) and (B, T, H, D, kk) == (1, 32768, 16, 128, 2048):
        with open(args.traffic_from) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch "):
                    name, val = line[len("hbm_bytes_per_launch "):].split(":", 1)
                    measured[name.strip()] = int(val)
        traffic_source = (f"{os.path.relpath(args.traffic_from, ROOT)} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, "
                          "copy-calibrated; a separate run of this code, not measured in this run)")
    gbytes = gather_bytes(B, H, T, D, kk)
    f_score = B * H * T * (T + 1) * D               # causal score GEMM, one pass
    f_chunk = B * H * ((T + 63) // 64) * 23.77e6     # chunk contractions (K3 + K5 + K4)
    gather_kernel = {"threshold": "gather_thr_kernel<false>", "tiled": "gather_list_kernel",
                     "direct": "sparse_gather_kernel<bf16_t, true, false>"}[args.gather]
    topk_kernel = {"threshold": "score_thr128_kernel<false>", "tiled": "score_topk_tiles_kernel<true, false>",
                   "direct": "score_topk_kernel<bf16_t, false, true, true, false, false, false>"}[args.gather]
    rooflines = {
        "score_topk": {"kernel": f"{topk_kernel} (K1)", "bound": "mfma",
                       "achieved": round(f_score / (stage_ms["score_topk"] / 1000.0) / 1e12, 2),
                       "peak": 2500.0, "unit": "TFLOP/s", "traffic": measured.get(topk_kernel),
                       "algorithmic_flops": f_score},
        # the threshold gather recomputes every causal score and multiplies the masked weights into K and V
        # (3 x F_score of MFMA work); the list forms gather k rows of K and V per query row (HBM-bound)
        "gather_gate": ({"kernel": f"{gather_kernel} (K2)", "bound": "mfma",
                         "achieved": round(3 * f_score / (stage_ms["gather_gate"] / 1000.0) / 1e12, 2),
                         "peak": 2500.0, "unit": "TFLOP/s", "traffic": measured.get(gather_kernel),
                         "algorithmic_flops": 3 * f_score}
                        if args.gather == "threshold" else
                        {"kernel": f"{gather_kernel} (K2)", "bound": "hbm",
                         "achieved": round(gbytes / (stage_ms["gather_gate"] / 1000.0) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "traffic": measured.get(gather_kernel),
                         "algorithmic_bytes": gbytes}),
        "chunk": {"kernel": "chunk kernels (K3-K5)", "bound": "mfma",
                  "achieved": round(f_chunk / (stage_ms["chunk"] / 1000.0) / 1e12, 2),
                  "peak": 2500.0, "unit": "TFLOP/s",
                  "traffic": (sum(v for n, v in measured.items() if n.startswith("chunk_")) or None),
                  "algorithmic_flops": f_chunk},
    }
    for r in rooflines.values():
        r["frac"] = round(r["achieved"] / r["peak"], 4)
        if r["traffic"] is not None:
            r["traffic_source"] = traffic_source
    if gather_form_ms is not None:
        # The north star's own K2: the selected K/V rows gathered per query row.  Its roofline is the HBM
        # bytes the counters see per launch over its measured time; the algorithmic gather bytes count
        # rows that neighbouring queries re-read from L2 / MALL, so bytes / time on them is an effective
        # rate, not a fraction of the HBM peak.
        gk = "sparse_gather_kernel<bf16_t, true, false>"
        rg = {"kernel": f"{gk} (K2 as a gather of the selected K/V rows, timed beside the step)",
              "ms": round(gather_form_ms, 3), "bound": "hbm", "achieved": None, "peak": HBM_PEAK_GBS,
              "unit": "GB/s", "frac": None, "traffic": measured.get(gk), "algorithmic_bytes": gbytes,
              "effective_GBps_on_algorithmic_bytes": round(gbytes / (gather_form_ms / 1000.0) / 1e9, 1)}
        if measured.get(gk):
            hb = measured[gk] / (gather_form_ms / 1000.0) / 1e9
            rg["achieved"] = round(hb, 1)
            rg["frac"] = round(hb / HBM_PEAK_GBS, 4)
            rg["traffic_source"] = traffic_source
        rooflines["row_gather_form"] = rg
    dominant = max(stage_ms, key=stage_ms.get)
    result = {
        "metric": METRIC,
        "value": round(B * T / (ms_step / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "sgsa_layer_fwd", "B": B, "T": T, "H": H, "D": D, "top_k": top_k,
                   "chunk": cfg["chunk"], "state": "fp32", "gather": args.gather},
        "stage_ms": {n: round(v, 3) for n, v in stage_ms.items()},
        "other_form": {"gather": other_name, "stage_ms": other_ms},
        # the north star's literal form of the layer, timed beside the step: row-list K1, the row gather
        # of the selected K/V rows, and the same chunk update
        "north_star_form_ms": (round(rows_k1_ms + gather_form_ms + stage_ms["chunk"], 3)
                               if gather_form_ms is not None else None),
        "roofline": rooflines[dominant],
        "rooflines": rooflines,
        "cpu_baseline": None,
    }
    if not args.no_other_configs and (B, T, H, D, kk) == (1, 32768, 16, 128, 2048):
        # BASELINE.json's other single-GPU configurations through the same layer path, outside the timed steps
        del idx, sc, tl, toff, tws
        torch.cuda.empty_cache()
        cpu = not args.no_cpu_baseline
        result["other_configs"] = [
            time_config("config 0", 1, 512, 4, 64, 32, torch.float32, cpu=cpu),
            time_config("config 1", 4, 8192, 16, 128, 256, torch.bfloat16, cpu=cpu),
            time_config("config 3", 1, 65536, 16, 128, 2048, torch.bfloat16, heavy=True, cpu=cpu),
        ]
        torch.cuda.empty_cache()
        # the headline shape with its first eighth of positions padded
        result["masked"] = time_masked(B, T, H, D, top_k, T // 8)
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log("cpu baseline (bounded sample)")
        result["cpu_baseline"] = cpu_baseline(q.to(bf), k.to(bf), v.to(bf), beta, gamma, budget, cfg)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
