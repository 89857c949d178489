#!/usr/bin/env python3
"""Throughput of the MI355X token-sampling path on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

One step = one fused sampling launch over one batch of synthetic logits
already resident in HBM (default workload: B=256 rows, V=128256 bf16 logits,
heterogeneous per-row temperature / top-k / top-p / min-p / repetition penalty
over 2048 history ids).  Several distinct input batches (> 256 MB together)
are rotated so that the 256 MB Infinity Cache cannot serve a repeated batch.

Prints one JSON line: rows/s (= sampled tokens/s) over exactly K timed steps
bracketed by device synchronisations, the dominant kernel's roofline (its
average launch duration from a HIP event pair on the launch stream around the
K back-to-back launches, against the algorithmic bytes of one launch and
MI355X's 8 TB/s HBM peak), and the CPU
baseline (the oracle's per-row restatement of the reference sampler, timed on
this host on a bounded sample of the same workload).

The default run then times the other configurations (B=64 V=32000 fp32 with
stop ids; B=512 V=262144 soft-capped fp32; speculative verify of 32 x 5
drafts at V=128256) with shorter timed regions, each under ``configs`` in
the same line with its own roofline, CPU baseline and parity counts
(``--headline-only`` skips them).  ``roofline.traffic`` is read from the
committed counter profile of the workload (``traffic_source`` says which).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
ISOLATED = 20  # launches timed one by one for the spread
METRIC = "sampled rows/sec at B=256,V=128256 mixed params; achieved HBM GB/s vs peak"
DEFAULT_WORKLOAD = "hetero_bf16_256x128256"
MALL_BYTES = 256 * 1024 * 1024
# timed after the headline in the default run, each with its own roofline
OTHER_CONFIGS = ("uniform_f32_64x32000", "softcap_zipf_f32_512x262144", "spec_f32_32x5x128256")


def _traffic_from_profile(workload: str):
    """HBM bytes per launch (per step, for a step of several kernels) measured
    by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel
    calibration), as recorded under profiles/ -- not
    measured in this run (counters need a profiler run of their own).
    Returns (bytes or None, source description)."""
    rel = os.path.join("profiles", f"{workload}_traffic.txt")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    if not os.path.exists(path):
        return None, "no counter profile recorded for this workload"
    val, date = None, ""
    for line in open(path):
        if line.startswith(("traffic_bytes_per_launch:", "traffic_bytes_per_step:")):
            val = float(line.split(":", 1)[1])
        elif line.startswith("measured:"):
            date = line.split(":", 1)[1].strip()
    return val, f"{rel} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of an earlier build, not this run" + \
        (f"; {date}" if date else "") + ")"


def _roofline(alg_bytes: int, ms: float, workload: str, **extra) -> dict:
    achieved = alg_bytes / (ms * 1e-3) / 1e9
    traffic, src = _traffic_from_profile(workload)
    return dict({"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                 "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": src,
                 "algorithmic_bytes": alg_bytes}, **extra)


def _timed_region(torch, dev, stream, K: int, launch):
    """K back-to-back launches bracketed by synchronisations (wall clock) and
    by one HIP event pair on the launch stream.  Returns (mean ms per launch
    from the events, wall seconds)."""
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    ev0.record(stream)
    for k in range(K):
        launch(k)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / K, wall


def _isolated_launches(torch, dev, stream, launch, n: int = ISOLATED):
    """Durations (ms, sorted) of n launches each bracketed by its own event
    pair, outside the timed region: the spread of a single launch (each pair
    adds a few microseconds of its own)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for k, (a, b) in enumerate(ev):
        a.record(stream)
        launch(k)
        b.record(stream)
    torch.cuda.synchronize(dev)
    return sorted(a.elapsed_time(b) for a, b in ev)


def cpu_baseline(w, seconds: float, got_tokens=None, got_mask=None):
    """The oracle's per-row restatement (one [1, V] call per row, as the
    reference inference engine makes them) on the first rows of the workload:
    the median rate of three segments of ``seconds / 3`` with all the threads
    torch uses, and one segment of ``seconds / 3`` on a single thread.

    ``got_tokens`` / ``got_mask`` (the GPU's tokens and keep bit-masks for the
    same batch): the oracle tokens of the rows the baseline sampled are
    checked against them, outside the timed segments, and the counts are
    returned under ``parity``."""
    import statistics

    import torch

    from oracle import sampler_oracle as O

    def row_params(w, b):
        hist = [] if w.history is None else [int(v) for v in w.history[b].tolist() if v >= 0]
        stops = [] if w.stop_ids is None else [int(v) for v in w.stop_ids.tolist()]
        return O.RowParams(float(w.temperature[b]), int(w.top_k[b]), float(w.top_p[b]), float(w.min_p[b]),
                           float(w.repetition_penalty[b]), hist, stops)

    x = w.logits.cpu()
    u = w.uniforms.cpu().tolist()
    params = [row_params(w, b) for b in range(w.batch)]
    # one warm-up row, then rows 0, 1, ... (cycling through the batch) until the time is spent
    O.sample_rows(x[:1], params[:1], u[:1], softcap=w.softcap, want_filtered=False)
    state = {"row": 0}

    oracle_tok = {}

    def segment(sec: float) -> float:
        rows = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < sec:
            b = state["row"] % w.batch
            r = O.sample_rows(x[b:b + 1], params[b:b + 1], u[b:b + 1], softcap=w.softcap, want_filtered=False)
            oracle_tok.setdefault(b, r[0].token)
            state["row"] += 1
            rows += 1
        return rows / (time.perf_counter() - t0)

    threads = torch.get_num_threads()
    rates = [segment(seconds / 3.0) for _ in range(3)]
    torch.set_num_threads(1)
    try:
        one = segment(seconds / 3.0)
    finally:
        torch.set_num_threads(threads)
    parity = None
    if got_tokens is not None:
        parity = _row_parity(w, x, params, u, oracle_tok, got_tokens, got_mask)
    return {"value": statistics.median(rates), "unit": "rows/s", "cores": threads, "kind": "port",
            "single_thread_value": one, "parity": parity,
            "sample": f"{state['row']} rows of {w.name} (seed 0, cycling through its {w.batch} rows), one [1,V] "
                      f"oracle call per row (torch {torch.__version__} CPU, ATEN_CPU_CAPABILITY "
                      f"{torch.backends.cpu.get_cpu_capability()}); value: median of 3 segments of "
                      f"{seconds / 3:.1f} s on {threads} threads ({', '.join(f'{r:.1f}' for r in rates)} rows/s); "
                      f"single_thread_value: one segment of {seconds / 3:.1f} s on 1 thread"}


def _row_parity(w, x, params, u, oracle_tok, got_tokens, got_mask=None):
    """EXACT / TIE / NEAR / CONSEQ / MISMATCH counts of the GPU tokens of the
    rows the CPU baseline sampled, against its oracle tokens (a differing
    token is classified with both keep masks and the rounding doubt)."""
    import torch

    from oracle import classify as C
    from oracle import sampler_oracle as O

    got = got_tokens.cpu().tolist()
    words = None if got_mask is None else got_mask.cpu().to(torch.int64) & 0xFFFFFFFF
    counts = {k: 0 for k in ("EXACT", "TIE", "NEAR", "CONSEQ", "MISMATCH")}
    for b, tok in sorted(oracle_tok.items()):
        if got[b] == tok:
            counts["EXACT"] += 1
            continue
        ref = O.sample_rows(x[b:b + 1], params[b:b + 1], u[b:b + 1], softcap=w.softcap)[0]
        keep = ~torch.isneginf(ref.filtered.float())
        gk = None
        if words is not None:
            gk = (((words[b].unsqueeze(-1) >> torch.arange(32)) & 1).reshape(-1)[:w.vocab]).bool()
        v = C.classify_row(x[b], params[b], u[b], keep, ref.token, gk, got[b], softcap=w.softcap)
        counts[v.kind] += 1
    counts["rows_checked"] = len(oracle_tok)
    counts["batch_rows"] = w.batch
    return counts


def cpu_baseline_spec(w, seconds: float, got=None):
    """The oracle's speculative verify (per sequence: filtered target and draft
    softmax at each examined position, accept test, residual or bonus draw) on
    the first sequences of the workload until ``seconds`` have been spent."""
    import torch

    from oracle import sampler_oracle as O

    p = O.RowParams(float(w.temperature), 0, float(w.top_p), 0.0, 1.0, [], [])
    O.speculative_verify(w.target[:1], w.draft[:1], w.draft_ids[:1], p, w.u_accept[:1], w.u_resample[:1])
    seqs = 0
    toks = 0
    results = {}
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        b = seqs % w.target.size(0)
        r = O.speculative_verify(w.target[b:b + 1], w.draft[b:b + 1], w.draft_ids[b:b + 1], p,
                                 w.u_accept[b:b + 1], w.u_resample[b:b + 1])[0]
        results.setdefault(b, r)
        toks += r.n_accepted + 1
        seqs += 1
    dt = time.perf_counter() - t0
    parity = None
    if got is not None:
        from oracle import classify as C
        n_acc, tokens = got[0].cpu().tolist(), got[1].cpu().tolist()
        counts = {"EXACT": 0, "NEAR": 0, "MISMATCH": 0}
        for b, r in sorted(results.items()):
            summ, _, _ = C.classify_spec(w.target[b:b + 1], w.draft[b:b + 1], w.draft_ids[b:b + 1], p,
                                         w.u_accept[b:b + 1], w.u_resample[b:b + 1], [n_acc[b]], [tokens[b]],
                                         ref=[r])
            for k in counts:
                counts[k] += summ[k]
        parity = dict(counts, sequences_checked=len(results), batch_sequences=w.target.size(0))
    return {"value": toks / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "parity": parity,
            "sample": f"{seqs} sequences of {w.name} (seed 0, cycling through its {w.target.size(0)}), one oracle "
                      f"verify per sequence (torch {torch.__version__} CPU, {torch.get_num_threads()} threads), "
                      f"{dt:.1f} s"}


def bench_spec(args, dev, name: str, steps: int, warmup: int, cpu_seconds: float):
    """Speculative verify: one step = the three launches of one batch (target
    rows with the bonus draw, draft rows, verify); tokens/s counts accepted
    drafts plus the resampled or bonus token of every sequence.  Returns the
    result dict, or None when a row failed."""
    import torch

    from rl_project_amd import sample_tokens, workloads
    from rl_project_amd.speculative import SpecPlan

    def draft_sampler(rows, u):
        # drafts drawn from the filtered draft distribution by the GPU sampler
        return sample_tokens(rows.to(dev), temperature=0.8, top_p=0.95, uniforms=u.to(dev)).tokens.cpu()

    ws = [workloads.make_spec(name, seed=0, draft_sampler=draft_sampler)]
    batch_bytes = (ws[0].target.numel() + ws[0].draft.numel()) * ws[0].target.element_size()
    nbuf = args.buffers or max(2, math.ceil(1.25 * MALL_BYTES / batch_bytes))
    for s in range(1, nbuf):
        ws.append(workloads.make_spec(name, seed=s, draft_sampler=draft_sampler))
    plans = []
    for w in ws:
        wd = w.to(dev)
        plans.append(SpecPlan(wd.target, wd.draft, wd.draft_ids, temperature=wd.temperature, top_p=wd.top_p,
                              u_accept=wd.u_accept, u_resample=wd.u_resample, return_ratio=False))
    stream = torch.cuda.current_stream(dev)
    for i in range(max(warmup, nbuf)):
        plans[i % nbuf].launch()
    torch.cuda.synchronize(dev)
    for pl in plans:
        if not bool(pl.status_ok().all()):
            print(f"{name}: speculative rows failed", file=sys.stderr)
            return None
    toks = [int((pl.n_accepted + 1).sum()) for pl in plans]

    K = steps
    step_ms, wall = _timed_region(torch, dev, stream, K, lambda k: plans[k % nbuf].launch())
    durs = _isolated_launches(torch, dev, stream, lambda k: plans[k % nbuf].launch())
    w = ws[0]
    B, Kd = w.draft_ids.shape
    n_tok = sum(toks[k % nbuf] for k in range(K))
    alg_bytes = w.algorithmic_bytes()
    result = {
        "metric": f"speculative verify tokens/sec at B={B}, K={Kd}, V={w.target.size(2)} fp32 (accepted + 1 per sequence)",
        "value": n_tok / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": warmup,
        "ms_per_step": wall * 1e3 / K,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": w.name, "sequences": B, "drafts": Kd, "vocab": w.target.size(2),
                   "input_buffers": nbuf, "tokens_per_step_mean": n_tok / K, "sequences_per_s": B * K / wall},
        "roofline": _roofline(alg_bytes, step_ms, w.name, step_ms_mean=step_ms,
                              isolated_step_ms_p10=durs[len(durs) // 10],
                              isolated_step_ms_p90=durs[(9 * len(durs)) // 10],
                              kernel="k_sample_rows32 (target and draft rows) + k_spec_verify"),
    }
    if not args.no_cpu_baseline:
        torch.cuda.synchronize(dev)
        plans[0].launch()      # the first batch's own outputs, checked against the oracle
        torch.cuda.synchronize(dev)
        result["cpu_baseline"] = cpu_baseline_spec(w, cpu_seconds, (plans[0].n_accepted, plans[0].tokens))
        result["parity"] = result["cpu_baseline"]["parity"]
    return result


def bench_rowstats(args, dev) -> int:
    """Full-distribution statistics of RL training: one step = the token
    log-probabilities and entropies of R positions of V-wide logits
    (rowstats_<dtype>_<R>x<V>; "_kl" adds KL to a reference model's logits,
    a second input of the same size)."""
    import torch

    from oracle import logprob_oracle as L
    from rl_project_amd import row_stats

    parts = args.workload.split("_")
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[parts[1]]
    R, V = (int(v) for v in parts[2].split("x"))
    kl = parts[-1] == "kl"
    esz = torch.empty(0, dtype=dt).element_size()
    per_buf = R * V * esz * (2 if kl else 1)
    nbuf = args.buffers or max(2, math.ceil(1.25 * MALL_BYTES / per_buf))
    bufs = []
    for s in range(nbuf):
        g = torch.Generator(device=dev).manual_seed(s)
        x = (2.5 * torch.randn(R, V, generator=g, device=dev)).to(dt)
        y = (x.float() + 0.5 * torch.randn(R, V, generator=g, device=dev)).to(dt) if kl else None
        lab = torch.randint(0, V, (R,), generator=g, device=dev)
        bufs.append((x, y, lab))
    launch = lambda k: row_stats(bufs[k % nbuf][0], bufs[k % nbuf][2], bufs[k % nbuf][1], entropy=True,  # noqa: E731
                                 check_labels=False)
    stream = torch.cuda.current_stream(dev)
    for i in range(max(args.warmup, nbuf)):
        launch(i)
    torch.cuda.synchronize(dev)
    K = args.steps
    kern_ms, wall = _timed_region(torch, dev, stream, K, launch)
    durs = _isolated_launches(torch, dev, stream, launch)
    alg_bytes = per_buf + R * (8 + 4 + 4 + (4 if kl else 0))
    result = {
        "metric": f"token log-prob + entropy{' + KL' if kl else ''} rows/sec over {R}x{V} {parts[1]} logits",
        "value": R * K / wall, "unit": "rows/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / K, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": parts[1], "data": "synthetic",
        "config": {"workload": args.workload, "rows": R, "vocab": V, "kl": kl, "input_buffers": nbuf},
        "roofline": _roofline(alg_bytes, kern_ms, args.workload, kernel_ms_mean=kern_ms,
                              isolated_launch_ms_p10=durs[len(durs) // 10],
                              isolated_launch_ms_p90=durs[(9 * len(durs)) // 10],
                              kernel=f"k_row_stats<{ {'bf16': 'BF16', 'f16': 'F16', 'f32': 'F32'}[parts[1]] }, "
                                     f"{str(kl).lower()}>"),
    }
    if not args.no_cpu_baseline:
        # the oracle (the reference's torch expressions) on the host, on the first rows
        x, y, lab = (t.cpu() if t is not None else None for t in bufs[0])
        rows = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            b = (rows % R)
            L.token_logprobs_from_logits(x[b:b + 16], lab[b:b + 16])
            L.entropy_from_logits(x[b:b + 16])
            if kl:
                L.kl_full_distribution(x[b:b + 16], y[b:b + 16])
            rows += 16
        dt_cpu = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": rows / dt_cpu, "unit": "rows/s", "cores": torch.get_num_threads(),
                                  "kind": "port", "sample": f"{rows} rows in 16-row calls of the oracle's "
                                  f"restatement (torch {torch.__version__} CPU, {torch.get_num_threads()} threads), "
                                  f"{dt_cpu:.1f} s"}
    print(json.dumps(result), flush=True)
    return 0


def bench_lmhead(args, dev) -> int:
    """The decode step's lm_head with the sampler in its epilogue
    (lmhead_bf16_<B>x<D>x<V>): one step = LmHeadPlan.launch() (history
    bitmap, sampled gemm, bound and raw-key thresholds, MFMA GEMM with the
    candidate epilogue, pick) for B rows of
    D-dimensional bf16 hidden states against a V x D bf16 weight, per-row
    top-k 1..64 with temperature, top-p, min-p and penalty.  Reported beside
    it: the unfused step (torch.matmul into [B, V] bf16 logits, then
    fl_sample over them)."""
    import torch

    from rl_project_amd.lmhead import LmHeadPlan
    from rl_project_amd.sampling import SamplerPlan

    parts = args.workload.split("_")
    B, D, V = (int(v) for v in parts[2].split("x"))
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(V, D, generator=g, device=dev) * (2.5 / D ** 0.5)).to(torch.bfloat16)
    gc = torch.Generator().manual_seed(1)
    kw = dict(temperature=torch.rand(B, generator=gc) * 1.4 + 0.1,
              top_k=torch.tensor([1, 5, 20, 50, 64], dtype=torch.int32)[torch.randint(0, 5, (B,), generator=gc)],
              top_p=torch.where(torch.rand(B, generator=gc) < 0.6, torch.rand(B, generator=gc) * 0.5 + 0.5,
                                torch.ones(B)),
              min_p=torch.where(torch.rand(B, generator=gc) < 0.3, torch.full((B,), 0.05), torch.zeros(B)),
              repetition_penalty=torch.rand(B, generator=gc) * 0.3 + 1.0,
              history=torch.randint(0, V, (B, 2048), generator=gc, dtype=torch.int32),
              uniforms=torch.rand(B, generator=gc))
    kd = {k: v.to(dev) for k, v in kw.items()}
    plan = LmHeadPlan(h, W, **kd)
    stream = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        plan.launch()
    torch.cuda.synchronize(dev)
    if int((plan.status != 0).sum()):
        print(f"rows failed: status {plan.status.tolist()[:16]}", file=sys.stderr)
        return 1
    K = args.steps
    step_ms, wall = _timed_region(torch, dev, stream, K, lambda k: plan.launch())
    durs = _isolated_launches(torch, dev, stream, lambda k: plan.launch())
    # the unfused step: GEMM into logits, then fl_sample
    logits = torch.empty(B, V, dtype=torch.bfloat16, device=dev)
    splan = SamplerPlan(logits, exact_repeat=False, **kd)   # (rows checked: status 0)

    def unfused(k):
        torch.matmul(h, W.t(), out=logits)
        splan.launch()
    for _ in range(args.warmup):
        unfused(0)
    unf_ms, _ = _timed_region(torch, dev, stream, K, unfused)
    gemm_ms, _ = _timed_region(torch, dev, stream, K, lambda k: torch.matmul(h, W.t(), out=logits))
    alg_bytes = V * D * 2 + B * D * 2 + B * 16
    flops = 2.0 * B * D * V
    result = {
        "metric": f"decode steps/sec: lm_head + sampling of {B} rows, D={D}, V={V} (bf16), no [B,V] logits in HBM",
        "value": K / wall, "unit": "steps/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / K, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": args.workload, "batch": B, "dim": D, "vocab": V, "history": 2048,
                   "tokens_per_s": B * K / wall},
        "roofline": _roofline(alg_bytes, step_ms, args.workload, step_ms_mean=step_ms,
                              isolated_step_ms_p10=durs[len(durs) // 10],
                              isolated_step_ms_p90=durs[(9 * len(durs)) // 10],
                              kernel="k_lm_prep + k_lm_sample + k_lm_thresh + k_lm_gemm + k_lm_pick",
                              mfma_tflops=flops / (step_ms * 1e-3) / 1e12, mfma_peak_tflops=2500.0),
        "unfused": {"ms_per_step": unf_ms, "matmul_ms": gemm_ms,
                    "note": "torch.matmul(h, W.T) into [B, V] bf16 logits, then fl_sample (SamplerPlan)"},
    }
    if not args.no_cpu_baseline:
        # the reference's step on the host: the float32 product rounded to bf16
        # logits, then the oracle's per-row filters and selection; the GPU's own
        # logits and tokens checked against the oracle
        from oracle import classify as C
        from oracle import sampler_oracle as O
        pl = LmHeadPlan(h, W, return_logits=True, **kd)
        pl.launch()
        torch.cuda.synchronize(dev)
        x = pl.logits.cpu()
        params = [O.RowParams(temperature=float(kw["temperature"][b]), top_k=int(kw["top_k"][b]),
                              top_p=float(kw["top_p"][b]), min_p=float(kw["min_p"][b]),
                              repetition_penalty=float(kw["repetition_penalty"][b]),
                              history=kw["history"][b].tolist()) for b in range(B)]
        ref = O.sample_rows(x, params, kw["uniforms"].tolist(), want_filtered=True)
        toks = pl.tokens.cpu().tolist()
        verdicts = [C.classify_row(x[b], params[b], float(kw["uniforms"][b]), ~torch.isneginf(ref[b].filtered.float()),
                                   ref[b].token, None, toks[b]) for b in range(B)]
        result["parity"] = C.summarise(verdicts)
        hc, Wc = h.float().cpu(), W.float().cpu()
        steps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or steps == 0:
            xl = (hc @ Wc.t()).to(torch.bfloat16)
            O.sample_rows(xl, params, kw["uniforms"].tolist(), want_filtered=False)
            steps += 1
        dt_cpu = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": steps / dt_cpu, "unit": "steps/s", "cores": torch.get_num_threads(),
                                  "kind": "port", "sample": f"{steps} steps of float32 torch.matmul + the oracle's "
                                  f"per-row sampling (torch {torch.__version__} CPU, {torch.get_num_threads()} "
                                  f"threads), {dt_cpu:.1f} s"}
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD)
    ap.add_argument("--buffers", type=int, default=0, help="distinct input batches (default: > 256 MB in total)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time (3 segments; a fourth on 1 thread)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the default workload (skip the other configurations)")
    ap.add_argument("--other-steps", type=int, default=50, help="timed steps of each other configuration")
    ap.add_argument("--other-cpu-seconds", type=float, default=6.0,
                    help="CPU baseline time of each other configuration")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run an elementwise read+write kernel (torch.neg) over MIB MiB, 5 launches: the "
                         "known-size kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: rows of a sampling batch are independent, so the path shards by "
              f"rows with no communication; --gpus {args.gpus} (WORLD_SIZE={world}) is not run.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.arange(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize(dev)
        print(json.dumps({"calibrate_copy_bytes": 4 * n, "launches": 5}), flush=True)
        return 0
    if args.workload.startswith("spec_"):
        res = bench_spec(args, dev, args.workload, args.steps, args.warmup, args.cpu_seconds)
        if res is None:
            return 1
        print(json.dumps(res), flush=True)
        return 0
    if args.workload.startswith("rowstats_"):
        return bench_rowstats(args, dev)
    if args.workload.startswith("lmhead_"):
        return bench_lmhead(args, dev)
    result = bench_rows(args, dev, args.workload, args.steps, args.warmup, args.cpu_seconds)
    if result is None:
        return 1
    result["metric"] = METRIC if args.workload == DEFAULT_WORKLOAD else result["metric"]
    if args.workload == DEFAULT_WORKLOAD and not args.headline_only:
        # the other configurations, after the headline's timed region, with
        # shorter timed regions and CPU samples: each its own roofline and
        # parity counts
        import torch

        result["configs"] = {}
        for name in OTHER_CONFIGS:
            torch.cuda.empty_cache()
            t0 = time.perf_counter()
            if name.startswith("spec_"):
                r = bench_spec(args, dev, name, args.other_steps, 5, args.other_cpu_seconds)
            else:
                r = bench_rows(args, dev, name, args.other_steps, 5, args.other_cpu_seconds)
            if r is None:
                return 1
            r["bench_seconds"] = time.perf_counter() - t0
            for k in ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "data"):
                r.pop(k, None)
            result["configs"][name] = r
            print(f"{name}: {r['value']:.4g} {r['unit']}, {r['ms_per_step']:.4f} ms/step", file=sys.stderr,
                  flush=True)
    print(json.dumps(result), flush=True)
    return 0


def bench_rows(args, dev, name: str, steps: int, warmup: int, cpu_seconds: float):
    """One step = one fl_sample launch over a batch of workload ``name``
    (input batches rotated past the Infinity Cache).  Returns the result dict,
    or None when a row of any rotated batch reports a status bit."""
    import torch

    from rl_project_amd import workloads
    from rl_project_amd.sampling import SamplerPlan

    w = workloads.make(name, seed=0)
    batch_bytes = w.logits.numel() * w.logits.element_size()
    nbuf = args.buffers or max(2, math.ceil(1.25 * MALL_BYTES / batch_bytes))
    wd = w.to(dev)
    bufs = [wd.logits]
    for s in range(1, nbuf):
        bufs.append(workloads.make(name, seed=s).logits.to(dev))
    kw = wd.kwargs()
    # (no exact-count repeat: every row of every rotated batch is checked
    # below for FL_ROW_LIMIT, the only status the repeat would act on)
    plans = [SamplerPlan(buf, exact_repeat=False, **kw) for buf in bufs]
    stream = torch.cuda.current_stream(dev)

    for i in range(max(warmup, nbuf)):
        plans[i % nbuf].launch()
    torch.cuda.synchronize(dev)
    for j, pl in enumerate(plans):
        status = pl.output.status
        if int((status != 0).sum()):
            print(f"{name}: rows of batch {j} failed: status {status.tolist()[:16]}", file=sys.stderr)
            return None

    K = steps
    kern_ms, wall = _timed_region(torch, dev, stream, K, lambda k: plans[k % nbuf].launch())
    durs = _isolated_launches(torch, dev, stream, lambda k: plans[k % nbuf].launch())

    B = w.batch
    alg_bytes = w.algorithmic_bytes()
    dtype = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[w.logits.dtype]
    result = {
        "metric": f"sampled rows/sec at B={B},V={w.vocab} ({name}); achieved HBM GB/s vs peak",
        "value": B * K / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": warmup,
        "ms_per_step": wall * 1e3 / K,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": w.name, "batch": B, "vocab": w.vocab,
                   "history": 0 if w.history is None else int(w.history.size(1)),
                   "input_buffers": nbuf, "tokens_per_s": B * K / wall,
                   "status_checked": f"every row of all {nbuf} rotated batches: 0"},
        "roofline": _roofline(alg_bytes, kern_ms, w.name, kernel_ms_mean=kern_ms,
                              isolated_launch_ms_p10=durs[len(durs) // 10],
                              isolated_launch_ms_p90=durs[(9 * len(durs)) // 10],
                              kernel=f"k_sample_rows16<{dtype.upper()}, {str(w.softcap > 0).lower()}>"
                              if w.logits.element_size() == 2 else "k_sample_rows32"),
    }
    if not args.no_cpu_baseline:
        from rl_project_amd import filtered_outputs
        plans[0].launch()      # the first batch's own tokens and keep masks, checked against the oracle
        kw_mask = dict(kw)
        kw_mask.pop("uniforms")
        _, _, mask0, _ = filtered_outputs(bufs[0], want_filtered=False, want_mask=True, **kw_mask)
        torch.cuda.synchronize(dev)
        result["cpu_baseline"] = cpu_baseline(w, cpu_seconds, plans[0].output.tokens.clone(), mask0)
        result["parity"] = result["cpu_baseline"]["parity"]
    del plans, bufs, wd
    return result


if __name__ == "__main__":
    sys.exit(main())
