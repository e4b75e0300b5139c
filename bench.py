"""Benchmark of the batched sampling step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3]

A step is one call of ``lmrs_sample_fwd`` (the C-ABI entry point) over the
whole batch of the configuration: penalties, temperature, top-k, top-p and the
draw for every row, logits already resident in HBM.  The logits are generated
once (synthetic, seeded) and replicated into enough rotating buffers that the
rotation exceeds the 256 MB last-level (MALL) cache, so every step streams its
logits from HBM.  The timed region is bracketed by HIP events recorded on the
stream the kernels are launched on.

Prints one JSON line: rows/s of the whole job, microseconds per step, the HBM
roofline of the step (algorithmic bytes / step time against 8 TB/s; measured
HBM traffic per launch from the committed rocprofv3 counter summary of the
same kernel and workload, named in traffic_source) and the
CPU baseline: the C restatement of the reference's CPU sampler timed on this
host's cores on a bounded sample of the same rows, whose tokens are also
compared with the GPU's.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak
LLC_BYTES = 256 << 20  # MI355X Infinity Cache (MALL)
METRIC = "sampled rows/sec + µs/step + % HBM peak, batch 256 × vocab 128256 bf16"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def workload_config(w) -> dict:
    desc = {
        "C1": "C1: batch 1 x vocab 32000 f32, T=0.8, top_k=50, top_p=0.9",
        "C2": "C2: batch 64 x vocab 128256 bf16 Student-t, per-row T, top_k, top_p",
        "C3": ("C3: batch 256 x vocab 128256 bf16 N(0,2.5^2), history 2048 Zipf(1.1) ids/row, "
               "repetition 1.1, presence 0.5, frequency 0.3, T=0.7, top_k=50, top_p=0.95"),
        "C4": "C4: batch 1024 x vocab 151936 bf16, half greedy, half full multinomial",
        "C5": "C5: batch 512 x vocab 256000 f32, top_p=0.99, repetition 1.05 over 512 ids/row",
    }[w.name]
    return {"workload": desc, "batch": w.batch, "vocab": w.vocab, "logits_dtype": w.dtype,
            "history_per_row": w.hist_len}


def kernel_label(w) -> str:
    """The kernel lmrs_sample_fwd launches for this workload (its dispatch rule)."""
    if w.dtype == "bf16" and w.vocab % 8 == 0 and 0 < w.vocab <= 40 * 4096:
        nch = next(n for n in (8, 16, 32, 40) if w.vocab <= n * 4096)
        if nch == 40 and w.batch > 256:  # more rows than MI355X's CUs: the persistent launch
            return f"bf16_fast_rounds_kernel<{nch}> (one launch per step)"
        return f"bf16_fast_kernel<{nch}> (one launch per step)"
    if w.dtype == "bf16":
        return "generic_sample_kernel<0> (one launch per step)"
    return "f32_sample_kernel (one launch per step)"


def traffic_file(w) -> str:
    """The committed counter summary of this workload's kernel (profiles/)."""
    kernel = kernel_label(w).split("<")[0].split(" ")[0]
    suffix = "_generic" if (w.name == "C3" and w.vocab != 128256) else ""
    return os.path.join(ROOT, "profiles", f"traffic_{kernel}_{w.name}{suffix}.txt")


def read_traffic(w):
    """HBM bytes per launch from the committed counter summary of the same
    kernel and workload (rocprofv3 FETCH_SIZE and WRITE_SIZE runs, scaled by
    a device copy's counters); None if absent."""
    path = traffic_file(w)
    if not os.path.exists(path):
        return None, None
    m = re.search(r"^traffic_bytes_per_launch\s*=\s*([0-9.]+)", open(path).read(), re.M)
    return (float(m.group(1)) if m else None), os.path.relpath(path, ROOT)


def cpu_baseline(w, gpu_out, seconds: float):
    """Times the oracle (the C restatement of the reference's CPU sampler) on
    the workload's rows, and compares its tokens with the GPU's.  Two legs of
    about `seconds` of wall time each: every available core with one row per
    thread at a time, and one thread with the rows in order, as the
    reference's worker samples a batch (crates/engine/src/worker/worker.rs:
    137-157).  The first is `cpu_baseline`; the second is reported beside it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from helpers import compare, run_oracle

    host_cores = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = host_cores
    # the GPU box grants 16 cores to a one-GPU job whatever the host has
    threads = max(1, min(16, affinity))

    def timed(nthreads, limit):
        t0 = time.perf_counter()
        ref = run_oracle(w, threads=nthreads)
        passes, dt = 1, time.perf_counter() - t0
        while dt < limit:
            run_oracle(w, threads=nthreads)
            passes += 1
            dt = time.perf_counter() - t0
        return ref, passes, dt

    ref, passes, dt = timed(threads, seconds)
    _, passes1, dt1 = timed(1, seconds)
    n = w.batch
    gpu = {k: v[:n] for k, v in gpu_out.items()}
    rep = compare(gpu, ref)
    base = {"value": passes * n / dt, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{passes} passes over all {n} rows of {w.name} ({dt:.1f} s, {threads} threads, "
                      f"oracle/lmrs_oracle.c sample_batch, one row per thread at a time)",
            "host_cores": host_cores, "affinity_cores": affinity,
            "one_thread": {"value": passes1 * n / dt1, "unit": "rows/s", "cores": 1,
                           "sample": f"{passes1} passes over all {n} rows in order on one thread ({dt1:.1f} s)"}}
    parity = {k: rep[k] for k in ("rows", "status_mismatch", "token_mismatch", "boundary_rows",
                                  "boundary_mismatch", "logit_mismatch", "max_prob_rel_err", "gpu_flagged")}
    return base, parity


def stream_ceiling(bufs, steps: int, warmup: int, dev) -> float:
    """GB/s of a read-only kernel with the sampler's access shape (one
    512-thread workgroup per row, pipelined non-temporal 16-byte loads:
    lmrs_amd/csrc/stream_probe.hip) over the same rotating buffers, timed like
    the step on its own stream.  None when the probe library is not built."""
    import ctypes

    import torch

    path = os.path.join(ROOT, "lmrs_amd", "liblmrs_stream_probe.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    L.lmrs_stream_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                    ctypes.c_void_p, ctypes.c_void_p]
    L.lmrs_stream_probe.restype = ctypes.c_int
    rows = bufs[0].shape[0]
    row_bytes = bufs[0].shape[1] * bufs[0].element_size()
    stride = bufs[0].stride(0) * bufs[0].element_size()
    if row_bytes % 16 or row_bytes // 16 > 40 * 512:  # beyond the probe's register-resident shapes
        return None
    out = torch.empty(rows, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream(device=dev)

    def launch(i):
        rc = L.lmrs_stream_probe(ctypes.c_void_p(bufs[i % len(bufs)].data_ptr()), row_bytes, stride, rows,
                                 ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(s.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"lmrs_stream_probe failed with code {rc}")

    with torch.cuda.stream(s):
        for i in range(warmup):
            launch(i)
        s.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(steps):
            launch(i)
        e1.record(s)
        e1.synchronize()
    ms = e0.elapsed_time(e1) / max(1, steps)
    log(f"bench: streaming read of one buffer (probe) {ms * 1e3:.1f} us")
    return rows * row_bytes / (ms * 1e-3) / 1e9


def copy_calibration(size_mb: int, reps: int) -> None:
    """A plain device copy of known size, for scaling the FETCH_SIZE /
    WRITE_SIZE counters to bytes (run under rocprofv3 --pmc)."""
    import torch

    n = size_mb << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "reps": reps}), flush=True)


def lm_head_bench(steps: int, warmup: int) -> dict:
    """Times lmrs_lm_head_fwd (the LM head's projection with the sampling
    prologue in its epilogue) at C3's rows and vocab with a 4096-wide hidden
    state: 256 x 4096 x 128256, two weight matrices in rotation (2.1 GB, over
    the MALL).  Reported beside the metric, never as it."""
    import torch

    from lmrs_amd import sampling as S

    rows, K, V = 256, 4096, 128256
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(rows, K, device=dev, generator=g).to(torch.bfloat16)
    ws = [(torch.randn(V, K, device=dev, generator=g) * (2.5 / K ** 0.5)).to(torch.bfloat16) for _ in range(2)]
    s = torch.cuda.Stream(device=dev)
    res = {}
    for fused in (True, False):
        with torch.cuda.stream(s):
            for i in range(warmup):
                S.lm_head(x, ws[i % 2], tile_max=fused, stream=s)
            s.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for i in range(steps):
                S.lm_head(x, ws[i % 2], tile_max=fused, stream=s)
            e1.record(s)
            e1.synchronize()
        res["fused" if fused else "plain"] = e0.elapsed_time(e1) / steps * 1e3
    us = res["fused"]
    flops = 2.0 * rows * K * V
    nbytes = V * K * 2 + rows * K * 2 + rows * V * 2 + rows * ((V + 63) // 64) * 8
    log(f"bench: lm_head {rows}x{K}x{V}: {us:.1f} us with the tile maxima, {res['plain']:.1f} us without")
    return {"kernel": "lm_head_kernel (lmrs_lm_head_fwd)", "shape": [rows, K, V], "us": us,
            "us_without_tile_max": res["plain"],
            "mfma": {"achieved": flops / (us * 1e-6) / 1e12, "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": flops / (us * 1e-6) / 1e12 / 2500.0},
            "hbm": {"achieved": nbytes / (us * 1e-6) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, "bytes": nbytes}}


def decode_bench(logits, steps: int) -> dict:
    """Times the engine's decode step end to end (lmrs_amd.engine.DecodeBatch.step:
    uniforms from each sequence's LCG, the launch, the outputs back on the
    host, the tokens appended to the device-resident histories) over 256
    sequences sampling from the workload's logits with T = 0.7 and top-k 50
    (the engine maps a request to one strategy, generation.rs:352-365).
    Reports the host wall time per step."""
    import statistics

    import torch

    from lmrs_amd import engine as E

    n = logits.shape[0]
    cfg = E.GenerationConfig(max_tokens=steps + 10, temperature=0.7, top_p=1.0, top_k=50)
    seqs = [E.SequenceState(cfg, seed=1 + i) for i in range(n)]
    batch = E.DecodeBatch(seqs)
    for _ in range(steps):
        batch.step(logits)
    torch.cuda.synchronize()
    t = sorted(batch.timings[3:]) or batch.timings
    med = statistics.median(t) * 1e6
    log(f"bench: decode step (DecodeBatch.step, {n} sequences, host wall) median {med:.1f} us")
    return {"sequences": n, "steps": len(batch.timings), "host_us_median": med,
            "host_us_p10": t[int(0.1 * (len(t) - 1))] * 1e6, "host_us_p90": t[int(0.9 * (len(t) - 1))] * 1e6,
            "history_len_at_end": len(seqs[0].generated),
            "what": "DecodeBatch.step wall time on the host: uniforms, one launch, one copy of the four "
                    "outputs back, in-place appends to the device histories"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C3", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--vocab", type=int, default=0,
                    help="keep only the first VOCAB logits of every row (e.g. an odd vocab on C3 runs the "
                         "generic bf16 kernel); a parity and counter case, not the metric")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--decode", type=int, metavar="STEPS", default=0,
                    help="also time the engine's decode step end to end (host wall) over STEPS steps "
                         "on the workload's logits; reported as 'decode_step'")
    ap.add_argument("--lm-head", action="store_true",
                    help="also time the LM head's projection with the fused sampling prologue "
                         "(256 x 4096 x 128256 bf16); reported as 'lm_head', not as the metric")
    ap.add_argument("--copy-calibration", type=int, metavar="MB", default=0,
                    help="run only a device copy of MB megabytes (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} (WORLD_SIZE {world}) is not supported; "
              "the sampling step has no cross-GPU part (rows are independent) -- run with --gpus 1",
              file=sys.stderr, flush=True)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, max(1, args.steps))
        return 0

    from lmrs_amd import sampling as S
    from lmrs_amd import workloads as W

    S.lib()  # fails loudly when the HIP library is not built
    w = W.CONFIGS[args.config]()
    if args.vocab:
        w = w.truncated(args.vocab)
    log(f"bench: {args.config} batch {w.batch} vocab {w.vocab} {w.dtype} ({kernel_label(w)})")
    dev = torch.device("cuda", 0)
    if w.dtype == "bf16":
        import numpy as np

        base = torch.from_numpy(w.logits.view(np.int16)).view(torch.bfloat16).to(dev)
    else:
        base = torch.from_numpy(w.logits).to(dev)
    nbytes = base.numel() * base.element_size()
    nrot = max(1, -(-2 * LLC_BYTES // nbytes))  # rotation covers twice the MALL
    bufs = [base] + [base.clone() for _ in range(nrot - 1)]
    off = ids = None
    if w.hist_offsets is not None:
        import numpy as np

        off = torch.from_numpy(w.hist_offsets.astype(np.int64)).to(dev)
        ids = torch.from_numpy(w.hist_ids.astype(np.uint32).view(np.int32)).to(dev)
    params = {k: torch.from_numpy(getattr(w, k)).to(dev) for k in
              ("repetition_penalty", "presence_penalty", "frequency_penalty", "temperature", "top_k", "top_p",
               "uniforms")}
    out = None
    batches = []
    for b in bufs:
        pb = S.prepare_batch(b, hist_offsets=off, hist_ids=ids, out=out, **params)
        out = pb.out
        batches.append(pb)

    stream = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    # The timed steps run back to back on one stream; an event every
    # GROUP steps gives the spread (median, p10, p90 of the group means)
    # without a gap between steps.
    GROUP = 10
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            batches[i % nrot].launch(stream)
        stream.synchronize()
        events = [torch.cuda.Event(enable_timing=True)]
        torch.cuda.synchronize()
        events[0].record(stream)
        for i in range(args.steps):
            batches[i % nrot].launch(stream)
            if (i + 1) % GROUP == 0 or i + 1 == args.steps:
                events.append(torch.cuda.Event(enable_timing=True))
                events[-1].record(stream)
        events[-1].synchronize()
    torch.cuda.synchronize()
    ms = events[0].elapsed_time(events[-1]) / max(1, args.steps)
    sizes = [GROUP] * (args.steps // GROUP) + ([args.steps % GROUP] if args.steps % GROUP else [])
    group_us = sorted(1e3 * events[j].elapsed_time(events[j + 1]) / sizes[j] for j in range(len(sizes)))
    pct = lambda q: group_us[min(len(group_us) - 1, int(q * (len(group_us) - 1) + 0.5))]  # noqa: E731
    spread = {"median": pct(0.5), "p10": pct(0.1), "p90": pct(0.9), "unit": "us/step",
              "over": f"{len(sizes)} groups of up to {GROUP} back-to-back steps"}
    log(f"bench: {args.steps} steps, {ms * 1e3:.1f} us/step (median {spread['median']:.1f}, "
        f"p10 {spread['p10']:.1f}, p90 {spread['p90']:.1f})")
    ceiling = stream_ceiling(bufs, args.steps, args.warmup, dev)

    # outputs of the last step (every rotation holds the same logits)
    res = {
        "token_id": out["token_ids"].cpu().numpy().view("uint32"),
        "log_prob": out["log_probs"].cpu().numpy(),
        "logit": out["logits"].cpu().numpy(),
        "status": out["status"].cpu().numpy(),
    }
    alg = w.algorithmic_bytes()
    achieved = alg / (ms * 1e-3) / 1e9
    traffic, traffic_src = read_traffic(w)
    line = {
        "metric": METRIC,
        "value": w.batch / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "us_per_step": ms * 1e3,
        "us_per_step_spread": spread,
        "hbm_peak_pct": 100.0 * achieved / HBM_PEAK_GBS,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == "bf16" else "f32",
        "data": "synthetic (seeded generator of the configuration's distributions)",
        "config": workload_config(w),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_src,
                     "algorithmic_bytes": alg, "kernel": kernel_label(w)},
        "rotating_buffers": nrot,
        # secondary denominator: the measured read rate of the same rotating
        # buffers by a load-only kernel of the sampler's access shape
        "stream_ceiling": {"achieved": ceiling, "unit": "GB/s",
                           "kernel": "lmrs_stream_probe (the load pass alone, same access shape)",
                           "frac": (alg / (ms * 1e-3) / 1e9) / ceiling if ceiling else None},
    }
    if args.lm_head:
        line["lm_head"] = lm_head_bench(max(5, args.steps // 10), 3)
    if args.decode:
        line["decode_step"] = decode_bench(bufs[0], args.decode)
    if not args.no_cpu:
        log("bench: CPU baseline (oracle) ...")
        line["cpu_baseline"], line["parity_sample"] = cpu_baseline(w, res, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
