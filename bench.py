"""Benchmark of the ChunkGatedDeltaRuleFwdH hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--op fwd_h|chunk_o|wy|forward]

A step is one FwdH call over the long-context prefill workload
B=1, T=32768, H=Hg=32, K=V=128, bf16 k/w/u, fp32 g (head-major), h0=None, final state on
(512 chunks per sequence walked inside the kernel).  Inputs are synthetic (seeded, the
distributions of the CPU-runnable reference case) and resident in HBM before timing.
Prints one JSON line: whole-job tokens/s, the dominant kernel's achieved HBM bandwidth
against MI355X's 8 TB/s, and the CPU oracle (numpy restatement of the reference chunk loop)
timed on this host's cores on a bounded sample of the same workload.

``--op chunk_o`` measures the chunk output (the consumer of FwdH's h and v_new) on the same
workload shape instead: q, k [1,32768,32,128], v_new [1,32768,32,128], h [1,512,32,128,128]
bf16 and fp32 g in HBM, one cgdr_chunk_o launch per step, with its own roofline and the numpy
oracle's chunk_o as the CPU baseline.  ``--op wy`` measures the WY producer (k, v, beta, the
per-token log-decay -> w, u, g) and ``--op forward`` the whole chunked forward (WY -> FwdH ->
chunk output, q k v beta g -> o and the final state) on the same shape.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cann-operator-challenge-august_amd"))

METRIC = "tokens/sec + achieved HBM GB/s at B=1,T=32k,H=32,K=V=128 bf16 (1 GPU)"
HBM_PEAK_GBPS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
F32_MFMA_PEAK_TFLOPS = 157.3   # dense fp32 MFMA, MI355X
WORKLOAD = dict(B=1, T=32768, H=32, Hg=32, K=128, V=128, chunk_size=64)


def algorithmic_bytes(B, T, H, Hg, K, V, NT, N, s_in=2, s_out=2, h0_bytes=0, final_bytes=4):
    """Each tensor counted once: k, w, u, g read; h, v_new, final written; h0 read if given."""
    return (B * T * (Hg * K + H * K + H * V) * s_in + 4 * B * T * H + N * H * K * V * h0_bytes
            + B * NT * H * K * V * s_out + B * T * H * V * s_out + N * H * K * V * final_bytes)


def algorithmic_flops(B, NT, H, K, V):
    return B * NT * H * 4 * 64 * K * V


def make_inputs(torch, dev, B, T, H, Hg, K, V, seed=0):
    """Synthetic inputs on the device: k L2-normalised randn, w = randn K^-1/2, u = randn,
    g = chunk-local cumsum of logsigmoid(randn) (non-increasing, <= 0 within each chunk),
    stored head-major."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    k = torch.randn(B, T, Hg, K, device=dev, generator=gen)
    k = torch.nn.functional.normalize(k, dim=-1).to(torch.bfloat16)
    w = (torch.randn(B, T, H, K, device=dev, generator=gen) * K ** -0.5).to(torch.bfloat16)
    u = torch.randn(B, T, H, V, device=dev, generator=gen).to(torch.bfloat16)
    inc = torch.nn.functional.logsigmoid(torch.randn(B, T, H, device=dev, generator=gen))
    NT = (T + 63) // 64
    pad = NT * 64 - T
    inc = torch.nn.functional.pad(inc, (0, 0, 0, pad)).view(B, NT, 64, H)
    g = inc.cumsum(dim=2).view(B, NT * 64, H)[:, :T]
    # g stored head-major ([B,H,T] memory, the layout of the contest run() and of the WY
    # producer's output), passed as a [B,T,H] view: the library reads it in place
    g = g.transpose(1, 2).contiguous().transpose(1, 2)
    return k, w, u, g


# FwdH workloads besides the headline prefill (each FwdH configuration at its own shape):
# two bf16 sequences with h0; 16 packed sequences of seeded lengths in [64, 8192] (none a
# multiple of 64) with per-sequence h0; wide value heads with a strongly decaying gate.
FWD_H_WORKLOADS = {
    "prefill": dict(desc="ChunkGatedDeltaRuleFwdH long-context prefill", B=1, T=32768, H=32, Hg=32, K=128,
                    V=128, h0=False, shift=0.0),
    "two_seq": dict(desc="ChunkGatedDeltaRuleFwdH two bf16 sequences with h0", B=2, T=2048, H=16, Hg=16,
                    K=128, V=128, h0=True, shift=0.0),
    "varlen": dict(desc="ChunkGatedDeltaRuleFwdH 16 packed sequences of lengths U[64,8192] with per-sequence h0",
                   B=1, T=None, H=32, Hg=32, K=128, V=128, h0=True, shift=0.0, n_seq=16),
    "wide_v": dict(desc="ChunkGatedDeltaRuleFwdH wide value heads, gate logsigmoid(randn-2)", B=4, T=8192, H=8,
                   Hg=8, K=128, V=256, h0=True, shift=-2.0),
    # the fp32 kernel (fp32 k/w/u/h/v_new): the CPU-runnable reference case and config 1's shape
    "config0_fp32": dict(desc="ChunkGatedDeltaRuleFwdH fp32, the CPU-runnable case", B=1, T=256, H=2, Hg=2, K=64,
                         V=64, h0=True, shift=0.0, dtype="f32"),
    "config1_fp32": dict(desc="ChunkGatedDeltaRuleFwdH fp32 at B=2, T=2048, H=16, K=V=128", B=2, T=2048, H=16,
                         Hg=16, K=128, V=128, h0=True, shift=0.0, dtype="f32"),
}


def make_workload_inputs(torch, dev, name: str, seed: int = 0):
    """Synthetic inputs of one FwdH workload, resident on the device (the distributions of
    make_inputs; g the chunk-local cumsum of logsigmoid(randn + shift), per sequence, stored
    head-major; h0 = randn * 0.1 fp32).  Returns (tensors, sizes); cu_seqlens stays on the host."""
    c = FWD_H_WORKLOADS[name]
    B, H, Hg, K, V = c["B"], c["H"], c["Hg"], c["K"], c["V"]
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    cu = None
    if c.get("n_seq"):
        lens = torch.randint(64, 8193, (c["n_seq"],), generator=gen)
        lens = torch.where(lens % 64 == 0, torch.where(lens < 8192, lens + 1, lens - 1), lens)
        cu = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)])
        T = int(cu[-1])
    else:
        T = c["T"]
        cu = None
    bounds = [(int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1)] if cu is not None else [(0, T)]
    N = len(bounds) if cu is not None else B
    NT = sum((e - s + 63) // 64 for s, e in bounds)
    k = torch.nn.functional.normalize(torch.randn(B, T, Hg, K, generator=gen), dim=-1)
    w = torch.randn(B, T, H, K, generator=gen) * K ** -0.5
    u = torch.randn(B, T, H, V, generator=gen)
    inc = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + c["shift"])
    g = torch.empty_like(inc)
    for s, e in bounds:          # chunk-local cumsum within each sequence
        L = e - s
        pad = (L + 63) // 64 * 64 - L
        x = torch.nn.functional.pad(inc[:, s:e], (0, 0, 0, pad)).view(B, -1, 64, H).cumsum(dim=2)
        g[:, s:e] = x.view(B, -1, H)[:, :L]
    h0 = torch.randn(N, H, K, V, generator=gen) * 0.1 if c["h0"] else None
    dt = torch.float32 if c.get("dtype") == "f32" else torch.bfloat16
    t = dict(k=k.to(dev, dt), w=w.to(dev, dt), u=u.to(dev, dt),
             g=g.to(dev).transpose(1, 2).contiguous().transpose(1, 2),
             initial_state=None if h0 is None else h0.to(dev), cu_seqlens=cu)
    return t, dict(B=B, T=T, H=H, Hg=Hg, K=K, V=V, N=N, NT=NT, chunk_size=64)


CPU_SAMPLE_SECONDS = 10.0


def head_parallel_cpu(run, n_heads: int, group: int, T: int, repeats: int, what: str):
    """Time an oracle over heads [0, n_heads) of T tokens on the host's cores.

    Heads are split over worker threads that each run single-threaded BLAS: the oracle's
    per-chunk GEMMs are too small for multi-threaded BLAS, which ran slower than one thread.
    The worker count is chosen by a sweep on the first min(T, 4096) tokens (each count timed
    twice, the faster run kept); the chosen count
    is then timed on all T tokens (median of at least `repeats` runs after that warm-up, and of
    at least CPU_SAMPLE_SECONDS of timed runs).  `run(lo, hi, t)`
    runs the oracle on heads [lo, hi) and the first t tokens; `group` keeps head slices whole
    multiples of the heads that share a key head."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    cores = len(os.sched_getaffinity(0))
    counts = [c for c in (1, 2, 4, 8, 16, 32, 64) if c <= min(cores, n_heads // group)]

    def timed(nw, t):
        units = n_heads // group
        cuts = [group * (units * i // nw) for i in range(nw + 1)]
        with ThreadPoolExecutor(nw) as ex:
            t0 = time.perf_counter()
            list(ex.map(lambda i: run(cuts[i], cuts[i + 1], t), range(nw)))
            return time.perf_counter() - t0

    ts = min(T, 4096)
    sweep = {}
    with threadpool_limits(1):
        timed(counts[-1], ts)   # warm-up (thread pools, first touch of the inputs)
        for _ in range(2):   # each count twice, the faster run kept (the first point ran cold)
            for nw in counts:
                sweep[nw] = min(sweep.get(nw, float("inf")), timed(nw, ts))
        best = min(sweep, key=sweep.get)
        # 1-thread rate: the chosen split's head slices run one after another on this thread
        # (one call over all heads is slower per head: numpy's temporaries then outgrow the caches)
        cuts = [group * ((n_heads // group) * i // best) for i in range(best + 1)]
        single = float("inf")
        for _ in range(2):
            t0 = time.perf_counter()
            for i in range(best):
                run(cuts[i], cuts[i + 1], ts)
            single = min(single, time.perf_counter() - t0)
        progress(f"cpu baseline: {best} worker threads fastest on {ts} tokens "
                 f"({', '.join(f'{c}: {s:.2f} s' for c, s in sweep.items())})")
        # at least `repeats` runs and at least CPU_SAMPLE_SECONDS of timed CPU work (a bounded
        # sample: at most 200 runs)
        times = []
        while len(times) < repeats or (sum(times) < CPU_SAMPLE_SECONDS and len(times) < 200):
            times.append(timed(best, T))
            if len(times) <= repeats or len(times) % 10 == 0:
                progress(f"cpu baseline run {len(times)}: {times[-1]:.2f} s (total {sum(times):.1f} s)")
        repeats = len(times)
    t = statistics.median(times)
    return dict(t=t, cores=best, host_cores=cores, sample_tokens=ts,
                single_thread_tokens_per_s=ts / single,
                sample=f"{what}, T={T} on {n_heads} heads split over {best} worker threads of one BLAS "
                       f"thread each (fastest of {counts} on {ts} tokens), median of {repeats} "
                       f"({t:.2f} s per run)")


def cpu_report(r, tokens: int, frac: float):
    """The cpu_baseline object from a head_parallel_cpu result, value scaled to all heads."""
    out = dict(value=tokens * frac / r["t"], unit="tokens/s", cores=r["cores"], kind="port",
               sample=r["sample"] + ("; value scaled to all heads" if frac < 1 else ""),
               host_cores=r["host_cores"])
    if r["single_thread_tokens_per_s"] is not None:
        out["single_thread"] = {"value": r["single_thread_tokens_per_s"] * frac, "unit": "tokens/s", "cores": 1,
                                "sample": f"the same head slices run one after another on one thread, first "
                                          f"{r['sample_tokens']} tokens"}
    return out


def cpu_baseline(torch, k, w, u, g, sample_heads: int, repeats: int = 3):
    """Time the numpy oracle (exact fp32 chunk loop) on the host, on a head subset."""
    from oracle import cgdr_oracle as O

    H, Hg = w.shape[2], k.shape[2]
    r = H // Hg
    kh = k[:, :, : max(1, sample_heads // r)].float().cpu().numpy()
    wh, uh, gh = (x[:, :, :sample_heads].float().cpu().numpy() for x in (w, u, g))
    run = lambda lo, hi, t: O.fwd_h(kh[:, :t, lo // r:hi // r], wh[:, :t, lo:hi], uh[:, :t, lo:hi], gh[:, :t, lo:hi])
    res = head_parallel_cpu(run, sample_heads, r, k.shape[1], repeats, "numpy oracle (exact fp32 chunk loop), B=1")
    return cpu_report(res, k.shape[0] * k.shape[1], sample_heads / H)


def chunk_o_bytes(B, T, H, Hg, K, V, NT, s=2):
    """q, k, v_new, h and g read once, o written once."""
    return B * T * Hg * K * s * 2 + B * T * H * V * s * 2 + B * NT * H * K * V * s + 4 * B * T * H


def chunk_o_flops(B, NT, H, K, V):
    """q k^T [64x64xK], q h [64xVxK], A' v [64xVx64] per chunk and head."""
    return B * NT * H * 2 * 64 * (64 * K + K * V + 64 * V)


def make_chunk_o_inputs(torch, dev, B, T, H, Hg, K, V, seed=0):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    NT = (T + 63) // 64
    q = torch.nn.functional.normalize(torch.randn(B, T, Hg, K, device=dev, generator=gen), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(B, T, Hg, K, device=dev, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, device=dev, generator=gen).to(torch.bfloat16)
    h = (torch.randn(B, NT, H, K, V, device=dev, generator=gen) * 0.3).to(torch.bfloat16)
    inc = torch.nn.functional.logsigmoid(torch.randn(B, NT * 64, H, device=dev, generator=gen) + 3.0)
    g = inc.view(B, NT, 64, H).cumsum(dim=2).view(B, NT * 64, H)[:, :T].contiguous()
    return q, k, v, h, g


def chunk_o_cpu_baseline(torch, q, k, v, h, g, sample_heads: int, repeats: int = 3):
    from oracle import cgdr_oracle as O

    H, Hg = v.shape[2], q.shape[2]
    r = H // Hg
    arr = lambda t: t.float().cpu().numpy()
    qh, kh = arr(q[:, :, : max(1, sample_heads // r)]), arr(k[:, :, : max(1, sample_heads // r)])
    vh, hh, gh = arr(v[:, :, :sample_heads]), arr(h[:, :, :sample_heads]), arr(g[:, :, :sample_heads])
    run = lambda lo, hi, t: O.chunk_o(qh[:, :t, lo // r:hi // r], kh[:, :t, lo // r:hi // r], vh[:, :t, lo:hi],
                                      hh[:, :(t + 63) // 64, lo:hi], g=gh[:, :t, lo:hi])
    res = head_parallel_cpu(run, sample_heads, r, q.shape[1], repeats, "numpy oracle chunk_o (exact fp32), B=1")
    return cpu_report(res, q.shape[0] * q.shape[1], sample_heads / H)


def progress(msg: str) -> None:
    """One line per finished phase on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_steps(torch, dev, step, steps, warmup):
    """`warmup` untimed steps, then exactly `steps` steps between two synchronisations.  One
    pair of HIP events on the launch stream brackets the timed steps (events around every step
    would add a ~7 us gap to each).  Returns the wall time, the events' time per step (the
    average launch duration while the host keeps the stream fed, else an upper bound of it) and
    the host's issue time per step."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    issue = time.perf_counter() - t0
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, e0.elapsed_time(e1) / steps, issue * 1e3 / steps


def timing_fields(avg_ms, host_ms):
    """kernel_ms is the events' time per step; launch_bound marks runs where the host's issue
    time per step comes within 10 % of it (then the GPU idled between launches, and kernel_ms
    overstates the launch duration)."""
    return {"kernel_ms": avg_ms, "host_ms_per_step": host_ms, "launch_bound": host_ms > 0.9 * avg_ms}


def wy_bytes(B, T, H, Hg, K, V, s=2):
    """k, v, beta (fp32), g read once; w, u, g_cumsum written once."""
    return B * T * (Hg * K + H * V) * s + 8 * B * T * H + B * T * H * (K + V) * s + 4 * B * T * H


def make_wy_inputs(torch, dev, B, T, H, Hg, K, V, seed=0):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    k = torch.nn.functional.normalize(torch.randn(B, T, Hg, K, device=dev, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, device=dev, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, device=dev, generator=gen))
    a = torch.nn.functional.logsigmoid(torch.randn(B, T, H, device=dev, generator=gen) + 2.0)
    q = torch.nn.functional.normalize(torch.randn(B, T, Hg, K, device=dev, generator=gen), dim=-1).to(torch.bfloat16)
    return q, k, v, beta, a


def wy_cpu_baseline(torch, k, v, beta, a, sample_heads, repeats):
    from oracle import cgdr_oracle as O

    H, Hg = v.shape[2], k.shape[2]
    r = H // Hg
    arr = lambda t: t.float().cpu().numpy()
    kh = arr(k[:, :, : max(1, sample_heads // r)])
    vh, bh, ah = arr(v[:, :, :sample_heads]), arr(beta[:, :, :sample_heads]), arr(a[:, :, :sample_heads])
    run = lambda lo, hi, t: O.wy_prepare(kh[:, :t, lo // r:hi // r], vh[:, :t, lo:hi], bh[:, :t, lo:hi], ah[:, :t, lo:hi])
    res = head_parallel_cpu(run, sample_heads, r, k.shape[1], repeats,
                            "numpy oracle wy_prepare (float64, one solve per chunk and head), B=1")
    return cpu_report(res, k.shape[0] * k.shape[1], sample_heads / H)


def main_wy(args, torch, cgdr_amd, dev, forward: bool):
    W = WORKLOAD
    B, T, H, Hg, K, V = W["B"], W["T"], W["H"], W["Hg"], W["K"], W["V"]
    NT = (T + 63) // 64
    q, k, v, beta, a = make_wy_inputs(torch, dev, B, T, H, Hg, K, V)
    torch.cuda.synchronize()
    progress("wy inputs resident in HBM")
    if forward:
        step = lambda: cgdr_amd.chunk_gated_delta_rule_fwd(q, k, v, a, beta, output_final_state=True)
        nbytes = (wy_bytes(B, T, H, Hg, K, V) + algorithmic_bytes(B, T, H, Hg, K, V, NT, B)
                  + chunk_o_bytes(B, T, H, Hg, K, V, NT))
        name, tfile = "forward", None
    else:
        step = lambda: cgdr_amd.wy_fwd(k, v, beta, g=a)
        nbytes = wy_bytes(B, T, H, Hg, K, V)
        name, tfile = "wy", os.path.join(ROOT, "profiles", "cgdr_wy_bf16_T32768_H32_hbm_traffic.md")
    wall, avg_ms, host_ms = time_steps(torch, dev, step, args.steps, args.warmup)
    progress(f"timed {args.steps} {name} steps")
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    traffic = None
    if tfile and os.path.exists(tfile):
        for line in open(tfile):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":")[1])
    what = ("chunked forward o, final_state from q, k, v, beta, g (WY -> FwdH -> chunk output)" if forward
            else "WY producer w, u, g_cumsum from k, v, beta, g")
    out = {
        "metric": f"{name} tokens/sec + achieved HBM GB/s at B=1,T=32k,H=32,K=V=128 bf16 (1 GPU)",
        "value": B * T * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": what + ", long-context prefill", **W, "parallelism": "none (1 GPU)"},
        "hbm_gbps": achieved,
        **timing_fields(avg_ms, host_ms),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic, "algorithmic_bytes": nbytes},
    }
    if not args.no_cpu_baseline and not forward:
        out["cpu_baseline"] = wy_cpu_baseline(torch, k, v, beta, a, args.cpu_sample_heads or 16, args.cpu_repeats or 3)
        out["cpu_baseline"]["speedup"] = out["value"] / out["cpu_baseline"]["value"]
    print(json.dumps(out), flush=True)


def main_chunk_o(args, torch, cgdr_amd, dev):
    W = WORKLOAD
    B, T, H, Hg, K, V = W["B"], W["T"], W["H"], W["Hg"], W["K"], W["V"]
    NT = (T + 63) // 64
    q, k, v, h, g = make_chunk_o_inputs(torch, dev, B, T, H, Hg, K, V)
    torch.cuda.synchronize()
    progress("chunk_o inputs resident in HBM")
    wall, avg_ms, host_ms = time_steps(torch, dev, lambda: cgdr_amd.chunk_fwd_o(q, k, v, h, g=g), args.steps,
                                       args.warmup)
    progress(f"timed {args.steps} chunk_o steps")
    nbytes = chunk_o_bytes(B, T, H, Hg, K, V, NT)
    flops = chunk_o_flops(B, NT, H, K, V)
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "cgdr_chunk_o_bf16_T32768_H32_hbm_traffic.md")
    if os.path.exists(tfile):
        for line in open(tfile):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":")[1])
    out = {
        "metric": "chunk output tokens/sec + achieved HBM GB/s at B=1,T=32k,H=32,K=V=128 bf16 (1 GPU)",
        "value": B * T * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "chunk output o from FwdH's h and v_new, long-context prefill", **W,
                   "parallelism": "none (1 GPU)"},
        "hbm_gbps": achieved,
        **timing_fields(avg_ms, host_ms),
        "tflops": flops / (avg_ms * 1e-3) / 1e12,
        "plan": cgdr_amd.chunk_o.plan(q, v),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic, "algorithmic_bytes": nbytes},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = chunk_o_cpu_baseline(torch, q, k, v, h, g, args.cpu_sample_heads or 16,
                                                   args.cpu_repeats or 3)
        out["cpu_baseline"]["speedup"] = out["value"] / out["cpu_baseline"]["value"]
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-heads", type=int, default=None,
                    help="heads of the CPU-baseline sample (default 32 for fwd_h, 8 for chunk_o)")
    ap.add_argument("--cpu-repeats", type=int, default=None, help="default 7 for fwd_h, 3 for chunk_o")
    ap.add_argument("--op", choices=("fwd_h", "chunk_o", "wy", "forward"), default="fwd_h",
                    help="fwd_h: the headline FwdH step (default); chunk_o: the chunk output; wy: the WY "
                         "producer; forward: WY -> FwdH -> chunk output")
    ap.add_argument("--workload", choices=tuple(FWD_H_WORKLOADS), default="prefill",
                    help="fwd_h shape: prefill (B=1 T=32768 H=32 K=V=128, the default), two_seq (B=2 T=2048 "
                         "H=16, h0), varlen (16 packed sequences of lengths U[64,8192], h0), wide_v (B=4 T=8192 "
                         "H=8 K=128 V=256, strongly decaying gate, h0); the CPU baseline runs on prefill only")
    ap.add_argument("--numerics", choices=("default", "contest"), default="default",
                    help="fwd_h rounding model: default (the Triton kernel's) or contest (run()'s casts)")
    ap.add_argument("--tuning", default=None,
                    help="fwd_h launch-plan overrides as JSON (fields of cgdr_fwd_h_tuning, e.g. "
                         "'{\"load_waves\": 2}'); outputs do not depend on them")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB fp32 elementwise copy (the reference kernel of known "
                         "HBM traffic that scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the FwdH path runs on one GPU and has no multi-GPU "
              f"component (--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    import torch

    import cgdr_amd

    progress("torch and cgdr_amd imported")
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "torch.mul(src, 1.0, out=dst)", "read_bytes": src.numel() * 4,
                          "write_bytes": dst.numel() * 4, "launches": 3}), flush=True)
        return
    if args.op == "chunk_o":
        return main_chunk_o(args, torch, cgdr_amd, dev)
    if args.op in ("wy", "forward"):
        return main_wy(args, torch, cgdr_amd, dev, forward=args.op == "forward")
    if args.workload == "prefill":
        W = WORKLOAD
        B, T, H, Hg, K, V = W["B"], W["T"], W["H"], W["Hg"], W["K"], W["V"]
        N, NT = B, (T + 63) // 64
        k, w, u, g = make_inputs(torch, dev, B, T, H, Hg, K, V)
        h0 = cu = None
    else:
        t_in, W = make_workload_inputs(torch, dev, args.workload)
        B, T, H, Hg, K, V, N, NT = (W[x] for x in ("B", "T", "H", "Hg", "K", "V", "N", "NT"))
        k, w, u, g, h0, cu = (t_in[x] for x in ("k", "w", "u", "g", "initial_state", "cu_seqlens"))
    torch.cuda.synchronize()
    progress(f"fwd_h inputs ({args.workload}) resident in HBM")

    tuning = json.loads(args.tuning) if args.tuning else None

    def step():
        return cgdr_amd.chunk_gated_delta_rule_fwd_h(k, w, u, g=g, initial_state=h0, output_final_state=True,
                                                     cu_seqlens=cu, numerics=args.numerics, tuning=tuning)

    wall, avg_ms, host_ms = time_steps(torch, dev, step, args.steps, args.warmup)
    progress(f"timed {args.steps} fwd_h steps: {avg_ms * 1e3:.1f} us per step by events, "
             f"{host_ms * 1e3:.1f} us host issue time per step")

    es = k.element_size()
    nbytes = algorithmic_bytes(B, T, H, Hg, K, V, NT, N, s_in=es, s_out=es, h0_bytes=4 if h0 is not None else 0)
    flops = algorithmic_flops(B, NT, H, K, V)
    ms_per_step = wall * 1e3 / args.steps
    tokens_per_s = B * T * args.steps / wall
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    plan = cgdr_amd.plan(k, u, cu_seqlens_len=None if cu is None else len(cu), numerics=args.numerics, NT=NT,
                         tuning=tuning)

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "cgdr_fwd_h_bf16_T32768_H32_hbm_traffic.md")
    if os.path.exists(tfile) and args.workload == "prefill" and args.numerics == "default":
        for line in open(tfile):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":")[1])

    out = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if es == 4 else "bf16",
        "data": "synthetic",
        "config": {"workload": FWD_H_WORKLOADS[args.workload]["desc"], **W,
                   "h0": "fp32 [N,H,K,V]" if h0 is not None else None, "output_final_state": True,
                   "numerics": args.numerics, "parallelism": "none (1 GPU)",
                   **({"tuning": tuning} if tuning else {})},
        "hbm_gbps": achieved,
        **timing_fields(avg_ms, host_ms),
        "tflops": flops / (avg_ms * 1e-3) / 1e12,
        "mfma_util": flops / (avg_ms * 1e-3) / 1e12 / (F32_MFMA_PEAK_TFLOPS if es == 4 else BF16_MFMA_PEAK_TFLOPS),
        "plan": plan,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "algorithmic_bytes": nbytes},
    }
    if not args.no_cpu_baseline and args.workload == "prefill":
        out["cpu_baseline"] = cpu_baseline(torch, k, w, u, g, args.cpu_sample_heads or 32, args.cpu_repeats or 7)
        out["cpu_baseline"]["speedup"] = tokens_per_s / out["cpu_baseline"]["value"]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
