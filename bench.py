"""Benchmark of the FA3 backward (shaobo_fa3_bwd_v2) on one MI355X.

A step is one full backward through the C ABI over resident fp16 inputs at
the headline shape B=1, H=4, S=2048, D=128, causal (BASELINE.json
configs[2]): the delta preprocess and the main kernel, two launches on the
null stream.  The timed region is `steps` back-to-back shaobo_fa3_bwd_v2
calls between two HIP events.  Per-kernel durations, back to back: the main
kernel alone over as many back-to-back launches between two events
(shaobo_fa3_ext_bwd_v2_stages with the main-kernel stage, on the workspace
the timed calls prepared), and the preprocess as the step minus that -- its
cost inside a step; the rooflines come from these.  The preprocess kernel
alone in back-to-back launches (the same kernel and grid through the
shaobo_fa3_bwd_dot_do_o component) is reported beside them: launches of a
short kernel wait for the host's submissions, so that figure exceeds the
kernel's share of a step.  For reference the line also carries the
durations measured by shaobo_fa3_ext_bwd_v2_timed (events recorded before,
between and after the two kernels of every call), which include each
marker's dispatch latency and so exceed the kernels' execution times.  Prints one JSON
line: TFLOP/s from FLOPs = 10*B*H*S^2*D*0.5, ms per backward, % of fp16 dense
MFMA peak, the main kernel's (MFMA) and the preprocess's (HBM) rooflines,
and the CPU oracle timed on the host as the reported CPU baseline.

--all measures every BASELINE config (P1-P5) in one run and prints one JSON
line per config (GPU ms per backward, TFLOP/s, % of peak, the main kernel's
time, and the CPU oracle's backward of the whole config on the host, with
the threads it used and the host's core count), then a markdown table of
the same figures on stderr.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config P3] [--all]
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-attention3_amd"))

METRIC = "FA bwd TFLOPS + % fp16 MFMA peak, B1 H4 S2048 D128 causal fp16; ms/bwd"
FP16_PEAK_TFLOPS = 2516.6   # MI355X dense fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    # name: (B, Hq, Hkv, S, D, causal)
    "P1": (1, 1, 1, 128, 128, True),
    "P2": (1, 1, 1, 1024, 128, True),
    "P3": (1, 4, 4, 2048, 128, True),
    "P4": (2, 32, 8, 4096, 128, True),
    "P5": (2, 16, 16, 8192, 64, False),
}


def register_shape(text):
    """A --shape "B,Hq,Hkv,S,D,causal|full" as a CONFIGS entry; returns its name."""
    parts = text.split(",")
    if len(parts) != 6 or parts[5] not in ("causal", "full"):
        raise SystemExit(f"--shape wants B,Hq,Hkv,S,D,causal|full, got {text!r}")
    B, Hq, Hkv, S, D = (int(x) for x in parts[:5])
    name = f"shape_{B}_{Hq}_{Hkv}_{S}_{D}_{parts[5]}"
    CONFIGS[name] = (B, Hq, Hkv, S, D, parts[5] == "causal")
    return name


def flops(B, Hq, S, D, causal):
    return 10.0 * B * Hq * S * S * D * (0.5 if causal else 1.0)


def make_inputs(torch, B, Hq, Hkv, S, D, causal, scale, seed=1234):
    """Seeded N(0,1) fp16 Q, K, V, dO; O and natural LSE from an fp32 GPU
    forward (input preparation, outside the timed region)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda h: torch.randn((B, h, S, D), generator=gen, device="cuda").half()  # noqa: E731
    q, k, v, do = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device="cuda")
    G = Hq // Hkv
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool, device="cuda"), 1) if causal else None
    for b in range(B):
        for h in range(Hq):
            s = torch.mm(q[b, h].float(), k[b, h // G].float().t().contiguous()) * scale
            if mask is not None:
                s.masked_fill_(mask, float("-inf"))
            lse[b, h] = torch.logsumexp(s, -1)
            out[b, h] = torch.mm(torch.softmax(s, -1), v[b, h // G].float()).half()
            del s
    return q, k, v, do, out, lse


class Hip:
    """Minimal hipEvent binding (events on the null stream)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.lib.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e):
        assert self.lib.hipEventRecord(e, None) == 0

    def elapsed_ms(self, a, b):
        self.lib.hipEventSynchronize(b)
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def sync(self):
        assert self.lib.hipDeviceSynchronize() == 0


def load_traffic(config):
    """HBM bytes per launch of the main kernel, measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE and scaled by a copy kernel of known size
    (profiles/traffic_bwd_main_kernel.json, written from those runs)."""
    path = os.path.join(ROOT, "profiles", "traffic_bwd_main_kernel.json")
    try:
        with open(path) as fh:
            entry = json.load(fh).get(config)
    except (OSError, ValueError):
        return None
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def preprocess_bytes(B, Hq, S, D):
    """Bytes one preprocess launch must move: read O and dO (fp16) and the
    LSE row; write delta, lse2 and -delta (fp32) per row."""
    rows = B * Hq * S
    return 2 * rows * D * 2 + rows * 4 * 4


def host_cores():
    """CPUs this process may run on (its affinity mask)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# The oracle runs on at most this many threads: a GPU box gives one GPU a
# 16-core share of its host, whatever the affinity mask shows.
CPU_SHARE_PER_GPU = 16


def cpu_full(cfg):
    """The CPU oracle's fp32 backward of the whole config on the host's
    cores (forward first, untimed): ms, threads, TFLOP/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fa3_oracle as O
    B, Hq, Hkv, S, D, causal = cfg
    scale = 1.0 / math.sqrt(D)
    threads = O.default_threads()
    x = O.make_inputs(B, Hq, Hkv, S, D)
    out, smax, ssum, _ = O.forward(x["q"], x["k"], x["v"], causal, scale, None, threads)
    t0 = time.perf_counter()
    O.backward(x["q"], x["k"], x["v"], out, x["dout"], smax, ssum, causal, scale, None, threads)
    sec = time.perf_counter() - t0
    return {"bwd_ms": round(sec * 1e3, 3), "threads": threads, "host_cores": host_cores(),
            "tflops": round(flops(B, Hq, S, D, causal) / sec / 1e12, 6)}


def cpu_baseline(cfg, budget_s):
    """Time the CPU oracle (fp32) on the host: its threaded backward on a
    bounded sample of the same workload -- whole (batch, kv-head) groups of
    the config, repeated until about budget_s seconds of CPU work have run --
    its threaded forward on the same sample, timed separately, and its
    single-threaded backward of the whole P1, P2 and P3 configs."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fa3_oracle as O
    B, Hq, Hkv, S, D, causal = cfg
    scale = 1.0 / math.sqrt(D)
    threads = O.default_threads()
    # whole config when small (P1-P3), else one (batch, kv-head) group
    groups = B * Hkv if B * Hq * S <= 8192 else 1
    x = O.make_inputs(B, Hq, Hkv, S, D)
    t0 = time.perf_counter()
    out, smax, ssum, _ = O.forward(x["q"], x["k"], x["v"], causal, scale, (0, groups), threads)
    fwd_s = time.perf_counter() - t0
    runs, t_total = 0, 0.0
    while t_total < budget_s or runs == 0:
        t0 = time.perf_counter()
        O.backward(x["q"], x["k"], x["v"], out, x["dout"], smax, ssum, causal, scale, (0, groups),
                   threads)
        t_total += time.perf_counter() - t0
        runs += 1
        if runs >= 1000:
            break
    sample_heads = groups * (Hq // Hkv)
    f = flops(1, sample_heads, S, D, causal)
    sec = t_total / runs
    single = {}
    for name in ("P1", "P2", "P3"):
        b1, hq1, hkv1, s1, d1, c1 = CONFIGS[name]
        x1 = O.make_inputs(b1, hq1, hkv1, s1, d1)
        sc1 = 1.0 / math.sqrt(d1)
        o1, m1, l1, _ = O.forward(x1["q"], x1["k"], x1["v"], c1, sc1, None, 1)
        t0 = time.perf_counter()
        O.backward(x1["q"], x1["k"], x1["v"], o1, x1["dout"], m1, l1, c1, sc1, None, 1)
        dt = time.perf_counter() - t0
        single[name] = {"bwd_ms": round(dt * 1e3, 3),
                        "tflops": round(flops(b1, hq1, s1, d1, c1) / dt / 1e12, 6)}
    return {"value": round(f / sec / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "host_cores": host_cores(),
            "threads_note": f"threads = min(host cores, {CPU_SHARE_PER_GPU}): the GPU box's "
                            "CPU share per GPU",
            "kind": "port",
            "sample": f"oracle fp32 backward of {sample_heads} of {B * Hq} query heads "
                      f"(S={S}, D={D}, causal={causal}), {runs} runs, {sec * 1e3:.1f} ms each",
            "ms_per_bwd_sample": round(sec * 1e3, 3),
            "fwd_ms_sample": round(fwd_s * 1e3, 3),
            "single_thread_bwd": single}


def measure(torch, lib, F, hip, name, steps, warmup, deterministic, dtype="fp16",
            layout="bhsd"):
    """GPU figures of one config: the timed backward calls, the per-kernel
    durations back to back, and the rooflines (no CPU baseline).  dtype /
    layout: the same inputs as bf16 and / or [B, S, H, D] tensors."""
    B, Hq, Hkv, S, D, causal = CONFIGS[name]
    scale = 1.0 / math.sqrt(D)
    q, k, v, do, out, lse = make_inputs(torch, B, Hq, Hkv, S, D, causal, scale)
    if dtype == "bf16":
        q, k, v, do, out = (x.to(torch.bfloat16) for x in (q, k, v, do, out))
    if layout == "bshd":
        q, k, v, do, out = (x.transpose(1, 2).contiguous() for x in (q, k, v, do, out))
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D,
                      causal=causal, softmax_scale=scale, deterministic=deterministic)
    if dtype == "bf16":
        p.dtype = F.DTYPE_BF16
    if layout == "bshd":
        p.layout = F.LAYOUT_BSHD
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((B, Hq, S), dtype=torch.float32, device="cuda")
    c = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    argv = [c(do), c(q), c(k), c(v), c(out), c(lse), c(dq), c(dk), c(dv), c(delta)]

    def step():
        st = lib.shaobo_fa3_bwd_v2(*argv, ctypes.byref(p))
        if st != F.SUCCESS:
            raise RuntimeError("shaobo_fa3_bwd_v2: " + F.status_name(st))

    # Warm-up: at least `warmup` steps and at least 0.3 s of GPU work, in
    # batches of 20 -- the GPU's clocks ramp up over tens of milliseconds of
    # sustained work, and a handful of steps measures the ramp instead of
    # the kernel.
    done = 0
    t_w = time.perf_counter()
    while done < warmup or time.perf_counter() - t_w < 0.3:
        for _ in range(20):
            step()
        done += 20
        torch.cuda.synchronize()
    warm_s = time.perf_counter() - t_w

    # ---- timed region: exactly `steps` backward lifecycles ----
    e0, e1 = hip.event(), hip.event()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hip.record(e0)
    for _ in range(steps):
        step()
    hip.record(e1)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = hip.elapsed_ms(e0, e1) / steps
    f = flops(B, Hq, S, D, causal)
    tflops = f / (ms * 1e-3) / 1e12

    # ---- per-kernel durations, back to back ----
    # the main kernel alone, on the workspace the timed calls left (their
    # row statistics); the preprocess's share of a step is the rest
    def main_step():
        st = lib.shaobo_fa3_ext_bwd_v2_stages(*argv, ctypes.byref(p), None, 2)
        if st != F.SUCCESS:
            raise RuntimeError("shaobo_fa3_ext_bwd_v2_stages: " + F.status_name(st))

    for _ in range(5):
        main_step()
    torch.cuda.synchronize()
    hip.record(e0)
    for _ in range(steps):
        main_step()
    hip.record(e1)
    torch.cuda.synchronize()
    main_ms = hip.elapsed_ms(e0, e1) / steps
    pre_step_ms = ms - main_ms
    # the preprocess alone: the dot_do_o component runs the same kernel on
    # the same rows (delta plus the packed sidecar: the same bytes); the
    # component takes fp16 BHSD only, as the reference's does
    pre_alone_ms = None
    if dtype == "fp16" and layout == "bhsd":
        pp = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hq, head_dim=D,
                           causal=causal, softmax_scale=scale)
        pp.softmax_aux_mode = F.AUX_LSE
        packed = torch.empty(B * Hq * S * 3, dtype=torch.float32, device="cuda")

        def pre_step():
            st = lib.shaobo_fa3_bwd_dot_do_o(c(do), c(out), c(lse), None, c(delta), c(packed),
                                             ctypes.byref(pp))
            if st != F.SUCCESS:
                raise RuntimeError("shaobo_fa3_bwd_dot_do_o: " + F.status_name(st))

        for _ in range(20):
            pre_step()
        torch.cuda.synchronize()
        hip.record(e0)
        for _ in range(steps):
            pre_step()
        hip.record(e1)
        torch.cuda.synchronize()
        pre_alone_ms = hip.elapsed_ms(e0, e1) / steps
    # the same number of calls through the timed entry, three events per
    # call, read after one sync (marker-inclusive durations)
    evs = [[hip.event() for _ in range(3)] for _ in range(steps)]
    ev_arrays = [(ctypes.c_void_p * 3)(*[e.value for e in trio]) for trio in evs]
    for i in range(steps):
        st = lib.shaobo_fa3_ext_bwd_v2_timed(*argv, ctypes.byref(p), None, ev_arrays[i])
        if st != F.SUCCESS:
            raise RuntimeError("shaobo_fa3_ext_bwd_v2_timed: " + F.status_name(st))
    torch.cuda.synchronize()
    pre_marked = sum(hip.elapsed_ms(t[0], t[1]) for t in evs) / steps
    main_marked = sum(hip.elapsed_ms(t[1], t[2]) for t in evs) / steps
    staged_ms = hip.elapsed_ms(evs[0][0], evs[-1][2]) / steps
    main_tflops = f / (main_ms * 1e-3) / 1e12
    pre_gbs = preprocess_bytes(B, Hq, S, D) / (pre_step_ms * 1e-3) / 1e9
    return {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": f"fa3_bwd_v2 {name} B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} "
                               f"{'causal' if causal else 'full'}",
                   "batch": B, "heads_q": Hq, "heads_kv": Hkv, "seq_len": S, "head_dim": D,
                   "causal": causal, "deterministic": deterministic, "layout": layout,
                   "flops_per_bwd": f},
        "pct_fp16_peak": round(100.0 * tflops / FP16_PEAK_TFLOPS, 3),
        "wall_s_timed": round(wall, 4),
        "warmup_steps_run": done,
        "warmup_s": round(warm_s, 3),
        "kernels_ms": {"preprocess_kernel": round(pre_step_ms, 5),
                       "bwd_main_kernel": round(main_ms, 5),
                       "preprocess_alone_back_to_back":
                           None if pre_alone_ms is None else round(pre_alone_ms, 5)},
        "kernels_ms_marked": {"preprocess_kernel": round(pre_marked, 5),
                              "bwd_main_kernel": round(main_marked, 5),
                              "ms_per_step": round(staged_ms, 5)},
        "roofline": {"kernel": "bwd_main_kernel", "bound": "mfma",
                     "achieved": round(main_tflops, 3),
                     "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(main_tflops / FP16_PEAK_TFLOPS, 5),
                     "traffic": load_traffic(name),
                     "traffic_source": "profiles/traffic_bwd_main_kernel.json (rocprofv3 "
                                       "FETCH_SIZE + WRITE_SIZE of this kernel, calibrated)"},
        "preprocess_roofline": {"kernel": "preprocess_kernel", "bound": "hbm",
                                "achieved": round(pre_gbs, 1), "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": round(pre_gbs / HBM_PEAK_GBS, 5),
                                "bytes": preprocess_bytes(B, Hq, S, D)},
    }


def run_all(torch, lib, F, hip, args):
    """Every BASELINE config: one JSON line each (GPU figures, the whole
    config's CPU oracle backward), then a markdown table on stderr."""
    rows = []
    for name in ("P1", "P2", "P3", "P4", "P5"):
        B, Hq, Hkv, S, D, causal = CONFIGS[name]
        # about 0.5 s of timed GPU work per config (at ~40 % of peak), 10..200 calls
        est_ms = flops(B, Hq, S, D, causal) / (0.4 * FP16_PEAK_TFLOPS * 1e12) * 1e3 + 0.02
        steps = max(10, min(200, int(500 / est_ms)))
        r = measure(torch, lib, F, hip, name, steps, 20, args.deterministic)
        torch.cuda.empty_cache()
        line = {"config": name, "workload": r["config"]["workload"],
                "gpu_ms_per_bwd": r["ms_per_step"], "tflops": r["value"],
                "pct_fp16_peak": r["pct_fp16_peak"], "steps": steps,
                "main_kernel_ms": r["kernels_ms"]["bwd_main_kernel"],
                "preprocess_ms": r["kernels_ms"]["preprocess_kernel"],
                "main_kernel_frac": r["roofline"]["frac"]}
        if args.cpu_budget > 0:
            line["cpu"] = cpu_full(CONFIGS[name])
        print(json.dumps(line), flush=True)
        rows.append(line)
    out = ["| Config | CPU bwd ms (threads / host cores) | GPU ms/bwd | GPU TFLOP/s | "
           "% fp16 peak | main kernel ms |", "|---|---|---|---|---|---|"]
    for r in rows:
        cpu = r.get("cpu")
        cpu_s = f"{cpu['bwd_ms']:.1f} ({cpu['threads']} / {cpu['host_cores']})" if cpu else "-"
        out.append(f"| {r['workload']} | {cpu_s} | {r['gpu_ms_per_bwd']:.5f} | {r['tflops']:.1f} "
                   f"| {r['pct_fp16_peak']:.2f} | {r['main_kernel_ms']:.5f} |")
    print("\n".join(out), file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warm-up steps (default 20); warm-up also lasts at least "
                         "0.3 s of GPU work, which brings the clocks to their steady state")
    ap.add_argument("--config", default="P3", choices=sorted(CONFIGS))
    ap.add_argument("--shape", default=None, metavar="B,Hq,Hkv,S,D,causal|full",
                    help="time this shape instead of a BASELINE config (a diagnostic line, "
                         "not the headline)")
    ap.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"],
                    help="the inputs' 16-bit type (a diagnostic line; the headline is fp16)")
    ap.add_argument("--layout", default="bhsd", choices=["bhsd", "bshd"],
                    help="tensor layout (a diagnostic line; the headline is BHSD)")
    ap.add_argument("--all", action="store_true",
                    help="every config P1-P5, one JSON line each (GPU and whole-config CPU)")
    ap.add_argument("--deterministic", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU oracle work for cpu_baseline (0 disables)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after timing, run a plain device copy of this many MiB "
                         "(reference kernel for rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); the backward shards by (batch, kv-head) "
              f"with no communication, so per-GPU throughput is the N=1 figure.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import shaobo_fa3 as F

    lib = F.load()
    hip = Hip()
    if args.all:
        run_all(torch, lib, F, hip, args)
        return
    warmup = 20 if args.warmup is None else args.warmup
    name = args.config
    if args.shape is not None:
        name = register_shape(args.shape)
    result = measure(torch, lib, F, hip, name, args.steps, warmup, args.deterministic,
                     args.dtype, args.layout)
    if args.calib_copy_mb > 0:
        # plain copy kernel of known size, for scaling rocprofv3 FETCH/WRITE_SIZE
        n = args.calib_copy_mb * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        result["calib_copy_bytes"] = n * 4
    if args.cpu_budget > 0:
        result["cpu_baseline"] = cpu_baseline(CONFIGS[name], args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
