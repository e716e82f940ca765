"""Per-workgroup timeline of the main kernel (BASELINE configs P1-P5).

Runs one BASELINE config with the timeline build of the library
(``make -C flash-attention3_amd timeline`` -> lib/libshaobo_fa3_bwd_timeline.so,
the main kernel compiled with -DFA3_TIMELINE) and prints a markdown summary of
where each unit's time goes:

    python flash-attention3_amd/timeline.py --config P3 [--raw gpurun_out/tl_P3.npy]

Stamps (s_memrealtime, 100 MHz) per workgroup: its entry; per unit u < 4: unit
start, resident tiles landed, loop start, last step done, unit end (stores
complete), and for split pieces the publish / wait / add events.  A workgroup
of the persistent plan (P4, P5) runs many jobs: its first three go to units
0-2 and each later one overwrites unit 3, which so holds its last job.  Every
timed launch is the main kernel alone (the stage entry) after a full call
filled the row statistics; the instrumented kernel waits for its stores at
each unit end, so its unit gaps and epilogues run a little long.  The timeline
build is a diagnostic: the product library compiles none of the stamps.
"""
import argparse
import ctypes
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)
sys.path.insert(0, ROOT)

ROW_WORDS = 64      # per workgroup: [0] entry, [29] descriptor, [30] HW_ID, [31] XCC_ID
UNIT_BASE = 1 << 21  # unit stamps: UNIT_BASE + 32 wg + 8 u + s
S_START, S_LOOP, S_LAST, S_END, S_PUB, S_PAST, S_ADDED, S_RES = range(8)


def record(cfg, launches=3):
    import torch
    import bench
    import shaobo_fa3 as F

    B, Hq, Hkv, S, D, causal = bench.CONFIGS[cfg]
    scale = 1.0 / math.sqrt(D)
    path = os.path.join(HERE, "lib", "libshaobo_fa3_bwd_timeline.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: make -C flash-attention3_amd timeline")
    lib = F._declare(ctypes.CDLL(path))
    lib.fa3_timeline_set.argtypes = [ctypes.c_void_p]
    lib.fa3_timeline_set.restype = None
    q, k, v, do, out, lse = bench.make_inputs(torch, B, Hq, Hkv, S, D, causal, scale)
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D,
                      causal=causal, softmax_scale=scale)
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    c = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    argv = [c(do), c(q), c(k), c(v), c(out), c(lse), c(dq), c(dk), c(dv), None]
    lib.fa3_timeline_set(None)
    st = lib.shaobo_fa3_bwd_v2(*argv, ctypes.byref(p))
    if st != F.SUCCESS:
        raise RuntimeError("shaobo_fa3_bwd_v2: " + F.status_name(st))

    def main_only():
        st = lib.shaobo_fa3_ext_bwd_v2_stages(*argv, ctypes.byref(p), None, 2)
        if st != F.SUCCESS:
            raise RuntimeError("shaobo_fa3_ext_bwd_v2_stages: " + F.status_name(st))

    for _ in range(200):  # warm clocks and caches as a loop of backward calls would
        main_only()
    torch.cuda.synchronize()
    ref = [t.clone() for t in (dq, dk, dv)]
    n_wg = (Hq * B) * (S // 64) * 2
    buf = torch.zeros(UNIT_BASE + 32 * max(n_wg, 1), dtype=torch.int64, device="cuda")
    lib.fa3_timeline_set(ctypes.c_void_p(buf.data_ptr()))
    try:
        for _ in range(launches):
            buf.zero_()
            main_only()
        torch.cuda.synchronize()
    finally:
        lib.fa3_timeline_set(None)
    same = all(torch.equal(a, b) for a, b in zip(ref, (dq, dk, dv)))
    raw = buf.cpu().numpy()
    rows = raw[:UNIT_BASE].reshape(-1, ROW_WORDS)
    n_wg = int(np.count_nonzero(rows[:, 0]))
    return rows[:n_wg], raw[UNIT_BASE:UNIT_BASE + 32 * n_wg].reshape(n_wg, 4, 8), same


def in_order(units):
    """Each workgroup's recorded units in the order they ran (by start stamp):
    [workgroup, position, stamp], zero where a workgroup ran fewer units (a
    short job after a piece records in slot 3, whatever ran before it)."""
    out = np.zeros_like(units)
    for w in range(len(units)):
        ran = [u for u in range(units.shape[1]) if units[w, u, S_START] > 0]
        for i, u in enumerate(sorted(ran, key=lambda u: units[w, u, S_START])):
            out[w, i] = units[w, u]
    return out


def summary(cfg, rows, units, same):
    us = lambda a, b: np.where((a > 0) & (b > 0), (a - b) / 100.0, np.nan)  # noqa: E731
    units = in_order(units)
    ent = rows[:, 0]
    t0 = ent.min()
    kind = rows[:, 29] & 3
    end = np.nanmax(np.where(units[:, :, S_END] > 0, (units[:, :, S_END] - t0) / 100.0, np.nan),
                    axis=1)
    out = [f"Workgroups {len(rows)}; last unit end {np.nanmax(end):.2f} µs after the first "
           f"entry (median workgroup {np.nanmedian(end):.2f}); instrumented outputs bit-equal "
           f"to the same library's uninstrumented launch: {same}.", "",
           "Per unit (in the order a workgroup runs them), medians over the workgroups that "
           "run it (µs):", "",
           "| unit | workgroups | before the unit (entry or gap) | resident tiles landed | "
           "first phase to loop start | loop | last step to unit end |",
           "|---|---|---|---|---|---|---|"]
    for u in range(units.shape[1]):
        m = units[:, u, S_START] > 0
        if not m.any():
            continue
        U = units[m, u]
        prev = ent[m] if u == 0 else units[m, u - 1, S_END]
        cols = [us(U[:, S_START], prev), us(U[:, S_RES], U[:, S_START]),
                us(U[:, S_LOOP], U[:, S_RES]), us(U[:, S_LAST], U[:, S_LOOP]),
                us(U[:, S_END], U[:, S_LAST])]
        out.append(f"| {u} | {int(m.sum())} | " +
                   " | ".join(f"{np.nanmedian(x):.2f}" for x in cols) + " |")
    if not rows[:, 29].any() and (units[:, 3, S_START] > 0).any():
        out += ["", "Persistent plan: units 0-2 are a workgroup's first three jobs and unit 3 "
                "its last; unit 3's first column spans the jobs between."]
    first = units[:, :, S_PUB] > 0
    second = units[:, :, S_PAST] > 0
    if first.any() or second.any():
        pub = us(units[:, :, S_PUB], units[:, :, S_LAST])[first]
        wait = us(units[:, :, S_PAST], units[:, :, S_LAST])[second]
        add = us(units[:, :, S_ADDED], units[:, :, S_PAST])[second]
        store = us(units[:, :, S_END], units[:, :, S_ADDED])[second]
        out += ["", f"Split pieces: first piece, last step to publish {np.nanmedian(pub):.2f} "
                f"({int(first.sum())} pieces); second piece, last step to past its wait "
                f"{np.nanmedian(wait):.2f}, partial sums added {np.nanmedian(add):.2f}, "
                f"converted and stored {np.nanmedian(store):.2f} ({int(second.sum())} pieces)."]
    if rows[:, 29].any():  # split plan: the workgroup kinds' ends
        out += ["", "Workgroup ends by split-plan kind (µs after the first entry, "
                "min / median / max): " +
                "; ".join(f"kind {k} {np.nanmin(end[kind == k]):.2f} / "
                          f"{np.nanmedian(end[kind == k]):.2f} / {np.nanmax(end[kind == k]):.2f}"
                          for k in range(4) if (kind == k).any()) + "."]
    out += ["", "The 12 workgroups that end last (kind, end µs; per unit: before, resident, "
            "first phase, loop, end):", "", "```"]
    for w in np.argsort(-np.nan_to_num(end, nan=-1.0))[:12]:
        parts = []
        for u in range(4):
            U = units[w, u]
            if U[S_START] <= 0:
                continue
            prev = ent[w] if u == 0 else units[w, u - 1, S_END]
            parts.append("(%.2f %.2f %.2f %.2f %.2f)" % tuple(
                (b - a) / 100.0 for a, b in [(prev, U[S_START]), (U[S_START], U[S_RES]),
                                             (U[S_RES], U[S_LOOP]), (U[S_LOOP], U[S_LAST]),
                                             (U[S_LAST], U[S_END])]))
        out.append(f"wg {w:3d} kind {kind[w]} end {end[w]:6.2f}  " + " ".join(parts))
    out.append("```")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", default="P3", choices=["P1", "P2", "P3", "P4", "P5"])
    ap.add_argument("--raw", default=None, help="also save the raw stamps (.npy)")
    args = ap.parse_args()
    rows, units, same = record(args.config)
    if args.raw:
        os.makedirs(os.path.dirname(os.path.abspath(args.raw)), exist_ok=True)
        np.save(args.raw, np.concatenate([rows.ravel(), units.ravel()]))
    print(summary(args.config, rows, units, same), flush=True)


if __name__ == "__main__":
    main()
