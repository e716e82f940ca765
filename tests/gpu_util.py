"""Helpers shared by the GPU tests: move oracle inputs to the device, call the
C ABI, and compare against the oracle with the reference's metrics."""
import ctypes
import sys

import numpy as np

import fa3_oracle as O
import shaobo_fa3 as F


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(t, torch):
    return torch.from_numpy(np.ascontiguousarray(t)).cuda()


def run_v2(g, torch, *, deterministic=False, with_softmax_d=True, lse=None, scale_is_set=True,
           workspace_pad=0, workspace=None):
    """Run shaobo_fa3_bwd_v2 on the oracle's inputs; returns numpy fp32
    (delta, dq, dk, dv) and the status."""
    lib = F.load()
    q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
    lse_d = dev(g["lse"] if lse is None else lse, torch)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D,
                      causal=g["causal"], softmax_scale=g["scale"] if scale_is_set else None,
                      deterministic=deterministic, sync=True)
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    assert nbytes > 0
    if workspace is None:
        ws = torch.empty(nbytes + workspace_pad, dtype=torch.uint8, device="cuda")
        # poison the workspace: the library must not rely on its contents
        ws.fill_(0xC3)
    else:
        ws = workspace
        assert ws.numel() >= nbytes
    p.workspace = ws.data_ptr()
    p.workspace_bytes = ws.numel()
    dq = torch.full_like(q, float("nan"))
    dk = torch.full_like(k, float("nan"))
    dv = torch.full_like(v, float("nan"))
    delta = torch.full((B, Hq, S), float("nan"), dtype=torch.float32, device="cuda") \
        if with_softmax_d else None
    ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = lib.shaobo_fa3_bwd_v2(ptr(do), ptr(q), ptr(k), ptr(v), ptr(out), ptr(lse_d), ptr(dq),
                               ptr(dk), ptr(dv), ptr(delta), ctypes.byref(p))
    torch.cuda.synchronize()
    res = {
        "status": st,
        "dq": dq.float().cpu().numpy(),
        "dk": dk.float().cpu().numpy(),
        "dv": dv.float().cpu().numpy(),
        "delta": None if delta is None else delta.cpu().numpy(),
    }
    return res


def check(res, g, names=("delta", "dq", "dk", "dv"), sel=None, reference_gates=False):
    """Assert the north-star bar (and optionally the reference's own gates)."""
    report = {}
    for n in names:
        a, e = res[n], g[n]
        if sel is not None:
            a, e = a[sel[n]], e[sel[n]]
        m = O.metrics(a, e)
        ok_ns, ok_ref = O.gates(n, m)
        report[n] = m
        assert ok_ns, f"{n} fails max|err|/max|ref| bar: {m}"
        if reference_gates:
            assert ok_ref, f"{n} fails the reference gate: {m}"
    return report
