"""GPU parity of shaobo_fa3_bwd_v2 (and the legacy / component entries)
against the CPU oracle, through the C ABI, on the BASELINE configs.

Bar (north star): max|err|/max|ref| <= 1e-2 for dQ/dK/dV, delta within 1e-4
relative; the reference's own gates (src/full_bwd_correctness.cpp:471-500)
are asserted too on its deterministic pattern inputs, for which its absolute
bounds were designed.  The full-size configs compare every (batch, kv-head)
group with the oracle.
"""
import ctypes

import numpy as np
import pytest

import fa3_oracle as O
import shaobo_fa3 as F
from gpu_util import check, dev, log, run_v2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.load()


CASES = [
    # B, Hq, Hkv, S, D, causal
    (1, 1, 1, 128, 128, True),    # P1 plumbing
    (1, 1, 1, 1024, 128, True),   # P2 diagnosis
    (1, 4, 4, 2048, 128, True),   # P3 headline
    (1, 1, 1, 128, 128, False),
    (1, 4, 2, 256, 128, True),    # GQA G=2
    (2, 8, 2, 256, 128, False),   # GQA G=4, batch 2, non-causal
    (1, 2, 2, 512, 64, True),     # D = 64
    (1, 2, 1, 384, 64, False),    # D = 64 GQA, S not a power of two
    # split plan (causal, one query head per KV head, S / 64 even and >= 4):
    (1, 1, 1, 256, 128, True),    # smallest: M = S / 128 = 2
    (1, 3, 3, 384, 128, True),    # odd M = 3, 3 groups (no XCD-aligned map)
    (2, 2, 2, 1024, 128, True),   # batch 2: 4 groups
    (1, 5, 5, 640, 64, True),     # M = 5, D = 64
    (1, 2, 2, 1536, 128, True),   # M = 12: short jobs after the pieces of kinds 1 and 2
    (1, 2, 2, 4096, 64, True),    # M = 32, D = 64, 256 jobs: the largest split plan
    (1, 8, 8, 2048, 64, True),    # 512 jobs: one job per workgroup (past the split plan's 256)
    (1, 9, 9, 2048, 64, True),    # 576 jobs: causal, one head per group, default plan
    (1, 4, 2, 1024, 128, True),   # head-split plan: G = 2, one head per chunk
    (1, 8, 1, 1024, 128, True),   # head-split plan: MQA, G = 8, one head per chunk
    (1, 16, 2, 2048, 64, False),  # head-split plan: full, D = 64, two heads per chunk
    (1, 12, 12, 512, 128, True),  # split plan over 12 groups: XCD-interleaved job map
    (1, 12, 12, 1024, 128, True), # 384 jobs: one job per workgroup, interleaved
    (3, 8, 2, 512, 64, False),    # 6 groups, head split, one job per workgroup, interleaved
    (1, 28, 7, 1024, 128, True),  # 7 groups in 56 parts over 8 XCDs, persistent, interleaved
    (1, 7, 7, 1920, 128, True),   # 8 parts do not divide a group's 60 jobs: the map's fallback
    (1, 12, 6, 1920, 128, True),  # ... GQA, persistent, fallback interleaved
    (1, 7, 7, 1920, 64, False),   # ... full attention, D = 64
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", CASES)
def test_v2_matches_oracle(B, Hq, Hkv, S, D, causal):
    log(f"[case] v2 B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}")
    g = O.golden(B, Hq, Hkv, S, D, causal)
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    rep = check(res, g)
    log({k: (round(v["max_rel"], 6), round(v["max_abs"], 6)) for k, v in rep.items()})


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,scale", [
    (1, 2, 1, 256, 64, False, 0.75),   # c = scale log2 e > 1: unscaled instantiation
    (1, 4, 2, 384, 128, True, 1.0),    # c > 1, causal, D = 128
    (1, 4, 2, 384, 128, True, 0.69),   # just below ln 2: operands scaled by c = 0.995
    (2, 4, 2, 256, 64, False, 0.02),   # small c, scaled
    (1, 1, 1, 256, 128, True, 1.0),    # split plan (unscaled at every scale)
    (1, 1, 1, 128, 128, True, 1.0),    # level-order default plan (causal, G = 1), unscaled
    (1, 9, 9, 2048, 64, True, 1.0),    # ... persistent (576 jobs), unscaled
    (1, 8, 1, 1024, 128, True, 1.0),   # head-split plan, unscaled
])
def test_v2_softmax_scales(B, Hq, Hkv, S, D, causal, scale):
    """The default plan's score waves multiply their resident operand (K, or
    Q in the dQ role) by c = scale log2 e only when c <= 1, where the product
    cannot overflow fp16; larger scales run the unscaled instantiations,
    which apply c in the loop.  Both sides of that threshold match the
    oracle."""
    log(f"[case] v2 scale={scale} B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}")
    g = O.golden(B, Hq, Hkv, S, D, causal, scale=scale)
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    rep = check(res, g)
    log({k: (round(v["max_rel"], 6), round(v["max_abs"], 6)) for k, v in rep.items()})


@pytest.mark.parametrize("S,causal", [(128, True), (1024, True), (256, False)])
def test_v2_reference_pattern_inputs(S, causal):
    """The reference's own deterministic inputs (generate_full_bwd_golden.py:
    135-151) under its own absolute gates."""
    log(f"[case] pattern S={S} causal={causal}")
    g = O.golden(1, 1, 1, S, 128, causal, kind="pattern")
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS
    check(res, g, reference_gates=True)


def test_v2_gqa_reference_gate_shape():
    """reference docs/tridao_fa3_bwd_api.md:108-119 gate shape Hq4/Hkv2/S128."""
    log("[case] pattern GQA Hq4 Hkv2 S128")
    g = O.golden(1, 4, 2, 128, 128, True, kind="pattern")
    res = run_v2(g, torch)
    check(res, g, reference_gates=True)


@pytest.mark.parametrize("hq,hkv,s,d", [(4, 2, 384, 128),    # one dKV job per KV head
                                          (8, 1, 1024, 128),   # head split: ordered reduction
                                          (2, 2, 1024, 128),   # split plan (causal, G = 1)
                                          (2, 2, 512, 64)])
def test_deterministic_mode_is_bitwise_repeatable(hq, hkv, s, d):
    """No atomics in the sums: two runs agree bit for bit, also when long
    causal jobs are split in two and their partial sums meet in whichever
    workgroup finishes second."""
    log(f"[case] deterministic S={s} Hq{hq} Hkv{hkv} D{d}")
    g = O.golden(1, hq, hkv, s, d, True)
    r1 = run_v2(g, torch, deterministic=True)
    r2 = run_v2(g, torch, deterministic=True)
    check(r1, g)
    for n in ("dq", "dk", "dv", "delta"):
        np.testing.assert_array_equal(r1[n], r2[n])


@pytest.mark.parametrize("hq,s,d", [(2, 1024, 128), (4, 2048, 128), (2, 512, 64)])
def test_split_plan_reused_workspace(hq, s, d):
    """Split plan, one workspace kept across calls on different inputs: the
    partial sums and synchronisation words of one call must never leak into
    the next (the words are compared with each launch's own epoch; partial
    sums are read only after the other piece of the same call has written
    them)."""
    log(f"[case] split plan reused workspace Hq{hq} S{s} D{d}")
    ws = None
    for seed in range(3):
        g = O.golden(1, hq, hq, s, d, True, seed_offset=101 * seed)
        if ws is None:
            lib = F.load()
            p = F.make_params(lib, batch=1, seqlen=s, heads_q=hq, head_dim=d, causal=True)
            ws = torch.empty(lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p)),
                             dtype=torch.uint8, device="cuda")
        res = run_v2(g, torch, workspace=ws)
        assert res["status"] == F.SUCCESS
        check(res, g)


@pytest.mark.parametrize("hq,s,d", [(4, 2048, 128), (2, 1024, 64)])
def test_split_plan_back_to_back_calls(hq, s, d):
    """Many v2 calls queued on the null stream without synchronisation (one
    workspace, as a training loop would): each call's preprocess rewrites the
    row arrays the previous call's main kernel read, so stream order must
    hold; the last result is bitwise the synchronised one."""
    log(f"[case] back-to-back calls Hq{hq} S{s} D{d}")
    lib = F.load()
    g = O.golden(1, hq, hq, s, d, True)
    ref = run_v2(g, torch)
    check(ref, g)
    q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
    lse = dev(g["lse"], torch)
    p = F.make_params(lib, batch=1, seqlen=s, heads_q=hq, head_dim=d, causal=True,
                      softmax_scale=g["scale"])
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    c = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    for _ in range(200):
        st = lib.shaobo_fa3_bwd_v2(c(do), c(q), c(k), c(v), c(out), c(lse), c(dq), c(dk), c(dv),
                                   None, ctypes.byref(p))
        assert st == F.SUCCESS
    torch.cuda.synchronize()
    for n, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        np.testing.assert_array_equal(t.float().cpu().numpy(), ref[n])


def test_split_wait_failure_is_reported():
    """A split job's second piece that gives up waiting for the first piece's
    partial sums writes the launch's epoch into the workspace's error word,
    and the synchronised call returns HIP_ERROR instead of a silently wrong
    sum.  Forced from the host: a spin limit of 0 polls makes every wait give
    up at once, while every workgroup still runs to its end.  A wait that
    finds the partial sums already published carries on, so whether a call
    fails depends on timing (at P3 a call has several waits that give up,
    typically): calls are repeated until one reports the failure, and every
    call that reports SUCCESS must be correct.  With the default limit back,
    the next call is correct and reports SUCCESS."""
    log("[case] split wait gives up (spin limit 0) at P3")
    lib = F.load()
    g = O.golden(1, 4, 4, 2048, 128, True)
    failed = 0
    lib.shaobo_fa3_ext_set_split_spin_limit(0)
    try:
        for _ in range(20):
            res = run_v2(g, torch)
            if res["status"] == F.HIP_ERROR:
                failed += 1
                break
            assert res["status"] == F.SUCCESS, F.status_name(res["status"])
            check(res, g)
    finally:
        lib.shaobo_fa3_ext_set_split_spin_limit(1 << 24)
    assert failed, "no split wait gave up in 20 calls with spin limit 0"
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    check(res, g)


def test_concurrent_calls_on_two_streams():
    """Two different problems launched on two streams through the stream entry
    (shaobo_fa3_bwd_v2_on_stream), each with its own workspace: the library
    keeps no state between calls, so both match their oracles."""
    log("[case] concurrent calls on two streams")
    lib = F.load()
    fn = lib.shaobo_fa3_bwd_v2_on_stream
    fn.argtypes = [ctypes.c_void_p] * 10 + [ctypes.POINTER(F.Params), ctypes.c_void_p]
    fn.restype = ctypes.c_int
    c = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    gs = [O.golden(1, 4, 4, 2048, 128, True), O.golden(2, 4, 2, 512, 64, False, seed_offset=7)]
    keep, outs = [], []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for g, stream in zip(gs, streams):
        B, Hq, S, D = g["q"].shape
        Hkv = g["k"].shape[1]
        q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
        lse = dev(g["lse"], torch)
        p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D,
                          causal=g["causal"], softmax_scale=g["scale"])
        nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        delta = torch.empty((B, Hq, S), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()  # inputs written before either stream starts
        st = fn(c(do), c(q), c(k), c(v), c(out), c(lse), c(dq), c(dk), c(dv), c(delta),
                ctypes.byref(p), ctypes.c_void_p(stream.cuda_stream))
        assert st == F.SUCCESS
        keep.append((q, k, v, do, out, lse, ws, p))
        outs.append((dq, dk, dv, delta))
    torch.cuda.synchronize()
    for g, (dq, dk, dv, delta) in zip(gs, outs):
        res = {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
               "dv": dv.float().cpu().numpy(), "delta": delta.cpu().numpy()}
        check(res, g)


def test_default_scale_and_internal_delta():
    """softmax_scale_is_set = 0 -> 1/sqrt(D); softmax_d = NULL keeps delta internal."""
    log("[case] default scale, softmax_d NULL")
    g = O.golden(1, 2, 2, 256, 128, True)
    res = run_v2(g, torch, with_softmax_d=False, scale_is_set=False)
    assert res["status"] == F.SUCCESS
    check(res, g, names=("dq", "dk", "dv"))


def test_legacy_entry_smax_ssum():
    """shaobo_fa3_bwd with SMAX_SSUM aux (raw max + sum, reference
    include/shaobo_fa3_api.h:135-147) gives the v2 result."""
    log("[case] legacy smax/ssum")
    lib = F.load()
    g = O.golden(1, 2, 1, 512, 128, True)
    t = {n: dev(g[n], torch) for n in ("q", "k", "v", "dout", "out", "scores_max",
                                         "scores_sum")}
    p = F.make_params(lib, batch=1, seqlen=512, heads_q=2, heads_kv=1, head_dim=128, causal=True,
                      softmax_scale=g["scale"], sync=True)
    p.softmax_aux_mode = F.AUX_SMAX_SSUM
    nbytes = lib.shaobo_fa3_bwd_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = (torch.empty_like(t[n]) for n in ("q", "k", "v"))
    c = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = lib.shaobo_fa3_bwd(c(t["dout"]), c(t["q"]), c(t["k"]), c(t["v"]), c(t["out"]),
                            c(t["scores_max"]), c(t["scores_sum"]), c(dq), c(dk), c(dv),
                            ctypes.byref(p))
    torch.cuda.synchronize()
    assert st == F.SUCCESS
    res = {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
           "dv": dv.float().cpu().numpy()}
    check(res, g, names=("dq", "dk", "dv"))


@pytest.mark.parametrize("lse_mode", [True, False])
def test_dot_do_o_component(lse_mode):
    """delta + packed sidecar [max_log2, inv_sum, delta] (reference
    src/dot_do_o_kernel.cpp:49-61)."""
    log(f"[case] dot_do_o lse_mode={lse_mode}")
    lib = F.load()
    g = O.golden(1, 2, 2, 256, 128, True)
    rows = 2 * 256
    p = F.make_params(lib, batch=1, seqlen=256, heads_q=2, head_dim=128, causal=True,
                      softmax_scale=g["scale"], sync=True)
    p.softmax_aux_mode = F.AUX_LSE if lse_mode else F.AUX_SMAX_SSUM
    do, out = dev(g["dout"], torch), dev(g["out"], torch)
    aux0 = dev(g["lse"] if lse_mode else g["scores_max"], torch)
    aux1 = None if lse_mode else dev(g["scores_sum"], torch)
    delta = torch.zeros(rows, dtype=torch.float32, device="cuda")
    packed = torch.zeros(rows * 3, dtype=torch.float32, device="cuda")
    c = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())  # noqa: E731
    st = lib.shaobo_fa3_bwd_dot_do_o(c(do), c(out), c(aux0), c(aux1), c(delta), c(packed),
                                     ctypes.byref(p))
    torch.cuda.synchronize()
    assert st == F.SUCCESS
    d = delta.cpu().numpy()
    pk = packed.cpu().numpy().reshape(rows, 3)
    ok, _ = O.gates("delta", O.metrics(d, g["delta"].ravel()))
    assert ok
    np.testing.assert_array_equal(pk[:, 2], d)
    log2e = np.float32(1.4426950408889634)
    if lse_mode:
        np.testing.assert_allclose(pk[:, 0], g["lse"].ravel() * log2e, rtol=1e-6)
        np.testing.assert_array_equal(pk[:, 1], 1.0)
    else:
        sl2 = np.float32(g["scale"]) * log2e
        np.testing.assert_allclose(pk[:, 0], g["scores_max"].ravel() * sl2, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(pk[:, 1], 1.0 / g["scores_sum"].ravel(), rtol=1e-6)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [
    (2, 32, 8, 4096, 128, True),    # P4 GQA
    (2, 16, 16, 8192, 64, False),   # P5
    (1, 32, 1, 4096, 128, True),    # MQA at batch 1: head-split plan, 4 heads per chunk
    (1, 19, 19, 4096, 64, True),    # 19 groups, 3 per XCD, 9.5 jobs per CU: tail interleaving
])
def test_full_size_configs(B, Hq, Hkv, S, D, causal):
    """The whole P4 / P5 backward against the oracle (forward and backward
    on the CPU, about 10 s with 16 threads), checked per (batch, kv-head)
    group -- dK / dV of the group's KV head, dQ / delta of its query heads,
    each against its own max|ref| -- so a job-map error confined to some
    groups cannot hide behind the others' magnitudes (the reference's gate
    compares whole tensors: src/full_bwd_correctness.cpp:471-500)."""
    log(f"[case] full-size B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}")
    g = O.golden(B, Hq, Hkv, S, D, causal)
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS
    check_per_group(res, g)


def check_per_group(res, g):
    """The bar on the whole tensors and on every (batch, kv-head) group: dK /
    dV of the group's KV head, dQ / delta of its query heads."""
    rep = check(res, g)
    log({k: round(v["max_rel"], 6) for k, v in rep.items()})
    B, Hq, _, _ = g["q"].shape
    Hkv = g["k"].shape[1]
    G = Hq // Hkv
    worst = {}
    for b in range(B):
        for hk in range(Hkv):
            qsel = (b, slice(hk * G, hk * G + G))
            sel = {"delta": qsel, "dq": qsel, "dk": (b, hk), "dv": (b, hk)}
            for n, m in check(res, g, sel=sel).items():
                worst[n] = max(worst.get(n, 0.0), m["max_rel"])
    log({"worst group": {k: round(v, 6) for k, v in worst.items()}})


@pytest.mark.parametrize("hq,hkv", [
    (16, 8),  # 1536 jobs, one dKV job per KV head
    (8, 2),   # 1024 jobs, head-split plan (a merged dKV job, 256 steps, would
              # outlast a CU's share of the work)
])
@pytest.mark.parametrize("dtype,layout,scale", [
    ("bf16", "bhsd", None),   # bf16 instantiation of the persistent plan
    ("fp16", "bshd", None),   # BSHD strides in the persistent job loop
    ("fp16", "bhsd", 1.0),    # scale 1: c = log2(e) > 1, the unscaled instantiation
])
def test_persistent_plan_variants(dtype, layout, scale, hq, hkv):
    """The persistent default plan (more than two jobs per CU) at B1 S4096
    D128 causal, GQA, in the instantiations the BASELINE configs do not reach
    -- bf16, BSHD, unscaled resident operands -- against the oracle, per
    (batch, kv-head) group; BSHD also bit-equal to BHSD."""
    log(f"[case] persistent plan {dtype} {layout} scale={scale} B1 Hq{hq} Hkv{hkv} S4096 D128 causal")
    g = O.golden(1, hq, hkv, 4096, 128, True, scale=scale, dtype=dtype)
    res = run_v2(g, torch, bshd=layout == "bshd")
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    check_per_group(res, g)
    if layout == "bshd":
        ref = run_v2(g, torch)
        for n in ("dq", "dk", "dv", "delta"):
            np.testing.assert_array_equal(res[n], ref[n])


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [
    (1, 1, 1, 128, 128, True),
    (1, 4, 4, 2048, 128, True),   # P3 shape, split plan
    (1, 4, 2, 256, 128, True),    # GQA
    (2, 8, 2, 256, 128, False),
    (1, 2, 2, 512, 64, True),
    (1, 8, 1, 1024, 128, True),   # head-split plan
])
def test_v2_bf16(B, Hq, Hkv, S, D, causal):
    """bf16 tensors (this build's extension): bf16 oracle, bf16 bar."""
    log(f"[case] bf16 B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}")
    g = O.golden(B, Hq, Hkv, S, D, causal, dtype="bf16")
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    rep = check(res, g)
    log({k: round(v["max_rel"], 6) for k, v in rep.items()})


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,dtype", [
    (1, 4, 4, 2048, 128, True, "fp16"),   # split plan
    (2, 8, 2, 256, 128, False, "fp16"),   # GQA, batch 2
    (1, 4, 2, 384, 64, True, "fp16"),
    (2, 4, 2, 256, 128, True, "bf16"),
    (1, 8, 2, 1024, 64, True, "bf16"),    # head-split plan: the reduction's BSHD strides
])
def test_v2_bshd(B, Hq, Hkv, S, D, causal, dtype):
    """[B, S, H, D] tensors (this build's extension), same values as BHSD:
    the result equals the BHSD run bit for bit and meets the bar."""
    log(f"[case] BSHD B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} {dtype}")
    g = O.golden(B, Hq, Hkv, S, D, causal, dtype=dtype)
    res = run_v2(g, torch, bshd=True)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    check(res, g)
    ref = run_v2(g, torch)
    for n in ("dq", "dk", "dv", "delta"):
        np.testing.assert_array_equal(res[n], ref[n])
