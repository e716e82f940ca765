"""GPU race checks (the counterpart of the reference's stress run that caught
races in its kernel, reference source_status.md:608-612): the main kernel's
race-check instantiation -- the same arithmetic, every job started on an LDS
poisoned with NaN bytes, a full wait and a barrier after every LDS phase of
the pipeline -- must give the fast kernel's outputs bit for bit, under the
split plan, the persistent plan and the one-job-per-workgroup plan.  A read
of LDS that a job did not write shows up as NaN (and fails the oracle
check), a race between the fast kernel's waves as a bitwise difference.
Also here: the split-wait give-up reported to unsynchronised callers, and
the split synchronisation words left cleared after a give-up."""
import ctypes

import numpy as np
import pytest

import fa3_oracle as O
import shaobo_fa3 as F
from gpu_util import check, log, run_v2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.load()


def race_checked(g, **kw):
    lib = F.load()
    lib.shaobo_fa3_ext_set_race_check(1)
    try:
        return run_v2(g, torch, **kw)
    finally:
        lib.shaobo_fa3_ext_set_race_check(0)


RACE_CASES = [
    # B, Hq, Hkv, S, D, causal, dtype, plan
    (1, 1, 1, 128, 128, True, "fp16"),     # P1: one job per workgroup
    (1, 1, 1, 1024, 128, True, "fp16"),    # P2: split plan
    (1, 4, 4, 2048, 128, True, "fp16"),    # P3: split plan (the headline)
    (1, 9, 9, 2048, 64, True, "fp16"),     # 576 jobs: persistent plan, D 64
    (4, 16, 8, 1024, 128, True, "fp16"),   # 1536 jobs: persistent plan, GQA, D 128
    (2, 16, 4, 1024, 128, True, "fp16"),   # 1024 jobs: head-split plan
    (1, 16, 2, 2048, 64, False, "fp16"),   # head-split plan, two query heads per chunk
    (2, 16, 4, 2048, 128, True, "fp16"),   # 1280 jobs: five per workgroup
    (2, 8, 8, 1024, 64, False, "fp16"),    # 512 jobs: one job per workgroup, full attention
    (3, 8, 8, 1024, 64, False, "fp16"),    # 768 jobs: persistent plan, full attention
    (1, 2, 2, 512, 128, True, "bf16"),     # bf16, split plan
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,dtype", RACE_CASES)
def test_race_check_kernel_is_bit_equal(B, Hq, Hkv, S, D, causal, dtype):
    log(f"[case] race check B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} {dtype}")
    g = O.golden(B, Hq, Hkv, S, D, causal, dtype=dtype)
    fast = run_v2(g, torch)
    slow = race_checked(g)
    assert fast["status"] == F.SUCCESS and slow["status"] == F.SUCCESS
    check(slow, g)
    for n in ("dq", "dk", "dv", "delta"):
        np.testing.assert_array_equal(slow[n], fast[n], err_msg=n)


def test_race_check_component_chain_unaffected():
    """The race-check switch selects the main kernel's instantiation only: the
    fused5 entry (which runs it) stays bit-equal to v2 under the switch."""
    log("[case] race check through the legacy entry (SMAX/SSUM)")
    lib = F.load()
    g = O.golden(1, 2, 2, 256, 128, True)
    fast = run_v2(g, torch)
    lib.shaobo_fa3_ext_set_race_check(1)
    try:
        slow = run_v2(g, torch, deterministic=True)
    finally:
        lib.shaobo_fa3_ext_set_race_check(0)
    for n in ("dq", "dk", "dv"):
        np.testing.assert_array_equal(slow[n], fast[n], err_msg=n)


def _split_sync_region(ws, B, H, S):
    """The split plan's synchronisation words of a v2 workspace (a uint8
    view): after the error word's 256-byte region come the -lse2 and -delta
    rows (B H S fp32 each, 256-byte aligned) and the 1 KiB of job-queue
    counters, then two 64-bit words per split job of each role (the words of
    jobs the plan leaves whole are never touched)."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    rows = align(B * H * S * 4)
    off = 256 + 2 * rows + 1024
    n_split = B * H * (S // 128)
    return ws[off:off + n_split * 4 * 8]


def _split_sync_words(ws, B, H, S):
    return _split_sync_region(ws, B, H, S).cpu().numpy().view(np.uint64)


def test_split_giveup_visible_without_sync():
    """A split wait that gives up in an unsynchronised call (spin limit 0,
    sync_after_launch = 0) is reported afterwards by the workspace query and
    counted by the GPU's give-up count; the query clears the word, so it
    reports once; the synchronisation words are all left cleared (a replay
    of a captured graph reuses the epoch and must not find a stale 'ready');
    the next call is correct and changes neither.  A wait that finds the
    partial sums already published carries on, so calls are repeated until
    one gives up; a call in between reports nothing and is correct."""
    log("[case] unsynchronised split give-up at P3, queried afterwards")
    lib = F.load()
    g = O.golden(1, 4, 4, 2048, 128, True)
    q, k, v, do, out = (torch.from_numpy(g[n]).cuda() for n in ("q", "k", "v", "dout", "out"))
    lse = torch.from_numpy(g["lse"]).cuda()
    p = F.make_params(lib, batch=1, seqlen=2048, heads_q=4, heads_kv=4, head_dim=128,
                      causal=True, softmax_scale=g["scale"], sync=False)
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    ws = torch.full((nbytes,), 0xC3, dtype=torch.uint8, device="cuda")
    # the synchronisation words start cleared, so that any word a launch
    # leaves set shows
    _split_sync_region(ws, 1, 4, 2048).zero_()
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    c = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = torch.cuda.current_stream().cuda_stream
    count0 = ctypes.c_ulonglong(0)
    assert lib.shaobo_fa3_ext_split_error_count(ctypes.c_void_p(stream),
                                                ctypes.byref(count0)) == F.SUCCESS
    # a poisoned workspace that no launch wrote is not an error
    assert lib.shaobo_fa3_ext_split_status(c(ws), ctypes.c_void_p(stream)) == F.SUCCESS

    def call():
        st = lib.shaobo_fa3_bwd_v2(c(do), c(q), c(k), c(v), c(out), c(lse), c(dq), c(dk), c(dv),
                                   None, ctypes.byref(p))
        assert st == F.SUCCESS, F.status_name(st)

    count1 = ctypes.c_ulonglong(0)
    lib.shaobo_fa3_ext_set_split_spin_limit(0)
    try:
        for _ in range(20):
            call()
            torch.cuda.synchronize()
            words = _split_sync_words(ws, 1, 4, 2048)
            assert (words == 0).all(), f"{int((words != 0).sum())} split words left set"
            assert lib.shaobo_fa3_ext_split_error_count(ctypes.c_void_p(stream),
                                                        ctypes.byref(count1)) == F.SUCCESS
            if count1.value > count0.value:
                break
            # no wait gave up in this call: nothing reported, and it is correct
            assert lib.shaobo_fa3_ext_split_status(c(ws), ctypes.c_void_p(stream)) == F.SUCCESS
            check({"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
                   "dv": dv.float().cpu().numpy()}, g, names=("dq", "dk", "dv"))
    finally:
        lib.shaobo_fa3_ext_set_split_spin_limit(1 << 24)
    assert count1.value > count0.value, "no split wait gave up in 20 calls with spin limit 0"
    assert lib.shaobo_fa3_ext_split_status(c(ws), ctypes.c_void_p(stream)) == F.HIP_ERROR
    assert lib.shaobo_fa3_ext_split_status(c(ws), ctypes.c_void_p(stream)) == F.SUCCESS
    # the same workspace again, default limit: correct, nothing reported
    call()
    torch.cuda.synchronize()
    assert lib.shaobo_fa3_ext_split_status(c(ws), ctypes.c_void_p(stream)) == F.SUCCESS
    count2 = ctypes.c_ulonglong(0)
    assert lib.shaobo_fa3_ext_split_error_count(ctypes.c_void_p(stream),
                                                ctypes.byref(count2)) == F.SUCCESS
    assert count2.value == count1.value
    assert (_split_sync_words(ws, 1, 4, 2048) == 0).all()
    res = {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
           "dv": dv.float().cpu().numpy()}
    check(res, g, names=("dq", "dk", "dv"))


def test_split_status_arguments():
    lib = F.load()
    assert lib.shaobo_fa3_ext_split_error_count(None, None) == F.INVALID_VALUE
    n = ctypes.c_ulonglong(0)
    assert lib.shaobo_fa3_ext_split_error_count(None, ctypes.byref(n)) == F.SUCCESS
    # the no-allocation scratch array (NULL workspace)
    assert lib.shaobo_fa3_ext_split_status(None, None) in (F.SUCCESS, F.HIP_ERROR)
    assert lib.shaobo_fa3_ext_split_status(None, None) == F.SUCCESS
