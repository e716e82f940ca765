"""GPU parity of the component entries against the CPU oracle, called the way
the reference's own harness chains them.

* "seven GEMM" chain (reference src/full_bwd_correctness.cpp:366-392):
  shaobo_fa3_bwd_dot_do_o (SMAX_SSUM) -> packed sidecar in reserved_ptr[3]
  -> shaobo_fa3_bwd_dkv (fp32 dK/dV) -> delta in reserved_ptr[0] ->
  shaobo_fa3_bwd_dq (fp32 dQ), with no workspace, as the reference calls
  them.
* shaobo_fa3_bwd_fused5 from a dot_do_o sidecar of either aux convention
  (reference tests/fused_bwd_correctness.cpp:240-262), fp16 outputs.
* the naive path 1 of shaobo_fa3_bwd_dkv / shaobo_fa3_bwd_dq (reference
  src/dkv_kernel.cpp:1320-1383, src/dq_kernel.cpp:1562-1625), which
  recomputes the forward from Q, K, V through an S^2-sized workspace.

Bar: max|err|/max|ref| <= 1e-2 against the oracle's fp32 gradients.
"""
import ctypes

import numpy as np
import pytest

import fa3_oracle as O
import shaobo_fa3 as F
from gpu_util import check, dev, log

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.load()


def c(x):
    return None if x is None else ctypes.c_void_p(x.data_ptr())


def sidecar(lib, g, p, lse_mode):
    """delta and the packed sidecar from shaobo_fa3_bwd_dot_do_o."""
    B, Hq, S, _ = g["q"].shape
    rows = B * Hq * S
    p.softmax_aux_mode = F.AUX_LSE if lse_mode else F.AUX_SMAX_SSUM
    aux0 = dev(g["lse"] if lse_mode else g["scores_max"], torch)
    aux1 = None if lse_mode else dev(g["scores_sum"], torch)
    delta = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    packed = torch.full((rows * 3,), float("nan"), dtype=torch.float32, device="cuda")
    do, out = dev(g["dout"], torch), dev(g["out"], torch)  # held until the call is done
    st = lib.shaobo_fa3_bwd_dot_do_o(c(do), c(out), c(aux0), c(aux1), c(delta), c(packed),
                                     ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    return delta, packed


@pytest.mark.parametrize("B,H,S,D", [(1, 2, 512, 128), (2, 1, 1024, 128), (1, 2, 256, 64),
                                     (1, 1, 128, 128)])
def test_seven_gemm_chain(B, H, S, D):
    log(f"[case] dot_do_o -> dkv -> dq B={B} H={H} S={S} D={D}")
    lib = F.load()
    g = O.golden(B, H, H, S, D, True)
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=H, head_dim=D, causal=True,
                      softmax_scale=g["scale"], sync=True)
    p.dkv_path = F.DKV_PATH_CANONICAL
    p.dq_path = F.DQ_PATH_CANONICAL
    assert lib.shaobo_fa3_bwd_dkv_workspace_bytes(ctypes.byref(p)) == 0
    assert lib.shaobo_fa3_bwd_dq_workspace_bytes(ctypes.byref(p)) == 0
    delta, packed = sidecar(lib, g, p, lse_mode=False)
    q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
    smax, ssum = dev(g["scores_max"], torch), dev(g["scores_sum"], torch)
    dq = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    dk = torch.full(k.shape, float("nan"), dtype=torch.float32, device="cuda")
    dv = torch.full(v.shape, float("nan"), dtype=torch.float32, device="cuda")
    p.reserved_ptr[3] = packed.data_ptr()
    st = lib.shaobo_fa3_bwd_dkv(c(do), c(q), c(k), c(v), c(out), c(smax), c(ssum), None, c(dk),
                                c(dv), ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    p.reserved_ptr[0] = delta.data_ptr()
    st = lib.shaobo_fa3_bwd_dq(c(do), c(q), c(k), c(v), c(out), c(smax), c(ssum), c(dq), None,
                               None, ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    torch.cuda.synchronize()
    res = {n: x.cpu().numpy() for n, x in (("dq", dq), ("dk", dk), ("dv", dv),
                                            ("delta", delta.view(B, H, S)))}
    rep = check(res, g)
    log({n: round(m["max_rel"], 6) for n, m in rep.items()})


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,lse_mode", [
    (1, 4, 2, 256, 128, True, True),      # GQA
    (1, 2, 2, 1024, 128, True, False),    # split plan, SMAX_SSUM sidecar
    (1, 2, 2, 256, 64, False, True),      # D = 64, non-causal
    (2, 8, 2, 256, 128, False, False),
])
def test_fused5(B, Hq, Hkv, S, D, causal, lse_mode):
    log(f"[case] fused5 B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} lse={lse_mode}")
    lib = F.load()
    g = O.golden(B, Hq, Hkv, S, D, causal)
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D, causal=causal,
                      softmax_scale=g["scale"], sync=True)
    delta, packed = sidecar(lib, g, p, lse_mode)
    nbytes = lib.shaobo_fa3_bwd_fused5_workspace_bytes(ctypes.byref(p))
    assert nbytes > 0
    ws = torch.full((nbytes,), 0xC3, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    q, k, v, do = (dev(g[n], torch) for n in ("q", "k", "v", "dout"))
    dq, dk, dv = (torch.full_like(x, float("nan")) for x in (q, k, v))
    st = lib.shaobo_fa3_bwd_fused5(c(do), c(q), c(k), c(v), c(packed), c(dq), c(dk), c(dv),
                                   ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    torch.cuda.synchronize()
    res = {n: x.float().cpu().numpy() for n, x in (("dq", dq), ("dk", dk), ("dv", dv))}
    rep = check(res, g, names=("dq", "dk", "dv"))
    log({n: round(m["max_rel"], 6) for n, m in rep.items()})


def test_fused5_matches_v2_bitwise():
    """fused5 on an LSE-mode sidecar (max_log2 = LSE log2 e, inv_sum = 1)
    feeds the kernel the same row statistics as v2, so the gradients agree
    bit for bit."""
    log("[case] fused5 vs v2")
    lib = F.load()
    g = O.golden(1, 2, 2, 512, 128, True)
    p = F.make_params(lib, batch=1, seqlen=512, heads_q=2, head_dim=128, causal=True,
                      softmax_scale=g["scale"], sync=True)
    _, packed = sidecar(lib, g, p, lse_mode=True)
    nbytes = lib.shaobo_fa3_bwd_fused5_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    assert lib.shaobo_fa3_bwd_fused5(c(do), c(q), c(k), c(v), c(packed), c(dq), c(dk), c(dv),
                                     ctypes.byref(p)) == F.SUCCESS
    dq2, dk2, dv2 = F.bwd_v2(do, q, k, v, out, dev(g["lse"], torch), causal=True,
                             softmax_scale=g["scale"], sync=True)
    torch.cuda.synchronize()
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2)):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


@pytest.mark.parametrize("B,H,S,D,causal", [(1, 2, 128, 128, True), (1, 1, 256, 128, False),
                                             (2, 1, 200, 128, True), (1, 2, 96, 64, False)])
def test_naive_path_1(B, H, S, D, causal):
    """dkv_path 1 -> fp32 dK / dV and dq_path 1 -> fp32 dQ, each through its
    own S^2-sized workspace (poisoned first), against the oracle; any
    sequence length (no tile alignment), either causal flag."""
    log(f"[case] naive path 1 B={B} H={H} S={S} D={D} causal={causal}")
    lib = F.load()
    g = O.golden(B, H, H, S, D, causal)
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=H, head_dim=D, causal=causal,
                      softmax_scale=g["scale"], sync=True)
    p.dkv_path, p.dq_path = 1, 1
    nbytes = lib.shaobo_fa3_bwd_dkv_workspace_bytes(ctypes.byref(p))
    rows = B * H * S
    assert nbytes == (2 * rows * S + 3 * rows) * 4
    assert lib.shaobo_fa3_bwd_dq_workspace_bytes(ctypes.byref(p)) == nbytes
    ws = torch.full((nbytes,), 0xC3, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    q, k, v, do, out = (dev(g[n], torch) for n in ("q", "k", "v", "dout", "out"))
    dq = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    dk = torch.full(k.shape, float("nan"), dtype=torch.float32, device="cuda")
    dv = torch.full(v.shape, float("nan"), dtype=torch.float32, device="cuda")
    st = lib.shaobo_fa3_bwd_dkv(c(do), c(q), c(k), c(v), c(out), None, None, None, c(dk), c(dv),
                                ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    ws.fill_(0xC3)
    st = lib.shaobo_fa3_bwd_dq(c(do), c(q), c(k), c(v), c(out), None, None, c(dq), None, None,
                               ctypes.byref(p))
    assert st == F.SUCCESS, F.status_name(st)
    torch.cuda.synchronize()
    res = {n: x.cpu().numpy() for n, x in (("dq", dq), ("dk", dk), ("dv", dv))}
    rep = check(res, g, names=("dq", "dk", "dv"))
    log({n: round(m["max_rel"], 6) for n, m in rep.items()})
