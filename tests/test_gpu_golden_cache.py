"""The reference harness flow from a golden cache (src/full_bwd_correctness.cpp:
186-233, 366-392, 471-500): load the cache, form LSE = max * scale + ln(sum),
run shaobo_fa3_bwd_v2 -- and the dot_do_o -> dkv -> dq chain -- and compare
with the cache's fp32 gradients under the reference's gates and the north-star
bar."""
import ctypes
import os
import sys

import numpy as np
import pytest

import golden_cache as GC
import shaobo_fa3 as F
from gpu_util import check, dev, log, run_v2

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden_cache as MK  # noqa: E402

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F.load()


def as_golden(arrays, causal, scale):
    """Cache arrays in the oracle's dict form used by the GPU helpers."""
    g = {"q": arrays["q.f16"], "k": arrays["k.f16"], "v": arrays["v.f16"],
         "dout": arrays["dout.f16"], "out": arrays["o.f16"],
         "scores_max": arrays["scores_max.f32"], "scores_sum": arrays["scores_sum.f32"],
         "delta": arrays["delta.f32"], "dq": arrays["dq.f32"], "dk": arrays["dk.f32"],
         "dv": arrays["dv.f32"], "causal": bool(causal), "scale": scale}
    g["lse"] = GC.lse_from(g["scores_max"], g["scores_sum"], scale)
    return g


@pytest.mark.parametrize("hq,hkv,s,causal", [(1, 1, 1024, 1), (4, 2, 128, 1), (2, 2, 256, 0)])
def test_v2_from_golden_cache(tmp_path, hq, hkv, s, causal):
    log(f"[case] golden cache v2 Hq{hq} Hkv{hkv} S{s} causal{causal}")
    dims = dict(batch=1, heads_q=hq, heads_kv=hkv, seqlen=s, head_dim=128)
    scale = GC.DEFAULT_SCALE
    path = GC.write(tmp_path, MK.oracle_arrays(causal=causal, scale=scale, **dims),
                    causal=causal, scale=scale, **dims)
    g = as_golden(GC.read(path, causal=causal, scale=scale, **dims), causal, scale)
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS
    check(res, g, reference_gates=True)


def test_component_chain_from_golden_cache(tmp_path):
    """SMAX_SSUM dot_do_o -> dkv (sidecar in reserved_ptr[3]) -> dq (delta in
    reserved_ptr[0]), fp32 outputs, no workspace; the cache's packed sidecar
    equals the one dot_do_o writes."""
    log("[case] golden cache seven-gemm chain")
    dims = dict(batch=1, heads_q=2, heads_kv=2, seqlen=512, head_dim=128)
    scale = GC.DEFAULT_SCALE
    path = GC.write(tmp_path, MK.oracle_arrays(causal=1, scale=scale, **dims), causal=1,
                    scale=scale, **dims)
    a = GC.read(path, causal=1, scale=scale, **dims)
    lib = F.load()
    p = F.make_params(lib, batch=1, seqlen=512, heads_q=2, head_dim=128, causal=True,
                      softmax_scale=scale, sync=True)
    p.softmax_aux_mode = F.AUX_SMAX_SSUM
    p.dkv_path, p.dq_path = F.DKV_PATH_CANONICAL, F.DQ_PATH_CANONICAL
    t = {n: dev(a[n], torch) for n in ("q.f16", "k.f16", "v.f16", "o.f16", "dout.f16",
                                        "scores_max.f32", "scores_sum.f32")}
    rows = 2 * 512
    delta = torch.zeros(rows, dtype=torch.float32, device="cuda")
    packed = torch.zeros(rows * 3, dtype=torch.float32, device="cuda")
    dq = torch.zeros((1, 2, 512, 128), dtype=torch.float32, device="cuda")
    dk, dv = torch.zeros_like(dq), torch.zeros_like(dq)
    c = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())  # noqa: E731
    assert lib.shaobo_fa3_bwd_dot_do_o(c(t["dout.f16"]), c(t["o.f16"]), c(t["scores_max.f32"]),
                                       c(t["scores_sum.f32"]), c(delta), c(packed),
                                       ctypes.byref(p)) == F.SUCCESS
    p.reserved_ptr[3] = packed.data_ptr()
    assert lib.shaobo_fa3_bwd_dkv(c(t["dout.f16"]), c(t["q.f16"]), c(t["k.f16"]), c(t["v.f16"]),
                                  c(t["o.f16"]), c(t["scores_max.f32"]), c(t["scores_sum.f32"]),
                                  None, c(dk), c(dv), ctypes.byref(p)) == F.SUCCESS
    p.reserved_ptr[0] = delta.data_ptr()
    assert lib.shaobo_fa3_bwd_dq(c(t["dout.f16"]), c(t["q.f16"]), c(t["k.f16"]), c(t["v.f16"]),
                                 c(t["o.f16"]), c(t["scores_max.f32"]), c(t["scores_sum.f32"]),
                                 c(dq), None, None, ctypes.byref(p)) == F.SUCCESS
    torch.cuda.synchronize()
    g = as_golden(a, 1, scale)
    res = {"delta": delta.cpu().numpy().reshape(1, 2, 512), "dq": dq.cpu().numpy(),
           "dk": dk.cpu().numpy(), "dv": dv.cpu().numpy()}
    check(res, g, reference_gates=True)
    pk = packed.cpu().numpy().reshape(1, 2, 512, 3)
    np.testing.assert_allclose(pk[..., :2], a["packed_sidecar.f32"][..., :2], rtol=1e-6)
    np.testing.assert_allclose(pk[..., 2], a["packed_sidecar.f32"][..., 2], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("hq,hkv", [(1, 1), (4, 2)])
def test_v2_on_reference_tool_cache(hq, hkv):
    """v2 on the inputs of a cache written by the reference's own tool
    (fixtures under tests/golden/reference_caches, made by
    tests/golden/make_reference_caches.py), against that tool's fp32
    gradients, under the reference's gates and the north-star bar."""
    log(f"[case] reference tool cache v2 Hq{hq} Hkv{hkv} S128")
    dims = dict(batch=1, heads_q=hq, heads_kv=hkv, seqlen=128, head_dim=128)
    path = os.path.join(HERE, "golden", "reference_caches", GC.cache_key(causal=1, **dims))
    g = as_golden(GC.read(path, causal=1, **dims), 1, GC.DEFAULT_SCALE)
    res = run_v2(g, torch)
    assert res["status"] == F.SUCCESS
    rep = check(res, g, reference_gates=True)
    log({n: round(m["max_rel"], 6) for n, m in rep.items()})
