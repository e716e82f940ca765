"""The stage-selecting extension entry shaobo_fa3_ext_bwd_v2_stages (no
reference counterpart; bench.py times the main kernel alone with it):
preprocess then main kernel equals one full call bit for bit, and repeated
main-kernel-only launches on one workspace keep producing the full result --
in the persistent plan (more than two jobs per CU) that needs the job queues
to reset themselves at the end of every launch, which the poisoned outputs
between the launches would expose."""
import ctypes

import pytest

import shaobo_fa3 as F
from gpu_util import log

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CASES = [
    # (B, Hq, Hkv, S, D, causal)   plan
    (1, 4, 4, 2048, 128, True),    # split plan (P3)
    (1, 5, 5, 4096, 128, False),   # persistent: 5 heads x 64 tiles x 2 roles = 640 jobs
    (1, 4, 4, 4096, 128, False),   # 512 jobs: one job per workgroup
    (2, 8, 2, 2048, 64, True),     # persistent, GQA, D 64 (B 2 x Hkv 2 x 32 x 5 = 640 jobs)
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", CASES)
def test_stages_match_full_call(B, Hq, Hkv, S, D, causal):
    log(f"stages B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} causal={causal}")
    lib = F.load()
    gen = torch.Generator(device="cuda").manual_seed(7)
    mk = lambda h: torch.randn((B, h, S, D), generator=gen, device="cuda").half()  # noqa: E731
    q, k, v, do, out = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq), mk(Hq)
    lse = torch.randn((B, Hq, S), generator=gen, device="cuda").float() + 8.0
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D,
                      causal=causal, softmax_scale=D ** -0.5, sync=True)
    nb = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    ws = torch.full((nb,), 0xC3, dtype=torch.uint8, device="cuda")
    p.workspace, p.workspace_bytes = ws.data_ptr(), nb
    c = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def outputs():
        return (torch.full_like(q, float("nan")), torch.full_like(k, float("nan")),
                torch.full_like(v, float("nan")),
                torch.full((B, Hq, S), float("nan"), dtype=torch.float32, device="cuda"))

    full = outputs()
    assert lib.shaobo_fa3_bwd_v2(c(do), c(q), c(k), c(v), c(out), c(lse), *map(c, full),
                                 ctypes.byref(p)) == F.SUCCESS
    staged = outputs()
    args = [c(do), c(q), c(k), c(v), c(out), c(lse), *map(c, staged), ctypes.byref(p), None]
    assert lib.shaobo_fa3_ext_bwd_v2_stages(*args, 1) == F.SUCCESS
    assert torch.equal(staged[3], full[3])  # delta from the preprocess alone
    assert all(torch.isnan(t).all() for t in staged[:3])  # no gradient written yet
    for rep in range(3):
        for t in staged[:3]:
            t.fill_(float("nan"))
        assert lib.shaobo_fa3_ext_bwd_v2_stages(*args, 2) == F.SUCCESS
        for name, a, b in zip(("dq", "dk", "dv"), staged[:3], full[:3]):
            assert torch.equal(a, b), f"{name} differs on main-kernel-only launch {rep}"
    assert lib.shaobo_fa3_ext_bwd_v2_stages(*args, 3) == F.SUCCESS
    assert all(torch.equal(a, b) for a, b in zip(staged, full))
