"""PyTorch custom op on the GPU: same result as shaobo_fa3_bwd_v2, correct on
a non-default stream and inside a captured CUDA (HIP) graph, and an autograd
round trip against fp32 torch autograd."""
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
    import shaobo_fa3_torch  # noqa: F401


def inputs(g):
    return tuple(dev(g[n], torch) for n in ("dout", "q", "k", "v", "out", "lse"))


def op(args, causal, scale):
    return torch.ops.shaobo_fa3.flash_attn_backward(*args, causal, scale, False)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [(1, 2, 2, 1024, 128, True),   # split plan
                                                 (1, 4, 2, 256, 128, True),
                                                 (1, 2, 1, 384, 64, False)])
def test_op_matches_v2_and_oracle(B, Hq, Hkv, S, D, causal):
    log(f"[case] torch op B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} causal={causal}")
    g = O.golden(B, Hq, Hkv, S, D, causal)
    args = inputs(g)
    dq, dk, dv, delta = op(args, causal, g["scale"])
    torch.cuda.synchronize()
    res = {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
           "dv": dv.float().cpu().numpy(), "delta": delta.cpu().numpy()}
    check(res, g)
    dout, q, k, v, out, lse = args
    r2 = F.bwd_v2(dout, q, k, v, out, lse, causal=causal, softmax_scale=g["scale"], sync=True)
    for a, b in zip((dq, dk, dv), r2):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_op_on_side_stream():
    """Inputs produced and the op run on a non-default stream: results are
    ordered on that stream (the default stream is kept busy meanwhile)."""
    log("[case] torch op on a side stream")
    g = O.golden(1, 2, 2, 512, 128, True)
    ref = op(inputs(g), True, g["scale"])
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    busy = torch.randn(4096, 4096, device="cuda")
    with torch.cuda.stream(s):
        args = tuple(t.clone() for t in inputs(g))
        for _ in range(3):
            busy = busy @ busy.t().contiguous() * 1e-3  # work on the side stream first
        got = op(args, True, g["scale"])
    s.synchronize()
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_op_in_captured_graph():
    """Capture the op in a graph, replay it several times with eager work and
    synchronisations in between, and compare every replay with the eager
    result (the library issues kernel launches only: no memsets)."""
    log("[case] torch op in a captured graph")
    g = O.golden(1, 2, 2, 1024, 128, True)
    static = inputs(g)
    eager = [t.cpu() for t in op(static, True, g["scale"])]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the capture stream
        op(static, True, g["scale"])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = op(static, True, g["scale"])
    for i in range(4):
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for a, b in zip(outs, eager):
            np.testing.assert_array_equal(a.cpu().numpy(), b.numpy(), err_msg=f"replay {i}")


def test_op_bf16():
    log("[case] torch op bf16")
    g = O.golden(1, 4, 2, 512, 128, True, dtype="bf16")
    dq, dk, dv, delta = op(inputs(g), True, g["scale"])
    torch.cuda.synchronize()
    assert dq.dtype == torch.bfloat16
    check({"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
           "dv": dv.float().cpu().numpy(), "delta": delta.cpu().numpy()}, g)


def test_autograd_attention():
    """attention(): torch forward, library backward; gradients against fp32
    torch autograd of the same forward."""
    import shaobo_fa3_torch as FT
    log("[case] autograd attention")
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 4, 512, 128, device="cuda").half().requires_grad_() for _ in range(3))
    k2 = torch.randn(1, 2, 512, 128, device="cuda").half().requires_grad_()
    v2 = torch.randn(1, 2, 512, 128, device="cuda").half().requires_grad_()
    for kk, vv in ((k, v), (k2, v2)):
        out = FT.attention(q, kk, vv, causal=True)
        dout = torch.randn_like(out)
        out.backward(dout)
        qf, kf, vf = (x.detach().float().requires_grad_() for x in (q, kk, vv))
        G = q.shape[1] // kk.shape[1]
        s = torch.matmul(qf, kf.repeat_interleave(G, 1).transpose(-1, -2).contiguous()) / 128 ** 0.5
        s = s.masked_fill(torch.triu(torch.ones(512, 512, dtype=torch.bool, device="cuda"), 1),
                          float("-inf"))
        ref = torch.matmul(torch.softmax(s, -1), vf.repeat_interleave(G, 1))
        ref.backward(dout.float())
        for got, want in ((q.grad, qf.grad), (kk.grad, kf.grad), (vv.grad, vf.grad)):
            err = (got.float() - want).abs().max() / want.abs().max()
            assert err < 1e-2, float(err)
        q.grad = None


def test_op_split_errors_reported_at_check():
    """The op never synchronises, so a split wait that gives up cannot fail
    the call; shaobo_fa3_torch.check_split_errors() -- the op's
    synchronisation point -- raises for it once, and passes again after a
    correct call."""
    import shaobo_fa3_torch as T
    log("[case] torch op: split give-up reported by check_split_errors")
    lib = F.load()
    g = O.golden(1, 4, 4, 2048, 128, True)  # split plan (P3: 64 split jobs per role)
    args = inputs(g)
    try:  # baseline: give-ups that earlier tests forced on purpose are consumed
        T.check_split_errors()
    except RuntimeError:
        pass
    # a wait that finds the partial sums already published carries on:
    # calls are repeated until one gives up
    raised = False
    lib.shaobo_fa3_ext_set_split_spin_limit(0)
    try:
        for _ in range(40):
            op(args, True, g["scale"])
            try:
                T.check_split_errors()
            except RuntimeError as e:
                assert "split wait" in str(e)
                raised = True
                break
    finally:
        lib.shaobo_fa3_ext_set_split_spin_limit(1 << 24)
    assert raised, "no split wait gave up in 40 calls with spin limit 0"
    dq, dk, dv, delta = op(args, True, g["scale"])
    T.check_split_errors()
    res = {"dq": dq.float().cpu().numpy(), "dk": dk.float().cpu().numpy(),
           "dv": dv.float().cpu().numpy(), "delta": delta.cpu().numpy()}
    check(res, g)
