"""Pins the CPU oracle (oracle/fa3_bwd_oracle.cpp) before it is trusted.

Each check is independent of the oracle's own formulas, chosen so a plausible
slip (dropped scale, wrong mask side, transposed operand, GQA head mapping,
fp16 rounding) fails at least one of them:
  * fp64 torch autograd of L = sum(dO * softmax(scale * QK^T + mask) V);
  * fp64 central finite differences of the same L (no autograd at all);
  * closed forms: S = 1 causal gives dV = dO and dQ = dK = 0; Q = 0 gives a
    uniform P (non-causal) whose dV is the mean of dO;
  * invariants: sum_j dV_j = sum_i dO_i; sum_j dK_j ~ 0;
  * GQA equals MHA with K/V replicated per group and dK/dV summed;
  * LSE equals logsumexp(scale * QK^T) in fp64;
  * fp16 conversion equals numpy's on every bit pattern.
The reference keeps no golden vectors in its tree (its cache lives outside
git, reference .gitignore:24-26), so these are the pins.
"""
import math

import numpy as np
import pytest

import fa3_oracle as O

torch = pytest.importorskip("torch")


def torch_reference(g):
    """fp64 autograd of L = sum(dO * O) with O = softmax(scale*QK^T + mask) V."""
    q, k, v, do = (torch.tensor(O.to_f32(g[n]).astype(np.float64), requires_grad=(n != "dout"))
                   for n in ("q", "k", "v", "dout"))
    B, Hq, S, D = q.shape
    G = Hq // k.shape[1]
    kk = k.repeat_interleave(G, dim=1)
    vv = v.repeat_interleave(G, dim=1)
    s = torch.matmul(q, kk.transpose(-1, -2).contiguous()) * g["scale"]
    if g["causal"]:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.matmul(torch.softmax(s, -1), vv)
    (o * do).sum().backward()
    return {"lse": lse.detach().numpy(), "out": o.detach().numpy(), "dq": q.grad.numpy(),
            "dk": k.grad.numpy(), "dv": v.grad.numpy()}


def rel(a, e):
    return float(np.abs(np.asarray(a, np.float64) - e).max() / max(1e-30, np.abs(e).max()))


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [
    (1, 1, 1, 16, 16, True), (1, 2, 1, 32, 16, False), (2, 4, 2, 64, 32, True),
    (1, 1, 1, 128, 128, True), (1, 2, 2, 128, 64, False)])
def test_oracle_matches_fp64_autograd(B, Hq, Hkv, S, D, causal):
    g = O.golden(B, Hq, Hkv, S, D, causal)
    t = torch_reference(g)
    assert rel(g["lse"], t["lse"]) < 1e-6
    # O is rounded to fp16 by the golden; everything downstream of delta
    # inherits that 2^-11 relative rounding, hence the 2e-3 bound on dQ/dK.
    assert rel(g["out"].astype(np.float32), t["out"]) < 1e-3
    assert rel(g["dv"], t["dv"]) < 1e-5
    assert rel(g["dq"], t["dq"]) < 2e-3
    assert rel(g["dk"], t["dk"]) < 2e-3


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [(1, 2, 1, 32, 16, True), (1, 2, 2, 128, 64, False),
                                                 (1, 1, 1, 128, 128, True)])
def test_oracle_bf16_matches_fp64_autograd(B, Hq, Hkv, S, D, causal):
    """bf16 tensors: same formulas, bf16 rounding of the inputs (taken as
    exact here) and of O, whose 2^-9 relative error now dominates dQ / dK."""
    g = O.golden(B, Hq, Hkv, S, D, causal, dtype="bf16")
    assert g["q"].dtype == np.uint16 and g["out"].dtype == np.uint16
    t = torch_reference(g)
    assert rel(g["lse"], t["lse"]) < 1e-6
    assert rel(O.to_f32(g["out"]), t["out"]) < 8e-3
    assert rel(g["dv"], t["dv"]) < 1e-5
    assert rel(g["dq"], t["dq"]) < 2e-2
    assert rel(g["dk"], t["dk"]) < 2e-2


def test_bf16_conversion_against_torch():
    """bf16 <-> fp32 of the oracle against torch's conversions: every bf16
    value, midpoints between neighbours (ties to even), random floats,
    infinities and NaN."""
    bits = np.arange(65536, dtype=np.uint16)
    f = np.empty(65536, np.float32)
    O.lib().fa3o_bf16_to_f32(bits, f, bits.size)
    ref = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    finite = np.unique(ref[np.isfinite(ref)])
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    samples = np.concatenate([finite, mids, rng.standard_normal(100000).astype(np.float32) * 1e3,
                              np.array([np.inf, -np.inf, 3.4e38, -1e-40, 1e-45], np.float32)])
    out = np.empty(samples.size, np.uint16)
    O.lib().fa3o_f32_to_bf16(np.ascontiguousarray(samples), out, samples.size)
    want = torch.from_numpy(samples).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(out, want)
    nan = np.array([np.nan], np.float32)
    O.lib().fa3o_f32_to_bf16(nan, out[:1], 1)
    assert np.isnan(O.bf16_to_f32(out[:1]))[0]


def test_oracle_matches_finite_differences():
    """Central differences of L in fp64 numpy, no autograd."""
    B, Hq, Hkv, S, D = 1, 2, 1, 6, 4
    g = O.golden(B, Hq, Hkv, S, D, True, scale=0.7)
    q, k, v, do = (g[n].astype(np.float64) for n in ("q", "k", "v", "dout"))

    def loss(q, k, v):
        total = 0.0
        for h in range(Hq):
            s = q[0, h] @ k[0, h // 2].T * 0.7
            s[np.triu_indices(S, 1)] = -np.inf
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            total += float((do[0, h] * (p @ v[0, h // 2])).sum())
        return total

    eps = 1e-6
    for name, arr, grad in (("q", q, g["dq"]), ("k", k, g["dk"]), ("v", v, g["dv"])):
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            plus, minus = arr.copy(), arr.copy()
            plus[idx] += eps
            minus[idx] -= eps
            args = {"q": q, "k": k, "v": v}
            args[name] = plus
            lp = loss(**args)
            args[name] = minus
            num[idx] = (lp - loss(**args)) / (2 * eps)
        assert rel(grad, num) < 3e-3, name


def test_single_key_causal_closed_form():
    """S = 1: P = [[1]], O = V exactly, so dV = dO and dS = dO.V - dO.O = 0,
    i.e. dQ = dK = 0 up to the two fp32 summation orders (|dO.V| ~ 10)."""
    g = O.golden(1, 2, 2, 1, 64, True)
    np.testing.assert_array_equal(g["dv"], g["dout"].astype(np.float32))
    assert np.abs(g["dq"]).max() < 1e-5 and np.abs(g["dk"]).max() < 1e-5


def test_zero_query_gives_uniform_attention():
    """Q = 0 (non-causal): P is uniform 1/S, so dV_j = mean_i dO_i."""
    B, H, S, D = 1, 1, 32, 16
    x = O.make_inputs(B, H, H, S, D)
    x["q"][:] = 0
    out, smax, ssum, lse = O.forward(x["q"], x["k"], x["v"], False, 0.25)
    np.testing.assert_allclose(lse, math.log(S), rtol=1e-6)
    _, dq, dk, dv = O.backward(x["q"], x["k"], x["v"], out, x["dout"], smax, ssum, False, 0.25)
    mean_do = x["dout"].astype(np.float64).mean(axis=2, keepdims=True)
    np.testing.assert_allclose(dv, np.broadcast_to(mean_do, dv.shape), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("causal", [True, False])
def test_sum_invariants(causal):
    g = O.golden(1, 2, 2, 256, 128, causal)
    sum_dv = g["dv"].astype(np.float64).sum(axis=2)
    sum_do = g["dout"].astype(np.float64).sum(axis=2)
    np.testing.assert_allclose(sum_dv, sum_do, rtol=1e-4, atol=1e-3)
    # sum_j dK_j = sum_i (sum_j dS_ij) q_i, and sum_j dS_ij = scale*(dO.O - delta) = 0
    # up to the fp16 rounding of O used in delta.
    sum_dk = np.abs(g["dk"].astype(np.float64).sum(axis=2)).max()
    assert sum_dk < 1e-2 * np.abs(g["dk"]).max() * 16


def test_gqa_equals_replicated_mha():
    B, Hq, Hkv, S, D = 1, 4, 2, 64, 32
    g = O.golden(B, Hq, Hkv, S, D, True)
    G = Hq // Hkv
    k_rep = np.repeat(g["k"], G, axis=1)
    v_rep = np.repeat(g["v"], G, axis=1)
    out, smax, ssum, lse = O.forward(g["q"], k_rep, v_rep, True, g["scale"])
    np.testing.assert_array_equal(out, g["out"])
    _, dq, dk, dv = O.backward(g["q"], k_rep, v_rep, out, g["dout"], smax, ssum, True, g["scale"])
    np.testing.assert_allclose(dq, g["dq"], rtol=0, atol=0)
    np.testing.assert_allclose(dk.reshape(B, Hkv, G, S, D).sum(2), g["dk"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dv.reshape(B, Hkv, G, S, D).sum(2), g["dv"], rtol=1e-5, atol=1e-6)


def test_subset_matches_full():
    """Computing only some (batch, kv-head) groups gives the same rows."""
    full = O.golden(2, 4, 2, 128, 64, True)
    part = O.golden(2, 4, 2, 128, 64, True, bkv=(1, 3))
    # kv groups 1..2 = (b0, hkv1), (b1, hkv0) -> q heads (b0: 2,3), (b1: 0,1)
    np.testing.assert_array_equal(part["dq"][0, 2:], full["dq"][0, 2:])
    np.testing.assert_array_equal(part["dq"][1, :2], full["dq"][1, :2])
    np.testing.assert_array_equal(part["dk"][0, 1], full["dk"][0, 1])
    np.testing.assert_array_equal(part["dv"][1, 0], full["dv"][1, 0])


def test_fp16_conversion_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    f = np.empty(65536, np.float32)
    O.lib().fa3o_f16_to_f32(bits, f, bits.size)
    ref = bits.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    # float -> half: every half value, midpoints between neighbours (ties to
    # even), and random floats, against numpy's rounding.
    finite = ref[np.isfinite(ref)]
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(0)
    samples = np.concatenate([finite, mids, rng.standard_normal(100000).astype(np.float32) * 300,
                              np.array([65504, 65519.99, 65520, 1e-8, -6e-8, 3e-8], np.float32)])
    out = np.empty(samples.size, np.uint16)
    O.lib().fa3o_f32_to_f16(np.ascontiguousarray(samples), out, samples.size)
    want = samples.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(out, want)


def test_randn_inputs_are_standard_normal():
    x = O.randn_f16((1 << 18,), 1234).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    np.testing.assert_array_equal(O.randn_f16((100,), 7), O.randn_f16((100,), 7))


def test_reference_pattern_inputs():
    """generate_full_bwd_golden.py:135-140 restated; checked against values
    worked by hand from the formula for the first elements of Q."""
    q = O.pattern_f16((8,), 3, 29, 0.009).astype(np.float64)
    # idx*3+7 mod 29 - 14: idx0 -> 7-14=-7, idx1 -> 10-14=-4, idx2 -> -1, idx3 -> 2 ...
    want = np.array([-7, -4, -1, 2, 5, 8, 11, 14], np.float64) * 0.009
    np.testing.assert_allclose(q, want.astype(np.float32).astype(np.float16), rtol=0, atol=0)


def test_metrics_definitions():
    m = O.metrics(np.array([1.0, 2.0, np.nan]), np.array([1.0, 1.0, 1.0]))
    assert m["nonfinite"] == 1 and m["max_abs"] == 1.0
    assert abs(m["rmse"] - math.sqrt(1 / 3)) < 1e-9  # reference divides by the full count
    assert abs(m["rel_l2"] - math.sqrt(1 / 2)) < 1e-9
