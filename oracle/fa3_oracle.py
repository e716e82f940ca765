"""numpy/ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/lib/libfa3_oracle.so (a restatement of the reference's fp32 CPU
golden, reference scripts/generate_full_bwd_golden.py:143-219; see
fa3_bwd_oracle.cpp for the formula-by-formula citations).  Used by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; never
by the shipped library.

Also holds the reference's five comparison metrics and gates
(reference src/full_bwd_correctness.cpp:104-137, 471-500).
"""
import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "lib", "libfa3_oracle.so")
REF_API_LIB = os.path.join(_HERE, "_ref", "libref_api.so")

# Per-tensor seeds of the build's N(0,1) inputs.
SEEDS = {"q": 0x51, "k": 0x4B, "v": 0x56, "dout": 0xD0}
# Reference deterministic pattern (mul, mod, scale): generate_full_bwd_golden.py:148-151.
PATTERN = {"q": (3, 29, 0.009), "k": (5, 31, 0.008), "v": (7, 37, 0.007), "dout": (11, 41, 0.006)}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"oracle not built: make -C {_HERE}")
        L = ctypes.CDLL(ORACLE_LIB)
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        i = ctypes.c_int
        L.fa3o_randn_f16.argtypes = [u16p, ctypes.c_size_t, ctypes.c_uint64]
        L.fa3o_pattern_f16.argtypes = [u16p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_float]
        L.fa3o_f16_to_f32.argtypes = [u16p, f32p, ctypes.c_size_t]
        L.fa3o_f32_to_f16.argtypes = [f32p, u16p, ctypes.c_size_t]
        L.fa3o_forward.argtypes = [u16p, u16p, u16p, i, i, i, i, i, i, ctypes.c_float, i, i,
                                   u16p, f32p, f32p, f32p, i]
        L.fa3o_backward.argtypes = [u16p, u16p, u16p, u16p, u16p, f32p, f32p, i, i, i, i, i, i,
                                    ctypes.c_float, i, i, f32p, f32p, f32p, f32p, i]
        L.fa3o_forward_fmt.argtypes = L.fa3o_forward.argtypes + [i]
        L.fa3o_backward_fmt.argtypes = L.fa3o_backward.argtypes + [i]
        L.fa3o_randn_fmt.argtypes = [u16p, ctypes.c_size_t, ctypes.c_uint64, i]
        L.fa3o_pattern_fmt.argtypes = [u16p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_float, i]
        L.fa3o_bf16_to_f32.argtypes = [u16p, f32p, ctypes.c_size_t]
        L.fa3o_f32_to_bf16.argtypes = [f32p, u16p, ctypes.c_size_t]
        _lib = L
    return _lib


def default_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def randn_f16(shape, seed):
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().fa3o_randn_f16(out, out.size, seed)
    return out.view(np.float16).reshape(shape)


def pattern_f16(shape, mul, mod, scale):
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().fa3o_pattern_f16(out, out.size, mul, mod, scale)
    return out.view(np.float16).reshape(shape)


# bf16 tensors travel as numpy uint16 arrays of their bit patterns (numpy has
# no bfloat16); fp16 tensors as float16.
def randn_bf16(shape, seed):
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().fa3o_randn_fmt(out, out.size, seed, 1)
    return out.reshape(shape)


def pattern_bf16(shape, mul, mod, scale):
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().fa3o_pattern_fmt(out, out.size, mul, mod, scale, 1)
    return out.reshape(shape)


def bf16_to_f32(bits):
    return (np.ascontiguousarray(bits).astype(np.uint32) << 16).view(np.float32)


def to_f32(a):
    """fp32 values of an fp16 array or of bf16 bits (uint16)."""
    return bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


def make_inputs(B, Hq, Hkv, S, D, kind="randn", seed_offset=0, dtype="fp16"):
    """Q, K, V, dO (BHSD): fp16 arrays, or bf16 bits as uint16 when dtype='bf16'."""
    qs, ks = (B, Hq, S, D), (B, Hkv, S, D)
    shapes = {"q": qs, "k": ks, "v": ks, "dout": qs}
    bf = dtype == "bf16"
    if kind == "randn":
        gen = randn_bf16 if bf else randn_f16
        return {n: gen(shapes[n], SEEDS[n] + seed_offset) for n in shapes}
    if kind == "pattern":
        gen = pattern_bf16 if bf else pattern_f16
        return {n: gen(shapes[n], *PATTERN[n]) for n in shapes}
    raise ValueError(kind)


def _u16(a):
    return np.ascontiguousarray(a).view(np.uint16)


def forward(q, k, v, causal, scale, bkv=None, threads=None):
    """fp32 CPU forward: returns O (the inputs' 16-bit type), scores_max,
    scores_sum, lse (natural)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    b0, b1 = (0, B * Hkv) if bkv is None else bkv
    fmt = 1 if q.dtype == np.uint16 else 0
    out = np.zeros((B, Hq, S, D), dtype=np.uint16)
    smax = np.zeros((B, Hq, S), np.float32)
    ssum = np.zeros((B, Hq, S), np.float32)
    lse = np.zeros((B, Hq, S), np.float32)
    lib().fa3o_forward_fmt(_u16(q), _u16(k), _u16(v), B, Hq, Hkv, S, D, int(causal), scale, b0,
                           b1, out, smax, ssum, lse, threads or default_threads(), fmt)
    return (out if fmt else out.view(np.float16)), smax, ssum, lse


def backward(q, k, v, out, dout, smax, ssum, causal, scale, bkv=None, threads=None):
    """fp32 CPU backward: returns delta, dq, dk, dv (fp32)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    b0, b1 = (0, B * Hkv) if bkv is None else bkv
    delta = np.zeros((B, Hq, S), np.float32)
    dq = np.zeros((B, Hq, S, D), np.float32)
    dk = np.zeros((B, Hkv, S, D), np.float32)
    dv = np.zeros((B, Hkv, S, D), np.float32)
    fmt = 1 if q.dtype == np.uint16 else 0
    lib().fa3o_backward_fmt(_u16(q), _u16(k), _u16(v), _u16(out), _u16(dout), smax, ssum, B, Hq,
                            Hkv, S, D, int(causal), scale, b0, b1, delta, dq, dk, dv,
                            threads or default_threads(), fmt)
    return delta, dq, dk, dv


def golden(B, Hq, Hkv, S, D, causal, scale=None, kind="randn", bkv=None, threads=None,
           seed_offset=0, dtype="fp16"):
    """Inputs + forward + backward in one call (dict of numpy arrays)."""
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    x = make_inputs(B, Hq, Hkv, S, D, kind, seed_offset, dtype)
    out, smax, ssum, lse = forward(x["q"], x["k"], x["v"], causal, scale, bkv, threads)
    delta, dq, dk, dv = backward(x["q"], x["k"], x["v"], out, x["dout"], smax, ssum, causal,
                                 scale, bkv, threads)
    x.update(out=out, scores_max=smax, scores_sum=ssum, lse=lse, delta=delta, dq=dq, dk=dk,
             dv=dv, scale=scale, causal=causal, dtype=dtype)
    return x


def metrics(actual, expected):
    """The reference's five metrics + non-finite count
    (reference src/full_bwd_correctness.cpp:104-137), plus max|err|/max|ref|."""
    a = np.asarray(actual, np.float32).ravel()
    e = np.asarray(expected, np.float32).ravel()
    fin = np.isfinite(a) & np.isfinite(e)
    nonfinite = int((~fin).sum())
    a64, e64 = a[fin].astype(np.float64), e[fin].astype(np.float64)
    d = np.abs(a[fin] - e[fin]).astype(np.float64)
    n = max(1.0, float(a.size))
    diff_sq = float((d * d).sum())
    exp_sq = float((e64 * e64).sum())
    act_sq = float((a64 * a64).sum())
    dot = float((a64 * e64).sum())
    norm = math.sqrt(act_sq * exp_sq)
    max_ref = float(np.abs(e64).max()) if e64.size else 0.0
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "mean_abs": float(d.sum() / n),
        "rmse": math.sqrt(diff_sq / n),
        "rel_l2": math.sqrt(diff_sq / max(1e-30, exp_sq)),
        "cosine_error": (1.0 - dot / norm) if norm > 1e-30 else 0.0,
        "nonfinite": nonfinite,
        "max_rel": (float(d.max()) / max_ref) if (d.size and max_ref > 0) else 0.0,
    }


# max|err|/max|ref| <= 1e-2 for dQ/dK/dV, delta within 1e-4 relative.
GRAD_MAX_REL = 1e-2
DELTA_REL = 1e-4


def gates(name, m):
    """(north_star_ok, reference_gate_ok).

    North star: max|err|/max|ref| <= 1e-2 for dQ/dK/dV; delta within 1e-4
    relative (rel_l2 and max|err|/max|ref|).  Reference gates
    (src/full_bwd_correctness.cpp:471-500): delta max_abs <= 5e-5 and
    rel_l2 <= 1e-4; dK/dV max_abs <= 3e-2 and rel_l2 <= 3e-2; dQ max_abs <=
    3e-2 and (rel_l2 <= 3e-2 or rmse <= 5e-5).  The reference's absolute
    bounds were set for its small-magnitude pattern inputs."""
    if m["nonfinite"]:
        return False, False
    if name == "delta":
        ok = m["rel_l2"] <= DELTA_REL and m["max_rel"] <= DELTA_REL
        ref_ok = m["max_abs"] <= 5e-5 and m["rel_l2"] <= 1e-4
    else:
        ok = m["max_rel"] <= GRAD_MAX_REL
        if name == "dq":
            ref_ok = m["max_abs"] <= 3e-2 and (m["rel_l2"] <= 3e-2 or m["rmse"] <= 5e-5)
        else:
            ref_ok = m["max_abs"] <= 3e-2 and m["rel_l2"] <= 3e-2
    return ok, ref_ok
