"""C ABI contract of libshaobo_fa3_bwd.so (host only, no GPU needed).

* The library loads and exports every function declared in include/*.h.
* ShaoboFa3Params / ShaoboFa3BwdCapabilities keep the reference byte layout
  (reference include/shaobo_fa3_api.h:53-109).
* The capability payload and the twelve validation cases of the reference's
  own contract test (reference tests/fused_bwd_api_contract.cpp:34-118).
* Differential check of shaobo_fa3_bwd_v2_validate against the reference's
  own validation code compiled from its sources (oracle/_ref/libref_api.so,
  reference src/shaobo_fa3_bwd_api.cpp:53-120) over thousands of random
  parameter structs.  The only allowed differences are this build's
  extensions: head_dim 64, BF16 and BSHD.
* Workspace sizing and the error paths of the launch entries that return
  before any HIP call.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import shaobo_fa3 as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_api.so")


@pytest.fixture(scope="module")
def lib():
    return F.load()


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(shaobo_fa3_\w+)\s*\(", text))
    return names


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert "shaobo_fa3_bwd_v2" in names and len(names) >= 9
    for n in sorted(names):
        assert hasattr(lib, n), n
    assert set(F.EXPORTS) <= names


def test_struct_layout():
    assert ctypes.sizeof(F.Params) == 296
    assert ctypes.sizeof(F.Capabilities) == 32
    offsets = {"struct_size": 0, "batch": 4, "causal": 32, "softmax_scale": 44, "dtype": 52,
               "sync_after_launch": 76, "cu_seqlens_q": 80, "cu_seqlens_k": 88,
               "max_seqlen_q": 96, "max_seqlen_k": 100, "workspace": 104,
               "workspace_bytes": 112, "reserved_i32": 120, "reserved_ptr": 184,
               "seqused_q": 248, "seqused_k": 256, "total_q": 264, "total_k": 272,
               "softcap": 280, "deterministic": 284, "sm_margin": 288,
               "softmax_scale_is_set": 292}
    for name, off in offsets.items():
        assert getattr(F.Params, name).offset == off, name


def test_params_init(lib):
    p = F.Params()
    ctypes.memset(ctypes.byref(p), 0x5A, ctypes.sizeof(p))
    lib.shaobo_fa3_params_init(ctypes.byref(p))
    assert p.struct_size == 296 and p.window_left == -1 and p.window_right == -1
    assert p.dtype == F.DTYPE_FP16 and p.layout == F.LAYOUT_BHSD
    assert p.softmax_aux_mode == F.AUX_LSE
    assert p.batch == 0 and p.workspace is None and p.softmax_scale_is_set == 0
    lib.shaobo_fa3_params_init(None)  # tolerated


def supported(lib):
    """reference tests/fused_bwd_api_contract.cpp:16-30"""
    p = F.make_params(lib, batch=1, seqlen=1024, heads_q=4, heads_kv=2, head_dim=128,
                      causal=True, softmax_scale=0.125)
    return p


def test_capabilities(lib):
    caps = F.Capabilities()
    assert lib.shaobo_fa3_bwd_get_capabilities(ctypes.byref(caps)) == F.INVALID_VALUE  # struct_size 0
    assert lib.shaobo_fa3_bwd_get_capabilities(None) == F.INVALID_VALUE
    caps.struct_size = ctypes.sizeof(caps)
    assert lib.shaobo_fa3_bwd_get_capabilities(ctypes.byref(caps)) == F.SUCCESS
    required = 0
    # the reference's bits, plus this build's BF16 and BSHD extensions
    for n in ("FIXED_LENGTH", "FP16", "CAUSAL", "GQA", "DETERMINISTIC", "SOFTMAX_LSE", "BHSD",
              "FULL_ATTENTION", "BF16", "BSHD"):
        required |= F.FEATURES[n]
    assert caps.api_version == F.API_VERSION
    assert caps.feature_mask & required == required
    for n in ("VARLEN", "LOCAL_WINDOW", "SOFTCAP"):
        assert not caps.feature_mask & F.FEATURES[n]
    assert caps.max_head_dim == 128 and caps.sequence_alignment == 128
    assert caps.min_head_dim == 64 and caps.head_dim_alignment == 64


CONTRACT_CASES = [
    # (name, mutation, expected)  reference tests/fused_bwd_api_contract.cpp:57-115
    ("fixed_gqa_causal", {}, F.SUCCESS),
    ("deterministic", {"deterministic": 1}, F.SUCCESS),
    ("full_attention", {"causal": 0}, F.SUCCESS),
    ("default_scale", {"softmax_scale_is_set": 0, "softmax_scale": 0.0}, F.SUCCESS),
    ("local_window", {"window_left": 128}, F.UNSUPPORTED),
    ("softcap", {"softcap": 1.0}, F.UNSUPPORTED),
    ("dropout", {"dropout_p": 0.1}, F.UNSUPPORTED),
    # the reference rejects these two (UNSUPPORTED); this build supports them
    ("bf16", {"dtype": F.DTYPE_BF16}, F.SUCCESS),
    ("bshd", {"layout": F.LAYOUT_BSHD}, F.SUCCESS),
    ("fp8", {"dtype": F.DTYPE_FP8}, F.UNSUPPORTED),
    ("layout_3", {"layout": 3}, F.UNSUPPORTED),
    ("varlen", {"cu_seqlens_q": "ptr"}, F.UNSUPPORTED),
    ("sm_margin", {"sm_margin": 1}, F.UNSUPPORTED),
    ("negative_scale", {"softmax_scale": -1.0}, F.INVALID_VALUE),
    ("old_struct", {"struct_size": 0}, F.INVALID_VALUE),
    # further cases of the same validation order (reference src/shaobo_fa3_bwd_api.cpp:70-118)
    ("zero_batch", {"batch": 0}, F.INVALID_VALUE),
    ("heads_not_divisible", {"num_heads_kv": 3}, F.INVALID_VALUE),
    ("causal_not_flag", {"causal": 2}, F.INVALID_VALUE),
    ("nan_scale", {"softmax_scale": float("nan")}, F.INVALID_VALUE),
    ("dropout_one", {"dropout_p": 1.0}, F.INVALID_VALUE),
    ("negative_softcap", {"softcap": -1.0}, F.INVALID_VALUE),
    ("seqlen_mismatch", {"seqlen_k": 512}, F.UNSUPPORTED),
    ("seqlen_unaligned", {"seqlen_q": 1000, "seqlen_k": 1000}, F.UNSUPPORTED),
    ("head_dim_96", {"head_dim_qk": 96, "head_dim_v": 96}, F.UNSUPPORTED),
    ("head_dim_mismatch", {"head_dim_v": 64}, F.UNSUPPORTED),
    ("max_seqlen_mismatch", {"max_seqlen_q": 512}, F.UNSUPPORTED),
    ("total_q_match", {"total_q": 1024}, F.SUCCESS),
    ("total_q_mismatch", {"total_q": 7}, F.UNSUPPORTED),
    ("window_as_long_as_seq", {"window_left": 1023, "window_right": 5000}, F.SUCCESS),
    ("window_right_noncausal", {"causal": 0, "window_right": 3}, F.UNSUPPORTED),
    ("head_dim_64", {"head_dim_qk": 64, "head_dim_v": 64}, F.SUCCESS),  # build extension
]


def apply(p, mutation, keep=None):
    for k, v in mutation.items():
        if v == "ptr":
            keep = (ctypes.c_int32 * 2)(0, 1024)
            v = ctypes.cast(keep, ctypes.c_void_p).value
        setattr(p, k, v)
    return keep


@pytest.mark.parametrize("name,mutation,expected", CONTRACT_CASES,
                         ids=[c[0] for c in CONTRACT_CASES])
def test_validation_contract(lib, name, mutation, expected):
    p = supported(lib)
    keep = apply(p, mutation)  # noqa: F841  (keeps the varlen array alive)
    assert lib.shaobo_fa3_bwd_v2_validate(ctypes.byref(p)) == expected
    ws = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    assert (ws > 0) == (expected == F.SUCCESS)


def test_validate_null(lib):
    assert lib.shaobo_fa3_bwd_v2_validate(None) == F.INVALID_VALUE
    assert lib.shaobo_fa3_bwd_v2_workspace_bytes(None) == 0


def test_status_strings(lib):
    for code, name in F.STATUS.items():
        assert lib.shaobo_fa3_status_string(code).decode() == name
    assert lib.shaobo_fa3_status_string(99).decode() == "unknown"


ERR_REGION = 256  # the error word's 256-byte region opens every workspace


def row_arrays_bytes(rows):
    """lse2 and -delta rows (fp32, each region 256-byte aligned) that the
    preprocess pass writes for the main kernel."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    return 2 * align(rows * 4)


QUEUE_BYTES = 8 * 128  # job-queue counters of the persistent main kernel, one 128-byte line each


def plain_bytes(batch, heads_q, seqlen):
    """Workspace without the split plan: the error word's region, the row
    arrays and the job-queue counters."""
    return ERR_REGION + row_arrays_bytes(batch * heads_q * seqlen) + QUEUE_BYTES


def split_plan_bytes(batch, heads, seqlen, head_dim):
    """Workspace of the split plan (causal, one query head per KV head, at
    most 256 jobs): the error word's region, lse2 and -delta rows, the
    job-queue counters, two
    64-bit synchronisation words per split job of each role (B*H*QT/2 jobs per
    role), then the fp32 partial sums of one piece per split job -- dK/dV:
    4 waves x 2 matrices x D/64 tiles x 4 KiB, dQ: 4 waves x D/64 tiles x
    4 KiB -- each region 256-byte aligned."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    rows = batch * heads * seqlen
    jobs = batch * heads * (seqlen // 64 // 2)
    off = ERR_REGION + row_arrays_bytes(rows) + QUEUE_BYTES
    off = align(off + jobs * 4 * 8)
    off = align(off + jobs * 4 * 2 * (head_dim // 64) * 4096)
    return align(off + jobs * 4 * (head_dim // 64) * 4096)


def test_workspace_sizes(lib):
    """v2's workspace: the error word's region, the row arrays and, where the
    split plan applies, its synchronisation words and partial sums; the
    reference contract test requires a non-zero size for a supported shape
    (fused_bwd_api_contract.cpp:60-63)."""
    def ws(**kw):
        p = F.make_params(lib, **kw)
        return lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    # causal MHA with few jobs: split plan
    assert ws(batch=1, seqlen=2048, heads_q=4) == split_plan_bytes(1, 4, 2048, 128)
    assert ws(batch=1, seqlen=2048, heads_q=4, deterministic=True) == split_plan_bytes(1, 4, 2048, 128)
    assert ws(batch=1, seqlen=512, heads_q=2, head_dim=64) == split_plan_bytes(1, 2, 512, 64)
    # no split: non-causal, GQA, too many jobs (512 here), or fewer than four query tiles
    assert ws(batch=1, seqlen=2048, heads_q=8) == plain_bytes(1, 8, 2048)
    assert ws(batch=1, seqlen=1024, heads_q=8) == split_plan_bytes(1, 8, 1024, 128)
    assert ws(batch=2, seqlen=8192, heads_q=16, head_dim=64, causal=False) == plain_bytes(2, 16, 8192)
    assert ws(batch=2, seqlen=4096, heads_q=32, heads_kv=8) == plain_bytes(2, 32, 4096)
    assert ws(batch=2, seqlen=4096, heads_q=4) == plain_bytes(2, 4, 4096)
    assert ws(batch=1, seqlen=128, heads_q=1) == plain_bytes(1, 1, 128)


def head_split_chunks(B, Hq, Hkv, S, causal):
    """The head-split plan's chunk count f (0: one dKV job per KV head), by
    the planner's estimate in dKV steps: a CU's share of all steps (256 CUs,
    a dQ step 0.75 of a dKV step); the merged plan takes max(share, G QT),
    f chunks of G / f heads (f <= 64) max(share, G QT / f) x (1 + 0.004 f) + 8;
    the least estimate wins if it is below 0.92 x the merged plan's."""
    qt, G = S // 64, Hq // Hkv
    steps = qt * (qt + 1) / 2 if causal else qt * qt
    share = B * Hq * steps * 1.75 / 256
    best, best_t = 0, 0.92 * max(share, G * qt)
    for f in range(2, min(G, 64) + 1):
        t = max(share, G // f * qt) * (1 + 0.004 * f) + 8
        if G % f == 0 and t < best_t:
            best, best_t = f, t
    return best


def test_head_split_workspace_sizes(lib):
    """GQA shapes whose merged dKV job (G QT steps: G query heads against one
    key tile) would set the kernel's length take the head-split plan: the
    plain workspace plus fp32 dK and dV per chunk of heads (2 B Hkv f S D x 4
    bytes).  The decision depends on the shape only."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731

    def ws(**kw):
        p = F.make_params(lib, **kw)
        return lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))

    def expect(B, Hq, Hkv, S, D, causal):
        f = head_split_chunks(B, Hq, Hkv, S, causal)
        return plain_bytes(B, Hq, S) + (align(2 * B * Hkv * f * S * D * 4) if f else 0)
    cases = [
        # B, Hq, Hkv, S, D, causal, chunks
        (1, 32, 1, 4096, 128, True, 8),   # MQA at batch 1: 2048 steps against a share of 455
        (2, 32, 1, 4096, 128, True, 4),
        (4, 32, 1, 4096, 128, True, 2),   # 2048 against 1820
        (8, 32, 1, 4096, 128, True, 0),   # 2048 against 3640
        (1, 8, 2, 4096, 128, True, 4),
        (1, 16, 2, 2048, 64, False, 4),
        (1, 4, 2, 1024, 128, True, 2),
        (2, 8, 2, 256, 128, False, 4),
        (2, 16, 4, 2048, 128, True, 0),   # 128 against 115.5: under 8 % to gain
        (2, 16, 8, 1024, 128, True, 0),
        (2, 32, 8, 4096, 128, True, 0),   # P4
        (1, 4, 2, 384, 128, True, 0),
    ]
    for B, Hq, Hkv, S, D, causal, f in cases:
        assert head_split_chunks(B, Hq, Hkv, S, causal) == f
        got = ws(batch=B, heads_q=Hq, heads_kv=Hkv, seqlen=S, head_dim=D, causal=causal)
        assert got == expect(B, Hq, Hkv, S, D, causal), (B, Hq, Hkv, S, D, causal)


def test_legacy_workspace_sizes(lib):
    """The legacy entry sizes like v2 in either aux mode."""
    def ws(mode, **kw):
        p = F.make_params(lib, **kw)
        p.softmax_aux_mode = mode
        return lib.shaobo_fa3_bwd_workspace_bytes(ctypes.byref(p))
    assert ws(F.AUX_LSE, batch=2, seqlen=4096, heads_q=4) == plain_bytes(2, 4, 4096)
    assert ws(F.AUX_SMAX_SSUM, batch=2, seqlen=4096, heads_q=4) == plain_bytes(2, 4, 4096)
    assert ws(F.AUX_SMAX_SSUM, batch=1, seqlen=2048, heads_q=4) == split_plan_bytes(1, 4, 2048, 128)
    assert ws(F.AUX_LSE, batch=1, seqlen=2048, heads_q=4) == split_plan_bytes(1, 4, 2048, 128)


def test_workspace_overflow_is_zero(lib):
    """Absurd shapes whose workspace arithmetic would overflow size_t or the
    kernel's 32-bit offsets report 0 bytes instead of a wrapped size."""
    p = F.make_params(lib, batch=1 << 30, seqlen=1 << 30, heads_q=1 << 20)
    p.softmax_aux_mode = F.AUX_SMAX_SSUM
    assert lib.shaobo_fa3_bwd_workspace_bytes(ctypes.byref(p)) == 0
    p = F.make_params(lib, batch=1 << 30, seqlen=1 << 30, heads_q=1 << 20)
    assert lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p)) == 0


def test_launch_error_paths_without_gpu(lib):
    """Validation, null tensors and short workspaces fail before any HIP call."""
    p = supported(lib)
    one = ctypes.c_void_p(16)
    args = [one] * 9 + [None]
    p.batch = 0
    assert lib.shaobo_fa3_bwd_v2(*args, ctypes.byref(p)) == F.INVALID_VALUE
    p = supported(lib)
    p.dtype = F.DTYPE_FP8
    assert lib.shaobo_fa3_bwd_v2(*args, ctypes.byref(p)) == F.UNSUPPORTED
    p = supported(lib)
    bad = list(args)
    bad[3] = None  # v
    assert lib.shaobo_fa3_bwd_v2(*bad, ctypes.byref(p)) == F.INVALID_VALUE
    p.workspace = 16
    p.workspace_bytes = 1
    assert lib.shaobo_fa3_bwd_v2(*args, ctypes.byref(p)) == F.INVALID_VALUE
    p.workspace = None
    p.workspace_bytes = 1 << 40
    assert lib.shaobo_fa3_bwd_v2(*args, ctypes.byref(p)) == F.INVALID_VALUE
    # legacy entry: SMAX_SSUM needs aux1; unknown aux mode is unsupported
    p = supported(lib)
    p.softmax_aux_mode = F.AUX_SMAX_SSUM
    assert lib.shaobo_fa3_bwd(one, one, one, one, one, one, None, one, one, one,
                              ctypes.byref(p)) == F.INVALID_VALUE
    p.softmax_aux_mode = 7
    assert lib.shaobo_fa3_bwd(*([one] * 10), ctypes.byref(p)) == F.UNSUPPORTED
    # dot_do_o component
    p = supported(lib)
    p.head_dim_qk = p.head_dim_v = 96
    assert lib.shaobo_fa3_bwd_dot_do_o(*([one] * 6), ctypes.byref(p)) == F.UNSUPPORTED
    p = supported(lib)
    assert lib.shaobo_fa3_bwd_dot_do_o(one, one, one, None, one, None,
                                       ctypes.byref(p)) == F.INVALID_VALUE
    # stage-selecting extension: a stage mask outside 1..3 is refused first,
    # then the v2 checks apply
    p = supported(lib)
    for stages in (0, 4, -1):
        assert lib.shaobo_fa3_ext_bwd_v2_stages(*args, ctypes.byref(p), None,
                                                stages) == F.INVALID_VALUE
    p.batch = 0
    assert lib.shaobo_fa3_ext_bwd_v2_stages(*args, ctypes.byref(p), None, 2) == F.INVALID_VALUE


def random_params(rng, p):
    """Random mutations drawn around the supported point, covering every
    validated field with valid, boundary and invalid values."""
    choices = {
        "batch": [1, 2, 0, -1],
        "seqlen_q": [128, 256, 1024, 1000, 0, -128],
        "seqlen_k": [128, 256, 1024, 1000, 0],
        "num_heads_q": [1, 2, 4, 8, 0, 3],
        "num_heads_kv": [1, 2, 4, 0, 3],
        "head_dim_qk": [128, 128, 64, 96, 256, 0],
        "head_dim_v": [128, 128, 64, 32],
        "causal": [0, 1, 1, 2, -1],
        "window_left": [-1, -1, 0, 5, 127, 1023, 4096],
        "window_right": [-1, -1, 0, 3, 1023, 4096],
        "softmax_scale": [0.125, 0.0, -1.0, float("inf"), float("nan"), 1e-3],
        "dropout_p": [0.0, 0.0, 0.1, 1.0, -0.1, float("nan")],
        "dtype": [0, 0, 1, 2, 7],
        "layout": [0, 0, 1, 3],
        "max_seqlen_q": [0, 0, 1024, 128, 7],
        "max_seqlen_k": [0, 0, 1024, 256],
        "total_q": [0, 0, 1024, 2048, 5],
        "total_k": [0, 0, 1024, 99],
        "softcap": [0.0, 0.0, 1.0, -1.0, float("inf")],
        "deterministic": [0, 1, 2],
        "sm_margin": [0, 0, 1],
        "softmax_scale_is_set": [0, 1, 1, 2],
        "sync_after_launch": [0, 0, 1, 5],
    }
    for name in rng.choice(list(choices), size=rng.integers(1, 5), replace=False):
        vals = choices[name]
        setattr(p, name, vals[rng.integers(len(vals))])
    if rng.random() < 0.05:
        p.struct_size = 200
    return p


@pytest.mark.skipif(not os.path.exists(REF_LIB),
                    reason="oracle/_ref/libref_api.so is built from /root/reference "
                           "(make -C oracle ref); absent where the reference is absent")
def test_validation_matches_reference_code(lib):
    ref = F.declare_abi(ctypes.CDLL(REF_LIB, mode=os.RTLD_LAZY))
    rng = np.random.default_rng(2024)
    seen = set()
    for _ in range(5000):
        p = random_params(rng, supported(lib))
        mine = lib.shaobo_fa3_bwd_v2_validate(ctypes.byref(p))
        theirs = ref.shaobo_fa3_bwd_v2_validate(ctypes.byref(p))
        seen.add(theirs)
        if mine != theirs:
            # head_dim 64, bf16 and BSHD are this build's extensions: the
            # reference rejects them as UNSUPPORTED when all else is valid.
            ext = (p.head_dim_qk == 64 and p.head_dim_v == 64) or p.dtype == F.DTYPE_BF16 \
                or p.layout == F.LAYOUT_BSHD
            assert ext and mine == F.SUCCESS and theirs == F.UNSUPPORTED, (mine, theirs)
    assert seen == {F.SUCCESS, F.INVALID_VALUE, F.UNSUPPORTED}
    # params_init agrees byte for byte
    a, b = F.Params(), F.Params()
    lib.shaobo_fa3_params_init(ctypes.byref(a))
    ref.shaobo_fa3_params_init(ctypes.byref(b))
    assert bytes(a) == bytes(b)


def component_params(lib, **kw):
    p = F.make_params(lib, **{"batch": 1, "seqlen": 256, "heads_q": 2, "head_dim": 128,
                              "causal": True, "softmax_scale": 0.125, **kw})
    p.dkv_path = F.DKV_PATH_CANONICAL
    p.dq_path = F.DQ_PATH_CANONICAL
    return p


def naive_bytes(batch, heads, seqlen):
    """Workspace of the naive path 1 (reference reference_workspace_bytes,
    src/dkv_kernel.cpp:77-86): fp32 prob and dP [rows][S], then row max,
    row sum and delta [rows]."""
    rows = batch * heads * seqlen
    return (2 * rows * seqlen + 3 * rows) * 4


def test_component_workspace_sizes(lib):
    """dkv / dq need no workspace on their canonical paths and the S^2-sized
    one on path 1 (as the reference, src/dkv_kernel.cpp:1289-1298,
    src/dq_kernel.cpp:1486-1495); fused5 needs the v2 plan, 0 for an
    unsupported shape."""
    for f, attr in (("dkv", "dkv_path"), ("dq", "dq_path")):
        fn = getattr(lib, f"shaobo_fa3_bwd_{f}_workspace_bytes")
        assert fn(ctypes.byref(component_params(lib))) == 0
        assert fn(None) == 0
        p = component_params(lib)
        setattr(p, attr, 1)
        assert fn(ctypes.byref(p)) == naive_bytes(1, 2, 256)
        p = component_params(lib, batch=2, seqlen=200, heads_q=3, causal=False)
        setattr(p, attr, 1)  # any length, either causal flag
        assert fn(ctypes.byref(p)) == naive_bytes(2, 3, 200)
        for name, mut in [("num_heads_kv", 1), ("seqlen_k", 128), ("dtype", F.DTYPE_BF16),
                          ("layout", F.LAYOUT_BSHD), ("head_dim_qk", 96), ("dropout_p", 0.1)]:
            p = component_params(lib)
            setattr(p, attr, 1)
            setattr(p, name, mut)
            assert fn(ctypes.byref(p)) == 0, (f, name)
        p = component_params(lib, batch=1 << 20, seqlen=1 << 20, heads_q=1 << 10)
        setattr(p, attr, 1)
        assert fn(ctypes.byref(p)) == 0  # overflows
    ws5 = lib.shaobo_fa3_bwd_fused5_workspace_bytes
    assert ws5(None) == 0
    assert ws5(ctypes.byref(component_params(lib, seqlen=2048, heads_q=4))) == \
        split_plan_bytes(1, 4, 2048, 128)
    p = component_params(lib, heads_q=4, heads_kv=2, causal=False)
    assert ws5(ctypes.byref(p)) == plain_bytes(1, 4, 256)
    p = component_params(lib)
    p.seqlen_k = 512
    assert ws5(ctypes.byref(p)) == 0
    p = component_params(lib, head_dim=96)
    assert ws5(ctypes.byref(p)) == 0


def test_component_error_paths_without_gpu(lib):
    """Shape / path checks come before pointer checks, as in the reference
    (src/dkv_kernel.cpp:1390-1398, src/dq_kernel.cpp:1515-1525,
    src/fused_bwd_kernel.cpp:1682-1703); every case returns before a launch."""
    one = ctypes.c_void_p(16)
    ten = [one] * 10
    for name, mut in [("dkv_path", 2), ("causal", 0), ("num_heads_kv", 1), ("head_dim_qk", 96),
                      ("seqlen_q", 200), ("dtype", F.DTYPE_BF16), ("layout", F.LAYOUT_BSHD)]:
        p = component_params(lib)
        p.reserved_ptr[3] = 16
        setattr(p, name, mut)
        assert lib.shaobo_fa3_bwd_dkv(*ten, ctypes.byref(p)) == F.UNSUPPORTED, name
    for name, mut in [("dq_path", 2), ("dq_path", 5), ("causal", 0), ("seqlen_k", 512)]:
        p = component_params(lib)
        p.reserved_ptr[0] = 16
        setattr(p, name, mut)
        assert lib.shaobo_fa3_bwd_dq(*ten, ctypes.byref(p)) == F.UNSUPPORTED, name
    assert lib.shaobo_fa3_bwd_dkv(*ten, None) == F.INVALID_VALUE
    assert lib.shaobo_fa3_bwd_dq(*ten, None) == F.INVALID_VALUE
    p = component_params(lib)  # sidecar missing in reserved_ptr[3]
    assert lib.shaobo_fa3_bwd_dkv(*ten, ctypes.byref(p)) == F.INVALID_VALUE
    p.reserved_ptr[3] = 16
    bad = list(ten)
    bad[8] = None  # dk
    assert lib.shaobo_fa3_bwd_dkv(*bad, ctypes.byref(p)) == F.INVALID_VALUE
    p = component_params(lib)  # delta missing in reserved_ptr[0]
    assert lib.shaobo_fa3_bwd_dq(*ten, ctypes.byref(p)) == F.INVALID_VALUE
    p.reserved_ptr[0] = 16
    bad = list(ten)
    bad[6] = None  # aux1 (row sum)
    assert lib.shaobo_fa3_bwd_dq(*bad, ctypes.byref(p)) == F.INVALID_VALUE
    # fused5
    eight = [one] * 8
    p = component_params(lib, heads_q=3, heads_kv=2)
    assert lib.shaobo_fa3_bwd_fused5(*eight, ctypes.byref(p)) == F.UNSUPPORTED
    p = component_params(lib)
    p.causal = 2
    assert lib.shaobo_fa3_bwd_fused5(*eight, ctypes.byref(p)) == F.UNSUPPORTED
    p = component_params(lib)
    bad = list(eight)
    bad[4] = None  # packed sidecar
    assert lib.shaobo_fa3_bwd_fused5(*bad, ctypes.byref(p)) == F.INVALID_VALUE
    p.workspace, p.workspace_bytes = 16, 8  # too small
    assert lib.shaobo_fa3_bwd_fused5(*eight, ctypes.byref(p)) == F.INVALID_VALUE
    p.workspace, p.workspace_bytes = None, 1 << 30
    assert lib.shaobo_fa3_bwd_fused5(*eight, ctypes.byref(p)) == F.INVALID_VALUE
    assert lib.shaobo_fa3_bwd_fused5(*eight, None) == F.INVALID_VALUE


def test_naive_path_error_paths_without_gpu(lib):
    """Path 1 of dkv / dq (reference src/dkv_kernel.cpp:1320-1334,
    src/dq_kernel.cpp:1562-1574): shape checks -> UNSUPPORTED, then missing
    pointers, a missing or short workspace -> INVALID_VALUE; every case
    returns before a launch."""
    one = ctypes.c_void_p(16)
    ten = [one] * 10
    need = naive_bytes(1, 2, 256)
    for fn, attr, out_idx in ((lib.shaobo_fa3_bwd_dkv, "dkv_path", 8),
                              (lib.shaobo_fa3_bwd_dq, "dq_path", 7)):
        for name, mut in [("num_heads_kv", 1), ("seqlen_k", 128), ("dtype", F.DTYPE_BF16),
                          ("layout", F.LAYOUT_BSHD), ("dropout_p", 0.1), ("head_dim_qk", 96)]:
            p = component_params(lib)
            setattr(p, attr, 1)
            setattr(p, name, mut)
            assert fn(*ten, ctypes.byref(p)) == F.UNSUPPORTED, (attr, name)
        p = component_params(lib)
        setattr(p, attr, 1)
        assert fn(*ten, ctypes.byref(p)) == F.INVALID_VALUE  # no workspace
        p.workspace, p.workspace_bytes = 16, need - 4
        assert fn(*ten, ctypes.byref(p)) == F.INVALID_VALUE  # short workspace
        p.workspace_bytes = need
        bad = list(ten)
        bad[out_idx] = None
        assert fn(*bad, ctypes.byref(p)) == F.INVALID_VALUE  # dk / dq missing
        bad = list(ten)
        bad[1] = None
        assert fn(*bad, ctypes.byref(p)) == F.INVALID_VALUE  # q missing
