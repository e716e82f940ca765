"""ctypes binding of libshaobo_fa3_bwd.so, the MI355X FA3 backward C ABI.

This is the reference-side binding a Python framework would add
(reference include/shaobo_fa3_api.h:53-147 mirrored field by field).  It only
marshals pointers: all compute happens in the HIP library, and loading fails
loudly when the library has not been built (no CPU fallback exists).

Torch is used only for device memory; ``bwd_v2`` takes CUDA (HIP) tensors.
"""
import ctypes
import math
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libshaobo_fa3_bwd.so")

API_VERSION = 2
STATUS = {0: "success", 1: "invalid_value", 2: "unsupported", 3: "not_implemented",
          4: "hip_error"}
SUCCESS, INVALID_VALUE, UNSUPPORTED, NOT_IMPLEMENTED, HIP_ERROR = range(5)
DTYPE_FP16, DTYPE_BF16, DTYPE_FP8 = range(3)
LAYOUT_BHSD, LAYOUT_BSHD = range(2)
AUX_SMAX_SSUM, AUX_LSE = range(2)

FEATURES = {name: 1 << bit for bit, name in enumerate([
    "FIXED_LENGTH", "VARLEN", "FP16", "BF16", "CAUSAL", "LOCAL_WINDOW", "GQA", "SOFTCAP",
    "DETERMINISTIC", "SOFTMAX_LSE", "BSHD", "BHSD", "FULL_ATTENTION"])}

EXPORTS = (
    "shaobo_fa3_params_init", "shaobo_fa3_bwd_get_capabilities", "shaobo_fa3_bwd_v2_validate",
    "shaobo_fa3_bwd_v2_workspace_bytes", "shaobo_fa3_bwd_v2", "shaobo_fa3_status_string",
    "shaobo_fa3_bwd_workspace_bytes", "shaobo_fa3_bwd", "shaobo_fa3_bwd_dot_do_o",
    "shaobo_fa3_bwd_fused5_workspace_bytes", "shaobo_fa3_bwd_fused5",
    "shaobo_fa3_bwd_dkv_workspace_bytes", "shaobo_fa3_bwd_dkv",
    "shaobo_fa3_bwd_dq_workspace_bytes", "shaobo_fa3_bwd_dq",
    "shaobo_fa3_bwd_v2_on_stream", "shaobo_fa3_ext_set_split_spin_limit",
    "shaobo_fa3_ext_bwd_v2_no_alloc", "shaobo_fa3_ext_bwd_v2_timed",
    "shaobo_fa3_ext_bwd_v2_stages", "shaobo_fa3_ext_split_status",
    "shaobo_fa3_ext_split_error_count",
)

# Size of the static device scratch array behind shaobo_fa3_ext_bwd_v2_no_alloc
# (SHAOBO_FA3_EXT_SCRATCH_BYTES in include/shaobo_fa3_ext.h).
NO_ALLOC_SCRATCH_BYTES = 32 << 20

# Component path selectors (params.dkv_path / params.dq_path) of the canonical
# dK/dV and dQ component kernels.
DKV_PATH_CANONICAL = 5
DQ_PATH_CANONICAL = 6


class Params(ctypes.Structure):
    """ShaoboFa3Params (sizeof 296 on x86-64)."""
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_k", ctypes.c_int32),
        ("num_heads_q", ctypes.c_int32),
        ("num_heads_kv", ctypes.c_int32),
        ("head_dim_qk", ctypes.c_int32),
        ("head_dim_v", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("window_left", ctypes.c_int32),
        ("window_right", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("dropout_p", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("softmax_aux_mode", ctypes.c_int32),
        ("dkv_path", ctypes.c_int32),
        ("dq_path", ctypes.c_int32),
        ("block_threads", ctypes.c_int32),
        ("sync_after_launch", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("max_seqlen_q", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("reserved_i32", ctypes.c_int32 * 16),
        ("reserved_ptr", ctypes.c_void_p * 8),
        ("seqused_q", ctypes.c_void_p),
        ("seqused_k", ctypes.c_void_p),
        ("total_q", ctypes.c_int64),
        ("total_k", ctypes.c_int64),
        ("softcap", ctypes.c_float),
        ("deterministic", ctypes.c_int32),
        ("sm_margin", ctypes.c_int32),
        ("softmax_scale_is_set", ctypes.c_int32),
    ]


class Capabilities(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("api_version", ctypes.c_uint32),
        ("feature_mask", ctypes.c_uint64),
        ("min_head_dim", ctypes.c_int32),
        ("max_head_dim", ctypes.c_int32),
        ("head_dim_alignment", ctypes.c_int32),
        ("sequence_alignment", ctypes.c_int32),
    ]


def _declare(lib):
    P = ctypes.POINTER(Params)
    vp = ctypes.c_void_p
    lib.shaobo_fa3_params_init.argtypes = [P]
    lib.shaobo_fa3_params_init.restype = None
    lib.shaobo_fa3_bwd_get_capabilities.argtypes = [ctypes.POINTER(Capabilities)]
    lib.shaobo_fa3_bwd_get_capabilities.restype = ctypes.c_int
    lib.shaobo_fa3_bwd_v2_validate.argtypes = [P]
    lib.shaobo_fa3_bwd_v2_validate.restype = ctypes.c_int
    if hasattr(lib, "shaobo_fa3_bwd_v2_workspace_bytes"):
        lib.shaobo_fa3_bwd_v2_workspace_bytes.argtypes = [P]
        lib.shaobo_fa3_bwd_v2_workspace_bytes.restype = ctypes.c_size_t
    if hasattr(lib, "shaobo_fa3_bwd_v2"):
        lib.shaobo_fa3_bwd_v2.argtypes = [vp] * 10 + [P]
        lib.shaobo_fa3_bwd_v2.restype = ctypes.c_int
    return lib


_LIB = None


def load(path=LIB_PATH):
    """Load the HIP library once; raises if it has not been built."""
    global _LIB
    if _LIB is None or path != LIB_PATH:
        if not os.path.exists(path):
            raise RuntimeError(f"libshaobo_fa3_bwd.so not built at {path}: run "
                               "`make -C flash-attention3_amd` (no CPU fallback exists)")
        lib = _declare(ctypes.CDLL(path))
        lib.shaobo_fa3_status_string.argtypes = [ctypes.c_int]
        lib.shaobo_fa3_status_string.restype = ctypes.c_char_p
        lib.shaobo_fa3_bwd_workspace_bytes.argtypes = [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.shaobo_fa3_bwd.argtypes = [ctypes.c_void_p] * 10 + [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd.restype = ctypes.c_int
        lib.shaobo_fa3_bwd_dot_do_o.argtypes = [ctypes.c_void_p] * 6 + [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd_dot_do_o.restype = ctypes.c_int
        for name in ("fused5", "dkv", "dq"):
            getattr(lib, f"shaobo_fa3_bwd_{name}_workspace_bytes").argtypes = [
                ctypes.POINTER(Params)]
            getattr(lib, f"shaobo_fa3_bwd_{name}_workspace_bytes").restype = ctypes.c_size_t
        lib.shaobo_fa3_bwd_fused5.argtypes = [ctypes.c_void_p] * 8 + [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd_fused5.restype = ctypes.c_int
        lib.shaobo_fa3_bwd_dkv.argtypes = [ctypes.c_void_p] * 10 + [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd_dkv.restype = ctypes.c_int
        lib.shaobo_fa3_bwd_dq.argtypes = [ctypes.c_void_p] * 10 + [ctypes.POINTER(Params)]
        lib.shaobo_fa3_bwd_dq.restype = ctypes.c_int
        lib.shaobo_fa3_ext_set_split_spin_limit.argtypes = [ctypes.c_int]
        lib.shaobo_fa3_ext_set_split_spin_limit.restype = None
        lib.shaobo_fa3_ext_bwd_v2_no_alloc.argtypes = [ctypes.c_void_p] * 10 + [
            ctypes.POINTER(Params), ctypes.c_void_p]
        lib.shaobo_fa3_ext_bwd_v2_no_alloc.restype = ctypes.c_int
        lib.shaobo_fa3_ext_bwd_v2_timed.argtypes = [ctypes.c_void_p] * 10 + [
            ctypes.POINTER(Params), ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
        lib.shaobo_fa3_ext_bwd_v2_timed.restype = ctypes.c_int
        lib.shaobo_fa3_ext_bwd_v2_stages.argtypes = [ctypes.c_void_p] * 10 + [
            ctypes.POINTER(Params), ctypes.c_void_p, ctypes.c_int]
        lib.shaobo_fa3_ext_bwd_v2_stages.restype = ctypes.c_int
        lib.shaobo_fa3_ext_split_status.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.shaobo_fa3_ext_split_status.restype = ctypes.c_int
        lib.shaobo_fa3_ext_split_error_count.argtypes = [
            ctypes.c_void_p, ctypes.POINTER(ctypes.c_ulonglong)]
        lib.shaobo_fa3_ext_split_error_count.restype = ctypes.c_int
        if path != LIB_PATH:
            return lib
        _LIB = lib
    return _LIB


def declare_abi(lib):
    """Attach the ABI signatures to another build of the same ABI."""
    return _declare(lib)


def make_params(lib=None, *, batch, seqlen, heads_q, heads_kv=None, head_dim=128, causal=True,
                softmax_scale=None, deterministic=False, sync=False):
    lib = lib or load()
    p = Params()
    lib.shaobo_fa3_params_init(ctypes.byref(p))
    p.batch = batch
    p.seqlen_q = p.seqlen_k = seqlen
    p.num_heads_q = heads_q
    p.num_heads_kv = heads_q if heads_kv is None else heads_kv
    p.head_dim_qk = p.head_dim_v = head_dim
    p.causal = int(bool(causal))
    if softmax_scale is not None:
        p.softmax_scale = softmax_scale
        p.softmax_scale_is_set = 1
    p.deterministic = int(bool(deterministic))
    p.sync_after_launch = int(bool(sync))
    return p


def status_name(code):
    return STATUS.get(code, "unknown")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def bwd_v2(dout, q, k, v, out, lse, *, causal=True, softmax_scale=None, deterministic=False,
           softmax_d=None, workspace=None, sync=False):
    """Run shaobo_fa3_bwd_v2 on torch device tensors (fp16 BHSD, fp32 LSE).

    Allocates dq/dk/dv (and the workspace unless one is given) with torch and
    returns (dq, dk, dv).  Raises RuntimeError with the status name on failure.
    """
    import torch
    lib = load()
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    p = make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=Hkv, head_dim=D, causal=causal,
                    softmax_scale=softmax_scale, deterministic=deterministic, sync=sync)
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    if nbytes == 0:
        raise RuntimeError("shaobo_fa3_bwd_v2: " +
                           status_name(lib.shaobo_fa3_bwd_v2_validate(ctypes.byref(p))))
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    p.workspace = workspace.data_ptr()
    p.workspace_bytes = workspace.numel() * workspace.element_size()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    st = lib.shaobo_fa3_bwd_v2(_ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
                               _ptr(dq), _ptr(dk), _ptr(dv), _ptr(softmax_d), ctypes.byref(p))
    if st != SUCCESS:
        raise RuntimeError("shaobo_fa3_bwd_v2: " + status_name(st))
    return dq, dk, dv


def default_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)
