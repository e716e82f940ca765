"""PyTorch binding of the MI355X FA3 backward as a custom op.

``torch.ops.shaobo_fa3.flash_attn_backward`` is the framework binding the
reference describes but does not ship (reference docs/tridao_fa3_bwd_api.md:
48-51, docs/fused5_gqa_contract_20260820.md:20-32): it allocates dQ, dK, dV,
softmax_d and the workspace with torch and launches on torch's current
stream through the library's stream entry point
(shaobo_fa3_bwd_v2_on_stream, include/shaobo_fa3_ext.h), so it orders
correctly with the surrounding torch work and with CUDA-graph capture of
that stream.  A fake (meta) implementation gives shapes for tracing.

The op launches without synchronising, so a split wait that gave up (the
library's bounded wait between two workgroups sharing one output tile) cannot
fail the call itself; ``check_split_errors`` is the op's synchronisation
point that reports it (through shaobo_fa3_ext_split_error_count).

``attention`` wraps it in an autograd function whose forward is a plain
torch computation (O and the natural-log LSE in fp32, O rounded to the inputs' dtype) --
an integration example and a test vehicle; the library provides the
backward only.
"""
import ctypes
import math
from typing import Optional, Tuple

import torch

import shaobo_fa3 as F

_ON_STREAM = None


def _lib():
    global _ON_STREAM
    lib = F.load()
    if _ON_STREAM is None:
        fn = lib.shaobo_fa3_bwd_v2_on_stream
        fn.argtypes = [ctypes.c_void_p] * 10 + [ctypes.POINTER(F.Params), ctypes.c_void_p]
        fn.restype = ctypes.c_int
        _ON_STREAM = fn
    return lib


def _check(dout, q, k, v, out, lse):
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape or out.shape != q.shape \
            or dout.shape != q.shape:
        raise ValueError("expected BHSD tensors: q, out, dout [B, Hq, S, D], k, v [B, Hkv, S, D]")
    B, Hq, S, D = q.shape
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D or Hq % k.shape[1]:
        raise ValueError("k / v shape does not match q")
    if lse.shape != (B, Hq, S) or lse.dtype != torch.float32:
        raise ValueError("softmax_lse must be fp32 [B, Hq, S]")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q, k, v, out, dout must be fp16 or bf16")
    for t in (dout, k, v, out):
        if t.dtype != q.dtype:
            raise ValueError("q, k, v, out, dout must share one dtype")
    for t in (dout, q, k, v, out, lse):
        if not t.is_contiguous():
            raise ValueError("tensors must be contiguous (BHSD)")
        if t.device != q.device or t.device.type != "cuda":
            raise ValueError("tensors must be on the same GPU")


@torch.library.custom_op("shaobo_fa3::flash_attn_backward", mutates_args=(),
                         device_types="cuda")
def flash_attn_backward(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        out: torch.Tensor, softmax_lse: torch.Tensor, causal: bool,
                        softmax_scale: Optional[float] = None, deterministic: bool = False
                        ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV, softmax_d) of softmax(scale Q K^T) V given dO, O and the
    natural-log LSE; fp16 or bf16 BHSD in and out, softmax_d fp32 [B, Hq, S]."""
    _check(dout, q, k, v, out, softmax_lse)
    lib = _lib()
    B, Hq, S, D = q.shape
    p = F.make_params(lib, batch=B, seqlen=S, heads_q=Hq, heads_kv=k.shape[1], head_dim=D,
                      causal=causal, softmax_scale=softmax_scale, deterministic=deterministic)
    if q.dtype == torch.bfloat16:
        p.dtype = F.DTYPE_BF16
    nbytes = lib.shaobo_fa3_bwd_v2_workspace_bytes(ctypes.byref(p))
    if nbytes == 0:
        raise RuntimeError("shaobo_fa3_bwd_v2: " +
                           F.status_name(lib.shaobo_fa3_bwd_v2_validate(ctypes.byref(p))))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    c = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        st = _ON_STREAM(c(dout), c(q), c(k), c(v), c(out), c(softmax_lse), c(dq), c(dk), c(dv),
                        c(delta), ctypes.byref(p), ctypes.c_void_p(stream))
    if st != F.SUCCESS:
        raise RuntimeError("shaobo_fa3_bwd_v2_on_stream: " + F.status_name(st))
    return dq, dk, dv, delta


_SPLIT_ERRORS_SEEN = {}


def check_split_errors(device=None):
    """Synchronise torch's current stream on `device` and raise RuntimeError
    if a split wait of the library gave up on that GPU since the previous
    check (those launches returned wrong gradients).  Call it where the
    caller synchronises anyway (end of a step, before reading a loss)."""
    lib = _lib()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None \
        else torch.device(device)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        n = ctypes.c_ulonglong(0)
        st = lib.shaobo_fa3_ext_split_error_count(ctypes.c_void_p(stream), ctypes.byref(n))
    if st != F.SUCCESS:
        raise RuntimeError("shaobo_fa3_ext_split_error_count: " + F.status_name(st))
    seen = _SPLIT_ERRORS_SEEN.get(dev.index, 0)
    _SPLIT_ERRORS_SEEN[dev.index] = n.value
    if n.value != seen:
        raise RuntimeError(f"shaobo_fa3: {n.value - seen} split wait(s) gave up on {dev}: "
                           "the gradients of those backward calls are wrong")


@flash_attn_backward.register_fake
def _(dout, q, k, v, out, softmax_lse, causal, softmax_scale=None, deterministic=False):
    _check(dout, q, k, v, out, softmax_lse)
    B, Hq, S, _ = q.shape
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            q.new_empty((B, Hq, S), dtype=torch.float32))


def reference_forward(q, k, v, causal, scale):
    """O (the inputs' dtype) and natural-log LSE (fp32) in fp32 torch math."""
    G = q.shape[1] // k.shape[1]
    kf = k.float().repeat_interleave(G, dim=1)
    vf = v.float().repeat_interleave(G, dim=1)
    s = torch.matmul(q.float(), kf.transpose(-1, -2).contiguous()) * scale
    if causal:
        S = q.shape[2]
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device=q.device), 1),
                          float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.matmul(torch.softmax(s, dim=-1), vf).to(q.dtype)
    return out.contiguous(), lse.contiguous()


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal, scale):
        out, lse = reference_forward(q, k, v, causal, scale)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal, ctx.scale = causal, scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv, _ = torch.ops.shaobo_fa3.flash_attn_backward(
            dout.contiguous(), q, k, v, out, lse, ctx.causal, ctx.scale, False)
        return dq, dk, dv, None, None


def attention(q, k, v, causal=True, softmax_scale=None):
    """softmax(scale Q K^T) V with the MI355X FA3 backward (fp16 / bf16 BHSD)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else softmax_scale
    return _Attention.apply(q, k, v, causal, scale)
