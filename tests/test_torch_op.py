"""PyTorch custom-op binding (flash-attention3_amd/shaobo_fa3_torch.py), host
side: registration, the fake implementation's shapes, argument checks.  The
GPU behaviour is in test_gpu_torch_op.py."""
import pytest

torch = pytest.importorskip("torch")
from torch._subclasses.fake_tensor import FakeTensorMode  # noqa: E402

import shaobo_fa3_torch  # noqa: E402,F401  (registers the op)


def tensors(B=2, Hq=4, Hkv=2, S=256, D=128, dtype=torch.float16):
    q = torch.empty(B, Hq, S, D, dtype=dtype, device="cuda")
    k = torch.empty(B, Hkv, S, D, dtype=dtype, device="cuda")
    v = torch.empty_like(k)
    out = torch.empty_like(q)
    dout = torch.empty_like(q)
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device="cuda")
    return dout, q, k, v, out, lse


def test_op_is_registered():
    assert hasattr(torch.ops.shaobo_fa3, "flash_attn_backward")


def test_fake_shapes_bf16():
    with FakeTensorMode():
        args = tensors(dtype=torch.bfloat16)
        dq, dk, dv, delta = torch.ops.shaobo_fa3.flash_attn_backward(*args, False, 0.1, False)
        assert dq.dtype == torch.bfloat16 and dk.shape == args[2].shape


def test_fake_shapes():
    with FakeTensorMode():
        dout, q, k, v, out, lse = tensors()
        dq, dk, dv, delta = torch.ops.shaobo_fa3.flash_attn_backward(dout, q, k, v, out, lse, True,
                                                                     None, False)
        assert dq.shape == q.shape and dq.dtype == torch.float16
        assert dk.shape == k.shape and dv.shape == v.shape
        assert delta.shape == (2, 4, 256) and delta.dtype == torch.float32


@pytest.mark.parametrize("bad", ["dtype", "lse_shape", "heads", "noncontig"])
def test_fake_rejects_bad_arguments(bad):
    with FakeTensorMode():
        dout, q, k, v, out, lse = tensors()
        if bad == "dtype":
            q = q.to(torch.bfloat16)  # mixed with fp16 k / v / out / dout
        elif bad == "lse_shape":
            lse = lse[:, :, :128]
        elif bad == "heads":
            k = torch.empty(2, 3, 256, 128, dtype=torch.float16, device="cuda")
            v = torch.empty_like(k)
        elif bad == "noncontig":
            q = q.transpose(1, 2)
        with pytest.raises(ValueError):
            torch.ops.shaobo_fa3.flash_attn_backward(dout, q, k, v, out, lse, True, None, False)
