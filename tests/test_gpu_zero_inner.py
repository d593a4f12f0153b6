"""GPU: products whose inner dimension is 0 write an all-zero output (the empty sum),
through the C ABI's fill kernel, for every GEMM-shaped operator that accepts K = 0
(or F = 0 for SwiGLU).  The output buffer is first filled with NaN and freed, so
torch's caching allocator hands the same dirty block back to the operator."""
import pytest
import torch

from kda import ops

pytestmark = pytest.mark.gpu
BF16, F32 = torch.bfloat16, torch.float32


def _dirty(shape, dtype):
    t = torch.full(shape, float("nan"), dtype=dtype, device="cuda")
    torch.cuda.synchronize()
    del t


def _z(*shape, dtype=F32):
    return torch.empty(shape, dtype=dtype, device="cuda")


def _r(*shape, dtype=F32):
    return torch.randn(shape, dtype=F32, device="cuda").to(dtype)


def _check_zero(out, shape, dtype, name):
    torch.cuda.synchronize()
    print(f"{name}: shape {tuple(out.shape)}", flush=True)
    assert out.shape == shape and out.dtype == dtype
    assert torch.count_nonzero(out).item() == 0 and not torch.isnan(out).any().item(), name


@pytest.mark.parametrize("dtype", [BF16, F32])
def test_matmul_k0(dtype):
    _dirty((72, 136), dtype)
    out = ops.matmul(_z(72, 0, dtype=dtype), _z(0, 136, dtype=dtype))
    _check_zero(out, (72, 136), dtype, f"matmul {dtype}")


def test_transpose_matmul_k0():
    _dirty((64, 40), F32)
    out = ops.transpose_matmul(_z(0, 64), _z(0, 40))
    _check_zero(out, (64, 40), F32, "transpose_matmul")


def test_bmm_k0():
    _dirty((3, 50, 24), F32)
    out = ops.bmm(_z(3, 50, 0), _z(3, 0, 24))
    _check_zero(out, (3, 50, 24), F32, "bmm")


def test_lora_k0():
    _dirty((33, 64), F32)
    out = ops.lora(_z(33, 0), _z(0, 64), _z(0, 32), _r(32, 64))
    _check_zero(out, (33, 64), F32, "lora")


@pytest.mark.parametrize("dtype", [BF16, F32])
def test_swiglu_f0(dtype):
    _dirty((40, 64), dtype)
    out = ops.swiglu(_r(40, 64, dtype=dtype), _z(64, 0, dtype=dtype), _z(0, 64, dtype=dtype),
                     _z(64, 0, dtype=dtype))
    _check_zero(out, (40, 64), dtype, f"swiglu {dtype}")
