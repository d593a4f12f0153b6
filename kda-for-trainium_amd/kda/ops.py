"""One Python callable per operator, backed by the gfx950 kernels in libkda.so.

Each callable takes the natural-layout tensors that the reference's adapter
hands to numpy ``forward(...)`` -- keyword names are forward()'s parameter
names (adapter/nkibench_case.py:147-155, 199-216) -- and returns the output
tensor, allocated on the inputs' device.  Inputs must be contiguous CUDA (ROCm)
tensors of the stated dtype; anything else raises ValueError before any launch.
Every kernel runs on the current torch stream of the inputs' device.  There is
no CPU or PyTorch fallback: without libkda.so these functions raise.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib

__all__ = [
    "silu",
    "adamw",
    "adamw_step_",
    "rope_single_freq_apply",
    "workspace_size",
    "matmul",
    "transpose_matmul",
    "bmm",
    "bmm_softmax",
    "lora",
    "rmsnorm_matmul",
    "rmsnorm_matmul_workspace_size",
    "add_rmsnorm_matmul",
    "matmul_add_rmsnorm",
    "swiglu",
    "mamba",
    "gqa",
    "gqa_full",
]

BF16 = torch.bfloat16
F32 = torch.float32


# ----------------------------------------------------------------- helpers

def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(name: str, t: torch.Tensor, dtype: torch.dtype,
           shape: Optional[Sequence[int]] = None, ndim: Optional[int] = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a GPU tensor (got device {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim} dims, got shape {tuple(t.shape)}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")


def _same_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on one device ({dev} vs {t.device})")


# ----------------------------------------------------------------- elementwise

def silu(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x / (1 + exp(-x)), fp32, any shape.

    Reference: workspaces/silu/runs/silu_v3_s7.py:31-71 (kernel(v1)); forward
    ``y = x/(1+exp(-x))`` per prompts/_gen_prompts.py:25.
    """
    _check("x", x, torch.float32)
    if out is None:
        out = torch.empty_like(x)
    else:
        _check("out", out, torch.float32, shape=x.shape)
        _same_device(x, out)
    _lib.call("kda_silu_f32", x.data_ptr(), out.data_ptr(), x.numel(), _stream(x))
    return out


def adamw(theta: torch.Tensor, g: torch.Tensor, m: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """NKIBench AdamW forward: returns the new theta, leaves m and v untouched.

    ``theta_t = theta - 1e-5*theta; m_t = 0.9m + 0.1g; v_t = 0.999v + 0.001g^2;
    new = theta_t - 0.01*m_t/(sqrt(1000*v_t) + 1e-8)`` -- i.e. one decoupled-
    weight-decay Adam step at step 1 with lr 1e-3, weight decay 1e-2, eps 1e-8
    (workspaces/adamw/docs/draft-phase1.md:20-26; kernel(v1..v4) =
    (theta, g, m, v) of workspaces/adamw/runs/adamw_v1.py:50-97).
    """
    for name, t in (("theta", theta), ("g", g), ("m", m), ("v", v)):
        _check(name, t, torch.float32, shape=theta.shape)
    _same_device(theta, g, m, v)
    out = torch.empty_like(theta)
    _lib.call("kda_adamw_f32", theta.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
              out.data_ptr(), None, None, theta.numel(),
              1e-3, 0.9, 0.999, 1e-8, 1e-2, 1, _stream(theta))
    return out


def adamw_step_(param: torch.Tensor, grad: torch.Tensor, m: torch.Tensor, v: torch.Tensor,
                lr: float = 1e-3, beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8,
                weight_decay: float = 1e-2, step: int = 1) -> torch.Tensor:
    """In-place fused AdamW step over flat fp32 buffers; updates param, m, v.

    Same update as torch.optim.AdamW (non-amsgrad, maximize=False) at the given
    step count: ``p *= 1-lr*wd; m = b1*m+(1-b1)*g; v = b2*v+(1-b2)*g^2;
    p -= lr/(1-b1^step) * m / (sqrt(v)/sqrt(1-b2^step) + eps)``.  One pass:
    reads p, g, m, v and writes p, m, v (28 bytes per element).
    """
    for name, t in (("param", param), ("grad", grad), ("m", m), ("v", v)):
        _check(name, t, torch.float32, shape=param.shape)
    _same_device(param, grad, m, v)
    if int(step) < 1:
        raise ValueError(f"step must be >= 1, got {step}")
    _lib.call("kda_adamw_f32", param.data_ptr(), grad.data_ptr(), m.data_ptr(), v.data_ptr(),
              param.data_ptr(), m.data_ptr(), v.data_ptr(), param.numel(),
              float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), int(step),
              _stream(param))
    return param


def rope_single_freq_apply(x_in: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Half-split RoPE along axis 0: x_in (D, S), cos/sin (D/2, S), fp32.

    ``out[:D/2] = x0*cos - x1*sin; out[D/2:] = x0*sin + x1*cos`` with
    x0 = x_in[:D/2], x1 = x_in[D/2:] (workspaces/rope_single_freq_apply/docs/
    draft-phase1.md:18-27; kernel(x_in, cos, sin) of
    workspaces/rope_single_freq_apply/runs/rope_v1.py:32-80).  Bit-identical to
    the numpy reference (no fused multiply-add).
    """
    _check("x_in", x_in, torch.float32, ndim=2)
    d, s = x_in.shape
    if d % 2:
        raise ValueError(f"x_in: head dim {d} must be even")
    _check("cos", cos, torch.float32, shape=(d // 2, s))
    _check("sin", sin, torch.float32, shape=(d // 2, s))
    _same_device(x_in, cos, sin)
    out = torch.empty_like(x_in)
    _lib.call("kda_rope_f32", x_in.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(),
              d, s, _stream(x_in))
    return out


# ----------------------------------------------------------------- GEMM family
#
# bf16 inputs run on bf16 MFMA with fp32 accumulation and return bf16.  fp32
# inputs (the reference's NKIBench operators) run on bf16 MFMA through a
# three-product split (x = hi + lo, A@B ~= Ah@Bh + Ah@Bl + Al@Bh, fp32
# accumulation) and return fp32; their intermediates live in a workspace that
# is allocated here unless the caller passes ``workspace`` (a uint8 GPU tensor of
# at least ``workspace_size(...)`` bytes).

def workspace_size(op: int, batch: int = 0, m: int = 0, k: int = 0, n: int = 0, r: int = 0) -> int:
    """Workspace bytes of operator id `op` (kda._lib.OP_*) at the given sizes."""
    size = _lib.query("kda_workspace_size", int(op), int(batch), int(m), int(k), int(n), int(r))
    if size < 0:
        raise ValueError(f"workspace_size: bad operator {op} or sizes")
    return size


def _workspace(workspace: Optional[torch.Tensor], need: int, device: torch.device) -> torch.Tensor:
    if workspace is None:
        return torch.empty(max(need, 16), dtype=torch.uint8, device=device)
    _check("workspace", workspace, torch.uint8, ndim=1)
    if workspace.device != device:
        raise ValueError("workspace must be on the inputs' device")
    return workspace


def _gemm_dims(name_a: str, a: torch.Tensor, name_b: str, b: torch.Tensor):
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError(f"{name_a}, {name_b}: expected 2-D tensors, got {tuple(a.shape)}, {tuple(b.shape)}")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"inner dims differ: {name_a} {tuple(a.shape)} vs {name_b} {tuple(b.shape)}")
    return a.shape[0], a.shape[1], b.shape[1]


def _same_dtype(*named):
    dt = named[0][1].dtype
    for name, t in named:
        _check(name, t, dt)
    if dt not in (BF16, F32):
        raise ValueError(f"unsupported dtype {dt} (bf16 or fp32)")
    _same_device(*(t for _, t in named))
    return dt


def matmul(lhs: torch.Tensor, rhs: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = lhs @ rhs, lhs (M, K), rhs (K, N); bf16 -> bf16, fp32 -> fp32 (split).

    Reference: workspaces/matmul/runs/matmul_v3_bf16_split.py:10-161, forward
    ``lhs @ rhs`` (workspaces/matmul/runs/offline_bf16_split_sim.py:137-139).
    """
    dt = _same_dtype(("lhs", lhs), ("rhs", rhs))
    m, k, n = _gemm_dims("lhs", lhs, "rhs", rhs)
    out = torch.empty((m, n), dtype=dt, device=lhs.device)
    if dt == BF16:
        _lib.call("kda_matmul_bf16", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), m, k, n, _stream(lhs))
        return out
    ws = _workspace(workspace, workspace_size(_lib.OP_MATMUL_F32, 1, m, k, n), lhs.device)
    _lib.call("kda_matmul_f32", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), m, k, n,
              ws.data_ptr(), ws.numel(), _stream(lhs))
    return out


def transpose_matmul(lhs: torch.Tensor, rhs: torch.Tensor,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = lhs.T @ rhs with lhs (K, M), rhs (K, N), fp32.

    Reference: workspaces/transpose_matmul/runs/tmm_v3_mblk16_bf16_split.py:10-41,
    forward ``transpose(lhs) @ rhs`` (workspaces/transpose_matmul/runs/offline_bf16_split_sim.py:101-104).
    """
    _same_dtype(("lhs", lhs), ("rhs", rhs))
    _check("lhs", lhs, F32, ndim=2)
    _check("rhs", rhs, F32, ndim=2)
    k, m = lhs.shape
    if rhs.shape[0] != k:
        raise ValueError(f"transpose_matmul: lhs {tuple(lhs.shape)} and rhs {tuple(rhs.shape)} differ in K")
    n = rhs.shape[1]
    out = torch.empty((m, n), dtype=F32, device=lhs.device)
    ws = _workspace(workspace, workspace_size(_lib.OP_TRANSPOSE_MATMUL_F32, 1, m, k, n), lhs.device)
    _lib.call("kda_transpose_matmul_f32", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), m, k, n,
              ws.data_ptr(), ws.numel(), _stream(lhs))
    return out


def bmm(lhs: torch.Tensor, rhs: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[b] = lhs[b] @ rhs[b], lhs (B, M, K), rhs (B, K, N), fp32.

    Reference: workspaces/bmm/runs/bmm_v2.py:10-41 (forward per-batch lhs[b] @ rhs[b],
    workspaces/bmm/docs/draft-phase1.md:3-5).
    """
    _same_dtype(("lhs", lhs), ("rhs", rhs))
    _check("lhs", lhs, F32, ndim=3)
    _check("rhs", rhs, F32, ndim=3)
    bsz, m, k = lhs.shape
    if rhs.shape[0] != bsz or rhs.shape[1] != k:
        raise ValueError(f"bmm: lhs {tuple(lhs.shape)} and rhs {tuple(rhs.shape)} are incompatible")
    n = rhs.shape[2]
    out = torch.empty((bsz, m, n), dtype=F32, device=lhs.device)
    ws = _workspace(workspace, workspace_size(_lib.OP_BMM_F32, bsz, m, k, n), lhs.device)
    _lib.call("kda_bmm_f32", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), bsz, m, k, n,
              ws.data_ptr(), ws.numel(), _stream(lhs))
    return out


def bmm_softmax(lhs: torch.Tensor, rhs: torch.Tensor,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = softmax(lhs @ rhs, axis=2) (max-shifted), lhs (B, M, K), rhs (B, K, N), fp32.

    K <= 64, N a multiple of 64.  One fused kernel: online row statistics, then
    the scores are recomputed and the probabilities written once.  Each lhs row
    and each 64-column rhs tile is scaled by a power of two and split into two
    fp16 limbs; the scores are three fp16 MFMA products.
    Reference: workspaces/bmm_softmax/runs/bmm_softmax_v4.py:10-181, forward
    workspaces/bmm_softmax/docs/draft-phase1.md:14-23.
    """
    _same_dtype(("lhs", lhs), ("rhs", rhs))
    _check("lhs", lhs, F32, ndim=3)
    _check("rhs", rhs, F32, ndim=3)
    bsz, m, k = lhs.shape
    if rhs.shape[0] != bsz or rhs.shape[1] != k:
        raise ValueError(f"bmm_softmax: lhs {tuple(lhs.shape)} and rhs {tuple(rhs.shape)} are incompatible")
    n = rhs.shape[2]
    out = torch.empty((bsz, m, n), dtype=F32, device=lhs.device)
    ws = _workspace(workspace, workspace_size(_lib.OP_BMM_SOFTMAX_F32, bsz, m, k, n), lhs.device)
    _lib.call("kda_bmm_softmax_f32", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), bsz, m, k, n,
              ws.data_ptr(), ws.numel(), _stream(lhs))
    return out


def lora(x: torch.Tensor, w: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
         workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = x @ w + (x @ a) @ b, x (M, K), w (K, N), a (K, R), b (R, N), fp32.

    Reference: workspaces/lora/runs/lora_v3_bf16_split.py:10-64, forward
    workspaces/lora/runs/offline_lora_bf16_split_sim.py:175-180.  Both terms
    accumulate in one GEMM (six K-segments).
    """
    _same_dtype(("x", x), ("w", w), ("a", a), ("b", b))
    for name, t in (("x", x), ("w", w), ("a", a), ("b", b)):
        _check(name, t, F32, ndim=2)
    m, k, n = _gemm_dims("x", x, "w", w)
    r = a.shape[1]
    if tuple(a.shape) != (k, r) or tuple(b.shape) != (r, n):
        raise ValueError(f"lora: a must be {(k, r)} and b {(r, n)}, got {tuple(a.shape)}, {tuple(b.shape)}")
    out = torch.empty((m, n), dtype=F32, device=x.device)
    ws = _workspace(workspace, workspace_size(_lib.OP_LORA_F32, 1, m, k, n, r), x.device)
    _lib.call("kda_lora_f32", x.data_ptr(), w.data_ptr(), a.data_ptr(), b.data_ptr(), out.data_ptr(),
              m, k, n, r, ws.data_ptr(), ws.numel(), _stream(x))
    return out


def rmsnorm_matmul(x: torch.Tensor, w: torch.Tensor, gamma: Optional[torch.Tensor] = None,
                   eps: float = 0.0, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = (x * rsqrt(mean_k(x^2) + eps) * gamma) @ w, x (M, K), w (K, N).

    bf16: gamma (K,) or None; a streaming pre-pass writes the per-row 1/rms and
    bf16(x * gamma), the GEMM applies 1/rms in its epilogue; bf16 output.
    fp32: the NKIBench forward ``x / sqrt(sum(x^2 / K)) @ w`` (no gain, no eps;
    gamma must be None and eps 0); fp32 output.
    Reference: workspaces/rmsnorm_matmul/runs/rmsnorm_matmul_v1.py:10-138 (forward
    workspaces/rmsnorm_matmul/runs/offline_bf16_split_sim.py:83-93); gain and eps
    as in workspaces/add_rmsnorm_matmul/runs/offline_bf16_split_sim.py:97-106.
    """
    dt = _same_dtype(("x", x), ("w", w))
    m, k, n = _gemm_dims("x", x, "w", w)
    out = torch.empty((m, n), dtype=dt, device=x.device)
    if dt == F32:
        if gamma is not None or eps != 0.0:
            raise ValueError("rmsnorm_matmul: the fp32 path is the NKIBench forward (no gamma, eps=0); "
                             "use add_rmsnorm_matmul for gain and eps")
        ws = _workspace(workspace, workspace_size(_lib.OP_RMSNORM_MATMUL_F32, 1, m, k, n), x.device)
        _lib.call("kda_rmsnorm_matmul_f32", x.data_ptr(), w.data_ptr(), out.data_ptr(), m, k, n,
                  ws.data_ptr(), ws.numel(), _stream(x))
        return out
    if gamma is None:
        gamma = torch.ones(k, dtype=BF16, device=x.device)
    _check("gamma", gamma, BF16, shape=(k,))
    _same_device(x, gamma)
    ws = _workspace(workspace, workspace_size(_lib.OP_RMSNORM_MATMUL_BF16, 1, m, k, n), x.device)
    _lib.call("kda_rmsnorm_matmul_bf16", x.data_ptr(), gamma.data_ptr(), w.data_ptr(),
              out.data_ptr(), m, k, n, float(eps), ws.data_ptr(), ws.numel(), _stream(x))
    return out


def rmsnorm_matmul_workspace_size(m: int, k: int) -> int:
    """Bytes of workspace the bf16 rmsnorm_matmul needs for an (m, k) x."""
    return workspace_size(_lib.OP_RMSNORM_MATMUL_BF16, 1, m, k, 0)


def add_rmsnorm_matmul(x: torch.Tensor, w: torch.Tensor, eps: float, z: torch.Tensor,
                       g: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x + z; out = (y / sqrt(sum(y^2 / K) + eps) * g) @ w.

    x, z (M, K), w (K, N), g (K,), all fp32 or all bf16 (output in the same dtype).
    fp32: the reference operator (three-product bf16 split).  bf16: y is summed in
    fp32, a pre-pass writes bf16(y * g) and 1/rms, the GEMM applies 1/rms in its
    epilogue.  Argument order of forward(x, w, eps, z, g)
    (workspaces/add_rmsnorm_matmul/docs/draft-phase1.md:10-24; kernel
    workspaces/add_rmsnorm_matmul/runs/add_rmsnorm_matmul_v1.py:8-146).
    """
    dt = _same_dtype(("x", x), ("w", w), ("z", z), ("g", g))
    _check("x", x, dt, ndim=2)
    m, k, n = _gemm_dims("x", x, "w", w)
    _check("z", z, dt, shape=(m, k))
    _check("g", g, dt, shape=(k,))
    out = torch.empty((m, n), dtype=dt, device=x.device)
    op, fn = ((_lib.OP_ADD_RMSNORM_MATMUL_F32, "kda_add_rmsnorm_matmul_f32") if dt == F32 else
              (_lib.OP_ADD_RMSNORM_MATMUL_BF16, "kda_add_rmsnorm_matmul_bf16"))
    ws = _workspace(workspace, workspace_size(op, 1, m, k, n), x.device)
    _lib.call(fn, x.data_ptr(), w.data_ptr(), float(eps), z.data_ptr(), g.data_ptr(),
              out.data_ptr(), m, k, n, ws.data_ptr(), ws.numel(), _stream(x))
    return out


def matmul_add_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, z: torch.Tensor,
                       g: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x @ w + z; out = y * g / sqrt(mean_n(y^2) + eps).

    x (M, K), w (K, N), z (M, N), g (N,), all fp32 or all bf16 (output in the same
    dtype).  The GEMM epilogue adds z and writes per-row partial sums of y^2 (from
    the fp32 accumulators); a row kernel applies the norm in place (bf16: y is
    rounded to bf16 once before that scaling).  Argument order of
    forward(x, w, eps, z, g) (workspaces/matmul_add_rmsnorm/docs/draft-phase1.md:10-22;
    kernel workspaces/matmul_add_rmsnorm/runs/matmul_add_rmsnorm_v2_bf16_split.py:8-212).
    """
    dt = _same_dtype(("x", x), ("w", w), ("z", z), ("g", g))
    _check("x", x, dt, ndim=2)
    m, k, n = _gemm_dims("x", x, "w", w)
    _check("z", z, dt, shape=(m, n))
    _check("g", g, dt, shape=(n,))
    out = torch.empty((m, n), dtype=dt, device=x.device)
    op, fn = ((_lib.OP_MATMUL_ADD_RMSNORM_F32, "kda_matmul_add_rmsnorm_f32") if dt == F32 else
              (_lib.OP_MATMUL_ADD_RMSNORM_BF16, "kda_matmul_add_rmsnorm_bf16"))
    ws = _workspace(workspace, workspace_size(op, 1, m, k, n), x.device)
    _lib.call(fn, x.data_ptr(), w.data_ptr(), float(eps), z.data_ptr(), g.data_ptr(),
              out.data_ptr(), m, k, n, ws.data_ptr(), ws.numel(), _stream(x))
    return out


def swiglu(x: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor, w_gate: torch.Tensor,
           h_workspace: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = (silu(x @ w_gate) * (x @ w_up)) @ w_down.

    x (M, K), w_up/w_gate (K, F), w_down (F, K); argument order of the reference
    forward(x, w_up, w_down, w_gate) (workspaces/swiglu/docs/draft-phase1.md:11-17,
    kernel in workspaces/swiglu/runs/swiglu_v1.py:38-146).  bf16: the gated
    activation h (M, F) is produced by one fused dual-GEMM kernel (gate and up
    share each x tile; silu(gate)*up in the epilogue) and consumed by the down
    GEMM; ``h_workspace`` optionally supplies h's (M, F) bf16 buffer and
    ``workspace`` the down GEMM's split-K partials (KDA_OP_SWIGLU_BF16 bytes).
    fp32: the same two kernels on split operands, h in fp32 (``workspace``).
    """
    dt = _same_dtype(("x", x), ("w_up", w_up), ("w_down", w_down), ("w_gate", w_gate))
    for name, t in (("w_up", w_up), ("w_down", w_down), ("w_gate", w_gate)):
        _check(name, t, dt, ndim=2)
    m, k, f = _gemm_dims("x", x, "w_up", w_up)
    if tuple(w_gate.shape) != (k, f) or tuple(w_down.shape) != (f, k):
        raise ValueError(f"swiglu: w_gate must be {(k, f)} and w_down {(f, k)}, got "
                         f"{tuple(w_gate.shape)}, {tuple(w_down.shape)}")
    out = torch.empty((m, k), dtype=dt, device=x.device)
    if dt == F32:
        ws = _workspace(workspace, workspace_size(_lib.OP_SWIGLU_F32, 1, m, k, f), x.device)
        _lib.call("kda_swiglu_f32", x.data_ptr(), w_up.data_ptr(), w_down.data_ptr(), w_gate.data_ptr(),
                  out.data_ptr(), m, k, f, ws.data_ptr(), ws.numel(), _stream(x))
        return out
    if h_workspace is None:
        h_workspace = torch.empty((m, f), dtype=BF16, device=x.device)
    _check("h_workspace", h_workspace, BF16, shape=(m, f))
    ws = _workspace(workspace, workspace_size(_lib.OP_SWIGLU_BF16, 1, m, k, f), x.device)
    _lib.call("kda_swiglu_bf16", x.data_ptr(), w_up.data_ptr(), w_down.data_ptr(), w_gate.data_ptr(),
              h_workspace.data_ptr(), out.data_ptr(), m, k, f, ws.data_ptr(), ws.numel(), _stream(x))
    return out


# ----------------------------------------------------------------- selective scan

def mamba(delta: torch.Tensor, u: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
          c: torch.Tensor) -> torch.Tensor:
    """Selective scan, fp32: delta, u (C, M); a (C, S); b, c (S, M) -> out (C, M), S <= 16.

    ``dA = exp(delta*a); dBu = delta*b*u; h = dA*h + dBu; out = sum_s c*h`` over M
    (workspaces/mamba/docs/draft-phase1.md:24-30; kernel(delta, u, a, b, c) of
    workspaces/mamba/runs/mamba_v4_s4unroll.py:7-117), evaluated as a chunked
    parallel scan: 8-step chunks folded into (prod dA, h) pairs, scanned across the
    lanes of a wave in fp64, then re-run from their entry states.  exp is numpy's
    float32 exp bit for bit; the states are summed in order s = 0..S-1.  Within
    ~2e-6 relative-L2 of the sequential numpy evaluation (not bit-identical: the
    entry state of each chunk is rounded once to fp32).
    """
    for name, t in (("delta", delta), ("u", u), ("a", a), ("b", b), ("c", c)):
        _check(name, t, F32, ndim=2)
    _same_device(delta, u, a, b, c)
    ch, m = delta.shape
    s = a.shape[1]
    if tuple(u.shape) != (ch, m) or tuple(a.shape) != (ch, s) or tuple(b.shape) != (s, m) \
            or tuple(c.shape) != (s, m):
        raise ValueError(f"mamba: inconsistent shapes delta {tuple(delta.shape)}, u {tuple(u.shape)}, "
                         f"a {tuple(a.shape)}, b {tuple(b.shape)}, c {tuple(c.shape)}")
    out = torch.empty((ch, m), dtype=F32, device=delta.device)
    _lib.call("kda_mamba_f32", delta.data_ptr(), u.data_ptr(), a.data_ptr(), b.data_ptr(), c.data_ptr(),
              out.data_ptr(), ch, m, s, _stream(delta))
    return out


# ----------------------------------------------------------------- attention

def gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
        scale: Optional[float] = None, out_layout: str = "bshd",
        workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Grouped-query softmax attention: per query head h (kv head h // (Hq/Hkv)),
    ``softmax(q k^T * scale) v`` with an fp32 online softmax (flash style).

    bf16 q/k/v run on bf16 MFMA and return bf16; fp32 q/k/v (the reference's
    gqa_full case) run on a two-limb fp16 split with fp32-class accuracy and
    return fp32 (workspace: KDA_OP_GQA_F32 bytes, allocated when not given).
    Any Hq that is a multiple of Hkv; head dim 128.

    q (B, S, Hq, D), k/v (B, S, Hkv, D); scale defaults to 1/sqrt(D); causal masks
    keys after the query.  out_layout "bshd" returns (B, S, Hq, D); "bhsd" returns
    (B, Hq, S, D), the layout of the reference's gqa_full output
    (workspaces/gqa_full/docs/draft-phase1.md:41-43; forward in
    workspaces/gqa_full/runs/offline_score_bf16_split_sim.py:100-123).
    """
    _check("q", q, q.dtype, ndim=4)
    _check("k", k, q.dtype, ndim=4)
    _check("v", v, q.dtype, ndim=4)
    _same_device(q, k, v)
    bsz, s, hq, d = q.shape
    if tuple(k.shape) != tuple(v.shape) or k.shape[0] != bsz or k.shape[1] != s or k.shape[3] != d:
        raise ValueError(f"gqa: k/v shape {tuple(k.shape)}/{tuple(v.shape)} incompatible with q {tuple(q.shape)}")
    hkv = k.shape[2]
    if hq % hkv:
        raise ValueError(f"gqa: Hq={hq} is not a multiple of Hkv={hkv}")
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    if q.dtype not in (BF16, F32):
        raise ValueError(f"gqa: unsupported dtype {q.dtype}")
    if out_layout == "bshd":
        out = torch.empty((bsz, s, hq, d), dtype=q.dtype, device=q.device)
        strides = (s * hq * d, hq * d, d)
    elif out_layout == "bhsd":
        out = torch.empty((bsz, hq, s, d), dtype=q.dtype, device=q.device)
        strides = (hq * s * d, d, s * d)
    else:
        raise ValueError(f"gqa: out_layout must be 'bshd' or 'bhsd', got {out_layout!r}")
    if q.dtype == BF16:
        _lib.call("kda_gqa_fwd_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                  bsz, s, hq, hkv, d, sc, 1 if causal else 0, *strides, _stream(q))
        return out
    ws = _workspace(workspace, workspace_size(_lib.OP_GQA_F32, bsz, s, hq, hkv), q.device)
    _lib.call("kda_gqa_fwd_f32", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              bsz, s, hq, hkv, d, sc, 1 if causal else 0, *strides, ws.data_ptr(), ws.numel(),
              _stream(q))
    return out


def gqa_full(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The NKIBench gqa_full forward: non-causal attention with scale 1/sqrt(D),
    query head h reading kv head h // (Hq/Hkv), returned as (B, Hq, S, D).

    q (B, S, Hq, D), k/v (B, S, Hkv, D) natural layout; the output layout is the
    reference's ``ref[0, qh, n, d]`` (workspaces/gqa_full/docs/draft-phase1.md:41-43;
    forward in workspaces/gqa_full/runs/offline_score_bf16_split_sim.py:100-123).
    """
    return gqa(q, k, v, causal=False, scale=None, out_layout="bhsd", workspace=workspace)
