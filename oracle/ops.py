"""numpy restatement of each operator's reference forward() -- oracle.

Test infrastructure only (see oracle/__init__.py).  Every function computes in
float32 (as the reference's numpy forward does) unless stated, in the
reference's operation order, and cites the file:line it follows.  Inputs may be
any float array; bf16 configurations pass bf16-valued float32 arrays.

PINNED_BY records, per function, the independent checks in tests/test_oracle.py
that would fail on a dropped term, a wrong sign/index or a transposed operand.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32

PINNED_BY = {
    "silu": "torch.nn.functional.silu (float64); silu(0)=0, silu(x)->x for x>>0, ->0 for x<<0",
    "adamw": "reference KAT: folded form 0.99999*th - 0.001(9m+g)/sqrt(999v+g^2) within 3.42e-8 "
             "(workspaces/adamw/docs/draft-phase1.md:99-105); torch.optim.AdamW step 1",
    "adamw_step": "torch.optim.AdamW with primed state (step 9 -> 10), float32 and float64; "
                  "g=m=v=0 reduces to pure decay",
    "rope_single_freq_apply": "complex multiply (x0 + i x1)(cos + i sin); norm preserved when "
                              "cos^2+sin^2=1",
    "rmsnorm_matmul": "torch.nn.functional.rms_norm then matmul (float64); unit-RMS invariant; "
                      "row scaling of x leaves output unchanged",
    "rmsnorm_matmul_gamma": "torch.nn.functional.rms_norm(weight=gamma, eps) @ W (float64)",
    "add_rmsnorm_matmul": "torch rms_norm(x+z, weight=g, eps) @ w (float64)",
    "matmul_add_rmsnorm": "torch rms_norm(x@w+z, weight=g, eps) (float64)",
    "swiglu": "torch F.silu(x@Wg)*(x@Wu)@Wd (float64); argument order (x, w_up, w_down, w_gate) "
              "checked by swapping w_up/w_gate changes the result",
    "matmul": "brute-force triple loop on tiny shapes (float64)",
    "transpose_matmul": "einsum('km,kn->mn') on tiny shapes (float64)",
    "bmm": "per-batch loop of np.dot (float64)",
    "bmm_softmax": "torch.softmax(torch.bmm) (float64); rows sum to 1",
    "lora": "x@(w + a@b) (float64) -- associativity of the low-rank update",
    "gqa": "torch scaled_dot_product_attention with kv heads repeated (float64); causal row 0 == v[0]",
    "mamba": "O(M^2) closed form state_i = sum_j prod_{j<k<=i} dA_k * dBu_j (float64) on tiny "
             "shapes; reference KAT ||out||~2.055, max|out|~0.0127 at seed 42 "
             "(workspaces/mamba/docs/draft-phase1.md:93-96); the state sum is sequential in s "
             "(bit-equal to an explicit s-loop, and differs in the last bits from a pairwise sum)",
}


def _f32(a):
    return np.asarray(a, dtype=F32)


# ----------------------------------------------------------------- elementwise

def silu(x):
    """y = x / (1 + exp(-x)) (prompts/_gen_prompts.py:25;
    workspaces/swiglu/runs/offline_bf16_split_sim.py:87-89)."""
    x = _f32(x)
    with np.errstate(over="ignore"):
        return (x / (F32(1.0) + np.exp(-x))).astype(F32)


def adamw(theta, g, m, v):
    """NKIBench AdamW forward, returns new theta only
    (workspaces/adamw/docs/draft-phase1.md:20-26)."""
    theta, g, m, v = map(_f32, (theta, g, m, v))
    theta_t = theta - F32(1e-5) * theta
    m_t = F32(0.9) * m + F32(0.1) * g
    v_t = F32(0.999) * v + F32(0.001) * g * g
    v_hat = v_t * F32(1000)
    return (theta_t - F32(0.01) * m_t / (np.sqrt(v_hat) + F32(1e-8))).astype(F32)


def adamw_step(param, grad, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
               weight_decay=1e-2, step=1):
    """Decoupled-weight-decay Adam step at `step` (torch.optim.AdamW algorithm, the
    update the NKIBench forward fixes at step 1: workspaces/adamw/docs/draft-phase1.md:20-26).
    Returns (param', m', v') as new float32 arrays."""
    p, g, m, v = map(_f32, (param, grad, m, v))
    p = p * F32(1.0 - lr * weight_decay)
    m = F32(beta1) * m + F32(1.0 - beta1) * g
    v = F32(beta2) * v + F32(1.0 - beta2) * (g * g)
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    step_size = F32(lr / bc1)
    denom = np.sqrt(v) / F32(math.sqrt(bc2)) + F32(eps)
    p = p - step_size * (m / denom)
    return p.astype(F32), m.astype(F32), v.astype(F32)


def rope_single_freq_apply(x_in, cos, sin):
    """Half-split RoPE along axis 0
    (workspaces/rope_single_freq_apply/docs/draft-phase1.md:18-27)."""
    x_in, cos, sin = map(_f32, (x_in, cos, sin))
    half = x_in.shape[0] // 2
    x0, x1 = x_in[:half], x_in[half:]
    out0 = x0 * cos - x1 * sin
    out1 = x0 * sin + x1 * cos
    return np.concatenate([out0, out1], axis=0).astype(F32)


# ----------------------------------------------------------------- norms + GEMMs

def rmsnorm_matmul(x, w):
    """NKIBench rmsnorm_matmul: x / sqrt(sum(x^2 / K)) @ w, no eps, no gain
    (workspaces/rmsnorm_matmul/runs/offline_bf16_split_sim.py:83-93)."""
    x, w = _f32(x), _f32(w)
    k = x.shape[1]
    squared = np.square(x)
    scaled = np.divide(squared, F32(k))
    rms_sum = np.sum(scaled, axis=1, keepdims=True)
    rms = np.sqrt(rms_sum)
    normalized = np.divide(x, rms)
    return np.matmul(normalized, w).astype(F32)


def rmsnorm_matmul_gamma(x, gamma, w, eps):
    """RMSNorm with gain and eps, then GEMM: (x * rsqrt(mean(x^2) + eps) * gamma) @ W.
    Same norm as workspaces/add_rmsnorm_matmul/runs/offline_bf16_split_sim.py:97-106
    without the residual add."""
    x, gamma, w = _f32(x), _f32(gamma), _f32(w)
    k = x.shape[1]
    t = np.sum(np.divide(np.square(x), F32(k)), axis=-1, keepdims=True)
    t = (t + F32(eps)).astype(F32)
    y = x / np.sqrt(t)
    y = y * gamma
    return np.matmul(y, w).astype(F32)


def add_rmsnorm_matmul(x, w, eps, z, g):
    """(x+z) -> RMSNorm over K (eps after mean) * g -> @ w
    (workspaces/add_rmsnorm_matmul/runs/offline_bf16_split_sim.py:97-106)."""
    x, w, z, g = map(_f32, (x, w, z, g))
    k = x.shape[1]
    y = (x + z).astype(F32)
    t = np.square(y)
    t = np.divide(t, F32(k))
    t = np.sum(t, axis=-1, keepdims=True)
    t = (t + F32(eps)).astype(F32)
    y = y / np.sqrt(t)
    y = y * g
    return np.matmul(y, w).astype(F32)


def matmul_add_rmsnorm(x, w, eps, z, g):
    """y = x@w + z; out = y * g / sqrt(mean_N(y^2) + eps)
    (workspaces/matmul_add_rmsnorm/runs/offline_bf16_split_sim.py:111-115)."""
    x, w, z, g = map(_f32, (x, w, z, g))
    y = (np.matmul(x, w) + z).astype(F32)
    rms = np.sqrt(np.mean(np.square(y), axis=-1, keepdims=True) + F32(eps)).astype(F32)
    return (y * g / rms).astype(F32)


def swiglu(x, w_up, w_down, w_gate):
    """(silu(x@w_gate) * (x@w_up)) @ w_down, argument order (x, w_up, w_down, w_gate)
    (workspaces/swiglu/runs/offline_bf16_split_sim.py:92-97)."""
    x, w_up, w_down, w_gate = map(_f32, (x, w_up, w_down, w_gate))
    up = np.matmul(x, w_up)
    gate = np.matmul(x, w_gate)
    h = silu(gate) * up
    return np.matmul(h, w_down).astype(F32)


def matmul(lhs, rhs):
    """lhs @ rhs (workspaces/matmul/runs/offline_bf16_split_sim.py:137-139 fp32 control)."""
    return np.matmul(_f32(lhs), _f32(rhs)).astype(F32)


def transpose_matmul(lhs, rhs):
    """transpose(lhs) @ rhs with lhs (K, M), rhs (K, N)
    (workspaces/transpose_matmul/runs/offline_bf16_split_sim.py:101-104)."""
    lhs_t = np.transpose(_f32(lhs), axes=(1, 0))
    return np.matmul(lhs_t, _f32(rhs)).astype(F32)


def bmm(lhs, rhs):
    """out[b] = lhs[b] @ rhs[b] (workspaces/bmm/docs/draft-phase1.md:3-5)."""
    return np.matmul(_f32(lhs), _f32(rhs)).astype(F32)


def bmm_softmax(lhs, rhs):
    """softmax(lhs @ rhs, axis=2), max-shifted
    (workspaces/bmm_softmax/docs/draft-phase1.md:14-23)."""
    x = np.matmul(_f32(lhs), _f32(rhs)).astype(F32)
    max_x = np.max(x, axis=2, keepdims=True)
    exp_x = np.exp(x - max_x)
    sum_exp = np.sum(exp_x, axis=2, keepdims=True)
    return (exp_x / sum_exp).astype(F32)


def lora(x, w, a, b):
    """x@w + (x@a)@b (workspaces/lora/runs/offline_lora_bf16_split_sim.py:175-180)."""
    x, w, a, b = map(_f32, (x, w, a, b))
    return (np.matmul(x, w) + np.matmul(np.matmul(x, a), b)).astype(F32)


# ----------------------------------------------------------------- attention

def gqa(q, k, v, causal=False, scale=None, heads=None, out_layout="bshd"):
    """Grouped-query softmax attention, fp32 softmax, max-shifted.

    q (B, S, Hq, D), k/v (B, S, Hkv, D); query head h reads kv head h // (Hq/Hkv)
    (kv repeat, workspaces/gqa_full/runs/offline_score_bf16_split_sim.py:100-106);
    per head softmax(q k^T * scale) v with scale default 1/sqrt(D) applied to the
    scores before the max (:109-116).  causal masks keys j > i.

    heads: optional list of (b, h) pairs to compute; then returns an array
    (len(heads), S, D) instead of the full output (used for sampled checks).
    out_layout: "bshd" -> (B, S, Hq, D); "bhsd" -> (B, Hq, S, D) (the NKIBench
    gqa_full output, workspaces/gqa_full/docs/draft-phase1.md:41-43).
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    bsz, s, hq, d = q.shape
    hkv = k.shape[2]
    n_rep = hq // hkv
    sc = F32(1.0 / math.sqrt(d) if scale is None else scale)
    mask = None
    if causal:
        mask = np.triu(np.ones((s, s), dtype=bool), k=1)

    def one(b, h):
        kh = h // n_rep
        qh, kk, vv = q[b, :, h, :], k[b, :, kh, :], v[b, :, kh, :]
        sco = (np.matmul(qh, kk.T) * sc).astype(F32)
        if mask is not None:
            sco = np.where(mask, F32(-np.inf), sco)
        sco = sco - np.max(sco, axis=-1, keepdims=True)
        e = np.exp(sco).astype(F32)
        a = (e / np.sum(e, axis=-1, keepdims=True)).astype(F32)
        return np.matmul(a, vv).astype(F32)

    if heads is not None:
        return np.stack([one(b, h) for b, h in heads], axis=0)
    out = np.empty((bsz, s, hq, d), dtype=F32)
    for b in range(bsz):
        for h in range(hq):
            out[b, :, h, :] = one(b, h)
    if out_layout == "bhsd":
        return np.ascontiguousarray(out.transpose(0, 2, 1, 3))
    return out


# ----------------------------------------------------------------- selective scan

def mamba(delta, u, a, b, c):
    """Selective scan, sequential over M, in the operation order of the reference's
    numpy forward (workspaces/mamba/docs/draft-phase1.md:24-30):
      deltaA   = exp(delta[:, None, :] * a[:, :, None])           (C, S, M)
      deltaB_u = delta[:, None, :] * b[None, :, :] * u[:, None, :] (C, S, M)
      state_i  = deltaA[..., i] * state_{i-1} + deltaB_u[..., i]   (state_{-1} = 0)
      out      = sum over axis 1 (S) of c[None] * scan_res          (C, M)
    numpy reduces axis 1 of a C-ordered (C, S, M) array one S-row at a time
    (s = 0, 1, ..., S-1), so the state sum is sequential in s.
    delta, u: (C, M); a: (C, S); b, c: (S, M) -> out (C, M), fp32."""
    delta, u, a, b, c = map(_f32, (delta, u, a, b, c))
    ch, m_len = delta.shape
    s_len = a.shape[1]
    delta_a = np.exp(delta[:, None, :] * a[:, :, None]).astype(F32)
    delta_bu = (delta[:, None, :] * b[None, :, :] * u[:, None, :]).astype(F32)
    scan_res = np.empty((ch, s_len, m_len), dtype=F32)
    state = np.zeros((ch, s_len), dtype=F32)
    for i in range(m_len):
        state = delta_a[..., i] * state + delta_bu[..., i]
        scan_res[..., i] = state
    return np.sum(c[None, :, :] * scan_res, axis=1).astype(F32)
