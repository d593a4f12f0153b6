"""Pins the numpy oracle against checks independent of its own formulas.

Each test fails on a plausible restatement mistake (dropped term, wrong sign or
index, transposed operand): library routines computed in float64 (torch CPU),
closed forms, invariants, brute force on tiny inputs, and the known answers the
reference's own files hold.  CPU only.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2, split_bf16x2, to_bf16_rne

T64 = torch.float64


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


# ---------------------------------------------------------------- bf16 helpers

def test_bf16_rne_reference_known_answers():
    # workspaces/matmul/runs/offline_bf16_split_sim.py:217-229
    assert to_bf16_rne(np.float32(1.0)) == np.float32(1.0)
    assert to_bf16_rne(np.float32(1.0 + 2.0 ** -8)) == np.float32(1.0)       # tie -> even
    assert to_bf16_rne(np.float32(1.0 + 3.0 * 2.0 ** -9)) == np.float32(1.0 + 2.0 ** -7)
    a = np.random.default_rng(0).normal(size=10000).astype(np.float32)
    hi, lo = split_bf16x2(a)
    assert rel_l2(hi + lo, a) < 3e-5


def test_bf16_rne_matches_torch_conversion():
    a = np.random.default_rng(1).normal(scale=10.0, size=100000).astype(np.float32)
    a[:4] = [0.0, -0.0, 3.0e38, -1.0e-40]
    want = torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(to_bf16_rne(a), want)


def test_rel_l2_definition():
    r = np.array([3.0, 4.0])
    assert rel_l2(r, r) == 0.0
    assert rel_l2(np.array([3.0, 5.0]), r) == pytest.approx(1.0 / 5.0)


# ---------------------------------------------------------------- elementwise

def test_silu_vs_torch_and_limits():
    x = oi.draw("silu", 0, dims=dict(M=64, N=96))["x"]
    assert rel_l2(oo.silu(x), F.silu(t64(x)).numpy()) < 1e-6
    edge = np.array([0.0, 30.0, -30.0, -100.0, 100.0], dtype=np.float32)
    y = oo.silu(edge)
    assert y[0] == 0.0 and y[1] == pytest.approx(30.0) and abs(y[2]) < 1e-11
    assert y[3] == 0.0 and y[4] == 100.0


def test_adamw_nkibench_reference_fold_kat():
    # The reference verified the folded algebra against its forward to 3.42e-8
    # (workspaces/adamw/docs/draft-phase1.md:99-105).
    d = oi.draw("adamw", 42, dims=dict(M=256, N=512))
    th, g, m, v = (d[k].astype(np.float64) for k in ("theta", "g", "m", "v"))
    folded = 0.99999 * th - 0.001 * (9 * m + g) / np.sqrt(999 * v + g * g)
    assert rel_l2(oo.adamw(**d), folded) < 1e-7


@pytest.mark.parametrize("step", [1, 10])
def test_adamw_step_vs_torch_optim(step):
    d = oi.draw("adamw_cfg", 3, dims=dict(N=4096))
    hp = dict(oi.ADAMW_CFG, step=step)
    p_ref = torch.nn.Parameter(t64(d["param"]).clone())
    opt = torch.optim.AdamW([p_ref], lr=hp["lr"], betas=(hp["beta1"], hp["beta2"]),
                            eps=hp["eps"], weight_decay=hp["weight_decay"])
    p_ref.grad = t64(d["grad"]).clone()
    opt.state[p_ref] = {"step": torch.tensor(float(step - 1), dtype=T64),
                        "exp_avg": t64(d["m"]).clone(), "exp_avg_sq": t64(d["v"]).clone()}
    opt.step()
    p, m, v = oo.adamw_step(d["param"], d["grad"], d["m"], d["v"], **hp)
    assert rel_l2(p, p_ref.detach().numpy()) < 1e-6
    assert rel_l2(m, opt.state[p_ref]["exp_avg"].numpy()) < 1e-6
    assert rel_l2(v, opt.state[p_ref]["exp_avg_sq"].numpy()) < 1e-6


def test_adamw_nkibench_is_step1_of_the_general_update():
    d = oi.draw("adamw", 5, dims=dict(M=32, N=64))
    p, _, _ = oo.adamw_step(d["theta"], d["g"], d["m"], d["v"], lr=1e-3, beta1=0.9,
                            beta2=0.999, eps=1e-8, weight_decay=1e-2, step=1)
    assert rel_l2(p, oo.adamw(**d)) < 1e-6


def test_adamw_zero_grad_and_moments_is_pure_decay():
    p0 = np.linspace(-1, 1, 101, dtype=np.float32)
    z = np.zeros_like(p0)
    p, m, v = oo.adamw_step(p0, z, z, z, lr=1e-2, weight_decay=0.1, step=7)
    np.testing.assert_allclose(p, p0 * np.float32(1 - 1e-3), rtol=1e-7)
    assert not m.any() and not v.any()


def test_rope_vs_complex_rotation():
    d = oi.draw("rope_single_freq_apply", 0, dims=dict(D=16, S=64))
    theta = np.random.default_rng(2).uniform(-3, 3, size=(8, 64))
    cos, sin = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    x = d["x_in"]
    out = oo.rope_single_freq_apply(x, cos, sin)
    z = (x[:8].astype(np.float64) + 1j * x[8:]) * (cos + 1j * sin.astype(np.float64))
    np.testing.assert_allclose(out[:8], z.real, atol=1e-5)
    np.testing.assert_allclose(out[8:], z.imag, atol=1e-5)
    # pure rotation preserves the norm of each (x0, x1) pair
    np.testing.assert_allclose(out[:8] ** 2 + out[8:] ** 2, x[:8] ** 2 + x[8:] ** 2, rtol=1e-5)


# ---------------------------------------------------------------- norms + GEMMs

def test_rmsnorm_matmul_vs_torch_rms_norm():
    d = oi.draw("rmsnorm_matmul", 0, dims=dict(M=48, K=64, N=40))
    want = F.rms_norm(t64(d["x"]), (64,), eps=0.0) @ t64(d["w"])
    assert rel_l2(oo.rmsnorm_matmul(**d), want.numpy()) < 1e-6
    # row scaling of x cancels inside the norm
    d2 = dict(d, x=d["x"] * np.float32(4.0))
    assert rel_l2(oo.rmsnorm_matmul(**d2), oo.rmsnorm_matmul(**d)) < 1e-6


def test_rmsnorm_matmul_gamma_vs_torch():
    d = oi.draw("rmsnorm_matmul_cfg", 0, dims=dict(M=32, K=128, N=48))
    want = F.rms_norm(t64(d["x"]), (128,), weight=t64(d["gamma"]), eps=d["eps"]) @ t64(d["w"])
    assert rel_l2(oo.rmsnorm_matmul_gamma(**d), want.numpy()) < 1e-6
    # the normalised rows have unit RMS before the gain
    x = t64(d["x"])
    xn = F.rms_norm(x, (128,), eps=0.0)
    np.testing.assert_allclose((xn ** 2).mean(-1).numpy(), 1.0, rtol=1e-10)


def test_add_rmsnorm_matmul_vs_torch():
    d = oi.draw("add_rmsnorm_matmul", 0, dims=dict(M=32, K=64, N=24))
    y = F.rms_norm(t64(d["x"]) + t64(d["z"]), (64,), weight=t64(d["g"]), eps=d["eps"])
    assert rel_l2(oo.add_rmsnorm_matmul(**d), (y @ t64(d["w"])).numpy()) < 1e-6


def test_matmul_add_rmsnorm_vs_torch():
    d = oi.draw("matmul_add_rmsnorm", 0, dims=dict(M=32, K=48, N=64))
    y = t64(d["x"]) @ t64(d["w"]) + t64(d["z"])
    want = F.rms_norm(y, (64,), weight=t64(d["g"]), eps=d["eps"])
    assert rel_l2(oo.matmul_add_rmsnorm(**d), want.numpy()) < 1e-6


def test_swiglu_vs_torch_and_argument_order():
    d = oi.draw("swiglu", 0, dims=dict(M=16, K=32, N=48))
    x, wu, wd, wg = (t64(d[k]) for k in ("x", "w_up", "w_down", "w_gate"))
    want = (F.silu(x @ wg) * (x @ wu)) @ wd
    assert rel_l2(oo.swiglu(**d), want.numpy()) < 1e-6
    swapped = oo.swiglu(d["x"], d["w_gate"], d["w_down"], d["w_up"])
    assert rel_l2(swapped, want.numpy()) > 0.1


def test_matmul_brute_force():
    d = oi.draw("matmul", 0, dims=dict(M=5, K=7, N=3))
    a, b = d["lhs"].astype(np.float64), d["rhs"].astype(np.float64)
    want = np.array([[sum(a[i, k] * b[k, j] for k in range(7)) for j in range(3)] for i in range(5)])
    assert rel_l2(oo.matmul(**d), want) < 1e-6


def test_transpose_matmul_einsum():
    d = oi.draw("transpose_matmul", 0, dims=dict(M=6, K=9, N=4))
    want = np.einsum("km,kn->mn", d["lhs"].astype(np.float64), d["rhs"].astype(np.float64))
    got = oo.transpose_matmul(**d)
    assert got.shape == (6, 4) and rel_l2(got, want) < 1e-6


def test_bmm_and_bmm_softmax():
    d = oi.draw("bmm", 0, dims=dict(B=3, M=8, K=4, N=10))
    want = np.stack([np.dot(d["lhs"][b].astype(np.float64), d["rhs"][b]) for b in range(3)])
    assert rel_l2(oo.bmm(**d), want) < 1e-6
    sm = oo.bmm_softmax(**d)
    np.testing.assert_allclose(sm.sum(-1), 1.0, rtol=1e-6)
    want_sm = torch.softmax(torch.bmm(t64(d["lhs"]), t64(d["rhs"])), dim=2).numpy()
    assert rel_l2(sm, want_sm) < 1e-6


def test_lora_associativity():
    d = oi.draw("lora", 0, dims=dict(M=12, K=16, N=20, R=4))
    x, w, a, b = (d[k].astype(np.float64) for k in ("x", "w", "a", "b"))
    assert rel_l2(oo.lora(**d), x @ (w + a @ b)) < 1e-6


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("causal", [False, True])
def test_gqa_vs_torch_sdpa(causal):
    d = oi.draw("gqa_cfg", 0, dims=dict(B=2, S=24, HQ=4, HKV=2, D=16))
    q, k, v = (t64(d[n]) for n in ("q", "k", "v"))
    kr = k.repeat_interleave(2, dim=2)
    vr = v.repeat_interleave(2, dim=2)
    want = F.scaled_dot_product_attention(q.transpose(1, 2), kr.transpose(1, 2),
                                          vr.transpose(1, 2), is_causal=causal).transpose(1, 2)
    got = oo.gqa(d["q"], d["k"], d["v"], causal=causal)
    assert got.shape == (2, 24, 4, 16)
    assert rel_l2(got, want.numpy()) < 1e-6
    if causal:
        # the first query sees only key 0
        np.testing.assert_allclose(got[:, 0, :, :], np.repeat(d["v"][:, 0], 2, axis=1), rtol=1e-6)
    # bhsd layout is a transpose of bshd; sampled heads match the full output
    bhsd = oo.gqa(d["q"], d["k"], d["v"], causal=causal, out_layout="bhsd")
    np.testing.assert_array_equal(bhsd, got.transpose(0, 2, 1, 3))
    sub = oo.gqa(d["q"], d["k"], d["v"], causal=causal, heads=[(1, 3), (0, 0)])
    np.testing.assert_array_equal(sub[0], got[1, :, 3]); np.testing.assert_array_equal(sub[1], got[0, :, 0])


# ---------------------------------------------------------------- mamba

def test_mamba_closed_form_tiny():
    d = oi.draw("mamba", 1, dims=dict(C=3, M=9, S=2))
    delta, u, a, b, c = (d[k].astype(np.float64) for k in ("delta", "u", "a", "b", "c"))
    C, M = delta.shape
    S = a.shape[1]
    want = np.zeros((C, M))
    for ch in range(C):
        for s in range(S):
            dA = np.exp(delta[ch] * a[ch, s])
            dBu = delta[ch] * b[s] * u[ch]
            for i in range(M):
                st = sum(np.prod(dA[j + 1:i + 1]) * dBu[j] for j in range(i + 1))
                want[ch, i] += c[s, i] * st
    assert rel_l2(oo.mamba(**d), want) < 1e-6


def test_mamba_state_sum_order():
    """The oracle sums the 16 states in sequence (s = 0..15), as numpy reduces axis 1
    of the reference's (C, S, M) array.  An explicit s-loop gives the same bits; a
    pairwise sum over a contiguous S axis (numpy's order for axis=-1) agrees to ~1e-7
    but not bit for bit, so a bit-exact comparison is only valid in one order."""
    d = oi.draw("mamba", 42, dims=dict(C=16, M=512, S=16))
    out = oo.mamba(**d)
    delta, u, a, b, c = (d[k] for k in ("delta", "u", "a", "b", "c"))
    F = np.float32
    state = np.zeros((16, 16), dtype=F)
    seq = np.empty((16, 512), dtype=F)
    pair = np.empty((16, 512), dtype=F)
    for i in range(512):
        dm = delta[:, i:i + 1]
        state = (np.exp(dm * a).astype(F) * state + (dm * b[None, :, i]) * u[:, i:i + 1]).astype(F)
        prod = state * c[None, :, i]
        acc = prod[:, 0].copy()
        for s in range(1, 16):
            acc = acc + prod[:, s]
        seq[:, i] = acc
        pair[:, i] = np.sum(prod, axis=1)          # contiguous axis: pairwise blocks
    np.testing.assert_array_equal(out, seq)
    assert (out != pair).sum() > 100
    assert rel_l2(pair, out) < 1e-6


def test_mamba_reference_known_answer_seed42():
    # workspaces/mamba/docs/draft-phase1.md:93-96: ||out|| ~ 2.055, max|out| ~ 0.0127
    out = oo.mamba(**oi.draw("mamba", 42))
    assert float(np.linalg.norm(out)) == pytest.approx(2.055, abs=5e-4)
    assert float(np.abs(out).max()) == pytest.approx(0.0127, abs=5e-5)


# ---------------------------------------------------------------- draws

def test_draws_differ_per_seed_and_are_reproducible():
    a = oi.draw("matmul", 0, dims=dict(M=4, K=4, N=4))
    b = oi.draw("matmul", 21, dims=dict(M=4, K=4, N=4))
    c = oi.draw("matmul", 0, dims=dict(M=4, K=4, N=4))
    assert not np.array_equal(a["lhs"], b["lhs"])
    np.testing.assert_array_equal(a["lhs"], c["lhs"])


def test_bf16_configs_are_bf16_valued():
    d = oi.draw("rmsnorm_matmul_cfg", 0, dims=dict(M=8, K=16, N=8))
    for k in ("x", "gamma", "w"):
        np.testing.assert_array_equal(d[k], to_bf16_rne(d[k]))


def test_every_oracle_function_declares_its_pin():
    for name in oo.PINNED_BY:
        assert callable(getattr(oo, name)), name
