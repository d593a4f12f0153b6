"""GPU parity: bf16 MFMA GEMMs (plain, RMSNorm-fused with and without a residual,
SwiGLU) vs the fp32 oracle.

Inputs are bf16 values; the oracle computes in fp32 on the same values.  Gate:
relative-L2 <= 1e-2 for bf16 operators (the kernels land near 1e-3: bf16
rounding of the output / of the gated activation)."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, to_dev, to_host
from kda import _lib, ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2, to_bf16_rne

pytestmark = pytest.mark.gpu
BF16_GATE = 1e-2
BF = torch.bfloat16


def _bf16_normal(rng, shape, std=1.0):
    return to_bf16_rne((rng.standard_normal(shape) * std).astype(np.float32))


@pytest.mark.parametrize("m,k,n", [(256, 64, 128), (512, 256, 384), (1, 8, 8), (37, 72, 40),
                                   (300, 200, 136), (1000, 520, 264)])
def test_matmul_bf16_shapes(dev, m, k, n):
    rng = np.random.default_rng(m * 7 + n)
    a, b = _bf16_normal(rng, (m, k)), _bf16_normal(rng, (k, n))
    got = to_host(ops.matmul(to_dev(a, dev, BF), to_dev(b, dev, BF)))
    err = rel_l2(got, oo.matmul(a, b))
    print(f"matmul_bf16 {m}x{k}x{n} rel_l2={err:.3e}", flush=True)
    assert err < 4e-3


def test_matmul_bf16_layout_identity(dev):
    # A = I picks rows of B exactly: catches any transposed / swizzled fragment.
    k = 256
    b = _bf16_normal(np.random.default_rng(0), (k, 384))
    got = to_host(ops.matmul(to_dev(np.eye(k, dtype=np.float32), dev, BF), to_dev(b, dev, BF)))
    np.testing.assert_array_equal(got, b)
    a = _bf16_normal(np.random.default_rng(1), (512, k))
    got = to_host(ops.matmul(to_dev(a, dev, BF), to_dev(np.eye(k, dtype=np.float32), dev, BF)))
    np.testing.assert_array_equal(got, a)


def test_rmsnorm_matmul_config_full_size_all_seeds(dev):
    for s in SEEDS:
        d = oi.draw("rmsnorm_matmul_cfg", s)
        got = ops.rmsnorm_matmul(to_dev(d["x"], dev, BF), to_dev(d["w"], dev, BF),
                                 gamma=to_dev(d["gamma"], dev, BF), eps=d["eps"])
        err = rel_l2(to_host(got), oo.rmsnorm_matmul_gamma(**d))
        print(f"rmsnorm_matmul_cfg seed={s} rel_l2={err:.3e}", flush=True)
        assert err < BF16_GATE


@pytest.mark.parametrize("dims", [dict(M=256, K=64, N=128), dict(M=77, K=136, N=56),
                                  dict(M=1, K=8, N=8), dict(M=513, K=1000, N=264),
                                  # K past what the norm pre-pass holds in registers (4096)
                                  dict(M=40, K=5000, N=72)])
def test_rmsnorm_matmul_ragged(dev, dims):
    d = oi.draw("rmsnorm_matmul_cfg", 3, dims=dims)
    got = ops.rmsnorm_matmul(to_dev(d["x"], dev, BF), to_dev(d["w"], dev, BF),
                             gamma=to_dev(d["gamma"], dev, BF), eps=d["eps"])
    err = rel_l2(to_host(got), oo.rmsnorm_matmul_gamma(**d))
    print(f"rmsnorm_matmul {dims} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


def test_rmsnorm_matmul_row_scale_invariance(dev):
    # scaling a row of x by a power of two leaves its output row unchanged (eps=0)
    d = oi.draw("rmsnorm_matmul_cfg", 4, dims=dict(M=256, K=512, N=256))
    x = d["x"].copy()
    x[::3] *= 8.0
    g = to_dev(d["gamma"], dev, BF)
    y0 = to_host(ops.rmsnorm_matmul(to_dev(d["x"], dev, BF), to_dev(d["w"], dev, BF), gamma=g))
    y1 = to_host(ops.rmsnorm_matmul(to_dev(x, dev, BF), to_dev(d["w"], dev, BF), gamma=g))
    np.testing.assert_array_equal(y0, y1)


def _residual_args(d, dev):
    return [to_dev(d["x"], dev, BF), to_dev(d["w"], dev, BF), d["eps"], to_dev(d["z"], dev, BF),
            to_dev(d["g"], dev, BF)]


@pytest.mark.parametrize("case,fn,ref", [
    ("add_rmsnorm_matmul_cfg", ops.add_rmsnorm_matmul, oo.add_rmsnorm_matmul),
    ("matmul_add_rmsnorm_cfg", ops.matmul_add_rmsnorm, oo.matmul_add_rmsnorm)])
def test_residual_rmsnorm_config_full_size_all_seeds(dev, case, fn, ref):
    # the fused residual variants at the RMSNorm->matmul shape (4096 x 4096 x 11008)
    for s in SEEDS:
        d = oi.draw(case, s)
        got = fn(*_residual_args(d, dev))
        assert got.dtype == BF
        err = rel_l2(to_host(got), ref(**d))
        print(f"{case} seed={s} rel_l2={err:.3e}", flush=True)
        assert err < BF16_GATE


RAGGED_RESIDUAL = [dict(M=256, K=64, N=128), dict(M=77, K=136, N=56), dict(M=1, K=8, N=8),
                   dict(M=513, K=1000, N=264), dict(M=300, K=200, N=1000),
                   # K past what the norm pre-pass holds in registers (4096)
                   dict(M=40, K=5000, N=72),
                   # enough 256 x 256 tiles to take the wide (64-column partial) path
                   dict(M=2048, K=256, N=8192)]


@pytest.mark.parametrize("dims", RAGGED_RESIDUAL)
@pytest.mark.parametrize("case,fn,ref", [
    ("add_rmsnorm_matmul_cfg", ops.add_rmsnorm_matmul, oo.add_rmsnorm_matmul),
    ("matmul_add_rmsnorm_cfg", ops.matmul_add_rmsnorm, oo.matmul_add_rmsnorm)])
def test_residual_rmsnorm_ragged(dev, case, fn, ref, dims):
    d = oi.draw(case, 6, dims=dims)
    err = rel_l2(to_host(fn(*_residual_args(d, dev))), ref(**d))
    print(f"{case} {dims} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


def test_add_rmsnorm_matmul_reduces_to_rmsnorm_matmul(dev):
    # z = 0: the same pre-pass arithmetic and GEMM as rmsnorm_matmul (bit for bit);
    # x and z swapped: the fp32 sum commutes (bit for bit)
    d = oi.draw("add_rmsnorm_matmul_cfg", 7, dims=dict(M=300, K=520, N=264))
    x, w, eps, z, g = _residual_args(d, dev)
    zero = torch.zeros_like(z)
    a = to_host(ops.add_rmsnorm_matmul(x, w, eps, zero, g))
    b = to_host(ops.rmsnorm_matmul(x, w, gamma=g, eps=eps))
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(to_host(ops.add_rmsnorm_matmul(x, w, eps, z, g)),
                                  to_host(ops.add_rmsnorm_matmul(z, w, eps, x, g)))


def test_matmul_add_rmsnorm_bf16_row_properties(dev):
    d = oi.draw("matmul_add_rmsnorm_cfg", 8, dims=dict(M=512, K=384, N=1032))
    x, w, _, z, g = _residual_args(d, dev)
    ones = torch.ones_like(g)
    # g = 1, eps = 0: every output row has unit mean square (up to bf16 rounding)
    out = to_host(ops.matmul_add_rmsnorm(x, w, 0.0, z, ones)).astype(np.float64)
    ms = np.mean(out * out, axis=1)
    assert np.max(np.abs(ms - 1.0)) < 1e-2, np.max(np.abs(ms - 1.0))
    # scaling a row of x and z by a power of two leaves its output row unchanged
    xs, zs = d["x"].copy(), d["z"].copy()
    xs[::5] *= 4.0
    zs[::5] *= 4.0
    y0 = to_host(ops.matmul_add_rmsnorm(x, w, 0.0, z, g))
    y1 = to_host(ops.matmul_add_rmsnorm(to_dev(xs, dev, BF), w, 0.0, to_dev(zs, dev, BF), g))
    np.testing.assert_array_equal(y0, y1)


def test_swiglu_config_full_size_all_seeds(dev):
    for s in SEEDS:
        d = oi.draw("swiglu_cfg", s)
        got = ops.swiglu(*(to_dev(d[k], dev, BF) for k in ("x", "w_up", "w_down", "w_gate")))
        err = rel_l2(to_host(got), oo.swiglu(**d))
        print(f"swiglu_cfg seed={s} rel_l2={err:.3e}", flush=True)
        assert err < BF16_GATE


def test_swiglu_config_without_split_k_workspace(dev):
    # a workspace too small for the split-K partials: the down GEMM runs unsplit
    d = oi.draw("swiglu_cfg", 1)
    args = [to_dev(d[k], dev, BF) for k in ("x", "w_up", "w_down", "w_gate")]
    tiny = torch.empty(16, dtype=torch.uint8, device=dev)
    got = to_host(ops.swiglu(*args, workspace=tiny))
    split = to_host(ops.swiglu(*args))
    want = oo.swiglu(**d)
    for name, out in (("unsplit", got), ("split", split)):
        err = rel_l2(out, want)
        print(f"swiglu_cfg {name} rel_l2={err:.3e}", flush=True)
        assert err < BF16_GATE
    # the two orders of the F sum differ by at most one bf16 rounding of the output
    assert rel_l2(got, split) < 2.0 ** -8


def test_swiglu_split_k_ragged_rows_dirty_workspace(dev):
    # M = 300 (a ragged second row of 256-row tiles), F = 17408: 272 gate/up tiles,
    # so on 256 CUs the last 1024 columns run as a round of 128x128 tiles; the
    # down GEMM's 14 tiles run with F split in two into fp32 partials.  The
    # workspace starts as 0xff bytes (nothing in it may be read before it is
    # written), and a second call on the same workspace gives the same bits.
    m, k, f = 300, 1792, 17408
    d = oi.draw("swiglu_cfg", 3, dims=dict(M=m, K=k, F=f))
    args = [to_dev(d[n], dev, BF) for n in ("x", "w_up", "w_down", "w_gate")]
    ws = torch.full((ops.workspace_size(_lib.OP_SWIGLU_BF16, 1, m, k, f),), 255,
                    dtype=torch.uint8, device=dev)
    first = ops.swiglu(*args, workspace=ws)
    second = ops.swiglu(*args, workspace=ws)
    err = rel_l2(to_host(first), oo.swiglu(**d))
    print(f"swiglu split-K M={m} K={k} F={f} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3
    assert torch.equal(first, second)


def test_swiglu_tail_down_launch_ragged_rows_dirty_workspace(dev):
    # M = 300, K = 1024, F = 16896: 264 gate/up tiles of 256x128 on 256 CUs, so the
    # last 512 columns (8 tiles, 4 per row tile) run in one launch with the down
    # GEMM's 8 tiles of 256x256: 8 workgroups compute a tail tile and then h's
    # first 7616 columns times w_down, parking the fp32 sums; 8 more compute the
    # remaining 9280 columns, waiting for the tail tiles of their row before its
    # last 512 columns and for the parked sums before the epilogue.  The second
    # row tile holds 44 rows.  The workspace starts as 0xff bytes (the flags are
    # cleared by the gate/up launch), a second call gives the same bits, and the
    # result matches the path without a workspace within one bf16 rounding.
    m, k, f = 300, 1024, 16896
    d = oi.draw("swiglu_cfg", 4, dims=dict(M=m, K=k, F=f))
    args = [to_dev(d[n], dev, BF) for n in ("x", "w_up", "w_down", "w_gate")]
    ws = torch.full((ops.workspace_size(_lib.OP_SWIGLU_BF16, 1, m, k, f),), 255,
                    dtype=torch.uint8, device=dev)
    first = ops.swiglu(*args, workspace=ws)
    second = ops.swiglu(*args, workspace=ws)
    unsplit = ops.swiglu(*args, workspace=torch.empty(16, dtype=torch.uint8, device=dev))
    err = rel_l2(to_host(first), oo.swiglu(**d))
    print(f"swiglu tail+down M={m} K={k} F={f} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3
    assert torch.equal(first, second)
    assert rel_l2(to_host(first), to_host(unsplit)) < 2.0 ** -8


@pytest.mark.parametrize("dims", [dict(M=256, K=128, F=64), dict(M=50, K=96, F=200),
                                  dict(M=300, K=264, F=136)])
def test_swiglu_ragged(dev, dims):
    d = oi.draw("swiglu_cfg", 5, dims=dims)
    got = ops.swiglu(*(to_dev(d[k], dev, BF) for k in ("x", "w_up", "w_down", "w_gate")))
    err = rel_l2(to_host(got), oo.swiglu(**d))
    print(f"swiglu {dims} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


# ---- launches of more than one round of tiles (more tiles than the device's 256
# CUs), with a partial last row (and column) of tiles.  Rows are independent and
# every tile is computed in the same k order, so the first 4096 rows of a 4300-row
# product (17 x 16 tiles of 256 x 256, the last row of tiles partial) must equal,
# bit for bit, the 4096-row product (16 x 16 tiles); K from two 32-deep k-tiles up.
MULTI_ROUND_K = [64, 96, 256]


@pytest.mark.parametrize("k", MULTI_ROUND_K)
def test_matmul_bf16_multi_round_rows_match_one_round(dev, k):
    rng = np.random.default_rng(k)
    a, b = _bf16_normal(rng, (4300, k)), _bf16_normal(rng, (k, 4096))
    ta, tb = to_dev(a, dev, BF), to_dev(b, dev, BF)
    big = ops.matmul(ta, tb)
    ref = ops.matmul(ta[:4096].contiguous(), tb)
    assert torch.equal(big[:4096], ref), f"K={k}: rows of the 4300-row product differ from the 4096-row one"
    err = rel_l2(to_host(big), oo.matmul(a, b))
    print(f"matmul_bf16 4300x{k}x4096 rel_l2={err:.3e}", flush=True)
    assert err < 4e-3


@pytest.mark.parametrize("k", MULTI_ROUND_K)
def test_rmsnorm_matmul_multi_round_rows_match_one_round(dev, k):
    d = oi.draw("rmsnorm_matmul_cfg", 8, dims=dict(M=4300, K=k, N=4096))
    x, w, g = to_dev(d["x"], dev, BF), to_dev(d["w"], dev, BF), to_dev(d["gamma"], dev, BF)
    big = ops.rmsnorm_matmul(x, w, gamma=g, eps=d["eps"])
    ref = ops.rmsnorm_matmul(x[:4096].contiguous(), w, gamma=g, eps=d["eps"])
    assert torch.equal(big[:4096], ref), f"K={k}: rows of the 4300-row product differ from the 4096-row one"
    err = rel_l2(to_host(big), oo.rmsnorm_matmul_gamma(**d))
    print(f"rmsnorm_matmul 4300x{k}x4096 rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


@pytest.mark.parametrize("dims", [dict(M=4100, K=128, N=4104), dict(M=4352, K=64, N=4360)])
def test_residual_rmsnorm_multi_round_ragged(dev, dims):
    """Both residual forms over more than one round of tiles, the last row and
    column of tiles partial."""
    for case, fn, ref in (("add_rmsnorm_matmul_cfg", ops.add_rmsnorm_matmul, oo.add_rmsnorm_matmul),
                          ("matmul_add_rmsnorm_cfg", ops.matmul_add_rmsnorm, oo.matmul_add_rmsnorm)):
        d = oi.draw(case, 9, dims=dims)
        err = rel_l2(to_host(fn(*_residual_args(d, dev))), ref(**d))
        print(f"{case} {dims} rel_l2={err:.3e}", flush=True)
        assert err < 5e-3


def test_swiglu_multi_round_gate_up(dev):
    """2100 rows, F = 4096: the gate/up launch has 9 x 32 = 288 tiles of 256 x 128
    (more than one round, the last row of tiles partial); the down GEMM is one round."""
    d = oi.draw("swiglu_cfg", 10, dims=dict(M=2100, K=1024, F=4096))
    got = ops.swiglu(*(to_dev(d[k], dev, BF) for k in ("x", "w_up", "w_down", "w_gate")))
    err = rel_l2(to_host(got), oo.swiglu(**d))
    print(f"swiglu 2100x1024x4096 rel_l2={err:.3e}", flush=True)
    assert err < 5e-3
