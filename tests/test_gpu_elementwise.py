"""GPU parity: SiLU, AdamW (NKIBench forward and in-place step), RoPE vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, elementwise_in_slices, to_dev, to_host
from kda import ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2

pytestmark = pytest.mark.gpu

FP32_GATE = 1e-5


@pytest.mark.parametrize("case", ["silu", "silu_cfg"])
def test_silu_full_size_all_seeds(dev, case):
    for s in SEEDS:
        x = oi.draw(case, s)["x"]
        got = to_host(ops.silu(to_dev(x, dev)))
        err = rel_l2(got, oo.silu(x))
        print(f"{case} seed={s} rel_l2={err:.3e}", flush=True)
        assert err < FP32_GATE


@pytest.mark.parametrize("n", [1, 3, 5, 1023, 4097, 262145])
def test_silu_ragged_and_misaligned(dev, n):
    x = np.random.default_rng(n).normal(scale=4.0, size=n + 1).astype(np.float32)
    xt = to_dev(x, dev)
    got = to_host(ops.silu(xt[1:]))            # offset 4 bytes: scalar path
    assert rel_l2(got, oo.silu(x[1:])) < FP32_GATE
    got = to_host(ops.silu(xt[:n]))            # aligned vector path + tail
    assert rel_l2(got, oo.silu(x[:n])) < FP32_GATE


@pytest.mark.parametrize("n", [4, 1020, 1028, 4096 * 257])
def test_silu_writes_nothing_past_its_output(dev, n):
    """The vector path stores through per-workgroup buffer windows: an output that
    ends inside a workgroup's range (n/4 not a multiple of 256) is written exactly,
    and the elements after it (and before it) stay as they were."""
    x = np.random.default_rng(n).normal(size=n).astype(np.float32)
    buf = torch.full((n + 64,), float("nan"), device=dev)
    out = buf[32:32 + n]                       # 128-byte aligned start, NaN guards both sides
    ops.silu(to_dev(x, dev), out=out)
    torch.cuda.synchronize(dev)
    assert rel_l2(to_host(out), oo.silu(x)) < FP32_GATE
    assert torch.isnan(buf[:32]).all() and torch.isnan(buf[32 + n:]).all()


def test_silu_extremes_and_empty(dev):
    x = np.array([0.0, -0.0, 88.0, -88.0, 100.0, -100.0, 1e-30, -1e30, 3.0, -3.0, 0.5, -0.5],
                 dtype=np.float32)
    got = to_host(ops.silu(to_dev(x, dev)))
    want = oo.silu(x)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)
    e = torch.empty(0, device=dev)
    assert ops.silu(e).numel() == 0


def test_adamw_nkibench_full_size_all_seeds(dev):
    for s in SEEDS:
        d = oi.draw("adamw", s)
        dd = {k: to_dev(v, dev) for k, v in d.items()}
        m0, v0 = dd["m"].clone(), dd["v"].clone()
        got = to_host(ops.adamw(**dd))
        err = rel_l2(got, oo.adamw(**d))
        print(f"adamw seed={s} rel_l2={err:.3e}", flush=True)
        assert err < FP32_GATE
        assert torch.equal(dd["m"], m0) and torch.equal(dd["v"], v0)


@pytest.mark.parametrize("seed", SEEDS)
def test_adamw_step_config_full_size(dev, seed):
    d = oi.draw("adamw_cfg", seed)
    dd = {k: to_dev(v, dev) for k, v in d.items()}
    ops.adamw_step_(dd["param"], dd["grad"], dd["m"], dd["v"], **oi.ADAMW_CFG)
    # the oracle is elementwise: evaluated on 1/16 slices in threads, same values
    p, m, v = elementwise_in_slices(
        lambda *a: oo.adamw_step(*a, **oi.ADAMW_CFG),
        [d["param"], d["grad"], d["m"], d["v"]], n_out=3)
    for name, got, want in (("param", dd["param"], p), ("m", dd["m"], m), ("v", dd["v"], v)):
        err = rel_l2(to_host(got), want)
        print(f"adamw_cfg seed={seed} {name} rel_l2={err:.3e}", flush=True)
        assert err < FP32_GATE


@pytest.mark.parametrize("n", [1, 7, 4099])
@pytest.mark.parametrize("step", [1, 10, 1000])
def test_adamw_step_ragged_sizes_and_steps(dev, n, step):
    d = oi.draw("adamw_cfg", n + step, dims=dict(N=n + 1))
    hp = dict(oi.ADAMW_CFG, step=step)
    for off in (0, 1):   # aligned vector path and misaligned scalar path
        dd = {k: to_dev(v, dev)[off:off + n] for k, v in d.items()}
        ops.adamw_step_(dd["param"], dd["grad"], dd["m"], dd["v"], **hp)
        p, m, v = oo.adamw_step(*(d[k][off:off + n] for k in ("param", "grad", "m", "v")), **hp)
        assert rel_l2(to_host(dd["param"]), p) < FP32_GATE
        assert rel_l2(to_host(dd["m"]), m) < FP32_GATE
        assert rel_l2(to_host(dd["v"]), v) < FP32_GATE


def test_rope_full_size_bit_exact(dev):
    for s in SEEDS:
        d = oi.draw("rope_single_freq_apply", s)
        got = to_host(ops.rope_single_freq_apply(*(to_dev(d[k], dev) for k in ("x_in", "cos", "sin"))))
        want = oo.rope_single_freq_apply(**d)
        print(f"rope seed={s} mismatches={(got != want).sum()}", flush=True)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dims", [dict(D=2, S=1), dict(D=128, S=6), dict(D=64, S=1001), dict(D=8, S=0)])
def test_rope_ragged(dev, dims):
    d = oi.draw("rope_single_freq_apply", 1, dims=dims)
    got = to_host(ops.rope_single_freq_apply(*(to_dev(d[k], dev) for k in ("x_in", "cos", "sin"))))
    np.testing.assert_array_equal(got, oo.rope_single_freq_apply(**d))
