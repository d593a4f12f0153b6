"""GPU parity: fp32 grouped-query attention (NKIBench gqa_full: fp32 q/k/v, two
query heads per kv head) vs the oracle, through the two-limb fp16 path.

Gate: relative-L2 <= 1e-5 (fp32).  The NKIBench shape (B1 S4096 Hq16 Hkv8 D128,
non-causal, BHSD output) is computed whole; the oracle checks every head on
seed 0 and sampled heads on the other seeds.  Power-of-two rescalings of q
(with the inverse softmax scale) and of v must give bit-identical / exactly
rescaled outputs, since every operand is normalised by its own power of two
before the split."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, threaded_heads, to_dev, to_host
from kda import ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2

pytestmark = pytest.mark.gpu
GATE = 1e-5


def _qkv(d, dev):
    return [to_dev(d[k], dev) for k in ("q", "k", "v")]


@pytest.mark.parametrize("seed", SEEDS)
def test_gqa_f32_nkibench_shape_sampled_heads(dev, seed):
    d = oi.draw("gqa_full", seed)
    out = to_host(ops.gqa(*_qkv(d, dev), causal=False, out_layout="bhsd"))
    assert out.shape == (1, 16, 4096, 128)
    if seed == 0:
        heads = [(0, h) for h in range(16)]     # every head on one seed
    else:
        rng = np.random.default_rng(seed)
        heads = [(0, 0), (0, 15)] + [(0, int(rng.integers(16)))]
    want = threaded_heads(lambda bh: oo.gqa(d["q"], d["k"], d["v"], causal=False, heads=[bh])[0], heads)
    got = np.stack([out[b, h] for b, h in heads])
    err = rel_l2(got, want)
    print(f"gqa_f32 seed={seed} heads={heads} rel_l2={err:.3e}", flush=True)
    assert err < GATE
    assert np.isfinite(out).all()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dims", [dict(B=1, S=64, HQ=2, HKV=1), dict(B=2, S=256, HQ=4, HKV=2),
                                  dict(B=1, S=100, HQ=2, HKV=1), dict(B=1, S=1, HQ=2, HKV=1),
                                  dict(B=2, S=333, HQ=4, HKV=2), dict(B=1, S=640, HQ=2, HKV=1)])
def test_gqa_f32_small_full_compare(dev, causal, dims):
    d = oi.draw("gqa_full", 7, dims=dict(dims, D=128))
    out = to_host(ops.gqa(*_qkv(d, dev), causal=causal))
    want = oo.gqa(d["q"], d["k"], d["v"], causal=causal)
    err = rel_l2(out, want)
    print(f"gqa_f32 {dims} causal={causal} rel_l2={err:.3e}", flush=True)
    assert err < GATE


def test_gqa_f32_power_of_two_rescaling_is_exact(dev):
    d = oi.draw("gqa_full", 3, dims=dict(B=1, S=192, HQ=4, HKV=2, D=128))
    q, k, v = _qkv(d, dev)
    base = to_host(ops.gqa(q, k, v, causal=True))
    # q * 2^20 with scale * 2^-20: identical scores, identical limbs
    sc = 1.0 / np.sqrt(128.0)
    a = to_host(ops.gqa(q * 2.0 ** 20, k, v, causal=True, scale=sc * 2.0 ** -20))
    np.testing.assert_array_equal(a, base)
    # v * 2^-30: output scaled exactly
    b = to_host(ops.gqa(q, k, v * 2.0 ** -30, causal=True))
    np.testing.assert_array_equal(b, base * np.float32(2.0 ** -30))


def test_gqa_f32_key_tiles_of_different_magnitude(dev):
    # keys of the first 64-key tile scaled up 2^10 (each tile has its own scale)
    d = oi.draw("gqa_full", 5, dims=dict(B=1, S=256, HQ=2, HKV=1, D=128))
    kk = d["k"].copy()
    kk[:, :64] *= np.float32(1024.0)
    qq = d["q"] * np.float32(1.0 / 256.0)
    out = to_host(ops.gqa(to_dev(qq, dev), to_dev(kk, dev), to_dev(d["v"], dev)))
    want = oo.gqa(qq, kk, d["v"])
    err = rel_l2(out, want)
    print(f"gqa_f32 mixed-magnitude key tiles rel_l2={err:.3e}", flush=True)
    assert err < GATE


def test_gqa_f32_causal_first_row_is_v0(dev):
    d = oi.draw("gqa_full", 11, dims=dict(B=2, S=128, HQ=4, HKV=2, D=128))
    out = to_host(ops.gqa(*_qkv(d, dev), causal=True))
    np.testing.assert_allclose(out[:, 0], np.repeat(d["v"][:, 0], 2, axis=1), rtol=1e-6, atol=0)


def test_gqa_f32_rejects_unsupported(dev):
    q = torch.zeros(1, 8, 6, 128, device=dev)
    kv = torch.zeros(1, 8, 4, 128, device=dev)
    with pytest.raises(ValueError, match="not a multiple"):
        ops.gqa(q, kv, kv)
    with pytest.raises(ValueError, match="head_dim"):
        ops.gqa(torch.zeros(1, 8, 2, 64, device=dev), torch.zeros(1, 8, 1, 64, device=dev),
                torch.zeros(1, 8, 1, 64, device=dev))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv", [(1, 1), (4, 1), (8, 1), (6, 2), (16, 2)])
def test_gqa_f32_group_sizes(dev, causal, hq, hkv):
    d = oi.draw("gqa_full", hq * 10 + hkv, dims=dict(B=1, S=200, HQ=hq, HKV=hkv, D=128))
    out = to_host(ops.gqa(*_qkv(d, dev), causal=causal))
    err = rel_l2(out, oo.gqa(d["q"], d["k"], d["v"], causal=causal))
    print(f"gqa f32 Hq={hq} Hkv={hkv} causal={causal} rel_l2={err:.3e}", flush=True)
    assert err < GATE


def test_gqa_full_kwargs_contract(dev):
    """ops.gqa_full(**{q, k, v}) is the NKIBench forward: non-causal, (B, Hq, S, D)."""
    d = oi.draw("gqa_full", 4, dims=dict(B=1, S=256, HQ=4, HKV=2, D=128))
    out = ops.gqa_full(**{k: to_dev(v, dev) for k, v in d.items()})
    assert tuple(out.shape) == (1, 4, 256, 128)
    want = oo.gqa(d["q"], d["k"], d["v"], causal=False, out_layout="bhsd")
    assert rel_l2(to_host(out), want) < GATE
