"""GPU parity: grouped-query flash attention (bf16, fp32 online softmax) vs the oracle.

Full-size causal configuration (B4 S4096 Hq32 Hkv8 D128): the GPU computes the
whole output; the oracle checks every (batch, head) slice on seed 0 and a
sample of slices on each of the five seeds.
Gate: relative-L2 <= 1e-2 (bf16)."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, threaded_heads, to_dev, to_host
from kda import ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
GATE = 1e-2


@pytest.mark.parametrize("seed", SEEDS)
def test_gqa_causal_config_full_size_sampled_heads(dev, seed):
    d = oi.draw("gqa_cfg", seed)
    out = ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=True)
    out = to_host(out)
    rng = np.random.default_rng(seed)
    heads = [(0, 0), (3, 31)] + [(int(rng.integers(4)), int(rng.integers(32))) for _ in range(2)]
    want = oo.gqa(d["q"], d["k"], d["v"], causal=True, heads=heads)
    got = np.stack([out[b, :, h, :] for b, h in heads])
    err = rel_l2(got, want)
    print(f"gqa_cfg seed={seed} heads={heads} rel_l2={err:.3e}", flush=True)
    assert err < GATE
    assert np.isfinite(out).all()


def test_gqa_causal_config_full_size_every_head(dev):
    """Seed 0: all 4 x 32 (batch, head) slices of the output against the oracle."""
    d = oi.draw("gqa_cfg", 0)
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=True))
    heads = [(b, h) for b in range(4) for h in range(32)]
    want = threaded_heads(lambda bh: oo.gqa(d["q"], d["k"], d["v"], causal=True, heads=[bh])[0], heads)
    got = np.stack([out[b, :, h, :] for b, h in heads])
    err = rel_l2(got, want)
    worst = max(rel_l2(got[i], want[i]) for i in range(len(heads)))
    print(f"gqa_cfg seed=0 all 128 heads rel_l2={err:.3e} worst head {worst:.3e}", flush=True)
    assert err < GATE and worst < GATE


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dims", [dict(B=1, S=64, HQ=4, HKV=1), dict(B=2, S=256, HQ=8, HKV=2),
                                  dict(B=1, S=100, HQ=4, HKV=1), dict(B=1, S=1, HQ=4, HKV=1),
                                  dict(B=2, S=333, HQ=8, HKV=2)])
def test_gqa_small_full_compare(dev, causal, dims):
    d = oi.draw("gqa_cfg", 7, dims=dict(dims, D=128))
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=causal))
    want = oo.gqa(d["q"], d["k"], d["v"], causal=causal)
    err = rel_l2(out, want)
    print(f"gqa {dims} causal={causal} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


@pytest.mark.parametrize("dims", [dict(B=5, S=3000, HQ=16, HKV=2), dict(B=2, S=2048, HQ=24, HKV=8)])
def test_gqa_causal_persistent_several_blocks_per_workgroup(dev, dims):
    """Causal launches run one workgroup per CU over more blocks than CUs: 940 blocks
    with partial last key tiles (8 heads per workgroup), and 384 blocks of one head
    each (G = 3), so workgroups run several blocks of different lengths and prefetch
    each next block's first tiles.  Sampled heads against the oracle."""
    d = oi.draw("gqa_cfg", 13, dims=dict(dims, D=128))
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=True))
    b_n, h_n = dims["B"], dims["HQ"]
    heads = [(0, 0), (b_n - 1, h_n - 1), (b_n // 2, h_n // 3), (1, h_n // 2 + 1)]
    want = threaded_heads(lambda bh: oo.gqa(d["q"], d["k"], d["v"], causal=True, heads=[bh])[0], heads)
    got = np.stack([out[b, :, h, :] for b, h in heads])
    err = rel_l2(got, want)
    print(f"gqa persistent {dims} heads={heads} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3 and np.isfinite(out).all()


def test_gqa_bhsd_layout_and_custom_scale(dev):
    d = oi.draw("gqa_cfg", 9, dims=dict(B=1, S=192, HQ=8, HKV=2, D=128))
    qkv = [to_dev(d[k], dev, BF) for k in ("q", "k", "v")]
    a = to_host(ops.gqa(*qkv, causal=False, scale=0.05, out_layout="bhsd"))
    want = oo.gqa(d["q"], d["k"], d["v"], causal=False, scale=0.05, out_layout="bhsd")
    assert a.shape == (1, 8, 192, 128)
    assert rel_l2(a, want) < 5e-3
    b = to_host(ops.gqa(*qkv, causal=False, scale=0.05))
    np.testing.assert_array_equal(a, b.transpose(0, 2, 1, 3))


def test_gqa_causal_first_row_is_v0(dev):
    d = oi.draw("gqa_cfg", 11, dims=dict(B=2, S=128, HQ=8, HKV=2, D=128))
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=True))
    np.testing.assert_array_equal(out[:, 0], np.repeat(d["v"][:, 0], 4, axis=1))


def test_gqa_rejects_unsupported(dev):
    q = torch.zeros(1, 8, 4, 64, device=dev, dtype=BF)
    kv = torch.zeros(1, 8, 1, 64, device=dev, dtype=BF)
    with pytest.raises(ValueError, match="head_dim"):
        ops.gqa(q, kv, kv)
    q = torch.zeros(1, 8, 6, 128, device=dev, dtype=BF)
    kv = torch.zeros(1, 8, 4, 128, device=dev, dtype=BF)
    with pytest.raises(ValueError, match="not a multiple"):
        ops.gqa(q, kv, kv)


# Every group size: a workgroup serves the largest power of two up to 8 that
# divides G of a kv head's query heads (G = 3, 6: 1 and 2 heads per workgroup).
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2), (6, 2), (6, 1), (16, 2), (16, 1), (12, 3)])
def test_gqa_group_sizes(dev, causal, hq, hkv):
    d = oi.draw("gqa_cfg", hq * 10 + hkv, dims=dict(B=2, S=300, HQ=hq, HKV=hkv, D=128))
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=causal))
    err = rel_l2(out, oo.gqa(d["q"], d["k"], d["v"], causal=causal))
    print(f"gqa bf16 Hq={hq} Hkv={hkv} causal={causal} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3


@pytest.mark.parametrize("causal", [True, False])
def test_gqa_output_8byte_aligned_matches_aligned(dev, causal):
    """Output rows that are only 8-byte aligned (base 8 bytes past a 16-byte
    boundary, which the launcher accepts) give the same bits as an aligned output,
    and nothing is written outside them.  B5 S3000 Hq16 Hkv2: 940 causal blocks, so
    workgroups run several blocks (staged q rows, stores left in flight)."""
    import math
    from kda import _lib
    b_n, s_n, hq, hkv, d_n = 5, 3000, 16, 2, 128
    d = oi.draw("gqa_cfg", 17, dims=dict(B=b_n, S=s_n, HQ=hq, HKV=hkv, D=d_n))
    q, k, v = (to_dev(d[n], dev, BF) for n in ("q", "k", "v"))
    want = ops.gqa(q, k, v, causal=causal)
    flat = torch.full((b_n * s_n * hq * d_n + 8,), float("nan"), device=dev, dtype=BF)
    out = flat[4:4 + b_n * s_n * hq * d_n]                  # 8 bytes past a 16-byte boundary
    assert out.data_ptr() % 16 == 8
    _lib.call("kda_gqa_fwd_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              b_n, s_n, hq, hkv, d_n, 1.0 / math.sqrt(d_n), 1 if causal else 0,
              s_n * hq * d_n, hq * d_n, d_n, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    got = out.view(b_n, s_n, hq, d_n)
    print(f"gqa 8-byte aligned output causal={causal}: equal={torch.equal(got, want)}", flush=True)
    assert torch.equal(got, want)
    assert torch.isnan(flat[:4]).all() and torch.isnan(flat[-4:]).all()   # nothing outside


@pytest.mark.parametrize("dims", [
    dict(B=4, S=600, HQ=32, HKV=32),   # G = 1: one head per workgroup, 384 blocks of 256 rows
    dict(B=4, S=333, HQ=64, HKV=8),    # G = 8: 352 blocks of 32 rows, partial last key tile
    dict(B=3, S=700, HQ=12, HKV=6),    # G = 2: 396 blocks of 128 rows
])
def test_gqa_causal_persistent_every_head(dev, dims):
    """More causal blocks than CUs at three heads-per-workgroup settings, so every
    workgroup runs several blocks (prefetched first tiles, q rows staged in LDS,
    stores left in flight across the block boundary); every head against the oracle."""
    d = oi.draw("gqa_cfg", 23, dims=dict(dims, D=128))
    out = to_host(ops.gqa(*(to_dev(d[k], dev, BF) for k in ("q", "k", "v")), causal=True))
    heads = [(b, h) for b in range(dims["B"]) for h in range(dims["HQ"])]
    want = threaded_heads(lambda bh: oo.gqa(d["q"], d["k"], d["v"], causal=True, heads=[bh])[0], heads)
    got = np.stack([out[b, :, h, :] for b, h in heads])
    err = rel_l2(got, want)
    print(f"gqa persistent every head {dims} rel_l2={err:.3e}", flush=True)
    assert err < 5e-3 and np.isfinite(out).all()
