"""GPU parity: the fp32 NKIBench GEMM operators (three-product bf16 split on MFMA)
vs the fp32 numpy oracle.  Gate: relative-L2 <= 1e-5 (stricter than the
reference's 2e-5, adapter/nkibench_case.py:51).

Full NKIBench shapes on the five seeds (different inputs per seed), plus small
and ragged shapes.  bmm's 1 GB output is compared whole on seed 0 and on three sampled
batches for the other seeds."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, batched_rel_l2, to_dev, to_host
from kda import ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2, split_bf16x2

pytestmark = pytest.mark.gpu
GATE = 1e-5


def _run(case, fn, oracle_fn, seed, dims=None):
    d = oi.draw(case, seed, dims=dims)
    dev_in = {k: (to_dev(v, "cuda") if isinstance(v, np.ndarray) else v) for k, v in d.items()}
    got = to_host(fn(**dev_in))
    want = oracle_fn(**d)
    err = rel_l2(got, want)
    print(f"{case} seed={seed} dims={dims} rel_l2={err:.3e}", flush=True)
    return err


CASES = {
    "matmul": (ops.matmul, oo.matmul),
    "transpose_matmul": (ops.transpose_matmul, oo.transpose_matmul),
    "lora": (ops.lora, oo.lora),
    "rmsnorm_matmul": (ops.rmsnorm_matmul, oo.rmsnorm_matmul),
    "add_rmsnorm_matmul": (ops.add_rmsnorm_matmul, oo.add_rmsnorm_matmul),
    "matmul_add_rmsnorm": (ops.matmul_add_rmsnorm, oo.matmul_add_rmsnorm),
    "swiglu": (ops.swiglu, oo.swiglu),
}


@pytest.mark.parametrize("case", list(CASES))
def test_full_size_all_seeds(case):
    fn, ref = CASES[case]
    for s in SEEDS:
        assert _run(case, fn, ref, s) < GATE


SMALL = {
    "matmul": [dict(M=256, K=64, N=256), dict(M=37, K=96, N=40), dict(M=300, K=160, N=264),
               dict(M=1, K=32, N=8)],
    "transpose_matmul": [dict(M=256, K=64, N=256), dict(M=40, K=96, N=72), dict(M=264, K=160, N=136)],
    "lora": [dict(M=256, K=64, N=256, R=32), dict(M=77, K=96, N=136, R=64),
             # x@a split along K into 16 and into 2 fp32 partials
             dict(M=512, K=1024, N=256, R=128), dict(M=300, K=640, N=200, R=64)],
    # K of 2048 and 2560 (several chunks per thread in the norm pass), M not a multiple of 4
    "rmsnorm_matmul": [dict(M=256, K=128, N=256), dict(M=50, K=96, N=72), dict(M=7, K=2048, N=40),
                       dict(M=37, K=2560, N=64)],
    "add_rmsnorm_matmul": [dict(M=256, K=128, N=256), dict(M=50, K=96, N=72), dict(M=5, K=2048, N=40),
                           dict(M=33, K=2560, N=64)],
    "matmul_add_rmsnorm": [dict(M=256, K=128, N=256), dict(M=50, K=96, N=200), dict(M=300, K=64, N=520)],
    # F = 38400: 300 tiles of 256x128 on 256 CUs, the last 44 x 128 columns as 128x128 tiles
    "swiglu": [dict(M=256, K=64, N=128), dict(M=50, K=96, N=160), dict(M=256, K=64, N=38400)],
}


@pytest.mark.parametrize("case,dims", [(c, d) for c, ds in SMALL.items() for d in ds])
def test_small_and_ragged(case, dims):
    fn, ref = CASES[case]
    assert _run(case, fn, ref, 7, dims=dims) < GATE


def test_bmm_full_size_sampled_batches():
    for s in SEEDS:
        d = oi.draw("bmm", s)
        out = ops.bmm(to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda"))
        rng = np.random.default_rng(s)
        picks = sorted({0, 15, int(rng.integers(16))})
        got = to_host(out[picks])
        want = oo.bmm(d["lhs"][picks], d["rhs"][picks])
        err = rel_l2(got, want)
        print(f"bmm seed={s} batches={picks} rel_l2={err:.3e}", flush=True)
        assert err < GATE
        del out
        torch.cuda.empty_cache()


def test_bmm_full_size_every_batch():
    """Seed 0 at the NKIBench shape: all 16 batches of the 1.07 GB output."""
    d = oi.draw("bmm", 0)
    out = ops.bmm(to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda"))
    err, per = batched_rel_l2(out, lambda b: oo.bmm(d["lhs"][b:b + 1], d["rhs"][b:b + 1]),
                              range(out.shape[0]))
    print(f"bmm seed=0 all {out.shape[0]} batches rel_l2={err:.3e} worst batch {max(per):.3e}", flush=True)
    assert out.shape[0] == 16 and err < GATE and max(per) < GATE
    del out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dims", [dict(B=3, M=256, K=64, N=256), dict(B=2, M=100, K=96, N=72),
                                  dict(B=2, M=130, K=32, N=200), dict(B=1, M=17, K=64, N=8),
                                  dict(B=7, M=2048, K=64, N=1280), dict(B=16, M=256, K=64, N=2048),
                                  dict(B=20, M=128, K=64, N=4096)])
def test_bmm_small(dims):
    # K = 64 with M and N multiples of 128 runs the persistent kernel: 1120, 512 and
    # 640 tiles (several per workgroup, uneven counts)
    assert _run("bmm", ops.bmm, oo.bmm, 5, dims=dims) < GATE


def test_bmm_persistent_matches_per_tile_kernel():
    """The persistent kernel (whole 128 x 128 tiles, K = 64) and the per-tile kernel
    (taken when N is not a multiple of 128) do the same arithmetic in the same
    order: widening rhs by 8 columns leaves the first 2048 columns bit-identical."""
    d = oi.draw("bmm", 3, dims=dict(B=16, M=384, K=64, N=2048))
    lhs, rhs = to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda")
    wide = torch.cat([rhs, torch.randn(16, 64, 8, device="cuda")], dim=2).contiguous()
    a = ops.bmm(lhs, rhs)
    b = ops.bmm(lhs, wide)
    torch.cuda.synchronize()
    assert torch.equal(a, b[:, :, :2048])
    assert rel_l2(to_host(a), oo.bmm(d["lhs"], d["rhs"])) < GATE


@pytest.mark.parametrize("dims", [dict(B=2, M=130, K=64, N=200), dict(B=3, M=64, K=32, N=72)])
def test_bmm_small_k_without_workspace(dims):
    # K <= 64 needs no workspace (fragments are split in registers): a NULL
    # workspace is accepted and gives the same products, same gate.
    from kda import _lib
    d = oi.draw("bmm", 11, dims=dims)
    lhs, rhs = to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda")
    b, m, k, n = dims["B"], dims["M"], dims["K"], dims["N"]
    out = torch.empty((b, m, n), dtype=torch.float32, device="cuda")
    _lib.call("kda_bmm_f32", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), b, m, k, n, None, 0,
              torch.cuda.current_stream().cuda_stream)
    err = rel_l2(to_host(out), oo.bmm(d["lhs"], d["rhs"]))
    print(f"bmm (no workspace) dims={dims} rel_l2={err:.3e}", flush=True)
    assert err < GATE


def test_matmul_f32_layout_identity():
    # A = I (hi = I, lo = 0) selects rows of B: the result is exactly hi(B) + lo(B),
    # so any transposed or swizzled fragment, or a dropped split term, shows up exactly
    k = 256
    b = np.random.default_rng(0).standard_normal((k, 264)).astype(np.float32)
    got = to_host(ops.matmul(to_dev(np.eye(k, dtype=np.float32), "cuda"), to_dev(b, "cuda")))
    hi, lo = split_bf16x2(b)
    np.testing.assert_array_equal(got, hi + lo)
    assert rel_l2(got, b) < 1e-5


def test_split_rounding_matches_rne_on_crafted_values():
    """The device's bf16 conversion (hi = bf16(x), lo = bf16(x - hi)) equals
    round-to-nearest-even on values built to hit its edge cases: exact ties of the
    hi rounding with even and odd last bits, one below and above a tie, ties of
    the residual, carries into the exponent, both signs, magnitudes 2^-100..2^100.
    A = I makes the output exactly hi(B) + lo(B)."""
    rng = np.random.default_rng(5)
    k, n = 256, 264
    top = rng.integers(0, 1 << 16, size=(k, n), dtype=np.uint32)
    exp = rng.integers(127 - 100, 127 + 100, size=(k, n), dtype=np.uint32)
    top = (top & np.uint32(0x807F)) | (exp << np.uint32(7))          # sign, exponent, 7 mantissa bits
    low_patterns = np.array([0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF, 0x4080, 0x2040, 0x1020,
                             0x0180, 0xC080, 0x80C0, 0x3F80], dtype=np.uint32)
    low = np.where(rng.random((k, n)) < 0.75,
                   low_patterns[rng.integers(0, len(low_patterns), size=(k, n))],
                   rng.integers(0, 1 << 16, size=(k, n), dtype=np.uint32))
    bits = (top << np.uint32(16)) | low
    bits[0, :8] = [0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000,    # ties, even / odd hi
                   0x7F7E8000, 0x7F7EFFFF, 0x0D800000, 0x0D808000]    # near bf16 max, tiny
    b = bits.view(np.float32)
    assert np.isfinite(b).all()
    hi, lo = split_bf16x2(b)
    assert np.isfinite(hi + lo).all()
    got = to_host(ops.matmul(to_dev(np.eye(k, dtype=np.float32), "cuda"), to_dev(b, "cuda")))
    np.testing.assert_array_equal(got.view(np.uint32), (hi + lo).view(np.uint32))


def test_lora_rank_zero_term_matches_matmul():
    # b = 0 removes the low-rank term: lora == matmul
    d = oi.draw("lora", 3, dims=dict(M=256, K=128, N=256, R=32))
    d["b"] = np.zeros_like(d["b"])
    dev_in = {k: to_dev(v, "cuda") for k, v in d.items()}
    a = to_host(ops.lora(**dev_in))
    m = to_host(ops.matmul(dev_in["x"], dev_in["w"]))
    np.testing.assert_array_equal(a, m)


def test_fp32_path_rejects_unaligned_k():
    x = torch.zeros(64, 40, device="cuda")
    w = torch.zeros(40, 64, device="cuda")
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.matmul(x, w)


@pytest.mark.parametrize("bits", [0xFFFFFFFF, 0x7F800001, 0xFFC00000])
@pytest.mark.parametrize("op", ["matmul", "bmm"])
def test_nan_inputs_propagate_through_the_split(op, bits):
    """A NaN in lhs (any payload, either sign) splits into NaN limbs: exactly the
    output rows it feeds are NaN, the others equal the NaN-free result."""
    rng = np.random.default_rng(bits & 0xFFFF)
    if op == "matmul":
        lhs = rng.normal(size=(96, 64)).astype(np.float32)
        rhs = rng.normal(size=(64, 72)).astype(np.float32)
        bad = (5, 17)
        fn = ops.matmul
    else:
        lhs = rng.normal(size=(2, 96, 64)).astype(np.float32)
        rhs = rng.normal(size=(2, 64, 64)).astype(np.float32)
        bad = (1, 5, 17)
        fn = ops.bmm
    clean = to_host(fn(to_dev(lhs, "cuda"), to_dev(rhs, "cuda")))
    lhs_nan = lhs.copy()
    lhs_nan.view(np.uint32)[bad] = np.uint32(bits)
    assert np.isnan(lhs_nan[bad])
    got = to_host(fn(to_dev(lhs_nan, "cuda"), to_dev(rhs, "cuda")))
    row = bad[:-1]
    assert np.isnan(got[row]).all()
    mask = np.ones(got.shape[:-1], dtype=bool)
    mask[row] = False
    np.testing.assert_array_equal(got[mask], clean[mask])
