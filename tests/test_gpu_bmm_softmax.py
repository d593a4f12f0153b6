"""GPU parity: fused bmm + row softmax (fp32 via two fp16 limbs per operand, three
MFMA products) vs the oracle.

Gate: relative-L2 <= 1e-5.  The full NKIBench shape (B16 M4096 K64 N4096, 1 GiB
output) is compared whole on seed 0 and on sampled batches for the other seeds;
invariants: rows sum to 1 and a per-row constant added to the scores leaves the
output unchanged."""
import numpy as np
import pytest
import torch

from gpu_util import SEEDS, batched_rel_l2, to_dev, to_host
from kda import ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2

pytestmark = pytest.mark.gpu
GATE = 1e-5


def test_bmm_softmax_full_size_sampled_batches():
    for s in SEEDS:
        d = oi.draw("bmm_softmax", s)
        out = ops.bmm_softmax(to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda"))
        rng = np.random.default_rng(s)
        picks = sorted({0, 15, int(rng.integers(16))})
        got = to_host(out[picks])
        want = oo.bmm_softmax(d["lhs"][picks], d["rhs"][picks])
        err = rel_l2(got, want)
        rows = float(torch.max(torch.abs(out.sum(dim=2) - 1.0)).item())
        print(f"bmm_softmax seed={s} batches={picks} rel_l2={err:.3e} max|rowsum-1|={rows:.2e}", flush=True)
        assert err < GATE
        assert rows < 1e-5
        del out
        torch.cuda.empty_cache()


def test_bmm_softmax_full_size_every_batch():
    """Seed 0 at the NKIBench shape: all 16 batches of the 1.07 GB output, and every
    row's sum."""
    d = oi.draw("bmm_softmax", 0)
    out = ops.bmm_softmax(to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda"))
    err, per = batched_rel_l2(out, lambda b: oo.bmm_softmax(d["lhs"][b:b + 1], d["rhs"][b:b + 1]),
                              range(out.shape[0]))
    rows = float(torch.max(torch.abs(out.sum(dim=2) - 1.0)).item())
    print(f"bmm_softmax seed=0 all {out.shape[0]} batches rel_l2={err:.3e} worst batch {max(per):.3e} "
          f"max|rowsum-1|={rows:.2e}", flush=True)
    assert out.shape[0] == 16 and err < GATE and max(per) < GATE
    assert rows < 1e-5
    del out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dims", [dict(B=2, M=128, K=64, N=256), dict(B=3, M=100, K=64, N=128),
                                  dict(B=1, M=17, K=32, N=64), dict(B=2, M=300, K=48, N=192)])
def test_bmm_softmax_small(dims):
    d = oi.draw("bmm_softmax", 9, dims=dims)
    got = to_host(ops.bmm_softmax(to_dev(d["lhs"], "cuda"), to_dev(d["rhs"], "cuda")))
    err = rel_l2(got, oo.bmm_softmax(**d))
    print(f"bmm_softmax {dims} rel_l2={err:.3e}", flush=True)
    assert err < GATE


def test_bmm_softmax_shift_invariance():
    # with lhs[:, :, 7] = c and rhs[:, 7, :] = 1, every score of a row gains c:
    # the softmax rows must not change (c = 0 vs c = 2, both exact in bf16 limbs)
    d = oi.draw("bmm_softmax", 4, dims=dict(B=2, M=128, K=64, N=256))
    lhs, rhs = d["lhs"].copy(), d["rhs"].copy()
    rhs[:, 7, :] = 1.0
    lhs[:, :, 7] = 0.0
    a = to_host(ops.bmm_softmax(to_dev(lhs, "cuda"), to_dev(rhs, "cuda")))
    lhs[:, :, 7] = 2.0
    b = to_host(ops.bmm_softmax(to_dev(lhs, "cuda"), to_dev(rhs, "cuda")))
    assert rel_l2(b, a) < 5e-6


def test_bmm_softmax_rejects_unsupported():
    x = torch.zeros(1, 16, 128, device="cuda")
    y = torch.zeros(1, 128, 64, device="cuda")
    with pytest.raises(ValueError, match="K=128"):
        ops.bmm_softmax(x, y)
    x = torch.zeros(1, 16, 64, device="cuda")
    y = torch.zeros(1, 64, 100, device="cuda")
    with pytest.raises(ValueError, match="multiple of 64"):
        ops.bmm_softmax(x, y)
