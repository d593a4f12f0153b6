"""kda_rmsnorm_matmul_bf16_noalloc (static per-device scratch, no allocation) against
kda_rmsnorm_matmul_bf16 with a caller workspace: bit-identical outputs on two calls in
a row, the second smaller (the scratch keeps the first call's contents), and the
size limit rejected before any launch.  Both are called through the C ABI."""
import numpy as np
import pytest
import torch

from gpu_util import to_dev, to_host
from kda import _lib, ops
from oracle import inputs as oi
from oracle import ops as oo
from oracle.numerics import rel_l2

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
SCRATCH = 64 << 20


def _inputs(dev, seed, m, k, n):
    d = oi.draw("rmsnorm_matmul_cfg", seed, dims=dict(M=m, K=k, N=n))
    return d, [to_dev(d[name], dev, BF) for name in ("x", "gamma", "w")]


def _with_workspace(x, gamma, w, eps):
    m, k = x.shape
    n = w.shape[1]
    y = torch.empty(m, n, dtype=BF, device=x.device)
    ws = torch.empty(ops.rmsnorm_matmul_workspace_size(m, k), dtype=torch.uint8, device=x.device)
    _lib.call("kda_rmsnorm_matmul_bf16", x.data_ptr(), gamma.data_ptr(), w.data_ptr(), y.data_ptr(),
              m, k, n, eps, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    return y


def _no_alloc(x, gamma, w, eps):
    m, k = x.shape
    n = w.shape[1]
    y = torch.empty(m, n, dtype=BF, device=x.device)
    _lib.call("kda_rmsnorm_matmul_bf16_noalloc", x.data_ptr(), gamma.data_ptr(), w.data_ptr(),
              y.data_ptr(), m, k, n, eps, torch.cuda.current_stream().cuda_stream)
    return y


def test_no_alloc_matches_workspace_entry_point_twice(dev):
    # first a large call (graded K, 24 MiB of the 64 MiB scratch), then a smaller one
    for seed, (m, k, n) in ((1, (3000, 4096, 1024)), (2, (130, 256, 264))):
        d, (x, gamma, w) = _inputs(dev, seed, m, k, n)
        want = _with_workspace(x, gamma, w, d["eps"])
        got = _no_alloc(x, gamma, w, d["eps"])
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={m} K={k} N={n}: outputs differ"
        err = rel_l2(to_host(got), oo.rmsnorm_matmul_gamma(**d))
        print(f"noalloc M={m} K={k} N={n}: bit-identical, rel_l2 vs oracle {err:.3e}", flush=True)
        assert err < 1e-2


def test_no_alloc_rejects_sizes_beyond_the_buffer(dev):
    # 2*M*K + 4*M > 64 MiB: rejected before any launch (tiny real buffers suffice)
    t = torch.zeros(64, dtype=BF, device=dev)
    m, k = 8192, 4096
    assert 2 * m * k + 4 * m > SCRATCH
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("kda_rmsnorm_matmul_bf16_noalloc", t.data_ptr(), t.data_ptr(), t.data_ptr(),
                  t.data_ptr(), m, k, 8, 1e-6, torch.cuda.current_stream().cuda_stream)
    assert np.isfinite(to_host(t)).all()
