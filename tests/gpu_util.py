"""Helpers shared by the GPU parity tests (host<->device moves, gates)."""
import numpy as np
import torch

SEEDS = [0, 21, 42, 63, 84]


def to_dev(a, dev, dtype=torch.float32):
    """numpy array (float32 values; bf16-valued for bf16 inputs) -> GPU tensor."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dev).to(dtype).contiguous()


def to_host(t):
    return t.detach().to(torch.float32).cpu().numpy()


def elementwise_in_slices(fn, arrays, n_out=1, parts=16):
    """fn(*arrays) for an elementwise fn, evaluated on `parts` contiguous slices in
    threads (numpy releases the GIL in its loops) and concatenated: the same values
    as one call, in a fraction of the time for 2^27-element buffers."""
    from concurrent.futures import ThreadPoolExecutor
    n = arrays[0].shape[0]
    bounds = [(i * n // parts, (i + 1) * n // parts) for i in range(parts)]
    with ThreadPoolExecutor(max_workers=8) as pool:
        res = list(pool.map(lambda b: fn(*(a[b[0]:b[1]] for a in arrays)), bounds))
    if n_out == 1:
        return np.concatenate(res)
    return tuple(np.concatenate([r[j] for r in res]) for j in range(n_out))


def threaded_heads(fn, heads, workers=8):
    """Stacks fn((b, h)) over heads, evaluated in a thread pool."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=workers) as pool:
        return np.stack(list(pool.map(fn, heads)))


def batched_rel_l2(out, ref_fn, batches, workers=4):
    """rel-L2 (float64 norms, as oracle.numerics.rel_l2) of a whole batched GPU
    output against ref_fn(b) -> the oracle's batch b, accumulated batch by batch so
    that only a few batches are on the host at once.  Returns (overall, per batch)."""
    from concurrent.futures import ThreadPoolExecutor

    def one(b):
        got = out[b].detach().to(torch.float32).cpu().numpy().astype(np.float64)
        want = np.asarray(ref_fn(b), dtype=np.float64).reshape(got.shape)
        return float(np.sum((got - want) ** 2)), float(np.sum(want ** 2))

    with ThreadPoolExecutor(max_workers=workers) as pool:
        parts = list(pool.map(one, batches))
    num = sum(p[0] for p in parts)
    den = sum(p[1] for p in parts)
    per = [float(np.sqrt(a / b)) if b else 0.0 for a, b in parts]
    return float(np.sqrt(num / den)), per
