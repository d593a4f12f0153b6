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
