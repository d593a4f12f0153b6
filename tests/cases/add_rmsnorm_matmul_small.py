"""A small case module in the NKIBench reference-file format with a scalar input:
y = x + z; y / sqrt(sum(y^2 / K) + eps) * g @ w, fp32 (eps is the third input)."""
import numpy as np


def get_inputs():
    x = np.random.normal(0.0, 1.0, (96, 128)).astype(np.float32)
    w = np.random.normal(0.0, 1.0, (128, 64)).astype(np.float32)
    eps = 1e-5
    z = np.random.normal(0.0, 1.0, (96, 128)).astype(np.float32)
    g = np.random.normal(0.0, 1.0, (128,)).astype(np.float32)
    return [x, w, eps, z, g]


def forward(x, w, eps, z, g):
    y = x + z
    k = np.float32(y.shape[1])
    y = y / np.sqrt(np.sum(np.square(y) / k, axis=1, keepdims=True) + np.float32(eps))
    y = y * g
    return np.matmul(y, w).astype(np.float32)
