"""A small case module in the NKIBench reference-file format: lhs @ rhs, fp32."""
import numpy as np


def get_inputs():
    lhs = np.random.normal(0.0, 1.0, (128, 256)).astype(np.float32)
    rhs = np.random.normal(0.0, 1.0, (256, 192)).astype(np.float32)
    return [lhs, rhs]


def forward(lhs, rhs):
    return np.matmul(lhs, rhs).astype(np.float32)
