"""A small case module in the NKIBench reference-file format (get_inputs / forward),
used to exercise kda.verify's loader.  SiLU, x (64, 1000) fp32."""
import numpy as np


def get_inputs():
    x = np.random.normal(0.0, 1.0, (64, 1000)).astype(np.float32)
    return [x]


def forward(x):
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)
