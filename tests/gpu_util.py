"""Helpers shared by the GPU parity tests: inputs from the oracle's seeded
generators, moved to the device for librq."""
import numpy as np
import torch

from rllm_amd.backend import HostTensor, Q8_1
from rllm_amd.dtype import DType


def make_weight(orc, t: int, n: int, k: int, seed: int, kind: str) -> np.ndarray:
    """GGUF bytes: 'random' = parity.rs-style random blocks, 'normal' = N(0, 0.02) quantized."""
    if kind == "random":
        return orc.random_weight(seed, t, n, k)
    return orc.quantize(t, orc.normal(seed, n * k, 0.0, 0.02), n, k)


def upload(gpu, t: int, w: np.ndarray, n: int, k: int):
    return gpu.upload(HostTensor(f"w{t}", DType(t), (n, k), w))


def q8_1_to_device(gpu, qs: np.ndarray, d: np.ndarray, s: np.ndarray) -> Q8_1:
    dev = gpu.device
    return Q8_1(
        torch.from_numpy(qs.astype(np.int8)).to(dev),
        torch.from_numpy(d.astype(np.uint16).view(np.int16)).to(dev),
        torch.from_numpy(s.astype(np.uint16).view(np.int16)).to(dev),
    )
