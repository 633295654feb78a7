"""Loader of the committed golden fixtures (``tests/golden/fp8_golden.npz``)."""

import pathlib

import numpy as np
import torch

PATH = pathlib.Path(__file__).resolve().parent / "golden" / "fp8_golden.npz"


def load() -> dict[str, np.ndarray]:
    with np.load(PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def e4m3(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(codes).view(torch.float8_e4m3fn)


def t(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a))
