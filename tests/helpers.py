"""Small conversions shared by the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch


def bf16_from_np(x: np.ndarray, device) -> torch.Tensor:
    """float32 numpy -> bf16 device tensor (round to nearest even)."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device).to(torch.bfloat16)


def bits_of(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns of a bf16/fp16 tensor as uint16 numpy."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32_of(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def np_of(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy()
