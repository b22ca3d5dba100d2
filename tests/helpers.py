"""numpy <-> torch plumbing shared by the tests (bit-level views, no value conversion)."""

from __future__ import annotations

import numpy as np
import torch


def bf16_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def u8_tensor(a: np.ndarray, device, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)
    return t.view(dtype) if dtype is not None else t


def f32_tensor(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bytes8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def f32_of_bf16(t: torch.Tensor) -> np.ndarray:
    from oracle.numerics import from_bf16_bits

    return from_bf16_bits(bits16(t))
