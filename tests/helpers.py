"""Host-side helpers shared by the tests: exact bf16 <-> uint16 transfers."""

from __future__ import annotations

import numpy as np


def to_bf16_tensor(bits: np.ndarray, device):
    """uint16 bf16 bit patterns → a torch bf16 tensor on `device` (bit-identical)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_bits(t) -> np.ndarray:
    """torch bf16 tensor → uint16 bit patterns on the host."""
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
