"""Host <-> device helpers for the GPU parity tests (torch is only the allocator here)."""
from __future__ import annotations

import numpy as np
import torch

from inferd_amd.ops import MoeW, QLinear


def dev(a: np.ndarray) -> torch.Tensor:
    """numpy -> cuda tensor; uint16 becomes bfloat16, uint32 becomes int32 (same bits)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def qlinear(wq, s, b, flipped=False, bits=4) -> QLinear:
    N = wq.shape[0]
    return QLinear(dev(wq), dev(s), dev(b), N, wq.shape[1] * 32 // bits, flipped, bits)


def moew(wq, s, b) -> MoeW:
    E, N, kw = wq.shape
    return MoeW(dev(wq), dev(s), dev(b), E, N, kw * 8)
