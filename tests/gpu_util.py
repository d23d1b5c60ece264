"""Device helpers for the GPU parity tests (torch is only memory plumbing)."""
from __future__ import annotations

import sys

import numpy as np
import torch


def say(*a):
    """Names the case on stdout before a GPU step, flushed."""
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def pos_tensor(values) -> torch.Tensor:
    return torch.tensor(list(values), dtype=torch.int32, device="cuda")


def randn_f16(shape, seed: int, scale=None) -> torch.Tensor:
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    if scale is not None:
        x = x * scale
    return x.to(torch.float16)


def cache_rows_f32(cache: torch.Tensor, b: int, L: int) -> np.ndarray:
    """[B][Hkv][cap][D] fp16 device cache -> token-major [L][Hkv][D] f32 host."""
    return cache[b, :, :L, :].permute(1, 0, 2).float().contiguous().cpu().numpy()
