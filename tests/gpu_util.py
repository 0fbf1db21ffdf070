"""Helpers shared by the GPU parity tests: device copies, synthetic experts, relative L2."""
from __future__ import annotations

import functools

import numpy as np
import torch

from tinystrata_amd import moe, ops

DEV = "cuda"


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_l2(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@functools.lru_cache(maxsize=None)
def pool(gu: int, d: int, n: int, ff: int, count: int, seed: int) -> np.ndarray:
    L = ops.native_expert_layout(gu, d, n, ff)
    return moe.synthetic_pool(L, count, seed)


def experts(gu: int, d: int, n: int, ff: int, n_expert: int, distinct: int = 8, seed: int = 0):
    """Host blobs [n_expert, stride] (expert x = pool[(x * 5 + 3) % distinct]) and the layer's device weights."""
    L = ops.native_expert_layout(gu, d, n, ff)
    p = pool(gu, d, n, ff, distinct, seed)
    order = (np.arange(n_expert) * 5 + 3) % distinct
    blobs = p[order]
    return L, blobs, p
