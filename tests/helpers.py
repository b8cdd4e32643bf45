"""Shared helpers for the tests: torch <-> oracle conversions and seeded inputs."""

from __future__ import annotations

import numpy as np
import torch

from oracle.numerics import T


def dt_of(t: torch.Tensor) -> str:
    if t.dtype == torch.bfloat16:
        return "bf16"
    if t.dtype == torch.float16:
        return "f16"
    if t.dtype == torch.float32:
        return "f32"
    raise TypeError(t.dtype)


def to_T(t: torch.Tensor) -> T:
    return T(t.detach().float().cpu().numpy(), dt_of(t), dim0=(t.dim() == 0))


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, seed, dtype=torch.bfloat16, std=1.0, mean=0.0):
    x = torch.randn(shape, generator=gen(seed), dtype=torch.float32) * std + mean
    return x.to(dtype)


def assert_same_bits(a: np.ndarray, b: np.ndarray, what: str = ""):
    """Exact equality of float32 arrays (NaN == NaN)."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    eq = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    bad = int((~eq).sum())
    if bad:
        idx = np.argwhere(~eq)[:5]
        raise AssertionError(f"{what}: {bad} of {a.size} differ; first at {idx.tolist()}: "
                             f"{a[tuple(idx[0])]} vs {b[tuple(idx[0])]}")


def bf16_ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 values (monotone map)."""
    def key(x):
        u = (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.int64)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(key(a) - key(b))


def f16_ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in fp16 steps between two arrays of fp16 values (monotone map)."""
    def key(x):
        u = np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16).astype(np.int64)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(key(a) - key(b))


def bf16_step(a) -> np.ndarray:
    """Spacing of the bf16 values at |a|, elementwise: 2^(e - 7) for a normal
    a = m * 2^e (1 <= m < 2), the subnormal spacing 2^-133 below 2^-126."""
    a = np.abs(np.asarray(a, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def nan_canon(codes: np.ndarray) -> np.ndarray:
    """e4m3fn codes with both NaN codes (0x7F, 0xFF) mapped to 0x7F.

    The sign of a NaN is not part of the contract: torch's own float32->bf16
    conversion returns 0x7FC0 on its scalar path and 0xFFFF on its vectorized
    path, so the sign a NaN carries into the e4m3 code depends on the path.
    """
    c = np.asarray(codes, dtype=np.uint8).copy()
    c[(c & 0x7F) == 0x7F] = 0x7F
    return c
