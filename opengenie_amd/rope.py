"""Split 3-D RoPE cos/sin tables for a video latent grid.

The fused preattention op consumes cos/sin in the layout the reference passes
to it, [B or 1, heads, tokens, head_dim/2] (triton_ltx_ops.py:1535). The
exact LTX-2 table recipe lives in ltx_core, which is not vendored, so this
module defines a deterministic table of the same shape and role: tokens are
numbered frame-major over a (t, h, w) grid; the heads*head_dim/2 rotation
frequencies of a token are dealt round-robin to the three axes, the j-th
frequency of an axis being theta**(-j / per_axis), and the angle is that
frequency times the token's coordinate on the axis.
"""

from __future__ import annotations

import torch


def video_rope_cos_sin(grid: tuple[int, int, int], *, heads: int = 32, head_dim: int = 128, theta: float = 10000.0,
                       device: str | torch.device = "cpu", dtype: torch.dtype = torch.bfloat16):
    """cos, sin of shape (1, heads, t*h*w, head_dim//2) for grid (t, h, w)."""
    gt, gh, gw = grid
    half = head_dim // 2
    nfreq = heads * half
    f = torch.arange(nfreq, device=device, dtype=torch.float64)
    axis = (f % 3).long()
    per_axis = (nfreq + 2) // 3
    freq = theta ** (-(torch.div(f, 3, rounding_mode="floor")) / per_axis)
    tt, hh, ww = torch.meshgrid(torch.arange(gt, device=device), torch.arange(gh, device=device),
                                torch.arange(gw, device=device), indexing="ij")
    pos = torch.stack([tt.reshape(-1), hh.reshape(-1), ww.reshape(-1)], dim=1).to(torch.float64)  # (N, 3)
    ang = pos[:, axis] * freq  # (N, nfreq)
    ang = ang.reshape(-1, heads, half).transpose(0, 1).unsqueeze(0)  # (1, heads, N, half)
    return ang.cos().to(dtype).contiguous(), ang.sin().to(dtype).contiguous()
