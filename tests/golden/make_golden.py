"""Writes tests/golden/golden.npz: small input/output vectors for every fused op.

The expected outputs come from torch (CPU, torch 2.10) evaluating the
reference's own torch expression for each op (tests/torch_reference.py, which
cites ltx_serve/triton_ltx_ops.py line by line). The shapes and Ada indices
follow the reference's tests (tests/test_triton_ltx_ops.py). Inputs are drawn
with seeded CPU generators. bf16 tensors are stored as uint16 bit patterns,
e4m3 tensors as uint8 codes, float32 as float32.

FP8 cases use scales whose torch semantics are the same on CPU and GPU: a
(1,)-shaped scale (float32 product) and a 0-dim power-of-two scale (its
reciprocal is exact in bf16).

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle.torch_ref as tr  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")


def rn(shape, seed, dtype=torch.bfloat16, std=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


def enc(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float8_e4m3fn:
        return t.contiguous().view(torch.uint8).numpy().copy()
    return t.contiguous().numpy().copy()


def main() -> None:
    d: dict[str, np.ndarray] = {}

    def put(case, **arrs):
        for k, v in arrs.items():
            d[f"{case}/{k}"] = enc(v) if isinstance(v, torch.Tensor) else np.asarray(v)

    # AdaZero from table (reference test :71-92 shape, fewer rows)
    x, tab, ts = rn((1, 3, 2048), 1), rn((6, 2048), 2, torch.float32), rn((1, 3, 6 * 2048), 3, std=0.5)
    put("adazero_from_ada", x=x, table=tab, ts=ts, out=tr.adazero_from_ada(x, 1e-6, tab, ts, 3, 4))
    # AdaZero from table, bf16 table, one timestep row for every token
    x, tab, ts = rn((1, 3, 4096), 4), rn((6, 4096), 5, std=0.02), rn((1, 1, 6 * 4096), 6, std=0.5)
    put("adazero_from_ada_uniform", x=x, table=tab, ts=ts,
        out=tr.adazero_from_ada(x, 1e-6, tab, ts.expand(1, 3, 6 * 4096), 0, 1))
    # AdaZero with stride-3 scale/shift views (reference test :8-26)
    x, ss = rn((1, 3, 2048), 7), rn((1, 3, 3, 2048), 8)
    put("adazero_strided", x=x, ss=ss, out=tr.adazero(x, 1e-6, ss[:, :, 1, :], ss[:, :, 2, :]))
    # AdaLN affine (reference test :119-140)
    x, tab, ts = rn((1, 2, 2048), 9), rn((9, 2048), 10, torch.float32), rn((1, 2, 9 * 2048), 11, std=0.5)
    put("adaln_affine_from_ada", x=x, table=tab, ts=ts, out=tr.adaln_affine_from_ada(x, tab, ts, 6, 7))
    # mul from Ada (reference test :143-163)
    put("mul_from_ada", out=tr.mul_from_ada(x, tab, ts, 8))  # inputs: adaln_affine_from_ada
    # residual gate from Ada (reference test :95-116)
    x, y = rn((1, 2, 2048), 12), rn((1, 2, 2048), 13)
    tab6, ts6 = rn((6, 2048), 14, torch.float32), rn((1, 2, 6 * 2048), 15, std=0.5)
    put("residual_gate_from_ada", x=x, y=y, table=tab6, ts=ts6, out=tr.residual_gate_from_ada(x, y, tab6, ts6, 5))
    # residual gate + bias from Ada (reference test :182-204)
    x, y = rn((1, 2, 2048), 16), rn((1, 2, 2048), 17)
    bias = rn((2048,), 18, torch.float32)
    put("residual_gate_bias_from_ada", x=x, y=y, bias=bias,  # table/ts: adaln_affine_from_ada
        out=tr.residual_gate_bias_from_ada(x, y, bias, tab, ts, 8))
    # residual gate with a strided gate (reference test :29-47)
    x, y, gates = rn((1, 3, 2048), 19), rn((1, 3, 2048), 20), rn((1, 3, 3, 2048), 21)
    put("residual_gate_bf16", x=x, y=y, gates=gates, out=tr.residual_gate(x, y, gates[:, :, 1, :]))
    # bias add (reference test :166-179)
    x, bias = rn((5, 2048), 22), rn((2048,), 23, torch.float32)
    put("bias_add", x=x, bias=bias, out=tr.bias_add(x, bias))
    # head gate mul (reference test :50-68)
    out, gl = rn((1, 5, 4096), 24), rn((1, 5, 32), 25)
    gates = (2.0 * torch.sigmoid(gl.float())).to(torch.bfloat16)
    put("head_gate_mul", x=out, gates=gates, out=tr.head_gate_mul(out, gates, 32, 128))
    # FP8 quantizer: (1,) scale and 0-dim power-of-two scale, with outliers
    xq = rn((32, 512), 26)
    xq.view(-1)[torch.randperm(xq.numel(), generator=torch.Generator().manual_seed(27))[:32]] *= 50
    s1 = torch.tensor([0.0371])
    s0 = torch.tensor(0.0625)
    put("fp8_quant", x=xq, scale1=s1, q1=tr.fp8_quantize_e4m3(xq, s1), scale0=s0, q0=tr.fp8_quantize_e4m3(xq, s0))
    # Q/K RMSNorm + split RoPE (reference test :207-229 with the restatement :232-249)
    q, k = rn((1, 4, 4096), 28), rn((1, 4, 4096), 29)
    qw, kw = rn((4096,), 30), rn((4096,), 31)
    fr = rn((1, 32, 4, 64), 32, torch.float32, std=3.0)
    cos, sin = fr.cos().to(torch.bfloat16), fr.sin().to(torch.bfloat16)
    oq, ok = tr.video_qk_rmsnorm_rope(q, k, qw, kw, 1e-6, cos, sin)
    put("video_qk_rmsnorm_rope", q=q, k=k, qw=qw, kw=kw, cos=cos, sin=sin, q_out=oq, k_out=ok)
    # FP8 linear: torch._scaled_mm (CPU) + bf16 bias add
    af = rn((64, 256), 33, torch.float32)
    sa = af.abs().amax() / 448
    a = torch.clamp(af / sa, -448, 448).to(torch.float8_e4m3fn)
    wf = rn((128, 256), 34, torch.float32, std=0.02)
    sb = wf.abs().amax() / 448
    w = torch.clamp(wf / sb, -448, 448).to(torch.float8_e4m3fn)
    bias = rn((128,), 35, std=0.01)
    put("fp8_linear", a=a, w=w, scale_a=sa.reshape(()), scale_b=sb.reshape(()), bias=bias,
        out=tr.fp8_linear(a, w, sa.reshape(()), sb.reshape(()), bias))
    # per-head quantizer, one all-zero head
    xh = rn((1, 6, 32, 128), 36)
    xh[:, :, 5, :] = 0
    qh, sh = tr.fp8_per_head(xh)
    put("fp8_per_head", x=xh, q=qh, scale=sh)

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT}: {len(d)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
