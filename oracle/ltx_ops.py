"""numpy restatement of the reference's torch path for each fused op.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Each function restates
the torch expression that plugyawn/opengenie evaluates for the op, at the
precision torch uses: every elementwise op is computed in float32 and rounded
to bfloat16 wherever torch's result dtype is bfloat16 (`numerics.T` tracks
that dtype). Citations are to `ltx_serve/triton_ltx_ops.py` unless stated.

Arrays: bf16 tensors are float32 arrays holding bf16 values. Functions take
`numerics.T` values (value + dtype tag) where the reference accepts more than
one dtype, and plain arrays where it accepts only bf16.
"""

from __future__ import annotations

import numpy as np

from .numerics import (
    E4M3_MAX,
    T,
    add,
    add_scalar,
    bf16_round,
    clamp,
    e4m3_decode,
    e4m3_encode,
    f32,
    mul,
    round_to,
    sub,
)


def bf(v) -> T:
    return T(v, "bf16")


# --------------------------------------------------------------------------
# Ada values from the scale/shift table
# --------------------------------------------------------------------------
def ada_values_from_table(table: T, timestep: T, batch: int, tokens: int, cols: int, *indices: int):
    """`_torch_ada_values_from_table` (:983-998).

    timestep is (B, Nt, P*C) with Nt == tokens or Nt == 1 (a broadcast view in
    torch; the values are identical). Returns one T of shape (B, tokens, C) per
    index: `table.to(ts.dtype)[i] + ts_view[:, :, i, :]` (:997-998).
    """
    params = table.v.shape[0]
    ts = timestep.v.reshape(batch, timestep.v.shape[1], params, cols)
    ts = np.broadcast_to(ts, (batch, tokens, params, cols))
    tab = table.to(timestep.dt)
    out = []
    for i in indices:
        out.append(add(T(tab.v[i].reshape(1, 1, cols), tab.dt), T(ts[:, :, i, :], timestep.dt)))
    return tuple(out)


# --------------------------------------------------------------------------
# RMSNorm
# --------------------------------------------------------------------------
def rms_norm(x: T, eps: float, weight: T | None = None) -> T:
    """torch.nn.functional.rms_norm(x, (C,), weight, eps) for bf16 x.

    inv = 1 / sqrt(mean(x^2) + eps) in float32 with the mean taken from the
    exact sum of squares (squares of bf16 values are exact in float32; the sum
    is accumulated in float64, whose rounding error is far below float32's);
    y = x * inv [* w] in float32, rounded once to x's dtype. The single
    rounding with a weight was probed on torch 2.10 CPU.
    """
    xv = x.v.astype(np.float64)
    ss = np.sum(xv * xv, axis=-1, keepdims=True)
    cols = x.v.shape[-1]
    mean = (ss / cols).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    y = x.v * inv
    if weight is not None:
        y = y * weight.v
    return T(bf16_round(y) if x.dt == "bf16" else f32(y), x.dt)


# --------------------------------------------------------------------------
# AdaZero family
# --------------------------------------------------------------------------
def adazero(x: T, eps: float, scale: T, shift: T) -> T:
    """`fused_adazero` torch path (:9-10): rms_norm(x) * (1 + scale) + shift."""
    n = rms_norm(x, eps)
    return add(mul(n, add_scalar(scale, 1.0)), shift)


def adazero_from_ada(x: T, eps: float, table: T, timestep: T, shift_index: int, scale_index: int) -> T:
    """`fused_adazero_from_ada` torch path (:50-60)."""
    b, n, c = x.v.shape
    shift, scale = ada_values_from_table(table, timestep, b, n, c, shift_index, scale_index)
    return adazero(x, eps, scale, shift)


def adaln_affine_from_ada(x: T, table: T, timestep: T, shift_index: int, scale_index: int) -> T:
    """`fused_adaln_affine_from_ada` torch path (:102-112): x * (1 + scale) + shift."""
    b, n, c = x.v.shape
    shift, scale = ada_values_from_table(table, timestep, b, n, c, shift_index, scale_index)
    return add(mul(x, add_scalar(scale, 1.0)), shift)


def mul_from_ada(x: T, table: T, timestep: T, gate_index: int) -> T:
    """`fused_mul_from_ada` torch path (:702-711): x * gate."""
    b, n, c = x.v.shape
    (gate,) = ada_values_from_table(table, timestep, b, n, c, gate_index)
    return mul(x, gate)


# --------------------------------------------------------------------------
# Residual gates
# --------------------------------------------------------------------------
def residual_gate(x: T, y: T, gate: T) -> T:
    """`x + y * gate` (:591-592); also `_simple_residual_gate` in the production
    residual mode "triton_simple_bf16_round" (:1955-1960, :1977-1981)."""
    return add(x, mul(y, gate))


def residual_gate_from_ada(x: T, y: T, table: T, timestep: T, gate_index: int) -> T:
    """`fused_residual_gate_from_ada` torch path (:650-659)."""
    b, n, c = x.v.shape
    (gate,) = ada_values_from_table(table, timestep, b, n, c, gate_index)
    return residual_gate(x, y, gate)


def bias_add(x: T, bias: T) -> T:
    """`fused_bias_add_bf16` torch path (:186-187): x + bias.to(x.dtype)."""
    return add(x, bias.to(x.dt))


def residual_gate_bias_from_ada(x: T, y_no_bias: T, bias: T, table: T, timestep: T, gate_index: int) -> T:
    """`fused_residual_gate_bias_from_ada` torch path (:214-228)."""
    y = bias_add(y_no_bias, bias)
    return residual_gate_from_ada(x, y, table, timestep, gate_index)


def head_gate_mul(out: T, gates: T, heads: int, dim_head: int) -> T:
    """`fused_head_gate_mul_bf16` torch path (:615-619)."""
    b, n, _ = out.v.shape
    o = T(out.v.reshape(b, n, heads, dim_head), out.dt)
    g = T(gates.v.reshape(b, n, heads, 1), gates.dt)
    r = mul(o, g)
    return T(r.v.reshape(b, n, heads * dim_head), r.dt)


# --------------------------------------------------------------------------
# FP8 quantizers
# --------------------------------------------------------------------------
def fp8_quantize_e4m3(x: T, input_scale: float, scale_is_0dim: bool, device: str = "cuda") -> np.ndarray:
    """`fused_fp8_quantize_e4m3` torch path (:146-148) -> uint8 e4m3fn codes.

    clamp(x * input_scale.reciprocal(), -448, 448).to(float8_e4m3fn), with
    r = float32(1 / s), x bf16 or fp16 (the reference's guard takes both,
    :1021-1022). Dtype of `x * r`: a 0-dim scale does not promote, so the
    product has x's dtype (rounded to it); a (1,)-shaped scale makes it
    float32. On a GPU the 0-dim float32 operand is itself converted to the
    common dtype (x's) before the multiply (TensorIterator casts
    non-CPU-scalar inputs to the common dtype); a 0-dim CPU tensor is read at
    full float32 precision. `device` selects which of the two the
    restatement follows.
    """
    r = np.float32(1.0) / np.float32(input_scale)
    if scale_is_0dim:
        rv = round_to(r, x.dt) if device == "cuda" else f32(r)
        with np.errstate(over="ignore", invalid="ignore"):
            y = T(round_to(x.v * rv, x.dt), x.dt)
    else:
        y = T(x.v * r, "f32")
    y = clamp(y, -E4M3_MAX, E4M3_MAX)
    return e4m3_encode(y.v)


def gelu_tanh(x: T) -> T:
    """torch.nn.functional.gelu(x, approximate='tanh') for bf16 or fp16 x, step
    by step as torch's GPU kernel evaluates it in float32 (the reference's
    torch path :165-169 on the GPU):

        x3 = (x * x) * x;  inner = beta * fma(kappa, x3, x);
        g = (0.5 * x) * (1 + tanh(inner)), rounded once to x's dtype,

    beta = float32(sqrt(2) * 2/sqrt(pi) * 0.5), kappa = float32(0.044715).
    The fused multiply-add is evaluated in extended precision (the product
    kappa * x3 is exact there) and rounded once to float32; tanh is the
    float64 tanh rounded to float32. Pinned exhaustively (all 65536 bf16
    inputs) against torch's gelu on the GPU by a GPU test."""
    v = x.v.astype(np.float32)
    beta = np.float32(np.sqrt(2.0) * (2.0 / np.sqrt(np.pi)) * 0.5)
    kappa = np.float32(0.044715)
    with np.errstate(over="ignore", invalid="ignore"):
        x3 = (v * v) * v
        ld = np.longdouble
        inner = beta * (ld(kappa) * ld(x3) + ld(v)).astype(np.float32)
        t = np.tanh(inner.astype(np.float64)).astype(np.float32)
        g = (np.float32(0.5) * v) * (np.float32(1.0) + t)
    g = g.astype(np.float32)
    return T(round_to(g, x.dt), x.dt)


def fp8_per_head_quantize(x: np.ndarray, device: str = "cuda"):
    """`_torch_fp8_quantize_e4m3_per_head_4d` (:976-980) for x [B, N, H, D].

    amax = max_{N,D} |x| (NaN if any element of the head is NaN, as torch's
    amax gives); scale[b, h] = clamp_min(amax, 1e-12) / 448; q =
    e4m3(clamp(x / scale, -448, 448)) with an IEEE float32 division.
    `/ 448` divides a tensor by a Python scalar: on the GPU torch evaluates
    that as a multiplication by the float32 reciprocal (`device="cuda"`,
    the production device), on the CPU as a division (`device="cpu"`); the
    two differ in the last bit of some scales.
    Returns (codes uint8 [B,N,H,D], scale float32 [B,H]).
    """
    xv = f32(x)
    amax = np.abs(xv).max(axis=(1, 3)).astype(np.float32)
    clamped = np.maximum(amax, np.float32(1e-12))
    if device == "cuda":
        scale = clamped * (np.float32(1.0) / np.float32(E4M3_MAX))
    else:
        scale = clamped / np.float32(E4M3_MAX)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = xv / scale[:, None, :, None]
        q = np.minimum(np.maximum(q, np.float32(-E4M3_MAX)), np.float32(E4M3_MAX))
    return e4m3_encode(q), scale.astype(np.float32)


# --------------------------------------------------------------------------
# FP8 linear
# --------------------------------------------------------------------------
def fp8_scaled_mm(a_codes: np.ndarray, w_codes: np.ndarray, scale_a: float, scale_b: float,
                  out_dt: str = "bf16") -> np.ndarray:
    """torch._scaled_mm(a, w.t(), scale_a, scale_b, out_dtype=bf16 or fp16).

    a [M, K] and w [N, K] are e4m3fn codes. The products of two e4m3 values
    are exact; the sum is taken in float64, scaled by scale_a*scale_b, rounded
    to float32 and then to the output dtype `out_dt` ('bf16' or 'f16'; an
    fp16 FP8Linear passes out_dtype=x.dtype, :1697-1709). Matches a
    float32-accumulating GEMM up to its accumulation rounding (the parity
    bar is a few output steps).
    """
    a = e4m3_decode(a_codes).astype(np.float64)
    w = e4m3_decode(w_codes).astype(np.float64)
    acc = a @ w.T
    out = (acc * (float(np.float32(scale_a)) * float(np.float32(scale_b)))).astype(np.float32)
    return round_to(out, out_dt)


def fp8_linear(a_codes, w_codes, scale_a, scale_b, bias: T | None, out_dt: str = "bf16") -> np.ndarray:
    """Patched `FP8Linear.forward` (:1691-1709): _scaled_mm, then `+ bias` in
    the output dtype (R(out + R(bias)), `fused_bias_add_bf16` /
    `output + bias.to(output.dtype)`, :742-760)."""
    out = fp8_scaled_mm(a_codes, w_codes, scale_a, scale_b, out_dt)
    if bias is None:
        return out
    return bias_add(T(out, out_dt), bias).v


def fp8_requantize_common_scale(w_codes: np.ndarray, w_scale: float, common: float) -> np.ndarray:
    """`_get_video_qkv_packed_requant_cache._requant` (:1331-1333): the e4m3
    weight dequantized with its own scale and requantized to the common one,
    clamp(float32(W) * w_scale / common, -448, 448).to(float8_e4m3fn), with a
    float32 product and an IEEE float32 division (both scales are tensors, so
    neither operation takes torch's scalar shortcut)."""
    deq = e4m3_decode(w_codes).astype(np.float32) * np.float32(w_scale)
    with np.errstate(invalid="ignore", over="ignore"):
        r = deq / np.float32(common)
    r = np.where(np.isnan(r), r, np.minimum(np.maximum(r, np.float32(-E4M3_MAX)), np.float32(E4M3_MAX)))
    return e4m3_encode(r.astype(np.float32))


# --------------------------------------------------------------------------
# Video Q/K preattention
# --------------------------------------------------------------------------
def split_rope(x: T, cos: T, sin: T) -> T:
    """Split RoPE as restated by the reference's test
    (tests/test_triton_ltx_ops.py:232-249): per head, first half f and second
    half s: [f*cos - s*sin, s*cos + f*sin], each torch op rounded per dtype.
    x is (B, N, H*D); cos/sin are (B or 1, H, N, D/2)."""
    b, n, dim = x.v.shape
    heads = cos.v.shape[1]
    hd = dim // heads
    half = hd // 2
    xh = x.v.reshape(b, n, heads, hd).transpose(0, 2, 1, 3)
    first = T(xh[..., :half], x.dt)
    second = T(xh[..., half:], x.dt)
    out_first = sub(mul(first, cos), mul(second, sin))
    out_second = add(mul(second, cos), mul(first, sin))
    dt = out_first.dt
    o = np.concatenate([out_first.v, out_second.v], axis=-1).transpose(0, 2, 1, 3).reshape(b, n, dim)
    return T(o, dt)


def video_qk_rmsnorm_rope(q: T, k: T, q_weight: T, k_weight: T, eps: float, cos: T, sin: T):
    """`_torch_video_qk_rmsnorm_rope` (:958-973) with the split RoPE of the
    reference test restatement (ltx_core's apply_rotary_emb is not vendored)."""
    qn = rms_norm(q, eps, q_weight)
    kn = rms_norm(k, eps, k_weight)
    return split_rope(qn, cos, sin), split_rope(kn, cos, sin)


def video_qk_bias_rmsnorm_rope(q: T, k: T, q_bias: T, k_bias: T, q_weight: T, k_weight: T, eps, cos, sin):
    """`fused_video_qk_bias_rmsnorm_rope` torch path (:519-522)."""
    return video_qk_rmsnorm_rope(bias_add(q, q_bias), bias_add(k, k_bias), q_weight, k_weight, eps, cos, sin)


def video_qkv_rmsnorm_rope_pack(q: T, k: T, v: T, q_weight: T, k_weight: T, eps, cos, sin) -> np.ndarray:
    """`fused_video_qkv_rmsnorm_rope_pack` (:381-429): [B, N, 3, H, D] of
    (rope(q), rope(k), v)."""
    qo, ko = video_qk_rmsnorm_rope(q, k, q_weight, k_weight, eps, cos, sin)
    b, n, dim = q.v.shape
    heads = cos.v.shape[1]
    return np.stack([qo.v, ko.v, v.v], axis=2).reshape(b, n, 3, heads, dim // heads)


# --------------------------------------------------------------------------
# Dense attention
# --------------------------------------------------------------------------
def fp8_dequant_per_head(codes: np.ndarray, descale: np.ndarray) -> np.ndarray:
    """e4m3 codes [B, N, H, D] times float32 descale [B, H], rounded to bf16
    (the dequantization of FP8 attention inputs, official_ltx23_benchmark.py
    :3333-3340 descales): R(float32(e4m3) * descale)."""
    v = e4m3_decode(codes) * f32(descale)[:, None, :, None]
    return bf16_round(f32(v))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    """softmax(q k^T * scale) v in float64 for [B, H, N, D] arrays (non-causal)."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    d = q.shape[-1]
    s = (q @ np.swapaxes(k, -1, -2)) * (scale if scale is not None else d ** -0.5)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return p @ v
