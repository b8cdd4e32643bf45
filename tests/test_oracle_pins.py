"""Pins for the numpy oracle (CPU only).

Each oracle function is checked against something independent of it: torch
executing the reference's own expression on the CPU (tests/torch_reference.py),
torch's own dtype conversions, closed forms and invariants. Shapes and Ada
indices follow the reference's tests (tests/test_triton_ltx_ops.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.torch_ref as tr
from oracle import ltx_ops as O
from oracle.numerics import T, bf16_from_bits, bf16_round, e4m3_decode, e4m3_encode, f16_from_bits, f16_round
from tests.helpers import (assert_same_bits, bf16_step, bf16_ulp_distance, f16_ulp_distance, nan_canon, np32,
                           randn, to_T)


# ----------------------------------------------------------------- numerics
def test_bf16_round_matches_torch_on_random_and_edge_bits():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=1 << 21, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x00008000, 0x80008000, 0x3F808000,
                      0x3F818000, 0x3F80FFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001],
                     dtype=np.uint32)
    a = np.concatenate([bits, edges]).view(np.float32)
    ours = bf16_round(a)
    ref = torch.from_numpy(a.copy()).to(torch.bfloat16).float().numpy()
    assert_same_bits(ours, ref, "bf16_round")


def test_f16_round_matches_torch_on_random_and_edge_bits():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2 ** 32, size=1 << 21, dtype=np.uint64).astype(np.uint32)
    # around the largest finite half (65504), its overflow midpoint (65520),
    # the subnormal range (2^-24 quantum) and ties at both
    edges = np.array([0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FF001, 0x33800000, 0x33000000, 0x33000001,
                      0x33C00000, 0x38800000, 0x387FC000, 0x387FE000, 0x3F801000, 0x3F803000, 0x7F800000,
                      0xFF800000, 0x7FC00000, 0x00000001, 0x80000001], dtype=np.uint32)
    a = np.concatenate([bits, edges]).view(np.float32)
    ours = f16_round(a)
    ref = torch.from_numpy(a.copy()).to(torch.float16).float().numpy()
    assert_same_bits(ours, ref, "f16_round")


def test_e4m3_encode_matches_torch_exhaustively_over_f16():
    x = f16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    ours = e4m3_encode(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(nan_canon(ours), nan_canon(ref))


def test_e4m3_encode_matches_torch_exhaustively_over_bf16():
    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    ours = e4m3_encode(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(nan_canon(ours), nan_canon(ref))


def test_e4m3_encode_matches_torch_on_float32_boundaries():
    # Every e4m3 value and the float32 neighbours of every midpoint between
    # consecutive e4m3 values (the cases a wrong tie rule or exponent fails).
    vals = e4m3_decode(np.arange(256, dtype=np.uint8))
    fin = np.sort(np.unique(vals[np.isfinite(vals)]))
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                           fin, np.float32([464, 479.99997, 480, 1e30, np.inf, -np.inf, 2.0 ** -10, 2.0 ** -11])])
    near = np.concatenate([near, -near]).astype(np.float32)
    rng = np.random.default_rng(2)
    rnd = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = np.concatenate([near, rnd])
    ours = e4m3_encode(a)
    ref = torch.from_numpy(a.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    assert_same_bits(e4m3_decode(codes), ref, "e4m3_decode")


# ----------------------------------------------------------------- rms_norm
@pytest.mark.parametrize("with_weight", [False, True])
def test_rms_norm_matches_torch_within_one_ulp(with_weight):
    x = randn((64, 4096), 11)
    w = randn((4096,), 12, std=0.05, mean=1.0) if with_weight else None
    ref = torch.nn.functional.rms_norm(x, (4096,), weight=w, eps=1e-6)
    ours = O.rms_norm(to_T(x), 1e-6, to_T(w) if w is not None else None)
    d = bf16_ulp_distance(ours.v, np32(ref))
    assert d.max() <= 1
    # torch's float32 reduction order is its own; disagreement must be rare.
    assert (d > 0).mean() < 1e-3


def test_rms_norm_closed_form_constant_rows():
    # A row of constant c has mean c^2: the output is c / sqrt(c^2 + eps).
    c = np.float32([0.5, 1.0, 3.0, -2.0, 0.0078125])
    x = np.repeat(c[:, None], 2048, axis=1).astype(np.float32)
    out = O.rms_norm(T(x, "bf16"), 1e-6)
    expect = bf16_round(c / np.sqrt(np.float32(c * c + np.float32(1e-6))))
    assert_same_bits(out.v[:, 0], expect, "constant rows")


# ----------------------------------------------------------------- Ada family
def _ada_inputs(seed, rows=9, cols=2048, params=6, table_dtype=torch.float32, ts_dtype=torch.bfloat16,
                broadcast=False):
    x = randn((1, rows, cols), seed)
    table = randn((params, cols), seed + 1, dtype=table_dtype)
    ts_rows = 1 if broadcast else rows
    ts = randn((1, ts_rows, params * cols), seed + 2, dtype=ts_dtype)
    if broadcast:
        ts = ts.expand(1, rows, params * cols)
    return x, table, ts


@pytest.mark.parametrize("table_dtype,ts_dtype", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                                  (torch.bfloat16, torch.float32), (torch.float32, torch.float32)])
def test_ada_values_match_torch(table_dtype, ts_dtype):
    x, table, ts = _ada_inputs(20, table_dtype=table_dtype, ts_dtype=ts_dtype)
    ref = tr.ada_values(table, ts, 1, 9, 2048, 3, 4)
    ours = O.ada_values_from_table(to_T(table), to_T(ts), 1, 9, 2048, 3, 4)
    for r, o in zip(ref, ours):
        assert_same_bits(o.v, np32(r), "ada value")


@pytest.mark.parametrize("table_dtype,ts_dtype,broadcast", [
    (torch.float32, torch.bfloat16, False), (torch.bfloat16, torch.bfloat16, True),
    (torch.bfloat16, torch.bfloat16, False), (torch.float32, torch.float32, False)])
def test_adazero_from_ada_matches_torch(table_dtype, ts_dtype, broadcast):
    x, table, ts = _ada_inputs(2, table_dtype=table_dtype, ts_dtype=ts_dtype, broadcast=broadcast)
    ref = tr.adazero_from_ada(x, 1e-6, table, ts, 3, 4)
    ours = O.adazero_from_ada(to_T(x), 1e-6, to_T(table), to_T(ts), 3, 4)
    assert ours.dt == ("bf16" if ref.dtype == torch.bfloat16 else "f32")
    d = bf16_ulp_distance(bf16_round(ours.v), bf16_round(np32(ref)))
    # Only the float32 sum of squares can differ from torch's; rare and small.
    assert (d > 0).mean() < 2e-3
    shift, scale = O.ada_values_from_table(to_T(table), to_T(ts), 1, 9, 2048, 3, 4)
    _adazero_differs_only_in_the_norm(x, scale, shift, ref)


def _adazero_differs_only_in_the_norm(x, scale: T, shift: T, ref: torch.Tensor) -> None:
    """Every difference between the oracle and torch comes from the RMSNorm
    step: the oracle's normalized row is within one bf16 step of torch's
    rms_norm, and the oracle's remaining steps, R(R(n * R(1 + scale)) +
    shift), applied to torch's own normalized row give torch's output bit for
    bit (so no element can be off by more than that one step carried through
    the two roundings)."""
    n_t = torch.nn.functional.rms_norm(x, (x.shape[-1],), eps=1e-6)
    assert bf16_ulp_distance(O.rms_norm(to_T(x), 1e-6).v, np32(n_t)).max() <= 1
    tail = O.add(O.mul(to_T(n_t), O.add_scalar(scale, 1.0)), shift)
    assert_same_bits(bf16_round(tail.v) if tail.dt == "bf16" else tail.v, np32(ref), "AdaZero after the norm")


def test_adazero_with_strided_scale_shift_matches_torch():
    # Reference test :8-26: scale/shift are stride-3 views of a (1,7,3,C) tensor.
    x = randn((1, 7, 2048), 0)
    ss = randn((1, 7, 3, 2048), 1)
    scale, shift = ss[:, :, 1, :], ss[:, :, 2, :]
    ref = tr.adazero(x, 1e-6, scale, shift)
    ours = O.adazero(to_T(x), 1e-6, to_T(scale), to_T(shift))
    assert (bf16_ulp_distance(ours.v, np32(ref)) > 0).mean() < 2e-3
    _adazero_differs_only_in_the_norm(x, to_T(scale), to_T(shift), ref)


@pytest.mark.parametrize("ts_dtype", [torch.bfloat16, torch.float32])
def test_adaln_affine_from_ada_matches_torch_exactly(ts_dtype):
    x, table, ts = _ada_inputs(4, params=9, ts_dtype=ts_dtype)
    ref = tr.adaln_affine_from_ada(x, table, ts, 6, 7)
    ours = O.adaln_affine_from_ada(to_T(x), to_T(table), to_T(ts), 6, 7)
    assert_same_bits(ours.v, np32(ref), "adaln_affine")


def test_mul_from_ada_matches_torch_exactly():
    x, table, ts = _ada_inputs(5, params=9)
    assert_same_bits(O.mul_from_ada(to_T(x), to_T(table), to_T(ts), 8).v,
                     np32(tr.mul_from_ada(x, table, ts, 8)), "mul_from_ada")


def test_residual_gate_from_ada_matches_torch_exactly():
    x, table, ts = _ada_inputs(3)
    y = randn((1, 9, 2048), 33)
    assert_same_bits(O.residual_gate_from_ada(to_T(x), to_T(y), to_T(table), to_T(ts), 5).v,
                     np32(tr.residual_gate_from_ada(x, y, table, ts, 5)), "residual_gate_from_ada")


def test_residual_gate_strided_gate_matches_torch_exactly():
    x = randn((1, 7, 2048), 1)
    y = randn((1, 7, 2048), 2)
    gate = randn((1, 7, 3, 2048), 3)[:, :, 1, :]
    assert_same_bits(O.residual_gate(to_T(x), to_T(y), to_T(gate)).v, np32(tr.residual_gate(x, y, gate)), "gate")


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16])
def test_bias_add_matches_torch_exactly(bias_dtype):
    x = randn((11, 2048), 6)
    bias = randn((2048,), 7, dtype=bias_dtype)
    assert_same_bits(O.bias_add(to_T(x), to_T(bias)).v, np32(tr.bias_add(x, bias)), "bias_add")


def test_residual_gate_bias_from_ada_matches_torch_exactly():
    x, table, ts = _ada_inputs(7, params=9)
    y = randn((1, 9, 2048), 71)
    bias = randn((2048,), 72, dtype=torch.float32)
    ref = tr.residual_gate_bias_from_ada(x, y, bias, table, ts, 8)
    ours = O.residual_gate_bias_from_ada(to_T(x), to_T(y), to_T(bias), to_T(table), to_T(ts), 8)
    assert_same_bits(ours.v, np32(ref), "residual_gate_bias_from_ada")


def test_head_gate_mul_matches_torch_exactly():
    out = randn((1, 13, 4096), 11)
    gates = (2.0 * torch.sigmoid(randn((1, 13, 32), 12))).to(torch.bfloat16)
    assert_same_bits(O.head_gate_mul(to_T(out), to_T(gates), 32, 128).v,
                     np32(tr.head_gate_mul(out, gates, 32, 128)), "head_gate_mul")


# ----------------------------------------------------------------- FP8 quant
@pytest.mark.parametrize("scale", [0.05, 0.37, 1.0, 3.3e-3, 0.11160714])
@pytest.mark.parametrize("zero_dim", [True, False])
def test_fp8_quantize_matches_torch_cpu_exhaustively(scale, zero_dim):
    # Every bf16 bit pattern, for a 0-dim and a (1,) scale (CPU semantics).
    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    xt = torch.from_numpy(x.copy()).to(torch.bfloat16)
    s = torch.tensor(scale, dtype=torch.float32)
    if not zero_dim:
        s = s.reshape(1)
    ref = tr.fp8_quantize_e4m3(xt, s).view(torch.uint8).numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        ours = O.fp8_quantize_e4m3(T(x, "bf16"), float(s.reshape(())), zero_dim, device="cpu")
    assert np.array_equal(nan_canon(ours), nan_canon(ref))


@pytest.mark.parametrize("scale", [0.05, 0.37, 1.0, 3.3e-3, 2.0e-5])
@pytest.mark.parametrize("zero_dim", [True, False])
def test_fp8_quantize_f16_matches_torch_cpu_exhaustively(scale, zero_dim):
    """Every fp16 bit pattern (the reference's guard takes fp16 x too,
    :1021-1022): the product has x's dtype for a 0-dim scale, float32 for a
    (1,) one. 2e-5 makes 1/s overflow fp16's range (CPU semantics keep the
    float32 reciprocal)."""
    x = f16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    xt = torch.from_numpy(x.copy()).to(torch.float16)
    s = torch.tensor(scale, dtype=torch.float32)
    if not zero_dim:
        s = s.reshape(1)
    ref = tr.fp8_quantize_e4m3(xt, s).view(torch.uint8).numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        ours = O.fp8_quantize_e4m3(T(x, "f16"), float(s.reshape(())), zero_dim, device="cpu")
    assert np.array_equal(nan_canon(ours), nan_canon(ref))


def test_fp8_quantize_gpu_semantics_differs_only_by_rounded_reciprocal():
    # With a reciprocal that is already a bf16 value the CPU and GPU forms agree.
    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    with np.errstate(over="ignore", invalid="ignore"):
        a = O.fp8_quantize_e4m3(T(x, "bf16"), 0.25, True, device="cuda")
        b = O.fp8_quantize_e4m3(T(x, "bf16"), 0.25, True, device="cpu")
    assert np.array_equal(a, b)


def test_fp8_per_head_matches_torch():
    x = randn((2, 33, 4, 64), 40)
    x[1, :, 2, :] = 0  # an all-zero head takes the 1e-12 clamp
    qref, sref = tr.fp8_per_head(x)
    q, s = O.fp8_per_head_quantize(np32(x), device="cpu")
    assert_same_bits(s, sref.numpy(), "per-head scale")
    assert np.array_equal(q, qref.view(torch.uint8).numpy())


def test_gelu_tanh_matches_torch_cpu_on_every_bf16():
    """All 65536 bf16 inputs: the oracle's float32 GELU steps equal torch's CPU
    gelu(approximate='tanh') except where torch's vectorised CPU tanh returns
    exactly -1 for an argument whose correctly rounded tanh is -(1 - 2^-24):
    there torch's GELU is -0 and the oracle's a tiny negative value (x in
    [-5.16, -5.06], four inputs). The GPU test pins the oracle against torch's
    GPU kernel, whose tanhf does not saturate there."""
    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    g = O.gelu_tanh(T(x, "bf16")).v
    ref = torch.nn.functional.gelu(torch.from_numpy(x.copy()).to(torch.bfloat16), approximate="tanh").float().numpy()
    eq = (g.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(g) & np.isnan(ref))
    bad = np.flatnonzero(~eq)
    assert bad.size <= 4, bad.size
    assert np.all((x[bad] > -5.2) & (x[bad] < -5.0)) and np.all(ref[bad] == 0) and np.all(np.abs(g[bad]) < 2e-7)


def test_gelu_tanh_matches_torch_cpu_on_every_f16():
    """All 65536 fp16 inputs against torch's CPU gelu(approximate='tanh') in
    fp16 (float32 steps, one rounding to fp16). As for bf16, the only
    differences are where torch's vectorised CPU tanh returns exactly -1 for
    an argument whose correctly rounded tanh is -(1 - 2^-24): torch's GELU is
    -0 there and the oracle's a tiny negative value (x in [-5.16, -5.06]).
    The GPU test pins the oracle against torch's GPU kernel on every input."""
    x = f16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    g = O.gelu_tanh(T(x, "f16")).v
    ref = torch.nn.functional.gelu(torch.from_numpy(x.copy()).to(torch.float16), approximate="tanh").float().numpy()
    eq = (g.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(g) & np.isnan(ref))
    bad = np.flatnonzero(~eq)
    assert bad.size <= 32, bad.size
    assert np.all((x[bad] > -5.2) & (x[bad] < -5.0)) and np.all(ref[bad] == 0) and np.all(np.abs(g[bad]) < 2e-7)


def test_gelu_tanh_fp8_matches_torch_cpu():
    x = randn((8, 2048), 41, std=2.0)
    s = torch.tensor(0.02)
    ref = tr.gelu_tanh_fp8_quantize_e4m3(x, s).view(torch.uint8).numpy()
    ours = O.fp8_quantize_e4m3(O.gelu_tanh(to_T(x)), 0.02, True, device="cpu")
    assert np.array_equal(ours, ref)


# ----------------------------------------------------------------- FP8 linear
def _fp8_codes(shape, seed, std):
    v = randn(shape, seed, dtype=torch.float32, std=std)
    s = v.abs().amax() / 448.0
    return torch.clamp(v / s, -448, 448).to(torch.float8_e4m3fn), float(s)


def test_fp8_scaled_mm_matches_torch_scaled_mm_cpu():
    a, sa = _fp8_codes((48, 256), 50, 1.0)
    w, sb = _fp8_codes((80, 256), 51, 0.02)
    bias = randn((80,), 52, std=0.01)
    ref = tr.fp8_linear(a, w, torch.tensor(sa), torch.tensor(sb), bias)
    ours = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), sa, sb, to_T(bias))
    np.testing.assert_allclose(ours, np32(ref), rtol=1e-2, atol=1e-3)
    assert (bf16_ulp_distance(ours, np32(ref)) > 1).mean() < 1e-3


def test_fp8_scaled_mm_fp16_matches_torch_scaled_mm_cpu():
    """An fp16 FP8Linear (out_dtype = x.dtype): _scaled_mm to fp16, then
    `+ bias.to(fp16)`; the same oracle with bf16 rounding must not pass."""
    a, sa = _fp8_codes((48, 256), 54, 1.0)
    w, sb = _fp8_codes((80, 256), 55, 0.02)
    bias = randn((80,), 56, std=0.01)
    ref = np32(tr.fp8_linear(a, w, torch.tensor(sa), torch.tensor(sb), bias, out_dtype=torch.float16))
    args = (a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), sa, sb, to_T(bias))
    ours = O.fp8_linear(*args, out_dt="f16")
    assert np.array_equal(ours, f16_round(ours))
    d = f16_ulp_distance(ours, ref)
    assert d.max() <= 1 and (d > 0).mean() < 0.02, (d.max(), (d > 0).mean())
    assert (f16_ulp_distance(O.fp8_linear(*args), ref) > 1).mean() > 0.5


def test_fp8_scaled_mm_brute_force_tiny():
    rng = np.random.default_rng(53)
    a = rng.integers(0, 256, size=(3, 16), dtype=np.uint8)
    w = rng.integers(0, 256, size=(5, 16), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0x01  # no NaN codes
    w[(w & 0x7F) == 0x7F] = 0x02
    out = O.fp8_scaled_mm(a, w, 0.5, 0.25)
    av, wv = e4m3_decode(a).astype(np.float64), e4m3_decode(w).astype(np.float64)
    for i in range(3):
        for j in range(5):
            s = sum(av[i, k] * wv[j, k] for k in range(16)) * 0.125
            assert out[i, j] == bf16_round(np.float32(s))
    bias = np.float32([3.0e-3, -7.1e-2, 1.9e-4, 0.5, -2.25])
    out16 = O.fp8_linear(a, w, 0.5, 0.25, T(bf16_round(bias), "bf16"), out_dt="f16")
    for i in range(3):
        for j in range(5):
            s = sum(av[i, k] * wv[j, k] for k in range(16)) * 0.125
            r = np.float16(np.float32(s))
            assert out16[i, j] == np.float32(np.float16(np.float32(r) + np.float32(np.float16(bf16_round(bias)[j]))))


# ----------------------------------------------------------------- Q/K RoPE
def _rope_inputs(seed, tokens=17, cos_dtype=torch.bfloat16):
    q = randn((1, tokens, 4096), seed)
    k = randn((1, tokens, 4096), seed + 1)
    qw = randn((4096,), seed + 2)
    kw = randn((4096,), seed + 3)
    freqs = randn((1, 32, tokens, 64), seed + 4, dtype=torch.float32)
    return q, k, qw, kw, freqs.cos().to(cos_dtype), freqs.sin().to(cos_dtype)


@pytest.mark.parametrize("cos_dtype", [torch.bfloat16, torch.float32])
def test_video_qk_rmsnorm_rope_matches_torch(cos_dtype):
    q, k, qw, kw, cos, sin = _rope_inputs(8, cos_dtype=cos_dtype)
    rq, rk = tr.video_qk_rmsnorm_rope(q, k, qw, kw, 1e-6, cos, sin)
    oq, ok = O.video_qk_rmsnorm_rope(to_T(q), to_T(k), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    for x, w, o, r in ((q, qw, oq, rq), (k, kw, ok, rk)):
        d = bf16_ulp_distance(bf16_round(o.v), bf16_round(np32(r)))
        assert (d > 0).mean() < 2e-3
        # every difference comes from the RMSNorm step: the normalized rows
        # are within one bf16 step, and the oracle's split RoPE of torch's own
        # normalized row is torch's output bit for bit
        n_t = torch.nn.functional.rms_norm(x, (4096,), weight=w, eps=1e-6)
        assert bf16_ulp_distance(O.rms_norm(to_T(x), 1e-6, to_T(w)).v, np32(n_t)).max() <= 1
        rot = O.split_rope(to_T(n_t), to_T(cos), to_T(sin))
        assert_same_bits(rot.v, np32(r), "split RoPE after the norm")


def test_split_rope_invariants():
    x = T(np32(randn((1, 5, 4096), 60)), "bf16")
    one = T(np.ones((1, 32, 5, 64), np.float32), "bf16")
    zero = T(np.zeros((1, 32, 5, 64), np.float32), "bf16")
    assert_same_bits(O.split_rope(x, one, zero).v, x.v, "identity rotation")
    quarter = O.split_rope(x, zero, one).v.reshape(1, 5, 32, 128)
    xh = x.v.reshape(1, 5, 32, 128)
    assert_same_bits(quarter[..., :64], -xh[..., 64:], "quarter turn, first half")
    assert_same_bits(quarter[..., 64:], xh[..., :64], "quarter turn, second half")


# ----------------------------------------------------------------- attention
def test_attention_matches_torch_sdpa_float64():
    q = randn((1, 2, 37, 64), 70, dtype=torch.float64)
    k = randn((1, 2, 37, 64), 71, dtype=torch.float64)
    v = randn((1, 2, 37, 64), 72, dtype=torch.float64)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v).numpy()
    np.testing.assert_allclose(O.attention(q.numpy(), k.numpy(), v.numpy()), ref, rtol=1e-10, atol=1e-12)


def test_attention_closed_forms():
    """One key: every query returns that key's value. Identical keys: the
    softmax is uniform, so every query returns the mean of the values."""
    rng = np.random.default_rng(73)
    q = rng.standard_normal((2, 3, 11, 64))
    v1 = rng.standard_normal((2, 3, 1, 64))
    k1 = rng.standard_normal((2, 3, 1, 64))
    np.testing.assert_allclose(O.attention(q, k1, v1), np.broadcast_to(v1, q.shape), rtol=0, atol=1e-14)
    k = np.repeat(rng.standard_normal((2, 3, 1, 64)), 9, axis=2)
    v = rng.standard_normal((2, 3, 9, 64))
    np.testing.assert_allclose(O.attention(q, k, v), np.broadcast_to(v.mean(axis=2, keepdims=True), q.shape),
                               rtol=1e-12, atol=1e-12)


def test_fp8_dequant_per_head_matches_torch():
    """codes x descale with one rounding, against torch's own e4m3 decode."""
    rng = np.random.default_rng(74)
    codes = rng.integers(0, 256, size=(2, 5, 3, 16), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # skip the NaN encodings
    descale = (rng.random((2, 3)) * 0.1 + 1e-3).astype(np.float32)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    ref = (t * torch.from_numpy(descale)[:, None, :, None]).to(torch.bfloat16).float().numpy()
    got = O.fp8_dequant_per_head(codes, descale)
    np.testing.assert_array_equal(np.asarray(got, dtype=np.float32), ref)


def test_fp8_requantize_common_scale_matches_torch():
    """Every e4m3 code (NaN included) requantized from several weight scales to
    common scales at and above them, against torch's expression (:1331-1333)."""
    codes = np.arange(256, dtype=np.uint8)
    w = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn)
    for ws in (3.1e-5, 4.4643e-05, 1.0e-3, 0.37):
        for ratio in (1.0, 1.37, 2.0, 7.91, 300.0):
            cs = np.float32(ws) * np.float32(ratio)
            ref = tr.fp8_requantize_common_scale(w, torch.tensor(ws, dtype=torch.float32),
                                                 torch.tensor(float(cs), dtype=torch.float32))
            ours = O.fp8_requantize_common_scale(codes, ws, float(cs))
            assert np.array_equal(nan_canon(ours), nan_canon(ref.view(torch.uint8).numpy())), (ws, ratio)
