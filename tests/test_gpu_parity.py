"""GPU parity: each HIP op against the numpy oracle on identical seeded inputs.

Inputs are drawn on the CPU with a seeded torch.Generator and copied to the
GPU, so the oracle and the kernel see the same bits. Bar: bit-exact for every
elementwise op and the FP8 codes; bf16 outputs of the RMS ops bit-exact
(the kernel and the oracle both take the mean from the exact sum of squares);
the FP8 GEMM within rtol 1e-2 (float32 accumulation order differs).
Every test runs with OPENGENIE_AMD_STRICT=1 and checks the HIP path ran.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.torch_ref as tr
from oracle import ltx_ops as O
from oracle.numerics import T, bf16_from_bits, bf16_round, e4m3_decode, e4m3_encode, f16_round
from tests.helpers import assert_same_bits, bf16_ulp_distance, f16_ulp_distance, nan_canon, np32, randn, to_T

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _strict(monkeypatch):
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    from opengenie_amd import ltx_ops

    ltx_ops.reset_hip_calls()
    yield


def _ran(name: str) -> None:
    from opengenie_amd import ltx_ops

    assert ltx_ops.collect_hip_calls().get(name, 0) > 0, f"{name} did not take the HIP path"


def g(t: torch.Tensor) -> torch.Tensor:
    return t.to(DEV)


def out_np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


# ------------------------------------------------------------ conversions
def test_selftest_conversions_match_oracle():
    """The device rounding primitives every kernel uses, bit by bit."""
    from opengenie_amd import _lib

    rng = np.random.default_rng(100)
    a = np.concatenate([
        rng.integers(0, 2 ** 32, size=1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32),
        bf16_from_bits(np.arange(1 << 16, dtype=np.uint16)),
        e4m3_decode(np.arange(256, dtype=np.uint8)),
    ]).astype(np.float32)
    # e4m3 midpoints and their float32 neighbours
    fin = np.unique(e4m3_decode(np.arange(256, dtype=np.uint8)))
    fin = fin[np.isfinite(fin)]
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    a = np.concatenate([a, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    x = torch.from_numpy(a).to(DEV)
    bo = torch.empty(a.size, dtype=torch.int16, device=DEV)
    eo = torch.empty(a.size, dtype=torch.uint8, device=DEV)
    _lib.call("oga_selftest_convert", x.data_ptr(), bo.data_ptr(), eo.data_ptr(), a.size,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got_b = bo.cpu().numpy().view(np.uint16)
    want_b = (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    assert np.array_equal(got_b[~nan], want_b[~nan])
    assert np.all((got_b[nan] & 0x7F80) == 0x7F80) and np.all(got_b[nan] & 0x7F)
    with np.errstate(invalid="ignore"):
        clamped = np.where(nan, a, np.clip(a, -448, 448)).astype(np.float32)
    assert np.array_equal(nan_canon(eo.cpu().numpy()), nan_canon(e4m3_encode(clamped)))


# ------------------------------------------------------------ Ada family
def _ada(seed, rows, cols, params, table_dtype, ts_dtype, broadcast=False, batch=1):
    x = randn((batch, rows, cols), seed)
    table = randn((params, cols), seed + 1, dtype=table_dtype, std=0.02 if table_dtype == torch.bfloat16 else 1.0)
    ts_rows = 1 if broadcast else rows
    ts = randn((batch, ts_rows, params * cols), seed + 2, dtype=ts_dtype, std=0.5)
    tsg = g(ts)
    if broadcast:
        tsg = tsg.expand(batch, rows, params * cols)
        ts = ts.expand(batch, rows, params * cols)
    return x, table, ts, g(x), g(table), tsg


ADA_CASES = [
    # rows, cols, params, table dtype, ts dtype, broadcast, batch
    (9, 2048, 6, torch.float32, torch.bfloat16, False, 1),   # reference test shape
    (9, 2048, 9, torch.float32, torch.bfloat16, False, 1),
    (33, 4096, 6, torch.bfloat16, torch.bfloat16, True, 1),  # uniform timestep row
    (17, 4096, 9, torch.bfloat16, torch.bfloat16, False, 2),
    (5, 4096, 6, torch.bfloat16, torch.float32, False, 1),   # float32 Ada values
    (7, 2048, 6, torch.float32, torch.float32, True, 3),
    (1, 4096, 6, torch.bfloat16, torch.bfloat16, False, 1),
]


@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch", ADA_CASES)
def test_adazero_from_ada(rows, cols, params, tdt, sdt, bc, batch):
    from opengenie_amd.ltx_ops import fused_adazero_from_ada

    x, table, ts, xg, tg, sg = _ada(200 + rows, rows, cols, params, tdt, sdt, bc, batch)
    out = fused_adazero_from_ada(xg, 1e-6, tg, sg, shift_index=3, scale_index=4)
    _ran("fused_adazero_from_ada")
    ref = O.adazero_from_ada(to_T(x), 1e-6, to_T(table), to_T(ts), 3, 4)
    assert_same_bits(out_np(out), bf16_round(ref.v), "adazero_from_ada")


@pytest.mark.parametrize("scale,zero_dim", [(8.0 / 448, True), (0.01, False), (0.5 / 448, True)])
@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch",
                         ADA_CASES + [(2304, 4096, 9, torch.bfloat16, torch.bfloat16, True, 1)])
def test_adazero_from_ada_fp8(rows, cols, params, tdt, sdt, bc, batch, scale, zero_dim):
    """AdaZero straight into the FP8 linear's e4m3 input: bit for bit the
    oracle's quantizer (GPU torch semantics) applied to the oracle's AdaZero
    rows; 0.5/448 saturates the tails at +-448."""
    from opengenie_amd.ltx_ops import fused_adazero_from_ada_fp8

    x, table, ts, xg, tg, sg = _ada(700 + rows, rows, cols, params, tdt, sdt, bc, batch)
    s = torch.tensor(scale, dtype=torch.float32) if zero_dim else torch.tensor([scale], dtype=torch.float32)
    out = fused_adazero_from_ada_fp8(xg, 1e-6, tg, sg, g(s), shift_index=3, scale_index=4)
    _ran("fused_adazero_from_ada_fp8")
    assert out.dtype == torch.float8_e4m3fn and out.shape == x.shape
    ref = O.adazero_from_ada(to_T(x), 1e-6, to_T(table), to_T(ts), 3, 4)
    codes = O.fp8_quantize_e4m3(O.bf(bf16_round(ref.v)), float(s.reshape(())), zero_dim, device="cuda")
    got = out.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, codes.reshape(got.shape)), int((got != codes.reshape(got.shape)).sum())
    if scale < 0.005:
        assert (np.abs(np32(out.float())) == 448).any()


@pytest.mark.parametrize("scale", [0.02, 0.5 / 448, 1.0e38, 3.0e38])
@pytest.mark.parametrize("zero_dim", [True, False])
def test_adazero_fp8_clean_and_unclean_rows(scale, zero_dim):
    """Finite Ada values, so a workgroup's rows take the clamp without a NaN
    select unless the row itself is not finite: rows with a NaN, an infinity,
    a mean square beyond float32 (finite in the float64 sum, inv = 0) and
    ordinary rows side by side, at scales whose r is normal and (1e38, 3e38)
    below 2^-126, where every row keeps the NaN-preserving clamp. Codes bit
    for bit against the oracle, NaN codes sign-free."""
    from opengenie_amd.ltx_ops import fused_adazero_from_ada_fp8

    cols, params, rows = 4096, 6, 300
    x = randn((1, rows, cols), 781)
    x[0, 7, 11] = float("nan")
    x[0, 100, 5] = float("inf")
    x[0, 101, 6] = float("-inf")
    x[0, 150] = x[0, 150] * 1e30
    x[0, 151] = 0.0
    table = randn((params, cols), 782, std=0.02)
    ts = randn((1, 1, params * cols), 783, std=0.5).expand(1, rows, params * cols)
    s = torch.tensor(scale, dtype=torch.float32) if zero_dim else torch.tensor([scale], dtype=torch.float32)
    out = fused_adazero_from_ada_fp8(g(x), 1e-6, g(table), g(ts), g(s), shift_index=3, scale_index=4)
    _ran("fused_adazero_from_ada_fp8")
    ref = O.adazero_from_ada(to_T(x), 1e-6, to_T(table), to_T(ts), 3, 4)
    with np.errstate(over="ignore", invalid="ignore"):
        codes = O.fp8_quantize_e4m3(O.bf(bf16_round(ref.v)), float(s.reshape(())), zero_dim, device="cuda")
    got = out.view(torch.uint8).cpu().numpy()
    assert np.array_equal(nan_canon(got), nan_canon(codes.reshape(got.shape)))
    assert ((got[0, 7] & 0x7F) == 0x7F).all()  # the NaN row is NaN throughout


def test_adazero_from_ada_special_values():
    """Rows with a NaN, an infinity, both infinities, all zeros, signed zeros
    and a mean square beyond float32 (1e30: inv = 0), and Ada columns with a
    NaN scale and infinite shifts: the bf16 AdaZero bit for bit (NaN == NaN)
    and its e4m3 codes, with saturation, NaN codes compared sign-free."""
    from opengenie_amd.ltx_ops import fused_adazero_from_ada, fused_adazero_from_ada_fp8

    cols, params = 4096, 6
    x = randn((1, 8, cols), 771)
    x[0, 1, 17] = float("nan")
    x[0, 2, 300] = float("inf")
    x[0, 3, 5], x[0, 3, 6] = float("inf"), float("-inf")
    x[0, 4] = 0.0
    x[0, 5, ::2] = -0.0
    x[0, 5, 1::2] = 0.0
    x[0, 6] = x[0, 6] * 1e30
    table = randn((params, cols), 772, std=0.02)
    table[4, 9] = float("nan")             # scale row: NaN column
    table[3, 10] = float("inf")            # shift row: +inf and -inf columns
    table[3, 11] = float("-inf")
    ts = randn((1, 1, params * cols), 773, std=0.5).expand(1, 8, params * cols)
    xg, tg, sg = g(x), g(table), g(ts)
    ref = O.adazero_from_ada(to_T(x), 1e-6, to_T(table), to_T(ts), 3, 4)
    out = fused_adazero_from_ada(xg, 1e-6, tg, sg, shift_index=3, scale_index=4)
    _ran("fused_adazero_from_ada")
    assert_same_bits(out_np(out), bf16_round(ref.v), "adazero special values")
    for scale in (0.5 / 448, 8.0 / 448):
        sc = torch.tensor(scale, dtype=torch.float32)
        q = fused_adazero_from_ada_fp8(xg, 1e-6, tg, sg, g(sc), shift_index=3, scale_index=4)
        _ran("fused_adazero_from_ada_fp8")
        codes = O.fp8_quantize_e4m3(O.bf(bf16_round(ref.v)), scale, True, device="cuda")
        got = q.view(torch.uint8).cpu().numpy()
        assert np.array_equal(nan_canon(got), nan_canon(codes.reshape(got.shape))), scale


@pytest.mark.parametrize("tdt", [torch.bfloat16, torch.float32])
def test_ada_elementwise_special_values(tdt):
    """AdaLN affine, gate multiply, residual gate and residual gate + bias on
    NaN, +-inf, signed zeros and bf16-overflowing products in x, y, the
    table, the timestep rows and the bias: bit for bit (NaN == NaN)."""
    from opengenie_amd.ltx_ops import (fused_adaln_affine_from_ada, fused_mul_from_ada,
                                       fused_residual_gate_bias_from_ada, fused_residual_gate_from_ada)

    cols, params, rows = 2048, 9, 12
    x = randn((1, rows, cols), 781)
    y = randn((1, rows, cols), 782)
    x[0, 0, :8] = torch.tensor([float("nan"), float("inf"), float("-inf"), 0.0, -0.0, 3e38, -3e38, 1e-38])
    y[0, 1, :8] = torch.tensor([float("inf"), float("nan"), -0.0, 0.0, 3e38, float("-inf"), 1e38, -1e38])
    x[0, 2] = -0.0
    y[0, 2] = 0.0
    table = randn((params, cols), 783, dtype=tdt, std=0.02)
    table[:, 20] = float("nan")
    table[:, 21] = float("inf")
    table[:, 22] = float("-inf")
    table[:, 23] = -1.0
    ts = randn((1, rows, params * cols), 784, std=0.5)
    tsv = ts.view(1, rows, params, cols)
    tsv[0, 3, :, 30] = float("inf")
    tsv[0, 4, :, 31] = float("nan")
    tsv[0, 5, :, 32] = 1e38
    bias = randn((cols,), 785, std=0.01)
    bias[40], bias[41] = float("inf"), float("nan")
    xg, yg, tg, sg, bg = g(x), g(y), g(table), g(ts), g(bias)
    T_ = (to_T(x), to_T(y), to_T(table), to_T(ts))
    cases = (
        (fused_adaln_affine_from_ada(xg, tg, sg, shift_index=6, scale_index=7),
         O.adaln_affine_from_ada(T_[0], T_[2], T_[3], 6, 7), "adaln_affine"),
        (fused_mul_from_ada(xg, tg, sg, gate_index=8), O.mul_from_ada(T_[0], T_[2], T_[3], 8), "mul"),
        (fused_residual_gate_from_ada(xg, yg, tg, sg, gate_index=5),
         O.residual_gate_from_ada(T_[0], T_[1], T_[2], T_[3], 5), "residual_gate"),
        (fused_residual_gate_bias_from_ada(xg, yg, bg, tg, sg, gate_index=2),
         O.residual_gate_bias_from_ada(T_[0], T_[1], to_T(bias), T_[2], T_[3], 2), "residual_gate_bias"),
    )
    for out, ref, what in cases:
        assert_same_bits(out_np(out), bf16_round(ref.v), what)


@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch", ADA_CASES)
def test_adaln_affine_from_ada(rows, cols, params, tdt, sdt, bc, batch):
    from opengenie_amd.ltx_ops import fused_adaln_affine_from_ada

    x, table, ts, xg, tg, sg = _ada(300 + rows, rows, cols, params, tdt, sdt, bc, batch)
    out = fused_adaln_affine_from_ada(xg, tg, sg, shift_index=params - 3, scale_index=params - 2)
    _ran("fused_adaln_affine_from_ada")
    ref = O.adaln_affine_from_ada(to_T(x), to_T(table), to_T(ts), params - 3, params - 2)
    assert_same_bits(out_np(out), bf16_round(ref.v), "adaln_affine_from_ada")


@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch", ADA_CASES)
def test_mul_from_ada(rows, cols, params, tdt, sdt, bc, batch):
    from opengenie_amd.ltx_ops import fused_mul_from_ada

    x, table, ts, xg, tg, sg = _ada(400 + rows, rows, cols, params, tdt, sdt, bc, batch)
    out = fused_mul_from_ada(xg, tg, sg, gate_index=params - 1)
    _ran("fused_mul_from_ada")
    ref = O.mul_from_ada(to_T(x), to_T(table), to_T(ts), params - 1)
    assert_same_bits(out_np(out), bf16_round(ref.v), "mul_from_ada")


@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch", ADA_CASES)
def test_residual_gate_from_ada(rows, cols, params, tdt, sdt, bc, batch):
    from opengenie_amd.ltx_ops import fused_residual_gate_from_ada

    x, table, ts, xg, tg, sg = _ada(500 + rows, rows, cols, params, tdt, sdt, bc, batch)
    y = randn((batch, rows, cols), 550 + rows)
    out = fused_residual_gate_from_ada(xg, g(y), tg, sg, gate_index=params - 1)
    _ran("fused_residual_gate_from_ada")
    ref = O.residual_gate_from_ada(to_T(x), to_T(y), to_T(table), to_T(ts), params - 1)
    assert_same_bits(out_np(out), bf16_round(ref.v), "residual_gate_from_ada")


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols,params,tdt,sdt,bc,batch", ADA_CASES)
def test_residual_gate_bias_from_ada(rows, cols, params, tdt, sdt, bc, batch, bias_dtype):
    from opengenie_amd.ltx_ops import fused_residual_gate_bias_from_ada

    x, table, ts, xg, tg, sg = _ada(600 + rows, rows, cols, params, tdt, sdt, bc, batch)
    y = randn((batch, rows, cols), 650 + rows)
    bias = randn((cols,), 660 + rows, dtype=bias_dtype, std=0.01)
    out = fused_residual_gate_bias_from_ada(xg, g(y), g(bias), tg, sg, gate_index=2)
    _ran("fused_residual_gate_bias_from_ada")
    ref = O.residual_gate_bias_from_ada(to_T(x), to_T(y), to_T(bias), to_T(table), to_T(ts), 2)
    assert_same_bits(out_np(out), bf16_round(ref.v), "residual_gate_bias_from_ada")


def test_adazero_strided_scale_shift():
    """Reference test :8-26 shape: stride-3 views for scale and shift."""
    from opengenie_amd.ltx_ops import fused_adazero

    x = randn((1, 7, 2048), 0)
    ss = randn((1, 7, 3, 2048), 1)
    out = fused_adazero(g(x), 1e-6, g(ss)[:, :, 1, :], g(ss)[:, :, 2, :])
    _ran("fused_adazero")
    ref = O.adazero(to_T(x), 1e-6, to_T(ss[:, :, 1, :]), to_T(ss[:, :, 2, :]))
    assert_same_bits(out_np(out), ref.v, "adazero strided")


@pytest.mark.parametrize("shape_s", [(1, 1, 4096), (2, 1, 4096), (4096,), (2, 5, 4096)])
def test_adazero_broadcast_scale_shift(shape_s):
    from opengenie_amd.ltx_ops import fused_adazero

    x = randn((2, 5, 4096), 10)
    sc = randn(shape_s, 11, dtype=torch.float32, std=0.1)
    sh = randn(shape_s, 12, std=0.1)
    out = fused_adazero(g(x), 1e-6, g(sc), g(sh))
    _ran("fused_adazero")
    ref = O.adazero(to_T(x), 1e-6, to_T(sc), to_T(sh))
    assert_same_bits(out_np(out), bf16_round(ref.v), "adazero broadcast")


def test_residual_gate_bf16_strided_gate():
    """Reference test :29-47: gate is a stride-3 view."""
    from opengenie_amd.ltx_ops import fused_residual_gate_bf16

    x, y = randn((1, 7, 2048), 1), randn((1, 7, 2048), 2)
    gates = randn((1, 7, 3, 2048), 3)
    out = fused_residual_gate_bf16(g(x), g(y), g(gates)[:, :, 1, :])
    _ran("fused_residual_gate_bf16")
    assert_same_bits(out_np(out), O.residual_gate(to_T(x), to_T(y), to_T(gates[:, :, 1, :])).v, "residual gate")


@pytest.mark.parametrize("gate_shape", [(1, 1, 4096), (4096,), (3, 1, 4096)])
def test_residual_gate_bf16_broadcast(gate_shape):
    from opengenie_amd.ltx_ops import fused_residual_gate_bf16

    x, y = randn((3, 11, 4096), 4), randn((3, 11, 4096), 5)
    gate = randn(gate_shape, 6)
    out = fused_residual_gate_bf16(g(x), g(y), g(gate))
    assert_same_bits(out_np(out), O.residual_gate(to_T(x), to_T(y), to_T(gate)).v, "residual gate bc")


@pytest.mark.parametrize("rows,cols", [(11, 2048), (64, 16384), (3, 4100), (5, 13)])
@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16])
def test_bias_add(rows, cols, bias_dtype):
    from opengenie_amd.ltx_ops import fused_bias_add_bf16

    x = randn((rows, cols), 20)
    bias = randn((cols,), 21, dtype=bias_dtype)
    out = fused_bias_add_bf16(g(x), g(bias))
    _ran("fused_bias_add_bf16")
    assert_same_bits(out_np(out), O.bias_add(to_T(x), to_T(bias)).v, "bias_add")


def test_head_gate_mul():
    from opengenie_amd.ltx_ops import fused_head_gate_mul_bf16

    out = randn((1, 13, 4096), 11)
    gates = (2.0 * torch.sigmoid(randn((1, 13, 32), 12))).to(torch.bfloat16)
    y = fused_head_gate_mul_bf16(g(out), g(gates), 32, 128)
    _ran("fused_head_gate_mul_bf16")
    assert_same_bits(out_np(y), O.head_gate_mul(to_T(out), to_T(gates), 32, 128).v, "head_gate_mul")


# ------------------------------------------------------------ FP8 quantizers
@pytest.mark.parametrize("zero_dim", [True, False])
@pytest.mark.parametrize("scale", [0.05, 0.37, 1.0, 3.3e-3, 0.11160714])
def test_fp8_quantize_exhaustive_bf16(scale, zero_dim):
    """All 65536 bf16 patterns; codes equal the oracle's GPU-torch semantics."""
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3

    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    xt = torch.from_numpy(x.copy()).to(torch.bfloat16)
    s = torch.tensor(scale, dtype=torch.float32)
    if not zero_dim:
        s = s.reshape(1)
    q = fused_fp8_quantize_e4m3(g(xt), g(s))
    _ran("fused_fp8_quantize_e4m3")
    torch.cuda.synchronize()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = O.fp8_quantize_e4m3(T(x, "bf16"), scale, zero_dim, device="cuda")
    assert np.array_equal(nan_canon(q.view(torch.uint8).cpu().numpy()), nan_canon(ref))


@pytest.mark.parametrize("zero_dim", [True, False])
def test_fp8_quantize_oracle_matches_torch_on_gpu(zero_dim):
    """Pins the oracle's device semantics: torch evaluating the reference's
    expression on the GPU gives the same codes as the oracle (device='cuda')."""
    x = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))
    xt = torch.from_numpy(x.copy()).to(torch.bfloat16)
    for scale in (0.05, 0.37, 3.3e-3, 0.11160714, 0.0123):
        s = torch.tensor(scale, dtype=torch.float32)
        if not zero_dim:
            s = s.reshape(1)
        ref = tr.fp8_quantize_e4m3(g(xt), g(s)).view(torch.uint8).cpu().numpy()
        with np.errstate(over="ignore", invalid="ignore"):
            ours = O.fp8_quantize_e4m3(T(x, "bf16"), scale, zero_dim, device="cuda")
        assert np.array_equal(nan_canon(ours), nan_canon(ref)), scale


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1000, 4096 * 3 + 5])
def test_fp8_quantize_ragged_sizes(n):
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3

    x = randn((n,), 30 + n, std=40.0)
    s = torch.tensor(0.07)
    q = fused_fp8_quantize_e4m3(g(x), g(s))
    torch.cuda.synchronize()
    ref = O.fp8_quantize_e4m3(to_T(x), 0.07, True, device="cuda")
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), ref)


ALL_BF16 = bf16_from_bits(np.arange(1 << 16, dtype=np.uint16))


@pytest.mark.parametrize("zero_dim", [True, False])
def test_gelu_tanh_fp8_quantize_exhaustive_vs_torch(zero_dim):
    """Every bf16 input (65536 patterns, so the whole domain) at several
    scales: the HIP codes equal torch evaluating the reference's torch path
    (:165-169) on the GPU, bit for bit."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    xt = g(torch.from_numpy(ALL_BF16.copy()).to(torch.bfloat16))
    for scale in (0.02, 0.37, 3.3e-3, 1.0, 0.11160714):
        s = torch.tensor(scale, dtype=torch.float32)
        if not zero_dim:
            s = s.reshape(1)
        q = fused_gelu_tanh_fp8_quantize_e4m3(xt, g(s))
        _ran("fused_gelu_tanh_fp8_quantize_e4m3")
        ref = tr.gelu_tanh_fp8_quantize_e4m3(xt, g(s)).view(torch.uint8).cpu().numpy()
        got = q.view(torch.uint8).cpu().numpy()
        assert np.array_equal(nan_canon(got), nan_canon(ref)), (scale, int((got != ref).sum()))


def test_gelu_tanh_oracle_matches_torch_on_gpu():
    """Pins the oracle's GELU on its whole bf16 domain against torch's GPU
    gelu(approximate='tanh'), and the oracle's GELU quantizer codes against
    the HIP kernel's."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    xt = torch.from_numpy(ALL_BF16.copy()).to(torch.bfloat16)
    ref = torch.nn.functional.gelu(g(xt), approximate="tanh").float().cpu().numpy()
    ours = O.gelu_tanh(T(ALL_BF16, "bf16")).v
    assert_same_bits(ours, ref, "oracle gelu vs torch gpu")
    q = fused_gelu_tanh_fp8_quantize_e4m3(g(xt), g(torch.tensor(0.02)))
    with np.errstate(over="ignore", invalid="ignore"):
        oq = O.fp8_quantize_e4m3(O.gelu_tanh(T(ALL_BF16, "bf16")), 0.02, True, device="cuda")
    assert np.array_equal(nan_canon(q.view(torch.uint8).cpu().numpy()), nan_canon(oq))


@pytest.mark.parametrize("shape", [(3, 12345), (1000, 16384), (9216, 16384)])
def test_gelu_tanh_fp8_quantize_streaming(shape):
    """The table kernel's walk over the tensor: a ragged size (not a multiple
    of 16 elements, one partial pass of the grid), a mid size and the FFN
    hidden of 9216 tokens; codes equal torch's on the GPU for every element."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    x = g(randn(shape, 31 + shape[0], std=2.0))
    s = g(torch.tensor(0.02))
    q = fused_gelu_tanh_fp8_quantize_e4m3(x, s)
    _ran("fused_gelu_tanh_fp8_quantize_e4m3")
    ref = tr.gelu_tanh_fp8_quantize_e4m3(x, s)
    assert torch.equal(q.view(torch.uint8), ref.view(torch.uint8)), int((q.view(torch.uint8) != ref.view(torch.uint8)).sum())


def test_gelu_tanh_fp8_quantize_special_values():
    """Signed zeros, infinities, NaN, saturated tails (tanh(u) = -1 in float32,
    GELU -0) and huge values give torch's codes exactly."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    vals = [0.0, -0.0, float("inf"), float("-inf"), float("nan"), 10.0, -10.0, 100.0, -100.0, 3e38, -3e38,
            -7.0, -8.0, 1e-30, -1e-30, 0.5, -0.5]
    x = torch.tensor(vals * 16, dtype=torch.bfloat16).reshape(16, len(vals))
    s = torch.tensor(0.02)
    q = fused_gelu_tanh_fp8_quantize_e4m3(g(x), g(s))
    _ran("fused_gelu_tanh_fp8_quantize_e4m3")
    torch.cuda.synchronize()
    ref = tr.gelu_tanh_fp8_quantize_e4m3(x, s).view(torch.uint8).numpy()
    got = q.view(torch.uint8).cpu().numpy()
    special = np.array([not (0.1 < abs(v) < 5) for v in vals] * 16).reshape(got.shape)
    assert np.array_equal(nan_canon(got[special]), nan_canon(ref[special]))


@pytest.mark.parametrize("shape", [(1, 33, 32, 128), (2, 17, 16, 128), (1, 40, 32, 64), (1, 9216 // 16, 32, 128)])
def test_fp8_per_head(shape):
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    x = randn(shape, 40)
    if shape[0] > 1:
        x[1, :, 3, :] = 0  # an all-zero head takes the 1e-12 clamp
    q, s = fused_fp8_quantize_e4m3_per_head_4d(g(x))
    _ran("fused_fp8_quantize_e4m3_per_head_4d")
    torch.cuda.synchronize()
    qr, sr = O.fp8_per_head_quantize(np32(x))
    assert_same_bits(s.cpu().numpy(), sr, "per-head scale")
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), qr)


def test_fp8_per_head_special_values():
    """Division edge cases: every finite bf16 value (scale at the top of the
    range), +-inf (infinite scale, inf / inf), and +-0, denormals and tiny
    values beside normal ones (zero codes keep their sign)."""
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    bits = np.arange(65536, dtype=np.uint32)
    exp = (bits >> 7) & 0xFF
    finite = bits[exp != 0xFF]
    x = np.random.default_rng(8).standard_normal((1, 512, 8, 128)).astype(np.float32)  # H*D = 1024 (guard)
    h0 = np.zeros(512 * 128, np.uint32)
    h0[: finite.size] = finite
    x[0, :, 0, :] = (h0 << 16).view(np.float32).reshape(512, 128)
    rng = np.random.default_rng(7)
    h1 = rng.standard_normal(512 * 128).astype(np.float32)
    h1[::97] = np.inf
    h1[::89] = -np.inf
    x[0, :, 1, :] = h1.reshape(512, 128)
    h2 = rng.standard_normal(512 * 128).astype(np.float32) * 3
    h2[::5] = 0.0
    h2[1::5] = -0.0
    h2[2::5] = ((rng.integers(1, 128, h2[2::5].size).astype(np.uint32) | 0x8000 * rng.integers(0, 2, h2[2::5].size).astype(np.uint32)) << 16).view(np.float32)  # bf16 denormals
    h2[3::5] *= 1e-4
    x[0, :, 2, :] = h2.reshape(512, 128)
    x[0, :, 3, :] = rng.standard_normal((512, 128)).astype(np.float32) * 1e-30
    # NaN: torch's amax propagates it, so the head's scale and codes are NaN
    x[0, 200, 4, 17] = np.nan
    x[0, 3, 5, 0] = np.nan
    x[0, 4, 5, 1] = np.inf
    xt = torch.from_numpy(x).to(torch.bfloat16)
    q, s = fused_fp8_quantize_e4m3_per_head_4d(g(xt))
    _ran("fused_fp8_quantize_e4m3_per_head_4d")
    torch.cuda.synchronize()
    qr, sr = O.fp8_per_head_quantize(np32(xt))
    assert np.isnan(sr[0, 4]) and np.isnan(sr[0, 5]) and np.isfinite(sr[0, 6])
    assert_same_bits(s.cpu().numpy(), sr, "per-head scale")
    got = q.view(torch.uint8).cpu().numpy()
    assert np.array_equal(nan_canon(got), nan_canon(qr))
    # and torch evaluating the reference expression (:976-980) on the GPU
    tq, ts = tr.fp8_per_head(g(xt))
    assert_same_bits(s.cpu().numpy(), ts.cpu().numpy(), "per-head scale vs torch")
    assert np.array_equal(nan_canon(got), nan_canon(tq.view(torch.uint8).cpu().numpy()))


# ------------------------------------------------------------ Q/K preattention
def _rope(seed, tokens, cos_dtype=torch.bfloat16, w_dtype=torch.bfloat16, cos_batch=1):
    q = randn((1, tokens, 4096), seed)
    k = randn((1, tokens, 4096), seed + 1)
    qw = randn((4096,), seed + 2, dtype=w_dtype, std=0.05, mean=1.0)
    kw = randn((4096,), seed + 3, dtype=w_dtype, std=0.05, mean=1.0)
    freqs = randn((cos_batch, 32, tokens, 64), seed + 4, dtype=torch.float32, std=3.0)
    return q, k, qw, kw, freqs.cos().to(cos_dtype), freqs.sin().to(cos_dtype)


@pytest.mark.parametrize("tokens,cos_dtype,w_dtype", [
    (17, torch.bfloat16, torch.bfloat16), (1, torch.bfloat16, torch.bfloat16), (130, torch.float32, torch.bfloat16),
    (64, torch.bfloat16, torch.float32)])
def test_video_qk_rmsnorm_rope(tokens, cos_dtype, w_dtype):
    from opengenie_amd.ltx_ops import fused_video_qk_rmsnorm_rope

    q, k, qw, kw, cos, sin = _rope(800 + tokens, tokens, cos_dtype, w_dtype)
    oq, ok = fused_video_qk_rmsnorm_rope(g(q), g(k), g(qw), g(kw), 1e-6, g(cos), g(sin))
    _ran("fused_video_qk_rmsnorm_rope")
    rq, rk = O.video_qk_rmsnorm_rope(to_T(q), to_T(k), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    assert_same_bits(out_np(oq), bf16_round(rq.v), "q")
    assert_same_bits(out_np(ok), bf16_round(rk.v), "k")


@pytest.mark.parametrize("cos_dtype", [torch.bfloat16, torch.float32])
def test_video_qk_rmsnorm_rope_special_values(cos_dtype):
    """Q/K RMSNorm + RoPE on tokens with a NaN, an infinity, all zeros, signed
    zeros and a mean square beyond float32, NaN/inf norm weights, and NaN/inf
    cos/sin entries: bit for bit (NaN == NaN)."""
    from opengenie_amd.ltx_ops import fused_video_qk_rmsnorm_rope

    q, k, qw, kw, cos, sin = _rope(990, 8, cos_dtype)
    q[0, 1, 70] = float("nan")
    k[0, 2, 4000] = float("inf")
    q[0, 3] = 0.0
    k[0, 3, ::2] = -0.0
    k[0, 3, 1::2] = 0.0
    q[0, 4] = q[0, 4] * 1e30
    k[0, 5, 7], k[0, 5, 71] = float("inf"), float("-inf")
    qw[200] = float("nan")
    kw[300] = float("inf")
    cos[0, 5, 6, 10] = float("nan")
    sin[0, 7, 7, 20] = float("inf")
    oq, ok = fused_video_qk_rmsnorm_rope(g(q), g(k), g(qw), g(kw), 1e-6, g(cos), g(sin))
    _ran("fused_video_qk_rmsnorm_rope")
    rq, rk = O.video_qk_rmsnorm_rope(to_T(q), to_T(k), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    assert_same_bits(out_np(oq), bf16_round(rq.v), "q")
    assert_same_bits(out_np(ok), bf16_round(rk.v), "k")


def test_video_qk_rmsnorm_rope_strided_cos():
    """cos/sin as non-contiguous views (head and token strides permuted)."""
    from opengenie_amd.ltx_ops import fused_video_qk_rmsnorm_rope

    q, k, qw, kw, cos, sin = _rope(900, 24)
    cos_v = g(cos.permute(0, 2, 1, 3).contiguous()).permute(0, 2, 1, 3)
    sin_v = g(sin.permute(0, 2, 1, 3).contiguous()).permute(0, 2, 1, 3)
    assert not cos_v.is_contiguous()
    oq, ok = fused_video_qk_rmsnorm_rope(g(q), g(k), g(qw), g(kw), 1e-6, cos_v, sin_v)
    rq, rk = O.video_qk_rmsnorm_rope(to_T(q), to_T(k), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    assert_same_bits(out_np(oq), rq.v, "q")
    assert_same_bits(out_np(ok), rk.v, "k")


def test_video_qk_rmsnorm_rope_separate_and_pack_and_bias():
    from opengenie_amd import ltx_ops as L

    q, k, qw, kw, cos, sin = _rope(950, 33)
    v = randn((1, 33, 4096), 960)
    rq, rk = O.video_qk_rmsnorm_rope(to_T(q), to_T(k), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    sq, sk = L.fused_video_qk_rmsnorm_rope_separate(g(q), g(k), g(qw), g(kw), 1e-6, g(cos), g(sin))
    assert_same_bits(out_np(sq), rq.v, "separate q")
    assert_same_bits(out_np(sk), rk.v, "separate k")
    qkv = L.fused_video_qkv_rmsnorm_rope_pack(g(q), g(k), g(v), g(qw), g(kw), 1e-6, g(cos), g(sin))
    ref = O.video_qkv_rmsnorm_rope_pack(to_T(q), to_T(k), to_T(v), to_T(qw), to_T(kw), 1e-6, to_T(cos), to_T(sin))
    assert_same_bits(out_np(qkv), ref, "pack")
    qb = randn((4096,), 970, dtype=torch.float32, std=0.1)
    kb = randn((4096,), 971, dtype=torch.float32, std=0.1)
    bq, bk = L.fused_video_qk_bias_rmsnorm_rope(g(q), g(k), g(qb), g(kb), g(qw), g(kw), 1e-6, g(cos), g(sin))
    rbq, rbk = O.video_qk_bias_rmsnorm_rope(to_T(q), to_T(k), to_T(qb), to_T(kb), to_T(qw), to_T(kw), 1e-6,
                                            to_T(cos), to_T(sin))
    assert_same_bits(out_np(bq), rbq.v, "bias q")
    assert_same_bits(out_np(bk), rbk.v, "bias k")


# ------------------------------------------------------------ q/k RMSNorm without RoPE
@pytest.mark.parametrize("rows,cols,w_dtype", [
    (37, 4096, torch.bfloat16), (1, 4096, torch.float32), (256, 4096, None), (300, 2048, torch.bfloat16),
    # more rows than the grid has waves: several rows per wave
    (20000, 2048, torch.bfloat16)])
def test_qk_rmsnorm(rows, cols, w_dtype):
    from opengenie_amd import ltx_ops as L

    x = randn((1, rows, cols), 990 + rows, std=2.0)
    w = None if w_dtype is None else randn((cols,), 991, dtype=w_dtype, std=0.05, mean=1.0)
    got = L.qk_rmsnorm(g(x), None if w is None else g(w), 1e-6)
    assert got.shape == x.shape and got.dtype == torch.bfloat16
    ref = O.rms_norm(to_T(x), 1e-6, None if w is None else to_T(w))
    assert_same_bits(out_np(got), ref.v, f"qk_rmsnorm {rows}x{cols}")
    _ran("qk_rmsnorm")


def test_qk_rmsnorm_special_values():
    """Each element is its own R(x * inv * w), as in torch's rms_norm: signed
    zeros keep their sign next to negative values, a row with an infinity or
    a NaN goes as torch's does, and an all-zero row takes inv = 1/sqrt(eps)."""
    from opengenie_amd import ltx_ops as L

    cols = 4096
    x = randn((8, cols), 995)
    x[0, ::2] = -0.0
    x[0, 1::2] = -x[0, 1::2].abs()
    x[1, 5] = float("inf")
    x[2, 77] = float("nan")
    x[3] = 0.0
    x[3, ::3] = -0.0
    x[4] = (x[4].float() * 1e-30).to(torch.bfloat16)  # squares below float32's range
    x[5, 0] = float("-inf")
    w = randn((cols,), 996, std=0.05, mean=1.0)
    w[64:80] = -w[64:80]
    got = L.qk_rmsnorm(g(x), g(w), 1e-6)
    ref = O.rms_norm(to_T(x), 1e-6, to_T(w))
    assert_same_bits(out_np(got), ref.v, "qk_rmsnorm special values")
    assert np.signbit(out_np(got)[0, ::2]).any()


# ------------------------------------------------------------ FP8 linear
def _fp8_weights(n, k, seed):
    wf = randn((n, k), seed, dtype=torch.float32, std=0.02)
    ws = wf.abs().amax() / 448.0
    w = torch.clamp(wf / ws, -448, 448).to(torch.float8_e4m3fn)
    return w, ws.reshape(())


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (512, 768, 1024), (300, 520, 384), (1, 16, 128),
                                   (1024, 4096, 4096),
                                   # more tiles than CUs: several tiles per persistent workgroup,
                                   # partial last row and column tiles, two and three slabs per tile
                                   (4100, 4224, 256), (2304, 8192, 512), (600, 16384, 384), (4352, 4096, 1024)])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32])
def test_fp8_linear(m, n, k, bias_dtype):
    from opengenie_amd.ltx_ops import fp8_scaled_mm

    x = randn((m, k), 70 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 71 + n)
    bias = randn((n,), 72, dtype=bias_dtype, std=0.01) if bias_dtype is not None else None
    out = fp8_scaled_mm(g(a), g(w), g(sa), g(sb), g(bias) if bias is not None else None)
    _ran("fp8_scaled_mm")
    ref = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), float(sa), float(sb),
                       to_T(bias) if bias is not None else None)
    got = out_np(out)
    close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
    # rtol 1e-2 against the float64-accumulated oracle. The FP8 MFMA's own
    # accumulation rounding followed by the two bf16 roundings moves a handful
    # of outputs (about 1 in 2e6) just past 1%: two bf16 steps next to a power
    # of two. A wrong k pairing, layout or tile would move whole rows or tiles.
    assert (~close).mean() < 1e-5, (~close).sum()
    assert (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all()
    # Tripwire for gross errors: accumulation order alone moves a small
    # fraction of outputs by more than one bf16 step (sums near zero, bias
    # cancellation).
    assert (bf16_ulp_distance(got, ref) > 1).mean() < 1e-2


@pytest.mark.parametrize("m,n,k", [(4352, 4096, 4096), (4352, 4096, 8192), (256, 4096, 4096)])
def test_fp8_linear_split_k_through_c_abi(m, n, k):
    """The split-K schedule (workspace given) and the whole-tile schedule
    (no workspace) through the C ABI, both against the oracle. 272 tiles on
    256 CUs leave 16 for a last round, each cut into K-chunks (4 of 1024 at
    K = 4096, 8 of 1024 at K = 8192); 256 rows make 16 tiles and no whole
    round, all of them cut (4 chunks each, the text projections' shape)."""
    from opengenie_amd import _lib

    lib = _lib.load()
    ws_bytes = int(lib.oga_fp8_linear_workspace_bytes(m, n, k))
    assert ws_bytes > 0  # these shapes leave a partial last round of tiles
    x = randn((m, k), 80 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 81 + n)
    bias = randn((n,), 82, std=0.01)
    ga, gw, gsa, gsb, gb = g(a), g(w), g(sa).float(), g(sb).float(), g(bias)
    ref = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), float(sa), float(sb), to_T(bias))
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for use_ws in (False, True):
        out = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        ws = torch.empty((ws_bytes // 4,), device="cuda", dtype=torch.float32) if use_ws else None
        _lib.call("oga_fp8_linear_ws", ga.data_ptr(), k, gw.data_ptr(), k, gsa.data_ptr(), gsb.data_ptr(),
                  gb.data_ptr(), _lib.DT_BF16, out.data_ptr(), n, m, n, k, ws.data_ptr() if use_ws else None,
                  ws_bytes if use_ws else 0, stream)
        torch.cuda.synchronize()
        got = out_np(out)
        close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
        assert (~close).mean() < 1e-5 and (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all()
        assert (bf16_ulp_distance(got, ref) > 1).mean() < 1e-2
        outs.append(got)
    # the two schedules differ only in the order of the float32 sums
    assert (bf16_ulp_distance(outs[0], outs[1]) > 1).mean() < 1e-3


@pytest.mark.parametrize("m,n,k", [(4352, 4096, 4096), (256, 4096, 4096), (9216, 4096, 16384)])
def test_fp8_linear_split_k_workspace_reuse(m, n, k):
    """The split-K schedule keeps nothing in its workspace from one call to
    the next: three calls on one workspace and one on a fresh workspace full
    of garbage give identical bits (the chunk sums are taken in chunk order),
    within the oracle's bar; 256 rows split every tile (no whole round), the
    down-projection's tail splits K = 16384."""
    from opengenie_amd import _lib

    lib = _lib.load()
    ws_bytes = int(lib.oga_fp8_linear_workspace_bytes(m, n, k))
    assert ws_bytes > 0
    x = randn((m, k), 380 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 381 + n)
    bias = randn((n,), 382, std=0.01)
    ga, gw, gsa, gsb, gb = g(a), g(w), g(sa).float(), g(sb).float(), g(bias)
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty((ws_bytes // 4,), device="cuda", dtype=torch.float32)
    outs = []
    for call in range(4):
        if call == 3:  # a fresh workspace full of garbage
            ws = torch.full((ws_bytes // 4,), -7.0, device="cuda", dtype=torch.float32)
        out = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        _lib.call("oga_fp8_linear_ws", ga.data_ptr(), k, gw.data_ptr(), k, gsa.data_ptr(), gsb.data_ptr(),
                  gb.data_ptr(), _lib.DT_BF16, out.data_ptr(), n, m, n, k, ws.data_ptr(), ws_bytes, stream)
        outs.append(out)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    if m <= 4352:
        ref = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), float(sa), float(sb),
                           to_T(bias))
        got = out_np(outs[0])
        close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
        assert (~close).mean() < 1e-5 and (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all()
    else:  # the configured down-projection: every output against the device checker of the decoded codes
        from tests.test_gpu_config_shapes import _device_fp8_linear, _linear_full_check

        _linear_full_check(outs[0], _device_fp8_linear(ga, gw, gsa, gsb, gb), "down-projection, split tail")


def _bias_epilogue_ref(out_nobias: np.ndarray, bias: torch.Tensor, r=bf16_round) -> np.ndarray:
    """R(out + R(bias)): the second rounding of the FP8 linear (:1705-1709),
    R the output dtype's rounding."""
    return r(out_nobias + r(np32(bias))[None, :])


@pytest.mark.parametrize("m,n,k", [(300, 520, 384), (512, 768, 1024), (1, 16, 128),
                                   (4352, 4096, 4096),  # whole-tile rounds + split-K last round
                                   (256, 4096, 4096),   # split-K only
                                   (600, 16384, 384)])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32, torch.float16])
def test_fp8_linear_fp16_output(m, n, k, bias_dtype):
    """An fp16 FP8Linear: out_dtype fp16, out = R(R(acc * sa * sb) + R(bias))
    with R rounding to fp16, against the oracle; every schedule of the
    kernel (one workgroup per tile, persistent, split-K reduce)."""
    from opengenie_amd.ltx_ops import fp8_scaled_mm

    x = randn((m, k), 270 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 271 + n)
    bias = randn((n,), 272, dtype=bias_dtype, std=0.01) if bias_dtype is not None else None
    out = fp8_scaled_mm(g(a), g(w), g(sa), g(sb), g(bias) if bias is not None else None, out_dtype=torch.float16)
    _ran("fp8_scaled_mm")
    assert out.dtype == torch.float16 and out.shape == (m, n)
    ref = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), float(sa), float(sb),
                       to_T(bias) if bias is not None else None, out_dt="f16")
    got = out_np(out)
    # fp16 carries 3 more mantissa bits than bf16, so the float32 sum order
    # shows in more outputs: within 2 fp16 steps, and at most a few percent
    # more than one step (sums near zero, bias cancellation).
    close = np.isclose(got, ref, rtol=2e-3, atol=1e-3 * float(np.abs(ref).max()))
    assert (~close).mean() < 1e-4, (~close).sum()
    assert (f16_ulp_distance(got[~close], ref[~close]) <= 2).all()
    if m * n >= 4096:  # a fraction of 16 outputs says nothing
        assert (f16_ulp_distance(got, ref) > 1).mean() < 3e-2
    else:
        assert f16_ulp_distance(got, ref).max() <= 2
    # the same oracle rounding to bf16 misses most outputs (only about one in
    # eight fp16 values is also a bf16 value): the rounding is fp16's
    if m * n >= 4096:
        ref_bf = O.fp8_linear(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), float(sa), float(sb),
                              to_T(bias) if bias is not None else None)
        assert (f16_ulp_distance(got, ref_bf) > 0).mean() > 0.75


@pytest.mark.parametrize("m,n,k,use_ws", [
    (4352, 4096, 4096, False),  # persistent whole-tile schedule
    (4352, 4096, 4096, True),   # + split-K last round
    (256, 4096, 4096, True),    # split-K only
    (300, 520, 384, False),     # one workgroup per tile (N not a multiple of 128)
])
def test_fp8_linear_fp16_bias_epilogue_is_exact(m, n, k, use_ws):
    """fp16 output through oga_fp8_linear_dt_ws: with and without an fp16
    bias, out_bias == R16(out_nobias + bias) bit for bit."""
    from opengenie_amd import _lib

    lib = _lib.load()
    x = randn((m, k), 280 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 281 + n)
    bias = randn((n,), 282, dtype=torch.float16, std=0.01)
    ga, gw, gsa, gsb, gb = g(a), g(w), g(sa).float(), g(sb).float(), g(bias)
    ws_bytes = int(lib.oga_fp8_linear_workspace_bytes(m, n, k)) if use_ws else 0
    if use_ws:
        assert ws_bytes > 0
    ws = torch.empty((max(ws_bytes, 4) // 4,), device="cuda", dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for bp in (None, gb):
        out = torch.empty((m, n), device="cuda", dtype=torch.float16)
        _lib.call("oga_fp8_linear_dt_ws", ga.data_ptr(), k, gw.data_ptr(), k, gsa.data_ptr(), gsb.data_ptr(),
                  bp.data_ptr() if bp is not None else None, _lib.DT_F16, out.data_ptr(), _lib.DT_F16, n, m, n, k,
                  ws.data_ptr() if use_ws else None, ws_bytes, stream)
        torch.cuda.synchronize()
        outs.append(out.cpu().view(torch.int16).numpy())
    nob = outs[0].view(np.float16).astype(np.float32)
    exp = _bias_epilogue_ref(nob, bias, f16_round).astype(np.float16).view(np.int16)
    assert np.array_equal(outs[1], exp), int((outs[1] != exp).sum())
    # an fp16 output with a bf16 bias is refused (the host converts it first)
    out = torch.empty((m, n), device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError):
        _lib.call("oga_fp8_linear_dt_ws", ga.data_ptr(), k, gw.data_ptr(), k, gsa.data_ptr(), gsb.data_ptr(),
                  g(bias.to(torch.bfloat16)).data_ptr(), _lib.DT_BF16, out.data_ptr(), _lib.DT_F16, n, m, n, k,
                  None, 0, stream)


def test_fp8_linear_fp16_output_against_torch_scaled_mm():
    """torch._scaled_mm with out_dtype fp16 on the same codes (hipBLASLt):
    the same roundings, so within one fp16 step bar the sum order."""
    from opengenie_amd.ltx_ops import fp8_scaled_mm

    m, n, k = 1024, 4096, 4096
    x = randn((m, k), 290, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = g(torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn))
    w, sb = _fp8_weights(n, k, 291)
    w, sa, sb = g(w), g(sa).float(), g(sb).float()
    bias = g(randn((n,), 292, std=0.01))
    try:
        ref = torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sb, out_dtype=torch.float16, use_fast_accum=True)
    except RuntimeError as exc:  # the installed hipBLASLt may lack an fp8 -> fp16 kernel
        pytest.skip(f"torch._scaled_mm fp16 output: {exc}")
    ref = ref + bias.to(torch.float16)
    out = fp8_scaled_mm(a, w, sa, sb, bias, out_dtype=torch.float16)
    _ran("fp8_scaled_mm")
    d = f16_ulp_distance(out_np(out), out_np(ref))
    assert (d > 1).mean() < 3e-2 and (d > 0).mean() < 0.5, ((d > 1).mean(), (d > 0).mean())


def test_fp8_linear_forward_fp16_module():
    """The patched FP8Linear.forward with an fp16 input: out_dtype = x.dtype,
    the fp16 quantizer and the fp16 GEMM both on the HIP path."""
    from opengenie_amd.ltx_ops import fp8_linear_forward

    class Lin(torch.nn.Module):
        pass

    lin = Lin()
    w, sb = _fp8_weights(1024, 512, 293)
    lin.weight = g(w)
    lin.weight_scale = g(sb).float()
    lin.input_scale = g(torch.tensor(0.0123))
    lin.bias = g(randn((1024,), 294, std=0.01))  # bf16, as a checkpoint holds it
    x = randn((1, 333, 512), 295, dtype=torch.float16)
    out = fp8_linear_forward(lin, g(x))
    _ran("fused_fp8_quantize_e4m3")
    _ran("fp8_scaled_mm")
    assert out.shape == (1, 333, 1024) and out.dtype == torch.float16
    q = O.fp8_quantize_e4m3(to_T(x), 0.0123, True, device="cuda").reshape(333, 512)
    ref = O.fp8_linear(q, w.view(torch.uint8).numpy(), 0.0123, float(sb), to_T(lin.bias.cpu()), out_dt="f16")
    got = out_np(out).reshape(333, 1024)
    close = np.isclose(got, ref, rtol=2e-3, atol=1e-3 * float(np.abs(ref).max()))
    assert (~close).mean() < 1e-4 and (f16_ulp_distance(got[~close], ref[~close]) <= 2).all()


@pytest.mark.parametrize("m,n,k,bias_dtype,use_ws", [
    (4352, 4096, 4096, torch.bfloat16, False),  # persistent whole-tile schedule
    (4352, 4096, 4096, torch.bfloat16, True),   # + split-K last round (16 tiles x 4 K-chunks)
    (256, 4096, 4096, torch.bfloat16, True),    # split-K only (16 tiles x 4 K-chunks, no whole round)
    (300, 520, 384, torch.float32, False),      # one-workgroup-per-tile kernel (N not a multiple of 128)
    (300, 520, 384, torch.bfloat16, False),
])
def test_fp8_linear_bias_epilogue_is_exact(m, n, k, bias_dtype, use_ws):
    """The bias epilogue pinned independently of the float32 accumulation
    order: the same GEMM with and without the bias gives, on every element,
    out_bias == R(out_nobias + R(bias)) bit for bit."""
    from opengenie_amd import _lib

    lib = _lib.load()
    x = randn((m, k), 180 + m, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn)
    w, sb = _fp8_weights(n, k, 181 + n)
    bias = randn((n,), 182, dtype=bias_dtype, std=0.01)
    ga, gw, gsa, gsb, gb = g(a), g(w), g(sa).float(), g(sb).float(), g(bias)
    ws_bytes = int(lib.oga_fp8_linear_workspace_bytes(m, n, k)) if use_ws else 0
    if use_ws:
        assert ws_bytes > 0
    ws = torch.empty((max(ws_bytes, 4) // 4,), device="cuda", dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for bp in (None, gb):
        out = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        _lib.call("oga_fp8_linear_ws", ga.data_ptr(), k, gw.data_ptr(), k, gsa.data_ptr(), gsb.data_ptr(),
                  bp.data_ptr() if bp is not None else None, _lib.DT_BF16 if bias_dtype == torch.bfloat16 else
                  _lib.DT_F32, out.data_ptr(), n, m, n, k, ws.data_ptr() if use_ws else None, ws_bytes, stream)
        outs.append(out_np(out))
    assert_same_bits(outs[1], _bias_epilogue_ref(outs[0], bias), "bias epilogue")


def test_fp8_grouped_linear_bias_epilogue_is_exact():
    """The grouped kernel's per-linear bias: with and without the biases,
    out_bias == R(out_nobias + R(bias_i)) for every linear and element."""
    import ctypes

    from opengenie_amd import _lib

    lib = _lib.load()
    m, n, k, groups = 1536, 4096, 4096, 3
    x = randn((m, k), 190, std=1.0)
    sa = (x.float().abs().amax() / 448.0).reshape(())
    a = g(torch.clamp(x.float() / sa, -448, 448).to(torch.float8_e4m3fn))
    gsa = g(sa).float()
    ws_ = [_fp8_weights(n, k, 191 + i) for i in range(groups)]
    w = [g(t[0]) for t in ws_]
    sb = [g(t[1]).float() for t in ws_]
    biases = [g(randn((n,), 195 + i, std=0.01)) for i in range(groups)]
    ws_bytes = int(lib.oga_fp8_linear_workspace_bytes(m, n * groups, k))
    ws = torch.empty((max(ws_bytes, 4) // 4,), device="cuda", dtype=torch.float32)
    arr = ctypes.c_void_p * groups
    res = []
    for with_bias in (False, True):
        outs = [torch.empty((m, n), device="cuda", dtype=torch.bfloat16) for _ in range(groups)]
        w_p = arr(*[t.data_ptr() for t in w])
        s_p = arr(*[t.data_ptr() for t in sb])
        b_p = arr(*[(t.data_ptr() if with_bias else None) for t in biases])
        o_p = arr(*[o.data_ptr() for o in outs])
        _lib.call("oga_fp8_linear_grouped_ws", a.data_ptr(), k, ctypes.addressof(w_p), k, gsa.data_ptr(),
                  ctypes.addressof(s_p), ctypes.addressof(b_p), _lib.DT_BF16, ctypes.addressof(o_p), n, m, n, groups,
                  k, ws.data_ptr() if ws_bytes else None, ws_bytes, torch.cuda.current_stream().cuda_stream)
        res.append([out_np(o) for o in outs])
    for i in range(groups):
        assert_same_bits(res[1][i], _bias_epilogue_ref(res[0][i], biases[i]), f"grouped bias epilogue {i}")


class _FP8Lin(torch.nn.Module):
    """Duck-typed FP8Linear: e4m3 weight, input/weight scales, bias."""

    def __init__(self, n, k, seed, input_scale):
        super().__init__()
        w, sb = _fp8_weights(n, k, seed)
        self.weight = g(w)
        self.weight_scale = g(sb).float()
        self.input_scale = input_scale
        self.bias = g(randn((n,), seed + 1, std=0.01))


@pytest.mark.parametrize("tokens", [300, 1536])
@pytest.mark.parametrize("names", [("to_q", "to_k", "to_v"), ("to_q", "to_k")])
def test_fp8_qkv_grouped_mm(tokens, names):
    """fp8_qkv_from_grouped_mm / fp8_qk_from_grouped_mm: one launch, each
    linear with its own weight scale and bias, against the oracle per linear
    (1536 tokens: more tiles than CUs, split-K tail)."""
    from opengenie_amd import ltx_ops as L

    attn = torch.nn.Module()
    s_in = g(torch.tensor(0.0123))
    for i, nm in enumerate(names):
        setattr(attn, nm, _FP8Lin(4096, 4096, 100 + 7 * i, s_in))
    x = randn((1, tokens, 4096), 99)
    fn = L.fp8_qkv_from_grouped_mm if len(names) == 3 else L.fp8_qk_from_grouped_mm
    outs = fn(attn, g(x))
    _ran("fp8_grouped_linear")
    torch.cuda.synchronize()
    assert len(outs) == len(names)
    q = O.fp8_quantize_e4m3(to_T(x), 0.0123, True, device="cuda").reshape(tokens, 4096)
    for nm, out in zip(names, outs):
        lin = getattr(attn, nm)
        assert out.shape == (1, tokens, 4096) and out.dtype == torch.bfloat16
        ref = O.fp8_linear(q, lin.weight.view(torch.uint8).cpu().numpy(), 0.0123, float(lin.weight_scale),
                           to_T(lin.bias.cpu()))
        got = out_np(out).reshape(tokens, 4096)
        close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
        assert (~close).mean() < 1e-5 and (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all(), nm
        assert (bf16_ulp_distance(got, ref) > 1).mean() < 1e-2, nm


def test_fp8_qkv_shared_quantized_input_and_guard():
    from opengenie_amd import ltx_ops as L

    attn = torch.nn.Module()
    s_in = g(torch.tensor(0.0123))
    for i, nm in enumerate(("to_q", "to_k", "to_v")):
        setattr(attn, nm, _FP8Lin(4096, 4096, 120 + 7 * i, s_in))
    x = g(randn((1, 64, 4096), 98))
    shared = L.fp8_qkv_from_shared_quantized_input(attn, x)
    grouped = L.fp8_qkv_from_grouped_mm(attn, x)
    torch.cuda.synchronize()
    for a, b in zip(shared, grouped):
        assert (bf16_ulp_distance(out_np(a), out_np(b)) > 1).mean() < 1e-3
    # a different input scale on to_v: the reference guards return None
    attn.to_v.input_scale = g(torch.tensor(0.02))
    assert L.fp8_qkv_from_grouped_mm(attn, x) is None
    assert L.fp8_qkv_from_shared_quantized_input(attn, x) is None
    assert L.fp8_qk_from_grouped_mm(attn, x) is not None
    # batch 2 is outside the guard
    assert L.fp8_qk_from_grouped_mm(attn, g(randn((2, 8, 4096), 97))) is None


def _qkv_attn(seed, s_in=0.0123, equal_weight_scales=False):
    attn = torch.nn.Module()
    si = g(torch.tensor(s_in))
    for i, nm in enumerate(("to_q", "to_k", "to_v")):
        setattr(attn, nm, _FP8Lin(4096, 4096, seed + 7 * i, si))
    if equal_weight_scales:  # one scale for all three (the weights stay as drawn)
        attn.to_k.weight_scale = attn.to_q.weight_scale.clone()
        attn.to_v.weight_scale = attn.to_q.weight_scale.clone()
    return attn


def _close_to(got, ref, what):
    close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
    assert (~close).mean() < 1e-5 and (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all(), what
    assert (bf16_ulp_distance(got, ref) > 1).mean() < 1e-2, what


@pytest.mark.parametrize("tokens", [300, 1536])
def test_fp8_qkv_from_packed_linear(tokens):
    """:822-850 — one launch writes the three linears into the columns of one
    (1, N, 3*4096) output whose split views are returned; equal to the grouped
    projection bit for bit and to the oracle per linear."""
    from opengenie_amd import ltx_ops as L

    attn = _qkv_attn(140, equal_weight_scales=True)
    x = g(randn((1, tokens, 4096), 141))
    L.reset_video_qkv_packed_stats()
    out = L.fp8_qkv_from_packed_linear(attn, x)
    assert out is not None and len(out) == 3
    q, k, v = out
    assert q.shape == (1, tokens, 4096) and q.stride() == (tokens * 3 * 4096, 3 * 4096, 1)
    assert k.data_ptr() == q.data_ptr() + 4096 * 2 and v.data_ptr() == q.data_ptr() + 2 * 4096 * 2
    grouped = L.fp8_qkv_from_grouped_mm(attn, x)
    qx = O.fp8_quantize_e4m3(to_T(x.cpu()), 0.0123, True, device="cuda").reshape(tokens, 4096)
    sb = float(attn.to_q.weight_scale)
    for nm, a, b in zip(("to_q", "to_k", "to_v"), out, grouped):
        assert_same_bits(out_np(a), out_np(b), f"packed vs grouped {nm}")
        lin = getattr(attn, nm)
        ref = O.fp8_linear(qx, lin.weight.view(torch.uint8).cpu().numpy(), 0.0123, sb, to_T(lin.bias.cpu()))
        _close_to(out_np(a).reshape(tokens, 4096), ref, nm)
    assert L.collect_video_qkv_packed_linear_stats() == {"calls": 1, "fallbacks": 0, "fallback_reasons": {}}
    # the reference's guards: unequal weight scales, batch 2
    attn.to_v.weight_scale = attn.to_v.weight_scale * 2
    assert L.fp8_qkv_from_packed_linear(attn, x) is None
    assert L.fp8_qkv_from_packed_linear(attn, g(randn((2, 8, 4096), 142))) is None
    assert L.collect_video_qkv_packed_linear_stats()["fallback_reasons"] == {"weight_scale": 1, "shape": 1}


def test_fp8_qkv_from_packed_requant():
    """:852-887 — the three weights requantized to their largest scale (the
    cached packed weight equals the oracle's requantization bit for bit), one
    GEMM of N = 3*4096, each projection against the oracle on the requantized
    weights; the check recorder compares with the exact per-linear projections."""
    from opengenie_amd import ltx_ops as L

    tokens = 700
    attn = _qkv_attn(150)
    scales = [float(getattr(attn, nm).weight_scale) for nm in ("to_q", "to_k", "to_v")]
    assert len(set(scales)) == 3
    x = g(randn((1, tokens, 4096), 151))
    L.reset_video_qkv_packed_stats(requant_checks=1)
    out = L.fp8_qkv_from_packed_requant(attn, x)
    assert out is not None
    common = float(np.max(np.float32(scales)))
    packed = attn._oga_qkv_packed_requant_cache["weight"].view(torch.uint8).cpu().numpy()
    qx = O.fp8_quantize_e4m3(to_T(x.cpu()), 0.0123, True, device="cuda").reshape(tokens, 4096)
    for i, nm in enumerate(("to_q", "to_k", "to_v")):
        lin = getattr(attn, nm)
        wr = O.fp8_requantize_common_scale(lin.weight.view(torch.uint8).cpu().numpy(), scales[i], common)
        assert np.array_equal(nan_canon(packed[i * 4096:(i + 1) * 4096]), nan_canon(wr)), nm
        ref = O.fp8_linear(qx, wr, 0.0123, common, to_T(lin.bias.cpu()))
        _close_to(out_np(out[i]).reshape(tokens, 4096), ref, nm)
    st = L.collect_video_qkv_packed_requant_stats()
    assert st["calls"] == 1 and len(st["checks"]) == 3
    assert all(np.isfinite(c["rms"]) and c["rms"] < 0.1 for c in st["checks"]), st["checks"]
    attn.to_k.input_scale = g(torch.tensor(0.02))
    assert L.fp8_qkv_from_packed_requant(attn, x) is None
    assert L.collect_video_qkv_packed_requant_stats()["fallback_reasons"] == {"input_scale": 1}


def test_fp8_linear_forward_module():
    """The patched FP8Linear.forward on a duck-typed module, 3-D input."""
    from opengenie_amd.ltx_ops import fp8_linear_forward

    class Lin(torch.nn.Module):
        pass

    lin = Lin()
    w, sb = _fp8_weights(512, 256, 90)
    lin.weight = g(w)
    lin.weight_scale = g(sb)
    lin.input_scale = g(torch.tensor(0.0123))
    lin.bias = g(randn((512,), 91, std=0.01))
    x = randn((1, 77, 256), 92)
    out = fp8_linear_forward(lin, g(x))
    assert out.shape == (1, 77, 512)
    q = O.fp8_quantize_e4m3(to_T(x), 0.0123, True, device="cuda").reshape(77, 256)
    ref = O.fp8_linear(q, w.view(torch.uint8).numpy(), 0.0123, float(sb), to_T(lin.bias.cpu()))
    np.testing.assert_allclose(out_np(out).reshape(77, 512), ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))


@pytest.mark.parametrize("tokens", [256, 77])
def test_fp8_kv_grouped_mm_of_the_text_context(tokens):
    """fp8_kv_from_grouped_mm: the text cross-attention's K and V projections
    as one grouped launch, each against the oracle and against its own
    FP8Linear forward (same roundings; only the float32 order of split
    K-chunks may differ); None when the two input scales differ."""
    from opengenie_amd import ltx_ops as L

    attn = torch.nn.Module()
    s_in = g(torch.tensor(0.0123))
    attn.to_k = _FP8Lin(4096, 4096, 400, s_in)
    attn.to_v = _FP8Lin(4096, 4096, 407, s_in)
    ctx = g(randn((1, tokens, 4096), 410))
    kv = L.fp8_kv_from_grouped_mm(attn, ctx)
    _ran("fp8_grouped_linear")
    assert kv is not None and len(kv) == 2
    q = O.fp8_quantize_e4m3(to_T(ctx.cpu()), 0.0123, True, device="cuda").reshape(tokens, 4096)
    for out, lin in zip(kv, (attn.to_k, attn.to_v)):
        assert out.shape == (1, tokens, 4096) and out.dtype == torch.bfloat16
        ref = O.fp8_linear(q, lin.weight.view(torch.uint8).cpu().numpy(), 0.0123, float(lin.weight_scale),
                           to_T(lin.bias.cpu()))
        got = out_np(out).reshape(tokens, 4096)
        close = np.isclose(got, ref, rtol=1e-2, atol=1e-3 * float(np.abs(ref).max()))
        assert (~close).mean() < 1e-5 and (bf16_ulp_distance(got[~close], ref[~close]) <= 2).all()
        one = out_np(L.fp8_linear_forward(lin, ctx)).reshape(tokens, 4096)
        assert (bf16_ulp_distance(got, one) > 1).mean() < 1e-3
    attn.to_v.input_scale = g(torch.tensor(0.02))
    assert L.fp8_kv_from_grouped_mm(attn, ctx) is None
