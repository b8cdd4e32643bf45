"""Golden fixtures (tests/golden/golden.npz, written by make_golden.py from
torch evaluating the reference's expressions on the CPU).

CPU: the oracle reproduces every fixture. GPU: the HIP ops reproduce them.
Elementwise ops and FP8 codes must match exactly; ops with an RMS reduction
may differ from torch's own float32 reduction order in rare elements."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import ltx_ops as O
from oracle.numerics import T, bf16_from_bits, bf16_round, e4m3_decode
from tests.helpers import assert_same_bits, bf16_step, bf16_ulp_distance, nan_canon

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
G = np.load(PATH)


def bf(key) -> np.ndarray:
    return bf16_from_bits(G[key])


def tbf(key) -> T:
    return T(bf(key), "bf16")


def tf(key) -> T:
    return T(G[key].astype(np.float32), "f32")


def tt(key, dev) -> torch.Tensor:
    a = G[key]
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    elif a.dtype == np.uint8:
        t = torch.from_numpy(a.copy())
    else:
        t = torch.from_numpy(a.copy())
    return t.to(dev)


RMS_CASES = ["adazero_from_ada", "adazero_from_ada_uniform", "adazero_strided", "video_qk_rmsnorm_rope"]


def _rms_close(got, want, what, norm=None, gain=None):
    """An RMS op's output against the fixture (torch's CPU evaluation):
    differences rare, and each within what one bf16 step of the normalized
    row `norm` carried through the op's roundings can make (at most twice
    that step times the op's gain on it, plus two steps of the output)."""
    d = bf16_ulp_distance(bf16_round(got), bf16_round(want))
    assert (d > 0).mean() < 5e-3, (what, (d > 0).mean())
    if norm is not None:
        g = 1.0 if gain is None else np.abs(np.asarray(gain, np.float64))
        tol = 2 * bf16_step(norm) * np.maximum(g, 1.0) + 2 * bf16_step(want)
        err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
        assert (err <= tol).all(), (what, float((err / tol).max()))


# ---------------------------------------------------------------- oracle
def test_oracle_reproduces_elementwise_fixtures():
    assert_same_bits(O.adaln_affine_from_ada(tbf("adaln_affine_from_ada/x"), tf("adaln_affine_from_ada/table"),
                                             tbf("adaln_affine_from_ada/ts"), 6, 7).v,
                     bf("adaln_affine_from_ada/out"), "adaln")
    assert_same_bits(O.mul_from_ada(tbf("adaln_affine_from_ada/x"), tf("adaln_affine_from_ada/table"),
                                    tbf("adaln_affine_from_ada/ts"), 8).v, bf("mul_from_ada/out"), "mul")
    k = "residual_gate_from_ada/"
    assert_same_bits(O.residual_gate_from_ada(tbf(k + "x"), tbf(k + "y"), tf(k + "table"), tbf(k + "ts"), 5).v,
                     bf(k + "out"), "resid")
    k = "residual_gate_bias_from_ada/"
    assert_same_bits(O.residual_gate_bias_from_ada(tbf(k + "x"), tbf(k + "y"), tf(k + "bias"),
                                                   tf("adaln_affine_from_ada/table"),
                                                   tbf("adaln_affine_from_ada/ts"), 8).v, bf(k + "out"), "resid bias")
    k = "residual_gate_bf16/"
    gates = bf(k + "gates")
    assert_same_bits(O.residual_gate(tbf(k + "x"), tbf(k + "y"), T(gates[:, :, 1, :], "bf16")).v, bf(k + "out"), "rg")
    assert_same_bits(O.bias_add(tbf("bias_add/x"), tf("bias_add/bias")).v, bf("bias_add/out"), "bias")
    assert_same_bits(O.head_gate_mul(tbf("head_gate_mul/x"), tbf("head_gate_mul/gates"), 32, 128).v,
                     bf("head_gate_mul/out"), "head gate")


def test_oracle_reproduces_fp8_fixtures():
    x = tbf("fp8_quant/x")
    q1 = O.fp8_quantize_e4m3(x, float(G["fp8_quant/scale1"][0]), False)
    q0 = O.fp8_quantize_e4m3(x, float(G["fp8_quant/scale0"]), True)
    assert np.array_equal(q1, G["fp8_quant/q1"]) and np.array_equal(q0, G["fp8_quant/q0"])
    q, s = O.fp8_per_head_quantize(bf("fp8_per_head/x"), device="cpu")
    assert np.array_equal(nan_canon(q), nan_canon(G["fp8_per_head/q"]))
    assert_same_bits(s, G["fp8_per_head/scale"], "per-head scale")
    k = "fp8_linear/"
    out = O.fp8_linear(G[k + "a"], G[k + "w"], float(G[k + "scale_a"]), float(G[k + "scale_b"]), tbf(k + "bias"))
    ref = bf(k + "out")
    np.testing.assert_allclose(out, ref, rtol=1e-2, atol=1e-3 * np.abs(ref).max())


def _norm_and_gain(case: str):
    """The oracle's normalized row and the factor the op multiplies it by
    (1 + scale for AdaZero), for the max-distance bound of _rms_close."""
    x = tbf(case + "x")
    n = O.rms_norm(x, 1e-6).v
    b, t, c = x.v.shape
    if case == "adazero_strided/":
        scale = bf(case + "ss")[:, :, 1, :]
    else:
        table = tf(case + "table") if case == "adazero_from_ada/" else tbf(case + "table")
        si = 4 if case == "adazero_from_ada/" else 1
        (scale,) = O.ada_values_from_table(table, tbf(case + "ts"), b, t, c, si)
        scale = scale.v
    return n, 1.0 + scale


def _rope_norm(x: T, w: T) -> np.ndarray:
    """Per element, the larger magnitude of the two normalized values a split
    RoPE output combines (itself and its partner 64 columns away)."""
    n = np.abs(O.rms_norm(x, 1e-6, w).v.reshape(x.v.shape[0], x.v.shape[1], 32, 2, 64))
    m = np.maximum(n[:, :, :, 0], n[:, :, :, 1])
    return np.concatenate([m, m], axis=-1).reshape(x.v.shape)


def test_oracle_reproduces_rms_fixtures():
    k = "adazero_from_ada/"
    _rms_close(O.adazero_from_ada(tbf(k + "x"), 1e-6, tf(k + "table"), tbf(k + "ts"), 3, 4).v, bf(k + "out"), k,
               *_norm_and_gain(k))
    k = "adazero_from_ada_uniform/"
    _rms_close(O.adazero_from_ada(tbf(k + "x"), 1e-6, tbf(k + "table"), tbf(k + "ts"), 0, 1).v, bf(k + "out"), k,
               *_norm_and_gain(k))
    k = "adazero_strided/"
    ss = bf(k + "ss")
    _rms_close(O.adazero(tbf(k + "x"), 1e-6, T(ss[:, :, 1, :], "bf16"), T(ss[:, :, 2, :], "bf16")).v,
               bf(k + "out"), k, *_norm_and_gain(k))
    k = "video_qk_rmsnorm_rope/"
    oq, ok = O.video_qk_rmsnorm_rope(tbf(k + "q"), tbf(k + "k"), tbf(k + "qw"), tbf(k + "kw"), 1e-6, tbf(k + "cos"),
                                     tbf(k + "sin"))
    _rms_close(oq.v, bf(k + "q_out"), "q", _rope_norm(tbf(k + "q"), tbf(k + "qw")))
    _rms_close(ok.v, bf(k + "k_out"), "k", _rope_norm(tbf(k + "k"), tbf(k + "kw")))


# ---------------------------------------------------------------- HIP
@pytest.mark.gpu
def test_hip_reproduces_fixtures(monkeypatch):
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    from opengenie_amd import ltx_ops as L

    d = "cuda"

    def np_out(t):
        torch.cuda.synchronize()
        return t.float().cpu().numpy()

    k = "adazero_from_ada/"
    _rms_close(np_out(L.fused_adazero_from_ada(tt(k + "x", d), 1e-6, tt(k + "table", d), tt(k + "ts", d),
                                               shift_index=3, scale_index=4)), bf(k + "out"), k, *_norm_and_gain(k))
    k = "adazero_from_ada_uniform/"
    xs = tt(k + "x", d)
    ts = tt(k + "ts", d).expand(1, xs.shape[1], -1)
    _rms_close(np_out(L.fused_adazero_from_ada(xs, 1e-6, tt(k + "table", d), ts, shift_index=0, scale_index=1)),
               bf(k + "out"), k, *_norm_and_gain(k))
    k = "adazero_strided/"
    ss = tt(k + "ss", d)
    _rms_close(np_out(L.fused_adazero(tt(k + "x", d), 1e-6, ss[:, :, 1, :], ss[:, :, 2, :])), bf(k + "out"), k,
               *_norm_and_gain(k))
    a = "adaln_affine_from_ada/"
    assert_same_bits(np_out(L.fused_adaln_affine_from_ada(tt(a + "x", d), tt(a + "table", d), tt(a + "ts", d),
                                                          shift_index=6, scale_index=7)), bf(a + "out"), "adaln")
    assert_same_bits(np_out(L.fused_mul_from_ada(tt(a + "x", d), tt(a + "table", d), tt(a + "ts", d), gate_index=8)),
                     bf("mul_from_ada/out"), "mul")
    k = "residual_gate_from_ada/"
    assert_same_bits(np_out(L.fused_residual_gate_from_ada(tt(k + "x", d), tt(k + "y", d), tt(k + "table", d),
                                                           tt(k + "ts", d), gate_index=5)), bf(k + "out"), k)
    k = "residual_gate_bias_from_ada/"
    assert_same_bits(np_out(L.fused_residual_gate_bias_from_ada(tt(k + "x", d), tt(k + "y", d), tt(k + "bias", d),
                                                                tt(a + "table", d), tt(a + "ts", d), gate_index=8)),
                     bf(k + "out"), k)
    k = "residual_gate_bf16/"
    assert_same_bits(np_out(L.fused_residual_gate_bf16(tt(k + "x", d), tt(k + "y", d), tt(k + "gates", d)[:, :, 1, :])),
                     bf(k + "out"), k)
    assert_same_bits(np_out(L.fused_bias_add_bf16(tt("bias_add/x", d), tt("bias_add/bias", d))), bf("bias_add/out"),
                     "bias")
    assert_same_bits(np_out(L.fused_head_gate_mul_bf16(tt("head_gate_mul/x", d), tt("head_gate_mul/gates", d), 32,
                                                       128)), bf("head_gate_mul/out"), "head gate")
    x = tt("fp8_quant/x", d)
    q1 = L.fused_fp8_quantize_e4m3(x, tt("fp8_quant/scale1", d))
    q0 = L.fused_fp8_quantize_e4m3(x, tt("fp8_quant/scale0", d))
    torch.cuda.synchronize()
    assert np.array_equal(q1.view(torch.uint8).cpu().numpy(), G["fp8_quant/q1"])
    assert np.array_equal(q0.view(torch.uint8).cpu().numpy(), G["fp8_quant/q0"])
    q, s = L.fused_fp8_quantize_e4m3_per_head_4d(tt("fp8_per_head/x", d))
    torch.cuda.synchronize()
    # The fixture is torch's CPU evaluation, where `amax / 448` divides; on
    # the GPU torch multiplies by float32(1/448), which the kernel follows:
    # the scales agree to one float32 ulp and equal the oracle's GPU rule.
    qr, sr = O.fp8_per_head_quantize(bf("fp8_per_head/x"), device="cuda")
    assert_same_bits(s.cpu().numpy(), sr, "per-head scale")
    assert np.array_equal(nan_canon(q.view(torch.uint8).cpu().numpy()), nan_canon(qr))
    ulps = np.abs(s.cpu().numpy().view(np.int32).astype(np.int64) - G["fp8_per_head/scale"].view(np.int32))
    assert ulps.max() <= 1
    k = "video_qk_rmsnorm_rope/"
    oq, ok = L.fused_video_qk_rmsnorm_rope(tt(k + "q", d), tt(k + "k", d), tt(k + "qw", d), tt(k + "kw", d), 1e-6,
                                           tt(k + "cos", d), tt(k + "sin", d))
    _rms_close(np_out(oq), bf(k + "q_out"), "q", _rope_norm(tbf(k + "q"), tbf(k + "qw")))
    _rms_close(np_out(ok), bf(k + "k_out"), "k", _rope_norm(tbf(k + "k"), tbf(k + "kw")))
    k = "fp8_linear/"
    a8 = tt(k + "a", d).view(torch.float8_e4m3fn)
    w8 = tt(k + "w", d).view(torch.float8_e4m3fn)
    out = L.fp8_scaled_mm(a8, w8, tt(k + "scale_a", d), tt(k + "scale_b", d), tt(k + "bias", d))
    ref = bf(k + "out")
    np.testing.assert_allclose(np_out(out), ref, rtol=1e-2, atol=1e-3 * np.abs(ref).max())
    assert e4m3_decode is not None
