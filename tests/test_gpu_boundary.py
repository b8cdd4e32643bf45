"""GPU: the drop-in boundary behaves as the reference's does.

- A contiguous view at an odd storage offset passes the reference's guards.
  Here the guards also check the C ABI's alignment preconditions, so in the
  default (non-strict) mode such a view takes the reference's torch
  expression: output identical to torch's, no exception.
- fp16 activations take the HIP quantizers, as the reference's guards take
  them (triton_ltx_ops.py:1021-1022, :1489-1499): codes equal torch's on the
  GPU over every fp16 bit pattern.
- The grouped Q/K/V projections keep the reference's bookkeeping
  (:890-955, :2114-2178), and the Q/K/V paths run under
  torch.inference_mode, as the reference's pipeline calls them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.torch_ref as tr
from oracle import ltx_ops as O
from oracle.numerics import T, f16_from_bits
from tests.helpers import assert_same_bits, nan_canon, np32, randn

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _calls():
    from opengenie_amd import ltx_ops

    ltx_ops.reset_hip_calls()
    yield


def _calls_now() -> dict:
    from opengenie_amd import ltx_ops

    return ltx_ops.collect_hip_calls()


def g(t: torch.Tensor) -> torch.Tensor:
    return t.to(DEV)


def odd(t: torch.Tensor) -> torch.Tensor:
    """The same values as a contiguous view starting one element past a
    16-byte boundary (storage offset 1)."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    assert v.is_contiguous() and v.data_ptr() % 16 != 0
    return v


def same(a: torch.Tensor, b: torch.Tensor) -> bool:
    torch.cuda.synchronize()
    if a.dtype == torch.float8_e4m3fn:
        return torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    return torch.equal(a, b)


# ------------------------------------------------ misaligned views, non-strict
def _ada_inputs(seed, tokens=37, cols=4096, rows=9):
    x = g(randn((1, tokens, cols), seed))
    y = g(randn((1, tokens, cols), seed + 1))
    table = g(randn((rows, cols), seed + 2, std=0.02))
    ts = g(randn((1, tokens, rows * cols), seed + 3, std=0.5))
    bias = g(randn((cols,), seed + 4, std=0.01))
    return x, y, table, ts, bias


def test_misaligned_ada_ops_take_the_torch_path(monkeypatch):
    from opengenie_amd import ltx_ops as L

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    x, y, table, ts, bias = _ada_inputs(10)
    xo, yo = odd(x), odd(y)
    # the references run on the very tensors passed (torch's own kernels may
    # take another reduction order for a misaligned view)
    assert same(L.fused_adazero_from_ada(xo, 1e-6, table, ts, shift_index=0, scale_index=1),
                tr.adazero_from_ada(xo, 1e-6, table, ts, 0, 1))
    scale, shift = tr.ada_values(table, ts, 1, x.shape[1], 4096, 1, 0)
    assert same(L.fused_adazero(xo, 1e-6, scale, shift), tr.adazero(xo, 1e-6, scale, shift))
    assert same(L.fused_adaln_affine_from_ada(xo, table, ts, shift_index=6, scale_index=7),
                tr.adaln_affine_from_ada(x, table, ts, 6, 7))
    assert same(L.fused_mul_from_ada(xo, table, ts, gate_index=8), tr.mul_from_ada(x, table, ts, 8))
    ref = tr.residual_gate_from_ada(x, y, table, ts, 8)
    assert same(L.fused_residual_gate_from_ada(xo, y, table, ts, gate_index=8), ref)
    assert same(L.fused_residual_gate_from_ada(x, yo, table, ts, gate_index=8), ref)
    ref = tr.residual_gate_bias_from_ada(x, y, bias, table, ts, 2)
    assert same(L.fused_residual_gate_bias_from_ada(xo, y, bias, table, ts, gate_index=2), ref)
    assert same(L.fused_residual_gate_bias_from_ada(x, yo, bias, table, ts, gate_index=2), ref)
    assert same(L.fused_residual_gate_bias_from_ada(x, y, odd(bias), table, ts, gate_index=2), ref)
    gate = g(randn((1, 1, 4096), 15))
    assert same(L.fused_residual_gate_bf16(xo, y, gate), tr.residual_gate(x, y, gate))
    assert same(L.fused_residual_gate_bf16(x, yo, gate), tr.residual_gate(x, y, gate))
    s = g(torch.tensor(4.0 / 448))
    q = L.fused_adazero_from_ada_fp8(xo, 1e-6, table, ts, s, shift_index=3, scale_index=4)
    assert same(q, tr.fp8_quantize_e4m3(tr.adazero_from_ada(xo, 1e-6, table, ts, 3, 4), s))
    calls = _calls_now()
    # none of the misaligned calls reached a kernel that reads the odd view
    for name in ("fused_adazero_from_ada", "fused_adazero", "fused_adaln_affine_from_ada", "fused_mul_from_ada",
                 "fused_residual_gate_bf16", "fused_adazero_from_ada_fp8"):
        assert name not in calls, (name, calls)


def test_misaligned_quantizers_take_the_torch_path(monkeypatch):
    from opengenie_amd import ltx_ops as L

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    for dtype in (torch.bfloat16, torch.float16):
        x = g(randn((33, 4096), 20, std=30.0).to(dtype))
        xo = odd(x)
        # the references run on the very tensors passed: torch's GPU gelu in
        # fp16 gives -0 on its vectorised (aligned) path and +0 on its scalar
        # path where tanh saturates to -1
        for s in (g(torch.tensor(0.05)), g(torch.tensor([0.05]))):
            assert same(L.fused_fp8_quantize_e4m3(xo, s), tr.fp8_quantize_e4m3(xo, s))
            assert same(L.fused_gelu_tanh_fp8_quantize_e4m3(xo, s), tr.gelu_tanh_fp8_quantize_e4m3(xo, s))
        xh = g(randn((1, 40, 32, 128), 21).to(dtype))
        qo, so = L.fused_fp8_quantize_e4m3_per_head_4d(odd(xh))
        qr, sr = tr.fp8_per_head(xh)
        assert same(qo, qr) and same(so, sr)
    calls = _calls_now()
    assert not any(k.startswith("fused_fp8") or k.startswith("fused_gelu") for k in calls), calls


def test_misaligned_preattention_takes_the_torch_path(monkeypatch):
    from opengenie_amd import ltx_ops as L

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    n = 45
    q = g(randn((1, n, 4096), 30))
    k = g(randn((1, n, 4096), 31))
    v = g(randn((1, n, 4096), 32))
    w = g(randn((4096,), 33, std=0.05, mean=1.0))
    freqs = randn((1, 32, n, 64), 34, dtype=torch.float32, std=3.0)
    cos, sin = g(freqs.cos().to(torch.bfloat16)), g(freqs.sin().to(torch.bfloat16))
    for args in ((odd(q), k, w, w), (q, odd(k), w, w), (q, k, odd(w), w), (q, k, w, odd(w))):
        # the reference on the very tensors passed (torch's rms_norm may take
        # another reduction order for a misaligned view)
        rq, rk = tr.video_qk_rmsnorm_rope(*args, 1e-6, cos, sin)
        oq, ok = L.fused_video_qk_rmsnorm_rope(*args, 1e-6, cos, sin)
        assert same(oq, rq) and same(ok, rk)
        oq, ok = L.fused_video_qk_rmsnorm_rope_separate(*args, 1e-6, cos, sin)
        assert same(oq, rq) and same(ok, rk)
    # the packed form has no torch path in the reference: None, no exception
    assert L.fused_video_qkv_rmsnorm_rope_pack(q, k, odd(v), w, w, 1e-6, cos, sin) is None
    assert L.fused_video_qkv_rmsnorm_rope_pack(odd(q), k, v, w, w, 1e-6, cos, sin) is None
    bias = g(randn((4096,), 35, std=0.01))
    ref = tr.video_qk_rmsnorm_rope(q + bias, k + bias, w, w, 1e-6, cos, sin)
    oq, ok = L.fused_video_qk_bias_rmsnorm_rope(q, k, odd(bias), bias, w, w, 1e-6, cos, sin)
    assert same(oq, ref[0]) and same(ok, ref[1])
    qo = odd(q)
    assert same(L.qk_rmsnorm(qo, w, 1e-6), torch.nn.functional.rms_norm(qo, (4096,), weight=w, eps=1e-6))
    calls = _calls_now()
    assert not any("rmsnorm" in k for k in calls), calls


def test_misaligned_attention_takes_the_torch_path(monkeypatch):
    from opengenie_amd import attention as A

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    q, k, v = (g(randn((1, 70, 4, 128), 40 + i)) for i in range(3))
    qo = odd(q)
    out = A.flash_attn_func(qo, k, v)
    assert same(out, A._torch_attention(qo, k, v, 128 ** -0.5, False))
    assert "flash_attn_func" not in _calls_now()


# ------------------------------------------------------- fp16 on the quantizers
ALL_F16 = f16_from_bits(np.arange(1 << 16, dtype=np.uint16))
F16_SCALES = (0.05, 0.37, 1.0, 3.3e-3, 2.0e-5)


@pytest.mark.parametrize("zero_dim", [True, False])
def test_fp8_quantize_exhaustive_f16(zero_dim, monkeypatch):
    """Every fp16 bit pattern at five scales (2e-5: 1/s beyond fp16's range,
    so a 0-dim scale's reciprocal becomes infinite in fp16 as torch's GPU
    multiply makes it): the HIP codes equal torch evaluating the reference
    expression on the GPU, and the oracle's GPU semantics."""
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3

    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    xt = g(torch.from_numpy(ALL_F16.copy()).to(torch.float16))
    for scale in F16_SCALES:
        s = torch.tensor(scale, dtype=torch.float32)
        if not zero_dim:
            s = s.reshape(1)
        got = fused_fp8_quantize_e4m3(xt, g(s)).view(torch.uint8).cpu().numpy()
        ref = tr.fp8_quantize_e4m3(xt, g(s)).view(torch.uint8).cpu().numpy()
        assert np.array_equal(nan_canon(got), nan_canon(ref)), (scale, int((got != ref).sum()))
        with np.errstate(over="ignore", invalid="ignore"):
            ours = O.fp8_quantize_e4m3(T(ALL_F16, "f16"), scale, zero_dim, device="cuda")
        assert np.array_equal(nan_canon(ours), nan_canon(ref)), scale
    assert _calls_now().get("fused_fp8_quantize_e4m3", 0) == len(F16_SCALES)


@pytest.mark.parametrize("zero_dim", [True, False])
def test_gelu_tanh_fp8_quantize_exhaustive_f16(zero_dim, monkeypatch):
    """Every fp16 input: the GELU quantizer's codes equal torch's GPU
    gelu(approximate='tanh') -> clamp -> e4m3 in fp16, and the oracle's fp16
    GELU equals torch's GPU gelu on every input."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    xt = g(torch.from_numpy(ALL_F16.copy()).to(torch.float16))
    for scale in (0.02, 0.37, 3.3e-3, 1.0):
        s = torch.tensor(scale, dtype=torch.float32)
        if not zero_dim:
            s = s.reshape(1)
        got = fused_gelu_tanh_fp8_quantize_e4m3(xt, g(s)).view(torch.uint8).cpu().numpy()
        ref = tr.gelu_tanh_fp8_quantize_e4m3(xt, g(s)).view(torch.uint8).cpu().numpy()
        assert np.array_equal(nan_canon(got), nan_canon(ref)), (scale, int((got != ref).sum()))
    ref_g = torch.nn.functional.gelu(xt, approximate="tanh").float().cpu().numpy()
    assert_same_bits(O.gelu_tanh(T(ALL_F16, "f16")).v, ref_g, "oracle fp16 gelu vs torch gpu")
    assert _calls_now().get("fused_gelu_tanh_fp8_quantize_e4m3", 0) == 4


def test_gelu_tables_of_both_dtypes_in_one_process(monkeypatch):
    """The bf16 and fp16 GELU tables are separate arrays, each built once on
    the GPU: alternating calls of the two dtypes, on two streams, keep giving
    torch's codes."""
    from opengenie_amd.ltx_ops import fused_gelu_tanh_fp8_quantize_e4m3

    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    s = g(torch.tensor(0.02))
    xs = {dt: g(randn((64, 4096), 50, std=3.0).to(dt)) for dt in (torch.bfloat16, torch.float16)}
    refs = {dt: tr.gelu_tanh_fp8_quantize_e4m3(x, s) for dt, x in xs.items()}
    side = torch.cuda.Stream()
    for i in range(6):
        dt = (torch.bfloat16, torch.float16)[i % 2]
        st = side if i % 3 == 2 else torch.cuda.current_stream()
        with torch.cuda.stream(st):
            q = fused_gelu_tanh_fp8_quantize_e4m3(xs[dt], s)
        st.synchronize()
        assert same(q, refs[dt]), (i, dt)


def test_fp8_per_head_f16(monkeypatch):
    """fp16 x [B, N, H, D] on the HIP per-head quantizer: scales and codes
    equal the oracle and torch's expression on the GPU (:976-980), with NaN,
    infinite, zero and subnormal elements in some heads."""
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    rng = np.random.default_rng(60)
    x = (rng.standard_normal((2, 77, 16, 64)) * 3).astype(np.float32)
    x[0, :, 1, :] = 0.0
    x[0, 5, 2, 3] = np.inf
    x[1, 9, 3, 0] = np.nan
    x[1, :, 4, :] = ALL_F16[rng.integers(1, 1024, size=(77, 64))]  # fp16 subnormals
    x[1, :, 5, :] = ALL_F16[rng.integers(0, 0x7C00, size=(77, 64))]  # every finite magnitude
    xt = torch.from_numpy(x).to(torch.float16)
    q, s = fused_fp8_quantize_e4m3_per_head_4d(g(xt))
    torch.cuda.synchronize()
    assert _calls_now().get("fused_fp8_quantize_e4m3_per_head_4d") == 1
    qr, sr = O.fp8_per_head_quantize(np32(xt))
    assert_same_bits(s.cpu().numpy(), sr, "per-head fp16 scale")
    got = q.view(torch.uint8).cpu().numpy()
    assert np.array_equal(nan_canon(got), nan_canon(qr))
    tq, ts = tr.fp8_per_head(g(xt))
    assert_same_bits(s.cpu().numpy(), ts.cpu().numpy(), "per-head fp16 scale vs torch")
    assert np.array_equal(nan_canon(got), nan_canon(tq.view(torch.uint8).cpu().numpy()))


# ------------------------------------------ grouped Q/K/V bookkeeping on the GPU
def _attn(seed):
    from opengenie_amd.block import random_video_block

    return random_video_block(4096, 32, seed=seed).attn1


def test_grouped_projection_stats_and_checks(monkeypatch):
    from opengenie_amd import ltx_ops as L

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    a = _attn(70)
    x = g(randn((1, 300, 4096), 71))
    L.reset_video_qkv_grouped_mm_stats(checks=1)
    L.reset_video_qk_grouped_mm_stats(checks=2)
    qkv = L.fp8_qkv_from_grouped_mm(a, x)
    qkv2 = L.fp8_qkv_from_grouped_mm(a, x)
    qk = L.fp8_qk_from_grouped_mm(a, x)
    assert qkv is not None and qk is not None and qkv2 is not None
    st = L.collect_video_qkv_grouped_mm_stats()
    assert st["calls"] == 2 and st["fallbacks"] == 0 and [c["tensor"] for c in st["checks"]] == ["q", "k", "v"]
    st2 = L.collect_video_qk_grouped_mm_stats()
    assert st2["calls"] == 1 and [c["tensor"] for c in st2["checks"]] == ["q", "k"]
    for c in st["checks"] + st2["checks"]:
        # the grouped kernel and the per-linear kernel share the roundings;
        # only the float32 summation order may differ
        assert c["rms"] < 1e-2 * 0.1 and c["mean_rel"] < 1e-2, c
    for out, lin in zip(qkv, (a.to_q, a.to_k, a.to_v)):
        ref = L.fp8_linear_forward(lin, x)
        assert out.shape == ref.shape == (1, 300, 4096)
    # guard reasons, in the reference's words
    b = _attn(72)
    b.to_k.input_scale = b.to_k.input_scale * 2
    assert L.fp8_qkv_from_grouped_mm(b, x) is None
    assert L.fp8_qk_from_grouped_mm(b, x) is None
    c = _attn(73)
    c.to_v.weight_scale = c.to_v.weight_scale.reshape(1).expand(2).contiguous()
    assert L.fp8_qkv_from_grouped_mm(c, x) is None
    assert L.fp8_qkv_from_grouped_mm(a, x[:, :, :2048].contiguous()) is None
    assert L.fp8_qkv_from_grouped_mm(a, x.float()) is None
    st = L.collect_video_qkv_grouped_mm_stats()
    assert st["calls"] == 2 and st["fallbacks"] == 4
    assert st["fallback_reasons"] == {"input_scale": 1, "scale_shape": 1, "shape": 1, "input": 1}
    assert L.collect_video_qk_grouped_mm_stats()["fallback_reasons"] == {"input_scale": 1}


def test_qkv_paths_under_inference_mode(monkeypatch):
    """The reference runs its pipeline, model loading included, under
    torch.inference_mode, so the linears' scales are inference tensors. Every
    Q/K/V path then works and gives the same projections as outside it, with
    and without frozen scales declared."""
    from opengenie_amd import ltx_ops as L
    from opengenie_amd.block import random_video_block

    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    x = g(randn((1, 260, 4096), 80))
    outside = _attn(81)
    refs = L.fp8_qkv_from_grouped_mm(outside, x)
    refs_qk = L.fp8_qk_from_grouped_mm(outside, x)
    for frozen in (False, True):
        prev = L.set_frozen_fp8_scales(frozen)
        try:
            with torch.inference_mode():
                a = random_video_block(4096, 32, seed=81).attn1
                assert a.to_q.input_scale.is_inference()
                for fn in (L.fp8_qkv_from_grouped_mm, L.fp8_qkv_from_shared_quantized_input,
                           L.fp8_qkv_from_packed_requant):
                    out = fn(a, x)
                    assert out is not None, fn.__name__
                    if fn is L.fp8_qkv_from_grouped_mm:
                        for o, r in zip(out, refs):
                            assert same(o, r)
                qk = L.fp8_qk_from_grouped_mm(a, x)
                assert qk is not None and same(qk[0], refs_qk[0]) and same(qk[1], refs_qk[1])
                # the packed form needs equal weight scales as well
                a.to_k.weight_scale = a.to_q.weight_scale
                a.to_v.weight_scale = a.to_q.weight_scale
                assert L.fp8_qkv_from_packed_linear(a, x) is not None
        finally:
            L.set_frozen_fp8_scales(prev)
