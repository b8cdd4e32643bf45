"""Guard behaviour of the drop-in host module on the CPU.

As in the reference, an input the fused kernel does not take falls back to
the reference's torch expression; on CPU tensors every op takes that path,
which is checked here against torch evaluating the same expression. Guard
reason strings follow triton_ltx_ops.py:1513-1537."""

from __future__ import annotations

import pytest
import torch

import oracle.torch_ref as tr
from opengenie_amd import ltx_ops as L
from tests.helpers import randn


def test_cpu_inputs_take_the_torch_path():
    x = randn((1, 9, 2048), 1)
    table = randn((6, 2048), 2, dtype=torch.float32)
    ts = randn((1, 9, 6 * 2048), 3)
    L.reset_hip_calls()
    out = L.fused_adazero_from_ada(x, 1e-6, table, ts, shift_index=3, scale_index=4)
    assert torch.equal(out, tr.adazero_from_ada(x, 1e-6, table, ts, 3, 4))
    assert L.collect_hip_calls() == {}


def test_cpu_fallbacks_equal_reference_expressions():
    x = randn((1, 9, 2048), 4)
    y = randn((1, 9, 2048), 5)
    table = randn((9, 2048), 6, dtype=torch.float32)
    ts = randn((1, 9, 9 * 2048), 7)
    bias = randn((2048,), 8, dtype=torch.float32)
    assert torch.equal(L.fused_adaln_affine_from_ada(x, table, ts, shift_index=6, scale_index=7),
                       tr.adaln_affine_from_ada(x, table, ts, 6, 7))
    assert torch.equal(L.fused_residual_gate_from_ada(x, y, table, ts, gate_index=8),
                       tr.residual_gate_from_ada(x, y, table, ts, 8))
    assert torch.equal(L.fused_residual_gate_bias_from_ada(x, y, bias, table, ts, gate_index=8),
                       tr.residual_gate_bias_from_ada(x, y, bias, table, ts, 8))
    assert torch.equal(L.fused_mul_from_ada(x, table, ts, gate_index=8), tr.mul_from_ada(x, table, ts, 8))
    assert torch.equal(L.fused_bias_add_bf16(x, bias), tr.bias_add(x, bias))
    s = torch.tensor(0.05)
    assert torch.equal(L.fused_fp8_quantize_e4m3(x, s).view(torch.uint8),
                       tr.fp8_quantize_e4m3(x, s).view(torch.uint8))


def test_adazero_fp8_cpu_path_is_the_composition():
    """fused_adazero_from_ada_fp8 on CPU tensors: the torch AdaZero expression
    followed by the FP8Linear input quantizer, code for code."""
    x = randn((1, 9, 2048), 11)
    table = randn((6, 2048), 12, dtype=torch.float32)
    ts = randn((1, 9, 6 * 2048), 13)
    s = torch.tensor(4.0 / 448)
    L.reset_hip_calls()
    q = L.fused_adazero_from_ada_fp8(x, 1e-6, table, ts, s, shift_index=3, scale_index=4)
    ref = tr.fp8_quantize_e4m3(tr.adazero_from_ada(x, 1e-6, table, ts, 3, 4), s)
    assert q.dtype == torch.float8_e4m3fn and torch.equal(q.view(torch.uint8), ref.view(torch.uint8))
    assert L.collect_hip_calls() == {}


def test_qkv_from_codes_guard():
    """fp8_qkv_from_quantized_e4m3 takes only contiguous e4m3 GPU codes of a
    (1, N, 4096) input; anything else returns None, as the grouped guard does."""
    from opengenie_amd.block import random_video_block

    blk = random_video_block(4096, 32, device="cpu", seed=5)
    codes = torch.zeros((1, 4, 4096), dtype=torch.float8_e4m3fn)
    assert L.fp8_qkv_from_quantized_e4m3(blk.attn1, codes, out_dtype=torch.bfloat16) is None
    assert L.fp8_qkv_from_quantized_e4m3(blk.attn1, codes.view(torch.uint8).to(torch.bfloat16),
                                         out_dtype=torch.bfloat16) is None


def test_residual_mode_selection():
    x, y, gate = randn((1, 3, 2048), 1), randn((1, 3, 2048), 2), randn((1, 3, 2048), 3)
    try:
        L.set_block_residual_mode("addcmul")
        assert torch.equal(L._simple_residual_gate(x, y, gate), torch.addcmul(x, y, gate))
        L.set_block_residual_mode("triton_simple_bf16_round")
        assert torch.equal(L._simple_residual_gate(x, y, gate), x + y * gate)
        with pytest.raises(ValueError):
            L.set_block_residual_mode("bogus")
    finally:
        L.set_block_residual_mode("triton_simple_bf16_round")


def test_preattention_guard_reasons():
    q = randn((1, 5, 4096), 1)
    w = randn((4096,), 2)
    cos = randn((1, 32, 5, 64), 3)
    assert L._fused_video_qk_rmsnorm_rope_guard_reason(q, q, w, w, cos, cos) == "qk_device_or_dtype"
    # The torch path is the reference's test restatement.
    oq, ok = L.fused_video_qk_rmsnorm_rope(q, q, w, w, 1e-6, cos, cos)
    rq, rk = tr.video_qk_rmsnorm_rope(q, q, w, w, 1e-6, cos, cos)
    assert torch.equal(oq, rq) and torch.equal(ok, rk)


def test_pack_returns_none_when_guard_fails():
    q = randn((1, 5, 4096), 1)
    w = randn((4096,), 2)
    cos = randn((1, 32, 5, 64), 3)
    assert L.fused_video_qkv_rmsnorm_rope_pack(q, q, q, w, w, 1e-6, cos, cos) is None


def test_ada_index_and_shape_errors():
    x = randn((1, 4, 2048), 1)
    table = randn((6, 2048), 2)
    ts = randn((1, 5, 6 * 2048), 3)  # token count mismatch
    with pytest.raises(ValueError):
        L.fused_adazero_from_ada(x, 1e-6, table, ts, shift_index=0, scale_index=1)


def test_strict_mode_only_affects_gpu_tensors(monkeypatch):
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    x = randn((1, 3, 2048), 1)
    bias = randn((2048,), 2)
    assert torch.equal(L.fused_bias_add_bf16(x, bias), tr.bias_add(x, bias))


def test_per_head_cpu_path():
    x = randn((1, 8, 4, 64), 9)
    q, s = L.fused_fp8_quantize_e4m3_per_head_4d(x)
    qr, sr = tr.fp8_per_head(x)
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s, sr)


def test_scale_equality_memo_follows_the_tensors():
    """With frozen scales declared, the Q/K/V guards' torch.equal of the input
    (and weight) scales is remembered per tuple of tensors and recomputed when
    a tensor changes in place, is replaced, or another tensor takes its place."""
    a = torch.tensor([0.5])
    b = torch.tensor([0.5])
    c = torch.tensor([0.5])
    with L.frozen_fp8_scales():
        assert L._all_equal([a, b, c])
        assert L._all_equal([a, b, c])  # remembered
        c.mul_(2.0)  # in place: version counter moves
        assert not L._all_equal([a, b, c])
        c.copy_(torch.tensor([0.5]))
        assert L._all_equal([a, b, c])
        c.data = torch.tensor([0.25])  # new storage
        assert not L._all_equal([a, b, c])
        d = torch.tensor([0.5])
        assert L._all_equal([a, b, d])
        assert not L._all_equal([a, torch.tensor([0.5, 0.5]), d])  # shapes differ: torch.equal is False
        for trial in range(3):  # fresh tensors each time (ids may be reused after collection)
            x, y = torch.tensor([float(trial)]), torch.tensor([float(trial) + (trial % 2)])
            assert L._all_equal([x, y]) == torch.equal(x, y)
    assert not L._FROZEN_SCALES and not L._EQUAL_MEMO


def test_scale_equality_default_compares_every_call():
    """By default (as the reference) every call compares: a write through
    `.data`, which the version counter does not see, is still noticed."""
    a = torch.tensor([0.5])
    b = torch.tensor([0.5])
    assert L._all_equal([a, b])
    b.data.copy_(torch.tensor([0.25]))
    assert not L._all_equal([a, b])
    b.data.copy_(torch.tensor([0.5]))
    assert L._all_equal([a, b])


@pytest.mark.parametrize("frozen", [False, True])
def test_scale_equality_under_inference_mode(frozen):
    """Scales created under torch.inference_mode (as the reference loads its
    model) have no version counter; the comparison works on them either way."""
    with torch.inference_mode():
        a = torch.tensor([0.5])
        b = torch.tensor([0.5])
        c = torch.tensor([0.75])
    prev = L.set_frozen_fp8_scales(frozen)
    try:
        with torch.inference_mode():
            assert L._all_equal([a, b])
            assert not L._all_equal([a, c])
            assert L._all_equal([a, b])
        assert L._all_equal([a, b]) and not L._all_equal([b, c])
    finally:
        L.set_frozen_fp8_scales(prev)


def _cpu_attn(seed=5):
    from opengenie_amd.block import random_video_block

    return random_video_block(4096, 32, device="cpu", seed=seed).attn1


@pytest.mark.parametrize("kind", ["qkv", "qk"])
def test_grouped_projection_bookkeeping_on_cpu(kind, monkeypatch):
    """fp8_qkv_from_grouped_mm / fp8_qk_from_grouped_mm keep the reference's
    bookkeeping (:890-955, :2114-2178): a failing guard returns None and
    counts its reason; an exception inside the projection returns None and
    counts its type name; under OPENGENIE_AMD_STRICT it propagates."""
    fn = L.fp8_qkv_from_grouped_mm if kind == "qkv" else L.fp8_qk_from_grouped_mm
    reset = L.reset_video_qkv_grouped_mm_stats if kind == "qkv" else L.reset_video_qk_grouped_mm_stats
    collect = L.collect_video_qkv_grouped_mm_stats if kind == "qkv" else L.collect_video_qk_grouped_mm_stats
    attn = _cpu_attn()
    x = randn((1, 4, 4096), 1)
    reset(checks=1)
    assert fn(attn, x) is None  # CPU input: the guard's "input" reason
    assert fn(attn, x[:, :, :2048]) is None
    st = collect()
    assert st == {"calls": 0, "fallbacks": 2, "fallback_reasons": {"input": 2}, "checks": []}

    def boom(*a, **k):
        raise RuntimeError("forced from the host")

    monkeypatch.setattr(L, "_grouped_guard_reason", lambda *a: None)
    monkeypatch.setattr(L, "_fp8_grouped_linear", boom)
    assert fn(attn, x) is None
    assert collect()["fallback_reasons"] == {"input": 2, "RuntimeError": 1}
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    with pytest.raises(RuntimeError):
        fn(attn, x)
    monkeypatch.delenv("OPENGENIE_AMD_STRICT")
    reset()
    assert collect() == {"calls": 0, "fallbacks": 0, "fallback_reasons": {}, "checks": []}


def test_grouped_guard_reasons_follow_the_reference_order():
    """The reasons of :1187-1233 in the reference's order, for the conditions
    that do not need a GPU tensor to reach (the device check comes first)."""
    attn = _cpu_attn(6)
    x = randn((1, 4, 4096), 2)
    names = ("to_q", "to_k", "to_v")
    assert L._grouped_guard_reason(attn, x, names) == "input"
    assert L._grouped_guard_reason(attn, x.float(), names) == "input"


def test_misaligned_views_fall_back_before_the_library():
    """A contiguous view at an odd storage offset passes the reference's
    guards; the guards here also check the C ABI's 16-byte precondition, so
    such a view takes the torch path (on the GPU the same guard sends it
    there instead of to an argument error)."""
    buf = torch.zeros(1 + 2 * 4096, dtype=torch.bfloat16)
    x = buf[1:].view(1, 2, 4096)
    assert x.is_contiguous() and x.data_ptr() % 16 == 2
    assert not L._aligned(x)
    assert L._vec_ok(buf[1:4097], torch.bfloat16) is False
    assert L._vec_ok(buf[1:4097], torch.float32) is True  # a converted copy is aligned
    assert L._vec_ok(buf[1:8193:2], torch.bfloat16) is True  # .contiguous() copies it
