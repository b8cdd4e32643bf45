"""The reference's torch expressions for each fused op, evaluated by torch.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). These are the
one-to-three-line torch fallbacks of `ltx_serve/triton_ltx_ops.py` (file:line
cited per function), written out so that torch itself evaluates them on
whatever device the inputs live on. They are the ground truth the numpy
oracle is pinned against, a second check of the HIP kernels on the GPU, and
the CPU baseline that bench.py times on the host's cores. Nothing here is
imported by the product package.
"""

from __future__ import annotations

import torch


def ada_values(table, timestep, batch, tokens, cols, *indices):
    """:983-998"""
    ts_view = timestep.reshape(batch, timestep.shape[1], table.shape[0], -1)
    tab = table.to(device=timestep.device, dtype=timestep.dtype)
    return tuple(tab[i].view(1, 1, cols) + ts_view[:, :, i, :] for i in indices)


def adazero(x, eps, scale, shift):
    """:9-10"""
    return torch.nn.functional.rms_norm(x, (x.shape[-1],), eps=eps) * (1 + scale) + shift


def adazero_from_ada(x, eps, table, timestep, shift_index, scale_index):
    """:50-60"""
    shift, scale = ada_values(table, timestep, x.shape[0], x.shape[1], x.shape[-1], shift_index, scale_index)
    return adazero(x, eps, scale, shift)


def adaln_affine_from_ada(x, table, timestep, shift_index, scale_index):
    """:102-112"""
    shift, scale = ada_values(table, timestep, x.shape[0], x.shape[1], x.shape[-1], shift_index, scale_index)
    return x * (1 + scale) + shift


def mul_from_ada(x, table, timestep, gate_index):
    """:702-711"""
    (gate,) = ada_values(table, timestep, x.shape[0], x.shape[1], x.shape[-1], gate_index)
    return x * gate


def residual_gate(x, y, gate):
    """:591-592 and the production `_simple_residual_gate` (:1955-1960)."""
    return x + y * gate


def residual_gate_from_ada(x, y, table, timestep, gate_index):
    """:650-659"""
    (gate,) = ada_values(table, timestep, x.shape[0], x.shape[1], x.shape[-1], gate_index)
    return residual_gate(x, y, gate)


def bias_add(x, bias):
    """:186-187"""
    return x + bias.to(x.dtype)


def residual_gate_bias_from_ada(x, y_no_bias, bias, table, timestep, gate_index):
    """:220-228"""
    y = y_no_bias + bias.to(y_no_bias.dtype)
    return residual_gate_from_ada(x, y, table, timestep, gate_index)


def head_gate_mul(out, gates, heads, dim_head):
    """:615-619"""
    b, n, _ = out.shape
    return (out.view(b, n, heads, dim_head) * gates.unsqueeze(-1)).view(b, n, heads * dim_head)


def fp8_quantize_e4m3(x, input_scale):
    """:146-148"""
    lo = torch.finfo(torch.float8_e4m3fn).min
    hi = torch.finfo(torch.float8_e4m3fn).max
    return torch.clamp(x * input_scale.reciprocal(), lo, hi).to(torch.float8_e4m3fn)


def gelu_tanh_fp8_quantize_e4m3(x, input_scale):
    """:165-169"""
    g = torch.nn.functional.gelu(x, approximate="tanh")
    lo = torch.finfo(torch.float8_e4m3fn).min
    hi = torch.finfo(torch.float8_e4m3fn).max
    return torch.clamp(g * input_scale.reciprocal(), lo, hi).to(torch.float8_e4m3fn)


def fp8_per_head(x):
    """:976-980"""
    m = torch.finfo(torch.float8_e4m3fn).max
    scale = x.float().abs().amax(dim=(1, 3)).clamp_min(1e-12) / m
    q = torch.clamp(x.float() / scale[:, None, :, None], -m, m).to(torch.float8_e4m3fn)
    return q, scale.to(torch.float32).contiguous()


def split_rope(x, cos, sin):
    """tests/test_triton_ltx_ops.py:232-249 (the reference's own restatement)."""
    b, n, dim = x.shape
    heads = cos.shape[1]
    hd = dim // heads
    half = hd // 2
    xh = x.reshape(b, n, heads, hd).transpose(1, 2)
    first = xh[..., :half]
    second = xh[..., half:]
    o1 = first * cos - second * sin
    o2 = second * cos + first * sin
    return torch.cat([o1, o2], dim=-1).transpose(1, 2).reshape(b, n, dim)


def video_qk_rmsnorm_rope(q, k, qw, kw, eps, cos, sin):
    """:958-973 with the split RoPE restatement above."""
    qn = torch.nn.functional.rms_norm(q, (q.shape[-1],), weight=qw, eps=eps)
    kn = torch.nn.functional.rms_norm(k, (k.shape[-1],), weight=kw, eps=eps)
    return split_rope(qn, cos, sin), split_rope(kn, cos, sin)


def fp8_linear(qinput, weight, input_scale, weight_scale, bias, out_dtype=torch.bfloat16):
    """:742-759 / :1691-1709: _scaled_mm then `+ bias.to(out_dtype)`."""
    out = torch._scaled_mm(qinput, weight.t(), scale_a=input_scale, scale_b=weight_scale,
                           out_dtype=out_dtype)
    if bias is not None:
        out = out + bias.to(out.dtype)
    return out


def fp8_linear_decoded(qinput, weight, input_scale, weight_scale, bias, out_dtype=torch.bfloat16):
    """The arithmetic of :1691-1709 with torch's float32 matmul of the decoded
    e4m3 codes in place of torch._scaled_mm (which runs below 1 GFLOP/s on a
    CPU): R(R(acc * (scale_a * scale_b)) + R(bias)), acc the float32 sum of
    the exact code products."""
    acc = qinput.float() @ weight.float().t()
    out = (acc * (input_scale.float() * weight_scale.float())).to(out_dtype)
    if bias is not None:
        out = out + bias.to(out.dtype)
    return out


def attention(q, k, v, scale=None):
    """Dense video self-attention as the reference computes it with FA3
    (official_ltx23_benchmark.py:3294-3369): softmax(q k^T * scale) v,
    non-causal, here through torch's scaled_dot_product_attention on
    [B, H, N, D] tensors."""
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale)


def fp8_requantize_common_scale(weight, weight_scale, common_scale):
    """:1331-1333"""
    dequant = weight.float() * weight_scale.detach().float()
    lo = torch.finfo(torch.float8_e4m3fn).min
    hi = torch.finfo(torch.float8_e4m3fn).max
    return torch.clamp(dequant / common_scale, lo, hi).to(torch.float8_e4m3fn)
