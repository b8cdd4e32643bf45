"""Dense video self-attention on MI355X: drop-in for the FlashAttention-3 call
the reference makes in the LTX video self-attention.

The reference replaces `ltx_core`'s `FlashAttention3.__call__(q, k, v, heads)`
with a function that views q/k/v (B, N, H*D) as [B, N, H, D], calls
`flash_attn_interface.flash_attn_func(q, k, v, q_descale=..., k_descale=...,
v_descale=..., window_size=...)` and reshapes the [B, N, H, D] result back
(benchmarks/official_ltx23_benchmark.py:3294-3369). FP8 inputs come from the
per-head quantizer (`_to_fp8_per_head`, :3333-3340) with descales [B, H].

`flash_attn_func` here takes the same arguments for the configuration the
reference uses (non-causal, no window) and runs the gfx950 HIP kernels
`oga_attention_ws` (bf16) and `oga_attention_fp8_ws` (e4m3 with descales) on
torch's current stream. Inputs the kernel does not cover
(CPU tensors, head_dim != 128, causal or windowed attention, a softmax scale
that is not positive, other dtypes)
take torch's scaled_dot_product_attention, like the fused ops' torch paths;
under OPENGENIE_AMD_STRICT=1 a GPU input that would fall back raises instead.
"""

from __future__ import annotations

import torch

from . import _lib
from .ltx_ops import _fallback, _hip, _stream, fused_fp8_quantize_e4m3

__all__ = ["flash_attn_func", "attention_video", "attention_video_e4m3_out"]

_FP8 = torch.float8_e4m3fn


def _strides3(t: torch.Tensor):
    return _lib.strides([t.stride(0), t.stride(1), t.stride(2)])


def _kernel_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    for t in (q, k, v):
        if not t.is_cuda or t.ndim != 4 or t.shape[-1] != 128 or t.stride(-1) != 1:
            return False
        if any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
            return False
    if q.shape[0] != k.shape[0] or k.shape != v.shape or q.shape[2] != k.shape[2]:
        return False
    return k.shape[1] > 0


def _dequant(x: torch.Tensor, descale: torch.Tensor) -> torch.Tensor:
    """e4m3 [B, N, H, D] with float32 descale [B, H] -> bf16, one rounding."""
    b, n, h, d = x.shape
    out = torch.empty((b, n, h, d), device=x.device, dtype=torch.bfloat16)
    xc = x.contiguous()
    ds = descale.to(torch.float32).reshape(b, h).contiguous()
    _lib.call("oga_fp8_dequant_per_head", xc.data_ptr(), ds.data_ptr(), out.data_ptr(), b, n, h, d, _stream(x))
    return out


def _fp8_kernel_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, descales) -> bool:
    for t in (q, k, v):
        if not t.is_cuda or t.ndim != 4 or t.shape[-1] != 128 or t.stride(-1) != 1:
            return False
        if any(s % 16 for s in t.stride()[:3]) or t.data_ptr() % 16:
            return False
    if q.shape[0] != k.shape[0] or k.shape != v.shape or q.shape[2] != k.shape[2] or k.shape[1] < 1:
        return False
    if not 0 <= k.stride(1) <= 1 << 26 or k.shape[1] > 1 << 25:  # the kernel's 32-bit DMA offsets
        return False
    b, h = q.shape[0], q.shape[2]
    return b <= 65535 and h <= 65535 and all(d.is_cuda and d.numel() == b * h for d in descales)


def _fp8_attention(q, k, v, q_descale, k_descale, v_descale, softmax_scale) -> torch.Tensor:
    """The e4m3 kernel: both products on FP8 MFMA, P rounded to e4m3."""
    b, nq, h, d = q.shape
    nk = k.shape[1]
    ds = [t.to(torch.float32).reshape(b, h).contiguous() for t in (q_descale, k_descale, v_descale)]
    out = torch.empty((b, nq, h, d), device=q.device, dtype=torch.bfloat16)
    ws_bytes = int(_lib.load().oga_attention_fp8_workspace_bytes(b, nq, nk, h, d))
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    _hip("flash_attn_func_fp8")
    _lib.call("oga_attention_fp8_ws", q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(),
              _strides3(v), ds[0].data_ptr(), ds[1].data_ptr(), ds[2].data_ptr(), out.data_ptr(), _strides3(out),
              b, nq, nk, h, d, float(softmax_scale), ws.data_ptr(), ws_bytes, _stream(q))
    return out


def _torch_attention(q, k, v, softmax_scale, causal):
    qf, kf, vf = (t.float().transpose(1, 2) for t in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, is_causal=causal, scale=softmax_scale)
    return o.transpose(1, 2).to(torch.bfloat16)


def flash_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    softmax_scale: float | None = None,
    causal: bool = False,
    q_descale: torch.Tensor | None = None,
    k_descale: torch.Tensor | None = None,
    v_descale: torch.Tensor | None = None,
    window_size: tuple[int, int] = (-1, -1),
    attention_chunk: int = 0,
    num_splits: int = 1,
    sm_margin: int = 0,
) -> torch.Tensor:
    """softmax(q k^T * scale) v for q [B, Nq, H, D], k/v [B, Nk, H, D] -> [B, Nq, H, D] bf16.

    e4m3 q, k and v with their [B, H] descales run the FP8 kernel, as FA3's
    FP8 path does: S = (q8 k8^T) qd kd scale on e4m3 MFMA, P rounded to e4m3,
    O = (P8 v8) vd / l. Other e4m3 inputs (mixed dtypes, layouts the kernel
    does not take) are dequantized with their descales (value * descale,
    rounded to bf16) for the bf16 kernel. `attention_chunk`, `num_splits` and
    `sm_margin` are FA3 scheduling knobs with no effect on the result.
    """
    del attention_chunk, num_splits, sm_margin
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    unsupported = causal or tuple(window_size) != (-1, -1) or not (0.0 < float(softmax_scale) < float("inf"))
    descales = (q_descale, k_descale, v_descale)
    if (not unsupported and all(t.dtype == _FP8 for t in (q, k, v)) and all(d is not None for d in descales)
            and _fp8_kernel_ok(q, k, v, descales)):
        return _fp8_attention(q, k, v, q_descale, k_descale, v_descale, softmax_scale)
    deq = []
    for t, ds in ((q, q_descale), (k, k_descale), (v, v_descale)):
        if t.dtype == _FP8:
            if ds is None:
                raise ValueError("float8_e4m3fn attention inputs need their descale")
            # the kernel reads 16-byte pieces of the contiguous codes
            if t.is_cuda and t.ndim == 4 and t.shape[-1] % 16 == 0 and (not t.is_contiguous()
                                                                       or t.data_ptr() % 16 == 0):
                _hip("fp8_dequant_per_head")
                t = _dequant(t, ds)
            else:
                t = (t.float() * ds.float()[:, None, :, None]).to(torch.bfloat16)
        deq.append(t)
    q, k, v = deq
    # The kernel takes the scale into its base-2 exponent with the running
    # max, which needs a positive scale.
    if unsupported or any(t.dtype != torch.bfloat16 for t in (q, k, v)) or not _kernel_ok(q, k, v):
        _fallback("flash_attn_func", q, k, v)
        return _torch_attention(q, k, v, softmax_scale, causal)
    b, nq, h, d = q.shape
    nk = k.shape[1]
    out = torch.empty((b, nq, h, d), device=q.device, dtype=torch.bfloat16)
    _hip("flash_attn_func")
    # Workspace for the key-split parts of a last partial round of blocks
    # (torch's caching allocator makes the per-call tensor cheap).
    ws_bytes = int(_lib.load().oga_attention_workspace_bytes(b, nq, nk, h, d))
    ws = torch.empty((ws_bytes // 4,), device=q.device, dtype=torch.float32) if ws_bytes else None
    _lib.call("oga_attention_ws", q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(), _strides3(v),
              out.data_ptr(), _strides3(out), b, nq, nk, h, d, float(softmax_scale),
              ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q))
    return out


def attention_video(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, *,
                    q_descale=None, k_descale=None, v_descale=None) -> torch.Tensor:
    """`FlashAttention3.__call__(q, k, v, heads)` as patched by the reference
    (official_ltx23_benchmark.py:3294-3369): (B, N, H*D) in and out."""
    b = q.shape[0]
    dim_head = q.shape[-1] // heads
    qv, kv, vv = (t.view(b, -1, heads, dim_head) for t in (q, k, v))
    out = flash_attn_func(qv, kv, vv, q_descale=q_descale, k_descale=k_descale, v_descale=v_descale)
    return out.reshape(b, -1, heads * dim_head)


def attention_video_e4m3_out(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int,
                             input_scale: torch.Tensor) -> torch.Tensor:
    """`attention_video(q, k, v, heads)` handed to the FP8 linear that reads
    it: the e4m3 codes `fused_fp8_quantize_e4m3(attention_video(...),
    input_scale)` (:144-161; the attention module's to_out quantizes its
    input so, :1691-1709 / :762-781), from one HIP pass whose epilogue
    quantizes the bf16 output instead of writing it
    (`oga_attention_e4m3_out_ws`). No counterpart in the reference; bit for
    bit the two calls. Inputs the bf16 kernel does not take, or a scale the
    quantizer does not take, run the two calls."""
    b = q.shape[0]
    dim_head = q.shape[-1] // heads
    qv, kv, vv = (t.view(b, -1, heads, dim_head) for t in (q, k, v))
    # the quantizer's guard (:1021-1022, the HIP quantizer's float32 scale on
    # the same device) holds for the fresh bf16 output the two calls make
    ok = (all(t.dtype == torch.bfloat16 for t in (qv, kv, vv)) and _kernel_ok(qv, kv, vv)
          and isinstance(input_scale, torch.Tensor) and input_scale.numel() == 1 and input_scale.is_cuda
          and input_scale.dtype == torch.float32 and input_scale.device == q.device)
    if not ok:
        _fallback("attention_video_e4m3_out", q, k, v)
        return fused_fp8_quantize_e4m3(attention_video(q, k, v, heads), input_scale)
    nq, nk = qv.shape[1], kv.shape[1]
    out = torch.empty((b, nq, heads * dim_head), device=q.device, dtype=_FP8)
    ov = out.view(b, nq, heads, dim_head)
    _hip("attention_video_e4m3_out")
    ws_bytes = int(_lib.load().oga_attention_workspace_bytes(b, nq, nk, heads, dim_head))
    ws = torch.empty((ws_bytes // 4,), device=q.device, dtype=torch.float32) if ws_bytes else None
    _lib.call("oga_attention_e4m3_out_ws", qv.data_ptr(), _strides3(qv), kv.data_ptr(), _strides3(kv), vv.data_ptr(),
              _strides3(vv), ov.data_ptr(), _strides3(ov), b, nq, nk, heads, dim_head, float(dim_head ** -0.5),
              input_scale.data_ptr(), int(input_scale.dim() == 0), ws.data_ptr() if ws is not None else None,
              ws_bytes, _stream(q))
    return out
