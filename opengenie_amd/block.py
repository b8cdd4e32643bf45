"""One LTX-2.3 video transformer-block slice on this library's kernels, in the
order the patched `BasicAVTransformerBlock.forward` runs its video branches
with the production flags (ltx_serve/triton_ltx_ops.py:2989-3298):

  self-attention   :3006-3083  AdaZero(shift 0, scale 1) -> to_q, to_k, to_v
                               FP8 linears (:1671-1718) -> Q/K RMSNorm + RoPE
                               (:1810-1875) -> attention (:2636) -> optional
                               per-head gate (:2282-2302) -> to_out FP8 linear
                               without bias (:762-781) -> residual gate + bias
                               (gate 2, :3057-3064)
  text cross-attn  :2810-2888  rms_norm -> AdaLN affine (6, 7); the context
                               affine from the prompt table in torch (as in
                               production, :2852-2856); the attention module's
                               own forward: FP8 linears, q/k RMSNorm (torch),
                               attention, to_out with bias -> residual gate
                               (gate 8)
  feed-forward     :3224-3258  AdaZero(3, 4) -> FP8 up-projection + bias ->
                               GELU-tanh -> FP8 down-projection + bias ->
                               residual gate (gate 5)

`ltx_core` (the model library the reference patches) is not a dependency: the
block's parameters are plain tensors and duck-typed FP8 linears carrying the
attributes of the reference's FP8Linear (e4m3 `weight` [N, K], float32
`weight_scale` and `input_scale`, bf16 `bias`). `random_video_block` draws
synthetic parameters of the LTX-2.3 video block's shapes (no checkpoint).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import ltx_ops as L
from .attention import attention_video, attention_video_e4m3_out

_FP8 = torch.float8_e4m3fn


class FP8Linear(torch.nn.Module):
    """Per-tensor-scaled FP8 linear: weight codes e4m3 [out, in], weight and
    input scales as float32 scalars, bf16 bias (or None)."""

    def __init__(self, weight: torch.Tensor, weight_scale: torch.Tensor, input_scale: torch.Tensor,
                 bias: torch.Tensor | None):
        super().__init__()
        self.weight = weight
        self.weight_scale = weight_scale
        self.input_scale = input_scale
        self.bias = bias

    @staticmethod
    def quantized(w: torch.Tensor, input_scale: float, bias: torch.Tensor | None) -> "FP8Linear":
        """From float weights: weight_scale = amax / 448, codes = e4m3(w / scale)."""
        ws = (w.abs().amax().float() / 448.0).clamp_min(1e-12)
        codes = (w.float() / ws).clamp(-448.0, 448.0).to(_FP8)
        return FP8Linear(codes, ws.reshape(()), torch.tensor(float(input_scale), device=w.device), bias)


@dataclass
class VideoAttention:
    to_q: FP8Linear
    to_k: FP8Linear
    to_v: FP8Linear
    to_out: FP8Linear
    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor
    heads: int
    to_gate_logits: torch.nn.Linear | None = None


@dataclass
class VideoBlock:
    table: torch.Tensor          # scale_shift_table (9, C)
    prompt_table: torch.Tensor   # prompt_scale_shift_table (2, C)
    attn1: VideoAttention        # video self-attention
    attn2: VideoAttention        # video -> text cross-attention
    ff_up: FP8Linear             # C -> 4C, GELU-tanh after it
    ff_down: FP8Linear           # 4C -> C
    eps: float = 1e-6


def random_video_block(dim: int = 4096, heads: int = 32, context_dim: int = 4096, ff_mult: int = 4, *,
                       gated: bool = False, seed: int = 0, device: str = "cuda") -> VideoBlock:
    """Synthetic parameters of the LTX-2.3 video block's shapes: weights
    ~N(0, 0.02), biases ~N(0, 0.01), norm weights ~1 + N(0, 0.05), tables
    ~N(0, 0.02), input scales sized for unit-variance activations."""
    gen = torch.Generator().manual_seed(seed)

    def randn(*shape, std=1.0):
        return (torch.randn(shape, generator=gen) * std).to(device)

    def lin(n, k, input_scale):
        return FP8Linear.quantized(randn(n, k, std=0.02), input_scale, randn(n, std=0.01).to(torch.bfloat16))

    def attention(kv_dim):
        return VideoAttention(
            to_q=lin(dim, dim, 8.0 / 448), to_k=lin(dim, kv_dim, 8.0 / 448), to_v=lin(dim, kv_dim, 8.0 / 448),
            to_out=lin(dim, dim, 2.0 / 448),
            q_norm_weight=(1 + randn(dim, std=0.05)).to(torch.bfloat16),
            k_norm_weight=(1 + randn(dim, std=0.05)).to(torch.bfloat16),
            heads=heads,
            to_gate_logits=None)

    attn1 = attention(dim)
    if gated:
        gl = torch.nn.Linear(dim, heads, bias=True, device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            gl.weight.copy_(randn(heads, dim, std=0.02))
            gl.bias.copy_(randn(heads, std=0.1))
        attn1.to_gate_logits = gl
    return VideoBlock(
        table=randn(9, dim, std=0.02).to(torch.bfloat16),
        prompt_table=randn(2, context_dim, std=0.02).to(torch.bfloat16),
        attn1=attn1,
        attn2=attention(context_dim),
        ff_up=lin(ff_mult * dim, dim, 8.0 / 448),
        ff_down=lin(dim, ff_mult * dim, 4.0 / 448))


@dataclass
class Stages:
    """Inputs and outputs of each step of a block slice, for per-step checks
    (each tensor as the step saw or produced it)."""
    t: dict = field(default_factory=dict)

    def __setitem__(self, k, v):
        self.t[k] = v

    def __getitem__(self, k):
        return self.t[k]


_MARK = None


class launch_marks:
    """`with launch_marks(fn): ...` calls fn(name) after each op of a block
    slice is enqueued (names as `branch.op`), e.g. to record a HIP event on
    the stream after every launch and time each op of the slice."""

    def __init__(self, fn):
        self.fn = fn

    def __enter__(self):
        global _MARK
        self._prev, _MARK = _MARK, self.fn
        return self

    def __exit__(self, *exc):
        global _MARK
        _MARK = self._prev
        return False


def _mark(name: str) -> None:
    if _MARK is not None:
        _MARK(name)


def _rms_norm(x: torch.Tensor, eps: float, weight: torch.Tensor | None = None) -> torch.Tensor:
    """ltx_core.utils.rms_norm / the attention module's q/k RMSNorm: torch's
    rms_norm over the last dimension."""
    return torch.nn.functional.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)


def video_self_attention(block: VideoBlock, vx: torch.Tensor, timesteps: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, stages: Stages | None = None, *, qkv_grouped: bool = False,
                         fuse_ada_quant: bool = False, next_adazero: dict | None = None,
                         fuse_out_quant: bool = False):
    """:3006-3083 with `_attention_without_out_bias` (:2561-2648). With
    `qkv_grouped` the three projections run as one grouped FP8 GEMM
    (`fp8_qkv_from_grouped_mm`, :890-925; off in the reference's
    production), otherwise as three FP8 linears. With `fuse_ada_quant` as
    well, and no head gates (their logits read the bf16 AdaZero rows), the
    AdaZero pass writes the grouped GEMM's e4m3 input itself. With
    `next_adazero` (the keyword arguments of the AdaZero pass that reads the
    output: shift_index, scale_index, and input_scale for e4m3 codes) the
    residual gate and that pass run as one (`fused_residual_gate_adazero_from_ada`)
    and the call returns (output, that pass's output). With
    `fuse_out_quant` (and no head gates) the attention writes the output
    projection's e4m3 input itself (`attention_video_e4m3_out`)."""
    a = block.attn1
    norm_vx = norm_q8 = qkv = None
    # The grouped projection's guard is checked before the e4m3 AdaZero pass,
    # so a failing guard costs no second AdaZero pass.
    if (fuse_ada_quant and qkv_grouped and a.to_gate_logits is None and vx.is_cuda
            and L._video_qkv_linears_ok(a, vx, ("to_q", "to_k", "to_v"), grouped=True)):
        norm_q8 = L.fused_adazero_from_ada_fp8(vx, block.eps, block.table, timesteps, a.to_q.input_scale,
                                               shift_index=0, scale_index=1)
        _mark("msa.adazero_fp8")
        qkv = L.fp8_qkv_from_quantized_e4m3(a, norm_q8, out_dtype=vx.dtype)
        _mark("msa.qkv_grouped")
    if qkv is None:
        norm_q8 = None
        norm_vx = L.fused_adazero_from_ada(vx, block.eps, block.table, timesteps, shift_index=0, scale_index=1)
        _mark("msa.adazero")
        qkv = L.fp8_qkv_from_grouped_mm(a, norm_vx) if qkv_grouped else None
        if qkv is not None:
            _mark("msa.quant_qkv_grouped")
    if qkv is not None:
        q, k, v = qkv
    else:
        q = L.fp8_linear_forward(a.to_q, norm_vx)
        _mark("msa.quant_q_linear")
        k = L.fp8_linear_forward(a.to_k, norm_vx)
        _mark("msa.quant_k_linear")
        v = L.fp8_linear_forward(a.to_v, norm_vx)
        _mark("msa.quant_v_linear")
    qr, kr = L.fused_video_qk_rmsnorm_rope(q, k, a.q_norm_weight, a.k_norm_weight, block.eps, cos, sin)
    _mark("msa.qk_rmsnorm_rope")
    o = o8 = gates = og = None
    if fuse_out_quant and a.to_gate_logits is None and L._is_fp8_linear(a.to_out):
        # the output projection without its bias (the residual gate adds it)
        o8 = attention_video_e4m3_out(qr, kr, v, a.heads, a.to_out.input_scale)
        _mark("msa.attention_e4m3")
        proj = L.fp8_scaled_mm(o8.reshape(-1, o8.shape[-1]), a.to_out.weight, a.to_out.input_scale,
                               a.to_out.weight_scale, None, out_dtype=vx.dtype).reshape(o8.shape[0], o8.shape[1], -1)
        _mark("msa.out_linear")
    else:
        o = attention_video(qr, kr, v, a.heads)
        _mark("msa.attention")
        if a.to_gate_logits is not None:
            gates = 2.0 * torch.sigmoid(a.to_gate_logits(norm_vx))
            og = L.fused_head_gate_mul_bf16(o, gates, a.heads, o.shape[-1] // a.heads)
            _mark("msa.head_gates")
        else:
            og = o
        proj = L.fp8_linear_without_bias(a.to_out, og, out_dtype=og.dtype)
        if proj is None:
            raise RuntimeError("to_out is not an FP8 linear")
        _mark("msa.quant_out_linear")
    nxt = None
    if next_adazero is not None:
        out, nxt = L.fused_residual_gate_adazero_from_ada(vx, proj, block.table, timesteps, gate_index=2,
                                                          eps=block.eps, bias=a.to_out.bias, **next_adazero)
        _mark("msa.residual_gate_bias_adazero")
    else:
        out = L.fused_residual_gate_bias_from_ada(vx, proj, a.to_out.bias, block.table, timesteps, gate_index=2)
        _mark("msa.residual_gate_bias")
    if stages is not None:
        for name, val in (("msa.x", vx), ("msa.norm", norm_vx), ("msa.norm_q8", norm_q8), ("msa.q", q), ("msa.k", k), ("msa.v", v),
                          ("msa.qr", qr), ("msa.kr", kr), ("msa.attn", o), ("msa.attn_q8", o8), ("msa.gates", gates),
                          ("msa.gated", og), ("msa.proj", proj), ("msa.out", out)):
            stages[name] = val
    return out if next_adazero is None else (out, nxt)


def video_text_cross_attention(block: VideoBlock, vx: torch.Tensor, context: torch.Tensor,
                               timesteps: torch.Tensor, prompt_timestep: torch.Tensor,
                               stages: Stages | None = None, *, fuse_norm: bool = False,
                               fuse_context: bool | None = None, fuse_ada_quant: bool = False,
                               pre_norm: torch.Tensor | None = None, next_adazero: dict | None = None,
                               fuse_out_quant: bool = False):
    """:2810-2888 (cross_attention_adaln, production flags). rms_norm
    followed by the AdaLN affine of Ada rows 6/7 is AdaZero's composition
    (R(R(R(rms_norm(x)) R(1 + scale)) + shift)); with `fuse_norm` it runs as
    one AdaZero pass instead of torch's rms_norm and the affine kernel.
    With `fuse_norm` the K and V projections of the text tokens run as one
    grouped FP8 GEMM when to_k and to_v share their input scale
    (`fp8_kv_from_grouped_mm`). `fuse_context` (default: `fuse_norm`) takes the reference's
    _FUSE_VIDEO_TEXT_CONTEXT_ADALN path (:2839-2850, off in its production):
    the context affine of the prompt table's rows 0/1 as one AdaLN-affine
    launch, the same expression as the torch form beside it. With `fuse_norm`
    the q/k RMSNorms (the module's q_norm/k_norm with no RoPE after them,
    :1866-1867) run as `qk_rmsnorm` launches instead of torch's rms_norm.
    `fuse_ada_quant` (with `fuse_norm`) has that AdaZero pass write the
    q-projection's e4m3 input directly. `pre_norm` is that pass's output
    computed already (by the previous residual gate's fused pass: bf16 rows,
    or e4m3 codes with `fuse_ada_quant`); `next_adazero` and
    `fuse_out_quant` as in `video_self_attention`."""
    a = block.attn2
    b = vx.shape[0]
    if fuse_context is None:
        fuse_context = fuse_norm
    if fuse_context:
        enc = L.fused_adaln_affine_from_ada(context, block.prompt_table, prompt_timestep, shift_index=0,
                                            scale_index=1)
    else:
        shift_kv, scale_kv = (block.prompt_table[None, None].to(device=vx.device, dtype=vx.dtype)
                              + prompt_timestep.reshape(b, prompt_timestep.shape[1], 2, -1)).unbind(dim=2)
        enc = context * (1 + scale_kv) + shift_kv
    _mark("ca.context_affine")
    attn_in_q8 = None
    if pre_norm is not None:
        normed = None
        attn_in, attn_in_q8 = (None, pre_norm) if pre_norm.dtype == torch.float8_e4m3fn else (pre_norm, None)
    elif fuse_norm and fuse_ada_quant:
        normed = attn_in = None
        attn_in_q8 = L.fused_adazero_from_ada_fp8(vx, block.eps, block.table, timesteps, a.to_q.input_scale,
                                                  shift_index=6, scale_index=7)
        _mark("ca.adazero_fp8")
    elif fuse_norm:
        normed = None
        attn_in = L.fused_adazero_from_ada(vx, block.eps, block.table, timesteps, shift_index=6, scale_index=7)
        _mark("ca.adazero")
    else:
        normed = _rms_norm(vx, block.eps)
        _mark("ca.rms_norm")
        attn_in = L.fused_adaln_affine_from_ada(normed, block.table, timesteps, shift_index=6, scale_index=7)
        _mark("ca.adaln_affine")
    qk_norm = L.qk_rmsnorm if fuse_norm else (lambda x, w, eps: _rms_norm(x, eps, w))
    if attn_in_q8 is not None:
        qp = L.fp8_linear_from_quantized_e4m3(a.to_q, attn_in_q8, out_dtype=vx.dtype)
        _mark("ca.q_linear")
    else:
        qp = L.fp8_linear_forward(a.to_q, attn_in)
        _mark("ca.quant_q_linear")
    kv = L.fp8_kv_from_grouped_mm(a, enc) if fuse_norm and enc.is_cuda else None
    if kv is not None:  # K and V of the text tokens as one grouped GEMM
        kp, v = kv
        _mark("ca.quant_kv_grouped")
    else:
        kp = L.fp8_linear_forward(a.to_k, enc)
        _mark("ca.quant_k_linear")
    q = qk_norm(qp, a.q_norm_weight, block.eps)
    _mark("ca.q_rmsnorm")
    k = qk_norm(kp, a.k_norm_weight, block.eps)
    _mark("ca.k_rmsnorm")
    if kv is None:
        v = L.fp8_linear_forward(a.to_v, enc)
        _mark("ca.quant_v_linear")
    o = o8 = None
    if fuse_out_quant and L._is_fp8_linear(a.to_out):
        o8 = attention_video_e4m3_out(q, k, v, a.heads, a.to_out.input_scale)
        _mark("ca.attention_e4m3")
        ca = L.fp8_linear_from_quantized_e4m3(a.to_out, o8, out_dtype=vx.dtype)
        _mark("ca.out_linear")
    else:
        o = attention_video(q, k, v, a.heads)
        _mark("ca.attention")
        ca = L.fp8_linear_forward(a.to_out, o)
        _mark("ca.quant_out_linear")
    nxt = None
    if next_adazero is not None:
        out, nxt = L.fused_residual_gate_adazero_from_ada(vx, ca, block.table, timesteps, gate_index=8,
                                                          eps=block.eps, count_video_ada=False, **next_adazero)
        _mark("ca.residual_gate_adazero")
    else:
        out = L.fused_residual_gate_from_ada(vx, ca, block.table, timesteps, gate_index=8, count_video_ada=False)
        _mark("ca.residual_gate")
    if stages is not None:
        for name, val in (("ca.x", vx), ("ca.enc", enc), ("ca.normed", normed), ("ca.in", attn_in),
                          ("ca.in_q8", attn_in_q8), ("ca.qp", qp),
                          ("ca.kp", kp), ("ca.q", q), ("ca.k", k), ("ca.v", v), ("ca.attn", o), ("ca.attn_q8", o8),
                          ("ca.proj", ca),
                          ("ca.out", out)):
            stages[name] = val
    return out if next_adazero is None else (out, nxt)


def video_feed_forward(block: VideoBlock, vx: torch.Tensor, timesteps: torch.Tensor, *,
                       fuse_gelu_quant: bool = False, fuse_ada_quant: bool = False,
                       stages: Stages | None = None, pre_norm: torch.Tensor | None = None) -> torch.Tensor:
    """:3224-3258. With `fuse_gelu_quant` the GELU-tanh runs inside the
    down-projection's input quantizer (`fused_gelu_tanh_fp8_quantize_e4m3`,
    :164-182, off in the reference's production); otherwise torch's GELU
    (tanh) in bf16, then the down-projection's own quantizer. With
    `fuse_ada_quant` the AdaZero pass writes the up-projection's e4m3 input.
    `pre_norm`: that pass's output computed already (bf16 rows or e4m3
    codes), as in `video_text_cross_attention`."""
    if pre_norm is not None and pre_norm.dtype == torch.float8_e4m3fn:
        y, yq = None, pre_norm
        h = L.fp8_linear_from_quantized_e4m3(block.ff_up, yq, out_dtype=vx.dtype)
        _mark("ff.up_linear")
    elif pre_norm is not None:
        y, yq = pre_norm, None
        h = L.fp8_linear_forward(block.ff_up, y)
        _mark("ff.quant_up_linear")
    elif fuse_ada_quant:
        y = None
        yq = L.fused_adazero_from_ada_fp8(vx, block.eps, block.table, timesteps, block.ff_up.input_scale,
                                          shift_index=3, scale_index=4)
        _mark("ff.adazero_fp8")
        h = L.fp8_linear_from_quantized_e4m3(block.ff_up, yq, out_dtype=vx.dtype)
        _mark("ff.up_linear")
    else:
        yq = None
        y = L.fused_adazero_from_ada(vx, block.eps, block.table, timesteps, shift_index=3, scale_index=4)
        _mark("ff.adazero")
        h = L.fp8_linear_forward(block.ff_up, y)
        _mark("ff.quant_up_linear")
    if fuse_gelu_quant:
        g = None
        qg = L.fused_gelu_tanh_fp8_quantize_e4m3(h, block.ff_down.input_scale)
        _mark("ff.gelu_quant")
        d = L.fp8_linear_from_quantized_e4m3(block.ff_down, qg, out_dtype=h.dtype)
        _mark("ff.down_linear")
    else:
        g = torch.nn.functional.gelu(h, approximate="tanh")
        _mark("ff.gelu")
        d = L.fp8_linear_forward(block.ff_down, g)
        _mark("ff.quant_down_linear")
    out = L.fused_residual_gate_from_ada(vx, d, block.table, timesteps, gate_index=5)
    _mark("ff.residual_gate")
    if stages is not None:
        for name, val in (("ff.x", vx), ("ff.norm", y), ("ff.norm_q8", yq), ("ff.h", h), ("ff.gelu", g), ("ff.down", d),
                          ("ff.out", out)):
            stages[name] = val
    return out


def video_block_forward(block: VideoBlock, vx: torch.Tensor, context: torch.Tensor, timesteps: torch.Tensor,
                        prompt_timestep: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *,
                        fuse_gelu_quant: bool = False, qkv_grouped: bool = False, fuse_norm: bool = False,
                        fuse_ada_quant: bool = False, fuse_residual_ada: bool = False,
                        fuse_out_quant: bool = False, stages: Stages | None = None) -> torch.Tensor:
    """The video branches of one block: self-attention, text cross-attention,
    feed-forward (:2989-3298 without the audio and audio-video branches).
    vx (B, N, C) bf16; context (B, T, C) bf16; timesteps (B, N, 9C) or a
    stride-0 token axis; prompt_timestep (B, T, 2C); cos/sin [B or 1, H, N, 64].
    `fuse_ada_quant` has each AdaZero pass that feeds an FP8 linear write that
    linear's e4m3 input instead of bf16 rows (`fused_adazero_from_ada_fp8`).
    `fuse_residual_ada` runs each branch's residual gate together with the
    next branch's AdaZero pass (`fused_residual_gate_adazero_from_ada`): the
    self-attention's with the cross-attention's (which is an AdaZero pass
    only with `fuse_norm`), the cross-attention's with the feed-forward's.
    `fuse_out_quant` has each attention write its output projection's e4m3
    input (`attention_video_e4m3_out`; the self-attention's only without
    head gates)."""
    ca_next = ff_next = None
    if fuse_residual_ada:
        if fuse_norm:
            ca_next = {"shift_index": 6, "scale_index": 7}
            if fuse_ada_quant:
                ca_next["input_scale"] = block.attn2.to_q.input_scale
        ff_next = {"shift_index": 3, "scale_index": 4}
        if fuse_ada_quant:
            ff_next["input_scale"] = block.ff_up.input_scale
    r = video_self_attention(block, vx, timesteps, cos, sin, stages, qkv_grouped=qkv_grouped,
                             fuse_ada_quant=fuse_ada_quant, next_adazero=ca_next, fuse_out_quant=fuse_out_quant)
    vx, pre_ca = r if ca_next is not None else (r, None)
    r = video_text_cross_attention(block, vx, context, timesteps, prompt_timestep, stages, fuse_norm=fuse_norm,
                                   fuse_ada_quant=fuse_ada_quant, pre_norm=pre_ca, next_adazero=ff_next,
                                   fuse_out_quant=fuse_out_quant)
    vx, pre_ff = r if ff_next is not None else (r, None)
    return video_feed_forward(block, vx, timesteps, fuse_gelu_quant=fuse_gelu_quant, fuse_ada_quant=fuse_ada_quant,
                              stages=stages, pre_norm=pre_ff)
