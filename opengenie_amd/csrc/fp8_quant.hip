// bf16 -> float8_e4m3fn activation quantizers.
//
// Reference: ltx_serve/triton_ltx_ops.py :144-161 (per tensor; torch path
// :146-148), :164-182 (GELU-tanh then quantize; torch :165-169), :265-317
// (per batch*head; torch :976-980).
//
// Per-tensor: q = e4m3(clamp(x * r, +-448)), r = 1/scale (IEEE division).
// torch's dtype rule decides the rounding of x * r: with a 0-dim scale the
// common dtype is bf16, so the float32 operand r is first converted to bf16
// and the product is rounded to bf16; with a (1,) scale the product stays
// float32. Every thread converts 16 elements: two 128-bit loads, one 128-bit
// store. The e4m3 rounding is the hardware v_cvt_pk_fp8_f32 (nearest even),
// applied after the clamp so saturation never engages.
#include "common.h"
#include "host.h"

namespace oga {

template <bool GELU>
OGA_DEVICE float pre(float x) {
  if (!GELU) return x;
  // torch gelu(approximate='tanh') in float32, rounded to the bf16 result.
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  const float inner = k0 * (x + k1 * x * x * x);
  return rbf(0.5f * x * (1.0f + tanhf(inner)));
}

template <bool GELU>
__global__ __launch_bounds__(256) void k_fp8_quant(const uint16_t* x, const float* scale, int zero_dim, uint8_t* q,
                                                   int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  float r = 1.0f / scale[0];
  if (zero_dim) r = rbf(r);
  if (i0 + 16 <= n) {
    const uint4 u0 = *(const uint4*)(x + i0);
    const uint4 u1 = *(const uint4*)(x + i0 + 8);
    float f[16];
    unpack8(u0, f);
    unpack8(u1, f + 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = pre<GELU>(f[i]) * r;
      if (zero_dim) v = rbf(v);
      f[i] = clamp448(v);
    }
    uint4 o;
    o.x = e4m3x4(f[0], f[1], f[2], f[3]);
    o.y = e4m3x4(f[4], f[5], f[6], f[7]);
    o.z = e4m3x4(f[8], f[9], f[10], f[11]);
    o.w = e4m3x4(f[12], f[13], f[14], f[15]);
    st_nt16(q + i0, o);
  } else {
    for (int64_t i = i0; i < n; ++i) {
      float v = pre<GELU>(__uint_as_float(((uint32_t)x[i]) << 16)) * r;
      if (zero_dim) v = rbf(v);
      v = clamp448(v);
      q[i] = (uint8_t)(e4m3x4(v, 0.0f, 0.0f, 0.0f) & 0xFF);
    }
  }
}

// ------------------------------------------------------------ per head
// Pass 1: partial amax over a block of tokens, for every head. Block
// (b, chunk) covers tokens [chunk*TPB, chunk*TPB + TPB); each wave walks
// TPB/4 token rows; lane l of vector step j sees head (j*512 + 8l) / D.
// partial[b, chunk, h] = max |x| over the block.
template <int CH, int D>
__global__ __launch_bounds__(256) void k_head_amax(const uint16_t* x, float* partial, int64_t tokens, int tpb,
                                                   int nchunk) {
  constexpr int H = CH * 512 / D;
  constexpr int LPH = D / 8;  // lanes per head inside one vector step
  __shared__ float red[4][H];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  float m[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) m[j] = 0.0f;
  const int64_t t0 = (int64_t)chunk * tpb;
  const int64_t t1 = min(t0 + tpb, tokens);
  for (int64_t t = t0 + w; t < t1; t += 4) {
    const uint16_t* row = x + (b * tokens + t) * (int64_t)(CH * 512);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      float f[8];
      unpack8(*(const uint4*)(row + j * 512 + lane * 8), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m[j] = fmaxf(m[j], fabsf(f[i]));
    }
  }
  // Reduce over the lanes of one head: 16 lanes (D=128) or 8 lanes (D=64).
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    float v = m[j];
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
    if (LPH == 16) v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));
    if (lane % LPH == 0) red[w][(j * 512 + lane * 8) / D] = v;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += 256) {
    const float v = fmaxf(fmaxf(red[0][h], red[1][h]), fmaxf(red[2][h], red[3][h]));
    partial[(b * nchunk + chunk) * H + h] = v;
  }
}

// Pass 2: scale[b, h] = max(amax, 1e-12) / 448 (IEEE division). One wave
// per (b, h): lanes stride over the block partials, then a wave-wide max.
__global__ __launch_bounds__(64) void k_head_scale(const float* partial, float* scale, int heads, int nchunk) {
  const int64_t bh = blockIdx.x;
  const int64_t b = bh / heads;
  const int h = (int)(bh - b * heads);
  const int lane = threadIdx.x;
  float m = 0.0f;
  for (int c = lane; c < nchunk; c += 64) m = fmaxf(m, partial[(b * nchunk + c) * heads + h]);
  m = row16_max(m);
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(m), 0x401F)));
  m = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)));
  if (lane == 0) scale[bh] = fmaxf(m, 1e-12f) / 448.0f;
}

// Pass 3: q = e4m3(clamp(x / scale[b, h], +-448)), 16 elements per thread
// (16 consecutive elements never straddle a head for D in {64, 128}).
__global__ __launch_bounds__(256) void k_head_quant(const uint16_t* x, const float* scale, uint8_t* q, int64_t n,
                                                    int64_t tokens, int heads, int d) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  const int64_t row = (int64_t)heads * d;
  const int64_t tok = i0 / row;
  const int64_t h = (i0 - tok * row) / d;
  const int64_t b = tok / tokens;
  const float s = scale[b * heads + h];
  const uint4 u0 = *(const uint4*)(x + i0);
  const uint4 u1 = *(const uint4*)(x + i0 + 8);
  float f[16];
  unpack8(u0, f);
  unpack8(u1, f + 8);
#pragma unroll
  for (int i = 0; i < 16; ++i) f[i] = clamp448(f[i] / s);
  uint4 o;
  o.x = e4m3x4(f[0], f[1], f[2], f[3]);
  o.y = e4m3x4(f[4], f[5], f[6], f[7]);
  o.z = e4m3x4(f[8], f[9], f[10], f[11]);
  o.w = e4m3x4(f[12], f[13], f[14], f[15]);
  st_nt16(q + i0, o);
}

// ------------------------------------------------------------ self-test
__global__ __launch_bounds__(256) void k_selftest_convert(const float* in, uint16_t* b, uint8_t* e, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = in[i];
  b[i] = (uint16_t)(__float_as_uint(rbf(v)) >> 16);
  e[i] = (uint8_t)(e4m3x4(clamp448(v), 0.0f, 0.0f, 0.0f) & 0xFF);
}

constexpr int kHeadTokensPerBlock = 16;

static int64_t head_chunks(int64_t tokens) { return (tokens + kHeadTokensPerBlock - 1) / kHeadTokensPerBlock; }

template <int CH, int D>
static void launch_head_amax(const uint16_t* x, float* partial, int64_t batch, int64_t tokens, hipStream_t st) {
  const int nchunk = (int)head_chunks(tokens);
  hipLaunchKernelGGL((k_head_amax<CH, D>), dim3((unsigned)nchunk, (unsigned)batch), dim3(256), 0, st, x, partial,
                     tokens, kHeadTokensPerBlock, nchunk);
}

}  // namespace oga

using namespace oga;

extern "C" int oga_fp8_quantize_e4m3(const void* x, const float* scale, int scale_is_0dim, void* q, int64_t n,
                                     void* stream) {
  if (!x || !scale || !q) return fail("null pointer");
  if (n < 0) return fail("bad size");
  if (n == 0) return OGA_OK;
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  const int64_t threads = (n + 15) / 16;
  hipLaunchKernelGGL(k_fp8_quant<false>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n);
  return launch_status();
}

extern "C" int oga_gelu_tanh_fp8_quantize_e4m3(const void* x, const float* scale, int scale_is_0dim, void* q,
                                               int64_t n, void* stream) {
  if (!x || !scale || !q) return fail("null pointer");
  if (n < 0) return fail("bad size");
  if (n == 0) return OGA_OK;
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  const int64_t threads = (n + 15) / 16;
  hipLaunchKernelGGL(k_fp8_quant<true>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n);
  return launch_status();
}

extern "C" int64_t oga_fp8_per_head_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim) {
  (void)head_dim;
  if (batch < 0 || tokens < 0 || heads < 0) return 0;
  return batch * head_chunks(tokens) * heads * (int64_t)sizeof(float);
}

extern "C" int oga_fp8_quantize_per_head(const void* x, void* q, float* scale_out, void* workspace, int64_t batch,
                                         int64_t tokens, int64_t heads, int64_t head_dim, void* stream) {
  if (!x || !q || !scale_out || !workspace) return fail("null pointer");
  if (batch < 1 || tokens < 1 || heads < 1) return fail("empty shape");
  if (batch > 65535) return unsupported("batch > 65535");
  if (head_dim != 64 && head_dim != 128) return unsupported("head_dim must be 64 or 128");
  const int64_t row = heads * head_dim;
  if (row != 1024 && row != 2048 && row != 4096) return unsupported("heads*head_dim must be 1024, 2048 or 4096");
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xs = (const uint16_t*)x;
  float* partial = (float*)workspace;
  const int ch = (int)(row / 512);
  if (head_dim == 128) {
    if (ch == 8) launch_head_amax<8, 128>(xs, partial, batch, tokens, st);
    else if (ch == 4) launch_head_amax<4, 128>(xs, partial, batch, tokens, st);
    else launch_head_amax<2, 128>(xs, partial, batch, tokens, st);
  } else {
    if (ch == 8) launch_head_amax<8, 64>(xs, partial, batch, tokens, st);
    else if (ch == 4) launch_head_amax<4, 64>(xs, partial, batch, tokens, st);
    else launch_head_amax<2, 64>(xs, partial, batch, tokens, st);
  }
  int rc = launch_status();
  if (rc) return rc;
  const int64_t bh = batch * heads;
  hipLaunchKernelGGL(k_head_scale, dim3((unsigned)bh), dim3(64), 0, st, partial, scale_out, (int)heads,
                     (int)head_chunks(tokens));
  if ((rc = launch_status())) return rc;
  const int64_t n = batch * tokens * row;
  const int64_t threads = n / 16;
  hipLaunchKernelGGL(k_head_quant, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, xs, scale_out,
                     (uint8_t*)q, n, tokens, (int)heads, (int)head_dim);
  return launch_status();
}

extern "C" int oga_selftest_convert(const float* in, uint16_t* bf16_out, uint8_t* e4m3_out, int64_t n, void* stream) {
  if (!in || !bf16_out || !e4m3_out) return fail("null pointer");
  if (n <= 0) return OGA_OK;
  hipLaunchKernelGGL(k_selftest_convert, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, in,
                     bf16_out, e4m3_out, n);
  return launch_status();
}
