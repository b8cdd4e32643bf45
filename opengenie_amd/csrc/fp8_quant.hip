// bf16 / fp16 -> float8_e4m3fn activation quantizers.
//
// Reference: ltx_serve/triton_ltx_ops.py :144-161 (per tensor; torch path
// :146-148), :164-182 (GELU-tanh then quantize; torch :165-169), :265-317
// (per batch*head; torch :976-980).
//
// Per-tensor: q = e4m3(clamp(x * r, +-448)), r = 1/scale (IEEE division).
// torch's dtype rule decides the rounding of x * r: with a 0-dim scale the
// common dtype is x's (bf16 or fp16), so the float32 operand r is first
// converted to x's dtype and the product is rounded to it; with a (1,) scale
// the product stays float32. Every kernel takes x's dtype as the template
// parameter XDT (OGA_DT_BF16 or OGA_DT_F16). Every thread converts 16 elements: two 128-bit loads, one 128-bit
// store. The e4m3 rounding is the hardware v_cvt_pk_fp8_f32 (nearest even),
// applied after the clamp so saturation never engages.
#include <atomic>
#include <mutex>

#include "common.h"
#include "host.h"

namespace oga {

// GELU-tanh as torch's GPU kernel for gelu(approximate='tanh') evaluates it
// in float32 for a bf16 input (ATen GeluCUDAKernelImpl):
//   inner = kBeta * (x + kKappa * x^3),  x^3 = (x * x) * x,
//   g     = (0.5 * x) * (1 + tanh(inner)),  rounded once to bf16,
// kBeta = float(sqrt(2) * 2/sqrt(pi) * 0.5), kKappa = float(0.044715), tanh
// the ROCm device library's tanhf. torch is compiled with the HIP default
// -ffp-contract=fast, so x + kKappa * x^3 is one fused multiply-add; every
// other step is a separate float32 operation. The result is the same bf16
// value torch produces for every one of the 65536 bf16 inputs.
constexpr int kGeluNone = 0, kGeluExact = 1;
constexpr float kGeluBeta = (float)(M_SQRT2 * M_2_SQRTPI * 0.5);
constexpr float kGeluKappa = 0.044715f;
template <int GELU, int XDT>
OGA_DEVICE float pre(float x) {
  if (GELU == kGeluNone) return x;
  const float x3 = (x * x) * x;
  const float inner = kGeluBeta * fmaf(kGeluKappa, x3, x);
  return rx16<XDT>((0.5f * x) * (1.0f + tanhf(inner)));
}

template <int GELU, int XDT>
__global__ __launch_bounds__(256) void k_fp8_quant(const uint16_t* x, const float* scale, int zero_dim, uint8_t* q,
                                                   int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  float r = 1.0f / scale[0];
  if (zero_dim) r = rx16<XDT>(r);
  if (i0 + 16 <= n) {
    const uint4 u0 = *(const uint4*)(x + i0);
    const uint4 u1 = *(const uint4*)(x + i0 + 8);
    float f[16];
    unpack8x<XDT>(u0, f);
    unpack8x<XDT>(u1, f + 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = pre<GELU, XDT>(f[i]) * r;
      if (zero_dim) v = rx16<XDT>(v);
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
      float v = pre<GELU, XDT>(x16_bits<XDT>(x[i])) * r;
      if (zero_dim) v = rx16<XDT>(v);
      v = clamp448(v);
      q[i] = (uint8_t)(e4m3x4(v, 0.0f, 0.0f, 0.0f) & 0xFF);
    }
  }
}

// ------------------------------------------------------------ GELU table
// The GELU quantizer reads gelu(x) rounded to x's dtype from a table: a
// 16-bit input has 65536 patterns, so k_gelu_table evaluates the formula of
// pre<kGeluExact, XDT> once per pattern (128 KiB of results) and the
// streaming kernel looks each element up in an LDS copy of it, which makes
// the pass HBM-bound instead of bound by tanhf's VALU work. The tables (one
// per dtype) live in file-scope device arrays per GPU, built by the first
// call on a GPU and only read after that (oga_gelu_tanh_fp8_quantize_e4m3).
static __device__ __align__(256) uint16_t gelu_table_bf16[65536];
static __device__ __align__(256) uint16_t gelu_table_f16[65536];
template <int XDT>
__global__ __launch_bounds__(256) void k_gelu_table(uint16_t* table) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;  // grid: 256 x 256
  const float g = pre<kGeluExact, XDT>(x16_bits<XDT>(i));
  table[i] = XDT == OGA_DT_F16 ? __builtin_bit_cast(uint16_t, (_Float16)g) : (uint16_t)(__float_as_uint(g) >> 16);
}

// q = e4m3(clamp(table[x] * r)) with the rounding rule of k_fp8_quant. One
// 1024-lane workgroup per CU (the table takes 128 KiB of LDS) walks the
// tensor in steps of gridDim.x * 1024 lanes * 32 elements; per step a lane
// converts two 16-element groups with all four 16-byte loads in flight.
constexpr int kGeluLanes = 1024;
template <int XDT>
__global__ __launch_bounds__(kGeluLanes) void k_gelu_quant(const uint16_t* x, const float* scale, int zero_dim,
                                                           uint8_t* q, int64_t n, const uint16_t* table) {
  __shared__ uint4 tab[65536 * 2 / 16];
  for (int k = threadIdx.x; k < 65536 * 2 / 16; k += kGeluLanes) tab[k] = ((const uint4*)table)[k];
  __syncthreads();
  const uint16_t* const t16 = (const uint16_t*)tab;
  float r = 1.0f / scale[0];
  if (zero_dim) r = rx16<XDT>(r);
  auto code = [&](uint32_t xb) {  // one element, x as its 16 bits
    float v = x16_bits<XDT>(t16[xb]) * r;
    if (zero_dim) v = rx16<XDT>(v);
    return clamp448(v);
  };
  auto conv16 = [&](const uint4& u0, const uint4& u1, int64_t i0) {
    const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    float f[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      f[2 * k] = code(w[k] & 0xFFFFu);
      f[2 * k + 1] = code(w[k] >> 16);
    }
    uint4 o;
    o.x = e4m3x4(f[0], f[1], f[2], f[3]);
    o.y = e4m3x4(f[4], f[5], f[6], f[7]);
    o.z = e4m3x4(f[8], f[9], f[10], f[11]);
    o.w = e4m3x4(f[12], f[13], f[14], f[15]);
    st_nt16(q + i0, o);
  };
  // A group of 16 elements at g < n, whole or the tensor's ragged end.
  auto group = [&](int64_t g) {
    if (g + 16 <= n) {
      conv16(*(const uint4*)(x + g), *(const uint4*)(x + g + 8), g);
    } else {
      for (int64_t i = g; i < n; ++i) q[i] = (uint8_t)(e4m3x4(code(x[i]), 0.0f, 0.0f, 0.0f) & 0xFF);
    }
  };
  const int64_t step = (int64_t)gridDim.x * kGeluLanes * 32;
  // Workgroup b's lanes cover elements 32768 b .. +32767 of every step: the
  // first group of lane t at 16 t, the second 16384 further on.
  for (int64_t base = ((int64_t)blockIdx.x * 2 * kGeluLanes + threadIdx.x) * 16; base < n; base += step) {
    const int64_t i1 = base + (int64_t)kGeluLanes * 16;
    if (i1 + 16 <= n) {
      const uint4 a0 = *(const uint4*)(x + base), a1 = *(const uint4*)(x + base + 8);
      const uint4 b0 = *(const uint4*)(x + i1), b1 = *(const uint4*)(x + i1 + 8);
      conv16(a0, a1, base);
      conv16(b0, b1, i1);
    } else {
      group(base);
      if (i1 < n) group(i1);
    }
  }
}

// ------------------------------------------------------------ per head
// The amax of |x| is taken on bit patterns: with the sign bit cleared, a
// bf16, fp16 (or float32) pattern orders as its magnitude, and every NaN
// pattern lies above infinity, so the maximum is NaN when any element is
// NaN, as torch's amax gives. Two 16-bit magnitudes are kept per dword and
// combined with one packed 16-bit max; the float32 conversion of the
// largest keeps the order.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
OGA_DEVICE u16x2 abs_bits2(uint32_t w) { return __builtin_bit_cast(u16x2, w & 0x7FFF7FFFu); }
OGA_DEVICE uint32_t umax_dpp(uint32_t v, int ctrl) {
  uint32_t o;
  switch (ctrl) {
    case 0: o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true); break;   // lane ^ 1
    case 1: o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true); break;   // lane ^ 2
    case 2: o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true); break;  // half-row mirror
    default: o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true); break; // row mirror
  }
  return max(v, o);
}

// Pass 1: partial amax over a block of tokens, for every head. Block
// (b, chunk) covers tokens [chunk*TPB, chunk*TPB + TPB); each wave walks
// TPB/4 token rows; lane l of vector step j sees head (j*512 + 8l) / D.
// partial[b, h, chunk] = max |x| over the block as a float32 bit pattern
// (a head's partials are contiguous for the reduction in pass 2).
template <int CH, int D, int TPB, int XDT>
__global__ __launch_bounds__(256) void k_head_amax(const uint16_t* x, float* partial, int64_t tokens, int nchunk) {
  constexpr int H = CH * 512 / D;
  constexpr int LPH = D / 8;  // lanes per head inside one vector step
  __shared__ uint32_t red[4][H];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  u16x2 m[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) m[j] = u16x2{0, 0};
  // The wave's TPB/4 token rows (CH 16-byte loads each) are all in flight
  // together before the maxima are taken.
  const int64_t t0 = (int64_t)chunk * TPB;
  constexpr int NR = TPB / 4;
  uint4 xv[NR][CH];
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int64_t t = t0 + w + 4 * u;
    if (t < tokens) {
      const uint16_t* row = x + (b * tokens + t) * (int64_t)(CH * 512);
#pragma unroll
      for (int j = 0; j < CH; ++j) xv[u][j] = *(const uint4*)(row + j * 512 + lane * 8);
    }
  }
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    if (t0 + w + 4 * u < tokens) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const uint4 v = xv[u][j];
        m[j] = __builtin_elementwise_max(m[j], abs_bits2(v.x));
        m[j] = __builtin_elementwise_max(m[j], abs_bits2(v.y));
        m[j] = __builtin_elementwise_max(m[j], abs_bits2(v.z));
        m[j] = __builtin_elementwise_max(m[j], abs_bits2(v.w));
      }
    }
  }
  // Reduce over the lanes of one head: 16 lanes (D=128) or 8 lanes (D=64).
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    // float32 pattern of the largest magnitude
    uint32_t v = __float_as_uint(x16_bits<XDT>(max((uint32_t)m[j].x, (uint32_t)m[j].y)));
    v = umax_dpp(v, 0);
    v = umax_dpp(v, 1);
    v = umax_dpp(v, 2);
    if (LPH == 16) v = umax_dpp(v, 3);
    if (lane % LPH == 0) red[w][(j * 512 + lane * 8) / D] = v;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += 256) {
    const uint32_t v = max(max(red[0][h], red[1][h]), max(red[2][h], red[3][h]));
    partial[(b * H + h) * nchunk + chunk] = __uint_as_float(v);
  }
}

// Pass 2: quantize. Workgroup (token chunk, h, b) first reduces the amax
// partials of head (b, h) to scale = max(amax, 1e-12) * float32(1/448)
// (workgroup 0 of the head stores it), then quantizes its chunk of tokens:
// q = e4m3(clamp(x / scale, +-448)). D/8 lanes cover one token's head slice
// (16 bytes each), so every load is a whole 2*D-byte slice and every store
// a whole D-byte slice.
constexpr int kQuantTokens = 64;
template <int D, int XDT>
__global__ __launch_bounds__(256) void k_head_scale_quant(const uint16_t* x, const float* partial, float* scale_out,
                                                          uint8_t* q, int64_t tokens, int heads, int nchunk) {
  constexpr int LPT = D / 8;      // lanes per token slice
  constexpr int TPP = 256 / LPT;  // token slices per pass
  __shared__ uint32_t red[4];
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // The chunk's x slices are loaded first, so that they are in flight with
  // the partials below (a slice past the last token re-reads the last one
  // and is not stored: no branch around a load).
  constexpr int NI = kQuantTokens / TPP;
  const int sub = threadIdx.x % LPT, tk = threadIdx.x / LPT;
  const int64_t t0 = (int64_t)blockIdx.x * kQuantTokens;
  const int64_t t1 = min(t0 + kQuantTokens, tokens);
  uint4 xv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t t = min(t0 + tk + i * TPP, t1 - 1);
    xv[i] = *(const uint4*)(x + ((b * tokens + t) * heads + h) * D + sub * 8);
  }
  // Partials are magnitudes as float32 bit patterns: their integer maximum
  // is the amax, NaN if any element of the head was NaN.
  // Four loads per thread and pass, all in flight with the x slices (an
  // index past the last partial re-reads it, which leaves the maximum).
  uint32_t m = 0;
  const float* const ph = partial + (b * heads + h) * nchunk;
  for (int c0 = threadIdx.x; c0 < nchunk; c0 += 1024) {
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __float_as_uint(ph[min(c0 + 256 * k, nchunk - 1)]);
    m = max(m, max(max(v[0], v[1]), max(v[2], v[3])));
  }
  m = umax_dpp(umax_dpp(umax_dpp(umax_dpp(m, 0), 1), 2), 3);
  m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, 0x401F));
  m = max((uint32_t)__builtin_amdgcn_readlane((int)m, 0), (uint32_t)__builtin_amdgcn_readlane((int)m, 32));
  if (lane == 0) red[w] = m;
  __syncthreads();
  // torch: clamp_min(amax, 1e-12) / 448, with a NaN amax kept (clamp
  // propagates NaN) so the whole head quantizes to NaN codes. torch's GPU
  // division of a tensor by a Python scalar multiplies by the float32
  // reciprocal of the scalar, so that is what this computes.
  const float amax = __uint_as_float(max(max(red[0], red[1]), max(red[2], red[3])));
  const float s = (amax != amax ? amax : fmaxf(amax, 1e-12f)) * (1.0f / 448.0f);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[b * heads + h] = s;

  // x / s as the compiler's IEEE float32 division computes it (v_div_scale,
  // v_rcp, three Newton/FMA corrections, v_div_fmas, v_div_fixup), with the
  // divisor-only part (the refined reciprocal r) hoisted out of the loop.
  // v_div_scale leaves both operands unscaled and v_div_fmas is a plain FMA
  // unless the denominator is denormal or above 2^126, the quotient is
  // above 2^96, or the numerator or quotient is tiny (exponent below -103,
  // or a denormal quotient). Here 2.2e-15 <= s <= 7.6e35 and |x / s| <= 448,
  // so only tiny quotients are left out, and those, like the fast path's,
  // round to a zero e4m3 code whose sign v_div_fixup sets; v_div_fixup also
  // returns the hardware's result for zero, infinite and NaN numerators.
  const float r0 = __builtin_amdgcn_rcpf(s);
  const float r = fmaf(fmaf(-s, r0, 1.0f), r0, r0);
  auto div = [&](float n) {
    float qv = n * r;
    qv = fmaf(fmaf(-s, qv, n), r, qv);
    qv = fmaf(fmaf(-s, qv, n), r, qv);
    return __builtin_amdgcn_div_fixupf(qv, s, n);
  };
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t t = t0 + tk + i * TPP;
    if (t < t1) {
      const int64_t e0 = ((b * tokens + t) * heads + h) * D + sub * 8;
      float f[8];
      unpack8x<XDT>(xv[i], f);
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] = clamp448(div(f[k]));
      typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 o = {e4m3x4(f[0], f[1], f[2], f[3]), e4m3x4(f[4], f[5], f[6], f[7])};
      __builtin_nontemporal_store(o, (u32x2*)(q + e0));
    }
  }
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

template <int CH, int D, int XDT>
static void launch_head_amax(const uint16_t* x, float* partial, int64_t batch, int64_t tokens, hipStream_t st) {
  const int nchunk = (int)head_chunks(tokens);
  hipLaunchKernelGGL((k_head_amax<CH, D, kHeadTokensPerBlock, XDT>), dim3((unsigned)nchunk, (unsigned)batch),
                     dim3(256), 0, st, x, partial, tokens, nchunk);
}

template <int XDT>
static void launch_per_head(const uint16_t* xs, uint8_t* q, float* scale_out, float* partial, int64_t batch,
                            int64_t tokens, int64_t heads, int64_t head_dim, hipStream_t st) {
  const int ch = (int)(heads * head_dim / 512);
  if (head_dim == 128) {
    if (ch == 8) launch_head_amax<8, 128, XDT>(xs, partial, batch, tokens, st);
    else if (ch == 4) launch_head_amax<4, 128, XDT>(xs, partial, batch, tokens, st);
    else launch_head_amax<2, 128, XDT>(xs, partial, batch, tokens, st);
  } else {
    if (ch == 8) launch_head_amax<8, 64, XDT>(xs, partial, batch, tokens, st);
    else if (ch == 4) launch_head_amax<4, 64, XDT>(xs, partial, batch, tokens, st);
    else launch_head_amax<2, 64, XDT>(xs, partial, batch, tokens, st);
  }
  const dim3 qgrid((unsigned)((tokens + kQuantTokens - 1) / kQuantTokens), (unsigned)heads, (unsigned)batch);
  if (head_dim == 128)
    hipLaunchKernelGGL((k_head_scale_quant<128, XDT>), qgrid, dim3(256), 0, st, xs, partial, scale_out, q, tokens,
                       (int)heads, (int)head_chunks(tokens));
  else
    hipLaunchKernelGGL((k_head_scale_quant<64, XDT>), qgrid, dim3(256), 0, st, xs, partial, scale_out, q, tokens,
                       (int)heads, (int)head_chunks(tokens));
}

static bool x16_dt_ok(int dt) { return dt == OGA_DT_BF16 || dt == OGA_DT_F16; }

}  // namespace oga

using namespace oga;

extern "C" int oga_fp8_quantize_e4m3(const void* x, int x_dtype, const float* scale, int scale_is_0dim, void* q,
                                     int64_t n, void* stream) {
  if (!x || !scale || !q) return fail("null pointer");
  if (!x16_dt_ok(x_dtype)) return unsupported("x dtype must be bf16 or fp16");
  if (n < 0) return fail("bad size");
  if (n == 0) return OGA_OK;
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  const int64_t threads = (n + 15) / 16;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (x_dtype == OGA_DT_F16)
    hipLaunchKernelGGL((k_fp8_quant<kGeluNone, OGA_DT_F16>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n);
  else
    hipLaunchKernelGGL((k_fp8_quant<kGeluNone, OGA_DT_BF16>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n);
  return launch_status();
}

// The GELU tables of a GPU: built once, by the first call on that GPU, on
// the caller's stream. Until the build is known to have completed, a call
// on any stream waits for it through an event recorded behind it (no host
// synchronisation); from then on calls only read the table. A call made
// while its stream is being captured into a graph, before the table is
// complete, puts the build into the graph instead (the graph then builds
// the table, with the same values, each time it runs).
namespace {
constexpr int kMaxGeluDevices = 64;
enum { kTableNone = 0, kTablePending = 1, kTableReady = 2 };
struct GeluTable {
  std::mutex mu;
  std::atomic<int> state{kTableNone};
  void* ptr = nullptr;
  hipEvent_t built = nullptr;
};
GeluTable g_gelu[2][kMaxGeluDevices];  // [bf16, fp16][device]
}  // namespace

static int gelu_table(int x_dtype, hipStream_t st, uint16_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxGeluDevices) return unsupported("device ordinal %d beyond %d", dev, kMaxGeluDevices);
  GeluTable& t = g_gelu[x_dtype == OGA_DT_F16 ? 1 : 0][dev];
  if (t.state.load(std::memory_order_acquire) == kTableReady) {
    *out = (uint16_t*)t.ptr;
    return OGA_OK;
  }
  std::lock_guard<std::mutex> lock(t.mu);
  if (!t.ptr) {
    e = x_dtype == OGA_DT_F16 ? hipGetSymbolAddress(&t.ptr, HIP_SYMBOL(gelu_table_f16))
                              : hipGetSymbolAddress(&t.ptr, HIP_SYMBOL(gelu_table_bf16));
    if (e != hipSuccess) return (int)e;
    if (!t.ptr) return fail("GELU table has no device address");
  }
  *out = (uint16_t*)t.ptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cap);
  if (e != hipSuccess) return (int)e;
  auto build = [&]() {
    if (x_dtype == OGA_DT_F16)
      hipLaunchKernelGGL(k_gelu_table<OGA_DT_F16>, dim3(256), dim3(256), 0, st, (uint16_t*)t.ptr);
    else
      hipLaunchKernelGGL(k_gelu_table<OGA_DT_BF16>, dim3(256), dim3(256), 0, st, (uint16_t*)t.ptr);
    return launch_status();
  };
  // Under capture the graph builds the table itself (same values), so it
  // never depends on an event recorded outside the graph.
  if (cap != hipStreamCaptureStatusNone) return build();
  if (t.state.load(std::memory_order_relaxed) == kTableNone) {
    int rc = build();
    if (rc) return rc;
    if (!t.built && (e = hipEventCreateWithFlags(&t.built, hipEventDisableTiming)) != hipSuccess) return (int)e;
    if ((e = hipEventRecord(t.built, st)) != hipSuccess) return (int)e;
    t.state.store(kTablePending, std::memory_order_release);
    return OGA_OK;
  }
  // Pending: done already, or make this stream wait for it.
  e = hipEventQuery(t.built);
  if (e == hipSuccess) {
    t.state.store(kTableReady, std::memory_order_release);
    return OGA_OK;
  }
  if (e != hipErrorNotReady) return (int)e;
  e = hipStreamWaitEvent(st, t.built, 0);
  return e == hipSuccess ? OGA_OK : (int)e;
}

extern "C" int oga_gelu_tanh_fp8_quantize_e4m3(const void* x, int x_dtype, const float* scale, int scale_is_0dim,
                                               void* q, int64_t n, void* stream) {
  if (!x || !scale || !q) return fail("null pointer");
  if (!x16_dt_ok(x_dtype)) return unsupported("x dtype must be bf16 or fp16");
  if (n < 0) return fail("bad size");
  if (n == 0) return OGA_OK;
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  uint16_t* table = nullptr;
  int rc = gelu_table(x_dtype, st, &table);
  if (rc) return rc;
  // Steps of 1024 lanes x 32 elements; at most one workgroup per CU.
  const int64_t steps = (n + 32 * kGeluLanes - 1) / (32 * kGeluLanes);
  const int64_t wgs = steps < (int64_t)cu_count() ? steps : (int64_t)cu_count();
  if (x_dtype == OGA_DT_F16)
    hipLaunchKernelGGL(k_gelu_quant<OGA_DT_F16>, dim3((unsigned)wgs), dim3(kGeluLanes), 0, st, (const uint16_t*)x,
                       scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n, (const uint16_t*)table);
  else
    hipLaunchKernelGGL(k_gelu_quant<OGA_DT_BF16>, dim3((unsigned)wgs), dim3(kGeluLanes), 0, st, (const uint16_t*)x,
                       scale, scale_is_0dim ? 1 : 0, (uint8_t*)q, n, (const uint16_t*)table);
  return launch_status();
}

extern "C" int64_t oga_fp8_per_head_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim) {
  (void)head_dim;
  if (batch < 0 || tokens < 0 || heads < 0) return 0;
  return batch * head_chunks(tokens) * heads * (int64_t)sizeof(float);
}

// Both passes of the per-head quantizer with the amax partials in `partial`
// (batch * head_chunks(tokens) * heads floats; pass 1 writes every one that
// pass 2 reads, so nothing needs clearing).
static int per_head_run(const void* x, int x_dtype, void* q, float* scale_out, float* partial, int64_t batch,
                        int64_t tokens, int64_t heads, int64_t head_dim, hipStream_t st) {
  if (!x || !q || !scale_out || !partial) return fail("null pointer");
  if (!x16_dt_ok(x_dtype)) return unsupported("x dtype must be bf16 or fp16");
  if (batch < 1 || tokens < 1 || heads < 1) return fail("empty shape");
  if (batch > 65535) return unsupported("batch > 65535");
  if (head_dim != 64 && head_dim != 128) return unsupported("head_dim must be 64 or 128");
  const int64_t row = heads * head_dim;
  if (row != 1024 && row != 2048 && row != 4096) return unsupported("heads*head_dim must be 1024, 2048 or 4096");
  if (!aligned(x, 16) || !aligned(q, 16)) return fail("x/q must be 16-byte aligned");
  if (x_dtype == OGA_DT_F16)
    launch_per_head<OGA_DT_F16>((const uint16_t*)x, (uint8_t*)q, scale_out, partial, batch, tokens, heads, head_dim,
                                st);
  else
    launch_per_head<OGA_DT_BF16>((const uint16_t*)x, (uint8_t*)q, scale_out, partial, batch, tokens, heads,
                                 head_dim, st);
  return launch_status();
}

// ------------------------------------------- allocation-free entry point
// The amax partials of oga_fp8_quantize_per_head_noalloc live in `scratch`,
// a file-scope device array of kPerHeadScratchBytes that every GPU the
// library runs on holds until the process ends. In host code `scratch` only
// names the symbol; its address on a device comes from hipGetSymbolAddress,
// called with that device current on the first call there and kept per
// device. Calls on one device share the array: calls that overlap in time on
// one GPU (different streams, or threads) race on it.
constexpr int64_t kPerHeadScratchBytes = 1 << 20;
static __device__ __align__(256) float scratch[kPerHeadScratchBytes / sizeof(float)];
constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];

static int scratch_ptr(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return unsupported("device ordinal %d beyond %d", dev, kMaxScratchDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return fail("scratch has no device address");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = (float*)p;
  return OGA_OK;
}

extern "C" int oga_fp8_quantize_per_head(const void* x, int x_dtype, void* q, float* scale_out, void* workspace,
                                         int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                                         void* stream) {
  if (!workspace) return fail("null pointer");
  return per_head_run(x, x_dtype, q, scale_out, (float*)workspace, batch, tokens, heads, head_dim,
                      (hipStream_t)stream);
}

extern "C" int64_t oga_fp8_per_head_noalloc_max_bytes(void) { return kPerHeadScratchBytes; }

extern "C" int oga_fp8_quantize_per_head_noalloc(const void* x, int x_dtype, void* q, float* scale_out,
                                                 int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                                                 void* stream) {
  if (batch < 1 || tokens < 1 || heads < 1) return fail("empty shape");
  const int64_t need = oga_fp8_per_head_workspace_bytes(batch, tokens, heads, head_dim);
  if (need > kPerHeadScratchBytes)
    return unsupported("per-head amax partials need %lld bytes, more than the %lld-byte static scratch "
                       "(use oga_fp8_quantize_per_head with a workspace)", (long long)need,
                       (long long)kPerHeadScratchBytes);
  float* partial = nullptr;
  const int rc = scratch_ptr(&partial);
  if (rc) return rc;
  return per_head_run(x, x_dtype, q, scale_out, partial, batch, tokens, heads, head_dim, (hipStream_t)stream);
}

extern "C" int oga_selftest_convert(const float* in, uint16_t* bf16_out, uint8_t* e4m3_out, int64_t n, void* stream) {
  if (!in || !bf16_out || !e4m3_out) return fail("null pointer");
  if (n <= 0) return OGA_OK;
  hipLaunchKernelGGL(k_selftest_convert, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, in,
                     bf16_out, e4m3_out, n);
  return launch_status();
}
