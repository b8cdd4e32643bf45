// Dense non-causal self-attention (bf16 in/out, float32 softmax and
// accumulation) for head_dim 128 on gfx950 MFMA.
//
// Reference: the video self-attention of the LTX block, which opengenie runs
// through FlashAttention-3's flash_attn_func(q, k, v) on [B, N, H, D] views
// (benchmarks/official_ltx23_benchmark.py:3294-3369; FlashAttention3.__call__
// of ltx_core), with softmax scale D^-0.5:
//   O[b, n, h] = sum_m softmax_m(q[b,n,h] . k[b,m,h] * scale) v[b,m,h].
// FP8 inputs (e4m3 with per-(b, h) descales, :3333-3340) go through
// oga_fp8_dequant_per_head first: each value times its float32 descale,
// rounded to bf16 (FA3 computes in FP8 directly; the reference benchmark
// checks the FP8 result against the bf16 one within a tolerance,
// video_self_attention_bench.py:288-305, and so do the tests here).
//
// Work decomposition. A workgroup of 4 waves owns 128 queries of one (b, h);
// wave w owns queries 32w .. 32w+31. Keys are visited 64 at a time; the K
// and V tiles of a step (64 x 128 bf16 each) are copied to LDS by DMA
// (global_load_lds_dwordx4), two steps in flight.
//
// Per step and wave, with v_mfma_f32_32x32x16_bf16:
//  * S^T = K Q^T as two 32-key x 32-query blocks (8 MFMAs each over d):
//    operand A = K rows from LDS, operand B = the wave's Q^T fragments, kept
//    in registers for the whole key loop. Lane l then holds 16 scores of
//    query l % 32 per block (keys 8g + 4(l/32) + r for accumulator 4g + r),
//    so a query's max and sum need one exchange with lane l ^ 32.
//  * online softmax in base 2 (the scale folded with log2 e), P rounded to
//    bf16 as FlashAttention does before the P.V product.
//  * O^T = V^T P^T as four 32-d x 32-query blocks over four 16-key chunks:
//    operand B = P^T straight from the score accumulators, operand A = V^T
//    read with ds_read_b64_tr_b16 (transposing reads) from the row-major V
//    tile. The k-slot order of both operands is the same permutation of the
//    16 keys of a chunk, so they pair up without moving P between lanes.
// LDS tiles: key row r (256 bytes = 16 chunks of 16 B) keeps chunk c at
// physical chunk c ^ (r % 16), so the 32-row fragment reads and the
// transposing reads hit distinct bank groups.
#include "common.h"
#include "host.h"

namespace oga {

constexpr int kAD = 128;      // head dim
constexpr int kAQ = 128;      // queries per workgroup
constexpr int kAK = 64;       // keys per step
constexpr int kATileU4 = kAK * kAD * 2 / 16;  // uint4 per K (or V) tile: 1024 (16 KiB)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  uint16_t* o;
  int64_t q_sb, q_sn, q_sh;  // element strides (batch, token, head); d stride 1
  int64_t k_sb, k_sn, k_sh;
  int64_t v_sb, v_sn, v_sh;
  int64_t o_sb, o_sn, o_sh;
  int64_t nq, nk;
  int heads;
  float scale_log2;  // softmax scale * log2(e)
};

OGA_DEVICE f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Byte offset of (key row r, element d) in a swizzled LDS tile.
OGA_DEVICE int tile_off(int r, int d) { return r * 256 + ((((d >> 3) ^ (r & 15)) << 4) | ((d & 7) << 1)); }

OGA_DEVICE float exchange32(float v) { return __shfl_xor(v, 32); }

// DMA of one 64-key tile of K or V (bf16 rows of kAD elements) into LDS:
// instruction i of wave w fills tile rows 4b .. 4b+3 (b = 4w + i); lane p
// writes the 16 bytes at row 4b + p/16, physical chunk p%16, i.e. logical
// chunk (p%16) ^ (row%16). Rows past the last key re-read the last key.
OGA_DEVICE void tile_dma(const uint16_t* base, int64_t row_stride, int64_t key0, int64_t nk, uint4* dst, int wv,
                         int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wv * 4 + i;
    const int row = blk * 4 + (lane >> 4);
    const int chunk = (lane & 15) ^ (row & 15);
    const int64_t key = min(key0 + row, nk - 1);
    __builtin_amdgcn_global_load_lds((const void*)(base + key * row_stride + chunk * 8), (lds_void*)(dst + blk * 64),
                                     16, 0, 0);
  }
}

OGA_DEVICE uint32_t pack2(float a, float b) { return pack_bf16(a, b); }

__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
  __shared__ uint4 sK0[kATileU4], sV0[kATileU4], sK1[kATileU4], sV1[kATileU4];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.x * kAQ + wv * 32;
  const int hl = lane >> 5;  // lane half
  const int ql = lane & 31;

  // Q^T fragments: step s covers d = 16s .. 16s+15; lane holds d = 16s + 8*hl .. +7
  // of query q0 + ql (queries past nq read the last query, never stored).
  bf16x8 qf[8];
  {
    const int64_t qi = min(q0 + ql, a.nq - 1);
    const uint16_t* qrow = (const uint16_t*)a.q + b * a.q_sb + qi * a.q_sn + (int64_t)h * a.q_sh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(bf16x8, *(const uint4*)(qrow + 16 * s + 8 * hl));
  }

  const uint16_t* kbase = (const uint16_t*)a.k + b * a.k_sb + (int64_t)h * a.k_sh;
  const uint16_t* vbase = (const uint16_t*)a.v + b * a.v_sb + (int64_t)h * a.v_sh;
  const int64_t nsteps = (a.nk + kAK - 1) / kAK;

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  tile_dma(kbase, a.k_sn, 0, a.nk, sK0, wv, lane);
  tile_dma(vbase, a.v_sn, 0, a.nk, sV0, wv, lane);

  auto step = [&](const uint4* sK, const uint4* sV, uint4* nK, uint4* nV, int64_t st) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's DMA of step st landed
    __syncthreads();                     // ... every wave's; the other buffers are free
    if (st + 1 < nsteps) {
      tile_dma(kbase, a.k_sn, (st + 1) * kAK, a.nk, nK, wv, lane);
      tile_dma(vbase, a.v_sn, (st + 1) * kAK, a.nk, nV, wv, lane);
    }
    const char* kb = (const char*)sK;
    // S^T blocks: key block j (keys 32j .. 32j+31), lane key row 32j + ql.
    f32x16 sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[j][e] = 0.0f;
      const int r = 32 * j + ql;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bf16x8 kf = __builtin_bit_cast(bf16x8, *(const uint4*)(kb + tile_off(r, 16 * s + 8 * hl)));
        sacc[j] = mfma_bf16(kf, qf[s], sacc[j]);
      }
    }
    // Scores in base 2; keys past nk masked.
    const int64_t key0 = st * kAK;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 32 * j + 8 * (e >> 2) + 4 * hl + (e & 3);
        float sv = sacc[j][e] * a.scale_log2;
        if (key0 + key >= a.nk) sv = -INFINITY;
        sacc[j][e] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, exchange32(mx));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);  // 0 on the first step (m_run = -inf)
    float psum = 0.0f;
    uint32_t pb[2][8];  // P as packed bf16: block j, 8 words (16 values)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = rbf(exp2f(sacc[j][e] - m_new));
        const float p1 = rbf(exp2f(sacc[j][e + 1] - m_new));
        psum += p0 + p1;
        pb[j][e >> 1] = pack2(p0, p1);
      }
    psum += exchange32(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[i][e] *= alpha;

    // O^T += V^T P^T over 16-key chunks c2 (keys 16 c2 .. 16 c2 + 15).
    const int a4 = lane & 3, j4 = (lane & 15) >> 2, g2 = (lane >> 4) & 1;
    const char* vb = (const char*)sV;
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {
      // B = P^T: accumulators 8(c2 % 2) .. +7 of block c2 / 2.
      const uint32_t* pw = &pb[c2 >> 1][4 * (c2 & 1)];
      uint4 pu;
      pu.x = pw[0]; pu.y = pw[1]; pu.z = pw[2]; pu.w = pw[3];
      const bf16x8 pf = __builtin_bit_cast(bf16x8, pu);
#pragma unroll
      for (int dblk = 0; dblk < 4; ++dblk) {
        // A = V^T: two transposing reads; read c supplies keys 16 c2 + 8c + 4 hl + j4
        // at d = 32 dblk + 16 g2 + 4 a4 .. +3.
        bf16x4 v0, v1;
        {
          const int d = 32 * dblk + 16 * g2 + 4 * a4;
          const int r0 = 16 * c2 + 4 * hl + j4;
          const int r1 = r0 + 8;
          v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + tile_off(r0, d)));
          v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + tile_off(r1, d)));
        }
        const bf16x8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o[dblk] = mfma_bf16(vf, pf, o[dblk]);
      }
    }
  };

  for (int64_t st = 0; st < nsteps; st += 2) {
    step(sK0, sV0, sK1, sV1, st);
    if (st + 1 < nsteps) step(sK1, sV1, sK0, sV0, st + 1);
  }

  // O = O^T / l: lane holds query q0 + ql, d = 32 dblk + 8 (e/4) + 4 hl + e%4.
  const int64_t qi = q0 + ql;
  if (qi < a.nq) {
    const float inv = 1.0f / l_run;
    uint16_t* orow = a.o + b * a.o_sb + qi * a.o_sn + (int64_t)h * a.o_sh;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 w;
        w.x = pack2(o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv);
        w.y = pack2(o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv);
        *(uint2*)(orow + 32 * dblk + 8 * g + 4 * hl) = w;
      }
  }
}

// out[b, n, h, d] = R(e4m3(x8[b, n, h, d]) * descale[b, h]); 16 values per
// thread (x8 contiguous [B, N, H, D], D a multiple of 16).
__global__ __launch_bounds__(256) void k_fp8_dequant_per_head(const uint8_t* x8, const float* descale, uint16_t* out,
                                                             int64_t n, int64_t tokens, int heads, int d) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  const int64_t row = (int64_t)heads * d;
  const int64_t tok = i0 / row;
  const int64_t hh = (i0 - tok * row) / d;
  const int64_t bb = tok / tokens;
  const float s = descale[bb * heads + hh];
  const uint4 u = *(const uint4*)(x8 + i0);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  float f[16];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);
    f[4 * k] = lo[0] * s;
    f[4 * k + 1] = lo[1] * s;
    f[4 * k + 2] = hi[0] * s;
    f[4 * k + 3] = hi[1] * s;
  }
  st_nt16(out + i0, pack8(f));
  st_nt16(out + i0 + 8, pack8(f + 8));
}

}  // namespace oga

using namespace oga;

extern "C" int oga_fp8_dequant_per_head(const void* x8, const float* descale, void* out, int64_t batch,
                                        int64_t tokens, int64_t heads, int64_t head_dim, void* stream) {
  if (!x8 || !descale || !out) return fail("null pointer");
  if (batch < 0 || tokens < 0 || heads < 0 || head_dim <= 0) return fail("bad shape");
  if (head_dim % 16) return unsupported("head_dim must be a multiple of 16");
  if (!aligned(x8, 16) || !aligned(out, 16)) return fail("x8/out must be 16-byte aligned");
  const int64_t n = batch * tokens * heads * head_dim;
  if (n == 0) return OGA_OK;
  const int64_t threads = n / 16;
  hipLaunchKernelGGL(k_fp8_dequant_per_head, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)x8, descale, (uint16_t*)out, n, tokens, (int)heads,
                     (int)head_dim);
  return launch_status();
}

extern "C" int oga_attention(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                             const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3],
                             int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim,
                             float softmax_scale, void* stream) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return fail("null pointer");
  if (head_dim != kAD) return unsupported("head_dim must be %d", kAD);
  if (batch < 0 || nq < 0 || nk < 0 || heads < 0) return fail("bad shape");
  if (batch == 0 || nq == 0 || heads == 0) return OGA_OK;
  if (nk == 0) return unsupported("no keys");
  if (batch > 65535 || heads > 65535) return unsupported("batch/heads too large");
  for (const int64_t* s : {q_strides, k_strides, v_strides, o_strides})
    for (int i = 0; i < 3; ++i)
      if (s[i] % 8) return fail("strides must be multiples of 8 elements");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 16))
    return fail("q/k/v/o must be 16-byte aligned");
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = (uint16_t*)o;
  a.q_sb = q_strides[0]; a.q_sn = q_strides[1]; a.q_sh = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sn = k_strides[1]; a.k_sh = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sn = v_strides[1]; a.v_sh = v_strides[2];
  a.o_sb = o_strides[0]; a.o_sn = o_strides[1]; a.o_sh = o_strides[2];
  a.nq = nq; a.nk = nk; a.heads = (int)heads;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  const dim3 grid((unsigned)((nq + kAQ - 1) / kAQ), (unsigned)heads, (unsigned)batch);
  hipLaunchKernelGGL(k_attention, grid, dim3(256), 0, (hipStream_t)stream, a);
  return launch_status();
}
