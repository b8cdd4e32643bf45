// FP8 (e4m3fn) x FP8 -> bf16 linear with the exact bias epilogue.
//
// Reference: ltx_serve/triton_ltx_ops.py :1671-1718 (patched FP8Linear
// forward: quantize, torch._scaled_mm(q, W.t(), scale_a, scale_b,
// out_dtype=bf16), then `+ bias` in bf16 through fused_bias_add_bf16), with
// :742-781 for the from-quantized / without-bias forms.
//   out = R(acc * (scale_a * scale_b));  out = R(out + R(bias))  (if bias)
// acc is the float32 sum over k of a[m,k]*w[n,k] (each product exact).
//
// Tiling (gfx950): a 256x256 output tile per workgroup of 8 waves (two per
// SIMD), each wave owning 128 (M) x 64 (N) as 8x4 blocks of
// v_mfma_f32_16x16x128_f8f6f4 with its 128 accumulators in VGPRs.
// K advances 128 bytes per step through a double-buffered LDS stage of
// 2 x (256x128 A + 256x128 W) = 128 KiB, filled by LDS-DMA
// (global_load_lds_dwordx4) so tiles never pass through VGPRs; the two
// buffers are separate LDS objects so the DMA into one is known not to alias
// the fragment reads of the other. Within a stage, row r's 16-byte
// chunk c is stored at chunk position c ^ (r & 7), so the 128-bit fragment
// reads of 8 consecutive rows hit 8 distinct bank groups.
// The weight tile is the MFMA's A operand and the activation tile its B
// operand, so each lane's 4 accumulator values are 4 consecutive output
// columns of one row: the epilogue stores 8 bytes per lane.
// Workgroups are numbered so that the eight XCDs (which receive workgroups
// round-robin) each own a contiguous, M-grouped range of tiles.
#include "common.h"
#include "host.h"

namespace oga {

constexpr int GM = 256, GN = 256, GK = 128;
constexpr int kGroupM = 8;

struct GemmArgs {
  const uint8_t* a;
  const uint8_t* w;
  const float* sa;
  const float* sb;
  const void* bias;
  uint16_t* out;
  int64_t lda, ldw, ldo;
  int m, n, k;
  int tiles_m, tiles_n;
  int bias_dt;
  int xcd_remap;
};

typedef __attribute__((address_space(3))) void lds_void;

OGA_DEVICE i32x8 lds_frag(const uint4* s, int row, int g) {
  const int sw = row & 7;
  const uint4 u0 = s[row * 8 + ((2 * g) ^ sw)];
  const uint4 u1 = s[row * 8 + ((2 * g + 1) ^ sw)];
  i32x8 r;
  r[0] = (int)u0.x; r[1] = (int)u0.y; r[2] = (int)u0.z; r[3] = (int)u0.w;
  r[4] = (int)u1.x; r[5] = (int)u1.y; r[6] = (int)u1.z; r[7] = (int)u1.w;
  return r;
}

// Stage: 256 rows x 128 bytes of A and of W, written straight from global
// memory into LDS (global_load_lds_dwordx4). One instruction fills 1 KiB of
// LDS: lane p writes 16-byte slot base+p. Slot s holds row s/8, physical
// chunk s%8 = logical chunk kc ^ (row & 7); so lane p of block b fetches row
// 8b + p/8, logical chunk (p%8) ^ ((p/8)%8). Wave w fills blocks 4w..4w+3
// of each operand.
struct StagePtrs {
  uint32_t a_off[4];
  uint32_t w_off[4];
};

OGA_DEVICE void stage_issue(const uint8_t* abase, const uint8_t* wbase, const StagePtrs& sp, uint32_t kofs,
                            uint4* dA, uint4* dW, int wv) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wv * 4 + i;
    __builtin_amdgcn_global_load_lds((const void*)(abase + (sp.a_off[i] + kofs)), (lds_void*)(dA + blk * 64), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(wbase + (sp.w_off[i] + kofs)), (lds_void*)(dW + blk * 64), 16, 0, 0);
  }
}

OGA_DEVICE void stage_compute(const uint4* sA, const uint4* sW, f32x4 (&acc)[8][4], int wm, int wn, int fr, int fg) {
  i32x8 wf[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) wf[nb] = lds_frag(sW, wn * 64 + nb * 16 + fr, fg);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const i32x8 af = lds_frag(sA, wm * 128 + mb * 16 + fr, fg);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      acc[mb][nb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[nb], af, acc[mb][nb], 0, 0, 0, 0, 0, 0);
  }
  // Schedule: the 8 weight-fragment reads and the first activation fragment,
  // then for each block the next block's 2 fragment reads ahead of its 4
  // MFMAs, so at most two activation fragments are live.
  __builtin_amdgcn_sched_group_barrier(0x100, 10, 0);
#pragma unroll
  for (int mb = 0; mb < 7; ++mb) {
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
}

// s_waitcnt vmcnt(0) (expcnt/lgkmcnt left at their maxima).
OGA_DEVICE void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__global__ __launch_bounds__(512, 1) void k_fp8_gemm(GemmArgs g) {
  __shared__ uint4 sA0[GM * GK / 16];
  __shared__ uint4 sW0[GN * GK / 16];
  __shared__ uint4 sA1[GM * GK / 16];
  __shared__ uint4 sW1[GN * GK / 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wv >> 2, wn = wv & 3;

  // Tile index: XCD-contiguous ranges, M-grouped inside each range.
  const int nt = g.tiles_m * g.tiles_n;
  int t = blockIdx.x;
  if (g.xcd_remap) t = (t & 7) * (nt >> 3) + (t >> 3);
  const int per_group = kGroupM * g.tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * kGroupM;
  const int gsize = min(g.tiles_m - first_m, kGroupM);
  const int tm = first_m + (t % per_group) % gsize;
  const int tn = (t % per_group) / gsize;
  const int64_t m0 = (int64_t)tm * GM, n0 = (int64_t)tn * GN;

  // Per-lane byte offsets of the 8 rows this lane fetches per operand.
  // Rows past the matrix edge re-read its last row (never stored).
  StagePtrs sp;
  {
    const int pr = lane >> 3;
    const int kc = (lane & 7) ^ (pr & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (wv * 4 + i) * 8 + pr;
      const int64_t ar = min((int64_t)row, (int64_t)g.m - 1 - m0);
      const int64_t wr = min((int64_t)row, (int64_t)g.n - 1 - n0);
      sp.a_off[i] = (uint32_t)(ar * g.lda + kc * 16);
      sp.w_off[i] = (uint32_t)(wr * g.ldw + kc * 16);
    }
  }

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fg = lane >> 4;
  const int ksteps = g.k / GK;  // >= 1
  const uint8_t* abase = g.a + m0 * g.lda;
  const uint8_t* wbase = g.w + n0 * g.ldw;
  stage_issue(abase, wbase, sp, 0, sA0, sW0, wv);
  // Steady state: two K steps per trip, no branches inside. At each barrier
  // the buffer about to be read is complete (vmcnt(0) then s_barrier) and
  // every wave has finished reading the buffer about to be refilled.
  int ks = 0;
  for (; ks + 2 < ksteps; ks += 2) {
    wait_vm0();
    __syncthreads();
    stage_issue(abase, wbase, sp, (uint32_t)(ks + 1) * GK, sA1, sW1, wv);
    stage_compute(sA0, sW0, acc, wm, wn, fr, fg);
    wait_vm0();
    __syncthreads();
    stage_issue(abase, wbase, sp, (uint32_t)(ks + 2) * GK, sA0, sW0, wv);
    stage_compute(sA1, sW1, acc, wm, wn, fr, fg);
  }
  // Tail: one or two steps remain; step ks is in buffer 0.
  wait_vm0();
  __syncthreads();
  if (ks + 1 < ksteps) {
    stage_issue(abase, wbase, sp, (uint32_t)(ks + 1) * GK, sA1, sW1, wv);
    stage_compute(sA0, sW0, acc, wm, wn, fr, fg);
    wait_vm0();
    __syncthreads();
    stage_compute(sA1, sW1, acc, wm, wn, fr, fg);
  } else {
    stage_compute(sA0, sW0, acc, wm, wn, fr, fg);
  }

  // Epilogue: lane holds out[m][n .. n+3] for each (mb, nb).
  const float s = g.sa[0] * g.sb[0];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int64_t ncol = n0 + wn * 64 + nb * 16 + 4 * fg;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    const bool has_bias = g.bias != nullptr;
    if (has_bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t c = min(ncol + i, (int64_t)g.n - 1);
        const float v = g.bias_dt == OGA_DT_BF16 ? __uint_as_float(((uint32_t)((const uint16_t*)g.bias)[c]) << 16)
                                                 : ((const float*)g.bias)[c];
        bv[i] = rbf(v);
      }
    }
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int64_t mrow = m0 + wm * 128 + mb * 16 + fr;
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = rbf(acc[mb][nb][i] * s);
        if (has_bias) v = v + bv[i];
        o[i] = v;
      }
      if (mrow < g.m) {
        uint16_t* dst = g.out + mrow * g.ldo + ncol;
        if (ncol + 3 < g.n) {
          uint2 pk;
          pk.x = pack_bf16(o[0], o[1]);
          pk.y = pack_bf16(o[2], o[3]);
          *(uint2*)dst = pk;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (ncol + i < g.n) dst[i] = (uint16_t)(pack_bf16(o[i], 0.f) & 0xFFFF);
        }
      }
    }
  }
}

}  // namespace oga

using namespace oga;

extern "C" int oga_fp8_linear(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                              const float* scale_b, const void* bias, int bias_dtype, void* out, int64_t ldo,
                              int64_t m, int64_t n, int64_t k, void* stream) {
  if (!a || !w || !scale_a || !scale_b || !out) return fail("null pointer");
  if (m < 0 || n < 0 || k < 0) return fail("bad shape");
  if (m == 0 || n == 0) return OGA_OK;
  if (k == 0 || k % GK) return unsupported("K must be a positive multiple of %d (got %lld)", GK, (long long)k);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return unsupported("dimension too large");
  if (lda < k || ldw < k || ldo < n) return fail("leading dimension smaller than the row");
  if (!aligned(a, 16) || !aligned(w, 16) || lda % 16 || ldw % 16) return fail("a/w rows must be 16-byte aligned");
  if (!aligned(out, 8) || ldo % 4) return fail("out rows must be 8-byte aligned");
  // Per-lane offsets into one 256-row tile are 32-bit.
  if (256 * lda + 16 > (int64_t)UINT32_MAX || 256 * ldw + 16 > (int64_t)UINT32_MAX)
    return unsupported("row stride too large");
  if (bias && !dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  GemmArgs g{};
  g.a = (const uint8_t*)a;
  g.w = (const uint8_t*)w;
  g.sa = scale_a;
  g.sb = scale_b;
  g.bias = bias;
  g.bias_dt = bias_dtype;
  g.out = (uint16_t*)out;
  g.lda = lda;
  g.ldw = ldw;
  g.ldo = ldo;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.tiles_m = (int)((m + GM - 1) / GM);
  g.tiles_n = (int)((n + GN - 1) / GN);
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  g.xcd_remap = (nt % 8) == 0;
  hipLaunchKernelGGL(k_fp8_gemm, dim3((unsigned)nt), dim3(512), 0, (hipStream_t)stream, g);
  return launch_status();
}
