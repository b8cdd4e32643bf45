// FP8 (e4m3fn) x FP8 -> bf16 linear with the exact bias epilogue.
//
// Reference: ltx_serve/triton_ltx_ops.py :1671-1718 (patched FP8Linear
// forward: quantize, torch._scaled_mm(q, W.t(), scale_a, scale_b,
// out_dtype=bf16), then `+ bias` in bf16 through fused_bias_add_bf16), with
// :742-781 for the from-quantized / without-bias forms.
//   out = R(acc * (scale_a * scale_b));  out = R(out + R(bias))  (if bias)
// acc is the float32 sum over k of a[m,k]*w[n,k] (each product exact).
//
// Tiling (gfx950). A workgroup of 8 waves, two per SIMD, owns a 256 (M) x
// 256 (N) output tile; wave (wm, wn) owns 128 (M) x 64 (N) of it as 2 x 4
// blocks of v_mfma_f32_32x32x64_f8f6f4, whose 128 float32 accumulators per
// lane live in the accumulation registers. K advances 64 bytes per step through a ring of
// four LDS stages (4 x (256x64 A + 256x64 W) = 128 KiB) filled by LDS-DMA
// (global_load_lds_dwordx4), so tiles never pass through VGPRs and three
// steps of loads are in flight while one is consumed. Each stage is a
// separate LDS object so the compiler can tell a DMA into one stage from the
// fragment reads of another.
//
// Per step (software-pipelined): 4 MFMAs on fragments read during the
// previous step, then one barrier that publishes the next stage and
// releases the previous one, the DMA for three steps ahead into the released
// stage, and 4 more MFMAs under which the next step's fragments are read.
//
// LDS layout of an operand stage (256 rows x 64 bytes): four rows share one
// 256-byte line of the 64 LDS banks, row m's 16-byte chunk k0 sitting at
//   (m / 4) * 256 + ((4 * (m % 4) + k0) ^ ((m / 4) % 16)) * 16,
// which makes the 128-bit fragment reads (32 rows x 2 chunks per
// instruction) and the 1 KiB DMA writes free of bank conflicts.
//
// The weight tile is the MFMA's A operand and the activation tile its B
// operand, so each lane's accumulators hold 4 consecutive output columns of
// one output row per group. The epilogue stages each wave's finished bf16
// block in LDS and writes whole 128-byte rows, so HBM sees full lines.
// Workgroups are numbered so that the eight XCDs (which receive workgroups
// round-robin) each own a contiguous, M-grouped range of tiles.
#include "common.h"
#include "host.h"

namespace oga {

constexpr int GM = 256, GN = 256, GK = 64, NST = 4;
constexpr int kGroupM = 8;
constexpr int kStageU4 = GM * GK / 16;  // uint4 per operand stage (1024 = 16 KiB)
constexpr int kWaves = 8;
// Epilogue staging: each wave's 128 x 64 bf16 block in LDS with a padded row
// pitch (128 + 16 bytes) so the 8-byte writes of 32 rows hit distinct banks.
constexpr int kOutPitch = 144;
constexpr int kOutWaveBytes = 128 * kOutPitch;
constexpr int kLdsU4 = (NST * 2 * kStageU4 > kWaves * kOutWaveBytes / 16) ? NST * 2 * kStageU4
                                                                          : kWaves * kOutWaveBytes / 16;
constexpr int kDmaPerOp = GM / 16 / kWaves;  // 1 KiB DMA instructions per wave per operand per stage

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

// Byte offset in an operand stage of row m's 16-byte chunk k0.
OGA_DEVICE int lds_pos(int m, int k0) { return (m >> 2) * 256 + (((m & 3) * 4 + k0) ^ ((m >> 2) & 15)) * 16; }

// One 32-row MFMA operand fragment: lane l reads its row's logical chunks
// 2h and 2h+1 (h = l / 32), at LDS byte addresses a0 + OFF and a1 + OFF.
// The reads are issued as inline assembly so that the compiler, which does
// not see them, adds no DMA-ordering waits of its own: the kernel orders LDS
// explicitly (vmcnt before the barrier, lgkm_wait before the MFMAs).
template <int OFF>
OGA_DEVICE i32x8 frag(uint32_t a0, uint32_t a1) {
  uint4 lo, hi;
  asm volatile("ds_read_b128 %0, %2 offset:%4\n\tds_read_b128 %1, %3 offset:%4"
               : "=v"(lo), "=v"(hi)
               : "v"(a0), "v"(a1), "i"(OFF));
  i32x8 r = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  return r;
}

// s_waitcnt vmcnt(N) (expcnt/lgkmcnt left at their maxima); N < 64.
#define OGA_WAIT_VM(N) __builtin_amdgcn_s_waitcnt(0x0F70 | ((N) & 15) | ((((N) >> 4) & 3) << 14))
// s_waitcnt lgkmcnt(N) that also names the fragments it makes valid, so no
// use of them can be scheduled before it; naming accumulators as well keeps
// the MFMAs that update them from being scheduled after it.
#define OGA_LGKM_WAIT(N, ...) asm volatile("s_waitcnt lgkmcnt(" #N ")" : __VA_ARGS__)
// Workgroup barrier without the release fence of __syncthreads(), which
// would drain every outstanding DMA (vmcnt(0)) and empty the prefetch ring.
// Callers first wait for their own DMA group and LDS reads; the memory
// clobber keeps the compiler from moving memory accesses across it.
#define OGA_BARRIER() asm volatile("s_barrier" ::: "memory")

OGA_DEVICE f32x16 mfma(const i32x8& w, const i32x8& a, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, 0, 0, 0, 0);
}

__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void k_fp8_gemm(
    GemmArgs g) {
  // Stage s: A tile at uint4 [2s*kStageU4, (2s+1)*kStageU4), W tile after it.
  __shared__ uint4 smem[kLdsU4];

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

  // DMA: instruction i of this wave fills stage rows 16b .. 16b+15 of an
  // operand (b = kDmaPerOp*wave + i), i.e. 1 KiB = LDS lines 4b .. 4b+3;
  // lane p writes the 16 bytes at line 4b + p/16, chunk position p%16, which
  // by the layout above hold row 4*(4b + p/16) + kc/4, chunk kc%4 with
  // kc = (p%16) ^ ((4b + p/16) % 16). Rows past the matrix edge re-read
  // its last row (their results are never stored). Offsets are bytes from
  // the tile's first row.
  uint32_t a_off[kDmaPerOp], w_off[kDmaPerOp];
#pragma unroll
  for (int i = 0; i < kDmaPerOp; ++i) {
    const int line = (wv * kDmaPerOp + i) * 4 + (lane >> 4);
    const int kc = (lane & 15) ^ (line & 15);
    const int row = line * 4 + (kc >> 2);
    const int lc = kc & 3;
    const int64_t ar = min((int64_t)row, (int64_t)g.m - 1 - m0);
    const int64_t wr = min((int64_t)row, (int64_t)g.n - 1 - n0);
    a_off[i] = (uint32_t)(ar * g.lda + lc * 16);
    w_off[i] = (uint32_t)(wr * g.ldw + lc * 16);
  }
  const uint8_t* abase = g.a + m0 * g.lda;
  const uint8_t* wbase = g.w + n0 * g.ldw;
  const int ksteps = g.k / GK;  // >= 1
  // K steps are visited in a rotated order, starting at an even step that
  // depends on the tile, so that the workgroups of one XCD, which would
  // otherwise all read the same 64-byte column of their rows at the same
  // time, spread their requests over the L2 channels. (The float32 sum over K
  // is taken in a different order; the result stays within the contract.)
  const int rot = ((4 * t) % ksteps) & ~1;
  const int klast = ksteps - 1;
  auto kphys = [&](int step) -> uint32_t {  // byte offset of logical step (clamped to K)
    int s2 = min(step, klast) + rot;
    if (s2 >= ksteps) s2 -= ksteps;
    return (uint32_t)s2 * GK;
  };
  // DMA of logical step `step` into stage S (one group = 2*kDmaPerOp
  // instructions per wave; groups complete in issue order).
  auto issue = [&](int S, int step) {
    uint4* d = smem + S * 2 * kStageU4;
    const uint32_t k0 = kphys(step);
#pragma unroll
    for (int i = 0; i < kDmaPerOp; ++i) {
      const int blk = wv * kDmaPerOp + i;
      __builtin_amdgcn_global_load_lds((const void*)(abase + (a_off[i] + k0)), (lds_void*)(d + blk * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(wbase + (w_off[i] + k0)), (lds_void*)(d + kStageU4 + blk * 64),
                                       16, 0, 0);
    }
  };

  // Fragment addressing: lane reads row (lane & 31) of a 32-row block,
  // chunks 2h and 2h+1 (h = lane / 32). By the layout, block b's chunk
  // positions depend on b's parity only, and blocks b and b + 2 are 4096
  // bytes apart: so each lane keeps, per operand, the stage-0 byte addresses
  // of its two chunks for an even and an odd block.
  const int fr = lane & 31, fh = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem;
  const uint32_t wbyte = kStageU4 * 16;  // W follows A inside a stage
  // W blocks of this wave: 2*wn + i (i = 0, 1); A blocks: 4*wm + j.
  const uint32_t lw00 = lds0 + wbyte + wn * 4096 + lds_pos(fr, 2 * fh);
  const uint32_t lw01 = lds0 + wbyte + wn * 4096 + lds_pos(fr, 2 * fh + 1);
  const uint32_t lw10 = lds0 + wbyte + wn * 4096 + lds_pos(32 + fr, 2 * fh);
  const uint32_t lw11 = lds0 + wbyte + wn * 4096 + lds_pos(32 + fr, 2 * fh + 1);
  const uint32_t la00 = lds0 + wm * 8192 + lds_pos(fr, 2 * fh);
  const uint32_t la01 = lds0 + wm * 8192 + lds_pos(fr, 2 * fh + 1);
  const uint32_t la10 = lds0 + wm * 8192 + lds_pos(32 + fr, 2 * fh);
  const uint32_t la11 = lds0 + wm * 8192 + lds_pos(32 + fr, 2 * fh + 1);
  constexpr uint32_t kStageBytes = 2 * kStageU4 * 16;

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Software pipeline. Stage s % NST holds step s. Entering step ks, the
  // first fragment set (w0, w1, a0, a1) of ks is already being read; the
  // step reads its a2, a3 under its first four MFMAs, then (if step ks + 1
  // exists) waits for its own DMA of ks + 1, joins the barrier that
  // publishes stage ks + 1 and releases stage ks - 1 (every wave finished
  // reading it before its previous second half), sends the DMA of step
  // ks + 3 into the released stage, and reads the first fragments of ks + 1
  // under its last four MFMAs. DMA groups in flight at the barrier wait:
  // ks + 1 and ks + 2, so vmcnt(2*kDmaPerOp) leaves ks + 1 complete.
  // Steps past the end of K (when K is not a multiple of NST*GK) run their
  // MFMAs on zeroed fragments, so the accumulators have one path.
  issue(0, 0);
  issue(1, 1);
  issue(2, 2);
  OGA_WAIT_VM(4 * kDmaPerOp);
  OGA_BARRIER();
  i32x8 xw0 = frag<0>(lw00, lw01), xw1 = frag<0>(lw10, lw11);
  i32x8 xa0 = frag<0>(la00, la01), xa1 = frag<0>(la10, la11);
  i32x8 yw0, yw1, ya0, ya1;

#define OGA_STEP(S, C, N)                                                                                      \
  {                                                                                                            \
    const int ks = kb + (S);                                                                                   \
    const bool live = ks < ksteps;                                                                             \
    const uint32_t so = (S) * kStageBytes;                                                                     \
    i32x8 a2 = frag<4096>(la00 + so, la01 + so);                                                               \
    i32x8 a3 = frag<4096>(la10 + so, la11 + so);                                                               \
    OGA_LGKM_WAIT(4, "+v"(C##w0), "+v"(C##w1), "+v"(C##a0), "+v"(C##a1), "+v"(acc[0][2]), "+v"(acc[1][2]),     \
                  "+v"(acc[0][3]), "+v"(acc[1][3]));                                                           \
    if (!live) C##w0 = C##w1 = C##a0 = C##a1 = i32x8{0, 0, 0, 0, 0, 0, 0, 0};                                 \
    acc[0][0] = mfma(C##w0, C##a0, acc[0][0]);                                                                 \
    acc[1][0] = mfma(C##w1, C##a0, acc[1][0]);                                                                 \
    acc[0][1] = mfma(C##w0, C##a1, acc[0][1]);                                                                 \
    acc[1][1] = mfma(C##w1, C##a1, acc[1][1]);                                                                 \
    if (ks + 1 < ksteps) {                                                                                     \
      OGA_WAIT_VM(2 * kDmaPerOp);                                                                              \
      asm volatile("s_barrier"                                                                                 \
                   : "+v"(acc[0][0]), "+v"(acc[1][0]), "+v"(acc[0][1]), "+v"(acc[1][1])                        \
                   :                                                                                           \
                   : "memory");                                                                                \
      issue(((S) + 3) % NST, ks + 3);                                                                          \
    }                                                                                                          \
    const uint32_t sn = (((S) + 1) % NST) * kStageBytes;                                                       \
    N##w0 = frag<0>(lw00 + sn, lw01 + sn);                                                                     \
    N##w1 = frag<0>(lw10 + sn, lw11 + sn);                                                                     \
    N##a0 = frag<0>(la00 + sn, la01 + sn);                                                                     \
    N##a1 = frag<0>(la10 + sn, la11 + sn);                                                                     \
    OGA_LGKM_WAIT(8, "+v"(a2), "+v"(a3), "+v"(acc[0][0]), "+v"(acc[1][0]), "+v"(acc[0][1]), "+v"(acc[1][1]));  \
    if (!live) a2 = a3 = i32x8{0, 0, 0, 0, 0, 0, 0, 0};                                                       \
    acc[0][2] = mfma(C##w0, a2, acc[0][2]);                                                                    \
    acc[1][2] = mfma(C##w1, a2, acc[1][2]);                                                                    \
    acc[0][3] = mfma(C##w0, a3, acc[0][3]);                                                                    \
    acc[1][3] = mfma(C##w1, a3, acc[1][3]);                                                                    \
  }

  for (int kb = 0; kb < ksteps; kb += NST) {
    OGA_STEP(0, x, y)
    OGA_STEP(1, y, x)
    OGA_STEP(2, x, y)
    OGA_STEP(3, y, x)
  }
#undef OGA_STEP
  OGA_LGKM_WAIT(0, "+v"(xw0), "+v"(xw1), "+v"(xa0), "+v"(xa1));

  // Epilogue. Block (i, j): lane holds, for q in 0..3, output row
  // m = wm*128 + 32j + (lane & 31) of the tile and columns n .. n+3 with
  // n = wn*64 + 32i + 8q + 4*(lane >> 5), in acc[i][j][4q .. 4q+3]. The
  // finished bf16 values go to this wave's LDS block, and are then written
  // to HBM as whole 128-byte rows, 16 bytes per lane.
  OGA_WAIT_VM(0);  // the last (clamped) DMA groups land before LDS is reused
  OGA_BARRIER();   // every wave has finished reading the stages
  const float s = g.sa[0] * g.sb[0];
  const bool has_bias = g.bias != nullptr;
  const uint32_t ob = lds0 + wv * kOutWaveBytes;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = i * 32 + q * 8 + 4 * fh;  // column inside the wave's block
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (has_bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t c = min(n0 + wn * 64 + nl + e, (int64_t)g.n - 1);
          const float v = g.bias_dt == OGA_DT_BF16 ? __uint_as_float(((uint32_t)((const uint16_t*)g.bias)[c]) << 16)
                                                   : ((const float*)g.bias)[c];
          bv[e] = rbf(v);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = rbf(acc[i][j][q * 4 + e] * s);
          if (has_bias) v = v + bv[e];
          o[e] = v;
        }
        uint2 pk;
        pk.x = pack_bf16(o[0], o[1]);
        pk.y = pack_bf16(o[2], o[3]);
        const uint32_t addr = ob + (j * 32 + fr) * kOutPitch + nl * 2;
        asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(pk) : "memory");
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // Row r of the block: 8 lanes x 16 bytes; 8 rows per pass, 16 passes.
  const int rsub = lane >> 3, cb = (lane & 7) * 8;  // column (bf16) inside the row
  const int64_t ncol = n0 + wn * 64 + cb;
#pragma unroll 4
  for (int pass = 0; pass < 16; ++pass) {
    const int r = pass * 8 + rsub;
    uint4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(ob + r * kOutPitch + cb * 2) : "memory");
    const int64_t mrow = m0 + wm * 128 + r;
    if (mrow < g.m) {
      uint16_t* dst = g.out + mrow * g.ldo + ncol;
      if (ncol + 8 <= g.n) {
        *(uint4*)dst = v;
      } else {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (ncol + e < g.n) dst[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
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
  if (!aligned(out, 16) || ldo % 8) return fail("out rows must be 16-byte aligned");
  // Per-lane byte offsets inside one 256-row tile (plus K) are 32-bit.
  if (256 * lda + k > (int64_t)UINT32_MAX || 256 * ldw + k > (int64_t)UINT32_MAX)
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
  if (nt > INT32_MAX) return unsupported("too many tiles");
  g.xcd_remap = (nt % 8) == 0;
  hipLaunchKernelGGL(k_fp8_gemm, dim3((unsigned)nt), dim3(64 * kWaves), 0, (hipStream_t)stream, g);
  return launch_status();
}
