// FP8 (e4m3fn) x FP8 -> bf16 (or fp16) linear with the exact bias epilogue.
//
// Reference: ltx_serve/triton_ltx_ops.py :1671-1718 (patched FP8Linear
// forward: quantize, torch._scaled_mm(q, W.t(), scale_a, scale_b,
// out_dtype=bf16), then `+ bias` in bf16 through fused_bias_add_bf16), with
// :742-781 for the from-quantized / without-bias forms.
//   out = R(acc * (scale_a * scale_b));  out = R(out + R(bias))  (if bias)
// acc is the float32 sum over k of a[m,k]*w[n,k] (each product exact); R
// rounds to the output dtype, bf16 or, for an fp16 FP8Linear (out_dtype =
// x.dtype, :1697-1709), fp16 (the O16 template flag of every epilogue).
//
// Tiling (gfx950). A workgroup of 4 waves, one per SIMD, owns a 256 (M) x
// 256 (N) output tile; wave (wm, wn) owns 128 (M) x 128 (N) of it as 4 x 4
// blocks of v_mfma_f32_32x32x64_f8f6f4, whose 256 float32 accumulators per
// lane live in the accumulation registers. One MFMA step covers 64 bytes of
// K; the operands move through LDS in slabs of 128 bytes of K (two steps),
// three A and two W slab buffers (5 x 32 KiB = 160 KiB), filled by LDS-DMA
// (global_load_lds / buffer_load ... lds, 16 bytes per lane) so tiles never
// pass through VGPRs. Each DMA instruction fetches eight whole 128-byte
// rows: full-line requests halve the address and tag work of the load path
// compared with 64-byte half lines.
//
// Step pair (2d, 2d+1) consumes slab d. Fragments are read one step ahead
// (double-buffered in VGPRs) between the step's first eight MFMAs. At the
// odd step 2d+1 every wave waits for its DMA of slab d+1 and joins one
// barrier, which publishes slab d+1 and tells that every wave has finished
// reading slab d (its last fragments were read during step 2d). The DMA of
// A slab d+2 (into the A buffer of slab d-1) is spread over the last eight
// MFMAs of step 2d, that of W slab d+2 (into slab d's W buffer) over the
// last eight of step 2d+1: A is sent two and a half steps, W one and a half
// steps before it is needed.
//
// Two kernels share this loop: k_fp8_gemm_ring (K >= 256, N % 128 == 0, bf16
// or no bias) is persistent, one workgroup per CU looping over tiles with
// the slab ring running on across tile boundaries; k_fp8_gemm (every other
// supported shape) runs one workgroup per tile.
//
// LDS layout of an operand slab (256 rows x 128 bytes): two rows share one
// 256-byte line of the 64 LDS banks; row r's 16-byte chunk c (c = 0..7)
// sits at byte
//   (r / 2) * 256 + ((8 * (r % 2) + c) ^ ((r / 2) % 8)) * 16,
// which keeps the 128-bit fragment reads (32 rows x 2 chunks per
// instruction) free of bank conflicts and lets each 1 KiB DMA write fill
// four whole lines. The A slabs fill LDS bytes [0, 96 KiB) and the W slabs
// [96 KiB, 160 KiB); every fragment read is a per-lane base plus the slab
// buffer's offset plus an immediate offset.
//
// The weight tile is the MFMA's A operand and the activation tile its B
// operand, so each lane's accumulators hold 4 consecutive output columns of
// one output row per group. The epilogue stages each wave's finished bf16
// block in LDS and writes whole rows, so HBM sees full lines.
// Workgroups are numbered so that the eight XCDs (which receive workgroups
// round-robin) each own a contiguous, M-grouped range of tiles.
#include "common.h"
#include "host.h"

namespace oga {

constexpr int GM = 256, GN = 256;
constexpr int GK = 64;                    // bytes of K per MFMA step
constexpr int GKS = 128;                  // bytes of K per LDS slab (two steps)
constexpr int kGroupM = 8;
constexpr int kSlabBytes = GM * GKS;      // one operand slab: 32 KiB
constexpr int kABufs = 3, kWBufs = 2;     // slab buffers per operand
constexpr int kWBase = kABufs * kSlabBytes;  // W buffers follow the A buffers (96 KiB)
constexpr int kWaves = 4;
// Epilogue staging: each wave's 128 x 128 bf16 block in LDS with a padded row
// pitch (256 + 16 bytes) so the 8-byte writes of 32 rows spread over the banks.
constexpr int kOutPitch = 272;
constexpr int kOutWaveBytes = 128 * kOutPitch;
constexpr int kLdsBytes = ((kABufs + kWBufs) * kSlabBytes > kWaves * kOutWaveBytes) ? (kABufs + kWBufs) * kSlabBytes
                                                                                    : kWaves * kOutWaveBytes;
constexpr int kDmaPerOp = GM * GKS / 1024 / kWaves;  // 1 KiB DMA instructions per wave per operand per slab (8)
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(3 * 4096 < 65536, "fragment offsets must fit the 16-bit immediate");

constexpr int kMaxGroups = 4;

// The output dtype's rounding, packing and unpacking (O16: fp16, else bf16).
template <bool O16>
OGA_DEVICE float rout(float v) { return O16 ? rhf(v) : rbf(v); }
template <bool O16>
OGA_DEVICE uint32_t pack_out(float lo, float hi) { return O16 ? pack_f16(lo, hi) : pack_bf16(lo, hi); }
template <bool O16>
OGA_DEVICE float out_lo(uint32_t w) { return O16 ? f16_lo(w) : bf16_lo(w); }
template <bool O16>
OGA_DEVICE float out_hi(uint32_t w) { return O16 ? f16_hi(w) : bf16_hi(w); }
// A 16-bit bias is in the output dtype (the host passes bias.to(fp16) for an
// fp16 output), so R(bias) is the value itself.

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
  int out_f16;  // output dtype fp16 (else bf16); the host picks the O16 instances by it
  int xcd_remap;
  // Persistent kernel: `units` work units, either whole tiles (the first
  // nfull tiles) or K-chunks of the remaining tiles, each cut into `split`
  // chunks of kchunk slabs, whose float32 partial sums go to ws.
  int nfull, split, kchunk, units;
  float* ws;
  // Persistent kernel: the N columns are `groups` linears of group_n columns
  // sharing the activation (1 group: the plain linear). Group i has its own
  // weight, weight scale, bias and output; a tile never straddles two.
  const uint8_t* wg[kMaxGroups];
  const float* sbg[kMaxGroups];
  const void* biasg[kMaxGroups];
  uint16_t* outg[kMaxGroups];
  int group_n;
};

// Group i's entry of a kernel-argument array, by a uniform select chain (no
// dynamic indexing, which would copy the arguments to scratch).
template <typename T>
OGA_DEVICE T pick(T const (&arr)[kMaxGroups], int i) {
  static_assert(kMaxGroups == 4, "select chain covers four groups");
  return i == 0 ? arr[0] : i == 1 ? arr[1] : i == 2 ? arr[2] : arr[3];
}

typedef __attribute__((address_space(3))) void lds_void;

// Byte offset in an operand slab of row r's 16-byte chunk c (0..7).
constexpr int slab_pos(int r, int c) { return (r >> 1) * 256 + (((r & 1) * 8 + c) ^ ((r >> 1) & 7)) * 16; }

// One 32-row MFMA operand fragment: lane l reads 32 bytes of its row at LDS
// byte addresses a0 + OFF and a1 + OFF. The reads are issued as inline
// assembly so that the compiler, which does not see them, adds no
// DMA-ordering waits of its own: the kernel orders LDS explicitly (vmcnt
// before the barrier, OGA_LGKM_WAIT before the MFMAs).
template <int OFF>
OGA_DEVICE i32x8 frag(uint32_t a0, uint32_t a1) {
  uint4 lo, hi;
  // Early-clobber outputs: the first read's data returns after the second
  // read has issued, so its destination must not share a register with a1.
  asm volatile("ds_read_b128 %0, %2 offset:%4\n\tds_read_b128 %1, %3 offset:%4"
               : "=&v"(lo), "=&v"(hi)
               : "v"(a0), "v"(a1), "i"(OFF));
  i32x8 r = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  return r;
}

// s_waitcnt vmcnt(N) (expcnt/lgkmcnt left at their maxima); N < 64.
#define OGA_WAIT_VM(N) __builtin_amdgcn_s_waitcnt(0x0F70 | ((N) & 15) | ((((N) >> 4) & 3) << 14))
// s_waitcnt lgkmcnt(N) that also names the fragments it makes valid, so no
// use of them can be scheduled before it.
#define OGA_LGKM_WAIT(N, ...) asm volatile("s_waitcnt lgkmcnt(" #N ")" : __VA_ARGS__)
// Workgroup barrier without the release fence of __syncthreads(), which
// would also wait for every outstanding DMA. Callers first wait for their
// own DMA and LDS reads; the memory clobber keeps the compiler from moving
// memory accesses across it.
#define OGA_BARRIER() asm volatile("s_barrier" ::: "memory")

OGA_DEVICE f32x16 mfma(const i32x8& w, const i32x8& a, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, 0, 0, 0, 0);
}


// Fragment read addresses folded into per-lane bases (checked for every lane,
// block, step parity and chunk pair): block b (rows 32b .. 32b+31), step
// parity p (chunks 4p .. 4p+3), lane (fr, fh) reading chunk 4p + 2fh + q:
//   slab_pos(32b + fr, 4p + 2fh + q)
//     = 4096 b + (fr/2)*256 + (8 (fr%2) + ((4p + 2fh + q) ^ ((fr/2) % 8))) * 16.
constexpr bool frag_bases_match() {
  for (int lane = 0; lane < 64; ++lane) {
    const int fr = lane & 31, fh = lane >> 5;
    for (int b = 0; b < 8; ++b)
      for (int p = 0; p < 2; ++p)
        for (int q = 0; q < 2; ++q) {
          const int c = 4 * p + 2 * fh + q;
          const int got = 4096 * b + (fr >> 1) * 256 + (8 * (fr & 1) + (c ^ ((fr >> 1) & 7))) * 16;
          if (slab_pos(32 * b + fr, c) != got) return false;
        }
  }
  return true;
}
static_assert(frag_bases_match(), "folded fragment addresses differ from slab_pos");

template <bool O16>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void k_fp8_gemm(
    GemmArgs g) {
  __shared__ uint4 smem[kLdsBytes / 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wv >> 1, wn = wv & 1;

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

  // DMA: instruction i of this wave fills slab rows 8b .. 8b+7 of an operand
  // (b = kDmaPerOp*wave + i), i.e. 1 KiB = LDS lines 4b .. 4b+3; lane p
  // writes the 16 bytes at line L = 4b + p/16, position p%16, which by the
  // layout hold row 2L + v/8, chunk v%8 with v = (p%16) ^ (L%8): the eight
  // lanes of each row cover its whole 128-byte line. Rows past the matrix
  // edge re-read its last row (their results are never stored). Offsets are
  // bytes from the tile's first row.
  uint32_t a_off[kDmaPerOp], w_off[kDmaPerOp];
#pragma unroll
  for (int i = 0; i < kDmaPerOp; ++i) {
    const int line = (wv * kDmaPerOp + i) * 4 + (lane >> 4);
    const int v = (lane & 15) ^ (line & 7);
    const int row = 2 * line + (v >> 3);
    const int c = v & 7;
    const int64_t ar = min((int64_t)row, (int64_t)g.m - 1 - m0);
    const int64_t wr = min((int64_t)row, (int64_t)g.n - 1 - n0);
    a_off[i] = (uint32_t)(ar * g.lda + c * 16);
    w_off[i] = (uint32_t)(wr * g.ldw + c * 16);
  }
  const uint8_t* abase = g.a + m0 * g.lda;
  const uint8_t* wbase = g.w + n0 * g.ldw;
  const int ksteps = g.k / GK;  // even, >= 2
  const int nslab = ksteps >> 1;
  uint8_t* lds_bytes = (uint8_t*)smem;
  // DMA instruction I (0..7) of operand A or W for slab d (< nslab) into
  // byte offset `buf` of LDS.
  auto dma = [&](auto i_c, auto w_c, uint32_t buf, int d) {
    constexpr int I = decltype(i_c)::value;
    constexpr bool W = decltype(w_c)::value;
    // readfirstlane hides the slab offset from loop strength reduction,
    // which would otherwise keep a 64-bit address per instruction live.
    const uint32_t k0 = __builtin_amdgcn_readfirstlane((uint32_t)d * GKS);
    const int blk = wv * kDmaPerOp + I;
    if constexpr (!W)
      __builtin_amdgcn_global_load_lds((const void*)(abase + (a_off[I] + k0)), (lds_void*)(lds_bytes + buf + blk * 1024),
                                       16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((const void*)(wbase + (w_off[I] + k0)), (lds_void*)(lds_bytes + buf + blk * 1024),
                                       16, 0, 0);
  };
  static_assert(kDmaPerOp == 8, "the DMA schedule below covers 8 instructions per operand");
  auto issue_all = [&](auto w_c, uint32_t buf, int d) {
    dma(IC<0>{}, w_c, buf, d); dma(IC<1>{}, w_c, buf, d); dma(IC<2>{}, w_c, buf, d); dma(IC<3>{}, w_c, buf, d);
    dma(IC<4>{}, w_c, buf, d); dma(IC<5>{}, w_c, buf, d); dma(IC<6>{}, w_c, buf, d); dma(IC<7>{}, w_c, buf, d);
  };
  // Buffers: A slab d in A buffer d % 3, W slab d in W buffer d % 2.
  auto abuf = [&](int d) { return (uint32_t)((d % kABufs) * kSlabBytes); };
  auto wbuf = [&](int d) { return (uint32_t)(kWBase + (d % kWBufs) * kSlabBytes); };

  // Per-lane fragment bases (frag_bases_match): [parity][chunk of the pair],
  // relative to the slab buffer. The wave's W blocks are 4wn + i and its A
  // blocks 4wm + j (i, j = 0..3).
  const int fr = lane & 31, fh = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  uint32_t lw[2][2], la[2][2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t in_line = (fr >> 1) * 256 + (8 * (fr & 1) + ((4 * p + 2 * fh + q) ^ ((fr >> 1) & 7))) * 16;
      lw[p][q] = lds0 + wn * 16384 + in_line;
      la[p][q] = lds0 + wm * 16384 + in_line;
    }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Fragments of step parity P from the slab buffers at byte offsets ab (A)
  // and wb (W): W block i / A block j.
#define OGA_FRAG_W(P, i) frag<(i) * 4096>(lw[P][0] + wb, lw[P][1] + wb)
#define OGA_FRAG_A(P, j) frag<(j) * 4096>(la[P][0] + ab, la[P][1] + ab)

  // Issue order of the DMA groups (8 instructions per wave each): A0 W0 A1
  // W1 in the prologue, then A(d+2) at even step 2d and W(d+2) at odd step
  // 2d+1. Prologue: slab 0 landed (A1, W1 may stay in flight), published,
  // step 0's fragments read.
  issue_all(IC<0>{}, abuf(0), 0);
  issue_all(IC<1>{}, wbuf(0), 0);
  if (nslab > 1) {
    issue_all(IC<0>{}, abuf(1), 1);
    issue_all(IC<1>{}, wbuf(1), 1);
    OGA_WAIT_VM(2 * kDmaPerOp);
  } else {
    OGA_WAIT_VM(0);
  }
  OGA_BARRIER();
  i32x8 xw[4], xa[4], yw[4], ya[4];
  {
    const uint32_t ab = abuf(0), wb = wbuf(0);
    xw[0] = OGA_FRAG_W(0, 0);
    xw[1] = OGA_FRAG_W(0, 1);
    xw[2] = OGA_FRAG_W(0, 2);
    xw[3] = OGA_FRAG_W(0, 3);
    xa[0] = OGA_FRAG_A(0, 0);
    xa[1] = OGA_FRAG_A(0, 1);
    xa[2] = OGA_FRAG_A(0, 2);
    xa[3] = OGA_FRAG_A(0, 3);
  }
  OGA_LGKM_WAIT(0, "+v"(xw[0]), "+v"(xw[1]), "+v"(xw[2]), "+v"(xw[3]), "+v"(xa[0]), "+v"(xa[1]), "+v"(xa[2]),
                "+v"(xa[3]));

#define OGA_MF(i, j) acc[i][j] = mfma(cw[i], ca[j], acc[i][j])
  // Even step 2d: its 16 MFMAs; the 8 fragments of step 2d+1 (same slab,
  // parity 1, published with it) read between the first eight, and the DMA
  // of A slab d+2 (into the A buffer of slab d-1, released by the barrier of
  // step 2d-1) one instruction after each of the last eight.
  // D: slab d + 2 exists (the last two slabs send no DMA).
  auto even_step = [&](auto d_c, int d, i32x8(&cw)[4], i32x8(&ca)[4], i32x8(&nw)[4], i32x8(&na)[4]) {
    constexpr bool D = decltype(d_c)::value;
    const uint32_t ab = abuf(d), wb = wbuf(d), an = abuf(d + 2);
    const int dn = d + 2;
    OGA_MF(0, 0); nw[0] = OGA_FRAG_W(1, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 1); nw[1] = OGA_FRAG_W(1, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 2); nw[2] = OGA_FRAG_W(1, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 3); nw[3] = OGA_FRAG_W(1, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 0); na[0] = OGA_FRAG_A(1, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 1); na[1] = OGA_FRAG_A(1, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 2); na[2] = OGA_FRAG_A(1, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 3); na[3] = OGA_FRAG_A(1, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 0); if constexpr (D) dma(IC<0>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 1); if constexpr (D) dma(IC<1>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 2); if constexpr (D) dma(IC<2>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 3); if constexpr (D) dma(IC<3>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 0); if constexpr (D) dma(IC<4>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 1); if constexpr (D) dma(IC<5>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 2); if constexpr (D) dma(IC<6>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 3); if constexpr (D) dma(IC<7>{}, IC<0>{}, an, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_LGKM_WAIT(0, "+v"(nw[0]), "+v"(nw[1]), "+v"(nw[2]), "+v"(nw[3]), "+v"(na[0]), "+v"(na[1]), "+v"(na[2]),
                  "+v"(na[3]));
  };
  // Odd step 2d+1: wait until this wave's A and W of slab d+1 landed (only
  // A slab d+2, sent at step 2d, may stay in flight), barrier (slab d+1
  // published; every wave done with slab d), then its 16 MFMAs with the
  // fragments of step 2d+2 (slab d+1, parity 0) read between the first
  // eight and the DMA of W slab d+2 (into slab d's W buffer) one instruction
  // after each of the last eight. (After the last step the reads re-read
  // settled LDS: every DMA has landed; the values go unused.)
  auto odd_step = [&](auto d_c, int d, i32x8(&cw)[4], i32x8(&ca)[4], i32x8(&nw)[4], i32x8(&na)[4]) {
    constexpr bool D = decltype(d_c)::value;
    const uint32_t ab = abuf(d + 1), wb = wbuf(d + 1), wn2 = wbuf(d + 2);
    const int dn = d + 2;
    if constexpr (D) OGA_WAIT_VM(kDmaPerOp);
    else OGA_WAIT_VM(0);  // no A slab d + 2 was sent
    OGA_BARRIER();
    __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 0); nw[0] = OGA_FRAG_W(0, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 1); nw[1] = OGA_FRAG_W(0, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 2); nw[2] = OGA_FRAG_W(0, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 3); nw[3] = OGA_FRAG_W(0, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 0); na[0] = OGA_FRAG_A(0, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 1); na[1] = OGA_FRAG_A(0, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 2); na[2] = OGA_FRAG_A(0, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 3); na[3] = OGA_FRAG_A(0, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 0); if constexpr (D) dma(IC<0>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 1); if constexpr (D) dma(IC<1>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 2); if constexpr (D) dma(IC<2>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 3); if constexpr (D) dma(IC<3>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 0); if constexpr (D) dma(IC<4>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 1); if constexpr (D) dma(IC<5>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 2); if constexpr (D) dma(IC<6>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 3); if constexpr (D) dma(IC<7>{}, IC<1>{}, wn2, dn); __builtin_amdgcn_sched_barrier(0);
    OGA_LGKM_WAIT(0, "+v"(nw[0]), "+v"(nw[1]), "+v"(nw[2]), "+v"(nw[3]), "+v"(na[0]), "+v"(na[1]), "+v"(na[2]),
                  "+v"(na[3]));
  };
#undef OGA_MF

  int d = 0;
  for (; d + 2 < nslab; ++d) {
    even_step(IC<1>{}, d, xw, xa, yw, ya);
    odd_step(IC<1>{}, d, yw, ya, xw, xa);
  }
  if (d + 1 < nslab) {
    even_step(IC<0>{}, d, xw, xa, yw, ya);
    odd_step(IC<0>{}, d, yw, ya, xw, xa);
    ++d;
  }
  even_step(IC<0>{}, d, xw, xa, yw, ya);
  odd_step(IC<0>{}, d, yw, ya, xw, xa);
#undef OGA_FRAG_W
#undef OGA_FRAG_A

  // Epilogue. Block (i, j): lane holds, for q in 0..3, output row
  // m = wm*128 + 32j + (lane & 31) of the tile and columns n .. n+3 with
  // n = wn*128 + 32i + 8q + 4*(lane >> 5), in acc[i][j][4q .. 4q+3]. The
  // finished bf16 values go to this wave's LDS block, and are then written
  // to HBM as whole 256-byte rows, 16 bytes per lane.
  //
  // Bias: the lane's 16 groups of 4 consecutive columns, loaded before the
  // DMA drain below so the two latencies overlap (one 8- or 16-byte load per
  // group when the wave's 128 columns are inside N and the bias is aligned).
  const bool has_bias = g.bias != nullptr;
  const int64_t ncol0 = n0 + wn * 128;  // first output column of the wave's block
  float bv[4][4][4];
  if (has_bias) {
    const bool bf = g.bias_dt != OGA_DT_F32;  // 16 bits: the output dtype
    const bool vec = ncol0 + 128 <= g.n && ((uintptr_t)g.bias % (bf ? 8 : 16)) == 0;
    if (vec) {
      if (bf) {
        uint2 raw[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) raw[i][q] = *(const uint2*)((const uint16_t*)g.bias + ncol0 + i * 32 + q * 8 + 4 * fh);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            bv[i][q][0] = out_lo<O16>(raw[i][q].x);
            bv[i][q][1] = out_hi<O16>(raw[i][q].x);
            bv[i][q][2] = out_lo<O16>(raw[i][q].y);
            bv[i][q][3] = out_hi<O16>(raw[i][q].y);
          }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 f = *(const float4*)((const float*)g.bias + ncol0 + i * 32 + q * 8 + 4 * fh);
            bv[i][q][0] = rout<O16>(f.x);
            bv[i][q][1] = rout<O16>(f.y);
            bv[i][q][2] = rout<O16>(f.z);
            bv[i][q][3] = rout<O16>(f.w);
          }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t c = min(ncol0 + i * 32 + q * 8 + 4 * fh + e, (int64_t)g.n - 1);
            if (bf) {
              bv[i][q][e] = out_lo<O16>((uint32_t)((const uint16_t*)g.bias)[c]);
            } else {
              bv[i][q][e] = rout<O16>(((const float*)g.bias)[c]);
            }
          }
    }
  }
  const float sc = g.sa[0] * g.sb[0];
  OGA_WAIT_VM(0);  // no DMA is in flight into LDS that is about to be reused
  OGA_BARRIER();   // every wave has finished reading the slabs
  const uint32_t ob = lds0 + wv * kOutWaveBytes;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = i * 32 + q * 8 + 4 * fh;  // column inside the wave's block
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = rout<O16>(acc[i][j][q * 4 + e] * sc);
          if (has_bias) v = v + bv[i][q][e];
          o[e] = v;
        }
        uint2 pk;
        pk.x = pack_out<O16>(o[0], o[1]);
        pk.y = pack_out<O16>(o[2], o[3]);
        const uint32_t addr = ob + (j * 32 + fr) * kOutPitch + nl * 2;
        asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(pk) : "memory");
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // Row r of the block: 16 lanes x 16 bytes; 4 rows per pass, 32 passes in
  // groups of 8 (8 LDS reads in flight, then 8 stores).
  const int rsub = lane >> 4, cb = (lane & 15) * 8;  // column (bf16) inside the row
  const int64_t ncol = ncol0 + cb;
  const uint32_t rd0 = ob + rsub * kOutPitch + cb * 2;
#pragma unroll
  for (int grp8 = 0; grp8 < 4; ++grp8) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v[u]) : "v"(rd0), "i"((grp8 * 8 + u) * 4 * kOutPitch));
    OGA_LGKM_WAIT(0, "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int r = (grp8 * 8 + u) * 4 + rsub;
      const int64_t mrow = m0 + wm * 128 + r;
      if (mrow < g.m) {
        uint16_t* dst = g.out + mrow * g.ldo + ncol;
        if (ncol + 8 <= g.n) {
          *(u32x4*)dst = v[u];
        } else {
          const uint32_t w4[4] = {v[u][0], v[u][1], v[u][2], v[u][3]};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (ncol + e < g.n) dst[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Persistent form (K >= 256, N a multiple of 128). One workgroup per CU runs
// tiles v, v + G, v + 2G, ... (G = grid size; with the XCD remap every tile
// of a workgroup lies in its XCD's range, and at any moment the XCD's
// workgroups work on consecutive tiles of that range) and keeps the slab
// ring running across tile boundaries: the DMA of a tile's last two slabs
// fetches slabs 0 and 1 of its next tile, so when the epilogue ends the next
// tile's first operands are in LDS and its first fragments in VGPRs. The
// epilogue stages each wave's output, 32 rows at a time, in its own quarter
// of the A buffer of the tile's last slab: no wave reads that buffer any
// more (the last odd step's barrier), no DMA targets it until the next
// tile's first even step, and the first DMA into that quarter is the same
// wave's own, issued after its staging reads completed. The stores are not
// waited for here; the next tile's first odd step waits for them with the
// DMA sent before them.
constexpr int kStagePitch = 136;  // bytes per staged row of 64 bf16 columns
static_assert(32 * kStagePitch <= kSlabBytes / kWaves, "a staging pass fits the wave's quarter of an A buffer");
// Staged row r, 16-byte chunk c (of 8) sits at byte r * kStagePitch + 16c.
// Writes: lane (fr, fh) stores 8 bytes of row fr at chunk c, half fh; each
// 32-lane half of a ds_write_b64 must touch 64 distinct banks. Reads: lane l
// loads row 4u + l/16 + 16*((l/8)%2), chunk l%8; each 16-lane group of a
// ds_read_b128 must touch 64 distinct banks.
constexpr bool stage_writes_conflict_free() {
  for (int c = 0; c < 8; ++c)
    for (int half = 0; half < 2; ++half) {
      unsigned long long banks = 0;
      for (int l = 32 * half; l < 32 * half + 32; ++l) {
        const int b = (((l & 31) * kStagePitch + (l >> 5) * 8 + 16 * c) >> 2) & 63;
        if ((banks >> b) & 3ull) return false;
        banks |= 3ull << b;  // b is even: no wrap
      }
    }
  return true;
}
constexpr bool stage_reads_conflict_free() {
  for (int u = 0; u < 4; ++u)
    for (int grp = 0; grp < 4; ++grp) {
      unsigned long long banks = 0;
      for (int l = 16 * grp; l < 16 * grp + 16; ++l) {
        const int row = 4 * u + (l >> 4) + 16 * ((l >> 3) & 1);
        const int b = ((row * kStagePitch + (l & 7) * 16) >> 2) & 63;
        for (int k = 0; k < 4; ++k) {
          if ((banks >> ((b + k) & 63)) & 1ull) return false;
          banks |= 1ull << ((b + k) & 63);
        }
      }
    }
  return true;
}
static_assert(stage_writes_conflict_free(), "staging writes would conflict");
static_assert(stage_reads_conflict_free(), "staging reads would conflict");
// Word 3 of a buffer resource on gfx9: 32-bit data format, no swizzle.
constexpr int kBufferWord3 = 0x00020000;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) uint16_t gu16;
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
// buffer_load_dwordx4 ... lds: LDS-DMA through a buffer resource; lanes out
// of the resource's range read nothing.
__device__ void buffer_load_lds(i32x4 rsrc, lds_void* lds, int size, int voffset, int soffset, int offset,
                                int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");
// buffer_store_dwordx4 through a buffer resource; lanes out of its range
// write nothing.
__device__ void buffer_store_x4(u32x4 data, i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.store.v4i32");
// Cache policy of the output stores: non-temporal (written once, not read
// back by this kernel; keeps L2 for the operand slabs).
constexpr int kStoreNT = 2;
// An accumulator as the MFMA left it in an AGPR, read into a VGPR where the
// epilogue needs it (so that only the values of one staging pass are live
// in VGPRs, not all of them from the end of the K loop on).
OGA_DEVICE float acc_read(float x) {
  float r;
  asm("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(x));
  return r;
}
// A 16-byte global load the compiler does not wait for by itself: the
// caller's own vmcnt waits cover it before the value is used, so the
// compiler adds no wait that would also drain the DMA sent after it.
OGA_DEVICE u32x4 load_x4_unwaited(gu32x4* p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
// 128 bf16 -0.0 values: the bias row of a linear without bias.
__device__ const uint16_t kNegZeroRow[128] = {
#define OGA_NZ8 0x8000, 0x8000, 0x8000, 0x8000, 0x8000, 0x8000, 0x8000, 0x8000
    OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8,
    OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8, OGA_NZ8,
#undef OGA_NZ8
};

template <bool PARTIAL, bool O16>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void k_fp8_gemm_ring(
    GemmArgs g) {
  __shared__ uint4 smem[(kABufs + kWBufs) * kSlabBytes / 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wv >> 1, wn = wv & 1;
  const int fr = lane & 31, fh = lane >> 5;
  const int per_group = kGroupM * g.tiles_n;
  const int nslab = g.k / GKS;  // >= 2
  uint8_t* lds_bytes = (uint8_t*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  // Work unit u in launch order -> tile origin, first k-slab, slab count and
  // (PARTIAL) split index. Whole tiles: units 0 .. nfull-1 are tiles
  // 0 .. nfull-1; PARTIAL: unit sp is K-chunk sp % split of tile
  // nfull + sp / split. The XCD remap makes each XCD's units a contiguous
  // range; tiles follow the M-grouped order of k_fp8_gemm.
  auto unit = [&](int u, int& m0, int& n0, int& kb, int& kn, int& sp) {
    int t;
    const int x = g.xcd_remap ? (u & 7) * (g.units >> 3) + (u >> 3) : u;
    if constexpr (!PARTIAL) {
      t = x;
      kb = 0;
      kn = nslab;
      sp = -1;
    } else {
      sp = x;
      t = g.nfull + sp / g.split;
      kb = (sp % g.split) * g.kchunk;
      kn = g.kchunk;
    }
    const int grp = t / per_group;
    const int first_m = grp * kGroupM;
    const int gsize = min(g.tiles_m - first_m, kGroupM);
    m0 = (first_m + (t % per_group) % gsize) * GM;
    n0 = ((t % per_group) / gsize) * GN;
  };
  // The operands are read through buffer resources based at the tile's first
  // row and sized to its rows inside the matrix: a DMA lane past the edge is
  // out of range and reads no memory, so the per-lane offsets are the same
  // for every tile. Lane offsets as in k_fp8_gemm; the slab offset is the
  // scalar offset.
  auto resource = [&](const void* base, uint32_t bytes) {
    const uint64_t addr = (uint64_t)base;
    const i32x4 r = {__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
                     __builtin_amdgcn_readfirstlane((int)((uint32_t)(addr >> 32) & 0xFFFFu)),
                     __builtin_amdgcn_readfirstlane((int)bytes), kBufferWord3};
    return r;
  };
  auto rsrc = [&](const uint8_t* base, int r0, int rows, int64_t ld) {
    // < 2^32 bytes: 256 * ld + K fits (host check)
    return resource(base + (int64_t)r0 * ld, (uint32_t)(min(rows - r0, GM) * ld));
  };
  // DMA instructions i and i + 2 of a wave cover rows 16 apart at the same
  // chunk (their line indices differ by 8), so two per-lane offsets per
  // operand serve all eight: instruction i reads row row_(i%2) + 16*(i/2).
  uint32_t a_off[2], w_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int line = (wv * kDmaPerOp + i) * 4 + (lane >> 4);
    const int c16 = (lane & 15) ^ (line & 7);
    const int row = 2 * line + (c16 >> 3);
    a_off[i] = (uint32_t)(row * g.lda + (c16 & 7) * 16);
    w_off[i] = (uint32_t)(row * g.ldw + (c16 & 7) * 16);
  }
  const uint32_t a_row16 = (uint32_t)(16 * g.lda), w_row16 = (uint32_t)(16 * g.ldw);
  // DMA instruction I of operand A or W for k-slab dk through resource rs
  // into byte offset `buf` of LDS. The row lies in the lane offset, which
  // the range check sees; the slab offset is the scalar offset.
  auto dma = [&](auto i_c, auto w_c, const i32x4& rs, uint32_t buf, int dk) {
    constexpr int I = decltype(i_c)::value;
    constexpr bool W = decltype(w_c)::value;
    const int blk = wv * kDmaPerOp + I;
    const uint32_t voff = W ? w_off[I & 1] + (I >> 1) * w_row16 : a_off[I & 1] + (I >> 1) * a_row16;
    buffer_load_lds(rs, (lds_void*)(lds_bytes + buf + blk * 1024), 16, (int)voff, dk * GKS, 0, 0);
  };
  auto issue_all = [&](auto w_c, const i32x4& rs, uint32_t buf, int dk) {
    dma(IC<0>{}, w_c, rs, buf, dk); dma(IC<1>{}, w_c, rs, buf, dk); dma(IC<2>{}, w_c, rs, buf, dk);
    dma(IC<3>{}, w_c, rs, buf, dk); dma(IC<4>{}, w_c, rs, buf, dk); dma(IC<5>{}, w_c, rs, buf, dk);
    dma(IC<6>{}, w_c, rs, buf, dk); dma(IC<7>{}, w_c, rs, buf, dk);
  };
  // Ring position s (counted across tiles): A slab in A buffer s % 3, W slab
  // in W buffer s % 2.
  auto abuf = [&](int s) { return (uint32_t)((s % kABufs) * kSlabBytes); };
  auto wbuf = [&](int s) { return (uint32_t)(kWBase + (s % kWBufs) * kSlabBytes); };

  // Fragment bases (as in k_fp8_gemm); the A bases are the W bases plus the
  // uniform (wm - wn) * 16 KiB, added with the slab buffer offset.
  uint32_t lw[2][2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t in_line = (fr >> 1) * 256 + (8 * (fr & 1) + ((4 * p + 2 * fh + q) ^ ((fr >> 1) & 7))) * 16;
      lw[p][q] = lds0 + wn * 16384 + in_line;
    }
  const uint32_t a_minus_w = (uint32_t)((wm - wn) * 16384);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

#define OGA_FRAG_W(P, i) frag<(i) * 4096>(lw[P][0] + wb, lw[P][1] + wb)
#define OGA_FRAG_A(P, j) frag<(j) * 4096>(lw[P][0] + ab, lw[P][1] + ab)
// MFMA of block (i, j); the first step of a tile (Z) starts from zero.
#define OGA_MF(i, j) acc[i][j] = mfma(cw[i], ca[j], Z ? kZero16 : acc[i][j])
  // Even step of ring slab s: as in k_fp8_gemm, with the A DMA of k-slab dk
  // through resource rs into ring slot s + 2; on a tile's first slab (z_c)
  // the MFMAs take zero accumulators.
  const f32x16 kZero16 = {};
  auto even_step = [&](auto z_c, int s, int dk, const i32x4& rs, i32x8(&cw)[4], i32x8(&ca)[4], i32x8(&nw)[4],
                       i32x8(&na)[4]) {
    constexpr bool Z = decltype(z_c)::value;
    const uint32_t ab = abuf(s) + a_minus_w, wb = wbuf(s), an = abuf(s + 2);
    OGA_MF(0, 0); nw[0] = OGA_FRAG_W(1, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 1); nw[1] = OGA_FRAG_W(1, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 2); nw[2] = OGA_FRAG_W(1, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 3); nw[3] = OGA_FRAG_W(1, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 0); na[0] = OGA_FRAG_A(1, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 1); na[1] = OGA_FRAG_A(1, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 2); na[2] = OGA_FRAG_A(1, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 3); na[3] = OGA_FRAG_A(1, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 0); dma(IC<0>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 1); dma(IC<1>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 2); dma(IC<2>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 3); dma(IC<3>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 0); dma(IC<4>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 1); dma(IC<5>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 2); dma(IC<6>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 3); dma(IC<7>{}, IC<0>{}, rs, an, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_LGKM_WAIT(0, "+v"(nw[0]), "+v"(nw[1]), "+v"(nw[2]), "+v"(nw[3]), "+v"(na[0]), "+v"(na[1]), "+v"(na[2]),
                  "+v"(na[3]));
  };
  // Odd step of ring slab s: wait for slab s + 1 (only the A DMA of the even
  // step may stay in flight; every older DMA, bias load and output store is
  // waited for), barrier, MFMAs with the fragments of slab s + 1 read between
  // the first eight, and the W DMA of k-slab dk through resource rs into
  // ring slot s + 2.
  auto odd_step = [&](int s, int dk, const i32x4& rs, i32x8(&cw)[4], i32x8(&ca)[4], i32x8(&nw)[4],
                      i32x8(&na)[4]) {
    constexpr bool Z = false;
    const uint32_t ab = abuf(s + 1) + a_minus_w, wb = wbuf(s + 1), wn2 = wbuf(s + 2);
    OGA_WAIT_VM(kDmaPerOp);
    OGA_BARRIER();
    __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 0); nw[0] = OGA_FRAG_W(0, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 1); nw[1] = OGA_FRAG_W(0, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 2); nw[2] = OGA_FRAG_W(0, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(0, 3); nw[3] = OGA_FRAG_W(0, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 0); na[0] = OGA_FRAG_A(0, 0); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 1); na[1] = OGA_FRAG_A(0, 1); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 2); na[2] = OGA_FRAG_A(0, 2); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(1, 3); na[3] = OGA_FRAG_A(0, 3); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 0); dma(IC<0>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 1); dma(IC<1>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 2); dma(IC<2>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(2, 3); dma(IC<3>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 0); dma(IC<4>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 1); dma(IC<5>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 2); dma(IC<6>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_MF(3, 3); dma(IC<7>{}, IC<1>{}, rs, wn2, dk); __builtin_amdgcn_sched_barrier(0);
    OGA_LGKM_WAIT(0, "+v"(nw[0]), "+v"(nw[1]), "+v"(nw[2]), "+v"(nw[3]), "+v"(na[0]), "+v"(na[1]), "+v"(na[2]),
                  "+v"(na[3]));
  };
#undef OGA_MF

  // Staging: a pass holds 32 rows x 64 columns of the wave's block (block
  // row j, column half h) inside the wave's 8 KiB quarter. Lane (fr, fh)
  // writes at sw + 64*(i - 2h) + 16q; lane l reads its row (srow, plus 4u)
  // at sr + 4u * kStagePitch.
  const int srow = (lane >> 4) + 16 * ((lane >> 3) & 1);
  const uint32_t sw = (uint32_t)(fr * kStagePitch + fh * 8);
  const uint32_t sr = (uint32_t)(srow * kStagePitch + (lane & 7) * 16);

  // sa * sb of each group, read before any DMA is in flight (read in the
  // epilogue, they would make it wait for every outstanding DMA).
  float scg[kMaxGroups];
#pragma unroll
  for (int i = 0; i < kMaxGroups; ++i)
    scg[i] = PARTIAL ? 0.0f : __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(g.sa[0] * g.sbg[i][0])));

  int v = blockIdx.x;
  int s = 0;
  int m0, n0, kb, kn, sp;
  unit(v, m0, n0, kb, kn, sp);
  // W of the group holding columns n0 .. n0 + 255, from its first row.
  auto wrsrc = [&](int n0) {
    const int gi = n0 / g.group_n, r0 = n0 - gi * g.group_n;
    return rsrc(pick(g.wg, gi), r0, g.group_n, g.ldw);
  };
  i32x4 ra = rsrc(g.a, m0, g.m, g.lda), rw = wrsrc(n0);
  issue_all(IC<0>{}, ra, abuf(0), kb);
  issue_all(IC<1>{}, rw, wbuf(0), kb);
  issue_all(IC<0>{}, ra, abuf(1), kb + 1);
  issue_all(IC<1>{}, rw, wbuf(1), kb + 1);
  OGA_WAIT_VM(2 * kDmaPerOp);
  OGA_BARRIER();
  i32x8 xw[4], xa[4], yw[4], ya[4];
  {
    const uint32_t ab = abuf(0) + a_minus_w, wb = wbuf(0);
    xw[0] = OGA_FRAG_W(0, 0);
    xw[1] = OGA_FRAG_W(0, 1);
    xw[2] = OGA_FRAG_W(0, 2);
    xw[3] = OGA_FRAG_W(0, 3);
    xa[0] = OGA_FRAG_A(0, 0);
    xa[1] = OGA_FRAG_A(0, 1);
    xa[2] = OGA_FRAG_A(0, 2);
    xa[3] = OGA_FRAG_A(0, 3);
  }
#undef OGA_FRAG_W
#undef OGA_FRAG_A
  OGA_LGKM_WAIT(0, "+v"(xw[0]), "+v"(xw[1]), "+v"(xw[2]), "+v"(xw[3]), "+v"(xa[0]), "+v"(xa[1]), "+v"(xa[2]),
                "+v"(xa[3]));

  for (;;) {
    // The next unit (after the last one: this unit again, whose first slabs
    // are then re-read and never consumed).
    const int vn = v + (int)gridDim.x;
    const bool more = vn < g.units;
    int nm0, nn0, nkb, nkn, nsp;
    unit(more ? vn : v, nm0, nn0, nkb, nkn, nsp);
    const i32x4 nra = rsrc(g.a, nm0, g.m, g.lda), nrw = wrsrc(nn0);
    // The group of this tile: its bias, output, scale and first column.
    const int gi = n0 / g.group_n, nc0 = n0 - gi * g.group_n;
    const void* const gbias = pick(g.biasg, gi);
    // Bias of the 16 columns this lane stores, (lane % 8) * 8 + 0..7 of each
    // 64-column half of the wave's block, as bf16 (R(bias)). A block wholly
    // past N reads the last 128 columns instead (its results are not
    // stored); without a bias the values are -0.0, which an add leaves every
    // value (signed zeros included) as it is. Loaded at the tile's start;
    // the wait of the first odd step covers them.
    u32x4 bq[2];
    if constexpr (!PARTIAL) {
      gu16* const bsrc = gbias ? (gu16*)gbias + min(nc0 + wn * 128, g.group_n - 128) : (gu16*)kNegZeroRow;
      bq[0] = load_x4_unwaited((gu32x4*)(bsrc + (lane & 7) * 8));
      bq[1] = load_x4_unwaited((gu32x4*)(bsrc + 64 + (lane & 7) * 8));
    }
    // All slabs of the unit; the DMA of its last two fetches the first two
    // slabs of the next unit.
    // The first slab's MFMAs start from zero accumulators.
    auto slab = [&](auto z_c, int d) {
      const bool here = d + 2 < kn;
      const int dk = here ? kb + d + 2 : nkb + d + 2 - kn;
      even_step(z_c, s, dk, here ? ra : nra, xw, xa, yw, ya);
      odd_step(s, dk, here ? rw : nrw, yw, ya, xw, xa);
      ++s;
    };
    slab(IC<1>{}, 0);
    for (int d = 1; d < kn; ++d) slab(IC<0>{}, d);

    if constexpr (PARTIAL) {
      // A K-chunk of a split tile: its float32 partial sums, as each lane
      // holds them, for k_fp8_splitk_reduce: [sp][wave][i][j][q] x 64 lanes
      // x 4 floats.
      f32x4* const pw = (f32x4*)g.ws + (int64_t)(sp * kWaves + wv) * 64 * 64 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 p4 = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            pw[((i * 4 + j) * 4 + q) * 64] = p4;
          }
    } else {
    // Epilogue of tile (m0, n0): out = R(R(acc * sc) + R(bias)). Eight
    // passes p = 2j + h (block row j, column half h) through the wave's
    // staging quarter of A buffer s - 1 (the tile's last slab): R(acc * sc)
    // is staged as bf16, read back as 16-byte row pieces, the bias added,
    // and stored. The passes overlap: pass p packs its values while the
    // reads of pass p - 1 are in flight, and finishes pass p - 1 (bias and
    // stores) while its own writes are.
    const uint32_t stg = lds0 + abuf(s - 1) + wv * (kSlabBytes / kWaves);
    const float sc = pick(scg, gi);
    // The stores of block row j go through a buffer resource over its 32
    // rows inside the matrix (none for a block past N), which drops rows
    // past M. Lane l stores row 4u + srow, columns h*64 + (lane%8)*8: the
    // row in the lane offset, h*128 bytes as the scalar offset (a lane's 16
    // bytes end inside its row, so the range check sees the row whether or
    // not it counts the scalar offset).
    const bool col_ok = nc0 + wn * 128 < g.group_n;
    const int rows_left = g.m - (m0 + wm * 128);
    uint16_t* const oblk = pick(g.outg, gi) + (int64_t)(m0 + wm * 128) * g.ldo + nc0 + wn * 128;
    const int olane = (srow * (int)g.ldo + (lane & 7) * 8) * 2;
    const int orow4 = 8 * (int)g.ldo;  // bytes of 4 rows
    uint2 pk[2][4];
    u32x4 ov[4];
    auto pack = [&](auto p_c) {
      constexpr int J = decltype(p_c)::value / 2, H = decltype(p_c)::value % 2;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16& a = acc[2 * H + ii][J];
          pk[ii][q].x = pack_out<O16>(acc_read(a[q * 4 + 0]) * sc, acc_read(a[q * 4 + 1]) * sc);
          pk[ii][q].y = pack_out<O16>(acc_read(a[q * 4 + 2]) * sc, acc_read(a[q * 4 + 3]) * sc);
        }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto write = [&]() {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          asm volatile("ds_write_b64 %0, %1 offset:%2" ::"v"(stg + sw), "v"(pk[ii][q]), "i"(ii * 64 + q * 16)
                       : "memory");
    };
    auto read = [&]() {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(ov[u]) : "v"(stg + sr), "i"(u * 4 * kStagePitch));
    };
    auto finish = [&](auto p_c) {
      constexpr int J = decltype(p_c)::value / 2, H = decltype(p_c)::value % 2;
      const int rows_j = col_ok ? min(max(rows_left - 32 * J, 0), 32) : 0;
      const i32x4 ro = resource(oblk + (int64_t)32 * J * g.ldo, (uint32_t)(rows_j * 2 * g.ldo));
      const u32x4 bw = bq[H];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = pack_out<O16>(out_lo<O16>(ov[u][e]) + out_lo<O16>(bw[e]),
                               out_hi<O16>(ov[u][e]) + out_hi<O16>(bw[e]));
        buffer_store_x4(y, ro, olane + u * orow4, H * 128, kStoreNT);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto next = [&](auto p_c) {  // pass p >= 1
      constexpr int P = decltype(p_c)::value;
      pack(IC<P>{});
      OGA_LGKM_WAIT(0, "+v"(ov[0]), "+v"(ov[1]), "+v"(ov[2]), "+v"(ov[3]));  // reads of p - 1
      write();
      finish(IC<P - 1>{});
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // writes of p
      read();
    };
    pack(IC<0>{});
    write();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    read();
    next(IC<1>{});
    next(IC<2>{});
    next(IC<3>{});
    next(IC<4>{});
    next(IC<5>{});
    next(IC<6>{});
    next(IC<7>{});
    OGA_LGKM_WAIT(0, "+v"(ov[0]), "+v"(ov[1]), "+v"(ov[2]), "+v"(ov[3]));
    finish(IC<7>{});
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
    v = vn;
    m0 = nm0;
    n0 = nn0;
    kb = nkb;
    kn = nkn;
    sp = nsp;
    ra = nra;
    rw = nrw;
  }
  OGA_WAIT_VM(0);  // the re-reads sent during the last tile
}


// Sum of the K-chunk partials of the split tiles, in chunk order, then the
// epilogue of k_fp8_gemm_ring: out = R(R(sum * sa * sb) + R(bias)). One
// workgroup per (split tile, wave quarter): the quarter's 4096 float4s of a
// chunk are the accumulators of one wave of the GEMM, float4 f = (block b =
// (i * 4 + j) * 4 + q, lane) holding row 32j + lane%32, columns 32i + 8q +
// 4(lane/32) + 0..3 of the quarter's 128 x 128 outputs. Thread t sums float4s
// t, t + 256, ... of every chunk (whole 4 KiB per wave and load), rounds
// R(sum * s) to bf16 and stages it in LDS in row order; after the barrier each
// thread reads 16-byte pieces of rows, adds R(bias) and stores them, so every
// wave's store covers four whole 256-byte row pieces.
constexpr int kReduceRow = 264;  // bytes per staged row of 128 bf16 (+8: the 32 rows of a write hit 64 banks)
constexpr bool reduce_writes_conflict_free() {
  // a half-wave (32 lanes, one lane%32 each: rows 32j + 0..31 at one column
  // pair) writes 8 bytes per lane: 64 distinct banks
  for (int half = 0; half < 2; ++half) {
    unsigned long long banks = 0;
    for (int fr = 0; fr < 32; ++fr) {
      const int bk = ((fr * kReduceRow + half * 8) >> 2) & 63;
      if ((banks >> bk) & 3ull) return false;
      banks |= 3ull << bk;
    }
  }
  return true;
}
static_assert(reduce_writes_conflict_free(), "reduce staging writes would conflict");
template <bool O16>
__global__ __launch_bounds__(256) void k_fp8_splitk_reduce(GemmArgs g) {
  constexpr int kPerTile = kWaves * 64 * 64;  // float4s per tile chunk
  constexpr int kPerWave = 64 * 64;            // float4s of one wave's accumulators
  __shared__ __attribute__((aligned(16))) uint8_t stage[128 * kReduceRow];
  const int x = blockIdx.x >> 2, wv = blockIdx.x & 3;
  const int wm = wv >> 1, wn = wv & 1;
  const int tid = threadIdx.x;
  const int t = g.nfull + x;
  const int per_group = kGroupM * g.tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * kGroupM;
  const int gsize = min(g.tiles_m - first_m, kGroupM);
  const int n0 = ((t % per_group) / gsize) * GN;
  const int gi = n0 / g.group_n;  // the tile's group (uniform per workgroup)
  const int row0 = (first_m + (t % per_group) % gsize) * GM + wm * 128;
  const int col0 = n0 - gi * g.group_n + wn * 128;  // inside the group
  const float sc = g.sa[0] * pick(g.sbg, gi)[0];
  // R(bias) of the 8 columns this thread stores (the same in every pass
  // below), loaded once, first (without a bias, -0.0, which an add leaves
  // every value as it is).
  const uint16_t* const bias = (const uint16_t*)pick(g.biasg, gi);
  const int c8 = tid & 15;
  const uint4 bw = *(const uint4*)(bias ? bias + min(col0 + 8 * c8, g.group_n - 8) : kNegZeroRow + 8 * c8);
  const f32x4* const p = (const f32x4*)g.ws + (int64_t)x * g.split * kPerTile + wv * kPerWave;
  f32x4 sum[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) sum[k] = p[tid + 256 * k];
  for (int c = 1; c < g.split; ++c) {
    f32x4 v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = p[(int64_t)c * kPerTile + tid + 256 * k];
#pragma unroll
    for (int k = 0; k < 16; ++k) sum[k] += v[k];
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int f = tid + 256 * k;
    const int b = f >> 6, lane = f & 63;
    const int i = b >> 4, j = (b >> 2) & 3, q = b & 3;
    const int r = 32 * j + (lane & 31);
    const int cc = 32 * i + 8 * q + 4 * (lane >> 5);
    uint2 pk;
    pk.x = pack_out<O16>(sum[k][0] * sc, sum[k][1] * sc);
    pk.y = pack_out<O16>(sum[k][2] * sc, sum[k][3] * sc);
    *(uint2*)(stage + r * kReduceRow + cc * 2) = pk;
  }
  __syncthreads();
  uint16_t* const out = pick(g.outg, gi);
  const uint32_t bb[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int r = (tid + 256 * k) >> 4;
    const int row = row0 + r, col = col0 + 8 * c8;
    if (row >= g.m || col >= g.group_n) continue;
    const uint2 lo = *(const uint2*)(stage + r * kReduceRow + c8 * 16);
    const uint2 hi = *(const uint2*)(stage + r * kReduceRow + c8 * 16 + 8);
    const uint32_t w[4] = {lo.x, lo.y, hi.x, hi.y};
    uint32_t y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)  // 16-bit pairs: the low half is the lower column
      y[e] = pack_out<O16>(out_lo<O16>(w[e]) + out_lo<O16>(bb[e]), out_hi<O16>(w[e]) + out_hi<O16>(bb[e]));
    *(uint4*)(out + (int64_t)row * g.ldo + col) = make_uint4(y[0], y[1], y[2], y[3]);
  }
}

}  // namespace oga

using namespace oga;

namespace {

// Split-K plan of the persistent kernel for tiles that do not fill a last
// round: with R >= 0 whole rounds over the CUs and r < CUs tiles left, each
// of the r tiles may be cut into S K-chunks (a power of two with r * S <= CUs
// and at least two slabs per chunk). The chunks run at once, so the round
// they form takes about nslab / S slab-times, and their float32 partials
// (r * S tiles of 256 KiB, written and read back by the reduce) cost about
// r * S / 15 slab-times at the device's bandwidth (a 256x256x128 slab takes
// ~1.56 us on one CU; a tile's partial round trip, 512 KiB at ~5 TB/s,
// ~0.1 us), plus ~2 slab-times for the two extra launches. S minimises that
// sum; S = 1: no split. With R = 0 (fewer tiles than CUs: the text
// projections of 256 context tokens make 16) the split spreads the tiles'
// K over the idle CUs.
struct SplitPlan {
  int nfull, split, kchunk, units;
  int64_t ws_bytes;
};
SplitPlan split_plan(int64_t m, int64_t n, int64_t k, int64_t cus) {
  const int64_t nt = ((m + GM - 1) / GM) * ((n + GN - 1) / GN);
  const int64_t nslab = k / GKS;
  SplitPlan p{(int)nt, 1, (int)nslab, (int)nt, 0};
  const int64_t rounds = nt / cus, rest = nt % cus;
  if (rest == 0) return p;
  // costs in fifteenths of a slab-time
  int64_t best = 15 * nslab;
  int sp = 1;
  for (int s = 2; rest * s <= cus && nslab % s == 0 && nslab / s >= 2; s *= 2) {
    const int64_t c = 15 * nslab / s + rest * s + 30;
    if (c < best) { best = c; sp = s; }
  }
  if (sp == 1) return p;
  p.nfull = (int)(rounds * cus);
  p.split = sp;
  p.kchunk = (int)(nslab / sp);
  p.units = (int)(p.nfull + rest * sp);
  p.ws_bytes = rest * sp * (int64_t)GM * GN * 4;
  return p;
}

// The persistent kernel and the reduce read the bias as 16-byte pieces of
// 16-bit values in the output dtype.
bool bias_ok(const void* bias, int bias_dtype, int out_dtype = OGA_DT_BF16) {
  return !bias || (bias_dtype == out_dtype && aligned(bias, 16));
}

// Common argument checks of the FP8 linear entry points (n: all columns).
int check_args(const void* a, int64_t lda, int64_t ldw, const float* scale_a, int64_t ldo, int64_t m, int64_t n,
               int64_t k, const void* workspace, int64_t workspace_bytes) {
  if (!a || !scale_a) return fail("null pointer");
  if (m < 0 || n < 0 || k < 0 || workspace_bytes < 0) return fail("bad shape");
  if (k == 0 || k % GKS) return unsupported("K must be a positive multiple of %d (got %lld)", GKS, (long long)k);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return unsupported("dimension too large");
  if (lda < k || ldw < k) return fail("leading dimension smaller than the row");
  if (!aligned(a, 16) || lda % 16 || ldw % 16) return fail("a/w rows must be 16-byte aligned");
  if (ldo % 8) return fail("out rows must be 16-byte aligned");
  // Per-lane byte offsets inside one 256-row tile (plus K) are 32-bit.
  if (256 * lda + k > (int64_t)UINT32_MAX || 256 * ldw + k > (int64_t)UINT32_MAX)
    return unsupported("row stride too large");
  if (workspace && !aligned(workspace, 16)) return fail("workspace must be 16-byte aligned");
  const int64_t nt = ((m + GM - 1) / GM) * ((n + GN - 1) / GN);
  if (nt > INT32_MAX / 16) return unsupported("too many tiles");
  return OGA_OK;
}

// The persistent schedule: whole tiles, then (split, workspace given) the
// K-chunks of the rest and their sums. g has its shape, operands and groups.
int launch_ring(GemmArgs& g, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  const int64_t cus = cu_count();
  SplitPlan p = split_plan(g.m, (int64_t)g.tiles_n * GN, g.k, cus);
  if (p.split > 1 && (!workspace || workspace_bytes < p.ws_bytes)) p = SplitPlan{(int)nt, 1, g.k / GKS, (int)nt, 0};
  g.nfull = p.nfull;
  g.split = p.split;
  g.kchunk = p.kchunk;
  g.ws = (float*)workspace;
  g.units = p.nfull;
  int64_t grid = g.units < cus ? g.units : cus;
  g.xcd_remap = (g.units % 8) == 0 && (grid % 8) == 0;
  if (grid > 0) {  // none when every tile is split (fewer tiles than CUs)
    if (g.out_f16)
      hipLaunchKernelGGL((k_fp8_gemm_ring<false, true>), dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, g);
    else
      hipLaunchKernelGGL((k_fp8_gemm_ring<false, false>), dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, g);
  }
  if (p.split > 1) {
    g.units = p.units - p.nfull;
    grid = g.units < cus ? g.units : cus;
    g.xcd_remap = (g.units % 8) == 0 && (grid % 8) == 0;
    // the K-chunks write float32 partials (no epilogue: one instance)
    hipLaunchKernelGGL((k_fp8_gemm_ring<true, false>), dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, g);
    if (g.out_f16)
      hipLaunchKernelGGL(k_fp8_splitk_reduce<true>, dim3((unsigned)((nt - p.nfull) * kWaves)), dim3(256), 0, stream,
                         g);
    else
      hipLaunchKernelGGL(k_fp8_splitk_reduce<false>, dim3((unsigned)((nt - p.nfull) * kWaves)), dim3(256), 0, stream,
                         g);
  }
  return launch_status();
}

void set_shape(GemmArgs& g, const void* a, int64_t lda, int64_t ldw, const float* scale_a, int64_t ldo, int64_t m,
               int64_t n, int64_t k) {
  g.a = (const uint8_t*)a;
  g.sa = scale_a;
  g.lda = lda;
  g.ldw = ldw;
  g.ldo = ldo;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.tiles_m = (int)((m + GM - 1) / GM);
  g.tiles_n = (int)((n + GN - 1) / GN);
}

}  // namespace

extern "C" int64_t oga_fp8_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % GKS || n % 128 || k < 2 * GKS) return 0;
  return split_plan(m, n, k, cu_count()).ws_bytes;
}

extern "C" int oga_fp8_linear_dt_ws(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                                    const float* scale_b, const void* bias, int bias_dtype, void* out, int out_dtype,
                                    int64_t ldo, int64_t m, int64_t n, int64_t k, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  if (!w || !scale_b || !out) return fail("null pointer");
  if (out_dtype != OGA_DT_BF16 && out_dtype != OGA_DT_F16) return unsupported("output dtype must be bf16 or fp16");
  if (const int rc = check_args(a, lda, ldw, scale_a, ldo, m, n, k, workspace, workspace_bytes)) return rc;
  if (m == 0 || n == 0) return OGA_OK;
  if (ldo < n) return fail("leading dimension smaller than the row");
  if (!aligned(w, 16)) return fail("a/w rows must be 16-byte aligned");
  if (!aligned(out, 16)) return fail("out rows must be 16-byte aligned");
  if (out_dtype == OGA_DT_F16 && bias && bias_dtype != OGA_DT_F16)
    return fail("an fp16 output takes an fp16 bias (bias.to(fp16))");
  if (out_dtype == OGA_DT_BF16 && bias && !dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  GemmArgs g{};
  set_shape(g, a, lda, ldw, scale_a, ldo, m, n, k);
  g.w = (const uint8_t*)w;
  g.sb = scale_b;
  g.bias = bias;
  g.bias_dt = bias_dtype;
  g.out = (uint16_t*)out;
  g.out_f16 = out_dtype == OGA_DT_F16;
  // The persistent kernel needs two slabs per tile, whole 128-column wave
  // blocks and no bias or a 16-byte aligned bf16 bias; other shapes take one
  // workgroup per tile.
  if (k >= 2 * GKS && n % 128 == 0 && bias_ok(bias, bias_dtype, out_dtype)) {
    for (int i = 0; i < kMaxGroups; ++i) {  // one group; the others repeat it
      g.wg[i] = g.w;
      g.sbg[i] = g.sb;
      g.biasg[i] = g.bias;
      g.outg[i] = g.out;
    }
    g.group_n = g.n;
    return launch_ring(g, workspace, workspace_bytes, (hipStream_t)stream);
  }
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  g.xcd_remap = (nt % 8) == 0;
  if (g.out_f16)
    hipLaunchKernelGGL(k_fp8_gemm<true>, dim3((unsigned)nt), dim3(64 * kWaves), 0, (hipStream_t)stream, g);
  else
    hipLaunchKernelGGL(k_fp8_gemm<false>, dim3((unsigned)nt), dim3(64 * kWaves), 0, (hipStream_t)stream, g);
  return launch_status();
}

extern "C" int oga_fp8_linear_ws(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                                 const float* scale_b, const void* bias, int bias_dtype, void* out, int64_t ldo,
                                 int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  return oga_fp8_linear_dt_ws(a, lda, w, ldw, scale_a, scale_b, bias, bias_dtype, out, OGA_DT_BF16, ldo, m, n, k,
                              workspace, workspace_bytes, stream);
}

extern "C" int oga_fp8_linear(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                              const float* scale_b, const void* bias, int bias_dtype, void* out, int64_t ldo,
                              int64_t m, int64_t n, int64_t k, void* stream) {
  return oga_fp8_linear_ws(a, lda, w, ldw, scale_a, scale_b, bias, bias_dtype, out, ldo, m, n, k, nullptr, 0, stream);
}

extern "C" int oga_fp8_linear_grouped_ws(const void* a, int64_t lda, const void* const* w, int64_t ldw,
                                         const float* scale_a, const float* const* scale_b,
                                         const void* const* bias, int bias_dtype, void* const* out, int64_t ldo,
                                         int64_t m, int64_t n_group, int64_t groups, int64_t k, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  if (!w || !scale_b || !bias || !out) return fail("null pointer");
  if (groups < 1 || groups > kMaxGroups) return unsupported("1 to %d groups (got %lld)", kMaxGroups, (long long)groups);
  if (n_group <= 0 || (groups > 1 && n_group % GN)) return unsupported("group width must be a multiple of %d", GN);
  if (const int rc = check_args(a, lda, ldw, scale_a, ldo, m, n_group * groups, k, workspace, workspace_bytes))
    return rc;
  if (m == 0) return OGA_OK;
  if (ldo < n_group) return fail("leading dimension smaller than the row");
  if (k < 2 * GKS || n_group % 128) return unsupported("grouped FP8 linear needs K >= %d and N %% 128 == 0", 2 * GKS);
  GemmArgs g{};
  set_shape(g, a, lda, ldw, scale_a, ldo, m, n_group * groups, k);
  g.group_n = (int)n_group;
  for (int i = 0; i < kMaxGroups; ++i) {
    const int j = i < groups ? i : 0;  // unused entries repeat group 0
    if (!w[j] || !scale_b[j] || !out[j]) return fail("null pointer");
    if (!aligned(w[j], 16) || !aligned(out[j], 16)) return fail("a/w rows and out must be 16-byte aligned");
    if (!bias_ok(bias[j], bias_dtype)) return unsupported("grouped FP8 linear takes no bias or a 16-byte aligned bf16 bias");
    g.wg[i] = (const uint8_t*)w[j];
    g.sbg[i] = scale_b[j];
    g.biasg[i] = bias[j];
    g.outg[i] = (uint16_t*)out[j];
  }
  g.w = g.wg[0];
  g.sb = g.sbg[0];
  g.bias = g.biasg[0];
  g.bias_dt = bias_dtype;
  g.out = g.outg[0];
  return launch_ring(g, workspace, workspace_bytes, (hipStream_t)stream);
}
