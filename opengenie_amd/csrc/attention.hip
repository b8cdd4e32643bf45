// Dense non-causal self-attention (bf16 in/out, float32 softmax and
// accumulation) for head_dim 128 on gfx950 MFMA.
//
// Reference: the video self-attention of the LTX block, which opengenie runs
// through FlashAttention-3's flash_attn_func(q, k, v) on [B, N, H, D] views
// (benchmarks/official_ltx23_benchmark.py:3294-3369; FlashAttention3.__call__
// of ltx_core), with softmax scale D^-0.5:
//   O[b, n, h] = sum_m softmax_m(q[b,n,h] . k[b,m,h] * scale) v[b,m,h].
// FP8 inputs (e4m3 with per-(b, h) descales, :3330-3340) run k_attention_fp8
// below, both products on e4m3 MFMA as FlashAttention-3's FP8 path does (the
// reference benchmark checks the FP8 result against the bf16 one within a
// tolerance, video_self_attention_bench.py:288-305, and so do the tests
// here); oga_fp8_dequant_per_head (each value times its float32 descale,
// rounded to bf16) serves e4m3 inputs that kernel does not take.
//
// Work decomposition. A workgroup of kAW waves (8) owns 32 kAW queries of one
// (b, h); wave w owns queries 32w .. 32w+31. Keys are visited 64 at a time;
// the K and V tiles of a step (64 x 128 bf16 each) are copied to LDS by DMA
// (global_load_lds_dwordx4) into a ring of kABufs (3) tile pairs, two steps
// in flight. For few keys (<= kShortSteps steps) the same kernel runs with 4
// waves and two pairs, two workgroups per CU.
//
// Per step and wave, with v_mfma_f32_32x32x16_bf16:
//  * S^T = K Q^T as two 32-key x 32-query blocks (8 MFMAs each over d):
//    operand A = K rows from LDS, operand B = the wave's Q^T fragments, kept
//    in registers for the whole key loop. Lane l then holds 16 scores of
//    query l % 32 per block (keys 8g + 4(l/32) + r for accumulator 4g + r),
//    so a query's max and sum need one exchange with lane l ^ 32.
//  * online softmax in base 2 (the scale folded with log2 e) with lazy
//    rescaling of O (only when a running max grows by more than 2^8), P
//    rounded to bf16 as FlashAttention does before the P.V product.
//  * O^T = V^T P^T as four 32-d x 32-query blocks over four 16-key chunks:
//    operand B = P^T straight from the score accumulators, operand A = V^T
//    read with ds_read_b64_tr_b16 (transposing reads) from the row-major V
//    tile. The k-slot order of both operands is the same permutation of the
//    16 keys of a chunk, so they pair up without moving P between lanes.
// LDS tiles: key row r (256 bytes = 16 chunks of 16 B) keeps chunk c at
// physical chunk c ^ swz(r % 16), so both the 32-row fragment reads and the
// transposing reads are free of bank conflicts.
#include <atomic>

#include "common.h"
#include "host.h"

namespace oga {

#ifndef OGA_ATT_WAVES
#define OGA_ATT_WAVES 8
#endif
#ifndef OGA_ATT_BUFS
#define OGA_ATT_BUFS 3
#endif
constexpr int kAD = 128;                   // head dim
constexpr int kAW = OGA_ATT_WAVES;         // waves per workgroup, 32 queries each
constexpr int kAQ = 32 * kAW;              // queries per workgroup
constexpr int kAK = 64;                    // keys per step
constexpr int kABufs = OGA_ATT_BUFS;       // K/V tile pairs in the LDS ring
static_assert(kAW == 4 || kAW == 8, "4 or 8 waves");
static_assert(kABufs == 2 || kABufs == 3, "2 or 3 tile pairs");
// Few keys (at most kShortSteps steps, the text cross-attention's 256): the
// per-workgroup Q loads and O stores are then a large part of the time, so
// the bf16 kernel runs with 4 waves and two tile pairs (64 KiB of LDS, one
// wave per SIMD), two workgroups per CU, one's loads and stores under the
// other's MFMAs; and no key split (its merge costs more than the shorter
// last round gains).
constexpr int kAWShort = 4, kABufsShort = 2, kShortSteps = 16;
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
  int nqb;        // query blocks per (batch, head)
  int qpb;        // queries per block (kAQ, or kF8Q for the FP8 kernel)
  int xcd_remap;  // nfull divisible by the 8 XCDs
  float scale_log2;  // softmax scale * log2(e)
  // Workgroups 0 .. nfull-1 each own query block blockIdx.x (remapped) over
  // all keys. The blocks nfull .. end, which would fill only part of a last
  // round of the CUs, are cut into ksplit parts over their key steps: later
  // workgroup nfull + u owns part u % ksplit of block nfull + u / ksplit and
  // leaves its unnormalized O (part_o, [u][qpb][kAD] float32) and its
  // running max and sum (part_ml, [u][qpb][2]) for k_attention_combine.
  int64_t nfull;
  int ksplit;
  float* part_o;
  float* part_ml;
  // FP8 kernel only: V rewritten as [B, H, D, vt_npad] (k_fp8_v_transpose)
  // and the [B, H] descales of q, k and v.
  const uint8_t* vt;
  int64_t vt_npad;
  const float* q_ds;
  const float* k_ds;
  const float* v_ds;
  // bf16 kernel and its merge: with oq set, the output goes to oq as the
  // e4m3 codes of the FP8 linear that reads it, e4m3(clamp(R(o) * r, +-448))
  // (o's strides, one byte per element; r = 1/scale in float32, and with
  // oq_bf16, for a 0-dim scale, r and the product rounded to bf16: the
  // input quantizer of that linear), instead of the bf16 o.
  uint8_t* oq;
  const float* oq_scale;
  int oq_bf16;
};

// 8 bf16 output values (one 16-byte piece) as the e4m3 codes the input
// quantizer of the following FP8 linear writes for them (rows.hip's Q8 path
// and k_fp8_quant compute the same expression).
OGA_DEVICE uint2 e4m3_of_bf16x8(const uint4& w, float r, bool rb) {
  float f[8];
  unpack8(w, f);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v = f[i] * r;
    if (rb) v = rbf(v);
    f[i] = clamp448(v);
  }
  return make_uint2(e4m3x4(f[0], f[1], f[2], f[3]), e4m3x4(f[4], f[5], f[6], f[7]));
}
OGA_DEVICE float e4m3_recip(const AttnArgs& a) {
  const float r = 1.0f / a.oq_scale[0];
  return a.oq_bf16 ? rbf(r) : r;
}

OGA_DEVICE f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Swizzle of key row r's 16 chunks: chunk c sits at physical chunk c ^ swz(r).
// swz is a bijection on r % 16 (so the 16 rows a K fragment read takes
// together hit 16 different 16-byte bank groups) whose bits 2-3 take four
// different values over any four consecutive rows (so the 4 rows x 64 bytes
// that 32 lanes of a transposing V read take together cover all 64 banks).
constexpr int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
// Byte offset of (key row r, element d) in a swizzled LDS tile.
constexpr int tile_off(int r, int d) { return r * 256 + ((((d >> 3) ^ swz(r & 15)) << 4) | ((d & 7) << 1)); }

// The kernel folds tile_off into per-lane bases plus immediate offsets:
//  K fragment of lane (ql, hl), d-step s, key block j:
//    j*8192 + ql*256 + ((2s ^ hl ^ swz(ql % 16)) << 4);
//  V^T transposing read of lane (a4, j4, g2, hl), chunk c2, half u, d-block dblk:
//    c2*4096 + u*2048 + (4hl + j4)*256
//      + ((4 (dblk ^ j4) + ((2g2 + a4/2) ^ (2u + hl))) << 4) + 8 (a4 & 1).
// Checked here for every lane and step.
constexpr int v_fold(int lane, int u, int dblk) {
  const int a4 = lane & 3, j4 = (lane & 15) >> 2, g2 = (lane >> 4) & 1, hl = lane >> 5;
  return u * 2048 + (4 * hl + j4) * 256 + ((4 * (dblk ^ j4) + ((2 * g2 + (a4 >> 1)) ^ (2 * u + hl))) << 4) +
         (a4 & 1) * 8;
}
constexpr bool folded_offsets_match() {
  for (int lane = 0; lane < 64; ++lane) {
    const int hl = lane >> 5, ql = lane & 31;
    for (int j = 0; j < 2; ++j)
      for (int s = 0; s < 8; ++s)
        if (tile_off(32 * j + ql, 16 * s + 8 * hl) != j * 8192 + ql * 256 + (((2 * s) ^ hl ^ swz(ql & 15)) << 4))
          return false;
    const int a4 = lane & 3, j4 = (lane & 15) >> 2, g2 = (lane >> 4) & 1;
    for (int c2 = 0; c2 < 4; ++c2)
      for (int u = 0; u < 2; ++u)
        for (int dblk = 0; dblk < 4; ++dblk) {
          const int want = tile_off(16 * c2 + 8 * u + 4 * hl + j4, 32 * dblk + 16 * g2 + 4 * a4);
          if (want != c2 * 4096 + v_fold(lane, u, dblk)) return false;
        }
  }
  return true;
}
// Bank check: the 32 lanes of a transposing read (one half, fixed chunk c2,
// half u, d-block) read 32 distinct 8-byte pieces covering all 64 banks.
constexpr bool v_reads_conflict_free() {
  for (int half = 0; half < 2; ++half)
    for (int u = 0; u < 2; ++u)
      for (int dblk = 0; dblk < 4; ++dblk) {
        unsigned long long banks = 0;
        for (int l = 32 * half; l < 32 * half + 32; ++l) {
          const int b = (v_fold(l, u, dblk) >> 2) & 63;
          banks |= 3ull << b;
        }
        if (banks != ~0ull) return false;
      }
  return true;
}
static_assert(v_reads_conflict_free(), "transposing V reads would conflict");
static_assert(folded_offsets_match(), "folded LDS offsets differ from tile_off");

// DMA of one 64-key tile of K or V (bf16 rows of kAD elements) into LDS by
// a workgroup of 16 / DI waves: instruction i of wave w fills tile rows
// 4b .. 4b+3 (b = DI w + i); lane p writes the 16 bytes at row 4b + p/16,
// physical chunk p%16, i.e. logical chunk (p%16) ^ swz(row%16). `off[i]` is
// that source's byte offset from the tile's first key row; in the last,
// partial step rows past the last key re-read the last key.
template <int DI>
struct TileSrc {
  uint32_t off[DI];
};
template <int DI>
OGA_DEVICE TileSrc<DI> tile_src(int64_t row_stride, int64_t first_key, int64_t nk, int wv, int lane, bool clamp) {
  TileSrc<DI> t;
#pragma unroll
  for (int i = 0; i < DI; ++i) {
    const int row = (wv * DI + i) * 4 + (lane >> 4);
    const int chunk = (lane & 15) ^ swz(row & 15);
    const int64_t r = clamp ? min((int64_t)row, nk - 1 - first_key) : (int64_t)row;
    t.off[i] = (uint32_t)(r * row_stride * 2 + chunk * 16);
  }
  return t;
}
template <int DI>
OGA_DEVICE void tile_dma(const char* tile_base, const TileSrc<DI>& t, uint4* dst, int wv) {
#pragma unroll
  for (int i = 0; i < DI; ++i)
    __builtin_amdgcn_global_load_lds((const void*)(tile_base + t.off[i]),
                                     (lds_void*)(dst + (wv * DI + i) * 64), 16, 0, 0);
}

OGA_DEVICE uint32_t pack2(float a, float b) { return pack_bf16(a, b); }

// LDS reads issued as inline assembly with immediate offsets, so that groups
// of them stay in flight together and need no address arithmetic;
// OGA_LGKM names the registers a wait makes valid. The offset field holds
// 16 bits: reads at 64 KiB and above (the third tile pair) move 64 KiB into
// the address.
template <int OFF>
OGA_DEVICE bf16x8 lds_b128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 2 * 65536, "LDS offset");
  uint4 v;
  if constexpr (OFF >= 65536)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr + 65536u), "i"(OFF - 65536));
  else
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return __builtin_bit_cast(bf16x8, v);
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
template <int OFF>
OGA_DEVICE u32x2 lds_tr16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 2 * 65536, "LDS offset");
  u32x2 v;
  if constexpr (OFF >= 65536)
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr + 65536u), "i"(OFF - 65536));
  else
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
#define OGA_LGKM(N, ...) asm volatile("s_waitcnt lgkmcnt(" #N ")" : __VA_ARGS__)

// max / sum of a value over lanes l and l ^ 32 (v_permlane32_swap).
OGA_DEVICE float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
OGA_DEVICE float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


// LDS: [K0 | V0 | K1 | V1 (| K2 | V2)], 16 KiB each; step st uses tile pair
// st % BUFS, and the DMA of step st + BUFS - 1 goes out during step st.
constexpr int kKBuf = 0, kVBuf = 16384, kParBytes = 32768;

// W waves (4 or 8) of 32 queries, BUFS (2 or 3) K/V tile pairs in the ring.
template <int W, int BUFS>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_attention(AttnArgs a) {
  static_assert(W == 4 || W == 8, "4 or 8 waves");
  static_assert(BUFS == 2 || BUFS == 3, "2 or 3 tile pairs");
  constexpr int kBfBufs = BUFS;
  constexpr int kQB = 32 * W;   // queries per workgroup
  constexpr int kDI = 16 / W;   // DMA instructions per wave per tile
  static_assert(2 * kBfBufs * kATileU4 * 16 <= 160 * 1024, "LDS budget");
  static_assert(W * 8192 <= 2 * kBfBufs * kATileU4 * 16, "the output staging fits the ring");
  __shared__ uint4 smem[2 * kBfBufs * kATileU4];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Workgroups go to the 8 XCDs round-robin. With the remap, XCD x runs a
  // contiguous range of (b, h, query block) triples, query block fastest, so
  // all query blocks of a head run together on one XCD and read that head's
  // K/V tiles through one L2.
  int64_t wg = blockIdx.x;
  int part = -1;  // -1: all key steps
  if (wg < a.nfull) {
    if (a.xcd_remap) wg = (wg & 7) * (a.nfull >> 3) + (wg >> 3);
  } else {
    const int64_t u = wg - a.nfull;
    wg = a.nfull + u / a.ksplit;
    part = (int)(u % a.ksplit);
  }
  const int qb = (int)(wg % a.nqb);
  const int64_t bh = wg / a.nqb;
  const int h = (int)(bh % a.heads);
  const int64_t b = bh / a.heads;
  const int64_t q0 = (int64_t)qb * kQB + wv * 32;
  const int hl = lane >> 5;  // lane half
  const int ql = lane & 31;
  // r of the e4m3 output (if any), read now: its load latency is then not
  // paid after the last step
  const float oq_r = a.oq ? e4m3_recip(a) : 0.0f;

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
  // Key steps st_begin .. st_end - 1 (at least one: ksplit <= all steps).
  const int64_t nsteps_all = (a.nk + kAK - 1) / kAK;
  const int64_t st_begin = part < 0 ? 0 : nsteps_all * part / a.ksplit;
  const int64_t st_end = part < 0 ? nsteps_all : nsteps_all * (part + 1) / a.ksplit;

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  // m_run: running max of the scaled (base-2) scores of query q0 + ql;
  // l_run: this lane's part of the running sum (keys of lane half hl).
  float m_run = -INFINITY, l_run = 0.0f;

  const TileSrc<kDI> ksrc = tile_src<kDI>(a.k_sn, 0, a.nk, wv, lane, false);
  const TileSrc<kDI> vsrc = tile_src<kDI>(a.v_sn, 0, a.nk, wv, lane, false);
  auto dma_step = [&](int64_t s2, uint4* dK, uint4* dV) {
    const int64_t key0 = s2 * kAK;
    const char* kt = (const char*)(kbase + key0 * a.k_sn);
    const char* vt = (const char*)(vbase + key0 * a.v_sn);
    if (key0 + kAK <= a.nk) {
      tile_dma(kt, ksrc, dK, wv);
      tile_dma(vt, vsrc, dV, wv);
    } else {
      tile_dma(kt, tile_src<kDI>(a.k_sn, key0, a.nk, wv, lane, true), dK, wv);
      tile_dma(vt, tile_src<kDI>(a.v_sn, key0, a.nk, wv, lane, true), dV, wv);
    }
  };
  // With three pairs the DMA runs two steps ahead; past the last step it
  // re-reads the last tile (an index past it would put rows outside K/V)
  // into a pair no later step reads, so that exactly one tile's DMA is sent
  // after each step's own.
  dma_step(st_begin, smem, smem + kATileU4);
  if (kBfBufs == 3) dma_step(min(st_begin + 1, st_end - 1), smem + 2 * kATileU4, smem + 3 * kATileU4);

  // LDS read addresses (tile_off with the swizzle folded per lane):
  //  K fragment (key row 32j + ql, d = 16s + 8hl): kaddr[s] + 8192 j;
  //  V^T read (key row 16c2 + 8u + 4hl + j4, d = 32dblk + 16g2 + 4a4):
  //  vaddr[dblk][u] + 4096 c2 + 2048 u.
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  uint32_t kaddr[8], vaddr[4][2];
  {
    const int x = hl ^ swz(ql & 15);
#pragma unroll
    for (int s = 0; s < 8; ++s) kaddr[s] = lds0 + ql * 256 + (((2 * s) ^ x) << 4);
    const int a4 = lane & 3, j4 = (lane & 15) >> 2, g2 = (lane >> 4) & 1;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        vaddr[dblk][u] = lds0 + kVBuf + (4 * hl + j4) * 256 +
                         ((4 * (dblk ^ j4) + ((2 * g2 + (a4 >> 1)) ^ (2 * u + hl))) << 4) + (a4 & 1) * 8;
  }
  // Key offset of accumulator e within a 32-key block, minus this lane's 4 hl.
  const int hl4 = 4 * hl;

  // S^T blocks of the step in pair PAR: key block j (keys 32j .. 32j+31) x
  // the wave's 32 queries.
  auto s_phase = [&](auto par_c, f32x16(&sacc)[2]) {
    constexpr int KB = decltype(par_c)::value * kParBytes + kKBuf;
    auto s_block = [&](auto j_c) {
      constexpr int OFF = KB + 8192 * decltype(j_c)::value;
      bf16x8 kf[8];
      kf[0] = lds_b128<OFF>(kaddr[0]);
      kf[1] = lds_b128<OFF>(kaddr[1]);
      kf[2] = lds_b128<OFF>(kaddr[2]);
      kf[3] = lds_b128<OFF>(kaddr[3]);
      kf[4] = lds_b128<OFF>(kaddr[4]);
      kf[5] = lds_b128<OFF>(kaddr[5]);
      kf[6] = lds_b128<OFF>(kaddr[6]);
      kf[7] = lds_b128<OFF>(kaddr[7]);
      OGA_LGKM(0, "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]),
               "+v"(kf[7]));
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma_bf16(kf[s], qf[s], acc);
      return acc;
    };
    sacc[0] = s_block(IC<0>{});
    sacc[1] = s_block(IC<1>{});
  };
  // V^T fragments of 16-key chunk C of pair PAR (4 d-blocks x 2 transposing
  // reads).
  auto read_v = [&](auto par_c, auto c_c, u32x2(&vr)[8]) {
    constexpr int C = decltype(c_c)::value;
    constexpr int OFF = decltype(par_c)::value * kParBytes + 4096 * C;  // vaddr includes kVBuf
    vr[0] = lds_tr16<OFF>(vaddr[0][0]);
    vr[1] = lds_tr16<OFF + 2048>(vaddr[0][1]);
    vr[2] = lds_tr16<OFF>(vaddr[1][0]);
    vr[3] = lds_tr16<OFF + 2048>(vaddr[1][1]);
    vr[4] = lds_tr16<OFF>(vaddr[2][0]);
    vr[5] = lds_tr16<OFF + 2048>(vaddr[2][1]);
    vr[6] = lds_tr16<OFF>(vaddr[3][0]);
    vr[7] = lds_tr16<OFF + 2048>(vaddr[3][1]);
  };
  // Online softmax of step st: keys past nk get score -inf; the running max
  // moves lazily (only when some query of the wave sees a score more than 8
  // above it, always on the first step), so P = 2^(s scale_log2 - m_run) <=
  // 256 and O, l are rescaled rarely. The float32 P feed l, their bf16
  // roundings the P.V product (as FlashAttention does).
  auto softmax = [&](int64_t st, f32x16(&sacc)[2], uint32_t(&pb)[2][8]) {
    const int64_t rem64 = a.nk - st * kAK;
    if (rem64 < kAK) {
      const int remh = (int)rem64 - hl4;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (32 * j + 8 * (e >> 2) + (e & 3) >= remh) sacc[j][e] = -INFINITY;
    }
    float mx = sacc[0][0];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = (j == 0 ? 1 : 0); e < 16; ++e) mx = __builtin_fmaxf(mx, sacc[j][e]);
    // Base-2 scores s * scale_log2 (scale_log2 > 0, so the max commutes).
    const float ms = max_halves(mx) * a.scale_log2;
    if (__any(ms > m_run + 8.0f)) {
      const float m_new = __builtin_fmaxf(m_run, ms);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first step (m_run = -inf)
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
    }
    const float nm = -m_run;
    float ps0, ps1;  // from the first terms (P >= 0 is never -0: 0 + x would be x)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e], a.scale_log2, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e + 1], a.scale_log2, nm));
        ps0 = (j == 0 && e == 0) ? p0 : ps0 + p0;
        ps1 = (j == 0 && e == 0) ? p1 : ps1 + p1;
        pb[j][e >> 1] = pack2(p0, p1);
      }
    l_run += ps0 + ps1;
  };
  // O^T += V^T P^T over the 16-key chunks c2 (keys 16 c2 .. 16 c2 + 15) of
  // pair PAR, chunk 0's V^T fragments already read into vr0; each next
  // chunk's reads go out before this chunk's MFMAs.
  auto pv_phase = [&](auto par_c, const uint32_t(&pb)[2][8], u32x2(&vr0)[8]) {
    u32x2 vr1[8];
    auto pv = [&](auto c_c, u32x2(&cur)[8], u32x2(&nxt)[8]) {
      constexpr int C = decltype(c_c)::value;
      if constexpr (C + 1 < 4) {
        read_v(par_c, IC<C + 1>{}, nxt);
        OGA_LGKM(8, "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]), "+v"(cur[5]),
                 "+v"(cur[6]), "+v"(cur[7]));
      } else {
        OGA_LGKM(0, "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]), "+v"(cur[5]),
                 "+v"(cur[6]), "+v"(cur[7]));
      }
      // B = P^T: accumulators 8(C % 2) .. +7 of block C / 2.
      const uint32_t* pw = &pb[C >> 1][4 * (C & 1)];
      const uint4 pu = {pw[0], pw[1], pw[2], pw[3]};
      const bf16x8 pf = __builtin_bit_cast(bf16x8, pu);
#pragma unroll
      for (int dblk = 0; dblk < 4; ++dblk) {
        const uint4 vu = {cur[2 * dblk][0], cur[2 * dblk][1], cur[2 * dblk + 1][0], cur[2 * dblk + 1][1]};
        o[dblk] = mfma_bf16(__builtin_bit_cast(bf16x8, vu), pf, o[dblk]);
      }
    };
    pv(IC<0>{}, vr0, vr1);
    pv(IC<1>{}, vr1, vr0);
    pv(IC<2>{}, vr0, vr1);
    pv(IC<3>{}, vr1, vr0);
  };
  // Wait until this wave's DMA of step st has landed (with three pairs, the
  // one DMA sent after it, of step st + 1, may stay in flight), join the
  // barrier (every wave's DMA of step st landed, every wave is past its last
  // read of the pair the next DMA fills) and send the DMA of step st + 2
  // (st + 1 with two pairs). The wait is explicit because the
  // barrier's workgroup fence does not wait for loads, and the LDS reads are
  // inline assembly the compiler does not order after the DMA; the barrier
  // is bare because __syncthreads()'s fence would add a vmcnt(0) (draining
  // the DMA sent ahead).
  auto bar_dma = [&](auto par_c, int64_t st) {
    constexpr int PAR = decltype(par_c)::value;
    if (kBfBufs == 3)
      asm volatile("s_waitcnt vmcnt(%0)" ::"i"(2 * kDI) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    constexpr int NP = (PAR + kBfBufs - 1) % kBfBufs;  // pair of step st + kBfBufs - 1
    if (kBfBufs == 3)
      dma_step(min(st + 2, st_end - 1), smem + 2 * NP * kATileU4, smem + (2 * NP + 1) * kATileU4);
    else if (st + 1 < st_end)
      dma_step(st + 1, smem + 2 * NP * kATileU4, smem + (2 * NP + 1) * kATileU4);
  };

  auto step = [&](auto par_c, int64_t st) {
    bar_dma(par_c, st);
    f32x16 sacc[2];
    uint32_t pb[2][8];
    u32x2 vr0[8];
    s_phase(par_c, sacc);
    read_v(par_c, IC<0>{}, vr0);  // in flight under the softmax
    softmax(st, sacc, pb);
    pv_phase(par_c, pb, vr0);
  };

  for (int64_t st = st_begin; st < st_end; st += kBfBufs) {
    step(IC<0>{}, st);
    if (st + 1 < st_end) step(IC<1>{}, st + 1);
    if constexpr (kBfBufs == 3)
      if (st + 2 < st_end) step(IC<2 % kBfBufs>{}, st + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-reads past the last step

  // O = O^T / l: lane holds query q0 + ql, d = 32 dblk + 8 (e/4) + 4 hl + e%4.
  // The wave's 32 x 128 tile goes through its own 8 KiB of LDS (free once
  // every wave has finished its last step) so that each global store writes
  // whole 256-byte query rows: stored straight from the registers, each row
  // took 16 partial-line stores, and the partly written lines reached HBM
  // more than once (up to 2.6x the output bytes at 8 waves per workgroup).
  // 16-byte chunk c of row r sits at chunk c ^ (r % 16) of the row.
  if (part >= 0) {
    // A part of a split block (every wave of the workgroup takes this
    // branch, so none waits at the barriers below): O^T rows unnormalized,
    // with m_run and the query's sum over this part's keys.
    const int64_t row = (int64_t)(blockIdx.x - a.nfull) * kQB + wv * 32 + ql;
    float* po = a.part_o + row * kAD;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(float4*)(po + 32 * dblk + 8 * g + 4 * hl) =
            make_float4(o[dblk][4 * g], o[dblk][4 * g + 1], o[dblk][4 * g + 2], o[dblk][4 * g + 3]);
    const float l_tot = sum_halves(l_run);
    if (hl == 0) *(float2*)(a.part_ml + 2 * row) = make_float2(m_run, l_tot);
    return;
  }
  const float inv = 1.0f / sum_halves(l_run);
  __syncthreads();
  char* const otile = (char*)smem + wv * 8192;
#pragma unroll
  for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack2(o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv);
      w.y = pack2(o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv);
      *(uint2*)(otile + ql * 256 + (((4 * dblk + g) ^ (ql & 15)) << 4) + 8 * hl) = w;
    }
  __syncthreads();
  const int oc = lane & 15;
  if (a.oq) {  // e4m3 codes of R(o) for the FP8 linear that reads it
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 4 * it + (lane >> 4);
      const uint4 w = *(const uint4*)(otile + r * 256 + ((oc ^ (r & 15)) << 4));
      const int64_t qr = q0 + r;
      if (qr < a.nq)
        *(uint2*)(a.oq + b * a.o_sb + qr * a.o_sn + (int64_t)h * a.o_sh + 8 * oc) = e4m3_of_bf16x8(w, oq_r, a.oq_bf16);
    }
    return;
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = 4 * it + (lane >> 4);
    const uint4 w = *(const uint4*)(otile + r * 256 + ((oc ^ (r & 15)) << 4));
    const int64_t qr = q0 + r;
    if (qr < a.nq) *(uint4*)(a.o + b * a.o_sb + qr * a.o_sn + (int64_t)h * a.o_sh + 8 * oc) = w;
  }
}

// ------------------------------------------------- few keys (text tokens)
// At most kFewKeys keys (the text cross-attention's 256): the whole K and V
// of a (batch, head) stay in LDS (4 tile pairs, 128 KiB, the swizzled layout
// of k_attention) for the workgroup's life. A workgroup of kFewW waves takes
// one (batch, head) and a range of its 32-query groups; after one barrier
// (K/V landed) each wave runs its groups on its own, with no further
// barrier: Q^T fragments from HBM, the key steps of k_attention against the
// resident tiles (S^T, online softmax, P.V), the output through the wave's
// own 4 KiB of staging in two 16-row passes. The two waves of a SIMD cover
// each other's Q loads and stores. (k_attention re-fetched K/V per block of
// queries and ran each block's Q loads, key steps and stores in lockstep
// across its workgroup, so the per-block fixed cost dominated at 4 steps.)
constexpr int kFewKeys = 256;                        // 4 steps of 64 keys
constexpr int kFewSteps = kFewKeys / kAK;
constexpr int kFewW = 8;                             // waves per workgroup (two per SIMD)
constexpr int kFewStage = kFewSteps * kParBytes;     // staging after the tiles: 128 KiB
constexpr int kFewStageWave = 4096;                  // 16 rows x 256 bytes
static_assert(kFewStage + kFewW * kFewStageWave <= 160 * 1024, "LDS budget");

__global__ __launch_bounds__(64 * kFewW) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_attention_fewkeys(
    AttnArgs a, int slices) {
  constexpr int kDI = 16 / kFewW;  // DMA instructions per wave per tile
  __shared__ uint4 smem[(kFewStage + kFewW * kFewStageWave) / 16];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int hl = lane >> 5, ql = lane & 31, hl4 = 4 * hl;
  // The eight XCDs receive workgroups round-robin (XCD = blockIdx.x % 8):
  // renumbered so that each XCD's workgroups are consecutive, the slices of a
  // head share one XCD and its L2 holds the head's K/V for all of them.
  const uint32_t xcd = blockIdx.x & 7, per = gridDim.x >> 3, extra = gridDim.x & 7;
  const int64_t wg = (int64_t)xcd * per + min(xcd, extra) + (blockIdx.x >> 3);
  const int64_t bh = wg / slices;
  const int slice = (int)(wg % slices);
  const int h = (int)(bh % a.heads);
  const int64_t b = bh / a.heads;
  const int64_t ngroups = (a.nq + 31) / 32;
  const int64_t g_begin = ngroups * slice / slices, g_end = ngroups * (slice + 1) / slices;
  const int nsteps = (int)((a.nk + kAK - 1) / kAK);  // 1 .. kFewSteps
  const float oq_r = a.oq ? e4m3_recip(a) : 0.0f;

  // K and V of the head into the tile pairs, once.
  const uint16_t* kbase = (const uint16_t*)a.k + b * a.k_sb + (int64_t)h * a.k_sh;
  const uint16_t* vbase = (const uint16_t*)a.v + b * a.v_sb + (int64_t)h * a.v_sh;
  for (int st = 0; st < nsteps; ++st) {
    const int64_t key0 = (int64_t)st * kAK;
    const bool clamp = key0 + kAK > a.nk;
    const TileSrc<kDI> ks = tile_src<kDI>(a.k_sn, key0, a.nk, wv, lane, clamp);
    const TileSrc<kDI> vs = tile_src<kDI>(a.v_sn, key0, a.nk, wv, lane, clamp);
    tile_dma<kDI>((const char*)(kbase + key0 * a.k_sn), ks, smem + 2 * st * kATileU4, wv);
    tile_dma<kDI>((const char*)(vbase + key0 * a.v_sn), vs, smem + (2 * st + 1) * kATileU4, wv);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  uint32_t kaddr[8], vaddr[4][2];
  {
    const int x = hl ^ swz(ql & 15);
#pragma unroll
    for (int s = 0; s < 8; ++s) kaddr[s] = lds0 + ql * 256 + (((2 * s) ^ x) << 4);
    const int a4 = lane & 3, j4 = (lane & 15) >> 2, g2 = (lane >> 4) & 1;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        vaddr[dblk][u] = lds0 + kVBuf + (4 * hl + j4) * 256 +
                         ((4 * (dblk ^ j4) + ((2 * g2 + (a4 >> 1)) ^ (2 * u + hl))) << 4) + (a4 & 1) * 8;
  }
  char* const stage = (char*)smem + kFewStage + wv * kFewStageWave;

  for (int64_t grp = g_begin + wv; grp < g_end; grp += kFewW) {
    const int64_t q0 = grp * 32;
    bf16x8 qf[8];
    {
      const int64_t qi = min(q0 + ql, a.nq - 1);
      const uint16_t* qrow = (const uint16_t*)a.q + b * a.q_sb + qi * a.q_sn + (int64_t)h * a.q_sh;
#pragma unroll
      for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(bf16x8, *(const uint4*)(qrow + 16 * s + 8 * hl));
    }
    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    // One key step against resident pair ST (k_attention's s_phase,
    // softmax and pv_phase).
    auto step = [&](auto st_c) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int KB = ST * kParBytes + kKBuf;
      f32x16 sacc[2];
      auto s_block = [&](auto j_c) {
        constexpr int OFF = KB + 8192 * decltype(j_c)::value;
        bf16x8 kf[8];
        kf[0] = lds_b128<OFF>(kaddr[0]);
        kf[1] = lds_b128<OFF>(kaddr[1]);
        kf[2] = lds_b128<OFF>(kaddr[2]);
        kf[3] = lds_b128<OFF>(kaddr[3]);
        kf[4] = lds_b128<OFF>(kaddr[4]);
        kf[5] = lds_b128<OFF>(kaddr[5]);
        kf[6] = lds_b128<OFF>(kaddr[6]);
        kf[7] = lds_b128<OFF>(kaddr[7]);
        OGA_LGKM(0, "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]),
                 "+v"(kf[7]));
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) acc = mfma_bf16(kf[s], qf[s], acc);
        return acc;
      };
      sacc[0] = s_block(IC<0>{});
      sacc[1] = s_block(IC<1>{});
      auto read_v = [&](auto c_c, u32x2(&vr)[8]) {
        constexpr int OFF = ST * kParBytes + 4096 * decltype(c_c)::value;  // vaddr includes kVBuf
        vr[0] = lds_tr16<OFF>(vaddr[0][0]);
        vr[1] = lds_tr16<OFF + 2048>(vaddr[0][1]);
        vr[2] = lds_tr16<OFF>(vaddr[1][0]);
        vr[3] = lds_tr16<OFF + 2048>(vaddr[1][1]);
        vr[4] = lds_tr16<OFF>(vaddr[2][0]);
        vr[5] = lds_tr16<OFF + 2048>(vaddr[2][1]);
        vr[6] = lds_tr16<OFF>(vaddr[3][0]);
        vr[7] = lds_tr16<OFF + 2048>(vaddr[3][1]);
      };
      u32x2 vr0[8], vr1[8];
      read_v(IC<0>{}, vr0);  // in flight under the softmax
      // softmax: keys past nk score -inf; the running max moves lazily
      const int64_t rem64 = a.nk - (int64_t)ST * kAK;
      if (rem64 < kAK) {
        int remh = (int)rem64 - hl4;
        asm volatile("" : "+v"(remh));  // compares here, not 32 lane masks hoisted out of the loop
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (32 * j + 8 * (e >> 2) + (e & 3) >= remh) sacc[j][e] = -INFINITY;
      }
      float mx = sacc[0][0];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = (j == 0 ? 1 : 0); e < 16; ++e) mx = __builtin_fmaxf(mx, sacc[j][e]);
      const float ms = max_halves(mx) * a.scale_log2;
      if (__any(ms > m_run + 8.0f)) {
        const float m_new = __builtin_fmaxf(m_run, ms);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
      }
      const float nm = -m_run;
      float ps0, ps1;  // from the first terms (P >= 0 is never -0: 0 + x would be x)
      uint32_t pb[2][8];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e], a.scale_log2, nm));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e + 1], a.scale_log2, nm));
          ps0 = (j == 0 && e == 0) ? p0 : ps0 + p0;
          ps1 = (j == 0 && e == 0) ? p1 : ps1 + p1;
          pb[j][e >> 1] = pack2(p0, p1);
        }
      l_run += ps0 + ps1;
      auto pv = [&](auto c_c, u32x2(&cur)[8], u32x2(&nxt)[8]) {
        constexpr int C = decltype(c_c)::value;
        if constexpr (C + 1 < 4) {
          read_v(IC<C + 1>{}, nxt);
          OGA_LGKM(8, "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]), "+v"(cur[5]),
                   "+v"(cur[6]), "+v"(cur[7]));
        } else {
          OGA_LGKM(0, "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]), "+v"(cur[5]),
                   "+v"(cur[6]), "+v"(cur[7]));
        }
        const uint32_t* pw = &pb[C >> 1][4 * (C & 1)];
        const uint4 pu = {pw[0], pw[1], pw[2], pw[3]};
        const bf16x8 pf = __builtin_bit_cast(bf16x8, pu);
#pragma unroll
        for (int dblk = 0; dblk < 4; ++dblk) {
          const uint4 vu = {cur[2 * dblk][0], cur[2 * dblk][1], cur[2 * dblk + 1][0], cur[2 * dblk + 1][1]};
          o[dblk] = mfma_bf16(__builtin_bit_cast(bf16x8, vu), pf, o[dblk]);
        }
      };
      pv(IC<0>{}, vr0, vr1);
      pv(IC<1>{}, vr1, vr0);
      pv(IC<2>{}, vr0, vr1);
      pv(IC<3>{}, vr1, vr0);
    };
    step(IC<0>{});
    if (nsteps > 1) step(IC<1>{});
    if (nsteps > 2) step(IC<2>{});
    if (nsteps > 3) step(IC<3>{});

    // O = O^T / l through the wave's staging, 16 query rows per pass: lanes
    // of rows 16p .. 16p+15 write their 256-byte rows (16-byte chunk c of
    // row r at chunk c ^ r), then the wave stores four whole rows per
    // instruction.
    const float inv = 1.0f / sum_halves(l_run);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if ((ql >> 4) == p) {
        const int r = ql & 15;
#pragma unroll
        for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            uint2 w;
            w.x = pack2(o[dblk][4 * gq] * inv, o[dblk][4 * gq + 1] * inv);
            w.y = pack2(o[dblk][4 * gq + 2] * inv, o[dblk][4 * gq + 3] * inv);
            *(uint2*)(stage + r * 256 + (((4 * dblk + gq) ^ r) << 4) + 8 * hl) = w;
          }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int oc = lane & 15;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = 4 * it + (lane >> 4);
        const uint4 w = *(const uint4*)(stage + r * 256 + ((oc ^ r) << 4));
        const int64_t qr = q0 + 16 * p + r;
        if (qr < a.nq) {
          const int64_t off = b * a.o_sb + qr * a.o_sn + (int64_t)h * a.o_sh + 8 * oc;
          if (a.oq)
            *(uint2*)(a.oq + off) = e4m3_of_bf16x8(w, oq_r, a.oq_bf16);
          else
            *(uint4*)(a.o + off) = w;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the staging reads, before the next pass writes
    }
  }
}

// ------------------------------------------------------- FP8 attention
// FlashAttention-3's FP8 path, as the reference calls it with per-head e4m3
// q, k, v and their [B, H] descales (official_ltx23_benchmark.py:3330-3340):
//   S = (q8 . k8) * qd * kd * scale,  P = softmax(S) rounded to e4m3,
//   O = (P8 . v8) * vd / l,  l the float32 row sum of P.
// Both products run on v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3): per 64-key
// step and wave, 2 key blocks x 2 d-steps of 64 for S^T and 4 d-blocks for
// O^T, 8 MFMAs where the bf16 kernel issues 32.
//
// Operands (lane l, h = l / 32). S^T = K Q^T: A = K row 32j + l%32, bytes
// 64s + 32h .. +31 of it; B = Q^T, the same bytes of query l%32, held in
// registers. The accumulator layout, the masking and the online softmax are
// the bf16 kernel's (lane l: query l%32, keys 8g + 4h + r of each 32-key
// block), except that the running max lags by at most 0.8 (not 8), which
// keeps every P of the offset form below e4m3's 448. O^T = V^T P^T: B = P^T,
// lane l holding the e4m3 P of its own 32
// keys kappa(h, s) = 32(s/16) + 8((s%16)/4) + 4h + s%4 in k-slot s, so P
// stays in its lane; A = V^T, lane l needing V[kappa(h, s)][d] for d-row
// 32 dblk + l%32. k_fp8_v_transpose first rewrites V as vt [B, H, D, npad]
// with each 64-key step in slot order (position 32h + s of step t holds key
// 64t + kappa(h, s), zero past the last key), so those 32 bytes are
// contiguous in a d-row.
//
// LDS per step: the K tile (64 rows x 128 bytes) in the FP8 GEMM's slab
// layout (two rows per 256-byte line, chunk c of row r at
// (8(r%2) + c) ^ ((r/2)%8)) and the V^T tile (128 d-rows x 64 bytes, chunk c
// of row d at c ^ ((d/4)%4)); three such 16 KiB pairs in a ring.
constexpr int kF8Tile = kAK * kAD;  // bytes of a K or V^T tile: 8 KiB
constexpr float kF8Offset = 8.0f;  // P = 2^(s - m + kF8Offset): a row's largest P is >= 256
// How far a row's scores may pass the running max before O and l are
// rescaled: 2^(8 + 0.8) = 445.7 stays below e4m3's largest finite 448.
constexpr float kF8Lag = 0.8f;
static_assert(kF8Offset + kF8Lag < 8.807f, "P must stay below 448 = 2^8.807");
constexpr int kF8Pair = 2 * kF8Tile;
constexpr int k8_off(int r, int c) { return (r >> 1) * 256 + (((r & 1) * 8 + c) ^ ((r >> 1) & 7)) * 16; }
constexpr int vt_off(int d, int c) { return d * 64 + ((c ^ ((d >> 2) & 3)) << 4); }
constexpr int kappa(int h, int slot) { return 32 * (slot >> 4) + 8 * ((slot & 15) >> 2) + 4 * h + (slot & 3); }
// Each 16-lane group of a ds_read_b128 touches 64 distinct banks.
constexpr bool f8_reads_conflict_free() {
  for (int grp = 0; grp < 4; ++grp)
    for (int j = 0; j < 2; ++j)
      for (int s = 0; s < 2; ++s)
        for (int q = 0; q < 2; ++q) {
          unsigned long long kb = 0, vb = 0;
          for (int l = 16 * grp; l < 16 * grp + 16; ++l) {
            const int ql = l & 31, h = l >> 5;
            const int bk = (k8_off(32 * j + ql, 4 * s + 2 * h + q) >> 2) & 63;
            const int bv = (vt_off(32 * (2 * j + s) + ql, 2 * h + q) >> 2) & 63;
            for (int i = 0; i < 4; ++i) {
              if (((kb >> ((bk + i) & 63)) & 1ull) || ((vb >> ((bv + i) & 63)) & 1ull)) return false;
              kb |= 1ull << ((bk + i) & 63);
              vb |= 1ull << ((bv + i) & 63);
            }
          }
        }
  return true;
}
static_assert(f8_reads_conflict_free(), "FP8 attention fragment reads would conflict");
// kappa is a bijection from (h, slot) onto the 64 keys of a step.
constexpr bool kappa_is_bijective() {
  unsigned long long seen = 0;
  for (int h = 0; h < 2; ++h)
    for (int sl = 0; sl < 32; ++sl) seen |= 1ull << kappa(h, sl);
  return seen == ~0ull;
}
static_assert(kappa_is_bijective(), "slot order must cover every key of a step once");

OGA_DEVICE f32x16 mfma_f8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
template <int OFF>
OGA_DEVICE i32x8 lds_b256(uint32_t a0, uint32_t a1) {
  static_assert(OFF >= 0 && OFF < 65536, "LDS offset");
  uint4 lo, hi;
  // Early-clobber outputs: the first read's data returns after the second
  // read has issued, so its destination must not share a register with a1.
  asm volatile("ds_read_b128 %0, %2 offset:%4\n\tds_read_b128 %1, %3 offset:%4"
               : "=&v"(lo), "=&v"(hi)
               : "v"(a0), "v"(a1), "i"(OFF));
  i32x8 r = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  return r;
}

#ifndef OGA_F8_WAVES
#define OGA_F8_WAVES 12
#endif
constexpr int kF8W = OGA_F8_WAVES;  // waves per FP8 workgroup, 32 queries each
constexpr int kF8Q = 32 * kF8W;      // queries per FP8 workgroup
constexpr int kF8DmaW = 8;           // waves whose DMA fills the tiles: one 1 KiB instruction per tile each
static_assert(kF8W == 8 || kF8W == 12, "8 waves (2 per SIMD) or 12 (3 per SIMD)");
constexpr int kF8Bufs = kABufs;  // K/V^T tile pairs in the FP8 kernel's ring
// Waves past the eighth send the same two DMA instructions per step as the
// others (so that every wave waits for the same count) into 2 KiB of their
// own after the ring, re-reading tile rows the first eight fetch.
constexpr int kF8DummyOff = kF8Bufs * kF8Pair;
constexpr int kF8Ring = kF8DummyOff + (kF8W - kF8DmaW) * 2048;
constexpr int kF8Lds = kF8Ring > kF8W * 8192 ? kF8Ring : kF8W * 8192;
static_assert(kF8Ring <= 65536, "the FP8 fragment reads address LDS with 16-bit offsets");

__global__ __launch_bounds__(64 * kF8W) __attribute__((amdgpu_waves_per_eu(kF8W / 4, kF8W / 4))) void k_attention_fp8(
    AttnArgs a) {
  __shared__ uint4 smem[kF8Lds / 16];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  int64_t wg = blockIdx.x;
  int part = -1;
  if (wg < a.nfull) {
    if (a.xcd_remap) wg = (wg & 7) * (a.nfull >> 3) + (wg >> 3);
  } else {
    const int64_t u = wg - a.nfull;
    wg = a.nfull + u / a.ksplit;
    part = (int)(u % a.ksplit);
  }
  const int qb = (int)(wg % a.nqb);
  const int64_t bh = wg / a.nqb;
  const int h = (int)(bh % a.heads);
  const int64_t b = bh / a.heads;
  const int64_t q0 = (int64_t)qb * kF8Q + wv * 32;
  const int hl = lane >> 5;
  const int ql = lane & 31;
  const float qd = a.q_ds[b * a.heads + h], kd = a.k_ds[b * a.heads + h], vd = a.v_ds[b * a.heads + h];
  const float sl2 = a.scale_log2 * (qd * kd);

  // Q^T fragments of d-steps 0, 1: bytes 64s + 32hl .. +31 of query q0 + ql.
  i32x8 qf[2];
  {
    const int64_t qi = min(q0 + ql, a.nq - 1);
    const uint8_t* qrow = (const uint8_t*)a.q + b * a.q_sb + qi * a.q_sn + (int64_t)h * a.q_sh;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint4 lo = *(const uint4*)(qrow + 64 * s + 32 * hl);
      const uint4 hi = *(const uint4*)(qrow + 64 * s + 32 * hl + 16);
      qf[s] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
  }
  const uint8_t* kbase = (const uint8_t*)a.k + b * a.k_sb + (int64_t)h * a.k_sh;
  const uint8_t* vtbase = a.vt + (b * a.heads + h) * (int64_t)kAD * a.vt_npad;
  const int64_t nsteps_all = (a.nk + kAK - 1) / kAK;
  const int64_t st_begin = part < 0 ? 0 : nsteps_all * part / a.ksplit;
  const int64_t st_end = part < 0 ? nsteps_all : nsteps_all * (part + 1) / a.ksplit;

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // DMA: wave wv fills bytes [1024 wv, 1024 wv + 1024) of each tile. K: lane
  // p writes line L = 4wv + p/16, position p%16, holding row 2L + v/8, chunk
  // v%8 with v = (p%16) ^ (L%8). V^T: lane p writes d-row 16wv + p/4,
  // position p%4, holding chunk (p%4) ^ ((d/4)%4) of the row.
  const int wd = wv % kF8DmaW;  // the tile part this wave's DMA reads
  const int kL = 4 * wd + (lane >> 4);
  const int kv = (lane & 15) ^ (kL & 7);
  const int krow = 2 * kL + (kv >> 3);
  const uint32_t koff_c = (uint32_t)((kv & 7) * 16);
  const int vd_row = 16 * wd + (lane >> 2);
  // Per-lane byte offsets from the step's first key (32 bits: the host keeps
  // 64 key rows of K and 128 d-rows of V^T below 2^32 bytes), added to a
  // wave-uniform base, so a step's DMA addresses cost no 64-bit vector math.
  const uint32_t vt_src = (uint32_t)(vd_row * a.vt_npad) + (uint32_t)(((lane & 3) ^ ((vd_row >> 2) & 3)) * 16);
  const uint32_t k_src = (uint32_t)(krow * a.k_sn) + koff_c;
  // LDS destinations (wave-uniform): the wave's 1 KiB of the pair's K and
  // V^T tiles, or, for a wave past the eighth, its own 2 KiB after the ring.
  const bool tile_wave = wv < kF8DmaW;
  const int k_dst = tile_wave ? wv * 64 : kF8DummyOff / 16 + (wv - kF8DmaW) * 128;
  const int v_dst = tile_wave ? kF8Tile / 16 + wv * 64 : kF8DummyOff / 16 + (wv - kF8DmaW) * 128 + 64;
  auto dma_step = [&](int64_t s2, uint4* dst) {
    const int64_t key0 = s2 * kAK;
    uint4* const kd = tile_wave ? dst + k_dst : smem + k_dst;
    uint4* const vdp = tile_wave ? dst + v_dst : smem + v_dst;
    // Rows past the last key (the last, partial step) re-read the last key.
    const int last = (int)min((int64_t)(kAK - 1), a.nk - 1 - key0);
    const uint32_t ko = krow <= last ? k_src : (uint32_t)(last * a.k_sn) + koff_c;
    __builtin_amdgcn_global_load_lds((const void*)(kbase + key0 * a.k_sn + ko), (lds_void*)kd, 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(vtbase + key0 + vt_src), (lds_void*)vdp, 16, 0, 0);
  };
  dma_step(st_begin, smem);
  if (kF8Bufs == 3) dma_step(min(st_begin + 1, st_end - 1), smem + kF8Pair / 16);

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  uint32_t kaddr[2][2], vaddr[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int q = 0; q < 2; ++q) kaddr[s][q] = lds0 + k8_off(ql, 4 * s + 2 * hl + q);
#pragma unroll
  for (int q = 0; q < 2; ++q) vaddr[q] = lds0 + kF8Tile + vt_off(ql, 2 * hl + q);
  const int hl4 = 4 * hl;

  // S^T of the step in pair PAR: two 32-key blocks, two d-steps each.
  auto s_phase = [&](auto par_c, f32x16(&sacc)[2]) {
    constexpr int KB = decltype(par_c)::value * kF8Pair;
    auto s_block = [&](auto j_c) {
      constexpr int J = decltype(j_c)::value;
      i32x8 kf0 = lds_b256<KB + 4096 * J>(kaddr[0][0], kaddr[0][1]);
      i32x8 kf1 = lds_b256<KB + 4096 * J>(kaddr[1][0], kaddr[1][1]);
      OGA_LGKM(0, "+v"(kf0), "+v"(kf1));
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
      acc = mfma_f8(kf0, qf[0], acc);
      return mfma_f8(kf1, qf[1], acc);
    };
    sacc[0] = s_block(IC<0>{});
    sacc[1] = s_block(IC<1>{});
  };
  // V^T fragments of the four d-blocks of pair PAR (waited for in pv).
  auto v_read = [&](auto par_c, i32x8(&vf)[4]) {
    constexpr int KB = decltype(par_c)::value * kF8Pair;
    vf[0] = lds_b256<KB + 0 * 2048>(vaddr[0], vaddr[1]);
    vf[1] = lds_b256<KB + 1 * 2048>(vaddr[0], vaddr[1]);
    vf[2] = lds_b256<KB + 2 * 2048>(vaddr[0], vaddr[1]);
    vf[3] = lds_b256<KB + 3 * 2048>(vaddr[0], vaddr[1]);
  };
  // Online softmax of step st: masking past the last key, the running max m
  // and P = 2^(s sl2 - m + 8) with FlashAttention-3's FP8 offset of 8. The
  // max lags by at most kF8Lag: O and l are rescaled only when some query's
  // scores pass m + kF8Lag, so every P <= 2^(8 + kF8Lag) < 448 stays finite
  // in e4m3, the largest P of a row is >= 256 (m never exceeds the row's
  // true max), and P down to 2^-6 stay in e4m3's normal range, where nearest
  // even errs by at most 2^-4 of P. (Without the offset a lagging max leaves
  // the largest P as small as 1 and pushes the small ones into e4m3's
  // subnormals.) P goes in float32 into l and as e4m3 into the B operand,
  // byte 16j + e = P of accumulator e of block j; the common factor 2^8
  // cancels in O / l (and in the key-split merge, which weights O and l
  // alike).
  auto softmax = [&](int64_t st, f32x16(&sacc)[2], i32x8& pf) {
    const int64_t rem64 = a.nk - st * kAK;
    if (rem64 < kAK) {
      const int remh = (int)rem64 - hl4;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (32 * j + 8 * (e >> 2) + (e & 3) >= remh) sacc[j][e] = -INFINITY;
    }
    float mx = sacc[0][0];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = (j == 0 ? 1 : 0); e < 16; ++e) mx = __builtin_fmaxf(mx, sacc[j][e]);
    const float ms = max_halves(mx) * sl2;
    if (__any(ms > m_run + kF8Lag)) {
      const float m_new = __builtin_fmaxf(m_run, ms);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
    }
    const float nm = kF8Offset - m_run;
    // (the sums start from their first term: P >= 0 is never -0, so 0 + x,
    // which the compiler may not drop, would be x)
    float ps0, ps1;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e], sl2, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e + 1], sl2, nm));
        const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e + 2], sl2, nm));
        const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][e + 3], sl2, nm));
        if (j == 0 && e == 0) {
          ps0 = p0 + p2;
          ps1 = p1 + p3;
        } else {
          ps0 += p0 + p2;
          ps1 += p1 + p3;
        }
        pf[4 * j + (e >> 2)] = (int)e4m3x4_valu(p0, p1, p2, p3);
      }
    l_run += ps0 + ps1;
  };
  auto pv = [&](i32x8(&vf)[4], const i32x8& pf) {
    OGA_LGKM(0, "+v"(vf[0]), "+v"(vf[1]), "+v"(vf[2]), "+v"(vf[3]));
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk) o[dblk] = mfma_f8(vf[dblk], pf, o[dblk]);
  };

  auto step = [&](auto par_c, int64_t st) {
    constexpr int PAR = decltype(par_c)::value;
    // This wave's two DMA instructions of step st have landed (those of
    // step st + 1 may still be in flight), then every wave's.
    if (kF8Bufs == 3)
      asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    {
      constexpr int NP = (PAR + kF8Bufs - 1) % kF8Bufs;
      if (kF8Bufs == 3)
        dma_step(min(st + 2, st_end - 1), smem + NP * (kF8Pair / 16));
      else if (st + 1 < st_end)
        dma_step(st + 1, smem + NP * (kF8Pair / 16));
    }
    f32x16 sacc[2];
    i32x8 vf[4], pf;
    s_phase(par_c, sacc);
    if constexpr (kF8W == 8) {
      // V^T fragments in flight under the softmax.
      v_read(par_c, vf);
      softmax(st, sacc, pf);
    } else {
      // With three waves per SIMD the fragments are read after the softmax
      // (168 VGPRs), the other waves covering the reads' latency.
      softmax(st, sacc, pf);
      v_read(par_c, vf);
    }
    pv(vf, pf);
  };

  for (int64_t st = st_begin; st < st_end; st += kF8Bufs) {
    step(IC<0>{}, st);
    if (st + 1 < st_end) step(IC<1>{}, st + 1);
    if constexpr (kF8Bufs == 3)
      if (st + 2 < st_end) step(IC<2 % kF8Bufs>{}, st + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if (part >= 0) {
    const int64_t row = (int64_t)(blockIdx.x - a.nfull) * kF8Q + wv * 32 + ql;
    float* po = a.part_o + row * kAD;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(float4*)(po + 32 * dblk + 8 * g + 4 * hl) = make_float4(o[dblk][4 * g] * vd, o[dblk][4 * g + 1] * vd,
                                                                  o[dblk][4 * g + 2] * vd, o[dblk][4 * g + 3] * vd);
    const float l_tot = sum_halves(l_run);
    if (hl == 0) *(float2*)(a.part_ml + 2 * row) = make_float2(m_run, l_tot);
    return;
  }
  const float inv = vd / sum_halves(l_run);
  __syncthreads();
  char* const otile = (char*)smem + wv * 8192;
#pragma unroll
  for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack2(o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv);
      w.y = pack2(o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv);
      *(uint2*)(otile + ql * 256 + (((4 * dblk + g) ^ (ql & 15)) << 4) + 8 * hl) = w;
    }
  __syncthreads();
  const int oc = lane & 15;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = 4 * it + (lane >> 4);
    const uint4 w = *(const uint4*)(otile + r * 256 + ((oc ^ (r & 15)) << 4));
    const int64_t qr = q0 + r;
    if (qr < a.nq) *(uint4*)(a.o + b * a.o_sb + qr * a.o_sn + (int64_t)h * a.o_sh + 8 * oc) = w;
  }
}

// vt[b, h, d, 64t + 32h' + s] = v[b, 64t + kappa(h', s), h, d] (zero for keys
// past nk): one workgroup per (64-key step t, head, batch) stages the 64 x
// 128-byte tile in LDS (rows padded to 144 bytes) and writes the 128 d-rows
// of 64 bytes in slot order.
__global__ __launch_bounds__(256) void k_fp8_v_transpose(const uint8_t* v, int64_t v_sb, int64_t v_sn, int64_t v_sh,
                                                         uint8_t* vt, int64_t nk, int64_t npad, int heads) {
  constexpr int kPitch = kAD + 16;
  __shared__ uint8_t tile[kAK * kPitch];
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t key0 = t * kAK;
  const uint8_t* src = v + b * v_sb + (int64_t)h * v_sh;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int i = threadIdx.x + 256 * it;  // 512 chunks of 16 bytes
    const int r = i >> 3, c = i & 7;
    uint4 val = {0u, 0u, 0u, 0u};
    if (key0 + r < nk) val = *(const uint4*)(src + (key0 + r) * v_sn + 16 * c);
    *(uint4*)(tile + r * kPitch + 16 * c) = val;
  }
  __syncthreads();
  uint8_t* dst = vt + ((b * heads + h) * (int64_t)kAD) * npad + key0;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int i = threadIdx.x + 256 * it;  // 128 d-rows x 4 chunks of 16 positions
    const int d = i >> 2, c = i & 3;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t x = 0;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int pos = 16 * c + 4 * k + bb;
        x |= (uint32_t)tile[kappa(pos >> 5, pos & 31) * kPitch + d] << (8 * bb);
      }
      w[k] = x;
    }
    *(uint4*)(dst + (int64_t)d * npad + 16 * c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// The split blocks' parts merged: for query row r of split block sb (block
// nfull + sb), with parts p of running max m_p and sum l_p,
// O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p, M = max_p m_p. One
// thread per (row, 8 consecutive d); rows past nq are not stored.
__global__ __launch_bounds__(256) void k_attention_combine(AttnArgs a, int64_t rows) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * (kAD / 8)) return;
  const int c = (int)(idx % (kAD / 8));
  const int64_t row = idx / (kAD / 8);
  const int64_t sb = row / a.qpb;
  const int qr = (int)(row % a.qpb);
  const int64_t wg = a.nfull + sb;
  const int qb = (int)(wg % a.nqb);
  const int64_t bh = wg / a.nqb;
  const int h = (int)(bh % a.heads);
  const int64_t b = bh / a.heads;
  const int64_t qi = (int64_t)qb * a.qpb + qr;
  if (qi >= a.nq) return;
  const int64_t r0 = sb * a.ksplit * a.qpb + qr;  // row of part 0; part p adds p * qpb
  float mx = -INFINITY;
  for (int p = 0; p < a.ksplit; ++p) mx = __builtin_fmaxf(mx, a.part_ml[2 * (r0 + (int64_t)p * a.qpb)]);
  float l = 0.0f, acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int p = 0; p < a.ksplit; ++p) {
    const int64_t rp = r0 + (int64_t)p * a.qpb;
    const float w = __builtin_amdgcn_exp2f(a.part_ml[2 * rp] - mx);
    l += w * a.part_ml[2 * rp + 1];
    const float4 x0 = *(const float4*)(a.part_o + rp * kAD + 8 * c);
    const float4 x1 = *(const float4*)(a.part_o + rp * kAD + 8 * c + 4);
    acc[0] += w * x0.x; acc[1] += w * x0.y; acc[2] += w * x0.z; acc[3] += w * x0.w;
    acc[4] += w * x1.x; acc[5] += w * x1.y; acc[6] += w * x1.z; acc[7] += w * x1.w;
  }
  const float inv = 1.0f / l;
  uint4 w;
  w.x = pack2(acc[0] * inv, acc[1] * inv);
  w.y = pack2(acc[2] * inv, acc[3] * inv);
  w.z = pack2(acc[4] * inv, acc[5] * inv);
  w.w = pack2(acc[6] * inv, acc[7] * inv);
  const int64_t off = b * a.o_sb + qi * a.o_sn + (int64_t)h * a.o_sh + 8 * c;
  if (a.oq)
    *(uint2*)(a.oq + off) = e4m3_of_bf16x8(w, e4m3_recip(a), a.oq_bf16);
  else
    *(uint4*)(a.o + off) = w;
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

namespace {
// The attention kernels: the bf16 kernel for many keys and for few
// (kShortSteps), and the FP8 kernel.
enum AttnKernel { kBf16Long = 0, kBf16Short = 1, kFp8 = 2 };
struct AttnCfg {
  const void* fn;
  int threads, qpb;
};
AttnCfg attn_cfg(AttnKernel k) {
  switch (k) {
    case kBf16Short: return {(const void*)k_attention<kAWShort, kABufsShort>, 64 * kAWShort, 32 * kAWShort};
    case kFp8: return {(const void*)k_attention_fp8, 64 * kF8W, kF8Q};
    default: return {(const void*)k_attention<kAW, kABufs>, 64 * kAW, kAQ};
  }
}
AttnKernel bf16_kernel(int64_t nk) { return (nk + kAK - 1) / kAK <= kShortSteps ? kBf16Short : kBf16Long; }

// Workgroups of an attention kernel resident at once on the current device
// (CUs x workgroups per CU), cached per device (relaxed atomics: threads
// filling an entry at once store the same value); 0 if the runtime cannot say.
int64_t attention_slots(AttnKernel kern) {
  static std::atomic<int64_t> cache[3][64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int64_t n = cache[kern][dev].load(std::memory_order_relaxed);
  if (n == 0) {
    const AttnCfg c = attn_cfg(kern);
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, c.fn, c.threads, 0) != hipSuccess)
      return 0;
    n = (int64_t)cus * per_cu > 0 ? (int64_t)cus * per_cu : -1;
    cache[kern][dev].store(n, std::memory_order_relaxed);
  }
  return n > 0 ? n : 0;
}

struct AttnPlan {
  int64_t wgs, nfull, units;  // query blocks, whole ones, split parts
  int ksplit;
};
// Blocks beyond the last whole round of the CUs are cut into k parts over
// their key steps (k <= 8 and <= the steps) when that shortens the last
// round by at least a tenth of a round: rem blocks in k parts take
// ceil(k rem / slots) rounds of 1/k of a block's time. Not for kShortSteps
// steps or fewer: a block's time is then mostly its Q loads and O stores,
// which every part repeats, and the merge adds a launch (at 256 keys the
// split ran 75.7 against 66.9 us unsplit).
AttnPlan attention_plan(int64_t wgs, int64_t nk, int64_t slots) {
  AttnPlan p{wgs, wgs, 0, 1};
  const int64_t rem = slots > 0 ? wgs % slots : 0;
  if (rem == 0) return p;
  const int64_t nsteps = (nk + kAK - 1) / kAK;
  if (nsteps <= kShortSteps) return p;
  double best = 1.0;
  for (int k = 2; k <= 8 && k <= nsteps; ++k) {
    const double c = (double)((k * rem + slots - 1) / slots) / k;
    if (c < best - 0.1) { best = c; p.ksplit = k; }
  }
  if (p.ksplit > 1) { p.nfull = wgs - rem; p.units = rem * p.ksplit; }
  return p;
}
int64_t attention_ws_bytes(const AttnPlan& p, int qpb) { return p.units * qpb * (kAD + 2) * (int64_t)sizeof(float); }

// oq_scale given: o is the e4m3 output of the quantizer with that scale
// (AttnArgs::oq).
int attention_run(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                  const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3], int64_t batch,
                  int64_t nq, int64_t nk, int64_t heads, int64_t head_dim, float softmax_scale, void* workspace,
                  int64_t workspace_bytes, void* stream, const float* oq_scale = nullptr, int oq_zero_dim = 0) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return fail("null pointer");
  if (head_dim != kAD) return unsupported("head_dim must be %d", kAD);
  if (batch < 0 || nq < 0 || nk < 0 || heads < 0) return fail("bad shape");
  if (batch == 0 || nq == 0 || heads == 0) return OGA_OK;
  if (nk == 0) return unsupported("no keys");
  if (heads > INT32_MAX) return unsupported("too many heads");
  for (const int64_t* s : {q_strides, k_strides, v_strides, o_strides})
    for (int i = 0; i < 3; ++i)
      if (s[i] % 8) return fail("strides must be multiples of 8 elements");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 16))
    return fail("q/k/v/o must be 16-byte aligned");
  if (!(softmax_scale > 0.0f) || !__builtin_isfinite(softmax_scale)) return unsupported("softmax_scale must be positive");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace)) return fail("bad workspace");
  if (workspace && !aligned(workspace, 16)) return fail("workspace must be 16-byte aligned");
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v;
  if (oq_scale) {
    a.oq = (uint8_t*)o;
    a.oq_scale = oq_scale;
    a.oq_bf16 = oq_zero_dim ? 1 : 0;
  } else {
    a.o = (uint16_t*)o;
  }
  a.q_sb = q_strides[0]; a.q_sn = q_strides[1]; a.q_sh = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sn = k_strides[1]; a.k_sh = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sn = v_strides[1]; a.v_sh = v_strides[2];
  a.o_sb = o_strides[0]; a.o_sn = o_strides[1]; a.o_sh = o_strides[2];
  a.nq = nq; a.nk = nk; a.heads = (int)heads;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  if (nk <= kFewKeys) {  // K/V of a head resident in LDS, no workspace
    const int64_t bhs = batch * heads;
    const int64_t groups = (nq + 31) / 32;
    int64_t slices = (int64_t)cu_count() / bhs;
    if (slices < 1) slices = 1;
    if (slices > groups) slices = groups;
    if (bhs * slices > (int64_t)UINT32_MAX || slices > INT32_MAX) return unsupported("too many query groups");
    hipLaunchKernelGGL(k_attention_fewkeys, dim3((unsigned)(bhs * slices)), dim3(64 * kFewW), 0,
                       (hipStream_t)stream, a, (int)slices);
    return launch_status();
  }
  const AttnKernel kern = bf16_kernel(nk);
  const AttnCfg cfg = attn_cfg(kern);
  const int64_t nqb = (nq + cfg.qpb - 1) / cfg.qpb;
  const int64_t wgs = nqb * heads * batch;
  if (nqb > INT32_MAX || wgs > UINT32_MAX / 8) return unsupported("too many query blocks");
  a.nqb = (int)nqb;
  a.qpb = cfg.qpb;
  AttnPlan plan{wgs, wgs, 0, 1};
  if (workspace_bytes > 0) {
    plan = attention_plan(wgs, nk, attention_slots(kern));
    if (attention_ws_bytes(plan, cfg.qpb) > workspace_bytes)
      return fail("workspace smaller than oga_attention_workspace_bytes");
  }
  a.nfull = plan.nfull;
  a.ksplit = plan.ksplit;
  a.part_o = (float*)workspace;
  a.part_ml = plan.units ? (float*)workspace + plan.units * cfg.qpb * kAD : nullptr;
  a.xcd_remap = plan.nfull % 8 == 0;
  if (kern == kBf16Short)
    hipLaunchKernelGGL((k_attention<kAWShort, kABufsShort>), dim3((unsigned)(plan.nfull + plan.units)),
                       dim3(cfg.threads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((k_attention<kAW, kABufs>), dim3((unsigned)(plan.nfull + plan.units)), dim3(cfg.threads), 0,
                       (hipStream_t)stream, a);
  if (plan.units) {
    const int64_t rows = (wgs - plan.nfull) * cfg.qpb;
    hipLaunchKernelGGL(k_attention_combine, dim3((unsigned)((rows * (kAD / 8) + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, a, rows);
  }
  return launch_status();
}

// FP8 attention: the V rewrite (vt, ceil(nk/64)*64 keys per d-row) at the
// start of the workspace, then the split parts' partials when the workspace
// also holds them.
int64_t vt_bytes(int64_t batch, int64_t heads, int64_t nk) {
  const int64_t npad = (nk + kAK - 1) / kAK * kAK;
  return (batch * heads * kAD * npad + 255) / 256 * 256;
}

int attention_fp8_run(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                      const void* v, const int64_t v_strides[3], const float* q_descale, const float* k_descale,
                      const float* v_descale, void* o, const int64_t o_strides[3], int64_t batch, int64_t nq,
                      int64_t nk, int64_t heads, int64_t head_dim, float softmax_scale, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return fail("null pointer");
  if (!q_descale || !k_descale || !v_descale) return fail("null descale");
  if (head_dim != kAD) return unsupported("head_dim must be %d", kAD);
  if (batch < 0 || nq < 0 || nk < 0 || heads < 0) return fail("bad shape");
  if (batch == 0 || nq == 0 || heads == 0) return OGA_OK;
  if (nk == 0) return unsupported("no keys");
  if (heads > 65535 || batch > 65535) return unsupported("batch and heads must be below 65536");
  // The DMA's per-lane offsets are 32-bit: 64 key rows of K and 128 d-rows
  // of the rewritten V^T (nk padded to 64) stay below 2^32 bytes.
  if (k_strides[1] < 0 || k_strides[1] > (int64_t(1) << 26)) return unsupported("key token stride out of range");
  if (nk > (int64_t(1) << 25)) return unsupported("more than 2^25 keys");
  for (const int64_t* st : {q_strides, k_strides, v_strides})
    for (int i = 0; i < 3; ++i)
      if (st[i] % 16) return fail("e4m3 strides must be multiples of 16 elements");
  for (int i = 0; i < 3; ++i)
    if (o_strides[i] % 8) return fail("output strides must be multiples of 8 elements");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 16))
    return fail("q/k/v/o must be 16-byte aligned");
  if (!(softmax_scale > 0.0f) || !__builtin_isfinite(softmax_scale)) return unsupported("softmax_scale must be positive");
  const int64_t vtb = vt_bytes(batch, heads, nk);
  if (!workspace || workspace_bytes < vtb) return fail("workspace smaller than oga_attention_fp8_workspace_bytes");
  if (!aligned(workspace, 256)) return fail("workspace must be 256-byte aligned");
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = (uint16_t*)o;
  a.q_sb = q_strides[0]; a.q_sn = q_strides[1]; a.q_sh = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sn = k_strides[1]; a.k_sh = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sn = v_strides[1]; a.v_sh = v_strides[2];
  a.o_sb = o_strides[0]; a.o_sn = o_strides[1]; a.o_sh = o_strides[2];
  a.nq = nq; a.nk = nk; a.heads = (int)heads;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.vt = (const uint8_t*)workspace;
  a.vt_npad = (nk + kAK - 1) / kAK * kAK;
  a.q_ds = q_descale; a.k_ds = k_descale; a.v_ds = v_descale;
  const int64_t nqb = (nq + kF8Q - 1) / kF8Q;
  const int64_t wgs = nqb * heads * batch;
  if (nqb > INT32_MAX || wgs > UINT32_MAX / 8) return unsupported("too many query blocks");
  a.nqb = (int)nqb;
  a.qpb = kF8Q;
  AttnPlan plan = attention_plan(wgs, nk, attention_slots(kFp8));
  if (vtb + attention_ws_bytes(plan, kF8Q) > workspace_bytes) plan = AttnPlan{wgs, wgs, 0, 1};
  a.nfull = plan.nfull;
  a.ksplit = plan.ksplit;
  a.part_o = plan.units ? (float*)((char*)workspace + vtb) : nullptr;
  a.part_ml = plan.units ? a.part_o + plan.units * kF8Q * kAD : nullptr;
  a.xcd_remap = plan.nfull % 8 == 0;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_fp8_v_transpose, dim3((unsigned)(a.vt_npad / kAK), (unsigned)heads, (unsigned)batch), dim3(256),
                     0, st, (const uint8_t*)v, a.v_sb, a.v_sn, a.v_sh, (uint8_t*)workspace, nk, a.vt_npad, (int)heads);
  int rc = launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(k_attention_fp8, dim3((unsigned)(plan.nfull + plan.units)), dim3(64 * kF8W), 0, st, a);
  if (plan.units) {
    const int64_t rows = (wgs - plan.nfull) * kF8Q;
    hipLaunchKernelGGL(k_attention_combine, dim3((unsigned)((rows * (kAD / 8) + 255) / 256)), dim3(256), 0, st, a,
                       rows);
  }
  return launch_status();
}
}  // namespace

extern "C" int oga_attention(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                             const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3],
                             int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim,
                             float softmax_scale, void* stream) {
  return attention_run(q, q_strides, k, k_strides, v, v_strides, o, o_strides, batch, nq, nk, heads, head_dim,
                       softmax_scale, nullptr, 0, stream);
}

extern "C" int64_t oga_attention_workspace_bytes(int64_t batch, int64_t nq, int64_t nk, int64_t heads,
                                                 int64_t head_dim) {
  if (batch <= 0 || nq <= 0 || nk <= 0 || heads <= 0 || head_dim != kAD) return 0;
  const AttnKernel kern = bf16_kernel(nk);
  const int qpb = attn_cfg(kern).qpb;
  const int64_t nqb = (nq + qpb - 1) / qpb;
  if (nqb > INT32_MAX || heads > INT32_MAX || nqb * heads > (int64_t)(UINT32_MAX / 8) / batch) return 0;
  return attention_ws_bytes(attention_plan(nqb * heads * batch, nk, attention_slots(kern)), qpb);
}

extern "C" int oga_attention_ws(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                                const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3],
                                int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim,
                                float softmax_scale, void* workspace, int64_t workspace_bytes, void* stream) {
  return attention_run(q, q_strides, k, k_strides, v, v_strides, o, o_strides, batch, nq, nk, heads, head_dim,
                       softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int oga_attention_e4m3_out_ws(const void* q, const int64_t q_strides[3], const void* k,
                                         const int64_t k_strides[3], const void* v, const int64_t v_strides[3],
                                         void* o8, const int64_t o_strides[3], int64_t batch, int64_t nq, int64_t nk,
                                         int64_t heads, int64_t head_dim, float softmax_scale,
                                         const float* out_scale, int scale_zero_dim, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  if (!out_scale) return fail("null output scale");
  return attention_run(q, q_strides, k, k_strides, v, v_strides, o8, o_strides, batch, nq, nk, heads, head_dim,
                       softmax_scale, workspace, workspace_bytes, stream, out_scale, scale_zero_dim);
}

extern "C" int64_t oga_attention_fp8_workspace_bytes(int64_t batch, int64_t nq, int64_t nk, int64_t heads,
                                                     int64_t head_dim) {
  if (batch <= 0 || nq <= 0 || nk <= 0 || heads <= 0 || head_dim != kAD) return 0;
  const int64_t nqb = (nq + kF8Q - 1) / kF8Q;
  if (nqb > INT32_MAX || heads > 65535 || batch > 65535) return 0;
  return vt_bytes(batch, heads, nk) +
         attention_ws_bytes(attention_plan(nqb * heads * batch, nk, attention_slots(kFp8)), kF8Q);
}

extern "C" int oga_attention_fp8_ws(const void* q8, const int64_t q_strides[3], const void* k8,
                                    const int64_t k_strides[3], const void* v8, const int64_t v_strides[3],
                                    const float* q_descale, const float* k_descale, const float* v_descale, void* o,
                                    const int64_t o_strides[3], int64_t batch, int64_t nq, int64_t nk, int64_t heads,
                                    int64_t head_dim, float softmax_scale, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  return attention_fp8_run(q8, q_strides, k8, k_strides, v8, v_strides, q_descale, k_descale, v_descale, o, o_strides,
                           batch, nq, nk, heads, head_dim, softmax_scale, workspace, workspace_bytes, stream);
}
