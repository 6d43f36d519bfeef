// Compacted QKV projection for gfx950, fused with the new K/V write into the paged cache.
//
// The reference projects every row of the sequence and zeroes the reuse rows afterwards
// (semblend_core/triton_kernels.py:451-522; fp32 linear, one rounding to the input dtype).
// Here only the computed rows are multiplied: row n of the product is hidden row positions[n],
// gathered while the tile is loaded. The product is taken transposed,
//     out^T[feature, row] = W[feature, :] . hidden[positions[row], :],
// on v_mfma_f32_32x32x16 (bf16 / fp16 in, fp32 accumulate). In that accumulator layout each
// lane owns one row (token) and four consecutive features per 4-register group, so the
// interleaved RoPE pairs (2i, 2i+1) of a head sit in one lane and the epilogue rotates them
// in registers before the single rounding to the output dtype.
//
// Tiles: 256 features x 256 rows per workgroup of 4 waves (each wave 128 x 128 = 4 x 4 MFMA
// blocks, 256 fp32 accumulators), one workgroup per CU; 128 x 128 (two per CU) when the row
// count is too small to give half the CUs a big tile. 64 hidden elements per k-step (each
// tile row one 128-byte line) in a 2-stage LDS ring (loads one step ahead, one barrier per
// step; 32 elements in 4 stages, half lines, was 1.5-4% slower). Both operands are read
// with their hidden dimension contiguous (W row-major [F, hidden], hidden [S, hidden]),
// moved global -> LDS with global_load_lds_dwordx4, 16-byte chunks of each tile row
// XOR-swizzled so that the ds_read_b128 fragment reads of 16 consecutive rows fall on
// distinct banks. Tiles are ordered XCD by XCD in bands of row tiles (qkv_tile) for L2 reuse.
//
// Epilogue (feature layout Q [Hq*D] | K [Hkv*D] | V [Hkv*D]):
//   split mode  Q -> q_out[row] (compact), K / V -> paged cache slot of positions[row];
//   dense mode  all features -> out[positions[row]] (the [S, F] drop-in layout).
// Bias (input dtype) is added in fp32; with RoPE, Q and K are rotated by the row's position
// (angle = float(p) * inv_freq[i]) with cos/sin from a per-(row, pair) table that a small
// kernel fills first (fp64 sincos rounded once to fp32, as in the RoPE kernels).

#include <algorithm>
#include <type_traits>

#include "sb_common.h"

namespace sb {
namespace {

typedef __bf16 qbf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 qf16x8_t __attribute__((ext_vector_type(8)));
typedef float qf32x16_t __attribute__((ext_vector_type(16)));

#ifndef SB_QKV_GROUP
#define SB_QKV_GROUP 8
#endif
constexpr int kQThreads = 256;
#ifndef SB_QKV_TK
#define SB_QKV_TK 64
#endif
#ifndef SB_QKV_STAGES
#define SB_QKV_STAGES 2
#endif
// Fragments of the next MFMA substep read while the current one's MFMAs issue (0: the
// compiler's own order).
#ifndef SB_QKV_FRAG_PIPE
#define SB_QKV_FRAG_PIPE 1
#endif
// Epilogue: blocks of RoPE table entries (4 groups x row blocks) loaded ahead of their use.
#ifndef SB_QKV_CS_AHEAD
#define SB_QKV_CS_AHEAD 1
#endif
// Substeps over which a step's refill loads are spread (the first ones of the step).
#ifndef SB_QKV_DMA_SPREAD
#define SB_QKV_DMA_SPREAD 2
#endif
constexpr int kTK = SB_QKV_TK;        // hidden elements per k-step (2 * kTK-byte tile rows)
constexpr int kStages = SB_QKV_STAGES;  // LDS ring depth: loads run kStages - 1 steps ahead
constexpr int kTileChunks = kTK / 8;  // 16-byte chunks per tile row
constexpr int kLoadRows = kQThreads / kTileChunks;  // tile rows one load of every thread fills
static_assert(kTK == 32 || kTK == 64, "tile rows of 64 or 128 bytes");
static_assert(kStages >= 2 && kStages <= 4, "the step waits cover rings of 2 to 4 stages");
constexpr int kGroup = SB_QKV_GROUP;  // row tiles per band of the tile order
constexpr int kXcds = 8;       // MI355X: workgroups go round-robin to 8 XCDs

// QKV_PARTIAL: the split form's product for small row counts, the hidden dimension split over
// grid.y (each slice's fp32 partial product to a workspace; qkv_epilogue_kernel sums the
// slices in order and runs the split form's epilogue).
enum QkvMode : int { QKV_SPLIT = 0, QKV_DENSE = 1, QKV_PARTIAL = 2 };

struct QkvArgs {
  const char* hidden;         // [S, hidden] rows
  int64_t h_s_row;            // bytes
  const char* weight;         // [F, hidden] rows
  int64_t w_s_row;            // bytes
  const char* bias;           // [F] in the input dtype, or nullptr
  const int32_t* positions;   // [R] hidden row (= sequence position) of each computed row
  const int32_t* count;       // device row count (overrides num_rows when smaller), or nullptr
  int64_t num_rows;           // R (grid bound)
  int64_t seq_len;            // hidden rows S
  int64_t k_steps;            // hidden / kTK
  int64_t num_features;       // F
  int64_t q_features;         // Hq * D
  int64_t kv_features;        // Hkv * D
  int head_dim;
  const float4* rope_cs;      // [R, D/4] of (cos, sin) pairs for pairs 2i, 2i+1, or nullptr
  char* out;                  // split: q_out [R, Hq*D] rows; dense: [S, F] rows
  int64_t o_s_row;            // bytes
  char* kv;                   // split: paged cache [NB, 2, Hkv, bs, D] under byte strides
  int64_t s_blk, s_kv, s_head, s_pos;
  const int32_t* block_table;
  int64_t block_size, nb_total, nb_per_seq;
  float* part;                // QKV_PARTIAL: [splits][R][F] fp32 partial products
  int64_t split_steps;        // QKV_PARTIAL: k-steps per slice of the hidden dimension
  int64_t splits;             // epilogue: slices to sum (0 or 1: one product)
};

// 16-byte chunk position of chunk c of tile row r. 256 bytes of banks hold 256 / (2 kTK)
// rows (4 for 64-byte rows, 2 for 128-byte rows); the XOR with r divided by that count
// spreads 16 consecutive rows read at one chunk over distinct bank groups, so the
// ds_read_b128 fragment reads are conflict-free.
__device__ __forceinline__ int qswz(int row, int chunk) {
  constexpr int shift = kTK == 32 ? 2 : 1;
  return chunk ^ ((row >> shift) & (kTileChunks - 1));
}

// s_waitcnt vmcnt(N) (6-bit count, split over bits 3:0 and 15:14), other counters untouched.
template <int N>
__device__ __forceinline__ void qkv_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}

// Tile of workgroup b. Workgroups are dispatched round-robin over the XCDs, so workgroup b
// runs on XCD b % 8; each XCD is given a contiguous range of the tile order, and the order
// walks bands of kGroup row tiles feature tile by feature tile, so the workgroups resident
// on one XCD at a time cover a compact block of feature x row tiles and share their W and
// hidden slices in that XCD's L2.
__device__ __forceinline__ void qkv_tile(int64_t b, int64_t n_ft, int64_t n_rt, int64_t* ft,
                                         int64_t* rt) {
  const int64_t total = n_ft * n_rt;
  const int64_t x = b % kXcds, i = b / kXcds;
  const int64_t per = total / kXcds, extra = total % kXcds;
  const int64_t q = x * per + min(x, extra) + i;
  const int64_t band = q / (kGroup * n_ft);
  const int64_t in_band = q - band * kGroup * n_ft;
  const int64_t rows_in_band = min<int64_t>(kGroup, n_rt - band * kGroup);
  *rt = band * kGroup + in_band % rows_in_band;
  *ft = in_band / rows_in_band;
}

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i's chunk lands at
// lds_wave + 16 i, lds_wave wave-uniform. Inline assembly so that the compiler does not order
// every later LDS read behind it; the kernel waits (vmcnt) before the barrier that publishes
// each stage.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void qkv_dma(const char* src, uint32_t lds_wave) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off"
      :
      : "s"(lds_wave), "v"(src)
      : "memory", "m0");
}
// LDS byte address of a pointer into a __shared__ array (wave-uniform arithmetic on it stays
// in scalar registers).
__device__ __forceinline__ uint32_t qkv_lds_addr(const void* p) {
  using lds_ptr = __attribute__((address_space(3))) const void*;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}
#pragma clang diagnostic pop

template <int DT>
__device__ __forceinline__ float qkv_elem(uint16_t h) {
  return DT == SB_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
// Two floats rounded to the input dtype (round to nearest even, one instruction per pair).
template <int DT>
__device__ __forceinline__ uint32_t qkv_pack2(float lo, float hi) {
  if (DT == SB_DTYPE_BF16) return pack2_bf16(lo, hi);
  return static_cast<uint32_t>(f32_to_f16(lo)) | (static_cast<uint32_t>(f32_to_f16(hi)) << 16);
}
// The same rounding without pack2_bf16's NaN canonicalisation (bf16: identical bits for every
// input but NaN; fp16 has none to drop). For callers that check for NaN separately.
template <int DT>
__device__ __forceinline__ uint32_t qkv_pack2_fast(float lo, float hi) {
  if (DT == SB_DTYPE_BF16) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
  }
  return qkv_pack2<DT>(lo, hi);
}

// cos / sin of every (computed row, rotary pair), correctly rounded to fp32 (fp64 sincos):
// entry e of row n = (cos, sin) of pairs 2e and 2e + 1, angle float(p) * inv_freq[pair];
// rows without a valid position get the identity. Layouts:
//   row-major (IL false)  table[n * D/4 + e], num_rows rows;
//   interleaved (IL true) table[((n / 32) * D/4 + e) * 32 + n % 32], rows padded to a
//   multiple of 32 (identity): the fused kernel's lanes hold 32 consecutive rows, so one
//   entry of all of them is 512 contiguous bytes.
template <bool IL>
__global__ void qkv_rope_table_kernel(const int32_t* positions, int64_t num_rows,
                                      int64_t seq_len, const float* inv_freq, int half_d,
                                      float4* table) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int quads = half_d / 2;
  const int64_t table_rows = IL ? (num_rows + 31) / 32 * 32 : num_rows;
  if (idx >= table_rows * quads) return;
  int64_t n;
  int k;
  if (IL) {
    const int64_t grp = idx / (32 * quads);
    const int64_t rem = idx - grp * 32 * quads;
    k = static_cast<int>(rem / 32);
    n = grp * 32 + (rem & 31);
  } else {
    n = idx / quads;
    k = static_cast<int>(idx - n * quads);
  }
  const int p = n < num_rows ? positions[n] : -1;
  float4 v = make_float4(1.f, 0.f, 1.f, 0.f);
  if (p >= 0 && p < seq_len) {
    sincos_rn(static_cast<float>(p) * inv_freq[2 * k], &v.y, &v.x);
    sincos_rn(static_cast<float>(p) * inv_freq[2 * k + 1], &v.w, &v.z);
  }
  table[idx] = v;
}

// The projection. Workgroup tile: TM = 64 BI features x TN = 64 BJ rows, 4 waves as 2 x 2,
// each wave BI x BJ MFMA blocks of 32 x 32 (BI = 4, BJ = 2..4: up to a 128 x 128 wave tile
// and 256 accumulators, one workgroup per CU; BI = BJ = 2: 64 x 64, two per CU).
template <int DT, int MODE, int BI, int BJ>
__global__ __launch_bounds__(kQThreads, BI * BJ > 4 ? 1 : 2) void qkv_mfma_kernel(QkvArgs a) {
  using vec8 = std::conditional_t<DT == SB_DTYPE_BF16, qbf16x8_t, qf16x8_t>;
  constexpr int TM = 64 * BI, TN = 64 * BJ;
  constexpr int LA = TM * kTileChunks / kQThreads;  // A loads per thread per stage (= BI)
  constexpr int LB = TN * kTileChunks / kQThreads;  // B loads per thread per stage (= BJ)
  constexpr int NKS = kTK / 16;                     // MFMA k-substeps per step
  // The LDS ring (A stages, then B stages); after the k loop it holds the output tile.
  __shared__ __align__(16) uint16_t smem[kStages * (TM + TN) * kTK];
  static_assert(TM * TN <= kStages * (TM + TN) * kTK, "output tile fits in the ring");
  auto As = [&](int stage) { return smem + stage * TM * kTK; };
  auto Bs = [&](int stage) { return smem + kStages * TM * kTK + stage * TN * kTK; };
  __shared__ int64_t brow[TN];   // byte offset of each tile row's hidden row
  __shared__ int bpos[TN];       // its position (-1: no row)
  __shared__ int64_t kvofs[TN];  // split: byte offset of its paged slot (-1: none)
  __shared__ __align__(16) float bias_s[TM];  // the tile's bias (0 without bias / past F)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
  const int lane = tid & 63, lq = lane & 31, lg = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t n_ft = (a.num_features + TM - 1) / TM;
  const int64_t n_rt = (a.num_rows + TN - 1) / TN;
  int64_t ft, rt;
  qkv_tile(blockIdx.x, n_ft, n_rt, &ft, &rt);
  const int64_t m0 = ft * TM;
  const int64_t n0 = rt * TN;
  int64_t rows = a.num_rows;
  if (a.count) rows = min(rows, static_cast<int64_t>(*a.count));
  if (n0 >= rows) return;  // uniform
  // This workgroup's k-steps: all of them, or (QKV_PARTIAL) slice blockIdx.y.
  int64_t kbeg = 0, nsteps = a.k_steps;
  if (MODE == QKV_PARTIAL) {
    kbeg = static_cast<int64_t>(blockIdx.y) * a.split_steps;
    nsteps = min(a.split_steps, a.k_steps - kbeg);
    if (nsteps <= 0) return;  // uniform
  }

  for (int t = tid; t < TN; t += kQThreads) {
    const int64_t n = n0 + t;
    int p = -1;
    if (n < rows) {
      p = a.positions[n];
      if (p < 0 || p >= a.seq_len) p = -1;
    }
    bpos[t] = p;
    brow[t] = static_cast<int64_t>(p < 0 ? 0 : p) * a.h_s_row;
    int64_t off = -1;
    if (MODE == QKV_SPLIT && p >= 0) {
      const int64_t lb = p / a.block_size;
      if (lb < a.nb_per_seq) {
        const int64_t pb = a.block_table[lb];
        if (pb >= 0 && pb < a.nb_total) off = pb * a.s_blk + (p - lb * a.block_size) * a.s_pos;
      }
    }
    kvofs[t] = off;
  }
  for (int t = tid; t < TM; t += kQThreads) {
    const int64_t f = m0 + t;
    bias_s[t] = (a.bias && f < a.num_features)
                    ? qkv_elem<DT>(reinterpret_cast<const uint16_t*>(a.bias)[f]) : 0.f;
  }
  __syncthreads();

  // DMA sources: slot s = q * 256 + tid of a stage holds tile row s / kTileChunks =
  // q * kLoadRows + tid / kTileChunks at position tid % kTileChunks, i.e. global chunk
  // qswz(row, tid % kTileChunks), which does not depend on q.
  const int chunk = qswz(tid / kTileChunks, tid % kTileChunks);
  const char* asrc[LA];
  const char* bsrc[LB];
#pragma unroll
  for (int q = 0; q < LA; ++q) {
    const int64_t f = min(m0 + q * kLoadRows + tid / kTileChunks, a.num_features - 1);
    asrc[q] = a.weight + f * a.w_s_row + 16 * chunk;
  }
#pragma unroll
  for (int q = 0; q < LB; ++q)
    bsrc[q] = a.hidden + brow[q * kLoadRows + tid / kTileChunks] + 16 * chunk;
  // Load q of a step (A loads first, then B), each 16 bytes per lane into its stage.
  auto issue_one = [&](int stage, int64_t kt, int q) {
    const int64_t ko = (kbeg + kt) * (kTK * 2);
    if (q < LA)
      qkv_dma(asrc[q] + ko, qkv_lds_addr(As(stage)) + (q * kQThreads + wave * 64) * 16);
    else
      qkv_dma(bsrc[q - LA] + ko,
              qkv_lds_addr(Bs(stage)) + ((q - LA) * kQThreads + wave * 64) * 16);
  };
  auto issue = [&](int stage, int64_t kt) {
#pragma unroll
    for (int q = 0; q < LA + LB; ++q) issue_one(stage, kt, q);
  };

  qf32x16_t acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Ring of kStages: step kt lives in stage kt % kStages; loads run kStages - 1 steps ahead.
  // One barrier per step both publishes step kt and retires step kt - 1, whose stage the
  // loads issued right after it refill.
#pragma unroll
  for (int s0 = 0; s0 < kStages - 1; ++s0)
    if (s0 < nsteps) issue(s0, s0);
  // Step kt; REFILL: whether it issues the loads of step kt + kStages - 1 (every step but
  // the last kStages - 1), a compile-time choice so that the loads need no branch.
  auto step = [&](int64_t kt, auto refill_c) {
    constexpr bool REFILL = decltype(refill_c)::value;
    const int st = static_cast<int>(kt % kStages);
    // Steps issued after this one: at most kStages - 2, fewer near the end; they may stay
    // in flight while step kt must have landed.
    const int64_t ahead = nsteps - 1 - kt;
    if (kStages >= 4 && ahead >= 2) qkv_wait_vm<2 * (LA + LB)>();
    else if (kStages >= 3 && ahead >= 1) qkv_wait_vm<LA + LB>();
    else qkv_wait_vm<0>();
    __syncthreads();
    const int rst = static_cast<int>((kt + kStages - 1) % kStages);
#if !SB_QKV_FRAG_PIPE
    if (REFILL) issue(rst, kt + kStages - 1);
#endif
    // Per k-substep: the wave's BI A and BJ B fragments, then BI x BJ MFMAs. The fragments
    // are double-buffered: those of substep ks + 1 are read while the MFMAs of substep ks
    // issue (scheduling barriers keep that order), so the LDS latency sits under BI x BJ
    // MFMAs instead of stalling the wave, the only one on its SIMD, before each of them.
    // The loads that refill the ring's free stage go out one after each MFMA.
    vec8 af[2][BI], bf[2][BJ];
    auto read_frags = [&](int ks, vec8* a_f, vec8* b_f) {
      const int c = 2 * ks + lg;
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const int r = wm * (32 * BI) + i * 32 + lq;
        a_f[i] = *reinterpret_cast<const vec8*>(As(st) + r * kTK + 8 * qswz(r, c));
      }
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const int r = wn * (32 * BJ) + j * 32 + lq;
        b_f[j] = *reinterpret_cast<const vec8*>(Bs(st) + r * kTK + 8 * qswz(r, c));
      }
    };
    read_frags(0, af[0], bf[0]);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#if SB_QKV_FRAG_PIPE
      if (ks + 1 < NKS) read_frags(ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#endif
      const vec8* a_f = af[ks & 1];
      const vec8* b_f = bf[ks & 1];
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int j = 0; j < BJ; ++j) {
          if (DT == SB_DTYPE_BF16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_f[i], b_f[j], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_f[i], b_f[j], acc[i][j], 0, 0, 0);
#if SB_QKV_FRAG_PIPE
          constexpr int kSpread = SB_QKV_DMA_SPREAD < NKS ? SB_QKV_DMA_SPREAD : NKS;
          constexpr int kPer = (LA + LB + kSpread - 1) / kSpread;  // loads per substep
          static_assert(kPer <= BI * BJ, "every load follows an MFMA of its substep");
          const int q = ks * kPer + i * BJ + j;
          if (REFILL && i * BJ + j < kPer && q < LA + LB) {
            issue_one(rst, kt + kStages - 1, q);
            __builtin_amdgcn_sched_barrier(0);
          }
#endif
        }
#if SB_QKV_FRAG_PIPE
      __builtin_amdgcn_sched_barrier(0);
#else
      if (ks + 1 < NKS) read_frags(ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
#endif
    }
  };
  {
    int64_t kt = 0;
    for (; kt + kStages - 1 < nsteps; ++kt) step(kt, std::true_type{});
    for (; kt < nsteps; ++kt) step(kt, std::false_type{});
  }

  if constexpr (MODE == QKV_PARTIAL) {
    // The slice's fp32 product: lane (lq, lg) of block (i, j) holds row wn*32*BJ + 32j + lq,
    // features wm*32*BI + 32i + 8g + 4lg .. +3 in register group g.
    float* pp = a.part + static_cast<int64_t>(blockIdx.y) * a.num_rows * a.num_features;
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int64_t n = n0 + wn * (32 * BJ) + j * 32 + lq;
      if (n >= rows) continue;
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t f = m0 + wm * (32 * BI) + i * 32 + 8 * g + 4 * lg;
          if (f < a.num_features)
            *reinterpret_cast<float4*>(pp + n * a.num_features + f) =
                make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                            acc[i][j][4 * g + 3]);
        }
    }
    return;
  }

  // Epilogue, phase 1: lane (lq, lg) of block (i, j) holds tile row wn*32*BJ + 32j + lq and,
  // in register group g, tile features wm*32*BI + 32i + 8g + 4lg .. +3. Bias, RoPE and the
  // rounding happen in registers; the rounded tile goes to LDS as [TN rows][TM features],
  // 8-byte units of row r XOR-swizzled by 2 (r % 16) so that the 32 rows a wave writes at
  // once spread over the banks (and 16-byte pairs of units stay adjacent for phase 2).
  // Feature indices fit 32 bits (F = (Hq + 2 Hkv) D): the head arithmetic below is unsigned
  // 32-bit and hoisted out of the row loops (64-bit divisions by a run-time head_dim expand to
  // long instruction sequences, and this part runs one wave per SIMD).
  const uint32_t kf0 = static_cast<uint32_t>(a.q_features);
  const uint32_t vf0 = static_cast<uint32_t>(a.q_features + a.kv_features);
  const uint32_t hd = static_cast<uint32_t>(a.head_dim);
  const int quads = a.head_dim / 4;
  // Table entry (within a row's D/4) of register group (i, g): Q and K features rotate by
  // their offset within the head. Whether a group rotates (Q or K, not V or past F) depends
  // on its 8-feature block only (head_dim and F are multiples of 8), so it is wave-uniform:
  // computed from scalar values, it makes a scalar branch.
  int tq[BI][4];
  bool rot_g[BI][4];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t fb = static_cast<uint32_t>(m0) + wm * (32 * BI) + i * 32 + 8 * g;
      const uint32_t f0 = fb + 4 * lg;
      rot_g[i][g] = fb < vf0;
      tq[i][g] = fb < vf0 ? static_cast<int>(((f0 < kf0 ? f0 : f0 - kf0) % hd) / 4) : 0;
    }
  // This lane's row in the interleaved table (entry e at row_cs[j][32 e]): block j holds 32
  // consecutive rows from a multiple of 32; groups past the last row are clamped to it (rows
  // past the count, and rows without a position, are never stored, so whatever they are
  // rotated by does not matter).
  const float4* row_cs[BJ];
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const int64_t grp = min((n0 + wn * (32 * BJ) + j * 32) / 32, (rows - 1) / 32);
    row_cs[j] = a.rope_cs ? a.rope_cs + grp * quads * 32 + lq : nullptr;
  }
  __syncthreads();  // every wave is done with the last stage
  // Group (i, g) by group: bias, RoPE, rounding. The table entries of block i + 1 are loaded
  // while block i is processed (one table round trip per block would otherwise serialise the
  // epilogue). The fast pass packs without NaN canonicalisation and sums every value into a
  // probe (NaN if any value is NaN, or +inf meets -inf); a wave whose probe is NaN anywhere
  // runs the pass again with exact NaN bits (it rewrites the same LDS words).
  auto phase1 = [&](auto exact_c, auto rope_c) {
    constexpr bool EXACT = decltype(exact_c)::value;
    constexpr bool ROPE = decltype(rope_c)::value;
    float probe = 0.f;
    constexpr int kAhead = SB_QKV_CS_AHEAD;  // blocks of table entries in flight
    float4 cs[kAhead + 1][4][BJ];
    auto load_cs = [&](int i, float4 (&dst)[4][BJ]) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < BJ; ++j) dst[g][j] = row_cs[j][32 * tq[i][g]];
    };
    if (ROPE) {
#pragma unroll
      for (int i = 0; i < kAhead && i < BI; ++i) load_cs(i, cs[i % (kAhead + 1)]);
    }
#pragma unroll
    for (int i = 0; i < BI; ++i) {
      if (ROPE && i + kAhead < BI) load_cs(i + kAhead, cs[(i + kAhead) % (kAhead + 1)]);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int fl = wm * (32 * BI) + i * 32 + 8 * g + 4 * lg;  // tile feature
        const float4 b = *reinterpret_cast<const float4*>(&bias_s[fl]);
        float v[BJ][4];
#pragma unroll
        for (int j = 0; j < BJ; ++j) {
          v[j][0] = acc[i][j][4 * g] + b.x;
          v[j][1] = acc[i][j][4 * g + 1] + b.y;
          v[j][2] = acc[i][j][4 * g + 2] + b.z;
          v[j][3] = acc[i][j][4 * g + 3] + b.w;
        }
        if (ROPE && rot_g[i][g]) {
#pragma unroll
          for (int j = 0; j < BJ; ++j) {
            const float4 c = cs[i % (kAhead + 1)][g][j];
            float ev = v[j][0], od = v[j][1];
            v[j][0] = ev * c.x - od * c.y;
            v[j][1] = ev * c.y + od * c.x;
            ev = v[j][2];
            od = v[j][3];
            v[j][2] = ev * c.z - od * c.w;
            v[j][3] = ev * c.w + od * c.z;
          }
        }
#pragma unroll
        for (int j = 0; j < BJ; ++j) {
          const int tr = wn * (32 * BJ) + j * 32 + lq;
          uint2 w;
          if (EXACT) {
            w.x = qkv_pack2<DT>(v[j][0], v[j][1]);
            w.y = qkv_pack2<DT>(v[j][2], v[j][3]);
          } else {
            w.x = qkv_pack2_fast<DT>(v[j][0], v[j][1]);
            w.y = qkv_pack2_fast<DT>(v[j][2], v[j][3]);
            probe += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
          }
          *reinterpret_cast<uint2*>(smem + tr * TM + 4 * ((fl / 4) ^ (2 * (tr & 15)))) = w;
        }
      }
    }
    return probe;
  };
  auto run_phase1 = [&](auto exact_c) {
    if (MODE != QKV_DENSE && a.rope_cs) return phase1(exact_c, std::true_type{});
    return phase1(exact_c, std::false_type{});
  };
  const float probe = run_phase1(std::false_type{});
  if (DT == SB_DTYPE_BF16 && __builtin_amdgcn_ballot_w64(probe != probe) != 0)
    run_phase1(std::true_type{});
  __syncthreads();

  // Phase 2: 16-byte chunks (8 features) of each tile row to their destination, consecutive
  // threads along a row: Q / dense rows and K / V head rows are contiguous, so the stores
  // coalesce. Chunks never straddle a head (head_dim % 8 == 0).
  // Each thread keeps one chunk column c (kQThreads is a multiple of CPR), so its feature
  // range, destination (Q / dense, K or V) and head offset are fixed for all its rows.
  constexpr int CPR = TM / 8;  // chunks per tile row
  static_assert(kQThreads % CPR == 0, "a thread keeps one chunk column");
  const int c = tid % CPR;
  const uint32_t f0 = static_cast<uint32_t>(m0) + 8 * c;
  if (f0 >= static_cast<uint32_t>(a.num_features)) return;
  int64_t kv_off = 0;  // K / V: plane + head + in-head byte offset of this chunk
  if (MODE != QKV_DENSE && f0 >= kf0) {
    const bool is_v = f0 >= vf0;
    const uint32_t rf = f0 - (is_v ? vf0 : kf0);
    const uint32_t h = rf / hd;
    kv_off = (is_v ? a.s_kv : 0) + static_cast<int64_t>(h) * a.s_head + 2 * (rf - h * hd);
  }
  for (int tr = tid / CPR; tr < TN; tr += kQThreads / CPR) {
    const int64_t n = n0 + tr;
    if (n >= rows) break;  // rows ascend with tr
    const int p = bpos[tr];
    uint4 w = *reinterpret_cast<const uint4*>(smem + tr * TM + 4 * ((2 * c) ^ (2 * (tr & 15))));
    if (MODE == QKV_DENSE) {
      if (p >= 0) *reinterpret_cast<uint4*>(a.out + p * a.o_s_row + 2 * f0) = w;
    } else if (f0 < kf0) {
      if (p < 0) w = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(a.out + n * a.o_s_row + 2 * f0) = w;
    } else {
      const int64_t slot = kvofs[tr];
      if (slot >= 0) *reinterpret_cast<uint4*>(a.kv + slot + kv_off) = w;
    }
  }
}

// Row gather for a library GEMM, plus the RoPE table in the same launch: threads
// [0, R * hidden / 8) copy 16-byte chunks of hidden row positions[n] to xg[n] (rows without
// a valid position are zero); the next R * D / 4 threads fill table entries as
// the row-major qkv_rope_table_kernel does.
__global__ __launch_bounds__(256) void qkv_gather_kernel(char* xg, const char* hidden,
                                                         int64_t h_s_row, int64_t hidden_dim,
                                                         const int32_t* positions,
                                                         int64_t num_rows, int64_t seq_len,
                                                         const float* inv_freq, int half_d,
                                                         float4* table) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t cpr = hidden_dim / 8;  // 16-byte chunks of a bf16 / fp16 row
  const int64_t n_copy = num_rows * cpr;
  if (idx < n_copy) {
    const int64_t n = idx / cpr;
    const int64_t c = idx - n * cpr;
    const int p = positions[n];
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (p >= 0 && p < seq_len) v = *reinterpret_cast<const uint4*>(hidden + p * h_s_row + 16 * c);
    *reinterpret_cast<uint4*>(xg + n * hidden_dim * 2 + 16 * c) = v;
    return;
  }
  if (!table) return;
  const int64_t t = idx - n_copy;
  const int quads = half_d / 2;
  if (t >= num_rows * quads) return;
  const int64_t n = t / quads;
  const int k = static_cast<int>(t - n * quads);
  const int p = positions[n];
  float4 v = make_float4(1.f, 0.f, 1.f, 0.f);
  if (p >= 0 && p < seq_len) {
    sincos_rn(static_cast<float>(p) * inv_freq[2 * k], &v.y, &v.x);
    sincos_rn(static_cast<float>(p) * inv_freq[2 * k + 1], &v.w, &v.z);
  }
  table[t] = v;
}

// Epilogue of a projection computed elsewhere (a library GEMM with fp32 output): for row n
// and the 8 features [f0, f0 + 8) of one thread, out = proj[n, f] + bias[f], Q and K rotated
// by the row's position from the same (cos, sin) table as the fused kernel, one rounding to
// the input dtype, then Q to q_out[n] and K / V to the paged slot of positions[n] (rows
// without a valid position: Q zero, no K / V write). Same results as the fused kernel's
// epilogue on the same fp32 products.
template <int DT>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(QkvArgs a, const float* proj,
                                                           int64_t p_s_row) {
  // Index arithmetic in unsigned 32 bits (the host bounds R * F / 8 below 2^31; features,
  // positions and block sizes fit): 64-bit divisions by run-time values expand to long call
  // sequences.
  const uint32_t cpr = static_cast<uint32_t>(a.num_features / 8);  // 8-feature chunks per row
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= static_cast<uint64_t>(a.num_rows) * cpr) return;
  const uint32_t n32 = idx / cpr;
  const int64_t n = n32;
  const uint32_t f0 = (idx - n32 * cpr) * 8;
  const int p = a.positions[n];
  const bool valid = p >= 0 && p < a.seq_len;
  const uint32_t kf0 = static_cast<uint32_t>(a.q_features);
  const uint32_t vf0 = static_cast<uint32_t>(a.q_features + a.kv_features);
  const uint32_t hd = static_cast<uint32_t>(a.head_dim);
  int64_t slot = -1;
  if (f0 >= kf0) {
    if (!valid) return;
    const uint32_t bs = static_cast<uint32_t>(a.block_size);
    const uint32_t lb = static_cast<uint32_t>(p) / bs;
    if (lb >= a.nb_per_seq) return;
    const int64_t pb = a.block_table[lb];
    if (pb < 0 || pb >= a.nb_total) return;
    slot = pb * a.s_blk + static_cast<int64_t>(static_cast<uint32_t>(p) - lb * bs) * a.s_pos;
  }
  uint4 w = make_uint4(0u, 0u, 0u, 0u);
  if (valid) {
    const float4* src = reinterpret_cast<const float4*>(proj + n * p_s_row + f0);
    const float4 x0 = src[0], x1 = src[1];
    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    // Slices of a split product, summed in slice order.
    for (int64_t sl = 1; sl < a.splits; ++sl) {
      const float4* ps = reinterpret_cast<const float4*>(proj + sl * a.num_rows * p_s_row +
                                                         n * p_s_row + f0);
      const float4 y0 = ps[0], y1 = ps[1];
      v[0] += y0.x; v[1] += y0.y; v[2] += y0.z; v[3] += y0.w;
      v[4] += y1.x; v[5] += y1.y; v[6] += y1.z; v[7] += y1.w;
    }
    if (a.bias) {
      const uint16_t* b = reinterpret_cast<const uint16_t*>(a.bias) + f0;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += qkv_elem<DT>(b[e]);
    }
    if (a.rope_cs && f0 < vf0) {
      const uint32_t rf = f0 - (f0 < kf0 ? 0 : kf0);
      const uint32_t d0 = rf % hd;  // multiple of 8: two table entries
      const int quads = a.head_dim / 4;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 c = a.rope_cs[n * quads + d0 / 4 + h];
        float ev = v[4 * h], od = v[4 * h + 1];
        v[4 * h] = ev * c.x - od * c.y;
        v[4 * h + 1] = ev * c.y + od * c.x;
        ev = v[4 * h + 2];
        od = v[4 * h + 3];
        v[4 * h + 2] = ev * c.z - od * c.w;
        v[4 * h + 3] = ev * c.w + od * c.z;
      }
    }
    w.x = qkv_pack2<DT>(v[0], v[1]);
    w.y = qkv_pack2<DT>(v[2], v[3]);
    w.z = qkv_pack2<DT>(v[4], v[5]);
    w.w = qkv_pack2<DT>(v[6], v[7]);
  }
  if (f0 < kf0) {
    *reinterpret_cast<uint4*>(a.out + n * a.o_s_row + 2 * f0) = w;
  } else {
    const bool is_v = f0 >= vf0;
    const uint32_t rf = f0 - (is_v ? vf0 : kf0);
    const uint32_t h = rf / hd;
    *reinterpret_cast<uint4*>(a.kv + slot + (is_v ? a.s_kv : 0) +
                              static_cast<int64_t>(h) * a.s_head + 2 * (rf - h * hd)) = w;
  }
}

// Checks shared by both entries; fills the operand part of QkvArgs.
int qkv_common(const char* fn, QkvArgs* a, const void* hidden, const void* weight,
               const void* bias, int64_t seq_len, int64_t hidden_dim, int64_t num_features,
               int64_t hidden_stride, int64_t weight_stride, int32_t dtype) {
  if (dtype != SB_DTYPE_BF16 && dtype != SB_DTYPE_F16)
    return fail(fn, "dtype must be bf16 or fp16 (the MFMA path)");
  if (!hidden || !weight) return fail(fn, "null pointer argument");
  // Rows without a valid position still load hidden row 0 (their results are not stored).
  if (seq_len < 1) return fail(fn, "seq_len must be positive");
  if (hidden_dim <= 0 || hidden_dim % 64 != 0)
    return fail(fn, "hidden size must be a positive multiple of 64");
  if (num_features <= 0 || num_features % 8 != 0)
    return fail(fn, "output features must be a positive multiple of 8");
  if (reinterpret_cast<uintptr_t>(hidden) % 16 || reinterpret_cast<uintptr_t>(weight) % 16 ||
      (hidden_stride * 2) % 16 || (weight_stride * 2) % 16)
    return fail(fn, "hidden and weight rows must be 16-byte aligned");
  if (bias && reinterpret_cast<uintptr_t>(bias) % 8) return fail(fn, "bias must be 8-byte aligned");
  a->hidden = static_cast<const char*>(hidden);
  a->h_s_row = hidden_stride * 2;
  a->weight = static_cast<const char*>(weight);
  a->w_s_row = weight_stride * 2;
  a->bias = static_cast<const char*>(bias);
  a->seq_len = seq_len;
  a->k_steps = hidden_dim / kTK;
  a->num_features = num_features;
  return SB_OK;
}

// Tile shape. 256 features x 64 BJ rows (one workgroup per CU) with BJ in {3, 2} chosen to
// minimise the work of the busiest CU, rounds x BJ (ties: larger tiles); 128 x 128 (two per
// CU) when the big tiles leave more than half the CUs idle, or leave some idle while the
// small ones fit one round of two per CU. (BJ = 4 spilled 5-6 VGPRs and never cost less than
// BJ = 2 in this model: at most a tie.) When even the 128 x 128 tiles number fewer than the
// CUs (a few hundred rows at the 7B shape), the split form also splits the hidden dimension
// over grid.y, into slices of at least kMinSplitSteps k-steps (QKV_PARTIAL and the summing
// epilogue). Qwen2.5-7B shape (3584 -> 4608 features), graph replays on one box, interleaved:
// slices of at least 12 steps 28-30 us at 64 rows (6 steps: 32 us, 19: 35 us), 30.5 us at 128
// and 35.5 us at 256 (library 28, 33, 46 us); small tiles from 1024 to 1536 rows 61-72 us
// against 75-77 us with the 256-feature tiles, which stay faster from 2048 rows (97 against
// 113 us).
constexpr int64_t kCus = 256;
#ifndef SB_QKV_MIN_SPLIT_STEPS
#define SB_QKV_MIN_SPLIT_STEPS 12
#endif
constexpr int64_t kMinSplitSteps = SB_QKV_MIN_SPLIT_STEPS;
struct QkvPlan {
  int bj = 0;               // 3 or 2: 256 x 64 bj tiles; 0: 128 x 128 tiles
  int64_t tiles = 0;
  int64_t splits = 1;       // slices of the hidden dimension (> 1: QKV_PARTIAL)
  int64_t split_steps = 0;  // k-steps per slice
};
QkvPlan qkv_plan(int64_t rows, int64_t features, int64_t k_steps, bool allow_split) {
  QkvPlan pl;
  const int64_t nft = (features + 255) / 256;
  int64_t best = 0;
  for (int c = 3; c >= 2; --c) {
    const int64_t t = nft * ((rows + 64 * c - 1) / (64 * c));
    const int64_t cost = ((t + kCus - 1) / kCus) * c;
    if (pl.bj == 0 || cost < best) {
      pl.bj = c;
      best = cost;
      pl.tiles = t;
    }
  }
  const int64_t small = ((features + 127) / 128) * ((rows + 127) / 128);
  if (pl.tiles * 2 < kCus || (pl.tiles < kCus && small <= 2 * kCus)) {
    pl.bj = 0;  // small tiles
    pl.tiles = small;
    if (allow_split && pl.tiles > 0 && pl.tiles < kCus) {
      const int64_t s = std::min<int64_t>((2 * kCus) / pl.tiles, k_steps / kMinSplitSteps);
      if (s > 1) {
        pl.split_steps = (k_steps + s - 1) / s;
        pl.splits = (k_steps + pl.split_steps - 1) / pl.split_steps;
      }
    }
  }
  return pl;
}

template <int MODE>
int launch_qkv(const char* fn, const QkvArgs& a, int32_t dtype, hipStream_t st,
               const QkvPlan& pl) {
  if (pl.tiles > 0x7fffffff || pl.splits > 65535) return fail(fn, "grid too large");
  const dim3 grid(static_cast<unsigned>(pl.tiles),
                  static_cast<unsigned>(MODE == QKV_PARTIAL ? pl.splits : 1));
  const int bj = pl.bj;
#define SB_QKV_CASE(DT, BI, BJ)                                                              \
  SB_LAUNCH("qkv_mfma", (qkv_mfma_kernel<DT, MODE, BI, BJ>), grid, dim3(kQThreads), st, a)
#define SB_QKV_DT(DT)                   \
  switch (bj) {                         \
    case 3: SB_QKV_CASE(DT, 4, 3); break; \
    case 2: SB_QKV_CASE(DT, 4, 2); break; \
    default: SB_QKV_CASE(DT, 2, 2); break; \
  }
  if (dtype == SB_DTYPE_BF16) {
    SB_QKV_DT(SB_DTYPE_BF16)
  } else {
    SB_QKV_DT(SB_DTYPE_F16)
  }
#undef SB_QKV_DT
#undef SB_QKV_CASE
  return check_launch(fn);
}

// The summing epilogue of a split product (and the library form's epilogue): one thread per
// 8 features of a row.
int launch_qkv_epilogue(const char* fn, const QkvArgs& a, const float* proj, int64_t p_s_row,
                        int32_t dtype, hipStream_t st) {
  const int64_t threads = a.num_rows * (a.num_features / 8);
  if (threads + 255 >= (int64_t{1} << 31)) return fail(fn, "grid too large");  // 32-bit indices
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (dtype == SB_DTYPE_BF16)
    SB_LAUNCH("qkv_epilogue", qkv_epilogue_kernel<SB_DTYPE_BF16>, grid, dim3(256), st, a, proj,
              p_s_row);
  else
    SB_LAUNCH("qkv_epilogue", qkv_epilogue_kernel<SB_DTYPE_F16>, grid, dim3(256), st, a, proj,
              p_s_row);
  return check_launch(fn);
}

// Workspace of the split form: the RoPE table first, then (split product) the slices.
constexpr int64_t kQkvWsAlign = 256;
int64_t qkv_table_bytes(int64_t num_rows, int64_t head_dim, bool rope) {
  // Rows padded to a multiple of 32 (the interleaved layout; the row-major one fits too).
  const int64_t rows = (num_rows + 31) / 32 * 32;
  const int64_t t = rope ? rows * head_dim * static_cast<int64_t>(sizeof(float)) : 0;
  return (t + kQkvWsAlign - 1) / kQkvWsAlign * kQkvWsAlign;
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int64_t sb_qkv_projection_paged_workspace_size(int64_t num_rows, int64_t num_q_heads,
                                                         int64_t num_kv_heads, int64_t head_dim,
                                                         int64_t hidden_dim, int32_t rope) {
  if (num_rows <= 0 || num_q_heads <= 0 || num_kv_heads < 0 || head_dim <= 0 || hidden_dim <= 0)
    return 0;
  const int64_t features = (num_q_heads + 2 * num_kv_heads) * head_dim;
  const QkvPlan pl = qkv_plan(num_rows, features, hidden_dim / kTK, true);
  const int64_t part = pl.splits > 1 ? pl.splits * num_rows * features * 4 : 0;
  return qkv_table_bytes(num_rows, head_dim, rope != 0) + part;
}

extern "C" int sb_qkv_projection_paged(
    void* q_out, const void* hidden, const void* weight, const void* bias,
    const int32_t* positions, int64_t num_rows, int64_t seq_len, int64_t hidden_dim,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, const float* inv_freq,
    void* workspace, int64_t workspace_bytes, void* kv_cache, const int32_t* block_table, int64_t block_size, int64_t num_blocks_total,
    int64_t num_blocks_per_seq, int64_t hidden_stride, int64_t weight_stride, int64_t q_stride,
    const int64_t* kv_strides, int32_t dtype, void* stream) {
  const char* fn = "sb_qkv_projection_paged";
  clear_error();
  if (num_rows == 0) return SB_OK;
  if (num_rows < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(fn, "invalid sizes");
  if (head_dim % 8 != 0) return fail(fn, "head_dim must be a multiple of 8");
  if (!q_out || !positions || !kv_cache || !block_table || !kv_strides)
    return fail(fn, "null pointer argument");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (kv_strides[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  QkvArgs a{};
  const int64_t qf = num_q_heads * head_dim, kvf = num_kv_heads * head_dim;
  int rc = qkv_common(fn, &a, hidden, weight, bias, seq_len, hidden_dim, qf + 2 * kvf,
                      hidden_stride, weight_stride, dtype);
  if (rc) return rc;
  if (reinterpret_cast<uintptr_t>(q_out) % 16 || (q_stride * 2) % 16 ||
      reinterpret_cast<uintptr_t>(kv_cache) % 16 || (kv_strides[0] * 2) % 16 ||
      (kv_strides[1] * 2) % 16 || (kv_strides[2] * 2) % 16 || (kv_strides[3] * 2) % 16)
    return fail(fn, "q_out and cache rows must be 16-byte aligned");
  a.positions = positions;
  a.num_rows = num_rows;
  a.q_features = qf;
  a.kv_features = kvf;
  a.head_dim = static_cast<int>(head_dim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const QkvPlan pl = qkv_plan(num_rows, a.num_features, a.k_steps, true);
  const int64_t ws_need = sb_qkv_projection_paged_workspace_size(
      num_rows, num_q_heads, num_kv_heads, head_dim, hidden_dim, inv_freq ? 1 : 0);
  if (ws_need > 0) {
    if (!workspace || reinterpret_cast<uintptr_t>(workspace) % 16)
      return fail(fn, "RoPE and the split product need a 16-byte aligned workspace");
    if (workspace_bytes < ws_need) return fail(fn, "workspace too small");
  }
  if (inv_freq) {
    // The fused kernel reads the interleaved layout, the split product's epilogue kernel the
    // row-major one.
    float4* table = static_cast<float4*>(workspace);
    const int64_t n = (num_rows + 31) / 32 * 32 * (head_dim / 4);
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (pl.splits > 1)
      SB_LAUNCH("qkv_rope_table", qkv_rope_table_kernel<false>, grid, dim3(256), st, positions,
                num_rows, seq_len, inv_freq, static_cast<int>(head_dim / 2), table);
    else
      SB_LAUNCH("qkv_rope_table", qkv_rope_table_kernel<true>, grid, dim3(256), st, positions,
                num_rows, seq_len, inv_freq, static_cast<int>(head_dim / 2), table);
    rc = check_launch(fn);
    if (rc) return rc;
    a.rope_cs = table;
  }
  a.out = static_cast<char*>(q_out);
  a.o_s_row = q_stride * 2;
  a.kv = static_cast<char*>(kv_cache);
  a.s_blk = kv_strides[0] * 2;
  a.s_kv = kv_strides[1] * 2;
  a.s_head = kv_strides[2] * 2;
  a.s_pos = kv_strides[3] * 2;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  if (pl.splits > 1) {
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      qkv_table_bytes(num_rows, head_dim, inv_freq != nullptr));
    a.split_steps = pl.split_steps;
    rc = launch_qkv<QKV_PARTIAL>(fn, a, dtype, st, pl);
    if (rc) return rc;
    a.splits = pl.splits;
    return launch_qkv_epilogue(fn, a, a.part, a.num_features, dtype, st);
  }
  return launch_qkv<QKV_SPLIT>(fn, a, dtype, st, pl);
}

extern "C" int sb_qkv_gather_rows(void* xg, const void* hidden, const int32_t* positions,
                                  int64_t num_rows, int64_t seq_len, int64_t hidden_dim,
                                  int64_t hidden_stride, const float* inv_freq,
                                  int64_t head_dim, void* rope_table, int32_t dtype,
                                  void* stream) {
  const char* fn = "sb_qkv_gather_rows";
  clear_error();
  if (num_rows == 0) return SB_OK;
  if (dtype != SB_DTYPE_BF16 && dtype != SB_DTYPE_F16) return fail(fn, "dtype must be bf16 or fp16");
  if (!xg || !hidden || !positions) return fail(fn, "null pointer argument");
  if (num_rows < 0 || hidden_dim <= 0 || hidden_dim % 8 != 0)
    return fail(fn, "hidden size must be a positive multiple of 8");
  if (reinterpret_cast<uintptr_t>(xg) % 16 || reinterpret_cast<uintptr_t>(hidden) % 16 ||
      (hidden_stride * 2) % 16)
    return fail(fn, "rows must be 16-byte aligned");
  if (inv_freq && (!rope_table || reinterpret_cast<uintptr_t>(rope_table) % 16 ||
                   head_dim <= 0 || head_dim % 4 != 0))
    return fail(fn, "RoPE needs a 16-byte aligned table and head_dim a multiple of 4");
  const int64_t threads = num_rows * (hidden_dim / 8) + (inv_freq ? num_rows * (head_dim / 4) : 0);
  if ((threads + 255) / 256 > 0x7fffffff) return fail(fn, "grid too large");
  SB_LAUNCH("qkv_gather", qkv_gather_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
            dim3(256), static_cast<hipStream_t>(stream), static_cast<char*>(xg),
            static_cast<const char*>(hidden), hidden_stride * 2, hidden_dim, positions, num_rows,
            seq_len, inv_freq, static_cast<int>(head_dim / 2),
            inv_freq ? static_cast<float4*>(rope_table) : nullptr);
  return check_launch(fn);
}

extern "C" int sb_qkv_epilogue_paged(
    void* q_out, const float* proj, const void* bias, const int32_t* positions,
    int64_t num_rows, int64_t seq_len, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, const void* rope_table, void* kv_cache, const int32_t* block_table,
    int64_t block_size, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    int64_t proj_stride, int64_t q_stride, const int64_t* kv_strides, int32_t dtype,
    void* stream) {
  const char* fn = "sb_qkv_epilogue_paged";
  clear_error();
  if (num_rows == 0) return SB_OK;
  if (dtype != SB_DTYPE_BF16 && dtype != SB_DTYPE_F16) return fail(fn, "dtype must be bf16 or fp16");
  if (num_rows < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(fn, "invalid sizes");
  if (head_dim % 8 != 0) return fail(fn, "head_dim must be a multiple of 8");
  if (!q_out || !proj || !positions || !kv_cache || !block_table || !kv_strides)
    return fail(fn, "null pointer argument");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (kv_strides[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t qf = num_q_heads * head_dim, kvf = num_kv_heads * head_dim;
  if (proj_stride < qf + 2 * kvf) return fail(fn, "projection rows shorter than the features");
  if (reinterpret_cast<uintptr_t>(proj) % 16 || (proj_stride * 4) % 16 ||
      reinterpret_cast<uintptr_t>(q_out) % 16 || (q_stride * 2) % 16 ||
      reinterpret_cast<uintptr_t>(kv_cache) % 16 || (kv_strides[0] * 2) % 16 ||
      (kv_strides[1] * 2) % 16 || (kv_strides[2] * 2) % 16 || (kv_strides[3] * 2) % 16 ||
      reinterpret_cast<uintptr_t>(rope_table) % 16)
    return fail(fn, "projection, q_out, cache rows and table must be 16-byte aligned");
  if (bias && reinterpret_cast<uintptr_t>(bias) % 2) return fail(fn, "misaligned bias");
  QkvArgs a{};
  a.bias = static_cast<const char*>(bias);
  a.positions = positions;
  a.num_rows = num_rows;
  a.seq_len = seq_len;
  a.num_features = qf + 2 * kvf;
  a.q_features = qf;
  a.kv_features = kvf;
  a.head_dim = static_cast<int>(head_dim);
  a.rope_cs = static_cast<const float4*>(rope_table);
  a.out = static_cast<char*>(q_out);
  a.o_s_row = q_stride * 2;
  a.kv = static_cast<char*>(kv_cache);
  a.s_blk = kv_strides[0] * 2;
  a.s_kv = kv_strides[1] * 2;
  a.s_head = kv_strides[2] * 2;
  a.s_pos = kv_strides[3] * 2;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  return launch_qkv_epilogue(fn, a, proj, proj_stride, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int64_t sb_masked_qkv_projection_workspace_size(int64_t seq_len) {
  return (seq_len + 1) * static_cast<int64_t>(sizeof(int32_t));
}

extern "C" int sb_masked_qkv_projection(void* out, const void* hidden, const void* weight,
                                        const void* bias, const uint8_t* compute_mask,
                                        void* workspace, int64_t workspace_bytes,
                                        int64_t seq_len, int64_t hidden_dim,
                                        int64_t out_features, int64_t hidden_stride,
                                        int64_t weight_stride, int64_t out_stride,
                                        int32_t dtype, void* stream) {
  const char* fn = "sb_masked_qkv_projection";
  clear_error();
  if (seq_len == 0) return SB_OK;
  if (seq_len < 0) return fail(fn, "invalid sizes");
  if (!out || !compute_mask || !workspace) return fail(fn, "null pointer argument");
  if (workspace_bytes < sb_masked_qkv_projection_workspace_size(seq_len))
    return fail(fn, "workspace too small");
  QkvArgs a{};
  int rc = qkv_common(fn, &a, hidden, weight, bias, seq_len, hidden_dim, out_features,
                      hidden_stride, weight_stride, dtype);
  if (rc) return rc;
  if (reinterpret_cast<uintptr_t>(out) % 16 || (out_stride * 2) % 16)
    return fail(fn, "output rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* pos = static_cast<int32_t*>(workspace);
  // Reuse rows are zero (the reference multiplies them by the mask); computed rows are
  // written by the projection.
  const int vpr = static_cast<int>(out_features * 2 / 8);
  const int64_t total = seq_len * vpr;
  SB_LAUNCH("zero_rows", zero_rows_kernel<8>, dim3(static_cast<unsigned>((total + 255) / 256)),
            dim3(256), st, static_cast<char*>(out), compute_mask, int64_t{1}, seq_len,
            int64_t{0}, out_stride * 2, vpr);
  SB_LAUNCH("mask_compact", mask_compact_kernel<0>, dim3(1), dim3(1024), st, compute_mask,
            seq_len, pos, pos + seq_len);
  rc = check_launch(fn);
  if (rc) return rc;
  a.positions = pos;
  a.count = pos + seq_len;
  a.num_rows = seq_len;
  a.q_features = out_features;  // every feature goes to the dense row; no RoPE
  a.kv_features = 0;
  a.head_dim = 8;
  a.out = static_cast<char*>(out);
  a.o_s_row = out_stride * 2;
  return launch_qkv<QKV_DENSE>(fn, a, dtype, st, qkv_plan(a.num_rows, a.num_features, a.k_steps, false));
}
