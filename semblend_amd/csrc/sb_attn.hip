// Partial-prefill attention for gfx950.
//
// Semantics (semblend_core/triton_kernels.py:558-652, CPU path :717-732): a query row at
// position p attends causally to keys 0..p of its KV head:
//     out = softmax(scale * q . K[0..p]^T) V[0..p]
// computed with fp32 accumulation and an online (running max / running sum) softmax.
//
// MFMA path (bf16 / fp16, head_dim 64 or 128). The query rows of one KV head are flattened
// as (row, q-head-in-group), so the whole GQA group shares every K/V tile. A workgroup owns
// 32 flattened rows per wave and one chunk of the key range, walked in tiles of 64 keys:
//   * S^T = K Q^T with v_mfma_f32_32x32x16: K tile rows are the A operand (one ds_read_b128
//     per lane per 16-wide k-step), Q stays in registers as the B operand exactly as given
//     (no pre-scaling, which would add a bf16 rounding whose error grows with the score). The
//     accumulation starts at 0; P = exp2(fma(scale * log2(e), s, -m_ref)), so the scale is
//     applied to the fp32 score. In the S^T accumulator each lane owns ONE query row and 16
//     keys.
//   * O^T += V^T P^T with the same MFMA: P^T comes straight from the S^T accumulators (after
//     exp2 and conversion) as the B operand. V stays in [key][d] layout in LDS; each A-operand
//     fragment is two ds_read_b64_tr_b16 transpose loads, which hand every lane 4 consecutive
//     keys of its d column in the key order of the P^T accumulator elements.
//   * Tiles move global -> LDS with global_load_lds_dwordx4 (no register staging). The 16-byte
//     chunks of every row are XOR-swizzled so that the fragment reads are conflict-free.
//   * Softmax reference per row: seeded with the row's first live tile max; afterwards it only
//     moves (rescaling O and l) when a tile's sum of P exceeds kPMax, which the v_dot2 sum of
//     the rounded P values shows at the cost of one compare. O / l is unchanged by the choice
//     of reference.
//   * Cross-tile pipeline: S(i+1) is computed on the matrix cores while P(i) is formed on the
//     vector ALUs, then O += V(i)^T P(i). K runs two tiles ahead and V one, in two LDS stages
//     each; one barrier per tile.
// Load balance: the key range of each row tile is split into chunks of `ksplit` keys. Work
// items are ordered (chunk ascending, tile descending), so with ascending positions the
// largest items start first. Tiles that need more than one chunk write unnormalised fp32
// partials (O, m, l) and a merge kernel combines them (log-sum-exp weights).
//
// VALU path (fp32 and any other head_dim): one wave per (row, q-head), a 64-key chunk per
// step, one key per lane for the scores and the PV sum over the chunk per output dimension.

#include "sb_common.h"

#include <algorithm>
#include <cstring>
#include <functional>
#include <mutex>
#include <type_traits>
#include <vector>

namespace sb {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaveRows = 32;   // flattened query rows per MFMA row group
// Wave priority (s_setprio) raised around the PV MFMA burst, so that of the two waves on a
// SIMD the one with MFMAs ready issues first while the other forms P on the VALUs. On the 7B
// workload with the hand-laid tile loop: priority 1 319-324 us, 2 328-329, 3 327-330, none
// about 360; raising it around the QK MFMA + softmax block instead was slower. 0 turns it off.
#ifndef SB_ATTN_PV_PRIO
#define SB_ATTN_PV_PRIO 1
#endif
// Score-to-P work of the QK block skewed over the MFMA steps (fma one step ahead, packing one
// step behind the exp2), or (0) each pair's dependent chain within its own step. Skewed:
// 350.6 / 351.9 us against 354.8 / 358.9 on the 7B workload (alternating runs, one box).
#ifndef SB_ATTN_VALU_SKEW
#define SB_ATTN_VALU_SKEW 1
#endif
// LDS fragment reads issued ahead of the MFMA that consumes them, through rings of kRing
// fragments (a power of two above kFragAhead). With the two-tile loop, two ahead: 333.2 /
// 336.0 us against 340.2 / 345.5 for three (7B workload, alternating runs, one box).
#ifndef SB_ATTN_FRAG_AHEAD
#define SB_ATTN_FRAG_AHEAD 2
#endif
#ifndef SB_ATTN_FRAG_RING
#define SB_ATTN_FRAG_RING 4
#endif
constexpr int kFragAhead = SB_ATTN_FRAG_AHEAD;
constexpr int kRing = SB_ATTN_FRAG_RING;
static_assert(kRing > kFragAhead && (kRing & (kRing - 1)) == 0, "fragment ring");
// Tile loop unrolled by two (stage parity and score-buffer roles fixed per copy).
#ifndef SB_ATTN_UNROLL2
#define SB_ATTN_UNROLL2 1
#endif
// Tile loads of the two-tile loop issued one after each early MFMA step of the QK block
// instead of in a burst at the top of the iteration.
#ifndef SB_ATTN_LOADS_IN_QK
#define SB_ATTN_LOADS_IN_QK 1
#endif
#ifndef SB_ATTN_ROW_GROUPS
#define SB_ATTN_ROW_GROUPS 1
#endif
// Instruction trims of the two-tile loop, together 1.4% on the 7B workload (272.1 -> 268.1 us,
// alternating runs on one box; each alone within the run-to-run spread), results unchanged:
//  * FILL_ONE_WAVE: the key offsets of tile it + 3 are written by one wave per tile (wave
//    it mod kWaves, one entry per lane) instead of a share of them by every wave;
//  * M0_AHEAD: M0 (the direct-to-LDS destination) is written one MFMA step before its load,
//    not right before it with a wait state;
//  * SADDR: paged loads with every key row of the cache within 4 GiB of the K / V base take
//    the base in scalar registers and a 32-bit per-lane offset (no 64-bit address arithmetic);
//    needs M0_AHEAD;
//  * DOT2_ZERO: the first v_dot2 of each 8-element P pack takes an inline zero accumulator
//    (VOP3) instead of a zeroed register.
#ifndef SB_ATTN_FILL_ONE_WAVE
#define SB_ATTN_FILL_ONE_WAVE 1
#endif
#ifndef SB_ATTN_M0_AHEAD
#define SB_ATTN_M0_AHEAD 1
#endif
#ifndef SB_ATTN_SADDR
#define SB_ATTN_SADDR 1
#endif
#ifndef SB_ATTN_DOT2_ZERO
#define SB_ATTN_DOT2_ZERO 1
#endif
// Row groups per wave: each K/V fragment read from LDS feeds this many MFMAs.
constexpr int kRowGroups = SB_ATTN_ROW_GROUPS;
#ifndef SB_ATTN_TILE_KEYS
#define SB_ATTN_TILE_KEYS 64
#endif
#ifndef SB_ATTN_OCCUPANCY
#define SB_ATTN_OCCUPANCY 2
#endif
// Waves per workgroup (32 flattened rows each); one 8-wave workgroup per CU shares each K/V
// tile load among 256 rows, half the direct-to-LDS traffic of two 4-wave workgroups: 7B
// workload 268.1 -> 265.3 us with the trims above (273.0 with neither; alternating runs on
// one box). Register-staged V tiles (global load, ds_write_b128) instead of direct-to-LDS
// loads were slower (270.7 us).
#ifndef SB_ATTN_WAVES
#define SB_ATTN_WAVES 8
#endif
constexpr int kTileKeys = SB_ATTN_TILE_KEYS;  // keys per LDS tile (32 or 64)
constexpr int kWaves = SB_ATTN_WAVES;         // waves per workgroup (each owns 32 rows)
constexpr int kThreads = 64 * kWaves;
constexpr int kHalves = kTileKeys / 32;       // 32-key MFMA blocks per tile
constexpr int kBtLds = 1024;    // block-table entries staged per chunk
// Longest key chunk of a paged launch: (kBtLds - 1) blocks, in whole 64-key tiles, so that a
// chunk starting anywhere inside a block touches at most kBtLds blocks of the table.
__host__ __device__ constexpr int64_t chunk_cap(int64_t block_size) {
  return (kBtLds - 1) * block_size / 64 * 64;
}

// One request of a batched (varlen) launch: its rows, its block-table row, and where its work
// items, merge workgroups and partial slots start in the launch.
constexpr int kMaxReqs = 16;
struct ReqSlice {
  int64_t item_begin;   // first attention workgroup of the request
  int64_t merge_begin;  // first merge workgroup
  int64_t row_begin;    // first entry in positions (and q / out rows)
  int64_t num_rows;
  int64_t bt_begin;     // first entry of the request's block table
  int64_t num_blocks;   // entries of that table
  int64_t n_tiles;      // row tiles of the request (partial layout)
  int64_t part_begin;   // first partial row slot
  int max_chunks;
};

struct AttnArgs {
  const char* q;        // query rows
  char* o;              // output rows
  int64_t q_s_row, q_s_head;  // byte strides; row = position (q_by_position) or compact index
  int64_t o_s_row, o_s_head;
  int q_by_position;
  const int32_t* positions;
  const int32_t* count_ptr;   // device row count (dense drop-in), or nullptr
  int64_t num_rows;           // host row count (upper bound when count_ptr != nullptr)
  const char* k;              // K base (paged: cache + kv stride 0)
  const char* v;              // V base
  int64_t k_s_head, v_s_head; // byte strides
  int64_t k_s_seq, v_s_seq;   // flat only
  int paged;
  const int32_t* block_table;
  int64_t block_size, nb_total, nb_per_seq;
  int bs_log2;                // log2(block_size) when a power of two, else -1
  int64_t s_block, s_pos;     // paged byte strides (shared by K and V)
  int narrow_ofs;             // power-of-two blocks, s_block < 2^32, s_pos and block_size
                              // < 2^24: key offsets by one 32 x 32 -> 64-bit multiply-add
  int64_t kv_len;             // addressable keys
  int num_kv_heads;
  int group;                  // q heads per kv head
  int head_dim;
  float scale;
  float scale_log2;           // scale * log2(e)
  int ksplit;                 // keys per work item after a row tile's first chunk
                              // (multiple of kTileKeys)
  int ksplit_first;           // keys of a row tile's first chunk (multiple of kTileKeys)
  int max_chunks;             // chunks of the longest key range (chunk_count(kv_len))
  int device_split;           // 1: ksplit, max_chunks and n_tiles follow the device row count
  int64_t n_tiles;            // row tiles per kv head used for the partial layout
  int tile_rows;              // flattened query rows per workgroup tile
  float* part_o;              // [Hkv][n_tiles][max_chunks][128][D] fp32, or nullptr
  float* part_ml;             // [Hkv][n_tiles][max_chunks][128][2] fp32 (m, l)
  const int32_t* item_order;  // single-request launches: work item of each workgroup (a
                              // host-planned order), or nullptr (workgroup b runs item b)
};

// Key chunks of a row tile: the first covers [0, ksplit_first), each later one ksplit keys.
__host__ __device__ inline int chunk_begin(const AttnArgs& a, int c) {
  return c == 0 ? 0 : a.ksplit_first + (c - 1) * a.ksplit;
}
__host__ __device__ inline int chunk_len(const AttnArgs& a, int c) {
  return c == 0 ? a.ksplit_first : a.ksplit;
}
__host__ __device__ inline int chunk_count(const AttnArgs& a, int64_t kend) {
  return kend <= a.ksplit_first
             ? 1
             : 1 + static_cast<int>((kend - a.ksplit_first + a.ksplit - 1) / a.ksplit);
}

// Kernel parameter: the call's arguments and, for a batched launch, the request table (read
// in place from the kernel-argument segment).
struct AttnBatch {
  AttnArgs a;
  int num_reqs;               // requests in `req` (0: one request, described by `a`)
  ReqSlice req[kMaxReqs];
};

// Batched launch: selects the request that workgroup `b` (an index into the launch's
// attention or merge grid) belongs to, narrows `a` to that request, and returns b relative to
// the request's first workgroup. A single-request launch returns b unchanged.
__device__ __forceinline__ int64_t select_request(const AttnBatch& batch, AttnArgs& a,
                                                  int64_t b, bool merge) {
  if (batch.num_reqs <= 0) return b;
  int r = 0;
  while (r + 1 < batch.num_reqs &&
         b >= (merge ? batch.req[r + 1].merge_begin : batch.req[r + 1].item_begin))
    ++r;
  const ReqSlice& s = batch.req[r];
  a.positions += s.row_begin;
  if (!a.q_by_position) {
    a.q += s.row_begin * a.q_s_row;
    a.o += s.row_begin * a.o_s_row;
  }
  a.num_rows = s.num_rows;
  a.block_table += s.bt_begin;
  a.nb_per_seq = s.num_blocks;
  a.kv_len = s.num_blocks * a.block_size;
  a.n_tiles = s.n_tiles;
  a.max_chunks = s.max_chunks;
  if (a.part_o) {
    a.part_o += s.part_begin * a.head_dim;
    a.part_ml += s.part_begin * 2;
  }
  return b - (merge ? s.merge_begin : s.item_begin);
}

// Rows of the call: the device-side count of a compacted mask (never more than num_rows).
__device__ __forceinline__ int64_t attn_num_rows(const AttnArgs& a) {
  return a.count_ptr ? min(static_cast<int64_t>(*a.count_ptr), a.num_rows) : a.num_rows;
}

__device__ __forceinline__ int clamp_block(const AttnArgs& a, int64_t pb) {
  return static_cast<int>(pb < 0 ? 0 : (pb >= a.nb_total ? a.nb_total - 1 : pb));
}

__device__ __forceinline__ const char* key_row(const AttnArgs& a, const char* base,
                                               int64_t s_head, int64_t s_seq, int64_t key,
                                               int kvh) {
  if (a.paged) {
    const int64_t lb = key / a.block_size;
    const int pb = clamp_block(a, a.block_table[lb]);
    return base + pb * a.s_block + kvh * s_head + (key - lb * a.block_size) * a.s_pos;
  }
  return base + kvh * s_head + key * s_seq;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// Value of v in lane (lane ^ 32): v_permlane32_swap exchanges the upper half of one register
// with the lower half of another, so swapping v with itself and picking the moved half gives
// the partner lane's value without a round trip through LDS.
__device__ __forceinline__ float xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

template <int DT> struct Mma;
template <> struct Mma<SB_DTYPE_BF16> {
  using vec8 = bf16x8_t;
  using elem = __bf16;
  __device__ __forceinline__ static f32x16_t mma(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static vec8 cvt8(const float* f) {
    vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = static_cast<__bf16>(f[e]);
    return r;
  }
  __device__ __forceinline__ static uint16_t cvt1(float f) { return f32_to_bf16(f); }
  // Two values rounded to a packed pair (one v_cvt_pk_bf16_f32), and acc + their sum.
  typedef __bf16 x2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static x2 cvt2(float a, float b) {
    const x2 r = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return r;
  }
  __device__ __forceinline__ static float sum2(x2 v, float acc) {
    const x2 one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
    return __builtin_amdgcn_fdot2_f32_bf16(v, one, acc, false);
  }
  // 0 + the sum of v, the zero as an inline constant of the VOP3 form (no zeroed register).
  __device__ __forceinline__ static float sum2z(x2 v, uint32_t one) {
    float r;
    asm volatile("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(v), "v"(one));
    return r;
  }
  static constexpr uint32_t kOnePair = 0x3f803f80u;
  // acc + sum of the 8 (rounded) elements of v, two per v_dot2.
  __device__ __forceinline__ static float sum8(vec8 v, float acc) {
    typedef __bf16 x2 __attribute__((ext_vector_type(2)));
    const x2 one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const x2 pr = {v[2 * e], v[2 * e + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
    }
    return acc;
  }
  // Largest tile sum of P accepted without moving the reference max (bf16 keeps fp32's
  // exponent range, so only fp32 overflow of O bounds it).
  static constexpr float kPMax = 0x1p64f;
};
template <> struct Mma<SB_DTYPE_F16> {
  using vec8 = f16x8_t;
  using elem = _Float16;
  __device__ __forceinline__ static f32x16_t mma(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static vec8 cvt8(const float* f) {
    vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = static_cast<_Float16>(f[e]);
    return r;
  }
  __device__ __forceinline__ static uint16_t cvt1(float f) { return f32_to_f16(f); }
  typedef _Float16 x2 __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static x2 cvt2(float a, float b) {
    const x2 r = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return r;
  }
  __device__ __forceinline__ static float sum2(x2 v, float acc) {
    const x2 one = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
    return __builtin_amdgcn_fdot2(v, one, acc, false);
  }
  __device__ __forceinline__ static float sum2z(x2 v, uint32_t one) {
    float r;
    asm volatile("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(v), "v"(one));
    return r;
  }
  static constexpr uint32_t kOnePair = 0x3c003c00u;
  __device__ __forceinline__ static float sum8(vec8 v, float acc) {
    typedef _Float16 x2 __attribute__((ext_vector_type(2)));
    const x2 one = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const x2 pr = {v[2 * e], v[2 * e + 1]};
      acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
  }
  // fp16 P saturates at 65504: keep every p below 2^8.
  static constexpr float kPMax = 256.f;
};

// 16-byte chunk position of chunk c of row r in the swizzled K and V tiles (CH chunks per
// row). K fragments are read as 16 bytes per lane from 32 consecutive rows at one chunk:
// rows r..r+15 land on distinct chunk positions. V is read with transpose loads that touch
// 4 consecutive rows x 32-64 bytes: rows r..r+3 land on disjoint 64-byte bank ranges.
template <int CH>
__device__ __forceinline__ int kswz(int r, int c) {
  return c ^ (r & (CH - 1));
}
template <int CH>
__device__ __forceinline__ int vswz(int r, int c) {
  return CH >= 16 ? c ^ (4 * (r & 3)) : c ^ (4 * ((r >> 1) & 1));
}

#define SB_GLOBAL __attribute__((address_space(1)))
#define SB_LDS __attribute__((address_space(3)))
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Waits until this wave's outstanding vector-memory operations (including direct-to-LDS
// loads) are complete: s_waitcnt vmcnt(0), other counters untouched.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i's chunk lands at
// LDS byte address lds_wave + 16 i, where lds_wave is wave-uniform. Written as inline
// assembly on purpose:
// the compiler treats a direct-to-LDS load it knows about as a pending write to the whole LDS
// variable and waits for it (vmcnt(0)) before any later read of that variable, which would
// serialise every prefetch with the tile being computed. Hidden from it, the loads overlap
// the compute; the kernel orders them itself with wait_vmem() before each barrier that
// publishes a tile. (Waits the compiler places for its own vector-memory loads stay safe:
// completions are counted in order, so extra outstanding loads only make them stricter.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is named as clobbered on purpose
__device__ __forceinline__ void dma_row_chunk(const char* src, uint32_t lds_wave) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off"
      :
      : "s"(lds_wave), "v"(src)
      : "memory", "m0");
}
// The same load in two parts, for callers that keep the M0 write and the load apart: the LDS
// destination goes to M0 first, and the load (which reads M0) must follow at least one other
// instruction later (the M0 write-to-use wait state). Nothing between them may write M0.
__device__ __forceinline__ void dma_set_m0(uint32_t lds_wave) {
  asm volatile("s_mov_b32 m0, %0" : : "s"(lds_wave) : "m0");
}
__device__ __forceinline__ void dma_at_m0(const char* src) {
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src) : "memory");
}
// The same with the wave's base address in scalar registers and a 32-bit byte offset per lane.
__device__ __forceinline__ void dma_at_m0_s(const char* base, uint32_t voff) {
  asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base) : "memory");
}
// LDS byte address of a pointer into a __shared__ array (wave-uniform arithmetic on it stays
// in scalar registers).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SB_LDS const void*)p));
}
#pragma clang diagnostic pop

// Resident workgroups of the MFMA kernel on 256 CUs (one 4-wave workgroup per CU with two
// row groups per wave, SB_ATTN_OCCUPANCY with one), and how many work items per slot the
// split aims for.
constexpr int kResidentSlots = kRowGroups == 1 ? 256 * SB_ATTN_OCCUPANCY * 4 / kWaves : 256;
#ifndef SB_ATTN_ITEMS_PER_SLOT
#define SB_ATTN_ITEMS_PER_SLOT 1
#endif
constexpr int kItemsPerSlot = SB_ATTN_ITEMS_PER_SLOT;

// Key-range split of a call: items no longer than the average work per slot (assuming the
// rows' key ranges average half the context), so that longest-first scheduling balances the
// CUs. Host plan and device-derived split use this one rule.
struct KeySplit {
  int ksplit;
  int max_chunks;
};
__host__ __device__ inline KeySplit key_split(int64_t n_tiles, int64_t num_kv_heads,
                                              int64_t kv_len, int64_t block_size, bool paged) {
  const int64_t kv_pad = (kv_len + kTileKeys - 1) / kTileKeys * kTileKeys;
  int64_t ks = n_tiles * num_kv_heads * (kv_len / 2) / (kResidentSlots * kItemsPerSlot);
  ks = ks / kTileKeys * kTileKeys;
  if (ks < 512) ks = 512;
  if (paged) {
    const int64_t cap = chunk_cap(block_size);
    if (ks > cap) ks = cap;
  }
  if (ks > kv_pad) ks = kv_pad;
  if (ks < kTileKeys) ks = kTileKeys;
  const int64_t chunks = (kv_len + ks - 1) / ks;
  return KeySplit{static_cast<int>(ks), static_cast<int>(chunks < 1 ? 1 : chunks)};
}
// The device-derived split of a dense call (device_split), from its row-tile count.
__device__ __forceinline__ void apply_device_split(AttnArgs& a, int64_t n_tiles_live) {
  if (!a.device_split) return;
  const KeySplit sp = key_split(n_tiles_live, a.num_kv_heads, a.kv_len, 1, false);
  a.ksplit = sp.ksplit;
  a.ksplit_first = sp.ksplit;
  a.max_chunks = sp.max_chunks;
  a.n_tiles = n_tiles_live;
}

// Work-item decode shared by the attention and merge kernels.
struct Item {
  int kvh;
  int64_t tile;
  int chunk;
};

__device__ __forceinline__ Item decode_item(const AttnArgs& a, int64_t n_tiles_live,
                                           int64_t b) {
  // b = (chunk * n_tiles_live + tile_rev) * Hkv + kvh; tiles taken in descending order.
  // Counting live tiles (not the launch's upper bound) puts every live item before the
  // items past the last chunk, which exit at once: with a row count known only on the
  // device (dense drop-in) the launch is sized for all rows and most items are such.
  Item it;
  it.kvh = static_cast<int>(b % a.num_kv_heads);
  const int64_t rest = b / a.num_kv_heads;
  const int64_t tile_rev = rest % n_tiles_live;
  it.chunk = static_cast<int>(min(rest / n_tiles_live, static_cast<int64_t>(0x7fffffff)));
  it.tile = n_tiles_live - 1 - tile_rev;
  return it;
}

// Key-row addressing, fixed per instantiation so that the tile loop carries no branch on it
// (and no scalar registers for the other forms).
enum AttnAddressing { kAddrFlat = 0, kAddrPagedNarrow = 1, kAddrPaged = 2 };

__host__ __forceinline__ int attn_addressing(const AttnArgs& a) {
  return !a.paged ? kAddrFlat : (a.narrow_ofs ? kAddrPagedNarrow : kAddrPaged);
}

template <int DT, int D, int RG, int AM>
__global__ __launch_bounds__(kThreads, RG == 1 ? SB_ATTN_OCCUPANCY * 4 / kWaves : 1) void
attn_mfma_kernel(const AttnBatch batch) {
  constexpr bool kPaged = AM != kAddrFlat;
  AttnArgs a = batch.a;
  int64_t b0 = blockIdx.x;
  if (batch.num_reqs <= 0 && a.item_order) {
    b0 = a.item_order[b0];
    if (b0 < 0 || b0 >= static_cast<int64_t>(gridDim.x)) return;  // not an item of the launch
  }
  const int64_t item_b = select_request(batch, a, b0, false);
  using M = Mma<DT>;
  using vec8 = typename M::vec8;
  constexpr int TR = kWaveRows * RG * kWaves;  // flattened rows per workgroup tile
  constexpr int NKS = D / 16;             // QK^T k-steps
  constexpr int NDT = D / 32;             // PV output d-tiles
  constexpr int CH = D / 8;               // 16-byte chunks per row
  constexpr int NLD = kTileKeys * CH / kThreads;  // direct-to-LDS loads per thread per tile
  // K and V tiles: kTileKeys rows of D elements, unpadded, 16-byte chunks XOR-swizzled by
  // row (kswz / vswz) so that the fragment reads below are free of bank conflicts.
  __shared__ __align__(16) uint16_t Ks[2][kTileKeys * D];
  __shared__ __align__(16) uint16_t Vs[2][kTileKeys * D];
  __shared__ int bt_s[kBtLds];
  __shared__ uint64_t kofs[3][kTileKeys];  // per-key byte offsets of K rows (3-slot ring)
  __shared__ uint64_t vofs[3][kTileKeys];  // ... and of V rows
  __shared__ int red_max[kWaves];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lg = lane >> 5;

  const int64_t n_rows = attn_num_rows(a);
  const int64_t rows_kv = n_rows * a.group;
  const int64_t n_tiles_live = (rows_kv + TR - 1) / TR;
  if (n_tiles_live <= 0) return;  // no rows (uniform)
  apply_device_split(a, n_tiles_live);
  const Item item = decode_item(a, n_tiles_live, item_b);
  if (item.tile < 0 || item.chunk >= a.max_chunks) return;  // uniform, before any barrier
  const int kvh = item.kvh;

  // The chunk's first key and its end within the table are known from the item alone, so
  // everything that needs only them (the block-table slice, the key offsets of the first
  // three tiles, the Q fragments of paged calls) is requested together with the positions,
  // and one barrier publishes it all: one global round trip before the first tile loads.
  const int k0 = chunk_begin(a, item.chunk);
  if (k0 >= a.kv_len) return;  // uniform, before any barrier
  const int kc = static_cast<int>(min(static_cast<int64_t>(k0 + chunk_len(a, item.chunk)),
                                      a.kv_len));
  int lb0 = 0;
  if (kPaged) {
    lb0 = static_cast<int>(k0 / a.block_size);
    const int nb = static_cast<int>((kc - 1) / a.block_size) - lb0 + 1;  // <= kBtLds
    for (int i = tid; i < nb; i += kThreads) bt_s[i] = clamp_block(a, a.block_table[lb0 + i]);
  }
  const char* kbase = a.k + kvh * a.k_s_head;
  const char* vbase = a.v + kvh * a.v_s_head;
  // Byte offset of key `key` relative to kbase / vbase, the key's block given (paged K and V
  // rows share one offset, kept in kofs only).
  auto key_offset = [&](int key, int pb) -> uint64_t {
    if (AM == kAddrPagedNarrow) {
      const uint32_t in_block =
          static_cast<uint32_t>(key) & (static_cast<uint32_t>(a.block_size) - 1u);
      return static_cast<uint64_t>(static_cast<uint32_t>(pb)) *
                 static_cast<uint32_t>(a.s_block) +
             __umul24(in_block, static_cast<uint32_t>(a.s_pos));
    }
    const int lb = a.bs_log2 >= 0 ? key >> a.bs_log2 : key / static_cast<int>(a.block_size);
    return static_cast<uint64_t>(pb) * a.s_block +
           static_cast<uint64_t>(key - lb * a.block_size) * a.s_pos;
  };
  auto key_block = [&](int key) -> int {
    if (AM == kAddrPagedNarrow) return key >> a.bs_log2;  // power-of-two blocks
    return a.bs_log2 >= 0 ? key >> a.bs_log2 : key / static_cast<int>(a.block_size);
  };
  // Offsets of the keys of tile `slot` (keys past kc_lim are clamped to it: masked later),
  // the blocks read from the staged slice.
  int kc_lim = kc - 1;
  auto fill_offsets = [&](int slot, int t0, int i) {
    const int key = min(t0 + i, kc_lim);
    if (kPaged) {
      kofs[slot][i] = key_offset(key, bt_s[key_block(key) - lb0]);
    } else {
      kofs[slot][i] = static_cast<uint64_t>(key) * a.k_s_seq;
      vofs[slot][i] = static_cast<uint64_t>(key) * a.v_s_seq;
    }
  };
  // The first three tiles' offsets, with the blocks read from the global table (the same
  // lines the slice loads fetch) so that they do not wait for the slice.
  if (tid < 3 * kTileKeys) {
    const int key = min(k0 + tid, kc_lim);
    const int slot = tid / kTileKeys, i = tid % kTileKeys;
    if (kPaged) {
      kofs[slot][i] = key_offset(key, clamp_block(a, a.block_table[key_block(key)]));
    } else {
      kofs[slot][i] = static_cast<uint64_t>(key) * a.k_s_seq;
      vofs[slot][i] = static_cast<uint64_t>(key) * a.v_s_seq;
    }
  }

  // This lane's query rows: one per row group.
  int p[RG], qh[RG];
  int64_t qrow[RG];
  int pmax_l = -1;
  vec8 qf[RG][NKS];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int64_t r = item.tile * TR + (wave * RG + g) * kWaveRows + lq;
    p[g] = -1;
    qrow[g] = 0;
    qh[g] = 0;
    const bool valid = r < rows_kv;
    if (valid) {
      const int64_t pi = r / a.group;
      qh[g] = kvh * a.group + static_cast<int>(r - pi * a.group);
      int pp = a.positions[pi];
      if (pp >= a.kv_len) pp = static_cast<int>(a.kv_len - 1);
      qrow[g] = a.q_by_position ? max(pp, 0) : pi;
      p[g] = pp < 0 ? -1 : pp;
    }
    pmax_l = max(pmax_l, p[g]);
    // Q fragments (B operand), the query rows as given; a paged call's row address does
    // not depend on its position, so these loads go out with the position's.
    const char* qp = a.q + qrow[g] * a.q_s_row + qh[g] * a.q_s_head;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      vec8 v = {};
      if (valid) v = *reinterpret_cast<const vec8*>(qp + (16 * s + 8 * lg) * 2);
      qf[g][s] = v;
    }
  }
  // Wave-uniform values are moved to scalar registers (readfirstlane) so that the compiler
  // sees them as uniform: branches on them stay scalar branches instead of being turned into
  // per-lane selects (the mask below would otherwise run on every tile).
  const int pmax_w = __builtin_amdgcn_readfirstlane(wave_max_i(pmax_l));
  if (lane == 0) red_max[wave] = pmax_w;
  __syncthreads();  // red_max, the block-table slice and the first offset tables
  int kend_l = red_max[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) kend_l = max(kend_l, red_max[w]);
  const int kend = __builtin_amdgcn_readfirstlane(kend_l) + 1;
  if (k0 >= kend) return;  // uniform: kend comes from shared memory
  const int k1 = min(kc, kend);
  kc_lim = k1 - 1;
  const int nchunks = chunk_count(a, kend);
  int plim[RG];  // keys beyond the chunk are masked as well
  int pmin_l = 0x7fffffff;
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    plim[g] = min(p[g], k1 - 1);
    if (p[g] >= 0) pmin_l = min(pmin_l, plim[g]);
    if (p[g] < 0) {  // a row with no position (negative) reads nothing: zero query
#pragma unroll
      for (int s = 0; s < NKS; ++s) qf[g][s] = vec8{};
    }
  }
  const int pmin_w = __builtin_amdgcn_readfirstlane(wave_min_i(pmin_l));
  const int pmax_c = min(pmax_w, k1 - 1);
  const float c_log2 = a.scale_log2;  // scale * log2(e): score units -> log2 domain
#if SB_ATTN_DOT2_ZERO
  uint32_t one_pair = M::kOnePair;  // (1, 1) in the input type, for the P pack sums
  asm volatile("" : "+v"(one_pair));  // one register for the whole loop
#endif

  // Softmax state per row: O and l are relative to a reference max m_ref (log2 domain,
  // of scale * log2(e) * s); negm = -m_ref enters every exp2 through one fma. A row is
  // "seeded" once m_ref is its first live tile's max;
  // rows with no key in this chunk start seeded (their scores are all masked).
  float m_ref[RG], l_run[RG];
  bool seeded[RG];
  float negm[RG];
  f32x16_t o[RG][NDT];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    m_ref[g] = 0.f;
    seeded[g] = plim[g] < k0;
    negm[g] = 0.f;
    l_run[g] = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[g][t][i] = 0.f;
  }

  // Tiles move from global memory straight into LDS (global_load_lds_dwordx4: each wave
  // instruction fills 1 KB of consecutive 16-byte slots; every lane fetches the chunk that
  // the swizzled layout puts in its slot). Loads are unconditional: every offset is a valid
  // row.
  // Slot q * kThreads + tid of a tile holds row q * (kThreads / CH) + tid / CH at position
  // tid % CH; both swizzles depend on the row modulo 16 only, so the 16-byte chunk a lane
  // fetches is the same for every q: one source pointer per lane for K and one for V.
  static_assert((kThreads / CH) % 16 == 0, "swizzle independent of the load index");
  const char* ksrc = kbase + 16 * kswz<CH>(tid / CH, tid % CH);
  const char* vsrc = vbase + 16 * vswz<CH>(tid / CH, tid % CH);
  auto load_rows = [&](const char* src, const uint64_t* ofs, uint16_t* dst) {
    // All row offsets first (back-to-back LDS reads, one wait), then the loads.
    uint64_t ro[NLD];
#pragma unroll
    for (int q = 0; q < NLD; ++q) ro[q] = ofs[q * (kThreads / CH) + tid / CH];
#pragma unroll
    for (int q = 0; q < NLD; ++q)
      dma_row_chunk(src + ro[q], lds_addr(dst) + (q * kThreads + wave * 64) * 16);
  };
  // The same loads in two parts: the row offsets first, then load q of the tile (K or V).
  auto read_ofs = [&](const uint64_t* ofs, uint64_t* ro) {
#pragma unroll
    for (int q = 0; q < NLD; ++q) ro[q] = ofs[q * (kThreads / CH) + tid / CH];
  };
  constexpr bool kSaddr = SB_ATTN_SADDR && SB_ATTN_M0_AHEAD && AM == kAddrPagedNarrow;
  const uint32_t k_lane = 16 * kswz<CH>(tid / CH, tid % CH);  // chunk part of the offsets
  const uint32_t v_lane = 16 * vswz<CH>(tid / CH, tid % CH);
  auto read_ofs32 = [&](const uint64_t* ofs, uint32_t lanep, uint32_t* ro) {
#pragma unroll
    for (int q = 0; q < NLD; ++q)
      ro[q] = static_cast<uint32_t>(ofs[q * (kThreads / CH) + tid / CH]) + lanep;
  };
  auto dma_one = [&](const char* src, uint64_t ro, uint16_t* dst, int q) {
    dma_row_chunk(src + ro, lds_addr(dst) + (q * kThreads + wave * 64) * 16);
  };
  auto dma_dst = [&](uint16_t* dst, int q) -> uint32_t {
    return lds_addr(dst) + (q * kThreads + wave * 64) * 16;
  };
  auto load_k = [&](int slot, int stage) { load_rows(ksrc, kofs[slot], Ks[stage]); };
  auto load_v = [&](int slot, int stage) {
    load_rows(vsrc, kPaged ? kofs[slot] : vofs[slot], Vs[stage]);
  };

  // K fragment of (half n % kHalves, k-step n / kHalves): key row 32 * half + lq, 16-byte
  // chunk 2 * kstep + lg.
  // The swizzle depends on the row modulo 16 only, so the byte offset is kl[kstep] (this
  // lane's part, half 0, stage 0) plus a constant per (stage, half).
  int kl[NKS];
#pragma unroll
  for (int k = 0; k < NKS; ++k) kl[k] = 2 * (lq * D + 8 * kswz<CH>(lq, 2 * k + lg));
  auto kfrag = [&](int stage, int n) -> vec8 {
    const char* base = reinterpret_cast<const char*>(&Ks[0][0]) +
                       stage * (kTileKeys * D * 2) + (n % kHalves) * (32 * D * 2);
    return *reinterpret_cast<const vec8*>(base + kl[n / kHalves]);
  };
  // V^T fragment of (d-tile t, step st, half j) for the A operand: lane (lq, lg) needs
  // d = 32t + lq at keys 32j + 16st + {4lg..4lg+3, 8+4lg..8+4lg+3} (the key order of the
  // P^T accumulator elements). Two ds_read_b64_tr_b16: in each group of 16 lanes, lane i
  // reads 4 consecutive d of key row kb + i/4, and the transpose hands lane i the 4 keys
  // kb..kb+3 of column d0 + i.
  // The V swizzle depends on the row modulo 4 only, which is (gi >> 2) mod 4 here: the byte
  // offset is vl[t] (this lane's part for d-tile t) plus a constant per (stage, j, st, e).
  const int grp = lane >> 4, gi = lane & 15;
  int vl[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    const int d = 32 * t + 16 * (grp & 1) + 4 * (gi & 3);
    const int row = 4 * lg + (gi >> 2);
    vl[t] = 2 * (row * D + 8 * vswz<CH>(row, d >> 3) + (d & 7));
  }
  auto vfrag = [&](int stage, int n) -> vec8 {
    const int t = n % NDT, st = (n / NDT) & 1, j = n / (2 * NDT);
    u32x2_t h[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const char* base = reinterpret_cast<const char*>(&Vs[0][0]) +
                         stage * (kTileKeys * D * 2) + (32 * j + 16 * st + 8 * e) * (D * 2);
      h[e] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                              (SB_LDS s16x4_t*)(base + vl[t])));
    }
    const u32x4_t w = {h[0].x, h[0].y, h[1].x, h[1].y};
    return __builtin_bit_cast(vec8, w);
  };
  using Scores = f32x16_t[RG][kHalves];
  // S^T = K Q^T for one tile (fp32 scores). (half, k-step) pairs alternate halves, so two
  // independent accumulation chains interleave; K fragments stream through a 4-deep ring.
  auto qk = [&](int stage, Scores& sc) {
    constexpr int NQ = kHalves * NKS;
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int j = 0; j < kHalves; ++j) sc[g][j] = f32x16_t{};
    vec8 ring[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) ring[n] = kfrag(stage, n);
#pragma unroll
    for (int n = 0; n < NQ; ++n) {
      const vec8 kf = ring[n & 3];
      if (n + 4 < NQ) ring[n & 3] = kfrag(stage, n + 4);
#pragma unroll
      for (int g = 0; g < RG; ++g)
        sc[g][n % kHalves] = M::mma(kf, qf[g][n / kHalves], sc[g][n % kHalves]);
    }
  };
  // Causal / chunk-end mask, only for tiles that cross some row's last key.
  auto mask = [&](int t0, Scores& sc) {
    if (t0 + kTileKeys - 1 > pmin_w) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < kHalves; ++j) {
          const int lim = plim[g] - (t0 + 32 * j + 4 * lg);  // key offset limit of this lane
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (8 * (i >> 2) + (i & 3) > lim) sc[g][j][i] = -INFINITY;
        }
    }
  };
  // P = exp2(scale * log2(e) * s - m_ref), rounded to the input type; the tile sum from the
  // rounded values.
  vec8 pb[RG][kHalves][2];
  float tsum[RG];
  auto exp_tile = [&](int g, const Scores& sc) {
    float acc[kHalves][2];  // independent partial sums (v_dot2 accumulates in place)
#pragma unroll
    for (int j = 0; j < kHalves; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float pf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pf[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(c_log2, sc[g][j][8 * h + e], negm[g]));
        pb[g][j][h] = M::cvt8(pf);
        acc[j][h] = M::sum8(pb[g][j][h], 0.f);
      }
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < kHalves; ++j) t += acc[j][0] + acc[j][1];
    tsum[g] = t;
  };

  // Software pipeline over tiles of kTileKeys keys. Iteration `it` computes S(it+1) = QK^T
  // of the next tile while it turns S(it) into P(it) (MFMA and VALU work interleave in one
  // block), then O += V(it)^T P(it). K has two LDS stages and runs two tiles ahead, V two
  // stages and one tile ahead: iteration `it` issues the loads of K(it+2) and V(it+1) into
  // the stages that QK(it) and PV(it-1) released (at its top, or spread over its QK block);
  // each wave waits for its own loads before the iteration's single barrier. Key offsets
  // come from a three-slot table ring (slot = tile mod 3) filled three tiles ahead.
  const int ntiles = (k1 - k0 + kTileKeys - 1) / kTileKeys;
  Scores s_cur, s_nxt;
  load_k(0, 0);
  if (ntiles > 1) load_k(1, 1);
  load_v(0, 0);
  wait_vmem();
  __syncthreads();
  qk(0, s_cur);
  mask(k0, s_cur);
  __syncthreads();  // K stage 0 is refilled at the top of the first iteration

  // slot = it mod 3 (offset-table ring), advanced once per tile. `parity` is it mod 2 as a
  // compile-time constant (or -1: taken from `it`); with `swap` the caller alternates the
  // roles of the two score buffers, so S(it+1) stays where QK^T left it.
  // With `ilv` (only where both loads are known to be due: K(it+2) and V(it+1)) the tile
  // loads go out inside the QK block, one after each of its first 2 NLD MFMA steps.
  auto iteration = [&](int it, int slot, auto has_next, auto parity, auto swap, Scores& s_cur,
                       Scores& s_nxt, auto ilv) {
    constexpr bool NEXT = decltype(has_next)::value;
    constexpr bool ILV = decltype(ilv)::value;
    static_assert(!ILV || NEXT, "interleaved loads ride on the QK block");
    constexpr int PAR = decltype(parity)::value;
    const int par = PAR >= 0 ? PAR : (it & 1);
    if (PAR >= 0) {
      // Loop-carried through an empty asm: the fragment addresses are then not loop
      // invariants, so the compiler folds the (stage, half) constants into the LDS
      // instructions' offsets instead of keeping one register per address.
#pragma unroll
      for (int k = 0; k < NKS; ++k) asm volatile("" : "+v"(kl[k]));
#pragma unroll
      for (int t = 0; t < NDT; ++t) asm volatile("" : "+v"(vl[t]));
    }
    const int t0 = k0 + it * kTileKeys;
    const int slot1 = slot == 2 ? 0 : slot + 1;  // (it + 1) mod 3
    const int slot2 = slot == 0 ? 2 : slot - 1;  // (it + 2) mod 3
    uint64_t ro_k[NLD], ro_v[NLD];
    uint32_t ro_k32[NLD], ro_v32[NLD];
    if (ILV && kSaddr) {
      read_ofs32(kofs[slot2], k_lane, ro_k32);
      read_ofs32(kofs[slot1], v_lane, ro_v32);
    } else if (ILV) {
      read_ofs(kofs[slot2], ro_k);
      read_ofs(kPaged ? kofs[slot1] : vofs[slot1], ro_v);
    } else {
      if (it + 2 < ntiles) load_k(slot2, par);
      if (it + 1 < ntiles) load_v(slot1, par ^ 1);
    }
    // Offsets of tile it+3: kTileKeys / kWaves entries from each wave, or (one-wave form) all
    // of them from one of waves 0-3 in turn. Waves w and w + 4 share a SIMD, and the older
    // one (w) wins the issue ties and then waits at the tile barrier for the other, so extra
    // work belongs on waves 0-3 (7B 16K: 271.3 -> 268.7 us against rotating over all eight;
    // moving the tile loads there as well was slower, 273.8 us).
#if SB_ATTN_FILL_ONE_WAVE
    static_assert(kTileKeys == 64, "one entry per lane");
    if (it + 3 < ntiles && wave == (it & (kWaves / 2 - 1)))
      fill_offsets(slot, t0 + 3 * kTileKeys, lane);
#else
    if (it + 3 < ntiles && lane < kTileKeys / kWaves)
      fill_offsets(slot, t0 + 3 * kTileKeys, wave * (kTileKeys / kWaves) + lane);
#endif
    const bool live = t0 <= pmax_c;
    // ---- S(it+1) on the matrix cores while P(it) is formed on the vector ALUs ----
    // The block is laid out by hand: step n reads the K fragment of step n + kFragAhead,
    // issues the MFMAs of step n and forms one share of P(it) (exp2, pair conversion, pair
    // sum); scheduling barriers keep the steps in this order, so every fragment read has
    // kFragAhead MFMAs to land and the vector work sits between independent MFMAs.
    bool bad_any = false;
    bool bad[RG];
    if (NEXT) {
      constexpr int NQ = kHalves * NKS;                // MFMA steps (each RG MFMAs)
      constexpr int NPAIR = RG * kHalves * 8;          // P pairs per lane
      static_assert(NPAIR % NQ == 0, "P pairs split evenly over the MFMA steps");
      constexpr int PPS = NPAIR / NQ;                  // pairs per step
      const int ks = par ^ 1;
      vec8 ring[kRing];
#pragma unroll
      for (int n = 0; n < kFragAhead; ++n) ring[n] = kfrag(ks, n);
      uint32_t pw[RG][kHalves][2][4];  // P words: [group][half][8-element pack][word]
      float acc[RG][kHalves][2];
#if SB_ATTN_VALU_SKEW
      // element e (0, 1) of P pair q
      auto s_at = [&](int q, int e) -> float {
        const int g = q / (kHalves * 8), r = q % (kHalves * 8);
        return s_cur[g][r / 8][8 * ((r / 4) % 2) + 2 * (r % 4) + e];
      };
      auto pack_pair = [&](int q, float e0, float e1) {
        const int g = q / (kHalves * 8), r = q % (kHalves * 8);
        const int hj = r / 8, h = (r / 4) % 2, w = r % 4;
        const auto pr = M::cvt2(e0, e1);
        pw[g][hj][h][w] = __builtin_bit_cast(uint32_t, pr);
#if SB_ATTN_DOT2_ZERO
        acc[g][hj][h] = w == 0 ? M::sum2z(pr, one_pair) : M::sum2(pr, acc[g][hj][h]);
#else
        acc[g][hj][h] = M::sum2(pr, w == 0 ? 0.f : acc[g][hj][h]);
#endif
      };
      float fa0[NPAIR], fa1[NPAIR], ea0[NPAIR], ea1[NPAIR];
#pragma unroll
      for (int q = 0; q < PPS; ++q) {
        fa0[q] = __builtin_fmaf(c_log2, s_at(q, 0), negm[q / (kHalves * 8)]);
        fa1[q] = __builtin_fmaf(c_log2, s_at(q, 1), negm[q / (kHalves * 8)]);
      }
#endif
#if SB_ATTN_M0_AHEAD
      // load n of the step loop: K(it+2) part n, then V(it+1) part n - NLD
      auto load_dst = [&](int n) -> uint32_t {
        return n < NLD ? dma_dst(Ks[par], n) : dma_dst(Vs[par ^ 1], n - NLD);
      };
      if (ILV) dma_set_m0(load_dst(0));
#endif
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < NQ; ++n) {
        if (n + kFragAhead < NQ) ring[(n + kFragAhead) % kRing] = kfrag(ks, n + kFragAhead);
        const int j = n % kHalves;
#pragma unroll
        for (int g = 0; g < RG; ++g)
          s_nxt[g][j] =
              M::mma(ring[n % kRing], qf[g][n / kHalves], n < kHalves ? f32x16_t{} : s_nxt[g][j]);
        if (ILV) {
          static_assert(2 * NLD <= NQ, "one load per MFMA step");
#if SB_ATTN_M0_AHEAD
          // M0 was written in the previous step (or before the loop), an MFMA ago.
          if (kSaddr) {
            if (n < NLD) dma_at_m0_s(kbase, ro_k32[n]);
            else if (n < 2 * NLD) dma_at_m0_s(vbase, ro_v32[n - NLD]);
          } else {
            if (n < NLD) dma_at_m0(ksrc + ro_k[n]);
            else if (n < 2 * NLD) dma_at_m0(vsrc + ro_v[n - NLD]);
          }
          if (n + 1 < 2 * NLD) dma_set_m0(load_dst(n + 1));
#else
          if (n < NLD) dma_one(ksrc, ro_k[n], Ks[par], n);
          else if (n < 2 * NLD) dma_one(vsrc, ro_v[n - NLD], Vs[par ^ 1], n - NLD);
#endif
        }
#if SB_ATTN_VALU_SKEW
        // Three-stage VALU pipeline over the pairs: the fmas of pair n + 1, the exp2 of pair
        // n and the packing and sum of pair n - 1 share step n, so no instruction of a step
        // waits for another of the same step.
#pragma unroll
        for (int pp = 0; pp < PPS; ++pp) {
          const int q = n * PPS + pp;
          if (q + PPS < NPAIR) {
            fa0[q + PPS] = __builtin_fmaf(c_log2, s_at(q + PPS, 0), negm[(q + PPS) / (kHalves * 8)]);
            fa1[q + PPS] = __builtin_fmaf(c_log2, s_at(q + PPS, 1), negm[(q + PPS) / (kHalves * 8)]);
          }
          ea0[q] = __builtin_amdgcn_exp2f(fa0[q]);
          ea1[q] = __builtin_amdgcn_exp2f(fa1[q]);
          if (q >= PPS) pack_pair(q - PPS, ea0[q - PPS], ea1[q - PPS]);
        }
#else
#pragma unroll
        for (int pp = 0; pp < PPS; ++pp) {
          const int q = n * PPS + pp;
          const int g = q / (kHalves * 8), r = q % (kHalves * 8);
          const int hj = r / 8, h = (r / 4) % 2, w = r % 4;
          const float e0 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(c_log2, s_cur[g][hj][8 * h + 2 * w], negm[g]));
          const float e1 = __builtin_amdgcn_exp2f(
              __builtin_fmaf(c_log2, s_cur[g][hj][8 * h + 2 * w + 1], negm[g]));
          const auto pr = M::cvt2(e0, e1);
          pw[g][hj][h][w] = __builtin_bit_cast(uint32_t, pr);
          acc[g][hj][h] = M::sum2(pr, w == 0 ? 0.f : acc[g][hj][h]);
        }
#endif
        __builtin_amdgcn_sched_barrier(0);
      }
#if SB_ATTN_VALU_SKEW
#pragma unroll
      for (int q = NPAIR - PPS; q < NPAIR; ++q) pack_pair(q, ea0[q], ea1[q]);
#endif
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        float t = 0.f;
#pragma unroll
        for (int hj = 0; hj < kHalves; ++hj)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4_t wv = {pw[g][hj][h][0], pw[g][hj][h][1], pw[g][hj][h][2],
                                pw[g][hj][h][3]};
            pb[g][hj][h] = __builtin_bit_cast(vec8, wv);
            t += acc[g][hj][h];
          }
        tsum[g] = t;
      }
    } else {
#pragma unroll
      for (int g = 0; g < RG; ++g) exp_tile(g, s_cur);
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const float pair = tsum[g] + xor32(tsum[g]);
      bad[g] = !seeded[g] || !(pair <= M::kPMax);
      bad_any |= bad[g];
    }
    if (NEXT) mask(t0 + kTileKeys, s_nxt);
    // ---- rare: seed the reference with the first live tile's max, or move it up when a
    // tile would push P past kPMax; O and l are rescaled by 2^(m_old - m_new). Scores are
    // kept unshifted, so S(it+1) needs no adjustment ----
    if (__any(bad_any)) {
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        float v = s_cur[g][0][0];
#pragma unroll
        for (int j = 0; j < kHalves; ++j)
#pragma unroll
          for (int i = 0; i < 16; ++i) v = fmaxf(v, s_cur[g][j][i]);
        const float smax = fmaxf(v, xor32(v));                    // row max of s
        const float mx = __builtin_fmaf(c_log2, smax, negm[g]);   // ... relative to m_ref
        if (bad[g] && mx != -INFINITY) {
          const float alpha = seeded[g] ? __builtin_amdgcn_exp2f(-mx) : 0.f;
          l_run[g] *= alpha;
#pragma unroll
          for (int t = 0; t < NDT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[g][t][i] *= alpha;
          m_ref[g] += mx;
          negm[g] = -m_ref[g];
          seeded[g] = true;
          exp_tile(g, s_cur);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) l_run[g] += tsum[g];
    // ---- O^T += V^T P^T; V fragments stream through a ring, kFragAhead ahead ----
    if (live) {
#if SB_ATTN_PV_PRIO
      __builtin_amdgcn_s_setprio(SB_ATTN_PV_PRIO);
#endif
      constexpr int NV = 2 * kHalves * NDT;  // (half, step, d-tile) triples
      const int vb = par;
      vec8 vring[kRing];
#pragma unroll
      for (int n = 0; n < kFragAhead; ++n) vring[n] = vfrag(vb, n);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        if (n + kFragAhead < NV) vring[(n + kFragAhead) % kRing] = vfrag(vb, n + kFragAhead);
        const int t = n % NDT, st = (n / NDT) & 1, j = n / (2 * NDT);
#pragma unroll
        for (int g = 0; g < RG; ++g) o[g][t] = M::mma(vring[n % kRing], pb[g][j][st], o[g][t]);
        __builtin_amdgcn_sched_barrier(0);
      }
#if SB_ATTN_PV_PRIO
      __builtin_amdgcn_s_setprio(0);
#endif
    }
    if (NEXT && !decltype(swap)::value) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < kHalves; ++j) s_cur[g][j] = s_nxt[g][j];
    }
    wait_vmem();
    __syncthreads();
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int slot = 0;
  auto next_slot = [](int sl) { return sl == 2 ? 0 : sl + 1; };
  using ILV = std::integral_constant<bool, SB_ATTN_LOADS_IN_QK != 0>;
  using NOILV = std::false_type;
#if SB_ATTN_UNROLL2
  // Two tiles per trip: the K/V stages are constants (fragment addresses fold into the LDS
  // instructions' offsets) and the score buffers swap roles instead of being copied. The
  // trip runs while both of its tiles have both loads due (tile it + 3 exists).
  int it = 0;
  for (; it + 3 < ntiles; it += 2) {
    iteration(it, slot, std::true_type{}, P0{}, std::true_type{}, s_cur, s_nxt, ILV{});
    slot = next_slot(slot);
    iteration(it + 1, slot, std::true_type{}, P1{}, std::true_type{}, s_nxt, s_cur, ILV{});
    slot = next_slot(slot);
  }
  // One to three tiles left; the scores of tile `it` are in s_cur.
  using PR = std::integral_constant<int, -1>;
  for (; it + 1 < ntiles; ++it) {
    iteration(it, slot, std::true_type{}, PR{}, std::false_type{}, s_cur, s_nxt, NOILV{});
    slot = next_slot(slot);
  }
  iteration(it, slot, std::false_type{}, PR{}, std::false_type{}, s_cur, s_nxt, NOILV{});
#else
  using PR = std::integral_constant<int, -1>;
  for (int it = 0; it + 1 < ntiles; ++it) {
    iteration(it, slot, std::true_type{}, PR{}, std::false_type{}, s_cur, s_nxt, NOILV{});
    slot = next_slot(slot);
  }
  iteration(ntiles - 1, slot, std::false_type{}, PR{}, std::false_type{}, s_cur, s_nxt, NOILV{});
#endif

  // ---- finish: lane holds d = 32t + 8*(i/4) + 4*lg + (i%4) of each of its rows ----
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const float l_tot = l_run[g] + xor32(l_run[g]);
    if (p[g] < 0) continue;
    const int row_in_tile = (wave * RG + g) * kWaveRows + lq;
    if (nchunks == 1) {
      const float inv = 1.f / l_tot;
      char* op = a.o + qrow[g] * a.o_s_row + qh[g] * a.o_s_head;
      // Two groups of 4 consecutive d (8 apart) per hardware pack of 8 (round to nearest even).
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int qp = 0; qp < 2; ++qp) {
          float f[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = o[g][t][8 * qp + e] * inv;
          const u32x4_t w = __builtin_bit_cast(u32x4_t, M::cvt8(f));
          const int d0 = 32 * t + 16 * qp + 4 * lg;
          *reinterpret_cast<uint2*>(op + d0 * 2) = make_uint2(w.x, w.y);
          *reinterpret_cast<uint2*>(op + (d0 + 8) * 2) = make_uint2(w.z, w.w);
        }
    } else {
      const int64_t slot =
          ((static_cast<int64_t>(kvh) * a.n_tiles + item.tile) * a.max_chunks + item.chunk) *
              TR + row_in_tile;
      float* po = a.part_o + slot * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = 32 * t + 8 * qd + 4 * lg;
          *reinterpret_cast<float4*>(po + d0) = make_float4(
              o[g][t][4 * qd], o[g][t][4 * qd + 1], o[g][t][4 * qd + 2], o[g][t][4 * qd + 3]);
        }
      if (lg == 0)
        *reinterpret_cast<float2*>(a.part_ml + slot * 2) =
            make_float2(l_tot > 0.f ? m_ref[g] : -INFINITY, l_tot);
    }
  }
}

// Combines the per-chunk partials of every row tile that needed more than one chunk:
//   M = max_c m_c,  O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.
// One workgroup per (32 rows of a row tile, KV head); 8 threads per row, each owning D / 8
// output elements, so the partial reads of a row are spread over 8 lanes.
// Chunks whose partials a merge lane loads in one batch. Six covers the host-planned split of
// the 7B 16K workload (up to five chunks per row tile): merge 15.3 -> 13.4 us against four
// (tiles with five chunks then took the two-pass loop); eight gives the same 13.5 us.
#ifndef SB_MERGE_BATCH_CHUNKS
#define SB_MERGE_BATCH_CHUNKS 6
#endif
constexpr int kMergeBatch = SB_MERGE_BATCH_CHUNKS;
// One unit: 32 rows of row tile `tile` of KV head `kvh` (mb = (tile * parts + part) * Hkv +
// kvh). Returns early when the unit has nothing to merge; its one barrier is reached by every
// thread of the workgroup (the returns before it are uniform).
template <int DT, int D>
__device__ __forceinline__ void merge_unit(const AttnArgs& a, int64_t mb, int64_t n_tiles_live,
                                           int64_t rows_kv, int* red) {
  const int tid = threadIdx.x;
  const int TR = a.tile_rows;  // 128 or 256
  const int parts = TR / 32;
  const int kvh = static_cast<int>(mb % a.num_kv_heads);
  const int64_t rest = mb / a.num_kv_heads;
  const int64_t tile = rest / parts;
  const int part = static_cast<int>(rest % parts);
  if (tile >= n_tiles_live) return;
  // kend of the whole row tile: the attention kernel chunked its key range by it.
  int pm = -1;
  for (int i = tid; i < TR; i += 256) {
    const int64_t r = tile * TR + i;
    if (r < rows_kv) {
      int pp = a.positions[r / a.group];
      if (pp >= a.kv_len) pp = static_cast<int>(a.kv_len - 1);
      pm = max(pm, pp);
    }
  }
  pm = wave_max_i(pm);
  if ((tid & 63) == 0) red[tid >> 6] = pm;
  __syncthreads();
  const int kend = max(max(red[0], red[1]), max(red[2], red[3])) + 1;
  const int nchunks = chunk_count(a, kend);
  if (nchunks <= 1) return;
  const int row_in_tile = part * 32 + tid / 8;
  const int64_t r = tile * TR + row_in_tile;
  if (r >= rows_kv) return;
  const int64_t pi = r / a.group;
  const int qh = kvh * a.group + static_cast<int>(r - pi * a.group);
  int p = a.positions[pi];
  if (p < 0) return;
  if (p >= a.kv_len) p = static_cast<int>(a.kv_len - 1);
  const int64_t qrow = a.q_by_position ? p : pi;
  constexpr int DPT = D / 8;  // values per lane (8 lanes per row)
  const int d_begin = (tid % 8) * DPT;
  const int64_t base = (static_cast<int64_t>(kvh) * a.n_tiles + tile) * a.max_chunks;
  float acc[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) acc[e] = 0.f;
  float lsum = 0.f;
  if (nchunks <= kMergeBatch) {
    // Every chunk's (m, l) and values requested at once: one round trip to memory.
    float2 ml[kMergeBatch];
    float4 v[kMergeBatch][DPT / 4];
#pragma unroll
    for (int ch = 0; ch < kMergeBatch; ++ch) {
      if (ch < nchunks) {
        const int64_t slot = (base + ch) * TR + row_in_tile;
        ml[ch] = *reinterpret_cast<const float2*>(a.part_ml + slot * 2);
#pragma unroll
        for (int q = 0; q < DPT / 4; ++q)
          v[ch][q] = *reinterpret_cast<const float4*>(a.part_o + slot * D + d_begin + 4 * q);
      }
    }
    float mmax = -INFINITY;
#pragma unroll
    for (int ch = 0; ch < kMergeBatch; ++ch)
      if (ch < nchunks) mmax = fmaxf(mmax, ml[ch].x);
#pragma unroll
    for (int ch = 0; ch < kMergeBatch; ++ch) {
      if (ch >= nchunks || ml[ch].x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml[ch].x - mmax);
      lsum += w * ml[ch].y;
#pragma unroll
      for (int q = 0; q < DPT / 4; ++q) {
        acc[4 * q] += w * v[ch][q].x;
        acc[4 * q + 1] += w * v[ch][q].y;
        acc[4 * q + 2] += w * v[ch][q].z;
        acc[4 * q + 3] += w * v[ch][q].w;
      }
    }
  } else {
    float mmax = -INFINITY;
    for (int ch = 0; ch < nchunks; ++ch)
      mmax = fmaxf(mmax, a.part_ml[((base + ch) * TR + row_in_tile) * 2]);
    // Each chunk's DPT values are loaded together (one 16-byte load per four), then weighted.
    for (int ch = 0; ch < nchunks; ++ch) {
      const int64_t slot = (base + ch) * TR + row_in_tile;
      const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + slot * 2);
      if (ml.x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml.x - mmax);
      lsum += w * ml.y;
      float4 v[DPT / 4];
#pragma unroll
      for (int q = 0; q < DPT / 4; ++q)
        v[q] = *reinterpret_cast<const float4*>(a.part_o + slot * D + d_begin + 4 * q);
#pragma unroll
      for (int q = 0; q < DPT / 4; ++q) {
        acc[4 * q] += w * v[q].x;
        acc[4 * q + 1] += w * v[q].y;
        acc[4 * q + 2] += w * v[q].z;
        acc[4 * q + 3] += w * v[q].w;
      }
    }
  }
  const float inv = 1.f / lsum;
  char* op = a.o + qrow * a.o_s_row + qh * a.o_s_head;
#pragma unroll
  for (int q = 0; q < DPT / 4; ++q) {
    const uint32_t w0 = static_cast<uint32_t>(Mma<DT>::cvt1(acc[4 * q] * inv)) |
                        (static_cast<uint32_t>(Mma<DT>::cvt1(acc[4 * q + 1] * inv)) << 16);
    const uint32_t w1 = static_cast<uint32_t>(Mma<DT>::cvt1(acc[4 * q + 2] * inv)) |
                        (static_cast<uint32_t>(Mma<DT>::cvt1(acc[4 * q + 3] * inv)) << 16);
    *reinterpret_cast<uint2*>(op + (d_begin + 4 * q) * 2) = make_uint2(w0, w1);
  }
}

// STRIDED (calls whose split follows the device row count): a fixed grid strides over the
// live units; a grid sized for every possible row tile would spend most of its workgroups on
// the count load alone. Otherwise one unit per workgroup.
template <int DT, int D, bool STRIDED>
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnBatch batch) {
  __shared__ int red[4];
  AttnArgs a = batch.a;
  const int64_t mb = select_request(batch, a, blockIdx.x, true);
  const int TR = a.tile_rows;
  const int64_t rows_kv = attn_num_rows(a) * a.group;
  const int64_t n_tiles_live = (rows_kv + TR - 1) / TR;
  if (!STRIDED) {
    merge_unit<DT, D>(a, mb, n_tiles_live, rows_kv, red);
    return;
  }
  apply_device_split(a, n_tiles_live);
  const int64_t units = n_tiles_live * a.num_kv_heads * (TR / 32);
  for (int64_t u = mb; u < units; u += gridDim.x) {
    merge_unit<DT, D>(a, u, n_tiles_live, rows_kv, red);
    __syncthreads();  // red[] is reused by the next unit
  }
}
template <int DT>
__device__ __forceinline__ float load_elem(const char* p, int64_t idx) {
  if (DT == SB_DTYPE_F32) return reinterpret_cast<const float*>(p)[idx];
  const uint16_t h = reinterpret_cast<const uint16_t*>(p)[idx];
  return DT == SB_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

template <int DT>
__device__ __forceinline__ void store_elem(char* p, int64_t idx, float f) {
  if (DT == SB_DTYPE_F32) {
    reinterpret_cast<float*>(p)[idx] = f;
  } else {
    reinterpret_cast<uint16_t*>(p)[idx] = DT == SB_DTYPE_BF16 ? f32_to_bf16(f) : f32_to_f16(f);
  }
}

constexpr int kValuMaxDim = 512;

template <int DT>
__global__ __launch_bounds__(64) void attn_valu_kernel(AttnArgs a) {
  __shared__ float qs[kValuMaxDim];
  __shared__ float ps[64];
  __shared__ const char* vrow[64];
  const int lane = threadIdx.x;
  const int64_t pi = blockIdx.x;
  const int qh = static_cast<int>(blockIdx.y);
  if (pi >= attn_num_rows(a)) return;
  int p = a.positions[pi];
  if (p < 0) return;
  if (p >= a.kv_len) p = static_cast<int>(a.kv_len - 1);
  const int kvh = qh / a.group;
  const int D = a.head_dim;
  const int64_t qrow = a.q_by_position ? p : pi;
  const char* qp = a.q + qrow * a.q_s_row + qh * a.q_s_head;
  for (int d = lane; d < D; d += 64) qs[d] = load_elem<DT>(qp, d);
  __syncthreads();

  constexpr int kU = kValuMaxDim / 64;
  float acc[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) acc[u] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  for (int t0 = 0; t0 <= p; t0 += 64) {
    const int key = t0 + lane;
    float sc = -INFINITY;
    // Each lane resolves its key's K and V rows once per chunk (block-table lookup); the V
    // row addresses go through LDS to the lanes that sum over keys.
    const char* vp = nullptr;
    if (key <= p) {
      const char* kp = key_row(a, a.k, a.k_s_head, a.k_s_seq, key, kvh);
      vp = key_row(a, a.v, a.v_s_head, a.v_s_seq, key, kvh);
      // four independent partial dot products (d, d + 1, d + 2, d + 3), summed at the end
      float dot[4] = {0.f, 0.f, 0.f, 0.f};
      int d = 0;
      for (; d + 4 <= D; d += 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dot[j] += qs[d + j] * load_elem<DT>(kp, d + j);
      }
      for (; d < D; ++d) dot[0] += qs[d] * load_elem<DT>(kp, d);
      sc = ((dot[0] + dot[1]) + (dot[2] + dot[3])) * a.scale;
    }
    vrow[lane] = vp;
    const float m_new = fmaxf(m_run, wave_max(sc));
    const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
    const float pk = key <= p ? expf(sc - m_new) : 0.f;
    l_run = l_run * alpha + wave_sum(pk);
    m_run = m_new;
    ps[lane] = pk;
    __syncthreads();
    const int nk = min(64, p - t0 + 1);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int d = lane + 64 * u;
      if (d < D) {
        float sum[4] = {0.f, 0.f, 0.f, 0.f};
        int kk = 0;
        for (; kk + 4 <= nk; kk += 4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) sum[j] += ps[kk + j] * load_elem<DT>(vrow[kk + j], d);
        }
        for (; kk < nk; ++kk) sum[0] += ps[kk] * load_elem<DT>(vrow[kk], d);
        acc[u] = acc[u] * alpha + ((sum[0] + sum[1]) + (sum[2] + sum[3]));
      }
    }
    __syncthreads();
  }
  char* op = a.o + qrow * a.o_s_row + qh * a.o_s_head;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int d = lane + 64 * u;
    if (d < D) store_elem<DT>(op, d, acc[u] / l_run);
  }
}

namespace {

// Launches the MFMA attention kernel instantiated for the addressing of `args.a`.
#define SB_ATT_LAUNCH(DT, D, grid, st, args)                                              \
  do {                                                                                    \
    switch (attn_addressing((args).a)) {                                                  \
      case kAddrFlat:                                                                     \
        SB_LAUNCH("attn_mfma", (attn_mfma_kernel<DT, D, kRowGroups, kAddrFlat>), grid,    \
                  dim3(kThreads), st, args);                                              \
        break;                                                                            \
      case kAddrPagedNarrow:                                                              \
        SB_LAUNCH("attn_mfma", (attn_mfma_kernel<DT, D, kRowGroups, kAddrPagedNarrow>),   \
                  grid, dim3(kThreads), st, args);                                        \
        break;                                                                            \
      default:                                                                            \
        SB_LAUNCH("attn_mfma", (attn_mfma_kernel<DT, D, kRowGroups, kAddrPaged>), grid,   \
                  dim3(kThreads), st, args);                                              \
    }                                                                                     \
  } while (0)

bool mfma_path(int32_t dtype, int64_t head_dim) {
  return (dtype == SB_DTYPE_BF16 || dtype == SB_DTYPE_F16) &&
         (head_dim == 64 || head_dim == 128);
}

// A host-planned launch of the single-request paged attention (sb_partial_attention_paged_plan):
// the key split (first chunk, later chunks) and the dispatch order of the work items.
struct OrderPlan {
  int ks_first = 0;
  int ks_rest = 0;
  int max_chunks = 0;
  const int32_t* order = nullptr;  // device: max_chunks * n_tiles * Hkv work items
};

// Chunking of the key range for one call. rows_upper bounds the query rows.
struct Plan {
  int ksplit;
  int ksplit_first;
  int max_chunks;
  int tile_rows;
  int64_t n_tiles;
  int64_t part_bytes;  // bytes of partials (O then m/l), 0 when no tile splits
};

Plan make_plan(int64_t rows_upper, int64_t group, int64_t num_kv_heads, int64_t kv_len,
               int64_t head_dim, int64_t block_size, bool paged,
               const OrderPlan* op = nullptr) {
  Plan pl{};
  pl.tile_rows = kWaveRows * kRowGroups * kWaves;
  pl.n_tiles = (rows_upper * group + pl.tile_rows - 1) / pl.tile_rows;
  if (op) {
    pl.ksplit = op->ks_rest;
    pl.ksplit_first = op->ks_first;
    pl.max_chunks = op->max_chunks;
  } else {
    const KeySplit sp = key_split(pl.n_tiles, num_kv_heads, kv_len, block_size, paged);
    pl.ksplit = sp.ksplit;
    pl.ksplit_first = sp.ksplit;
    pl.max_chunks = sp.max_chunks;
  }
  if (pl.max_chunks > 1)
    pl.part_bytes =
        num_kv_heads * pl.n_tiles * pl.max_chunks * pl.tile_rows * (head_dim + 2) * 4;
  return pl;
}

// Split of a call whose row count is known only on the device (dense drop-in): the kernels
// derive it from that count with key_split; the launch covers the largest item count and
// the workspace the largest partials over every possible count of row tiles.
constexpr int64_t kMergeStrideGrid = 2048;  // merge workgroups of a device-split call
struct DeviceSplitBounds {
  int64_t items;      // workgroups of the attention launch
  int64_t part_rows;  // flattened rows of split-key partials (O rows, then m/l pairs)
};
DeviceSplitBounds device_split_bounds(int64_t n_tiles_upper, int64_t num_kv_heads,
                                      int64_t kv_len, int tile_rows) {
  DeviceSplitBounds b{0, 0};
  for (int64_t t = 1; t <= n_tiles_upper; ++t) {
    const KeySplit sp = key_split(t, num_kv_heads, kv_len, 1, false);
    b.items = std::max<int64_t>(b.items, t * num_kv_heads * sp.max_chunks);
    if (sp.max_chunks > 1)
      b.part_rows = std::max<int64_t>(b.part_rows, num_kv_heads * t * sp.max_chunks * tile_rows);
  }
  return b;
}

int launch_attention(const char* fn, AttnArgs a, int32_t dtype, int64_t rows_upper,
                     bool aligned16, void* workspace, int64_t workspace_bytes,
                     hipStream_t st, const OrderPlan* op = nullptr) {
  if (rows_upper <= 0) return SB_OK;
  // The MFMA kernel masks keys with -inf scores before the scale is applied, so it takes
  // positive scales; any other scale goes to the VALU kernel, which never forms a masked score.
  if (mfma_path(dtype, a.head_dim) && aligned16 && a.scale_log2 > 0.f) {
    const Plan pl = make_plan(rows_upper, a.group, a.num_kv_heads, a.kv_len, a.head_dim,
                              a.block_size, a.paged != 0, op);
    a.ksplit = pl.ksplit;
    a.ksplit_first = pl.ksplit_first;
    a.item_order = op ? op->order : nullptr;
    a.max_chunks = pl.max_chunks;
    a.n_tiles = pl.n_tiles;
    a.tile_rows = pl.tile_rows;
    int64_t part_rows = pl.part_bytes > 0 ? a.num_kv_heads * pl.n_tiles * pl.max_chunks *
                                                pl.tile_rows
                                          : 0;
    int64_t gx = pl.n_tiles * a.num_kv_heads * pl.max_chunks;
    if (a.device_split) {
      // The kernels split by the device row count: cover every count that can occur.
      const DeviceSplitBounds b =
          device_split_bounds(pl.n_tiles, a.num_kv_heads, a.kv_len, pl.tile_rows);
      part_rows = b.part_rows;
      gx = b.items;
    }
    if (part_rows > 0) {
      const int64_t need = part_rows * (a.head_dim + 2) * 4;
      if (!workspace || workspace_bytes < need)
        return fail(fn, "workspace too small for the split-key partials");
      a.part_o = static_cast<float*>(workspace);
      a.part_ml = a.part_o + part_rows * static_cast<int64_t>(a.head_dim);
    }
    if (gx > 0x7fffffff) return fail(fn, "grid too large");
    dim3 grid(static_cast<unsigned>(gx));
    int64_t mx = pl.n_tiles * a.num_kv_heads * (pl.tile_rows / 32);
    if (a.device_split) mx = std::min<int64_t>(mx, kMergeStrideGrid);  // strided merge
    dim3 mgrid(static_cast<unsigned>(mx));
    AttnBatch one{};
    one.a = a;
    one.num_reqs = 0;
#define SB_ATT_CASE(DT, D)                                                              \
  if (dtype == DT && a.head_dim == D) {                                                 \
    SB_ATT_LAUNCH(DT, D, grid, st, one);                                               \
    if (part_rows > 0 && a.device_split)                                                \
      SB_LAUNCH("attn_merge", (attn_merge_kernel<DT, D, true>), mgrid, dim3(256), st, one); \
    else if (part_rows > 0)                                                             \
      SB_LAUNCH("attn_merge", (attn_merge_kernel<DT, D, false>), mgrid, dim3(256), st, one); \
    return check_launch(fn);                                                            \
  }
    SB_ATT_CASE(SB_DTYPE_BF16, 128)
    SB_ATT_CASE(SB_DTYPE_BF16, 64)
    SB_ATT_CASE(SB_DTYPE_F16, 128)
    SB_ATT_CASE(SB_DTYPE_F16, 64)
#undef SB_ATT_CASE
  }
  if (a.head_dim > kValuMaxDim) return fail(fn, "head_dim above 512 is not supported");
  if (rows_upper > 0x7fffffff) return fail(fn, "too many rows");
  dim3 grid(static_cast<unsigned>(rows_upper), static_cast<unsigned>(a.num_kv_heads * a.group));
  if (dtype == SB_DTYPE_F32) SB_LAUNCH("attn_valu", attn_valu_kernel<SB_DTYPE_F32>, grid, dim3(64), st, a);
  else if (dtype == SB_DTYPE_BF16) SB_LAUNCH("attn_valu", attn_valu_kernel<SB_DTYPE_BF16>, grid, dim3(64), st, a);
  else SB_LAUNCH("attn_valu", attn_valu_kernel<SB_DTYPE_F16>, grid, dim3(64), st, a);
  return check_launch(fn);
}

// Batched (varlen) launches over several requests that share the paged cache: one common
// key split for the batch (the average work per resident workgroup slot over all requests),
// requests taken longest context first, at most kMaxReqs per launch.
struct VarlenPlan {
  int ksplit = 0;
  int64_t part_bytes = 0;          // largest partial buffer of one launch
  std::vector<int> order;          // requests, longest context first (empty ones dropped)
  std::vector<int64_t> n_tiles, max_chunks, row_begin;
};

VarlenPlan make_varlen_plan(int64_t num_reqs, const int64_t* rows, const int64_t* blocks,
                            int64_t block_size, int64_t group, int64_t num_kv_heads,
                            int64_t head_dim) {
  VarlenPlan pl;
  const int tr = kWaveRows * kRowGroups * kWaves;
  pl.n_tiles.assign(num_reqs, 0);
  pl.max_chunks.assign(num_reqs, 1);
  pl.row_begin.assign(num_reqs, 0);
  int64_t work = 0, kv_max = 0, run = 0;
  for (int64_t r = 0; r < num_reqs; ++r) {
    pl.row_begin[r] = run;
    run += rows[r];
    pl.n_tiles[r] = (rows[r] * group + tr - 1) / tr;
    const int64_t kv = blocks[r] * block_size;
    if (rows[r] > 0 && blocks[r] > 0) {
      pl.order.push_back(static_cast<int>(r));
      work += pl.n_tiles[r] * num_kv_heads * (kv / 2);
      kv_max = kv > kv_max ? kv : kv_max;
    }
  }
  std::stable_sort(pl.order.begin(), pl.order.end(), [&](int x, int y) {
    return blocks[x] * block_size > blocks[y] * block_size;
  });
  int64_t ks = work / kResidentSlots;
  ks = ks / kTileKeys * kTileKeys;
  if (ks < 512) ks = 512;
  const int64_t cap = chunk_cap(block_size);
  if (ks > cap) ks = cap;
  const int64_t kv_pad = (kv_max + kTileKeys - 1) / kTileKeys * kTileKeys;
  if (ks > kv_pad) ks = kv_pad;
  if (ks < kTileKeys) ks = kTileKeys;
  pl.ksplit = static_cast<int>(ks);
  for (size_t g0 = 0; g0 < pl.order.size(); g0 += kMaxReqs) {
    int64_t part_rows = 0;
    for (size_t i = g0; i < pl.order.size() && i < g0 + kMaxReqs; ++i) {
      const int r = pl.order[i];
      const int64_t kv = blocks[r] * block_size;
      pl.max_chunks[r] = (kv + ks - 1) / ks;
      if (pl.max_chunks[r] > 1) part_rows += num_kv_heads * pl.n_tiles[r] * pl.max_chunks[r] * tr;
    }
    const int64_t bytes = part_rows * (head_dim + 2) * 4;
    if (bytes > pl.part_bytes) pl.part_bytes = bytes;
  }
  return pl;
}

// `a` describes the shared cache, q, out and strides; positions, q and out hold the requests'
// rows back to back; request r's block table is block_tables[r * bt_stride ...].
int launch_attention_varlen(const char* fn, AttnArgs a, int32_t dtype, int64_t num_reqs,
                            const int64_t* rows, const int64_t* blocks, int64_t bt_stride,
                            bool aligned16, void* workspace, int64_t workspace_bytes,
                            hipStream_t st) {
  const VarlenPlan pl = make_varlen_plan(num_reqs, rows, blocks, a.block_size, a.group,
                                         a.num_kv_heads, a.head_dim);
  if (!(mfma_path(dtype, a.head_dim) && aligned16 && a.scale_log2 > 0.f)) {
    // VALU path: one launch per request.
    for (int r : pl.order) {
      AttnArgs b = a;
      b.positions = a.positions + pl.row_begin[r];
      b.q = a.q + pl.row_begin[r] * a.q_s_row;
      b.o = a.o + pl.row_begin[r] * a.o_s_row;
      b.num_rows = rows[r];
      b.block_table = a.block_table + r * bt_stride;
      b.nb_per_seq = blocks[r];
      b.kv_len = blocks[r] * a.block_size;
      const int rc = launch_attention(fn, b, dtype, rows[r], aligned16, workspace,
                                      workspace_bytes, st);
      if (rc) return rc;
    }
    return SB_OK;
  }
  if (pl.part_bytes > 0 && (!workspace || workspace_bytes < pl.part_bytes))
    return fail(fn, "workspace too small for the split-key partials");
  const int tr = kWaveRows * kRowGroups * kWaves;
  a.ksplit = pl.ksplit;
  a.ksplit_first = pl.ksplit;
  a.tile_rows = tr;
  a.part_o = pl.part_bytes > 0 ? static_cast<float*>(workspace) : nullptr;
  for (size_t g0 = 0; g0 < pl.order.size(); g0 += kMaxReqs) {
    AttnBatch b{};
    b.a = a;
    b.num_reqs = 0;
    int64_t items = 0, merges = 0, part_rows = 0, part_total = 0;
    bool split = false;
    for (size_t i = g0; i < pl.order.size() && i < g0 + kMaxReqs; ++i) {
      const int r = pl.order[i];
      if (pl.max_chunks[r] > 1) part_total += a.num_kv_heads * pl.n_tiles[r] * pl.max_chunks[r] * tr;
    }
    for (size_t i = g0; i < pl.order.size() && i < g0 + kMaxReqs; ++i) {
      const int r = pl.order[i];
      ReqSlice& sl = b.req[b.num_reqs++];
      sl.item_begin = items;
      sl.merge_begin = merges;
      sl.row_begin = pl.row_begin[r];
      sl.num_rows = rows[r];
      sl.bt_begin = r * bt_stride;
      sl.num_blocks = blocks[r];
      sl.n_tiles = pl.n_tiles[r];
      sl.max_chunks = static_cast<int>(pl.max_chunks[r]);
      sl.part_begin = part_rows;
      items += pl.n_tiles[r] * a.num_kv_heads * pl.max_chunks[r];
      merges += pl.n_tiles[r] * a.num_kv_heads * (tr / 32);
      if (pl.max_chunks[r] > 1) {
        part_rows += a.num_kv_heads * pl.n_tiles[r] * pl.max_chunks[r] * tr;
        split = true;
      }
    }
    if (b.a.part_o) b.a.part_ml = b.a.part_o + part_total * a.head_dim;
    if (items > 0x7fffffff || merges > 0x7fffffff) return fail(fn, "grid too large");
    const dim3 grid(static_cast<unsigned>(items));
    const dim3 mgrid(static_cast<unsigned>(merges));
#define SB_ATT_VCASE(DT, D)                                                             \
  if (dtype == DT && a.head_dim == D) {                                                 \
    SB_ATT_LAUNCH(DT, D, grid, st, b);                                                 \
    if (split) SB_LAUNCH("attn_merge", (attn_merge_kernel<DT, D, false>), mgrid, dim3(256), st, b); \
    const int rc = check_launch(fn);                                                    \
    if (rc) return rc;                                                                  \
    continue;                                                                           \
  }
    SB_ATT_VCASE(SB_DTYPE_BF16, 128)
    SB_ATT_VCASE(SB_DTYPE_BF16, 64)
    SB_ATT_VCASE(SB_DTYPE_F16, 128)
    SB_ATT_VCASE(SB_DTYPE_F16, 64)
#undef SB_ATT_VCASE
    return fail(fn, "internal: no MFMA kernel for this dtype / head_dim");
  }
  return SB_OK;
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((int64_t{1} << l) < v) ++l;
  return l;
}

int64_t part_bytes_for(int32_t dtype, int64_t rows_upper, int64_t group, int64_t num_kv_heads,
                       int64_t kv_len, int64_t head_dim, int64_t block_size, bool paged) {
  if (!mfma_path(dtype, head_dim)) return 0;
  return make_plan(rows_upper, group, num_kv_heads, kv_len, head_dim, block_size, paged)
      .part_bytes;
}

// ---- Host planning of the single-request paged attention ----
// Given the query positions on the host, the planner knows every work item's key range, so it
// can (a) split the tail of each row tile's key range more finely than the default rule and
// (b) dispatch the items longest first, which the hardware dispatcher (in workgroup order, to
// whichever slot frees first) then turns into a longest-processing-time schedule. The default
// order (chunk ascending, row tile descending) leaves short first chunks of short row tiles
// ahead of long second chunks, and one long chunk per row tile leaves the last slots
// idle: on the Qwen2.5-7B 16K workload, 0.88 of the ideal makespan against 0.95 planned (one
// tile of per-item overhead in the schedule model).

// Per-item set-up (Q loads, block-table staging, pipeline fill) in 64-key-tile units.
constexpr double kItemOverheadTiles = 1.0;

// Makespan of a longest-first list schedule of `costs` (sorted descending) on `slots` slots.
double lpt_makespan(const std::vector<double>& costs, int slots) {
  std::vector<double> load(static_cast<size_t>(slots), 0.0);
  std::make_heap(load.begin(), load.end(), std::greater<double>());
  for (double c : costs) {
    std::pop_heap(load.begin(), load.end(), std::greater<double>());
    load.back() += c;
    std::push_heap(load.begin(), load.end(), std::greater<double>());
  }
  return *std::max_element(load.begin(), load.end());
}

struct HostOrderPlan {
  int ks_first = 0, ks_rest = 0, max_chunks = 0;
  std::vector<int32_t> order;  // work items, longest first
};

HostOrderPlan plan_paged_order(const int32_t* pos, int64_t num_rows, int64_t group,
                               int64_t num_kv_heads, int64_t kv_len, int64_t block_size) {
  HostOrderPlan hp;
  const int tr = kWaveRows * kRowGroups * kWaves;
  const int64_t rows_kv = num_rows * group;
  const int64_t n_tiles = (rows_kv + tr - 1) / tr;
  // Key range of each row tile, as the kernel finds it (positions clamped to the table).
  std::vector<int64_t> kend(static_cast<size_t>(n_tiles), 0);
  for (int64_t t = 0; t < n_tiles; ++t) {
    int64_t m = -1;
    const int64_t r_end = std::min<int64_t>((t + 1) * tr, rows_kv);
    for (int64_t pi = t * tr / group; pi <= (r_end - 1) / group; ++pi) {
      int64_t pp = pos[pi];
      if (pp >= kv_len) pp = kv_len - 1;
      if (pp >= 0) m = std::max(m, pp);
    }
    kend[static_cast<size_t>(t)] = m + 1;
  }
  const KeySplit base = key_split(n_tiles, num_kv_heads, kv_len, block_size, true);
  AttnArgs geo{};
  auto cost_of = [&](int chunk, int64_t t) -> int64_t {  // 64-key tiles of one item
    const int64_t k0 = chunk_begin(geo, chunk);
    const int64_t k1 = std::min<int64_t>(k0 + chunk_len(geo, chunk), kend[static_cast<size_t>(t)]);
    return k1 > k0 ? (k1 - k0 + kTileKeys - 1) / kTileKeys : 0;
  };
  // Candidate splits: the default first chunk, later chunks of 1, 1/2 or 1/4 of it (at least
  // 512 keys); the shortest modelled makespan wins, ties going to the longer later chunks
  // (fewer split-key partials to write and merge).
  double best = 0.0;
  for (int div : {1, 2, 4}) {
    int rest = base.ksplit / div / kTileKeys * kTileKeys;
    if (div > 1 && rest < 512) break;
    if (rest < kTileKeys) rest = kTileKeys;
    geo.ksplit_first = base.ksplit;
    geo.ksplit = rest;
    std::vector<double> costs;
    for (int64_t t = 0; t < n_tiles; ++t)
      for (int c = 0; c < chunk_count(geo, kend[static_cast<size_t>(t)]); ++c) {
        const int64_t tiles = cost_of(c, t);
        if (tiles > 0)
          for (int64_t h = 0; h < num_kv_heads; ++h)
            costs.push_back(static_cast<double>(tiles) + kItemOverheadTiles);
      }
    std::sort(costs.begin(), costs.end(), std::greater<double>());
    const double ms = costs.empty() ? 0.0 : lpt_makespan(costs, kResidentSlots);
    if (div == 1 || ms < best * 0.995) {
      best = ms;
      hp.ks_first = geo.ksplit_first;
      hp.ks_rest = geo.ksplit;
    }
  }
  geo.ksplit_first = hp.ks_first;
  geo.ksplit = hp.ks_rest;
  hp.max_chunks = chunk_count(geo, kv_len);
  // Every work item of the launch (the encoding of decode_item), longest first; items past a
  // row tile's key range run last and exit at once.
  const int64_t n_items = static_cast<int64_t>(hp.max_chunks) * n_tiles * num_kv_heads;
  std::vector<std::pair<int64_t, int32_t>> keyed(static_cast<size_t>(n_items));
  for (int64_t b = 0; b < n_items; ++b) {
    const int64_t rest = b / num_kv_heads;
    const int64_t tile = n_tiles - 1 - rest % n_tiles;
    const int chunk = static_cast<int>(rest / n_tiles);
    keyed[static_cast<size_t>(b)] = {-cost_of(chunk, tile), static_cast<int32_t>(b)};
  }
  std::stable_sort(keyed.begin(), keyed.end(),
                   [](const auto& x, const auto& y) { return x.first < y.first; });
  hp.order.resize(static_cast<size_t>(n_items));
  for (int64_t i = 0; i < n_items; ++i) hp.order[static_cast<size_t>(i)] = keyed[static_cast<size_t>(i)].second;
  return hp;
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int64_t sb_partial_prefill_attention_workspace_size(int64_t num_heads,
                                                               int64_t seq_len,
                                                               int64_t head_dim,
                                                               int32_t dtype) {
  // positions (S) + count, rounded to 256 bytes, then the split-key partials of the largest
  // split the device row count can select.
  const int64_t idx = ((seq_len + 1) * 4 + 255) / 256 * 256;
  if (!mfma_path(dtype, head_dim) || num_heads <= 0 || seq_len <= 0) return idx;
  const int tile_rows = kWaveRows * kRowGroups * kWaves;
  const DeviceSplitBounds b =
      device_split_bounds((seq_len + tile_rows - 1) / tile_rows, num_heads, seq_len, tile_rows);
  return idx + b.part_rows * (head_dim + 2) * 4;
}

extern "C" int sb_partial_prefill_attention(void* out, const void* q, const void* k,
                                            const void* v, const uint8_t* compute_mask,
                                            void* workspace, int64_t workspace_bytes,
                                            int64_t num_heads, int64_t seq_len,
                                            int64_t head_dim, float scale, const int64_t* qs,
                                            const int64_t* ks, const int64_t* vs,
                                            const int64_t* os, int32_t dtype, void* stream) {
  const char* fn = "sb_partial_prefill_attention";
  clear_error();
  if (num_heads == 0 || seq_len == 0 || head_dim == 0) return SB_OK;
  if (elem_size(dtype) == 0) return fail(fn, "invalid dtype");
  if (!out || !q || !k || !v || !compute_mask || !workspace || !qs || !ks || !vs || !os)
    return fail(fn, "null pointer argument");
  if (qs[2] != 1 || ks[2] != 1 || vs[2] != 1 || os[2] != 1)
    return fail(fn, "head_dim must be contiguous (stride 1)");
  if (seq_len > 0x7ffffffe) return fail(fn, "sequence too long");
  if (workspace_bytes < sb_partial_prefill_attention_workspace_size(num_heads, seq_len,
                                                                    head_dim, dtype))
    return fail(fn, "workspace too small");
  const int64_t es = elem_size(dtype);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* pos = static_cast<int32_t*>(workspace);
  const int64_t idx_bytes = ((seq_len + 1) * 4 + 255) / 256 * 256;

  // Zero the rows that are not computed (output semantics of torch.zeros_like + row writes).
  {
    const int vb = vec_bytes({reinterpret_cast<int64_t>(out), os[0] * es, os[1] * es,
                              head_dim * es});
    const int vpr = static_cast<int>(head_dim * es / vb);
    const int64_t total = num_heads * seq_len * vpr;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    char* o = static_cast<char*>(out);
    const int64_t sh = os[0] * es, ss = os[1] * es;
    if (vb >= 16) SB_LAUNCH("zero_rows", zero_rows_kernel<16>, grid, dim3(256), st, o, compute_mask, num_heads, seq_len, sh, ss, vpr);
    else if (vb == 8) SB_LAUNCH("zero_rows", zero_rows_kernel<8>, grid, dim3(256), st, o, compute_mask, num_heads, seq_len, sh, ss, vpr);
    else if (vb == 4) SB_LAUNCH("zero_rows", zero_rows_kernel<4>, grid, dim3(256), st, o, compute_mask, num_heads, seq_len, sh, ss, vpr);
    else SB_LAUNCH("zero_rows", zero_rows_kernel<2>, grid, dim3(256), st, o, compute_mask, num_heads, seq_len, sh, ss, vpr);
  }
  SB_LAUNCH("mask_compact", mask_compact_kernel<0>, dim3(1), dim3(1024), st, compute_mask, seq_len,
            pos, pos + seq_len);
  int rc = check_launch(fn);
  if (rc) return rc;

  AttnArgs a{};
  a.q = static_cast<const char*>(q);
  a.o = static_cast<char*>(out);
  a.q_s_row = qs[1] * es;
  a.q_s_head = qs[0] * es;
  a.o_s_row = os[1] * es;
  a.o_s_head = os[0] * es;
  a.q_by_position = 1;
  a.positions = pos;
  a.count_ptr = pos + seq_len;
  a.num_rows = seq_len;
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.k_s_head = ks[0] * es;
  a.v_s_head = vs[0] * es;
  a.k_s_seq = ks[1] * es;
  a.v_s_seq = vs[1] * es;
  a.paged = 0;
  a.block_size = 1;
  a.bs_log2 = -1;
  a.kv_len = seq_len;
  a.num_kv_heads = static_cast<int>(num_heads);
  a.group = 1;
  a.head_dim = static_cast<int>(head_dim);
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.device_split = 1;  // the row count is known on the device only
  const bool aligned16 =
      vec_bytes({reinterpret_cast<int64_t>(q), reinterpret_cast<int64_t>(k),
                 reinterpret_cast<int64_t>(v), reinterpret_cast<int64_t>(out), qs[0] * es,
                 qs[1] * es, ks[0] * es, ks[1] * es, vs[0] * es, vs[1] * es, os[0] * es,
                 os[1] * es}) >= 16;
  return launch_attention(fn, a, dtype, seq_len, aligned16,
                          static_cast<char*>(workspace) + idx_bytes,
                          workspace_bytes - idx_bytes, st);
}

extern "C" int64_t sb_partial_attention_paged_workspace_size(int64_t num_rows,
                                                             int64_t num_q_heads,
                                                             int64_t num_kv_heads,
                                                             int64_t head_dim,
                                                             int64_t block_size,
                                                             int64_t num_blocks_per_seq,
                                                             int32_t dtype) {
  if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0) return 0;
  return part_bytes_for(dtype, num_rows, num_q_heads / num_kv_heads, num_kv_heads,
                        num_blocks_per_seq * block_size, head_dim, block_size, true);
}

namespace {

// Shared argument checks and set-up of the paged entry points (single and batched).
int paged_args(const char* fn, AttnArgs* pa, bool* aligned16, void* out, const void* q,
               const void* kv_cache, const int32_t* block_table, const int32_t* positions,
               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
               int64_t num_blocks_total, float scale, const int64_t* qs, const int64_t* os,
               const int64_t* kvs, int32_t dtype) {
  if (elem_size(dtype) == 0) return fail(fn, "invalid dtype");
  if (!out || !q || !kv_cache || !block_table || !positions || !qs || !os || !kvs)
    return fail(fn, "null pointer argument");
  if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(fn, "num_q_heads must be a multiple of num_kv_heads");
  if (block_size <= 0 || num_blocks_total <= 0) return fail(fn, "empty block table or pool");
  if (qs[2] != 1 || os[2] != 1 || kvs[4] != 1)
    return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  AttnArgs a{};
  a.q = static_cast<const char*>(q);
  a.o = static_cast<char*>(out);
  a.q_s_row = qs[0] * es;
  a.q_s_head = qs[1] * es;
  a.o_s_row = os[0] * es;
  a.o_s_head = os[1] * es;
  a.q_by_position = 0;
  a.positions = positions;
  a.count_ptr = nullptr;
  a.k = static_cast<const char*>(kv_cache);
  a.v = static_cast<const char*>(kv_cache) + kvs[1] * es;
  a.k_s_head = kvs[2] * es;
  a.v_s_head = kvs[2] * es;
  a.paged = 1;
  a.block_table = block_table;
  a.block_size = block_size;
  a.bs_log2 = log2_exact(block_size);
  a.nb_total = num_blocks_total;
  a.s_block = kvs[0] * es;
  a.s_pos = kvs[3] * es;
  // Narrow addressing: 32-bit block strides and in-block offsets, and (for 32-bit load
  // offsets) every row of the cache within 4 GiB of the K and V bases.
  const int64_t extent = (num_blocks_total - 1) * a.s_block + (block_size - 1) * a.s_pos +
                         (num_kv_heads - 1) * std::max(a.k_s_head, a.v_s_head) + head_dim * es;
  a.narrow_ofs = a.bs_log2 >= 0 && a.s_block >= 0 && a.s_block <= 0xFFFFFFFFll &&
                 a.s_pos >= 0 && a.s_pos < (1ll << 24) && block_size < (1ll << 24) &&
                 extent < (1ll << 32);
  a.num_kv_heads = static_cast<int>(num_kv_heads);
  a.group = static_cast<int>(num_q_heads / num_kv_heads);
  a.head_dim = static_cast<int>(head_dim);
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  *aligned16 = vec_bytes({reinterpret_cast<int64_t>(q), reinterpret_cast<int64_t>(kv_cache),
                          reinterpret_cast<int64_t>(out), qs[0] * es, qs[1] * es, os[0] * es,
                          os[1] * es, kvs[0] * es, kvs[1] * es, kvs[2] * es, kvs[3] * es}) >= 16;
  *pa = a;
  return SB_OK;
}

}  // namespace

extern "C" int sb_partial_attention_paged(void* out, const void* q, const void* kv_cache,
                                          const int32_t* block_table, const int32_t* positions,
                                          void* workspace, int64_t workspace_bytes,
                                          int64_t num_rows, int64_t num_q_heads,
                                          int64_t num_kv_heads, int64_t head_dim,
                                          int64_t block_size, int64_t num_blocks_total,
                                          int64_t num_blocks_per_seq, float scale,
                                          const int64_t* qs, const int64_t* os,
                                          const int64_t* kvs, int32_t dtype, void* stream) {
  const char* fn = "sb_partial_attention_paged";
  clear_error();
  if (num_rows == 0 || num_q_heads == 0 || head_dim == 0) return SB_OK;
  if (num_blocks_per_seq <= 0) return fail(fn, "empty block table or pool");
  AttnArgs a;
  bool aligned16 = false;
  const int rc = paged_args(fn, &a, &aligned16, out, q, kv_cache, block_table, positions,
                            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_total,
                            scale, qs, os, kvs, dtype);
  if (rc) return rc;
  a.num_rows = num_rows;
  a.nb_per_seq = num_blocks_per_seq;
  a.kv_len = num_blocks_per_seq * block_size;
  return launch_attention(fn, a, dtype, num_rows, aligned16, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream));
}

// Launch plan of sb_partial_attention_paged_planned from HOST positions (see the header).
extern "C" int64_t sb_partial_attention_paged_plan(const int32_t* positions, int64_t num_rows,
                                                   int64_t num_q_heads, int64_t num_kv_heads,
                                                   int64_t head_dim, int64_t block_size,
                                                   int64_t num_blocks_per_seq, int32_t dtype,
                                                   int32_t* plan, int64_t capacity) {
  const char* fn = "sb_partial_attention_paged_plan";
  clear_error();
  // errors are returned negated, apart from the entry counts
  auto err = [&](const char* msg) { return -static_cast<int64_t>(fail(fn, msg)); };
  if (num_rows < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      block_size <= 0 || num_blocks_per_seq <= 0)
    return err("invalid shape");
  if (num_rows > 0 && !positions) return err("null positions");
  const int64_t kv_len = num_blocks_per_seq * block_size;
  if (kv_len > 0x7ffffffe) return err("sequence too long");
  HostOrderPlan hp;
  if (num_rows > 0 && mfma_path(dtype, head_dim))
    hp = plan_paged_order(positions, num_rows, num_q_heads / num_kv_heads, num_kv_heads, kv_len,
                          block_size);
  const int64_t need = 3 + static_cast<int64_t>(hp.order.size());
  if (!plan) return need;
  if (capacity < need) return err("plan buffer too small");
  plan[0] = hp.ks_first;
  plan[1] = hp.ks_rest;
  plan[2] = hp.max_chunks;
  if (!hp.order.empty()) std::memcpy(plan + 3, hp.order.data(), hp.order.size() * sizeof(int32_t));
  return need;
}

extern "C" int64_t sb_partial_attention_paged_planned_workspace_size(
    int64_t num_rows, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int32_t max_chunks, int32_t dtype) {
  if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_chunks <= 1 ||
      !mfma_path(dtype, head_dim))
    return 0;
  const int tr = kWaveRows * kRowGroups * kWaves;
  const int64_t n_tiles = (num_rows * (num_q_heads / num_kv_heads) + tr - 1) / tr;
  return num_kv_heads * n_tiles * max_chunks * tr * (head_dim + 2) * 4;
}

extern "C" int sb_partial_attention_paged_planned(
    void* out, const void* q, const void* kv_cache, const int32_t* block_table,
    const int32_t* positions, const int32_t* item_order, int64_t num_items, int32_t ks_first,
    int32_t ks_rest, int32_t max_chunks, void* workspace, int64_t workspace_bytes,
    int64_t num_rows,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
    int64_t num_blocks_total, int64_t num_blocks_per_seq, float scale, const int64_t* qs,
    const int64_t* os, const int64_t* kvs, int32_t dtype, void* stream) {
  const char* fn = "sb_partial_attention_paged_planned";
  clear_error();
  if (num_rows == 0 || num_q_heads == 0 || head_dim == 0) return SB_OK;
  if (num_blocks_per_seq <= 0) return fail(fn, "empty block table or pool");
  AttnArgs a;
  bool aligned16 = false;
  const int rc = paged_args(fn, &a, &aligned16, out, q, kv_cache, block_table, positions,
                            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_total,
                            scale, qs, os, kvs, dtype);
  if (rc) return rc;
  a.num_rows = num_rows;
  a.nb_per_seq = num_blocks_per_seq;
  a.kv_len = num_blocks_per_seq * block_size;
  OrderPlan op;
  const bool use = mfma_path(dtype, head_dim) && max_chunks > 0;
  if (use) {
    // The split must cover the key range in at most max_chunks chunks that each fit the
    // kernel's staged block-table slice.
    const int64_t cap = chunk_cap(block_size);
    if (!item_order) return fail(fn, "null item order");
    const int64_t n_tiles = (num_rows * (num_q_heads / num_kv_heads) +
                             kWaveRows * kRowGroups * kWaves - 1) /
                            (kWaveRows * kRowGroups * kWaves);
    if (num_items != static_cast<int64_t>(max_chunks) * n_tiles * num_kv_heads)
      return fail(fn, "num_items is not max_chunks * row tiles * num_kv_heads");
    if (ks_first <= 0 || ks_rest <= 0 || ks_first % kTileKeys || ks_rest % kTileKeys ||
        ks_first > cap || ks_rest > cap)
      return fail(fn, "invalid key split");
    AttnArgs geo{};
    geo.ksplit_first = ks_first;
    geo.ksplit = ks_rest;
    if (chunk_count(geo, a.kv_len) != max_chunks)
      return fail(fn, "max_chunks does not match the key split and the block table");
    op.ks_first = ks_first;
    op.ks_rest = ks_rest;
    op.max_chunks = max_chunks;
    op.order = item_order;
  }
  return launch_attention(fn, a, dtype, num_rows, aligned16, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream), use ? &op : nullptr);
}

extern "C" int64_t sb_partial_attention_paged_varlen_workspace_size(
    int64_t num_reqs, const int64_t* rows_per_req, const int64_t* blocks_per_req,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
    int32_t dtype) {
  if (num_reqs <= 0 || !rows_per_req || !blocks_per_req || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || block_size <= 0)
    return 0;
  const int64_t group = num_q_heads / num_kv_heads;
  if (!mfma_path(dtype, head_dim)) return 0;
  return make_varlen_plan(num_reqs, rows_per_req, blocks_per_req, block_size, group,
                          num_kv_heads, head_dim)
      .part_bytes;
}

extern "C" int sb_partial_attention_paged_varlen(
    void* out, const void* q, const void* kv_cache, const int32_t* block_tables,
    int64_t block_table_stride, const int32_t* positions, int64_t num_reqs,
    const int64_t* rows_per_req, const int64_t* blocks_per_req, void* workspace,
    int64_t workspace_bytes, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t num_blocks_total, float scale, const int64_t* qs,
    const int64_t* os, const int64_t* kvs, int32_t dtype, void* stream) {
  const char* fn = "sb_partial_attention_paged_varlen";
  clear_error();
  if (num_reqs == 0 || num_q_heads == 0 || head_dim == 0) return SB_OK;
  if (num_reqs < 0 || !rows_per_req || !blocks_per_req)
    return fail(fn, "null per-request array");
  int64_t total_rows = 0;
  for (int64_t r = 0; r < num_reqs; ++r) {
    if (rows_per_req[r] < 0 || blocks_per_req[r] < 0)
      return fail(fn, "negative per-request row or block count");
    if (rows_per_req[r] > 0 && blocks_per_req[r] > block_table_stride)
      return fail(fn, "a request has more blocks than the block-table row holds");
    total_rows += rows_per_req[r];
  }
  if (total_rows == 0) return SB_OK;
  AttnArgs a;
  bool aligned16 = false;
  const int rc = paged_args(fn, &a, &aligned16, out, q, kv_cache, block_tables, positions,
                            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_total,
                            scale, qs, os, kvs, dtype);
  if (rc) return rc;
  return launch_attention_varlen(fn, a, dtype, num_reqs, rows_per_req, blocks_per_req,
                                 block_table_stride, aligned16, workspace, workspace_bytes,
                                 static_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------------------------------
// No-allocation form of sb_partial_attention_paged: the split-key partials live in a fixed
// device array of this library instead of a caller workspace.
// ------------------------------------------------------------------------------------------

namespace sb {
namespace {

// Largest partial buffer the no-allocation entry serves (the Qwen2.5-7B 16K-context call
// with 2458 recompute rows needs 72 MB). Every GPU the library runs on holds one copy of the
// array, from module load until the process ends.
constexpr int64_t kNoAllocScratchBytes = int64_t{128} << 20;

}  // namespace
}  // namespace sb

// File scope, one copy per device. Host code never passes this name to a kernel: the host
// symbol is only a handle; the device address comes from hipGetSymbolAddress below.
static __device__ __align__(256) char scratch[sb::kNoAllocScratchBytes];

namespace sb {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device (with that
// device current) and kept; nullptr with the error recorded when the lookup fails.
void* scratch_for_current_device(const char* fn) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(std::string(fn) + ": hipGetDevice failed: " + hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error(std::string(fn) + ": device index out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !ptr) {
      set_error(std::string(fn) + ": hipGetSymbolAddress(scratch) failed: " +
                hipGetErrorString(r));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace sb

extern "C" int64_t sb_partial_attention_paged_noalloc_max_scratch(void) {
  return sb::kNoAllocScratchBytes;
}

extern "C" int sb_partial_attention_paged_noalloc(
    void* out, const void* q, const void* kv_cache, const int32_t* block_table,
    const int32_t* positions, int64_t num_rows, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t block_size, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    float scale, const int64_t* qs, const int64_t* os, const int64_t* kvs, int32_t dtype,
    void* stream) {
  const char* fn = "sb_partial_attention_paged_noalloc";
  clear_error();
  if (num_rows == 0 || num_q_heads == 0 || head_dim == 0) return SB_OK;
  if (num_blocks_per_seq <= 0) return fail(fn, "empty block table or pool");
  const int64_t need = sb_partial_attention_paged_workspace_size(
      num_rows, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_per_seq, dtype);
  if (need > kNoAllocScratchBytes)
    return fail(fn, "this call needs " + std::to_string(need) +
                        " bytes of split-key partials; the no-allocation entry holds at most " +
                        std::to_string(kNoAllocScratchBytes) +
                        " (use sb_partial_attention_paged with a workspace)");
  AttnArgs a;
  bool aligned16 = false;
  const int rc = paged_args(fn, &a, &aligned16, out, q, kv_cache, block_table, positions,
                            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_total,
                            scale, qs, os, kvs, dtype);
  if (rc) return rc;
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_for_current_device(fn);
    if (!ws) return SB_ERR_INVALID_ARGUMENT;
  }
  a.num_rows = num_rows;
  a.nb_per_seq = num_blocks_per_seq;
  a.kv_len = num_blocks_per_seq * block_size;
  return launch_attention(fn, a, dtype, num_rows, aligned16, ws, need,
                          static_cast<hipStream_t>(stream));
}
