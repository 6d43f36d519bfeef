// Row movers for the KV-reuse path: donor-KV scatter (flat and paged), fused scatter + RoPE,
// in-place paged RoPE, snapshot permutations (delta and NoPE forms) and the flat
// rope_correct_k. Every operation moves head_dim-long rows between two row addressings:
//
//   ROW_FLAT_POS   row of a [.., S, D] tensor selected by a position value   (donor buffers)
//   ROW_PAGED_POS  slot of a paged cache selected by a logical position
//                  through a block table                                     (KV caches)
//   ROW_INDEX      row i of a dense [P, .., D] staging buffer                (snapshots)
//
// One thread owns one VB-byte vector of one pair's row and walks every (layer, head) plane
// in its group, so a rotation's cos/sin are evaluated once per (pair, frequency) and reused
// for all layers and heads. Rows are head_dim * elem bytes long; a 128-dim bf16 row is
// 16 lanes x 16 bytes, so a wave moves four 256-byte rows per instruction.
//
// RoPE arithmetic follows the interleaved (GPT-J) convention of
// semblend_core/rope_correction.py:163-178 and :317-326, in fp32:
//   e' = e*c - o*s,  o' = e*s + o*c,  theta = delta * inv_freq[i]
// with one rounding to the cache dtype (the CPU path of the reference, :328). This file is
// compiled with -ffp-contract=off so each product and sum rounds exactly like torch's CPU
// elementwise ops.

#include <algorithm>
#include <cstring>

#include "sb_common.h"

namespace sb {

// ROW_DONOR_GROUPED: ROW_DONOR_POS with the pairs grouped by donor so that every workgroup's
// pairs share one donor (the donor index is then wave-uniform and its strides and layer table
// are read by scalar loads).
enum RowMode : int {
  ROW_FLAT_POS = 0,
  ROW_PAGED_POS = 1,
  ROW_INDEX = 2,
  ROW_DONOR_POS = 3,
  ROW_DONOR_GROUPED = 4
};
// Rotation of K rows: none; by (destination - source position); NoPE (strip R(source), apply
// R(destination)); by one delta for every pair; by a per-pair delta (MoveArgs::deltas).
enum RotMode : int { ROT_NONE = 0, ROT_DELTA = 1, ROT_NOPE = 2, ROT_CONST = 3, ROT_PAIR = 4 };

// Launch shape and access hints, tuned on MI355X for the 7B-shape workloads (28 layers x
// 4 KV heads x 128, bf16). 256-thread blocks (128/512/1024 were slower). The pair movers keep
// 4 rows in flight per thread and walk 2 layers x all heads of one plane (1.6 GB scatter:
// 288 us; 4 layers 292, 7 layers 300, 8 rows in flight 298; 1 or 2 rows in flight 302-306).
// Nontemporal loads and stores: the rows are touched once (316 -> 291 us for the scatter).
// The row-centric RoPE runs short threads: about 16384 blocks (4 of the 112 rows of
// K[28,4,8192,128] per thread, cos/sin evaluated once for them) with 2 rows in flight: 76.8 us
// against 84.3 us for 4096 blocks of 14 rows, 8 in flight; 2 rows per thread 103 us (the
// cos/sin dominate), 7 rows 79.3 us; 4 rows in flight 79.7 us, 1 row 88.3 us (interleaved
// runs in one process, one box). A plain 16-byte copy behaves the same way: one vector per
// thread moves 6.5 TB/s, four 6.2-6.3, eight 4.3.
#ifndef SB_MOVE_THREADS
#define SB_MOVE_THREADS 256
#endif
#ifndef SB_MOVE_BATCH
#define SB_MOVE_BATCH 4
#endif
#ifndef SB_ROPE_BATCH
#define SB_ROPE_BATCH 2
#endif
#ifndef SB_ROPE_TARGET_BLOCKS
#define SB_ROPE_TARGET_BLOCKS 16384
#endif
// (layer, head) rows per thread of the row-centric RoPE; 0 derives it from the block target.
#ifndef SB_ROPE_ROWS_PER_GROUP
#define SB_ROPE_ROWS_PER_GROUP 0
#endif
// Pair movers' access hints (nontemporal loads / stores). A launch whose source rows repeat
// across pairs (several targets of one donor row) reads through the caches instead
// (MoveArgs::cached_loads): the repeats then hit L2 / Infinity Cache rather than HBM.
#ifndef SB_MOVE_NT_LOAD
#define SB_MOVE_NT_LOAD 1
#endif
#ifndef SB_MOVE_NT_STORE
#define SB_MOVE_NT_STORE 1
#endif
// Layers per thread of the pair movers (with at least 8192 pairs). Multi-layer paged launches
// slice the K plane and the V plane separately (grid.y): K in groups of SB_K_PLANE_LPG layers
// (a rotating launch evaluates cos/sin once per group), V in groups of SB_V_PLANE_LPG. On the
// 7B workload (28 layers, 13926 pairs, graph replays on one box): plain scatter K 8 / V 2
// 279 us against one interleaved group of 1 layer 284-288 us (2: 280-281 us on another box,
// 1: 274-276); rotating launches V 2 layers (four-donor composite 290 us) against 1 (305 us).
// Single-plane-pair launches (the flat scatter) use SB_SCATTER_LPG for both planes.
#ifndef SB_SCATTER_LPG
#define SB_SCATTER_LPG 1
#endif
#ifndef SB_K_PLANE_LPG
#define SB_K_PLANE_LPG 8
#endif
#ifndef SB_V_PLANE_LPG
#define SB_V_PLANE_LPG 2
#endif
constexpr int kThreads = SB_MOVE_THREADS;
constexpr int kBatch = SB_MOVE_BATCH;      // pair movers: rows loaded before the first store
constexpr int kRopeBatch = SB_ROPE_BATCH;  // row-centric RoPE: the same

struct RowSide {
  char* base;              // layer-0 base address (used when layers == nullptr)
  const uint64_t* layers;  // device table of per-layer base addresses, or nullptr
  int64_t s_layer;         // byte strides
  int64_t s_kv;
  int64_t s_head;
  int64_t s_row;           // FLAT_POS: sequence stride; PAGED_POS: block stride; INDEX: pair stride
  int64_t s_pos;           // PAGED_POS: position-in-block stride
  int64_t bound;           // FLAT_POS: sequence length
};

// Composite (multi-donor) sources: each pair names a donor; donor k's layer l starts at
// layers[k * num_layers + l] and its rows are [2, H, S_k, D] under its own strides. The
// strides of the launch's donors travel in the kernel arguments (at most kMaxDonors per
// launch; the host launches once per group of donors).
constexpr int kMaxDonors = 16;
struct DonorSet {
  const uint64_t* layers;  // device [num_donors, num_layers] table of base addresses
  const int32_t* index;    // per-pair donor index
  int first;               // donors [first, first + count) are moved by this launch
  int count;
  int64_t s_kv[kMaxDonors];    // byte strides of each donor of the launch
  int64_t s_head[kMaxDonors];
  int64_t s_seq[kMaxDonors];
  int64_t bound[kMaxDonors];   // rows held by each donor tensor
  int64_t first_pos[kMaxDonors];  // sequence position of each donor tensor's row 0
  // Grouped launches (ROW_DONOR_GROUPED sources): the pairs are grouped by donor, donor k's
  // pairs (padded with skipped pairs) ending at pair seg_end[k], every boundary a multiple of
  // kGroupedPairAlign, so that each workgroup's pairs share one donor; index is unused.
  int64_t seg_end[kMaxDonors];
};
// Boundary alignment of grouped launches: a multiple of every workgroup's pair count
// (kThreads / threads-per-row, a power of two up to kThreads).
constexpr int64_t kGroupedPairAlign = 256;

struct MoveArgs {
  RowSide src, dst;
  DonorSet donors;         // donor sources (ROW_DONOR_POS, ROW_DONOR_GROUPED) only
  const int32_t* src_pos;  // per-pair source positions (FLAT_POS / PAGED_POS sources)
  const int32_t* dst_pos;  // per-pair destination positions
  const int32_t* repeat;   // ROT_CONST: rotations to apply per pair (nullptr = 1)
  const int32_t* deltas;   // ROT_PAIR: per-pair delta
  const int32_t* block_table;
  int64_t block_size;
  int64_t nb_total;
  int64_t nb_per_seq;
  const float* inv_freq;
  int64_t const_delta;     // ROT_CONST
  int64_t num_pairs;
  int num_heads;
  int num_layers;
  int layers_per_group;
  int kv_first;            // first kv plane (0 = K, 1 = V)
  int num_kv;              // 1 or 2 planes
  // Launches over both planes of many layers: grid.y slices [0, k_slices) move (and, when
  // rotating, rotate) K in groups of layers_per_group layers, the rest copy V in groups of
  // v_layers_per_group (0: one interleaved decode with layers_per_group for both planes).
  int k_slices;
  int v_layers_per_group;
  int src_index_check;     // ROW_INDEX source: also require src_pos to be a valid paged slot
  int cached_loads;        // source rows may repeat across pairs: cached, not nontemporal, loads
  int vpr;                 // vectors per row
  int tpr_log2;            // log2(threads per row)
};

// Resolves a logical position to the byte offset of its slot (without layer/kv/head terms).
__device__ __forceinline__ bool paged_slot(const MoveArgs& a, int64_t pos, int64_t s_blk,
                                           int64_t s_pos, int64_t* off) {
  if (pos < 0) return false;
  const int64_t lb = pos / a.block_size;
  if (lb >= a.nb_per_seq) return false;
  const int64_t pb = a.block_table[lb];
  if (pb < 0 || pb >= a.nb_total) return false;
  *off = pb * s_blk + (pos - lb * a.block_size) * s_pos;
  return true;
}

template <int MODE>
__device__ __forceinline__ bool resolve_row(const MoveArgs& a, const RowSide& s,
                                            const int32_t* pos, int64_t i, int64_t* off) {
  if (MODE == ROW_INDEX) {
    *off = i * s.s_row;
    return true;
  } else if (MODE == ROW_FLAT_POS) {
    const int64_t p = pos[i];
    if (p < 0 || p >= s.bound) return false;
    *off = p * s.s_row;
    return true;
  } else {
    return paged_slot(a, pos[i], s.s_row, s.s_pos, off);
  }
}

// Base address of layer l of a row side. SCALAR: the table entry is read through the constant
// address space with a wave-uniform index, i.e. by a scalar load (the table is written by the
// host before the launch and only read here). Otherwise it is a vector load from the same
// address in every lane, which the compiler emits for a table it cannot prove unaliased by the
// kernel's stores.
//
// Measured on the 7B workload (28 layers, 13926 pairs), each launch timed after a RoPE pass as
// in a KV-reuse step: scalar reads help only the donor-grouped composite source, whose table
// pointer was per-lane before (four-donor composite 305 -> 299 us); for the plain and the
// one-donor scatters they cost 1-3% (289 -> 293 us, 285 -> 293 us): with the table load out of
// each row's dependence chain the waves keep more row loads in flight, which helps when the
// rows come from the Infinity Cache (back-to-back launches: 274 -> 266 us) and hurts when they
// come from HBM.
typedef __attribute__((address_space(4))) const uint64_t sb_const_u64;
template <bool SCALAR>
__device__ __forceinline__ char* layer_base(const RowSide& s, int l) {
  if (!s.layers) return s.base + l * s.s_layer;
  if (SCALAR) {
    const sb_const_u64* t = (const sb_const_u64*)(s.layers);
    return reinterpret_cast<char*>(t[__builtin_amdgcn_readfirstlane(l)]);
  }
  return reinterpret_cast<char*>(s.layers[l]);
}

// Unpacks VB bytes held as W 32-bit words into E fp32 values (and back).
template <int DT, int W>
__device__ __forceinline__ void unpack_words(const uint32_t* w, float* f) {
  if (DT == SB_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < W; ++k) f[k] = __uint_as_float(w[k]);
  } else {
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint16_t lo = static_cast<uint16_t>(w[k] & 0xffffu);
      const uint16_t hi = static_cast<uint16_t>(w[k] >> 16);
      f[2 * k] = DT == SB_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      f[2 * k + 1] = DT == SB_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}

template <int DT, int W>
__device__ __forceinline__ void pack_words(const float* f, uint32_t* w) {
  if (DT == SB_DTYPE_BF16) {
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = pack2_bf16(f[2 * k], f[2 * k + 1]);
    return;
  }
  if (DT == SB_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = __float_as_uint(f[k]);
  } else {
#pragma unroll
    for (int k = 0; k < W; ++k)
      w[k] = static_cast<uint32_t>(f32_to_f16(f[2 * k])) |
             (static_cast<uint32_t>(f32_to_f16(f[2 * k + 1])) << 16);
  }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 16/8/4-byte vector load and store through the global address space (every buffer here is
// device memory; generic pointers would compile to flat instructions, which also count
// against the LDS counter and serialise waits); NT selects the nontemporal forms.
#define SB_GLOBAL __attribute__((address_space(1)))

template <int VB, bool NT>
__device__ __forceinline__ void load_vec(const char* p, uint32_t* w) {
  if (VB == 16) {
    const SB_GLOBAL u32x4_t* q = (const SB_GLOBAL u32x4_t*)p;
    const u32x4_t v = NT ? __builtin_nontemporal_load(q) : *q;
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if (VB == 8) {
    const u32x2_t v = *(const SB_GLOBAL u32x2_t*)p;
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = *(const SB_GLOBAL uint32_t*)p;
  }
}

template <int VB, bool NT>
__device__ __forceinline__ void store_vec(char* p, const uint32_t* w) {
  if (VB == 16) {
    const u32x4_t v = {w[0], w[1], w[2], w[3]};
    SB_GLOBAL u32x4_t* q = (SB_GLOBAL u32x4_t*)p;
    if (NT) __builtin_nontemporal_store(v, q);
    else *q = v;
  } else if (VB == 8) {
    const u32x2_t v = {w[0], w[1]};
    *(SB_GLOBAL u32x2_t*)p = v;
  } else {
    *(SB_GLOBAL uint32_t*)p = w[0];
  }
}

// In-register rotation of E/2 interleaved pairs: e' = e*c - o*s, o' = e*s + o*c.
template <int NP>
__device__ __forceinline__ void rotate_pairs(float* f, const float* c, const float* s) {
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const float e = f[2 * k], o = f[2 * k + 1];
    const float ec = e * c[k], os = o * s[k], es = e * s[k], oc = o * c[k];
    f[2 * k] = ec - os;
    f[2 * k + 1] = es + oc;
  }
}

// NoPE two-step: strip R(-src) then apply R(tgt) (rope_correction.py:564-578, :806-821).
template <int NP>
__device__ __forceinline__ void nope_pairs(float* f, const float* cs, const float* ss,
                                           const float* ct, const float* st) {
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const float e = f[2 * k], o = f[2 * k + 1];
    const float re = e * cs[k] + o * ss[k];
    const float ro = -(e * ss[k]) + o * cs[k];
    f[2 * k] = re * ct[k] - ro * st[k];
    f[2 * k + 1] = re * st[k] + ro * ct[k];
  }
}

// In-place RoPE by one delta at positions passed by value in the launch itself (the kernel
// argument block), so a short host list reaches the kernel without a host-to-device copy.
// Other launches pass the empty InlineArg<false>.
constexpr int kInlinePositions = SB_INLINE_POSITIONS_MAX;
// Constant RoPE deltas are int64 on the ABI; the angle delta * inv_freq (inv_freq[0] = 1)
// must stay within the range sincos_cw reduces exactly.
constexpr int64_t kMaxRopeDelta = int64_t{1} << 31;
template <bool INLINE> struct InlineArg {};
template <> struct InlineArg<true> {
  int32_t pos[kInlinePositions];
  int32_t aux[kInlinePositions];  // ROT_CONST: repeat counts (when has_aux); ROT_PAIR: deltas
  int has_aux;
};
static_assert(sizeof(MoveArgs) + sizeof(InlineArg<true>) <= 4096, "kernel arguments over 4 KB");

// Waves per SIMD that the delta-rotating movers are compiled for. Occupancy decides their
// speed: with a general-purpose double sincos they took 74-80 VGPRs (6 waves) and the fused
// RoPE scatter of Qwen2.5-7B ran at 331 us; capped at 64 VGPRs (8 waves, spilling) at 288 us.
// With sincos_cw the cap costs no spills (45-51 VGPRs; left alone the scheduler takes 58-64)
// and the scatter takes 272 us. The other rotation forms keep the compiler's choice.
#ifndef SB_MOVE_ROT_WAVES
#define SB_MOVE_ROT_WAVES 8
#endif
template <int DT, int VB, int ROT, int SRCM, int DSTM, bool INLINE>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(ROT == ROT_DELTA || ROT == ROT_PAIR ? SB_MOVE_ROT_WAVES : 1)))
void move_rows_kernel(MoveArgs a, InlineArg<INLINE> ix) {
  constexpr int W = VB / 4;
  constexpr int E = (DT == SB_DTYPE_F32) ? W : 2 * W;
  constexpr int NP = E / 2;
  constexpr int NPA = NP > 0 ? NP : 1;  // plain copies of 4-byte fp32 words have no pairs
  const int tpr = 1 << a.tpr_log2;
  const int lane = threadIdx.x & (tpr - 1);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (kThreads >> a.tpr_log2) +
                    (threadIdx.x >> a.tpr_log2);
  if (i >= a.num_pairs) return;
  // Positions (and repeat counts) from device arrays, or from the launch's own argument block.
  // Read through local pointers: the argument `a` is only ever read member by member, which
  // keeps its arrays (the donor table) in the argument segment rather than in scratch.
  const int32_t* src_pos = a.src_pos;
  const int32_t* dst_pos = a.dst_pos;
  const int32_t* repeat = a.repeat;
  const int32_t* deltas = a.deltas;
  if constexpr (INLINE) {
    src_pos = ix.pos;
    dst_pos = ix.pos;
    repeat = (ROT == ROT_CONST && ix.has_aux) ? ix.aux : nullptr;
    deltas = ix.aux;
  }

  int kv, l0, lpg;
  if (a.k_slices > 0) {
    const int y = static_cast<int>(blockIdx.y);
    const bool k_slice = y < a.k_slices;
    kv = k_slice ? 0 : 1;
    lpg = k_slice ? a.layers_per_group : a.v_layers_per_group;
    l0 = (k_slice ? y : y - a.k_slices) * lpg;
  } else {
    kv = a.kv_first + static_cast<int>(blockIdx.y % a.num_kv);
    lpg = a.layers_per_group;
    l0 = static_cast<int>(blockIdx.y / a.num_kv) * lpg;
  }
  const int l1 = min(l0 + lpg, a.num_layers);

  RowSide src = a.src;
  int64_t src_off, dst_off;
  if (SRCM == ROW_DONOR_POS || SRCM == ROW_DONOR_GROUPED) {
    int dn;
    if (SRCM == ROW_DONOR_GROUPED) {
      // The workgroup's donor, from its first pair: uniform, so the donor's strides and layer
      // table come through scalar loads.
      const int64_t first_pair = static_cast<int64_t>(blockIdx.x) * (kThreads >> a.tpr_log2);
      int k = 0;
      while (k + 1 < a.donors.count && first_pair >= a.donors.seg_end[k]) ++k;
      dn = __builtin_amdgcn_readfirstlane(k);
    } else {
      dn = a.donors.index[i] - a.donors.first;
      if (dn < 0 || dn >= a.donors.count) return;  // another launch's donor, or invalid
    }
    src.layers = a.donors.layers + static_cast<int64_t>(a.donors.first + dn) * a.num_layers;
    src.s_kv = a.donors.s_kv[dn];
    src.s_head = a.donors.s_head[dn];
    // Rows are addressed relative to the donor tensor's first position; the rotation below
    // still uses the pair's sequence positions.
    const int64_t p = static_cast<int64_t>(src_pos[i]) - a.donors.first_pos[dn];
    if (p < 0 || p >= a.donors.bound[dn]) return;
    src_off = p * a.donors.s_seq[dn];
  } else if (!resolve_row<SRCM>(a, src, src_pos, i, &src_off)) {
    return;
  }
  if (!resolve_row<DSTM>(a, a.dst, dst_pos, i, &dst_off)) return;
  if (SRCM == ROW_INDEX && a.src_index_check) {
    int64_t unused;
    if (!paged_slot(a, src_pos[i], 0, 0, &unused)) return;
  }
  const bool rotate = (ROT != ROT_NONE) && kv == 0;
  int reps = 1;
  if (ROT == ROT_CONST && repeat) reps = repeat[i];

  float ang_a = 0.f, ang_b = 0.f;  // angle multipliers (fp32, as torch computes them)
  // position differences in 64 bits (int32 - int32 may not fit 32): |t - d| < 2^32
  if (ROT == ROT_DELTA)
    ang_a = static_cast<float>(static_cast<int64_t>(dst_pos[i]) - src_pos[i]);
  if (ROT == ROT_CONST) ang_a = static_cast<float>(a.const_delta);
  if (ROT == ROT_PAIR) ang_a = static_cast<float>(deltas[i]);
  if (ROT == ROT_NOPE) {
    ang_a = static_cast<float>(src_pos[i]);
    ang_b = static_cast<float>(dst_pos[i]);
  }

  const int nrows = (l1 - l0) * a.num_heads;
  auto row_of = [&](const RowSide& side, int r) {
    const int l = l0 + r / a.num_heads;
    const int h = r - (r / a.num_heads) * a.num_heads;
    // (a grouped composite source, src.layers, is uniform per workgroup)
    const char* base = (SRCM == ROW_DONOR_GROUPED && &side == &src) ? layer_base<true>(side, l)
                                                                      : layer_base<false>(side, l);
    return const_cast<char*>(base) + kv * side.s_kv + h * side.s_head;
  };
  for (int j = lane; j < a.vpr; j += tpr) {
    float c0[NPA], s0[NPA], c1[NPA], s1[NPA];
    if (ROT != ROT_NONE && rotate) {
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        const float f = a.inv_freq[j * NP + k];
        sincos_rn(ang_a * f, &s0[k], &c0[k]);
        if (ROT == ROT_NOPE) sincos_rn(ang_b * f, &s1[k], &c1[k]);
      }
    }
    const int64_t vofs = static_cast<int64_t>(j) * VB;
    for (int r0 = 0; r0 < nrows; r0 += kBatch) {
      uint32_t w[kBatch][W];
      if (a.cached_loads) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
          if (r0 + b < nrows) load_vec<VB, false>(row_of(src, r0 + b) + src_off + vofs, w[b]);
      } else {
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
          if (r0 + b < nrows)
            load_vec<VB, SB_MOVE_NT_LOAD>(row_of(src, r0 + b) + src_off + vofs, w[b]);
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (r0 + b >= nrows) continue;
        if (ROT != ROT_NONE && rotate) {
          float f[E];
          unpack_words<DT, W>(w[b], f);
          if (ROT == ROT_NOPE) {
            nope_pairs<NP>(f, c0, s0, c1, s1);
          } else {
            for (int rep = 0; rep < reps; ++rep) {
              if (rep > 0) {
#pragma unroll
                for (int k = 0; k < E; ++k) f[k] = Codec<DT>::round_trip(f[k]);
              }
              rotate_pairs<NP>(f, c0, s0);
            }
          }
          pack_words<DT, W>(f, w[b]);
        }
        store_vec<VB, SB_MOVE_NT_STORE>(row_of(a.dst, r0 + b) + dst_off + vofs, w[b]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Row-centric flat RoPE (rope_correct_k): one thread per (position s, vector j), walking all
// (layer, head) rows of that position. A prepass records, for every position, how many
// pairs name it as donor position and the first such pair (ws[0:S] counts,
// ws[S:2S] = P - first_index, via atomicMax so the smallest index wins).
// ---------------------------------------------------------------------------------------
__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void rope_index_kernel(const int32_t* dpos, int64_t num_pairs, int64_t seq_len,
                                  int32_t* ws) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= num_pairs) return;
  const int64_t d = dpos[i];
  if (d < 0 || d >= seq_len) return;
  atomicAdd(&ws[d], 1);
  atomicMax(&ws[seq_len + d], static_cast<int32_t>(num_pairs - i));
}

// Both steps in one single-workgroup launch (zero the table, barrier, count), for tables and
// pair lists small enough that one workgroup builds them in about the time of a launch.
constexpr int kIndexThreads = 1024;
constexpr int64_t kIndexFusedMax = 1 << 20;  // seq_len * 2 + num_pairs
__global__ __launch_bounds__(kIndexThreads) void rope_index_fused_kernel(const int32_t* dpos,
                                                                         int64_t num_pairs,
                                                                         int64_t seq_len,
                                                                         int32_t* ws) {
  const int tid = threadIdx.x;
  for (int64_t i = tid; i < 2 * seq_len; i += kIndexThreads) ws[i] = 0;
  __syncthreads();
  for (int64_t i = tid; i < num_pairs; i += kIndexThreads) {
    const int64_t d = dpos[i];
    if (d < 0 || d >= seq_len) continue;
    atomicAdd(&ws[d], 1);
    atomicMax(&ws[seq_len + d], static_cast<int32_t>(num_pairs - i));
  }
}

struct RopeRowsArgs {
  char* out;
  const char* k;
  int64_t o_s_layer, o_s_head, o_s_seq;  // byte strides
  int64_t k_s_layer, k_s_head, k_s_seq;
  const int32_t* dpos;
  const int32_t* tpos;
  const int32_t* ws;
  const float* inv_freq;
  int64_t num_pairs;
  int64_t seq_len;
  int num_layers;
  int num_heads;
  int rows_per_group;  // (layer, head) rows handled per grid.y slice
  int in_place;
  int vpr;
  int tpr_log2;
};

// The pair-centric form (donor positions distinct) has no multi-pair path. Its knobs: waves
// per SIMD (1: the compiler's choice, 67 VGPRs and 7 waves with sincos_cw) and rows per batch.
// On the 7B workload (28 x 4 x 8192 rows, 4 rows per thread) the defaults take 76.8 us, 8
// waves 77.3 us. (With the general-purpose double sincos it held 90 VGPRs, and 8 waves
// spilled 46 registers: 107 us at 14 rows per thread.)
#ifndef SB_ROPE_DISTINCT_WAVES
#define SB_ROPE_DISTINCT_WAVES 1
#endif
#ifndef SB_ROPE_DISTINCT_BATCH
#define SB_ROPE_DISTINCT_BATCH SB_ROPE_BATCH
#endif
template <int DT, int VB, bool INDEXED>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(INDEXED ? 1 : SB_ROPE_DISTINCT_WAVES)))
void rope_rows_kernel(RopeRowsArgs a) {
  constexpr int W = VB / 4;
  constexpr int E = (DT == SB_DTYPE_F32) ? W : 2 * W;
  constexpr int NP = E / 2;
  constexpr int kRows = INDEXED ? kRopeBatch : SB_ROPE_DISTINCT_BATCH;
  const int tpr = 1 << a.tpr_log2;
  const int lane = threadIdx.x & (tpr - 1);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (kThreads >> a.tpr_log2) +
                    (threadIdx.x >> a.tpr_log2);
  int64_t s, first;
  int cnt;
  if (INDEXED) {
    // Row-centric: thread t owns position t; the index names its pairs.
    s = t;
    if (s >= a.seq_len) return;
    cnt = a.ws[s];
    if (cnt == 0 && a.in_place) return;
    first = a.num_pairs - a.ws[a.seq_len + s];
  } else {
    // Pair-centric (in place, donor positions distinct by the caller's guarantee): thread t
    // owns pair t and rotates the row at its donor position.
    if (t >= a.num_pairs) return;
    s = a.dpos[t];
    if (s < 0 || s >= a.seq_len) return;
    cnt = 1;
    first = t;
  }

  const int total_rows = a.num_layers * a.num_heads;
  const int r_begin = static_cast<int>(blockIdx.y) * a.rows_per_group;
  const int r_end = min(r_begin + a.rows_per_group, total_rows);
  auto k_row = [&](int r) {
    const int l = r / a.num_heads;
    const int h = r - l * a.num_heads;
    return a.k + l * a.k_s_layer + h * a.k_s_head + s * a.k_s_seq;
  };
  auto o_row = [&](int r) {
    const int l = r / a.num_heads;
    const int h = r - l * a.num_heads;
    return a.out + l * a.o_s_layer + h * a.o_s_head + s * a.o_s_seq;
  };

  if (INDEXED && cnt > 1) {
    // Several pairs rotate this row (rare): apply them in pair order, rounding to the tensor
    // dtype after each one, as the reference's sequential loop does. One row at a time.
    for (int j = lane; j < a.vpr; j += tpr) {
      const int64_t vofs = static_cast<int64_t>(j) * VB;
      for (int r = r_begin; r < r_end; ++r) {
        uint32_t w[W];
        load_vec<VB, false>(k_row(r) + vofs, w);
        float f[E];
        unpack_words<DT, W>(w, f);
        int seen = 0;
        for (int64_t p = first; p < a.num_pairs && seen < cnt; ++p) {
          if (a.dpos[p] != s) continue;
          if (seen > 0) {
#pragma unroll
            for (int k = 0; k < E; ++k) f[k] = Codec<DT>::round_trip(f[k]);
          }
          const float delta = static_cast<float>(static_cast<int64_t>(a.tpos[p]) - a.dpos[p]);
          float cc[NP], ss[NP];
          for (int k = 0; k < NP; ++k)
            sincos_rn(delta * a.inv_freq[j * NP + k], &ss[k], &cc[k]);
          rotate_pairs<NP>(f, cc, ss);
          ++seen;
        }
        pack_words<DT, W>(f, w);
        store_vec<VB, true>(o_row(r) + vofs, w);
      }
    }
    return;
  }

  // At most one pair: rotate by its delta (cnt == 1) or copy (cnt == 0, out of place).
  for (int j = lane; j < a.vpr; j += tpr) {
    const int64_t vofs = static_cast<int64_t>(j) * VB;
    float c[NP], sn[NP];
    if (cnt == 1) {
      const float delta =
          static_cast<float>(static_cast<int64_t>(a.tpos[first]) - a.dpos[first]);
#pragma unroll
      for (int k = 0; k < NP; ++k) sincos_rn(delta * a.inv_freq[j * NP + k], &sn[k], &c[k]);
    }
    for (int r0 = r_begin; r0 < r_end; r0 += kRows) {
      uint32_t w[kRows][W];
#pragma unroll
      for (int b = 0; b < kRows; ++b)
        if (r0 + b < r_end) load_vec<VB, true>(k_row(r0 + b) + vofs, w[b]);
#pragma unroll
      for (int b = 0; b < kRows; ++b) {
        if (r0 + b >= r_end) continue;
        if (cnt == 1) {
          float f[E];
          unpack_words<DT, W>(w[b], f);
          rotate_pairs<NP>(f, c, sn);
          pack_words<DT, W>(f, w[b]);
        }
        store_vec<VB, true>(o_row(r0 + b) + vofs, w[b]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
namespace {

struct Geometry {
  int vb;        // vector bytes
  int vpr;       // vectors per row
  int tpr_log2;  // log2 threads per row
};

bool make_geometry(int64_t head_dim, int64_t esize, std::initializer_list<int64_t> byte_terms,
                   bool rotate, Geometry* g) {
  const int64_t row_bytes = head_dim * esize;
  int vb = vec_bytes(byte_terms);
  int row_vb = vec_bytes({row_bytes});
  vb = vb < row_vb ? vb : row_vb;
  if (vb < 4) return false;
  if (rotate && vb < 2 * esize) return false;
  g->vb = vb;
  g->vpr = static_cast<int>(row_bytes / vb);
  int64_t tpr = next_pow2(g->vpr);
  if (tpr > kThreads) tpr = kThreads;
  int lg = 0;
  while ((int64_t{1} << lg) < tpr) ++lg;
  g->tpr_log2 = lg;
  return true;
}

template <int ROT, int SRCM, int DSTM>
int launch_move(const char* fn, const MoveArgs& a0, int32_t dtype, const Geometry& g,
                int grid_y, hipStream_t stream) {
  MoveArgs a = a0;
  a.vpr = g.vpr;
  a.tpr_log2 = g.tpr_log2;
  const int64_t rows_per_block = kThreads >> g.tpr_log2;
  const int64_t gx = (a.num_pairs + rows_per_block - 1) / rows_per_block;
  if (gx > 0x7fffffff || grid_y > 65535) return fail(fn, "grid too large");
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(grid_y));
#define SB_MOVE_CASE(DT, VB)                                                              \
  if (dtype == DT && g.vb == VB) {                                                        \
    SB_LAUNCH("move_rows", (move_rows_kernel<DT, VB, ROT, SRCM, DSTM, false>), grid,     \
              dim3(kThreads), stream, a, InlineArg<false>{});                             \
    return check_launch(fn);                                                              \
  }
  if (ROT == ROT_NONE) {
    // Plain copies do not depend on the element type: move raw 32-bit words.
    dtype = SB_DTYPE_F32;
    SB_MOVE_CASE(SB_DTYPE_F32, 16)
    SB_MOVE_CASE(SB_DTYPE_F32, 8)
    SB_MOVE_CASE(SB_DTYPE_F32, 4)
  } else {
    SB_MOVE_CASE(SB_DTYPE_F32, 16)
    SB_MOVE_CASE(SB_DTYPE_F32, 8)
    SB_MOVE_CASE(SB_DTYPE_BF16, 16)
    SB_MOVE_CASE(SB_DTYPE_BF16, 8)
    SB_MOVE_CASE(SB_DTYPE_BF16, 4)
    SB_MOVE_CASE(SB_DTYPE_F16, 16)
    SB_MOVE_CASE(SB_DTYPE_F16, 8)
    SB_MOVE_CASE(SB_DTYPE_F16, 4)
  }
#undef SB_MOVE_CASE
  return fail(fn, "unsupported dtype / vector width combination");
}

template <int ROT>
int launch_rope_delta_inline(const char* fn, const MoveArgs& a0, const InlineArg<true>& ix,
                             int32_t dtype, const Geometry& g, int grid_y, hipStream_t stream) {
  MoveArgs a = a0;
  a.vpr = g.vpr;
  a.tpr_log2 = g.tpr_log2;
  const int64_t rows_per_block = kThreads >> g.tpr_log2;
  dim3 grid(static_cast<unsigned>((a.num_pairs + rows_per_block - 1) / rows_per_block),
            static_cast<unsigned>(grid_y));
#define SB_INLINE_CASE(DT, VB)                                                            \
  if (dtype == DT && g.vb == VB) {                                                        \
    SB_LAUNCH("move_rows",                                                                \
              (move_rows_kernel<DT, VB, ROT, ROW_PAGED_POS, ROW_PAGED_POS, true>), grid,   \
              dim3(kThreads), stream, a, ix);                                             \
    return check_launch(fn);                                                              \
  }
  SB_INLINE_CASE(SB_DTYPE_F32, 16)
  SB_INLINE_CASE(SB_DTYPE_F32, 8)
  SB_INLINE_CASE(SB_DTYPE_BF16, 16)
  SB_INLINE_CASE(SB_DTYPE_BF16, 8)
  SB_INLINE_CASE(SB_DTYPE_BF16, 4)
  SB_INLINE_CASE(SB_DTYPE_F16, 16)
  SB_INLINE_CASE(SB_DTYPE_F16, 8)
  SB_INLINE_CASE(SB_DTYPE_F16, 4)
#undef SB_INLINE_CASE
  return fail(fn, "unsupported dtype / vector width combination");
}

bool valid_dtype(int32_t dtype) { return elem_size(dtype) != 0; }

// Flat-position side: [.., S, D] indexed by position; strides in elements -> bytes.
RowSide side_flat(void* base, const uint64_t* layers, int64_t s_layer, int64_t s_kv,
                  int64_t s_head, int64_t s_seq, int64_t bound, int64_t es) {
  RowSide s{};
  s.base = static_cast<char*>(base);
  s.layers = layers;
  s.s_layer = s_layer * es;
  s.s_kv = s_kv * es;
  s.s_head = s_head * es;
  s.s_row = s_seq * es;
  s.s_pos = 0;
  s.bound = bound;
  return s;
}

// Paged side: kv_strides = (block, kv, head, pos, dim) in elements.
RowSide side_paged(void* base, const uint64_t* layers, const int64_t* st, int64_t es) {
  RowSide s{};
  s.base = static_cast<char*>(base);
  s.layers = layers;
  s.s_layer = 0;
  s.s_kv = st[1] * es;
  s.s_head = st[2] * es;
  s.s_row = st[0] * es;
  s.s_pos = st[3] * es;
  s.bound = 0;
  return s;
}

// Dense staging side [P, planes, H, D] (contiguous), indexed by pair. With planes == 1 the
// kv stride is 0, so whichever kv plane is moved lands at the start of each row.
RowSide side_index(void* base, int64_t num_heads, int64_t head_dim, int64_t es, int planes) {
  RowSide s{};
  s.base = static_cast<char*>(base);
  s.layers = nullptr;
  s.s_layer = 0;
  s.s_head = head_dim * es;
  s.s_kv = planes == 2 ? num_heads * head_dim * es : 0;
  s.s_row = planes * num_heads * head_dim * es;
  s.s_pos = 0;
  s.bound = 0;
  return s;
}

enum LayerGroupKind { kGroupCopy, kGroupK, kGroupV };
int layers_per_group_for(int64_t num_layers, int64_t num_pairs, LayerGroupKind kind);

// Grid slices of a launch over both planes of many layers: K in long layer groups (cos/sin
// once per group when rotating), V in short ones (more slices in flight).
int split_planes(MoveArgs& a, int64_t num_layers, int64_t num_pairs) {
  a.layers_per_group = layers_per_group_for(num_layers, num_pairs, kGroupK);
  a.v_layers_per_group = layers_per_group_for(num_layers, num_pairs, kGroupV);
  a.k_slices = static_cast<int>((num_layers + a.layers_per_group - 1) / a.layers_per_group);
  return a.k_slices +
         static_cast<int>((num_layers + a.v_layers_per_group - 1) / a.v_layers_per_group);
}

int layers_per_group_for(int64_t num_layers, int64_t num_pairs, LayerGroupKind kind) {
  // Enough grid.y slices to fill the chip when there are few pairs; otherwise walk several
  // layers per thread so index work (and, when rotating, the fp64 cos/sin) is amortised.
  const int64_t lpg = kind == kGroupK   ? SB_K_PLANE_LPG
                     : kind == kGroupV ? SB_V_PLANE_LPG
                                       : SB_SCATTER_LPG;
  if (num_pairs >= 8192) return static_cast<int>(num_layers < lpg ? num_layers : lpg);
  return 1;
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_scatter_donor_kv(void* target, const void* donor, const int32_t* donor_pos,
                                   const int32_t* target_pos, int64_t num_pairs,
                                   int64_t num_layers, int64_t num_heads, int64_t head_dim,
                                   int64_t target_seq_len, int64_t donor_seq_len,
                                   const int64_t* ts, const int64_t* ds, int32_t dtype,
                                   void* stream) {
  const char* fn = "sb_scatter_donor_kv";
  clear_error();
  if (num_pairs == 0 || num_layers == 0 || num_heads == 0 || head_dim == 0) return SB_OK;
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if (!target || !donor || !donor_pos || !target_pos || !ts || !ds)
    return fail(fn, "null pointer argument");
  if (ts[4] != 1 || ds[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {reinterpret_cast<int64_t>(target), reinterpret_cast<int64_t>(donor),
                      ts[0] * es, ts[1] * es, ts[2] * es, ts[3] * es, ds[0] * es, ds[1] * es,
                      ds[2] * es, ds[3] * es},
                     false, &g))
    return fail(fn, "rows are not 4-byte aligned");
  MoveArgs a{};
  a.src = side_flat(const_cast<void*>(donor), nullptr, ds[0], ds[1], ds[2], ds[3],
                    donor_seq_len, es);
  a.dst = side_flat(target, nullptr, ts[0], ts[1], ts[2], ts[3], target_seq_len, es);
  a.src_pos = donor_pos;
  a.dst_pos = target_pos;
  a.num_pairs = num_pairs;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = static_cast<int>(num_layers);
  a.layers_per_group = layers_per_group_for(num_layers, num_pairs, kGroupCopy);
  a.kv_first = 0;
  a.num_kv = 2;
  const int groups = static_cast<int>((num_layers + a.layers_per_group - 1) / a.layers_per_group);
  return launch_move<ROT_NONE, ROW_FLAT_POS, ROW_FLAT_POS>(fn, a, dtype, g, 2 * groups,
                                                           static_cast<hipStream_t>(stream));
}

static int paged_scatter_impl(const char* fn, void* kv_base, const uint64_t* kv_layers,
                              const void* donor_base, const uint64_t* donor_layers,
                              int64_t num_layers, const int32_t* block_table,
                              const int32_t* donor_pos, const int32_t* target_pos,
                              const float* inv_freq, int64_t num_pairs, int64_t num_heads,
                              int64_t block_size, int64_t head_dim, int64_t donor_seq_len,
                              int64_t num_blocks_total, int64_t num_blocks_per_seq,
                              const int64_t* ks, const int64_t* ds, int32_t dtype,
                              bool rope, int32_t flags, void* stream) {
  clear_error();
  if (num_pairs == 0 || num_layers == 0 || num_heads == 0 || head_dim == 0) return SB_OK;
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if ((!kv_base && !kv_layers) || (!donor_base && !donor_layers) || !block_table ||
      !donor_pos || !target_pos || !ks || !ds)
    return fail(fn, "null pointer argument");
  if (rope && !inv_freq) return fail(fn, "null inv_freq");
  if (rope && (head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (flags & ~SB_SCATTER_FLAGS_ALL) return fail(fn, "unknown flags");
  if (ks[4] != 1 || ds[3] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  // Per-layer tables are checked for 16-byte alignment by the caller.
  const int64_t kb = kv_layers ? 16 : reinterpret_cast<int64_t>(kv_base);
  const int64_t db = donor_layers ? 16 : reinterpret_cast<int64_t>(donor_base);
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {kb, db, ks[0] * es, ks[1] * es, ks[2] * es, ks[3] * es, ds[0] * es,
                      ds[1] * es, ds[2] * es},
                     rope, &g))
    return fail(fn, "rows are not aligned for vector access");
  MoveArgs a{};
  a.src = side_flat(const_cast<void*>(donor_base), donor_layers, 0, ds[0], ds[1], ds[2],
                    donor_seq_len, es);
  a.dst = side_paged(kv_base, kv_layers, ks, es);
  a.src_pos = donor_pos;
  a.dst_pos = target_pos;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  a.inv_freq = inv_freq;
  a.num_pairs = num_pairs;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = static_cast<int>(num_layers);
  a.kv_first = 0;
  a.num_kv = 2;
  a.cached_loads = (flags & SB_SCATTER_REPEATED_DONOR_ROWS) ? 1 : 0;
  const int slices = split_planes(a, num_layers, num_pairs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rope)
    return launch_move<ROT_DELTA, ROW_FLAT_POS, ROW_PAGED_POS>(fn, a, dtype, g, slices, st);
  return launch_move<ROT_NONE, ROW_FLAT_POS, ROW_PAGED_POS>(fn, a, dtype, g, slices, st);
}

extern "C" int sb_scatter_donor_kv_paged(void* kv_cache, const void* donor_kv,
                                         const int32_t* block_table, const int32_t* donor_pos,
                                         const int32_t* target_pos, int64_t num_pairs,
                                         int64_t num_heads, int64_t block_size,
                                         int64_t head_dim, int64_t donor_seq_len,
                                         int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                         const int64_t* kv_strides, const int64_t* d_strides,
                                         int32_t dtype, void* stream) {
  return paged_scatter_impl("sb_scatter_donor_kv_paged", kv_cache, nullptr, donor_kv, nullptr,
                            1, block_table, donor_pos, target_pos, nullptr, num_pairs,
                            num_heads, block_size, head_dim, donor_seq_len, num_blocks_total,
                            num_blocks_per_seq, kv_strides, d_strides, dtype, false, 0, stream);
}

extern "C" int sb_scatter_donor_kv_paged_layers(
    const uint64_t* kv_layer_ptrs, const uint64_t* donor_layer_ptrs, int64_t num_layers,
    const int32_t* block_table, const int32_t* donor_pos, const int32_t* target_pos,
    int64_t num_pairs, int64_t num_heads, int64_t block_size, int64_t head_dim,
    int64_t donor_seq_len, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    const int64_t* kv_strides, const int64_t* d_strides, int32_t dtype, int32_t flags,
    void* stream) {
  if (!kv_layer_ptrs || !donor_layer_ptrs) {
    clear_error();
    if (num_pairs == 0 || num_layers == 0) return SB_OK;
    return fail("sb_scatter_donor_kv_paged_layers", "null layer table");
  }
  return paged_scatter_impl("sb_scatter_donor_kv_paged_layers", nullptr, kv_layer_ptrs,
                            nullptr, donor_layer_ptrs, num_layers, block_table, donor_pos,
                            target_pos, nullptr, num_pairs, num_heads, block_size, head_dim,
                            donor_seq_len, num_blocks_total, num_blocks_per_seq, kv_strides,
                            d_strides, dtype, false, flags, stream);
}

extern "C" int sb_rope_correct_scatter_paged(void* kv_cache, const void* donor_kv,
                                             const int32_t* block_table,
                                             const int32_t* donor_pos,
                                             const int32_t* target_pos, const float* inv_freq,
                                             int64_t num_pairs, int64_t num_heads,
                                             int64_t block_size, int64_t head_dim,
                                             int64_t donor_seq_len, int64_t num_blocks_total,
                                             int64_t num_blocks_per_seq,
                                             const int64_t* kv_strides,
                                             const int64_t* d_strides, int32_t dtype,
                                             void* stream) {
  return paged_scatter_impl("sb_rope_correct_scatter_paged", kv_cache, nullptr, donor_kv,
                            nullptr, 1, block_table, donor_pos, target_pos, inv_freq,
                            num_pairs, num_heads, block_size, head_dim, donor_seq_len,
                            num_blocks_total, num_blocks_per_seq, kv_strides, d_strides, dtype,
                            true, 0, stream);
}

extern "C" int sb_rope_correct_scatter_paged_layers(
    const uint64_t* kv_layer_ptrs, const uint64_t* donor_layer_ptrs, int64_t num_layers,
    const int32_t* block_table, const int32_t* donor_pos, const int32_t* target_pos,
    const float* inv_freq, int64_t num_pairs, int64_t num_heads, int64_t block_size,
    int64_t head_dim, int64_t donor_seq_len, int64_t num_blocks_total,
    int64_t num_blocks_per_seq, const int64_t* kv_strides, const int64_t* d_strides,
    int32_t dtype, int32_t flags, void* stream) {
  if (!kv_layer_ptrs || !donor_layer_ptrs) {
    clear_error();
    if (num_pairs == 0 || num_layers == 0) return SB_OK;
    return fail("sb_rope_correct_scatter_paged_layers", "null layer table");
  }
  return paged_scatter_impl("sb_rope_correct_scatter_paged_layers", nullptr, kv_layer_ptrs,
                            nullptr, donor_layer_ptrs, num_layers, block_table, donor_pos,
                            target_pos, inv_freq, num_pairs, num_heads, block_size, head_dim,
                            donor_seq_len, num_blocks_total, num_blocks_per_seq, kv_strides,
                            d_strides, dtype, true, flags, stream);
}

// Composite (multi-donor) scatter over many layers: pair i moves donor
// donor_index[i]'s rows at donor_pos[i] to target_pos[i] of every layer's paged cache,
// rotating K by (target - donor) when inv_freq is given.
static int composite_impl(
    const char* fn, const uint64_t* kv_layer_ptrs, int64_t num_layers,
    const uint64_t* donor_layer_ptrs, int64_t num_donors, const int64_t* donor_strides,
    const int32_t* donor_index, const int64_t* segment_ends, const int32_t* donor_pos,
    const int32_t* target_pos, const float* inv_freq, int64_t num_pairs, int64_t num_heads,
    int64_t block_size, int64_t head_dim, const int32_t* block_table, int64_t num_blocks_total,
    int64_t num_blocks_per_seq, const int64_t* kv_strides, int32_t dtype, int32_t flags,
    void* stream) {
  clear_error();
  if (num_pairs == 0 || num_layers == 0 || num_heads == 0 || head_dim == 0 || num_donors == 0)
    return SB_OK;
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if (!kv_layer_ptrs || !donor_layer_ptrs || !donor_strides || (!donor_index && !segment_ends) ||
      !donor_pos || !target_pos || !block_table || !kv_strides)
    return fail(fn, "null pointer argument");
  if (segment_ends) {
    if (num_donors > kMaxDonors) return fail(fn, "a grouped launch takes at most 16 donors");
    int64_t prev = 0;
    for (int64_t k = 0; k < num_donors; ++k) {
      const int64_t e = segment_ends[k];
      const bool last = k + 1 == num_donors;
      if (e < prev || (last ? e != num_pairs : e % kGroupedPairAlign != 0))
        return fail(fn, "segment ends must rise, sit on multiples of 256 and end at num_pairs");
      prev = e;
    }
  }
  const bool rope = inv_freq != nullptr;
  if (rope && (head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (flags & ~SB_SCATTER_FLAGS_ALL) return fail(fn, "unknown flags");
  if (kv_strides[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  if (num_donors > 0x7fffffff || num_layers > 0x7fffffff)
    return fail(fn, "too many donors or layers");
  const int64_t es = elem_size(dtype);
  // The donors' strides bound the vector width like the cache's do (layer tables are
  // checked for 16-byte alignment by the caller).
  int64_t donor_vb = 16;
  for (int64_t k = 0; k < num_donors; ++k) {
    const int64_t* d = donor_strides + 5 * k;
    if (d[3] < 0) return fail(fn, "negative donor sequence length");
    for (int t = 0; t < 3; ++t)
      while (donor_vb > 1 && (d[t] * es) % donor_vb != 0) donor_vb >>= 1;
  }
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {16, donor_vb, kv_strides[0] * es, kv_strides[1] * es, kv_strides[2] * es,
                      kv_strides[3] * es},
                     rope, &g))
    return fail(fn, "rows are not aligned for vector access");
  MoveArgs a{};
  a.dst = side_paged(nullptr, kv_layer_ptrs, kv_strides, es);
  a.donors.layers = donor_layer_ptrs;
  a.donors.index = donor_index;
  if (segment_ends)
    for (int64_t k = 0; k < num_donors; ++k) a.donors.seg_end[k] = segment_ends[k];
  a.src_pos = donor_pos;
  a.dst_pos = target_pos;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  a.inv_freq = inv_freq;
  a.num_pairs = num_pairs;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = static_cast<int>(num_layers);
  a.kv_first = 0;
  a.num_kv = 2;
  a.cached_loads = (flags & SB_SCATTER_REPEATED_DONOR_ROWS) ? 1 : 0;
  const int slices = split_planes(a, num_layers, num_pairs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int64_t first = 0; first < num_donors; first += kMaxDonors) {
    const int count = static_cast<int>(std::min<int64_t>(kMaxDonors, num_donors - first));
    a.donors.first = static_cast<int>(first);
    a.donors.count = count;
    for (int k = 0; k < count; ++k) {
      const int64_t* d = donor_strides + 5 * (first + k);
      a.donors.s_kv[k] = d[0] * es;
      a.donors.s_head[k] = d[1] * es;
      a.donors.s_seq[k] = d[2] * es;
      a.donors.bound[k] = d[3];
      a.donors.first_pos[k] = d[4];
    }
    int rc;
    if (segment_ends)
      rc = rope ? launch_move<ROT_DELTA, ROW_DONOR_GROUPED, ROW_PAGED_POS>(fn, a, dtype, g,
                                                                          slices, st)
                : launch_move<ROT_NONE, ROW_DONOR_GROUPED, ROW_PAGED_POS>(fn, a, dtype, g,
                                                                         slices, st);
    else
      rc = rope ? launch_move<ROT_DELTA, ROW_DONOR_POS, ROW_PAGED_POS>(fn, a, dtype, g, slices,
                                                                      st)
                : launch_move<ROT_NONE, ROW_DONOR_POS, ROW_PAGED_POS>(fn, a, dtype, g, slices,
                                                                     st);
    if (rc) return rc;
  }
  return SB_OK;
}

extern "C" int sb_composite_scatter_paged_layers(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const uint64_t* donor_layer_ptrs,
    int64_t num_donors, const int64_t* donor_strides, const int32_t* donor_index,
    const int32_t* donor_pos, const int32_t* target_pos, const float* inv_freq,
    int64_t num_pairs, int64_t num_heads, int64_t block_size, int64_t head_dim,
    const int32_t* block_table, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    const int64_t* kv_strides, int32_t dtype, int32_t flags, void* stream) {
  if (!donor_index && num_pairs != 0) {
    clear_error();
    return fail("sb_composite_scatter_paged_layers", "null pointer argument");
  }
  return composite_impl("sb_composite_scatter_paged_layers", kv_layer_ptrs, num_layers,
                        donor_layer_ptrs, num_donors, donor_strides, donor_index, nullptr,
                        donor_pos, target_pos, inv_freq, num_pairs, num_heads, block_size,
                        head_dim, block_table, num_blocks_total, num_blocks_per_seq, kv_strides,
                        dtype, flags, stream);
}

// The composite scatter with its pairs grouped by donor (host segment ends): each workgroup's
// pairs share one donor, whose strides and layer table the workgroup reads once.
extern "C" int sb_composite_scatter_paged_layers_grouped(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const uint64_t* donor_layer_ptrs,
    int64_t num_donors, const int64_t* donor_strides, const int64_t* segment_ends,
    const int32_t* donor_pos, const int32_t* target_pos, const float* inv_freq,
    int64_t num_pairs, int64_t num_heads, int64_t block_size, int64_t head_dim,
    const int32_t* block_table, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    const int64_t* kv_strides, int32_t dtype, int32_t flags, void* stream) {
  if (!segment_ends && num_pairs != 0) {
    clear_error();
    return fail("sb_composite_scatter_paged_layers_grouped", "null segment ends");
  }
  return composite_impl("sb_composite_scatter_paged_layers_grouped", kv_layer_ptrs,
                        num_layers, donor_layer_ptrs, num_donors, donor_strides, nullptr,
                        segment_ends, donor_pos, target_pos, inv_freq, num_pairs, num_heads,
                        block_size, head_dim, block_table, num_blocks_total,
                        num_blocks_per_seq, kv_strides, dtype, flags, stream);
}

namespace sb {
namespace {
int rope_k_impl(const char* fn, void* out, const void* k, const int32_t* donor_pos,
                const int32_t* target_pos, const float* inv_freq, int32_t* workspace,
                bool distinct, int64_t num_pairs, int64_t num_layers, int64_t num_heads,
                int64_t seq_len, int64_t head_dim, const int64_t* os, const int64_t* ks,
                int32_t dtype, void* stream);
}  // namespace
}  // namespace sb

extern "C" int sb_rope_correct_k(void* out, const void* k, const int32_t* donor_pos,
                                 const int32_t* target_pos, const float* inv_freq,
                                 int32_t* workspace, int64_t num_pairs, int64_t num_layers,
                                 int64_t num_heads, int64_t seq_len, int64_t head_dim,
                                 const int64_t* os, const int64_t* ks, int32_t dtype,
                                 void* stream) {
  return rope_k_impl("sb_rope_correct_k", out, k, donor_pos, target_pos, inv_freq, workspace,
                     false, num_pairs, num_layers, num_heads, seq_len, head_dim, os, ks, dtype,
                     stream);
}

extern "C" int sb_rope_correct_k_distinct(void* k, const int32_t* donor_pos,
                                          const int32_t* target_pos, const float* inv_freq,
                                          int64_t num_pairs, int64_t num_layers,
                                          int64_t num_heads, int64_t seq_len, int64_t head_dim,
                                          const int64_t* ks, int32_t dtype, void* stream) {
  return rope_k_impl("sb_rope_correct_k_distinct", k, k, donor_pos, target_pos, inv_freq,
                     nullptr, true, num_pairs, num_layers, num_heads, seq_len, head_dim, ks, ks,
                     dtype, stream);
}

namespace sb {
namespace {
int rope_k_impl(const char* fn, void* out, const void* k, const int32_t* donor_pos,
                const int32_t* target_pos, const float* inv_freq, int32_t* workspace,
                bool distinct, int64_t num_pairs, int64_t num_layers, int64_t num_heads,
                int64_t seq_len, int64_t head_dim, const int64_t* os, const int64_t* ks,
                int32_t dtype, void* stream) {
  clear_error();
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if (!out || !k || !os || !ks) return fail(fn, "null pointer argument");
  if (num_layers == 0 || num_heads == 0 || seq_len == 0 || head_dim == 0) return SB_OK;
  if (num_pairs > 0 && (!donor_pos || !target_pos || !inv_freq))
    return fail(fn, "null pointer argument");
  if ((head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (os[3] != 1 || ks[3] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  if (num_pairs > 0x7ffffffe) return fail(fn, "too many pairs");
  const int64_t es = elem_size(dtype);
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {reinterpret_cast<int64_t>(out), reinterpret_cast<int64_t>(k), os[0] * es,
                      os[1] * es, os[2] * es, ks[0] * es, ks[1] * es, ks[2] * es},
                     true, &g))
    return fail(fn, "rows are not aligned for vector access");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool in_place = out == k;
  if (num_pairs == 0 && in_place) return SB_OK;
  if (distinct && !in_place) return fail(fn, "the distinct-donor form runs in place");
  if (!distinct && !workspace) return fail(fn, "null workspace");

  // Per-position pair index: counts in ws[0:S], (P - first pair) in ws[S:2S]. Not needed
  // when the caller guarantees distinct donor positions (one thread per pair, in place).
  int32_t* ws = distinct ? nullptr : workspace;
  const int64_t n = 2 * seq_len;
  if (distinct) {
    // no index
  } else if (n + num_pairs <= kIndexFusedMax) {
    SB_LAUNCH("rope_index", rope_index_fused_kernel, dim3(1), dim3(kIndexThreads), st,
              donor_pos, num_pairs, seq_len, ws);
  } else {
    SB_LAUNCH("fill_i32", fill_i32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
              dim3(256), st, ws, n, 0);
    if (num_pairs > 0)
      SB_LAUNCH("rope_index", rope_index_kernel,
                dim3(static_cast<unsigned>((num_pairs + 255) / 256)), dim3(256), st,
                donor_pos, num_pairs, seq_len, ws);
  }
  {
    int rc = check_launch(fn);
    if (rc) return rc;
  }
  RopeRowsArgs a{};
  a.out = static_cast<char*>(out);
  a.k = static_cast<const char*>(k);
  a.o_s_layer = os[0] * es; a.o_s_head = os[1] * es; a.o_s_seq = os[2] * es;
  a.k_s_layer = ks[0] * es; a.k_s_head = ks[1] * es; a.k_s_seq = ks[2] * es;
  a.dpos = donor_pos;
  a.tpos = target_pos;
  a.ws = ws;
  a.inv_freq = inv_freq;
  a.num_pairs = num_pairs;
  a.seq_len = seq_len;
  a.num_layers = static_cast<int>(num_layers);
  a.num_heads = static_cast<int>(num_heads);
  a.in_place = in_place ? 1 : 0;
  a.vpr = g.vpr;
  a.tpr_log2 = g.tpr_log2;
  const int total_rows = static_cast<int>(num_layers * num_heads);
  // Split the (layer, head) rows over grid.y so that short sequences still fill 256 CUs.
  const int64_t rows_per_block = kThreads >> g.tpr_log2;
  const int64_t units = distinct ? num_pairs : seq_len;  // threads groups: pairs or positions
  const int64_t gx = (units + rows_per_block - 1) / rows_per_block;
  if (gx > 0x7fffffff) return fail(fn, "grid too large");
  int splits = 1;
  while (splits < total_rows && gx * splits < SB_ROPE_TARGET_BLOCKS) splits *= 2;
  if (splits > total_rows) splits = total_rows;
  a.rows_per_group = (total_rows + splits - 1) / splits;
#if SB_ROPE_ROWS_PER_GROUP > 0
  a.rows_per_group = total_rows < SB_ROPE_ROWS_PER_GROUP ? total_rows : SB_ROPE_ROWS_PER_GROUP;
#endif
  const int gy = (total_rows + a.rows_per_group - 1) / a.rows_per_group;
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
#define SB_ROWS_CASE(DT, VB)                                                              \
  if (dtype == DT && g.vb == VB) {                                                        \
    if (ws)                                                                               \
      SB_LAUNCH("rope_rows", (rope_rows_kernel<DT, VB, true>), grid, dim3(kThreads), st, a); \
    else                                                                                  \
      SB_LAUNCH("rope_rows", (rope_rows_kernel<DT, VB, false>), grid, dim3(kThreads), st,  \
                a);                                                                       \
    return check_launch(fn);                                                              \
  }
  SB_ROWS_CASE(SB_DTYPE_F32, 16)
  SB_ROWS_CASE(SB_DTYPE_F32, 8)
  SB_ROWS_CASE(SB_DTYPE_BF16, 16)
  SB_ROWS_CASE(SB_DTYPE_BF16, 8)
  SB_ROWS_CASE(SB_DTYPE_BF16, 4)
  SB_ROWS_CASE(SB_DTYPE_F16, 16)
  SB_ROWS_CASE(SB_DTYPE_F16, 8)
  SB_ROWS_CASE(SB_DTYPE_F16, 4)
#undef SB_ROWS_CASE
  return fail(fn, "unsupported dtype / vector width combination");
}
}  // namespace
}  // namespace sb

namespace sb {
namespace {
// Checks and launch arguments shared by the two in-place delta RoPE entries; positions and
// repeat are filled in by the caller.
int rope_delta_setup(const char* fn, void* k_plane, const int32_t* block_table,
                     int64_t num_positions, int64_t delta, const float* inv_freq,
                     int64_t num_heads, int64_t block_size, int64_t head_dim,
                     int64_t num_blocks_total, int64_t num_blocks_per_seq, const int64_t* ks,
                     int32_t dtype, MoveArgs* out, Geometry* g) {
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if (!k_plane || !block_table || !inv_freq || !ks) return fail(fn, "null pointer argument");
  if ((head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (ks[3] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  if (delta <= -kMaxRopeDelta || delta >= kMaxRopeDelta)
    return fail(fn, "|delta| must be below 2^31 (the range of the kernels' sin/cos)");
  const int64_t es = elem_size(dtype);
  if (!make_geometry(head_dim, es,
                     {reinterpret_cast<int64_t>(k_plane), ks[0] * es, ks[1] * es, ks[2] * es},
                     true, g))
    return fail(fn, "rows are not aligned for vector access");
  // k_strides = (block, head, pos, dim); expressed as a paged side with a single kv plane.
  const int64_t st5[5] = {ks[0], 0, ks[1], ks[2], ks[3]};
  MoveArgs a{};
  a.src = side_paged(k_plane, nullptr, st5, es);
  a.dst = a.src;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  a.inv_freq = inv_freq;
  a.const_delta = delta;
  a.num_pairs = num_positions;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = 1;
  a.layers_per_group = 1;
  a.kv_first = 0;
  a.num_kv = 1;
  *out = a;
  return SB_OK;
}
}  // namespace
}  // namespace sb

extern "C" int sb_apply_rope_delta_inplace(void* k_plane, const int32_t* block_table,
                                           const int32_t* positions, const int32_t* repeat,
                                           int64_t num_positions, int64_t delta,
                                           const float* inv_freq, int64_t num_heads,
                                           int64_t block_size, int64_t head_dim,
                                           int64_t num_blocks_total,
                                           int64_t num_blocks_per_seq, const int64_t* ks,
                                           int32_t dtype, void* stream) {
  const char* fn = "sb_apply_rope_delta_inplace";
  clear_error();
  if (num_positions == 0 || num_heads == 0 || head_dim == 0 || delta == 0) return SB_OK;
  if (!positions) return fail(fn, "null pointer argument");
  MoveArgs a;
  Geometry g;
  const int rc = rope_delta_setup(fn, k_plane, block_table, num_positions, delta, inv_freq,
                                  num_heads, block_size, head_dim, num_blocks_total,
                                  num_blocks_per_seq, ks, dtype, &a, &g);
  if (rc) return rc;
  a.src_pos = positions;
  a.dst_pos = positions;
  a.repeat = repeat;
  return launch_move<ROT_CONST, ROW_PAGED_POS, ROW_PAGED_POS>(fn, a, dtype, g, 1,
                                                              static_cast<hipStream_t>(stream));
}

extern "C" int sb_apply_rope_delta_inplace_host(void* k_plane, const int32_t* block_table,
                                                const int32_t* positions,
                                                const int32_t* repeat, int64_t num_positions,
                                                int64_t delta, const float* inv_freq,
                                                int64_t num_heads, int64_t block_size,
                                                int64_t head_dim, int64_t num_blocks_total,
                                                int64_t num_blocks_per_seq, const int64_t* ks,
                                                int32_t dtype, void* stream) {
  const char* fn = "sb_apply_rope_delta_inplace_host";
  clear_error();
  if (num_positions == 0 || num_heads == 0 || head_dim == 0 || delta == 0) return SB_OK;
  if (!positions) return fail(fn, "null pointer argument");
  if (num_positions < 0 || num_positions > kInlinePositions)
    return fail(fn, "more positions than SB_INLINE_POSITIONS_MAX");
  MoveArgs a;
  Geometry g;
  const int rc = rope_delta_setup(fn, k_plane, block_table, num_positions, delta, inv_freq,
                                  num_heads, block_size, head_dim, num_blocks_total,
                                  num_blocks_per_seq, ks, dtype, &a, &g);
  if (rc) return rc;
  InlineArg<true> ix;
  std::memset(&ix, 0, sizeof(ix));
  std::memcpy(ix.pos, positions, static_cast<size_t>(num_positions) * sizeof(int32_t));
  if (repeat) {
    std::memcpy(ix.aux, repeat, static_cast<size_t>(num_positions) * sizeof(int32_t));
    ix.has_aux = 1;
  }
  return launch_rope_delta_inline<ROT_CONST>(fn, a, ix, dtype, g, 1,
                                             static_cast<hipStream_t>(stream));
}

namespace sb {
namespace {
// Checks and launch arguments of the two multi-layer per-position delta entries (positions
// and deltas are filled in by the caller); returns the grid.y of the launch in *groups.
int rope_deltas_layers_setup(const char* fn, const uint64_t* kv_layer_ptrs, int64_t num_layers,
                             const int32_t* block_table, int64_t num_positions,
                             const float* inv_freq, int64_t num_heads, int64_t block_size,
                             int64_t head_dim, int64_t num_blocks_total,
                             int64_t num_blocks_per_seq, const int64_t* ks, int32_t dtype,
                             MoveArgs* out, Geometry* g, int* groups) {
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if (!kv_layer_ptrs || !block_table || !inv_freq || !ks) return fail(fn, "null pointer argument");
  if (num_positions < 0 || num_layers < 0 || num_layers > 65535)
    return fail(fn, "invalid position or layer count");
  if ((head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (ks[3] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  // Per-layer tables are checked for 16-byte alignment by the caller.
  if (!make_geometry(head_dim, es, {16, ks[0] * es, ks[1] * es, ks[2] * es}, true, g))
    return fail(fn, "rows are not aligned for vector access");
  // k_strides = (block, head, pos, dim): a paged side with a single kv plane.
  const int64_t st5[5] = {ks[0], 0, ks[1], ks[2], ks[3]};
  MoveArgs a{};
  a.src = side_paged(nullptr, kv_layer_ptrs, st5, es);
  a.dst = a.src;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  a.inv_freq = inv_freq;
  a.num_pairs = num_positions;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = static_cast<int>(num_layers);
  a.layers_per_group = layers_per_group_for(num_layers, num_positions, kGroupK);
  a.kv_first = 0;
  a.num_kv = 1;
  *groups = static_cast<int>((num_layers + a.layers_per_group - 1) / a.layers_per_group);
  *out = a;
  return SB_OK;
}
}  // namespace
}  // namespace sb

// In-place RoPE of the K plane of many layers' paged caches, one delta per position, in one
// launch: grid.x over the positions, grid.y over groups of layers (each thread evaluates the
// cos/sin of its position once per group). Positions must be distinct within a call (their
// rows are rotated concurrently); a caller that rotates a position several times splits the
// list into calls with one occurrence each.
extern "C" int sb_apply_rope_deltas_inplace_layers(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const int32_t* block_table,
    const int32_t* positions, const int32_t* deltas, int64_t num_positions,
    const float* inv_freq, int64_t num_heads, int64_t block_size, int64_t head_dim,
    int64_t num_blocks_total, int64_t num_blocks_per_seq, const int64_t* ks, int32_t dtype,
    void* stream) {
  const char* fn = "sb_apply_rope_deltas_inplace_layers";
  clear_error();
  if (num_positions == 0 || num_layers == 0 || num_heads == 0 || head_dim == 0) return SB_OK;
  if (!positions || !deltas) return fail(fn, "null pointer argument");
  MoveArgs a;
  Geometry g;
  int groups = 0;
  const int rc = rope_deltas_layers_setup(fn, kv_layer_ptrs, num_layers, block_table,
                                          num_positions, inv_freq, num_heads, block_size,
                                          head_dim, num_blocks_total, num_blocks_per_seq, ks,
                                          dtype, &a, &g, &groups);
  if (rc) return rc;
  a.src_pos = positions;
  a.dst_pos = positions;
  a.deltas = deltas;
  return launch_move<ROT_PAIR, ROW_PAGED_POS, ROW_PAGED_POS>(fn, a, dtype, g, groups,
                                                             static_cast<hipStream_t>(stream));
}

// The same with positions and deltas in HOST memory, at most SB_INLINE_POSITIONS_MAX: they
// travel in the launch's argument block, so no device buffer or copy is involved (and a
// captured launch holds them).
extern "C" int sb_apply_rope_deltas_inplace_layers_host(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const int32_t* block_table,
    const int32_t* positions, const int32_t* deltas, int64_t num_positions,
    const float* inv_freq, int64_t num_heads, int64_t block_size, int64_t head_dim,
    int64_t num_blocks_total, int64_t num_blocks_per_seq, const int64_t* ks, int32_t dtype,
    void* stream) {
  const char* fn = "sb_apply_rope_deltas_inplace_layers_host";
  clear_error();
  if (num_positions == 0 || num_layers == 0 || num_heads == 0 || head_dim == 0) return SB_OK;
  if (!positions || !deltas) return fail(fn, "null pointer argument");
  if (num_positions < 0 || num_positions > kInlinePositions)
    return fail(fn, "more positions than SB_INLINE_POSITIONS_MAX");
  MoveArgs a;
  Geometry g;
  int groups = 0;
  const int rc = rope_deltas_layers_setup(fn, kv_layer_ptrs, num_layers, block_table,
                                          num_positions, inv_freq, num_heads, block_size,
                                          head_dim, num_blocks_total, num_blocks_per_seq, ks,
                                          dtype, &a, &g, &groups);
  if (rc) return rc;
  InlineArg<true> ix;
  std::memset(&ix, 0, sizeof(ix));
  std::memcpy(ix.pos, positions, static_cast<size_t>(num_positions) * sizeof(int32_t));
  std::memcpy(ix.aux, deltas, static_cast<size_t>(num_positions) * sizeof(int32_t));
  return launch_rope_delta_inline<ROT_PAIR>(fn, a, ix, dtype, g, groups,
                                            static_cast<hipStream_t>(stream));
}

namespace sb {
namespace {

// Dense staging side [L, P, planes, H, D] (contiguous): side_index with a layer stride.
RowSide side_index_layers(void* base, int64_t num_pairs, int64_t num_heads, int64_t head_dim,
                          int64_t es, int planes) {
  RowSide s = side_index(base, num_heads, head_dim, es, planes);
  s.s_layer = num_pairs * s.s_row;
  return s;
}

// Layers per grid.y slice of the permutation launches: one layer per slice (every slice is a
// pair-parallel grid already; longer groups only help the rotating scatter's cos/sin reuse).
constexpr int kPermuteLpg = 1;

int permute_impl(const char* fn, void* kv_cache, const uint64_t* layers, int64_t num_layers,
                 const int32_t* block_table, const int32_t* src_pos, const int32_t* tgt_pos,
                 const float* inv_freq, void* workspace, int64_t num_pairs, int64_t num_heads,
                 int64_t block_size, int64_t head_dim, int64_t num_blocks_total,
                 int64_t num_blocks_per_seq, const int64_t* ks, int32_t dtype,
                 hipStream_t st) {
  clear_error();
  if (num_pairs == 0 || num_heads == 0 || head_dim == 0 || num_layers == 0) return SB_OK;
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if ((!kv_cache && !layers) || !block_table || !src_pos || !tgt_pos || !inv_freq ||
      !workspace || !ks)
    return fail(fn, "null pointer argument");
  if (num_layers < 0 || num_layers > 65535) return fail(fn, "invalid layer count");
  if ((head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (ks[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {reinterpret_cast<int64_t>(kv_cache), reinterpret_cast<int64_t>(workspace),
                      ks[0] * es, ks[1] * es, ks[2] * es, ks[3] * es},
                     true, &g))
    return fail(fn, "rows are not aligned for vector access");
  const int grid_y = static_cast<int>(2 * ((num_layers + kPermuteLpg - 1) / kPermuteLpg));
  // Phase 1: snapshot every source row (K and V) of every layer into workspace[L, P, 2, H, D].
  MoveArgs a{};
  a.src = side_paged(kv_cache, layers, ks, es);
  a.dst = side_index_layers(workspace, num_pairs, num_heads, head_dim, es, 2);
  a.src_pos = src_pos;
  a.dst_pos = tgt_pos;
  a.block_table = block_table;
  a.block_size = block_size;
  a.nb_total = num_blocks_total;
  a.nb_per_seq = num_blocks_per_seq;
  a.inv_freq = inv_freq;
  a.num_pairs = num_pairs;
  a.num_heads = static_cast<int>(num_heads);
  a.num_layers = static_cast<int>(num_layers);
  a.layers_per_group = kPermuteLpg;
  a.kv_first = 0;
  a.num_kv = 2;
  int rc = launch_move<ROT_NONE, ROW_PAGED_POS, ROW_INDEX>(fn, a, dtype, g, grid_y, st);
  if (rc) return rc;
  // Phase 2: write every target: V copied, K rotated by (tgt - src).
  MoveArgs b = a;
  b.src = a.dst;
  b.dst = a.src;
  b.src_index_check = 1;
  return launch_move<ROT_DELTA, ROW_INDEX, ROW_PAGED_POS>(fn, b, dtype, g, grid_y, st);
}

int nope_impl(const char* fn, void* kv_cache, const uint64_t* layers, int64_t num_layers,
              const int32_t* block_table, const int32_t* src_pos, const int32_t* tgt_pos,
              int64_t num_pairs, const int32_t* v_src_pos, const int32_t* v_tgt_pos,
              int64_t num_v_pairs, const float* inv_freq, void* workspace, int64_t num_heads,
              int64_t block_size, int64_t head_dim, int64_t num_blocks_total,
              int64_t num_blocks_per_seq, const int64_t* ks, int32_t dtype, hipStream_t st) {
  clear_error();
  if ((num_pairs == 0 && num_v_pairs == 0) || num_heads == 0 || head_dim == 0 ||
      num_layers == 0)
    return SB_OK;
  if (!valid_dtype(dtype)) return fail(fn, "invalid dtype");
  if ((!kv_cache && !layers) || !block_table || !inv_freq || !workspace || !ks)
    return fail(fn, "null pointer argument");
  if (num_layers < 0 || num_layers > 65535) return fail(fn, "invalid layer count");
  if (num_pairs > 0 && (!src_pos || !tgt_pos)) return fail(fn, "null pointer argument");
  if (num_v_pairs > 0 && (!v_src_pos || !v_tgt_pos)) return fail(fn, "null pointer argument");
  if ((head_dim % 2) != 0) return fail(fn, "head_dim must be even for RoPE");
  if (block_size <= 0) return fail(fn, "block_size must be positive");
  if (ks[4] != 1) return fail(fn, "head_dim must be contiguous (stride 1)");
  const int64_t es = elem_size(dtype);
  Geometry g;
  if (!make_geometry(head_dim, es,
                     {reinterpret_cast<int64_t>(kv_cache), reinterpret_cast<int64_t>(workspace),
                      ks[0] * es, ks[1] * es, ks[2] * es, ks[3] * es},
                     true, &g))
    return fail(fn, "rows are not aligned for vector access");
  const int grid_y = static_cast<int>((num_layers + kPermuteLpg - 1) / kPermuteLpg);
  char* ws_k = static_cast<char*>(workspace);
  char* ws_v = ws_k + num_layers * num_pairs * num_heads * head_dim * es;

  MoveArgs base{};
  base.block_table = block_table;
  base.block_size = block_size;
  base.nb_total = num_blocks_total;
  base.nb_per_seq = num_blocks_per_seq;
  base.inv_freq = inv_freq;
  base.num_heads = static_cast<int>(num_heads);
  base.num_layers = static_cast<int>(num_layers);
  base.layers_per_group = kPermuteLpg;
  base.num_kv = 1;
  const RowSide cache = side_paged(kv_cache, layers, ks, es);
  const RowSide snap_k = side_index_layers(ws_k, num_pairs, num_heads, head_dim, es, 1);
  const RowSide snap_v = side_index_layers(ws_v, num_v_pairs, num_heads, head_dim, es, 1);
  int rc;
  // Snapshot K at every source (kv plane 0) and V at every resolved V source (plane 1) of
  // every layer before anything is written.
  if (num_pairs > 0) {
    MoveArgs a = base;
    a.src = cache;
    a.dst = snap_k;
    a.src_pos = src_pos;
    a.dst_pos = tgt_pos;
    a.num_pairs = num_pairs;
    a.kv_first = 0;
    rc = launch_move<ROT_NONE, ROW_PAGED_POS, ROW_INDEX>(fn, a, dtype, g, grid_y, st);
    if (rc) return rc;
  }
  if (num_v_pairs > 0) {
    MoveArgs a = base;
    a.src = cache;
    a.dst = snap_v;
    a.src_pos = v_src_pos;
    a.dst_pos = v_tgt_pos;
    a.num_pairs = num_v_pairs;
    a.kv_first = 1;
    rc = launch_move<ROT_NONE, ROW_PAGED_POS, ROW_INDEX>(fn, a, dtype, g, grid_y, st);
    if (rc) return rc;
  }
  if (num_v_pairs > 0) {
    MoveArgs a = base;
    a.src = snap_v;
    a.dst = cache;
    a.src_pos = v_src_pos;
    a.dst_pos = v_tgt_pos;
    a.num_pairs = num_v_pairs;
    a.kv_first = 1;
    a.src_index_check = 1;
    rc = launch_move<ROT_NONE, ROW_INDEX, ROW_PAGED_POS>(fn, a, dtype, g, grid_y, st);
    if (rc) return rc;
  }
  if (num_pairs > 0) {
    MoveArgs a = base;
    a.src = snap_k;
    a.dst = cache;
    a.src_pos = src_pos;
    a.dst_pos = tgt_pos;
    a.num_pairs = num_pairs;
    a.kv_first = 0;
    a.src_index_check = 1;
    rc = launch_move<ROT_NOPE, ROW_INDEX, ROW_PAGED_POS>(fn, a, dtype, g, grid_y, st);
    if (rc) return rc;
  }
  return SB_OK;
}

}  // namespace
}  // namespace sb

extern "C" int sb_permute_paged_kv_with_rope(void* kv_cache, const int32_t* block_table,
                                             const int32_t* src_pos, const int32_t* tgt_pos,
                                             const float* inv_freq, void* workspace,
                                             int64_t num_pairs, int64_t num_heads,
                                             int64_t block_size, int64_t head_dim,
                                             int64_t num_blocks_total,
                                             int64_t num_blocks_per_seq, const int64_t* ks,
                                             int32_t dtype, void* stream) {
  if (!kv_cache && num_pairs != 0) {
    clear_error();
    return fail("sb_permute_paged_kv_with_rope", "null pointer argument");
  }
  return permute_impl("sb_permute_paged_kv_with_rope", kv_cache, nullptr, 1, block_table,
                      src_pos, tgt_pos, inv_freq, workspace, num_pairs, num_heads, block_size,
                      head_dim, num_blocks_total, num_blocks_per_seq, ks, dtype,
                      static_cast<hipStream_t>(stream));
}

extern "C" int sb_permute_paged_kv_with_rope_layers(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const int32_t* block_table,
    const int32_t* src_pos, const int32_t* tgt_pos, const float* inv_freq, void* workspace,
    int64_t num_pairs, int64_t num_heads, int64_t block_size, int64_t head_dim,
    int64_t num_blocks_total, int64_t num_blocks_per_seq, const int64_t* kv_strides,
    int32_t dtype, void* stream) {
  if (!kv_layer_ptrs && num_pairs != 0 && num_layers != 0) {
    clear_error();
    return fail("sb_permute_paged_kv_with_rope_layers", "null layer table");
  }
  return permute_impl("sb_permute_paged_kv_with_rope_layers", nullptr, kv_layer_ptrs,
                      num_layers, block_table, src_pos, tgt_pos, inv_freq, workspace,
                      num_pairs, num_heads, block_size, head_dim, num_blocks_total,
                      num_blocks_per_seq, kv_strides, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sb_nope_permute_paged_kv(void* kv_cache, const int32_t* block_table,
                                        const int32_t* src_pos, const int32_t* tgt_pos,
                                        int64_t num_pairs, const int32_t* v_src_pos,
                                        const int32_t* v_tgt_pos, int64_t num_v_pairs,
                                        const float* inv_freq, void* workspace,
                                        int64_t num_heads, int64_t block_size,
                                        int64_t head_dim, int64_t num_blocks_total,
                                        int64_t num_blocks_per_seq, const int64_t* ks,
                                        int32_t dtype, void* stream) {
  if (!kv_cache && (num_pairs != 0 || num_v_pairs != 0)) {
    clear_error();
    return fail("sb_nope_permute_paged_kv", "null pointer argument");
  }
  return nope_impl("sb_nope_permute_paged_kv", kv_cache, nullptr, 1, block_table, src_pos,
                   tgt_pos, num_pairs, v_src_pos, v_tgt_pos, num_v_pairs, inv_freq, workspace,
                   num_heads, block_size, head_dim, num_blocks_total, num_blocks_per_seq, ks,
                   dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sb_nope_permute_paged_kv_layers(
    const uint64_t* kv_layer_ptrs, int64_t num_layers, const int32_t* block_table,
    const int32_t* src_pos, const int32_t* tgt_pos, int64_t num_pairs,
    const int32_t* v_src_pos, const int32_t* v_tgt_pos, int64_t num_v_pairs,
    const float* inv_freq, void* workspace, int64_t num_heads, int64_t block_size,
    int64_t head_dim, int64_t num_blocks_total, int64_t num_blocks_per_seq,
    const int64_t* kv_strides, int32_t dtype, void* stream) {
  if (!kv_layer_ptrs && (num_pairs != 0 || num_v_pairs != 0) && num_layers != 0) {
    clear_error();
    return fail("sb_nope_permute_paged_kv_layers", "null layer table");
  }
  return nope_impl("sb_nope_permute_paged_kv_layers", nullptr, kv_layer_ptrs, num_layers,
                   block_table, src_pos, tgt_pos, num_pairs, v_src_pos, v_tgt_pos, num_v_pairs,
                   inv_freq, workspace, num_heads, block_size, head_dim, num_blocks_total,
                   num_blocks_per_seq, kv_strides, dtype, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------------------
// Flat device copy: the achievable-bandwidth reference the movers are measured against. One
// 16-byte vector per thread, nontemporal load and store, 256-thread blocks. On MI355X this
// moves 6.5 TB/s (1 GiB and 235-470 MB copies); four vectors per thread 6.2-6.3 TB/s, eight
// 4.3 TB/s, the runtime's device-to-device copy 5.1-5.4 TB/s.
// ---------------------------------------------------------------------------------------
namespace sb {
__global__ __launch_bounds__(256) void copy_vec16_kernel(const char* src, char* dst,
                                                         int64_t num_vec) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= num_vec) return;
  uint32_t w[4];
  load_vec<16, true>(src + i * 16, w);
  store_vec<16, true>(dst + i * 16, w);
}
}  // namespace sb

extern "C" int sb_device_copy(void* dst, const void* src, int64_t num_bytes, void* stream) {
  const char* fn = "sb_device_copy";
  clear_error();
  if (num_bytes == 0) return SB_OK;
  if (!dst || !src) return fail(fn, "null pointer argument");
  if (num_bytes < 0 || num_bytes % 16 != 0) return fail(fn, "num_bytes must be a multiple of 16");
  if (reinterpret_cast<uintptr_t>(dst) % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return fail(fn, "buffers must be 16-byte aligned");
  const int64_t num_vec = num_bytes / 16;
  const int64_t blocks = (num_vec + 255) / 256;
  if (blocks > 0x7fffffff) return fail(fn, "copy too large");
  SB_LAUNCH("copy", copy_vec16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256),
            static_cast<hipStream_t>(stream), static_cast<const char*>(src),
            static_cast<char*>(dst), num_vec);
  return check_launch(fn);
}
