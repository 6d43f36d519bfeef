// Shared device/host helpers for libsemblend_hip (gfx950, wave64).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/semblend_hip.h"
#include "sb_sincos.h"

namespace sb {

// ---------------------------------------------------------------------------------------
// Error reporting: a thread-local message behind sb_last_error_string().
// ---------------------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
int fail(const char* fn, const std::string& msg);            // SB_ERR_INVALID_ARGUMENT
int check_launch(const char* fn);                            // hipGetLastError -> code

// Timing events of one kernel launch while kernel timing is enabled
// (sb_kernel_timing_enable): two pooled HIP events, logged under `name`, which the launch
// passes to hipExtLaunchKernelGGL so that the runtime stamps them with the kernel's own start
// and end. Both are null (no timing) when timing is off.
class KernelTimer {
 public:
  explicit KernelTimer(const char* name);
  hipEvent_t start() const { return start_; }
  hipEvent_t stop() const { return stop_; }

 private:
  hipEvent_t start_ = nullptr;
  hipEvent_t stop_ = nullptr;
};

// Launches KERNEL (parenthesise template-ids) with no dynamic LDS on STREAM, logged under NAME
// when kernel timing is enabled.
#define SB_LAUNCH(NAME, KERNEL, GRID, BLOCK, STREAM, ...)                                 \
  do {                                                                                   \
    ::sb::KernelTimer sb_kt_(NAME);                                                      \
    hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, STREAM, sb_kt_.start(), sb_kt_.stop(), \
                          0, __VA_ARGS__);                                               \
  } while (0)

inline int64_t elem_size(int32_t dtype) {
  return dtype == SB_DTYPE_F32 ? 4 : (dtype == SB_DTYPE_F16 || dtype == SB_DTYPE_BF16) ? 2 : 0;
}

// Largest power-of-two byte width in {16,8,4,2,1} that divides every value given.
inline int vec_bytes(std::initializer_list<int64_t> byte_quantities) {
  int vb = 16;
  for (int64_t q : byte_quantities) {
    while (vb > 1 && (q % vb) != 0) vb >>= 1;
  }
  return vb;
}

inline int64_t next_pow2(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

// ---------------------------------------------------------------------------------------
// Scalar conversions. fp32 -> bf16 is round-to-nearest-even with NaN mapped to 0x7FC0,
// the same rule as torch's c10::BFloat16 constructor, so results match torch's
// .to(torch.bfloat16) bit for bit.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Two floats to a bf16 pair (low half = lo) with v_cvt_pk_bf16_f32: round to nearest even
// in one instruction where the integer form above takes about five per value. The hardware
// writes a quiet NaN of its own; it is replaced by 0x7FC0, so the bits equal f32_to_bf16's.
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  uint32_t w = __builtin_bit_cast(uint32_t, v);
  if (lo != lo) w = (w & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) w = (w & 0x0000ffffu) | 0x7fc00000u;
  return w;
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(x);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 x = static_cast<_Float16>(f);  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, x);
}

// Element codec by dtype tag, used by the RoPE kernels that work on 16-byte vectors.
template <int DT> struct Codec;

template <> struct Codec<SB_DTYPE_F32> {
  static constexpr int kElems16 = 4;  // elements per 16-byte vector
  __device__ __forceinline__ static void unpack(const uint4& v, float* f) {
    f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                      __float_as_uint(f[3]));
  }
  __device__ __forceinline__ static float round_trip(float f) { return f; }
};

template <> struct Codec<SB_DTYPE_BF16> {
  static constexpr int kElems16 = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
      f[2 * i + 1] = bf16_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16(f[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16(f[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ __forceinline__ static float round_trip(float f) {
    return bf16_to_f32(f32_to_bf16(f));
  }
};

template <> struct Codec<SB_DTYPE_F16> {
  static constexpr int kElems16 = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = f16_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
      f[2 * i + 1] = f16_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_f16(f[2 * i])) |
             (static_cast<uint32_t>(f32_to_f16(f[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ __forceinline__ static float round_trip(float f) {
    return f16_to_f32(f32_to_f16(f));
  }
};

// Byte-vector load/store of width VB (1, 2, 4, 8 or 16 bytes).
template <int VB> struct ByteVec;
template <> struct ByteVec<16> { using T = uint4; };
template <> struct ByteVec<8> { using T = uint2; };
template <> struct ByteVec<4> { using T = uint32_t; };
template <> struct ByteVec<2> { using T = uint16_t; };
template <> struct ByteVec<1> { using T = uint8_t; };

// fp32 sin/cos rounded correctly: evaluated in fp64 and rounded once to fp32. These are the
// values a correctly rounded libm returns, which torch's CPU kernels also produce for all but
// rare arguments. Matching them matters where e*c - o*s cancels: for an output of ~1e-6 from
// O(1) inputs, a one-ulp difference in cos or sin is several bf16 ulps of the result.
// x is a RoPE angle (an int32 position, or an int32 target minus a valid donor position, or a
// constant delta below 2^31, times an inverse frequency <= 1), so |x| < 2^32, the range of
// sincos_cw.
__device__ __forceinline__ void sincos_rn(float x, float* s, float* c) {
  double sd, cd;
  sincos_cw(static_cast<double>(x), &sd, &cd);
  *s = static_cast<float>(sd);
  *c = static_cast<float>(cd);
}

// ---------------------------------------------------------------------------------------
// Dense drop-in helpers shared by the attention and projection entries: compact a bool mask
// into ascending positions (+ count) in one workgroup, and write zeros into the output rows
// whose mask entry is 0 (rows of [heads, seq, ...] under byte strides).
// ---------------------------------------------------------------------------------------
template <int kUnused = 0>
__global__ __launch_bounds__(1024) void mask_compact_kernel(const uint8_t* mask, int64_t n,
                                                            int32_t* pos_out,
                                                            int32_t* count_out) {
  // Each thread takes 16 consecutive mask bytes per round (one 16-byte load when the mask is
  // 16-byte aligned), so a round covers 16384 positions; a wave scan of the per-thread
  // counts and the per-wave totals in LDS give every thread its output offset.
  constexpr int kPer = 16;
  constexpr int kThreadsC = 1024;
  __shared__ int wsum[kThreadsC / 64];
  __shared__ int base;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool aligned = (reinterpret_cast<uintptr_t>(mask) & 15) == 0;
  if (tid == 0) base = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < n; c0 += static_cast<int64_t>(kThreadsC) * kPer) {
    const int64_t i0 = c0 + static_cast<int64_t>(tid) * kPer;
    uint32_t bits = 0;  // bit k: mask[i0 + k] != 0
    if (aligned && i0 + kPer <= n) {
      const uint4 v = *reinterpret_cast<const uint4*>(mask + i0);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int b = 0; b < 4; ++b) bits |= (((w[q] >> (8 * b)) & 0xffu) != 0u) << (4 * q + b);
    } else {
      for (int k = 0; k < kPer; ++k)
        if (i0 + k < n && mask[i0 + k] != 0) bits |= 1u << k;
    }
    const int cnt = __popc(bits);
    int incl = cnt;  // inclusive scan over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int off = base + incl - cnt;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    while (bits) {
      const int k = __ffs(bits) - 1;
      pos_out[off++] = static_cast<int32_t>(i0 + k);
      bits &= bits - 1;
    }
    __syncthreads();
    if (tid == 0) {
      int t = 0;
      for (int w = 0; w < kThreadsC / 64; ++w) t += wsum[w];
      base += t;
    }
    __syncthreads();
  }
  if (tid == 0) *count_out = base;
}

template <int VB>
__global__ void zero_rows_kernel(char* out, const uint8_t* mask, int64_t num_heads,
                                 int64_t seq_len, int64_t s_head, int64_t s_seq, int vpr) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = num_heads * seq_len * vpr;
  if (idx >= total) return;
  const int64_t j = idx % vpr;
  const int64_t row = idx / vpr;
  const int64_t s = row % seq_len;
  const int64_t h = row / seq_len;
  if (mask[s]) return;
  char* p = out + h * s_head + s * s_seq + j * VB;
  if (VB == 16) *reinterpret_cast<uint4*>(p) = make_uint4(0, 0, 0, 0);
  else if (VB == 8) *reinterpret_cast<uint2*>(p) = make_uint2(0, 0);
  else if (VB == 4) *reinterpret_cast<uint32_t*>(p) = 0u;
  else *reinterpret_cast<uint16_t*>(p) = 0;
}

}  // namespace sb
