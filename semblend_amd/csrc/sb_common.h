// Shared device/host helpers for libsemblend_hip (gfx950, wave64).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/semblend_hip.h"

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

}  // namespace sb
