// Shared helpers for the gfx950 kernels and their C-ABI wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/nanopd.h"

namespace npd {

// Records a formatted message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a failed HIP call (or a failed launch) to NPD_E_LAUNCH.
int check_launch(const char* what);

// Compute units of the calling thread's current device (queried once per
// device, 256 if the query fails).
int device_cus();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Every workspace starts with a fixed region of int32 merge counters that all
// attention ops share: partial results are only ever written after it, and
// every call leaves the counters it used at zero. So a zero-filled workspace
// stays valid across calls of any shape (and across ops), in stream order.
constexpr int64_t kCounterBytes = 1 << 20;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

// ---------------------------------------------------------------------------
// Element conversions. Both storage types are 2 bytes; arithmetic is fp32.
// bf16 -> f32 is exact (the bf16 bits are the high half of the f32 bits);
// f32 -> bf16 rounds to nearest even, NaN stays NaN.
// ---------------------------------------------------------------------------
struct BF16 {
  static constexpr uint32_t kOne2 = 0x3f803f80u;   // packed (1.0, 1.0)
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ uint32_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  }
  // Dot product of two packed pairs, accumulated in fp32 (v_dot2_f32_bf16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  // Two floats -> packed pair, round to nearest even (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    const v2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct F16 {
  static constexpr uint32_t kOne2 = 0x3c003c00u;   // packed (1.0, 1.0)
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(h2, w).x);
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(h2, w).y);
  }
  static __device__ __forceinline__ uint32_t from_float(float f) {
    _Float16 h = static_cast<_Float16>(f);  // round to nearest even
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
  }
  // v_dot2_f32_f16: products of fp16 pairs summed into an fp32 accumulator.
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
  // Two floats -> packed pair, round to nearest even.
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    const h2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Four OCP e4m3 bytes (one dword) -> two packed pairs of TT, exact (every
// e4m3 value is a bf16 and an fp16 value): v_cvt_scalef32_pk_{bf16,f16}_fp8
// with scale 1 converts the byte pair of the low (kHi false) or high half.
template <class TT, bool kHi>
__device__ __forceinline__ uint32_t e4m3x2_to(uint32_t w) {
  if constexpr (std::is_same<TT, BF16>::value)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, kHi));
  else
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, kHi));
}

// Largest finite OCP e4m3 magnitude, and x / scale clamped to it (NaN passes
// through): the input of the e4m3 rounding of the FP8 pool's store.
constexpr float kE4m3Max = 448.f;
__device__ __forceinline__ float e4m3_clamp(float x) {
  return x != x ? x : fminf(fmaxf(x, -kE4m3Max), kE4m3Max);
}
// One value -> its e4m3 byte: x / scale (IEEE fp32 division), clamped, then
// rounded to the nearest e4m3 value, ties to even (v_cvt_pk_fp8_f32).
__device__ __forceinline__ uint32_t e4m3_byte(float x, float scale) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(x / scale), 0.f, 0, false) & 0xffu;
}

// ---------------------------------------------------------------------------
// DPP lane exchanges within rows of 16 lanes, and wave reductions built on
// them (every lane of the wave active).
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               CTRL, 0xF, 0xF, false));
}
constexpr int kDppRor8 = 0x128;        // row_ror:8      -> lane ^ 8 within a row of 16
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror -> lane ^ 7 within 8
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppMirror = 0x140;      // row_mirror      -> lane ^ 15 within a row of 16

template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
// Sum / max over the whole wave (all 64 lanes active), returned as a
// wave-uniform value: four DPP steps give every lane its row's total, then the
// four row totals are read into scalars.
__device__ __forceinline__ int wave_sum_i(int x) {
  x += dpp_i<kDppXor1>(x);
  x += dpp_i<kDppXor2>(x);
  x += dpp_i<kDppHalfMirror>(x);
  x += dpp_i<kDppMirror>(x);
  return __builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16) +
         __builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48);
}
__device__ __forceinline__ float uniform_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ float lane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ float wave_sum_f(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppMirror>(x);
  return (lane_f(x, 0) + lane_f(x, 16)) + (lane_f(x, 32) + lane_f(x, 48));
}
__device__ __forceinline__ float wave_max_f(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return fmaxf(fmaxf(lane_f(x, 0), lane_f(x, 16)), fmaxf(lane_f(x, 32), lane_f(x, 48)));
}
// Max / sum over the 4 lanes l, l^16, l^32, l^48 (the 4 rows of 16 lanes),
// with the gfx950 row-swap permutes: v_permlane16_swap with both operands x
// hands every lane {x, x of lane^16} in some order, and v_permlane32_swap
// {x, x of lane^32}.
__device__ __forceinline__ float row_max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ int wave_max_i(int x) {
  x = max(x, dpp_i<kDppXor1>(x));
  x = max(x, dpp_i<kDppXor2>(x));
  x = max(x, dpp_i<kDppHalfMirror>(x));
  x = max(x, dpp_i<kDppMirror>(x));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Agent-scope relaxed atomic accesses: written through to, and read from, the
// device-coherent level, so partials published by a workgroup on one XCD are
// seen by a workgroup on another without an L2 writeback or invalidate.
// 8-byte granularity. A writer waits for its stores to complete
// (s_waitcnt 0) before it signals, through an atomic counter, that they are there.
__device__ __forceinline__ void st_coherent2(float* p, float x, float y) {
  const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ld_coherent2(const float* p, float& x, float& y) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  x = __uint_as_float((uint32_t)v);
  y = __uint_as_float((uint32_t)(v >> 32));
}

}  // namespace npd
