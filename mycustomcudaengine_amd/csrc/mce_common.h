// Shared host/device helpers for the gfx950 kernels of libmce.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "mce_abi.h"

namespace mce {

// ---------------------------------------------------------------- host side

// Records a formatted message for mce_last_error() and returns `code`.
int set_error(int code, const char *fmt, ...);
void clear_error();

// Maps a failed launch (hipGetLastError after the launch) to MCE_ERR_LAUNCH.
int check_launch(const char *what);

// Compute units of the current device (cached per device; 256 if unknown).
int cu_count();

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

#define MCE_REQUIRE(cond, ...)                                                 \
  do {                                                                         \
    if (!(cond)) return ::mce::set_error(MCE_ERR_INVALID, __VA_ARGS__);        \
  } while (0)

// -------------------------------------------------------------- device side

typedef _Float16 f16;
typedef uint16_t bf16_bits;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Storage-type traits: conversion of 16-bit storage values to/from fp32.
struct F16T {
  static constexpr int code = MCE_F16;
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(f16, (uint16_t)(w & 0xffffu));
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(f16, (uint16_t)(w >> 16));
  }
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (f16)x);
  }
  // c + a.lo * b.lo + a.hi * b.hi over packed pairs (v_dot2_f32_f16)
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  // two probabilities as a packed operand (v_cvt_pkrtz_f16_f32)
  __device__ static inline uint32_t pack_p(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
  }
};

struct BF16T {
  static constexpr int code = MCE_BF16;
  __device__ static inline float lo(uint32_t w) {
    return __builtin_bit_cast(float, w << 16);
  }
  __device__ static inline float hi(uint32_t w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
  // Round to nearest even; NaN stays NaN.
  __device__ static inline uint16_t from_float(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
  // c + a.lo * b.lo + a.hi * b.hi over packed pairs (v_dot2_f32_bf16)
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  // two probabilities as a packed operand (v_cvt_pk_bf16_f32, nearest even)
  __device__ static inline uint32_t pack_p(float a, float b) {
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <class T>
__device__ inline uint32_t pack2(float a, float b) {
  return (uint32_t)T::from_float(a) | ((uint32_t)T::from_float(b) << 16);
}

// 16-lane row reductions with DPP (every lane of the row gets the result).
// Each step pairs lanes symmetrically -- quad_perm [1,0,3,2] (0xB1) and
// [2,3,0,1] (0x4E), row_half_mirror (0x141), row_mirror (0x140) -- so both
// partners add the same two values and all 16 lanes end bit-identical
// (rotations would pair lanes asymmetrically and let the rounding differ).
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
}

// max(a, b) as med3(a, b, FLT_MAX): one v_med3_f32.  fmaxf in IEEE mode first
// quiets signalling NaNs, a v_max_f32 x, x, x per operand the compiler cannot
// prove canonical (DPP, permlane and select results); a med3 with +inf is
// folded back into that max.  The maxima here are of scores and running
// maxima, finite or -inf (never +inf); a NaN operand gives an unspecified
// one of the two.
__device__ __forceinline__ float max_nq(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, 3.402823466e+38f);
}

__device__ inline float row16_max(float v) {
  v = max_nq(v, dpp_f<0xB1>(v));
  v = max_nq(v, dpp_f<0x4E>(v));
  v = max_nq(v, dpp_f<0x141>(v));
  v = max_nq(v, dpp_f<0x140>(v));
  return v;
}

__device__ inline float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}

// Exchanges across 16-lane rows on the VALU.  v_permlane16_swap swaps the
// odd rows of one operand with the even rows of the other, and
// v_permlane32_swap the two 32-lane halves; given x twice, each leaves every
// lane holding x[l] and x[l ^ 16] (x[l ^ 32]), in some order.  Max and the
// sum of two values do not depend on that order, so both lanes of a pair get
// the same result, bit for bit -- what a __shfl_xor (an LDS-routed
// ds_bpermute, ~100 cycles of latency) would give.
__device__ __forceinline__ float xor16_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return max_nq(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float xor16_add(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return max_nq(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float xor32_add(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Inclusive prefix sum over the 64 lanes, all in DPP (gfx9-family): a
// log-step scan inside each 16-lane row (row_shr 1, 2, 4, 8, lanes shifted in
// from outside the row read 0), then lane 15 of rows 0 and 2 added to rows 1
// and 3 (row_bcast:15) and lane 31 to rows 2 and 3 (row_bcast:31).  Integer
// adds, so the result is exact; no LDS round trips (a __shfl_up is a
// ds_bpermute).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}
__device__ inline int wave_incl_scan(int v) {
  v += dpp_i<0x111, 0xf>(v);  // row_shr:1
  v += dpp_i<0x112, 0xf>(v);  // row_shr:2
  v += dpp_i<0x114, 0xf>(v);  // row_shr:4
  v += dpp_i<0x118, 0xf>(v);  // row_shr:8
  v += dpp_i<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_i<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Full 64-lane sum; every lane gets the result.
__device__ inline float wave_sum(float v) { return xor32_add(xor16_add(row16_sum(v))); }

__device__ inline float wave_max(float v) { return xor32_max(xor16_max(row16_max(v))); }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Rotary rotation of one (x_i, x_{i+D/2}) pair by (c, s), fp32: the single
// definition every RoPE path uses.  Contraction into FMAs is off, so each
// product and the sum round separately and every caller rounds identically
// (the compiler would otherwise pick the fused operand per call site).
__device__ inline void rope_pair(float x0, float x1, float c, float s, float &r0, float &r1) {
#pragma clang fp contract(off)
  r0 = x0 * c - x1 * s;
  r1 = x0 * s + x1 * c;
}

// RMSNorm pieces shared by every kernel that normalises rows, so that they
// all round identically: the sum of squares of a 16-byte chunk accumulated
// in a fixed order with explicit FMAs, and y = x * (inv_rms * w).
template <class T>
__device__ inline float sumsq8(const u32x4 &v, float ss) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = T::lo(v[k]), b = T::hi(v[k]);
    ss = __builtin_fmaf(a, a, ss);
    ss = __builtin_fmaf(b, b, ss);
  }
  return ss;
}

template <class T>
__device__ inline u32x4 rms_scale8(const u32x4 &v, const u32x4 &w, float inv) {
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = T::lo(v[k]) * (inv * T::lo(w[k]));
    const float b = T::hi(v[k]) * (inv * T::hi(w[k]));
    o[k] = pack2<T>(a, b);
  }
  return o;
}

// 1 / sqrt(mean of squares + eps), the RMSNorm row scale.
__device__ inline float rms_inv(float ss, int hidden, float eps) {
  return 1.0f / sqrtf(ss / (float)hidden + eps);
}

// Workgroup barrier that orders LDS accesses only.  The fences are scoped to
// the local (LDS) address space, so the wait before s_barrier covers this
// wave's LDS operations (lgkmcnt) while global loads issued earlier stay in
// flight; __syncthreads() also waits for those (vmcnt(0)), which drains any
// register prefetch at every barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace mce
