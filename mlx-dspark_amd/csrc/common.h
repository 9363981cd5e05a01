// Shared helpers for the gfx950 kernels behind include/dspark_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/dspark_hip.h"

namespace dsk {

// ---- error reporting: a thread-local message per failing call ---------------------------
void set_error(const char* fmt, ...);

#define DSK_REQUIRE(cond, ...)              \
  do {                                      \
    if (!(cond)) {                          \
      ::dsk::set_error(__VA_ARGS__);        \
      return DSK_EINVAL;                    \
    }                                       \
  } while (0)

#define DSK_LAUNCH_CHECK(what)                                                    \
  do {                                                                            \
    hipError_t e_ = hipGetLastError();                                            \
    if (e_ != hipSuccess) {                                                       \
      ::dsk::set_error("%s: launch failed: %s", what, hipGetErrorString(e_));     \
      return DSK_ELAUNCH;                                                         \
    }                                                                             \
  } while (0)

static inline hipStream_t as_stream(dsk_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---- vector types ---------------------------------------------------------------------
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- bf16 <-> f32 (round to nearest even, as MLX/torch do) -----------------------------
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  // v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
#endif
}

// two values in one v_cvt_pk_bf16_f32 (lo in bits 0..15): the same rounding as f32_to_bf16
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__host__ __device__ __forceinline__ uint32_t f32_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
__host__ __device__ __forceinline__ float bits_f32(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// ---- float32 probabilities as three bf16 terms ------------------------------------------
// hi = bf16(p), mid = bf16(p - hi), lo = bf16(p - hi - mid), two values per word (the first in
// bits 0..15). Both differences are exact in float32 (each operand pair lies within a factor of
// two of the rounded value's binade), so hi + mid + lo equals p to within 2^-26 of |p|: three
// bf16 MFMAs against the three terms compute P.V at float32 precision, where one bf16 P would
// lose up to 2^-9 of every probability.
struct Bf16x2Terms {
  uint32_t hi, mid, lo;
};
__device__ __forceinline__ Bf16x2Terms split3_bf16x2(float p0, float p1) {
  Bf16x2Terms t;
  t.hi = pack_bf16x2(p0, p1);
  const float r0 = p0 - bits_f32(t.hi << 16), r1 = p1 - bits_f32(t.hi & 0xffff0000u);
  t.mid = pack_bf16x2(r0, r1);
  t.lo = pack_bf16x2(r0 - bits_f32(t.mid << 16), r1 - bits_f32(t.mid & 0xffff0000u));
  return t;
}

// The first two terms alone (hi + lo, lo = bf16(p - hi)): within 2^-17 of |p|.
__device__ __forceinline__ void split2_bf16x2(float p0, float p1, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16x2(p0, p1);
  lo = pack_bf16x2(p0 - bits_f32(hi << 16), p1 - bits_f32(hi & 0xffff0000u));
}

// The first NT terms (1: bf16(p), 2: hi + lo, 3: hi + mid + lo) of two probabilities.
template <int NT>
__device__ __forceinline__ void split_terms_bf16x2(float p0, float p1, uint32_t (&t)[NT]) {
  static_assert(NT >= 1 && NT <= 3, "1 to 3 terms");
  if constexpr (NT == 3) {
    const Bf16x2Terms x = split3_bf16x2(p0, p1);
    t[0] = x.hi;
    t[1] = x.mid;
    t[2] = x.lo;
  } else if constexpr (NT == 2) {
    split2_bf16x2(p0, p1, t[0], t[1]);
  } else {
    t[0] = pack_bf16x2(p0, p1);
  }
}

// ---- wave-level reductions (wave64) ----------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Packed activation layout (the W8 GEMM's A operand): element (m, k) of an [M, K] bf16
// activation, G = K / 64, lives at P[m/16][k/64][m%16 + 16 * ((k%64)/16)][k%16].
__host__ __device__ __forceinline__ int64_t apack_index(int64_t m, int64_t k, int64_t G) {
  return ((((m >> 4) * G + (k >> 6)) * 64 + (m & 15) + 16 * ((k >> 4) & 3)) << 4) + (k & 15);
}

}  // namespace dsk
