// Shared helpers of the gfx950 kernels: status reporting for the C ABI,
// bf16 bit conversions and wave64 cross-lane reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <initializer_list>

#include "../../include/wf_api.h"

namespace wf {

// ----------------------------------------------------------------- status
// Thread-local message behind wf_last_error().  set_error() formats it and
// returns the status so entry points can `return set_error(...)`.
char* error_buffer();
int set_error(int status, const char* fmt, ...);

// Check the launch that was just enqueued on this thread.
int check_launch(const char* what);

#define WF_REQUIRE(cond, status, ...)                 \
  do {                                                \
    if (!(cond)) return ::wf::set_error((status), __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// True when the product of the non-negative factors is below ``limit`` (> 0), decided without forming a
// product that could overflow int64: size checks of the entry points must not rely on wrapped arithmetic.
inline bool product_below(std::initializer_list<int64_t> factors, int64_t limit) {
  for (int64_t f : factors) {
    if (f < 0) return false;
    if (f == 0) return true;
  }
  int64_t p = 1;
  for (int64_t f : factors) {
    if (p > (limit - 1) / f) return false;
    p *= f;
  }
  return p < limit;
}

// ------------------------------------------------------------------- bf16
// bf16 -> fp32 is exact: the bf16 bits are the high half of the fp32 bits.
__device__ __host__ inline float bf16_lo_to_f32(uint32_t packed) {
  uint32_t u = packed << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
__device__ __host__ inline float bf16_hi_to_f32(uint32_t packed) {
  uint32_t u = packed & 0xffff0000u;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
__device__ __host__ inline float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
__device__ __host__ inline uint32_t f32_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
__device__ __host__ inline float bits_f32(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// fp32 -> bf16 round-to-nearest-even (NaN stays a quiet NaN), matching
// torch's float -> bfloat16 conversion.
__device__ __host__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

#if defined(__HIPCC__)
// Two fp32 -> packed bf16x2 (low half = a), RNE.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16_rne(a)) |
         (static_cast<uint32_t>(f32_to_bf16_rne(b)) << 16);
}

// The same conversion in one instruction (v_cvt_pk_bf16_f32, round to
// nearest even; equal to pack_bf16x2 for every non-NaN input).
__device__ inline uint32_t pack_bf16x2_hw(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const f2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}

// GELU(approximate='tanh'): 0.5 x (1 + tanh(u)) = x / (1 + e^{-2u}) with
// u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as x * rcp(1 + 2^{-2u log2 e})
// on the hardware exponential and reciprocal (relative error ~3e-7 against
// the tanh form; x -> -inf gives -0, x -> +inf gives x).  The FFN activation
// of the Wan block (naive_rt/rolling_forcing/wan/modules/causal_model.py:342-344).
__device__ inline float gelu_tanh(float x) {
  const float inner = x * fmaf(0.044715f, x * x, 1.0f);     // x + 0.044715 x^3
  const float e = __builtin_amdgcn_exp2f(-2.3022082f * inner);  // 2 sqrt(2/pi) log2(e) = 2.3022082
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// ------------------------------------------------------- wave64 reductions
// DPP controls (gfx9): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror (lane i <-> 7-i within 8) = 0x141.
// Max over aligned groups of 8 lanes; every lane of the group gets the max.
__device__ inline float group8_max(float v) {
  int iv = __builtin_bit_cast(int, v);
  float o;
  o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(iv, iv, 0xB1, 0xF, 0xF, false));
  v = fmaxf(v, o);
  iv = __builtin_bit_cast(int, v);
  o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(iv, iv, 0x4E, 0xF, 0xF, false));
  v = fmaxf(v, o);
  iv = __builtin_bit_cast(int, v);
  o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(iv, iv, 0x141, 0xF, 0xF, false));
  return fmaxf(v, o);
}
#endif  // __HIPCC__

}  // namespace wf
