// OCP FP8 e4m3fn codec (1 sign, 4 exponent bits with bias 7, 3 mantissa
// bits; no infinities; S.1111.111 is the only NaN; largest finite 448).
//
// Written from the OCP 8-bit floating point specification.  Encoding is
// round-to-nearest-even; a magnitude that rounds above 448 (anything > 464,
// including infinities and NaN) becomes the NaN code with the sign kept.
// This is the behaviour of torch's `.to(torch.float8_e4m3fn)`, which the
// reference relies on (wave_rt/runtime/fp8.py:35,48;
// wave_rt/denoiser/exchange/common.py:150; onesided.py:152).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "wf_common.hpp"

namespace wf {

constexpr float kE4M3Max = 448.0f;
// bf16(1e-8): the scale floor of the reference's `.clamp(min=1e-8)` on a
// bf16 tensor (bits 0x322c).
constexpr uint16_t kScaleFloorBf16Bits = 0x322c;

// Portable encoder (host and device).  Used for the exact-semantics cast
// entry point and as the CPU-checkable statement of the rounding rule.
__host__ __device__ inline uint8_t e4m3_encode_sw(float f) {
  const uint32_t u = f32_bits(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x43E80000u) return static_cast<uint8_t>(sign | 0x7fu);  // > 464, inf, NaN
  if (a < 0x3C800000u) {
    // Below 2^-6 the e4m3 grid is uniform with step 2^-9: round |f| * 512
    // (exact scaling) to the nearest integer, ties to even.  A result of 8
    // is 2^-6, whose code 0x08 is the smallest normal.
    const float m = bits_f32(a) * 512.0f;
    return static_cast<uint8_t>(sign | static_cast<uint32_t>(rintf(m)));
  }
  // Normal range: keep exponent + 3 mantissa bits of the fp32 pattern with
  // round-to-nearest-even on the 20 dropped bits, then rebias 127 -> 7.
  const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
  return static_cast<uint8_t>(sign | (r - (120u << 3)));
}

// Exact decode (host and device).
__host__ __device__ inline float e4m3_decode_sw(uint8_t c) {
  const uint32_t sign = static_cast<uint32_t>(c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu;
  const uint32_t m = c & 0x7u;
  if ((c & 0x7fu) == 0x7fu) return bits_f32(sign | 0x7fc00000u);
  if (e == 0) return bits_f32(f32_bits(static_cast<float>(m) * (1.0f / 512.0f)) | sign);
  return bits_f32(sign | ((e + 120u) << 23) | (m << 20));
}

#if defined(__HIPCC__)
// Hardware pack of four fp32 values into four e4m3fn bytes (byte i = v_i),
// v_cvt_pk_fp8_f32 (round-to-nearest-even).  Callers pass magnitudes
// already clamped to [-448, 448]; in that range the result equals
// e4m3_encode_sw (checked over every bf16 value and every fp32 value next
// to an e4m3 rounding boundary by the encode entry point's tests).
__device__ inline uint32_t e4m3_pack4_hw(float v0, float v1, float v2, float v3) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, w, true);
  return static_cast<uint32_t>(w);
}

// Hardware decode of the four e4m3fn bytes of `w` (v_cvt_pk_f32_fp8).
__device__ inline void e4m3_unpack4_hw(uint32_t w, float& v0, float& v1, float& v2, float& v3) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  v0 = lo[0];
  v1 = lo[1];
  v2 = hi[0];
  v3 = hi[1];
}
#endif

}  // namespace wf
