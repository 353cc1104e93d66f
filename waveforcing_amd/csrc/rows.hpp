// Row-engine helpers of the token-row kernels (norms, modulation, per-token
// quantization, fused K/V packing).
//
// A row of n_chunks 8-element (16-byte bf16) chunks is owned by LPR lanes:
// LPR = 64 (one wave per row, four rows per 256-thread workgroup) for rows
// up to 64 * 4 chunks, or LPR = 256 (the whole workgroup, one row) above.
// Lane l of the row owns chunks l, l + LPR, ..., l + (NC - 1) LPR, so every
// load and store instruction of a wave covers 64 consecutive chunks.  NC is
// a template constant: a row's values stay in NC * 8 registers and all of a
// row's loads are in flight before its first reduction.
//
// Reductions are DPP trees inside a wave (no LDS traffic), then, for
// LPR = 256, one LDS exchange between the four waves.
#pragma once

#include <type_traits>

#include "wf_common.hpp"

namespace wf {
namespace rows {

template <int CTRL, int ROW_MASK = 0xF>
__device__ inline float dpp(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF,
                                                                false));
}

// DPP controls (gfx9): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
// Sum / max over each aligned group of 16 lanes; every lane gets its group's value.
__device__ inline float group16_sum(float v) {
  v += dpp<0xB1>(0.f, v);
  v += dpp<0x4E>(0.f, v);
  v += dpp<0x141>(0.f, v);
  v += dpp<0x140>(0.f, v);
  return v;
}
__device__ inline float group16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(0.f, v));
  v = fmaxf(v, dpp<0x4E>(0.f, v));
  v = fmaxf(v, dpp<0x141>(0.f, v));
  v = fmaxf(v, dpp<0x140>(0.f, v));
  return v;
}
// Whole-wave sum / max of non-negative values (max), broadcast to every lane.
__device__ inline float wave_sum(float v) {
  v = group16_sum(v);
  v += dpp<0x142, 0xA>(0.f, v);  // rows 1, 3 += last lane of rows 0, 2
  v += dpp<0x143, 0xC>(0.f, v);  // rows 2, 3 += lane 31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ inline float wave_max_nonneg(float v) {
  v = group16_max(v);
  v = fmaxf(v, dpp<0x142, 0xA>(0.f, v));
  v = fmaxf(v, dpp<0x143, 0xC>(0.f, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Row-wide reductions.  For LPR = 256 `red` is a 4-float LDS slot used by
// this reduction only (every reduction of a kernel takes its own slot).
template <int LPR>
__device__ inline float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (LPR == 64) {
    return v;
  } else {
    static_assert(LPR == 256, "rows of 64 or 256 lanes");
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
  }
}
template <int LPR>
__device__ inline float row_max_nonneg(float v, float* red) {
  v = wave_max_nonneg(v);
  if constexpr (LPR == 64) {
    return v;
  } else {
    static_assert(LPR == 256, "rows of 64 or 256 lanes");
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
}

__device__ inline float rbf(float f) { return bf16_lo_to_f32(pack_bf16x2_hw(f, 0.f)); }
// Round a and b to bf16 (RNE) in one v_cvt_pk_bf16_f32; equal to
// f32_to_bf16_rne for every non-NaN value.
__device__ inline void rbf2(float& a, float& b) {
  const uint32_t p = pack_bf16x2_hw(a, b);
  a = bf16_lo_to_f32(p);
  b = bf16_hi_to_f32(p);
}
// Round the 8 values of a chunk to bf16.
__device__ inline void rbf8(float* f) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) rbf2(f[i], f[i + 1]);
}

__device__ inline void unpack8(const uint4& w, float* f) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo_to_f32(u[i]);
    f[2 * i + 1] = bf16_hi_to_f32(u[i]);
  }
}
__device__ inline uint4 pack8(const float* f) {
  return make_uint4(pack_bf16x2_hw(f[0], f[1]), pack_bf16x2_hw(f[2], f[3]), pack_bf16x2_hw(f[4], f[5]),
                    pack_bf16x2_hw(f[6], f[7]));
}

__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ inline void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }

// int8 code of x with scale s: round_half_even(RN32(x / s)) clamped to
// +-127, given rd = RN64(1 / s) (i8_recip).  RN32(x / s) is computed as
// RN32(RN64(x * rd)): the fp64 product is within 2^-52 (relative) of x / s,
// while the quotient of two fp32 values is never an fp32 rounding midpoint
// (a 25-bit odd significand times a 24-bit one needs more than 24 bits) and
// otherwise lies at least 2^-49 (relative) away from every midpoint, so the
// fp32 rounding of the product is that of the IEEE quotient.  gfx950 runs
// fp64 multiplies and conversions at the rate of its unpacked fp32 ones.
__device__ inline double i8_recip(float s) { return 1.0 / static_cast<double>(s); }
__device__ inline int quant_i8(float x, double rd) {
  const float q = static_cast<float>(static_cast<double>(x) * rd);
  return static_cast<int>(fminf(fmaxf(rintf(q), -127.0f), 127.0f));
}
__device__ inline uint2 quant8_i8(const float* v, double rd) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= (static_cast<uint32_t>(quant_i8(v[i], rd)) & 0xffu) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= (static_cast<uint32_t>(quant_i8(v[4 + i], rd)) & 0xffu) << (8 * i);
  return make_uint2(lo, hi);
}
// Per-token int8 scale: max(amax / 127, 1e-8) in fp32.
__device__ inline float i8_scale(float amax) { return fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f); }

// (LPR, NC) of a row of n_chunks chunks: the smallest NC with LPR = 64 up to
// 4 chunks per lane, else LPR = 256 with up to 8.  Returns false when the row
// is wider than 2048 chunks (16384 bf16).
inline bool pick_shape(int64_t n_chunks, int& lpr, int& nc) {
  if (n_chunks <= 64 * 4) {
    lpr = 64;
    nc = static_cast<int>((n_chunks + 63) / 64);
    return true;
  }
  if (n_chunks <= 256 * 8) {
    lpr = 256;
    nc = static_cast<int>((n_chunks + 255) / 256);
    return true;
  }
  return false;
}

// Calls f(ic<LPR>, ic<NC>) for the shape picked above (NC >= 1).
template <int V>
using icst = std::integral_constant<int, V>;
template <typename F>
inline void dispatch_shape(int lpr, int nc, F&& f) {
  if (lpr == 64) {
    switch (nc) {
      case 1: f(icst<64>{}, icst<1>{}); break;
      case 2: f(icst<64>{}, icst<2>{}); break;
      case 3: f(icst<64>{}, icst<3>{}); break;
      default: f(icst<64>{}, icst<4>{}); break;
    }
  } else {
    switch (nc) {
      case 2: f(icst<256>{}, icst<2>{}); break;
      case 3: f(icst<256>{}, icst<3>{}); break;
      case 4: f(icst<256>{}, icst<4>{}); break;
      case 5: f(icst<256>{}, icst<5>{}); break;
      case 6: f(icst<256>{}, icst<6>{}); break;
      case 7: f(icst<256>{}, icst<7>{}); break;
      default: f(icst<256>{}, icst<8>{}); break;
    }
  }
}

}  // namespace rows
}  // namespace wf
