// Per-row symmetric int8 quantization (per-token activations, and per
// output channel weights: both are rows of a row-major matrix).
//
//   s[m] = max(max_k |x[m,k]| / 127, 1e-8)              (fp32)
//   q    = clamp(round_half_even(x / s), -127, 127)     (x / s: IEEE fp32)
//
// The workload's W8A8 scheme (the reference's own W8A8 is FP8 per tensor,
// wave_rt/runtime/fp8.py:33-35,47-48; this is its per-token / per-channel
// int8 counterpart with the same clamp(min=1e-8) floor).
//
// x / s is formed as q = |x| * r, r = RN(1/s), refined once with the exact
// residual fma(-q, s, |x|); a 1-ulp error of that quotient can only change
// the integer rounding when the quotient sits within one ulp of k + 1/2, and
// those elements are recomputed with a full IEEE division, so the result is
// round_half_even(RN(x / s)) exactly.
//
// One workgroup (256 threads) per row for long rows: each thread owns 16
// consecutive bf16 (two 16-byte loads) and writes 16 int8 codes (one
// 16-byte store) per pass.  The row is read from HBM once and kept in
// registers between the amax reduction and the quantization pass when
// K <= 4096 (the 1.3B/14B widths up to 4096); longer rows take a second
// read (served by L2).
#include "launchers.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

constexpr int kThreads = 256;
constexpr int kElemsPerThread = 16;
constexpr int kRegPasses = 1;  // 4096 elements per row held in registers

__device__ inline float row_reduce_max(float v, float* red) {
  // wave64: butterfly via DPP-free shuffles (cheap at this volume)
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w]);
  return m;
}

__device__ inline int8_t quant_one(float x, float s, float r) {
  const float ax = fabsf(x);
  float q = ax * r;
  q = fmaf(fmaf(-q, s, ax), r, q);
  const float k = rintf(q);
  const float d = fabsf(q - k);
  // 1 ulp of q for q < 2^24 is at most q * 2^-23.
  if (fabsf(d - 0.5f) <= q * 1.1920929e-7f) q = __fdiv_rn(ax, s);
  float qi = fminf(rintf(q), 127.0f);
  qi = x < 0.f ? -qi : qi;
  return static_cast<int8_t>(static_cast<int>(qi));
}

__device__ inline void load16(const uint16_t* row, int64_t k0, int64_t K, uint4& a, uint4& b) {
  if (k0 + 16 <= K) {
    const uint4* p = reinterpret_cast<const uint4*>(row + k0);
    a = p[0];
    b = p[1];
  } else {
    uint32_t w[8];
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = (k0 + 2 * i < K) ? row[k0 + 2 * i] : 0u;
      const uint32_t hi = (k0 + 2 * i + 1 < K) ? row[k0 + 2 * i + 1] : 0u;
      w[i] = lo | (hi << 16);
    }
    a = make_uint4(w[0], w[1], w[2], w[3]);
    b = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

__device__ inline float amax16(const uint4& a, const uint4& b) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo_to_f32(w[i])), fabsf(bf16_hi_to_f32(w[i]))));
  return m;
}

__device__ inline void quant16_store(const uint4& a, const uint4& b, float s, float r, int8_t* out, int64_t k0,
                                     int64_t K) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t packed[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int8_t q0 = quant_one(bf16_lo_to_f32(w[2 * i]), s, r);
    const int8_t q1 = quant_one(bf16_hi_to_f32(w[2 * i]), s, r);
    const int8_t q2 = quant_one(bf16_lo_to_f32(w[2 * i + 1]), s, r);
    const int8_t q3 = quant_one(bf16_hi_to_f32(w[2 * i + 1]), s, r);
    packed[i] = (static_cast<uint32_t>(static_cast<uint8_t>(q0))) |
                (static_cast<uint32_t>(static_cast<uint8_t>(q1)) << 8) |
                (static_cast<uint32_t>(static_cast<uint8_t>(q2)) << 16) |
                (static_cast<uint32_t>(static_cast<uint8_t>(q3)) << 24);
  }
  if (k0 + 16 <= K) {
    *reinterpret_cast<uint4*>(out + k0) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  } else {
    for (int i = 0; i < 16 && k0 + i < K; ++i) out[k0 + i] = static_cast<int8_t>(packed[i / 4] >> (8 * (i % 4)));
  }
}

__global__ __launch_bounds__(kThreads) void quant_rows_i8_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                                 int64_t K, int64_t ldx, int8_t* __restrict__ q,
                                                                 int64_t ldq, float* __restrict__ scales) {
  __shared__ float red[kThreads / 64];
  const int64_t m = blockIdx.x;
  if (m >= M) return;
  const uint16_t* row = x + m * ldx;
  int8_t* qrow = q + m * ldq;
  const int64_t span = static_cast<int64_t>(kThreads) * kElemsPerThread;
  const int64_t k_first = static_cast<int64_t>(threadIdx.x) * kElemsPerThread;

  uint4 ra[kRegPasses], rb[kRegPasses];
  float amax = 0.f;
#pragma unroll
  for (int p = 0; p < kRegPasses; ++p) {
    const int64_t k0 = k_first + p * span;
    if (k0 < K) {
      load16(row, k0, K, ra[p], rb[p]);
      amax = fmaxf(amax, amax16(ra[p], rb[p]));
    } else {
      ra[p] = make_uint4(0, 0, 0, 0);
      rb[p] = ra[p];
    }
  }
  for (int64_t k0 = k_first + kRegPasses * span; k0 < K; k0 += span) {
    uint4 a, b;
    load16(row, k0, K, a, b);
    amax = fmaxf(amax, amax16(a, b));
  }
  amax = row_reduce_max(amax, red);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
  const float r = __frcp_rn(s);
  if (threadIdx.x == 0) scales[m] = s;
#pragma unroll
  for (int p = 0; p < kRegPasses; ++p) {
    const int64_t k0 = k_first + p * span;
    if (k0 < K) quant16_store(ra[p], rb[p], s, r, qrow, k0, K);
  }
  for (int64_t k0 = k_first + kRegPasses * span; k0 < K; k0 += span) {
    uint4 a, b;
    load16(row, k0, K, a, b);
    quant16_store(a, b, s, r, qrow, k0, K);
  }
}

}  // namespace

int launch_quant_rows_i8(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                         hipStream_t stream) {
  hipLaunchKernelGGL(quant_rows_i8_kernel, dim3(static_cast<uint32_t>(M)), dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(x), M, K, ldx, q, ldq, scales);
  return check_launch("wf_quant_rows_i8");
}

}  // namespace wf

extern "C" int wf_quant_rows_i8(const void* x, int64_t m, int64_t k, int64_t ldx, int8_t* q, float* scales,
                                void* stream) {
  static const char* fn = "wf_quant_rows_i8";
  WF_REQUIRE(m >= 0 && k >= 0 && ldx >= k, WF_E_INVALID, "%s: bad sizes m=%lld k=%lld ldx=%lld", fn, (long long)m,
             (long long)k, (long long)ldx);
  if (m == 0 || k == 0) return WF_OK;
  WF_REQUIRE(x && q && scales, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(m < (1ll << 31), WF_E_SHAPE, "%s: m=%lld too large", fn, (long long)m);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (ldx % 8) == 0 &&
                 (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && (k % 16) == 0,
             WF_E_ALIGN, "%s: x and q must be 16-byte aligned with ldx %% 8 == 0 and k %% 16 == 0", fn);
  return wf::launch_quant_rows_i8(x, m, k, ldx, q, k, scales, wf::as_stream(stream));
}
