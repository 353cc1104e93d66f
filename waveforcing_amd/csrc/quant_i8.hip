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
// x / s is formed as RN32(RN64(x * RN64(1/s))), which equals the IEEE fp32
// quotient for every fp32 x and s (rows::quant_i8 gives the argument), then
// rounded half to even, so the result is round_half_even(RN(x / s)) exactly.
//
// With GELU, every element is first replaced by bf16(gelu_tanh(x)) (the
// FFN activation applied to fc_in's bf16 output, causal_model.py:342-344)
// and those values are quantized: the same values the fc_in GEMM's GELU
// epilogue would have stored, so moving the activation here changes no bit
// and takes its VALU work off the GEMM's critical path.
//
// Rows up to 16384 wide run on the row engine of rows.hpp (one wave per row
// up to 2048, one workgroup per row above; the row stays in registers
// between the absmax reduction and the quantization pass).  Wider rows use
// one wave per row that reads the row twice (the second read is served by L2).
#include "launchers.hpp"
#include "rows.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr int kRegChunks = 8;  // 8 chunks x 8 elements x 64 lanes = 4096 per row in registers

__device__ inline float wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ inline float amax8(const uint4& a) {
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo_to_f32(w[i])), fabsf(bf16_hi_to_f32(w[i]))));
  return m;
}

// 8 bf16 values -> bf16(gelu_tanh(x)) of each (the GEMM epilogue's arithmetic).
__device__ inline uint4 gelu8(const uint4& a) {
  float v[8];
  rows::unpack8(a, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = gelu_tanh(v[i]);
  return rows::pack8(v);
}

template <bool GELU>
__device__ inline uint4 load_chunk(const uint16_t* p) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  if constexpr (GELU) return gelu8(a);
  return a;
}

// 8 bf16 values -> 8 int8 codes (rows::quant8_i8 with rd = RN64(1/s)).
__device__ inline uint2 quant8(const uint4& a, double rd) {
  float v[8];
  rows::unpack8(a, v);
  return rows::quant8_i8(v, rd);
}

// K % 8 == 0 (checked at the entry point): every 8-element chunk is whole.
template <bool GELU>
__global__ __launch_bounds__(kThreads) void quant_rows_i8_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                                 int64_t K, int64_t ldx, int8_t* __restrict__ q,
                                                                 int64_t ldq, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (m >= M) return;  // whole wave exits together
  const uint16_t* row = x + m * ldx;
  int8_t* qrow = q + m * ldq;
  const int64_t n_chunks = K / 8;

  uint4 reg[kRegChunks];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int64_t ch = lane + 64 * c;
    reg[c] = ch < n_chunks ? load_chunk<GELU>(row + ch * 8) : make_uint4(0, 0, 0, 0);
    amax = fmaxf(amax, amax8(reg[c]));
  }
  for (int64_t ch = lane + 64 * kRegChunks; ch < n_chunks; ch += 64)
    amax = fmaxf(amax, amax8(load_chunk<GELU>(row + ch * 8)));
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
  const double rd = rows::i8_recip(s);
  if (lane == 0) scales[m] = s;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int64_t ch = lane + 64 * c;
    if (ch < n_chunks) *reinterpret_cast<uint2*>(qrow + ch * 8) = quant8(reg[c], rd);
  }
  for (int64_t ch = lane + 64 * kRegChunks; ch < n_chunks; ch += 64)
    *reinterpret_cast<uint2*>(qrow + ch * 8) = quant8(load_chunk<GELU>(row + ch * 8), rd);
}

// Row-engine variant: LPR lanes per row, NC chunks of 8 per lane.
template <int LPR, int NC, bool GELU>
__global__ __launch_bounds__(256) void quant_rows_i8_row_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                                int64_t ldx, int8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ scales) {
  constexpr int RPB = 256 / LPR;
  __shared__ float red[4];
  const int lane = static_cast<int>(threadIdx.x) % LPR;
  const int m = static_cast<int>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / LPR;
  if (m >= M) return;  // uniform per row
  const int n_chunks = K >> 3;
  const uint16_t* row = x + static_cast<int64_t>(m) * ldx;
  uint4 reg[NC];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    reg[c] = ch < n_chunks ? rows::ld16(row + ch * 8) : make_uint4(0, 0, 0, 0);
  }
  if constexpr (GELU) {
#pragma unroll
    for (int c = 0; c < NC; ++c) reg[c] = gelu8(reg[c]);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) amax = fmaxf(amax, amax8(reg[c]));
  amax = rows::row_max_nonneg<LPR>(amax, red);
  const float s = rows::i8_scale(amax);
  const double rd = rows::i8_recip(s);
  if (lane == 0) scales[m] = s;
  int8_t* qrow = q + static_cast<int64_t>(m) * ldq;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    if (ch < n_chunks) *reinterpret_cast<uint2*>(qrow + ch * 8) = quant8(reg[c], rd);
  }
}

template <bool GELU>
void launch_rows(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                 hipStream_t stream) {
  int lpr = 0, nc = 0;
  if (rows::pick_shape(K / 8, lpr, nc)) {
    const uint32_t grid = static_cast<uint32_t>((M + 256 / lpr - 1) / (256 / lpr));
    rows::dispatch_shape(lpr, nc, [&](auto L, auto C) {
      hipLaunchKernelGGL((quant_rows_i8_row_kernel<decltype(L)::value, decltype(C)::value, GELU>), dim3(grid),
                         dim3(256), 0, stream, static_cast<const uint16_t*>(x), static_cast<int>(M),
                         static_cast<int>(K), ldx, q, ldq, scales);
    });
  } else {
    hipLaunchKernelGGL(quant_rows_i8_kernel<GELU>, dim3(static_cast<uint32_t>((M + kRowsPerBlock - 1) / kRowsPerBlock)),
                       dim3(kThreads), 0, stream, static_cast<const uint16_t*>(x), M, K, ldx, q, ldq, scales);
  }
}

}  // namespace

int launch_quant_rows_i8(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                         hipStream_t stream, bool gelu) {
  if (gelu)
    launch_rows<true>(x, M, K, ldx, q, ldq, scales, stream);
  else
    launch_rows<false>(x, M, K, ldx, q, ldq, scales, stream);
  return check_launch("wf_act_quant_i8");
}

}  // namespace wf

extern "C" int wf_act_quant_i8(const void* x, int64_t m, int64_t k, int64_t ldx, int8_t* q, float* scales,
                                void* stream) {
  static const char* fn = "wf_act_quant_i8";
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
