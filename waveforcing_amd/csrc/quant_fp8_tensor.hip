// Per-tensor e4m3 quantization of a bf16 matrix, the reference's FP8 linear
// modes (wave_rt/runtime/fp8.py):
//   weights (fp8.py:33-35), fp32 arithmetic:
//     s = max(amax|w| / 448, 1e-8);  code = e4m3(fp32(w) / s)
//   activations (fp8.py:47-48), bf16 tensor arithmetic:
//     s = max(bf16(amax|x| / 448), bf16(1e-8));  code = e4m3(bf16(x / s))
// Quotients are the IEEE (correctly rounded) fp32 ones, as torch's are.  The quotient's
// magnitude is at most 448 (weights: 448 * (1 + 2^-23); activations, with s
// rounded to bf16: 450 after the bf16 rounding), where e4m3's round-to-
// nearest-even gives 448 (values up to 464 round there); clamping to 448 and
// converting with v_cvt_pk_fp8_f32 reproduces torch's cast.
//
// Two passes, no atomics: amax partials per workgroup, then every
// quantization workgroup reduces the partials itself (at most 4 KB, from L2)
// before encoding its share; workgroup 0 writes the scale.
#include "fp8_codec.hpp"
#include "launchers.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

constexpr int kThreads = 256;
constexpr int kChunksPerThread = 4;  // 8-element chunks per thread per pass of the amax loop
constexpr int kQuantBlocks = 2048;   // cap of the quantizing grid

__device__ inline float block_max(float v, float* red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

struct Geometry {
  const uint16_t* x;
  int64_t ldx;
  int64_t rows;
  int chunks_per_row;  // k / 8
  int64_t total;       // rows * chunks_per_row
};

__device__ inline const uint16_t* chunk_ptr(const Geometry& g, int64_t c) {
  const int64_t r = c / g.chunks_per_row;
  return g.x + r * g.ldx + (c - r * g.chunks_per_row) * 8;
}

__global__ __launch_bounds__(kThreads) void amax_partials_kernel(Geometry g, float* __restrict__ partials) {
  __shared__ float red[4];
  float m = 0.f;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < g.total;
       c += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint4 w = *reinterpret_cast<const uint4*>(chunk_ptr(g, c));
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo_to_f32(u[i])), fabsf(bf16_hi_to_f32(u[i]))));
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

template <bool ACT>
__global__ __launch_bounds__(kThreads) void quant_tensor_kernel(Geometry g, const float* __restrict__ partials,
                                                                int n_partials, uint8_t* __restrict__ codes,
                                                                float* __restrict__ scale_out) {
  __shared__ float red[4];
  float m = 0.f;
  for (int i = threadIdx.x; i < n_partials; i += kThreads) m = fmaxf(m, partials[i]);
  const float amax = block_max(m, red);
  float s;
  if (ACT) {
    s = bf16_bits_to_f32(f32_to_bf16_rne(__fdiv_rn(amax, kE4M3Max)));
    s = fmaxf(s, bf16_bits_to_f32(kScaleFloorBf16Bits));
  } else {
    s = fmaxf(__fdiv_rn(amax, kE4M3Max), 1e-8f);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
  // RN32(x / s) as RN32(RN64(x * RN64(1 / s))): equal to the IEEE fp32
  // quotient for all fp32 x, s (an fp32 quotient is never an fp32 rounding
  // midpoint and otherwise lies >= 2^-49 relative from one; the fp64 product
  // is within 2^-52), at fp64-multiply cost instead of a division sequence.
  const double rd = 1.0 / static_cast<double>(s);
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < g.total;
       c += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint4 w = *reinterpret_cast<const uint4*>(chunk_ptr(g, c));
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
    float q[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q[2 * i] = static_cast<float>(static_cast<double>(bf16_lo_to_f32(u[i])) * rd);
      q[2 * i + 1] = static_cast<float>(static_cast<double>(bf16_hi_to_f32(u[i])) * rd);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (ACT) q[i] = bf16_bits_to_f32(f32_to_bf16_rne(q[i]));
      q[i] = fminf(fmaxf(q[i], -kE4M3Max), kE4M3Max);
    }
    *reinterpret_cast<uint2*>(codes + c * 8) =
        make_uint2(e4m3_pack4_hw(q[0], q[1], q[2], q[3]), e4m3_pack4_hw(q[4], q[5], q[6], q[7]));
  }
}

// out[i] = fp32(code[i]) * s, 16 codes per thread per pass.  The product of a 4-bit e4m3 significand and an
// 8-bit (bf16-derived) scale significand is exact in fp32: this is the reference's
// `codes.view(e4m3).to(bf16) * scale` with a 1-element fp32 scale, whose result type is fp32
// (wave_rt/denoiser/exchange/common.py:161-164).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void dequant_tensor_f32_kernel(const u32x4* __restrict__ codes,
                                                                      const float* __restrict__ scale, int64_t n16,
                                                                      f32x4* __restrict__ out) {
  const float s = scale[0];
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const u32x4 w = __builtin_nontemporal_load(codes + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a, b, c, d;
      e4m3_unpack4_hw(w[j], a, b, c, d);
      const f32x4 v = {a * s, b * s, c * s, d * s};
      __builtin_nontemporal_store(v, out + 4 * i + j);
    }
  }
}

}  // namespace

int launch_fp8_quant_pertensor(const void* x, int64_t rows, int64_t k, int64_t ldx, int mode, uint8_t* codes,
                               float* scale, float* partials, hipStream_t stream) {
  Geometry g{static_cast<const uint16_t*>(x), ldx, rows, static_cast<int>(k / 8), rows * (k / 8)};
  const int64_t want = (g.total + kThreads * kChunksPerThread - 1) / (kThreads * kChunksPerThread);
  const int n_partials = static_cast<int>(want < WF_FP8_AMAX_PARTIALS ? (want > 0 ? want : 1) : WF_FP8_AMAX_PARTIALS);
  hipLaunchKernelGGL(amax_partials_kernel, dim3(n_partials), dim3(kThreads), 0, stream, g, partials);
  // At most 2048 quantizing workgroups, each first reducing the (<= 1024) partials from L2: with one
  // workgroup per 2048 elements the partials' reads added up to about the tensor's own size.
  const int64_t qblocks = (g.total + kThreads - 1) / kThreads;
  const dim3 qgrid(static_cast<uint32_t>(qblocks < kQuantBlocks ? (qblocks > 0 ? qblocks : 1) : kQuantBlocks));
  if (mode == WF_FP8_TENSOR_ACT)
    hipLaunchKernelGGL((quant_tensor_kernel<true>), qgrid, dim3(kThreads), 0, stream, g, partials, n_partials, codes,
                       scale);
  else
    hipLaunchKernelGGL((quant_tensor_kernel<false>), qgrid, dim3(kThreads), 0, stream, g, partials, n_partials, codes,
                       scale);
  return check_launch("wf_fp8_quant_pertensor");
}

}  // namespace wf

extern "C" int wf_fp8_quant_pertensor(const void* x, int64_t rows, int64_t k, int64_t ldx, int32_t mode,
                                      uint8_t* codes, float* scale, float* ws_partials, void* stream) {
  static const char* fn = "wf_fp8_quant_pertensor";
  WF_REQUIRE(rows > 0 && k > 0 && ldx >= k, WF_E_INVALID, "%s: bad sizes rows=%lld k=%lld ldx=%lld (amax of an empty tensor is undefined)", fn,
             (long long)rows, (long long)k, (long long)ldx);
  WF_REQUIRE(mode == WF_FP8_TENSOR_WEIGHT || mode == WF_FP8_TENSOR_ACT, WF_E_INVALID, "%s: unknown mode %d", fn,
             mode);
  WF_REQUIRE(k % 8 == 0 && ldx % 8 == 0, WF_E_SHAPE, "%s: k and ldx must be multiples of 8", fn);
  WF_REQUIRE(x && codes && scale && ws_partials, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(codes) & 7u) == 0,
             WF_E_ALIGN, "%s: x must be 16-byte and codes 8-byte aligned", fn);
  return wf::launch_fp8_quant_pertensor(x, rows, k, ldx, mode, codes, scale, ws_partials, wf::as_stream(stream));
}

extern "C" int wf_fp8_dequant_pertensor_f32(const uint8_t* codes, const float* scale, int64_t n, float* out,
                                            void* stream) {
  static const char* fn = "wf_fp8_dequant_pertensor_f32";
  WF_REQUIRE(n >= 0, WF_E_INVALID, "%s: n=%lld is negative", fn, (long long)n);
  if (n == 0) return WF_OK;
  WF_REQUIRE(n % 16 == 0, WF_E_SHAPE, "%s: n=%lld must be a multiple of 16", fn, (long long)n);
  WF_REQUIRE(n < (1ll << 40), WF_E_SHAPE, "%s: n=%lld too large", fn, (long long)n);
  WF_REQUIRE(codes && scale && out, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(codes) & 15u) == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(scale) & 3u) == 0,
             WF_E_ALIGN, "%s: codes and out must be 16-byte aligned", fn);
  const int64_t n16 = n / 16;
  const int64_t blocks = (n16 + wf::kThreads - 1) / wf::kThreads;
  const dim3 grid(static_cast<uint32_t>(blocks < 8192 ? blocks : 8192));
  hipLaunchKernelGGL(wf::dequant_tensor_f32_kernel, grid, dim3(wf::kThreads), 0, wf::as_stream(stream),
                     reinterpret_cast<const wf::u32x4*>(codes), scale, n16, reinterpret_cast<wf::f32x4*>(out));
  return wf::check_launch(fn);
}
