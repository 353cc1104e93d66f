// Flow-matching re-noising of a latent for the next DMD step.
//
//   out = bf16( RN32( RN32((1 - sigma) * x0) + RN32(sigma * noise) ) )
//
// FlowMatchScheduler.add_noise (naive_rt/rolling_forcing/utils/scheduler.py:
// 159-176) as _det_renoise calls it (wave_rt/denoiser/engine.py:221-235):
// one sigma for every frame, float32 arithmetic in that order (1 - sigma is
// itself an fp32 operation), the result cast to the noise dtype (bf16).
//
// x0 and out are [B, C, T, plane] bf16 (the latent's b, c, t, h*w order).
// The noise is either in the same layout or, as _det_renoise draws it,
// frame-major [B, T, C, plane] (its permute(0, 2, 1, 3, 4).flatten(0, 1)
// view of the latent); the kernel reads it in place, so the permuted copies
// of the reference disappear.  Elementwise and HBM-bound (6 bytes per
// element): 8 elements per thread when the plane is a multiple of 8 and the
// tensors are 16-byte aligned, one per thread otherwise.
#include "rows.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

__device__ inline int64_t noise_offset(int64_t row, int C, int T, int64_t plane, bool frame_major) {
  if (!frame_major) return row * plane;
  const int64_t b = row / (static_cast<int64_t>(C) * T);
  const int c = static_cast<int>((row / T) % C);
  const int t = static_cast<int>(row % T);
  return ((b * T + t) * C + c) * plane;
}

__device__ inline float renoise1(float x, float n, float a, float sigma) { return a * x + sigma * n; }

template <bool FRAME_MAJOR>
__global__ __launch_bounds__(256) void flow_add_noise_vec8_kernel(const uint16_t* __restrict__ x0,
                                                                  const uint16_t* __restrict__ noise,
                                                                  uint16_t* out, int C, int T, int64_t plane,
                                                                  int64_t n_vec, float sigma) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n_vec) return;
  const int64_t e = i * 8;
  const int64_t row = e / plane;
  const int64_t p = e - row * plane;
  const float a = 1.0f - sigma;
  float xv[8], nv[8];
  rows::unpack8(rows::ld16(x0 + e), xv);
  rows::unpack8(rows::ld16(noise + noise_offset(row, C, T, plane, FRAME_MAJOR) + p), nv);
#pragma unroll
  for (int k = 0; k < 8; ++k) xv[k] = renoise1(xv[k], nv[k], a, sigma);
  rows::st16(out + e, rows::pack8(xv));
}

template <bool FRAME_MAJOR>
__global__ __launch_bounds__(256) void flow_add_noise_kernel(const uint16_t* __restrict__ x0,
                                                             const uint16_t* __restrict__ noise, uint16_t* out,
                                                             int C, int T, int64_t plane, int64_t n, float sigma) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / plane;
  const int64_t p = e - row * plane;
  const float a = 1.0f - sigma;
  const float x = bf16_bits_to_f32(x0[e]);
  const float nz = bf16_bits_to_f32(noise[noise_offset(row, C, T, plane, FRAME_MAJOR) + p]);
  out[e] = f32_to_bf16_rne(renoise1(x, nz, a, sigma));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wf

extern "C" int wf_flow_add_noise_bf16(const void* x0, const void* noise, int64_t batch, int64_t channels,
                                      int64_t frames, int64_t plane, int32_t noise_frame_major, float sigma,
                                      void* out, void* stream) {
  static const char* fn = "wf_flow_add_noise_bf16";
  WF_REQUIRE(batch >= 0 && channels >= 0 && frames >= 0 && plane >= 0, WF_E_INVALID, "%s: negative size", fn);
  const int64_t n = batch * channels * frames * plane;
  if (n == 0) return WF_OK;
  WF_REQUIRE(x0 && noise && out, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(channels < (1ll << 31) && frames < (1ll << 31) && n < (1ll << 40), WF_E_SHAPE, "%s: sizes too large", fn);
  WF_REQUIRE(!(noise_frame_major && out == noise), WF_E_INVALID,
             "%s: out may alias x0 but not a frame-major noise tensor", fn);
  const bool fm = noise_frame_major != 0;
  const int C = static_cast<int>(channels), T = static_cast<int>(frames);
  const hipStream_t s = wf::as_stream(stream);
  const auto* xp = static_cast<const uint16_t*>(x0);
  const auto* np = static_cast<const uint16_t*>(noise);
  auto* op = static_cast<uint16_t*>(out);
  if (plane % 8 == 0 && wf::aligned16(x0) && wf::aligned16(noise) && wf::aligned16(out)) {
    const int64_t n_vec = n / 8;
    const dim3 grid(static_cast<uint32_t>((n_vec + 255) / 256));
    if (fm)
      hipLaunchKernelGGL(wf::flow_add_noise_vec8_kernel<true>, grid, dim3(256), 0, s, xp, np, op, C, T, plane, n_vec,
                         sigma);
    else
      hipLaunchKernelGGL(wf::flow_add_noise_vec8_kernel<false>, grid, dim3(256), 0, s, xp, np, op, C, T, plane, n_vec,
                         sigma);
  } else {
    const dim3 grid(static_cast<uint32_t>((n + 255) / 256));
    if (fm)
      hipLaunchKernelGGL(wf::flow_add_noise_kernel<true>, grid, dim3(256), 0, s, xp, np, op, C, T, plane, n, sigma);
    else
      hipLaunchKernelGGL(wf::flow_add_noise_kernel<false>, grid, dim3(256), 0, s, xp, np, op, C, T, plane, n, sigma);
  }
  return wf::check_launch(fn);
}
