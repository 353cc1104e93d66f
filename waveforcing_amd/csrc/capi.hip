// Status reporting of the C ABI and the elementwise FP8 cast entry points.
#include <cstring>

#include "fp8_codec.hpp"
#include "wf_common.hpp"

namespace wf {

char* error_buffer() {
  static thread_local char buf[512];
  return buf;
}

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(static_cast<int>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  return WF_OK;
}

namespace {

// One thread per 4 values.  |x| <= 448 takes the hardware converter (the
// path the pack kernel uses), everything else the portable encoder, so the
// result is torch's cast over the whole fp32 range.
__global__ __launch_bounds__(256) void encode_f32_kernel(const float* __restrict__ x,
                                                         uint8_t* __restrict__ codes, int64_t n) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i0 >= n) return;
  if (i0 + 4 <= n) {
    float v[4];
    bool in_range = true;
    for (int j = 0; j < 4; ++j) {
      v[j] = x[i0 + j];
      in_range = in_range && (fabsf(v[j]) <= kE4M3Max);
    }
    uint32_t w;
    if (in_range) {
      w = e4m3_pack4_hw(v[0], v[1], v[2], v[3]);
    } else {
      w = 0;
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = fabsf(v[j]) <= kE4M3Max ? (e4m3_pack4_hw(v[j], 0.f, 0.f, 0.f) & 0xffu)
                                                   : e4m3_encode_sw(v[j]);
        w |= c << (8 * j);
      }
    }
    for (int j = 0; j < 4; ++j) codes[i0 + j] = static_cast<uint8_t>(w >> (8 * j));
  } else {
    for (int64_t i = i0; i < n; ++i) {
      const float v = x[i];
      codes[i] = fabsf(v) <= kE4M3Max ? static_cast<uint8_t>(e4m3_pack4_hw(v, 0.f, 0.f, 0.f) & 0xffu)
                                      : e4m3_encode_sw(v);
    }
  }
}

__global__ __launch_bounds__(256) void decode_f32_kernel(const uint8_t* __restrict__ codes,
                                                         float* __restrict__ out, int64_t n) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i0 >= n) return;
  if (i0 + 4 <= n) {
    uint32_t w = 0;
    for (int j = 0; j < 4; ++j) w |= static_cast<uint32_t>(codes[i0 + j]) << (8 * j);
    float v[4];
    e4m3_unpack4_hw(w, v[0], v[1], v[2], v[3]);
    for (int j = 0; j < 4; ++j) out[i0 + j] = v[j];
  } else {
    for (int64_t i = i0; i < n; ++i) {
      float v0, v1, v2, v3;
      e4m3_unpack4_hw(codes[i], v0, v1, v2, v3);
      out[i] = v0;
    }
  }
}

}  // namespace
}  // namespace wf

extern "C" {

const char* wf_last_error(void) { return wf::error_buffer(); }

int wf_abi_version(void) { return (1 << 16) | 1; }

int wf_fp8_e4m3_encode_f32(const float* x, uint8_t* codes, int64_t n, void* stream) {
  WF_REQUIRE(n >= 0, WF_E_INVALID, "wf_fp8_e4m3_encode_f32: n=%lld < 0", (long long)n);
  if (n == 0) return WF_OK;
  WF_REQUIRE(x && codes, WF_E_INVALID, "wf_fp8_e4m3_encode_f32: null pointer");
  const int64_t threads = (n + 3) / 4;
  const int64_t blocks = (threads + 255) / 256;
  WF_REQUIRE(blocks < (1ll << 31), WF_E_SHAPE, "wf_fp8_e4m3_encode_f32: n too large");
  hipLaunchKernelGGL(wf::encode_f32_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     wf::as_stream(stream), x, codes, n);
  return wf::check_launch("wf_fp8_e4m3_encode_f32");
}

int wf_fp8_e4m3_decode_f32(const uint8_t* codes, float* out, int64_t n, void* stream) {
  WF_REQUIRE(n >= 0, WF_E_INVALID, "wf_fp8_e4m3_decode_f32: n=%lld < 0", (long long)n);
  if (n == 0) return WF_OK;
  WF_REQUIRE(codes && out, WF_E_INVALID, "wf_fp8_e4m3_decode_f32: null pointer");
  const int64_t threads = (n + 3) / 4;
  const int64_t blocks = (threads + 255) / 256;
  WF_REQUIRE(blocks < (1ll << 31), WF_E_SHAPE, "wf_fp8_e4m3_decode_f32: n too large");
  hipLaunchKernelGGL(wf::decode_f32_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     wf::as_stream(stream), codes, out, n);
  return wf::check_launch("wf_fp8_e4m3_decode_f32");
}

}  // extern "C"
