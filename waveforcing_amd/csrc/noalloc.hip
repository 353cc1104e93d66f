// The W8A8 int8 linear for callers that cannot allocate: wf_w8a8_linear with
// its activation workspace (int8 codes [m][k] and fp32 row scales [m]) held
// in a file-scope device array instead of caller-passed buffers.
//
// The array is one per GPU (each device's copy of the code object has its own
// at its own address), lives until the process ends and is shared by every
// call on that GPU: calls that overlap on one GPU race on it.  The kernels
// write every code and scale they read in the same call (the row quantizer
// fills codes and scales before the GEMM reads them, in stream order), so
// nothing carries over from an earlier call and nothing needs clearing.
//
// The host never passes the array's name to a kernel or a copy: on the host
// that name is a stand-in, not a device address.  The device address comes
// from hipGetSymbolAddress, once per device with that device current, and
// is kept per device.
#include <atomic>
#include <mutex>

#include "launchers.hpp"
#include "wf_common.hpp"

namespace {
constexpr int64_t kScratchCodeBytes = WF_W8A8_STATIC_MAX_CODES;   // int8 codes, m * k
constexpr int64_t kScratchRows = WF_W8A8_STATIC_MAX_ROWS;         // fp32 scales, m
}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchCodeBytes + kScratchRows * 4];

namespace wf {
namespace {

constexpr int kMaxDevices = 64;
std::atomic<uint8_t*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array (looked up once per device).
int scratch_of_current_device(uint8_t** out, const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(static_cast<int>(e), "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  WF_REQUIRE(dev >= 0 && dev < kMaxDevices, WF_E_INVALID, "%s: device %d beyond %d devices", fn, dev, kMaxDevices);
  uint8_t* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr)
        return set_error(e != hipSuccess ? static_cast<int>(e) : WF_E_INVALID,
                         "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                         e != hipSuccess ? hipGetErrorString(e) : "null address");
      p = static_cast<uint8_t*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return WF_OK;
}

}  // namespace
}  // namespace wf

extern "C" int wf_w8a8_linear_static(const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qw,
                                     const float* sw, const void* bias, int64_t n, void* y, int64_t ldy,
                                     int32_t flags, void* stream) {
  static const char* fn = "wf_w8a8_linear_static";
  WF_REQUIRE(m >= 0 && n >= 0 && k > 0 && ldx >= k && ldy >= n, WF_E_INVALID,
             "%s: bad sizes m=%lld n=%lld k=%lld ldx=%lld ldy=%lld", fn, (long long)m, (long long)n, (long long)k,
             (long long)ldx, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(m <= kScratchRows && wf::product_below({m, k}, kScratchCodeBytes + 1), WF_E_SHAPE,
             "%s: m=%lld x k=%lld exceeds the static workspace (m <= %lld, m*k <= %lld bytes)", fn, (long long)m,
             (long long)k, (long long)kScratchRows, (long long)kScratchCodeBytes);
  WF_REQUIRE(x && qw && sw && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(n < (1ll << 31) && wf::product_below({n + 256, k}, (1ll << 31) - 16), WF_E_SHAPE,
             "%s: weights of 2 GiB or more are not supported", fn);
  WF_REQUIRE(k % 16 == 0 && ldx % 8 == 0, WF_E_SHAPE, "%s: k %% 16 and ldx %% 8 must be 0", fn);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(qw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(sw) & 15u) == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0 &&
                 (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: x, qw, sw must be 16-byte and y, bias 8-byte aligned", fn);
  WF_REQUIRE((flags & ~(WF_GEMM_GELU_TANH | WF_LINEAR_GELU_INPUT)) == 0, WF_E_INVALID, "%s: unknown flags 0x%x", fn,
             flags);
  uint8_t* base = nullptr;
  if (int rc = wf::scratch_of_current_device(&base, fn)) return rc;
  int8_t* q = reinterpret_cast<int8_t*>(base);
  float* sx = reinterpret_cast<float*>(base + kScratchCodeBytes);   // 256-byte aligned (the code region is)
  hipStream_t st = wf::as_stream(stream);
  if (int rc = wf::launch_quant_rows_i8(x, m, k, ldx, q, k, sx, st, (flags & WF_LINEAR_GELU_INPUT) != 0)) return rc;
  return wf::launch_gemm_i8(q, qw, m, n, k, sx, sw, bias, y, ldy, nullptr, flags & WF_GEMM_GELU_TANH, st);
}
