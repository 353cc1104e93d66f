// W8A8 int8 GEMM on the gfx950 i8 matrix cores with a fused dequant + bias
// (+ optional GELU-tanh) bf16 epilogue.
//
//   acc[m,n] = sum_k qx[m,k] * qw[n,k]                      (int32, exact)
//   y[m,n]   = bf16( (float(acc) * sx[m]) * sw[n] + bias[n] )  (fp32, this order,
//                                                             no fused multiply-add)
//   gelu:      y = bf16( gelu_tanh(float(y)) )
//
// This is the per-token / per-channel int8 counterpart of the reference's
// W8A8 linear (wave_rt/runtime/fp8.py:46-56: quantized GEMM, x scale_a x
// scale_b, + bias, bf16 out) and of the FFN's GELU(approximate='tanh')
// (naive_rt/rolling_forcing/wan/modules/causal_model.py:342-344).
//
// Tiling: a 256-thread workgroup computes a 256 (M) x 128 (N) tile, K in
// steps of 128 bytes.  Both operands are K-contiguous ("NT"), so global
// loads are 16-byte vectors along K, staged through LDS (double buffered,
// rows padded to 144 B so the 16-byte fragment reads of 8 consecutive rows
// hit distinct banks).  The four waves form a 2 x 2 grid of 128 x 64 wave
// tiles, each 4 x 2 blocks of v_mfma_i32_32x32x32_i8.  The weight fragment is
// the MFMA's first operand and the activation fragment the second, so the
// 32x32 result block is (n, m): each lane ends up with 4 consecutive output
// features of one token per accumulator group, stored as one 8-byte bf16
// vector.  Tiles are ordered so that the workgroups a given XCD receives
// (blockIdx % 8) cover a contiguous band of M, keeping their activation rows
// and the weight in that XCD's L2.
#include "launchers.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 128, BK = 128;
constexpr int PITCH = BK + 16;                 // LDS row pitch in bytes
constexpr int A_STAGE = BM * PITCH;            // 36864 B
constexpr int B_STAGE = BN * PITCH;            // 18432 B
constexpr int STAGE = A_STAGE + B_STAGE;       // 55296 B
constexpr int A_CHUNKS = BM * BK / 16 / 256;   // 16-byte loads per thread per stage (8)
constexpr int B_CHUNKS = BN * BK / 16 / 256;   // (4)
constexpr int NUM_XCD = 8;

struct GemmArgs {
  const int8_t* a;     // [M, K]
  const int8_t* w;     // [N, K]
  const float* sx;     // [M]
  const float* sw;     // [N]
  const uint16_t* bias;  // [N] bf16 or null
  uint16_t* y;         // [M, N] bf16 (ldy)
  int32_t* acc_out;    // [M, N] int32 or null
  int M, N, K;
  int64_t ldy;
};

__device__ inline float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}

__device__ inline float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_rne(f)); }

template <bool HAS_BIAS, bool GELU>
__global__ __launch_bounds__(256, 1) void gemm_i8_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int n_tiles = tiles_m * tiles_n;
  const int per_xcd = (n_tiles + NUM_XCD - 1) / NUM_XCD;
  const int t = (blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
  if (t >= n_tiles) return;
  const int m0 = (t / tiles_n) * BM;
  const int n0 = (t % tiles_n) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // 0..1 -> 128-row half of the tile
  const int wn = wave & 1;   // 0..1 -> 64-col half
  const int l32 = lane & 31;
  const int half = lane >> 5;

  // Global -> register staging of one K step.
  uint4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, col = (c & 7) * 16;
      const int gm = m0 + row, gk = k0 + col;
      ra[i] = (gm < p.M && gk < p.K) ? *reinterpret_cast<const uint4*>(p.a + static_cast<int64_t>(gm) * p.K + gk)
                                    : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, col = (c & 7) * 16;
      const int gn = n0 + row, gk = k0 + col;
      rb[i] = (gn < p.N && gk < p.K) ? *reinterpret_cast<const uint4*>(p.w + static_cast<int64_t>(gn) * p.K + gk)
                                    : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_stage = [&](int buf) {
    uint8_t* sa = lds + buf * STAGE;
    uint8_t* sb = sa + A_STAGE;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<uint4*>(sa + (c >> 3) * PITCH + (c & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<uint4*>(sb + (c >> 3) * PITCH + (c & 7) * 16) = rb[i];
    }
  };

  v16i acc[2][4];  // [n block j][m block i]
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int nk = (p.K + BK - 1) / BK;
  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int kb = 0; kb < nk; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nk) load_stage((kb + 1) * BK);
    const uint8_t* sa = lds + cur * STAGE;
    const uint8_t* sb = sa + A_STAGE;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int col = s * 32 + half * 16;
      v4i fa[4], fw[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = *reinterpret_cast<const v4i*>(sa + (wm * 128 + i * 32 + l32) * PITCH + col);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        fw[j] = *reinterpret_cast<const v4i*>(sb + (wn * 64 + j * 32 + l32) * PITCH + col);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[j][i], 0, 0, 0);
    }
    if (kb + 1 < nk) store_stage(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  Block (j, i) element (n, m): m = l32, n = 8*(r/4) + 4*half + r%4.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + wm * 128 + i * 32 + l32;
    const bool row_ok = gm < p.M;
    const float sxm = row_ok ? p.sx[gm] : 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int gn = n0 + wn * 64 + j * 32 + 8 * g + 4 * half;
        // N % 4 == 0 (checked at the entry point): a 4-wide group is all in or all out.
        if (row_ok && gn < p.N) {
          const int a0 = acc[j][i][4 * g + 0], a1 = acc[j][i][4 * g + 1];
          const int a2 = acc[j][i][4 * g + 2], a3 = acc[j][i][4 * g + 3];
          const float4 swv = *reinterpret_cast<const float4*>(p.sw + gn);
          float y0 = __fmul_rn(__fmul_rn(static_cast<float>(a0), sxm), swv.x);
          float y1 = __fmul_rn(__fmul_rn(static_cast<float>(a1), sxm), swv.y);
          float y2 = __fmul_rn(__fmul_rn(static_cast<float>(a2), sxm), swv.z);
          float y3 = __fmul_rn(__fmul_rn(static_cast<float>(a3), sxm), swv.w);
          if (HAS_BIAS) {
            const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + gn);
            y0 = __fadd_rn(y0, bf16_lo_to_f32(bb.x));
            y1 = __fadd_rn(y1, bf16_hi_to_f32(bb.x));
            y2 = __fadd_rn(y2, bf16_lo_to_f32(bb.y));
            y3 = __fadd_rn(y3, bf16_hi_to_f32(bb.y));
          }
          if (GELU) {
            y0 = gelu_tanh(round_bf16(y0));
            y1 = gelu_tanh(round_bf16(y1));
            y2 = gelu_tanh(round_bf16(y2));
            y3 = gelu_tanh(round_bf16(y3));
          }
          const uint2 packed = make_uint2(
              static_cast<uint32_t>(f32_to_bf16_rne(y0)) | (static_cast<uint32_t>(f32_to_bf16_rne(y1)) << 16),
              static_cast<uint32_t>(f32_to_bf16_rne(y2)) | (static_cast<uint32_t>(f32_to_bf16_rne(y3)) << 16));
          *reinterpret_cast<uint2*>(p.y + static_cast<int64_t>(gm) * p.ldy + gn) = packed;
          if (p.acc_out)
            *reinterpret_cast<int4*>(p.acc_out + static_cast<int64_t>(gm) * p.N + gn) = make_int4(a0, a1, a2, a3);
        }
      }
    }
  }
}

}  // namespace

int launch_gemm_i8(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int gelu,
                   hipStream_t stream) {
  GemmArgs p;
  p.a = a;
  p.w = w;
  p.sx = sx;
  p.sw = sw;
  p.bias = static_cast<const uint16_t*>(bias);
  p.y = static_cast<uint16_t*>(y);
  p.acc_out = acc_out;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.ldy = ldy;
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int64_t grid = (tiles + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
  const dim3 g(static_cast<uint32_t>(grid)), b(256);
  if (bias && gelu)
    hipLaunchKernelGGL((gemm_i8_kernel<true, true>), g, b, 0, stream, p);
  else if (bias)
    hipLaunchKernelGGL((gemm_i8_kernel<true, false>), g, b, 0, stream, p);
  else if (gelu)
    hipLaunchKernelGGL((gemm_i8_kernel<false, true>), g, b, 0, stream, p);
  else
    hipLaunchKernelGGL((gemm_i8_kernel<false, false>), g, b, 0, stream, p);
  return check_launch("wf_gemm_i8");
}

}  // namespace wf

extern "C" int wf_gemm_i8(const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k, const float* sx,
                          const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int32_t flags,
                          void* stream) {
  static const char* fn = "wf_gemm_i8";
  WF_REQUIRE(m >= 0 && n >= 0 && k >= 0 && ldy >= n, WF_E_INVALID, "%s: bad sizes m=%lld n=%lld k=%lld ldy=%lld", fn,
             (long long)m, (long long)n, (long long)k, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(a && w && sx && sw && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), WF_E_SHAPE, "%s: size exceeds 2^31", fn);
  WF_REQUIRE(k % 16 == 0 && k > 0, WF_E_SHAPE, "%s: k=%lld must be a positive multiple of 16", fn, (long long)k);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && (reinterpret_cast<uintptr_t>(sw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(acc_out) & 15u) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: a, w, sw, acc_out must be 16-byte and y, bias 8-byte aligned", fn);
  WF_REQUIRE((flags & ~1) == 0, WF_E_INVALID, "%s: unknown flags 0x%x", fn, flags);
  return wf::launch_gemm_i8(a, w, m, n, k, sx, sw, bias, y, ldy, acc_out, flags & 1, wf::as_stream(stream));
}

extern "C" int wf_w8a8_linear(const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qw, const float* sw,
                              const void* bias, int64_t n, void* y, int64_t ldy, int32_t flags, int8_t* ws_q,
                              float* ws_sx, void* stream) {
  static const char* fn = "wf_w8a8_linear";
  WF_REQUIRE(m >= 0 && n >= 0 && k > 0 && ldx >= k && ldy >= n, WF_E_INVALID,
             "%s: bad sizes m=%lld n=%lld k=%lld ldx=%lld ldy=%lld", fn, (long long)m, (long long)n, (long long)k,
             (long long)ldx, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(x && qw && sw && y && ws_q && ws_sx, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), WF_E_SHAPE, "%s: size exceeds 2^31", fn);
  WF_REQUIRE(k % 16 == 0 && ldx % 8 == 0, WF_E_SHAPE, "%s: k %% 16 and ldx %% 8 must be 0", fn);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(qw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(ws_q) & 15u) == 0 && (reinterpret_cast<uintptr_t>(sw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: x, qw, sw, ws_q must be 16-byte and y, bias 8-byte aligned", fn);
  WF_REQUIRE((flags & ~1) == 0, WF_E_INVALID, "%s: unknown flags 0x%x", fn, flags);
  hipStream_t st = wf::as_stream(stream);
  if (int rc = wf::launch_quant_rows_i8(x, m, k, ldx, ws_q, k, ws_sx, st)) return rc;
  return wf::launch_gemm_i8(ws_q, qw, m, n, k, ws_sx, sw, bias, y, ldy, nullptr, flags & 1, st);
}
