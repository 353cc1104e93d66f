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
// Tiling (template parameters; the launcher's choice is measured): a
// workgroup computes a BM x BN tile with WM x WN waves, each wave a grid of
// 32x32 v_mfma_i32_32x32x32_i8 blocks; K advances 128 bytes per step.  Both
// operands are K-contiguous ("NT").  Global -> register staging uses buffer
// loads (the descriptor range zero-fills rows past M/N, so loads carry no
// predicate or branch) issued PGR steps ahead; LDS holds two stages with rows
// padded to 144 B so the 16-byte fragment reads of 8 consecutive rows hit
// distinct banks; each wave reads the fragments of sub-step s+1 while the
// MFMAs of sub-step s run.  The weight fragment is the MFMA's first operand
// and the activation fragment the second, so the 32x32 result block is
// (n, m): each lane ends up with 4 consecutive output features of one token
// per accumulator group, stored as one 8-byte bf16 vector.  Tiles are
// ordered so that the workgroups one XCD receives (blockIdx % 8) form a
// contiguous range, walked in bands of GROUP_M tile rows, so co-resident
// workgroups share A and W panels in that XCD's L2.
#include <utility>

#include "launchers.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BK = 128;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9-family parts:
// DATA_FORMAT = 32 bit.  With it, offsets >= num_records read as zero.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kOutOfRange = 0x7ffffff0;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int PITCH = BK + 16;  // LDS row pitch in bytes
constexpr int NUM_XCD = 8;

template <int N, typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

struct GemmArgs {
  const int8_t* a;       // [M, K]
  const int8_t* w;       // [N, K]
  const float* sx;       // [M]
  const float* sw;       // [N]
  const uint16_t* bias;  // [N] bf16 or null
  uint16_t* y;           // [M, N] bf16 (ldy)
  int32_t* acc_out;      // [M, N] int32 or null
  int M, N, K;
  int64_t ldy;
};

__device__ inline float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}

__device__ inline float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_rne(f)); }

// BM x BN workgroup tile, WM x WN waves, each wave (BM/WM) x (BN/WN) as
// MI x NI blocks of 32x32.  OCC = waves per SIMD the register budget is
// sized for (1: one workgroup of 4 waves per CU; 2: two).
template <int BM, int BN, int WM, int WN, int OCC, int PGR, bool XCD_REMAP, int GROUP_M, bool HAS_BIAS, bool GELU>
__global__ __launch_bounds__(WM * WN * 64, OCC) void gemm_i8_kernel(GemmArgs p) {
  constexpr int THREADS = WM * WN * 64;
  constexpr int A_STAGE = BM * PITCH;
  constexpr int B_STAGE = BN * PITCH;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int A_CHUNKS = BM * BK / 16 / THREADS;
  constexpr int B_CHUNKS = BN * BK / 16 / THREADS;
  constexpr int MI = BM / WM / 32;
  constexpr int NI = BN / WN / 32;
  static_assert(A_CHUNKS * 16 * THREADS == BM * BK && B_CHUNKS * 16 * THREADS == BN * BK, "tile/threads");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int n_tiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (XCD_REMAP) {
    const int per_xcd = (n_tiles + NUM_XCD - 1) / NUM_XCD;
    t = (blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
  }
  if (t >= n_tiles) return;
  int tm = t / tiles_n, tn = t % tiles_n;
  if (GROUP_M > 0) {
    // Grouped order: bands of GROUP_M tile rows swept column by column, so
    // the workgroups resident on one XCD at a time form a compact block and
    // share A rows and W rows in that XCD's L2.
    const int per_group = GROUP_M * tiles_n;
    const int first_m = (t / per_group) * GROUP_M;
    const int rows = min(tiles_m - first_m, GROUP_M);
    const int r = t % per_group;
    tm = first_m + r % rows;
    tn = r / rows;
  }
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  // Global -> register staging: PGR register buffers, so the loads of K
  // step kb + PGR are issued while step kb computes and have PGR compute
  // steps to arrive.  Buffer indices are compile-time (loop unrolled by PGR).
  uint4 ra[PGR][A_CHUNKS], rb[PGR][B_CHUNKS];
  // Buffer loads: the descriptor's range (M*K, N*K bytes) makes the hardware
  // return zeros for rows past M / N, and K-tail chunks are pointed past the
  // range, so the loads need no predicate and no branch.
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.a), 0, p.M * p.K, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_w =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.w), 0, p.N * p.K, kBufferRsrcWord3);
  int off_a[A_CHUNKS], col_a[A_CHUNKS], off_b[B_CHUNKS], col_b[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + THREADS * i;
    col_a[i] = (c & 7) * 16;
    off_a[i] = (m0 + (c >> 3)) * p.K + col_a[i];
  }
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + THREADS * i;
    col_b[i] = (c & 7) * 16;
    off_b[i] = (n0 + (c >> 3)) * p.K + col_b[i];
  }
  auto load_stage = [&](auto buf, int k0) {
    constexpr int u = decltype(buf)::value;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int off = (k0 + col_a[i] < p.K) ? off_a[i] + k0 : kOutOfRange;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, off, 0, 0);
      ra[u][i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int off = (k0 + col_b[i] < p.K) ? off_b[i] + k0 : kOutOfRange;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc_w, off, 0, 0);
      rb[u][i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  auto store_stage = [&](auto buf, int lbuf) {
    constexpr int u = decltype(buf)::value;
    uint8_t* sa = lds + lbuf * STAGE;
    uint8_t* sb = sa + A_STAGE;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + THREADS * i;
      *reinterpret_cast<uint4*>(sa + (c >> 3) * PITCH + (c & 7) * 16) = ra[u][i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + THREADS * i;
      *reinterpret_cast<uint4*>(sb + (c >> 3) * PITCH + (c & 7) * 16) = rb[u][i];
    }
  };

  v16i acc[NI][MI];  // [n block j][m block i]
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[j][i] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  auto compute = [&](int lbuf) {
    const uint8_t* sa = lds + lbuf * STAGE + (wm * (BM / WM) + l32) * PITCH + half * 16;
    const uint8_t* sb = lds + lbuf * STAGE + A_STAGE + (wn * (BN / WN) + l32) * PITCH + half * 16;
    // Fragments of sub-step s + 1 are read while the MFMAs of sub-step s run.
    v4i fa[2][MI], fw[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) fa[0][i] = *reinterpret_cast<const v4i*>(sa + i * 32 * PITCH);
#pragma unroll
    for (int j = 0; j < NI; ++j) fw[0][j] = *reinterpret_cast<const v4i*>(sb + j * 32 * PITCH);
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int cb = s & 1;
      if (s + 1 < BK / 32) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
          fa[cb ^ 1][i] = *reinterpret_cast<const v4i*>(sa + i * 32 * PITCH + (s + 1) * 32);
#pragma unroll
        for (int j = 0; j < NI; ++j)
          fw[cb ^ 1][j] = *reinterpret_cast<const v4i*>(sb + j * 32 * PITCH + (s + 1) * 32);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[cb][j], fa[cb][i], acc[j][i], 0, 0, 0);
    }
  };

  // Steps past K load zeros (a zero contribution), so the step count is
  // padded to a multiple of PGR and every step runs unconditionally.
  const int nk = ((p.K + BK - 1) / BK + PGR - 1) / PGR * PGR;
  static_for<PGR>([&](auto u) { load_stage(u, u.value * BK); });
  store_stage(std::integral_constant<int, 0>{}, 0);
  __syncthreads();

  for (int kb0 = 0; kb0 < nk; kb0 += PGR) {
    static_for<PGR>([&](auto u) {
      constexpr int U = decltype(u)::value;
      const int kb = kb0 + U;
      // register buffer U held step kb, already in LDS: refill it with step kb + PGR
      load_stage(u, (kb + PGR) * BK);
      compute(kb & 1);
      store_stage(std::integral_constant<int, (U + 1) % PGR>{}, (kb + 1) & 1);
      __syncthreads();
    });
  }

  // Epilogue.  Block (j, i) element (n, m): m = l32, n = 8*(r/4) + 4*half + r%4.
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int gm = m0 + wm * (BM / WM) + i * 32 + l32;
    const bool row_ok = gm < p.M;
    const float sxm = row_ok ? p.sx[gm] : 0.f;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int gn = n0 + wn * (BN / WN) + j * 32 + 8 * g + 4 * half;
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

template <int BM, int BN, int WM, int WN, int OCC, int PGR, bool XCD_REMAP, int GROUP_M>
int launch_cfg(const GemmArgs& p, bool bias, bool gelu, hipStream_t stream) {
  const int64_t tiles = ((static_cast<int64_t>(p.M) + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int64_t grid = XCD_REMAP ? (tiles + NUM_XCD - 1) / NUM_XCD * NUM_XCD : tiles;
  const dim3 g(static_cast<uint32_t>(grid)), b(WM * WN * 64);
  if (bias && gelu)
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WM, WN, OCC, PGR, XCD_REMAP, GROUP_M, true, true>), g, b, 0, stream, p);
  else if (bias)
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WM, WN, OCC, PGR, XCD_REMAP, GROUP_M, true, false>), g, b, 0, stream, p);
  else if (gelu)
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WM, WN, OCC, PGR, XCD_REMAP, GROUP_M, false, true>), g, b, 0, stream, p);
  else
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WM, WN, OCC, PGR, XCD_REMAP, GROUP_M, false, false>), g, b, 0, stream, p);
  return check_launch("wf_gemm_i8");
}

GemmArgs make_args(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out) {
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
  return p;
}

}  // namespace

int launch_gemm_i8(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int gelu,
                   hipStream_t stream) {
  const GemmArgs p = make_args(a, w, M, N, K, sx, sw, bias, y, ldy, acc_out);
  // 128 x 256 tiles, 2 x 4 waves of 64 x 64, two workgroups per CU, loads
  // two K steps ahead, XCD-contiguous grouped order (bands of 8 tile rows):
  // the best of a sweep over tile shape, waves, occupancy, prefetch depth and
  // rasterization on the Wan-1.3B/14B linear shapes.
  return launch_cfg<128, 256, 2, 4, 2, 2, true, 8>(p, bias != nullptr, gelu != 0, stream);
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
  WF_REQUIRE((m + 256) * k < (1ll << 31) - 16 && (n + 256) * k < (1ll << 31) - 16, WF_E_SHAPE,
             "%s: operands of 2 GiB or more are not supported", fn);
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
  WF_REQUIRE((m + 256) * k < (1ll << 31) - 16 && (n + 256) * k < (1ll << 31) - 16, WF_E_SHAPE,
             "%s: operands of 2 GiB or more are not supported", fn);
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
