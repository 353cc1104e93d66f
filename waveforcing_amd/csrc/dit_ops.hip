// The Wan DiT's layers around the quantized blocks, in bf16 as the reference
// runs them (its W8A8 swap replaces only the blocks' linears,
// wave_rt/runtime/fp8.py:93-137):
//
//  * a bf16 GEMM on the matrix cores for the patch embedding, the text and
//    time embeddings, the time projection and the output head
//    (naive_rt/rolling_forcing/wan/modules/causal_model.py:517-528,406-433):
//      y[m,n] = act_out( bf16( sum_k act_in(a[m,k]) * w[n,k] + bias[n] ) )
//    with fp32 accumulation; act_in = SiLU (the time projection's
//    nn.SiLU() before its Linear), act_out = SiLU or GELU(tanh), each
//    applied to a bf16 value and rounded to bf16 as torch's bf16 modules do;
//  * the patch gather of the Conv3d patch embedding (kernel = stride =
//    (1, 2, 2)): token (f, y, x) takes the 2 x 2 patch of every channel in
//    the weight's (c, kh, kw) order, so the embedding is that GEMM;
//  * unpatchify (causal_model.py:1080-1103: 'fhwpqrc->cfphqwr') fused with
//    the flow-matching x0 conversion of wan_wrapper.py:169-193,
//    x0 = xt - sigma * flow in float64, written in the (B, T, C, H, W)
//    layout the wavefront hands on (backend.py:456-490), converted to bf16
//    as torch converts float64 (through float32).
//
// GEMM structure: a workgroup of 4 waves owns a 64 x 128 output tile, each
// wave 32 rows x 64 columns as two v_mfma_f32_32x32x16_bf16 blocks.  The
// operand fragments of that MFMA are 16 contiguous bytes of one row of A
// and of W (lane l: row l % 32, K elements 8 (l / 32) .. + 7), so they are
// loaded straight from global memory (neighbouring K steps share cache
// lines), one K step ahead of the MFMAs.  Each wave's results go out through
// its own LDS rows as 128-byte row segments.  These GEMMs are a few percent
// of a chunk's work (0.9 GFLOP for the patch embedding or the head at 1.3B).
#include <type_traits>

#include "wf_common.hpp"

namespace wf {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kTileM = 64, kTileN = 128;

// x * sigmoid(x) = x / (1 + e^-x), on the hardware exponential and reciprocal.
__device__ inline float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

__device__ inline float bf16_round(float x) { return __uint_as_float(pack_bf16x2_hw(x, 0.f) << 16); }

template <bool SILU_IN>
__device__ inline v8bf load_frag(const uint16_t* row, int k, int K) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (k < K) v = *reinterpret_cast<const uint4*>(row + k);
  if constexpr (SILU_IN) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = pack_bf16x2_hw(silu(bf16_lo_to_f32(w[i])), silu(bf16_hi_to_f32(w[i])));
    v = make_uint4(o[0], o[1], o[2], o[3]);
  }
  return __builtin_bit_cast(v8bf, v);
}

struct Bf16GemmArgs {
  const uint16_t* a;
  const uint16_t* w;
  const uint16_t* bias;
  uint16_t* y;
  int64_t lda, ldy;
  int M, N, K;
};

// ACT_OUT: 0 none, 1 SiLU, 2 GELU(tanh).
template <bool SILU_IN, int ACT_OUT>
__global__ __launch_bounds__(kWaves * 64) void gemm_bf16_kernel(Bf16GemmArgs p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const int m0 = blockIdx.y * kTileM + (wave >> 1) * 32;
  const int n0 = blockIdx.x * kTileN + (wave & 1) * 64;
  // rows past M / N read a clamped row (their results are not stored)
  const uint16_t* arow = p.a + static_cast<int64_t>(min(m0 + l32, p.M - 1)) * p.lda;
  const uint16_t* wrow0 = p.w + static_cast<int64_t>(min(n0 + l32, p.N - 1)) * p.K;
  const uint16_t* wrow1 = p.w + static_cast<int64_t>(min(n0 + 32 + l32, p.N - 1)) * p.K;
  v16f acc0 = {}, acc1 = {};
  const int kh = 8 * half;
  v8bf a = load_frag<SILU_IN>(arow, kh, p.K);
  v8bf w0 = load_frag<false>(wrow0, kh, p.K);
  v8bf w1 = load_frag<false>(wrow1, kh, p.K);
  for (int k = 16; k < p.K + 16; k += 16) {
    // the next step's fragments load under this step's MFMAs (zeros past K)
    const v8bf an = load_frag<SILU_IN>(arow, k + kh, p.K);
    const v8bf w0n = load_frag<false>(wrow0, k + kh, p.K);
    const v8bf w1n = load_frag<false>(wrow1, k + kh, p.K);
    acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, a, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, a, acc1, 0, 0, 0);
    a = an;
    w0 = w0n;
    w1 = w1n;
  }
  // lane's row m0 + l32; register r of block j is column n0 + 32 j + 8 (r / 4) + 4 half + r % 4.  The
  // wave's 32 x 64 results go through its own LDS rows, so each row is stored as one 128-byte segment.
  constexpr int YP = 64 * 2 + 8;  // staged row pitch (bytes)
  __shared__ __attribute__((aligned(16))) uint8_t ys[kWaves * 32 * YP];
  uint8_t* yw = ys + wave * 32 * YP;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const v16f& acc = j == 0 ? acc0 : acc1;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + 32 * j + 8 * g + 4 * half;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = acc[4 * g + e];
        if (p.bias && n < p.N) t = __fadd_rn(t, bf16_bits_to_f32(p.bias[n + e]));
        t = bf16_round(t);
        if constexpr (ACT_OUT == 1) t = silu(t);
        if constexpr (ACT_OUT == 2) t = gelu_tanh(t);
        v[e] = t;
      }
      *reinterpret_cast<uint2*>(yw + l32 * YP + 2 * (32 * j + 8 * g + 4 * half)) =
          make_uint2(pack_bf16x2_hw(v[0], v[1]), pack_bf16x2_hw(v[2], v[3]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + (lane >> 4);
    const int m = m0 + row, n = n0 + 4 * (lane & 15);
    const uint2 w = *reinterpret_cast<const uint2*>(yw + row * YP + 8 * (lane & 15));
    if (m < p.M && n < p.N) *reinterpret_cast<uint2*>(p.y + static_cast<int64_t>(m) * p.ldy + n) = w;
  }
}

// Patch gather: out[b][t][c * 4 + kh * 2 + kw] = x[b][c][f][2 y + kh][2 x + kw], token t = (f, y, x).
// One thread per (b, t, c): 4 values, one 8-byte store.
__global__ __launch_bounds__(256) void patchify_kernel(const uint16_t* __restrict__ x, int64_t B, int C, int F, int H,
                                                       int W, uint16_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int hp = H / 2, wp = W / 2;
  const int64_t tokens = static_cast<int64_t>(F) * hp * wp;
  if (i >= B * tokens * C) return;
  const int c = static_cast<int>(i % C);
  const int64_t bt = i / C;
  const int64_t t = bt % tokens;
  const int64_t b = bt / tokens;
  const int xw = static_cast<int>(t % wp), yh = static_cast<int>((t / wp) % hp), f = static_cast<int>(t / (wp * hp));
  const uint16_t* src = x + (((b * C + c) * F + f) * H + 2 * yh) * static_cast<int64_t>(W) + 2 * xw;
  const uint32_t top = *reinterpret_cast<const uint32_t*>(src);
  const uint32_t bot = *reinterpret_cast<const uint32_t*>(src + W);
  *reinterpret_cast<uint2*>(out + (b * tokens + t) * (4 * C) + 4 * c) = make_uint2(top, bot);
}

// float64 -> bf16 as torch converts it: to float32 (round to nearest even), then to bf16.
__device__ inline uint16_t f64_to_bf16_via_f32(double d) { return f32_to_bf16_rne(static_cast<float>(d)); }

// x0[b][f][c][y][x] = bf16(xt[b][c][f][y][x] - sigma * flow[b][c][f][y][x]) in float64, with flow the
// unpatchified head output: flow[b][c][f][2 y' + q][2 x' + r] = head[b][t(f, y', x')][(2 q + r) * C + c].
// One thread per (b, f, c, y, x pair): two outputs.
__global__ __launch_bounds__(256) void unpatchify_x0_kernel(const uint16_t* __restrict__ head,
                                                            const uint16_t* __restrict__ xt, int64_t B, int C, int F,
                                                            int H, int W, double sigma, uint16_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int wh = W / 2;
  const int64_t total = B * F * static_cast<int64_t>(C) * H * wh;
  if (i >= total) return;
  const int xp = static_cast<int>(i % wh);
  int64_t r = i / wh;
  const int yy = static_cast<int>(r % H);
  r /= H;
  const int c = static_cast<int>(r % C);
  r /= C;
  const int f = static_cast<int>(r % F);
  const int64_t b = r / F;
  const int hp = H / 2;
  const int64_t t = (static_cast<int64_t>(f) * hp + yy / 2) * wh + xp;
  const int q = yy & 1;
  const uint16_t* hrow = head + (b * (static_cast<int64_t>(F) * hp * wh) + t) * (4 * C);
  const uint16_t fl0 = hrow[(2 * q + 0) * C + c];
  const uint16_t fl1 = hrow[(2 * q + 1) * C + c];
  const uint32_t xv = *reinterpret_cast<const uint32_t*>(xt + (((b * C + c) * F + f) * H + yy) * static_cast<int64_t>(W) +
                                                         2 * xp);
  const double x0a = static_cast<double>(bf16_lo_to_f32(xv)) - sigma * static_cast<double>(bf16_bits_to_f32(fl0));
  const double x0b = static_cast<double>(bf16_hi_to_f32(xv)) - sigma * static_cast<double>(bf16_bits_to_f32(fl1));
  const uint32_t o = static_cast<uint32_t>(f64_to_bf16_via_f32(x0a)) |
                     (static_cast<uint32_t>(f64_to_bf16_via_f32(x0b)) << 16);
  *reinterpret_cast<uint32_t*>(out + (((b * F + f) * C + c) * H + yy) * static_cast<int64_t>(W) + 2 * xp) = o;
}

template <bool SILU_IN, int ACT>
void launch_gemm(const Bf16GemmArgs& p, hipStream_t st) {
  const dim3 grid((p.N + kTileN - 1) / kTileN, (p.M + kTileM - 1) / kTileM);
  hipLaunchKernelGGL((gemm_bf16_kernel<SILU_IN, ACT>), grid, dim3(kWaves * 64), 0, st, p);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wf

extern "C" {

int wf_gemm_bf16(const void* a, int64_t m, int64_t k, int64_t lda, const void* w, int64_t n, const void* bias,
                 void* y, int64_t ldy, int32_t flags, void* stream) {
  static const char* fn = "wf_gemm_bf16";
  WF_REQUIRE(m >= 0 && n >= 0 && k > 0 && lda >= k && ldy >= n, WF_E_INVALID,
             "%s: bad sizes m=%lld n=%lld k=%lld lda=%lld ldy=%lld", fn, (long long)m, (long long)n, (long long)k,
             (long long)lda, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(a && w && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(m < (1 << 30) && n < (1 << 30) && k < (1 << 30), WF_E_SHAPE, "%s: size too large", fn);
  WF_REQUIRE(k % 8 == 0 && lda % 8 == 0 && n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE,
             "%s: k and lda must be multiples of 8, n and ldy of 4", fn);
  WF_REQUIRE(wf::a16(a) && wf::a16(w) && (reinterpret_cast<uintptr_t>(y) & 7u) == 0 &&
                 (reinterpret_cast<uintptr_t>(bias) & 1u) == 0,
             WF_E_ALIGN, "%s: a and w must be 16-byte, y 8-byte aligned", fn);
  const int act = (flags & WF_BF16_SILU_OUT) ? 1 : (flags & WF_BF16_GELU_OUT) ? 2 : 0;
  WF_REQUIRE((flags & ~(WF_BF16_SILU_IN | WF_BF16_SILU_OUT | WF_BF16_GELU_OUT)) == 0 &&
                 !((flags & WF_BF16_SILU_OUT) && (flags & WF_BF16_GELU_OUT)),
             WF_E_INVALID, "%s: bad flags 0x%x", fn, flags);
  wf::Bf16GemmArgs p;
  p.a = static_cast<const uint16_t*>(a);
  p.w = static_cast<const uint16_t*>(w);
  p.bias = static_cast<const uint16_t*>(bias);
  p.y = static_cast<uint16_t*>(y);
  p.lda = lda;
  p.ldy = ldy;
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  hipStream_t st = wf::as_stream(stream);
  const bool silu_in = (flags & WF_BF16_SILU_IN) != 0;
  if (silu_in) {
    if (act == 0) wf::launch_gemm<true, 0>(p, st);
    else if (act == 1) wf::launch_gemm<true, 1>(p, st);
    else wf::launch_gemm<true, 2>(p, st);
  } else {
    if (act == 0) wf::launch_gemm<false, 0>(p, st);
    else if (act == 1) wf::launch_gemm<false, 1>(p, st);
    else wf::launch_gemm<false, 2>(p, st);
  }
  return wf::check_launch(fn);
}

int wf_patchify_bf16(const void* x, int64_t b, int32_t c, int32_t f, int32_t h, int32_t w, void* out, void* stream) {
  static const char* fn = "wf_patchify_bf16";
  WF_REQUIRE(b >= 0 && c > 0 && f > 0 && h > 0 && w > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(h % 2 == 0 && w % 2 == 0, WF_E_SHAPE, "%s: h=%d and w=%d must be even (2 x 2 patches)", fn, h, w);
  if (b == 0) return WF_OK;
  WF_REQUIRE(x && out, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 3u) == 0 && (reinterpret_cast<uintptr_t>(out) & 7u) == 0, WF_E_ALIGN,
             "%s: x must be 4-byte and out 8-byte aligned", fn);
  // one thread per item: a launch holds fewer than 2^32 threads
  WF_REQUIRE(wf::product_below({b, f, h / 2, w / 2, c}, (1ll << 32) - 256), WF_E_SHAPE,
             "%s: b*f*(h/2)*(w/2)*c must stay below 2^32 - 256", fn);
  const int64_t items = b * static_cast<int64_t>(f) * (h / 2) * (w / 2) * c;
  hipLaunchKernelGGL(wf::patchify_kernel, dim3(static_cast<uint32_t>((items + 255) / 256)), dim3(256), 0,
                     wf::as_stream(stream), static_cast<const uint16_t*>(x), b, c, f, h, w,
                     static_cast<uint16_t*>(out));
  return wf::check_launch(fn);
}

int wf_unpatchify_flow_x0_bf16(const void* head, const void* xt, int64_t b, int32_t c, int32_t f, int32_t h,
                               int32_t w, double sigma, void* x0, void* stream) {
  static const char* fn = "wf_unpatchify_flow_x0_bf16";
  WF_REQUIRE(b >= 0 && c > 0 && f > 0 && h > 0 && w > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(h % 2 == 0 && w % 2 == 0, WF_E_SHAPE, "%s: h=%d and w=%d must be even (2 x 2 patches)", fn, h, w);
  if (b == 0) return WF_OK;
  WF_REQUIRE(head && xt && x0, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(xt) & 3u) == 0 && (reinterpret_cast<uintptr_t>(x0) & 3u) == 0 &&
                 (reinterpret_cast<uintptr_t>(head) & 1u) == 0,
             WF_E_ALIGN, "%s: xt and x0 must be 4-byte aligned", fn);
  // one thread per item: a launch holds fewer than 2^32 threads
  WF_REQUIRE(wf::product_below({b, f, c, h, w / 2}, (1ll << 32) - 256), WF_E_SHAPE,
             "%s: b*f*c*h*(w/2) must stay below 2^32 - 256", fn);
  const int64_t items = b * static_cast<int64_t>(f) * c * h * (w / 2);
  hipLaunchKernelGGL(wf::unpatchify_x0_kernel, dim3(static_cast<uint32_t>((items + 255) / 256)), dim3(256), 0,
                     wf::as_stream(stream), static_cast<const uint16_t*>(head), static_cast<const uint16_t*>(xt), b, c,
                     f, h, w, sigma, static_cast<uint16_t*>(x0));
  return wf::check_launch(fn);
}

}  // extern "C"
