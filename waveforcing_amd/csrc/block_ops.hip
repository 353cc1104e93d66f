// Row-wise kernels of the Wan attention block around the quantized linears
// and the attention (naive_rt/rolling_forcing/wan/modules/causal_model.py:
// 349-402, model.py:70-99), following the reference's dtypes: the block runs
// in bf16, norms compute in fp32 and round to bf16, and every bf16 operation
// of the modulation and the gated residuals rounds to bf16.
//
// One wave per token row (dim up to 5120 = 10 chunks of 8 per lane held in
// registers), 4 rows per 256-thread workgroup, no LDS: row reductions are
// wave64 butterflies.
#include "wf_common.hpp"

namespace wf {
namespace {

constexpr int kRows = 4;       // rows (waves) per workgroup
constexpr int kMaxChunks = 10; // 8-element chunks per lane: dim <= 5120

__device__ inline float wave_sum(float v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ inline float wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ inline float rbf(float f) { return bf16_bits_to_f32(f32_to_bf16_rne(f)); }

__device__ inline void unpack8(const uint4& w, float* f) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo_to_f32(u[i]);
    f[2 * i + 1] = bf16_hi_to_f32(u[i]);
  }
}
__device__ inline uint4 pack8(const float* f) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    u[i] = static_cast<uint32_t>(f32_to_bf16_rne(f[2 * i])) |
           (static_cast<uint32_t>(f32_to_bf16_rne(f[2 * i + 1])) << 16);
  return make_uint4(u[0], u[1], u[2], u[3]);
}

// int8 code of x with scale s (reciprocal r): round_half_even(RN(x / s)),
// as in the per-row quantization kernel.
__device__ inline int quant_i8(float x, float s, float r) {
  const float ax = fabsf(x);
  float q = ax * r;
  q = fmaf(fmaf(-q, s, ax), r, q);
  const float k = rintf(q);
  if (fabsf(fabsf(q - k) - 0.5f) <= q * 1.1920929e-7f) q = __fdiv_rn(ax, s);
  float qi = fminf(rintf(q), 127.0f);
  return static_cast<int>(x < 0.f ? -qi : qi);
}

struct LnArgs {
  const uint16_t* x;     // bf16 [T, ldx]
  int64_t ldx;
  int T, dim;
  float eps;
  const uint16_t* w;     // LayerNorm affine weight bf16 [dim] or null
  const uint16_t* b;     // affine bias bf16 [dim] or null
  const uint16_t* shift; // modulation shift e_a bf16 [F, dim] or null
  const uint16_t* scale; // modulation scale e_b bf16 [F, dim] (applied as 1 + e_b) or null
  int frame_tokens;      // tokens per frame (row t uses modulation row t / frame_tokens)
  uint16_t* out;         // bf16 [T, ldo] or null
  int64_t ldo;
  int8_t* q;             // int8 [T, dim] or null
  float* qs;             // fp32 [T] (with q)
};

// y = LN(x) [* w + b]  (fp32, rounded to bf16: WanLayerNorm, model.py:89-99)
// y = bf16(bf16(y * bf16(1 + e_b)) + e_a)   (causal_model.py:381,393-394)
// optional bf16 output and per-token int8 quantization of y.
__global__ __launch_bounds__(256) void ln_mod_quant_kernel(LnArgs a) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kRows + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const int n_chunks = a.dim / 8;
  const uint16_t* row = a.x + static_cast<int64_t>(t) * a.ldx;
  float v[kMaxChunks][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch < n_chunks) {
      unpack8(*reinterpret_cast<const uint4*>(row + ch * 8), v[c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += v[c][i];
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(a.dim);
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (lane + 64 * c < n_chunks) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[c][i] - mean;
        sq += d * d;
      }
    }
  }
  const float var = wave_sum(sq) / static_cast<float>(a.dim);
  const float rstd = 1.0f / sqrtf(var + a.eps);
  const int f = t / a.frame_tokens;
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch < n_chunks) {
      float wv[8], bv[8], sh[8], sc[8];
      if (a.w) unpack8(*reinterpret_cast<const uint4*>(a.w + ch * 8), wv);
      if (a.b) unpack8(*reinterpret_cast<const uint4*>(a.b + ch * 8), bv);
      if (a.shift) unpack8(*reinterpret_cast<const uint4*>(a.shift + static_cast<int64_t>(f) * a.dim + ch * 8), sh);
      if (a.scale) unpack8(*reinterpret_cast<const uint4*>(a.scale + static_cast<int64_t>(f) * a.dim + ch * 8), sc);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float y = (v[c][i] - mean) * rstd;
        if (a.w) y = y * wv[i];
        if (a.b) y = y + bv[i];
        y = rbf(y);
        if (a.scale) y = rbf(y * rbf(1.0f + sc[i]));
        if (a.shift) y = rbf(y + sh[i]);
        v[c][i] = y;
        amax = fmaxf(amax, fabsf(y));
      }
      if (a.out) *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(t) * a.ldo + ch * 8) = pack8(v[c]);
    }
  }
  if (a.q) {
    amax = wave_max(amax);
    const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
    const float r = __frcp_rn(s);
    if (lane == 0) a.qs[t] = s;
    int8_t* qrow = a.q + static_cast<int64_t>(t) * a.dim;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      const int ch = lane + 64 * c;
      if (ch < n_chunks) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lo |= (static_cast<uint32_t>(quant_i8(v[c][i], s, r)) & 0xffu) << (8 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) hi |= (static_cast<uint32_t>(quant_i8(v[c][4 + i], s, r)) & 0xffu) << (8 * i);
        *reinterpret_cast<uint2*>(qrow + ch * 8) = make_uint2(lo, hi);
      }
    }
  }
}

struct RmsArgs {
  const uint16_t* x;  // bf16 [T, ldx]
  int64_t ldx;
  int T, dim, head_dim;
  float eps;
  const uint16_t* w;  // RMSNorm weight bf16 [dim]
  const float* cos;   // [T, head_dim / 2] fp32 or null (no rotation)
  const float* sin;
  uint16_t* out;      // bf16 [T, ldo]
  int64_t ldo;
};

// y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)         (WanRMSNorm, model.py:78-86)
// then, per head, pairs (y[2i], y[2i+1]) rotated by the token's angle i:
// (a cos - b sin, a sin + b cos) in fp32, rounded to bf16 (is_neox_style=False,
// backend.py:119-121; causal_rope_apply, causal_model.py:27-55).
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(RmsArgs a) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kRows + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const int n_chunks = a.dim / 8;
  const uint16_t* row = a.x + static_cast<int64_t>(t) * a.ldx;
  float v[kMaxChunks][8];
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch < n_chunks) {
      unpack8(*reinterpret_cast<const uint4*>(row + ch * 8), v[c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) sq += v[c][i] * v[c][i];
    }
  }
  const float ms = wave_sum(sq) / static_cast<float>(a.dim);
  const float rn = 1.0f / sqrtf(ms + a.eps);
  const int half = a.head_dim / 2;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch < n_chunks) {
      float wv[8];
      unpack8(*reinterpret_cast<const uint4*>(a.w + ch * 8), wv);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = rbf(rbf(v[c][i] * rn) * wv[i]);
      if (a.cos) {
        // element e = ch * 8 + i; pair index within the head: (e % head_dim) / 2
        const int p0 = ((ch * 8) % a.head_dim) / 2;
        const float4 c4 = *reinterpret_cast<const float4*>(a.cos + static_cast<int64_t>(t) * half + p0);
        const float4 s4 = *reinterpret_cast<const float4*>(a.sin + static_cast<int64_t>(t) * half + p0);
        const float cs[4] = {c4.x, c4.y, c4.z, c4.w};
        const float sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x0 = y[2 * j], x1 = y[2 * j + 1];
          y[2 * j] = x0 * cs[j] - x1 * sn[j];
          y[2 * j + 1] = x0 * sn[j] + x1 * cs[j];
        }
      }
      *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(t) * a.ldo + ch * 8) = pack8(y);
    }
  }
}

// x = bf16(x + bf16(y * gate[t / frame_tokens]))   (causal_model.py:386,397-398)
// or x = bf16(x + y) without a gate (cross-attention residual, :390).
__global__ __launch_bounds__(256) void gate_residual_kernel(uint16_t* __restrict__ x, int64_t ldx,
                                                            const uint16_t* __restrict__ y, int64_t ldy,
                                                            const uint16_t* __restrict__ gate, int T, int dim,
                                                            int frame_tokens) {
  const int n_chunks = dim / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(T) * n_chunks) return;
  const int t = static_cast<int>(idx / n_chunks);
  const int ch = static_cast<int>(idx % n_chunks);
  float xv[8], yv[8], g[8];
  uint4* xp = reinterpret_cast<uint4*>(x + static_cast<int64_t>(t) * ldx + ch * 8);
  unpack8(*xp, xv);
  unpack8(*reinterpret_cast<const uint4*>(y + static_cast<int64_t>(t) * ldy + ch * 8), yv);
  if (gate) {
    unpack8(*reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(t / frame_tokens) * dim + ch * 8), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = rbf(xv[i] + rbf(yv[i] * g[i]));
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = rbf(xv[i] + yv[i]);
  }
  *xp = pack8(xv);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wf

extern "C" {

int wf_ln_modulate_quant(const void* x, int64_t T, int32_t dim, int64_t ldx, float eps, const void* w, const void* b,
                         const void* shift, const void* scale, int32_t frame_tokens, void* out, int64_t ldo,
                         int8_t* q, float* q_scales, void* stream) {
  static const char* fn = "wf_ln_modulate_quant";
  WF_REQUIRE(T >= 0 && dim > 0 && ldx >= dim && frame_tokens > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(dim % 8 == 0 && dim <= 64 * 8 * wf::kMaxChunks, WF_E_SHAPE, "%s: dim=%d (need %% 8 == 0, <= 5120)", fn,
             dim);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && (out || q), WF_E_INVALID, "%s: null input or no output", fn);
  WF_REQUIRE(!q || q_scales, WF_E_INVALID, "%s: q without q_scales", fn);
  WF_REQUIRE(!out || ldo >= dim, WF_E_INVALID, "%s: ldo < dim", fn);
  WF_REQUIRE(wf::a16(x) && ldx % 8 == 0 && (!out || (wf::a16(out) && ldo % 8 == 0)) && (!q || (reinterpret_cast<uintptr_t>(q) & 7u) == 0) &&
                 (!w || wf::a16(w)) && (!b || wf::a16(b)) && (!shift || wf::a16(shift)) && (!scale || wf::a16(scale)),
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  wf::LnArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<int>(T), dim, eps,
               static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
               static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), frame_tokens,
               static_cast<uint16_t*>(out), ldo, q, q_scales};
  hipLaunchKernelGGL(wf::ln_mod_quant_kernel, dim3(static_cast<uint32_t>((T + wf::kRows - 1) / wf::kRows)),
                     dim3(256), 0, wf::as_stream(stream), a);
  return wf::check_launch(fn);
}

int wf_rmsnorm_rope(const void* x, int64_t T, int32_t dim, int64_t ldx, int32_t head_dim, float eps, const void* w,
                    const float* cos, const float* sin, void* out, int64_t ldo, void* stream) {
  static const char* fn = "wf_rmsnorm_rope";
  WF_REQUIRE(T >= 0 && dim > 0 && head_dim > 0 && ldx >= dim && ldo >= dim, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(dim % 8 == 0 && dim <= 64 * 8 * wf::kMaxChunks && dim % head_dim == 0 && head_dim % 8 == 0, WF_E_SHAPE,
             "%s: dim=%d head_dim=%d unsupported", fn, dim, head_dim);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && w && out && ((cos == nullptr) == (sin == nullptr)), WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(wf::a16(x) && wf::a16(w) && wf::a16(out) && ldx % 8 == 0 && ldo % 8 == 0 && (!cos || (wf::a16(cos) && wf::a16(sin))),
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  wf::RmsArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<int>(T), dim, head_dim, eps,
                static_cast<const uint16_t*>(w), cos, sin, static_cast<uint16_t*>(out), ldo};
  hipLaunchKernelGGL(wf::rmsnorm_rope_kernel, dim3(static_cast<uint32_t>((T + wf::kRows - 1) / wf::kRows)),
                     dim3(256), 0, wf::as_stream(stream), a);
  return wf::check_launch(fn);
}

int wf_gate_residual(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, int64_t T, int32_t dim,
                     int32_t frame_tokens, void* stream) {
  static const char* fn = "wf_gate_residual";
  WF_REQUIRE(T >= 0 && dim > 0 && ldx >= dim && ldy >= dim && frame_tokens > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(dim % 8 == 0, WF_E_SHAPE, "%s: dim %% 8 != 0", fn);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(wf::a16(x) && wf::a16(y) && (!gate || wf::a16(gate)) && ldx % 8 == 0 && ldy % 8 == 0, WF_E_ALIGN,
             "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  const int64_t n = T * (dim / 8);
  hipLaunchKernelGGL(wf::gate_residual_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                     wf::as_stream(stream), static_cast<uint16_t*>(x), ldx, static_cast<const uint16_t*>(y), ldy,
                     static_cast<const uint16_t*>(gate), static_cast<int>(T), dim, frame_tokens);
  return wf::check_launch(fn);
}

}  // extern "C"
