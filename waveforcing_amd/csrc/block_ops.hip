// Row-wise kernels of the Wan attention block around the quantized linears
// and the attention (naive_rt/rolling_forcing/wan/modules/causal_model.py:
// 349-402, model.py:70-99), following the reference's dtypes: the block runs
// in bf16, norms compute in fp32 and round to bf16, and every bf16 operation
// of the modulation and the gated residuals rounds to bf16.
//
// The norm kernels run on the row engine of rows.hpp: a token row is owned
// by one wave (dim <= 2048) or one 256-thread workgroup (dim <= 16384), with
// NC chunks of 8 values per lane fixed at compile time, so a row stays in
// registers and all of its loads are issued before the first reduction.
#include "rows.hpp"

namespace wf {
namespace {

using namespace rows;

struct LnArgs {
  uint16_t* x;             // bf16 [T, ldx]; updated in place when ry != null
  int64_t ldx;
  const uint16_t* ry;      // residual addend bf16 [T, ldry] or null
  int64_t ldry;
  const uint16_t* rgate;   // residual gate bf16 [frames, ld_rgate] or null
  int64_t ld_rgate;
  int T, dim;
  float eps;
  const uint16_t* w;       // LayerNorm affine weight bf16 [dim] or null
  const uint16_t* b;       // affine bias bf16 [dim] or null
  const uint16_t* shift;   // modulation shift e_a bf16 [frames, ld_mod] or null
  const uint16_t* scale;   // modulation scale e_b bf16 [frames, ld_mod] (as 1 + e_b) or null
  int64_t ld_mod;
  int frame_tokens;        // row t uses frame row t / frame_tokens
  uint16_t* out;           // bf16 [T, ldo] or null
  int64_t ldo;
  int8_t* q;               // int8 [T, dim] or null
  float* qs;               // fp32 [T] (with q)
};

// Which operands a launch has.  Form 0 reads that from the null-ness of LnArgs' pointers at run time
// (every combination); the others fix it at compile time for the block's norms, so their kernels carry
// no branches on it (the same operations in the same order: bit-identical to form 0).
struct LnForm {
  int res;    // 0: no residual, 1: x + y, 2: x + y * gate
  bool mod;   // shift and scale modulation
  bool aff;   // affine weight and bias
  bool out;   // bf16 output
  bool q;     // int8 output
};
constexpr LnForm kLnForms[] = {
    {0, false, false, false, false},  // 0: run-time
    {2, true, false, false, true},    // 1: LN1 after the previous block's gated residual, modulation, int8
    {0, true, false, false, true},    // 2: LN1 of a stack's first block
    {1, true, false, false, true},    // 3: cross-attention residual + LN2, modulation, int8
    {2, false, true, false, true},    // 4: self-attention gated residual + norm3 (affine), int8
};
constexpr int kNumLnForms = sizeof(kLnForms) / sizeof(kLnForms[0]);

// [x = bf16(x + bf16(ry * rgate[f]))  or  x = bf16(x + ry)]   (causal_model.py:386,390,397-398)
// y = LN(x) [* w + b]  (fp32 statistics, rounded to bf16: WanLayerNorm, model.py:89-99)
// y = bf16(bf16(y * bf16(1 + e_b)) + e_a)                     (causal_model.py:381,393-394)
// optional bf16 output and per-token int8 quantization of y.
template <int LPR, int NC, int FORM>
__global__ __launch_bounds__(256) void ln_mod_quant_kernel(LnArgs a) {
  constexpr int RPB = 256 / LPR;
  constexpr LnForm F = kLnForms[FORM];
  const bool has_ry = FORM ? F.res > 0 : a.ry != nullptr;
  const bool has_gate = FORM ? F.res == 2 : a.rgate != nullptr;
  const bool has_shift = FORM ? F.mod : a.shift != nullptr;
  const bool has_scale = FORM ? F.mod : a.scale != nullptr;
  const bool has_w = FORM ? F.aff : a.w != nullptr;
  const bool has_b = FORM ? F.aff : a.b != nullptr;
  const bool has_out = FORM ? F.out : a.out != nullptr;
  const bool has_q = FORM ? F.q : a.q != nullptr;
  __shared__ float red[3][4];
  const int lane = static_cast<int>(threadIdx.x) % LPR;
  const int t = static_cast<int>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / LPR;
  if (t >= a.T) return;  // uniform per row (a wave, or the workgroup for LPR = 256)
  const int n_chunks = a.dim >> 3;
  const int f = t / a.frame_tokens;
  uint16_t* row = a.x + static_cast<int64_t>(t) * a.ldx;

  // The row is kept as packed bf16 (4 registers per chunk) and unpacked in
  // each pass; the affine and modulation rows are fetched with the row, so
  // every load is in flight before the first reduction.
  const bool mod = has_shift || has_scale;
  uint4 xr[NC], pa[NC], pb[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    const bool ok = ch < n_chunks;
    const uint4 z = make_uint4(0, 0, 0, 0);
    xr[c] = ok ? ld16(row + ch * 8) : z;
    if (has_ry) {
      uint4 yr = ok ? ld16(a.ry + static_cast<int64_t>(t) * a.ldry + ch * 8) : z;
      uint4 gr = has_gate && ok ? ld16(a.rgate + static_cast<int64_t>(f) * a.ld_rgate + ch * 8) : z;
      // residual, applied as soon as its operands arrive
      float v[8], y[8];
      unpack8(xr[c], v);
      unpack8(yr, y);
      if (has_gate) {
        float g[8];
        unpack8(gr, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = y[i] * g[i];
        rbf8(y);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = v[i] + y[i];
      xr[c] = pack8(v);
      if (ok) st16(row + ch * 8, xr[c]);
    }
    // pa/pb: (shift, scale) of the modulation if there is one, else the affine (w, b)
    if (mod) {
      if (has_shift) pa[c] = ok ? ld16(a.shift + static_cast<int64_t>(f) * a.ld_mod + ch * 8) : z;
      if (has_scale) pb[c] = ok ? ld16(a.scale + static_cast<int64_t>(f) * a.ld_mod + ch * 8) : z;
    } else {
      if (has_w) pa[c] = ok ? ld16(a.w + ch * 8) : z;
      if (has_b) pb[c] = ok ? ld16(a.b + ch * 8) : z;
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float v[8];
    unpack8(xr[c], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) sum += v[i];
  }
  const float mean = row_sum<LPR>(sum, red[0]) / static_cast<float>(a.dim);
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (lane + LPR * c < n_chunks) {
      float v[8];
      unpack8(xr[c], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[i] - mean;
        sq += d * d;
      }
    }
  }
  const float var = row_sum<LPR>(sq, red[1]) / static_cast<float>(a.dim);
  const float rstd = 1.0f / sqrtf(var + a.eps);
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    if (ch < n_chunks) {
      float v[8], y[8];
      unpack8(xr[c], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (v[i] - mean) * rstd;
      if (has_w) {
        float wv[8];
        unpack8(mod ? ld16(a.w + ch * 8) : pa[c], wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = y[i] * wv[i];
      }
      if (has_b) {
        float bv[8];
        unpack8(mod ? ld16(a.b + ch * 8) : pb[c], bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = y[i] + bv[i];
      }
      rbf8(y);
      if (has_scale) {
        float sc[8];
        unpack8(pb[c], sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = 1.0f + sc[i];
        rbf8(sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = y[i] * sc[i];
        rbf8(y);
      }
      if (has_shift) {
        float sh[8];
        unpack8(pa[c], sh);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = y[i] + sh[i];
        rbf8(y);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(y[i]));
      xr[c] = pack8(y);
      if (has_out) st16(a.out + static_cast<int64_t>(t) * a.ldo + ch * 8, xr[c]);
    }
  }
  if (has_q) {
    amax = row_max_nonneg<LPR>(amax, red[2]);
    const float s = i8_scale(amax);
    const double rd = i8_recip(s);
    if (lane == 0) a.qs[t] = s;
    int8_t* qrow = a.q + static_cast<int64_t>(t) * a.dim;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + LPR * c;
      if (ch < n_chunks) {
        float y[8];
        unpack8(xr[c], y);
        *reinterpret_cast<uint2*>(qrow + ch * 8) = quant8_i8(y, rd);
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
// In place (out == x) is allowed: a row is read whole before it is written.
template <int LPR, int NC>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(RmsArgs a) {
  constexpr int RPB = 256 / LPR;
  __shared__ float red[4];
  const int lane = static_cast<int>(threadIdx.x) % LPR;
  const int t = static_cast<int>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / LPR;
  if (t >= a.T) return;
  const int n_chunks = a.dim >> 3;
  const uint16_t* row = a.x + static_cast<int64_t>(t) * a.ldx;
  float v[NC][8];
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    unpack8(ch < n_chunks ? ld16(row + ch * 8) : make_uint4(0, 0, 0, 0), v[c]);
#pragma unroll
    for (int i = 0; i < 8; ++i) sq += v[c][i] * v[c][i];
  }
  const float ms = row_sum<LPR>(sq, red) / static_cast<float>(a.dim);
  const float rn = 1.0f / sqrtf(ms + a.eps);
  const int half = a.head_dim / 2;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    if (ch < n_chunks) {
      float wv[8];
      unpack8(ld16(a.w + ch * 8), wv);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = v[c][i] * rn;
      rbf8(y);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = y[i] * wv[i];
      rbf8(y);
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
      st16(a.out + static_cast<int64_t>(t) * a.ldo + ch * 8, pack8(y));
    }
  }
}

// x = bf16(x + bf16(y * gate[t / frame_tokens]))   (causal_model.py:386,397-398)
// or x = bf16(x + y) without a gate (cross-attention residual, :390).
__global__ __launch_bounds__(256) void gate_residual_kernel(uint16_t* __restrict__ x, int64_t ldx,
                                                            const uint16_t* __restrict__ y, int64_t ldy,
                                                            const uint16_t* __restrict__ gate, int64_t ld_gate,
                                                            int T, int dim, int frame_tokens) {
  const int n_chunks = dim / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(T) * n_chunks) return;
  const int t = static_cast<int>(idx / n_chunks);
  const int ch = static_cast<int>(idx % n_chunks);
  float xv[8], yv[8], g[8];
  uint16_t* xp = x + static_cast<int64_t>(t) * ldx + ch * 8;
  unpack8(ld16(xp), xv);
  unpack8(ld16(y + static_cast<int64_t>(t) * ldy + ch * 8), yv);
  if (gate) {
    unpack8(ld16(gate + static_cast<int64_t>(t / frame_tokens) * ld_gate + ch * 8), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) yv[i] = yv[i] * g[i];
    rbf8(yv);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) xv[i] = xv[i] + yv[i];
  rbf8(xv);
  st16(xp, pack8(xv));
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_ln(const LnArgs& a, hipStream_t stream, const char* fn) {
  int lpr = 0, nc = 0;
  pick_shape(a.dim / 8, lpr, nc);
  const uint32_t grid = static_cast<uint32_t>((a.T + 256 / lpr - 1) / (256 / lpr));
  const LnForm have{a.ry ? (a.rgate ? 2 : 1) : 0, a.shift && a.scale, a.w && a.b, a.out != nullptr,
                    a.q != nullptr};
  const bool partial = (!a.shift != !a.scale) || (!a.w != !a.b) || (have.mod && have.aff);
  int form = 0;
  for (int i = 1; i < kNumLnForms && !partial; ++i) {
    const LnForm& f = kLnForms[i];
    if (f.res == have.res && f.mod == have.mod && f.aff == have.aff && f.out == have.out && f.q == have.q) form = i;
  }
  dispatch_shape(lpr, nc, [&](auto L, auto C) {
    constexpr int l = decltype(L)::value, c = decltype(C)::value;
    switch (form) {
      case 1: hipLaunchKernelGGL((ln_mod_quant_kernel<l, c, 1>), dim3(grid), dim3(256), 0, stream, a); break;
      case 2: hipLaunchKernelGGL((ln_mod_quant_kernel<l, c, 2>), dim3(grid), dim3(256), 0, stream, a); break;
      case 3: hipLaunchKernelGGL((ln_mod_quant_kernel<l, c, 3>), dim3(grid), dim3(256), 0, stream, a); break;
      case 4: hipLaunchKernelGGL((ln_mod_quant_kernel<l, c, 4>), dim3(grid), dim3(256), 0, stream, a); break;
      default: hipLaunchKernelGGL((ln_mod_quant_kernel<l, c, 0>), dim3(grid), dim3(256), 0, stream, a); break;
    }
  });
  static_assert(kNumLnForms == 5, "one launch case per form");
  return check_launch(fn);
}

}  // namespace
}  // namespace wf

extern "C" {

int wf_gate_residual_ln_quant(void* x, int64_t T, int32_t dim, int64_t ldx, const void* y, int64_t ldy,
                              const void* gate, int64_t ld_gate, float eps, const void* w, const void* b,
                              const void* shift, const void* scale, int64_t ld_mod, int32_t frame_tokens, void* out,
                              int64_t ldo, int8_t* q, float* q_scales, void* stream) {
  static const char* fn = "wf_gate_residual_ln_quant";
  WF_REQUIRE(T >= 0 && dim > 0 && ldx >= dim && frame_tokens > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(dim % 8 == 0 && dim <= 16384, WF_E_SHAPE, "%s: dim=%d (need %% 8 == 0, <= 16384)", fn, dim);
  WF_REQUIRE(T < (1ll << 24), WF_E_SHAPE, "%s: T=%lld too large (a launch holds at most 2^32 threads)", fn,
             (long long)T);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && (out || q), WF_E_INVALID, "%s: null input or no output", fn);
  WF_REQUIRE(!y || ldy >= dim, WF_E_INVALID, "%s: ldy < dim", fn);
  WF_REQUIRE(!gate || y, WF_E_INVALID, "%s: gate without y", fn);
  WF_REQUIRE(!gate || ld_gate >= dim, WF_E_INVALID, "%s: ld_gate < dim", fn);
  WF_REQUIRE(!(shift || scale) || ld_mod >= dim, WF_E_INVALID, "%s: ld_mod < dim", fn);
  WF_REQUIRE(!q || q_scales, WF_E_INVALID, "%s: q without q_scales", fn);
  WF_REQUIRE(!out || ldo >= dim, WF_E_INVALID, "%s: ldo < dim", fn);
  WF_REQUIRE(!out || !y || out != x, WF_E_INVALID, "%s: out must not alias x when a residual is applied", fn);
  WF_REQUIRE(wf::a16(x) && ldx % 8 == 0 && (!out || (wf::a16(out) && ldo % 8 == 0)) &&
                 (!y || (wf::a16(y) && ldy % 8 == 0)) && (!gate || (wf::a16(gate) && ld_gate % 8 == 0)) &&
                 (!q || (reinterpret_cast<uintptr_t>(q) & 7u) == 0) && (!w || wf::a16(w)) && (!b || wf::a16(b)) &&
                 (!shift || wf::a16(shift)) && (!scale || wf::a16(scale)) && ((!shift && !scale) || ld_mod % 8 == 0),
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  wf::LnArgs a{static_cast<uint16_t*>(x), ldx, static_cast<const uint16_t*>(y), ldy,
               static_cast<const uint16_t*>(gate), ld_gate, static_cast<int>(T), dim, eps,
               static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
               static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), ld_mod, frame_tokens,
               static_cast<uint16_t*>(out), ldo, q, q_scales};
  return wf::launch_ln(a, wf::as_stream(stream), fn);
}

int wf_ln_modulate_quant(const void* x, int64_t T, int32_t dim, int64_t ldx, float eps, const void* w, const void* b,
                         const void* shift, const void* scale, int64_t ld_mod, int32_t frame_tokens, void* out,
                         int64_t ldo, int8_t* q, float* q_scales, void* stream) {
  return wf_gate_residual_ln_quant(const_cast<void*>(x), T, dim, ldx, nullptr, 0, nullptr, 0, eps, w, b, shift, scale,
                                   ld_mod, frame_tokens, out, ldo, q, q_scales, stream);
}

int wf_rmsnorm_rope(const void* x, int64_t T, int32_t dim, int64_t ldx, int32_t head_dim, float eps, const void* w,
                    const float* cos, const float* sin, void* out, int64_t ldo, void* stream) {
  static const char* fn = "wf_rmsnorm_rope";
  WF_REQUIRE(T >= 0 && dim > 0 && head_dim > 0 && ldx >= dim && ldo >= dim, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(dim % 8 == 0 && dim <= 16384 && dim % head_dim == 0 && head_dim % 8 == 0, WF_E_SHAPE,
             "%s: dim=%d head_dim=%d unsupported", fn, dim, head_dim);
  WF_REQUIRE(T < (1ll << 24), WF_E_SHAPE, "%s: T=%lld too large (a launch holds at most 2^32 threads)", fn,
             (long long)T);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && w && out && ((cos == nullptr) == (sin == nullptr)), WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(wf::a16(x) && wf::a16(w) && wf::a16(out) && ldx % 8 == 0 && ldo % 8 == 0 &&
                 (!cos || (wf::a16(cos) && wf::a16(sin))),
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  {
    // In place needs the same rows; otherwise the output must not overlap the input rows.
    const char* xb = static_cast<const char*>(x);
    const char* ob = static_cast<const char*>(out);
    const int64_t span_x = ((T - 1) * ldx + dim) * 2, span_o = ((T - 1) * ldo + dim) * 2;
    WF_REQUIRE((out == x && ldo == ldx) || ob + span_o <= xb || xb + span_x <= ob, WF_E_INVALID,
               "%s: out overlaps x without being x itself", fn);
  }
  wf::RmsArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<int>(T), dim, head_dim, eps,
                static_cast<const uint16_t*>(w), cos, sin, static_cast<uint16_t*>(out), ldo};
  int lpr = 0, nc = 0;
  wf::rows::pick_shape(dim / 8, lpr, nc);
  const uint32_t grid = static_cast<uint32_t>((T + 256 / lpr - 1) / (256 / lpr));
  wf::rows::dispatch_shape(lpr, nc, [&](auto L, auto C) {
    hipLaunchKernelGGL((wf::rmsnorm_rope_kernel<decltype(L)::value, decltype(C)::value>), dim3(grid), dim3(256), 0,
                       wf::as_stream(stream), a);
  });
  return wf::check_launch(fn);
}

int wf_gate_residual(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, int64_t ld_gate, int64_t T,
                     int32_t dim, int32_t frame_tokens, void* stream) {
  static const char* fn = "wf_gate_residual";
  WF_REQUIRE(T >= 0 && dim > 0 && ldx >= dim && ldy >= dim && frame_tokens > 0, WF_E_INVALID, "%s: bad sizes", fn);
  WF_REQUIRE(!gate || ld_gate >= dim, WF_E_INVALID, "%s: ld_gate < dim", fn);
  WF_REQUIRE(dim % 8 == 0, WF_E_SHAPE, "%s: dim %% 8 != 0", fn);
  WF_REQUIRE(T * (dim / 8) < (1ll << 32) - 256, WF_E_SHAPE, "%s: T=%lld too large (a launch holds at most 2^32 threads)",
             fn, (long long)T);
  if (T == 0) return WF_OK;
  WF_REQUIRE(x && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(wf::a16(x) && wf::a16(y) && (!gate || (wf::a16(gate) && ld_gate % 8 == 0)) && ldx % 8 == 0 &&
                 ldy % 8 == 0,
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", fn);
  const int64_t n = T * (dim / 8);
  hipLaunchKernelGGL(wf::gate_residual_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                     wf::as_stream(stream), static_cast<uint16_t*>(x), ldx, static_cast<const uint16_t*>(y), ldy,
                     static_cast<const uint16_t*>(gate), ld_gate, static_cast<int>(T), dim, frame_tokens);
  return wf::check_launch(fn);
}

}  // extern "C"
