// FP8 e4m3fn paged KV pool: pack (quantize + page scatter) and
// gather-dequant, both HBM-bound streaming kernels.
//
// Work split: one (token, head) row of head_dim = 128 bf16 values (256 B)
// is owned by an aligned group of 8 lanes, 16 values (32 B in, 16 B of
// codes out) per lane, so every code store is one 16-byte vector store and a
// wave writes 8 rows = 1 KiB of consecutive codes.  The per-row absmax is an
// 8-lane DPP reduction.  Each workgroup of 256 threads owns one block of 32
// consecutive rows of K or of V.  Blocks are numbered K first, then V, and
// the workgroups one XCD receives (blockIdx % 8) take a contiguous range of
// them, so neighbouring rows (which share 64-byte lines of the scale
// arrays, laid out token-fastest per (page, head)) are written through the
// same L2.
//
// Arithmetic per row, following wave_rt/denoiser/exchange/common.py:145-150
// with the amax taken per (token, head):
//   amax  = max |x|                      (exact, a bf16 value)
//   s     = bf16_rne(amax / 448)         (bf16 arithmetic as in the reference)
//   s     = max(s, bf16(1e-8))           (.clamp(min=1e-8)), then to fp32
//   code  = e4m3_rne(min(|x| / s, 448)) with the sign of x
// amax / 448 is taken as amax * RN(1/448): rounded to bf16 it equals the
// bf16 of the IEEE quotient for every bf16 amax (amax / 448 = (m / 7) 2^k
// with an 8-bit m is either a short exact value or a repeating binary
// fraction far from every bf16 rounding boundary; checked exhaustively).
// |x| / s: q = |x| * r with r = v_rcp_f32(s) (within one ulp of 1/s), then
// one residual step q += fma(-q, s, |x|) * r.  The quotient of two 8-bit
// significands is either exact (and the residual step returns it exactly)
// or at least 2^-14 (relative) away from every e4m3 rounding boundary, so
// the code equals that of the IEEE quotient (checked over every pair of
// significands, for both reciprocals next to 1/s).
//
// Two fused producers feed the same pages:
// * kv_pack_kernel<..., ROPE = true> rotates K by a per-token RoPE table
//   before quantizing it: the anchor re-RoPE of the exchange
//   (wave_rt/denoiser/exchange/common.py:70-91), whose rotated bf16 K the
//   reference copies into slot 0 (paged.py:222-227), packed in one pass;
// * k_norm_rope_pack_kernel takes K straight from the fused QKV output:
//   RMSNorm over the token's full row, RoPE, FP8 pack, and V's pack, one
//   token row per wave or workgroup (the row engine of rows.hpp).
// The rotation of a pair (a, b) by angle i is (a c - b s, a s + b c) in fp32
// with the table's fp32 cos/sin (the library is built without FMA
// contraction), rounded to bf16 before the quantization, as the reference
// rounds the rotated K to bf16 (`.type_as(v)`, common.py:86-88).
#include "fastdiv.hpp"
#include "fp8_codec.hpp"
#include "rows.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

constexpr int kHeadDim = 128;
// Non-temporal hints, chosen by sweeps on MI355X (rows per lane group
// {1, 2, 4, 8}, persistent grids, block-to-XCD maps, hints): streaming
// stores for pack (6.0 TB/s over 30 layers in one launch), streaming loads
// and stores for unpack (6.0 TB/s).
constexpr bool kPackNtLoad = false, kPackNtStore = true;
constexpr bool kUnpackNtLoad = true, kUnpackNtStore = true;
constexpr int kRowsPerBlock = 32;
constexpr uint32_t kNumXcd = 8;

// Row block, and whether it is V, of workgroup blockIdx.x over n_items
// blocks (n_blocks K blocks first, then V blocks when n_items = 2 n_blocks),
// XCD-contiguous.  Returns false past the end.
__device__ inline bool block_of(uint32_t n_blocks, uint32_t n_items, uint32_t& blk, bool& is_v) {
  const uint32_t per_xcd = (n_items + kNumXcd - 1) / kNumXcd;
  const uint32_t w = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
  if (w >= n_items) return false;
  is_v = w >= n_blocks;
  blk = is_v ? w - n_blocks : w;
  return true;
}

struct PoolView {
  uint8_t* codes;
  float* scales;
};

struct PageGeom {
  FastDiv heads;       // row -> (token, head)
  FastDiv page;        // token -> (logical page, row in page)
  const int32_t* table;
  uint32_t n_table;
  uint32_t page_tokens;
  uint32_t n_heads;
  int32_t pool_pages;
};

// Locate row r = token * n_heads + head in the pool.  Returns false when its
// logical page has no valid physical page.
__device__ inline bool locate(const PageGeom& g, uint32_t r, int64_t& code_row, int64_t& scale_idx) {
  uint32_t t, h, lp, rip;
  g.heads.divmod(r, t, h);
  g.page.divmod(t, lp, rip);
  if (lp >= g.n_table) return false;
  const int32_t page = g.table[lp];
  if (page < 0 || page >= g.pool_pages) return false;
  code_row = (static_cast<int64_t>(page) * g.page_tokens + rip) * g.n_heads + h;
  scale_idx = (static_cast<int64_t>(page) * g.n_heads + h) * g.page_tokens + rip;
  return true;
}

// Four e4m3 codes of bf16-exact values x[0..3] with scale s (r within one ulp of 1/s).
__device__ inline uint32_t quant4f(const float* x, float s, float r) {
  float q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ax = fabsf(x[i]);
    float qi = ax * r;
    const float e = fmaf(-qi, s, ax);
    qi = fmaf(e, r, qi);
    qi = fminf(qi, kE4M3Max);
    q[i] = bits_f32(f32_bits(qi) | (f32_bits(x[i]) & 0x80000000u));
  }
  return e4m3_pack4_hw(q[0], q[1], q[2], q[3]);
}

__device__ inline uint32_t quant4(uint32_t w01, uint32_t w23, float s, float r) {
  const float x[4] = {bf16_lo_to_f32(w01), bf16_hi_to_f32(w01), bf16_lo_to_f32(w23), bf16_hi_to_f32(w23)};
  return quant4f(x, s, r);
}

// Rotate the 4 pairs of 8 fp32 values by (c[j], s[j]) and round to bf16.
__device__ inline void rope4_bf16(float* y, const float4& c4, const float4& s4) {
  const float cs[4] = {c4.x, c4.y, c4.z, c4.w};
  const float sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = y[2 * j], x1 = y[2 * j + 1];
    y[2 * j] = x0 * cs[j] - x1 * sn[j];
    y[2 * j + 1] = x0 * sn[j] + x1 * cs[j];
  }
  rows::rbf8(y);
}

// The same on a 16-byte chunk of 8 bf16 values.
__device__ inline uint4 rope_chunk(const uint4& w, const float4& c4, const float4& s4) {
  float y[8];
  rows::unpack8(w, y);
  rope4_bf16(y, c4, s4);
  return rows::pack8(y);
}

__device__ inline float absmax8(const uint4& a, const uint4& b) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo_to_f32(w[i])), fabsf(bf16_hi_to_f32(w[i]))));
  return m;
}

// bf16(amax / 448) as bf16(amax * RN(1/448)) (see above), floored at bf16(1e-8).
constexpr float kInvE4M3Max = 1.0f / kE4M3Max;
__device__ inline float scale_from_amax(float amax) {
  const float s = bf16_bits_to_f32(static_cast<uint16_t>(pack_bf16x2_hw(amax * kInvE4M3Max, 0.f)));
  return fmaxf(s, bf16_bits_to_f32(kScaleFloorBf16Bits));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ inline uint4 ld16(const uint4* p) {
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
  } else {
    return *p;
  }
}

template <bool NT>
__device__ inline void st16(uint4* p, const uint4& v) {
  if constexpr (NT) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  } else {
    *p = v;
  }
}

// ROPE: K rows are rotated first, token t by row t % rope_rows of cos/sin
// [rope_rows][64] (rope_rows = n_tokens: one row per token; a chunk's
// token count: one table for a batch of equal chunks).
template <bool NT_LOAD, bool NT_STORE, bool ROPE>
__global__ __launch_bounds__(256) void kv_pack_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                                                      int64_t ld_kv, uint32_t n_rows, uint32_t n_blocks,
                                                      uint32_t n_items, PageGeom geom, PoolView kpool,
                                                      PoolView vpool, const float* __restrict__ cos,
                                                      const float* __restrict__ sin, FastDiv rope_rows) {
  uint32_t blk;
  bool is_v;
  if (!block_of(n_blocks, n_items, blk, is_v)) return;
  const uint4* __restrict__ src = is_v ? v : k;
  const PoolView pool = is_v ? vpool : kpool;
  const uint32_t lane8 = threadIdx.x & 7u;
  const uint32_t r = blk * kRowsPerBlock + (threadIdx.x >> 3);

  uint4 a = make_uint4(0, 0, 0, 0), b = a;
  if (r < n_rows) {
    uint32_t t, h;
    geom.heads.divmod(r, t, h);
    const uint4* p = src + (static_cast<int64_t>(t) * ld_kv + h * kHeadDim) / 8 + lane8 * 2;
    a = ld16<NT_LOAD>(p);
    b = ld16<NT_LOAD>(p + 1);
    if constexpr (ROPE) {
      if (!is_v) {
        uint32_t chunk, tr;
        rope_rows.divmod(t, chunk, tr);
        // pairs 8 lane8 .. 8 lane8 + 7 of the head
        const float4* cp = reinterpret_cast<const float4*>(cos + static_cast<int64_t>(tr) * (kHeadDim / 2)) + lane8 * 2;
        const float4* sp = reinterpret_cast<const float4*>(sin + static_cast<int64_t>(tr) * (kHeadDim / 2)) + lane8 * 2;
        a = rope_chunk(a, cp[0], sp[0]);
        b = rope_chunk(b, cp[1], sp[1]);
      }
    }
  }
  // every lane of the 8-lane group takes part in the reduction
  const float amax = group8_max(absmax8(a, b));
  const float s = scale_from_amax(amax);
  const float rcp = __builtin_amdgcn_rcpf(s);
  uint4 c;
  c.x = quant4(a.x, a.y, s, rcp);
  c.y = quant4(a.z, a.w, s, rcp);
  c.z = quant4(b.x, b.y, s, rcp);
  c.w = quant4(b.z, b.w, s, rcp);
  int64_t code_row, scale_idx;
  if (r < n_rows && locate(geom, r, code_row, scale_idx)) {
    st16<NT_STORE>(reinterpret_cast<uint4*>(pool.codes + code_row * kHeadDim) + lane8, c);
    if (lane8 == 0) pool.scales[scale_idx] = s;
  }
}

// ------------------------------------------- K RMSNorm + RoPE + K/V pack
struct KNormPackArgs {
  const uint16_t* k;    // bf16 [T][ld_kv]: n_heads * 128 values per token
  const uint16_t* v;    // bf16 [T][ld_kv] or null
  int64_t ld_kv;
  int T;
  float eps;
  const uint16_t* w;    // RMSNorm weight [n_heads * 128] bf16
  const float* cos;     // [T][64] or null (no rotation)
  const float* sin;
  uint16_t* ku;         // normalized, un-rotated K [T][ld_ku] bf16, or null
  int64_t ld_ku;
  uint16_t* q;          // Q [T][ld_q] bf16, RMSNorm'd (weight wq) and rotated in place, or null
  int64_t ld_q;
  const uint16_t* wq;
  PageGeom geom;
  PoolView kpool, vpool;
};

// Page position of token t: code row of head 0 and scale index of head 0
// (head h adds h * 128 codes and h * page_tokens scales).  False when the
// token's logical page has no valid physical page.
__device__ inline bool token_slot(const PageGeom& g, uint32_t t, int64_t& code_row0, int64_t& scale0) {
  uint32_t lp, rip;
  g.page.divmod(t, lp, rip);
  if (lp >= g.n_table) return false;
  const int32_t page = g.table[lp];
  if (page < 0 || page >= g.pool_pages) return false;
  code_row0 = (static_cast<int64_t>(page) * g.page_tokens + rip) * g.n_heads;
  scale0 = static_cast<int64_t>(page) * g.n_heads * g.page_tokens + rip;
  return true;
}

// Quantize the 8 bf16-exact values y of chunk ch (head ch / 16) with the
// head's scale, which the 16 lanes holding that head reduce together, and
// store 8 codes (+ the scale from the head's first lane).
__device__ inline void pack_head_chunk(const float* y, int ch, bool valid, bool placed, const PageGeom& g,
                                       int64_t code_row0, int64_t scale0, const PoolView& pool) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(y[i]));
  const float amax = rows::group16_max(m);
  const float s = scale_from_amax(amax);
  const float r = __builtin_amdgcn_rcpf(s);
  const uint2 c = make_uint2(quant4f(y, s, r), quant4f(y + 4, s, r));
  if (valid && placed) {
    const int h = ch >> 4;
    *reinterpret_cast<uint2*>(pool.codes + (code_row0 + h) * kHeadDim + (ch & 15) * 8) = c;
    if ((ch & 15) == 0) pool.scales[scale0 + static_cast<int64_t>(h) * g.page_tokens] = s;
  }
}

// One token row per LPR lanes (rows.hpp): K = RMSNorm(k) over the row
// (y = bf16(bf16(k * rsqrt(mean(k^2) + eps)) * w), WanRMSNorm, model.py:78-86,
// with the reduction of rmsnorm_rope_kernel), optionally stored un-rotated,
// then rotated per head and packed; V packed as is.  Lane chunk ch covers
// elements 8 ch .. 8 ch + 7, so a head's 16 chunks sit in 16 aligned lanes.
template <int LPR, int NC>
__global__ __launch_bounds__(256) void k_norm_rope_pack_kernel(KNormPackArgs a) {
  constexpr int RPB = 256 / LPR;
  __shared__ float red[4], redq[4];
  // Row blocks go XCD-contiguously (as block_of), so the token-fastest scale
  // lines of neighbouring tokens are written through one L2.
  const uint32_t n_blk = (static_cast<uint32_t>(a.T) + RPB - 1) / RPB;
  const uint32_t per_xcd = (n_blk + kNumXcd - 1) / kNumXcd;
  const uint32_t blk = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
  const int lane = static_cast<int>(threadIdx.x) % LPR;
  const int t = static_cast<int>(blk) * RPB + static_cast<int>(threadIdx.x) / LPR;
  if (blk >= n_blk || t >= a.T) return;
  const int n_chunks = static_cast<int>(a.geom.n_heads) * (kHeadDim / 8);
  const uint16_t* krow = a.k + static_cast<int64_t>(t) * a.ld_kv;
  const bool rot = a.cos != nullptr;
  // every load of the row is issued before the first reduction
  uint4 kw[NC], vw[NC], ww[NC];
  float4 cs[NC], sn[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    const bool valid = ch < n_chunks;
    kw[c] = valid ? rows::ld16(krow + ch * 8) : make_uint4(0, 0, 0, 0);
    ww[c] = valid ? rows::ld16(a.w + ch * 8) : make_uint4(0, 0, 0, 0);
    const int64_t p0 = static_cast<int64_t>(t) * (kHeadDim / 2) + (ch & 15) * 4;  // first pair of the chunk
    cs[c] = valid && rot ? *reinterpret_cast<const float4*>(a.cos + p0) : make_float4(1.f, 1.f, 1.f, 1.f);
    sn[c] = valid && rot ? *reinterpret_cast<const float4*>(a.sin + p0) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (a.v) {
    const uint16_t* vrow = a.v + static_cast<int64_t>(t) * a.ld_kv;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + LPR * c;
      vw[c] = ch < n_chunks ? rows::ld16(vrow + ch * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  uint4 qw[NC], wqw[NC];
  uint16_t* qrow = a.q ? a.q + static_cast<int64_t>(t) * a.ld_q : nullptr;
  if (a.q) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + LPR * c;
      const bool valid = ch < n_chunks;
      qw[c] = valid ? rows::ld16(qrow + ch * 8) : make_uint4(0, 0, 0, 0);
      wqw[c] = valid ? rows::ld16(a.wq + ch * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  int64_t code_row0 = 0, scale0 = 0;
  const bool placed = token_slot(a.geom, static_cast<uint32_t>(t), code_row0, scale0);
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float x[8];
    rows::unpack8(kw[c], x);
#pragma unroll
    for (int i = 0; i < 8; ++i) sq += x[i] * x[i];
  }
  const float ms = rows::row_sum<LPR>(sq, red) / static_cast<float>(n_chunks * 8);
  const float rn = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + LPR * c;
    const bool valid = ch < n_chunks;
    float x[8], wv[8], y[8];
    rows::unpack8(kw[c], x);
    rows::unpack8(ww[c], wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = x[i] * rn;
    rows::rbf8(y);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = y[i] * wv[i];
    rows::rbf8(y);
    if (a.ku && valid) rows::st16(a.ku + static_cast<int64_t>(t) * a.ld_ku + ch * 8, rows::pack8(y));
    if (rot) rope4_bf16(y, cs[c], sn[c]);
    pack_head_chunk(y, ch, valid, placed, a.geom, code_row0, scale0, a.kpool);
  }
  if (a.v) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + LPR * c;
      float y[8];
      rows::unpack8(vw[c], y);
      pack_head_chunk(y, ch, ch < n_chunks, placed, a.geom, code_row0, scale0, a.vpool);
    }
  }
  if (a.q) {
    // Q: the same RMSNorm (its own weight) and rotation, written back in place
    // (the row was read whole above); wf_rmsnorm_rope's arithmetic
    float sqq = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8];
      rows::unpack8(qw[c], x);
#pragma unroll
      for (int i = 0; i < 8; ++i) sqq += x[i] * x[i];
    }
    const float msq = rows::row_sum<LPR>(sqq, redq) / static_cast<float>(n_chunks * 8);
    const float rq = 1.0f / sqrtf(msq + a.eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int ch = lane + LPR * c;
      float x[8], wv[8];
      rows::unpack8(qw[c], x);
      rows::unpack8(wqw[c], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = x[i] * rq;
      rows::rbf8(x);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = x[i] * wv[i];
      rows::rbf8(x);
      if (rot) rope4_bf16(x, cs[c], sn[c]);
      if (ch < n_chunks) rows::st16(qrow + ch * 8, rows::pack8(x));
    }
  }
}

__device__ inline uint2 dequant4(uint32_t w, float s) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  float v0, v1, v2, v3;
  e4m3_unpack4_hw(w, v0, v1, v2, v3);
  const f2 lo = {v0 * s, v1 * s};
  const f2 hi = {v2 * s, v3 * s};
  const b2 blo = __builtin_convertvector(lo, b2);
  const b2 bhi = __builtin_convertvector(hi, b2);
  return make_uint2(__builtin_bit_cast(uint32_t, blo), __builtin_bit_cast(uint32_t, bhi));
}

template <bool NT_LOAD, bool NT_STORE>
__global__ __launch_bounds__(256) void kv_unpack_kernel(PoolView kpool, PoolView vpool, uint32_t n_rows,
                                                        uint32_t n_blocks, uint32_t n_items, PageGeom geom,
                                                        uint4* __restrict__ kout, uint4* __restrict__ vout) {
  uint32_t blk;
  bool is_v;
  if (!block_of(n_blocks, n_items, blk, is_v)) return;
  const PoolView pool = is_v ? vpool : kpool;
  uint4* __restrict__ dst = is_v ? vout : kout;
  const uint32_t lane8 = threadIdx.x & 7u;
  const uint32_t r = blk * kRowsPerBlock + (threadIdx.x >> 3);
  int64_t code_row = 0, scale_idx = 0;
  if (!(r < n_rows && locate(geom, r, code_row, scale_idx))) return;
  const uint4 c = ld16<NT_LOAD>(reinterpret_cast<const uint4*>(pool.codes + code_row * kHeadDim) + lane8);
  const float s = pool.scales[scale_idx];
  const uint2 o0 = dequant4(c.x, s);
  const uint2 o1 = dequant4(c.y, s);
  const uint2 o2 = dequant4(c.z, s);
  const uint2 o3 = dequant4(c.w, s);
  uint4* p = dst + static_cast<int64_t>(r) * (kHeadDim / 8) + lane8 * 2;
  st16<NT_STORE>(p, make_uint4(o0.x, o0.y, o1.x, o1.y));
  st16<NT_STORE>(p + 1, make_uint4(o2.x, o2.y, o3.x, o3.y));
}

int check_pool_args(const char* fn, int64_t n_tokens, int32_t n_heads, int32_t head_dim, const int32_t* page_table,
                    int64_t n_table, int32_t page_tokens, int64_t pool_pages) {
  WF_REQUIRE(n_tokens >= 0 && n_heads > 0 && page_tokens > 0 && n_table >= 0 && pool_pages >= 0, WF_E_INVALID,
             "%s: negative or zero size (n_tokens=%lld n_heads=%d page_tokens=%d n_table=%lld pool_pages=%lld)", fn,
             (long long)n_tokens, n_heads, page_tokens, (long long)n_table, (long long)pool_pages);
  WF_REQUIRE(head_dim == kHeadDim, WF_E_SHAPE, "%s: head_dim=%d unsupported (must be 128)", fn, head_dim);
  WF_REQUIRE(wf::product_below({n_tokens, n_heads}, 1ll << 31), WF_E_SHAPE,
             "%s: n_tokens=%lld x n_heads=%d reaches 2^31", fn, (long long)n_tokens, n_heads);
  WF_REQUIRE(pool_pages < (1ll << 31) && n_table < (1ll << 31), WF_E_SHAPE, "%s: pool or table too large", fn);
  WF_REQUIRE(n_table * page_tokens >= n_tokens, WF_E_SHAPE,
             "%s: page table covers %lld tokens < n_tokens=%lld", fn, (long long)(n_table * page_tokens),
             (long long)n_tokens);
  WF_REQUIRE(n_tokens == 0 || page_table, WF_E_INVALID, "%s: null page table", fn);
  return WF_OK;
}

PageGeom make_geom(int32_t n_heads, const int32_t* page_table, int64_t n_table, int32_t page_tokens,
                   int64_t pool_pages) {
  PageGeom g;
  g.heads = FastDiv(static_cast<uint32_t>(n_heads));
  g.page = FastDiv(static_cast<uint32_t>(page_tokens));
  g.table = page_table;
  g.n_table = static_cast<uint32_t>(n_table);
  g.page_tokens = static_cast<uint32_t>(page_tokens);
  g.n_heads = static_cast<uint32_t>(n_heads);
  g.pool_pages = static_cast<int32_t>(pool_pages);
  return g;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// wf_fp8_kv_pack and wf_fp8_kv_pack_rope[_tiled] (cos/sin null: no rotation;
// rope_rows: rows of the table, token t uses row t % rope_rows).
int launch_pack(const char* fn, const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                int64_t ld_kv, const float* cos, const float* sin, int64_t rope_rows, const int32_t* page_table,
                int64_t n_table, int32_t page_tokens, uint8_t* k_codes, uint8_t* v_codes, float* k_scales,
                float* v_scales, int64_t pool_pages, void* stream) {
  if (int st = check_pool_args(fn, n_tokens, n_heads, head_dim, page_table, n_table, page_tokens, pool_pages))
    return st;
  if (n_tokens == 0) return WF_OK;
  WF_REQUIRE(!cos || (rope_rows > 0 && rope_rows <= n_tokens), WF_E_INVALID,
             "%s: rope_rows=%lld must be in [1, n_tokens=%lld]", fn, (long long)rope_rows, (long long)n_tokens);
  WF_REQUIRE(k && k_codes && k_scales, WF_E_INVALID, "%s: null K pointer", fn);
  WF_REQUIRE(ld_kv >= static_cast<int64_t>(n_heads) * head_dim && ld_kv % 8 == 0, WF_E_INVALID,
             "%s: ld_kv=%lld must be >= n_heads*head_dim and a multiple of 8", fn, (long long)ld_kv);
  const bool has_v = v != nullptr;
  WF_REQUIRE(!has_v || (v_codes && v_scales), WF_E_INVALID, "%s: V given without V pool", fn);
  WF_REQUIRE(aligned16(k) && aligned16(k_codes) && (!has_v || (aligned16(v) && aligned16(v_codes))), WF_E_ALIGN,
             "%s: K/V and code pools must be 16-byte aligned", fn);
  const uint32_t n_rows = static_cast<uint32_t>(n_tokens * n_heads);
  const PageGeom geom = make_geom(n_heads, page_table, n_table, page_tokens, pool_pages);
  const uint32_t n_blocks = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const uint32_t items = has_v ? 2 * n_blocks : n_blocks;
  const dim3 grid((items + kNumXcd - 1) / kNumXcd * kNumXcd);
  const uint4* k4 = reinterpret_cast<const uint4*>(k);
  const uint4* v4 = reinterpret_cast<const uint4*>(v);
  if (cos) {
    hipLaunchKernelGGL((kv_pack_kernel<kPackNtLoad, kPackNtStore, true>), grid, dim3(256), 0, as_stream(stream), k4,
                       v4, ld_kv, n_rows, n_blocks, items, geom, PoolView{k_codes, k_scales},
                       PoolView{v_codes, v_scales}, cos, sin, FastDiv(static_cast<uint32_t>(rope_rows)));
  } else {
    hipLaunchKernelGGL((kv_pack_kernel<kPackNtLoad, kPackNtStore, false>), grid, dim3(256), 0, as_stream(stream), k4,
                       v4, ld_kv, n_rows, n_blocks, items, geom, PoolView{k_codes, k_scales},
                       PoolView{v_codes, v_scales}, nullptr, nullptr, FastDiv(1));
  }
  return check_launch(fn);
}

}  // namespace
}  // namespace wf

namespace wf {
namespace {
// Rows [T][dim] at a (stride lda) and at b (stride ldb) share no element.
bool rows_disjoint(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t T, int64_t dim) {
  const int64_t d = (reinterpret_cast<intptr_t>(b) - reinterpret_cast<intptr_t>(a)) / 2;  // bf16 elements
  const int64_t span_a = (T - 1) * lda + dim, span_b = (T - 1) * ldb + dim;
  if (d >= span_a || -d >= span_b) return true;
  if (lda != ldb || (reinterpret_cast<intptr_t>(b) - reinterpret_cast<intptr_t>(a)) % 2) return false;
  const int64_t r = ((d % lda) + lda) % lda;  // interleaved rows, e.g. column slices of one QKV output
  return r >= dim && r <= lda - dim;
}

int k_norm_pack(const char* fn, void* q, int64_t ld_q, const void* norm_q, const void* k, const void* v,
                int64_t n_tokens, int32_t n_heads, int32_t head_dim, int64_t ld_kv, float eps, const void* norm_w,
                const float* cos, const float* sin, void* ku_out, int64_t ld_ku, const int32_t* page_table,
                int64_t n_table, int32_t page_tokens, uint8_t* k_codes, uint8_t* v_codes, float* k_scales,
                float* v_scales, int64_t pool_pages, void* stream) {
  if (int st = wf::check_pool_args(fn, n_tokens, n_heads, head_dim, page_table, n_table, page_tokens, pool_pages))
    return st;
  if (n_tokens == 0) return WF_OK;
  const int64_t dim = static_cast<int64_t>(n_heads) * head_dim;
  int lpr = 0, nc = 0;
  WF_REQUIRE(wf::rows::pick_shape(dim / 8, lpr, nc), WF_E_SHAPE, "%s: n_heads*head_dim=%lld exceeds 16384", fn,
             (long long)dim);
  WF_REQUIRE(k && norm_w && k_codes && k_scales, WF_E_INVALID, "%s: null K, weight or K pool", fn);
  WF_REQUIRE(!v || (v_codes && v_scales), WF_E_INVALID, "%s: V given without V pool", fn);
  WF_REQUIRE((cos == nullptr) == (sin == nullptr), WF_E_INVALID, "%s: cos and sin must both be given or both null",
             fn);
  WF_REQUIRE(ld_kv >= dim && ld_kv % 8 == 0, WF_E_INVALID, "%s: ld_kv=%lld must be >= n_heads*head_dim and %% 8 == 0",
             fn, (long long)ld_kv);
  WF_REQUIRE(!ku_out || (ld_ku >= dim && ld_ku % 8 == 0), WF_E_INVALID, "%s: ld_ku must be >= n_heads*head_dim and "
             "%% 8 == 0", fn);
  WF_REQUIRE(wf::aligned16(k) && wf::aligned16(v) && wf::aligned16(norm_w) && wf::aligned16(cos) &&
                 wf::aligned16(sin) && wf::aligned16(ku_out) && wf::aligned16(k_codes) && wf::aligned16(v_codes),
             WF_E_ALIGN, "%s: tensors must be 16-byte aligned", fn);
  if (ku_out) {
    // in place over K (a lane rewrites only the chunks it has read) or disjoint from K and V
    const uintptr_t kb = reinterpret_cast<uintptr_t>(k), ub = reinterpret_cast<uintptr_t>(ku_out);
    const uintptr_t span_k = static_cast<uintptr_t>((n_tokens - 1) * ld_kv + dim) * 2;
    const uintptr_t span_u = static_cast<uintptr_t>((n_tokens - 1) * ld_ku + dim) * 2;
    const bool in_place = ub == kb && ld_ku == ld_kv;
    WF_REQUIRE(in_place || ub + span_u <= kb || kb + span_k <= ub, WF_E_INVALID,
               "%s: ku_out must be K itself (same stride) or not overlap it", fn);
    if (v) {
      const uintptr_t vb = reinterpret_cast<uintptr_t>(v);
      WF_REQUIRE(ub + span_u <= vb || vb + span_k <= ub, WF_E_INVALID, "%s: ku_out overlaps V", fn);
    }
  }
  if (q) {
    WF_REQUIRE(norm_q && ld_q >= dim && ld_q % 8 == 0 && wf::aligned16(q) && wf::aligned16(norm_q), WF_E_INVALID,
               "%s: q needs its weight, ld_q >= n_heads*head_dim with ld_q %% 8 == 0 and 16-byte alignment", fn);
    WF_REQUIRE(rows_disjoint(q, ld_q, k, ld_kv, n_tokens, dim) && (!v || rows_disjoint(q, ld_q, v, ld_kv, n_tokens, dim)) &&
                   (!ku_out || rows_disjoint(q, ld_q, ku_out, ld_ku, n_tokens, dim)),
               WF_E_INVALID, "%s: q must not overlap K, V or ku_out", fn);
  }
  wf::KNormPackArgs a;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.ld_kv = ld_kv;
  a.T = static_cast<int>(n_tokens);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(norm_w);
  a.cos = cos;
  a.sin = sin;
  a.ku = static_cast<uint16_t*>(ku_out);
  a.ld_ku = ld_ku;
  a.q = static_cast<uint16_t*>(q);
  a.ld_q = ld_q;
  a.wq = static_cast<const uint16_t*>(norm_q);
  a.geom = wf::make_geom(n_heads, page_table, n_table, page_tokens, pool_pages);
  a.kpool = wf::PoolView{k_codes, k_scales};
  a.vpool = wf::PoolView{v_codes, v_scales};
  const uint32_t n_blk = static_cast<uint32_t>((n_tokens + 256 / lpr - 1) / (256 / lpr));
  const uint32_t grid = (n_blk + wf::kNumXcd - 1) / wf::kNumXcd * wf::kNumXcd;
  wf::rows::dispatch_shape(lpr, nc, [&](auto L, auto C) {
    hipLaunchKernelGGL((wf::k_norm_rope_pack_kernel<decltype(L)::value, decltype(C)::value>), dim3(grid), dim3(256),
                       0, wf::as_stream(stream), a);
  });
  return wf::check_launch(fn);
}
}  // namespace
}  // namespace wf

extern "C" {

int wf_fp8_kv_pack(const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                   int64_t ld_kv, const int32_t* page_table, int64_t n_table, int32_t page_tokens, uint8_t* k_codes,
                   uint8_t* v_codes, float* k_scales, float* v_scales, int64_t pool_pages, void* stream) {
  return wf::launch_pack("wf_fp8_kv_pack", k, v, n_tokens, n_heads, head_dim, ld_kv, nullptr, nullptr, 0, page_table,
                         n_table, page_tokens, k_codes, v_codes, k_scales, v_scales, pool_pages, stream);
}

int wf_fp8_kv_pack_rope(const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                        int64_t ld_kv, const float* cos, const float* sin, const int32_t* page_table, int64_t n_table,
                        int32_t page_tokens, uint8_t* k_codes, uint8_t* v_codes, float* k_scales, float* v_scales,
                        int64_t pool_pages, void* stream) {
  static const char* fn = "wf_fp8_kv_pack_rope";
  WF_REQUIRE(n_tokens == 0 || (cos && sin), WF_E_INVALID, "%s: null RoPE table", fn);
  WF_REQUIRE(wf::aligned16(cos) && wf::aligned16(sin), WF_E_ALIGN, "%s: RoPE tables must be 16-byte aligned", fn);
  return wf::launch_pack(fn, k, v, n_tokens, n_heads, head_dim, ld_kv, cos, sin, n_tokens, page_table, n_table,
                         page_tokens, k_codes, v_codes, k_scales, v_scales, pool_pages, stream);
}

int wf_fp8_kv_pack_rope_tiled(const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                              int64_t ld_kv, const float* cos, const float* sin, int64_t rope_rows,
                              const int32_t* page_table, int64_t n_table, int32_t page_tokens, uint8_t* k_codes,
                              uint8_t* v_codes, float* k_scales, float* v_scales, int64_t pool_pages, void* stream) {
  static const char* fn = "wf_fp8_kv_pack_rope_tiled";
  WF_REQUIRE(n_tokens == 0 || (cos && sin), WF_E_INVALID, "%s: null RoPE table", fn);
  WF_REQUIRE(wf::aligned16(cos) && wf::aligned16(sin), WF_E_ALIGN, "%s: RoPE tables must be 16-byte aligned", fn);
  return wf::launch_pack(fn, k, v, n_tokens, n_heads, head_dim, ld_kv, cos, sin, rope_rows, page_table, n_table,
                         page_tokens, k_codes, v_codes, k_scales, v_scales, pool_pages, stream);
}


int wf_k_norm_rope_kv_pack(const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                           int64_t ld_kv, float eps, const void* norm_w, const float* cos, const float* sin,
                           void* ku_out, int64_t ld_ku, const int32_t* page_table, int64_t n_table,
                           int32_t page_tokens, uint8_t* k_codes, uint8_t* v_codes, float* k_scales, float* v_scales,
                           int64_t pool_pages, void* stream) {
  return wf::k_norm_pack("wf_k_norm_rope_kv_pack", nullptr, 0, nullptr, k, v, n_tokens, n_heads, head_dim, ld_kv, eps,
                         norm_w, cos, sin, ku_out, ld_ku, page_table, n_table, page_tokens, k_codes, v_codes, k_scales,
                         v_scales, pool_pages, stream);
}

int wf_qk_norm_rope_kv_pack(void* q, int64_t ld_q, const void* norm_q, const void* k, const void* v, int64_t n_tokens,
                            int32_t n_heads, int32_t head_dim, int64_t ld_kv, float eps, const void* norm_k,
                            const float* cos, const float* sin, void* ku_out, int64_t ld_ku,
                            const int32_t* page_table, int64_t n_table, int32_t page_tokens, uint8_t* k_codes,
                            uint8_t* v_codes, float* k_scales, float* v_scales, int64_t pool_pages, void* stream) {
  static const char* fn = "wf_qk_norm_rope_kv_pack";
  WF_REQUIRE(q != nullptr, WF_E_INVALID, "%s: null q (use wf_k_norm_rope_kv_pack without q)", fn);
  return wf::k_norm_pack(fn, q, ld_q, norm_q, k, v, n_tokens, n_heads, head_dim, ld_kv, eps, norm_k, cos, sin, ku_out,
                         ld_ku, page_table, n_table, page_tokens, k_codes, v_codes, k_scales, v_scales, pool_pages,
                         stream);
}

int wf_fp8_kv_unpack(const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales, const float* v_scales,
                     int64_t pool_pages, const int32_t* page_table, int64_t n_table, int32_t page_tokens,
                     int64_t n_tokens, int32_t n_heads, int32_t head_dim, void* k_out, void* v_out, void* stream) {
  static const char* fn = "wf_fp8_kv_unpack";
  if (int st = wf::check_pool_args(fn, n_tokens, n_heads, head_dim, page_table, n_table, page_tokens, pool_pages))
    return st;
  if (n_tokens == 0) return WF_OK;
  WF_REQUIRE(k_codes && k_scales && k_out, WF_E_INVALID, "%s: null K pointer", fn);
  const bool has_v = v_out != nullptr;
  WF_REQUIRE(!has_v || (v_codes && v_scales), WF_E_INVALID, "%s: V output given without V pool", fn);
  WF_REQUIRE(wf::aligned16(k_out) && wf::aligned16(k_codes) &&
                 (!has_v || (wf::aligned16(v_out) && wf::aligned16(v_codes))),
             WF_E_ALIGN, "%s: outputs and code pools must be 16-byte aligned", fn);
  const uint32_t n_rows = static_cast<uint32_t>(n_tokens * n_heads);
  const wf::PageGeom geom = wf::make_geom(n_heads, page_table, n_table, page_tokens, pool_pages);
  const uint32_t n_blocks = (n_rows + wf::kRowsPerBlock - 1) / wf::kRowsPerBlock;
  const uint32_t items = has_v ? 2 * n_blocks : n_blocks;
  const dim3 grid((items + wf::kNumXcd - 1) / wf::kNumXcd * wf::kNumXcd);
  hipLaunchKernelGGL((wf::kv_unpack_kernel<wf::kUnpackNtLoad, wf::kUnpackNtStore>), grid, dim3(256), 0,
                     wf::as_stream(stream), wf::PoolView{const_cast<uint8_t*>(k_codes), const_cast<float*>(k_scales)},
                     wf::PoolView{const_cast<uint8_t*>(v_codes), const_cast<float*>(v_scales)}, n_rows, n_blocks, items, geom,
                     reinterpret_cast<uint4*>(k_out), reinterpret_cast<uint4*>(v_out));
  return wf::check_launch(fn);
}

}  // extern "C"

#ifdef WF_HBM_PROBE
// Instrumented build only (not declared in wf_api.h): the HBM ceilings for the pack's and the unpack's traffic
// mixes.  wf_probe_stream_2to1: each thread reads 16 bytes and writes 8 per iteration (the high bytes of eight
// bf16, a stand-in for the pack's 2 : 1 read : write ratio), fully coalesced, grid-stride over n 16-byte
// items; wf_probe_stream_1to2: reads 8 and writes 16 (eight bytes widened to bf16 high bytes, the unpack's
// 1 : 2); `nontemporal` marks the stores as streaming.  waveforcing_amd/hbm_ceiling.py sweeps the grid and
// times them beside the pack and the unpack.
namespace wf {
namespace {
template <bool NT>
__global__ __launch_bounds__(256) void stream_2to1_kernel(const uint4* __restrict__ src, uint2* __restrict__ dst,
                                                          int64_t n) {
  typedef unsigned int u2v __attribute__((ext_vector_type(2)));
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const uint4 v = src[i];
    const u2v w = {(v.x >> 8 & 0xffu) | (v.x >> 16 & 0xff00u) | (v.y << 8 & 0xff0000u) | (v.y & 0xff000000u),
                   (v.z >> 8 & 0xffu) | (v.z >> 16 & 0xff00u) | (v.w << 8 & 0xff0000u) | (v.w & 0xff000000u)};
    if constexpr (NT)
      __builtin_nontemporal_store(w, reinterpret_cast<u2v*>(dst) + i);
    else
      *reinterpret_cast<u2v*>(dst + i) = w;
  }
}
template <bool NT>
__global__ __launch_bounds__(256) void stream_1to2_kernel(const uint2* __restrict__ src, uint4* __restrict__ dst,
                                                          int64_t n) {
  typedef unsigned int u4v __attribute__((ext_vector_type(4)));
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const uint2 v = src[i];
    const u4v w = {(v.x & 0xffu) << 8 | (v.x & 0xff00u) << 16, (v.x >> 8 & 0xff00u) | (v.x & 0xff000000u),
                   (v.y & 0xffu) << 8 | (v.y & 0xff00u) << 16, (v.y >> 8 & 0xff00u) | (v.y & 0xff000000u)};
    if constexpr (NT)
      __builtin_nontemporal_store(w, reinterpret_cast<u4v*>(dst) + i);
    else
      *reinterpret_cast<u4v*>(dst + i) = w;
  }
}
}  // namespace
}  // namespace wf

extern "C" int wf_probe_stream_1to2(const void* src, void* dst, int64_t n, int32_t grid, int32_t nontemporal,
                                    void* stream) {
  WF_REQUIRE(src && dst && n > 0 && grid > 0, WF_E_INVALID, "wf_probe_stream_1to2: bad arguments");
  WF_REQUIRE((reinterpret_cast<uintptr_t>(src) & 7u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0,
             WF_E_ALIGN, "wf_probe_stream_1to2: src must be 8-byte and dst 16-byte aligned");
  const auto* s = static_cast<const uint2*>(src);
  auto* d = static_cast<uint4*>(dst);
  if (nontemporal)
    hipLaunchKernelGGL(wf::stream_1to2_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                       wf::as_stream(stream), s, d, n);
  else
    hipLaunchKernelGGL(wf::stream_1to2_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                       wf::as_stream(stream), s, d, n);
  return wf::check_launch("wf_probe_stream_1to2");
}

extern "C" int wf_probe_stream_2to1(const void* src, void* dst, int64_t n, int32_t grid, int32_t nontemporal,
                                    void* stream) {
  WF_REQUIRE(src && dst && n > 0 && grid > 0, WF_E_INVALID, "wf_probe_stream_2to1: bad arguments");
  WF_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0,
             WF_E_ALIGN, "wf_probe_stream_2to1: src must be 16-byte and dst 8-byte aligned");
  const auto* s = static_cast<const uint4*>(src);
  auto* d = static_cast<uint2*>(dst);
  if (nontemporal)
    hipLaunchKernelGGL(wf::stream_2to1_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                       wf::as_stream(stream), s, d, n);
  else
    hipLaunchKernelGGL(wf::stream_2to1_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                       wf::as_stream(stream), s, d, n);
  return wf::check_launch("wf_probe_stream_2to1");
}
#endif
