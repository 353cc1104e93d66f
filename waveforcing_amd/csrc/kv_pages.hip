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
// |x| / s is the correctly rounded fp32 quotient: q = |x| * r with
// r = RN(1/s), then one residual step q += fma(-q, s, |x|) * r.  The
// quotient of two 8-bit significands is either exact (and the residual step
// returns it exactly) or at least 2^-14 (relative) away from every e4m3
// rounding boundary, so the code equals that of the IEEE quotient.
#include "fastdiv.hpp"
#include "fp8_codec.hpp"
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

__device__ inline uint32_t quant4(uint32_t w01, uint32_t w23, float s, float r) {
  const float x[4] = {bf16_lo_to_f32(w01), bf16_hi_to_f32(w01), bf16_lo_to_f32(w23), bf16_hi_to_f32(w23)};
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

__device__ inline float absmax8(const uint4& a, const uint4& b) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo_to_f32(w[i])), fabsf(bf16_hi_to_f32(w[i]))));
  return m;
}

__device__ inline float scale_from_amax(float amax) {
  const float s = bf16_bits_to_f32(f32_to_bf16_rne(__fdiv_rn(amax, kE4M3Max)));
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

template <bool NT_LOAD, bool NT_STORE>
__global__ __launch_bounds__(256) void kv_pack_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                                                      int64_t ld_kv, uint32_t n_rows, uint32_t n_blocks,
                                                      uint32_t n_items, PageGeom geom, PoolView kpool,
                                                      PoolView vpool) {
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
  }
  // every lane of the 8-lane group takes part in the reduction
  const float amax = group8_max(absmax8(a, b));
  const float s = scale_from_amax(amax);
  const float rcp = __frcp_rn(s);
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
  WF_REQUIRE(n_tokens * n_heads < (1ll << 31), WF_E_SHAPE, "%s: n_tokens*n_heads=%lld exceeds 2^31", fn,
             (long long)(n_tokens * n_heads));
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

}  // namespace
}  // namespace wf

extern "C" {

int wf_fp8_kv_pack(const void* k, const void* v, int64_t n_tokens, int32_t n_heads, int32_t head_dim,
                   int64_t ld_kv, const int32_t* page_table, int64_t n_table, int32_t page_tokens, uint8_t* k_codes,
                   uint8_t* v_codes, float* k_scales, float* v_scales, int64_t pool_pages, void* stream) {
  static const char* fn = "wf_fp8_kv_pack";
  if (int st = wf::check_pool_args(fn, n_tokens, n_heads, head_dim, page_table, n_table, page_tokens, pool_pages))
    return st;
  if (n_tokens == 0) return WF_OK;
  WF_REQUIRE(k && k_codes && k_scales, WF_E_INVALID, "%s: null K pointer", fn);
  WF_REQUIRE(ld_kv >= static_cast<int64_t>(n_heads) * head_dim && ld_kv % 8 == 0, WF_E_INVALID,
             "%s: ld_kv=%lld must be >= n_heads*head_dim and a multiple of 8", fn, (long long)ld_kv);
  const bool has_v = v != nullptr;
  WF_REQUIRE(!has_v || (v_codes && v_scales), WF_E_INVALID, "%s: V given without V pool", fn);
  WF_REQUIRE(wf::aligned16(k) && wf::aligned16(k_codes) && (!has_v || (wf::aligned16(v) && wf::aligned16(v_codes))),
             WF_E_ALIGN, "%s: K/V and code pools must be 16-byte aligned", fn);
  const uint32_t n_rows = static_cast<uint32_t>(n_tokens * n_heads);
  const wf::PageGeom geom = wf::make_geom(n_heads, page_table, n_table, page_tokens, pool_pages);
  const uint32_t n_blocks = (n_rows + wf::kRowsPerBlock - 1) / wf::kRowsPerBlock;
  const uint32_t items = has_v ? 2 * n_blocks : n_blocks;
  const dim3 grid((items + wf::kNumXcd - 1) / wf::kNumXcd * wf::kNumXcd);
  hipLaunchKernelGGL((wf::kv_pack_kernel<wf::kPackNtLoad, wf::kPackNtStore>), grid, dim3(256), 0,
                     wf::as_stream(stream), reinterpret_cast<const uint4*>(k), reinterpret_cast<const uint4*>(v), ld_kv,
                     n_rows, n_blocks, items, geom, wf::PoolView{k_codes, k_scales}, wf::PoolView{v_codes, v_scales});
  return wf::check_launch(fn);
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
