// Block-causal attention over the FP8 paged KV context (bf16 matrix cores).
//
//   out[q, h, :] = softmax_j( scale * <Q[q,h,:], K[j,h,:]> ) . V[j,h,:]
//   K[j,h,:] = code_k[j,h,:] * s_k[j,h],  V likewise (e4m3fn codes, fp32 scales)
//
// over the n_kv logical keys of a page table, with no mask inside the context:
// the reference's wavefront attention is non-causal (backend.py:141-148,
// causal=False) and block causality comes from which chunks the exchange
// puts into the context.  Restates the attention the reference dispatches
// (flash_attn_func / sageattn / SDPA, backend.py:141-148; the SDPA fallback
// naive_rt/rolling_forcing/wan/modules/attention.py:75-89) on the FP8 pages
// that replace the bf16 slab views of paged.py:246-247.
//
// Work split: a workgroup of WAVES waves owns 32 * WAVES queries of one
// head; each wave owns 32 queries.  Keys advance in tiles of 64.  Per tile the workgroup
// loads the K and V codes of the tile (through buffer descriptors over the
// pools: keys past n_kv or on invalid pages read as zero) and the per-key
// scales, dequantizes the codes once to bf16 into LDS, K as [key][d] and
// V transposed as [d][key'] with the key order permuted within each group of
// 16 (key bits 2 and 3 swapped) so that the PV operand fragment is one
// 16-byte read that matches the register layout of P.
//
// The score block is computed transposed, S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16 (K fragment first operand, Q^T fragment second,
// Q^T kept in registers for the whole kernel): each lane then holds one
// query column and 16 keys per 32-key block, so the online-softmax row max
// is an in-lane max plus one exchange with lane ^ 32, and the lane's P values
// are directly the second operand of O^T = V^T P^T.  K and V enter LDS as
// bf16(code * s), the pages' gather-dequant values; the softmax works in
// base 2 with the scale folded into one FMA per score.
#include <utility>

#include "fastdiv.hpp"
#include "fp8_codec.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int D = 128;
constexpr int BKV = 64;          // keys per tile
constexpr int KP = D * 2 + 16;   // K tile row pitch (bytes, bf16 + pad) = 272
constexpr int VP = BKV * 2 + 16; // V^T tile row pitch (bytes) = 144
constexpr int K_TILE = BKV * KP;
constexpr int V_TILE = D * VP;
constexpr int STAGE = K_TILE + V_TILE;
constexpr int kBufferRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kOutOfRange = 0x7ffffff0;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;  // bf16 [Lq, ldq_tok] with head h at offset h * D
  int64_t ldq;        // elements between consecutive query tokens
  const uint8_t* k_codes;
  const uint8_t* v_codes;
  const float* k_scales;
  const float* v_scales;
  const int32_t* table;
  const uint16_t* k_dense;  // dense bf16 K [n_kv, ldkv] (dense-context variant)
  const uint16_t* v_dense;
  int64_t ldkv;
  uint16_t* out;  // bf16 [Lq, ldo] with head h at offset h * D
  int64_t ldo;
  int Lq, H, n_kv, n_table, page_tokens, pool_pages;
  FastDiv page_div;
  float qk_scale;  // softmax scale * log2(e)
};

// XOR swizzle (in key positions, a multiple of 8 = one 16-byte fragment) of
// V^T row d: the transposing writes of lanes holding d, d+4, d+8, ... would
// otherwise all hit 4 bank groups; fragments stay contiguous 16-byte reads.
__device__ inline int vswz(int d) { return ((d >> 4) & 7) * 8; }

// Two fp32 holding e4m3-exact values -> packed bf16x2 (truncation is exact).
__device__ inline uint32_t f32x2_to_bf16x2_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
}

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ inline uint32_t cvt_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}

// Dequantize 4 e4m3 codes (bytes of w) with per-code scales into 2 dwords of
// packed bf16: bf16_rne(float(code) * s), the pages' gather-dequant value.
__device__ inline uint2 dequant4_bf16(uint32_t w, float s0, float s1, float s2, float s3) {
  float a, b, c, d;
  e4m3_unpack4_hw(w, a, b, c, d);
  return make_uint2(cvt_bf16x2(a * s0, b * s1), cvt_bf16x2(c * s2, d * s3));
}

// Decode 4 e4m3 codes (bytes of w) into 2 dwords of packed bf16.
__device__ inline uint2 decode4_bf16(uint32_t w) {
  float a, b, c, d;
  e4m3_unpack4_hw(w, a, b, c, d);
  return make_uint2(f32x2_to_bf16x2_exact(a, b), f32x2_to_bf16x2_exact(c, d));
}

template <int N, typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// WAVES waves of 32 queries each share one decoded K/V tile; PGR register
// buffers let the loads of tile it + PGR fly while tile it computes.
template <int WAVES, int PGR, bool DENSE>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void attn_paged_fp8_kernel(AttnArgs p) {
  constexpr int THREADS = WAVES * 64;
  constexpr int BQ = WAVES * 32;
  constexpr int KCH = BKV * 8 / THREADS;  // 16-code K chunks per thread per tile
  constexpr int VT = BKV * D / 16 / THREADS;  // 4-key x 4-d V tasks per thread per tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;
  // Work item w = head * q_tiles + q_tile.  Workgroups are dealt to the 8
  // XCDs round-robin (blockIdx % 8); each XCD gets a contiguous range of
  // work items, so the query tiles of one head share that head's K/V tiles
  // in one L2.
  const int q_tiles = (p.Lq + BQ - 1) / BQ;
  const int n_items = q_tiles * p.H;
  const int per_xcd = (n_items + 7) / 8;
  const int w_item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (w_item >= n_items) return;
  const int h = w_item / q_tiles;
  const int q0 = (w_item % q_tiles) * BQ;

  const int64_t pool_bytes = static_cast<int64_t>(p.pool_pages) * p.page_tokens * p.H * D;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.k_codes), 0,
                                                                      static_cast<int>(pool_bytes), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.v_codes), 0,
                                                                      static_cast<int>(pool_bytes), kBufferRsrcWord3);
  const int scale_bytes = p.pool_pages * p.H * p.page_tokens * 4;
  const __amdgpu_buffer_rsrc_t rsk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.k_scales), 0, scale_bytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.v_scales), 0, scale_bytes, kBufferRsrcWord3);

  // A 64-key tile spans at most two pages (page_tokens >= 64, checked on the
  // host).  map_tile resolves them once per tile into base offsets (uniform
  // across the workgroup); a key k of the tile is then one compare and one
  // multiply-add.  Offsets of keys past n_kv or on invalid pages are pushed
  // out of the buffer range, so they read as zero.
  const int HD = p.H * D;
  int t_split = 0, t_valid = 0, t_cb0 = 0, t_cb1 = 0, t_sb0 = 0, t_sb1 = 0;
  bool t_ok0 = false, t_ok1 = false;
  auto map_tile = [&](int t0) {
    uint32_t lp, rip;
    p.page_div.divmod(static_cast<uint32_t>(t0), lp, rip);
    const int pg0 = static_cast<int>(lp) < p.n_table ? p.table[lp] : -1;
    const int pg1 = static_cast<int>(lp) + 1 < p.n_table ? p.table[lp + 1] : -1;
    t_ok0 = pg0 >= 0 && pg0 < p.pool_pages;
    t_ok1 = pg1 >= 0 && pg1 < p.pool_pages;
    t_split = p.page_tokens - static_cast<int>(rip);
    t_valid = p.n_kv - t0;
    t_cb0 = t_ok0 ? ((pg0 * p.page_tokens + static_cast<int>(rip)) * p.H + h) * D : 0;
    t_cb1 = t_ok1 ? (pg1 * p.page_tokens * p.H + h) * D : 0;
    t_sb0 = t_ok0 ? ((pg0 * p.H + h) * p.page_tokens + static_cast<int>(rip)) * 4 : 0;
    t_sb1 = t_ok1 ? ((pg1 * p.H + h) * p.page_tokens) * 4 : 0;
  };
  auto key_offsets = [&](int k, int& code_off, int& scale_off) {
    const bool first = k < t_split;
    const bool ok = k < t_valid && (first ? t_ok0 : t_ok1);
    const int kr = first ? k : k - t_split;
    code_off = ok ? (first ? t_cb0 : t_cb1) + kr * HD : kOutOfRange;
    scale_off = ok ? (first ? t_sb0 : t_sb1) + kr * 4 : kOutOfRange;
  };

  // ---- per-thread staging of one K/V tile ----------------------------------
  // K: 2 x 16 codes (key = c / 8, d0 = 16 * (c % 8)), c = tid + 256 * i.
  // V: 2 tasks of 4 keys x 4 d (dword loads), task = tid + 256 * i:
  //    key group kg = task / 32 (keys 4kg..4kg+3), d = 4 * (task % 32).
  // Each thread also loads the scales of the keys it decodes.
  u32x4 rk_code[PGR][KCH];
  uint32_t rv_code[PGR][VT][4];
  float rk_s[PGR][KCH];
  float rv_s[PGR][VT][4];
  // second halves of the dense bf16 variant's staging (unused for FP8 pages)
  u32x4 rk_hi[DENSE ? PGR : 1][DENSE ? KCH : 1];
  uint32_t rv_hi[DENSE ? PGR : 1][DENSE ? VT : 1][4];

  auto load_tile = [&](auto buf, int t0) {
    constexpr int u = decltype(buf)::value;
    if constexpr (DENSE) {
      // K: 16 bf16 = two 16-byte halves per chunk; V: 4 keys x 4 d (8 bytes per key)
      const int kv_bytes = p.n_kv * static_cast<int>(p.ldkv) * 2;
      const __amdgpu_buffer_rsrc_t rkd =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.k_dense), 0, kv_bytes, kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t rvd =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.v_dense), 0, kv_bytes, kBufferRsrcWord3);
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int c = tid + THREADS * i;
        const int key = t0 + (c >> 3);
        const int off = key < p.n_kv ? (key * static_cast<int>(p.ldkv) + h * D + (c & 7) * 16) * 2 : kOutOfRange;
        rk_code[u][i] = __builtin_amdgcn_raw_buffer_load_b128(rkd, off, 0, 0);
        rk_hi[u][i] = __builtin_amdgcn_raw_buffer_load_b128(rkd, off == kOutOfRange ? off : off + 16, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < VT; ++i) {
        const int task = tid + THREADS * i;
        const int kg = task >> 5, d0 = (task & 31) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = t0 + 4 * kg + j;
          const int off = key < p.n_kv ? (key * static_cast<int>(p.ldkv) + h * D + d0) * 2 : kOutOfRange;
          const auto w2 = __builtin_amdgcn_raw_buffer_load_b64(rvd, off, 0, 0);
          rv_code[u][i][j] = w2[0];
          rv_hi[u][i][j] = w2[1];
        }
      }
      return;
    }
    map_tile(t0);
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + THREADS * i;
      int co, so;
      key_offsets(c >> 3, co, so);
      rk_code[u][i] = __builtin_amdgcn_raw_buffer_load_b128(rk, co == kOutOfRange ? co : co + (c & 7) * 16, 0, 0);
      rk_s[u][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsk, so, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < VT; ++i) {
      const int task = tid + THREADS * i;
      const int kg = task >> 5, d0 = (task & 31) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int co, so;
        key_offsets(4 * kg + j, co, so);
        rv_code[u][i][j] = __builtin_amdgcn_raw_buffer_load_b32(rv, co == kOutOfRange ? co : co + d0, 0, 0);
        rv_s[u][i][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsv, so, 0, 0));
      }
    }
  };

  auto store_tile = [&](auto buf, int lbuf) {
    constexpr int u = decltype(buf)::value;
    uint8_t* sk = lds + lbuf * STAGE;
    uint8_t* sv = sk + K_TILE;
    if constexpr (DENSE) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int c = tid + THREADS * i;
        uint4* dst = reinterpret_cast<uint4*>(sk + (c >> 3) * KP + (c & 7) * 32);
        dst[0] = make_uint4(rk_code[u][i][0], rk_code[u][i][1], rk_code[u][i][2], rk_code[u][i][3]);
        dst[1] = make_uint4(rk_hi[u][i][0], rk_hi[u][i][1], rk_hi[u][i][2], rk_hi[u][i][3]);
      }
#pragma unroll
      for (int i = 0; i < VT; ++i) {
        const int task = tid + THREADS * i;
        const int kg = task >> 5, d0 = (task & 31) * 4;
        const int pos = ((kg & ~3) * 4 + ((kg & 1) << 3) + ((kg & 2) << 1)) ^ vswz(d0);
        // key j holds d0, d0+1 in rv_code[j] and d0+2, d0+3 in rv_hi[j]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t* src = (j < 2) ? rv_code[u][i] : rv_hi[u][i];
          const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;  // high or low bf16 of each key word
          const uint32_t lo = __builtin_amdgcn_perm(src[1], src[0], sel);
          const uint32_t hi = __builtin_amdgcn_perm(src[3], src[2], sel);
          *reinterpret_cast<uint2*>(sv + (d0 + j) * VP + pos * 2) = make_uint2(lo, hi);
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + THREADS * i;
      const float ks = rk_s[u][i];
      const uint2 a = dequant4_bf16(rk_code[u][i][0], ks, ks, ks, ks);
      const uint2 b = dequant4_bf16(rk_code[u][i][1], ks, ks, ks, ks);
      const uint2 e = dequant4_bf16(rk_code[u][i][2], ks, ks, ks, ks);
      const uint2 f = dequant4_bf16(rk_code[u][i][3], ks, ks, ks, ks);
      uint4* dst = reinterpret_cast<uint4*>(sk + (c >> 3) * KP + (c & 7) * 32);
      dst[0] = make_uint4(a.x, a.y, b.x, b.y);
      dst[1] = make_uint4(e.x, e.y, f.x, f.y);
    }
#pragma unroll
    for (int i = 0; i < VT; ++i) {
      const int task = tid + THREADS * i;
      const int kg = task >> 5, d0 = (task & 31) * 4;
      // position of key group kg in the permuted order (swap of key bits 2, 3)
      const int pos = ((kg & ~3) * 4 + ((kg & 1) << 3) + ((kg & 2) << 1)) ^ vswz(d0);  // d0..d0+3 share vswz
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // byte j of the four key dwords = the codes of d0 + j for keys 4kg..4kg+3
        const uint32_t lo = __builtin_amdgcn_perm(rv_code[u][i][1], rv_code[u][i][0], 0x0c0c0400u + 0x00000101u * j);
        const uint32_t hi = __builtin_amdgcn_perm(rv_code[u][i][3], rv_code[u][i][2], 0x0c0c0400u + 0x00000101u * j);
        const uint2 dec = dequant4_bf16(lo | (hi << 16), rv_s[u][i][0], rv_s[u][i][1], rv_s[u][i][2], rv_s[u][i][3]);
        *reinterpret_cast<uint2*>(sv + (d0 + j) * VP + pos * 2) = dec;
      }
    }
  };

  // ---- Q^T fragments for this wave's 32 queries (kept for the whole kernel)
  v8bf qf[8];
  {
    const int q = q0 + wave * 32 + l32;
    const bool ok = q < p.Lq;
    const uint16_t* qp = p.q + static_cast<int64_t>(ok ? q : 0) * p.ldq + h * D + half * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      uint4 v = *reinterpret_cast<const uint4*>(qp + ks * 16);
      if (!ok) v = make_uint4(0, 0, 0, 0);
      qf[ks] = __builtin_bit_cast(v8bf, v);
    }
  }

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  float m_run = -INFINITY;
  float l_run = 0.f;

  const int n_tiles = (p.n_kv + BKV - 1) / BKV;
  // Tiles past the context read as zero (all keys masked by n_kv), so the
  // step count is padded to a multiple of PGR and every step is
  // unconditional.
  const int n_steps = (n_tiles + PGR - 1) / PGR * PGR;
  static_for<PGR>([&](auto u) { load_tile(u, u.value * BKV); });
  store_tile(std::integral_constant<int, 0>{}, 0);
  __syncthreads();

  for (int it0 = 0; it0 < n_steps; it0 += PGR) {
  static_for<PGR>([&](auto uu) {
    constexpr int U = decltype(uu)::value;
    const int it = it0 + U;
    const int cur = it & 1;
    load_tile(uu, (it + PGR) * BKV);
    const uint8_t* sk = lds + cur * STAGE;
    const uint8_t* sv = sk + K_TILE;

    // S^T = K Q^T for 2 blocks of 32 keys
    v16f s[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      s[b] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
      const uint8_t* kr = sk + (b * 32 + l32) * KP + half * 16;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const v8bf kf = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(kr + ks * 32));
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[b], 0, 0, 0);
      }
    }
    // masking of keys past n_kv (last tile only), tile max of the raw scores
    const int key_base = it * BKV;
    const bool partial = key_base + BKV > p.n_kv;
    float mt = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int kk = b * 32 + g * 8 + half * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (partial && key_base + kk + e >= p.n_kv) s[b][4 * g + e] = -INFINITY;
          mt = fmaxf(mt, s[b][4 * g + e]);
        }
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    // exponents in base 2: p = 2^(c * (s - m)), c = softmax_scale * log2(e) > 0
    const float c = p.qk_scale;
    const float m_new = fmaxf(m_run, mt);
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(c * (m_run - m_new));
    m_run = m_new;
    const float neg_mc = (m_new == -INFINITY) ? 0.f : -m_new * c;
    float lsum = 0.f;
    v8bf pf[4];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        uint32_t pk[4];
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2) {
          const int g = hh * 2 + g2;
          float pv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g + e], c, neg_mc));
            lsum += pv[e];
          }
          pk[2 * g2] = cvt_bf16x2(pv[0], pv[1]);
          pk[2 * g2 + 1] = cvt_bf16x2(pv[2], pv[3]);
        }
        pf[b * 2 + hh] = __builtin_bit_cast(v8bf, make_uint4(pk[0], pk[1], pk[2], pk[3]));
      }
    }
    l_run = l_run * alpha + lsum;
    if (__ballot(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
    }

    // O^T += V^T P^T : 4 blocks of 32 d, 4 steps of 16 keys
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = db * 32 + l32;
      const uint8_t* vr = sv + d * VP;
      const int sw = vswz(d);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v8bf vf = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(vr + (((t * 16 + half * 8) ^ sw) * 2)));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[t], o[db], 0, 0, 0);
      }
    }
    store_tile(std::integral_constant<int, (U + 1) % PGR>{}, cur ^ 1);
    __syncthreads();
  });
  }

  // normalize and store: lane's query q, d = 32*db + 8*(r/4) + 4*half + r%4
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const int q = q0 + wave * 32 + l32;
  if (q < p.Lq) {
    uint16_t* op = p.out + static_cast<int64_t>(q) * p.ldo + h * D + half * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint2 w = make_uint2(cvt_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                                   cvt_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv));
        *reinterpret_cast<uint2*>(op + db * 32 + g * 8) = w;
      }
    }
  }
}

}  // namespace

template <int WAVES, int PGR, bool DENSE = false>
int launch_attn(const AttnArgs& p, int64_t lq, int n_heads, hipStream_t stream) {
  const int64_t items = (lq + WAVES * 32 - 1) / (WAVES * 32) * n_heads;
  const dim3 grid(static_cast<uint32_t>((items + 7) / 8 * 8));
  hipLaunchKernelGGL((attn_paged_fp8_kernel<WAVES, PGR, DENSE>), grid, dim3(WAVES * 64), 0, stream, p);
  return check_launch(DENSE ? "wf_attn_dense_bf16" : "wf_attn_paged_fp8");
}

}  // namespace wf

extern "C" int wf_attn_paged_fp8(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                 const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales,
                                 const float* v_scales, int64_t pool_pages, int32_t page_tokens,
                                 const int32_t* page_table, int64_t n_table, int64_t n_kv, float softmax_scale,
                                 void* out, int64_t ldo, void* stream) {
  static const char* fn = "wf_attn_paged_fp8";
  WF_REQUIRE(lq >= 0 && n_heads > 0 && n_kv >= 0 && page_tokens > 0 && n_table >= 0 && pool_pages >= 0,
             WF_E_INVALID, "%s: negative or zero size", fn);
  WF_REQUIRE(head_dim == wf::D, WF_E_SHAPE, "%s: head_dim=%d unsupported (must be 128)", fn, head_dim);
  WF_REQUIRE(ldq >= static_cast<int64_t>(n_heads) * head_dim && ldo >= static_cast<int64_t>(n_heads) * head_dim,
             WF_E_INVALID, "%s: ldq/ldo smaller than n_heads*head_dim", fn);
  if (lq == 0) return WF_OK;
  WF_REQUIRE(q && out, WF_E_INVALID, "%s: null q/out", fn);
  WF_REQUIRE(n_kv == 0 || (k_codes && v_codes && k_scales && v_scales && page_table), WF_E_INVALID,
             "%s: null KV pool or page table", fn);
  WF_REQUIRE(page_tokens >= wf::BKV, WF_E_SHAPE, "%s: page_tokens=%d must be >= %d", fn, page_tokens, wf::BKV);
  WF_REQUIRE(n_table * page_tokens >= n_kv, WF_E_SHAPE, "%s: page table covers %lld keys < n_kv=%lld", fn,
             (long long)(n_table * page_tokens), (long long)n_kv);
  WF_REQUIRE(pool_pages * page_tokens * n_heads * head_dim < (1ll << 31) - 16, WF_E_SHAPE,
             "%s: a code pool of 2 GiB or more is not supported", fn);
  WF_REQUIRE(n_kv < (1ll << 31) && lq < (1ll << 31) && n_table < (1ll << 31), WF_E_SHAPE, "%s: size too large", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15u) == 0 && (ldq % 8) == 0 &&
                 (reinterpret_cast<uintptr_t>(out) & 7u) == 0 && (ldo % 4) == 0,
             WF_E_ALIGN, "%s: q must be 16-byte aligned (ldq %% 8 == 0), out 8-byte aligned (ldo %% 4 == 0)", fn);
  wf::AttnArgs p;
  p.q = static_cast<const uint16_t*>(q);
  p.ldq = ldq;
  p.k_codes = k_codes;
  p.v_codes = v_codes;
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  p.table = page_table;
  p.k_dense = nullptr;
  p.v_dense = nullptr;
  p.ldkv = 0;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.Lq = static_cast<int>(lq);
  p.H = n_heads;
  p.n_kv = static_cast<int>(n_kv);
  p.n_table = static_cast<int>(n_table);
  p.page_tokens = page_tokens;
  p.pool_pages = static_cast<int>(pool_pages);
  p.page_div = wf::FastDiv(static_cast<uint32_t>(page_tokens));
  p.qk_scale = softmax_scale * wf::kLog2e;
  // 8 waves (256 queries) share each decoded K/V tile, one tile of register
  // prefetch: the best of {4, 8} waves x {1, 2} tiles of prefetch measured on
  // the 1.3B / 14B context shapes.
  return wf::launch_attn<8, 1>(p, lq, n_heads, wf::as_stream(stream));
}

extern "C" int wf_attn_dense_bf16(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                  const void* k, const void* v, int64_t n_kv, int64_t ldkv, float softmax_scale,
                                  void* out, int64_t ldo, void* stream) {
  static const char* fn = "wf_attn_dense_bf16";
  WF_REQUIRE(lq >= 0 && n_heads > 0 && n_kv >= 0, WF_E_INVALID, "%s: negative or zero size", fn);
  WF_REQUIRE(head_dim == wf::D, WF_E_SHAPE, "%s: head_dim=%d unsupported (must be 128)", fn, head_dim);
  const int64_t hd = static_cast<int64_t>(n_heads) * head_dim;
  WF_REQUIRE(ldq >= hd && ldo >= hd && ldkv >= hd, WF_E_INVALID, "%s: row strides smaller than n_heads*head_dim", fn);
  if (lq == 0) return WF_OK;
  WF_REQUIRE(q && out && (n_kv == 0 || (k && v)), WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(n_kv * ldkv * 2 < (1ll << 31) - 16 && lq < (1ll << 31), WF_E_SHAPE, "%s: K/V of 2 GiB or more", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15u) == 0 && ldq % 8 == 0 && (reinterpret_cast<uintptr_t>(k) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(v) & 15u) == 0 && ldkv % 8 == 0 &&
                 (reinterpret_cast<uintptr_t>(out) & 7u) == 0 && ldo % 4 == 0,
             WF_E_ALIGN, "%s: q, k, v must be 16-byte aligned (strides %% 8 == 0), out 8-byte aligned", fn);
  wf::AttnArgs p{};
  p.q = static_cast<const uint16_t*>(q);
  p.ldq = ldq;
  p.k_dense = static_cast<const uint16_t*>(k);
  p.v_dense = static_cast<const uint16_t*>(v);
  p.ldkv = ldkv;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.Lq = static_cast<int>(lq);
  p.H = n_heads;
  p.n_kv = static_cast<int>(n_kv);
  p.page_tokens = 1;
  p.page_div = wf::FastDiv(1);
  p.qk_scale = softmax_scale * wf::kLog2e;
  return wf::launch_attn<8, 1, true>(p, lq, n_heads, wf::as_stream(stream));
}
