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
// Work split: a workgroup of 8 waves owns 256 queries of one head; each wave
// owns 32 queries.  Keys advance in tiles of 64.  Thread t of the workgroup
// stages key t/8, d-chunk t%8 (16 codes) of both K and V for every tile:
// one 16-byte code load per pool, one scale load per pool (keys past n_kv or
// on invalid pages read as zero through the buffer descriptors), then
// bf16(code * s) into LDS as [key][d] rows.  The loads of tile i+2 fly while
// tile i computes, and tile i+1 is dequantized into the other LDS stage
// while the score matrix products of tile i run.
//
// The score block is computed transposed, S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16 (K fragment first operand, Q^T fragment second,
// Q^T kept in registers for the whole kernel): each lane then holds one
// query column and 16 keys per 32-key block, so the row max is an in-lane
// max plus one v_permlane32_swap with lane ^ 32, and the lane's P values
// are directly the second operand of O^T = V^T P^T.  The V^T operand is
// read from the [key][d] rows with ds_read_b64_tr_b16 (a 16-lane transposing
// read), the source rows chosen so the key order of each lane's operand
// matches its P registers.
//
// Schedule of one tile (straight-line apart from the rare rescale; the last
// tile is peeled for the masking of keys past n_kv, tiles past the end load
// as zeros into the stage nobody reads any more):
//   * the 16 K fragments are read first, then the 16 score MFMAs alternate
//     with the next tile's dequantization (sched_group_barrier: 1 MFMA, 4
//     VALU), whose result is then written to the other stage;
//   * the 32 V^T reads are issued before the softmax, so they land during it;
//   * each 16-key step's exponentials feed its 4 PV MFMAs, so the
//     exponentials of step t+1 issue under the MFMAs of step t.
// A wave issues a VALU instruction at most every ~8 cycles on gfx950, so
// the vector work only hides when it sits between the wave's own MFMAs.
//
// Softmax in base 2 with the scale folded into one FMA per score, and lazy
// rescaling: a query's running maximum used in the exponent is raised only
// when its tile maximum exceeds it by more than kTau (log2 units), so
// P <= 2^kTau and the O / row-sum rescale is rare; the final normalisation
// divides by the row sum taken against the same maximum, so the result is
// unchanged.  The decision is per query, so every output row depends only on
// its own query and the context.
// K stays exactly bf16(code * s): with heavy-tailed K the scores reach
// magnitudes where any further rounding of K (e.g. folding the scale into
// it) moves P by percents.
#include <utility>

#include "fastdiv.hpp"
#include "fp8_codec.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef short v2s16 __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int D = 128;
constexpr int BKV = 64;                 // keys per tile
constexpr int WAVES = 8;
constexpr int THREADS = WAVES * 64;     // one (key, 16-d chunk) of the tile per thread
constexpr int BQ = WAVES * 32;          // queries per workgroup
constexpr int KP = D * 2 + 16;          // K row pitch (bytes) = 272
constexpr int VP = D * 2 + 64;          // V row pitch (bytes) = 320: the 4 rows one
                                        // half-wave reads per transposing load are
                                        // 64 bytes apart modulo 256 (no bank overlap)
constexpr int K_TILE = BKV * KP;
constexpr int V_TILE = BKV * VP;
constexpr int STAGE = K_TILE + V_TILE;
// The quantized-QK form keeps K as e4m3 codes in LDS: [key][d] rows of 128 codes at a 144-byte pitch (the 16-byte
// fragment reads of 16 consecutive rows then start 36 dwords apart, on 16 distinct 4-bank groups), then V as
// above, then the tile's 64 K scales.
constexpr int KP8 = D + 16;
constexpr int K8_TILE = BKV * KP8;
constexpr int KS_BYTES = BKV * 4;
constexpr int STAGE8 = K8_TILE + V_TILE + KS_BYTES;
// The fp8-PV form keeps V as codes too: [key][d] rows of 128 codes whose four 32-byte d blocks are permuted per
// key (block db of key k at position db ^ sig(k), sig(k) = bit 1 of k | bit 3 of k << 1), so the transposing
// 8-byte reads of a half-wave (8 keys x 32 bytes) fall on 64 distinct banks; after V the tile's u_k and V scales.
constexpr int V8_TILE = BKV * D;
constexpr int STAGE_PV8 = K8_TILE + V8_TILE + 2 * KS_BYTES;
constexpr int OPITCH = D * 2 + 8;       // staged output row pitch (bytes)
constexpr int OUT_STAGING = WAVES * 32 * OPITCH;
constexpr int kBufferRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kOutOfRange = 0x7ffffff0;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kTau = 8.0f;            // lazy-rescale threshold, log2 units
static_assert(THREADS == BKV * 8, "one thread per (key, 16-d chunk)");

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

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ inline uint32_t cvt_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf));
}

// Dequantize 4 e4m3 codes (bytes of w) with one scale into 2 dwords of
// packed bf16: bf16_rne(float(code) * s), the pages' gather-dequant value.
__device__ inline uint2 dequant4_bf16(uint32_t w, float s) {
  float a, b, c, d;
  e4m3_unpack4_hw(w, a, b, c, d);
  return make_uint2(cvt_bf16x2(a * s, b * s), cvt_bf16x2(c * s, d * s));
}

// Sum of the two bf16 halves of x, added to acc (v_dot2c_f32_bf16 with 1.0).
__device__ inline float add_bf16x2(uint32_t x, float acc) {
  const v2bf one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, x), one, acc, false);
}

// 4 bf16 of a transposing LDS read (see the V^T operand below).
__device__ inline v4s read_tr(const uint8_t* addr) {
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(addr));
}

// 8 bytes of an 8-bit transposing LDS read (ds_read_b64_tr_b8): within each 16-lane group, lane i receives
// byte i % 8 of the 8-byte chunks addressed by lanes 2 j + i / 8 as its bytes j = 0..7.
__device__ inline v2i read_tr8(const uint8_t* addr) {
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(addr));
}

// max / sum of v over lanes l and l ^ 32 (v_permlane32_swap): a lane's two
// halves of a score column.  The swap is inline asm: the ROCm 7.2 compiler
// reads both results of __builtin_amdgcn_permlane32_swap from the
// destination register (r0 + r1 becomes 2 r0).  The s_nop is the VALU ->
// permlane wait state the compiler emits before the builtin; the asm is not
// volatile, so it schedules like any other instruction.
__device__ inline void swap_halves(float& lo, float& hi) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
}
__device__ inline float pair_max(float v) {
  float a = v, b = v;
  swap_halves(a, b);
  return fmaxf(a, b);
}
__device__ inline float pair_sum(float v) {
  float a = v, b = v;
  swap_halves(a, b);
  return a + b;
}

// QK8: the quantized-QK form (the counterpart of the reference's SageAttention backend, backend.py:57-62,
// 144-146).  Each query is quantized once to e4m3 with a power-of-two scale s_q = 2^e_q, the smallest with
// amax|q| <= 448 s_q (the codes are the e4m3 rounding of q 2^-e_q, an exact scaling), the e4m3 K codes of the
// pages are used as they are, and S^T = K_codes Q_codes^T runs on the fp8 matrix cores
// (v_mfma_scale_f32_32x32x64_f8f6f4), which apply 2^e_q to each query's column as its block scale.  The
// staging stores u_k = s_k * softmax scale * log2(e) per key, the same for every query, so a score's exponent
// is one FMA, s'' u_k - m; the tile's maximum is bounded by max s'' * max u_k (exact maxima only in the rare
// rescale).  V and P stay exact as in the bf16 form.
//
// PV8 (with QK8): the fp8-PV form, the counterpart of the fp8 P.V product of the reference's SageAttention
// backend.  V stays as the pages' codes in LDS and O^T += V^T P^T runs on the fp8 matrix cores too: the key
// scale s_v goes into P, each query's 64 values p_k s_v,k of a tile are rounded to e4m3 after division by
// 2^E, the smallest power of two that brings their maximum to <= 448 (the same rule as the queries'), and 2^E
// is the MFMA's block scale of that query's column.  The row sum stays the fp32 sum of the unrounded p_k.
template <bool DENSE, bool QK8, bool PV8>
__global__ __launch_bounds__(THREADS, 1) void attn_paged_fp8_kernel(AttnArgs p) {
  static_assert(!(DENSE && QK8), "the quantized-QK form reads FP8 pages");
  static_assert(!PV8 || QK8, "the fp8-PV form extends the quantized-QK form");
  constexpr int kStage = PV8 ? STAGE_PV8 : QK8 ? STAGE8 : STAGE;
  constexpr int kVOff = QK8 ? K8_TILE : K_TILE;              // V rows within a stage
  constexpr int kSOff = K8_TILE + (PV8 ? V8_TILE : V_TILE);  // u_k within a stage (QK8)
  constexpr int kVSOff = kSOff + KS_BYTES;                   // V scales within a stage (PV8)
  constexpr int kLds = 2 * kStage > OUT_STAGING ? 2 * kStage : OUT_STAGING;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];

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

  // ---- staging role: key skey of the tile, d = 16 * schunk .. + 15 ---------
  const int skey = tid >> 3;
  const int schunk = tid & 7;
  const int HD = p.H * D;
  const int lane_co = skey * HD + schunk * 16;  // this thread's key row within a page, codes
  const int lane_so = skey * 4;                 // and scales

  __amdgpu_buffer_rsrc_t rk, rv, rsk, rsv;
  if constexpr (DENSE) {
    const int kv_bytes = p.n_kv * static_cast<int>(p.ldkv) * 2;
    rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.k_dense), 0, kv_bytes, kBufferRsrcWord3);
    rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.v_dense), 0, kv_bytes, kBufferRsrcWord3);
    rsk = rk;
    rsv = rv;
  } else {
    const int64_t pool_bytes = static_cast<int64_t>(p.pool_pages) * p.page_tokens * HD;
    rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.k_codes), 0, static_cast<int>(pool_bytes),
                                           kBufferRsrcWord3);
    rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.v_codes), 0, static_cast<int>(pool_bytes),
                                           kBufferRsrcWord3);
    const int scale_bytes = p.pool_pages * p.H * p.page_tokens * 4;
    rsk = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.k_scales), 0, scale_bytes, kBufferRsrcWord3);
    rsv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.v_scales), 0, scale_bytes, kBufferRsrcWord3);
  }

  // One tile's staging registers: 16 codes (or 2 x 8 bf16) of K and of V, and the scales.
  u32x4 sk0, sv0, sk1, sv1;
  float ssk = 0.f, ssv = 0.f;

  // Page cursor of a tile (uniform across the workgroup): keys [0, split) of a tile starting at key t0 sit
  // on the physical page of logical page lp from row r0 (split = page_tokens - r0), keys [split, 64) on
  // the next logical page's from row 0 (a 64-key tile spans at most two pages: page_tokens >= 64,
  // checked on the host).  cb0 / cb1 and sb0 / sb1 are the code and scale byte offsets a lane adds its
  // key's row offset to (codes: skey * H * D + h * D + 16 schunk; scales: 4 skey), pushed beyond the
  // buffer ranges (>= kOutOfRange > pool size, reading as zero) for an invalid page.  The bases are
  // uint32: cb1 / sb1 wrap below zero when the next page is physical page 0 and a lane adds at least
  // `split` rows back; an out-of-range base plus a row offset stays above every buffer range.
  struct Cursor {
    int r0;
    uint32_t cb0, cb1, sb0, sb1;
  };
  // With the page lookups: the first tile and every tile that starts on a new page.  The lookups are
  // awaited here (the empty asm uses them), never across the next tile's LDS reads: a page-table load
  // in flight there turns the waits for its K-fragment reads into waits for everything (it counts in
  // lgkmcnt with them and returns out of order).
  auto cursor_at = [&](int t0) -> Cursor {
    if constexpr (DENSE) {
      (void)t0;
      return Cursor{0, 0u, 0u, 0u, 0u};
    } else {
      uint32_t lp, rip;
      p.page_div.divmod(static_cast<uint32_t>(t0), lp, rip);
      const int lpi = static_cast<int>(lp), r0 = static_cast<int>(rip);
      const int last = p.n_table - 1;  // >= 0 whenever n_kv > 0
      const int pg0 = p.table[min(lpi, last)];
      const int pg1 = p.table[min(lpi + 1, last)];
      asm volatile("" ::"s"(pg0), "s"(pg1));
      const bool ok0 = lpi <= last && pg0 >= 0 && pg0 < p.pool_pages;
      const bool ok1 = lpi + 1 <= last && pg1 >= 0 && pg1 < p.pool_pages;
      const int split = p.page_tokens - r0;
      // Bit masks rather than conditionals keep the compiler from branching around the multiplies.
      const uint32_t m0 = 0u - static_cast<uint32_t>(ok0), m1 = 0u - static_cast<uint32_t>(ok1);
      const int q0 = pg0 & static_cast<int>(m0), q1 = pg1 & static_cast<int>(m1);
      const uint32_t far0 = static_cast<uint32_t>(kOutOfRange) & ~m0, far1 = static_cast<uint32_t>(kOutOfRange) & ~m1;
      return Cursor{r0,
                    (static_cast<uint32_t>((q0 * p.page_tokens + r0) * HD + h * D) & m0) | far0,
                    (static_cast<uint32_t>((q1 * p.page_tokens - split) * HD + h * D) & m1) | far1,
                    (static_cast<uint32_t>(((q0 * p.H + h) * p.page_tokens + r0) * 4) & m0) | far0,
                    (static_cast<uint32_t>(((q1 * p.H + h) * p.page_tokens - split) * 4) & m1) | far1};
    }
  };
  // The cursor of the tile after c's, at key t0n = c's + 64.  Within a page only the bases move: 64 rows
  // of codes (64 H D bytes) and of scales (256 bytes) on both pages (split shrinks by 64).  A far base
  // stays far: a page holds fewer than 2^31 bytes, so at most that much is added to kOutOfRange before
  // the next page starts, below 2^32.
  auto cursor_next = [&](const Cursor& c, int t0n) -> Cursor {
    if constexpr (DENSE) {
      (void)t0n;
      return c;
    } else {
      if (c.r0 + BKV >= p.page_tokens) return cursor_at(t0n);
      const uint32_t dc = static_cast<uint32_t>(BKV * HD), ds = static_cast<uint32_t>(BKV * 4);
      return Cursor{c.r0 + BKV, c.cb0 + dc, c.cb1 + dc, c.sb0 + ds, c.sb1 + ds};
    }
  };

  // Issue the loads of the tile starting at key t0 (cursor c).
  auto load_tile = [&](int t0, const Cursor& c) {
    if constexpr (DENSE) {
      (void)c;
      const int key = min(t0 + skey, p.n_kv);
      const uint32_t off = static_cast<uint32_t>((key * static_cast<int>(p.ldkv) + h * D + schunk * 16) * 2) +
                           (key < p.n_kv ? 0u : static_cast<uint32_t>(kOutOfRange));
      sk0 = __builtin_amdgcn_raw_buffer_load_b128(rk, static_cast<int>(off), 0, 0);
      sk1 = __builtin_amdgcn_raw_buffer_load_b128(rk, static_cast<int>(off + 16), 0, 0);
      sv0 = __builtin_amdgcn_raw_buffer_load_b128(rv, static_cast<int>(off), 0, 0);
      sv1 = __builtin_amdgcn_raw_buffer_load_b128(rv, static_cast<int>(off + 16), 0, 0);
    } else {
      // Branch-free: keys past n_kv are pushed out of range like an invalid page.
      const bool first = skey < p.page_tokens - c.r0;
      const uint32_t lm = 0u - static_cast<uint32_t>(skey < p.n_kv - t0);   // all ones for keys before n_kv
      const uint32_t lfar = static_cast<uint32_t>(kOutOfRange) & ~lm;
      const uint32_t co = (((first ? c.cb0 : c.cb1) + static_cast<uint32_t>(lane_co)) & lm) | lfar;
      const uint32_t so = (((first ? c.sb0 : c.sb1) + static_cast<uint32_t>(lane_so)) & lm) | lfar;
      sk0 = __builtin_amdgcn_raw_buffer_load_b128(rk, static_cast<int>(co), 0, 0);
      sv0 = __builtin_amdgcn_raw_buffer_load_b128(rv, static_cast<int>(co), 0, 0);
      ssk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsk, static_cast<int>(so), 0, 0));
      ssv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsv, static_cast<int>(so), 0, 0));
    }
  };

  // The staged tile as bf16 [key][d] row pieces (registers only), and their
  // write into LDS stage `buf`.
  auto dequant_tile = [&](uint4* out) {
    if constexpr (PV8) {
      // K and V codes as they are, u_k and the V scale alongside
      out[0] = make_uint4(sk0[0], sk0[1], sk0[2], sk0[3]);
      out[1] = make_uint4(__builtin_bit_cast(uint32_t, __fmul_rn(ssk, p.qk_scale)), __builtin_bit_cast(uint32_t, ssv),
                          0u, 0u);
      out[2] = make_uint4(sv0[0], sv0[1], sv0[2], sv0[3]);
    } else if constexpr (QK8) {
      // K codes as they are, the key's exponent factor u_k = s_k * softmax scale * log2(e) alongside; V as in
      // the bf16 form
      out[0] = make_uint4(sk0[0], sk0[1], sk0[2], sk0[3]);
      out[1] = make_uint4(__builtin_bit_cast(uint32_t, __fmul_rn(ssk, p.qk_scale)), 0u, 0u, 0u);
      const uint2 e = dequant4_bf16(sv0[0], ssv), f = dequant4_bf16(sv0[1], ssv);
      const uint2 g = dequant4_bf16(sv0[2], ssv), i = dequant4_bf16(sv0[3], ssv);
      out[2] = make_uint4(e.x, e.y, f.x, f.y);
      out[3] = make_uint4(g.x, g.y, i.x, i.y);
    } else if constexpr (DENSE) {
      out[0] = make_uint4(sk0[0], sk0[1], sk0[2], sk0[3]);
      out[1] = make_uint4(sk1[0], sk1[1], sk1[2], sk1[3]);
      out[2] = make_uint4(sv0[0], sv0[1], sv0[2], sv0[3]);
      out[3] = make_uint4(sv1[0], sv1[1], sv1[2], sv1[3]);
    } else {
      const uint2 a = dequant4_bf16(sk0[0], ssk), b = dequant4_bf16(sk0[1], ssk);
      const uint2 c = dequant4_bf16(sk0[2], ssk), d = dequant4_bf16(sk0[3], ssk);
      out[0] = make_uint4(a.x, a.y, b.x, b.y);
      out[1] = make_uint4(c.x, c.y, d.x, d.y);
      const uint2 e = dequant4_bf16(sv0[0], ssv), f = dequant4_bf16(sv0[1], ssv);
      const uint2 g = dequant4_bf16(sv0[2], ssv), i = dequant4_bf16(sv0[3], ssv);
      out[2] = make_uint4(e.x, e.y, f.x, f.y);
      out[3] = make_uint4(g.x, g.y, i.x, i.y);
    }
  };
  auto write_tile = [&](int buf, const uint4* v) {
    if constexpr (PV8) {
      uint8_t* sb = lds + buf * kStage;
      *reinterpret_cast<uint4*>(sb + skey * KP8 + schunk * 16) = v[0];
      if (schunk == 0) *reinterpret_cast<uint32_t*>(sb + kSOff + skey * 4) = v[1].x;
      if (schunk == 1) *reinterpret_cast<uint32_t*>(sb + kVSOff + skey * 4) = v[1].y;
      const int sig = ((skey >> 1) & 1) | ((skey >> 2) & 2);
      *reinterpret_cast<uint4*>(sb + kVOff + skey * D + (((schunk >> 1) ^ sig) << 5) + 16 * (schunk & 1)) = v[2];
      return;
    }
    uint4* dv = reinterpret_cast<uint4*>(lds + buf * kStage + kVOff + skey * VP + schunk * 32);
    if constexpr (QK8) {
      *reinterpret_cast<uint4*>(lds + buf * kStage + skey * KP8 + schunk * 16) = v[0];
      if (schunk == 0) *reinterpret_cast<uint32_t*>(lds + buf * kStage + kSOff + skey * 4) = v[1].x;
    } else {
      uint4* dk = reinterpret_cast<uint4*>(lds + buf * kStage + skey * KP + schunk * 32);
      dk[0] = v[0];
      dk[1] = v[1];
    }
    dv[0] = v[2];
    dv[1] = v[3];
  };
  auto store_tile = [&](int buf) {
    uint4 v[4];
    dequant_tile(v);
    write_tile(buf, v);
  };

  // ---- Q^T fragments for this wave's 32 queries (kept for the whole kernel)
  v8bf qf[QK8 ? 1 : 8];
  v8i qc[2];             // QK8: e4m3 codes of d = 64 m + 32 half + 0..31 (m = 0, 1)
  int q_scale = 127;     // QK8: the query's block scale for the MFMA, E8M0 (127 + e_q)
  if constexpr (QK8) {
    // lane (l32, half) holds d = 64 m + 32 half + 0..31 of query l32, the K positions its fp8 operand bytes
    // stand for (the K fragments below use the same assignment)
    const int q = q0 + wave * 32 + l32;
    const bool ok = q < p.Lq;
    const uint16_t* qp = p.q + static_cast<int64_t>(ok ? q : 0) * p.ldq + h * D + half * 32;
    uint4 raw[8];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        raw[4 * m + j] = *reinterpret_cast<const uint4*>(qp + 64 * m + 8 * j);
        if (!ok) raw[4 * m + j] = make_uint4(0, 0, 0, 0);
      }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo_to_f32(w[e])), fabsf(bf16_hi_to_f32(w[e]))));
    }
    amax = pair_max(amax);
    // e_q: amax = f 2^E with f in [0.5, 1); amax <= 448 2^e (448 = 0.875 2^9) holds from e = E - 9 when
    // f <= 0.875, else from e = E - 8.  A zero row keeps e_q = 0 (all codes zero).
    int e_q = 0;
    if (amax > 0.f) {
      const int E = __builtin_amdgcn_frexp_expf(amax);
      e_q = __builtin_amdgcn_frexp_mantf(amax) <= 0.875f ? E - 9 : E - 8;
      e_q = min(max(e_q, -127), 127);  // the E8M0 range
    }
    q_scale = 127 + e_q;
    auto code = [&](float v) { return fminf(fmaxf(__builtin_ldexpf(v, -e_q), -448.0f), 448.0f); };
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      uint32_t c8[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 r = raw[4 * m + j];
        c8[2 * j] = e4m3_pack4_hw(code(bf16_lo_to_f32(r.x)), code(bf16_hi_to_f32(r.x)), code(bf16_lo_to_f32(r.y)),
                                  code(bf16_hi_to_f32(r.y)));
        c8[2 * j + 1] = e4m3_pack4_hw(code(bf16_lo_to_f32(r.z)), code(bf16_hi_to_f32(r.z)),
                                      code(bf16_lo_to_f32(r.w)), code(bf16_hi_to_f32(r.w)));
      }
      qc[m] = v8i{static_cast<int>(c8[0]), static_cast<int>(c8[1]), static_cast<int>(c8[2]), static_cast<int>(c8[3]),
                  static_cast<int>(c8[4]), static_cast<int>(c8[5]), static_cast<int>(c8[6]), static_cast<int>(c8[7])};
    }
  } else {
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

  // Per-lane LDS byte offsets (within a stage).  K fragment of key block b,
  // d-step ks: row b*32 + l32, bytes 32 ks + 16 half.  V^T operand for d
  // block db, 16-key step t, read r (keys 0-3 / 4-7 of the lane's 8): the
  // transposing read gives lane i of a 16-lane group element (i % 4) of the
  // 8-byte chunk addressed by lane 4j + i / 4 as its element j.  Lane s of
  // group G points at row 16t + 8r + 4 (G / 2) + s / 4, d = 32 db + 16 (G % 2)
  // + 4 (s % 4): lane i then holds d = 32 db + 16 (G % 2) + i and keys
  // 16t + 8r + 4 half + j, the key order of its P registers.
  const int k_lane = QK8 ? l32 * KP8 + half * 32 : l32 * KP + half * 16;
  const int v_lane = kVOff + (4 * half + ((lane & 15) >> 2)) * VP + (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
  // PV8: the V^T operand of d block db gives lane (m, half) d = 32 db + m at 32 keys, its bytes 8 r + j (read r
  // = 0..3) for key 16 r + 8 (j / 4) + 4 half + j % 4, which is the key of P byte 8 r + j (P bytes 16 b + i are
  // the score registers s[b][i]).  Lane s of a 16-lane group therefore addresses key 16 r + key0 with
  // j = s / 2, at d = 32 db + 16 (group % 2) + 8 (s % 2), in the key's permuted d block.
  int v8_off[4];
  if constexpr (PV8) {
    const int jj = (lane & 15) >> 1;
    const int key0 = 8 * (jj >> 2) + 4 * half + (jj & 3);
    const int sig = ((jj >> 1) & 1) | ((jj >> 2) << 1);  // sig(16 r + key0)
    const int o8 = 16 * ((lane >> 4) & 1) + 8 * (lane & 1);
#pragma unroll
    for (int db = 0; db < 4; ++db) v8_off[db] = kVOff + key0 * D + ((db ^ sig) << 5) + o8;
  }

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  // Softmax state.  The bf16 form keeps its maxima in raw score units and scales by c in the exponent's
  // FMA; the QK8 form's scores enter the exponent through u_k, so its maxima are in exponent units (c = 1).
  const float c = QK8 ? 1.0f : p.qk_scale;
  float m_use = -INFINITY;  // maximum used in the exponents
  float m_thr = -INFINITY;  // rescale when a tile's maximum exceeds this
  float neg_mc = 0.f;       // -m_use * c
  float l_run = 0.f;        // this half's row sum (its 32 of every 64 keys)

  const int n_tiles = (p.n_kv + BKV - 1) / BKV;
  Cursor cur_next{};  // the cursor of the tile loaded in the next iteration

  // One tile: scores with the staging of the next tile (into the other stage,
  // freed by the last barrier) and the loads of the one after; the column
  // max and the rare rescale; then the exponentials with O^T += V^T P^T.
  // Straight-line apart from the rescale: tiles past the end load as zeros
  // and land in the stage nobody reads any more; the last tile is peeled for
  // the masking of keys past n_kv.
  auto body = [&](int it, auto LAST) {
    const int cur = it & 1;
    const uint8_t* st = lds + cur * kStage;

    uint4 nxt[4];
    v16f s[2];
    float4 skv[2][4];  // QK8: u_k of the lane's keys 32 b + 8 g + 4 half + 0..3
    if constexpr (QK8) {
      // K code fragments (32 bytes per MFMA: d = 64 m + 32 half + 0..31 of key 32 b + l32) and the lane's
      // key scales (the same 16 per half-wave: broadcast reads), all in flight before the first MFMA
      v8i kf8[2][2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const uint8_t* a = st + k_lane + b * 32 * KP8 + 64 * m;
          const v4i lo = *reinterpret_cast<const v4i*>(a);
          const v4i hi = *reinterpret_cast<const v4i*>(a + 16);
          kf8[b][m] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          skv[b][g] = *reinterpret_cast<const float4*>(st + kSOff + 4 * (32 * b + 8 * g + 4 * half));
      dequant_tile(nxt);
#pragma unroll
      for (int b = 0; b < 2; ++b) s[b] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          s[b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf8[b][m], qc[m], s[b], 0, 0, 0, 127, 0, q_scale);
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the 8 K-fragment and 8 scale reads first
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // then 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // and 8 VALU, alternating
      }
    } else {
      // K fragments of the tile, all in flight before the first MFMA.
      v8bf kf[2][8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          kf[b][ks] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(st + k_lane + b * 32 * KP + ks * 32));
      // S^T = K Q^T for 2 blocks of 32 keys, with the next tile's dequantization
      // (registers only) between the MFMAs.
      dequant_tile(nxt);
#pragma unroll
      for (int b = 0; b < 2; ++b) s[b] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int b = 0; b < 2; ++b) s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[b][ks], qf[ks], s[b], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the 16 K-fragment reads first
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // then 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // and 4 VALU, alternating
      }
    }
    // the next tile into the other stage (freed by the last barrier), the
    // loads of the one after, and this tile's V^T operands (in flight
    // during the softmax).
    write_tile(cur ^ 1, nxt);
    load_tile((it + 2) * BKV, cur_next);
    v8bf vf[PV8 ? 1 : 4][4];
    v8i vf8[4];
    float4 svv[2][4];  // PV8: s_v of the lane's keys 32 b + 8 g + 4 half + 0..3
    if constexpr (PV8) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint8_t* va = st + v8_off[db];
        const v2i r0 = read_tr8(va), r1 = read_tr8(va + 16 * D), r2 = read_tr8(va + 32 * D), r3 = read_tr8(va + 48 * D);
        vf8[db] = v8i{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
      }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          svv[b][g] = *reinterpret_cast<const float4*>(st + kVSOff + 4 * (32 * b + 8 * g + 4 * half));
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const uint8_t* va = st + v_lane + (16 * t) * VP + db * 64;
          const v4s lo = read_tr(va);
          const v4s hi = read_tr(va + 8 * VP);
          vf[t][db] = __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    }

    // QK8: u_k of the lane's 32 keys as an array (element 4 g + e of block b), 1 for keys past n_kv (whose
    // scale reads as zero: their masked score of -inf then still yields a zero weight)
    float u[2][16];
    if constexpr (QK8) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u[b][4 * g] = skv[b][g].x;
          u[b][4 * g + 1] = skv[b][g].y;
          u[b][4 * g + 2] = skv[b][g].z;
          u[b][4 * g + 3] = skv[b][g].w;
        }
    }
    if constexpr (decltype(LAST)::value) {
      const int key_base = it * BKV;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool past = key_base + b * 32 + g * 8 + half * 4 + e >= p.n_kv;
            s[b][4 * g + e] = past ? -INFINITY : s[b][4 * g + e];
            if constexpr (QK8) u[b][4 * g + e] = past ? 1.0f : u[b][4 * g + e];
          }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) mt = fmaxf(mt, s[b][e]);
    if constexpr (QK8) {
      // an upper bound of the half's largest exponent s'' u_k: max s'' times the largest u_k when max s'' >= 0,
      // else 0 (every exponent is negative); the exact maximum is taken only when the bound asks for a rescale
      float um = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) um = fmaxf(um, u[b][e]);
      mt = mt >= 0.f ? mt * um : 0.f;
    }
    mt = pair_max(mt);
    // exponents in base 2: p = 2^(c * (s - m_use)), c = softmax_scale * log2(e) >= 0 (QK8: 2^(s'' u_k - m_use)).
    // Each query decides for itself (the wave only branches when one of its queries rescales), so a query's
    // output does not depend on which queries share its wave.
    const bool fire = mt > m_thr;
    if (__ballot(fire)) {
      if constexpr (QK8) {
        float ex = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int e = 0; e < 16; ++e) ex = fmaxf(ex, s[b][e] * u[b][e]);
        mt = pair_max(ex);
      }
      const float m_new = fire ? fmaxf(m_use, mt) : m_use;
      const float alpha =
          !fire ? 1.f : (m_use == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(c * (m_use - m_new));
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
      l_run *= alpha;
      m_use = m_new;
      m_thr = m_new + kTau / c;
      neg_mc = (m_new == -INFINITY) ? 0.f : -m_new * c;
    }
    if constexpr (PV8) {
      // p_k (row sum) and p_k s_v,k; their maximum over the query's 64 keys (both halves) sets 2^E; the
      // e4m3 codes of p_k s_v,k / 2^E are P's bytes (byte 16 b + i = score register s[b][i])
      float pv[2][16];
      float ls[4];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float sv4[4] = {svv[b][g].x, svv[b][g].y, svv[b][g].z, svv[b][g].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float pe = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g + e], u[b][4 * g + e], neg_mc));
            ls[e] = (b == 0 && g == 0) ? pe : ls[e] + pe;
            pv[b][4 * g + e] = pe * sv4[e];
          }
        }
      l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
      float mx = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, pv[b][e]);
      mx = pair_max(mx);
      // E: mx = f 2^X with f in [0.5, 1); mx <= 448 2^E from E = X - 9 when f <= 0.875, else X - 8 (E = 0 for
      // an all-zero P); clamped to [-126, 127], where 2^E is a normal float and 127 + E an E8M0 scale
      int E = 0;
      if (mx > 0.f) {
        const int X = __builtin_amdgcn_frexp_expf(mx);
        E = __builtin_amdgcn_frexp_mantf(mx) <= 0.875f ? X - 9 : X - 8;
        E = min(max(E, -126), 127);
      }
      const float sc = __builtin_bit_cast(float, static_cast<uint32_t>(127 + E) << 23);  // 2^E
      int pw[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int b = w >> 2, i = 4 * (w & 3);
        // the first conversion's untouched high half is any value (here pv's own bits): the second overwrites it
        v2s16 t = __builtin_bit_cast(v2s16, pv[b][i]);
        t = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(t, pv[b][i], pv[b][i + 1], sc, false);
        t = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(t, pv[b][i + 2], pv[b][i + 3], sc, true);
        pw[w] = __builtin_bit_cast(int, t);
      }
      const v8i pb = {pw[0], pw[1], pw[2], pw[3], pw[4], pw[5], pw[6], pw[7]};
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf8[db], pb, o[db], 0, 0, 0, 127, 0, 127 + E);
      cur_next = cursor_next(cur_next, (it + 3) * BKV);
      __syncthreads();
      return;
    }
    // P for 16-key step t (keys 16t..16t+15 of the tile): elements 0-3 are
    // keys 4 half + 0..3, elements 4-7 keys 8 + 4 half + 0..3; each step's
    // P feeds its 4 PV MFMAs (O^T += V^T P^T: 4 blocks of 32 d).
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int b = t >> 1, g0 = 2 * (t & 1);
      float pv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (QK8) {
          pv[e] = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g0 + e], u[b][4 * g0 + e], neg_mc));
          pv[4 + e] = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g0 + 4 + e], u[b][4 * g0 + 4 + e], neg_mc));
        } else {
          pv[e] = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g0 + e], c, neg_mc));
          pv[4 + e] = __builtin_amdgcn_exp2f(fmaf(s[b][4 * g0 + 4 + e], c, neg_mc));
        }
      }
      const uint32_t w0 = cvt_bf16x2(pv[0], pv[1]), w1 = cvt_bf16x2(pv[2], pv[3]);
      const uint32_t w2 = cvt_bf16x2(pv[4], pv[5]), w3 = cvt_bf16x2(pv[6], pv[7]);
      const v8bf pf = __builtin_bit_cast(v8bf, make_uint4(w0, w1, w2, w3));
      l_run = add_bf16x2(w3, add_bf16x2(w2, add_bf16x2(w1, add_bf16x2(w0, l_run))));
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[t][db], pf, o[db], 0, 0, 0);
    }
    cur_next = cursor_next(cur_next, (it + 3) * BKV);
    __syncthreads();
  };

  if (n_tiles > 0) {
    cur_next = cursor_at(0);
    load_tile(0, cur_next);
    store_tile(0);
    cur_next = cursor_next(cur_next, BKV);
    load_tile(BKV, cur_next);
    cur_next = cursor_next(cur_next, 2 * BKV);
    __syncthreads();
    for (int it = 0; it + 1 < n_tiles; ++it) body(it, std::false_type{});
    body(n_tiles - 1, std::true_type{});
  }

  // normalize, stage through LDS as bf16 [query][d] rows (every wave its own 32 rows; the last
  // tile's barrier has retired every read of the stages), then store 256-byte row segments.
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  static_assert(OUT_STAGING <= kLds, "output staging fits the stages");
  uint8_t* ow = lds + wave * 32 * OPITCH;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 w = make_uint2(cvt_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                                 cvt_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv));
      *reinterpret_cast<uint2*>(ow + l32 * OPITCH + 64 * db + 16 * g + 8 * half) = w;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 2 * i + half;
    const uint2 w = *reinterpret_cast<const uint2*>(ow + row * OPITCH + 8 * l32);
    const int qr = q0 + wave * 32 + row;
    if (qr < p.Lq) *reinterpret_cast<uint2*>(p.out + static_cast<int64_t>(qr) * p.ldo + h * D + 4 * l32) = w;
  }
}

}  // namespace

template <bool DENSE, bool QK8, bool PV8>
int launch_attn(const AttnArgs& p, int64_t lq, int n_heads, hipStream_t stream) {
  const int64_t items = (lq + BQ - 1) / BQ * n_heads;
  const dim3 grid(static_cast<uint32_t>((items + 7) / 8 * 8));
  hipLaunchKernelGGL((attn_paged_fp8_kernel<DENSE, QK8, PV8>), grid, dim3(THREADS), 0, stream, p);
  return check_launch(DENSE  ? "wf_attn_dense_bf16"
                      : PV8 ? "wf_attn_paged_fp8_qkpv8"
                      : QK8 ? "wf_attn_paged_fp8_qk8"
                            : "wf_attn_paged_fp8");
}

}  // namespace wf

namespace {
// form: 0 the exact bf16 form, 1 quantized QK, 2 quantized QK and fp8 PV
int attn_paged_entry(const char* fn, int form, const void* q, int64_t lq, int32_t n_heads, int32_t head_dim,
                     int64_t ldq, const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales,
                     const float* v_scales, int64_t pool_pages, int32_t page_tokens, const int32_t* page_table,
                     int64_t n_table, int64_t n_kv, float softmax_scale, void* out, int64_t ldo, void* stream) {
  WF_REQUIRE(lq >= 0 && n_heads > 0 && n_kv >= 0 && page_tokens > 0 && n_table >= 0 && pool_pages >= 0,
             WF_E_INVALID, "%s: negative or zero size", fn);
  WF_REQUIRE(head_dim == wf::D, WF_E_SHAPE, "%s: head_dim=%d unsupported (must be 128)", fn, head_dim);
  WF_REQUIRE(softmax_scale >= 0.f && softmax_scale < 3.0e38f, WF_E_INVALID,
             "%s: softmax_scale=%g must be finite and non-negative", fn, static_cast<double>(softmax_scale));
  WF_REQUIRE(ldq >= static_cast<int64_t>(n_heads) * head_dim && ldo >= static_cast<int64_t>(n_heads) * head_dim,
             WF_E_INVALID, "%s: ldq/ldo smaller than n_heads*head_dim", fn);
  if (lq == 0) return WF_OK;
  WF_REQUIRE(q && out, WF_E_INVALID, "%s: null q/out", fn);
  WF_REQUIRE(n_kv == 0 || (k_codes && v_codes && k_scales && v_scales && page_table), WF_E_INVALID,
             "%s: null KV pool or page table", fn);
  WF_REQUIRE(page_tokens >= wf::BKV, WF_E_SHAPE, "%s: page_tokens=%d must be >= %d", fn, page_tokens, wf::BKV);
  WF_REQUIRE(n_kv < (1ll << 31) && lq < (1ll << 31) && n_table < (1ll << 31), WF_E_SHAPE, "%s: size too large", fn);
  WF_REQUIRE(n_table * page_tokens >= n_kv, WF_E_SHAPE, "%s: page table covers %lld keys < n_kv=%lld", fn,
             (long long)(n_table * page_tokens), (long long)n_kv);
  WF_REQUIRE(wf::product_below({pool_pages, page_tokens, n_heads, head_dim}, (1ll << 31) - 16), WF_E_SHAPE,
             "%s: a code pool of 2 GiB or more is not supported", fn);
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
  switch (form) {
    case 1: return wf::launch_attn<false, true, false>(p, lq, n_heads, wf::as_stream(stream));
    case 2: return wf::launch_attn<false, true, true>(p, lq, n_heads, wf::as_stream(stream));
    default: return wf::launch_attn<false, false, false>(p, lq, n_heads, wf::as_stream(stream));
  }
}
}  // namespace

extern "C" int wf_attn_paged_fp8(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                 const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales,
                                 const float* v_scales, int64_t pool_pages, int32_t page_tokens,
                                 const int32_t* page_table, int64_t n_table, int64_t n_kv, float softmax_scale,
                                 void* out, int64_t ldo, void* stream) {
  return attn_paged_entry("wf_attn_paged_fp8", 0, q, lq, n_heads, head_dim, ldq, k_codes, v_codes, k_scales,
                          v_scales, pool_pages, page_tokens, page_table, n_table, n_kv, softmax_scale, out, ldo,
                          stream);
}

extern "C" int wf_attn_paged_fp8_qk8(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                     const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales,
                                     const float* v_scales, int64_t pool_pages, int32_t page_tokens,
                                     const int32_t* page_table, int64_t n_table, int64_t n_kv, float softmax_scale,
                                     void* out, int64_t ldo, void* stream) {
  return attn_paged_entry("wf_attn_paged_fp8_qk8", 1, q, lq, n_heads, head_dim, ldq, k_codes, v_codes, k_scales,
                          v_scales, pool_pages, page_tokens, page_table, n_table, n_kv, softmax_scale, out, ldo,
                          stream);
}

extern "C" int wf_attn_paged_fp8_qkpv8(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                       const uint8_t* k_codes, const uint8_t* v_codes, const float* k_scales,
                                       const float* v_scales, int64_t pool_pages, int32_t page_tokens,
                                       const int32_t* page_table, int64_t n_table, int64_t n_kv,
                                       float softmax_scale, void* out, int64_t ldo, void* stream) {
  return attn_paged_entry("wf_attn_paged_fp8_qkpv8", 2, q, lq, n_heads, head_dim, ldq, k_codes, v_codes, k_scales,
                          v_scales, pool_pages, page_tokens, page_table, n_table, n_kv, softmax_scale, out, ldo,
                          stream);
}

extern "C" int wf_attn_dense_bf16(const void* q, int64_t lq, int32_t n_heads, int32_t head_dim, int64_t ldq,
                                  const void* k, const void* v, int64_t n_kv, int64_t ldkv, float softmax_scale,
                                  void* out, int64_t ldo, void* stream) {
  static const char* fn = "wf_attn_dense_bf16";
  WF_REQUIRE(lq >= 0 && n_heads > 0 && n_kv >= 0, WF_E_INVALID, "%s: negative or zero size", fn);
  WF_REQUIRE(head_dim == wf::D, WF_E_SHAPE, "%s: head_dim=%d unsupported (must be 128)", fn, head_dim);
  WF_REQUIRE(softmax_scale >= 0.f && softmax_scale < 3.0e38f, WF_E_INVALID,
             "%s: softmax_scale=%g must be finite and non-negative", fn, static_cast<double>(softmax_scale));
  const int64_t hd = static_cast<int64_t>(n_heads) * head_dim;
  WF_REQUIRE(ldq >= hd && ldo >= hd && ldkv >= hd, WF_E_INVALID, "%s: row strides smaller than n_heads*head_dim", fn);
  if (lq == 0) return WF_OK;
  WF_REQUIRE(q && out && (n_kv == 0 || (k && v)), WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(wf::product_below({n_kv, ldkv, 2}, (1ll << 31) - 16) && lq < (1ll << 31), WF_E_SHAPE,
             "%s: K/V of 2 GiB or more", fn);
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
  return wf::launch_attn<true, false, false>(p, lq, n_heads, wf::as_stream(stream));
}
