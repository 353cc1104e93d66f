// W8A8 GEMMs on the gfx950 matrix cores with fused dequant + bias epilogues.
//
// int8 (per-token / per-channel scales):
//   acc[m,n] = sum_k qx[m,k] * qw[n,k]                      (int32, exact)
//   y[m,n]   = bf16( (float(acc) * sx[m]) * sw[n] + bias[n] )  (fp32, this order,
//                                                             no fused multiply-add)
//   gelu:      y = bf16( gelu_tanh(float(y)) )
// the per-token / per-channel int8 counterpart of the reference's W8A8 linear
// (wave_rt/runtime/fp8.py:46-56) with the FFN's GELU(approximate='tanh')
// folded in (naive_rt/rolling_forcing/wan/modules/causal_model.py:342-344).
//
// e4m3 (per-tensor scales, the reference's own mode):
//   acc[m,n] = sum_k e4m3(a[m,k]) * e4m3(w[n,k])            (fp32)
//   y[m,n]   = bf16( acc * (s_a * s_w) + bias[n] )
// torch._scaled_mm(x_fp8, w_fp8.t(), scale_a, scale_b, bias, bf16) at
// wave_rt/runtime/fp8.py:49-56.
//
// Structure (one 128 x 256 or 256 x 256 output tile per workgroup of 8 waves,
// each wave 64 x 64 or 128 x 64 as 2 x 2 or 4 x 2 blocks of 32 x 32 MFMAs:
// v_mfma_i32_32x32x32_i8, or v_mfma_f32_32x32x64_f8f6f4 with e4m3 operands;
// both operands K-contiguous; the host plans the tiles per shape, see
// plan_tiles: one tile for the whole output, or whole rounds of 256-row
// tiles followed by a launch of 128-row tiles over the rest):
//  * Global -> LDS by DMA (buffer_load_dwordx4 ... lds): each instruction
//    moves 1 KB = 8 rows x 128 K-bytes into a contiguous LDS block, no
//    registers involved.  Lane l lands at byte 16 l, i.e. row l/8, position
//    l%8; it fetches K chunk (l%8) ^ ((row/2)%8), so LDS holds chunk c of row
//    r at 16 (c ^ ((r/2)%8)) and the 16-byte fragment reads of 16 consecutive
//    rows hit 16 distinct bank groups.  The buffer descriptor's range
//    zero-fills rows past M / N, and K-tail chunks are pointed past it.
//  * Prologue: the waves that win the issue arbitration of their SIMD (0..3)
//    fetch all of stage 0, their SIMD mates stage 1, so the first stage is
//    not queued behind the second.
//  * Three LDS stages of 48 KB (the 256-row tile: two of 64 KB, see Tile).  A K step (128 bytes) is SUB sub-steps of one
//    MFMA depth (4 x 32 bytes for int8, 2 x 64 for e4m3); fragments of
//    sub-step g+1 are read while the MFMAs of g issue, the reads and DMAs
//    spread between the MFMAs.  A lane's operand bytes are the same K
//    positions of its row in both operands, so any fixed assignment of K to
//    operand bytes yields the full dot product.  The workgroup barrier sits
//    in the last sub-step, after its fragments are in registers, so that
//    sub-step's MFMAs cover the first reads of the next stage; the DMA of
//    step j is spread over the last sub-step of step j-3 and the first SUB-1
//    of step j-2.
//    The last three steps are peeled so that no step past K is fetched.
//  * Epilogue: the row scales are loaded at kernel start, the tile's column
//    scales and bias reach LDS by DMA (three instructions, not a copy per
//    lane, which would queue ~100 KB per CU ahead of the first stage);
//    results are converted with v_cvt_pk_bf16_f32 (round to nearest even);
//    each wave stages 32-row slabs of its sub-tile in its own LDS area (two
//    slab areas in turn) and stores them as full 128-byte row segments while
//    it converts the next slab.
//  * Tiles are ordered so that the workgroups one XCD receives (blockIdx % 8)
//    form a contiguous range, walked in bands of 8 tile rows, so co-resident
//    workgroups share A and W panels in that XCD's L2.  Shapes with more
//    tiles than CUs run several rounds of workgroups: measured against a
//    persistent form (one workgroup per CU walking its tiles as one K-step
//    pipeline, whose epilogue had no free LDS to stage in), the rounds are
//    4-7 % faster on every multi-round Wan shape.
//
// Phase timing (built only with -DWF_GEMM_PHASES, never in the product library): the first and the
// fifth wave of every workgroup (the two waves of SIMD 0) record, at kernel entry, after the prologue
// barrier, after the K loop's last barrier and after the epilogue's last store, the shader clock
// (s_memtime, wave 0) and the 100 MHz reference clock (s_memrealtime, wave 4) into a buffer registered
// with wf_gemm_set_phase_buffer: 8 stamps per workgroup, [wave 0: 4][wave 4: 4].  waveforcing_amd/gemm_phases.py builds that variant and summarizes the
// stamps (prologue, cycles per K step, epilogue).
#include <atomic>
#include <type_traits>
#include <utility>

#include "launchers.hpp"
#include "wf_common.hpp"

namespace wf {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BK = 128;  // K bytes per step
constexpr int GROUP_M = 8;
constexpr int NUM_XCD = 8;
// The per-column epilogue operands in LDS, past the stages: sw (fp32) at 0, the bias as it arrives (bf16)
// at 1024 and converted to fp32 at 2048.
constexpr int EPI_BYTES = 3072;

// Workgroup tile: BM x 256 outputs, 8 waves in 2 x 4, each (BM / 2) x 64 as MI x 2 blocks of 32 x 32;
// ST LDS stages of (BM + 256) x 128 bytes.
//  * Tile<128, 3>: 48 KB stages; the DMA of step j is spread over the last sub-step of step j-3 and the
//    first SUB-1 sub-steps of step j-2.
//  * Tile<256, 2>: 64 KB stages, a third fewer operand bytes per MFMA through the vector-memory path (64 KB
//    per 256 MFMAs instead of 48 KB per 128); the DMA of step j is issued in the last sub-step of step j-2,
//    right after the barrier that frees its stage, and is waited for at step j-1's barrier.
template <int BM_, int ST_>
struct Tile {
  static constexpr int BM = BM_, BN = 256, WM = 2, WN = 4;
  static constexpr int NW = WM * WN;
  static constexpr int THREADS = NW * 64;
  static constexpr int MI = BM / WM / 32, NI = BN / WN / 32;  // 32x32 blocks per wave
  static constexpr int A_BYTES = BM * BK;
  static constexpr int STAGE = (BM + BN) * BK;
  static constexpr int ST = ST_;
  static constexpr int NBA = BM / 8 / NW, NBB = BN / 8 / NW;  // 1 KB DMA blocks per wave and step
  static constexpr int NDMA = NBA + NBB;
  // Per-wave output staging: two 32-row slabs of the wave's sub-tile, used in turn.
  static constexpr int WPITCH = BN / WN * 2 + 16;
  static_assert(ST == 2 || ST == 3, "two or three stages");
  static_assert(NBA * 8 * NW == BM && NBB * 8 * NW == BN, "DMA blocks");
  static_assert(NW * 2 * 32 * WPITCH <= ST * STAGE, "wave staging fits the stages");
  static_assert(ST * STAGE + EPI_BYTES <= 160 * 1024, "LDS of one workgroup");
};
using TileStd = Tile<128, 3>;
using TileBig = Tile<256, 2>;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9-family parts:
// DATA_FORMAT = 32 bit.  With it, offsets >= num_records read as zero.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kOutOfRange = 0x7ffffff0;

// int8 x int8 -> int32, K = 32 per MFMA (one 16-byte piece per lane).
struct OpI8 {
  static constexpr int SUB = 4;
  static constexpr int PIECES = 1;
  typedef v16i acc_t;
  __device__ static acc_t mfma(const v4i* w, const v4i* a, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w[0], a[0], c, 0, 0, 0);
  }
};
// e4m3 x e4m3 -> fp32, K = 64 per MFMA (two 16-byte pieces per lane).  Zero
// scale operands select the unscaled v_mfma_f32_32x32x64_f8f6f4; format 0
// is OCP e4m3 for both operands.
struct OpFp8 {
  static constexpr int SUB = 2;
  static constexpr int PIECES = 2;
  typedef v16f acc_t;
  __device__ static acc_t mfma(const v4i* w, const v4i* a, acc_t c) {
    const v8i wv = __builtin_shufflevector(w[0], w[1], 0, 1, 2, 3, 4, 5, 6, 7);
    const v8i av = __builtin_shufflevector(a[0], a[1], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wv, av, c, 0, 0, 0, 0, 0, 0);
  }
};

template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <int V>
using ic = std::integral_constant<int, V>;

// s_waitcnt with vmcnt(VM), lgkmcnt(LGKM) (15 = no wait), expcnt unchanged.
template <int VM, int LGKM>
__device__ inline void wait_counts() {
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "wait counts");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | 0x70 | (LGKM << 8));
}

__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds_block, int offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_block, 16, offset, 0, 0, 0);
}
__device__ inline void dma4(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds_block, int offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_block, 4, offset, 0, 0, 0);
}


// A rectangle of the output that one launch covers with its workgroup tile: rows [m0, m1), columns [n0, n1);
// m0 and n0 lie on the launch's tile grid and every tile but those at M or N lies wholly inside.
struct Rect {
  int m0, m1, n0, n1;
};

struct GemmArgs {
  const void* a;         // [M, K] int8 or e4m3
  const void* w;         // [N, K]
  const float* sx;       // int8: [M];  e4m3: [1] (s_a)
  const float* sw;       // int8: [N];  e4m3: [1] (s_w)
  const uint16_t* bias;  // [N] bf16 or null
  uint16_t* y;           // [M, N] bf16 (ldy)
  int32_t* acc_out;      // int8 only: [M, N] int32 or null
  int M, N, K;
  int64_t ldy;
  int vec16;             // y and ldy allow 16-byte row stores
  uint64_t* phases;      // phase-timing stamps (instrumented build only), or null
  Rect rect[2];          // the output this launch covers: rect[0], then rect[1] when n_rect == 2
  int n_rect;
};

// Stamp `slot` of this workgroup's phase record (instrumented build only; a no-op otherwise).
__device__ inline void phase_stamp(const GemmArgs& p, int wave, int lane, int slot) {
#ifdef WF_GEMM_PHASES
  if (p.phases != nullptr && (wave == 0 || wave == 4)) {
    // wave 0: the shader clock (cycles); its SIMD mate: the constant 100 MHz reference clock at the same
    // points (the same barriers), which turns the cycle counts into a frequency
    const uint64_t t = wave == 0 ? __builtin_amdgcn_s_memtime() : __builtin_amdgcn_s_memrealtime();
    if (lane == 0) p.phases[static_cast<int64_t>(blockIdx.x) * 8 + (wave == 0 ? 0 : 4) + slot] = t;
  }
#else
  (void)p;
  (void)wave;
  (void)lane;
  (void)slot;
#endif
}

// The epilogue operands of the 256 columns from n0 into epi: sw by wave 0 (one 1 KB DMA), bias by wave 1
// (two 256-byte DMAs).  Columns past N read as zero (N % 4 == 0, so no access straddles the end).
template <bool SW, bool BIAS>
__device__ inline void epi_dma(const GemmArgs& p, int wave, int lane, int n0, uint8_t* epi) {
  if constexpr (SW) {
    if (wave == 0)
      dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.sw), 0, p.N * 4, kBufferRsrcWord3), epi,
            (n0 + 4 * lane) * 4);
  }
  if constexpr (BIAS) {
    if (wave == 1) {
      const __amdgpu_buffer_rsrc_t rb =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.bias), 0, p.N * 2, kBufferRsrcWord3);
      dma4(rb, epi + 1024, (n0 + 2 * lane) * 2);
      dma4(rb, epi + 1280, (n0 + 128 + 2 * lane) * 2);
    }
  }
}

template <typename T, typename OP, bool HAS_BIAS, bool GELU, bool ACC>
__global__ __launch_bounds__(T::THREADS, 1) void gemm_w8a8_kernel(GemmArgs p) {
  constexpr int BM = T::BM, BN = T::BN, WM = T::WM, WN = T::WN, NW = T::NW, MI = T::MI, NI = T::NI;
  constexpr int A_BYTES = T::A_BYTES, STAGE = T::STAGE, ST = T::ST, NBA = T::NBA, NDMA = T::NDMA;
  constexpr int WPITCH = T::WPITCH;
  constexpr bool kI8 = std::is_same<OP, OpI8>::value;
  constexpr int SUB = OP::SUB;
  constexpr int PIECES = OP::PIECES;
  constexpr int CPS = BK / 16 / SUB;  // 16-byte K chunks per sub-step (2 per lane pair)
  static_assert(CPS == 2 * PIECES, "sub-step geometry");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[ST * STAGE + EPI_BYTES];
  uint8_t* const epi = lds + ST * STAGE;

  // The launch's tiles: those of rect[0], then those of rect[1].
  const int tm0 = (p.rect[0].m1 - p.rect[0].m0 + BM - 1) / BM, tn0 = (p.rect[0].n1 - p.rect[0].n0 + BN - 1) / BN;
  const int tm1 = p.n_rect > 1 ? (p.rect[1].m1 - p.rect[1].m0 + BM - 1) / BM : 0;
  const int tn1 = p.n_rect > 1 ? (p.rect[1].n1 - p.rect[1].n0 + BN - 1) / BN : 0;
  const int c0 = tm0 * tn0;
  const int n_tiles = c0 + tm1 * tn1;
  const int per_xcd = (n_tiles + NUM_XCD - 1) / NUM_XCD;
  const int t_all = (blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
  if (t_all >= n_tiles) return;
  const bool second = t_all >= c0;
  const int t = second ? t_all - c0 : t_all;
  const int tiles_m = second ? tm1 : tm0, tiles_n = second ? tn1 : tn0;
  // Grouped order within the rectangle: bands of GROUP_M tile rows swept column by column.
  const int per_group = GROUP_M * tiles_n;
  const int first_m = (t / per_group) * GROUP_M;
  const int band = min(tiles_m - first_m, GROUP_M);
  const int m0 = (second ? p.rect[1].m0 : p.rect[0].m0) + (first_m + (t % per_group) % band) * BM;
  const int n0 = (second ? p.rect[1].n0 : p.rect[0].n0) + ((t % per_group) / band) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  phase_stamp(p, wave, lane, 0);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  // Epilogue operands: the row scales now (their latency hides under the K loop), the per-column sw and
  // bias by DMA into LDS ahead of the stages (three instructions instead of a per-lane copy each).
  float sxv[MI];
  float scale = 0.f;
  if constexpr (kI8) {
#pragma unroll
    for (int i = 0; i < MI; ++i) sxv[i] = p.sx[min(m0 + wm * (BM / WM) + i * 32 + l32, p.M - 1)];
  } else {
    scale = p.sx[0] * p.sw[0];
  }
  epi_dma<kI8, HAS_BIAS>(p, wave, lane, n0, epi);

  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.a), 0, p.M * p.K, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_w =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.w), 0, p.N * p.K, kBufferRsrcWord3);

  // DMA block j of this wave: A rows (j * NW + wave) * 8 .. + 7 for j < NBA,
  // else W rows ((j - NBA) * NW + wave) * 8 .. + 7.
  int doff[NDMA], dcol[NDMA];
#pragma unroll
  for (int j = 0; j < NDMA; ++j) {
    const bool is_a = j < NBA;
    const int r = ((is_a ? j : j - NBA) * NW + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    dcol[j] = c * 16;
    doff[j] = ((is_a ? m0 : n0) + r) * p.K + c * 16;
  }
  auto dma = [&](auto J, int k0, int stage) {
    constexpr int j = decltype(J)::value;
    const int off = (k0 + dcol[j] < p.K) ? doff[j] + k0 : kOutOfRange;
    if constexpr (j < NBA)
      dma16(rsrc_a, lds + stage * STAGE + (j * NW + wave) * 1024, off);
    else
      dma16(rsrc_w, lds + stage * STAGE + A_BYTES + ((j - NBA) * NW + wave) * 1024, off);
  };
  // Block j of wave w (w = wave +- NW/2): its rows are this wave's plus (w - wave) * 8, with the same
  // swizzled chunk (the row difference is a multiple of 16).
  auto dma_of = [&](auto J, int k0, int stage, int w) {
    constexpr int j = decltype(J)::value;
    const int off = (k0 + dcol[j] < p.K) ? doff[j] + (w - wave) * 8 * p.K + k0 : kOutOfRange;
    if constexpr (j < NBA)
      dma16(rsrc_a, lds + stage * STAGE + (j * NW + w) * 1024, off);
    else
      dma16(rsrc_w, lds + stage * STAGE + A_BYTES + ((j - NBA) * NW + w) * 1024, off);
  };

  // Fragment pieces: sub-step s, lane half h, piece e is K chunk
  // c = s*CPS + h*PIECES + e of the lane's row R, at R*128 + 16*(c ^ ((R/2)%8)).
  // The rows one lane reads differ by multiples of 32, so the offsets are per lane.
  const int x = (l32 >> 1) & 7;
  const int lane_a = (wm * (BM / WM) + l32) * BK;
  const int lane_b = A_BYTES + (wn * (BN / WN) + l32) * BK;
  int koff[SUB][PIECES];
#pragma unroll
  for (int s = 0; s < SUB; ++s)
#pragma unroll
    for (int e = 0; e < PIECES; ++e) koff[s][e] = 16 * ((s * CPS + half * PIECES + e) ^ x);

  typename OP::acc_t acc[NI][MI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[j][i] = typename OP::acc_t{};
  v4i fa[2][MI][PIECES], fw[2][NI][PIECES];

  // Read o (fragment o / PIECES, A blocks first, piece o % PIECES) of sub-step s into buffer B.
  auto frag_read = [&](auto O, auto B, int stage, int s) {
    constexpr int o = decltype(O)::value;
    constexpr int b = decltype(B)::value;
    constexpr int q = o / PIECES, e = o % PIECES;
    if constexpr (q < MI)
      fa[b][q][e] = *reinterpret_cast<const v4i*>(lds + stage * STAGE + lane_a + koff[s][e] + q * 32 * BK);
    else
      fw[b][q - MI][e] = *reinterpret_cast<const v4i*>(lds + stage * STAGE + lane_b + koff[s][e] + (q - MI) * 32 * BK);
  };
  // The MFMAs of buffer B with, spread between them, the reads of sub-step rs
  // of rstage into buffer 1-B and DMA slot SLOT (of SUB per step) for the
  // step at K offset dk0 into dstage.  Three stages spread a step's DMAs evenly over the SUB slots; two
  // stages put them all in slot 0 (the sub-step right after the barrier), for the longest lead.
  // RD / DM switch the reads and the DMAs off (the last steps have no next sub-step or step to fetch).
  auto substep = [&](auto B, int rstage, int rs, auto SLOT, int dk0, int dstage, auto RD, auto DM) {
    constexpr int b = decltype(B)::value;
    constexpr int slot = decltype(SLOT)::value;
    constexpr bool rd = decltype(RD)::value, dm = decltype(DM)::value;
    constexpr int d_lo = ST == 3 ? (slot * NDMA + SUB - 1) / SUB : 0;
    constexpr int d_hi = !dm ? d_lo : ST == 3 ? ((slot + 1) * NDMA + SUB - 1) / SUB : (slot == 0 ? NDMA : 0);
    constexpr int NMF = MI * NI, NRD = rd ? (MI + NI) * PIECES : 0;
    constexpr int NOPS = NRD + d_hi - d_lo;
    static_for<NMF>([&](auto Q) {
      constexpr int q = decltype(Q)::value;
      constexpr int jj = q / MI, ii = q % MI;
      acc[jj][ii] = OP::mfma(fw[b][jj], fa[b][ii], acc[jj][ii]);
      constexpr int o_lo = (q * NOPS + NMF - 1) / NMF, o_hi = ((q + 1) * NOPS + NMF - 1) / NMF;
      static_for<o_hi - o_lo>([&](auto U) {
        constexpr int o = o_lo + decltype(U)::value;
        if constexpr (o < NRD)
          frag_read(ic<o>{}, ic<b ^ 1>{}, rstage, rs);
        else
          dma(ic<d_lo + o - NRD>{}, dk0, dstage);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Steps past K load zeros (a zero contribution): every step runs the same
  // code, and the last DMAs (of steps nk .. nk+2) only fill unused stages.
  const int nk = (p.K + BK - 1) / BK;
  // Prologue: waves 0..NW/2-1, which win the issue arbitration of the SIMD they share with wave + NW/2,
  // fetch all of stage 0 (their blocks and their SIMD mate's); the mates fetch stage 1.  So stage 0 is
  // not queued behind stage 1, and only stage 0 is waited for here (the mates' stage-1 DMAs are older
  // than the NDMA most recent ones at the first step's wait, which therefore covers them).
  if (wave < NW / 2) {
    static_for<NDMA>([&](auto J) {
      dma_of(J, 0, 0, wave);
      dma_of(J, 0, 0, wave + NW / 2);
    });
    wait_counts<0, 0>();
  } else {
    static_for<NDMA>([&](auto J) {
      dma_of(J, BK, 1, wave);
      dma_of(J, BK, 1, wave - NW / 2);
    });
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  phase_stamp(p, wave, lane, 1);
  // the bias as fp32 for the epilogue (published by the first K step's barrier)
  if constexpr (HAS_BIAS) {
    if (wave == 1) {
      const uint2 b = *reinterpret_cast<const uint2*>(epi + 1024 + lane * 8);
      *reinterpret_cast<float4*>(epi + 2048 + lane * 16) =
          make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xffff0000u), __uint_as_float(b.y << 16),
                      __uint_as_float(b.y & 0xffff0000u));
    }
  }
  if constexpr (ST == 3) {
    if (nk >= 3) static_for<(NDMA + SUB - 1) / SUB>([&](auto J) { dma(J, 2 * BK, 2); });
  }
  static_for<(MI + NI) * PIECES>([&](auto O) { frag_read(O, ic<0>{}, 0, 0); });
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (ST == 3) {
  // Step kb: sub-steps 1..SUB-1 fetch slots 1.. of step kb+2 (PRE), the last sub-step, after the barrier,
  // slot 0 of step kb+3 (POST).  Only steps below nk are fetched, so the last three steps are peeled:
  // step nk-3 has no POST, step nk-2 neither, and step nk-1 also no barrier and no fragment reads.
  int c0 = 0, c1 = 1, c2 = 2;  // stages of steps kb, kb+1, kb+2
  auto step = [&](int kb, auto PRE, auto POST, auto LAST) {
    constexpr bool pre = decltype(PRE)::value, last = decltype(LAST)::value;
    const int k2 = (kb + 2) * BK;
    static_for<SUB - 1>([&](auto S) {
      constexpr int s = decltype(S)::value;
      substep(ic<s & 1>{}, c0, s + 1, ic<s + 1>{}, k2, c2, ic<1>{}, PRE);
    });
    if constexpr (!last) {
      // Own reads of this stage done, own DMAs of step kb+1 landed (with PRE only step kb+2's, NDMA of
      // them, may still be in flight; without it none are); the barrier makes that hold for every wave.
      if constexpr (pre)
        wait_counts<NDMA, 0>();
      else
        wait_counts<0, 0>();
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    substep(ic<(SUB - 1) & 1>{}, c1, 0, ic<0>{}, (kb + 3) * BK, c0, ic<!last>{}, POST);
    const int c = c0;
    c0 = c1;
    c1 = c2;
    c2 = c;
  };
  int kb = 0;
  for (; kb < nk - 3; ++kb) step(kb, ic<1>{}, ic<1>{}, ic<0>{});
  if (nk >= 3) step(kb++, ic<1>{}, ic<0>{}, ic<0>{});
  if (nk >= 2) step(kb++, ic<0>{}, ic<0>{}, ic<0>{});
  step(kb, ic<0>{}, ic<0>{}, ic<1>{});
  } else {
  // Two stages.  Step kb: sub-steps 1..SUB-1 read from stage c0 and fetch nothing; at the barrier every DMA
  // issued so far (step kb+1's) has landed and every wave is done with c0; the last sub-step reads
  // sub-step 0 of step kb+1 from c1 and fetches all of step kb+2 into c0 (POST).  Peeled: step nk-2 has
  // no POST, step nk-1 no barrier and no fragment reads.
  int c0 = 0, c1 = 1;  // stages of steps kb, kb+1
  auto step = [&](int kb, auto POST, auto LAST) {
    constexpr bool last = decltype(LAST)::value;
    static_for<SUB - 1>([&](auto S) {
      constexpr int s = decltype(S)::value;
      substep(ic<s & 1>{}, c0, s + 1, ic<s + 1>{}, 0, 0, ic<1>{}, ic<0>{});
    });
    if constexpr (!last) {
      wait_counts<0, 0>();
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    substep(ic<(SUB - 1) & 1>{}, c1, 0, ic<0>{}, (kb + 2) * BK, c0, ic<!last>{}, POST);
    const int c = c0;
    c0 = c1;
    c1 = c;
  };
  int kb = 0;
  for (; kb < nk - 2; ++kb) step(kb, ic<1>{}, ic<0>{});
  if (nk >= 2) step(kb++, ic<0>{}, ic<0>{});
  step(kb, ic<0>{}, ic<1>{});
  }
  // The epilogue operands from LDS, then all DMAs landed, all LDS accesses done and all waves past
  // their last LDS read before the stages are reused for the output staging.  The fp32 bias is wave 1's
  // write after the prologue barrier: with two or more K steps the first step's barrier (after an LDS
  // wait) has published it, so the operands are read before the drain to overlap it; with one K step
  // only the barrier below publishes it.
  float4 swv[NI][4], bfv[NI][4];
  auto read_epi = [&]() {
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = wn * (BN / WN) + j * 32 + 8 * g + 4 * half;
        if constexpr (kI8) swv[j][g] = *reinterpret_cast<const float4*>(epi + c * 4);
        if constexpr (HAS_BIAS) bfv[j][g] = *reinterpret_cast<const float4*>(epi + 2048 + c * 4);
      }
  };
  if (nk >= 2) read_epi();
  wait_counts<0, 0>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  phase_stamp(p, wave, lane, 2);
  if (nk < 2) read_epi();

  // Each wave converts its 64 x 64 sub-tile as two 32-row slabs; a slab goes to the wave's own LDS area
  // as bf16 rows and leaves as full 128-byte row segments (8 rows per store instruction) while the next
  // slab is converted.  Block (j, i) element (n, m): m = l32, n = 8*(r/4) + 4*half + r%4.
  uint8_t* const wst = lds + wave * (2 * 32 * WPITCH);
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    // slabs alternate between two areas: a wave's LDS accesses execute in order, so slab i + 2's writes
    // follow slab i's read-back
    uint8_t* const slab = wst + (i & 1) * 32 * WPITCH;
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cw = j * 32 + 8 * g + 4 * half;  // column within the wave's 64
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (kI8) {
            const float sw4[4] = {swv[j][g].x, swv[j][g].y, swv[j][g].z, swv[j][g].w};
            y[e] = __fmul_rn(__fmul_rn(static_cast<float>(acc[j][i][4 * g + e]), sxv[i]), sw4[e]);
          } else {
            y[e] = __fmul_rn(acc[j][i][4 * g + e], scale);
          }
          if constexpr (HAS_BIAS) {
            const float b4[4] = {bfv[j][g].x, bfv[j][g].y, bfv[j][g].z, bfv[j][g].w};
            y[e] = __fadd_rn(y[e], b4[e]);
          }
          if (GELU) y[e] = gelu_tanh(__uint_as_float(pack_bf16x2_hw(y[e], 0.f) << 16));
        }
        *reinterpret_cast<uint2*>(slab + l32 * WPITCH + cw * 2) =
            make_uint2(pack_bf16x2_hw(y[0], y[1]), pack_bf16x2_hw(y[2], y[3]));
        if constexpr (kI8 && ACC) {
          const int gm = m0 + wm * (BM / WM) + i * 32 + l32, gn = n0 + wn * (BN / WN) + cw;
          if (gm < p.M && gn < p.N)
            *reinterpret_cast<int4*>(p.acc_out + static_cast<int64_t>(gm) * p.N + gn) =
                make_int4(acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]);
        }
      }
    // the slab's rows are read back by other lanes of this wave: LDS executes a wave's accesses in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int ch = lane & 7;
    const int gn = n0 + wn * (BN / WN) + ch * 8;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rr = it * 8 + (lane >> 3);
      const uint4 v = *reinterpret_cast<const uint4*>(slab + rr * WPITCH + ch * 16);
      const int gm = m0 + wm * (BM / WM) + i * 32 + rr;
      if (gm < p.M && gn < p.N) {
        uint16_t* dst = p.y + static_cast<int64_t>(gm) * p.ldy + gn;
        if (p.vec16 && gn + 8 <= p.N) {
          *reinterpret_cast<uint4*>(dst) = v;
        } else {
          // N % 4 == 0 (checked at the entry point): the first 4 columns are in.
          *reinterpret_cast<uint2*>(dst) = make_uint2(v.x, v.y);
          if (gn + 8 <= p.N) *reinterpret_cast<uint2*>(dst + 4) = make_uint2(v.z, v.w);
        }
      }
    }
  }
  phase_stamp(p, wave, lane, 3);
}

// The phase-stamp buffer of the instrumented build (null in the product library).
uint64_t* g_phase_buffer = nullptr;

GemmArgs make_args(const void* a, const void* w, int64_t M, int64_t N, int64_t K, const float* sx, const float* sw,
                   const void* bias, void* y, int64_t ldy, int32_t* acc_out) {
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
  p.vec16 = (ldy % 8 == 0) && ((reinterpret_cast<uintptr_t>(y) & 15u) == 0);
  p.phases = g_phase_buffer;
  p.rect[0] = Rect{0, p.M, 0, p.N};
  p.rect[1] = Rect{0, 0, 0, 0};
  p.n_rect = 1;
  return p;
}

template <typename T, typename OP, bool ACC>
void launch_kernel(const GemmArgs& p, bool bias, bool gelu, hipStream_t stream) {
  int64_t tiles = 0;
  for (int r = 0; r < p.n_rect; ++r)
    tiles += static_cast<int64_t>((p.rect[r].m1 - p.rect[r].m0 + T::BM - 1) / T::BM) *
             ((p.rect[r].n1 - p.rect[r].n0 + T::BN - 1) / T::BN);
  if (tiles == 0) return;
  const dim3 grid(static_cast<uint32_t>((tiles + NUM_XCD - 1) / NUM_XCD * NUM_XCD));
  const dim3 block(T::THREADS);
  if (bias && gelu)
    hipLaunchKernelGGL((gemm_w8a8_kernel<T, OP, true, true, ACC>), grid, block, 0, stream, p);
  else if (bias)
    hipLaunchKernelGGL((gemm_w8a8_kernel<T, OP, true, false, ACC>), grid, block, 0, stream, p);
  else if (gelu)
    hipLaunchKernelGGL((gemm_w8a8_kernel<T, OP, false, true, ACC>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((gemm_w8a8_kernel<T, OP, false, false, ACC>), grid, block, 0, stream, p);
}

// Tile plan: -1 the cost model below; 0 / 1 force the 128- / 256-row tile for the whole output (settable only
// in the instrumented libraries, for A/B runs).
int g_tile_policy = -1;

// Compute units of the current device (one workgroup per CU at a time), cached per device (host threads may
// call concurrently; each stores the same value).
int device_cus() {
  static std::atomic<int> cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cus[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int n = 0;
    v = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : 256;
    cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Both tiles run one workgroup per CU, so a launch takes about ceil(tiles / CUs) rounds of its tile's time.
// A 256-row tile holds twice the work of a 128-row tile and takes about kBigTileCost times as long (1.62-1.83
// on the eight Wan-1.3B / 14B linears at 4680 tokens, int8 and e4m3 alike).  Plans: the 128-row tile
// everywhere; the 256-row tile everywhere; or F whole rounds of 256-row tiles (F x CUs of them in row-major
// order over the 256-row grid: whole tile rows, then a prefix of the next) followed by a second launch of
// 128-row tiles over the rest (the suffix of that tile row and every row below), so that neither launch
// ends on a mostly idle round.  The second launch has a fixed cost (about 3 us of launch gap and ramp, a
// third of a 128-row round at K = 1536, under a tenth from K = 4096), so mixed plans are considered from
// kMixedMinK on.  The cheapest plan by the model is taken when it costs at least kPlanMargin less than the
// 128-row tile alone.
constexpr double kBigTileCost = 1.75;
constexpr double kPlanMargin = 0.95;
constexpr int kMixedMinK = 4096;

struct Plan {
  int big_rects = 0;  // 0: no 256-row launch
  Rect big[2] = {};
  int std_rects = 0;  // 0: no 128-row launch
  Rect std_[2] = {};
};

int64_t rect_tiles(const Rect& r, int bm) {
  return static_cast<int64_t>((r.m1 - r.m0 + bm - 1) / bm) * ((r.n1 - r.n0 + 255) / 256);
}

Plan plan_tiles(int M, int N, int K) {
  Plan all_std;
  all_std.std_rects = 1;
  all_std.std_[0] = Rect{0, M, 0, N};
  Plan all_big;
  all_big.big_rects = 1;
  all_big.big[0] = Rect{0, M, 0, N};
  if (g_tile_policy == 0) return all_std;
  if (g_tile_policy == 1) return all_big;
  const int64_t cus = device_cus();
  const int64_t tn = (N + 255) / 256;
  const int64_t big_tiles = static_cast<int64_t>((M + 255) / 256) * tn;
  const double cost_std = static_cast<double>((rect_tiles(all_std.std_[0], 128) + cus - 1) / cus);
  Plan best = all_std;
  double best_cost = cost_std;
  const double cost_big = kBigTileCost * static_cast<double>((big_tiles + cus - 1) / cus);
  if (cost_big < kPlanMargin * best_cost) {
    best = all_big;
    best_cost = cost_big;
  }
  for (int64_t f = 1; K >= kMixedMinK && f * cus < big_tiles; ++f) {
    const int64_t nb = f * cus;
    const int full = static_cast<int>(nb / tn), part = static_cast<int>(nb % tn);
    Plan pl;
    const int row_a = 256 * full;                     // end of the whole 256-row tile rows
    const int row_b = min(row_a + 256, M);            // end of the partly covered tile row
    if (full > 0) pl.big[pl.big_rects++] = Rect{0, row_a, 0, N};
    if (part > 0) {
      pl.big[pl.big_rects++] = Rect{row_a, row_b, 0, 256 * part};
      pl.std_[pl.std_rects++] = Rect{row_a, row_b, 256 * part, N};
      if (row_b < M) pl.std_[pl.std_rects++] = Rect{row_b, M, 0, N};
    } else if (row_a < M) {
      pl.std_[pl.std_rects++] = Rect{row_a, M, 0, N};
    }
    int64_t ns = 0;
    for (int r = 0; r < pl.std_rects; ++r) ns += rect_tiles(pl.std_[r], 128);
    const double cost = kBigTileCost * static_cast<double>(f) + static_cast<double>((ns + cus - 1) / cus);
    if (cost < kPlanMargin * cost_std && cost < best_cost) {
      best = pl;
      best_cost = cost;
    }
  }
  return best;
}

template <typename OP>
int launch(const GemmArgs& p0, bool bias, bool gelu, hipStream_t stream, const char* fn) {
  const bool acc = std::is_same<OP, OpI8>::value && p0.acc_out != nullptr;
  const Plan plan = plan_tiles(p0.M, p0.N, p0.K);
  GemmArgs p = p0;
  if (plan.big_rects > 0) {
    p.n_rect = plan.big_rects;
    p.rect[0] = plan.big[0];
    p.rect[1] = plan.big[1];
    if (acc)
      launch_kernel<TileBig, OP, true>(p, bias, gelu, stream);
    else
      launch_kernel<TileBig, OP, false>(p, bias, gelu, stream);
  }
  if (plan.std_rects > 0) {
    p.n_rect = plan.std_rects;
    p.rect[0] = plan.std_[0];
    p.rect[1] = plan.std_[1];
    if (acc)
      launch_kernel<TileStd, OP, true>(p, bias, gelu, stream);
    else
      launch_kernel<TileStd, OP, false>(p, bias, gelu, stream);
  }
  return check_launch(fn);
}

}  // namespace

int launch_gemm_i8(const int8_t* a, const int8_t* w, int64_t M, int64_t N, int64_t K, const float* sx,
                   const float* sw, const void* bias, void* y, int64_t ldy, int32_t* acc_out, int gelu,
                   hipStream_t stream) {
  return launch<OpI8>(make_args(a, w, M, N, K, sx, sw, bias, y, ldy, acc_out), bias != nullptr, gelu != 0, stream,
                      "wf_gemm_i8");
}

int launch_gemm_fp8_pertensor(const uint8_t* a, const uint8_t* w, int64_t M, int64_t N, int64_t K,
                              const float* a_scale, const float* w_scale, const void* bias, void* y, int64_t ldy,
                              hipStream_t stream) {
  return launch<OpFp8>(make_args(a, w, M, N, K, a_scale, w_scale, bias, y, ldy, nullptr), bias != nullptr, false,
                       stream, "wf_gemm_fp8_pertensor");
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
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && wf::product_below({m + 256, k}, (1ll << 31) - 16) &&
                 wf::product_below({n + 256, k}, (1ll << 31) - 16),
             WF_E_SHAPE,
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
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && wf::product_below({m + 256, k}, (1ll << 31) - 16) &&
                 wf::product_below({n + 256, k}, (1ll << 31) - 16),
             WF_E_SHAPE,
             "%s: operands of 2 GiB or more are not supported", fn);
  WF_REQUIRE(k % 16 == 0 && ldx % 8 == 0, WF_E_SHAPE, "%s: k %% 16 and ldx %% 8 must be 0", fn);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(qw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(ws_q) & 15u) == 0 && (reinterpret_cast<uintptr_t>(sw) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: x, qw, sw, ws_q must be 16-byte and y, bias 8-byte aligned", fn);
  WF_REQUIRE((flags & ~(WF_GEMM_GELU_TANH | WF_LINEAR_GELU_INPUT)) == 0, WF_E_INVALID, "%s: unknown flags 0x%x", fn,
             flags);
  hipStream_t st = wf::as_stream(stream);
  if (int rc = wf::launch_quant_rows_i8(x, m, k, ldx, ws_q, k, ws_sx, st, (flags & WF_LINEAR_GELU_INPUT) != 0))
    return rc;
  return wf::launch_gemm_i8(ws_q, qw, m, n, k, ws_sx, sw, bias, y, ldy, nullptr, flags & WF_GEMM_GELU_TANH, st);
}

extern "C" int wf_gemm_fp8_pertensor(const uint8_t* a, const uint8_t* w, int64_t m, int64_t n, int64_t k,
                                     const float* a_scale, const float* w_scale, const void* bias, void* y,
                                     int64_t ldy, void* stream) {
  static const char* fn = "wf_gemm_fp8_pertensor";
  WF_REQUIRE(m >= 0 && n >= 0 && k >= 0 && ldy >= n, WF_E_INVALID, "%s: bad sizes m=%lld n=%lld k=%lld ldy=%lld", fn,
             (long long)m, (long long)n, (long long)k, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(a && w && a_scale && w_scale && y, WF_E_INVALID, "%s: null pointer", fn);
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && wf::product_below({m + 256, k}, (1ll << 31) - 16) &&
                 wf::product_below({n + 256, k}, (1ll << 31) - 16),
             WF_E_SHAPE,
             "%s: operands of 2 GiB or more are not supported", fn);
  WF_REQUIRE(k % 16 == 0 && k > 0, WF_E_SHAPE, "%s: k=%lld must be a positive multiple of 16", fn, (long long)k);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: a, w must be 16-byte and y, bias 8-byte aligned", fn);
  return wf::launch_gemm_fp8_pertensor(a, w, m, n, k, a_scale, w_scale, bias, y, ldy, wf::as_stream(stream));
}

extern "C" int wf_fp8_linear_pertensor(const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* w_codes,
                                       const float* w_scale, const void* bias, int64_t n, void* y, int64_t ldy,
                                       uint8_t* ws_codes, float* ws_scale, float* ws_partials, void* stream) {
  static const char* fn = "wf_fp8_linear_pertensor";
  WF_REQUIRE(m >= 0 && n >= 0 && k > 0 && ldx >= k && ldy >= n, WF_E_INVALID,
             "%s: bad sizes m=%lld n=%lld k=%lld ldx=%lld ldy=%lld", fn, (long long)m, (long long)n, (long long)k,
             (long long)ldx, (long long)ldy);
  if (m == 0 || n == 0) return WF_OK;
  WF_REQUIRE(x && w_codes && w_scale && y && ws_codes && ws_scale && ws_partials, WF_E_INVALID, "%s: null pointer",
             fn);
  WF_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && wf::product_below({m + 256, k}, (1ll << 31) - 16) &&
                 wf::product_below({n + 256, k}, (1ll << 31) - 16),
             WF_E_SHAPE,
             "%s: operands of 2 GiB or more are not supported", fn);
  WF_REQUIRE(k % 16 == 0 && ldx % 8 == 0, WF_E_SHAPE, "%s: k %% 16 and ldx %% 8 must be 0", fn);
  WF_REQUIRE(n % 4 == 0 && ldy % 4 == 0, WF_E_SHAPE, "%s: n and ldy must be multiples of 4", fn);
  WF_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w_codes) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(ws_codes) & 15u) == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0 &&
                 (reinterpret_cast<uintptr_t>(bias) & 7u) == 0,
             WF_E_ALIGN, "%s: x, w_codes, ws_codes must be 16-byte and y, bias 8-byte aligned", fn);
  hipStream_t st = wf::as_stream(stream);
  if (int rc = wf::launch_fp8_quant_pertensor(x, m, k, ldx, WF_FP8_TENSOR_ACT, ws_codes, ws_scale, ws_partials, st))
    return rc;
  return wf::launch_gemm_fp8_pertensor(ws_codes, w_codes, m, n, k, ws_scale, w_scale, bias, y, ldy, st);
}

#ifdef WF_GEMM_PHASES
// Instrumented build only (not declared in wf_api.h): register a device buffer of 8 uint64 per workgroup
// for the phase stamps of the following GEMM launches, or null to stop recording.
extern "C" int wf_gemm_set_phase_buffer(uint64_t* stamps) {
  wf::g_phase_buffer = stamps;
  return WF_OK;
}
#endif
#if defined(WF_GEMM_PHASES) || defined(WF_GEMM_TILE_LAB)
// Instrumented builds only: the tile plan of the following GEMM launches (-1 the product's plan, 0 the
// 128 x 256 tile over the whole output, 1 the 256 x 256 tile over the whole output).
extern "C" int wf_gemm_set_tile_policy(int policy) {
  WF_REQUIRE(policy >= -1 && policy <= 1, WF_E_INVALID, "wf_gemm_set_tile_policy: policy %d not in -1..1", policy);
  wf::g_tile_policy = policy;
  return WF_OK;
}
#endif
