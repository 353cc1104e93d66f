/*
 * wf_api.h - C ABI of libwf_mi355x.so, the gfx950 (MI355X) implementation of
 * the quantized DiT-block path of the Wan2.1 block-causal denoiser:
 *
 *   - FP8 e4m3fn K/V packing into a paged, layer-wise KV pool, and the
 *     gather-dequant of those pages;
 *   - per-token int8 activation quantization and the W8A8 int8 GEMM
 *     (i8 MFMA, int32 accumulation, per-channel dequant + bias, bf16 out);
 *   - the reference's own per-tensor e4m3 W8A8 linear (FP8 MFMA);
 *   - block-causal attention over the FP8 paged context.
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer unless stated otherwise.  Tensors are
 *     dense row-major; "bf16" buffers hold IEEE bfloat16 bit patterns.
 *   - The library never allocates, frees or caches device memory.  Any
 *     workspace is passed in by the caller.  The one exception,
 *     wf_w8a8_linear_static, keeps its workspace in a fixed static device
 *     array instead (see its declaration).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Calls only
 *     enqueue work; none of them synchronizes the device.
 *   - Return value: 0 = success, > 0 = a hipError_t from the launch,
 *     < 0 = a WF_E_* argument error.  wf_last_error() returns a
 *     thread-local message describing the last non-zero status.
 *   - Page tables are int32 device arrays of physical page ids.  Entries
 *     outside [0, pool_pages) are never written or read: the pack skips
 *     them, the gather-dequant leaves their tokens' output rows untouched,
 *     and attention reads their keys as zero K and zero V -- such a key
 *     still takes part in the softmax with score 0 (it is not masked like
 *     the keys past n_kv), so it dilutes the output.  Callers validate
 *     tables on the host (waveforcing_amd.kv.PageTable does).
 */
#ifndef WF_API_H
#define WF_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WF_OK 0
#define WF_E_INVALID (-1)     /* null pointer or negative size */
#define WF_E_SHAPE (-2)       /* unsupported shape (e.g. head_dim != 128) */
#define WF_E_ALIGN (-3)       /* pointer not aligned as required */

/* ------------------------------------------------------------------ misc */

/* Thread-local text of the last non-zero status returned on this thread. */
const char* wf_last_error(void);

/* ABI version: (major << 16) | minor. */
int wf_abi_version(void);

/* OCP e4m3fn round-to-nearest-even cast of n fp32 values, with the same
 * results as torch's `x.to(torch.float8_e4m3fn)`: magnitudes that round
 * above 448 and NaN become the NaN code 0x7f (sign kept), -0 keeps its sign.
 * Replaces the elementwise casts at wave_rt/denoiser/exchange/common.py:150
 * and wave_rt/denoiser/exchange/onesided.py:152 (scale == 1 case). */
int wf_fp8_e4m3_encode_f32(const float* x, uint8_t* codes, int64_t n,
                           void* stream);

/* Exact e4m3fn -> fp32 decode of n codes (0x7f / 0xff decode to NaN).
 * Replaces the upcast at wave_rt/denoiser/exchange/onesided.py:177-178. */
int wf_fp8_e4m3_decode_f32(const uint8_t* codes, float* out, int64_t n,
                           void* stream);

/* ------------------------------------------------------- FP8 paged KV pool
 *
 * Pool layout (one pool for K, one for V):
 *   codes  u8   [pool_pages][page_tokens][n_heads][head_dim]
 *   scales f32  [pool_pages][n_heads][page_tokens]
 * Logical token t of a packed sequence lives in physical page
 * page_table[t / page_tokens], row t % page_tokens.
 *
 * Per (token, head) row x[0..head_dim):
 *   s    = float( bf16( bf16(max|x|) / 448 ) ), then s = max(s, bf16(1e-8))
 *   code = e4m3_rne( clamp( float(x) / s, -448, 448 ) )   (fp32 division)
 * which is wave_rt/denoiser/exchange/common.py:145-150 with the amax taken
 * per (token, head) in place of per tensor.
 */

/* Pack bf16 K and V [n_tokens][n_heads][head_dim] (token stride ld_kv
 * elements, >= n_heads * head_dim, % 8 == 0) into the pools.
 * `v` / `v_codes` / `v_scales` may all be NULL to pack K only.
 * head_dim must be 128.  Replaces the quantize half of
 * _all_gather_fp8 (wave_rt/denoiser/exchange/common.py:143-150) and the
 * slot copies of _publish_paged (wave_rt/denoiser/exchange/paged.py:120-141)
 * on a single GPU. */
int wf_fp8_kv_pack(const void* k, const void* v, int64_t n_tokens,
                   int32_t n_heads, int32_t head_dim, int64_t ld_kv,
                   const int32_t* page_table, int64_t n_table,
                   int32_t page_tokens, uint8_t* k_codes, uint8_t* v_codes,
                   float* k_scales, float* v_scales, int64_t pool_pages,
                   void* stream);

/* wf_fp8_kv_pack with K rotated first: each head's interleaved pairs
 * (k[2i], k[2i+1]) of token t become (a c - b s, a s + b c) in fp32 with
 * c = cos[t][i], s = sin[t][i] (fp32 [n_tokens][head_dim / 2], 16-byte
 * aligned), rounded to bf16, and the rounded values are quantized.  V is
 * packed unrotated.  The anchor re-RoPE of the exchange and its slot copy in
 * one pass: _anchor_working's _apply_rotary_emb(ku, cos, sin,
 * is_neox_style=False).type_as(v) (wave_rt/denoiser/exchange/common.py:70-91)
 * followed by Kb[off:off + T].copy_(ak) (paged.py:222-227). */
int wf_fp8_kv_pack_rope(const void* k, const void* v, int64_t n_tokens,
                        int32_t n_heads, int32_t head_dim, int64_t ld_kv,
                        const float* cos, const float* sin,
                        const int32_t* page_table, int64_t n_table,
                        int32_t page_tokens, uint8_t* k_codes,
                        uint8_t* v_codes, float* k_scales, float* v_scales,
                        int64_t pool_pages, void* stream);

/* wf_fp8_kv_pack_rope with a tiled table: token t is rotated by row
 * t % rope_rows of cos/sin ([rope_rows][head_dim / 2] fp32), 1 <= rope_rows
 * <= n_tokens.  One launch re-RoPEs a batch of equal chunks, e.g. the anchor
 * of every layer (K [n_layers * T][H][D] with rope_rows = T and a page table
 * over every layer's anchor pages in one pool): the per-layer
 * _anchor_working rotation + slot copy (wave_rt/denoiser/exchange/
 * common.py:70-91, paged.py:215-227), which uses the same table for every
 * layer of a step, for all layers at once. */
int wf_fp8_kv_pack_rope_tiled(const void* k, const void* v, int64_t n_tokens,
                              int32_t n_heads, int32_t head_dim, int64_t ld_kv,
                              const float* cos, const float* sin,
                              int64_t rope_rows, const int32_t* page_table,
                              int64_t n_table, int32_t page_tokens,
                              uint8_t* k_codes, uint8_t* v_codes,
                              float* k_scales, float* v_scales,
                              int64_t pool_pages, void* stream);

/* K straight from the fused QKV output into the pages: per token,
 * y = bf16(bf16(k * rsqrt(mean(k^2) + eps)) * norm_w) over the full row of
 * n_heads * head_dim values (as wf_rmsnorm_rope), stored to ku_out (bf16,
 * row stride ld_ku; may be K itself with ld_ku == ld_kv, or NULL) before the
 * rotation, rotated by cos/sin as in wf_fp8_kv_pack_rope (NULL: no
 * rotation), and packed; V (NULL: K only) is packed as by wf_fp8_kv_pack.
 * Results equal wf_rmsnorm_rope followed by wf_fp8_kv_pack, bit for bit.
 * n_heads * head_dim <= 16384.  Replaces norm_k (naive_rt/rolling_forcing/
 * wan/modules/causal_model.py:112-116), the key RoPE of the patched forward
 * (wave_rt/runtime/backend.py:119-121) and the self-slot publish/copy of
 * the paged exchange (wave_rt/denoiser/exchange/paged.py:206-237); ku_out
 * keeps the un-rotated key the exchange passes as unroped_key (backend.py:
 * 122-133) for a later anchor re-RoPE. */
int wf_k_norm_rope_kv_pack(const void* k, const void* v, int64_t n_tokens,
                           int32_t n_heads, int32_t head_dim, int64_t ld_kv,
                           float eps, const void* norm_w, const float* cos,
                           const float* sin, void* ku_out, int64_t ld_ku,
                           const int32_t* page_table, int64_t n_table,
                           int32_t page_tokens, uint8_t* k_codes,
                           uint8_t* v_codes, float* k_scales, float* v_scales,
                           int64_t pool_pages, void* stream);

/* Gather + dequantize the first n_tokens logical tokens of the pools back to
 * bf16 [n_tokens][n_heads][head_dim]: out = bf16_rne(float(code) * s).
 * `v_*` may be NULL to unpack K only.  Replaces the dequant of
 * _all_gather_fp8 (wave_rt/denoiser/exchange/common.py:161-164, which
 * yields fp32; here rounded once to bf16) and the context assembly of
 * _make_denoise_exch_paged (wave_rt/denoiser/exchange/paged.py:215-247). */
int wf_fp8_kv_unpack(const uint8_t* k_codes, const uint8_t* v_codes,
                     const float* k_scales, const float* v_scales,
                     int64_t pool_pages, const int32_t* page_table,
                     int64_t n_table, int32_t page_tokens, int64_t n_tokens,
                     int32_t n_heads, int32_t head_dim, void* k_out,
                     void* v_out, void* stream);

/* ------------------------------------------------------------- W8A8 int8
 *
 * Per-token activation / per-output-channel weight symmetric int8 scheme,
 * the int8 counterpart of WaveFp8Linear (wave_rt/runtime/fp8.py:21-61,
 * which quantizes per tensor to e4m3).
 */

/* Per-row int8 quantization of bf16 x [m][k] (row stride ldx elements):
 *   s[r] = max(max_c |x[r,c]| / 127, 1e-8)                 (fp32)
 *   q    = clamp(round_half_even(x / s), -127, 127)        (IEEE fp32 x / s)
 * q is dense int8 [m][k].  Used for activations (rows = tokens) and for
 * weights (rows = output channels).  k % 16 == 0; x, q 16-byte aligned.
 * Replaces the activation/weight quantization of WaveFp8Linear
 * (wave_rt/runtime/fp8.py:33-35 weights, :47-48 activations). */
int wf_act_quant_i8(const void* x, int64_t m, int64_t k, int64_t ldx,
                    int8_t* q, float* scales, void* stream);

#define WF_GEMM_GELU_TANH 1

/* int8 GEMM y[m][n] = bf16((float(acc) * sx[m]) * sw[n] + bias[n]) with
 * acc = sum_k a[m,k] * w[n,k] (int32, exact), each fp32 step rounded
 * separately.  a [m][k] and w [n][k] are int8 row-major (K contiguous);
 * bias is bf16 [n] or NULL; y has row stride ldy elements.  If acc_out is
 * non-NULL the int32 accumulators are also written ([m][n], dense).
 * flags & WF_GEMM_GELU_TANH applies GELU(tanh) to the bf16-rounded result
 * (nn.GELU(approximate='tanh') of the FFN, causal_model.py:342-344).
 * k % 16 == 0, n % 4 == 0, ldy % 4 == 0.  Replaces the torch._scaled_mm call
 * of WaveFp8Linear._raw (wave_rt/runtime/fp8.py:49-56). */
int wf_gemm_i8(const int8_t* a, const int8_t* w, int64_t m, int64_t n,
               int64_t k, const float* sx, const float* sw, const void* bias,
               void* y, int64_t ldy, int32_t* acc_out, int32_t flags,
               void* stream);

#define WF_LINEAR_GELU_INPUT 2

/* Fused W8A8 linear: wf_act_quant_i8 of x into the caller's workspace
 * (ws_q int8 [m][k], ws_sx fp32 [m]) followed by wf_gemm_i8 against the
 * pre-quantized weight (qw int8 [n][k], sw fp32 [n]).  The call contract of
 * WaveFp8Linear.forward (wave_rt/runtime/fp8.py:58-61) on 2-D input.
 * flags: WF_GEMM_GELU_TANH applies GELU(tanh) to the output (as wf_gemm_i8);
 * WF_LINEAR_GELU_INPUT quantizes bf16(GELU(tanh)(x)) in place of x -- the FFN
 * activation between fc_in and fc_out (causal_model.py:342-344) applied by
 * fc_out's input quantizer, with the values fc_in's GELU epilogue would have
 * produced. */
int wf_w8a8_linear(const void* x, int64_t m, int64_t k, int64_t ldx,
                   const int8_t* qw, const float* sw, const void* bias,
                   int64_t n, void* y, int64_t ldy, int32_t flags,
                   int8_t* ws_q, float* ws_sx, void* stream);

/* Maximum sizes of wf_w8a8_linear_static's per-GPU workspace. */
#define WF_W8A8_STATIC_MAX_CODES (64ll << 20)  /* m * k int8 activation codes */
#define WF_W8A8_STATIC_MAX_ROWS 65536ll        /* m fp32 row scales */

/* wf_w8a8_linear without the workspace arguments, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The activation codes and row scales go to a workspace held by
 * the library in a static device array of WF_W8A8_STATIC_MAX_CODES +
 * 4 * WF_W8A8_STATIC_MAX_ROWS bytes per GPU, kept until the process ends;
 * the call allocates and frees nothing.  m * k > WF_W8A8_STATIC_MAX_CODES or
 * m > WF_W8A8_STATIC_MAX_ROWS returns WF_E_SHAPE.  Every call on one GPU
 * shares that GPU's workspace: calls that overlap on one GPU (on different
 * streams, or from several threads) race and must be serialized by the
 * caller.  Results equal wf_w8a8_linear's bit for bit. */
int wf_w8a8_linear_static(const void* x, int64_t m, int64_t k, int64_t ldx,
                          const int8_t* qw, const float* sw, const void* bias,
                          int64_t n, void* y, int64_t ldy, int32_t flags,
                          void* stream);

/* ------------------------------------------------- W8A8 e4m3, per tensor
 *
 * The reference's WaveFp8Linear arithmetic (wave_rt/runtime/fp8.py:21-61):
 * one fp32 scale per weight tensor and one per activation tensor, e4m3fn
 * codes, fp32 accumulation.
 */

#define WF_FP8_TENSOR_WEIGHT 0   /* fp32 arithmetic (fp8.py:33-35) */
#define WF_FP8_TENSOR_ACT 1      /* bf16 tensor arithmetic (fp8.py:47-48) */
#define WF_FP8_AMAX_PARTIALS 1024 /* floats of the ws_partials workspace */

/* Per-tensor e4m3 quantization of bf16 x [rows][k] (row stride ldx):
 *   WF_FP8_TENSOR_WEIGHT: s = max(amax|x| / 448, 1e-8) in fp32,
 *                         codes = e4m3(fp32(x) / s);
 *   WF_FP8_TENSOR_ACT:    s = max(bf16(amax|x| / 448), bf16(1e-8)),
 *                         codes = e4m3(bf16(x / s)).
 * codes are dense u8 [rows][k]; *scale (device fp32) receives s.  ws_partials
 * holds WF_FP8_AMAX_PARTIALS floats of scratch.  rows > 0, k % 8 == 0.
 * Replaces WaveFp8Linear.__init__'s weight quantization (fp8.py:33-35) and
 * the activation quantization of WaveFp8Linear._raw (fp8.py:47-48). */
int wf_fp8_quant_pertensor(const void* x, int64_t rows, int64_t k,
                           int64_t ldx, int32_t mode, uint8_t* codes,
                           float* scale, float* ws_partials, void* stream);

/* e4m3 GEMM y[m][n] = bf16(acc * (a_scale * w_scale) + bias[n]) with
 * acc = sum_k e4m3(a[m,k]) * e4m3(w[n,k]) in fp32; a_scale and w_scale point
 * to one device fp32 each; bias bf16 [n] or NULL; y row stride ldy.
 * k % 16 == 0, n % 4 == 0, ldy % 4 == 0.  Replaces torch._scaled_mm in
 * WaveFp8Linear._raw (fp8.py:49-56). */
int wf_gemm_fp8_pertensor(const uint8_t* a, const uint8_t* w, int64_t m,
                          int64_t n, int64_t k, const float* a_scale,
                          const float* w_scale, const void* bias, void* y,
                          int64_t ldy, void* stream);

/* The whole reference linear on 2-D input: wf_fp8_quant_pertensor(x, ACT)
 * into the caller's workspace (ws_codes u8 [m][k], ws_scale fp32 [1],
 * ws_partials) followed by wf_gemm_fp8_pertensor against the weight codes
 * and scale from WF_FP8_TENSOR_WEIGHT.  WaveFp8Linear._raw, fp8.py:46-56. */
int wf_fp8_linear_pertensor(const void* x, int64_t m, int64_t k, int64_t ldx,
                            const uint8_t* w_codes, const float* w_scale,
                            const void* bias, int64_t n, void* y, int64_t ldy,
                            uint8_t* ws_codes, float* ws_scale,
                            float* ws_partials, void* stream);

/* ------------------------------------------------ FP8 KV, per tensor
 *
 * The reference's per-tensor FP8 KV exchange (_all_gather_fp8,
 * wave_rt/denoiser/exchange/common.py:143-164): one scale per [2, T, H, D]
 * K/V tensor.  The quantization is wf_fp8_quant_pertensor(kv viewed as
 * [2 T H][D], WF_FP8_TENSOR_ACT): the scale is computed in bf16 arithmetic
 * and the quotient rounded to bf16 before the e4m3 cast, as the reference's
 * bf16 tensor divided by a 0-dim fp32 scale is (common.py:145-150).
 */

/* out[i] = fp32(e4m3(codes[i])) * (*scale) for i < n (exact in fp32), the
 * reference's dequant codes.view(e4m3).to(bf16) * scale with a 1-element
 * fp32 scale, whose result is fp32 (common.py:161-164).  scale points to
 * one device fp32.  n % 16 == 0; codes and out 16-byte aligned. */
int wf_fp8_dequant_pertensor_f32(const uint8_t* codes, const float* scale,
                                 int64_t n, float* out, void* stream);

/* ------------------------------------------------------------- attention */

/* Attention of bf16 queries q [lq][n_heads][128] (token stride ldq
 * elements) over the first n_kv logical keys of the FP8 paged pools (layout
 * as for wf_fp8_kv_pack), non-causal within the context:
 *   out[q,h,:] = softmax_j(softmax_scale * <q[q,h,:], K[j,h,:]>) . V[j,h,:]
 * with K = code_k * s_k and V = code_v * s_v per (key, head); fp32
 * accumulation, bf16 out [lq][n_heads][128] (token stride ldo).
 * page_tokens >= 64; each code pool < 2 GiB.  n_kv == 0 writes zero rows
 * (the pools may then be NULL).  Replaces the attention
 * dispatch of the patched self-attention (wave_rt/runtime/backend.py:141-148:
 * fa_func / sageattn / SDPA over the paged context views of
 * wave_rt/denoiser/exchange/paged.py:246-247). */
int wf_attn_paged_fp8(const void* q, int64_t lq, int32_t n_heads,
                      int32_t head_dim, int64_t ldq, const uint8_t* k_codes,
                      const uint8_t* v_codes, const float* k_scales,
                      const float* v_scales, int64_t pool_pages,
                      int32_t page_tokens, const int32_t* page_table,
                      int64_t n_table, int64_t n_kv, float softmax_scale,
                      void* out, int64_t ldo, void* stream);

/* The quantized-QK form of wf_attn_paged_fp8, same arguments: the
 * counterpart of the reference's SageAttention backend (enable_sage /
 * sageattn, wave_rt/runtime/backend.py:57-62,144-146), which quantizes Q and
 * K before QK^T.  Each query row (per head) is quantized to e4m3 with a
 * power-of-two scale s_q, the smallest with amax|q| <= 448 s_q; scores are
 * sum_d code_q * code_k from the fp8 matrix cores (fp32 accumulation) times
 * s_k * s_q; V and the softmax are exact as in wf_attn_paged_fp8.
 * Approximate by design (e4m3 queries carry 3 mantissa bits). */
int wf_attn_paged_fp8_qk8(const void* q, int64_t lq, int32_t n_heads,
                          int32_t head_dim, int64_t ldq,
                          const uint8_t* k_codes, const uint8_t* v_codes,
                          const float* k_scales, const float* v_scales,
                          int64_t pool_pages, int32_t page_tokens,
                          const int32_t* page_table, int64_t n_table,
                          int64_t n_kv, float softmax_scale, void* out,
                          int64_t ldo, void* stream);

/* wf_attn_paged_fp8_qk8 with the P.V product on the fp8 matrix cores as
 * well, same arguments: the counterpart of the fp8 P.V product of the
 * reference's SageAttention backend (sageattn, wave_rt/runtime/backend.py:
 * 57-62,144-146).  V stays as the pages' e4m3 codes; each query's weights
 * p_k * s_v,k of a 64-key tile are rounded to e4m3 after division by a
 * power of two 2^E (the smallest with their maximum <= 448 * 2^E), which
 * the matrix cores multiply back; the row sum is the fp32 sum of the
 * unrounded p_k.  Approximate by design: each weight carries 3 mantissa
 * bits. */
int wf_attn_paged_fp8_qkpv8(const void* q, int64_t lq, int32_t n_heads,
                            int32_t head_dim, int64_t ldq,
                            const uint8_t* k_codes, const uint8_t* v_codes,
                            const float* k_scales, const float* v_scales,
                            int64_t pool_pages, int32_t page_tokens,
                            const int32_t* page_table, int64_t n_table,
                            int64_t n_kv, float softmax_scale, void* out,
                            int64_t ldo, void* stream);

/* Attention of q [lq][n_heads][128] over dense bf16 K, V [n_kv][n_heads][128]
 * (token stride ldkv elements), same math and output as wf_attn_paged_fp8
 * with unit scales.  Replaces the text cross-attention's flash_attention
 * call (naive_rt/rolling_forcing/wan/modules/model.py:189, the SDPA
 * fallback attention.py:75-89) over the cached 512-token text K/V. */
int wf_attn_dense_bf16(const void* q, int64_t lq, int32_t n_heads,
                       int32_t head_dim, int64_t ldq, const void* k,
                       const void* v, int64_t n_kv, int64_t ldkv,
                       float softmax_scale, void* out, int64_t ldo,
                       void* stream);

/* ------------------------------------------------- block row-wise stages */

/* y = LayerNorm(x) (fp32 statistics, optional bf16 affine w/b, rounded to
 * bf16), then, if given, the bf16 modulation y = bf16(bf16(y * bf16(1 +
 * scale[f])) + shift[f]) with f = row / frame_tokens (scale/shift bf16
 * frame rows of stride ld_mod elements, at least ceil(T / frame_tokens)
 * of them: the kernel cannot check); writes y (bf16, row stride ldo) if
 * out != NULL and its per-token int8 quantization (as wf_act_quant_i8) if
 * q != NULL.  dim % 8 == 0, dim <= 16384.  Replaces norm1/norm2 +
 * modulation (naive_rt/rolling_forcing/wan/modules/causal_model.py:381,
 * 393-394) and norm3 (:390, model.py:89-99) feeding the W8A8 linears. */
int wf_ln_modulate_quant(const void* x, int64_t T, int32_t dim, int64_t ldx,
                         float eps, const void* w, const void* b,
                         const void* shift, const void* scale,
                         int64_t ld_mod, int32_t frame_tokens, void* out,
                         int64_t ldo, int8_t* q, float* q_scales,
                         void* stream);

/* The residual that precedes a norm, fused into it: first, in place,
 * x = bf16(x + bf16(y * gate[f])) (gate frame rows of stride ld_gate,
 * at least ceil(T / frame_tokens) of them), or
 * x = bf16(x + y) when gate is NULL, then wf_ln_modulate_quant of the
 * updated x (out must not alias x).  y == NULL skips the residual.  The
 * self-attention residual + norm3 (causal_model.py:386-390) and the
 * cross-attention residual + norm2 + modulation (:390-394). */
int wf_gate_residual_ln_quant(void* x, int64_t T, int32_t dim, int64_t ldx,
                              const void* y, int64_t ldy, const void* gate,
                              int64_t ld_gate, float eps, const void* w,
                              const void* b, const void* shift,
                              const void* scale, int64_t ld_mod,
                              int32_t frame_tokens, void* out, int64_t ldo,
                              int8_t* q, float* q_scales, void* stream);

/* y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w) over the full row (dim),
 * then, if cos/sin ([T][head_dim/2] fp32) are given, each head's
 * interleaved pairs (y[2i], y[2i+1]) are rotated by angle i of the row.
 * Replaces norm_q/norm_k (causal_model.py:112-116, model.py:70-86) and the
 * RoPE of the patched forward (wave_rt/runtime/backend.py:119-121). */
int wf_rmsnorm_rope(const void* x, int64_t T, int32_t dim, int64_t ldx,
                    int32_t head_dim, float eps, const void* w,
                    const float* cos, const float* sin, void* out,
                    int64_t ldo, void* stream);

/* In place x = bf16(x + bf16(y * gate[row / frame_tokens])), or
 * x = bf16(x + y) when gate is NULL (ceil(T / frame_tokens) gate bf16
 * frame rows of stride ld_gate elements).  The gated residuals of
 * causal_model.py:386,397-398 and the cross-attention residual of :390. */
int wf_gate_residual(void* x, int64_t ldx, const void* y, int64_t ldy,
                     const void* gate, int64_t ld_gate, int64_t T,
                     int32_t dim, int32_t frame_tokens, void* stream);

/* wf_k_norm_rope_kv_pack with Q done in the same pass: Q [n_tokens][ld_q]
 * (the Q columns of the fused QKV output) gets
 * bf16(bf16(q * rsqrt(mean(q^2) + eps)) * norm_q) and the same rotation as
 * K, written back in place; bit-identical to wf_rmsnorm_rope on Q followed by
 * wf_k_norm_rope_kv_pack.  The self-attention q/k RMSNorm + RoPE and K/V
 * publish of one layer (causal_model.py:112-116, wave_rt/runtime/
 * backend.py:119-121, paged.py:215-237) in one launch.  q must not overlap
 * K, V or ku_out (interleaved column slices of one QKV row are fine). */
int wf_qk_norm_rope_kv_pack(void* q, int64_t ld_q, const void* norm_q,
                            const void* k, const void* v, int64_t n_tokens,
                            int32_t n_heads, int32_t head_dim, int64_t ld_kv,
                            float eps, const void* norm_k, const float* cos,
                            const float* sin, void* ku_out, int64_t ld_ku,
                            const int32_t* page_table, int64_t n_table,
                            int32_t page_tokens, uint8_t* k_codes,
                            uint8_t* v_codes, float* k_scales,
                            float* v_scales, int64_t pool_pages, void* stream);

/* ---------------------------------------------------------------------
 * The DiT around the blocks (bf16, as the reference runs it)
 * ------------------------------------------------------------------- */

#define WF_BF16_SILU_IN 1    /* SiLU on a's elements (rounded to bf16) first */
#define WF_BF16_SILU_OUT 2   /* SiLU on the bf16 output, rounded to bf16 */
#define WF_BF16_GELU_OUT 4   /* GELU(tanh) on the bf16 output, rounded to bf16 */

/* bf16 GEMM y[m][n] = act_out(bf16(sum_k act_in(a[m,k]) * w[n,k] + bias[n]))
 * with fp32 accumulation: a [m][k] (row stride lda), w [n][k] dense (nn.Linear
 * layout), bias bf16 [n] or NULL, y bf16 (row stride ldy).  k, lda % 8 == 0;
 * n, ldy % 4 == 0; a, w 16-byte and y 8-byte aligned.  The bf16 linears of
 * the Wan DiT outside its blocks: the text embedding (Linear, GELU(tanh),
 * Linear), the time embedding (Linear, SiLU, Linear), the time projection
 * (SiLU, Linear), the head's Linear, and the patch embedding over
 * wf_patchify_bf16's patches (naive_rt/rolling_forcing/wan/modules/
 * causal_model.py:406-433,517-528). */
int wf_gemm_bf16(const void* a, int64_t m, int64_t k, int64_t lda,
                 const void* w, int64_t n, const void* bias, void* y,
                 int64_t ldy, int32_t flags, void* stream);

/* Patches of the Conv3d patch embedding (kernel = stride = (1, 2, 2)):
 * x bf16 [b][c][f][h][w] -> out bf16 [b][f * (h/2) * (w/2)][c * 4] with
 * out[b][t][4 ci + 2 kh + kw] = x[b][ci][fi][2 yi + kh][2 xi + kw] for token
 * t = (fi, yi, xi) -- the (c, kt, kh, kw) order of the Conv3d weight, so the
 * embedding is wf_gemm_bf16 against the weight viewed as [dim][4 c]
 * (causal_model.py:517-518, the flatten(2).transpose(1, 2) of :826-830).
 * h and w even. */
int wf_patchify_bf16(const void* x, int64_t b, int32_t c, int32_t f,
                     int32_t h, int32_t w, void* out, void* stream);

/* Unpatchify the head output and convert the flow prediction to x0:
 * flow[b][ci][fi][2 yi + q][2 xi + r] = head[b][t(fi, yi, xi)][(2 q + r) c + ci]
 * ('fhwpqrc->cfphqwr', causal_model.py:1080-1103, patch (1, 2, 2)), then
 * x0 = xt - sigma * flow in float64 (wan_wrapper.py:169-193), converted to
 * bf16 through float32 as torch converts float64, and written as
 * x0 [b][f][c][h][w] (the (B, T, C, H, W) x0 of forward_chunk,
 * wave_rt/runtime/backend.py:456-490).  xt bf16 [b][c][f][h][w]; h, w even. */
int wf_unpatchify_flow_x0_bf16(const void* head, const void* xt, int64_t b,
                               int32_t c, int32_t f, int32_t h, int32_t w,
                               double sigma, void* x0, void* stream);

/* ---------------------------------------------------------------------
 * Re-noising for the next DMD step
 * ------------------------------------------------------------------- */

/* out = bf16((1 - sigma) * x0 + sigma * noise), every product, the
 * difference 1 - sigma and the sum an fp32 operation: the
 * FlowMatchScheduler.add_noise of _det_renoise
 * (naive_rt/rolling_forcing/utils/scheduler.py:159-176,
 * wave_rt/denoiser/engine.py:221-235) with one sigma for all frames.
 * x0 and out are bf16 [batch][channels][frames][plane] (plane = h * w);
 * noise is bf16 in the same layout, or frame-major
 * [batch][frames][channels][plane] when noise_frame_major != 0 (the order
 * _det_renoise draws it in).  out may alias x0, not a frame-major noise. */
int wf_flow_add_noise_bf16(const void* x0, const void* noise, int64_t batch,
                           int64_t channels, int64_t frames, int64_t plane,
                           int32_t noise_frame_major, float sigma, void* out,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WF_API_H */
