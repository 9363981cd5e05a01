/*
 * dspark_hip.h -- C ABI of the MI355X speculative-decoding verify engine
 * (libdspark_hip.so, gfx950).
 *
 * The reference (regeter/mlx-dspark v0.3.1) has no native code: every kernel on its hot
 * path is an MLX primitive called from Python. Each entry point below replaces one of those
 * primitive call sites; the comment names the reference call site (file:line, paths
 * relative to the reference root) whose behaviour it reproduces.
 *
 * Conventions (all entry points):
 *   - return 0 (DSK_OK) on success, a negative DSK_E* code on failure; the message is kept
 *     per thread and returned by dsk_last_error(). Nothing throws across this boundary.
 *   - every device buffer is allocated by the caller; kernels never allocate and never
 *     synchronise. Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 *   - lengths that change from one decode round to the next (sequence lengths, accepted
 *     counts) live in device memory, so a captured HIP graph replays correctly.
 *   - bf16 tensors are passed as uint16_t (raw bits); "W8" means MLX's affine 8-bit format,
 *     group 64: w = scale * q + bias with bf16 scale/bias per 64 consecutive input columns.
 */
#ifndef DSPARK_HIP_H
#define DSPARK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dsk_stream_t; /* hipStream_t */

enum {
  DSK_OK = 0,
  DSK_EINVAL = -1,  /* bad shape / argument */
  DSK_ELAUNCH = -2, /* HIP launch or runtime error */
  DSK_ERANGE = -3,  /* size beyond a documented maximum */
  DSK_ENOWS = -4    /* workspace too small */
};

enum { DSK_F32 = 0, DSK_BF16 = 1 };

enum { DSK_KV_BF16 = 0, DSK_KV_U8 = 1 };

const char* dsk_last_error(void);
int dsk_abi_version(void);

/* ---------------------------------------------------------------------------------------
 * W8 weights.
 * Replaces nn.quantize(..., bits=8, group_size=64) (src/mlx_dspark/load.py:204-206,
 * :285-286) for the weights this engine creates, and the MLX-format packed weight that
 * nn.QuantizedLinear holds (external mlx; used by the target layers reached from
 * src/mlx_dspark/target.py:66-67, the layer loop of _run_mlxlm).
 *
 * dsk_w8_quantize: w [N, K] (f32 or bf16, row-major) -> q [N, K] u8 (byte order identical
 *   to MLX's uint32 packing, low byte first), scales/biases [N, K/64] bf16.
 *   Rule per group of 64: lo = min, hi = max, scale = bf16((hi - lo) / 255) (scale = 1
 *   when hi == lo), bias = bf16(lo), q = clamp(rint((w - bias) / scale), 0, 255).
 * dsk_w8_repack: MLX layout -> the engine's tiled HBM layout consumed by dsk_w8_gemm:
 *   wt [N/16][K/64][64 lanes][16 B], sb [N/16][K/64][16] u32 (bf16 scale | bf16 bias << 16).
 *   N % 16 == 0, K % 64 == 0. paired != 0 (gated MLPs, N % 32 == 0): rows [0, N/2) are the
 *   gate projection and [N/2, N) the up projection; tile 2p takes gate rows 16p..16p+15 and
 *   tile 2p+1 up rows 16p..16p+15, as dsk_w8_gemm's gated epilogues expect.
 * ------------------------------------------------------------------------------------- */
int dsk_w8_quantize(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q,
                    uint16_t* scales, uint16_t* biases, dsk_stream_t stream);
int dsk_w8_repack(const uint8_t* q, const uint16_t* scales, const uint16_t* biases, int64_t N,
                  int64_t K, int paired, uint8_t* wt, uint32_t* sb, dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Packed activations.
 * The W8 GEMM reads its activation operand in a packed layout: element (m, k) of an [M, K]
 * bf16 matrix lives at P[m/16][k/64][m%16 + 16*((k%64)/16)][k%16] (dsk_act_pack_bytes(M, K)
 * bytes; rows past M are padding with arbitrary values).
 *
 * dsk_act_pack builds it, fusing what precedes every projection of a decoder layer:
 *   v = part ? sum_{s < nsplit} part[s][m][k] : 0      (fp32 partial sums of a split-K
 *                                                       GEMM, slice stride M*K, in order)
 *   part_norm_w != NULL (gemma sandwich norms: the post-attention / post-feedforward norm of
 *   the projection output before the residual add):
 *     v = bf16((bf16(v) * rsqrt(mean_k(bf16(v)^2) + eps)) * part_norm_w[k])
 *   v = h ? (part ? bf16(h[m][k] + v) : h[m][k]) : bf16(v)    (residual add; h updated in
 *                                                               place when part != NULL)
 *   copy[m][k] = v                                     (copy != NULL: hidden-state tap)
 *   out = packed(norm_w ? bf16((v * rsqrt(mean_k(v^2) + eps)) * norm_w[k]) : v)
 * It replaces the residual adds of the Qwen3 layers (mlx_lm), the hidden-state capture of
 * src/mlx_dspark/target.py:68-69 and mx.fast.rms_norm (src/mlx_dspark/model.py:28,
 * nn.RMSNorm at :103-106, :165-170, :233-235, dflash_model.py:96-99, and the Qwen3 input /
 * post-attention / final norms inside mlx_lm). M <= 64, K % 64 == 0, K <= 24576, row strides
 * multiples of 8, 16-byte aligned pointers; out may be NULL (h update / copy only).
 * ------------------------------------------------------------------------------------- */
size_t dsk_act_pack_bytes(int M, int64_t K);
int dsk_act_pack(const float* part, int nsplit, const uint16_t* part_norm_w, uint16_t* h,
                 int64_t ldh, uint16_t* copy, int64_t ldc, int M, int64_t K,
                 const uint16_t* norm_w, float eps, uint16_t* out, dsk_stream_t stream);
/* dsk_act_pack with the residual-stream result scaled before it is stored, copied and normed:
 * v = bf16(v * out_scale) after the residual add (the gemma4 drafter layer's layer_scalar,
 * src/mlx_dspark/model.py:181-184). out_scale 1 is dsk_act_pack. */
int dsk_act_pack_scaled(const float* part, int nsplit, const uint16_t* part_norm_w, uint16_t* h,
                        int64_t ldh, uint16_t* copy, int64_t ldc, int M, int64_t K,
                        const uint16_t* norm_w, float eps, float out_scale, uint16_t* out,
                        dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * W8 skinny GEMM: y[M, N] = x[M, K] . deq(W)[N, K]^T
 * Replaces mx.quantized_matmul behind nn.QuantizedLinear (external mlx), reached from
 * src/mlx_dspark/target.py:66-74 (every target projection and the lm_head / tied
 * embed_tokens.as_linear), src/mlx_dspark/batch_engine.py:199-204 (batched verify) and
 * the drafter linears (src/mlx_dspark/model.py:97-101, :230-236; dflash_model.py:93-96).
 *
 * x: packed (dsk_act_pack). W: dsk_w8_repack layout. M <= 64, N % 16 == 0, K % 256 == 0.
 * epi = DSK_EPI_STORE: y f32 or bf16 [M, N] (row stride ldy) = residual + x.W^T, residual
 *   NULL or bf16 [M, N] with row stride ldr (may alias y when y is bf16); softcap > 0
 *   applies y = tanh(y / softcap) * softcap (src/mlx_dspark/model.py:264-268).
 * epi = DSK_EPI_PARTIAL: y f32 [S][M][N], S = dsk_w8_gemm_splits(M, N, K) partial sums over
 *   disjoint K ranges (their sum, in slice order, is the product; dsk_act_pack and
 *   dsk_qkv_rope_append take them as input).
 * epi = DSK_EPI_SWIGLU / DSK_EPI_GEGLU: W is a paired gate|up repack (N = 2 I, I % 128 == 0);
 *   y = packed bf16 [M, I] of bf16(bf16(act(bf16(gate))) * bf16(up)), act = silu or
 *   tanh-approximated gelu (the MLP of src/mlx_dspark/model.py:35-45 and of the Qwen3 /
 *   Gemma layers), ready as the next GEMM's x.
 * No workspace; no state is kept between calls.
 * ------------------------------------------------------------------------------------- */
enum { DSK_EPI_STORE = 0, DSK_EPI_SWIGLU = 1, DSK_EPI_GEGLU = 2, DSK_EPI_PARTIAL = 3, DSK_EPI_RESIDUAL = 4 };
int dsk_w8_gemm_splits(int M, int64_t N, int64_t K);
int dsk_w8_gemm(const uint16_t* x, const uint8_t* wt, const uint32_t* sb, int M, int64_t N,
                int64_t K, int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual,
                int64_t ldr, float softcap, dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Normed-later activations: the RMSNorm that precedes a projection applied after it.
 * Replaces, for the Qwen3 layout, the chain residual add -> mx.fast.rms_norm -> quantized
 * matmul of every decoder layer (input / post-attention norms inside mlx_lm, reached from the
 * layer loop of src/mlx_dspark/target.py:66-67) and the final norm before the head
 * (target.py:70-74). RMSNorm(h) . W^T = r * (bf16(h * w) . W^T) with r = rsqrt(mean(h^2) + eps)
 * per row, so the producer of h writes x = bf16(h * w) packed plus per-16-column partial sums
 * of h^2, ssq[m][k / 16] (fp32, [M][K / 16]), and the consuming GEMM multiplies each output of
 * row m by r_m = rsqrt(sum_t ssq[m][t] / K + eps) before its epilogue (the partials summed
 * in tile order t, t + 64, ... per lane, then across the wave: the same order in every
 * kernel). Each 16-column partial is the balanced tree ((h0^2 + h1^2) + (h2^2 + h3^2)) + ...
 *
 * dsk_act_pack_rn: dsk_act_pack's residual add (part may be NULL: v = h), then copy[m][k] = v,
 *   out = packed bf16(v * norm_w[k]) (norm_w NULL: v) and ssq_out[m][k / 16].
 * dsk_w8_gemm_rn: dsk_w8_gemm (bits 8) or dsk_w4_gemm (bits 4) whose x is normed later when
 *   x_ssq != NULL (x_tiles = K / 16 partials of x's rows, eps the norm's epsilon), plus
 *   epi = DSK_EPI_RESIDUAL (o_proj / down_proj and the residual add after them): no K split;
 *   h[m][n] = bf16(h[m][n] + y) in place (row stride ldh), copy[m][n] = h (row stride ldc,
 *   or NULL: hidden-state tap, target.py:68-69), y = packed bf16(h * next_norm_w[n]) (the
 *   next projection's x, normed later; next_norm_w NULL: h; y may be NULL) and ssq_out as
 *   above. N % 64 == 0; the other limits are dsk_w8_gemm's.
 * ------------------------------------------------------------------------------------- */
int dsk_act_pack_rn(const float* part, int nsplit, uint16_t* h, int64_t ldh, uint16_t* copy,
                    int64_t ldc, int M, int64_t K, const uint16_t* norm_w, uint16_t* out,
                    float* ssq_out, dsk_stream_t stream);
int dsk_w8_gemm_rn(const uint16_t* x, const uint8_t* wt, const uint32_t* sb, int bits, int M,
                   int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy, float softcap,
                   const float* x_ssq, int x_tiles, float eps, uint16_t* h, int64_t ldh,
                   uint16_t* copy, int64_t ldc, const uint16_t* next_norm_w, float* ssq_out,
                   dsk_stream_t stream);

/* Tuning entry, with no counterpart in the reference: dsk_w8_gemm_rn with an explicit plan instead
 * of the library's own, for plan sweeps (the planner's rules were fitted from such sweeps):
 * slab_tiles 16-row weight tiles per workgroup (dividing N / 16; even for the gated epilogues),
 * batch_groups 2 or 4 groups of 64 along K per load batch, waves 4 / 8 / 16, k_splits K splits
 * (DSK_EPI_PARTIAL only: y then holds k_splits slices [M][N]), pipelined loads (1) or not (0).
 * A plan with no compiled kernel, or whose cross-wave reduction exceeds 64 KB of LDS, is
 * rejected with DSK_EINVAL. */
int dsk_w8_gemm_rn_planned(const uint16_t* x, const uint8_t* wt, const uint32_t* sb, int bits, int M,
                           int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy,
                           float softcap, const float* x_ssq, int x_tiles, float eps, uint16_t* h,
                           int64_t ldh, uint16_t* copy, int64_t ldc, const uint16_t* next_norm_w,
                           float* ssq_out, int slab_tiles, int batch_groups, int waves, int k_splits,
                           int pipelined, dsk_stream_t stream);

/* Introspection entry, with no counterpart in the reference: the plan dsk_w8_gemm / dsk_w8_gemm_rn
 * run for this shape and epilogue, as plan[5] = {slab_tiles, batch_groups, waves, k_splits,
 * pipelined} in the terms of dsk_w8_gemm_rn_planned (for plan sweeps and to name the kernel
 * instantiation a measurement covers). */
int dsk_w8_gemm_plan(int M, int64_t N, int64_t K, int epi, int bits, int* plan);

/* ---------------------------------------------------------------------------------------
 * Dense prefill (src/mlx_dspark/generate.py:613-656, _prefill_tapped: the prompt in chunks of
 * PREFILL_CHUNK = 2048 rows through the target). A long prompt runs layer by layer over all of
 * its rows: each layer's weights are expanded to bf16 once and multiplied by a library GEMM
 * (hipBLASLt), with these kernels around it.
 * dsk_w8_dequant_rows: a dsk_w8_repack (bits 8) / dsk_w4_repack (bits 4) weight -> bf16 [N, K]
 *   rows out[n][k] = bf16(s * q + b) in source row order (paired: gate rows, then up rows).
 * dsk_rows_rmsnorm: y[m] = bf16((x[m] * rsqrt(mean(x[m]^2) + eps)) * w) for M rows (the
 *   RMSNorm formula of dsk_act_pack), row strides ldx / ldy.
 * dsk_rows_gated: out[m][i] = bf16(bf16(act(gate)) * up) with gate = gu[m][i], up = gu[m][I + i],
 *   act = DSK_EPI_SWIGLU (SiLU) or DSK_EPI_GEGLU (tanh GeLU), as dsk_w8_gemm's gated epilogue.
 * ------------------------------------------------------------------------------------- */
int dsk_w8_dequant_rows(const uint8_t* wt, const uint32_t* sb, int bits, int64_t N, int64_t K,
                        int paired, uint16_t* out, dsk_stream_t stream);
int dsk_rows_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps, int64_t M,
                     int64_t K, uint16_t* y, int64_t ldy, dsk_stream_t stream);
int dsk_rows_gated(const uint16_t* gu, int64_t ldg, int64_t M, int64_t I, int act, uint16_t* out,
                   int64_t ldo, dsk_stream_t stream);

/* 4-bit codes (MLX nn.quantize bits=4, group 64: the reference's drafter default,
 * src/mlx_dspark/load.py:155-215, :224-289 with bits=4; 4-bit target checkpoints).
 * dsk_w4_quantize: as dsk_w8_quantize with codes 0..15 (s = (max - min) / 15), one per byte.
 * dsk_w4_repack: codes [N, K] one per byte -> wt [N * K / 2] in the W8 tile order with two
 *   codes per byte (byte j of a lane's 8 = columns 2j | 2j+1 << 4); sb as dsk_w8_repack.
 * dsk_w4_gemm: dsk_w8_gemm (same arguments, epilogues and limits) on that layout; its
 *   DSK_EPI_PARTIAL slice count is dsk_w4_gemm_splits(M, N, K). */
int dsk_w4_gemm_splits(int M, int64_t N, int64_t K);
int dsk_w4_quantize(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q,
                    uint16_t* scales, uint16_t* biases, dsk_stream_t stream);
int dsk_w4_repack(const uint8_t* q, const uint16_t* scales, const uint16_t* biases, int64_t N,
                  int64_t K, int paired, uint8_t* wt, uint32_t* sb, dsk_stream_t stream);
int dsk_w4_gemm(const uint16_t* x, const uint8_t* wt, const uint32_t* sb, int M, int64_t N,
                int64_t K, int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual,
                int64_t ldr, float softcap, dsk_stream_t stream);

/* W8 row gather (embedding lookup): out[i, :] = bf16(deq(table)[ids[i], :]) * scale.
 * Replaces nn.QuantizedEmbedding (mm.embed_tokens, src/mlx_dspark/target.py:63;
 * drafter.embed, src/mlx_dspark/model.py:244-245; dflash_model.py:198).
 * table in MLX layout: q [V, H] u8, scales/biases [V, H/64] bf16. */
int dsk_w8_embed(const int32_t* ids, int n, const uint8_t* q, const uint16_t* scales,
                 const uint16_t* biases, int64_t V, int64_t H, float scale, uint16_t* out,
                 int64_t ldo, dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Paged KV cache.
 * Replaces mlx_lm KVCache / QuantizedKVCache (src/mlx_dspark/target.py:36-48) and the
 * per-row BatchCache (src/mlx_dspark/batch_engine.py:61-163).
 * A pool holds fixed pages of `page` tokens; page p, kv-head h, slot t:
 *   bf16: kv[p][h][t][hd] bf16
 *   u8:   kv[p][h][t][hd] u8 + sb[p][h][t][hd/64] u32 (bf16 scale | bf16 bias << 16),
 *         affine group-64 along head_dim, same rule as dsk_w8_quantize.
 * block_table [B, max_pages] int32 maps a row's logical page j to a physical page.
 * seq_lens [B] int32 = tokens cached per row before the call (device memory).
 * ------------------------------------------------------------------------------------- */

/* qkv: the fused projection of B*W rows (row b*W + i), either bf16 [B*W, (nq + 2*nkv) * hd]
 * (qkv_splits == 0) or the fp32 partial sums of dsk_w8_gemm DSK_EPI_PARTIAL
 * [qkv_splits][B*W][(nq + 2*nkv) * hd] (summed in order and rounded to bf16) -> per-head RMSNorm of q and k
 * (q_norm/k_norm weights [hd] bf16), rotate-half RoPE at position seq_lens[b] + i
 * (inv_freq [hd/2] f32), K/V appended to the pool at that position, and
 * q_out [B*W, nq*hd] bf16. Replaces the Qwen3 attention prologue inside mlx_lm and
 * DSparkAttention._kv/update_ctx (src/mlx_dspark/model.py:113-128). k_norm may be NULL
 * (no norm). pos_offset is added to every position. nq may be 0 (K/V rows only, as for a
 * drafter's context rows; q_out may then be NULL). */
int dsk_qkv_rope_append(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                        const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                        const float* inv_freq, const int32_t* seq_lens, int pos_offset,
                        const int32_t* block_table, int max_pages, int page, int kv_dtype,
                        void* k_pool, void* v_pool, uint32_t* k_sb, uint32_t* v_sb,
                        uint16_t* q_out, dsk_stream_t stream);
/* dsk_qkv_rope_append with an RMSNorm on V as well (v_norm weights [hd] bf16, NULL for
 * none; V is not rotated): the gemma4 DSpark drafter's v_norm, which with k_eq_v normalises
 * the shared k_proj output (src/mlx_dspark/model.py:113-124; RMSNormNoScale is a v_norm of
 * ones). head_dim 128, 256 or 512. */
int dsk_qkv_norm_rope_append(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv,
                             int hd, const uint16_t* q_norm, const uint16_t* k_norm,
                             const uint16_t* v_norm, float eps, const float* inv_freq,
                             const int32_t* seq_lens, int pos_offset, const int32_t* block_table,
                             int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool,
                             uint32_t* k_sb, uint32_t* v_sb, uint16_t* q_out, dsk_stream_t stream);

/* Attention of W new queries per row over the row's paged KV (already holding the W new
 * tokens at positions seq_lens[b] .. seq_lens[b]+W-1).
 * causal != 0: query i sees keys j <= seq_lens[b] + i  (mlx_lm create_attention_mask with
 *   offset, src/mlx_dspark/target.py:64; build_batch_mask, batch_engine.py:170-178).
 *   window > 0 additionally hides keys j <= seq_lens[b] + i - window (sliding layers).
 * causal == 0: every query sees all seq_lens[b] + W keys (DSpark/DFlash block attention,
 *   src/mlx_dspark/model.py:130-155, dflash_model.py:123-133).
 * q [B*W, nq*hd] bf16 -> out [B*W, nq*hd] bf16. GQA: q head h reads kv head h/(nq/nkv).
 * max_ctx bounds seq_lens[b] + W (sizes the split grid so the launch is graph-stable).
 * softcap > 0: scores = tanh(scores / softcap) * softcap before the mask.
 * out_packed != 0 writes the output in the packed activation layout (the o-projection's x).
 * Probabilities stay float32: the P.V products run as three bf16 MFMAs over P's hi + mid + lo
 * terms (within 2^-26 of the float32 value) and the row sums add the float32 P; the many-query
 * form below (a prefill, MFMA-heavy) uses the first two terms (within 2^-17) for both.
 * workspace: dsk_attn_ws_bytes(...) bytes for the split partials (fp32 o / l per split and
 * fp32 (m, l); the splits are combined by a second kernel on the same stream; no state is
 * kept between calls). Every block_table entry of a row must name a valid page: a split
 * reads its whole key range through the table before it knows the row's length.
 * head_dim 128 or 256, or 512 (the gemma4 drafter's global head) without the fused entry.
 * Verify passes (at most 80 query rows W * nq / nkv per kv head at head_dim 128, 64 at 256, page
 * a multiple of 32) take splits of 256 (128) keys; with a sliding window only the splits of one
 * window are launched, each row's placed from its seq_lens entry on the device.
 * W > 64 (a prefill's many queries), head_dim 128, no softcap, unpacked output and at most
 * 1024 pages per row: one workgroup per 256 query rows of a (row, kv head) streams that block's
 * whole key range, with no splits, no combine and no workspace use. Other many-query passes take
 * groups of 4 query tiles over splits of 1024 keys, a causal split past every query of a group
 * skipped (each row's combine reads the splits up to its own position). */
size_t dsk_attn_ws_bytes(int B, int W, int nq, int hd, int max_ctx);
int dsk_attention(const uint16_t* q, int B, int W, int nq, int nkv, int hd, float scale,
                  int causal, int window, float softcap, const int32_t* seq_lens,
                  int max_ctx, const int32_t* block_table, int max_pages, int page,
                  int kv_dtype, const void* k_pool, const void* v_pool,
                  const uint32_t* k_sb, const uint32_t* v_sb, uint16_t* out, int out_packed,
                  void* workspace, size_t ws_bytes, dsk_stream_t stream);

/* dsk_qkv_rope_append (pos_offset 0) for a projection whose input was normed later
 * (dsk_w8_gemm_rn): the summed split-K partials of row m are multiplied by
 * r_m = rsqrt(sum_t x_ssq[m][t] / (16 x_tiles) + x_eps) before they are rounded to bf16, q/k
 * normed and roped (the input RMSNorm of the Qwen3 layer, applied after q/k/v_proj);
 * qkv_splits >= 1 (f32 slices). */
int dsk_qkv_rope_append_rn(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                           const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                           const float* inv_freq, const int32_t* seq_lens, const int32_t* block_table,
                           int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool,
                           uint32_t* k_sb, uint32_t* v_sb, uint16_t* q_out, const float* x_ssq,
                           int x_tiles, float x_eps, dsk_stream_t stream);

/* dsk_qkv_rope_append followed by dsk_attention in one kernel (plus the split combine):
 * from the qkv projection (bf16 or fp32 split-K slices, as for dsk_qkv_rope_append, with
 * pos_offset 0) each workgroup forms its queries (q RMSNorm, RoPE at seq_lens[b] + i); the
 * workgroup whose key range holds the W new tokens normalises and rotates their K, appends
 * K/V to the pool and attends to the appended values directly. Same masks, output and
 * workspace (dsk_attn_ws_bytes) as dsk_attention; W <= 64; q_norm/k_norm may be NULL and,
 * when given, are 16-byte aligned. Replaces the attention block of a decoder layer between
 * the qkv and o projections (mlx_lm Qwen3 attention reached from
 * src/mlx_dspark/target.py:66-67; DSparkAttention, src/mlx_dspark/model.py:130-155;
 * DFlash attention, src/mlx_dspark/dflash_model.py:100-133). */
int dsk_qkv_attention(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                      const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                      const float* inv_freq, float scale, int causal, int window, float softcap,
                      const int32_t* seq_lens, int max_ctx, const int32_t* block_table,
                      int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool,
                      uint32_t* k_sb, uint32_t* v_sb, uint16_t* out, int out_packed,
                      void* workspace, size_t ws_bytes, dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Acceptance.
 * ------------------------------------------------------------------------------------- */

/* Greedy: tt[b, i] = argmax_v logits[b, i, :] (lowest index on ties), i < W;
 * n[b] = number of leading i < W-1 with draft[b, i] == tt[b, i];  token[b] = tt[b, n[b]];
 * seq_lens[b] += n[b] + 1 when seq_lens != NULL (the KV rollback to the accepted length:
 * W tokens were appended by the verify, W - 1 - n are trimmed).
 * Replaces src/mlx_dspark/generate.py:910-933 (DSpark), :557-579 (DFlash),
 * src/mlx_dspark/batch_engine.py:573-595 (batched). logits f32 or bf16 [B, W, V]
 * (row stride ldl elements), draft [B, W-1] int32. */
int dsk_accept_greedy(const void* logits, int dtype, int64_t ldl, int B, int W, int64_t V,
                      const int32_t* draft, int32_t* tt, int32_t* n_out, int32_t* token_out,
                      int32_t* seq_lens, void* workspace, size_t ws_bytes,
                      dsk_stream_t stream);
/* Workspace of dsk_accept_greedy (B, W, V) and of dsk_accept_sample (B, L + 1 = W, V). No state
 * is kept in it between calls; dsk_accept_ws_init only validates it. */
size_t dsk_accept_ws_bytes(int B, int W, int64_t V);
int dsk_accept_ws_init(void* workspace, size_t ws_bytes, dsk_stream_t stream);

/* dsk_accept_greedy without a workspace argument and without any allocation: the slice
 * partials live in a file-scope device array of 512 KiB (2 x 1024 rows x 64 slices x 4 B) that
 * each GPU the library runs on holds until the process ends. No counterpart in the reference
 * (MLX allocates inside its graph); it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops that forbid hipMalloc). Same arguments, results
 * and limits as dsk_accept_greedy, plus B * W <= 1024 (DSK_ERANGE beyond). Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (concurrent streams) race. */
int dsk_accept_greedy_static(const void* logits, int dtype, int64_t ldl, int B, int W, int64_t V,
                             const int32_t* draft, int32_t* tt, int32_t* n_out, int32_t* token_out,
                             int32_t* seq_lens, dsk_stream_t stream);

/* Speculative sampling: replaces _spec_sample_accept (src/mlx_dspark/generate.py:659-688)
 * with truncate_probs / sample_probs (src/mlx_dspark/sampling.py:18-49).
 * p_logits [B, L+1, V] f32 (target), q_logits [B, L, V] f32 (draft; NULL = one-hot q at
 * the drafted token, the lookup-draft case of generate.py:819-821), draft [B, L] int32,
 * V <= 2^19.
 * p = truncate(softmax(p_logits / T)); q = truncate(softmax(q_logits / T)) or, when
 * q_mul_inv_t != 0, softmax(q_logits * (1/T)) (src/mlx_dspark/model.py:297, :304).
 * Canonical arithmetic (shared bit for bit with the CPU oracle): e_j = exp(y_j - max y) by
 * the library's own exp, masses floor(e_j * 2^31) summed as integers, top-k keeps e_j >= the
 * k-th largest e, top-p keeps e_j >= the largest c whose mass at or above c reaches
 * ceil(top_p * Z), both keep e_j >= the larger threshold (the reference's top-k followed by
 * top-p on the zeroed values); a kept element's probability is e_j / (kept mass).
 * Position i accepts when u < min(1, p(d)/max(q(d), 1e-9)); the first rejected position n draws
 * from the residual max(p - q, 0), or, when every draft is accepted, position L draws from p;
 * draws are inverse CDFs over the fixed-point masses in index order.
 * Uniforms come from Philox4x32-10 keyed by (seed) at counter offset `offset`: the accept
 * test of (b, i) uses counter {i, b, 0, offset}, the draw at (b, i) {i, b, 1, offset}.
 * Outputs: n_out[b] accepted drafts, token_out[b] residual/bonus token, seq_lens[b] +=
 * n + 1 when non-NULL; accept_out [B, L] u8 and sample_out [B, L+1] int32 when non-NULL
 * (per-position accept flags and the token each position would emit; sample_out makes every
 * position draw, otherwise only position n does).
 * Every row is split over many workgroups; six kernels on `stream` (five without top-k /
 * top-p), no counters kept between calls: workspace of dsk_accept_ws_bytes(B, L + 1, V). */
int dsk_accept_sample(const float* p_logits, const float* q_logits, int64_t V, int B, int L,
                      const int32_t* draft, float temperature, float top_p, int top_k,
                      int q_mul_inv_t, uint64_t seed, uint32_t offset, int32_t* n_out,
                      int32_t* token_out, int32_t* seq_lens, uint8_t* accept_out,
                      int32_t* sample_out, void* workspace, size_t ws_bytes,
                      const uint32_t* offset_dev, dsk_stream_t stream);

/* offset_dev (dsk_accept_sample, dsk_sample_rows): when non-NULL, the Philox offset is read
 * from this device word instead of `offset`, so a captured graph can replay a sampled round
 * with a per-round offset the host writes before each replay. */

/* Row-wise sampling of truncate(softmax(logits / T)) (temperature > 0) or argmax
 * (temperature == 0, at most 1024 rows): replaces _sample_arr / _pick
 * (src/mlx_dspark/generate.py:135-146) and the DFlash draft sampling (generate.py:541-557).
 * logits f32 [R, V], V <= 2^19; the same canonical distribution as dsk_accept_sample; the draw
 * of row r uses Philox counter {row0 + r, 0, 2, offset}. probs_out [R, V] f32 (the truncated
 * distribution) may be NULL. workspace: dsk_sample_ws_bytes(R, V) bytes. */
size_t dsk_sample_ws_bytes(int R, int64_t V);
int dsk_sample_rows(const float* logits, int64_t V, int R, float temperature, float top_p,
                    int top_k, int mul_inv_t, uint64_t seed, uint32_t offset, int row0,
                    int32_t* token_out, float* probs_out, const uint32_t* offset_dev,
                    void* workspace, size_t ws_bytes, dsk_stream_t stream);

/* Greedy pick per row, each row split over 64 workgroups: token_out[r] = argmax_v logits[r][v]
 * (lowest index on ties, 0 for a row of -inf / NaN). Replaces mx.argmax(head, axis=-1), the
 * DFlash greedy draft (src/mlx_dspark/generate.py:557), and _pick at temperature 0
 * (generate.py:135-141). logits [R, ldl] f32 or bf16 (dtype), R <= 1024; workspace of
 * dsk_argmax_ws_bytes(R) (slice maxima; two kernels, no counters). */
size_t dsk_argmax_ws_bytes(int R);
int dsk_argmax_rows(const void* logits, int dtype, int64_t ldl, int64_t V, int R, int32_t* token_out,
                    void* workspace, size_t ws_bytes, dsk_stream_t stream);

/* Device-side length update: lens[b] += (n ? n[b] : 0) + add. Advances a drafter context
 * or KV length by the accepted count without a host round trip (the reference does this
 * on the host: n_cached += n + 1, src/mlx_dspark/generate.py:938; ctx append of the
 * accepted rows, :935-937). */
int dsk_lens_add(int32_t* lens, const int32_t* n, int B, int add, dsk_stream_t stream);

/* Read-only touch of bytes [p, p + bytes) by `workgroups` workgroups, for overlap experiments: a
 * side stream running it during the attention stage brings the next GEMMs' weights into the
 * memory-side cache. No counterpart in the reference (MLX schedules its own kernels); the engine
 * uses it only when asked (Qwen3W8.prefetch_weights). sink: 16 bytes the kernel may write. */
int dsk_prefetch(const void* p, size_t bytes, int workgroups, void* sink, dsk_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * DSpark drafter heads.
 * ------------------------------------------------------------------------------------- */

/* Block sampling with the rank-R Markov head: replaces DSparkDrafter.sample_block /
 * sample_block_probs (src/mlx_dspark/model.py:270-309) and the batched form
 * _batched_sample_block (src/mlx_dspark/batch_engine.py:414-428).
 *   prev = first_prev[b]; for i < cap:
 *     l_i[v] = bf16(bf16(base[b][i][v]) + bf16(sum_r deq(w2)[v][r] * bf16(deq(w1)[prev][r])))
 *     greedy (temperature == 0): tok[b][i] = argmax_v l_i (lowest index on ties)
 *     sampled: tok[b][i] ~ truncate(softmax(l_i * (1/T))) (dsk_sample_rows, Philox row
 *              (row0 + b)*cap + i: a batch of more than 16 rows called in pieces of 16 with row0
 *              = the piece's first row draws what one call over all rows would),
 *              q_logits_out[b][i] = l_i (the draft distribution's logits, for dsk_accept_sample
 *              with q_mul_inv_t = 1)
 *     prev = tok[b][i]
 * base f32 [B][cap][V] (row stride ldb), first_prev int32 [B] (device), w1: MLX-layout W8 table
 * [V, R] (q u8, scales/biases bf16 [V, R/64]), w2: dsk_w8_repack layout of [V, R]. R == 256,
 * B <= 16, V % 16 == 0. tok_out int32 [B][cap]. workspace: dsk_markov_ws_bytes(B, V, sampled). */
size_t dsk_markov_ws_bytes(int B, int64_t V, int sampled);
int dsk_markov_block(const float* base, int64_t ldb, int B, int cap, int64_t V, int R,
                     const int32_t* first_prev, const uint8_t* w1q, const uint16_t* w1s,
                     const uint16_t* w1b, const uint8_t* w2t, const uint32_t* w2sb,
                     float temperature, float top_p, int top_k, uint64_t seed, uint32_t offset,
                     int row0, int32_t* tok_out, float* q_logits_out, void* workspace, size_t ws_bytes,
                     dsk_stream_t stream);

/* Presence / frequency penalties on verify logits: logits[r][ids[j]] -= vals[j] for
 * j in [row_ptr[r], row_ptr[r+1]) (ids distinct within a row). The host builds the rows as
 * _Penalizer.block_penalty does (src/mlx_dspark/generate.py:202-228): base completion counts
 * plus each row's draft prefix. */
int dsk_logits_penalize(float* logits, int64_t ldl, int R, const int32_t* row_ptr,
                        const int32_t* ids, const float* vals, dsk_stream_t stream);

/* Per-token log-probabilities of committed tokens (OpenAI logprobs): for each row r of
 * logits [R][V] (row stride ldl, fp32), lse = max + log(sum exp(x - max)) (the raw target
 * distribution, independent of temperature and penalties), chosen[r] = x[tokens[r]] - lse,
 * and the top_k (0..64) largest entries as (top_ids, top_vals = x - lse) [R][top_k], ordered by
 * value descending then index ascending. Replaces _logprobs_for_block
 * (src/mlx_dspark/generate.py:149-176). */
int dsk_row_logprobs(const float* logits, int64_t ldl, int R, int64_t V, const int32_t* tokens,
                     int top_k, float* chosen, int32_t* top_ids, float* top_vals, dsk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSPARK_HIP_H */
