/*
 * kx355 — C ABI of the MI355X (gfx950) DiT-block kernels.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers. Activations are bf16 (raw 16-bit patterns; fp16 for the
 *     _f16 entry points at the end), tables and modulation vectors fp32, packed weights uint32.
 *     "ld*" arguments are row strides in elements. Sizes are int64_t.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the null stream).
 *   - The library never allocates or frees device memory; the caller owns every buffer.
 *   - Return value: 0 on success, a negative KX_ERR_* code otherwise; kx_last_error() gives the
 *     message of the calling thread's last failure.
 *   - Reference paths are relative to the dmlsrc/KinoMLX checkout.
 */
#ifndef KX355_H
#define KX355_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kx_stream_t; /* hipStream_t */

enum {
  KX_OK = 0,
  KX_ERR_INVALID = -1,     /* bad argument: null pointer, size, stride or alignment */
  KX_ERR_UNSUPPORTED = -2, /* valid request this build has no kernel for */
  KX_ERR_LAUNCH = -3       /* the HIP launch reported an error */
};

/* Element type of tensors that may be fp32, bf16 or fp16 (where an entry point says so). */
enum { KX_F32 = 0, KX_BF16 = 1, KX_F16 = 2 };

/* Norm kinds for kx_adaln_norm_bf16; KX_NORM_IN_F32 may be or-ed in for an fp32 input. */
enum { KX_NORM_RMS = 0, KX_NORM_LAYER = 1, KX_NORM_IN_F32 = 1 << 4 };

/* RoPE kinds for kx_rmsnorm_rope_bf16. */
enum { KX_ROPE_NONE = 0, KX_ROPE_SPLIT = 1, KX_ROPE_PAIR = 2 };

/* GEMM / quantized-GEMM epilogue flags: bias, activation (bits 4-7), gated residual. */
enum {
  KX_EPI_BIAS = 1,
  KX_EPI_ACT_GELU_TANH = 1 << 4,
  KX_EPI_ACT_SILU = 2 << 4,
  KX_EPI_ACT_SIGMOID2 = 3 << 4, /* 2 * sigmoid(.) — LTX gate logits */
  KX_EPI_ACT_SIGMOID = 4 << 4,  /* sigmoid(.) — Krea 2 output gate */
  KX_EPI_GATED_RESIDUAL = 1 << 8, /* c = resid + gate[col] * act(acc + bias) */
  KX_EPI_RESID_F32 = 1 << 9,      /* resid is fp32 (a residual stream carried in fp32) */
  KX_EPI_OUT_F32 = 1 << 10,       /* c is fp32 */
  KX_EPI_QK_NORM_ROPE = 1 << 11   /* per-head RMSNorm + pair RoPE on the Q and K columns
                                     (kx_gemm_qknorm_rope_bf16 only) */
};

int kx_abi_version(void);
const char* kx_last_error(void);

/*
 * Modulated norm: y = norm(x) * (1 + scale) + shift, fp32 opmath, one rounding.
 *   KX_NORM_RMS  : norm = x * rsqrt(mean(x^2) + eps)
 *     replaces transformer._adaln / _compiled_adaln
 *     (kinomlx/models/ltx2/transformer/transformer.py:16-23,42) over
 *     fused_ops.rms_norm(weight=None) (kinomlx/kernels/fused_ops.py:437-441).
 *   KX_NORM_LAYER: norm = (x - mean) * rsqrt(var + eps)
 *     replaces flux2 normalized (kinomlx/models/flux2/transformer.py:56-57).
 * shift/scale are fp32 rows of `dim`; row r of x uses modulation row (r / mod_div) at
 * mod_stride elements per row (mod_stride 0 broadcasts one row). shift == scale == NULL gives
 * the plain norm (fused_ops.rms_norm(weight=None)). With KX_NORM_IN_F32 in `kind`, x is fp32
 * (the block's residual stream); y is always bf16.
 */
int kx_adaln_norm_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                       int64_t dim, const float* shift, const float* scale, int64_t mod_div,
                       int64_t mod_stride, float eps, int kind, kx_stream_t stream);

/*
 * Weighted RMSNorm, optionally fused with RoPE on the normalized value:
 *   n = x * rsqrt(mean(x^2 over each norm group) + eps) * (w + weight_offset)
 *   then y = rope(n) (fp32 opmath, one rounding).
 * norm_width == dim: one norm over the row (LTX q_norm/k_norm, full width,
 *   kinomlx/models/ltx2/transformer/attention.py:121-133 -> fused_ops.rms_norm weighted,
 *   kinomlx/kernels/fused_ops.py:141-193,412-457).
 * norm_width == head_dim: per-head norm (FLUX QKNorm kinomlx/models/flux2/transformer.py:68-75,
 *   Krea2RMSNorm kinomlx/models/krea2/transformer/model.py:29-46 with weight_offset 1).
 * rope_kind KX_ROPE_SPLIT: split-half rotation (kinomlx/kernels/split_rope.py:35-56), tables
 *   cos/sin[t * table_ld + h * table_hs + i], i < head_dim / 2.
 * rope_kind KX_ROPE_PAIR: adjacent pairs (kinomlx/models/flux2/transformer.py:25-29), tables
 *   cos/sin[t * table_ld + h * table_hs + d], d < head_dim.
 * Token t of row r is r when table_batched, else r % tokens. w is fp32 or bf16 (w_dtype).
 */
int kx_rmsnorm_rope_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                         int64_t dim, int64_t norm_width, const void* w, int w_dtype, float eps,
                         float weight_offset, int rope_kind, const float* cos, const float* sin,
                         int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,
                         int64_t head_dim, kx_stream_t stream);

/*
 * kx_attention_gqa_fwd_bf16 with an additive score bias (the reference's masked SDPA,
 * kinomlx/models/ltx2/transformer/attention.py:136-185, masks from preprocessing.py:85-105):
 * score(b, h, i, j) = q_i . k_j * scale + bias[b * bias_bs + h * bias_hs + i * bias_qs + j],
 * bias bf16 with keys contiguous (strides in elements, 0 broadcasts; multiples of 4, 8-byte
 * aligned). A bias below -1e20 * scale (-inf, the bf16 minimum) removes the key (p = 0); a row
 * with every key removed averages V uniformly (the reference's equal finite scores).
 */
int kx_attention_bias_fwd_bf16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                               int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq,
                               int64_t tk, int64_t heads, int64_t kv_heads, int64_t head_dim,
                               float scale, const void* gate, int64_t ld_gate, const void* bias,
                               int64_t bias_bs, int64_t bias_hs, int64_t bias_qs, kx_stream_t stream);

/*
 * kx_attention_bias_fwd_bf16 (bias may be NULL) split over keys, for calls with few query tiles
 * and many keys (the 127-query audio -> video direction): the keys are cut into at most `splits`
 * slices of whole 64-key tiles, each slice's workgroups write unnormalized fp32 O rows and
 * (running max, row sum) into `workspace` (splits * batch * heads * tq * (head_dim + 2) floats,
 * caller-owned), and one pass merges the slices (rescaling each by 2^(m - max)), normalizes,
 * gates and rounds. Same result as the unsplit call up to the order of the fp32 sums.
 */
int kx_attention_split_fwd_bf16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                                int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk,
                                int64_t heads, int64_t kv_heads, int64_t head_dim, float scale,
                                const void* gate, int64_t ld_gate, const void* bias, int64_t bias_bs,
                                int64_t bias_hs, int64_t bias_qs, void* workspace, int64_t workspace_bytes,
                                int splits, kx_stream_t stream);

/*
 * Split-half RoPE, standalone: replaces split_rope.rotate (kinomlx/kernels/split_rope.py:144-163,
 * arithmetic :35-56). x/y are (batch, tokens, heads * 2 * half) rows at stride ldx/ldy; tables
 * token-major (table_batch, tokens, heads * half), table_batched selects per-batch tables.
 * Each product is rounded in fp32 before the difference/sum, then one cast: bit-equal to the
 * reference graph's fp32 arithmetic.
 */
int kx_rope_split_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t batch,
                       int64_t tokens, int64_t heads, int64_t half, const float* cos,
                       const float* sin, int table_batched, kx_stream_t stream);

/*
 * Adjacent-pair RoPE, standalone: replaces flux2.transformer.rotate
 * (kinomlx/models/flux2/transformer.py:25-29) and krea2 apply_rotary_embedding
 * (kinomlx/models/krea2/transformer/model.py:69-92). Rows r < rows of x/y hold heads * head_dim
 * values; tables cos/sin[tok * table_ld + h * table_hs + d] with tok = r (table_batched) or
 * r % tokens.
 */
int kx_rope_pair_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                      int64_t heads, int64_t head_dim, const float* cos, const float* sin,
                      int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,
                      kx_stream_t stream);

/*
 * Non-causal flash attention on token-major flattened heads: replaces
 * dense_attention.dense_attention (kinomlx/models/ltx2/kernels/dense_attention.py:106-153) and
 * the unmasked SDPA calls (kinomlx/models/ltx2/transformer/attention.py:144-161,
 * kinomlx/models/flux2/kv.py:48-54).
 *   o[b, i, h*D:(h+1)*D] = softmax_j(q_i . k_j * scale) v_j   (fp32 scores and accumulation)
 * q: (batch, tq) rows at ldq; k, v: (batch, tk) rows at ldk/ldv; o: (batch, tq) rows at ldo.
 * gate (optional, bf16 (batch * tq, heads) at ld_gate) multiplies each head's output row before
 * the one rounding (the LTX per-head gate, attention.py:360-366). head_dim is 64 or 128.
 */
int kx_attention_fwd_bf16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                          int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq,
                          int64_t tk, int64_t heads, int64_t head_dim, float scale,
                          const void* gate, int64_t ld_gate, kx_stream_t stream);

/*
 * Grouped-query form of kx_attention_fwd_bf16: k and v hold kv_heads heads ((batch * tk,
 * kv_heads * head_dim) rows at ldk/ldv) and query head h reads key/value head
 * h / (heads / kv_heads); heads % kv_heads == 0. Replaces the SDPA call of Krea2Attention
 * (kinomlx/models/krea2/transformer/model.py:134-185, num_kv_heads <= num_heads), whose K/V
 * are not repeated per query head here. kx_attention_fwd_bf16 is this call with
 * kv_heads == heads.
 */
int kx_attention_gqa_fwd_bf16(const void* q, int64_t ldq, const void* k, int64_t ldk,
                              const void* v, int64_t ldv, void* o, int64_t ldo, int64_t batch,
                              int64_t tq, int64_t tk, int64_t heads, int64_t kv_heads,
                              int64_t head_dim, float scale, const void* gate, int64_t ld_gate,
                              kx_stream_t stream);

/*
 * Self-attention q_norm / k_norm + split RoPE of the same tokens in one pass: Q rows at xq / ldq
 * and K rows at xk / ldk (column slices of one fused projection are fine), each normalized over
 * its full width dim with its own weight (wq, wk: w_dtype, plus weight_offset), then rotated by
 * the same split-half tables (cos / sin as kx_rmsnorm_rope_bf16 with KX_ROPE_SPLIT, 128-wide
 * heads), written to yq / yk. Each row's arithmetic is that of kx_rmsnorm_rope_bf16; the tables
 * are read once for both. Replaces the q_norm / k_norm + apply_rotary_emb pair of
 * Attention.__call__ (kinomlx/models/ltx2/transformer/attention.py:353-359, rope.py:18-61) when
 * q and k share the positional embedding. Returns KX_ERR_UNSUPPORTED (no work done) unless dim
 * is 1024, 2048 or 4096 with 16-byte aligned rows and tables.
 */
int kx_qk_rmsnorm_rope_bf16(const void* xq, int64_t ldq, const void* xk, int64_t ldk, void* yq,
                            int64_t ldyq, void* yk, int64_t ldyk, int64_t rows, int64_t dim,
                            const void* wq, const void* wk, int w_dtype, float eps,
                            float weight_offset, const float* cos, const float* sin,
                            int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,
                            kx_stream_t stream);

/*
 * Dense bf16 linear on MFMA: c = epilogue(a · wᵀ) with fp32 accumulation and one rounding.
 * Replaces mpp_linear.linear / mx.addmm(bias, x, Wᵀ) (kinomlx/kernels/mpp_linear.py:469-506,
 * kinomlx/models/ltx2/transformer/attention.py:41-109, kinomlx/modeling/layers.py).
 *   a: (m, k) at lda; w: (n, k) at ldw — the reference's (out, in) layout; c: (m, n) at ldc.
 *   bias: bf16 (n) with KX_EPI_BIAS. Activations per KX_EPI_ACT_*.
 *   KX_EPI_GATED_RESIDUAL: c = resid + gate * act(acc + bias), resid (m, n) at ldr, gate
 *   fp32 row (r / gate_div) at gate_stride (0 broadcasts). c may alias resid when both have
 *   the same element type. resid is bf16, or fp32 with KX_EPI_RESID_F32; c is bf16, or fp32
 *   with KX_EPI_OUT_F32 (fp32 operands need 16-byte aligned rows).
 * Requires k % 8 == 0, lda/ldw % 8 == 0 and 16-byte aligned a/w.
 */
int kx_gemm_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                 void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue,
                 const void* resid, int64_t ldr, const float* gate, int64_t gate_div,
                 int64_t gate_stride, kx_stream_t stream);

/*
 * kx_gemm_bf16 for products whose output tiles leave most CUs idle (a few hundred rows): K is
 * cut into `splits` slices, each multiplied by its own row of workgroups into an fp32 partial
 * product in `workspace` (splits * m * n floats, caller-owned), then one pass sums the slices and
 * applies the epilogue (bias, activation, gated residual, output type) as kx_gemm_bf16 does.
 * Same products as the reference call of kx_gemm_bf16 (mpp_linear.linear / mx.addmm,
 * kinomlx/kernels/mpp_linear.py:469-506); the sum order over K differs (fp32 throughout).
 * Requires n % 4 == 0, k % (64 * splits) == 0, 2 <= splits <= 64.
 */
int kx_gemm_splitk_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                        int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid,
                        int64_t ldr, const float* gate, int64_t gate_div, int64_t gate_stride, void* workspace,
                        int64_t workspace_bytes, int splits, kx_stream_t stream);

/* Size of the static device array kx_gemm_splitk_noalloc_bf16 keeps its partial products in. */
#define KX_SPLITK_SCRATCH_BYTES (16ll << 20)

/*
 * kx_gemm_splitk_bf16 without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It
 * has no counterpart in the reference. The fp32 partial products go to a static device array of
 * KX_SPLITK_SCRATCH_BYTES (16 MiB) that each device holds from the library's load until the
 * process ends; the call allocates nothing and returns KX_ERR_INVALID when splits * m * n * 4
 * exceeds it. Every call on a device shares that device's array: calls that overlap on one device
 * (two streams, or two threads) race, so the caller orders them. Same kernels, results and checks
 * as kx_gemm_splitk_bf16 (bit-identical output).
 */
int kx_gemm_splitk_noalloc_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                                void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue,
                                const void* resid, int64_t ldr, const float* gate, int64_t gate_div,
                                int64_t gate_stride, int splits, kx_stream_t stream);

/*
 * Projection with the attention's per-head Q/K RMSNorm and adjacent-pair RoPE in its epilogue:
 * c = x w^T + bias (bf16 out), where columns [0, q_end) are query heads and [q_end, k_end) key
 * heads of 128 (the rest, V and anything after, plain). For each row m and head: v = acc + bias
 * rounded to bf16 (the value the plain projection would store), n = v * rsqrt(mean(v^2) + eps) *
 * (w_norm[d] + weight_offset) in fp32, then
 * out[2i] = n[2i] c[2i] - n[2i+1] s[2i], out[2i+1] = n[2i+1] c[2i+1] + n[2i] s[2i+1] (each product
 * rounded in fp32 before the sum), one bf16 rounding. Tables: cos/sin + (m / table_rows) *
 * table_bs + (m % table_rows) * table_ld + head * table_hs + d. Replaces the projection, QKNorm
 * and rotate of FLUX.2 DoubleAttention / SingleAttention (kinomlx/models/flux2/transformer.py:68-75,
 * 25-29, 88-164) and of Krea2Attention (kinomlx/models/krea2/transformer/model.py:29-46, 69-92,
 * 134-185); the bf16 q/k round trip through HBM between the projection and the norm pass is
 * removed. norm weights fp32 or bf16 (norm_dtype KX_F32 / KX_BF16);
 * requires k % 64 == 0 and 16-byte aligned table rows.
 */
int kx_gemm_qknorm_rope_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                             int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t q_end, int64_t k_end,
                             const void* norm_q, const void* norm_k, int norm_dtype, float eps, float weight_offset,
                             const float* cos, const float* sin, int64_t table_ld, int64_t table_hs,
                             int64_t table_rows, int64_t table_bs, kx_stream_t stream);

/*
 * Group-wise affine int4/int8 weight-quantized linear, dequantized inside the MFMA mainloop:
 * replaces nn.QuantizedLinear / mx.quantized_matmul(x, wq, scales, biases, transpose=True,
 * group_size, bits, mode="affine") + bias (kinomlx/models/ltx2/weights/quantization.py:28-44,
 * kinomlx/_mlx_nn.py:20). wq: uint32 (n, k * bits / 32), element j of a word at bits
 * [bits*j, bits*(j+1)); scales/biases: bf16 (n, k / group_size). The dequantized weight is
 * bf16(fp32(scale) * q + fp32(bias)). Epilogue flags and residual/gate as kx_gemm_bf16.
 * Requires bits in {4, 8}, group_size == 64, k % 64 == 0.
 */
int kx_qgemm_affine_bf16(const void* a, int64_t lda, const uint32_t* wq, const void* scales,
                         const void* biases, const void* bias, void* c, int64_t ldc, int64_t m,
                         int64_t n, int64_t k, int group_size, int bits, int epilogue,
                         const void* resid, int64_t ldr, const float* gate, int64_t gate_div,
                         int64_t gate_stride, kx_stream_t stream);

/*
 * Test hook and load-time helper: dequantize packed affine weights to bf16 (n, k), with the
 * same arithmetic as kx_qgemm_affine_bf16's mainloop (the MLX dequantize semantics behind
 * mx.quantized_matmul, called from kinomlx/models/ltx2/weights/quantization.py:32-41).
 */
int kx_dequant_affine_bf16(const uint32_t* wq, const void* scales, const void* biases, void* out,
                           int64_t n, int64_t k, int group_size, int bits, kx_stream_t stream);

/*
 * Quantize-on-load: bf16 weight w (n, k) at row stride ldw -> the packed affine format above
 * (wq (n, k * bits / 32) uint32, scales / biases (n, k / 64) bf16). Per group of 64 along K:
 * scale = bf16((max - min) / (2^bits - 1)) (1 when not positive), bias = bf16(min),
 * code = clamp(rint((w - bias) / scale), 0, 2^bits - 1) in fp32. Replaces the mx.quantize call
 * of the weight preparation (kinomlx/models/ltx2/preparation.py:139-157, affine mode, defaults
 * kinomlx/models/ltx2/weights/tensors.py:185-203); the scale/bias choice is this build's own
 * (MLX's quantizer is not part of the reference tree). Requires k % 64 == 0, ldw % 8 == 0 and a
 * 16-byte aligned w; group_size 64, bits 4 or 8.
 */
int kx_quantize_affine_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, void* biases,
                            int64_t n, int64_t k, int group_size, int bits, kx_stream_t stream);

/*
 * Load-time layout for kx_qgemm_affine_tiled_bf16 (no counterpart in the reference: its
 * quantized weights stay in the packed layout above; this is the same data regrouped so that
 * each 256-row weight tile and 32-wide K stage is one contiguous block). With npad = n rounded
 * up to 256 (rows past n repeat row n - 1):
 *   wt : npad * k * bits / 8 bytes; block (nb, kb) at ((nb * k/32 + kb) * 256 + r) * (4 * bits)
 *        holds row nb*256 + r's packed bytes of k = 32 kb .. 32 kb + 31;
 *   sbt: npad * (k / 128) * 8 bytes; block (nb, p) at ((nb * k/128 + p) * 256 + r) * 8 holds
 *        bf16 scale[2p], scale[2p+1], bias[2p], bias[2p+1] of row nb*256 + r.
 * Requires k % 128 == 0, group_size 64, bits 4 or 8.
 */
int kx_qweight_tile_affine(const uint32_t* wq, const void* scales, const void* biases, void* wt,
                           void* sbt, int64_t n, int64_t k, int group_size, int bits,
                           kx_stream_t stream);

/*
 * kx_qgemm_affine_bf16 on the tiled layout of kx_qweight_tile_affine: the same result
 * (bit-exact dequantization, fp32 accumulation, one rounding), with each stage's packed weights
 * and scale / bias pairs read as contiguous blocks. Replaces the same reference call
 * (kinomlx/models/ltx2/weights/quantization.py:28-44); QuantizedLinear prepares the layout once.
 * Requires k % 128 == 0 and lda <= 2^22.
 */
int kx_qgemm_affine_tiled_bf16(const void* a, int64_t lda, const void* wt, const void* sbt,
                               const void* bias, void* c, int64_t ldc, int64_t m, int64_t n,
                               int64_t k, int bits, int epilogue, const void* resid, int64_t ldr,
                               const float* gate, int64_t gate_div, int64_t gate_stride,
                               kx_stream_t stream);

/*
 * mxfp8 weight-quantized linear (OCP MX: FP8 E4M3 elements, one E8M0 scale byte per group of 32
 * along K), dequantized inside the MFMA mainloop: replaces nn.QuantizedLinear /
 * mx.quantized_matmul(x, wq, scales, transpose=True, group_size=32, bits=8, mode="mxfp8") + bias,
 * the mode transformer_quantize="mxfp8-blocks" installs on every block linear
 * (kinomlx/models/ltx2/weights/quantization.py:199-216, tensors.py:185-203). wq: uint32
 * (n, k / 4), element j of a word in byte j; scales: uint8 (n, k / 32). The weight operand is
 * bf16(e4m3(q) * 2^(s - 127)), exact. Epilogue flags and residual/gate as kx_gemm_bf16.
 * Requires group_size == 32 and k % 32 == 0.
 */
int kx_qgemm_mxfp8_bf16(const void* a, int64_t lda, const uint32_t* wq, const void* scales,
                        const void* bias, void* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                        int group_size, int epilogue, const void* resid, int64_t ldr, const float* gate,
                        int64_t gate_div, int64_t gate_stride, kx_stream_t stream);

/*
 * mxfp8 weights -> the bf16 (n, k) weight (out features n, in features k), exactly. transposed = 0:
 * the layout above (wq (n, k / 4), scales (n, k / 32)). transposed = 1: the pretransposed layout
 * of transformer_quantize="mxfp8-blocks-pretranspose", quantized from weight.T (wq (k, n / 4),
 * scales (k, n / 32), groups along n), which _PretransposedQuantizedLinear multiplies with
 * mx.quantized_matmul(..., transpose=False) (kinomlx/models/ltx2/weights/quantization.py:17-44,
 * kinomlx/models/ltx2/preparation.py:139-157); transposed needs n % 32 == 0 and k % 8 == 0.
 */
int kx_dequant_mxfp8_bf16(const uint32_t* wq, const void* scales, void* out, int64_t n, int64_t k,
                          int group_size, int transposed, kx_stream_t stream);

/*
 * Quantize-on-load to mxfp8: bf16 w (n, k) at row stride ldw -> wq (n, k / 4) uint32 and scales
 * (n, k / 32) uint8. Per group of 32: X = floor(log2(max |w|)) - 8 clamped to [-127, 127] (-127 for
 * a zero group), scale byte X + 127, codes E4M3(w * 2^-X) rounded to nearest even, saturated at
 * +-448 (the OCP MX conversion). Replaces mx.quantize(weight, 32, 8, mode="mxfp8") of the weight
 * preparation (kinomlx/models/ltx2/preparation.py:139-157); MLX's own exponent choice is not part of
 * the reference tree. Requires group_size 32, k % 32 == 0, ldw % 8 == 0, 16-byte aligned w.
 */
int kx_quantize_mxfp8_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, int64_t n, int64_t k,
                           int group_size, kx_stream_t stream);

/* FP4 weight formats: E2M1 elements, eight per little-endian uint32 (element j at bits [4j, 4j+4)),
 * with one scale byte per group along K: KX_FP4_MX = mxfp4 (OCP MX, E8M0 scale 2^(S - 127), group
 * 32), KX_FP4_NV = nvfp4 (E4M3 scale, group 16). The reference routes feed-forward layers to them
 * through video_ff_quantize_specs (kinomlx/models/ltx2/settings.py:39,107,281; defaults
 * kinomlx/models/ltx2/weights/tensors.py:190-195; packed by mx.quantize(w, group_size, 4, mode),
 * kinomlx/models/ltx2/preparation.py:152). */
enum { KX_FP4_MX = 0, KX_FP4_NV = 1 };

/* (n, k) bf16 <- FP4 words (n, k / 8) and scale bytes (n, k / group_size), exactly:
 * w = e2m1(q) * scale (the product has at most 6 significant bits). The dequantize -> dense GEMM
 * route of the fp4 QuantizedLinear. */
int kx_dequant_fp4_bf16(const uint32_t* wq, const void* scales, void* out, int64_t n, int64_t k, int group_size,
                        int scale_kind, kx_stream_t stream);

/* FP4 quantize-on-load of a bf16 (n, k) weight with 16-byte aligned rows at ldw: per group,
 * mxfp4: X = floor(log2(max |w|)) - 2 clamped to [-127, 127] (-127 for zeros), scale byte X + 127,
 * codes E2M1(w * 2^-X); nvfp4: s = E4M3(max |w| / 6), codes E2M1(fp32(w / s)) (zeros when s is 0);
 * E2M1 rounds to nearest even and saturates at +-6. This build's quantizer: MLX's own scale choice
 * is not reproduced. */
int kx_quantize_fp4_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, int64_t n, int64_t k,
                         int group_size, int scale_kind, kx_stream_t stream);

/* Modulation values: out[b, t, r, c] = fp32(table[r, c]) + fp32(ts[b, t, r, c]) for a (rows, dim)
 * table (KX_F32, KX_BF16 or KX_F16) and an optional timestep modulation ts (null: the table alone) with
 * element strides ts_bs / ts_ts / ts_rs (dim contiguous; 0 broadcasts); with round_dtype KX_BF16 or
 * KX_F16 each sum is rounded to that type (KX_F32: kept); out is fp32 (batch, tokens, rows, dim)
 * contiguous. BasicAVTransformerBlock._ada_values and the prompt / A/V tables
 * (kinomlx/models/ltx2/transformer/transformer.py:179-199,209-219): scale_shift_table + timestep;
 * LTXAVModel._output (kinomlx/models/ltx2/transformer/model.py:577-593): the output head's
 * (shift, scale), rounded to the hidden state's type. */
int kx_table_add_f32(const void* table, int table_dtype, const void* ts, int ts_dtype, int64_t ts_bs,
                     int64_t ts_ts, int64_t ts_rs, float* out, int64_t batch, int64_t tokens, int64_t rows,
                     int64_t dim, int round_dtype, kx_stream_t stream);

/* tanh GELU in fp32, inner argument clamped to +-10: fused_ops.gelu_approx
 * (kinomlx/kernels/fused_ops.py:27-35,327-350). */
int kx_gelu_tanh_bf16(const void* x, void* y, int64_t count, kx_stream_t stream);

/* x / (1 + exp(-x)) in fp32: fused_ops.silu (kinomlx/kernels/fused_ops.py:40-45,353-372). */
int kx_silu_bf16(const void* x, void* y, int64_t count, kx_stream_t stream);

/* SwiGLU: y[r, j] = silu(x[r, j]) * x[r, hidden + j], x (rows, 2 * hidden) at ldx:
 * flux2 swiglu (kinomlx/models/flux2/transformer.py:63-65). */
int kx_swiglu_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                   int64_t hidden, kx_stream_t stream);

/* y = x * (1 + scale) + shift (modulation vectors fp32, rows as kx_adaln_norm_bf16):
 * transformer._modulate (kinomlx/models/ltx2/transformer/transformer.py:33-34). */
int kx_modulate_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                     const float* shift, const float* scale, int64_t mod_div,
                     int64_t mod_stride, kx_stream_t stream);

/* y = x + r * gate (gate fp32 rows as kx_adaln_norm_bf16): transformer._gated_residual
 * (transformer.py:26-30); with x == NULL, y = r * gate (transformer._gate, :37-38). */
int kx_gated_residual_bf16(const void* x, int64_t ldx, const void* r, int64_t ldr, void* y,
                           int64_t ldy, int64_t rows, int64_t dim, const float* gate,
                           int64_t gate_div, int64_t gate_stride, kx_stream_t stream);

/* LTX split-RoPE tables: cos, sin (batch, tokens, half) fp32, token-major (the head-major
 * (B, H, T, half/H) views precompute_freqs_cis returns share this storage). positions fp32
 * (batch, axes, tokens, pos_stride) contiguous; with middle the position is the mean of elements
 * 0 and 1, else element 0. With pad = half - axes * n, columns j < pad hold (1, 0) and column
 * pad + f * axes + a the angle ((p / max_pos[a]) * 2 - 1) * grid[f], grid (n,) fp32 from
 * _frequency_grid. precompute_freqs_cis (kinomlx/models/ltx2/transformer/rope.py:95-176). */
int kx_ltx_rope_tables(const float* positions, int64_t pos_stride, int middle, const float* max_pos,
                       const float* grid, float* cos, float* sin, int64_t batch, int64_t axes,
                       int64_t tokens, int64_t n, int64_t half, kx_stream_t stream);

/* ---- the steps either side of the blocks (element-wise, contiguous tensors) ------------------ */

/* Sinusoidal timestep features, out (n, dim) in out_dtype (KX_F32 or KX_BF16): with half = dim/2,
 * s_i = t[i] * time_scale and f_j = exp((neg_log_period * j) / half) in fp32, out[i, j] =
 * cos(s_i f_j) for j < half, sin(s_i f_(j-half)) for j < 2 half, 0 in a last odd column;
 * neg_log_period = -ln(max_period). get_timestep_embedding
 * (kinomlx/models/ltx2/transformer/timestep.py:13-28) of the preprocessor's scaled timesteps
 * (preprocessing.py:66-75, time_scale 1 for the plain function); the bf16 output is its
 * `.astype(hidden_dtype)` in TimestepEmbedding (timestep.py:40-41). */
int kx_timestep_embedding(const float* t, void* out, int64_t n, int64_t dim, int out_dtype,
                          float time_scale, float neg_log_period, kx_stream_t stream);

/* out = sample + dtype(delta * velocity), fp32 multiply, sample and velocity of one dtype:
 * euler_velocity_step (kinomlx/samplers/steps.py:8-32), delta = sigma_next - sigma. */
int kx_euler_velocity_step(const void* sample, const void* velocity, void* out, int64_t n,
                           int dtype, float delta, kx_stream_t stream);

/* out = denoised + ratio * (sample - denoised) in fp32, rounded once to sample_dtype:
 * euler_step (kinomlx/samplers/steps.py:35-72), ratio = sigma_next / sigma. */
int kx_euler_step(const void* sample, int sample_dtype, const void* denoised, int denoised_dtype,
                  void* out, int64_t n, float ratio, kx_stream_t stream);

/* X0 conversion: out[r, c] = latent[r, c] - timesteps[r / ts_div] * velocity[r, c] in fp32,
 * rounded once to latent_dtype; (rows, dim) = (B*T, C), ts_div = T for per-batch timesteps, 1 for
 * per-token ones. _to_denoised (kinomlx/models/ltx2/transformer/wrappers.py:48-66). */
int kx_to_denoised(const void* latent, int latent_dtype, const void* velocity, int velocity_dtype,
                   const float* timesteps, void* out, int64_t rows, int64_t dim, int64_t ts_div,
                   kx_stream_t stream);

/* Conditioning composite: out[r, c] = denoised[r, c] * mask[r] + clean[r, c] * (1 - mask[r]) in
 * fp32, rounded once to denoised_dtype: post_process_latent (kinomlx/models/ltx2/state.py:70-83). */
int kx_mask_composite(const void* denoised, int denoised_dtype, const void* clean, int clean_dtype,
                      const float* mask, void* out, int64_t rows, int64_t dim, kx_stream_t stream);

/* *flag = 1 if every one of the n elements of x is finite, else 0 (flag: one device int, written
 * on the stream; x may be NULL when n == 0): the per-step check mx.all(mx.isfinite(latent))
 * (kinomlx/models/ltx2/denoise.py:244-258). */
int kx_all_finite(const void* x, int64_t n, int dtype, int* flag, kx_stream_t stream);

/*
 * ---- fp16 activations ----------------------------------------------------------------------
 * The reference runs the LTX-2 transformer in FP16 by default (docs/PERFORMANCE.md:228-230,
 * --transformer-dtype, kinomlx/models/ltx2/settings.py:233), and every hot-path operator takes
 * float16 as well as bfloat16: dense_attention (kinomlx/models/ltx2/kernels/dense_attention.py:
 * 47,112-116), split_rope.rotate (kinomlx/kernels/split_rope.py:32), the {half, bfloat} MPP GEMMs
 * (kinomlx/kernels/mpp_linear.py:145-294), fused_ops.rms_norm / gelu_approx / silu
 * (kinomlx/kernels/fused_ops.py:327-457). Each entry point below is its _bf16 namesake's contract
 * with fp16 in place of bf16 for every 16-bit tensor (inputs, outputs, bias, gate, score bias,
 * 16-bit residual): the same kernels, with v_mfma_f32_*_f16 products and fp16 roundings (round
 * to nearest even; a value beyond 65504 becomes infinity, as an fp16 cast does). fp32 tables,
 * modulation vectors, residual streams and workspaces are unchanged; norm weights may be
 * KX_F32, KX_BF16 or KX_F16.
 */
int kx_adaln_norm_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                      const float* shift, const float* scale, int64_t mod_div, int64_t mod_stride, float eps,
                      int kind, kx_stream_t stream);
int kx_rmsnorm_rope_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                        int64_t norm_width, const void* w, int w_dtype, float eps, float weight_offset,
                        int rope_kind, const float* cos, const float* sin, int64_t table_ld, int64_t table_hs,
                        int64_t tokens, int table_batched, int64_t head_dim, kx_stream_t stream);
int kx_qk_rmsnorm_rope_f16(const void* xq, int64_t ldq, const void* xk, int64_t ldk, void* yq, int64_t ldyq,
                           void* yk, int64_t ldyk, int64_t rows, int64_t dim, const void* wq, const void* wk,
                           int w_dtype, float eps, float weight_offset, const float* cos, const float* sin,
                           int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,
                           kx_stream_t stream);
int kx_rope_split_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t batch, int64_t tokens,
                      int64_t heads, int64_t half, const float* cos, const float* sin, int table_batched,
                      kx_stream_t stream);
int kx_rope_pair_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t heads,
                     int64_t head_dim, const float* cos, const float* sin, int64_t table_ld, int64_t table_hs,
                     int64_t tokens, int table_batched, kx_stream_t stream);
int kx_attention_fwd_f16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                         void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk, int64_t heads,
                         int64_t head_dim, float scale, const void* gate, int64_t ld_gate, kx_stream_t stream);
int kx_attention_gqa_fwd_f16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                             void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk, int64_t heads,
                             int64_t kv_heads, int64_t head_dim, float scale, const void* gate, int64_t ld_gate,
                             kx_stream_t stream);
int kx_attention_bias_fwd_f16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                              int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk,
                              int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, const void* gate,
                              int64_t ld_gate, const void* bias, int64_t bias_bs, int64_t bias_hs,
                              int64_t bias_qs, kx_stream_t stream);
int kx_attention_split_fwd_f16(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                               int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk,
                               int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, const void* gate,
                               int64_t ld_gate, const void* bias, int64_t bias_bs, int64_t bias_hs,
                               int64_t bias_qs, void* workspace, int64_t workspace_bytes, int splits,
                               kx_stream_t stream);
int kx_gemm_f16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc,
                int64_t m, int64_t n, int64_t k, int epilogue, const void* resid, int64_t ldr, const float* gate,
                int64_t gate_div, int64_t gate_stride, kx_stream_t stream);
int kx_gemm_splitk_f16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                       int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid, int64_t ldr,
                       const float* gate, int64_t gate_div, int64_t gate_stride, void* workspace,
                       int64_t workspace_bytes, int splits, kx_stream_t stream);
int kx_gelu_tanh_f16(const void* x, void* y, int64_t count, kx_stream_t stream);
int kx_silu_f16(const void* x, void* y, int64_t count, kx_stream_t stream);
int kx_swiglu_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t hidden,
                  kx_stream_t stream);
int kx_modulate_f16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                    const float* shift, const float* scale, int64_t mod_div, int64_t mod_stride, kx_stream_t stream);
int kx_gated_residual_f16(const void* x, int64_t ldx, const void* r, int64_t ldr, void* y, int64_t ldy,
                          int64_t rows, int64_t dim, const float* gate, int64_t gate_div, int64_t gate_stride,
                          kx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KX355_H */
