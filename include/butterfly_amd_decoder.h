/*
 * butterfly_amd decoder steps -- C ABI of the row-wise and elementwise steps of
 * the swapped decoder (bf16 in and out, fp32 inside), one launch each.
 *
 * Conventions are those of butterfly_amd.h (device pointers, 16-byte aligned
 * contiguous tensors, work enqueued on `stream`, 0 or a negative BFLY_ERR_*).
 * The rounding points are those of the PyTorch forms in butterfly_amd/decoder.py:
 * bf16 after a residual add, after each norm, after RoPE, after SiLU and after
 * the product.
 */
#ifndef BUTTERFLY_AMD_DECODER_H_
#define BUTTERFLY_AMD_DECODER_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Device: h = x + residual (bf16), norm_out = RMSNorm(h) * weight over `dim`
 * (eps inside the square root), for `rows` rows.  With residual == NULL (and
 * h_out == NULL) it is the plain RMSNorm of x.  dim a multiple of 256, at most
 * 8192.  The decoder layers' input / post-attention norms and the final norm;
 * no counterpart in the reference's own code (the decoders it swaps into keep
 * their norms).
 */
int bfly_add_rms_norm(const void* x, const void* residual, const void* weight, int64_t rows, int dim,
                      float eps, void* h_out, void* norm_out, hipStream_t stream);

/*
 * Device: the projection tail of the swapped attention -- per-head RMSNorm of q
 * [B*T rows of Hq*d] and k [B*T rows of Hkv*d] (rows *_row_stride elements apart,
 * so q, k and v may be column ranges of one fused projection output) with
 * q_weight / k_weight [d], rotate-half RoPE
 * with cos/sin [T, d] (fp32, row t = this call's t-th position), and the move to
 * heads-first q_out [B, Hq, T, d], k_out and v_out [B, Hkv, T, d] (v unchanged).
 * head_dim 128 or 256.  Replaces q_norm / k_norm / transpose / RoPE of
 * bna/integrations/qwen_torch.py:550-562 (qwen_mlx.py:288-357).
 */
int bfly_qk_norm_rope(const void* q, const void* k, const void* v, int64_t q_row_stride, int64_t k_row_stride,
                      int64_t v_row_stride, const void* q_weight, const void* k_weight,
                      const float* cos, const float* sin, int64_t batch, int64_t seq_len, int hq, int hkv,
                      int head_dim, float eps, void* q_out, void* k_out, void* v_out, hipStream_t stream);

/*
 * Device: out [rows, cols] = SiLU(gate) * up, the SwiGLU MLP's product; gate and
 * up rows are in_row_stride elements apart (2 * cols for a fused gate|up
 * projection output).  No counterpart in the reference's own code.
 */
int bfly_silu_mul(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t in_row_stride, void* out,
                  hipStream_t stream);

/*
 * Device: out[r] (int64) = index of the greedy pick of row r of x (bf16, `rows`
 * rows of n elements, element (r, i) at x[r * row_stride + i * col_stride]),
 * in torch.argmax's order: NaN first, then the largest value, then the lowest
 * index among equals.  rows at most 65535.  `workspace` (device, 8-byte
 * aligned, `workspace_bytes` long; rows * 3 KiB + 8 bytes is enough) holds per-workgroup
 * candidates so that a row is scanned by up to 256 workgroups; a smaller or
 * NULL workspace gives fewer workgroups per row (one at the least), never a
 * different result.  The decoder's greedy step inside a captured decode graph
 * (torch's argmax reduction records a memset node there); no counterpart in the
 * reference's own code.
 */
int bfly_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t row_stride, int64_t col_stride,
                     void* workspace, int64_t workspace_bytes, void* out, hipStream_t stream);

/*
 * Device: bfly_argmax_rows that allocates nothing and takes no workspace: the
 * per-workgroup candidates live in a static device array of the library
 * (64 * 3 KiB + 8 bytes per GPU, held until the process ends), so rows is at
 * most 64 (larger counts return BFLY_ERR_INVALID).  Same result as
 * bfly_argmax_rows.  Calls on one GPU share that array: calls that overlap on
 * one GPU (other streams or threads) race.  The first call on a device looks
 * up that device's copy of the array (make it outside graph capture).  No
 * counterpart in the reference: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation).
 */
int bfly_argmax_rows_noalloc(const void* x, int64_t rows, int64_t n, int64_t row_stride, int64_t col_stride,
                             void* out, hipStream_t stream);

/*
 * Device: out[n] (bf16) = sum_i x_i * (code_ni * scale_ng + bias_ng) for one row x
 * (in_features bf16, 16-byte aligned): a quantized linear layer's product at
 * batch 1, read from the 4-bit codes.  packed: [out_features][in_features / 2]
 * bytes, two codes per byte, low nibble first (16-byte aligned).  scale_bias:
 * [out_features][in_features / group] pairs of bf16 (scale, bias), 4-byte
 * aligned.  group a multiple of 32; in_features a multiple of group and at most
 * 8192.  fp32 accumulation.  Replaces the 4-bit affine quantized matmul of the
 * reference's quantized projections (mlx.nn.QuantizedLinear as used at
 * bna/integrations/qwen_mlx.py:1115-1157).
 */
int bfly_q4_gemv(const void* x, const void* packed, const void* scale_bias, int64_t out_features,
                 int64_t in_features, int group, void* out, hipStream_t stream);

/*
 * Device: the SwiGLU MLP's first half at batch 1 in one launch: out[n] (bf16) =
 * SiLU(g_n) * u_n with g_n the bfly_q4_gemv product of weight row n and u_n that
 * of row n + up_row_offset (a fused gate|up weight: up_row_offset =
 * out_features), each rounded to bf16 first, as bfly_silu_mul over the two
 * projections' outputs computes it.  Same weight layout and limits as
 * bfly_q4_gemv.  No counterpart in the reference's own code.
 */
int bfly_q4_gemv_silu(const void* x, const void* packed, const void* scale_bias, int64_t out_features,
                      int64_t in_features, int group, int64_t up_row_offset, void* out, hipStream_t stream);

/*
 * Device: bfly_add_rms_norm of one row followed by bfly_q4_gemv of the normed row, in
 * one launch: h_out = x + residual (bf16; skipped when residual and h_out are NULL),
 * out = W RMSNorm(h) * norm_weight, with the rounding points and summation order of
 * the two separate calls (bit-identical outputs).  in_features (the row's length)
 * 2048, 4096 or 6144; x, residual, norm_weight and h_out 16-byte aligned;
 * weight layout and other limits as bfly_q4_gemv.  The decoder's input and final
 * norms with the product that consumes them; no counterpart in the reference's
 * own code.
 */
int bfly_add_rms_norm_q4_gemv(const void* x, const void* residual, const void* norm_weight, float eps,
                              void* h_out, const void* packed, const void* scale_bias, int64_t out_features,
                              int64_t in_features, int group, void* out, hipStream_t stream);

/*
 * Device: bfly_add_rms_norm of one row followed by bfly_q4_gemv_silu of the normed
 * row, in one launch (the post-attention norm with the MLP's gate|up product);
 * bit-identical to the two calls.  Limits as bfly_add_rms_norm_q4_gemv and
 * bfly_q4_gemv_silu.  No counterpart in the reference's own code.
 */
int bfly_add_rms_norm_q4_gemv_silu(const void* x, const void* residual, const void* norm_weight, float eps,
                                   void* h_out, const void* packed, const void* scale_bias,
                                   int64_t out_features, int64_t in_features, int group,
                                   int64_t up_row_offset, void* out, hipStream_t stream);

/*
 * Device: bfly_add_rms_norm_q4_gemv that also leaves one greedy candidate per workgroup (the
 * largest bf16 output its waves wrote, torch.argmax's order: NaN first, then larger, then the
 * lower index, as one 64-bit key) in `workspace` (bfly_q4_argmax_workspace_bytes bytes,
 * 16-byte aligned: an int64 count, then up to 1024 keys from byte 16; the launch writes the
 * count too, so nothing needs clearing), for bfly_greedy_advance.  out_features < 2^31.  The decoder's final norm with the lm_head at batch 1; no counterpart
 * in the reference's own code (its greedy loop takes mx.argmax of the logits).
 */
int64_t bfly_q4_argmax_workspace_bytes(int64_t out_features, int64_t in_features);
int bfly_add_rms_norm_q4_gemv_argmax(const void* x, const void* residual, const void* norm_weight, float eps,
                                     void* h_out, const void* packed, const void* scale_bias, int64_t out_features,
                                     int64_t in_features, int group, void* out, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream);

/*
 * Device: the greedy pick over the candidates bfly_add_rms_norm_q4_gemv_argmax left in
 * `workspace` (the argmax of its whole output), and a decode loop's bookkeeping in the same
 * launch: token[0] = the pick, tokens_out[counters[1]] = the pick while counters[1] <
 * tokens_cap, counters[0] and counters[1] (position, output column) + 1, and the next step's
 * input row x_next[0 .. hidden) = embed[pick] (bf16 [vocab][hidden], the tied embedding table;
 * hidden a multiple of 8; embed, x_next 16-byte aligned).  One workgroup; capturable.  Replaces
 * the reference's greedy step around the model call (argmax, token append, embedding lookup of
 * the next input); no counterpart in its own code.
 */
int bfly_greedy_advance(const void* workspace, int64_t workspace_bytes, const void* embed, int64_t vocab,
                        int64_t hidden, void* x_next, int64_t* token, int64_t* tokens_out, int64_t tokens_cap,
                        int64_t* counters, hipStream_t stream);

/*
 * Device: bfly_add_rms_norm_q4_gemv_silu whose input row x is given as n_parts = 4
 * fp32 partial rows x_parts[g * in_features + i] and formed as
 * x_i = bf16((p0_i + p1_i) + (p2_i + p3_i)): the o_parts of
 * bfly_decode_step_qk_norm_oproj (include/butterfly_amd.h), for which x is then
 * bfly_q4_gemv's output projection of the attention row bit for bit.  x_parts
 * 16-byte aligned; other limits as bfly_add_rms_norm_q4_gemv_silu.  No counterpart
 * in the reference's own code.
 */
int bfly_add_rms_norm_q4_gemv_silu_parts(const float* x_parts, int n_parts, const void* residual,
                                         const void* norm_weight, float eps, void* h_out, const void* packed,
                                         const void* scale_bias, int64_t out_features, int64_t in_features,
                                         int group, int64_t up_row_offset, void* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BUTTERFLY_AMD_DECODER_H_ */
