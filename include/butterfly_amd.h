/*
 * butterfly_amd -- C ABI of the MI355X (gfx950) Butterfly compressed-attention library.
 *
 * Conventions
 *   - Every tensor argument is a caller-owned DEVICE pointer, row-major and
 *     contiguous in the stated shape ([B, H, T, d] means d fastest), with a
 *     16-byte aligned base address (the kernels use 16-byte vector accesses).
 *   - `dtype` is BFLY_DTYPE_F32 or BFLY_DTYPE_BF16 and applies to every
 *     floating-point tensor of the call.
 *   - Work is enqueued on `stream`; nothing synchronises and nothing allocates.
 *   - Return 0 on success, a negative BFLY_ERR_* code otherwise; the message of
 *     the last failure on the calling thread is returned by bfly_last_error().
 *   - Partner rules: BFLY_RULE_* (the reference's ButterflyPartnerRule strings).
 *
 * Reference citations are `path:line` in Hmbown/Butterfly.
 */
#ifndef BUTTERFLY_AMD_H_
#define BUTTERFLY_AMD_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BFLY_ABI_VERSION 2

#define BFLY_OK 0
#define BFLY_ERR_INVALID (-1)     /* bad shape / argument: ValueError in the reference */
#define BFLY_ERR_UNSUPPORTED (-2) /* valid but not implemented on this path */
#define BFLY_ERR_HIP (-3)         /* HIP runtime failure */
#define BFLY_ERR_CAPACITY (-4)    /* cache capacity exhausted: RuntimeError in the reference */

#define BFLY_DTYPE_F32 0
#define BFLY_DTYPE_BF16 1

#define BFLY_RULE_XOR 0
#define BFLY_RULE_BIT_REVERSAL 1
#define BFLY_RULE_BENES 2
#define BFLY_RULE_CAUSAL_SHIFT 3
#define BFLY_RULE_FIXED_STRIDE 4
#define BFLY_RULE_RANDOM 5

#define BFLY_MAX_PARTNERS 16

/*
 * The staged topology of one layer at one block count: what a neighbour row
 * is computed from (filled by bfly_topology_init).
 */
typedef struct bfly_topology {
  int32_t rule;                 /* BFLY_RULE_* */
  int32_t width;                /* ceil(log2 N), 1 if N <= 1 */
  int32_t stage_idx;
  int32_t stage_count;
  int32_t local_window_blocks;
  int32_t sink_count;
  int32_t partner_count;        /* <= BFLY_MAX_PARTNERS */
  int32_t partner_bits[BFLY_MAX_PARTNERS];
} bfly_topology_t;

/* Message of the last failed call on this thread ("" if none). */
const char* bfly_last_error(void);

/* BFLY_ABI_VERSION of the loaded library. */
int bfly_abi_version(void);

/*
 * Host scalar topology metadata.
 * Replaces butterfly_width / butterfly_stage_meta (bna/topology/butterfly.py:39-65).
 * width = ceil(log2 N) (1 if N <= 1); stage_count = width, or max(1, 2*width-2)
 * for benes; stage_idx = layer_idx mod stage_count.
 */
int bfly_stage_meta(int64_t num_blocks, int64_t layer_idx, int partner_rule,
                    int32_t* stage_idx, int32_t* stage_count, int32_t* width);

/*
 * Host: partner bits of one stage, written to bits[0..partner_count).
 * Replaces butterfly_partner_bits (bna/topology/butterfly.py:77-105).
 */
int bfly_partner_bits(int stage_idx, int stage_count, int width, int partner_count,
                      int partner_rule, int32_t* bits);

/*
 * Host: the topology of layer `layer_idx` at `num_blocks` blocks.
 * Replaces butterfly_layout_metadata (bna/topology/butterfly.py:144-180).
 */
int bfly_topology_init(int64_t num_blocks, int64_t layer_idx, int partner_rule, int local_window_blocks,
                       int sink_count, int partner_count, bfly_topology_t* out);

/*
 * Device: the block-neighbour (partner) table of one layer.
 * Replaces the row loop of build_block_butterfly_layout
 * (bna/torch/attention_wayfinder_permute.py:627-662; bna/mlx/attention.py:235-262)
 * built on butterfly_partner_block / build_butterfly_neighbor_role_row
 * (bna/topology/butterfly.py:108-141, 219-284).
 * neighbors: int32 [num_blocks, kcap]; row b = ordered unique
 * [b, b-1..b-lwb, partners, sinks] (entries in [0, N)), padded with -1.
 * degree: int32 [num_blocks], the row lengths (K = max over blocks).
 * kcap must be >= 1 + local_window_blocks + partner_count + sink_count.
 */
int bfly_block_neighbors(int64_t num_blocks, int64_t layer_idx, int partner_rule,
                         int local_window_blocks, int sink_count, int partner_count,
                         int32_t* neighbors, int kcap, int32_t* degree, hipStream_t stream);

/*
 * Device: one-shot prefill routing tables (block-level cut-off
 * local_start = max(0, b*BS - W + 1)).
 * Replaces _compressed_butterfly_block_index_tensors
 * (bna/torch/attention_wayfinder_permute.py:912-966; bna/mlx/attention.py:1202-1263).
 * raw_idx int32 [N, W+BS-1]; raw_mask uint8 [N, BS, W+BS-1];
 * summary_idx int32 [N, kcap]; summary_mask uint8 [N, BS, kcap].
 */
int bfly_prefill_tables(const int32_t* neighbors, int64_t num_blocks, int kcap, int block_size,
                        int64_t seq_len, int window, int32_t* raw_idx, uint8_t* raw_mask,
                        int32_t* summary_idx, uint8_t* summary_mask, hipStream_t stream);

/*
 * Device: active-row routing tables (token-level cut-off local_start = max(0, p - W + 1)).
 * tail_len < 0: replaces _compressed_butterfly_active_index_tensors
 *   (bna/torch/attention_wayfinder_permute.py:969-1019; bna/mlx/attention.py:1266-1324).
 * tail_len >= 0: replaces _compressed_butterfly_active_indices_from_tail
 *   (bna/mlx/attention.py:1601-1666): raw slots restricted to the tail
 *   [tail_start, tail_start+tail_len) and re-based to it; summaries limited to
 *   n < num_summary_blocks.
 * query_positions int32 [tq]; raw_idx int32 [tq, W]; raw_mask uint8 [tq, W];
 * summary_idx int32 [tq, kcap]; summary_mask uint8 [tq, kcap].
 */
int bfly_active_tables(const int32_t* neighbors, int64_t num_blocks, int kcap, int block_size,
                       int64_t kv_len, int window, const int32_t* query_positions, int64_t tq,
                       int64_t tail_start, int64_t tail_len, int64_t num_summary_blocks,
                       int32_t* raw_idx, uint8_t* raw_mask, int32_t* summary_idx,
                       uint8_t* summary_mask, hipStream_t stream);

/*
 * Device: mean-pool compressor. For each of `rows` (= B*H) sequences of
 * seq_len tokens, out[row, n] = mean of the valid tokens of block n
 * (fp32 accumulate, divide by max(count,1), round to dtype).
 * Replaces _block_mean_summaries_torch (bna/torch/attention_wayfinder_permute.py:1022-1043)
 * and _block_mean_summaries_impl (bna/mlx/attention.py:1373-1393).
 * x: [rows, seq_len, d] -> out: [rows, num_blocks, d]. x2/out2 may be NULL;
 * when given they are pooled in the same launch (keys and values together).
 */
int bfly_block_mean(const void* x, void* out, const void* x2, void* out2, int dtype, int64_t rows,
                    int64_t seq_len, int head_dim, int block_size, int64_t num_blocks,
                    hipStream_t stream);

/*
 * Device: one-shot compressed Butterfly prefill (q_len == k_len).
 * Replaces butterfly_compressed_attention (bna/torch/attention_wayfinder_permute.py:1046-1122)
 * and compressed_butterfly_attention (bna/mlx/attention.py:1401-1468):
 * each query p of block b attends, in one softmax, to the raw keys
 * [max(0, p-W+1), p] and to the mean summaries of the routed neighbours n of b
 * with n < b and (n+1)*BS <= max(0, b*BS - W + 1).
 * q: [B, Hq, T, d]; k, v: [B, Hkv, T, d]; k_summary, v_summary: [B, Hkv, N, d]
 * (from bfly_block_mean); neighbors: int32 [N, kcap]; out: [B, Hq, T, d].
 * Query head h reads kv head h / (Hq/Hkv).  scale multiplies q.k.
 */
int bfly_prefill(const void* q, const void* k, const void* v, const void* k_summary,
                 const void* v_summary, int dtype, int64_t batch, int hq, int hkv, int64_t seq_len,
                 int head_dim, const int32_t* neighbors, int64_t num_blocks, int kcap,
                 int block_size, int window, float scale, void* out, hipStream_t stream);

/*
 * Device: sliding-window attention stream with online-softmax state.
 * Replaces _swa_stream_attention (bna/mlx/attention.py:304-369): query t attends to
 * raw keys [max(0, t - window + 1), t] (window < 1 counts as 1).
 * q: [B, Hq, T, d]; k, v: [B, Hkv, T, d] (head h reads kv head h / (Hq/Hkv));
 * o: [B, Hq, T, d] in dtype; l, m: fp32 [B, Hq, T] = sum of exp(score - m) and the row max.
 * head_dim <= 512.
 */
int bfly_swa_stream(const void* q, const void* k, const void* v, int dtype, int64_t batch, int hq, int hkv,
                    int64_t seq_len, int head_dim, int window, float scale, void* o, float* l, float* m,
                    hipStream_t stream);

/*
 * Device: compressed-block attention stream with online-softmax state.
 * Replaces _compressed_stream_attention (bna/mlx/attention.py:372-516).
 * routed == NULL (HCA mode, :411-439): query t of block b = t / block_size attends to
 * every summary n < b (n < num_summaries).  Otherwise (routed mode, :441-516) it attends
 * to routed[h, b, j] for j < kcap where 0 <= routed[h, b, j] < b (and < num_summaries);
 * routed: int32 [Hq, routed_blocks, kcap] with routed_blocks >= ceil(T / block_size).
 * Rows with no key give o = 0, l = 0, m = -1e30.  Shapes as bfly_swa_stream with
 * k_summary, v_summary: [B, Hkv, num_summaries, d].
 */
int bfly_compressed_stream(const void* q, const void* k_summary, const void* v_summary, int dtype,
                           int64_t batch, int hq, int hkv, int64_t seq_len, int head_dim, int64_t num_summaries,
                           int block_size, const int32_t* routed, int64_t routed_blocks, int kcap, float scale,
                           void* o, float* l, float* m, hipStream_t stream);

/*
 * Device: merge of two (o, l, m) streams into one softmax over the union of their keys.
 * Replaces _online_softmax_merge (bna/mlx/attention.py:519-548):
 * out = (e^(ma-mt) la oa + e^(mb-mt) lb ob) / max(e^(ma-mt) la + e^(mb-mt) lb, 1e-9),
 * mt = max(ma, mb).  oa, ob: [rows, d] in dtype_a / dtype_b; la, ma, lb, mb: fp32 [rows];
 * out: fp32 [rows, d].
 */
int bfly_softmax_merge(const void* oa, int dtype_a, const float* la, const float* ma, const void* ob,
                       int dtype_b, const float* lb, const float* mb, int64_t rows, int head_dim, float* out,
                       hipStream_t stream);

/*
 * Device: active rows over a two-pool cache (token-level cut-off).
 * Replaces compressed_butterfly_attention_from_cache (bna/mlx/attention.py:1816-1876,
 * streams :1669-1813 merged by :519-548) and, with a linear cache
 * (ring_capacity == 0, tail_start == 0, pools = block means of the full K/V,
 * summary_count = N), butterfly_compressed_attention_active
 * (bna/torch/attention_wayfinder_permute.py:1125-1197).
 * Query r sits at position query_positions[r] (device int32 [tq]) or, when
 * query_positions is NULL, at q_pos0 + r.  It attends to the tail keys in
 * [max(tail_start, p-W+1), p] (p < kv_len) and to the routed summaries n of block
 * min(p/BS, N-1) with n < that block, n < summary_count and (n+1)*BS <= max(0, p-W+1).
 * q: [B, Hq, tq, d].  tail_k/tail_v: [B, Hkv, C, d] holding position p at
 * slot p mod C (ring_capacity C > 0), or, when C == 0, the linear tail
 * [B, Hkv, kv_len - tail_start, d] holding position p at row p - tail_start.
 * pool_k/pool_v: [B, Hkv, pool_capacity, d] with rows [0, summary_count) valid.
 * out: [B, Hq, tq, d].
 */
int bfly_attend_cache(const void* q, int dtype, int64_t batch, int hq, int hkv, int64_t tq,
                      int head_dim, const int32_t* query_positions, int64_t q_pos0,
                      const void* tail_k, const void* tail_v, int64_t ring_capacity,
                      int64_t tail_start, int64_t kv_len, const void* pool_k, const void* pool_v,
                      int64_t pool_capacity, int64_t summary_count, const int32_t* neighbors,
                      int64_t num_blocks, int kcap, int block_size, int window, float scale,
                      void* out, hipStream_t stream);

/*
 * Device (host loop): a streaming chunked prefill of one layer over a two-pool
 * cache that already holds a first chunk.  For chunk c (q[c]: [B, Hq, len_c, d],
 * k[c]/v[c]: [B, Hkv, len_c, d], out[c]: [B, Hq, len_c, d], host pointer arrays):
 * the counter bookkeeping and append + block pooling of
 * CompressedKVCache.update_and_fetch (bna/mlx/compressed_cache.py:94-172, with
 * the cache's own window cache_window), then the chunk's queries attend from the
 * cache as compressed_butterfly_attention_from_cache does with the layout of the
 * live kv_len (bna/mlx/attention.py:1816-1876; stage = layer_idx mod stage count)
 * -- the per-chunk schedule of the Qwen layer swap (bna/integrations/
 * qwen_mlx.py:1515-1581) with no host round trip between chunks.
 * counters (host int64[4], in/out): {offset, tail_size, summary_count,
 * summary_offset}; they are left at the last completed chunk, and *chunks_done
 * counts the chunks whose work was enqueued.  ring_k/ring_v: [B, Hkv,
 * ring_capacity, d] (position p at slot p mod ring_capacity); pool_k/pool_v:
 * [B, Hkv, pool_capacity, d].  bf16 with head_dim 64/128/256 and window <= 64
 * only (BFLY_ERR_UNSUPPORTED otherwise, before any work); BFLY_ERR_CAPACITY when
 * the tail or the pool overflows (the reference's RuntimeError).
 */
int bfly_stream_chunks(int64_t n_chunks, const void* const* q, const void* const* k, const void* const* v,
                       void* const* out, const int64_t* chunk_len, int dtype, int64_t batch, int hq, int hkv,
                       int head_dim, void* ring_k, void* ring_v, int64_t ring_capacity, void* pool_k, void* pool_v,
                       int64_t pool_capacity, int64_t* counters, int cache_window, int64_t layer_idx,
                       int partner_rule, int local_window_blocks, int sink_count, int partner_count, int block_size,
                       int window, float scale, int64_t* chunks_done, hipStream_t stream);

/*
 * Device: one decode step -- a single new query per sequence at position
 * p = kv_len - 1 over the two-pool cache, with the cache append fused in.
 * Replaces, for one active row, compressed_butterfly_attention_from_cache
 * (bna/mlx/attention.py:1816-1876) preceded by the tail append of
 * CompressedKVCache.update_and_fetch (bna/mlx/compressed_cache.py:104-118).
 * When k_new/v_new ([B, Hkv, 1, d]) are given they are the token at p: they are
 * written to ring slot p mod ring_capacity and scored from the staged copy.
 * Keys: tail positions [max(tail_start, p-W+1), p] and the routed summaries n of
 * block min(p/BS, N-1) with n < that block, n < summary_count and
 * (n+1)*BS <= max(0, p-W+1), one softmax (the exact two-stream merge).
 * q/out: [B, Hq, 1, d].  ring_k/ring_v: [B, Hkv, C, d] ring (C = ring_capacity > 0),
 * or, when C == 0, the linear tail [B, Hkv, kv_len - tail_start, d].
 * pool_k/pool_v: [B, Hkv, pool_capacity, d].  head_dim 64 or 128 (256 for bf16);
 * window <= 64.  The routed row of block min(p/BS, N-1) is computed in the
 * kernel from `topology` (host struct, from bfly_topology_init at num_blocks),
 * so a step needs no device table and no dependent table read.
 */
int bfly_decode(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                int64_t ring_capacity, int64_t tail_start, int64_t kv_len, const void* pool_k,
                const void* pool_v, int64_t pool_capacity, int64_t summary_count,
                const bfly_topology_t* topology, int64_t num_blocks, int block_size, int window,
                float scale, void* out, hipStream_t stream);

/*
 * Length in int64 words of the bfly_decode_step counter array for n = batch*hkv
 * sequences: an 8-word header (word 4: error) and n*c + 8 copies of 32 words,
 * c = 64 copies per sequence when n <= 16 (the attending workgroups of
 * bfly_decode_step_qk_norm_oproj), else 1; sequence s owns copies s + n*j
 * (j < c), the step's eight route workgroups the last eight.  No counterpart in
 * the reference (its counters are host attributes).
 */
int64_t bfly_decode_state_words(int64_t batch, int hkv);

/*
 * Device: one decode step with the cache counters held on the device, so a
 * step has fixed arguments and can be captured in a HIP graph.  Same result as
 * CompressedKVCache.update_and_fetch of one token (bna/mlx/compressed_cache.py:94-172:
 * append, summarise every block with end + cache_window <= offset, trim whole
 * blocks while tail_size - BS >= cache_window, where cache_window is the cache's
 * own local_window_tokens) followed by compressed_butterfly_attention_from_cache
 * for that token with the attention window `window` (bna/mlx/attention.py:1816-1876),
 * with the layout of the live kv_len (stage = layer_idx mod stage_count at
 * ceil(kv_len / BS) blocks).  cache_window in [1, 2^20); the ring must hold
 * cache_window + BS rows.
 * state: device int64[bfly_decode_state_words(batch, hkv)]: state[4] is the
 * error word; copy g (32 words at state[8 + 32g ..], the copies of sequence
 * b*Hkv + kv head and the route workgroups' as bfly_decode_state_words lays
 * them out) holds {offset, tail_size, summary_count, summary_offset} in words
 * 0..3, advanced by the step (all copies stay equal; initialise every copy; the
 * host reads copy 0), and words 4..31 hold the kernel's
 * own cache of the next step's routed row (initialise to zero: zero is "none";
 * the kernel uses an entry only when it names the step's kv_len and
 * arguments).  On a capacity
 * overflow the step changes nothing and sets state[4] = 1 (the reference's
 * RuntimeError; read it back to raise); later steps then change nothing either
 * until the host rewrites the counters.
 * Other arguments as bfly_decode; ring_k/ring_v is the ring (capacity > 0).
 */
int bfly_decode_step(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                     const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                     int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                     int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks,
                     int sink_count, int partner_count, int block_size, int window, int cache_window,
                     float scale, void* out, hipStream_t stream);

/*
 * Device: bfly_decode_step for a decoder whose attention applies per-head q/k
 * RMSNorm and rotate-half RoPE after its projections: q and k_new are the raw
 * projection rows (for batch 1 they may be views of one fused q|k|v output), and
 * the kernel norms them (q_norm_weight / k_norm_weight [128] bf16, eps) and
 * rotates them at position kv_len - 1 with row kv_len - 1 of rope_cos / rope_sin
 * ([rope_rows][128] fp32), then appends the normed k and attends as
 * bfly_decode_step does.  The q and k rows are bit-identical to
 * bfly_qk_norm_rope's (include/butterfly_amd_decoder.h).  bf16, head_dim 128
 * only (else BFLY_ERR_INVALID).  A position at or past rope_rows sets the step
 * error word to 2 (state[4] = 2; a capacity overflow sets 1) and changes nothing.  Replaces the projection tail of the
 * swapped attention (bna/integrations/qwen_torch.py:550-562, qwen_mlx.py:288-357)
 * and the step of bfly_decode_step (bna/mlx/compressed_cache.py:94-172,
 * bna/mlx/attention.py:1816-1876) in one launch.
 */
int bfly_decode_step_qk_norm(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                             const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                             int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                             int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks,
                             int sink_count, int partner_count, int block_size, int window, int cache_window,
                             float scale, const void* q_norm_weight, const void* k_norm_weight, const float* rope_cos,
                             const float* rope_sin, int64_t rope_rows, float eps, void* out, hipStream_t stream);

/*
 * Device: bfly_decode_step_qk_norm with the attention output projection of a
 * decoder layer applied in the same launch, as partial products per kv head:
 * o_parts[g][b][i] (fp32, [hkv][batch][o_out_features]) = row i of
 * W_o[:, 512 g .. 512 g + 511] times the attention output of kv head g's four
 * query heads, W_o in bfly_q4_gemv's 4-bit layout (o_packed / o_scale_bias,
 * in_features = hq * head_dim = 2048, group o_group: a power of two in [32, 2048]).
 * The partial rows combined as (p0 + p1) + (p2 + p3) and rounded to bf16 equal
 * bfly_q4_gemv over `out` bit for bit (bfly_add_rms_norm_q4_gemv_silu_parts takes
 * them so).  `out` still receives the attention output.  Shapes: 16 query heads
 * over 4 kv heads of 128, batch * 4 <= 16, o_out_features a multiple of 32 up to
 * 2048 or of 64 up to 4096 (else BFLY_ERR_INVALID).  The launch runs
 * o_out_features / 32 (beyond 2048: / 64) workgroups per sequence, each computing
 * the attention (every one appends the same token and pools the same due block)
 * and 32 (64) rows of the product.  Replaces
 * the swapped attention's output projection (bna/integrations/qwen_mlx.py:1295-1792
 * projects the attention output with the layer's o_proj; qwen_torch.py:1221-1622)
 * together with bfly_decode_step_qk_norm in one launch.
 */
int bfly_decode_step_qk_norm_oproj(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                                   const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                                   int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                                   int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks,
                                   int sink_count, int partner_count, int block_size, int window, int cache_window,
                                   float scale, const void* q_norm_weight, const void* k_norm_weight,
                                   const float* rope_cos, const float* rope_sin, int64_t rope_rows, float eps,
                                   const void* o_packed, const void* o_scale_bias, int64_t o_out_features,
                                   int o_group, float* o_parts, void* out, hipStream_t stream);

/*
 * Device: append `step` new tokens at positions [offset, offset+step) of the
 * tail ring (slot = position mod ring_capacity).
 * Replaces the tail append of CompressedKVCache.update_and_fetch
 * (bna/mlx/compressed_cache.py:104-118).  k_new/v_new: [B, Hkv, step, d];
 * ring_k/ring_v: [B, Hkv, ring_capacity, d].  Requires step <= ring_capacity.
 */
int bfly_cache_append(const void* k_new, const void* v_new, int dtype, int64_t batch, int hkv,
                      int64_t step, int head_dim, void* ring_k, void* ring_v,
                      int64_t ring_capacity, int64_t offset, hipStream_t stream);

/*
 * Device: summarise `n_blocks` complete blocks starting at position
 * first_block_pos (a multiple of block_size) from the tail ring into pool slots
 * [first_slot, first_slot + n_blocks): fp32 mean over block_size tokens, rounded to dtype.
 * Replaces the summarise loop of CompressedKVCache.update_and_fetch
 * (bna/mlx/compressed_cache.py:120-149).
 */
int bfly_cache_compress(const void* ring_k, const void* ring_v, int dtype, int64_t batch, int hkv,
                        int head_dim, int64_t ring_capacity, int64_t first_block_pos,
                        int64_t n_blocks, int block_size, void* pool_k, void* pool_v,
                        int64_t pool_capacity, int64_t first_slot, hipStream_t stream);

/*
 * Device: one chunk's whole cache update in one launch -- bfly_cache_append of
 * k_new/v_new at `offset`, then bfly_cache_compress of the `n_blocks` due blocks
 * from first_block_pos into pool slots [first_slot, first_slot + n_blocks).
 * The blocks' tokens are read where they are before the append (ring below
 * `offset`, k_new/v_new from it), so the result equals the two calls in order,
 * bit for bit.  The due blocks must lie in the post-append tail
 * [offset + step - ring_capacity, offset + step).  Replaces the append and
 * summarise steps of CompressedKVCache.update_and_fetch
 * (bna/mlx/compressed_cache.py:104-149).
 */
int bfly_cache_update(const void* k_new, const void* v_new, int dtype, int64_t batch, int hkv,
                      int64_t step, int head_dim, void* ring_k, void* ring_v, int64_t ring_capacity,
                      int64_t offset, int64_t first_block_pos, int64_t n_blocks, int block_size,
                      void* pool_k, void* pool_v, int64_t pool_capacity, int64_t first_slot,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BUTTERFLY_AMD_H_ */
