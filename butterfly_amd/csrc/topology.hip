// Staged Butterfly block topology on gfx950: host scalar metadata, the device
// block-neighbour (partner) table and the device routing tables.
//
// Reference semantics: bna/topology/butterfly.py (partner rules, stage
// metadata, ordered row), bna/torch/attention_wayfinder_permute.py:568-682
// (layout rows), :912-1019 (routing tables), bna/mlx/attention.py:1601-1666
// (tail-relative active tables).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "bfly_topology.h"

namespace bfly {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

static int host_width(int64_t n) {
  if (n <= 1) return 1;
  // Same floating-point expression as the reference (math.ceil(math.log2(n))).
  return (int)ceil(log2((double)n));
}

static bool valid_rule(int rule) { return rule >= BFLY_RULE_XOR && rule <= BFLY_RULE_RANDOM; }

// One thread per block: row = ordered unique [b, b-1..b-lwb, partners, sinks].
__global__ void neighbors_kernel(int64_t nblocks, bfly_topology_t topo, int32_t* __restrict__ out, int kcap,
                                 int32_t* __restrict__ degree) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  int32_t* row = out + b * kcap;
  const int len = neighbor_row(b, nblocks, topo, row, kcap);
  for (int i = len; i < kcap; ++i) row[i] = -1;
  degree[b] = len;
}

// One workgroup per block b.  Block-level cut-off.
__global__ void prefill_tables_kernel(const int32_t* __restrict__ nbr, int kcap, int bs,
                                      int64_t T, int W, int32_t* __restrict__ raw_idx,
                                      uint8_t* __restrict__ raw_mask,
                                      int32_t* __restrict__ sidx, uint8_t* __restrict__ smask) {
  const int64_t b = blockIdx.x;
  const int slots = W + bs - 1;
  const int64_t qstart = b * bs;
  const int64_t lstart = qstart - W + 1 > 0 ? qstart - W + 1 : 0;
  __shared__ uint8_t used[64];
  __shared__ int32_t chosen[64];
  if (threadIdx.x == 0) {
    int c = 0;
    for (int j = 0; j < kcap; ++j) {
      used[j] = 0;
      chosen[j] = 0;
    }
    for (int j = 0; j < kcap; ++j) {
      int64_t n = nbr[b * kcap + j];
      if (n < 0 || n >= b) continue;
      if ((n + 1) * bs > lstart) continue;
      chosen[c] = (int32_t)n;
      used[c] = 1;
      if (++c >= kcap) break;
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < slots; j += blockDim.x) {
    int64_t p = lstart + j;
    int64_t c = p < 0 ? 0 : (p > T - 1 ? (T - 1 > 0 ? T - 1 : 0) : p);
    raw_idx[b * slots + j] = (int32_t)c;
  }
  for (int j = threadIdx.x; j < kcap; j += blockDim.x) sidx[b * kcap + j] = chosen[j];
  const int64_t total = (int64_t)bs * slots;
  for (int64_t e = threadIdx.x; e < total; e += blockDim.x) {
    int i = (int)(e / slots), j = (int)(e % slots);
    int64_t qp = qstart + i, rp = lstart + j;
    bool ok = qp < T && rp < T && rp <= qp && rp >= qp - W + 1;
    raw_mask[(b * bs + i) * slots + j] = ok ? 1 : 0;
  }
  const int64_t stotal = (int64_t)bs * kcap;
  for (int64_t e = threadIdx.x; e < stotal; e += blockDim.x) {
    int i = (int)(e / kcap), j = (int)(e % kcap);
    bool ok = used[j] && (qstart + i < T);
    smask[(b * bs + i) * kcap + j] = ok ? 1 : 0;
  }
}

// One thread per query row.  Token-level cut-off; optional tail restriction.
__global__ void active_tables_kernel(const int32_t* __restrict__ nbr, int64_t nblocks, int kcap,
                                     int bs, int64_t kv_len, int W,
                                     const int32_t* __restrict__ qpos, int64_t tq,
                                     int64_t tail_start, int64_t tail_len, int64_t nsum,
                                     int32_t* __restrict__ raw_idx, uint8_t* __restrict__ raw_mask,
                                     int32_t* __restrict__ sidx, uint8_t* __restrict__ smask) {
  int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= tq) return;
  const int64_t p = qpos[r];
  int64_t blk = p / (bs > 1 ? bs : 1);
  if (blk < 0) blk = 0;
  if (blk > nblocks - 1) blk = nblocks - 1 > 0 ? nblocks - 1 : 0;
  const int64_t lstart = p - W + 1 > 0 ? p - W + 1 : 0;
  const bool tail = tail_len >= 0;
  for (int j = 0; j < W; ++j) {
    int64_t rp = lstart + j;
    bool ok = rp <= p && rp < kv_len;
    int64_t idx;
    if (tail) {
      ok = ok && rp >= tail_start && rp < tail_start + tail_len;
      int64_t hi = tail_len - 1 > 0 ? tail_len - 1 : 0;
      idx = rp - tail_start;
      idx = idx < 0 ? 0 : (idx > hi ? hi : idx);
    } else {
      int64_t hi = kv_len - 1 > 0 ? kv_len - 1 : 0;
      idx = rp < 0 ? 0 : (rp > hi ? hi : rp);
    }
    raw_idx[r * W + j] = (int32_t)idx;
    raw_mask[r * W + j] = ok ? 1 : 0;
  }
  for (int j = 0; j < kcap; ++j) {
    sidx[r * kcap + j] = 0;
    smask[r * kcap + j] = 0;
  }
  int c = 0;
  for (int j = 0; j < kcap; ++j) {
    int64_t n = nbr[blk * kcap + j];
    if (n < 0 || n >= blk) continue;
    if (tail && n >= nsum) continue;
    if ((n + 1) * bs > lstart) continue;
    sidx[r * kcap + c] = (int32_t)n;
    smask[r * kcap + c] = 1;
    if (++c >= kcap) break;
  }
}

}  // namespace bfly

using namespace bfly;

extern "C" const char* bfly_last_error(void) { return g_err; }

extern "C" int bfly_abi_version(void) { return BFLY_ABI_VERSION; }

extern "C" int bfly_stage_meta(int64_t num_blocks, int64_t layer_idx, int partner_rule,
                               int32_t* stage_idx, int32_t* stage_count, int32_t* width) {
  BFLY_CHECK_ARG(valid_rule(partner_rule), "unsupported partner rule %d", partner_rule);
  BFLY_CHECK_ARG(stage_idx && stage_count && width, "null output pointer");
  int w = host_width(num_blocks);
  int count = partner_rule == BFLY_RULE_BENES ? (2 * w - 2 > 1 ? 2 * w - 2 : 1) : w;
  int64_t s = layer_idx % count;
  if (s < 0) s += count;  // Python modulo semantics for negative layer indices
  *stage_idx = (int32_t)s;
  *stage_count = count;
  *width = w;
  return BFLY_OK;
}

extern "C" int bfly_partner_bits(int stage_idx, int stage_count, int width, int partner_count,
                                 int partner_rule, int32_t* bits) {
  BFLY_CHECK_ARG(valid_rule(partner_rule), "unsupported partner rule %d", partner_rule);
  if (width <= 0 || partner_count <= 0) return BFLY_OK;
  BFLY_CHECK_ARG(bits != nullptr, "null bits pointer");
  BFLY_CHECK_ARG(stage_count > 0, "stage_count must be positive");
  for (int j = 0; j < partner_count; ++j) {
    if (partner_rule == BFLY_RULE_BENES) {
      int base = stage_count <= 1 ? 0 : stage_idx % stage_count;
      int phase = (base + j) % stage_count;
      bits[j] = width <= 1 ? 0 : (phase < width ? phase : 2 * width - 2 - phase);
    } else {
      bits[j] = (stage_idx + j) % width;
    }
  }
  return BFLY_OK;
}

extern "C" int bfly_topology_init(int64_t num_blocks, int64_t layer_idx, int partner_rule, int local_window_blocks,
                                  int sink_count, int partner_count, bfly_topology_t* out) {
  BFLY_CHECK_ARG(num_blocks > 0 && num_blocks <= INT32_MAX, "num_blocks out of range: %lld", (long long)num_blocks);
  BFLY_CHECK_ARG(local_window_blocks >= 0 && sink_count >= 0 && partner_count >= 0, "negative topology parameter");
  BFLY_CHECK_ARG(partner_count <= BFLY_MAX_PARTNERS, "partner_count > %d", BFLY_MAX_PARTNERS);
  BFLY_CHECK_ARG(out != nullptr, "null output pointer");
  bfly_topology_t t{};
  int rc = bfly_stage_meta(num_blocks, layer_idx, partner_rule, &t.stage_idx, &t.stage_count, &t.width);
  if (rc) return rc;
  rc = bfly_partner_bits(t.stage_idx, t.stage_count, t.width, partner_count, partner_rule, t.partner_bits);
  if (rc) return rc;
  t.rule = partner_rule;
  t.local_window_blocks = local_window_blocks;
  t.sink_count = sink_count;
  t.partner_count = partner_count;
  *out = t;
  return BFLY_OK;
}

extern "C" int bfly_block_neighbors(int64_t num_blocks, int64_t layer_idx, int partner_rule,
                                    int local_window_blocks, int sink_count, int partner_count,
                                    int32_t* neighbors, int kcap, int32_t* degree,
                                    hipStream_t stream) {
  BFLY_CHECK_ARG(kcap >= 1 + local_window_blocks + partner_count + sink_count && kcap <= 64,
                 "kcap=%d must be in [1+lwb+partners+sinks, 64]", kcap);
  BFLY_CHECK_ARG(neighbors && degree, "null output pointer");
  bfly_topology_t t;
  int rc = bfly_topology_init(num_blocks, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count, &t);
  if (rc) return rc;
  const int threads = 256;
  const int grid = (int)((num_blocks + threads - 1) / threads);
  hipLaunchKernelGGL(neighbors_kernel, dim3(grid), dim3(threads), 0, stream, num_blocks, t, neighbors, kcap, degree);
  BFLY_CHECK_LAUNCH("bfly_block_neighbors");
  return BFLY_OK;
}

extern "C" int bfly_prefill_tables(const int32_t* neighbors, int64_t num_blocks, int kcap,
                                   int block_size, int64_t seq_len, int window, int32_t* raw_idx,
                                   uint8_t* raw_mask, int32_t* summary_idx, uint8_t* summary_mask,
                                   hipStream_t stream) {
  BFLY_CHECK_ARG(seq_len > 0, "T must be positive");
  BFLY_CHECK_ARG(window > 0, "local_window_tokens must be positive");
  BFLY_CHECK_ARG(block_size > 0 && kcap > 0 && kcap <= 64, "bad block_size/kcap");
  BFLY_CHECK_ARG(num_blocks == (seq_len + block_size - 1) / block_size,
                 "num_blocks=%lld does not cover seq_len=%lld", (long long)num_blocks,
                 (long long)seq_len);
  BFLY_CHECK_ARG(neighbors && raw_idx && raw_mask && summary_idx && summary_mask, "null pointer");
  hipLaunchKernelGGL(prefill_tables_kernel, dim3((unsigned)num_blocks), dim3(256), 0, stream,
                     neighbors, kcap, block_size, seq_len, window, raw_idx, raw_mask, summary_idx,
                     summary_mask);
  BFLY_CHECK_LAUNCH("bfly_prefill_tables");
  return BFLY_OK;
}

extern "C" int bfly_active_tables(const int32_t* neighbors, int64_t num_blocks, int kcap,
                                  int block_size, int64_t kv_len, int window,
                                  const int32_t* query_positions, int64_t tq, int64_t tail_start,
                                  int64_t tail_len, int64_t num_summary_blocks, int32_t* raw_idx,
                                  uint8_t* raw_mask, int32_t* summary_idx, uint8_t* summary_mask,
                                  hipStream_t stream) {
  BFLY_CHECK_ARG(kv_len > 0, "kv_len must be positive");
  BFLY_CHECK_ARG(window > 0, "local_window_tokens must be positive");
  BFLY_CHECK_ARG(block_size > 0 && kcap > 0 && kcap <= 64 && num_blocks > 0,
                 "bad block_size/kcap/num_blocks");
  if (tq == 0) return BFLY_OK;
  BFLY_CHECK_ARG(tq > 0 && neighbors && query_positions && raw_idx && raw_mask && summary_idx &&
                     summary_mask,
                 "null pointer or negative tq");
  const int threads = 128;
  hipLaunchKernelGGL(active_tables_kernel, dim3((unsigned)((tq + threads - 1) / threads)),
                     dim3(threads), 0, stream, neighbors, num_blocks, kcap, block_size, kv_len,
                     window, query_positions, tq, tail_start, tail_len, num_summary_blocks,
                     raw_idx, raw_mask, summary_idx, summary_mask);
  BFLY_CHECK_LAUNCH("bfly_active_tables");
  return BFLY_OK;
}
