// Device-side staged Butterfly topology shared by the table builder and the
// decode kernel.  Reference: butterfly_partner_block (bna/topology/butterfly.py:108-141)
// and the ordered, de-duplicated row [b, b-1..b-lwb, partners, sinks]
// (butterfly.py:219-284; bna/torch/attention_wayfinder_permute.py:627-662).
#pragma once

#include "bfly_common.h"

namespace bfly {

__device__ __forceinline__ int64_t bit_reverse(int64_t value, int nbits) {
  int64_t out = 0;
  for (int i = 0; i < nbits; ++i) out = (out << 1) | ((value >> i) & 1);
  return out;
}

// Partner of `block` for one bit; -1 where the reference returns None.
__device__ __forceinline__ int64_t partner_block(int64_t block, int bit, int64_t nblocks, int rule, int width) {
  if (bit < 0 || bit >= (width > 1 ? width : 1)) return -1;
  int64_t p;
  switch (rule) {
    case BFLY_RULE_CAUSAL_SHIFT: p = block - ((int64_t)1 << bit); break;
    case BFLY_RULE_XOR:
    case BFLY_RULE_BENES: p = block ^ ((int64_t)1 << bit); break;
    case BFLY_RULE_FIXED_STRIDE: p = block - 1; break;
    case BFLY_RULE_RANDOM: {
      if (block <= 0) return -1;
      uint32_t seed = (uint32_t)block * 2654435761u + (uint32_t)bit * 374761393u;
      p = (int64_t)(seed % (uint64_t)block);
      break;
    }
    default: p = bit_reverse(bit_reverse(block, width) ^ ((int64_t)1 << bit), width); break;
  }
  if (p < 0 || p >= nblocks || p > block) return -1;
  return p;
}

// Row of block b into row[0..cap); returns its length.  `row` may live in
// global memory or LDS (the de-duplication reads it back).
__device__ __forceinline__ int neighbor_row(int64_t b, int64_t nblocks, const bfly_topology_t& t, int32_t* row,
                                            int cap) {
  int len = 0;
  auto push = [&](int64_t v) {
    if (v < 0 || v >= nblocks) return;
    for (int i = 0; i < len; ++i)
      if (row[i] == (int32_t)v) return;
    if (len < cap) row[len++] = (int32_t)v;
  };
  push(b);
  for (int off = 1; off <= t.local_window_blocks; ++off) {
    if (b - off < 0) break;
    push(b - off);
  }
  // constant trip count so the bit array stays in registers (no private copy)
#pragma unroll
  for (int j = 0; j < BFLY_MAX_PARTNERS; ++j)
    if (j < t.partner_count) push(partner_block(b, t.partner_bits[j], nblocks, t.rule, t.width));
  const int64_t ns = t.sink_count < nblocks ? t.sink_count : nblocks;
  for (int64_t s = 0; s < ns; ++s) push(s);
  return len;
}

}  // namespace bfly
