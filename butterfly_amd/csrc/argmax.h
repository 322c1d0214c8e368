// Greedy selection (torch.argmax's order) shared by the argmax passes (decoder_ops.hip) and the
// 4-bit product that leaves per-workgroup candidates (qgemv.hip).
#pragma once

#include "bfly_common.h"

namespace bfly {

// Greedy selection order of torch.argmax: NaN above every number, then larger
// values, then the lower index among equals.
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float bv, int64_t bi) {
  if (bi < 0) return true;
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

__device__ __forceinline__ void argmax_combine(float& bv, int64_t& bi, float v, int64_t i) {
  if (i >= 0 && argmax_better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

// Block-wide combine of every thread's (value, index) candidate (64 NW threads): thread 0
// holds the result.
template <int NW = 4>
__device__ __forceinline__ void argmax_block(float& bv, int64_t& bi) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int64_t oi = __shfl_xor(bi, o);
    argmax_combine(bv, bi, ov, oi);
  }
  __shared__ float sv[NW];
  __shared__ int64_t si[NW];
  const int t = threadIdx.x;
  if ((t & 63) == 0) {
    sv[t >> 6] = bv;
    si[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0)
    for (int w = 1; w < NW; ++w) argmax_combine(bv, bi, sv[w], si[w]);
}

// (value, index) as one 64-bit key that orders like the selection above: the value's bits
// mapped to an unsigned order (-0 taken as +0, every NaN above every number), then the index
// reversed, so the larger key is the better candidate and 0 is below every key.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (v != v) hi = 0xFFFFFFFFu;
  return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - i);
}
__device__ __forceinline__ int64_t argmax_key_index(uint64_t k) { return (int64_t)(0xFFFFFFFFu - (uint32_t)k); }

}  // namespace bfly
