// Residual add + RMSNorm of one row by 256 threads, shared by the row kernel
// (decoder_ops.hip) and the 4-bit products that take their input through it
// (qgemv.hip).  Rounding points are those of the PyTorch form in
// butterfly_amd/decoder.py: h = bf16(x + y), n = bf16((h * r) * w) with
// r = rsqrt(mean(h^2) + eps); the mean square sums each thread's PER elements
// in order with fma, then the 64 lanes of each wave by xor shuffles (32, 16, ...,
// 1), then the four waves as (w0 + w1) + (w2 + w3).
#pragma once

#include "bfly_common.h"

namespace bfly {

__device__ __forceinline__ float dec_wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Thread t < 256 of the participating threads holds elements [t PER, t PER + PER)
// of the row (dim = 256 PER).  x, y (may be null), h_out (null when y is), n_out:
// the row's first element; w: the norm weight.  Every thread of the workgroup calls
// it (the barrier is the workgroup's); threads with `active` false only take the
// barrier.  part: 4 floats of LDS.  kVec: 16-byte pieces (PER a multiple of 8 and
// every pointer 16-byte aligned).
template <int PER, bool kVec>
__device__ __forceinline__ void add_rmsnorm_row(const __bf16* __restrict__ x, const __bf16* __restrict__ y,
                                                const __bf16* __restrict__ w, __bf16* __restrict__ h_out,
                                                __bf16* __restrict__ n_out, int dim, float eps, int t, bool active,
                                                float* part) {
#pragma clang fp contract(off)
  const int64_t base = (int64_t)t * PER;
  float h[PER];
  if (active) {
    if constexpr (kVec) {
#pragma unroll
      for (int c = 0; c < PER / 8; ++c) {
        const bf16x8 xv = *reinterpret_cast<const bf16x8*>(x + base + 8 * c);
        bf16x8 yv{};
        if (y != nullptr) yv = *reinterpret_cast<const bf16x8*>(y + base + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float v = (float)xv[e];
          if (y != nullptr) v = (float)(__bf16)(v + (float)yv[e]);   // residual stream in bf16
          h[8 * c + e] = v;
        }
      }
      if (y != nullptr && h_out != nullptr) {
#pragma unroll
        for (int c = 0; c < PER / 8; ++c) {
          bf16x8 hv;
#pragma unroll
          for (int e = 0; e < 8; ++e) hv[e] = (__bf16)h[8 * c + e];
          *reinterpret_cast<bf16x8*>(h_out + base + 8 * c) = hv;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        float v = (float)x[base + e];
        if (y != nullptr) v = (float)(__bf16)(v + (float)y[base + e]);   // residual stream in bf16
        h[e] = v;
      }
      if (y != nullptr && h_out != nullptr) {
#pragma unroll
        for (int e = 0; e < PER; ++e) h_out[base + e] = (__bf16)h[e];
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) ss = fmaf(h[e], h[e], ss);
    ss = dec_wave_sum64(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
  }
  __syncthreads();
  if (!active) return;
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = rsqrtf(tot / (float)dim + eps);
  if constexpr (kVec) {
#pragma unroll
    for (int c = 0; c < PER / 8; ++c) {
      const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + t * PER + 8 * c);
      bf16x8 nv;
#pragma unroll
      for (int e = 0; e < 8; ++e) nv[e] = (__bf16)(h[8 * c + e] * r * (float)wv[e]);
      *reinterpret_cast<bf16x8*>(n_out + base + 8 * c) = nv;
    }
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) n_out[base + e] = (__bf16)(h[e] * r * (float)w[t * PER + e]);
  }
}

}  // namespace bfly
