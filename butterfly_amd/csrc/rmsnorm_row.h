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

// The row's inputs of one thread in 16-byte pieces: x, y (zero when null) and the norm weight.
template <int PER>
struct RmsRowIn {
  bf16x8 x[PER / 8], y[PER / 8], w[PER / 8];
};

// Thread t < 256 of the participating threads holds elements [t PER, t PER + PER)
// of the row (dim = 256 PER), 16-byte pieces (PER a multiple of 8, every pointer 16-byte
// aligned).  Requested apart from the arithmetic, so that a caller can issue them ahead of
// other loads and not wait for those.  kX false: x is not read (the caller forms in.x).
template <int PER, bool kX = true>
__device__ __forceinline__ RmsRowIn<PER> rms_row_load(const __bf16* __restrict__ x, const __bf16* __restrict__ y,
                                                      const __bf16* __restrict__ w, int t, bool active) {
  RmsRowIn<PER> in{};
  if (active) {
    const int64_t base = (int64_t)t * PER;
#pragma unroll
    for (int c = 0; c < PER / 8; ++c) {
      if constexpr (kX) in.x[c] = *reinterpret_cast<const bf16x8*>(x + base + 8 * c);
      if (y != nullptr) in.y[c] = *reinterpret_cast<const bf16x8*>(y + base + 8 * c);
      in.w[c] = *reinterpret_cast<const bf16x8*>(w + base + 8 * c);
    }
  }
  return in;
}

// The residual add + RMSNorm of rms_row_load's pieces: h_out (null when y is) and n_out get
// the row's elements [t PER, t PER + PER).  Every thread of the workgroup calls it (the
// barrier is the workgroup's); threads with `active` false only take the barrier.  part: 4
// floats of LDS.
template <int PER>
__device__ __forceinline__ void add_rmsnorm_row_from(const RmsRowIn<PER>& in, bool has_y, __bf16* __restrict__ h_out,
                                                     __bf16* __restrict__ n_out, int dim, float eps, int t,
                                                     bool active, float* part) {
#pragma clang fp contract(off)
  const int64_t base = (int64_t)t * PER;
  float h[PER];
  if (active) {
#pragma unroll
    for (int c = 0; c < PER / 8; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = (float)in.x[c][e];
        if (has_y) v = (float)(__bf16)(v + (float)in.y[c][e]);   // residual stream in bf16
        h[8 * c + e] = v;
      }
    if (has_y && h_out != nullptr) {
#pragma unroll
      for (int c = 0; c < PER / 8; ++c) {
        bf16x8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = (__bf16)h[8 * c + e];
        *reinterpret_cast<bf16x8*>(h_out + base + 8 * c) = hv;
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
#pragma unroll
  for (int c = 0; c < PER / 8; ++c) {
    bf16x8 nv;
#pragma unroll
    for (int e = 0; e < 8; ++e) nv[e] = (__bf16)(h[8 * c + e] * r * (float)in.w[c][e]);
    *reinterpret_cast<bf16x8*>(n_out + base + 8 * c) = nv;
  }
}

// Both steps at once; kVec false: element loads (any alignment), the same arithmetic.
template <int PER, bool kVec>
__device__ __forceinline__ void add_rmsnorm_row(const __bf16* __restrict__ x, const __bf16* __restrict__ y,
                                                const __bf16* __restrict__ w, __bf16* __restrict__ h_out,
                                                __bf16* __restrict__ n_out, int dim, float eps, int t, bool active,
                                                float* part) {
#pragma clang fp contract(off)
  if constexpr (kVec) {
    const RmsRowIn<PER> in = rms_row_load<PER>(x, y, w, t, active);
    add_rmsnorm_row_from<PER>(in, y != nullptr, h_out, n_out, dim, eps, t, active, part);
  } else {
    const int64_t base = (int64_t)t * PER;
    float h[PER];
    if (active) {
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
#pragma unroll
    for (int e = 0; e < PER; ++e) n_out[base + e] = (__bf16)(h[e] * r * (float)w[t * PER + e]);
  }
}

}  // namespace bfly
