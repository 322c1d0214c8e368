// Elementwise and row-wise steps of the swapped decoder on gfx950 (bf16 in and
// out, fp32 inside), each one launch where the PyTorch formulation takes five to
// eight: residual add + RMSNorm, per-head q/k RMSNorm + rotate-half RoPE + the
// [B, T, H*d] -> [B, H, T, d] layout change, and SiLU(gate) * up.
//
// Reference: the projection step of the swapped attention applies q_norm and
// k_norm per head, transposes to heads-first and applies rotate-half RoPE
// (bna/integrations/qwen_torch.py:550-562; qwen_mlx.py:288-357).  The rounding
// points follow the PyTorch forms in butterfly_amd/decoder.py exactly (bf16
// after the residual add, after each norm, after RoPE, after SiLU and after the
// product), so results differ from them only by the fp32 summation order of the
// mean square and by the last bit of rsqrt/exp.
#include <mutex>

#include "bfly_common.h"
#include "argmax.h"
#include "rmsnorm_row.h"
#include "../../include/butterfly_amd_decoder.h"

// products and sums are rounded one by one, as the PyTorch forms do
#pragma clang fp contract(off)

namespace bfly {

// Any dim that is a multiple of 256: the sum of squares from global memory,
// then the row is read again (it is in cache) for the output.
__global__ void __launch_bounds__(256) add_rmsnorm_any_kernel(const __bf16* __restrict__ x,
                                                              const __bf16* __restrict__ y,
                                                              const __bf16* __restrict__ w, __bf16* __restrict__ h_out,
                                                              __bf16* __restrict__ n_out, int dim, float eps) {
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int per = dim / 256;
  const int64_t base = row * dim + (int64_t)t * per;
  auto hval = [&](int e) {
    float v = (float)x[base + e];
    if (y != nullptr) v = (float)(__bf16)(v + (float)y[base + e]);
    return v;
  };
  float ss = 0.f;
  for (int e = 0; e < per; ++e) {
    const float v = hval(e);
    if (y != nullptr && h_out != nullptr) h_out[base + e] = (__bf16)v;
    ss = fmaf(v, v, ss);
  }
  ss = dec_wave_sum64(ss);
  __shared__ float part[4];
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = rsqrtf(tot / (float)dim + eps);
  for (int e = 0; e < per; ++e) n_out[base + e] = (__bf16)(hval(e) * r * (float)w[t * per + e]);
}

// One workgroup of 256 threads per row; each thread holds `PER` consecutive
// elements (dim = 256 * PER).
// kVec: every pointer is 16-byte aligned and PER a multiple of 8, so each
// thread moves its elements as 16-byte pieces.
template <int PER, bool kVec>
__global__ void __launch_bounds__(256) add_rmsnorm_kernel(const __bf16* __restrict__ x, const __bf16* __restrict__ y,
                                                          const __bf16* __restrict__ w, __bf16* __restrict__ h_out,
                                                          __bf16* __restrict__ n_out, int dim, float eps) {
  const int64_t row = (int64_t)blockIdx.x * dim;
  __shared__ float part[4];
  add_rmsnorm_row<PER, kVec>(x + row, y != nullptr ? y + row : nullptr, w, h_out != nullptr ? h_out + row : nullptr,
                             n_out + row, dim, eps, (int)threadIdx.x, true, part);
}

// One wave per (row of B*T, head): q/k heads are normed over d with their weight,
// rounded to bf16, rotated with cos/sin of the row's position, rounded to bf16 and
// written heads-first; v heads are only moved.  Lane l holds elements l and
// l + d/2, the two halves rotate-half pairs.
template <int D>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const __bf16* __restrict__ q, const __bf16* __restrict__ k,
                                                           const __bf16* __restrict__ v, const __bf16* __restrict__ qw,
                                                           const __bf16* __restrict__ kw, const float* __restrict__ cosv,
                                                           const float* __restrict__ sinv, __bf16* __restrict__ qo,
                                                           __bf16* __restrict__ ko, __bf16* __restrict__ vo, int64_t rows,
                                                           int t_len, int hq, int hkv, int64_t sq, int64_t sk,
                                                           int64_t sv, float eps) {
  constexpr int HALF = D / 2;
  constexpr int PER = HALF / 64;   // elements per lane in each half
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nh = hq + 2 * hkv;
  if (item >= rows * nh) return;
  const int64_t row = item / nh;                  // b * T + t
  const int head = (int)(item - row * nh);
  const int64_t b = row / t_len;
  const int tt = (int)(row - b * t_len);
  const __bf16* src;
  __bf16* dst;
  const __bf16* w = nullptr;
  if (head < hq) {
    src = q + row * sq + (int64_t)head * D;
    dst = qo + ((b * hq + head) * t_len + tt) * D;
    w = qw;
  } else if (head < hq + hkv) {
    const int hk = head - hq;
    src = k + row * sk + (int64_t)hk * D;
    dst = ko + ((b * hkv + hk) * t_len + tt) * D;
    w = kw;
  } else {
    const int hv = head - hq - hkv;
    src = v + row * sv + (int64_t)hv * D;
    dst = vo + ((b * hkv + hv) * t_len + tt) * D;
  }
  float lo[PER], hi[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    lo[e] = (float)src[lane * PER + e];
    hi[e] = (float)src[HALF + lane * PER + e];
  }
  if (w == nullptr) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      dst[lane * PER + e] = (__bf16)lo[e];
      dst[HALF + lane * PER + e] = (__bf16)hi[e];
    }
    return;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) ss = fmaf(lo[e], lo[e], fmaf(hi[e], hi[e], ss));
  ss = dec_wave_sum64(ss);
  const float r = rsqrtf(ss / (float)D + eps);
  const float* c = cosv + (int64_t)tt * D;
  const float* s = sinv + (int64_t)tt * D;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int i = lane * PER + e;
    const float a = (float)(__bf16)(lo[e] * r * (float)w[i]);            // normed, rounded as the module does
    const float bb = (float)(__bf16)(hi[e] * r * (float)w[HALF + i]);
    dst[i] = (__bf16)(a * c[i] + (-bb) * s[i]);                         // x*cos + rotate_half(x)*sin
    dst[HALF + i] = (__bf16)(bb * c[HALF + i] + a * s[HALF + i]);
  }
}

// The same step with 16-byte accesses: a group of HALF / 8 lanes per (row,
// head) item, lane j of the group holding elements [8j, 8j + 8) of both halves
// (the rotate-half partners).  Same rounding points; the sum of squares runs
// over the group with shuffles.  Needs 16-byte aligned rows (strides multiples
// of 8, aligned base pointers).
template <int D>
__global__ void __launch_bounds__(256) qk_norm_rope_vec_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ qw, const __bf16* __restrict__ kw, const float* __restrict__ cosv,
    const float* __restrict__ sinv, __bf16* __restrict__ qo, __bf16* __restrict__ ko, __bf16* __restrict__ vo,
    int64_t rows, int t_len, int hq, int hkv, int64_t sq, int64_t sk, int64_t sv, float eps) {
  constexpr int HALF = D / 2;
  constexpr int G = HALF / 8;    // lanes per item: 8 (d = 128) or 16 (d = 256)
  const int gl = threadIdx.x % G;
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) / G;
  const int nh = hq + 2 * hkv;
  if (item >= rows * nh) return;   // whole groups: items are group-uniform
  const int64_t row = item / nh;   // b * T + t
  const int head = (int)(item - row * nh);
  const int64_t b = row / t_len;
  const int tt = (int)(row - b * t_len);
  const __bf16* src;
  __bf16* dst;
  const __bf16* w = nullptr;
  if (head < hq) {
    src = q + row * sq + (int64_t)head * D;
    dst = qo + ((b * hq + head) * t_len + tt) * D;
    w = qw;
  } else if (head < hq + hkv) {
    const int hk = head - hq;
    src = k + row * sk + (int64_t)hk * D;
    dst = ko + ((b * hkv + hk) * t_len + tt) * D;
    w = kw;
  } else {
    const int hv = head - hq - hkv;
    src = v + row * sv + (int64_t)hv * D;
    dst = vo + ((b * hkv + hv) * t_len + tt) * D;
  }
  const int i0 = 8 * gl;
  const bf16x8 lov = *reinterpret_cast<const bf16x8*>(src + i0);
  const bf16x8 hiv = *reinterpret_cast<const bf16x8*>(src + HALF + i0);
  if (w == nullptr) {
    *reinterpret_cast<bf16x8*>(dst + i0) = lov;
    *reinterpret_cast<bf16x8*>(dst + HALF + i0) = hiv;
    return;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf((float)lov[e], (float)lov[e], fmaf((float)hiv[e], (float)hiv[e], ss));
#pragma unroll
  for (int o = 1; o < G; o <<= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss / (float)D + eps);
  const bf16x8 wlo = *reinterpret_cast<const bf16x8*>(w + i0);
  const bf16x8 whi = *reinterpret_cast<const bf16x8*>(w + HALF + i0);
  const float* c = cosv + (int64_t)tt * D;
  const float* sn = sinv + (int64_t)tt * D;
  float clo[8], chi[8], slo[8], shi[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float4 a = *reinterpret_cast<const float4*>(c + i0 + 4 * h);
    const float4 bq = *reinterpret_cast<const float4*>(c + HALF + i0 + 4 * h);
    const float4 cc = *reinterpret_cast<const float4*>(sn + i0 + 4 * h);
    const float4 d = *reinterpret_cast<const float4*>(sn + HALF + i0 + 4 * h);
    clo[4 * h] = a.x; clo[4 * h + 1] = a.y; clo[4 * h + 2] = a.z; clo[4 * h + 3] = a.w;
    chi[4 * h] = bq.x; chi[4 * h + 1] = bq.y; chi[4 * h + 2] = bq.z; chi[4 * h + 3] = bq.w;
    slo[4 * h] = cc.x; slo[4 * h + 1] = cc.y; slo[4 * h + 2] = cc.z; slo[4 * h + 3] = cc.w;
    shi[4 * h] = d.x; shi[4 * h + 1] = d.y; shi[4 * h + 2] = d.z; shi[4 * h + 3] = d.w;
  }
  bf16x8 olo, ohi;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = (float)(__bf16)((float)lov[e] * r * (float)wlo[e]);    // normed, rounded as the module does
    const float bb = (float)(__bf16)((float)hiv[e] * r * (float)whi[e]);
    olo[e] = (__bf16)(a * clo[e] + (-bb) * slo[e]);                        // x*cos + rotate_half(x)*sin
    ohi[e] = (__bf16)(bb * chi[e] + a * shi[e]);
  }
  *reinterpret_cast<bf16x8*>(dst + i0) = olo;
  *reinterpret_cast<bf16x8*>(dst + HALF + i0) = ohi;
}

// rows x cols elements; gate and up rows are `stride` elements apart (a fused
// gate|up projection output has stride 2 * cols), out is contiguous.  The
// vector form moves 8 consecutive elements of a row per thread (cols and
// stride multiples of 8, pointers 16-byte aligned), with the same arithmetic.
__global__ void __launch_bounds__(256) silu_mul_vec_kernel(const __bf16* __restrict__ g, const __bf16* __restrict__ u,
                                                           __bf16* __restrict__ out, int64_t cols8, int64_t stride8,
                                                           int64_t n8) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int64_t r = i / cols8, c = i - r * cols8;
  const bf16x8 gv = reinterpret_cast<const bf16x8*>(g)[r * stride8 + c];
  const bf16x8 uv = reinterpret_cast<const bf16x8*>(u)[r * stride8 + c];
  bf16x8 ov;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = (float)gv[e];
    const float sg = (float)(__bf16)(x / (1.f + expf(-x)));
    ov[e] = (__bf16)(sg * (float)uv[e]);
  }
  reinterpret_cast<bf16x8*>(out)[i] = ov;
}

__global__ void __launch_bounds__(256) silu_mul_kernel(const __bf16* __restrict__ g, const __bf16* __restrict__ u,
                                                       __bf16* __restrict__ out, int64_t cols, int64_t stride,
                                                       int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = i / cols, c = i - r * cols;
  const float x = (float)g[r * stride + c];
  const float sg = (float)(__bf16)(x / (1.f + expf(-x)));
  out[i] = (__bf16)(sg * (float)u[r * stride + c]);
}

}  // namespace bfly

using namespace bfly;

extern "C" int bfly_add_rms_norm(const void* x, const void* residual, const void* weight, int64_t rows, int dim,
                                 float eps, void* h_out, void* norm_out, hipStream_t stream) {
  BFLY_CHECK_ARG(x && weight && norm_out, "null pointer");
  BFLY_CHECK_ARG((residual == nullptr) == (h_out == nullptr), "residual and h_out must both be given or both NULL");
  BFLY_CHECK_ARG(rows > 0 && rows <= INT32_MAX, "rows=%lld out of range", (long long)rows);
  BFLY_CHECK_ARG(dim > 0 && dim % 256 == 0 && dim <= 256 * 32, "dim=%d must be a multiple of 256 up to 8192", dim);
  const __bf16* xp = static_cast<const __bf16*>(x);
  const __bf16* yp = static_cast<const __bf16*>(residual);
  const __bf16* wp = static_cast<const __bf16*>(weight);
  __bf16* hp = static_cast<__bf16*>(h_out);
  __bf16* np = static_cast<__bf16*>(norm_out);
  dim3 grid((unsigned)rows);
  const bool vec = aligned16(x) && aligned16(residual) && aligned16(weight) && aligned16(h_out) && aligned16(norm_out);
#define BFLY_ADD_RMS(P)                                                                                    \
  if (vec)                                                                                                 \
    hipLaunchKernelGGL((add_rmsnorm_kernel<P, true>), grid, dim3(256), 0, stream, xp, yp, wp, hp, np, dim, eps); \
  else                                                                                                     \
    hipLaunchKernelGGL((add_rmsnorm_kernel<P, false>), grid, dim3(256), 0, stream, xp, yp, wp, hp, np, dim, eps);
  switch (dim / 256) {
    case 4: hipLaunchKernelGGL((add_rmsnorm_kernel<4, false>), grid, dim3(256), 0, stream, xp, yp, wp, hp, np, dim, eps); break;
    case 8: BFLY_ADD_RMS(8) break;
    case 16: BFLY_ADD_RMS(16) break;
    case 24: BFLY_ADD_RMS(24) break;
    case 32: BFLY_ADD_RMS(32) break;
    default: hipLaunchKernelGGL(add_rmsnorm_any_kernel, grid, dim3(256), 0, stream, xp, yp, wp, hp, np, dim, eps); break;
  }
#undef BFLY_ADD_RMS
  BFLY_CHECK_LAUNCH("bfly_add_rms_norm");
  return BFLY_OK;
}

extern "C" int bfly_qk_norm_rope(const void* q, const void* k, const void* v, int64_t q_row_stride,
                                 int64_t k_row_stride, int64_t v_row_stride, const void* q_weight,
                                 const void* k_weight, const float* cos, const float* sin, int64_t batch,
                                 int64_t seq_len, int hq, int hkv, int head_dim, float eps, void* q_out, void* k_out,
                                 void* v_out, hipStream_t stream) {
  BFLY_CHECK_ARG(q && k && v && q_weight && k_weight && cos && sin && q_out && k_out && v_out, "null pointer");
  BFLY_CHECK_ARG(batch > 0 && seq_len > 0 && hq > 0 && hkv > 0, "bad shape");
  BFLY_CHECK_ARG(head_dim == 128 || head_dim == 256, "bfly_qk_norm_rope: head_dim=%d unsupported (128, 256)",
                 head_dim);
  BFLY_CHECK_ARG(q_row_stride >= (int64_t)hq * head_dim && k_row_stride >= (int64_t)hkv * head_dim &&
                     v_row_stride >= (int64_t)hkv * head_dim,
                 "row strides must cover a row's heads");
  const int64_t rows = batch * seq_len;
  const int64_t items = rows * (hq + 2 * hkv);
  BFLY_CHECK_ARG((items + 3) / 4 <= INT32_MAX && seq_len <= INT32_MAX, "too many rows");
  dim3 grid((unsigned)((items + 3) / 4));
  const __bf16 *qp = static_cast<const __bf16*>(q), *kp = static_cast<const __bf16*>(k),
               *vp = static_cast<const __bf16*>(v), *qw = static_cast<const __bf16*>(q_weight),
               *kw = static_cast<const __bf16*>(k_weight);
  __bf16 *qo = static_cast<__bf16*>(q_out), *ko = static_cast<__bf16*>(k_out), *vo = static_cast<__bf16*>(v_out);
  const bool vec = q_row_stride % 8 == 0 && k_row_stride % 8 == 0 && v_row_stride % 8 == 0 && aligned16(q) &&
                   aligned16(k) && aligned16(v) && aligned16(q_weight) && aligned16(k_weight) && aligned16(cos) &&
                   aligned16(sin) && aligned16(q_out) && aligned16(k_out) && aligned16(v_out);
  if (vec) {
    const int64_t threads = items * (head_dim / 16);
    BFLY_CHECK_ARG((threads + 255) / 256 <= INT32_MAX, "too many rows");
    dim3 vgrid((unsigned)((threads + 255) / 256));
    if (head_dim == 128)
      hipLaunchKernelGGL(qk_norm_rope_vec_kernel<128>, vgrid, dim3(256), 0, stream, qp, kp, vp, qw, kw, cos, sin, qo,
                         ko, vo, rows, (int)seq_len, hq, hkv, q_row_stride, k_row_stride, v_row_stride, eps);
    else
      hipLaunchKernelGGL(qk_norm_rope_vec_kernel<256>, vgrid, dim3(256), 0, stream, qp, kp, vp, qw, kw, cos, sin, qo,
                         ko, vo, rows, (int)seq_len, hq, hkv, q_row_stride, k_row_stride, v_row_stride, eps);
  } else if (head_dim == 128)
    hipLaunchKernelGGL(qk_norm_rope_kernel<128>, grid, dim3(256), 0, stream, qp, kp, vp, qw, kw, cos, sin, qo, ko, vo,
                       rows, (int)seq_len, hq, hkv, q_row_stride, k_row_stride, v_row_stride, eps);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<256>, grid, dim3(256), 0, stream, qp, kp, vp, qw, kw, cos, sin, qo, ko, vo,
                       rows, (int)seq_len, hq, hkv, q_row_stride, k_row_stride, v_row_stride, eps);
  BFLY_CHECK_LAUNCH("bfly_qk_norm_rope");
  return BFLY_OK;
}

extern "C" int bfly_silu_mul(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t in_row_stride,
                             void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(gate && up && out, "null pointer");
  BFLY_CHECK_ARG(rows > 0 && cols > 0 && in_row_stride >= cols, "bad shape");
  const int64_t n = rows * cols;
  BFLY_CHECK_ARG((n + 255) / 256 <= INT32_MAX, "bad length");
  if (cols % 8 == 0 && in_row_stride % 8 == 0 && aligned16(gate) && aligned16(up) && aligned16(out)) {
    const int64_t n8 = n / 8;
    hipLaunchKernelGGL(silu_mul_vec_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const __bf16*>(gate), static_cast<const __bf16*>(up), static_cast<__bf16*>(out),
                       cols / 8, in_row_stride / 8, n8);
  } else {
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const __bf16*>(gate), static_cast<const __bf16*>(up), static_cast<__bf16*>(out),
                       cols, in_row_stride, n);
  }
  BFLY_CHECK_LAUNCH("bfly_silu_mul");
  return BFLY_OK;
}

namespace bfly {

// Pass 1: workgroup (p, r) scans elements [p * span, (p + 1) * span) of row r
// (span a multiple of 8) and leaves its candidate in part_v / part_i [r * parts + p],
// or, with a single part, the answer in out[r].  Rows that are contiguous with a
// 16-byte aligned start are read 8 elements per load.
__global__ void __launch_bounds__(256) argmax_part_kernel(const __bf16* __restrict__ x, int64_t n, int64_t row_stride,
                                                          int64_t col_stride, bool vec, int64_t span, int parts,
                                                          float* __restrict__ part_v, int64_t* __restrict__ part_i,
                                                          int64_t* __restrict__ out) {
  const int p = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const __bf16* row = x + (int64_t)r * row_stride;
  const int64_t lo = (int64_t)p * span, hi = lo + span < n ? lo + span : n;
  float bv = 0.f;
  int64_t bi = -1;
  if (vec) {
    const int64_t c_lo = lo >> 3, c_hi = hi >> 3;  // whole 8-element pieces; lo is a multiple of 8
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll 2
    for (int64_t c = c_lo + t; c < c_hi; c += 256) {
      const uint4 u = r4[c];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = __uint_as_float((j & 1) ? (w[j >> 1] & 0xffff0000u) : (w[j >> 1] << 16));
        argmax_combine(bv, bi, v, c * 8 + j);
      }
    }
    for (int64_t i = (c_hi << 3) + t; i < hi; i += 256) argmax_combine(bv, bi, (float)row[i], i);
  } else {
#pragma unroll 4
    for (int64_t i = lo + t; i < hi; i += 256) argmax_combine(bv, bi, (float)row[i * col_stride], i);
  }
  argmax_block(bv, bi);
  if (t == 0) {
    if (parts == 1) {
      out[r] = bi;
    } else {
      part_v[(int64_t)r * parts + p] = bv;
      part_i[(int64_t)r * parts + p] = bi;
    }
  }
}

// Pass 2: one workgroup per row combines its `parts` (at most 256) candidates.
__global__ void __launch_bounds__(256) argmax_final_kernel(const float* __restrict__ part_v,
                                                           const int64_t* __restrict__ part_i, int parts,
                                                           int64_t* __restrict__ out) {
  const int r = blockIdx.x, t = threadIdx.x;
  float bv = 0.f;
  int64_t bi = -1;
  if (t < parts) {
    bv = part_v[(int64_t)r * parts + t];
    bi = part_i[(int64_t)r * parts + t];
  }
  argmax_block(bv, bi);
  if (t == 0) out[r] = bi;
}

// bfly_greedy_advance: the greedy pick over the per-workgroup candidates a product left in
// its workspace (bfly_add_rms_norm_q4_gemv_argmax: an int64 count at byte 0, then
// kGreedyMaxCand 64-bit argmax_key candidates from byte 16), and a decode loop's bookkeeping for
// the token: token[0], tokens_out[counters[1]] (while below tokens_cap), both counters + 1, and
// the next step's input row x_next = embed[token] (hidden bf16).  Every slot is requested with
// the count (slots past it are dropped), so the pick waits for one round trip.  One workgroup.
constexpr int kGreedyMaxCand = 1024;
__global__ void __launch_bounds__(256) greedy_advance_kernel(const unsigned char* __restrict__ ws,
                                                             const __bf16* __restrict__ embed, int64_t vocab,
                                                             int64_t hidden, __bf16* __restrict__ x_next,
                                                             int64_t* __restrict__ token,
                                                             int64_t* __restrict__ tokens_out, int64_t tokens_cap,
                                                             int64_t* __restrict__ counters) {
  const int t = threadIdx.x;
  const int64_t g = *reinterpret_cast<const int64_t*>(ws);
  const uint64_t* cand = reinterpret_cast<const uint64_t*>(ws + 16);
  uint64_t c[kGreedyMaxCand / 256];
#pragma unroll
  for (int k = 0; k < kGreedyMaxCand / 256; ++k) c[k] = cand[t + 256 * k];
  uint64_t best = 0;
#pragma unroll
  for (int k = 0; k < kGreedyMaxCand / 256; ++k)
    if (t + 256 * k < g && c[k] > best) best = c[k];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t ob = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), o) << 32) |
                        (uint32_t)__shfl_xor((int)(uint32_t)best, o);
    best = ob > best ? ob : best;
  }
  __shared__ uint64_t wb[4];
  __shared__ int64_t tok_s;
  if ((t & 63) == 0) wb[t >> 6] = best;
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) best = wb[w] > best ? wb[w] : best;
    const int64_t bi = best != 0 ? argmax_key_index(best) : -1;
    tok_s = bi;
    token[0] = bi;
    const int64_t col = counters[1];
    if (col >= 0 && col < tokens_cap) tokens_out[col] = bi;
    counters[0] += 1;
    counters[1] += 1;
  }
  __syncthreads();
  const int64_t tk = tok_s;
  if (tk < 0 || tk >= vocab) return;
  const uint4* src = reinterpret_cast<const uint4*>(embed + tk * hidden);
  for (int64_t c8 = t; c8 < hidden / 8; c8 += 256) reinterpret_cast<uint4*>(x_next)[c8] = src[c8];
}

}  // namespace bfly

extern "C" int bfly_greedy_advance(const void* workspace, int64_t workspace_bytes, const void* embed, int64_t vocab,
                                   int64_t hidden, void* x_next, int64_t* token, int64_t* tokens_out,
                                   int64_t tokens_cap, int64_t* counters, hipStream_t stream) {
  BFLY_CHECK_ARG(workspace && embed && x_next && token && tokens_out && counters, "null pointer");
  BFLY_CHECK_ARG(workspace_bytes >= 16 + 8 * (int64_t)bfly::kGreedyMaxCand,
                 "workspace_bytes=%lld: the candidate workspace holds %lld bytes (bfly_q4_argmax_workspace_bytes)",
                 (long long)workspace_bytes, (long long)(16 + 8 * (int64_t)bfly::kGreedyMaxCand));
  BFLY_CHECK_ARG(vocab > 0 && hidden > 0 && hidden % 8 == 0 && tokens_cap > 0, "bad shape");
  BFLY_CHECK_ARG(aligned16(workspace) && aligned16(embed) && aligned16(x_next),
                 "workspace, embed and x_next must be 16-byte aligned");
  hipLaunchKernelGGL(bfly::greedy_advance_kernel, dim3(1), dim3(256), 0, stream,
                     static_cast<const unsigned char*>(workspace), static_cast<const __bf16*>(embed), vocab, hidden,
                     static_cast<__bf16*>(x_next), token, tokens_out, tokens_cap, counters);
  BFLY_CHECK_LAUNCH("bfly_greedy_advance");
  return BFLY_OK;
}

// The two passes of bfly_argmax_rows over a workspace the caller checked.
static int argmax_launch(const void* x, int64_t rows, int64_t n, int64_t row_stride, int64_t col_stride,
                         void* workspace, int64_t workspace_bytes, void* out, hipStream_t stream, const char* what) {
  if (rows == 1) row_stride = 0;  // a single row: its stride is never used (a [1, n] view may carry any)
  const bool vec = col_stride == 1 && row_stride % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  // about 4096 elements per workgroup, at most 256 parts, as many as the workspace holds
  int64_t parts = (n + 4095) / 4096;
  if (parts > 256) parts = 256;
  // part_v (rows * parts floats), padding to 8 bytes, part_i (rows * parts int64)
  const int64_t fit = reinterpret_cast<uintptr_t>(workspace) % 8 == 0 && workspace_bytes >= 8
                          ? (workspace_bytes - 4) / (rows * (int64_t)(sizeof(float) + sizeof(int64_t)))
                          : 0;
  if (parts > fit) parts = fit > 1 ? fit : 1;
  const int64_t span = ((n + parts - 1) / parts + 7) / 8 * 8;
  float* part_v = static_cast<float*>(workspace);
  int64_t* part_i = parts > 1 ? reinterpret_cast<int64_t*>(part_v + rows * parts + (rows * parts & 1)) : nullptr;
  hipLaunchKernelGGL(bfly::argmax_part_kernel, dim3((unsigned)parts, (unsigned)rows), dim3(256), 0, stream,
                     static_cast<const __bf16*>(x), n, row_stride, col_stride, vec, span, (int)parts, part_v, part_i,
                     static_cast<int64_t*>(out));
  if (parts > 1)
    hipLaunchKernelGGL(bfly::argmax_final_kernel, dim3((unsigned)rows), dim3(256), 0, stream, part_v, part_i,
                       (int)parts, static_cast<int64_t*>(out));
  BFLY_CHECK_LAUNCH(what);
  return BFLY_OK;
}

extern "C" int bfly_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t row_stride, int64_t col_stride,
                                void* workspace, int64_t workspace_bytes, void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(x && out, "null pointer");
  BFLY_CHECK_ARG(rows > 0 && rows <= 65535 && n > 0 && col_stride > 0 && row_stride >= 0, "bad shape");
  BFLY_CHECK_ARG(workspace_bytes >= 0 && (workspace != nullptr || workspace_bytes == 0), "bad workspace");
  return argmax_launch(x, rows, n, row_stride, col_stride, workspace, workspace_bytes, out, stream,
                       "bfly_argmax_rows");
}

// ---------------------------------------------------------------------------------------------
// bfly_argmax_rows_noalloc: the same passes with the per-workgroup candidates in a
// file-scope device array instead of a caller workspace, for callers that cannot
// allocate.  Every GPU the library runs on holds its own copy of `scratch` until the
// process ends; calls on one GPU share it, so calls that overlap on one GPU (another
// stream, another thread) race.  Pass 1 writes every candidate slot that pass 2 reads,
// so nothing needs clearing between calls.
constexpr int64_t kNoAllocMaxRows = 64;
// rows * 256 parts * (float + int64) + 8 bytes of alignment padding
constexpr int64_t kNoAllocScratchBytes = kNoAllocMaxRows * 256 * 12 + 8;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kNoAllocMaxDevices] = {};   // device address of `scratch`, per device

// The device address of the current device's copy of `scratch`, looked up once per device
// (host code never passes the array's own name to a kernel: that is a host-side stand-in).
int scratch_address(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    ::bfly::set_error("bfly_argmax_rows_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return BFLY_ERR_HIP;
  }
  if (dev < 0 || dev >= kNoAllocMaxDevices) {
    ::bfly::set_error("bfly_argmax_rows_noalloc: device %d outside the %d it tracks", dev, kNoAllocMaxDevices);
    return BFLY_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      ::bfly::set_error("bfly_argmax_rows_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return BFLY_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return BFLY_OK;
}

}  // namespace

extern "C" int bfly_argmax_rows_noalloc(const void* x, int64_t rows, int64_t n, int64_t row_stride,
                                        int64_t col_stride, void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(x && out, "null pointer");
  BFLY_CHECK_ARG(rows > 0 && n > 0 && col_stride > 0 && row_stride >= 0, "bad shape");
  BFLY_CHECK_ARG(rows <= kNoAllocMaxRows,
                 "bfly_argmax_rows_noalloc: rows=%lld above the %lld its static workspace holds; "
                 "use bfly_argmax_rows with a workspace", (long long)rows, (long long)kNoAllocMaxRows);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != BFLY_OK) return rc;
  return argmax_launch(x, rows, n, row_stride, col_stride, ws, kNoAllocScratchBytes, out, stream,
                       "bfly_argmax_rows_noalloc");
}
