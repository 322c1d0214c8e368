// One-row projections over 4-bit affine weights on gfx950 (a decode step at
// batch 1): y = W x, with W stored as two 4-bit codes per byte (low nibble
// first) and one bf16 (scale, bias) pair per group of G codes along the input
// dimension, w = code * scale + bias.
//
// Reference: the swapped decoder's projections are quantized linear layers with
// 4-bit affine weights, group 64, bf16 scales and biases
// (bna/integrations/qwen_mlx.py:1115-1157 builds them as mlx.nn.QuantizedLinear
// with weight / scales / biases).  The product is taken group by group in the
// factorised form of w = code * scale + bias:
//   y_n = sum_g ( scale_ng * sum_{i in g} x_i code_ni + bias_ng * sum_{i in g} x_i ),
// so the kernel streams half a byte per weight and never expands W in memory.
// fp32 throughout; y is rounded once to bf16.  The results equal the product
// with the fp32 weights code * scale + bias up to the fp32 summation order.
#include "bfly_common.h"
#include "argmax.h"
#include "q4_piece.h"
#include "rmsnorm_row.h"
#include "../../include/butterfly_amd_decoder.h"

namespace bfly {

constexpr int kQ4MaxPieces = 4;        // pieces per lane: in_features <= 64 * 4 * 32 = 8192
constexpr int64_t kQ4MaxWaves = 8192;  // grid cap; the waves stride over the row sets

// SiLU(gate) * up with the rounding points of the separate steps: the projection
// outputs are bf16, SiLU is rounded to bf16, then the product (the formula of
// decoder_ops.hip's silu_mul kernels).
__device__ __forceinline__ __bf16 q4_silu_times(float g, float u) {
#pragma clang fp contract(off)
  const float x = (float)(__bf16)g;
  const float sg = (float)(__bf16)(x / (1.f + expf(-x)));
  return (__bf16)(sg * (float)(__bf16)u);
}

// x: in_features bf16.  w: [rows][pieces] 16-byte pieces.  sb: [rows][groups]
// words, bf16 scale in the low half and bf16 bias in the high half.
// One wave per row set at a time (the grid strides over the sets).  A set is R
// rows, or with kSilu R/2 gate rows and the R/2 up rows up_off further.  Lane l
// owns the pieces p = l + 64 j (j < NP) of every row; each piece lies in one
// group, so a lane needs one (scale, bias) word per piece.  The lane's x values
// stay in registers for all its sets, the odd (high-nibble) ones divided by 16:
// masking the high nibbles in place gives 16 * code, and (x / 16) * (16 * code)
// is x * code exactly.
struct Q4Args {
  const __bf16* x;
  const u32x4* w;
  const uint32_t* sb;
  __bf16* y;
  int64_t n_sets, n_out, up_off;
  int pieces, groups, pieces_per_group;
};

struct Q4NoSink {
  __device__ void operator()(int64_t, __bf16) const {}
};

// The sets of one wave: set0, set0 + stride, ... < n_sets.  form_x() runs after the first
// set's weights are requested and before x (xsrc, bf16) is read: the fused form computes x
// there.  kXFirst (x already in memory): x is requested before the weights, so that its
// pre-sums wait for x alone.  sink(o, y) sees every output the lane writes.
template <int NP, int R, bool kSilu, bool kXFirst, class XPtr, class FormX, class Sink = Q4NoSink>
__device__ __forceinline__ void q4_sets(const Q4Args& a, int lane, int64_t set0, int64_t stride, XPtr xsrc,
                                        FormX&& form_x, Sink&& sink = Sink{}) {
  const int pieces = a.pieces, groups = a.groups;
  const u32x4* __restrict__ w = a.w;
  const uint32_t* __restrict__ sb = a.sb;
  constexpr int OUTS = kSilu ? R / 2 : R;   // outputs per set
  const int64_t n_out = a.n_out;
  float xq[NP][kQ4PieceCodes];
  float xs[NP];
  int pc[NP], gi[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int p = lane + 64 * j;
    pc[j] = p < pieces ? p : 0;   // a lane past the row reads piece 0 and weighs it by zeros
    gi[j] = pc[j] / a.pieces_per_group;
  }
  // The weights of a set are requested one set ahead: the first set's before the
  // row is formed, the next set's before the current one is reduced.
  u32x4 wv[R][NP];
  uint32_t sv[R][NP];
  auto load_set = [&](int64_t set) {
    const int64_t o0 = set * OUTS;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t o = o0 + (kSilu ? r % OUTS : r);
      const int64_t row = (o < n_out ? o : 0) + (kSilu && r >= OUTS ? a.up_off : 0);
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        wv[r][j] = __builtin_nontemporal_load(w + row * pieces + pc[j]);
        sv[r][j] = sb[row * groups + gi[j]];
      }
    }
  };
  // issued on every path (a wave past the sets loads set 0 and drops it): behind a branch, the
  // wait in form_x() for loads issued before these would count as on the path without them
  // and wait for these too
  bf16x8 xr[NP][4];
  auto read_x = [&] {
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[j][c] = xsrc[(int64_t)pc[j] * 4 + c];
  };
  if constexpr (kXFirst) {
    // returned from before any load: the weights, used after a later return, would be sunk
    // behind it and x's pre-sums
    if (set0 >= a.n_sets) return;
    read_x();
    __builtin_amdgcn_sched_barrier(0);
  }
  load_set(set0 < a.n_sets ? set0 : 0);
  // the scheduler keeps the order: x's requests, the weights', then x's pre-sums (it would
  // hoist the pre-sums above the weights, which then were requested only after x arrived)
  if constexpr (kXFirst) __builtin_amdgcn_sched_barrier(0);
  form_x();
  if constexpr (!kXFirst) {
    if (set0 >= a.n_sets) return;
    read_x();
  }

#pragma unroll
  for (int j = 0; j < NP; ++j) q4_piece_x(xr[j], lane + 64 * j < pieces, xq[j], xs[j]);

  for (int64_t set = set0; set < a.n_sets; set += stride) {
    const int64_t o0 = set * OUTS;
    float tot[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NP; ++j) acc += q4_piece_dot(wv[r][j], sv[r][j], xq[j], xs[j]);
      tot[r] = acc;
    }
    if (set + stride < a.n_sets) load_set(set + stride);
#pragma unroll
    for (int r = 0; r < R; ++r) tot[r] = q4_wave_sum(tot[r]);
    float mine = 0.f, mate = 0.f;
#pragma unroll
    for (int r = 0; r < OUTS; ++r) {
      if (lane == r) {
        mine = tot[r];
        if constexpr (kSilu) mate = tot[r + OUTS];
      }
    }
    const int64_t o = o0 + lane;
    if (lane < OUTS && o < n_out) {
      const __bf16 yv = kSilu ? q4_silu_times(mine, mate) : (__bf16)mine;
      a.y[o] = yv;
      sink(o, yv);
    }
  }
}

template <int NP, int R, bool kSilu>
__global__ void __launch_bounds__(64) q4_gemv_kernel(Q4Args a) {
  q4_sets<NP, R, kSilu, true>(a, (int)threadIdx.x, blockIdx.x, gridDim.x, reinterpret_cast<const bf16x8*>(a.x),
                              [] {});
}

// The residual add + RMSNorm of the input row inside the product: NW waves (8 or 12);
// threads 0..255 form h = x + residual and its normed row exactly as bfly_add_rms_norm does
// (into LDS; workgroup 0 also writes h), then each of the NW waves runs its sets on that row.
// in_features = 256 PER.  kParts: x is not given as a row but as four fp32 partial rows
// (parts[g * in_features + i]), and x_i = bf16((p0_i + p1_i) + (p2_i + p3_i)) -- the
// rounding of a product whose four 16-piece partials are combined by q4_wave_sum.
// One greedy candidate (argmax_key of the best output) per workgroup.
constexpr int kQ4MaxCand = (int)(kQ4MaxWaves / 8);   // workgroups of at least 8 waves

struct Q4NormArgs {
  const __bf16* x;
  const __bf16* residual;   // or null (then h_out is null: a plain RMSNorm)
  const __bf16* weight;
  __bf16* h_out;
  float eps;
  const float* parts;       // kParts: the four partial rows
  uint64_t* cand;           // kArgmax: one greedy candidate key per workgroup
  int64_t* cand_n;          // kArgmax: the candidate count (the grid), written by workgroup 0
};

template <int NP, int R, bool kSilu, int PER, int NW, bool kParts, bool kArgmax = false>
__global__ void __launch_bounds__(64 * NW) q4_norm_gemv_kernel(Q4Args a, Q4NormArgs nm) {
  static_assert(NW >= 4, "the row is formed by the first 256 threads");
  constexpr int DIM = 256 * PER;
  __shared__ __attribute__((aligned(16))) __bf16 xn[DIM];
  __shared__ float part[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t waves = (int64_t)gridDim.x * NW;
  uint64_t bk = 0;     // kArgmax: this lane's greedy candidate (argmax_key; 0 = none)
  __shared__ unsigned long long wg_key;
  __shared__ unsigned int wg_done;
  if constexpr (kArgmax) {
    if (tid == 0) {   // ordered before every wave's use by the norm's barriers
      wg_key = 0;
      wg_done = 0;
    }
  }
  // the norm's inputs are requested before the weights, so that forming the row waits for them
  // alone and runs while the weights are in flight
  RmsRowIn<PER> in = rms_row_load<PER, !kParts>(nm.x, nm.residual, nm.weight, tid, tid < 256);
  f32x4 pp[kParts ? 4 : 1][kParts ? PER / 4 : 1];
  if constexpr (kParts) {
    if (tid < 256) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int c = 0; c < PER / 4; ++c)
          pp[g][c] = *reinterpret_cast<const f32x4*>(nm.parts + (int64_t)g * DIM + (int64_t)tid * PER + 4 * c);
    }
  }
  q4_sets<NP, R, kSilu, false>(a, lane, (int64_t)blockIdx.x * NW + wave, waves, reinterpret_cast<const bf16x8*>(xn), [&] {
    if constexpr (kParts) {
#pragma unroll
      for (int c = 0; c < PER / 8; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * c + e;
          in.x[c][e] = (__bf16)((pp[0][i / 4][i % 4] + pp[1][i / 4][i % 4]) + (pp[2][i / 4][i % 4] + pp[3][i / 4][i % 4]));
        }
    }
    add_rmsnorm_row_from<PER>(in, nm.residual != nullptr, blockIdx.x == 0 ? nm.h_out : nullptr, xn, DIM, nm.eps, tid,
                              tid < 256, part);
    __syncthreads();   // the normed row is in LDS
  }, [&](int64_t o, __bf16 yv) {
    if constexpr (kArgmax) {
      const uint64_t k = argmax_key((float)yv, (uint32_t)o);
      bk = k > bk ? k : bk;
    }
  });
  if constexpr (kArgmax) {
    // the workgroup's greedy candidate over the outputs its waves wrote (torch.argmax's order
    // on the bf16 values), for bfly_greedy_advance
    // only lanes 0..3 hold outputs: two steps within the quad; then each wave folds its key
    // into the workgroup's by an LDS max and counts itself done, and the last one writes the
    // workgroup's candidate (no barrier: a wave that is done leaves the CU at once)
#pragma unroll
    for (int o = 1; o <= 2; o <<= 1) {
      const uint64_t ok = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(bk >> 32), o) << 32) |
                          (uint32_t)__shfl_xor((int)(uint32_t)bk, o);
      bk = ok > bk ? ok : bk;
    }
    if (lane == 0) {
      atomicMax(&wg_key, (unsigned long long)bk);
      if (atomicAdd(&wg_done, 1u) == (unsigned)NW - 1) {
        nm.cand[blockIdx.x] = atomicMax(&wg_key, 0ull);   // every wave's key is in
        if (blockIdx.x == 0) *nm.cand_n = gridDim.x;
      }
    }
  }
}

template <int NP, int R, bool kSilu>
void q4_launch(Q4Args a, hipStream_t stream) {
  constexpr int OUTS = kSilu ? R / 2 : R;
  a.n_sets = (a.n_out + OUTS - 1) / OUTS;
  const int64_t iters = (a.n_sets + kQ4MaxWaves - 1) / kQ4MaxWaves;
  const int64_t grid = (a.n_sets + iters - 1) / iters;
  hipLaunchKernelGGL((q4_gemv_kernel<NP, R, kSilu>), dim3((unsigned)grid), dim3(64), 0, stream, a);
}

// Rows per set: four when the sets still cover the chip twice over, else two
// (small projections want more waves; two rows keep two pieces in flight).
template <bool kSilu>
void q4_dispatch(Q4Args a, int64_t in_features, int group, hipStream_t stream) {
  a.pieces = (int)(in_features / kQ4PieceCodes);
  a.groups = (int)(in_features / group);
  a.pieces_per_group = group / kQ4PieceCodes;
  const int np = (a.pieces + 63) / 64;
  const int64_t sets4 = (a.n_out + (kSilu ? 1 : 3)) / (kSilu ? 2 : 4);
  const bool four = np == 1 && sets4 >= 2048;
  switch (np) {
    case 1:
      if (four)
        q4_launch<1, 4, kSilu>(a, stream);
      else
        q4_launch<1, 2, kSilu>(a, stream);
      break;
    case 2: q4_launch<2, 2, kSilu>(a, stream); break;
    case 3: q4_launch<3, 2, kSilu>(a, stream); break;
    default: q4_launch<4, 2, kSilu>(a, stream); break;
  }
}

// Workgroups of a normed product's launch (the grid caps the waves at kQ4MaxWaves).
template <int R, bool kSilu, int NW = 8>
int64_t q4_norm_grid(int64_t n_out) {
  constexpr int OUTS = kSilu ? R / 2 : R;
  const int64_t n_sets = (n_out + OUTS - 1) / OUTS;
  const int64_t iters = (n_sets + kQ4MaxWaves - 1) / kQ4MaxWaves;
  const int64_t waves = (n_sets + iters - 1) / iters;
  return (waves + NW - 1) / NW;
}

template <int NP, int R, bool kSilu, int PER, int NW = 8, bool kParts = false, bool kArgmax = false>
void q4_norm_launch(Q4Args a, Q4NormArgs nm, hipStream_t stream) {
  constexpr int OUTS = kSilu ? R / 2 : R;
  a.n_sets = (a.n_out + OUTS - 1) / OUTS;
  hipLaunchKernelGGL((q4_norm_gemv_kernel<NP, R, kSilu, PER, NW, kParts, kArgmax>),
                     dim3((unsigned)q4_norm_grid<R, kSilu, NW>(a.n_out)), dim3(64 * NW), 0, stream, a, nm);
}

// in_features = 256 PER with PER in {8, 16, 24} (one to three pieces per lane; a fourth would
// not fit the registers of two waves per SIMD); rows per set as q4_dispatch chooses them.  The
// SiLU form at four rows per set runs 12 waves per workgroup: cfg5's gate|up (3072 sets) is then
// 256 workgroups, one per CU, where 8 waves gave 384 and half the CUs ran two (7.26 -> 6.35 us,
// graph-replayed over 24 weight sets; other shapes measured no faster).
template <bool kSilu, bool kParts = false, bool kArgmax = false>
void q4_norm_dispatch(Q4Args a, Q4NormArgs nm, int64_t in_features, int group, hipStream_t stream) {
  a.pieces = (int)(in_features / kQ4PieceCodes);
  a.groups = (int)(in_features / group);
  a.pieces_per_group = group / kQ4PieceCodes;
  const int64_t sets4 = (a.n_out + (kSilu ? 1 : 3)) / (kSilu ? 2 : 4);
  switch (in_features / 256) {
    case 8:
      if (sets4 >= 2048 && kSilu)
        q4_norm_launch<1, 4, kSilu, 8, 12, kParts, kArgmax>(a, nm, stream);
      else if (sets4 >= 2048)
        q4_norm_launch<1, 4, kSilu, 8, 8, kParts, kArgmax>(a, nm, stream);
      else
        q4_norm_launch<1, 2, kSilu, 8, 8, kParts, kArgmax>(a, nm, stream);
      break;
    case 16: q4_norm_launch<2, 2, kSilu, 16, 8, kParts, kArgmax>(a, nm, stream); break;
    default: q4_norm_launch<3, 2, kSilu, 24, 8, kParts, kArgmax>(a, nm, stream); break;
  }
}

// Workgroups of the plain (no SiLU) normed product q4_norm_dispatch launches: its greedy
// candidates.
int64_t q4_norm_plain_grid(int64_t n_out, int64_t in_features) {
  return in_features == 2048 && (n_out + 3) / 4 >= 2048 ? q4_norm_grid<4, false>(n_out) : q4_norm_grid<2, false>(n_out);
}

int q4_norm_check(const void* x, const void* residual, const void* weight, void* h_out, int64_t in_features) {
  BFLY_CHECK_ARG(weight != nullptr, "null norm weight");
  BFLY_CHECK_ARG((residual == nullptr) == (h_out == nullptr), "residual and h_out must both be given or both NULL");
  BFLY_CHECK_ARG(in_features % 2048 == 0 && in_features <= 6144,
                 "in_features=%lld: the normed product takes 2048, 4096 or 6144", (long long)in_features);
  BFLY_CHECK_ARG(aligned16(x) && aligned16(residual) && aligned16(weight) && aligned16(h_out),
                 "x, residual, weight and h_out must be 16-byte aligned");
  return BFLY_OK;
}

Q4Args q4_args(const void* x, const void* packed, const void* scale_bias, int64_t out_features, void* out) {
  Q4Args a{};
  a.x = static_cast<const __bf16*>(x);
  a.w = static_cast<const u32x4*>(packed);
  a.sb = static_cast<const uint32_t*>(scale_bias);
  a.y = static_cast<__bf16*>(out);
  a.n_out = out_features;
  return a;
}

int q4_check(const void* x, const void* packed, const void* scale_bias, int64_t out_features, int64_t in_features,
             int group, const void* out) {
  BFLY_CHECK_ARG(x && packed && scale_bias && out, "null pointer");
  BFLY_CHECK_ARG(group > 0 && group % kQ4PieceCodes == 0, "group=%d must be a positive multiple of 32", group);
  BFLY_CHECK_ARG(in_features > 0 && in_features % group == 0, "in_features=%lld must be a multiple of group=%d",
                 (long long)in_features, group);
  BFLY_CHECK_ARG(in_features <= 64LL * kQ4MaxPieces * kQ4PieceCodes, "in_features=%lld above the supported 8192",
                 (long long)in_features);
  BFLY_CHECK_ARG(out_features > 0, "bad out_features=%lld", (long long)out_features);
  BFLY_CHECK_ARG(aligned16(x) && aligned16(packed), "x and the packed codes must be 16-byte aligned");
  BFLY_CHECK_ARG(((uintptr_t)scale_bias & 3) == 0 && ((uintptr_t)out & 1) == 0, "misaligned scale_bias or out");
  return BFLY_OK;
}

}  // namespace bfly

using namespace bfly;

extern "C" int bfly_q4_gemv(const void* x, const void* packed, const void* scale_bias, int64_t out_features,
                            int64_t in_features, int group, void* out, hipStream_t stream) {
  const int rc = q4_check(x, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  q4_dispatch<false>(q4_args(x, packed, scale_bias, out_features, out), in_features, group, stream);
  BFLY_CHECK_LAUNCH("bfly_q4_gemv");
  return BFLY_OK;
}

extern "C" int bfly_q4_gemv_silu(const void* x, const void* packed, const void* scale_bias, int64_t out_features,
                                 int64_t in_features, int group, int64_t up_row_offset, void* out,
                                 hipStream_t stream) {
  const int rc = q4_check(x, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  BFLY_CHECK_ARG(up_row_offset >= out_features, "up_row_offset=%lld overlaps the gate rows",
                 (long long)up_row_offset);
  Q4Args a = q4_args(x, packed, scale_bias, out_features, out);
  a.up_off = up_row_offset;
  q4_dispatch<true>(a, in_features, group, stream);
  BFLY_CHECK_LAUNCH("bfly_q4_gemv_silu");
  return BFLY_OK;
}

extern "C" int bfly_add_rms_norm_q4_gemv(const void* x, const void* residual, const void* norm_weight, float eps,
                                         void* h_out, const void* packed, const void* scale_bias,
                                         int64_t out_features, int64_t in_features, int group, void* out,
                                         hipStream_t stream) {
  int rc = q4_check(x, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  rc = q4_norm_check(x, residual, norm_weight, h_out, in_features);
  if (rc) return rc;
  const Q4NormArgs nm{static_cast<const __bf16*>(x), static_cast<const __bf16*>(residual),
                      static_cast<const __bf16*>(norm_weight), static_cast<__bf16*>(h_out), eps};
  q4_norm_dispatch<false>(q4_args(x, packed, scale_bias, out_features, out), nm, in_features, group, stream);
  BFLY_CHECK_LAUNCH("bfly_add_rms_norm_q4_gemv");
  return BFLY_OK;
}

extern "C" int bfly_add_rms_norm_q4_gemv_silu(const void* x, const void* residual, const void* norm_weight, float eps,
                                              void* h_out, const void* packed, const void* scale_bias,
                                              int64_t out_features, int64_t in_features, int group,
                                              int64_t up_row_offset, void* out, hipStream_t stream) {
  int rc = q4_check(x, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  rc = q4_norm_check(x, residual, norm_weight, h_out, in_features);
  if (rc) return rc;
  BFLY_CHECK_ARG(up_row_offset >= out_features, "up_row_offset=%lld overlaps the gate rows",
                 (long long)up_row_offset);
  const Q4NormArgs nm{static_cast<const __bf16*>(x), static_cast<const __bf16*>(residual),
                      static_cast<const __bf16*>(norm_weight), static_cast<__bf16*>(h_out), eps};
  Q4Args a = q4_args(x, packed, scale_bias, out_features, out);
  a.up_off = up_row_offset;
  q4_norm_dispatch<true>(a, nm, in_features, group, stream);
  BFLY_CHECK_LAUNCH("bfly_add_rms_norm_q4_gemv_silu");
  return BFLY_OK;
}

extern "C" int bfly_add_rms_norm_q4_gemv_silu_parts(const float* x_parts, int n_parts, const void* residual,
                                                    const void* norm_weight, float eps, void* h_out,
                                                    const void* packed, const void* scale_bias, int64_t out_features,
                                                    int64_t in_features, int group, int64_t up_row_offset, void* out,
                                                    hipStream_t stream) {
  BFLY_CHECK_ARG(x_parts != nullptr && n_parts == 4, "x_parts: four partial rows (n_parts=%d)", n_parts);
  BFLY_CHECK_ARG(aligned16(x_parts), "x_parts must be 16-byte aligned");
  // x is only checked for null / alignment; the partial rows stand in for it
  int rc = q4_check(x_parts, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  rc = q4_norm_check(x_parts, residual, norm_weight, h_out, in_features);
  if (rc) return rc;
  BFLY_CHECK_ARG(up_row_offset >= out_features, "up_row_offset=%lld overlaps the gate rows",
                 (long long)up_row_offset);
  const Q4NormArgs nm{nullptr, static_cast<const __bf16*>(residual), static_cast<const __bf16*>(norm_weight),
                      static_cast<__bf16*>(h_out), eps, x_parts};
  Q4Args a = q4_args(x_parts, packed, scale_bias, out_features, out);
  a.x = nullptr;
  a.up_off = up_row_offset;
  q4_norm_dispatch<true, true>(a, nm, in_features, group, stream);
  BFLY_CHECK_LAUNCH("bfly_add_rms_norm_q4_gemv_silu_parts");
  return BFLY_OK;
}

// Workspace of bfly_add_rms_norm_q4_gemv_argmax: the int64 candidate count at 0 and
// kQ4MaxCand 64-bit candidate keys from byte 16 (one per workgroup), so a reader can request
// every slot together with the count (bfly_greedy_advance).
constexpr int64_t kQ4ArgmaxWsBytes = 16 + 8 * (int64_t)kQ4MaxCand;

extern "C" int64_t bfly_q4_argmax_workspace_bytes(int64_t out_features, int64_t in_features) {
  if (out_features <= 0 || in_features <= 0) return 0;
  return kQ4ArgmaxWsBytes;
}

extern "C" int bfly_add_rms_norm_q4_gemv_argmax(const void* x, const void* residual, const void* norm_weight, float eps,
                                                void* h_out, const void* packed, const void* scale_bias,
                                                int64_t out_features, int64_t in_features, int group, void* out,
                                                void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  int rc = q4_check(x, packed, scale_bias, out_features, in_features, group, out);
  if (rc) return rc;
  rc = q4_norm_check(x, residual, norm_weight, h_out, in_features);
  if (rc) return rc;
  BFLY_CHECK_ARG(out_features < INT32_MAX, "out_features=%lld: rows are kept as int32", (long long)out_features);
  BFLY_CHECK_ARG(q4_norm_plain_grid(out_features, in_features) <= kQ4MaxCand, "too many workgroups");
  BFLY_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= kQ4ArgmaxWsBytes,
                 "workspace: %lld bytes, 16-byte aligned, needed (bfly_q4_argmax_workspace_bytes)",
                 (long long)kQ4ArgmaxWsBytes);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  Q4NormArgs nm{static_cast<const __bf16*>(x), static_cast<const __bf16*>(residual),
                static_cast<const __bf16*>(norm_weight), static_cast<__bf16*>(h_out), eps, nullptr,
                reinterpret_cast<uint64_t*>(ws + 16)};
  // the count the candidates are read with: written by the launch's workgroup 0 (no host copy
  // and no fill node: the call stays capturable)
  nm.cand_n = reinterpret_cast<int64_t*>(ws);
  q4_norm_dispatch<false, false, true>(q4_args(x, packed, scale_bias, out_features, out), nm, in_features, group,
                                       stream);
  BFLY_CHECK_LAUNCH("bfly_add_rms_norm_q4_gemv_argmax");
  return BFLY_OK;
}
