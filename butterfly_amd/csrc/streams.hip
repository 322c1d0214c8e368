// Stream-level attention on gfx950: the two streams and the merge that the
// reference composes its one-shot entry from, exposed on their own.
//
// Reference semantics: _swa_stream_attention (bna/mlx/attention.py:304-369),
// _compressed_stream_attention (:372-516; HCA mode, dense over every earlier
// block summary, :411-439; routed mode :441-516) and _online_softmax_merge
// (:519-548).  Each stream returns (o, l, m): o = softmax-weighted values in
// the query dtype, l = sum of exp(score - m), m = row max, both fp32; a row with
// nothing to attend returns (0, 0, -1e30) so that it merges as a no-op.
//
// stream_kernel: one wave per (batch, query head, query).  Keys are visited in
// groups of 64 (one per lane) with a running max and rescaled accumulators, so
// any window or summary count works in constant LDS; the result equals the
// reference's single-pass softmax up to fp32 rounding.  These are the
// reference's ablation and composition paths, not the fused hot path
// (attention.hip), so the kernel favours generality over bandwidth.
#include "bfly_common.h"

namespace bfly {

constexpr int kStreamMaxD = 512;
constexpr float kStreamNeg = -1e30f;   // empty-stream max, bna/mlx/attention.py:38
constexpr float kStreamEps = 1e-9f;    // normaliser floor, bna/mlx/attention.py:39

enum StreamMode { kSwa = 0, kHca = 1, kRouted = 2 };

struct StreamArgs {
  const void* q;
  const void* k;            // raw keys [B, Hkv, krows, d] (SWA) or summaries [B, Hkv, krows, d]
  const void* v;
  void* o;
  float* l;
  float* m;
  const int32_t* routed;    // [Hq, routed_blocks, kcap] (routed mode)
  int64_t batch;
  int hq, hkv;
  int64_t tq;
  int d;
  int64_t krows;
  int mode;
  int window;
  int bs;
  int64_t nsum;
  int64_t routed_blocks;
  int kcap;
  float scale;
};

__device__ __forceinline__ float stream_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float stream_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T>
__global__ void __launch_bounds__(64) stream_kernel(StreamArgs a) {
  constexpr int kSlices = kStreamMaxD / 64;
  const int64_t t = blockIdx.x;
  const int64_t bh = blockIdx.y;                 // batch * hq + query head
  const int64_t bi = bh / a.hq;
  const int h = (int)(bh - bi * a.hq);
  const int kvh = h / (a.hq / a.hkv);
  const int lane = threadIdx.x;
  const int d = a.d;

  __shared__ float qs[kStreamMaxD];
  __shared__ float es[64];
  __shared__ int64_t rows[64];
  const T* qrow = reinterpret_cast<const T*>(a.q) + (bh * a.tq + t) * d;
  for (int c = lane; c < d; c += 64) qs[c] = to_f32(qrow[c]);
  const int64_t kv_off = (bi * a.hkv + kvh) * a.krows * d;
  const T* kb = reinterpret_cast<const T*>(a.k) + kv_off;
  const T* vb = reinterpret_cast<const T*>(a.v) + kv_off;

  // the row's candidate keys: SWA positions [lo, t]; HCA summaries [0, qb);
  // routed entries routed[h, qb, 0..kcap) with 0 <= idx < qb (and < nsum)
  const int64_t qb = a.mode == kSwa ? 0 : t / a.bs;
  int64_t lo = 0, nk = 0;
  if (a.mode == kSwa) {
    lo = t - a.window + 1;
    if (lo < 0) lo = 0;
    nk = t - lo + 1;
  } else if (a.mode == kHca) {
    nk = qb < a.nsum ? qb : a.nsum;
  } else {
    nk = qb < a.routed_blocks ? a.kcap : 0;
  }
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.f;
  float acc[kSlices];
#pragma unroll
  for (int i = 0; i < kSlices; ++i) acc[i] = 0.f;
  for (int64_t c0 = 0; c0 < nk; c0 += 64) {
    const int64_t j = c0 + lane;
    int64_t row = -1;
    if (j < nk) {
      if (a.mode == kSwa) {
        row = lo + j;
      } else if (a.mode == kHca) {
        row = j;
      } else {
        const int idx = a.routed[((int64_t)h * a.routed_blocks + qb) * a.kcap + j];
        if (idx >= 0 && idx < qb && idx < a.nsum) row = idx;
      }
    }
    float s = -INFINITY;
    if (row >= 0) {
      const T* kr = kb + row * d;
      float dot = 0.f;
      for (int c = 0; c < d; ++c) dot = fmaf(qs[c], to_f32(kr[c]), dot);
      s = dot * a.scale;
    }
    const float cm = stream_wave_max(s);
    if (cm == -INFINITY) continue;              // no valid key in this group (wave-uniform)
    const float nm = fmaxf(m_run, cm);
    const float alpha = expf(m_run - nm);       // 0 while m_run is still -inf
    const float e = row >= 0 ? expf(s - nm) : 0.f;
    l_run = l_run * alpha + stream_wave_sum(e);
    es[lane] = e;
    rows[lane] = row;
    __syncthreads();
    const int cnt = (int)(nk - c0 < 64 ? nk - c0 : 64);
#pragma unroll
    for (int i = 0; i < kSlices; ++i) acc[i] *= alpha;
    for (int jj = 0; jj < cnt; ++jj) {
      const int64_t r = rows[jj];
      if (r < 0) continue;
      const T* vr = vb + r * d;
      const float ej = es[jj];
#pragma unroll
      for (int i = 0; i < kSlices; ++i) {
        const int c = lane + 64 * i;
        if (c < d) acc[i] = fmaf(ej, to_f32(vr[c]), acc[i]);
      }
    }
    __syncthreads();
    m_run = nm;
  }

  T* orow = reinterpret_cast<T*>(a.o) + (bh * a.tq + t) * d;
  const int64_t lm = bh * a.tq + t;
  const bool any = m_run != -INFINITY;
  const float inv = any ? 1.f / fmaxf(l_run, kStreamEps) : 0.f;
#pragma unroll
  for (int i = 0; i < kSlices; ++i) {
    const int c = lane + 64 * i;
    if (c < d) orow[c] = from_f32<T>(any ? acc[i] * inv : 0.f);
  }
  if (lane == 0) {
    a.l[lm] = any ? l_run : 0.f;
    a.m[lm] = any ? m_run : kStreamNeg;
  }
}

template <typename TA, typename TB>
__global__ void __launch_bounds__(256) merge_kernel(const TA* __restrict__ oa, const float* __restrict__ la,
                                                    const float* __restrict__ ma, const TB* __restrict__ ob,
                                                    const float* __restrict__ lb, const float* __restrict__ mb,
                                                    int64_t n, int d, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = i / d;
  const float mt = fmaxf(ma[r], mb[r]);
  const float ca = expf(ma[r] - mt), cb = expf(mb[r] - mt);
  const float lt = ca * la[r] + cb * lb[r];
  out[i] = (ca * la[r] * to_f32(oa[i]) + cb * lb[r] * to_f32(ob[i])) / fmaxf(lt, kStreamEps);
}

static int launch_stream(const StreamArgs& a, int dtype, hipStream_t stream, const char* what) {
  BFLY_CHECK_ARG(a.tq <= INT32_MAX && a.batch * a.hq <= 65535, "%s: grid too large", what);
  if (a.tq == 0) return BFLY_OK;
  dim3 grid((unsigned)a.tq, (unsigned)(a.batch * a.hq));
  if (dtype == BFLY_DTYPE_F32)
    hipLaunchKernelGGL(stream_kernel<float>, grid, dim3(64), 0, stream, a);
  else
    hipLaunchKernelGGL(stream_kernel<__bf16>, grid, dim3(64), 0, stream, a);
  BFLY_CHECK_LAUNCH(what);
  return BFLY_OK;
}

}  // namespace bfly

using namespace bfly;

static bool stream_dtype_ok(int dtype) { return dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16; }

extern "C" int bfly_swa_stream(const void* q, const void* k, const void* v, int dtype, int64_t batch, int hq,
                               int hkv, int64_t seq_len, int head_dim, int window, float scale, void* o,
                               float* l, float* m, hipStream_t stream) {
  BFLY_CHECK_ARG(stream_dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(seq_len >= 0 && head_dim > 0 && head_dim <= kStreamMaxD, "bad seq_len/head_dim (head_dim <= %d)",
                 kStreamMaxD);
  if (seq_len == 0) return BFLY_OK;
  BFLY_CHECK_ARG(q && k && v && o && l && m, "null pointer");
  StreamArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.l = l; a.m = m; a.routed = nullptr;
  a.batch = batch; a.hq = hq; a.hkv = hkv; a.tq = seq_len; a.d = head_dim; a.krows = seq_len;
  a.mode = kSwa; a.window = window > 1 ? window : 1;   // max(1, n_win), attention.py:331
  a.bs = 1; a.nsum = 0; a.routed_blocks = 0; a.kcap = 0; a.scale = scale;
  return launch_stream(a, dtype, stream, "bfly_swa_stream");
}

extern "C" int bfly_compressed_stream(const void* q, const void* k_summary, const void* v_summary, int dtype,
                                      int64_t batch, int hq, int hkv, int64_t seq_len, int head_dim,
                                      int64_t num_summaries, int block_size, const int32_t* routed,
                                      int64_t routed_blocks, int kcap, float scale, void* o, float* l, float* m,
                                      hipStream_t stream) {
  BFLY_CHECK_ARG(stream_dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(seq_len >= 0 && head_dim > 0 && head_dim <= kStreamMaxD, "bad seq_len/head_dim (head_dim <= %d)",
                 kStreamMaxD);
  BFLY_CHECK_ARG(block_size > 0 && num_summaries >= 0, "bad block_size/num_summaries");
  if (seq_len == 0) return BFLY_OK;
  BFLY_CHECK_ARG(q && o && l && m, "null pointer");
  BFLY_CHECK_ARG(num_summaries == 0 || (k_summary && v_summary), "null summary pointer");
  const int64_t qblocks = (seq_len + block_size - 1) / block_size;
  if (routed) {
    BFLY_CHECK_ARG(kcap > 0, "routed_indices need at least one slot");
    BFLY_CHECK_ARG(routed_blocks >= qblocks, "routed_indices cover %lld query blocks, the queries span %lld",
                   (long long)routed_blocks, (long long)qblocks);
  }
  StreamArgs a{};
  a.q = q; a.k = k_summary; a.v = v_summary; a.o = o; a.l = l; a.m = m; a.routed = routed;
  a.batch = batch; a.hq = hq; a.hkv = hkv; a.tq = seq_len; a.d = head_dim; a.krows = num_summaries;
  a.mode = routed ? kRouted : kHca; a.window = 0; a.bs = block_size; a.nsum = num_summaries;
  a.routed_blocks = routed ? routed_blocks : 0; a.kcap = routed ? kcap : 0; a.scale = scale;
  return launch_stream(a, dtype, stream, "bfly_compressed_stream");
}

extern "C" int bfly_softmax_merge(const void* oa, int dtype_a, const float* la, const float* ma, const void* ob,
                                  int dtype_b, const float* lb, const float* mb, int64_t rows, int head_dim,
                                  float* out, hipStream_t stream) {
  BFLY_CHECK_ARG(stream_dtype_ok(dtype_a) && stream_dtype_ok(dtype_b), "unsupported dtype %d/%d", dtype_a, dtype_b);
  BFLY_CHECK_ARG(rows >= 0 && head_dim > 0, "bad rows/head_dim");
  if (rows == 0) return BFLY_OK;
  BFLY_CHECK_ARG(oa && la && ma && ob && lb && mb && out, "null pointer");
  const int64_t n = rows * head_dim;
  const int64_t blocks = (n + 255) / 256;
  BFLY_CHECK_ARG(blocks <= INT32_MAX, "bfly_softmax_merge: too many elements");
  const bool fa = dtype_a == BFLY_DTYPE_F32, fb = dtype_b == BFLY_DTYPE_F32;
#define BFLY_MERGE(TA, TB)                                                                          \
  hipLaunchKernelGGL((merge_kernel<TA, TB>), dim3((unsigned)blocks), dim3(256), 0, stream,           \
                     (const TA*)oa, la, ma, (const TB*)ob, lb, mb, n, head_dim, out)
  if (fa && fb) BFLY_MERGE(float, float);
  else if (fa) BFLY_MERGE(float, __bf16);
  else if (fb) BFLY_MERGE(__bf16, float);
  else BFLY_MERGE(__bf16, __bf16);
#undef BFLY_MERGE
  BFLY_CHECK_LAUNCH("bfly_softmax_merge");
  return BFLY_OK;
}
