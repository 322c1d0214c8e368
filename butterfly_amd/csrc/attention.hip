// Butterfly compressed attention on gfx950: one softmax per query over the
// sliding window of raw keys and the routed block summaries.
//
// Reference semantics: butterfly_compressed_attention /
// butterfly_compressed_attention_active
// (bna/torch/attention_wayfinder_permute.py:1046-1197) and the two-stream
// from-cache entry (bna/mlx/attention.py:1669-1876, merge :519-548).  Scoring
// both streams in one register tile under one running max and one running sum
// is the online log-sum-exp merge of the two streams evaluated in place.
//
// Two kernels:
//  * attn_mfma_kernel<D>: bf16, head_dim 64/128/256, W <= 64, BS >= 64.
//    Work unit = (batch, kv head, segment of 64-position chunks).  Keys of the
//    current and previous 64-position page live in an LDS ring (K row-major,
//    V transposed), plus a 16-slot tile of routed summary rows.  Each wave owns
//    16 query positions and loops over the GQA group's query heads:
//      S^T = K Q^T  and  O^T = V^T P^T  on v_mfma_f32_16x16x32_bf16,
//    fp32 softmax with wavefront shuffles between the 4 lane groups.
//  * attn_generic_kernel<T>: fp32 or bf16, any shape; one wave per
//    (batch, kv head, query); lanes over keys for scores and over d for output.
#include "bfly_common.h"

namespace bfly {

struct AttnArgs {
  const void* q;
  void* out;
  const void* k;          // raw keys: linear [B, Hkv, kv_rows, d] (row = p - key_lo) or ring
  const void* v;
  const void* ks;         // summary pool [B, Hkv, pool_rows, d]
  const void* vs;
  const int32_t* nbr;     // [nblocks, kcap]
  const int32_t* qpos;    // optional [tq]
  int64_t batch;
  int hq, hkv;
  int64_t tq;
  int d;
  int64_t q_pos0;
  int64_t kv_rows;        // rows per (b, kv head) of k/v
  int64_t ring;           // 0: linear
  int64_t key_lo;         // first valid raw key position (tail_start, or 0)
  int64_t kv_len;         // raw keys are positions < kv_len
  int64_t pool_rows;
  int64_t nsum;           // summaries n >= nsum are unavailable
  int64_t nblocks;
  int kcap, bs, W;
  float scale;
  int token_cutoff;       // 0: block-level summary cut-off (one-shot), 1: token-level
};

__device__ __forceinline__ int64_t clamp_block(int64_t p, const AttnArgs& a) {
  int64_t b = p / a.bs;
  if (b < 0) b = 0;
  if (b > a.nblocks - 1) b = a.nblocks - 1;
  return b;
}

__device__ __forceinline__ int64_t summary_cutoff(int64_t p, int64_t blk, const AttnArgs& a) {
  int64_t c = a.token_cutoff ? p - a.W + 1 : blk * a.bs - a.W + 1;
  return c > 0 ? c : 0;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// --------------------------------------------------------------------------------------------
// Generic kernel: grid (tq, batch*hkv), block 64 (one wave).
constexpr int kGenericMaxKeys = 2048;
constexpr int kGenericMaxD = 512;

template <typename T>
__global__ void __launch_bounds__(64) attn_generic_kernel(AttnArgs a) {
  const int64_t r = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t bi = bh / a.hkv;
  const int kvh = (int)(bh % a.hkv);
  const int lane = threadIdx.x;
  const int g = a.hq / a.hkv;
  const int d = a.d;
  const int64_t p = a.qpos ? (int64_t)a.qpos[r] : a.q_pos0 + r;

  __shared__ float qs[kGenericMaxD];
  __shared__ float ps[kGenericMaxKeys];
  __shared__ int sel[64];
  __shared__ int nsel;

  int64_t lo = p - a.W + 1;
  if (lo < a.key_lo) lo = a.key_lo;
  if (lo < 0) lo = 0;
  int64_t hi = p < a.kv_len - 1 ? p : a.kv_len - 1;
  const int nw = hi >= lo ? (int)(hi - lo + 1) : 0;

  if (lane == 0) {
    const int64_t blk = clamp_block(p, a);
    const int64_t cut = summary_cutoff(p, blk, a);
    int c = 0;
    for (int j = 0; j < a.kcap; ++j) {
      int64_t n = a.nbr[blk * a.kcap + j];
      if (n < 0 || n >= blk || n >= a.nsum) continue;
      if ((n + 1) * a.bs > cut) continue;
      sel[c++] = (int)n;
    }
    nsel = c;
  }
  __syncthreads();
  const int nk = nw + nsel;

  const T* kbase = reinterpret_cast<const T*>(a.k) + (bi * a.hkv + kvh) * a.kv_rows * d;
  const T* vbase = reinterpret_cast<const T*>(a.v) + (bi * a.hkv + kvh) * a.kv_rows * d;
  const T* ksb = reinterpret_cast<const T*>(a.ks) + (bi * a.hkv + kvh) * a.pool_rows * d;
  const T* vsb = reinterpret_cast<const T*>(a.vs) + (bi * a.hkv + kvh) * a.pool_rows * d;
  auto krow = [&](int idx) -> const T* {
    if (idx < nw) {
      int64_t pos = lo + idx;
      int64_t rr = a.ring ? posmod(pos, a.ring) : pos - a.key_lo;
      return kbase + rr * d;
    }
    return ksb + (int64_t)sel[idx - nw] * d;
  };
  auto vrow = [&](int idx) -> const T* {
    if (idx < nw) {
      int64_t pos = lo + idx;
      int64_t rr = a.ring ? posmod(pos, a.ring) : pos - a.key_lo;
      return vbase + rr * d;
    }
    return vsb + (int64_t)sel[idx - nw] * d;
  };

  for (int hh = 0; hh < g; ++hh) {
    const int h = kvh * g + hh;
    const T* qrow = reinterpret_cast<const T*>(a.q) + ((bi * a.hq + h) * a.tq + r) * d;
    T* orow = reinterpret_cast<T*>(a.out) + ((bi * a.hq + h) * a.tq + r) * d;
    __syncthreads();
    for (int c = lane; c < d; c += 64) qs[c] = to_f32(qrow[c]);
    __syncthreads();
    float mloc = -INFINITY;
    for (int idx = lane; idx < nk; idx += 64) {
      const T* kr = krow(idx);
      float s = 0.f;
      for (int c = 0; c < d; ++c) s = fmaf(qs[c], to_f32(kr[c]), s);
      s *= a.scale;
      ps[idx] = s;
      mloc = fmaxf(mloc, s);
    }
    const float m = wave_max(mloc);
    float lloc = 0.f;
    for (int idx = lane; idx < nk; idx += 64) {
      float e = nk > 0 ? expf(ps[idx] - m) : 0.f;
      ps[idx] = e;
      lloc += e;
    }
    const float l = wave_sum(lloc);
    __syncthreads();
    const float inv = 1.f / fmaxf(l, 1e-9f);
    for (int c = lane; c < d; c += 64) {
      float acc = 0.f;
      for (int idx = 0; idx < nk; ++idx) acc = fmaf(ps[idx], to_f32(vrow(idx)[c]), acc);
      orow[c] = from_f32<T>(acc * inv);
    }
  }
}

// --------------------------------------------------------------------------------------------
// MFMA kernel.
constexpr int kPage = 64;              // positions per chunk / ring page
constexpr int kRing = 2 * kPage;       // ring slots (window <= 64 needs pages c-1, c)
constexpr int kSumSlots = 16;          // one 16-row MFMA tile of routed summaries
constexpr int kSlots = kRing + kSumSlots;
constexpr int kVPitch = kSlots + 4;    // bf16 per V^T row (296 B): spreads 16 rows over banks

template <int D>
struct MfmaCfg {
  static constexpr int KP = D + 8;                 // bf16 per K row (pad 16 B)
  static constexpr int KSTEPS = D / 32;            // MFMA k-steps over head_dim
  static constexpr int DTILES = D / 16;            // output d tiles
  static constexpr int K_BYTES = kSlots * KP * 2;
  static constexpr int V_BYTES = D * kVPitch * 2;
  static constexpr int LDS = K_BYTES + V_BYTES;
};

__device__ __forceinline__ int xcd_remap(int bid, int n) {
  // Consecutive workgroup ids are dispatched round-robin over the 8 XCDs;
  // give each XCD a contiguous run of segments so neighbouring segments (which
  // share a halo page) hit the same L2.
  if (n % 8 != 0) return bid;
  return (bid % 8) * (n / 8) + bid / 8;
}

template <int D>
__global__ void __launch_bounds__(256, D <= 128 ? 2 : 1)
attn_mfma_kernel(AttnArgs a, int seg_chunks, int64_t c_first, int64_t nchunks) {
  using C = MfmaCfg<D>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::LDS];
  __shared__ int cand_n[kSumSlots], cand_b[kSumSlots];
  __bf16* Ks = reinterpret_cast<__bf16*>(smem);                 // [kSlots][KP]
  __bf16* Vt = reinterpret_cast<__bf16*>(smem + C::K_BYTES);    // [D][kVPitch]

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lg = lane >> 4, lq = lane & 15;
  const int seg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = blockIdx.y;
  const int64_t bi = bh / a.hkv;
  const int kvh = (int)(bh % a.hkv);
  const int gsz = a.hq / a.hkv;
  const int64_t cbeg = c_first + (int64_t)seg * seg_chunks;
  int64_t cend = cbeg + seg_chunks;
  if (cend > c_first + nchunks) cend = c_first + nchunks;
  const int64_t qlo = a.q_pos0, qhi = a.q_pos0 + a.tq;

  const __bf16* kbase = reinterpret_cast<const __bf16*>(a.k) + (bi * a.hkv + kvh) * a.kv_rows * D;
  const __bf16* vbase = reinterpret_cast<const __bf16*>(a.v) + (bi * a.hkv + kvh) * a.kv_rows * D;
  const __bf16* ksb = reinterpret_cast<const __bf16*>(a.ks) + (bi * a.hkv + kvh) * a.pool_rows * D;
  const __bf16* vsb = reinterpret_cast<const __bf16*>(a.vs) + (bi * a.hkv + kvh) * a.pool_rows * D;
  const float sl2 = a.scale * 1.4426950408889634f;   // scores in log2 units

  auto key_ok = [&](int64_t p) { return p >= 0 && p >= a.key_lo && p < a.kv_len; };
  auto row_of = [&](int64_t p) { return a.ring ? posmod(p, a.ring) : p - a.key_lo; };

  // Stage one 64-position page into the ring: K row-major, V transposed.
  auto load_page = [&](int64_t pg) {
    const int sbase = (int)posmod(pg, 2) * kPage;
    const int64_t p0 = pg * kPage;
    constexpr int PIECES = D / 8;                  // 16-byte pieces per row
    for (int i = tid; i < kPage * PIECES; i += 256) {
      const int r = i / PIECES, pc = i % PIECES;
      const int64_t p = p0 + r;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (key_ok(p)) val = *reinterpret_cast<const uint4*>(kbase + row_of(p) * D + pc * 8);
      *reinterpret_cast<uint4*>(Ks + (sbase + r) * C::KP + pc * 8) = val;
    }
    for (int i = tid; i < (kPage / 2) * PIECES; i += 256) {
      const int kp = i % (kPage / 2), pc = i / (kPage / 2);
      const int64_t p = p0 + 2 * kp;
      uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
      if (key_ok(p)) v0 = *reinterpret_cast<const uint4*>(vbase + row_of(p) * D + pc * 8);
      if (key_ok(p + 1)) v1 = *reinterpret_cast<const uint4*>(vbase + row_of(p + 1) * D + pc * 8);
      const uint16_t* e0 = reinterpret_cast<const uint16_t*>(&v0);
      const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&v1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t pair = (uint32_t)e0[j] | ((uint32_t)e1[j] << 16);
        *reinterpret_cast<uint32_t*>(Vt + (pc * 8 + j) * kVPitch + sbase + 2 * kp) = pair;
      }
    }
  };

  for (int64_t c = cbeg; c < cend; ++c) {
    // ---------------- stage keys/values and summaries
    if (c == cbeg) load_page(c - 1);
    load_page(c);
    {
      // Summary candidates of the blocks this chunk's valid queries fall in.
      int64_t vp0 = c * kPage > qlo ? c * kPage : qlo;
      int64_t vp1 = (c + 1) * kPage < qhi ? (c + 1) * kPage - 1 : qhi - 1;
      const int64_t bA = clamp_block(vp0, a), bB = clamp_block(vp1, a);
      constexpr int PIECES = D / 8;
      for (int i = tid; i < kSumSlots * PIECES; i += 256) {
        const int s = i / PIECES, pc = i % PIECES;
        int cnt = 0, cn = -1, cb = -1;
        for (int64_t bb = bA; bb <= bB && cn < 0; ++bb) {
          for (int j = 0; j < a.kcap; ++j) {
            int64_t n = a.nbr[bb * a.kcap + j];
            if (n < 0 || n >= bb || n >= a.nsum) continue;
            if (cnt == s) {
              cn = (int)n;
              cb = (int)bb;
              break;
            }
            ++cnt;
          }
        }
        uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        if (cn >= 0) {
          kv = *reinterpret_cast<const uint4*>(ksb + (int64_t)cn * D + pc * 8);
          vv = *reinterpret_cast<const uint4*>(vsb + (int64_t)cn * D + pc * 8);
        }
        *reinterpret_cast<uint4*>(Ks + (kRing + s) * C::KP + pc * 8) = kv;
        const __bf16* ve = reinterpret_cast<const __bf16*>(&vv);
#pragma unroll
        for (int j = 0; j < 8; ++j) Vt[(pc * 8 + j) * kVPitch + kRing + s] = ve[j];
        if (pc == 0) {
          cand_n[s] = cn;
          cand_b[s] = cb;
        }
      }
    }
    __syncthreads();

    // ---------------- compute: wave owns positions [pw, pw+16)
    const int64_t pw = c * kPage + wave * 16;
    const int64_t qp = pw + lq;                       // this lane's query position
    const bool wave_active = (pw + 15 >= qlo) && (pw < qhi);
    if (wave_active) {
      const bool row_ok = qp >= qlo && qp < qhi;
      const int64_t qblk = clamp_block(qp, a);
      const int64_t qcut = summary_cutoff(qp, qblk, a);
      int64_t wlo = qp - a.W + 1;
      if (wlo < a.key_lo) wlo = a.key_lo;
      if (wlo < 0) wlo = 0;
      // Summary-slot eligibility of this lane's query for slots 4*lg + i.
      bool sum_ok[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int s = 4 * lg + i;
        const int n = cand_n[s];
        sum_ok[i] = row_ok && n >= 0 && cand_b[s] == qblk && (int64_t)(n + 1) * a.bs <= qcut;
      }
      const int64_t tile0 = pw - kPage;                 // position of window tile 0, key 0
      for (int hh = 0; hh < gsz; ++hh) {
        const int h = kvh * gsz + hh;
        // Q^T fragments: lane holds query qp, d in [lg*D/4, (lg+1)*D/4); k-step ks
        // takes d = lg*D/4 + 8*ks + [0, 8) (the K fragments use the same map).
        bf16x8 qf[C::KSTEPS];
        const __bf16* qrow = reinterpret_cast<const __bf16*>(a.q) +
                             ((bi * a.hq + h) * a.tq + (row_ok ? qp - a.q_pos0 : 0)) * D;
#pragma unroll
        for (int ks = 0; ks < C::KSTEPS; ++ks) {
          if (row_ok)
            qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + lg * (D / 4) + 8 * ks);
          else
            qf[ks] = bf16x8{};
        }
        // S^T for 5 window tiles + 1 summary tile.
        f32x4 st[6];
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 6; ++t) {
          const int slot0 = t < 5 ? (int)posmod(tile0 + 16 * t, kRing) : kRing;
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < C::KSTEPS; ++ks) {
            const bf16x8 kf = *reinterpret_cast<const bf16x8*>(
                Ks + (slot0 + lq) * C::KP + lg * (D / 4) + 8 * ks);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], acc, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bool ok;
            if (t < 5) {
              const int64_t kp = tile0 + 16 * t + 4 * lg + i;
              ok = row_ok && kp >= wlo && kp <= qp;
            } else {
              ok = sum_ok[i];
            }
            const float s = ok ? acc[i] * sl2 : -INFINITY;
            acc[i] = s;
            mx = fmaxf(mx, s);
          }
          st[t] = acc;
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float msafe = mx == -INFINITY ? 0.f : mx;
        float lsum = 0.f;
        bf16x8 pf[3];
#pragma unroll
        for (int t = 0; t < 6; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(st[t][i] - msafe);
            lsum += e;
            pf[t / 2][(t % 2) * 4 + i] = (__bf16)e;
          }
        }
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
        const float inv = 1.f / fmaxf(lsum, 1e-30f);
        // O^T = V^T P^T, one 16-row d tile at a time.
        __bf16* orow = reinterpret_cast<__bf16*>(a.out) +
                       ((bi * a.hq + h) * a.tq + (row_ok ? qp - a.q_pos0 : 0)) * D;
#pragma unroll 2
        for (int dt = 0; dt < C::DTILES; ++dt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          const __bf16* vrow = Vt + (dt * 16 + lq) * kVPitch;
#pragma unroll
          for (int pr = 0; pr < 3; ++pr) {
            const int sa = pr < 2 ? (int)posmod(tile0 + 32 * pr, kRing) : (int)posmod(tile0 + 64, kRing);
            const int sb = pr < 2 ? (int)posmod(tile0 + 32 * pr + 16, kRing) : kRing;
            const bf16x4 va = *reinterpret_cast<const bf16x4*>(vrow + sa + 4 * lg);
            const bf16x4 vb = *reinterpret_cast<const bf16x4*>(vrow + sb + 4 * lg);
            const bf16x8 vf = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[pr], acc, 0, 0, 0);
          }
          if (row_ok) {
            bf16x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (__bf16)(acc[i] * inv);
            *reinterpret_cast<bf16x4*>(orow + dt * 16 + 4 * lg) = o;
          }
        }
      }
    }
    __syncthreads();
  }
}

static int launch_attention(const AttnArgs& a, int dtype, hipStream_t stream, const char* what) {
  BFLY_CHECK_ARG(aligned16(a.q) && aligned16(a.out) && aligned16(a.k) && aligned16(a.v) && aligned16(a.ks) &&
                     aligned16(a.vs),
                 "%s: tensor pointers must be 16-byte aligned", what);
  const bool contiguous = a.qpos == nullptr;
  const bool mfma_ok = dtype == BFLY_DTYPE_BF16 && contiguous && a.W <= kPage && a.bs >= kPage &&
                       2 * a.kcap <= kSumSlots && (a.d == 64 || a.d == 128 || a.d == 256);
  if (a.tq == 0) return BFLY_OK;
  if (mfma_ok) {
    const int64_t c_first = floordiv(a.q_pos0, kPage);
    const int64_t c_last = floordiv(a.q_pos0 + a.tq - 1, kPage);
    const int64_t nchunks = c_last - c_first + 1;
    // Segment length: aim for >= 2 resident workgroups per CU (256 CUs) while
    // keeping the halo page (re-read once per segment) a small fraction.
    const int64_t groups = a.batch * a.hkv;
    int seg = 1;
    while (seg < 8 && (nchunks + 2 * seg - 1) / (2 * seg) * groups >= 512) seg *= 2;
    int64_t nseg = (nchunks + seg - 1) / seg;
    BFLY_CHECK_ARG(nseg <= INT32_MAX && groups <= 65535, "%s: grid too large", what);
    dim3 grid((unsigned)nseg, (unsigned)groups);
    switch (a.d) {
      case 64: hipLaunchKernelGGL(attn_mfma_kernel<64>, grid, dim3(256), 0, stream, a, seg, c_first, nchunks); break;
      case 128: hipLaunchKernelGGL(attn_mfma_kernel<128>, grid, dim3(256), 0, stream, a, seg, c_first, nchunks); break;
      default: hipLaunchKernelGGL(attn_mfma_kernel<256>, grid, dim3(256), 0, stream, a, seg, c_first, nchunks); break;
    }
  } else {
    BFLY_CHECK_ARG(a.d <= kGenericMaxD, "%s: head_dim=%d > %d", what, a.d, kGenericMaxD);
    BFLY_CHECK_ARG(a.W + a.kcap <= kGenericMaxKeys, "%s: window + kcap > %d", what, kGenericMaxKeys);
    BFLY_CHECK_ARG(a.kcap <= 64, "%s: kcap > 64", what);
    BFLY_CHECK_ARG(a.tq <= INT32_MAX && a.batch * a.hkv <= 65535, "%s: grid too large", what);
    dim3 grid((unsigned)a.tq, (unsigned)(a.batch * a.hkv));
    if (dtype == BFLY_DTYPE_F32)
      hipLaunchKernelGGL(attn_generic_kernel<float>, grid, dim3(64), 0, stream, a);
    else
      hipLaunchKernelGGL(attn_generic_kernel<__bf16>, grid, dim3(64), 0, stream, a);
  }
  BFLY_CHECK_LAUNCH(what);
  return BFLY_OK;
}

}  // namespace bfly

using namespace bfly;

extern "C" int bfly_prefill(const void* q, const void* k, const void* v, const void* k_summary,
                            const void* v_summary, int dtype, int64_t batch, int hq, int hkv,
                            int64_t seq_len, int head_dim, const int32_t* neighbors,
                            int64_t num_blocks, int kcap, int block_size, int window, float scale,
                            void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16, "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(q && k && v && k_summary && v_summary && neighbors && out, "null pointer");
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(seq_len > 0 && head_dim > 0, "bad seq_len/head_dim");
  BFLY_CHECK_ARG(window > 0, "local_window_tokens must be positive");
  BFLY_CHECK_ARG(block_size > 0 && num_blocks == (seq_len + block_size - 1) / block_size,
                 "num_blocks=%lld does not match seq_len=%lld/block_size=%d", (long long)num_blocks,
                 (long long)seq_len, block_size);
  BFLY_CHECK_ARG(kcap > 0, "kcap must be positive");
  AttnArgs a{};
  a.q = q; a.out = out; a.k = k; a.v = v; a.ks = k_summary; a.vs = v_summary;
  a.nbr = neighbors; a.qpos = nullptr;
  a.batch = batch; a.hq = hq; a.hkv = hkv; a.tq = seq_len; a.d = head_dim;
  a.q_pos0 = 0; a.kv_rows = seq_len; a.ring = 0; a.key_lo = 0; a.kv_len = seq_len;
  a.pool_rows = num_blocks; a.nsum = num_blocks; a.nblocks = num_blocks;
  a.kcap = kcap; a.bs = block_size; a.W = window; a.scale = scale; a.token_cutoff = 0;
  return launch_attention(a, dtype, stream, "bfly_prefill");
}

extern "C" int bfly_attend_cache(const void* q, int dtype, int64_t batch, int hq, int hkv,
                                 int64_t tq, int head_dim, const int32_t* query_positions,
                                 int64_t q_pos0, const void* tail_k, const void* tail_v,
                                 int64_t ring_capacity, int64_t tail_start, int64_t kv_len,
                                 const void* pool_k, const void* pool_v, int64_t pool_capacity,
                                 int64_t summary_count, const int32_t* neighbors,
                                 int64_t num_blocks, int kcap, int block_size, int window,
                                 float scale, void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16, "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(tq >= 0 && head_dim > 0, "bad tq/head_dim");
  if (tq == 0) return BFLY_OK;
  BFLY_CHECK_ARG(q && tail_k && tail_v && pool_k && pool_v && neighbors && out, "null pointer");
  BFLY_CHECK_ARG(kv_len > 0, "kv_len must be positive");
  BFLY_CHECK_ARG(window > 0, "local_window_tokens must be positive");
  BFLY_CHECK_ARG(block_size > 0 && num_blocks > 0 && kcap > 0, "bad block_size/num_blocks/kcap");
  BFLY_CHECK_ARG(ring_capacity >= 0 && tail_start >= 0 && tail_start <= kv_len, "bad tail bounds");
  BFLY_CHECK_ARG(ring_capacity == 0 || kv_len - tail_start <= ring_capacity,
                 "tail [%lld, %lld) does not fit ring capacity %lld", (long long)tail_start,
                 (long long)kv_len, (long long)ring_capacity);
  BFLY_CHECK_ARG(summary_count >= 0 && summary_count <= pool_capacity, "summary_count > pool capacity");
  BFLY_CHECK_ARG(query_positions != nullptr || (q_pos0 >= 0 && q_pos0 + tq <= kv_len),
                 "query positions [%lld, %lld) outside [0, kv_len=%lld)", (long long)q_pos0,
                 (long long)(q_pos0 + tq), (long long)kv_len);
  AttnArgs a{};
  a.q = q; a.out = out; a.k = tail_k; a.v = tail_v; a.ks = pool_k; a.vs = pool_v;
  a.nbr = neighbors; a.qpos = query_positions;
  a.batch = batch; a.hq = hq; a.hkv = hkv; a.tq = tq; a.d = head_dim;
  a.q_pos0 = q_pos0; a.kv_rows = ring_capacity ? ring_capacity : kv_len - tail_start; a.ring = ring_capacity;
  a.key_lo = tail_start; a.kv_len = kv_len;
  a.pool_rows = pool_capacity; a.nsum = summary_count; a.nblocks = num_blocks;
  a.kcap = kcap; a.bs = block_size; a.W = window; a.scale = scale; a.token_cutoff = 1;
  return launch_attention(a, dtype, stream, "bfly_attend_cache");
}
