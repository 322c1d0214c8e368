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
// Three kernels:
//  * attn_mfma_kernel<D>: bf16, head_dim 64/128/256, W <= 64, BS >= 64.
//    Work unit = (batch, kv head, segment of 64-position chunks).  Keys of the
//    current and previous 64-position page live in an LDS ring (K row-major,
//    V transposed), plus a 16-slot tile of routed summary rows.  Each wave owns
//    16 query positions and loops over the GQA group's query heads:
//      S^T = K Q^T  and  O^T = V^T P^T  on v_mfma_f32_16x16x32_bf16,
//    fp32 softmax with wavefront shuffles between the 4 lane groups.
//  * attn_f32_tile_kernel<D>: fp32, head_dim 64/128, W <= 64, GQA groups of at
//    most 4, BS a multiple of 16; one workgroup per (batch, kv head, 16-query
//    tile), keys staged in LDS, both products on v_mfma_f32_16x16x4_f32.
//  * attn_generic_kernel<T>: fp32 or bf16, any shape; one wave per
//    (batch, kv head, query); lanes over keys for scores and over d for output.
#include <stdlib.h>

#include <type_traits>

#include "bfly_topology.h"
#include "cache_update.h"

namespace bfly {

struct AttnArgs {
  const void* q;
  void* out;
  const void* k;          // raw keys: linear [B, Hkv, kv_rows, d] (row = p - key_lo) or ring
  const void* v;
  const void* ks;         // summary pool [B, Hkv, pool_rows, d]
  const void* vs;
  const int32_t* nbr;     // [nblocks, kcap], or null: the MFMA kernel computes rows from topo
  bfly_topology_t topo;   // the layout at nblocks blocks (used when nbr is null)
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
// Generic kernel: grid (tq, batch*hkv), block 64 (one wave).  Up to kGenericHeads query heads of
// the GQA group at a time share every K and V row read (scores: one lane per key, the row read in
// 4-element pieces; output: one lane per d); each head's score and output sums keep the order
// of a plain loop over d and over keys.
constexpr int kGenericMaxKeys = 2048;
constexpr int kGenericMaxD = 512;
constexpr int kGenericHeads = 4;

// dynamic LDS of attn_generic_kernel: q rows and scores of kGenericHeads heads
inline size_t generic_lds_bytes(int d, int W, int kcap) {
  return (size_t)kGenericHeads * (size_t)(d + W + kcap) * sizeof(float);
}

// 4 consecutive elements of a row as fp32 (16 bytes for fp32, 8 for bf16; d % 4 == 0 keeps
// every row start aligned to the piece)
__device__ __forceinline__ void load4_f32(const float* p, float (&x)[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
}
__device__ __forceinline__ void load4_f32(const __bf16* p, float (&x)[4]) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xFFFF0000u);
  x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xFFFF0000u);
}

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
  constexpr int GH = kGenericHeads;

  // dynamic LDS: q rows [GH][d], then scores [GH][W + kcap] (generic_lds_bytes)
  extern __shared__ float gen_lds[];
  const int kmax = a.W + a.kcap;
  auto qs = [&](int hh, int c) -> float& { return gen_lds[hh * d + c]; };
  auto ps = [&](int hh, int idx) -> float& { return gen_lds[GH * d + hh * kmax + idx]; };
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
  const bool vec = (d & 3) == 0;

  for (int h0 = 0; h0 < g; h0 += GH) {
    const int nh = g - h0 < GH ? g - h0 : GH;
    const T* qhead = reinterpret_cast<const T*>(a.q) + ((bi * a.hq + kvh * g + h0) * a.tq + r) * d;
    __syncthreads();
    for (int i = lane; i < GH * d; i += 64) {
      const int hh = i / d, c = i - hh * d;
      // heads past the group repeat its last one (computed, never stored)
      qs(hh, c) = to_f32(qhead[(int64_t)(hh < nh ? hh : nh - 1) * a.tq * d + c]);
    }
    __syncthreads();
    float mloc[GH];
#pragma unroll
    for (int hh = 0; hh < GH; ++hh) mloc[hh] = -INFINITY;
    for (int idx = lane; idx < nk; idx += 64) {
      const T* kr = krow(idx);
      float s[GH];
#pragma unroll
      for (int hh = 0; hh < GH; ++hh) s[hh] = 0.f;
      if (vec) {
        for (int c = 0; c < d; c += 4) {
          float kx[4];
          load4_f32(kr + c, kx);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int hh = 0; hh < GH; ++hh) s[hh] = fmaf(qs(hh, c + e), kx[e], s[hh]);
        }
      } else {
        for (int c = 0; c < d; ++c) {
          const float kx = to_f32(kr[c]);
#pragma unroll
          for (int hh = 0; hh < GH; ++hh) s[hh] = fmaf(qs(hh, c), kx, s[hh]);
        }
      }
#pragma unroll
      for (int hh = 0; hh < GH; ++hh) {
        s[hh] *= a.scale;
        ps(hh, idx) = s[hh];
        mloc[hh] = fmaxf(mloc[hh], s[hh]);
      }
    }
    float inv[GH];
#pragma unroll
    for (int hh = 0; hh < GH; ++hh) {
      const float m = wave_max(mloc[hh]);
      float lloc = 0.f;
      for (int idx = lane; idx < nk; idx += 64) {
        const float e = expf(ps(hh, idx) - m);
        ps(hh, idx) = e;
        lloc += e;
      }
      inv[hh] = 1.f / fmaxf(wave_sum(lloc), 1e-9f);
    }
    __syncthreads();
    for (int c = lane; c < d; c += 64) {
      float acc[GH];
#pragma unroll
      for (int hh = 0; hh < GH; ++hh) acc[hh] = 0.f;
      for (int idx = 0; idx < nk; ++idx) {
        const float vx = to_f32(vrow(idx)[c]);
#pragma unroll
        for (int hh = 0; hh < GH; ++hh) acc[hh] = fmaf(ps(hh, idx), vx, acc[hh]);
      }
      for (int hh = 0; hh < nh; ++hh)
        reinterpret_cast<T*>(a.out)[((bi * a.hq + kvh * g + h0 + hh) * a.tq + r) * d + c] = from_f32<T>(acc[hh] * inv[hh]);
    }
  }
}

// --------------------------------------------------------------------------------------------
// fp32 tile kernel: contiguous query ranges, W <= 64, d in {64, 128}, GQA groups of at most 4
// heads, block_size % 16 == 0, neighbour rows from a table with 1 <= kcap <= 16.  One 256-thread
// workgroup per (batch, kv head, 16-query tile at positions 16k .. 16k + 15); wave w computes
// query head w of the group.  The tile's key rows: the window [k0, k0 + 16 nwt) covering
// [q0 - W + 1, q0 + 15], then one 16-row tile of the routed summary rows of the tile's block in
// neighbour-row order (slot j = the row's j-th entry; the 16 queries share the block because
// block_size % 16 == 0).
//   * fp32 products on bf16 MFMA (v_mfma_f32_16x16x32_bf16): every fp32 operand x is split into
//     three bf16 parts by truncation, x = hi + mid + lo exactly (hi keeps the sign, exponent and
//     top 7 stored mantissa bits of x, mid those of x - hi, and lo = x - hi - mid has at most 8
//     significant bits), and a product a b is summed in the fp32 accumulator as the six part
//     products ah bh + ah bm + am bh + ah bl + am bm + al bh, each exact in fp32 (of the three
//     dropped ones, |am bl| and |al bm| are below 2^-21 |a b| and |al bl| below 2^-28 |a b|,
//     since |am| < 2^-7 |a| and |al| < 2^-14 |a|): the "bf16x6" scheme of Henry, Tang and Heinecke,
//     "Leveraging the bfloat16 artificial intelligence datatype for higher-precision
//     computations" (ARITH 2019).  Six 16x16x32 bf16 MFMAs (16 cycles each) replace eight
//     16x16x4 fp32 ones (32 cycles each).
//   * Requests, in this order: the block's neighbour-row entries (lane j < 16 of every wave holds
//     slot j's pool row), Q, the window's K rows tile by tile, then, once the entries are in, the
//     summary K rows, the window's V rows and the summary V rows.  Loads complete in order: the
//     scores of a pair of key tiles start when that pair's K parts are in LDS, while the later
//     rows are still arriving.  V stays in registers until the scores are done and then its parts
//     overwrite K's in the same LDS buffer (77 KB at d = 128: two workgroups per CU).
//   * Window rows: when the window lies inside the keys that exist (and, in a ring, does not
//     wrap), a thread's rows are one run from the window's first row; otherwise each row is
//     clamped into [wlo, whi] (rows past the window repeat its ends; they are masked).
//   * S^T = K Q^T: lane l (r = l % 16, lane group lg = l / 16) supplies K[tile row r][d] and
//     Q[q0 + r][d] for d = lg D/4 + 8 ks + 0..7 in k-step ks and receives the scores of tile rows
//     4 lg + i for query q0 + r.  Every tile is computed (no branch joins inside the unrolled
//     loops, which would copy the accumulators); unused tiles hold copies of valid rows and are
//     masked.
//   * Masks: window keys [max(p - W + 1, key_lo, 0), min(p, kv_len - 1)]; summary slot j is used
//     when its neighbour n satisfies 0 <= n < block, n < nsum and (n + 1) BS <= the cut-off
//     (block-level for one-shot prefill, token-level for active rows).
//   * Softmax in fp32 over the lane's scores and the four lane groups (xor shuffles 16, 32), the
//     scale and log2(e) folded into the scores and exp2 on v_exp_f32.
//   * O^T = V^T P^T over key tile pairs (2 pr, 2 pr + 1): the lane's 8 probabilities are keys
//     4 lg + 0..3 of both tiles, and its V^T fragment the same keys' values at one d, read from the
//     row-major V parts by transposing LDS reads (pieces swizzled by row).  Output tile (mt, half)
//     row r is d = 32 mt + 8 (r / 4) + 4 half + r % 4, so each lane ends with 8 consecutive d of
//     its query per mt.
// Positions and ring slots are 32-bit (the host sends only caches and rings below 2^30 rows here).
constexpr int kF32MaxKcap = 16;
constexpr int kF32WinTiles = 5;        // (64 - 1 + 15) / 16 + 1
constexpr int kF32Tiles = kF32WinTiles + 1;
constexpr int kF32Rows = 16 * kF32Tiles;

// The three bf16 parts (bit patterns, two per dword, element 0 in the low half) of four floats.
struct Parts4 {
  uint2 h, m, l;
};
__device__ __forceinline__ Parts4 split_parts(f32x4 x) {
  uint32_t hb[4], mb[4], lb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[i] = __float_as_uint(x[i]) & 0xffff0000u;
    const float rest = x[i] - __uint_as_float(hb[i]);          // exact
    mb[i] = __float_as_uint(rest) & 0xffff0000u;
    lb[i] = __float_as_uint(rest - __uint_as_float(mb[i]));     // exact, low 16 bits zero
  }
  auto pk = [](uint32_t e0, uint32_t e1) { return (e0 >> 16) | (e1 & 0xffff0000u); };
  return {{pk(hb[0], hb[1]), pk(hb[2], hb[3])}, {pk(mb[0], mb[1]), pk(mb[2], mb[3])},
          {pk(lb[0], lb[1]), pk(lb[2], lb[3])}};
}
__device__ __forceinline__ bf16x8 join8(uint2 a, uint2 b) {
  return __builtin_bit_cast(bf16x8, uint4{a.x, a.y, b.x, b.y});
}
// c + a b in the six part products (small terms first)
__device__ __forceinline__ f32x4 mfma_x6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], c, 0, 0, 0);
}

template <int D>
__global__ void __launch_bounds__(256, 2) attn_f32_tile_kernel(AttnArgs a, int tile0, int ntiles, int per_xcd) {
  constexpr int DG = D / 4;                                 // d per lane group
  constexpr int KP = D + 8;                                 // K part row pitch (bf16; 16-byte pad)
  constexpr int KSTEPS = D / 32;
  constexpr int PER_ROW = D / 4;                            // 4-float pieces per row
  constexpr int RSTEP = 256 / PER_ROW;                      // rows between a thread's pieces
  constexpr int UPT = 16 / RSTEP;                           // pieces per thread in a 16-row tile
  constexpr int WIN_STAGE = kF32WinTiles * UPT;             // a thread's window pieces
  constexpr int STAGE = kF32Tiles * UPT;                    // ... and with the summary tile's
  constexpr int KPART = kF32Rows * KP, VPART = kF32Rows * D;
  static_assert(256 % PER_ROW == 0 && 16 % RSTEP == 0, "a thread's pieces are one column, RSTEP rows apart");
  static_assert(kF32Tiles % 2 == 0, "key tiles are scored in pairs");
  __shared__ __attribute__((aligned(16))) __bf16 lds[3 * KPART];   // K parts, then V parts
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // workgroups are dispatched to the 8 XCDs round-robin: XCD x = blockIdx % 8 takes the items
  // x per_xcd .. x per_xcd + per_xcd - 1, consecutive tiles of one (batch, kv head), which share
  // most of their window rows in that XCD's L2
  const int item = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (item >= ntiles * (int)(a.batch * a.hkv)) return;   // the whole workgroup
  const int tile = tile0 + item % ntiles;
  const int bh = item / ntiles;
  const int64_t bi = bh / a.hkv;
  const int kvh = bh % a.hkv;
  const int gsz = a.hq / a.hkv;
  const int r = lane & 15, lg = lane >> 4;
  const int q0 = tile * 16;
  const int p = q0 + r;                                     // this lane's query (column r)
  const int qlo = (int)a.q_pos0, qhi = (int)(a.q_pos0 + a.tq);
  const bool qok = p >= qlo && p < qhi && w < gsz;
  const int qrow = p >= qlo && p < qhi ? p - qlo : 0;
  const int key_lo = (int)a.key_lo, kv_len = (int)a.kv_len, W = a.W, bs = a.bs;
  const int ring = (int)a.ring;
  // the workgroup's window: [q0 - W + 1, q0 + 15] clipped to the keys that exist
  const int wlo = max(max(q0 - W + 1, key_lo), 0);
  const int whi = min(q0 + 15, kv_len - 1);
  const int nwt = (W - 1 + 15) / 16 + 1;                    // window tiles
  const int kstart = q0 - 16 * (nwt - 1);
  const int blk = min((int)((uint32_t)max(q0, 0) / (uint32_t)bs), (int)a.nblocks - 1);
  const int hq_i = kvh * gsz + (w < gsz ? w : 0);           // a wave past the group repeats head 0
  const float* kb = reinterpret_cast<const float*>(a.k) + (bi * a.hkv + kvh) * a.kv_rows * D;
  const float* vb = reinterpret_cast<const float*>(a.v) + (bi * a.hkv + kvh) * a.kv_rows * D;
  const float* ksb = reinterpret_cast<const float*>(a.ks) + (bi * a.hkv + kvh) * a.pool_rows * D;
  const float* vsb = reinterpret_cast<const float*>(a.vs) + (bi * a.hkv + kvh) * a.pool_rows * D;

  // the block's neighbour-row entry of slot lane % 16 (the host sends kcap >= 1)
  const int nb_raw = a.nbr[(int64_t)blk * a.kcap + min(lane & 15, a.kcap - 1)];
  const float* qp = reinterpret_cast<const float*>(a.q) + ((bi * a.hq + hq_i) * a.tq + qrow) * D + DG * lg;
  f32x4 qv[DG / 4];
#pragma unroll
  for (int c = 0; c < DG / 4; ++c) qv[c] = *reinterpret_cast<const f32x4*>(qp + 4 * c);

  // a thread's pieces: column c4 of rows row0 + RSTEP u (u < WIN_STAGE: window row kstart + that;
  // then summary slot row0 + RSTEP (u - WIN_STAGE)); LDS row row0 + RSTEP u either way
  const int c4 = tid % PER_ROW, row0 = tid / PER_ROW;
  int woff[WIN_STAGE];   // the window pieces' rows among the head's K/V rows
  const bool run = kstart >= wlo && kstart + 16 * kF32WinTiles - 1 <= whi &&
                   (ring == 0 || (int)((uint32_t)kstart % (uint32_t)ring) + 16 * kF32WinTiles <= ring);
  if (run) {
    const int base = ring ? (int)((uint32_t)kstart % (uint32_t)ring) : kstart - key_lo;
#pragma unroll
    for (int u = 0; u < WIN_STAGE; ++u) woff[u] = base + row0 + RSTEP * u;
  } else {
    const int last = (int)min(a.kv_rows - 1, (int64_t)INT32_MAX);
#pragma unroll
    for (int u = 0; u < WIN_STAGE; ++u) {
      const int pos = min(max(kstart + row0 + RSTEP * u, wlo), whi);   // >= 0: wlo >= 0, whi >= 0
      const int ro = ring ? (int)((uint32_t)pos % (uint32_t)ring) : pos - key_lo;
      woff[u] = min(max(ro, 0), last);
    }
  }
  f32x4 kx[STAGE], vx[STAGE];
#pragma unroll
  for (int u = 0; u < WIN_STAGE; ++u) kx[u] = *reinterpret_cast<const f32x4*>(kb + (int64_t)woff[u] * D + 4 * c4);
  // nothing below moves above the window requests: the first use of the entries waits for them
  __builtin_amdgcn_sched_barrier(0);
  // lane j < 16 of every wave: slot j's pool row, or -1 where the slot is unused (j >= kcap, no
  // neighbour, not an earlier block, or not summarised yet)
  const int nb_lane = (lane & 15) < a.kcap && nb_raw >= 0 && nb_raw < blk && nb_raw < a.nsum ? nb_raw : -1;
  // the summary pieces' pool rows (the entries were requested first: this waits for them alone);
  // unused slots read pool row 0 and are masked
  int soff[STAGE - WIN_STAGE];
#pragma unroll
  for (int u = WIN_STAGE; u < STAGE; ++u) soff[u - WIN_STAGE] = max(__shfl(nb_lane, row0 + RSTEP * (u - WIN_STAGE)), 0);
#pragma unroll
  for (int u = WIN_STAGE; u < STAGE; ++u)
    kx[u] = *reinterpret_cast<const f32x4*>(ksb + (int64_t)soff[u - WIN_STAGE] * D + 4 * c4);
#pragma unroll
  for (int u = 0; u < WIN_STAGE; ++u) vx[u] = *reinterpret_cast<const f32x4*>(vb + (int64_t)woff[u] * D + 4 * c4);
#pragma unroll
  for (int u = WIN_STAGE; u < STAGE; ++u)
    vx[u] = *reinterpret_cast<const f32x4*>(vsb + (int64_t)soff[u - WIN_STAGE] * D + 4 * c4);
  // every request is out before the first wait for data (Q's split below)
  __builtin_amdgcn_sched_barrier(0);
  // this lane's summary slots 4 lg + jj
  int sn[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) sn[jj] = __shfl(nb_lane, 4 * lg + jj);
  const int cut = max(a.token_cutoff ? p - W + 1 : blk * bs - W + 1, 0);
  const int klo = max(max(p - W + 1, key_lo), 0), khi = min(p, kv_len - 1);
  const float sl2 = a.scale * 1.4426950408889634f;          // scale * log2(e)

  // Q's parts in MFMA B-operand form: k-step ks holds d = DG lg + 8 ks + 0..7
  bf16x8 qf[KSTEPS][3];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    const Parts4 x0 = split_parts(qv[2 * ks]), x1 = split_parts(qv[2 * ks + 1]);
    qf[ks][0] = join8(x0.h, x1.h);
    qf[ks][1] = join8(x0.m, x1.m);
    qf[ks][2] = join8(x0.l, x1.l);
  }

  f32x4 c[kF32Tiles];
#pragma unroll
  for (int t = 0; t < kF32Tiles; ++t) c[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t0 = 0; t0 < kF32Tiles; t0 += 2) {
#pragma unroll
    for (int u = t0 * UPT; u < (t0 + 2) * UPT; ++u) {
      const Parts4 x = split_parts(kx[u]);
      const int off = (row0 + RSTEP * u) * KP + 4 * c4;
      *reinterpret_cast<uint2*>(lds + off) = x.h;
      *reinterpret_cast<uint2*>(lds + KPART + off) = x.m;
      *reinterpret_cast<uint2*>(lds + 2 * KPART + off) = x.l;
    }
    __syncthreads();   // K parts of tiles t0, t0 + 1 in LDS
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
      for (int t = t0; t < t0 + 2; ++t) {
        const int off = (16 * t + r) * KP + DG * lg + 8 * ks;
        const bf16x8 kf[3] = {*reinterpret_cast<const bf16x8*>(lds + off),
                              *reinterpret_cast<const bf16x8*>(lds + KPART + off),
                              *reinterpret_cast<const bf16x8*>(lds + 2 * KPART + off)};
        c[t] = mfma_x6(kf, qf[ks], c[t]);
      }
    }
  }
  float sc[kF32Tiles][4];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < kF32Tiles; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      bool ok;
      if (t < kF32WinTiles) {
        const int kpos = kstart + 16 * t + 4 * lg + jj;
        ok = t < nwt && kpos >= klo && kpos <= khi;
      } else {
        ok = sn[jj] >= 0 && (sn[jj] + 1) * bs <= cut;
      }
      sc[t][jj] = ok ? c[t][jj] * sl2 : -INFINITY;
      m = fmaxf(m, sc[t][jj]);
    }
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  if (m == -INFINITY) m = 0.f;   // a column with nothing to attend (outside the query range)
  float l = 0.f;
#pragma unroll
  for (int t = 0; t < kF32Tiles; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      sc[t][jj] = __builtin_amdgcn_exp2f(sc[t][jj] - m);   // exp2(-inf) = 0
      l += sc[t][jj];
    }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  // P's parts in MFMA B-operand form: pair pr holds keys 4 lg + 0..3 of tiles 2 pr and 2 pr + 1
  bf16x8 pf[kF32Tiles / 2][3];
#pragma unroll
  for (int pr = 0; pr < kF32Tiles / 2; ++pr) {
    const Parts4 x0 = split_parts(f32x4{sc[2 * pr][0], sc[2 * pr][1], sc[2 * pr][2], sc[2 * pr][3]});
    const Parts4 x1 = split_parts(f32x4{sc[2 * pr + 1][0], sc[2 * pr + 1][1], sc[2 * pr + 1][2], sc[2 * pr + 1][3]});
    pf[pr][0] = join8(x0.h, x1.h);
    pf[pr][1] = join8(x0.m, x1.m);
    pf[pr][2] = join8(x0.l, x1.l);
  }

  __syncthreads();   // every wave is done with K
#pragma unroll
  for (int u = 0; u < STAGE; ++u) {
    const Parts4 x = split_parts(vx[u]);
    const int row = row0 + RSTEP * u;
    const int off = row * D + (c4 ^ (2 * vrow_swizzle<D>(row))) * 4;
    *reinterpret_cast<uint2*>(lds + off) = x.h;
    *reinterpret_cast<uint2*>(lds + VPART + off) = x.m;
    *reinterpret_cast<uint2*>(lds + 2 * VPART + off) = x.l;
  }
  __syncthreads();   // V parts in LDS

  const float inv = 1.f / fmaxf(l, 1e-9f);
  float* op = reinterpret_cast<float*>(a.out) + ((bi * a.hq + hq_i) * a.tq + qrow) * D + 8 * lg;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
    f32x4 o[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      // lane (lg, r) reads d 32 mt + 8 (r & 3) + 4 half + 0..3 of key row 4 lg + (r >> 2) of
      // each tile: lane r of the group receives d row r's four keys 4 lg + 0..3
      const int unit = mt * 8 + (r & 3) * 2 + half;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pr = 0; pr < kF32Tiles / 2; ++pr) {
        const int ra = 32 * pr + 4 * lg + (r >> 2), rb = ra + 16;
        const int oa = ra * D + (unit ^ (2 * vrow_swizzle<D>(ra))) * 4;
        const int ob = rb * D + (unit ^ (2 * vrow_swizzle<D>(rb))) * 4;
        bf16x8 vf[3];
#pragma unroll
        for (int pt = 0; pt < 3; ++pt)
          vf[pt] = __builtin_shufflevector(read_tr(lds + pt * VPART + oa), read_tr(lds + pt * VPART + ob), 0, 1, 2,
                                           3, 4, 5, 6, 7);
        acc = mfma_x6(vf, pf[pr], acc);
      }
      o[half] = acc;
    }
    // o[half][i] is O[q0 + r][32 mt + 8 lg + 4 half + i]
    if (qok) {
      *reinterpret_cast<f32x4*>(op + 32 * mt) = f32x4{o[0][0] * inv, o[0][1] * inv, o[0][2] * inv, o[0][3] * inv};
      *reinterpret_cast<f32x4*>(op + 32 * mt + 4) = f32x4{o[1][0] * inv, o[1][1] * inv, o[1][2] * inv, o[1][3] * inv};
    }
  }
}

// --------------------------------------------------------------------------------------------
// MFMA kernel.
constexpr int kPage = 64;              // positions per chunk / ring page
constexpr int kRing = 2 * kPage;       // ring slots (window <= 64 needs pages c-1, c)
constexpr int kSumSlots = 16;          // one 16-row MFMA tile of routed summaries
constexpr int kSlots = kRing + kSumSlots;
constexpr int kMaxSegChunks = 8;       // chunks per workgroup (host picks 1, 2, 4 or 8)
constexpr int kMaxKcap = kSumSlots / 2;
constexpr int kMaxSegBlocks = kMaxSegChunks * kPage / kPage + 1;   // block_size >= kPage
constexpr int kQPipe = 2;              // query heads whose Q fragments are held in registers (one pair)

template <int D>
struct MfmaCfg {
  // d = 256: 512 threads, one query head per wave (waves w and w + 4 share query rows 16 (w & 3)..
  // and take the two heads of a pair), so a wave holds one head's Q, S and O and two waves fit
  // per SIMD; smaller d: 256 threads, each wave runs a head pair over its 16 query rows
  static constexpr bool kWaveHead = D == 256;
  // d = 256: the two staged pages sit at fixed rows, the chunk's halo (page c - 1) at 0..63 and
  // its own page at 64..127, so every tile a wave reads is at a constant offset from a few
  // per-lane bases (the offsets fold into the LDS instructions); a segment of several chunks
  // shifts the page it keeps between the halves.  Smaller d keep pages at rows (page & 1) * 64.
  static constexpr bool kFixedPages = D == 256;
  static constexpr int NTHR = kWaveHead ? 512 : 256;
  static constexpr int KP = D + 8;                 // bf16 per K row (pad 16 B)
  static constexpr int KSTEPS = D / 32;            // MFMA k-steps over head_dim
  static constexpr int DTILES = D / 16;            // output d tiles
  static constexpr int PIECES = D / 8;             // 16-byte pieces per row
  static constexpr int KLD = kPage * PIECES / NTHR;        // K (and V) pieces per thread per page
  static constexpr int SITEMS = kSumSlots * PIECES;        // summary pieces per chunk
  static constexpr int SLD = (SITEMS + NTHR - 1) / NTHR;
  static constexpr int K_BYTES = kSlots * KP * 2;
  static constexpr int V_BYTES = kSlots * D * 2;           // V row-major, unpadded, swizzled
  static constexpr int LDS = K_BYTES + V_BYTES;
  __device__ static constexpr int vswz(int row) { return vrow_swizzle<D>(row); }
};

// Swap 16 bytes with lane ^ 8 (within each 16-lane row): DPP row_ror:8 rotates
// each row of 16 lanes by 8, which is lane ^ 8; a VALU move, no LDS traffic.
__device__ __forceinline__ uint32_t ror8(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xf, 0xf, false);
}
__device__ __forceinline__ bf16x8 xchg8(bf16x8 v) {
  uint4 u = __builtin_bit_cast(uint4, v);
  u.x = ror8(u.x);
  u.y = ror8(u.y);
  u.z = ror8(u.z);
  u.w = ror8(u.w);
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ int xcd_remap(int bid, int n) {
  // Consecutive workgroup ids are dispatched round-robin over the 8 XCDs;
  // give each XCD a contiguous run of segments so neighbouring segments (which
  // share a halo page) hit the same L2.
  if (n % 8 != 0) return bid;
  return (bid % 8) * (n / 8) + bid / 8;
}

// Positions, block ids and counts fit in int32 (the host checks kv_len and the
// query range); only tensor offsets use 64-bit arithmetic.
struct MfmaArgs {
  int qlo, qhi;          // query positions [qlo, qhi)
  int key_lo, kv_len;    // raw keys are positions [key_lo, kv_len)
  int ring;              // 0: linear rows (row = p - key_lo); else row = p mod ring (ring >= kPage)
  int nblocks, nsum, kcap, bs, W;
  int token_cutoff;
  // fused launch (kUpd): grid rows >= attn_y run a cache update instead
  // (cache_update_body over upd_x x upd_rows x K|V work items, upd_wgs in all; NTHR / 256 per workgroup)
  UpdateJob upd;
  int attn_y, upd_x, upd_rows;
  int64_t upd_wgs;
};

// A batched streaming launch: the attention of up to kMaxUpdateParts consecutive chunks whose
// cache updates are all done, one grid row band per chunk.  Each chunk keeps the arguments of
// its own cache state (the counters right after its update), so its results are those of a
// launch of its own.
struct ChunkArgs {
  const void* q;
  void* out;
  const void* k;          // the chunk's own keys and values, [batch x kv heads, tq, d]
  const void* v;
  int tq, qlo, qhi, key_lo, kv_len, nsum, nblocks, c_first, nchunks;
  bfly_topology_t topo;
};
struct ChunkBatch {
  int rows_per_chunk;     // grid rows of one chunk (batch x kv heads x head parts)
  int nch;                // chunks in the batch
  int from_inputs;        // 1: every chunk starts on a page boundary; pages of the batch's own
                          // tokens come from the chunk inputs (else every page from the ring)
  ChunkArgs c[kMaxUpdateParts];
};
struct NoBatch {};

// Work unit = (batch, kv head, segment of seg_chunks 64-position chunks).
// Software pipeline per chunk c (even segments walk chunks upwards, odd ones
// downwards; see `dir`):
//   LDS <- staged page (K rows, V rows) and routed summary rows
//   barrier
//   issue global loads of the next chunk's page and summaries into registers
//   query heads in pairs: S^T = K Q^T for both heads from one K fragment read,
//     softmax, O^T = V^T P^T for both heads from one V fragment read; after a
//     head's scores its register Q slot is refilled with the next (chunk, head)
//   barrier
// so HBM traffic of chunk c+1 overlaps the MFMA/softmax work of chunk c.
//
// kUpd (the streaming prefill's fused launch): the grid carries extra rows of
// workgroups that run the NEXT chunk's cache update (append + pooling) while
// the attention workgroups run this chunk; the host fuses only when the update
// writes no ring slot or pool row that this chunk's attention reads.
template <int D, bool kUpd = false, bool kBatch = false, bool kSplitD = false>
__global__ void __launch_bounds__(MfmaCfg<D>::NTHR, D <= 128 || MfmaCfg<D>::kWaveHead ? 2 : 1)
attn_mfma_kernel(AttnArgs a_in, MfmaArgs m_in, int seg_chunks, int c_first_in, int nchunks_in, int hper,
                 std::conditional_t<kBatch, ChunkBatch, NoBatch> cb) {
  AttnArgs a = a_in;
  MfmaArgs m = m_in;
  int c_first = c_first_in, nchunks = nchunks_in;
  using C = MfmaCfg<D>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::LDS];
  __shared__ int cand_n[kSumSlots], cand_b[kSumSlots];
  __shared__ int s_nbr[kMaxSegBlocks * kMaxKcap];
  __bf16* Ks = reinterpret_cast<__bf16*>(smem);                 // [kSlots][KP]
  __bf16* Vs = reinterpret_cast<__bf16*>(smem + C::K_BYTES);    // [kSlots][D], pieces swizzled by row
  static_assert(C::LDS >= C::NTHR / 256 * 256 * 8 * 4, "pooling scratch aliases the staging tiles");
  if constexpr (kUpd) {
    // (the kernel argument itself, not the local copy: the job's part arrays are indexed at
    // run time, which would put a modified copy in scratch memory)
    // Each 256 threads of an update workgroup run one work item (kUpdPerWg per workgroup), with
    // their own pooling scratch; a group whose item is past the end exits (an exited wave no
    // longer counts at a barrier).
    const MfmaArgs& mu = m_in;
    if ((int)blockIdx.y >= mu.attn_y) {
      constexpr int kUpdPerWg = MfmaCfg<D>::NTHR / 256;
      const int grp = (int)threadIdx.x >> 8;
      const int64_t lin = ((int64_t)(blockIdx.y - mu.attn_y) * gridDim.x + blockIdx.x) * kUpdPerWg + grp;
      if (lin >= mu.upd_wgs) return;
      const int64_t per_kv = (int64_t)mu.upd_x * mu.upd_rows;
      const int kv = (int)(lin / per_kv);
      const int64_t r = lin - kv * per_kv;
      const int64_t row = r / mu.upd_x;
      cache_update_body<__bf16, 8>(mu.upd, r - row * mu.upd_x, row, kv, reinterpret_cast<float*>(smem) + grp * 256 * 8,
                                   (int)threadIdx.x & 255);
      return;
    }
  }

  int yrow = (int)blockIdx.y;
  int seg = xcd_remap(blockIdx.x, gridDim.x);
  if constexpr (kBatch) {
    // this workgroup's chunk (zc), row (batch x kv head x head part) and segment.  Workgroups
    // go to the 8 XCDs round-robin by linear id; when they divide evenly, each XCD takes a
    // contiguous run of the order (row, chunk, segment), so that a segment and the one before
    // it, whose last page is its halo, mostly share an L2 (the first segment of a chunk takes
    // its halo from the previous chunk's last).
    const int nsg = (int)gridDim.x, rpc = cb.rows_per_chunk;
    const int total = rpc * cb.nch * nsg;
    int zc;
    if (total % 8 == 0) {
      const int lin = (int)blockIdx.y * nsg + (int)blockIdx.x;
      const int ord = (lin & 7) * (total >> 3) + (lin >> 3);
      yrow = ord / (cb.nch * nsg);
      const int rem = ord - yrow * cb.nch * nsg;
      zc = rem / nsg;
      seg = rem - zc * nsg;
    } else {
      zc = yrow / rpc;
      yrow -= zc * rpc;
      seg = (int)blockIdx.x;
    }
    const ChunkArgs& ck = cb.c[zc];
    a.q = ck.q;
    a.out = ck.out;
    a.tq = ck.tq;
    a.topo = ck.topo;
    m.qlo = ck.qlo;
    m.qhi = ck.qhi;
    m.key_lo = ck.key_lo;
    m.kv_len = ck.kv_len;
    m.nsum = ck.nsum;
    m.nblocks = ck.nblocks;
    c_first = ck.c_first;
    nchunks = ck.nchunks;
  }

  constexpr int NTHR = C::NTHR, NWAVES = NTHR / 64;
  constexpr bool kWaveHead = C::kWaveHead;
  constexpr bool kFixed = C::kFixedPages;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lg = lane >> 4, lq = lane & 15;
  // query rows 16 qwave .. 16 qwave + 15 of each 64-position chunk; with kWaveHead, head
  // parity hpar (the wave takes heads hlo + hpar, hlo + hpar + 2, ...)
  const int qwave = kWaveHead ? (wave & 3) : wave;
  const int hpar = kWaveHead ? (wave >> 2) : 0;
  // small grids split a GQA group's heads over workgroups of hper heads each
  const int gsz = a.hq / a.hkv;
  const int nparts = (gsz + hper - 1) / hper;
  const int bh = yrow / nparts, hpart = yrow - bh * nparts;
  const int bi = bh / a.hkv;
  const int kvh = bh - bi * a.hkv;
  const int hlo = hpart * hper;
  const int hhi = min(gsz, hlo + hper);
  const int cbeg = c_first + seg * seg_chunks;
  const int cend = min(cbeg + seg_chunks, c_first + nchunks);
  if constexpr (kBatch) {
    if (cbeg >= cend) return;   // the grid's segments cover the batch's longest chunk
  }

  const int64_t kv_off = ((int64_t)bi * a.hkv + kvh) * a.kv_rows * D;
  const int64_t pool_off = ((int64_t)bi * a.hkv + kvh) * a.pool_rows * D;
  const __bf16* kbase = reinterpret_cast<const __bf16*>(a.k) + kv_off;
  const __bf16* vbase = reinterpret_cast<const __bf16*>(a.v) + kv_off;
  const __bf16* ksb = reinterpret_cast<const __bf16*>(a.ks) + pool_off;
  const __bf16* vsb = reinterpret_cast<const __bf16*>(a.vs) + pool_off;
  const float sl2 = a.scale * 1.4426950408889634f;   // host guarantees scale > 0

  auto blk_of = [&](int p) { return min(max(p / m.bs, 0), m.nblocks - 1); };
  auto chunk_blocks = [&](int c, int& bA, int& bB) {
    bA = blk_of(max(c * kPage, m.qlo));
    bB = blk_of(min((c + 1) * kPage, m.qhi) - 1);
  };

  // ---- neighbour rows of every query block of the segment, once, into LDS (see the
  // prologue below for when)
  int b_lo, b_hi, tmp;
  chunk_blocks(cbeg, b_lo, tmp);
  chunk_blocks(cend - 1, tmp, b_hi);
  auto build_rows = [&]() {
  if (a.nbr != nullptr) {
    const int cnt = (b_hi - b_lo + 1) * m.kcap;
    for (int i = tid; i < cnt; i += NTHR) s_nbr[i] = a.nbr[(int64_t)b_lo * m.kcap + i];
  } else {
    // the table builder's row (neighbor_row, bfly_block_neighbors), one wave per
    // block and one lane per row entry: lane j holds the j-th candidate of
    // [b, b-1..b-lwb, partners, sinks], a lane keeps it if no lower lane holds
    // the same block, and a ballot gives the kept entries their slots (first
    // occurrences in candidate order, cut at kcap, -1 padding)
    const bfly_topology_t& t = a.topo;
    const int lwb = t.local_window_blocks, np = t.partner_count;
    const int nsk = t.sink_count < m.nblocks ? t.sink_count : m.nblocks;
    const int kc = min(1 + lwb + np + nsk, 64);   // candidates past lane 63 lie beyond kcap (<= 8 here)
    const int jp = min(max(lane - 1 - lwb, 0), BFLY_MAX_PARTNERS - 1);
    int bit = 0;
#pragma unroll
    for (int jj = 0; jj < BFLY_MAX_PARTNERS; ++jj) bit = jj == jp ? t.partner_bits[jj] : bit;
    for (int bb = b_lo + wave; bb <= b_hi; bb += NWAVES) {
      int cand = -1;
      if (lane == 0) {
        cand = bb;
      } else if (lane <= lwb) {
        cand = bb - lane;
      } else if (lane <= lwb + np) {
        cand = (int)partner_block(bb, bit, m.nblocks, t.rule, t.width);
      } else if (lane < kc) {
        cand = lane - 1 - lwb - np;
      }
      if (cand < 0 || cand >= m.nblocks) cand = -1;
      bool keep = cand >= 0;
      for (int i = 0; i < kc; ++i) {
        const int ci = __builtin_amdgcn_readlane(cand, i);
        if (i < lane && ci == cand) keep = false;
      }
      const unsigned long long mask = __ballot(keep);
      const int slot = __popcll(mask & ((1ull << lane) - 1ull));
      int* row = s_nbr + (bb - b_lo) * m.kcap;
      if (keep && slot < m.kcap) row[slot] = cand;
      if (lane >= __popcll(mask) && lane < m.kcap) row[lane] = -1;
    }
  }
  };

  // ---- register staging of one page (K rows and V row pairs) and of the routed summaries
  uint4 kst[C::KLD], vst[C::KLD];
  // (into kst / vst, or the given registers)
  auto fetch_page_to = [&](int pg, uint4 (&kst)[C::KLD], uint4 (&vst)[C::KLD]) {
    const int p0 = pg * kPage;
    // row of position p0 (+ r): linear, or ring slot (ring >= kPage, so one wrap at most)
    int r0 = 0;
    if (m.ring) {
      r0 = p0 % m.ring;
      if (r0 < 0) r0 += m.ring;
    } else {
      r0 = p0 - m.key_lo;
    }
    auto rowp = [&](int r) {
      int rr = r0 + r;
      if (m.ring && rr >= m.ring) rr -= m.ring;
      return rr;
    };
    auto ok = [&](int p) { return p >= m.key_lo && p >= 0 && p < m.kv_len; };
    // Loads are unconditional (row 0 stands in for an invalid position) and the
    // value is zeroed afterwards, so no branch splits the load batch.
    auto ld = [&](const __bf16* base, int r, int pc) {
      const bool v = ok(p0 + r);
      const uint4 x = *reinterpret_cast<const uint4*>(base + (int64_t)(v ? rowp(r) : 0) * D + pc * 8);
      return v ? x : make_uint4(0, 0, 0, 0);
    };
    if constexpr (kBatch) {
      // A streaming batch whose chunks all start on a page boundary reads its own tokens (the
      // pages from its first chunk's on) from the chunk inputs: the cache update copies to the
      // ring only the tokens later steps read there.  Such a page lies in one chunk.
      if (cb.from_inputs && p0 >= cb.c[0].qlo) {
        // the chunk holding p0: selects over the slots (workgroup-uniform)
        const __bf16* kc = reinterpret_cast<const __bf16*>(cb.c[0].k);
        const __bf16* vc = reinterpret_cast<const __bf16*>(cb.c[0].v);
        int lo = cb.c[0].qlo, len = cb.c[0].tq;
#pragma unroll
        for (int j = 1; j < kMaxUpdateParts; ++j) {
          const bool in = j < cb.nch && p0 >= cb.c[j].qlo;
          kc = in ? reinterpret_cast<const __bf16*>(cb.c[j].k) : kc;
          vc = in ? reinterpret_cast<const __bf16*>(cb.c[j].v) : vc;
          lo = in ? cb.c[j].qlo : lo;
          len = in ? cb.c[j].tq : len;
        }
        // rows past the chunk's end are past kv_len (the attended chunk's end), so invalid
        const int64_t rb = (int64_t)bh * len + (p0 - lo);
        auto ldc = [&](const __bf16* base, int r, int pc) {
          const bool v = ok(p0 + r);
          const uint4 x = *reinterpret_cast<const uint4*>(base + (rb + (v ? r : 0)) * D + pc * 8);
          return v ? x : make_uint4(0, 0, 0, 0);
        };
#pragma unroll
        for (int it = 0; it < C::KLD; ++it) {
          const int i = tid + it * NTHR;
          kst[it] = ldc(kc, i / C::PIECES, i % C::PIECES);
        }
#pragma unroll
        for (int it = 0; it < C::KLD; ++it) {
          const int i = tid + it * NTHR;
          vst[it] = ldc(vc, i / C::PIECES, i % C::PIECES);
        }
        return;
      }
    }
#pragma unroll
    for (int it = 0; it < C::KLD; ++it) {
      const int i = tid + it * NTHR;
      kst[it] = ld(kbase, i / C::PIECES, i % C::PIECES);
    }
#pragma unroll
    for (int it = 0; it < C::KLD; ++it) {
      const int i = tid + it * NTHR;
      vst[it] = ld(vbase, i / C::PIECES, i % C::PIECES);
    }
  };
  auto fetch_page = [&](int pg) { fetch_page_to(pg, kst, vst); };
  // page pg into rows half * 64.. (kFixed) or (pg & 1) * 64..
  auto store_page_from = [&](int pg, int half, const uint4 (&kst)[C::KLD], const uint4 (&vst)[C::KLD]) {
    const int sbase = (kFixed ? half : (pg & 1)) * kPage;
#pragma unroll
    for (int it = 0; it < C::KLD; ++it) {
      const int i = tid + it * NTHR;
      const int r = i / C::PIECES, pc = i % C::PIECES;
      *reinterpret_cast<uint4*>(Ks + (sbase + r) * C::KP + pc * 8) = kst[it];
    }
#pragma unroll
    for (int it = 0; it < C::KLD; ++it) {
      const int i = tid + it * NTHR;
      const int r = sbase + i / C::PIECES, pc = i % C::PIECES;
      *reinterpret_cast<uint4*>(Vs + r * D + (pc ^ C::vswz(r)) * 8) = vst[it];
    }
  };
  auto store_page = [&](int pg, int half) { store_page_from(pg, half, kst, vst); };

  uint4 skst[C::SLD], svst[C::SLD];
  int scn[C::SLD], scb[C::SLD];
  // Summary candidates of chunk c: the s-th entry, over the chunk's query
  // blocks in order, of each block's routed neighbours n < block (n < nsum).
  auto fetch_sum = [&](int c) {
    int bA, bB;
    chunk_blocks(c, bA, bB);
#pragma unroll
    for (int it = 0; it < C::SLD; ++it) {
      const int i = tid + it * NTHR;
      const int s = i / C::PIECES, pc = i % C::PIECES;
      int cn = -1, cb = -1;
      if (i < C::SITEMS) {
        int cnt = 0;
        for (int bb = bA; bb <= bB && cn < 0; ++bb) {
          for (int j = 0; j < m.kcap; ++j) {
            const int n = s_nbr[(bb - b_lo) * m.kcap + j];
            if (n < 0 || n >= bb || n >= m.nsum) continue;
            if (cnt == s) {
              cn = n;
              cb = bb;
              break;
            }
            ++cnt;
          }
        }
      }
      scn[it] = cn;
      scb[it] = cb;
      const int64_t srow = (int64_t)(cn >= 0 ? cn : 0) * D + (i < C::SITEMS ? pc * 8 : 0);
      const uint4 kx = *reinterpret_cast<const uint4*>(ksb + srow);
      const uint4 vx = *reinterpret_cast<const uint4*>(vsb + srow);
      skst[it] = cn >= 0 ? kx : make_uint4(0, 0, 0, 0);
      svst[it] = cn >= 0 ? vx : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_sum = [&]() {
#pragma unroll
    for (int it = 0; it < C::SLD; ++it) {
      const int i = tid + it * NTHR;
      if (i >= C::SITEMS) continue;
      const int s = i / C::PIECES, pc = i % C::PIECES;
      *reinterpret_cast<uint4*>(Ks + (kRing + s) * C::KP + pc * 8) = skst[it];
      *reinterpret_cast<uint4*>(Vs + (kRing + s) * D + (pc ^ C::vswz(kRing + s)) * 8) = svst[it];
      if (pc == 0) {
        cand_n[s] = scn[it];
        cand_b[s] = scb[it];
      }
    }
  };

  // ---- register-resident Q fragments: lane holds query (chunk row wave*16+lq),
  // d in [lg*D/4, (lg+1)*D/4); k-step ks takes d = lg*D/4 + 8*ks + [0, 8)
  // (the K fragments use the same map, so the k permutation cancels).
  constexpr int QSLOTS = kWaveHead ? 1 : kQPipe;   // a wave-per-head wave holds one head's Q
  bf16x8 qbuf[QSLOTS][C::KSTEPS];
#pragma unroll
  for (int u = 0; u < QSLOTS; ++u)
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) qbuf[u][ks] = bf16x8{};
  const __bf16* qhead0 = reinterpret_cast<const __bf16*>(a.q) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz) * a.tq * D;
  auto load_q = [&](int u, int c, int hh) {
    const int qp = c * kPage + qwave * 16 + lq;
    const bool ok = qp >= m.qlo && qp < m.qhi;
    // Rows outside the query range read row 0 instead: their scores are masked
    // and their outputs are never stored.
    const __bf16* qrow = qhead0 + ((int64_t)hh * a.tq + (ok ? qp - m.qlo : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) qbuf[u][ks] = *reinterpret_cast<const bf16x8*>(qrow + lg * (D / 4) + 8 * ks);
  };
  // After head hh of chunk c used slot u = hh % kQPipe, refill it with the next
  // (chunk, head) that uses the slot.
  // Odd segments walk their chunks backwards: the page a segment shares with its
  // left neighbour (the neighbour's last page, the segment's halo) is then read by
  // both at about the same time, and the second read hits the XCD's L2.  Chunk c
  // needs pages c - 1 and c; the page it adds to the ring is c forwards, c - 1
  // backwards.
  const int dir = (seg & 1) ? -1 : 1;
  const int cfirst = dir > 0 ? cbeg : cend - 1;
  const int cstop = dir > 0 ? cend : cbeg - 1;
  auto new_page = [&](int c) { return dir > 0 ? c : c - 1; };
  auto refill_q = [&](int u, int c, int hh) {
    if constexpr (kWaveHead) {
      // this wave's next head: two on, or the first of its parity in the next chunk
      int nh = hh + 2, nc = c;
      if (nh >= hhi) {
        nh = hlo + hpar;
        nc = c + dir;
      }
      if (nc != cstop && nh < hhi) load_q(0, nc, nh);
    } else {
      int nh = hh + kQPipe, nc = c;
      if (nh >= hhi) {
        nh = hlo + u;
        nc = c + dir;
      }
      if (nc != cstop) load_q(u, nc, nh);
    }
  };

  // Split d (kSplitD; d = 256, a segment of one chunk and four query heads, as in the batched
  // streaming launches): each wave first scores its two heads (hlo + hpar, hlo + 2 + hpar) and forms their P
  // and 1/l; once every wave is done with K, the waves of a pair (same rows, hpar 0 and 1) trade
  // their P and 1/l through the K rows, and each computes PV and the output for all four heads
  // on its half of d (hpar): every V fragment read then feeds four heads instead of one.  Each
  // output element is the same MFMA chain over the same operands as in the head-per-wave form.
  // (kSplitD: the host launches it only for segments of one chunk and workgroups of four heads)
  static_assert(!kSplitD || kWaveHead, "split d is the d = 256 form");
  if constexpr (kWaveHead) {
    if (hlo + hpar < hhi) load_q(0, cfirst, hlo + hpar);
  } else {
#pragma unroll
    for (int u = 0; u < kQPipe; ++u)
      if (hlo + u < hhi) load_q(u, cfirst, hlo + u);
  }
  if constexpr (kFixed) {
    // both pages of the first chunk requested together, then the rows built while they are in
    // flight (walking forwards, the first page is the chunk's halo; backwards, its own page)
    uint4 k0[C::KLD], v0[C::KLD];
    fetch_page_to(dir > 0 ? cbeg - 1 : cend - 1, k0, v0);
    fetch_page(new_page(cfirst));
    build_rows();
    store_page_from(dir > 0 ? cbeg - 1 : cend - 1, dir > 0 ? 0 : 1, k0, v0);
  } else {
    // the rows are built while the first page is in flight
    fetch_page(dir > 0 ? cbeg - 1 : cend - 1);
    build_rows();
    store_page(dir > 0 ? cbeg - 1 : cend - 1, 0);
    fetch_page(new_page(cfirst));
  }
  __syncthreads();   // s_nbr visible
  fetch_sum(cfirst);

  __bf16* ohead0 = reinterpret_cast<__bf16*>(a.out) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz) * a.tq * D;
  // kFixed: per-lane bases (elements) of the fragments a wave reads.  K: row 16 qwave + lq of
  // the window tiles (tile t adds 16 t rows), row 128 + lq of the summary tile, at d
  // lg * D / 4.  V (transposing reads): rows 16 qwave + 4 lg + (lq >> 2) and 128 + ..., at the
  // 8-byte unit mt * 8 + (lq & 3) * 2 + half XOR the rows' swizzle ((lq >> 2) & 3) * 8, which is
  // vr[mt & 3] + (mt >> 2) * 128 + half * 4 elements.
  int klane = 0, ksum = 0, vlane[4] = {0, 0, 0, 0}, vsum[4] = {0, 0, 0, 0};
  if constexpr (kFixed) {
    klane = (16 * qwave + lq) * C::KP + lg * (D / 4);
    ksum = (kRing + lq) * C::KP + lg * (D / 4);
    const int x = (lq >> 2) & 3;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int vr = (r ^ x) * 32 + (lq & 3) * 8;
      vlane[r] = (16 * qwave + 4 * lg + (lq >> 2)) * D + vr;
      vsum[r] = (kRing + 4 * lg + (lq >> 2)) * D + vr;
    }
  }

  for (int c = cfirst; c != cstop; c += dir) {
    if constexpr (kFixed) {
      // the page this chunk shares with the previous one moves to its place: forwards the old
      // own page becomes the halo (rows 64.. -> 0..), backwards the old halo the own page
      if (c != cfirst) {
        const int src = dir > 0 ? kPage : 0, dst = kPage - src;
        // (a native vector type: arrays of HIP's uint4 struct stay in scratch memory)
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        u32x4 kx[C::KLD], vx[C::KLD];
#pragma unroll
        for (int it = 0; it < C::KLD; ++it) {
          const int i = tid + it * NTHR;
          const int r = i / C::PIECES, pc = i % C::PIECES;
          kx[it] = *reinterpret_cast<const u32x4*>(Ks + (src + r) * C::KP + pc * 8);
          vx[it] = *reinterpret_cast<const u32x4*>(Vs + (src + r) * D + pc * 8);   // same swizzle 64 rows on
        }
#pragma unroll
        for (int it = 0; it < C::KLD; ++it) {
          const int i = tid + it * NTHR;
          const int r = i / C::PIECES, pc = i % C::PIECES;
          *reinterpret_cast<u32x4*>(Ks + (dst + r) * C::KP + pc * 8) = kx[it];
          *reinterpret_cast<u32x4*>(Vs + (dst + r) * D + pc * 8) = vx[it];
        }
        __syncthreads();   // every copy read before the new page lands on its source rows
      }
    }
    store_page(new_page(c), dir > 0 ? 1 : 0);
    store_sum();
    __syncthreads();
    if (!kSplitD && c + dir != cstop) {
      fetch_page(new_page(c + dir));
      fetch_sum(c + dir);
    }

    // ---------------- per-lane state shared by every head: wave owns positions [pw, pw+16)
    const int pw = c * kPage + qwave * 16;
    const int qp = pw + lq;                          // this lane's query position
    const bool wave_active = (pw + 15 >= m.qlo) && (pw < m.qhi);
    const bool row_ok = qp >= m.qlo && qp < m.qhi;
    const int qblk = blk_of(qp);
    const int qcut = max(0, (m.token_cutoff ? qp : qblk * m.bs) - m.W + 1);
    const int wlo = max(max(qp - m.W + 1, m.key_lo), 0);
    // ok[t][i]: key 4*lg+i of tile t (window tiles 0..4 start at pw-64; tile 5 = summaries)
    bool ok[6][4];
#pragma unroll
    for (int t = 0; t < 5; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kp = pw - kPage + 16 * t + 4 * lg + i;
        ok[t][i] = row_ok && kp >= wlo && kp <= qp;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int s = 4 * lg + i;
      const int n = cand_n[s];
      ok[5][i] = row_ok && n >= 0 && cand_b[s] == qblk && (n + 1) * m.bs <= qcut;
    }
    int slot[6];
#pragma unroll
    for (int t = 0; t < 5; ++t) slot[t] = kFixed ? 16 * (qwave + t) : (pw - kPage + 16 * t) & (kRing - 1);
    slot[5] = kRing;

    // softmax of one head's 24 scores (already masked to -inf) -> bf16 P, 1/l
    auto softmax = [&](f32x4 (&st)[6], bf16x8 (&pf)[3], float& inv) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 6; ++t) mx = fmaxf(mx, fmaxf(fmaxf(st[t][0], st[t][1]), fmaxf(st[t][2], st[t][3])));
      mx = col_max4(mx);
      const float nm = mx == -INFINITY ? 0.f : -mx * sl2;
      float lsum = 0.f;
#pragma unroll
      for (int t = 0; t < 6; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __builtin_amdgcn_exp2f(fmaf(st[t][i], sl2, nm));
          lsum += e;
          pf[t / 2][(t % 2) * 4 + i] = (__bf16)e;
        }
      lsum = col_sum4(lsum);
      inv = __builtin_amdgcn_rcpf(fmaxf(lsum, 1e-30f));
    };

    if constexpr (kSplitD) {
      {
        bf16x8 pa[2][3];
        float inva[2] = {0.f, 0.f};
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          if (!wave_active) continue;
          f32x4 st[6];
#pragma unroll
          for (int t = 0; t < 6; ++t) {
            bf16x8 kf[C::KSTEPS];
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks)
              kf[ks] = *reinterpret_cast<const bf16x8*>(Ks + (t < 5 ? klane + 16 * t * C::KP : ksum) + 8 * ks);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qbuf[0][ks], acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) st[t][i] = ok[t][i] ? acc[i] : -INFINITY;
          }
          refill_q(0, c, hlo + 2 * it + hpar);   // the second head's Q, loaded during the first's softmax
          softmax(st, pa[it], inva[it]);
        }
        __syncthreads();   // every wave is done with K: its rows take the exchange
        // [wave pair slot qwave * 2 + hpar][it][pr][lane] P pieces, then [slot][it][lane] 1/l
        constexpr int kXP = 8 * 2 * 3 * 64 * 16;
        static_assert(kXP + 8 * 2 * 64 * 4 <= C::K_BYTES, "the exchange fits the K rows");
        bf16x8* xp = reinterpret_cast<bf16x8*>(smem);
        float* xi = reinterpret_cast<float*>(smem + kXP);
        const int me = qwave * 2 + hpar, mate = qwave * 2 + (hpar ^ 1);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
#pragma unroll
          for (int pr = 0; pr < 3; ++pr) xp[((me * 2 + it) * 3 + pr) * 64 + lane] = pa[it][pr];
          xi[(me * 2 + it) * 64 + lane] = inva[it];
        }
        __syncthreads();   // both waves of every pair have published
        if (wave_active) {
          // this wave's half of d: tiles mt = 4 hpar .. 4 hpar + 3, i.e. the V bases plus hpar * 128
          int vlh[4], vsh[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            vlh[r] = vlane[r] + hpar * 128;
            vsh[r] = vsum[r] + hpar * 128;
          }
          const bool lo8 = lq < 8;
          const int pA = pw + (lq & 7), pB = pA + 8;
          const bool okA = pA >= m.qlo && pA < m.qhi, okB = pB >= m.qlo && pB < m.qhi;
          __bf16* oA = ohead0 + (int64_t)(okA ? pA - m.qlo : 0) * D;
          __bf16* oB = ohead0 + (int64_t)(okB ? pB - m.qlo : 0) * D;
          const int64_t hstride = (int64_t)a.tq * D;
          // two passes of a head pair: (hlo + 2 it + hpar, own) and (hlo + 2 it + (hpar ^ 1), mate's)
#pragma unroll
          for (int it = 0; it < 2; ++it) {
            bf16x8 pf[2][3];
            float inv[2];
#pragma unroll
            for (int pr = 0; pr < 3; ++pr) {
              pf[0][pr] = pa[it][pr];
              pf[1][pr] = xp[((mate * 2 + it) * 3 + pr) * 64 + lane];
            }
            inv[0] = inva[it];
            inv[1] = xi[(mate * 2 + it) * 64 + lane];
            const int64_t ho[2] = {(hlo + 2 * it + hpar) * hstride, (hlo + 2 * it + (hpar ^ 1)) * hstride};
#pragma unroll
            for (int mpi = 0; mpi < 2; ++mpi) {
              bf16x8 w[2][2];
#pragma unroll
              for (int sub = 0; sub < 2; ++sub) {
                const int r = 2 * mpi + sub;   // mt & 3 (mt = 4 hpar + r)
                f32x4 o[2][2];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                  bf16x8 vf[3];
#pragma unroll
                  for (int pr = 0; pr < 3; ++pr) {
                    const int ta = 2 * pr, tb = 2 * pr + 1;
                    const bf16x4 va = read_tr(Vs + vlh[r] + 16 * ta * D + half * 4);
                    const bf16x4 vb = read_tr(Vs + (tb < 5 ? vlh[r] + 16 * tb * D : vsh[r]) + half * 4);
                    vf[pr] = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
                  }
#pragma unroll
                  for (int jh = 0; jh < 2; ++jh) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int pr = 0; pr < 3; ++pr)
                      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[pr], pf[jh][pr], acc, 0, 0, 0);
                    o[jh][half] = acc;
                  }
                }
#pragma unroll
                for (int jh = 0; jh < 2; ++jh)
#pragma unroll
                  for (int i = 0; i < 4; ++i) {
                    w[jh][sub][i] = (__bf16)(o[jh][0][i] * inv[jh]);
                    w[jh][sub][4 + i] = (__bf16)(o[jh][1][i] * inv[jh]);
                  }
              }
              // whole 128-byte lines per store, as in the head-per-wave form (mp = 2 hpar + mpi)
              const int dA = (4 * hpar + 2 * mpi + (lo8 ? 0 : 1)) * 32 + lg * 8;
#pragma unroll
              for (int jh = 0; jh < 2; ++jh) {
                const bf16x8 x = xchg8(lo8 ? w[jh][1] : w[jh][0]);
                const bf16x8 sa = lo8 ? w[jh][0] : x, sb = lo8 ? x : w[jh][1];
                if (okA) __builtin_nontemporal_store(sa, reinterpret_cast<bf16x8*>(oA + ho[jh] + dA));
                if (okB) __builtin_nontemporal_store(sb, reinterpret_cast<bf16x8*>(oB + ho[jh] + dA));
              }
            }
          }
        }
        break;   // the segment's only chunk (no page or Q is carried over)
      }
    }
    for (int hb = hlo; hb < hhi && !kSplitD; hb += kQPipe) {
#pragma unroll
      for (int pp = 0; pp < kQPipe / 2; ++pp) {
        // kWaveHead: this wave's head of the pair alone, in Q slot 0
        const int h0 = kWaveHead ? hb + hpar : hb + 2 * pp;
        if (h0 >= hhi) break;
        const bool two = !kWaveHead && h0 + 1 < hhi;
        const int u0 = kWaveHead ? 0 : 2 * pp, u1 = kWaveHead ? 0 : 2 * pp + 1;
        if (!wave_active) {
          refill_q(u0, c, h0);
          if (two) refill_q(u1, c, h0 + 1);
          continue;
        }
        auto pair_body = [&](auto two_tag) {
          constexpr bool kTwo = decltype(two_tag)::value;
          // S^T for both heads; one K fragment read feeds two MFMAs.  For d = 256 a
          // pair with one head (an odd group, or one head per workgroup) runs the
          // kTwo = false copy of this body, which issues no MFMA for the missing
          // head; smaller d keep one copy (registers), where the second head of
          // such a pair is computed on a stale Q slot and discarded.
          f32x4 s0[6], s1[6];
  #pragma unroll
          for (int t = 0; t < 6; ++t) {
            bf16x8 kf[C::KSTEPS];
  #pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks)
              kf[ks] = *reinterpret_cast<const bf16x8*>(
                  kFixed ? Ks + (t < 5 ? klane + 16 * t * C::KP : ksum) + 8 * ks
                         : Ks + (slot[t] + lq) * C::KP + lg * (D / 4) + 8 * ks);
            f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks) {
              a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qbuf[u0][ks], a0, 0, 0, 0);
              if constexpr (kTwo) a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qbuf[u1][ks], a1, 0, 0, 0);
            }
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              s0[t][i] = ok[t][i] ? a0[i] : -INFINITY;
              if constexpr (kTwo) s1[t][i] = ok[t][i] ? a1[i] : -INFINITY;
            }
          }
          refill_q(u0, c, h0);
          if (kTwo && two) refill_q(u1, c, h0 + 1);
          bf16x8 p0[3], p1[3];
          float inv0, inv1 = 0.f;
          softmax(s0, p0, inv0);
          if constexpr (kTwo) softmax(s1, p1, inv1);
          // O^T = V^T P^T.  Tile (mt, half), row r holds d = mt*32 + (r/4)*8 + half*4 + r%4,
          // so the two halves give each lane 8 consecutive d (16 bytes) of its position.
          // The V^T fragments come from row-major V by transposing reads: lane (lg, lq)
          // reads the 4 d (8 bytes) mt*32 + (lq&3)*8 + half*4 of key row
          // slot + 4lg + (lq>>2), so lane lq of the group receives d row lq's four keys
          // slot + 4lg + 0..3, the order of its P fragment.
          // Tiles mt and mt+1 together hold d [mt*32, mt*32+64) = one 128-byte line per
          // position.  Lanes lq and lq^8 swap one 16-byte piece so that each store
          // instruction writes 8 whole lines (positions 0..7, then 8..15): whole-line
          // non-temporal stores stream to HBM at full rate, half lines do not.
          const bool lo8 = lq < 8;
          const int pA = pw + (lq & 7), pB = pA + 8;        // positions of the two store passes
          const bool okA = pA >= m.qlo && pA < m.qhi, okB = pB >= m.qlo && pB < m.qhi;
          __bf16* oA0 = ohead0 + ((int64_t)h0 * a.tq + (okA ? pA - m.qlo : 0)) * D;
          __bf16* oB0 = ohead0 + ((int64_t)h0 * a.tq + (okB ? pB - m.qlo : 0)) * D;
          const int64_t hstride = (int64_t)a.tq * D;
  #pragma unroll
          for (int mp = 0; mp < C::DTILES / 4; ++mp) {
            bf16x8 w0[2], w1[2];
  #pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
              const int mt = 2 * mp + sub;
              f32x4 o0[2], o1[2];
  #pragma unroll
              for (int half = 0; half < 2; ++half) {
                const int unit = mt * 8 + (lq & 3) * 2 + half;   // 8-byte unit of the row
                bf16x8 vf[3];
  #pragma unroll
                for (int pr = 0; pr < 3; ++pr) {
                  const int ra = slot[2 * pr] + 4 * lg + (lq >> 2), rb = slot[2 * pr + 1] + 4 * lg + (lq >> 2);
                  // kFixed: rows 16 (qwave + t) + 4 lg + (lq >> 2) (t < 5) or 128 + ..., whose
                  // swizzle is the lane's (lq >> 2) & 3; unit ^ that swizzle is then
                  // ((mt ^ x) * 8 + low bits) with x = (lq >> 2) & 3, i.e. vr[mt & 3] + (mt >> 2) * 128
                  const int tail = (mt >> 2) * 128 + half * 4;
                  const int ta = 2 * pr, tb = 2 * pr + 1;
                  const bf16x4 va = read_tr(kFixed ? Vs + vlane[mt & 3] + 16 * ta * D + tail
                                                   : Vs + ra * D + (unit ^ (2 * C::vswz(ra))) * 4);
                  const bf16x4 vb = read_tr(kFixed ? Vs + (tb < 5 ? vlane[mt & 3] + 16 * tb * D : vsum[mt & 3]) + tail
                                                   : Vs + rb * D + (unit ^ (2 * C::vswz(rb))) * 4);
                  vf[pr] = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
                }
                f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
                for (int pr = 0; pr < 3; ++pr) {
                  a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[pr], p0[pr], a0, 0, 0, 0);
                  if constexpr (kTwo) a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[pr], p1[pr], a1, 0, 0, 0);
                }
                o0[half] = a0;
                o1[half] = a1;
              }
  #pragma unroll
              for (int i = 0; i < 4; ++i) {
                w0[sub][i] = (__bf16)(o0[0][i] * inv0);
                w0[sub][4 + i] = (__bf16)(o0[1][i] * inv0);
                if constexpr (kTwo) {
                  w1[sub][i] = (__bf16)(o1[0][i] * inv1);
                  w1[sub][4 + i] = (__bf16)(o1[1][i] * inv1);
                }
              }
            }
            // lanes lq < 8 keep tile mt (sub 0) and receive the partner's tile mt;
            // lanes lq >= 8 keep tile mt+1 (sub 1) and receive the partner's tile mt+1
            const bf16x8 x0 = xchg8(lo8 ? w0[1] : w0[0]);
            const int dA = (2 * mp + (lo8 ? 0 : 1)) * 32 + lg * 8;   // d of this lane's piece
            const bf16x8 a0 = lo8 ? w0[0] : x0, b0 = lo8 ? x0 : w0[1];
            // O is written once and never re-read here: non-temporal stores keep it
            // from evicting the K/V pages and Q rows still in flight from L2.
            if (okA) __builtin_nontemporal_store(a0, reinterpret_cast<bf16x8*>(oA0 + dA));
            if (okB) __builtin_nontemporal_store(b0, reinterpret_cast<bf16x8*>(oB0 + dA));
            if constexpr (kTwo) {
              const bf16x8 x1 = xchg8(lo8 ? w1[1] : w1[0]);
              const bf16x8 a1 = lo8 ? w1[0] : x1, b1 = lo8 ? x1 : w1[1];
              if (two && okA) __builtin_nontemporal_store(a1, reinterpret_cast<bf16x8*>(oA0 + hstride + dA));
              if (two && okB) __builtin_nontemporal_store(b1, reinterpret_cast<bf16x8*>(oB0 + hstride + dA));
            }
          }
        };
        if constexpr (kWaveHead) {
          pair_body(std::false_type{});
        } else {
          pair_body(std::true_type{});
        }
      }
    }
    __syncthreads();
  }
}

// One attention launch: the MFMA kernel where its conditions hold, else the fp32 tile kernel
// or the generic one.
static int launch_attention(const AttnArgs& a, int dtype, hipStream_t stream, const char* what) {
  BFLY_CHECK_ARG(aligned16(a.q) && aligned16(a.out) && aligned16(a.k) && aligned16(a.v) && aligned16(a.ks) &&
                     aligned16(a.vs),
                 "%s: tensor pointers must be 16-byte aligned", what);
  const bool contiguous = a.qpos == nullptr;
  // The MFMA kernel keeps positions in int32 and assumes a positive scale (it
  // folds the scale into exp2) and a ring of at least one page.
  const bool mfma_ok = dtype == BFLY_DTYPE_BF16 && contiguous && a.W <= kPage && a.bs >= kPage &&
                       2 * a.kcap <= kSumSlots && (a.d == 64 || a.d == 128 || a.d == 256) && a.scale > 0.f &&
                       (a.ring == 0 || a.ring >= kPage) && a.kv_len + 2 * kPage < INT32_MAX &&
                       a.nblocks < INT32_MAX && a.kv_rows < INT32_MAX && a.pool_rows < INT32_MAX;
  if (a.tq == 0) return BFLY_OK;
  BFLY_CHECK_ARG(mfma_ok || a.nbr != nullptr, "%s: neighbour rows from the topology need the MFMA path", what);
  if (mfma_ok) {
    const int64_t c_first = floordiv(a.q_pos0, kPage);
    const int64_t c_last = floordiv(a.q_pos0 + a.tq - 1, kPage);
    const int64_t nchunks = c_last - c_first + 1;
    // Segment length: aim for >= 2 resident workgroups per CU (256 CUs) while
    // keeping the halo page (re-read once per segment) a small fraction.
    const int64_t groups = a.batch * a.hkv;
    int seg = 1;
    while (seg < kMaxSegChunks && (nchunks + 2 * seg - 1) / (2 * seg) * groups >= 512) seg *= 2;
    // Tuning override (chunks per workgroup): BFLY_PREFILL_SEG in {1, 2, 4, 8}.
    static const int seg_env = [] {
      const char* e = getenv("BFLY_PREFILL_SEG");
      const int v = e ? atoi(e) : 0;
      return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
    }();
    if (seg_env) seg = seg_env;
    int64_t nseg = (nchunks + seg - 1) / seg;
    BFLY_CHECK_ARG(nseg <= INT32_MAX && groups <= 65535, "%s: grid too large", what);
    MfmaArgs m{};
    m.qlo = (int)a.q_pos0;
    m.qhi = (int)(a.q_pos0 + a.tq);
    m.key_lo = (int)a.key_lo;
    m.kv_len = (int)a.kv_len;
    m.ring = (int)a.ring;
    m.nblocks = (int)a.nblocks;
    m.nsum = (int)(a.nsum < a.nblocks ? a.nsum : a.nblocks);
    m.kcap = a.kcap;
    m.bs = a.bs;
    m.W = a.W;
    m.token_cutoff = a.token_cutoff;
    // Head split: a grid far below the resident capacity (e.g. one 384-query chunk)
    // spreads the group's head pairs over more workgroups (each reloads the small
    // K/V pages); results are unchanged, every head is computed the same way.
    const int64_t capacity = a.d <= 128 ? 512 : 256;
    const int gsz = a.hq / a.hkv;
    int hsplit = 1;
    while (hsplit < gsz && nseg * groups * hsplit * 2 <= capacity) hsplit *= 2;
    // heads per workgroup: whole pairs while there are two or more, else one
    // (the pair's second MFMA column then runs on a stale slot and is dropped)
    const int hq_per = (gsz + hsplit - 1) / hsplit;
    const int hper = hq_per >= 2 ? (hq_per + 1) & ~1 : 1;
    const int nparts = (gsz + hper - 1) / hper;
    BFLY_CHECK_ARG(groups * nparts <= 65535, "%s: grid too large", what);
    dim3 grid((unsigned)nseg, (unsigned)(groups * nparts));
    switch (a.d) {
      case 64: hipLaunchKernelGGL(attn_mfma_kernel<64>, grid, dim3(256), 0, stream, a, m, seg, (int)c_first, (int)nchunks, hper, NoBatch{}); break;
      case 128: hipLaunchKernelGGL(attn_mfma_kernel<128>, grid, dim3(256), 0, stream, a, m, seg, (int)c_first, (int)nchunks, hper, NoBatch{}); break;
      default: hipLaunchKernelGGL(attn_mfma_kernel<256>, grid, dim3(MfmaCfg<256>::NTHR), 0, stream, a, m, seg, (int)c_first, (int)nchunks, hper, NoBatch{}); break;
    }
  } else if (dtype == BFLY_DTYPE_F32 && contiguous && a.nbr != nullptr && a.W <= 64 && a.bs % 16 == 0 &&
             a.hq / a.hkv <= 4 &&
             (a.d == 64 || a.d == 128) && a.kcap >= 1 && a.kcap <= kF32MaxKcap &&
             a.kv_len + 2 * kF32Rows < (1 << 30) && a.ring < (1 << 30) && a.nblocks >= 1 &&
             a.nblocks * (int64_t)a.bs < (1 << 30) &&
             a.q_pos0 >= 0 && a.q_pos0 + a.tq < (1 << 30) && a.pool_rows > 0) {
    const int64_t tile0 = floordiv(a.q_pos0, 16);
    const int64_t ntiles = floordiv(a.q_pos0 + a.tq - 1, 16) - tile0 + 1;
    const int64_t items = ntiles * a.batch * a.hkv;
    const int64_t per_xcd = (items + 7) / 8;
    BFLY_CHECK_ARG(8 * per_xcd <= INT32_MAX, "%s: grid too large", what);
    const dim3 grid((unsigned)(8 * per_xcd));
    if (a.d == 64)
      hipLaunchKernelGGL(attn_f32_tile_kernel<64>, grid, dim3(256), 0, stream, a, (int)tile0, (int)ntiles, (int)per_xcd);
    else
      hipLaunchKernelGGL(attn_f32_tile_kernel<128>, grid, dim3(256), 0, stream, a, (int)tile0, (int)ntiles, (int)per_xcd);
  } else {
    BFLY_CHECK_ARG(a.d <= kGenericMaxD, "%s: head_dim=%d > %d", what, a.d, kGenericMaxD);
    BFLY_CHECK_ARG(a.W + a.kcap <= kGenericMaxKeys, "%s: window + kcap > %d", what, kGenericMaxKeys);
    BFLY_CHECK_ARG(a.kcap <= 64, "%s: kcap > 64", what);
    BFLY_CHECK_ARG(a.tq <= INT32_MAX && a.batch * a.hkv <= 65535, "%s: grid too large", what);
    dim3 grid((unsigned)a.tq, (unsigned)(a.batch * a.hkv));
    const size_t lds = generic_lds_bytes(a.d, a.W, a.kcap);
    if (dtype == BFLY_DTYPE_F32)
      hipLaunchKernelGGL(attn_generic_kernel<float>, grid, dim3(64), lds, stream, a);
    else
      hipLaunchKernelGGL(attn_generic_kernel<__bf16>, grid, dim3(64), lds, stream, a);
  }
  BFLY_CHECK_LAUNCH(what);
  return BFLY_OK;
}

// The attention of n (<= kMaxUpdateParts) consecutive streaming chunks in one launch (MFMA
// path, neighbour rows from each chunk's topology): ch[j] holds chunk j's arguments as
// bfly_stream_chunks builds them for a launch of its own; they differ only in the query range,
// q / out and the cache state.  Optionally with a cache update on extra grid rows.  The grid
// shape follows launch_attention's rules for the whole batch.
static int launch_attention_batch(const AttnArgs* ch, const void* const* kin, const void* const* vin, int n,
                                  bool from_inputs, hipStream_t stream, const char* what,
                                  const UpdateJob* upd = nullptr, int64_t upd_rows = 0) {
  BFLY_CHECK_ARG(n >= 1 && n <= kMaxUpdateParts, "%s: batch of %d chunks", what, n);
  const AttnArgs& a = ch[0];
  ChunkBatch cb{};
  cb.nch = n;
  cb.from_inputs = from_inputs ? 1 : 0;
  int64_t nch_max = 0;
  for (int j = 0; j < n; ++j) {
    const AttnArgs& c = ch[j];
    BFLY_CHECK_ARG(aligned16(c.q) && aligned16(c.out) && aligned16(kin[j]) && aligned16(vin[j]),
                   "%s: tensor pointers must be 16-byte aligned", what);
    BFLY_CHECK_ARG(c.tq > 0 && c.nbr == nullptr && c.qpos == nullptr, "%s: chunk %d arguments", what, j);
    // consecutive chunks: chunk j's keys are positions [q_pos0, q_pos0 + tq), the next one's follow
    BFLY_CHECK_ARG(j == 0 || c.q_pos0 == ch[j - 1].q_pos0 + ch[j - 1].tq, "%s: chunk %d not consecutive", what, j);
    BFLY_CHECK_ARG(!from_inputs || c.q_pos0 % kPage == 0, "%s: chunk %d off the page grid", what, j);
    const int64_t cf = floordiv(c.q_pos0, kPage);
    const int64_t nc = floordiv(c.q_pos0 + c.tq - 1, kPage) - cf + 1;
    nch_max = nc > nch_max ? nc : nch_max;
    ChunkArgs& k = cb.c[j];
    k.q = c.q;
    k.out = c.out;
    k.k = kin[j];
    k.v = vin[j];
    k.tq = (int)c.tq;
    k.qlo = (int)c.q_pos0;
    k.qhi = (int)(c.q_pos0 + c.tq);
    k.key_lo = (int)c.key_lo;
    k.kv_len = (int)c.kv_len;
    k.nsum = (int)(c.nsum < c.nblocks ? c.nsum : c.nblocks);
    k.nblocks = (int)c.nblocks;
    k.c_first = (int)cf;
    k.nchunks = (int)nc;
    k.topo = c.topo;
  }
  const int64_t groups = a.batch * a.hkv;
  int seg = 1;
  while (seg < kMaxSegChunks && (nch_max + 2 * seg - 1) / (2 * seg) * groups * n >= 512) seg *= 2;
  const int64_t nseg = (nch_max + seg - 1) / seg;
  const int64_t capacity = a.d <= 128 ? 512 : 256;
  const int gsz = a.hq / a.hkv;
  int hsplit = 1;
  while (hsplit < gsz && nseg * groups * n * hsplit * 2 <= capacity) hsplit *= 2;
  const int hq_per = (gsz + hsplit - 1) / hsplit;
  const int hper = hq_per >= 2 ? (hq_per + 1) & ~1 : 1;
  const int nparts = (gsz + hper - 1) / hper;
  cb.rows_per_chunk = (int)(groups * nparts);
  // d = 256 workgroups of one chunk and four heads: the split-d form of the kernel
  const bool splitd = a.d == 256 && seg == 1 && hper == 4 && gsz % 4 == 0;
  BFLY_CHECK_ARG(nseg <= INT32_MAX && groups * nparts * n <= 65535, "%s: grid too large", what);
  MfmaArgs m{};
  m.ring = (int)a.ring;
  m.kcap = a.kcap;
  m.bs = a.bs;
  m.W = a.W;
  m.token_cutoff = a.token_cutoff;
  dim3 grid((unsigned)nseg, (unsigned)(groups * nparts * n));
  if (upd != nullptr) {
    const int64_t ux = update_x(upd->n_blocks, upd->step - upd->append_from, upd->d, 8);
    m.upd = *upd;
    m.attn_y = (int)grid.y;
    m.upd_x = (int)ux;
    m.upd_rows = (int)upd_rows;
    m.upd_wgs = ux * upd_rows * 2;   // work items; a d = 256 workgroup (512 threads) runs two
    const int64_t per_wg = a.d == 256 ? MfmaCfg<256>::NTHR / 256 : 1;
    const int64_t extra = ((m.upd_wgs + per_wg - 1) / per_wg + nseg - 1) / nseg;
    BFLY_CHECK_ARG(ux <= INT32_MAX && upd_rows <= 65535 && grid.y + extra <= 65535, "%s: grid too large", what);
    grid.y += (unsigned)extra;
    switch (a.d) {
      case 64: hipLaunchKernelGGL((attn_mfma_kernel<64, true, true>), grid, dim3(256), 0, stream, a, m, seg, 0, 0, hper, cb); break;
      case 128: hipLaunchKernelGGL((attn_mfma_kernel<128, true, true>), grid, dim3(256), 0, stream, a, m, seg, 0, 0, hper, cb); break;
      default:
        if (splitd)
          hipLaunchKernelGGL((attn_mfma_kernel<256, true, true, true>), grid, dim3(MfmaCfg<256>::NTHR), 0, stream, a, m, seg, 0, 0, hper, cb);
        else
          hipLaunchKernelGGL((attn_mfma_kernel<256, true, true>), grid, dim3(MfmaCfg<256>::NTHR), 0, stream, a, m, seg, 0, 0, hper, cb);
        break;
    }
  } else {
    switch (a.d) {
      case 64: hipLaunchKernelGGL((attn_mfma_kernel<64, false, true>), grid, dim3(256), 0, stream, a, m, seg, 0, 0, hper, cb); break;
      case 128: hipLaunchKernelGGL((attn_mfma_kernel<128, false, true>), grid, dim3(256), 0, stream, a, m, seg, 0, 0, hper, cb); break;
      default:
        if (splitd)
          hipLaunchKernelGGL((attn_mfma_kernel<256, false, true, true>), grid, dim3(MfmaCfg<256>::NTHR), 0, stream, a, m, seg, 0, 0, hper, cb);
        else
          hipLaunchKernelGGL((attn_mfma_kernel<256, false, true>), grid, dim3(MfmaCfg<256>::NTHR), 0, stream, a, m, seg, 0, 0, hper, cb);
        break;
    }
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

// Streaming chunked prefill of one layer over a two-pool cache, host loop in C++
// (the per-chunk work of ButterflyAttentionCore with a CompressedKVCache:
// bna/integrations/qwen_mlx.py:1515-1581 over bna/mlx/compressed_cache.py:94-172).
// Per chunk: the counter bookkeeping of update_and_fetch (append, summarise every
// block with end + W_cache <= offset, trim whole blocks while
// tail_size - BS >= max(W_cache, step + W_cache - 1)), the cache update (append +
// pooling of the due blocks), the layout of the live kv_len (bfly_topology_init;
// the attention kernel builds the neighbour rows itself), and the attention of the
// chunk's queries from the cache -- the same kernels and arguments as the
// per-chunk path.  Chunk c's attention and chunk c+1's update share one launch
// when they touch disjoint ring slots and pool rows: the update writes positions
// [P, P + len_{c+1}) (P = end of chunk c) and pool rows >= the summaries chunk c
// reads, while chunk c's attention reads pages no lower than P - len_c - 2*64,
// so len_c + len_{c+1} + 2*64 <= ring capacity keeps them apart.
namespace {

struct StreamCounters {
  int64_t offset, tail, count, sum_off;
};

struct PlannedUpdate {
  UpdateJob job;
  int64_t n_new;
  bool overflow;
};

// _advance of the cache for one chunk (counters move; the update is described, not launched)
int plan_update(StreamCounters& s, int64_t step, const void* k, const void* v, void* ring_k, void* ring_v,
                int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity, int block_size,
                int cache_window, int head_dim, PlannedUpdate* out) {
  if (s.tail + step > ring_capacity) {
    set_error("CompressedKVCache.tail_capacity=%lld too small to fit tail_size=%lld + step=%lld",
              (long long)ring_capacity, (long long)s.tail, (long long)step);
    return BFLY_ERR_CAPACITY;
  }
  const int64_t offset0 = s.offset;
  s.tail += step;
  s.offset += step;
  const int64_t first_pos = s.sum_off, first_slot = s.count;
  int64_t n_new = 0;
  bool overflow = false;
  while (s.sum_off + block_size <= s.offset - cache_window) {
    const int64_t block_start = s.sum_off - (s.offset - s.tail);
    if (block_start < 0 || block_start + block_size > s.tail) break;
    if (s.count + n_new >= pool_capacity) {
      overflow = true;
      break;
    }
    ++n_new;
    s.sum_off += block_size;
  }
  out->job = UpdateJob{k, v, ring_k, ring_v, pool_k, pool_v, step, ring_capacity, pool_capacity, offset0,
                       first_pos, first_slot, (int)n_new, block_size, head_dim};
  out->n_new = n_new;
  out->overflow = overflow;
  return BFLY_OK;
}

// after the update's launch: pooled count, then the trim (or the overflow error)
int finish_update(StreamCounters& s, const PlannedUpdate& u, int64_t step, int64_t pool_capacity, int block_size,
                  int cache_window) {
  s.count += u.n_new;
  if (u.overflow) {
    set_error("CompressedKVCache.summary_capacity=%lld exhausted at offset=%lld", (long long)pool_capacity,
              (long long)s.offset);
    return BFLY_ERR_CAPACITY;
  }
  const int64_t target = cache_window > step + cache_window - 1 ? cache_window : step + cache_window - 1;
  while (s.tail - block_size >= target) s.tail -= block_size;
  return BFLY_OK;
}

}  // namespace

extern "C" int bfly_stream_chunks(int64_t n_chunks, const void* const* q, const void* const* k,
                                  const void* const* v, void* const* out, const int64_t* chunk_len, int dtype,
                                  int64_t batch, int hq, int hkv, int head_dim, void* ring_k, void* ring_v,
                                  int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                                  int64_t* counters, int cache_window, int64_t layer_idx, int partner_rule,
                                  int local_window_blocks, int sink_count, int partner_count, int block_size,
                                  int window, float scale, int64_t* chunks_done, hipStream_t stream) {
  BFLY_CHECK_ARG(n_chunks >= 0 && q && k && v && out && chunk_len && counters && chunks_done, "null pointer");
  BFLY_CHECK_ARG(ring_k && ring_v && pool_k && pool_v, "null pointer");
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(batch * hkv <= 65535, "batch*hkv too large");
  BFLY_CHECK_ARG(block_size > 0 && window > 0 && cache_window > 0, "bad block_size/window");
  BFLY_CHECK_ARG(local_window_blocks >= 0 && sink_count >= 0 && partner_count >= 0 &&
                     partner_count <= BFLY_MAX_PARTNERS,
                 "bad topology parameters");
  BFLY_CHECK_ARG(aligned16(ring_k) && aligned16(ring_v) && aligned16(pool_k) && aligned16(pool_v),
                 "tensor pointers must be 16-byte aligned");
  *chunks_done = 0;
  StreamCounters s{counters[0], counters[1], counters[2], counters[3]};
  BFLY_CHECK_ARG(s.offset > 0 && s.tail >= 0 && s.tail <= s.offset && s.count >= 0 && s.count <= pool_capacity &&
                     s.sum_off >= 0,
                 "the cache must hold a first chunk (offset > 0) and valid counters");
  int64_t total = s.offset;
  for (int64_t c = 0; c < n_chunks; ++c) {
    BFLY_CHECK_ARG(chunk_len[c] > 0 && q[c] && k[c] && v[c] && out[c], "chunk %lld: empty or null", (long long)c);
    BFLY_CHECK_ARG(aligned16(k[c]) && aligned16(v[c]), "chunk %lld: k/v must be 16-byte aligned", (long long)c);
    total += chunk_len[c];
  }
  const int kcap = 1 + local_window_blocks + partner_count + sink_count;
  // the MFMA attention kernel is the one that builds neighbour rows from the topology
  const bool mfma_ok = dtype == BFLY_DTYPE_BF16 && window <= kPage && block_size >= kPage && 2 * kcap <= kSumSlots &&
                       (head_dim == 64 || head_dim == 128 || head_dim == 256) && scale > 0.f &&
                       ring_capacity >= kPage && ring_capacity >= block_size && total + 2 * kPage < INT32_MAX &&
                       ring_capacity < INT32_MAX && pool_capacity < INT32_MAX;
  if (!mfma_ok) {
    set_error("bfly_stream_chunks: configuration outside the MFMA attention path");
    return BFLY_ERR_UNSUPPORTED;
  }
  const int64_t rows = batch * hkv;
  auto publish = [&](const StreamCounters& st) {
    counters[0] = st.offset;
    counters[1] = st.tail;
    counters[2] = st.count;
    counters[3] = st.sum_off;
  };
  // Chunks go in batches: one attention launch per batch, each chunk with the arguments of
  // its own cache state (so its output is that of a launch of its own), and one update job per
  // batch that appends all its chunks and pools every block that becomes due over them (the
  // per-chunk counter steps run on the host; the pooled blocks are consecutive).  A batch's
  // update rides with the previous batch's attention when the two touch disjoint ring slots.
  // Batch tokens are capped at (ring - 2*64) / 2 so that consecutive batches can share a
  // launch; with a ring of a few chunks that is one chunk per batch, the per-chunk schedule.
  struct Batch {
    int64_t first = 0, count = 0, total = 0;
    AttnArgs args[kMaxUpdateParts];
    UpdateJob job{};
    StreamCounters end{};
    bool overflow = false;   // the last chunk exhausted the pool: its update runs, its attention not
    bool from_inputs = false;   // the attention reads the batch's own tokens from the chunk inputs
    int stop_rc = BFLY_OK;   // the chunk after the batch does not fit (its error)
  };
  const int64_t budget = (ring_capacity - 2 * kPage) / 2;
  auto plan_batch = [&](const StreamCounters& s0, int64_t from, Batch& bt) -> int {
    bt = Batch{};
    bt.first = from;
    bt.end = s0;
    StreamCounters st = s0;
    int64_t blocks = 0;
    for (int64_t c = from; c < n_chunks && bt.count < kMaxUpdateParts; ++c) {
      const int64_t len = chunk_len[c];
      if (bt.count > 0 && (bt.total + len > budget || s0.tail + bt.total + len > ring_capacity)) break;
      StreamCounters nx = st;
      PlannedUpdate pu{};
      const int prc = plan_update(nx, len, k[c], v[c], ring_k, ring_v, ring_capacity, pool_k, pool_v, pool_capacity,
                                  block_size, cache_window, head_dim, &pu);
      if (prc) {                      // does not fit: the batch ends before it, the error is its
        bt.stop_rc = prc;
        break;
      }
      if (pu.overflow && bt.count > 0) break;   // it starts the next batch, alone
      const int frc = finish_update(nx, pu, len, pool_capacity, block_size, cache_window);
      if (bt.count == 0) bt.job = pu.job;      // offset, first pooled block and slot of the batch
      bt.job.k_part[bt.count] = k[c];
      bt.job.v_part[bt.count] = v[c];
      bt.job.part_end[bt.count] = bt.total + len;
      blocks += pu.n_new;
      bt.total += len;
      const int64_t nblocks = (nx.offset + block_size - 1) / block_size;
      AttnArgs& a = bt.args[bt.count];
      a = AttnArgs{};
      const int trc = bfly_topology_init(nblocks, layer_idx, partner_rule, local_window_blocks, sink_count,
                                         partner_count, &a.topo);
      if (trc) return trc;
      a.q = q[c]; a.out = out[c]; a.k = ring_k; a.v = ring_v; a.ks = pool_k; a.vs = pool_v;
      a.nbr = nullptr; a.qpos = nullptr;
      a.batch = batch; a.hq = hq; a.hkv = hkv; a.tq = len; a.d = head_dim;
      a.q_pos0 = nx.offset - len; a.kv_rows = ring_capacity; a.ring = ring_capacity;
      a.key_lo = nx.offset - nx.tail; a.kv_len = nx.offset;
      a.pool_rows = pool_capacity; a.nsum = nx.count; a.nblocks = nblocks;
      a.kcap = kcap; a.bs = block_size; a.W = window; a.scale = scale; a.token_cutoff = 1;
      ++bt.count;
      st = nx;
      if (pu.overflow) {              // finish_update reported it
        bt.overflow = true;
        (void)frc;
        break;
      }
    }
    bt.end = st;
    bt.job.step = bt.total;
    bt.job.n_blocks = (int)blocks;
    bt.job.nparts = (int)bt.count;
    // When every chunk of the batch starts on a page boundary, its attention reads the batch's
    // own tokens from the chunk inputs and only the tokens in the tail the batch leaves are
    // copied to the ring: every later read of the ring (pooling, attention windows, the cache's
    // views) lies in a later tail, which starts no earlier.
    bt.from_inputs = true;
    for (int64_t j = 0; j < bt.count; ++j) bt.from_inputs = bt.from_inputs && bt.args[j].q_pos0 % kPage == 0;
    const int64_t keep_from = st.offset - st.tail - bt.job.offset;
    bt.job.append_from = !bt.from_inputs || keep_from < 0 ? 0 : (keep_from > bt.total ? bt.total : keep_from);
    return BFLY_OK;
  };
  auto launch_update = [&](const UpdateJob& j) -> int { return launch_update_job(j, rows, stream); };
  if (n_chunks == 0) return BFLY_OK;
  // the first batch's update runs alone; every later one rides with the previous attention
  // when their ring slots are disjoint
  Batch cur{}, nxt{};
  int rc = plan_batch(s, 0, cur);
  if (rc) return rc;
  if (cur.count == 0) return cur.stop_rc;
  rc = launch_update(cur.job);
  if (rc) return rc;
  s = cur.end;
  publish(s);
  if (cur.overflow) return BFLY_ERR_CAPACITY;   // the message was set when it was planned
  for (;;) {
    const int64_t next_from = cur.first + cur.count;
    if (cur.stop_rc == BFLY_OK && next_from < n_chunks) {
      rc = plan_batch(s, next_from, nxt);
      if (rc) return rc;
    } else {
      nxt = Batch{};
      nxt.stop_rc = cur.stop_rc;
    }
    if (nxt.count > 0 && cur.total + nxt.total + 2 * kPage <= ring_capacity) {
      rc = launch_attention_batch(cur.args, cur.job.k_part, cur.job.v_part, (int)cur.count, cur.from_inputs,
                                  stream, "bfly_stream_chunks", &nxt.job, rows);
      if (rc) return rc;
    } else {
      rc = launch_attention_batch(cur.args, cur.job.k_part, cur.job.v_part, (int)cur.count, cur.from_inputs,
                                  stream, "bfly_stream_chunks");
      if (rc) return rc;
      if (nxt.count > 0) {
        rc = launch_update(nxt.job);
        if (rc) return rc;
      }
    }
    *chunks_done = next_from;
    if (nxt.count == 0) return nxt.stop_rc;
    s = nxt.end;
    publish(s);
    if (nxt.overflow) return BFLY_ERR_CAPACITY;
    cur = nxt;
  }
}
