// Butterfly decode on gfx950: one new query per sequence over the two-pool
// cache (ring tail of raw tokens + pool of mean-pooled block summaries).
//
// Reference semantics: compressed_butterfly_attention_from_cache
// (bna/mlx/attention.py:1816-1876) for one active row at p = kv_len - 1:
// the SWA stream over tail keys [max(tail_start, p-W+1), p] (:1669-1710) and
// the routed-summary stream over the neighbours n of block p/BS with n < p/BS,
// n < summary_count and (n+1)*BS <= max(0, p-W+1) (:1713-1813), merged by
// online softmax (:519-548).  Both streams are scored under one max and one
// sum here, which is that merge evaluated exactly; it equals the Torch
// active-row path (bna/torch/attention_wayfinder_permute.py:1125-1197).
//
// The cache append of the new token (bna/mlx/compressed_cache.py:104-118) is
// fused in: the kernel writes k_new/v_new to ring slot p mod C and scores the
// new token from the k_new/v_new registers it staged, so nothing is read back
// through memory in the same launch.
//
// Work unit = one workgroup per (batch, kv head), 256 threads.  Each wave
// computes the routed row of the query block from the topology (no table read:
// one candidate per lane, first-occurrence dedup by shuffles, slots by ballot),
// so every thread issues its q, window-row and summary-row loads in one batch;
// one barrier later the <= 64 window rows and <= 16 summaries sit in LDS.
// Wave w takes query heads w, w+4, ... of the GQA group with its own q and p
// buffers (no further workgroup barriers).  Scores: lanes over keys; softmax
// reductions: wavefront shuffles; output: lanes over head_dim.
//
// Step mode (bfly_decode_step): the cache counters (offset, tail_size,
// summary_count, summary_offset) live in a device array.  Every workgroup
// derives the post-update counters from them with the reference's rules
// (append one token, summarise every block with end + W <= offset, trim whole
// blocks while tail_size - BS >= W; compressed_cache.py:94-172), pools a newly
// due block itself (same summation order as bfly_cache_compress), computes the
// layer's topology at the live block count, and attends; each workgroup keeps
// its own copy of the counters and writes it back.  A step then has fixed
// arguments and can be captured in a HIP graph.  The MFMA kernel runs eight
// more workgroups (one per XCD) that keep counter copies of their own and
// write the next step's routed row into the copies of the workgroups on their
// XCD, so the next step reads it with its counters (an L2 hit) and issues its
// summary loads together with the window loads instead of after the selection.
#include "bfly_topology.h"
#include "q4_piece.h"

namespace bfly {

constexpr int kDecMaxWin = 64;
constexpr int kDecMaxSum = 16;
constexpr int kDecMaxKeys = kDecMaxWin + kDecMaxSum;
constexpr int kDecMaxNew = 2;   // blocks pooled in one step (one per 128 steps in steady state)

// Device cache counters of step mode: state[4] is the error word; workgroup g
// (= batch * Hkv + kv head) keeps its own copy of kStSlot words at
// state[8 + kStSlot * g ...]: {offset, tail_size, summary_count,
// summary_offset} in words 0..3, advanced by the workgroup itself, so a step
// needs no cross-workgroup synchronisation (every copy evolves identically;
// the host reads copy 0).  The MFMA kernel's kRouteGroups extra workgroups
// (route workgroup r is blockIdx r and keeps copy batch * Hkv + r; attending
// workgroup g is blockIdx g + 8) advance their own copies the same way, and
// route workgroup r writes two route buffers, at words 4 and 16 of the copies
// of the attending workgroups g with g mod 8 = r (buffer 0 shares the
// counters' cache line).  Workgroups are dispatched to the eight XCDs
// round-robin, so those copies are written and read on one XCD.
//
// Route buffer b (12 words) holds the routed row of the step whose post-update
// kv_len has parity b, written during the step before it: word 0 a key
// (kv_len | ns << 32 | W << 40 | rule << 48 | 1 << 62), word 1 layer_idx,
// word 2 block_size | ring << 32, word 3 pool_rows | lwb << 30 | sinks << 34 |
// partners << 38 | cache window << 43 (pool_rows < 2^30, lwb, sinks and partners
// 4 bits each, cache window < 2^20; route_key below), words 4..11 the ns pool
// rows as int32.  A step uses it only
// when every word matches its own kv_len and arguments (anything else, a zero
// key included, falls back to computing the row).  A launch uses the buffer
// of its own parity and writes only the other one.  The attending workgroups
// request the row entries of both buffers together with the counters (one
// round trip instead of two) and keep those of their own parity, so no word
// written within a launch is used by it.
enum { kStOffset = 0, kStTail = 1, kStCount = 2, kStSumOff = 3 };
constexpr int kStError = 4;
constexpr int64_t kErrCapacity = 1;   // state[kStError]: tail or pool capacity exceeded
constexpr int64_t kErrRope = 2;       // state[kStError]: position past the RoPE tables (fused q/k norm)
constexpr int kStHeader = 8;
constexpr int kStSlot = 32;
constexpr int kStRoute = 4;
constexpr int kRouteWords = 12;
constexpr int kRouteGroups = 8;
__device__ __forceinline__ int64_t* dec_slot(int64_t* state, int64_t g) { return state + kStHeader + kStSlot * g; }

// Counter copies per sequence.  A step with the attention output projection fused in
// (bfly_decode_step_qk_norm_oproj) runs several attending workgroups per sequence, each
// with its own copy, so a state of at most kOprojMaxSeq sequences keeps kOprojSubs copies
// per sequence: sequence s owns copies s + nseq * c (c < cps), the route workgroups' eight
// follow at nseq * cps.  Every kernel advances all copies of its sequences, so the entry
// points can take turns on one state.
constexpr int kOprojMaxSeq = 16;
constexpr int kOprojSubs = 64;
__host__ __device__ __forceinline__ int dec_copies(int64_t nseq) { return nseq <= kOprojMaxSeq ? kOprojSubs : 1; }

// The advanced counters into copies first + stride * c, c in [c0, c1): thread tid writes
// copy c0 + tid.  clear: also zero both route-buffer keys (kernels that keep no routed rows).
__device__ __forceinline__ void dec_put_counters(int64_t* state, int64_t first, int64_t stride, int c0, int c1,
                                                 int tid, int64_t off, int64_t ts, int64_t sc, int64_t so,
                                                 bool clear) {
  const int c = c0 + tid;
  if (c < c1) {
    int64_t* slot = dec_slot(state, first + stride * c);
    slot[kStOffset] = off;
    slot[kStTail] = ts;
    slot[kStCount] = sc;
    slot[kStSumOff] = so;
    if (clear) {
      slot[kStRoute] = 0;
      slot[kStRoute + kRouteWords] = 0;
    }
  }
}


struct StepArgs {
  int64_t* state;
  int64_t layer_idx;
  int rule, lwb, sinks, partners;
};

// layer mod count (non-negative), one 32-bit division for any real layer index
__device__ __forceinline__ int64_t dec_mod_layer(int64_t x, int count) {
  if (x >= 0 && x <= INT32_MAX) return (int64_t)((uint32_t)x % (uint32_t)count);
  return posmod(x, count);
}

// bfly_topology_init on the device: width = ceil(log2 N) (1 if N <= 1),
// stage = layer mod stage_count, partner bits per the rule
// (bna/topology/butterfly.py:39-105).
__device__ __forceinline__ bfly_topology_t topology_at(int64_t n, const StepArgs& s) {
  bfly_topology_t t{};
  const int w = n <= 1 ? 1 : 64 - __clzll((unsigned long long)(n - 1));
  const int count = s.rule == BFLY_RULE_BENES ? (2 * w - 2 > 1 ? 2 * w - 2 : 1) : w;
  int64_t st = dec_mod_layer(s.layer_idx, count);
  t.rule = s.rule;
  t.width = w;
  t.stage_idx = (int)st;
  t.stage_count = count;
  t.local_window_blocks = s.lwb;
  t.sink_count = s.sinks;
  t.partner_count = s.partners;
#pragma unroll
  for (int j = 0; j < BFLY_MAX_PARTNERS; ++j) {
    if (j >= s.partners) continue;
    if (s.rule == BFLY_RULE_BENES) {
      const int base = count <= 1 ? 0 : (int)st % count;
      const int phase = (base + j) % count;
      t.partner_bits[j] = w <= 1 ? 0 : (phase < w ? phase : 2 * w - 2 - phase);
    } else {
      t.partner_bits[j] = (int)((st + j) % w);
    }
  }
  return t;
}

// Division of n < 2^31 by a fixed d >= 1 without a divide: with l = ceil(log2 d)
// and m = ceil(2^(31+l) / d) (< 2^32), floor(n / d) = (n * m) >> (31 + l),
// exact because m * d - 2^(31+l) < d <= 2^l (Granlund and Montgomery, "Division
// by invariant integers using multiplication", PLDI 1994, theorem 4.2).
struct FastDiv {
  uint32_t m = 1u << 31;
  int sh = 31;
  uint32_t d = 1;
  __host__ static FastDiv make(uint32_t d) {
    FastDiv f;
    int l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    f.m = (uint32_t)(((1ull << (31 + l)) + d - 1) / d);
    f.sh = 31 + l;
    f.d = d;
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (uint32_t)(((uint64_t)n * m) >> sh); }
  __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};

struct DecodeArgs {
  const void* q;          // [B, Hq, 1, d]
  void* out;              // [B, Hq, 1, d]
  const void* k_new;      // [B, Hkv, 1, d] or null
  const void* v_new;
  void* ring_k;           // ring [B, Hkv, C, d] (C > 0) or linear tail [B, Hkv, kv_len - tail_start, d]
  void* ring_v;
  const void* pool_k;     // [B, Hkv, pool_rows, d]
  const void* pool_v;
  bfly_topology_t topo;   // routed row of the query block, computed in-kernel
  int64_t ring;           // C, 0 = linear tail
  int64_t kv_rows;        // rows per (b, kv head) of ring_k / ring_v
  int64_t tail_start;
  int64_t kv_len;         // query position is kv_len - 1
  int64_t pool_rows;
  int64_t nsum;
  int64_t nblocks;
  int hq, hkv, bs, W;
  int CW;                 // step mode: the cache's own local window (summarise and trim rules)
  float scale;
  FastDiv bs_div, ring_div, hkv_div;   // MFMA path: block_size, ring capacity, Hkv
  int gsz;                             // MFMA path: hq / hkv
  int nseq;                            // MFMA step path: batch * hkv (attending sequences)
  int cps;                             // step mode: counter copies per sequence (dec_copies)
  // fused output projection (bfly_decode_step_qk_norm_oproj): W_o in bfly_q4_gemv's layout
  // ([o_rows][64] pieces, o_groups (scale, bias) words per row, o_ppg pieces per group as a
  // shift), o_subs attending workgroups per sequence, fp32 partial rows [hkv][batch][o_rows]
  const u32x4* ow;
  const uint32_t* osb;
  float* opart;
  int o_rows, o_groups, o_ppg_log2, o_subs;
  FastDiv nseq_div;
  // MFMA step path, d = 128: when qn_w is set, q and k_new are the raw projection
  // rows and the kernel applies the per-head q/k RMSNorm and rotate-half RoPE at
  // position kv_len - 1 itself (rope_cos / rope_sin: [rope_rows][128] fp32)
  const __bf16* qn_w;
  const __bf16* kn_w;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_rows;
  float qk_eps;
};

__device__ __forceinline__ float dec_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float dec_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}


// Non-negative 64-bit quotient / remainder by a positive int: one 32-bit
// division when the dividend fits (always, for any realistic cache), else the
// 64-bit routine.  The operands are workgroup-uniform.
__device__ __forceinline__ int64_t dec_div(int64_t x, int64_t d) {
  if (x >= 0 && x <= INT32_MAX && d <= INT32_MAX) return (int64_t)((uint32_t)x / (uint32_t)d);
  return x / d;
}
__device__ __forceinline__ int64_t dec_mod(int64_t x, int64_t d) {
  if (x >= 0 && x <= INT32_MAX && d <= INT32_MAX) return (int64_t)((uint32_t)x % (uint32_t)d);
  return posmod(x, d);
}

// This step's cache counters: from the arguments, or (step mode) derived on the
// device from the counter array with the reference's update rules.
struct DecState {
  int64_t kv_len, tail_start, nsum, nblocks;
  int64_t sc0, so0, ts1, sc1, so1;   // step mode: counts before/after, tail size after
  int n_new;                         // blocks that become due in this step
  bool err;
  bfly_topology_t topo;
};

template <bool kStep>
__device__ __forceinline__ DecState dec_state(const DecodeArgs& a, const StepArgs& sa) {
  DecState s{};
  s.kv_len = a.kv_len;
  s.tail_start = a.tail_start;
  s.nsum = a.nsum;
  s.nblocks = a.nblocks;
  s.topo = a.topo;
  if constexpr (kStep) {
    const int64_t* slot = dec_slot(sa.state, blockIdx.x);
    const int64_t off0 = slot[kStOffset], ts0 = slot[kStTail];
    s.sc0 = slot[kStCount];
    s.so0 = slot[kStSumOff];
    const int64_t off1 = off0 + 1;
    s.ts1 = ts0 + 1;
    bool err = s.ts1 > a.ring;                              // tail capacity (compressed_cache.py:105-110)
    s.sc1 = s.sc0;
    s.so1 = s.so0;
    while (!err && s.so1 + a.bs <= off1 - a.CW) {           // summarise (:120-149)
      const int64_t bstart = s.so1 - (off1 - s.ts1);
      if (bstart < 0 || bstart + a.bs > s.ts1) break;
      if (s.sc1 >= a.pool_rows || s.n_new == kDecMaxNew) {  // pool capacity (:128-132)
        err = true;
        break;
      }
      ++s.n_new;
      ++s.sc1;
      s.so1 += a.bs;
    }
    while (s.ts1 - a.bs >= a.CW) s.ts1 -= a.bs;             // trim: target max(CW, step + CW - 1) = CW
    s.err = err;
    s.kv_len = off1;
    s.tail_start = off1 - s.ts1;
    s.nsum = s.sc1;
    s.nblocks = dec_div(off1 + a.bs - 1, a.bs);
    s.topo = topology_at(s.nblocks, sa);
  }
  return s;
}

// Step mode: pool the blocks that became due for this (batch, kv head) into the
// pool and into `newrow` (K, V per block), in the summation order of
// block_mean_kernel (slot s sums tokens s, s+RS, ...; the slots are added in
// order; divided by BS; rounded once).
template <typename T, int D>
__device__ __forceinline__ void dec_pool(const DecodeArgs& a, const DecState& s, const T* rk, const T* rv, T* pk,
                                         T* pv, float* part, T (*newrow)[D], int tid) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LPR = D / VEC;
  constexpr int RS = 256 / LPR;
  for (int j = 0; j < s.n_new; ++j) {
    const int64_t pos0 = s.so0 + (int64_t)j * a.bs;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const T* src = kv ? rv : rk;
      T* dst = (kv ? pv : pk) + (s.sc0 + j) * D;
      const int c = tid % LPR, sl = tid / LPR;
      float acc[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
      for (int tok = sl; tok < a.bs; tok += RS) {
        const uint4 raw = *reinterpret_cast<const uint4*>(src + dec_mod(pos0 + tok, a.ring) * D + c * VEC);
        const T* x = reinterpret_cast<const T*>(&raw);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += to_f32(x[e]);
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) part[sl * D + c * VEC + e] = acc[e];
      __syncthreads();
      for (int col = tid; col < D; col += 256) {
        float tot = 0.f;
        for (int k = 0; k < RS; ++k) tot += part[k * D + col];
        const T val = from_f32<T>(tot / (float)a.bs);
        dst[col] = val;
        newrow[2 * j + kv][col] = val;
      }
      __syncthreads();
    }
  }
}

// Routed summaries of the query block (token-level cut-off), computed by one
// wave on its own: lane j < kc holds entry j of the ordered row
// [b, b-1..b-lwb, partners, sinks] (-1 where the reference pushes nothing),
// keeps it at its first occurrence, and the ballot of the entries that pass the
// filter gives their slots in row order (written to sel).  Returns the count.
__device__ __forceinline__ int dec_select(int64_t p, const DecodeArgs& a, const DecState& s, int lane, int* sel) {
  int64_t blk = dec_div(p, a.bs);
  if (blk > s.nblocks - 1) blk = s.nblocks - 1;
  int64_t cut = p - a.W + 1;
  if (cut < 0) cut = 0;
  const bfly_topology_t& topo = s.topo;
  const int lwb = topo.local_window_blocks, npart = topo.partner_count;
  const int64_t nsink = topo.sink_count < s.nblocks ? topo.sink_count : s.nblocks;
  const int kc = 1 + lwb + npart + topo.sink_count;
  int64_t cand = -1;
  if (lane < kc) {
    if (lane == 0) {
      cand = blk;
    } else if (lane <= lwb) {
      cand = blk - lane >= 0 ? blk - lane : -1;
    } else if (lane <= lwb + npart) {
      const int j = lane - 1 - lwb;
      int bit = 0;
#pragma unroll
      for (int jj = 0; jj < BFLY_MAX_PARTNERS; ++jj)
        if (jj == j) bit = topo.partner_bits[jj];
      cand = partner_block(blk, bit, s.nblocks, topo.rule, topo.width);
    } else {
      const int64_t sk = lane - 1 - lwb - npart;
      cand = sk < nsink ? sk : -1;
    }
    if (cand >= s.nblocks) cand = -1;
  }
  const int c32 = (int)cand;
  bool keep = cand >= 0;
  for (int i = 0; i < kc; ++i) {                  // kc is uniform: lane i's entry as a scalar
    const int ci = __builtin_amdgcn_readlane(c32, i);
    if (i < lane && ci == c32) keep = false;
  }
  const bool take = keep && cand < blk && cand < s.nsum && (cand + 1) * a.bs <= cut;
  const unsigned long long mask = __ballot(take);
  if (take) sel[__popcll(mask & ((1ull << lane) - 1ull))] = c32;
  __builtin_amdgcn_wave_barrier();
  return __popcll(mask);
}

template <typename T, int D, bool kStep>
__global__ void __launch_bounds__(256, 1) decode_kernel(DecodeArgs a, StepArgs sa) {
  constexpr int VEC = 16 / (int)sizeof(T);     // elements per 16-byte piece
  constexpr int PIECES = D / VEC;
  constexpr int KP = D + VEC;                  // padded K row: rows 16 B apart in bank space
  constexpr int DPL = D / 64;                  // q/output elements per lane
  constexpr int LPR = D / VEC;                 // compressor: lanes per row
  constexpr int RS = 256 / LPR;                // compressor: row slots
  __shared__ __attribute__((aligned(16))) T Ks[kDecMaxKeys * KP];
  __shared__ __attribute__((aligned(16))) T Vs[kDecMaxKeys * D];
  __shared__ __attribute__((aligned(16))) float qs[4][D];
  __shared__ __attribute__((aligned(16))) float ps[4][kDecMaxKeys];
  __shared__ int selw[4][kDecMaxSum];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t bh = blockIdx.x;
  const int64_t bi = bh / a.hkv;
  const int kvh = (int)(bh - bi * a.hkv);
  const int gsz = a.hq / a.hkv;

  // ---- this step's counters: from the arguments, or (step mode) derived on the device
  const DecState st = dec_state<kStep>(a, sa);
  if (kStep && st.err) {
    if (tid == 0) sa.state[kStError] = kErrCapacity;      // the host raises at its next synchronisation
    return;                                               // uniform: every workgroup sees the same counters
  }
  const int64_t kv_len = st.kv_len, tail_start = st.tail_start;
  const int64_t p = kv_len - 1;
  int64_t lo = p - a.W + 1;
  if (lo < tail_start) lo = tail_start;
  if (lo < 0) lo = 0;
  const int nw = (int)(p - lo + 1);

  const T* knew = a.k_new ? reinterpret_cast<const T*>(a.k_new) + bh * D : nullptr;
  const T* vnew = a.v_new ? reinterpret_cast<const T*>(a.v_new) + bh * D : nullptr;
  T* rk = reinterpret_cast<T*>(a.ring_k) + bh * a.kv_rows * D;
  T* rv = reinterpret_cast<T*>(a.ring_v) + bh * a.kv_rows * D;
  T* pk = reinterpret_cast<T*>(const_cast<void*>(a.pool_k)) + bh * a.pool_rows * D;
  T* pv = reinterpret_cast<T*>(const_cast<void*>(a.pool_v)) + bh * a.pool_rows * D;

  // ---- this wave's first q row into registers (its load overlaps the staging below)
  float qv[DPL];
  {
    const int hh = wave < gsz ? wave : 0;
    const T* qrow = reinterpret_cast<const T*>(a.q) + (bi * a.hq + (int64_t)kvh * gsz + hh) * D + lane * DPL;
#pragma unroll
    for (int e = 0; e < DPL; ++e) qv[e] = to_f32(qrow[e]);
  }
  // ---- step mode: pool the newly due blocks of this (batch, kv head)
  __shared__ __attribute__((aligned(16))) T newrow[kStep ? kDecMaxNew * 2 : 1][kStep ? D : 1];
  if constexpr (kStep) {
    __shared__ float part[RS * D];
    dec_pool<T, D>(a, st, rk, rv, pk, pv, part, newrow, tid);
  }
  // ---- routed summaries of the query block, computed by every wave on its own
  const int ns = dec_select(p, a, st, lane, selw[wave]);
  const int nk = nw + ns;

  // ---- window rows (the newest from k_new/v_new when given, also appended to the
  // ring) and routed summaries: all loads of a thread issued together, then LDS
  constexpr int kStage = (kDecMaxKeys * PIECES + 255) / 256;
  {
    uint4 kx[kStage], vx[kStage];
    const int64_t slot_lo = a.ring ? dec_mod(lo, a.ring) : lo - tail_start;
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int i = tid + it * 256;
      kx[it] = vx[it] = make_uint4(0, 0, 0, 0);
      if (i < nk * PIECES) {
        const int r = i / PIECES, pc = i % PIECES;
        if (r < nw) {
          const int64_t pos = lo + r;
          int64_t row = slot_lo + r;
          if (a.ring && row >= a.ring) row -= a.ring;
          if (knew != nullptr && pos == p) {
            kx[it] = *reinterpret_cast<const uint4*>(knew + pc * VEC);
            vx[it] = *reinterpret_cast<const uint4*>(vnew + pc * VEC);
            *reinterpret_cast<uint4*>(rk + row * D + pc * VEC) = kx[it];
            *reinterpret_cast<uint4*>(rv + row * D + pc * VEC) = vx[it];
          } else {
            kx[it] = *reinterpret_cast<const uint4*>(rk + row * D + pc * VEC);
            vx[it] = *reinterpret_cast<const uint4*>(rv + row * D + pc * VEC);
          }
        } else {
          const int64_t n = selw[wave][r - nw];
          if (kStep && n >= st.sc0) {        // pooled in this step: take the LDS copy
            kx[it] = *reinterpret_cast<const uint4*>(&newrow[2 * (n - st.sc0)][pc * VEC]);
            vx[it] = *reinterpret_cast<const uint4*>(&newrow[2 * (n - st.sc0) + 1][pc * VEC]);
          } else {
            kx[it] = *reinterpret_cast<const uint4*>(pk + n * D + pc * VEC);
            vx[it] = *reinterpret_cast<const uint4*>(pv + n * D + pc * VEC);
          }
        }
      }
    }
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int i = tid + it * 256;
      if (i < nk * PIECES) {
        const int r = i / PIECES, pc = i % PIECES;
        *reinterpret_cast<uint4*>(Ks + r * KP + pc * VEC) = kx[it];
        *reinterpret_cast<uint4*>(Vs + r * D + pc * VEC) = vx[it];
      }
    }
  }
  // this wave's first head: q (already in registers) into its LDS slot
  if (wave < gsz) {
#pragma unroll
    for (int e = 0; e < DPL; ++e) qs[wave][lane * DPL + e] = qv[e] * a.scale;
  }
  __syncthreads();   // window and summary rows visible to every wave

  // ---- heads: wave w takes heads w, w+4, ...; qs[wave] and ps[wave] are the
  // wave's own, so the rounds need no workgroup barrier
  for (int hh = wave; hh < gsz; hh += 4) {
    const int64_t h = (int64_t)kvh * gsz + hh;
    if (hh != wave) {
      const T* qrow = reinterpret_cast<const T*>(a.q) + (bi * a.hq + h) * D + lane * DPL;
#pragma unroll
      for (int e = 0; e < DPL; ++e) qs[wave][lane * DPL + e] = to_f32(qrow[e]) * a.scale;
    }
    __builtin_amdgcn_wave_barrier();
    // scores: lane owns keys lane and lane + 64; 4 partial sums per dot product
    float s[2];
    float mloc = -INFINITY;
#pragma unroll
    for (int rnd = 0; rnd < 2; ++rnd) {
      const int key = lane + 64 * rnd;
      float acc = 0.f;
      if (key < nk) {
        const T* krow = Ks + key * KP;
        float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pc = 0; pc < PIECES; ++pc) {
          const uint4 raw = *reinterpret_cast<const uint4*>(krow + pc * VEC);
          const T* kv = reinterpret_cast<const T*>(&raw);
#pragma unroll
          for (int e = 0; e < VEC; ++e) part[e & 3] = fmaf(qs[wave][pc * VEC + e], to_f32(kv[e]), part[e & 3]);
        }
        acc = (part[0] + part[1]) + (part[2] + part[3]);
        mloc = fmaxf(mloc, acc);
      }
      s[rnd] = acc;
    }
    const float m = dec_wave_max(mloc);
    float lloc = 0.f;
#pragma unroll
    for (int rnd = 0; rnd < 2; ++rnd) {
      const int key = lane + 64 * rnd;
      const float e = key < nk ? __expf(s[rnd] - m) : 0.f;
      s[rnd] = e;
      lloc += e;
    }
    const float inv = 1.f / fmaxf(dec_wave_sum(lloc), 1e-9f);
#pragma unroll
    for (int rnd = 0; rnd < 2; ++rnd) {
      const int key = lane + 64 * rnd;
      if (key < kDecMaxKeys) ps[wave][key] = key < nk ? s[rnd] * inv : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    // output: lane owns d = lane*DPL + [0, DPL); keys in groups of 4 with
    // independent accumulators (rows past nk carry p = 0 and are skipped)
    float acc[DPL][4];
#pragma unroll
    for (int e = 0; e < DPL; ++e)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[e][j] = 0.f;
    const int nk4 = nk & ~3;
    for (int key = 0; key < nk4; key += 4) {
      const float4 p4 = *reinterpret_cast<const float4*>(&ps[wave][key]);
      const float pj[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const T* vrow = Vs + (key + j) * D + lane * DPL;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e][j] = fmaf(pj[j], to_f32(vrow[e]), acc[e][j]);
      }
    }
    for (int key = nk4; key < nk; ++key) {
      const float pk_ = ps[wave][key];
      const T* vrow = Vs + key * D + lane * DPL;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e][0] = fmaf(pk_, to_f32(vrow[e]), acc[e][0]);
    }
    T* orow = reinterpret_cast<T*>(a.out) + (bi * a.hq + h) * D;
#pragma unroll
    for (int e = 0; e < DPL; ++e)
      orow[lane * DPL + e] = from_f32<T>((acc[e][0] + acc[e][1]) + (acc[e][2] + acc[e][3]));
    __builtin_amdgcn_wave_barrier();   // qs/ps reused by this wave's next head
  }
  if constexpr (kStep) {
    // Each workgroup advances its own counter copy; no workgroup reads another's
    // copy, pool, ring or output within the step, so no atomic or fence is
    // needed: the next launch sees everything at the kernel boundary.
    // (this kernel keeps no routed rows: their keys are cleared)
    dec_put_counters(sa.state, blockIdx.x, gridDim.x, 0, a.cps, tid, st.kv_len, st.ts1, st.sc1, st.so1, true);
  }
}


// ---------------------------------------------------------------------------------------------
// bf16 decode on MFMA.  The GQA group's query heads are the 16 columns of one
// v_mfma_f32_16x16x32_bf16 tile (heads 16g..16g+15 per pass; one pass up to 16
// heads), so each wave computes the scores of every head at once:
//   S^T = K Q^T over 5 tiles of 16 keys (window <= 64 + summaries <= 16, zero-padded),
//   fp32 softmax per column (shuffles between the 4 lane groups),
//   O^T = V^T P^T with V transposed in LDS; wave w takes output d-tiles w, w+4, ...
// Staging, selection, pooling and counters follow decode_kernel, in 32-bit
// arithmetic: the host sends a cache here only when every position, row and
// element offset stays below 2^30 (else decode_kernel runs), and in step mode
// the kernel flags counters outside that range as an error.
constexpr int kDecMfmaKeys = kDecMaxKeys;   // 80 keys staged: 5 score tiles, PV k-steps padded to 96 in registers
constexpr int kDecPosLimit = 1 << 30;

struct DecState32 {
  int kv_len, tail_start, nsum, nblocks;
  int sc0, so0, ts1, sc1, so1;   // step mode: counts before/after, tail size after
  int n_new;                     // blocks that become due in this step
  int stage, count, width;       // step mode: topology at nblocks
  bool err;
};

// Step-mode counter update of dec_state (compressed_cache.py:94-172) from the
// counters before the step, and the topology of bfly_topology_init at the live
// block count (butterfly.py:39-105).
__device__ __forceinline__ DecState32 dec_advance32(int64_t off0, int64_t ts0, int64_t sc0, int64_t so0,
                                                    const DecodeArgs& a, const StepArgs& sa) {
  DecState32 s{};
  {
    const bool range = (uint64_t)off0 < (uint64_t)kDecPosLimit && (uint64_t)ts0 < (uint64_t)kDecPosLimit &&
                       (uint64_t)sc0 < (uint64_t)kDecPosLimit && (uint64_t)so0 < (uint64_t)kDecPosLimit;
    const int ring = (int)a.ring, bs = a.bs, CW = a.CW, pool_rows = (int)a.pool_rows;
    const int off1 = (int)off0 + 1;
    int ts1 = (int)ts0 + 1, sc1 = (int)sc0, so1 = (int)so0, n_new = 0;
    bool err = !range || ts1 > ring;                        // tail capacity (compressed_cache.py:105-110)
    while (!err && so1 + bs <= off1 - CW) {                 // summarise (:120-149)
      const int bstart = so1 - (off1 - ts1);
      if (bstart < 0 || bstart + bs > ts1) break;
      if (sc1 >= pool_rows || n_new == kDecMaxNew) {        // pool capacity (:128-132)
        err = true;
        break;
      }
      ++n_new;
      ++sc1;
      so1 += bs;
    }
    while (ts1 - bs >= CW) ts1 -= bs;                       // trim: target max(CW, step + CW - 1) = CW
    s.err = err;
    s.sc0 = (int)sc0;
    s.so0 = (int)so0;
    s.ts1 = ts1;
    s.sc1 = sc1;
    s.so1 = so1;
    s.n_new = n_new;
    s.kv_len = off1;
    s.tail_start = off1 - ts1;
    s.nsum = sc1;
    s.nblocks = (int)a.bs_div.div((uint32_t)(off1 + bs - 1));
    const int w = s.nblocks <= 1 ? 1 : 32 - __clz(s.nblocks - 1);
    s.width = w;
    s.count = sa.rule == BFLY_RULE_BENES ? (2 * w - 2 > 1 ? 2 * w - 2 : 1) : w;
    s.stage = (int)dec_mod_layer(sa.layer_idx, s.count);
  }
  return s;
}

template <bool kStep>
__device__ __forceinline__ DecState32 dec_state32(const DecodeArgs& a, const StepArgs& sa, int64_t g) {
  DecState32 s{};
  if constexpr (kStep) {
    const int64_t* slot = dec_slot(sa.state, g);
    s = dec_advance32(slot[kStOffset], slot[kStTail], slot[kStCount], slot[kStSumOff], a, sa);
  } else {
    s.kv_len = (int)a.kv_len;
    s.tail_start = (int)a.tail_start;
    s.nsum = (int)a.nsum;
    s.nblocks = (int)a.nblocks;
    s.width = a.topo.width;
  }
  return s;
}

// partner_block (bfly_topology.h) for blocks below 2^30.
__device__ __forceinline__ int partner32(int block, int bit, int nblocks, int rule, int width) {
  if (bit < 0 || bit >= (width > 1 ? width : 1)) return -1;
  int p;
  switch (rule) {
    case BFLY_RULE_CAUSAL_SHIFT: p = block - (1 << bit); break;
    case BFLY_RULE_XOR:
    case BFLY_RULE_BENES: p = block ^ (1 << bit); break;
    case BFLY_RULE_FIXED_STRIDE: p = block - 1; break;
    case BFLY_RULE_RANDOM: {
      if (block <= 0) return -1;
      const uint32_t seed = (uint32_t)block * 2654435761u + (uint32_t)bit * 374761393u;
      p = (int)(seed % (uint32_t)block);
      break;
    }
    default: {   // bit reversal over `width` bits (block < 2^width)
      const int sh = 32 - width;
      const uint32_t rev = __builtin_bitreverse32((uint32_t)block) >> sh;
      p = (int)(__builtin_bitreverse32(rev ^ (1u << bit)) >> sh);
      break;
    }
  }
  if (p < 0 || p >= nblocks || p > block) return -1;
  return p;
}

// dec_select in 32-bit; in step mode lane j derives its partner bit from the
// stage (bfly_topology_init's rule) instead of reading a bit array.
template <bool kStep>
__device__ __forceinline__ int dec_select32(int p, int blk, const DecodeArgs& a, const StepArgs& sa,
                                            const DecState32& s, int lane, int* sel) {
  const int cut = max(p - a.W + 1, 0);
  const int rule = kStep ? sa.rule : a.topo.rule;
  const int lwb = kStep ? sa.lwb : a.topo.local_window_blocks;
  const int npart = kStep ? sa.partners : a.topo.partner_count;
  const int sinks = kStep ? sa.sinks : a.topo.sink_count;
  const int nsink = min(sinks, s.nblocks);
  const int kc = 1 + lwb + npart + sinks;
  // Every lane evaluates each kind of entry and keeps its own by selects (no
  // divergent branches: this runs on the decode's critical path).
  const int jp = min(max(lane - 1 - lwb, 0), BFLY_MAX_PARTNERS - 1);   // partner index
  int bit = 0;
  if constexpr (kStep) {
    // stage + j reduced mod count (benes) or width
    const int ph0 = s.stage + jp;
    if (rule == BFLY_RULE_BENES) {
      const int ph = ph0 % s.count;
      bit = s.width <= 1 ? 0 : (ph < s.width ? ph : 2 * s.width - 2 - ph);
    } else {
      bit = ph0 % s.width;
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < BFLY_MAX_PARTNERS; ++jj) bit = jj == jp ? a.topo.partner_bits[jj] : bit;
  }
  const int c_part = partner32(blk, bit, s.nblocks, rule, s.width);
  const int sk = lane - 1 - lwb - npart;
  int cand = lane == 0 ? blk
             : lane <= lwb ? blk - lane
             : lane <= lwb + npart ? c_part
             : sk < nsink ? sk : -1;
  if (lane >= kc || cand < 0 || cand >= s.nblocks) cand = -1;
  bool keep = cand >= 0;
  for (int i = 0; i < kc; ++i) {                  // kc is uniform: lane i's entry as a scalar
    const int ci = __builtin_amdgcn_readlane(cand, i);
    if (i < lane && ci == cand) keep = false;
  }
  const bool take = keep && cand < blk && cand < s.nsum && (cand + 1) * a.bs <= cut;
  const unsigned long long mask = __ballot(take);
  if (take) sel[__popcll(mask & ((1ull << lane) - 1ull))] = cand;
  __builtin_amdgcn_wave_barrier();
  return __popcll(mask);
}

// The four header words of a route buffer for the step that ends at kv_len.
struct RouteKey {
  int64_t key, layer, geom, shape;
};
__device__ __forceinline__ RouteKey route_key(int kv_len, int ns, const DecodeArgs& a, const StepArgs& sa) {
  RouteKey r;
  r.key = (int64_t)(uint32_t)kv_len | ((int64_t)ns << 32) | ((int64_t)a.W << 40) | ((int64_t)sa.rule << 48) |
          (1ll << 62);
  r.layer = sa.layer_idx;
  r.geom = (int64_t)(uint32_t)a.bs | (a.ring << 32);
  // pool_rows < 2^30 (MFMA path), lwb, sinks, partners <= 15, CW < 2^20 (host checks)
  r.shape = (int64_t)(uint32_t)a.pool_rows | ((int64_t)sa.lwb << 30) | ((int64_t)sa.sinks << 34) |
            ((int64_t)sa.partners << 38) | ((int64_t)a.CW << 43);
  return r;
}

// Route workgroup r of a step launch (blockIdx.x = r < kRouteGroups, 256
// threads; nseq here counts the attending copies, sequences x copies per
// sequence, and its own counter copy is nseq + r): it advances its own counter
// copy like every other workgroup, computes the routed row of the NEXT step (whose
// counters are the ones this step writes back) with the same functions and
// inputs as that step's own dec_state32 + dec_select32, and writes it into the
// route buffer of that step's kv_len parity in the attending copies j with
// j mod 8 = r (attending workgroup j is blockIdx j + 8 and reads copies
// spw*j .. spw*j + spw - 1, so it runs on the same XCD).  Every sequence of a
// step has the same counters, so one row serves every copy.  It touches no q,
// cache row or output.  sel / hdr: the caller's LDS.
__device__ __forceinline__ void dec_route_workgroup(const DecodeArgs& a, const StepArgs& sa, int tid, int64_t nseq,
                                                    int spw, int* sel, int64_t* hdr, int nthreads = 256) {
  const int64_t g0 = blockIdx.x;
  const DecState32 st = dec_state32<true>(a, sa, nseq + g0);
  // uniform: the attending workgroups report it (and, like them, leave the copy as it was)
  if (st.err || (a.qn_w != nullptr && st.kv_len - 1 >= a.rope_rows)) return;
  const DecState32 nx = dec_advance32(st.kv_len, st.ts1, st.sc1, st.so1, a, sa);
  if (!nx.err) {                               // uniform; else the next step computes its own row
    if (tid < 64) {
      const int p1 = nx.kv_len - 1;
      const int blk1 = min((int)a.bs_div.div((uint32_t)p1), nx.nblocks - 1);
      const int ns1 = dec_select32<true>(p1, blk1, a, sa, nx, tid, sel);
      if (tid == 0) {
        const RouteKey k = route_key(nx.kv_len, ns1, a, sa);
        hdr[0] = k.key;
        hdr[1] = k.layer;
        hdr[2] = k.geom;
        hdr[3] = k.shape;
      }
      if (tid >= ns1 && tid < kDecMaxSum) sel[tid] = 0;
    }
    __syncthreads();
    const int rb = nx.kv_len & 1;
    const int64_t nwg = (nseq + spw - 1) / spw;
    const int64_t mine = nwg > g0 ? (nwg - g0 + 7) / 8 : 0;    // attending workgroups g0, g0 + 8, ...
    const int per = spw * kRouteWords;
    for (int64_t e = tid; e < mine * per; e += nthreads) {
      const int64_t m = e / per;
      const int rem = (int)(e - m * per);
      const int64_t g = (g0 + 8 * m) * spw + rem / kRouteWords;
      const int w = rem % kRouteWords;
      if (g >= nseq) continue;
      const int64_t val =
          w < 4 ? hdr[w] : (int64_t)(uint32_t)sel[2 * (w - 4)] | ((int64_t)sel[2 * (w - 4) + 1] << 32);
      sa.state[kStHeader + kStSlot * g + kStRoute + kRouteWords * rb + w] = val;
    }
  }
  if (tid == 0) {
    int64_t* slot = dec_slot(sa.state, nseq + g0);
    slot[kStOffset] = st.kv_len;
    slot[kStTail] = st.ts1;
    slot[kStCount] = st.sc1;
    slot[kStSumOff] = st.so1;
  }
}

// x where c holds, else zero (a value select: no branch, no memory)
// ---- q/k RMSNorm + rotate-half RoPE of the new token (d = 128) inside the step.
// Rounding points and the summation order of the mean square are those of
// decoder_ops.hip's qk_norm_rope_vec_kernel<128>: chunk gl pairs d in
// [8 gl, 8 gl + 8) with d + 64, summed as fma(lo, lo, fma(hi, hi, s)) element
// by element, and the eight chunk sums are added in xor-butterfly order (1, 2,
// 4); the norm is ((x * r) * w) and the rotation x * cos -+ partner * sin, each
// product and sum rounded on its own, with bf16 after the norm and after RoPE.
// So the rows are bit-identical to that kernel's.
__device__ __forceinline__ float dec_qkn_chunk(const float* lo, const float* hi) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = fmaf(lo[e], lo[e], fmaf(hi[e], hi[e], s));
  return s;
}
__device__ __forceinline__ float dec_qkn_norm(float x, float r, float w) {
#pragma clang fp contract(off)
  return (float)(__bf16)(x * r * w);
}
__device__ __forceinline__ __bf16 dec_qkn_rope(float own, float par, float c, float sn, bool lo) {
#pragma clang fp contract(off)
  return lo ? (__bf16)(own * c + (-par) * sn) : (__bf16)(own * c + par * sn);
}
__device__ __forceinline__ float dec_bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float dec_bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Norm weights and the RoPE row of one lane's piece d = 8 pc + e (and the partner
// piece's weights), requested as soon as the position is known.  q and k share the
// RoPE row and differ in the norm weights.
struct DecQknK {
  bf16x8 w, wp;
  f32x4 c[2], s[2];
};
__device__ __forceinline__ DecQknK dec_qkn_load(const __bf16* nw, const DecodeArgs& a, int p, int pc) {
  DecQknK o;
  const int d0 = 8 * pc;
  o.w = *reinterpret_cast<const bf16x8*>(nw + d0);
  o.wp = *reinterpret_cast<const bf16x8*>(nw + (d0 ^ 64));
  const float* cr = a.rope_cos + (int64_t)p * 128 + d0;
  const float* sr = a.rope_sin + (int64_t)p * 128 + d0;
  o.c[0] = *reinterpret_cast<const f32x4*>(cr);
  o.c[1] = *reinterpret_cast<const f32x4*>(cr + 4);
  o.s[0] = *reinterpret_cast<const f32x4*>(sr);
  o.s[1] = *reinterpret_cast<const f32x4*>(sr + 4);
  return o;
}

// One 16-byte piece of a q or k row: lane (tid % 16) = pc holds d = 8 pc + e and
// the 16 lanes of the row are one DPP row, so the partner piece pc ^ 8 is a
// rotation by 8 and the chunk sums combine by quad permutations (xor 1, 2) and a
// rotation by 4 (lanes pc and pc ^ 8 hold the same chunk sum).  Every lane of the
// wave runs it (DPP); lanes whose row is not wanted ignore the result.
__device__ __forceinline__ uint4 dec_qkn_k(uint4 x, const DecQknK& pk, float eps, int pc) {
  const bool lo = pc < 8;
  const uint32_t u[4] = {x.x, x.y, x.z, x.w};
  float own[8], par[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t pw = (uint32_t)__builtin_amdgcn_mov_dpp((int)u[t], 0x128, 0xf, 0xf, false);   // row_ror:8
    own[2 * t] = dec_bf_lo(u[t]);
    own[2 * t + 1] = dec_bf_hi(u[t]);
    par[2 * t] = dec_bf_lo(pw);
    par[2 * t + 1] = dec_bf_hi(pw);
  }
  float ss = lo ? dec_qkn_chunk(own, par) : dec_qkn_chunk(par, own);
  ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0x124, 0xf, 0xf, false));  // row_ror:4
  const float r = rsqrtf(ss / 128.f + eps);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float on = dec_qkn_norm(own[e], r, (float)pk.w[e]);
    const float pn = dec_qkn_norm(par[e], r, (float)pk.wp[e]);
    o[e] = dec_qkn_rope(on, pn, pk.c[e >> 2][e & 3], pk.s[e >> 2][e & 3], lo);
  }
  return __builtin_bit_cast(uint4, o);
}

__device__ __forceinline__ uint4 keep_if(bool c, uint4 x) {
  return make_uint4(c ? x.x : 0u, c ? x.y : 0u, c ? x.z : 0u, c ? x.w : 0u);
}

// dec_pool with 32-bit ring offsets (same summation order).
template <int D>
__device__ __forceinline__ void dec_pool32(const DecodeArgs& a, const DecState32& s, const __bf16* rk,
                                        const __bf16* rv, __bf16* pk, __bf16* pv, float* part, int tid) {
  constexpr int VEC = 8;
  constexpr int LPR = D / VEC;
  constexpr int RS = 256 / LPR;
  const int ring = (int)a.ring;
  for (int j = 0; j < s.n_new; ++j) {
    const int pos0 = s.so0 + j * a.bs;
    int row0 = (int)a.ring_div.mod((uint32_t)pos0);
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const __bf16* src = kv ? rv : rk;
      __bf16* dst = (kv ? pv : pk) + (uint32_t)(s.sc0 + j) * D;
      const int c = tid % LPR, sl = tid / LPR;
      float acc[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
      for (int tok = sl; tok < a.bs; tok += RS) {
        int row = row0 + tok;
        while (row >= ring) row -= ring;
        const uint4 raw = *reinterpret_cast<const uint4*>(src + (uint32_t)row * D + c * VEC);
        const __bf16* x = reinterpret_cast<const __bf16*>(&raw);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += (float)x[e];
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) part[sl * D + c * VEC + e] = acc[e];
      __syncthreads();
      for (int col = tid; col < D; col += 256) {
        float tot = 0.f;
        for (int k = 0; k < RS; ++k) tot += part[k * D + col];
        const __bf16 val = (__bf16)(tot / (float)a.bs);
        dst[col] = val;
      }
      __syncthreads();
    }
  }
}

// `state` and `q` lead the argument list: the hardware preloads leading pointer
// arguments into SGPRs (the library is built with a kernarg preload count), so
// the counter read needs no kernel-argument load first.
// kQkn: the fused q/k norm + RoPE (d = 128, bfly_decode_step_qk_norm); a separate
// instance with room for its registers, for the batch-1 decoder steps it serves.
// kOS > 0 (with kQkn): the attention output projection as well
// (bfly_decode_step_qk_norm_oproj): o_subs attending workgroups per sequence, each
// computing the sequence's attention and rows [16 kOS sub, 16 kOS (sub + 1)) of the
// partial product W_o[:, 512 kvh .. 512 kvh + 511] o_kvh (kOS sets of four rows per
// wave; GQA groups of four heads of 128:
// sixteen pieces of W_o's rows per kv head).  A lane's piece arithmetic and the sum
// over the sixteen lanes of a row of 16 are those of bfly_q4_gemv, whose total over
// the four kv heads is (p0 + p1) + (p2 + p3), so the partial rows combined in that
// order (bfly_add_rms_norm_q4_gemv_silu_parts) round to bfly_q4_gemv's output bit for
// bit.  Every attending workgroup of a sequence appends the new token and pools a due
// block (the same values), so none reads what another writes in the launch.
template <int D, bool kStep, bool kQkn = false, int kOS = 0>
__global__ void __launch_bounds__(kOS > 0 ? 512 : 256, kQkn ? 1 : (D <= 128 ? 3 : 1))
decode_mfma_kernel(int64_t* state, const void* q, DecodeArgs a, StepArgs sa_in) {
  constexpr bool kOproj = kOS > 0;
  static_assert(!kOproj || (kStep && kQkn && D == 128), "the fused projection rides on the q/k-norm step");
  StepArgs sa = sa_in;
  sa.state = state;
  using T = __bf16;
  constexpr int VEC = 8;
  constexpr int PIECES = D / VEC;
  constexpr int KSTEPS = D / 32;
  constexpr int MTILES = D / 32;                 // output tiles of 32 d (two 16-row halves each)
  constexpr int NT = kDecMfmaKeys / 16;          // key tiles (5)
  constexpr int NPR = (NT + 1) / 2;              // PV k-steps of 32 keys (3, the last half zero)
  constexpr int KP = D + VEC;                    // K row pitch (bf16)
  constexpr int LPR = D / VEC;
  constexpr int RS = 256 / LPR;
  constexpr int KITEMS = kDecMfmaKeys * PIECES;          // K pieces
  // K rows and V rows share one LDS block with the pooling scratch (pooling ends
  // with a barrier before the staging writes); V rows are unpadded and swizzled
  constexpr int KS_BYTES = kDecMfmaKeys * KP * 2, VT_BYTES = kDecMfmaKeys * D * 2;
  constexpr int STAGE_BYTES = KS_BYTES + VT_BYTES > RS * D * 4 ? KS_BYTES + VT_BYTES : RS * D * 4;
  __shared__ __attribute__((aligned(16))) unsigned char stage_lds[STAGE_BYTES];
  T* Ks = reinterpret_cast<T*>(stage_lds);
  T* Vs = reinterpret_cast<T*>(stage_lds + KS_BYTES);   // [80][D], pieces swizzled by row
  __shared__ int selw[4][kDecMaxSum];
  __shared__ int64_t route_hdr[4];
  // kQkn: the 16 normed + rotated q rows of a head group (row pitch 136: the fragment
  // reads of 16 rows at one column hit distinct banks)
  constexpr bool qkn = kQkn && D == 128;
  constexpr int QP = 136;
  __shared__ __attribute__((aligned(16))) T q_lds[qkn ? 16 * QP : 8];
  // kOproj: the attention output of the group's four heads (the projection's input slice), and
  // the workgroup's slice of W_o ([16 kOS rows][16 pieces] and their scale words)
  __shared__ __attribute__((aligned(16))) T o_lds[kOproj ? 4 * D : 8];
  __shared__ u32x4 ow_lds[kOproj ? 16 * kOS * 16 : 1];
  __shared__ uint32_t osb_lds[kOproj ? 16 * kOS * 16 : 1];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lg = lane >> 4, lq = lane & 15;
  if constexpr (kOproj) {
    // Threads 256..511 only bring the W_o slice into LDS and exit: their loads do not queue
    // ahead of the attention waves' own (a wave's loads return in order).  An exited wave no
    // longer counts at a barrier, so the attention waves' staging barrier, which every step
    // takes before the projection, completes only after these writes.
    if (tid >= 256) {
      if (blockIdx.x >= kRouteGroups) {
        const int t2 = tid - 256;
        const int jw = (int)blockIdx.x - kRouteGroups;
        const int sub = (int)a.nseq_div.div((uint32_t)jw);
        const int bh = jw - sub * a.nseq;
        const int kvh = bh - (int)a.hkv_div.div((uint32_t)bh) * a.hkv;
        const uint32_t pc = (uint32_t)(t2 & 15);
        const uint32_t piece = 16u * (uint32_t)kvh + pc;
        const uint32_t grp = piece >> a.o_ppg_log2;
        u32x4 w[kOS];
        uint32_t sc[kOS];
#pragma unroll
        for (int k = 0; k < kOS; ++k) {
          const uint32_t row = (uint32_t)(16 * kOS * sub + (t2 >> 4) + 16 * k);
          w[k] = __builtin_nontemporal_load(a.ow + row * 64u + piece);
          sc[k] = a.osb[row * (uint32_t)a.o_groups + grp];
        }
#pragma unroll
        for (int k = 0; k < kOS; ++k) {
          const int rl = (t2 >> 4) + 16 * k;
          ow_lds[rl * 16 + (int)pc] = w[k];
          osb_lds[rl * 16 + (int)pc] = sc[k];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      }
      return;
    }
  }
  // step mode: the route workgroups come first (no argument is needed to tell
  // them apart), attending workgroup j is blockIdx j + kRouteGroups
  if constexpr (kStep) {
    if (blockIdx.x < kRouteGroups) {
      dec_route_workgroup(a, sa, tid, (int64_t)a.nseq * a.cps, 1, selw[0], route_hdr);
      return;
    }
  }
  // attending workgroup j: its own counter copy j, sequence bh = j mod nseq and
  // sub-workgroup j / nseq (kOproj; found after the counters are requested)
  const int jw = kStep ? (int)blockIdx.x - kRouteGroups : (int)blockIdx.x;
  // step mode: this workgroup's counter copy and both route buffers' headers,
  // requested first (the state pointer needs no argument load); the kv_len
  // parity picks a route buffer below
  // The row-list entries this thread's summary pieces need are requested from both
  // buffers in the same round trip (the slot is one 256-byte line): waiting for
  // them then adds no round trip after the counters.
  constexpr int SKN = kDecMaxSum * PIECES;                         // summary K pieces
  constexpr int SK = (SKN + 255) / 256;
  int64_t cnt[4] = {}, rh[2][4] = {};
  uint64_t rsel2[SK] = {};                       // entry of buffer b in bits 32 b (shifted, not indexed:
                                                 // a parity-indexed array would live in LDS)
  if constexpr (kStep) {
    const int64_t* slot = dec_slot(sa.state, jw);
#pragma unroll
    for (int w = 0; w < 4; ++w) cnt[w] = slot[w];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int w = 0; w < 4; ++w) rh[b][w] = slot[kStRoute + kRouteWords * b + w];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int* rl = reinterpret_cast<const int*>(slot + kStRoute + kRouteWords * b + 4);
#pragma unroll
      for (int it = 0; it < SK; ++it)
        rsel2[it] |= (uint64_t)(uint32_t)rl[min(tid + it * 256, SKN - 1) / PIECES] << (32 * b);
    }
    // keep these loads ahead of the first use of an argument: both round trips
    // then overlap instead of following each other
    __builtin_amdgcn_sched_barrier(0);
  }
  const int sub = kOproj ? (int)a.nseq_div.div((uint32_t)jw) : 0;
  const int bh = kOproj ? jw - sub * a.nseq : jw;
  const int bi = (int)a.hkv_div.div((uint32_t)bh);
  const int kvh = bh - bi * a.hkv;
  const int gsz = a.gsz;
  const T* qhead = reinterpret_cast<const T*>(q) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz) * D;

  // Q^T fragments of heads 16*hg + lq (B operand: d = lg*(D/4) + 8*ks + [0, 8)).
  // Columns past the group read its last head: they are computed and never
  // stored.  The loads are unconditional, so nothing waits on them before the
  // scores.
  bf16x8 qf[KSTEPS];
  auto load_q = [&](int hg) {
    const int head = min(16 * hg + lq, gsz - 1);
    const T* qrow = qhead + (uint32_t)head * D + lg * (D / 4);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 8 * ks);
  };
  // kQkn: thread tid holds piece tid % 16 of raw q row 16 hg + tid / 16 (the group's
  // last head past gsz); the 256 threads transform the 16 rows of a head group into
  // q_lds, from which every wave reads its fragments
  uint4 q_raw{};
  auto load_q_raw = [&](int hg) {
    const int head = min(16 * hg + (tid >> 4), gsz - 1);
    q_raw = *reinterpret_cast<const uint4*>(qhead + (uint32_t)head * D + (tid & 15) * VEC);
  };
  if constexpr (qkn) load_q_raw(0);
  else load_q(0);

  const DecState32 st =
      kStep ? dec_advance32(cnt[kStOffset], cnt[kStTail], cnt[kStCount], cnt[kStSumOff], a, sa) : dec_state32<false>(a, sa, bh);
  // with the fused q/k norm, a position past the RoPE table is an error of the step
  if (kStep && (st.err || (qkn && st.kv_len - 1 >= a.rope_rows))) {
    if (tid == 0) sa.state[kStError] = st.err ? kErrCapacity : kErrRope;
    return;
  }
  // the row-list entries of this step's route buffer (kv_len parity)
  int rsel[SK];
#pragma unroll
  for (int it = 0; it < SK; ++it) rsel[it] = (int)(uint32_t)(rsel2[it] >> (32 * (st.kv_len & 1)));
  const int p = st.kv_len - 1;
  DecQknK qkn_k{};
  bf16x8 qn_w{}, qn_wp{};   // q's norm weights of this thread's piece (RoPE row: qkn_k's)
  if constexpr (qkn) {
    qkn_k = dec_qkn_load(a.kn_w, a, p, tid % PIECES);
    qn_w = *reinterpret_cast<const bf16x8*>(a.qn_w + 8 * (tid % PIECES));
    qn_wp = *reinterpret_cast<const bf16x8*>(a.qn_w + ((8 * (tid % PIECES)) ^ 64));
  }
  // norm + RoPE of this thread's q piece into q_lds
  auto put_q = [&]() {
    const DecQknK pq{qn_w, qn_wp, {qkn_k.c[0], qkn_k.c[1]}, {qkn_k.s[0], qkn_k.s[1]}};
    *reinterpret_cast<uint4*>(q_lds + (tid >> 4) * QP + (tid & 15) * VEC) = dec_qkn_k(q_raw, pq, a.qk_eps, tid & 15);
  };
  auto read_q = [&]() {
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(q_lds + lq * QP + lg * (D / 4) + 8 * ks);
  };
  const int lo = max(max(p - a.W + 1, st.tail_start), 0);
  const int nw = p - lo + 1;
  const int ring = (int)a.ring;

  const T* knew = a.k_new ? reinterpret_cast<const T*>(a.k_new) + (int64_t)bh * D : nullptr;
  const T* vnew = a.v_new ? reinterpret_cast<const T*>(a.v_new) + (int64_t)bh * D : nullptr;
  T* rk = reinterpret_cast<T*>(a.ring_k) + (int64_t)bh * a.kv_rows * D;
  T* rv = reinterpret_cast<T*>(a.ring_v) + (int64_t)bh * a.kv_rows * D;
  T* pk = reinterpret_cast<T*>(const_cast<void*>(a.pool_k)) + (int64_t)bh * a.pool_rows * D;
  T* pv = reinterpret_cast<T*>(const_cast<void*>(a.pool_v)) + (int64_t)bh * a.pool_rows * D;

  if constexpr (kStep) {
    if (st.n_new > 0) dec_pool32<D>(a, st, rk, rv, pk, pv, reinterpret_cast<float*>(stage_lds), tid);
  }
  const int slot_lo = ring ? (int)a.ring_div.mod((uint32_t)lo) : lo - st.tail_start;
  const int r_new = knew != nullptr ? nw - 1 : -1;   // row of position p: read from k_new/v_new

  // element offset of window row r (< nw) in the ring or linear tail
  auto ring_off = [&](int r) -> uint32_t {
    int row = slot_lo + r;
    if (ring && row >= ring) row -= ring;
    return (uint32_t)row * D;
  };
  // Window row r, clamped to the last one: every load is issued unconditionally
  // from valid memory, and rows r >= nw are zeroed when they are written to LDS.
  auto win_row = [&](int r, bool vside) -> const T* {
    r = min(r, nw - 1);
    if (r == r_new) return vside ? vnew : knew;
    return (vside ? rv : rk) + ring_off(r);
  };

  // ---- staging: keys 0..63 are the window rows (lo + r), keys 64..79 the routed
  // summaries in row order; unused keys are zero rows and masked in the scores.
  // K and V are stored row-major (V with swizzled pieces, read back transposed).
  // Window rows are requested first, the routed selection runs while they are in
  // flight, then the summary rows are requested.
  constexpr int WK = kDecMaxWin * PIECES / 256;                   // window K pieces per thread
  static_assert(kDecMaxWin * PIECES % 256 == 0, "staging split");
  static_assert(kDecMaxWin + kDecMaxSum == kDecMfmaKeys, "key layout");
  int ns;
  {
    uint4 kx[WK], vx[WK], skx[SK], svx[SK];
#pragma unroll
    for (int it = 0; it < WK; ++it) {
      const int i = tid + it * 256;
      kx[it] = *reinterpret_cast<const uint4*>(win_row(i / PIECES, false) + (i % PIECES) * VEC);
      vx[it] = *reinterpret_cast<const uint4*>(win_row(i / PIECES, true) + (i % PIECES) * VEC);
    }
    bool pre = false;   // this step's routed row was left by the previous step
    if constexpr (kStep) {
      const int rb = st.kv_len & 1;
      const RouteKey want = route_key(st.kv_len, 0, a, sa);
      const int64_t k0 = rb ? rh[1][0] : rh[0][0];
      pre = (k0 & ~(0x1fll << 32)) == want.key && (rb ? rh[1][1] : rh[0][1]) == want.layer &&
            (rb ? rh[1][2] : rh[0][2]) == want.geom && (rb ? rh[1][3] : rh[0][3]) == want.shape;
      if (pre) ns = min((int)((k0 >> 32) & 0x1f), kDecMaxSum);
    }
    if (!pre) {
      const int blk = min((int)a.bs_div.div((uint32_t)p), st.nblocks - 1);
      ns = dec_select32<kStep>(p, blk, a, sa, st, lane, selw[wave]);
    }
    // summary j: pool row n (row 0 stands in for j >= ns; zeroed below); a row
    // left by the previous step is clamped to the pool, so no load leaves it
#pragma unroll
    for (int it = 0; it < SK; ++it) {
      const int i = min(tid + it * 256, SKN - 1);
      const int j = i / PIECES;
      int n = 0;
      if (j < ns) n = pre ? min(max(rsel[it], 0), (int)a.pool_rows - 1) : selw[wave][j];
      skx[it] = *reinterpret_cast<const uint4*>(pk + (uint32_t)n * D + (i % PIECES) * VEC);
      svx[it] = *reinterpret_cast<const uint4*>(pv + (uint32_t)n * D + (i % PIECES) * VEC);
    }
    // append the new token to its ring slot; requested after every staging load so
    // that its wait coincides with theirs (the staging reads it from k_new/v_new)
    if (knew != nullptr && tid < 2 * PIECES && !(qkn && tid < PIECES)) {   // normed k: appended below
      const int pc = tid % PIECES;
      const T* src = tid < PIECES ? knew : vnew;
      T* dst = tid < PIECES ? rk : rv;
      *reinterpret_cast<uint4*>(dst + ring_off(nw - 1) + pc * VEC) = *reinterpret_cast<const uint4*>(src + pc * VEC);
    }
    auto put_v = [&](int r, int pc, uint4 x) {
      *reinterpret_cast<uint4*>(Vs + r * D + (pc ^ vrow_swizzle<D>(r)) * VEC) = x;
    };
#pragma unroll
    for (int it = 0; it < WK; ++it) {
      const int i = tid + it * 256;
      const int r = i / PIECES, pc = i % PIECES;
      uint4 kv = kx[it];
      if constexpr (D == 128) {
        // the wave's four rows of this iteration hold the new one: norm + RoPE it
        // (wave-uniform branch) and append the result to its ring slot
        const int row0 = it * (256 / PIECES) + wave * (64 / PIECES);
        if (qkn && knew != nullptr && nw - 1 >= row0 && nw - 1 < row0 + 64 / PIECES) {
          // every lane runs the transform (DPP); only the new row's lanes keep it
          const uint4 kn = dec_qkn_k(kv, qkn_k, a.qk_eps, pc);
          if (r == nw - 1) {
            kv = kn;
            *reinterpret_cast<uint4*>(rk + ring_off(nw - 1) + pc * VEC) = kv;
          }
        }
      }
      *reinterpret_cast<uint4*>(Ks + r * KP + pc * VEC) = keep_if(r < nw, kv);
      put_v(r, pc, keep_if(r < nw, vx[it]));
    }
#pragma unroll
    for (int it = 0; it < SK; ++it) {
      const int i = tid + it * 256;
      const int j = i / PIECES, pc = i % PIECES;
      if (i < SKN) {
        *reinterpret_cast<uint4*>(Ks + (kDecMaxWin + j) * KP + pc * VEC) = keep_if(j < ns, skx[it]);
        put_v(kDecMaxWin + j, pc, keep_if(j < ns, svx[it]));
      }
    }
    if constexpr (qkn) put_q();
  }
  __syncthreads();
  if constexpr (qkn) read_q();

  const float sl2 = a.scale * 1.4426950408889634f;   // host guarantees scale > 0 on this path
  for (int hg = 0; 16 * hg < gsz; ++hg) {
    if (hg > 0) {
      if constexpr (qkn) {
        load_q_raw(hg);
        __syncthreads();                 // every wave has read the previous group's rows
        put_q();
        __syncthreads();
        read_q();
      } else {
        load_q(hg);
      }
    }
    // S^T: lane (lg, lq) holds keys 16t + 4lg + i of head 16hg + lq
    f32x4 sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      bf16x8 kf[KSTEPS];
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        kf[ks] = *reinterpret_cast<const bf16x8*>(Ks + (16 * t + lq) * KP + lg * (D / 4) + 8 * ks);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[ks], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * t + 4 * lg + i;
        sc[t][i] = key < nw || (key >= kDecMaxWin && key < kDecMaxWin + ns) ? acc[i] : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) mx = fmaxf(mx, fmaxf(fmaxf(sc[t][0], sc[t][1]), fmaxf(sc[t][2], sc[t][3])));
    mx = col_max4(mx);
    const float nm = -mx * sl2;                      // nw >= 1: every column has a finite max
    float lsum = 0.f;
    bf16x8 pf[NPR];
    pf[NPR - 1] = bf16x8{};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(sc[t][i], sl2, nm));
        lsum += e;
        pf[t / 2][(t % 2) * 4 + i] = (__bf16)e;
      }
    lsum = col_sum4(lsum);
    const float inv = __builtin_amdgcn_rcpf(fmaxf(lsum, 1e-30f));
    const int head = 16 * hg + lq;
    __bf16* orow = reinterpret_cast<__bf16*>(a.out) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz + head) * D;
    // O^T = V^T P^T: tile (mt, half) row r holds d = mt*32 + (r/4)*8 + half*4 + r%4, and its
    // k index runs over keys (tile 2pr, 4lg..4lg+3) then (tile 2pr+1, 4lg..4lg+3), the
    // order of this lane's P fragment, so no lane exchange is needed.
    for (int mt = wave; mt < MTILES; mt += 4) {
      f32x4 o[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // transposing reads of row-major V: lane (lg, lq) reads the 4 d
        // mt*32 + (lq&3)*8 + half*4 of key 16t + 4lg + (lq>>2), so lane lq receives
        // d row lq's keys 16t + 4lg + 0..3
        const int unit = mt * 8 + (lq & 3) * 2 + half;
        auto vfrag = [&](int t) {
          const int r = 16 * t + 4 * lg + (lq >> 2);
          return read_tr(Vs + r * D + (unit ^ (2 * vrow_swizzle<D>(r))) * 4);
        };
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pr = 0; pr < NPR; ++pr) {
          const bf16x4 va = vfrag(2 * pr);
          const bf16x4 vb = 2 * pr + 1 < NT ? vfrag(2 * pr + 1) : bf16x4{};
          const bf16x8 vf = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[pr], acc, 0, 0, 0);
        }
        o[half] = acc;
      }
      if (head < gsz) {
        bf16x8 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w[i] = (__bf16)(o[0][i] * inv);
          w[4 + i] = (__bf16)(o[1][i] * inv);
        }
        if (!kOproj || sub == 0) *reinterpret_cast<bf16x8*>(orow + mt * 32 + lg * 8) = w;
        if constexpr (kOproj) *reinterpret_cast<bf16x8*>(o_lds + head * D + mt * 32 + lg * 8) = w;
      }
    }
  }
  if constexpr (kOproj) {
    // the partial product of this workgroup's rows over the group's 512 outputs: lane (r4, pc)
    // = (lane / 16, lane % 16) takes piece pc of local rows 4 kOS wave + 4 s + r4 (W_o's rows
    // 16 kOS sub + ..., pieces 16 kvh + pc), over o_lds[32 pc, 32 pc + 32) (head pc / 4, d from
    // 32 (pc % 4))
    __syncthreads();
    const int pc = lane & 15;
    bf16x8 xr[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xr[c] = *reinterpret_cast<const bf16x8*>(o_lds + pc * 32 + 8 * c);
    float xq[kQ4PieceCodes], xs;
    q4_piece_x(xr, true, xq, xs);
    float* prow = a.opart + ((int64_t)kvh * (a.nseq / a.hkv) + bi) * a.o_rows;
#pragma unroll
    for (int st4 = 0; st4 < kOS; ++st4) {
      const int rl = 4 * kOS * wave + 4 * st4 + (lane >> 4);
      float acc = 0.f;
      acc += q4_piece_dot(ow_lds[rl * 16 + pc], osb_lds[rl * 16 + pc], xq, xs);
      acc = q4_row16_sum(acc);
      if (pc == 0) prow[16 * kOS * sub + 4 * kOS * wave + 4 * st4 + (lane >> 4)] = acc;
    }
  }
  if constexpr (kStep) {
    // each workgroup advances its own counter copy (see decode_kernel); the first
    // workgroup of a sequence also the copies no attending workgroup of this launch owns
    if (tid == 0)
      dec_put_counters(sa.state, bh, a.nseq, sub, sub + 1, 0, st.kv_len, st.ts1, st.sc1, st.so1, false);
    const int own = kOproj ? a.o_subs : 1;
    if (sub == 0 && tid >= 1)
      dec_put_counters(sa.state, bh, a.nseq, own, a.cps, tid - 1, st.kv_len, st.ts1, st.sc1, st.so1, false);
  }
}

// ---------------------------------------------------------------------------------------------
// Step-mode decode with the key tiles split over the waves (bf16, d = 128, GQA groups of at
// most 16), for batches that fill the chip.  One workgroup per sequence as above, but:
//   - window K is not staged: wave w loads the MFMA A fragments of key tile w (window keys
//     16w .. 16w + 15) straight from the ring into registers and computes only that tile's
//     scores (the workgroup kernel computes every tile in every wave); wave 0 also computes
//     the summary tile, whose 16 rows it stages in LDS by DMA (so no wave holds two tiles of
//     K fragments in registers);
//   - V goes to LDS by DMA (global_load_lds_dwordx4: lane l of an instruction writes bytes
//     16 l of its 1 KiB, so the row swizzles are chosen through the source addresses) -- no
//     register staging and no LDS writes by the waves;
//   - the routed summaries' V enters the last PV k-step as register fragments: lane (lq, lg)
//     loads the 2-byte elements that the transposing LDS read would give it, so only the 64
//     window rows of V are staged;
//   - the waves exchange per-head tile maxima and the fp32 exponentials through LDS (two
//     barriers; the exponentials of tiles 0..3 reuse the summary K rows); every wave then sums
//     the exponentials in the workgroup kernel's order, forms the same P fragments, and
//     computes O^T = V^T P^T for its output tile.
// 22 KiB of LDS and at most 72 VGPRs, so 7 sequences are resident per CU.  Masks,
// exponentials, summation order and MFMA inputs are the workgroup kernel's, so the results
// are bit-identical to it.
constexpr int kSplitOffSK = kDecMaxWin * 128 * 2;                  // V window rows [64][128]
constexpr int kSplitOffEx4 = kSplitOffSK + kDecMaxSum * 128 * 2;   // summary K [16][128] / ex tiles 0..3
constexpr int kSplitOffTmax = kSplitOffEx4 + 64 * 4 * 4;           // ex tile 4 [64][4]
constexpr int kSplitOffSel = kSplitOffTmax + 5 * 16 * 4;           // tmax [5][16]
constexpr int kSplitLds = kSplitOffSel + 4 * kDecMaxSum * 4;       // selw [4][16]
static_assert(kDecMaxSum * 128 * 2 == 4 * 64 * 4 * 4, "ex tiles 0..3 fill the summary K rows");

// piece pc of summary K row r sits at pc ^ (r & 15): the fragment reads of 16 rows hit 16
// distinct 16-byte positions
__device__ __forceinline__ constexpr int krow_swizzle(int row) { return row & 15; }

// global_load_lds_dwordx4: lane l's 16 bytes at g go to LDS bytes lds + 16 l (lds wave-uniform).
// Issued as assembly so that the compiler's wait counting sees only loads into registers:
// with an LDS DMA in its count it cannot rely on return order and waits for everything before
// any register use.  Loads still return in order among themselves, so its waits stay
// sufficient; whoever reads the LDS waits for the DMA itself (s_waitcnt vmcnt(0)).
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

__global__ void __launch_bounds__(256, 7)   // 7 waves per SIMD: 7 sequences per CU (LDS)
decode_split_kernel(int64_t* state, const void* q, DecodeArgs a, StepArgs sa_in) {
  StepArgs sa = sa_in;
  sa.state = state;
  using T = __bf16;
  constexpr int D = 128, VEC = 8, KSTEPS = D / 32, NT = kDecMfmaKeys / 16, NPR = (NT + 1) / 2;
  static_assert(NT == 5 && D / 32 == 4, "one key tile and one output tile per wave, tile 4 on wave 0");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kSplitLds];
  T* Vs = reinterpret_cast<T*>(lds);                                 // pieces swizzled by row
  T* SKs = reinterpret_cast<T*>(lds + kSplitOffSK);                  // until the first barrier
  auto ex = [&](int t) -> float* {                                   // [64][4] per tile, after it
    return reinterpret_cast<float*>(lds + (t < 4 ? kSplitOffSK + t * 1024 : kSplitOffEx4));
  };
  float(*tmax)[16] = reinterpret_cast<float(*)[16]>(lds + kSplitOffTmax);
  int(*selw)[kDecMaxSum] = reinterpret_cast<int(*)[kDecMaxSum]>(lds + kSplitOffSel);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lg = lane >> 4, lq = lane & 15;
  if (blockIdx.x < kRouteGroups) {
    dec_route_workgroup(a, sa, tid, (int64_t)a.nseq * a.cps, 1, selw[0], reinterpret_cast<int64_t*>(lds));
    return;
  }
  const int bh = (int)blockIdx.x - kRouteGroups;
  const int64_t* slot = dec_slot(sa.state, bh);
  int64_t cnt[4], rh[2][4];
  // row-list entry lq of both buffers, buffer b in bits 32 b (shifted, not indexed: a
  // parity-indexed array would live in LDS)
  uint64_t rk2 = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) cnt[w] = slot[w];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int w = 0; w < 4; ++w) rh[b][w] = slot[kStRoute + kRouteWords * b + w];
    const int* rl = reinterpret_cast<const int*>(slot + kStRoute + kRouteWords * b + 4);
    rk2 |= (uint64_t)(uint32_t)rl[lq] << (32 * b);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int bi = (int)a.hkv_div.div((uint32_t)bh);
  const int kvh = bh - bi * a.hkv;
  const int gsz = a.gsz;
  const T* qhead = reinterpret_cast<const T*>(q) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz) * D;
  bf16x8 qf[KSTEPS];
  {
    const T* qrow = qhead + (uint32_t)min(lq, gsz - 1) * D + lg * (D / 4);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 8 * ks);
  }
  const DecState32 st = dec_advance32(cnt[kStOffset], cnt[kStTail], cnt[kStCount], cnt[kStSumOff], a, sa);
  if (st.err) {                                  // uniform: every workgroup sees the same counters
    if (tid == 0) sa.state[kStError] = kErrCapacity;
    return;
  }
  // entry lq of this step's route buffer (used when the buffer's key matches); lane
  // 16 g + j holds entry j for every g
  const int rsel_k = (int)(uint32_t)(rk2 >> (32 * (st.kv_len & 1)));
  const int p = st.kv_len - 1;
  const int lo = max(max(p - a.W + 1, st.tail_start), 0);
  const int nw = p - lo + 1;
  const int ring = (int)a.ring;
  const T* knew = reinterpret_cast<const T*>(a.k_new) + (int64_t)bh * D;
  const T* vnew = reinterpret_cast<const T*>(a.v_new) + (int64_t)bh * D;
  T* rk = reinterpret_cast<T*>(a.ring_k) + (int64_t)bh * a.kv_rows * D;
  T* rv = reinterpret_cast<T*>(a.ring_v) + (int64_t)bh * a.kv_rows * D;
  T* pk = reinterpret_cast<T*>(const_cast<void*>(a.pool_k)) + (int64_t)bh * a.pool_rows * D;
  T* pv = reinterpret_cast<T*>(const_cast<void*>(a.pool_v)) + (int64_t)bh * a.pool_rows * D;
  // blocks that became due: pooled (LDS scratch = the V rows, free until the DMA below),
  // written to the pool and read back after the barrier that ends dec_pool32
  if (st.n_new > 0) dec_pool32<D>(a, st, rk, rv, pk, pv, reinterpret_cast<float*>(lds), tid);
  const int slot_lo = (int)a.ring_div.mod((uint32_t)lo);
  const int r_new = nw - 1;                      // position p: read from k_new / v_new
  auto ring_off = [&](int r) -> uint32_t {
    int row = slot_lo + r;
    if (row >= ring) row -= ring;
    return (uint32_t)row * D;
  };
  // window row r clamped to the last one (finite data; masked keys get P = 0)
  auto win_row = [&](int r, bool vside) -> const T* {
    r = min(r, nw - 1);
    if (r == r_new) return vside ? vnew : knew;
    return (vside ? rv : rk) + ring_off(r);
  };
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // Requests in the order of their use: this wave's K fragments (window tile `wave`), the
  // summary K rows (wave 0, DMA), then the V rows (DMA) and the summary V fragments, which are
  // needed only after the first barrier.
  bf16x8 kf[KSTEPS];
  {
    const T* src = win_row(16 * wave + lq, false) + lg * (D / 4);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) kf[ks] = *reinterpret_cast<const bf16x8*>(src + 8 * ks);
  }
  // routed selection: left by the previous step's route workgroups, or computed by each wave
  int ns;
  bool pre;
  {
    const int rb = st.kv_len & 1;
    const RouteKey want = route_key(st.kv_len, 0, a, sa);
    const int64_t k0 = rb ? rh[1][0] : rh[0][0];
    pre = (k0 & ~(0x1fll << 32)) == want.key && (rb ? rh[1][1] : rh[0][1]) == want.layer &&
          (rb ? rh[1][2] : rh[0][2]) == want.geom && (rb ? rh[1][3] : rh[0][3]) == want.shape;
    if (pre) {
      ns = min((int)((k0 >> 32) & 0x1f), kDecMaxSum);
    } else {
      const int blk = min((int)a.bs_div.div((uint32_t)p), st.nblocks - 1);
      ns = dec_select32<true>(p, blk, a, sa, st, lane, selw[wave]);
    }
  }
  // pool row of summary j < 16 (row 0 when j >= ns); rs = entry j of the route buffer.
  // Branch-free: selw is read either way (unused when the route buffer is)
  auto entry = [&](int j, int rs) -> int {
    const int e = pre ? min(max(rs, 0), (int)a.pool_rows - 1) : selw[wave][j];
    return j < ns ? e : 0;
  };
  // route-buffer entries of summaries 4 lg + jj (summary V fragments) and 4 jj + lg (summary K
  // rows), fetched together from the lanes that hold them (lane j holds entry j)
  int ev[4], ek[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    ev[jj] = __builtin_amdgcn_ds_bpermute(4 * (4 * lg + jj), rsel_k);
    ek[jj] = __builtin_amdgcn_ds_bpermute(4 * (4 * jj + lg), rsel_k);
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)lds;
  if (wave == 0) {
    // summary K rows 4 i + lg (instruction i), pieces swizzled by row
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + lg;
      const int pc = lq ^ krow_swizzle(r);
      lds_dma16(pk + (uint32_t)entry(r, ek[i]) * D + pc * VEC, lds0 + kSplitOffSK + 1024 * i);
    }
  }
  // this wave's 16 V rows by DMA (rows 4 i + lg of instruction i, pieces swizzled by row)
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int i = 4 * wave + ii;
    const int r = 4 * i + lg;
    const int pc = lq ^ vrow_swizzle<D>(r);
    lds_dma16(win_row(r, true) + pc * VEC, lds0 + 1024 * i);
  }
  // summary V fragments of output tile mt = wave: element jj of half h is summary 4 lg + jj at
  // d = 32 wave + 8 (lq >> 2) + 4 h + (lq & 3) -- what read_tr would return for staged row
  // 64 + 4 lg + jj.  Summaries past ns read pool row 0 and are zeroed at their use, as the
  // workgroup kernel zeroes its staged rows.  16-bit vector lanes, so that the loads fill
  // register halves in place (no packing that would wait for them here).
  typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
  u16x4 svraw[2] = {u16x4{}, u16x4{}};
  {
    const unsigned short* col = reinterpret_cast<const unsigned short*>(pv) + wave * 32 + 8 * (lq >> 2) + (lq & 3);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const unsigned short* src = col + (uint32_t)entry(4 * lg + jj, ev[jj]) * D;
      svraw[0][jj] = src[0];
      svraw[1][jj] = src[4];
    }
  }
  // scores of this wave's tile (and of the summary tile on wave 0), column maxima
  const float sl2 = a.scale * 1.4426950408889634f;
  auto tile_scores = [&](const bf16x8 (&k)[KSTEPS], int t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k[ks], qf[ks], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 16 * t + 4 * lg + i;
      acc[i] = key < nw || (key >= kDecMaxWin && key < kDecMaxWin + ns) ? acc[i] : -INFINITY;
    }
    return acc;
  };
  const f32x4 sc = tile_scores(kf, wave);
  // append the new token's K to its ring slot: window row nw - 1 was read from k_new, and the
  // lanes of row 16 wave + lq = nw - 1 hold it (d = 32 lg + 8 ks + 0..7)
  if (16 * wave + lq == nw - 1) {
    T* dst = rk + ring_off(nw - 1) + lg * (D / 4);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) *reinterpret_cast<bf16x8*>(dst + 8 * ks) = kf[ks];
  }
  f32x4 sc4 = {};
  {
    float m = col_max4(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    if (lg == 0) tmax[wave][lq] = m;
    if (wave == 0) {
      // the summary rows (this wave's DMA) have landed: a full wait, since LDS-DMA and loads
      // returning to registers are not guaranteed to complete in issue order (the compiler
      // waits for everything before the first score MFMA for the same reason)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      bf16x8 kf4[KSTEPS];
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        kf4[ks] = *reinterpret_cast<const bf16x8*>(SKs + lq * D + ((4 * lg + ks) ^ krow_swizzle(lq)) * VEC);
      sc4 = tile_scores(kf4, NT - 1);
      m = col_max4(fmaxf(fmaxf(sc4[0], sc4[1]), fmaxf(sc4[2], sc4[3])));
      if (lg == 0) tmax[NT - 1][lq] = m;
    }
  }
  __syncthreads();
  float mx = tmax[0][lq];
#pragma unroll
  for (int t = 1; t < NT; ++t) mx = fmaxf(mx, tmax[t][lq]);
  const float nm = -mx * sl2;                    // nw >= 1: every column has a finite max
  {
    f32x4 e;
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(sc[i], sl2, nm));
    *reinterpret_cast<f32x4*>(ex(wave) + lane * 4) = e;
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(sc4[i], sl2, nm));
      *reinterpret_cast<f32x4*>(ex(NT - 1) + lane * 4) = e;
    }
  }
  // this wave's V rows have landed (the DMA counts as outstanding vector memory); after the
  // barrier every wave's have
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // append the new token's V (staged row nw - 1, read from v_new)
  if (wave == 1 && lane < 16) {
    const int r = nw - 1;
    *reinterpret_cast<uint4*>(rv + ring_off(r) + lane * VEC) =
        *reinterpret_cast<const uint4*>(Vs + r * D + (lane ^ vrow_swizzle<D>(r)) * VEC);
  }
  float lsum = 0.f;
  bf16x8 pf[NPR];
  pf[NPR - 1] = bf16x8{};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const f32x4 e = *reinterpret_cast<const f32x4*>(ex(t) + lane * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lsum += e[i];
      pf[t / 2][(t % 2) * 4 + i] = (__bf16)e[i];
    }
  }
  lsum = col_sum4(lsum);
  const float inv = __builtin_amdgcn_rcpf(fmaxf(lsum, 1e-30f));
  bf16x4 svf[2];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const bool live = 4 * lg + jj < ns;
#pragma unroll
    for (int h = 0; h < 2; ++h) svf[h][jj] = __builtin_bit_cast(T, (unsigned short)(live ? svraw[h][jj] : 0));
  }
  // O^T = V^T P^T for output tile mt = wave (as the workgroup kernel); the summary tile's V
  // fragments come from registers
  const int mt = wave;
  f32x4 o[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int unit = mt * 8 + (lq & 3) * 2 + half;
    auto vfrag = [&](int t) {
      const int r = 16 * t + 4 * lg + (lq >> 2);
      return read_tr(Vs + r * D + (unit ^ (2 * vrow_swizzle<D>(r))) * 4);
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pr = 0; pr < NPR; ++pr) {
      const bf16x4 va = 2 * pr == NT - 1 ? svf[half] : vfrag(2 * pr);
      const bf16x4 vb = 2 * pr + 1 < NT ? vfrag(2 * pr + 1) : bf16x4{};
      const bf16x8 vf = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[pr], acc, 0, 0, 0);
    }
    o[half] = acc;
  }
  if (lq < gsz) {
    __bf16* orow = reinterpret_cast<__bf16*>(a.out) + ((int64_t)bi * a.hq + (int64_t)kvh * gsz + lq) * D;
    bf16x8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = (__bf16)(o[0][i] * inv);
      w[4 + i] = (__bf16)(o[1][i] * inv);
    }
    *reinterpret_cast<bf16x8*>(orow + mt * 32 + lg * 8) = w;
  }
  dec_put_counters(sa.state, bh, a.nseq, 0, a.cps, tid, st.kv_len, st.ts1, st.sc1, st.so1, false);
}

// Sequences (batch x kv heads) from which the step runs decode_split_kernel: measured on
// MI355X at d = 128, the workgroup kernel is 0.1-0.2 us faster up to 256 sequences and the
// split kernel 16-19 % faster from 1024 (BFLY_DECODE_SPLIT_MIN overrides; 0 disables it).
static int64_t decode_split_min() {
  static const int64_t v = [] {
    const char* e = getenv("BFLY_DECODE_SPLIT_MIN");
    return e && *e ? (int64_t)atoll(e) : (int64_t)512;
  }();
  return v;
}

// bf16 with a positive scale (folded into exp2) runs on MFMA when its 32-bit
// positions and offsets suffice
static bool decode_on_mfma(const DecodeArgs& a, int d, bool step) {
  const int64_t lim = kDecPosLimit;
  const bool fits = a.kv_rows * d < lim && a.pool_rows * d < lim && a.ring < lim &&
                    (step ? (a.pool_rows + 2) * a.bs + a.ring + (a.W > a.CW ? a.W : a.CW) < lim
                          : a.kv_len < lim && a.nblocks < lim && a.nsum < lim);
  return a.scale > 0.f && fits;
}

template <typename T, bool kStep>
static void launch_decode(const DecodeArgs& a, const StepArgs& sa, int d, int64_t grid, hipStream_t stream) {
  // bf16 with a positive scale (folded into exp2) runs on MFMA when its 32-bit
  // positions and offsets suffice; fp32 and larger caches on the lane-per-key kernel
  if constexpr (sizeof(T) == 2) {
    if (decode_on_mfma(a, d, kStep)) {
      DecodeArgs m = a;
      m.bs_div = FastDiv::make((uint32_t)a.bs);
      m.ring_div = FastDiv::make(a.ring > 0 ? (uint32_t)a.ring : 1u);
      m.hkv_div = FastDiv::make((uint32_t)a.hkv);
      m.gsz = a.hq / a.hkv;
      m.nseq = (int)grid;
      const int64_t mgrid = kStep ? grid + kRouteGroups : grid;   // step mode: plus the route workgroups
      if constexpr (kStep) {
        if (a.ow != nullptr) {   // the fused output projection: o_subs attending workgroups per sequence
          m.nseq_div = FastDiv::make((uint32_t)grid);
          const dim3 og((unsigned)(grid * a.o_subs + kRouteGroups));
          // 512 threads: 256 attend, 256 bring the W_o slice into LDS
          if (a.o_rows == 32 * a.o_subs)
            hipLaunchKernelGGL((decode_mfma_kernel<128, true, true, 2>), og, dim3(512), 0, stream, sa.state, m.q, m, sa);
          else
            hipLaunchKernelGGL((decode_mfma_kernel<128, true, true, 4>), og, dim3(512), 0, stream, sa.state, m.q, m, sa);
          return;
        }
        const int64_t smin = decode_split_min();
        if (d == 128 && a.qn_w == nullptr && m.gsz <= 16 && smin > 0 && grid >= smin) {
          hipLaunchKernelGGL(decode_split_kernel, dim3((unsigned)mgrid), dim3(256), 0, stream, sa.state, m.q, m, sa);
          return;
        }
      }
      switch (d) {
        case 64:
          hipLaunchKernelGGL((decode_mfma_kernel<64, kStep>), dim3((unsigned)mgrid), dim3(256), 0, stream, sa.state,
                             m.q, m, sa);
          return;
        case 128:
          if (kStep && a.qn_w != nullptr)
            hipLaunchKernelGGL((decode_mfma_kernel<128, kStep, true>), dim3((unsigned)mgrid), dim3(256), 0, stream,
                               sa.state, m.q, m, sa);
          else
            hipLaunchKernelGGL((decode_mfma_kernel<128, kStep>), dim3((unsigned)mgrid), dim3(256), 0, stream, sa.state,
                               m.q, m, sa);
          return;
        default:
          hipLaunchKernelGGL((decode_mfma_kernel<256, kStep>), dim3((unsigned)mgrid), dim3(256), 0, stream, sa.state,
                             m.q, m, sa);
          return;
      }
    }
  }
  switch (d) {
    case 64:
      hipLaunchKernelGGL((decode_kernel<T, 64, kStep>), dim3((unsigned)grid), dim3(256), 0, stream, a, sa);
      break;
    case 128:
      hipLaunchKernelGGL((decode_kernel<T, 128, kStep>), dim3((unsigned)grid), dim3(256), 0, stream, a, sa);
      break;
    default:
      // fp32 rows of 256 do not fit the LDS staging; the host rejects that case.
      if constexpr (sizeof(T) == 2)
        hipLaunchKernelGGL((decode_kernel<T, 256, kStep>), dim3((unsigned)grid), dim3(256), 0, stream, a, sa);
      break;
  }
}

}  // namespace bfly

using namespace bfly;

extern "C" int bfly_decode(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                           const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                           int64_t ring_capacity, int64_t tail_start, int64_t kv_len,
                           const void* pool_k, const void* pool_v, int64_t pool_capacity,
                           int64_t summary_count, const bfly_topology_t* topology, int64_t num_blocks,
                           int block_size, int window, float scale, void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16, "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(q && ring_k && ring_v && pool_k && pool_v && topology && out, "null pointer");
  BFLY_CHECK_ARG((k_new == nullptr) == (v_new == nullptr), "k_new/v_new must both be given or both NULL");
  BFLY_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(ring_k) && aligned16(ring_v) && aligned16(pool_k) &&
                     aligned16(pool_v) && aligned16(k_new) && aligned16(v_new),
                 "tensor pointers must be 16-byte aligned");
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(batch * hkv <= INT32_MAX, "batch*hkv too large");
  BFLY_CHECK_ARG(head_dim == 64 || head_dim == 128 || (head_dim == 256 && dtype == BFLY_DTYPE_BF16),
                 "bfly_decode: head_dim=%d unsupported (64, 128; 256 for bf16)", head_dim);
  BFLY_CHECK_ARG(window > 0 && window <= kDecMaxWin, "bfly_decode: window=%d must be in [1, %d]", window, kDecMaxWin);
  BFLY_CHECK_ARG(1 + topology->local_window_blocks + topology->partner_count + topology->sink_count <= kDecMaxSum &&
                     topology->partner_count >= 0 && topology->partner_count <= BFLY_MAX_PARTNERS,
                 "bfly_decode: the routed row must fit %d slots", kDecMaxSum);
  BFLY_CHECK_ARG(block_size > 0 && num_blocks > 0, "bad block_size/num_blocks");
  BFLY_CHECK_ARG(kv_len > 0 && tail_start >= 0 && tail_start < kv_len, "tail [%lld, %lld) must hold the query",
                 (long long)tail_start, (long long)kv_len);
  BFLY_CHECK_ARG(num_blocks * (int64_t)block_size >= kv_len, "num_blocks does not cover kv_len");
  BFLY_CHECK_ARG(ring_capacity >= 0 && (ring_capacity == 0 || kv_len - tail_start <= ring_capacity),
                 "tail [%lld, %lld) does not fit ring capacity %lld", (long long)tail_start, (long long)kv_len,
                 (long long)ring_capacity);
  BFLY_CHECK_ARG(summary_count >= 0 && summary_count <= pool_capacity && pool_capacity > 0,
                 "summary_count must be in [0, pool_capacity]");
  DecodeArgs a{};
  a.q = q; a.out = out; a.k_new = k_new; a.v_new = v_new;
  a.ring_k = ring_k; a.ring_v = ring_v; a.pool_k = pool_k; a.pool_v = pool_v; a.topo = *topology;
  a.ring = ring_capacity;
  a.kv_rows = ring_capacity ? ring_capacity : kv_len - tail_start;
  a.tail_start = tail_start; a.kv_len = kv_len;
  a.pool_rows = pool_capacity; a.nsum = summary_count; a.nblocks = num_blocks;
  a.hq = hq; a.hkv = hkv; a.bs = block_size; a.W = window; a.CW = window; a.scale = scale;
  const StepArgs none{};
  if (dtype == BFLY_DTYPE_F32)
    launch_decode<float, false>(a, none, head_dim, batch * hkv, stream);
  else
    launch_decode<__bf16, false>(a, none, head_dim, batch * hkv, stream);
  BFLY_CHECK_LAUNCH("bfly_decode");
  return BFLY_OK;
}

extern "C" int64_t bfly_decode_state_words(int64_t batch, int hkv) {
  if (batch <= 0 || hkv <= 0) return 0;
  const int64_t nseq = batch * hkv;
  return kStHeader + kStSlot * (nseq * dec_copies(nseq) + kRouteGroups);
}

static int decode_step(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim, const void* k_new,
                       const void* v_new, void* ring_k, void* ring_v, int64_t ring_capacity, void* pool_k,
                       void* pool_v, int64_t pool_capacity, int64_t* state, int64_t layer_idx, int partner_rule,
                       int local_window_blocks, int sink_count, int partner_count, int block_size, int window,
                       int cache_window, float scale, void* out, const DecodeArgs* qkn, hipStream_t stream,
                       const DecodeArgs* oproj = nullptr) {
  BFLY_CHECK_ARG(dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16, "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(q && k_new && v_new && ring_k && ring_v && pool_k && pool_v && state && out, "null pointer");
  BFLY_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(ring_k) && aligned16(ring_v) && aligned16(pool_k) &&
                     aligned16(pool_v) && aligned16(k_new) && aligned16(v_new) &&
                     (reinterpret_cast<uintptr_t>(state) & 7) == 0,
                 "tensor pointers must be 16-byte aligned (state 8-byte)");
  BFLY_CHECK_ARG(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts hq=%d hkv=%d", hq, hkv);
  BFLY_CHECK_ARG(batch * hkv <= INT32_MAX - kRouteGroups, "batch*hkv too large");
  BFLY_CHECK_ARG(head_dim == 64 || head_dim == 128 || (head_dim == 256 && dtype == BFLY_DTYPE_BF16),
                 "bfly_decode_step: head_dim=%d unsupported (64, 128; 256 for bf16)", head_dim);
  BFLY_CHECK_ARG(window > 0 && window <= kDecMaxWin, "bfly_decode_step: window=%d must be in [1, %d]", window,
                 kDecMaxWin);
  BFLY_CHECK_ARG(partner_rule >= BFLY_RULE_XOR && partner_rule <= BFLY_RULE_RANDOM, "unsupported partner rule %d",
                 partner_rule);
  BFLY_CHECK_ARG(local_window_blocks >= 0 && sink_count >= 0 && partner_count >= 0 &&
                     partner_count <= BFLY_MAX_PARTNERS &&
                     1 + local_window_blocks + partner_count + sink_count <= kDecMaxSum,
                 "bfly_decode_step: the routed row must fit %d slots", kDecMaxSum);
  BFLY_CHECK_ARG(cache_window > 0 && cache_window < (1 << 20),
                 "bfly_decode_step: cache_window=%d must be in [1, 2^20)", cache_window);
  BFLY_CHECK_ARG(block_size > 0 && ring_capacity >= cache_window + block_size && pool_capacity > 0,
                 "bfly_decode_step: ring must hold cache_window + BS rows and the pool at least one");
  DecodeArgs a{};
  a.q = q; a.out = out; a.k_new = k_new; a.v_new = v_new;
  a.ring_k = ring_k; a.ring_v = ring_v; a.pool_k = pool_k; a.pool_v = pool_v;
  a.ring = ring_capacity; a.kv_rows = ring_capacity; a.pool_rows = pool_capacity;
  a.hq = hq; a.hkv = hkv; a.bs = block_size; a.W = window; a.CW = cache_window; a.scale = scale;
  a.cps = dec_copies(batch * hkv);
  if (qkn != nullptr) {
    BFLY_CHECK_ARG(dtype == BFLY_DTYPE_BF16 && head_dim == 128 && decode_on_mfma(a, head_dim, true),
                   "bfly_decode_step_qk_norm: bf16, head_dim 128 and a positive scale only");
    a.qn_w = qkn->qn_w; a.kn_w = qkn->kn_w; a.rope_cos = qkn->rope_cos; a.rope_sin = qkn->rope_sin;
    a.rope_rows = qkn->rope_rows; a.qk_eps = qkn->qk_eps;
  }
  if (oproj != nullptr) {
    a.ow = oproj->ow; a.osb = oproj->osb; a.opart = oproj->opart;
    a.o_rows = oproj->o_rows; a.o_groups = oproj->o_groups; a.o_ppg_log2 = oproj->o_ppg_log2;
    a.o_subs = oproj->o_subs;
  }
  StepArgs sa{state, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count};
  if (dtype == BFLY_DTYPE_F32)
    launch_decode<float, true>(a, sa, head_dim, batch * hkv, stream);
  else
    launch_decode<__bf16, true>(a, sa, head_dim, batch * hkv, stream);
  BFLY_CHECK_LAUNCH(qkn ? "bfly_decode_step_qk_norm" : "bfly_decode_step");
  return BFLY_OK;
}

extern "C" int bfly_decode_step(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                                const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                                int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                                int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks,
                                int sink_count, int partner_count, int block_size, int window, int cache_window,
                                float scale, void* out, hipStream_t stream) {
  return decode_step(q, dtype, batch, hq, hkv, head_dim, k_new, v_new, ring_k, ring_v, ring_capacity, pool_k, pool_v,
                     pool_capacity, state, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count,
                     block_size, window, cache_window, scale, out, nullptr, stream);
}

extern "C" int bfly_decode_step_qk_norm(const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim,
                                        const void* k_new, const void* v_new, void* ring_k, void* ring_v,
                                        int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
                                        int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks,
                                        int sink_count, int partner_count, int block_size, int window,
                                        int cache_window, float scale, const void* q_norm_weight, const void* k_norm_weight, const float* rope_cos,
                                        const float* rope_sin, int64_t rope_rows, float eps, void* out,
                                        hipStream_t stream) {
  BFLY_CHECK_ARG(q_norm_weight && k_norm_weight && rope_cos && rope_sin, "null pointer");
  BFLY_CHECK_ARG(aligned16(q_norm_weight) && aligned16(k_norm_weight) && aligned16(rope_cos) && aligned16(rope_sin),
                 "norm weights and RoPE tables must be 16-byte aligned");
  BFLY_CHECK_ARG(rope_rows > 0 && eps >= 0.f, "bad rope_rows / eps");
  DecodeArgs n{};
  n.qn_w = static_cast<const __bf16*>(q_norm_weight);
  n.kn_w = static_cast<const __bf16*>(k_norm_weight);
  n.rope_cos = rope_cos;
  n.rope_sin = rope_sin;
  n.rope_rows = rope_rows;
  n.qk_eps = eps;
  return decode_step(q, dtype, batch, hq, hkv, head_dim, k_new, v_new, ring_k, ring_v, ring_capacity, pool_k, pool_v,
                     pool_capacity, state, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count,
                     block_size, window, cache_window, scale, out, &n, stream);
}

extern "C" int bfly_decode_step_qk_norm_oproj(
    const void* q, int dtype, int64_t batch, int hq, int hkv, int head_dim, const void* k_new, const void* v_new,
    void* ring_k, void* ring_v, int64_t ring_capacity, void* pool_k, void* pool_v, int64_t pool_capacity,
    int64_t* state, int64_t layer_idx, int partner_rule, int local_window_blocks, int sink_count, int partner_count,
    int block_size, int window, int cache_window, float scale, const void* q_norm_weight, const void* k_norm_weight,
    const float* rope_cos, const float* rope_sin, int64_t rope_rows, float eps, const void* o_packed,
    const void* o_scale_bias, int64_t o_out_features, int o_group, float* o_parts, void* out, hipStream_t stream) {
  BFLY_CHECK_ARG(q_norm_weight && k_norm_weight && rope_cos && rope_sin && o_packed && o_scale_bias && o_parts,
                 "null pointer");
  BFLY_CHECK_ARG(aligned16(q_norm_weight) && aligned16(k_norm_weight) && aligned16(rope_cos) && aligned16(rope_sin) &&
                     aligned16(o_packed) && aligned16(o_parts) && (reinterpret_cast<uintptr_t>(o_scale_bias) & 3) == 0,
                 "norm weights, RoPE tables, W_o codes and o_parts must be 16-byte aligned (scales 4-byte)");
  BFLY_CHECK_ARG(rope_rows > 0 && eps >= 0.f, "bad rope_rows / eps");
  BFLY_CHECK_ARG(head_dim == 128 && hkv == 4 && hq == 16,
                 "bfly_decode_step_qk_norm_oproj: 16 query heads over 4 kv heads of 128 (got hq=%d hkv=%d d=%d)", hq,
                 hkv, head_dim);
  BFLY_CHECK_ARG(batch > 0 && batch * hkv <= kOprojMaxSeq, "bfly_decode_step_qk_norm_oproj: batch * hkv <= %d",
                 kOprojMaxSeq);
  BFLY_CHECK_ARG(o_group >= 32 && o_group <= 2048 && (o_group & (o_group - 1)) == 0,
                 "o_group=%d must be a power of two in [32, 2048]", o_group);
  // 32 rows per attending workgroup (two sets of four per wave) while that needs at most
  // kOprojSubs workgroups per sequence, else 64
  const bool rows32 = o_out_features % 32 == 0 && o_out_features <= 32 * kOprojSubs;
  BFLY_CHECK_ARG(o_out_features > 0 && (rows32 || (o_out_features % 64 == 0 && o_out_features <= 64 * kOprojSubs)),
                 "o_out_features=%lld must be a multiple of 32 up to %d or of 64 up to %d", (long long)o_out_features,
                 32 * kOprojSubs, 64 * kOprojSubs);
  DecodeArgs n{};
  n.qn_w = static_cast<const __bf16*>(q_norm_weight);
  n.kn_w = static_cast<const __bf16*>(k_norm_weight);
  n.rope_cos = rope_cos;
  n.rope_sin = rope_sin;
  n.rope_rows = rope_rows;
  n.qk_eps = eps;
  DecodeArgs o{};
  o.ow = static_cast<const u32x4*>(o_packed);
  o.osb = static_cast<const uint32_t*>(o_scale_bias);
  o.opart = o_parts;
  o.o_rows = (int)o_out_features;
  o.o_groups = 2048 / o_group;
  o.o_ppg_log2 = __builtin_ctz((unsigned)(o_group / kQ4PieceCodes));
  o.o_subs = (int)(o_out_features / (rows32 ? 32 : 64));
  return decode_step(q, dtype, batch, hq, hkv, head_dim, k_new, v_new, ring_k, ring_v, ring_capacity, pool_k, pool_v,
                     pool_capacity, state, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count,
                     block_size, window, cache_window, scale, out, &n, stream, &o);
}
