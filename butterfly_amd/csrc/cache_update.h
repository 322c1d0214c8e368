// Block mean pooling and the one-launch cache update (append + pooling of the
// due blocks), as device functions shared by the compressor kernels and the
// streaming prefill's fused launch.
//
// Reference semantics: _block_mean_summaries_torch
// (bna/torch/attention_wayfinder_permute.py:1022-1043) and the summarise and
// append steps of CompressedKVCache.update_and_fetch
// (bna/mlx/compressed_cache.py:104-149).
//
// Fixed summation order (documented so results are reproducible): thread slot
// s (of RS slots) sums tokens s, s+RS, s+2RS, ... sequentially; the RS partial
// sums are then added in slot order 0..RS-1; the total is divided by the
// valid-token count and rounded (RNE) to the storage type.
#pragma once

#include "bfly_common.h"

namespace bfly {

// Mean of `cnt` token rows into dst (256 threads: t = 0..255 of the group that runs it; the
// workgroup barrier is taken once); tok_ptr(tok) is the row of token tok; `part` is 256 * 8
// floats of LDS scratch.  INFLIGHT
// 16-byte loads per thread are requested before their adds (8 keeps the
// compressor's registers low; the update job's pooling takes 16, a whole block
// at d = 256 in one round trip).
template <typename T, int VEC, int INFLIGHT = 8, class TokPtr>
__device__ __forceinline__ void pool_rows(TokPtr tok_ptr, int64_t cnt, T* dst, int d, float* part, int t) {
  const int lpr = d / VEC;               // lanes per token row
  const int rs = 256 / lpr;              // token slots
  const int c = t % lpr, s = t / lpr;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  if (s < rs) {
    if constexpr (VEC * sizeof(T) == 16) {
      // INFLIGHT loads per thread, then the adds in token order
      for (int64_t base = s; base < cnt; base += INFLIGHT * (int64_t)rs) {
        uint4 raw[INFLIGHT];
#pragma unroll
        for (int u = 0; u < INFLIGHT; ++u) {
          // unconditional (past the block's end: its last token again, not added): a
          // conditional load would be a branch that waits for each load in turn
          const int64_t tok = base + (int64_t)u * rs;
          raw[u] = *reinterpret_cast<const uint4*>(tok_ptr(tok < cnt ? tok : cnt - 1) + c * VEC);
        }
        // every load is issued before the first add (the scheduler hoisted adds between them,
        // each add's wait then also waiting for the loads before it); a row past the end adds +0
        // (acc is never -0, so acc + 0 is acc): no branch, into which the compiler would sink
        // that row's load and wait for it alone
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < INFLIGHT; ++u) {
          const bool in = base + (int64_t)u * rs < cnt;
          const T* v = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] += in ? to_f32(v[e]) : 0.f;
        }
      }
    } else {
      for (int64_t tok = s; tok < cnt; tok += rs) {
        const T* ptr = tok_ptr(tok) + c * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += to_f32(ptr[e]);
      }
    }
  }
  if (s < rs) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) part[s * d + c * VEC + e] = acc[e];
  }
  __syncthreads();
  const float denom = cnt > 0 ? (float)cnt : 1.f;
  for (int col = t; col < d; col += 256) {
    float tot = 0.f;
    for (int k = 0; k < rs; ++k) tot += part[k * d + col];
    dst[col] = from_f32<T>(tot / denom);
  }
}

// One chunk's cache update (compressed_cache.py:104-149): the append of
// k_new/v_new to ring slots (offset + t) mod C, and the mean of every block
// that became due, whose tokens are read where they are before the update (the
// ring for positions < offset, k_new/v_new for the rest), so the two parts are
// independent: the pooled blocks and the new tokens all lie in the post-append
// tail, which holds at most C positions, so their ring slots are distinct.
// Work: x in [0, n_blocks + append workgroups), rows, K|V.
// Chunks whose appends one update job may carry (the streaming loop's batches).
constexpr int kMaxUpdateParts = 10;
// Rounds of 16-byte pieces per thread in an update's append workgroups.
constexpr int kAppendRounds = 8;

struct UpdateJob {
  const void* k_new;
  const void* v_new;     // [rows, step, d]
  void* ring_k;
  void* ring_v;          // [rows, ring, d]
  void* pool_k;
  void* pool_v;          // [rows, pool_rows, d]
  int64_t step, ring, pool_rows, offset, first_pos, first_slot;
  int n_blocks, bs, d;
  // nparts > 0: the step's new tokens come from nparts consecutive chunks instead of
  // k_new / v_new: tokens [part_end[j-1], part_end[j]) are chunk j's, laid out
  // [rows, chunk length, d] at k_part[j] / v_part[j] (part_end[nparts-1] == step)
  int nparts;
  const void* k_part[kMaxUpdateParts];
  const void* v_part[kMaxUpdateParts];
  int64_t part_end[kMaxUpdateParts];
  // new tokens t < append_from are not copied to the ring (the streaming loop: tokens below the
  // tail that the update leaves, which no later step reads; its attention reads the batch's own
  // tokens from the chunk inputs)
  int64_t append_from;
};

// The part of an update's input that holds new token t (< step): its buffer (K or V), first
// token and length, found by selects over every part slot (constant indices).  With a
// workgroup-uniform t this is scalar work; with a lane-dependent t the compiler makes the
// pointer selection a vector load from a selected address, whose wait also waits for every
// row load issued before it (loads complete in order), so the rows' lookups go first.
struct FreshPart {
  const void* base;
  int64_t t0, len;
};
__device__ __forceinline__ FreshPart update_part_of(const UpdateJob& u, int kv, int64_t t) {
  const bool single = u.nparts == 0;
  FreshPart f{single ? (kv ? u.v_new : u.k_new) : (kv ? u.v_part[0] : u.k_part[0]), 0,
              single ? u.step : u.part_end[0]};
#pragma unroll
  for (int j = 1; j < kMaxUpdateParts; ++j) {
    const void* pj = kv ? u.v_part[j] : u.k_part[j];
    const bool in = j < u.nparts && t >= u.part_end[j - 1];   // part_end increases: the last such j
    f.base = in ? pj : f.base;
    f.len = in ? u.part_end[j] - u.part_end[j - 1] : f.len;
    f.t0 = in ? u.part_end[j - 1] : f.t0;
  }
  return f;
}

// Row of new token t of batch row `row` in part f (t0 <= t < t0 + len).
template <typename T>
__device__ __forceinline__ const T* update_part_row(const FreshPart& f, int64_t row, int64_t t, int d) {
  return reinterpret_cast<const T*>(f.base) + (row * f.len + (t - f.t0)) * d;
}

// Row of new token t (< step) of batch row `row` in an update's input, any t.
template <typename T>
__device__ __forceinline__ const T* update_fresh_row(const UpdateJob& u, int kv, int64_t row, int64_t t) {
  return update_part_row<T>(update_part_of(u, kv, t), row, t, u.d);
}

// Work item (bx, row, kv) of an update, run by 256 threads (t = 0..255; the pooling items take the
// workgroup barrier once, the append items none).  A workgroup's new
// tokens normally lie in one part (the parts are whole chunks): its part is then looked up once,
// from workgroup-uniform values (scalar work), and every row follows by adding; a workgroup
// whose tokens straddle parts looks each row up.
template <typename T, int VEC>
__device__ __forceinline__ void cache_update_body(const UpdateJob& u, int64_t bx, int64_t row, int kv, float* part,
                                                  int t) {
  const int d = u.d;
  T* ring = reinterpret_cast<T*>(kv ? u.ring_v : u.ring_k) + row * u.ring * d;
  if (bx >= u.n_blocks) {
    // append: kAppendRounds x 256 / (d / VEC) tokens per workgroup, one 16-byte piece per
    // thread and round; every round's load is issued before the first store
    const int lpr = d / VEC, tpw = 256 / lpr;
    const int c = t % lpr;
    if (t / lpr >= tpw) return;
    const int64_t wg_tok0 = u.append_from + (bx - u.n_blocks) * tpw * kAppendRounds;
    const int64_t tok0 = wg_tok0 + t / lpr;
    if (tok0 >= u.step) return;
    const int64_t wg_last = min(wg_tok0 + (int64_t)tpw * kAppendRounds, u.step) - 1;
    const FreshPart f = update_part_of(u, kv, wg_tok0);
    const bool one_part = wg_last < f.t0 + f.len;
    // loads unconditional (past the last token: the last token again), stores kept in range
    // (a native vector type: arrays of HIP's uint4 struct are copied by memcpy and stay in
    // scratch memory)
    // (each branch issues its own loads: pointers merged from the two would be flat pointers,
    // whose loads the scalar-load waits also count)
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 x[kAppendRounds];
    if (one_part) {
#pragma unroll
      for (int i = 0; i < kAppendRounds; ++i)
        x[i] = *reinterpret_cast<const u32x4*>(
            update_part_row<T>(f, row, min(tok0 + (int64_t)i * tpw, u.step - 1), d) + c * VEC);
    } else {
#pragma unroll
      for (int i = 0; i < kAppendRounds; ++i)
        x[i] = *reinterpret_cast<const u32x4*>(
            update_fresh_row<T>(u, kv, row, min(tok0 + (int64_t)i * tpw, u.step - 1)) + c * VEC);
    }
    int64_t slot = posmod(u.offset + tok0, u.ring);   // then + tpw per round (tpw < ring: one wrap)
#pragma unroll
    for (int i = 0; i < kAppendRounds; ++i) {
      if (tok0 + (int64_t)i * tpw < u.step) *reinterpret_cast<u32x4*>(ring + slot * d + c * VEC) = x[i];
      slot += tpw;
      if (slot >= u.ring) slot -= u.ring;
    }
    return;
  }
  const int64_t n = bx;
  const int64_t p0 = u.first_pos + n * u.bs;
  const int64_t r0 = posmod(p0, u.ring);   // tokens < bs <= ring: one wrap at most
  T* dst = reinterpret_cast<T*>(kv ? u.pool_v : u.pool_k) + (row * u.pool_rows + u.first_slot + n) * d;
  auto ring_row = [&](int64_t tok) -> const T* {
    int64_t r = r0 + tok;
    if (r >= u.ring) r -= u.ring;
    return ring + r * d;
  };
  if (p0 + u.bs <= u.offset) {   // the whole block was appended before: ring rows
    pool_rows<T, VEC, 16>(ring_row, (int64_t)u.bs, dst, d, part, t);
    return;
  }
  if (p0 >= u.offset) {          // the whole block is new
    const FreshPart f = update_part_of(u, kv, p0 - u.offset);
    if (p0 + u.bs - 1 - u.offset < f.t0 + f.len) {
      const int64_t f0 = p0 - u.offset;
      pool_rows<T, VEC, 16>([&](int64_t tok) { return update_part_row<T>(f, row, f0 + tok, d); }, (int64_t)u.bs, dst,
                            d, part, t);
      return;
    }
  }
  auto tok_ptr = [&](int64_t tok) -> const T* {
    const int64_t p = p0 + tok;
    if (p >= u.offset) return update_fresh_row<T>(u, kv, row, p - u.offset);
    return ring_row(tok);
  };
  pool_rows<T, VEC, 16>(tok_ptr, (int64_t)u.bs, dst, d, part, t);
}

// One bf16 update job in one launch (compress.hip); rows = batch x kv heads.
int launch_update_job(const UpdateJob& u, int64_t rows, hipStream_t stream);

// Workgroups along x of an update with a 16-byte row split (VEC elements per
// 16 bytes): the due blocks, then the append workgroups (step: the tokens copied).
inline int64_t update_x(int64_t n_blocks, int64_t step, int head_dim, int vec) {
  const int tpw = 256 / (head_dim / vec) * kAppendRounds;
  return n_blocks + (step + tpw - 1) / tpw;
}

}  // namespace bfly
