// Mean-pool block compressor and two-pool cache maintenance on gfx950.
//
// Reference semantics: _block_mean_summaries_torch
// (bna/torch/attention_wayfinder_permute.py:1022-1043), the summarise and
// append steps of CompressedKVCache.update_and_fetch
// (bna/mlx/compressed_cache.py:104-149).
//
// These kernels are HBM-bound: every input byte is read once with 16-byte
// vector loads, accumulated in fp32 registers and reduced through LDS.
// Fixed summation order (documented so results are reproducible): thread slot
// s (of RS slots) sums tokens s, s+RS, s+2RS, ... sequentially; the RS partial
// sums are then added in slot order 0..RS-1; the total is divided by the
// valid-token count and rounded (RNE) to the storage type.
#include "cache_update.h"

namespace bfly {

struct PoolJob {
  const void* src;      // [rows, src_rows_per_seq, d]
  void* dst;            // [rows, dst_rows_per_seq, d]
  int64_t src_rows;     // rows per sequence in src (T, or ring capacity)
  int64_t dst_rows;     // rows per sequence in dst
  int64_t ring;         // 0: linear source; else position p lives at p mod ring
  int64_t base_pos;     // position of token 0 of block 0
  int64_t dst_slot0;    // dst row of block 0
  int64_t seq_len;      // valid tokens are positions < base_pos + seq_len
};

template <typename T, int VEC>
__global__ void __launch_bounds__(256) block_mean_kernel(PoolJob j0, PoolJob j1, int d, int bs) {
  const PoolJob& job = blockIdx.z == 0 ? j0 : j1;
  const int64_t n = blockIdx.x;          // block index
  const int64_t row = blockIdx.y;        // sequence (b*h)
  const int64_t first = n * bs;
  int64_t cnt = job.seq_len - first;
  cnt = cnt < bs ? cnt : bs;
  if (cnt < 0) cnt = 0;
  const T* src = reinterpret_cast<const T*>(job.src) + row * job.src_rows * d;
  // row of token 0 of the block; tokens are < bs <= ring, so one wrap at most
  const int64_t r0 = job.ring ? posmod(job.base_pos + first, job.ring) : job.base_pos + first;
  auto tok_ptr = [&](int64_t tok) {
    int64_t r = r0 + tok;
    if (job.ring && r >= job.ring) r -= job.ring;
    return src + r * d;
  };
  T* dst = reinterpret_cast<T*>(job.dst) + (row * job.dst_rows + job.dst_slot0 + n) * d;
  __shared__ float part[256 * 8];
  pool_rows<T, VEC>(tok_ptr, cnt, dst, d, part, (int)threadIdx.x);
}

// One chunk's cache update in one launch: cache_update_body over the grid
// (n_blocks + append workgroups, rows, K|V).
template <typename T, int VEC>
__global__ void __launch_bounds__(256) cache_update_kernel(UpdateJob u) {
  __shared__ float part[256 * 8];
  cache_update_body<T, VEC>(u, blockIdx.x, blockIdx.y, blockIdx.z, part, (int)threadIdx.x);
}

// One update job (bf16, 16-byte row split: d in {64, 128, 256}) in one launch; the streaming
// loop's batches, whose new tokens may come from several chunk buffers.
int launch_update_job(const UpdateJob& u, int64_t rows, hipStream_t stream) {
  BFLY_CHECK_ARG((u.d == 64 || u.d == 128 || u.d == 256) && rows > 0 && rows <= 65535, "update job shape");
  // the due blocks lie inside the post-append tail: [offset + step - ring, offset + step)
  BFLY_CHECK_ARG(u.n_blocks == 0 || (u.first_pos >= u.offset + u.step - u.ring &&
                                     u.first_pos + (int64_t)u.n_blocks * u.bs <= u.offset + u.step),
                 "update job: due blocks outside the tail after the append");
  BFLY_CHECK_ARG(u.append_from >= 0 && u.append_from <= u.step, "update job: append_from outside the step");
  if (u.step == u.append_from && u.n_blocks == 0) return BFLY_OK;
  const int64_t ux = update_x(u.n_blocks, u.step - u.append_from, u.d, 8);
  BFLY_CHECK_ARG(ux <= INT32_MAX, "update job: grid too large");
  hipLaunchKernelGGL((cache_update_kernel<__bf16, 8>), dim3((unsigned)ux, (unsigned)rows, 2), dim3(256), 0, stream, u);
  BFLY_CHECK_LAUNCH("cache update job");
  return BFLY_OK;
}

template <typename T>
static int launch_pool(const PoolJob& a, const PoolJob* b, int64_t rows, int d, int bs,
                       int64_t nblocks, hipStream_t stream) {
  dim3 grid((unsigned)nblocks, (unsigned)rows, b ? 2 : 1);
  const PoolJob& bj = b ? *b : a;
  constexpr int V16 = 16 / sizeof(T);
  if (d % V16 == 0 && d / V16 <= 256 && 256 * V16 <= 256 * 8) {
    hipLaunchKernelGGL((block_mean_kernel<T, V16>), grid, dim3(256), 0, stream, a, bj, d, bs);
  } else if (d <= 256) {
    hipLaunchKernelGGL((block_mean_kernel<T, 1>), grid, dim3(256), 0, stream, a, bj, d, bs);
  } else {
    set_error("head_dim=%d unsupported by the compressor", d);
    return BFLY_ERR_UNSUPPORTED;
  }
  return BFLY_OK;
}

template <typename T>
__global__ void append_kernel(const T* __restrict__ kn, const T* __restrict__ vn, T* __restrict__ rk,
                              T* __restrict__ rv, int64_t step, int d, int64_t ring,
                              int64_t offset, int64_t total_vec, int vec) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool isv = blockIdx.y == 1;
  if (i >= total_vec) return;
  const int64_t per_row = d / vec;
  const int64_t e = (i % per_row) * vec;
  const int64_t rowi = i / per_row;          // (bh, t) flattened
  const int64_t t = rowi % step, bh = rowi / step;
  const int64_t slot = posmod(offset + t, ring);
  const T* src = (isv ? vn : kn) + rowi * d + e;
  T* dst = (isv ? rv : rk) + (bh * ring + slot) * d + e;
  if (vec * sizeof(T) == 16) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else {
    for (int k = 0; k < vec; ++k) dst[k] = src[k];
  }
}

}  // namespace bfly

using namespace bfly;

static bool dtype_ok(int dtype) { return dtype == BFLY_DTYPE_F32 || dtype == BFLY_DTYPE_BF16; }

extern "C" int bfly_block_mean(const void* x, void* out, const void* x2, void* out2, int dtype,
                               int64_t rows, int64_t seq_len, int head_dim, int block_size,
                               int64_t num_blocks, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(x && out, "null pointer");
  BFLY_CHECK_ARG((x2 == nullptr) == (out2 == nullptr), "x2/out2 must both be given or both NULL");
  BFLY_CHECK_ARG(aligned16(x) && aligned16(out) && aligned16(x2) && aligned16(out2),
                 "tensor pointers must be 16-byte aligned");
  BFLY_CHECK_ARG(rows > 0 && rows <= 65535, "rows=%lld out of range", (long long)rows);
  BFLY_CHECK_ARG(seq_len > 0 && head_dim > 0 && block_size > 0, "non-positive shape");
  BFLY_CHECK_ARG(num_blocks * block_size >= seq_len && num_blocks <= INT32_MAX,
                 "num_blocks*block_size must cover seq_len");
  PoolJob a{x, out, seq_len, num_blocks, 0, 0, 0, seq_len};
  PoolJob b{x2, out2, seq_len, num_blocks, 0, 0, 0, seq_len};
  int rc = dtype == BFLY_DTYPE_F32
               ? launch_pool<float>(a, x2 ? &b : nullptr, rows, head_dim, block_size, num_blocks, stream)
               : launch_pool<__bf16>(a, x2 ? &b : nullptr, rows, head_dim, block_size, num_blocks, stream);
  if (rc) return rc;
  BFLY_CHECK_LAUNCH("bfly_block_mean");
  return BFLY_OK;
}

extern "C" int bfly_cache_append(const void* k_new, const void* v_new, int dtype, int64_t batch,
                                 int hkv, int64_t step, int head_dim, void* ring_k, void* ring_v,
                                 int64_t ring_capacity, int64_t offset, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(k_new && v_new && ring_k && ring_v, "null pointer");
  BFLY_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(ring_k) && aligned16(ring_v),
                 "tensor pointers must be 16-byte aligned");
  BFLY_CHECK_ARG(batch > 0 && hkv > 0 && head_dim > 0 && step >= 0, "bad shape");
  BFLY_CHECK_ARG(ring_capacity > 0 && step <= ring_capacity, "step=%lld exceeds ring capacity %lld",
                 (long long)step, (long long)ring_capacity);
  BFLY_CHECK_ARG(offset >= 0, "negative offset");
  if (step == 0) return BFLY_OK;
  const int esz = dtype == BFLY_DTYPE_F32 ? 4 : 2;
  const int vec = (head_dim * esz) % 16 == 0 ? 16 / esz : 1;
  const int64_t total = batch * hkv * step * (head_dim / vec);
  const int threads = 256;
  dim3 grid((unsigned)((total + threads - 1) / threads), 2);
  if (dtype == BFLY_DTYPE_F32)
    hipLaunchKernelGGL(append_kernel<float>, grid, dim3(threads), 0, stream, (const float*)k_new,
                       (const float*)v_new, (float*)ring_k, (float*)ring_v, step, head_dim,
                       ring_capacity, offset, total, vec);
  else
    hipLaunchKernelGGL(append_kernel<__bf16>, grid, dim3(threads), 0, stream, (const __bf16*)k_new,
                       (const __bf16*)v_new, (__bf16*)ring_k, (__bf16*)ring_v, step, head_dim,
                       ring_capacity, offset, total, vec);
  BFLY_CHECK_LAUNCH("bfly_cache_append");
  return BFLY_OK;
}

extern "C" int bfly_cache_compress(const void* ring_k, const void* ring_v, int dtype,
                                   int64_t batch, int hkv, int head_dim, int64_t ring_capacity,
                                   int64_t first_block_pos, int64_t n_blocks, int block_size,
                                   void* pool_k, void* pool_v, int64_t pool_capacity,
                                   int64_t first_slot, hipStream_t stream) {
  BFLY_CHECK_ARG(dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(ring_k && ring_v && pool_k && pool_v, "null pointer");
  BFLY_CHECK_ARG(aligned16(ring_k) && aligned16(ring_v) && aligned16(pool_k) && aligned16(pool_v),
                 "tensor pointers must be 16-byte aligned");
  BFLY_CHECK_ARG(batch > 0 && hkv > 0 && head_dim > 0 && block_size > 0, "bad shape");
  BFLY_CHECK_ARG(batch * hkv <= 65535, "batch*hkv too large");
  BFLY_CHECK_ARG(ring_capacity >= block_size, "ring smaller than a block");
  BFLY_CHECK_ARG(n_blocks >= 0 && first_slot >= 0 && first_slot + n_blocks <= pool_capacity,
                 "summary pool overflow: slots [%lld, %lld) of %lld", (long long)first_slot,
                 (long long)(first_slot + n_blocks), (long long)pool_capacity);
  if (n_blocks == 0) return BFLY_OK;
  const int64_t seq = n_blocks * (int64_t)block_size;
  PoolJob a{ring_k, pool_k, ring_capacity, pool_capacity, ring_capacity, first_block_pos, first_slot, seq};
  PoolJob b{ring_v, pool_v, ring_capacity, pool_capacity, ring_capacity, first_block_pos, first_slot, seq};
  int rc = dtype == BFLY_DTYPE_F32
               ? launch_pool<float>(a, &b, batch * hkv, head_dim, block_size, n_blocks, stream)
               : launch_pool<__bf16>(a, &b, batch * hkv, head_dim, block_size, n_blocks, stream);
  if (rc) return rc;
  BFLY_CHECK_LAUNCH("bfly_cache_compress");
  return BFLY_OK;
}

extern "C" int bfly_cache_update(const void* k_new, const void* v_new, int dtype, int64_t batch, int hkv,
                                 int64_t step, int head_dim, void* ring_k, void* ring_v, int64_t ring_capacity,
                                 int64_t offset, int64_t first_block_pos, int64_t n_blocks, int block_size,
                                 void* pool_k, void* pool_v, int64_t pool_capacity, int64_t first_slot,
                                 hipStream_t stream) {
  BFLY_CHECK_ARG(dtype_ok(dtype), "unsupported dtype %d", dtype);
  BFLY_CHECK_ARG(k_new && v_new && ring_k && ring_v && pool_k && pool_v, "null pointer");
  BFLY_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(ring_k) && aligned16(ring_v) &&
                     aligned16(pool_k) && aligned16(pool_v),
                 "tensor pointers must be 16-byte aligned");
  BFLY_CHECK_ARG(batch > 0 && hkv > 0 && head_dim > 0 && step >= 0 && block_size > 0, "bad shape");
  BFLY_CHECK_ARG(batch * hkv <= 65535, "batch*hkv too large");
  BFLY_CHECK_ARG(ring_capacity >= block_size && step <= ring_capacity, "step=%lld exceeds ring capacity %lld",
                 (long long)step, (long long)ring_capacity);
  BFLY_CHECK_ARG(offset >= 0, "negative offset");
  BFLY_CHECK_ARG(n_blocks >= 0 && n_blocks <= INT32_MAX && first_slot >= 0 && first_slot + n_blocks <= pool_capacity,
                 "summary pool overflow: slots [%lld, %lld) of %lld", (long long)first_slot,
                 (long long)(first_slot + n_blocks), (long long)pool_capacity);
  // the due blocks lie inside the post-append tail: [offset + step - ring, offset + step)
  BFLY_CHECK_ARG(n_blocks == 0 || (first_block_pos >= 0 && first_block_pos >= offset + step - ring_capacity &&
                                   first_block_pos + n_blocks * (int64_t)block_size <= offset + step),
                 "due blocks [%lld, %lld) outside the tail after the append", (long long)first_block_pos,
                 (long long)(first_block_pos + n_blocks * (int64_t)block_size));
  if (step == 0 && n_blocks == 0) return BFLY_OK;
  const int esz = dtype == BFLY_DTYPE_F32 ? 4 : 2;
  const int vec = 16 / esz;
  if ((head_dim * esz) % 16 != 0 || head_dim / vec > 256) {
    // shapes without a 16-byte row split: the two separate launches
    int rc = bfly_cache_append(k_new, v_new, dtype, batch, hkv, step, head_dim, ring_k, ring_v, ring_capacity,
                               offset, stream);
    if (rc) return rc;
    return bfly_cache_compress(ring_k, ring_v, dtype, batch, hkv, head_dim, ring_capacity, first_block_pos,
                               n_blocks, block_size, pool_k, pool_v, pool_capacity, first_slot, stream);
  }
  const int64_t ux = update_x(n_blocks, step, head_dim, vec);
  BFLY_CHECK_ARG(ux <= INT32_MAX, "grid too large");
  UpdateJob u{k_new, v_new, ring_k, ring_v, pool_k, pool_v, step, ring_capacity, pool_capacity, offset,
              first_block_pos, first_slot, (int)n_blocks, block_size, head_dim};
  dim3 grid((unsigned)ux, (unsigned)(batch * hkv), 2);
  if (dtype == BFLY_DTYPE_F32)
    hipLaunchKernelGGL((cache_update_kernel<float, 4>), grid, dim3(256), 0, stream, u);
  else
    hipLaunchKernelGGL((cache_update_kernel<__bf16, 8>), grid, dim3(256), 0, stream, u);
  BFLY_CHECK_LAUNCH("bfly_cache_update");
  return BFLY_OK;
}
