// Shared helpers for the Butterfly compressed-attention HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/butterfly_amd.h"

namespace bfly {

// Per-thread last-error string returned by bfly_last_error().
void set_error(const char* fmt, ...);

#define BFLY_CHECK_ARG(cond, ...)          \
  do {                                     \
    if (!(cond)) {                         \
      ::bfly::set_error(__VA_ARGS__);      \
      return BFLY_ERR_INVALID;             \
    }                                      \
  } while (0)

#define BFLY_CHECK_LAUNCH(what)                                              \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      ::bfly::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
      return BFLY_ERR_HIP;                                                   \
    }                                                                        \
  } while (0)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }

// Max / sum of v over lanes L, L^16, L^32, L^48 (the four lane groups that hold
// one MFMA column), on the VALU: v_permlane16_swap / v_permlane32_swap exchange
// rows of 16 / halves of 32 lanes, so max(a, b) of a swapped pair is the
// reduction with lane ^ 16 (^ 32) in every lane.  Same order as two xor
// shuffles (16, then 32), so the sums are bit-identical to that form.
__device__ __forceinline__ float col_max4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Four bf16 of column-major data from row-major LDS: within each 16-lane group,
// lane i receives element (i & 3) of the 8 bytes read by lanes 4j + (i >> 2),
// j = 0..3, as its elements j (ds_read_b64_tr_b16).
__device__ __forceinline__ bf16x4 read_tr(const __bf16* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(const_cast<__bf16*>(p)));
  return __builtin_bit_cast(bf16x4, v);
}

// Row-major bf16 V tiles in LDS keep their 16-byte pieces XOR-swizzled by the
// row (piece pc of row r at pc ^ vrow_swizzle<D>(r)), so that the transposing
// reads of four consecutive rows (read_tr over rows 4k..4k+3) hit distinct banks.
template <int D>
__device__ __forceinline__ constexpr int vrow_swizzle(int row) {
  return D == 64 ? ((row >> 1) & 1) * 4 : (row & 3) * 4;
}

// Vectorised paths issue 16-byte loads/stores: tensor base pointers must be 16-byte aligned.
__host__ __forceinline__ bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0..N-1, so
// register arrays indexed by I never become private (scratch) memory.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// Floor division / modulo for possibly negative positions.
__host__ __device__ __forceinline__ int64_t floordiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__host__ __device__ __forceinline__ int64_t posmod(int64_t a, int64_t b) {
  int64_t r = a % b;
  return r < 0 ? r + b : r;
}

}  // namespace bfly
