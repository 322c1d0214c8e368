// The per-lane arithmetic of the one-row 4-bit products (qgemv.hip), shared with the
// decode step that applies the attention output projection itself (decode.hip), so
// that both give the same bits for the same row.
//
// Layout (bfly_q4_gemv): W is [rows][pieces] 16-byte pieces of 32 codes, two codes
// per byte (low nibble first); one 32-bit word of bf16 (scale, bias) per group of
// codes along the input dimension; w = code * scale + bias.  A lane takes one piece
// of a row: x_i code_i summed over the piece's even and odd codes separately, then
// scale * (even + odd) + bias * sum(x_i).
#pragma once

#include "bfly_common.h"

namespace bfly {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ4PieceCodes = 32;   // codes in one 16-byte piece of a row

// The 32 x values of a piece from four 8-element bf16 pieces: xq[i] = x_i, the odd
// ones divided by 16 (masking the high nibbles in place gives 16 * code, and
// (x / 16) * (16 * code) is x * code exactly), and xs = the sum of the x_i in order.
// A lane past the row (valid false) gets zeros.
__device__ __forceinline__ void q4_piece_x(const bf16x8 (&xr)[4], bool valid, float (&xq)[kQ4PieceCodes],
                                           float& xs) {
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) xq[8 * c + e] = valid ? (float)xr[c][e] : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kQ4PieceCodes; ++i) {
    s += xq[i];
    if (i & 1) xq[i] *= 0.0625f;
  }
  xs = s;
}

// One piece's part of a row's product: scale * sum(x code) + bias * sum(x).
__device__ __forceinline__ float q4_piece_dot(const u32x4& wv, uint32_t sv, const float (&xq)[kQ4PieceCodes],
                                              float xs) {
  const uint32_t dw[4] = {wv[0], wv[1], wv[2], wv[3]};
  float lo_sum = 0.f, hi_sum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t lo = dw[t] & 0x0F0F0F0Fu, hi = dw[t] & 0xF0F0F0F0u;
    // opaque to the combiner, so each byte converts with v_cvt_f32_ubyte{0..3}
    // instead of a bit-field extract of the unmasked word and a conversion
    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      lo_sum += xq[8 * t + 2 * b] * (float)((lo >> (8 * b)) & 0xFFu);
      hi_sum += xq[8 * t + 2 * b + 1] * (float)((hi >> (8 * b)) & 0xFFu);
    }
  }
  const float scale = __uint_as_float(sv << 16);
  const float bias = __uint_as_float(sv & 0xFFFF0000u);
  return scale * (lo_sum + hi_sum) + bias * xs;
}

// v summed over the 16 lanes of each row of 16 (rotations by 8 and 4, then two quad
// permutations, DPP): every lane of the row holds the row's total.
__device__ __forceinline__ float q4_row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  return v;
}

// v summed over the 64 lanes, the total in every lane, no LDS traffic: the rows of 16
// first (q4_row16_sum), then rows 0 + 1 and 2 + 3 (v_permlane16_swap), then the two
// halves (v_permlane32_swap).  With row r's total t_r the result is
// (t_0 + t_1) + (t_2 + t_3), the order in which a row's four 16-piece partials are
// combined where they are computed apart (bfly_add_rms_norm_q4_gemv_silu_parts).
__device__ __forceinline__ float q4_wave_sum(float v) {
  v = q4_row16_sum(v);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

}  // namespace bfly
