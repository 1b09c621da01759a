#pragma once

// fp32 products on bf16 MFMAs ("bf16x6"), shared by the flash prefill and the
// fp32 GEMM: splitting, the six-term product and the LDS chunk swizzles of
// three-part stages.

#include <cstdint>

#include "weight_pack.hpp"

namespace opworks::detail {

// ---- fp32 products on bf16 MFMAs ("bf16x6") --------------------------------
// An fp32 value splits exactly into three bf16 parts, x = x0 + x1 + x2 (each round to nearest
// of the remaining residual; 3 x 8 significand bits cover fp32's 24). A product keeps the six
// terms with i + j <= 2, x_i y_j, each exact in fp32, accumulated by the MFMA in fp32; the
// dropped terms x1 y2, x2 y1 (each at most 2^-24 of |x y|) and x2 y2 stay within 2^-23. Dot
// products then carry fp32's error (checked in float64 against fp32 sums of length 64: the same
// worst case, 6.7e-8 of sum |x y|), at 16 cycles per 16x16x32 bf16 MFMA against 32 per 16x16x4
// fp32 one: per 16x16x64 block, 12 x 16 against 16 x 32 cycles.
using bf16x8v = __bf16 __attribute__((ext_vector_type(8)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

using bf16x2v = __bf16 __attribute__((ext_vector_type(2)));

// (a, b) -> packed bf16 words, a in the low half, rounded to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    const bf16x2v v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
}
// (a, b) -> three packed words w0, w1, w2 with a == lo(w0) + lo(w1) + lo(w2), b likewise in the
// high halves; each residual is exact in fp32
__device__ __forceinline__ void split3x2(float a, float b, uint32_t &w0, uint32_t &w1, uint32_t &w2) {
    w0 = cvt_pk_bf16(a, b);
    a -= __uint_as_float(w0 << 16);
    b -= __uint_as_float(w0 & 0xffff0000u);
    w1 = cvt_pk_bf16(a, b);
    a -= __uint_as_float(w1 << 16);
    b -= __uint_as_float(w1 & 0xffff0000u);
    w2 = cvt_pk_bf16(a, b);
}
// eight floats -> their three bf16x8 parts
__device__ __forceinline__ void split3x8(const float (&x)[8], bf16x8v (&part)[3]) {
    uint32_t w[3][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        split3x2(x[2 * j], x[2 * j + 1], w[0][j], w[1][j], w[2][j]);
#pragma unroll
    for (int p = 0; p < 3; ++p)
        part[p] = __builtin_bit_cast(bf16x8v, u32x4{w[p][0], w[p][1], w[p][2], w[p][3]});
}
// acc += term `term` of a b with both operands as three parts; terms 0..5 in turn add the six
// products, smallest first: a2 b0, a1 b1, a0 b2, a1 b0, a0 b1, a0 b0
__device__ __forceinline__ f32x4 mfma_x6_term(int term, const bf16x8v (&a)[3], const bf16x8v (&b)[3], f32x4 acc) {
    constexpr int ia[6] = {2, 1, 0, 1, 0, 0}, ib[6] = {0, 1, 2, 0, 1, 0};
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[ia[term]], b[ib[term]], acc, 0, 0, 0);
}
// LDS chunk swizzles of the three-part stages, for the fragment reads: lane (l16, g) reads the
// 16-byte chunk of row l16 that g selects. Measured with the bank-conflict counter on an LDS
// probe of these exact address patterns (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE): rows padded
// to 144 or 80 bytes ran 2-way, 128-byte rows with chunk c ^ 2 ((r / 4) mod 4) also 2-way, and the
// two swizzles below conflict-free:
//  * 128-byte rows (K at head_dim 64): chunk c of row r in c ^ ((r >> 1) & 7), the bf16 GEMM's;
//  * 64-byte rows (V^T, and K at head_dim 32): chunk c of row r in c ^ 2 bit3(r) ^ bit4(r).
// The staging writes (one 8-byte piece per lane) meet at most two-way conflicts.
template <int kD> __device__ __forceinline__ int x6_k_chunk(int c, int r) {
    if constexpr (kD == 64)
        return c ^ ((r >> 1) & 7);
    else
        return c ^ (2 * ((r >> 3) & 1)) ^ ((r >> 4) & 1);
}
__device__ __forceinline__ int x6_v_chunk(int c, int d) { return c ^ (2 * ((d >> 3) & 1)) ^ ((d >> 4) & 1); }

} // namespace opworks::detail
