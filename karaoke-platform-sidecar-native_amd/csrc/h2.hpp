// Two-piece fp16 representation of fp32 values (the default fp32 path's
// operands on the fp16 matrix cores): a value x of an operand whose elements
// are all bounded by B is scaled by 2^e, e = h2_exponent(B) (so |x 2^e| < 2^14),
// and y = x 2^e is held as h = fp16(y), m = fp16(y - h), both nearest even;
// y - h is exact in fp32 and h + m carries 22 significant bits (exact to
// 2^-25 absolute where m is subnormal).
//
// "h2 rows": a fp32 matrix [rows][K] (K a multiple of 16) re-encoded in place
// of its fp32 bytes (the same row pitch): every chunk of 16 k-values of a row
// is 64 bytes -- 16-byte slot 0 holds h of k 0-3 and 8-11, slot 1 h of k 4-7
// and 12-15, slots 2 and 3 the same for m.  A lane of a 32x32x16 MFMA takes k
// {4j..4j+3, 8+4j..8+4j+3} for its half j, so its h operand is slot j and its
// m operand slot 2+j: one 16-byte read each, the read pattern of the fp32
// rows the GEMMs split themselves.
#pragma once

#include "common.hpp"

namespace vh {

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

// The exponent e with bound * 2^e < 2^14 (the largest such, clamped to
// [-100, 100]); 0 for a zero, infinite or NaN bound.
VH_HOST_DEVICE inline int h2_exponent(float bound) {
    if (!(bound > 0.0f) || !(bound <= 3.4e38f)) return 0;
    int E;
    (void)frexpf(bound, &E);  // bound < 2^E
    const int e = 14 - E;
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

// Bounds for which the fp16 two-piece attention kernels may run.  They undo
// the q and k scales with the single power of two 2^-(ek + eq), and the
// output's with 2^-(ev + 5); with B in [2^-40, 2^60] every exponent lies in
// [-62, 56], so ek + eq stays in [-125, 113] and ev + 5 in [-57, 61]: every
// scale and unscale is a normal fp32 power of two.  Beyond that range the
// attention runs on the kernels without piece scales (the three-piece bf16
// split for long sequences, the fp32 MFMA kernel for short ones).
constexpr float H2_ATT_BOUND_MIN = 0x1p-40f;
constexpr float H2_ATT_BOUND_MAX = 0x1p60f;
VH_HOST_DEVICE inline bool h2_attention_bound_ok(float b) { return b >= H2_ATT_BOUND_MIN && b <= H2_ATT_BOUND_MAX; }

// The fp16 two-piece attention's exponents for a bound B on |q|, |k|, |v|
// (before rotation): k and q (times the softmax scale and log2 e, qs) from
// the rotated bound sqrt(2) B, v from B.  One definition for the attention
// kernels and for the fused-projection epilogue that splits k and v ahead of
// them, so both scale alike.
VH_HOST_DEVICE inline void att_h2_exponents(float bnd, float qs, int &ek, int &eq, int &ev) {
    ek = h2_exponent(1.4142135f * 1.0001f * bnd);
    eq = h2_exponent(1.4142135f * 1.0001f * bnd * qs);
    ev = h2_exponent(bnd);
}

// Two fp32 -> two fp16 (nearest even) in one dword: one v_cvt_pk_f16_f32.
VH_DEVICE uint32_t pack_f16x2(float a, float b) {
    typedef float floatx2 __attribute__((ext_vector_type(2)));
    typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){a, b}, halfx2));
}

// The m pieces of two values x0 s, x1 s whose h pieces hp holds (as
// pack_f16x2 made them): x s - h formed inside one v_fma_mix_f32 per value
// (the fp16 h read in place, no conversion, one rounding) and the pair
// rounded to fp16 by one v_cvt_pk_f16_f32, 3 VALU per pair instead of 5.
// For a power-of-two s, x s is exact, so these are the bits of fp16(y - h),
// y = x s (the weights, the GEMM's A, k and v).  For any other s (the
// attention's q times its softmax scale) h + m is the split of the exact
// product x s, which can differ in m's last bits from splitting the rounded
// fp32 product (and is at least as accurate).  s must not be a compile-time
// 1 (the multiply-add would fold back into a conversion and a subtraction):
// pass opaque_one() for unscaled values.
VH_DEVICE uint32_t m_pair_f16(float x0, float x1, float s, uint32_t hp) {
    typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
    const halfx2 h = __builtin_bit_cast(halfx2, hp);
    return pack_f16x2(__builtin_fmaf(x0, s, -(float)h[0]), __builtin_fmaf(x1, s, -(float)h[1]));
}

// 1.0f that the compiler does not constant-fold (see m_pair_f16).
VH_DEVICE float opaque_one() {
    float one = 1.0f;
    asm("" : "+v"(one));
    return one;
}

// Eight fp32 values times s -> their h and m fp16 pieces, packed as the MFMA
// operand wants them (a lane's eight k-values): 2.5 VALU per value.
VH_DEVICE void split8_h2(floatx4 lo, floatx4 hi, float s, halfx8 &h, halfx8 &m) {
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    uint32_t ph[4], pm[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        ph[e] = pack_f16x2(x[2 * e] * s, x[2 * e + 1] * s);
        pm[e] = m_pair_f16(x[2 * e], x[2 * e + 1], s, ph[e]);
    }
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    h = __builtin_bit_cast(halfx8, (u32x4){ph[0], ph[1], ph[2], ph[3]});
    m = __builtin_bit_cast(halfx8, (u32x4){pm[0], pm[1], pm[2], pm[3]});
}

// The same for unscaled values (s = 1): 2 VALU per value.
VH_DEVICE void split8_h2_unit(floatx4 lo, floatx4 hi, halfx8 &h, halfx8 &m) {
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const float one = opaque_one();
    uint32_t ph[4], pm[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        ph[e] = pack_f16x2(x[2 * e], x[2 * e + 1]);
        pm[e] = m_pair_f16(x[2 * e], x[2 * e + 1], one, ph[e]);
    }
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    h = __builtin_bit_cast(halfx8, (u32x4){ph[0], ph[1], ph[2], ph[3]});
    m = __builtin_bit_cast(halfx8, (u32x4){pm[0], pm[1], pm[2], pm[3]});
}

// Byte offsets, inside the 64-byte chunk of an h2 row, of the h piece of the
// four consecutive k-values 4j..4j+3 (j = 0..3 within the chunk); the m
// piece lies 32 bytes further.
VH_HOST_DEVICE inline int h2_row_offset(int j) { return 16 * (j & 1) + 8 * (j >> 1); }

// Four consecutive values (k 4j..4j+3 of the chunk at `chunk`) times s into
// an h2 row: 8 bytes of h and 8 of m.
VH_DEVICE void store4_h2(unsigned char *chunk, int j, floatx4 v, float s) {
    const uint32_t h01 = pack_f16x2(v[0] * s, v[1] * s), h23 = pack_f16x2(v[2] * s, v[3] * s);
    const uint32_t m01 = m_pair_f16(v[0], v[1], s, h01), m23 = m_pair_f16(v[2], v[3], s, h23);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const int o = h2_row_offset(j);
    *reinterpret_cast<u32x2 *>(chunk + o) = u32x2{h01, h23};
    *reinterpret_cast<u32x2 *>(chunk + 32 + o) = u32x2{m01, m23};
}

// The same for four lanes holding the four groups 4j..4j+3 of one chunk, the
// lanes of groups j and j^2 being XOR apart (lane j of a quad: XOR = 2; the
// band-axis attention's lane groups: XOR = 32): they swap one piece, so each
// lane writes a whole 16-byte slot -- groups 0, 1 the h slots, groups 2, 3 the
// m slots -- instead of two 8-byte halves.  Every one of the four lanes takes
// part.
template <int XOR>
VH_DEVICE void store4_h2_swap(unsigned char *chunk, int j, floatx4 v, float s) {
    const uint32_t h01 = pack_f16x2(v[0] * s, v[1] * s), h23 = pack_f16x2(v[2] * s, v[3] * s);
    const uint32_t m01 = m_pair_f16(v[0], v[1], s, h01), m23 = m_pair_f16(v[2], v[3], s, h23);
    const bool h_slot = j < 2;
    const uint32_t r0 = (uint32_t)__shfl_xor((int)(h_slot ? m01 : h01), XOR, 64);
    const uint32_t r1 = (uint32_t)__shfl_xor((int)(h_slot ? m23 : h23), XOR, 64);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    // slot j = h of groups j, j+2; slot 2 + (j-2) = m of groups j-2, j
    if (h_slot) *reinterpret_cast<u32x4 *>(chunk + 16 * j) = u32x4{h01, h23, r0, r1};
    else *reinterpret_cast<u32x4 *>(chunk + 32 + 16 * (j - 2)) = u32x4{r0, r1, m01, m23};
}
VH_DEVICE void store4_h2_quad(unsigned char *chunk, int j, floatx4 v, float s) { store4_h2_swap<2>(chunk, j, v, s); }

// Eight values of one chunk -- k 0-3 and 8-11 (half 0) or k 4-7 and 12-15
// (half 1), the pieces of one MFMA operand half -- times s into an h2 row: h
// to slot `half`, m to slot 2 + `half`, 16 bytes each.
VH_DEVICE void store8_h2_half(unsigned char *chunk, int half, floatx4 lo, floatx4 hi, float s) {
    halfx8 h, m;
    split8_h2(lo, hi, s, h, m);
    *reinterpret_cast<halfx8 *>(chunk + 16 * half) = h;
    *reinterpret_cast<halfx8 *>(chunk + 32 + 16 * half) = m;
}

}  // namespace vh
