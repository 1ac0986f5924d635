// Exact three-piece bf16 splits of fp32 values, shared by the split-product GEMMs and attention.
//
// x = x1 + x2 + x3 exactly: x1 = bf16(x) to nearest even (the hardware convert), x2 = bf16(x − x1),
// x3 = x − x1 − x2. Each remainder is exact in fp32 and 24 significand bits = 8 + 8 + 8, so x3 is itself
// a bf16 value. A product a·b accumulated in fp32 from the six piece products a3b1, a1b3, a2b2, a2b1,
// a1b2, a1b1 (the three dropped ones are below 2⁻²⁴ of the product) carries fp32 rounding only.
#pragma once

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

namespace laya {

// Two values to nearest-even bf16 with one convert; the pair's fp32 values are the low half shifted up
// and the high half masked, so each level costs one convert, two bit operations and two subtractions.
__device__ __forceinline__ unsigned bf16_pair(float a, float b, float& ra, float& rb) {
    const unsigned u = __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2{a, b}), bf16x2));
    ra = a - __builtin_bit_cast(float, u << 16);
    rb = b - __builtin_bit_cast(float, u & 0xffff0000u);
    return u;
}

__device__ __forceinline__ void split3_4(f32x4 x, bf16x4& h1, bf16x4& h2, bf16x4& h3) {
    float r0, r1, r2, r3, q0, q1, q2, q3;
    const unsigned a01 = bf16_pair(x[0], x[1], r0, r1), a23 = bf16_pair(x[2], x[3], r2, r3);
    const unsigned b01 = bf16_pair(r0, r1, q0, q1), b23 = bf16_pair(r2, r3, q2, q3);
    const unsigned c01 = __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2{q0, q1}), bf16x2));
    const unsigned c23 = __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2{q2, q3}), bf16x2));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    h1 = __builtin_bit_cast(bf16x4, (u32x2{a01, a23}));
    h2 = __builtin_bit_cast(bf16x4, (u32x2{b01, b23}));
    h3 = __builtin_bit_cast(bf16x4, (u32x2{c01, c23}));
}

// Two-piece fp16 split of s·x, s a power of two that brings the operand's largest magnitude into
// [2¹⁴, 2¹⁵): hi = f16(s·x) to nearest even, lo = f16(s·x − hi) (the remainder is exact in fp32, one
// fused mix-precision subtract). hi + lo holds s·x to 2⁻²² of its magnitude for every element above
// 2⁻¹⁸ of the operand's largest, and to 2⁻⁴⁰ of the largest below that. A product a·b accumulated in
// fp32 from the three piece products alo·bhi, ahi·blo, ahi·bhi (the dropped alo·blo is below 2⁻²² of
// the product) is within a few 2⁻²⁴ of the exact product, under the fp32 accumulation's own rounding.
__device__ __forceinline__ void split2h_4(f32x4 x, float s, f16x4& hi, f16x4& lo) {
    const f32x4 v = x * s;
    hi = __builtin_convertvector(v, f16x4);
    lo = __builtin_convertvector(v - __builtin_convertvector(hi, f32x4), f16x4);
}

// One fp16 piece of s·x for bf16-valued x (an fp32 whose low 16 bits are zero), s the operand's scale as
// above: s·x carries 8 significant bits, so f16(s·x) is s·x exactly wherever |s·x| ≥ 2⁻¹⁷ (fp16's
// subnormal spacing 2⁻²⁴ times 2⁷), i.e. for every element above 2⁻³¹ of the operand's largest; below
// that it is within 2⁻²⁵, 2⁻³⁹ of the largest, the order of the two-piece form's own bound there. The
// two-piece form's lo piece is then zero and its products with it add nothing: dropping them leaves the
// same sums.
__device__ __forceinline__ f16x4 split1h_4(f32x4 x, float s) { return __builtin_convertvector(x * s, f16x4); }

// The same split at unit scale: hi = f16(x), lo = f16(x − hi). `one` is 1.0 held where the compiler cannot
// fold it, so the exact remainder x·1 − hi is one fused mix-precision multiply-add on the fp16 hi rather
// than a convert back to fp32 and a subtraction.
__device__ __forceinline__ void split2h_4u(f32x4 x, float one, f16x4& hi, f16x4& lo) {
    hi = __builtin_convertvector(x, f16x4);
    const f32x4 h = __builtin_convertvector(hi, f32x4);
    f32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __builtin_fmaf(x[i], one, -h[i]);
    lo = __builtin_convertvector(r, f16x4);
}

// The scale exponent of an operand whose largest finite magnitude has the fp32 bit pattern `amax`:
// s = 2^e with e = 14 − exponent(amax), clamped to [−126, 126] (an all-zero operand takes 2¹²⁶).
__device__ __forceinline__ int pair_scale_exp(unsigned amax) {
    const int e = 14 - ((int)(amax >> 23) - 127);
    return e < -126 ? -126 : e > 126 ? 126 : e;
}
__device__ __forceinline__ float exp2_int(int e) { return __builtin_bit_cast(float, (unsigned)(e + 127) << 23); }

}  // namespace laya
