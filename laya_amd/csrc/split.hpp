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

namespace laya {

__device__ __forceinline__ void split3_4(f32x4 x, bf16x4& h1, bf16x4& h2, bf16x4& h3) {
    h1 = __builtin_convertvector(x, bf16x4);
    const f32x4 r = x - __builtin_convertvector(h1, f32x4);
    h2 = __builtin_convertvector(r, bf16x4);
    const f32x4 r2 = r - __builtin_convertvector(h2, f32x4);
    h3 = __builtin_convertvector(r2, bf16x4);
}

}  // namespace laya
