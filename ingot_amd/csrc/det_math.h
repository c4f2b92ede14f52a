// Deterministic fp32 arithmetic shared by the HIP kernels and the CPU code.
//
// Routing decisions (which experts a token goes to) must be bit-identical on
// the CPU and on the GPU, ties included (src/lib.rs:43-60 sorts with
// f32::total_cmp and breaks ties toward the lower expert id). A last-ulp
// difference in a router logit or in a sigmoid score can flip a near-tie, so
// every fp32 value that feeds a selection is computed here by one fixed
// sequence of IEEE-754 operations (explicit fused multiply-adds, no
// contraction, no reassociation, correctly rounded division), which both
// compilers must reproduce exactly.
//
//  * ingot_det_expf: exp(x) by Cody-Waite range reduction x = n*ln2 + r with a
//    two-part ln2, then the degree-7 Taylor polynomial of e^r in Horner form
//    (coefficients 1/k!), scaled by 2^n through the exponent bits. Relative
//    error is a few ulp on the whole fp32 range; underflow flushes to 0 below
//    -103.9 and overflow saturates to +inf above 88.73.
//  * ingot_orderable: maps fp32 bits to a uint32 whose unsigned order is the
//    IEEE total order (f32::total_cmp): -NaN < -inf < ... < -0 < +0 < ... <
//    +inf < +NaN.
//  * Router logits: see ingot_router_partial / ingot_butterfly64 below.
#pragma once
#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define INGOT_DET __host__ __device__ inline
#else
#define INGOT_DET static inline
#endif

#if defined(__clang__)
#define INGOT_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define INGOT_NO_CONTRACT
#endif

INGOT_DET uint32_t ingot_f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
INGOT_DET float ingot_u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

INGOT_DET uint32_t ingot_orderable(float f) {
    uint32_t u = ingot_f2u(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Selection key: higher value first, equal values resolved toward the lower id.
INGOT_DET uint64_t ingot_select_key(float v, uint32_t id) {
    return ((uint64_t)ingot_orderable(v) << 32) | (uint64_t)(0xffffffffu - id);
}

INGOT_DET float ingot_fma(float a, float b, float c) {
#ifdef __HIP_DEVICE_COMPILE__
    return __builtin_fmaf(a, b, c);
#else
    return __builtin_fmaf(a, b, c);
#endif
}

INGOT_DET float ingot_rint(float x) {
    return __builtin_rintf(x);
}

INGOT_DET float ingot_det_expf(float x) {
    INGOT_NO_CONTRACT
    if (x != x) return x;
    if (x > 88.7228391f) return ingot_u2f(0x7f800000u);
    if (x < -103.972084f) return 0.0f;
    const float log2e = 1.44269502f;
    const float ln2_hi = 0.693145752f;       // 0x3f317200: 16 significant bits, n*ln2_hi exact
    const float ln2_lo = 1.42860677e-06f;    // ln2 - ln2_hi
    float n = ingot_rint(x * log2e);
    float r = ingot_fma(-n, ln2_hi, x);
    r = ingot_fma(-n, ln2_lo, r);
    // e^r = sum_k r^k / k!, k = 0..7, Horner.
    float p = 1.98412698e-04f;               // 1/5040
    p = ingot_fma(p, r, 1.38888889e-03f);    // 1/720
    p = ingot_fma(p, r, 8.33333333e-03f);    // 1/120
    p = ingot_fma(p, r, 4.16666667e-02f);    // 1/24
    p = ingot_fma(p, r, 1.66666667e-01f);    // 1/6
    p = ingot_fma(p, r, 0.5f);
    p = ingot_fma(p, r, 1.0f);
    p = ingot_fma(p, r, 1.0f);
    int32_t e = (int32_t)n;
    // 2^e in two steps so that results in the subnormal range stay exact
    // multiplications by powers of two.
    int32_t e1 = e / 2, e2 = e - e1;
    float s1 = ingot_u2f((uint32_t)(e1 + 127) << 23);
    float s2 = ingot_u2f((uint32_t)(e2 + 127) << 23);
    return (p * s1) * s2;
}

// sigmoid(x) = 1 / (1 + e^-x), correctly rounded division on both sides.
INGOT_DET float ingot_det_sigmoid(float x) {
    INGOT_NO_CONTRACT
    float e = ingot_det_expf(-x);
    return 1.0f / (1.0f + e);
}

// Router logit reduction order (fp32 router matrix W[E][H], H % 256 == 0).
// The H columns are split over 64 slots: slot l owns columns
// 4*l + 256*i + c for i = 0..H/256-1, c = 0..3, accumulated in that order by
// fused multiply-adds starting from +0. The 64 slot sums are then combined by
// the butterfly v_l <- v_l + v_(l xor m) for m = 32, 16, 8, 4, 2, 1; the logit
// is v_0. On the GPU slot l is wave lane l; the CPU replays the same tree.
INGOT_DET float ingot_router_partial(const float* w_row, const float* x, uint32_t H, uint32_t l) {
    INGOT_NO_CONTRACT
    float acc = 0.0f;
    for (uint32_t i = 0; i < H / 256; ++i)
        for (uint32_t c = 0; c < 4; ++c) {
            uint32_t j = 4 * l + 256 * i + c;
            acc = ingot_fma(w_row[j], x[j], acc);
        }
    return acc;
}

INGOT_DET float ingot_butterfly64(float* v) {
    INGOT_NO_CONTRACT
    float t[64];
    for (uint32_t m = 32; m >= 1; m >>= 1) {
        for (uint32_t l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ m];
        for (uint32_t l = 0; l < 64; ++l) v[l] = t[l];
    }
    return v[0];
}
