// Device-side decoding of GGUF blocks for the MoE kernels (gfx950).
//
// Every supported format is handled in "chunks" of 32 weights of one row:
//   chunk c of a row covers 32 columns chosen by the format so that one chunk
//   is one natural unit of its block layout (a 32-value group of a 256-value
//   superblock, or one 32-value block):
//     Q4_K, Q5_K  superblock c/8, quarter q=(c%8)/2, half h=c%2: 16 bytes of
//             nibbles holding columns 64q+16h+[0,16) (low nibbles, group 2q)
//             and 64q+32+16h+[0,16) (high nibbles, group 2q+1)
//     other 256-value superblocks (Q2_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S,
//             IQ3_XXS, IQ3_S, IQ4_XS, IQ1_M): superblock c/8, group c%8:
//             columns 32*(c%8)+[0,32)
//     Q2_0    half c%2 of 64-value block c/2
//     Q8_0, Q4_0, IQ4_NL, F32, F16, BF16: block / columns 32c+[0,32)
//   Chunks 2s and 2s+1 together always cover the 64 columns [64s, 64s+64):
//   the GEMM kernels stage weights in 64-column slabs built from two chunks.
//
// The formulas are the reference's (kernels/iq3_mix.metal:13-36 for Q4_K,
// Q5_K, IQ2_XS and IQ3_XXS; kernels/moe.metal:13-89 for F32, F16, Q4_0, Q8_0,
// Q2_K, Q6_K, IQ2_XXS, IQ1_M, BF16, Q2_0, IQ2_S, IQ3_S, IQ4_NL and IQ4_XS), organised for 16-byte loads and factored scales: a chunk dot
// product is sum_i w_i x_i with w_i = scale * small_int_i - min, evaluated as
// scale * sum_i small_int_i x_i - min * sum_i x_i.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codebooks.h"

namespace ingot {

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// 4 bytes from a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t i) { return (w >> (8 * i)) & 0xffu; }
__device__ __forceinline__ float ubyte_f(uint32_t w, uint32_t i) { return (float)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ float sbyte_f(uint32_t w, uint32_t i) { return (float)(int8_t)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ float flip_sign(float v, uint32_t bit) {
    return __int_as_float(__float_as_int(v) ^ (int)(bit << 31));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

template <int KIND>
struct Fmt;

// ------------------------------------------------------------------ Q4_K (12)
template <>
struct Fmt<12> {
    static constexpr uint32_t BLOCK = 256, BYTES = 144;
    // Column of value i (0..31) of chunk c.
    __device__ static uint32_t col(uint32_t c, uint32_t i) {
        uint32_t q = c & 7u;
        return (c >> 3) * 256u + 64u * (q >> 1) + 16u * (q & 1u) + (i < 16 ? i : 16u + i);
    }
    __device__ static void load_x(const float* x, uint32_t c, float* xv) {
        uint32_t q = c & 7u;
        const float* p = x + (c >> 3) * 256u + 64u * (q >> 1) + 16u * (q & 1u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 a = reinterpret_cast<const float4*>(p)[i];
            float4 b = reinterpret_cast<const float4*>(p + 32)[i];
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
            xv[16 + 4 * i] = b.x; xv[17 + 4 * i] = b.y; xv[18 + 4 * i] = b.z; xv[19 + 4 * i] = b.w;
        }
    }
    // Scale (sc) and min (m) of the chunk's two groups, from the 16-byte header
    // {d, dmin, scales[12]} (ggml get_scale_min_k4, kernels/iq3_mix.metal:13-15).
    // Branch-free (lanes of a wave hold different quarters): both 6-bit
    // unpackings are formed and selected, and the quarter's odd half moves
    // its two bytes down.
    __device__ static void scales(uint4 hdr, uint32_t c, float& d0, float& m0, float& d1, float& m1) {
        const uint32_t qq = (c & 7u) >> 1;  // 64-column quarter: groups 2qq, 2qq+1
        const uint32_t sc_lo = hdr.y & 0x3f3f3f3fu, mn_lo = hdr.z & 0x3f3f3f3fu;
        const uint32_t sc_hi = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
        const uint32_t sh = 16u * (qq & 1u);
        const uint32_t scw = (qq < 2u ? sc_lo : sc_hi) >> sh, mw = (qq < 2u ? mn_lo : mn_hi) >> sh;
        const float d = half_bits_to_float(hdr.x), dm = half_bits_to_float(hdr.x >> 16);
        d0 = d * ubyte_f(scw, 0);
        d1 = d * ubyte_f(scw, 1);
        m0 = dm * ubyte_f(mw, 0);
        m1 = dm * ubyte_f(mw, 1);
    }
    // Raw bytes of a chunk for the GEMM staging path: {header, nibbles}.
    struct Raw {
        uint4 a, b;
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        uint32_t q = c & 7u;
        Raw r;
        r.a = *reinterpret_cast<const uint4*>(b);
        r.b = *reinterpret_cast<const uint4*>(b + 16 + 32 * (q >> 1) + 16 * (q & 1u));
        return r;
    }
    // A nibble byte (0..15) read as an OCP fp8 e4m3 value is exactly
    // q * 2^-9 (subnormal m/8 * 2^-6 below 8, 2^-6 (1 + m/8) from 8), so one
    // v_cvt_pk_f32_fp8 converts two nibbles; the sums carry 2^-9 and the
    // scaled term is multiplied back by 2^9 (exact: powers of two commute
    // with every rounding in the normal range, so the result is the
    // q-weighted sum's).
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float xs0, float xs1) {
        float d0, m0, d1, m1;
        scales(r.a, c, d0, m0, d1, m1);
        const uint32_t w[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = w[k] & 0x0f0f0f0fu, hi = (w[k] >> 4) & 0x0f0f0f0fu;
            const f32x2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
            const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
            slo = __builtin_fmaf(l01.x, xv[4 * k], slo);
            shi = __builtin_fmaf(h01.x, xv[16 + 4 * k], shi);
            slo = __builtin_fmaf(l01.y, xv[4 * k + 1], slo);
            shi = __builtin_fmaf(h01.y, xv[16 + 4 * k + 1], shi);
            slo = __builtin_fmaf(l23.x, xv[4 * k + 2], slo);
            shi = __builtin_fmaf(h23.x, xv[16 + 4 * k + 2], shi);
            slo = __builtin_fmaf(l23.y, xv[4 * k + 3], slo);
            shi = __builtin_fmaf(h23.y, xv[16 + 4 * k + 3], shi);
        }
        return 512.0f * (d0 * slo + d1 * shi) - (m0 * xs0 + m1 * xs1);
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float xs0, float xs1) {
        return dot_raw(load_raw(row, c), c, xv, xs0, xs1);
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        float d0, m0, d1, m1;
        scales(r.a, c, d0, m0, d1, m1);
        uint32_t v[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo = v[k] & 0x0f0f0f0fu, hi = (v[k] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w[4 * k + j] = d0 * ubyte_f(lo, j) - m0;
                w[16 + 4 * k + j] = d1 * ubyte_f(hi, j) - m1;
            }
        }
    }
};

// --------------------------------------------------------- contiguous chunks
// Formats whose chunk c covers columns 32c..32c+31 in order.
// Codebooks in LDS. A lookup with a per-lane index into __constant__ memory
// is a vector memory access chained after the weight load that supplies the
// index, so every kernel that decodes an IQ format copies the
// codebook into LDS first: stage_codebooks<KIND>() at kernel start, followed
// by a barrier before the first decode.
__device__ inline uint64_t* lds_iq2xs_grid() {
    __shared__ uint64_t g[512];
    return g;
}
__device__ inline uint32_t* lds_iq3xxs_grid() {
    __shared__ uint32_t g[256];
    return g;
}
// The same grid for the f16 GEMM with each entry's 4 bytes spread into two
// u16 pairs ({b0, b1}, {b2, b3}): the operand build multiplies them as they are.
__device__ inline uint2* lds_iq3xxs_grid_u16() {
    __shared__ uint2 g[256];
    return g;
}
__device__ inline float* lds_iq4nl_values() {
    __shared__ float v[16];
    return v;
}
__device__ inline uint64_t* lds_iq2xxs_grid() {
    __shared__ uint64_t g[256];
    return g;
}
__device__ inline uint64_t* lds_iq2s_grid() {
    __shared__ uint64_t g[1024];
    return g;
}
__device__ inline uint32_t* lds_iq3s_grid() {
    __shared__ uint32_t g[512];
    return g;
}
__device__ inline uint64_t* lds_iq1s_grid() {
    __shared__ uint64_t g[2048];
    return g;
}
template <int KIND>
__device__ inline void stage_codebooks() {
    if constexpr (KIND == 17) {
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) lds_iq2xs_grid()[i] = ingot_iq2xs_grid[i];
    } else if constexpr (KIND == 18) {
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) lds_iq3xxs_grid()[i] = ingot_iq3xxs_grid[i];
    } else if constexpr (KIND == 20 || KIND == 23) {
        if (threadIdx.x < 16u) lds_iq4nl_values()[threadIdx.x] = (float)ingot_kvalues_iq4nl[threadIdx.x];
    } else if constexpr (KIND == 16) {
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) lds_iq2xxs_grid()[i] = ingot_iq2xxs_grid[i];
    } else if constexpr (KIND == 22) {
        for (uint32_t i = threadIdx.x; i < 1024u; i += blockDim.x) lds_iq2s_grid()[i] = ingot_iq2s_grid[i];
    } else if constexpr (KIND == 21) {
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) lds_iq3s_grid()[i] = ingot_iq3s_grid[i];
    } else if constexpr (KIND == 29) {
        for (uint32_t i = threadIdx.x; i < 2048u; i += blockDim.x) lds_iq1s_grid()[i] = ingot_iq1s_grid[i];
    }
}
template <int KIND>
constexpr bool has_codebook() {
    return KIND == 16 || KIND == 17 || KIND == 18 || KIND == 20 || KIND == 21 || KIND == 22 || KIND == 23 ||
           KIND == 29;
}

// Tables of the f16 grouped GEMM, whose B operands are integers held as f16
// bit patterns (an f16 with bits b <= 2047 has the value b * 2^-24 exactly).
//   iq3 sign masks: entry i spreads the 8 signs of ingot_ksign(i) over four
//     f16 pairs, sign of value 2j in bit 15 and of 2j + 1 in bit 31 of word j.
//   iq4_nl pairs: entry b holds the two codebook values of the nibbles of b
//     (low nibble in the low half) as sign-magnitude f16 bit patterns.
__device__ inline uint4* lds_iq3_signmask() {
    __shared__ uint4 m[128];
    return m;
}
__device__ inline uint32_t* lds_iq4nl_pairs() {
    __shared__ uint32_t p[256];
    return p;
}
__device__ inline uint32_t iq4nl_f16_bits(int v) { return v < 0 ? 0x8000u | (uint32_t)(-v) : (uint32_t)v; }
// 8-bit sign masks (entry s: bit 2j of s in bit 15, bit 2j + 1 in bit 31 of
// word j), for the formats with explicit sign bytes.
__device__ inline uint4* lds_sign8mask() {
    __shared__ uint4 m[256];
    return m;
}
__device__ inline uint4 sign_mask8(uint32_t sg) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (((sg >> (2 * j)) & 1u) << 15) | (((sg >> (2 * j + 1)) & 1u) << 31);
    return make_uint4(w[0], w[1], w[2], w[3]);
}
template <int KIND>
__device__ inline void stage_f16_tables() {
    if constexpr (KIND == 22) {
        for (uint32_t i = threadIdx.x; i < 1024u; i += blockDim.x) lds_iq2s_grid()[i] = ingot_iq2s_grid[i];
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) lds_sign8mask()[i] = sign_mask8(i);
    } else if constexpr (KIND == 21) {
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) lds_iq3s_grid()[i] = ingot_iq3s_grid[i];
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) lds_sign8mask()[i] = sign_mask8(i);
    } else if constexpr (KIND == 17) {
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) lds_iq2xs_grid()[i] = ingot_iq2xs_grid[i];
        for (uint32_t i = threadIdx.x; i < 128u; i += blockDim.x) {
            const uint32_t s = ingot_ksign(i);
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = (((s >> (2 * j)) & 1u) << 15) | (((s >> (2 * j + 1)) & 1u) << 31);
            lds_iq3_signmask()[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else if constexpr (KIND == 18) {
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) {
            const uint32_t e = ingot_iq3xxs_grid[i];
            lds_iq3xxs_grid_u16()[i] =
                make_uint2((e & 0xffu) | ((e << 8) & 0xff0000u), ((e >> 16) & 0xffu) | ((e >> 8) & 0xff0000u));
        }
        for (uint32_t i = threadIdx.x; i < 128u; i += blockDim.x) {
            const uint32_t s = ingot_ksign(i);
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = (((s >> (2 * j)) & 1u) << 15) | (((s >> (2 * j + 1)) & 1u) << 31);
            lds_iq3_signmask()[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else if constexpr (KIND == 20 || KIND == 23) {
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x)
            lds_iq4nl_pairs()[i] =
                iq4nl_f16_bits(ingot_kvalues_iq4nl[i & 15u]) | (iq4nl_f16_bits(ingot_kvalues_iq4nl[i >> 4]) << 16);
    }
}

// Tables of the decode GEMV formats that take their inputs as f16 pairs
// (half_x<KIND>): the input is staged as f16 hi + scaled lo, and the chunk
// dot product runs on v_dot2 (exact f16 products, fp32 sums).
//   iq2_xs grid (f16): entry i holds the 8 grid values of ingot_iq2xs_grid[i]
//     as f16 numbers (value 2j in the low half of word j); signs come from
//     the iq3 sign masks (same 7-bit sign index, same parity rule).
//   iq2_xxs and iq2_s grids (f16): the same for their codebooks; IQ2_XXS
//     takes the iq3 sign masks, IQ2_S its explicit sign bytes through the
//     8-bit sign masks (entry s: bit 2j of s in bit 15, bit 2j + 1 in bit 31
//     of word j).
//   iq3_s grid (f16): entry i holds its 4 values as two f16 pairs.
template <int KIND>
constexpr bool half_x() {
    return KIND == 16 || KIND == 17 || KIND == 21 || KIND == 22;
}
__device__ inline uint4* lds_iq2xs_grid_h() {
    __shared__ uint4 g[512];
    return g;
}
__device__ inline uint4* lds_iq2xxs_grid_h() {
    __shared__ uint4 g[256];
    return g;
}
__device__ inline uint4* lds_iq2s_grid_h() {
    __shared__ uint4 g[1024];
    return g;
}
__device__ inline uint2* lds_iq3s_grid_h() {
    __shared__ uint2 g[512];
    return g;
}
__device__ inline uint32_t f16_bits_of(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
// Bytes 2j, 2j + 1 of a codebook entry as an f16 pair.
__device__ inline uint32_t grid_pair_h(uint64_t g, int j) {
    return f16_bits_of((float)((g >> (16 * j)) & 255u)) | (f16_bits_of((float)((g >> (16 * j + 8)) & 255u)) << 16);
}
template <int KIND>
__device__ inline void stage_half_tables() {
    if constexpr (KIND == 16 || KIND == 17) {
        for (uint32_t i = threadIdx.x; i < (KIND == 17 ? 512u : 256u); i += blockDim.x) {
            const uint64_t g = KIND == 17 ? ingot_iq2xs_grid[i] : ingot_iq2xxs_grid[i];
            const uint4 h = make_uint4(grid_pair_h(g, 0), grid_pair_h(g, 1), grid_pair_h(g, 2), grid_pair_h(g, 3));
            if constexpr (KIND == 17) lds_iq2xs_grid_h()[i] = h;
            else lds_iq2xxs_grid_h()[i] = h;
        }
        for (uint32_t i = threadIdx.x; i < 128u; i += blockDim.x) lds_iq3_signmask()[i] = sign_mask8(ingot_ksign(i));
    } else if constexpr (KIND == 21 || KIND == 22) {
        if constexpr (KIND == 22) {
            for (uint32_t i = threadIdx.x; i < 1024u; i += blockDim.x) {
                const uint64_t g = ingot_iq2s_grid[i];
                lds_iq2s_grid_h()[i] = make_uint4(grid_pair_h(g, 0), grid_pair_h(g, 1), grid_pair_h(g, 2), grid_pair_h(g, 3));
            }
        } else {
            for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) {
                const uint64_t g = ingot_iq3s_grid[i];
                lds_iq3s_grid_h()[i] = make_uint2(grid_pair_h(g, 0), grid_pair_h(g, 1));
            }
        }
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) lds_sign8mask()[i] = sign_mask8(i);
    }
}

// Two-phase table staging for the decode kernels (NT threads per block):
// load() issues the global loads of this thread's table entries into
// registers, store() writes the LDS tables that stage_half_tables (HALF) or
// stage_codebooks would write. A kernel calls load() before its other loads
// and store() once those are issued: vector-memory loads complete in issue
// order, so the tables' loads hold back no later load, and store() waits for
// nothing but them.
template <int KIND, bool HALF, uint32_t NT>
struct TableStage {
    static constexpr uint32_t N = KIND == 16   ? 256u
                                  : KIND == 17 ? 512u
                                  : KIND == 18 ? 256u
                                  : KIND == 20 || KIND == 23 ? 16u
                                  : KIND == 21 ? 512u
                                  : KIND == 22 ? 1024u
                                  : KIND == 29 ? 2048u
                                               : 0u;
    static constexpr uint32_t PER = (N + NT - 1) / NT;
    uint64_t v[PER > 0 ? PER : 1];
    static __device__ __forceinline__ uint64_t src(uint32_t i) {
        if constexpr (KIND == 16) return ingot_iq2xxs_grid[i];
        else if constexpr (KIND == 17) return ingot_iq2xs_grid[i];
        else if constexpr (KIND == 18) return ingot_iq3xxs_grid[i];
        else if constexpr (KIND == 20 || KIND == 23) return (uint64_t)(uint8_t)ingot_kvalues_iq4nl[i];
        else if constexpr (KIND == 21) return ingot_iq3s_grid[i];
        else if constexpr (KIND == 22) return ingot_iq2s_grid[i];
        else if constexpr (KIND == 29) return ingot_iq1s_grid[i];
        else return 0;
    }
    __device__ __forceinline__ void load() {
#pragma unroll
        for (uint32_t p = 0; p < PER; ++p) {
            const uint32_t i = threadIdx.x + NT * p;
            v[p] = i < N ? src(i) : 0ull;
        }
    }
    __device__ __forceinline__ void store() const {
#pragma unroll
        for (uint32_t p = 0; p < PER; ++p) {
            const uint32_t i = threadIdx.x + NT * p;
            if (i >= N) continue;
            const uint64_t g = v[p];
            if constexpr (HALF) {
                const uint4 h = make_uint4(grid_pair_h(g, 0), grid_pair_h(g, 1), grid_pair_h(g, 2), grid_pair_h(g, 3));
                if constexpr (KIND == 16) lds_iq2xxs_grid_h()[i] = h;
                else if constexpr (KIND == 17) lds_iq2xs_grid_h()[i] = h;
                else if constexpr (KIND == 22) lds_iq2s_grid_h()[i] = h;
                else if constexpr (KIND == 21) lds_iq3s_grid_h()[i] = make_uint2(h.x, h.y);
            } else {
                if constexpr (KIND == 16) lds_iq2xxs_grid()[i] = g;
                else if constexpr (KIND == 17) lds_iq2xs_grid()[i] = g;
                else if constexpr (KIND == 18) lds_iq3xxs_grid()[i] = (uint32_t)g;
                else if constexpr (KIND == 20 || KIND == 23) lds_iq4nl_values()[i] = (float)(int8_t)(uint8_t)g;
                else if constexpr (KIND == 21) lds_iq3s_grid()[i] = (uint32_t)g;
                else if constexpr (KIND == 22) lds_iq2s_grid()[i] = g;
                else if constexpr (KIND == 29) lds_iq1s_grid()[i] = g;
            }
        }
        if constexpr (HALF && (KIND == 16 || KIND == 17)) {
            for (uint32_t i = threadIdx.x; i < 128u; i += NT) lds_iq3_signmask()[i] = sign_mask8(ingot_ksign(i));
        } else if constexpr (HALF && (KIND == 21 || KIND == 22)) {
            for (uint32_t i = threadIdx.x; i < 256u; i += NT) lds_sign8mask()[i] = sign_mask8(i);
        }
    }
};

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

struct Contig {
    __device__ static uint32_t col(uint32_t c, uint32_t i) { return 32u * c + i; }
    __device__ static void load_x(const float* x, uint32_t c, float* xv) {
        const float4* p = reinterpret_cast<const float4*>(x + 32u * c);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 a = p[i];
            xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
        }
    }
};

// ------------------------------------------------------------------- F32 (0)
template <>
struct Fmt<0> : Contig {
    static constexpr uint32_t BLOCK = 1, BYTES = 4;
    struct Raw {
        float4 v[8];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        Raw r;
        const float4* p = reinterpret_cast<const float4*>(row + 128u * c);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = p[i];
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w[4 * i] = r.v[i].x; w[4 * i + 1] = r.v[i].y; w[4 * i + 2] = r.v[i].z; w[4 * i + 3] = r.v[i].w;
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float, float) {
        float w[32];
        dequant_raw(r, c, w);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s = __builtin_fmaf(w[i], xv[i], s);
        return s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// ------------------------------------------------------------------ Q8_0 (8)
template <>
struct Fmt<8> : Contig {
    static constexpr uint32_t BLOCK = 32, BYTES = 34;
    struct Raw {
        uint32_t d;
        uint32_t q[8];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + c * BYTES;
        Raw r;
        r.d = ld_u16(b);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.q[i] = ld_u32_a2(b + 2 + 4 * i);
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        float d = half_bits_to_float(r.d);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) w[4 * i + j] = d * sbyte_f(r.q[i], j);
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) s = __builtin_fmaf(sbyte_f(r.q[i], j), xv[4 * i + j], s);
        return half_bits_to_float(r.d) * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// ------------------------------------------------- Q4_0 (2) and IQ4_NL (20)
// 18-byte blocks: fp16 d, 16 bytes of nibbles; value i < 16 is the low nibble
// of byte i, value i >= 16 the high nibble of byte i - 16.
template <bool NL>
struct Nibble32 : Contig {
    static constexpr uint32_t BLOCK = 32, BYTES = 18;
    struct Raw {
        uint32_t d;
        uint32_t q[4];
    };
    __device__ static float value(uint32_t nib) {
        if constexpr (NL) return lds_iq4nl_values()[nib];
        else return (float)((int)nib - 8);
    }
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + c * BYTES;
        Raw r;
        r.d = ld_u16(b);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = ld_u32_a2(b + 2 + 4 * i);
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        float d = half_bits_to_float(r.d);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t byte = byte_of(r.q[i], j);
                w[4 * i + j] = d * value(byte & 15u);
                w[16 + 4 * i + j] = d * value(byte >> 4);
            }
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t byte = byte_of(r.q[i], j);
                s = __builtin_fmaf(value(byte & 15u), xv[4 * i + j], s);
                s = __builtin_fmaf(value(byte >> 4), xv[16 + 4 * i + j], s);
            }
        return half_bits_to_float(r.d) * s;
    }
};
template <>
struct Fmt<2> : Nibble32<false> {};
template <>
struct Fmt<20> : Nibble32<true> {};

// --------------------------------------------------------------- IQ2_XS (17)
// 74-byte superblocks (2-byte aligned): fp16 d @0, 32 u16 codes @2 (9-bit grid
// index | 7-bit sign index << 9, one per 8 values), 8 scale bytes @66 (4 bits
// per 16 values). w = d * (0.5 + s) * 0.25 * grid * sign.
template <>
struct Fmt<17> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 74;
    struct Raw {
        uint32_t d, scale;
        uint32_t code[4];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        uint32_t g = c & 7u;
        Raw r;
        r.d = ld_u16(b);
        r.scale = b[66 + g];
#pragma unroll
        for (int l = 0; l < 4; ++l) r.code[l] = ld_u16(b + 2 + 8 * g + 2 * l);
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        float d = half_bits_to_float(r.d);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            float db = d * (0.5f + (float)((r.scale >> (4 * (l / 2))) & 15u)) * 0.25f;
            uint64_t grid = lds_iq2xs_grid()[r.code[l] & 511u];
            uint32_t sg = ingot_ksign(r.code[l] >> 9);
#pragma unroll
            for (int v = 0; v < 8; ++v)
                w[8 * l + v] = flip_sign(db * (float)((grid >> (8 * v)) & 255u), (sg >> v) & 1u);
        }
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
    // The same sum with the inputs as f16 pairs: xh[q] holds values 2q, 2q+1
    // (hi), xl[q] their remainders times 2^11; the signed grid values are f16
    // numbers (sign masks XORed in), so every v_dot2 product is exact.
    __device__ static float dot_raw_h(const Raw& r, const uint32_t* xh, const uint32_t* xl) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint4 g = lds_iq2xs_grid_h()[r.code[l] & 511u];
            const uint4 m = lds_iq3_signmask()[(r.code[l] >> 9) & 127u];
            const uint32_t gs[4] = {g.x ^ m.x, g.y ^ m.y, g.z ^ m.z, g.w ^ m.w};
            float th = 0.f, tl = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                th = dot2_f16(gs[q], xh[4 * l + q], th);
                tl = dot2_f16(gs[q], xl[4 * l + q], tl);
            }
            const float t = __builtin_fmaf(tl, 1.0f / 2048.0f, th);
            s = __builtin_fmaf(0.5f + (float)((r.scale >> (4 * (l / 2))) & 15u), t, s);
        }
        return half_bits_to_float(r.d) * 0.25f * s;
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            uint64_t grid = lds_iq2xs_grid()[r.code[l] & 511u];
            uint32_t sg = ingot_ksign(r.code[l] >> 9);
            float t = 0.f;
#pragma unroll
            for (int v = 0; v < 8; ++v)
                t = __builtin_fmaf((float)((grid >> (8 * v)) & 255u), flip_sign(xv[8 * l + v], (sg >> v) & 1u), t);
            s = __builtin_fmaf(0.5f + (float)((r.scale >> (4 * (l / 2))) & 15u), t, s);
        }
        return half_bits_to_float(r.d) * 0.25f * s;
    }
};

// -------------------------------------------------------------- IQ3_XXS (18)
// 98-byte superblocks (2-byte aligned): fp16 d @0, 64 grid bytes @2 (one
// 4-value codebook entry each), 8 u32 @66 (four 7-bit sign indices and a
// 4-bit scale in bits 28..31 per 32 values). w = d * (0.5 + s) * 0.5 * grid * sign.
template <>
struct Fmt<18> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 98;
    struct Raw {
        uint32_t d, aux;
        uint32_t gb[4];  // 8 grid bytes, two per u16 word
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        uint32_t g = c & 7u;
        Raw r;
        r.d = ld_u16(b);
        r.aux = ld_u32_a2(b + 66 + 4 * g);
#pragma unroll
        for (int l = 0; l < 4; ++l) r.gb[l] = ld_u16(b + 2 + 8 * g + 2 * l);
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        float db = half_bits_to_float(r.d) * (0.5f + (float)(r.aux >> 28)) * 0.5f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            uint32_t sg = ingot_ksign((r.aux >> (7 * l)) & 127u);
            uint32_t lo = lds_iq3xxs_grid()[r.gb[l] & 255u], hi = lds_iq3xxs_grid()[r.gb[l] >> 8];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                w[8 * l + v] = flip_sign(db * ubyte_f(lo, v), (sg >> v) & 1u);
                w[8 * l + 4 + v] = flip_sign(db * ubyte_f(hi, v), (sg >> (4 + v)) & 1u);
            }
        }
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            uint32_t sg = ingot_ksign((r.aux >> (7 * l)) & 127u);
            uint32_t lo = lds_iq3xxs_grid()[r.gb[l] & 255u], hi = lds_iq3xxs_grid()[r.gb[l] >> 8];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                s = __builtin_fmaf(ubyte_f(lo, v), flip_sign(xv[8 * l + v], (sg >> v) & 1u), s);
                s = __builtin_fmaf(ubyte_f(hi, v), flip_sign(xv[8 * l + 4 + v], (sg >> (4 + v)) & 1u), s);
            }
        }
        return half_bits_to_float(r.d) * (0.5f + (float)(r.aux >> 28)) * 0.5f * s;
    }
};

// ------------------------------------------------------ F16 (1), BF16 (30)
// Two bytes per value; chunk c is bytes 64c..64c+63 of the row.
template <bool BF>
struct Half16 : Contig {
    static constexpr uint32_t BLOCK = 1, BYTES = 2;
    struct Raw {
        uint4 v[4];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        Raw r;
        const uint4* p = reinterpret_cast<const uint4*>(row + 64u * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = p[i];
        return r;
    }
    // Value 2j + h of the 32-bit word w.
    __device__ static float val(uint32_t w, int h) {
        if constexpr (BF) return __uint_as_float(h ? (w & 0xffff0000u) : (w << 16));
        else return half_bits_to_float(h ? (w >> 16) : w);
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w[8 * i + 2 * j] = val(q[j], 0);
                w[8 * i + 2 * j + 1] = val(q[j], 1);
            }
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = __builtin_fmaf(val(q[j], 0), xv[8 * i + 2 * j], s);
                s = __builtin_fmaf(val(q[j], 1), xv[8 * i + 2 * j + 1], s);
            }
        }
        return s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};
template <>
struct Fmt<1> : Half16<false> {};
template <>
struct Fmt<30> : Half16<true> {};

// -------------------------------------------------------------- Q2_0 (42)
// 18-byte blocks of 64 values (2-byte aligned): fp16 d @0, 16 bytes of 2-bit
// codes @2, value k in bits 2(k%4) of byte k/4. w = d * (code - 1).
// Chunk c is half c%2 of block c/2.
template <>
struct Fmt<42> : Contig {
    static constexpr uint32_t BLOCK = 64, BYTES = 18;
    struct Raw {
        uint32_t d;
        uint32_t q[2];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 1) * BYTES;
        Raw r;
        r.d = ld_u16(b);
        r.q[0] = ld_u32_a2(b + 2 + 8 * (c & 1u));
        r.q[1] = ld_u32_a2(b + 6 + 8 * (c & 1u));
        return r;
    }
    __device__ static float code(const Raw& r, int i) { return (float)((r.q[i >> 4] >> (2 * (i & 15))) & 3u); }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = d * (code(r, i) - 1.0f);
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float xs0, float xs1) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s = __builtin_fmaf(code(r, i), xv[i], s);
        return half_bits_to_float(r.d) * (s - (xs0 + xs1));
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// --------------------------------------------------------------- Q2_K (10)
// 84-byte superblocks: 16 scale bytes @0 (scale low nibble, min high nibble,
// per 16 values), 64 bytes of 2-bit quants @16, fp16 d @80 and dmin @82.
// Value k: quant bits 2((k%128)/32) of byte 16 + 32(k/128) + k%32.
// w = d * (sc & 15) * q - dmin * (sc >> 4). Chunk c: group g = c%8 of
// superblock c/8, i.e. bytes 16 + 32(g/4) .. +32 at shift 2(g%4).
template <>
struct Fmt<10> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 84;
    struct Raw {
        uint32_t dd, sc;
        uint32_t q[8];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u;
        Raw r;
        r.dd = ld_u32_a2(b + 80);
        r.sc = ld_u16(b + 2 * g);
        const uint8_t* q = b + 16 + 32 * (g >> 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.q[i] = ld_u32_a2(q + 4 * i);
        return r;
    }
    __device__ static uint32_t qword(const Raw& r, uint32_t c, int i) { return (r.q[i] >> (2 * (c & 3u))) & 0x03030303u; }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        const float d = half_bits_to_float(r.dd), dm = half_bits_to_float(r.dd >> 16);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t sc = (r.sc >> (8 * h)) & 255u;
            const float ds = d * (float)(sc & 15u), m = dm * (float)(sc >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = qword(r, c, 4 * h + i);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[16 * h + 4 * i + j] = ds * ubyte_f(q, j) - m;
            }
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float xs0, float xs1) {
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = qword(r, c, 4 * h + i);
#pragma unroll
                for (int j = 0; j < 4; ++j) s[h] = __builtin_fmaf(ubyte_f(q, j), xv[16 * h + 4 * i + j], s[h]);
            }
        const float d = half_bits_to_float(r.dd), dm = half_bits_to_float(r.dd >> 16);
        const uint32_t s0 = r.sc & 255u, s1 = (r.sc >> 8) & 255u;
        return d * ((float)(s0 & 15u) * s[0] + (float)(s1 & 15u) * s[1]) -
               dm * ((float)(s0 >> 4) * xs0 + (float)(s1 >> 4) * xs1);
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// --------------------------------------------------------------- Q5_K (13)
// 176-byte superblocks: Q4_K's 16-byte header {d, dmin, scales[12]} @0, 32
// bytes of fifth bits @16 (bit g of byte k%32 for value k of group g), 128
// bytes of nibbles @48 laid out as Q4_K's. Chunks follow Q4_K's (16 nibble
// bytes, both nibbles), so the fifth bits are bits 2qq and 2qq+1 of the 16
// bytes @16 + 16h. w = d*sc*q - dmin*m, q = nibble | bit << 4.
template <>
struct Fmt<13> : Fmt<12> {
    static constexpr uint32_t BYTES = 176;
    struct Raw {
        uint4 a, b, h;
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t q = c & 7u;
        Raw r;
        r.a = *reinterpret_cast<const uint4*>(b);
        r.b = *reinterpret_cast<const uint4*>(b + 48 + 32 * (q >> 1) + 16 * (q & 1u));
        r.h = *reinterpret_cast<const uint4*>(b + 16 + 16 * (q & 1u));
        return r;
    }
    // Bytes 4k..4k+3 of the low (h = 0) or high (h = 1) group as 5-bit values.
    __device__ static uint32_t q5(const Raw& r, uint32_t c, int k, int h) {
        const uint32_t w[4] = {r.b.x, r.b.y, r.b.z, r.b.w}, hb[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
        const uint32_t bit = 2u * ((c & 7u) >> 1) + (uint32_t)h;
        return ((w[k] >> (4 * h)) & 0x0f0f0f0fu) | (((hb[k] >> bit) & 0x01010101u) << 4);
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        float d0, m0, d1, m1;
        scales(r.a, c, d0, m0, d1, m1);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = q5(r, c, k, 0), hi = q5(r, c, k, 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w[4 * k + j] = d0 * ubyte_f(lo, j) - m0;
                w[16 + 4 * k + j] = d1 * ubyte_f(hi, j) - m1;
            }
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float xs0, float xs1) {
        float d0, m0, d1, m1;
        scales(r.a, c, d0, m0, d1, m1);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = q5(r, c, k, 0), hi = q5(r, c, k, 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                slo = __builtin_fmaf(ubyte_f(lo, j), xv[4 * k + j], slo);
                shi = __builtin_fmaf(ubyte_f(hi, j), xv[16 + 4 * k + j], shi);
            }
        }
        return d0 * slo + d1 * shi - (m0 * xs0 + m1 * xs1);
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float xs0, float xs1) {
        return dot_raw(load_raw(row, c), c, xv, xs0, xs1);
    }
};

// --------------------------------------------------------------- Q6_K (14)
// 210-byte superblocks (2-byte aligned): 128 bytes of low nibbles @0, 64
// bytes of high 2-bit pairs @128, 16 int8 scales @192 (per 16 values), fp16
// d @208. Value k (n = k/128, l = k%32, t = (k%128)/32): low nibble
// (t >= 2: high half) of byte 64n + 32(t%2) + l, high bits 2t of byte
// 128 + 32n + l, scale 192 + 8n + 2t + l/16. w = d * scale * (q - 32).
template <>
struct Fmt<14> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 210;
    struct Raw {
        uint32_t d, sc;
        uint32_t ql[8], qh[8];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u, n = g >> 2, t = g & 3u;
        Raw r;
        r.d = ld_u16(b + 208);
        r.sc = ld_u16(b + 192 + 8 * n + 2 * t);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            r.ql[i] = ld_u32_a2(b + 64 * n + 32 * (t & 1u) + 4 * i);
            r.qh[i] = ld_u32_a2(b + 128 + 32 * n + 4 * i);
        }
        return r;
    }
    __device__ static uint32_t q6(const Raw& r, uint32_t c, int i) {
        const uint32_t t = c & 3u;
        return ((r.ql[i] >> (t >= 2u ? 4 : 0)) & 0x0f0f0f0fu) | (((r.qh[i] >> (2 * t)) & 0x03030303u) << 4);
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float ds = d * (float)(int8_t)((r.sc >> (8 * h)) & 255u);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = q6(r, c, 4 * h + i);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[16 * h + 4 * i + j] = ds * (ubyte_f(q, j) - 32.0f);
            }
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float xs0, float xs1) {
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = q6(r, c, 4 * h + i);
#pragma unroll
                for (int j = 0; j < 4; ++j) s[h] = __builtin_fmaf(ubyte_f(q, j), xv[16 * h + 4 * i + j], s[h]);
            }
        const float sc0 = (float)(int8_t)(r.sc & 255u), sc1 = (float)(int8_t)((r.sc >> 8) & 255u);
        return half_bits_to_float(r.d) *
               (sc0 * __builtin_fmaf(-32.0f, xs0, s[0]) + sc1 * __builtin_fmaf(-32.0f, xs1, s[1]));
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// ------------------------------------------------------------ IQ2_XXS (16)
// 66-byte superblocks (2-byte aligned): fp16 d @0, then per group of 32
// values 8 bytes @2 + 8g: four 8-value grid indices and a u32 holding four
// 7-bit sign indices (bits 7l) and a 4-bit scale (bits 28..31).
// w = d * (0.5 + s) * 0.25 * grid * sign.
template <>
struct Fmt<16> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 66;
    struct Raw {
        uint32_t d, idx, aux;
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* a = row + (c >> 3) * BYTES + 2 + 8 * (c & 7u);
        Raw r;
        r.d = ld_u16(a - 2 - 8 * (c & 7u));
        r.idx = ld_u32_a2(a);
        r.aux = ld_u32_a2(a + 4);
        return r;
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        const float db = half_bits_to_float(r.d) * (0.5f + (float)(r.aux >> 28)) * 0.25f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t grid = lds_iq2xxs_grid()[byte_of(r.idx, l)];
            const uint32_t sg = ingot_ksign((r.aux >> (7 * l)) & 127u);
#pragma unroll
            for (int v = 0; v < 8; ++v) w[8 * l + v] = flip_sign(db * (float)((grid >> (8 * v)) & 255u), (sg >> v) & 1u);
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t grid = lds_iq2xxs_grid()[byte_of(r.idx, l)];
            const uint32_t sg = ingot_ksign((r.aux >> (7 * l)) & 127u);
#pragma unroll
            for (int v = 0; v < 8; ++v)
                s = __builtin_fmaf((float)((grid >> (8 * v)) & 255u), flip_sign(xv[8 * l + v], (sg >> v) & 1u), s);
        }
        return half_bits_to_float(r.d) * (0.5f + (float)(r.aux >> 28)) * 0.25f * s;
    }
    // As Fmt<17>::dot_raw_h: f16 grid values with the sign masks XORed in,
    // inputs as f16 hi pairs and remainders times 2^11.
    __device__ static float dot_raw_h(const Raw& r, const uint32_t* xh, const uint32_t* xl) {
        float th = 0.f, tl = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint4 g = lds_iq2xxs_grid_h()[byte_of(r.idx, l)];
            const uint4 m = lds_iq3_signmask()[(r.aux >> (7 * l)) & 127u];
            const uint32_t gs[4] = {g.x ^ m.x, g.y ^ m.y, g.z ^ m.z, g.w ^ m.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                th = dot2_f16(gs[q], xh[4 * l + q], th);
                tl = dot2_f16(gs[q], xl[4 * l + q], tl);
            }
        }
        const float s = __builtin_fmaf(tl, 1.0f / 2048.0f, th);
        return half_bits_to_float(r.d) * (0.5f + (float)(r.aux >> 28)) * 0.25f * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// -------------------------------------------------------------- IQ2_S (22)
// 82-byte superblocks (2-byte aligned): fp16 d @0, grid index low bytes @2
// (4 per group), sign bytes @34 (4 per group, one bit per value), index high
// bits @66 (one byte per group, 2 bits per 8 values), scales @74 (one byte
// per group, 4 bits per 16 values). w = d * (0.5 + s) * 0.25 * grid * sign.
template <>
struct Fmt<22> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 82;
    struct Raw {
        uint32_t d, idx, sgn, hs;  // hs: high-bits byte | scale byte << 8
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u;
        Raw r;
        r.d = ld_u16(b);
        r.idx = ld_u32_a2(b + 2 + 4 * g);
        r.sgn = ld_u32_a2(b + 34 + 4 * g);
        r.hs = (uint32_t)b[66 + g] | ((uint32_t)b[74 + g] << 8);
        return r;
    }
    __device__ static uint64_t grid(const Raw& r, int l) {
        return lds_iq2s_grid()[byte_of(r.idx, l) | (((r.hs & 255u) << (8 - 2 * l)) & 0x300u)];
    }
    __device__ static float scale(const Raw& r, int l) { return 0.5f + (float)((r.hs >> (8 + 4 * (l / 2))) & 15u); }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const float db = d * scale(r, l) * 0.25f;
            const uint64_t gr = grid(r, l);
            const uint32_t sg = byte_of(r.sgn, l);
#pragma unroll
            for (int v = 0; v < 8; ++v) w[8 * l + v] = flip_sign(db * (float)((gr >> (8 * v)) & 255u), (sg >> v) & 1u);
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint64_t gr = grid(r, l);
            const uint32_t sg = byte_of(r.sgn, l);
            float t = 0.f;
#pragma unroll
            for (int v = 0; v < 8; ++v)
                t = __builtin_fmaf((float)((gr >> (8 * v)) & 255u), flip_sign(xv[8 * l + v], (sg >> v) & 1u), t);
            s = __builtin_fmaf(scale(r, l), t, s);
        }
        return half_bits_to_float(r.d) * 0.25f * s;
    }
    __device__ static float dot_raw_h(const Raw& r, const uint32_t* xh, const uint32_t* xl) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint4 g = lds_iq2s_grid_h()[byte_of(r.idx, l) | (((r.hs & 255u) << (8 - 2 * l)) & 0x300u)];
            const uint4 m = lds_sign8mask()[byte_of(r.sgn, l)];
            const uint32_t gs[4] = {g.x ^ m.x, g.y ^ m.y, g.z ^ m.z, g.w ^ m.w};
            float th = 0.f, tl = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                th = dot2_f16(gs[q], xh[4 * l + q], th);
                tl = dot2_f16(gs[q], xl[4 * l + q], tl);
            }
            s = __builtin_fmaf(scale(r, l), __builtin_fmaf(tl, 1.0f / 2048.0f, th), s);
        }
        return half_bits_to_float(r.d) * 0.25f * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// -------------------------------------------------------------- IQ3_S (21)
// 110-byte superblocks (2-byte aligned): fp16 d @0, 64 grid index low bytes
// @2 (8 per group, 4 values each), index ninth bits @66 (one byte per group),
// sign bytes @74 (4 per group), scales @106 (4 bits per group).
// w = d * (1 + 2s) * grid * sign.
template <>
struct Fmt<21> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 110;
    struct Raw {
        uint32_t d, q0, q1, sgn, hs;  // hs: ninth-bits byte | scale << 8
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u;
        Raw r;
        r.d = ld_u16(b);
        r.q0 = ld_u32_a2(b + 2 + 8 * g);
        r.q1 = ld_u32_a2(b + 6 + 8 * g);
        r.sgn = ld_u32_a2(b + 74 + 4 * g);
        r.hs = (uint32_t)b[66 + g] | ((((uint32_t)b[106 + g / 2] >> (4 * (g & 1u))) & 15u) << 8);
        return r;
    }
    // Codebook index of grid entry j (0..7) of the group (4 values each).
    __device__ static uint32_t grid_index(const Raw& r, int j) {
        return byte_of(j < 4 ? r.q0 : r.q1, j & 3) | (((r.hs & 255u) << (8 - j)) & 256u);
    }
    __device__ static uint32_t grid(const Raw& r, int j) { return lds_iq3s_grid()[grid_index(r, j)]; }
    __device__ static void dequant_raw(const Raw& r, uint32_t, float* w) {
        const float db = half_bits_to_float(r.d) * (float)(1u + 2u * (r.hs >> 8));
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t sg = byte_of(r.sgn, l);
#pragma unroll
            for (int hg = 0; hg < 2; ++hg) {
                const uint32_t gr = grid(r, 2 * l + hg);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    w[8 * l + 4 * hg + v] = flip_sign(db * ubyte_f(gr, v), (sg >> (4 * hg + v)) & 1u);
            }
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t sg = byte_of(r.sgn, l);
#pragma unroll
            for (int hg = 0; hg < 2; ++hg) {
                const uint32_t gr = grid(r, 2 * l + hg);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    s = __builtin_fmaf(ubyte_f(gr, v), flip_sign(xv[8 * l + 4 * hg + v], (sg >> (4 * hg + v)) & 1u), s);
            }
        }
        return half_bits_to_float(r.d) * (float)(1u + 2u * (r.hs >> 8)) * s;
    }
    __device__ static float dot_raw_h(const Raw& r, const uint32_t* xh, const uint32_t* xl) {
        float th = 0.f, tl = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint4 m = lds_sign8mask()[byte_of(r.sgn, l)];
            const uint2 g0 = lds_iq3s_grid_h()[grid_index(r, 2 * l)], g1 = lds_iq3s_grid_h()[grid_index(r, 2 * l + 1)];
            const uint32_t gs[4] = {g0.x ^ m.x, g0.y ^ m.y, g1.x ^ m.z, g1.y ^ m.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                th = dot2_f16(gs[q], xh[4 * l + q], th);
                tl = dot2_f16(gs[q], xl[4 * l + q], tl);
            }
        }
        const float s = __builtin_fmaf(tl, 1.0f / 2048.0f, th);
        return half_bits_to_float(r.d) * (float)(1u + 2u * (r.hs >> 8)) * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// ------------------------------------------------------------- IQ4_XS (23)
// 136-byte superblocks (8-byte aligned): fp16 d @0, u16 of 2-bit scale high
// parts @2, 4 bytes of 4-bit scale low parts @4, 128 nibble bytes @8 (16 per
// group: values 0-15 low nibbles, 16-31 high nibbles, as IQ4_NL).
// w = d * (scale - 32) * kvalues_iq4nl[q].
template <>
struct Fmt<23> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 136;
    struct Raw {
        uint32_t h0, h1;  // d | scales_h << 16, scales_l
        uint32_t q[4];
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u;
        const uint2 h = *reinterpret_cast<const uint2*>(b);
        const uint2 q0 = *reinterpret_cast<const uint2*>(b + 8 + 16 * g);
        const uint2 q1 = *reinterpret_cast<const uint2*>(b + 16 + 16 * g);
        Raw r;
        r.h0 = h.x;
        r.h1 = h.y;
        r.q[0] = q0.x; r.q[1] = q0.y; r.q[2] = q1.x; r.q[3] = q1.y;
        return r;
    }
    __device__ static float scale(const Raw& r, uint32_t c) {
        const uint32_t g = c & 7u;
        const uint32_t lo = (byte_of(r.h1, g >> 1) >> (4 * (g & 1u))) & 15u, hi = ((r.h0 >> 16) >> (2 * g)) & 3u;
        return (float)((int)(lo | (hi << 4)) - 32);
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        const float ds = half_bits_to_float(r.h0) * scale(r, c);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t byte = byte_of(r.q[i], j);
                w[4 * i + j] = ds * lds_iq4nl_values()[byte & 15u];
                w[16 + 4 * i + j] = ds * lds_iq4nl_values()[byte >> 4];
            }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t byte = byte_of(r.q[i], j);
                s = __builtin_fmaf(lds_iq4nl_values()[byte & 15u], xv[4 * i + j], s);
                s = __builtin_fmaf(lds_iq4nl_values()[byte >> 4], xv[16 + 4 * i + j], s);
            }
        return half_bits_to_float(r.h0) * scale(r, c) * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// -------------------------------------------------------------- IQ1_M (29)
// 56-byte superblocks (8-byte aligned): 32 grid index low bytes @0 (4 per
// group), 16 bytes @32 (per 8 values: 3 index high bits and a delta sign
// bit, two per byte), four u16 @48 holding 3-bit scales (per 16 values) and,
// in their top nibbles, the fp16 d. w = d * (2s + 1) * (grid + delta),
// grid in {-1, 0, 1}, delta = -1/8 when the bit is set, else +1/8.
template <>
struct Fmt<29> : Contig {
    static constexpr uint32_t BLOCK = 256, BYTES = 56;
    struct Raw {
        uint32_t qs, qh, sc0, sc1;
    };
    __device__ static Raw load_raw(const uint8_t* row, uint32_t c) {
        const uint8_t* b = row + (c >> 3) * BYTES;
        const uint32_t g = c & 7u;
        const uint2 s = *reinterpret_cast<const uint2*>(b + 48);
        Raw r;
        r.qs = *reinterpret_cast<const uint32_t*>(b + 4 * g);
        r.qh = ld_u16(b + 32 + 2 * g);
        r.sc0 = s.x;
        r.sc1 = s.y;
        return r;
    }
    __device__ static float d(const Raw& r) {
        const uint32_t bits = ((r.sc0 >> 12) & 0xfu) | ((r.sc0 >> 24) & 0xf0u) | ((r.sc1 >> 4) & 0xf00u) |
                              ((r.sc1 >> 16) & 0xf000u);
        return half_bits_to_float(bits);
    }
    // Scale factor 2s + 1 of sub-block l (0..3) of chunk c.
    __device__ static float scale(const Raw& r, uint32_t c, int l) {
        const uint32_t g = c & 7u;
        const uint32_t w = ((g >> 1) < 2u ? r.sc0 : r.sc1) >> (16 * ((g >> 1) & 1u));
        return (float)(2u * ((w >> (6 * (g & 1u) + 3 * (l / 2))) & 7u) + 1u);
    }
    __device__ static uint64_t grid(const Raw& r, int l, float& delta) {
        const uint32_t hb = (r.qh >> (8 * (l / 2) + 4 * (l % 2))) & 15u;
        delta = (hb & 8u) ? -0.125f : 0.125f;
        return lds_iq1s_grid()[byte_of(r.qs, l) | ((hb & 7u) << 8)];
    }
    __device__ static void dequant_raw(const Raw& r, uint32_t c, float* w) {
        const float dd = d(r);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            float delta;
            const uint64_t gr = grid(r, l, delta);
            const float ds = dd * scale(r, c, l);
#pragma unroll
            for (int v = 0; v < 8; ++v) w[8 * l + v] = ds * ((float)(int8_t)((gr >> (8 * v)) & 255u) + delta);
        }
    }
    __device__ static float dot_raw(const Raw& r, uint32_t c, const float* xv, float, float) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            float delta;
            const uint64_t gr = grid(r, l, delta);
            float t = 0.f, sx = 0.f;
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                t = __builtin_fmaf((float)(int8_t)((gr >> (8 * v)) & 255u), xv[8 * l + v], t);
                sx += xv[8 * l + v];
            }
            s = __builtin_fmaf(scale(r, c, l), __builtin_fmaf(delta, sx, t), s);
        }
        return d(r) * s;
    }
    __device__ static float dot(const uint8_t* row, uint32_t c, const float* xv, float a, float b) {
        return dot_raw(load_raw(row, c), c, xv, a, b);
    }
};

// Scalar decode of weight j of a row, any supported kind (slow path for the
// generic projection / dequant drop-ins).
__device__ inline float dequant_value(const uint8_t* row, uint32_t kind, uint32_t j) {
    switch (kind) {
        case 0: return reinterpret_cast<const float*>(row)[j];
        case 1: return half_bits_to_float(ld_u16(row + 2 * j));
        case 2: {
            const uint8_t* b = row + (j / 32) * 18;
            uint32_t k = j % 32;
            return half_bits_to_float(ld_u16(b)) * (float)((int)((b[2 + k % 16] >> (4 * (k / 16))) & 15) - 8);
        }
        case 8: {
            const uint8_t* b = row + (j / 32) * 34;
            return half_bits_to_float(ld_u16(b)) * (float)(int8_t)b[2 + j % 32];
        }
        case 20: {
            const uint8_t* b = row + (j / 32) * 18;
            uint32_t k = j % 32;
            return half_bits_to_float(ld_u16(b)) * (float)ingot_kvalues_iq4nl[(b[2 + k % 16] >> (4 * (k / 16))) & 15];
        }
        case 12: {
            const uint8_t* b = row + (j / 256) * 144;
            uint32_t k = j % 256, g = k / 32, sc, m;
            const uint8_t* s = b + 4;
            if (g < 4) {
                sc = s[g] & 63;
                m = s[g + 4] & 63;
            } else {
                sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
                m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
            }
            uint32_t q = (b[16 + 32 * (k / 64) + k % 32] >> (4 * (g % 2))) & 15;
            float d1 = half_bits_to_float(ld_u16(b)) * (float)sc, m1 = half_bits_to_float(ld_u16(b + 2)) * (float)m;
            return d1 * (float)q - m1;
        }
        case 17: {
            const uint8_t* b = row + (j / 256) * 74;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t q = ld_u16(b + 2 + 2 * (4 * g + l));
            float grid = (float)((ingot_iq2xs_grid[q & 511] >> (8 * v)) & 255);
            float db = half_bits_to_float(ld_u16(b)) * (0.5f + (float)((b[66 + g] >> (4 * (l / 2))) & 15)) * 0.25f;
            return flip_sign(db * grid, (ingot_ksign(q >> 9) >> v) & 1u);
        }
        case 18: {
            const uint8_t* b = row + (j / 256) * 98;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t aux = ld_u32_a2(b + 66 + 4 * g);
            float grid = (float)((ingot_iq3xxs_grid[b[2 + 8 * g + 2 * l + v / 4]] >> (8 * (v % 4))) & 255);
            float db = half_bits_to_float(ld_u16(b)) * (0.5f + (float)(aux >> 28)) * 0.5f;
            return flip_sign(db * grid, (ingot_ksign((aux >> (7 * l)) & 127) >> v) & 1u);
        }
        case 30: return __uint_as_float((uint32_t)ld_u16(row + 2 * j) << 16);
        case 13: {
            const uint8_t* b = row + (j / 256) * 176;
            uint32_t k = j % 256, g = k / 32, sc, m;
            const uint8_t* s = b + 4;
            if (g < 4) {
                sc = s[g] & 63;
                m = s[g + 4] & 63;
            } else {
                sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
                m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
            }
            uint32_t q = ((b[48 + 32 * (k / 64) + k % 32] >> (4 * (g % 2))) & 15) | (((b[16 + k % 32] >> g) & 1u) << 4);
            float d1 = half_bits_to_float(ld_u16(b)) * (float)sc, m1 = half_bits_to_float(ld_u16(b + 2)) * (float)m;
            return d1 * (float)q - m1;
        }
        case 10: {
            const uint8_t* b = row + (j / 256) * 84;
            uint32_t k = j % 256, sc = b[k / 16];
            uint32_t q = (b[16 + (k / 128) * 32 + k % 32] >> (2 * ((k % 128) / 32))) & 3;
            return half_bits_to_float(ld_u16(b + 80)) * (float)(sc & 15) * (float)q -
                   half_bits_to_float(ld_u16(b + 82)) * (float)(sc >> 4);
        }
        case 14: {
            const uint8_t* b = row + (j / 256) * 210;
            uint32_t k = j % 256, n = k / 128, l = k % 32, t = (k % 128) / 32;
            uint32_t low = (b[n * 64 + l + (t % 2) * 32] >> (t >= 2 ? 4 : 0)) & 15;
            uint32_t high = (b[128 + n * 32 + l] >> (2 * t)) & 3;
            return half_bits_to_float(ld_u16(b + 208)) * (float)(int8_t)b[192 + n * 8 + l / 16 + 2 * t] *
                   (float)((int)(low | (high << 4)) - 32);
        }
        case 16: {
            const uint8_t* b = row + (j / 256) * 66;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            const uint8_t* a = b + 2 + g * 8;
            uint32_t aux = ld_u32_a2(a + 4);
            float grid = (float)((ingot_iq2xxs_grid[a[l]] >> (8 * v)) & 255);
            float db = half_bits_to_float(ld_u16(b)) * (0.5f + (float)(aux >> 28)) * 0.25f;
            return flip_sign(db * grid, (ingot_ksign((aux >> (7 * l)) & 127) >> v) & 1u);
        }
        case 29: {
            const uint8_t* b = row + (j / 256) * 56;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t sc[4];
            for (int i = 0; i < 4; ++i) sc[i] = ld_u16(b + 48 + 2 * i);
            uint32_t bits = (sc[0] >> 12) | ((sc[1] >> 8) & 240) | ((sc[2] >> 4) & 3840) | (sc[3] & 61440);
            uint32_t high = b[32 + g * 2 + l / 2];
            uint32_t index = b[g * 4 + l] | (((high >> (4 * (l % 2))) & 7) << 8);
            float delta = (high & (8u << (4 * (l % 2)))) ? -0.125f : 0.125f;
            float grid = (float)(int8_t)((ingot_iq1s_grid[index] >> (8 * v)) & 255);
            uint32_t scale = (sc[g / 2] >> (6 * (g % 2) + 3 * (l / 2))) & 7;
            return half_bits_to_float(bits) * (float)(2 * scale + 1) * (grid + delta);
        }
        case 42: {
            const uint8_t* b = row + (j / 64) * 18;
            uint32_t k = j % 64;
            return half_bits_to_float(ld_u16(b)) * (float)((int)((b[2 + k / 4] >> (2 * (k % 4))) & 3) - 1);
        }
        case 22: {
            const uint8_t* b = row + (j / 256) * 82;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t index = b[2 + 4 * g + l] | (((uint32_t)b[66 + g] << (8 - 2 * l)) & 0x300);
            float grid = (float)((ingot_iq2s_grid[index] >> (8 * v)) & 255);
            float db = half_bits_to_float(ld_u16(b)) * (0.5f + (float)((b[74 + g] >> (4 * (l / 2))) & 15)) * 0.25f;
            return flip_sign(db * grid, (b[34 + 4 * g + l] >> v) & 1u);
        }
        case 21: {
            const uint8_t* b = row + (j / 256) * 110;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8, hg = v / 4;
            uint32_t index = b[2 + g * 8 + 2 * l + hg] | (((uint32_t)b[66 + g] << (8 - 2 * l - hg)) & 256);
            float grid = (float)((ingot_iq3s_grid[index] >> (8 * (v % 4))) & 255);
            float db = half_bits_to_float(ld_u16(b)) * (float)(1 + 2 * ((b[106 + g / 2] >> (4 * (g % 2))) & 15));
            return flip_sign(db * grid, (b[74 + g * 4 + l] >> v) & 1u);
        }
        case 23: {
            const uint8_t* b = row + (j / 256) * 136;
            uint32_t k = j % 256, g = k / 32, v = k % 32;
            uint32_t high = ld_u16(b + 2);
            int scale = (int)(((b[4 + g / 2] >> (4 * (g % 2))) & 15) | (((high >> (2 * g)) & 3) << 4)) - 32;
            uint32_t q = (b[8 + g * 16 + v % 16] >> (4 * (v / 16))) & 15;
            return half_bits_to_float(ld_u16(b)) * (float)scale * (float)ingot_kvalues_iq4nl[q];
        }
        default: return __builtin_nanf("");
    }
}

}  // namespace ingot
