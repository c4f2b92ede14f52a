// HIP kernels of the MoE-layer hot path for gfx950 (wave64, MFMA, 160 KB LDS).
//
// Decode (few pairs) and prefill (many pairs) take different kernels:
//   router   k_router        logits = W_r x (fixed fp32 order), optional fused
//                            RMSNorm, optional shared-expert gate logit
//   route    k_route         per-token top-K, one wave per token (wave_route);
//                            softmax or sigmoid+bias weights
//   decode   k_dec_gate_up2  each wave selects its pair's expert (wave_kth, or
//                            wave_route for two pairs per wave), then act[p] =
//                            w_k SwiGLU(G_e x_t, U_e x_t), one wave per pair;
//                            above 128 experts it also requests the down rows
//                            k_dec_down will read
//            k_gemv_gate_up  the same for the shared expert (no routing)
//            k_dec_down      out[t] = sum_k D_e act[p] (+ shared, + residual)
//   prefill  k_dispatch      stable expert grouping, tile list (one block)
//            (its other blocks split x into f16 hi + lo for k_gemm_f16)
//            k_gemm_f16      f16-MFMA grouped GEMM on integer weight operands
//                            (Q4_K, Q5_K, Q6_K, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S,
//                            IQ4_NL, IQ4_XS), A split into f16 hi + lo
//            k_gemm<GATEUP>  MFMA f32 grouped GEMM, dequantised weights in LDS
//                            (every other format)
//            k_combine       out[t] = sum_k w_k Y[inverse[p]] (+ shared, + residual)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "det_math.h"
#include "formats.cuh"

namespace ingot {

constexpr int WAVE = 64;
constexpr uint32_t FLAG_NONFINITE = 1u;  // a router logit or bias
// An operand of the split-f16 arithmetic left the range in which it is exact
// (see ACT_EXP_C); the outputs of the forwards since the last check are not
// valid, and the fp32 GEMM must be used for these inputs.
constexpr uint32_t FLAG_RANGE = 2u;
// A kernel that writes a layer output (k_dec_down, k_gemv_shared_down_add,
// k_combine) wrote a non-finite value; the reference rejects such an output
// on read-back (src/metal.rs:1575-1577).
constexpr uint32_t FLAG_OUT_NONFINITE = 4u;

// ------------------------------------------- f16-split operand scaling
// Every operand that is split into f16 hi + lo (x for the f16 GEMM and the
// v_dot2 decode formats, the prefill activations, the decode activations of
// the v_dot2 formats) is first multiplied by an exact power of two, so that
// neither half overflows and the lo half stays out of the f16 subnormals for
// every value within 2^13 of the largest.
//   * x: per token, max|x_t| 2^e_t in [2^10, 2^11) (x_exp of the token's
//     maximum, which the router stores). Its 32-column sums are then below
//     2^16 and enter the Q4_K mins MFMA divided by 32.
//   * decode activations (k_dec_down): per token, the same rule on the
//     block's maximum.
//   * prefill activations: the gate/up epilogue unscales g and u by 2^-e_t
//     before the SwiGLU and stores act 2^a_t, a_t = act_exp(xstat[t]) =
//     2 n_t + ACT_EXP_C with n_t = x_exp(||x_t||_2). g and u are products of
//     weight rows with x, of the order of |w| ||x_t||_2 whatever the shape of
//     x (one large component or many small ones), and the SwiGLU of the two
//     of the order of their product, so this puts a row's values near 2^5 for
//     weights of the usual size (N(0, 0.02) at H = 2048) whatever the scale of
//     x. Its validity is checked, not assumed: the epilogue keeps each row's
//     max |act| (rowmax), and the down GEMM raises FLAG_RANGE unless it is
//     zero or in [ACT_RANGE_LO, ACT_RANGE_HI) (below, products of the lo half
//     lose bits; above, the group sums could overflow). The combine multiplies
//     the routed sum by 2^-a_t.
// xstat[t] = {max |x_t|, ||x_t 2^e_t||_2} (the router writes it).
constexpr int ACT_EXP_C = -7;
constexpr float ACT_RANGE_HI = 16384.f;  // 2^14
constexpr float ACT_RANGE_LO = 0.125f;   // 2^-3

// e with m 2^e in [2^10, 2^11) for finite m > 0; 0 for zero or non-finite m.
__device__ __forceinline__ int x_exp(float m) {
    if (!(m > 0.f) || !isfinite(m)) return 0;
    int k;
    (void)frexpf(m, &k);  // m = f 2^k, f in [0.5, 1)
    return 11 - k;
}
// Units exponent of a token's prefill activations (above), from its xstat.
__device__ __forceinline__ int act_exp(float2 st) { return 2 * (x_exp(st.y) + x_exp(st.x)) + ACT_EXP_C; }
__device__ __forceinline__ float2 ld_xstat(const float* xstat, uint32_t t) {
    return reinterpret_cast<const float2*>(xstat)[t];
}
__device__ __forceinline__ float4 ldexp4(float4 a, int e) {
    return make_float4(ldexpf(a.x, e), ldexpf(a.y, e), ldexpf(a.z, e), ldexpf(a.w, e));
}
__device__ __forceinline__ float max_abs4(float4 a) {
    return fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
}

// The xor butterfly v_l <- v_l + v_(l xor m), m = 32, 16, ..., 1: the router's
// fixed reduction tree (det_math.h). Each partner value is fetched by an exact
// lane permutation: m = 32 through the LDS crossbar, m = 16 by ds_swizzle
// (bitmask mode, xor 16 within 32 lanes), m = 8 by DPP row_ror:8 ((l + 8) mod 16
// = l xor 8 in either rotate direction), m = 4 by DPP quad_perm [3,2,1,0]
// (l xor 3) followed by row_half_mirror (l xor 7), m = 2 and 1 by quad_perm.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = v + __shfl_xor(v, 32);
    v = v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
    v = v + dpp_mov<0x128>(v);
    v = v + dpp_mov<0x141>(dpp_mov<0x1b>(v));
    v = v + dpp_mov<0x4e>(v);
    v = v + dpp_mov<0xb1>(v);
    return v;
}

// Wave sum through DPP (no LDS crossbar): quad xor 1 and xor 2, half-row and
// row mirrors give every lane its 16-lane row sum; the four row sums are read
// with readlane. Fixed order, so deterministic; it is not the router's order
// (the router keeps wave_sum, whose tree the CPU replays).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0xb1>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    v = dpp_add<0x140>(v);  // row_mirror
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}
// Wave maximum of non-negative values (same DPP pattern).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<0xb1>(v));
    v = fmaxf(v, dpp_mov<0x4e>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ float swiglu(float g, float u, float limit) {
    if (limit > 0.f) {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
    }
    // SiLU through the hardware exp2 (__expf) and reciprocal (v_rcp_f32): about
    // 1e-6 relative, against the layer's 1e-4 bar; the accurate expf and IEEE
    // division cost the f16 GEMM's epilogue about 20 more instructions per
    // element. exp(-g) = inf for g < -88 gives g * 0 = -0, as g / inf does.
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// ------------------------------------------------------------ wave routing
// Orders one wave's LDS accesses around a point (lanes exchange data through
// LDS; a wave's LDS instructions execute in issue order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-wave LDS scratch of wave_route: 64 candidate slots x (key, id, weight
// input), then the same for 64 junk slots (one per lane) that lanes without a
// candidate write instead. Kernels that route use at most ROUTE_MAX_WAVES
// waves per block (12: the one-token decode blocks at 512 experts).
constexpr uint32_t ROUTE_MAX_WAVES = 12;
__device__ inline uint32_t* route_lds() {
    __shared__ __align__(16) uint32_t r[ROUTE_MAX_WAVES][6 * 64];
    return r[threadIdx.x >> 6];
}

// Selection keys of one token in one wave, E <= 64 * NE, the whole wave
// active (src/lib.rs:43-60, kernels/glm.metal:81-98). Candidate j of a lane is
// expert e = lane + 64 j with selection key s = logit (+ bias) (softmax) or
// sigmoid(logit) (+ bias) (sigmoid routing), and weight input wv = s
// (softmax) or sigmoid(logit). Keys compare in IEEE total order
// (f32::total_cmp) as uint32 through ingot_orderable; an absent candidate
// (e >= E) has key 0. Selection order: higher key first, equal keys toward
// the lower id. Returns whether this lane saw a non-finite logit or bias.
template <int NE>
__device__ __forceinline__ bool route_keys(const float* __restrict__ l, const float* __restrict__ bias, uint32_t E,
                                  uint32_t sigmoid_mode, uint32_t (&key)[NE], float (&wv)[NE], bool (&ok)[NE]) {
    INGOT_NO_CONTRACT
    const uint32_t lane = threadIdx.x & 63u;
    // All loads first, unconditional (index clamped), so they are in flight
    // together; absent candidates are masked afterwards.
    float lv[NE], bv[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) lv[j] = l[min(lane + 64u * j, E - 1u)];
    if (bias) {
#pragma unroll
        for (int j = 0; j < NE; ++j) bv[j] = bias[min(lane + 64u * j, E - 1u)];
    }
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        ok[j] = lane + 64u * j < E;
        const float v = lv[j];
        const float b = bias ? bv[j] : 0.f;
        bad |= ok[j] && (!isfinite(v) || !isfinite(b));
        float sk;
        if (sigmoid_mode) {
            wv[j] = ingot_det_sigmoid(v);
            sk = bias ? wv[j] + b : wv[j];
        } else {
            sk = bias ? v + b : v;
            wv[j] = sk;
        }
        key[j] = ok[j] ? ingot_orderable(sk) : 0u;
        wv[j] = ok[j] ? wv[j] : 0.f;
    }
    return bad;
}

// Threshold for the n highest keys (1 <= n <= E), from the top bits down,
// keeping at least n keys >= T (ballot counts, no data movement). Stops with
// exact = true as soon as exactly n keys are >= T; otherwise T ends at the
// n-th highest key value. Absent candidates (key 0) are never counted for a
// threshold above 0. With at most 4 keys per lane, two bits per step: the
// counts at T | v << s for v = 1, 2, 3 are independent ballots, and T takes
// the highest v whose count is still >= n (the counts fall as v grows), so
// the chain of dependent ballot -> count -> T steps is 16 long instead of 32
// (1.3k instead of 2.5k cycles per wave for one key per lane). Both forms
// give the same T when they end without an exact stop, and the same set of
// keys >= T when they stop at exactly n.
template <int NE>
__device__ __forceinline__ uint32_t route_threshold(const uint32_t (&key)[NE], uint32_t n, bool& exact) {
    uint32_t T = 0;
    exact = false;
    if constexpr (NE <= 4) {
#pragma unroll
        for (int s = 30; s >= 0; s -= 2) {
            uint32_t vs = 0, cs = 0;
#pragma unroll
            for (uint32_t v = 1; v < 4u; ++v) {
                const uint32_t c = T | (v << s);
                uint32_t cnt = 0;
#pragma unroll
                for (int j = 0; j < NE; ++j) cnt += (uint32_t)__popcll(__ballot(key[j] >= c));
                if (cnt >= n) {
                    vs = v;
                    cs = cnt;
                }
            }
            T |= vs << s;
            if (cs == n) {
                exact = true;
                break;
            }
        }
        return T;
    }
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = T | (1u << bit);
        uint32_t cnt = 0;
#pragma unroll
        for (int j = 0; j < NE; ++j) cnt += (uint32_t)__popcll(__ballot(key[j] >= c));
        if (cnt >= n) {
            T = c;
            if (cnt == n) {
                exact = true;
                break;
            }
        }
    }
    return T;
}

// Top-K selection of one token by one wave (route_keys order):
//   1. candidates, a superset of the top K of at most 64 keys: with several
//      keys per lane (NE > 1), every key >= M, M the K-th highest of the
//      lanes' maxima (the K lanes with the highest maxima hold K keys >= M, so
//      the K-th highest key is >= M and so is every key of the top K; finding
//      M takes ballots over one key per lane instead of NE). Otherwise (one key per lane,
//      or more than 64 keys >= M, as when many keys are equal) exactly the top
//      K: T = route_threshold(K); the K keys >= T when exact, else the keys
//      above T, then keys equal to T by ascending id until there are K;
//   2. the C candidates are compacted in id order into LDS, lane m < C takes
//      candidate m, reads all C keys (LDS broadcast) and counts those that
//      precede it (higher key, or equal key and lower id: an earlier
//      position), and a candidate of rank < K sends its id and weight input
//      to lane rank (ds_permute).
// Every key that precedes a candidate is itself a candidate, so these ranks
// are the ranks among all keys. Lane k < K ends with selection k's id and
// weight input. Returns whether this lane saw a non-finite logit or bias.
// wave_route_compact: step 1 and the compaction of step 2 (C candidates in
// the wave's LDS scratch, in id order: key r[m], id r[64 + m], weight input
// r[128 + m]); wave_route_rank: the ranks and the placement. The caller may
// issue loads between them (wave_route_compact ends with the scratch
// visible to the whole wave).
template <int NE>
__device__ __forceinline__ bool wave_route_compact(const float* __restrict__ l, const float* __restrict__ bias, uint32_t E,
                                                   uint32_t K, uint32_t sigmoid_mode, uint32_t& C_out) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t key[NE];
    float wv[NE];
    bool ok[NE];
    const bool bad = route_keys<NE>(l, bias, E, sigmoid_mode, key, wv, ok);
    uint64_t sel[NE];
    uint32_t C = 0;  // candidates (0: not formed yet)
    if constexpr (NE > 1) {
        uint32_t mk[1] = {key[0]};
#pragma unroll
        for (int j = 1; j < NE; ++j) mk[0] = max(mk[0], key[j]);
        bool ex1;
        const uint32_t M = route_threshold<1>(mk, K, ex1);
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            sel[j] = __ballot(ok[j] && key[j] >= M);
            C += (uint32_t)__popcll(sel[j]);
        }
        if (C > 64u) C = 0;
    }
    if (C == 0) {
    C = K;
    bool exact;
    const uint32_t T = route_threshold<NE>(key, K, exact);
    if (exact) {  // T > 0: absent candidates excluded
#pragma unroll
        for (int j = 0; j < NE; ++j) sel[j] = __ballot(key[j] >= T);
    } else {
        // K <= E: at least K - (keys above T) present candidates equal T.
        uint32_t need = K;
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            sel[j] = __ballot(ok[j] && key[j] > T);
            need -= (uint32_t)__popcll(sel[j]);
        }
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            uint64_t eq = __ballot(ok[j] && key[j] == T);
            while (need != 0u && eq != 0ull) {
                const uint64_t low = eq & (~eq + 1ull);
                sel[j] |= low;
                eq ^= low;
                --need;
            }
        }
    }
    }
    // 2. compaction in id order (slot j, then lane), ranking, placement. C <=
    // 64 (the candidates were formed so), so every position is below 64; a
    // lane without a candidate in slot j writes its junk slot (192 + lane), so
    // the writes need no branch.
    uint32_t* r = route_lds();
    uint32_t before = 0;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const uint32_t pos = before + __builtin_amdgcn_mbcnt_hi((uint32_t)(sel[j] >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)sel[j], 0u));
        const uint32_t at = ((sel[j] >> lane) & 1ull) ? (pos & 63u) : 192u + lane;
        r[at] = key[j];
        r[64 + at] = lane + 64u * j;
        r[128 + at] = __float_as_uint(wv[j]);
        before += (uint32_t)__popcll(sel[j]);
    }
    wave_sync();
    C_out = C;
    return bad;
}
// rank: this lane's candidate's rank (lane < C).
__device__ __forceinline__ void wave_route_rank(uint32_t C, uint32_t E, uint32_t K, uint32_t& my_id, float& my_v,
                                                uint32_t& rank) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t* r = route_lds();
    const bool cand = lane < C;
    const uint32_t ck = cand ? r[lane] : 0u, cid = cand ? r[64 + lane] : 0u;
    const float cv = cand ? __uint_as_float(r[128 + lane]) : 0.f;
    // Rank: the candidates that precede this one, sixteen per step (four
    // broadcast reads issued together; slots past C are masked); key and
    // position compare as one 64-bit value (key, 63 - position).
    // (slots past C read as key 0 through a uniform mask: candidate keys are
    // >= 1, so they never precede a candidate)
    const uint64_t mine = ((uint64_t)ck << 32) | (63u - lane);
    rank = 0;
    for (uint32_t m = 0; m < C; m += 16) {  // m <= 48: reads stay in r[0, 64)
        uint4 k4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) k4[q] = *reinterpret_cast<const uint4*>(r + m + 4u * q);
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) {
            const uint4 v = k4[q / 4];
            const uint32_t p = m + q, live = p < C ? 0xffffffffu : 0u;
            const uint32_t km = (q % 4 == 0 ? v.x : q % 4 == 1 ? v.y : q % 4 == 2 ? v.z : v.w) & live;
            rank += ((((uint64_t)km << 32) | (63u - p)) > mine) ? 1u : 0u;
        }
    }
    // Placement: candidate of rank k < K sends its id and weight input to lane
    // k (ds_permute: a forward permute through the LDS crossbar); the others
    // send to lane 63, unread when K < 64 (K = 64 makes every lane a candidate
    // of a distinct rank).
    const uint32_t dst = (cand && rank < K) ? rank : 63u;
    const uint32_t pid = (uint32_t)__builtin_amdgcn_ds_permute((int)(dst << 2), (int)cid);
    const uint32_t pv = (uint32_t)__builtin_amdgcn_ds_permute((int)(dst << 2), (int)__float_as_uint(cv));
    const bool sel_k = lane < K;
    my_id = sel_k ? min(pid, E - 1u) : 0u;  // (always below E: a guard for the weight addresses)
    my_v = sel_k ? __uint_as_float(pv) : 0.f;
    wave_sync();  // the scratch is reused by the next call
}
template <int NE>
__device__ __forceinline__ bool wave_route(const float* __restrict__ l, const float* __restrict__ bias, uint32_t E, uint32_t K,
                                  uint32_t sigmoid_mode, uint32_t& my_id, float& my_v) {
    uint32_t C, rank;
    const bool bad = wave_route_compact<NE>(l, bias, E, K, sigmoid_mode, C);
    wave_route_rank(C, E, K, my_id, my_v, rank);
    return bad;
}

// Routing weight of selection k held by lane k < K (wave_route's my_v):
// softmax over the K selected logits, max-subtracted, summed in selection
// order (src/lib.rs:53-58); sigmoid routing: score / sum of the selected
// scores * scale (kernels/glm.metal:93-97).
__device__ inline float wave_route_weight(float my_v, uint32_t K, uint32_t sigmoid_mode, float scale) {
    INGOT_NO_CONTRACT
    const float top = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), 0));
    const float num = sigmoid_mode ? my_v : ingot_det_expf(my_v - top);
    float total = 0.f;
    for (uint32_t k = 0; k < K; ++k) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), (int)k));
    return sigmoid_mode ? num / total * scale : num / total;
}

// Selection k (0-based, k < K <= E) of one token alone, from the keys of
// route_keys: the (k+1)-th highest key, equal keys toward the lower id.
// Returns its expert id (wave-uniform); wv_k receives its weight input.
//   exact threshold: exactly k+1 keys are >= T, so selection k is the lowest
//   of them, and among equal lowest keys the one with the highest id;
//   otherwise T is the (k+1)-th key value: with g keys above T, selection k
//   is the (k+1-g)-th lowest id among the keys equal to T.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)0xffffffff, (int)v, 0xb1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)0xffffffff, (int)v, 0x4e, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)0xffffffff, (int)v, 0x141, 0xf, 0xf, false)); // row_half_mirror
    v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)0xffffffff, (int)v, 0x140, 0xf, 0xf, false)); // row_mirror
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return min(min(a, b), min(c, d));
}

template <int NE>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&key)[NE], const float (&wv)[NE], const bool (&ok)[NE],
                                    uint32_t k, float& wv_k) {
    bool exact;
    const uint32_t T = route_threshold<NE>(key, k + 1u, exact);
    uint32_t id = 0;
    if (exact) {
        uint32_t lo = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < NE; ++j) lo = min(lo, key[j] >= T ? key[j] : 0xffffffffu);
        lo = wave_min_u32(lo);
        bool found = false;
#pragma unroll
        for (int j = NE - 1; j >= 0; --j) {
            const uint64_t bj = __ballot(key[j] == lo);
            if (!found && bj) {
                id = 64u * j + 63u - (uint32_t)__builtin_clzll(bj);
                found = true;
            }
        }
    } else {
        uint32_t need = k + 1u;
#pragma unroll
        for (int j = 0; j < NE; ++j) need -= (uint32_t)__popcll(__ballot(ok[j] && key[j] > T));
        bool found = false;
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            uint64_t eq = __ballot(ok[j] && key[j] == T);
            const uint32_t n = (uint32_t)__popcll(eq);
            if (!found) {
                if (need <= n) {
                    for (uint32_t q = 1; q < need; ++q) eq &= eq - 1ull;
                    id = 64u * j + (uint32_t)__builtin_ctzll(eq);
                    found = true;
                } else {
                    need -= n;
                }
            }
        }
    }
    // The owner's candidates are read slot by slot and then selected, so the
    // candidate array is never indexed by a run-time value (that would put it
    // in memory).
    const uint32_t owner = id & 63u, slot = id >> 6;
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const float rj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv[j]), (int)owner));
        mine = (uint32_t)j == slot ? rj : mine;
    }
    wv_k = mine;
    return id;
}


// ---------------------------------------------------------------- router
// Residual add ahead of the norm (the reference's add_rms, kernels/generic.metal:
// 390-405): the rows s = x + a replace the wave's inputs, and the writing wave
// stores s, the layer's new residual stream, to xs.
template <int NT, int HB>
__device__ __forceinline__ void add_residual(float (&xr)[NT][HB * 4], const float* __restrict__ a,
                                             float* __restrict__ xs, uint32_t t0, uint32_t T, uint32_t lane,
                                             bool write) {
    constexpr uint32_t H = 256u * HB;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t tt = min(t0 + t, T - 1);
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(a + (uint64_t)tt * H + 4u * lane + 256u * i);
            xr[t][4 * i] += v.x; xr[t][4 * i + 1] += v.y; xr[t][4 * i + 2] += v.z; xr[t][4 * i + 3] += v.w;
        }
        if (write && t0 + t < T) {
#pragma unroll
            for (int i = 0; i < HB; ++i)
                *reinterpret_cast<float4*>(xs + (uint64_t)(t0 + t) * H + 4u * lane + 256u * i) =
                    make_float4(xr[t][4 * i], xr[t][4 * i + 1], xr[t][4 * i + 2], xr[t][4 * i + 3]);
        }
    }
}

// xstat[t] = {max |x_t|, ||x_t 2^e_t||_2} (e_t = x_exp(max)) of one token held
// by a wave as the router holds it (HB * 4 values per lane); lane 0 stores.
template <int HB>
__device__ __forceinline__ void token_stats(const float (&xr)[HB * 4], float* __restrict__ xstat, uint32_t t,
                                            uint32_t T, uint32_t lane) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < HB * 4; ++j) m = fmaxf(m, fabsf(xr[j]));
    m = wave_max(m);
    const int e = x_exp(m);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < HB * 4; ++j) {
        const float v = ldexpf(xr[j], e);
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0 && t < T) reinterpret_cast<float2*>(xstat)[t] = make_float2(m, sqrtf(ss));
}

// One wave per (group of TOK tokens, group of experts). Lane l holds the
// columns 4l + 256i + c (i < HB = H/256, c < 4) of each of its tokens, which
// is the slot layout of the fixed reduction order (det_math.h): each logit is
// the lane's fused multiply-add chain followed by the xor butterfly, so it is
// bit-identical to the CPU's ingot_router_partial + ingot_butterfly64.
// With a norm gain the wave first computes RMSNorm of its tokens in the same
// order (sum of squares over the slots, butterfly, 1/sqrt(ss/H + eps), (x*r)*g)
// and writes the normalised rows (block (.., 0), wave 0 only). With an
// addend a the rows are x + a first (add_residual), stored to xs.
// Expert index E (when sgvec != NULL) is the shared-expert gate vector: its
// product goes to sgl[t]. xstat[t] receives {max |x_t|, ||x_t 2^e_t||_2} of the
// expert input (after the residual add and the norm; e_t = x_exp(max)),
// written by wave 0 of the by == 0 blocks: the scales of the f16 splits.
template <int TOK, int HB>
__global__ __launch_bounds__(256) void k_router(const float* __restrict__ x, const float* __restrict__ addend,
                                                const float* __restrict__ W, const float* __restrict__ sgvec,
                                                const float* __restrict__ gain, float eps, uint32_t T, uint32_t E,
                                                uint32_t epw, float* __restrict__ logits, float* __restrict__ sgl,
                                                float* __restrict__ xn, float* __restrict__ xs,
                                                float* __restrict__ xstat) {
    INGOT_NO_CONTRACT
    constexpr uint32_t H = 256u * HB;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * TOK;
    // Decode (one token per block): the wave's first router row is loaded
    // before the input, independent of it, so the two loads (and the optional
    // RMSNorm) overlap.
    const uint32_t rows = E + (sgvec ? 1u : 0u);
    const uint32_t e0 = (blockIdx.y * (blockDim.x >> 6) + wave) * epw;
    float wv0[TOK == 1 ? HB * 4 : 1];
    if constexpr (TOK == 1) {
        const float* wr = e0 < E ? W + (uint64_t)e0 * H : (e0 < rows ? sgvec : W);
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(wr + 4u * lane + 256u * i);
            wv0[4 * i] = v.x; wv0[4 * i + 1] = v.y; wv0[4 * i + 2] = v.z; wv0[4 * i + 3] = v.w;
        }
    }
    float xr[TOK][HB * 4];
#pragma unroll
    for (int t = 0; t < TOK; ++t) {
        uint32_t tt = min(t0 + t, T - 1);
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            float4 v = *reinterpret_cast<const float4*>(x + (uint64_t)tt * H + 4u * lane + 256u * i);
            xr[t][4 * i] = v.x; xr[t][4 * i + 1] = v.y; xr[t][4 * i + 2] = v.z; xr[t][4 * i + 3] = v.w;
        }
    }
    if (addend) add_residual<TOK, HB>(xr, addend, xs, t0, T, lane, blockIdx.y == 0 && wave == 0);
    if (gain) {
        float g[HB * 4];
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            float4 v = *reinterpret_cast<const float4*>(gain + 4u * lane + 256u * i);
            g[4 * i] = v.x; g[4 * i + 1] = v.y; g[4 * i + 2] = v.z; g[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) ss = __builtin_fmaf(xr[t][j], xr[t][j], ss);
            ss = wave_sum(ss);
            float mean = ss / (float)H;
            float r = 1.0f / sqrtf(mean + eps);
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) xr[t][j] = (xr[t][j] * r) * g[j];
        }
        if (blockIdx.y == 0 && wave == 0) {
#pragma unroll
            for (int t = 0; t < TOK; ++t) {
                if (t0 + t >= T) break;
#pragma unroll
                for (int i = 0; i < HB; ++i)
                    *reinterpret_cast<float4*>(xn + (uint64_t)(t0 + t) * H + 4u * lane + 256u * i) =
                        make_float4(xr[t][4 * i], xr[t][4 * i + 1], xr[t][4 * i + 2], xr[t][4 * i + 3]);
            }
        }
    }
    if (xstat && blockIdx.y == 0 && wave == 0) {
#pragma unroll
        for (int t = 0; t < TOK; ++t) token_stats<HB>(xr[t], xstat, t0 + t, T, lane);
    }
    for (uint32_t k = 0; k < epw; ++k) {
        uint32_t e = e0 + k;
        if (e >= rows) break;
        const float* wr = e < E ? W + (uint64_t)e * H : sgvec;
        float wv[HB * 4];
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            if (TOK == 1 && k == 0) {
                wv[4 * i] = wv0[TOK == 1 ? 4 * i : 0];
                wv[4 * i + 1] = wv0[TOK == 1 ? 4 * i + 1 : 0];
                wv[4 * i + 2] = wv0[TOK == 1 ? 4 * i + 2 : 0];
                wv[4 * i + 3] = wv0[TOK == 1 ? 4 * i + 3 : 0];
            } else {
                float4 v = *reinterpret_cast<const float4*>(wr + 4u * lane + 256u * i);
                wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
            }
        }
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) acc = __builtin_fmaf(wv[j], xr[t][j], acc);
            acc = wave_sum(acc);
            if (lane == 0 && t0 + t < T) {
                if (e < E) logits[(uint64_t)(t0 + t) * E + e] = acc;
                else sgl[t0 + t] = acc;
            }
        }
    }
}

// Transposed xor butterfly over 64 sums at once: each lane holds v[0..63]
// (its partial of 64 independent sums); lane l returns the full sum of output
// l. At step m (32, 16, ..., 1) a lane keeps the half of its remaining outputs
// selected by bit m of its lane index and adds the partner's (lane xor m)
// partials of that half. Every partial sum is formed from the same two
// operands as in wave_sum (fp addition is commutative), so each output equals
// wave_sum of that output bit for bit.
template <int M>
__device__ __forceinline__ float xor_partner(float v) {
    if constexpr (M == 32) return __shfl_xor(v, 32);
    else if constexpr (M == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
    else if constexpr (M == 8) return dpp_mov<0x128>(v);
    else if constexpr (M == 4) return dpp_mov<0x141>(dpp_mov<0x1b>(v));
    else if constexpr (M == 2) return dpp_mov<0x4e>(v);
    else return dpp_mov<0xb1>(v);
}
template <int C, int M>
__device__ __forceinline__ void transpose_step(float* v, bool hi) {
#pragma unroll
    for (int i = 0; i < C / 2; ++i) {
        const float a = v[i], b = v[i + C / 2];
        const float keep = hi ? b : a, send = hi ? a : b;
        v[i] = keep + xor_partner<M>(send);
    }
}
// 32 sums: five transposed steps leave output ((l >> 1) & 31) in lane l, and
// the last step (m = 1) adds the partner's partial of the same output.
__device__ __forceinline__ float transpose_sum32(float (&v)[32], uint32_t lane) {
    transpose_step<32, 32>(v, lane & 32u);
    transpose_step<16, 16>(v, lane & 16u);
    transpose_step<8, 8>(v, lane & 8u);
    transpose_step<4, 4>(v, lane & 4u);
    transpose_step<2, 2>(v, lane & 2u);
    return v[0] + xor_partner<1>(v[0]);
}
__device__ __forceinline__ float transpose_sum64(float (&v)[64], uint32_t lane) {
    transpose_step<64, 32>(v, lane & 32u);
    transpose_step<32, 16>(v, lane & 16u);
    transpose_step<16, 8>(v, lane & 8u);
    transpose_step<8, 4>(v, lane & 4u);
    transpose_step<4, 2>(v, lane & 2u);
    transpose_step<2, 1>(v, lane & 1u);
    return v[0];
}

// Prefill router: grid (ceil(T / (4 TPW)), E / EB), 256 threads, TPW tokens
// per wave and EB experts per block, TPW EB = 32 or 64 (the launcher takes
// TPW = 4: each router value read from LDS feeds four FMAs; EB = 16, or 8 when
// 16 would leave fewer than two blocks per CU). Wave w of block (bx, by)
// computes the logits of tokens 4 TPW bx + TPW w .. + TPW - 1 for experts
// EB by .. + EB - 1: lane l keeps the fixed-order FMA chain of its columns
// 4 l + 256 i + c (as k_router) for each of the TPW EB (token, expert) pairs,
// and one transposed butterfly leaves pair i = TPW EB == 64 ? l : l / 2,
// (t, e) = (i / EB, i % EB), in lane l.
// The block's router rows pass through LDS in double-buffered chunks of 4.
// The residual add (addend: s written to xs by the by == 0 blocks), RMSNorm
// (gain: written to xn by the by == 0 blocks) and the shared-expert gate logit
// (sgvec: by == 0 blocks, wave_sum) and the per-token input statistics (xstat:
// by == 0 blocks) are computed as in k_router.
template <int HB, int EB, int TPW>
__global__ __launch_bounds__(256) void k_router_t(const float* __restrict__ x, const float* __restrict__ addend,
                                                  const float* __restrict__ W, const float* __restrict__ sgvec,
                                                  const float* __restrict__ gain, float eps, uint32_t T, uint32_t E,
                                                  float* __restrict__ logits, float* __restrict__ sgl,
                                                  float* __restrict__ xn, float* __restrict__ xs,
                                                  float* __restrict__ xstat) {
    INGOT_NO_CONTRACT
    constexpr uint32_t H = 256u * HB, Q = H / 4u;  // Q float4 per row
    constexpr int CH = 4;                         // router rows per LDS chunk
    __shared__ float4 sw[2][CH][Q];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, tid = threadIdx.x;
    constexpr uint32_t NC = EB / CH;  // chunks
    const uint32_t t0 = blockIdx.x * (4u * TPW) + TPW * wave, e0 = blockIdx.y * (uint32_t)EB;
    float xr[TPW][HB * 4];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const uint32_t tt = min(t0 + t, T - 1);
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(x + (uint64_t)tt * H + 4u * lane + 256u * i);
            xr[t][4 * i] = v.x; xr[t][4 * i + 1] = v.y; xr[t][4 * i + 2] = v.z; xr[t][4 * i + 3] = v.w;
        }
    }
    if (addend) add_residual<TPW, HB>(xr, addend, xs, t0, T, lane, blockIdx.y == 0);
    if (gain) {
        float g[HB * 4];
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(gain + 4u * lane + 256u * i);
            g[4 * i] = v.x; g[4 * i + 1] = v.y; g[4 * i + 2] = v.z; g[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) ss = __builtin_fmaf(xr[t][j], xr[t][j], ss);
            ss = wave_sum(ss);
            const float mean = ss / (float)H;
            const float r = 1.0f / sqrtf(mean + eps);
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) xr[t][j] = (xr[t][j] * r) * g[j];
            if (blockIdx.y == 0 && t0 + t < T) {
#pragma unroll
                for (int i = 0; i < HB; ++i)
                    *reinterpret_cast<float4*>(xn + (uint64_t)(t0 + t) * H + 4u * lane + 256u * i) =
                        make_float4(xr[t][4 * i], xr[t][4 * i + 1], xr[t][4 * i + 2], xr[t][4 * i + 3]);
            }
        }
    }
    if (sgvec && blockIdx.y == 0) {
        float wv[HB * 4];
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(sgvec + 4u * lane + 256u * i);
            wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < HB * 4; ++j) acc = __builtin_fmaf(wv[j], xr[t][j], acc);
            acc = wave_sum(acc);
            if (lane == 0 && t0 + t < T) sgl[t0 + t] = acc;
        }
    }
    if (xstat && blockIdx.y == 0) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) token_stats<HB>(xr[t], xstat, t0 + t, T, lane);
    }
    // Router rows e0 .. e0 + EB - 1 in NC chunks of 4 through LDS.
    constexpr uint32_t PER = CH * Q / 256u;  // float4 per thread per chunk
    float4 stage[PER];
    float p[TPW * EB];
#pragma unroll
    for (int i = 0; i < TPW * EB; ++i) p[i] = 0.f;
#pragma unroll
    for (uint32_t k = 0; k < PER; ++k) {
        const uint32_t idx = tid + 256u * k;
        sw[0][idx / Q][idx % Q] = reinterpret_cast<const float4*>(W + (uint64_t)(e0 + idx / Q) * H)[idx % Q];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t c = 0; c < NC; ++c) {
        if (c + 1 < NC) {
#pragma unroll
            for (uint32_t k = 0; k < PER; ++k) {
                const uint32_t idx = tid + 256u * k;
                stage[k] = reinterpret_cast<const float4*>(W + (uint64_t)(e0 + CH * (c + 1) + idx / Q) * H)[idx % Q];
            }
        }
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            float wv[HB * 4];
#pragma unroll
            for (int i = 0; i < HB; ++i) {
                const float4 v = sw[c & 1u][r][lane + 64u * i];
                wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < HB * 4; ++j) acc = __builtin_fmaf(wv[j], xr[t][j], acc);
                p[t * EB + CH * c + r] = acc;
            }
        }
        if (c + 1 < NC) {
#pragma unroll
            for (uint32_t k = 0; k < PER; ++k) {
                const uint32_t idx = tid + 256u * k;
                sw[(c + 1) & 1u][idx / Q][idx % Q] = stage[k];
            }
            __syncthreads();
        }
    }
    static_assert(TPW * EB == 32 || TPW * EB == 64, "32 or 64 logits per wave");
    if constexpr (TPW * EB == 64) {
        const float v = transpose_sum64(p, lane);
        const uint32_t t = t0 + lane / EB, e = e0 + lane % EB;
        if (t < T) logits[(uint64_t)t * E + e] = v;
    } else {
        const float v = transpose_sum32(p, lane);
        const uint32_t t = t0 + (lane >> 1) / EB, e = e0 + (lane >> 1) % EB;
        if (t < T && (lane & 1u) == 0) logits[(uint64_t)t * E + e] = v;
    }
}

// ----------------------------------------------------------------- route
// One wave per token (wave_route, wave_route_weight), E <= 64 * NE. Softmax
// mode (src/lib.rs:43-60): selection and weights on l (+ bias when given),
// w_k = exp(v_k - v_top) / sum. Sigmoid mode (kernels/glm.metal:81-98):
// selection on sigmoid(l) + bias, w_k = sigmoid(l_k) / sum * scale. A
// non-finite logit or bias raises FLAG_NONFINITE; the ids written are still
// valid expert indices. K <= 64.
template <int NE>
__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits, const float* __restrict__ bias,
                                               uint32_t T, uint32_t E, uint32_t K, uint32_t sigmoid_mode,
                                               float scale, uint32_t* __restrict__ ids, float* __restrict__ wts,
                                               uint32_t* __restrict__ flags) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (t >= T) return;  // whole waves
    uint32_t my_id;
    float my_v;
    const bool bad = wave_route<NE>(logits + (uint64_t)t * E, bias, E, K, sigmoid_mode, my_id, my_v);
    if (__any(bad) && lane == 0) atomicOr(flags, FLAG_NONFINITE);
    const float w = wave_route_weight(my_v, K, sigmoid_mode, scale);
    if (lane < K) {
        ids[(uint64_t)t * K + lane] = my_id;
        wts[(uint64_t)t * K + lane] = w;
    }
}

// ------------------------------------------- decode: interleaved staging
// The decode kernels stage 32-value chunks in LDS interleaved by lane: float4
// i (values 4i..4i+3 in the format's chunk order, xv[q] = x[col(c, q)]) of
// chunk c = l + 64 j sits at float4 slot (8 j + i) * 64 + l, so each of the
// eight ds_read_b128 that fetch a wave's chunk j reads 64 consecutive float4
// (no bank conflicts; the formats' natural column order puts eight lanes of a
// read on the same banks).
__device__ __forceinline__ uint32_t ilv_slot(uint32_t c, uint32_t i) { return ((c >> 6) * 8u + i) * 64u + (c & 63u); }
__device__ __forceinline__ void load_x_ilv(const float4* __restrict__ s, uint32_t j, uint32_t lane, float* xv) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 a = s[(8u * j + i) * 64u + lane];
        xv[4 * i] = a.x;
        xv[4 * i + 1] = a.y;
        xv[4 * i + 2] = a.z;
        xv[4 * i + 3] = a.w;
    }
}

// f16 hi + scaled lo of four values, for the formats that take f16 input
// pairs (half_x): {hi(x0, x1), hi(x2, x3), lo(x0, x1), lo(x2, x3)}, hi rounded
// toward zero and lo = (x - hi) * 2^11 (exact before its own rounding), so
// x = hi + lo / 2^11 to about 2^-20 relative. Stored in the float4 slot.
__device__ __forceinline__ float4 split_h4(float4 a) {
    const f16x2 h01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a.x, a.y));
    const f16x2 h23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a.z, a.w));
    const float r0 = (a.x - (float)h01.x) * 2048.0f, r1 = (a.y - (float)h01.y) * 2048.0f;
    const float r2 = (a.z - (float)h23.x) * 2048.0f, r3 = (a.w - (float)h23.y) * 2048.0f;
    const uint4 u = make_uint4(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23),
                               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1)),
                               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r2, r3)));
    return __builtin_bit_cast(float4, u);
}
__device__ __forceinline__ void load_xh_ilv(const float4* __restrict__ s, uint32_t j, uint32_t lane, uint32_t* xh,
                                            uint32_t* xl) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4 a = __builtin_bit_cast(uint4, s[(8u * j + i) * 64u + lane]);
        xh[2 * i] = a.x;
        xh[2 * i + 1] = a.y;
        xl[2 * i] = a.z;
        xl[2 * i + 1] = a.w;
    }
}

// ---------------------------------------------- decode: routed gate/up
// grid (ceil(F / RPW), T), 512 threads (8 waves), E <= 64 * NE. Wave w owns
// pairs k = w, w+8, ... of the block's token: it finds each pair's expert
// itself (wave_kth, selection k alone: no barrier, nothing shared) and issues
// that pair's weight loads at once. The routing weights need every
// selection's weight input: each wave leaves its pairs' in LDS, and after the
// barrier that publishes the staged input every wave forms the softmax (or
// sigmoid) weights in selection order (wave_route_weight); the waves of
// block 0 write the token's ids and weights for the down kernel. Wave w
// computes rows [RPW*bx, +RPW) of the gate and up projections and stores
// w_k * SwiGLU(g, u) (the routing weight folded in for the down kernel);
// each lane keeps its input chunks in registers. The formats with f16 input
// pairs (half_x) split x 2^e_t (x_exp of the max in the router's xstat[t]) and
// take 2^-e_t out of the row sums.
//   KS >= 0: the shared expert (format KS, ffn width F, weights sgate/sup)
// runs in the pair slot k = 8 NP - 1 of wave 7, which the routed pairs leave
// free (K < 8 NP), writing sact[t][r] = SwiGLU (its gate is applied by the
// down kernel); its input is staged a second time when its format takes the
// other input form.
//   PRE: the routing is an input (k_route ran: ids and wts hold every pair's
// expert and weight); the blocks skip the selection.
constexpr uint32_t GU_WAVES = 8;

template <int KIND, int CPL, int RPW, int NP, int NE, int KS = -1, bool PRE = false, int GW = GU_WAVES>
__global__ __launch_bounds__(64 * GW) void k_dec_gate_up2(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                      uint64_t gstride, uint64_t ustride, uint32_t F, uint32_t H,
                                                      const float* __restrict__ x, const float* __restrict__ xstat,
                                                      const float* __restrict__ logits,
                                                      const float* __restrict__ bias, uint32_t E, uint32_t K,
                                                      uint32_t sigmoid_mode, float scale, float limit,
                                                      uint32_t* __restrict__ ids, float* __restrict__ wts,
                                                      uint32_t* __restrict__ flags, float* __restrict__ act,
                                                      const uint8_t* __restrict__ sgate = nullptr,
                                                      const uint8_t* __restrict__ sup = nullptr, uint64_t sgstride = 0,
                                                      uint64_t sustride = 0, float* __restrict__ sact = nullptr,
                                                      const uint8_t* __restrict__ pfd = nullptr, uint64_t pfds = 0,
                                                      const uint8_t* __restrict__ pfs = nullptr, uint64_t pfss = 0) {
    using Fm = Fmt<KIND>;
    static_assert(GW >= 8 && GW <= (int)ROUTE_MAX_WAVES && GW * NP >= 8, "8 to 12 waves, at least 8 pair slots");
    constexpr bool HX = half_x<KIND>();  // input staged as f16 pairs (split_h4)
    constexpr int KSV = KS < 0 ? KIND : KS;
    using Fs = Fmt<KSV>;
    constexpr bool SH = KS >= 0, HS = SH && half_x<KSV>(), XS2 = SH && HS != HX;
    __shared__ float4 s_x4[1024];  // interleaved chunks (ilv_slot), H <= 4096
    __shared__ float4 s_xs4[XS2 ? 1024 : 1];  // the shared expert's input form
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t nch = H / 32u;
    const uint32_t r0 = blockIdx.x * RPW;
    // The token's input, two interleaved float4 slots per thread (slot u: lane
    // u % 64, chunk l + 64 (u / 512), float4 (u / 64) % 8), is loaded into
    // registers now and written to LDS after the weight loads are issued, so
    // its latency overlaps the routing's logit loads.
    // Codebooks: loaded first, written to LDS once the weight loads are out.
    TableStage<KIND, HX, 512> tab;
    TableStage<KSV, HS, 512> tabs;
    tab.load();
    if constexpr (SH && KSV != KIND) tabs.load();
    const float* xt = x + (uint64_t)t * H;
    float4 xa[2];
    bool xok[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t u = threadIdx.x + 64u * GW * m, ji = u >> 6, c = (u & 63u) + 64u * (ji >> 3);
        xok[m] = (ji >> 3) < (uint32_t)CPL && c < nch;
        xa[m] = xok[m] ? *reinterpret_cast<const float4*>(xt + Fm::col(c, 4u * (ji & 7u)))
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float xm = (HX || HS) ? xstat[2u * t] : 0.f;
    // The shared expert's rows (wave 7), loaded before the routing: they do
    // not depend on it.
    const bool shw = SH && wave == GW - 1u;
    typename Fs::Raw sg[SH ? RPW : 1][SH ? CPL : 1], su[SH ? RPW : 1][SH ? CPL : 1];
    if constexpr (SH) {
        if (shw) {
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const uint32_t r = min(r0 + i, F - 1);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const uint32_t c = min(lane + 64u * j, nch - 1);
                    sg[i][j] = Fs::load_raw(sgate + (uint64_t)r * sgstride, c);
                    su[i][j] = Fs::load_raw(sup + (uint64_t)r * sustride, c);
                }
            }
        }
    }
    __shared__ float s_sv[64];  // weight input of each selection
    uint32_t eid[NP];
    float ev[NP];
    // the pair each of the wave's slots computes (K: none, not stored)
    uint32_t kp[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) kp[n] = wave + GW * n;
    bool bad = false;
    // One pair per wave with wave_route: when every candidate has a wave (C <=
    // GW), wave w loads candidate w's rows while the ranks are formed, and
    // computes the pair of that candidate's rank (none if it is K or more).
    uint32_t spec_c = 0;
    if constexpr (PRE) {
        // routing done by k_route (batches of several tokens): ids and weights are inputs
#pragma unroll
        for (int n = 0; n < NP; ++n) {
            const uint32_t k = wave + GW * n;
            eid[n] = min(ids[(uint64_t)t * K + (k < K ? k : 0u)], E - 1u);
            ev[n] = 0.f;
        }
    } else if constexpr (NP == 1 && NE <= 2) {
        uint32_t key[NE];
        float wv[NE];
        bool ok[NE];
        bad = route_keys<NE>(logits + (uint64_t)t * E, bias, E, sigmoid_mode, key, wv, ok);
        eid[0] = wave_kth<NE>(key, wv, ok, wave < K ? wave : 0u, ev[0]);
    } else {
        // Several pairs per wave, or several keys per lane: the whole
        // selection once (wave_route: the candidates by the lanes' maxima,
        // then their ranks) instead of a search per pair; lane k holds
        // selection k.
        uint32_t my_id, C, rank;
        float my_v;
        bad = wave_route_compact<NE>(logits + (uint64_t)t * E, bias, E, K, sigmoid_mode, C);
        if (NP == 1 && C <= GW) {
            spec_c = C;
            eid[0] = route_lds()[64u + min(wave, C - 1u)];  // (a wave past C re-reads the last candidate's rows)
            ev[0] = 0.f;
        } else {
            wave_route_rank(C, E, K, my_id, my_v, rank);
#pragma unroll
            for (int n = 0; n < NP; ++n) {
                const uint32_t k = kp[n], kk = k < K ? k : 0u;  // no such pair: re-read pair 0's rows (not stored)
                eid[n] = (uint32_t)__builtin_amdgcn_readlane((int)my_id, (int)kk);
                ev[n] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), (int)kk));
            }
        }
    }
    // Weight loads of the wave's pairs k = wave + 8n (n < NP; K <= 8 NP);
    // a pair beyond K re-reads pair 0's rows and is not stored.
    typename Fm::Raw rg[NP][RPW][CPL], ru[NP][RPW][CPL];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t e = eid[n];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const uint32_t r = min(r0 + i, F - 1);
            const uint8_t* grow = gate + ((uint64_t)e * F + r) * gstride;
            const uint8_t* urow = up + ((uint64_t)e * F + r) * ustride;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + 64u * j, nch - 1);
                rg[n][i][j] = Fm::load_raw(grow, c);
                ru[n][i][j] = Fm::load_raw(urow, c);
            }
        }
    }
    // Down rows ahead of k_dec_down (pfd: the routed down matrix, pfs: the
    // shared expert's): this wave's experts' rows in this block's slice of H,
    // the slice that block blockIdx.x of the down kernel reads when its grid
    // splits H over as many blocks (else the rows still reach the MALL). One
    // byte per 128-byte line, requested after the wave's own weight loads and
    // left in registers until the empty asm at the end of the kernel, so the
    // down kernel's weight loads hit cache instead of waiting on HBM after its
    // expert ids arrive. Nothing is stored.
    uint32_t pfv[NP + 1][2] = {};
    if (pfd) {
        const uint32_t rs = (H + gridDim.x - 1) / gridDim.x, pr0 = min(blockIdx.x * rs, H);
        const uint32_t nr = min(pr0 + rs, H) - pr0;
#pragma unroll
        for (int n = 0; n < NP; ++n) {
            const uint32_t k = kp[n];
            if (n == 0 || k < K) {
                const uint8_t* pb = pfd + ((uint64_t)eid[n] * H + pr0) * pfds;
                const uint64_t span = (uint64_t)nr * pfds;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint64_t o = 128ull * (lane + 64u * i);
                    if (o < span) pfv[n][i] = pb[o];
                }
            }
        }
        if (SH && shw && pfs) {
            const uint8_t* pb = pfs + (uint64_t)pr0 * pfss;
            const uint64_t span = (uint64_t)nr * pfss;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint64_t o = 128ull * (lane + 64u * i);
                if (o < span) pfv[NP][i] = pb[o];
            }
        }
    }
    if (!PRE && spec_c != 0u) {
        // the ranks, with the candidates' loads in flight: this wave's
        // candidate's rank is its pair, and selection k's weight input is
        // lane k's after the placement
        uint32_t my_id, rank;
        float my_v;
        wave_route_rank(spec_c, E, K, my_id, my_v, rank);
        const uint32_t kw = (uint32_t)__builtin_amdgcn_readlane((int)rank, (int)min(wave, spec_c - 1u));
        kp[0] = wave < spec_c && kw < K ? kw : K;
        ev[0] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), (int)(kp[0] < K ? kp[0] : 0u)));
    }
    // (read only after the barrier below)
    tab.store();
    if constexpr (SH && KSV != KIND) tabs.store();
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t k = kp[n];
        if (!PRE && k < K && lane == 0) {
            s_sv[k] = ev[n];
            if (blockIdx.x == 0) ids[(uint64_t)t * K + k] = eid[n];
        }
    }
    const int xe = x_exp(xm);
#pragma unroll
    for (int m = 0; m < 2; ++m)
        if (xok[m]) {
            s_x4[threadIdx.x + 64u * GW * m] = HX ? split_h4(ldexp4(xa[m], xe)) : xa[m];
            if constexpr (XS2) s_xs4[threadIdx.x + 64u * GW * m] = HS ? split_h4(ldexp4(xa[m], xe)) : xa[m];
        }
    __syncthreads();
    // Routing weights in selection order; block 0's wave 0 publishes them.
    const float w = PRE ? (lane < K ? wts[(uint64_t)t * K + lane] : 0.f)
                        : wave_route_weight(lane < K ? s_sv[lane] : 0.f, K, sigmoid_mode, scale);
    if (!PRE && blockIdx.x == 0 && wave == 0) {
        if (flags && __any(bad) && lane == 0) atomicOr(flags, FLAG_NONFINITE);
        if (lane < K) wts[(uint64_t)t * K + lane] = w;
    }
    float wk[NP];  // routing weight of each of the wave's pairs: act is stored as w_k * SwiGLU
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t k = kp[n];
        wk[n] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (int)(k < K ? k : 0u)));
    }
    float xv[HX ? 1 : CPL][HX ? 1 : 32], xs0[CPL], xs1[CPL];
    uint32_t xh[HX ? CPL : 1][16], xl[HX ? CPL : 1][16];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if constexpr (HX) {
            load_xh_ilv(s_x4, j, lane, xh[j], xl[j]);
        } else {
            load_x_ilv(s_x4, j, lane, xv[j]);
            xs0[j] = xs1[j] = 0.f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                xs0[j] += xv[j][q];
                xs1[j] += xv[j][16 + q];
            }
        }
    }
    auto dotc = [&](const typename Fm::Raw& r, int j, uint32_t c) -> float {
        if constexpr (HX) return Fm::dot_raw_h(r, xh[j], xl[j]);
        else return Fm::dot_raw(r, c, xv[j], xs0[j], xs1[j]);
    };
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t k = kp[n];
        if (k < K) {  // a pair beyond K (its loads re-read pair 0's rows) is skipped
            float gs[RPW], us[RPW];
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                gs[i] = us[i] = 0.f;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    if (lane + 64u * j >= nch) continue;
                    const uint32_t c = lane + 64u * j;
                    gs[i] += dotc(rg[n][i][j], j, c);
                    us[i] += dotc(ru[n][i][j], j, c);
                }
            }
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                float g = wave_sum_dpp(gs[i]), u = wave_sum_dpp(us[i]);
                if constexpr (HX) {
                    g = ldexpf(g, -xe);
                    u = ldexpf(u, -xe);
                }
                if (k < K && lane == (uint32_t)i && r0 + i < F)
                    act[((uint64_t)t * K + k) * F + r0 + i] = swiglu(g, u, limit) * wk[n];
            }
        }
    }
    if constexpr (SH) {
        if (shw) {
            float gs[RPW], us[RPW];
#pragma unroll
            for (int i = 0; i < RPW; ++i) gs[i] = us[i] = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = lane + 64u * j;
                if (c >= nch) continue;
                if constexpr (HS) {
                    uint32_t sh[16], sl[16];
                    if constexpr (XS2) load_xh_ilv(s_xs4, j, lane, sh, sl);
                    else load_xh_ilv(s_x4, j, lane, sh, sl);
#pragma unroll
                    for (int i = 0; i < RPW; ++i) {
                        gs[i] += Fs::dot_raw_h(sg[i][j], sh, sl);
                        us[i] += Fs::dot_raw_h(su[i][j], sh, sl);
                    }
                } else {
                    float sv[32];
                    if constexpr (XS2) load_x_ilv(s_xs4, j, lane, sv);
                    else load_x_ilv(s_x4, j, lane, sv);
                    float s0 = 0.f, s1 = 0.f;
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        s0 += sv[q];
                        s1 += sv[16 + q];
                    }
#pragma unroll
                    for (int i = 0; i < RPW; ++i) {
                        gs[i] += Fs::dot_raw(sg[i][j], c, sv, s0, s1);
                        us[i] += Fs::dot_raw(su[i][j], c, sv, s0, s1);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                float g = wave_sum_dpp(gs[i]), u = wave_sum_dpp(us[i]);
                if constexpr (HS) {
                    g = ldexpf(g, -xe);
                    u = ldexpf(u, -xe);
                }
                if (lane == (uint32_t)i && r0 + i < F) sact[(uint64_t)t * F + r0 + i] = swiglu(g, u, limit);
            }
        }
    }
#pragma unroll
    for (int n = 0; n <= NP; ++n) asm volatile("" ::"v"(pfv[n][0]), "v"(pfv[n][1]));
}

// ------------------------------------------------ decode: down + combine
// grid (ceil(H / (DOWN_WAVES * RPW)), T), DOWN_THREADS threads. The K pairs'
// chunks (plus the shared expert's) form one virtual row spread over the
// lanes (chunk v = l + 64 j, j < VPL); each wave owns RPW output rows, so the
// wave sum is sum_k w_k (D_e act_k)[i] (+ gate * (S_down sact)[i]) directly.
// The routed activations arrive already scaled by their pair's routing
// weight (the gate/up kernel stores w_k * act). Each thread loads its share
// of the virtual row's activations at kernel start, after the chunk ids and
// before the weights, so the loads complete in that order; the shared
// expert's values are scaled by its gate, and the block stages them in LDS
// interleaved (ilv_slot) with the two 16-value sums of every chunk.
constexpr uint32_t DOWN_WAVES = 8;
constexpr uint32_t DOWN_THREADS = 64 * DOWN_WAVES;
constexpr uint32_t DOWN_LDS_FLOATS = 12288;                        // 48 KB of staged activations
constexpr uint32_t DOWN_ACT4 = DOWN_LDS_FLOATS / 4 / DOWN_THREADS;  // float4 loads per thread

template <int KD, int KS, int VPL, int RPW>
__global__ __launch_bounds__(DOWN_THREADS) void k_dec_down(const uint8_t* __restrict__ down, uint64_t dstride,
                                                           const uint8_t* __restrict__ sdown, uint64_t sdstride,
                                                           uint32_t H, uint32_t F, uint32_t SF,
                                                           const float* __restrict__ act, const float* __restrict__ sact,
                                                           const uint32_t* __restrict__ ids,
                                                           const float* __restrict__ sgl, uint32_t K,
                                                           const float* __restrict__ res, float* __restrict__ out,
                                                           uint32_t* __restrict__ flags) {
    using Fd = Fmt<KD>;
    using Fs = Fmt<(KS < 0 ? KD : KS)>;
    constexpr bool HD = half_x<KD>(), HS = KS >= 0 && half_x<(KS < 0 ? KD : KS)>();  // f16-pair inputs
    __shared__ float4 s_act4[DOWN_LDS_FLOATS / 4];
    __shared__ float s_sum[DOWN_LDS_FLOATS / 16];
    // Codebooks: loaded first, written to LDS once the weight loads are out
    // (decoded after the barrier that follows the activation staging).
    TableStage<KD, HD, DOWN_THREADS> tab;
    TableStage<(KS < 0 ? KD : KS), HS, DOWN_THREADS> tabs;
    tab.load();
    if constexpr (KS >= 0 && KS != KD) tabs.load();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, tid = threadIdx.x;
    const uint32_t t = blockIdx.y;
    const uint32_t nchF = F / 32u, nchS = KS >= 0 ? SF / 32u : 0u;
    const uint32_t nv = K * nchF + nchS, KF = K * F;
    const uint32_t r0 = (blockIdx.x * DOWN_WAVES + wave) * RPW;
    // Every load below is unconditional (indices clamped into the virtual
    // row), so the compiler's load counting can wait for each chunk's weights
    // alone; lanes past the virtual row load valid bytes and discard them.
    // One chunk format for routed and shared experts keeps the weight loads
    // branch-free too.
    constexpr bool UNI = KS < 0 || KS == KD;
    const uint32_t KC = K * nchF;  // routed chunks
    // The residual of this lane's output row (lane i < RPW writes row r0 + i),
    // loaded first so that its latency overlaps the others'.
    float resv = 0.f;
    if (res) resv = res[(uint64_t)t * H + min(r0 + min(lane, (uint32_t)RPW - 1u), H - 1u)];
    // 1. expert ids of this lane's chunks of the virtual row (chunk v: pair
    //    v / nchF; the quotient by multiply-high, exact for v < 2^32 / nchF)
    const uint32_t mag = 0xffffffffu / nchF + 1u;
    uint32_t eid[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) eid[j] = ids[(uint64_t)t * K + __umulhi(min(lane + 64u * j, KC - 1u), mag)];
    // 2. this thread's activations: slot u = tid + DOWN_THREADS m is float4
    //    u % 8 of chunk u / 8 (a chunk's two 16-value groups in two lane quads)
    float4 av[DOWN_ACT4];
    const float* at = act + (uint64_t)t * KF;
    const float* st = sact + (uint64_t)t * SF;
#pragma unroll
    for (int m = 0; m < (int)DOWN_ACT4; ++m) {
        const uint32_t u = tid + DOWN_THREADS * m, i4 = 4u * (u & 7u), vc = min(u >> 3, nv - 1u);
        const uint32_t vr = min(vc, KC - 1u), k = __umulhi(vr, mag);
        const float* p = at + k * F + Fd::col(vr - k * nchF, i4);
        if constexpr (KS >= 0) p = vc >= KC ? st + Fs::col(vc - KC, i4) : p;
        av[m] = *reinterpret_cast<const float4*>(p);
    }
    const float sgv = (KS >= 0 && sgl) ? sgl[t] : 0.f;
    __builtin_amdgcn_sched_barrier(0);
    // 3. weight loads for all RPW rows
    const uint8_t* base[VPL];
    uint64_t stride[VPL];
    uint32_t cc[VPL];
    bool isS[VPL], has[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t v = lane + 64u * j, vr = min(v, KC - 1u);
        has[j] = v < nv;
        isS[j] = KS >= 0 && v >= KC && v < nv;
        base[j] = isS[j] ? sdown : down + (uint64_t)eid[j] * H * dstride;
        stride[j] = isS[j] ? sdstride : dstride;
        cc[j] = isS[j] ? v - KC : vr - __umulhi(vr, mag) * nchF;
    }
    typename Fd::Raw rd[RPW][VPL];
    typename Fs::Raw rs[UNI ? 1 : RPW][UNI ? 1 : VPL];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const uint32_t r = min(r0 + i, H - 1);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if constexpr (UNI) {
                rd[i][j] = Fd::load_raw(base[j] + (uint64_t)r * stride[j], cc[j]);
            } else {
                if (!has[j]) continue;
                if (isS[j]) rs[UNI ? 0 : i][UNI ? 0 : j] = Fs::load_raw(base[j] + (uint64_t)r * stride[j], cc[j]);
                else rd[i][j] = Fd::load_raw(base[j] + (uint64_t)r * stride[j], cc[j]);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    tab.store();
    if constexpr (KS >= 0 && KS != KD) tabs.store();
    // 4. stage the activations (shared expert's times its gate) and each
    //    chunk's two 16-value sums (xs0, xs1 of the formats' dot products).
    //    Chunks of the f16-pair formats are split after scaling by 2^ea, ea
    //    from the block's maximum over them (x_exp), and their dot products
    //    are scaled back.
    const float gate = KS >= 0 ? (sgl ? ingot_det_sigmoid(sgv) : 1.0f) : 1.0f;
    constexpr bool ANYH = HD || HS;
    float amax = 0.f;
#pragma unroll
    for (int m = 0; m < (int)DOWN_ACT4; ++m) {
        const uint32_t u = tid + DOWN_THREADS * m, v = u >> 3;
        if (KS >= 0 && v >= K * nchF) {
            av[m].x *= gate;
            av[m].y *= gate;
            av[m].z *= gate;
            av[m].w *= gate;
        }
        if (ANYH && v < nv && (v < KC ? HD : HS)) amax = fmaxf(amax, max_abs4(av[m]));
    }
    int ea = 0;
    if constexpr (ANYH) {
        __shared__ float s_amax[DOWN_WAVES];
        amax = wave_max(amax);
        if (lane == 0) s_amax[wave] = amax;
        __syncthreads();
#pragma unroll
        for (uint32_t w = 0; w < DOWN_WAVES; ++w) amax = fmaxf(amax, s_amax[w]);
        ea = x_exp(amax);
    }
#pragma unroll
    for (int m = 0; m < (int)DOWN_ACT4; ++m) {
        const uint32_t u = tid + DOWN_THREADS * m, v = u >> 3;
        const float4 a = av[m];
        const bool half = v < KC ? HD : HS;
        if (v < nv) s_act4[ilv_slot(v, u & 7u)] = half ? split_h4(ldexp4(a, ea)) : a;
        float g = (a.x + a.y) + (a.z + a.w);
        g = dpp_add<0xb1>(g);  // quad_perm [1,0,3,2]
        g = dpp_add<0x4e>(g);  // quad_perm [2,3,0,1]
        if ((u & 3u) == 0 && v < nv) s_sum[2u * v + ((u >> 2) & 1u)] = g;
    }
    __syncthreads();
    // 5. the dot products (f16-pair chunks into acch, in units of 2^ea)
    float acc[RPW], acch[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = acch[i] = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        if (!has[j]) continue;
        if ((HD && !isS[j]) || (HS && isS[j])) {
            uint32_t xh[16], xl[16];
            load_xh_ilv(s_act4, j, lane, xh, xl);
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                if constexpr (HS && !UNI) {
                    if (isS[j]) {
                        acch[i] += Fs::dot_raw_h(rs[UNI ? 0 : i][UNI ? 0 : j], xh, xl);
                        continue;
                    }
                }
                if constexpr (HD) acch[i] += Fd::dot_raw_h(rd[i][j], xh, xl);
            }
        } else {
            float xv[32];
            load_x_ilv(s_act4, j, lane, xv);
            const float2 xs = reinterpret_cast<const float2*>(s_sum)[lane + 64u * j];
            const float xs0 = xs.x, xs1 = xs.y;
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                if (!UNI && isS[j]) acc[i] += Fs::dot_raw(rs[UNI ? 0 : i][UNI ? 0 : j], cc[j], xv, xs0, xs1);
                else acc[i] += Fd::dot_raw(rd[i][j], cc[j], xv, xs0, xs1);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        float sum = ANYH ? acc[i] + ldexpf(acch[i], -ea) : acc[i];
        sum = wave_sum_dpp(sum);
        const uint32_t r = r0 + i;
        if (lane == (uint32_t)i && r < H) {
            if (res) sum += resv;
            out[(uint64_t)t * H + r] = sum;
            if (!isfinite(sum)) atomicOr(flags, FLAG_OUT_NONFINITE);
        }
    }
}

// ----------------------------------------------------------- decode: gate/up
// grid (ceil(F / (4*RPW)), pairs); a wave owns RPW rows of one pair. Lane l
// owns chunks l + 64j (j < CPL) of the H columns: their 32 inputs stay in
// registers for all the wave's rows, and each row costs the lane one header
// and one 16-byte nibble load per chunk (Q4_K). ids == NULL: shared-expert
// mode (expert 0, token = pair).
template <int KIND, int CPL, int RPW>
__global__ __launch_bounds__(256) void k_gemv_gate_up(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                      uint64_t gstride, uint64_t ustride, uint32_t F, uint32_t H,
                                                      const float* __restrict__ x, const uint32_t* __restrict__ ids,
                                                      uint32_t K, float limit, float* __restrict__ act) {
    using Fm = Fmt<KIND>;
    if constexpr (has_codebook<KIND>()) {
        stage_codebooks<KIND>();
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t p = blockIdx.y;
    const uint32_t e = ids ? ids[p] : 0u, t = ids ? p / K : p;
    const uint32_t nch = H / 32u;
    float xv[CPL][32], xs0[CPL], xs1[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        uint32_t c = lane + 64u * j;
        xs0[j] = xs1[j] = 0.f;
        if (c < nch) {
            Fm::load_x(x + (uint64_t)t * H, c, xv[j]);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                xs0[j] += xv[j][i];
                xs1[j] += xv[j][16 + i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) xv[j][i] = 0.f;
        }
    }
    const uint32_t r0 = (blockIdx.x * 4u + wave) * RPW;
    float gs[RPW], us[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        gs[i] = us[i] = 0.f;
        uint32_t r = min(r0 + i, F - 1);
        const uint8_t* grow = gate + ((uint64_t)e * F + r) * gstride;
        const uint8_t* urow = up + ((uint64_t)e * F + r) * ustride;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            uint32_t c = lane + 64u * j;
            if (c < nch) {
                gs[i] += Fm::dot(grow, c, xv[j], xs0[j], xs1[j]);
                us[i] += Fm::dot(urow, c, xv[j], xs0[j], xs1[j]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        float g = wave_sum(gs[i]), u = wave_sum(us[i]);
        if (lane == (uint32_t)i && r0 + i < F) act[(uint64_t)p * F + r0 + i] = swiglu(g, u, limit);
    }
}

// Adds a separately computed shared-expert down product to out (used when the
// shared down format has no fused instantiation): out[t] += s * S_down sact[t].
template <int KS, int CPL>
__global__ __launch_bounds__(256) void k_gemv_shared_down_add(const uint8_t* __restrict__ sdown, uint64_t sdstride,
                                                              uint32_t H, uint32_t SF, const float* __restrict__ sact,
                                                              const float* __restrict__ sgl, float* __restrict__ out,
                                                              uint32_t* __restrict__ flags) {
    using Fs = Fmt<KS>;
    if constexpr (has_codebook<KS>()) {
        stage_codebooks<KS>();
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y, r = blockIdx.x * 4u + wave;
    if (r >= H) return;
    const uint32_t nch = SF / 32u;
    float w = sgl ? ingot_det_sigmoid(sgl[t]) : 1.0f;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        uint32_t c = lane + 64u * j;
        if (c >= nch) continue;
        float xv[32], s0 = 0.f, s1 = 0.f;
        Fs::load_x(sact + (uint64_t)t * SF, c, xv);
#pragma unroll
        for (int i = 0; i < 32; ++i) xv[i] *= w;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 += xv[i];
            s1 += xv[16 + i];
        }
        acc += Fs::dot(sdown + (uint64_t)r * sdstride, c, xv, s0, s1);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        const float o = out[(uint64_t)t * H + r] + acc;
        out[(uint64_t)t * H + r] = o;
        if (!isfinite(o)) atomicOr(flags, FLAG_OUT_NONFINITE);
    }
}

// ------------------------------------------------------- prefill: dispatch
// Block-wide exclusive scan of one value per thread (blockDim 1024 = 16 waves).
// Inclusive prefix sum over a wave by DPP: row_shr 1, 2, 4, 8 within each
// 16-lane row, then row_bcast 15 (rows 1, 3) and row_bcast 31 (rows 2, 3)
// carry the row totals. The whole wave must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_add_u32(uint32_t v) {
    return v + (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, true);
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v = dpp_add_u32<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add_u32<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add_u32<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add_u32<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add_u32<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_add_u32<0x143, 0xc>(v);  // row_bcast:31
    return v;
}

__device__ inline uint32_t block_exclusive_scan_1024(uint32_t v, uint32_t* wsum, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_incl_scan(v);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        const uint32_t s = lane < 16 ? wsum[lane] : 0u, si = wave_incl_scan(s);
        if (lane < 16) wsum[16 + lane] = si - s;
        if (lane == 15) *total = si;
    }
    __syncthreads();
    return inc - v + wsum[16 + wave];
}

// One block of 1024 threads (16 waves), E <= 1024: the whole prefill
// dispatch (kernels/prefill.metal:7-38). Writes counts[E], first[E]
// (exclusive scan, experts ascending), the stable pair order pairs[] (experts
// ascending, pair index ascending within an expert), inverse[p] (packed
// position of pair p) and the tile list of TM-pair tiles {expert, first pair
// of the tile, n in tile, number of non-empty tiles}, padded with zero tiles
// to cap. Tile order: the shared expert's tiles when S > 0 (expert id E,
// positions P..P+S-1, pairs[P + t] = t K so that pairs[q] / K is the token),
// every expert's full tiles (experts ascending), then the partial last tiles
// by decreasing n, so that work scheduled last is the cheapest; results do
// not depend on the order, each tile's rows being computed independently.
//   Stable placement: wave w owns the contiguous pair segment
//   [w seg, (w + 1) seg); a histogram per wave gives each wave's start inside
//   every expert's range; the wave then walks its segment 64 pairs at a time,
//   and a pair's rank among earlier lanes with the same expert comes from
//   ballots over the bits of the expert id. A wave reads its ids DSP_BATCH
//   per lane at a time, all loads issued before the first is used.
// Blocks 1.. (when xh != NULL) split the token inputs into f16 hi + lo for
// the f16 GEMM (split_f16_part), beside the dispatch. Block 0 also clears the
// per-row activation maxima (rowmax[0 .. nrow)) that the gate/up GEMM raises.
constexpr uint32_t DSP_BATCH = 8;
__device__ inline void split_f16_part(const float* __restrict__ x, uint64_t n, _Float16* __restrict__ xh,
                                      _Float16* __restrict__ xl, float* __restrict__ xs, uint32_t order, uint64_t g,
                                      const float* __restrict__ xstat, uint32_t H);

#ifndef INGOT_KIND_UNIT  // compiled in moe_hip.hip only
__global__ __launch_bounds__(1024) void k_dispatch(const uint32_t* __restrict__ ids, uint32_t P, uint32_t E,
                                                   uint32_t TM, uint32_t cap, uint32_t* __restrict__ counts,
                                                   uint32_t* __restrict__ first, uint32_t* __restrict__ tiles,
                                                   uint32_t* __restrict__ pairs, uint32_t* __restrict__ inverse,
                                                   uint32_t S, uint32_t K, const float* __restrict__ x, uint64_t xn,
                                                   _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                   float* __restrict__ xs, uint32_t xorder,
                                                   const float* __restrict__ xstat, uint32_t H,
                                                   uint32_t* __restrict__ rowmax, uint32_t nrow) {
    if (blockIdx.x > 0) {
        split_f16_part(x, xn, xh, xl, xs, xorder, (uint64_t)(blockIdx.x - 1u) * blockDim.x + threadIdx.x, xstat, H);
        return;
    }
    if (rowmax)
        for (uint32_t i = threadIdx.x; i < nrow; i += 1024u) rowmax[i] = 0u;
    __shared__ uint32_t hist[16][1024];  // per wave, per expert; then each wave's running position
    __shared__ uint32_t wsum[32];
    __shared__ uint32_t tot[3];
    __shared__ uint32_t rbin[1024];  // partial tiles per remainder, then their start positions
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
#pragma unroll
    for (int w = 0; w < 16; ++w) hist[w][tid] = 0;
    rbin[tid] = 0;
    __syncthreads();
    const uint32_t seg = (P + 15u) / 16u, s0 = min(P, wave * seg), s1 = min(P, s0 + seg);
    // The first batch of ids stays in registers for the placement pass.
    uint32_t xv0[DSP_BATCH];
#pragma unroll
    for (int i = 0; i < (int)DSP_BATCH; ++i) xv0[i] = P ? ids[min(s0 + 64u * i + lane, P - 1u)] : 0u;
    for (uint32_t b0 = s0; b0 < s1; b0 += 64u * DSP_BATCH) {
        uint32_t xv[DSP_BATCH];
#pragma unroll
        for (int i = 0; i < (int)DSP_BATCH; ++i) xv[i] = b0 == s0 ? xv0[i] : ids[min(b0 + 64u * i + lane, P - 1u)];
#pragma unroll
        for (int i = 0; i < (int)DSP_BATCH; ++i)
            if (b0 + 64u * i + lane < s1) atomicAdd(&hist[wave][xv[i]], 1u);
    }
    __syncthreads();
    // Expert tid: its count, and each wave's offset within the expert.
    uint32_t n = 0;
    if (tid < E) {
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            const uint32_t h = hist[w][tid];
            hist[w][tid] = n;
            n += h;
        }
    }
    const uint32_t nfull = n / TM, rem = n - nfull * TM;
    const uint32_t f = block_exclusive_scan_1024(n, wsum, &tot[0]);
    __syncthreads();
    const uint32_t t0 = block_exclusive_scan_1024(nfull, wsum, &tot[1]);  // full tiles
    if (tid < E) {
        counts[tid] = n;
        first[tid] = f;
#pragma unroll
        for (int w = 0; w < 16; ++w) hist[w][tid] += f;
    }
    if (rem) atomicAdd(&rbin[rem], 1u);
    __syncthreads();
    // Start of each remainder's run among the partial tiles (larger remainders
    // first): exclusive scan over remainders TM-1 .. 1.
    const uint32_t rr = tid < TM ? TM - 1u - tid : 0u;
    const uint32_t c = (tid < TM && rr > 0) ? rbin[rr] : 0u;
    const uint32_t before = block_exclusive_scan_1024(c, wsum, &tot[2]);
    const uint32_t nt_all = tot[2];
    __syncthreads();
    // The shared expert's S rows (S = 0: none) come first, as expert E over
    // positions P..P+S-1, whose pairs entry t K names token t.
    const uint32_t nsh = (S + TM - 1u) / TM;
    if (tid < TM && rr > 0) rbin[rr] = nsh + tot[1] + before;
    __syncthreads();
    const uint32_t ntiles = min(nsh + tot[1] + nt_all, cap);
    for (uint32_t j = tid; j < nsh && j < cap; j += 1024u) {
        uint32_t* tl = tiles + 4u * j;
        tl[0] = E;
        tl[1] = P + j * TM;
        tl[2] = min(TM, S - j * TM);
        tl[3] = ntiles;
    }
    for (uint32_t t = tid; t < S; t += 1024u) pairs[P + t] = t * K;
    if (tid < E) {
        for (uint32_t k = 0; k < nfull && nsh + t0 + k < cap; ++k) {
            uint32_t* tl = tiles + 4u * (nsh + t0 + k);
            tl[0] = tid;
            tl[1] = f + k * TM;
            tl[2] = TM;
            tl[3] = ntiles;
        }
        if (rem) {
            const uint32_t t = atomicAdd(&rbin[rem], 1u);
            if (t < cap) {
                uint32_t* tl = tiles + 4u * t;
                tl[0] = tid;
                tl[1] = f + nfull * TM;
                tl[2] = rem;
                tl[3] = ntiles;
            }
        }
    }
    for (uint32_t t = nsh + tot[1] + nt_all + tid; t < cap; t += 1024u) {
        uint32_t* tl = tiles + 4u * t;
        tl[0] = tl[1] = tl[2] = 0;
        tl[3] = ntiles;
    }
    // Stable placement, wave by wave over its own segment (no barrier needed:
    // each wave only touches its own row of hist).
    uint32_t nbits = 1;
    while ((1u << nbits) < E) ++nbits;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (uint32_t b0 = s0; b0 < s1; b0 += 64u * DSP_BATCH) {
        uint32_t xv[DSP_BATCH];
#pragma unroll
        for (int i = 0; i < (int)DSP_BATCH; ++i) xv[i] = b0 == s0 ? xv0[i] : ids[min(b0 + 64u * i + lane, P - 1u)];
#pragma unroll
        for (int i = 0; i < (int)DSP_BATCH; ++i) {
            const uint32_t base = b0 + 64u * i;
            if (base >= s1) break;
            const uint32_t p = base + lane;
            const bool live = p < s1;
            const uint32_t e = live ? xv[i] : 0u;
            uint64_t same = __ballot(live);
            for (uint32_t b = 0; b < nbits; ++b) {
                const uint64_t one = __ballot(live && ((e >> b) & 1u));
                same &= ((e >> b) & 1u) ? one : ~one;
            }
            if (live) {
                const uint32_t pos = hist[wave][e] + (uint32_t)__popcll(same & lt);
                pairs[pos] = p;
                inverse[p] = pos;
            }
            // every lane has read the running positions before the leaders advance them
            wave_sync();
            if (live && (same & lt) == 0) hist[wave][e] += (uint32_t)__popcll(same);
            wave_sync();
        }
    }
}
#endif  // INGOT_KIND_UNIT

// ---------------------------------------------------- prefill: grouped GEMM
// One block (256 threads, 4 waves) per (row tile, token tile). A token tile
// {expert, first, n} covers packed positions first..first+n-1 (n <= 64).
//   GATEUP: A = input rows x[token(pairs[q])] (H cols), B = 64 gate rows and
//           the same 64 up rows of the expert; out act[q][row] = SwiGLU.
//   !GATEUP: A = act[q] (F cols), B = 128 down rows; out Y[q][row].
// The K dimension runs in 64-column slabs: the block stages A (64 x 64 fp32)
// and B (128 rows x 64, dequantised from two 32-value chunks per row) in LDS,
// with the next slab's global loads issued before the current slab's MFMAs.
// Each wave computes a 64 x 32 output block (4 x 2 tiles of
// v_mfma_f32_16x16x4f32). The MFMA k-index of lane i at step ks is
// 4*(i/16)+ks inside a 16-column group, so each lane fetches 4 consecutive
// columns of A and B with one 128-bit LDS read.
constexpr uint32_t TM = 64, LDS_STRIDE = 68;
// slot_of entry of an expert that is not in the device slots for this pass.
constexpr uint32_t NO_SLOT = 0xffffffffu;

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int KIND, bool GATEUP>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                              uint64_t stride0, uint64_t stride1, uint32_t rows_per_expert,
                                              uint32_t kdim, const float* __restrict__ a_src,
                                              const uint32_t* __restrict__ pairs, uint32_t K,
                                              const uint32_t* __restrict__ tiles, uint32_t ldo, float limit,
                                              float* __restrict__ out, const uint32_t* __restrict__ slot_of) {
    using Fm = Fmt<KIND>;
    __shared__ float As[TM * LDS_STRIDE];
    __shared__ float Bs[128 * LDS_STRIDE];
    const uint32_t* tile = tiles + 4u * blockIdx.y;
    const uint32_t n = tile[2];
    if (n == 0) return;
    // Cached experts (slot_of != NULL): the tile's expert lives in slot
    // slot_of[e] of the weight arrays, or is not resident in this pass (NO_SLOT).
    const uint32_t ew = slot_of ? slot_of[tile[0]] : tile[0];
    if (ew == NO_SLOT) return;
    if constexpr (has_codebook<KIND>()) {
        stage_codebooks<KIND>();
        __syncthreads();
    }
    const uint32_t e = tile[0], q0 = tile[1];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // Output rows of this block: GATEUP 64 (gate and up), else 128.
    const uint32_t row0 = blockIdx.x * (GATEUP ? 64u : 128u);

    // A loader: 4 float4 per thread; element idx = tid + 256 i -> row idx/16, col4 idx%16.
    const float* arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t m = (tid + 256u * i) >> 4;
        arow[i] = nullptr;
        if (m < n) {
            uint32_t q = q0 + m;
            uint64_t r = GATEUP ? (pairs ? pairs[q] / K : q) : q;
            arow[i] = a_src + r * kdim;
        }
    }
    const uint32_t acol = 4u * (tid & 15u);
    // B loader: thread -> (B row brow = tid/2, chunk half h = tid%2).
    const uint32_t brow = tid >> 1, bh = tid & 1u;
    const uint8_t* bptr;
    if (GATEUP) {
        const uint8_t* base = brow < 64 ? w0 : w1;
        uint64_t st = brow < 64 ? stride0 : stride1;
        uint32_t r = row0 + (brow & 63u);
        bptr = base + ((uint64_t)ew * rows_per_expert + r) * st;
    } else {
        bptr = w0 + ((uint64_t)ew * rows_per_expert + row0 + brow) * stride0;
    }

    // Only the first ceil(n / 16) 16-row blocks of the tile issue MFMAs.
    auto run = [&](auto mbe_tag) {
        constexpr int MBE = decltype(mbe_tag)::value;
        floatx4 acc[MBE][2];
#pragma unroll
        for (int i = 0; i < MBE; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

        float4 ar[4];
        typename Fm::Raw br;
        auto load = [&](uint32_t s) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ar[i] = arow[i] ? *reinterpret_cast<const float4*>(arow[i] + 64u * s + acol) : make_float4(0.f, 0.f, 0.f, 0.f);
            br = Fm::load_raw(bptr, 2u * s + bh);
        };
        const uint32_t slabs = kdim / 64u;
        load(0);
        for (uint32_t s = 0; s < slabs; ++s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t m = (tid + 256u * i) >> 4;
                *reinterpret_cast<float4*>(&As[m * LDS_STRIDE + acol]) = ar[i];
            }
            {
                float wv[32];
                Fm::dequant_raw(br, 2u * s + bh, wv);
                float* dst = &Bs[brow * LDS_STRIDE];
                // Chunk value i -> slab column: Fm::col(chunk, i) - 64 s.
#pragma unroll
                for (int i = 0; i < 32; i += 4) {
                    uint32_t cl = Fm::col(2u * s + bh, i) - 64u * s;
                    *reinterpret_cast<float4*>(dst + cl) = make_float4(wv[i], wv[i + 1], wv[i + 2], wv[i + 3]);
                }
            }
            __syncthreads();
            if (s + 1 < slabs) load(s + 1);
#pragma unroll
            for (uint32_t kk = 0; kk < 4; ++kk) {
                const uint32_t kc = kk * 16u + 4u * (lane >> 4);
                float4 a[MBE], b[2];
#pragma unroll
                for (int mb = 0; mb < MBE; ++mb)
                    a[mb] = *reinterpret_cast<const float4*>(&As[(mb * 16u + (lane & 15u)) * LDS_STRIDE + kc]);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    // GATEUP: nb 0 = gate rows 16w.., nb 1 = up rows 64+16w..; else rows 32w + 16nb..
                    uint32_t br_ = GATEUP ? (nb * 64u + 16u * wave) : (32u * wave + 16u * nb);
                    b[nb] = *reinterpret_cast<const float4*>(&Bs[(br_ + (lane & 15u)) * LDS_STRIDE + kc]);
                }
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                    for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb) {
                            float av = ks == 0 ? a[mb].x : ks == 1 ? a[mb].y : ks == 2 ? a[mb].z : a[mb].w;
                            float bv = ks == 0 ? b[nb].x : ks == 1 ? b[nb].y : ks == 2 ? b[nb].z : b[nb].w;
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[mb][nb], 0, 0, 0);
                        }
            }
            __syncthreads();
        }
        // Epilogue: lane holds D[m = 4*(lane/16) + j][n = lane%16] of each tile.
#pragma unroll
        for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t m = mb * 16u + 4u * (lane >> 4) + j;
                if (m >= n) continue;
                uint64_t q = q0 + m;
                if (GATEUP) {
                    uint32_t r = row0 + 16u * wave + (lane & 15u);
                    out[q * ldo + r] = swiglu(acc[mb][0][j], acc[mb][1][j], limit);
                } else {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        uint32_t r = row0 + 32u * wave + 16u * nb + (lane & 15u);
                        out[q * ldo + r] = acc[mb][nb][j];
                    }
                }
            }
    };
    switch ((n + 15u) >> 4) {
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 3: run(std::integral_constant<int, 3>{}); break;
        default: run(std::integral_constant<int, 4>{}); break;
    }
}

// ------------------ prefill: grouped GEMM on f16 MFMA (Q4_K, IQ3_XXS, IQ4_NL)
// Same tile list as k_gemm, computed on v_mfma_f32_16x16x32_f16 with fp32
// accumulation and no loss against fp32 operands:
//   * A (inputs or activations, fp32) arrives split in HBM as f16 hi + lo
//     (ah, al: [rows][kdim], a = hi + lo to 2^-22 |a|) and is staged per
//     64-column slab in LDS; both halves enter the MFMA.
//   * B is not dequantised. Each format's weight is an integer times scales,
//     and the MFMA takes the integer (at most 2047, sign in bit 15) as the raw
//     bits of an f16: bits b <= 2047 are the exact value b 2^-24 (subnormal
//     below 1024, exponent field 1 up to 2047).
//       Q4_K    w = d sc_g q - dmin mn_g (q a nibble, sc_g and mn_g 6-bit
//               integers of the 32-column group g, d and dmin f16 per
//               256-column superblock; ggml get_scale_min_k4,
//               kernels/iq3_mix.metal:13-23): B = q sc_g <= 945, so a
//               superblock accumulates in units of D = d 2^24.
//       IQ3_XXS w = d (0.5 + s_g) 0.5 grid sign (kernels/iq3_mix.metal:31-35):
//               B = (1 + 2 s_g) grid <= 31 * 62 with the sign, D = d 2^22.
//       IQ4_NL  w = d_g kv[q] (kernels/moe.metal:76-80): B = kv[q], |kv| <=
//               127, with the sign. d_g belongs to one 32-column block, so
//               each block's two MFMAs (A hi, A lo) start from zero and their
//               sum is added to the accumulator times d_g 2^24.
//   * The Q4_K mins term dmin sum_g mn_g S_g, with S_g = sum of a over the
//     group (precomputed per A row: gs [rows][kdim/32]), is one more MFMA per
//     superblock: A = (S hi, S lo) of the 8 groups, B = mn_g as subnormals.
//   * Between superblocks (Q4_K, IQ3_XXS) the accumulator moves from units
//     D_sb to D_sb+1: acc = acc D_sb / D_sb+1 (- macc Dmin_sb / D_sb+1 for
//     Q4_K; D = 1 for the true units after the last superblock; a zero d gives
//     D = 1 and zeroes B).
// Block = 2 waves, tile of 64 tokens x 128 rows; wave tile 64 x 64 (4 x 4
// MFMA tiles). Lane l owns B row (l % 16) of each 16-row block; which 8
// columns of a slab it feeds to MFMA gi depends on the format's byte order:
//   Q4_K    columns 32 gi + 8 (l / 16) .. + 7 (the slab's two groups are the
//           low and high nibbles of the same 8 bytes);
//   IQ3_XXS superblock columns 64 kq + 16 sq + 8 gi .. + 7 in slab sq
//           (kq = l / 16; grid bytes 16 kq + 4 sq + 2 gi, + 1), so that a lane
//           reads its 16 grid bytes and 2 sign/scale words once per superblock;
//           A is stored in the matching order (A_IQ3XXS) so that slab sq is one
//           contiguous run of 64 columns;
//   IQ4_NL  block gi, bytes 4 (l / 16) .. + 3, each holding values j (low
//           nibble) and j + 16 (high): the lane's 8 values are block columns
//           4 kq + i + 16 h at position 2 i + h; A is stored in that order
//           (A_IQ4NL).
//   The gate/up kernel writes act in the order of the down projection's
//   format; the dispatch launch's split blocks (split_f16_part) write x in
//   the order of gate/up's.
//   GATEUP: block b covers act columns 64 b..+63; wave w gate and up rows
//   64 b + 32 w ..+31 (n-blocks 0,1 gate, 2,3 up). Writes act = SwiGLU split
//   into out_h/out_l [P][F] and, for a Q4_K down projection, its 32-column
//   sums out_gs [P][F/32].
//   !GATEUP: block b covers rows 128 b..+127, wave w rows 128 b + 64 w..+63;
//   writes fp32 Y [P][ldo].
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef short short2v __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Column orders of an A operand (x split, act) in HBM; a_pos maps a column to
// its stored position.
//   A_IQ4NL: within each 32-column group, column 4 kq + i + 16 h -> 8 kq + 2 i + h
//     (kq, i < 4; h < 2): a lane's 4 IQ4_NL bytes hold these 8 values.
//   A_IQ3XXS: within each 256-column superblock, the 16-column pieces are
//     transposed, column 64 kq + 16 sq + j -> 64 sq + 16 kq + j (kq, sq < 4):
//     lane kq reads its grid bytes 16 kq .. +15 once per superblock and uses
//     4 of them (16 columns) in slab sq, so slab sq's A is one contiguous run.
//   A_F32: act in natural order as fp32 (out), for a down projection that
//     runs on the fp32 GEMM (a format without an f16 path).
//   A_Q6K: bits 5 and 6 of the column index swapped, column 128 n + 64 g +
//     32 p + c -> 128 n + 64 p + 32 g + c (c < 32): slab 2 n + p of a Q6_K
//     superblock holds the low-nibble and high-nibble columns of its ql bytes.
enum : int { A_NATURAL = 0, A_IQ4NL = 1, A_IQ3XXS = 2, A_F32 = 3, A_Q6K = 4 };
template <int ORD>
__device__ __forceinline__ uint32_t a_pos(uint32_t c) {
    if constexpr (ORD == A_IQ4NL) {
        const uint32_t k = c & 31u;
        return (c & ~31u) | (8u * ((k & 15u) >> 2) + 2u * (k & 3u) + (k >> 4));
    } else if constexpr (ORD == A_IQ3XXS) {
        return (c & ~255u) | (((c >> 4) & 3u) << 6) | (((c >> 6) & 3u) << 4) | (c & 15u);
    } else if constexpr (ORD == A_Q6K) {
        return (c & ~96u) | (((c >> 5) & 1u) << 6) | (((c >> 6) & 1u) << 5);
    }
    return c;
}

__device__ __forceinline__ void split_f16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Integer scales and mins of a Q4_K superblock header {d, dmin, scales[12]}:
// byte j of sc03/mn03 holds sc_j/mn_j for j < 4, of sc47/mn47 for j + 4.
__device__ __forceinline__ void q4k_sc_mn(uint4 h, uint32_t& sc03, uint32_t& sc47, uint32_t& mn03, uint32_t& mn47) {
    sc03 = h.y & 0x3f3f3f3fu;
    mn03 = h.z & 0x3f3f3f3fu;
    sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    mn47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
}

// Bytes 0,1 and 2,3 of w as two u16 pairs (perm selector 0x0c = zero byte).
__device__ __forceinline__ uint32_t bytes01(uint32_t w) { return __builtin_amdgcn_perm(0u, w, 0x0c010c00u); }
__device__ __forceinline__ uint32_t bytes23(uint32_t w) { return __builtin_amdgcn_perm(0u, w, 0x0c030c02u); }

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ uint32_t mul_u16x2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2v, a) * __builtin_bit_cast(short2v, b));
}
// a * b + c per 16-bit half (the products used here stay below 0x8000, so a
// c of sign bits is an OR).
__device__ __forceinline__ uint32_t mad_u16x2(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2v, a) * __builtin_bit_cast(short2v, b) +
                                            __builtin_bit_cast(short2v, c));
}

// 8 nibbles (already masked to 0x0f0f0f0f in lo4/hi4 bytes) times the
// replicated scale scl2 = sc | sc << 16 -> half8 of subnormal f16 bits.
__device__ __forceinline__ half8 q4_operand(uint32_t b0, uint32_t b1, uint32_t scl2) {
    const uint4 v = make_uint4(mul_u16x2(bytes01(b0), scl2), mul_u16x2(bytes23(b0), scl2), mul_u16x2(bytes01(b1), scl2),
                               mul_u16x2(bytes23(b1), scl2));
    return __builtin_bit_cast(half8, v);
}

constexpr uint32_t TM16 = 64;  // tokens per tile of the f16 GEMM

// Tiled weight layout of the f16 GEMM (k_tile_weights): a matrix's rows in
// groups of 16 (a B row block), each group's 16 rows of bytes (16 x the row
// stride, the same span as in GGUF order) rearranged into records, one per
// superblock (IQ4_NL: per 64-column slab), in which each load
// instruction of the GEMM reads one contiguous span: lane l = 16 kq + ln
// (row ln of the group, column quarter kq) finds its bytes at l times their
// size. Record bytes:
//   Q4_K (2304 per superblock): the 16 rows' 16-byte headers {d, dmin,
//     scales} at 16 ln; then per slab sq = 0..3 of the superblock, at
//     256 + 512 sq + 8 l, the 8 nibble bytes 16 + 32 sq + 8 kq .. + 7 of row ln.
//   IQ3_XXS (1568 per superblock): at 16 l the 16 grid-index bytes
//     2 + 16 kq .. + 15 of row ln; at 1024 + 8 l its aux words 66 + 8 kq .. + 7;
//     at 1536 + 2 ln the row's d.
//   IQ4_NL (576 per slab of two 18-byte blocks): at 8 l the nibble bytes
//     2 + 4 kq .. + 3 of the slab's first block, then those of its second;
//     at 512 + 4 ln the row's two d.
constexpr uint32_t TILE_Q4K = 2304, TILE_IQ3XXS = 1568, TILE_IQ4NL = 576;
//   Q5_K (2816): headers as Q4_K; at 256 + 8 l the qh bytes 16 + 8 kq .. + 7
//     of row ln; per slab, at 768 + 512 sq + 8 l, the nibble bytes
//     48 + 32 sq + 8 kq .. + 7.
//   IQ2_XS (1184): at 16 l the codes 2 + 16 kq .. + 15 of row ln; at
//     1024 + 8 ln the row's 8 scale bytes; at 1152 + 2 ln its d.
//   IQ2_S (1312): at 16 l the index bytes 2 + 8 kq .. + 7 of row ln, then its
//     sign bytes 34 + 8 kq .. + 7; at 1024 + 4 l the qh bytes 66 + 2 kq, + 1
//     and the scale bytes 74 + 2 kq, + 1; at 1280 + 2 ln the row's d.
//   IQ3_S (1760): at 16 l the grid-index bytes 2 + 16 kq .. + 15 of row ln;
//     at 1024 + 8 l its sign bytes 74 + 8 kq .. + 7; at 1536 + 12 ln the row's
//     8 qh bytes and 4 scale bytes; at 1728 + 2 ln its d.
//   IQ4_XS (2176): per slab sq, at 512 sq + 8 l the nibble bytes 4 kq .. + 3
//     of blocks 2 sq and 2 sq + 1 of row ln; at 2048 + 8 ln the row's d,
//     scales_h and scales_l.
//   Q6_K (3360): per slab sq, at 512 sq + 8 l the ql bytes
//     64 (sq / 2) + 32 (sq % 2) + 8 kq .. + 7 of row ln; per half n, at
//     2048 + 512 n + 8 l its qh bytes 128 + 32 n + 8 kq .. + 7; at 3072 + 16 ln
//     the row's 16 scale bytes; at 3328 + 2 ln its d.
constexpr uint32_t TILE_Q5K = 2816, TILE_IQ2XS = 1184, TILE_IQ2S = 1312, TILE_IQ3S = 1760, TILE_IQ4XS = 2176,
                   TILE_Q6K = 3360;
__host__ __device__ constexpr uint32_t tile_record(int kind) {
    return kind == 12   ? TILE_Q4K
           : kind == 13 ? TILE_Q5K
           : kind == 14 ? TILE_Q6K
           : kind == 17 ? TILE_IQ2XS
           : kind == 18 ? TILE_IQ3XXS
           : kind == 20 ? TILE_IQ4NL
           : kind == 21 ? TILE_IQ3S
           : kind == 22 ? TILE_IQ2S
           : kind == 23 ? TILE_IQ4XS
                        : 0u;
}

// Raw buffer access: base and size in a buffer resource (scalar registers),
// per-lane byte offset in a vector register, uniform byte offset in a scalar
// register; reads past `bytes` return zero. Word 3 is the gfx9 raw-buffer
// configuration (no format conversion).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt fields at their maxima).
template <uint32_t N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15u) | ((N >> 4) << 14));
}

// Grouped GEMM on f16 MFMA for Q4_K, IQ3_XXS and IQ4_NL weights (see the
// block comment above). e_shared names the tile expert id whose weights are
// ws0/ws1 (the shared expert, run in the same launch); no tile carries it when
// it is 0xffffffff. AORD (gate/up only) is the column order in which act is
// stored: the order the down projection's format reads (a_pos).
//   Pipeline. A slabs go straight from L2 to LDS (buffer_load ... lds; lane i
// of a load writes 16 bytes at M0 + 16 i), two buffers by slab parity, so A
// takes no registers. Per slab s: barrier; A(s + 1) into the other buffer, the
// B ring's loads, at a superblock's first slab the next header (these loads
// kept together and in this order); MFMAs of slab s with the operands decoded
// one slab earlier, and the decode of slab s + 1 (into a second operand set,
// interleaved with the MFMAs, when the tile has at most two row blocks; after
// them otherwise); at a superblock's end the mins and the unit change; then a
// wait for this wave's A(s + 1) only (vector-memory loads complete in issue
// order, so vmcnt counts the B loads issued after it), which the next barrier
// publishes. Every A DMA has landed before the block exits.
//   TT (tile tokens) 64: 2 waves; wave w owns B rows (gate/up: gate and up rows
// 32 w .. + 31 of the block's 64; down: rows 64 w .. + 63 of its 128) for all
// 64 tokens, as 4 x 4 MFMA tiles. TT 128 (tiles of up to 128 pairs, for
// batches in which an expert can take more than 64): 4 waves; wave w owns
// gate and up rows 16 w .. + 15 (down: rows 32 w .. + 31) for all 128 tokens,
// as 8 x 2 MFMA tiles. Each decoded B fragment then feeds 16 MFMAs instead of
// 8 and each weight byte is fetched once per 128 tokens instead of 64; the A
// slab (128 rows) is shared by the 4 waves through LDS.
//   TL: the weights are in the tiled layout of k_tile_weights, where each B
// load instruction reads one contiguous span
// (every lane the bytes it decodes) instead of 16 rows' scattered pieces.
template <int KIND, bool GATEUP, int AORD, int TT, bool TL = false>
__global__ __launch_bounds__(TT * 2) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_f16(
    const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, const uint8_t* __restrict__ ws0,
    const uint8_t* __restrict__ ws1, uint32_t e_shared, uint64_t stride0, uint64_t stride1, uint32_t rows_per_expert,
    uint32_t kdim, const _Float16* __restrict__ ah, const _Float16* __restrict__ al, const float* __restrict__ gs,
    const uint32_t* __restrict__ pairs, uint32_t K, const uint32_t* __restrict__ tiles, uint32_t ldo, float limit,
    float* __restrict__ out, _Float16* __restrict__ out_h, _Float16* __restrict__ out_l, float* __restrict__ out_gs,
    uint32_t nblk, uint32_t a_rows, const float* __restrict__ xstat, uint32_t* __restrict__ rowmax,
    uint32_t* __restrict__ flags, const uint32_t* __restrict__ slot_of) {
    static_assert(KIND == 12 || KIND == 13 || KIND == 14 || KIND == 17 || KIND == 18 || KIND == 20 || KIND == 21 ||
                      KIND == 22 || KIND == 23,
                  "f16 GEMM formats: Q4_K, Q5_K, Q6_K, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL, IQ4_XS");
    static_assert(AORD == A_NATURAL || GATEUP, "the permuted act layout is written by the gate/up kernel");
    static_assert(TT == 64 || TT == 128, "tiles of 64 or 128 tokens");
    // NB: 16-row B blocks per wave (gate/up: HB = NB / 2 gate, HB up); NW waves.
    constexpr int NB = TT == 128 ? 2 : 4;
    constexpr uint32_t NW = TT / 32u, HB = NB / 2;
    // Q5_K is Q4_K with a fifth bit per value (b[16 + k % 32] bit k / 32 of its
    // superblock, kernels/iq3_mix.metal:19-23): the same header, scales, mins
    // and operand build, nibbles 32 bytes later in a 176-byte superblock, and
    // a lane's 8 fifth-bit bytes (the same byte positions as its nibble bytes,
    // bits 2 sq and 2 sq + 1 for slab sq) loaded with each header. q * sc is at
    // most 31 * 63 = 1953, an exact f16 integer as for Q4_K.
    constexpr bool Q5K = KIND == 13, Q4K = KIND == 12 || Q5K, IQ3 = KIND == 18, IQ4 = KIND == 20;
    // IQ2_XS takes IQ3_XXS's path: 74-byte superblocks (2 bytes off a dword
    // every other one, like 98), lane kq's 16 bytes of 9+7-bit codes at
    // 2 + 16 kq (8 codes: 64 columns, two per slab, in A_IQ3XXS order), all 8
    // scale bytes at 66, d at 0. B = (1 + 2 s) * grid * sign <= 31 * 43, an
    // exact f16 integer, times the superblock's d / 8 (the unit d * 2^21).
    // IQ2_S too (82-byte superblocks): lane kq's 8 index bytes at 2 + 8 kq
    // and 8 sign bytes at 34 + 8 kq, the index high bits (66) and scales (74)
    // of its two 32-value groups among the 16 bytes at 66; B = (1 + 2 s) *
    // grid * sign <= 31 * 43 and the unit d * 2^21, as for IQ2_XS.
    // IQ3_S too (110-byte superblocks, kernels/moe.metal:65-75): lane kq's 16
    // grid-index bytes at 2 + 16 kq (as IQ3_XXS's grid bytes; 4-value entries
    // of the 512-entry grid), the ninth index bit from qh[2 kq], qh[2 kq + 1]
    // (66), its 8 sign bytes at 74 + 8 kq, the scale byte 106 + kq (a nibble per
    // 32-value group). B = (1 + 2 s) * grid * sign <= 31 * 15, unit d * 2^24.
    constexpr bool IQ2 = KIND == 17, IQ2S = KIND == 22, IQ3S = KIND == 21, IQG = IQ2 || IQ2S || IQ3 || IQ3S;
    // IQ4_XS takes IQ4_NL's path (B = the codebook value, a unit per 32-column
    // block): its blocks' 16 quant bytes sit at 8 + 16 g of a 136-byte
    // superblock (dword aligned), and a block's unit is d * (scale - 32), the
    // 6-bit scale from the 8-byte superblock header read with each slab.
    constexpr bool IQ4X = KIND == 23, IQN = IQ4 || IQ4X;
    // Q6_K (210-byte superblocks, kernels/moe.metal:22-28): w = d sc (q - 32),
    // q = 4 bits of ql | 2 bits of qh, sc an int8 per 16 columns; |sc (q - 32)|
    // reaches 4096, past the 2048 that f16 holds exactly, so B enters twice:
    // B_r = sc (q - 32) rounded to f16 (an integer, exact up to 2048, even
    // above) and B_e = sc (q - 32) - B_r in {-1, 0, 1} (one f16 fma, exact),
    // with MFMAs A hi x B_r, A hi x B_e, A lo x B_r (A lo x B_e is below 2^-22
    // of the product). B is integer-valued (no 2^-24 unit): D = d. Slab sq of a
    // superblock is half n = sq / 2, p = sq % 2; lane kq reads ql bytes
    // 64 n + 32 p + 8 kq .. + 7 (low nibbles: columns 128 n + 32 p + l, MFMA 0;
    // high: + 64, MFMA 1; l = 8 kq + j) and the qh bytes 32 n + 8 kq .. + 7 of
    // its half (once per half), so A is stored with bits 5 and 6 of each column
    // index swapped (A_Q6K). A lane's superblock may start 2 bytes off a dword
    // (210-byte superblocks, rows of any multiple of 256 columns): its loads
    // take the dword-aligned window and shift by 16 bits where it does (no
    // byte it uses sits in a dword past its superblock), and d comes from a
    // 16-bit load.
    constexpr bool Q6K = KIND == 14;
    // (two operand sets per fragment: TT 128's 2 row blocks per wave fit the registers, 4 do not)
    static_assert(!Q6K || TT == 128, "Q6_K runs on 128-token tiles (which also take tiles of 64)");
    constexpr uint32_t IQB = IQ2 ? 74u : IQ2S ? 82u : IQ3S ? 110u : Q6K ? 210u : 98u;
    constexpr uint32_t SBB = Q5K ? 176u : 144u, QOFF = Q5K ? 48u : 16u;
    // tiled record bytes (per superblock; IQ4_NL: per slab)
    constexpr uint32_t TREC = tile_record(KIND);
    constexpr uint32_t UNR = 4u;
    // A slab buffers (hi, lo; by slab parity): 64 halves (128 B) per token row,
    // 16-byte chunk c of row r at slot c ^ ((r >> 1) & 7), so that the fragment
    // reads (16 rows at one chunk) touch every bank once. Separate objects, so
    // that the compiler sees that a DMA into one never aliases reads of the
    // other. S tiles (Q4_K group sums) by superblock parity.
    __shared__ _Float16 Ah0[TT * 64], Ah1[TT * 64], Al0[TT * 64], Al1[TT * 64];
    __shared__ _Float16 Ss[2][TT * 16];  // per row: S hi of groups 0..7, S lo of groups 0..7
    // Tile rounds of 8 (one tile per XCD) alternate direction: XCD x takes tile
    // 8 ti + x in even rounds and 8 ti + 7 - x in odd ones. The tiles come
    // sorted by decreasing size, so a fixed direction would give XCD 0 the
    // largest tile of every round (a dispatch simulation over C1's tiles with
    // measured block times: XCD spans 62-85 us against 70-76 us snaked;
    // measured: C1 gate/up about 1.4 us shorter, C3 gate/up 176-178 to
    // 169-170 us, C3 down 114-116 to 111-113).
    const uint32_t nt = tiles[3], slot = blockIdx.x >> 3, ti = slot / nblk, xcd = blockIdx.x & 7u;
    const uint32_t t = ti * 8u + ((ti & 1u) ? 7u - xcd : xcd);
    if (t >= nt) return;
    const uint32_t* tile = tiles + 4u * t;
    const uint32_t n = tile[2];
    if (n == 0) return;
    // Cached experts (slot_of != NULL, entry E for the shared expert's tiles):
    // the expert's weights are in slot slot_of[e], or it is not resident in this
    // pass (NO_SLOT) and the tile waits for a later one.
    const uint32_t ew = slot_of ? slot_of[tile[0]] : tile[0];
    if (ew == NO_SLOT) return;
    if constexpr (!Q4K && !Q6K) {
        stage_f16_tables<KIND>();
        __syncthreads();
    }
    const uint32_t e = tile[0], q0 = tile[1];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, kq = lane >> 4, ln = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t row0 = (slot - ti * nblk) * (GATEUP ? 64u : 128u);
    const uint32_t ngroups = kdim / 32u;

    // A DMA: instruction i of wave w fills tile rows 8 (NW i + w) .. + 7; lane l
    // writes row r = 8 (NW i + w) + l / 8 at LDS slot l % 8, which holds chunk
    // (l % 8) ^ ((r >> 1) & 7) of the row (the swizzle of the fragment reads).
    uint32_t avo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = 8u * (NW * i + wave) + (lane >> 3);
        const uint32_t q = q0 + (r < n ? r : 0u);
        const uint32_t arow = GATEUP ? (pairs ? pairs[q] / K : q) : q;
        avo[i] = 2u * (arow * kdim + 8u * ((lane & 7u) ^ ((r >> 1) & 7u)));
    }
    const uint32_t am = tid >> 1, ahalf = tid & 1u;
    uint32_t soff = 0;
    if constexpr (Q4K) {
        const uint32_t q = q0 + (am < n ? am : 0u);
        const uint32_t r = GATEUP ? (pairs ? pairs[q] / K : q) : q;
        soff = 4u * (r * ngroups + 4u * ahalf);
    }
    // GATEUP: the split exponent e_t of each tile row's token and the units
    // exponent a_t of its activations, for the epilogue (published by the main
    // loop's first barrier). Down: row block 0 of each tile checks that its
    // activation rows were split in range.
    __shared__ int2 s_rowe[TT];
    // TT 128 gate/up: each wave's 16-column halves of the act group sums
    __shared__ float gpart[GATEUP && TT == 128 ? 4 : 1][TT];
    // gate/up: each wave's maximum of |act| over its columns of a row, reduced
    // over the NW waves before one atomicMax per row and block (one per wave
    // before: C1 gate/up 86.2-86.6 to 81.9-85.7 us, the Q4_K/Q6_K mix at 512
    // tokens 111.8-114.3 to 101.6-105.1)
    __shared__ uint32_t rpart[GATEUP ? NW : 1][TT];
    if constexpr (GATEUP) {
        if (tid < TT) {
            const uint32_t q = q0 + (tid < n ? tid : 0u);
            const float2 st = ld_xstat(xstat, pairs ? pairs[q] / K : q);
            s_rowe[tid] = make_int2(x_exp(st.x), act_exp(st));
        }
    } else {
        if (rowmax != nullptr && slot - ti * nblk == 0u) {
            bool bad = false;
            if (tid < n) {
                const float m = __uint_as_float(rowmax[q0 + tid]);
                bad = !(m == 0.f || (m >= ACT_RANGE_LO && m < ACT_RANGE_HI));  // NaN: bad
            }
            if (__any(bad) && lane == 0u) atomicOr(flags, FLAG_RANGE);
        }
    }
    const bool sh_tile = e == e_shared;
    const uint8_t* const wb0 = sh_tile ? ws0 : w0 + (uint64_t)ew * rows_per_expert * stride0;
    const uint8_t* const wb1 = GATEUP ? (sh_tile ? ws1 : w1 + (uint64_t)ew * rows_per_expert * stride1) : wb0;
    const __amdgpu_buffer_rsrc_t ra_h = make_rsrc(ah, (uint32_t)(kdim * 2u) * a_rows);
    const __amdgpu_buffer_rsrc_t ra_l = make_rsrc(al, (uint32_t)(kdim * 2u) * a_rows);
    const __amdgpu_buffer_rsrc_t rgs = make_rsrc(gs, ngroups * 4u * a_rows);
    const __amdgpu_buffer_rsrc_t rw0 = make_rsrc(wb0, (uint32_t)(rows_per_expert * stride0));
    const __amdgpu_buffer_rsrc_t rw1 = GATEUP ? make_rsrc(wb1, (uint32_t)(rows_per_expert * stride1)) : rw0;
    uint32_t bsoff[NB], boff[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (GATEUP) {
            const uint32_t st = (uint32_t)(nb < (int)HB ? stride0 : stride1);
            bsoff[nb] = (row0 + 16u * HB * wave + 16u * (nb % HB)) * st;
            boff[nb] = ln * st;
        } else {
            bsoff[nb] = (row0 + 16u * NB * wave + 16u * nb) * (uint32_t)stride0;
            boff[nb] = ln * (uint32_t)stride0;
        }
    }
    const uint32_t slabs = kdim / 64u, sbs = kdim / 256u;
    // Q6_K: each lane's row start (bytes from the expert's base)
    uint32_t q6r[Q6K ? NB : 1];
    if constexpr (Q6K) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) q6r[nb] = bsoff[nb] + boff[nb];
    }

    float4 ps;
#define INGOT_LOAD_S(SB) ps = __builtin_bit_cast(float4, buf_load16(rgs, soff, 32u * ((SB) < sbs ? (SB) : sbs - 1u)))
    uint4 nhdr[NB];
    uint2 nqh[Q5K ? NB : 1];
    uint32_t n5[NB], n_d[NB];
    uint3 n3[NB], ns3[IQ2S ? NB : 1];
    uint4 nqh3[IQ3S ? NB : 1];  // IQ3_S: bytes 64 .. 79 (qh) and 104 .. 111 (scales) of the superblock's dword window
    uint2 nsc3[IQ3S ? NB : 1];
    auto load_hdr = [&](uint32_t sb) {
        sb = sb < sbs ? sb : sbs - 1u;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const __amdgpu_buffer_rsrc_t rw = GATEUP && nb >= (int)HB ? rw1 : rw0;
            if constexpr (TL && Q4K) nhdr[nb] = buf_load16(rw, 16u * ln, bsoff[nb] + sb * TREC);
            else if constexpr (Q4K) nhdr[nb] = buf_load16(rw, boff[nb], bsoff[nb] + sb * SBB);
            if constexpr (TL && Q5K) nqh[nb] = buf_load8(rw, 8u * lane, bsoff[nb] + sb * TREC + 256u);
            else if constexpr (Q5K) nqh[nb] = buf_load8(rw, boff[nb] + 8u * kq, bsoff[nb] + sb * SBB + 16u);
            if constexpr (TL && IQ2S) {
                const uint32_t u = bsoff[nb] + sb * TREC;
                const uint4 is = buf_load16(rw, 16u * lane, u);  // index bytes, sign bytes
                n3[nb] = make_uint3(is.x, is.y, 0u);
                ns3[nb] = make_uint3(is.z, is.w, 0u);
                nhdr[nb].x = buf_load4(rw, 4u * lane, u + 1024u);  // qh16 | sc16 << 16
                n_d[nb] = buf_load4(rw, 4u * (ln >> 1), u + 1280u);
            } else if constexpr (TL && IQ3S) {
                const uint32_t u = bsoff[nb] + sb * TREC;
                nhdr[nb] = buf_load16(rw, 16u * lane, u);  // grid-index bytes
                const uint2 g = buf_load8(rw, 8u * lane, u + 1024u);  // sign bytes
                n3[nb] = make_uint3(g.x, g.y, 0u);
                const auto h = __builtin_amdgcn_raw_buffer_load_b96(rw, (int)(12u * ln), (int)(u + 1536u), 0);
                nqh3[nb] = make_uint4(h[0], h[1], h[2], 0u);  // the row's qh bytes, scale bytes
                n_d[nb] = buf_load4(rw, 4u * (ln >> 1), u + 1728u);
            } else if constexpr (IQ2S) {
                const uint32_t u = (bsoff[nb] + sb * IQB) & ~3u;
                nhdr[nb] = buf_load16(rw, boff[nb], u + 64u);  // index high bits and scales
                n5[nb] = buf_load4(rw, boff[nb], u + 80u);
                const uint2 q = buf_load8(rw, boff[nb] + 8u * kq, u);
                n3[nb] = make_uint3(q.x, q.y, buf_load4(rw, boff[nb] + 8u * kq, u + 8u));
                const uint2 g = buf_load8(rw, boff[nb] + 8u * kq, u + 32u);
                ns3[nb] = make_uint3(g.x, g.y, buf_load4(rw, boff[nb] + 8u * kq, u + 40u));
                n_d[nb] = buf_load4(rw, boff[nb], u);
            } else if constexpr (IQ3S) {
                const uint32_t u = (bsoff[nb] + sb * IQB) & ~3u;
                nhdr[nb] = buf_load16(rw, boff[nb] + 16u * kq, u);  // grid-index bytes
                n5[nb] = buf_load4(rw, boff[nb] + 16u * kq, u + 16u);
                const uint2 g = buf_load8(rw, boff[nb] + 8u * kq, u + 72u);  // sign bytes
                n3[nb] = make_uint3(g.x, g.y, buf_load4(rw, boff[nb] + 8u * kq, u + 80u));
                nqh3[nb] = buf_load16(rw, boff[nb], u + 64u);
                nsc3[nb] = buf_load8(rw, boff[nb], u + 104u);
                n_d[nb] = buf_load4(rw, boff[nb], u);
            } else if constexpr (TL && (IQ3 || IQ2)) {
                // IQ3_XXS: the lane's grid-index bytes and aux words, the row's d;
                // IQ2_XS: the lane's codes, the row's 8 scale bytes and d
                const uint32_t u = bsoff[nb] + sb * TREC;
                nhdr[nb] = buf_load16(rw, 16u * lane, u);
                const uint2 a = buf_load8(rw, IQ3 ? 8u * lane : 8u * ln, u + 1024u);
                n3[nb] = make_uint3(a.x, a.y, 0u);
                n_d[nb] = buf_load4(rw, 4u * (ln >> 1), u + (IQ3 ? 1536u : 1152u));
            } else if constexpr (IQG) {
                const uint32_t u = (bsoff[nb] + sb * IQB) & ~3u;
                nhdr[nb] = buf_load16(rw, boff[nb] + 16u * kq, u);
                n5[nb] = buf_load4(rw, boff[nb] + 16u * kq, u + 16u);
                // IQ3_XXS: the lane's two aux words at 66 + 8 kq; IQ2_XS: all 8 scale bytes at 66.
                const uint32_t ao = IQ2 ? boff[nb] : boff[nb] + 8u * kq;
                const uint2 a = buf_load8(rw, ao, u + 64u);
                n3[nb] = make_uint3(a.x, a.y, buf_load4(rw, ao, u + 72u));
                n_d[nb] = buf_load4(rw, boff[nb], u);
            } else if constexpr (TL && Q6K) {
                const uint32_t u = bsoff[nb] + sb * TREC;
                nhdr[nb] = buf_load16(rw, 16u * ln, u + 3072u);  // the row's 16 scale bytes
                n5[nb] = 0u;
                n_d[nb] = buf_load4(rw, 4u * (ln >> 1), u + 3328u);
            } else if constexpr (Q6K) {
                // the 16 scale bytes (192) in a 20-byte window, d (208)
                const uint32_t b = q6r[nb] + sb * IQB, a = b & ~3u;
                nhdr[nb] = buf_load16(rw, a, 192u);
                n5[nb] = buf_load4(rw, a, 208u);
                n_d[nb] = __builtin_amdgcn_raw_buffer_load_b16(rw, (int)b, 208, 0);
            }
        }
    };
    uint4 nq[4][NB];
    uint32_t n1[4][NB];
    uint2 nd[4][NB];
    // Q6_K: ev (the slab is the first of its half, a compile-time constant at
    // each call) also loads the half's qh window.
    auto load_slab = [&](uint32_t rs, uint32_t s, bool ev = false) {
        s = s < slabs ? s : slabs - 1u;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const __amdgpu_buffer_rsrc_t rw = GATEUP && nb >= (int)HB ? rw1 : rw0;
            if constexpr (TL && Q6K) {
                // ql bytes of the slab, and at a half's first slab its qh bytes
                const uint32_t u = bsoff[nb] + (s >> 2) * TREC, hn = (s >> 1) & 1u;
                const uint2 l = buf_load8(rw, 8u * lane, u + 512u * (s & 3u));
                nq[rs][nb].x = l.x;
                nq[rs][nb].y = l.y;
                nq[rs][nb].z = 0u;
                if (ev) {
                    const uint2 h = buf_load8(rw, 8u * lane, u + 2048u + 512u * hn);
                    nq[rs][nb].w = h.x;
                    nd[rs][nb] = make_uint2(h.y, 0u);
                }
            } else if constexpr (Q6K) {
                const uint32_t a = (q6r[nb] + 8u * kq + (s >> 2) * IQB) & ~3u, hn = (s >> 1) & 1u;
                const auto l = __builtin_amdgcn_raw_buffer_load_b96(rw, (int)a, (int)(64u * hn + 32u * (s & 1u)), 0);
                nq[rs][nb].x = l[0];
                nq[rs][nb].y = l[1];
                nq[rs][nb].z = l[2];
                if (ev) {
                    const auto h = __builtin_amdgcn_raw_buffer_load_b96(rw, (int)a, (int)(128u + 32u * hn), 0);
                    nq[rs][nb].w = h[0];
                    nd[rs][nb] = make_uint2(h[1], h[2]);
                }
            } else if constexpr (TL && Q4K) {
                const uint2 v = buf_load8(rw, 8u * lane, bsoff[nb] + (s >> 2) * TREC + (Q5K ? 768u : 256u) + 512u * (s & 3u));
                nq[rs][nb].x = v.x;
                nq[rs][nb].y = v.y;
            } else if constexpr (Q4K) {
                const uint2 v = buf_load8(rw, boff[nb] + 8u * kq, bsoff[nb] + (s >> 2) * SBB + QOFF + 32u * (s & 3u));
                nq[rs][nb].x = v.x;
                nq[rs][nb].y = v.y;
            } else if constexpr (TL && IQ4X) {
                const uint32_t u = bsoff[nb] + (s >> 2) * TREC;
                const uint2 q = buf_load8(rw, 8u * lane, u + 512u * (s & 3u));
                nq[rs][nb].x = q.x;
                n1[rs][nb] = q.y;
                nd[rs][nb] = buf_load8(rw, 8u * ln, u + 2048u);
            } else if constexpr (IQ4X) {
                const uint32_t u = bsoff[nb] + (s >> 2) * 136u, g0 = 2u * (s & 3u);
                nq[rs][nb].x = buf_load4(rw, boff[nb] + 4u * kq, u + 8u + 16u * g0);
                n1[rs][nb] = buf_load4(rw, boff[nb] + 4u * kq, u + 24u + 16u * g0);
                nd[rs][nb] = buf_load8(rw, boff[nb], u);
            } else if constexpr (TL && IQ4) {
                // qa, qb (the two blocks' nibble words) and the row's d0 | d1 << 16
                const uint32_t u = bsoff[nb] + TREC * s;
                const uint2 q = buf_load8(rw, 8u * lane, u);
                nq[rs][nb].x = q.x;
                nq[rs][nb].y = q.y;
                n1[rs][nb] = q.y;
                const uint32_t dw = buf_load4(rw, 4u * ln, u + 512u);
                nd[rs][nb] = make_uint2(dw, dw);
            } else if constexpr (IQ4) {
                const uint32_t u = bsoff[nb] + 36u * s;
                const uint2 q = buf_load8(rw, boff[nb] + 4u * kq, u);
                nq[rs][nb].x = q.x;
                nq[rs][nb].y = q.y;
                n1[rs][nb] = buf_load4(rw, boff[nb] + 4u * kq, u + 20u);
                nd[rs][nb] = make_uint2(buf_load4(rw, boff[nb], u), buf_load4(rw, boff[nb], u + 16u));
            }
        }
    };
    auto dbits = [&](int nb, uint32_t sb) -> uint32_t {
        if constexpr (TL && IQG) return (ln & 1u) ? n_d[nb] >> 16 : n_d[nb];
        if constexpr (IQG) return (sb & 1u) ? n_d[nb] >> 16 : n_d[nb];
        if constexpr (TL && Q6K) return ((ln & 1u) ? n_d[nb] >> 16 : n_d[nb]) & 0xffffu;
        if constexpr (Q6K) return n_d[nb];
        return nhdr[nb].x;
    };
    auto unit = [](uint32_t bits) {
        const float d = half_bits_to_float(bits);
        return d != 0.f ? d * ((IQ2 || IQ2S) ? 2097152.f : IQ3 ? 4194304.f : Q6K ? 1.f : 16777216.f) : 1.f;
    };
    // Superblock state for the decode (and, at the superblock's end, the mins
    // and the unit change).
    struct SbState {
        uint32_t sc[NB][2], mn[NB][2];
        uint2 qh[Q5K ? NB : 1];
        uint32_t gw[NB][4], aw[NB][2];
        float dsc[NB], dmn[NB];
        uint32_t sh[Q6K ? NB : 1];  // Q6_K: the lane's superblock misalignment in bits (0 or 16)
    };
    auto take_hdr = [&](SbState& st, uint32_t sb) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint32_t db = dbits(nb, sb);
            st.dsc[nb] = unit(db);
            if constexpr (Q4K) {
                q4k_sc_mn(nhdr[nb], st.sc[nb][0], st.sc[nb][1], st.mn[nb][0], st.mn[nb][1]);
                if constexpr (Q5K) st.qh[nb] = nqh[nb];
                // dmin 2^24, times 32: the group sums enter the MFMA divided by 32
                st.dmn[nb] = half_bits_to_float(nhdr[nb].x >> 16) * 536870912.f;
                if (half_bits_to_float(nhdr[nb].x) == 0.f) st.sc[nb][0] = st.sc[nb][1] = 0u;
            } else if constexpr (TL && IQ2S) {
                st.gw[nb][0] = n3[nb].x;
                st.gw[nb][1] = n3[nb].y;
                st.gw[nb][2] = ns3[nb].x;
                st.gw[nb][3] = ns3[nb].y;
                st.aw[nb][0] = nhdr[nb].x;
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (TL && IQ3S) {
                st.gw[nb][0] = nhdr[nb].x;
                st.gw[nb][1] = nhdr[nb].y;
                st.gw[nb][2] = nhdr[nb].z;
                st.gw[nb][3] = nhdr[nb].w;
                st.aw[nb][0] = n3[nb].x;
                st.aw[nb][1] = n3[nb].y;
                const uint32_t qh16 = ((kq < 2u ? nqh3[nb].x : nqh3[nb].y) >> (16u * (kq & 1u))) & 0xffffu;
                const uint32_t sc8 = (nqh3[nb].z >> (8u * kq)) & 255u;
                st.mn[nb][0] = qh16 | (sc8 << 16);
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (IQ2S) {
                // gw: the lane's index words (0, 1) and sign words (2, 3);
                // aw[0]: index high-bit bytes of its groups 2 kq, 2 kq + 1 in
                // bits 0..15, their scale bytes in bits 16..31.
                const bool odd = (sb & 1u) != 0u;
                auto al = [&](uint32_t hi, uint32_t lo) { return odd ? hi : __builtin_amdgcn_alignbit(hi, lo, 16u); };
                st.gw[nb][0] = al(n3[nb].y, n3[nb].x);
                st.gw[nb][1] = al(n3[nb].z, n3[nb].y);
                st.gw[nb][2] = al(ns3[nb].y, ns3[nb].x);
                st.gw[nb][3] = al(ns3[nb].z, ns3[nb].y);
                const uint32_t w[5] = {nhdr[nb].x, nhdr[nb].y, nhdr[nb].z, nhdr[nb].w, n5[nb]};
                uint32_t h[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) h[i] = al(w[i + 1], w[i]);
                const uint32_t sh = 16u * (kq & 1u);
                const uint32_t qh16 = ((kq < 2u ? h[0] : h[1]) >> sh) & 0xffffu;
                const uint32_t sc16 = ((kq < 2u ? h[2] : h[3]) >> sh) & 0xffffu;
                st.aw[nb][0] = qh16 | (sc16 << 16);
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (IQ3S) {
                // gw: the lane's 16 grid-index bytes; aw: its 8 sign bytes; mn[0]:
                // qh[2 kq], qh[2 kq + 1] in bits 0..15 and the scale byte in 16..23.
                const bool odd = (sb & 1u) != 0u;
                auto al = [&](uint32_t hi, uint32_t lo) { return odd ? hi : __builtin_amdgcn_alignbit(hi, lo, 16u); };
                const uint32_t w[5] = {nhdr[nb].x, nhdr[nb].y, nhdr[nb].z, nhdr[nb].w, n5[nb]};
#pragma unroll
                for (int i = 0; i < 4; ++i) st.gw[nb][i] = al(w[i + 1], w[i]);
                st.aw[nb][0] = al(n3[nb].y, n3[nb].x);
                st.aw[nb][1] = al(n3[nb].z, n3[nb].y);
                const uint32_t h0 = al(nqh3[nb].y, nqh3[nb].x), h1 = al(nqh3[nb].z, nqh3[nb].y);
                const uint32_t qh16 = ((kq < 2u ? h0 : h1) >> (16u * (kq & 1u))) & 0xffffu;
                const uint32_t sc8 = (al(nsc3[nb].y, nsc3[nb].x) >> (8u * kq)) & 255u;
                st.mn[nb][0] = qh16 | (sc8 << 16);
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (TL && (IQ3 || IQ2)) {
                st.gw[nb][0] = nhdr[nb].x;
                st.gw[nb][1] = nhdr[nb].y;
                st.gw[nb][2] = nhdr[nb].z;
                st.gw[nb][3] = nhdr[nb].w;
                st.aw[nb][0] = n3[nb].x;
                st.aw[nb][1] = n3[nb].y;
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (IQG) {
                const bool odd = (sb & 1u) != 0u;
                const uint32_t w[5] = {nhdr[nb].x, nhdr[nb].y, nhdr[nb].z, nhdr[nb].w, n5[nb]};
                const uint32_t v[3] = {n3[nb].x, n3[nb].y, n3[nb].z};
#pragma unroll
                for (int i = 0; i < 4; ++i) st.gw[nb][i] = odd ? w[i + 1] : __builtin_amdgcn_alignbit(w[i + 1], w[i], 16u);
#pragma unroll
                for (int i = 0; i < 2; ++i) st.aw[nb][i] = odd ? v[i + 1] : __builtin_amdgcn_alignbit(v[i + 1], v[i], 16u);
                st.sc[nb][0] = half_bits_to_float(db) == 0.f ? 0u : 1u;
            } else if constexpr (Q6K) {
                // gw: the 16 int8 scales (zero with d, which zeroes B)
                st.sh[nb] = TL ? 0u : ((q6r[nb] + sb * IQB) & 2u) << 3;
                const uint32_t w[5] = {nhdr[nb].x, nhdr[nb].y, nhdr[nb].z, nhdr[nb].w, n5[nb]};
                const bool z = half_bits_to_float(db) == 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) st.gw[nb][i] = z ? 0u : __builtin_amdgcn_alignbit(w[i + 1], w[i], st.sh[nb]);
            }
        }
    };
    // Q6_K: the qh words of the half being decoded (set at its first slab), and
    // the perm selector of the lane's two scale bytes (byte kq / 2 of scale
    // words 2 n, 2 n + 1; + 2 in a half's second slab).
    uint2 qhc[Q6K ? NB : 1];
    const uint32_t q6sel = 0x0c040c00u + (kq >> 1) * 0x00010001u;
    // Decode of slab position sq (within its superblock) into fb (Q6_K: B_r
    // into fb, B_e into fe); IQ4_NL also yields the units of its two blocks and
    // whether a d is zero.
    auto decode = [&](const SbState& st, uint32_t sq, const uint4* qv, const uint2* dv, half8 (*fb)[2],
                      float (*dg)[2], half8 (*fe)[2]) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if constexpr (Q6K) {
                const uint32_t p = sq & 1u, hn = sq >> 1;
                if (p == 0u)
                    qhc[nb] = make_uint2(__builtin_amdgcn_alignbit(dv[nb].x, qv[nb].w, st.sh[nb]),
                                         __builtin_amdgcn_alignbit(dv[nb].y, dv[nb].x, st.sh[nb]));
                const uint32_t L[2] = {__builtin_amdgcn_alignbit(qv[nb].y, qv[nb].x, st.sh[nb]),
                                       __builtin_amdgcn_alignbit(qv[nb].z, qv[nb].y, st.sh[nb])};
                const uint32_t H[2] = {qhc[nb].x, qhc[nb].y};
                // int8 scale b -> f16 bits 0x6400 | (b ^ 0x80) = 1152 + sc
                const uint32_t scw = __builtin_amdgcn_perm(st.gw[nb][2u * hn + 1u], st.gw[nb][2u * hn],
                                                           q6sel + 0x00020002u * p) ^ 0x64806480u;
                const half2v sc = __builtin_bit_cast(half2v, scw) - half2v{(_Float16)1152.f, (_Float16)1152.f};
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const half2v s = gi ? __builtin_shufflevector(sc, sc, 1, 1) : __builtin_shufflevector(sc, sc, 0, 0);
                    uint32_t r[4], e[4];
#pragma unroll
                    for (int w = 0; w < 2; ++w) {
                        // 6-bit q of the 4 values: nibble gi of the ql bytes, qh bits 2 (p + 2 gi) + 0, 1
                        const uint32_t q = gi ? ((L[w] >> 4) & 0x0f0f0f0fu) | ((H[w] >> (2u * p)) & 0x30303030u)
                                              : (L[w] & 0x0f0f0f0fu) | ((H[w] << (4u - 2u * p)) & 0x30303030u);
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            // f16 bits 0x6400 | q = 1024 + q, minus 1056: q - 32
                            const uint32_t x = __builtin_amdgcn_perm(0x64646464u, q, hh ? 0x04030402u : 0x04010400u);
                            const half2v v = __builtin_bit_cast(half2v, x) - half2v{(_Float16)1056.f, (_Float16)1056.f};
                            const half2v br = v * s;
                            const half2v be = __builtin_elementwise_fma(v, s, -br);
                            r[2 * w + hh] = __builtin_bit_cast(uint32_t, br);
                            e[2 * w + hh] = __builtin_bit_cast(uint32_t, be);
                        }
                    }
                    fb[nb][gi] = __builtin_bit_cast(half8, make_uint4(r[0], r[1], r[2], r[3]));
                    fe[nb][gi] = __builtin_bit_cast(half8, make_uint4(e[0], e[1], e[2], e[3]));
                }
            } else if constexpr (Q4K) {
                const uint32_t scw = st.sc[nb][sq >> 1] >> (16u * (sq & 1u));
                const uint32_t s0_ = __builtin_amdgcn_perm(0u, scw, 0x0c000c00u);
                const uint32_t s1_ = __builtin_amdgcn_perm(0u, scw, 0x0c010c01u);
                uint32_t lx = qv[nb].x & 0x0f0f0f0fu, ly = qv[nb].y & 0x0f0f0f0fu;
                uint32_t hx = (qv[nb].x >> 4) & 0x0f0f0f0fu, hy = (qv[nb].y >> 4) & 0x0f0f0f0fu;
                if constexpr (Q5K) {
                    const uint32_t b0 = 2u * sq;
                    lx |= ((st.qh[nb].x >> b0) & 0x01010101u) << 4;
                    ly |= ((st.qh[nb].y >> b0) & 0x01010101u) << 4;
                    hx |= ((st.qh[nb].x >> (b0 + 1u)) & 0x01010101u) << 4;
                    hy |= ((st.qh[nb].y >> (b0 + 1u)) & 0x01010101u) << 4;
                }
                fb[nb][0] = q4_operand(lx, ly, s0_);
                fb[nb][1] = q4_operand(hx, hy, s1_);
            } else if constexpr (IQ2S) {
                // codes 8 kq + 2 sq + gi: byte l = 2 (sq & 1) + gi of index
                // and sign word sq / 2, group 2 kq + sq / 2.
                const uint32_t grp = sq >> 1;
                const uint32_t qsw = st.gw[nb][grp], sgw = st.gw[nb][2u + grp];
                const uint32_t qh = (st.aw[nb][0] >> (8u * grp)) & 255u;
                const uint32_t sc = (st.aw[nb][0] >> (16u + 8u * grp)) & 255u;
                const uint32_t f = st.sc[nb][0] * (2u * ((sc >> (4u * (sq & 1u))) & 15u) + 1u);
                const uint32_t f2 = f | (f << 16);
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const uint32_t l = 2u * (sq & 1u) + (uint32_t)gi;
                    const uint32_t idx = ((qsw >> (8u * l)) & 255u) | (((qh >> (2u * l)) & 3u) << 8);
                    const uint64_t e = lds_iq2s_grid()[idx];
                    const uint4 m = lds_sign8mask()[(sgw >> (8u * l)) & 255u];
                    const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
                    fb[nb][gi] = __builtin_bit_cast(
                        half8, make_uint4(mad_u16x2(bytes01(lo), f2, m.x), mad_u16x2(bytes23(lo), f2, m.y),
                                          mad_u16x2(bytes01(hi), f2, m.z), mad_u16x2(bytes23(hi), f2, m.w)));
                }
            } else if constexpr (IQ3S) {
                // group 2 kq + sq / 2 of the superblock, its 8-value pieces l = 2 (sq & 1) + gi
                const uint32_t gq = sq >> 1, x = st.mn[nb][0];
                const uint32_t qh8 = (x >> (8u * gq)) & 255u;
                const uint32_t f = st.sc[nb][0] * (2u * ((x >> (16u + 4u * gq)) & 15u) + 1u);
                const uint32_t f2 = f | (f << 16);
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const uint32_t l = 2u * (sq & 1u) + (uint32_t)gi;
                    const uint32_t wq = st.gw[nb][2u * gq + (l >> 1)] >> (16u * (l & 1u));
                    const uint32_t i0 = (wq & 255u) | (((qh8 >> (2u * l)) & 1u) << 8);
                    const uint32_t i1 = ((wq >> 8) & 255u) | (((qh8 >> (2u * l + 1u)) & 1u) << 8);
                    const uint32_t e0 = lds_iq3s_grid()[i0], e1 = lds_iq3s_grid()[i1];
                    const uint4 m = lds_sign8mask()[(st.aw[nb][gq] >> (8u * l)) & 255u];
                    fb[nb][gi] = __builtin_bit_cast(
                        half8, make_uint4(mad_u16x2(bytes01(e0), f2, m.x), mad_u16x2(bytes23(e0), f2, m.y),
                                          mad_u16x2(bytes01(e1), f2, m.z), mad_u16x2(bytes23(e1), f2, m.w)));
                }
            } else if constexpr (IQ2) {
                const uint32_t g = st.gw[nb][sq];  // codes 8 kq + 2 sq (low half) and + 1
                const uint32_t sw = (kq < 2u ? st.aw[nb][0] : st.aw[nb][1]) >> (16u * (kq & 1u));
                const uint32_t f = st.sc[nb][0] * (2u * ((sw >> (8u * (sq >> 1) + 4u * (sq & 1u))) & 15u) + 1u);
                const uint32_t f2 = f | (f << 16);
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const uint32_t code = (g >> (16 * gi)) & 0xffffu;
                    const uint64_t e = lds_iq2xs_grid()[code & 511u];
                    const uint4 m = lds_iq3_signmask()[code >> 9];
                    const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
                    fb[nb][gi] = __builtin_bit_cast(
                        half8, make_uint4(mad_u16x2(bytes01(lo), f2, m.x), mad_u16x2(bytes23(lo), f2, m.y),
                                          mad_u16x2(bytes01(hi), f2, m.z), mad_u16x2(bytes23(hi), f2, m.w)));
                }
            } else if constexpr (IQ3) {
                const uint32_t g = st.gw[nb][sq];
                const uint32_t x = st.aw[nb][sq >> 1];
                const uint32_t f = st.sc[nb][0] * (2u * (x >> 28) + 1u);
                const uint32_t f2 = f | (f << 16);
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const uint4 m = lds_iq3_signmask()[(x >> (14u * (sq & 1u) + 7u * gi)) & 127u];
                    const uint2 e0 = lds_iq3xxs_grid_u16()[(g >> (16 * gi)) & 255u];
                    const uint2 e1 = lds_iq3xxs_grid_u16()[(g >> (16 * gi + 8)) & 255u];
                    fb[nb][gi] = __builtin_bit_cast(
                        half8, make_uint4(mad_u16x2(e0.x, f2, m.x), mad_u16x2(e0.y, f2, m.y),
                                          mad_u16x2(e1.x, f2, m.z), mad_u16x2(e1.y, f2, m.w)));
                }
            } else {
                uint32_t qa, qb;
                float d0, d1;
                if constexpr (IQ4X) {
                    qa = qv[nb].x;
                    qb = qv[nb].z;
                    const float d = half_bits_to_float(dv[nb].x);
                    const uint32_t g0 = 2u * sq, sh = dv[nb].x >> 16, sl = (dv[nb].y >> (8u * sq)) & 255u;
                    const int s0 = (int)((sl & 15u) | (((sh >> (2u * g0)) & 3u) << 4)) - 32;
                    const int s1 = (int)((sl >> 4) | (((sh >> (2u * g0 + 2u)) & 3u) << 4)) - 32;
                    d0 = d * (float)s0;
                    d1 = d * (float)s1;
                } else {
                    qa = TL ? qv[nb].x : __builtin_amdgcn_alignbit(qv[nb].y, qv[nb].x, 16u);
                    qb = qv[nb].z;
                    d0 = half_bits_to_float(dv[nb].x & 0xffffu);
                    d1 = half_bits_to_float(dv[nb].y >> 16);
                }
                const uint32_t* const P = lds_iq4nl_pairs();
                uint4 b0 = make_uint4(P[qa & 255u], P[(qa >> 8) & 255u], P[(qa >> 16) & 255u], P[qa >> 24]);
                uint4 b1 = make_uint4(P[qb & 255u], P[(qb >> 8) & 255u], P[(qb >> 16) & 255u], P[qb >> 24]);
                if (d0 == 0.f) b0 = make_uint4(0u, 0u, 0u, 0u);
                if (d1 == 0.f) b1 = make_uint4(0u, 0u, 0u, 0u);
                fb[nb][0] = __builtin_bit_cast(half8, b0);
                fb[nb][1] = __builtin_bit_cast(half8, b1);
                dg[nb][0] = d0 != 0.f ? d0 * 16777216.f : 1.f;
                dg[nb][1] = d1 != 0.f ? d1 * 16777216.f : 1.f;
            }
        }
    };

    // Q4_K group sums of this thread's row divided by 32 (exact; they reach
    // 2^16 for x and 2^19 for act within range), split hi/lo, into an S buffer.
    auto store_s = [&](_Float16* sb_) {
        const float v[4] = {ps.x, ps.y, ps.z, ps.w};
        _Float16 h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) split_f16(v[j] * 0.03125f, h[j], l[j]);
        *reinterpret_cast<uint2*>(&sb_[am * 16u + 4u * ahalf]) = make_uint2(pack_h2(h[0], h[1]), pack_h2(h[2], h[3]));
        *reinterpret_cast<uint2*>(&sb_[am * 16u + 8u + 4u * ahalf]) = make_uint2(pack_h2(l[0], l[1]), pack_h2(l[2], l[3]));
    };
    // Vector-memory loads issued after a slab's A DMA: the B ring's, and at a
    // superblock's first slab its header (and Q4_K group sums).
    constexpr uint32_t B_PER_SLAB = Q4K ? NB : IQ4 ? (TL ? 2u : 4u) * NB : IQ4X ? (TL ? 2u : 3u) * NB : 0u;
    constexpr uint32_t B_PER_SB = Q5K                ? 2u * NB + 1u
                                  : Q4K              ? NB + 1u
                                  : IQ2S             ? (TL ? 3u : 7u) * NB
                                  : IQ3S             ? (TL ? 4u : 7u) * NB
                                  : IQG              ? (TL ? 3u : 5u) * NB
                                  : Q6K              ? (TL ? 2u : 3u) * NB
                                                     : 0u;
    auto run = [&](auto mbe_tag) {
        constexpr int MBE = decltype(mbe_tag)::value;
        constexpr uint32_t DEPTH = (!Q4K && !Q6K && MBE <= 2) ? 4u : 2u;
        // Two operand sets let the decode of slab s + 1 interleave with slab s's
        // MFMAs; with 3-4 row blocks of 4 B blocks the registers hold one set
        // (IQ4_NL: two), and the decode follows the MFMAs in program order.
        constexpr uint32_t NFB = (IQN || MBE <= 2 || NB == 2) ? 2u : 1u;
        typedef __attribute__((address_space(3))) void lds_void;
        auto dma_a = [&](uint32_t buf, uint32_t s) {
#pragma unroll
            // Row groups past the tile's 16 MBE rows (odd MBE at TT 128) are
            // loaded too, from clamped rows into LDS rows nobody reads: no branch.
            for (int i = 0; i < (2 * MBE + (int)NW - 1) / (int)NW; ++i) {
                const uint32_t roff = 8u * (NW * i + wave) * 64u;
                _Float16* const dh = (buf ? Ah1 : Ah0) + roff;
                _Float16* const dl = (buf ? Al1 : Al0) + roff;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_h, (lds_void*)dh, 16, avo[i], 128u * s, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_l, (lds_void*)dl, 16, avo[i], 128u * s, 0, 0);
            }
        };
        floatx4 acc[MBE][NB];
        float dlast[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) dlast[j] = 1.f;
#pragma unroll
        for (int i = 0; i < MBE; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // Prologue: A(0) into buffer 0; B ring; header of superblock 0; decode B(0).
        dma_a(0u, 0u);
        if constexpr (!IQN) load_hdr(0);
        if constexpr (Q4K) {
            INGOT_LOAD_S(0u);
            store_s(Ss[0]);
        }
#pragma unroll
        for (uint32_t d = 0; d < DEPTH; ++d) load_slab(d, d, (d & 1u) == 0u);
        SbState cur, nxt;
        if constexpr (!IQN) take_hdr(cur, 0u);
        half8 fb[NFB][NB][2], fe[Q6K ? NFB : 1][NB][2];
        float dgs[NFB][NB][2];
        {
            uint4 qv[NB];
            uint2 dv[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                qv[nb] = nq[0][nb];
                if constexpr (IQN) qv[nb].z = n1[0][nb];
                if constexpr (IQN || Q6K) dv[nb] = nd[0][nb];
            }
            load_slab(0, DEPTH, true);
            decode(cur, 0u, qv, dv, fb[0], dgs[0], fe[0]);
        }
        for (uint32_t s0 = 0; s0 < slabs; s0 += UNR) {
            const uint32_t sb = s0 >> 2;
            _Float16* const sbuf = Ss[sb & 1u];
#pragma unroll
            for (uint32_t sq = 0; sq < UNR; ++sq) {
                const uint32_t s = s0 + sq;
                if constexpr (IQN) {
                    if (s >= slabs) break;  // uniform
                }
                __syncthreads();  // A(s), S of this superblock visible; the other A buffer free
                // Loads of this slab, in this order and kept together: A(s + 1) into
                // the other buffer (unconditionally: past the last slab it re-reads
                // the last one into a buffer nobody reads; drained at the end), the
                // B ring, the next superblock's header. The wait before the next
                // barrier counts the loads issued after the A DMA.
                __builtin_amdgcn_sched_barrier(0);
                const bool more = s + 1u < slabs;
                dma_a((sq + 1u) & 1u, more ? s + 1u : s);
                // B of slab s + 1 out of the ring, B(s + 1 + DEPTH) into its slot.
                const uint32_t rs = (sq + 1u) % DEPTH;
                uint4 qv[NB];
                uint2 dv[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    qv[nb] = nq[rs][nb];
                    if constexpr (IQN) qv[nb].z = n1[rs][nb];
                    if constexpr (IQN || Q6K) dv[nb] = nd[rs][nb];
                }
                // (s is a multiple of UNR plus sq: slab s + 1 + DEPTH opens a half when sq is odd)
                load_slab(rs, s + 1u + DEPTH, (sq & 1u) != 0u);
                if constexpr (!IQN) {
                    if (sq == 0) {
                        load_hdr(sb + 1);
                        if constexpr (Q4K) INGOT_LOAD_S(sb + 1u);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (!IQN) {
                    // past the last superblock: the clamped header, never used
                    if (sq == 3) take_hdr(nxt, sb + 1u);
                }
                // Decode B(s + 1) while this slab's MFMAs issue.
                const uint32_t cb = NFB == 2u ? (sq & 1u) : 0u, nb_ = NFB == 2u ? cb ^ 1u : 0u;
                // (after the last slab: a decode of clamped bytes that nothing reads;
                // kept unconditional so that the decode shares a block with the MFMAs)
                if (NFB == 2u) decode(sq == 3 ? nxt : cur, (sq + 1u) & 3u, qv, dv, fb[nb_], dgs[nb_], fe[Q6K ? nb_ : 0u]);
                const _Float16* const bh = (sq & 1u) ? Ah1 : Ah0;
                const _Float16* const bl = (sq & 1u) ? Al1 : Al0;
                if constexpr (!IQN) {
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
                        for (int part = 0; part < 2; ++part)
#pragma unroll
                            for (int mb = 0; mb < MBE; ++mb) {
                                const uint32_t ar = mb * 16u + ln;
                                const uint32_t ch = IQG ? 2u * kq + gi : 4u * gi + kq;
                                const uint32_t off = ar * 64u + 8u * (ch ^ ((ar >> 1) & 7u));
                                const half8 a = *reinterpret_cast<const half8*>(part ? &bl[off] : &bh[off]);
#pragma unroll
                                for (int nb = 0; nb < NB; ++nb)
                                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, fb[cb][nb][gi], acc[mb][nb], 0, 0, 0);
                                if constexpr (Q6K) {
                                    if (part == 0) {
#pragma unroll
                                        for (int nb = 0; nb < NB; ++nb)
                                            acc[mb][nb] =
                                                __builtin_amdgcn_mfma_f32_16x16x32_f16(a, fe[cb][nb][gi], acc[mb][nb], 0, 0, 0);
                                    }
                                }
                            }
                    if constexpr (IQG && MBE <= 2) {
                        // IQ tiles of 1-2 row blocks: the slab's codebook and A reads
                        // (about 6 per A fragment) all first, then the MFMAs with the
                        // decode's VALU between them (C3 gate/up 270.5 to 265.8 us).
                        __builtin_amdgcn_sched_group_barrier(0x100, 64, 0);
#pragma unroll
                        for (int f = 0; f < 4 * MBE; ++f) {
                            __builtin_amdgcn_sched_group_barrier(0x008, NB, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                        }
                    } else {
                        // Issue order within the slab: PF A-fragment reads ahead, then
                        // per fragment its NB MFMAs, the read PF fragments on and (with
                        // two operand sets) a share of the next slab's B decode (VALU),
                        // so that LDS latency and the decode hide behind the MFMAs.
                        // Q6_K: A hi fragments (the first MBE of each 2 MBE) feed 2 NB MFMAs.
                        constexpr int NF = 4 * MBE, PF = 4, VPF = NFB == 2u ? (Q6K ? 4 * NB : NB == 2 ? 2 : 4) : 0;
                        __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
                        for (int f = 0; f < NF; ++f) {
                            if (Q6K && ((f / MBE) & 1) == 0) __builtin_amdgcn_sched_group_barrier(0x008, 2 * NB, 0);
                            else __builtin_amdgcn_sched_group_barrier(0x008, NB, 0);
                            if (f + PF < NF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                            if (VPF > 0) __builtin_amdgcn_sched_group_barrier(0x002, VPF, 0);
                        }
                    }
                } else {
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const float f1 = dlast[nb] * __builtin_amdgcn_rcpf(dgs[cb][nb][gi]);
                            dlast[nb] = dgs[cb][nb][gi];
#pragma unroll
                            for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
                                for (int j = 0; j < 4; ++j) acc[mb][nb][j] *= f1;
                        }
#pragma unroll
                        for (int part = 0; part < 2; ++part)
#pragma unroll
                            for (int mb = 0; mb < MBE; ++mb) {
                                const uint32_t ar = mb * 16u + ln;
                                const uint32_t off = ar * 64u + 8u * ((4u * gi + kq) ^ ((ar >> 1) & 7u));
                                const half8 a = *reinterpret_cast<const half8*>(part ? &bl[off] : &bh[off]);
#pragma unroll
                                for (int nb = 0; nb < NB; ++nb)
                                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, fb[cb][nb][gi], acc[mb][nb], 0, 0, 0);
                            }
                    }
                }
                if (NFB == 1u) decode(sq == 3 ? nxt : cur, (sq + 1u) & 3u, qv, dv, fb[0], dgs[0], fe[0]);
                if constexpr (Q4K) {
                    if (sq == 3) {
                        half8 fm[NB];
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const uint4 v = kq < 2 ? make_uint4(bytes01(cur.mn[nb][0]), bytes23(cur.mn[nb][0]),
                                                                bytes01(cur.mn[nb][1]), bytes23(cur.mn[nb][1]))
                                                   : make_uint4(0, 0, 0, 0);
                            fm[nb] = __builtin_bit_cast(half8, v);
                        }
                        float f1[NB], f2[NB];
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const float rn = more ? __builtin_amdgcn_rcpf(nxt.dsc[nb]) : 1.f;
                            f1[nb] = cur.dsc[nb] * rn;
                            f2[nb] = -cur.dmn[nb] * rn;
                        }
#pragma unroll
                        for (int mb = 0; mb < MBE; ++mb) {
                            const half8 sa =
                                *reinterpret_cast<const half8*>(&sbuf[(mb * 16u + ln) * 16u + 8u * (kq & 1u)]);
                            floatx4 mc[NB];
#pragma unroll
                            for (int nb = 0; nb < NB; ++nb)
                                mc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sa, fm[nb], floatx4{0.f, 0.f, 0.f, 0.f},
                                                                                0, 0, 0);
#pragma unroll
                            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                                for (int j = 0; j < 4; ++j)
                                    acc[mb][nb][j] = acc[mb][nb][j] * f1[nb] + mc[nb][j] * f2[nb];
                        }
                        cur = nxt;
                        // S of the next superblock into the other buffer (last read
                        // at the previous superblock's end, two barriers ago).
                        store_s(Ss[(sb + 1u) & 1u]);  // past the last superblock: clamped, unread
                    }
                } else if constexpr (IQG || Q6K) {
                    if (sq == 3) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const float f1 = cur.dsc[nb] * (more ? __builtin_amdgcn_rcpf(nxt.dsc[nb]) : 1.f);
#pragma unroll
                            for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
                                for (int j = 0; j < 4; ++j) acc[mb][nb][j] *= f1;
                        }
                        cur = nxt;
                    }
                }
                // This wave's A(s + 1) has landed (the loads issued after it may
                // stay in flight) before the barrier that publishes it; the slab's
                // MFMAs stay on this side of it.
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (Q6K) {
                    // ql per slab, qh at odd sq (the load opens a half), the header at sq 0
                    if (sq == 0) wait_vmcnt<NB + B_PER_SB>();
                    else if (sq & 1u) wait_vmcnt<2u * NB>();
                    else wait_vmcnt<NB>();
                } else if (sq == 0 && !IQN) wait_vmcnt<B_PER_SLAB + B_PER_SB>();
                else wait_vmcnt<B_PER_SLAB>();
            }
        }
        // No A DMA may still be writing LDS when the block exits.
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        if constexpr (IQN) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[mb][nb][j] *= dlast[nb];
        }
#pragma unroll
        for (int mb = 0; mb < MBE; ++mb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t m = mb * 16u + 4u * kq + j;
                const uint64_t q = q0 + m;
                if (GATEUP && AORD == A_F32) {
                    const int e = s_rowe[m].x;
#pragma unroll
                    for (int h = 0; h < (int)HB; ++h) {
                        const float v = swiglu(ldexpf(acc[mb][h][j], -e), ldexpf(acc[mb][HB + h][j], -e), limit);
                        if (m < n) out[q * ldo + row0 + 16u * HB * wave + 16u * h + ln] = v;
                    }
                } else if (GATEUP) {
                    // g, u in true units, then act 2^a_t; act column row0 + 16 HB w + 16 h + ln
                    const int e = s_rowe[m].x, ea = s_rowe[m].y;
                    float v[HB];
#pragma unroll
                    for (int h = 0; h < (int)HB; ++h)
                        v[h] = ldexpf(swiglu(ldexpf(acc[mb][h][j], -e), ldexpf(acc[mb][HB + h][j], -e), limit), ea);
                    // the row's max |act| over the 16 lanes of this row (bit patterns
                    // as integers: NaN stays above infinity)
                    uint32_t rm = __float_as_uint(fabsf(v[0]));
#pragma unroll
                    for (int h = 1; h < (int)HB; ++h) rm = max(rm, __float_as_uint(fabsf(v[h])));
                    rm = max(rm, (uint32_t)__builtin_amdgcn_mov_dpp((int)rm, 0xb1, 0xf, 0xf, false));
                    rm = max(rm, (uint32_t)__builtin_amdgcn_mov_dpp((int)rm, 0x4e, 0xf, 0xf, false));
                    rm = max(rm, (uint32_t)__builtin_amdgcn_mov_dpp((int)rm, 0x141, 0xf, 0xf, false));
                    rm = max(rm, (uint32_t)__builtin_amdgcn_mov_dpp((int)rm, 0x140, 0xf, 0xf, false));
                    if (ln == 0u) rpart[wave][m] = rm;
                    _Float16 hh[HB], ll[HB];
#pragma unroll
                    for (int h = 0; h < (int)HB; ++h) split_f16(v[h], hh[h], ll[h]);
                    if (m < n) {
                        if (AORD == A_IQ4NL && HB == 2) {
                            // columns c and c + 16 of a 32-column block are neighbours
                            const uint64_t o = q * ldo + row0 + 32u * wave + 8u * (ln >> 2) + 2u * (ln & 3u);
                            *reinterpret_cast<uint32_t*>(out_h + o) = pack_h2(hh[0], hh[HB - 1]);
                            *reinterpret_cast<uint32_t*>(out_l + o) = pack_h2(ll[0], ll[HB - 1]);
                        } else {
#pragma unroll
                            for (int h = 0; h < (int)HB; ++h) {
                                const uint64_t o = q * ldo + a_pos<AORD>(row0 + 16u * HB * wave + 16u * h + ln);
                                out_h[o] = hh[h];
                                out_l[o] = ll[h];
                            }
                        }
                    }
                    if (out_gs != nullptr) {
                        float gsum = v[0];
#pragma unroll
                        for (int h = 1; h < (int)HB; ++h) gsum += v[h];
                        gsum += dpp_mov<0xb1>(gsum);
                        gsum += dpp_mov<0x4e>(gsum);
                        gsum += dpp_mov<0x141>(gsum);
                        gsum += dpp_mov<0x140>(gsum);
                        if constexpr (HB == 2) {
                            if (m < n && ln == 0) out_gs[q * (ldo / 32u) + (row0 + 32u * wave) / 32u] = gsum;
                        } else {
                            if (ln == 0) gpart[wave][m] = gsum;  // half of a 32-column group
                        }
                    }
                } else {
                    if (m < n) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
                            out[q * ldo + row0 + 16u * NB * wave + 16u * nb + ln] = acc[mb][nb][j];
                    }
                }
            }
        if constexpr (GATEUP && AORD != A_F32) {
            if ((HB == 1 && out_gs != nullptr) || rowmax != nullptr) __syncthreads();
            if constexpr (HB == 1) {
                // 32-column group g of the block's 64 act columns = waves 2 g, 2 g + 1
                if (out_gs != nullptr) {
                    const uint32_t g = tid / TT, m = tid % TT;
                    if (m < n) out_gs[(q0 + m) * (ldo / 32u) + row0 / 32u + g] = gpart[2u * g][m] + gpart[2u * g + 1u][m];
                }
            }
            if (rowmax != nullptr && tid < n) {
                uint32_t v = rpart[0][tid];
#pragma unroll
                for (uint32_t w = 1; w < NW; ++w) v = max(v, rpart[w][tid]);
                atomicMax(rowmax + q0 + tid, v);
            }
        }
    };
    switch ((n + 15u) >> 4) {
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 3: run(std::integral_constant<int, 3>{}); break;
        case 4: run(std::integral_constant<int, 4>{}); break;
        default:
            if constexpr (TT == 128) {
                switch ((n + 15u) >> 4) {
                    case 5: run(std::integral_constant<int, 5>{}); break;
                    case 6: run(std::integral_constant<int, 6>{}); break;
                    case 7: run(std::integral_constant<int, 7>{}); break;
                    default: run(std::integral_constant<int, 8>{}); break;
                }
            }
            break;
    }
#undef INGOT_LOAD_S
}

// x [T][H] fp32 -> xh, xl [T][H] f16 with x 2^e_t = xh + xl (+ O(2^-22 |x|)),
// e_t = x_exp(max |x_t|) per token (xstat), stored in column order `order` (A_NATURAL;
// A_IQ3XXS and A_Q6K, whose permutations keep runs of 4 columns together, H % 256 == 0;
// or A_IQ4NL, which spreads them 2 apart within each 32-column block), and the
// natural 32-column sums of x 2^e_t, xs [T][H/32], used by the Q4_K mins term.
// Item g covers x[4g, 4g + 4) (8 consecutive items per 32-column group, so the
// threads of a wave cover whole groups; n is a multiple of 32).
__device__ inline void split_f16_part(const float* __restrict__ x, uint64_t n, _Float16* __restrict__ xh,
                                      _Float16* __restrict__ xl, float* __restrict__ xs, uint32_t order, uint64_t g,
                                      const float* __restrict__ xstat, uint32_t H) {
    const uint64_t i = g * 4u;
    const bool live = i < n;
    const float4 v = live ? ldexp4(*reinterpret_cast<const float4*>(x + i), x_exp(xstat[2u * (i / H)]))
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    const float a[4] = {v.x, v.y, v.z, v.w};
    if (live) {
        if (order == A_IQ4NL) {  // the 4 columns land 2 apart
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint64_t o = (i & ~31ull) | a_pos<A_IQ4NL>((uint32_t)(i + j) & 31u);
                split_f16(a[j], xh[o], xl[o]);
            }
        } else {
            const uint64_t o = order == A_IQ3XXS ? (i & ~255ull) | a_pos<A_IQ3XXS>((uint32_t)i & 255u)
                               : order == A_Q6K  ? (i & ~255ull) | a_pos<A_Q6K>((uint32_t)i & 255u)
                                                 : i;
#pragma unroll
            for (int j = 0; j < 4; ++j) split_f16(a[j], xh[o + j], xl[o + j]);
        }
    }
    float s = (a[0] + a[1]) + (a[2] + a[3]);
    s += dpp_mov<0xb1>(s);
    s += dpp_mov<0x4e>(s);
    s += dpp_mov<0x141>(s);
    if (live && (threadIdx.x & 7u) == 0) xs[i / 32u] = s;
}

#ifndef INGOT_KIND_UNIT  // format-independent kernels: compiled in moe_hip.hip only
// Plain grid-stride copy of n16 16-byte words (counter calibration workload).
__global__ __launch_bounds__(256) void k_copy16(uint4* __restrict__ dst, const uint4* __restrict__ src, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Streaming read of n16 16-byte words, the floor a decode stage of the same
// bytes cannot beat: a block of 256 lanes reads READ_BLOCK_WORDS consecutive
// words (16 KiB), each lane READ_UNROLL of them 4 KiB apart with every load in flight,
// and folds them with XOR. Nothing is stored unless a lane's fold equals an
// arbitrary constant (the stores keep the loads live; sink holds one word per
// block). n16 == 0 gives an empty kernel node: a dependent launch doing nothing.
constexpr uint32_t READ_UNROLL = 4;
constexpr uint64_t READ_BLOCK_WORDS = 256ull * READ_UNROLL;
__global__ __launch_bounds__(256) void k_read16(const uint4* __restrict__ src, uint64_t n16,
                                                uint32_t* __restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * READ_BLOCK_WORDS + threadIdx.x;
    uint4 v[READ_UNROLL];
#pragma unroll
    for (uint32_t j = 0; j < READ_UNROLL; ++j) {
        const uint64_t i = base + 256ull * j;
        v[j] = i < n16 ? src[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    uint32_t acc = 0;
#pragma unroll
    for (uint32_t j = 0; j < READ_UNROLL; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

// Dense token tiles for the shared expert: tile t = {0, 64 t, min(64, T - 64 t), 0}.
__global__ void k_dense_tiles(uint32_t T, uint32_t cap, uint32_t* __restrict__ tiles) {
    uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= cap) return;
    uint32_t first = t * TM;
    tiles[4 * t] = 0;
    tiles[4 * t + 1] = first < T ? first : 0;
    tiles[4 * t + 2] = first < T ? min(TM, T - first) : 0;
    tiles[4 * t + 3] = min(cap, (T + TM - 1) / TM);
}

// ------------------------------------------------------- prefill: combine
// out[t][i] = sum_k w[t,k] Y[inverse[t*K+k]][i] in route order (kernels/prefill.metal:39),
// + sigmoid(sgl[t]) (or 1) * Ys[t][i] for a shared expert, + res[t][i].
// xstat != NULL: the f16 GEMM's rows of Y (the routed ones, and Ys when
// shared_scaled) are in units of 2^a_t (act_exp) and are scaled back.
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ Y, const float* __restrict__ Ys,
                                                 const uint32_t* __restrict__ inverse, const float* __restrict__ wts,
                                                 const float* __restrict__ sgl, const float* __restrict__ res,
                                                 uint32_t T, uint32_t H, uint32_t K, float* __restrict__ out,
                                                 const float* __restrict__ xstat, uint32_t shared_scaled,
                                                 uint32_t* __restrict__ flags) {
    // grid (ceil(H / 1024), T): the token is uniform in the block, so its
    // packed positions and weights are scalar loads. The shared row and the
    // residual are loaded first, then the routed rows in batches of CB whose
    // loads are all issued before the first is used (one memory round trip per
    // batch instead of one per pair; the K % CB left over one at a time); the
    // sum keeps the route order.
    constexpr uint32_t CB = 8;
    const uint32_t t = blockIdx.y, c = 4u * (blockIdx.x * blockDim.x + threadIdx.x);
    if (c >= H) return;
    const int ue = xstat ? -act_exp(ld_xstat(xstat, t)) : 0;
    float4 ys = make_float4(0.f, 0.f, 0.f, 0.f), r = ys;
    if (Ys) ys = *reinterpret_cast<const float4*>(Ys + (uint64_t)t * H + c);
    if (res) r = *reinterpret_cast<const float4*>(res + (uint64_t)t * H + c);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t k = 0;
    for (; k + CB <= K; k += CB) {
        float w[CB];
        uint32_t iv[CB];
        float4 y[CB];
#pragma unroll
        for (uint32_t u = 0; u < CB; ++u) {
            w[u] = wts[t * K + k + u];
            iv[u] = inverse[t * K + k + u];
        }
#pragma unroll
        for (uint32_t u = 0; u < CB; ++u) y[u] = *reinterpret_cast<const float4*>(Y + (uint64_t)iv[u] * H + c);
#pragma unroll
        for (uint32_t u = 0; u < CB; ++u) {
            s.x = __builtin_fmaf(w[u], y[u].x, s.x);
            s.y = __builtin_fmaf(w[u], y[u].y, s.y);
            s.z = __builtin_fmaf(w[u], y[u].z, s.z);
            s.w = __builtin_fmaf(w[u], y[u].w, s.w);
        }
    }
    for (; k < K; ++k) {
        const float w = wts[t * K + k];
        const float4 y = *reinterpret_cast<const float4*>(Y + (uint64_t)inverse[t * K + k] * H + c);
        s.x = __builtin_fmaf(w, y.x, s.x);
        s.y = __builtin_fmaf(w, y.y, s.y);
        s.z = __builtin_fmaf(w, y.z, s.z);
        s.w = __builtin_fmaf(w, y.w, s.w);
    }
    s = ldexp4(s, ue);
    if (Ys) {
        const float w = sgl ? ingot_det_sigmoid(sgl[t]) : 1.0f;
        if (shared_scaled) ys = ldexp4(ys, ue);
        s.x = __builtin_fmaf(ys.x, w, s.x);
        s.y = __builtin_fmaf(ys.y, w, s.y);
        s.z = __builtin_fmaf(ys.z, w, s.z);
        s.w = __builtin_fmaf(ys.w, w, s.w);
    }
    if (res) {
        s.x += r.x; s.y += r.y; s.z += r.z; s.w += r.w;
    }
    *reinterpret_cast<float4*>(out + (uint64_t)t * H + c) = s;
    if (!(isfinite(s.x) && isfinite(s.y) && isfinite(s.z) && isfinite(s.w))) atomicOr(flags, FLAG_OUT_NONFINITE);
}

// ---------------------------------------------- generic (drop-in) kernels
// y[g][r] = sum_j W_g[r][j] x_g[j], one wave per (row, matrix g); scalar
// decode of any supported kind. The input of matrix g starts at x + g*xstride.
__global__ __launch_bounds__(256) void k_project_generic(const uint8_t* __restrict__ w, uint64_t stride, uint32_t kind,
                                                         uint32_t cols, uint32_t rows, const float* __restrict__ x,
                                                         uint64_t xstride, float* __restrict__ y) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6), g = blockIdx.y;
    if (r >= rows) return;
    const uint8_t* row = w + ((uint64_t)g * rows + r) * stride;
    const float* xv = x + (uint64_t)g * xstride;
    float s = 0.f;
    for (uint32_t j = lane; j < cols; j += 64u) s += dequant_value(row, kind, j) * xv[j];
    s = wave_sum(s);
    if (lane == 0) y[(uint64_t)g * rows + r] = s;
}

__global__ void k_dequant_generic(const uint8_t* __restrict__ w, uint64_t stride, uint32_t kind, uint32_t cols,
                                  uint64_t nrows, float* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * cols) return;
    const uint64_t r = i / cols;
    out[i] = dequant_value(w + r * stride, kind, (uint32_t)(i % cols));
}

__global__ void k_swiglu(const float* __restrict__ g, const float* __restrict__ u, uint64_t n, float* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = swiglu(g[i], u[i], 0.f);
}

// Gpu::moe combine (kernels/moe.metal:412-422): out[i] = sum_e routed[e][i] w[e]
// + shared[i] sigmoid(shared_logit) (shared may be NULL).
__global__ void k_combine_host(const float* __restrict__ routed, const float* __restrict__ shared,
                               const float* __restrict__ w, const float* __restrict__ slogit, uint32_t H, uint32_t K,
                               float* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    float s = 0.f;
    for (uint32_t e = 0; e < K; ++e) s += routed[(uint64_t)e * H + i] * w[e];
    if (shared) s += shared[i] / (1.0f + expf(-slogit[0]));
    out[i] = s;
}

// The GGUF-order byte of a tiled group's byte r (see TILE_Q4K): its offset
// from the group's first row.
__device__ __forceinline__ uint64_t tiled_source(uint32_t kind, uint32_t r, uint64_t stride) {
    if (kind == 12) {
        const uint32_t sb = r / TILE_Q4K, q = r % TILE_Q4K;
        if (q < 256u) return (q >> 4) * stride + 144u * sb + (q & 15u);
        const uint32_t t = q - 256u, sq = t >> 9, u = t & 511u, l = u >> 3;
        return (l & 15u) * stride + 144u * sb + 16u + 32u * sq + 8u * (l >> 4) + (u & 7u);
    }
    if (kind == 13) {
        const uint32_t sb = r / TILE_Q5K, q = r % TILE_Q5K;
        if (q < 256u) return (q >> 4) * stride + 176u * sb + (q & 15u);
        if (q < 768u) {
            const uint32_t t = q - 256u, l = t >> 3;
            return (l & 15u) * stride + 176u * sb + 16u + 8u * (l >> 4) + (t & 7u);
        }
        const uint32_t t = q - 768u, sq = t >> 9, u = t & 511u, l = u >> 3;
        return (l & 15u) * stride + 176u * sb + 48u + 32u * sq + 8u * (l >> 4) + (u & 7u);
    }
    if (kind == 14) {
        const uint32_t sb = r / TILE_Q6K, q = r % TILE_Q6K;
        if (q < 2048u) {
            const uint32_t sq = q >> 9, u = q & 511u, l = u >> 3;
            return (l & 15u) * stride + 210u * sb + 64u * (sq >> 1) + 32u * (sq & 1u) + 8u * (l >> 4) + (u & 7u);
        }
        if (q < 3072u) {
            const uint32_t t = q - 2048u, n = t >> 9, u = t & 511u, l = u >> 3;
            return (l & 15u) * stride + 210u * sb + 128u + 32u * n + 8u * (l >> 4) + (u & 7u);
        }
        if (q < 3328u) {
            const uint32_t t = q - 3072u;
            return (t >> 4) * stride + 210u * sb + 192u + (t & 15u);
        }
        const uint32_t t = q - 3328u;
        return (t >> 1) * stride + 210u * sb + 208u + (t & 1u);
    }
    if (kind == 17) {
        const uint32_t sb = r / TILE_IQ2XS, q = r % TILE_IQ2XS;
        if (q < 1024u) return ((q >> 4) & 15u) * stride + 74u * sb + 2u + 16u * (q >> 8) + (q & 15u);
        if (q < 1152u) return ((q - 1024u) >> 3) * stride + 74u * sb + 66u + (q & 7u);
        const uint32_t t = q - 1152u;
        return (t >> 1) * stride + 74u * sb + (t & 1u);
    }
    if (kind == 22) {
        const uint32_t sb = r / TILE_IQ2S, q = r % TILE_IQ2S;
        if (q < 1024u) {
            const uint32_t l = q >> 4, b = q & 15u;
            return (l & 15u) * stride + 82u * sb + (b < 8u ? 2u : 26u) + 8u * (l >> 4) + b;
        }
        if (q < 1280u) {
            const uint32_t t = q - 1024u, l = t >> 2, b = t & 3u;
            return (l & 15u) * stride + 82u * sb + (b < 2u ? 66u : 72u) + 2u * (l >> 4) + b;
        }
        const uint32_t t = q - 1280u;
        return (t >> 1) * stride + 82u * sb + (t & 1u);
    }
    if (kind == 21) {
        const uint32_t sb = r / TILE_IQ3S, q = r % TILE_IQ3S;
        if (q < 1024u) return ((q >> 4) & 15u) * stride + 110u * sb + 2u + 16u * (q >> 8) + (q & 15u);
        if (q < 1536u) {
            const uint32_t t = q - 1024u, l = t >> 3;
            return (l & 15u) * stride + 110u * sb + 74u + 8u * (l >> 4) + (t & 7u);
        }
        if (q < 1728u) {
            const uint32_t t = q - 1536u, row = t / 12u, b = t % 12u;
            return row * stride + 110u * sb + (b < 8u ? 66u + b : 98u + b);
        }
        const uint32_t t = q - 1728u;
        return (t >> 1) * stride + 110u * sb + (t & 1u);
    }
    if (kind == 23) {
        const uint32_t sb = r / TILE_IQ4XS, q = r % TILE_IQ4XS;
        if (q < 2048u) {
            const uint32_t sq = q >> 9, u = q & 511u, l = u >> 3, b = u & 7u;
            return (l & 15u) * stride + 136u * sb + 8u + 16u * (2u * sq + (b >> 2)) + 4u * (l >> 4) + (b & 3u);
        }
        const uint32_t t = q - 2048u;
        return (t >> 3) * stride + 136u * sb + (t & 7u);
    }
    if (kind == 18) {
        const uint32_t sb = r / TILE_IQ3XXS, q = r % TILE_IQ3XXS;
        if (q < 1024u) return ((q >> 4) & 15u) * stride + 98u * sb + 2u + 16u * (q >> 8) + (q & 15u);
        if (q < 1536u) {
            const uint32_t t = q - 1024u, l = t >> 3;
            return (l & 15u) * stride + 98u * sb + 66u + 8u * (l >> 4) + (t & 7u);
        }
        const uint32_t t = q - 1536u;
        return (t >> 1) * stride + 98u * sb + (t & 1u);
    }
    // IQ4_NL
    const uint32_t sl = r / TILE_IQ4NL, q = r % TILE_IQ4NL;
    if (q < 512u) {
        const uint32_t l = q >> 3, b = q & 7u;
        return (l & 15u) * stride + 36u * sl + 18u * (b >> 2) + 2u + 4u * (l >> 4) + (b & 3u);
    }
    const uint32_t t = q - 512u, b = t & 3u;
    return (t >> 2) * stride + 36u * sl + (b < 2u ? b : 16u + b);
}

// dst = src (count x rows rows of `stride` bytes, rows % 16 == 0) in the
// tiled layout; one byte per thread.
__global__ __launch_bounds__(256) void k_tile_weights(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                      uint64_t nbytes, uint32_t kind, uint64_t stride) {
    const uint64_t gbytes = 16u * stride;
    for (uint64_t o = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; o < nbytes;
         o += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t g = o / gbytes;
        dst[o] = src[g * gbytes + tiled_source(kind, (uint32_t)(o - g * gbytes), stride)];
    }
}

#endif  // INGOT_KIND_UNIT
}  // namespace ingot
