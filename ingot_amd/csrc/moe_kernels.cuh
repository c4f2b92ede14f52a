// HIP kernels of the MoE-layer hot path for gfx950 (wave64, MFMA, 160 KB LDS).
//
// Decode (few pairs) and prefill (many pairs) take different kernels:
//   router   k_router        logits = W_r x (fixed fp32 order), optional fused
//                            RMSNorm, optional shared-expert gate logit
//   route    k_route         per-token top-K on 64-bit (orderable value, ~id)
//                            keys; softmax or sigmoid+bias weights
//   decode   k_dec_gate_up2  routing of the block's token (block_route), then
//                            act[p] = SwiGLU(G_e x_t, U_e x_t), one wave per pair
//            k_gemv_gate_up  the same for the shared expert (no routing)
//            k_dec_down      out[t] = sum_k w_k D_e act[p] (+ shared, + residual)
//   prefill  k_dispatch_count / k_dispatch_place   stable expert grouping
//            k_gemm<GATEUP>  MFMA f32 grouped GEMM, dequantised weights in LDS
//            k_combine       out[t] = sum_k w_k Y[inverse[p]] (+ shared, + residual)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "det_math.h"
#include "formats.cuh"

namespace ingot {

constexpr int WAVE = 64;
constexpr uint32_t FLAG_NONFINITE = 1u;

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

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float swiglu(float g, float u, float limit) {
    if (limit > 0.f) {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
    }
    return g / (1.0f + expf(-g)) * u;
}

// ------------------------------------------------------ block-level routing
// The same selection and weights as k_route for one token, computed by a
// whole block without a serial chain: every candidate's rank is the number of
// larger keys (keys are unique), so candidate i with rank r < K is the r-th
// selection. LDS: keys [E] u64, vals [E] f32, sel_id/sel_v/w [K].
struct RouteLds {
    uint64_t* keys;
    float* vals;
    uint32_t* sel_id;
    float* sel_v;
    float* w;
};

__device__ inline void block_route(const float* __restrict__ l, const float* __restrict__ bias, uint32_t E, uint32_t K,
                                   uint32_t sigmoid_mode, float scale, RouteLds s, uint32_t* __restrict__ flags) {
    INGOT_NO_CONTRACT
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    bool bad = false;
    for (uint32_t e = tid; e < E; e += nt) {
        float v = l[e];
        float b = bias ? bias[e] : 0.f;
        bad |= !isfinite(v) || !isfinite(b);
        float key_v, wv;
        if (sigmoid_mode) {
            wv = ingot_det_sigmoid(v);
            key_v = bias ? wv + b : wv;
        } else {
            key_v = bias ? v + b : v;
            wv = key_v;
        }
        s.keys[e] = ingot_select_key(key_v, e);
        s.vals[e] = wv;
    }
    const uint32_t E16 = (E + 15u) & ~15u;
    for (uint32_t e = E + tid; e < E16; e += nt) s.keys[e] = 0;  // below every real key
    if (flags && __any(bad) && (tid & 63u) == 0) atomicOr(flags, FLAG_NONFINITE);
    __syncthreads();
    for (uint32_t e = tid; e < E; e += nt) {
        const uint64_t mine = s.keys[e];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < E16; j += 16) {
            ulonglong2 kv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) kv[q] = *reinterpret_cast<const ulonglong2*>(&s.keys[j + 2 * q]);
#pragma unroll
            for (int q = 0; q < 8; ++q) rank += (kv[q].x > mine ? 1u : 0u) + (kv[q].y > mine ? 1u : 0u);
        }
        if (rank < K) {
            s.sel_id[rank] = e;
            s.sel_v[rank] = s.vals[e];
        }
    }
    __syncthreads();
    float num = 0.f, total = 0.f;
    if (tid < K) {
        const float top = s.sel_v[0];
        num = sigmoid_mode ? s.sel_v[tid] : ingot_det_expf(s.sel_v[tid] - top);
        s.w[tid] = num;
    }
    __syncthreads();
    if (tid < K)
        for (uint32_t k = 0; k < K; ++k) total += s.w[k];  // selection order, as the CPU sums
    __syncthreads();  // every numerator read before any weight is written
    if (tid < K) s.w[tid] = sigmoid_mode ? num / total * scale : num / total;
    __syncthreads();
}

// ---------------------------------------------------------------- router
// One wave per (group of TOK tokens, group of experts). Lane l holds the
// columns 4l + 256i + c (i < HB = H/256, c < 4) of each of its tokens, which
// is the slot layout of the fixed reduction order (det_math.h): each logit is
// the lane's fused multiply-add chain followed by the xor butterfly, so it is
// bit-identical to the CPU's ingot_router_partial + ingot_butterfly64.
// With a norm gain the wave first computes RMSNorm of its tokens in the same
// order (sum of squares over the slots, butterfly, 1/sqrt(ss/H + eps), (x*r)*g)
// and writes the normalised rows (block (.., 0), wave 0 only).
// Expert index E (when sgvec != NULL) is the shared-expert gate vector: its
// product goes to sgl[t].
template <int TOK, int HB>
__global__ __launch_bounds__(256) void k_router(const float* __restrict__ x, const float* __restrict__ W,
                                                const float* __restrict__ sgvec, const float* __restrict__ gain,
                                                float eps, uint32_t T, uint32_t E, uint32_t epw,
                                                float* __restrict__ logits, float* __restrict__ sgl,
                                                float* __restrict__ xn) {
    INGOT_NO_CONTRACT
    constexpr uint32_t H = 256u * HB;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * TOK;
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
    const uint32_t rows = E + (sgvec ? 1u : 0u);
    const uint32_t e0 = (blockIdx.y * 4u + wave) * epw;
    for (uint32_t k = 0; k < epw; ++k) {
        uint32_t e = e0 + k;
        if (e >= rows) break;
        const float* wr = e < E ? W + (uint64_t)e * H : sgvec;
        float wv[HB * 4];
#pragma unroll
        for (int i = 0; i < HB; ++i) {
            float4 v = *reinterpret_cast<const float4*>(wr + 4u * lane + 256u * i);
            wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
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

// ----------------------------------------------------------------- route
// One wave per token, E <= 64 * NE. Softmax mode (src/lib.rs:43-60):
// selection and weights on l (+ bias when given), w_k = exp(v_k - v_top) /
// sum. Sigmoid mode (kernels/glm.metal:81-98): selection on sigmoid(l) + bias,
// w_k = sigmoid(l_k) / sum * scale. Keys (orderable(v) << 32 | ~id) make the
// wave maximum unique and resolve ties toward the lower id, exactly as a
// stable descending sort with f32::total_cmp does (+0 above -0). Everything
// stays in registers: the winner's weight input is fetched from its owning
// lane, lane k keeps the k-th selection, and lane 0 sums the weights in
// selection order. A non-finite logit or bias raises FLAG_NONFINITE; the ids
// written are still valid expert indices. K <= 64.
template <int NE>
__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits, const float* __restrict__ bias,
                                               uint32_t T, uint32_t E, uint32_t K, uint32_t sigmoid_mode,
                                               float scale, uint32_t* __restrict__ ids, float* __restrict__ wts,
                                               uint32_t* __restrict__ flags) {
    INGOT_NO_CONTRACT
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (t >= T) return;
    const float* l = logits + (uint64_t)t * E;
    uint64_t key[NE];
    float wv[NE];  // weight input of each candidate: l + bias (softmax) or sigmoid(l)
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        uint32_t e = lane + 64u * j;
        key[j] = 0;
        wv[j] = 0.f;
        if (e < E) {
            float v = l[e];
            float b = bias ? bias[e] : 0.f;
            bad |= !isfinite(v) || !isfinite(b);
            float s;
            if (sigmoid_mode) {
                wv[j] = ingot_det_sigmoid(v);
                s = bias ? wv[j] + b : wv[j];
            } else {
                s = bias ? v + b : v;
                wv[j] = s;
            }
            key[j] = ingot_select_key(s, e);
        }
    }
    if (__any(bad) && lane == 0) atomicOr(flags, FLAG_NONFINITE);
    uint32_t my_id = 0;
    float my_v = 0.f;
    for (uint32_t k = 0; k < K; ++k) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < NE; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            uint64_t o = shfl_xor_u64(best, m);
            best = o > best ? o : best;
        }
        const uint32_t id = 0xffffffffu - (uint32_t)best;
        const uint32_t owner = id & 63u, slot = id >> 6;
        float mine = 0.f;
#pragma unroll
        for (int j = 0; j < NE; ++j)
            if ((uint32_t)j == slot) {
                mine = wv[j];
                if (lane == owner) key[j] = 0;
            }
        const float v = __shfl(mine, (int)owner);
        if (lane == k) {
            my_id = id;
            my_v = v;
        }
    }
    // lane k < K: weight numerator of selection k
    const float top = __shfl(my_v, 0);
    const float num = sigmoid_mode ? my_v : ingot_det_expf(my_v - top);
    float total = 0.f;
    for (uint32_t k = 0; k < K; ++k) total += __shfl(num, (int)k);
    if (lane < K) {
        ids[(uint64_t)t * K + lane] = my_id;
        wts[(uint64_t)t * K + lane] = sigmoid_mode ? num / total * scale : num / total;
    }
}

// ---------------------------------------------- decode: routed gate/up
// grid (ceil(F / RPW), T), 512 threads (8 waves). The block routes its token
// (block_route; block 0 of each token writes ids/weights for the down kernel)
// while it stages the token's input in LDS. Wave w then computes rows
// [RPW*bx, +RPW) of the gate and up projections of pairs k = w, w+8, ...;
// each lane keeps its input chunks in registers.
constexpr uint32_t GU_WAVES = 8;

template <int KIND, int CPL, int RPW, int NP>
__global__ __launch_bounds__(512) void k_dec_gate_up2(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                      uint64_t gstride, uint64_t ustride, uint32_t F, uint32_t H,
                                                      const float* __restrict__ x, const float* __restrict__ logits,
                                                      const float* __restrict__ bias, uint32_t E, uint32_t K,
                                                      uint32_t sigmoid_mode, float scale, float limit,
                                                      uint32_t* __restrict__ ids, float* __restrict__ wts,
                                                      uint32_t* __restrict__ flags, float* __restrict__ act) {
    using Fm = Fmt<KIND>;
    __shared__ float s_x[4096];
    __shared__ uint64_t s_keys[1024];
    __shared__ float s_vals[1024];
    __shared__ uint32_t s_id[64];
    __shared__ float s_v[64], s_w[64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t nch = H / 32u;
    const uint32_t r0 = blockIdx.x * RPW;
    // Stage the token's input while the block routes it.
    {
        const float4* x4 = reinterpret_cast<const float4*>(x + (uint64_t)t * H);
        for (uint32_t i = threadIdx.x; i < H / 4u; i += 512u) reinterpret_cast<float4*>(s_x)[i] = x4[i];
    }
    block_route(logits + (uint64_t)t * E, bias, E, K, sigmoid_mode, scale, RouteLds{s_keys, s_vals, s_id, s_v, s_w},
                blockIdx.x == 0 ? flags : nullptr);
    if (blockIdx.x == 0 && threadIdx.x < K) {
        ids[(uint64_t)t * K + threadIdx.x] = s_id[threadIdx.x];
        wts[(uint64_t)t * K + threadIdx.x] = s_w[threadIdx.x];
    }
    // Weight loads of the wave's pairs k = wave + 8n (n < NP; K <= 8 NP);
    // a pair beyond K re-reads pair 0's rows and is not stored.
    typename Fm::Raw rg[NP][RPW][CPL], ru[NP][RPW][CPL];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t k = wave + GU_WAVES * n;
        const uint32_t e = s_id[k < K ? k : 0u];
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
    float xv[CPL][32], xs0[CPL], xs1[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t c = min(lane + 64u * j, nch - 1);
        Fm::load_x(s_x, c, xv[j]);
        xs0[j] = xs1[j] = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            xs0[j] += xv[j][q];
            xs1[j] += xv[j][16 + q];
        }
    }
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const uint32_t k = wave + GU_WAVES * n;
        float gs[RPW], us[RPW];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            gs[i] = us[i] = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (lane + 64u * j >= nch) continue;
                const uint32_t c = lane + 64u * j;
                gs[i] += Fm::dot_raw(rg[n][i][j], c, xv[j], xs0[j], xs1[j]);
                us[i] += Fm::dot_raw(ru[n][i][j], c, xv[j], xs0[j], xs1[j]);
            }
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const float g = wave_sum_dpp(gs[i]), u = wave_sum_dpp(us[i]);
            if (k < K && lane == (uint32_t)i && r0 + i < F) act[((uint64_t)t * K + k) * F + r0 + i] = swiglu(g, u, limit);
        }
    }
}

// ------------------------------------------------ decode: down + combine
// grid (ceil(H / (4*RPW)), T), 256 threads. The token's K activations (and
// the shared expert's) are staged in LDS once per block; each wave owns RPW
// output rows. The K pairs' chunks (plus the shared expert's) form one
// virtual row spread over the lanes (VPL chunks per lane), with each pair's
// routing weight folded into its activations, so the wave sum is
// sum_k w_k (D_e act_k)[i] (+ gate * (S_down sact)[i]) directly.
constexpr uint32_t DOWN_LDS_FLOATS = 12288;  // 48 KB of staged activations

template <int KD, int KS, int VPL, int RPW>
__global__ __launch_bounds__(256) void k_dec_down(const uint8_t* __restrict__ down, uint64_t dstride,
                                                  const uint8_t* __restrict__ sdown, uint64_t sdstride, uint32_t H,
                                                  uint32_t F, uint32_t SF, const float* __restrict__ act,
                                                  const float* __restrict__ sact, const uint32_t* __restrict__ ids,
                                                  const float* __restrict__ wts, const float* __restrict__ sgl,
                                                  uint32_t K, const float* __restrict__ res, float* __restrict__ out) {
    using Fd = Fmt<KD>;
    using Fs = Fmt<(KS < 0 ? KD : KS)>;
    __shared__ float s_act[DOWN_LDS_FLOATS];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, tid = threadIdx.x;
    const uint32_t t = blockIdx.y;
    const uint32_t nchF = F / 32u, nchS = KS >= 0 ? SF / 32u : 0u;
    const uint32_t nv = K * nchF + nchS;
    const uint32_t r0 = (blockIdx.x * 4u + wave) * RPW;
    // 1. this lane's chunks of the virtual row: expert row base, chunk, weight
    const uint8_t* base[VPL];
    uint32_t cc[VPL], aoff[VPL];
    float w[VPL];
    bool isS[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t v = lane + 64u * j;
        base[j] = nullptr;
        cc[j] = 0;
        aoff[j] = 0;
        w[j] = 0.f;
        isS[j] = false;
        if (v < K * nchF) {
            const uint32_t k = v / nchF, p = t * K + k;
            base[j] = down + (uint64_t)ids[p] * H * dstride;
            cc[j] = v % nchF;
            aoff[j] = k * F;
            w[j] = wts[p];
        } else if (v < nv) {
            base[j] = sdown;
            cc[j] = v - K * nchF;
            aoff[j] = K * F;
            isS[j] = true;
            w[j] = sgl ? ingot_det_sigmoid(sgl[t]) : 1.0f;
        }
    }
    // 2. weight loads for all RPW rows, issued before the activations arrive
    typename Fd::Raw rd[RPW][VPL];
    typename Fs::Raw rs[KS >= 0 ? RPW : 1][KS >= 0 ? VPL : 1];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const uint32_t r = min(r0 + i, H - 1);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (!base[j]) continue;
            if (KS >= 0 && isS[j]) rs[KS >= 0 ? i : 0][KS >= 0 ? j : 0] = Fs::load_raw(base[j] + (uint64_t)r * sdstride, cc[j]);
            else rd[i][j] = Fd::load_raw(base[j] + (uint64_t)r * dstride, cc[j]);
        }
    }
    // 3. stage the token's activations
    {
        const float4* a4 = reinterpret_cast<const float4*>(act + (uint64_t)t * K * F);
        float4* d4 = reinterpret_cast<float4*>(s_act);
        for (uint32_t i = tid; i < K * F / 4u; i += 256u) d4[i] = a4[i];
        if (KS >= 0) {
            const float4* s4 = reinterpret_cast<const float4*>(sact + (uint64_t)t * SF);
            for (uint32_t i = tid; i < SF / 4u; i += 256u) d4[K * F / 4u + i] = s4[i];
        }
    }
    __syncthreads();
    // 4. weighted activations of each chunk into registers, then the dot products
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        if (!base[j]) continue;
        float xv[32], xs0 = 0.f, xs1 = 0.f;
        if (KS >= 0 && isS[j]) Fs::load_x(s_act + aoff[j], cc[j], xv);
        else Fd::load_x(s_act + aoff[j], cc[j], xv);
#pragma unroll
        for (int q = 0; q < 32; ++q) xv[q] *= w[j];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            xs0 += xv[q];
            xs1 += xv[16 + q];
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            if (KS >= 0 && isS[j]) acc[i] += Fs::dot_raw(rs[KS >= 0 ? i : 0][KS >= 0 ? j : 0], cc[j], xv, xs0, xs1);
            else acc[i] += Fd::dot_raw(rd[i][j], cc[j], xv, xs0, xs1);
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        float sum = wave_sum_dpp(acc[i]);
        const uint32_t r = r0 + i;
        if (lane == (uint32_t)i && r < H) {
            if (res) sum += res[(uint64_t)t * H + r];
            out[(uint64_t)t * H + r] = sum;
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
                                                              const float* __restrict__ sgl, float* __restrict__ out) {
    using Fs = Fmt<KS>;
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
    if (lane == 0) out[(uint64_t)t * H + r] += acc;
}

// ------------------------------------------------------- prefill: dispatch
// Block-wide exclusive scan of one value per thread (blockDim 1024 = 16 waves).
__device__ inline uint32_t block_exclusive_scan_1024(uint32_t v, uint32_t* wsum, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_up(inc, d);
        if (lane >= (uint32_t)d) inc += o;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        uint32_t s = lane < 16 ? wsum[lane] : 0u, si = s;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            uint32_t o = __shfl_up(si, d);
            if (lane >= (uint32_t)d) si += o;
        }
        if (lane < 16) wsum[16 + lane] = si - s;
        if (lane == 15) *total = si;
    }
    __syncthreads();
    return inc - v + wsum[16 + wave];
}

// One block of 1024 threads, E <= 1024. Counts pairs per expert, writes
// counts[E], first[E] (exclusive scan: experts ascending) and the tile list:
// for each expert ceil(n/TM) tiles {expert, first pair of the tile, n in tile,
// 0}, experts ascending, padded with zero tiles to cap (the layout of
// kernels/prefill.metal:7-23 with TM-pair tiles).
__global__ __launch_bounds__(1024) void k_dispatch_count(const uint32_t* __restrict__ ids, uint32_t P, uint32_t E,
                                                         uint32_t TM, uint32_t cap, uint32_t* __restrict__ counts,
                                                         uint32_t* __restrict__ first, uint32_t* __restrict__ tiles) {
    __shared__ uint32_t cnt[1024];
    __shared__ uint32_t wsum[32];
    __shared__ uint32_t tot[2];
    const uint32_t tid = threadIdx.x;
    cnt[tid] = 0;
    __syncthreads();
    for (uint32_t p = tid; p < P; p += 1024u) atomicAdd(&cnt[ids[p]], 1u);
    __syncthreads();
    uint32_t n = tid < E ? cnt[tid] : 0u;
    uint32_t nt = (n + TM - 1) / TM;
    uint32_t f = block_exclusive_scan_1024(n, wsum, &tot[0]);
    __syncthreads();
    uint32_t t0 = block_exclusive_scan_1024(nt, wsum, &tot[1]);
    if (tid < E) {
        counts[tid] = n;
        first[tid] = f;
        for (uint32_t k = 0; k < nt && t0 + k < cap; ++k) {
            uint32_t* tl = tiles + 4u * (t0 + k);
            tl[0] = tid;
            tl[1] = f + k * TM;
            tl[2] = min(TM, n - k * TM);
            tl[3] = 0;
        }
    }
    __syncthreads();
    for (uint32_t t = tot[1] + tid; t < cap; t += 1024u) {
        uint32_t* tl = tiles + 4u * t;
        tl[0] = tl[1] = tl[2] = tl[3] = 0;
    }
}

// One block (256 threads) per expert: pair indices of the expert in ascending
// order at pairs[first[e]...], and each pair's packed position in inverse[p]
// (kernels/prefill.metal:25-38).
__global__ __launch_bounds__(256) void k_dispatch_place(const uint32_t* __restrict__ ids, uint32_t P,
                                                        const uint32_t* __restrict__ counts,
                                                        const uint32_t* __restrict__ first, uint32_t* __restrict__ pairs,
                                                        uint32_t* __restrict__ inverse) {
    const uint32_t e = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    if (counts[e] == 0) return;
    __shared__ uint32_t ws[4];
    const uint32_t chunk = (P + 255u) / 256u, s = min(P, tid * chunk), end = min(P, s + chunk);
    uint32_t mine = 0;
    for (uint32_t i = s; i < end; ++i) mine += ids[i] == e;
    uint32_t inc = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_up(inc, d);
        if (lane >= (uint32_t)d) inc += o;
    }
    if (lane == 63) ws[wave] = inc;
    __syncthreads();
    uint32_t before = inc - mine;
    for (uint32_t w = 0; w < wave; ++w) before += ws[w];
    uint32_t at = first[e] + before;
    for (uint32_t i = s; i < end; ++i)
        if (ids[i] == e) {
            inverse[i] = at;
            pairs[at++] = i;
        }
}

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

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int KIND, bool GATEUP>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                              uint64_t stride0, uint64_t stride1, uint32_t rows_per_expert,
                                              uint32_t kdim, const float* __restrict__ a_src,
                                              const uint32_t* __restrict__ pairs, uint32_t K,
                                              const uint32_t* __restrict__ tiles, uint32_t ldo, float limit,
                                              float* __restrict__ out) {
    using Fm = Fmt<KIND>;
    __shared__ float As[TM * LDS_STRIDE];
    __shared__ float Bs[128 * LDS_STRIDE];
    const uint32_t* tile = tiles + 4u * blockIdx.y;
    const uint32_t n = tile[2];
    if (n == 0) return;
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
        bptr = base + ((uint64_t)e * rows_per_expert + r) * st;
    } else {
        bptr = w0 + ((uint64_t)e * rows_per_expert + row0 + brow) * stride0;
    }

    floatx4 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
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
            float4 a[4], b[2];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
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
                for (int mb = 0; mb < 4; ++mb)
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
    for (int mb = 0; mb < 4; ++mb)
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
}

// -------------------------------- prefill: split-precision f16 MFMA GEMM (Q4_K)
// Same tiling and tile list as k_gemm, on v_mfma_f32_16x16x32_f16 with fp32
// accumulation. Each operand is split into f16 hi + lo (v = hi + lo with
// |v - hi - lo| <= 2^-22 |v| in the f16 normal range) and every product is
// taken as hi*hi + hi*lo + lo*hi, so the result matches fp32 operands to about
// 2^-21 relative while running at the f16 MFMA rate.
//   A (inputs or activations) arrives pre-split in HBM (ah, al: [rows][kdim] f16)
//   and is staged per 64-column slab in LDS.
//   B (weights) is decoded by each wave straight into MFMA fragments: lane l
//   owns row (l % 16) of an N-block and columns 8*(l/16)..+7 of each 32-column
//   group; for Q4_K the slab's two groups are the low and high nibbles of the
//   same 8 bytes (kernels/iq3_mix.metal:19-23 layout).
// GATEUP writes act = SwiGLU(gate, up) already split (out_h, out_l: [P][F] f16);
// the down GEMM writes fp32 Y.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
constexpr uint32_t A16_STRIDE = 72;  // halves per LDS row: 64 + 8 pad (144 B) against bank conflicts

__device__ __forceinline__ void split_f16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// 8 fp32 values -> f16 hi and lo halves (packed pairs, round toward zero:
// hi = rtz(v), lo = rtz(v - hi), |v - hi - lo| < 2^-20 |v|).
__device__ __forceinline__ void split8(const float* v, uint4& hi, uint4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto hp = __builtin_amdgcn_cvt_pkrtz(v[2 * i], v[2 * i + 1]);
        const auto lp = __builtin_amdgcn_cvt_pkrtz(v[2 * i] - (float)hp[0], v[2 * i + 1] - (float)hp[1]);
        h[i] = __builtin_bit_cast(uint32_t, hp);
        l[i] = __builtin_bit_cast(uint32_t, lp);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

constexpr uint32_t TM16 = 64;  // tokens per tile of the f16 GEMM

template <bool GATEUP>
__global__ __launch_bounds__(256) void k_gemm_q4k_f16(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                                      uint64_t stride0, uint64_t stride1, uint32_t rows_per_expert,
                                                      uint32_t kdim, const _Float16* __restrict__ ah,
                                                      const _Float16* __restrict__ al, const uint32_t* __restrict__ pairs,
                                                      uint32_t K, const uint32_t* __restrict__ tiles, uint32_t ldo,
                                                      float limit, float* __restrict__ out, _Float16* __restrict__ out_h,
                                                      _Float16* __restrict__ out_l) {
    constexpr int MB = TM16 / 16;
    // A tiles: 64 halves (128 B) per row, 16-byte chunk c of row r stored at
    // chunk c ^ ((r >> 1) & 7): the stores (4 threads per row) and the MFMA
    // fragment reads (16 rows at one chunk) then touch every bank once.
    __shared__ _Float16 Ash[TM16 * 64];
    __shared__ _Float16 Asl[TM16 * 64];
    const uint32_t* tile = tiles + 4u * blockIdx.y;
    const uint32_t n = tile[2];
    if (n == 0) return;
    const uint32_t e = tile[0], q0 = tile[1];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, kq = lane >> 4;
    const uint32_t row0 = blockIdx.x * (GATEUP ? 64u : 128u);

    // A loader: TM16 rows x 64 halves per part; thread -> row tid / (256 / TM16)
    constexpr uint32_t TPR = 256u / TM16, HPT = 64u / TPR;  // threads per row, halves per thread
    constexpr int AV = HPT / 8;                             // uint4 loads per part
    const uint32_t am = tid / TPR, acol = HPT * (tid % TPR);
    const _Float16 *arow_h = nullptr, *arow_l = nullptr;
    if (am < n) {
        const uint32_t q = q0 + am;
        const uint64_t r = GATEUP ? (pairs ? pairs[q] / K : q) : q;
        arow_h = ah + r * kdim;
        arow_l = al + r * kdim;
    }
    const uint8_t* brow[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        if (GATEUP) {
            const uint32_t r = row0 + 16u * wave + (lane & 15u);
            brow[nb] = (nb == 0 ? w0 : w1) + ((uint64_t)e * rows_per_expert + r) * (nb == 0 ? stride0 : stride1);
        } else {
            const uint32_t r = row0 + 32u * wave + 16u * nb + (lane & 15u);
            brow[nb] = w0 + ((uint64_t)e * rows_per_expert + r) * stride0;
        }
    }

    floatx4 acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // A: one slab ahead (L2-resident inputs). B: one Q4_K superblock (4 slabs)
    // ahead, because weights stream from HBM.
    uint4 pa_h[AV], pa_l[AV];
    auto load_a = [&](uint32_t s) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            pa_h[i] = arow_h ? *reinterpret_cast<const uint4*>(arow_h + 64u * s + acol + 8u * i) : make_uint4(0, 0, 0, 0);
            pa_l[i] = arow_l ? *reinterpret_cast<const uint4*>(arow_l + 64u * s + acol + 8u * i) : make_uint4(0, 0, 0, 0);
        }
    };
    uint4 hdr[2], nhdr[2];
    uint2 qs[2][4], nqs[2][4];
    auto load_b = [&](uint32_t sb) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const uint8_t* b = brow[nb] + sb * 144u;
            nhdr[nb] = *reinterpret_cast<const uint4*>(b);
#pragma unroll
            for (int q = 0; q < 4; ++q) nqs[nb][q] = *reinterpret_cast<const uint2*>(b + 16u + 32u * q + 8u * kq);
        }
    };
    const uint32_t slabs = kdim / 64u, sbs = kdim / 256u;
    load_a(0);
    load_b(0);
    for (uint32_t sb = 0; sb < sbs; ++sb) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            hdr[nb] = nhdr[nb];
#pragma unroll
            for (int q = 0; q < 4; ++q) qs[nb][q] = nqs[nb][q];
        }
        if (sb + 1 < sbs) load_b(sb + 1);
#pragma unroll
        for (uint32_t sq = 0; sq < 4; ++sq) {
            const uint32_t s = 4u * sb + sq;
#pragma unroll
            for (int i = 0; i < AV; ++i) {
                const uint32_t off = am * 64u + 8u * (((acol >> 3) + i) ^ ((am >> 1) & 7u));
                *reinterpret_cast<uint4*>(&Ash[off]) = pa_h[i];
                *reinterpret_cast<uint4*>(&Asl[off]) = pa_l[i];
            }
            // This slab's B fragments: group 0 = low nibbles, group 1 = high nibbles.
            uint4 bh[2][2], bl[2][2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                float d0, m0, d1, m1;
                Fmt<12>::scales(hdr[nb], 2u * sq, d0, m0, d1, m1);
                float v0[8], v1[8];
                const uint32_t wq[2] = {qs[nb][sq].x, qs[nb][sq].y};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t lo = wq[h] & 0x0f0f0f0fu, hi = (wq[h] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        v0[4 * h + j] = d0 * ubyte_f(lo, j) - m0;
                        v1[4 * h + j] = d1 * ubyte_f(hi, j) - m1;
                    }
                }
                split8(v0, bh[nb][0], bl[nb][0]);
                split8(v1, bh[nb][1], bl[nb][1]);
            }
            __syncthreads();
            if (s + 1 < slabs) load_a(s + 1);
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                half8 fbh[2], fbl[2];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    fbh[nb] = __builtin_bit_cast(half8, bh[nb][gi]);
                    fbl[nb] = __builtin_bit_cast(half8, bl[nb][gi]);
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const uint32_t ar = mb * 16u + (lane & 15u);
                    const uint32_t off = ar * 64u + 8u * ((4u * gi + kq) ^ ((ar >> 1) & 7u));
                    const half8 a_h = *reinterpret_cast<const half8*>(&Ash[off]);
                    const half8 a_l = *reinterpret_cast<const half8*>(&Asl[off]);
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, fbh[nb], acc[mb][nb], 0, 0, 0);
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, fbl[nb], acc[mb][nb], 0, 0, 0);
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, fbh[nb], acc[mb][nb], 0, 0, 0);
                    }
                }
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t m = mb * 16u + 4u * kq + j;
            if (m >= n) continue;
            const uint64_t q = q0 + m;
            if (GATEUP) {
                const uint32_t r = row0 + 16u * wave + (lane & 15u);
                _Float16 xh, xl;
                split_f16(swiglu(acc[mb][0][j], acc[mb][1][j], limit), xh, xl);
                out_h[q * ldo + r] = xh;
                out_l[q * ldo + r] = xl;
            } else {
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) out[q * ldo + row0 + 32u * wave + 16u * nb + (lane & 15u)] = acc[mb][nb][j];
            }
        }
}

// x [T][H] fp32 -> xh, xl [T][H] f16 with x = xh + xl (+ O(2^-22 |x|)).
__global__ void k_split_f16(const float* __restrict__ x, uint64_t n, _Float16* __restrict__ xh,
                            _Float16* __restrict__ xl) {
    const uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4u;
    if (i >= n) return;
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    const float a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) split_f16(a[j], xh[i + j], xl[i + j]);
}

// Dense token tiles for the shared expert: tile t = {0, 64 t, min(64, T - 64 t), 0}.
__global__ void k_dense_tiles(uint32_t T, uint32_t cap, uint32_t* __restrict__ tiles) {
    uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= cap) return;
    uint32_t first = t * TM;
    tiles[4 * t] = 0;
    tiles[4 * t + 1] = first < T ? first : 0;
    tiles[4 * t + 2] = first < T ? min(TM, T - first) : 0;
    tiles[4 * t + 3] = 0;
}

// ------------------------------------------------------- prefill: combine
// out[t][i] = sum_k w[t,k] Y[inverse[t*K+k]][i] in route order (kernels/prefill.metal:39),
// + sigmoid(sgl[t]) (or 1) * Ys[t][i] for a shared expert, + res[t][i].
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ Y, const float* __restrict__ Ys,
                                                 const uint32_t* __restrict__ inverse, const float* __restrict__ wts,
                                                 const float* __restrict__ sgl, const float* __restrict__ res,
                                                 uint32_t T, uint32_t H, uint32_t K, float* __restrict__ out) {
    const uint64_t i4 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t per = H / 4u;
    if (i4 >= (uint64_t)T * per) return;
    const uint32_t t = (uint32_t)(i4 / per), c = (uint32_t)(i4 % per) * 4u;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t k = 0; k < K; ++k) {
        uint32_t p = t * K + k;
        float w = wts[p];
        float4 y = *reinterpret_cast<const float4*>(Y + (uint64_t)inverse[p] * H + c);
        s.x += w * y.x; s.y += w * y.y; s.z += w * y.z; s.w += w * y.w;
    }
    if (Ys) {
        float w = sgl ? ingot_det_sigmoid(sgl[t]) : 1.0f;
        float4 y = *reinterpret_cast<const float4*>(Ys + (uint64_t)t * H + c);
        s.x += y.x * w; s.y += y.y * w; s.z += y.z * w; s.w += y.w * w;
    }
    if (res) {
        float4 r = *reinterpret_cast<const float4*>(res + (uint64_t)t * H + c);
        s.x += r.x; s.y += r.y; s.z += r.z; s.w += r.w;
    }
    *reinterpret_cast<float4*>(out + (uint64_t)t * H + c) = s;
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

// Non-finite scan of a device buffer: sets FLAG_NONFINITE in flags.
__global__ void k_check_finite(const float* __restrict__ v, uint64_t n, uint32_t* __restrict__ flags) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool bad = i < n && !isfinite(v[i]);
    if (__any(bad) && (threadIdx.x & 63u) == 0) atomicOr(flags, FLAG_NONFINITE);
}

}  // namespace ingot
