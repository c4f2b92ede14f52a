// Definitions of the per-format launchers declared in kind_launch.h. Included
// only by the kinds_*.hip translation units, each of which instantiates the
// formats it owns with INGOT_INSTANTIATE_KIND / INGOT_INSTANTIATE_FUSED.
#pragma once
#include "kind_launch.h"
#define INGOT_KIND_UNIT  // leave out the format-independent kernels
#include "moe_kernels.cuh"

namespace ingot {

template <int KIND>
bool launch_gemv_gate_up_k(hipStream_t s, uint32_t cpl, uint32_t rpw, dim3 grid, const GateUpArgs& a) {
#define GU(C, R)                                                                                                  \
    hipLaunchKernelGGL((k_gemv_gate_up<KIND, C, R>), grid, dim3(256), 0, s, a.g, a.u, a.gs, a.us, a.F, a.H, a.x, \
                       a.ids, a.K, a.limit, a.act)
    if (rpw == 1) {
        if (cpl == 1) { GU(1, 1); return true; }
        if (cpl == 2) { GU(2, 1); return true; }
        return false;
    }
    if (cpl == 1) { GU(1, GEMV_RPW); return true; }
    if (cpl == 2) { GU(2, GEMV_RPW); return true; }
#undef GU
    return false;
}

template <int KS>
bool launch_shared_add_k(hipStream_t s, uint32_t cpl, dim3 grid, const uint8_t* sd, uint64_t sds, uint32_t H,
                         uint32_t SF, const float* sact, const float* sgl, float* out, uint32_t* flags) {
    if (cpl == 1) {
        hipLaunchKernelGGL((k_gemv_shared_down_add<KS, 1>), grid, dim3(256), 0, s, sd, sds, H, SF, sact, sgl, out,
                           flags);
        return true;
    }
    if (cpl == 2) {
        hipLaunchKernelGGL((k_gemv_shared_down_add<KS, 2>), grid, dim3(256), 0, s, sd, sds, H, SF, sact, sgl, out,
                           flags);
        return true;
    }
    return false;
}

template <int KIND, bool GATEUP>
bool launch_gemm_k(hipStream_t s, dim3 grid, const GemmArgs& a) {
    hipLaunchKernelGGL((k_gemm<KIND, GATEUP>), grid, dim3(256), 0, s, a.w0, a.w1, a.s0, a.s1, a.rows, a.kdim, a.a,
                       a.pairs, a.K, a.tiles, a.ldo, a.limit, a.out, a.slot_of);
    return true;
}

template <int KIND, int NE>
static bool dec_gate_up_cpl(hipStream_t s, uint32_t cpl, uint32_t np, uint32_t rpw, dim3 grid,
                            const DecGateUpArgs& a) {
    // routing precomputed by k_route (a.pre): the instantiation that reads it, above 128 experts only
#define DGU_(C, N, R, P)                                                                                         \
    hipLaunchKernelGGL((k_dec_gate_up2<KIND, C, R, N, NE, -1, P>), grid, dim3(512), 0, s, a.g, a.u, a.gs, a.us,  \
                       a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit, a.ids, a.w, \
                       a.flags, a.act, nullptr, nullptr, 0, 0, nullptr, a.pfd, a.pfds, a.pfs, a.pfss)
#define DGU(C, N, R)                     \
    do {                                 \
        if (NE > 2 && a.pre) DGU_(C, N, R, (NE > 2)); \
        else DGU_(C, N, R, false);       \
    } while (0)
    if (rpw == 3) {
        if (cpl == 1 && np == 1) { DGU(1, 1, 3); return true; }
        return false;
    }
    if (cpl == 1 && np == 1) { DGU(1, 1, 2); return true; }
    if (cpl == 1 && np == 2) { DGU(1, 2, 2); return true; }
    if (cpl == 2 && np == 1) { DGU(2, 1, 2); return true; }
    if (cpl == 2 && np == 2) { DGU(2, 2, 2); return true; }
#undef DGU
#undef DGU_
    return false;
}

// Candidates per lane of the routing (E <= 64 NE): 2 up to 128 experts, 8 for
// the IQ2_XS 512-expert shape, 16 otherwise (one instantiation per count
// keeps each kernel's code small).
template <int KIND>
bool launch_dec_gate_up_k(hipStream_t s, uint32_t cpl, uint32_t np, uint32_t rpw, dim3 grid, const DecGateUpArgs& a) {
    if (a.E <= 128) return dec_gate_up_cpl<KIND, 2>(s, cpl, np, rpw, grid, a);
    if constexpr (KIND == 17)
        if (a.E <= 512 && cpl == 1 && np == 2 && rpw == 2) {
            // one token, K <= 12: twelve waves of one pair each (with eight,
            // the waves holding two pairs set the kernel's end); batches keep
            // eight-wave blocks, two of which fit a CU
            if (a.K <= 12 && !a.pre) {
                hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 1, 8, -1, false, 12>), grid, dim3(768), 0, s, a.g, a.u,
                                   a.gs, a.us, a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale,
                                   a.limit, a.ids, a.w, a.flags, a.act, nullptr, nullptr, 0, 0, nullptr, a.pfd, a.pfds,
                                   a.pfs, a.pfss);
                return true;
            }
            if (a.pre)
                hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 2, 8, -1, true>), grid, dim3(512), 0, s, a.g, a.u, a.gs,
                                   a.us, a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit,
                                   a.ids, a.w, a.flags, a.act, nullptr, nullptr, 0, 0, nullptr, a.pfd, a.pfds, a.pfs,
                                   a.pfss);
            else
                hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 2, 8>), grid, dim3(512), 0, s, a.g, a.u, a.gs, a.us,
                                   a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit, a.ids,
                                   a.w, a.flags, a.act, nullptr, nullptr, 0, 0, nullptr, a.pfd, a.pfds, a.pfs, a.pfss);
            return true;
        }
    return dec_gate_up_cpl<KIND, 16>(s, cpl, np, rpw, grid, a);
}

template <int KIND, int KS>
bool launch_dec_gate_up_fused_k(hipStream_t s, uint32_t cpl, uint32_t np, uint32_t rpw, dim3 grid,
                                const DecGateUpArgs& a, const uint8_t* sg, const uint8_t* su, uint64_t sgs,
                                uint64_t sus, float* sact) {
    // the configs[2] shape: 512 experts, one chunk per lane, two pairs per wave, 2 rows
    if (a.E > 512 || a.E <= 128 || cpl != 1 || np != 2 || rpw != 2) return false;
    if (a.K + 1 <= 12 && !a.pre) {  // one token: twelve waves, one pair each, the shared expert in wave 11
        hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 1, 8, KS, false, 12>), grid, dim3(768), 0, s, a.g, a.u, a.gs,
                           a.us, a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit, a.ids,
                           a.w, a.flags, a.act, sg, su, sgs, sus, sact, a.pfd, a.pfds, a.pfs, a.pfss);
        return true;
    }
    if (a.pre)
        hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 2, 8, KS, true>), grid, dim3(512), 0, s, a.g, a.u, a.gs, a.us,
                           a.F, a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit, a.ids, a.w,
                           a.flags, a.act, sg, su, sgs, sus, sact, a.pfd, a.pfds, a.pfs, a.pfss);
    else
        hipLaunchKernelGGL((k_dec_gate_up2<KIND, 1, 2, 2, 8, KS>), grid, dim3(512), 0, s, a.g, a.u, a.gs, a.us, a.F,
                           a.H, a.x, a.xstat, a.logits, a.bias, a.E, a.K, a.mode, a.scale, a.limit, a.ids, a.w, a.flags,
                           a.act, sg, su, sgs, sus, sact, a.pfd, a.pfds, a.pfs, a.pfss);
    return true;
}

template <int KD, int KS>
bool launch_dec_down_k(hipStream_t s, uint32_t vpl, dim3 grid, const DownArgs& a) {
#define DD(V)                                                                                                      \
    case V:                                                                                                        \
        hipLaunchKernelGGL((k_dec_down<KD, KS, V, DEC_RPW>), grid, dim3(DOWN_THREADS), 0, s, a.down, a.dstride,    \
                           a.sdown, a.sdstride, a.H, a.F, a.SF, a.act, a.sact, a.ids, a.sgl, a.K, a.res, a.out,    \
                           a.flags);                                                                       \
        return true;
    switch (vpl) {
        DD(1) DD(2) DD(3) DD(4) DD(5) DD(6)  // K F + SF <= DOWN_LDS_FLOATS: at most 384 chunks
        default: return false;
    }
#undef DD
}

template <int KIND, bool GATEUP>
bool launch_gemm_f16_k(hipStream_t s, int aord, bool tt128, bool tl, dim3 grid, const GemmF16Args& a) {
    // Q4_K and Q5_K have both tile sizes, Q6_K only TT 128, the others only TT 64.
    constexpr bool T128 = KIND == 12 || KIND == 13 || KIND == 14, T64 = KIND != 14;
#define F16L(AO, TT, TLV)                                                                                        \
    hipLaunchKernelGGL((k_gemm_f16<KIND, GATEUP, AO, TT, TLV>), grid, dim3(2 * TT), 0, s, a.w0, a.w1, a.ws0,     \
                       a.ws1, a.e_shared, a.stride0, a.stride1, a.rows_per_expert, a.kdim, a.ah, a.al, a.gs,     \
                       a.pairs, a.K, a.tiles, a.ldo, a.limit, a.out, a.out_h, a.out_l, a.out_gs, a.nblk,        \
                       a.a_rows, a.xstat, a.rowmax, a.flags, a.slot_of)
#define F16T(AO, TT)                    \
    do {                                \
        if (tl) F16L(AO, TT, true);     \
        else F16L(AO, TT, false);       \
        return true;                    \
    } while (0)
#define F16A(TT)                                  \
    do {                                          \
        if constexpr (GATEUP) {                   \
            switch (aord) {                       \
                case A_IQ4NL: F16T(A_IQ4NL, TT);  \
                case A_IQ3XXS: F16T(A_IQ3XXS, TT); \
                case A_Q6K: F16T(A_Q6K, TT);      \
                case A_F32: F16T(A_F32, TT);      \
                default: F16T(A_NATURAL, TT);     \
            }                                     \
        } else {                                  \
            F16T(A_NATURAL, TT);                  \
        }                                         \
    } while (0)
    if (tt128 || !T64) {
        if constexpr (T128) F16A(128);
        return false;
    }
    if constexpr (T64) F16A(64);
    return false;
#undef F16A
#undef F16T
#undef F16L
}

}  // namespace ingot

#define INGOT_INSTANTIATE_F16(K)                                                                          \
    namespace ingot {                                                                                     \
    template bool launch_gemm_f16_k<K, true>(hipStream_t, int, bool, bool, dim3, const GemmF16Args&);  \
    template bool launch_gemm_f16_k<K, false>(hipStream_t, int, bool, bool, dim3, const GemmF16Args&); \
    }

#define INGOT_INSTANTIATE_KIND(K)                                                                                \
    namespace ingot {                                                                                            \
    template bool launch_gemv_gate_up_k<K>(hipStream_t, uint32_t, uint32_t, dim3, const GateUpArgs&);            \
    template bool launch_shared_add_k<K>(hipStream_t, uint32_t, dim3, const uint8_t*, uint64_t, uint32_t,        \
                                         uint32_t, const float*, const float*, float*, uint32_t*);               \
    template bool launch_gemm_k<K, true>(hipStream_t, dim3, const GemmArgs&);                                    \
    template bool launch_gemm_k<K, false>(hipStream_t, dim3, const GemmArgs&);                                   \
    template bool launch_dec_gate_up_k<K>(hipStream_t, uint32_t, uint32_t, uint32_t, dim3, const DecGateUpArgs&); \
    template bool launch_dec_down_k<K, -1>(hipStream_t, uint32_t, dim3, const DownArgs&);                        \
    }

#define INGOT_INSTANTIATE_FUSED(KD, KS) \
    namespace ingot {                   \
    template bool launch_dec_down_k<KD, KS>(hipStream_t, uint32_t, dim3, const DownArgs&); \
    }
#define INGOT_INSTANTIATE_FUSED_GATE_UP(KG, KS)                                                                  \
    namespace ingot {                                                                                            \
    template bool launch_dec_gate_up_fused_k<KG, KS>(hipStream_t, uint32_t, uint32_t, uint32_t, dim3,           \
                                                     const DecGateUpArgs&, const uint8_t*, const uint8_t*, uint64_t, \
                                                     uint64_t, float*);                                          \
    }
