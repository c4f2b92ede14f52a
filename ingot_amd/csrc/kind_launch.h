// Per-format kernel launchers of the MoE layer.
//
// Every kernel templated on a GGUF format (decode gate/up and down, the
// separate shared-expert GEMV pair, the fp32-MFMA grouped GEMM) is
// instantiated in exactly one translation unit, kinds_*.hip, so that the
// formats compile in parallel and each kernel's code object is registered
// once. moe_hip.hip selects the format at run time through these
// declarations. Each launcher returns false when no instantiation covers the
// shape.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// GGML type ids with kernels (src/gguf.rs:470-491): F32, F16, Q4_0, Q8_0,
// Q2_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S,
// IQ4_XS, IQ1_M, BF16, Q2_0.
#define INGOT_KINDS(X) \
    X(0) X(1) X(2) X(8) X(10) X(12) X(13) X(14) X(16) X(17) X(18) X(20) X(21) X(22) X(23) X(29) X(30) X(42)

// Routed down + shared down fused in one decode kernel: (down kind, shared down kind).
#define INGOT_FUSED_DOWN(X) X(17, 8) X(12, 12) X(20, 20) X(8, 8) X(21, 42)
// (routed gate/up kind, shared gate/up kind) pairs whose shared expert runs in
// the routed decode gate/up kernel's free pair slot (configs[2]; the IQ2_S /
// IQ4_XS shared mix of an IQ2_XS-class checkpoint).
#define INGOT_FUSED_GATE_UP(X) X(17, 8) X(22, 23)

namespace ingot {

constexpr int GEMV_RPW = 4;  // rows per wave of the separate gate/up GEMV (1 when that leaves CUs idle)
constexpr int DEC_RPW = 1;   // down rows per wave of the decode down kernel

struct GateUpArgs {
    const uint8_t *g, *u;
    uint64_t gs, us;
    uint32_t F, H;
    const float* x;
    const uint32_t* ids;
    uint32_t K;
    float limit;
    float* act;
};

struct DecGateUpArgs {
    const uint8_t *g, *u;
    uint64_t gs, us;
    uint32_t F, H;
    const float *x, *xstat, *logits, *bias;
    uint32_t E, K, mode;
    float scale, limit;
    uint32_t *ids;
    float* w;
    uint32_t* flags;
    float* act;
    uint32_t pre;  // 1: ids and w hold the routing (k_route ran), inputs of the kernel
    // down matrices whose rows the kernel requests ahead of k_dec_down (NULL: none)
    const uint8_t *pfd = nullptr, *pfs = nullptr;
    uint64_t pfds = 0, pfss = 0;
};

struct DownArgs {
    const uint8_t *down, *sdown;
    uint64_t dstride, sdstride;
    uint32_t H, F, SF;
    const float *act, *sact;
    const uint32_t* ids;
    const float* sgl;
    uint32_t K;
    const float* res;
    float* out;
    uint32_t* flags;  // FLAG_OUT_NONFINITE
};

struct GemmArgs {
    const uint8_t *w0, *w1;
    uint64_t s0, s1;
    uint32_t rows, kdim;
    const float* a;
    const uint32_t* pairs;
    uint32_t K;
    const uint32_t* tiles;
    uint32_t ldo;
    float limit;
    float* out;
    const uint32_t* slot_of;  // cached experts: expert -> device slot (NO_SLOT: skip), or NULL
};

// k_gemv_gate_up: act = SwiGLU(G x, U x) for `pairs` (grid.y) pairs, cpl chunks
// per lane, rpw (GEMV_RPW or 1) rows per wave.
template <int KIND>
bool launch_gemv_gate_up_k(hipStream_t s, uint32_t cpl, uint32_t rpw, dim3 grid, const GateUpArgs& a);
// k_gemv_shared_down_add: out[t] += sigmoid gate * D_s sact[t].
template <int KS>
bool launch_shared_add_k(hipStream_t s, uint32_t cpl, dim3 grid, const uint8_t* sd, uint64_t sds, uint32_t H,
                         uint32_t SF, const float* sact, const float* sgl, float* out, uint32_t* flags);
// k_gemm<KIND, GATEUP>: fp32-MFMA grouped GEMM over dispatch tiles.
template <int KIND, bool GATEUP>
bool launch_gemm_k(hipStream_t s, dim3 grid, const GemmArgs& a);
// k_dec_gate_up2: decode routing + gate/up + SwiGLU (rpw rows per wave, np pairs per wave).
template <int KIND>
bool launch_dec_gate_up_k(hipStream_t s, uint32_t cpl, uint32_t np, uint32_t rpw, dim3 grid, const DecGateUpArgs& a);
// k_dec_down<KD, KS>: decode down + combine (+ shared expert when KS >= 0) + residual.
template <int KD, int KS>
bool launch_dec_down_k(hipStream_t s, uint32_t vpl, dim3 grid, const DownArgs& a);
// k_dec_gate_up2<KIND, .., KS>: the same with the shared expert (format KS, width F)
// in wave 7's free pair slot (K < 8 np); false if no instantiation covers the shape.
template <int KIND, int KS>
bool launch_dec_gate_up_fused_k(hipStream_t s, uint32_t cpl, uint32_t np, uint32_t rpw, dim3 grid,
                                const DecGateUpArgs& a, const uint8_t* sg, const uint8_t* su, uint64_t sgs,
                                uint64_t sus, float* sact);

// Arguments of k_gemm_f16 (its parameters, in order).
struct GemmF16Args {
    const uint8_t *w0, *w1, *ws0, *ws1;
    uint32_t e_shared;
    uint64_t stride0, stride1;
    uint32_t rows_per_expert, kdim;
    const _Float16 *ah, *al;
    const float* gs;
    const uint32_t* pairs;
    uint32_t K;
    const uint32_t* tiles;
    uint32_t ldo;
    float limit;
    float* out;
    _Float16 *out_h, *out_l;
    float* out_gs;
    uint32_t nblk, a_rows;
    const float* xstat;
    uint32_t* rowmax;
    uint32_t* flags;
    const uint32_t* slot_of;
};
// The formats of the f16 grouped GEMM.
#define INGOT_F16_KINDS(X) X(12) X(13) X(14) X(17) X(18) X(20) X(21) X(22) X(23)
// k_gemm_f16<KIND, GATEUP, aord, TT, tl>: TT 128 when tt128 (Q4_K, Q5_K; Q6_K
// always), else 64; false if no instantiation covers the arguments.
template <int KIND, bool GATEUP>
bool launch_gemm_f16_k(hipStream_t s, int aord, bool tt128, bool tl, dim3 grid, const GemmF16Args& a);

#define INGOT_DECLARE_F16(K)                                                                                \
    extern template bool launch_gemm_f16_k<K, true>(hipStream_t, int, bool, bool, dim3, const GemmF16Args&); \
    extern template bool launch_gemm_f16_k<K, false>(hipStream_t, int, bool, bool, dim3, const GemmF16Args&);

#define INGOT_DECLARE_KIND(K)                                                                               \
    extern template bool launch_gemv_gate_up_k<K>(hipStream_t, uint32_t, uint32_t, dim3, const GateUpArgs&); \
    extern template bool launch_shared_add_k<K>(hipStream_t, uint32_t, dim3, const uint8_t*, uint64_t,      \
                                                uint32_t, uint32_t, const float*, const float*, float*,     \
                                                uint32_t*);                                                 \
    extern template bool launch_gemm_k<K, true>(hipStream_t, dim3, const GemmArgs&);                        \
    extern template bool launch_gemm_k<K, false>(hipStream_t, dim3, const GemmArgs&);                       \
    extern template bool launch_dec_gate_up_k<K>(hipStream_t, uint32_t, uint32_t, uint32_t, dim3,           \
                                                 const DecGateUpArgs&);                                     \
    extern template bool launch_dec_down_k<K, -1>(hipStream_t, uint32_t, dim3, const DownArgs&);
INGOT_KINDS(INGOT_DECLARE_KIND)
#undef INGOT_DECLARE_KIND
#define INGOT_DECLARE_FUSED(KD, KS) \
    extern template bool launch_dec_down_k<KD, KS>(hipStream_t, uint32_t, dim3, const DownArgs&);
INGOT_FUSED_DOWN(INGOT_DECLARE_FUSED)
#undef INGOT_DECLARE_FUSED
#define INGOT_DECLARE_FUSED_GU(KG, KS)                                                                          \
    extern template bool launch_dec_gate_up_fused_k<KG, KS>(hipStream_t, uint32_t, uint32_t, uint32_t, dim3, \
                                                            const DecGateUpArgs&, const uint8_t*, const uint8_t*, \
                                                            uint64_t, uint64_t, float*);
INGOT_FUSED_GATE_UP(INGOT_DECLARE_FUSED_GU)
#undef INGOT_DECLARE_FUSED_GU
INGOT_F16_KINDS(INGOT_DECLARE_F16)

}  // namespace ingot
