/* CPU oracle for the MoE-layer hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or as the timed CPU baseline).
 * The product path (libingot_moe.so) never calls it.
 *
 * It restates, in plain C++ with no GPU, the reference's MoE layer:
 *   - GGUF block geometry            src/gguf.rs:470-491
 *   - matrix validation              src/metal.rs:1602-1621
 *   - dequantization formulas        kernels/iq3_mix.metal:13-36 (Q4_K,
 *                                    IQ2_XS, IQ3_XXS), kernels/moe.metal:11-89
 *                                    (F32, F16, Q8_0, IQ4_NL)
 *   - softmax top-k routing          src/lib.rs:43-60, kernels/generic.metal:479-494
 *   - sigmoid + bias routing         kernels/glm.metal:81-98
 *   - SwiGLU / GLM clamped SwiGLU    kernels/moe.metal:405-410, kernels/glm.metal:100-103
 *   - combine / shared-expert gate   kernels/moe.metal:412-422, kernels/glm.metal:105-110,
 *                                    tools/check_rust_moe.py:55-75
 *   - RMSNorm + residual             kernels/generic.metal:392-409
 *   - expert dispatch (layout/pairs) kernels/prefill.metal:7-38
 *
 * Two precisions of the expert products: ORACLE_F64 accumulates every dot
 * product, the activation and the combine in double (the parity oracle);
 * ORACLE_F32 accumulates in float (the CPU baseline timed beside the GPU).
 * Routing is fp32 in both, computed by the fixed operation sequence of
 * ingot_amd/csrc/det_math.h so that expert ids are exact.
 *
 * Parity pinning of each function is documented in the test files that
 * check it (tests/test_oracle_*.py).
 */
#pragma once
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_OK = 0, ORACLE_INVALID = 1, ORACLE_NONFINITE = 2 };
enum { ORACLE_F64 = 64, ORACLE_F32 = 32 };
enum { ORACLE_ROUTE_SOFTMAX = 0, ORACLE_ROUTE_SIGMOID = 1 };

typedef struct oracle_matrix {
    const uint8_t* data;
    uint64_t nbytes;
    uint64_t cols, rows, count;
    uint32_t kind;
    uint64_t stride;
} oracle_matrix;

typedef struct oracle_layer {
    uint32_t hidden, experts, top_k, routing;
    float route_scale, swiglu_limit;
    const float* router;        /* [E][H] */
    const float* router_bias;   /* [E] or NULL */
    oracle_matrix gate, up, down;
    int has_shared;
    oracle_matrix shared_gate, shared_up, shared_down;
    const float* shared_gate_vec; /* [H] or NULL */
    const float* norm_gain;       /* [H] or NULL: out = x + MoE(RMSNorm(x)) */
    float norm_eps;
} oracle_layer;

int oracle_geometry(uint32_t kind, uint32_t* block, uint32_t* bytes);
int oracle_validate_matrix(const oracle_matrix* m);

/* One value / one row of a quantized row (row points at the row's first block). */
float oracle_dequant_value(const uint8_t* row, uint32_t kind, uint64_t j);
void oracle_dequant_row(const uint8_t* row, uint32_t kind, uint64_t cols, float* out);

int oracle_route_softmax(const float* logits, uint32_t E, uint32_t K, uint32_t* ids, float* w);
int oracle_route_sigmoid(const float* logits, const float* bias, uint32_t E, uint32_t K,
                         float scale, uint32_t* ids, float* w);
/* logits[t][e] = router logit in the fixed reduction order (+ bias[e] in softmax mode
 * when add_bias != 0). */
void oracle_router_logits(const float* W, const float* x, uint32_t T, uint32_t E, uint32_t H,
                          const float* bias, int add_bias, float* logits);

/* y[r] = sum_j W[r][j] x[j] for a single matrix (count 1), f64 accumulation. */
int oracle_project(const oracle_matrix* m, const float* x, double* y);

/* Full layer: out[T][H]; ids/w [T][K] (may be NULL). threads <= 0: all cores.
 * ORACLE_NONFINITE for a non-finite input, or (after writing out, ids and w)
 * for a non-finite output value. */
int oracle_moe_forward(const oracle_layer* L, const float* x, uint32_t T, float* out,
                       uint32_t* ids, float* w, int precision, int threads);

/* Expert dispatch, kernels/prefill.metal:7-38, with the tile size as a parameter.
 * counts[E], first[E], pairs[P], inverse[P]; tiles[cap][4] = {expert, first, n, mode}
 * with mode = n >= 2; unused tiles are zero. Returns the number of used tiles. */
uint32_t oracle_dispatch(const uint32_t* ids, uint32_t P, uint32_t E, uint32_t tile,
                         uint32_t cap, uint32_t* counts, uint32_t* first,
                         uint32_t* pairs, uint32_t* inverse, uint32_t* tiles);

float oracle_det_expf(float x);
float oracle_det_sigmoid(float x);

#ifdef __cplusplus
}
#endif
