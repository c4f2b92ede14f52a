/* ingot_moe.h: C ABI of the MI355X (gfx950) backend for Ingot's MoE-layer hot path.
 *
 * The library (ingot_amd/libingot_moe.so, HIP, one GPU) replaces the Metal
 * backend for this path: routing, token-to-expert dispatch, grouped
 * gate/up/SwiGLU/down expert products on GGUF-quantized weights, and the
 * weighted combine. Plain C types only; no torch or HIP types appear here
 * (streams are passed as void*).
 *
 * Reference interfaces each entry point replaces (paths in majiayu000/ingot):
 *   ingot_geometry           gguf::geometry              src/gguf.rs:470-491
 *   ingot_validate_matrix    Gpu::validate_matrix        src/metal.rs:1602-1621
 *   ingot_route              route()                     src/lib.rs:43-60
 *   ingot_ctx_create/destroy Gpu::new / Drop             src/metal.rs:238-533
 *   ingot_device_name        Gpu::name                   src/metal.rs:1247
 *   ingot_project            Gpu::project                src/metal.rs:1622-1632
 *   ingot_dequant            Gpu::dequant                src/metal.rs:1581-1601
 *   ingot_moe                Gpu::moe                    src/metal.rs:1664-1713
 *   ingot_route_batch        route_topk / route_gpu_batch / glm_route kernels
 *                            (kernels/generic.metal:479-494, kernels/qwen.metal:177-180,
 *                            kernels/glm.metal:81-98) as encoded by Generic::ffn
 *                            (src/generic.rs:510-530) and Glm::moe (src/glm.rs:983-991)
 *   ingot_layer_create       resident expert weights: Gpu::load_weight +
 *                            ExpertWeights::Resident (src/metal.rs:546-582,
 *                            src/weights.rs:55-58), built per layer by
 *                            Loader::layers (src/generic_arch.rs:370-376)
 *   ingot_layer_forward      the trunks' MoE FFN call: Generic::ffn MoE branch
 *                            (src/generic.rs:510-574) and moe_packed (:578-662),
 *                            Qwen::ffn (src/qwen.rs:1062-1260), resident_ffn_packed
 *                            (src/qwen_prefill.rs:30-116), Glm::moe (src/glm.rs:974-1060),
 *                            plus the pre-FFN RMSNorm and residual add of
 *                            Generic::hidden (src/generic.rs:716-724) when a norm
 *                            gain is given
 *   ingot_layer_forward_add  the same with the attention output's residual add
 *                            (add_rms, kernels/generic.metal:390-405) fused in
 *   ingot_layer_create_cached
 *                            bounded-memory experts: ExpertWeights::Cached +
 *                            ExpertCache (src/weights.rs:46-95), forwarded as in
 *                            the cached branch of Qwen::ffn (src/qwen.rs:1171-1253)
 *   ingot_expert_cache_*     ExpertCache::hit / ExpertCache::slot (src/weights.rs:59-95)
 *
 * Errors follow the reference: an invalid argument, shape or format is
 * INGOT_INVALID (io::ErrorKind::InvalidData via invalid(), src/lib.rs:39-41);
 * non-finite input or output is INGOT_NONFINITE (src/metal.rs:1575-1577,
 * :1680); a HIP failure is INGOT_DEVICE and is sticky: every later call on the
 * context fails until it is destroyed and recreated (src/metal.rs:170-190,
 * :1349-1353). ingot_last_error() returns the message of the last failure.
 *
 * Threading: a context, and the layers created on it, belong to one host
 * thread at a time (Gpu is !Send in the reference). Synchronous entry points
 * (host buffers) wait for completion; ingot_layer_forward and
 * ingot_route_batch take device pointers and are asynchronous on the
 * context's stream.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ingot_status {
    INGOT_OK = 0,
    INGOT_INVALID = 1,
    INGOT_NONFINITE = 2,
    INGOT_DEVICE = 3,
    INGOT_UNSUPPORTED = 4,
    /* No counterpart in the reference (its fp32 kernels have no operand range
     * limit): reported by ingot_ctx_check_device_flags when an operand of the
     * split-f16 prefill GEMM left the range in which it is exact (see
     * ingot_layer_set_gemm_mode). The outputs of the forwards since the last
     * check are not valid; re-run them with INGOT_GEMM_FP32. */
    INGOT_RANGE = 5
};

/* GGML type ids the kernels decode: every id the reference loader accepts
 * (src/gguf.rs:470-491; ingot_geometry answers for all of them). */
enum ingot_kind {
    INGOT_F32 = 0,
    INGOT_F16 = 1,
    INGOT_Q4_0 = 2,
    INGOT_Q8_0 = 8,
    INGOT_Q2_K = 10,
    INGOT_Q4_K = 12,
    INGOT_Q5_K = 13,
    INGOT_Q6_K = 14,
    INGOT_IQ2_XXS = 16,
    INGOT_IQ2_XS = 17,
    INGOT_IQ3_XXS = 18,
    INGOT_IQ4_NL = 20,
    INGOT_IQ3_S = 21,
    INGOT_IQ2_S = 22,
    INGOT_IQ4_XS = 23,
    INGOT_IQ1_M = 29,
    INGOT_BF16 = 30,
    INGOT_Q2_0 = 42
};

enum ingot_routing { INGOT_ROUTE_SOFTMAX = 0, INGOT_ROUTE_SIGMOID = 1 };

/* gguf::Matrix (src/gguf.rs:462-469): `count` matrices of rows x cols stored
 * back to back, row r of matrix e at byte (e * rows + r) * stride. data is a
 * host pointer to nbytes of GGUF block bytes. */
typedef struct ingot_matrix {
    const uint8_t* data;
    uint64_t nbytes;
    uint64_t cols;
    uint64_t rows;
    uint64_t count;
    uint32_t kind;
    uint64_t stride;
} ingot_matrix;

typedef struct ingot_ctx ingot_ctx;
typedef struct ingot_layer ingot_layer;
typedef struct ingot_graph ingot_graph;

/* ---- host-only helpers (no GPU needed) ---- */
int ingot_geometry(uint32_t kind, uint32_t* block_values, uint32_t* block_bytes);
int ingot_validate_matrix(const ingot_matrix* m);
const char* ingot_status_string(int status);
/* 1 if the kernels decode `kind`, else 0. */
int ingot_kind_supported(uint32_t kind);

/* ---- context ----
 * Lifetime: every layer created on a context (ingot_layer_create, _clone,
 * _create_cached) holds a pointer to it and must be destroyed before it.
 * ingot_ctx_destroy refuses, with INGOT_INVALID and the context left intact,
 * while layers are alive on it (the reference gets the same order from
 * ownership: Gpu owns its buffers, src/metal.rs:46-63). */
int ingot_ctx_create(int device, ingot_ctx** out);
int ingot_ctx_destroy(ingot_ctx* ctx);
const char* ingot_last_error(const ingot_ctx* ctx);
/* Launch on a caller-owned hipStream_t (NULL: the context's own stream). */
int ingot_ctx_set_stream(ingot_ctx* ctx, void* hip_stream);
void* ingot_ctx_stream(const ingot_ctx* ctx);
int ingot_ctx_synchronize(ingot_ctx* ctx);
const char* ingot_device_name(ingot_ctx* ctx);

/* ---- drop-ins for the reference's public Gpu API (host buffers, synchronous) ---- */
/* route(): ids[K] (uint32) and weights[K] for one token's E logits. */
int ingot_route(ingot_ctx* ctx, const float* logits, uint32_t E, uint32_t K, uint32_t* ids, float* weights);
/* Gpu::project: y[rows] = m . x, m.count must be 1. */
int ingot_project(ingot_ctx* ctx, const ingot_matrix* m, const float* x, float* y);
/* Gpu::dequant: out[count * rows * cols] floats. */
int ingot_dequant(ingot_ctx* ctx, const ingot_matrix* m, float* out);
/* Gpu::moe: routed[3] = gate, up, down holding the K selected experts
 * (count = K, expert k uses weights[k]); shared[3] and shared_gate (a
 * [cols = H, rows = 1] matrix) may be NULL for a layer without a shared
 * expert; out[H] = sum_k w_k E_k(x) + sigmoid(shared_gate . x) S(x). */
int ingot_moe(ingot_ctx* ctx, const ingot_matrix routed[3], const ingot_matrix* shared,
              const ingot_matrix* shared_gate, const float* x, const float* weights, uint32_t K,
              float* out);

/* ---- device routing (device pointers, asynchronous) ----
 * logits [T][E]; softmax mode: selection and weights on logits + bias (bias
 * may be NULL); sigmoid mode: selection on sigmoid(l) + bias, weights
 * sigmoid(l) / sum * scale. ids [T][K] uint32, weights [T][K]. A non-finite
 * logit sets the context's device error flag (reported by
 * ingot_ctx_check_device_flags). */
int ingot_route_batch(ingot_ctx* ctx, const float* d_logits, const float* d_bias, uint32_t T, uint32_t E,
                      uint32_t K, uint32_t routing, float scale, uint32_t* d_ids, float* d_weights);
/* Synchronizes, reads and clears the device flags of the context and of every
 * layer on it. Each layer's kernels raise flags in a word of its own; the
 * check records per layer what its forwards raised (ingot_layer_flag_status)
 * and returns the status of the earliest-created flagged layer (else of the
 * context's own ingot_route_batch calls), its message naming that layer:
 * INGOT_NONFINITE if a kernel met a non-finite router logit since the last
 * check, else INGOT_RANGE if a prefill forward's activations left the
 * split-f16 range, else INGOT_NONFINITE if a layer forward wrote a non-finite
 * output value (the device-side form of the reference's read-back check,
 * src/metal.rs:1575-1577). An engine with several layers in one graph
 * recomputes from the first flagged layer of its stack onward (later layers
 * may be flagged only because their input came from it) instead of the whole
 * stack. */
int ingot_ctx_check_device_flags(ingot_ctx* ctx);
/* What the layer's own forwards raised before the last
 * ingot_ctx_check_device_flags (INGOT_OK, INGOT_NONFINITE or INGOT_RANGE; the
 * reference fails the one command whose output is non-finite,
 * src/metal.rs:1575-1577). */
int ingot_layer_flag_status(const ingot_layer* layer);

/* ---- resident layer ---- */
typedef struct ingot_layer_desc {
    uint32_t hidden;         /* H: embedding_length */
    uint32_t experts;        /* E: expert_count */
    uint32_t top_k;          /* K: expert_used_count */
    uint32_t routing;        /* ingot_routing */
    float route_scale;       /* sigmoid mode: weight scale (GLM expert_weights_scale); softmax: 1 */
    float swiglu_limit;      /* 0: plain SwiGLU; > 0: GLM clamp g <= L, |u| <= L */
    const float* router;     /* host [E][H] fp32 (ffn_gate_inp) */
    const float* router_bias;/* host [E] or NULL (softmax: added to logits; sigmoid: selection only) */
    ingot_matrix gate;       /* routed experts [cols H, rows F, count E] */
    ingot_matrix up;         /* [H, F, E] */
    ingot_matrix down;       /* [F, H, E] */
    ingot_matrix shared_gate;/* optional shared expert [H, SF, 1] (data NULL: none) */
    ingot_matrix shared_up;  /* [H, SF, 1] */
    ingot_matrix shared_down;/* [SF, H, 1] */
    const float* shared_gate_vec; /* host [H] or NULL: shared expert scaled by sigmoid(v . x), else by 1 */
    const float* norm_gain;  /* host [H] or NULL: out = x + MoE(RMSNorm(x)) */
    float norm_eps;
} ingot_layer_desc;

/* Copies the layer to device memory (every expert resident). A matrix in a
 * format the f16 prefill GEMM decodes (rows a multiple of 16) gets a second
 * copy at the first ingot_layer_reserve (or forward) of a batch that takes
 * the prefill path: the same bytes reordered so that each of that GEMM's
 * weight loads reads one contiguous span. It doubles those matrices' device
 * memory; a layer that only decodes never makes it. */
int ingot_layer_create(ingot_ctx* ctx, const ingot_layer_desc* desc, ingot_layer** out);
/* A second resident copy of the same weights at new device addresses (not for
 * cached layers). */
int ingot_layer_clone(const ingot_layer* src, ingot_layer** out);
/* A layer whose routed experts stay in the caller's host memory (desc's gate,
 * up and down bytes, which must stay valid and unchanged while the layer
 * lives) and are copied on demand into `slots` device expert slots, 1 <= slots
 * <= E (router, vectors and the shared expert are resident). ingot_layer_forward
 * on it routes on the device, reads the routing back to the host, then runs
 * the routed experts in order of first use in passes of at most `slots`
 * experts: each expert of a pass takes a hit slot or the least recently used
 * slot that the pass has not claimed (an empty slot first, ties to the lower
 * slot), a miss copies the expert's bytes into it, and the pass's grouped
 * products run on those slots. The forward synchronizes the context stream,
 * cannot be captured into a graph (INGOT_INVALID), and has no allocation-free
 * variant. Outputs equal a resident layer's bit for bit. */
int ingot_layer_create_cached(ingot_ctx* ctx, const ingot_layer_desc* desc, uint32_t slots, ingot_layer** out);
/* Counters of a cached layer since creation: hits, misses and bytes copied
 * into slots. */
int ingot_layer_cache_stats(const ingot_layer* layer, uint64_t* hits, uint64_t* misses, uint64_t* bytes);

/* The cache policy alone, on the host (no device): for tests of it.
 * hit: the slot holding expert `id`, its age refreshed, or -1.
 * claim: the slot for `id` before a read: a hit (*load = 0), or the least
 *   recently used slot not among pinned[npinned], emptied (*load = 1: read the
 *   expert, then commit); -1 when every slot is pinned ("no reusable expert
 *   slot"), leaving the slots unchanged. A read that fails is simply not
 *   committed: the slot stays empty.
 * state: ids[slots] (-1: empty), hits and misses (a miss counts at commit). */
typedef struct ingot_expert_cache ingot_expert_cache;
ingot_expert_cache* ingot_expert_cache_create(uint32_t slots);
void ingot_expert_cache_destroy(ingot_expert_cache* cache);
int ingot_expert_cache_hit(ingot_expert_cache* cache, uint32_t id);
int ingot_expert_cache_claim(ingot_expert_cache* cache, uint32_t id, const uint32_t* pinned, uint32_t npinned,
                             int* load);
int ingot_expert_cache_commit(ingot_expert_cache* cache, uint32_t slot, uint32_t id);
int ingot_expert_cache_state(const ingot_expert_cache* cache, int64_t* ids, uint64_t* hits, uint64_t* misses);
void ingot_layer_destroy(ingot_layer* layer);
/* Reserve workspace for up to T tokens, and make the prefill GEMM's weight
 * copies when T tokens take the prefill path (done implicitly by forward;
 * call it before graph capture, which must not allocate). */
int ingot_layer_reserve(ingot_layer* layer, uint32_t T);
/* out[T][H] = layer(x[T][H]); device pointers, asynchronous on the context
 * stream. d_ids [T][K] / d_weights [T][K] receive the routing when non-NULL.
 * A non-finite router logit or output value sets the context's device flags
 * (ingot_ctx_check_device_flags). */
int ingot_layer_forward(ingot_layer* layer, const float* d_x, uint32_t T, float* d_out, uint32_t* d_ids,
                        float* d_weights);
/* No counterpart in the reference: the same forward as ingot_layer_forward for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc or
 * hipFree: its workspace is a static device array of 32 MiB (33554432 bytes)
 * per GPU, held from the library's first context on that GPU until the
 * process ends, and T is limited to what fits (ingot_layer_static_bytes; a
 * larger T is INGOT_INVALID): every decode and MTP-verify batch of the
 * configurations here, and prefill up to about 200 tokens of a
 * Qwen3-30B-A3B-shaped layer. Every static forward on one GPU shares that
 * array, so calls that overlap on one GPU (other streams, other threads, other
 * contexts) race; the array keeps the last call's contents. */
int ingot_layer_forward_static(ingot_layer* layer, const float* d_x, uint32_t T, float* d_out, uint32_t* d_ids,
                               float* d_weights);
/* Bytes of workspace a forward of T tokens of this layer uses. */
uint64_t ingot_layer_static_bytes(const ingot_layer* layer, uint32_t T);
/* out[T][H] = s + MoE(RMSNorm(s)) with s = x + a: the residual add before the
 * pre-FFN norm fused into the router, replacing add_rms (kernels/generic.metal:
 * 390-405, called as rms(x, Some(a), ffn_norm) at src/generic.rs:716-724)
 * followed by the MoE FFN and its residual add. Needs a layer created with a
 * norm gain (else INGOT_INVALID); otherwise as ingot_layer_forward. */
int ingot_layer_forward_add(ingot_layer* layer, const float* d_x, const float* d_a, uint32_t T, float* d_out,
                            uint32_t* d_ids, float* d_weights);
/* Prefill GEMM arithmetic. INGOT_GEMM_AUTO (default): experts in Q4_K, Q5_K,
 * Q6_K, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S (these four with rows of a multiple of
 * 512 columns), IQ4_NL and IQ4_XS use the split-precision f16 MFMA GEMM
 * (fp32-accurate to ~2^-21 relative: each operand is scaled by a power of two
 * per token and split into f16 hi + lo; the B operand is the format's integer,
 * for Q6_K an f16-rounded part and its exact remainder), other formats the fp32
 * MFMA GEMM. x may take any finite values. The activations are scaled by
 * 2^(2 e_t - 15) (e_t the exponent that brings the token's max |x| into
 * [2^10, 2^11)); when a row's max |act| so scaled leaves [2^-3, 2^14) (weights
 * far from the usual size) the forward raises the device flag that
 * ingot_ctx_check_device_flags reports as INGOT_RANGE, and its outputs must
 * be recomputed with INGOT_GEMM_FP32.
 * INGOT_GEMM_FP32: always the fp32 MFMA GEMM. */
enum ingot_gemm_mode { INGOT_GEMM_AUTO = 0, INGOT_GEMM_FP32 = 1 };
int ingot_layer_set_gemm_mode(ingot_layer* layer, uint32_t mode);
/* Device bytes held by the layer's weights (with the reordered copies). */
uint64_t ingot_layer_weight_bytes(const ingot_layer* layer);

/* ---- graphs and timing on the context stream ---- */
int ingot_graph_begin(ingot_ctx* ctx);
int ingot_graph_end(ingot_ctx* ctx, ingot_graph** out);
int ingot_graph_launch(ingot_ctx* ctx, ingot_graph* g);
void ingot_graph_destroy(ingot_graph* g);
/* Records HIP events around `launches` replays of g on the context stream and
 * returns the elapsed milliseconds. */
int ingot_graph_time(ingot_ctx* ctx, ingot_graph* g, uint32_t launches, float* ms);

/* Kernel-level timing for roofline reporting: captures `reps` replays of one
 * stage of the last forward of `layer` (same inputs, which must still be
 * allocated) in a HIP graph, launches it once to warm up, then times one
 * launch between HIP events on the context stream and returns the mean
 * milliseconds per stage launch.
 * stage: 0 router, 1 route, 2 gate/up, 3 down (+combine at decode), 4 combine,
 * 5 dispatch. Returns INGOT_INVALID if the stage did not run in that forward,
 * if a reserve has reallocated the workspace since, and for cached layers
 * (their GEMM stages exist only inside a forward's expert passes). */
int ingot_layer_time_stage(ingot_layer* layer, uint32_t stage, uint32_t reps, float* ms);
/* The same over n layers (resident copies) replayed round-robin, so that
 * consecutive launches read weights at different addresses. */
int ingot_layers_time_stage(ingot_layer* const* layers, uint32_t n, uint32_t stage, uint32_t reps, float* ms);
/* Name of the HIP kernel that implements `stage` in the last forward. */
const char* ingot_layer_stage_kernel(const ingot_layer* layer, uint32_t stage);
/* The prefill dispatch of the last forward (synchronizes; INGOT_INVALID if that
 * forward ran the decode kernels, was a static forward, or a reserve has
 * reallocated the workspace since), P = T * K pairs: counts[E] and first[E]
 * (expert_layout), pairs[P + S] (expert_pairs; S = T when the shared expert ran
 * in the same GEMM launches, its rows P + t naming token t as t K, else 0),
 * inverse[P], tiles[min(tiles_cap, info[2])][4] = {expert (E: the shared
 * expert), first packed pair, n, number of non-empty tiles}; info[4] receives
 * {P, S, length of the tile list, pairs per tile (64, or 128 when T > 64,
 * T K >= 32 E and both projections are Q4_K, Q5_K or Q6_K on the f16 GEMM)}.
 * pairs must hold P + T
 * entries. The
 * reference's counterparts are the layout, pairs and tile buffers of
 * kernels/prefill.metal:7-38 (src/qwen_prefill.rs:30-116); this accessor exists
 * for parity tests of those integer arrays. */
int ingot_layer_dispatch_debug(ingot_layer* layer, uint32_t* counts, uint32_t* first, uint32_t* pairs,
                               uint32_t* inverse, uint32_t* tiles, uint32_t tiles_cap, uint32_t* info);

/* ---- device memory helpers (so callers without a tensor library can drive it) ---- */
int ingot_malloc(ingot_ctx* ctx, uint64_t bytes, void** d_ptr);
int ingot_free(ingot_ctx* ctx, void* d_ptr);
int ingot_memcpy_h2d(ingot_ctx* ctx, void* d_dst, const void* h_src, uint64_t bytes);
int ingot_memcpy_d2h(ingot_ctx* ctx, void* h_dst, const void* d_src, uint64_t bytes);
/* Free and total device memory of the context's GPU (hipMemGetInfo). */
int ingot_device_mem_info(ingot_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes);
/* Device-to-device copy by a plain streaming HIP kernel (16 bytes per lane,
 * bytes a multiple of 16). No counterpart in the reference: it is the known-size
 * workload against which hardware byte counters (FETCH_SIZE, WRITE_SIZE) are
 * calibrated. */
int ingot_device_copy(ingot_ctx* ctx, void* d_dst, const void* d_src, uint64_t bytes);
/* Streaming read of `bytes` (a multiple of 16) at d_src by a plain HIP kernel,
 * asynchronous on the context stream (graph-capturable); d_sink must hold
 * max(1, ceil(bytes / 16384)) words, which the kernel almost never writes.
 * bytes == 0 launches an empty kernel. No counterpart in the reference's MoE
 * path: it is the floor of a decode stage reading the same bytes from HBM,
 * like the reference's STREAM bench (src/expert_bench.rs:203-290). */
int ingot_device_read(ingot_ctx* ctx, const void* d_src, uint64_t bytes, uint32_t* d_sink);

#ifdef __cplusplus
}
#endif
