// C ABI of the MI355X MoE-layer backend (declared in include/ingot_moe.h).
// Host code: argument validation with the reference's error contract,
// device residency of expert weights, workspace, kernel selection, HIP graphs
// and event timing. Kernels live in moe_kernels.cuh.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "../../include/ingot_moe.h"
#include "kind_launch.h"
#include "moe_kernels.cuh"

using namespace ingot;

// Device flag words of a context: word 0 belongs to the context's own calls
// (ingot_route, ingot_route_batch), word i >= 1 to the layer attached to slot
// i, so that a check can name the layer whose kernels raised a flag.
constexpr uint32_t FLAG_WORDS = 1024;

struct ingot_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    bool poisoned = false;
    std::string err;
    std::string name;
    uint32_t* d_flags = nullptr;  // FLAG_WORDS words
    void* scratch = nullptr;  // this device's copy of `scratch` (hipGetSymbolAddress)
    hipStream_t copy = nullptr;  // cached layers' expert copies (created with the first one)
    std::vector<ingot_layer*> slot{nullptr};  // slot[i]: the live layer owning flag word i (slot 0 unused)
    uint32_t live = 0;                         // live layers on this context
    uint32_t next_seq = 0;                     // creation number of the next layer
};

// Workspace of the allocation-free forward (ingot_layer_forward_static): one
// copy per device, held by every GPU the library runs on until the process
// ends. Host code never passes the array's name to a kernel (in host code it is
// a stand-in, not a device address): ingot_ctx_create looks up this device's
// address once with hipGetSymbolAddress and keeps it in ctx->scratch. All
// static forwards on one GPU share it, so calls that overlap on one GPU race.
constexpr uint64_t STATIC_SCRATCH_BYTES = 32ull << 20;
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

struct ingot_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

int fail(ingot_ctx* ctx, int status, const std::string& msg) {
    if (ctx) {
        ctx->err = msg;
        if (status == INGOT_DEVICE) ctx->poisoned = true;
    }
    return status;
}

#define HIP_TRY(ctx, call)                                                                        \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return fail((ctx), INGOT_DEVICE, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define CHECK_CTX(ctx)                                                                       \
    do {                                                                                     \
        if (!(ctx)) return INGOT_INVALID;                                                    \
        if ((ctx)->poisoned) return fail((ctx), INGOT_DEVICE, "device failed earlier: recreate the context"); \
        HIP_TRY((ctx), hipSetDevice((ctx)->device));                                         \
    } while (0)

#define LAUNCH_CHECK(ctx)                                                                         \
    do {                                                                                          \
        hipError_t e_ = hipGetLastError();                                                        \
        if (e_ != hipSuccess) return fail((ctx), INGOT_DEVICE, std::string("kernel launch: ") + hipGetErrorString(e_)); \
    } while (0)

bool all_finite(const float* v, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) return false;
    return true;
}

int geometry(uint32_t kind, uint32_t* block, uint32_t* bytes) {
    uint32_t b = 0, n = 0;
    switch (kind) {  // src/gguf.rs:470-491
        case 0: b = 1; n = 4; break;
        case 1: case 30: b = 1; n = 2; break;
        case 2: b = 32; n = 18; break;
        case 8: b = 32; n = 34; break;
        case 10: b = 256; n = 84; break;
        case 12: b = 256; n = 144; break;
        case 13: b = 256; n = 176; break;
        case 14: b = 256; n = 210; break;
        case 16: b = 256; n = 66; break;
        case 17: b = 256; n = 74; break;
        case 18: b = 256; n = 98; break;
        case 20: b = 32; n = 18; break;
        case 21: b = 256; n = 110; break;
        case 22: b = 256; n = 82; break;
        case 23: b = 256; n = 136; break;
        case 29: b = 256; n = 56; break;
        case 42: b = 64; n = 18; break;
        default: return INGOT_INVALID;
    }
    if (block) *block = b;
    if (bytes) *bytes = n;
    return INGOT_OK;
}

bool supported(uint32_t kind) {
    switch (kind) {
#define K_(KV) case KV:
        INGOT_KINDS(K_)
#undef K_
        return true;
        default: return false;
    }
}

// src/metal.rs:1602-1621.
int validate(const ingot_matrix* m) {
    uint32_t block, bytes;
    if (!m || geometry(m->kind, &block, &bytes) != INGOT_OK) return INGOT_INVALID;
    if (m->cols == 0 || m->rows == 0 || m->count == 0 || m->cols % block) return INGOT_INVALID;
    if (m->stride != m->cols / block * bytes) return INGOT_INVALID;
    unsigned __int128 total = (unsigned __int128)m->stride * m->rows * m->count;
    if (total != m->nbytes) return INGOT_INVALID;
    const uint64_t lim = 0xffffffffull;
    if (m->cols > lim || m->rows > lim || m->count > lim || m->stride > lim) return INGOT_INVALID;
    if (!m->data) return INGOT_INVALID;
    return INGOT_OK;
}

struct DevMatrix {
    uint8_t* d = nullptr;
    uint8_t* t = nullptr;  // the same bytes in the f16 GEMM's tiled layout (tiled_kind), or NULL
    uint64_t nbytes = 0, cols = 0, rows = 0, count = 0, stride = 0;
    uint32_t kind = 0;
};

// Device allocations of one synchronous call, freed on every return path.
struct DevScope {
    std::vector<void*> p;
    DevScope() = default;
    DevScope(const DevScope&) = delete;
    DevScope& operator=(const DevScope&) = delete;
    ~DevScope() {
        for (void* q : p) (void)hipFree(q);
    }
    template <typename T>
    hipError_t alloc(T** d, uint64_t bytes) {
        void* q = nullptr;
        const hipError_t e = hipMalloc(&q, bytes);
        if (e == hipSuccess) p.push_back(q);
        *d = static_cast<T*>(q);
        return e;
    }
};

int upload_matrix(ingot_ctx* ctx, const ingot_matrix* m, DevMatrix* out) {
    uint8_t* d = nullptr;
    HIP_TRY(ctx, hipMalloc(&d, m->nbytes));
    const hipError_t e = hipMemcpy(d, m->data, m->nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(ctx, INGOT_DEVICE, std::string("hipMemcpy: ") + hipGetErrorString(e));
    }
    out->d = d;
    out->nbytes = m->nbytes;
    out->cols = m->cols;
    out->rows = m->rows;
    out->count = m->count;
    out->stride = m->stride;
    out->kind = m->kind;
    return INGOT_OK;
}

// An upload into a scope's allocation (freed with the scope).
int upload_scoped(ingot_ctx* ctx, DevScope& sc, const ingot_matrix* m, DevMatrix* out) {
    const int st = upload_matrix(ctx, m, out);
    if (st == INGOT_OK) sc.p.push_back(out->d);
    return st;
}

// Formats with a tiled layout for the f16 GEMM (k_tile_weights): every f16
// GEMM format, for the column counts the f16 GEMM takes them at, in whole
// 16-row groups.
bool tiled_kind(const DevMatrix& m) {
    bool cols_ok = false;
    switch (m.kind) {
        case 12: case 13: case 14: case 23: cols_ok = m.cols % 256 == 0; break;
        case 17: case 18: case 21: case 22: cols_ok = m.cols % 512 == 0; break;
        case 20: cols_ok = m.cols % 64 == 0; break;
        default: break;
    }
    return cols_ok && m.rows % 16 == 0;
}

// m->t = m->d in the tiled layout (resident layers, at the first reserve of a
// batch that takes the prefill path; the decode kernels and the fp32 GEMM
// keep reading m->d).
int make_tiled(ingot_ctx* ctx, DevMatrix* m) {
    if (!m->d || m->t || !tiled_kind(*m)) return INGOT_OK;
    // The copy is optional: without room for it the GEMM keeps reading GGUF order.
    if (hipMalloc(reinterpret_cast<void**>(&m->t), m->nbytes) != hipSuccess) {
        (void)hipGetLastError();
        m->t = nullptr;
        return INGOT_OK;
    }
    const uint64_t blocks = std::min<uint64_t>((m->nbytes + 255) / 256, 1u << 20);
    hipLaunchKernelGGL(k_tile_weights, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, m->d, m->t, m->nbytes,
                       m->kind, m->stride);
    HIP_TRY(ctx, hipGetLastError());
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return INGOT_OK;
}

template <typename T>
int upload(ingot_ctx* ctx, const T* h, uint64_t n, T** d) {
    HIP_TRY(ctx, hipMalloc(reinterpret_cast<void**>(d), sizeof(T) * n));
    const hipError_t e = hipMemcpy(*d, h, sizeof(T) * n, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(*d);
        *d = nullptr;
        return fail(ctx, INGOT_DEVICE, std::string("hipMemcpy: ") + hipGetErrorString(e));
    }
    return INGOT_OK;
}

// ------------------------------------------------------------------ launchers
// Each returns false if no instantiation covers the shape.

bool launch_router(hipStream_t s, uint32_t HB, uint32_t T, uint32_t E, bool has_sg, const float* x,
                   const float* addend, const float* W, const float* sgvec, const float* gain, float eps,
                   float* logits, float* sgl, float* xn, float* xs, float* xstat) {
    const uint32_t rows = E + (has_sg ? 1u : 0u);
    // Below 64 tokens one token and one router row per wave keeps the grid
    // wide (T x E / 4 blocks); from 64 tokens the transposed kernel (H of
    // 1024 or 2048).
    const bool decode = T < 64;
    if (!decode && E % 32u == 0 && (HB == 4 || HB == 8)) {
        // 4 tokens per wave (16 per block); 16 experts per block when that
        // leaves at least two blocks per CU, else 8
        const bool eb16 = (T + 15) / 16 * (E / 16) >= 512;
        const dim3 grid((T + 15) / 16, E / (eb16 ? 16 : 8));
#define RT(HBV, EBV) hipLaunchKernelGGL((k_router_t<HBV, EBV, 4>), grid, dim3(256), 0, s, x, addend, W, sgvec, gain, eps, T, E, logits, sgl, xn, xs, xstat)
        if (HB == 8) {
            if (eb16) RT(8, 16);
            else RT(8, 8);
        } else {
            if (eb16) RT(4, 16);
            else RT(4, 8);
        }
#undef RT
        return true;
    }
    // Decode: one router row per one-wave block (every row on its own CU). From
    // 64 tokens at H = 4096 (no transposed kernel): 2 router rows per wave,
    // which gives 4x the waves of 8 (C3 router 11.8 to 6.9 us).
    const uint32_t epw = decode ? 1u : (HB == 16 ? 2u : 8u), wpb = decode ? 1u : 4u;
    const uint32_t gy = (rows + wpb * epw - 1) / (wpb * epw);
#define ROUTER(TOK, HBV)                                                                                       \
    do {                                                                                                       \
        dim3 grid((T + TOK - 1) / TOK, gy);                                                                    \
        hipLaunchKernelGGL((k_router<TOK, HBV>), grid, dim3(64 * wpb), 0, s, x, addend, W, sgvec, gain, eps, T,  \
                           E, epw, logits, sgl, xn, xs, xstat);                                                 \
        return true;                                                                                           \
    } while (0)
    if (HB == 8) {
        if (decode) ROUTER(1, 8);
        ROUTER(4, 8);
    }
    if (HB == 16) {
        if (decode) ROUTER(1, 16);
        ROUTER(2, 16);
    }
    if (HB == 4) {
        if (decode) ROUTER(1, 4);
        ROUTER(4, 4);
    }
#undef ROUTER
    return false;
}

// Top-K routing, keys per lane NE = E/64 rounded up to a power of two; one
// one-wave block per token (four tokens per block measured 0.1 us slower at 4
// and 64 tokens: the selection's ballot, count and compare chain runs on the
// scalar unit, one per CU).
void launch_route(hipStream_t s, const float* logits, const float* bias, uint32_t T, uint32_t E, uint32_t K,
                  uint32_t mode, float scale, uint32_t* ids, float* w, uint32_t* flags) {
    dim3 grid(T);
    const uint32_t ne = (E + 63) / 64;
#define ROUTE(NEV) hipLaunchKernelGGL((k_route<NEV>), grid, dim3(64), 0, s, logits, bias, T, E, K, mode, scale, ids, w, flags)
    if (ne <= 1) ROUTE(1);
    else if (ne <= 2) ROUTE(2);
    else if (ne <= 4) ROUTE(4);
    else if (ne <= 8) ROUTE(8);
    else ROUTE(16);
#undef ROUTE
}

bool launch_gemv_gate_up(hipStream_t s, uint32_t kind, const uint8_t* g, const uint8_t* u, uint64_t gs, uint64_t us,
                         uint32_t F, uint32_t H, uint32_t pairs, const float* x, const uint32_t* ids, uint32_t K,
                         float limit, float* act) {
    const uint32_t cpl = (H / 32 + 63) / 64;
    // One row per wave when GEMV_RPW rows per wave would leave fewer blocks than CUs.
    const uint32_t rpw = (F + 4 * GEMV_RPW - 1) / (4 * GEMV_RPW) * pairs < 256 ? 1u : (uint32_t)GEMV_RPW;
    dim3 grid((F + 4 * rpw - 1) / (4 * rpw), pairs);
    const GateUpArgs a{g, u, gs, us, F, H, x, ids, K, limit, act};
    switch (kind) {
#define K_(KV) case KV: return launch_gemv_gate_up_k<KV>(s, cpl, rpw, grid, a);
        INGOT_KINDS(K_)
#undef K_
        default: return false;
    }
}

bool launch_shared_down_add(hipStream_t s, uint32_t ks, const uint8_t* sd, uint64_t sds, uint32_t H, uint32_t SF,
                            uint32_t T, const float* sact, const float* sgl, float* out, uint32_t* flags) {
    const uint32_t cpl = (SF / 32 + 63) / 64;
    dim3 grid((H + 3) / 4, T);
    switch (ks) {
#define K_(KV) case KV: return launch_shared_add_k<KV>(s, cpl, grid, sd, sds, H, SF, sact, sgl, out, flags);
        INGOT_KINDS(K_)
#undef K_
        default: return false;
    }
}

template <bool GATEUP>
bool launch_gemm(hipStream_t s, uint32_t kind, dim3 grid, const uint8_t* w0, const uint8_t* w1, uint64_t s0,
                 uint64_t s1, uint32_t rows, uint32_t kdim, const float* a, const uint32_t* pairs, uint32_t K,
                 const uint32_t* tiles, uint32_t ldo, float limit, float* out, const uint32_t* slot_of = nullptr) {
    const GemmArgs g{w0, w1, s0, s1, rows, kdim, a, pairs, K, tiles, ldo, limit, out, slot_of};
    switch (kind) {
#define K_(KV) case KV: return launch_gemm_k<KV, GATEUP>(s, grid, g);
        INGOT_KINDS(K_)
#undef K_
        default: return false;
    }
}

// Formats the f16 grouped GEMM decodes, for a matrix of kdim columns: Q4_K, Q5_K,
// Q6_K; IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S when their rows are a whole number of dwords
// (kdim % 512 == 0; their loads assume 4-byte aligned rows); IQ4_NL and IQ4_XS (A read
// permuted: x as split by the dispatch, act as stored by the gate/up kernel).
bool f16_gemm_kind(uint32_t kind, uint32_t kdim, bool gateup) {
    switch (kind) {
        case 12: case 13: return kdim % 256 == 0;
        case 14: return kdim % 256 == 0;
        case 17: case 18: case 21: case 22: return kdim % 512 == 0;
        case 20: return kdim % 64 == 0;
        case 23: return kdim % 256 == 0;
        default: return false;
    }
}

// Column order of A that an f16 GEMM over weights of `kind` reads.
int a_order(uint32_t kind) {
    return (kind == 20 || kind == 23) ? A_IQ4NL
           : (kind == 17 || kind == 18 || kind == 21 || kind == 22) ? A_IQ3XXS
           : kind == 14                                             ? A_Q6K
                                                                    : A_NATURAL;
}

// Formats with a 128-token-tile instantiation of the f16 GEMM (tt128):
// Q4_K, Q5_K and Q6_K, whose B operands need no LDS tables. Q6_K has only
// that one (it also runs the 64-token tiles of a batch without tt128).
bool f16_tt128_kind(uint32_t kind) { return kind == 12 || kind == 13 || kind == 14; }

// gate/up: `kind` its weights, `aord` the order it writes act in (the down
// projection's a_order); tt128: tiles of up to 128 tokens (f16_tt128_kind).
// tl: the weights are the tiled copies (tiled_kind). The kernels are
// instantiated per format in the kinds_*.hip units (launch_gemm_f16_k).
template <bool GATEUP, typename... Args>
bool launch_gemm_f16(hipStream_t s, uint32_t kind, int aord, bool tt128, bool tl, dim3 grid, Args... args) {
    const GemmF16Args a{args...};
    switch (kind) {
#define K_(KV) case KV: return launch_gemm_f16_k<KV, GATEUP>(s, aord, tt128, tl, grid, a);
        INGOT_F16_KINDS(K_)
#undef K_
        default: return false;
    }
}

}  // namespace

// Rows per wave: 3 when that spreads the blocks more evenly over the 256 CUs
// (F = 768 at one token: 256 blocks of 3 rows instead of 384 of 2, half of
// the CUs running two) and for batches of several tokens (a block's routing
// and load round trip then cover half as many rows again: C0's layer gate/up
// at 2 / 4 / 8 tokens 12.0 / 21.0 / 37.8 us against 12.6-12.8 / 21.8-22.0 /
// 38.8-39.9 with 2 rows; 4 and 6 rows measured no better), else 2.
static uint32_t dec_gate_up_rows(uint32_t F, uint32_t T, uint32_t cpl, uint32_t np) {
    if (cpl != 1 || np != 1) return 2;
    if (T >= 2) return 3;
    auto per_cu = [&](uint32_t r) { return ((F + r - 1) / r * T + 255) / 256 * r; };
    return per_cu(3) < per_cu(2) ? 3 : 2;
}

static bool launch_dec_gate_up(hipStream_t s, uint32_t kind, const uint8_t* g, const uint8_t* u, uint64_t gs,
                               uint64_t us, uint32_t F, uint32_t H, uint32_t T, const float* x, const float* xstat,
                               const float* logits, const float* bias, uint32_t E, uint32_t K, uint32_t mode,
                               float scale, float limit, uint32_t* ids, float* w, uint32_t* flags, float* act,
                               uint32_t pre, const uint8_t* pfd, uint64_t pfds) {
    const uint32_t cpl = (H / 32 + 63) / 64, np = (K + GU_WAVES - 1) / GU_WAVES;
    const uint32_t rpw = dec_gate_up_rows(F, T, cpl, np);
    dim3 grid((F + rpw - 1) / rpw, T);
    DecGateUpArgs a{g, u, gs, us, F, H, x, xstat, logits, bias, E, K, mode, scale, limit, ids, w, flags, act, pre};
    a.pfd = pfd;
    a.pfds = pfds;
    switch (kind) {
#define K_(KV) case KV: return launch_dec_gate_up_k<KV>(s, cpl, np, rpw, grid, a);
        INGOT_KINDS(K_)
#undef K_
        default: return false;
    }
}

// The same with the shared expert (gate/up format skind, ffn width F) in the
// routed kernel's free pair slot, for the pairs of INGOT_FUSED_GATE_UP; false
// (nothing launched) when no instantiation covers the shape.
static bool launch_dec_gate_up_fused(hipStream_t s, uint32_t kind, uint32_t skind, const uint8_t* g,
                                     const uint8_t* u, uint64_t gs, uint64_t us, const uint8_t* sg, const uint8_t* su,
                                     uint64_t sgs, uint64_t sus, uint32_t F, uint32_t H, uint32_t T, const float* x,
                                     const float* xstat, const float* logits, const float* bias, uint32_t E,
                                     uint32_t K, uint32_t mode, float scale, float limit, uint32_t* ids, float* w,
                                     uint32_t* flags, float* act, float* sact, uint32_t pre, const uint8_t* pfd,
                                     uint64_t pfds, const uint8_t* pfs, uint64_t pfss) {
    const uint32_t cpl = (H / 32 + 63) / 64, np = (K + GU_WAVES - 1) / GU_WAVES;
    if (K >= GU_WAVES * np) return false;  // no free pair slot
    const uint32_t rpw = dec_gate_up_rows(F, T, cpl, np);
    const dim3 grid((F + rpw - 1) / rpw, T);
    DecGateUpArgs a{g, u, gs, us, F, H, x, xstat, logits, bias, E, K, mode, scale, limit, ids, w, flags, act, pre};
    a.pfd = pfd;
    a.pfds = pfds;
    a.pfs = pfs;
    a.pfss = pfss;
#define FG_(KG, KS)                                                                                              \
    if (kind == KG && skind == KS) return launch_dec_gate_up_fused_k<KG, KS>(s, cpl, np, rpw, grid, a, sg, su, sgs, \
                                                                             sus, sact);
    INGOT_FUSED_GATE_UP(FG_)
#undef FG_
    return false;
}

// Decode down + combine: routed-only for every kind, plus a fused shared expert
// for the format pairs the configurations use (can_fuse_shared). Returns false
// if no instantiation covers the shape.
static bool can_fuse_shared(uint32_t kd, int ks) {
#define F_(KD, KS) if (kd == KD && ks == KS) return true;
    INGOT_FUSED_DOWN(F_)
#undef F_
    return false;
}

static bool gemv_down(hipStream_t s, uint32_t kd, int ks, const DownArgs& a, uint32_t T) {
    const uint32_t nv = a.K * (a.F / 32) + (ks >= 0 ? a.SF / 32 : 0);
    const uint32_t vpl = (nv + 63) / 64;
    dim3 grid((a.H + DOWN_WAVES * DEC_RPW - 1) / (DOWN_WAVES * DEC_RPW), T);
    if (ks < 0) {
        switch (kd) {
#define K_(KV) case KV: return launch_dec_down_k<KV, -1>(s, vpl, grid, a);
            INGOT_KINDS(K_)
#undef K_
            default: return false;
        }
    }
#define F_(KD, KS) if (kd == KD && ks == KS) return launch_dec_down_k<KD, KS>(s, vpl, grid, a);
    INGOT_FUSED_DOWN(F_)
#undef F_
    return false;
}

// ------------------------------------------------------------------ layer
enum Stage { ST_ROUTER = 0, ST_ROUTE = 1, ST_GATEUP = 2, ST_DOWN = 3, ST_COMBINE = 4, ST_DISPATCH = 5, ST_N = 6 };

// Per-forward workspace: the device buffers the kernels use beyond the
// inputs, outputs and weights, carved from one block of memory sized for a
// number of tokens (the layer's own allocation, or the static scratch array
// of the allocation-free forward).
struct Ws {
    float *xn = nullptr, *logits = nullptr, *sgl = nullptr, *wts = nullptr, *act = nullptr, *sact = nullptr,
          *Y = nullptr;
    uint32_t *ids = nullptr, *counts = nullptr, *first = nullptr, *tiles = nullptr, *pairs = nullptr,
             *inverse = nullptr, *stiles = nullptr;
    _Float16 *xh = nullptr, *xl = nullptr, *acth = nullptr, *actl = nullptr;
    float *xs = nullptr, *acts = nullptr;  // 32-column sums of x and act (Q4_K mins term)
    float* resid = nullptr;                 // x + a of ingot_layer_forward_add (the new residual stream)
    float* xstat = nullptr;                 // per token {max |x|, ||x 2^e||}: scales of the f16 splits
    uint32_t* rowmax = nullptr;             // per-row max |act| of the f16 GEMM (range check)
    uint32_t* slot_of = nullptr;            // cached layers: expert -> slot of the current pass (E + 1 entries)
    uint32_t tile_cap = 0, stile_cap = 0;
};

// The reference's expert cache policy (ExpertCache, src/weights.rs:46-95): slot
// i holds expert id[i] (-1: empty) last used at age[i]; a hit refreshes the age;
// a miss takes the least recently used slot that is not pinned (an empty slot
// counts as age 0; ties to the lower slot), empties it for the read, and the
// read's success fills it (commit) with the age of the claim. A failed read
// leaves the slot empty.
struct ExpertCache {
    std::vector<int64_t> id;
    std::vector<uint64_t> age, claim_age;
    uint64_t clock = 0, hits = 0, misses = 0, bytes = 0;
    explicit ExpertCache(uint32_t n) : id(n, -1), age(n, 0), claim_age(n, 0) {}
    uint32_t slots() const { return (uint32_t)id.size(); }
    int hit(uint32_t e) {
        for (uint32_t i = 0; i < slots(); ++i)
            if (id[i] == (int64_t)e) {
                age[i] = ++clock;
                ++hits;
                return (int)i;
            }
        return -1;
    }
    // The slot for expert e: a hit (*load = 0), or a slot emptied for the read
    // (*load = 1); -1 when every slot is pinned ("no reusable expert slot").
    int claim(uint32_t e, const uint32_t* pinned, uint32_t np, int* load) {
        *load = 0;
        const int h = hit(e);
        if (h >= 0) return h;
        ++clock;
        int best = -1;
        uint64_t best_age = 0;
        for (uint32_t i = 0; i < slots(); ++i) {
            bool pin = false;
            for (uint32_t j = 0; j < np; ++j) pin = pin || pinned[j] == i;
            if (pin) continue;
            const uint64_t a = id[i] < 0 ? 0 : age[i];
            if (best < 0 || a < best_age) {
                best = (int)i;
                best_age = a;
            }
        }
        if (best < 0) return -1;
        id[best] = -1;
        claim_age[best] = clock;
        *load = 1;
        return best;
    }
    void commit(uint32_t slot, uint32_t e) {
        id[slot] = e;
        age[slot] = claim_age[slot];
        ++misses;
    }
};

struct ingot_layer {
    ingot_ctx* ctx = nullptr;
    uint32_t H = 0, E = 0, K = 0, F = 0, SF = 0, routing = 0;
    float scale = 1.f, limit = 0.f, eps = 0.f;
    bool has_shared = false, has_sgvec = false, has_norm = false, has_bias = false;
    uint32_t gemm_mode = INGOT_GEMM_AUTO;
    float *router = nullptr, *bias = nullptr, *sgvec = nullptr, *gain = nullptr;
    DevMatrix gate, up, down, sgate, sup, sdown;
    bool tiled = false;  // the tiled copies (DevMatrix::t) are made
    // the layer's own workspace, for up to cap_T tokens
    uint32_t cap_T = 0;
    void* ws = nullptr;
    Ws w;
    std::function<void(hipStream_t)> stage[ST_N];
    const char* stage_name[ST_N] = {};
    // Cached layer (ingot_layer_create_cached): gate/up/down hold `cache` slots;
    // the experts stay in host memory at hgate/hup/hdown (the caller's bytes,
    // expert e at e * rows * stride). pass: the expert -> slot table and whether
    // the shared expert runs, read by the GEMM stages of the current pass.
    bool cached = false;
    std::unique_ptr<ExpertCache> cache;
    const uint8_t *hgate = nullptr, *hup = nullptr, *hdown = nullptr;
    struct Pass {
        const uint32_t* slot_of = nullptr;
        bool first = true;
    } pass;
    // the dispatch buffers of the last prefill forward (ingot_layer_dispatch_debug);
    // last_static: that forward used the shared static array
    uint32_t last_T = 0, last_P = 0, last_S = 0, last_cap = 0, last_tm = 0;
    bool last_prefill = false, last_static = false;
    Ws last;
    // flag word ctx->d_flags[slot]; seq: creation number on the context;
    // flag_status: what its kernels raised before the last flag check
    uint32_t slot = 0, seq = 0;
    int flag_status = INGOT_OK;
};

// The layer's device flag word.
static uint32_t* layer_flags(const ingot_layer* L) { return L->ctx->d_flags + L->slot; }

// Gives L a flag word (the lowest free slot) and its creation number.
static int attach(ingot_ctx* ctx, ingot_layer* L) {
    uint32_t i = 1;
    while (i < ctx->slot.size() && ctx->slot[i]) ++i;
    if (i >= FLAG_WORDS) return fail(ctx, INGOT_UNSUPPORTED, "more than 1023 live layers on one context");
    if (i == ctx->slot.size()) ctx->slot.push_back(nullptr);
    ctx->slot[i] = L;
    L->slot = i;
    L->seq = ctx->next_seq++;
    ++ctx->live;
    return INGOT_OK;
}

// Releases L's flag word, cleared so that the next layer in the slot starts clean.
static void detach(ingot_layer* L) {
    ingot_ctx* ctx = L->ctx;
    if (!L->slot || L->slot >= ctx->slot.size() || ctx->slot[L->slot] != L) return;
    const uint32_t zero = 0;
    (void)hipMemcpy(layer_flags(L), &zero, 4, hipMemcpyHostToDevice);
    ctx->slot[L->slot] = nullptr;
    L->slot = 0;
    --ctx->live;
}

static void free_dev(ingot_layer* L) {
    for (DevMatrix* m : {&L->gate, &L->up, &L->down, &L->sgate, &L->sup, &L->sdown}) {
        if (m->d) (void)hipFree(m->d);
        if (m->t) (void)hipFree(m->t);
    }
    for (float* p : {L->router, L->bias, L->sgvec, L->gain})
        if (p) (void)hipFree(p);
    if (L->ws) (void)hipFree(L->ws);
}

// Lays out the workspace of up to T tokens at base (nullptr: sizes only) and
// returns its size in bytes.
static uint64_t carve(const ingot_layer* L, uint32_t T, void* base, Ws* out) {
    const uint64_t P = (uint64_t)T * L->K;
    // With a shared expert, rows P..P+T-1 of the packed buffers (pairs, act,
    // Y) belong to it, and the tile list has room for its tiles.
    const uint64_t PS = P + (L->SF ? T : 0);
    Ws w;
    w.stile_cap = (T + TM - 1) / TM;
    w.tile_cap = (uint32_t)((P + TM - 1) / TM + L->E + (L->SF ? w.stile_cap : 0));
    struct Part {
        void** p;
        uint64_t bytes;
    };
    const Part parts[] = {
        {(void**)&w.xn, 4ull * T * L->H},       {(void**)&w.logits, 4ull * T * L->E},
        {(void**)&w.sgl, 4ull * T},             {(void**)&w.ids, 4ull * P},
        {(void**)&w.wts, 4ull * P},             {(void**)&w.act, 4ull * P * L->F},
        {(void**)&w.sact, 4ull * T * (L->SF ? L->SF : 1)},
        {(void**)&w.Y, 4ull * PS * L->H},
        {(void**)&w.counts, 4ull * L->E},       {(void**)&w.first, 4ull * L->E},
        {(void**)&w.tiles, 16ull * w.tile_cap}, {(void**)&w.pairs, 4ull * PS},
        {(void**)&w.inverse, 4ull * P},         {(void**)&w.stiles, 16ull * w.stile_cap},
        {(void**)&w.xh, 2ull * T * L->H},       {(void**)&w.xl, 2ull * T * L->H},
        {(void**)&w.acth, 2ull * PS * L->F},    {(void**)&w.actl, 2ull * PS * L->F},
        {(void**)&w.xs, 4ull * T * (L->H / 32)}, {(void**)&w.acts, 4ull * PS * (L->F / 32)},
        {(void**)&w.resid, L->has_norm ? 4ull * T * L->H : 0ull},
        {(void**)&w.xstat, 8ull * T},            {(void**)&w.rowmax, 4ull * PS},
        {(void**)&w.slot_of, L->cached ? 4ull * (L->E + 1) : 0ull},
    };
    uint64_t off = 0;
    for (const Part& p : parts) {
        *p.p = base ? static_cast<char*>(base) + off : nullptr;
        off += (p.bytes + 255) & ~255ull;
    }
    if (out) *out = w;
    return off;
}

// Pairs up to this count take the GEMV (decode) kernels; more take the
// dispatch + grouped MFMA GEMM (prefill) kernels. Whole-layer us over 32
// weight copies, decode kernels against the prefill path: C0's layer at 6 / 8
// tokens (48 / 64 pairs) 47.7 / 59.6 against 62.2 / 65.8; configs[2]'s (512
// experts, top-10) at 2 / 4 / 6 tokens 30.3 / 47.6 / 65.0 against 112.5 /
// 124.9 / 128.7.
static const uint32_t GEMV_MAX_PAIRS = 64;

// Whether a forward of T tokens takes the decode kernels (else routing,
// dispatch and the grouped GEMMs). A cached layer reads the routing back to
// the host before its expert products, so it always takes the GEMM path.
static bool takes_decode(const ingot_layer* L, uint32_t T) {
    const uint32_t K = L->K, F = L->F, SF = L->SF, P = T * K;
    const bool hs = L->has_shared;
    const int ks = hs ? (int)L->sdown.kind : -1;
    const bool fuse_shared = hs && can_fuse_shared(L->down.kind, ks);
    const uint32_t nv = K * (F / 32) + (fuse_shared ? SF / 32 : 0);
    return !L->cached && P <= GEMV_MAX_PAIRS && K <= 2 * GU_WAVES && (uint64_t)K * F + (hs ? SF : 0) <= DOWN_LDS_FLOATS &&
           (nv + 63) / 64 <= 8 && (!hs || fuse_shared || (SF / 32 + 63) / 64 <= 2) && L->H <= 4096;
}

// The f16 GEMM addresses its A operands (x split: T rows of H; act split: P + T
// rows of F) and their group sums with 32-bit byte offsets.
static bool f16_gemm_fits(uint64_t kdim, uint64_t rows) { return 2ull * kdim * rows < (1ull << 32); }

// Which prefill GEMMs a batch of T tokens runs. f16gu: gate/up on the f16 GEMM
// (both projections' formats allow it, or only gate/up's, which then writes
// fp32 act for the fp32 down GEMM); f16: down too; merge: the shared expert
// joins the same launches (its formats and width equal the routed experts').
struct PrefillPlan {
    bool f16gu = false, f16 = false, merge = false;
};

static PrefillPlan prefill_plan(const ingot_layer* L, uint32_t T) {
    PrefillPlan p;
    const uint64_t P = (uint64_t)T * L->K, PS = P + (L->has_shared ? T : 0u);
    p.f16gu = L->gemm_mode == INGOT_GEMM_AUTO && f16_gemm_kind(L->gate.kind, L->H, true) && f16_gemm_fits(L->H, T) &&
              f16_gemm_fits(L->F, PS);
    p.f16 = p.f16gu && f16_gemm_kind(L->down.kind, L->F, false);
    p.merge = p.f16 && L->has_shared && L->SF == L->F && L->sgate.kind == L->gate.kind &&
              L->sup.kind == L->up.kind && L->sdown.kind == L->down.kind && L->sgate.stride == L->gate.stride &&
              L->sup.stride == L->up.stride && L->sdown.stride == L->down.stride;
    return p;
}

static int reserve(ingot_layer* L, uint32_t T) {
    ingot_ctx* ctx = L->ctx;
    // The workspace first: it is required, the tiled copies below are not.
    if (T > L->cap_T) {
        const uint64_t total = carve(L, T, nullptr, nullptr);
        void* ws = nullptr;
        if (L->ws) (void)hipFree(L->ws);
        L->ws = nullptr;
        L->cap_T = 0;
        L->w = Ws();
        // the last forward's dispatch buffers and stage closures pointed into the freed block
        if (!L->last_static) {
            L->last_prefill = false;
            for (auto& f : L->stage) f = nullptr;
        }
        HIP_TRY(ctx, hipMalloc(&ws, total));
        L->ws = ws;
        carve(L, T, ws, &L->w);
        L->cap_T = T;
    }
    // The f16 GEMM's tiled weight copies, made by the first reserve (or
    // forward) of a batch that runs that GEMM, only for the matrices it reads
    // at this batch size: a layer that only decodes, or runs the fp32 GEMM,
    // never holds them. Until they exist (and under graph capture, which
    // cannot allocate) the GEMM reads GGUF order; a copy without room is
    // skipped (make_tiled), and the GEMM then reads that matrix in GGUF order.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (!L->cached && !L->tiled && cs == hipStreamCaptureStatusNone && !takes_decode(L, T)) {
        const PrefillPlan p = prefill_plan(L, T);
        if (p.f16gu) {
            std::vector<DevMatrix*> ms{&L->gate, &L->up};
            if (p.f16) ms.push_back(&L->down);
            if (p.merge) ms.insert(ms.end(), {&L->sgate, &L->sup, &L->sdown});
            for (DevMatrix* m : ms) {
                const int st = make_tiled(ctx, m);
                if (st != INGOT_OK) return st;
            }
            L->tiled = true;
        }
    }
    return INGOT_OK;
}

// ------------------------------------------------------------------ C ABI
extern "C" {

int ingot_geometry(uint32_t kind, uint32_t* block_values, uint32_t* block_bytes) {
    return geometry(kind, block_values, block_bytes);
}
int ingot_validate_matrix(const ingot_matrix* m) { return validate(m); }
int ingot_kind_supported(uint32_t kind) { return supported(kind) ? 1 : 0; }

const char* ingot_status_string(int status) {
    switch (status) {
        case INGOT_OK: return "ok";
        case INGOT_INVALID: return "invalid argument, shape or format";
        case INGOT_NONFINITE: return "non-finite values";
        case INGOT_DEVICE: return "device failure";
        case INGOT_UNSUPPORTED: return "unsupported format or shape";
        case INGOT_RANGE: return "operands outside the split-f16 range: use INGOT_GEMM_FP32";
        default: return "unknown status";
    }
}

int ingot_ctx_create(int device, ingot_ctx** out) {
    if (!out) return INGOT_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return INGOT_DEVICE;
    if (device < 0 || device >= n) return INGOT_INVALID;
    ingot_ctx* ctx = new ingot_ctx();
    ctx->device = device;
    auto bad = [&](hipError_t e) {
        if (e == hipSuccess) return false;
        if (ctx->d_flags) (void)hipFree(ctx->d_flags);
        if (ctx->own) (void)hipStreamDestroy(ctx->own);
        delete ctx;
        return true;
    };
    if (bad(hipSetDevice(device))) return INGOT_DEVICE;
    hipDeviceProp_t prop;
    if (bad(hipGetDeviceProperties(&prop, device))) return INGOT_DEVICE;
    ctx->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    if (bad(hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking))) return INGOT_DEVICE;
    ctx->stream = ctx->own;
    if (bad(hipMalloc(&ctx->d_flags, 4ull * FLAG_WORDS))) return INGOT_DEVICE;
    if (bad(hipMemset(ctx->d_flags, 0, 4ull * FLAG_WORDS))) return INGOT_DEVICE;
    void* sp = nullptr;
    if (bad(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch))) || !sp) return INGOT_DEVICE;
    ctx->scratch = sp;
    *out = ctx;
    return INGOT_OK;
}

int ingot_ctx_destroy(ingot_ctx* ctx) {
    if (!ctx) return INGOT_INVALID;
    // A layer keeps a pointer to its context (stream, flags): destroying the
    // context under it would leave the layer's later calls on freed memory.
    if (ctx->live)
        return fail(ctx, INGOT_INVALID,
                    std::to_string(ctx->live) + " layer(s) still alive on this context: destroy them first");
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->copy) {
        (void)hipStreamSynchronize(ctx->copy);
        (void)hipStreamDestroy(ctx->copy);
    }
    if (ctx->d_flags) (void)hipFree(ctx->d_flags);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    delete ctx;
    return INGOT_OK;
}

const char* ingot_last_error(const ingot_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

int ingot_ctx_set_stream(ingot_ctx* ctx, void* hip_stream) {
    CHECK_CTX(ctx);
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own;
    return INGOT_OK;
}
void* ingot_ctx_stream(const ingot_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int ingot_ctx_synchronize(ingot_ctx* ctx) {
    CHECK_CTX(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return INGOT_OK;
}

const char* ingot_device_name(ingot_ctx* ctx) { return ctx ? ctx->name.c_str() : ""; }

// The status a set of flag bits reports, most severe first.
static int flag_status(uint32_t f) {
    if (f & FLAG_NONFINITE) return INGOT_NONFINITE;
    if (f & FLAG_RANGE) return INGOT_RANGE;
    if (f & FLAG_OUT_NONFINITE) return INGOT_NONFINITE;
    return INGOT_OK;
}

int ingot_ctx_check_device_flags(ingot_ctx* ctx) {
    CHECK_CTX(ctx);
    const uint32_t n = (uint32_t)ctx->slot.size();
    std::vector<uint32_t> f(n, 0u);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(f.data(), ctx->d_flags, 4ull * n, hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemset(ctx->d_flags, 0, 4ull * n));
    // Each layer keeps what its own kernels raised. The status returned is
    // that of the earliest-created flagged layer (in a stack built in order,
    // the root cause: a later layer may only have inherited its bad input),
    // else that of the context's own calls.
    uint32_t nflagged = 0, fl = f[0];
    const ingot_layer* first = nullptr;
    for (uint32_t i = 1; i < n; ++i) {
        ingot_layer* L = ctx->slot[i];
        if (!L) continue;
        L->flag_status = flag_status(f[i]);
        if (f[i]) {
            ++nflagged;
            if (!first || L->seq < first->seq) {
                first = L;
                fl = f[i];
            }
        }
    }
    const int st = flag_status(fl);
    if (st == INGOT_OK) return INGOT_OK;
    std::string msg = (fl & FLAG_NONFINITE) ? "non-finite router logits"
                      : (fl & FLAG_RANGE)
                          ? "prefill activations outside the range of the split-f16 GEMM: re-run with INGOT_GEMM_FP32"
                          : "layer output contains non-finite values";
    if (first)
        msg = "layer " + std::to_string(first->seq) + " (creation order; " + std::to_string(nflagged) +
              " layer(s) flagged): " + msg;
    return fail(ctx, st, msg);
}

int ingot_device_mem_info(ingot_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes) {
    CHECK_CTX(ctx);
    if (!free_bytes || !total_bytes) return INGOT_INVALID;
    size_t fr = 0, to = 0;
    HIP_TRY(ctx, hipMemGetInfo(&fr, &to));
    *free_bytes = fr;
    *total_bytes = to;
    return INGOT_OK;
}

int ingot_malloc(ingot_ctx* ctx, uint64_t bytes, void** d_ptr) {
    CHECK_CTX(ctx);
    if (!d_ptr) return INGOT_INVALID;
    HIP_TRY(ctx, hipMalloc(d_ptr, bytes ? bytes : 1));
    return INGOT_OK;
}
int ingot_free(ingot_ctx* ctx, void* d_ptr) {
    CHECK_CTX(ctx);
    if (d_ptr) HIP_TRY(ctx, hipFree(d_ptr));
    return INGOT_OK;
}
int ingot_memcpy_h2d(ingot_ctx* ctx, void* d_dst, const void* h_src, uint64_t bytes) {
    CHECK_CTX(ctx);
    HIP_TRY(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return INGOT_OK;
}
int ingot_memcpy_d2h(ingot_ctx* ctx, void* h_dst, const void* d_src, uint64_t bytes) {
    CHECK_CTX(ctx);
    HIP_TRY(ctx, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return INGOT_OK;
}

int ingot_device_copy(ingot_ctx* ctx, void* d_dst, const void* d_src, uint64_t bytes) {
    CHECK_CTX(ctx);
    if ((bytes & 15u) || !d_dst || !d_src) return fail(ctx, INGOT_INVALID, "device_copy: bytes must be a multiple of 16");
    const uint64_t n16 = bytes / 16u;
    if (n16 == 0) return INGOT_OK;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n16 + 255u) / 256u, 65536u);
    hipLaunchKernelGGL(k_copy16, dim3(blocks), dim3(256), 0, ctx->stream, static_cast<uint4*>(d_dst),
                       static_cast<const uint4*>(d_src), n16);
    LAUNCH_CHECK(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return INGOT_OK;
}

int ingot_device_read(ingot_ctx* ctx, const void* d_src, uint64_t bytes, uint32_t* d_sink) {
    CHECK_CTX(ctx);
    if ((bytes & 15u) || !d_sink || (bytes && !d_src))
        return fail(ctx, INGOT_INVALID, "device_read: bytes must be a multiple of 16, sink non-null");
    const uint64_t n16 = bytes / 16u;
    const uint64_t blocks = std::max<uint64_t>(1u, (n16 + READ_BLOCK_WORDS - 1) / READ_BLOCK_WORDS);
    if (blocks > 0x7fffffffu) return fail(ctx, INGOT_INVALID, "device_read: too many bytes for one launch");
    hipLaunchKernelGGL(k_read16, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, static_cast<const uint4*>(d_src),
                       n16, d_sink);
    LAUNCH_CHECK(ctx);
    return INGOT_OK;
}

// ---- route() drop-in (src/lib.rs:43-60) ----
int ingot_route(ingot_ctx* ctx, const float* logits, uint32_t E, uint32_t K, uint32_t* ids, float* weights) {
    if (!logits || !ids || !weights || K == 0 || K > E) return fail(ctx, INGOT_INVALID, "invalid router scores or expert count");
    if (!all_finite(logits, E)) return fail(ctx, INGOT_INVALID, "invalid router scores or expert count");
    CHECK_CTX(ctx);
    if (E > 1024 || K > 64) return fail(ctx, INGOT_UNSUPPORTED, "more than 1024 experts or 64 selected");
    float* d = nullptr;
    HIP_TRY(ctx, hipMalloc(&d, 4ull * E + 8ull * K));
    uint32_t* dids = reinterpret_cast<uint32_t*>(d + E);
    float* dw = d + E + K;
    int st = INGOT_OK;
    if (hipMemcpy(d, logits, 4ull * E, hipMemcpyHostToDevice) != hipSuccess) st = INGOT_DEVICE;
    if (st == INGOT_OK) {
        launch_route(ctx->stream, d, nullptr, 1u, E, K, 0u, 1.0f, dids, dw, ctx->d_flags);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess ||
            hipMemcpy(ids, dids, 4ull * K, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(weights, dw, 4ull * K, hipMemcpyDeviceToHost) != hipSuccess)
            st = INGOT_DEVICE;
    }
    (void)hipFree(d);
    if (st != INGOT_OK) return fail(ctx, st, "route: device failure");
    return INGOT_OK;
}

int ingot_route_batch(ingot_ctx* ctx, const float* d_logits, const float* d_bias, uint32_t T, uint32_t E, uint32_t K,
                      uint32_t routing, float scale, uint32_t* d_ids, float* d_weights) {
    CHECK_CTX(ctx);
    if (!d_logits || !d_ids || !d_weights || T == 0 || K == 0 || K > E || routing > 1)
        return fail(ctx, INGOT_INVALID, "invalid router scores or expert count");
    if (E > 1024 || K > 64) return fail(ctx, INGOT_UNSUPPORTED, "more than 1024 experts or 64 selected");
    launch_route(ctx->stream, d_logits, d_bias, T, E, K, routing, routing ? scale : 1.0f, d_ids, d_weights,
                 ctx->d_flags);
    LAUNCH_CHECK(ctx);
    return INGOT_OK;
}

// ---- Gpu::project / Gpu::dequant drop-ins ----
int ingot_project(ingot_ctx* ctx, const ingot_matrix* m, const float* x, float* y) {
    if (validate(m) != INGOT_OK) return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
    if (!x || !y || m->count != 1 || !all_finite(x, m->cols)) return fail(ctx, INGOT_INVALID, "projection shape mismatch");
    CHECK_CTX(ctx);
    if (!supported(m->kind)) return fail(ctx, INGOT_UNSUPPORTED, "GGML type has no kernel here");
    DevScope sc;
    DevMatrix dm;
    float* d = nullptr;
    int st = upload_scoped(ctx, sc, m, &dm);
    if (st != INGOT_OK) return st;
    HIP_TRY(ctx, sc.alloc(&d, 4ull * (m->cols + m->rows)));
    HIP_TRY(ctx, hipMemcpy(d, x, 4ull * m->cols, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(k_project_generic, dim3((uint32_t)((m->rows + 3) / 4), 1), dim3(256), 0, ctx->stream, dm.d,
                       m->stride, m->kind, (uint32_t)m->cols, (uint32_t)m->rows, d, 0ull, d + m->cols);
    LAUNCH_CHECK(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(y, d + m->cols, 4ull * m->rows, hipMemcpyDeviceToHost));
    if (!all_finite(y, m->rows)) return fail(ctx, INGOT_NONFINITE, "output contains non-finite values");
    return INGOT_OK;
}

int ingot_dequant(ingot_ctx* ctx, const ingot_matrix* m, float* out) {
    if (validate(m) != INGOT_OK || !out) return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
    CHECK_CTX(ctx);
    if (!supported(m->kind)) return fail(ctx, INGOT_UNSUPPORTED, "GGML type has no kernel here");
    DevScope sc;
    DevMatrix dm;
    int st = upload_scoped(ctx, sc, m, &dm);
    if (st != INGOT_OK) return st;
    const uint64_t nrows = m->rows * m->count, n = nrows * m->cols;
    float* d = nullptr;
    HIP_TRY(ctx, sc.alloc(&d, 4ull * n));
    hipLaunchKernelGGL(k_dequant_generic, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, ctx->stream, dm.d,
                       m->stride, m->kind, (uint32_t)m->cols, nrows, d);
    LAUNCH_CHECK(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(out, d, 4ull * n, hipMemcpyDeviceToHost));
    if (!all_finite(out, n)) return fail(ctx, INGOT_NONFINITE, "output contains non-finite values");
    return INGOT_OK;
}

// ---- Gpu::moe drop-in (src/metal.rs:1634-1713): gate, up, SwiGLU, per-expert
// down for the K selected experts, the same for the shared expert, the shared
// gate projection and the combine, as one ordered sequence on the stream. ----
int ingot_moe(ingot_ctx* ctx, const ingot_matrix routed[3], const ingot_matrix* shared,
              const ingot_matrix* shared_gate, const float* x, const float* weights, uint32_t K, float* out) {
    if (!routed || !x || !weights || !out) return fail(ctx, INGOT_INVALID, "MoE input shape mismatch");
    const bool has_shared = shared != nullptr;
    if (has_shared != (shared_gate != nullptr)) return fail(ctx, INGOT_INVALID, "MoE input shape mismatch");
    for (int i = 0; i < 3; ++i)
        if (validate(&routed[i]) != INGOT_OK || (has_shared && validate(&shared[i]) != INGOT_OK))
            return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
    if (has_shared && validate(shared_gate) != INGOT_OK) return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
    const uint64_t H = routed[0].cols;
    if (!all_finite(x, H) || !all_finite(weights, K) || routed[0].count != K ||
        (has_shared && (shared[0].cols != H || shared[0].count != 1 || shared_gate->cols != H ||
                        shared_gate->rows != 1 || shared_gate->count != 1)))
        return fail(ctx, INGOT_INVALID, "MoE input shape mismatch");
    auto ffn_ok = [](const ingot_matrix* m) {
        return m[0].cols == m[1].cols && m[0].rows == m[1].rows && m[0].count == m[1].count &&
               m[2].cols == m[0].rows && m[2].rows == m[0].cols && m[2].count == m[0].count;
    };
    if (!ffn_ok(routed) || (has_shared && !ffn_ok(shared))) return fail(ctx, INGOT_INVALID, "FFN matrix shapes do not match");
    CHECK_CTX(ctx);
    for (int i = 0; i < 3; ++i)
        if (!supported(routed[i].kind) || (has_shared && !supported(shared[i].kind)) ||
            (has_shared && !supported(shared_gate->kind)))
            return fail(ctx, INGOT_UNSUPPORTED, "GGML type has no kernel here");
    const uint32_t F = (uint32_t)routed[0].rows, SF = has_shared ? (uint32_t)shared[0].rows : 0;
    DevScope sc;
    DevMatrix dr[3], ds[3], dg;
    int st = INGOT_OK;
    for (int i = 0; i < 3 && st == INGOT_OK; ++i) st = upload_scoped(ctx, sc, &routed[i], &dr[i]);
    for (int i = 0; i < 3 && st == INGOT_OK && has_shared; ++i) st = upload_scoped(ctx, sc, &shared[i], &ds[i]);
    if (st == INGOT_OK && has_shared) st = upload_scoped(ctx, sc, shared_gate, &dg);
    if (st != INGOT_OK) return st;
    // scratch: x[H] w[K] g,u,a [K F] y [K H] sg,su,sa [SF] sy [H] slogit [1] out [H]
    const uint64_t n = H + K + 3ull * K * F + (uint64_t)K * H + 3ull * SF + H + 1 + H;
    float* d = nullptr;
    HIP_TRY(ctx, sc.alloc(&d, 4 * n));
    float *dx = d, *dw = dx + H, *g = dw + K, *u = g + (uint64_t)K * F, *a = u + (uint64_t)K * F,
          *y = a + (uint64_t)K * F, *sg = y + (uint64_t)K * H, *su = sg + SF, *sa = su + SF, *sy = sa + SF,
          *sl = sy + H, *dout = sl + 1;
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx, hipMemcpy(dx, x, 4 * H, hipMemcpyHostToDevice));
    HIP_TRY(ctx, hipMemcpy(dw, weights, 4ull * K, hipMemcpyHostToDevice));
    auto project = [&](const DevMatrix& m, const float* in, uint64_t instride, float* o) {
        hipLaunchKernelGGL(k_project_generic, dim3((uint32_t)((m.rows + 3) / 4), (uint32_t)m.count), dim3(256), 0, s,
                           m.d, m.stride, m.kind, (uint32_t)m.cols, (uint32_t)m.rows, in, instride, o);
    };
    project(dr[0], dx, 0, g);
    project(dr[1], dx, 0, u);
    hipLaunchKernelGGL(k_swiglu, dim3((uint32_t)((K * F + 255) / 256)), dim3(256), 0, s, g, u, (uint64_t)K * F, a);
    project(dr[2], a, F, y);
    if (has_shared) {
        project(ds[0], dx, 0, sg);
        project(ds[1], dx, 0, su);
        hipLaunchKernelGGL(k_swiglu, dim3((SF + 255) / 256), dim3(256), 0, s, sg, su, (uint64_t)SF, sa);
        project(ds[2], sa, SF, sy);
        project(dg, dx, 0, sl);
    }
    hipLaunchKernelGGL(k_combine_host, dim3((uint32_t)((H + 255) / 256)), dim3(256), 0, s, y,
                       has_shared ? sy : nullptr, dw, sl, (uint32_t)H, K, dout);
    LAUNCH_CHECK(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(s));
    HIP_TRY(ctx, hipMemcpy(out, dout, 4 * H, hipMemcpyDeviceToHost));
    if (!all_finite(out, H)) return fail(ctx, INGOT_NONFINITE, "output contains non-finite values");
    return INGOT_OK;
}

// ---- resident layer ----
// slots == 0: every expert resident; else a cached layer with `slots` device
// expert slots (ingot_layer_create_cached).
static int create_layer(ingot_ctx* ctx, const ingot_layer_desc* d, uint32_t slots, ingot_layer** out) {
    if (!d || !out) return fail(ctx, INGOT_INVALID, "null layer description");
    *out = nullptr;
    const uint32_t H = d->hidden, E = d->experts, K = d->top_k;
    if (H == 0 || E == 0 || K == 0 || K > E || !d->router || d->routing > 1)
        return fail(ctx, INGOT_INVALID, "invalid layer geometry or routing");
    for (const ingot_matrix* m : {&d->gate, &d->up, &d->down})
        if (validate(m) != INGOT_OK) return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
    const uint32_t F = (uint32_t)d->gate.rows;
    if (d->gate.cols != H || d->up.cols != H || d->up.rows != F || d->down.cols != F || d->down.rows != H ||
        d->gate.count != E || d->up.count != E || d->down.count != E)
        return fail(ctx, INGOT_INVALID, "FFN matrix shapes do not match");
    const bool has_shared = d->shared_gate.data != nullptr;
    uint32_t SF = 0;
    if (has_shared) {
        for (const ingot_matrix* m : {&d->shared_gate, &d->shared_up, &d->shared_down})
            if (validate(m) != INGOT_OK) return fail(ctx, INGOT_INVALID, "invalid quantized matrix layout");
        SF = (uint32_t)d->shared_gate.rows;
        if (d->shared_gate.cols != H || d->shared_up.cols != H || d->shared_up.rows != SF ||
            d->shared_down.cols != SF || d->shared_down.rows != H || d->shared_gate.count != 1 ||
            d->shared_up.count != 1 || d->shared_down.count != 1)
            return fail(ctx, INGOT_INVALID, "FFN matrix shapes do not match");
    } else if (d->shared_gate_vec) {
        return fail(ctx, INGOT_INVALID, "shared gate vector without a shared expert");
    }
    if (!all_finite(d->router, (uint64_t)E * H) || (d->router_bias && !all_finite(d->router_bias, E)) ||
        (d->shared_gate_vec && !all_finite(d->shared_gate_vec, H)) || (d->norm_gain && !all_finite(d->norm_gain, H)))
        return fail(ctx, INGOT_INVALID, "non-finite router, bias or gain");
    CHECK_CTX(ctx);
    if (E > 1024 || K > 64) return fail(ctx, INGOT_UNSUPPORTED, "more than 1024 experts or 64 selected");
    if (H % 256 || !(H / 256 == 4 || H / 256 == 8 || H / 256 == 16))
        return fail(ctx, INGOT_UNSUPPORTED, "hidden size must be 1024, 2048 or 4096");
    if (F % 64 || (has_shared && SF % 64)) return fail(ctx, INGOT_UNSUPPORTED, "expert ffn size must be a multiple of 64");
    if (d->gate.kind != d->up.kind || (has_shared && d->shared_gate.kind != d->shared_up.kind))
        return fail(ctx, INGOT_UNSUPPORTED, "gate and up must share a format");
    for (const ingot_matrix* m : {&d->gate, &d->down})
        if (!supported(m->kind)) return fail(ctx, INGOT_UNSUPPORTED, "GGML type has no kernel here");
    if (has_shared)
        for (const ingot_matrix* m : {&d->shared_gate, &d->shared_down})
            if (!supported(m->kind)) return fail(ctx, INGOT_UNSUPPORTED, "GGML type has no kernel here");

    ingot_layer* L = new ingot_layer();
    L->ctx = ctx;
    L->H = H; L->E = E; L->K = K; L->F = F; L->SF = SF; L->routing = d->routing;
    L->scale = d->routing ? d->route_scale : 1.0f;
    L->limit = d->swiglu_limit;
    L->eps = d->norm_eps;
    L->has_shared = has_shared;
    L->has_sgvec = d->shared_gate_vec != nullptr;
    L->has_norm = d->norm_gain != nullptr;
    L->has_bias = d->router_bias != nullptr;
    int st = upload(ctx, d->router, (uint64_t)E * H, &L->router);
    if (st == INGOT_OK && L->has_bias) st = upload(ctx, d->router_bias, E, &L->bias);
    if (st == INGOT_OK && L->has_sgvec) st = upload(ctx, d->shared_gate_vec, H, &L->sgvec);
    if (st == INGOT_OK && L->has_norm) st = upload(ctx, d->norm_gain, H, &L->gain);
    if (slots == 0) {
        if (st == INGOT_OK) st = upload_matrix(ctx, &d->gate, &L->gate);
        if (st == INGOT_OK) st = upload_matrix(ctx, &d->up, &L->up);
        if (st == INGOT_OK) st = upload_matrix(ctx, &d->down, &L->down);
    } else {
        // Device slots for `slots` experts of each matrix; the experts stay in
        // the caller's host bytes.
        L->cached = true;
        L->cache = std::make_unique<ExpertCache>(slots);
        L->hgate = d->gate.data;
        L->hup = d->up.data;
        L->hdown = d->down.data;
        for (auto [m, dm] : {std::pair{&d->gate, &L->gate}, std::pair{&d->up, &L->up}, std::pair{&d->down, &L->down}}) {
            if (st != INGOT_OK) break;
            const uint64_t bytes = (uint64_t)slots * m->rows * m->stride;
            const hipError_t e = hipMalloc(reinterpret_cast<void**>(&dm->d), bytes);
            if (e != hipSuccess) {
                dm->d = nullptr;
                st = fail(ctx, INGOT_DEVICE, std::string("hipMalloc: ") + hipGetErrorString(e));
                break;
            }
            dm->nbytes = bytes;
            dm->cols = m->cols;
            dm->rows = m->rows;
            dm->count = slots;
            dm->stride = m->stride;
            dm->kind = m->kind;
        }
    }
    if (st == INGOT_OK && has_shared) st = upload_matrix(ctx, &d->shared_gate, &L->sgate);
    if (st == INGOT_OK && has_shared) st = upload_matrix(ctx, &d->shared_up, &L->sup);
    if (st == INGOT_OK && has_shared) st = upload_matrix(ctx, &d->shared_down, &L->sdown);
    if (st == INGOT_OK) st = attach(ctx, L);
    if (st != INGOT_OK) {
        free_dev(L);
        delete L;
        return st;
    }
    *out = L;
    return INGOT_OK;
}

int ingot_layer_create(ingot_ctx* ctx, const ingot_layer_desc* d, ingot_layer** out) {
    return create_layer(ctx, d, 0, out);
}

int ingot_layer_create_cached(ingot_ctx* ctx, const ingot_layer_desc* d, uint32_t slots, ingot_layer** out) {
    if (slots == 0) return fail(ctx, INGOT_INVALID, "a cached layer needs at least one expert slot");
    if (d && slots > d->experts) return fail(ctx, INGOT_INVALID, "more expert slots than experts");
    return create_layer(ctx, d, slots, out);
}

int ingot_layer_cache_stats(const ingot_layer* L, uint64_t* hits, uint64_t* misses, uint64_t* bytes) {
    if (!L || !hits || !misses || !bytes) return INGOT_INVALID;
    if (!L->cached) return fail(L->ctx, INGOT_INVALID, "the layer's experts are resident, not cached");
    *hits = L->cache->hits;
    *misses = L->cache->misses;
    *bytes = L->cache->bytes;
    return INGOT_OK;
}

// Host-only mirror of the cache policy (no device), for tests of it.
struct ingot_expert_cache {
    ExpertCache c;
    explicit ingot_expert_cache(uint32_t n) : c(n) {}
};

ingot_expert_cache* ingot_expert_cache_create(uint32_t slots) { return slots ? new ingot_expert_cache(slots) : nullptr; }
void ingot_expert_cache_destroy(ingot_expert_cache* c) { delete c; }
int ingot_expert_cache_hit(ingot_expert_cache* c, uint32_t id) { return c ? c->c.hit(id) : -1; }
int ingot_expert_cache_claim(ingot_expert_cache* c, uint32_t id, const uint32_t* pinned, uint32_t npinned, int* load) {
    if (!c || !load || (npinned && !pinned)) return -1;
    return c->c.claim(id, pinned, npinned, load);
}
int ingot_expert_cache_commit(ingot_expert_cache* c, uint32_t slot, uint32_t id) {
    if (!c || slot >= c->c.slots()) return INGOT_INVALID;
    c->c.commit(slot, id);
    return INGOT_OK;
}
int ingot_expert_cache_state(const ingot_expert_cache* c, int64_t* ids, uint64_t* hits, uint64_t* misses) {
    if (!c || !ids || !hits || !misses) return INGOT_INVALID;
    for (uint32_t i = 0; i < c->c.slots(); ++i) ids[i] = c->c.id[i];
    *hits = c->c.hits;
    *misses = c->c.misses;
    return INGOT_OK;
}

int ingot_layer_clone(const ingot_layer* src, ingot_layer** out) {
    if (!src || !out) return INGOT_INVALID;
    ingot_ctx* ctx = src->ctx;
    CHECK_CTX(ctx);
    if (src->cached) return fail(ctx, INGOT_INVALID, "a cached layer cannot be cloned");
    ingot_layer* L = new ingot_layer();
    L->ctx = ctx;
    L->H = src->H; L->E = src->E; L->K = src->K; L->F = src->F; L->SF = src->SF; L->routing = src->routing;
    L->scale = src->scale; L->limit = src->limit; L->eps = src->eps;
    L->has_shared = src->has_shared; L->has_sgvec = src->has_sgvec; L->has_norm = src->has_norm;
    L->has_bias = src->has_bias;
    L->gemm_mode = src->gemm_mode;
    L->tiled = src->tiled;
    auto dup = [&](const void* s, uint64_t bytes, void** dst) -> int {
        if (!s) return INGOT_OK;
        HIP_TRY(ctx, hipMalloc(dst, bytes));
        HIP_TRY(ctx, hipMemcpy(*dst, s, bytes, hipMemcpyDeviceToDevice));
        return INGOT_OK;
    };
    int st = dup(src->router, 4ull * src->E * src->H, (void**)&L->router);
    if (st == INGOT_OK) st = dup(src->bias, 4ull * src->E, (void**)&L->bias);
    if (st == INGOT_OK) st = dup(src->sgvec, 4ull * src->H, (void**)&L->sgvec);
    if (st == INGOT_OK) st = dup(src->gain, 4ull * src->H, (void**)&L->gain);
    const DevMatrix* sm[6] = {&src->gate, &src->up, &src->down, &src->sgate, &src->sup, &src->sdown};
    DevMatrix* dm[6] = {&L->gate, &L->up, &L->down, &L->sgate, &L->sup, &L->sdown};
    for (int i = 0; i < 6 && st == INGOT_OK; ++i) {
        *dm[i] = *sm[i];
        dm[i]->d = dm[i]->t = nullptr;
        st = dup(sm[i]->d, sm[i]->nbytes, (void**)&dm[i]->d);
        if (st == INGOT_OK) st = dup(sm[i]->t, sm[i]->nbytes, (void**)&dm[i]->t);
    }
    if (st == INGOT_OK) st = attach(ctx, L);
    if (st != INGOT_OK) {
        free_dev(L);
        delete L;
        return st;
    }
    *out = L;
    return INGOT_OK;
}

void ingot_layer_destroy(ingot_layer* L) {
    if (!L) return;
    (void)hipSetDevice(L->ctx->device);
    (void)hipStreamSynchronize(L->ctx->stream);
    detach(L);
    free_dev(L);
    delete L;
}

int ingot_layer_flag_status(const ingot_layer* L) { return L ? L->flag_status : INGOT_INVALID; }

int ingot_layer_set_gemm_mode(ingot_layer* L, uint32_t mode) {
    if (!L || mode > INGOT_GEMM_FP32) return INGOT_INVALID;
    L->gemm_mode = mode;
    return INGOT_OK;
}

uint64_t ingot_layer_weight_bytes(const ingot_layer* L) {
    if (!L) return 0;
    uint64_t b = 4ull * L->E * L->H;
    for (const DevMatrix* m : {&L->gate, &L->up, &L->down, &L->sgate, &L->sup, &L->sdown})
        b += m->nbytes * (m->t ? 2u : 1u);
    return b;
}

int ingot_layer_reserve(ingot_layer* L, uint32_t T) {
    if (!L || T == 0) return INGOT_INVALID;
    CHECK_CTX(L->ctx);
    return reserve(L, T);
}

// The stages of a cached layer's forward (src/qwen.rs:1171-1253): routing and
// dispatch, then the routing is read back to the host; the routed experts, in
// order of first use, go through the cache in passes of at most `slots`
// experts (the slots of a pass are pinned while it claims the next ones; a miss
// copies the expert's gate, up and down bytes into its slot); each pass runs
// the grouped GEMMs on the tiles of its experts (slot_of maps expert -> slot,
// NO_SLOT skips a tile; the shared expert runs in the first pass); the combine
// follows the last pass. Every copy and launch is ordered on the context's
// stream, so a slot is refilled only after the pass that read it; the call
// returns after the stream drains (the host tables and the routing it read).
static int cached_expert_passes(ingot_layer* L, const Ws& w, uint32_t T) {
    ingot_ctx* ctx = L->ctx;
    hipStream_t s = ctx->stream;
    const uint32_t E = L->E, P = T * L->K;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(ctx, hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(ctx, INGOT_INVALID, "a cached layer reads its routing on the host and cannot be graph-captured");
    for (int i : {ST_ROUTER, ST_ROUTE, ST_DISPATCH}) L->stage[i](s);
    std::vector<uint32_t> ids(P);
    HIP_TRY(ctx, hipMemcpyAsync(ids.data(), w.ids, 4ull * P, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    std::vector<uint32_t> order;
    std::vector<char> seen(E, 0);
    for (uint32_t e : ids) {
        if (e >= E) return fail(ctx, INGOT_NONFINITE, "routing failed: non-finite router logits");
        if (!seen[e]) {
            seen[e] = 1;
            order.push_back(e);
        }
    }
    const DevMatrix* dev[3] = {&L->gate, &L->up, &L->down};
    const uint8_t* host[3] = {L->hgate, L->hup, L->hdown};
    std::vector<std::vector<uint32_t>> tables;  // kept until the stream drains
    ExpertCache& c = *L->cache;
    // Copies run on their own stream, so that a pass's misses load while the
    // previous pass computes: a copy into a slot that an earlier pass of this
    // forward read first waits for that pass's done event, and each pass's
    // products wait for its copies. The cache decisions (claims, commits,
    // counters) are made on the host in the same order as without overlap.
    if (!ctx->copy) HIP_TRY(ctx, hipStreamCreateWithFlags(&ctx->copy, hipStreamNonBlocking));
    hipStream_t cst = ctx->copy;
    struct Events {
        std::vector<hipEvent_t> v;
        ~Events() {
            for (hipEvent_t e : v) (void)hipEventDestroy(e);
        }
    } evs;
    auto record = [&](hipStream_t st, hipEvent_t* e) -> hipError_t {
        hipError_t r = hipEventCreateWithFlags(e, hipEventDisableTiming);
        if (r != hipSuccess) return r;
        evs.v.push_back(*e);
        return hipEventRecord(*e, st);
    };
    std::vector<int> slot_pass(c.slots(), -1);  // last pass of this forward that read the slot
    std::vector<hipEvent_t> done;                // per pass: its down kernel has run
    int waited = -1;                             // cst already waits for the passes up to this one
    size_t i = 0;
    for (bool first = true; first || i < order.size(); first = false) {
        const int k = (int)done.size();
        bool copied = false;
        std::vector<uint32_t> pinned;
        tables.emplace_back(E + 1, NO_SLOT);
        std::vector<uint32_t>& slot_of = tables.back();
        while (i < order.size() && pinned.size() < c.slots()) {
            const uint32_t e = order[i];
            int load = 0;
            const int slot = c.claim(e, pinned.data(), (uint32_t)pinned.size(), &load);
            if (slot < 0) return fail(ctx, INGOT_INVALID, "no reusable expert slot");
            if (load) {
                const int prev = slot_pass[slot];
                if (prev > waited) {
                    HIP_TRY(ctx, hipStreamWaitEvent(cst, done[prev], 0));
                    waited = prev;
                }
                for (int m = 0; m < 3; ++m) {
                    const uint64_t bytes = dev[m]->rows * dev[m]->stride;
                    HIP_TRY(ctx, hipMemcpyAsync(dev[m]->d + (uint64_t)slot * bytes, host[m] + (uint64_t)e * bytes, bytes,
                                                hipMemcpyHostToDevice, cst));
                    c.bytes += bytes;
                }
                c.commit((uint32_t)slot, e);
                copied = true;
            }
            slot_pass[slot] = k;
            slot_of[e] = (uint32_t)slot;
            pinned.push_back((uint32_t)slot);
            ++i;
        }
        if (copied) {
            hipEvent_t ev;
            HIP_TRY(ctx, record(cst, &ev));
            HIP_TRY(ctx, hipStreamWaitEvent(s, ev, 0));
        }
        slot_of[E] = first ? 0u : NO_SLOT;
        HIP_TRY(ctx, hipMemcpyAsync(w.slot_of, slot_of.data(), 4ull * (E + 1), hipMemcpyHostToDevice, s));
        L->pass = {w.slot_of, first};
        L->stage[ST_GATEUP](s);
        L->stage[ST_DOWN](s);
        hipEvent_t d;
        HIP_TRY(ctx, record(s, &d));
        done.push_back(d);
    }
    L->pass = {};
    L->stage[ST_COMBINE](s);
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return INGOT_OK;
}

// One forward on the workspace w (sized for at least T tokens).
// d_a != NULL (ingot_layer_forward_add, norm layers only): the router adds
// d_a to d_x, normalises the sum and stores it to w.resid, which is then the
// residual the down / combine kernels add.
static int layer_forward(ingot_layer* L, const Ws& w, const float* d_x, const float* d_a, uint32_t T, float* d_out,
                         uint32_t* d_ids, float* d_weights) {
    ingot_ctx* ctx = L->ctx;
    hipStream_t s = ctx->stream;
    const uint32_t H = L->H, E = L->E, K = L->K, F = L->F, SF = L->SF, P = T * K;
    const float* xin = L->has_norm ? w.xn : d_x;
    const float* res = L->has_norm ? (d_a ? w.resid : d_x) : nullptr;
    const float* sgl = L->has_sgvec ? w.sgl : nullptr;
    for (auto& f : L->stage) f = nullptr;

    const bool hs_ = L->has_shared;
    const int ks_ = hs_ ? (int)L->sdown.kind : -1;
    const bool fuse_shared = hs_ && can_fuse_shared(L->down.kind, ks_);
    const bool decode = takes_decode(L, T);
    uint32_t* flags = layer_flags(L);
    float* xstat = w.xstat;

    // 1. router (+ RMSNorm, + shared gate logit, + per-token input maximum)
    {
        const float *x = d_x, *a = d_a, *W = L->router, *sgv = L->sgvec, *g = L->gain;
        float *lg = w.logits, *sl = w.sgl, *xn = w.xn, *rs = w.resid;
        float eps = L->eps;
        bool has_sg = L->has_sgvec;
        uint32_t HB = H / 256;
        L->stage[ST_ROUTER] = [=](hipStream_t ss) {
            launch_router(ss, HB, T, E, has_sg, x, a, W, sgv, g, eps, lg, sl, xn, rs, xstat);
        };
        L->stage_name[ST_ROUTER] = "k_router";
    }
    // 2. route (prefill; decode batches of several tokens over more than 128
    //    experts, whose gate/up blocks then read the routing instead of each
    //    repeating its token's: the search over 512 experts costs more than
    //    the extra launch, over 128 it does not)
    const bool pre_route = decode && T >= 2 && E > 128;
    if (!decode || pre_route) {
        const float *lg = w.logits, *b = L->bias;
        uint32_t* ids = w.ids;
        float* wt = w.wts;
        uint32_t mode = L->routing;
        float scale = L->scale;
        L->stage[ST_ROUTE] = [=](hipStream_t ss) {
            launch_route(ss, lg, b, T, E, K, mode, scale, ids, wt, flags);
        };
        L->stage_name[ST_ROUTE] = "k_route";
    }
    L->last_prefill = !decode;
    if (decode) {
        // router -> routed gate/up (block routing) [+ shared gate/up] -> down + combine
        const DevMatrix gate = L->gate, up = L->up, down = L->down, sgate = L->sgate, sup = L->sup, sdown = L->sdown;
        uint32_t* ids = w.ids;
        float* wts = w.wts;
        float *act = w.act, *sact = w.sact, limit = L->limit;
        const float *lg = w.logits, *b = L->bias;
        const uint32_t mode = L->routing;
        const float scale = L->scale;
        const bool hs = hs_;
        // Down rows requested ahead by the gate/up kernel above 128 experts:
        // there the selection over 8+ keys per lane leaves HBM idle for about
        // 2 us of the gate/up launch (C2 b=1 step 22.2 -> 20.5 us); at 128
        // experts its weight stream already fills HBM, and the extra bytes
        // delay its end by more than the down kernel gains (C0 16.0 -> 16.2).
        const bool pf = E > 128;
        const uint8_t* pfd = pf ? down.d : nullptr;
        const uint8_t* pfs = pf && hs ? sdown.d : nullptr;
        L->stage[ST_GATEUP] = [=](hipStream_t ss) {
            // a shared expert as wide as the routed ones joins the routed kernel where that is instantiated
            if (hs && SF == F && sgate.kind == sup.kind &&
                launch_dec_gate_up_fused(ss, gate.kind, sgate.kind, gate.d, up.d, gate.stride, up.stride, sgate.d,
                                         sup.d, sgate.stride, sup.stride, F, H, T, xin, xstat, lg, b, E, K, mode,
                                         scale, limit, ids, wts, flags, act, sact, pre_route ? 1u : 0u, pfd,
                                         down.stride, pfs, sdown.stride))
                return;
            launch_dec_gate_up(ss, gate.kind, gate.d, up.d, gate.stride, up.stride, F, H, T, xin, xstat, lg, b, E, K,
                               mode, scale, limit, ids, wts, flags, act, pre_route ? 1u : 0u, pfd, down.stride);
            if (hs)
                launch_gemv_gate_up(ss, sgate.kind, sgate.d, sup.d, sgate.stride, sup.stride, SF, H, T, xin, nullptr, 1,
                                    limit, sact);
        };
        L->stage_name[ST_GATEUP] = "k_dec_gate_up2";
        DownArgs a{down.d, sdown.d, down.stride, sdown.stride, H, F, SF, act, sact, ids, sgl, K, res, d_out, flags};
        if (!hs || fuse_shared) {
            const int ks = hs ? ks_ : -1;
            L->stage[ST_DOWN] = [=](hipStream_t ss) { gemv_down(ss, down.kind, ks, a, T); };
        } else {
            DownArgs ar = a;
            ar.sdown = nullptr;
            L->stage[ST_DOWN] = [=](hipStream_t ss) {
                gemv_down(ss, down.kind, -1, ar, T);
                launch_shared_down_add(ss, sdown.kind, sdown.d, sdown.stride, H, SF, T, sact, sgl, d_out, flags);
            };
        }
        L->stage_name[ST_DOWN] = "k_dec_down";
    } else {
        const DevMatrix gate = L->gate, up = L->up, down = L->down, sgate = L->sgate, sup = L->sup, sdown = L->sdown;
        const uint32_t *ids = w.ids;
        uint32_t *counts = w.counts, *first = w.first, *tiles = w.tiles, *pairs = w.pairs, *inverse = w.inverse,
                 *stiles = w.stiles, *rowmax = w.rowmax;
        const uint32_t cap = (P + TM - 1) / TM + E, scap = (T + TM - 1) / TM;
        // Shared-expert rows of Y follow this call's P routed rows.
        float *act = w.act, *sact = w.sact, *Y = w.Y, *Ys = w.Y + (uint64_t)P * H, limit = L->limit;
        const float* wts = w.wts;
        bool hs = L->has_shared;
        // The f16 GEMM runs when both projections' formats allow it; the shared
        // expert then joins the same launches (as tile expert E over rows
        // P..P+T-1) when it has the routed experts' formats and width, and
        // otherwise runs on the fp32 GEMM beside them. When only gate/up's
        // format allows it (a Q4_K_M layer's Q6_K down), gate/up runs on the
        // f16 GEMM writing fp32 act and the down projection on the fp32 GEMM,
        // over the same 64-token tiles.
        const PrefillPlan plan = prefill_plan(L, T);
        const bool f16gu = plan.f16gu, f16 = plan.f16, merge = plan.merge;
        const int aord = f16 ? a_order(down.kind) : A_F32, xord = a_order(gate.kind);
        const bool mins = f16 && (down.kind == 12 || down.kind == 13);
        // 128-token tiles when an expert can take more than 64 pairs (each takes at
        // most one per token), the launch averages at least 32 pairs per expert
        // and both projections have the TT 128 kernel. Below that average most
        // tiles have one or two 16-row blocks, which run faster as 64-token
        // tiles (each wave decoding four B blocks instead of two). Gate/up +
        // down us, 128- against 64-token tiles, at 128 experts top-8: uniform
        // routing 128 tokens 125.5 / 113.5, 256 137 / 124.5, 512 168 / 160;
        // the Zipf-biased C1 router 128 tokens 79 / 70, 256 90 / 91, 512 127.5
        // / 131. (A Q6_K projection runs its 128-token kernel on either.)
        const bool tt128 = f16 && T > TM && (uint64_t)T * K >= 32ull * E && f16_tt128_kind(gate.kind) &&
                           f16_tt128_kind(down.kind);
        const uint32_t tm = tt128 ? 2u * TM : TM;
        // The f16 GEMMs read the tiled copies where every matrix of the launch has one.
        const bool tlg = f16gu && gate.t && up.t && (!merge || (sgate.t && sup.t));
        const bool tld = f16 && down.t && (!merge || sdown.t);
        const uint8_t *g16 = tlg ? gate.t : gate.d, *u16 = tlg ? up.t : up.d, *d16 = tld ? down.t : down.d;
        const uint8_t *sg16 = tlg ? sgate.t : sgate.d, *su16 = tlg ? sup.t : sup.d, *sd16 = tld ? sdown.t : sdown.d;
        const uint32_t S = merge ? T : 0u, capf = cap + (merge ? scap : 0u), e_sh = merge ? E : 0xffffffffu;
        _Float16 *xh = w.xh, *xl = w.xl, *acth = w.acth, *actl = w.actl;
        float *xs = w.xs, *acts = w.acts;
        // rows whose maxima the f16 gate/up raises (act split in the f16 GEMM's units)
        uint32_t* rmx = f16 ? rowmax : nullptr;
        const uint32_t nrow = f16 ? P + S : 0u;
        L->last_T = T;
        L->last_P = P;
        L->last_S = S;
        L->last_cap = capf;
        L->last_tm = tm;
        // Dispatch stage: expert grouping, and for the f16 GEMM the split of x
        // into f16 hi/lo with its 32-column sums.
        L->stage[ST_DISPATCH] = [=](hipStream_t ss) {
            // With the f16 GEMM, blocks 1.. of the dispatch launch split x into f16 hi + lo.
            const uint64_t n = f16gu ? (uint64_t)T * H : 0ull;
            const uint32_t nsplit = (uint32_t)((n / 4 + 1023) / 1024);
            hipLaunchKernelGGL(k_dispatch, dim3(1 + nsplit), dim3(1024), 0, ss, ids, P, E, tm, capf, counts, first, tiles,
                               pairs, inverse, S, K, xin, n, xh, xl, xs, (uint32_t)xord, (const float*)xstat, H, rmx,
                               nrow);
            if (hs && !merge)
                hipLaunchKernelGGL(k_dense_tiles, dim3((scap + 63) / 64), dim3(64), 0, ss, T, scap, stiles);
        };
        L->stage_name[ST_DISPATCH] = "k_dispatch";
        ingot_layer* const LL = L;
        L->stage[ST_GATEUP] = [=](hipStream_t ss) {
            const uint32_t* so = LL->pass.slot_of;
            if (f16gu) {
                launch_gemm_f16<true>(ss, gate.kind, aord, tt128, tlg, dim3(8 * (F / 64) * ((capf + 7) / 8)), g16, u16,
                                      merge ? sg16 : nullptr, merge ? su16 : nullptr, e_sh, gate.stride, up.stride,
                                      F, H, (const _Float16*)xh, (const _Float16*)xl, (const float*)xs,
                                      (const uint32_t*)pairs, K, (const uint32_t*)tiles, F, limit,
                                      f16 ? (float*)nullptr : act, acth, actl, mins ? acts : nullptr, F / 64, T,
                                      (const float*)xstat, rmx, flags, so);
            } else {
                launch_gemm<true>(ss, gate.kind, dim3(F / 64, cap), gate.d, up.d, gate.stride, up.stride, F, H, xin,
                                  pairs, K, tiles, F, limit, act, so);
            }
            if (hs && !merge && LL->pass.first)
                launch_gemm<true>(ss, sgate.kind, dim3(SF / 64, scap), sgate.d, sup.d, sgate.stride, sup.stride, SF, H,
                                  xin, nullptr, 1, stiles, SF, limit, sact);
        };
        L->stage_name[ST_GATEUP] = f16gu ? "k_gemm_f16<gate_up>" : "k_gemm<gate_up>";
        L->stage[ST_DOWN] = [=](hipStream_t ss) {
            const uint32_t* so = LL->pass.slot_of;
            if (f16)
                launch_gemm_f16<false>(ss, down.kind, A_NATURAL, tt128, tld, dim3(8 * (H / 128) * ((capf + 7) / 8)), d16,
                                       (const uint8_t*)nullptr, merge ? sd16 : nullptr, (const uint8_t*)nullptr, e_sh,
                                       down.stride, 0ull, H, F, (const _Float16*)acth, (const _Float16*)actl,
                                       (const float*)acts, (const uint32_t*)nullptr, K, (const uint32_t*)tiles, H, 0.f,
                                       Y, (_Float16*)nullptr, (_Float16*)nullptr, (float*)nullptr, H / 128,
                                       (uint32_t)(P + S), (const float*)xstat, rmx, flags, so);
            else
                launch_gemm<false>(ss, down.kind, dim3(H / 128, cap), down.d, nullptr, down.stride, 0, H, F, act,
                                   nullptr, K, tiles, H, 0.f, Y, so);
            if (hs && !merge && LL->pass.first)
                launch_gemm<false>(ss, sdown.kind, dim3(H / 128, scap), sdown.d, nullptr, sdown.stride, 0, H, SF, sact,
                                   nullptr, 1, stiles, H, 0.f, Ys);
        };
        L->stage_name[ST_DOWN] = f16 ? "k_gemm_f16<down>" : "k_gemm<down>";
        // The f16 down GEMM's rows of Y are in the act units of their token.
        const float* yscale = f16 ? xstat : nullptr;
        const uint32_t shared_scaled = merge ? 1u : 0u;
        L->stage[ST_COMBINE] = [=](hipStream_t ss) {
            hipLaunchKernelGGL(k_combine, dim3((H / 4 + 255) / 256, T), dim3(256), 0, ss, Y, hs ? Ys : nullptr,
                               inverse, wts, sgl, res, T, H, K, d_out, yscale, shared_scaled, flags);
        };
        L->stage_name[ST_COMBINE] = "k_combine";
    }
    L->last = w;
    if (L->cached) {
        const int st = cached_expert_passes(L, w, T);
        if (st != INGOT_OK) return st;
    } else {
        const int order[] = {ST_ROUTER, ST_ROUTE, ST_DISPATCH, ST_GATEUP, ST_DOWN, ST_COMBINE};
        for (int i : order)
            if (L->stage[i]) L->stage[i](s);
    }
    LAUNCH_CHECK(ctx);
    if (d_ids) HIP_TRY(ctx, hipMemcpyAsync(d_ids, w.ids, 4ull * P, hipMemcpyDeviceToDevice, s));
    if (d_weights) HIP_TRY(ctx, hipMemcpyAsync(d_weights, w.wts, 4ull * P, hipMemcpyDeviceToDevice, s));
    return INGOT_OK;
}

int ingot_layer_forward(ingot_layer* L, const float* d_x, uint32_t T, float* d_out, uint32_t* d_ids, float* d_weights) {
    if (!L) return INGOT_INVALID;
    CHECK_CTX(L->ctx);
    if (!d_x || !d_out || T == 0) return fail(L->ctx, INGOT_INVALID, "MoE input shape mismatch");
    const int st = reserve(L, T);
    if (st != INGOT_OK) return st;
    L->last_static = false;
    return layer_forward(L, L->w, d_x, nullptr, T, d_out, d_ids, d_weights);
}

int ingot_layer_forward_static(ingot_layer* L, const float* d_x, uint32_t T, float* d_out, uint32_t* d_ids,
                               float* d_weights) {
    if (!L) return INGOT_INVALID;
    CHECK_CTX(L->ctx);
    if (L->cached) return fail(L->ctx, INGOT_INVALID, "a cached layer copies experts into its slots: not allocation-free");
    if (!d_x || !d_out || T == 0) return fail(L->ctx, INGOT_INVALID, "MoE input shape mismatch");
    const uint64_t need = carve(L, T, nullptr, nullptr);
    if (need > STATIC_SCRATCH_BYTES)
        return fail(L->ctx, INGOT_INVALID,
                    std::to_string(T) + " tokens need " + std::to_string(need) +
                        " bytes of workspace; the static scratch holds " + std::to_string(STATIC_SCRATCH_BYTES));
    Ws w;
    carve(L, T, L->ctx->scratch, &w);
    L->last_static = true;
    return layer_forward(L, w, d_x, nullptr, T, d_out, d_ids, d_weights);
}

uint64_t ingot_layer_static_bytes(const ingot_layer* L, uint32_t T) {
    return L && T ? carve(L, T, nullptr, nullptr) : 0ull;
}

int ingot_layer_forward_add(ingot_layer* L, const float* d_x, const float* d_a, uint32_t T, float* d_out,
                            uint32_t* d_ids, float* d_weights) {
    if (!L) return INGOT_INVALID;
    CHECK_CTX(L->ctx);
    if (!d_x || !d_a || !d_out || T == 0) return fail(L->ctx, INGOT_INVALID, "MoE input shape mismatch");
    if (!L->has_norm) return fail(L->ctx, INGOT_INVALID, "the residual add needs the layer's RMSNorm gain");
    const int st = reserve(L, T);
    if (st != INGOT_OK) return st;
    L->last_static = false;
    return layer_forward(L, L->w, d_x, d_a, T, d_out, d_ids, d_weights);
}

int ingot_layers_time_stage(ingot_layer* const* layers, uint32_t n, uint32_t stage, uint32_t reps, float* ms) {
    if (!layers || n == 0 || !ms || stage >= ST_N || reps == 0) return INGOT_INVALID;
    ingot_ctx* ctx = layers[0]->ctx;
    CHECK_CTX(ctx);
    for (uint32_t i = 0; i < n; ++i) {
        if (!layers[i] || layers[i]->ctx != ctx) return fail(ctx, INGOT_INVALID, "layers of different contexts");
        // A cached layer's GEMM stages read the expert -> slot table of a pass,
        // which exists only inside its forward.
        if (layers[i]->cached) return fail(ctx, INGOT_INVALID, "a cached layer's stages cannot be replayed");
        if (!layers[i]->stage[stage]) return fail(ctx, INGOT_INVALID, "stage did not run in the last forward");
    }
    hipStream_t s = ctx->stream;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    HIP_TRY(ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (uint32_t i = 0; i < reps; ++i) layers[i % n]->stage[stage](s);
    hipError_t le = hipGetLastError();
    hipError_t ce = hipStreamEndCapture(s, &graph);
    if (le != hipSuccess || ce != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return fail(ctx, INGOT_DEVICE, std::string("stage capture: ") + hipGetErrorString(le != hipSuccess ? le : ce));
    }
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    float t = 0;
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipGraphLaunch(exec, s);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(a, s);
    if (e == hipSuccess) e = hipGraphLaunch(exec, s);
    if (e == hipSuccess) e = hipEventRecord(b, s);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (exec) (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(ctx, INGOT_DEVICE, std::string("stage timing: ") + hipGetErrorString(e));
    *ms = t / reps;
    return INGOT_OK;
}

int ingot_layer_time_stage(ingot_layer* L, uint32_t stage, uint32_t reps, float* ms) {
    return ingot_layers_time_stage(&L, 1, stage, reps, ms);
}

const char* ingot_layer_stage_kernel(const ingot_layer* L, uint32_t stage) {
    if (!L || stage >= ST_N || !L->stage[stage]) return "";
    return L->stage_name[stage];
}

int ingot_layer_dispatch_debug(ingot_layer* L, uint32_t* counts, uint32_t* first, uint32_t* pairs,
                               uint32_t* inverse, uint32_t* tiles, uint32_t tiles_cap, uint32_t* info) {
    if (!L) return INGOT_INVALID;
    ingot_ctx* ctx = L->ctx;
    CHECK_CTX(ctx);
    if (!L->last_prefill || !L->stage[ST_DISPATCH])
        return fail(ctx, INGOT_INVALID, "the last forward did not run the prefill dispatch");
    // A static forward's buffers are in the shared array, which any later static
    // forward on this GPU overwrites.
    if (L->last_static)
        return fail(ctx, INGOT_INVALID, "the last forward used the shared static workspace: its buffers are not kept");
    if (!counts || !first || !pairs || !inverse || !tiles || !info)
        return fail(ctx, INGOT_INVALID, "null output buffer");
    const Ws& w = L->last;
    const uint32_t n = std::min(tiles_cap, L->last_cap);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(counts, w.counts, 4ull * L->E, hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(first, w.first, 4ull * L->E, hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(pairs, w.pairs, 4ull * (L->last_P + L->last_S), hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(inverse, w.inverse, 4ull * L->last_P, hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(tiles, w.tiles, 16ull * n, hipMemcpyDeviceToHost));
    info[0] = L->last_P;
    info[1] = L->last_S;
    info[2] = L->last_cap;
    info[3] = L->last_tm;
    return INGOT_OK;
}

// ---- graphs ----
int ingot_graph_begin(ingot_ctx* ctx) {
    CHECK_CTX(ctx);
    HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return INGOT_OK;
}

int ingot_graph_end(ingot_ctx* ctx, ingot_graph** out) {
    CHECK_CTX(ctx);
    if (!out) return INGOT_INVALID;
    ingot_graph* g = new ingot_graph();
    hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
    if (e != hipSuccess) {
        delete g;
        return fail(ctx, INGOT_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    }
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        delete g;
        return fail(ctx, INGOT_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    *out = g;
    return INGOT_OK;
}

int ingot_graph_launch(ingot_ctx* ctx, ingot_graph* g) {
    CHECK_CTX(ctx);
    if (!g) return INGOT_INVALID;
    HIP_TRY(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return INGOT_OK;
}

void ingot_graph_destroy(ingot_graph* g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int ingot_graph_time(ingot_ctx* ctx, ingot_graph* g, uint32_t launches, float* ms) {
    CHECK_CTX(ctx);
    if (!g || !ms || launches == 0) return INGOT_INVALID;
    hipEvent_t a, b;
    HIP_TRY(ctx, hipEventCreate(&a));
    HIP_TRY(ctx, hipEventCreate(&b));
    HIP_TRY(ctx, hipEventRecord(a, ctx->stream));
    for (uint32_t i = 0; i < launches; ++i) HIP_TRY(ctx, hipGraphLaunch(g->exec, ctx->stream));
    HIP_TRY(ctx, hipEventRecord(b, ctx->stream));
    HIP_TRY(ctx, hipEventSynchronize(b));
    HIP_TRY(ctx, hipEventElapsedTime(ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return INGOT_OK;
}

}  // extern "C"
