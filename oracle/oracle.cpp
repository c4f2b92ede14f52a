// CPU oracle for the MoE-layer hot path. TEST INFRASTRUCTURE ONLY: see oracle.h
// for who may load it. Each function cites the reference file:line it restates.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../ingot_amd/csrc/codebooks.h"
#include "../ingot_amd/csrc/det_math.h"

namespace {

// IEEE binary16 -> binary32, exact (GGUF block scales are fp16).
float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: renormalise
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    return ingot_u2f(bits);
}

inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
inline float hf(const uint8_t* p) { return half_to_float(rd16(p)); }

// ggml get_scale_min_k4 as used at kernels/iq3_mix.metal:13-15: six-bit
// scale and min of 32-value group j from the 12 packed scale bytes.
inline void scale_min_k4(const uint8_t* s, uint32_t j, uint32_t* sc, uint32_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

}  // namespace

extern "C" {

// src/gguf.rs:470-491: (values per block, bytes per block) for each GGML type id.
int oracle_geometry(uint32_t kind, uint32_t* block, uint32_t* bytes) {
    uint32_t b = 0, n = 0;
    switch (kind) {
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
        default: return ORACLE_INVALID;
    }
    if (block) *block = b;
    if (bytes) *bytes = n;
    return ORACLE_OK;
}

// src/metal.rs:1602-1621 (validate_matrix).
int oracle_validate_matrix(const oracle_matrix* m) {
    uint32_t block, bytes;
    if (!m || oracle_geometry(m->kind, &block, &bytes) != ORACLE_OK) return ORACLE_INVALID;
    if (m->cols == 0 || m->rows == 0 || m->count == 0 || m->cols % block != 0) return ORACLE_INVALID;
    if (m->stride != m->cols / block * bytes) return ORACLE_INVALID;
    unsigned __int128 total = (unsigned __int128)m->stride * m->rows * m->count;
    if (total != m->nbytes) return ORACLE_INVALID;
    const uint64_t lim = 0xffffffffull;
    if (m->cols > lim || m->rows > lim || m->count > lim || m->stride > lim) return ORACLE_INVALID;
    return ORACLE_OK;
}

// One weight of a row. Formulas: kernels/moe.metal:13-89 (F32 :13, F16 :14,
// Q4_0 :15, Q8_0 :16, Q2_K :17-21, Q6_K :22-28, IQ2_XXS :29-36, IQ1_M :37-46,
// BF16 :47-50, Q2_0 :51-55, IQ2_S :56-64, IQ3_S :65-75, IQ4_NL :76-80,
// IQ4_XS :81-89) and kernels/iq3_mix.metal:17-36 (Q4_K and Q5_K :19-23,
// IQ2_XS :25-30, IQ3_XXS :31-35). Each value is evaluated in
// float as the ggml dequantize_row_* routines do (scale product first).
float oracle_dequant_value(const uint8_t* row, uint32_t kind, uint64_t j) {
    switch (kind) {
        case 0: {
            float f;
            std::memcpy(&f, row + 4 * j, 4);
            return f;
        }
        case 1: return hf(row + 2 * j);
        case 30: return ingot_u2f((uint32_t)rd16(row + 2 * j) << 16);
        case 2: {
            const uint8_t* b = row + (j / 32) * 18;
            uint32_t k = j % 32;
            int q = (int)((b[2 + k % 16] >> (4 * (k / 16))) & 15) - 8;
            return hf(b) * (float)q;
        }
        case 8: {
            const uint8_t* b = row + (j / 32) * 34;
            return hf(b) * (float)(int8_t)b[2 + j % 32];
        }
        case 20: {
            const uint8_t* b = row + (j / 32) * 18;
            uint32_t k = j % 32;
            uint32_t q = (b[2 + k % 16] >> (4 * (k / 16))) & 15;
            return hf(b) * (float)ingot_kvalues_iq4nl[q];
        }
        case 12: {
            const uint8_t* b = row + (j / 256) * 144;
            uint32_t k = j % 256, g = k / 32, sc, mn;
            scale_min_k4(b + 4, g, &sc, &mn);
            uint32_t q = (b[16 + 32 * (k / 64) + k % 32] >> (4 * (g % 2))) & 15;
            float d1 = hf(b) * (float)sc;
            float m1 = hf(b + 2) * (float)mn;
            return d1 * (float)q - m1;
        }
        case 17: {
            const uint8_t* b = row + (j / 256) * 74;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t q = rd16(b + 2 + 2 * (4 * g + l));
            float grid = (float)((ingot_iq2xs_grid[q & 511] >> (8 * v)) & 255);
            float sign = (ingot_ksign(q >> 9) & (1u << v)) ? -1.0f : 1.0f;
            float db = hf(b) * (0.5f + (float)((b[66 + g] >> (4 * (l / 2))) & 15)) * 0.25f;
            return db * grid * sign;
        }
        case 18: {
            const uint8_t* b = row + (j / 256) * 98;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t aux = rd32(b + 66 + 4 * g);
            float grid = (float)((ingot_iq3xxs_grid[b[2 + 8 * g + 2 * l + v / 4]] >> (8 * (v % 4))) & 255);
            float sign = (ingot_ksign((aux >> (7 * l)) & 127) & (1u << v)) ? -1.0f : 1.0f;
            float db = hf(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
            return db * grid * sign;
        }
        case 13: {  // Q5_K, kernels/iq3_mix.metal:19-23: Q4_K's nibble plus bit g of qh[k % 32] as 16
            const uint8_t* b = row + (j / 256) * 176;
            uint32_t k = j % 256, g = k / 32, sc, mn;
            scale_min_k4(b + 4, g, &sc, &mn);
            uint32_t q = (b[48 + 32 * (k / 64) + k % 32] >> (4 * (g % 2))) & 15;
            q |= ((b[16 + k % 32] >> g) & 1u) << 4;
            float d1 = hf(b) * (float)sc;
            float m1 = hf(b + 2) * (float)mn;
            return d1 * (float)q - m1;
        }
        case 10: {  // Q2_K, kernels/moe.metal:17-21
            const uint8_t* b = row + (j / 256) * 84;
            uint32_t k = j % 256, sc = b[k / 16];
            uint32_t q = (b[16 + (k / 128) * 32 + k % 32] >> (2 * ((k % 128) / 32))) & 3;
            return hf(b + 80) * (float)(sc & 15) * (float)q - hf(b + 82) * (float)(sc >> 4);
        }
        case 14: {  // Q6_K, kernels/moe.metal:22-28
            const uint8_t* b = row + (j / 256) * 210;
            uint32_t k = j % 256, n = k / 128, l = k % 32, t = (k % 128) / 32;
            uint32_t low = (b[n * 64 + l + (t % 2) * 32] >> (t >= 2 ? 4 : 0)) & 15;
            uint32_t high = (b[128 + n * 32 + l] >> (2 * t)) & 3;
            int scale = (int8_t)b[192 + n * 8 + l / 16 + 2 * t];
            return hf(b + 208) * (float)scale * (float)((int)(low | (high << 4)) - 32);
        }
        case 16: {  // IQ2_XXS, kernels/moe.metal:29-36
            const uint8_t* b = row + (j / 256) * 66;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            const uint8_t* a = b + 2 + g * 8;
            uint32_t packed = rd32(a + 4);
            float grid = (float)((ingot_iq2xxs_grid[a[l]] >> (8 * v)) & 255);
            float sign = (ingot_ksign((packed >> (7 * l)) & 127) & (1u << v)) ? -1.0f : 1.0f;
            return hf(b) * (0.5f + (float)(packed >> 28)) * 0.25f * grid * sign;
        }
        case 29: {  // IQ1_M, kernels/moe.metal:37-46
            const uint8_t* b = row + (j / 256) * 56;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t sc[4];
            for (int i = 0; i < 4; ++i) sc[i] = rd16(b + 48 + 2 * i);
            uint32_t bits = (sc[0] >> 12) | ((sc[1] >> 8) & 240) | ((sc[2] >> 4) & 3840) | (sc[3] & 61440);
            uint32_t high = b[32 + g * 2 + l / 2];
            uint32_t index = b[g * 4 + l] | (((high >> (4 * (l % 2))) & 7) << 8);
            float delta = (high & (8u << (4 * (l % 2)))) ? -0.125f : 0.125f;
            float grid = (float)(int8_t)((ingot_iq1s_grid[index] >> (8 * v)) & 255);
            uint32_t scale = (sc[g / 2] >> (6 * (g % 2) + 3 * (l / 2))) & 7;
            return half_to_float((uint16_t)bits) * (float)(2 * scale + 1) * (grid + delta);
        }
        case 42: {  // Q2_0, kernels/moe.metal:51-55: consecutive 2-bit codes, 64 per block
            const uint8_t* b = row + (j / 64) * 18;
            uint32_t k = j % 64;
            return hf(b) * (float)((int)((b[2 + k / 4] >> (2 * (k % 4))) & 3) - 1);
        }
        case 22: {  // IQ2_S, kernels/moe.metal:56-64
            const uint8_t* b = row + (j / 256) * 82;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8;
            uint32_t index = b[2 + 4 * g + l] | (((uint32_t)b[66 + g] << (8 - 2 * l)) & 0x300);
            float grid = (float)((ingot_iq2s_grid[index] >> (8 * v)) & 255);
            uint32_t scale = (b[74 + g] >> (4 * (l / 2))) & 15;
            float sign = (b[34 + 4 * g + l] & (1u << v)) ? -1.0f : 1.0f;
            return hf(b) * (0.5f + (float)scale) * 0.25f * grid * sign;
        }
        case 21: {  // IQ3_S, kernels/moe.metal:65-75
            const uint8_t* b = row + (j / 256) * 110;
            uint32_t k = j % 256, g = k / 32, l = (k % 32) / 8, v = k % 8, hg = v / 4;
            uint32_t index = b[2 + g * 8 + 2 * l + hg] | (((uint32_t)b[66 + g] << (8 - 2 * l - hg)) & 256);
            float grid = (float)((ingot_iq3s_grid[index] >> (8 * (v % 4))) & 255);
            uint32_t scale = (b[106 + g / 2] >> (4 * (g % 2))) & 15;
            float sign = (b[74 + g * 4 + l] & (1u << v)) ? -1.0f : 1.0f;
            return hf(b) * (float)(1 + 2 * scale) * grid * sign;
        }
        case 23: {  // IQ4_XS, kernels/moe.metal:81-89
            const uint8_t* b = row + (j / 256) * 136;
            uint32_t k = j % 256, g = k / 32, v = k % 32;
            uint32_t high = rd16(b + 2);
            int scale = (int)(((b[4 + g / 2] >> (4 * (g % 2))) & 15) | (((high >> (2 * g)) & 3) << 4)) - 32;
            uint32_t q = (b[8 + g * 16 + v % 16] >> (4 * (v / 16))) & 15;
            return hf(b) * (float)scale * (float)ingot_kvalues_iq4nl[q];
        }
        default: return NAN;
    }
}

void oracle_dequant_row(const uint8_t* row, uint32_t kind, uint64_t cols, float* out) {
    for (uint64_t j = 0; j < cols; ++j) out[j] = oracle_dequant_value(row, kind, j);
}

float oracle_det_expf(float x) { return ingot_det_expf(x); }
float oracle_det_sigmoid(float x) { return ingot_det_sigmoid(x); }

// src/lib.rs:43-60: reject K == 0, K > E and non-finite logits; stable sort by
// f32::total_cmp descending (ties keep the lower id first); truncate to K;
// w_k = exp(l_k - l_max) / sum over the selected, summed in selection order.
int oracle_route_softmax(const float* logits, uint32_t E, uint32_t K, uint32_t* ids, float* w) {
    if (K == 0 || K > E) return ORACLE_INVALID;
    for (uint32_t e = 0; e < E; ++e)
        if (!std::isfinite(logits[e])) return ORACLE_INVALID;
    std::vector<uint32_t> order(E);
    for (uint32_t e = 0; e < E; ++e) order[e] = e;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
        return ingot_orderable(logits[a]) > ingot_orderable(logits[b]);
    });
    float top = logits[order[0]];
    float total = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
        ids[k] = order[k];
        w[k] = ingot_det_expf(logits[order[k]] - top);
        total += w[k];
    }
    for (uint32_t k = 0; k < K; ++k) w[k] /= total;
    return ORACLE_OK;
}

// kernels/glm.metal:81-98: select K experts on sigmoid(l_e) + bias_e (ties to the
// lower id); weights sigmoid(l_sel) / sum_sel * scale; the bias never enters the
// weights. Argument checks follow route() (src/lib.rs:44).
int oracle_route_sigmoid(const float* logits, const float* bias, uint32_t E, uint32_t K,
                         float scale, uint32_t* ids, float* w) {
    if (K == 0 || K > E) return ORACLE_INVALID;
    std::vector<float> sel(E);
    for (uint32_t e = 0; e < E; ++e) {
        if (!std::isfinite(logits[e]) || (bias && !std::isfinite(bias[e]))) return ORACLE_INVALID;
        float s = ingot_det_sigmoid(logits[e]);
        sel[e] = bias ? s + bias[e] : s;
    }
    std::vector<uint32_t> order(E);
    for (uint32_t e = 0; e < E; ++e) order[e] = e;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
        return ingot_orderable(sel[a]) > ingot_orderable(sel[b]);
    });
    float total = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
        ids[k] = order[k];
        w[k] = ingot_det_sigmoid(logits[order[k]]);
        total += w[k];
    }
    for (uint32_t k = 0; k < K; ++k) w[k] = w[k] / total * scale;
    return ORACLE_OK;
}

void oracle_router_logits(const float* W, const float* x, uint32_t T, uint32_t E, uint32_t H,
                          const float* bias, int add_bias, float* logits) {
    float v[64];
    for (uint32_t t = 0; t < T; ++t)
        for (uint32_t e = 0; e < E; ++e) {
            for (uint32_t l = 0; l < 64; ++l)
                v[l] = ingot_router_partial(W + (uint64_t)e * H, x + (uint64_t)t * H, H, l);
            float s = ingot_butterfly64(v);
            if (add_bias && bias) s = s + bias[e];
            logits[(uint64_t)t * E + e] = s;
        }
}

int oracle_project(const oracle_matrix* m, const float* x, double* y) {
    if (oracle_validate_matrix(m) != ORACLE_OK || m->count != 1) return ORACLE_INVALID;
    std::vector<float> row(m->cols);
    for (uint64_t r = 0; r < m->rows; ++r) {
        oracle_dequant_row(m->data + r * m->stride, m->kind, m->cols, row.data());
        double s = 0;
        for (uint64_t j = 0; j < m->cols; ++j) s += (double)row[j] * (double)x[j];
        y[r] = s;
    }
    return ORACLE_OK;
}

}  // extern "C"

namespace {

// RMSNorm in the fixed fp32 order used by the GPU (its output feeds the router,
// so it must be bit-identical): sum of squares over the 64 router slots and the
// butterfly tree, mean = ss / H, r = 1 / sqrt(mean + eps), y = (x * r) * g.
// Formula: kernels/generic.metal:392-409 (add_rms).
void rms_norm_det(const float* x, const float* g, uint32_t H, float eps, float* y) {
    float v[64];
    for (uint32_t l = 0; l < 64; ++l) v[l] = ingot_router_partial(x, x, H, l);
    float ss = ingot_butterfly64(v);
    float mean = ss / (float)H;
    float r = 1.0f / std::sqrt(mean + eps);
    for (uint32_t j = 0; j < H; ++j) y[j] = (x[j] * r) * g[j];
}

template <typename Acc>
Acc dot(const float* a, const float* b, uint64_t n);

template <>
double dot<double>(const float* a, const float* b, uint64_t n) {
    double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    uint64_t j = 0;
    for (; j + 4 <= n; j += 4) {
        s0 += (double)a[j] * b[j];
        s1 += (double)a[j + 1] * b[j + 1];
        s2 += (double)a[j + 2] * b[j + 2];
        s3 += (double)a[j + 3] * b[j + 3];
    }
    for (; j < n; ++j) s0 += (double)a[j] * b[j];
    return (s0 + s1) + (s2 + s3);
}

template <>
float dot<float>(const float* a, const float* b, uint64_t n) {
    float s[16] = {0};
    uint64_t j = 0;
    for (; j + 16 <= n; j += 16)
        for (int k = 0; k < 16; ++k) s[k] = __builtin_fmaf(a[j + k], b[j + k], s[k]);
    for (; j < n; ++j) s[0] = __builtin_fmaf(a[j], b[j], s[0]);
    for (int w = 8; w >= 1; w >>= 1)
        for (int k = 0; k < w; ++k) s[k] += s[k + w];
    return s[0];
}

template <typename Acc>
Acc swiglu(Acc g, Acc u, float limit) {
    // kernels/moe.metal:405-410; with a limit, kernels/glm.metal:100-103.
    if (limit > 0) {
        g = std::min(g, (Acc)limit);
        u = std::min(std::max(u, (Acc)-limit), (Acc)limit);
    }
    return g / ((Acc)1 + std::exp(-g)) * u;
}

template <typename Fn>
void parallel_for(uint64_t n, int threads, Fn fn) {
    if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    if ((uint64_t)threads > n) threads = (int)std::max<uint64_t>(1, n);
    std::atomic<uint64_t> next(0);
    auto work = [&]() {
        for (uint64_t i; (i = next.fetch_add(1)) < n;) fn(i);
    };
    if (threads == 1) {
        work();
        return;
    }
    std::vector<std::thread> pool;
    for (int i = 0; i < threads; ++i) pool.emplace_back(work);
    for (auto& t : pool) t.join();
}

// One expert group: the (token) inputs routed to one expert's three matrices.
struct Group {
    const uint8_t *gate, *up, *down;
    uint32_t gkind, ukind, dkind;
    uint64_t gstride, ustride, dstride;
    std::vector<uint32_t> slots;   // activation / output slot of each member
    std::vector<uint32_t> inputs;  // row of the normalised input of each member
};

template <typename Acc>
void run_groups(const std::vector<Group>& groups, const float* xin, uint32_t H, uint32_t F,
                float limit, std::vector<Acc>& act_slots, std::vector<Acc>& y_slots, int threads) {
    const uint32_t RB = 16;
    // gate/up + SwiGLU: work items (group, block of F rows).
    uint64_t fblocks = (F + RB - 1) / RB;
    parallel_for(groups.size() * fblocks, threads, [&](uint64_t item) {
        const Group& G = groups[item / fblocks];
        if (G.slots.empty()) return;
        uint32_t r0 = (uint32_t)(item % fblocks) * RB, r1 = std::min(F, r0 + RB);
        std::vector<float> gr(H), ur(H);
        for (uint32_t r = r0; r < r1; ++r) {
            oracle_dequant_row(G.gate + r * G.gstride, G.gkind, H, gr.data());
            oracle_dequant_row(G.up + r * G.ustride, G.ukind, H, ur.data());
            for (size_t i = 0; i < G.slots.size(); ++i) {
                const float* xv = xin + (uint64_t)G.inputs[i] * H;
                Acc g = dot<Acc>(gr.data(), xv, H), u = dot<Acc>(ur.data(), xv, H);
                act_slots[(uint64_t)G.slots[i] * F + r] = swiglu<Acc>(g, u, limit);
            }
        }
    });
    // down: work items (group, block of H rows). The activation is read as Acc
    // (double in the f64 oracle, float in the f32 layer).
    uint64_t hblocks = (H + RB - 1) / RB;
    parallel_for(groups.size() * hblocks, threads, [&](uint64_t item) {
        const Group& G = groups[item / hblocks];
        if (G.slots.empty()) return;
        uint32_t r0 = (uint32_t)(item % hblocks) * RB, r1 = std::min(H, r0 + RB);
        std::vector<float> dr(F);
        std::vector<double> dd(F);
        for (uint32_t r = r0; r < r1; ++r) {
            oracle_dequant_row(G.down + r * G.dstride, G.dkind, F, dr.data());
            for (size_t i = 0; i < G.slots.size(); ++i) {
                const Acc* a = act_slots.data() + (uint64_t)G.slots[i] * F;
                Acc s;
                if constexpr (sizeof(Acc) == 8) {
                    double t0 = 0, t1 = 0;
                    uint32_t j = 0;
                    for (; j + 2 <= F; j += 2) {
                        t0 += (double)dr[j] * a[j];
                        t1 += (double)dr[j + 1] * a[j + 1];
                    }
                    for (; j < F; ++j) t0 += (double)dr[j] * a[j];
                    s = t0 + t1;
                } else {
                    s = dot<float>(dr.data(), (const float*)a, F);
                }
                y_slots[(uint64_t)G.slots[i] * H + r] = s;
            }
        }
    });
}

template <typename Acc>
int forward(const oracle_layer* L, const float* x, uint32_t T, float* out, uint32_t* ids_out,
            float* w_out, int threads) {
    const uint32_t H = L->hidden, E = L->experts, K = L->top_k;
    const uint32_t F = (uint32_t)L->gate.rows;
    if (H == 0 || H % 256 != 0 || E == 0 || K == 0 || K > E) return ORACLE_INVALID;
    for (const oracle_matrix* m : {&L->gate, &L->up, &L->down})
        if (oracle_validate_matrix(m) != ORACLE_OK || m->count != E) return ORACLE_INVALID;
    if (L->gate.cols != H || L->up.cols != H || L->up.rows != F || L->down.cols != F || L->down.rows != H)
        return ORACLE_INVALID;
    uint32_t SF = 0;
    if (L->has_shared) {
        SF = (uint32_t)L->shared_gate.rows;
        for (const oracle_matrix* m : {&L->shared_gate, &L->shared_up, &L->shared_down})
            if (oracle_validate_matrix(m) != ORACLE_OK || m->count != 1) return ORACLE_INVALID;
        if (L->shared_gate.cols != H || L->shared_up.cols != H || L->shared_up.rows != SF ||
            L->shared_down.cols != SF || L->shared_down.rows != H)
            return ORACLE_INVALID;
    }
    for (uint64_t i = 0; i < (uint64_t)T * H; ++i)
        if (!std::isfinite(x[i])) return ORACLE_NONFINITE;

    // Pre-norm (optional), router logits and routing: fp32, fixed order.
    std::vector<float> xn((uint64_t)T * H);
    if (L->norm_gain) {
        for (uint32_t t = 0; t < T; ++t)
            rms_norm_det(x + (uint64_t)t * H, L->norm_gain, H, L->norm_eps, xn.data() + (uint64_t)t * H);
    } else {
        std::memcpy(xn.data(), x, sizeof(float) * (uint64_t)T * H);
    }
    std::vector<float> logits((uint64_t)T * E);
    const bool softmax = L->routing == ORACLE_ROUTE_SOFTMAX;
    oracle_router_logits(L->router, xn.data(), T, E, H, L->router_bias, softmax ? 1 : 0, logits.data());
    std::vector<uint32_t> ids((uint64_t)T * K);
    std::vector<float> w((uint64_t)T * K);
    for (uint32_t t = 0; t < T; ++t) {
        int st = softmax ? oracle_route_softmax(&logits[(uint64_t)t * E], E, K, &ids[(uint64_t)t * K], &w[(uint64_t)t * K])
                         : oracle_route_sigmoid(&logits[(uint64_t)t * E], L->router_bias, E, K, L->route_scale,
                                                &ids[(uint64_t)t * K], &w[(uint64_t)t * K]);
        if (st != ORACLE_OK) return st;
    }

    // Group pairs by expert (stable), as the prefill dispatch does.
    const uint32_t P = T * K;
    std::vector<Group> groups(E + (L->has_shared ? 1 : 0));
    for (uint32_t e = 0; e < E; ++e) {
        Group& G = groups[e];
        G.gate = L->gate.data + (uint64_t)e * F * L->gate.stride;
        G.up = L->up.data + (uint64_t)e * F * L->up.stride;
        G.down = L->down.data + (uint64_t)e * H * L->down.stride;
        G.gkind = L->gate.kind; G.ukind = L->up.kind; G.dkind = L->down.kind;
        G.gstride = L->gate.stride; G.ustride = L->up.stride; G.dstride = L->down.stride;
    }
    for (uint32_t p = 0; p < P; ++p) {
        groups[ids[p]].slots.push_back(p);
        groups[ids[p]].inputs.push_back(p / K);
    }
    std::vector<Acc> act((uint64_t)P * F), y((uint64_t)P * H);
    run_groups<Acc>(groups, xn.data(), H, F, L->swiglu_limit, act, y, threads);

    std::vector<Acc> sact, sy;
    std::vector<Acc> sgate(T, (Acc)1);
    if (L->has_shared) {
        std::vector<Group> sg(1);
        Group& G = sg[0];
        G.gate = L->shared_gate.data; G.up = L->shared_up.data; G.down = L->shared_down.data;
        G.gkind = L->shared_gate.kind; G.ukind = L->shared_up.kind; G.dkind = L->shared_down.kind;
        G.gstride = L->shared_gate.stride; G.ustride = L->shared_up.stride; G.dstride = L->shared_down.stride;
        for (uint32_t t = 0; t < T; ++t) {
            G.slots.push_back(t);
            G.inputs.push_back(t);
        }
        sact.resize((uint64_t)T * SF);
        sy.resize((uint64_t)T * H);
        run_groups<Acc>(sg, xn.data(), H, SF, L->swiglu_limit, sact, sy, threads);
        if (L->shared_gate_vec) {
            // Qwen shared-expert gate: sigmoid(v . x) (kernels/moe.metal:421,
            // tools/check_rust_moe.py:73-75).
            for (uint32_t t = 0; t < T; ++t) {
                Acc s = dot<Acc>(L->shared_gate_vec, xn.data() + (uint64_t)t * H, H);
                sgate[t] = (Acc)1 / ((Acc)1 + std::exp(-s));
            }
        }
    }

    // Combine in route order k = 0..K-1 (kernels/moe.metal:412-422, glm.metal:105-110).
    for (uint32_t t = 0; t < T; ++t)
        for (uint32_t i = 0; i < H; ++i) {
            Acc s = 0;
            for (uint32_t k = 0; k < K; ++k)
                s += (Acc)w[(uint64_t)t * K + k] * y[(uint64_t)(t * K + k) * H + i];
            if (L->has_shared) s += sy[(uint64_t)t * H + i] * sgate[t];
            if (L->norm_gain) s += (Acc)x[(uint64_t)t * H + i];
            out[(uint64_t)t * H + i] = (float)s;
        }
    if (ids_out) std::memcpy(ids_out, ids.data(), sizeof(uint32_t) * P);
    if (w_out) std::memcpy(w_out, w.data(), sizeof(float) * P);
    // The reference rejects a non-finite output on read-back (src/metal.rs:1575-1577).
    for (uint64_t i = 0; i < (uint64_t)T * H; ++i)
        if (!std::isfinite(out[i])) return ORACLE_NONFINITE;
    return ORACLE_OK;
}

}  // namespace

extern "C" {

int oracle_moe_forward(const oracle_layer* L, const float* x, uint32_t T, float* out,
                       uint32_t* ids, float* w, int precision, int threads) {
    if (!L || !x || !out || T == 0) return ORACLE_INVALID;
    if (precision == ORACLE_F64) return forward<double>(L, x, T, out, ids, w, threads);
    if (precision == ORACLE_F32) return forward<float>(L, x, T, out, ids, w, threads);
    return ORACLE_INVALID;
}

// kernels/prefill.metal:7-38 (expert_layout + expert_pairs): per-expert counts
// and first offsets, pair indices stable within an expert, the inverse map, and
// `tile`-pair tiles {expert, first, n, mode = n >= 2} in expert order, zero-padded
// to `cap` entries.
uint32_t oracle_dispatch(const uint32_t* ids, uint32_t P, uint32_t E, uint32_t tile, uint32_t cap,
                         uint32_t* counts, uint32_t* first, uint32_t* pairs, uint32_t* inverse,
                         uint32_t* tiles) {
    std::vector<uint32_t> n(E, 0);
    for (uint32_t p = 0; p < P; ++p) n[ids[p]]++;
    uint32_t a = 0;
    std::vector<uint32_t> at(E);
    for (uint32_t e = 0; e < E; ++e) {
        counts[e] = n[e];
        first[e] = a;
        at[e] = a;
        a += n[e];
    }
    for (uint32_t p = 0; p < P; ++p) {
        uint32_t pos = at[ids[p]]++;
        pairs[pos] = p;
        inverse[p] = pos;
    }
    uint32_t used = 0;
    for (uint32_t e = 0; e < E; ++e)
        for (uint32_t k = 0; k * tile < n[e]; ++k) {
            uint32_t nt = std::min(tile, n[e] - k * tile);
            if (used < cap) {
                tiles[4 * used] = e;
                tiles[4 * used + 1] = first[e] + k * tile;
                tiles[4 * used + 2] = nt;
                tiles[4 * used + 3] = nt >= 2 ? 1u : 0u;
            }
            ++used;
        }
    for (uint32_t t = used; t < cap; ++t) tiles[4 * t] = tiles[4 * t + 1] = tiles[4 * t + 2] = tiles[4 * t + 3] = 0;
    return used;
}

}  // extern "C"
