// Synthetic inputs and GGUF-block quantizers (host only). See include/ingot_synth.h.
//
// The quantizers are this project's own: any valid block is acceptable for
// parity, because the CPU oracle and the GPU kernels decode the same bytes.
// They aim at reasonable reconstruction error, not at ggml's exact choices.
#include "../../include/ingot_synth.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "codebooks.h"

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct SplitMix64 {
    uint64_t s;
    uint64_t next() {
        s += 0x9e3779b97f4a7c15ull;
        return mix64(s);
    }
    double unit() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }  // [0, 1)
};

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

void normal_row(uint64_t key, uint64_t r, uint64_t cols, float mean, float sigma, float* out) {
    SplitMix64 g{ingot_synth_stream(key, r, 0, 0)};
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t j = 0; j < cols; j += 2) {
        double u1 = 1.0 - g.unit();  // (0, 1]
        double u2 = g.unit();
        double rad = std::sqrt(-2.0 * std::log(u1));
        double z0 = rad * std::cos(two_pi * u2), z1 = rad * std::sin(two_pi * u2);
        out[j] = (float)(mean + sigma * z0);
        if (j + 1 < cols) out[j + 1] = (float)(mean + sigma * z1);
    }
}

uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
    if (ax < 0x38800000u) {                                   // below 2^-14: subnormal half
        if (ax < 0x33000000u) return (uint16_t)sign;           // < 2^-25: zero
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;  // value = m * 2^(e-150); half ulp = 2^-24
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15, m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) ++q;
    return (uint16_t)(sign | q);
}

float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
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
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
inline void put32(uint8_t* p, uint32_t v) {
    for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
inline int nearest_int(float v) { return (int)std::lrintf(v); }

// ---- Q8_0: d = amax / 127, q = round(x / d). 34-byte blocks of 32.
void quant_q8_0(const float* x, uint64_t cols, uint8_t* out) {
    for (uint64_t b = 0; b < cols / 32; ++b) {
        const float* v = x + 32 * b;
        uint8_t* o = out + 34 * b;
        float amax = 0;
        for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint16_t dh = f2h(amax / 127.0f);
        float d = h2f(dh), id = d != 0 ? 1.0f / d : 0.0f;
        put16(o, dh);
        for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(int8_t)std::clamp(nearest_int(v[i] * id), -127, 127);
    }
}

// ---- Q4_0: d = (value of largest magnitude) / -8, q = clamp(round(x/d) + 8, 0, 15).
void quant_q4_0(const float* x, uint64_t cols, uint8_t* out) {
    for (uint64_t b = 0; b < cols / 32; ++b) {
        const float* v = x + 32 * b;
        uint8_t* o = out + 18 * b;
        float mx = 0;
        for (int i = 0; i < 32; ++i)
            if (std::fabs(v[i]) > std::fabs(mx)) mx = v[i];
        uint16_t dh = f2h(mx / -8.0f);
        float d = h2f(dh), id = d != 0 ? 1.0f / d : 0.0f;
        put16(o, dh);
        for (int i = 0; i < 16; ++i) {
            int lo = std::clamp(nearest_int(v[i] * id) + 8, 0, 15);
            int hi = std::clamp(nearest_int(v[i + 16] * id) + 8, 0, 15);
            o[2 + i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// ---- IQ4_NL: d = (value of largest magnitude) / kvalues[0], nearest codebook entry.
void quant_iq4_nl(const float* x, uint64_t cols, uint8_t* out) {
    for (uint64_t b = 0; b < cols / 32; ++b) {
        const float* v = x + 32 * b;
        uint8_t* o = out + 18 * b;
        float mx = 0;
        for (int i = 0; i < 32; ++i)
            if (std::fabs(v[i]) > std::fabs(mx)) mx = v[i];
        uint16_t dh = f2h(mx / (float)ingot_kvalues_iq4nl[0]);
        float d = h2f(dh);
        put16(o, dh);
        uint8_t q[32];
        for (int i = 0; i < 32; ++i) {
            int best = 0;
            float be = INFINITY;
            for (int c = 0; c < 16; ++c) {
                float e = std::fabs(d * (float)ingot_kvalues_iq4nl[c] - v[i]);
                if (e < be) {
                    be = e;
                    best = c;
                }
            }
            q[i] = (uint8_t)best;
        }
        for (int i = 0; i < 16; ++i) o[2 + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
    }
}

// ---- Q4_K: 144-byte superblocks of 256 = 8 groups of 32 with six-bit scale
// and min each: w = d*sc*q - dmin*m.
void quant_q4_k(const float* x, uint64_t cols, uint8_t* out) {
    for (uint64_t b = 0; b < cols / 256; ++b) {
        const float* v = x + 256 * b;
        uint8_t* o = out + 144 * b;
        float scale[8], minv[8], smax = 0, mmax = 0;
        for (int g = 0; g < 8; ++g) {
            float lo = 0, hi = -INFINITY;
            for (int i = 0; i < 32; ++i) {
                lo = std::min(lo, v[32 * g + i]);
                hi = std::max(hi, v[32 * g + i]);
            }
            scale[g] = (hi - lo) / 15.0f;
            minv[g] = -lo;
            smax = std::max(smax, scale[g]);
            mmax = std::max(mmax, minv[g]);
        }
        uint16_t dh = f2h(smax / 63.0f), mh = f2h(mmax / 63.0f);
        float d = h2f(dh), dm = h2f(mh);
        uint8_t sc[8], mn[8];
        for (int g = 0; g < 8; ++g) {
            sc[g] = (uint8_t)std::clamp(d > 0 ? nearest_int(scale[g] / d) : 0, 0, 63);
            mn[g] = (uint8_t)std::clamp(dm > 0 ? nearest_int(minv[g] / dm) : 0, 0, 63);
        }
        put16(o, dh);
        put16(o + 2, mh);
        uint8_t* s = o + 4;
        std::memset(s, 0, 12);
        for (int j = 0; j < 4; ++j) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int g = 0; g < 8; ++g) {
            float dg = d * (float)sc[g], mg = dm * (float)mn[g];
            for (int i = 0; i < 32; ++i)
                q[32 * g + i] = (uint8_t)std::clamp(dg > 0 ? nearest_int((v[32 * g + i] + mg) / dg) : 0, 0, 15);
        }
        uint8_t* qs = o + 16;
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 32; ++i) qs[32 * c + i] = (uint8_t)(q[64 * c + i] | (q[64 * c + 32 + i] << 4));
    }
}

// ---- Codebook lookup tables for the IQ quantizers: every combination of
// per-coordinate magnitude levels maps to the codebook entry nearest to it.
struct IqTables {
    uint16_t iq2[6561];  // 8 coordinates, levels {8, 25, 43}
    uint8_t iq3[4096];   // 4 coordinates, levels {4, 12, ..., 52, 62}
    IqTables() {
        const int l2[3] = {8, 25, 43};
        for (int c = 0; c < 6561; ++c) {
            int lv[8], t = c;
            for (int i = 0; i < 8; ++i) {
                lv[i] = l2[t % 3];
                t /= 3;
            }
            long best = -1, be = 0;
            for (int gi = 0; gi < 512; ++gi) {
                long e = 0;
                for (int i = 0; i < 8; ++i) {
                    long gv = (long)((ingot_iq2xs_grid[gi] >> (8 * i)) & 255) - lv[i];
                    e += gv * gv;
                }
                if (best < 0 || e < be) {
                    be = e;
                    best = gi;
                }
            }
            iq2[c] = (uint16_t)best;
        }
        const int l3[8] = {4, 12, 20, 28, 36, 44, 52, 62};
        for (int c = 0; c < 4096; ++c) {
            int lv[4], t = c;
            for (int i = 0; i < 4; ++i) {
                lv[i] = l3[t % 8];
                t /= 8;
            }
            long best = -1, be = 0;
            for (int gi = 0; gi < 256; ++gi) {
                long e = 0;
                for (int i = 0; i < 4; ++i) {
                    long gv = (long)((ingot_iq3xxs_grid[gi] >> (8 * i)) & 255) - lv[i];
                    e += gv * gv;
                }
                if (best < 0 || e < be) {
                    be = e;
                    best = gi;
                }
            }
            iq3[c] = (uint8_t)best;
        }
    }
};
const IqTables& iq_tables() {
    static IqTables t;
    return t;
}

// Sign pattern of 8 values with an even count of negatives (the format stores
// 7 bits; the 8th is the parity). If the count is odd, the value of smallest
// magnitude takes the opposite sign.
uint32_t sign_bits8(const float* v) {
    uint32_t bits = 0;
    int neg = 0, imin = 0;
    for (int i = 0; i < 8; ++i) {
        if (v[i] < 0) {
            bits |= 1u << i;
            ++neg;
        }
        if (std::fabs(v[i]) < std::fabs(v[imin])) imin = i;
    }
    if (neg & 1) bits ^= 1u << imin;
    return bits;
}

int nearest_level(float a, const int* levels, int n) {
    int best = 0;
    float be = INFINITY;
    for (int i = 0; i < n; ++i) {
        float e = std::fabs(a - (float)levels[i]);
        if (e < be) {
            be = e;
            best = i;
        }
    }
    return best;
}

// ---- IQ2_XS: 74-byte superblocks: fp16 d, 32 u16 codes (9-bit grid index,
// 7-bit sign index per 8 values), 8 scale bytes (4 bits per 16 values).
// w = d * (0.5 + s) * 0.25 * grid * sign.
void quant_iq2_xs(const float* x, uint64_t cols, uint8_t* out) {
    const IqTables& T = iq_tables();
    const int lv[3] = {8, 25, 43};
    for (uint64_t b = 0; b < cols / 256; ++b) {
        const float* v = x + 256 * b;
        uint8_t* o = out + 74 * b;
        float amax = 0;
        for (int i = 0; i < 256; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint16_t dh = f2h(amax / (15.5f * 0.25f * 43.0f));
        float d = h2f(dh);
        put16(o, dh);
        for (int g = 0; g < 8; ++g) {
            uint8_t sbyte = 0;
            for (int h = 0; h < 2; ++h) {
                const float* hv = v + 32 * g + 16 * h;
                float hmax = 0;
                for (int i = 0; i < 16; ++i) hmax = std::max(hmax, std::fabs(hv[i]));
                int s = d > 0 ? std::clamp(nearest_int(hmax / (d * 0.25f * 43.0f) - 0.5f), 0, 15) : 0;
                sbyte |= (uint8_t)(s << (4 * h));
                float unit = d * (0.5f + (float)s) * 0.25f;
                for (int l2 = 0; l2 < 2; ++l2) {
                    int l = 2 * h + l2;
                    const float* sv = v + 32 * g + 8 * l;
                    uint32_t sb = sign_bits8(sv);
                    int combo = 0;
                    for (int i = 7; i >= 0; --i)
                        combo = combo * 3 + nearest_level(unit > 0 ? std::fabs(sv[i]) / unit : 0.0f, lv, 3);
                    uint32_t code = T.iq2[combo] | ((sb & 127u) << 9);
                    put16(o + 2 + 2 * (4 * g + l), (uint16_t)code);
                }
            }
            o[66 + g] = sbyte;
        }
    }
}

// ---- IQ3_XXS: 98-byte superblocks: fp16 d, 64 grid bytes (4 values each),
// 8 u32 words (four 7-bit sign indices + 4-bit scale per 32 values).
// w = d * (0.5 + s) * 0.5 * grid * sign.
void quant_iq3_xxs(const float* x, uint64_t cols, uint8_t* out) {
    const IqTables& T = iq_tables();
    const int lv[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    for (uint64_t b = 0; b < cols / 256; ++b) {
        const float* v = x + 256 * b;
        uint8_t* o = out + 98 * b;
        float amax = 0;
        for (int i = 0; i < 256; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint16_t dh = f2h(amax / (15.5f * 0.5f * 62.0f));
        float d = h2f(dh);
        put16(o, dh);
        for (int g = 0; g < 8; ++g) {
            const float* gv = v + 32 * g;
            float gmax = 0;
            for (int i = 0; i < 32; ++i) gmax = std::max(gmax, std::fabs(gv[i]));
            int s = d > 0 ? std::clamp(nearest_int(gmax / (d * 0.5f * 62.0f) - 0.5f), 0, 15) : 0;
            float unit = d * (0.5f + (float)s) * 0.5f;
            uint32_t aux = (uint32_t)s << 28;
            for (int l = 0; l < 4; ++l) {
                const float* sv = gv + 8 * l;
                aux |= (sign_bits8(sv) & 127u) << (7 * l);
                for (int half = 0; half < 2; ++half) {
                    int combo = 0;
                    for (int i = 3; i >= 0; --i)
                        combo = combo * 8 + nearest_level(unit > 0 ? std::fabs(sv[4 * half + i]) / unit : 0.0f, lv, 8);
                    o[2 + 8 * g + 2 * l + half] = T.iq3[combo];
                }
            }
            put32(o + 66 + 4 * g, aux);
        }
    }
}

bool quant_row(uint32_t kind, const float* x, uint64_t cols, uint8_t* out) {
    switch (kind) {
        case 0: std::memcpy(out, x, 4 * cols); return true;
        case 2: quant_q4_0(x, cols, out); return true;
        case 8: quant_q8_0(x, cols, out); return true;
        case 12: quant_q4_k(x, cols, out); return true;
        case 17: quant_iq2_xs(x, cols, out); return true;
        case 18: quant_iq3_xxs(x, cols, out); return true;
        case 20: quant_iq4_nl(x, cols, out); return true;
        default: return false;
    }
}

// Formats without a quantizer here get random valid blocks: every quant,
// index, sign and sub-scale byte uniformly random, the fp16 block scales set
// so that weights come out about `sigma` in size (times a per-block factor in
// [0.5, 1.5)). F16 and BF16 rows hold N(0, sigma) values. Parity tests only
// need both sides to decode the same bytes; uniform bytes reach every
// codebook entry, sign pattern and scale.
struct RandomLayout {
    uint32_t block, bytes;
    uint32_t d_at, dmin_at;  // byte offsets of the fp16 scales (dmin_at == bytes: none)
    float d_div, dmin_div;   // d = sigma / d_div
};

bool random_layout(uint32_t kind, RandomLayout* L) {
    switch (kind) {
        case 10: *L = {256, 84, 80, 82, 8.f, 16.f}; return true;       // Q2_K
        case 13: *L = {256, 176, 0, 2, 400.f, 800.f}; return true;     // Q5_K
        case 14: *L = {256, 210, 208, 210, 1000.f, 1.f}; return true;  // Q6_K
        case 16: *L = {256, 66, 0, 66, 50.f, 1.f}; return true;        // IQ2_XXS
        case 21: *L = {256, 110, 0, 110, 128.f, 1.f}; return true;     // IQ3_S
        case 22: *L = {256, 82, 0, 82, 50.f, 1.f}; return true;        // IQ2_S
        case 23: *L = {256, 136, 0, 136, 1000.f, 1.f}; return true;    // IQ4_XS
        case 29: *L = {256, 56, 56, 56, 8.f, 1.f}; return true;        // IQ1_M (d in the scale words' top nibbles)
        case 42: *L = {64, 18, 0, 18, 1.f, 1.f}; return true;          // Q2_0
        default: return false;
    }
}

bool random_row(uint32_t kind, uint64_t key, uint64_t r, uint64_t cols, float sigma, uint8_t* out) {
    SplitMix64 g{ingot_synth_stream(key, r, 1, kind)};
    if (kind == 1 || kind == 30) {
        std::vector<float> v(cols);
        normal_row(key, r, cols, 0.0f, sigma, v.data());
        for (uint64_t j = 0; j < cols; ++j) {
            uint16_t h;
            if (kind == 1) {
                h = f2h(v[j]);
            } else {
                float f = v[j];
                ingot_round_bf16(&f, 1);
                uint32_t u;
                std::memcpy(&u, &f, 4);
                h = (uint16_t)(u >> 16);
            }
            put16(out + 2 * j, h);
        }
        return true;
    }
    RandomLayout L;
    if (!random_layout(kind, &L) || cols % L.block) return false;
    const uint64_t nb = cols / L.block;
    for (uint64_t i = 0; i < nb * L.bytes; i += 8) {
        uint64_t v = g.next();
        for (uint64_t b = 0; b < 8 && i + b < nb * L.bytes; ++b) out[i + b] = (uint8_t)(v >> (8 * b));
    }
    for (uint64_t i = 0; i < nb; ++i) {
        uint8_t* b = out + i * L.bytes;
        const float jit = (float)(0.5 + g.unit());
        const uint16_t d = f2h(sigma / L.d_div * jit);
        if (kind == 29) {
            for (int w = 0; w < 4; ++w) {
                uint16_t sc = (uint16_t)(b[48 + 2 * w] | (b[49 + 2 * w] << 8));
                sc = (uint16_t)((sc & 0x0fffu) | (((d >> (4 * w)) & 15u) << 12));
                put16(b + 48 + 2 * w, sc);
            }
            continue;
        }
        put16(b + L.d_at, d);
        if (L.dmin_at < L.bytes) put16(b + L.dmin_at, f2h(sigma / L.dmin_div * jit));
    }
    return true;
}

}  // namespace

extern "C" {

uint64_t ingot_synth_stream(uint64_t a, uint64_t b, uint64_t c, uint64_t d) {
    uint64_t k = 0x243f6a8885a308d3ull;  // digits of pi: an arbitrary non-zero start
    for (uint64_t v : {a, b, c, d}) k = mix64(k ^ mix64(v + 0x9e3779b97f4a7c15ull));
    return k;
}

void ingot_synth_normal(uint64_t key, uint64_t rows, uint64_t cols, float mean, float sigma, float* out,
                        int threads) {
    parallel_for(rows, threads, [&](uint64_t r) { normal_row(key, r, cols, mean, sigma, out + r * cols); });
}

void ingot_synth_uniform(uint64_t key, uint64_t rows, uint64_t cols, float lo, float hi, float* out,
                         int threads) {
    parallel_for(rows, threads, [&](uint64_t r) {
        SplitMix64 g{ingot_synth_stream(key, r, 0, 0)};
        for (uint64_t j = 0; j < cols; ++j) out[r * cols + j] = (float)(lo + (hi - lo) * g.unit());
    });
}

void ingot_round_bf16(float* x, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t u;
        std::memcpy(&u, &x[i], 4);
        if ((u & 0x7fffffffu) <= 0x7f800000u) u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        std::memcpy(&x[i], &u, 4);
    }
}

uint16_t ingot_f32_to_f16(float f) { return f2h(f); }
float ingot_f16_to_f32(uint16_t h) { return h2f(h); }

uint64_t ingot_quant_row_bytes(uint32_t kind, uint64_t cols) {
    switch (kind) {
        case 0: return 4 * cols;
        case 2: return cols % 32 ? 0 : cols / 32 * 18;
        case 8: return cols % 32 ? 0 : cols / 32 * 34;
        case 20: return cols % 32 ? 0 : cols / 32 * 18;
        case 12: return cols % 256 ? 0 : cols / 256 * 144;
        case 17: return cols % 256 ? 0 : cols / 256 * 74;
        case 18: return cols % 256 ? 0 : cols / 256 * 98;
        case 1: case 30: return 2 * cols;
        default: {
            RandomLayout L;
            if (!random_layout(kind, &L) || cols % L.block) return 0;
            return cols / L.block * L.bytes;
        }
    }
}

int ingot_quantize(uint32_t kind, const float* src, uint64_t rows, uint64_t cols, uint8_t* dst, int threads) {
    uint64_t stride = ingot_quant_row_bytes(kind, cols);
    if (!stride) return 1;
    iq_tables();
    parallel_for(rows, threads, [&](uint64_t r) { quant_row(kind, src + r * cols, cols, dst + r * stride); });
    return 0;
}

int ingot_synth_quantized(uint32_t kind, uint64_t key, uint64_t count, uint64_t rows, uint64_t cols, float sigma,
                          uint8_t* dst, int threads) {
    uint64_t stride = ingot_quant_row_bytes(kind, cols);
    if (!stride) return 1;
    iq_tables();
    const uint64_t chunk = 16;
    uint64_t total = count * rows, items = (total + chunk - 1) / chunk;
    parallel_for(items, threads, [&](uint64_t it) {
        std::vector<float> buf(cols);
        for (uint64_t r = it * chunk; r < std::min(total, (it + 1) * chunk); ++r) {
            if (random_row(kind, key, r, cols, sigma, dst + r * stride)) continue;
            normal_row(key, r, cols, 0.0f, sigma, buf.data());
            quant_row(kind, buf.data(), cols, dst + r * stride);
        }
    });
    return 0;
}

}  // extern "C"
