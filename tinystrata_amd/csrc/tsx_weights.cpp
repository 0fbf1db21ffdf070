// tsx_weights.cpp - host-side weight quantizers that write valid GGUF blocks of the expert formats (Q8_0, Q4_K,
// IQ3_XXS, IQ3_S) from fp32 rows.  They make the synthetic expert weights of the tests and the benchmark.
//
// The reference quantizes with ggml's quantize_q8_0 / quantize_q4_K / quantize_iq3_xxs / quantize_iq3_s (an
// un-vendored dependency, called from tests/native-expert-pool.cpp:52-61 through ggml_quantize_chunk).  Q8_0 here is
// ggml's closed form (d = amax / 127, q = round(x / d)); Q4_K and the two IQ3 formats are simpler searches of this
// library's own (per-sub-block range fit; nearest codebook word per 4 values with per-coordinate level rounding),
// so their bytes are valid blocks of the format but not ggml's bytes for the same floats.
#include "tsx_moe.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "tsx_half.hpp"

namespace {

using tsx::f2h;
using tsx::h2f;

// For each 4-tuple of level numbers (3 bits each, 4096 tuples) the codebook word nearest to it in value space:
// the search of a 4-value group rounds each magnitude to its nearest level, then takes this word.
struct Nearest {
    uint16_t xxs[4096];
    uint16_t s[4096];
};
const Nearest& nearest() {
    static Nearest n;
    static std::once_flag once;
    std::call_once(once, [] {
        for (int c = 0; c < 4096; ++c) {
            float vx[4], vs[4];
            for (int k = 0; k < 4; ++k) {
                vx[k] = (float) tsx_iq3xxs_level((c >> (3 * k)) & 7);
                vs[k] = (float) tsx_iq3s_level((c >> (3 * k)) & 7);
            }
            float bx = 1e30f, bs = 1e30f;
            for (int i = 0; i < 512; ++i) {
                const uint32_t ws = tsx_iq3s_word(i);
                float ds = 0.f;
                for (int k = 0; k < 4; ++k) { const float t = (float) ((ws >> (8 * k)) & 255) - vs[k]; ds += t * t; }
                if (ds < bs) { bs = ds; n.s[c] = (uint16_t) i; }
                if (i < 256) {
                    const uint32_t wx = tsx_iq3xxs_word(i);
                    float dx = 0.f;
                    for (int k = 0; k < 4; ++k) { const float t = (float) ((wx >> (8 * k)) & 255) - vx[k]; dx += t * t; }
                    if (dx < bx) { bx = dx; n.xxs[c] = (uint16_t) i; }
                }
            }
        }
    });
    return n;
}

int nearest_level_xxs(float v) {  // levels 4,12,...,52,62
    int best = 0;
    float bd = 1e30f;
    for (int i = 0; i < 8; ++i) {
        const float d = std::fabs(v - (float) tsx_iq3xxs_level((uint32_t) i));
        if (d < bd) { bd = d; best = i; }
    }
    return best;
}
int nearest_level_s(float v) {  // levels 1,3,...,15
    const int i = (int) std::lround((v - 1.0f) * 0.5f);
    return std::clamp(i, 0, 7);
}

void quant_q8_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[32 * b + j]));
        const float d = amax / 127.f, id = d != 0.f ? 1.0f / d : 0.0f;
        const uint16_t dh = f2h(d);
        std::memcpy(out + 34 * b, &dh, 2);
        for (int j = 0; j < 32; ++j) out[34 * b + 2 + j] = (uint8_t) (int8_t) std::roundf(x[32 * b + j] * id);
    }
}

void quant_q4_K(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 256; ++b, x += 256) {
        uint8_t* blk = out + 144 * b;
        float scale[8], minv[8];
        for (int j = 0; j < 8; ++j) {
            float mn = 0.f, mx = 0.f;
            for (int i = 0; i < 32; ++i) { mn = std::min(mn, x[32 * j + i]); mx = std::max(mx, x[32 * j + i]); }
            scale[j] = (mx - mn) / 15.f;
            minv[j] = -mn;
        }
        const float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(minv, minv + 8);
        const uint16_t dh = f2h(ms / 63.f), mh = f2h(mm / 63.f);
        const float d = h2f(dh), dmin = h2f(mh);
        int sc[8], m[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = d > 0.f ? std::clamp((int) std::lround(scale[j] / d), 0, 63) : 0;
            m[j] = dmin > 0.f ? std::clamp((int) std::lround(minv[j] / dmin), 0, 63) : 0;
        }
        std::memcpy(blk, &dh, 2);
        std::memcpy(blk + 2, &mh, 2);
        uint8_t* s12 = blk + 4;
        for (int j = 0; j < 4; ++j) {
            s12[j] = (uint8_t) ((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t) ((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t) ((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; ++j) {
            const float a = d * (float) sc[j], off = dmin * (float) m[j];
            for (int i = 0; i < 32; ++i)
                q[32 * j + i] = a > 0.f ? (uint8_t) std::clamp((int) std::lround((x[32 * j + i] + off) / a), 0, 15) : 0;
        }
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 32; ++i) blk[16 + 32 * c + i] = (uint8_t) (q[64 * c + i] | (q[64 * c + 32 + i] << 4));
    }
}

void quant_iq3_xxs(const float* x, int64_t n, uint8_t* out) {
    const Nearest& nt = nearest();
    for (int64_t b = 0; b < n / 256; ++b, x += 256) {
        uint8_t* blk = out + 98 * b;
        float db[8];
        for (int j = 0; j < 8; ++j) {
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[32 * j + i]));
            db[j] = amax / 62.f;
        }
        const uint16_t dh = f2h(*std::max_element(db, db + 8) * 4.f / 31.f);
        const float d = h2f(dh);
        std::memcpy(blk, &dh, 2);
        for (int j = 0; j < 8; ++j) {
            const int ls = d > 0.f ? std::clamp((int) std::lround((db[j] * 4.f / d - 1.f) * 0.5f), 0, 15) : 0;
            const float eff = d * (float) (2 * ls + 1) * 0.25f;
            const float* v = x + 32 * j;
            uint32_t aux = (uint32_t) ls << 28;
            for (int l = 0; l < 4; ++l) {  // 8 values: two grid words and 7 sign bits (+ even parity)
                uint32_t bits = 0;
                int amin = 0;
                for (int i = 0; i < 8; ++i) {
                    if (v[8 * l + i] < 0.f) bits |= 1u << i;
                    if (std::fabs(v[8 * l + i]) < std::fabs(v[8 * l + amin])) amin = i;
                }
                if (__builtin_popcount(bits) & 1) bits ^= 1u << amin;  // odd: flip the smallest value's sign
                aux |= (bits & 127u) << (7 * l);
                for (int h = 0; h < 2; ++h) {
                    int code = 0;
                    for (int k = 0; k < 4; ++k) {
                        const float mag = eff > 0.f ? std::fabs(v[8 * l + 4 * h + k]) / eff : 0.f;
                        code |= nearest_level_xxs(mag) << (3 * k);
                    }
                    blk[2 + 8 * j + 2 * l + h] = (uint8_t) nt.xxs[code];
                }
            }
            std::memcpy(blk + 2 + 64 + 4 * j, &aux, 4);
        }
    }
}

void quant_iq3_s(const float* x, int64_t n, uint8_t* out) {
    const Nearest& nt = nearest();
    for (int64_t b = 0; b < n / 256; ++b, x += 256) {
        uint8_t* blk = out + 110 * b;
        std::memset(blk, 0, 110);
        float db[8];
        for (int j = 0; j < 8; ++j) {
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[32 * j + i]));
            db[j] = amax / 15.f;
        }
        const uint16_t dh = f2h(*std::max_element(db, db + 8) / 31.f);
        const float d = h2f(dh);
        std::memcpy(blk, &dh, 2);
        for (int j = 0; j < 8; ++j) {
            const int s = d > 0.f ? std::clamp((int) std::lround((db[j] / d - 1.f) * 0.5f), 0, 15) : 0;
            const float eff = d * (float) (2 * s + 1);
            blk[106 + j / 2] |= (uint8_t) (s << (4 * (j % 2)));
            const float* v = x + 32 * j;
            for (int k = 0; k < 8; ++k) {
                int code = 0;
                for (int i = 0; i < 4; ++i) {
                    const float val = v[4 * k + i];
                    code |= nearest_level_s(eff > 0.f ? std::fabs(val) / eff : 0.f) << (3 * i);
                    if (val < 0.f) blk[74 + 4 * j + k / 2] |= (uint8_t) (1u << (4 * (k % 2) + i));
                }
                const int idx = nt.s[code];
                blk[2 + 8 * j + k] = (uint8_t) (idx & 255);
                blk[66 + j] |= (uint8_t) (((idx >> 8) & 1) << k);
            }
        }
    }
}

}  // namespace

extern "C" TSX_API int tsx_moe_quantize_weights(int type, const float* x, int64_t n_rows, int64_t n_cols, void* out) {
    const size_t rb = tsx_row_bytes(type, n_cols);
    if (x == nullptr || out == nullptr || n_rows < 0 || rb == 0 || !tsx_weight_type_ok(type)) return TSX_ERR_ARG;
    for (int64_t r = 0; r < n_rows; ++r) {
        const float* xr = x + r * n_cols;
        uint8_t* o = (uint8_t*) out + (size_t) r * rb;
        switch (type) {
            case TSX_Q8_0: quant_q8_0(xr, n_cols, o); break;
            case TSX_Q4_K: quant_q4_K(xr, n_cols, o); break;
            case TSX_IQ3_XXS: quant_iq3_xxs(xr, n_cols, o); break;
            case TSX_IQ3_S: quant_iq3_s(xr, n_cols, o); break;
            default: return TSX_ERR_UNSUPPORTED;
        }
    }
    return TSX_OK;
}
