// tsx_cpu_rows.cpp - one routed expert's rows on the CPU, for the hybrid CPU/GPU split: experts without a slot in
// HBM run here while the GPU runs the resident ones.
//
// Reference: strata::kernels::cpu::native_gu_rows / native_down_rows / native_quant_act / native_quant_h
// (include/strata/kernels/cpu/native_expert.hpp:41-65; src/kernels/cpu/native_expert.cpp:147-299) and the
// multi-token IQ rows (src/kernels/cpu/iq_avx512.cpp:108-186): a weight block is decoded once and dotted with every
// token of the job.  The activations here are Q8_1 (the GPU kernels' contract), not ggml's vec_dot_type, so a miss
// served by the CPU has the same integer sub-block sums S_j = sum w_int * a_int as it would on the GPU.
//
// Per row and token: acc = sum over 32-value units u (in order) of d8_u * (a_u * S_u - b_u * M_u) in double, with
// a_u the unit's weight scale (d * (2 ls + 1) / 4 for IQ3_XXS, d * (2 ls + 1) for IQ3_S, d * sc for Q4_K, d for
// Q8_0), b_u = dmin * m (Q4_K, else 0) and M_u the unit's sum of activation codes; the row's value is (float) acc.
// The integer dot of a unit is one AVX2 maddubs chain where the CPU has AVX2, else a scalar loop (same integers).
#pragma STDC FP_CONTRACT OFF

#include <immintrin.h>

#include <cmath>
#include <cstring>

#include "tsx_common.hpp"
#include "tsx_half.hpp"
#include "tsx_pool.h"

namespace tsx {
namespace {

constexpr int kQ8_1 = 9;

inline uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}
inline uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}

// ------------------------------------------------------------------ integer dot of 32 int8 pairs
int dot32_scalar(const int8_t* w, const int8_t* a) {
    int s = 0;
    for (int i = 0; i < 32; ++i) s += (int) w[i] * (int) a[i];
    return s;
}
// |w| (unsigned) times a with w's sign, pairs summed to int16 (|w| <= 128, |a| <= 127: no saturation), then to int32
__attribute__((target("avx2"))) inline int dot32_avx2(const int8_t* w, const int8_t* a) {
    const __m256i vw = _mm256_loadu_si256((const __m256i*) w), va = _mm256_loadu_si256((const __m256i*) a);
    const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(vw, vw), _mm256_sign_epi8(va, vw));
    const __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
    const __m128i s4 = _mm_add_epi32(_mm256_castsi256_si128(p32), _mm256_extracti128_si256(p32, 1));
    const __m128i s2 = _mm_add_epi32(s4, _mm_shuffle_epi32(s4, 0x4E));
    const __m128i s1 = _mm_add_epi32(s2, _mm_shuffle_epi32(s2, 0xB1));
    return _mm_cvtsi128_si32(s1);
}

// ------------------------------------------------------------------ weight units
// Up to 8 units (one 256-value block, or one 32-value Q8_0 block): int8 weights and the double scale pieces
struct Units {
    alignas(32) int8_t w[8][32];
    double a[8], b[8];
    int n;
};

inline uint32_t sign_byte_xxs(uint32_t v7) { return v7 | ((uint32_t) __builtin_popcount(v7) & 1u) << 7; }

void put_word(int8_t* dst, uint32_t g, uint32_t signs4) {  // 4 grid bytes with 4 sign bits
    for (int i = 0; i < 4; ++i) {
        const int v = (int) ((g >> (8 * i)) & 0xFFu);
        dst[i] = (int8_t) (((signs4 >> i) & 1u) ? -v : v);
    }
}

// block `blk` of a row of `type` -> its units
void decode_block(int type, const uint8_t* blk, Units& U) {
    switch (type) {
        case TSX_IQ3_XXS: {  // {d; qs[64] grid indices; 8 x u32: 4 x 7 sign bits, 4-bit scale}
            const double d = (double) h2f(rd16(blk));
            for (int j = 0; j < 8; ++j) {
                const uint32_t aux = rd32(blk + 66 + 4 * j);
                for (int l = 0; l < 4; ++l) {
                    const uint32_t s8 = sign_byte_xxs((aux >> (7 * l)) & 127u);
                    put_word(U.w[j] + 8 * l, tsx_iq3xxs_word(blk[2 + 8 * j + 2 * l]), s8 & 15u);
                    put_word(U.w[j] + 8 * l + 4, tsx_iq3xxs_word(blk[2 + 8 * j + 2 * l + 1]), s8 >> 4);
                }
                U.a[j] = d * 0.25 * (int) (2 * (aux >> 28) + 1);
                U.b[j] = 0.0;
            }
            U.n = 8;
            return;
        }
        case TSX_IQ3_S: {  // {d; qs[64]; qh[8]; signs[32]; scales[4]}
            const double d = (double) h2f(rd16(blk));
            for (int j = 0; j < 8; ++j) {
                const uint32_t qh = blk[66 + j];
                for (int q = 0; q < 8; ++q) {
                    const int idx = (int) (blk[2 + 8 * j + q] | ((qh >> q) & 1u) << 8);
                    put_word(U.w[j] + 4 * q, tsx_iq3s_word(idx), (uint32_t) (blk[74 + 4 * j + q / 2] >> (4 * (q & 1))));
                }
                U.a[j] = d * (int) (2 * ((blk[106 + j / 2] >> (4 * (j & 1))) & 15u) + 1);
                U.b[j] = 0.0;
            }
            U.n = 8;
            return;
        }
        case TSX_Q4_K: {  // {d, dmin; scales[12] (6-bit sc, m); qs[128]}
            const float d = h2f(rd16(blk)), dmin = h2f(rd16(blk + 2));
            const uint8_t* sc = blk + 4;
            for (int j = 0; j < 8; ++j) {
                int s, m;
                if (j < 4) {
                    s = sc[j] & 63;
                    m = sc[j + 4] & 63;
                } else {
                    s = (sc[j + 4] & 15) | (sc[j - 4] >> 6) << 4;
                    m = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4;
                }
                const uint8_t* qs = blk + 16 + 32 * (j / 2);
                for (int i = 0; i < 32; ++i) U.w[j][i] = (int8_t) ((j & 1) ? qs[i] >> 4 : qs[i] & 15);
                U.a[j] = (double) d * s;
                U.b[j] = (double) dmin * m;
            }
            U.n = 8;
            return;
        }
        default: {  // Q8_0 {d; qs[32]}
            std::memcpy(U.w[0], blk + 2, 32);
            U.a[0] = (double) h2f(rd16(blk));
            U.b[0] = 0.0;
            U.n = 1;
            return;
        }
    }
}

// ------------------------------------------------------------------ the same units with AVX2
// The grid words of a unit come from one 8-lane gather; the 32 sign bits (byte v / 8, bit v % 8 for value v) become
// a byte mask m, and w = (g ^ m) - m negates where it is set.
struct HostGrids {
    uint32_t xxs[256], s[512];
    HostGrids() {
        for (int i = 0; i < 256; ++i) xxs[i] = tsx_iq3xxs_word(i);
        for (int i = 0; i < 512; ++i) s[i] = tsx_iq3s_word(i);
    }
};
const HostGrids g_grids;

__attribute__((target("avx2"))) inline __m256i sign_mask(uint32_t sw) {
    const __m256i sel = _mm256_setr_epi8(0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 3, 3,
                                         3, 3, 3, 3, 3, 3);
    const __m256i bit = _mm256_set1_epi64x((long long) 0x8040201008040201ULL);
    const __m256i v = _mm256_shuffle_epi8(_mm256_set1_epi32((int) sw), sel);
    return _mm256_cmpeq_epi8(_mm256_and_si256(v, bit), bit);
}
__attribute__((target("avx2"))) inline void put_unit(int8_t* dst, __m256i g, uint32_t sw) {
    const __m256i m = sign_mask(sw);
    _mm256_store_si256((__m256i*) dst, _mm256_sub_epi8(_mm256_xor_si256(g, m), m));
}

__attribute__((target("avx2"))) inline void decode_block_avx2(int type, const uint8_t* blk, Units& U) {
    switch (type) {
        case TSX_IQ3_XXS: {
            const double d = (double) h2f(rd16(blk));
            for (int j = 0; j < 8; ++j) {
                const uint32_t aux = rd32(blk + 66 + 4 * j);
                const __m256i idx = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*) (blk + 2 + 8 * j)));
                const __m256i g = _mm256_i32gather_epi32((const int*) g_grids.xxs, idx, 4);
                uint32_t sw = 0;
                for (int l = 0; l < 4; ++l) sw |= sign_byte_xxs((aux >> (7 * l)) & 127u) << (8 * l);
                put_unit(U.w[j], g, sw);
                U.a[j] = d * 0.25 * (int) (2 * (aux >> 28) + 1);
                U.b[j] = 0.0;
            }
            U.n = 8;
            return;
        }
        case TSX_IQ3_S: {
            const double d = (double) h2f(rd16(blk));
            const __m256i shifts = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
            for (int j = 0; j < 8; ++j) {
                const __m256i lo = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*) (blk + 2 + 8 * j)));
                const __m256i hi = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(blk[66 + j]), shifts),
                                                    _mm256_set1_epi32(1));
                const __m256i g = _mm256_i32gather_epi32((const int*) g_grids.s,
                                                         _mm256_or_si256(lo, _mm256_slli_epi32(hi, 8)), 4);
                put_unit(U.w[j], g, rd32(blk + 74 + 4 * j));
                U.a[j] = d * (int) (2 * ((blk[106 + j / 2] >> (4 * (j & 1))) & 15u) + 1);
                U.b[j] = 0.0;
            }
            U.n = 8;
            return;
        }
        case TSX_Q4_K: {
            const float d = h2f(rd16(blk)), dmin = h2f(rd16(blk + 2));
            const uint8_t* sc = blk + 4;
            const __m256i low4 = _mm256_set1_epi8(15);
            for (int j = 0; j < 8; ++j) {
                int s, m;
                if (j < 4) {
                    s = sc[j] & 63;
                    m = sc[j + 4] & 63;
                } else {
                    s = (sc[j + 4] & 15) | (sc[j - 4] >> 6) << 4;
                    m = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4;
                }
                const __m256i q = _mm256_loadu_si256((const __m256i*) (blk + 16 + 32 * (j / 2)));
                _mm256_store_si256((__m256i*) U.w[j],
                                   _mm256_and_si256((j & 1) ? _mm256_srli_epi16(q, 4) : q, low4));
                U.a[j] = (double) d * s;
                U.b[j] = (double) dmin * m;
            }
            U.n = 8;
            return;
        }
        default: decode_block(type, blk, U); return;
    }
}
// y[r][t] = row r . act[t] for two rows (rows[1] may equal rows[0]) and nt tokens; n_in values (whole blocks of the
// type).  Two rows at once keep two independent accumulation chains in flight; each row's sum runs over its units in
// order, so the value is the one-row value.  One body, compiled twice: with the AVX2 decode and dot (the CPU has
// AVX2), and scalar.
#define TSX_ROW_DOT_BODY(DECODE, DOT)                                                               \
    const int qk = type == TSX_Q8_0 ? 32 : 256;                                                     \
    const size_t bb = tsx_type_block_bytes(type);                                                   \
    const bool q4k = type == TSX_Q4_K;                                                              \
    double acc[2][TSX_CPU_MAXT];                                                                    \
    for (int t = 0; t < nt; ++t) acc[0][t] = acc[1][t] = 0.0;                                       \
    Units U[2];                                                                                     \
    for (int64_t blk = 0; blk < n_in / qk; ++blk) {                                                 \
        DECODE(type, rows[0] + blk * bb, U[0]);                                                     \
        DECODE(type, rows[1] + blk * bb, U[1]);                                                     \
        const int64_t u0 = blk * (qk / 32);                                                         \
        for (int j = 0; j < U[0].n; ++j) {                                                          \
            const int64_t u = u0 + j;                                                               \
            for (int t = 0; t < nt; ++t) {                                                          \
                const int8_t* a8 = (const int8_t*) (act[t] + 36 * u + 4);                           \
                const int S0 = DOT(U[0].w[j], a8), S1 = DOT(U[1].w[j], a8);                         \
                const int M = q4k ? msum[t][u] : 0;                                                 \
                acc[0][t] += d8[t][u] * (U[0].a[j] * S0 - U[0].b[j] * M);                           \
                acc[1][t] += d8[t][u] * (U[1].a[j] * S1 - U[1].b[j] * M);                           \
            }                                                                                       \
        }                                                                                           \
    }                                                                                               \
    for (int t = 0; t < nt; ++t) {                                                                  \
        y[0][t] = (float) acc[0][t];                                                                \
        y[1][t] = (float) acc[1][t];                                                                \
    }

void row_dot_scalar(int type, const uint8_t* const* rows, int64_t n_in, const uint8_t* const* act, int nt,
                    float (*y)[TSX_CPU_MAXT], const double* const* d8, const int* const* msum) {
    TSX_ROW_DOT_BODY(decode_block, dot32_scalar)
}
__attribute__((target("avx2"))) void row_dot_avx2(int type, const uint8_t* const* rows, int64_t n_in,
                                                  const uint8_t* const* act, int nt, float (*y)[TSX_CPU_MAXT],
                                                  const double* const* d8, const int* const* msum) {
    TSX_ROW_DOT_BODY(decode_block_avx2, dot32_avx2)
}
#undef TSX_ROW_DOT_BODY
using RowDot = void (*)(int, const uint8_t* const*, int64_t, const uint8_t* const*, int, float (*)[TSX_CPU_MAXT],
                        const double* const*, const int* const*);
const RowDot row_dot2 = __builtin_cpu_supports("avx2") ? row_dot_avx2 : row_dot_scalar;

// per-token unit scales and code sums of nt Q8_1 rows of nu units (the caller's buffers)
void unpack_acts(const void* const* act, int nt, int64_t nu, bool sums, double* d8, int* ms, const double** pd,
                 const int** pm) {
    for (int t = 0; t < nt; ++t) {
        const uint8_t* a = (const uint8_t*) act[t];
        for (int64_t u = 0; u < nu; ++u) {
            d8[t * nu + u] = (double) h2f(rd16(a + 36 * u));
            if (sums) {
                int s = 0;
                for (int i = 0; i < 32; ++i) s += (int8_t) a[36 * u + 4 + i];
                ms[t * nu + u] = s;
            }
        }
        pd[t] = d8 + t * nu;
        pm[t] = ms + t * nu;
    }
}

inline float q8_1_finite(float v) { return std::fabs(v) > 65504.0f ? std::copysign(65504.0f, v) : v; }

// Q8_1 of n values: per 32, the largest magnitude and the sum by a 32-lane xor butterfly (the order of the GPU
// quantizers' reductions), d = amax / 127, codes round(x / d) within +-127 (0 when amax is 0)
void quant_q8_1(const float* x, int64_t n, uint8_t* dst) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* xb = x + 32 * b;
        float am[32], sm[32], ta[32], ts[32];
        for (int l = 0; l < 32; ++l) {
            am[l] = std::fabs(xb[l]);
            sm[l] = xb[l];
        }
        for (int o = 16; o > 0; o >>= 1) {
            for (int l = 0; l < 32; ++l) {
                ta[l] = std::fmax(am[l], am[l ^ o]);
                ts[l] = sm[l] + sm[l ^ o];
            }
            std::memcpy(am, ta, sizeof am);
            std::memcpy(sm, ts, sizeof sm);
        }
        const float amax = am[0], d = q8_1_finite(amax / 127.0f);
        uint8_t* y = dst + 36 * b;
        for (int l = 0; l < 32; ++l) {
            int q = 0;
            if (amax != 0.0f) {
                const float r = std::round(xb[l] / d);
                q = (int) (r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r);
            }
            y[4 + l] = (uint8_t) (int8_t) q;
        }
        const uint16_t hd = f2h(q8_1_finite(d)), hs = f2h(q8_1_finite(sm[0]));
        std::memcpy(y, &hd, 2);
        std::memcpy(y + 2, &hs, 2);
    }
}

bool fmt_ok(const tsx_cpu_fmt* f) { return f && f->gu_act == kQ8_1 && f->d_act == kQ8_1 && f->n_embd > 0; }

}  // namespace

// the rows of one phase, shared with the pool
int cpu_gu_rows(const tsx_cpu_fmt& f, const uint8_t* blob, const void* const* act, int nt, float* const* ff, int r0,
                int r1) {
    const int64_t N = f.n_embd, nu = N / 32;
    const bool q4k = f.gu_type == TSX_Q4_K;
    double d8[TSX_CPU_MAXT * 512];
    int ms[TSX_CPU_MAXT * 512];
    if (nu > 512) return TSX_ERR_UNSUPPORTED;
    const double* pd[TSX_CPU_MAXT];
    const int* pm[TSX_CPU_MAXT];
    unpack_acts(act, nt, nu, q4k, d8, ms, pd, pm);
    const uint8_t* const* a = (const uint8_t* const*) act;
    float gu[2][TSX_CPU_MAXT];
    for (int r = r0; r < r1; ++r) {  // gate row r and up row r together
        const uint8_t* rows[2] = {blob + (uint64_t) r * f.gu_row, blob + f.up_off + (uint64_t) r * f.gu_row};
        row_dot2(f.gu_type, rows, N, a, nt, gu, pd, pm);
        for (int t = 0; t < nt; ++t) {
            const float s = gu[0][t] / (1.0f + std::exp(-gu[0][t]));
            ff[t][r] = s * gu[1][t];
        }
    }
    return TSX_OK;
}

int cpu_down_rows(const tsx_cpu_fmt& f, const uint8_t* blob, const void* const* hq, int nt, float* const* out,
                  int r0, int r1) {
    const int64_t FF = f.n_ff, nu = FF / 32;
    const bool q4k = f.d_type == TSX_Q4_K;
    double d8[TSX_CPU_MAXT * 256];
    int ms[TSX_CPU_MAXT * 256];
    if (nu > 256) return TSX_ERR_UNSUPPORTED;
    const double* pd[TSX_CPU_MAXT];
    const int* pm[TSX_CPU_MAXT];
    unpack_acts(hq, nt, nu, q4k, d8, ms, pd, pm);
    const uint8_t* const* a = (const uint8_t* const*) hq;
    float y[2][TSX_CPU_MAXT];
    for (int r = r0; r < r1; r += 2) {  // rows r and r + 1 together (r alone twice at an odd end)
        const int r2 = r + 1 < r1 ? r + 1 : r;
        const uint8_t* rows[2] = {blob + f.down_off + (uint64_t) r * f.d_row, blob + f.down_off + (uint64_t) r2 * f.d_row};
        row_dot2(f.d_type, rows, FF, a, nt, y, pd, pm);
        for (int t = 0; t < nt; ++t) {
            out[t][r] = y[0][t];
            out[t][r2] = y[1][t];
        }
    }
    return TSX_OK;
}

void cpu_quant(const float* x, int64_t n, void* dst) { quant_q8_1(x, n, (uint8_t*) dst); }

}  // namespace tsx

using namespace tsx;

extern "C" {

TSX_API int tsx_cpu_fmt_init(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, tsx_cpu_fmt* f) {
    clear_error();
    TSX_REQUIRE(f != nullptr, "tsx_cpu_fmt_init: null output");
    auto ok = [](int t) { return t == TSX_IQ3_XXS || t == TSX_IQ3_S || t == TSX_Q4_K || t == TSX_Q8_0; };
    if (!ok(gu_type) || !ok(d_type) || n_embd <= 0 || n_ff <= 0 || n_embd % 256 || n_ff % 256 || n_embd > 16384 ||
        n_ff > 8192) {
        set_error("tsx_cpu_fmt_init: types %d/%d, n_embd %lld, n_ff %lld not supported (expert types; multiples of "
                  "256; n_embd <= 16384, n_ff <= 8192)", gu_type, d_type, (long long) n_embd, (long long) n_ff);
        return TSX_ERR_UNSUPPORTED;
    }
    tsx_expert_layout L;
    if (tsx_moe_expert_layout(gu_type, d_type, n_embd, n_ff, &L) != TSX_OK) return TSX_ERR_UNSUPPORTED;
    f->gu_type = gu_type;
    f->d_type = d_type;
    f->gu_act = f->d_act = kQ8_1;
    f->n_embd = n_embd;
    f->n_ff = n_ff;
    f->gu_row = L.gu_row;
    f->d_row = L.d_row;
    f->up_off = L.up_off;
    f->down_off = L.down_off;
    f->bytes = L.bytes;
    f->act_bytes = (uint64_t) (n_embd / 32) * 36;
    f->h_bytes = (uint64_t) (n_ff / 32) * 36;
    return TSX_OK;
}

TSX_API int tsx_cpu_quant_act(const tsx_cpu_fmt* f, const float* x, void* dst) {
    clear_error();
    TSX_REQUIRE(fmt_ok(f) && x && dst, "tsx_cpu_quant_act: format, x and dst");
    cpu_quant(x, f->n_embd, dst);
    return TSX_OK;
}

TSX_API int tsx_cpu_quant_h(const tsx_cpu_fmt* f, const float* h, void* dst) {
    clear_error();
    TSX_REQUIRE(fmt_ok(f) && h && dst, "tsx_cpu_quant_h: format, h and dst");
    cpu_quant(h, f->n_ff, dst);
    return TSX_OK;
}

TSX_API int tsx_cpu_gu_rows(const tsx_cpu_fmt* f, const uint8_t* blob, const void* const* act, int nt,
                            float* const* ff, int r0, int r1) {
    clear_error();
    TSX_REQUIRE(fmt_ok(f) && blob && act && ff && nt >= 1 && nt <= TSX_CPU_MAXT && 0 <= r0 && r0 <= r1 &&
                    r1 <= f->n_ff, "tsx_cpu_gu_rows: format, blob, 1..8 tokens, 0 <= r0 <= r1 <= n_ff");
    return cpu_gu_rows(*f, blob, act, nt, ff, r0, r1);
}

TSX_API int tsx_cpu_down_rows(const tsx_cpu_fmt* f, const uint8_t* blob, const void* const* hq, int nt,
                              float* const* out, int r0, int r1) {
    clear_error();
    TSX_REQUIRE(fmt_ok(f) && blob && hq && out && nt >= 1 && nt <= TSX_CPU_MAXT && 0 <= r0 && r0 <= r1 &&
                    r1 <= f->n_embd, "tsx_cpu_down_rows: format, blob, 1..8 tokens, 0 <= r0 <= r1 <= n_embd");
    return cpu_down_rows(*f, blob, hq, nt, out, r0, r1);
}

}  // extern "C"
