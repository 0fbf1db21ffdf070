/* oracle/oracle.c - TEST INFRASTRUCTURE ONLY: a plain-C restatement of TinyStrata's MoE expert matmul (the ggml
 * mul_mat_id path) used as the parity checker for the HIP library.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path (tinystrata_amd/) never does.
 *
 * What each function restates (reference paths are relative to the TinyStrata repository root):
 *   orc_f2h / orc_h2f          IEEE binary16 round-to-nearest-even, the conversion __float2half performs.
 *   orc_quantize_q8_1          q8_1_store + q8_1_finite/quant/ds: src/kernels/cuda/iq_kernels.cu:1467-1487,
 *                              include/strata/kernels/q8_1_finite.hpp:16-31 (the block sum in the warp's xor-tree
 *                              order, so the stored fp16 sum is the GPU's bit for bit).
 *   orc_quantize_q8_K          ggml quantize_row_q8_K_ref, as restated by q8k_quant_avx2:
 *                              src/kernels/cpu/iq_avx2.cpp:387-454.
 *   orc_quantize_q8_0          ggml quantize_row_q8_0_ref (the Q8_0 vec_dot_type of src/kernels/cpu/native_expert.cpp:62-91).
 *   orc_dequantize             the block decodes of ggml-common.h formats: IQ3_XXS / IQ3_S as
 *                              src/kernels/cpu/iq_avx512.cpp:108-153 (Fmt<18>, Fmt<21>), Q4_K scales as
 *                              src/kernels/cuda/iq_kernels.cu:353-365 (k_scale_min) and src/kernels/cpu/kq_avx2.cpp:84-110.
 *   orc_subblock_sums          the integer contract: S_j = sum w_int * a_int per 32-value sub-block (and for Q4_K
 *                              M_j = sum a_int), src/kernels/cuda/iq_kernels.cu:188-236 (IQ3), 314-387 (Q4_K),
 *                              555-564 (Q8_0).
 *   orc_mmvq_q8_1              y = W . x against Q8_1 activations (the GPU contract), per sub-block
 *                              d_w * K * (2ls+1) * d8 * S (IQ3_XXS, K = 1/4, src/kernels/cpu/iq_avx512.cpp:108),
 *                              d_w * (2s+1) * d8 * S (IQ3_S), d*sc*d8*S - dmin*m*d8*M (Q4_K, iq_kernels.cu:314-330),
 *                              d_w * d8 * S (Q8_0).  Accumulated in double (the exact value of the quantized product
 *                              to ~1e-15), the yardstick the 1e-3 relative L2 bound is measured against.
 *   orc_mmvq_ggml              the reference CPU semantics: IQ3/Q4_K against Q8_K, Q8_0 against Q8_0
 *                              (src/kernels/cpu/iq_avx512.cpp:155-186, src/kernels/cpu/kq_avx2.cpp:84-189).
 *   orc_router_topk            route_topk<NE,K>: src/kernels/cuda/native_router.cu:42-95 (softmax, NaN -> -FLT_MAX,
 *                              K rounds of argmax with ties to the lower id, weights / max(sum, 6.1035e-5)).
 *   orc_group                  k_group: src/qwen35/q36_engine.cu:394-422 (one group per used expert, ascending id,
 *                              entries in entry order).
 *   orc_route_sort             k_route_count/scan/scatter: src/qwen35/q36_engine.cu:483-510 (inside an expert the
 *                              entries here are in entry order; the reference's atomic order changes no output).
 *   orc_expert_gu/_down        native_expert_grouped's two halves: src/kernels/cuda/iq_kernels.cu:1310-1465 and
 *                              1496-1515 (gate/up rows, h = (g/(1+exp(-g)))*u rounded on its own, Q8_1 of h, down rows
 *                              into out[ent_dst[e]]).
 *   orc_combine                k_moe_out: src/qwen35/q36_engine.cu:304-332 (w0*p0 then fmaf in pick order, plus
 *                              sigmoid(sgate)*shared, added to x).
 *   orc_moe_layer              the whole layer in either activation mode, structured as src/lfm2/cpu_experts.cpp:145-235.
 */
#include "../include/tsx_formats.h"
#include "../include/tsx_grids.h"

#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(_OPENMP)
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ fp16 */
ORC_API float orc_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {  /* subnormal: m * 2^-24, exact in binary32 */
            float v = (float) m * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

ORC_API uint16_t orc_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);  /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                     /* below 2^-14: subnormal half (or zero) */
        if (ax < 0x33000000u) return (uint16_t) sign;           /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int) e;                        /* value = m * 2^(e-150); half ulp = 2^-24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t) (sign | q);
    }
    uint32_t q = ((ax - 0x38000000u) >> 13);  /* rebias exponent 127 -> 15 */
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t) (sign | q);
}

static inline uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }

/* ------------------------------------------------------------------ activation quantizers */
static inline float q8_1_finite(float v) { return fabsf(v) > 65504.0f ? copysignf(65504.0f, v) : v; }

/* One q8_1 block of 32 values, as one 32-lane warp computes it (amax by max, sum by an xor butterfly). */
static void q8_1_block(const float* x, tsx_block_q8_1* y) {
    float amax[32], sum[32], ta[32], ts[32];
    for (int l = 0; l < 32; ++l) { amax[l] = fabsf(x[l]); sum[l] = x[l]; }
    for (int o = 16; o > 0; o >>= 1) {
        for (int l = 0; l < 32; ++l) { ta[l] = fmaxf(amax[l], amax[l ^ o]); ts[l] = sum[l] + sum[l ^ o]; }
        memcpy(amax, ta, sizeof ta);
        memcpy(sum, ts, sizeof ts);
    }
    const float am = amax[0];
    const float d = q8_1_finite(am / 127.0f);
    for (int l = 0; l < 32; ++l) {
        int8_t q = 0;
        if (am != 0.0f) {
            const float r = roundf(x[l] / d);
            q = (int8_t) (r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r);
        }
        y->qs[l] = q;
    }
    y->d = orc_f2h(q8_1_finite(d));
    y->s = orc_f2h(q8_1_finite(sum[0]));
}

ORC_API void orc_quantize_q8_1(const float* x, int64_t n_rows, int64_t n_cols, void* vy) {
    tsx_block_q8_1* y = (tsx_block_q8_1*) vy;
    const int64_t nb = n_cols / 32;
    for (int64_t r = 0; r < n_rows; ++r)
        for (int64_t b = 0; b < nb; ++b) q8_1_block(x + r * n_cols + b * 32, y + r * nb + b);
}

static inline int nearest_int(float fval) {
    const float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

ORC_API void orc_quantize_q8_K(const float* x, int64_t n, void* vy) {
    tsx_block_q8_K* y = (tsx_block_q8_K*) vy;
    for (int64_t i = 0; i < n / 256; ++i, x += 256) {
        float amax = 0.f, mx = 0.f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; mx = x[j]; }
        }
        if (amax == 0.f) {
            y[i].d = 0.f;
            memset(y[i].qs, 0, 256);
            memset(y[i].bsums, 0, sizeof y[i].bsums);  /* the reference leaves them unwritten */
            continue;
        }
        const float iscale = -127.f / mx;
        for (int j = 0; j < 256; ++j) {
            volatile float p = iscale * x[j];  /* the product rounded on its own, as the reference */
            const int v = nearest_int(p);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int k = 0; k < 16; ++k) s += y[i].qs[16 * j + k];
            y[i].bsums[j] = (int16_t) s;
        }
        y[i].d = 1.f / iscale;
    }
}

ORC_API void orc_quantize_q8_0(const float* x, int64_t n, void* vy) {
    tsx_block_q8_0* y = (tsx_block_q8_0*) vy;
    for (int64_t i = 0; i < n / 32; ++i) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[i * 32 + j]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        y[i].d = orc_f2h(d);
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t) roundf(x[i * 32 + j] * id);
    }
}

/* ------------------------------------------------------------------ block decodes (per 32-value sub-block) */
static inline uint32_t ksign8(uint32_t v7) {  /* ksigns_iq2xs: 7 sign bits + an even-parity bit 7 */
    return v7 | ((uint32_t) __builtin_popcount(v7) & 1u) << 7;
}

/* w[32] = signed grid bytes of sub-block j; *iscale = the integer sub-block scale; *d = fp16 block scale */
static void iq3xxs_sub(const uint8_t* blk, int j, int8_t w[32], int* iscale, float* d) {
    const uint8_t* qs = blk + 2 + 8 * j;
    const uint32_t aux = rd32(blk + 2 + 64 + 4 * j);
    for (int l = 0; l < 4; ++l) {
        const uint32_t s = ksign8((aux >> (7 * l)) & 127u);
        const uint32_t g0 = tsx_iq3xxs_word(qs[2 * l]), g1 = tsx_iq3xxs_word(qs[2 * l + 1]);
        for (int i = 0; i < 4; ++i) {
            const int v0 = (int) ((g0 >> (8 * i)) & 255u), v1 = (int) ((g1 >> (8 * i)) & 255u);
            w[8 * l + i] = (int8_t) (((s >> i) & 1u) ? -v0 : v0);
            w[8 * l + 4 + i] = (int8_t) (((s >> (4 + i)) & 1u) ? -v1 : v1);
        }
    }
    *iscale = 2 * (int) (aux >> 28) + 1;
    *d = orc_h2f(rd16(blk));
}

static void iq3s_sub(const uint8_t* blk, int j, int8_t w[32], int* iscale, float* d) {
    const uint8_t* qs = blk + 2 + 8 * j;
    const uint32_t qh = blk[66 + j];
    const uint8_t* sg = blk + 74 + 4 * j;
    for (int k = 0; k < 8; ++k) {
        const uint32_t g = tsx_iq3s_word((int) (qs[k] | (((qh >> k) & 1u) << 8)));
        const uint32_t s = sg[k / 2] >> (4 * (k % 2));
        for (int i = 0; i < 4; ++i) {
            const int v = (int) ((g >> (8 * i)) & 255u);
            w[4 * k + i] = (int8_t) (((s >> i) & 1u) ? -v : v);
        }
    }
    *iscale = 2 * (int) ((blk[106 + j / 2] >> (4 * (j % 2))) & 15u) + 1;
    *d = orc_h2f(rd16(blk));
}

/* Q4_K 6-bit scale/min of sub-block j (ggml get_scale_min_k4) */
static void q4k_scale_min(const uint8_t* sc12, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = sc12[j] & 63;
        *m = sc12[j + 4] & 63;
    } else {
        *sc = (sc12[j + 4] & 0xF) | ((sc12[j - 4] >> 6) << 4);
        *m = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
    }
}

static void q4k_sub(const uint8_t* blk, int j, int8_t w[32], int* sc, int* m, float* d, float* dmin) {
    const uint8_t* qs = blk + 16 + 32 * (j / 2);
    for (int i = 0; i < 32; ++i) w[i] = (int8_t) ((j & 1) ? (qs[i] >> 4) : (qs[i] & 15));
    q4k_scale_min(blk + 4, j, sc, m);
    *d = orc_h2f(rd16(blk));
    *dmin = orc_h2f(rd16(blk + 2));
}

/* Q6_K block -> 256 signed codes (code - 32) and the 16 signed scales, in ggml's dequantize_row_q6_K order: for each
 * 128-value half, value l (0..31) of quarter q takes the low (q = 0, 1) or high (q = 2, 3) nibble of ql[l + 32 (q % 2)]
 * and bits 2q, 2q + 1 of qh[l]; scale index = l / 16 + 2q (the reference reads the same layout,
 * src/lfm2/matvec.cu:762-794) */
static void q6k_block(const uint8_t* blk, int8_t v[256], int8_t sc[16]) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    for (int half = 0; half < 2; ++half) {
        for (int l = 0; l < 32; ++l) {
            const int h = qh[32 * half + l];
            v[128 * half + l] = (int8_t) (((ql[64 * half + l] & 0xF) | ((h & 3) << 4)) - 32);
            v[128 * half + l + 32] = (int8_t) (((ql[64 * half + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32);
            v[128 * half + l + 64] = (int8_t) (((ql[64 * half + l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
            v[128 * half + l + 96] = (int8_t) (((ql[64 * half + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32);
        }
    }
    memcpy(sc, blk + 192, 16);
}

/* One sub-block (32 values) of a row: integer weights and the float pieces of its scale.
 * value(i) = a * k(i) * w[i] - b, k(i) = k16[i / 16] (1 except Q6_K), b only for Q4_K; Q4_0's w are the raw codes
 * 0..15 and its value a * (w[i] - 8) */
typedef struct { int8_t w[32]; double a, b; int isc, mn; float d, dmin; int k16[2]; } sub_t;

static int decode_sub(int type, const uint8_t* row, int64_t u, sub_t* s) {
    s->b = 0.0;
    s->mn = 0;
    s->k16[0] = s->k16[1] = 1;
    switch (type) {
        case TSX_Q4_0: {
            const uint8_t* blk = row + u * 18;
            for (int i = 0; i < 16; ++i) {
                s->w[i] = (int8_t) (blk[2 + i] & 15);
                s->w[16 + i] = (int8_t) (blk[2 + i] >> 4);
            }
            s->d = orc_h2f(rd16(blk));
            s->isc = 1;
            s->a = s->d;
            return 0;
        }
        case TSX_Q6_K: {
            const uint8_t* blk = row + (u / 8) * 210;
            int8_t v[256], sc[16];
            q6k_block(blk, v, sc);
            const int j = (int) (u % 8);
            memcpy(s->w, v + 32 * j, 32);
            s->k16[0] = sc[2 * j];
            s->k16[1] = sc[2 * j + 1];
            s->d = orc_h2f(rd16(blk + 208));
            s->isc = 1;
            s->a = s->d;
            return 0;
        }
        case TSX_IQ3_XXS: {
            const uint8_t* blk = row + (u / 8) * 98;
            iq3xxs_sub(blk, (int) (u % 8), s->w, &s->isc, &s->d);
            s->a = (double) s->d * 0.25 * s->isc;
            return 0;
        }
        case TSX_IQ3_S: {
            const uint8_t* blk = row + (u / 8) * 110;
            iq3s_sub(blk, (int) (u % 8), s->w, &s->isc, &s->d);
            s->a = (double) s->d * s->isc;
            return 0;
        }
        case TSX_Q4_K: {
            const uint8_t* blk = row + (u / 8) * 144;
            q4k_sub(blk, (int) (u % 8), s->w, &s->isc, &s->mn, &s->d, &s->dmin);
            s->a = (double) s->d * s->isc;
            s->b = (double) s->dmin * s->mn;
            return 0;
        }
        case TSX_Q8_0: {
            const uint8_t* blk = row + u * 34;
            memcpy(s->w, blk + 2, 32);
            s->d = orc_h2f(rd16(blk));
            s->isc = 1;
            s->a = s->d;
            return 0;
        }
        default: return -1;
    }
}

ORC_API int orc_dequantize(int type, const void* w, int64_t n, float* out) {
    if (!tsx_mmvq_type_ok(type) || n % tsx_type_qk(type) != 0) return -1;
    const uint8_t* p = (const uint8_t*) w;
    for (int64_t u = 0; u < n / 32; ++u) {
        sub_t s;
        decode_sub(type, p, u, &s);
        const int off = type == TSX_Q4_0 ? 8 : 0;
        for (int i = 0; i < 32; ++i) out[u * 32 + i] = (float) (s.a * s.k16[i / 16] * (s.w[i] - off) - s.b);
    }
    return 0;
}

/* the exact integer sum of one sub-block against a Q8_1 block: sum k(i) w[i] a[i] (and sum a[i]) */
static void sub_sums(const sub_t* s, const tsx_block_q8_1* a, int32_t* S, int32_t* M) {
    int32_t lo = 0, hi = 0, m = 0;
    for (int i = 0; i < 16; ++i) { lo += (int32_t) s->w[i] * a->qs[i]; m += a->qs[i]; }
    for (int i = 16; i < 32; ++i) { hi += (int32_t) s->w[i] * a->qs[i]; m += a->qs[i]; }
    *S = s->k16[0] * lo + s->k16[1] * hi;
    *M = m;
}

/* ------------------------------------------------------------------ integer sums and dot products */
/* sums[(r * ncols + c) * nsub + u] = S_u; qsums the same for M_u = sum a_int (null = not wanted) */
ORC_API int orc_subblock_sums(int type, const void* w, int64_t n_in, int64_t n_rows, const void* xq, int64_t ncols,
                              int32_t* sums, int32_t* qsums) {
    if (!tsx_mmvq_type_ok(type) || n_in % tsx_type_qk(type) != 0) return -1;
    const size_t rb = tsx_row_bytes(type, n_in);
    const int64_t nsub = n_in / 32;
    const tsx_block_q8_1* x = (const tsx_block_q8_1*) xq;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
        const uint8_t* row = (const uint8_t*) w + r * rb;
        for (int64_t u = 0; u < nsub; ++u) {
            sub_t s;
            decode_sub(type, row, u, &s);
            for (int64_t c = 0; c < ncols; ++c) {
                const tsx_block_q8_1* a = x + c * nsub + u;
                int32_t S, M;
                sub_sums(&s, a, &S, &M);
                sums[(r * ncols + c) * nsub + u] = S;
                if (qsums) qsums[(r * ncols + c) * nsub + u] = M;
            }
        }
    }
    return 0;
}

/* y[c * n_rows + r] = W[r] . x[c], Q8_1 activations */
ORC_API int orc_mmvq_q8_1(int type, const void* w, int64_t n_in, int64_t n_rows, const void* xq, int64_t ncols, float* y) {
    if (!tsx_mmvq_type_ok(type) || n_in % tsx_type_qk(type) != 0) return -1;
    const size_t rb = tsx_row_bytes(type, n_in);
    const int64_t nsub = n_in / 32;
    const tsx_block_q8_1* x = (const tsx_block_q8_1*) xq;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
        const uint8_t* row = (const uint8_t*) w + r * rb;
        double acc[64];
        for (int64_t c0 = 0; c0 < ncols; c0 += 64) {
            const int64_t nc = ncols - c0 < 64 ? ncols - c0 : 64;
            for (int64_t c = 0; c < nc; ++c) acc[c] = 0.0;
            for (int64_t u = 0; u < nsub; ++u) {
                sub_t s;
                decode_sub(type, row, u, &s);
                for (int64_t c = 0; c < nc; ++c) {
                    const tsx_block_q8_1* a = x + (c0 + c) * nsub + u;
                    int32_t S, M;
                    sub_sums(&s, a, &S, &M);
                    const double d8 = orc_h2f(a->d);
                    if (type == TSX_Q4_0)  /* the reference's affine form with the block's stored sum */
                        acc[c] += s.a * (S * d8 - 8.0 * orc_h2f(a->s));
                    else
                        acc[c] += d8 * (s.a * S - s.b * M);
                }
            }
            for (int64_t c = 0; c < nc; ++c) y[(c0 + c) * n_rows + r] = (float) acc[c];
        }
    }
    return 0;
}

/* The reference CPU arithmetic: IQ3_XXS / IQ3_S / Q4_K rows against Q8_K, Q8_0 rows against Q8_0.
 * Integer sums per 256-block (IQ3: sum_j (2ls+1) S_j; Q4_K: sum_j sc_j S_j and sum_j m_j M_j with M_j from bsums),
 * then the block's float scale, accumulated in double. */
ORC_API int orc_mmvq_ggml(int type, const void* w, int64_t n_in, int64_t n_rows, const void* xq, int64_t ncols, float* y) {
    if (!tsx_weight_type_ok(type) || n_in % tsx_type_qk(type) != 0) return -1;
    const size_t rb = tsx_row_bytes(type, n_in);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
        const uint8_t* row = (const uint8_t*) w + r * rb;
        for (int64_t c = 0; c < ncols; ++c) {
            double acc = 0.0;
            if (type == TSX_Q8_0) {
                const tsx_block_q8_0* a = (const tsx_block_q8_0*) xq + c * (n_in / 32);
                for (int64_t b = 0; b < n_in / 32; ++b) {
                    const uint8_t* blk = row + b * 34;
                    int32_t S = 0;
                    for (int i = 0; i < 32; ++i) S += (int32_t) ((const int8_t*) blk)[2 + i] * a[b].qs[i];
                    acc += (double) orc_h2f(rd16(blk)) * orc_h2f(a[b].d) * S;
                }
            } else {
                const tsx_block_q8_K* a = (const tsx_block_q8_K*) xq + c * (n_in / 256);
                for (int64_t b = 0; b < n_in / 256; ++b) {
                    int64_t isum = 0, msum = 0;
                    float d = 0.f, dmin = 0.f;
                    for (int j = 0; j < 8; ++j) {
                        sub_t s;
                        decode_sub(type, row, b * 8 + j, &s);
                        d = s.d;
                        dmin = s.dmin;
                        int32_t S = 0;
                        for (int i = 0; i < 32; ++i) S += (int32_t) s.w[i] * a[b].qs[32 * j + i];
                        isum += (int64_t) s.isc * S;
                        if (type == TSX_Q4_K) msum += (int64_t) s.mn * (a[b].bsums[2 * j] + a[b].bsums[2 * j + 1]);
                    }
                    const double K = type == TSX_IQ3_XXS ? 0.25 : 1.0;
                    acc += (double) a[b].d * ((double) d * K * (double) isum - (double) dmin * (double) msum);
                }
            }
            y[c * n_rows + r] = (float) acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ routing */
ORC_API int orc_router_topk(const float* logits, int n_tok, int n_expert, int k, int32_t* ids, float* wts) {
    if (n_tok < 0 || n_expert <= 0 || k <= 0 || k > n_expert || k > 32) return -1;
    float* p = (float*) malloc(sizeof(float) * (size_t) n_expert);
    for (int t = 0; t < n_tok; ++t) {
        const float* l = logits + (size_t) t * n_expert;
        float mx = -INFINITY;
        for (int e = 0; e < n_expert; ++e) mx = fmaxf(mx, l[e]);
        double sum = 0.0;
        for (int e = 0; e < n_expert; ++e) { p[e] = expf(l[e] - mx); sum += p[e]; }
        const float rcp = 1.0f / (float) sum;
        for (int e = 0; e < n_expert; ++e) {
            p[e] *= rcp;
            if (isnan(p[e])) p[e] = -FLT_MAX;
        }
        double sel = 0.0;
        for (int r = 0; r < k; ++r) {
            int best = -1;
            for (int e = 0; e < n_expert; ++e)
                if (best < 0 || p[e] > p[best]) best = e;  /* strict: ties keep the lower id */
            ids[(size_t) t * k + r] = best;
            wts[(size_t) t * k + r] = p[best];
            sel += p[best];
            p[best] = -INFINITY;
        }
        float ssum = (float) sel;
        if (ssum < 6.103515625e-5f) ssum = 6.103515625e-5f;
        const float inv = 1.0f / ssum;
        for (int r = 0; r < k; ++r) wts[(size_t) t * k + r] *= inv;
    }
    free(p);
    return 0;
}

ORC_API int orc_group(const int32_t* ids, int n_ent, int k, int n_expert, uint64_t blobs, uint64_t stride,
                      uint64_t* grp_ptr, int32_t* grp_start, int32_t* n_groups, int32_t* ent_dst, int32_t* ent_tok) {
    int32_t* cnt = (int32_t*) calloc((size_t) n_expert, sizeof(int32_t));
    int32_t* off = (int32_t*) calloc((size_t) n_expert, sizeof(int32_t));
    for (int e = 0; e < n_ent; ++e) {
        if (ids[e] < 0 || ids[e] >= n_expert) { free(cnt); free(off); return -1; }
        cnt[ids[e]]++;
    }
    int g = 0, pos = 0;
    for (int x = 0; x < n_expert; ++x) {
        off[x] = pos;
        if (cnt[x] == 0) continue;
        grp_ptr[g] = blobs + (uint64_t) x * stride;
        grp_start[g] = pos;
        pos += cnt[x];
        ++g;
    }
    grp_start[g] = pos;
    *n_groups = g;
    for (int e = 0; e < n_ent; ++e) {
        const int p = off[ids[e]]++;
        ent_dst[p] = e;
        ent_tok[p] = e / k;
    }
    free(cnt);
    free(off);
    return 0;
}

ORC_API int orc_route_sort(const int32_t* ids, int n_ent, int k, int n_expert, int32_t* bounds, int32_t* ent_dst,
                           int32_t* ent_tok, int32_t* rinv, int32_t* max_rows) {
    int32_t* cur = (int32_t*) calloc((size_t) n_expert + 1, sizeof(int32_t));
    for (int e = 0; e < n_ent; ++e) {
        if (ids[e] < 0 || ids[e] >= n_expert) { free(cur); return -1; }
        cur[ids[e]]++;
    }
    int pos = 0, mx = 0;
    for (int x = 0; x < n_expert; ++x) {
        const int c = cur[x];
        bounds[x] = pos;
        cur[x] = pos;
        pos += c;
        if (c > mx) mx = c;
    }
    bounds[n_expert] = pos;
    *max_rows = mx;
    for (int e = 0; e < n_ent; ++e) {
        const int r = cur[ids[e]]++;
        ent_dst[r] = e;
        ent_tok[r] = e / k;
        rinv[e] = r;
    }
    free(cur);
    return 0;
}

ORC_API void orc_combine(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                         const float* shared, const float* sgate, int sg_stride, int n, int n_tok) {
    for (int t = 0; t < n_tok; ++t) {
        const float* pk[32];
        for (int j = 0; j < k; ++j) pk[j] = parts + (size_t) (prow ? prow[t * k + j] : t * k + j) * n;
        const float* wr = wts + (size_t) t * k;
        const float gs = sgate ? 1.0f / (1.0f + expf(-sgate[(size_t) t * sg_stride])) : 0.0f;
        for (int i = 0; i < n; ++i) {
            float acc = wr[0] * pk[0][i];
            for (int j = 1; j < k; ++j) acc = fmaf(wr[j], pk[j][i], acc);
            if (shared) acc += gs * shared[(size_t) t * n + i];
            x[(size_t) t * n + i] += acc;
        }
    }
}

/* ------------------------------------------------------------------ grouped experts (Q8_1 contract) */
static inline float swiglu(float g, float u) {
    const float s = g / (1.0f + expf(-g));
    volatile float h = s * u;  /* rounded on its own, never contracted into a later add */
    return h;
}

/* gate/up half: h[e][n_ff] floats and hq[e][n_ff/32] Q8_1 blocks for entries [0, n_ent) of the groups.
 * blob[g] host pointers; entries of group g are [grp_start[g], grp_start[g+1]). */
ORC_API int orc_expert_gu(const tsx_expert_layout* L, const uint8_t* const* blob, const int32_t* grp_start, int n_groups,
                          const int32_t* ent_tok, const void* x_q8_1, float* h, void* hq) {
    const int64_t N = L->n_embd, FF = L->n_ff, xb = N / 32;
    const tsx_block_q8_1* X = (const tsx_block_q8_1*) x_q8_1;
    for (int g = 0; g < n_groups; ++g) {
        const int e0 = grp_start[g], e1 = grp_start[g + 1];
        for (int e = e0; e < e1; ++e) {
            float* gv = (float*) malloc(sizeof(float) * (size_t) FF * 2);
            const tsx_block_q8_1* xt = X + (int64_t) ent_tok[e] * xb;
            if (orc_mmvq_q8_1(L->gu_type, blob[g], N, FF, xt, 1, gv) != 0 ||
                orc_mmvq_q8_1(L->gu_type, blob[g] + L->up_off, N, FF, xt, 1, gv + FF) != 0) { free(gv); return -1; }
            for (int64_t r = 0; r < FF; ++r) h[(int64_t) e * FF + r] = swiglu(gv[r], gv[FF + r]);
            free(gv);
        }
    }
    const int n_ent = grp_start[n_groups];
    if (hq) orc_quantize_q8_1(h, n_ent, FF, hq);
    return 0;
}

/* down half: out[ent_dst[e]][n_embd] = down rows . hq[e] */
ORC_API int orc_expert_down(const tsx_expert_layout* L, const uint8_t* const* blob, const int32_t* grp_start, int n_groups,
                            const int32_t* ent_dst, const void* hq, float* out) {
    const int64_t N = L->n_embd, FF = L->n_ff, hb = FF / 32;
    const tsx_block_q8_1* H = (const tsx_block_q8_1*) hq;
    for (int g = 0; g < n_groups; ++g)
        for (int e = grp_start[g]; e < grp_start[g + 1]; ++e)
            if (orc_mmvq_q8_1(L->d_type, blob[g] + L->down_off, FF, N, H + (int64_t) e * hb, 1,
                              out + (int64_t) ent_dst[e] * N) != 0) return -1;
    return 0;
}

/* ------------------------------------------------------------------ the whole layer */
/* mode 0: Q8_1 activations (the GPU contract); mode 1: the reference CPU's (Q8_K for IQ3/Q4_K, Q8_0 for Q8_0).
 * blobs: n_expert blobs `stride` bytes apart; shared: one more blob or null (its output weighted by
 * sigmoid(sgate[t])).  y[T][N] = sum_k w_k down_k + gs * shared (no residual).  ids/wts out: [T][K]. */
static void act_bytes(int mode, int wtype, int64_t n, size_t* bytes) {
    if (mode == 0) *bytes = (size_t) (n / 32) * 36;
    else if (wtype == TSX_Q8_0) *bytes = (size_t) (n / 32) * 34;
    else *bytes = (size_t) (n / 256) * 292;
}
static void quant_act(int mode, int wtype, const float* x, int64_t n, void* dst) {
    if (mode == 0) orc_quantize_q8_1(x, 1, n, dst);
    else if (wtype == TSX_Q8_0) orc_quantize_q8_0(x, n, dst);
    else orc_quantize_q8_K(x, n, dst);
}
static int rows_dot(int mode, int type, const uint8_t* w, int64_t n_in, int64_t n_rows, const void* a, float* y) {
    return mode == 0 ? orc_mmvq_q8_1(type, w, n_in, n_rows, a, 1, y) : orc_mmvq_ggml(type, w, n_in, n_rows, a, 1, y);
}

static int one_expert(int mode, const tsx_expert_layout* L, const uint8_t* blob, const float* x, float* out) {
    const int64_t N = L->n_embd, FF = L->n_ff;
    size_t ab = 0, hb = 0;
    act_bytes(mode, L->gu_type, N, &ab);
    act_bytes(mode, L->d_type, FF, &hb);
    void* a = malloc(ab);
    void* hq = malloc(hb);
    float* gu = (float*) malloc(sizeof(float) * (size_t) FF * 3);
    int rc = 0;
    quant_act(mode, L->gu_type, x, N, a);
    rc |= rows_dot(mode, L->gu_type, blob, N, FF, a, gu);
    rc |= rows_dot(mode, L->gu_type, blob + L->up_off, N, FF, a, gu + FF);
    for (int64_t r = 0; r < FF; ++r) gu[2 * FF + r] = swiglu(gu[r], gu[FF + r]);
    quant_act(mode, L->d_type, gu + 2 * FF, FF, hq);
    rc |= rows_dot(mode, L->d_type, blob + L->down_off, FF, N, hq, out);
    free(a);
    free(hq);
    free(gu);
    return rc;
}

ORC_API int orc_moe_layer(int mode, const tsx_expert_layout* L, int n_tok, int n_expert, int k, const float* x,
                          const float* logits, const uint8_t* blobs, uint64_t stride, const uint8_t* shared,
                          const float* sgate, float* y, int32_t* ids, float* wts) {
    const int64_t N = L->n_embd;
    if (orc_router_topk(logits, n_tok, n_expert, k, ids, wts) != 0) return -1;
    float* parts = (float*) malloc(sizeof(float) * (size_t) n_tok * k * N);
    float* sh = shared ? (float*) malloc(sizeof(float) * (size_t) n_tok * N) : NULL;
    int rc = 0;
    for (int e = 0; e < n_tok * k; ++e)
        rc |= one_expert(mode, L, blobs + (uint64_t) ids[e] * stride, x + (int64_t) (e / k) * N, parts + (int64_t) e * N);
    if (shared)
        for (int t = 0; t < n_tok; ++t) rc |= one_expert(mode, L, shared, x + (int64_t) t * N, sh + (int64_t) t * N);
    memset(y, 0, sizeof(float) * (size_t) n_tok * N);
    orc_combine(y, parts, NULL, wts, k, sh, sgate, 1, (int) N, n_tok);
    free(parts);
    free(sh);
    return rc;
}

/* FNV-1a over the expanded grid words (IQ3_XXS then IQ3_S), to pin the table data */
ORC_API uint64_t orc_grid_hash(void) {
    uint64_t h = 1469598103934665603ull;
    for (int i = 0; i < 256 + 512; ++i) {
        const uint32_t w = i < 256 ? tsx_iq3xxs_word(i) : tsx_iq3s_word(i - 256);
        for (int b = 0; b < 4; ++b) h = (h ^ ((w >> (8 * b)) & 255u)) * 1099511628211ull;
    }
    return h;
}

ORC_API int orc_threads(void) {
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}
