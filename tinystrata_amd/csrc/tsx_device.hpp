// tsx_device.hpp - device-side pieces shared by the MoE kernels for gfx950 (CDNA4, wave64).
//
// A weight row is read as "units": 32 consecutive values (one Q8_1 activation block's worth).  unit_load<T>
// decodes one unit of a row of format T into eight packed int8 words (w[k] = values 4k..4k+3) and the float
// factors of its scale, value = a * w - b (b only for Q4_K, whose min multiplies the sum of the activation codes).
// The integer sub-block sum S = sum_k dot4(w[k], q[k]) is exact and order-independent; that is the contract the
// tests pin bit for bit against the oracle.
//
// Block decodes follow the GGUF formats (reference: src/kernels/cuda/iq_kernels.cu:188-236 for IQ3_XXS/IQ3_S,
// 314-387 for Q4_K, 555-564 for Q8_0; src/kernels/cpu/iq_avx512.cpp:108-153 for the per-64 decode).  The IQ3_XXS
// sub-block scale is applied exactly, (2ls+1)/4, as the reference CPU does (iq_avx512.cpp:108, K = 0.25), not with
// ggml-cuda's truncating (ls*S + S/2)/2 (iq_kernels.cu:207-208).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "tsx_moe.h"

namespace tsx {

constexpr int kWave = 64;

// ------------------------------------------------------------------ codebooks, expanded at compile time
struct GridTables {
    uint32_t xxs[256];
    uint32_t s[512];
};
constexpr GridTables make_grid_tables() {
    GridTables g{};
    for (int i = 0; i < 256; ++i) g.xxs[i] = tsx_iq3xxs_word(i);
    for (int i = 0; i < 512; ++i) g.s[i] = tsx_iq3s_word(i);
    return g;
}
static __constant__ const GridTables kGrid = make_grid_tables();

// ------------------------------------------------------------------ scalar helpers
__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 2-byte-aligned loads (IQ3 blocks are 98 / 110 bytes, Q8_0 34: their fields sit on even addresses)
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*) p; }
__device__ __forceinline__ uint32_t ld32a2(const uint8_t* p) {
    const uint16_t* q = (const uint16_t*) p;
    return (uint32_t) q[0] | (uint32_t) q[1] << 16;
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*) p; }

// the 4 bytes of a grid word negated where the nibble's bits are set: (g ^ 0xFF) + 1 per byte (no carry: g > 0)
__device__ __forceinline__ int signed4(uint32_t g, uint32_t nib) {
    const uint32_t one = (nib * 0x204081u) & 0x01010101u;  // bit i of nib -> byte i = 1
    return (int) ((g ^ (one * 0xFFu)) + one);
}
// ksigns_iq2xs: 7 sign bits plus an even-parity bit 7
__device__ __forceinline__ uint32_t ksign8(uint32_t v7) { return v7 | ((uint32_t) __builtin_popcount(v7) & 1u) << 7; }

// ------------------------------------------------------------------ unit decode
struct Unit {
    int w[8];
    float a, b;
};

template <int T> struct Fmt;
template <> struct Fmt<TSX_IQ3_XXS> { static constexpr int upb = 8, bytes = 98; };
template <> struct Fmt<TSX_IQ3_S> { static constexpr int upb = 8, bytes = 110; };
template <> struct Fmt<TSX_Q4_K> { static constexpr int upb = 8, bytes = 144; };
template <> struct Fmt<TSX_Q8_0> { static constexpr int upb = 1, bytes = 34; };

template <int T> __device__ __forceinline__ void unit_load(const uint8_t* row, int u, Unit& o);

template <> __device__ __forceinline__ void unit_load<TSX_IQ3_XXS>(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + (u >> 3) * 98;
    const int j = u & 7;
    const float d = h2f((uint16_t) ld16(blk));
    const uint32_t q0 = ld32a2(blk + 2 + 8 * j), q1 = ld32a2(blk + 6 + 8 * j);
    const uint32_t aux = ld32a2(blk + 66 + 4 * j);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t s = ksign8((aux >> (7 * l)) & 127u);
        const uint32_t q = l < 2 ? q0 : q1;
        const uint32_t i0 = (q >> (16 * (l & 1))) & 255u, i1 = (q >> (16 * (l & 1) + 8)) & 255u;
        o.w[2 * l] = signed4(kGrid.xxs[i0], s & 15u);
        o.w[2 * l + 1] = signed4(kGrid.xxs[i1], s >> 4);
    }
    o.a = d * 0.25f * (float) (2 * (int) (aux >> 28) + 1);
    o.b = 0.f;
}

template <> __device__ __forceinline__ void unit_load<TSX_IQ3_S>(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + (u >> 3) * 110;
    const int j = u & 7;
    const float d = h2f((uint16_t) ld16(blk));
    const uint32_t q0 = ld32a2(blk + 2 + 8 * j), q1 = ld32a2(blk + 6 + 8 * j);
    const uint32_t qh = blk[66 + j];
    const uint32_t sg = ld32a2(blk + 74 + 4 * j);
    const uint32_t sc = (blk[106 + (j >> 1)] >> (4 * (j & 1))) & 15u;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t q = k < 4 ? q0 : q1;
        const uint32_t idx = ((q >> (8 * (k & 3))) & 255u) | (((qh >> k) & 1u) << 8);
        o.w[k] = signed4(kGrid.s[idx], (sg >> (4 * k)) & 15u);
    }
    o.a = d * (float) (2 * (int) sc + 1);
    o.b = 0.f;
}

template <> __device__ __forceinline__ void unit_load<TSX_Q4_K>(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + (u >> 3) * 144;
    const int j = u & 7;
    const float d = h2f((uint16_t) ld16(blk)), dmin = h2f((uint16_t) ld16(blk + 2));
    const uint8_t* qs = blk + 16 + 32 * (j >> 1);
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int k = 0; k < 8; ++k) o.w[k] = (int) ((ld32a2(qs + 4 * k) >> sh) & 0x0F0F0F0Fu);
    const uint8_t* s12 = blk + 4;
    int sc, m;
    if (j < 4) {
        sc = s12[j] & 63;
        m = s12[j + 4] & 63;
    } else {
        sc = (s12[j + 4] & 15) | ((s12[j - 4] >> 6) << 4);
        m = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
    o.a = d * (float) sc;
    o.b = dmin * (float) m;
}

template <> __device__ __forceinline__ void unit_load<TSX_Q8_0>(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + u * 34;
    const float d = h2f((uint16_t) ld16(blk));
#pragma unroll
    for (int k = 0; k < 8; ++k) o.w[k] = (int) ld32a2(blk + 2 + 4 * k);
    o.a = d;
    o.b = 0.f;
}

// one Q8_1 activation block: d and the 32 codes as 8 words
struct Act {
    int q[8];
    float d;
};
__device__ __forceinline__ void act_load(const tsx_block_q8_1* x, Act& a) {
    const uint32_t* p = (const uint32_t*) x;
    a.d = h2f((uint16_t) (p[0] & 0xFFFFu));
#pragma unroll
    for (int k = 0; k < 8; ++k) a.q[k] = (int) p[1 + k];
}

// the unit's contribution to a row . activation dot product; *S (and *M) the exact integer sums
template <int T>
__device__ __forceinline__ float unit_dot(const Unit& w, const Act& x, int& S, int& M) {
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = dot4(w.w[k], x.q[k], s);
    S = s;
    if constexpr (T == TSX_Q4_K) {
        int m = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) m = dot4(0x01010101, x.q[k], m);
        M = m;
        return x.d * (w.a * (float) s - w.b * (float) m);
    } else {
        M = 0;
        return x.d * (w.a * (float) s);
    }
}

// ------------------------------------------------------------------ wave reductions
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WIDTH);
    return v;
}

// ------------------------------------------------------------------ Q8_1 of 32 values held by 32 lanes
// lane i (i = lane & 31) holds x; the 32-lane xor tree for amax and for the sum (the order the oracle restates)
__device__ __forceinline__ float q8_1_finite(float v) { return fabsf(v) > 65504.0f ? copysignf(65504.0f, v) : v; }
__device__ __forceinline__ void q8_1_store32(float x, tsx_block_q8_1* y, int i) {
    float amax = fabsf(x), sum = x;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, 32));
        sum += __shfl_xor(sum, o, 32);
    }
    const float d = q8_1_finite(amax / 127.0f);
    int8_t q = 0;
    if (amax != 0.0f) {
        const float r = roundf(x / d);
        q = (int8_t) (r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r);
    }
    y->qs[i] = q;
    if (i == 0) {
        y->d = f2h(q8_1_finite(d));
        y->s = f2h(q8_1_finite(sum));
    }
}

}  // namespace tsx
