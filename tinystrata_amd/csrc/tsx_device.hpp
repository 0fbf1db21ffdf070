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

#include <cfloat>
#include <cstdint>

#include "tsx_moe.h"

namespace tsx {

constexpr int kWave = 64;

// 16 bytes as one vector: what the 128-bit global and LDS loads move
typedef int v4i __attribute__((ext_vector_type(4)));
// a pointer into LDS: accesses through it are ds_read / ds_write even where the compiler cannot tell a generic
// pointer's target (a flat access counts against vmcnt and waits behind the wave's global loads)
template <typename T> using lds_ptr = __attribute__((address_space(3))) T*;
// a pointer into global memory, for addresses computed through integers: loads through it are global_load, not flat
// (a flat load also counts against lgkmcnt, so every later LDS wait would wait for it)
template <typename T> using gbl_ptr = __attribute__((address_space(1))) T*;
template <typename T> __device__ __forceinline__ gbl_ptr<const T> gbl_at(uintptr_t a) { return (gbl_ptr<const T>) a; }

// ------------------------------------------------------------------ codebooks and sign tables, built at compile time
// A sign entry turns 8 signs into what negates the matching bytes of two grid words: w = (g ^ mask) + (mask & 0x01..),
// with mask = 0xFF in every negated byte (no carry crosses a byte: every grid byte is > 0).
// xxs_sign is indexed by IQ3_XXS's 7-bit sign field (the 8th sign is the parity of the 7: ksigns_iq2xs),
// s_sign by IQ3_S's sign byte.  Entry = {mask of values 0-3, mask of values 4-7}.
struct SignEntry {
    uint32_t mask_lo, mask_hi;
};
__device__ __forceinline__ uint32_t apply_signs(uint32_t g, uint32_t mask) { return (g ^ mask) + (mask & 0x01010101u); }
struct GridTables {
    uint32_t xxs[256];
    uint32_t s[512];
    SignEntry xxs_sign[128];
    SignEntry s_sign[256];
};
constexpr uint32_t spread_nibble(uint32_t nib) {  // bit i -> byte i = 1
    return (nib & 1u) | (nib & 2u) << 7 | (nib & 4u) << 14 | (nib & 8u) << 21;
}
constexpr SignEntry sign_entry(uint32_t s8) {
    const uint32_t lo = spread_nibble(s8 & 15u), hi = spread_nibble(s8 >> 4);
    return SignEntry{lo * 0xFFu, hi * 0xFFu};
}
constexpr uint32_t parity7(uint32_t v) {
    uint32_t p = 0;
    for (int b = 0; b < 7; ++b) p ^= (v >> b) & 1u;
    return p;
}
constexpr GridTables make_grid_tables() {
    GridTables g{};
    for (int i = 0; i < 256; ++i) g.xxs[i] = tsx_iq3xxs_word(i);
    for (int i = 0; i < 512; ++i) g.s[i] = tsx_iq3s_word(i);
    for (uint32_t v = 0; v < 128; ++v) g.xxs_sign[v] = sign_entry(v | parity7(v) << 7);
    for (uint32_t b = 0; b < 256; ++b) g.s_sign[b] = sign_entry(b);
    return g;
}
static __constant__ const GridTables kGrid = make_grid_tables();

// where a kernel reads the tables from: the constant tables, or a copy in LDS
struct GridRef {
    const uint32_t* xxs;
    const uint32_t* s;
    const SignEntry* xxs_sign;
    const SignEntry* s_sign;
};
__device__ __forceinline__ GridRef grid_const() { return GridRef{kGrid.xxs, kGrid.s, kGrid.xxs_sign, kGrid.s_sign}; }
// Bank-private copies of T's tables in LDS.  Lanes of a wave pick codebook entries at random, so one shared copy
// makes them collide in the LDS banks (several passes per read); with R copies of each entry, entry i's copy for
// lane l at slot i * R + l % R, lanes l and l' < R apart always read different banks.  The sign entries of IQ3_S
// are copied fewer times so that both tables, the weight slab and the activations fit one block's LDS.
template <int T> constexpr int rep_grid_copies() { return T == TSX_IQ3_XXS ? 32 : T == TSX_IQ3_S ? 16 : 0; }
template <int T> constexpr int rep_sign_copies() { return T == TSX_IQ3_XXS ? 32 : T == TSX_IQ3_S ? 16 : 0; }
template <int T> constexpr int rep_grid_entries() { return T == TSX_IQ3_XXS ? 256 : T == TSX_IQ3_S ? 512 : 0; }
template <int T> constexpr int rep_sign_entries() { return T == TSX_IQ3_XXS ? 128 : T == TSX_IQ3_S ? 256 : 0; }
template <int T> constexpr int rep_grid_bytes() { return rep_grid_entries<T>() * rep_grid_copies<T>() * 4; }
// LDS bytes of the copies (0 for formats without a codebook); a multiple of 16
template <int T> constexpr int rep_lds_bytes() { return rep_grid_bytes<T>() + rep_sign_entries<T>() * rep_sign_copies<T>() * 8; }
// the 16-byte stores that fill the copies: four copies of a grid word, or two of a sign entry, each
template <int T> constexpr int rep_stores() {
    return rep_grid_entries<T>() * rep_grid_copies<T>() / 4 + rep_sign_entries<T>() * rep_sign_copies<T>() / 2;
}
// what a lane reads the copies through: its own slot of every entry
template <int T>
struct RepTab {
    const uint32_t* grid;
    const uint64_t* sign;
};
// the values this thread stores (store q = tid + n * k), requested from the constant tables: issue early, store
// later with rep_store.  PER >= rep_stores<T>() / n.
template <int T, int PER>
__device__ __forceinline__ void rep_fetch(uint64_t (&v)[PER], int tid, int n) {
    constexpr int NG = rep_grid_entries<T>() * rep_grid_copies<T>() / 4, NS = rep_stores<T>() - NG;
    const uint32_t* g = T == TSX_IQ3_XXS ? kGrid.xxs : kGrid.s;
    const uint64_t* sg = (const uint64_t*) (T == TSX_IQ3_XXS ? kGrid.xxs_sign : kGrid.s_sign);
#pragma unroll
    for (int k = 0; k < PER; ++k) {  // unconditional (clamped) loads keep the wait counts exact
        const int q = min(tid + n * k, NG + NS - 1);
        v[k] = q < NG ? (uint64_t) g[q * 4 / rep_grid_copies<T>()] : sg[(q - NG) * 2 / rep_sign_copies<T>()];
    }
}
template <int T, int PER>
__device__ __forceinline__ RepTab<T> rep_store(uint8_t* lds, const uint64_t (&v)[PER], int tid, int n) {
    constexpr int NG = rep_grid_entries<T>() * rep_grid_copies<T>() / 4, NS = rep_stores<T>() - NG;
    const lds_ptr<v4i> dst = (lds_ptr<v4i>) lds;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int q = tid + n * k;
        const int lo = (int) (uint32_t) v[k], hi = (int) (uint32_t) (v[k] >> 32);
        if (q < NG) dst[q] = v4i{lo, lo, lo, lo};
        else if (q < NG + NS) dst[q] = v4i{lo, hi, lo, hi};
    }
    const int lane = __lane_id();
    return RepTab<T>{(const uint32_t*) lds + lane % max(rep_grid_copies<T>(), 1),
                     (const uint64_t*) (lds + rep_grid_bytes<T>()) + lane % max(rep_sign_copies<T>(), 1)};
}

// a lane's view of copies stored earlier by rep_store (by whichever threads stored them)
template <int T>
__device__ __forceinline__ RepTab<T> rep_view(const uint8_t* lds) {
    const int lane = __lane_id();
    return RepTab<T>{(const uint32_t*) lds + lane % max(rep_grid_copies<T>(), 1),
                     (const uint64_t*) (lds + rep_grid_bytes<T>()) + lane % max(rep_sign_copies<T>(), 1)};
}
// table reads, by where the tables are: the constant tables (GridRef) or a lane's copies (RepTab)
template <int T> __device__ __forceinline__ uint32_t tab_grid(const GridRef& g, uint32_t i) {
    return T == TSX_IQ3_XXS ? g.xxs[i] : g.s[i];
}
template <int T> __device__ __forceinline__ SignEntry tab_sign(const GridRef& g, uint32_t i) {
    return T == TSX_IQ3_XXS ? g.xxs_sign[i] : g.s_sign[i];
}
template <int T> __device__ __forceinline__ uint32_t tab_grid(const RepTab<T>& r, uint32_t i) {
    return r.grid[i * rep_grid_copies<T>()];
}
template <int T> __device__ __forceinline__ SignEntry tab_sign(const RepTab<T>& r, uint32_t i) {
    const uint64_t v = r.sign[i * rep_sign_copies<T>()];
    return SignEntry{(uint32_t) v, (uint32_t) (v >> 32)};
}

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


// ------------------------------------------------------------------ unit decode
struct Unit {
    int w[8];
    float a, b;
    int k0, k1;  // Q6_K: the integer scales of the unit's two 16-value halves
};

template <int T> struct Fmt;
template <> struct Fmt<TSX_IQ3_XXS> { static constexpr int upb = 8, bytes = 98; };
template <> struct Fmt<TSX_IQ3_S> { static constexpr int upb = 8, bytes = 110; };
template <> struct Fmt<TSX_Q4_K> { static constexpr int upb = 8, bytes = 144; };
template <> struct Fmt<TSX_Q8_0> { static constexpr int upb = 1, bytes = 34; };
template <> struct Fmt<TSX_Q4_0> { static constexpr int upb = 1, bytes = 18; };
template <> struct Fmt<TSX_Q6_K> { static constexpr int upb = 8, bytes = 210; };


template <typename Tab>
__device__ __forceinline__ void unit_load_iq3xxs(const uint8_t* row, int u, Unit& o, const Tab& g) {
    const uint8_t* blk = row + (u >> 3) * 98;
    const int j = u & 7;
    const float d = h2f((uint16_t) ld16(blk));
    const uint32_t q0 = ld32a2(blk + 2 + 8 * j), q1 = ld32a2(blk + 6 + 8 * j);
    const uint32_t aux = ld32a2(blk + 66 + 4 * j);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const SignEntry sg = tab_sign<TSX_IQ3_XXS>(g, (aux >> (7 * l)) & 127u);
        const uint32_t q = l < 2 ? q0 : q1;
        const uint32_t i0 = (q >> (16 * (l & 1))) & 255u, i1 = (q >> (16 * (l & 1) + 8)) & 255u;
        o.w[2 * l] = (int) apply_signs(tab_grid<TSX_IQ3_XXS>(g, i0), sg.mask_lo);
        o.w[2 * l + 1] = (int) apply_signs(tab_grid<TSX_IQ3_XXS>(g, i1), sg.mask_hi);
    }
    o.a = d * 0.25f * (float) (2 * (int) (aux >> 28) + 1);
    o.b = 0.f;
}

template <typename Tab>
__device__ __forceinline__ void unit_load_iq3s(const uint8_t* row, int u, Unit& o, const Tab& g) {
    const uint8_t* blk = row + (u >> 3) * 110;
    const int j = u & 7;
    const float d = h2f((uint16_t) ld16(blk));
    const uint32_t q0 = ld32a2(blk + 2 + 8 * j), q1 = ld32a2(blk + 6 + 8 * j);
    const uint32_t qh = blk[66 + j];
    const uint32_t sb = ld32a2(blk + 74 + 4 * j);
    const uint32_t sc = (blk[106 + (j >> 1)] >> (4 * (j & 1))) & 15u;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const SignEntry sg = tab_sign<TSX_IQ3_S>(g, (sb >> (8 * l)) & 255u);
        const uint32_t q = l < 2 ? q0 : q1;
        const int k0 = 2 * l, k1 = 2 * l + 1;
        const uint32_t i0 = ((q >> (8 * (k0 & 3))) & 255u) | (((qh >> k0) & 1u) << 8);
        const uint32_t i1 = ((q >> (8 * (k1 & 3))) & 255u) | (((qh >> k1) & 1u) << 8);
        o.w[k0] = (int) apply_signs(tab_grid<TSX_IQ3_S>(g, i0), sg.mask_lo);
        o.w[k1] = (int) apply_signs(tab_grid<TSX_IQ3_S>(g, i1), sg.mask_hi);
    }
    o.a = d * (float) (2 * (int) sc + 1);
    o.b = 0.f;
}

__device__ __forceinline__ void unit_load_q4k(const uint8_t* row, int u, Unit& o) {
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

__device__ __forceinline__ void unit_load_q80(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + u * 34;
    const float d = h2f((uint16_t) ld16(blk));
#pragma unroll
    for (int k = 0; k < 8; ++k) o.w[k] = (int) ld32a2(blk + 2 + 4 * k);
    o.a = d;
    o.b = 0.f;
}

// Q4_0: the 4-bit codes as they are (0..15); the -8 offset is applied with the activation block's sum
__device__ __forceinline__ void unit_load_q40(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + u * 18;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t q = ld32a2(blk + 2 + 4 * k);
        o.w[k] = (int) (q & 0x0F0F0F0Fu);              // values 4k .. 4k + 3
        o.w[4 + k] = (int) ((q >> 4) & 0x0F0F0F0Fu);   // values 16 + 4k ..
    }
    o.a = h2f((uint16_t) ld16(blk));
    o.b = 0.f;
}

// Q6_K unit u = half u / 4, quarter u % 4 of the block: value l (0..31) of the quarter is the low (quarters 0, 1)
// or high (2, 3) nibble of ql[64 half + 32 (quarter % 2) + l] with bits 2 quarter .. 2 quarter + 1 of
// qh[32 half + l] above it, minus 32; the scale of values 0-15 is scales[8 half + 2 quarter], of 16-31 the next.
// The codes stay unsigned (0..63): the -32 is applied with each half's activation sum
__device__ __forceinline__ void unit_load_q6k(const uint8_t* row, int u, Unit& o) {
    const uint8_t* blk = row + (u >> 3) * 210;
    const int j = u & 7, half = j >> 2, qt = j & 3;
    const uint8_t* ql = blk + 64 * half + 32 * (qt & 1);
    const uint8_t* qh = blk + 128 + 32 * half;
    const int lsh = 4 * (qt >> 1), hsh = 2 * qt;
#pragma unroll
    for (int k = 0; k < 8; ++k)
        o.w[k] = (int) (((ld32a2(ql + 4 * k) >> lsh) & 0x0F0F0F0Fu) | (((ld32a2(qh + 4 * k) >> hsh) & 0x03030303u) << 4));
    const int8_t* sc = (const int8_t*) (blk + 192 + 8 * half + 2 * qt);
    o.k0 = sc[0];
    o.k1 = sc[1];
    o.a = h2f((uint16_t) ld16(blk + 208));
    o.b = 0.f;
}

// unit u of a row of format T; g: where the codebooks are read (GridRef or RepTab<T>)
template <int T, typename Tab>
__device__ __forceinline__ void unit_load(const uint8_t* row, int u, Unit& o, const Tab& g) {
    if constexpr (T == TSX_IQ3_XXS) unit_load_iq3xxs(row, u, o, g);
    else if constexpr (T == TSX_IQ3_S) unit_load_iq3s(row, u, o, g);
    else if constexpr (T == TSX_Q4_K) unit_load_q4k(row, u, o);
    else if constexpr (T == TSX_Q4_0) unit_load_q40(row, u, o);
    else if constexpr (T == TSX_Q6_K) unit_load_q6k(row, u, o);
    else unit_load_q80(row, u, o);
}

// one Q8_1 activation block: d, the sum field s and the 32 codes as 8 words
struct Act {
    int q[8];
    float d, s;
};
__device__ __forceinline__ void act_load(const tsx_block_q8_1* x, Act& a) {
    const uint32_t* p = (const uint32_t*) x;
    a.d = h2f((uint16_t) (p[0] & 0xFFFFu));
    a.s = h2f((uint16_t) (p[0] >> 16));
#pragma unroll
    for (int k = 0; k < 8; ++k) a.q[k] = (int) p[1 + k];
}

// the unit's contribution to a row . activation dot product; *S (and *M) the exact integer sums
template <int T>
__device__ __forceinline__ float unit_dot(const Unit& w, const Act& x, int& S, int& M) {
    if constexpr (T == TSX_Q6_K) {
        // S = k0 * sum over values 0-15 of (code - 32) * a + k1 * the same over 16-31, exact in int32
        int s0 = 0, s1 = 0, m0 = 0, m1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s0 = dot4(w.w[k], x.q[k], s0);
            s1 = dot4(w.w[4 + k], x.q[4 + k], s1);
            m0 = dot4(0x01010101, x.q[k], m0);
            m1 = dot4(0x01010101, x.q[4 + k], m1);
        }
        S = w.k0 * (s0 - 32 * m0) + w.k1 * (s1 - 32 * m1);
        M = m0 + m1;
        return x.d * (w.a * (float) S);
    }
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = dot4(w.w[k], x.q[k], s);
    S = s;
    if constexpr (T == TSX_Q4_0) {
        // the reference's affine form: d_w (S d_x - 8 s_x) with the activation block's sum field s_x
        M = 0;
        return w.a * ((float) s * x.d - 8.0f * x.s);
    } else if constexpr (T == TSX_Q4_K) {
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

// ------------------------------------------------------------------ DPP reductions (no LDS round trips)
// Four DPP steps reduce each 16-lane row (xor 1, xor 2, then the half-row and row mirrors); the row totals are then
// combined from lanes 15, 31, 47 and 63 with readlane.  Every lane of the span ends with the same bits (each DPP step
// combines a value with its partner symmetrically, and the last step hands every lane one scalar).  For spans of 32
// or 64 lanes all 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_of(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
template <typename Op>
__device__ __forceinline__ float row_reduce16(float v, Op op) {
    v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));  // row_mirror
    return v;
}
// over each half wave (lanes 0-31, 32-63)
template <typename Op>
__device__ __forceinline__ float reduce32(float v, Op op) {
    v = row_reduce16(v, op);
    const float lo = op(lane_of(v, 15), lane_of(v, 31)), hi = op(lane_of(v, 47), lane_of(v, 63));
    return (__lane_id() < 32) ? lo : hi;
}
// over the wave
template <typename Op>
__device__ __forceinline__ float reduce64(float v, Op op) {
    v = row_reduce16(v, op);
    return op(op(lane_of(v, 15), lane_of(v, 31)), op(lane_of(v, 47), lane_of(v, 63)));
}
struct OpAddF {
    __device__ float operator()(float a, float b) const { return a + b; }
};
// op over aligned groups of W consecutive lanes (W = 2, 4, 8, 16, 32 or 64), every lane of a group ending with the
// result
template <int W, typename Op>
__device__ __forceinline__ float lanes_reduce(float v, Op op) {
    static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "lanes_reduce width");
    if constexpr (W == 32) {
        return reduce32(v, op);
    } else if constexpr (W == 64) {
        return reduce64(v, op);
    } else {
        v = op(v, dpp_mov<0xB1>(v));
        if constexpr (W >= 4) v = op(v, dpp_mov<0x4E>(v));
        if constexpr (W >= 8) v = op(v, dpp_mov<0x141>(v));
        if constexpr (W >= 16) v = op(v, dpp_mov<0x140>(v));
        return v;
    }
}
template <int W>
__device__ __forceinline__ float lanes_sum(float v) {
    return lanes_reduce<W>(v, OpAddF());
}

// ------------------------------------------------------------------ wave argmax on (value, id) keys
// A float's order as an unsigned word (larger float -> larger word; -inf below -FLT_MAX below every probability).
__device__ __forceinline__ uint32_t ord_key(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// (hi, lo) is the larger 64-bit key of the pair: hi = ord_key(value), lo = ~id (ties go to the lower id)
__device__ __forceinline__ void key_max(uint32_t& hi, uint32_t& lo, uint32_t oh, uint32_t ol) {
    const bool take = oh > hi || (oh == hi && ol > lo);
    hi = take ? oh : hi;
    lo = take ? ol : lo;
}
template <int CTRL>
__device__ __forceinline__ void key_step(uint32_t& hi, uint32_t& lo) {
    const uint32_t oh = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) hi, CTRL, 0xF, 0xF, false);
    const uint32_t ol = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) lo, CTRL, 0xF, 0xF, false);
    key_max(hi, lo, oh, ol);
}
// the wave's largest key, the same in every lane (all 64 lanes active)
__device__ __forceinline__ void wave_key_max(uint32_t& hi, uint32_t& lo) {
    key_step<0xB1>(hi, lo);
    key_step<0x4E>(hi, lo);
    key_step<0x141>(hi, lo);
    key_step<0x140>(hi, lo);
    uint32_t h = (uint32_t) __builtin_amdgcn_readlane((int) hi, 15), l = (uint32_t) __builtin_amdgcn_readlane((int) lo, 15);
    key_max(h, l, (uint32_t) __builtin_amdgcn_readlane((int) hi, 31), (uint32_t) __builtin_amdgcn_readlane((int) lo, 31));
    key_max(h, l, (uint32_t) __builtin_amdgcn_readlane((int) hi, 47), (uint32_t) __builtin_amdgcn_readlane((int) lo, 47));
    key_max(h, l, (uint32_t) __builtin_amdgcn_readlane((int) hi, 63), (uint32_t) __builtin_amdgcn_readlane((int) lo, 63));
    hi = h;
    lo = l;
}

struct OpMax {
    __device__ float operator()(float a, float b) const { return __builtin_fmaxf(a, b); }
};
struct OpAdd {
    __device__ float operator()(float a, float b) const { return a + b; }
};

// ------------------------------------------------------------------ Q8_1 of 32 values held by 32 lanes
// lane i (i = lane & 31) holds x; the 32-lane xor tree for amax and for the sum (the order the oracle restates)
__device__ __forceinline__ float q8_1_finite(float v) { return fabsf(v) > 65504.0f ? copysignf(65504.0f, v) : v; }
// The Q8_1 code of v in a block of scale d = q8_1_finite(amax / 127) (amax the block's largest magnitude):
// roundf(v / d) clamped to [-127, 127], 0 when amax is 0 - the reference quantizer's code, bit for bit.  rd = 1 / d is
// the correctly rounded reciprocal (q8_1_rcp, once per block); the quotient is Markstein's corrected product
// q = v rd, r = v - d q (exact by fma), q + r rd, which is the correctly rounded v / d when rd is and nothing under- or
// overflows (d >= 2^-100; a smaller d takes the division).  roundf ties away from zero; the clamp is one v_med3.
// d = q8_1_finite(amax / 127) without a division: Markstein's corrected product with the correctly rounded
// reciprocal of 127, which equals the IEEE quotient for every non-negative finite float (checked exhaustively)
__device__ __forceinline__ float q8_1_scale(float amax) {
    constexpr float R = 1.0f / 127.0f;
    const float q0 = amax * R;
    return q8_1_finite(__builtin_fmaf(__builtin_fmaf(-127.0f, q0, amax), R, q0));
}
// 1 / d correctly rounded, for q8_1_code_rd: in [2^-100, 2^100] the hardware reciprocal and one fma Newton step,
// which equal the IEEE quotient for every float of that range (checked exhaustively on gfx950); elsewhere (q8_1_code_rd
// divides there instead) the IEEE quotient
__device__ __forceinline__ float q8_1_rcp(float d) {
    if (d >= 0x1p-100f && d <= 0x1p100f) {
        const float r0 = __builtin_amdgcn_rcpf(d);
        return __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
    }
    return 1.0f / d;
}
__device__ __forceinline__ int q8_1_round_clamp(float z) {  // roundf (ties away from zero), clamped to [-127, 127]
    const float t = __builtin_truncf(z);
    const float r = t + (__builtin_fabsf(z - t) >= 0.5f ? __builtin_copysignf(1.0f, z) : 0.0f);
    return (int) __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
}
__device__ __forceinline__ int q8_1_code_rd(float v, float amax, float d, float rd) {
    if (amax == 0.0f) return 0;
    float z;
    if (d >= 0x1p-100f) {
        const float q = v * rd;
        z = __builtin_fmaf(__builtin_fmaf(-d, q, v), rd, q);
    } else {
        z = v / d;
    }
    return q8_1_round_clamp(z);
}
// q8_1_code_rd's four codes of one lane's quad (block scale d of block amax), with one wave-uniform branch: when every
// block of the wave with a nonzero amax has d in [2^-100, 2^100] (where q8_1_rcp is the corrected reciprocal), the
// corrected products run straight through for every lane (a zero block's codes are 0: its reciprocal is never used);
// otherwise each value takes q8_1_code_rd.  Call with every lane of the wave.
__device__ __forceinline__ void q8_1_codes4(const float4& x, float amax, float d, int (&q)[4]) {
    const float v[4] = {x.x, x.y, x.z, x.w};
    if (__builtin_amdgcn_ballot_w64(amax != 0.0f && !(d >= 0x1p-100f && d <= 0x1p100f)) == 0) {
        const float r0 = __builtin_amdgcn_rcpf(d);
        const float rd = __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float p = v[k] * rd;
            const int c = q8_1_round_clamp(__builtin_fmaf(__builtin_fmaf(-d, p, v[k]), rd, p));
            q[k] = amax == 0.0f ? 0 : c;
        }
    } else {
        const float rd = q8_1_rcp(d);
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = q8_1_code_rd(v[k], amax, d, rd);
    }
}
__device__ __forceinline__ void q8_1_store32(float x, tsx_block_q8_1* y, int i) {
    float amax = fabsf(x), sum = x;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, 32));
        sum += __shfl_xor(sum, o, 32);
    }
    const float d = q8_1_scale(amax);
    y->qs[i] = (int8_t) q8_1_code_rd(x, amax, d, q8_1_rcp(d));
    if (i == 0) {
        y->d = f2h(q8_1_finite(d));
        y->s = f2h(q8_1_finite(sum));
    }
}


// The MoE block's norm of one row held in LDS (s_row[0..n), written by the calling threads, each of which passes the
// sum of the squares of the values it wrote, in its own order): the sums over each wave, then over the waves in
// order, give r = 1 / sqrt(sum / n + eps); h[i] = (row[i] * r) * w[i] (two roundings) and, when hq is not null, h's
// Q8_1 image, 32 consecutive lanes per block (n a multiple of 32).  All NT threads of the block take part.
template <int NT>
__device__ __forceinline__ void norm_row_out(const float* s_row, float q, int n, const float* __restrict__ w, float eps,
                                             float* __restrict__ h, tsx_block_q8_1* __restrict__ hq, float* s_red) {
#pragma clang fp contract(off)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = q;
    __syncthreads();
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) sum += s_red[k];
    const float r = rsqrtf(sum / (float) n + eps);
    for (int i = threadIdx.x; i < n; i += NT) {
        const float hv = s_row[i] * r * w[i];
        h[i] = hv;
        if (hq) q8_1_store32(hv, hq + i / 32, i & 31);
    }
}

// the wave's largest (smallest) 32-bit unsigned value, the same in every lane (all 64 lanes active): four DPP steps
// within each 16-lane row, two row broadcasts (lane 15 of rows 0 and 2 into rows 1 and 3, then lane 31 into rows 2
// and 3), and lane 63 read out.  Lanes a step does not write keep `old`, the operation's identity.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t old = 0u) {
    return (uint32_t) __builtin_amdgcn_update_dpp((int) old, (int) v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));        // quad_perm [1,0,3,2]
    v = max(v, dpp_u32<0x4E>(v));        // quad_perm [2,3,0,1]
    v = max(v, dpp_u32<0x141>(v));       // row_half_mirror
    v = max(v, dpp_u32<0x140>(v));       // row_mirror
    v = max(v, dpp_u32<0x142, 0xA>(v));  // row_bcast:15
    v = max(v, dpp_u32<0x143, 0xC>(v));  // row_bcast:31
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    constexpr uint32_t id = 0xFFFFFFFFu;
    v = min(v, dpp_u32<0xB1>(v, id));
    v = min(v, dpp_u32<0x4E>(v, id));
    v = min(v, dpp_u32<0x141>(v, id));
    v = min(v, dpp_u32<0x140>(v, id));
    v = min(v, dpp_u32<0x142, 0xA>(v, id));
    v = min(v, dpp_u32<0x143, 0xC>(v, id));
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}

// ------------------------------------------------------------------ routing of one token by one wave
// Reference route_topk<NE,K> (src/kernels/cuda/native_router.cu:42-95): softmax with the max subtracted and one
// reciprocal of the sum, NaN probabilities as -FLT_MAX, k rounds of argmax (ties to the lower id), weights divided by
// max(sum of the picks, 6.1035e-5).  Expert e = lane + 64 i; n_expert a multiple of 64 up to kMaxExperts (V = n_expert
// / 64 columns, a template argument).  Each lane sorts its V keys; each round takes the wave's largest head (a DPP
// reduction), then the lowest id holding it (from the one lane holding it, or a second reduction when heads are equal),
// and the winning lane pops its head.
// ids / wts may point to global memory or LDS; every lane of the wave must call.  route_fetch and route_select split
// the routing so that a kernel can request the logits before anything else and wait for them alone.
constexpr int kMaxExperts = 512;
constexpr int kRouteV = kMaxExperts / 64;  // logits per lane
__device__ __forceinline__ void route_fetch(const float* __restrict__ l, int n_expert, int lane, float (&v)[kRouteV]) {
#pragma unroll
    for (int i = 0; i < kRouteV; ++i)  // unconditional (clamped) loads keep the wait counts exact
        v[i] = l[min(lane + 64 * i, n_expert - 1)];
}
// the softmax probabilities' order keys (NaN as -FLT_MAX) of the lane's V experts, sorted largest first with their
// ids (a stable network: equal keys keep the lower id first)
template <int V>
__device__ __forceinline__ void route_prep_v(const float (&lv)[kRouteV], int lane, uint32_t (&key)[V], uint32_t (&id)[V]) {
    float v[V];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        v[i] = lv[i];
        mx = __builtin_fmaxf(mx, v[i]);
    }
    mx = reduce64(mx, OpMax());
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    const float rcp = 1.0f / reduce64(sum, OpAddF());
#pragma unroll
    for (int i = 0; i < V; ++i) {
        float p = v[i] * rcp;
        if (__builtin_isnan(p)) p = -FLT_MAX;
        key[i] = ord_key(p);
    }
#pragma unroll
    for (int i = 0; i < V; ++i) id[i] = (uint32_t) (64 * i + lane);
#pragma unroll
    for (int i = 1; i < V; ++i)
#pragma unroll
        for (int j = i; j > 0; --j) {
            const bool sw = key[j] > key[j - 1];
            const uint32_t k0 = key[j - 1], k1 = key[j], i0 = id[j - 1], i1 = id[j];
            key[j - 1] = sw ? k1 : k0;
            key[j] = sw ? k0 : k1;
            id[j - 1] = sw ? i1 : i0;
            id[j] = sw ? i0 : i1;
        }
}
template <int V>
__device__ __forceinline__ void route_select_v(const float (&lv)[kRouteV], int k, int lane, int32_t* ids, float* wts) {
    // k rounds: the wave's largest head each, whose lane pops it
    uint32_t key[V], id[V];
    route_prep_v<V>(lv, lane, key, id);
    float sel_sum = 0.f, my_p = 0.f;
    int my_id = 0;
    for (int r = 0; r < k; ++r) {
        // the wave's largest head, then the lowest id holding it: read from the one lane holding it, or (equal heads
        // in several lanes) the smallest of their ids
        const uint32_t wm = wave_max_u32(key[0]);
        const uint64_t hit = __ballot(key[0] == wm);
        int x = __builtin_amdgcn_readlane((int) id[0], (int) __builtin_ctzll(hit));
        if (__builtin_expect(__builtin_popcountll(hit) != 1, 0))
            x = (int) wave_min_u32(key[0] == wm ? id[0] : 0xFFFFFFFFu);
        const bool win = lane == (x & 63);
#pragma unroll
        for (int i = 0; i + 1 < V; ++i) {
            key[i] = win ? key[i + 1] : key[i];
            id[i] = win ? id[i + 1] : id[i];
        }
        key[V - 1] = win ? 0u : key[V - 1];  // below every other key
        const float p = key_value(wm);
        sel_sum += p;
        if (lane == r) {
            my_id = x;
            my_p = p;
        }
    }
    const float inv = 1.0f / __builtin_fmaxf(sel_sum, 6.103515625e-5f);
    if (lane < k) {
        ids[lane] = my_id;
        wts[lane] = my_p * inv;
    }
}
// route_select_v's rounds with each pick published as it is found: the wave stores pick r + 1 into pub[r] (LDS words
// that start at 0, so a reader polls for a nonzero word) with a relaxed workgroup-scope atomic store, which is a plain
// ds_write (a volatile store through a generic pointer became a system-coherent flat store and a wait for it, a memory
// round trip in every round), and after round 0 the whole wave calls after0().  ids / wts as route_select_v, written
// at the end.
template <int V, typename After0>
__device__ __forceinline__ void route_publish_v(const float (&lv)[kRouteV], int k, int lane, int32_t* pub,
                                                int32_t* ids, float* wts, After0 after0) {
    uint32_t key[V], id[V];
    route_prep_v<V>(lv, lane, key, id);
    float sel_sum = 0.f, my_p = 0.f;
    int my_id = 0;
    for (int r = 0; r < k; ++r) {
        const uint32_t wm = wave_max_u32(key[0]);
        const uint64_t hit = __ballot(key[0] == wm);
        // the one lane holding it (the common case, no branch taken), or, equal heads in several lanes, the smallest
        // of their ids
        int x = __builtin_amdgcn_readlane((int) id[0], (int) __builtin_ctzll(hit));
        if (__builtin_expect(__builtin_popcountll(hit) != 1, 0))
            x = (int) wave_min_u32(key[0] == wm ? id[0] : 0xFFFFFFFFu);
        // every lane stores the same word: no exec-mask branch in the round (stamps: the eight rounds 0.3 us sooner)
        __hip_atomic_store(pub + r, x + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const bool win = lane == (x & 63);
#pragma unroll
        for (int i = 0; i + 1 < V; ++i) {
            key[i] = win ? key[i + 1] : key[i];
            id[i] = win ? id[i + 1] : id[i];
        }
        key[V - 1] = win ? 0u : key[V - 1];
        const float p = key_value(wm);
        sel_sum += p;
        if (lane == r) {
            my_id = x;
            my_p = p;
        }
        if (r == 0) after0();
    }
    const float inv = 1.0f / __builtin_fmaxf(sel_sum, 6.103515625e-5f);
    if (lane < k) {
        ids[lane] = my_id;
        wts[lane] = my_p * inv;
    }
}
template <typename After0>
__device__ __forceinline__ void route_publish(const float (&v)[kRouteV], int n_expert, int k, int lane, int32_t* pub,
                                              int32_t* ids, float* wts, After0 after0) {
    switch (n_expert / 64) {
        case 1: route_publish_v<1>(v, k, lane, pub, ids, wts, after0); break;
        case 2: route_publish_v<2>(v, k, lane, pub, ids, wts, after0); break;
        case 3: route_publish_v<3>(v, k, lane, pub, ids, wts, after0); break;
        case 4: route_publish_v<4>(v, k, lane, pub, ids, wts, after0); break;
        case 5: route_publish_v<5>(v, k, lane, pub, ids, wts, after0); break;
        case 6: route_publish_v<6>(v, k, lane, pub, ids, wts, after0); break;
        case 7: route_publish_v<7>(v, k, lane, pub, ids, wts, after0); break;
        default: route_publish_v<8>(v, k, lane, pub, ids, wts, after0); break;
    }
}
__device__ __forceinline__ void route_select(const float (&v)[kRouteV], int n_expert, int k, int lane, int32_t* ids,
                                             float* wts) {
    switch (n_expert / 64) {
        case 1: route_select_v<1>(v, k, lane, ids, wts); break;
        case 2: route_select_v<2>(v, k, lane, ids, wts); break;
        case 3: route_select_v<3>(v, k, lane, ids, wts); break;
        case 4: route_select_v<4>(v, k, lane, ids, wts); break;
        case 5: route_select_v<5>(v, k, lane, ids, wts); break;
        case 6: route_select_v<6>(v, k, lane, ids, wts); break;
        case 7: route_select_v<7>(v, k, lane, ids, wts); break;
        default: route_select_v<8>(v, k, lane, ids, wts); break;
    }
}
__device__ __forceinline__ void route_token(const float* __restrict__ l, int n_expert, int k, int lane, int32_t* ids,
                                            float* wts) {
    float v[kRouteV];
    route_fetch(l, n_expert, lane, v);
    route_select(v, n_expert, k, lane, ids, wts);
}

}  // namespace tsx
