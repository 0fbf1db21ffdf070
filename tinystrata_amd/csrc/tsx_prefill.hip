// tsx_prefill.hip - the prompt path's grouped expert products on gfx950 (the reference's prefill::mmq).
//
// Reference: mmq::quantize / Context::run / swiglu (src/prefill/moe_mmq.cu:123-131, 309-384), the call sequence of
// src/qwen35/q36_engine.cu:2855-2885.  The reference hands the products to ggml's MMQ kernels (not vendored); this
// file has its own.
//
// Activation layout (library-private, sized by tsx_moe_mmq_q8_bytes): three planes for rows padded to kRowPad,
//   q [rows_pad][cols] int8   the Q8_1 codes, row-major (16-byte aligned rows: cols is a multiple of 32)
//   d [rows_pad][cols/32] f32 the block scale, the fp16 value of the Q8_1 contract widened to float
//   m [rows_pad][cols/32] i32 the sum of the block's codes (Q4_K's min term)
// so a tile of tokens loads its codes with 16-byte loads and its scales without fp16 conversions.
#include <type_traits>

#include "tsx_common.hpp"
#include "tsx_device.hpp"

namespace tsx {
namespace {

constexpr int kRowPad = 64;
constexpr int kThreads = 256;

struct MmqPlanes {
    int8_t* q;
    float* d;
    int32_t* m;
    int64_t rows_pad, cols;
};
__host__ __device__ inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t) 255; }
__host__ __device__ inline int64_t pad_rows(int64_t rows) { return (rows + kRowPad - 1) / kRowPad * kRowPad + kRowPad; }
__host__ __device__ inline MmqPlanes planes(void* base, int64_t rows, int64_t cols) {
    MmqPlanes p;
    p.rows_pad = pad_rows(rows);
    p.cols = cols;
    uint8_t* b = (uint8_t*) base;
    p.q = (int8_t*) b;
    p.d = (float*) (b + align256(p.rows_pad * cols));
    p.m = (int32_t*) (b + align256(p.rows_pad * cols) + align256(p.rows_pad * (cols / 32) * 4));
    return p;
}

// zero codes and scales of the padding rows [rows, rows_pad) (a tile that over-reads them multiplies zeros), in the
// quantize launch's last kPadBlocks blocks
constexpr int kPadBlocks = 32;
__device__ __forceinline__ void zero_pad_rows(const MmqPlanes& P, int64_t rows, int block) {
    const int64_t nb = P.cols / 32;
    const int64_t n_q = (P.rows_pad - rows) * P.cols, n_s = (P.rows_pad - rows) * nb;
    const int64_t step = (int64_t) kPadBlocks * blockDim.x;
    for (int64_t i = (int64_t) block * blockDim.x + threadIdx.x; i < n_q / 4; i += step)
        ((uint32_t*) (P.q + rows * P.cols))[i] = 0u;  // rows * cols and cols are multiples of 32
    for (int64_t i = (int64_t) block * blockDim.x + threadIdx.x; i < n_s; i += step) {
        P.d[rows * nb + i] = 0.f;
        P.m[rows * nb + i] = 0;
    }
}

// 8 lanes per Q8_1 block, 4 values each (float4 loads, 4-byte code stores, DPP reductions within the 8 lanes):
// row i of the output is row ids[i] (or i) of x.  The codes of q8_1_store32, byte for byte.  Blocks past the
// quantize's own zero the padding rows.
__global__ void __launch_bounds__(kThreads) mmq_quantize_kernel(const float* __restrict__ x, const int32_t* __restrict__ ids,
                                                                MmqPlanes P, int64_t cols, int64_t ld, int64_t rows,
                                                                int qblocks) {
    if ((int) blockIdx.x >= qblocks) {
        zero_pad_rows(P, rows, (int) blockIdx.x - qblocks);
        return;
    }
    const int64_t nq = cols / 4;  // quads per row
    const int64_t qi = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = qi < rows * nq;
    const int64_t qc = valid ? qi : rows * nq - 1;  // every lane takes part in the reductions
    const int64_t i = qc / nq, c4 = qc % nq;
    const int64_t src = ids ? ids[i] : i;
    const float4 v = *(const float4*) (x + src * ld + 4 * c4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = lanes_reduce<8>(amax, OpMax());
    const float d = q8_1_finite(amax / 127.0f), rd = 1.0f / d;
    auto code = [&](float f) { return q8_1_code_rd(f, amax, d, rd); };
    const int q0 = code(v.x), q1 = code(v.y), q2 = code(v.z), q3 = code(v.w);
    const float qs = lanes_reduce<8>((float) (q0 + q1 + q2 + q3), OpAddF());  // |sum| <= 32 * 127: exact in fp32
    if (valid) {
        *(uint32_t*) (P.q + i * cols + 4 * c4) = ((uint32_t) q0 & 0xFFu) | ((uint32_t) q1 & 0xFFu) << 8 |
                                                 ((uint32_t) q2 & 0xFFu) << 16 | ((uint32_t) q3 & 0xFFu) << 24;
        if ((c4 & 7) == 0) {
            const int64_t b = c4 / 8;
            P.d[i * (cols / 32) + b] = h2f(f2h(q8_1_finite(d)));
            P.m[i * (cols / 32) + b] = (int32_t) qs;
        }
    }
}

// the same for rows that are not 16-byte aligned: one 32-lane group per Q8_1 block, one value per lane
__global__ void __launch_bounds__(kThreads) mmq_quantize1_kernel(const float* __restrict__ x, const int32_t* __restrict__ ids,
                                                                 MmqPlanes P, int64_t cols, int64_t ld, int64_t rows,
                                                                 int qblocks) {
    if ((int) blockIdx.x >= qblocks) {
        zero_pad_rows(P, rows, (int) blockIdx.x - qblocks);
        return;
    }
    const int64_t nb = cols / 32;
    const int64_t gi = ((int64_t) blockIdx.x * blockDim.x + threadIdx.x) / 32;
    const int lane = threadIdx.x & 31;
    if (gi >= rows * nb) return;  // whole 32-lane groups
    const int64_t i = gi / nb, b = gi % nb;
    const int64_t src = ids ? ids[i] : i;
    const float v = x[src * ld + 32 * b + lane];
    float amax = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    const float d = q8_1_finite(amax / 127.0f);
    const int q = q8_1_code_rd(v, amax, d, 1.0f / d);
    int qs = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) qs += __shfl_xor(qs, o, 32);
    P.q[i * cols + 32 * b + lane] = (int8_t) q;
    if (lane == 0) {
        P.d[i * nb + b] = h2f(f2h(q8_1_finite(d)));
        P.m[i * nb + b] = qs;
    }
}

// ------------------------------------------------------------------ grouped product (row-dot form)
// block (row chunk, expert): weight rows of one expert against all of its token rows, kNC tokens per pass
constexpr int kNC = 4;
template <int T, int LPR>
__global__ void __launch_bounds__(kThreads) mmq_rows_kernel(const uint8_t* __restrict__ w, uint64_t expert_bytes,
                                                            uint64_t row_bytes, int w_rows, int w_cols, MmqPlanes P,
                                                            const int32_t* __restrict__ bounds,
                                                            const int32_t* __restrict__ ids, float* __restrict__ dst,
                                                            int64_t ld_dst) {
    constexpr int RPW = kWave / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPR, l = lane % LPR;
    const int r = (blockIdx.x * (kThreads / kWave) + wave) * RPW + slot;
    if (r >= w_rows) return;
    const int x = blockIdx.y;
    const int b0 = bounds[x], b1 = bounds[x + 1];
    const uint8_t* wr = w + (uint64_t) x * expert_bytes + (uint64_t) r * row_bytes;
    const int nu = w_cols / 32;
    for (int t0 = b0; t0 < b1; t0 += kNC) {
        const int n = min(kNC, b1 - t0);
        float acc[kNC] = {0.f, 0.f, 0.f, 0.f};
        for (int u = l; u < nu; u += LPR) {
            Unit wu;
            unit_load<T>(wr, u, wu, grid_const());
#pragma unroll
            for (int c = 0; c < kNC; ++c) {
                if (c < n) {
                    const int64_t row = t0 + c;
                    Act a;
                    const int4* qp = (const int4*) (P.q + row * P.cols + 32 * u);
                    const int4 q0 = qp[0], q1 = qp[1];
                    a.q[0] = q0.x; a.q[1] = q0.y; a.q[2] = q0.z; a.q[3] = q0.w;
                    a.q[4] = q1.x; a.q[5] = q1.y; a.q[6] = q1.z; a.q[7] = q1.w;
                    a.d = P.d[row * nu + u];
                    int S, M;
                    acc[c] += unit_dot<T>(wu, a, S, M);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < kNC; ++c) acc[c] = group_sum<LPR>(acc[c]);
        if (l == 0)
            for (int c = 0; c < n; ++c) {
                const int64_t row = t0 + c;
                dst[(int64_t) (ids ? ids[row] : row) * ld_dst + r] = acc[c];
            }
    }
}

// ------------------------------------------------------------------ grouped product (f16 MFMA, exact unit sums)
// Block (weight-row tile bx, token tile by): BM = 32 * NW rows of one expert's matrix against up to 64 of the
// expert's sorted token rows.  The token tiles of all experts are numbered in expert order (tiles of expert x =
// ceil(rows_x / 64)); each block finds its expert from `bounds` with a block scan, so the launch needs no host-side
// count.
//
// The product runs on v_mfma_f32_16x16x32_f16, one MFMA per 32-value unit, with operands that are small integers and
// therefore exact in fp16: A = the unit's weight codes times the integer part of its scale (IQ3_XXS: grid * sign *
// (2 ls + 1) <= 1922; IQ3_S: <= 15 * 31; Q4_K: q * sc <= 945; Q8_0: the code), B = the Q8_1 activation codes.  Every
// product and partial sum is an integer below 2^24, so the fp32 result is exactly (integer scale) x S, S the unit's
// int8 dot product: the same integer sums as an int8 MFMA, with the integer scale already applied.  What is left per
// output per unit is one fma with the activation scale, t += d_x * D; the weight row's float scale multiplies t once
// per 256-value chunk (Q4_K adds its min term, one more fma; Q8_0 has a float scale per unit).  The int8 MFMA would
// need three VALU operations per output per unit (convert, scale product, fma) against one here.
//
// Each wave owns 32 weight rows (two 16-row MFMA tiles) and every token of the tile, so it decodes its own A
// fragments straight into registers from its raw GGUF blocks (staged per wave in LDS with 16-byte loads aligned
// down) and only the activation tile is shared.  Activation codes are widened to fp16 while staging
// (0x64XX - 1152 = XX - 128 per byte).  K advances one 256-value chunk at a time; the next chunk's weight pieces and
// activation codes are in flight in registers while the current one is multiplied, and the activation tile is
// double-buffered when LDS allows (one block barrier per chunk).
constexpr int kBN = 64;
constexpr int kChunk = 256;
constexpr int kBStride = kChunk + 8;  // fp16 per activation-tile row: 528 bytes puts 16 lanes' 16-byte reads on all banks
constexpr int kMaxExpertsMmq = 512;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// fp16 codebooks: grid entry -> its 4 magnitudes as two fp16 pairs; 8 signs -> the XOR masks of four fp16 pairs
struct HalfTables {
    uint32_t xxs[2 * 256], xxs_sign[4 * 128], s[2 * 512], s_sign[4 * 256];
};
constexpr uint32_t half_bits(uint32_t v) {  // exact fp16 of an integer in [0, 2048)
    if (v == 0) return 0;
    int e = 0;
    while ((v >> (e + 1)) != 0) ++e;
    return (uint32_t) ((e + 15) << 10) | ((v << (10 - e)) & 1023u);
}
constexpr uint32_t half_pair(uint32_t a, uint32_t b) { return half_bits(a) | half_bits(b) << 16; }
constexpr uint32_t sign_word(uint32_t s8, int k) { return ((s8 >> (2 * k)) & 1u) << 15 | ((s8 >> (2 * k + 1)) & 1u) << 31; }
constexpr HalfTables make_half_tables() {
    HalfTables h{};
    for (int i = 0; i < 256; ++i) {
        const uint32_t w = tsx_iq3xxs_word(i);
        h.xxs[2 * i] = half_pair(w & 255u, (w >> 8) & 255u);
        h.xxs[2 * i + 1] = half_pair((w >> 16) & 255u, w >> 24);
    }
    for (int i = 0; i < 512; ++i) {
        const uint32_t w = tsx_iq3s_word(i);
        h.s[2 * i] = half_pair(w & 255u, (w >> 8) & 255u);
        h.s[2 * i + 1] = half_pair((w >> 16) & 255u, w >> 24);
    }
    for (uint32_t v = 0; v < 128; ++v)
        for (int k = 0; k < 4; ++k) h.xxs_sign[4 * v + k] = sign_word(v | parity7(v) << 7, k);
    for (uint32_t b = 0; b < 256; ++b)
        for (int k = 0; k < 4; ++k) h.s_sign[4 * b + k] = sign_word(b, k);
    return h;
}
static __constant__ const HalfTables kHalf = make_half_tables();
template <int T> constexpr int half_grid_words() { return T == TSX_IQ3_XXS ? 512 : T == TSX_IQ3_S ? 1024 : 0; }
template <int T> constexpr int half_table_words() { return 2 * half_grid_words<T>(); }

constexpr int lds_round(int bytes) { return (bytes + 15) / 16 * 16; }
template <int T> constexpr int chunk_bytes() { return T == TSX_Q8_0 ? 8 * 34 : Fmt<T>::bytes; }
// LDS bytes per row of a chunk's raw blocks: the block plus up to 15 bytes of alignment in front of it, rounded to
// an odd number of 16-byte pieces so that 16 lanes reading the same field of 16 rows hit 16 different bank quads.
// A chunk of whole 16-byte pieces (Q4_K's 144 bytes, Q8_0's 272) always starts 16-byte aligned - rows, chunks and
// experts are whole pieces apart - so it takes its own pieces only
template <int T> constexpr bool chunk_aligned() { return chunk_bytes<T>() % 16 == 0; }
template <int T> constexpr int raw_stride() {
    return ((chunk_bytes<T>() + (chunk_aligned<T>() ? 0 : 15) + 15) / 16 | 1) * 16;
}
template <int T, int NW, int NB> constexpr int f16_lds_bytes() {
    return NB * (kBN * kBStride * 2 + kBN * 8 * 4 * (T == TSX_Q4_K ? 2 : 1)) + NW * 32 * raw_stride<T>() +
           half_table_words<T>() * 4 + NW * (32 * 4 + 8 * 32 * 4 * 3) + 64;
}
template <int T, int NW> constexpr int f16_buffers() { return f16_lds_bytes<T, NW, 2>() <= 150 * 1024 ? 2 : 1; }

__device__ __forceinline__ uint32_t hmul(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}
__device__ __forceinline__ uint32_t hadd(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) + __builtin_bit_cast(h2, b));
}
__device__ __forceinline__ uint32_t hpair(uint32_t v) {  // small integer -> the fp16 pair (v, v)
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16) (float) v);
    return h | h << 16;
}
// four signed bytes -> two fp16 pairs (bytes 0,1 and 2,3)
__device__ __forceinline__ void i8_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;
    lo = hadd(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), 0xE480E480u);
    hi = hadd(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), 0xE480E480u);
}
// four bytes in [0, 15] times the pair sc -> two fp16 pairs: (1024 + b) * sc - 1024 * sc, exact in one fma
__device__ __forceinline__ void nib_to_h(uint32_t w, h2 sc, h2 nsc, uint32_t& lo, uint32_t& hi) {
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u));
    const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u));
    lo = __builtin_bit_cast(uint32_t, a * sc + nsc);
    hi = __builtin_bit_cast(uint32_t, b * sc + nsc);
}
// the LDS address of p held in a register the compiler cannot see into, so that constant offsets from it go into
// the 16-bit offset field of the LDS instructions instead of an add per access
template <typename T> __device__ __forceinline__ lds_ptr<const T> lds_base(const void* p) {
    uint32_t a = (uint32_t) (uintptr_t) (lds_ptr<const void>) p;
    asm volatile("" : "+v"(a));
    return (lds_ptr<const T>) (uintptr_t) a;
}
__device__ __forceinline__ void wave_lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// exclusive prefix sum over the NT threads of the block (v per thread), and the total
template <int NT>
__device__ __forceinline__ int block_scan(int v, int* s_wave, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int off = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        off += w < wave ? s_wave[w] : 0;
        total += s_wave[w];
    }
    return off + inc - v;
}

// FUSE: the gate/up product with SwiGLU and the Q8_1 of h fused in (NW = 8).  Block bx takes gate rows
// [128 bx, 128 bx + 128) in waves 0-3 and the matching up rows (n_ff further) in waves 4-7; the activation rows are
// xids[sorted row] of P (sorted row r itself when xids is null); h leaves as Q8_1 planes H, one row per sorted row.
template <int T, int NW, bool FUSE = false>
__global__ void __launch_bounds__(64 * NW) mmq_f16_kernel(const uint8_t* __restrict__ w, uint64_t expert_bytes,
                                                          uint64_t row_bytes, int w_cols, int n_exp, MmqPlanes P,
                                                          const int32_t* __restrict__ bounds,
                                                          const int32_t* __restrict__ ids, float* __restrict__ dst,
                                                          int64_t ld_dst, const int32_t* __restrict__ xids = nullptr,
                                                          MmqPlanes H = MmqPlanes{}, int n_ff = 0) {
    constexpr int NT = 64 * NW, BM = 32 * NW, NB = f16_buffers<T, NW>();
    constexpr int CB = chunk_bytes<T>(), RS = raw_stride<T>(), PR = RS / 16, RW = (32 * PR + 63) / 64;
    constexpr int BP = kBN * 16 / NT, DP = kBN * 8 / NT, EPT = kMaxExpertsMmq / NT;
    constexpr int TW = half_table_words<T>(), GW = half_grid_words<T>(), TPT = (TW + NT - 1) / NT;
    constexpr bool Q4K = T == TSX_Q4_K, Q80 = T == TSX_Q8_0, IQ3S = T == TSX_IQ3_S;
    // LDS as one array laid out by hand: the codebooks at address 0 and the arrays read per unit next, so that
    // their addresses fit the 16-bit offsets of the LDS instructions; the raw weight slabs and the activation tiles
    // last (the compiler would order separate arrays by size, the large ones first)
    constexpr int XXS = T == TSX_IQ3_XXS;
    constexpr int O_TAB = 0, O_AM = O_TAB + lds_round((TW > 0 ? TW : 4) * 4);
    constexpr int O_SC = O_AM + lds_round((XXS ? NW : 1) * 8 * 32 * 8);
    constexpr int O_UF = O_SC + lds_round((IQ3S || Q4K ? NW : 1) * 8 * 32 * 4);
    constexpr int O_RD = O_UF + lds_round((Q4K || Q80 ? NW : 1) * 8 * 32 * 4);
    constexpr int O_DX = O_RD + lds_round(NW * 32 * 4);
    constexpr int O_DM = O_DX + lds_round(NB * kBN * 8 * 4);
    constexpr int O_SCAN = O_DM + lds_round((Q4K ? NB * kBN : 1) * 8 * 4);
    constexpr int O_RAW = O_SCAN + lds_round((NW + 2) * 4);
    constexpr int O_TB = O_RAW + lds_round(NW * 32 * RS);
    constexpr int LDS_BYTES = O_TB + NB * kBN * kBStride * 2;
    __shared__ __attribute__((aligned(16))) uint8_t s_lds[LDS_BYTES];
    auto& s_tab = *reinterpret_cast<uint32_t(*)[TW > 0 ? TW : 4]>(s_lds + O_TAB);
    auto& s_am = *reinterpret_cast<uint2(*)[XXS ? NW : 1][8][32]>(s_lds + O_AM);         // IQ3_XXS: aux word, m pair
    auto& s_sc = *reinterpret_cast<uint32_t(*)[IQ3S || Q4K ? NW : 1][8][32]>(s_lds + O_SC);  // integer scale, fp16 pair
    auto& s_uf = *reinterpret_cast<float(*)[Q4K || Q80 ? NW : 1][8][32]>(s_lds + O_UF);     // Q4_K: dmin * m; Q8_0: d
    auto& s_rd = *reinterpret_cast<float(*)[NW][32]>(s_lds + O_RD);                         // row scale per chunk
    auto& s_dx = *reinterpret_cast<float(*)[NB][kBN][8]>(s_lds + O_DX);
    auto& s_dm = *reinterpret_cast<float(*)[Q4K ? NB : 1][Q4K ? kBN : 1][8]>(s_lds + O_DM);
    int* const s_scan = reinterpret_cast<int*>(s_lds + O_SCAN);
    int& s_x = s_scan[NW];
    int& s_tile0 = s_scan[NW + 1];
    auto& s_raw = *reinterpret_cast<uint8_t(*)[NW][32 * RS]>(s_lds + O_RAW);
    auto& tB = *reinterpret_cast<_Float16(*)[NB][kBN * kBStride]>(s_lds + O_TB);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bx = blockIdx.x, by = blockIdx.y;
    const int lr = lane & 15, g = lane >> 4;

    // 1. which expert and which of its token tiles: EPT experts per thread, a block scan of tile counts
    int tc[EPT], mine = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int x = EPT * tid + e;
        const int b0 = bounds[min(x, n_exp)], b1 = bounds[min(x + 1, n_exp)];
        tc[e] = x < n_exp ? (b1 - b0 + kBN - 1) / kBN : 0;
        mine += tc[e];
    }
    int total;
    int start = block_scan<NT>(mine, s_scan, total);
    if (by >= total) return;  // the whole block: fewer tiles than the grid's upper bound
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        if (start <= by && by < start + tc[e]) {
            s_x = EPT * tid + e;
            s_tile0 = start;
        }
        start += tc[e];
    }
    __syncthreads();
    const int x = s_x;
    const int row0 = bounds[x] + (by - s_tile0) * kBN;
    const int nrows = min(kBN, bounds[x + 1] - row0);
    const int ntt = (nrows + 15) >> 4;  // 16-token MFMA tiles with rows in them
    const int wrow = FUSE ? (wave < NW / 2 ? 0 : n_ff) + (BM / 2) * bx + 32 * (wave % (NW / 2)) : bx * BM + 32 * wave;
    const uint8_t* wbase = w + (uint64_t) x * expert_bytes + (uint64_t) wrow * row_bytes;
    const int nu = w_cols / 32, nchunks = w_cols / kChunk;
    // the activation rows this thread loads (the same every chunk): rows past the tile's last take its last row
    int64_t arow_b[BP], arow_d[DP];
#pragma unroll
    for (int h = 0; h < BP; ++h) {
        const int rr = (tid + NT * h) >> 4;
        arow_b[h] = xids ? (int64_t) xids[row0 + min(rr, nrows - 1)] : (int64_t) (row0 + rr);
    }
#pragma unroll
    for (int h = 0; h < DP; ++h) {
        const int rr = (tid + NT * h) >> 3;
        arow_d[h] = xids ? (int64_t) xids[row0 + min(rr, nrows - 1)] : (int64_t) (row0 + rr);
    }

    // chunk c in flight: this wave's raw weight pieces, the block's share of activation codes and scales
    v4i rw[RW], av[BP];
    float ad[DP];
    int am[DP];
    auto fetch = [&](int c) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int q = min(lane + 64 * i, 32 * PR - 1), r = q / PR, pc = q - r * PR;
            const uint64_t o = (uint64_t) r * row_bytes + (uint64_t) c * CB;
            const int need = (int) (((o & 15) + CB + 15) / 16);  // pieces that start before the block's end
            rw[i] = __builtin_nontemporal_load((const v4i*) (wbase + (o & ~(uint64_t) 15)) + min(pc, need - 1));
        }
#pragma unroll
        for (int h = 0; h < BP; ++h) {
            const int pi = tid + NT * h, q = pi & 15;
            av[h] = *(const v4i*) (P.q + arow_b[h] * P.cols + kChunk * c + 16 * q);
        }
#pragma unroll
        for (int h = 0; h < DP; ++h) {
            const int e = tid + NT * h, u = e & 7;
            const int64_t o = arow_d[h] * nu + 8 * c + u;
            ad[h] = P.d[o];
            if constexpr (Q4K) am[h] = P.m[o];
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < RW; ++i)
            if (lane + 64 * i < 32 * PR) ((v4i*) s_raw[wave])[lane + 64 * i] = rw[i];
#pragma unroll
        for (int h = 0; h < BP; ++h) {
            const int pi = tid + NT * h, rr = pi >> 4, q = pi & 15;
            uint32_t o[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) i8_to_h((uint32_t) av[h][k], o[2 * k], o[2 * k + 1]);
            v4i* d = (v4i*) (&tB[buf][rr * kBStride + 16 * q]);
            d[0] = v4i{(int) o[0], (int) o[1], (int) o[2], (int) o[3]};
            d[1] = v4i{(int) o[4], (int) o[5], (int) o[6], (int) o[7]};
        }
#pragma unroll
        for (int h = 0; h < DP; ++h) {
            const int e = tid + NT * h, rr = e >> 3, u = e & 7;
            s_dx[buf][rr][u] = ad[h];
            if constexpr (Q4K) s_dm[buf][rr][u] = ad[h] * (float) am[h];
        }
    };

    uint32_t tw[TPT > 0 ? TPT : 1];
    if constexpr (TW > 0) {
        const uint32_t* src = T == TSX_IQ3_XXS ? kHalf.xxs : kHalf.s;
        const uint32_t* sgn = T == TSX_IQ3_XXS ? kHalf.xxs_sign : kHalf.s_sign;
#pragma unroll
        for (int k = 0; k < TPT; ++k) {
            const int i = min(tid + NT * k, TW - 1);
            tw[k] = i < GW ? src[i] : sgn[i - GW];
        }
    }
    fetch(0);
    if constexpr (TW > 0) {
#pragma unroll
        for (int k = 0; k < TPT; ++k)
            if (tid + NT * k < TW) s_tab[tid + NT * k] = tw[k];
    }
    stage(0);
    if (nchunks > 1) fetch(1);
    __syncthreads();

    // the chunk loop, specialised on the number of 16-token tiles that hold rows (no per-tile branches inside)
    auto run = [&](auto ntt_c) {
        constexpr int NTT = decltype(ntt_c)::value;
        float acc[2][NTT][4], tacc[2][NTT][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][tj][i] = tacc[t][tj][i] = 0.f;

        for (int c = 0; c < nchunks; ++c) {
            const int buf = NB == 2 ? (c & 1) : 0;
            const _Float16* B = tB[buf];
            const uint8_t* slab = s_raw[wave];
            const lds_ptr<const v4i> bq = lds_base<v4i>(B + lr * kBStride + 8 * g);  // this lane's activation pieces
            // the wave's rows: per-row and per-unit factors (lane = row r, units 4 hl .. 4 hl + 3)
            {
                const int r = lane & 31, hl = lane >> 5;
                const uint8_t* b = slab + r * RS + (int) (((uint64_t) r * row_bytes + (uint64_t) c * CB) & 15);
                if constexpr (T == TSX_IQ3_XXS) {
                    if (hl == 0) s_rd[wave][r] = 0.25f * h2f((uint16_t) ld16(b));
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int j = 4 * hl + k;
                        const uint32_t aux = ld32a2(b + 66 + 4 * j);
                        s_am[wave][j][r] = uint2{aux, hpair(2 * (aux >> 28) + 1)};
                    }
                } else if constexpr (IQ3S) {
                    if (hl == 0) s_rd[wave][r] = h2f((uint16_t) ld16(b));
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int j = 4 * hl + k;
                        s_sc[wave][j][r] = hpair(2 * ((b[106 + (j >> 1)] >> (4 * (j & 1))) & 15u) + 1);
                    }
                } else if constexpr (Q4K) {
                    const float d = h2f((uint16_t) ld16(b)), dmin = h2f((uint16_t) ld16(b + 2));
                    if (hl == 0) s_rd[wave][r] = d;
                    const uint8_t* s12 = b + 4;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int j = 4 * hl + k;
                        int sc, m;
                        if (j < 4) {
                            sc = s12[j] & 63;
                            m = s12[j + 4] & 63;
                        } else {
                            sc = (s12[j + 4] & 15) | ((s12[j - 4] >> 6) << 4);
                            m = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
                        }
                        s_sc[wave][j][r] = hpair((uint32_t) sc);
                        s_uf[wave][j][r] = dmin * (float) m;
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int j = 4 * hl + k;
                        s_uf[wave][j][r] = h2f((uint16_t) ld16(b + 34 * j));
                    }
                }
            }
            wave_lds_order();
            // the lane's decode rows (one per 16-row tile)
            const uint8_t* blk[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int r = 16 * t + lr;
                blk[t] = slab + r * RS + (int) (((uint64_t) r * row_bytes + (uint64_t) c * CB) & 15);
            }
            // unit u's weight fragments (rows 16 t + lr, values 8 g .. 8 g + 7 of the unit)
            auto decode = [&](int u, v4i (&A)[2]) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint8_t* b = blk[t];
                    const int r = 16 * t + lr;
                    uint32_t f[4];
                    if constexpr (T == TSX_IQ3_XXS) {
                        const uint32_t qp = ld16(b + 2 + 8 * u + 2 * g);
                        const uint2 am = s_am[wave][u][r];
                        const uint32_t aux = am.x, m = am.y;
                        const uint2 g0 = *(const uint2*) (s_tab + 2 * (qp & 255u));
                        const uint2 g1 = *(const uint2*) (s_tab + 2 * (qp >> 8));
                        const uint4 sm = *(const uint4*) (s_tab + GW + 4 * ((aux >> (7 * g)) & 127u));
                        f[0] = hmul(g0.x ^ sm.x, m);
                        f[1] = hmul(g0.y ^ sm.y, m);
                        f[2] = hmul(g1.x ^ sm.z, m);
                        f[3] = hmul(g1.y ^ sm.w, m);
                    } else if constexpr (IQ3S) {
                        const uint32_t qp = ld16(b + 2 + 8 * u + 2 * g);
                        const uint32_t qh = (uint32_t) b[66 + u] >> (2 * g);
                        const uint32_t i0 = (qp & 255u) | (qh & 1u) << 8, i1 = (qp >> 8) | (qh & 2u) << 7;
                        const uint2 g0 = *(const uint2*) (s_tab + 2 * i0);
                        const uint2 g1 = *(const uint2*) (s_tab + 2 * i1);
                        const uint4 sm = *(const uint4*) (s_tab + GW + 4 * (uint32_t) b[74 + 4 * u + g]);
                        const uint32_t m = s_sc[wave][u][r];
                        f[0] = hmul(g0.x ^ sm.x, m);
                        f[1] = hmul(g0.y ^ sm.y, m);
                        f[2] = hmul(g1.x ^ sm.z, m);
                        f[3] = hmul(g1.y ^ sm.w, m);
                    } else if constexpr (Q4K) {
                        const uint8_t* q = b + 16 + 32 * (u >> 1) + 8 * g;
                        const int sh = 4 * (u & 1);
                        const uint32_t w0 = (ld32a2(q) >> sh) & 0x0F0F0F0Fu, w1 = (ld32a2(q + 4) >> sh) & 0x0F0F0F0Fu;
                        const h2 sc = __builtin_bit_cast(h2, s_sc[wave][u][r]);
                        const h2 nsc = sc * (_Float16) -1024.0f;
                        nib_to_h(w0, sc, nsc, f[0], f[1]);
                        nib_to_h(w1, sc, nsc, f[2], f[3]);
                    } else {
                        const uint8_t* q = b + 34 * u + 2 + 8 * g;
                        i8_to_h(ld32a2(q), f[0], f[1]);
                        i8_to_h(ld32a2(q + 4), f[2], f[3]);
                    }
                    A[t] = v4i{(int) f[0], (int) f[1], (int) f[2], (int) f[3]};
                }
            };
            // unit u's activation fragments and scales (tokens 16 tj + lr)
            auto load_b = [&](int u, v4i (&Bf)[NTT], float (&dx)[NTT]) {
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) {
                    const int tok = 16 * tj + lr;
                    Bf[tj] = bq[(tj * 16 * kBStride + 32 * u) / 8];
                    dx[tj] = s_dx[buf][tok][u];
                }
            };
            // software pipeline over the chunk's 8 units: unit u + 1's fragments are read and decoded while unit u's
            // products run on the matrix cores, and each product is scaled only after the next unit's decode
            v4i A[2], Bf[NTT];
            float dx[NTT];
            decode(0, A);
            load_b(0, Bf, dx);
#pragma unroll 1
            for (int u = 0; u < 8; ++u) {
                v4f D[2][NTT];
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        D[t][tj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, A[t]),
                                                                         __builtin_bit_cast(v8h, Bf[tj]),
                                                                         v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                float dxu[NTT];
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) dxu[tj] = dx[tj];
                // per-output-row unit factors (Q8_0 scale): rows 16 t + 4 g + i
                float4 uf[2];
                if constexpr (Q80) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) uf[t] = *(const float4*) &s_uf[wave][u][16 * t + 4 * g];
                }
                if (u + 1 < 8) {
                    decode(u + 1, A);
                    load_b(u + 1, Bf, dx);
                }
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const float ufa[4] = {uf[t].x, uf[t].y, uf[t].z, uf[t].w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if constexpr (Q80) acc[t][tj][i] += (ufa[i] * dxu[tj]) * D[t][tj][i];
                            else tacc[t][tj][i] += dxu[tj] * D[t][tj][i];
                        }
                    }
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) asm volatile("" ::"v"(Bf[tj]), "v"(dx[tj]));  // read in this step
            }
            if constexpr (Q4K) {
                // the chunk's min term, sum over units u of (dmin m)[row][u] * (dx s)[token][u]: a [rows x 8] by
                // [8 x tokens] product on the fp32 matrix cores (two K = 4 steps), rows 16 t + lr by units 4 h + g
                // in A, units by tokens 16 tj + lr in B, accumulated into the outputs
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float am[2];
#pragma unroll
                    for (int t = 0; t < 2; ++t) am[t] = -s_uf[wave][4 * h + g][16 * t + lr];
#pragma unroll
                    for (int tj = 0; tj < NTT; ++tj) {
                        const float bm = s_dm[buf][16 * tj + lr][4 * h + g];
#pragma unroll
                        for (int t = 0; t < 2; ++t) {
                            const v4f C = {acc[t][tj][0], acc[t][tj][1], acc[t][tj][2], acc[t][tj][3]};
                            const v4f D = __builtin_amdgcn_mfma_f32_16x16x4f32(am[t], bm, C, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[t][tj][i] = D[i];
                        }
                    }
                }
            }
            if constexpr (!Q80) {  // the chunk's row scale
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float4 rd4 = *(const float4*) &s_rd[wave][16 * t + 4 * g];
                    const float rd[4] = {rd4.x, rd4.y, rd4.z, rd4.w};
#pragma unroll
                    for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            acc[t][tj][i] += rd[i] * tacc[t][tj][i];
                            tacc[t][tj][i] = 0.f;
                        }
                }
            }
            if (c + 1 < nchunks) {
                if constexpr (NB == 1) __syncthreads();  // every wave is done with the single activation tile
                wave_lds_order();                        // this wave is done with its raw slab and factor rows
                stage(NB == 2 ? (c + 1) & 1 : 0);
                if (c + 2 < nchunks) fetch(c + 2);
                __syncthreads();
            }
        }

        if constexpr (FUSE) {
#pragma clang fp contract(off)
            // the block's gate (columns 0-127) and up (128-255) outputs through LDS, in runs of TOK tokens: the
            // activation tiles' LDS once every wave is past its last chunk
            constexpr int OS = 2 * (BM / 2) + 1;  // floats per token: odd, so 16 tokens' writes hit distinct banks
            constexpr int TOK = NB * kBN * kBStride * 2 >= kBN * OS * 4 ? kBN : kBN / 2;
            float* so = (float*) &tB[0][0];
            __syncthreads();
            for (int t0 = 0; t0 < 16 * NTT; t0 += TOK) {
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) {
                    const int tok = 16 * tj + lr - t0;
                    if (tok >= 0 && tok < TOK)
#pragma unroll
                        for (int t = 0; t < 2; ++t)
#pragma unroll
                            for (int i = 0; i < 4; ++i) so[tok * OS + 32 * wave + 16 * t + 4 * g + i] = acc[t][tj][i];
                }
                __syncthreads();
                // h = silu(gate) * up (the product rounded on its own) and its Q8_1 blocks: 8 lanes per 32 values,
                // 4 each, every lane taking part in the reductions
                const int ntok = min(TOK, 16 * NTT - t0);  // a multiple of 16: whole rounds of the block
                for (int q0 = 0; q0 < ntok * (BM / 8); q0 += NT) {
                    const int q = q0 + tid, tok = q / (BM / 8), f4 = q % (BM / 8);
                    const float* gp = so + tok * OS + 4 * f4;
                    float hv[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float gt = gp[k];
                        hv[k] = (gt / (1.0f + expf(-gt))) * gp[BM / 2 + k];
                    }
                    float amax = fmaxf(fmaxf(fabsf(hv[0]), fabsf(hv[1])), fmaxf(fabsf(hv[2]), fabsf(hv[3])));
                    amax = lanes_reduce<8>(amax, OpMax());
                    const float d = q8_1_finite(amax / 127.0f), rd = 1.0f / d;
                    int qv[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) qv[k] = q8_1_code_rd(hv[k], amax, d, rd);
                    const float qs = lanes_reduce<8>((float) (qv[0] + qv[1] + qv[2] + qv[3]), OpAddF());
                    if (t0 + tok < nrows) {
                        const int64_t hr = row0 + t0 + tok, col = (int64_t) (BM / 2) * bx + 4 * f4;
                        *(uint32_t*) (H.q + hr * H.cols + col) = ((uint32_t) qv[0] & 0xFFu) |
                                                                 ((uint32_t) qv[1] & 0xFFu) << 8 |
                                                                 ((uint32_t) qv[2] & 0xFFu) << 16 |
                                                                 ((uint32_t) qv[3] & 0xFFu) << 24;
                        if ((f4 & 7) == 0) {
                            H.d[hr * (H.cols / 32) + col / 32] = h2f(f2h(q8_1_finite(d)));
                            H.m[hr * (H.cols / 32) + col / 32] = (int32_t) qs;
                        }
                    }
                }
                __syncthreads();
            }
        } else {
            // out: weight row 16 t + 4 g + i of the wave, token 16 tj + lr
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj) {
                const int tok = 16 * tj + lr;
                if (tok < nrows) {
                    const int64_t drow = ids ? ids[row0 + tok] : row0 + tok;
                    float* o = dst + drow * ld_dst + (int64_t) bx * BM + 32 * wave + 4 * g;
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[16 * t + i] = acc[t][tj][i];
                }
            }
        }
    };
    if (ntt == 1) run(std::integral_constant<int, 1>{});
    else if (ntt == 2) run(std::integral_constant<int, 2>{});
    else if (ntt == 3) run(std::integral_constant<int, 3>{});
    else run(std::integral_constant<int, 4>{});
}

__global__ void __launch_bounds__(kThreads) mmq_swiglu_kernel(const float* __restrict__ gu, float* __restrict__ h,
                                                              int64_t rows, int64_t n_ff, int interleaved) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n_ff) return;
    const int64_t r = i / n_ff, k = i % n_ff;
    const float* row = gu + r * 2 * n_ff;
    const float g = interleaved ? row[2 * k] : row[k], u = interleaved ? row[2 * k + 1] : row[n_ff + k];
    h[i] = (g / (1.0f + expf(-g))) * u;
}

template <typename F>
int with_type(int type, F&& f) {
    switch (type) {
        case TSX_IQ3_XXS: return f(std::integral_constant<int, TSX_IQ3_XXS>{});
        case TSX_IQ3_S: return f(std::integral_constant<int, TSX_IQ3_S>{});
        case TSX_Q4_K: return f(std::integral_constant<int, TSX_Q4_K>{});
        case TSX_Q8_0: return f(std::integral_constant<int, TSX_Q8_0>{});
        default: return TSX_ERR_UNSUPPORTED;
    }
}
template <typename F>
int with_lpr(int lpr, F&& f) {
    switch (lpr) {
        case 8: return f(std::integral_constant<int, 8>{});
        case 16: return f(std::integral_constant<int, 16>{});
        case 32: return f(std::integral_constant<int, 32>{});
        default: return f(std::integral_constant<int, 64>{});
    }
}
int lanes_per_row(int nu) {
    int l = 8;
    while (l < nu && l < 64) l <<= 1;
    return l;
}

}  // namespace
}  // namespace tsx

using namespace tsx;

extern "C" {

TSX_API size_t tsx_moe_mmq_q8_bytes(int64_t rows, int64_t cols) {
    if (rows < 0 || cols <= 0 || cols % 32 != 0) return 0;
    const int64_t rp = pad_rows(rows);
    return (size_t) (align256(rp * cols) + 2 * align256(rp * (cols / 32) * 4));
}

TSX_API int tsx_moe_mmq_quantize(const float* x, const int32_t* ids, void* xq, int type, int64_t cols, int64_t ld,
                                 int64_t rows, void* stream) {
    (void) type;  // one layout serves every weight type
    TSX_REQUIRE(x && xq && cols > 0 && cols % 32 == 0 && ld >= cols && rows >= 0 && aligned(xq, 256),
                "tsx_moe_mmq_quantize: x, xq (256-byte aligned), cols a multiple of 32, ld >= cols");
    const MmqPlanes P = planes(xq, rows, cols);
    const hipStream_t s = (hipStream_t) stream;
    // one launch: the quantize's blocks, then kPadBlocks that zero the padding rows
    if (aligned(x, 16) && ld % 4 == 0) {
        const int qb = (int) ((rows * (cols / 4) + kThreads - 1) / kThreads);
        mmq_quantize_kernel<<<(unsigned) (qb + kPadBlocks), kThreads, 0, s>>>(x, ids, P, cols, ld, rows, qb);
    } else {
        const int qb = (int) ((rows * (cols / 32) * 32 + kThreads - 1) / kThreads);
        mmq_quantize1_kernel<<<(unsigned) (qb + kPadBlocks), kThreads, 0, s>>>(x, ids, P, cols, ld, rows, qb);
    }
    return launch_status("tsx_moe_mmq_quantize");
}

TSX_API int tsx_moe_mmq_run(const tsx_mmq_product* p, void* stream) {
    TSX_REQUIRE(p != nullptr, "tsx_moe_mmq_run: null product");
    const size_t rb = tsx_row_bytes(p->type, p->w_cols);
    if (!tsx_weight_type_ok(p->type) || rb == 0 || (p->w_cols % 256 != 0 && p->type != TSX_Q8_0)) {
        set_error("tsx_moe_mmq_run: type %d with %lld columns not supported", p->type, (long long) p->w_cols);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(p->w && p->xq && p->bounds && p->dst && p->n >= 0 && p->w_rows >= 0 && p->total_rows >= 0 &&
                    p->ld_dst >= p->w_rows && aligned(p->xq, 256) && p->expert_bytes >= rb * (uint64_t) p->w_rows,
                "tsx_moe_mmq_run: w, xq (256-byte aligned), bounds, dst, ld_dst >= w_rows, expert_bytes >= the matrix");
    if (p->n == 0 || p->w_rows == 0) return TSX_OK;
    const MmqPlanes P = planes((void*) p->xq, p->total_rows, p->w_cols);
    const hipStream_t s = (hipStream_t) stream;
    // the f16-MFMA tiles where the shape fits them (rows in multiples of 64), else the row-dot kernel
    if (p->w_cols % kChunk == 0 && p->w_rows % 64 == 0 && p->n <= kMaxExpertsMmq && aligned(p->w, 16) &&
        p->expert_bytes % 16 == 0) {
        const int64_t max_tiles = (p->total_rows + kBN - 1) / kBN + p->n;
        const int nw = p->w_rows % 256 == 0 ? 8 : p->w_rows % 128 == 0 ? 4 : 2;
        return with_type(p->type, [&](auto T) {
            constexpr int TT = decltype(T)::value;
            const dim3 grid((unsigned) (p->w_rows / (32 * nw)), (unsigned) max_tiles);
            const uint8_t* w = (const uint8_t*) p->w;
            if (nw == 8)
                mmq_f16_kernel<TT, 8><<<grid, 512, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst);
            else if (nw == 4)
                mmq_f16_kernel<TT, 4><<<grid, 256, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst);
            else
                mmq_f16_kernel<TT, 2><<<grid, 128, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst);
            return launch_status("tsx_moe_mmq_run/mfma");
        });
    }
    const int lpr = lanes_per_row((int) (p->w_cols / 32)), rows = (kThreads / kWave) * (kWave / lpr);
    return with_type(p->type, [&](auto T) {
        return with_lpr(lpr, [&](auto LPR) {
            const dim3 grid((unsigned) ((p->w_rows + rows - 1) / rows), (unsigned) p->n);
            mmq_rows_kernel<decltype(T)::value, decltype(LPR)::value><<<grid, kThreads, 0, s>>>(
                (const uint8_t*) p->w, p->expert_bytes, rb, (int) p->w_rows, (int) p->w_cols, P, p->bounds, p->ids, p->dst,
                p->ld_dst);
            return launch_status("tsx_moe_mmq_run");
        });
    });
}

TSX_API int tsx_moe_mmq_gate_up_swiglu(const void* w, int type, int64_t n_ff, int64_t n_embd, uint64_t expert_bytes,
                                       int n_exp, const void* xq, int64_t x_rows, const int32_t* xids,
                                       const int32_t* bounds, int64_t n_rows, void* hq, void* stream) {
    const size_t rb = tsx_row_bytes(type, n_embd);
    if (!tsx_weight_type_ok(type) || rb == 0 || n_embd % kChunk != 0 || n_ff <= 0 || n_ff % 128 != 0 ||
        n_exp > kMaxExpertsMmq) {
        set_error("tsx_moe_mmq_gate_up_swiglu: type %d, %lld x %lld, %d experts not supported (n_embd a multiple of "
                  "256, n_ff of 128, at most %d experts)",
                  type, (long long) n_embd, (long long) n_ff, n_exp, kMaxExpertsMmq);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(w && xq && bounds && hq && n_exp >= 0 && x_rows >= 0 && n_rows >= 0 && aligned(w, 16) &&
                    expert_bytes % 16 == 0 && expert_bytes >= rb * (uint64_t) (2 * n_ff) && aligned(xq, 256) &&
                    aligned(hq, 256),
                "tsx_moe_mmq_gate_up_swiglu: w, xq, bounds, hq (xq and hq 256-byte aligned, w and expert_bytes "
                "16-byte), expert_bytes >= the gate and up rows");
    if (n_exp == 0 || n_rows == 0) return TSX_OK;
    const MmqPlanes P = planes((void*) xq, x_rows, n_embd), H = planes(hq, n_rows, n_ff);
    const hipStream_t s = (hipStream_t) stream;
    const int64_t max_tiles = (n_rows + kBN - 1) / kBN + n_exp;
    return with_type(type, [&](auto T) {
        const dim3 grid((unsigned) (n_ff / 128), (unsigned) max_tiles);
        mmq_f16_kernel<decltype(T)::value, 8, true><<<grid, 512, 0, s>>>(
            (const uint8_t*) w, expert_bytes, rb, (int) n_embd, n_exp, P, bounds, nullptr, nullptr, 0, xids, H, (int) n_ff);
        return launch_status("tsx_moe_mmq_gate_up_swiglu");
    });
}

TSX_API int tsx_moe_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream) {
    TSX_REQUIRE(gu && h && rows >= 0 && n_ff > 0, "tsx_moe_mmq_swiglu: gu, h, n_ff > 0");
    if (rows == 0) return TSX_OK;
    const int64_t n = rows * n_ff;
    mmq_swiglu_kernel<<<(unsigned) ((n + kThreads - 1) / kThreads), kThreads, 0, (hipStream_t) stream>>>(gu, h, rows, n_ff,
                                                                                                       interleaved);
    return launch_status("tsx_moe_mmq_swiglu");
}

}  // extern "C"
