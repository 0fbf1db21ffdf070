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
__device__ __forceinline__ void quantize_quads(const float* __restrict__ x, const int32_t* __restrict__ ids,
                                               const MmqPlanes& P, int64_t cols, int64_t ld, int64_t rows, int block) {
    const int64_t nq = cols / 4;  // quads per row
    const int64_t qi = (int64_t) block * blockDim.x + threadIdx.x;
    const bool valid = qi < rows * nq;
    const int64_t qc = valid ? qi : rows * nq - 1;  // every lane takes part in the reductions
    const int64_t i = qc / nq, c4 = qc % nq;
    const int64_t src = ids ? ids[i] : i;
    const float4 v = *(const float4*) (x + src * ld + 4 * c4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = lanes_reduce<8>(amax, OpMax());
    const float d = q8_1_scale(amax);
    int qv[4];
    q8_1_codes4(v, amax, d, qv);
    const int q0 = qv[0], q1 = qv[1], q2 = qv[2], q3 = qv[3];
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
__global__ void __launch_bounds__(kThreads) mmq_quantize_kernel(const float* __restrict__ x, const int32_t* __restrict__ ids,
                                                                MmqPlanes P, int64_t cols, int64_t ld, int64_t rows,
                                                                int qblocks) {
    if ((int) blockIdx.x >= qblocks) zero_pad_rows(P, rows, (int) blockIdx.x - qblocks);
    else quantize_quads(x, ids, P, cols, ld, rows, (int) blockIdx.x);
}
// the prompt's token quantize and its router top-k in one launch (independent work): the first rblocks route four
// tokens each (a wave per token, route_token; their dependent loads start first), the next qblocks quantize and the
// last kPadBlocks zero the padding rows
__global__ void __launch_bounds__(kThreads) mmq_quantize_route_kernel(const float* __restrict__ x, MmqPlanes P,
                                                                      int64_t cols, int64_t ld, int64_t rows, int qblocks,
                                                                      int rblocks, const float* __restrict__ logits,
                                                                      int32_t* __restrict__ rids, float* __restrict__ rwts,
                                                                      int n_expert, int k) {
    const int b = (int) blockIdx.x;
    if (b < rblocks) {
        const int t = b * 4 + (int) (threadIdx.x >> 6);
        if (t < rows)
            route_token(logits + (int64_t) t * n_expert, n_expert, k, (int) (threadIdx.x & 63), rids + (int64_t) t * k,
                        rwts + (int64_t) t * k);
    } else if (b < rblocks + qblocks) {
        quantize_quads(x, nullptr, P, cols, ld, rows, b - rblocks);
    } else {
        zero_pad_rows(P, rows, b - rblocks - qblocks);
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
    const float d = q8_1_scale(amax);
    const int q = q8_1_code_rd(v, amax, d, q8_1_rcp(d));
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
// Block (weight-row tile bx, token tile by): BM = 32 * NW rows of one expert's matrix against up to kBN of the
// expert's sorted token rows.  The token tiles are numbered full tiles first (expert order), then each expert's
// partial last tile; each block finds its expert from `bounds` with a block scan, so the launch needs no host-side
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
// sorted token rows per block tile: 128 for the codebook formats (the decode of a weight fragment serves more tokens,
// and an expert's weights are read once per 128 of its rows); 64 for Q4_K (its experts are mostly small) and Q8_0
// (its wider raw rows fill the LDS)
template <int T> constexpr int bn_of() { return T == TSX_Q8_0 || T == TSX_Q4_K ? 64 : 128; }
// waves per block: 8 (256 weight rows), except Q4_K's 4 (128 rows) with one activation buffer, 69 KB of LDS, so that
// two blocks share a CU.  A SIMD's two waves then come from different blocks: the older of two waves of one block
// wins most issue slots and finishes a chunk ~1.5 us before the younger, which then runs alone until the chunk's
// barrier, while waves of two blocks wait at different barriers (configs[3] 263 -> 258 us per layer)
template <int T> constexpr int nw_of() { return T == TSX_Q4_K ? 4 : 8; }
constexpr int kChunk = 256;
constexpr int kUpfrontTiles = 4;  // chunk loops with at most this many 16-token tiles decode kUpfrontUnits at a time
constexpr int kUpfrontUnits = 2;
// products of at most this many columns (a down product) take two 256-row column blocks per block in turn: the
// second's first chunk is requested during the first's last, hiding a block's set-up and first-chunk latency
constexpr int kPassCols = 512;
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
// copies of the fp16 codebooks in LDS, interleaved entry by entry (entry i's copy c at slot i * copies + c; lane l
// reads copy l % copies).  One: the lookups make about half of the product's LDS bank-conflict cycles (a timing copy
// with lane-private lookup addresses ran the configs[4] gate/up 10 % faster), but eight copies, all the LDS beside the
// tiles holds, cut the conflicts by 5 % only - lanes on the same copy still fall on the same few banks, and a lane of
// its own per copy needs 32 of them
template <int T> constexpr int tab_copies() { return 1; }
template <int T> constexpr int rep_table_words() { return half_table_words<T>() * tab_copies<T>(); }

constexpr int lds_round(int bytes) { return (bytes + 15) / 16 * 16; }
template <int T> constexpr int chunk_bytes() { return T == TSX_Q8_0 ? 8 * 34 : Fmt<T>::bytes; }
// LDS bytes per row of a chunk's raw blocks: the block plus up to 15 bytes of alignment in front of it, rounded to
// an odd number of 16-byte pieces so that 16 lanes reading the same field of 16 rows hit 16 different bank quads.
// A chunk of whole 16-byte pieces (Q4_K's 144 bytes, Q8_0's 272) always starts 16-byte aligned - rows, chunks and
// experts are whole pieces apart - so it takes its own pieces only
template <int T> constexpr bool chunk_aligned() { return chunk_bytes<T>() % 16 == 0; }
template <int T> constexpr int raw_stride() {
    // a block of an even size starts at an even offset (the base, expert and row strides are multiples of 16 and the
    // blocks even), so at most 14 bytes into its first piece
    return ((chunk_bytes<T>() + (chunk_aligned<T>() ? 0 : chunk_bytes<T>() % 2 == 0 ? 14 : 15) + 15) / 16 | 1) * 16;
}
// silu(g) * u as the prompt path forms it (the fused gate/up epilogue and mmq_swiglu_kernel alike): g / (1 + e^-g)
// with e^-g = 2^(-g log2 e) on the hardware exp2 and the quotient as g times the hardware reciprocal, the product
// rounded on its own.  Within a few ulps of g / (1 + expf(-g)) * u: the prompt layer's parity is 1e-3 relative L2,
// and this is the epilogue's dominant cost with the library exp and an IEEE division (~5 vs ~25 instructions)
__device__ __forceinline__ float prompt_swiglu(float g, float u) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504f);
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// the hand-laid LDS of mmq_f16_kernel: the codebooks at address 0 and the arrays read per unit next, so that their
// addresses fit the 16-bit offsets of the LDS instructions; the raw weight slabs and the activation tiles last (the
// compiler would order separate arrays by size, the large ones first)
template <int T, int NW, int NB> struct F16Layout {
    static constexpr bool Q4K = T == TSX_Q4_K, Q80 = T == TSX_Q8_0, XXS = T == TSX_IQ3_XXS;
    static constexpr int TW = rep_table_words<T>();
    static constexpr int TAB = 0, AM = TAB + lds_round((TW > 0 ? TW : 4) * 4);
    static constexpr int SC = AM + lds_round((XXS ? NW : 1) * 8 * 32 * 8);
    static constexpr int UF = SC + lds_round((XXS ? 1 : NW) * 8 * 32 * 4);
    static constexpr int RW = UF + lds_round((Q4K || Q80 ? NW : 1) * 8 * 32 * 4);
    static constexpr int DW = RW + lds_round(NW * 32 * 4);
    static constexpr int RHO = DW + lds_round(NW * 32 * 4);
    static constexpr int BN = bn_of<T>();
    static constexpr int RS = BN / 16 == 8 ? 12 : BN / 16;  // floats per (unit, lane token) of the ratio array
    static constexpr int DL = RHO + lds_round(NB * 8 * 16 * RS * 4);
    static constexpr int DM = DL + lds_round(BN * 4);
    static constexpr int SCAN = DM + lds_round((Q4K ? NB * 8 * (BN + 16) : 1) * 4);
    static constexpr int DR = SCAN + lds_round((NW + 1) * 8);
    static constexpr int RAW = DR + lds_round(BN * 4);
    static constexpr int TB = RAW + lds_round(NW * 32 * raw_stride<T>());
    static constexpr int BYTES = TB + NB * BN * kBStride * 2;
};
template <int T, int NW> constexpr int f16_buffers() {
    return T == TSX_Q4_K && NW == 4 ? 1 : F16Layout<T, NW, 2>::BYTES <= 150 * 1024 ? 2 : 1;
}

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
// four bytes in [0, 15] times the pair sc -> two fp16 pairs: (1024 + b) * sc - 1024 * sc, exact only as one fused
// multiply-add (the product alone, up to 1039 * 63, would round in fp16), so the fma is explicit rather than left to
// contraction
__device__ __forceinline__ void nib_to_h(uint32_t w, h2 sc, h2 nsc, uint32_t& lo, uint32_t& hi) {
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u));
    const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u));
    lo = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, sc, nsc));
    hi = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, sc, nsc));
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
template <int NT, typename V>
__device__ __forceinline__ V block_scan(V v, V* s_wave, V& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    V inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const V t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    V off = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        off += w < wave ? s_wave[w] : 0;
        total += s_wave[w];
    }
    return off + inc - v;
}

// FUSE: the gate/up product with SwiGLU and the Q8_1 of h fused in (NW = nw_of<T>()).  Block bx takes h columns
// [16 NW bx, 16 NW bx + 16 NW): wave w multiplies gate rows 16 NW bx + 16 w + [0, 16) (its first 16-row tile) and the
// up rows n_ff further (its second), so that each lane holds matching gate and up outputs; the activation rows are
// xids[sorted row] of P (sorted row r itself when xids is null); h leaves as Q8_1 planes H, one row per sorted row.
template <int T, int NW, bool FUSE = false, int CP = 1>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) mmq_f16_kernel(const uint8_t* __restrict__ w, uint64_t expert_bytes,
                                                          uint64_t row_bytes, int w_cols, int n_exp, MmqPlanes P,
                                                          const int32_t* __restrict__ bounds,
                                                          const int32_t* __restrict__ ids, float* __restrict__ dst,
                                                          int64_t ld_dst, const int32_t* __restrict__ xids = nullptr,
                                                          MmqPlanes H = MmqPlanes{}, int n_ff = 0, int tpg = 0) {
    constexpr int NT = 64 * NW, BM = 32 * NW, NB = f16_buffers<T, NW>(), kBN = bn_of<T>();
    constexpr int CB = chunk_bytes<T>(), RS = raw_stride<T>(), PR = RS / 16, RW = (32 * PR + 63) / 64;
    constexpr int BP = kBN * 16 / NT, EPT = kMaxExpertsMmq / NT;
    constexpr int TC = tab_copies<T>(), TW = rep_table_words<T>(), GW = half_grid_words<T>(), TPT = (TW + NT - 1) / NT;
    constexpr bool Q4K = T == TSX_Q4_K, Q80 = T == TSX_Q8_0, IQ3S = T == TSX_IQ3_S;
    constexpr int XXS = T == TSX_IQ3_XXS;
    static_assert(kBN <= NT, "one thread per token stages the token's scales");
    using L = F16Layout<T, NW, NB>;
    __shared__ __attribute__((aligned(16))) uint8_t s_lds[L::BYTES];
    auto& s_tab = *reinterpret_cast<uint32_t(*)[TW > 0 ? TW : 4]>(s_lds + L::TAB);
    auto& s_am = *reinterpret_cast<uint2(*)[XXS ? NW : 1][8][32]>(s_lds + L::AM);  // IQ3_XXS: aux word, scale pair
    auto& s_sc = *reinterpret_cast<uint32_t(*)[XXS ? 1 : NW][8][32]>(s_lds + L::SC);  // scale pair (Q8_0: 0/1 mask)
    auto& s_uf = *reinterpret_cast<float(*)[Q4K || Q80 ? NW : 1][8][32]>(s_lds + L::UF);  // Q4_K: dmin m / w'; Q8_0: ratio
    auto& s_rw = *reinterpret_cast<float(*)[NW][32]>(s_lds + L::RW);  // row ratio at the chunk's first unit
    auto& s_dw = *reinterpret_cast<float(*)[NW][32]>(s_lds + L::DW);  // the row's scale w' so far
    // token ratio per unit, [unit][token % 16][token / 16]: a lane reads the ratios of its 8 (4) tokens 16 apart
    // with two (one) 16-byte reads, the 16 tokens of a lane group on distinct banks (rows of 12 floats when 8 are
    // used)
    auto& s_rho = *reinterpret_cast<float(*)[NB][8][16][L::RS]>(s_lds + L::RHO);
    float* const s_dl = reinterpret_cast<float*>(s_lds + L::DL);             // the token's D' so far
    // Q4_K min-term factors: rows of kBN + 16 floats, so that lane groups 0 and 1 (units 4 h, 4 h + 1) of one
    // 32-lane half read different banks
    auto& s_dm = *reinterpret_cast<float(*)[Q4K ? NB : 1][8][Q4K ? kBN + 16 : 1]>(s_lds + L::DM);
    uint64_t* const s_scan = reinterpret_cast<uint64_t*>(s_lds + L::SCAN);
    int& s_x = reinterpret_cast<int*>(s_scan + NW)[0];
    int& s_tile0 = reinterpret_cast<int*>(s_scan + NW)[1];
    int* const s_drow = reinterpret_cast<int*>(s_lds + L::DR);  // the output row of each token of the tile
    auto& s_raw = *reinterpret_cast<uint8_t(*)[NW][32 * RS]>(s_lds + L::RAW);
    auto& tB = *reinterpret_cast<_Float16(*)[NB][kBN * kBStride]>(s_lds + L::TB);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Which (column block bx, token tile by), set once the tiles are counted (step 1): workgroups go to the 8 XCDs in
    // turn by their linear index, so with tpg > 0 the s-th block to reach XCD x takes item ((s / G) * 8 + x) * G +
    // s % G of the (tile-major) items, G = gridDim.x * tpg: runs of tpg consecutive tiles, all their column blocks,
    // share an XCD and its L2 (a tile's activation rows serve every column block, and an expert's weights its next
    // tiles), while the runs still come in tile order over the whole chip.  The map is a bijection on each 8 G
    // items, and applies to the whole rounds of 8 G items that full tiles fill.
    int bx = blockIdx.x, by = blockIdx.y;
    const int lr = lane & 15, g = lane >> 4;
    // this lane's copy of the codebooks (grid words, then sign entries)
    const uint32_t* const gtab = &s_tab[0] + 2 * (lane % TC);
    const uint32_t* const stab = &s_tab[0] + GW * TC + 4 * (lane % TC);

    // 1. which expert and which of its token tiles: EPT experts per thread, a block scan of tile counts.  Tiles are
    // numbered by their length, longest first, so that the hardware dispatches the long blocks first and the short
    // ones fill the end of the launch: the full tiles of every expert (expert order), then the partial last tiles of
    // more than kBN / 2 rows, of more than kBN / 4, and the shorter ones.  Counts travel packed in four 16-bit fields
    // (a total is at most gridDim.y < 2^16)
    uint64_t tc[EPT], mine = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int x = EPT * tid + e;
        const int b0 = bounds[min(x, n_exp)], b1 = bounds[min(x + 1, n_exp)];
        const int rows = x < n_exp ? b1 - b0 : 0, rest = rows % kBN;
        const int cl = rest > kBN / 2 ? 1 : rest > kBN / 4 ? 2 : 3;  // the partial tile's field
        tc[e] = (uint64_t) (rows / kBN) | (uint64_t) (rest > 0) << (16 * cl);
        mine += tc[e];
    }
    uint64_t total;
    uint64_t start = block_scan<NT>(mine, s_scan, total);
    const int nfull = (int) (total & 0xFFFF);
    // the XCD order over the whole rounds of full tiles; the rest (the last full tiles and the partial
    // tiles, one per expert, whose weights no other tile shares) in linear order, longest first over the whole chip
    if (tpg > 0) {
        const int nbx = (int) gridDim.x, lin = bx + nbx * by, G = nbx * tpg;
        if (lin < nfull / (8 * tpg) * 8 * G) {
            const int xcd = lin & 7, sx = lin >> 3;
            const int item = ((sx / G) * 8 + xcd) * G + sx % G;
            bx = item % nbx;
            by = item / nbx;
        }
    }
    // the tile's class (0 full, 1-3 partial) and its index among the class's tiles
    int cls = 0, want = by;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int n = (int) (total >> (16 * k) & 0xFFFF);
        if (cls == k && want >= n) {
            want -= n;
            ++cls;
        }
    }
    if (cls == 4) return;  // the whole block: fewer tiles than the grid's upper bound
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int s0 = (int) (start >> (16 * cls) & 0xFFFF), n = (int) (tc[e] >> (16 * cls) & 0xFFFF);
        if (s0 <= want && want < s0 + n) {
            s_x = EPT * tid + e;
            s_tile0 = cls > 0 ? (int) (tc[e] & 0xFFFF) : want - s0;  // the tile's index within its expert
        }
        start += tc[e];
    }
    __syncthreads();
    const int x = s_x;
    const int row0 = bounds[x] + s_tile0 * kBN;
    const int nrows = min(kBN, bounds[x + 1] - row0);
    const int ntt = (nrows + 15) >> 4;  // 16-token MFMA tiles with rows in them
    const int wrow = FUSE ? (BM / 2) * bx + 16 * wave : bx * CP * BM + 32 * wave;
    const uint8_t* wbase = w + (uint64_t) x * expert_bytes + (uint64_t) wrow * row_bytes;
    // byte offset of the wave's row r (0-31) from wbase: FUSE rows 16-31 are the up rows of rows 0-15
    auto roff = [&](int r) -> uint64_t {
        return FUSE ? (uint64_t) ((r & 15) + (r >= 16 ? n_ff : 0)) * row_bytes : (uint64_t) r * row_bytes;
    };
    // where row r's chunk c starts in its slab row: the block's offset within its first 16-byte piece (0 for the
    // formats whose chunks are whole pieces: the base, expert and row strides are multiples of 16)
    auto slab_off = [&](int r, int c) -> int {
        if constexpr (chunk_aligned<T>()) return 0;
        else return (int) ((roff(r) + (uint64_t) c * CB) & 15);
    };
    const int nu = w_cols / 32, nchunks = w_cols / kChunk;
    // the activation rows this thread loads (the same every chunk): rows past the tile's last take its last row
    int32_t arow_b[BP];  // row indices (32-bit: widened where the addresses are formed)
#pragma unroll
    for (int h = 0; h < BP; ++h) {
        const int r = row0 + min((tid + NT * h) >> 4, nrows - 1);
        arow_b[h] = xids ? xids[r] : r;
    }
    // thread tid < kBN stages token tid's scales (tokens past the tile's last take its last row's)
    int32_t arow_s;
    {
        const int r = row0 + min(tid, nrows - 1);
        arow_s = xids ? xids[r] : r;
    }

    // chunk c in flight: this wave's raw weight pieces, the block's share of activation codes, and (threads below
    // kBN) a token's eight block scales (Q4_K: and code sums)
    v4i rw[RW], av[BP];
    float4 ad[2];
    int4 am4[2];
    auto fetch = [&](int v) {
        const int pass = CP > 1 ? v / nchunks : 0, c = v - pass * nchunks;
        const uint8_t* wb = wbase + (uint64_t) pass * BM * row_bytes;  // BM rows further per column pass
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int q = min(lane + 64 * i, 32 * PR - 1), r = q / PR, pc = q - r * PR;
            const uint64_t o = roff(r) + (uint64_t) c * CB;
            const int need = (int) (((o & 15) + CB + 15) / 16);  // pieces that start before the block's end
            rw[i] = __builtin_nontemporal_load((const v4i*) (wb + (o & ~(uint64_t) 15)) + min(pc, need - 1));
        }
#pragma unroll
        for (int h = 0; h < BP; ++h) {
            const int pi = tid + NT * h, q = pi & 15;
            av[h] = *(const v4i*) (P.q + (int64_t) arow_b[h] * P.cols + kChunk * c + 16 * q);
        }
        if (tid < kBN) {
            const float4* dp = (const float4*) (P.d + (int64_t) arow_s * nu + 8 * c);
            ad[0] = dp[0];
            ad[1] = dp[1];
            if constexpr (Q4K) {
                const int4* mp = (const int4*) (P.m + (int64_t) arow_s * nu + 8 * c);
                am4[0] = mp[0];
                am4[1] = mp[1];
            }
        }
    };
    // The outputs are accumulated in the scale of the current unit: before unit u's products are added, the
    // accumulator is multiplied by D'(u-1) / D'(u) for its token and, at a chunk's first unit, w'(c-1) / w'(c) for
    // its row (D' the token's Q8_1 scale of the unit, w' the row's float scale of the chunk; a zero scale takes the
    // last nonzero one, its codes or weights contributing zero), and the result is multiplied by the last D' and w'
    // at the end.  Scales are fp16 values, so every ratio lies in [2^-40, 2^40] and the accumulator stays far from
    // overflow.  Here: the token's ratios for the chunk's eight units, D' after them, and (Q4_K) the min term's
    // activation factor dx * (code sum) / D'(the chunk's last unit).
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
        if (tid < kBN) {
            const float d8[8] = {ad[0].x, ad[0].y, ad[0].z, ad[0].w, ad[1].x, ad[1].y, ad[1].z, ad[1].w};
            float prev = s_dl[tid], rho[8], dn8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float dn = d8[u] != 0.f ? d8[u] : prev;
                rho[u] = prev * __builtin_amdgcn_rcpf(dn);  // within 2 ulp: the ratios only need to chain
                dn8[u] = dn;
                prev = dn;
            }
            s_dl[tid] = prev;
#pragma unroll
            for (int u = 0; u < 8; ++u) s_rho[buf][u][tid & 15][tid >> 4] = rho[u];
            if constexpr (Q4K) {
                const int m8[8] = {am4[0].x, am4[0].y, am4[0].z, am4[0].w, am4[1].x, am4[1].y, am4[1].z, am4[1].w};
                float mf[8];
                const float rp = __builtin_amdgcn_rcpf(prev);
#pragma unroll
                for (int u = 0; u < 8; ++u) mf[u] = d8[u] * (float) m8[u] * rp;
#pragma unroll
                for (int u = 0; u < 8; ++u) s_dm[buf][u][tid] = mf[u];
            }
            (void) dn8;
        }
    };

    uint32_t tw[TPT > 0 ? TPT : 1];
    if constexpr (TW > 0) {
        const uint32_t* src = T == TSX_IQ3_XXS ? kHalf.xxs : kHalf.s;
        const uint32_t* sgn = T == TSX_IQ3_XXS ? kHalf.xxs_sign : kHalf.s_sign;
#pragma unroll
        for (int k = 0; k < TPT; ++k) {
            // word i of the copies: grid words first (entry, copy, word of two), then the sign entries (of four)
            const int i = min(tid + NT * k, TW - 1), j = i - GW * TC;
            tw[k] = j < 0 ? src[2 * (i / (2 * TC)) + (i & 1)] : sgn[4 * (j / (4 * TC)) + (j & 3)];
        }
    }
    if (tid < kBN) s_dl[tid] = 1.0f;   // read back only by the same thread (stage)
    // the tile's output rows, requested now rather than in the epilogue, where each token tile's row lookup would
    // wait for its own round trip before that tile's stores (the block barriers before the epilogue order these)
    if (!FUSE && tid < kBN) s_drow[tid] = ids ? ids[row0 + min(tid, nrows - 1)] : row0 + tid;
    if (lane < 32) s_dw[wave][lane] = 1.0f;  // read back only by the same wave (the row factors)
    fetch(0);
    if constexpr (TW > 0) {
#pragma unroll
        for (int k = 0; k < TPT; ++k)
            if (tid + NT * k < TW) s_tab[tid + NT * k] = tw[k];
    }
    stage(0);
    __syncthreads();

    // the chunk loop, specialised on the number of 16-token tiles that hold rows (no per-tile branches inside)
    auto run = [&](auto ntt_c) {
        constexpr int NTT = decltype(ntt_c)::value;
        float acc[2][NTT][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][tj][i] = 0.f;

        // to the outputs' scale: the row's last w' and the token's last D'
        auto to_scale = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float4 w4 = *(const float4*) &s_dw[wave][16 * t + 4 * g];
                const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) {
                    const float dl = s_dl[16 * tj + lr];
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][tj][i] = acc[t][tj][i] * wv[i] * dl;
                }
            }
        };
        // out: weight row 16 t + 4 g + i of the wave (column pass pass), token 16 tj + lr
        auto out_rows = [&](int pass) __attribute__((always_inline)) {
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj) {
                const int tok = 16 * tj + lr;
                if (tok < nrows) {
                    const int64_t drow = s_drow[tok];
                    float* o = dst + drow * ld_dst + (int64_t) (bx * CP + pass) * BM + 32 * wave + 4 * g;
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[16 * t + i] = acc[t][tj][i];
                }
            }
        };
        for (int v = 0; v < CP * nchunks; ++v) {
            const int pass = CP > 1 ? v / nchunks : 0, c = v - pass * nchunks;
            const int buf = NB == 2 ? (v & 1) : 0;
            const _Float16* B = tB[buf];
            const uint8_t* slab = s_raw[wave];
            const lds_ptr<const v4i> bq = lds_base<v4i>(B + lr * kBStride + 8 * g);  // this lane's activation pieces
            // the wave's rows: the chunk's row scale w' and ratio, and the per-unit integer scales (lane = row r,
            // units 4 hl .. 4 hl + 3); a zero row scale zeroes the row's weights for the chunk
            {
                const int r = lane & 31, hl = lane >> 5;
                const uint8_t* b = slab + r * RS + slab_off(r, c);
                const float wold = s_dw[wave][r];
                if constexpr (T == TSX_IQ3_XXS || IQ3S || Q4K) {
                    // Q4_K: d and dmin in one aligned word
                    const uint32_t dd = Q4K ? ld32(b) : ld16(b);
                    const float d = h2f((uint16_t) dd);
                    const float dw = XXS ? 0.25f * d : d;
                    const float wn = dw != 0.f ? dw : wold;
                    const bool live = dw != 0.f;
                    const uint32_t keep = 0u - (uint32_t) live;  // a mask: the compiler would branch on live
                    // the hardware reciprocal: the ratios only need to chain (the last w' multiplies the result), and
                    // each is within 2 ulp of the quotient
                    const float rwn = __builtin_amdgcn_rcpf(wn);
                    if (hl == 0) {
                        s_rw[wave][r] = wold * rwn;
                        s_dw[wave][r] = wn;
                    }
                    if constexpr (T == TSX_IQ3_XXS) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int j = 4 * hl + k;
                            const uint32_t aux = ld32a2(b + 66 + 4 * j);
                            s_am[wave][j][r] = uint2{aux, hpair(2 * (aux >> 28) + 1) & keep};
                        }
                    } else if constexpr (IQ3S) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int j = 4 * hl + k;
                            s_sc[wave][j][r] = hpair(2 * ((b[106 + (j >> 1)] >> (4 * (j & 1))) & 15u) + 1) & keep;
                        }
                    } else {
                        const float dmin = h2f((uint16_t) (dd >> 16)), dr = dmin * rwn;
                        // the 12 scale bytes as three aligned words; sub-blocks 4 hl + k: scale byte k of SC, min
                        // byte k of M (sub-blocks 0-3: the low 6 bits of bytes 0-3 and 4-7; 4-7: the nibbles of bytes
                        // 8-11 with the top 2 bits of bytes 0-3 and 4-7 above them)
                        // (selected with masks: the compiler would otherwise branch on the lane's half)
                        const uint32_t w0 = ld32(b + 4), w1 = ld32(b + 8), w2 = ld32(b + 12);
                        const uint32_t lo = 0u - (uint32_t) (hl == 0);
                        const uint32_t SC = (w0 & 0x3F3F3F3Fu & lo) |
                                            (((w2 & 0x0F0F0F0Fu) | ((w0 >> 2) & 0x30303030u)) & ~lo);
                        const uint32_t M = (w1 & 0x3F3F3F3Fu & lo) |
                                           ((((w2 >> 4) & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u)) & ~lo);
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int j = 4 * hl + k;
                            s_sc[wave][j][r] = hpair((SC >> (8 * k)) & 255u) & keep;
                            s_uf[wave][j][r] = dr * (float) ((M >> (8 * k)) & 255u);
                        }
                    }
                } else {  // Q8_0: a float scale per unit, its ratio applied at every unit
                    if (hl == 0) {
                        float wv = wold;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const float d = h2f((uint16_t) ld16(b + 34 * j));
                            const float wn = d != 0.f ? d : wv;
                            s_uf[wave][j][r] = wv * __builtin_amdgcn_rcpf(wn);
                            s_sc[wave][j][r] = d != 0.f ? 0x3C003C00u : 0u;
                            wv = wn;
                        }
                        s_dw[wave][r] = wv;
                    }
                }
            }
            wave_lds_order();
            // the lane's decode rows (one per 16-row tile)
            const uint8_t* blk[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int r = 16 * t + lr;
                blk[t] = slab + r * RS + slab_off(r, c);
            }
            // unit u's weight fragments (rows 16 t + lr, values 8 g .. 8 g + 7 of the unit), in two halves: raw()
            // reads the unit's indices and scales (the slab and the per-unit arrays), expand() looks the codebooks up
            // and forms the fp16 fragments, so that a unit's indices can be requested ahead of the products they
            // would otherwise wait behind
            struct Raw {
                uint32_t a[2][3];
            };
            auto raw = [&](int u, Raw& R) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint8_t* b = blk[t];
                    const int r = 16 * t + lr;
                    if constexpr (T == TSX_IQ3_XXS) {
                        const uint2 am = s_am[wave][u][r];
                        R.a[t][0] = ld16(b + 2 + 8 * u + 2 * g);
                        R.a[t][1] = am.x;  // aux word: scale and sign indices
                        R.a[t][2] = am.y;  // the scale pair
                    } else if constexpr (IQ3S) {
                        R.a[t][0] = ld16(b + 2 + 8 * u + 2 * g) | ((uint32_t) b[66 + u] >> (2 * g)) << 16;
                        R.a[t][1] = b[74 + 4 * u + g];
                        R.a[t][2] = s_sc[wave][u][r];
                    } else if constexpr (Q4K) {
                        const uint2 q = *(const uint2*) (b + 16 + 32 * (u >> 1) + 8 * g);  // 8-byte aligned
                        R.a[t][0] = q.x;
                        R.a[t][1] = q.y;
                        R.a[t][2] = s_sc[wave][u][r];
                    } else {
                        const uint8_t* q = b + 34 * u + 2 + 8 * g;
                        R.a[t][0] = ld32a2(q);
                        R.a[t][1] = ld32a2(q + 4);
                        R.a[t][2] = s_sc[wave][u][r];
                    }
                }
            };
            auto expand = [&](int u, const Raw& R, v4i (&A)[2]) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    uint32_t f[4];
                    if constexpr (T == TSX_IQ3_XXS) {
                        const uint32_t qp = R.a[t][0], aux = R.a[t][1], m = R.a[t][2];
                        const uint2 g0 = *(const uint2*) (gtab + 2 * TC * (qp & 255u));
                        const uint2 g1 = *(const uint2*) (gtab + 2 * TC * (qp >> 8));
                        const uint4 sm = *(const uint4*) (stab + 4 * TC * ((aux >> (7 * g)) & 127u));
                        f[0] = hmul(g0.x ^ sm.x, m);
                        f[1] = hmul(g0.y ^ sm.y, m);
                        f[2] = hmul(g1.x ^ sm.z, m);
                        f[3] = hmul(g1.y ^ sm.w, m);
                    } else if constexpr (IQ3S) {
                        const uint32_t qp = R.a[t][0] & 0xFFFFu, qh = R.a[t][0] >> 16, m = R.a[t][2];
                        const uint32_t i0 = (qp & 255u) | (qh & 1u) << 8, i1 = (qp >> 8) | (qh & 2u) << 7;
                        const uint2 g0 = *(const uint2*) (gtab + 2 * TC * i0);
                        const uint2 g1 = *(const uint2*) (gtab + 2 * TC * i1);
                        const uint4 sm = *(const uint4*) (stab + 4 * TC * R.a[t][1]);
                        f[0] = hmul(g0.x ^ sm.x, m);
                        f[1] = hmul(g0.y ^ sm.y, m);
                        f[2] = hmul(g1.x ^ sm.z, m);
                        f[3] = hmul(g1.y ^ sm.w, m);
                    } else if constexpr (Q4K) {
                        const int sh = 4 * (u & 1);
                        const uint32_t w0 = (R.a[t][0] >> sh) & 0x0F0F0F0Fu, w1 = (R.a[t][1] >> sh) & 0x0F0F0F0Fu;
                        const h2 sc = __builtin_bit_cast(h2, R.a[t][2]);
                        const h2 nsc = sc * (_Float16) -1024.0f;
                        nib_to_h(w0, sc, nsc, f[0], f[1]);
                        nib_to_h(w1, sc, nsc, f[2], f[3]);
                    } else {
                        const uint32_t m = R.a[t][2];
                        i8_to_h(R.a[t][0], f[0], f[1]);
                        i8_to_h(R.a[t][1], f[2], f[3]);
#pragma unroll
                        for (int k = 0; k < 4; ++k) f[k] = hmul(f[k], m);
                    }
                    A[t] = v4i{(int) f[0], (int) f[1], (int) f[2], (int) f[3]};
                }
            };
            auto decode = [&](int u, v4i (&A)[2]) {
                Raw R;
                raw(u, R);
                expand(u, R, A);
            };
            // unit u: every accumulator to the unit's scale (ROW: with the rows' ratios, rows 16 t + 4 g + i), then
            // the unit's products (weight fragments Af) added in place, token tile by token tile (each tile's
            // activation fragment and ratio read just before its products); NEXT: then the next unit's weights are
            // decoded into Af
            auto step = [&](int u, v4i (&Af)[2], auto row_c, auto next_c) {
                constexpr bool ROW = decltype(row_c)::value;
                float rr[2][4];
                if constexpr (ROW) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const float4 v = Q80 ? *(const float4*) &s_uf[wave][u][16 * t + 4 * g]
                                             : *(const float4*) &s_rw[wave][16 * t + 4 * g];
                        rr[t][0] = v.x;
                        rr[t][1] = v.y;
                        rr[t][2] = v.z;
                        rr[t][3] = v.w;
                    }
                }
                // NEXT (Q4_K, whose registers allow it): the next unit's raw words, requested ahead of this unit's
                // products
                Raw Rn;
                if constexpr (decltype(next_c)::value && Q4K) {
                    if (u + 1 < 8) raw(u + 1, Rn);
                }
                float4 rv[(NTT + 3) / 4];
#pragma unroll
                for (int q = 0; q < (NTT + 3) / 4; ++q) rv[q] = *(const float4*) &s_rho[buf][u][lr][4 * q];
                // the unit's products at raised wave priority, so that they issue back to back while the SIMD's
                // other wave decodes
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) {
                    const v4i bf = bq[(tj * 16 * kBStride + 32 * u) / 8];
                    const float rh = rv[tj >> 2][tj & 3];
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        v4f C;
#pragma unroll
                        for (int i = 0; i < 4; ++i) C[i] = acc[t][tj][i] * (ROW ? rh * rr[t][i] : rh);
                        const v4f D = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, Af[t]),
                                                                            __builtin_bit_cast(v8h, bf), C, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[t][tj][i] = D[i];
                    }
                }
                __builtin_amdgcn_s_setprio(0);
                if constexpr (decltype(next_c)::value) {
                    if constexpr (Q4K) {
                        if (u + 1 < 8) expand(u + 1, Rn, Af);
                    } else {
                        if (u + 1 < 8) decode(u + 1, Af);
                    }
                }
            };
            using No = std::integral_constant<bool, false>;
            using Yes = std::integral_constant<bool, true>;
            // (Q8_0's wider raw rows leave no registers for it, nor IQ3_S's fused launch beyond 2 tiles)
            if constexpr (NTT <= (Q80 ? 0 : IQ3S && FUSE ? 2 : kUpfrontTiles)) {
                // few token tiles: each unit's products are too short to cover its decode's chain of dependent
                // LDS reads, so the units are decoded kUpfrontUnits at a time, their lookups in flight together (the
                // registers are there: the kernel's allocation is set by the 8-tile path)
                constexpr int UG = kUpfrontUnits;
                v4i Au[UG][2];
#pragma unroll
                for (int h = 0; h < 8 / UG; ++h) {
#pragma unroll
                    for (int k = 0; k < UG; ++k) decode(UG * h + k, Au[k]);
                    if (h == 0) {
                        step(0, Au[0], Yes{}, No{});
                        if (v + 1 < CP * nchunks) fetch(v + 1);
                    }
#pragma unroll
                    for (int k = h == 0 ? 1 : 0; k < UG; ++k)
                        step(UG * h + k, Au[k], std::integral_constant<bool, Q80>{}, No{});
                }
            } else {
                v4i A[2];
                decode(0, A);
                step(0, A, Yes{}, Yes{});
                // the next chunk's loads, issued behind the first unit's products rather than in a burst between
                // barriers (the vector memory path takes ~0.7 us to accept a chunk's 72 KB)
                if (v + 1 < CP * nchunks) fetch(v + 1);
#pragma unroll 1
                for (int u = 1; u < 8; ++u) {
                    if constexpr (Q80) step(u, A, Yes{}, Yes{});
                    else step(u, A, No{}, Yes{});
                }
            }
            if constexpr (Q4K) {
                // the chunk's min term in the chunk's last scale: sum over units u of -(dmin m / w')[row][u] *
                // (dx s / D'_7)[token][u], a [rows x 8] by [8 x tokens] product on the fp32 matrix cores (two K = 4
                // steps), rows 16 t + lr by units 4 h + g in A, units by tokens 16 tj + lr in B
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float am[2];
#pragma unroll
                    for (int t = 0; t < 2; ++t) am[t] = -s_uf[wave][4 * h + g][16 * t + lr];
#pragma unroll
                    for (int tj = 0; tj < NTT; ++tj) {
                        const float bm = s_dm[buf][4 * h + g][16 * tj + lr];
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
            if constexpr (CP > 1) {
                if (c == nchunks - 1) {  // the pass's outputs, then the next pass's rows from zero
                    to_scale();
                    out_rows(pass);
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int tj = 0; tj < NTT; ++tj)
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[t][tj][i] = 0.f;
                }
            }
            if (v + 1 < CP * nchunks) {
                // every wave is done with the single activation tile (and, after a pass, with the tokens' D')
                if (NB == 1 || (CP > 1 && c == nchunks - 1)) __syncthreads();
                wave_lds_order();                        // this wave is done with its raw slab and factor rows
                stage(NB == 2 ? (v + 1) & 1 : 0);
                __syncthreads();
            }
        }
        if constexpr (CP == 1) to_scale();
        if constexpr (FUSE) {
#pragma clang fp contract(off)
            // h = silu(gate) * up in registers (lane: h columns 16 w + 4 g + i, tokens 16 tj + lr), the product
            // rounded on its own, then its Q8_1 blocks.  A block's 32 columns are the 16 of waves 2 m and 2 m + 1:
            // each reduces its half of the token's amax and code sum over its four lane groups and the halves meet
            // in LDS (the activation tile's, once every wave is past its last chunk)
            float* s_ex = (float*) &tB[0][0];  // [2][NW][16 NTT]: amax halves, then code-sum halves
            constexpr int EX = 16 * NTT;
            __syncthreads();
            float hv[NTT][4], am[NTT];
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj) {
#pragma unroll
                for (int i = 0; i < 4; ++i) hv[tj][i] = prompt_swiglu(acc[0][tj][i], acc[1][tj][i]);
                float a = fmaxf(fmaxf(fabsf(hv[tj][0]), fabsf(hv[tj][1])), fmaxf(fabsf(hv[tj][2]), fabsf(hv[tj][3])));
                a = fmaxf(a, __shfl_xor(a, 16, 64));
                a = fmaxf(a, __shfl_xor(a, 32, 64));
                am[tj] = a;
                if (g == 0) s_ex[wave * EX + 16 * tj + lr] = a;
            }
            __syncthreads();
            float dd[NTT];
            const int col = (BM / 2) * bx + 16 * wave + 4 * g;
#pragma unroll
            for (int tj = 0; tj < NTT; ++tj) {
                const float amax = fmaxf(am[tj], s_ex[(wave ^ 1) * EX + 16 * tj + lr]);
                const float d = q8_1_scale(amax);
                int qv[4];
                q8_1_codes4(float4{hv[tj][0], hv[tj][1], hv[tj][2], hv[tj][3]}, amax, d, qv);
                float qs = (float) (qv[0] + qv[1] + qv[2] + qv[3]);  // |sum| <= 32 * 127: exact in fp32
                qs += __shfl_xor(qs, 16, 64);
                qs += __shfl_xor(qs, 32, 64);
                if (g == 0) s_ex[NW * EX + wave * EX + 16 * tj + lr] = qs;
                dd[tj] = d;
                const int tok = 16 * tj + lr;
                if (tok < nrows)
                    *(uint32_t*) (H.q + (int64_t) (row0 + tok) * H.cols + col) =
                        ((uint32_t) qv[0] & 0xFFu) | ((uint32_t) qv[1] & 0xFFu) << 8 |
                        ((uint32_t) qv[2] & 0xFFu) << 16 | ((uint32_t) qv[3] & 0xFFu) << 24;
            }
            __syncthreads();
            if ((wave & 1) == 0 && g == 0) {
#pragma unroll
                for (int tj = 0; tj < NTT; ++tj) {
                    const int tok = 16 * tj + lr;
                    if (tok < nrows) {
                        const int64_t hi = (int64_t) (row0 + tok) * (H.cols / 32) + col / 32;
                        const float* sq = s_ex + NW * EX + 16 * tj + lr;
                        const float qs = sq[wave * EX] + sq[(wave + 1) * EX];
                        H.d[hi] = h2f(f2h(q8_1_finite(dd[tj])));
                        H.m[hi] = (int32_t) qs;
                    }
                }
            }
        } else if constexpr (CP == 1) {
            out_rows(0);
        }
    };
    // partial tiles run the next size up in {1, 2, 3, 4, 6, 8} 16-token tiles (the extra ones multiply padding)
    if (ntt == 1) run(std::integral_constant<int, 1>{});
    else if (ntt == 2) run(std::integral_constant<int, 2>{});
    else if (ntt == 3) run(std::integral_constant<int, 3>{});
    else if (kBN == 64 || ntt == 4) run(std::integral_constant<int, 4>{});
    else if (kBN == 96 || ntt <= 6) run(std::integral_constant<int, (kBN >= 96 ? 6 : 4)>{});
    else run(std::integral_constant<int, (kBN >= 128 ? 8 : 4)>{});
}

__global__ void __launch_bounds__(kThreads) mmq_swiglu_kernel(const float* __restrict__ gu, float* __restrict__ h,
                                                              int64_t rows, int64_t n_ff, int interleaved) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n_ff) return;
    const int64_t r = i / n_ff, k = i % n_ff;
    const float* row = gu + r * 2 * n_ff;
    const float g = interleaved ? row[2 * k] : row[k], u = interleaved ? row[2 * k + 1] : row[n_ff + k];
    h[i] = prompt_swiglu(g, u);
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

TSX_API int tsx_moe_mmq_quantize_route(const float* x, void* xq, int type, int64_t cols, int64_t ld, int64_t rows,
                                       const float* logits, int32_t* ids, float* weights, int n_expert, int k,
                                       void* stream) {
    (void) type;  // one layout serves every weight type
    if (n_expert <= 0 || n_expert % 64 != 0 || n_expert > kMaxExpertsMmq || k < 1 || k > 16 || k > n_expert) {
        set_error("tsx_moe_mmq_quantize_route: %d experts / top-%d not supported (a multiple of 64 up to 512, k 1..16)",
                  n_expert, k);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(x && xq && logits && ids && weights && cols > 0 && cols % 32 == 0 && ld >= cols && ld % 4 == 0 &&
                    rows >= 0 && aligned(xq, 256) && aligned(x, 16) && aligned(logits, 4) && aligned(ids, 4) &&
                    aligned(weights, 4),
                "tsx_moe_mmq_quantize_route: x (16-byte aligned, ld a multiple of 4), xq (256-byte aligned), cols a "
                "multiple of 32, logits, ids, weights");
    const MmqPlanes P = planes(xq, rows, cols);
    const int qb = (int) ((rows * (cols / 4) + kThreads - 1) / kThreads);
    const int rb = (int) ((rows + 3) / 4);
    mmq_quantize_route_kernel<<<(unsigned) (qb + kPadBlocks + rb), kThreads, 0, (hipStream_t) stream>>>(
        x, P, cols, ld, rows, qb, rb, logits, ids, weights, n_expert, k);
    return launch_status("tsx_moe_mmq_quantize_route");
}

// runs of kXcdTiles consecutive token tiles per XCD (mmq_f16_kernel's tpg) over the whole rounds of full tiles; the
// tile grid padded to whole rounds of runs over the 8 XCDs, its extra blocks returning at once like the tiles past the
// routing's count.  With every tile in the runs, 2 measured best of 0, 1, 2, 4, 8 (configs[3] gate/up 168 -> 162 us,
// configs[4] 345.5 -> 343 us; 8 lost 10 %); with the partial tiles outside them, 4 against 2: configs[4] gate/up
// 344.5 -> 337.3 us, configs[3] 136.1 -> 135.1 us, and 8 within 1 % of 4
constexpr int kXcdTiles = 4;
inline int64_t xcd_tiles(int64_t tiles) { return (tiles + 8 * kXcdTiles - 1) / (8 * kXcdTiles) * (8 * kXcdTiles); }

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
        const int nw = p->type == TSX_Q4_K && p->w_rows % 128 == 0 ? 4 : p->w_rows % 256 == 0 ? 8 : p->w_rows % 128 == 0 ? 4 : 2;
        return with_type(p->type, [&](auto T) {
            constexpr int TT = decltype(T)::value;
            const int64_t max_tiles = xcd_tiles((p->total_rows + bn_of<TT>() - 1) / bn_of<TT>() + p->n);
            const dim3 grid((unsigned) (p->w_rows / (32 * nw)), (unsigned) max_tiles);
            const uint8_t* w = (const uint8_t*) p->w;
            if (nw == 8 && p->w_cols <= kPassCols && p->w_rows % 512 == 0)
                mmq_f16_kernel<TT, 8, false, 2><<<dim3(grid.x / 2, grid.y), 512, 0, s>>>(
                    w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds, p->ids, p->dst, p->ld_dst, nullptr,
                    MmqPlanes{}, 0, kXcdTiles);
            else if (nw == 8)
                mmq_f16_kernel<TT, 8><<<grid, 512, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst, nullptr, MmqPlanes{}, 0, kXcdTiles);
            else if (nw == 4)
                mmq_f16_kernel<TT, 4><<<grid, 256, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst, nullptr, MmqPlanes{}, 0, kXcdTiles);
            else
                mmq_f16_kernel<TT, 2><<<grid, 128, 0, s>>>(w, p->expert_bytes, rb, (int) p->w_cols, p->n, P, p->bounds,
                                                           p->ids, p->dst, p->ld_dst, nullptr, MmqPlanes{}, 0, kXcdTiles);
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
    return with_type(type, [&](auto T) {
        constexpr int BN = bn_of<decltype(T)::value>();
        const int64_t max_tiles = xcd_tiles((n_rows + BN - 1) / BN + n_exp);
        constexpr int NW = nw_of<decltype(T)::value>();
        const dim3 grid((unsigned) (n_ff / (16 * NW)), (unsigned) max_tiles);
        mmq_f16_kernel<decltype(T)::value, NW, true><<<grid, 64 * NW, 0, s>>>(
            (const uint8_t*) w, expert_bytes, rb, (int) n_embd, n_exp, P, bounds, nullptr, nullptr, 0, xids, H, (int) n_ff,
            kXcdTiles);
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
