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

// one 32-lane group per Q8_1 block: row i of the output is row ids[i] (or i) of x
__global__ void __launch_bounds__(kThreads) mmq_quantize_kernel(const float* __restrict__ x, const int32_t* __restrict__ ids,
                                                                MmqPlanes P, int64_t cols, int64_t ld, int64_t rows) {
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
    int q = 0;
    if (amax != 0.0f) {
        const float r = roundf(v / d);
        q = (int) (r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r);
    }
    int qs = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) qs += __shfl_xor(qs, o, 32);
    P.q[i * cols + 32 * b + lane] = (int8_t) q;
    if (lane == 0) {
        P.d[i * nb + b] = h2f(f2h(q8_1_finite(d)));
        P.m[i * nb + b] = qs;
    }
}

// zero codes and scales of the padding rows [rows, rows_pad): a tile that over-reads them multiplies zeros
__global__ void mmq_pad_kernel(MmqPlanes P, int64_t rows) {
    const int64_t nb = P.cols / 32;
    const int64_t n_q = (P.rows_pad - rows) * P.cols, n_s = (P.rows_pad - rows) * nb;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n_q; i += (int64_t) gridDim.x * blockDim.x)
        P.q[rows * P.cols + i] = 0;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n_s; i += (int64_t) gridDim.x * blockDim.x) {
        P.d[rows * nb + i] = 0.f;
        P.m[rows * nb + i] = 0;
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

// ------------------------------------------------------------------ grouped product (int8 MFMA)
// Block (weight-row tile bx, token tile by): 64 rows of one expert's matrix against 64 of the expert's sorted token
// rows.  The token tiles of all experts are numbered in expert order (tiles of expert x = ceil(rows_x / 64)); each
// block finds its expert from `bounds` with a block scan, so the launch needs no host-side count.  With
// w_rows / 64 a multiple of 8 every token tile of one weight tile runs on the same XCD (blocks are dealt to the 8
// XCDs round robin), so a weight tile is fetched from HBM once per XCD and then hits that XCD's L2.
//
// K advances one 256-value chunk at a time, software-pipelined: chunk c+1's weight blocks and activation codes are
// loaded into registers while chunk c is multiplied.  A chunk's raw GGUF blocks (one per row) are copied into LDS
// with 16-byte loads aligned down (IQ3 blocks are 98 / 110 bytes: a row's chunk starts at any even offset), decoded
// to int8 (with the per-unit float scales, and for Q4_K the min terms) into a row-padded LDS tile next to the
// chunk's activation codes, and each wave multiplies its 32 x 32 corner with v_mfma_i32_16x16x32_i8: one MFMA per
// 32-value unit, so its int32 result is exactly the unit's integer sum S, scaled in fp32:
// acc += a_w * d_x * S (- b_w * d_x * sum(q_x) for Q4_K).  The scaling costs ~3 VALU operations per output per unit
// against 32 MACs on the matrix core, which is what bounds this kernel's MFMA utilisation.
constexpr int kBM = 64, kBN = 64;
constexpr int kChunk = 256;
constexpr int kTileStride = kChunk + 16;  // LDS bytes per tile row: the padding spreads a wave's 8-byte reads over all banks
constexpr int kMaxExpertsMmq = 512;
typedef int v4i32 __attribute__((ext_vector_type(4)));

template <int T> constexpr int chunk_bytes() { return T == TSX_Q8_0 ? 8 * 34 : Fmt<T>::bytes; }
// LDS bytes per row of a chunk's raw blocks: the block plus up to 15 bytes of alignment in front of it
template <int T> constexpr int raw_stride() { return (chunk_bytes<T>() + 15 + 15) / 16 * 16; }
template <int T> constexpr int raw_loads() { return (kBM * raw_stride<T>() / 16 + 255) / 256; }

// exclusive prefix sum over the 256 threads of the block (v per thread), and the total
__device__ __forceinline__ int block_scan_256(int v, int* s_wave, int& total) {
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
    for (int w = 0; w < wave; ++w) off += s_wave[w];
    total = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
    return off + inc - v;
}

template <int T>
__global__ void __launch_bounds__(256) mmq_mfma_kernel(const uint8_t* __restrict__ w, uint64_t expert_bytes,
                                                       uint64_t row_bytes, int w_cols, int n_exp, MmqPlanes P,
                                                       const int32_t* __restrict__ bounds, const int32_t* __restrict__ ids,
                                                       float* __restrict__ dst, int64_t ld_dst) {
    constexpr int GW = (grid_lds_words<T>() + 255) / 256;
    constexpr int CB = chunk_bytes<T>(), RS = raw_stride<T>(), PR = RS / 16, RL = raw_loads<T>();
    __shared__ __attribute__((aligned(16))) uint8_t s_raw[kBM * RS];
    __shared__ __attribute__((aligned(16))) int8_t tA[kBM * kTileStride], tB[kBN * kTileStride];
    __shared__ __attribute__((aligned(16))) uint32_t s_grid[GW > 0 ? GW * 256 : 4];
    __shared__ __attribute__((aligned(16))) float s_aw[8][kBM], s_bw[8][kBM], s_dx[8][kBN], s_dm[8][kBN];
    __shared__ int s_wave[4], s_x, s_tile0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bx = blockIdx.x, by = blockIdx.y;

    // 1. which expert and which of its token tiles: two experts per thread, a block scan of tile counts
    const int x0 = 2 * tid, x1 = 2 * tid + 1;
    const int b0 = bounds[min(x0, n_exp)], b1 = bounds[min(x1, n_exp)], b2 = bounds[min(x1 + 1, n_exp)];
    const int t0 = x0 < n_exp ? (b1 - b0 + kBN - 1) / kBN : 0, t1 = x1 < n_exp ? (b2 - b1 + kBN - 1) / kBN : 0;
    int total;
    const int start = block_scan_256(t0 + t1, s_wave, total);
    if (by >= total) return;  // the whole block: fewer tiles than the grid's upper bound
    if (start <= by && by < start + t0) { s_x = x0; s_tile0 = start; }
    if (start + t0 <= by && by < start + t0 + t1) { s_x = x1; s_tile0 = start + t0; }
    __syncthreads();
    const int x = s_x;
    const int row0 = bounds[x] + (by - s_tile0) * kBN;
    const int nrows = min(kBN, bounds[x + 1] - row0);
    const uint8_t* wbase = w + (uint64_t) x * expert_bytes + (uint64_t) bx * kBM * row_bytes;
    const int nu = w_cols / 32, nchunks = w_cols / kChunk;

    // chunk c in flight: each row's raw block (the 16-byte pieces that hold it) and the activation codes / scales
    v4i rw[RL], av[4];
    float ad[2];
    int am[2];
    auto fetch = [&](int c) {
#pragma unroll
        for (int i = 0; i < RL; ++i) {
            const int q = min(tid + 256 * i, kBM * PR - 1), r = q / PR, pc = q - r * PR;
            const uint64_t o = (uint64_t) r * row_bytes + (uint64_t) c * CB;
            const int need = (int) (((o & 15) + CB + 15) / 16);  // pieces that start before the block's end
            rw[i] = __builtin_nontemporal_load((const v4i*) (wbase + (o & ~(uint64_t) 15)) + min(pc, need - 1));
        }
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int pi = tid + 256 * h, rr = pi >> 4, q = pi & 15;
            av[h] = *(const v4i*) (P.q + (int64_t) (row0 + rr) * P.cols + kChunk * c + 16 * q);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pi = tid + 256 * h, rr = pi >> 3, u = pi & 7;
            const int64_t o = (int64_t) (row0 + rr) * nu + 8 * c + u;
            ad[h] = P.d[o];
            if constexpr (T == TSX_Q4_K) am[h] = P.m[o];
        }
    };
    uint32_t gw[GW > 0 ? GW : 1];
    if constexpr (GW > 0) grid_fetch<T, GW>(gw, tid, 256);
    fetch(0);
    GridRef grid = grid_const();
    if constexpr (GW > 0) grid = grid_store<T, GW>(s_grid, gw, tid, 256);

    const int wr = wave >> 1, wc = wave & 1;  // the wave's 32 x 32 corner
    const int lr = lane & 15, lg = lane >> 4;
    float acc[2][2][4];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[ti][tj][i] = 0.f;

    for (int c = 0; c < nchunks; ++c) {
        // chunk c from registers into LDS
#pragma unroll
        for (int i = 0; i < RL; ++i)
            if (tid + 256 * i < kBM * PR) ((v4i*) s_raw)[tid + 256 * i] = rw[i];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int pi = tid + 256 * h, rr = pi >> 4, q = pi & 15;
            *(v4i*) (tB + rr * kTileStride + 16 * q) = av[h];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pi = tid + 256 * h, rr = pi >> 3, u = pi & 7;
            s_dx[u][rr] = ad[h];
            if constexpr (T == TSX_Q4_K) s_dm[u][rr] = ad[h] * (float) am[h];
        }
        __syncthreads();
        if (c + 1 < nchunks) fetch(c + 1);
        // decode: 64 rows x 8 units, two per thread
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pr = tid + 256 * h, rr = pr >> 3, u = pr & 7;
            const int off = (int) (((uint64_t) rr * row_bytes + (uint64_t) c * CB) & 15);
            Unit wu;
            unit_load<T>(s_raw + rr * RS + off, u, wu, grid);
            v4i* dA = (v4i*) (tA + rr * kTileStride + 32 * u);
            dA[0] = v4i{wu.w[0], wu.w[1], wu.w[2], wu.w[3]};
            dA[1] = v4i{wu.w[4], wu.w[5], wu.w[6], wu.w[7]};
            s_aw[u][rr] = wu.a;
            if constexpr (T == TSX_Q4_K) s_bw[u][rr] = wu.b;
        }
        __syncthreads();
        // the wave's corner, one MFMA per unit per 16 x 16 tile
#pragma unroll 2
        for (int u = 0; u < 8; ++u) {
            long av8[2], bv8[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                av8[t] = *(const long*) (tA + (32 * wr + 16 * t + lr) * kTileStride + 32 * u + 8 * lg);
                bv8[t] = *(const long*) (tB + (32 * wc + 16 * t + lr) * kTileStride + 32 * u + 8 * lg);
            }
            const float4 aw0 = *(const float4*) &s_aw[u][32 * wr + 4 * lg];
            const float4 aw1 = *(const float4*) &s_aw[u][32 * wr + 16 + 4 * lg];
            const float aws[2][4] = {{aw0.x, aw0.y, aw0.z, aw0.w}, {aw1.x, aw1.y, aw1.z, aw1.w}};
#pragma unroll
            for (int tj = 0; tj < 2; ++tj) {
                const float dx = s_dx[u][32 * wc + 16 * tj + lr];
#pragma unroll
                for (int ti = 0; ti < 2; ++ti) {
                    const v4i32 z = {0, 0, 0, 0};
                    const v4i32 S = __builtin_amdgcn_mfma_i32_16x16x32_i8(av8[ti], bv8[tj], z, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[ti][tj][i] += (aws[ti][i] * dx) * (float) S[i];
                }
                if constexpr (T == TSX_Q4_K) {
                    const float dm = s_dm[u][32 * wc + 16 * tj + lr];
                    const float4 bw0 = *(const float4*) &s_bw[u][32 * wr + 4 * lg];
                    const float4 bw1 = *(const float4*) &s_bw[u][32 * wr + 16 + 4 * lg];
                    const float bws[2][4] = {{bw0.x, bw0.y, bw0.z, bw0.w}, {bw1.x, bw1.y, bw1.z, bw1.w}};
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[ti][tj][i] -= bws[ti][i] * dm;
                }
            }
        }
        __syncthreads();  // the tiles are consumed before the next chunk overwrites them
    }

    // out: row 4 lg + i of tile ti, token lr of tile tj
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
        const int tok = 32 * wc + 16 * tj + lr;
        if (tok < nrows) {
            const int64_t drow = ids ? ids[row0 + tok] : row0 + tok;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    dst[drow * ld_dst + (int64_t) bx * kBM + 32 * wr + 16 * ti + 4 * lg + i] = acc[ti][tj][i];
        }
    }
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
    if (rows > 0) {
        const int64_t threads = rows * (cols / 32) * 32;
        mmq_quantize_kernel<<<(unsigned) ((threads + kThreads - 1) / kThreads), kThreads, 0, s>>>(x, ids, P, cols, ld, rows);
        const int rc = launch_status("tsx_moe_mmq_quantize");
        if (rc != TSX_OK) return rc;
    }
    mmq_pad_kernel<<<64, kThreads, 0, s>>>(P, rows);
    return launch_status("tsx_moe_mmq_quantize/pad");
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
    // the int8-MFMA tiles where the shape fits them, else the row-dot kernel
    if (p->w_cols % kChunk == 0 && p->w_rows % kBM == 0 && p->n <= kMaxExpertsMmq && aligned(p->w, 16) &&
        p->expert_bytes % 16 == 0) {
        const int64_t max_tiles = (p->total_rows + kBN - 1) / kBN + p->n;
        return with_type(p->type, [&](auto T) {
            const dim3 grid((unsigned) (p->w_rows / kBM), (unsigned) max_tiles);
            mmq_mfma_kernel<decltype(T)::value><<<grid, 256, 0, s>>>((const uint8_t*) p->w, p->expert_bytes, rb,
                                                                     (int) p->w_cols, p->n, P, p->bounds, p->ids,
                                                                     p->dst, p->ld_dst);
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

TSX_API int tsx_moe_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream) {
    TSX_REQUIRE(gu && h && rows >= 0 && n_ff > 0, "tsx_moe_mmq_swiglu: gu, h, n_ff > 0");
    if (rows == 0) return TSX_OK;
    const int64_t n = rows * n_ff;
    mmq_swiglu_kernel<<<(unsigned) ((n + kThreads - 1) / kThreads), kThreads, 0, (hipStream_t) stream>>>(gu, h, rows, n_ff,
                                                                                                       interleaved);
    return launch_status("tsx_moe_mmq_swiglu");
}

}  // extern "C"
