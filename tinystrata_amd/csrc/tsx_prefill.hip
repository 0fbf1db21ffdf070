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
    const int lpr = lanes_per_row((int) (p->w_cols / 32)), rows = (kThreads / kWave) * (kWave / lpr);
    return with_type(p->type, [&](auto T) {
        return with_lpr(lpr, [&](auto LPR) {
            const dim3 grid((unsigned) ((p->w_rows + rows - 1) / rows), (unsigned) p->n);
            mmq_rows_kernel<decltype(T)::value, decltype(LPR)::value><<<grid, kThreads, 0, (hipStream_t) stream>>>(
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
