// tsx_decode.hip - decode / small-M MoE experts on gfx950: Q8_1 activation quantizers, the grouped expert rows
// (native_expert_grouped), the single-matrix mmvq and the integer-sum check kernel.
//
// Reference: src/kernels/cuda/iq_kernels.cu (grouped driver 2835-2982, gate/up rows 1310-1397, SwiGLU + Q8_1
// 1489-1515, down rows 1407-1465, q8_1 1467-1487, mmvq 716-740); src/kernels/cuda/native_mmvq.cu:154-185.
//
// Layout on the chip: a weight row is split over LPR lanes of a wave64 (LPR = the row's 32-value units rounded
// up to a power of two, at most 64), so a wave reads 64/LPR rows at once; each lane decodes a unit once and
// applies it to every entry of the group (up to NC at a time), then the row's lanes reduce.  A block is 4 waves;
// gate and up rows of the same index lie in the same block row so the whole expert is read once per group.
#include "tsx_common.hpp"
#include "tsx_device.hpp"

namespace tsx {
namespace {

constexpr int kThreads = 256;
constexpr int kNC = 4;  // entries per pass over a row's units

// ------------------------------------------------------------------ Q8_1 quantizers
__global__ void __launch_bounds__(kThreads) quantize_q8_1_kernel(const float* __restrict__ x, tsx_block_q8_1* __restrict__ y,
                                                                 int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;  // n is a multiple of 32: a 32-lane group is in or out as a whole
    q8_1_store32(x[i], y + i / 32, (int) (i & 31));
}

__global__ void __launch_bounds__(kThreads) swiglu_q8_1_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                               tsx_block_q8_1* __restrict__ y, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    const float h = (gv / (1.0f + expf(-gv))) * u[i];
    q8_1_store32(h, y + i / 32, (int) (i & 31));
}

// SwiGLU + Q8_1 over the call's entries [grp_start[0], grp_start[*n_groups]) only
__global__ void __launch_bounds__(kThreads) swiglu_entries_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                                  const int32_t* __restrict__ grp_start,
                                                                  const int32_t* __restrict__ n_groups, int n_ff,
                                                                  tsx_block_q8_1* __restrict__ hq) {
#pragma clang fp contract(off)
    const int64_t lo = (int64_t) grp_start[0] * n_ff, hi = (int64_t) grp_start[*n_groups] * n_ff;
    for (int64_t i = lo + (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += (int64_t) gridDim.x * blockDim.x) {
        const float gv = gate[i];
        const float h = (gv / (1.0f + expf(-gv))) * up[i];
        q8_1_store32(h, hq + i / 32, (int) (i & 31));
    }
}

// ------------------------------------------------------------------ row dots
// acc[c] = row . x[c] for c < n, the row's LPR lanes each taking units l, l + LPR, ...; reduced over the LPR lanes
template <int T, int LPR, int NC>
__device__ __forceinline__ void row_dots(const uint8_t* __restrict__ row, const tsx_block_q8_1* const (&xs)[NC], int n,
                                         int nu, int l, float (&acc)[NC]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.f;
    for (int u = l; u < nu; u += LPR) {
        Unit w;
        unit_load<T>(row, u, w, grid_const());
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (c < n) {
                Act a;
                act_load(xs[c] + u, a);
                int S, M;
                acc[c] += unit_dot<T>(w, a, S, M);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = group_sum<LPR>(acc[c]);
}

// gate and up rows of every group: gate[e][r], up[e][r] for the group's entries e
template <int T, int LPR>
__global__ void __launch_bounds__(kThreads) expert_gu_kernel(const uint64_t* __restrict__ grp_ptr,
                                                             const int32_t* __restrict__ grp_start,
                                                             const int32_t* __restrict__ n_groups,
                                                             const int32_t* __restrict__ ent_tok,
                                                             const tsx_block_q8_1* __restrict__ xq, tsx_expert_layout L,
                                                             float* __restrict__ gate, float* __restrict__ up) {
    constexpr int RPW = kWave / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPR, l = lane % LPR;
    const int FF = (int) L.n_ff, nu = (int) (L.n_embd / 32);
    const int row = (blockIdx.x * (kThreads / kWave) + wave) * RPW + slot;
    const bool valid = row < 2 * FF;
    const bool is_up = valid && row >= FF;
    const int r = is_up ? row - FF : (valid ? row : 0);
    const uint64_t off = (is_up ? L.up_off : 0) + (uint64_t) r * L.gu_row;
    float* dst = is_up ? up : gate;
    const int ng = *n_groups;
    for (int g = blockIdx.y; g < ng; g += gridDim.y) {
        if (!valid) continue;
        const uint8_t* wr = (const uint8_t*) grp_ptr[g] + off;
        const int e0 = grp_start[g], e1 = grp_start[g + 1];
        for (int e = e0; e < e1; e += kNC) {
            const int n = min(kNC, e1 - e);
            const tsx_block_q8_1* xs[kNC];
#pragma unroll
            for (int c = 0; c < kNC; ++c) xs[c] = xq + (int64_t) ent_tok[e + min(c, n - 1)] * nu;
            float acc[kNC];
            row_dots<T, LPR, kNC>(wr, xs, n, nu, l, acc);
            if (l == 0)
                for (int c = 0; c < n; ++c) dst[(int64_t) (e + c) * FF + r] = acc[c];
        }
    }
}

// down rows: out[ent_dst[e]][r] = down_r . hq[e]
template <int T, int LPR>
__global__ void __launch_bounds__(kThreads) expert_down_kernel(const uint64_t* __restrict__ grp_ptr,
                                                               const int32_t* __restrict__ grp_start,
                                                               const int32_t* __restrict__ n_groups,
                                                               const int32_t* __restrict__ ent_dst,
                                                               const tsx_block_q8_1* __restrict__ hq, tsx_expert_layout L,
                                                               float* __restrict__ out) {
    constexpr int RPW = kWave / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPR, l = lane % LPR;
    const int N = (int) L.n_embd, nu = (int) (L.n_ff / 32);
    const int r = (blockIdx.x * (kThreads / kWave) + wave) * RPW + slot;
    const bool valid = r < N;
    const uint64_t off = L.down_off + (uint64_t) (valid ? r : 0) * L.d_row;
    const int ng = *n_groups;
    for (int g = blockIdx.y; g < ng; g += gridDim.y) {
        if (!valid) continue;
        const uint8_t* wr = (const uint8_t*) grp_ptr[g] + off;
        const int e0 = grp_start[g], e1 = grp_start[g + 1];
        for (int e = e0; e < e1; e += kNC) {
            const int n = min(kNC, e1 - e);
            const tsx_block_q8_1* xs[kNC];
#pragma unroll
            for (int c = 0; c < kNC; ++c) xs[c] = hq + (int64_t) (e + min(c, n - 1)) * nu;
            float acc[kNC];
            row_dots<T, LPR, kNC>(wr, xs, n, nu, l, acc);
            if (l == 0)
                for (int c = 0; c < n; ++c) out[(int64_t) ent_dst[e + c] * N + r] = acc[c];
        }
    }
}

// y[c][r] = W[r] . x[c], ncols <= 8 columns
template <int T, int LPR>
__global__ void __launch_bounds__(kThreads) mmvq_kernel(const uint8_t* __restrict__ w, uint64_t row_bytes,
                                                        const tsx_block_q8_1* __restrict__ x, float* __restrict__ y,
                                                        int n_in, int n_out, int ncols) {
    constexpr int RPW = kWave / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPR, l = lane % LPR;
    const int nu = n_in / 32;
    const int r = (blockIdx.x * (kThreads / kWave) + wave) * RPW + slot;
    if (r >= n_out) return;  // whole LPR groups leave together
    const uint8_t* wr = w + (uint64_t) r * row_bytes;
    for (int c0 = 0; c0 < ncols; c0 += kNC) {
        const int n = min(kNC, ncols - c0);
        const tsx_block_q8_1* xs[kNC];
#pragma unroll
        for (int c = 0; c < kNC; ++c) xs[c] = x + (int64_t) (c0 + min(c, n - 1)) * nu;
        float acc[kNC];
        row_dots<T, LPR, kNC>(wr, xs, n, nu, l, acc);
        if (l == 0)
            for (int c = 0; c < n; ++c) y[(int64_t) (c0 + c) * n_out + r] = acc[c];
    }
}

// Several matrices of one format and shape (blockIdx.y = matrix j), one activation column each: y_j[r] = W_j[r] . x_j.
// The matrices come from MatSource: a table indexed on the device (mmvq_ids) or up to 8 pointers (mmvq_slots).
struct IdsSource {
    const void* const* table;
    const int32_t* ids;
    int n_table;
    uint64_t offset;
    const uint8_t* x;
    uint64_t x_stride;
    int x_every;
    float* y;
    uint64_t y_stride;
    __device__ bool at(int j, const uint8_t*& w, const tsx_block_q8_1*& xj, float*& yj) const {
        const int id = ids[j];
        yj = y + (uint64_t) j * y_stride;
        if (id < 0 || id >= n_table) return false;
        w = (const uint8_t*) table[id] + offset;
        xj = (const tsx_block_q8_1*) (x + (uint64_t) (j / x_every) * x_stride);
        return true;
    }
};
struct SlotsSource {
    const void* w[8];
    const void* x[8];
    float* y[8];
    __device__ bool at(int j, const uint8_t*& wj, const tsx_block_q8_1*& xj, float*& yj) const {
        wj = (const uint8_t*) w[j];
        xj = (const tsx_block_q8_1*) x[j];
        yj = y[j];
        return true;
    }
};
template <int T, int LPR, typename Src>
__global__ void __launch_bounds__(kThreads) mmvq_many_kernel(Src src, uint64_t row_bytes, int n_in, int n_out) {
    constexpr int RPW = kWave / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPR, l = lane % LPR;
    const int r = (blockIdx.x * (kThreads / kWave) + wave) * RPW + slot;
    if (r >= n_out) return;  // whole LPR groups leave together
    const uint8_t* w = nullptr;
    const tsx_block_q8_1* xj = nullptr;
    float* yj = nullptr;
    if (!src.at((int) blockIdx.y, w, xj, yj)) {  // an id outside the table: the matrix's outputs are zero
        if (l == 0) yj[r] = 0.f;
        return;
    }
    const tsx_block_q8_1* xs[1] = {xj};
    float acc[1];
    row_dots<T, LPR, 1>(w + (uint64_t) r * row_bytes, xs, 1, n_in / 32, l, acc);
    if (l == 0) yj[r] = acc[0];
}

// the integer contract, one thread per (row, unit)
template <int T>
__global__ void __launch_bounds__(kThreads) subblock_sums_kernel(const uint8_t* __restrict__ w, uint64_t row_bytes,
                                                                 int nu, int64_t n_rows,
                                                                 const tsx_block_q8_1* __restrict__ x, int64_t ncols,
                                                                 int32_t* __restrict__ sums, int32_t* __restrict__ qsums) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * nu) return;
    const int64_t r = i / nu;
    const int u = (int) (i % nu);
    Unit wu;
    unit_load<T>(w + (uint64_t) r * row_bytes, u, wu, grid_const());
    for (int64_t c = 0; c < ncols; ++c) {
        Act a;
        act_load(x + c * nu + u, a);
        int S, M;
        unit_dot<T>(wu, a, S, M);
        if constexpr (T != TSX_Q4_K) {
            M = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) M = dot4(0x01010101, a.q[k], M);
        }
        sums[(r * ncols + c) * nu + u] = S;
        if (qsums) qsums[(r * ncols + c) * nu + u] = M;
    }
}

// ------------------------------------------------------------------ dispatch helpers
int lanes_per_row(int nu) {
    int l = 8;
    while (l < nu && l < 64) l <<= 1;
    return l;
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

// the formats of the single-matrix and id-indexed products
template <typename F>
int with_mmvq_type(int type, F&& f) {
    switch (type) {
        case TSX_Q4_0: return f(std::integral_constant<int, TSX_Q4_0>{});
        case TSX_Q6_K: return f(std::integral_constant<int, TSX_Q6_K>{});
        default: return with_type(type, f);
    }
}

unsigned blocks_for(int64_t n, int per) { return (unsigned) ((n + per - 1) / per); }

template <typename Src>
int launch_many(const char* what, int type, const Src& src, int count, int n_in, int n_out, void* stream) {
    const size_t rb = tsx_row_bytes(type, n_in);
    const int lpr = lanes_per_row(n_in / 32), rows = (kThreads / kWave) * (kWave / lpr);
    return with_mmvq_type(type, [&](auto T) {
        return with_lpr(lpr, [&](auto LPR) {
            const dim3 grid(blocks_for(n_out, rows), (unsigned) count);
            mmvq_many_kernel<decltype(T)::value, decltype(LPR)::value, Src>
                <<<grid, kThreads, 0, (hipStream_t) stream>>>(src, rb, n_in, n_out);
            return launch_status(what);
        });
    });
}


}  // namespace
}  // namespace tsx

using namespace tsx;

extern "C" {

TSX_API int tsx_moe_quantize_q8_1(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream) {
    TSX_REQUIRE(x && y && n_rows >= 0 && n_cols > 0 && n_cols % 32 == 0 && aligned(y, 4),
                "tsx_moe_quantize_q8_1: x, y (4-byte aligned), n_cols a multiple of 32");
    const int64_t n = n_rows * n_cols;
    if (n == 0) return TSX_OK;
    quantize_q8_1_kernel<<<blocks_for(n, kThreads), kThreads, 0, (hipStream_t) stream>>>(x, (tsx_block_q8_1*) y, n);
    return launch_status("tsx_moe_quantize_q8_1");
}

TSX_API int tsx_moe_swiglu_quantize_q8_1(const float* gate, const float* up, int64_t n, void* y, void* stream) {
    TSX_REQUIRE(gate && up && y && n >= 0 && n % 32 == 0 && aligned(y, 4),
                "tsx_moe_swiglu_quantize_q8_1: gate, up, y, n a multiple of 32");
    if (n == 0) return TSX_OK;
    swiglu_q8_1_kernel<<<blocks_for(n, kThreads), kThreads, 0, (hipStream_t) stream>>>(gate, up, (tsx_block_q8_1*) y, n);
    return launch_status("tsx_moe_swiglu_quantize_q8_1");
}

TSX_API int tsx_moe_expert_grouped(const tsx_expert_layout* Lp, const uint64_t* grp_ptr, const int32_t* grp_start,
                                   const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok,
                                   int64_t cap_groups, int64_t cap_entries, const void* x_q8_1, void* scratch,
                                   float* out, void* stream, int64_t grid_groups) {
    TSX_REQUIRE(Lp != nullptr, "tsx_moe_expert_grouped: null layout");
    const tsx_expert_layout L = *Lp;
    if (cap_groups <= 0 || cap_entries <= 0) return TSX_OK;
    if (!tsx_moe_expert_supported(L.gu_type, L.d_type, L.n_embd, L.n_ff)) {
        set_error("tsx_moe_expert_grouped: types (%d, %d) at %lld x %lld not supported", L.gu_type, L.d_type,
                  (long long) L.n_embd, (long long) L.n_ff);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(grp_ptr && grp_start && n_groups && ent_dst && ent_tok && x_q8_1 && scratch && out,
                "tsx_moe_expert_grouped: a null pointer");
    TSX_REQUIRE(aligned(scratch, 256) && aligned(x_q8_1, 4) && aligned(out, 4),
                "tsx_moe_expert_grouped: scratch must be 256-byte aligned, x and out 4-byte aligned");
    const hipStream_t s = (hipStream_t) stream;
    const size_t f = (size_t) cap_entries * (size_t) L.n_ff * sizeof(float), fa = (f + 255) & ~(size_t) 255;
    float* gate = (float*) scratch;
    float* up = (float*) ((uint8_t*) scratch + fa);
    tsx_block_q8_1* hq = (tsx_block_q8_1*) ((uint8_t*) scratch + 3 * fa);
    const auto* X = (const tsx_block_q8_1*) x_q8_1;
    const int64_t gy = (grid_groups <= 0 || grid_groups > cap_groups) ? cap_groups : grid_groups;

    const int lpr_gu = lanes_per_row((int) (L.n_embd / 32)), lpr_d = lanes_per_row((int) (L.n_ff / 32));
    const int rows_gu = (kThreads / kWave) * (kWave / lpr_gu), rows_d = (kThreads / kWave) * (kWave / lpr_d);
    int rc = with_type(L.gu_type, [&](auto T) {
        return with_lpr(lpr_gu, [&](auto LPR) {
            const dim3 grid(blocks_for(2 * L.n_ff, rows_gu), (unsigned) gy);
            expert_gu_kernel<decltype(T)::value, decltype(LPR)::value>
                <<<grid, kThreads, 0, s>>>(grp_ptr, grp_start, n_groups, ent_tok, X, L, gate, up);
            return launch_status("tsx_moe_expert_grouped/gate-up");
        });
    });
    if (rc != TSX_OK) return rc;
    {
        const int64_t nh = cap_entries * L.n_ff;
        swiglu_entries_kernel<<<blocks_for(nh, kThreads), kThreads, 0, s>>>(gate, up, grp_start, n_groups, (int) L.n_ff, hq);
        rc = launch_status("tsx_moe_expert_grouped/swiglu");
        if (rc != TSX_OK) return rc;
    }
    return with_type(L.d_type, [&](auto T) {
        return with_lpr(lpr_d, [&](auto LPR) {
            const dim3 grid(blocks_for(L.n_embd, rows_d), (unsigned) gy);
            expert_down_kernel<decltype(T)::value, decltype(LPR)::value>
                <<<grid, kThreads, 0, s>>>(grp_ptr, grp_start, n_groups, ent_dst, hq, L, out);
            return launch_status("tsx_moe_expert_grouped/down");
        });
    });
}

TSX_API int tsx_moe_mmvq(int type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                         void* stream) {
    const size_t rb = tsx_row_bytes(type, n_in);
    if (!tsx_mmvq_type_ok(type) || rb == 0) {
        set_error("tsx_moe_mmvq: type %d with %d values per row not supported", type, n_in);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(w && x_q8_1 && y && n_out >= 0 && ncols >= 1 && ncols <= 8 && aligned(x_q8_1, 4),
                "tsx_moe_mmvq: w, x, y and 1..8 columns");
    if (n_out == 0) return TSX_OK;
    const int lpr = lanes_per_row(n_in / 32), rows = (kThreads / kWave) * (kWave / lpr);
    return with_mmvq_type(type, [&](auto T) {
        return with_lpr(lpr, [&](auto LPR) {
            mmvq_kernel<decltype(T)::value, decltype(LPR)::value><<<blocks_for(n_out, rows), kThreads, 0, (hipStream_t) stream>>>(
                (const uint8_t*) w, rb, (const tsx_block_q8_1*) x_q8_1, y, n_in, n_out, ncols);
            return launch_status("tsx_moe_mmvq");
        });
    });
}

TSX_API int tsx_moe_mmvq_ids_supported(int type) { return tsx_mmvq_type_ok(type); }

TSX_API int tsx_moe_mmvq_ids(int type, const tsx_mmvq_ids* a, int count, int n_in, int n_out, void* stream) {
    if (!tsx_mmvq_type_ok(type) || tsx_row_bytes(type, n_in) == 0) {
        set_error("tsx_moe_mmvq_ids: type %d with %d values per row not supported", type, n_in);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(a && a->table && a->ids && a->x && a->y && a->n_table >= 0 && a->x_every > 0 && n_out > 0 &&
                    count >= 0 && count <= 65535 && aligned(a->x, 4) && a->x_stride % 4 == 0,
                "tsx_moe_mmvq_ids: table, ids, x (4-byte aligned, x_stride a multiple of 4), y, x_every > 0, n_out > 0 "
                "and 0..65535 matrices");
    if (count == 0) return TSX_OK;
    const IdsSource src{a->table, a->ids, a->n_table, a->offset, (const uint8_t*) a->x, a->x_stride, a->x_every,
                        a->y, a->y_stride};
    return launch_many("tsx_moe_mmvq_ids", type, src, count, n_in, n_out, stream);
}

TSX_API int tsx_moe_mmvq_slots(int type, const tsx_mmvq_slots* a, int count, int n_in, int n_out, void* stream) {
    if (!tsx_mmvq_type_ok(type) || tsx_row_bytes(type, n_in) == 0) {
        set_error("tsx_moe_mmvq_slots: type %d with %d values per row not supported", type, n_in);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(a && count >= 0 && count <= 8 && n_out > 0, "tsx_moe_mmvq_slots: slots, 0..8 matrices, n_out > 0");
    SlotsSource src{};
    for (int j = 0; j < count; ++j) {
        TSX_REQUIRE(a->w[j] && a->x[j] && a->y[j] && aligned(a->x[j], 4), "tsx_moe_mmvq_slots: slot %d: w, x (4-byte "
                                                                          "aligned), y", j);
        src.w[j] = a->w[j];
        src.x[j] = a->x[j];
        src.y[j] = a->y[j];
    }
    if (count == 0) return TSX_OK;
    return launch_many("tsx_moe_mmvq_slots", type, src, count, n_in, n_out, stream);
}

TSX_API int tsx_moe_subblock_sums(int type, const void* w, int64_t n_in, int64_t n_rows, const void* x_q8_1,
                                  int64_t ncols, int32_t* sums, int32_t* qsums, void* stream) {
    const size_t rb = tsx_row_bytes(type, n_in);
    if (!tsx_mmvq_type_ok(type) || rb == 0) {
        set_error("tsx_moe_subblock_sums: type %d with %lld values per row not supported", type, (long long) n_in);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(w && x_q8_1 && sums && n_rows >= 0 && ncols >= 1 && aligned(x_q8_1, 4),
                "tsx_moe_subblock_sums: w, x, sums");
    const int nu = (int) (n_in / 32);
    if (n_rows == 0) return TSX_OK;
    return with_mmvq_type(type, [&](auto T) {
        subblock_sums_kernel<decltype(T)::value><<<blocks_for(n_rows * nu, kThreads), kThreads, 0, (hipStream_t) stream>>>(
            (const uint8_t*) w, rb, nu, n_rows, (const tsx_block_q8_1*) x_q8_1, ncols, sums, qsums);
        return launch_status("tsx_moe_subblock_sums");
    });
}

}  // extern "C"
