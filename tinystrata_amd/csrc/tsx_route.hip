// tsx_route.hip - the `ids` half of mul_mat_id on gfx950: router top-k, decode grouping, the prompt's expert sort,
// and the router-weighted combine.
//
// Reference: route_topk (src/kernels/cuda/native_router.cu:42-95), k_group (src/qwen35/q36_engine.cu:394-422),
// k_route_count / k_route_scan / k_route_scatter (src/qwen35/q36_engine.cu:483-510), k_moe_out
// (src/qwen35/q36_engine.cu:304-332).
//
// Differences by design: the router takes any expert count that is a multiple of 64 (up to 512) and k <= 16 (the
// reference: 256 and 8 only) with one wave64 per token; the prompt sort keeps the entries of an expert in entry
// order (a deterministic scatter built from wave ballots) and returns max_rows on the device, so no host round trip
// is needed before the grouped product.
#include "tsx_common.hpp"
#include "tsx_device.hpp"

namespace tsx {
namespace {

// one wave per token; expert e = lane + 64 i
__global__ void __launch_bounds__(256) router_topk_kernel(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts, int n_expert, int k, int n_tok) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_tok) return;
    route_token(logits + (int64_t) t * n_expert, n_expert, k, lane, ids + (int64_t) t * k, wts + (int64_t) t * k);
}

// decode grouping, one block: per-expert counts, then one thread lays out the groups and the entries in order
__global__ void __launch_bounds__(256) group_kernel(const int32_t* __restrict__ ids, int n_ent, int k, int n_expert,
                                                    const uint8_t* blobs, uint64_t stride, uint64_t* __restrict__ grp_ptr,
                                                    int32_t* __restrict__ grp_start, int32_t* __restrict__ n_groups,
                                                    int32_t* __restrict__ ent_dst, int32_t* __restrict__ ent_tok,
                                                    const int32_t* __restrict__ slot_of) {
    // slot_of (may be null): expert x's blob is slot slot_of[x] of `blobs`, and entries of experts without a slot
    // (slot_of[x] < 0) are left out; null: expert x's blob is blob x
    __shared__ int cnt[kMaxExperts], off[kMaxExperts];
    auto grouped = [&](int x) { return x >= 0 && x < n_expert && (!slot_of || slot_of[x] >= 0); };
    for (int x = threadIdx.x; x < n_expert; x += blockDim.x) cnt[x] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < n_ent; e += blockDim.x) {
        const int x = ids[e];
        if (grouped(x)) atomicAdd(&cnt[x], 1);
    }
    __syncthreads();
    // groups and offsets: each thread takes two consecutive experts; exclusive scans of their entry counts and of
    // their used flags over the block (within a wave by shuffles, then over the four waves' totals)
    {
        __shared__ int wsum[2][4];
        const int t = threadIdx.x, x0 = 2 * t, lane = t & 63, wave = t >> 6;
        const int c0 = x0 < n_expert ? cnt[x0] : 0, c1 = x0 + 1 < n_expert ? cnt[x0 + 1] : 0;
        int s = c0 + c1, g = (c0 > 0) + (c1 > 0);
        for (int o = 1; o < 64; o <<= 1) {
            const int ps = __shfl_up(s, o, 64), pg = __shfl_up(g, o, 64);
            if (lane >= o) {
                s += ps;
                g += pg;
            }
        }
        if (lane == 63) {
            wsum[0][wave] = s;
            wsum[1][wave] = g;
        }
        __syncthreads();
        for (int w = 0; w < wave; ++w) {
            s += wsum[0][w];
            g += wsum[1][w];
        }
        const int pos = s - c0 - c1, gi = g - (c0 > 0) - (c1 > 0);  // exclusive
        if (x0 < n_expert) off[x0] = pos;
        if (x0 + 1 < n_expert) off[x0 + 1] = pos + c0;
        if (c0 > 0) {
            grp_ptr[gi] = (uint64_t) (blobs + (uint64_t) (slot_of ? slot_of[x0] : x0) * stride);
            grp_start[gi] = pos;
        }
        if (c1 > 0) {
            grp_ptr[gi + (c0 > 0)] = (uint64_t) (blobs + (uint64_t) (slot_of ? slot_of[x0 + 1] : x0 + 1) * stride);
            grp_start[gi + (c0 > 0)] = pos + c0;
        }
        if (t == (int) blockDim.x - 1) {  // inclusive totals of the last thread
            grp_start[g] = s;
            *n_groups = g;
        }
    }
    __syncthreads();
    // the entries in entry order: wave-sized chunks, ranks from ballots, chunks committed in order
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int base = 0; base < n_ent; base += blockDim.x) {
        for (int w = 0; w < (int) (blockDim.x >> 6); ++w) {
            if (wave == w) {
                const int e = base + w * 64 + lane;
                int x = e < n_ent ? ids[e] : -1;
                const bool ok = grouped(x);
                if (!ok) x = -1;  // one class for every invalid id: -1 differs from 0..511 in bit 9
                uint64_t same = __ballot(1);
#pragma unroll
                for (int b = 0; b < 10; ++b) {
                    const uint64_t bits = __ballot((x >> b) & 1);
                    same &= ((x >> b) & 1) ? bits : ~bits;
                }
                const int rank = __builtin_popcountll(same & ((1ull << lane) - 1ull));
                if (ok) {
                    const int p = off[x] + rank;
                    ent_dst[p] = e;
                    ent_tok[p] = e / k;
                }
                // the lowest lane of each expert advances its cursor once the whole wave has read it
                const int total = __builtin_popcountll(same);
                __builtin_amdgcn_wave_barrier();
                if (ok && rank == 0) off[x] += total;
            }
            __syncthreads();
        }
    }
}

// the prompt sort, one block per tile of 1024 entries and no workspace: every block counts every entry (per expert:
// all of them, and those of the tiles before its own), scans the totals into bounds, then scatters its own tile
// stably - lanes of a wave that share an expert found with ballots, per-wave counts committed in wave order.
constexpr int kSortThreads = 1024, kSortWaves = kSortThreads / 64, kSortBatch = 8;
// the lanes of the wave holding the same expert as this lane (x = -1 for none): a mask over the wave
__device__ __forceinline__ uint64_t same_expert(int x) {
    uint64_t same = __ballot(1);
#pragma unroll
    for (int b = 0; b < 10; ++b) {  // experts < 512 (and -1) take 10 bits
        const uint64_t bits = __ballot((x >> b) & 1);
        same &= ((x >> b) & 1) ? bits : ~bits;
    }
    return same;
}
__global__ void __launch_bounds__(kSortThreads) route_sort_kernel(const int32_t* __restrict__ ids, int n_ent, int k,
                                                                  int n_expert, int32_t* __restrict__ bounds,
                                                                  int32_t* __restrict__ ent_dst, int32_t* __restrict__ ent_tok,
                                                                  int32_t* __restrict__ rinv, int32_t* __restrict__ max_rows) {
    __shared__ int cnt[kMaxExperts], before[kMaxExperts], start[kMaxExperts];
    __shared__ int wcnt[kSortWaves][kMaxExperts], wbef[kSortWaves][kMaxExperts];
    __shared__ int s_wsum[kSortWaves], s_wmax[kSortWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile0 = blockIdx.x * kSortThreads;
    // this thread's own entry of the tile, requested first (its scatter comes last)
    const int e = tile0 + tid;
    int x = e < n_ent ? ids[e] : -1;
    // each wave clears its own counts (only it adds to them, below): no division and no block barrier
    for (int xx = lane; xx < n_expert; xx += 64) wcnt[wave][xx] = 0;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // every entry's expert counted (a wave's 64 entries lie in one tile) in entries [lo, hi), kSortBatch tiles' ids
    // requested at once so that one load latency covers them
    auto count = [&](int lo, int hi) {
        for (int base = lo; base < hi; base += kSortThreads * kSortBatch) {
            int xs[kSortBatch];
#pragma unroll
            for (int j = 0; j < kSortBatch; ++j) {
                const int e = base + j * kSortThreads + tid;
                xs[j] = e < hi ? ids[e] : -1;
            }
#pragma unroll
            for (int j = 0; j < kSortBatch; ++j) {
                const int x = xs[j];
                // LDS atomics into the wave's own counts: no other wave touches them, and a wave's lanes share an
                // expert a few times at most (a token picks an expert once); an id out of range is dropped
                if (x >= 0 && x < n_expert) atomicAdd(&wcnt[wave][x], 1);
            }
        }
    };
    // the earlier tiles first: the wave's counts then are its counts before this block's tile (copied by the wave
    // itself, after its own atomics), and the rest of the entries complete them
    count(0, min(tile0, n_ent));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int xx = lane; xx < n_expert; xx += 64) wbef[wave][xx] = wcnt[wave][xx];
    count(min(tile0, n_ent), n_ent);
    __syncthreads();
    for (int xx = tid; xx < n_expert; xx += kSortThreads) {  // the waves' counts summed (wcnt cleared for the scatter)
        int c = 0, b = 0;
        for (int w = 0; w < kSortWaves; ++w) {
            c += wcnt[w][xx];
            b += wbef[w][xx];
            wcnt[w][xx] = 0;
        }
        cnt[xx] = c;
        before[xx] = b;
    }
    __syncthreads();
    // bounds: exclusive scan of the counts over experts (expert x = thread x), and the largest count
    {
        const int v = tid < n_expert ? cnt[tid] : 0;
        int inc = v, mx = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(inc, o, 64);
            if (lane >= o) inc += t;
            mx = max(mx, __shfl_xor(mx, o, 64));
        }
        if (lane == 63) s_wsum[wave] = inc;
        if (lane == 0) s_wmax[wave] = mx;
        __syncthreads();
        int off = 0, total = 0, gmax = 0;
        for (int w = 0; w < kSortWaves; ++w) {
            off += w < wave ? s_wsum[w] : 0;
            total += s_wsum[w];
            gmax = max(gmax, s_wmax[w]);
        }
        if (tid < n_expert) {
            start[tid] = off + inc - v + before[tid];  // this tile's first row of expert tid
            if (blockIdx.x == 0) bounds[tid] = off + inc - v;
        }
        if (blockIdx.x == 0 && tid == 0) {
            bounds[n_expert] = total;
            *max_rows = gmax;
        }
    }
    // this tile's entries, stably
    if (x < 0 || x >= n_expert) x = -1;
    const uint64_t same = same_expert(x);
    const int rank = __builtin_popcountll(same & ((1ull << lane) - 1ull));
    if (x >= 0 && rank == 0) wcnt[wave][x] = __builtin_popcountll(same);
    __syncthreads();
    for (int xx = tid; xx < n_expert; xx += kSortThreads) {  // exclusive scan over the waves
        int run = start[xx];
        for (int w = 0; w < kSortWaves; ++w) {
            const int c = wcnt[w][xx];
            wcnt[w][xx] = run;
            run += c;
        }
    }
    __syncthreads();
    if (x >= 0) {
        const int r = wcnt[wave][x] + rank;
        ent_dst[r] = e;
        ent_tok[r] = e / k;
        rinv[e] = r;
    }
}

// x[t][i] += sum_j w_j parts[p(t,j)][i] (first product, then FMA, pick order) + sigmoid(sgate) * shared[t][i]
// row e of parts = row miss[e] of rows where miss[e] >= 0 (an entry the CPU computed), else unchanged
// (reference k_merge_cpu, src/qwen35/q36_engine.cu:455-460, with compact row indices)
__global__ void __launch_bounds__(256) merge_rows_kernel(float* __restrict__ parts, const float* __restrict__ rows,
                                                         const int32_t* __restrict__ miss, int64_t n) {
    const int e = blockIdx.y;
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int m = miss[e];
    if (m < 0 || i >= n) return;
    parts[(int64_t) e * n + i] = rows[(int64_t) m * n + i];
}

__global__ void __launch_bounds__(256) combine_kernel(float* __restrict__ x, const float* __restrict__ parts,
                                                      const int32_t* __restrict__ prow, const float* __restrict__ wts, int k,
                                                      const float* __restrict__ shared, const float* __restrict__ sgate,
                                                      int sg_stride, int n) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float* wr = wts + (int64_t) t * k;
    auto part = [&](int j) { return parts[(int64_t) (prow ? prow[t * k + j] : t * k + j) * n + i]; };
    float acc = wr[0] * part(0);
    for (int j = 1; j < k; ++j) acc = __builtin_fmaf(wr[j], part(j), acc);
    if (shared) {
        const float gs = 1.0f / (1.0f + expf(-sgate[(int64_t) t * sg_stride]));
        acc += gs * shared[(int64_t) t * n + i];
    }
    x[(int64_t) t * n + i] += acc;
}

// the same, four columns per thread (n a multiple of 4, every row 16-byte aligned)
__global__ void __launch_bounds__(256) combine4_kernel(float* __restrict__ x, const float* __restrict__ parts,
                                                       const int32_t* __restrict__ prow, const float* __restrict__ wts,
                                                       int k, const float* __restrict__ shared,
                                                       const float* __restrict__ sgate, int sg_stride, int n) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int i = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const float* wr = wts + (int64_t) t * k;
    auto part = [&](int j) {
        return *(const float4*) (parts + (int64_t) (prow ? prow[t * k + j] : t * k + j) * n + i);
    };
    float4 p = part(0);
    const float w0 = wr[0];
    float4 acc = {w0 * p.x, w0 * p.y, w0 * p.z, w0 * p.w};
    for (int j = 1; j < k; ++j) {
        p = part(j);
        const float wj = wr[j];
        acc = {__builtin_fmaf(wj, p.x, acc.x), __builtin_fmaf(wj, p.y, acc.y), __builtin_fmaf(wj, p.z, acc.z),
               __builtin_fmaf(wj, p.w, acc.w)};
    }
    if (shared) {
        const float gs = 1.0f / (1.0f + expf(-sgate[(int64_t) t * sg_stride]));
        const float4 sh = *(const float4*) (shared + (int64_t) t * n + i);
        acc = {acc.x + gs * sh.x, acc.y + gs * sh.y, acc.z + gs * sh.z, acc.w + gs * sh.w};
    }
    float4* xo = (float4*) (x + (int64_t) t * n + i);
    const float4 xv = *xo;
    *xo = float4{xv.x + acc.x, xv.y + acc.y, xv.z + acc.z, xv.w + acc.w};
}

// tsx_moe_combine's arithmetic per value, then the norm (norm_row_out): one block per token row, the combined row
// kept in LDS
constexpr int kNormThreads = 256;
constexpr int kNormMaxK = 16;
__global__ void __launch_bounds__(kNormThreads) combine_norm_kernel(float* __restrict__ x, const float* __restrict__ parts,
                                                                   const int32_t* __restrict__ prow,
                                                                   const float* __restrict__ wts, int k,
                                                                   const float* __restrict__ shared,
                                                                   const float* __restrict__ sgate, int sg_stride, int n,
                                                                   const float* __restrict__ norm_w, float eps,
                                                                   float* __restrict__ h, tsx_block_q8_1* __restrict__ hq) {
#pragma clang fp contract(off)
    extern __shared__ float s_row[];
    __shared__ const float* s_part[kNormMaxK];
    __shared__ float s_red[kNormThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid < k) s_part[tid] = parts + (int64_t) (prow ? prow[t * k + tid] : t * k + tid) * n;
    __syncthreads();
    const float* wr = wts + (int64_t) t * k;
    const float gs = shared ? 1.0f / (1.0f + expf(-sgate[(int64_t) t * sg_stride])) : 0.f;
    float* xr = x + (int64_t) t * n;
    float q = 0.f;
    for (int i = tid; i < n; i += kNormThreads) {
        float acc = wr[0] * s_part[0][i];
        for (int j = 1; j < k; ++j) acc = __builtin_fmaf(wr[j], s_part[j][i], acc);
        if (shared) acc += gs * shared[(int64_t) t * n + i];
        const float v = xr[i] + acc;
        xr[i] = v;
        s_row[i] = v;
        q += v * v;
    }
    norm_row_out<kNormThreads>(s_row, q, n, norm_w, eps, h + (int64_t) t * n, hq ? hq + (int64_t) t * (n / 32) : nullptr,
                               s_red);
}

}  // namespace
}  // namespace tsx

using namespace tsx;

extern "C" {

TSX_API int tsx_moe_router_topk(const float* logits, int32_t* ids, float* weights, int n_expert, int k, int n_tok,
                                void* stream) {
    if (n_expert <= 0 || n_expert % 64 != 0 || n_expert > kMaxExperts || k < 1 || k > 16 || k > n_expert) {
        set_error("tsx_moe_router_topk: %d experts / top-%d not supported (a multiple of 64 up to 512, k 1..16)", n_expert, k);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(logits && ids && weights && n_tok >= 0 && aligned(logits, 4) && aligned(ids, 4) && aligned(weights, 4),
                "tsx_moe_router_topk: logits, ids, weights (4-byte aligned)");
    if (n_tok == 0) return TSX_OK;
    router_topk_kernel<<<(unsigned) ((n_tok + 3) / 4), 256, 0, (hipStream_t) stream>>>(logits, ids, weights, n_expert, k, n_tok);
    return launch_status("tsx_moe_router_topk");
}

TSX_API int tsx_moe_group(const int32_t* ids, int n_ent, int k, int n_expert, const void* blobs, uint64_t stride,
                          uint64_t* grp_ptr, int32_t* grp_start, int32_t* n_groups, int32_t* ent_dst, int32_t* ent_tok,
                          void* stream) {
    if (n_expert <= 0 || n_expert > kMaxExperts) {
        set_error("tsx_moe_group: %d experts (at most 512)", n_expert);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(ids && grp_ptr && grp_start && n_groups && ent_dst && ent_tok && n_ent >= 0 && k >= 1,
                "tsx_moe_group: a null pointer or a bad count");
    group_kernel<<<1, 256, 0, (hipStream_t) stream>>>(ids, n_ent, k, n_expert, (const uint8_t*) blobs, stride, grp_ptr,
                                                      grp_start, n_groups, ent_dst, ent_tok, nullptr);
    return launch_status("tsx_moe_group");
}

TSX_API int tsx_moe_group_resident(const int32_t* ids, int n_ent, int k, int n_expert, const int32_t* slot_of,
                                   const void* slots, uint64_t stride, uint64_t* grp_ptr, int32_t* grp_start,
                                   int32_t* n_groups, int32_t* ent_dst, int32_t* ent_tok, void* stream) {
    if (n_expert <= 0 || n_expert > kMaxExperts) {
        set_error("tsx_moe_group_resident: %d experts (at most 512)", n_expert);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(ids && slot_of && slots && grp_ptr && grp_start && n_groups && ent_dst && ent_tok && n_ent >= 0 &&
                    k >= 1, "tsx_moe_group_resident: a null pointer or a bad count");
    group_kernel<<<1, 256, 0, (hipStream_t) stream>>>(ids, n_ent, k, n_expert, (const uint8_t*) slots, stride,
                                                      grp_ptr, grp_start, n_groups, ent_dst, ent_tok, slot_of);
    return launch_status("tsx_moe_group_resident");
}

TSX_API int tsx_moe_merge_rows(float* parts, const float* rows, const int32_t* miss, int n_ent, int64_t n,
                               void* stream) {
    TSX_REQUIRE(parts && rows && miss && n_ent >= 0 && n >= 0, "tsx_moe_merge_rows: parts, rows, miss, sizes");
    if (n_ent == 0 || n == 0) return TSX_OK;
    merge_rows_kernel<<<dim3((unsigned) ((n + 255) / 256), (unsigned) n_ent), 256, 0, (hipStream_t) stream>>>(
        parts, rows, miss, n);
    return launch_status("tsx_moe_merge_rows");
}

TSX_API int tsx_moe_route_sort(const int32_t* ids, int n_ent, int k, int n_expert, int32_t* bounds, int32_t* ent_dst,
                               int32_t* ent_tok, int32_t* rinv, int32_t* max_rows, void* stream) {
    if (n_expert <= 0 || n_expert > kMaxExperts) {
        set_error("tsx_moe_route_sort: %d experts (at most 512)", n_expert);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(ids && bounds && ent_dst && ent_tok && rinv && max_rows && n_ent >= 0 && k >= 1,
                "tsx_moe_route_sort: a null pointer or a bad count");
    const unsigned tiles = (unsigned) std::max(1, (n_ent + kSortThreads - 1) / kSortThreads);
    route_sort_kernel<<<tiles, kSortThreads, 0, (hipStream_t) stream>>>(ids, n_ent, k, n_expert, bounds, ent_dst,
                                                                        ent_tok, rinv, max_rows);
    return launch_status("tsx_moe_route_sort");
}

TSX_API int tsx_moe_combine(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                            const float* shared, const float* sgate, int sg_stride, int n, int n_tok, void* stream) {
    TSX_REQUIRE(x && parts && wts && k >= 1 && n >= 0 && n_tok >= 0 && (!shared || sgate),
                "tsx_moe_combine: x, parts, wts, k >= 1 (and sgate with shared)");
    if (n == 0 || n_tok == 0) return TSX_OK;
    if (n % 4 == 0 && aligned(x, 16) && aligned(parts, 16) && (!shared || aligned(shared, 16))) {
        combine4_kernel<<<dim3((unsigned) ((n / 4 + 255) / 256), (unsigned) n_tok), 256, 0, (hipStream_t) stream>>>(
            x, parts, prow, wts, k, shared, sgate, sg_stride, n);
        return launch_status("tsx_moe_combine");
    }
    combine_kernel<<<dim3((unsigned) ((n + 255) / 256), (unsigned) n_tok), 256, 0, (hipStream_t) stream>>>(
        x, parts, prow, wts, k, shared, sgate, sg_stride, n);
    return launch_status("tsx_moe_combine");
}

TSX_API int tsx_moe_combine_norm(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                                 const float* shared, const float* sgate, int sg_stride, int n, int n_tok,
                                 const float* norm_w, float eps, float* h, void* hq, void* stream) {
    TSX_REQUIRE(x && parts && wts && norm_w && h && k >= 1 && k <= kNormMaxK && n_tok >= 0 && (!shared || sgate),
                "tsx_moe_combine_norm: x, parts, wts, norm_w, h, k 1..16 (and sgate with shared)");
    if (n < 32 || n % 32 != 0 || n > 16384) {
        set_error("tsx_moe_combine_norm: n = %d (a multiple of 32 up to 16384)", n);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(aligned(hq, 2), "tsx_moe_combine_norm: hq 2-byte aligned");
    if (n_tok == 0) return TSX_OK;
    combine_norm_kernel<<<(unsigned) n_tok, kNormThreads, (size_t) n * 4, (hipStream_t) stream>>>(
        x, parts, prow, wts, k, shared, sgate, sg_stride, n, norm_w, eps, h, (tsx_block_q8_1*) hq);
    return launch_status("tsx_moe_combine_norm");
}

}  // extern "C"
