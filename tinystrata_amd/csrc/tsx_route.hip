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
                                                    int32_t* __restrict__ ent_dst, int32_t* __restrict__ ent_tok) {
    __shared__ int cnt[kMaxExperts], off[kMaxExperts];
    for (int x = threadIdx.x; x < n_expert; x += blockDim.x) cnt[x] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < n_ent; e += blockDim.x) {
        const int x = ids[e];
        if (x >= 0 && x < n_expert) atomicAdd(&cnt[x], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int g = 0, pos = 0;
        for (int x = 0; x < n_expert; ++x) {
            off[x] = pos;
            if (cnt[x] == 0) continue;
            grp_ptr[g] = (uint64_t) (blobs + (uint64_t) x * stride);
            grp_start[g] = pos;
            pos += cnt[x];
            ++g;
        }
        grp_start[g] = pos;
        *n_groups = g;
    }
    __syncthreads();
    // the entries in entry order: wave-sized chunks, ranks from ballots, chunks committed in order
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int base = 0; base < n_ent; base += blockDim.x) {
        for (int w = 0; w < (int) (blockDim.x >> 6); ++w) {
            if (wave == w) {
                const int e = base + w * 64 + lane;
                int x = e < n_ent ? ids[e] : -1;
                const bool ok = x >= 0 && x < n_expert;
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

// the prompt sort: counts, scan, then a stable scatter (16 waves per tile, per-wave counts committed in order)
constexpr int kSortThreads = 1024, kSortWaves = kSortThreads / 64;
__global__ void __launch_bounds__(kSortThreads) route_sort_kernel(const int32_t* __restrict__ ids, int n_ent, int k,
                                                                  int n_expert, int32_t* __restrict__ bounds,
                                                                  int32_t* __restrict__ ent_dst, int32_t* __restrict__ ent_tok,
                                                                  int32_t* __restrict__ rinv, int32_t* __restrict__ max_rows) {
    __shared__ int cnt[kMaxExperts], cur[kMaxExperts];
    __shared__ int wcnt[kSortWaves][kMaxExperts];
    __shared__ int s_max;
    for (int x = threadIdx.x; x < n_expert; x += blockDim.x) cnt[x] = 0;
    if (threadIdx.x == 0) s_max = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < n_ent; e += blockDim.x) {
        const int x = ids[e];
        if (x >= 0 && x < n_expert) atomicAdd(&cnt[x], 1);  // an id out of range is dropped
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int pos = 0, mx = 0;
        for (int x = 0; x < n_expert; ++x) {
            bounds[x] = pos;
            cur[x] = pos;
            pos += cnt[x];
            mx = max(mx, cnt[x]);
        }
        bounds[n_expert] = pos;
        s_max = mx;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int base = 0; base < n_ent; base += kSortThreads) {
        for (int i = threadIdx.x; i < kSortWaves * n_expert; i += kSortThreads) wcnt[i / n_expert][i % n_expert] = 0;
        __syncthreads();
        const int e = base + threadIdx.x;
        int x = e < n_ent ? ids[e] : -1;
        if (x < 0 || x >= n_expert) x = -1;
        uint64_t same = __ballot(1);
#pragma unroll
        for (int b = 0; b < 10; ++b) {
            const uint64_t bits = __ballot((x >> b) & 1);
            same &= ((x >> b) & 1) ? bits : ~bits;
        }
        const int rank = __builtin_popcountll(same & ((1ull << lane) - 1ull));
        if (x >= 0 && rank == 0) wcnt[wave][x] = __builtin_popcountll(same);
        __syncthreads();
        for (int xx = threadIdx.x; xx < n_expert; xx += kSortThreads) {  // exclusive scan over the waves
            int run = cur[xx];
            for (int w = 0; w < kSortWaves; ++w) {
                const int c = wcnt[w][xx];
                wcnt[w][xx] = run;
                run += c;
            }
            cur[xx] = run;
        }
        __syncthreads();
        if (x >= 0) {
            const int r = wcnt[wave][x] + rank;
            ent_dst[r] = e;
            ent_tok[r] = e / k;
            rinv[e] = r;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *max_rows = s_max;
}

// x[t][i] += sum_j w_j parts[p(t,j)][i] (first product, then FMA, pick order) + sigmoid(sgate) * shared[t][i]
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
                                                      grp_start, n_groups, ent_dst, ent_tok);
    return launch_status("tsx_moe_group");
}

TSX_API int tsx_moe_route_sort(const int32_t* ids, int n_ent, int k, int n_expert, int32_t* bounds, int32_t* ent_dst,
                               int32_t* ent_tok, int32_t* rinv, int32_t* max_rows, void* stream) {
    if (n_expert <= 0 || n_expert > kMaxExperts) {
        set_error("tsx_moe_route_sort: %d experts (at most 512)", n_expert);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(ids && bounds && ent_dst && ent_tok && rinv && max_rows && n_ent >= 0 && k >= 1,
                "tsx_moe_route_sort: a null pointer or a bad count");
    route_sort_kernel<<<1, kSortThreads, 0, (hipStream_t) stream>>>(ids, n_ent, k, n_expert, bounds, ent_dst, ent_tok,
                                                                    rinv, max_rows);
    return launch_status("tsx_moe_route_sort");
}

TSX_API int tsx_moe_combine(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                            const float* shared, const float* sgate, int sg_stride, int n, int n_tok, void* stream) {
    TSX_REQUIRE(x && parts && wts && k >= 1 && n >= 0 && n_tok >= 0 && (!shared || sgate),
                "tsx_moe_combine: x, parts, wts, k >= 1 (and sgate with shared)");
    if (n == 0 || n_tok == 0) return TSX_OK;
    combine_kernel<<<dim3((unsigned) ((n + 255) / 256), (unsigned) n_tok), 256, 0, (hipStream_t) stream>>>(
        x, parts, prow, wts, k, shared, sgate, sg_stride, n);
    return launch_status("tsx_moe_combine");
}

}  // extern "C"
