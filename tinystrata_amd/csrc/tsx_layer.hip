// tsx_layer.hip - a whole decode MoE layer (1..8 tokens) in two launches on gfx950.
//
// Reference: the MoE block of src/qwen35/q36_engine.cu:2821-2925 - k_route_group (src/qwen35/q36_kernels.cuh:383-474),
// native_expert_grouped (src/kernels/cuda/iq_kernels.cu:2835-2982), the shared expert (mmvq, SwiGLU + Q8_1, mmvq:
// q36_engine.cu:2906-2913) and k_moe_out_small without the norm (q36_kernels.cuh:248-290).  The reference spends
// five to eight launches per layer on that sequence; here it is two, with nothing between them on the host.
//
// At one token the layer is bound by latency and by the vector ALU, not by HBM: 11.3 MB is 1.4 us of HBM time, a
// dependent global round trip costs about a microsecond, and decoding the IQ3 codebooks costs ~100 VALU operations
// per 32 weights - about 2 us of the whole chip's vector issue for one token-layer.  So the work is cut fine enough
// to reach every CU, each launch keeps its chain of dependent memory accesses short (A: logits -> routing ->
// weights; B: one table read -> weights) and issues everything else alongside, and cross-lane reductions use DPP
// and readlane rather than LDS permutes.
//
// Launch A, 256 blocks (one per CU) of 1024 threads.  Every block
//   1. routes every token (route_select: one wave per token, the code of tsx_moe_router_topk) and groups the entries
//      by expert in LDS (ascending id, entries in entry order), while its other waves quantize the activations to
//      Q8_1 in LDS;
//   2. takes an equal run of the layer's slices (a slice: gate and up rows [32 j, 32 j + 32) of one group's expert;
//      the groups' slices one after another, the shared expert's last), so every CU has the same rows however many
//      groups the routing made;
//   3. streams each slice's rows into wave-private LDS slabs with 16-byte loads (rows too long for one slab come in
//      chunks; a wave requests its next chunk's rows before computing the current one), dots them with every entry
//      of the slice's group (each unit decoded once for all entries), applies SwiGLU (the product rounded on its own)
//      and writes the slice's Q8_1 block of h per entry.  Block 0 also writes ids / wts and the tables launch B
//      needs.
// Launch B, grid n_embd/8, 1024 threads.  Every block owns 8 output rows: it reads the tables and every entry's h in
//   one round trip, loads those 8 rows of every used expert's down matrix (and the shared expert's) into LDS,
//   dots, and combines in pick order: y += w0*p0, fmaf(wj, pj, .) ..., + sigmoid(sgate)*shared -
//   tsx_moe_combine's arithmetic.
//
// Every load a block can issue before it needs the data is issued unconditionally (indices clamped into range),
// so the compiler's wait counts stay exact and the loads stay in flight together.
//
// Memory per layer at config 2 (N 2048, FF 512, IQ3_XXS gate/up, IQ3_S down, 8 routed + 1 shared expert): launch A
// reads 9 x 802,816 B of gate/up rows in 144 blocks of 50 KB; launch B 9 x 450,560 B of down rows in 256 blocks of
// 15.8 KB.
#include "tsx_common.hpp"
#include "tsx_device.hpp"

#include <climits>
#include <mutex>
#include <type_traits>

namespace tsx {
namespace {

constexpr int kMaxTok = 8;            // tokens per decode layer call
constexpr int kMaxEnt = 64;           // routed entries (tokens x k)
constexpr int kNC = 4;                // entries per pass over a row's units
constexpr int kThreadsA = 1024;
constexpr int kWavesA = kThreadsA / 64;
constexpr int kSliceA = 32;           // gate (and up) rows of a launch A slice: one Q8_1 block of h per entry
constexpr int kBlocksA = 256;         // launch A: one block per CU, each an equal run of slices
constexpr int kSlabA = 64 * 1024;     // most LDS bytes of a chunk of gate + up rows: 4 KB per wave
constexpr int kWLoadsA = kSlabA / kWavesA / 16 / 64;  // 16-byte loads per lane of a wave's rows
constexpr int kXLoads = 2;            // activation quads per thread per round of launch A
constexpr int kThreadsB = 1024;
constexpr int kRowsB = 8;             // output rows per block of launch B
constexpr int kNormRowThreads = 1024;  // the norm launch: threads per token row
constexpr int kSlabB = 64 * 1024;     // most LDS bytes of a chunk of groups' down rows (8 rows of each)
constexpr int kBLoads = kSlabB / 16 / kThreadsB;  // 16-byte loads per thread in flight: a whole chunk
constexpr int kHLoads = 3;            // 16-byte pieces of h per thread prefetched by launch B
constexpr int kHLoadsT = 5;           // the same for fp32 h of several tokens (36 positions x 512: 4.5 per thread)
constexpr int kItemsB = 2;            // launch B: (row, unit) items per thread decoded together
static_assert(kMaxTok <= kThreadsA / 64, "one wave per token in the routing");

// the tables launch A leaves for launch B, at the start of the scratch buffer
struct LayerTables {
    int32_t n_groups;
    int32_t pad[3];
    int32_t grp_expert[kMaxEnt];
    int32_t grp_start[kMaxEnt + 4];
    int32_t ent_pos[kMaxEnt];     // entry e = t*k + j -> its position in expert order
    float wts[kMaxEnt];
};
constexpr int kTableWords = sizeof(LayerTables) / 4;
static_assert(kTableWords <= kThreadsB, "launch B reads the tables in one round");
constexpr size_t kTablesBytes = (sizeof(LayerTables) + 255) & ~(size_t) 255;

struct LayerArgs {
    tsx_expert_layout L;
    const uint8_t* blobs;
    uint64_t stride;
    int n_expert, k, n_tok;
    const float* logits;
    const float* x;
    const uint8_t* shared;
    const float* sgate;
    int sg_stride;
    int rows_c;                   // gate (and up) rows per chunk of launch A: 32, 16 or 8
    int chunks_a;                 // chunks per slice: 32 / rows_c
    int slab_a, slab_b;           // LDS bytes of the weight slabs (<= kSlabA, kSlabB: what the codebooks leave)
    float* y;
    int32_t* ids;
    float* wts;
    LayerTables* tab;
    int8_t* hc;                   // Q8_1 codes of h [P][n_ff], P = n_tok * k (+ n_tok shared): expert order positions
    float* hd;                    // their scales [P][n_ff / 32], right after the codes
    float* hf;                    // one-token launch A: h in fp32 [P][n_ff] (where hc would be); launch B quantizes it
    int h_fp32;                   // launch B reads hf instead of hc / hd
    int rows_w;                   // one-token launch A: rows per wave (the slab holds rows_w rows of each wave)
    int s1_ppb;                   // slot-by-slot launch A: row pairs of every slot per block (n_ff / grid)
    int s1_wave[16];              // its waves: slot | first row << 8 | end row << 16 (rows of the slot's 2 ppb)
};

// one Q8_1 activation unit (32 codes + scale) from LDS planes (codes row-major, one float scale per 32)
__device__ __forceinline__ void act_planes(const int8_t* codes, const float* d, Act& a) {
    // the pointers are generic; the casts keep the reads ds_read (a flat load would wait behind the global loads)
    const lds_ptr<const v4i> p = (lds_ptr<const v4i>) codes;
    const v4i q0 = p[0], q1 = p[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a.q[i] = q0[i];
        a.q[4 + i] = q1[i];
    }
    a.d = *(lds_ptr<const float>) d;
}


// Q8_1 of a 32-value block held as 4 floats by each of 8 consecutive lanes (lane l of the block: values 4l..4l+3)
// into LDS planes.  All 64 lanes of the wave take part.
__device__ __forceinline__ void q8_1_quad_to_lds(const float4& x, bool valid, int8_t* codes, float* d, int l8) {
    float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    amax = lanes_reduce<8>(amax, OpMax());
    const float dd = q8_1_scale(amax);
    int c[4];
    q8_1_codes4(x, amax, dd, c);
    const uint32_t packed = ((uint32_t) c[0] & 0xFFu) | ((uint32_t) c[1] & 0xFFu) << 8 |
                            ((uint32_t) c[2] & 0xFFu) << 16 | ((uint32_t) c[3] & 0xFFu) << 24;
    if (valid) {
        *(uint32_t*) codes = packed;
        if (l8 == 0) *d = h2f(f2h(dd));
    }
}

// x / d for 0 <= x < 2^22 and d >= 1, from rd ~ 1 / d (v_rcp_f32 is within an ulp): the float quotient is within one
// of the truth (an integer division would put ~40 instructions on the path to the weight loads)
__device__ __forceinline__ int div_small(int x, int d, float rd) {
    int q = (int) ((float) x * rd);
    q -= q * d > x ? 1 : 0;
    q += (q + 1) * d <= x ? 1 : 0;
    return q;
}

// the sums of the first nu accumulators over each W-lane row (nu the same in every lane of the wave)
template <int W>
__device__ __forceinline__ void sum_acc(float (&acc)[kNC], int nu) {
#pragma unroll
    for (int c = 0; c < kNC; ++c)
        if (c < nu) acc[c] = lanes_sum<W>(acc[c]);
}

// ------------------------------------------------------------------ launch A
template <int GT>
__global__ void __launch_bounds__(kThreadsA) layer_gu_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    constexpr int RP = (rep_stores<GT>() + kThreadsA - 1) / kThreadsA;
    using Tab = std::conditional_t<(RP > 0), RepTab<GT>, GridRef>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int32_t s_ids[kMaxEnt], s_sorted[kMaxEnt], s_pos_ent[kMaxEnt], s_ent_pos[kMaxEnt];
    __shared__ int32_t s_grp_expert[kMaxEnt], s_grp_start[kMaxEnt + 1];
    __shared__ float s_wts[kMaxEnt];
    __shared__ int s_ngroups;
    __shared__ float s_gu[kMaxTok][2 * kSliceA];
    __shared__ int s_prow[kMaxEnt + kMaxTok];  // position -> its token's activation row

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int T = a.n_tok, k = a.k, n_ent = T * k;
    const tsx_expert_layout L = a.L;
    const int N = (int) L.n_embd, NU = N / 32, FF = (int) L.n_ff;

    // 0. the routing waves' logits are requested first (their wait then covers those loads alone), then what does
    //    not depend on the routing: the codebooks and, by the waves that do not route, the first round of every
    //    token's activations
    float lg[kRouteV];
    if (wave < T) route_fetch(a.logits + (int64_t) wave * a.n_expert, a.n_expert, lane, lg);
    uint64_t rv[RP > 0 ? RP : 1];
    if constexpr (RP > 0) rep_fetch<GT, RP>(rv, tid, kThreadsA);
    const int nq_all = T * N / 4;
    const int xt = tid - 64 * T, nxt = kThreadsA - 64 * T;  // the waves that do not route (T <= 8 of 16 route)
    const float4* x4 = (const float4*) a.x;
    float4 xv[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(max(xt, 0) + nxt * i, nq_all - 1)];
    int8_t* s_xq = (int8_t*) (smem + a.slab_a + rep_lds_bytes<GT>());
    float* s_xd = (float*) (s_xq + T * N);

    // 1. routing (one wave per token) while the other waves quantize every token's activations to Q8_1 planes in
    //    LDS (row t: token t); then grouping, identical in every block
    if (wave < T) {
        route_select(lg, a.n_expert, k, lane, s_ids + wave * k, s_wts + wave * k);
    } else {
        for (int base = 0; base < nq_all; base += nxt * kXLoads) {
            if (base > 0) {
#pragma unroll
                for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(base + xt + nxt * i, nq_all - 1)];
            }
#pragma unroll
            for (int i = 0; i < kXLoads; ++i) {
                const int qd = base + xt + nxt * i;
                if (base + nxt * i < nq_all)  // the same for every thread of these waves
                    q8_1_quad_to_lds(xv[i], qd < nq_all, s_xq + 4 * qd, s_xd + qd / 8, xt & 7);
            }
        }
    }
    Tab grid;
    if constexpr (RP > 0) grid = rep_store<GT, RP>(smem + a.slab_a, rv, tid, kThreadsA);
    else grid = grid_const();
    __syncthreads();
    if (wave == 0) {  // rank of entry `lane` in (expert, entry) order
        const int e = lane;
        const int key = e < n_ent ? s_ids[e] * 64 + e : INT_MAX;
        int rank = 0;
        for (int i = 0; i < n_ent; ++i) rank += __builtin_amdgcn_readlane(key, i) < key;
        if (e < n_ent) {
            s_sorted[rank] = s_ids[e];
            s_pos_ent[rank] = e;
            s_ent_pos[e] = rank;
        }
    }
    __syncthreads();
    if (wave == 0) {  // a group starts where the expert changes
        const int p = lane;
        const int xp = p < n_ent ? s_sorted[p] : -1;
        const bool start = p < n_ent && (p == 0 || s_sorted[p - 1] != xp);
        const uint64_t mask = __ballot(start);
        if (start) {
            const int g = __builtin_popcountll(mask & (~0ull >> (63 - p))) - 1;
            s_grp_expert[g] = xp;
            s_grp_start[g] = p;
        }
        if (lane == 0) {
            const int ng = __builtin_popcountll(mask);
            s_ngroups = ng;
            s_grp_start[ng] = n_ent;
        }
    }
    __syncthreads();
    const int ng = s_ngroups;
    if (blockIdx.x == 0) {
        if (tid < n_ent) {
            a.ids[tid] = s_ids[tid];
            a.wts[tid] = s_wts[tid];
            a.tab->wts[tid] = s_wts[tid];
            a.tab->ent_pos[tid] = s_ent_pos[tid];
        }
        if (tid <= ng) {
            if (tid < ng) a.tab->grp_expert[tid] = s_grp_expert[tid];
            a.tab->grp_start[tid] = s_grp_start[tid];
        }
        if (tid == 0) a.tab->n_groups = ng;
    }

    // 2. this block's slices.  A slice is 32 pairs - gate rows and up rows [32 j, 32 j + 32) - of one group's expert:
    //    one Q8_1 block of h per entry.  The groups' n_ff / 32 slices come one after another, the shared expert's
    //    last, and every block takes an equal run of them, so every CU has the same rows however many groups the
    //    routing made.
    const int spg = FF / kSliceA, G = ng + (a.shared ? 1 : 0), total = G * spg, nb = (int) gridDim.x;
    const float rspg = __builtin_amdgcn_rcpf((float) spg);
    const int share = div_small(total + nb - 1, nb, __builtin_amdgcn_rcpf((float) nb));
    const int s0 = (int) blockIdx.x * share, s1 = min(total, s0 + share);
    if (s0 >= s1) return;  // the whole block: nothing this far

    // 3. each wave's rows of the first chunk in flight.  A slice comes in nchunks chunks of 2 * rows_c rows (gate
    //    rows, then up rows); wave w owns rpw of them and is the only reader of its LDS copy, so it starts computing
    //    as soon as its own rows have arrived, and requests the next chunk's (of this slice or the next) first.
    const int rows_c = a.rows_c, nchunks = a.chunks_a;
    const int rpw = 2 * rows_c / kWavesA;          // rows per wave: 4, 2 or 1
    const bool w_up = wave >= kWavesA / 2;
    const int wr0 = rpw * (wave % (kWavesA / 2));  // the wave's first row within the chunk's gate (or up) rows
    const uint64_t gu_row = L.gu_row;
    const int np = (int) (rpw * gu_row / 16);      // 16-byte pieces of the wave's rows (<= 64 * kWLoadsA)
    struct Slice {
        const uint8_t* blob;
        int p0, n_e, j;  // the group's first position and entry count (<= T: a token picks an expert once); slice j
    };
    auto slice_at = [&](int sl) {
        const int g = div_small(sl, spg, rspg);
        Slice r;
        r.blob = g < ng ? a.blobs + (uint64_t) s_grp_expert[g] * a.stride : a.shared;
        r.p0 = g < ng ? s_grp_start[g] : n_ent;
        r.n_e = g < ng ? s_grp_start[g + 1] - r.p0 : T;
        r.j = sl - g * spg;
        return r;
    };
    v4i reg[kWLoadsA];
    auto issue = [&](const Slice& si, int c) {
        const gbl_ptr<const v4i> src = gbl_at<v4i>(
            (uintptr_t) (si.blob + (w_up ? L.up_off : 0) + (uint64_t) (kSliceA * si.j + c * rows_c + wr0) * gu_row));
#pragma unroll
        for (int i = 0; i < kWLoadsA; ++i)  // unconditional (clamped) loads keep the wait counts exact
            reg[i] = __builtin_nontemporal_load(src + min(lane + 64 * i, np - 1));
    };
    v4i* wslab = (v4i*) smem + wave * (a.slab_a / 16 / kWavesA);
    Slice cur = slice_at(s0);
    issue(cur, 0);
    if (tid < n_ent) s_prow[tid] = div_small(s_pos_ent[tid], k, __builtin_amdgcn_rcpf((float) k));  // position ->
    if (tid < T) s_prow[n_ent + tid] = tid;                                                            // its token's row
    __syncthreads();  // activations, codebooks and positions are in LDS

    // 4. each chunk: the wave's rows into its LDS slab, then against every entry of the slice's group, tpr lanes per
    //    row; a finished slice's h = silu(gate) * up and its Q8_1 block for each entry
    const int tpr = 64 / rpw;
    const int lr = lane / tpr, l = lane % tpr;
    const uint8_t* row = (const uint8_t*) wslab + (uint64_t) lr * gu_row;
    for (int sl = s0; sl < s1; ++sl) {
        const Slice nxt = sl + 1 < s1 ? slice_at(sl + 1) : cur;
        const int p0 = cur.p0, n_e = cur.n_e;
        for (int c = 0; c < nchunks; ++c) {
#pragma unroll
            for (int i = 0; i < kWLoadsA; ++i)
                if (lane + 64 * i < np) wslab[lane + 64 * i] = reg[i];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave's LDS writes land before its reads
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            if (c + 1 < nchunks) issue(cur, c + 1);
            else if (sl + 1 < s1) issue(nxt, 0);
            for (int e0 = 0; e0 < n_e; e0 += kNC) {
                const int n = min(kNC, n_e - e0);
                // the entries' activation rows, looked up once per pass for the block types with a long unit
                // decode; a Q8_0 unit is a single load and dot, where the four live offsets cost more than the
                // lookups they save
                constexpr bool kHoist = GT != TSX_Q8_0;
                int xo[kNC], xso[kNC];
#pragma unroll
                for (int cc = 0; cc < kNC; ++cc) {
                    xo[cc] = xso[cc] = 0;
                    if (kHoist && cc < n) {
                        const int xr = s_prow[p0 + e0 + cc];
                        xo[cc] = (int) __umul24((unsigned) xr, (unsigned) N);
                        xso[cc] = (int) __umul24((unsigned) xr, (unsigned) NU);
                    }
                }
                float acc[kNC] = {0.f, 0.f, 0.f, 0.f};
                for (int u = l; u < NU; u += tpr) {
                    Unit w;
                    unit_load<GT>(row, u, w, grid);
#pragma unroll
                    for (int cc = 0; cc < kNC; ++cc) {
                        if (cc < n) {
                            Act xa;
                            if constexpr (kHoist) {
                                act_planes(s_xq + xo[cc] + 32 * u, s_xd + xso[cc] + u, xa);
                            } else {
                                const int xr = s_prow[p0 + e0 + cc];
                                act_planes(s_xq + xr * N + 32 * u, s_xd + xr * NU + u, xa);
                            }
                            int S, M;
                            acc[cc] += unit_dot<GT>(w, xa, S, M);
                        }
                    }
                }
                switch (tpr) {  // the tpr lanes of a row are consecutive and tpr divides 64
                    case 16: sum_acc<16>(acc, T); break;
                    case 32: sum_acc<32>(acc, T); break;
                    default: sum_acc<64>(acc, T); break;
                }
                if (l == 0) {
                    const int col = (w_up ? kSliceA : 0) + c * rows_c + wr0 + lr;
                    for (int cc = 0; cc < n; ++cc) s_gu[e0 + cc][col] = acc[cc];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave's reads are done before the next chunk
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        __syncthreads();
        {  // 32-lane group e takes entry e (all lanes take part)
            const int e = min(tid >> 5, kMaxTok - 1), i = tid & 31;
            const float gt = s_gu[e][i];
            const float h = (gt / (1.0f + expf(-gt))) * s_gu[e][kSliceA + i];
            const float amax = lanes_reduce<32>(fabsf(h), OpMax());
            const float dd = q8_1_scale(amax);
            if ((tid >> 5) < n_e) {
                const int64_t p = p0 + e;
                a.hc[p * FF + kSliceA * cur.j + i] = (int8_t) q8_1_code_rd(h, amax, dd, q8_1_rcp(dd));
                if (i == 0) a.hd[p * (FF / 32) + cur.j] = h2f(f2h(dd));
            }
        }
        if (sl + 1 < s1) __syncthreads();  // s_gu is free for the next slice
        cur = nxt;
    }
}

// ------------------------------------------------------------------ launch A at one token
// At one token the slices above (32 gate/up row pairs of one expert: one Q8_1 block of h) number (k + 1) * n_ff / 32,
// 144 at configs[1], fewer than the 256 CUs, so 112 CUs would idle while the rest decode 64 rows each.  This launch
// spreads the (k + 1) * n_ff gate/up row pairs evenly over all the blocks instead, in the order [shared expert | pick 0 |
// pick 1 | ...], and writes h in fp32 (a Q8_1 block of h may straddle two blocks); launch B quantizes it.  A block
// needs the routing only as far as its last pick: a block of the shared expert issues its row loads at once, the others
// after as many argmax rounds as their picks need.  Row i of a block (pair i / 2, gate for even i, up for odd) belongs
// to wave i % 16; the 64 lanes of the wave take the row's units in turn and reduce the row with DPP; SwiGLU pairs the
// two rows through LDS.  The last block, whose last pick is the k-th, writes the tables launch B reads.
constexpr int kPiecesRow1 = 3;        // 16-byte loads per lane and row (rows of at most 3 KB)
constexpr int kMaxRowsW1 = 4;         // rows per wave
template <int GT>
__global__ void __launch_bounds__(kThreadsA) layer_gu1_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    constexpr int RPH = (rep_stores<GT>() + kThreadsA - 1) / kThreadsA;
    using Tab = std::conditional_t<(RPH > 0), RepTab<GT>, GridRef>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int32_t s_pick[16];
    __shared__ float s_pw[16];
    __shared__ float s_row[kWavesA * kMaxRowsW1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k;
    const tsx_expert_layout L = a.L;
    const int N = (int) L.n_embd, NU = N / 32, FF = (int) L.n_ff;
    const int sh = a.shared ? 1 : 0;
    const int P = (k + sh) * FF;  // row pairs: [shared | pick 0 | ... | pick k-1]
    const int nb = (int) gridDim.x, b = (int) blockIdx.x;
    // 32-bit: every wave of the block runs this, and a 64-bit division is a long scalar sequence that the CU's
    // one scalar unit would serialize over the 16 waves
    const int p0 = (int) ((uint32_t) b * (uint32_t) P / (uint32_t) nb),
              p1 = (int) ((uint32_t) (b + 1) * (uint32_t) P / (uint32_t) nb);
    const int nrows = 2 * (p1 - p0);
    const int rounds = max(0, (p1 - 1) / FF + 1 - sh);  // the picks this block's pairs reach

    // 0. the routing wave's logits first, then the codebooks and, by the other waves, the activations
    float lg[kRouteV];
    if (wave == 0 && rounds > 0) route_fetch(a.logits, a.n_expert, lane, lg);
    uint64_t rv[RPH > 0 ? RPH : 1];
    if constexpr (RPH > 0) rep_fetch<GT, RPH>(rv, tid, kThreadsA);
    const int nq_all = N / 4, xt = tid - 64, nxt = kThreadsA - 64;
    const float4* x4 = (const float4*) a.x;
    float4 xv[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(max(xt, 0) + nxt * i, nq_all - 1)];
    // the row loads below must not be issued ahead of these: a wait for these would then wait for the rows too
    __builtin_amdgcn_sched_barrier(0);
    const int rows_w = a.rows_w;
    const uint64_t gu_row = L.gu_row;
    const int ppr = (int) (gu_row / 16);  // 16-byte pieces per row
    const int cpr = (ppr + 63) / 64;      // loads per lane and row
    const int my_rows = wave < nrows ? (nrows - 1 - wave) / kWavesA + 1 : 0;  // rows wave, wave + 16, ...
    v4i* wslab = (v4i*) smem + wave * (rows_w * ppr);
    int8_t* s_xq = (int8_t*) (smem + (size_t) kWavesA * rows_w * gu_row + rep_lds_bytes<GT>());
    float* s_xd = (float*) (s_xq + N);

    // the rest for the wave's row count as straight-line code: the loads of all its rows in flight together, and
    // every row's unit decode independent of the others', so all their codebook lookups are in flight at once
    auto body = [&](auto RC) {
        constexpr int R = decltype(RC)::value;
        v4i reg[R > 0 ? R : 1][kPiecesRow1];
        // row j of the wave (block row wave + 16 j): pair p0 + i / 2, gate rows for even i, up rows for odd; the
        // address is the same in every lane
        auto row_base = [&](int j) -> uintptr_t {
            const int i = wave + kWavesA * j, pr = p0 + i / 2, slot = pr / FF, r = pr - slot * FF;
            const uint8_t* blob = slot < sh ? a.shared : a.blobs + (uint64_t) s_pick[slot - sh] * a.stride;
            return (uintptr_t) (blob + ((i & 1) ? L.up_off : 0) + (uint64_t) r * gu_row);
        };
        auto issue = [&]() {
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const gbl_ptr<const v4i> src = gbl_at<v4i>(row_base(j));
#pragma unroll
                for (int c = 0; c < kPiecesRow1; ++c)
                    if (c < cpr) reg[j][c] = __builtin_nontemporal_load(src + min(lane + 64 * c, ppr - 1));
            }
        };
        // a block of the shared expert alone needs no routing: its rows are requested before anything else waits
        if (R > 0 && rounds == 0) issue();
        __builtin_amdgcn_sched_barrier(0);

        // 1. routing (wave 0, as many rounds as the block's picks need) while the other waves quantize x into LDS
        if (wave == 0) {
            if (rounds > 0) route_select(lg, a.n_expert, rounds, lane, s_pick, s_pw);
        } else {
            for (int base = 0; base < nq_all; base += nxt * kXLoads) {
                if (base > 0) {
#pragma unroll
                    for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(base + xt + nxt * i, nq_all - 1)];
                }
#pragma unroll
                for (int i = 0; i < kXLoads; ++i) {
                    const int qd = base + xt + nxt * i;
                    if (base + nxt * i < nq_all)  // the same for every thread of these waves
                        q8_1_quad_to_lds(xv[i], qd < nq_all, s_xq + 4 * qd, s_xd + qd / 8, xt & 7);
                }
            }
        }
        Tab grid;
        if constexpr (RPH > 0) {
            uint8_t* tabs = smem + (size_t) kWavesA * rows_w * gu_row;
            rep_store<GT, RPH>(tabs, rv, tid, kThreadsA);
            grid = rep_view<GT>(tabs);
        } else {
            grid = grid_const();
        }
        __syncthreads();  // picks, activations and codebooks are in LDS
        if (R > 0 && rounds > 0) issue();
        __builtin_amdgcn_sched_barrier(0);
        if (rounds == k && b == nb - 1) {  // the tables launch B reads: group g = pick g, entry g, position g
            if (tid < k) {
                a.ids[tid] = s_pick[tid];
                a.wts[tid] = s_pw[tid];
                a.tab->wts[tid] = s_pw[tid];
                a.tab->ent_pos[tid] = tid;
                a.tab->grp_expert[tid] = s_pick[tid];
            }
            if (tid <= k) a.tab->grp_start[tid] = tid;
            if (tid == 0) a.tab->n_groups = k;
        }
        if constexpr (R > 0) {
            // 2. the rows into the wave's slab, then each row's dot with x, the 64 lanes reduced with DPP
#pragma unroll
            for (int j = 0; j < R; ++j)
#pragma unroll
                for (int c = 0; c < kPiecesRow1; ++c)
                    if (c < cpr && lane + 64 * c < ppr) wslab[j * ppr + lane + 64 * c] = reg[j][c];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave's LDS writes land before its reads
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            float acc[R] = {};
            for (int u = lane; u < NU; u += 64) {
                Act xa;
                act_planes(s_xq + 32 * u, s_xd + u, xa);
                Unit w[R];
#pragma unroll
                for (int j = 0; j < R; ++j) unit_load<GT>((const uint8_t*) (wslab + j * ppr), u, w[j], grid);
#pragma unroll
                for (int j = 0; j < R; ++j) {
                    int S, M;
                    acc[j] += unit_dot<GT>(w[j], xa, S, M);
                }
            }
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const float v = lanes_sum<64>(acc[j]);
                if (lane == 0) s_row[wave + kWavesA * j] = v;
            }
        }
        __syncthreads();
    };
    switch (my_rows) {  // the same in every lane of the wave; every case holds the same two block barriers
        case 0: body(std::integral_constant<int, 0>{}); break;
        case 1: body(std::integral_constant<int, 1>{}); break;
        case 2: body(std::integral_constant<int, 2>{}); break;
        case 3: body(std::integral_constant<int, 3>{}); break;
        default: body(std::integral_constant<int, 4>{}); break;
    }
    // 3. h = silu(gate) * up per pair (the product rounded on its own), in fp32 at its position: pick j -> j, shared -> k
    for (int i = tid; 2 * i < nrows; i += kThreadsA) {
        const int pr = p0 + i, slot = pr / FF, r = pr - slot * FF;
        const int pos = slot < sh ? k : slot - sh;
        const float gt = s_row[2 * i];
        a.hf[(int64_t) pos * FF + r] = (gt / (1.0f + expf(-gt))) * s_row[2 * i + 1];
    }
}

// ------------------------------------------------------------------ launch A at one token, slot by slot
// The one-token launch above gives each block a run of consecutive row pairs, so the blocks of the last pick wait for
// all k rounds of the top-k before they can request a row, and the launch ends with them.  Here every block takes the
// same pairs [q0, q1) = [n_ff b / nb, n_ff (b + 1) / nb) of EVERY slot (slot 0 the shared expert when there is one,
// then picks 0 .. k-1): the blocks have equal work and equal routing, and within a block each slot's waves request
// their rows as soon as the routing wave (wave 0) has published that slot's pick in LDS, so the early picks' rows are
// in flight, and then dotted, while the later rounds still run; the shared expert's rows are requested at once.
// Waves are dealt to the slots from the last slot backwards (the routing wave first, to the last pick, whose id it
// knows first), as evenly as 16 waves allow; a slot's rows (gate and up of each pair, in pair order) are split over
// its waves (the host's table, s1_wave).  Waves 1-15 quantize x into LDS and store the codebook copies while wave 0
// routes, and count themselves in an LDS word that every wave reads before its first dot: the block meets only at
// the start (before anything waits for memory) and at the end, so no wave idles at a barrier while the routing runs.
// Launch B is unchanged: it reads h in fp32 and the tables block 0 writes.
constexpr int kRowsS1 = 64;  // rows of a block: slots x 2 pairs per slot, at most
template <int GT>
__global__ void __launch_bounds__(kThreadsA) layer_gu1s_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    constexpr int kHelp = kThreadsA - 64;  // the threads of waves 1-15
    constexpr int RPH = (rep_stores<GT>() + kHelp - 1) / kHelp;
    using Tab = std::conditional_t<(RPH > 0), RepTab<GT>, GridRef>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int32_t s_pub[16];  // pick j + 1 once wave 0 has found it (0 before)
    __shared__ int32_t s_ready;    // helper waves whose x planes and codebook copies are in LDS
    __shared__ int32_t s_ids[16];
    __shared__ float s_pw[16];
    __shared__ float s_row[kRowsS1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k;
    const tsx_expert_layout L = a.L;
    const int N = (int) L.n_embd, NU = N / 32, FF = (int) L.n_ff;
    const int sh = a.shared ? 1 : 0, S = k + sh;
    const int b = (int) blockIdx.x;
    // no division here: every wave runs this prologue, and the CU's one scalar unit would serialize a division's
    // long scalar sequence over the 16 waves (a 64-bit one held the last wave ~1.3 us)
    const int q0 = b * a.s1_ppb, q1 = q0 + a.s1_ppb;
    const int rs = 2 * a.s1_ppb;  // rows of each slot in this block
    // this wave's slot and its rows of the slot (the host's table: tsx_moe_decode_layer)
    const int wm = a.s1_wave[wave];
    const int slot = wm & 255, j0 = (wm >> 8) & 255, j1 = wm >> 16;
    const int my_rows = j1 - j0;

    if (tid < 16) s_pub[tid] = 0;
    if (tid == 16) s_ready = 0;
    // 0. requested first: wave 0 the logits, waves 1-15 the codebooks and the activations
    float lg[kRouteV];
    if (wave == 0) route_fetch(a.logits, a.n_expert, lane, lg);
    uint64_t rv[RPH > 0 ? RPH : 1];
    if constexpr (RPH > 0)
        if (wave > 0) rep_fetch<GT, RPH>(rv, tid - 64, kHelp);
    const int nq_all = N / 4, xt = tid - 64, nxt = kHelp;
    const float4* x4 = (const float4*) a.x;
    float4 xv[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(max(xt, 0) + nxt * i, nq_all - 1)];
    __builtin_amdgcn_sched_barrier(0);
    // the words above are set before any wave polls them: the block meets once here, while the loads are in flight
    // (nothing waits for them yet, and every wave of the block has started within ~0.1 us)
    __syncthreads();
    const uint64_t gu_row = L.gu_row;
    const int ppr = (int) (gu_row / 16), cpr = (ppr + 63) / 64;
    v4i* wslab = (v4i*) smem + wave * (a.rows_w * ppr);
    uint8_t* tabs = smem + (size_t) kWavesA * a.rows_w * gu_row;
    int8_t* s_xq = (int8_t*) (tabs + rep_lds_bytes<GT>());
    float* s_xd = (float*) (s_xq + N);

    // a wave's rows: j0 + j of its slot, pair q0 + (j0 + j) / 2, gate rows for even, up rows for odd (the address is
    // the same in every lane); issued into registers, then into the wave's slab, dotted with x, reduced over the wave
    auto rows = [&](auto RC, auto& reg, const uint8_t* blob) {
        constexpr int R = decltype(RC)::value;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int jj = j0 + j;
            const gbl_ptr<const v4i> src =
                gbl_at<v4i>((uintptr_t) (blob + ((jj & 1) ? L.up_off : 0) + (uint64_t) (q0 + jj / 2) * gu_row));
#pragma unroll
            for (int c = 0; c < kPiecesRow1; ++c)
                if (c < cpr) reg[j][c] = __builtin_nontemporal_load(src + min(lane + 64 * c, ppr - 1));
        }
    };
    auto dots = [&](auto RC, auto& reg, const Tab& grid) {
        constexpr int R = decltype(RC)::value;
        // x and the codebooks: every helper wave has counted itself in s_ready after its LDS stores
        while (__hip_atomic_load(&s_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kWavesA - 1)
            __builtin_amdgcn_s_sleep(1);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int c = 0; c < kPiecesRow1; ++c)
                if (c < cpr && lane + 64 * c < ppr) wslab[j * ppr + lane + 64 * c] = reg[j][c];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave's LDS writes land before its reads
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        float acc[R] = {};
        for (int u = lane; u < NU; u += 64) {
            Act xa;
            act_planes(s_xq + 32 * u, s_xd + u, xa);
            Unit w[R];
#pragma unroll
            for (int j = 0; j < R; ++j) unit_load<GT>((const uint8_t*) (wslab + j * ppr), u, w[j], grid);
#pragma unroll
            for (int j = 0; j < R; ++j) {
                int Sx, Mx;
                acc[j] += unit_dot<GT>(w[j], xa, Sx, Mx);
            }
        }
        // every row's 64-lane sum first, so that the reduction chains interleave, then lane 0's stores
        float v[R];
#pragma unroll
        for (int j = 0; j < R; ++j) v[j] = lanes_sum<64>(acc[j]);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < R; ++j) s_row[slot * rs + j0 + j] = v[j];
        }
    };
    // the slot's pick, polled in LDS until wave 0 has published it (relaxed atomic loads: a fresh ds_read every time
    // round)
    auto pick_blob = [&]() -> const uint8_t* {
        if (sh && slot == 0) return a.shared;
        int id1;
        while ((id1 = __hip_atomic_load(s_pub + slot - sh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
            __builtin_amdgcn_s_sleep(1);
        return a.blobs + (uint64_t) (id1 - 1) * a.stride;
    };
    // per row count (the same in every lane of a wave) as straight-line code
    auto with_rows = [&](auto fn) {
        switch (my_rows) {
            case 0: fn(std::integral_constant<int, 0>{}); break;
            case 1: fn(std::integral_constant<int, 1>{}); break;
            case 2: fn(std::integral_constant<int, 2>{}); break;
            case 3: fn(std::integral_constant<int, 3>{}); break;
            default: fn(std::integral_constant<int, 4>{}); break;
        }
    };

    if (wave == 0) {
        // 1. the routing, then this wave's rows of the last pick; at raised issue priority, for the other waves
        //    dot the early picks' rows on the same SIMD meanwhile
        __builtin_amdgcn_s_setprio(2);
        route_publish(lg, a.n_expert, k, lane, s_pub, s_ids, s_pw, [] {});
        __builtin_amdgcn_s_setprio(0);
        Tab grid;
        if constexpr (RPH > 0) grid = rep_view<GT>(tabs);
        else grid = grid_const();
        with_rows([&](auto RC) {
            constexpr int R = decltype(RC)::value;
            if constexpr (R > 0) {
                v4i reg[R][kPiecesRow1];
                rows(RC, reg, pick_blob());
                dots(RC, reg, grid);
            }
        });
    } else {
        // 1. x into Q8_1 LDS planes and the codebook copies, while wave 0 routes (one copy of this code for every
        //    helper wave, ahead of the per-row-count code)
        for (int bq = 0; bq < nq_all; bq += nxt * kXLoads) {
            if (bq > 0) {
#pragma unroll
                for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(bq + xt + nxt * i, nq_all - 1)];
            }
#pragma unroll
            for (int i = 0; i < kXLoads; ++i) {
                const int qd = bq + xt + nxt * i;
                if (bq + (xt & ~63) + nxt * i < nq_all)  // whole waves: one with no quad of x skips the quantize
                    q8_1_quad_to_lds(xv[i], qd < nq_all, s_xq + 4 * qd, s_xd + qd / 8, xt & 7);
            }
        }
        Tab grid;
        if constexpr (RPH > 0) grid = rep_store<GT, RPH>(tabs, rv, tid - 64, kHelp);
        else grid = grid_const();
        // this wave's LDS stores are done: count it in (read by every wave before its first dot)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_fetch_add(&s_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        with_rows([&](auto RC) {
            constexpr int R = decltype(RC)::value;
            v4i reg[R > 0 ? R : 1][kPiecesRow1];
            // 2. the rows (the shared expert's at once, a routed slot's once its pick is out), their dots; the row
            //    loads come after the stores above, for a load issued on one path only would make the waits for x
            //    and the codebooks wait for it too
            if constexpr (R > 0) {
                rows(RC, reg, pick_blob());
                dots(RC, reg, grid);
            }
        });
    }
    __syncthreads();  // every row's dot is in s_row; the ids and weights in s_ids / s_pw
    // 3. h = silu(gate) * up per pair (the product rounded on its own), in fp32 at its position: pick j -> j,
    //    shared -> k; block 0 writes the tables launch B reads (group g = pick g, entry g, position g)
    for (int i = tid; i < S * (q1 - q0); i += kThreadsA) {
        const int s = i / (q1 - q0), pr = q0 + i % (q1 - q0);
        const int pos = s < sh ? k : s - sh;
        const float gt = s_row[s * rs + 2 * (pr - q0)];
        a.hf[(int64_t) pos * FF + pr] = (gt / (1.0f + expf(-gt))) * s_row[s * rs + 2 * (pr - q0) + 1];
    }
    if (b == 0) {
        if (tid < k) {
            a.ids[tid] = s_ids[tid];
            a.wts[tid] = s_pw[tid];
            a.tab->wts[tid] = s_pw[tid];
            a.tab->ent_pos[tid] = tid;
            a.tab->grp_expert[tid] = s_ids[tid];
        }
        if (tid <= k) a.tab->grp_start[tid] = tid;
        if (tid == 0) a.tab->n_groups = k;
    }
}

// ------------------------------------------------------------------ launch A, a few tokens, group by group
// Two to kTokT tokens: as layer_gu1s_kernel, every block takes the same pairs [q0, q1) of every expert the call
// uses, so every CU has the same rows however the routing falls; but the rows are those of the groups (each distinct
// expert once, with every entry that picked it, and the shared expert with every token), for at one token a row's
// decode is the costly part and several tokens' picks coincide (correlated verify tokens: ~18 distinct experts of 32
// picks).  Waves 0..T-1 route one token each; the last to finish groups the entries (layer_gu_kernel's order: expert
// id, then entry) and publishes the group count in LDS, while waves kTokT..15 quantize every token's activations to
// Q8_1 planes and store the codebook copies.  Then the block's rows - group g's row j, j < 2 ppb, the shared
// expert's last - are dealt to the waves in turn, each wave requests all of its rows at once (at most kItemsT), and
// dots each, decoded once, with every entry of its group.  h leaves in fp32 at the entries' positions in expert order,
// the shared expert's at n_ent + t, as launch B reads them.
constexpr int kTokT = 4;                 // tokens of this launch at most
constexpr int kItemsT = 9;               // rows per wave at most (4 tokens x 8 picks + 1 shared, 4 rows each, over 16)
// rows per wave at most for rows of CPR 16-byte pieces per lane: rows of over 1 KB hold twice the registers in flight
// per row, and nine (seven, IQ3_S) of them spilled
template <int CPR> constexpr int items_t() { return CPR == 1 ? kItemsT : 6; }
constexpr int kRowsGB = 2;               // rows a wave decodes together (its slab)
constexpr int kRowsGut = (kMaxEnt + kTokT) * 4;  // s_row: (position, row of the block) at most 2 ppb = 4 rows

template <int GT, int CPR>
__global__ void __launch_bounds__(kThreadsA) layer_gut_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    constexpr int kHelp = kThreadsA - 64 * kTokT;  // the threads of waves kTokT..15
    constexpr int RPH = (rep_stores<GT>() + kHelp - 1) / kHelp;
    using Tab = std::conditional_t<(RPH > 0), RepTab<GT>, GridRef>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int32_t s_ready;    // helper waves whose x planes and codebook copies are in LDS
    __shared__ int32_t s_routed;   // routing waves done
    __shared__ int32_t s_groups;   // the group count + 1 once the entries are grouped (0 before)
    __shared__ int32_t s_ids[kMaxEnt], s_pos_ent[kMaxEnt], s_ent_pos[kMaxEnt];
    __shared__ __attribute__((aligned(16))) int32_t s_key[kMaxEnt];  // the grouping's keys
    __shared__ int32_t s_grp_expert[kMaxEnt], s_grp_start[kMaxEnt + 1];
    __shared__ float s_pw[kMaxEnt];
    __shared__ float s_row[kRowsGut];  // (position, row j of the block) -> its dot

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k, T = a.n_tok, n_ent = T * k;
    const tsx_expert_layout L = a.L;
    const int N = (int) L.n_embd, NU = N / 32, FF = (int) L.n_ff;
    const int sh = a.shared ? 1 : 0;
    const int b = (int) blockIdx.x;
    const int q0 = b * a.s1_ppb, np = a.s1_ppb, rs = 2 * np;  // no division in the prologue (layer_gu1s_kernel)
    const int lrs = rs == 4 ? 2 : rs == 2 ? 1 : 0;              // rs is 2 or 4
    const float rk = __builtin_amdgcn_rcpf((float) k);        // entry e -> token e / k (div_small)

    if (tid == 0) s_ready = 0;
    if (tid == 1) s_routed = 0;
    if (tid == 2) s_groups = 0;
    // 0. requested first: the routing waves their token's logits, the others the codebooks and the activations
    float lg[kRouteV];
    if (wave < T) route_fetch(a.logits + (int64_t) wave * a.n_expert, a.n_expert, lane, lg);
    const int ht = tid - 64 * kTokT;
    uint64_t rv[RPH > 0 ? RPH : 1];
    if constexpr (RPH > 0)
        if (wave >= kTokT) rep_fetch<GT, RPH>(rv, ht, kHelp);
    const int nq_all = T * N / 4;
    const float4* x4 = (const float4*) a.x;
    float4 xv[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(max(ht, 0) + kHelp * i, nq_all - 1)];
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();  // the words above are set before any wave polls them
    const uint64_t gu_row = L.gu_row;
    const int ppr = (int) (gu_row / 16);
    v4i* wslab = (v4i*) smem + wave * (kRowsGB * ppr);  // a batch of rows per wave
    uint8_t* tabs = smem + (size_t) kWavesA * kRowsGB * gu_row;
    int8_t* s_xq = (int8_t*) (tabs + rep_lds_bytes<GT>());
    float* s_xd = (float*) (s_xq + (size_t) T * N);

    // the entries' ranks in (expert, entry) order and the groups (layer_gu_kernel's grouping), by one wave
    // (each entry's rank counted against the 64 keys read back from LDS four at a time - a loop of dependent
    // readlanes took ~1 us - then the ids and entries moved to their ranks' lanes with ds_permute, a cross-lane push)
    auto group = [&]() {
        const int e = lane;
        const int id = e < n_ent ? s_ids[e] : 0;
        const int key = e < n_ent ? id * 64 + e : INT_MAX;
        __hip_atomic_store(s_key + e, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // the wave's own stores, then its reads
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        int rank = 0;
#pragma unroll
        for (int q = 0; q < kMaxEnt / 4; ++q) {
            const int4 v = ((const int4*) s_key)[q];
            rank += (v.x < key) + (v.y < key) + (v.z < key) + (v.w < key);
        }
        const int dst = (e < n_ent ? rank : e) * 4;  // lanes past the entries keep their own place
        const int xs = __builtin_amdgcn_ds_permute(dst, e < n_ent ? id : -1);
        const int es = __builtin_amdgcn_ds_permute(dst, e);
        if (e < n_ent) s_ent_pos[e] = rank;
        if (lane < n_ent) s_pos_ent[lane] = es;
        const int xp = lane < n_ent ? xs : -1;
        const int xprev = __shfl_up(xs, 1, 64);
        const bool start = lane < n_ent && (lane == 0 || xprev != xp);
        const uint64_t mask = __ballot(start);
        const int ng = __builtin_popcountll(mask);
        if (start) {
            const int g = __builtin_popcountll(mask & (~0ull >> (63 - lane))) - 1;
            s_grp_expert[g] = xp;
            s_grp_start[g] = lane;
        }
        if (lane == 0) s_grp_start[ng] = n_ent;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_store(&s_groups, ng + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };

    Tab grid;
    if (wave < kTokT) {
        if (wave < T) {
            // 1. the routing of token `wave`, at raised issue priority; the last wave to finish groups the entries
            __builtin_amdgcn_s_setprio(2);
            route_select(lg, a.n_expert, k, lane, s_ids + wave * k, s_pw + wave * k);
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            int done = 0;
            if (lane == 0) done = __hip_atomic_fetch_add(&s_routed, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            done = __builtin_amdgcn_readfirstlane(done);
            if (done == T - 1) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                __builtin_amdgcn_s_setprio(2);
                group();
                __builtin_amdgcn_s_setprio(0);
            }
        }
        if constexpr (RPH > 0) grid = rep_view<GT>(tabs);
        else grid = grid_const();
    } else {
        // 1. every token's x into Q8_1 LDS planes and the codebook copies, while the routing waves route
        for (int bq = 0; bq < nq_all; bq += kHelp * kXLoads) {
            if (bq > 0) {
#pragma unroll
                for (int i = 0; i < kXLoads; ++i) xv[i] = x4[min(bq + ht + kHelp * i, nq_all - 1)];
            }
#pragma unroll
            for (int i = 0; i < kXLoads; ++i) {
                const int qd = bq + ht + kHelp * i;
                if (bq + (ht & ~63) + kHelp * i < nq_all)  // whole waves
                    q8_1_quad_to_lds(xv[i], qd < nq_all, s_xq + 4 * qd, s_xd + qd / 8, ht & 7);
            }
        }
        if constexpr (RPH > 0) grid = rep_store<GT, RPH>(tabs, rv, ht, kHelp);
        else grid = grid_const();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_fetch_add(&s_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // 2. the groups, polled in LDS; the block's rows: item i = group i >> lrs (the shared expert as group ng), row
    //    i & (rs - 1) of it, dealt to the waves in turn - the helpers first, the routing waves (done last) last
    int g1;
    while ((g1 = __hip_atomic_load(&s_groups, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int ng = g1 - 1, items = (ng + sh) << lrs;
    const int wpos = wave >= kTokT ? wave - kTokT : wave + (kWavesA - kTokT);
    constexpr int IT = items_t<CPR>();
    // every wave requests IT rows unconditionally (a row past its items repeats its last), so that the
    // compiler's wait counts stay exact
    v4i reg[IT][CPR];
    int it_g[IT], it_j[IT];
#pragma unroll
    for (int m = 0; m < IT; ++m) {
        const int i = min(wpos + kWavesA * m, items - 1);
        const int g = i >> lrs, j = i & (rs - 1);
        it_g[m] = g;
        it_j[m] = j;
        const uint8_t* blob = g < ng ? a.blobs + (uint64_t) s_grp_expert[g] * a.stride : a.shared;
        const gbl_ptr<const v4i> src =
            gbl_at<v4i>((uintptr_t) (blob + ((j & 1) ? L.up_off : 0) + (uint64_t) (q0 + j / 2) * gu_row));
#pragma unroll
        for (int c = 0; c < CPR; ++c) reg[m][c] = __builtin_nontemporal_load(src + min(lane + 64 * c, ppr - 1));
    }
    // x and the codebooks: every helper wave has counted itself in s_ready after its stores
    while (__hip_atomic_load(&s_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kWavesA - kTokT)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    // 3. the rows in batches of kRowsGB through the wave's slab, each unit of a row decoded once and dotted with
    //    every entry of the row's group (the shared expert: every token); the batch's rows decode together
#pragma unroll
    for (int bb = 0; bb < (IT + kRowsGB - 1) / kRowsGB; ++bb) {
        const int m0 = bb * kRowsGB, left = items - (wpos + kWavesA * m0);
        if (left <= 0) break;  // the same in every lane of the wave
        const int nrow = min(kRowsGB, (left + kWavesA - 1) / kWavesA);
        int lo[kRowsGB], n[kRowsGB];
        bool shr[kRowsGB];
#pragma unroll
        for (int r = 0; r < kRowsGB; ++r) {
            const int m = min(m0 + r, IT - 1), g = it_g[m];
            shr[r] = g >= ng;
            lo[r] = g < ng ? s_grp_start[g] : 0;
            n[r] = r < nrow ? (g < ng ? s_grp_start[g + 1] - lo[r] : T) : 0;
#pragma unroll
            for (int c = 0; c < CPR; ++c)
                if (r < nrow && lane + 64 * c < ppr) wslab[r * ppr + lane + 64 * c] = reg[m][c];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave's LDS writes land before its reads
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        float acc[kRowsGB][kTokT] = {};
        for (int u = lane; u < NU; u += 64) {
            Unit w[kRowsGB];
#pragma unroll
            for (int r = 0; r < kRowsGB; ++r)
                if (r < nrow) unit_load<GT>((const uint8_t*) (wslab + r * ppr), u, w[r], grid);
#pragma unroll
            for (int r = 0; r < kRowsGB; ++r) {
#pragma unroll
                for (int c = 0; c < kTokT; ++c) {
                    if (c < n[r]) {
                        // the entry's token (the shared expert: token c)
                        const int tk = shr[r] ? c : div_small(s_pos_ent[lo[r] + c], k, rk);
                        Act xa;
                        act_planes(s_xq + (size_t) tk * N + 32 * u, s_xd + tk * NU + u, xa);
                        int Sx, Mx;
                        acc[r][c] += unit_dot<GT>(w[r], xa, Sx, Mx);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRowsGB; ++r) {
            const int m = min(m0 + r, IT - 1), j = it_j[m];
#pragma unroll
            for (int c = 0; c < kTokT; ++c) {
                if (c < n[r]) {
                    const float v = lanes_sum<64>(acc[r][c]);
                    if (lane == 0) s_row[((shr[r] ? n_ent + c : lo[r] + c) << lrs) + j] = v;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the slab's reads are done before the next batch
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // overwrites it
    }
    __syncthreads();  // every dot is in s_row
    // 4. h = silu(gate) * up per (position, pair), the product rounded on its own, in fp32 at the position
    const int P = n_ent + (sh ? T : 0);
    for (int i = tid; i < P * np; i += kThreadsA) {
        const int pos = i / np, p = i - pos * np;
        const float* row = s_row + (pos << lrs) + 2 * p;
        const float gt = row[0];
        a.hf[(int64_t) pos * FF + q0 + p] = (gt / (1.0f + expf(-gt))) * row[1];
    }
    if (b == 0) {
        if (tid < n_ent) {
            a.ids[tid] = s_ids[tid];
            a.wts[tid] = s_pw[tid];
            a.tab->wts[tid] = s_pw[tid];
            a.tab->ent_pos[tid] = s_ent_pos[tid];
        }
        if (tid <= ng) {
            if (tid < ng) a.tab->grp_expert[tid] = s_grp_expert[tid];
            a.tab->grp_start[tid] = s_grp_start[tid];
        }
        if (tid == 0) a.tab->n_groups = ng;
    }
}

// ------------------------------------------------------------------ launch B
// Block b owns output rows [8 b, 8 b + 8).  It reads the tables and every entry's h in one round trip, then loads the
// 8 rows of every used expert's down matrix (and the shared expert's: 8 contiguous rows each) into LDS with every
// thread's loads in flight at once (chunks of groups when they exceed the slab), dots each row with its group's
// entries (tpr lanes per row, as many rows at once as the block has lanes for) and combines in pick order.
// NR: rounds of 16-byte row loads per thread in flight (kBLoads, or 1 when a chunk's pieces fit one round: fewer
// redundant clamped loads, and waits that stay exact)
template <int DT, int NR, int HL = kHLoads>
__global__ void __launch_bounds__(kThreadsB) layer_down_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    constexpr int RP = (rep_stores<DT>() + kThreadsB - 1) / kThreadsB;
    using Tab = std::conditional_t<(RP > 0), RepTab<DT>, GridRef>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ LayerTables s_tab;
    __shared__ float s_part[kMaxEnt + kMaxTok][kRowsB];
    __shared__ float s_sgate[kMaxTok];  // the token's shared-expert gate, sigmoid applied

    const int tid = threadIdx.x;
    const int T = a.n_tok, k = a.k, n_ent = T * k;
    const tsx_expert_layout L = a.L;
    const int N = (int) L.n_embd, FF = (int) L.n_ff, NUd = FF / 32;
    const uint64_t d_row = L.d_row;
    const int r0 = blockIdx.x * kRowsB;

    // requested together, the tables first (the first wait is for them alone): the tables, the codebooks and every
    // entry's h (codes, then scales: contiguous in the scratch, as in LDS), whose positions are fixed: n_tok * k
    // routed, then n_tok shared
    const uint32_t tw = ((const uint32_t*) a.tab)[min(tid, kTableWords - 1)];
    uint64_t rv[RP > 0 ? RP : 1];
    if constexpr (RP > 0) rep_fetch<DT, RP>(rv, tid, kThreadsB);
    const int P = n_ent + (a.shared ? T : 0);
    // h: the Q8_1 planes (16-byte pieces; n_ff is a multiple of 128), or fp32 h (float4 quads) quantized here
    const int nh = a.h_fp32 ? P * FF / 4 : (P * FF + P * NUd * 4) / 16;
    const v4i* hsrc = (const v4i*) (a.h_fp32 ? (const void*) a.hf : (const void*) a.hc);
    v4i hv[HL];
#pragma unroll
    for (int i = 0; i < HL; ++i) hv[i] = hsrc[min(tid + kThreadsB * i, nh - 1)];
    const float sg = a.shared ? a.sgate[(int64_t) min(tid, T - 1) * a.sg_stride] : 0.f;
    const int ty = min(tid / kRowsB, T - 1), ry = tid % kRowsB;  // the y value this thread combines into
    const float y0 = a.y[(int64_t) ty * N + r0 + ry];
    if (tid < kTableWords) ((uint32_t*) &s_tab)[tid] = tw;
    __syncthreads();
    const int ng = s_tab.n_groups;
    const int G = ng + (a.shared ? 1 : 0);  // group ng is the shared expert: positions [n_ent, n_ent + T)
    // where group g's 8 down rows start (group ng is the shared expert), read by each thread from the tables: no
    // block barrier between the tables and the row loads
    auto gsrc = [&](int g) {
        return (g < ng ? a.blobs + (uint64_t) s_tab.grp_expert[g] * a.stride : a.shared) + L.down_off +
               (uint64_t) r0 * d_row;
    };
    auto grp_lo = [&](int g) { return g < ng ? s_tab.grp_start[g] : n_ent; };
    auto grp_hi = [&](int g) { return g < ng ? s_tab.grp_start[g + 1] : n_ent + T; };

    // the groups' rows in chunks of gpc groups, every piece of a chunk in flight at once
    const int gb = (int) (kRowsB * d_row), ppg = gb / 16;  // bytes and 16-byte pieces of a group's 8 rows
    const int gpc = max(1, a.slab_b / gb), nchunks = (G + gpc - 1) / gpc;
    const float rppg = __builtin_amdgcn_rcpf((float) ppg);
    v4i reg[NR];
    auto issue = [&](int ch) {
        const int g0 = ch * gpc, np = min(gpc, G - g0) * ppg;
#pragma unroll
        for (int i = 0; i < NR; ++i) {  // unconditional (clamped) loads keep the wait counts exact
            const int q = min(tid + kThreadsB * i, np - 1), g = div_small(q, ppg, rppg), pp = q - g * ppg;
            reg[i] = __builtin_nontemporal_load(gbl_at<v4i>((uintptr_t) gsrc(g0 + g)) + pp);
        }
    };
    issue(0);
    // the row loads stay here, ahead of the work below (the compiler would otherwise sink them towards their use)
    __builtin_amdgcn_sched_barrier(0);

    // h into LDS: the prefetched pieces, then any rest
    if (tid < T) s_sgate[tid] = 1.0f / (1.0f + expf(-sg));  // the shared expert's gate, ahead of the combine
    int8_t* s_hq = (int8_t*) (smem + a.slab_b + rep_lds_bytes<DT>());
    float* s_hd = (float*) (s_hq + (size_t) P * FF);
    if (a.h_fp32) {  // every Q8_1 block of h from its eight quads (consecutive lanes), as launch A would write it
        // (the conditions are the same in every lane of a wave: whole waves take part in each block's reduction,
        // and a wave with no quad left skips the round)
        const int w0 = tid & ~63;
#pragma unroll
        for (int i = 0; i < HL; ++i) {
            const int q = tid + kThreadsB * i;
            if (kThreadsB * i + w0 < nh)
                q8_1_quad_to_lds(__builtin_bit_cast(float4, hv[i]), q < nh, s_hq + 4 * q, s_hd + q / 8, tid & 7);
        }
        for (int base = kThreadsB * HL; base + w0 < nh; base += kThreadsB) {
            const int q = base + tid;
            q8_1_quad_to_lds(__builtin_bit_cast(float4, hsrc[min(q, nh - 1)]), q < nh, s_hq + 4 * q, s_hd + q / 8,
                             tid & 7);
        }
    } else {
        v4i* hdst = (v4i*) s_hq;
#pragma unroll
        for (int i = 0; i < HL; ++i)
            if (tid + kThreadsB * i < nh) hdst[tid + kThreadsB * i] = hv[i];
        for (int idx = tid + kThreadsB * HL; idx < nh; idx += kThreadsB) hdst[idx] = hsrc[idx];
    }
    Tab grid;
    if constexpr (RP > 0) grid = rep_store<DT, RP>(smem + a.slab_b, rv, tid, kThreadsB);
    else grid = grid_const();

    v4i* slab = (v4i*) smem;
    for (int ch = 0; ch < nchunks; ++ch) {
        const int g0 = ch * gpc, gn = min(gpc, G - g0), np = gn * ppg;
#pragma unroll
        for (int i = 0; i < NR; ++i)
            if (tid + kThreadsB * i < np) slab[tid + kThreadsB * i] = reg[i];
        for (int q = tid + kThreadsB * NR; q < np; q += kThreadsB) {  // a chunk larger than the loads in flight
            const int g = q / ppg, pp = q - g * ppg;
            slab[q] = gbl_at<v4i>((uintptr_t) gsrc(g0 + g))[pp];
        }
        __syncthreads();  // the chunk (and h, the codebooks) are in LDS
        if (ch + 1 < nchunks) issue(ch + 1);
        const int R = gn * kRowsB;
        if (NUd == 8 || NUd == 16 || NUd == 32) {
            // items (row, unit) to consecutive threads, a row's NUd units to NUd lanes of one wave (whose rows then
            // share a group: NUd lanes per row, 64 / NUd rows per wave, 8 rows per group), in rounds of kThreadsB
            // items, kItemsB at a time (their codebook lookups in flight together); each item's unit is dotted with
            // every entry of its group and each row reduced over its lanes with DPP.  Rounds past the chunk's items
            // are skipped by whole waves, so every thread has at most one item more than any other
            const int items = R * NUd, lgu = NUd == 8 ? 3 : NUd == 16 ? 4 : 5;
            for (int m0 = 0; kThreadsB * m0 < items; m0 += kItemsB) {
                int rr[kItemsB], lo[kItemsB], hi[kItemsB], uu[kItemsB];
                Unit w[kItemsB];
#pragma unroll
                for (int m = 0; m < kItemsB; ++m) {
                    const int it = min(tid + kThreadsB * (m0 + m), items - 1), ri = it >> lgu, g = ri / kRowsB;
                    rr[m] = ri % kRowsB;
                    uu[m] = it & (NUd - 1);
                    lo[m] = grp_lo(g0 + g);
                    hi[m] = grp_hi(g0 + g);
                    if (kThreadsB * (m0 + m) + (tid & ~63) < items)  // whole waves (24-bit products: full rate)
                        unit_load<DT>((const uint8_t*) smem + __umul24(g, gb) + __umul24(rr[m], (uint32_t) d_row), uu[m],
                                      w[m], grid);
                }
#pragma unroll
                for (int m = 0; m < kItemsB; ++m) {
                    if (kThreadsB * (m0 + m) + (tid & ~63) < items) {
                        for (int e = lo[m]; e < hi[m]; ++e) {  // the same in every lane of the wave
                            Act xa;
                            act_planes(s_hq + __umul24(e, FF) + 32 * uu[m], s_hd + (e << lgu) + uu[m], xa);
                            int S, M;
                            const float v = unit_dot<DT>(w[m], xa, S, M);
                            const float t = NUd == 8 ? lanes_sum<8>(v) : NUd == 16 ? lanes_sum<16>(v) : lanes_sum<32>(v);
                            if ((tid & (NUd - 1)) == 0 && tid + kThreadsB * (m0 + m) < items) s_part[e][rr[m]] = t;
                        }
                    }
                }
            }
            __syncthreads();  // the chunk's rows are done before the next chunk overwrites the slab
            continue;
        }
        // rows ri = g * 8 + r of the chunk, tpr lanes each (consecutive lanes; tpr divides 64), in passes of
        // kThreadsB / tpr rows when the chunk has more
        int tpr = 64;
        while (tpr > 4 && R * tpr > kThreadsB) tpr >>= 1;
        const int l = tid % tpr;
        for (int ri = tid / tpr; ri < R; ri += kThreadsB / tpr) {
            const int g = ri / kRowsB, rr = ri % kRowsB;
            const uint8_t* row = (const uint8_t*) smem + g * gb + rr * d_row;
            const int q0 = grp_lo(g0 + g), q1 = grp_hi(g0 + g);
            for (int e0 = q0; e0 < q1; e0 += kNC) {
                const int n = min(kNC, q1 - e0);
                float acc[kNC] = {0.f, 0.f, 0.f, 0.f};
                for (int u = l; u < NUd; u += tpr) {
                    Unit w;
                    unit_load<DT>(row, u, w, grid);
#pragma unroll
                    for (int cc = 0; cc < kNC; ++cc) {
                        if (cc < n) {
                            Act xa;
                            act_planes(s_hq + (size_t) (e0 + cc) * FF + 32 * u, s_hd + (e0 + cc) * NUd + u, xa);
                            int S, M;
                            acc[cc] += unit_dot<DT>(w, xa, S, M);
                        }
                    }
                }
                switch (tpr) {
                    case 4: sum_acc<4>(acc, T); break;
                    case 8: sum_acc<8>(acc, T); break;
                    case 16: sum_acc<16>(acc, T); break;
                    case 32: sum_acc<32>(acc, T); break;
                    default: sum_acc<64>(acc, T); break;
                }
                if (l == 0)
                    for (int cc = 0; cc < n; ++cc) s_part[e0 + cc][rr] = acc[cc];
            }
        }
        __syncthreads();  // the chunk's rows are done before the next chunk overwrites the slab
    }

    // combine in pick order (tsx_moe_combine's arithmetic), into y
    if (tid < T * kRowsB) {
        const int t = tid / kRowsB, r = tid % kRowsB;
        const float* wr = s_tab.wts + t * k;
        const int32_t* ep = s_tab.ent_pos + t * k;
        // eight picks at a time, their weight and part reads issued together (one LDS round trip per eight, not two
        // per pick); the products are summed in pick order as before
        float acc = 0.f;
        for (int j0 = 0; j0 < k; j0 += 8) {
            float wv[8], pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int jj = min(j0 + i, k - 1);
                wv[i] = wr[jj];
                pv[i] = s_part[ep[jj]][r];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (j0 + i < k) acc = j0 + i == 0 ? wv[i] * pv[i] : __builtin_fmaf(wv[i], pv[i], acc);
        }
        if (a.shared) acc += s_sgate[t] * s_part[n_ent + t][r];
        a.y[(int64_t) t * N + r0 + r] = y0 + acc;
    }
}

// the MoE block's end (optional third launch, one block per token): h = (y * r) * norm_w, r = 1 / sqrt(mean(y^2) +
// eps), and h's Q8_1 image - tsx_moe_combine_norm's norm half.  A separate launch: the norm needs every column of y,
// which launch B's blocks finish on different XCDs, and a cross-block hand-off inside launch B (device-scope stores,
// a completion count, device-scope loads) measured slower than the launch boundary
__global__ void __launch_bounds__(kNormRowThreads) layer_norm_kernel(const float* __restrict__ y, int n,
                                                                     const float* __restrict__ norm_w, float eps,
                                                                     float* __restrict__ h, tsx_block_q8_1* __restrict__ hq) {
    constexpr int kPer = 4096 / kNormRowThreads;  // n <= 4096: every value's load in flight at once
    __shared__ float s_row[4096];
    __shared__ float s_red[kNormRowThreads / 64];
    const int t = blockIdx.x;
    float v[kPer];
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
        const int i = threadIdx.x + kNormRowThreads * m;
        v[m] = i < n ? y[(int64_t) t * n + i] : 0.f;
    }
    float q = 0.f;
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
        const int i = threadIdx.x + kNormRowThreads * m;
        if (i < n) s_row[i] = v[m];
        q += v[m] * v[m];
    }
    norm_row_out<kNormRowThreads>(s_row, q, n, norm_w, eps, h + (int64_t) t * n, hq ? hq + (int64_t) t * (n / 32) : nullptr,
                                  s_red);
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

// the largest rows_c in {32, 16, 8} whose gate + up chunk fits the slab with every wave's rows 16-byte aligned
int pick_rows_c(const tsx_expert_layout& L, int slab_a) {
    for (int rc = kSliceA; rc >= 8; rc >>= 1)
        if (2 * rc * L.gu_row <= (uint64_t) slab_a && ((2 * rc / kWavesA) * L.gu_row) % 16 == 0) return rc;
    return 0;
}
size_t rep_bytes(int type) {
    return (size_t) with_type(type, [](auto T) { return rep_lds_bytes<decltype(T)::value>(); });
}
size_t x_planes_bytes(const tsx_expert_layout& L, int n_tok) {
    return (size_t) n_tok * L.n_embd + (size_t) n_tok * (L.n_embd / 32) * 4;
}
size_t h_planes_bytes(const tsx_expert_layout& L, int n_tok, int k, bool shared) {
    const int P = n_tok * k + (shared ? n_tok : 0);
    return (size_t) P * L.n_ff + (size_t) P * (L.n_ff / 32) * 4;
}
// the largest slab (a multiple of `unit` bytes, at most `most`) that fits beside `fixed` bytes in `limit`
int fit_slab(size_t limit, size_t fixed, int most, int unit) {
    if (limit <= fixed) return 0;
    return (int) std::min<size_t>((size_t) most, (limit - fixed) / unit * unit);
}
size_t h_bytes(int n_tok, int k, int64_t n_ff) {  // codes then scales, the whole [n_tok * k + n_tok] positions
    const size_t P = (size_t) (n_tok * k + n_tok);
    return P * (size_t) n_ff + P * (size_t) (n_ff / 32) * 4;
}
constexpr size_t kLdsPerWorkgroup = 160 * 1024;  // gfx950
// lets a kernel take more than the default 64 KB of dynamic LDS: up to what its static LDS leaves of the 160 KB.
// Returns that limit (0 when the runtime refused); once per kernel.
size_t set_max_lds(const void* kern) {
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, kern) != hipSuccess) return 0;
    const size_t limit = kLdsPerWorkgroup - fa.sharedSizeBytes;
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int) limit) == hipSuccess ? limit : 0;
}
}  // namespace

// The scratch of tsx_moe_decode_layer_noalloc: one copy on every GPU the library runs on, held until the process
// ends.  Host code never passes this name to a kernel (on the host it is a stand-in, not a device address): it uses
// the per-device address that hipGetSymbolAddress returned for it.
constexpr size_t kNoAllocScratchBytes = 128 * 1024;
static __device__ __align__(256) uint8_t noalloc_scratch[kNoAllocScratchBytes];
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};
}  // namespace

// The current device's address of noalloc_scratch (looked up once per device, with that device current); nullptr
// with the error recorded and *rc set (the hipError_t, or TSX_ERR_UNSUPPORTED for a device index past the table)
// when the runtime refuses.
void* noalloc_scratch_ptr(int* rc) {
    int device = -1;
    const hipError_t ge = hipGetDevice(&device);
    if (ge != hipSuccess || device < 0 || device >= kMaxDevices) {
        set_error("tsx_moe_decode_layer_noalloc: no current device (or one past the first %d)", kMaxDevices);
        if (rc) *rc = ge != hipSuccess ? (int) ge : (int) TSX_ERR_UNSUPPORTED;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("tsx_moe_decode_layer_noalloc: hipGetSymbolAddress on device %d: %s", device,
                      hipGetErrorString(e));
            if (rc) *rc = e != hipSuccess ? (int) e : (int) hipErrorInvalidSymbol;
            return nullptr;
        }
        g_noalloc_ptr[device] = p;
    }
    return g_noalloc_ptr[device];
}

}  // namespace tsx

using namespace tsx;

extern "C" {

TSX_API size_t tsx_moe_decode_layer_scratch_bytes(int n_tok, int k, int64_t n_ff) {
    if (n_tok < 1 || k < 1 || n_ff <= 0 || n_ff % 32 != 0) return 0;
    // h as Q8_1 planes, or in fp32 wherever a slot-by-slot launch A can take the call (one token; up to kTokT tokens
    // at n_ff <= 2 kBlocksA, two rows of a slot per block): every routed position and every token's shared one
    const bool fp32 = n_tok == 1 || (n_tok <= kTokT && n_ff <= 2 * kBlocksA);
    const size_t h32 = fp32 ? (size_t) (n_tok * k + n_tok) * (size_t) n_ff * 4 : 0;
    const size_t h = std::max(h_bytes(n_tok, k, n_ff), h32);
    return kTablesBytes + ((h + 255) & ~(size_t) 255);
}

// tsx_moe_decode_layer, and with norm_w the norm epilogue of tsx_moe_decode_layer_norm
static int decode_layer(const tsx_expert_layout* Lp, const void* blobs, uint64_t stride, int n_expert, int k,
                        int n_tok, const float* logits, const float* x, const void* shared, const float* sgate,
                        int sg_stride, float* y, int32_t* ids, float* wts, const float* norm_w, float eps, float* h,
                        void* hq, void* scratch, void* stream) {
    TSX_REQUIRE(Lp != nullptr, "tsx_moe_decode_layer: null layout");
    const tsx_expert_layout L = *Lp;
    if (!tsx_moe_expert_supported(L.gu_type, L.d_type, L.n_embd, L.n_ff) || L.n_embd > 4096 || L.n_ff > 1024 ||
        L.n_ff % 128 != 0 || n_tok < 1 || n_tok > kMaxTok || k < 1 || n_tok * k > kMaxEnt || n_expert % 64 != 0 ||
        n_expert > kMaxExperts || k > n_expert) {
        set_error("tsx_moe_decode_layer: types (%d, %d) at %lld x %lld, %d tokens, %d experts top-%d not supported "
                  "(n_embd <= 4096, n_ff a multiple of 128 up to 1024, 1..8 tokens, tokens * k <= 64, experts a "
                  "multiple of 64 up to 512)",
                  L.gu_type, L.d_type, (long long) L.n_embd, (long long) L.n_ff, n_tok, n_expert, k);
        return TSX_ERR_UNSUPPORTED;
    }
    // LDS of each launch: the weight slab, the codebook copies, the activations (x, or every entry's h); the slabs
    // take what the rest leaves of each kernel's limit
    size_t lim_a = 0, lim_b = 0;
    with_type(L.gu_type, [&](auto T) {
        static const size_t limit = set_max_lds((const void*) layer_gu_kernel<decltype(T)::value>);
        lim_a = limit;
        return 0;
    });
    with_type(L.d_type, [&](auto T) {
        static const size_t limit = set_max_lds((const void*) layer_down_kernel<decltype(T)::value, kBLoads>);
        static const size_t limit1 = set_max_lds((const void*) layer_down_kernel<decltype(T)::value, 1>);
        static const size_t limit2 = set_max_lds((const void*) layer_down_kernel<decltype(T)::value, kBLoads, kHLoadsT>);
        static const size_t limit3 = set_max_lds((const void*) layer_down_kernel<decltype(T)::value, 1, kHLoadsT>);
        lim_b = std::min(std::min(limit, limit1), std::min(limit2, limit3));
        return 0;
    });
    const size_t fixed_a = rep_bytes(L.gu_type) + x_planes_bytes(L, n_tok);
    const size_t fixed_b = rep_bytes(L.d_type) + h_planes_bytes(L, n_tok, k, shared != nullptr);
    const int slab_a = fit_slab(lim_a, fixed_a, kSlabA, 16 * kWavesA), slab_b = fit_slab(lim_b, fixed_b, kSlabB, 16);
    const int rows_c = pick_rows_c(L, slab_a);
    if (rows_c == 0 || (kRowsB * L.d_row) % 16 != 0 || kRowsB * L.d_row > (uint64_t) slab_b || L.up_off % 16 != 0 ||
        L.down_off % 16 != 0) {
        set_error("tsx_moe_decode_layer: row sizes (%llu, %llu) do not tile into 16-byte LDS slabs of %d and %d bytes",
                  (unsigned long long) L.gu_row, (unsigned long long) L.d_row, slab_a, slab_b);
        return TSX_ERR_UNSUPPORTED;
    }
    TSX_REQUIRE(blobs && logits && x && y && ids && wts && scratch && (!shared || sgate),
                "tsx_moe_decode_layer: a null pointer (sgate is needed with a shared expert)");
    TSX_REQUIRE(aligned(blobs, 16) && stride % 16 == 0 && (!shared || aligned(shared, 16)) && aligned(scratch, 256) &&
                    aligned(x, 16) && aligned(y, 4) && aligned(logits, 4),
                "tsx_moe_decode_layer: blobs, stride, shared and x 16-byte aligned, scratch 256-byte aligned");
    TSX_REQUIRE(!norm_w || (h && aligned(h, 4) && (!hq || aligned(hq, 2)) && L.n_embd % 32 == 0),
                "tsx_moe_decode_layer_norm: h (4-byte aligned) with norm_w; hq 2-byte aligned");
    LayerArgs a{};
    a.L = L;
    a.blobs = (const uint8_t*) blobs;
    a.stride = stride;
    a.n_expert = n_expert;
    a.k = k;
    a.n_tok = n_tok;
    a.logits = logits;
    a.x = x;
    a.shared = (const uint8_t*) shared;
    a.sgate = sgate;
    a.sg_stride = sg_stride;
    a.rows_c = rows_c;
    a.chunks_a = kSliceA / rows_c;
    a.slab_a = slab_a;
    a.slab_b = slab_b;
    a.y = y;
    a.ids = ids;
    a.wts = wts;
    a.tab = (LayerTables*) scratch;
    const int P = n_tok * k + (shared ? n_tok : 0);  // h is packed for the positions this call uses
    a.hc = (int8_t*) ((uint8_t*) scratch + kTablesBytes);
    a.hd = (float*) (a.hc + (size_t) P * L.n_ff);
    a.hf = (float*) a.hc;
    a.h_fp32 = 0;
    a.rows_w = 0;
    const hipStream_t s = (hipStream_t) stream;
    // one token: the row pairs spread over every CU (launch B quantizes the fp32 h) when the rows tile the slab
    int rc = TSX_ERR_UNSUPPORTED;
    if (n_tok == 1 && L.gu_row % 16 == 0) {
        // slot by slot where 16 waves can take every slot's rows, at most kMaxRowsW1 per wave, and the grid divides
        // n_ff: waves are dealt to slots S-1, S-2, ... in turn, base of them each and one more for the last extra
        // slots, and a slot's rows split evenly over its waves
        const int S = k + (shared ? 1 : 0), nb = std::min(kBlocksA, (int) L.n_ff);
        const int ppb = (int) L.n_ff / nb, rs = 2 * ppb, per = S <= kWavesA ? kWavesA / S : 0;
        const int rows_w = per > 0 && L.n_ff % nb == 0 ? (rs + per - 1) / per : INT_MAX;
        if (rows_w <= kMaxRowsW1) {
            // the waves in this order: those of wave 0's SIMD first (waves 4 j share a SIMD), so that the latest picks
            // go to them and they wait, rather than dot, while wave 0 routes
            int order[kWavesA], n = 0;
            for (int w = 0; w < kWavesA; w += 4) order[n++] = w;
            for (int w = 0; w < kWavesA; ++w)
                if (w % 4) order[n++] = w;
            const int extra = kWavesA % S;
            int w = 0;
            for (int slot = S - 1; slot >= 0; --slot) {
                const int ws = per + (slot >= S - extra ? 1 : 0);
                for (int iw = 0; iw < ws; ++iw, ++w)
                    a.s1_wave[order[w]] = slot | (rs * iw / ws) << 8 | (rs * (iw + 1) / ws) << 16;
            }
            a.s1_ppb = ppb;
        }
        size_t lim1 = 0;
        with_type(L.gu_type, [&](auto T) {
            static const size_t limit = set_max_lds((const void*) layer_gu1s_kernel<decltype(T)::value>);
            lim1 = limit;
            return 0;
        });
        const size_t lds1 = rows_w <= kMaxRowsW1 ? (size_t) kWavesA * rows_w * L.gu_row + rep_bytes(L.gu_type) +
                                                       x_planes_bytes(L, 1)
                                                 : SIZE_MAX;
        if (rows_w <= kMaxRowsW1 && S * rs <= kRowsS1 && L.gu_row <= (uint64_t) 64 * kPiecesRow1 * 16 &&
            lds1 <= lim1) {
            a.h_fp32 = 1;
            a.rows_w = rows_w;
            rc = with_type(L.gu_type, [&](auto T) {
                layer_gu1s_kernel<decltype(T)::value><<<nb, kThreadsA, lds1, s>>>(a);
                return launch_status("tsx_moe_decode_layer/gate-up");
            });
        }
    }
    if (n_tok == 1 && L.gu_row % 16 == 0 && !a.h_fp32) {
        const int pairs = (k + (shared ? 1 : 0)) * (int) L.n_ff, nb = std::min(kBlocksA, pairs);
        const int rows = 2 * ((pairs + nb - 1) / nb), rows_w = (rows + kWavesA - 1) / kWavesA;
        size_t lim1 = 0;
        with_type(L.gu_type, [&](auto T) {
            static const size_t limit = set_max_lds((const void*) layer_gu1_kernel<decltype(T)::value>);
            lim1 = limit;
            return 0;
        });
        const size_t lds1 = (size_t) kWavesA * rows_w * L.gu_row + rep_bytes(L.gu_type) + x_planes_bytes(L, 1);
        if (rows_w <= kMaxRowsW1 && L.gu_row <= (uint64_t) 64 * kPiecesRow1 * 16 && lds1 <= lim1) {
            a.h_fp32 = 1;
            a.rows_w = rows_w;
            rc = with_type(L.gu_type, [&](auto T) {
                layer_gu1_kernel<decltype(T)::value><<<nb, kThreadsA, lds1, s>>>(a);
                return launch_status("tsx_moe_decode_layer/gate-up");
            });
        }
    }
    if (n_tok >= 2 && n_tok <= kTokT && L.n_ff <= 2 * kBlocksA && L.gu_row % 16 == 0 &&
        L.gu_row <= (uint64_t) 64 * 16 * 2) {
        // a few tokens group by group: the block's rows of every group (at most one per routed entry, and the shared
        // expert) dealt over the 16 waves, at most items_t<cpr>() each
        const int nb = std::min(kBlocksA, (int) L.n_ff), ppb = (int) L.n_ff / nb, rs = 2 * ppb;
        const int most = (n_tok * k + (shared ? 1 : 0)) * rs;
        const int cpr = (int) ((L.gu_row / 16 + 63) / 64);
        size_t limt = 0;
        with_type(L.gu_type, [&](auto T) {
            static const size_t l1 = set_max_lds((const void*) layer_gut_kernel<decltype(T)::value, 1>);
            static const size_t l2 = set_max_lds((const void*) layer_gut_kernel<decltype(T)::value, 2>);
            limt = std::min(l1, l2);
            return 0;
        });
        const size_t ldst = (size_t) kWavesA * kRowsGB * L.gu_row + rep_bytes(L.gu_type) + x_planes_bytes(L, n_tok);
        if (L.n_ff % nb == 0 && (rs == 2 || rs == 4) && most <= kWavesA * (cpr == 1 ? items_t<1>() : items_t<2>()) &&
            ldst <= limt) {
            a.s1_ppb = ppb;
            a.h_fp32 = 1;
            a.rows_w = kRowsGB;
            rc = with_type(L.gu_type, [&](auto T) {
                if (cpr == 1) layer_gut_kernel<decltype(T)::value, 1><<<nb, kThreadsA, ldst, s>>>(a);
                else layer_gut_kernel<decltype(T)::value, 2><<<nb, kThreadsA, ldst, s>>>(a);
                return launch_status("tsx_moe_decode_layer/gate-up");
            });
        }
    }
    if (!a.h_fp32)
        rc = with_type(L.gu_type, [&](auto T) {
            auto kern = layer_gu_kernel<decltype(T)::value>;
            const size_t lds = (size_t) slab_a + fixed_a;
            // as many blocks as the routing could give slices, at most one per CU
            const int most = (std::min(n_tok * k, n_expert) + (shared ? 1 : 0)) * (int) (L.n_ff / kSliceA);
            kern<<<std::min(kBlocksA, most), kThreadsA, lds, s>>>(a);
            return launch_status("tsx_moe_decode_layer/gate-up");
        });
    if (rc != TSX_OK) return rc;
    // one round of row loads when the largest chunk (the slab's groups, or every group the routing can make) fits it
    const int gb = (int) (kRowsB * L.d_row), gmax = std::min(n_tok * k, n_expert) + (shared ? 1 : 0);
    const bool one_round = (int64_t) std::min(std::max(1, slab_b / gb), gmax) * (gb / 16) <= kThreadsB;
    rc = with_type(L.d_type, [&](auto T) {
        // fp32 h of several tokens: every piece requested in the first round (one more dependent round cost ~1 us)
        const bool hl = a.h_fp32 && n_tok > 1;
        auto kern = one_round ? (hl ? layer_down_kernel<decltype(T)::value, 1, kHLoadsT> : layer_down_kernel<decltype(T)::value, 1>)
                              : (hl ? layer_down_kernel<decltype(T)::value, kBLoads, kHLoadsT>
                                    : layer_down_kernel<decltype(T)::value, kBLoads>);
        const size_t lds = (size_t) slab_b + fixed_b;
        kern<<<(unsigned) (L.n_embd / kRowsB), kThreadsB, lds, s>>>(a);
        return launch_status("tsx_moe_decode_layer/down");
    });
    if (rc != TSX_OK || norm_w == nullptr) return rc;
    layer_norm_kernel<<<(unsigned) n_tok, kNormRowThreads, 0, s>>>(y, (int) L.n_embd, norm_w, eps, h,
                                                                  (tsx_block_q8_1*) hq);
    return launch_status("tsx_moe_decode_layer_norm/norm");
}

TSX_API int tsx_moe_decode_layer(const tsx_expert_layout* Lp, const void* blobs, uint64_t stride, int n_expert, int k,
                                 int n_tok, const float* logits, const float* x, const void* shared, const float* sgate,
                                 int sg_stride, float* y, int32_t* ids, float* wts, void* scratch, void* stream) {
    return decode_layer(Lp, blobs, stride, n_expert, k, n_tok, logits, x, shared, sgate, sg_stride, y, ids, wts, nullptr,
                        0.f, nullptr, nullptr, scratch, stream);
}

TSX_API int tsx_moe_decode_layer_norm(const tsx_expert_layout* Lp, const void* blobs, uint64_t stride, int n_expert,
                                      int k, int n_tok, const float* logits, const float* x, const void* shared,
                                      const float* sgate, int sg_stride, float* y, int32_t* ids, float* wts,
                                      const float* norm_w, float eps, float* h, void* hq, void* scratch,
                                      void* stream) {
    TSX_REQUIRE(norm_w != nullptr, "tsx_moe_decode_layer_norm: null norm_w (tsx_moe_decode_layer has no norm)");
    return decode_layer(Lp, blobs, stride, n_expert, k, n_tok, logits, x, shared, sgate, sg_stride, y, ids, wts, norm_w,
                        eps, h, hq, scratch, stream);
}

TSX_API size_t tsx_moe_decode_layer_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

TSX_API int tsx_moe_decode_layer_noalloc(const tsx_expert_layout* Lp, const void* blobs, uint64_t stride, int n_expert,
                                         int k, int n_tok, const float* logits, const float* x, const void* shared,
                                         const float* sgate, int sg_stride, float* y, int32_t* ids, float* wts,
                                         void* stream) {
    TSX_REQUIRE(Lp != nullptr, "tsx_moe_decode_layer_noalloc: null layout");
    const size_t need = tsx_moe_decode_layer_scratch_bytes(n_tok, k, Lp->n_ff);
    if (need > kNoAllocScratchBytes) {
        set_error("tsx_moe_decode_layer_noalloc: %d tokens x top-%d at n_ff %lld need %zu scratch bytes, more than the "
                  "%zu this entry point holds per GPU",
                  n_tok, k, (long long) Lp->n_ff, need, kNoAllocScratchBytes);
        return TSX_ERR_UNSUPPORTED;
    }
    int rc = TSX_OK;
    void* p = noalloc_scratch_ptr(&rc);
    if (!p) return rc;
    // every word launch B reads of the scratch is written by launch A of the same call first: nothing to clear
    return tsx_moe_decode_layer(Lp, blobs, stride, n_expert, k, n_tok, logits, x, shared, sgate, sg_stride, y, ids, wts,
                                p, stream);
}

}  // extern "C"
