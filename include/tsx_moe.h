/* tsx_moe.h - the C ABI of libtsx_moe.so, TinyStrata's MoE expert matmul (ggml mul_mat_id) for AMD MI355X (gfx950).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed as void*; nothing here allocates,
 * waits on the host or synchronizes a stream, so a caller can capture any sequence of calls in a HIP graph (the
 * expert-id gather/scatter and the per-expert row counts stay on the device).  Pointers are caller-owned device
 * memory, 4-byte aligned at least, and non-overlapping unless a function says otherwise.  Status codes:
 * TSX_OK = 0 (launched), TSX_ERR_UNSUPPORTED = -1 (a type or shape this library has no kernel for),
 * TSX_ERR_ARG = -2 (a null pointer, a negative size or a misaligned buffer), a positive value = the hipError_t of
 * the launch.  tsx_moe_last_error() returns the message of the last failure on the calling thread.
 *
 * The interface is the reference's operator API for this path with the reference's own thin-C-ABI pattern
 * (strata_kq_abi / strata_kq_init / strata_kq_run: include/strata/prefill/mmq_kq_abi.hpp:14-18,
 * src/prefill/mmq_kq_lib.cu:33-60); each declaration names the reference function it stands in for.
 * The C++ wrappers in tinystrata_amd/csrc/strata_kernels.hpp keep the reference's names, signatures and error
 * behaviour on top of these.
 */
#ifndef TSX_MOE_H
#define TSX_MOE_H

#include <stddef.h>
#include <stdint.h>

#include "tsx_formats.h"
#include "tsx_grids.h"

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TSX_API __attribute__((visibility("default")))
#else
#define TSX_API
#endif

#define TSX_MOE_ABI_VERSION 1

enum { TSX_OK = 0, TSX_ERR_UNSUPPORTED = -1, TSX_ERR_ARG = -2 };

/* ------------------------------------------------------------------------------------------------ library */
/* ABI version * 100000 + sizeof(tsx_mmq_product), checked by a loader before use.
 * Replaces strata_kq_abi (include/strata/prefill/mmq_kq_abi.hpp:14; src/prefill/mmq_kq_lib.cu:33). */
TSX_API int tsx_moe_abi(void);
/* Makes `device` current and starts the HIP runtime on it.  0 = ready, else the hipError_t.
 * Replaces strata_kq_init (include/strata/prefill/mmq_kq_abi.hpp:16; src/prefill/mmq_kq_lib.cu:38-43). */
TSX_API int tsx_moe_init(int device);
/* The message of the calling thread's last failed call ("" if none). */
TSX_API const char* tsx_moe_last_error(void);

/* ------------------------------------------------------------------------------------------------ formats */
/* Bytes of one row of n values of `type`; 0 for a type outside the path or n not whole blocks.
 * Replaces strata::kernels::iq_row_bytes (include/strata/kernels/iq_kernels.hpp:21). */
TSX_API size_t tsx_moe_row_bytes(int type, int64_t n);
/* The [gate | up | down] blob layout.  TSX_OK or TSX_ERR_UNSUPPORTED.
 * Replaces strata::kernels::native_expert_layout (include/strata/kernels/iq_kernels.hpp:54;
 * src/kernels/cuda/iq_kernels.cu:2120-2138). */
TSX_API int tsx_moe_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, tsx_expert_layout* out);
/* 1 when tsx_moe_expert_grouped has kernels for this type pair and shape, else 0.
 * Replaces strata::kernels::native_expert_supported (include/strata/kernels/iq_kernels.hpp:57;
 * src/kernels/cuda/iq_kernels.cu:2114-2118). */
TSX_API int tsx_moe_expert_supported(int gu_type, int d_type, int64_t n_embd, int64_t n_ff);
/* Scratch bytes tsx_moe_expert_grouped needs for cap_entries entries (the reference's formula).
 * Replaces strata::kernels::native_expert_scratch_bytes (include/strata/kernels/iq_kernels.hpp:60;
 * src/kernels/cuda/iq_kernels.cu:2140-2143). */
TSX_API size_t tsx_moe_expert_scratch_bytes(int64_t cap_entries, int64_t n_ff);
/* Byte offset of the Q8_1 image of the SwiGLU output inside that scratch ([cap_entries][n_ff/32] blocks); the
 * tests read the down projection's integer activations from there.  No reference counterpart. */
TSX_API size_t tsx_moe_expert_scratch_hq_offset(int64_t cap_entries, int64_t n_ff);

/* ------------------------------------------------------------------------------------------------ activations */
/* y = Q8_1 blocks of n_rows rows of n_cols floats (n_cols a multiple of 32): per 32 values d = amax/127 (fp16),
 * s = sum of the floats (fp16), q = round(x/d) clamped to +-127, both fp16 fields held finite.
 * Replaces strata::kernels::quantize_q8_1_rows (include/strata/kernels/iq_kernels.hpp:24;
 * src/kernels/cuda/iq_kernels.cu:1467-1487) and native_quantize_q8_1 (include/strata/kernels/native_mmvq.hpp:26-42). */
TSX_API int tsx_moe_quantize_q8_1(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream);
/* y = Q8_1 of silu(gate) * up over n values (n a multiple of 32), the product rounded before the block sum.
 * Replaces strata::kernels::native_swiglu_quantize_q8_1 (include/strata/kernels/native_mmvq.hpp;
 * src/kernels/cuda/native_mmvq.cu:171-185). */
TSX_API int tsx_moe_swiglu_quantize_q8_1(const float* gate, const float* up, int64_t n, void* y, void* stream);

/* ------------------------------------------------------------------------------------------------ decode */
/* Grouped experts: group g's blob at device address grp_ptr[g]; its entries [grp_start[g], grp_start[g+1]) read
 * token ent_tok[e]'s Q8_1 activation (n_embd/32 blocks per token in x_q8_1) and write row ent_dst[e] of `out`
 * (n_embd floats): out = down . Q8_1(silu(gate . x) * (up . x)).  *n_groups and grp_start are read on the device.
 * grid_groups (1..cap_groups, 0 = cap_groups) block rows stride over the groups; the results do not depend on it.
 * Replaces strata::kernels::native_expert_grouped (include/strata/kernels/iq_kernels.hpp:75-78;
 * src/kernels/cuda/iq_kernels.cu:2835-2982). */
TSX_API int tsx_moe_expert_grouped(const tsx_expert_layout* L, const uint64_t* grp_ptr, const int32_t* grp_start,
                                   const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok,
                                   int64_t cap_groups, int64_t cap_entries, const void* x_q8_1, void* scratch,
                                   float* out, void* stream, int64_t grid_groups);
/* y[c][r] = W[r] . x[c] for ncols (1..8) columns of Q8_1 activations (n_in/32 blocks per column).  Types: the expert
 * formats (IQ3_XXS, IQ3_S, Q4_K, Q8_0) and Q4_0, Q6_K.
 * Replaces strata::kernels::iq_mmvq (include/strata/kernels/iq_kernels.hpp:27) and native_mmvq
 * (include/strata/kernels/native_mmvq.hpp:128-131): the shared expert's projections. */
TSX_API int tsx_moe_mmvq(int type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                         void* stream);

/* Several matrices of one format and shape in one launch, the matrices picked on the device: matrix j (j < count,
 * count <= 65535) is table[ids[j]] + offset bytes, times the Q8_1 column x + (j / x_every) * x_stride bytes, into
 * y + j * y_stride floats (n_out of them).  An id outside [0, n_table) gives zeros (the reference leaves it to the
 * caller).  Types as tsx_moe_mmvq.  Replaces lfm_native_mmvq_ids / MmvqIds and lfm_native_mmvq_ids_supported
 * (include/strata/lfm2/matvec.hpp:153-168; src/lfm2/matvec.cu:3134-3139): a decode step's routed experts with
 * nothing of the host. */
typedef struct {
    const void* const* table; /* device array of matrix base pointers */
    const int32_t* ids;       /* device [count] */
    int32_t n_table;
    uint64_t offset;
    const void* x;
    uint64_t x_stride;
    int32_t x_every;
    float* y;
    uint64_t y_stride;
} tsx_mmvq_ids;
TSX_API int tsx_moe_mmvq_ids_supported(int type);
TSX_API int tsx_moe_mmvq_ids(int type, const tsx_mmvq_ids* a, int count, int n_in, int n_out, void* stream);
/* Up to 8 matrices given by the host: matrix j times its own column x[j] into y[j], as tsx_moe_mmvq(type, w[j], x[j],
 * y[j], n_in, n_out, 1) would each.  Replaces lfm_native_mmvq_slots / MmvqSlots
 * (include/strata/lfm2/matvec.hpp:146-152). */
typedef struct {
    const void* w[8];
    const void* x[8];
    float* y[8];
} tsx_mmvq_slots;
TSX_API int tsx_moe_mmvq_slots(int type, const tsx_mmvq_slots* a, int count, int n_in, int n_out, void* stream);

/* The whole decode MoE layer for 1..8 tokens in two launches: routing (tsx_moe_router_topk's arithmetic), grouping,
 * Q8_1 of x, the grouped gate/up rows with SwiGLU + Q8_1, the down rows and the combine:
 *   y[t] += sum_j wts[t][j] * expert(ids[t][j], x[t])  (first product, then FMA, pick order)
 *         + sigmoid(sgate[t * sg_stride]) * expert(shared, x[t])          (when shared is not null)
 * where expert(b, x) = down . Q8_1(silu(gate . Q8_1(x)) * (up . Q8_1(x))) of the blob at b; expert e's blob is at
 * blobs + e * stride.  ids / wts [n_tok][k] receive the routing.  y may alias x.  Limits: n_embd <= 4096,
 * n_ff <= 1024, n_tok * k <= 64, n_expert a multiple of 64 up to 512; blobs, stride and shared 16-byte aligned.
 * scratch: tsx_moe_decode_layer_scratch_bytes(n_tok, k, n_ff) bytes, 256-byte aligned (the tables, and h as Q8_1
 * planes or, where launch A leaves it in fp32 - one token, or up to four at n_ff <= 512 - as floats).
 * Replaces the MoE block's call sequence at src/qwen35/q36_engine.cu:2821-2925: k_route_group
 * (src/qwen35/q36_kernels.cuh:383-474), native_expert_grouped (src/kernels/cuda/iq_kernels.cu:2835-2982), the shared
 * expert's mmvq / SwiGLU / mmvq (q36_engine.cu:2906-2913) and k_moe_out_small without the norm
 * (q36_kernels.cuh:248-290). */
TSX_API size_t tsx_moe_decode_layer_scratch_bytes(int n_tok, int k, int64_t n_ff);
/* tsx_moe_decode_layer with the MoE block's end as k_moe_out_small has it (src/qwen35/q36_kernels.cuh:248-290):
 * after y[t] is formed, h[t][i] = (y[t][i] * r) * norm_w[i] with r = 1 / sqrt(mean over i of y[t][i]^2 + eps) (the
 * next layer's attention norm; two roundings, no fma) into h [n_tok][n_embd] (fp32), and, when hq is not null, its
 * Q8_1 image [n_tok][n_embd / 32] (the next layer's input: the bytes tsx_moe_quantize_q8_1 would write from h).
 * The norm is a third launch of one workgroup per token.  Same limits and scratch as tsx_moe_decode_layer; n_embd a
 * multiple of 32. */
TSX_API int tsx_moe_decode_layer_norm(const tsx_expert_layout* L, const void* blobs, uint64_t stride, int n_expert,
                                      int k, int n_tok, const float* logits, const float* x, const void* shared,
                                      const float* sgate, int sg_stride, float* y, int32_t* ids, float* wts,
                                      const float* norm_w, float eps, float* h, void* hq, void* scratch, void* stream);
TSX_API int tsx_moe_decode_layer(const tsx_expert_layout* L, const void* blobs, uint64_t stride, int n_expert, int k,
                                 int n_tok, const float* logits, const float* x, const void* shared, const float* sgate,
                                 int sg_stride, float* y, int32_t* ids, float* wts, void* scratch, void* stream);

/* tsx_moe_decode_layer without a scratch argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that allocate nothing after start-up, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  The scratch is a fixed device array of tsx_moe_decode_layer_noalloc_max_bytes() (128 KiB) per
 * GPU, held until the process ends; its address is looked up once per device (with that device current), by
 * tsx_moe_init when it can (a failure there is ignored) and otherwise on the first call, which then returns the
 * runtime's hipError_t if the lookup fails.  A call needing more scratch than that
 * (tsx_moe_decode_layer_scratch_bytes) returns TSX_ERR_UNSUPPORTED.
 * Nothing is allocated or freed.  Calls share their GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race; calls in one stream's order do not. */
TSX_API size_t tsx_moe_decode_layer_noalloc_max_bytes(void);
TSX_API int tsx_moe_decode_layer_noalloc(const tsx_expert_layout* L, const void* blobs, uint64_t stride, int n_expert,
                                         int k, int n_tok, const float* logits, const float* x, const void* shared,
                                         const float* sgate, int sg_stride, float* y, int32_t* ids, float* wts,
                                         void* stream);

/* ------------------------------------------------------------------------------------------------ routing */
/* logits [n_tok][n_expert] -> ids [n_tok][k] and weights [n_tok][k]: softmax, k rounds of argmax (ties to the
 * lower id; NaN probabilities never win), weights renormalized by max(sum of the picks, 6.1035e-5).
 * n_expert a multiple of 64 up to 512, k 1..16.
 * Replaces strata::kernels::native_router_topk (include/strata/kernels/native_router.hpp:5-6;
 * src/kernels/cuda/native_router.cu:42-111), which took only (256, 8). */
TSX_API int tsx_moe_router_topk(const float* logits, int32_t* ids, float* weights, int n_expert, int k, int n_tok,
                                void* stream);
/* The routed entries (entry e = t*k + j) grouped per used expert, ascending id, entries in entry order:
 * grp_ptr[g] = blobs + x*stride, grp_start[0..G], *n_groups = G, ent_dst[p] = e, ent_tok[p] = e / k.
 * grp_ptr/grp_start hold up to min(n_ent, n_expert) (+1) groups.  One workgroup; n_expert <= 512.
 * Replaces the reference's k_group (src/qwen35/q36_engine.cu:394-422) / k_group_small
 * (src/qwen35/q36_kernels.cuh:343-381). */
TSX_API int tsx_moe_group(const int32_t* ids, int n_ent, int k, int n_expert, const void* blobs, uint64_t stride,
                          uint64_t* grp_ptr, int32_t* grp_start, int32_t* n_groups, int32_t* ent_dst,
                          int32_t* ent_tok, void* stream);
/* tsx_moe_group for a hybrid layer: only the entries whose expert has an HBM slot (slot_of[x] >= 0; slot_of is
 * n_expert device ints) are grouped, and group g's blob is slot slot_of[x] of `slots` (stride bytes apart).
 * Replaces k_group_hy (src/qwen35/q36_engine.cu:423-452). */
TSX_API int tsx_moe_group_resident(const int32_t* ids, int n_ent, int k, int n_expert, const int32_t* slot_of,
                                   const void* slots, uint64_t stride, uint64_t* grp_ptr, int32_t* grp_start,
                                   int32_t* n_groups, int32_t* ent_dst, int32_t* ent_tok, void* stream);
/* Row e of parts (n floats) = row miss[e] of rows where miss[e] >= 0, else unchanged: the CPU's rows of a hybrid
 * layer merged into the GPU's before the combine.  Replaces k_merge_cpu (src/qwen35/q36_engine.cu:455-460, called at :3205) in the compact form. */
TSX_API int tsx_moe_merge_rows(float* parts, const float* rows, const int32_t* miss, int n_ent, int64_t n,
                               void* stream);
/* The prompt's entries sorted by expert: bounds[x]..bounds[x+1] are expert x's sorted rows (n_expert + 1 ints);
 * sorted row r holds entry ent_dst[r] of token ent_tok[r]; rinv[e] = entry e's sorted row; *max_rows = the most
 * rows of one expert.  Rows inside an expert are in entry order.  All on the device (no host round trip).
 * Replaces k_route_count / k_route_scan / k_route_scatter (src/qwen35/q36_engine.cu:483-510) and the
 * max_rows read back at src/qwen35/q36_engine.cu:2864-2869. */
TSX_API int tsx_moe_route_sort(const int32_t* ids, int n_ent, int k, int n_expert, int32_t* bounds, int32_t* ent_dst,
                               int32_t* ent_tok, int32_t* rinv, int32_t* max_rows, void* stream);
/* x[t] += w[t][0]*parts[p(t,0)] then fmaf(w[t][j], parts[p(t,j)], .) in pick order, + sigmoid(sgate[t*sg_stride])
 * * shared[t] (shared/sgate may be null); p(t,j) = prow ? prow[t*k+j] : t*k+j.  n values per row.
 * Replaces k_moe_out / k_moe_out_small without the norm (src/qwen35/q36_engine.cu:304-332;
 * src/qwen35/q36_kernels.cuh:248-290). */
TSX_API int tsx_moe_combine(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                            const float* shared, const float* sgate, int sg_stride, int n, int n_tok, void* stream);
/* tsx_moe_combine (the same x bits), then h[t] = (x[t] * r) * norm_w with r = 1 / sqrt(mean(x[t]^2) + eps) into
 * h [n_tok][n] and, when hq is not null, its Q8_1 image [n_tok][n / 32]: the whole of k_moe_out / k_moe_out_small
 * with the norm (src/qwen35/q36_engine.cu:304-332; src/qwen35/q36_kernels.cuh:248-290).  k 1..16, n a multiple of 32
 * up to 16384.  One workgroup per token. */
TSX_API int tsx_moe_combine_norm(float* x, const float* parts, const int32_t* prow, const float* wts, int k,
                                 const float* shared, const float* sgate, int sg_stride, int n, int n_tok,
                                 const float* norm_w, float eps, float* h, void* hq, void* stream);

/* ------------------------------------------------------------------------------------------------ prefill */
/* Bytes of `rows` activation rows of `cols` values quantized for tsx_moe_mmq_run.
 * Replaces strata::prefill::mmq::q8_bytes (include/strata/prefill/moe_mmq.hpp:36). */
TSX_API size_t tsx_moe_mmq_q8_bytes(int64_t rows, int64_t cols);
/* Row i of xq = Q8_1 of row ids[i] of x (row i when ids is null), `ld` floats per row of x.  The values are the
 * Q8_1 contract above; the layout is this library's tile layout (tsx_moe_mmq_q8_bytes), for weights of `type`.
 * Replaces strata::prefill::mmq::quantize (include/strata/prefill/moe_mmq.hpp:39-41; src/prefill/moe_mmq.cu:309-325). */
TSX_API int tsx_moe_mmq_quantize(const float* x, const int32_t* ids, void* xq, int type, int64_t cols, int64_t ld,
                                 int64_t rows, void* stream);
/* tsx_moe_mmq_quantize of the `rows` token rows of x (ids = NULL) and tsx_moe_router_topk of their logits
 * ([rows][n_expert]) in one launch: the two are independent, so their blocks share it.  The same bytes as the two
 * calls; x 16-byte aligned with ld a multiple of 4, n_expert and k as tsx_moe_router_topk.  Replaces the pair
 * native_router_topk (include/strata/kernels/native_router.hpp:5-6) + mmq::quantize of the tokens
 * (include/strata/prefill/moe_mmq.hpp:39-41) at the prompt call site (src/qwen35/q36_engine.cu:2855-2872). */
TSX_API int tsx_moe_mmq_quantize_route(const float* x, void* xq, int type, int64_t cols, int64_t ld, int64_t rows,
                                       const float* logits, int32_t* ids, float* weights, int n_expert, int k,
                                       void* stream);
/* One grouped product over n experts whose weights lie expert_bytes apart from w: for expert x, activation rows
 * [bounds[x], bounds[x+1]) of xq times its [w_rows][w_cols] matrix into dst rows ids[row] (row when ids is null),
 * ld_dst floats apart.  bounds on the device (n + 1 ints); total_rows = rows of xq.  max_rows may be 0: the tiles
 * are found on the device.
 * Replaces strata::prefill::mmq::Product / Context::run (include/strata/prefill/moe_mmq.hpp:58-85;
 * src/prefill/moe_mmq.cu:334-384). */
typedef struct {
    const void* w;
    int32_t type;
    int32_t n;
    int64_t w_rows, w_cols;
    uint64_t expert_bytes;
    const void* xq;
    const int32_t* bounds;
    const int32_t* ids;
    int64_t total_rows, max_rows;
    float* dst;
    int64_t ld_dst;
} tsx_mmq_product;
TSX_API int tsx_moe_mmq_run(const tsx_mmq_product* p, void* stream);
/* h[r][k] = silu(g) * u of GU rows [2*n_ff wide]: interleaved (gate 2k, up 2k+1) or split (gate k, up n_ff + k).
 * Replaces strata::prefill::mmq::swiglu (include/strata/prefill/moe_mmq.hpp:112; src/prefill/moe_mmq.cu:123-131). */
TSX_API int tsx_moe_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream);
/* The gate/up product of the prompt path with SwiGLU and the Q8_1 quantization of h fused in: for each expert's
 * sorted rows [bounds[e], bounds[e+1]) (rows of xq taken through xids, or the sorted rows themselves when xids is
 * NULL), h = silu(x . gate) * (x . up) quantized into hq (tsx_moe_mmq_q8_bytes(n_rows, n_ff) bytes, row r = sorted
 * row r), the codes tsx_moe_mmq_quantize writes for the same h.  Gate rows are rows [0, n_ff) of each expert's
 * matrix, up rows [n_ff, 2 n_ff).  No single reference function: it stands in for the sequence mmq::quantize of the
 * gathered rows, Context::run of the gate/up product, mmq::swiglu and mmq::quantize of h
 * (src/qwen35/q36_engine.cu:2855-2872; src/prefill/moe_mmq.cu:123-131, 309-384), the x rows quantized once per
 * token instead of once per routed row. */
TSX_API int tsx_moe_mmq_gate_up_swiglu(const void* w, int type, int64_t n_ff, int64_t n_embd, uint64_t expert_bytes,
                                       int n_exp, const void* xq, int64_t x_rows, const int32_t* xids,
                                       const int32_t* bounds, int64_t n_rows, void* hq, void* stream);

/* ------------------------------------------------------------------------------------------------ checks and data */
/* The integer contract: sums[(r*ncols + c)*nsub + u] = sum over sub-block u (32 values) of w_int * a_int, and
 * qsums (may be null) the same for sum a_int, for rows [0, n_rows) of W against ncols Q8_1 activations.
 * No reference counterpart: the tests compare these to the oracle bit for bit. */
TSX_API int tsx_moe_subblock_sums(int type, const void* w, int64_t n_in, int64_t n_rows, const void* x_q8_1,
                                  int64_t ncols, int32_t* sums, int32_t* qsums, void* stream);
/* Host: rows of fp32 into GGUF blocks of `type` (Q8_0, Q4_K, IQ3_XXS, IQ3_S).  Stands in for ggml's quantizers
 * (ggml_quantize_chunk, used by tests/native-expert-pool.cpp:52-61) to make synthetic expert weights. */
TSX_API int tsx_moe_quantize_weights(int type, const float* x, int64_t n_rows, int64_t n_cols, void* out);

#ifdef __cplusplus
}
#endif
#endif
