/* tsx_pool.h - the host side of the hybrid CPU/GPU expert split: experts without a slot in HBM are computed by a
 * pool of CPU worker threads while the GPU runs the resident ones, and their output rows are merged into the
 * GPU's before the combine.
 *
 * The CPU rows use the same activation contract as the GPU kernels (Q8_1: one fp16 scale per 32 values, int8
 * codes; h re-quantized to Q8_1 after SwiGLU), so a routed entry gives the same integer sub-block sums on either
 * side.  The reference's CPU path quantizes to ggml's vec_dot_type instead (Q8_K for IQ3/Q4_K, Q8_0 for Q8_0;
 * src/kernels/cpu/native_expert.cpp:50-126); the oracle's mode 1 reports that gap.
 *
 * Functions return TSX_OK, TSX_ERR_UNSUPPORTED, TSX_ERR_ARG, or TSX_ERR_STALLED (the pool saw no progress for the
 * stall limit; it then refuses further work).  tsx_moe_last_error() has the message.  Only
 * tsx_moe_hybrid_decode_layer touches the GPU.
 */
#ifndef TSX_POOL_H
#define TSX_POOL_H

#include "tsx_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { TSX_ERR_STALLED = -5 };

#define TSX_CPU_MAXT 8           /* tokens per job (reference MAXT, include/strata/kernels/cpu/pool.hpp:32) */
#define TSX_POOL_MAX_SPLIT 96    /* experts per batch (reference kMaxSplitMulti, pool.hpp:150) */

/* One layer's expert geometry on the CPU.  Replaces strata::kernels::cpu::NativeFmt
 * (include/strata/kernels/cpu/native_expert.hpp:23-37); gu_act = d_act = 9 (Q8_1). */
typedef struct tsx_cpu_fmt {
    int32_t gu_type, d_type;
    int32_t gu_act, d_act;
    int64_t n_embd, n_ff;
    uint64_t gu_row, d_row;
    uint64_t up_off, down_off;
    uint64_t bytes;
    uint64_t act_bytes, h_bytes; /* Q8_1 of n_embd values, of n_ff values */
} tsx_cpu_fmt;

/* One expert applied to up to TSX_CPU_MAXT tokens: act[t] = token t's activation (act_bytes), out[t] = its
 * n_embd output floats.  Replaces strata::kernels::cpu::ExpertJobMulti (include/strata/kernels/cpu/pool.hpp:35-41). */
typedef struct tsx_cpu_job {
    const uint8_t* blob;
    int32_t nt;
    int32_t pad;
    float* out[TSX_CPU_MAXT];
    const void* act[TSX_CPU_MAXT];
} tsx_cpu_job;

/* ------------------------------------------------------------------------------------------------ CPU rows */
/* Fills f for a layer (gate/up and down types of the expert path, n_embd and n_ff multiples of 256).
 * Replaces strata::kernels::cpu::native_fmt (native_expert.hpp:50). */
TSX_API int tsx_cpu_fmt_init(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, tsx_cpu_fmt* f);
/* x (n_embd floats) -> Q8_1 (act_bytes).  Replaces native_quant_act (native_expert.hpp:53). */
TSX_API int tsx_cpu_quant_act(const tsx_cpu_fmt* f, const float* x, void* dst);
/* h (n_ff floats) -> Q8_1 (h_bytes).  Replaces native_quant_h (native_expert.hpp:55). */
TSX_API int tsx_cpu_quant_h(const tsx_cpu_fmt* f, const float* h, void* dst);
/* ff[t][r] = silu(gate_r . act[t]) * (up_r . act[t]) for rows r in [r0, r1), nt tokens (1..TSX_CPU_MAXT); the
 * product rounded on its own.  Replaces native_gu_rows (native_expert.hpp:61-62). */
TSX_API int tsx_cpu_gu_rows(const tsx_cpu_fmt* f, const uint8_t* blob, const void* const* act, int nt,
                            float* const* ff, int r0, int r1);
/* out[t][r] = down_r . hq[t] for rows r in [r0, r1).  Replaces native_down_rows (native_expert.hpp:64-65). */
TSX_API int tsx_cpu_down_rows(const tsx_cpu_fmt* f, const uint8_t* blob, const void* const* hq, int nt,
                              float* const* out, int r0, int r1);

/* ------------------------------------------------------------------------------------------------ the pool */
typedef struct tsx_pool tsx_pool;
/* n_workers <= 0: one per physical core the process may run on, less one for the host thread.  pin: each worker
 * on its own physical core (Linux sysfs topology; ignored where it is unavailable).  host_works: the calling
 * thread drains jobs too.  tasks: row tasks per phase (0 = three per participating thread).
 * Replaces the strata::kernels::cpu::ExpertPool constructor (include/strata/kernels/cpu/pool.hpp:112-114). */
TSX_API int tsx_pool_create(int n_workers, int pin, int host_works, int tasks, tsx_pool** out);
TSX_API void tsx_pool_destroy(tsx_pool* p);
TSX_API int tsx_pool_workers(const tsx_pool* p);
TSX_API int tsx_pool_host_works(const tsx_pool* p);
/* Evaluates n jobs (any number; batches of TSX_POOL_MAX_SPLIT): gate/up rows, SwiGLU + Q8_1 of h, down rows, as
 * dependent row tasks per expert when several experts and threads take part, else as three phases.  Returns when
 * every job's outputs are written.  One caller at a time per pool.  After TSX_ERR_STALLED, workers may still be
 * running the batch: the jobs and their buffers must stay valid until tsx_pool_destroy has returned.
 * Replaces ExpertPool::run_split_multi_native (pool.hpp:139; src/kernels/cpu/pool.cpp:773-817). */
TSX_API int tsx_pool_run(tsx_pool* p, const tsx_cpu_fmt* f, const tsx_cpu_job* jobs, int n);
/* Accumulated milliseconds: [0] the host waiting for workers to leave the slot it is about to reuse, [1] the host
 * from publishing a batch until its last chunk finished, [2] gate/up row chunks, [3] quantizing h, [4] down row
 * chunks (2-4 summed over every thread), [5] threads waiting for an h another thread is making; and *bytes = expert
 * blob bytes evaluated.  Replaces ExpertPool::phase_ms and the ms_multi_* counters (pool.hpp:140-143,160-167). */
TSX_API int tsx_pool_stats(const tsx_pool* p, double* ms6, int64_t* bytes);
/* The pool's state as one line of text into buf (n bytes, truncated): the current batch's sequence number, its
 * experts, finished / total and unclaimed chunks, the workers attached to each of the two slots, idle workers and
 * sleepers, FAILED after a stall, and each worker's state (idle, sleeping, waiting-h, or the expert it works on).
 * Safe to call from any thread at any time.  Replaces ExpertPool::diag (pool.hpp:118-119,
 * src/kernels/cpu/pool.cpp:457-476). */
TSX_API int tsx_pool_diag(const tsx_pool* p, char* buf, size_t n);
/* How long a parked worker spins before it sleeps, in microseconds (default 20000): a test knob, as the reference's
 * STRATA_POOL_SPIN_US (pool.hpp:180-181).  Only between runs. */
TSX_API int tsx_pool_set_spin_us(tsx_pool* p, int64_t us);
/* The stall limit in milliseconds (default 60000; reference kStall, pool.hpp:187). */
TSX_API int tsx_pool_set_stall_ms(tsx_pool* p, int64_t ms);

/* ------------------------------------------------------------------------------------------------ hybrid */
/* The CPU half of a hybrid decode layer (reference moe_hybrid_cpu, src/qwen35/q36_engine.cu:3090-3209, compact
 * form): entries e = t*k + j of ids[n_tok][k] whose expert has slot_of[x] < 0 are the misses.  Each missed
 * token's x row (n_embd floats) is quantized once; jobs take up to TSX_CPU_MAXT tokens of one expert; miss i
 * (in entry order) writes row i of cpu_out (n_embd floats).  miss[e] = i for a miss, -1 for a resident entry;
 * *n_miss = the count.  host_blobs: every expert's blob, `stride` bytes apart, in host memory.  After
 * TSX_ERR_STALLED, workers may still be running the stalled batch, reading host_blobs and the quantized x and
 * writing cpu_out: host_blobs and cpu_out must stay valid until tsx_pool_destroy has returned. */
TSX_API int tsx_moe_hybrid_cpu(tsx_pool* p, const tsx_cpu_fmt* f, const uint8_t* host_blobs, uint64_t stride,
                               const int32_t* slot_of, int n_expert, int k, int n_tok, const int32_t* ids,
                               const float* x, float* cpu_out, int32_t* miss, int32_t* n_miss);

/* A whole hybrid decode layer in one call (reference moe_hybrid_gpu + moe_hybrid_cpu + the combine,
 * src/qwen35/q36_engine.cu:3052-3209).  Enqueued on `stream`: routing, the ids and x to the pinned host buffers,
 * the resident entries grouped into their slots and run, the shared expert; then the host waits for the ids and x
 * alone and runs the misses on the pool while the GPU works, uploads the CPU rows and the miss map, merges them
 * into `parts` and enqueues the combine (y += ...).  Returns after the last enqueue; n_miss is written.  The pinned
 * buffers are reused by the next call on the same stream (its copies run after this call's uploads).  After
 * TSX_ERR_STALLED, workers may still be running the stalled batch: host_blobs and h_rows must stay valid until
 * tsx_pool_destroy has returned. */
typedef struct tsx_hybrid_layer {
    tsx_expert_layout L;
    int32_t n_expert, k, n_tok, sg_stride;
    const uint8_t* host_blobs; /* host: every expert, stride bytes apart */
    uint64_t stride;
    const int32_t* slot_of;    /* host [n_expert]: slot or -1 */
    const int32_t* d_slot_of;  /* device copy of slot_of */
    const void* slots;         /* device: the resident blobs, stride bytes apart */
    const void* shared;        /* device: the shared expert's blob, or null */
    const float* sgate;        /* device [n_tok * sg_stride] (with shared) */
    const float* x;            /* device [n_tok][n_embd] */
    const float* logits;       /* device [n_tok][n_expert] */
    float* y;                  /* device [n_tok][n_embd], += */
    int32_t* ids;              /* device [n_tok * k] */
    float* wts;                /* device [n_tok * k] */
    uint64_t* grp_ptr;         /* device: min(n_ent, n_expert) groups */
    int32_t* grp_start;
    int32_t* n_groups;
    int32_t* ent_dst;
    int32_t* ent_tok;
    void* xq;                  /* device [n_tok][n_embd / 32 * 36] */
    void* scratch;             /* device, tsx_moe_expert_scratch_bytes(n_ent, n_ff) */
    float* parts;              /* device [n_ent][n_embd] */
    float* sh_gate;            /* device [n_tok][n_ff] (with shared) */
    float* sh_up;
    void* sh_hq;               /* device [n_tok][n_ff / 32 * 36] */
    float* sh_out;             /* device [n_tok][n_embd] */
    int32_t* h_ids;            /* pinned host [n_tok * k] */
    float* h_x;                /* pinned host [n_tok][n_embd] */
    float* h_rows;             /* pinned host [n_ent][n_embd] */
    int32_t* h_miss;           /* pinned host [n_ent] */
    float* d_rows;             /* device [n_ent][n_embd] */
    int32_t* d_miss;           /* device [n_ent] */
    int32_t n_miss;            /* out */
    int32_t pad;
} tsx_hybrid_layer;
TSX_API int tsx_moe_hybrid_decode_layer(tsx_pool* p, const tsx_cpu_fmt* f, tsx_hybrid_layer* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TSX_POOL_H */
