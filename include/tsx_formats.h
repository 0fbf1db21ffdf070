/* tsx_formats.h - the GGUF block formats of the MoE expert path, as plain C.
 *
 * Block layouts follow ggml's ggml-common.h so that expert blobs taken from a GGUF file are read unchanged:
 *   Q8_0   (type 8)  {fp16 d; int8 qs[32]}                                   34 B / 32 values
 *   Q8_1   (type 9)  {fp16 d; fp16 s; int8 qs[32]}                           36 B / 32 values
 *   Q4_K   (type 12) {fp16 d, dmin; u8 scales[12]; u8 qs[128]}               144 B / 256 values
 *   Q8_K   (type 15) {f32 d; int8 qs[256]; int16 bsums[16]}                  292 B / 256 values
 *   IQ3_XXS(type 18) {fp16 d; u8 qs[64] grid idx; u8 ss[32] 8 x u32 signs+scale} 98 B / 256 values
 *   IQ3_S  (type 21) {fp16 d; u8 qs[64]; u8 qh[8]; u8 signs[32]; u8 scales[4]} 110 B / 256 values
 *   Q4_0   (type 2)  {fp16 d; u8 qs[16]: value i low nibble, i + 16 high}    18 B / 32 values
 *   Q6_K   (type 14) {u8 ql[128]; u8 qh[64]; int8 scales[16]; fp16 d}        210 B / 256 values
 * Reference: third_party/ggml/ggml-common.h:251-256 (q8_0), 258-269 (q8_1), 327-338 (q4_K), 371-376 (q8_K),
 * 407-411 (iq3_xxs), 415-422 (iq3_s), and the block_q4_0 / block_q6_K definitions there; type ids
 * include/strata/artifact/gguf_reader.hpp:60-100.  Q4_0 and Q6_K are taken by the single-matrix and id-indexed
 * products only (the LFM2 / Gemma matrices, include/strata/lfm2/matvec.hpp:153-168), not by the expert blob.
 *
 * The expert blob is [gate rows | up rows | down rows] of these blocks, as in the reference's NativeExpertLayout
 * (include/strata/kernels/iq_kernels.hpp:44-53, src/kernels/cuda/iq_kernels.cu:2120-2138).
 */
#ifndef TSX_FORMATS_H
#define TSX_FORMATS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TSX_Q4_0 = 2,
    TSX_Q8_0 = 8,
    TSX_Q8_1 = 9,
    TSX_Q4_K = 12,
    TSX_Q6_K = 14,
    TSX_Q8_K = 15,
    TSX_IQ3_XXS = 18,
    TSX_IQ3_S = 21,
};

#define TSX_QK_K 256
#define TSX_QK8 32

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } tsx_block_q8_0;
typedef struct { uint16_t d; uint16_t s; int8_t qs[32]; } tsx_block_q8_1;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } tsx_block_q4_K;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } tsx_block_q8_K;
typedef struct { uint16_t d; uint8_t qs[96]; } tsx_block_iq3_xxs;
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t signs[32]; uint8_t scales[4]; } tsx_block_iq3_s;
typedef struct { uint16_t d; uint8_t qs[16]; } tsx_block_q4_0;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } tsx_block_q6_K;
#pragma pack(pop)

#ifdef __cplusplus
static_assert(sizeof(tsx_block_q8_0) == 34, "q8_0");
static_assert(sizeof(tsx_block_q8_1) == 36, "q8_1");
static_assert(sizeof(tsx_block_q4_K) == 144, "q4_K");
static_assert(sizeof(tsx_block_q8_K) == 292, "q8_K");
static_assert(sizeof(tsx_block_iq3_xxs) == 98, "iq3_xxs");
static_assert(sizeof(tsx_block_iq3_s) == 110, "iq3_s");
static_assert(sizeof(tsx_block_q4_0) == 18, "q4_0");
static_assert(sizeof(tsx_block_q6_K) == 210, "q6_K");
#else
_Static_assert(sizeof(tsx_block_q8_0) == 34, "q8_0");
_Static_assert(sizeof(tsx_block_q8_1) == 36, "q8_1");
_Static_assert(sizeof(tsx_block_q4_K) == 144, "q4_K");
_Static_assert(sizeof(tsx_block_q8_K) == 292, "q8_K");
_Static_assert(sizeof(tsx_block_iq3_xxs) == 98, "iq3_xxs");
_Static_assert(sizeof(tsx_block_iq3_s) == 110, "iq3_s");
_Static_assert(sizeof(tsx_block_q4_0) == 18, "q4_0");
_Static_assert(sizeof(tsx_block_q6_K) == 210, "q6_K");
#endif

/* values per block and bytes per block of a type; 0 for a type outside this path */
static inline int tsx_type_qk(int type) {
    switch (type) {
        case TSX_Q4_0: case TSX_Q8_0: case TSX_Q8_1: return 32;
        case TSX_Q4_K: case TSX_Q6_K: case TSX_Q8_K: case TSX_IQ3_XXS: case TSX_IQ3_S: return 256;
        default: return 0;
    }
}
static inline size_t tsx_type_block_bytes(int type) {
    switch (type) {
        case TSX_Q4_0: return 18;
        case TSX_Q8_0: return 34;
        case TSX_Q8_1: return 36;
        case TSX_Q6_K: return 210;
        case TSX_Q4_K: return 144;
        case TSX_Q8_K: return 292;
        case TSX_IQ3_XXS: return 98;
        case TSX_IQ3_S: return 110;
        default: return 0;
    }
}
/* the weight formats the expert kernels take */
static inline int tsx_weight_type_ok(int type) {
    return type == TSX_Q8_0 || type == TSX_Q4_K || type == TSX_IQ3_XXS || type == TSX_IQ3_S;
}
/* the weight formats the single-matrix and id-indexed products take: the expert formats, Q4_0 and Q6_K */
static inline int tsx_mmvq_type_ok(int type) { return tsx_weight_type_ok(type) || type == TSX_Q4_0 || type == TSX_Q6_K; }
/* bytes of one row of n values (n a multiple of the block); 0 when it is not */
static inline size_t tsx_row_bytes(int type, int64_t n) {
    const int qk = tsx_type_qk(type);
    if (qk == 0 || n <= 0 || n % qk != 0) return 0;
    return (size_t) (n / qk) * tsx_type_block_bytes(type);
}

/* One expert blob: [gate rows | up rows | down rows], raw GGUF blocks (reference NativeExpertLayout). */
typedef struct {
    int32_t gu_type, d_type;
    int64_t n_embd, n_ff;
    uint64_t gu_row, d_row;     /* bytes per row */
    uint64_t up_off, down_off;  /* byte offsets inside the blob */
    uint64_t bytes;             /* the whole blob */
} tsx_expert_layout;

static inline tsx_expert_layout tsx_make_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff) {
    tsx_expert_layout L;
    L.gu_type = gu_type;
    L.d_type = d_type;
    L.n_embd = n_embd;
    L.n_ff = n_ff;
    L.gu_row = tsx_row_bytes(gu_type, n_embd);
    L.d_row = tsx_row_bytes(d_type, n_ff);
    L.up_off = (uint64_t) n_ff * L.gu_row;
    L.down_off = 2 * L.up_off;
    L.bytes = L.down_off + (uint64_t) n_embd * L.d_row;
    return L;
}

#ifdef __cplusplus
}
#endif
#endif
