/* tsx_gguf.h - GGUF model files for libtsx_moe.so: the tensor directory of a (split) GGUF v3 model, and one layer's
 * routed experts repacked into the [gate | up | down] blobs the expert kernels read.
 *
 * Reference interfaces replaced:
 *   - strata::GgufFile / GgufModel / TensorInfo / MetaValue / tensor_payload_bytes / block_geometry
 *     (include/strata/artifact/gguf_reader.hpp:233-666): mmap, header, metadata of every value type, tensor
 *     directory, alignment, payload sizes, split models;
 *   - strata::gguf_split_paths (include/strata/artifact/gguf_split.hpp:25-55): the shards of a split model from
 *     any one of them;
 *   - the expert repack of the engine's loader and expert_blob (src/qwen35/q36_engine.cu:1144-1168,1196-1201):
 *     ffn_{gate,up,down}_exps of a layer -> per-expert blobs `stride` bytes apart, stride = the blob rounded up
 *     to lcm(both block sizes, 16).
 *
 * Return codes are those of tsx_moe.h (TSX_OK, TSX_ERR_UNSUPPORTED, TSX_ERR_ARG, or a hipError_t for the upload),
 * plus TSX_ERR_FORMAT for a file that is not a well-formed GGUF v3 model and TSX_ERR_NOT_FOUND for a missing
 * tensor or key; tsx_moe_last_error() names the file and the fault.  A handle is used by one thread at a time.
 */
#ifndef TSX_GGUF_H
#define TSX_GGUF_H

#include "tsx_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { TSX_ERR_FORMAT = -3, TSX_ERR_NOT_FOUND = -4 };

typedef struct tsx_gguf tsx_gguf; /* an open model: every shard mapped read-only */

typedef struct {
    const char* name;  /* valid while the model is open */
    int32_t type;      /* ggml type id */
    int32_t n_dims;    /* 1..4 */
    int64_t ne[4];     /* GGUF order: ne[0] varies fastest (a row); dims past n_dims are 1 */
    uint64_t offset;   /* from the start of its shard's data section */
    uint64_t bytes;    /* payload bytes; 0 for a type of unknown block geometry */
    const void* data;  /* the payload in the mapping; null when bytes is 0 or the payload is not inside the file */
    int32_t shard;     /* 0-based shard index */
} tsx_gguf_tensor;

/* Values per block and bytes per block of a ggml type id (block_geometry); TSX_ERR_UNSUPPORTED for an id of unknown
 * geometry. */
TSX_API int tsx_gguf_block_geometry(int type, int* elems, int* bytes);

/* The shard paths of the model `any_shard` belongs to (<stem>-NNNNN-of-MMMMM.gguf, or the path alone), written as
 * NUL-separated strings into buf (n_paths set); TSX_ERR_NOT_FOUND when a shard is missing, TSX_ERR_ARG when buf is
 * too small (the bytes needed in *n_bytes). */
TSX_API int tsx_gguf_split_paths(const char* any_shard, char* buf, size_t cap, int* n_paths, size_t* n_bytes);

/* Opens the model whose shards are paths[0..n_paths) in split order (the metadata shard first).  Refused: a bad
 * magic, a version other than 3, a truncated header, an unknown metadata type, arrays nested deeper than two or
 * longer than 2^24, a tensor with 0 or more than 4 dims, a duplicate tensor name (in a shard or across shards), a
 * data section past the end of a file that has tensors, and shards whose split.count / split.no /
 * split.tensors.count do not describe this model. */
TSX_API int tsx_gguf_open(const char* const* paths, int n_paths, tsx_gguf** out);
/* tsx_gguf_open over tsx_gguf_split_paths(any_shard). */
TSX_API int tsx_gguf_open_model(const char* any_shard, tsx_gguf** out);
TSX_API void tsx_gguf_close(tsx_gguf* g);

TSX_API int tsx_gguf_shard_count(const tsx_gguf* g);
/* version, alignment and data-section start of a shard */
TSX_API int tsx_gguf_shard_info(const tsx_gguf* g, int shard, uint32_t* version, uint64_t* alignment,
                                uint64_t* data_start, uint64_t* file_size);
TSX_API int64_t tsx_gguf_tensor_count(const tsx_gguf* g);
/* tensor i in directory order (shard by shard) */
TSX_API int tsx_gguf_tensor_at(const tsx_gguf* g, int64_t i, tsx_gguf_tensor* out);
TSX_API int tsx_gguf_find(const tsx_gguf* g, const char* name, tsx_gguf_tensor* out);

/* Metadata of the metadata shard (shard 0).  Value types: 0 U8, 1 I8, 2 U16, 3 I16, 4 U32, 5 I32, 6 F32, 7 BOOL,
 * 8 STRING, 9 ARRAY, 10 U64, 11 I64, 12 F64.  Signed integers are sign-extended into *i; *u holds the same bits.
 * For an array: *type = 9, *elem_type and *count describe it, and tsx_gguf_meta_item reads its items (the first
 * 64 are kept; the count is what the file declares). */
TSX_API int tsx_gguf_meta_count(const tsx_gguf* g);
TSX_API const char* tsx_gguf_meta_key(const tsx_gguf* g, int i);
TSX_API int tsx_gguf_meta(const tsx_gguf* g, const char* key, int* type, uint64_t* u, int64_t* i, double* f,
                          const char** s, int* elem_type, uint64_t* count);
TSX_API int tsx_gguf_meta_item(const tsx_gguf* g, const char* key, uint64_t item, uint64_t* u, double* f,
                               const char** s);

/* One layer's routed experts (or its shared expert) as the expert kernels take them. */
typedef struct {
    tsx_expert_layout L;
    uint64_t stride;      /* bytes between blobs: L.bytes rounded up to lcm(gate block, down block, 16) */
    int64_t n_expert;
    const void* gate;     /* the tensors' payloads (expert e's gate rows at gate + e * L.up_off) */
    const void* up;
    const void* down;     /* expert e's down rows at down + e * (L.bytes - L.down_off) */
} tsx_gguf_experts;

/* shared = 0: blk.<layer>.ffn_gate_exps / ffn_up_exps / ffn_down_exps.weight, gate and up of one type and shape
 * [n_embd, n_ff, n_expert], down [n_ff, n_embd, n_expert]; shared = 1: the shared expert's ffn_{gate,up,down}_shexp
 * ([n_embd, n_ff], [n_ff, n_embd]; n_expert = 1).  The payloads must lie inside their files and the type pair and
 * shape must be one the expert kernels take (tsx_moe_expert_supported).  Replaces the loader's ffn_*_exps lookup
 * and checks (src/qwen35/q36_engine.cu:1144-1168; the shared expert's matrices :1135-1137). */
TSX_API int tsx_gguf_layer_experts(const tsx_gguf* g, int layer, int shared, tsx_gguf_experts* out);
/* Expert e's blob into host memory dst (L.bytes). */
TSX_API int tsx_gguf_expert_blob(const tsx_gguf_experts* X, int64_t e, void* dst);
/* Experts e0 .. e0 + n - 1 into device memory: expert e0 + j's blob at dst + j * dst_stride (dst_stride >= L.bytes,
 * a multiple of 16; dst 16-byte aligned), three strided copies on `stream`.  The mapping must stay open until the
 * copies are done (the call returns once they are enqueued; synchronize the stream before closing the model). */
TSX_API int tsx_gguf_upload_experts(const tsx_gguf_experts* X, int64_t e0, int64_t n, void* dst, uint64_t dst_stride,
                                    void* stream);

#ifdef __cplusplus
}
#endif
#endif
