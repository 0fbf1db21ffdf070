// strata_kernels.hpp - the reference's C++ operator API for the MoE expert path, on top of libtsx_moe's C ABI.
//
// Same namespaces, names, argument meanings and error behaviour as TinyStrata's headers, so an engine that calls
//   include/strata/kernels/iq_kernels.hpp:17-78   (iq_supported, iq_row_bytes, quantize_q8_1_rows, iq_mmvq,
//                                                  NativeExpertLayout, native_expert_layout / _supported /
//                                                  _scratch_bytes, native_expert_grouped)
//   include/strata/kernels/native_mmvq.hpp:26-42,125-131 (native_q8_1_bytes, native_quantize_q8_1,
//                                                  native_swiglu_quantize_q8_1, native_mmvq_supported,
//                                                  native_mmvq_weight_bytes, native_mmvq)
//   include/strata/kernels/native_router.hpp:5-6   (native_router_topk_supported, native_router_topk)
//   include/strata/prefill/moe_mmq.hpp:16-120      (prefill::mmq::built, supported, fits, matrix_bytes, q8_bytes,
//                                                  quantize, fp4_activations, scale_gu_rows, scale_down_rows,
//                                                  Product, Context, swiglu, iota)
//   include/strata/prefill/mmq_ids_margin.hpp:13-47 (kMmqTileColsMax/Step, mmq_ids_margin_rows,
//                                                  mmq_ids_table_rows, IdsLayout, ids_layout, packed_ids_layout)
// links against this library instead.  Errors: unsupported types/shapes in the expert and mmq paths print a message
// and exit(1) (src/kernels/cuda/iq_kernels.cu:31-34, src/prefill/moe_mmq.cu:39-44); the router throws
// std::invalid_argument / std::runtime_error (src/kernels/cuda/native_router.cu:103-110); the mmvq byte and launch
// helpers throw std::invalid_argument for an unsupported id (include/strata/kernels/native_mmvq.hpp:122-127).
#pragma once

#include <cstddef>
#include <cstdint>
#include <limits>

namespace strata::kernels {

bool iq_supported(int ggml_type) noexcept;
size_t iq_row_bytes(int ggml_type, int64_t n) noexcept;
void quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream);
void iq_mmvq(int ggml_type, const void* w, const void* x_q8_1, float* y, int n_in, int n_out, int ncols, void* stream);

struct NativeExpertLayout {
    int gu_type = -1, d_type = -1;
    int64_t n_embd = 0, n_ff = 0;
    size_t gu_row = 0, d_row = 0;
    size_t up_off = 0, down_off = 0;
    size_t bytes = 0;
    size_t tail_off = 0;  // no NVFP4 here: always 0
};
NativeExpertLayout native_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff);
bool native_expert_supported(int gu_type, int d_type, int64_t n_embd, int64_t n_ff) noexcept;
size_t native_expert_scratch_bytes(int64_t cap_entries, int64_t n_ff);
void native_expert_grouped(const NativeExpertLayout& L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                           const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok, int64_t cap_groups,
                           int64_t cap_entries, const void* x_q8_1, void* scratch, float* out, void* stream,
                           int64_t grid_groups = 0);

std::size_t native_q8_1_bytes(int n_in, int ncols = 1);
void native_quantize_q8_1(const float* x, void* x_q8_1, int n_in, int ncols, void* stream);
void native_swiglu_quantize_q8_1(const float* gate, const float* up, void* x_q8_1, int n_in, int ncols, void* stream);
bool native_mmvq_supported(int ggml_type) noexcept;
std::size_t native_mmvq_weight_bytes(int ggml_type, int n_in, int n_out);
void native_mmvq(int ggml_type, const void* weights, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                 void* stream);

// Several matrices of one format and shape in one launch (include/strata/lfm2/matvec.hpp:146-168): up to 8 given by
// the host (MmvqSlots), or picked on the device through a table of matrix pointers (MmvqIds).  False, with nothing
// launched, for a format there is no kernel for.
struct MmvqSlots {
    const void* w[8];
    const void* x[8];
    float* y[8];
};
bool lfm_native_mmvq_slots(int ggml_type, const MmvqSlots& slots, int count, int n_in, int n_out, void* stream);
struct MmvqIds {
    const void* const* table;
    const int32_t* ids;
    std::size_t offset;
    const void* x;
    std::size_t x_stride;
    int x_every;
    float* y;
    std::size_t y_stride;
};
bool lfm_native_mmvq_ids_supported(int ggml_type);
bool lfm_native_mmvq_ids(int ggml_type, const MmvqIds& ids, int count, int n_in, int n_out, void* stream);

bool native_router_topk_supported(int n_expert, int k);
void native_router_topk(const float* logits, int32_t* ids, float* weights, int n_expert, int k, int n_tok, void* stream);

}  // namespace strata::kernels

namespace strata::prefill::mmq {

// ---- row-map storage (include/strata/prefill/mmq_ids_margin.hpp:13-47).  The reference's tile loop can read a whole
// tile of row ids past an expert's last row (up to kMmqTileColsMax columns, in steps of kMmqTileColsStep), so a row map
// is stored with a margin of one widest tile beyond max_rows rounded up to whole tiles.  The kernels here read a row
// id only for rows inside their expert, so the margin is never read; callers size and fill it the same way all the
// same, and these helpers give the same sizes and the same refusals (false or 0, with the output untouched).
constexpr int kMmqTileColsMax = 128;
constexpr int kMmqTileColsStep = 8;

// *out = max_rows rounded up to a multiple of tile_cols_max, plus one more tile_cols_max
inline bool mmq_ids_margin_rows(int64_t max_rows, int tile_cols_max, int64_t* out) {
    if (out == nullptr || max_rows < 0 || tile_cols_max <= 0) return false;
    constexpr int64_t top = std::numeric_limits<int64_t>::max();
    const int64_t t = tile_cols_max;
    const int64_t whole = max_rows / t + (max_rows % t ? 1 : 0);  // tiles covering max_rows
    if (whole > top / t) return false;
    const int64_t covered = whole * t;
    if (covered > top - t) return false;
    *out = covered + t;
    return true;
}

// logical_rows plus that margin; 0 when it cannot be represented
inline uint64_t mmq_ids_table_rows(uint64_t logical_rows, uint64_t max_rows, int tile_cols_max = kMmqTileColsMax) {
    constexpr uint64_t top = std::numeric_limits<uint64_t>::max();
    if (max_rows > (uint64_t) std::numeric_limits<int64_t>::max()) return 0;
    int64_t margin = 0;
    if (!mmq_ids_margin_rows((int64_t) max_rows, tile_cols_max, &margin)) return 0;
    if (logical_rows > top - (uint64_t) margin) return 0;
    return logical_rows + (uint64_t) margin;
}

struct IdsLayout {
    size_t logical_rows = 0, storage_rows = 0, storage_bytes = 0;
};

// an int32 row map of logical_rows ids stored with the margin: false (out untouched) when the stored rows exceed
// what an int32 id or a size_t byte count can hold
inline bool ids_layout(uint64_t logical_rows, uint64_t max_rows, IdsLayout& out) {
    const uint64_t rows = mmq_ids_table_rows(logical_rows, max_rows);
    if (rows == 0 || rows > (uint64_t) std::numeric_limits<int32_t>::max()) return false;
    if (rows > (uint64_t) (std::numeric_limits<size_t>::max() / sizeof(int32_t))) return false;
    out.logical_rows = (size_t) logical_rows;
    out.storage_rows = (size_t) rows;
    out.storage_bytes = (size_t) rows * sizeof(int32_t);
    return true;
}

// one int32 buffer holding, in this order: the row map (ids.storage_rows words at `place`), bounds (experts + 1),
// relative bounds (2 experts + 2), weights (logical_rows) and a classes x (experts + 1) table; offsets in words
struct PackedIdsLayout {
    IdsLayout ids;
    size_t place = 0, bounds = 0, relative = 0, weights = 0, classes = 0, words = 0, bytes = 0;
};

inline bool packed_ids_layout(uint64_t logical_rows, uint64_t max_rows, uint64_t experts, uint64_t classes,
                              PackedIdsLayout& out) {
    constexpr uint64_t i32 = (uint64_t) std::numeric_limits<int32_t>::max();
    IdsLayout ids;
    if (!ids_layout(logical_rows, max_rows, ids) || experts > i32 || classes > i32) return false;
    // every term is now below 2^31, so the sums below stay far inside uint64
    const uint64_t at_bounds = logical_rows + ids.storage_rows;
    const uint64_t at_relative = at_bounds + experts + 1;
    const uint64_t at_weights = at_relative + 2 * experts + 2;
    const uint64_t at_classes = at_weights + logical_rows;
    const uint64_t words = at_classes + classes * (experts + 1);
    if (words > (uint64_t) (std::numeric_limits<size_t>::max() / sizeof(int32_t))) return false;
    PackedIdsLayout p;
    p.ids = ids;
    p.place = (size_t) logical_rows;
    p.bounds = (size_t) at_bounds;
    p.relative = (size_t) at_relative;
    p.weights = (size_t) at_weights;
    p.classes = (size_t) at_classes;
    p.words = (size_t) words;
    p.bytes = (size_t) words * sizeof(int32_t);
    out = p;
    return true;
}

bool built();
bool supported(int ggml_type);
bool fits(int ggml_type, int64_t w_rows);
size_t matrix_bytes(int ggml_type, int64_t rows, int64_t cols);
size_t q8_bytes(int64_t rows, int64_t cols);
void quantize(const float* x, const int32_t* ids, void* xq, int ggml_type, int64_t cols, int64_t ld, int64_t rows,
              void* stream, float* yscale = nullptr);
// NVFP4 experts are not on this path: no type takes FP4 activations, and the NVFP4 tail scalings print a message and
// exit(1) as the reference does for a type it has no kernel for
enum class Nvfp4Mode { W4A8, W4A4, FP16 };
Nvfp4Mode nvfp4_mode();
bool fp4_activations(int ggml_type);
void scale_gu_rows(float* gu, int64_t ld, int64_t n_ff, const int32_t* bounds, int n, const float* tails, int64_t row0,
                   int64_t nrows, void* stream);
void scale_down_rows(float* d, int64_t ld, const int32_t* bounds, int n, const float* tails, int64_t nrows, void* stream);

struct Product {
    const void* w = nullptr;
    int type = -1;
    int64_t w_rows = 0, w_cols = 0;
    size_t expert_bytes = 0;
    int n = 0;
    const void* xq = nullptr;
    const int32_t* bounds = nullptr;
    const int32_t* ids = nullptr;
    int64_t total_rows = 0, max_rows = 0;
    float* dst = nullptr;
    int64_t ld_dst = 0;
    const float* y_scale = nullptr;  // NVFP4 only in the reference: must be null here
};

// One per prompt path, as in the reference.  The kernels here keep no state between launches (no stream-k fixup
// buffer), so the context holds nothing; it keeps the reference's shape (a private handle) so code built against
// either header agrees on its size.
class Context {
public:
    Context();
    ~Context();
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    void run(const Product& p, void* stream);

private:
    void* ctx_ = nullptr;
};

void swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, void* stream);
void iota(int32_t* dst, int64_t n, void* stream);

}  // namespace strata::prefill::mmq
