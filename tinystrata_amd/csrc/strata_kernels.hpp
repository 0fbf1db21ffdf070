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
//                                                  quantize, Product, Context::run, swiglu, iota)
// links against this library instead.  Errors: unsupported types/shapes in the expert and mmq paths print a message
// and exit(1) (src/kernels/cuda/iq_kernels.cu:31-34, src/prefill/moe_mmq.cu:39-44); the router throws
// std::invalid_argument / std::runtime_error (src/kernels/cuda/native_router.cu:103-110); the mmvq byte and launch
// helpers throw std::invalid_argument for an unsupported id (include/strata/kernels/native_mmvq.hpp:122-127).
#pragma once

#include <cstddef>
#include <cstdint>

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

bool built();
bool supported(int ggml_type);
bool fits(int ggml_type, int64_t w_rows);
size_t matrix_bytes(int ggml_type, int64_t rows, int64_t cols);
size_t q8_bytes(int64_t rows, int64_t cols);
void quantize(const float* x, const int32_t* ids, void* xq, int ggml_type, int64_t cols, int64_t ld, int64_t rows,
              void* stream, float* yscale = nullptr);

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

class Context {
public:
    Context() = default;
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    void run(const Product& p, void* stream);
};

void swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, void* stream);
void iota(int32_t* dst, int64_t n, void* stream);

}  // namespace strata::prefill::mmq
