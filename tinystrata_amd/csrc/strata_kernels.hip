// strata_kernels.hip - the reference's C++ operator API (strata_kernels.hpp) over libtsx_moe's C ABI.
#include "strata_kernels.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "tsx_moe.h"

namespace {
// the reference's expert/mmq convention: say what failed and stop the process
void check_exit(int rc, const char* what) {
    if (rc == TSX_OK) return;
    std::fprintf(stderr, "%s: %s\n", what, tsx_moe_last_error());
    std::exit(1);
}
tsx_expert_layout to_c(const strata::kernels::NativeExpertLayout& L) {
    tsx_expert_layout c;
    c.gu_type = L.gu_type;
    c.d_type = L.d_type;
    c.n_embd = L.n_embd;
    c.n_ff = L.n_ff;
    c.gu_row = L.gu_row;
    c.d_row = L.d_row;
    c.up_off = L.up_off;
    c.down_off = L.down_off;
    c.bytes = L.bytes;
    return c;
}
__global__ void iota_kernel(int32_t* dst, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (int32_t) i;
}
}  // namespace

namespace strata::kernels {

bool iq_supported(int t) noexcept { return tsx_weight_type_ok(t) != 0; }
size_t iq_row_bytes(int t, int64_t n) noexcept { return tsx_row_bytes(t, n); }

void quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream) {
    check_exit(tsx_moe_quantize_q8_1(x, n_rows, n_cols, y, stream), "quantize_q8_1_rows");
}

void iq_mmvq(int t, const void* w, const void* x, float* y, int n_in, int n_out, int ncols, void* stream) {
    check_exit(tsx_moe_mmvq(t, w, x, y, n_in, n_out, ncols, stream), "iq_mmvq");
}

NativeExpertLayout native_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff) {
    const tsx_expert_layout c = tsx_make_layout(gu_type, d_type, n_embd, n_ff);
    NativeExpertLayout L;
    L.gu_type = c.gu_type;
    L.d_type = c.d_type;
    L.n_embd = c.n_embd;
    L.n_ff = c.n_ff;
    L.gu_row = c.gu_row;
    L.d_row = c.d_row;
    L.up_off = c.up_off;
    L.down_off = c.down_off;
    L.bytes = c.bytes;
    return L;
}

bool native_expert_supported(int g, int d, int64_t n_embd, int64_t n_ff) noexcept {
    return tsx_moe_expert_supported(g, d, n_embd, n_ff) != 0;
}

size_t native_expert_scratch_bytes(int64_t cap, int64_t n_ff) { return tsx_moe_expert_scratch_bytes(cap, n_ff); }

void native_expert_grouped(const NativeExpertLayout& L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                           const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok, int64_t cap_groups,
                           int64_t cap_entries, const void* x_q8_1, void* scratch, float* out, void* stream,
                           int64_t grid_groups) {
    if (L.tail_off != 0) {
        std::fprintf(stderr, "native_expert_grouped: NVFP4 experts are not on this path\n");
        std::exit(1);
    }
    const tsx_expert_layout c = to_c(L);
    check_exit(tsx_moe_expert_grouped(&c, (const uint64_t*) grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups,
                                      cap_entries, x_q8_1, scratch, out, stream, grid_groups),
               "native_expert_grouped");
}

std::size_t native_q8_1_bytes(int n_in, int ncols) { return (size_t) (n_in / 32) * 36u * (size_t) ncols; }

void native_quantize_q8_1(const float* x, void* x_q8_1, int n_in, int ncols, void* stream) {
    check_exit(tsx_moe_quantize_q8_1(x, ncols, n_in, x_q8_1, stream), "native_quantize_q8_1");
}

void native_swiglu_quantize_q8_1(const float* gate, const float* up, void* x_q8_1, int n_in, int ncols, void* stream) {
    check_exit(tsx_moe_swiglu_quantize_q8_1(gate, up, (int64_t) n_in * ncols, x_q8_1, stream), "native_swiglu_quantize_q8_1");
}

bool native_mmvq_supported(int t) noexcept { return tsx_mmvq_type_ok(t) != 0; }

std::size_t native_mmvq_weight_bytes(int t, int n_in, int n_out) {
    const size_t rb = tsx_row_bytes(t, n_in);
    if (!tsx_mmvq_type_ok(t) || rb == 0) throw std::invalid_argument("native_mmvq_weight_bytes: unsupported type or width");
    return rb * (size_t) n_out;
}

void native_mmvq(int t, const void* w, const void* x, float* y, int n_in, int n_out, int ncols, void* stream) {
    if (!native_mmvq_supported(t)) throw std::invalid_argument("native_mmvq: unsupported GGML type " + std::to_string(t));
    const int rc = tsx_moe_mmvq(t, w, x, y, n_in, n_out, ncols, stream);
    if (rc == TSX_ERR_UNSUPPORTED || rc == TSX_ERR_ARG) throw std::invalid_argument(tsx_moe_last_error());
    if (rc != TSX_OK) throw std::runtime_error(tsx_moe_last_error());
}

bool lfm_native_mmvq_ids_supported(int t) { return tsx_moe_mmvq_ids_supported(t) != 0; }

bool lfm_native_mmvq_ids(int t, const MmvqIds& m, int count, int n_in, int n_out, void* stream) {
    if (!lfm_native_mmvq_ids_supported(t)) return false;
    if (n_out <= 0 || count < 0 || count > 65535 || m.x_every <= 0)
        throw std::invalid_argument("lfm_native_mmvq_ids requires n_out > 0, 1 to 65535 matrices and x_every > 0");
    // the reference does not bound the ids: the table is taken as large as an int32 id can reach
    const tsx_mmvq_ids a{m.table, m.ids, INT32_MAX, m.offset, m.x, m.x_stride, m.x_every, m.y, m.y_stride};
    const int rc = tsx_moe_mmvq_ids(t, &a, count, n_in, n_out, stream);
    if (rc == TSX_ERR_UNSUPPORTED) return false;
    if (rc != TSX_OK) throw std::runtime_error(tsx_moe_last_error());
    return true;
}

bool lfm_native_mmvq_slots(int t, const MmvqSlots& m, int count, int n_in, int n_out, void* stream) {
    if (!lfm_native_mmvq_ids_supported(t)) return false;
    tsx_mmvq_slots a{};
    for (int j = 0; j < 8; ++j) {
        a.w[j] = m.w[j];
        a.x[j] = m.x[j];
        a.y[j] = m.y[j];
    }
    const int rc = tsx_moe_mmvq_slots(t, &a, count, n_in, n_out, stream);
    if (rc == TSX_ERR_UNSUPPORTED) return false;
    if (rc != TSX_OK) throw std::runtime_error(tsx_moe_last_error());
    return true;
}

bool native_router_topk_supported(int n_expert, int k) {
    return n_expert > 0 && n_expert % 64 == 0 && n_expert <= 512 && k >= 1 && k <= 16 && k <= n_expert;
}

void native_router_topk(const float* logits, int32_t* ids, float* weights, int n_expert, int k, int n_tok, void* stream) {
    if (!stream || n_tok < 1 || !native_router_topk_supported(n_expert, k))
        throw std::invalid_argument("native_router_topk: a stream, a supported (experts, k) and aligned buffers");
    const int rc = tsx_moe_router_topk(logits, ids, weights, n_expert, k, n_tok, stream);
    if (rc == TSX_ERR_ARG || rc == TSX_ERR_UNSUPPORTED)
        throw std::invalid_argument("native_router_topk: a stream, a supported (experts, k) and aligned buffers");
    if (rc != TSX_OK) throw std::runtime_error(tsx_moe_last_error());
}

}  // namespace strata::kernels

namespace strata::prefill::mmq {

bool built() { return true; }
bool supported(int t) { return tsx_weight_type_ok(t) != 0; }
bool fits(int t, int64_t w_rows) { return supported(t) && w_rows > 0; }
size_t matrix_bytes(int t, int64_t rows, int64_t cols) { return tsx_row_bytes(t, cols) * (size_t) rows; }
size_t q8_bytes(int64_t rows, int64_t cols) { return tsx_moe_mmq_q8_bytes(rows, cols); }

void quantize(const float* x, const int32_t* ids, void* xq, int t, int64_t cols, int64_t ld, int64_t rows, void* stream,
              float* yscale) {
    if (yscale != nullptr) {
        std::fprintf(stderr, "prefill mmq: FP4 activations are not on this path\n");
        std::exit(1);
    }
    check_exit(tsx_moe_mmq_quantize(x, ids, xq, t, cols, ld, rows, stream), "prefill mmq: quantize");
}

Nvfp4Mode nvfp4_mode() { return Nvfp4Mode::W4A8; }
bool fp4_activations(int) { return false; }

void scale_gu_rows(float*, int64_t, int64_t, const int32_t*, int, const float*, int64_t, int64_t, void*) {
    std::fprintf(stderr, "prefill mmq: NVFP4 expert scales are not on this path\n");
    std::exit(1);
}

void scale_down_rows(float*, int64_t, const int32_t*, int, const float*, int64_t, void*) {
    std::fprintf(stderr, "prefill mmq: NVFP4 expert scales are not on this path\n");
    std::exit(1);
}

Context::Context() = default;
Context::~Context() { (void) ctx_; }

void Context::run(const Product& p, void* stream) {
    if (p.n <= 0) return;
    if (p.y_scale != nullptr) {
        std::fprintf(stderr, "prefill mmq: FP4 activations are not on this path\n");
        std::exit(1);
    }
    tsx_mmq_product c;
    c.w = p.w;
    c.type = p.type;
    c.n = p.n;
    c.w_rows = p.w_rows;
    c.w_cols = p.w_cols;
    c.expert_bytes = p.expert_bytes;
    c.xq = p.xq;
    c.bounds = p.bounds;
    c.ids = p.ids;
    c.total_rows = p.total_rows;
    c.max_rows = p.max_rows;
    c.dst = p.dst;
    c.ld_dst = p.ld_dst;
    check_exit(tsx_moe_mmq_run(&c, stream), "prefill mmq: mul_mat_q");
}

void swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, void* stream) {
    check_exit(tsx_moe_mmq_swiglu(gu, h, rows, n_ff, interleaved ? 1 : 0, stream), "prefill mmq: swiglu");
}

void iota(int32_t* dst, int64_t n, void* stream) {
    if (n <= 0) return;
    iota_kernel<<<(unsigned) ((n + 255) / 256), 256, 0, (hipStream_t) stream>>>(dst, n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "prefill mmq: iota: %s\n", hipGetErrorString(e));
        std::exit(1);
    }
}

}  // namespace strata::prefill::mmq
