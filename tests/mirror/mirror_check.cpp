// mirror_check.cpp - test library: drives the C++ operator API of strata_kernels.hpp (the reference's
// strata::kernels / strata::prefill::mmq interface) from C++ and exposes each call as a plain extern "C" function for
// the tests to reach through ctypes.  Built beside libtsx_moe.so (tinystrata_amd/libtsx_mirror_check.so) and linked
// against it; nothing in the library itself uses it.
//
// Error behaviour under test: the router and mmvq helpers throw (std::invalid_argument / std::runtime_error), which
// the entry points catch and return as 1 / 2 with the message; the expert and mmq wrappers end the process on an
// unsupported call, which no test triggers.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "strata_kernels.hpp"

namespace K = strata::kernels;
namespace M = strata::prefill::mmq;

namespace {
void put(char* msg, int cap, const char* what) {
    if (msg != nullptr && cap > 0) std::snprintf(msg, (size_t) cap, "%s", what);
}
template <typename F>
int caught(char* msg, int cap, F&& f) {
    try {
        f();
        put(msg, cap, "");
        return 0;
    } catch (const std::invalid_argument& e) {
        put(msg, cap, e.what());
        return 1;
    } catch (const std::runtime_error& e) {
        put(msg, cap, e.what());
        return 2;
    }
}
}  // namespace

extern "C" {

// NativeExpertLayout as native_expert_layout gives it: gu_row, d_row, up_off, down_off, bytes, tail_off
int smc_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, uint64_t* out6) {
    if (!K::native_expert_supported(gu_type, d_type, n_embd, n_ff)) return 0;
    const K::NativeExpertLayout L = K::native_expert_layout(gu_type, d_type, n_embd, n_ff);
    const uint64_t v[6] = {L.gu_row, L.d_row, L.up_off, L.down_off, L.bytes, L.tail_off};
    std::memcpy(out6, v, sizeof v);
    return 1;
}

uint64_t smc_expert_scratch_bytes(int64_t cap_entries, int64_t n_ff) {
    return K::native_expert_scratch_bytes(cap_entries, n_ff);
}

// native_expert_grouped with the layout built by native_expert_layout
int smc_expert_grouped(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, const unsigned long long* grp_ptr,
                       const int32_t* grp_start, const int32_t* n_groups, const int32_t* ent_dst,
                       const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries, const void* x_q8_1,
                       void* scratch, float* out, void* stream, int64_t grid_groups) {
    if (!K::native_expert_supported(gu_type, d_type, n_embd, n_ff)) return -1;
    const K::NativeExpertLayout L = K::native_expert_layout(gu_type, d_type, n_embd, n_ff);
    K::native_expert_grouped(L, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups, cap_entries, x_q8_1,
                             scratch, out, stream, grid_groups);
    return 0;
}

int smc_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream) {
    K::quantize_q8_1_rows(x, n_rows, n_cols, y, stream);
    return 0;
}

int smc_router_topk(const float* logits, int32_t* ids, float* weights, int n_expert, int k, int n_tok, void* stream,
                    char* msg, int cap) {
    return caught(msg, cap, [&] { K::native_router_topk(logits, ids, weights, n_expert, k, n_tok, stream); });
}

int smc_router_topk_supported(int n_expert, int k) { return K::native_router_topk_supported(n_expert, k) ? 1 : 0; }

int smc_mmvq(int type, const void* w, const void* x, float* y, int n_in, int n_out, int ncols, void* stream, char* msg,
             int cap) {
    return caught(msg, cap, [&] { K::native_mmvq(type, w, x, y, n_in, n_out, ncols, stream); });
}

int smc_mmvq_weight_bytes(int type, int n_in, int n_out, uint64_t* out, char* msg, int cap) {
    return caught(msg, cap, [&] { *out = K::native_mmvq_weight_bytes(type, n_in, n_out); });
}

// prefill: the caller's sequence (quantize, Product, Context::run, swiglu, iota)
uint64_t smc_mmq_q8_bytes(int64_t rows, int64_t cols) { return M::q8_bytes(rows, cols); }
int smc_mmq_supported(int type, int64_t w_rows) { return M::supported(type) && M::fits(type, w_rows) ? 1 : 0; }

int smc_mmq_quantize(const float* x, const int32_t* ids, void* xq, int type, int64_t cols, int64_t ld, int64_t rows,
                     void* stream) {
    M::quantize(x, ids, xq, type, cols, ld, rows, stream);
    return 0;
}

int smc_mmq_run(const void* w, int type, int64_t w_rows, int64_t w_cols, uint64_t expert_bytes, int n, const void* xq,
                const int32_t* bounds, const int32_t* ids, int64_t total_rows, int64_t max_rows, float* dst,
                int64_t ld_dst, void* stream) {
    M::Context ctx;
    M::Product p;
    p.w = w;
    p.type = type;
    p.w_rows = w_rows;
    p.w_cols = w_cols;
    p.expert_bytes = (size_t) expert_bytes;
    p.n = n;
    p.xq = xq;
    p.bounds = bounds;
    p.ids = ids;
    p.total_rows = total_rows;
    p.max_rows = max_rows;
    p.dst = dst;
    p.ld_dst = ld_dst;
    ctx.run(p, stream);
    return 0;
}

int smc_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream) {
    M::swiglu(gu, h, rows, n_ff, interleaved != 0, stream);
    return 0;
}

int smc_mmq_iota(int32_t* dst, int64_t n, void* stream) {
    M::iota(dst, n, stream);
    return 0;
}

// the row-map helpers (host only)
int smc_margin_rows(int64_t max_rows, int tile_cols_max, int64_t* out) {
    return M::mmq_ids_margin_rows(max_rows, tile_cols_max, out) ? 1 : 0;
}
int smc_margin_rows_null(int64_t max_rows, int tile_cols_max) {
    return M::mmq_ids_margin_rows(max_rows, tile_cols_max, nullptr) ? 1 : 0;
}
uint64_t smc_table_rows(uint64_t logical_rows, uint64_t max_rows, int tile_cols_max) {
    return M::mmq_ids_table_rows(logical_rows, max_rows, tile_cols_max);
}
uint64_t smc_table_rows_default(uint64_t logical_rows, uint64_t max_rows) {
    return M::mmq_ids_table_rows(logical_rows, max_rows);
}
// io3: in, what the layout holds before the call; out, after it
int smc_ids_layout(uint64_t logical_rows, uint64_t max_rows, uint64_t* io3) {
    M::IdsLayout L;
    L.logical_rows = (size_t) io3[0];
    L.storage_rows = (size_t) io3[1];
    L.storage_bytes = (size_t) io3[2];
    const bool ok = M::ids_layout(logical_rows, max_rows, L);
    io3[0] = L.logical_rows;
    io3[1] = L.storage_rows;
    io3[2] = L.storage_bytes;
    return ok ? 1 : 0;
}
// out10: ids (logical, storage, bytes), place, bounds, relative, weights, classes, words, bytes
int smc_packed_ids_layout(uint64_t logical_rows, uint64_t max_rows, uint64_t experts, uint64_t classes,
                          uint64_t* out10) {
    M::PackedIdsLayout p;
    if (!M::packed_ids_layout(logical_rows, max_rows, experts, classes, p)) return 0;
    const uint64_t v[10] = {p.ids.logical_rows, p.ids.storage_rows, p.ids.storage_bytes, p.place, p.bounds,
                            p.relative, p.weights, p.classes, p.words, p.bytes};
    std::memcpy(out10, v, sizeof v);
    return 1;
}
int smc_tile_cols(int* max_step) {
    max_step[0] = M::kMmqTileColsMax;
    max_step[1] = M::kMmqTileColsStep;
    return 1;
}

}  // extern "C"
