// api_shape.cpp - built twice by tests/test_mirror_api.py: against the reference's own headers
// (-DAPI_SHAPE_REFERENCE -I<reference>/include) and against strata_kernels.hpp, each time linked to libtsx_moe.so.
// The link proves that every operator-API function the reference's callers use resolves to this library with the
// reference's exact signature (C++ mangled names carry the parameter types); the printed sizes and field offsets of
// the argument structs must then agree between the two builds.  It calls nothing: running it needs no GPU.
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <initializer_list>

#ifdef API_SHAPE_REFERENCE
#include "strata/kernels/iq_kernels.hpp"
#include "strata/kernels/native_mmvq.hpp"
#include "strata/kernels/native_router.hpp"
#include "strata/prefill/moe_mmq.hpp"
#else
#include "strata_kernels.hpp"
#endif

namespace K = strata::kernels;
namespace M = strata::prefill::mmq;

#define FIELD(T, f) std::printf(#T "." #f " %zu\n", offsetof(T, f))

int main() {
    // each function by address, with its exact type (a different signature fails to compile or to link)
    void* volatile sink[] = {
        (void*) (bool (*)(int) noexcept) & K::iq_supported,
        (void*) (size_t (*)(int, int64_t) noexcept) & K::iq_row_bytes,
        (void*) (void (*)(const float*, int64_t, int64_t, void*, void*)) & K::quantize_q8_1_rows,
        (void*) (void (*)(int, const void*, const void*, float*, int, int, int, void*)) & K::iq_mmvq,
        (void*) (K::NativeExpertLayout(*)(int, int, int64_t, int64_t)) & K::native_expert_layout,
        (void*) (bool (*)(int, int, int64_t, int64_t) noexcept) & K::native_expert_supported,
        (void*) (size_t (*)(int64_t, int64_t)) & K::native_expert_scratch_bytes,
        (void*) (void (*)(const K::NativeExpertLayout&, const unsigned long long*, const int32_t*, const int32_t*,
                          const int32_t*, const int32_t*, int64_t, int64_t, const void*, void*, float*, void*,
                          int64_t)) & K::native_expert_grouped,
        (void*) (std::size_t (*)(int, int)) & K::native_q8_1_bytes,
        (void*) (void (*)(const float*, void*, int, int, void*)) & K::native_quantize_q8_1,
        (void*) (void (*)(const float*, const float*, void*, int, int, void*)) & K::native_swiglu_quantize_q8_1,
        (void*) (bool (*)(int) noexcept) & K::native_mmvq_supported,
        (void*) (std::size_t (*)(int, int, int)) & K::native_mmvq_weight_bytes,
        (void*) (void (*)(int, const void*, const void*, float*, int, int, int, void*)) & K::native_mmvq,
        (void*) (bool (*)(int, int)) & K::native_router_topk_supported,
        (void*) (void (*)(const float*, int32_t*, float*, int, int, int, void*)) & K::native_router_topk,
        (void*) (bool (*)()) & M::built,
        (void*) (bool (*)(int)) & M::supported,
        (void*) (bool (*)(int, int64_t)) & M::fits,
        (void*) (size_t (*)(int, int64_t, int64_t)) & M::matrix_bytes,
        (void*) (size_t (*)(int64_t, int64_t)) & M::q8_bytes,
        (void*) (void (*)(const float*, const int32_t*, void*, int, int64_t, int64_t, int64_t, void*, float*)) &
            M::quantize,
        (void*) (bool (*)(int)) & M::fp4_activations,
        (void*) (void (*)(float*, int64_t, int64_t, const int32_t*, int, const float*, int64_t, int64_t, void*)) &
            M::scale_gu_rows,
        (void*) (void (*)(float*, int64_t, const int32_t*, int, const float*, int64_t, void*)) & M::scale_down_rows,
        (void*) (void (*)(const float*, float*, int64_t, int64_t, bool, void*)) & M::swiglu,
        (void*) (void (*)(int32_t*, int64_t, void*)) & M::iota,
    };
    void (M::Context::*run)(const M::Product&, void*) = &M::Context::run;
    (void) run;
    {  // the constructor and destructor are out of line in both headers: this links them
        M::Context* c = sink[0] == nullptr ? new M::Context() : nullptr;
        delete c;
    }
    std::printf("functions %zu\n", sizeof sink / sizeof sink[0]);

    std::printf("NativeExpertLayout %zu\n", sizeof(K::NativeExpertLayout));
    FIELD(K::NativeExpertLayout, gu_type);
    FIELD(K::NativeExpertLayout, d_type);
    FIELD(K::NativeExpertLayout, n_embd);
    FIELD(K::NativeExpertLayout, n_ff);
    FIELD(K::NativeExpertLayout, gu_row);
    FIELD(K::NativeExpertLayout, d_row);
    FIELD(K::NativeExpertLayout, up_off);
    FIELD(K::NativeExpertLayout, down_off);
    FIELD(K::NativeExpertLayout, bytes);
    FIELD(K::NativeExpertLayout, tail_off);
    std::printf("Product %zu\n", sizeof(M::Product));
    FIELD(M::Product, w);
    FIELD(M::Product, type);
    FIELD(M::Product, w_rows);
    FIELD(M::Product, w_cols);
    FIELD(M::Product, expert_bytes);
    FIELD(M::Product, n);
    FIELD(M::Product, xq);
    FIELD(M::Product, bounds);
    FIELD(M::Product, ids);
    FIELD(M::Product, total_rows);
    FIELD(M::Product, max_rows);
    FIELD(M::Product, dst);
    FIELD(M::Product, ld_dst);
    FIELD(M::Product, y_scale);
    std::printf("Context %zu\n", sizeof(M::Context));
    std::printf("IdsLayout %zu\n", sizeof(M::IdsLayout));
    FIELD(M::IdsLayout, logical_rows);
    FIELD(M::IdsLayout, storage_rows);
    FIELD(M::IdsLayout, storage_bytes);
    std::printf("PackedIdsLayout %zu\n", sizeof(M::PackedIdsLayout));
    FIELD(M::PackedIdsLayout, ids);
    FIELD(M::PackedIdsLayout, place);
    FIELD(M::PackedIdsLayout, bounds);
    FIELD(M::PackedIdsLayout, relative);
    FIELD(M::PackedIdsLayout, weights);
    FIELD(M::PackedIdsLayout, classes);
    FIELD(M::PackedIdsLayout, words);
    FIELD(M::PackedIdsLayout, bytes);
    std::printf("tile %d %d\n", M::kMmqTileColsMax, M::kMmqTileColsStep);

    // the row-map helpers' values over a grid that crosses tile edges and every overflow guard
    const int64_t i64max = INT64_MAX;
    const uint64_t u64max = UINT64_MAX;
    const int64_t rows[] = {-1, 0, 1, 7, 8, 127, 128, 129, 4096, 32768, INT32_MAX, i64max / 128, i64max - 200, i64max};
    const int tiles[] = {-8, 0, 1, 8, 64, 120, 128};
    for (int64_t r : rows)
        for (int t : tiles) {
            int64_t m = -7;
            const bool ok = M::mmq_ids_margin_rows(r, t, &m);
            std::printf("margin %lld %d -> %d %lld\n", (long long) r, t, (int) ok, (long long) m);
        }
    std::printf("margin null %d\n", (int) M::mmq_ids_margin_rows(5, 128, nullptr));
    const uint64_t logical[] = {0, 1, 100, 800, 32768, (uint64_t) INT32_MAX - 300, (uint64_t) INT32_MAX, u64max - 256,
                                u64max};
    const uint64_t maxr[] = {0, 1, 100, 129, 4096, (uint64_t) i64max, (uint64_t) i64max + 1, u64max};
    for (uint64_t l : logical)
        for (uint64_t m : maxr) {
            std::printf("table %llu %llu -> %llu %llu\n", (unsigned long long) l, (unsigned long long) m,
                        (unsigned long long) M::mmq_ids_table_rows(l, m),
                        (unsigned long long) M::mmq_ids_table_rows(l, m, 8));
            M::IdsLayout L{11, 22, 88};
            const bool ok = M::ids_layout(l, m, L);
            std::printf("ids %d %zu %zu %zu\n", (int) ok, L.logical_rows, L.storage_rows, L.storage_bytes);
        }
    const uint64_t experts[] = {0, 4, 256, (uint64_t) INT32_MAX, (uint64_t) INT32_MAX + 1, u64max};
    for (uint64_t l : {uint64_t(0), uint64_t(32), uint64_t(4096 * 8)})
        for (uint64_t e : experts)
            for (uint64_t c : experts) {
                M::PackedIdsLayout p;
                const bool ok = M::packed_ids_layout(l, l / 8 + 1, e, c, p);
                std::printf("packed %llu %llu %llu -> %d %zu %zu %zu %zu %zu %zu %zu %zu\n", (unsigned long long) l,
                            (unsigned long long) e, (unsigned long long) c, (int) ok, p.ids.storage_rows, p.place,
                            p.bounds, p.relative, p.weights, p.classes, p.words, p.bytes);
            }
    return 0;
}
