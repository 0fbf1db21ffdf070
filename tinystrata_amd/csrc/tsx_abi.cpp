// tsx_abi.cpp - the library-level entry points of libtsx_moe.so: ABI handshake, device start, errors, layouts.
// Reference: strata_kq_abi / strata_kq_init (src/prefill/mmq_kq_lib.cu:33-43), native_expert_layout /
// native_expert_supported / native_expert_scratch_bytes (src/kernels/cuda/iq_kernels.cu:2114-2143).
#include "tsx_common.hpp"

#include <cstdio>
#include <string>

namespace tsx {
namespace {
thread_local std::string g_error;
}
void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
}
void clear_error() { g_error.clear(); }
const char* error_cstr() { return g_error.c_str(); }
int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return TSX_OK;
    set_error("%s: %s", what, hipGetErrorString(e));
    return (int) e;
}
}  // namespace tsx

extern "C" {

TSX_API int tsx_moe_abi(void) { return TSX_MOE_ABI_VERSION * 100000 + (int) sizeof(tsx_mmq_product); }

TSX_API int tsx_moe_init(int device) {
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipFree(nullptr);
    if (e != hipSuccess) {
        tsx::set_error("tsx_moe_init(%d): %s", device, hipGetErrorString(e));
        return (int) e;
    }
    // the no-allocation decode layer's scratch address on this device, looked up now rather than on its first call;
    // best effort: only tsx_moe_decode_layer_noalloc needs it, and that call looks it up again and reports a failure
    if (!tsx::noalloc_scratch_ptr(nullptr)) {
        (void) hipGetLastError();  // the runtime's error state stays clear for the caller's next HIP call
        tsx::clear_error();
    }
    return TSX_OK;
}

TSX_API const char* tsx_moe_last_error(void) { return tsx::error_cstr(); }

TSX_API size_t tsx_moe_row_bytes(int type, int64_t n) { return tsx_row_bytes(type, n); }

TSX_API int tsx_moe_expert_supported(int gu_type, int d_type, int64_t n_embd, int64_t n_ff) {
    return tsx_weight_type_ok(gu_type) && tsx_weight_type_ok(d_type) && n_embd > 0 && n_ff > 0 &&
           tsx_row_bytes(gu_type, n_embd) != 0 && tsx_row_bytes(d_type, n_ff) != 0 && n_embd % 256 == 0 &&
           n_ff % 32 == 0 && n_embd <= 16384 && n_ff <= 16384;
}

TSX_API int tsx_moe_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, tsx_expert_layout* out) {
    if (out == nullptr) return TSX_ERR_ARG;
    if (!tsx_moe_expert_supported(gu_type, d_type, n_embd, n_ff)) {
        tsx::set_error("expert layout: types (%d, %d) at %lld x %lld not supported", gu_type, d_type,
                       (long long) n_embd, (long long) n_ff);
        return TSX_ERR_UNSUPPORTED;
    }
    *out = tsx_make_layout(gu_type, d_type, n_embd, n_ff);
    return TSX_OK;
}

TSX_API size_t tsx_moe_expert_scratch_bytes(int64_t cap, int64_t n_ff) {
    if (cap <= 0 || n_ff <= 0) return 0;
    const size_t f = (size_t) cap * (size_t) n_ff * sizeof(float);
    return 3 * ((f + 255) & ~(size_t) 255) + (((size_t) cap * (size_t) (n_ff / 32) * 36 + 255) & ~(size_t) 255);
}

TSX_API size_t tsx_moe_expert_scratch_hq_offset(int64_t cap, int64_t n_ff) {
    const size_t f = (size_t) cap * (size_t) n_ff * sizeof(float);
    return 3 * ((f + 255) & ~(size_t) 255);
}

}  // extern "C"
