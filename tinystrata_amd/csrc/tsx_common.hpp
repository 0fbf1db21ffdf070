// tsx_common.hpp - host-side helpers shared by the entry points of libtsx_moe.so (argument checks, errors).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>

#include "tsx_moe.h"

namespace tsx {

// The calling thread's last failure message (tsx_moe_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
const char* error_cstr();

// TSX_OK, or the launch's hipError_t with the message recorded
int launch_status(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t) p % a) == 0; }

// The current device's address of the no-allocation decode layer's scratch array (tsx_layer.hip); nullptr, with the
// error recorded, when the runtime refuses the lookup.
void* noalloc_scratch_ptr(int* rc);

#define TSX_REQUIRE(cond, ...)                  \
    do {                                        \
        if (!(cond)) {                          \
            ::tsx::set_error(__VA_ARGS__);      \
            return TSX_ERR_ARG;                 \
        }                                       \
    } while (0)

}  // namespace tsx
