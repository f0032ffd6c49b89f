// Shared definitions for the krunch MI355X (gfx950) library.
//
// All device code in this library is compiled with -ffp-contract=off: every
// float multiply and add is rounded on its own, so the same source gives the
// same bits in every kernel that inlines it (packed compress and stepped
// decompress must agree bit for bit) and on the CPU oracle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef _Float16 kr_half;
typedef _Float16 kr_half4 __attribute__((ext_vector_type(4)));
typedef _Float16 kr_half8 __attribute__((ext_vector_type(8)));
typedef float kr_float4 __attribute__((ext_vector_type(4)));
typedef int kr_int4 __attribute__((ext_vector_type(4)));

// fp32 -> fp16 with the value first materialised in fp32. Without the empty
// asm the AMDGPU backend folds fp16(a * b) into one v_fma_mixlo_f16 (a single
// rounding straight to fp16) even under -ffp-contract=off, and whether it
// does depends on the surrounding code: two kernels computing the same
// expression could then round differently. Every fp16 store of a computed
// value goes through here, so every kernel rounds to fp32, then to fp16.
__device__ __forceinline__ _Float16 kr_f16(float v) {
    __asm__ volatile("" : "+v"(v));
    return (_Float16)v;
}

// ---------------------------------------------------------------------------
// Range-coder constants (32-bit state; the coding spec is a 32-bit range coder
// with E1/E2/E3 renormalisation, krunch_ac/cpu_reference.py:28-33 and
// krunch_ac/cuda/range_coder.cuh:7-20).
// ---------------------------------------------------------------------------
#define KR_RC_HALF 0x80000000u
#define KR_RC_QUARTER 0x40000000u
#define KR_RC_3QUARTER 0xC0000000u
#define KR_CDF_PRECISION_DEFAULT 24

// Per-stream coder state, 16 bytes, same field order as the reference
// (range_coder.cuh:24-40): encoder {low, high, pending, bit_offset},
// decoder {low, high, value, bit_offset}.
struct kr_rc_state {
    uint32_t low;
    uint32_t high;
    uint32_t pending_or_value;
    uint32_t bit_offset;
};

// ---------------------------------------------------------------------------
// Error reporting for the C ABI: every entry point returns 0 on success or a
// negative code, and leaves a message retrievable with kr_last_error().
// ---------------------------------------------------------------------------
enum {
    KR_OK = 0,
    KR_EINVAL = -1,
    KR_EHIP = -2,
    KR_ENOMEM = -3,
    KR_EUNSUPPORTED = -4,
};

int kr_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define KR_REQUIRE(cond, ...)                       \
    do {                                            \
        if (!(cond)) return kr_fail(KR_EINVAL, __VA_ARGS__); \
    } while (0)

#define KR_HIP(call)                                                              \
    do {                                                                          \
        hipError_t kr_e_ = (call);                                                \
        if (kr_e_ != hipSuccess)                                                  \
            return kr_fail(KR_EHIP, "%s failed: %s (%s:%d)", #call,               \
                           hipGetErrorString(kr_e_), __FILE__, __LINE__);         \
    } while (0)

// Launch-error check after a <<<>>> launch.
#define KR_LAUNCHED() KR_HIP(hipGetLastError())

static inline hipStream_t kr_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float kr_h2f(kr_half h) { return (float)h; }

// Logistic function, one definition for every kernel that needs it.
__device__ __forceinline__ float kr_sigmoid(float x) {
    return 1.0f / (1.0f + __expf(-x));
}
