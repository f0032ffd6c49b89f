// Device helpers shared by the GEMM kernels of kr_gemm.hip and kr_wide.hip:
// the fused epilogues (one element, or 4 consecutive columns of a row), the
// swizzled LDS position of the persistent kernels' stages, and the int8 view
// of an operand fragment.
#pragma once
#include "kr_gemm.h"
#include "kr_math.h"

namespace {

__device__ __forceinline__ kr_int4 as_i4(kr_half8 v) { return __builtin_bit_cast(kr_int4, v); }

// Stage layout of the persistent kernels (16-byte units): row r, 8-wide k
// chunk kc at 64 (r / 8) + 8 (r % 8) + (kc ^ ((r / 2) % 8)).
__device__ __forceinline__ int big_pos(int r, int kc) {
    return 64 * (r >> 3) + 8 * (r & 7) + (kc ^ ((r >> 1) & 7));
}

// DET: the w8a8 codec's sigmoid (kr_sigmoid_k); int8 kernels pass I8.
template <int EP, bool DET = false>
__device__ __forceinline__ void store_one(const kr_gemm_args& g, int m, int n, float acc) {
    const size_t o = (size_t)m * (size_t)g.ldo + (size_t)n;
    if constexpr (EP == KR_EP_F32) {
        reinterpret_cast<float*>(g.out)[o] = acc;
    } else {
        const float h = (float)kr_f16(acc);
        float y;
        if constexpr (EP == KR_EP_F16) y = h;
        else if constexpr (EP == KR_EP_SIGMOID) y = kr_sigmoid_t<DET>(h);
        else if constexpr (EP == KR_EP_RELUSQ) { const float r = h > 0.0f ? h : 0.0f; y = r * r; }
        else if constexpr (EP == KR_EP_RESID) y = (float)g.res[o] + h;
        else {
            const float gh = (float)kr_f16((float)g.gate[o] * h);
            y = (float)g.res[o] + gh;
        }
        reinterpret_cast<kr_half*>(g.out)[o] = kr_f16(y);
    }
}

// Epilogue of 4 consecutive columns n..n+3 of row m (vec: aligned vector
// access allowed and all 4 columns < N).
template <int EP, bool DET>
__device__ __forceinline__ void store_row4(const kr_gemm_args& g, int m, int n, kr_float4 acc,
                                           bool vec) {
    if (!vec) {
        #pragma unroll
        for (int r = 0; r < 4; r++)
            if (n + r < g.N) store_one<EP, DET>(g, m, n + r, acc[r]);
        return;
    }
    const size_t o = (size_t)m * (size_t)g.ldo + (size_t)n;
    if constexpr (EP == KR_EP_F32) {
        *reinterpret_cast<kr_float4*>(reinterpret_cast<float*>(g.out) + o) = acc;
    } else {
        kr_half4 rv = kr_half4{0, 0, 0, 0}, gv = kr_half4{0, 0, 0, 0};
        if constexpr (EP == KR_EP_RESID || EP == KR_EP_GATED) rv = *reinterpret_cast<const kr_half4*>(g.res + o);
        if constexpr (EP == KR_EP_GATED) gv = *reinterpret_cast<const kr_half4*>(g.gate + o);
        kr_half4 h;
        #pragma unroll
        for (int r = 0; r < 4; r++) {
            const float x = (float)kr_f16(acc[r]);
            float y;
            if constexpr (EP == KR_EP_F16) y = x;
            else if constexpr (EP == KR_EP_SIGMOID) y = kr_sigmoid_t<DET>(x);
            else if constexpr (EP == KR_EP_RELUSQ) { const float rr = x > 0.0f ? x : 0.0f; y = rr * rr; }
            else if constexpr (EP == KR_EP_RESID) y = (float)rv[r] + x;
            else y = (float)rv[r] + (float)kr_f16((float)gv[r] * x);
            h[r] = kr_f16(y);
        }
        *reinterpret_cast<kr_half4*>(reinterpret_cast<kr_half*>(g.out) + o) = h;
    }
}

}  // namespace
