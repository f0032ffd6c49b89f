// Cross-lane exchanges inside one 64-lane wave, as VALU operations.
//
// kr_xor<O>(v) returns the value of v in lane (lane ^ O), O in {1, 2, 4, 8,
// 16, 32}: the pairing of a __shfl_xor butterfly, but through DPP (O <= 8:
// quad permutes, the half-row mirror and a row rotate) and the gfx950
// permlane swaps (O = 16, 32) instead of an LDS-path ds_bpermute. A reduction
// that combines v with kr_xor<O>(v) for O = 32, 16, ..., 1 therefore adds
// exactly the pairs, in exactly the order, of the ds_bpermute butterfly.
// Lane layouts checked on MI355X against lane ^ O for every lane. All 64
// lanes must be active (callers reduce under wave-uniform control flow).
#pragma once
#include <hip/hip_runtime.h>

template <int O>
__device__ __forceinline__ int kr_xor_i(int v) {
    if constexpr (O == 1) {
        return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    } else if constexpr (O == 2) {
        return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    } else if constexpr (O == 4) {
        // quad_perm [3,2,1,0] (lane ^ 3), then row_half_mirror (lane ^ 7 within 8)
        const int t = __builtin_amdgcn_update_dpp(0, v, 0x1B, 0xF, 0xF, false);
        return __builtin_amdgcn_update_dpp(0, t, 0x141, 0xF, 0xF, false);
    } else if constexpr (O == 8) {
        return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (O == 16) {
        // swap odd rows of the first copy with even rows of the second
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        static_assert(O == 32, "kr_xor: O must be a power of two <= 32");
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((threadIdx.x & 32) ? r[0] : r[1]);
    }
}

template <int O>
__device__ __forceinline__ float kr_xor(float v) {
    return __builtin_bit_cast(float, kr_xor_i<O>(__builtin_bit_cast(int, v)));
}
template <int O>
__device__ __forceinline__ int kr_xor(int v) { return kr_xor_i<O>(v); }
template <int O>
__device__ __forceinline__ unsigned kr_xor(unsigned v) { return (unsigned)kr_xor_i<O>((int)v); }

// Butterfly over all 64 lanes, strides 32, 16, ..., 1; every lane ends with
// op applied in the same tree (op commutative).
template <typename T, typename Op>
__device__ __forceinline__ T kr_wave_reduce(T v, Op op) {
    v = op(v, kr_xor<32>(v));
    v = op(v, kr_xor<16>(v));
    v = op(v, kr_xor<8>(v));
    v = op(v, kr_xor<4>(v));
    v = op(v, kr_xor<2>(v));
    v = op(v, kr_xor<1>(v));
    return v;
}
