// Deterministic float32 exp used by the head softmax and, in the w8a8 codec,
// by the sigmoid and the WKV update.
//
// Cody-Waite reduction x = n*ln2 + r (ln2 split into a 15-bit high part and a
// low part, each step a fused multiply-add), then e^r by a degree-6 polynomial
// in Horner form by fused multiply-adds, scale by 2^n (exact). The polynomial
// is a minimax fit of e^r on [-ln2/2, ln2/2] for relative error, its
// coefficients rounded to float32 one at a time (lowest order first) with the
// higher ones refitted; c0 = c1 = 1, so kexp(0) = 1 exactly. In exact
// arithmetic it is within 0.053 ulp of e^r (the degree-7 Taylor polynomial,
// one fused multiply-add more, is within 0.118 ulp). Every step is one
// IEEE-rounded operation, so the CPU oracle's C restatement (fmaf, correctly
// rounded like v_fma_f32) produces identical bits. Defined for x <= 0; inputs
// below -87 (or NaN / -inf) return 0 so the result is never subnormal.
#pragma once
#include "kr_common.h"

#define KR_EXP_LOG2E 0x1.715476p+0f
#define KR_EXP_LN2_HI 0x1.62e4p-1f
#define KR_EXP_LN2_LO 0x1.7f7d1cp-20f
#define KR_EXP_C6 0x1.6a3d04p-10f
#define KR_EXP_C5 0x1.123856p-7f
#define KR_EXP_C4 0x1.5558bep-5f
#define KR_EXP_C3 0x1.555494p-3f
#define KR_EXP_C2 0x1.fffffcp-2f

__device__ __forceinline__ float kr_kexp(float x) {
    // Branch-free: the arithmetic runs on a clamped copy (NaN and -inf become
    // -87.5, so every intermediate is finite) and the result is selected.
    const float xc = fmaxf(x, -87.5f);
    const float n = __builtin_rintf(__fmul_rn(xc, KR_EXP_LOG2E));
    float r = __builtin_fmaf(-n, KR_EXP_LN2_HI, xc);
    r = __builtin_fmaf(-n, KR_EXP_LN2_LO, r);
    float p = KR_EXP_C6;
    p = __builtin_fmaf(p, r, KR_EXP_C5);
    p = __builtin_fmaf(p, r, KR_EXP_C4);
    p = __builtin_fmaf(p, r, KR_EXP_C3);
    p = __builtin_fmaf(p, r, KR_EXP_C2);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float y = __builtin_ldexpf(p, (int)n);
    return x >= -87.0f ? y : 0.0f;
}

// Logistic function from kr_kexp (its argument -|x| is never positive):
// 1 / (1 + e) for x >= 0, e / (1 + e) for x < 0, e = exp(-|x|). Used by the
// w8a8 codec, whose every activation feeds a rounding to int8: with a
// restatable exp the CPU oracle reproduces its activations bit for bit.
__device__ __forceinline__ float kr_sigmoid_k(float x) {
    const float e = kr_kexp(-fabsf(x));
    const float d = 1.0f + e;
    return x >= 0.0f ? 1.0f / d : e / d;
}

// DET selects kr_kexp / kr_sigmoid_k (the w8a8 codec) over the hardware
// exp (the fp16 codec).
template <bool DET>
__device__ __forceinline__ float kr_exp_t(float x) {
    if constexpr (DET) return kr_kexp(x);
    else return __expf(x);
}
template <bool DET>
__device__ __forceinline__ float kr_sigmoid_t(float x) {
    if constexpr (DET) return kr_sigmoid_k(x);
    else return kr_sigmoid(x);
}
