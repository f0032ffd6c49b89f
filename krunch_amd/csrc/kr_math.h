// Deterministic float32 exp used by the head softmax.
//
// Cody-Waite reduction x = n*ln2 + r (ln2 split into a 15-bit high part and a
// low part), degree-7 Taylor polynomial of e^r in Horner form, scale by 2^n.
// Every step is one IEEE-rounded multiply or add (no fma), so the CPU oracle
// restated with numpy float32 arithmetic produces identical bits. Defined for
// x <= 0; inputs below -87 (or NaN / -inf) return 0 so the result is never
// subnormal.
#pragma once
#include "kr_common.h"

#define KR_EXP_LOG2E 0x1.715476p+0f
#define KR_EXP_LN2_HI 0x1.62e4p-1f
#define KR_EXP_LN2_LO 0x1.7f7d1cp-20f
#define KR_EXP_C7 0x1.a01a02p-13f
#define KR_EXP_C6 0x1.6c16c2p-10f
#define KR_EXP_C5 0x1.111112p-7f
#define KR_EXP_C4 0x1.555556p-5f
#define KR_EXP_C3 0x1.555556p-3f

__device__ __forceinline__ float kr_kexp(float x) {
    if (!(x >= -87.0f)) return 0.0f;
    const float n = __builtin_rintf(__fmul_rn(x, KR_EXP_LOG2E));
    const float r = __fsub_rn(__fsub_rn(x, __fmul_rn(n, KR_EXP_LN2_HI)),
                              __fmul_rn(n, KR_EXP_LN2_LO));
    float p = KR_EXP_C7;
    p = __fadd_rn(__fmul_rn(p, r), KR_EXP_C6);
    p = __fadd_rn(__fmul_rn(p, r), KR_EXP_C5);
    p = __fadd_rn(__fmul_rn(p, r), KR_EXP_C4);
    p = __fadd_rn(__fmul_rn(p, r), KR_EXP_C3);
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    const int e = (int)n + 127;
    return __fmul_rn(p, __int_as_float(e << 23));
}
