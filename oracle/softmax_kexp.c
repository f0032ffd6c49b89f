/* Oracle (TEST INFRASTRUCTURE ONLY): the deterministic float32 exp of the
 * build's head softmax, restated in C because it is built on fused
 * multiply-adds: C's fmaf is correctly rounded (one rounding of x*y + z),
 * as the GPU's v_fma_f32 is, while numpy has no float32 FMA.
 *
 *   xc = max(x, -87.5)                 (NaN and -inf -> -87.5)
 *   n  = rint(xc * log2(e))            (round half to even)
 *   r  = fma(-n, ln2_lo, fma(-n, ln2_hi, xc))
 *   p  = Horner by fma of a degree-6 polynomial of e^r: a minimax fit on
 *        [-ln2/2, ln2/2] for relative error (c0 = c1 = 1; c2..c6 rounded to
 *        float32 one at a time, lowest order first, the rest refitted)
 *   e  = ldexp(p, n)                   (exact: the result is normal)
 *   kexp(x) = e if x >= -87 else 0
 *
 * ln2_hi has 15 significant bits, so n * ln2_hi is exact and the first fma
 * rounds only the (exact, by Sterbenz) difference.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static float f32_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static float kexp1(float x) {
    const float log2e = f32_bits(0x3FB8AA3Bu);
    const float ln2_hi = f32_bits(0x3F317200u);
    const float ln2_lo = f32_bits(0x35BFBE8Eu);
    const float c6 = f32_bits(0x3AB51E82u), c5 = f32_bits(0x3C091C2Bu),
                c4 = f32_bits(0x3D2AAC5Fu), c3 = f32_bits(0x3E2AAA4Au),
                c2 = f32_bits(0x3EFFFFFEu);
    const float xc = fmaxf(x, -87.5f);
    const float n = rintf(xc * log2e);
    float r = fmaf(-n, ln2_hi, xc);
    r = fmaf(-n, ln2_lo, r);
    float p = c6;
    p = fmaf(p, r, c5);
    p = fmaf(p, r, c4);
    p = fmaf(p, r, c3);
    p = fmaf(p, r, c2);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const float e = ldexpf(p, (int)n);
    return x >= -87.0f ? e : 0.0f;
}

void orc_kexp(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = kexp1(x[i]);
}
