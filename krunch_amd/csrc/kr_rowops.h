// Row operations shared by the layer kernels and the fused decode kernel:
// LayerNorm of one row held by one wave, the token-shift mix, and row stores
// into row-major or fragment-packed [*, C] operands. Every caller compiles
// these same sources with the same flags, so a row gets the same bits from
// any kernel that runs it.
#pragma once
#include "kr_common.h"
#include "kr_gemm.h"
#include "kr_model.h"
#include "kr_wave.h"

namespace {

constexpr float kLnEps = 1e-5f;

// ---------------------------------------------------------------------------
// LayerNorm over one row held by one wave: lane l owns the 4-element groups
// at columns 256*i + 4*l. Sums use a fixed lane order then an xor butterfly,
// so every lane ends with the same value and the result is row-local.
// ---------------------------------------------------------------------------
template <int G>   // G = C / 256 groups of 4 per lane
struct RowF {
    float v[G][4];
};

template <int G>
__device__ __forceinline__ void load_row(const kr_half* __restrict__ p, int lane, RowF<G>& r) {
    #pragma unroll
    for (int i = 0; i < G; i++) {
        const kr_half4 h = *reinterpret_cast<const kr_half4*>(p + 256 * i + 4 * lane);
        #pragma unroll
        for (int q = 0; q < 4; q++) r.v[i][q] = (float)h[q];
    }
}

__device__ __forceinline__ float wave_sum(float s) {
    return kr_wave_reduce(s, [](float a, float b) { return a + b; });
}

// Per-lane copies of a [C] fp16 coefficient vector (the lane's 4-column groups).
template <int G>
struct CoefH {
    kr_half4 v[G];
};

template <int G>
__device__ __forceinline__ void load_coef(const kr_half* __restrict__ p, int lane, CoefH<G>& c) {
    #pragma unroll
    for (int i = 0; i < G; i++) c.v[i] = *reinterpret_cast<const kr_half4*>(p + 256 * i + 4 * lane);
}

template <int G>
__device__ __forceinline__ void store_coef(kr_half* __restrict__ p, int lane, const CoefH<G>& c) {
    #pragma unroll
    for (int i = 0; i < G; i++) *reinterpret_cast<kr_half4*>(p + 256 * i + 4 * lane) = c.v[i];
}

template <int G>
__device__ __forceinline__ void to_float(const CoefH<G>& h, RowF<G>& r) {
    #pragma unroll
    for (int i = 0; i < G; i++)
        #pragma unroll
        for (int q = 0; q < 4; q++) r.v[i][q] = (float)h.v[i][q];
}

template <int G>
__device__ __forceinline__ void layer_norm_row(RowF<G>& r, const CoefH<G>& w, const CoefH<G>& b) {
    constexpr float invC = 1.0f / (float)(256 * G);
    float s = 0.0f;
    #pragma unroll
    for (int i = 0; i < G; i++)
        #pragma unroll
        for (int q = 0; q < 4; q++) s = s + r.v[i][q];
    const float mean = wave_sum(s) * invC;
    float ss = 0.0f;
    #pragma unroll
    for (int i = 0; i < G; i++)
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float d = r.v[i][q] - mean;
            ss = ss + d * d;
        }
    const float rstd = 1.0f / sqrtf(wave_sum(ss) * invC + kLnEps);
    #pragma unroll
    for (int i = 0; i < G; i++) {
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float y = (r.v[i][q] - mean) * rstd * (float)w.v[i][q] + (float)b.v[i][q];
            r.v[i][q] = (float)kr_f16(y);   // activations are fp16
        }
    }
}

template <int G>
__device__ __forceinline__ void store_row(kr_half* __restrict__ p, int lane, const RowF<G>& r) {
    #pragma unroll
    for (int i = 0; i < G; i++) {
        kr_half4 h;
        #pragma unroll
        for (int q = 0; q < 4; q++) h[q] = kr_f16(r.v[i][q]);
        *reinterpret_cast<kr_half4*>(p + 256 * i + 4 * lane) = h;
    }
}

// kr_frag_index(row, col, C) as a row part (wave-uniform: the address stays
// in scalar registers) plus a 32-bit column part.
__device__ __forceinline__ size_t frag_row_base(size_t row, int C) {
    return (row >> 4) * (size_t)(C >> 5) * 512 + (row & 15) * 8;
}
__device__ __forceinline__ unsigned frag_col_off(int col) {
    return (unsigned)(col >> 5) * 512u + (unsigned)((col & 31) >> 3) * 128u + (unsigned)(col & 7);
}

// Row `row` of a fragment-packed [*, C] operand (kr_frag_index): the lane's
// 4-column groups are 4 consecutive halves there too.
template <int G>
__device__ __forceinline__ void store_row_frag(kr_half* __restrict__ out, size_t row, int lane,
                                               const RowF<G>& r) {
    constexpr int C = 256 * G;
    #pragma unroll
    for (int i = 0; i < G; i++) {
        kr_half4 h;
        #pragma unroll
        for (int q = 0; q < 4; q++) h[q] = kr_f16(r.v[i][q]);
        *reinterpret_cast<kr_half4*>(out + frag_row_base(row, C) + frag_col_off(256 * i + 4 * lane)) = h;
    }
}

// mix = fp16(xx * tm + sx * (1 - tm))   (premix_kernels.cu:19-54 semantics),
// stored into row `row` of a row-major or fragment-packed [*, C] operand.
template <int G>
__device__ __forceinline__ void store_mix(kr_half* __restrict__ out, size_t row, bool frag,
                                          const CoefH<G>& tm, int lane,
                                          const RowF<G>& cur, const RowF<G>& prev) {
    constexpr int C = 256 * G;
    #pragma unroll
    for (int i = 0; i < G; i++) {
        const kr_half4 t = tm.v[i];
        kr_half4 h;
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float m = (float)t[q];
            h[q] = kr_f16(cur.v[i][q] * m + prev.v[i][q] * (1.0f - m));
        }
        const int col = 256 * i + 4 * lane;
        kr_half* base = out + (frag ? frag_row_base(row, C) : row * C);
        *reinterpret_cast<kr_half4*>(base + (frag ? frag_col_off(col) : (unsigned)col)) = h;
    }
}

// w8a8: the fp16 mix row quantised per row by the rule of kr_quantize_rows
// (kr_gemm.h), row-major or fragment-packed for the small-M int8 GEMM. The
// mixes are held as fp16 while the row maximum is reduced (half the
// registers of fp32 copies; LN-mix occupancy matters, see ln_mix_kernel).
template <int G>
__device__ __forceinline__ void store_mix_q8(int8_t* __restrict__ out, float* __restrict__ scales,
                                             size_t row, bool frag, const CoefH<G>& tm, int lane,
                                             const RowF<G>& cur, const RowF<G>& prev) {
    constexpr int C = 256 * G;
    kr_half4 h[G];
    float amax = 0.0f;
    #pragma unroll
    for (int i = 0; i < G; i++)
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float m = (float)tm.v[i][q];
            h[i][q] = kr_f16(cur.v[i][q] * m + prev.v[i][q] * (1.0f - m));
            amax = fmaxf(amax, fabsf((float)h[i][q]));
        }
    amax = kr_wave_reduce(amax, [](float a, float b) { return fmaxf(a, b); });
    const float inv = kr_q8_inv(amax);
    #pragma unroll
    for (int i = 0; i < G; i++) {
        const uint32_t w = kr_q8_pack4((float)h[i][0], (float)h[i][1], (float)h[i][2],
                                       (float)h[i][3], inv);
        const int col = 256 * i + 4 * lane;
        // kr_frag_index_i8 (col even): twice the 16-bit view's index
        int8_t* base = out + (frag ? 2 * frag_row_base(row, C / 2) : row * C);
        *reinterpret_cast<uint32_t*>(base + (frag ? 2 * frag_col_off(col / 2) : (unsigned)col)) = w;
    }
    if (lane == 0) scales[row] = kr_q8_scale(amax);
}

// The loads only need to reach L2: their values are folded into one register
// the compiler must keep, and nothing is stored. The 16-byte chunks XCD x
// stages (all regions, groups x, x + 8, ...) are numbered in one sequence and
// dealt over the XCD's staging threads, eight loads in flight per thread, so a
// thread waits on memory about twice rather than once per group. The region
// tables are read with constant indices only (kernel arguments in scalar
// registers) and a chunk's region picked by selects: an array element at a
// run-time index would be fetched from argument memory before every load,
// and each of the eight loads would wait for the one before.
// p: the staging block (p % 8 = the XCD it runs on); tid: its thread, 0..255.
__device__ void prefetch_panels(const PrefetchSet& pf, int p, int tid) {
    const int x = p & 7, nr = pf.blocks >> 3;
    const int t = (p >> 3) * 256 + tid, T = nr * 256;
    const char* base[4];
    long long gb[4];
    int per[4], cum[5];
    cum[0] = 0;
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        base[i] = pf.base[i];
        gb[i] = pf.group_bytes[i];
        const int groups_x = i < pf.n ? (pf.n_groups[i] - x + 7) / 8 : 0;   // groups x, x+8, ...
        per[i] = i < pf.n ? (int)(gb[i] >> 4) : 1;                         // chunks per group
        cum[i + 1] = cum[i] + groups_x * per[i];
    }
    unsigned acc = 0;
    for (int c0 = t; c0 < cum[4]; c0 += 8 * T) {
        uint4 v[8];
        #pragma unroll
        for (int u = 0; u < 8; u++) {
            const int c = c0 + u * T;
            v[u] = make_uint4(0, 0, 0, 0);
            if (c < cum[4]) {
                // the region holding chunk c: the last one starting at or before it
                const bool r1 = c >= cum[1], r2 = c >= cum[2], r3 = c >= cum[3];
                const char* b = r3 ? base[3] : (r2 ? base[2] : (r1 ? base[1] : base[0]));
                const long long g = r3 ? gb[3] : (r2 ? gb[2] : (r1 ? gb[1] : gb[0]));
                const int pr = r3 ? per[3] : (r2 ? per[2] : (r1 ? per[1] : per[0]));
                const int cs = r3 ? cum[3] : (r2 ? cum[2] : (r1 ? cum[1] : cum[0]));
                const int r = c - cs, gi = r / pr, o = r - gi * pr;
                v[u] = reinterpret_cast<const uint4*>(b + (long long)(x + 8 * gi) * g)[o];
            }
        }
        #pragma unroll
        for (int u = 0; u < 8; u++) acc ^= v[u].x;
    }
    asm volatile("" :: "v"(acc));
}

// Layer 0's LN1-mix of decoded token id for stream b (kr_embed_mix, kr_model.h).
template <int G>
__device__ __forceinline__ void embed_mix_row(const kr_embed_mix& e, size_t b, int id, int lane) {
    constexpr int C = 256 * G;
    id = id < 0 ? 0 : (id >= e.V ? e.V - 1 : id);
    CoefH<G> w, bias, tm[3], prev_h, cur_h;
    load_coef<G>(e.ln_w, lane, w);
    load_coef<G>(e.ln_b, lane, bias);
    #pragma unroll
    for (int m = 0; m < 3; m++) load_coef<G>(e.tm[m], lane, tm[m]);
    load_coef<G>(e.src + b * C, lane, prev_h);
    load_coef<G>(e.emb + (size_t)id * C, lane, cur_h);
    store_coef<G>(e.xw + b * C, lane, cur_h);
    store_coef<G>(e.state + b * C, lane, prev_h);
    RowF<G> prev, cur;
    to_float<G>(prev_h, prev);
    to_float<G>(cur_h, cur);
    layer_norm_row<G>(cur, w, bias);
    #pragma unroll
    for (int m = 0; m < 3; m++) {
        if (e.q[0]) store_mix_q8<G>(e.q[m], e.qs[m], b, true, tm[m], lane, cur, prev);
        else store_mix<G>(e.out[m], b, true, tm[m], lane, cur, prev);
    }
    store_row<G>(e.pend + b * C, lane, cur);
}

// embed_mix_row for C = 256 G, G in 1..4 (all 64 lanes of the wave, id
// wave-uniform).
__device__ __forceinline__ void embed_mix(const kr_embed_mix& e, size_t b, int id, int lane) {
    switch (e.C >> 8) {
        case 1: embed_mix_row<1>(e, b, id, lane); break;
        case 2: embed_mix_row<2>(e, b, id, lane); break;
        case 3: embed_mix_row<3>(e, b, id, lane); break;
        case 4: embed_mix_row<4>(e, b, id, lane); break;
        default: break;
    }
}

}  // namespace
