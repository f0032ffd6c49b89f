// RWKV-4 layer kernels and the host driver of the packed / stepped forward.
//
// Numerics follow the production op order of the reference layer
// (krunch_ac/cuda/layer_cpp.cpp:456-637) with fp16 activations between
// stages:
//   xx = LN1(x); kx,vx,rx = mix(xx, shifted xx)            [ln_mix_kernel]
//   k = kx@Kw, v = vx@Vw (fp32), r = sigmoid(fp16(rx@Rw))   [3 GEMMs]
//   y = WKV(k, v); ry = fp16(r * fp16(y))                   [wkv_kernel]
//   x = x + fp16(ry@Ow)                                     [GEMM, RESID]
//   xx2 = LN2(x); fkx, frx = mix(xx2, shifted xx2)          [ln_mix_kernel]
//   rf = sigmoid(fp16(frx@fRw)); kf = relu(fp16(fkx@fKw))^2 [2 GEMMs]
//   x = x + fp16(rf * fp16(kf@fVw))                         [GEMM, GATED]
// Packed (T tokens per stream) and stepped (T = 1) calls run the same
// kernels, so every row is computed by the same instruction sequence.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "kr_gemm.h"
#include "kr_math.h"
#include "kr_model.h"
#include "kr_rowops.h"
#include "kr_wave.h"

namespace {

struct LnMixArgs {
    const kr_half* x;          // [B*T, C]
    const kr_half* ln_w;
    const kr_half* ln_b;
    const kr_half* tm[3];      // NMIX coefficient vectors
    kr_half* out[3];           // NMIX outputs [B*T, C]
    kr_half* state;            // [B, C] shifted-in row for t = 0; rewritten with LN(x[T-1])
    int B, T, run;             // rows per wave
    int frag;                  // mix outputs fragment-packed (small-M GEMM operands)
    int8_t* q[3];              // w8a8: NMIX int8 outputs instead of out[] (per-row quantised)
    float* qs[3];              // w8a8: their per-row scales
    // Embedding gather fused in (layer 0): row r of x is emb[ids[r]] (ids
    // clamped into [0, V), as embed_kernel does), read from the table and
    // also written to xw, the residual stream the later products add onto.
    const int32_t* ids;
    const kr_half* emb;
    int V;
    kr_half* xw;
    PrefetchSet pf;            // optional L2 staging of the next products' weights
    int ln_blocks;             // workgroups doing LN-mix rows (set by the launcher)
    int one_row;               // one row per workgroup (wave 0; set by the launcher)
};

// One wave per run of `run` consecutive tokens of one stream. The wave that
// owns t = 0 reads the carried state first and rewrites it last (with the
// LayerNorm of row T-1), so no other wave touches the state. Every
// coefficient and the first rows are loaded before any store, so a T = 1
// row costs one memory round trip.
// NMIX == 0: plain LayerNorm into out[0] (ln_out before the head).
// Q8: the w8a8 form (mixes quantised into a.q[]), its own instantiation.
// At least 3 waves per SIMD (<= 168 registers) for C <= 768: the L2 staging
// workgroups this kernel also runs need the occupancy. Measured on MI355X
// (fp16 decode KB/s, one box, A/B twice): fp16 and int8 forms in one kernel
// 1,737 (LN2 at 207 registers, 2 waves); split, no bound 1,818 (LN1 at 186);
// split, 3 waves 1,874 (LN1 spilling 60 bytes); 4 waves 1,800 (116-byte
// spills). With the row index wave-uniform and the fragment index split into
// a uniform row part and a 32-bit column part (addresses in scalar
// registers), every form fits 3 waves without spilling (fp16 156 / 130,
// int8 168 / 148 registers): w8a8 decode 1,727 -> 1,886.
template <int G, int NMIX, bool Q8>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G <= 3 ? 3 : 1)))
ln_mix_kernel(LnMixArgs a) {
    constexpr int C = 256 * G;
    constexpr int NM = NMIX > 0 ? NMIX : 1;
    if ((int)blockIdx.x >= a.ln_blocks) {   // staging workgroups (uniform per workgroup)
        prefetch_panels(a.pf, (int)blockIdx.x - a.ln_blocks, (int)threadIdx.x);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int runs = (a.T + a.run - 1) / a.run;
    int gw = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (a.one_row) gw = threadIdx.x < 64 ? (int)blockIdx.x : a.B * runs;
    // wave-uniform: every row pointer then lives in scalar registers
    gw = __builtin_amdgcn_readfirstlane(gw);
    if (gw >= a.B * runs) return;
    const int b = gw / runs, t0 = (gw % runs) * a.run;
    const int t1 = min(a.T, t0 + a.run);
    const size_t row0 = (size_t)b * a.T;

    CoefH<G> w, bias, tm[NM];
    load_coef<G>(a.ln_w, lane, w);
    load_coef<G>(a.ln_b, lane, bias);
    if constexpr (NMIX > 0) {
        #pragma unroll
        for (int m = 0; m < NMIX; m++) load_coef<G>(a.tm[m], lane, tm[m]);
    }
    // source of row r of x: the residual stream, or the embedding table
    auto xrow = [&](size_t r) -> const kr_half* {
        if (!a.ids) return a.x + r * C;
        int id = a.ids[r];
        id = id < 0 ? 0 : (id >= a.V ? a.V - 1 : id);
        return a.emb + (size_t)id * C;
    };
    // the first row and the row shifted in ahead of it, both in flight at once
    CoefH<G> prev_h, first_h;
    if constexpr (NMIX > 0)
        load_coef<G>(t0 == 0 ? a.state + (size_t)b * C : xrow(row0 + t0 - 1), lane, prev_h);
    load_coef<G>(xrow(row0 + t0), lane, first_h);
    RowF<G> prev, cur;
    if constexpr (NMIX > 0) {
        to_float<G>(prev_h, prev);
        if (t0 != 0) layer_norm_row<G>(prev, w, bias);
    }
    CoefH<G> next_h;
    for (int t = t0; t < t1; t++) {
        if constexpr (!Q8) {
            // the next row in flight while this one is computed (runs of
            // rows; the int8 form has no registers to spare for it)
            if (t > t0) first_h = next_h;
            if (t + 1 < t1) load_coef<G>(xrow(row0 + t + 1), lane, next_h);
        } else {
            if (t != t0) load_coef<G>(xrow(row0 + t), lane, first_h);
        }
        if (a.ids) store_coef<G>(a.xw + (row0 + t) * C, lane, first_h);
        to_float<G>(first_h, cur);
        layer_norm_row<G>(cur, w, bias);
        if constexpr (NMIX == 0) {
            if (a.frag) store_row_frag<G>(a.out[0], row0 + t, lane, cur);
            else store_row<G>(a.out[0] + (row0 + t) * C, lane, cur);
        } else {
            #pragma unroll
            for (int m = 0; m < NMIX; m++) {
                if constexpr (Q8) store_mix_q8<G>(a.q[m], a.qs[m], row0 + t, a.frag != 0, tm[m], lane, cur, prev);
                else store_mix<G>(a.out[m], row0 + t, a.frag != 0, tm[m], lane, cur, prev);
            }
            prev = cur;
        }
    }
    if constexpr (NMIX > 0) {
        if (t0 == 0) {
            if (t1 < a.T) {
                load_row<G>(xrow(row0 + a.T - 1), lane, cur);
                layer_norm_row<G>(cur, w, bias);
            }
            store_row<G>(a.state + (size_t)b * C, lane, cur);
        }
    }
}

// ---------------------------------------------------------------------------
// WKV recurrence (wkv_kernel.cu:52-73 semantics), one lane per (stream,
// channel), sequential over T; fused with the receptance product:
// ry = fp16(r * fp16(y)), written row-major or fragment-packed (ry_frag) for
// the output projection. State aa, bb, pp is read once and written once.
// ---------------------------------------------------------------------------
constexpr int kWkvChunk = 16;

struct WkvState {
    float a, b, p;
};

// One token of the recurrence; returns ry.
// DET: exps by kr_kexp and an IEEE division (the w8a8 codec, which the oracle
// restates bit for bit; every exp argument here is <= 0). Otherwise (the fp16
// codec) the hardware exp and the quotient as numerator times the hardware
// reciprocal (~1 ulp; y is rounded to fp16 next): the packed and stepped
// paths both run this function, so their bits agree.
template <bool DET>
__device__ __forceinline__ kr_half wkv_token(WkvState& st, float w, float u, float kk, float vv,
                                             float rr) {
    const float ww = u + kk;
    const float p1 = fmaxf(st.p, ww);
    const float e1 = kr_exp_t<DET>(st.p - p1), e2 = kr_exp_t<DET>(ww - p1);
    const float num = e1 * st.a + e2 * vv, den = e1 * st.b + e2;   // den >= min(1, bb) > 0
    float y;
    if constexpr (DET) y = num / den;
    else y = num * __builtin_amdgcn_rcpf(den);
    const kr_half ry = kr_f16(rr * (float)kr_f16(y));
    const float ww2 = w + st.p;
    const float p2 = fmaxf(ww2, kk);
    const float f1 = kr_exp_t<DET>(ww2 - p2), f2 = kr_exp_t<DET>(kk - p2);
    st.a = f1 * st.a + f2 * vv;
    st.b = f1 * st.b + f2;
    st.p = p2;
    return ry;
}

template <bool DET>
__global__ void __launch_bounds__(256) wkv_kernel(const float* __restrict__ k,
                                                  const float* __restrict__ v,
                                                  const kr_half* __restrict__ r,
                                                  const float* __restrict__ decay,
                                                  const float* __restrict__ first,
                                                  float* __restrict__ aa, float* __restrict__ bb,
                                                  float* __restrict__ pp, kr_half* __restrict__ ry,
                                                  int B, int T, int C, int ry_frag) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= C || b >= B) return;
    const size_t s = (size_t)b * C + c;
    const size_t base = (size_t)b * T * C + c;
    const float w = decay[c], u = first[c];
    WkvState st{aa[s], bb[s], pp[s]};
    auto ry_at = [&](int t) -> size_t {
        return ry_frag ? kr_frag_index((long long)b * T + t, c, C) : base + (size_t)t * C;
    };
    // A chunk's loads are unconditional (tokens past T re-read token T-1) and
    // r stays fp16 until its token is computed, so all 3 x kWkvChunk loads are
    // in flight at once. A load under `t < T` with its conversion beside it
    // makes the compiler wait for each token's loads in turn (one memory
    // latency per token).
    for (int t0 = 0; t0 < T; t0 += kWkvChunk) {
        float kk[kWkvChunk], vv[kWkvChunk];
        kr_half rh[kWkvChunk];
        #pragma unroll
        for (int q = 0; q < kWkvChunk; q++) {
            const size_t i = base + (size_t)min(t0 + q, T - 1) * C;
            kk[q] = k[i];
            vv[q] = v[i];
            rh[q] = r[i];
        }
        #pragma unroll
        for (int q = 0; q < kWkvChunk; q++)
            if (t0 + q < T) ry[ry_at(t0 + q)] = wkv_token<DET>(st, w, u, kk[q], vv[q], (float)rh[q]);
    }
    aa[s] = st.a;
    bb[s] = st.b;
    pp[s] = st.p;
}

// ---------------------------------------------------------------------------
// Stepped K, V, R products fused with the WKV update (T = 1 rows): the three
// small-M products and wkv_kernel in one launch, with the arithmetic of the
// unfused sequence (split-K slices folded in order; k, v fp32; r =
// fp16(sigmoid(fp16(acc))); wkv_token), so the bits are those of the packed
// path.
//
// One workgroup per (16*TM rows) x (16*NS columns) tile of all three
// products, 3*S waves (S = C/256 K slices): wave (j, s) loads its slice of
// the fragment-packed mix operand of product j and of the weight panels and
// runs the MFMA chains. The slice partials meet in LDS, and the waves then
// fold (k, v, r) of each 16 x 16 tile and apply WKV, updating the state in
// place and writing ry fragment-packed for the output projection. k, v and r
// never leave the CU; the WKV operands of a tile are copied into LDS while
// the products run.
// ---------------------------------------------------------------------------
struct KvrWkvArgs {
    const kr_half* A[3];       // mixes for K, V, R: fragment-packed [M16, C] (int8: same bytes)
    const kr_half* Wf[3];      // K, V, R weights, W^T fragment-packed ([C, C])
    const float* sa[3];        // w8a8: per-row scales of the three mixes
    const float* sw[3];        // w8a8: per-output-channel scales of K, V, R
    const float* decay;        // [C] time decay (already -exp)
    const float* first;        // [C] time first
    float* aa;                 // [M, C] WKV state, updated in place
    float* bb;
    float* pp;
    kr_half* ry;               // fragment-packed [M16, C] (K = C operand of the output GEMM;
                               // for w8a8 quantised by that product on load)
    int M;
};

__device__ __forceinline__ kr_int4 as_int4(kr_half8 v) { return __builtin_bit_cast(kr_int4, v); }

// Asynchronous 16-byte copy global -> LDS (lane l writes lds_base + 16 l);
// counted in vmcnt like a load, no VGPRs held.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)src,
        (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// I8 (w8a8): int8 operands in the same 1 KB block layout (a 16 x 64 int8
// block is the 16 x 32 block of the 16-bit view), v_mfma_i32_16x16x64_i8,
// the slice partials summed exactly in int32, then value = (float(acc) *
// sa[m]) * sw[n], the int8 GEMM's dequantisation.
template <int S, int TM, int NS, bool I8>
__global__ void __launch_bounds__(192 * S) kvr_wkv_kernel(KvrWkvArgs a) {
    constexpr int C = 256 * S, NW = 3 * S, TT = TM * NS;
    constexpr int KB = I8 ? C / 64 : C / 32;          // 1 KB blocks per fragment row
    constexpr int QS = I8 ? 4 : 8;                    // blocks per 256-wide slice
    __shared__ __attribute__((aligned(16))) float part[3 * S * TT * 256];   // slice partials
    __shared__ __attribute__((aligned(16))) char wk[TT * 5 * 1024];         // WKV operands

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = wave / S, s = wave % S;
    const int M = a.M;
    // tile; the column groups are dealt so that one group's weight panels
    // stay on one XCD (workgroups go to the 8 XCDs round robin)
    constexpr int ng = C / (16 * NS);
    const int mt = (M + 16 * TM - 1) / (16 * TM);
    int m_t, n_g;
    if constexpr ((ng & 7) == 0) {
        const int k = blockIdx.x >> 3;
        n_g = (k / mt) * 8 + (blockIdx.x & 7);
        m_t = k % mt;
    } else {
        m_t = blockIdx.x / ng;
        n_g = blockIdx.x % ng;
    }
    const int m0 = m_t * 16 * TM, n0 = n_g * 16 * NS;
    const int last_mb = (M - 1) >> 4;

    // ---- operands of product j over slice s, then the WKV operands into LDS
    const kr_half* Aj = j == 0 ? a.A[0] : (j == 1 ? a.A[1] : a.A[2]);
    const kr_half* Wf = j == 0 ? a.Wf[0] : (j == 1 ? a.Wf[1] : a.Wf[2]);
    kr_half8 av[TM][QS], b[NS][QS];
    #pragma unroll
    for (int i = 0; i < TM; i++) {
        const kr_half* ap = Aj + ((size_t)min((m0 >> 4) + i, last_mb) * KB + QS * s) * 512 + lane * 8;
        #pragma unroll
        for (int q = 0; q < QS; q++) av[i][q] = *reinterpret_cast<const kr_half8*>(ap + 512 * q);
    }
    #pragma unroll
    for (int t = 0; t < NS; t++) {
        const kr_half* bp = Wf + ((size_t)((n0 >> 4) + t) * KB + QS * s) * 512 + lane * 8;
        #pragma unroll
        for (int q = 0; q < QS; q++) b[t][q] = *reinterpret_cast<const kr_half8*>(bp + 512 * q);
    }
    // in tile t a lane owns row tile_m(t), columns tile_n(t) .. +3
    auto tile_m = [&](int t) { return m0 + 16 * (t / NS) + (lane & 15); };
    auto tile_n = [&](int t) { return n0 + 16 * (t % NS) + 4 * (lane >> 4); };
    // w8a8 scales of this wave's tile (each wave folds at most one tile when
    // TT <= NW; more tiles reload them in the loop below)
    float q_sa[3] = {0.f, 0.f, 0.f};
    kr_float4 q_sw[3] = {};
    if constexpr (I8) {
        if (wave < TT) {
            const int qm = min(tile_m(wave), M - 1), qn = tile_n(wave);
            #pragma unroll
            for (int jj = 0; jj < 3; jj++) {
                q_sa[jj] = a.sa[jj][qm];
                q_sw[jj] = *reinterpret_cast<const kr_float4*>(a.sw[jj] + qn);
            }
        }
    }
    for (int t = wave; t < TT; t += NW) {
        const int en = tile_n(t);
        const size_t o = (size_t)min(tile_m(t), M - 1) * C + en;
        char* d = wk + t * 5 * 1024;
        lds_dma16(a.aa + o, d);
        lds_dma16(a.bb + o, d + 1024);
        lds_dma16(a.pp + o, d + 2048);
        lds_dma16(a.decay + en, d + 3072);
        lds_dma16(a.first + en, d + 4096);
    }

    // ---- MFMA chains (weight fragment in the A slot: lanes hold 4 columns of a row)
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int t = 0; t < NS; t++) {
            float* pd = part + ((j * S + s) * TT + i * NS + t) * 256 + lane * 4;
            if constexpr (I8) {
                kr_int4 acc = kr_int4{0, 0, 0, 0};
                #pragma unroll
                for (int q = 0; q < QS; q++)
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_int4(b[t][q]), as_int4(av[i][q]),
                                                                acc, 0, 0, 0);
                *reinterpret_cast<kr_int4*>(pd) = acc;
            } else {
                kr_float4 acc = kr_float4{0.f, 0.f, 0.f, 0.f};
                #pragma unroll
                for (int q = 0; q < QS; q++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[t][q], av[i][q], acc, 0, 0, 0);
                *reinterpret_cast<kr_float4*>(pd) = acc;
            }
        }
    // the WKV copies of every wave must have landed before the barrier
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // ---- fold the slices in order, then WKV on (k, v, r) of each tile
    for (int t = wave; t < TT; t += NW) {
        const int em = tile_m(t), en = tile_n(t);
        if (em >= M) continue;
        auto fold = [&](int jj) {
            if constexpr (I8) {
                kr_int4 iv = *reinterpret_cast<const kr_int4*>(part + (jj * S * TT + t) * 256 + lane * 4);
                #pragma unroll
                for (int q = 1; q < S; q++)
                    iv = iv + *reinterpret_cast<const kr_int4*>(part + ((jj * S + q) * TT + t) * 256 + lane * 4);
                float sa = q_sa[jj];
                kr_float4 sw = q_sw[jj];
                if (t != wave) {   // a second tile of this wave
                    sa = a.sa[jj][tile_m(t)];
                    sw = *reinterpret_cast<const kr_float4*>(a.sw[jj] + tile_n(t));
                }
                kr_float4 v;
                #pragma unroll
                for (int e = 0; e < 4; e++) v[e] = __fmul_rn(__fmul_rn((float)iv[e], sa), sw[e]);
                return v;
            } else {
                kr_float4 v = *reinterpret_cast<const kr_float4*>(part + (jj * S * TT + t) * 256 + lane * 4);
                #pragma unroll
                for (int q = 1; q < S; q++)
                    v = v + *reinterpret_cast<const kr_float4*>(part + ((jj * S + q) * TT + t) * 256 + lane * 4);
                return v;
            }
        };
        const kr_float4 k = fold(0), v = fold(1), rv = fold(2);
        const char* d = wk + t * 5 * 1024 + 16 * lane;
        kr_float4 sa = *reinterpret_cast<const kr_float4*>(d);
        kr_float4 sb = *reinterpret_cast<const kr_float4*>(d + 1024);
        kr_float4 sp = *reinterpret_cast<const kr_float4*>(d + 2048);
        const kr_float4 dw = *reinterpret_cast<const kr_float4*>(d + 3072);
        const kr_float4 du = *reinterpret_cast<const kr_float4*>(d + 4096);
        kr_half4 ry;
        #pragma unroll
        for (int e = 0; e < 4; e++) {
            const float r = (float)kr_f16(kr_sigmoid_t<I8>((float)kr_f16(rv[e])));
            WkvState st{sa[e], sb[e], sp[e]};
            ry[e] = wkv_token<I8>(st, dw[e], du[e], k[e], v[e], r);
            sa[e] = st.a;
            sb[e] = st.b;
            sp[e] = st.p;
        }
        const size_t o = (size_t)em * C + en;
        *reinterpret_cast<kr_float4*>(a.aa + o) = sa;
        *reinterpret_cast<kr_float4*>(a.bb + o) = sb;
        *reinterpret_cast<kr_float4*>(a.pp + o) = sp;
        *reinterpret_cast<kr_half4*>(a.ry + kr_frag_index(em, en, C)) = ry;
    }
}

// x[row] = emb[ids[row]] (ids clamped into [0, V) so a bad id cannot read
// out of bounds; callers validate ids before upload).
template <int G>
__global__ void __launch_bounds__(256) embed_kernel(const int32_t* __restrict__ ids,
                                                    const kr_half* __restrict__ emb, int V,
                                                    kr_half* __restrict__ x, int M) {
    constexpr int C = 256 * G;
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= M) return;
    int id = ids[row];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    #pragma unroll
    for (int i = 0; i < G; i++)
        *reinterpret_cast<kr_half4*>(x + (size_t)row * C + 256 * i + 4 * lane) =
            *reinterpret_cast<const kr_half4*>(emb + (size_t)id * C + 256 * i + 4 * lane);
}

// Fresh state: att_xx = ffn_xx = 0, aa = bb = 0, pp = -1e30 (cpp_path.py:94-106).
__global__ void state_init_kernel(char* __restrict__ state, int n_layer, int B, int C) {
    const size_t BC = (size_t)B * C;
    const size_t per = BC * 16;
    const size_t total_words = per * n_layer / 4;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total_words;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t off = (i * 4) % per;
        const bool is_pp = off >= BC * 12;
        reinterpret_cast<float*>(state)[i] = is_pp ? -1e30f : 0.0f;
    }
}

__global__ void neg_exp_kernel(const float* __restrict__ raw, float* __restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = -expf(raw[i]);
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
inline const kr_half* H(const void* p) { return reinterpret_cast<const kr_half*>(p); }
inline kr_half* Hm(void* p) { return reinterpret_cast<kr_half*>(p); }

template <int NMIX>
int launch_ln_mix(int G, const LnMixArgs& a_in, hipStream_t s) {
    LnMixArgs a = a_in;
    const int runs = (a.T + a.run - 1) / a.run;
    const long long waves = (long long)a.B * runs;
    if (waves == 0) return KR_OK;
    // LN-mix workgroups rounded to a multiple of 8 so the staging ones that
    // follow keep blockIdx % 8 == XCD (the spare LN-mix ones exit at once)
    // T = 1 rows (the decode step): one row per workgroup, spread over the
    // CUs; otherwise four waves (runs of rows) per workgroup
    a.one_row = a.T == 1 && waves <= 1024 ? 1 : 0;
    a.ln_blocks = (int)((a.one_row ? waves : (waves + 3) / 4) + 7) / 8 * 8;
    if (a.pf.n == 0) a.pf.blocks = 0;
    const int blocks = a.ln_blocks + a.pf.blocks;
    const bool q8 = NMIX > 0 && a.q[0] != nullptr;
#define KR_LN(G_)                                                         \
    case G_:                                                              \
        if (q8) ln_mix_kernel<G_, NMIX, true><<<blocks, 256, 0, s>>>(a);  \
        else ln_mix_kernel<G_, NMIX, false><<<blocks, 256, 0, s>>>(a);    \
        break;
    switch (G) {
        KR_LN(1) KR_LN(2) KR_LN(3) KR_LN(4)
        default: return kr_fail(KR_EUNSUPPORTED, "C=%d unsupported (256..1024, step 256)", 256 * G);
    }
#undef KR_LN
    KR_LAUNCHED();
    return KR_OK;
}

// Tile shape of the fused K, V, R + WKV launch: the fewest operand lines on
// the busiest CU (workgroups spread over 256 CUs, each reading 3 x (16*TM +
// 16*NS) rows of C), ties to more workgroups. 3 x 2 serves 342..480 rows in
// one round of workgroups where 2 x 2 needs two (measured on MI355X at
// B = 384: decode +4.5%, A B twice on one box).
template <int S, int TM, int NS, bool I8>
int launch_kvr_wkv_shape(const KvrWkvArgs& a, hipStream_t s) {
    const int mt = (a.M + 16 * TM - 1) / (16 * TM);
    const int blocks = mt * (256 * S / (16 * NS));
    kvr_wkv_kernel<S, TM, NS, I8><<<blocks, 192 * S, 0, s>>>(a);
    KR_LAUNCHED();
    return KR_OK;
}

constexpr int kKvrShapes[5][2] = {{2, 2}, {2, 1}, {1, 2}, {1, 1}, {3, 2}};   // (TM, NS)

// Shape of the K/V/R + WKV launch for M rows and C = 256 S channels (index
// into kKvrShapes): busiest-CU line model, ties to more workgroups.
int kvr_wkv_shape(int S, int M) {
    long long best = -1;
    int bi = 0;
    for (int i = 0; i < 5; i++) {
        const int TM = kKvrShapes[i][0], NS = kKvrShapes[i][1];
        const long long wgs = (long long)((M + 16 * TM - 1) / (16 * TM)) * (256 * S / (16 * NS));
        const long long cost = ((wgs + 255) / 256) * (TM + NS) * 4096 - std::min(wgs, 256ll);
        if (best < 0 || cost < best) { best = cost; bi = i; }
    }
    return bi;
}

template <int S, bool I8>
int launch_kvr_wkv_s(const KvrWkvArgs& a, hipStream_t s) {
    switch (kvr_wkv_shape(S, a.M)) {
        case 0: return launch_kvr_wkv_shape<S, 2, 2, I8>(a, s);
        case 1: return launch_kvr_wkv_shape<S, 2, 1, I8>(a, s);
        case 2: return launch_kvr_wkv_shape<S, 1, 2, I8>(a, s);
        case 4: return launch_kvr_wkv_shape<S, 3, 2, I8>(a, s);
        default: return launch_kvr_wkv_shape<S, 1, 1, I8>(a, s);
    }
}

template <bool I8>
int launch_kvr_wkv(int G, const KvrWkvArgs& a, hipStream_t s) {
    if (a.M == 0) return KR_OK;
    switch (G) {
        case 1: return launch_kvr_wkv_s<1, I8>(a, s);
        case 2: return launch_kvr_wkv_s<2, I8>(a, s);
        case 3: return launch_kvr_wkv_s<3, I8>(a, s);
        case 4: return launch_kvr_wkv_s<4, I8>(a, s);
        default: return kr_fail(KR_EUNSUPPORTED, "C=%d unsupported (256..1024, step 256)", 256 * G);
    }
}

// Workspace carve-up for M rows.
struct Work {
    kr_half *kx, *vx, *rx, *r, *ry, *fkx, *frx, *rf, *kf;
    float *k, *v;
    // w8a8 operands and their per-row scales
    int8_t *kx8, *vx8, *rx8, *ry8, *fkx8, *frx8, *kf8;
    float *kxs, *vxs, *rxs, *rys, *fkxs, *frxs, *kfs;
};

inline size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// Buffers hold M rounded up to 16 rows so fragment-packed operands are whole blocks.
size_t work_bytes(long long M, int C, int F) {
    M = kr_frag_rows(M);
    const size_t h = (size_t)M * C * 2, f = (size_t)M * C * 4, kf = (size_t)M * F * 2;
    const size_t b = (size_t)M * C, bf = (size_t)M * F, sc = (size_t)M * 4;
    return 8 * up256(h) + 2 * up256(f) + up256(kf) + 6 * up256(b) + up256(bf) + 7 * up256(sc);
}

Work carve(void* ws, long long M, int C, int F) {
    M = kr_frag_rows(M);
    char* p = static_cast<char*>(ws);
    auto take = [&](size_t bytes) { char* q = p; p += up256(bytes); return q; };
    const size_t h = (size_t)M * C * 2, f = (size_t)M * C * 4;
    Work w;
    w.kx = reinterpret_cast<kr_half*>(take(h));
    w.vx = reinterpret_cast<kr_half*>(take(h));
    w.rx = reinterpret_cast<kr_half*>(take(h));
    w.r = reinterpret_cast<kr_half*>(take(h));
    w.ry = reinterpret_cast<kr_half*>(take(h));
    w.fkx = reinterpret_cast<kr_half*>(take(h));
    w.frx = reinterpret_cast<kr_half*>(take(h));
    w.rf = reinterpret_cast<kr_half*>(take(h));
    w.k = reinterpret_cast<float*>(take(f));
    w.v = reinterpret_cast<float*>(take(f));
    w.kf = reinterpret_cast<kr_half*>(take((size_t)M * F * 2));
    int8_t** q8[6] = {&w.kx8, &w.vx8, &w.rx8, &w.ry8, &w.fkx8, &w.frx8};
    for (auto b : q8) *b = reinterpret_cast<int8_t*>(take((size_t)M * C));
    w.kf8 = reinterpret_cast<int8_t*>(take((size_t)M * F));
    float** sc[7] = {&w.kxs, &w.vxs, &w.rxs, &w.rys, &w.fkxs, &w.frxs, &w.kfs};
    for (auto b : sc) *b = reinterpret_cast<float*>(take((size_t)M * 4));
    return w;
}

int rows_per_run(int T) { return T >= 64 ? 16 : (T >= 8 ? 4 : 1); }

kr_gemm_args gemm_args(const kr_half* A, int M, int K, const void* Wt, int N, void* out,
                       const kr_half* res = nullptr, const kr_half* gate = nullptr,
                       const void* Wf = nullptr, bool a_frag = false, bool out_frag = false) {
    kr_gemm_args g{};
    g.Wf = H(Wf);
    g.a_frag = a_frag ? 1 : 0;
    g.out_frag = out_frag ? 1 : 0;
    g.A = A;
    g.lda = K;
    g.Wt = H(Wt);
    g.ldw = K;
    g.out = out;
    g.ldo = N;
    g.res = res;
    g.gate = gate;
    g.M = M;
    g.N = N;
    g.K = K;
    return g;
}

#define KR_TRY(expr)              \
    do {                          \
        int kr_rc_ = (expr);      \
        if (kr_rc_) return kr_rc_; \
    } while (0)

// Small-M calls (the stepped decode) keep every GEMM operand fragment-packed:
// the LN-mix, WKV and ReLU^2 producers write that layout directly.
bool use_fragments(const kr_layer_weights& L, long long M) {
    return M <= KR_GEMM_SMALL_M && L.Kf && L.Vf && L.Rf && L.Of && L.fKf && L.fVf && L.fRf;
}

// The int8 layer's small-M fragment path (its weights fragment-packed).
bool use_fragments_q8(const kr_layer_q8& Q, long long M) {
    return M <= KR_GEMM_SMALL_M && Q.K.qf && Q.V.qf && Q.R.qf && Q.O.qf && Q.fK.qf && Q.fV.qf &&
           Q.fR.qf;
}

// Layer 0's LN1-mix can run in the previous decode kernel (kr_embed_mix)
// when the layer is a stepped one on fragment-packed weights
// (layer_step_fused, or layer_forward_q8's stepped path).
bool kr_embed_mix_layer_ok(const kr_layer_weights& L, long long M, int T) {
    return T == 1 && (L.q8 ? use_fragments_q8(*L.q8, M) : use_fragments(L, M));
}

// Phase marks for the layer profiler: event i is recorded on the stream
// before phase i starts (i = 0..6) and event 7 after the last one. Phases:
// ln1_mix, kvr_matmul, wkv, ow_matmul_residual, ln2_mix, ffn_rk_matmul,
// ffn_v_matmul_residual. A fused launch that covers two phases leaves the
// second one empty. ev == nullptr records nothing.
// Marks lo .. lo + n - 1 are recorded, into ev[0 .. n - 1] (the layer
// profiler records all eight; the decode-step timing only the two around
// one phase).
// stamps (the decode-step timing of phase lo, whose one launch must be a
// small-M panel product): mark(lo) arms the buffer, and the events ev[0],
// ev[1] when given, for that launch, which stores its waves' start and end
// times there (the events take its dispatch's start and end); mark(lo + 1)
// disarms them and puts the launch's grid size in *grid.
struct Phases {
    hipEvent_t* ev = nullptr;
    hipStream_t s = nullptr;
    int lo = 0, n = 8;
    unsigned long long* stamps = nullptr;
    int max_groups = 0;
    int* grid = nullptr;
    int mark(int i) const {
        if (stamps) {
            if (i == lo) {
                kr_gemm_time_next_panel(stamps, max_groups, ev ? ev[0] : nullptr,
                                        ev ? ev[1] : nullptr);
            } else if (i == lo + 1) {
                const int taken = kr_gemm_timed_launch_taken();
                kr_gemm_time_next_panel(nullptr, 0);
                KR_REQUIRE(taken != 0, "step timing: phase %d ran no small-M panel launch", lo);
                KR_REQUIRE(taken > 0, "step timing: phase %d's launch has %d workgroups, more "
                           "than the %d the timing buffer holds", lo, -taken, max_groups);
                *grid = taken;
            }
            return KR_OK;
        }
        if (!ev || i < lo || i >= lo + n) return KR_OK;
        KR_HIP(hipEventRecord(ev[i - lo], s));
        return KR_OK;
    }
};

// Add the fragment-packed weight Wf ([N rows padded to 16] x K) to a staging
// set, cut into the column groups of NS 16-column panels that the product
// reading it will use; only when the groups are dealt to XCDs in eights.
// elem: bytes per weight (2 fp16, 1 int8; a 16-row fragment row is 16*K*elem).
void stage_weight(PrefetchSet& pf, const void* Wf, int N, int K, int NS, int elem = 2) {
    // whole groups only (the buffer ends at the last one), dealt in eights
    if (!Wf || NS <= 0 || pf.n >= 4 || N % (16 * NS) != 0 || (N / (16 * NS)) % 8 != 0) return;
    const int groups = N / (16 * NS);
    pf.base[pf.n] = static_cast<const char*>(Wf);
    pf.group_bytes[pf.n] = (long long)NS * 16 * K * elem;
    pf.n_groups[pf.n] = groups;
    pf.n++;
}

constexpr int kStageBlocks = 512;   // staging workgroups per LN-mix launch (64 per XCD)

// w8a8 layer: the same op order with the seven products on
// int8 MFMA. LN-mix writes its operands quantised per row. On the small-M
// fragment path the output projection and the channel-mix value product
// quantise their fp16 operands (the WKV output, the ReLU^2 output) on load;
// on the large-M path a row kernel quantises them first. Both give the same
// int8 operands and scales.
kr_gemm_args gemm_q8(const int8_t* A, const float* sa, int M, int K, const kr_matrix_q8& W,
                     int N, void* out, bool fr, const kr_half* res = nullptr,
                     const kr_half* gate = nullptr) {
    kr_gemm_args g = gemm_args(reinterpret_cast<const kr_half*>(A), M, K, W.q, N, out, res, gate,
                               W.qf, fr);
    g.i8 = 1;
    g.sa = sa;
    g.sw = W.scale;
    return g;
}

// The same with A as fp16 fragment-packed, quantised per row by the product.
kr_gemm_args gemm_q8_q16(const kr_half* A, int M, int K, const kr_matrix_q8& W, int N, void* out,
                         const kr_half* res = nullptr, const kr_half* gate = nullptr) {
    kr_gemm_args g = gemm_args(A, M, K, W.q, N, out, res, gate, W.qf, true);
    g.i8 = 1;
    g.sw = W.scale;
    g.a_q16 = 1;
    return g;
}

// Layer 0 of a forward that starts from token ids: its LN1-mix gathers the
// embedding rows itself and writes x (no separate embed launch). mixed: the
// previous decode kernel already ran that LN1-mix (kr_embed_mix), so the
// stepped layer starts at its K, V, R products.
struct EmbedSrc {
    const int32_t* ids;
    const kr_half* emb;
    int V;
    bool mixed;
};

inline void set_embed(LnMixArgs& a, const EmbedSrc* e, kr_half* x) {
    a.ids = e ? e->ids : nullptr;
    a.emb = e ? e->emb : nullptr;
    a.V = e ? e->V : 0;
    a.xw = e ? x : nullptr;
}

// The weights a stepped layer's LN1-mix launch stages into L2: the K, V, R
// products' and the output projection's (fp16 or int8), as their launches
// deal them.
PrefetchSet att_stage_set(const kr_layer_weights& L, int C, int M, const Work& w, kr_half* x) {
    PrefetchSet pf{};
    const int ns_kvr = kKvrShapes[kvr_wkv_shape(C / 256, M)][1];
    if (L.q8) {
        const kr_layer_q8& Q = *L.q8;
        stage_weight(pf, Q.K.qf, C, C, ns_kvr, 1);
        stage_weight(pf, Q.V.qf, C, C, ns_kvr, 1);
        stage_weight(pf, Q.R.qf, C, C, ns_kvr, 1);
        const kr_gemm_args o = gemm_q8_q16(w.ry, M, C, Q.O, C, x, x);
        stage_weight(pf, Q.O.qf, C, C, kr_gemm_panel_ns(&o, 1), 1);
    } else {
        stage_weight(pf, L.Kf, C, C, ns_kvr);
        stage_weight(pf, L.Vf, C, C, ns_kvr);
        stage_weight(pf, L.Rf, C, C, ns_kvr);
        const kr_gemm_args o = gemm_args(w.ry, M, C, L.Ot, C, x, x, nullptr, L.Of, true);
        stage_weight(pf, L.Of, C, C, kr_gemm_panel_ns(&o, 1));
    }
    pf.blocks = kStageBlocks;
    return pf;
}

int layer_forward_q8(const kr_layer_weights& L, int C, int F, kr_half* x, int B, int T,
                     const kr_layer_state& st, const Work& w, hipStream_t s,
                     const EmbedSrc* e, const Phases& ph) {
    const kr_layer_q8& Q = *L.q8;
    const int M = B * T, G = C / 256;
    const bool fr = use_fragments_q8(Q, M);
    LnMixArgs a{};
    a.x = x;
    a.ln_w = H(L.ln1_w);
    a.ln_b = H(L.ln1_b);
    a.tm[0] = H(L.tm_k); a.tm[1] = H(L.tm_v); a.tm[2] = H(L.tm_r);
    a.q[0] = w.kx8; a.q[1] = w.vx8; a.q[2] = w.rx8;
    a.qs[0] = w.kxs; a.qs[1] = w.vxs; a.qs[2] = w.rxs;
    a.state = Hm(st.att_xx);
    a.B = B;
    a.T = T;
    a.run = rows_per_run(T);
    a.frag = fr ? 1 : 0;
    set_embed(a, e, x);
    // stepped: LN1 stages the int8 K, V, R and output-projection weights in
    // their XCDs' L2, LN2 the value product's (as layer_step_fused does)
    PrefetchSet pf_ffn{};
    if (fr && T == 1) {
        a.pf = att_stage_set(L, C, M, w, x);
        const kr_gemm_args v = gemm_q8_q16(w.kf, M, F, Q.fV, C, x, x, w.rf);
        stage_weight(pf_ffn, Q.fV.qf, C, F, kr_gemm_panel_ns(&v, 1), 1);
        pf_ffn.blocks = kStageBlocks;
    }
    KR_TRY(ph.mark(0));
    if (!(e && e->mixed)) KR_TRY(launch_ln_mix<3>(G, a, s));
    set_embed(a, nullptr, x);
    a.pf = pf_ffn;
    KR_TRY(ph.mark(1));
    if (fr && T == 1) {
        // stepped: the three int8 products and the WKV update in one launch
        KvrWkvArgs kw{};
        kw.A[0] = reinterpret_cast<const kr_half*>(w.kx8);
        kw.A[1] = reinterpret_cast<const kr_half*>(w.vx8);
        kw.A[2] = reinterpret_cast<const kr_half*>(w.rx8);
        kw.Wf[0] = H(Q.K.qf); kw.Wf[1] = H(Q.V.qf); kw.Wf[2] = H(Q.R.qf);
        kw.sa[0] = w.kxs; kw.sa[1] = w.vxs; kw.sa[2] = w.rxs;
        kw.sw[0] = Q.K.scale; kw.sw[1] = Q.V.scale; kw.sw[2] = Q.R.scale;
        kw.decay = L.decay;
        kw.first = L.first;
        kw.aa = st.aa;
        kw.bb = st.bb;
        kw.pp = st.pp;
        kw.ry = w.ry;
        kw.M = M;
        KR_TRY(launch_kvr_wkv<true>(G, kw, s));
        KR_TRY(ph.mark(2));
    } else {
        {
            const kr_gemm_args jobs[3] = {gemm_q8(w.kx8, w.kxs, M, C, Q.K, C, w.k, fr),
                                          gemm_q8(w.vx8, w.vxs, M, C, Q.V, C, w.v, fr),
                                          gemm_q8(w.rx8, w.rxs, M, C, Q.R, C, w.r, fr)};
            const int eps[3] = {KR_EP_F32, KR_EP_F32, KR_EP_SIGMOID};
            KR_TRY(kr_gemm_launch_multi(jobs, eps, 3, s));
        }
        KR_TRY(ph.mark(2));
        dim3 grid((C + 255) / 256, B);
        wkv_kernel<true><<<grid, 256, 0, s>>>(w.k, w.v, w.r, L.decay, L.first, st.aa, st.bb, st.pp,
                                        w.ry, B, T, C, fr ? 1 : 0);
        KR_LAUNCHED();
    }
    KR_TRY(ph.mark(3));
    if (fr) {
        KR_TRY(kr_gemm_launch(gemm_q8_q16(w.ry, M, C, Q.O, C, x, x), KR_EP_RESID, s));
    } else {
        KR_TRY(kr_impl_quantize_rows(w.ry, C, M, C, w.ry8, w.rys, 0, s));
        KR_TRY(kr_gemm_launch(gemm_q8(w.ry8, w.rys, M, C, Q.O, C, x, false, x), KR_EP_RESID, s));
    }
    KR_TRY(ph.mark(4));
    a.ln_w = H(L.ln2_w);
    a.ln_b = H(L.ln2_b);
    a.tm[0] = H(L.ftm_k); a.tm[1] = H(L.ftm_r);
    a.q[0] = w.fkx8; a.q[1] = w.frx8;
    a.qs[0] = w.fkxs; a.qs[1] = w.frxs;
    a.state = Hm(st.ffn_xx);
    KR_TRY(launch_ln_mix<2>(G, a, s));
    KR_TRY(ph.mark(5));
    {
        kr_gemm_args jobs[2] = {gemm_q8(w.frx8, w.frxs, M, C, Q.fR, C, w.rf, fr),
                                gemm_q8(w.fkx8, w.fkxs, M, C, Q.fK, F, w.kf, fr)};
        jobs[1].out_frag = fr ? 1 : 0;     // the value product's fp16 operand
        const int eps[2] = {KR_EP_SIGMOID, KR_EP_RELUSQ};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 2, s));
    }
    KR_TRY(ph.mark(6));
    if (fr) {
        KR_TRY(kr_gemm_launch(gemm_q8_q16(w.kf, M, F, Q.fV, C, x, x, w.rf), KR_EP_GATED, s));
    } else {
        KR_TRY(kr_impl_quantize_rows(w.kf, F, M, F, w.kf8, w.kfs, 0, s));
        KR_TRY(kr_gemm_launch(gemm_q8(w.kf8, w.kfs, M, F, Q.fV, C, x, false, x, w.rf),
                              KR_EP_GATED, s));
    }
    return ph.mark(7);
}

// Stepped (T = 1) fp16 layer with fragment-packed weights: LN1-mix, the
// K, V, R products fused with WKV, the output projection, LN2-mix and the
// channel mix (six launches).

int layer_step_fused(const kr_layer_weights& L, int C, int F, kr_half* x, int B,
                     const kr_layer_state& st, const Work& w, hipStream_t s,
                     const EmbedSrc* e, const Phases& ph) {
    const int M = B, G = C / 256;
    // Weights the next products read, staged into their XCDs' L2 by the
    // LN-mix launches (which wait on memory latency, not bandwidth): LN1 stages
    // K, V, R and the output projection, LN2 the channel-mix value product.
    // Staging bytes still cost HBM time inside the LN-mix launch; staging the
    // channel-mix R/K weights too (another 5.9 MB) lengthened LN2 by more than
    // it saved, measured on MI355X at B = 256.
    const PrefetchSet pf_att = att_stage_set(L, C, M, w, x);
    PrefetchSet pf_ffn{};
    {
        const kr_gemm_args v = gemm_args(w.kf, M, F, L.fVt, C, x, x, w.rf, L.fVf, true);
        stage_weight(pf_ffn, L.fVf, C, F, kr_gemm_panel_ns(&v, 1));
        pf_ffn.blocks = kStageBlocks;
    }
    LnMixArgs a{};
    a.x = x;
    a.ln_w = H(L.ln1_w);
    a.ln_b = H(L.ln1_b);
    a.tm[0] = H(L.tm_k); a.tm[1] = H(L.tm_v); a.tm[2] = H(L.tm_r);
    a.out[0] = w.kx; a.out[1] = w.vx; a.out[2] = w.rx;
    a.state = Hm(st.att_xx);
    a.B = B;
    a.T = 1;
    a.run = 1;
    a.frag = 1;
    set_embed(a, e, x);
    a.pf = pf_att;
    KR_TRY(ph.mark(0));
    if (!(e && e->mixed)) KR_TRY(launch_ln_mix<3>(G, a, s));
    set_embed(a, nullptr, x);
    KR_TRY(ph.mark(1));
    KvrWkvArgs kw{};
    kw.A[0] = w.kx; kw.A[1] = w.vx; kw.A[2] = w.rx;
    kw.Wf[0] = H(L.Kf); kw.Wf[1] = H(L.Vf); kw.Wf[2] = H(L.Rf);
    kw.decay = L.decay;
    kw.first = L.first;
    kw.aa = st.aa;
    kw.bb = st.bb;
    kw.pp = st.pp;
    kw.ry = w.ry;
    kw.M = M;
    KR_TRY(launch_kvr_wkv<false>(G, kw, s));
    KR_TRY(ph.mark(2));
    KR_TRY(ph.mark(3));      // WKV ran inside the K/V/R launch
    KR_TRY(kr_gemm_launch(gemm_args(w.ry, M, C, L.Ot, C, x, x, nullptr, L.Of, true), KR_EP_RESID, s));
    KR_TRY(ph.mark(4));
    a.ln_w = H(L.ln2_w);
    a.ln_b = H(L.ln2_b);
    a.tm[0] = H(L.ftm_k); a.tm[1] = H(L.ftm_r);
    a.out[0] = w.fkx; a.out[1] = w.frx;
    a.state = Hm(st.ffn_xx);
    a.pf = pf_ffn;
    KR_TRY(launch_ln_mix<2>(G, a, s));
    KR_TRY(ph.mark(5));
    {
        const kr_gemm_args jobs[2] = {
            gemm_args(w.frx, M, C, L.fRt, C, w.rf, nullptr, nullptr, L.fRf, true),
            gemm_args(w.fkx, M, C, L.fKt, F, w.kf, nullptr, nullptr, L.fKf, true, true)};
        const int eps[2] = {KR_EP_SIGMOID, KR_EP_RELUSQ};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 2, s));
    }
    KR_TRY(ph.mark(6));
    KR_TRY(kr_gemm_launch(gemm_args(w.kf, M, F, L.fVt, C, x, x, w.rf, L.fVf, true), KR_EP_GATED, s));
    return ph.mark(7);
}

int layer_forward(const kr_layer_weights& L, int C, int F, kr_half* x, int B, int T,
                  const kr_layer_state& st, const Work& w, hipStream_t s,
                  const EmbedSrc* e = nullptr, const Phases& ph = Phases{}) {
    KR_REQUIRE(!(e && e->mixed) || kr_embed_mix_layer_ok(L, (long long)B * T, T),
               "forward: layer 0's LN1-mix can only be skipped in a stepped layer on "
               "fragment-packed weights (fp16 or w8a8)");
    if (L.q8) return layer_forward_q8(L, C, F, x, B, T, st, w, s, e, ph);
    const int M = B * T, G = C / 256;
    const bool fr = use_fragments(L, M);
    if (fr && T == 1) return layer_step_fused(L, C, F, x, B, st, w, s, e, ph);
    LnMixArgs a{};
    a.x = x;
    a.ln_w = H(L.ln1_w);
    a.ln_b = H(L.ln1_b);
    a.tm[0] = H(L.tm_k); a.tm[1] = H(L.tm_v); a.tm[2] = H(L.tm_r);
    a.out[0] = w.kx; a.out[1] = w.vx; a.out[2] = w.rx;
    a.state = Hm(st.att_xx);
    a.B = B;
    a.T = T;
    a.run = rows_per_run(T);
    a.frag = fr ? 1 : 0;
    set_embed(a, e, x);
    KR_TRY(ph.mark(0));
    KR_TRY(launch_ln_mix<3>(G, a, s));
    set_embed(a, nullptr, x);
    KR_TRY(ph.mark(1));
    {
        const kr_gemm_args jobs[3] = {
            gemm_args(w.kx, M, C, L.Kt, C, w.k, nullptr, nullptr, L.Kf, fr),
            gemm_args(w.vx, M, C, L.Vt, C, w.v, nullptr, nullptr, L.Vf, fr),
            gemm_args(w.rx, M, C, L.Rt, C, w.r, nullptr, nullptr, L.Rf, fr)};
        const int eps[3] = {KR_EP_F32, KR_EP_F32, KR_EP_SIGMOID};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 3, s));
    }
    KR_TRY(ph.mark(2));
    {
        dim3 grid((C + 255) / 256, B);
        wkv_kernel<false><<<grid, 256, 0, s>>>(w.k, w.v, w.r, L.decay, L.first, st.aa, st.bb, st.pp,
                                        w.ry, B, T, C, fr ? 1 : 0);
        KR_LAUNCHED();
    }
    KR_TRY(ph.mark(3));
    KR_TRY(kr_gemm_launch(gemm_args(w.ry, M, C, L.Ot, C, x, x, nullptr, L.Of, fr), KR_EP_RESID, s));
    KR_TRY(ph.mark(4));
    a.ln_w = H(L.ln2_w);
    a.ln_b = H(L.ln2_b);
    a.tm[0] = H(L.ftm_k); a.tm[1] = H(L.ftm_r);
    a.out[0] = w.fkx; a.out[1] = w.frx;
    a.state = Hm(st.ffn_xx);
    KR_TRY(launch_ln_mix<2>(G, a, s));
    KR_TRY(ph.mark(5));
    {
        const kr_gemm_args jobs[2] = {
            gemm_args(w.frx, M, C, L.fRt, C, w.rf, nullptr, nullptr, L.fRf, fr),
            gemm_args(w.fkx, M, C, L.fKt, F, w.kf, nullptr, nullptr, L.fKf, fr, fr)};
        const int eps[2] = {KR_EP_SIGMOID, KR_EP_RELUSQ};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 2, s));
    }
    KR_TRY(ph.mark(6));
    KR_TRY(kr_gemm_launch(gemm_args(w.kf, M, F, L.fVt, C, x, x, w.rf, L.fVf, fr), KR_EP_GATED, s));
    return ph.mark(7);
}

int check_model(const kr_model_weights* m) {
    KR_REQUIRE(m && m->layers && m->emb && m->headT && m->ln_out_w && m->ln_out_b,
               "model: null pointer");
    KR_REQUIRE(m->n_layer >= 1 && m->n_layer <= 64, "model: bad n_layer %d", m->n_layer);
    KR_REQUIRE(m->C % 256 == 0 && m->C >= 256 && m->C <= 1024, "model: C=%d unsupported", m->C);
    KR_REQUIRE(m->F % 64 == 0 && m->F >= 64, "model: F=%d unsupported", m->F);
    KR_REQUIRE(m->V >= 1 && m->V <= 65536, "model: V=%d unsupported", m->V);
    return KR_OK;
}

// State buffer layout per layer: [att_xx fp16 | ffn_xx fp16 | aa | bb | pp fp32], each [B, C].
kr_layer_state state_of(void* state, int layer, int B, int C) {
    const size_t per = (size_t)B * C * (2 + 2 + 4 * 3);
    char* p = static_cast<char*>(state) + per * layer;
    kr_layer_state st;
    st.att_xx = p;
    st.ffn_xx = p + (size_t)B * C * 2;
    st.aa = reinterpret_cast<float*>(p + (size_t)B * C * 4);
    st.bb = reinterpret_cast<float*>(p + (size_t)B * C * 8);
    st.pp = reinterpret_cast<float*>(p + (size_t)B * C * 12);
    return st;
}

// ---------------------------------------------------------------------------
// Layer phase profiler (the role of layer_cpp.cpp:111-157): when on, each
// kr_layer_step call records HIP events between its phases on its stream,
// waits for the last one and adds the elapsed times to running sums. Off by
// default; KRUNCH_PHASE_PROFILE=1 turns it on at first use, kr_phase_profile
// at any time. Calls made during stream capture are never profiled.
// ---------------------------------------------------------------------------
constexpr int kPhases = 7;
const char* const kPhaseNames[kPhases] = {"ln1_mix", "kvr_matmul", "wkv", "ow_matmul_residual",
                                          "ln2_mix", "ffn_rk_matmul", "ffn_v_matmul_residual"};

struct PhaseProfiler {
    std::mutex mu;
    int enabled = -1;               // -1: not decided yet (read the environment)
    int dev = -1;                   // device the events belong to
    hipEvent_t ev[kPhases + 1] = {};
    double sum_ms[kPhases] = {};
    long long calls = 0;
};
PhaseProfiler g_prof;

// with g_prof.mu held
int profile_state() {
    if (g_prof.enabled < 0) {
        const char* e = std::getenv("KRUNCH_PHASE_PROFILE");
        g_prof.enabled = (e && std::strcmp(e, "1") == 0) ? 1 : 0;
    }
    return g_prof.enabled;
}

bool profile_on() {
    std::lock_guard<std::mutex> lock(g_prof.mu);
    return profile_state() == 1;
}

// with g_prof.mu held: events on the current device
int profile_events() {
    int dev = 0;
    KR_HIP(hipGetDevice(&dev));
    if (g_prof.dev == dev && g_prof.ev[0]) return KR_OK;
    for (auto& e : g_prof.ev)
        if (e) { (void)hipEventDestroy(e); e = nullptr; }
    g_prof.dev = -1;
    for (auto& e : g_prof.ev) KR_HIP(hipEventCreate(&e));
    g_prof.dev = dev;
    return KR_OK;
}

// ---------------------------------------------------------------------------
// Decode-step timing: when a phase p whose launch is a small-M panel product
// is selected (3 output projection, 5 channel-mix R + K, 6 value product),
// every layer of a stepped forward launches that product with a stamp
// buffer: each of its waves stores its start and end on the 100 MHz steady
// counter (also inside a captured decode graph, at every replay). Outside
// stream capture the launch also takes two HIP events through
// hipExtLaunchKernel, which record its dispatch's start and end. Reading
// returns, per layer, the last launch's event duration (eager steps) and its
// wave span (last end minus first start), in microseconds. No other launch
// changes.
// ---------------------------------------------------------------------------
constexpr int kMaxTimedLayers = 64;
constexpr int kStampGroups = 2048;                 // workgroups per timed launch
constexpr size_t kStampLayerU64 = 2ull * KR_STAMP_WAVES * kStampGroups;

struct StepTiming {
    std::mutex mu;
    int phase = -1;                 // -1: off
    int dev = -1;                   // device of `stamps` and `ev`
    unsigned long long* stamps = nullptr;   // [kMaxTimedLayers][kStampLayerU64]
    hipEvent_t ev[kMaxTimedLayers][2] = {};
    int n = 0;                      // layers the last timed forward launched
    bool eager = false;             // ... outside stream capture (events recorded)
    int grid[kMaxTimedLayers] = {};
};
StepTiming g_step;

// ---------------------------------------------------------------------------
// Allocation-free layer step (kr_layer_step_noalloc): the workspace is this
// file-scope device array, KR_NOALLOC_SCRATCH_BYTES per GPU, held until the
// process ends. Host code never passes `scratch` itself (in host code the
// name stands for a host-side shadow, not a device address): the device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and only that address is handed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[KR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on first use there).
int scratch_on_current_device(void** out) {
    int dev = 0;
    KR_HIP(hipGetDevice(&dev));
    KR_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        KR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        KR_REQUIRE(p != nullptr, "no device address for the static scratch on device %d", dev);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KR_OK;
}

}  // namespace

// Entry points used by kr_engine.cpp.
// ids (nullable): x starts as the embedding of these [B, T] token ids, gathered
// by layer 0's LN1-mix (which writes x); otherwise x holds the input rows.
int kr_impl_forward_layers(const kr_model_weights* m, void* x, int B, int T, void* state,
                           void* ws, size_t ws_bytes, hipStream_t s, const int32_t* ids) {
    KR_TRY(check_model(m));
    KR_REQUIRE(x && state && ws, "forward: null pointer");
    const long long M = (long long)B * T;
    KR_REQUIRE(B >= 1 && T >= 1 && M <= (1ll << 31) / m->F, "forward: bad B=%d T=%d", B, T);
    KR_REQUIRE(ws_bytes >= work_bytes(M, m->C, m->F), "forward: workspace too small");
    const Work w = carve(ws, M, m->C, m->F);
    const EmbedSrc e{ids, H(m->emb), m->V, false};
    for (int i = 0; i < m->n_layer; i++)
        KR_TRY(layer_forward(m->layers[i], m->C, m->F, Hm(x), B, T, state_of(state, i, B, m->C),
                             w, s, i == 0 && ids ? &e : nullptr));
    return KR_OK;
}

// The layer stack for streams [b0, b0 + B) of a state buffer holding state_B
// streams (one group of a larger batch; rows of each [state_B, C] component).
int kr_impl_forward_layers_view(const kr_model_weights* m, void* x, int B, int T, void* state,
                                int state_B, int b0, void* ws, size_t ws_bytes, hipStream_t s,
                                const int32_t* ids, bool l0_mixed) {
    KR_TRY(check_model(m));
    KR_REQUIRE(x && state && ws, "forward: null pointer");
    KR_REQUIRE(b0 >= 0 && B >= 1 && b0 + B <= state_B, "forward: bad stream range");
    const long long M = (long long)B * T;
    KR_REQUIRE(T >= 1 && M <= (1ll << 31) / m->F, "forward: bad T=%d", T);
    KR_REQUIRE(ws_bytes >= work_bytes(M, m->C, m->F), "forward: workspace too small");
    const Work w = carve(ws, M, m->C, m->F);
    const size_t off = (size_t)b0 * m->C;
    KR_REQUIRE(!l0_mixed || ids, "forward: a mixed layer 0 needs the token ids");
    const EmbedSrc e{ids, H(m->emb), m->V, l0_mixed};
    int tphase = -1;
    if (T == 1) {
        std::lock_guard<std::mutex> lock(g_step.mu);
        int dev = 0;
        KR_HIP(hipGetDevice(&dev));
        if (g_step.phase >= 0 && g_step.stamps && g_step.dev == dev) {
            tphase = g_step.phase;
            g_step.n = std::min(m->n_layer, kMaxTimedLayers);
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            KR_HIP(hipStreamIsCapturing(s, &cs));
            g_step.eager = cs == hipStreamCaptureStatusNone;
        }
    }
    for (int i = 0; i < m->n_layer; i++) {
        kr_layer_state st = state_of(state, i, state_B, m->C);
        st.att_xx = static_cast<kr_half*>(st.att_xx) + off;
        st.ffn_xx = static_cast<kr_half*>(st.ffn_xx) + off;
        st.aa += off;
        st.bb += off;
        st.pp += off;
        Phases ph;
        if (tphase >= 0 && i < kMaxTimedLayers) {
            ph.lo = tphase;
            if (g_step.eager) ph.ev = g_step.ev[i];
            ph.stamps = g_step.stamps + (size_t)i * kStampLayerU64;
            ph.max_groups = kStampGroups;
            ph.grid = &g_step.grid[i];
        }
        KR_TRY(layer_forward(m->layers[i], m->C, m->F, Hm(x), B, T, st, w, s,
                             i == 0 && ids ? &e : nullptr, ph));
    }
    return KR_OK;
}

// Arguments of layer 0's LN1-mix inside the decode kernel (kr_embed_mix) for
// a stepped forward of streams [b0, b0 + B) of a state holding state_B
// streams, run with workspace ws and residual stream x. first: the run's
// first step, whose carried row is the state's; later steps read the row the
// previous step left in pend (the workspace's r rows, which the stepped fp16
// layer does not use). *dev: where the decode kernel reads its copy of *em
// (the workspace's k buffer, also unused there; one slot per value of first).
// False when layer 0 is not that layer.
bool kr_impl_embed_mix_args(const kr_model_weights* m, int B, void* state, int state_B, int b0,
                            void* ws, void* x, bool first, kr_embed_mix* em, kr_embed_mix** dev) {
    if (!m || !m->layers || m->n_layer < 1 || !m->emb || !state || !ws || !x || !em || !dev)
        return false;
    if (m->C % 256 || m->C < 256 || m->C > 1024 || B < 1 || b0 < 0 || b0 + B > state_B) return false;
    // every layer must be a stepped layer on fragment-packed weights: only
    // those leave the workspace's r rows (pend) and k buffer (the
    // descriptors) alone between two decode kernels
    for (int i = 0; i < m->n_layer; i++)
        if (!kr_embed_mix_layer_ok(m->layers[i], B, 1)) return false;
    const kr_layer_weights& L = m->layers[0];
    const Work w = carve(ws, B, m->C, m->F);
    kr_half* sx = static_cast<kr_half*>(state_of(state, 0, state_B, m->C).att_xx) + (size_t)b0 * m->C;
    *em = kr_embed_mix{};
    em->emb = H(m->emb);
    em->V = m->V;
    em->C = m->C;
    em->ln_w = H(L.ln1_w);
    em->ln_b = H(L.ln1_b);
    em->tm[0] = H(L.tm_k); em->tm[1] = H(L.tm_v); em->tm[2] = H(L.tm_r);
    em->out[0] = w.kx; em->out[1] = w.vx; em->out[2] = w.rx;
    if (L.q8) {
        em->q[0] = w.kx8; em->q[1] = w.vx8; em->q[2] = w.rx8;
        em->qs[0] = w.kxs; em->qs[1] = w.vxs; em->qs[2] = w.rxs;
    }
    em->state = sx;
    em->pend = w.r;
    em->src = first ? sx : w.r;
    em->xw = Hm(x);
    // staged by the decode kernel's waves 4..15: 3 blocks of 256 threads per
    // row, the rows of one XCD in whole eights
    em->pf = att_stage_set(L, m->C, B, w, Hm(x));
    em->pf.blocks = (B / 8) * 3 * 8;
    *dev = reinterpret_cast<kr_embed_mix*>(w.k) + (first ? 0 : 1);
    return true;
}

int kr_impl_embed(const kr_model_weights* m, const int32_t* ids, int M, void* x, hipStream_t s) {
    if (M == 0) return KR_OK;
    const int blocks = (M + 3) / 4, G = m->C / 256;
    switch (G) {
        case 1: embed_kernel<1><<<blocks, 256, 0, s>>>(ids, H(m->emb), m->V, Hm(x), M); break;
        case 2: embed_kernel<2><<<blocks, 256, 0, s>>>(ids, H(m->emb), m->V, Hm(x), M); break;
        case 3: embed_kernel<3><<<blocks, 256, 0, s>>>(ids, H(m->emb), m->V, Hm(x), M); break;
        case 4: embed_kernel<4><<<blocks, 256, 0, s>>>(ids, H(m->emb), m->V, Hm(x), M); break;
        default: return kr_fail(KR_EUNSUPPORTED, "C=%d unsupported", m->C);
    }
    KR_LAUNCHED();
    return KR_OK;
}

// logits[M, ld] = fp16(LN_out(x) @ head); xn is an [M, C] fp16 scratch.
// Up to 512 rows (the decode step) with a fragment-packed head: LN_out writes
// xn fragment-packed and the small-M head kernel reads it. That needs xn to
// hold M rounded up to 16 rows (xn_rows16). Otherwise xn is row-major and the
// large-M head kernel runs. Both kernels follow the head's one-chain
// contract (kr_gemm.h), so a row's logits do not depend on the path.
int kr_impl_head(const kr_model_weights* m, const void* x, int M, void* xn, void* logits,
                 long long ld, hipStream_t s, bool xn_rows16) {
    if (M == 0) return KR_OK;
    // up to 512 rows in one small-M launch (groups of 128 rows, each held in
    // registers by its workgroups). Measured at 512 rows on MI355X: two
    // 256-row small-M launches took 2 x ~30 us against 66.8 us for one
    // 256x128 launch, and one 512-row launch decodes 0.7% faster than the two
    // (B = 512, A B twice on one box).
    const bool small = xn_rows16 && m->headF && kr_gemm_head_small_ok(M, m->V, m->C);
    LnMixArgs a{};
    a.x = H(x);
    a.ln_w = H(m->ln_out_w);
    a.ln_b = H(m->ln_out_b);
    a.out[0] = Hm(xn);
    a.B = M;
    a.T = 1;
    a.run = 1;
    a.frag = small ? 1 : 0;
    KR_TRY(launch_ln_mix<0>(m->C / 256, a, s));
    if (small) return kr_gemm_head_small(H(xn), H(m->headF), M, m->V, m->C, Hm(logits), ld, s);
    return kr_gemm_head_big(H(xn), m->C, H(m->headT), m->C, M, m->V, m->C, Hm(logits), ld, s);
}

size_t kr_impl_work_bytes(long long M, int C, int F) { return work_bytes(M, C, F); }

void* kr_impl_head_scratch(void* ws, long long M, int C, int F) { return carve(ws, M, C, F).kx; }

kr_layer_state kr_impl_state_of(void* state, int layer, int B, int C) {
    return state_of(state, layer, B, C);
}

extern "C" {

size_t kr_state_bytes(int n_layer, int B, int C) { return (size_t)n_layer * B * C * 16; }

int kr_state_init(void* state, int n_layer, int B, int C, void* stream) {
    KR_REQUIRE(state && n_layer >= 1 && B >= 1 && C >= 1, "kr_state_init: bad args");
    state_init_kernel<<<256, 256, 0, kr_stream(stream)>>>(static_cast<char*>(state), n_layer, B, C);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_prepare_decay(const float* raw, float* out, int n, void* stream) {
    KR_REQUIRE(raw && out && n >= 0, "kr_prepare_decay: bad args");
    if (n == 0) return KR_OK;
    neg_exp_kernel<<<(n + 255) / 256, 256, 0, kr_stream(stream)>>>(raw, out, n);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_layer_step(const kr_layer_weights* L, int C, int F, void* x, int B, int T,
                  void* att_xx, float* aa, float* bb, float* pp, void* ffn_xx, void* ws,
                  size_t ws_bytes, void* stream) {
    KR_REQUIRE(L && x && att_xx && aa && bb && pp && ffn_xx && ws, "kr_layer_step: null pointer");
    KR_REQUIRE(C % 256 == 0 && C >= 256 && C <= 1024 && F % 64 == 0, "kr_layer_step: bad C/F");
    KR_REQUIRE(B >= 1 && T >= 1, "kr_layer_step: bad B=%d T=%d", B, T);
    const long long M = (long long)B * T;
    KR_REQUIRE(ws_bytes >= work_bytes(M, C, F), "kr_layer_step: workspace too small");
    kr_layer_state st{att_xx, aa, bb, pp, ffn_xx};
    const hipStream_t s = kr_stream(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    KR_HIP(hipStreamIsCapturing(s, &cap));
    if (!profile_on() || cap != hipStreamCaptureStatusNone)
        return layer_forward(*L, C, F, Hm(x), B, T, st, carve(ws, M, C, F), s);
    // Profiled call: events between the phases, then a wait for the last one
    // (one synchronisation per call, as the reference's profiler does).
    std::lock_guard<std::mutex> lock(g_prof.mu);
    KR_TRY(profile_events());
    Phases ph;
    ph.ev = g_prof.ev;
    ph.s = s;
    KR_TRY(layer_forward(*L, C, F, Hm(x), B, T, st, carve(ws, M, C, F), s, nullptr, ph));
    KR_HIP(hipEventSynchronize(g_prof.ev[kPhases]));
    for (int i = 0; i < kPhases; i++) {
        float ms = 0.f;
        KR_HIP(hipEventElapsedTime(&ms, g_prof.ev[i], g_prof.ev[i + 1]));
        g_prof.sum_ms[i] += ms;
    }
    g_prof.calls++;
    return KR_OK;
}

int kr_layer_step_noalloc(const kr_layer_weights* L, int C, int F, void* x, int B, int T,
                          void* att_xx, float* aa, float* bb, float* pp, void* ffn_xx,
                          void* stream) {
    KR_REQUIRE(L && x && att_xx && aa && bb && pp && ffn_xx,
               "kr_layer_step_noalloc: null pointer");
    KR_REQUIRE(C % 256 == 0 && C >= 256 && C <= 1024 && F % 64 == 0,
               "kr_layer_step_noalloc: bad C/F");
    KR_REQUIRE(B >= 1 && T >= 1, "kr_layer_step_noalloc: bad B=%d T=%d", B, T);
    const long long M = (long long)B * T;
    const size_t need = work_bytes(M, C, F);
    KR_REQUIRE(need <= (size_t)KR_NOALLOC_SCRATCH_BYTES,
               "kr_layer_step_noalloc: %lld rows need %zu workspace bytes, more than the "
               "%zu-byte static scratch (use kr_layer_step with a workspace)",
               M, need, (size_t)KR_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    KR_TRY(scratch_on_current_device(&ws));
    kr_layer_state st{att_xx, aa, bb, pp, ffn_xx};
    return layer_forward(*L, C, F, Hm(x), B, T, st, carve(ws, M, C, F), kr_stream(stream));
}

int kr_phase_profile(int enable) {
    std::lock_guard<std::mutex> lock(g_prof.mu);
    const int before = profile_state();
    if (enable == 0 || enable == 1) g_prof.enabled = enable;
    return before;
}

int kr_phase_count(void) { return kPhases; }

const char* kr_phase_name(int i) { return (i >= 0 && i < kPhases) ? kPhaseNames[i] : nullptr; }

int kr_read_phase_times(double* ms, int n, long long* call_count) {
    KR_REQUIRE(ms || n == 0, "kr_read_phase_times: null pointer");
    std::lock_guard<std::mutex> lock(g_prof.mu);
    for (int i = 0; i < n && i < kPhases; i++) ms[i] = g_prof.sum_ms[i];
    if (call_count) *call_count = g_prof.calls;
    return KR_OK;
}

int kr_reset_phase_times(void) {
    std::lock_guard<std::mutex> lock(g_prof.mu);
    for (double& v : g_prof.sum_ms) v = 0.0;
    g_prof.calls = 0;
    return KR_OK;
}

int kr_step_timing(int phase, int* previous) {
    KR_REQUIRE(phase == -1 || phase == 3 || phase == 5 || phase == 6,
               "kr_step_timing: phase %d is not a panel-product phase (3, 5 or 6)", phase);
    std::lock_guard<std::mutex> lock(g_step.mu);
    if (previous) *previous = g_step.phase;
    if (phase >= 0) {
        // the stamp buffer of the current device, cleared (slots of waves a
        // launch does not have stay zero and are skipped when reading)
        int dev = 0;
        KR_HIP(hipGetDevice(&dev));
        if (g_step.stamps && g_step.dev != dev) {
            KR_REQUIRE(false, "kr_step_timing: already in use on device %d", g_step.dev);
        }
        const size_t bytes = (size_t)kMaxTimedLayers * kStampLayerU64 * 8;
        if (!g_step.stamps) {
            for (auto& pair : g_step.ev)
                for (auto& e : pair) KR_HIP(hipEventCreate(&e));
            void* p = nullptr;
            KR_HIP(hipMalloc(&p, bytes));
            g_step.stamps = static_cast<unsigned long long*>(p);
            g_step.dev = dev;
        }
        KR_HIP(hipMemset(g_step.stamps, 0, bytes));
    }
    g_step.phase = phase;
    g_step.n = 0;
    return KR_OK;
}

int kr_step_timing_read(double* launch_us, double* span_us, int n, int* n_read) {
    KR_REQUIRE(n == 0 || (launch_us && span_us), "kr_step_timing_read: null pointer");
    std::lock_guard<std::mutex> lock(g_step.mu);
    KR_REQUIRE(g_step.stamps && g_step.n > 0, "kr_step_timing_read: no timed step has run");
    int dev = 0, khz = 0;
    KR_HIP(hipGetDevice(&dev));
    KR_REQUIRE(dev == g_step.dev, "kr_step_timing_read: the timed step ran on device %d",
               g_step.dev);
    KR_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    KR_REQUIRE(khz > 0, "kr_step_timing_read: no steady-counter rate");
    KR_HIP(hipDeviceSynchronize());
    const int k = std::min(n, g_step.n);
    std::vector<unsigned long long> h;
    for (int i = 0; i < k; i++) {
        const size_t used = 2ull * KR_STAMP_WAVES * g_step.grid[i];
        h.resize(used);
        KR_HIP(hipMemcpy(h.data(), g_step.stamps + (size_t)i * kStampLayerU64, used * 8,
                         hipMemcpyDeviceToHost));
        unsigned long long t0 = ~0ull, t1 = 0;
        for (size_t j = 0; j < used; j += 2) {
            if (!h[j]) continue;
            t0 = std::min(t0, h[j]);
            t1 = std::max(t1, h[j + 1]);
        }
        KR_REQUIRE(t1 > 0, "kr_step_timing_read: layer %d has no stamps", i);
        span_us[i] = (double)(t1 - t0) * 1000.0 / khz;
        launch_us[i] = -1.0;
        if (g_step.eager) {
            float ms = 0.f;
            KR_HIP(hipEventElapsedTime(&ms, g_step.ev[i][0], g_step.ev[i][1]));
            launch_us[i] = 1000.0 * ms;
        }
    }
    if (n_read) *n_read = k;
    g_step.n = 0;
    return KR_OK;
}

int kr_wkv(int B, int T, int C, const float* decay, const float* first, const float* k,
           const float* v, const uint16_t* r, float* aa, float* bb, float* pp, uint16_t* ry,
           void* stream) {
    KR_REQUIRE(decay && first && k && v && r && aa && bb && pp && ry, "kr_wkv: null pointer");
    KR_REQUIRE(B >= 1 && T >= 0 && C >= 1, "kr_wkv: bad shape");
    if (T == 0) return KR_OK;
    dim3 grid((C + 255) / 256, B);
    wkv_kernel<false><<<grid, 256, 0, kr_stream(stream)>>>(k, v, reinterpret_cast<const kr_half*>(r),
                                                    decay, first, aa, bb, pp,
                                                    reinterpret_cast<kr_half*>(ry), B, T, C, 0);
    KR_LAUNCHED();
    return KR_OK;
}

}  // extern "C"
