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
#include <vector>

#include "kr_gemm.h"
#include "kr_model.h"

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
    for (int o = 32; o > 0; o >>= 1) s = s + __shfl_xor(s, o);
    return s;
}

template <int G>
__device__ __forceinline__ void layer_norm_row(RowF<G>& r, const kr_half* __restrict__ w,
                                               const kr_half* __restrict__ b, int lane) {
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
        const kr_half4 wh = *reinterpret_cast<const kr_half4*>(w + 256 * i + 4 * lane);
        const kr_half4 bh = *reinterpret_cast<const kr_half4*>(b + 256 * i + 4 * lane);
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float y = (r.v[i][q] - mean) * rstd * (float)wh[q] + (float)bh[q];
            r.v[i][q] = (float)(kr_half)y;   // activations are fp16
        }
    }
}

template <int G>
__device__ __forceinline__ void store_row(kr_half* __restrict__ p, int lane, const RowF<G>& r) {
    #pragma unroll
    for (int i = 0; i < G; i++) {
        kr_half4 h;
        #pragma unroll
        for (int q = 0; q < 4; q++) h[q] = (kr_half)r.v[i][q];
        *reinterpret_cast<kr_half4*>(p + 256 * i + 4 * lane) = h;
    }
}

// mix = fp16(xx * tm + sx * (1 - tm))   (premix_kernels.cu:19-54 semantics)
template <int G>
__device__ __forceinline__ void store_mix(kr_half* __restrict__ out, const kr_half* __restrict__ tm,
                                          int lane, const RowF<G>& cur, const RowF<G>& prev) {
    #pragma unroll
    for (int i = 0; i < G; i++) {
        const kr_half4 t = *reinterpret_cast<const kr_half4*>(tm + 256 * i + 4 * lane);
        kr_half4 h;
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float m = (float)t[q];
            h[q] = (kr_half)(cur.v[i][q] * m + prev.v[i][q] * (1.0f - m));
        }
        *reinterpret_cast<kr_half4*>(out + 256 * i + 4 * lane) = h;
    }
}

struct LnMixArgs {
    const kr_half* x;          // [B*T, C]
    const kr_half* ln_w;
    const kr_half* ln_b;
    const kr_half* tm[3];      // NMIX coefficient vectors
    kr_half* out[3];           // NMIX outputs [B*T, C]
    kr_half* state;            // [B, C] shifted-in row for t = 0; rewritten with LN(x[T-1])
    int B, T, run;             // rows per wave
};

// One wave per run of `run` consecutive tokens of one stream. The wave that
// owns t = 0 reads the carried state first and rewrites it last (with the
// LayerNorm of row T-1), so no other wave touches the state.
// NMIX == 0: plain LayerNorm into out[0] (ln_out before the head).
template <int G, int NMIX>
__global__ void __launch_bounds__(256) ln_mix_kernel(LnMixArgs a) {
    constexpr int C = 256 * G;
    const int lane = threadIdx.x & 63;
    const int gw = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int runs = (a.T + a.run - 1) / a.run;
    if (gw >= a.B * runs) return;
    const int b = gw / runs, t0 = (gw % runs) * a.run;
    const int t1 = min(a.T, t0 + a.run);
    const size_t row0 = (size_t)b * a.T;

    RowF<G> prev, cur;
    if constexpr (NMIX > 0) {
        if (t0 == 0) {
            load_row<G>(a.state + (size_t)b * C, lane, prev);
        } else {
            load_row<G>(a.x + (row0 + t0 - 1) * C, lane, prev);
            layer_norm_row<G>(prev, a.ln_w, a.ln_b, lane);
        }
    }
    for (int t = t0; t < t1; t++) {
        load_row<G>(a.x + (row0 + t) * C, lane, cur);
        layer_norm_row<G>(cur, a.ln_w, a.ln_b, lane);
        if constexpr (NMIX == 0) {
            store_row<G>(a.out[0] + (row0 + t) * C, lane, cur);
        } else {
            #pragma unroll
            for (int m = 0; m < NMIX; m++)
                store_mix<G>(a.out[m] + (row0 + t) * C, a.tm[m], lane, cur, prev);
            prev = cur;
        }
    }
    if constexpr (NMIX > 0) {
        if (t0 == 0) {
            if (t1 < a.T) {
                load_row<G>(a.x + (row0 + a.T - 1) * C, lane, cur);
                layer_norm_row<G>(cur, a.ln_w, a.ln_b, lane);
            }
            store_row<G>(a.state + (size_t)b * C, lane, cur);
        }
    }
}

// ---------------------------------------------------------------------------
// WKV recurrence (wkv_kernel.cu:52-73 semantics), one lane per (stream,
// channel), sequential over T; fused with the receptance product:
// ry = fp16(r * fp16(y)). State aa, bb, pp is read once and written once.
// ---------------------------------------------------------------------------
constexpr int kWkvChunk = 8;

__global__ void __launch_bounds__(256) wkv_kernel(const float* __restrict__ k,
                                                  const float* __restrict__ v,
                                                  const kr_half* __restrict__ r,
                                                  const float* __restrict__ decay,
                                                  const float* __restrict__ first,
                                                  float* __restrict__ aa, float* __restrict__ bb,
                                                  float* __restrict__ pp, kr_half* __restrict__ ry,
                                                  int B, int T, int C) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= C || b >= B) return;
    const float w = decay[c], u = first[c];
    const size_t s = (size_t)b * C + c;
    float a_ = aa[s], b_ = bb[s], p_ = pp[s];
    const size_t base = (size_t)b * T * C + c;
    for (int t0 = 0; t0 < T; t0 += kWkvChunk) {
        float kk[kWkvChunk], vv[kWkvChunk], rr[kWkvChunk];
        #pragma unroll
        for (int q = 0; q < kWkvChunk; q++) {
            if (t0 + q < T) {
                const size_t i = base + (size_t)(t0 + q) * C;
                kk[q] = k[i];
                vv[q] = v[i];
                rr[q] = (float)r[i];
            }
        }
        #pragma unroll
        for (int q = 0; q < kWkvChunk; q++) {
            if (t0 + q < T) {
                const float ww = u + kk[q];
                const float p1 = fmaxf(p_, ww);
                const float e1 = __expf(p_ - p1), e2 = __expf(ww - p1);
                const float y = (e1 * a_ + e2 * vv[q]) / (e1 * b_ + e2);
                ry[base + (size_t)(t0 + q) * C] = (kr_half)(rr[q] * (float)(kr_half)y);
                const float ww2 = w + p_;
                const float p2 = fmaxf(ww2, kk[q]);
                const float f1 = __expf(ww2 - p2), f2 = __expf(kk[q] - p2);
                a_ = f1 * a_ + f2 * vv[q];
                b_ = f1 * b_ + f2;
                p_ = p2;
            }
        }
    }
    aa[s] = a_;
    bb[s] = b_;
    pp[s] = p_;
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
int launch_ln_mix(int G, const LnMixArgs& a, hipStream_t s) {
    const int runs = (a.T + a.run - 1) / a.run;
    const long long waves = (long long)a.B * runs;
    const int blocks = (int)((waves + 3) / 4);
    if (blocks == 0) return KR_OK;
    switch (G) {
        case 1: ln_mix_kernel<1, NMIX><<<blocks, 256, 0, s>>>(a); break;
        case 2: ln_mix_kernel<2, NMIX><<<blocks, 256, 0, s>>>(a); break;
        case 3: ln_mix_kernel<3, NMIX><<<blocks, 256, 0, s>>>(a); break;
        case 4: ln_mix_kernel<4, NMIX><<<blocks, 256, 0, s>>>(a); break;
        default: return kr_fail(KR_EUNSUPPORTED, "C=%d unsupported (256..1024, step 256)", 256 * G);
    }
    KR_LAUNCHED();
    return KR_OK;
}

// Workspace carve-up for M rows.
struct Work {
    kr_half *kx, *vx, *rx, *r, *ry, *fkx, *frx, *rf, *kf;
    float *k, *v;
};

inline size_t up256(size_t b) { return (b + 255) / 256 * 256; }

size_t work_bytes(long long M, int C, int F) {
    const size_t h = (size_t)M * C * 2, f = (size_t)M * C * 4, kf = (size_t)M * F * 2;
    return 8 * up256(h) + 2 * up256(f) + up256(kf);
}

Work carve(void* ws, long long M, int C, int F) {
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
    return w;
}

int rows_per_run(int T) { return T >= 64 ? 16 : (T >= 8 ? 4 : 1); }

kr_gemm_args gemm_args(const kr_half* A, int M, int K, const void* Wt, int N, void* out,
                       const kr_half* res = nullptr, const kr_half* gate = nullptr) {
    kr_gemm_args g{};
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

int layer_forward(const kr_layer_weights& L, int C, int F, kr_half* x, int B, int T,
                  const kr_layer_state& st, const Work& w, hipStream_t s) {
    const int M = B * T, G = C / 256;
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
    KR_TRY(launch_ln_mix<3>(G, a, s));
    {
        const kr_gemm_args jobs[3] = {gemm_args(w.kx, M, C, L.Kt, C, w.k),
                                      gemm_args(w.vx, M, C, L.Vt, C, w.v),
                                      gemm_args(w.rx, M, C, L.Rt, C, w.r)};
        const int eps[3] = {KR_EP_F32, KR_EP_F32, KR_EP_SIGMOID};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 3, s));
    }
    {
        dim3 grid((C + 255) / 256, B);
        wkv_kernel<<<grid, 256, 0, s>>>(w.k, w.v, w.r, L.decay, L.first, st.aa, st.bb, st.pp,
                                        w.ry, B, T, C);
        KR_LAUNCHED();
    }
    KR_TRY(kr_gemm_launch(gemm_args(w.ry, M, C, L.Ot, C, x, x), KR_EP_RESID, s));
    a.ln_w = H(L.ln2_w);
    a.ln_b = H(L.ln2_b);
    a.tm[0] = H(L.ftm_k); a.tm[1] = H(L.ftm_r);
    a.out[0] = w.fkx; a.out[1] = w.frx;
    a.state = Hm(st.ffn_xx);
    KR_TRY(launch_ln_mix<2>(G, a, s));
    {
        const kr_gemm_args jobs[2] = {gemm_args(w.frx, M, C, L.fRt, C, w.rf),
                                      gemm_args(w.fkx, M, C, L.fKt, F, w.kf)};
        const int eps[2] = {KR_EP_SIGMOID, KR_EP_RELUSQ};
        KR_TRY(kr_gemm_launch_multi(jobs, eps, 2, s));
    }
    KR_TRY(kr_gemm_launch(gemm_args(w.kf, M, F, L.fVt, C, x, x, w.rf), KR_EP_GATED, s));
    return KR_OK;
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

}  // namespace

// Entry points used by kr_engine.cpp.
int kr_impl_forward_layers(const kr_model_weights* m, void* x, int B, int T, void* state,
                           void* ws, size_t ws_bytes, hipStream_t s) {
    KR_TRY(check_model(m));
    KR_REQUIRE(x && state && ws, "forward: null pointer");
    const long long M = (long long)B * T;
    KR_REQUIRE(B >= 1 && T >= 1 && M <= (1ll << 31) / m->F, "forward: bad B=%d T=%d", B, T);
    KR_REQUIRE(ws_bytes >= work_bytes(M, m->C, m->F), "forward: workspace too small");
    const Work w = carve(ws, M, m->C, m->F);
    for (int i = 0; i < m->n_layer; i++)
        KR_TRY(layer_forward(m->layers[i], m->C, m->F, Hm(x), B, T, state_of(state, i, B, m->C),
                             w, s));
    return KR_OK;
}

// The layer stack for streams [b0, b0 + B) of a state buffer holding state_B
// streams (one group of a larger batch; rows of each [state_B, C] component).
int kr_impl_forward_layers_view(const kr_model_weights* m, void* x, int B, int T, void* state,
                                int state_B, int b0, void* ws, size_t ws_bytes, hipStream_t s) {
    KR_TRY(check_model(m));
    KR_REQUIRE(x && state && ws, "forward: null pointer");
    KR_REQUIRE(b0 >= 0 && B >= 1 && b0 + B <= state_B, "forward: bad stream range");
    const long long M = (long long)B * T;
    KR_REQUIRE(T >= 1 && M <= (1ll << 31) / m->F, "forward: bad T=%d", T);
    KR_REQUIRE(ws_bytes >= work_bytes(M, m->C, m->F), "forward: workspace too small");
    const Work w = carve(ws, M, m->C, m->F);
    const size_t off = (size_t)b0 * m->C;
    for (int i = 0; i < m->n_layer; i++) {
        kr_layer_state st = state_of(state, i, state_B, m->C);
        st.att_xx = static_cast<kr_half*>(st.att_xx) + off;
        st.ffn_xx = static_cast<kr_half*>(st.ffn_xx) + off;
        st.aa += off;
        st.bb += off;
        st.pp += off;
        KR_TRY(layer_forward(m->layers[i], m->C, m->F, Hm(x), B, T, st, w, s));
    }
    return KR_OK;
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
int kr_impl_head(const kr_model_weights* m, const void* x, int M, void* xn, void* logits,
                 long long ld, hipStream_t s) {
    if (M == 0) return KR_OK;
    LnMixArgs a{};
    a.x = H(x);
    a.ln_w = H(m->ln_out_w);
    a.ln_b = H(m->ln_out_b);
    a.out[0] = Hm(xn);
    a.B = M;
    a.T = 1;
    a.run = 1;
    KR_TRY(launch_ln_mix<0>(m->C / 256, a, s));
    kr_gemm_args g{};
    g.A = H(xn);
    g.lda = m->C;
    g.Wt = H(m->headT);
    g.ldw = m->C;
    g.out = logits;
    g.ldo = ld;
    g.res = nullptr;
    g.gate = nullptr;
    g.M = M;
    g.N = m->V;
    g.K = m->C;
    return kr_gemm_launch(g, KR_EP_F16, s);
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
    return layer_forward(*L, C, F, Hm(x), B, T, st, carve(ws, M, C, F), kr_stream(stream));
}

int kr_wkv(int B, int T, int C, const float* decay, const float* first, const float* k,
           const float* v, const uint16_t* r, float* aa, float* bb, float* pp, uint16_t* ry,
           void* stream) {
    KR_REQUIRE(decay && first && k && v && r && aa && bb && pp && ry, "kr_wkv: null pointer");
    KR_REQUIRE(B >= 1 && T >= 0 && C >= 1, "kr_wkv: bad shape");
    if (T == 0) return KR_OK;
    dim3 grid((C + 255) / 256, B);
    wkv_kernel<<<grid, 256, 0, kr_stream(stream)>>>(k, v, reinterpret_cast<const kr_half*>(r),
                                                    decay, first, aa, bb, pp,
                                                    reinterpret_cast<kr_half*>(ry), B, T, C);
    KR_LAUNCHED();
    return KR_OK;
}

}  // extern "C"
