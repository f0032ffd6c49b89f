// Model-level entry points: packed compress windows and stepped, fused
// decode steps (optionally replayed from one captured HIP graph), plus the
// error/introspection calls of the C ABI.
//
// Compress follows InferenceEngine._compress_chunk_cpp (krunch/inference.py:
// 293-361) generalised to B chunks per call (the layer op accepts [B,T,C],
// layer_cpp.cpp:469-474): embed -> layers -> per row block (head GEMM ->
// softmax/CDF -> symbol interval). Decompress follows
// _decompress_chunks_batched_cpp (inference.py:363-443): per step embed the
// previous symbols -> layers (T = 1) -> head -> fused CDF search + range
// decode; decoded symbols never leave the GPU.
#include <stdarg.h>
#include <stdio.h>
#include <string>

#include "kr_model.h"

// ids (nullable): x starts as the embedding of these token ids, gathered by
// layer 0's LN1-mix, which also writes x.
int kr_impl_forward_layers(const kr_model_weights* m, void* x, int B, int T, void* state,
                           void* ws, size_t ws_bytes, hipStream_t s, const int32_t* ids);
int kr_impl_forward_layers_view(const kr_model_weights* m, void* x, int B, int T, void* state,
                                int state_B, int b0, void* ws, size_t ws_bytes, hipStream_t s,
                                const int32_t* ids, bool l0_mixed);
bool kr_impl_embed_mix_args(const kr_model_weights* m, int B, void* state, int state_B, int b0,
                            void* ws, void* x, bool first, kr_embed_mix* em, kr_embed_mix** dev);
int kr_impl_cdf_decode(const uint16_t* logits, int B, int V, long long ld,
                       const uint8_t* input_buf, uint32_t in_len,
                       const int32_t* base_byte_offsets, const int32_t* byte_limits,
                       uint32_t* states, int32_t* out_syms, int32_t* tokens,
                       long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                       int cdf_precision, const kr_embed_mix* em, void* stream);
int kr_impl_embed(const kr_model_weights* m, const int32_t* ids, int M, void* x, hipStream_t s);
// xn_rows16: xn holds M rounded up to 16 rows (allows the small-M head).
int kr_impl_head(const kr_model_weights* m, const void* x, int M, void* xn, void* logits,
                 long long ld, hipStream_t s, bool xn_rows16);
size_t kr_impl_work_bytes(long long M, int C, int F);
void* kr_impl_head_scratch(void* ws, long long M, int C, int F);

extern "C" {
int kr_softmax_cdf_pairs(const uint16_t* logits, int N, int V, long long ld,
                         const int32_t* symbols, uint32_t* pairs, int cdf_precision,
                         void* stream);
int kr_probs_to_cdf(const float* probs, int N, int V, long long ld, uint32_t* cdf_out,
                    int cdf_precision, void* stream);
}

namespace {
thread_local std::string g_err;
}

int kr_fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define KR_TRY(expr)              \
    do {                          \
        int kr_rc_ = (expr);      \
        if (kr_rc_) return kr_rc_; \
    } while (0)

namespace {

struct DecodeStepArgs {
    const kr_model_weights* m;
    int B;
    void* state;
    int32_t* syms;
    void* x;
    void* ws;
    size_t ws_bytes;
    void* logits;
    long long ld;
    const uint8_t* in;
    uint32_t in_len;
    const int32_t* base;
    const int32_t* limits;
    uint32_t* ac_states;
    int32_t* tokens;
    long long tok_stride;
    int32_t* tok_count;
    const int32_t* n_tokens;
    int prec;
    int state_B;   // streams held by `state` (>= b0 + B)
    int b0;        // first stream of this call within `state`
};

// em (device copy of a kr_embed_mix): the decode kernel also runs layer 0's
// LN1-mix of the decoded symbols for the next step; l0_mixed: the previous
// step's decode kernel did that, so this step starts at layer 0's K, V, R
// products.
int decode_step(const DecodeStepArgs& a, hipStream_t s, const kr_embed_mix* em = nullptr,
                bool l0_mixed = false) {
    KR_TRY(kr_impl_forward_layers_view(a.m, a.x, a.B, 1, a.state, a.state_B, a.b0, a.ws,
                                       a.ws_bytes, s, a.syms, l0_mixed));
    void* xn = kr_impl_head_scratch(a.ws, a.B, a.m->C, a.m->F);
    KR_TRY(kr_impl_head(a.m, a.x, a.B, xn, a.logits, a.ld, s, true));
    return kr_impl_cdf_decode(reinterpret_cast<const uint16_t*>(a.logits), a.B, a.m->V, a.ld,
                              a.in, a.in_len, a.base, a.limits, a.ac_states, a.syms, a.tokens,
                              a.tok_stride, a.tok_count, a.n_tokens, a.prec, em, s);
}

int check_decode(const DecodeStepArgs& a) {
    KR_REQUIRE(a.m && a.state && a.syms && a.x && a.ws && a.logits && a.in && a.ac_states,
               "decode: null pointer");
    KR_REQUIRE(a.B >= 1, "decode: bad B=%d", a.B);
    KR_REQUIRE(a.ld >= a.m->V, "decode: logits ld %lld < V %d", a.ld, a.m->V);
    KR_REQUIRE(a.ws_bytes >= kr_impl_work_bytes(a.B, a.m->C, a.m->F), "decode: workspace too small");
    KR_REQUIRE(!a.tokens || a.tok_count, "decode: tokens need tok_count");
    return KR_OK;
}

}  // namespace

extern "C" {

const char* kr_last_error(void) { return g_err.c_str(); }

int kr_abi_version(void) { return 2; }

size_t kr_forward_workspace_bytes(long long M, int C, int F) {
    return kr_impl_work_bytes(M, C, F);
}

int kr_forward_layers(const kr_model_weights* m, void* x, int B, int T, void* state, void* ws,
                      size_t ws_bytes, void* stream) {
    return kr_impl_forward_layers(m, x, B, T, state, ws, ws_bytes, kr_stream(stream), nullptr);
}

int kr_embed(const kr_model_weights* m, const int32_t* ids, int M, void* x, void* stream) {
    KR_REQUIRE(m && ids && x && M >= 0, "kr_embed: bad args");
    return kr_impl_embed(m, ids, M, x, kr_stream(stream));
}

int kr_head_logits(const kr_model_weights* m, const void* x, int M, void* xn, void* logits,
                   long long ld, void* stream) {
    KR_REQUIRE(m && x && xn && logits && M >= 0 && ld >= m->V, "kr_head_logits: bad args");
    return kr_impl_head(m, x, M, xn, logits, ld, kr_stream(stream), M % 16 == 0);
}

int kr_compress_window(const kr_model_weights* m, const int32_t* inputs, const int32_t* targets,
                       int B, int T, void* state, void* x, void* ws, size_t ws_bytes,
                       void* logits, long long ld, int head_rows, uint32_t* pairs,
                       int cdf_precision, void* stream) {
    KR_REQUIRE(m && inputs && targets && state && x && ws && logits && pairs,
               "kr_compress_window: null pointer");
    KR_REQUIRE(B >= 1 && T >= 1 && head_rows >= 1 && ld >= m->V, "kr_compress_window: bad shape");
    const long long M = (long long)B * T;
    KR_REQUIRE(ws_bytes >= kr_impl_work_bytes(M, m->C, m->F), "kr_compress_window: workspace too small");
    hipStream_t s = kr_stream(stream);
    KR_TRY(kr_impl_forward_layers(m, x, B, T, state, ws, ws_bytes, s, inputs));
    void* xn = kr_impl_head_scratch(ws, M, m->C, m->F);
    for (long long r0 = 0; r0 < M; r0 += head_rows) {
        const int n = (int)((M - r0) < head_rows ? (M - r0) : head_rows);
        const void* xr = static_cast<const char*>(x) + (size_t)r0 * m->C * 2;
        void* xnr = static_cast<char*>(xn) + (size_t)r0 * m->C * 2;
        KR_TRY(kr_impl_head(m, xr, n, xnr, logits, ld, s, head_rows % 16 == 0));
        KR_TRY(kr_softmax_cdf_pairs(reinterpret_cast<const uint16_t*>(logits), n, m->V, ld,
                                    targets + r0, pairs + 2 * r0, cdf_precision, stream));
    }
    return KR_OK;
}

int kr_decode_step(const kr_model_weights* m, int B, void* state, int32_t* syms, void* x,
                   void* ws, size_t ws_bytes, void* logits, long long ld, const uint8_t* input_buf,
                   uint32_t in_len, const int32_t* base_byte_offsets, const int32_t* byte_limits,
                   uint32_t* ac_states, int32_t* tokens, long long tok_stride, int32_t* tok_count,
                   const int32_t* n_tokens, int cdf_precision, void* stream) {
    DecodeStepArgs a{m, B, state, syms, x, ws, ws_bytes, logits, ld, input_buf, in_len,
                     base_byte_offsets, byte_limits, ac_states, tokens, tok_stride, tok_count,
                     n_tokens, cdf_precision, B, 0};
    KR_TRY(check_decode(a));
    return decode_step(a, kr_stream(stream));
}

size_t kr_decode_workspace_bytes(int B, int n_groups, int C, int F) {
    if (B < 1 || n_groups < 1) return 0;
    const int G = n_groups > B ? B : n_groups;
    const int Bg = (B + G - 1) / G;
    const size_t per = (kr_impl_work_bytes(Bg, C, F) + 255) / 256 * 256;
    return per * (size_t)G;
}

int kr_decode_run(const kr_model_weights* m, int B, void* state, int32_t* syms, void* x,
                  void* ws, size_t ws_bytes, void* logits, long long ld, const uint8_t* input_buf,
                  uint32_t in_len, const int32_t* base_byte_offsets, const int32_t* byte_limits,
                  uint32_t* ac_states, int32_t* tokens, long long tok_stride, int32_t* tok_count,
                  const int32_t* n_tokens, int cdf_precision, int n_steps, int n_groups,
                  int use_graph, void* stream) {
    KR_REQUIRE(m && B >= 1 && n_groups >= 1 && n_groups <= 16, "kr_decode_run: bad B/n_groups");
    KR_REQUIRE(n_steps >= 0, "kr_decode_run: bad n_steps");
    const int G = n_groups > B ? B : n_groups;
    const int Bg = (B + G - 1) / G;
    const size_t per_ws = (kr_impl_work_bytes(Bg, m->C, m->F) + 255) / 256 * 256;
    KR_REQUIRE(ws_bytes >= per_ws * G, "kr_decode_run: workspace too small (need %zu)", per_ws * G);
    // One argument set per group of streams [b0, b0 + Bg).
    DecodeStepArgs grp[16];
    int ng = 0;
    for (int b0 = 0; b0 < B; b0 += Bg, ng++) {
        const int n = B - b0 < Bg ? B - b0 : Bg;
        DecodeStepArgs a{m, n, state, syms + b0,
                         static_cast<char*>(x) + (size_t)b0 * m->C * 2,
                         static_cast<char*>(ws) + per_ws * ng, per_ws,
                         static_cast<char*>(logits) + (size_t)b0 * ld * 2, ld, input_buf, in_len,
                         base_byte_offsets ? base_byte_offsets + b0 : nullptr,
                         byte_limits ? byte_limits + b0 : nullptr, ac_states + 4 * (size_t)b0,
                         tokens ? tokens + (size_t)b0 * tok_stride : nullptr, tok_stride,
                         tok_count ? tok_count + b0 : nullptr, n_tokens ? n_tokens + b0 : nullptr,
                         cdf_precision, B, b0};
        KR_TRY(check_decode(a));
        grp[ng] = a;
    }
    hipStream_t s = kr_stream(stream);
    if (n_steps == 0) return KR_OK;
    if (!use_graph) {
        for (int i = 0; i < n_steps; i++)
            for (int g = 0; g < ng; g++) KR_TRY(decode_step(grp[g], s));
        return KR_OK;
    }
    // Warm per-V caches (CDF summation plan) outside the capture: a
    // zero-row launch builds the plan without running a kernel.
    KR_TRY(kr_probs_to_cdf(reinterpret_cast<const float*>(logits), 0, m->V, m->V, ac_states,
                           cdf_precision, stream));
    // One stream group (the default): layer 0's LN1-mix of each decoded
    // symbol runs in the decode kernel of the step that decoded it, so every
    // step after the first starts at layer 0's K, V, R products (one launch
    // fewer per step). Two graphs: the first step, and the later steps.
    kr_embed_mix em_first{}, em_next{};
    kr_embed_mix *dev_first = nullptr, *dev_next = nullptr;
    const bool fold = ng == 1 &&
                      kr_impl_embed_mix_args(m, B, state, B, 0, grp[0].ws, grp[0].x, true,
                                             &em_first, &dev_first) &&
                      kr_impl_embed_mix_args(m, B, state, B, 0, grp[0].ws, grp[0].x, false,
                                             &em_next, &dev_next);
    // Several groups: one graph per step, the groups as independent branches
    // (fork/join through events), so their latency-bound kernels overlap.
    hipStream_t cap[16] = {};
    hipEvent_t ev[18] = {};
    hipGraph_t graph[2] = {};
    hipGraphExec_t exec[2] = {};
    int rc = KR_OK;
    bool capturing = false;
    auto cleanup = [&]() {
        if (capturing) {
            hipGraph_t g2 = nullptr;
            (void)hipStreamEndCapture(cap[0], &g2);
            if (g2) (void)hipGraphDestroy(g2);
        }
        for (auto& x : exec) if (x) (void)hipGraphExecDestroy(x);
        for (auto& g : graph) if (g) (void)hipGraphDestroy(g);
        for (auto& e : ev) if (e) (void)hipEventDestroy(e);
        for (auto& c : cap) if (c) (void)hipStreamDestroy(c);
    };
    auto hip_fail = [&](hipError_t e, const char* what) {
        rc = kr_fail(KR_EHIP, "kr_decode_run: %s: %s", what, hipGetErrorString(e));
        cleanup();
        return rc;
    };
    hipError_t e;
    for (int g = 0; g < ng; g++)
        if ((e = hipStreamCreateWithFlags(&cap[g], hipStreamNonBlocking)) != hipSuccess)
            return hip_fail(e, "stream");
    for (int i = 0; i < ng + 2; i++)
        if ((e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming)) != hipSuccess)
            return hip_fail(e, "event");
    if (fold) {
        if ((e = hipMemcpyAsync(dev_first, &em_first, sizeof em_first, hipMemcpyHostToDevice, s)) !=
                hipSuccess ||
            (e = hipMemcpyAsync(dev_next, &em_next, sizeof em_next, hipMemcpyHostToDevice, s)) !=
                hipSuccess)
            return hip_fail(e, "layer-0 mix arguments");
    }
    // ev[0]: caller -> capture stream; ev[1]: fork; ev[2+g]: join of group g; ev[ng+1] reused at the end
    if ((e = hipEventRecord(ev[0], s)) != hipSuccess) return hip_fail(e, "record");
    if ((e = hipStreamWaitEvent(cap[0], ev[0], 0)) != hipSuccess) return hip_fail(e, "wait");
    // graph i: step kind 0 (unfolded, or a folded run's first step) or 1 (a
    // folded run's later steps)
    auto capture = [&](int i) -> int {
        hipError_t ce;
        if ((ce = hipStreamBeginCapture(cap[0], hipStreamCaptureModeThreadLocal)) != hipSuccess)
            return hip_fail(ce, "begin capture");
        capturing = true;
        if ((ce = hipEventRecord(ev[1], cap[0])) != hipSuccess) return hip_fail(ce, "fork record");
        for (int g = 1; g < ng; g++)
            if ((ce = hipStreamWaitEvent(cap[g], ev[1], 0)) != hipSuccess) return hip_fail(ce, "fork wait");
        if (fold) rc = decode_step(grp[0], cap[0], i == 0 ? dev_first : dev_next, i == 1);
        else
            for (int g = 0; g < ng && rc == KR_OK; g++) rc = decode_step(grp[g], cap[g]);
        if (rc) { cleanup(); return rc; }
        for (int g = 1; g < ng; g++) {
            if ((ce = hipEventRecord(ev[1 + g], cap[g])) != hipSuccess) return hip_fail(ce, "join record");
            if ((ce = hipStreamWaitEvent(cap[0], ev[1 + g], 0)) != hipSuccess) return hip_fail(ce, "join wait");
        }
        ce = hipStreamEndCapture(cap[0], &graph[i]);
        capturing = false;
        if (ce != hipSuccess) return hip_fail(ce, "end capture");
        if ((ce = hipGraphInstantiate(&exec[i], graph[i], nullptr, nullptr, 0)) != hipSuccess)
            return hip_fail(ce, "instantiate");
        return KR_OK;
    };
    if (capture(0)) return rc;
    if (fold && n_steps > 1 && capture(1)) return rc;
    for (int i = 0; i < n_steps; i++)
        if ((e = hipGraphLaunch(exec[fold && i > 0 ? 1 : 0], cap[0])) != hipSuccess)
            return hip_fail(e, "graph launch");
    if ((e = hipEventRecord(ev[ng + 1], cap[0])) != hipSuccess) return hip_fail(e, "record");
    if ((e = hipStreamWaitEvent(s, ev[ng + 1], 0)) != hipSuccess) return hip_fail(e, "wait");
    if ((e = hipStreamSynchronize(cap[0])) != hipSuccess) return hip_fail(e, "sync");
    cleanup();
    return KR_OK;
}

}  // extern "C"
