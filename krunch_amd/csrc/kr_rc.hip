// Range-coder kernels and their C-ABI entry points.
//
// One lane per independent stream; the coder is serial within a stream. The
// entry points keep the reference's argument meaning and state layout
// (krunch_ac/cuda/main.cpp encode_step / decode_step and their _batched
// forms; encode_kernel.cu, decode_kernel.cu) and add buffer bounds: output
// writes stop at out_cap, input reads past a stream's limit return zeros.
#include "kr_rc_device.h"

namespace {

constexpr int kRcThreads = 64;

__device__ __forceinline__ uint32_t stream_base(const int32_t* base, int b) {
    return base ? (uint32_t)base[b] : 0u;
}

__device__ __forceinline__ void note_overflow(uint32_t* err, uint32_t overflow) {
    if (overflow && err) atomicOr(err, 1u);
}

// Symbols outside [0, V) would index past a CDF row: clamp and flag (bit 1).
__device__ __forceinline__ int checked_symbol(int s, int V, uint32_t* err) {
    if (s < 0 || s >= V) {
        if (err) atomicOr(err, 2u);
        return 0;
    }
    return s;
}

// N rows of one stream, full CDF rows (cdf_stride entries per row).
__global__ void rc_encode_rows_kernel(const int32_t* __restrict__ cdf, int cdf_stride,
                                      const int32_t* __restrict__ symbols, int N,
                                      uint8_t* __restrict__ out, uint32_t out_cap,
                                      kr_rc_state* state, int prec, uint32_t* err) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    uint32_t low = state->low, high = state->high, pending = state->pending_or_value;
    kr_bit_sink sink;
    sink.open(out, state->bit_offset, out_cap);
    for (int i = 0; i < N; i++) {
        const int32_t* row = cdf + (size_t)i * (size_t)cdf_stride;
        const int s = checked_symbol(symbols[i], cdf_stride - 1, err);
        kr_rc_encode(low, high, pending, (uint32_t)row[s], (uint32_t)row[s + 1], prec, sink);
    }
    state->bit_offset = sink.close();
    state->low = low;
    state->high = high;
    state->pending_or_value = pending;
    note_overflow(err, sink.overflow);
}

// One symbol per stream, CDF rows [B, V+1].
__global__ void rc_encode_step_batched_kernel(const int32_t* __restrict__ cdfs, int V,
                                              const int32_t* __restrict__ symbols,
                                              uint8_t* __restrict__ out, uint32_t out_cap,
                                              const int32_t* __restrict__ base,
                                              kr_rc_state* states, int B, int prec,
                                              uint32_t* err) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const uint32_t o = stream_base(base, b);
    const int32_t* row = cdfs + (size_t)b * (size_t)(V + 1);
    kr_rc_state st = states[b];
    kr_bit_sink sink;
    sink.open(out + o, st.bit_offset, out_cap > o ? out_cap - o : 0u);
    const int s = checked_symbol(symbols[b], V, err);
    kr_rc_encode(st.low, st.high, st.pending_or_value, (uint32_t)row[s], (uint32_t)row[s + 1],
                 prec, sink);
    st.bit_offset = sink.close();
    states[b] = st;
    note_overflow(err, sink.overflow);
}

// T symbols per stream from precomputed intervals: pairs[b*pair_stride + t] =
// (cdf[sym], cdf[sym+1]). Equivalent to T calls of the batched step.
__global__ void rc_encode_pairs_kernel(const uint2* __restrict__ pairs, int T,
                                       long long pair_stride, const int32_t* __restrict__ n_valid,
                                       uint8_t* __restrict__ out, uint32_t out_cap,
                                       const int32_t* __restrict__ base, kr_rc_state* states,
                                       int B, int prec, uint32_t* err) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    int n = T;
    if (n_valid) n = max(0, min(T, (int)n_valid[b]));
    if (n == 0) return;
    const uint32_t o = stream_base(base, b);
    kr_rc_state st = states[b];
    kr_bit_sink sink;
    sink.open(out + o, st.bit_offset, out_cap > o ? out_cap - o : 0u);
    const uint2* p = pairs + (size_t)b * (size_t)pair_stride;
    for (int t = 0; t < n; t++) {
        const uint2 iv = p[t];
        kr_rc_encode(st.low, st.high, st.pending_or_value, iv.x, iv.y, prec, sink);
    }
    st.bit_offset = sink.close();
    states[b] = st;
    note_overflow(err, sink.overflow);
}

__global__ void rc_encode_finalize_kernel(uint8_t* __restrict__ out, uint32_t out_cap,
                                          const int32_t* __restrict__ base, kr_rc_state* states,
                                          int B, uint32_t* err) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const uint32_t o = stream_base(base, b);
    kr_rc_state st = states[b];
    kr_bit_sink sink;
    sink.open(out + o, st.bit_offset, out_cap > o ? out_cap - o : 0u);
    kr_rc_flush(st.low, st.pending_or_value, sink);
    st.bit_offset = sink.close();
    st.pending_or_value = 0;
    states[b] = st;
    note_overflow(err, sink.overflow);
}

__device__ __forceinline__ kr_bit_source open_source(const uint8_t* in, uint32_t in_len,
                                                     const int32_t* base, const int32_t* limits,
                                                     int b, uint32_t bitpos) {
    kr_bit_source src;
    const uint32_t o = stream_base(base, b);
    uint32_t lim = in_len > o ? in_len - o : 0u;
    if (limits && (uint32_t)limits[b] < lim) lim = (uint32_t)limits[b];
    src.buf = in + (o < in_len ? o : 0u);
    src.limit = lim;
    src.pos = bitpos;
    return src;
}

__global__ void rc_decode_init_kernel(const uint8_t* __restrict__ in, uint32_t in_len,
                                      const int32_t* __restrict__ base,
                                      const int32_t* __restrict__ limits, kr_rc_state* states,
                                      int B) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    kr_bit_source src = open_source(in, in_len, base, limits, b, 0u);
    uint32_t value = 0;
    for (int i = 0; i < 32; i++) value = (value << 1) | src.get();
    kr_rc_state st;
    st.low = 0;
    st.high = 0xFFFFFFFFu;
    st.pending_or_value = value;
    st.bit_offset = src.pos;
    states[b] = st;
}

__global__ void rc_decode_step_kernel(const int32_t* __restrict__ cdfs, int V,
                                      const uint8_t* __restrict__ in, uint32_t in_len,
                                      const int32_t* __restrict__ base,
                                      const int32_t* __restrict__ limits, kr_rc_state* states,
                                      int32_t* __restrict__ out_syms, int B, int prec) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int32_t* row = cdfs + (size_t)b * (size_t)(V + 1);
    kr_rc_state st = states[b];
    kr_bit_source src = open_source(in, in_len, base, limits, b, st.bit_offset);
    const uint32_t target = kr_rc_target(st.low, st.high, st.pending_or_value, prec);
    int lo = 0, hi = V;                 // largest sym with cdf[sym] <= target
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)row[mid + 1] <= target) lo = mid + 1;
        else hi = mid;
    }
    const int sym = lo < V ? lo : V - 1;
    out_syms[b] = sym;
    kr_rc_consume(st.low, st.high, st.pending_or_value, (uint32_t)row[sym],
                  (uint32_t)row[sym + 1], prec, src);
    st.bit_offset = src.pos;
    states[b] = st;
}

inline int blocks_for(int B) { return (B + kRcThreads - 1) / kRcThreads; }

}  // namespace

extern "C" {

int kr_encode_step(const int32_t* cdf, int cdf_stride, const int32_t* symbols, int N,
                   uint8_t* output_buf, uint32_t out_cap, uint32_t* state, int cdf_precision,
                   uint32_t* err_flag, void* stream) {
    KR_REQUIRE(cdf && symbols && output_buf && state, "kr_encode_step: null pointer");
    KR_REQUIRE(N >= 0 && cdf_stride >= 2, "kr_encode_step: bad N=%d or stride=%d", N, cdf_stride);
    KR_REQUIRE(cdf_precision >= 1 && cdf_precision <= 31, "bad cdf_precision %d", cdf_precision);
    if (N == 0) return KR_OK;
    rc_encode_rows_kernel<<<1, 1, 0, kr_stream(stream)>>>(
        cdf, cdf_stride, symbols, N, output_buf, out_cap, reinterpret_cast<kr_rc_state*>(state),
        cdf_precision, err_flag);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_encode_finalize(uint8_t* output_buf, uint32_t out_cap, uint32_t* state,
                       uint32_t* err_flag, void* stream) {
    KR_REQUIRE(output_buf && state, "kr_encode_finalize: null pointer");
    rc_encode_finalize_kernel<<<1, kRcThreads, 0, kr_stream(stream)>>>(
        output_buf, out_cap, nullptr, reinterpret_cast<kr_rc_state*>(state), 1, err_flag);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_encode_step_batched(const int32_t* cdfs, int V, const int32_t* symbols,
                           uint8_t* output_buf, uint32_t out_cap,
                           const int32_t* base_byte_offsets, uint32_t* states, int B,
                           int cdf_precision, uint32_t* err_flag, void* stream) {
    KR_REQUIRE(cdfs && symbols && output_buf && base_byte_offsets && states,
               "kr_encode_step_batched: null pointer");
    KR_REQUIRE(V >= 1 && B >= 0, "kr_encode_step_batched: bad V=%d B=%d", V, B);
    if (B == 0) return KR_OK;
    rc_encode_step_batched_kernel<<<blocks_for(B), kRcThreads, 0, kr_stream(stream)>>>(
        cdfs, V, symbols, output_buf, out_cap, base_byte_offsets,
        reinterpret_cast<kr_rc_state*>(states), B, cdf_precision, err_flag);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_encode_pairs_batched(const uint32_t* pairs, int T, long long pair_stride,
                            const int32_t* n_valid, uint8_t* output_buf, uint32_t out_cap,
                            const int32_t* base_byte_offsets, uint32_t* states, int B,
                            int cdf_precision, uint32_t* err_flag, void* stream) {
    KR_REQUIRE(pairs && output_buf && states, "kr_encode_pairs_batched: null pointer");
    KR_REQUIRE(T >= 0 && B >= 0 && pair_stride >= T, "kr_encode_pairs_batched: bad shape");
    if (B == 0 || T == 0) return KR_OK;
    rc_encode_pairs_kernel<<<blocks_for(B), kRcThreads, 0, kr_stream(stream)>>>(
        reinterpret_cast<const uint2*>(pairs), T, pair_stride, n_valid, output_buf, out_cap,
        base_byte_offsets, reinterpret_cast<kr_rc_state*>(states), B, cdf_precision, err_flag);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_encode_finalize_batched(uint8_t* output_buf, uint32_t out_cap,
                               const int32_t* base_byte_offsets, uint32_t* states, int B,
                               uint32_t* err_flag, void* stream) {
    KR_REQUIRE(output_buf && states, "kr_encode_finalize_batched: null pointer");
    if (B == 0) return KR_OK;
    rc_encode_finalize_kernel<<<blocks_for(B), kRcThreads, 0, kr_stream(stream)>>>(
        output_buf, out_cap, base_byte_offsets, reinterpret_cast<kr_rc_state*>(states), B,
        err_flag);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_decode_init_batched(const uint8_t* input_buf, uint32_t in_len,
                           const int32_t* base_byte_offsets, const int32_t* byte_limits,
                           uint32_t* states, int B, void* stream) {
    KR_REQUIRE(input_buf && states, "kr_decode_init_batched: null pointer");
    if (B == 0) return KR_OK;
    rc_decode_init_kernel<<<blocks_for(B), kRcThreads, 0, kr_stream(stream)>>>(
        input_buf, in_len, base_byte_offsets, byte_limits, reinterpret_cast<kr_rc_state*>(states),
        B);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_decode_step_batched(const int32_t* cdfs, int V, const uint8_t* input_buf, uint32_t in_len,
                           const int32_t* base_byte_offsets, const int32_t* byte_limits,
                           uint32_t* states, int32_t* out_syms, int B, int cdf_precision,
                           void* stream) {
    KR_REQUIRE(cdfs && input_buf && states && out_syms, "kr_decode_step_batched: null pointer");
    KR_REQUIRE(V >= 1, "kr_decode_step_batched: bad V=%d", V);
    if (B == 0) return KR_OK;
    rc_decode_step_kernel<<<blocks_for(B), kRcThreads, 0, kr_stream(stream)>>>(
        cdfs, V, input_buf, in_len, base_byte_offsets, byte_limits,
        reinterpret_cast<kr_rc_state*>(states), out_syms, B, cdf_precision);
    KR_LAUNCHED();
    return KR_OK;
}

}  // extern "C"
