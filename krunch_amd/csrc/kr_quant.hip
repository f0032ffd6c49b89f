// w8a8 quantisation: symmetric int8 with fp32 scales,
// one scale per row. Used for the weights (rows of W^T = output channels) at
// preparation time and for activations (rows = tokens) on the fly.
//
//   amax = max_k |x[k]|;  s = amax / 127;  inv = 127 / amax   (s = inv = 1
//   when amax = 0; IEEE divides)
//   q[k] = round(x[k] * inv), the exact product rounded to the nearest
//          integer, ties to even (kr_q8_bits in kr_gemm.h: one FMA)
//
// so the int8 GEMM value (float(sum q_a q_w) * s_a) * s_w approximates x @ W.
// The output is row-major [M, K] int8 or fragment-packed (kr_frag_index_i8),
// the operand layout of the small-M int8 GEMM.
#include "kr_gemm.h"
#include "kr_wave.h"

namespace {

__device__ __forceinline__ float wave_maxf(float v) {
    v = kr_wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
    return v;
}


// One wave per row; lane l owns the 4-column groups at 256*i + 4*l.
__global__ void __launch_bounds__(256) row_quant_kernel(const kr_half* __restrict__ x, long long ldx,
                                                        int M, int K, int8_t* __restrict__ q,
                                                        float* __restrict__ scales, int packed) {
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= M) return;
    const kr_half* xr = x + (size_t)row * (size_t)ldx;
    float amax = 0.0f;
    for (int c = 4 * lane; c < K; c += 256) {
        const kr_half4 h = *reinterpret_cast<const kr_half4*>(xr + c);
        #pragma unroll
        for (int r = 0; r < 4; r++) amax = fmaxf(amax, fabsf((float)h[r]));
    }
    amax = wave_maxf(amax);
    const float inv = kr_q8_inv(amax);
    for (int c = 4 * lane; c < K; c += 256) {
        const kr_half4 h = *reinterpret_cast<const kr_half4*>(xr + c);
        const size_t o = packed ? kr_frag_index_i8(row, c, K) : (size_t)row * (size_t)K + c;
        *reinterpret_cast<uint32_t*>(q + o) =
            kr_q8_pack4((float)h[0], (float)h[1], (float)h[2], (float)h[3], inv);
    }
    if (lane == 0) scales[row] = kr_q8_scale(amax);
}

// K = 256 KI: the lane's KI groups are loaded together and kept in
// registers, so a row costs one memory round trip (the loop above waits for
// each load in turn and reads the row twice). Same operations, same bits.
template <int KI>
__global__ void __launch_bounds__(256) row_quant_reg_kernel(const kr_half* __restrict__ x,
                                                            long long ldx, int M,
                                                            int8_t* __restrict__ q,
                                                            float* __restrict__ scales, int packed) {
    constexpr int K = 256 * KI;
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (row >= M) return;
    const kr_half* xr = x + (size_t)row * (size_t)ldx;
    kr_half4 h[KI];
    #pragma unroll
    for (int i = 0; i < KI; i++) h[i] = *reinterpret_cast<const kr_half4*>(xr + 256 * i + 4 * lane);
    float amax = 0.0f;
    #pragma unroll
    for (int i = 0; i < KI; i++)
        #pragma unroll
        for (int r = 0; r < 4; r++) amax = fmaxf(amax, fabsf((float)h[i][r]));
    amax = wave_maxf(amax);
    const float inv = kr_q8_inv(amax);
    #pragma unroll
    for (int i = 0; i < KI; i++) {
        const int c = 256 * i + 4 * lane;
        const size_t o = packed ? kr_frag_index_i8(row, c, K) : (size_t)row * (size_t)K + c;
        *reinterpret_cast<uint32_t*>(q + o) =
            kr_q8_pack4((float)h[i][0], (float)h[i][1], (float)h[i][2], (float)h[i][3], inv);
    }
    if (lane == 0) scales[row] = kr_q8_scale(amax);
}

}  // namespace

int kr_impl_quantize_rows(const void* x, long long ldx, int M, int K, void* q, float* scales,
                          int packed, hipStream_t s) {
    KR_REQUIRE(x && q && scales && M >= 0 && K >= 64 && K % 64 == 0 && ldx >= K && ldx % 4 == 0,
               "quantize: bad args (K must be a multiple of 64)");
    KR_REQUIRE(((uintptr_t)x & 7) == 0 && ((uintptr_t)q & 3) == 0, "quantize: misaligned pointer");
    if (M == 0) return KR_OK;
    const kr_half* xh = reinterpret_cast<const kr_half*>(x);
    int8_t* q8 = reinterpret_cast<int8_t*>(q);
    const int grid = (M + 3) / 4;
    switch (K % 256 == 0 ? K / 256 : 0) {
#define KR_RQ(KI_) \
        case KI_: row_quant_reg_kernel<KI_><<<grid, 256, 0, s>>>(xh, ldx, M, q8, scales, packed); break;
        KR_RQ(1) KR_RQ(2) KR_RQ(3) KR_RQ(4) KR_RQ(6) KR_RQ(8) KR_RQ(12)
#undef KR_RQ
        default: row_quant_kernel<<<grid, 256, 0, s>>>(xh, ldx, M, K, q8, scales, packed); break;
    }
    KR_LAUNCHED();
    return KR_OK;
}

extern "C" {

size_t kr_quant_bytes(int M, int K, int packed) {
    if (M < 0 || K < 64 || K % 64) return 0;
    return (size_t)(packed ? kr_frag_rows(M) : M) * (size_t)K;
}

int kr_quantize_rows(const uint16_t* x, long long ldx, int M, int K, int8_t* q, float* scales,
                     int packed, void* stream) {
    return kr_impl_quantize_rows(x, ldx, M, K, q, scales, packed, kr_stream(stream));
}

int kr_det_matmul_i8(const int8_t* xq, const float* sa, int M, int K, const int8_t* wq,
                     const float* sw, int N, void* out, long long ldo, int epilogue,
                     const uint16_t* res, const uint16_t* gate, int packed, void* stream) {
    KR_REQUIRE(packed >= 0 && packed <= 2, "kr_det_matmul_i8: packed must be 0, 1 or 2");
    kr_gemm_args g{};
    g.A = reinterpret_cast<const kr_half*>(xq);
    g.lda = K;
    if (packed) g.Wf = reinterpret_cast<const kr_half*>(wq);
    else g.Wt = reinterpret_cast<const kr_half*>(wq);
    g.ldw = K;
    g.out = out;
    g.ldo = ldo;
    g.res = reinterpret_cast<const kr_half*>(res);
    g.gate = reinterpret_cast<const kr_half*>(gate);
    g.M = M;
    g.N = N;
    g.K = K;
    g.a_frag = packed ? 1 : 0;
    g.a_q16 = packed == 2 ? 1 : 0;
    g.i8 = 1;
    g.sa = sa;
    g.sw = sw;
    return kr_gemm_launch(g, epilogue, kr_stream(stream));
}

}  // extern "C"
