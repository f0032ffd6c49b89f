// fp16 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x32_f16), LDS-staged.
//
// Replaces the reference's deterministic WMMA matmuls (det_matmul_tc*.cu,
// routed by layer_cpp.cpp:206-290 and :728-822) for both the packed
// compress forward (M = B*T rows) and the stepped decompress forward
// (M = B rows). Reduction contract: each output is acc = 0, then one MFMA
// per 32-wide K slice in increasing K order, fp32 accumulate; no split-K.
// Tile shape only changes which rows/columns a workgroup owns, never the
// per-element instruction sequence, so packed and stepped logits agree bit
// for bit.
//
// Workgroup: 256 threads = 4 waves in a 2x2 grid; wave tile (BM/2)x(BN/2)
// made of 16x16 MFMA tiles. K is staged 64 at a time through LDS (row pitch
// 72 halves so the 16 rows read by one ds_read_b128 land on distinct banks),
// with the next slice's global loads in flight during the MFMAs.
#include "kr_gemm.h"

namespace {

constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;

template <int EP>
__device__ __forceinline__ void store_one(const kr_gemm_args& g, int m, int n, float acc) {
    const size_t o = (size_t)m * (size_t)g.ldo + (size_t)n;
    if constexpr (EP == KR_EP_F32) {
        reinterpret_cast<float*>(g.out)[o] = acc;
    } else {
        const float h = (float)(kr_half)acc;
        float y;
        if constexpr (EP == KR_EP_F16) y = h;
        else if constexpr (EP == KR_EP_SIGMOID) y = kr_sigmoid(h);
        else if constexpr (EP == KR_EP_RELUSQ) { const float r = h > 0.0f ? h : 0.0f; y = r * r; }
        else if constexpr (EP == KR_EP_RESID) y = (float)g.res[o] + h;
        else {
            const float gh = (float)(kr_half)((float)g.gate[o] * h);
            y = (float)g.res[o] + gh;
        }
        reinterpret_cast<kr_half*>(g.out)[o] = (kr_half)y;
    }
}

template <int BM, int BN, int EP>
__global__ void __launch_bounds__(256) gemm_kernel(kr_gemm_args g) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int A_CHUNKS = BM * (kBK / 8) / 256;   // 16-byte chunks per thread
    constexpr int W_CHUNKS = BN * (kBK / 8) / 256;
    static_assert(A_CHUNKS >= 1 && W_CHUNKS >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) kr_half As[BM * kPitch];
    __shared__ __attribute__((aligned(16))) kr_half Ws[BN * kPitch];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    kr_half8 ra[A_CHUNKS], rw[W_CHUNKS];
    auto load_tiles = [&](int k0) {
        #pragma unroll
        for (int i = 0; i < A_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            const int m = m0 + r;
            if (m < g.M)
                ra[i] = *reinterpret_cast<const kr_half8*>(g.A + (size_t)m * g.lda + k0 + col);
            else
                ra[i] = kr_half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        #pragma unroll
        for (int i = 0; i < W_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            const int n = n0 + r;
            if (n < g.N)
                rw[i] = *reinterpret_cast<const kr_half8*>(g.Wt + (size_t)n * g.ldw + k0 + col);
            else
                rw[i] = kr_half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    };
    auto stash_tiles = [&]() {
        #pragma unroll
        for (int i = 0; i < A_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            *reinterpret_cast<kr_half8*>(&As[r * kPitch + col]) = ra[i];
        }
        #pragma unroll
        for (int i = 0; i < W_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            *reinterpret_cast<kr_half8*>(&Ws[r * kPitch + col]) = rw[i];
        }
    };

    kr_float4 acc[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = kr_float4{0.f, 0.f, 0.f, 0.f};

    const int KT = g.K / kBK;
    load_tiles(0);
    const int lrow = lane & 15, lk = (lane >> 4) * 8;
    for (int kt = 0; kt < KT; kt++) {
        __syncthreads();
        stash_tiles();
        __syncthreads();
        if (kt + 1 < KT) load_tiles((kt + 1) * kBK);
        #pragma unroll
        for (int ks = 0; ks < kBK; ks += 32) {
            kr_half8 a[TM], b[TN];
            #pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const kr_half8*>(
                    &As[(wm * WM + i * 16 + lrow) * kPitch + ks + lk]);
            #pragma unroll
            for (int j = 0; j < TN; j++)
                b[j] = *reinterpret_cast<const kr_half8*>(
                    &Ws[(wn * WN + j * 16 + lrow) * kPitch + ks + lk]);
            #pragma unroll
            for (int i = 0; i < TM; i++)
                #pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }

    // D layout of the 16x16 MFMA: lane holds rows 4*(lane/16) + r, column lane%16.
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int j = 0; j < TN; j++)
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * WM + i * 16 + (lane >> 4) * 4 + r;
                const int n = n0 + wn * WN + j * 16 + (lane & 15);
                if (m < g.M && n < g.N) store_one<EP>(g, m, n, acc[i][j][r]);
            }
}

template <int BM, int BN>
int launch_tile(const kr_gemm_args& g, int ep, hipStream_t s) {
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
    switch (ep) {
        case KR_EP_F32: gemm_kernel<BM, BN, KR_EP_F32><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_F16: gemm_kernel<BM, BN, KR_EP_F16><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_SIGMOID: gemm_kernel<BM, BN, KR_EP_SIGMOID><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RELUSQ: gemm_kernel<BM, BN, KR_EP_RELUSQ><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RESID: gemm_kernel<BM, BN, KR_EP_RESID><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_GATED: gemm_kernel<BM, BN, KR_EP_GATED><<<grid, 256, 0, s>>>(g); break;
        default: return kr_fail(KR_EINVAL, "unknown epilogue %d", ep);
    }
    KR_LAUNCHED();
    return KR_OK;
}

// Transpose W [K, N] -> Wt [N, K] (rows of Wt beyond N are not touched).
__global__ void transpose_kernel(const kr_half* __restrict__ W, long long ldw_in, int K, int N,
                                 kr_half* __restrict__ Wt, long long ldt) {
    __shared__ kr_half tile[32][33];
    const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, n = n0 + tx;
        if (k < K && n < N) tile[r][tx] = W[(size_t)k * ldw_in + n];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int n = n0 + r, k = k0 + tx;
        if (n < N && k < K) Wt[(size_t)n * ldt + k] = tile[tx][r];
    }
}

}  // namespace

int kr_gemm_launch(const kr_gemm_args& g, int ep, hipStream_t s) {
    KR_REQUIRE(g.A && g.Wt && g.out, "gemm: null pointer");
    KR_REQUIRE(g.M >= 0 && g.N >= 1 && g.K >= kBK && g.K % kBK == 0,
               "gemm: unsupported shape M=%d N=%d K=%d (K must be a multiple of %d)", g.M, g.N,
               g.K, kBK);
    KR_REQUIRE(g.lda % 8 == 0 && g.ldw % 8 == 0 && g.lda >= g.K && g.ldw >= g.K,
               "gemm: lda/ldw must be >= K and multiples of 8");
    KR_REQUIRE(((uintptr_t)g.A & 15) == 0 && ((uintptr_t)g.Wt & 15) == 0,
               "gemm: A and Wt must be 16-byte aligned");
    KR_REQUIRE(g.ldo >= g.N, "gemm: ldo < N");
    KR_REQUIRE((ep != KR_EP_RESID && ep != KR_EP_GATED) || g.res, "gemm: residual missing");
    KR_REQUIRE(ep != KR_EP_GATED || g.gate, "gemm: gate missing");
    if (g.M == 0) return KR_OK;
    if (g.M >= 4096) return launch_tile<128, 128>(g, ep, s);
    if (g.M >= 1024) return launch_tile<64, 64>(g, ep, s);
    return launch_tile<32, 32>(g, ep, s);
}

extern "C" {

int kr_transpose_f16(const uint16_t* W, long long ldw, int K, int N, uint16_t* Wt, long long ldt,
                     void* stream) {
    KR_REQUIRE(W && Wt && K >= 1 && N >= 1 && ldw >= N && ldt >= K, "kr_transpose_f16: bad args");
    dim3 grid((N + 31) / 32, (K + 31) / 32);
    transpose_kernel<<<grid, 256, 0, kr_stream(stream)>>>(
        reinterpret_cast<const kr_half*>(W), ldw, K, N, reinterpret_cast<kr_half*>(Wt), ldt);
    KR_LAUNCHED();
    return KR_OK;
}

int kr_det_matmul(const uint16_t* x, int M, int K, const uint16_t* Wt, long long ldw, int N,
                  void* out, long long ldo, int epilogue, const uint16_t* res,
                  const uint16_t* gate, void* stream) {
    kr_gemm_args g;
    g.A = reinterpret_cast<const kr_half*>(x);
    g.lda = K;
    g.Wt = reinterpret_cast<const kr_half*>(Wt);
    g.ldw = ldw;
    g.out = out;
    g.ldo = ldo;
    g.res = reinterpret_cast<const kr_half*>(res);
    g.gate = reinterpret_cast<const kr_half*>(gate);
    g.M = M;
    g.N = N;
    g.K = K;
    return kr_gemm_launch(g, epilogue, kr_stream(stream));
}

}  // extern "C"
