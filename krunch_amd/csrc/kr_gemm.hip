// fp16 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Replaces the reference's deterministic WMMA matmuls (det_matmul_tc*.cu,
// routed by layer_cpp.cpp:206-290 and :728-822) for both the packed
// compress forward (M = B*T rows) and the stepped decompress forward
// (M = B rows). The reduction contract (kr_gemm.h) is split-K over 256-wide
// K slices: each slice is one MFMA chain from zero, the slice sums are added
// left to right in fp32. Two kernels implement it:
//
//  * tile kernel (large M): 256 threads = 4 waves in a 2x2 grid, wave tile
//    (BM/2)x(BN/2) of 16x16 MFMA tiles, K staged 64 at a time through LDS
//    (row pitch 72 halves: the 16 rows read by one ds_read_b128 land on
//    distinct banks) with the next slice's global loads in flight; the
//    running slice accumulator is folded into the total every 256 K.
//  * skinny kernel (small M): one workgroup per 16 x (16*TN) output tile,
//    one wave per K slice; operands are loaded straight from global memory
//    (A is small and L2-resident, W streams once), 8 MFMAs per slice; the
//    slice partials are added in slice order through LDS by wave 0, which
//    applies the epilogue. Parallelism comes from the K slices, not from M.
#include "kr_gemm.h"

namespace {

constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;
constexpr int kKS = KR_GEMM_KSPLIT;
static_assert(kKS % kBK == 0, "split must be a multiple of the LDS K tile");

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

__device__ __forceinline__ kr_float4 add4(kr_float4 a, kr_float4 b) {
    return kr_float4{a[0] + b[0], a[1] + b[1], a[2] + b[2], a[3] + b[3]};
}

// ---------------------------------------------------------------------------
// Tile kernel (large M)
// ---------------------------------------------------------------------------
template <int BM, int BN, int EP>
__global__ void __launch_bounds__(256, 2) gemm_tile_kernel(kr_gemm_args g) {
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

    kr_float4 acc[TM][TN], tot[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int j = 0; j < TN; j++) {
            acc[i][j] = kr_float4{0.f, 0.f, 0.f, 0.f};
            tot[i][j] = acc[i][j];
        }

    const int KT = g.K / kBK;
    constexpr int TILES_PER_SPLIT = kKS / kBK;
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
        if ((kt + 1) % TILES_PER_SPLIT == 0) {     // end of a 256-wide K slice
            const bool first = kt + 1 == TILES_PER_SPLIT;
            #pragma unroll
            for (int i = 0; i < TM; i++)
                #pragma unroll
                for (int j = 0; j < TN; j++) {
                    tot[i][j] = first ? acc[i][j] : add4(tot[i][j], acc[i][j]);
                    acc[i][j] = kr_float4{0.f, 0.f, 0.f, 0.f};
                }
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
                if (m < g.M && n < g.N) store_one<EP>(g, m, n, tot[i][j][r]);
            }
}

// ---------------------------------------------------------------------------
// Skinny kernel (small M)
// ---------------------------------------------------------------------------

// One workgroup per (16*TM) x (16*TN) output tile of one job, one wave per
// 256-wide K slice (S = K/256 waves). A wave first issues every operand load
// of its slice (A rows are small and L2-resident; W streams once), then runs
// the 8-deep MFMA chains; the slice partials meet in LDS and wave 0 adds them
// in slice order and applies the job's epilogue. Several jobs with the same
// M and K (e.g. the K, V, R projections) share one launch.
template <int TM, int TN>
__global__ void __launch_bounds__(768) gemm_skinny_kernel(kr_gemm_multi mj) {
    extern __shared__ __attribute__((aligned(16))) float part_lds[];   // [S][TM*TN][256]
    const int lane = threadIdx.x & 63, s = threadIdx.x >> 6;
    // Job of this workgroup; fields are copied with constant indices so every
    // kernel-argument load is issued up front (no dependent scalar loads).
    const int bid = blockIdx.x;
    const int j = bid < mj.tiles[0] ? 0 : (bid < mj.tiles[0] + mj.tiles[1] ? 1 : 2);
    const int tile = bid - (j > 0 ? mj.tiles[0] : 0) - (j > 1 ? mj.tiles[1] : 0);
    kr_gemm_args g;
    int ep;
    if (j == 0) { g = mj.job[0]; ep = mj.ep[0]; }
    else if (j == 1) { g = mj.job[1]; ep = mj.ep[1]; }
    else { g = mj.job[2]; ep = mj.ep[2]; }
    const int S = g.K / kKS;
    const int ntn = (g.N + 16 * TN - 1) / (16 * TN);
    const int m0 = (tile / ntn) * 16 * TM, n0 = (tile % ntn) * 16 * TN;
    // Wave 0 applies the epilogue; fetch its residual / gate operands now so
    // their latency overlaps the operand loads.
    kr_half4 res_v[TM][TN], gate_v[TM][TN];
    if (s == 0 && (ep == KR_EP_RESID || ep == KR_EP_GATED)) {
        #pragma unroll
        for (int i = 0; i < TM; i++)
            #pragma unroll
            for (int t = 0; t < TN; t++)
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = min(m0 + 16 * i + (lane >> 4) * 4 + r, g.M - 1);
                    const int n = min(n0 + 16 * t + (lane & 15), g.N - 1);
                    const size_t o = (size_t)m * (size_t)g.ldo + (size_t)n;
                    res_v[i][t][r] = g.res[o];
                    gate_v[i][t][r] = ep == KR_EP_GATED ? g.gate[o] : (kr_half)0.0f;
                }
    }
    const int k0 = s * kKS + (lane >> 4) * 8;
    kr_half8 a[TM][8], b[TN][8];
    #pragma unroll
    for (int i = 0; i < TM; i++) {
        // rows beyond M / N load a valid row; their outputs are never stored
        const int r = min(m0 + 16 * i + (lane & 15), g.M - 1);
        const kr_half* ap = g.A + (size_t)r * g.lda + k0;
        #pragma unroll
        for (int q = 0; q < 8; q++) a[i][q] = *reinterpret_cast<const kr_half8*>(ap + 32 * q);
    }
    #pragma unroll
    for (int t = 0; t < TN; t++) {
        const int r = min(n0 + 16 * t + (lane & 15), g.N - 1);
        const kr_half* bp = g.Wt + (size_t)r * g.ldw + k0;
        #pragma unroll
        for (int q = 0; q < 8; q++) b[t][q] = *reinterpret_cast<const kr_half8*>(bp + 32 * q);
    }
    __builtin_amdgcn_sched_barrier(0);     // all loads in flight before the MFMAs
    kr_float4 p[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int t = 0; t < TN; t++) {
            p[i][t] = kr_float4{0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int q = 0; q < 8; q++)
                p[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][q], b[t][q], p[i][t], 0, 0, 0);
        }
    if (S > 1) {
        if (s > 0) {
            #pragma unroll
            for (int i = 0; i < TM; i++)
                #pragma unroll
                for (int t = 0; t < TN; t++)
                    *reinterpret_cast<kr_float4*>(
                        part_lds + ((size_t)s * TM * TN + i * TN + t) * 256 + lane * 4) = p[i][t];
        }
        __syncthreads();
        if (s != 0) return;
        for (int q = 1; q < S; q++)
            #pragma unroll
            for (int i = 0; i < TM; i++)
                #pragma unroll
                for (int t = 0; t < TN; t++)
                    p[i][t] = add4(p[i][t], *reinterpret_cast<const kr_float4*>(
                        part_lds + ((size_t)q * TM * TN + i * TN + t) * 256 + lane * 4));
    }
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int t = 0; t < TN; t++)
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * i + (lane >> 4) * 4 + r;
                const int n = n0 + 16 * t + (lane & 15);
                if (m >= g.M || n >= g.N) continue;
                const size_t o = (size_t)m * (size_t)g.ldo + (size_t)n;
                const float acc = p[i][t][r];
                if (ep == KR_EP_F32) {
                    reinterpret_cast<float*>(g.out)[o] = acc;
                    continue;
                }
                const float h = (float)(kr_half)acc;
                float y;
                if (ep == KR_EP_F16) y = h;
                else if (ep == KR_EP_SIGMOID) y = kr_sigmoid(h);
                else if (ep == KR_EP_RELUSQ) { const float rr = h > 0.0f ? h : 0.0f; y = rr * rr; }
                else if (ep == KR_EP_RESID) y = (float)res_v[i][t][r] + h;
                else y = (float)res_v[i][t][r] + (float)(kr_half)((float)gate_v[i][t][r] * h);
                reinterpret_cast<kr_half*>(g.out)[o] = (kr_half)y;
            }
}

template <int BM, int BN>
int launch_tile(const kr_gemm_args& g, int ep, hipStream_t s) {
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
    switch (ep) {
        case KR_EP_F32: gemm_tile_kernel<BM, BN, KR_EP_F32><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_F16: gemm_tile_kernel<BM, BN, KR_EP_F16><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_SIGMOID: gemm_tile_kernel<BM, BN, KR_EP_SIGMOID><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RELUSQ: gemm_tile_kernel<BM, BN, KR_EP_RELUSQ><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RESID: gemm_tile_kernel<BM, BN, KR_EP_RESID><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_GATED: gemm_tile_kernel<BM, BN, KR_EP_GATED><<<grid, 256, 0, s>>>(g); break;
        default: return kr_fail(KR_EINVAL, "unknown epilogue %d", ep);
    }
    KR_LAUNCHED();
    return KR_OK;
}

template <int TM, int TN>
int launch_skinny(kr_gemm_multi mj, hipStream_t s) {
    const int S = mj.job[0].K / kKS;
    int total = 0;
    for (int j = 0; j < mj.njobs; j++) {
        const kr_gemm_args& g = mj.job[j];
        mj.tiles[j] = ((g.M + 16 * TM - 1) / (16 * TM)) * ((g.N + 16 * TN - 1) / (16 * TN));
        total += mj.tiles[j];
    }
    const size_t lds = S > 1 ? (size_t)S * TM * TN * 256 * sizeof(float) : 0;
    gemm_skinny_kernel<TM, TN><<<total, dim3(64 * S), lds, s>>>(mj);
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

constexpr int kSkinnyMaxM = 512;

}  // namespace

int check_args(const kr_gemm_args& g, int ep) {
    KR_REQUIRE(g.A && g.Wt && g.out, "gemm: null pointer");
    KR_REQUIRE(g.M >= 0 && g.N >= 1 && g.K >= kKS && g.K % kKS == 0,
               "gemm: unsupported shape M=%d N=%d K=%d (K must be a multiple of %d)", g.M, g.N,
               g.K, kKS);
    KR_REQUIRE(g.lda % 8 == 0 && g.ldw % 8 == 0 && g.lda >= g.K && g.ldw >= g.K,
               "gemm: lda/ldw must be >= K and multiples of 8");
    KR_REQUIRE(((uintptr_t)g.A & 15) == 0 && ((uintptr_t)g.Wt & 15) == 0,
               "gemm: A and Wt must be 16-byte aligned");
    KR_REQUIRE(g.ldo >= g.N, "gemm: ldo < N");
    KR_REQUIRE(ep >= KR_EP_F32 && ep <= KR_EP_GATED, "gemm: unknown epilogue %d", ep);
    KR_REQUIRE((ep != KR_EP_RESID && ep != KR_EP_GATED) || g.res, "gemm: residual missing");
    KR_REQUIRE(ep != KR_EP_GATED || g.gate, "gemm: gate missing");
    return KR_OK;
}

int kr_gemm_launch_multi(const kr_gemm_args* jobs, const int* eps, int njobs, hipStream_t s) {
    KR_REQUIRE(njobs >= 1 && njobs <= KR_GEMM_MAX_JOBS, "gemm: bad job count %d", njobs);
    for (int j = 0; j < njobs; j++) {
        const int rc = check_args(jobs[j], eps[j]);
        if (rc) return rc;
    }
    const int M = jobs[0].M, K = jobs[0].K;
    bool same = true, small_n = true;
    for (int j = 1; j < njobs; j++) same = same && jobs[j].M == M && jobs[j].K == K;
    for (int j = 0; j < njobs; j++) small_n = small_n && jobs[j].N < 16384;
    if (M == 0) return KR_OK;
    if (M <= kSkinnyMaxM && same && small_n) {
        KR_REQUIRE(K / kKS <= 12, "gemm: K=%d too large for the small-M path", K);
        kr_gemm_multi mj{};
        mj.njobs = njobs;
        for (int j = 0; j < njobs; j++) { mj.job[j] = jobs[j]; mj.ep[j] = eps[j]; }
        return M >= 32 ? launch_skinny<2, 2>(mj, s) : launch_skinny<1, 2>(mj, s);
    }
    for (int j = 0; j < njobs; j++) {
        const kr_gemm_args& g = jobs[j];
        int rc;
        if (g.M >= 4096) rc = launch_tile<128, 128>(g, eps[j], s);
        else if (g.M > kSkinnyMaxM) rc = launch_tile<64, 64>(g, eps[j], s);
        else rc = launch_tile<64, 128>(g, eps[j], s);   // small M, huge N (the head)
        if (rc) return rc;
    }
    return KR_OK;
}

int kr_gemm_launch(const kr_gemm_args& g, int ep, hipStream_t s) {
    return kr_gemm_launch_multi(&g, &ep, 1, s);
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
    kr_gemm_args g{};
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
