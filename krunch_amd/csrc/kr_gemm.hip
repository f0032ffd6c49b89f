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
//  * panel kernel (small M): one workgroup per (16*TM) x (16*NS) output
//    tile, one wave per K slice; operands are loaded straight from global
//    memory (fragment-packed on the decode path), A once and the NS weight
//    panels streamed, 8 MFMAs per (row block, panel); the slice partials are
//    added in slice order through LDS and the epilogue is shared out over the
//    waves. Parallelism comes from the K slices, not from M.
#include <hip/hip_ext.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "kr_gemm.h"
#include "kr_gemm_epilogue.h"
#include "kr_math.h"
#include "kr_wave.h"
#include "krunch_hip.h"

namespace {

constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;
constexpr int kKS = KR_GEMM_KSPLIT;
static_assert(kKS % kBK == 0, "split must be a multiple of the LDS K tile");

__device__ __forceinline__ kr_float4 add4(kr_float4 a, kr_float4 b) {
    return kr_float4{a[0] + b[0], a[1] + b[1], a[2] + b[2], a[3] + b[3]};
}

// ---------------------------------------------------------------------------
// Tile kernel (large M)
// ---------------------------------------------------------------------------

// Workgroup -> output tile. Workgroups are dealt to the 8 XCDs round robin
// and each XCD has its own L2, so the launch holds 8 * ceil(T/8) workgroups
// and XCD x takes the x-th contiguous eighth of the tile order; the order
// walks groups of kGroupM row tiles, rows fastest, so an XCD reuses each
// weight tile across the row tiles of a group and each A tile across the
// column tiles of its band. Returns false for the padding workgroups.
constexpr int kGroupM = 8;

__device__ __forceinline__ bool tile_of(const kr_gemm_args& g, int BM, int BN, int& m_t, int& n_t) {
    const int gy = (g.M + BM - 1) / BM, gx = (g.N + BN - 1) / BN;
    const int T = gx * gy, per = (T + 7) / 8;
    const int t = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (t >= T) return false;
    const int in_group = kGroupM * gx;
    const int first_m = (t / in_group) * kGroupM;
    const int gm = min(gy - first_m, kGroupM);
    const int r = t % in_group;
    m_t = first_m + r % gm;
    n_t = r / gm;
    return true;
}

// I8: int8 operands moved as 16-bit pairs (a 64-half K tile = 128 int8 k; a
// 32-half k step = one v_mfma_i32_16x16x64_i8), int32 accumulation.
template <int BM, int BN, int EP, bool I8>
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
    int m_t, n_t;
    if (!tile_of(g, BM, BN, m_t, n_t)) return;
    const int m0 = m_t * BM, n0 = n_t * BN;
    const int K16 = I8 ? g.K >> 1 : g.K;
    const long long lda16 = I8 ? g.lda >> 1 : g.lda, ldw16 = I8 ? g.ldw >> 1 : g.ldw;

    kr_half8 ra[A_CHUNKS], rw[W_CHUNKS];
    auto load_tiles = [&](int k0) {
        #pragma unroll
        for (int i = 0; i < A_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            const int m = m0 + r;
            if (m < g.M)
                ra[i] = *reinterpret_cast<const kr_half8*>(g.A + (size_t)m * lda16 + k0 + col);
            else
                ra[i] = kr_half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        #pragma unroll
        for (int i = 0; i < W_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c >> 3, col = (c & 7) * 8;
            const int n = n0 + r;
            if (n < g.N)
                rw[i] = *reinterpret_cast<const kr_half8*>(g.Wt + (size_t)n * ldw16 + k0 + col);
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

    typedef typename std::conditional<I8, kr_int4, kr_float4>::type Acc;
    Acc acc[TM][TN];
    kr_float4 tot[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; i++)
        #pragma unroll
        for (int j = 0; j < TN; j++) {
            acc[i][j] = Acc{0, 0, 0, 0};
            tot[i][j] = kr_float4{0.f, 0.f, 0.f, 0.f};
        }

    const int KT = K16 / kBK;
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
                for (int j = 0; j < TN; j++) {
                    if constexpr (I8)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(a[i]), as_i4(b[j]),
                                                                         acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j],
                                                                          0, 0, 0);
                }
        }
        if (!I8 && (kt + 1) % TILES_PER_SPLIT == 0) {     // end of a 256-wide K slice
            const bool first = kt + 1 == TILES_PER_SPLIT;
            #pragma unroll
            for (int i = 0; i < TM; i++)
                #pragma unroll
                for (int j = 0; j < TN; j++) {
                    if constexpr (!I8) {
                        tot[i][j] = first ? acc[i][j] : add4(tot[i][j], acc[i][j]);
                        acc[i][j] = Acc{0, 0, 0, 0};
                    }
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
                if (m < g.M && n < g.N) {
                    float v;
                    if constexpr (I8) v = __fmul_rn(__fmul_rn((float)acc[i][j][r], g.sa[m]), g.sw[n]);
                    else v = tot[i][j][r];
                    store_one<EP, I8>(g, m, n, v);
                }
            }
}

// ---------------------------------------------------------------------------
// Wide tile kernel (large M, fp16)
// ---------------------------------------------------------------------------

// 256 x 128 output tile per workgroup of 8 waves (4 x 2), each wave 64 x 64 =
// 4 x 4 MFMA tiles. Time on MI355X is set by the L2 lines a CU has in flight
// (about 64 at ~470 cycles), so the tile is as large as the registers allow
// (the 256-wide slice partials and the running total both stay in
// registers): per 64-wide K step a CU fetches 384 lines for 2M MACs, where the
// 128 x 128 kernel fetches 512 lines for the same MACs at two workgroups per
// CU. With one workgroup per CU the loads must run ahead of the MFMAs: both
// operands go global -> LDS by asynchronous copies (no registers held) into a
// 3-stage ring, two K steps ahead of the step being multiplied, with one
// barrier per step.
//
// The copies are issued as inline assembly with explicit vmcnt waits: the
// compiler's own tracking of LDS copies waits for all of them before any LDS
// read, which would serialise the ring. Nothing else in the loop touches
// vector memory, so the counts are exact: 6 copies per wave per K step.
//
// LDS layout of a stage (16-byte units): row r, 8-wide k chunk kc at
// 64 (r / 8) + 8 (r % 8) + (kc ^ ((r / 2) % 8)). One copy instruction fills
// 64 consecutive units = 8 whole rows (8 full 128-byte lines of the operand);
// an MFMA fragment read (16 rows, one chunk) hits 16 distinct bank groups.
// The weight fragment takes the MFMA's A slot, so a lane ends with 4
// consecutive columns of one row (vector stores); every output element is
// still the 8-deep chain per 256-wide slice folded in order, the bits of the
// other kernels.
// Tile shapes BM x BN of the persistent kernel: 256 x 128 (4 x 2 waves) or
// 128 x 256 (2 x 4 waves); either way a stage holds BM + BN = 384 rows of a
// 64-wide K step (48 KB) and every wave owns a 64 x 64 output block.
constexpr int kBigRows = 384;
constexpr int kBigStage = kBigRows * 8;          // 16-byte units per stage (48 KB)


// 16-byte asynchronous copy global -> LDS: lane l writes LDS byte address
// lds + 16 l. Invisible to the compiler's wait-count tracking (see above).
__device__ __forceinline__ void big_copy(const void* src, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :: "s"(lds), "v"(src) : "memory", "m0");
}

// Tile t of the launch (the dealing of tile_of, for a launch of `grid`
// virtual blocks, in groups of group_m row tiles): false past the last tile.
template <int BM>
__device__ __forceinline__ bool big_tile(const kr_gemm_args& g, int vb, int group_m, int& m_t,
                                         int& n_t) {
    constexpr int BN = kBigRows - BM;
    const int gy = (g.M + BM - 1) / BM, gx = (g.N + BN - 1) / BN;
    const int T = gx * gy, per = (T + 7) / 8;
    const int t = (vb & 7) * per + (vb >> 3);
    if (t >= T || (vb >> 3) >= per) return false;
    const int in_group = group_m * gx;
    const int first_m = (t / in_group) * group_m;
    const int gm = min(gy - first_m, group_m);
    const int r = t % in_group;
    m_t = first_m + r % gm;
    n_t = r / gm;
    return true;
}

// Row tiles per group of the persistent kernel's tile order: as many as keep
// an XCD's A panels (group_m x 256 rows x K) within about half of its 4 MB
// L2, at most 8 (fp16: 5 at K = 768, 1 at K = 3072). Measured on MI355X:
// the head at K = 768 runs 439 -> 395 us per 4096-row launch with 5 row
// tiles per group instead of 8 (8 put 3 MB of A panels in each L2), and
// the channel-mix value product at K = 3072 is fastest with 1; the fp16
// compress window takes 118.5-118.9 ms against 120.1-120.7 at 8 (A B A B
// on one box, same bits), w8a8 compress +1.1%.
int big_group_m(int K, bool i8, int BM) {
    const long long panel = (long long)BM * K * (i8 ? 1 : 2);
    const long long g = (2ll << 20) / panel;
    return (int)std::min<long long>(8, std::max<long long>(1, g));
}

// Persistent: workgroup w takes virtual blocks w, w + G, w + 2G, ... (G =
// gridDim.x, a multiple of 8, so a workgroup stays on one XCD) and keeps the
// copy ring running across its tiles: the first two K steps of the next tile
// are in flight while the current tile finishes and stores.
// I8: int8 operands (w8a8), moved as 16-bit pairs: a 64-half K step is 128
// int8 k and each 32-half block one v_mfma_i32_16x16x64_i8; the int32 sum is
// exact (no slices), dequantised once per output: (float(acc) * sa[m]) * sw[n].
template <int EP, bool I8, int BM>
__global__ void __launch_bounds__(512, 1) gemm_big_kernel(kr_gemm_args g, int n_virtual, int group_m) {
    constexpr int BN = kBigRows - BM, WN = BN / 64, AU = BM / 8;   // AU: copy units of A
    static_assert(BM == 256 || BM == 128, "tile shape");
    __shared__ __attribute__((aligned(1024))) kr_half8 ring[3 * kBigStage];   // 3 x 48 KB
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int G = gridDim.x;
    const int KS = (I8 ? g.K >> 1 : g.K) / 64;    // 64-half K steps (fp16: K % 256 == 0)
    const long long lda16 = I8 ? g.lda >> 1 : g.lda, ldw16 = I8 ? g.ldw >> 1 : g.ldw;

    // Copy instruction u = 6 wave + i of a stage: u < AU fills A rows 8u..8u+7,
    // u >= AU fills W rows 8(u-AU).. (rows past M or N repeat the last one;
    // their outputs are never stored). Lane l moves chunk (row 8u' + l/8,
    // kc = (l % 8) ^ ((row / 2) % 8)).
    const unsigned ring_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)ring;
    unsigned dst[6];
    int crow[6], ckc[6];
    #pragma unroll
    for (int i = 0; i < 6; i++) {
        const int u = wave * 6 + i;
        crow[i] = 8 * (u < AU ? u : u - AU) + (lane >> 3);
        ckc[i] = (lane & 7) ^ ((crow[i] >> 1) & 7);
        dst[i] = ring_base + (unsigned)(u * 1024);
    }
    auto sources = [&](int m0, int n0, const char* (&src)[6]) {
        #pragma unroll
        for (int i = 0; i < 6; i++) {
            if (wave * 6 + i < AU)
                src[i] = reinterpret_cast<const char*>(g.A + (size_t)min(m0 + crow[i], g.M - 1) * lda16 + ckc[i] * 8);
            else
                src[i] = reinterpret_cast<const char*>(g.Wt + (size_t)min(n0 + crow[i], g.N - 1) * ldw16 + ckc[i] * 8);
        }
    };
    // step number q of this workgroup (running over its tiles) -> ring stage q % 3
    auto issue = [&](const char* (&src)[6], int ks, int q) {
        const unsigned so = (unsigned)((q % 3) * kBigStage * 16);
        #pragma unroll
        for (int i = 0; i < 6; i++) big_copy(src[i] + (size_t)ks * 128, dst[i] + so);
    };

    int vb = blockIdx.x, m_t, n_t;
    if (!big_tile<BM>(g, vb, group_m, m_t, n_t)) return;
    const char* src[6];
    const char* nsrc[6];
    sources(m_t * BM, n_t * BN, src);
    int q = 0;                                     // running step number
    issue(src, 0, 0);
    issue(src, 1, 1);
    const int lr = lane & 15, lq = lane >> 4;
    const uintptr_t ovec = EP == KR_EP_F32 ? 15 : 7;
    const bool vec_ok = (g.ldo & 3) == 0 && ((uintptr_t)g.out & ovec) == 0 &&
                        ((EP != KR_EP_RESID && EP != KR_EP_GATED) || ((uintptr_t)g.res & 7) == 0) &&
                        (EP != KR_EP_GATED || ((uintptr_t)g.gate & 7) == 0);
    while (true) {
        const int m0 = m_t * BM, n0 = n_t * BN;
        int nm_t = 0, nn_t = 0;
        const bool has_next = vb + G < n_virtual && big_tile<BM>(g, vb + G, group_m, nm_t, nn_t);
        if (has_next) sources(nm_t * BM, nn_t * BN, nsrc);
        typedef typename std::conditional<I8, kr_int4, kr_float4>::type Acc;
        Acc acc[4][4];
        kr_float4 tot[4][4];
        if constexpr (I8) {
            #pragma unroll
            for (int i = 0; i < 4; i++)
                #pragma unroll
                for (int t = 0; t < 4; t++) acc[i][t] = Acc{0, 0, 0, 0};
        }
        for (int ks = 0; ks < KS; ks++, q++) {
            // this wave's copies of step q have landed once at most the next
            // step's remain in flight
            const bool more = ks + 1 < KS || has_next;
            if (more) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();   // every wave's copies of step q are in; step q-1's stage is free
            if (ks + 2 < KS) issue(src, ks + 2, q + 2);
            else if (has_next) issue(nsrc, ks + 2 - KS, q + 2);
            const kr_half8* As = ring + (q % 3) * kBigStage;
            const kr_half8* Ws = As + BM * 8;
            if (!I8 && (ks & 3) == 0) {
                #pragma unroll
                for (int i = 0; i < 4; i++)
                    #pragma unroll
                    for (int t = 0; t < 4; t++) acc[i][t] = Acc{0, 0, 0, 0};
            }
            #pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                kr_half8 a[4], w[4];
                #pragma unroll
                for (int i = 0; i < 4; i++) a[i] = As[big_pos(64 * wm + 16 * i + lr, 4 * kb + lq)];
                #pragma unroll
                for (int t = 0; t < 4; t++) w[t] = Ws[big_pos(64 * wn + 16 * t + lr, 4 * kb + lq)];
                // all eight fragment reads before the 16 MFMAs: one LDS wait per
                // 32-wide block instead of one per row block
                __builtin_amdgcn_sched_barrier(0);
                #pragma unroll
                for (int i = 0; i < 4; i++)
                    #pragma unroll
                    for (int t = 0; t < 4; t++) {
                        if constexpr (I8)
                            acc[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(w[t]), as_i4(a[i]),
                                                                             acc[i][t], 0, 0, 0);
                        else
                            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[t], a[i], acc[i][t], 0, 0, 0);
                    }
            }
            if constexpr (!I8) {
                if ((ks & 3) == 3) {               // end of a 256-wide K slice
                    #pragma unroll
                    for (int i = 0; i < 4; i++)
                        #pragma unroll
                        for (int t = 0; t < 4; t++) tot[i][t] = ks == 3 ? acc[i][t] : add4(tot[i][t], acc[i][t]);
                }
            }
        }
        if constexpr (I8) {   // dequantise: (float(acc) * sa[m]) * sw[n]
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const float sa = g.sa[min(m0 + 64 * wm + 16 * i + lr, g.M - 1)];
                #pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int n = n0 + 64 * wn + 16 * t + 4 * lq;
                    #pragma unroll
                    for (int r = 0; r < 4; r++)
                        tot[i][t][r] = __fmul_rn(__fmul_rn((float)acc[i][t][r], sa), g.sw[min(n + r, g.N - 1)]);
                }
            }
        }
        // lane: row 64 wm + 16 i + lane % 16, columns 64 wn + 16 t + 4 (lane / 16) .. + 3
        const bool full_m = m0 + BM <= g.M;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + 64 * wm + 16 * i + lr;
            if (!full_m && m >= g.M) continue;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                const int n = n0 + 64 * wn + 16 * t + 4 * lq;
                store_row4<EP, I8>(g, m, n, tot[i][t], vec_ok && n + 3 < g.N);
            }
        }
        if (!has_next) break;
        vb += G;
        m_t = nm_t;
        n_t = nn_t;
        #pragma unroll
        for (int i = 0; i < 6; i++) src[i] = nsrc[i];
    }
}

template <bool I8, int BM>
int launch_big_bm(const kr_gemm_args& g, int ep, hipStream_t s) {
    constexpr int BN = kBigRows - BM;
    const long long T = (long long)((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM);
    const int n_virtual = (int)((T + 7) / 8 * 8);
    const int grid = n_virtual < 256 ? n_virtual : 256;   // one workgroup per CU
    const int gm = big_group_m(g.K, I8, BM);
    switch (ep) {
        case KR_EP_F32: gemm_big_kernel<KR_EP_F32, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        case KR_EP_F16: gemm_big_kernel<KR_EP_F16, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        case KR_EP_SIGMOID: gemm_big_kernel<KR_EP_SIGMOID, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        case KR_EP_RELUSQ: gemm_big_kernel<KR_EP_RELUSQ, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        case KR_EP_RESID: gemm_big_kernel<KR_EP_RESID, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        case KR_EP_GATED: gemm_big_kernel<KR_EP_GATED, I8, BM><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
        default: return kr_fail(KR_EINVAL, "unknown epilogue %d", ep);
    }
    KR_LAUNCHED();
    return KR_OK;
}

// Tile shape: both shapes copy the same bytes per MAC (M N K (1/BM + 1/BN));
// they differ in which operand is re-read. The layer products of a compress
// window (M = B T >> N) re-read A, hundreds of MB that stream from HBM, once
// per BN columns: 128 x 256 tiles halve that. The head (N = V >> M rows per
// block) re-reads W, 77 MB, once per BM rows: it keeps 256 x 128. Measured
// on MI355X (A B A B, one box): fp16 compress 8,575 / 8,520 KB/s with
// 256 x 128 everywhere against 8,576 / 8,570 with this rule, w8a8 compress
// 9,755 / 9,747 against 9,849 / 9,856 (same bits: one reduction contract).
int big_tile_rows(const kr_gemm_args& g) {
    return (long long)g.M >= 4ll * g.N && g.N >= 256 ? 128 : 256;
}

template <bool I8>
int launch_big(const kr_gemm_args& g, int ep, hipStream_t s) {
    return big_tile_rows(g) == 128 ? launch_big_bm<I8, 128>(g, ep, s)
                                   : launch_big_bm<I8, 256>(g, ep, s);
}

// ---------------------------------------------------------------------------
// Panel kernel (small M)
// ---------------------------------------------------------------------------

// One workgroup per (16*TM) x (16*NS) output tile of one job, one wave per
// 256-wide K slice (S = K/256 waves). A wave loads its slice of the TM A
// fragments once, then streams NS weight panels of 16 columns (double
// buffered), running one 8-deep MFMA chain per (row block, panel). The slice
// partials meet in LDS; the TM*NS result tiles are then shared out over the
// waves, each adding the S partials of a tile in slice order and applying the
// job's epilogue. Several jobs with the same M and K (e.g. the K, V, R
// projections) share one launch.
//
// Time on MI355X is set by the L2 requests a CU has in flight (about 64 lines
// at ~470 cycles each), so the tile shape is chosen on the host to minimise
// the operand bytes the busiest CU reads: a larger NS re-reads A less often.
//
// FRAG: A and W^T are fragment-packed (kr_frag_index), so every operand load
// is one contiguous 1 KB read per wave; otherwise they are row-major and each
// load gathers 16 rows x 64 bytes (about 3x slower).
//
// The MFMA is issued as W^T x A^T, i.e. the weight fragment in the A-operand
// slot: the result lane then holds 4 consecutive output columns of one row,
// so the epilogue reads and writes 8-byte (fp16) or 16-byte (fp32) vectors.
// Every output element is still the same k-ordered chain of products.
//
// Workgroup -> tile: when a job has a multiple of 8 column groups, the
// workgroups of one column group (which share its weight panels) all land on
// the same XCD (workgroups are dealt to the 8 XCDs round robin), so each
// weight byte is fetched into one L2.
//
// QA (w8a8, a_q16): A arrives as fp16 in the fp16 fragment layout and is
// quantised here, one scale per row: each wave takes max |x| over its slice
// of its rows, the waves meet in LDS for the row maximum, and every wave
// rounds its own slice to int8 (kr_q8_pack4) in registers. For finite
// activations the bits are those of kr_quantize_rows followed by the int8
// product, without the separate quantisation launch; the cost is twice the A
// bytes. (The maximum compares fp16 bit patterns, so a NaN outranks every
// finite value here, where kr_quantize_rows' fmaxf skips it.)
constexpr int kEpiPrefetch = 4;   // epilogue tiles per wave with prefetched res/gate

typedef unsigned short kr_u16x2 __attribute__((ext_vector_type(2)));

template <int TM, int NS, bool FRAG, int MAXT, bool I8, bool QA>
__global__ void __launch_bounds__(MAXT) gemm_panel_kernel(kr_gemm_multi mj) {
    static_assert(!QA || (I8 && FRAG), "on-load quantisation needs the int8 fragment path");
    constexpr int TT = TM * NS;
    // 1 KB operand blocks per wave slice: 8 x (16x32 fp16) or 4 x (16x64 int8);
    // either way a wave covers 256 k. int8 operands move as 16-bit pairs.
    constexpr int QPS = I8 ? 4 : 8;
    typedef typename std::conditional<I8, kr_int4, kr_float4>::type Acc;
    extern __shared__ __attribute__((aligned(16))) float part_lds[];   // [S][TT][256]
    const int lane = threadIdx.x & 63, s = threadIdx.x >> 6;
    // decode-step timing only (stamps non-null): this wave's start and end
    const unsigned long long t_start = mj.stamps ? (unsigned long long)wall_clock64() : 0ull;
    auto stamp_end = [&]() {
        if (mj.stamps && lane == 0) {
            typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<u64x2*>(mj.stamps + 2 * (KR_STAMP_WAVES * blockIdx.x + s)) =
                u64x2{t_start, (unsigned long long)wall_clock64()};
        }
    };
    // Job of this workgroup; fields are copied with constant indices so every
    // kernel-argument load is issued up front (no dependent scalar loads).
    const int bid = blockIdx.x;
    const int j = bid < mj.tiles[0] ? 0 : (bid < mj.tiles[0] + mj.tiles[1] ? 1 : 2);
    const int w = bid - (j > 0 ? mj.tiles[0] : 0) - (j > 1 ? mj.tiles[1] : 0);
    kr_gemm_args g;
    int ep;
    if (j == 0) { g = mj.job[0]; ep = mj.ep[0]; }
    else if (j == 1) { g = mj.job[1]; ep = mj.ep[1]; }
    else { g = mj.job[2]; ep = mj.ep[2]; }
    const int S = g.K / kKS;
    const int mt = (g.M + 16 * TM - 1) / (16 * TM);
    const int ng = (g.N + 16 * NS - 1) / (16 * NS);
    int m_t, n_g;
    if ((ng & 7) == 0) {
        const int k = w >> 3;
        n_g = (k / mt) * 8 + (w & 7);
        m_t = k % mt;
    } else {
        m_t = w / ng;
        n_g = w % ng;
    }
    const int m0 = m_t * 16 * TM, n0 = n_g * 16 * NS;
    const int last_mb = (g.M - 1) >> 4, last_nb = (g.N - 1) >> 4;
    const long long lda16 = I8 ? g.lda >> 1 : g.lda, ldw16 = I8 ? g.ldw >> 1 : g.ldw;

    // ---- operand loads: A once, W panels double buffered (int8, and fp16
    // with three panels of one row block: all NS panels loaded up front)
    constexpr int NB = (I8 || NS == 3) ? NS : 2;
    kr_half8 a[TM][QPS];
    kr_half8 b[NB][QPS];
    // QA: int8 block q of the slice holds, in lane (r, j) = (l % 16, l / 16),
    // the 16 halves k = 64q + 16j .. +15 of row r: fp16 block 2q + j/2 of the
    // slice, lanes r + 32(j % 2) and r + 32(j % 2) + 16.
    kr_half8 af[QA ? TM : 1][QA ? QPS : 1][2];
    const int kb = (I8 ? g.K >> 1 : g.K) >> 5;   // 1 KB blocks per row
    auto load_w = [&](int t, kr_half8 (&dst)[QPS]) {
        // panels beyond N re-read the last one; their outputs are never stored
        if constexpr (FRAG) {
            const int nb = min((n0 >> 4) + t, last_nb);
            const kr_half* bp = g.Wf + ((size_t)nb * kb + QPS * s) * 512 + lane * 8;
            #pragma unroll
            for (int q = 0; q < QPS; q++) dst[q] = *reinterpret_cast<const kr_half8*>(bp + 512 * q);
        } else {
            const int r = min(n0 + 16 * t + (lane & 15), g.N - 1);
            const kr_half* bp = g.Wt + (size_t)r * ldw16 + s * QPS * 32 + (lane >> 4) * 8;
            #pragma unroll
            for (int q = 0; q < QPS; q++) dst[q] = *reinterpret_cast<const kr_half8*>(bp + 32 * q);
        }
    };
    #pragma unroll
    for (int i = 0; i < TM; i++) {
        if constexpr (QA) {
            const int mb = min((m0 >> 4) + i, last_mb), j16 = lane >> 4;
            const kr_half* ap = g.A + ((size_t)mb * (g.K >> 5) + 8 * s + (j16 >> 1)) * 512 +
                                ((lane & 15) + 32 * (j16 & 1)) * 8;
            #pragma unroll
            for (int q = 0; q < QPS; q++) {
                af[i][q][0] = *reinterpret_cast<const kr_half8*>(ap + 1024 * q);
                af[i][q][1] = *reinterpret_cast<const kr_half8*>(ap + 1024 * q + 128);
            }
        } else if constexpr (FRAG) {
            const int mb = min((m0 >> 4) + i, last_mb);
            const kr_half* ap = g.A + ((size_t)mb * kb + QPS * s) * 512 + lane * 8;
            #pragma unroll
            for (int q = 0; q < QPS; q++) a[i][q] = *reinterpret_cast<const kr_half8*>(ap + 512 * q);
        } else {
            const int r = min(m0 + 16 * i + (lane & 15), g.M - 1);
            const kr_half* ap = g.A + (size_t)r * lda16 + s * QPS * 32 + (lane >> 4) * 8;
            #pragma unroll
            for (int q = 0; q < QPS; q++) a[i][q] = *reinterpret_cast<const kr_half8*>(ap + 32 * q);
        }
    }
    #pragma unroll
    for (int t = 0; t < (NB < NS ? NB : NS); t++) load_w(t, b[t]);

    // ---- epilogue operands of this wave's tiles (t = s, s + S, ...), fetched
    // behind the operand loads. The vector path needs 4-column groups that
    // never straddle N and aligned pointers.
    const bool has_res = ep == KR_EP_RESID || ep == KR_EP_GATED;
    const uintptr_t ovec = ep == KR_EP_F32 ? 15 : 7;
    const bool vec = g.out_frag ||
                     ((g.N & 3) == 0 && (g.ldo & 3) == 0 && ((uintptr_t)g.out & ovec) == 0 &&
                      (!has_res || ((uintptr_t)g.res & 7) == 0) &&
                      (ep != KR_EP_GATED || ((uintptr_t)g.gate & 7) == 0));
    const int my_tiles = s < TT ? (TT - 1 - s) / S + 1 : 0;
    const bool prefetch = has_res && vec && my_tiles <= kEpiPrefetch;
    kr_half4 res_v[kEpiPrefetch], gate_v[kEpiPrefetch];
    auto tile_mn = [&](int t, int& m, int& nb) {
        m = m0 + 16 * (t / NS) + (lane & 15);
        nb = n0 + 16 * (t % NS) + 4 * (lane >> 4);
    };
    if (prefetch) {
        const kr_half* gp = ep == KR_EP_GATED ? g.gate : g.res;
        #pragma unroll
        for (int e = 0; e < kEpiPrefetch; e++) {
            if (e < my_tiles) {
                int m, nb;
                tile_mn(s + e * S, m, nb);
                const size_t o = (size_t)min(m, g.M - 1) * (size_t)g.ldo + (size_t)min(nb, g.N - 4);
                res_v[e] = *reinterpret_cast<const kr_half4*>(g.res + o);
                gate_v[e] = *reinterpret_cast<const kr_half4*>(gp + o);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);     // loads in flight before the MFMAs

    // ---- QA: row maxima over all slices, then this slice rounded to int8
    float amax_r[TM];                      // QA: row maximum, then row scale
    if constexpr (QA) {
        float* qmax = part_lds + (size_t)S * TT * 256;     // [S][TM][16]
        #pragma unroll
        for (int i = 0; i < TM; i++) {
            // |x| as fp16 bit patterns: unsigned order is value order (finite x)
            kr_u16x2 m2 = {0, 0};
            #pragma unroll
            for (int q = 0; q < QPS; q++)
                #pragma unroll
                for (int h = 0; h < 2; h++) {
                    const kr_int4 w4 = __builtin_bit_cast(kr_int4, af[i][q][h]);
                    #pragma unroll
                    for (int d = 0; d < 4; d++)
                        m2 = __builtin_elementwise_max(
                            m2, __builtin_bit_cast(kr_u16x2, (unsigned)w4[d] & 0x7fff7fffu));
                }
            unsigned mm = m2[0] > m2[1] ? m2[0] : m2[1];
            mm = max(mm, kr_xor<16>(mm));
            mm = max(mm, kr_xor<32>(mm));
            amax_r[i] = (float)__builtin_bit_cast(kr_half, (unsigned short)mm);
            if (S > 1 && lane < 16) qmax[(s * TM + i) * 16 + lane] = amax_r[i];
        }
        if (S > 1) {
            __syncthreads();
            #pragma unroll
            for (int i = 0; i < TM; i++) {
                float am = qmax[i * 16 + (lane & 15)];
                for (int q = 1; q < S; q++) am = fmaxf(am, qmax[(q * TM + i) * 16 + (lane & 15)]);
                amax_r[i] = am;
            }
        }
        #pragma unroll
        for (int i = 0; i < TM; i++) {
            const float inv = kr_q8_inv(amax_r[i]);
            const float sc = kr_q8_scale(amax_r[i]);
            #pragma unroll
            for (int q = 0; q < QPS; q++) {
                kr_int4 w4;
                #pragma unroll
                for (int d = 0; d < 4; d++) {
                    const kr_half8& h = af[i][q][d >> 1];
                    const int e = 4 * (d & 1);
                    w4[d] = (int)kr_q8_pack4((float)h[e], (float)h[e + 1], (float)h[e + 2],
                                             (float)h[e + 3], inv);
                }
                a[i][q] = __builtin_bit_cast(kr_half8, w4);
            }
            amax_r[i] = sc;                // from here on: the row's scale
        }
    }

    // ---- MFMA chains, one per (row block, panel)
    Acc p[TM][NS];
    #pragma unroll
    for (int t = 0; t < NS; t++) {
        #pragma unroll
        for (int i = 0; i < TM; i++) {
            p[i][t] = Acc{0, 0, 0, 0};
            #pragma unroll
            for (int q = 0; q < QPS; q++) {
                if constexpr (I8)
                    p[i][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(b[t % NB][q]),
                                                                   as_i4(a[i][q]), p[i][t], 0, 0, 0);
                else
                    p[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[t % NB][q], a[i][q], p[i][t],
                                                                    0, 0, 0);
            }
        }
        if (t + NB < NS) load_w(t + NB, b[t % NB]);
    }
    // int8: exact int32 sums dequantised once per output
    auto dequant = [&](int t, kr_int4 acc) -> kr_float4 {
        int m, nb;
        tile_mn(t, m, nb);
        float sa;
        if constexpr (QA) {
            // the lane's row of row block t / NS is the one amax_r holds
            sa = amax_r[0];
            #pragma unroll
            for (int i = 1; i < TM; i++)
                if (t / NS == i) sa = amax_r[i];
        } else {
            sa = g.sa[min(m, g.M - 1)];
        }
        kr_float4 y;
        #pragma unroll
        for (int r = 0; r < 4; r++) y[r] = __fmul_rn(__fmul_rn((float)acc[r], sa), g.sw[min(nb + r, g.N - 1)]);
        return y;
    };

    // ---- slice partials in LDS, then each tile summed in slice order
    auto epilogue = [&](int t, int e, kr_float4 acc) {
        int m, nb;
        tile_mn(t, m, nb);
        if (m >= g.M || nb >= g.N) return;
        const size_t o = (size_t)m * (size_t)g.ldo + (size_t)nb;
        if (vec) {
            if (ep == KR_EP_F32) {
                *reinterpret_cast<kr_float4*>(reinterpret_cast<float*>(g.out) + o) = acc;
                return;
            }
            kr_half4 rv = kr_half4{0, 0, 0, 0}, gv = kr_half4{0, 0, 0, 0};
            if (has_res) {
                if (prefetch) {
                    #pragma unroll
                    for (int x = 0; x < kEpiPrefetch; x++)
                        if (x == e) { rv = res_v[x]; gv = gate_v[x]; }
                } else {
                    rv = *reinterpret_cast<const kr_half4*>(g.res + o);
                    if (ep == KR_EP_GATED) gv = *reinterpret_cast<const kr_half4*>(g.gate + o);
                }
            }
            kr_half4 h;
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const float x = (float)kr_f16(acc[r]);
                float y;
                if (ep == KR_EP_F16) y = x;
                else if (ep == KR_EP_SIGMOID) y = kr_sigmoid_t<I8>(x);
                else if (ep == KR_EP_RELUSQ) { const float rr = x > 0.0f ? x : 0.0f; y = rr * rr; }
                else if (ep == KR_EP_RESID) y = (float)rv[r] + x;
                else y = (float)rv[r] + (float)kr_f16((float)gv[r] * x);
                h[r] = kr_f16(y);
            }
            kr_half* dst = reinterpret_cast<kr_half*>(g.out) +
                           (g.out_frag ? kr_frag_index(m, nb, g.N) : o);
            *reinterpret_cast<kr_half4*>(dst) = h;
        } else {
            #pragma unroll
            for (int r = 0; r < 4; r++)
                if (nb + r < g.N) {
                    switch (ep) {
                        case KR_EP_F32: store_one<KR_EP_F32, I8>(g, m, nb + r, acc[r]); break;
                        case KR_EP_F16: store_one<KR_EP_F16, I8>(g, m, nb + r, acc[r]); break;
                        case KR_EP_SIGMOID: store_one<KR_EP_SIGMOID, I8>(g, m, nb + r, acc[r]); break;
                        case KR_EP_RELUSQ: store_one<KR_EP_RELUSQ, I8>(g, m, nb + r, acc[r]); break;
                        case KR_EP_RESID: store_one<KR_EP_RESID, I8>(g, m, nb + r, acc[r]); break;
                        default: store_one<KR_EP_GATED, I8>(g, m, nb + r, acc[r]); break;
                    }
                }
        }
    };
    if (S == 1) {
        #pragma unroll
        for (int t = 0; t < TT; t++) {
            if constexpr (I8) epilogue(t, t, dequant(t, p[t / NS][t % NS]));
            else epilogue(t, t, p[t / NS][t % NS]);
        }
        stamp_end();
        return;
    }
    #pragma unroll
    for (int t = 0; t < TT; t++)
        *reinterpret_cast<Acc*>(part_lds + ((size_t)s * TT + t) * 256 + lane * 4) = p[t / NS][t % NS];
    __syncthreads();
    for (int e = 0; e < my_tiles; e++) {
        const int t = s + e * S;
        Acc acc = *reinterpret_cast<const Acc*>(part_lds + (size_t)t * 256 + lane * 4);
        for (int q = 1; q < S; q++)
            acc = acc + *reinterpret_cast<const Acc*>(part_lds + ((size_t)q * TT + t) * 256 + lane * 4);
        if constexpr (I8) epilogue(t, e, dequant(t, acc));
        else epilogue(t, e, acc);
    }
    stamp_end();
}

template <int BM, int BN, bool I8>
int launch_tile(const kr_gemm_args& g, int ep, hipStream_t s) {
    const long long T = (long long)((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM);
    const dim3 grid((unsigned)((T + 7) / 8 * 8));
    switch (ep) {
        case KR_EP_F32: gemm_tile_kernel<BM, BN, KR_EP_F32, I8><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_F16: gemm_tile_kernel<BM, BN, KR_EP_F16, I8><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_SIGMOID: gemm_tile_kernel<BM, BN, KR_EP_SIGMOID, I8><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RELUSQ: gemm_tile_kernel<BM, BN, KR_EP_RELUSQ, I8><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_RESID: gemm_tile_kernel<BM, BN, KR_EP_RESID, I8><<<grid, 256, 0, s>>>(g); break;
        case KR_EP_GATED: gemm_tile_kernel<BM, BN, KR_EP_GATED, I8><<<grid, 256, 0, s>>>(g); break;
        default: return kr_fail(KR_EINVAL, "unknown epilogue %d", ep);
    }
    KR_LAUNCHED();
    return KR_OK;
}

struct PanelShape {
    int TM, NS;
};

thread_local unsigned long long* t_panel_stamps = nullptr;
thread_local int t_panel_cap = 0;
thread_local int t_panel_taken = 0;
thread_local hipEvent_t t_panel_ev[2] = {};

template <int TM, int NS, bool FRAG, int MAXT, bool I8, bool QA>
int launch_panel(kr_gemm_multi mj, hipStream_t s) {
    const int S = mj.job[0].K / kKS;
    int total = 0;
    for (int j = 0; j < mj.njobs; j++) {
        const kr_gemm_args& g = mj.job[j];
        mj.tiles[j] = ((g.M + 16 * TM - 1) / (16 * TM)) * ((g.N + 16 * NS - 1) / (16 * NS));
        total += mj.tiles[j];
    }
    size_t lds = S > 1 ? (size_t)S * TM * NS * 256 * sizeof(float) : 0;
    if (QA && S > 1) lds += (size_t)S * TM * 16 * sizeof(float);
    mj.stamps = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    if (t_panel_stamps) {
        // the buffer holds KR_STAMP_WAVES slots for t_panel_cap workgroups
        const bool fits = total <= t_panel_cap && S <= KR_STAMP_WAVES;
        if (fits) {
            mj.stamps = t_panel_stamps;
            ev0 = t_panel_ev[0];
            ev1 = t_panel_ev[1];
        }
        t_panel_stamps = nullptr;
        t_panel_ev[0] = t_panel_ev[1] = nullptr;
        t_panel_taken = fits ? total : -total;
    }
    if (ev0)
        hipExtLaunchKernelGGL(gemm_panel_kernel<TM, NS, FRAG, MAXT, I8, QA>, dim3(total),
                              dim3(64 * S), (uint32_t)lds, s, ev0, ev1, 0u, mj);
    else
        gemm_panel_kernel<TM, NS, FRAG, MAXT, I8, QA><<<total, dim3(64 * S), lds, s>>>(mj);
    KR_LAUNCHED();
    return KR_OK;
}

}  // namespace

void kr_gemm_time_next_panel(unsigned long long* stamps, int max_groups, hipEvent_t start,
                             hipEvent_t stop) {
    t_panel_stamps = max_groups > 0 ? stamps : nullptr;
    t_panel_cap = max_groups;
    t_panel_taken = 0;
    t_panel_ev[0] = t_panel_stamps && start && stop ? start : nullptr;
    t_panel_ev[1] = t_panel_stamps && start && stop ? stop : nullptr;
}

int kr_gemm_timed_launch_taken() { return t_panel_taken; }

namespace {

// Shapes compiled per block size: up to 4 slices TM {1, 2, 4} x NS {1, 2};
// up to 12 slices TM {1, 2} x NS {1, 2}; up to 16 slices TM 1 x NS {1, 2}.
// Wider panels (NS > 2) cut the bytes a CU reads but, with the registers a
// wave has, the third panel's loads wait for the first panel's MFMAs:
// measured on MI355X at M = 256 they are 25-55% slower, so every wave keeps
// all of its operand loads in flight at once. Taller tiles (TM = 4) keep
// that property at K <= 1024, where the A fragments of 4 row blocks fit.
// int8 operands also take NS = 3 and 4 (four int8 panels hold the registers
// of two fp16 ones, all in flight at once), and one-row-block fp16 tiles
// NS = 3 with all three panels loaded up front. At M = 256 and N = 768,
// NS = 3 makes 16 column groups: one workgroup per CU, and a multiple of 8,
// so the XCD dealing and L2 staging apply (measured on MI355X: w8a8 decode
// +2.8% against 1 x 4, fp16 decode +0.9% against 2 x 2).
constexpr PanelShape kShapes256[] = {{1, 1}, {1, 2}, {2, 1}, {2, 2}, {4, 1}, {4, 2},
                                     {1, 4}, {2, 4}, {1, 3}, {2, 3}};
constexpr PanelShape kShapes768[] = {{1, 1}, {1, 2}, {2, 1}, {2, 2}, {1, 4}, {1, 3}};
constexpr PanelShape kShapes1024[] = {{1, 1}, {1, 2}};

// Busiest-CU operand bytes (in 128-byte lines) for a shape: workgroups are
// spread over the 256 CUs, each reading (16*TM + 16*NS) x K halves (QA: A
// rows count twice against int8 weight rows); ties go to the shape that
// occupies more CUs.
long long panel_cost(const kr_gemm_multi& mj, PanelShape sh) {
    long long wgs = 0;
    for (int j = 0; j < mj.njobs; j++) {
        const kr_gemm_args& g = mj.job[j];
        wgs += (long long)((g.M + 16 * sh.TM - 1) / (16 * sh.TM)) *
               ((g.N + 16 * sh.NS - 1) / (16 * sh.NS));
    }
    // QA: each workgroup quantises its rows over the whole K, and every column
    // group repeats that for the same rows, so one row block per workgroup
    // (measured on MI355X at M = 256: the value product 7.4 us at TM 1 x NS 4
    // against 8.8 at 2 x 2, the output projection 5.2 against 5.9);
    // 4 panels only for int8 weights
    if (mj.job[0].a_q16 && sh.TM > 1) return LLONG_MAX;
    if (!mj.job[0].i8 && sh.NS > 2 && !(sh.NS == 3 && sh.TM == 1)) return LLONG_MAX;
    // int8 operands: at most 2 row blocks (the stepped channel-mix R/K
    // product at M = 256: w8a8 decode 1,880 -> 1,919 KB/s at 2 x 2 against
    // 4 x 2, measured on MI355X; the fp16 product keeps 4 x 2, 1,883 against
    // 1,878)
    if (mj.job[0].i8 && sh.TM > 2) return LLONG_MAX;
    const int ta = mj.job[0].a_q16 ? 2 * sh.TM : sh.TM;
    const long long per_wg = (long long)(ta + sh.NS) * mj.job[0].K / 4;
    return ((wgs + 255) / 256) * per_wg * 4096 - std::min<long long>(wgs, 256);
}

template <size_t N>
PanelShape choose_shape(const kr_gemm_multi& mj, const PanelShape (&shapes)[N]) {
    PanelShape best = shapes[0];
    long long best_cost = panel_cost(mj, best);
    for (size_t i = 1; i < N; i++) {
        const long long c = panel_cost(mj, shapes[i]);
        if (c < best_cost) { best_cost = c; best = shapes[i]; }
    }
    return best;
}

PanelShape choose_small_shape(const kr_gemm_multi& mj) {
    const int S = mj.job[0].K / kKS;
    if (S <= 4) return choose_shape(mj, kShapes256);
    if (S <= 12) return choose_shape(mj, kShapes768);
    return choose_shape(mj, kShapes1024);
}

template <bool FRAG, int MAXT, bool I8, bool QA, size_t N>
int launch_best(const kr_gemm_multi& mj, const PanelShape (&shapes)[N], hipStream_t s) {
    const PanelShape best = choose_shape(mj, shapes);
#define KR_PANEL(TM_, NS_) \
    if (best.TM == TM_ && best.NS == NS_) return launch_panel<TM_, NS_, FRAG, MAXT, I8, QA>(mj, s);
    if constexpr (MAXT == 256) {
        KR_PANEL(1, 1) KR_PANEL(1, 2)
        if constexpr (!QA) { KR_PANEL(2, 1) KR_PANEL(2, 2) KR_PANEL(4, 1) KR_PANEL(4, 2) }
        KR_PANEL(1, 3)
        if constexpr (I8) { KR_PANEL(1, 4) }
        if constexpr (I8 && !QA) { KR_PANEL(2, 4) KR_PANEL(2, 3) }
    } else if constexpr (MAXT == 768) {
        KR_PANEL(1, 1) KR_PANEL(1, 2) KR_PANEL(1, 3)
        if constexpr (!QA) { KR_PANEL(2, 1) KR_PANEL(2, 2) }
        if constexpr (I8) { KR_PANEL(1, 4) }
    } else {
        KR_PANEL(1, 1) KR_PANEL(1, 2)
    }
#undef KR_PANEL
    return kr_fail(KR_EINVAL, "gemm: no panel shape");
}

template <bool FRAG, bool I8, bool QA = false>
int launch_small(const kr_gemm_multi& mj, hipStream_t s) {
    const int S = mj.job[0].K / kKS;
    if (S <= 4) return launch_best<FRAG, 256, I8, QA>(mj, kShapes256, s);
    if (S <= 12) return launch_best<FRAG, 768, I8, QA>(mj, kShapes768, s);
    return launch_best<FRAG, 1024, I8, QA>(mj, kShapes1024, s);
}

// ---------------------------------------------------------------------------
// Small-M head (the decode step: M <= 512 rows x V = 50277 columns, K = C):
// the A operand stays in registers for the whole launch and each workgroup
// streams its own contiguous run of 16-column weight blocks exactly once.
//
// The persistent 256x128 kernel re-reads all M rows of A for every
// 128-column tile: 393 tiles at V = 50277 over 256 CUs, 9,216 L2 lines on the
// busiest CU. Here a workgroup of four waves takes one group of 64 RBW rows
// (wave w: row blocks RBW w .. RBW w + RBW - 1 of the group, RBW x K/32
// fragments of the fragment-packed A held in registers) and one contiguous
// run of 16-column weight blocks, which it streams once: a weight block (16
// columns x K, contiguous in the fragment layout) goes into an LDS ring of
// kHeadStages stages by asynchronous copies issued kHeadStages - 1 blocks
// ahead, and all four waves multiply each block with their rows. The mh row
// groups of one column run are workgroups b, b + 8, ..., which the dispatcher
// places on one XCD, so its L2 fetches each weight block once for all of them.
// The head's reduction contract (kr_gemm.h, the head): one
// v_mfma_f32_16x16x32_f16 chain over the whole K from zero, MFMA issued as
// W^T x A^T, then out = fp16(acc); gemm_wide_kernel gives the same bits.
constexpr int kHeadStages = 4;
// Row blocks per wave. Every weight block needs all of a workgroup's A in
// registers, so the A load (all rows of the group) is not overlapped by any
// MFMA; two row groups of 128 rows halve it and double each CU's weight
// stream. Measured on MI355X at M = 256 (A B on three boxes, decode KB/s):
// 2 row blocks per wave with two row groups 2,015 / 2,025 / 2,030 against
// 1,972 / 1,989 / 2,017 for 4 (one group of 256 rows); the isolated launch
// 28.0-28.4 us against 28.7-29.9 with the weights in the memory-side cache
// and 33.4 against 37.9-38.4 without. The two row groups on different XCDs
// (weights fetched into two L2s): 1,915. A 6-stage ring or two workgroups
// per CU (3 stages each): 2,008 / 2,012 against 2,025.
constexpr int kHeadRBW = 2;

// RBW row blocks (16 rows) per wave, four waves: 64 RBW rows per workgroup;
// mh row groups share each column run (gridDim.x = mh x the runs).
template <int KB, int RBW>   // KB = K / 32 fragments per row: K = 256, 512 or 768
__global__ void __launch_bounds__(256, 1) gemm_head_small_kernel(
        const kr_half* __restrict__ Af, const kr_half* __restrict__ Wf, kr_half* __restrict__ out,
        long long ldo, int M, int N, int vec, int mh) {
    constexpr int NW = 4;            // waves
    constexpr int CPW = KB / NW;     // 1 KB copies per wave per block
    constexpr int S = KB / 8;        // groups of 8 fragments (256 k) per LDS wait
    constexpr int AHEAD = (kHeadStages - 2) * CPW;
    static_assert(KB % NW == 0 && AHEAD <= 24, "copy split");
    __shared__ __attribute__((aligned(1024))) kr_half8 ring[kHeadStages * KB * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int nb_total = (N + 15) >> 4;
    // row group h and column run cr of this workgroup: with a multiple of 8
    // runs, the groups of run cr are workgroups 8 mh (cr / 8) + cr % 8 + 8 h
    const int bx = blockIdx.x, ncr = (int)gridDim.x / mh;
    int h, cr;
    if ((ncr & 7) == 0) {
        h = (bx >> 3) % mh;
        cr = (bx / (8 * mh)) * 8 + (bx & 7);
    } else {
        h = bx % mh;
        cr = bx / mh;
    }
    const int b0 = (int)(((long long)cr * nb_total) / ncr);
    const int b1 = (int)(((long long)(cr + 1) * nb_total) / ncr);
    const int nblk = b1 - b0;
    // this wave's rows (row blocks past the last one re-read it; never stored)
    const int last_mb = (M - 1) >> 4;
    const int mb0 = h * (RBW * NW) + RBW * wave;
    const bool active = mb0 <= last_mb;
    kr_half8 a[RBW][KB];
    if (active) {
        #pragma unroll
        for (int i = 0; i < RBW; i++) {
            const size_t blk = (size_t)min(mb0 + i, last_mb) * KB;
            #pragma unroll
            for (int q = 0; q < KB; q++)
                a[i][q] = *reinterpret_cast<const kr_half8*>(Af + (blk + q) * 512 + lane * 8);
        }
    }
    const unsigned ring_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)ring;
    // weight block b0 + j -> stage j % kHeadStages; wave w copies fragments CPW w ..
    auto issue = [&](int j) {
        const char* src = reinterpret_cast<const char*>(
            Wf + ((size_t)(b0 + j) * KB + (size_t)wave * CPW) * 512 + lane * 8);
        const unsigned dst = ring_base + (unsigned)(((j % kHeadStages) * KB + wave * CPW) * 1024);
        #pragma unroll
        for (int u = 0; u < CPW; u++) big_copy(src + u * 1024, dst + u * 1024);
    };
    #pragma unroll
    for (int j = 0; j < kHeadStages - 1; j++)
        if (j < nblk) issue(j);
    for (int j = 0; j < nblk; j++) {
        // the copies of blocks j + 1 .. j + kHeadStages - 2 may stay in flight
        // (later stores only make the wait stricter: operations retire in
        // order); near the end everything is waited for
        if (j + kHeadStages - 2 < nblk) {
            if constexpr (AHEAD == 24) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
            else if constexpr (AHEAD == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
            else if constexpr (AHEAD == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
            else if constexpr (AHEAD == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            else if constexpr (AHEAD == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
            else if constexpr (AHEAD == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();   // every wave's copies of block j are in; block j - 1's stage is free
        if (j + kHeadStages - 1 < nblk) issue(j + kHeadStages - 1);
        if (!active) continue;
        const kr_half8* st = ring + (j % kHeadStages) * KB * 64;
        kr_float4 tot[RBW];
        #pragma unroll
        for (int i = 0; i < RBW; i++) tot[i] = kr_float4{0, 0, 0, 0};
        #pragma unroll
        for (int sl = 0; sl < S; sl++) {
            // 8 weight fragments read before their MFMAs (one LDS wait)
            kr_half8 w[8];
            #pragma unroll
            for (int q = 0; q < 8; q++) w[q] = st[(8 * sl + q) * 64 + lane];
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int q = 0; q < 8; q++) {
                #pragma unroll
                for (int i = 0; i < RBW; i++)
                    tot[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[q], a[i][8 * sl + q], tot[i], 0, 0, 0);
            }
        }
        // lane: row 16 (mb0 + i) + lane % 16, columns n .. n + 3
        const int n = 16 * (b0 + j) + 4 * (lane >> 4);
        #pragma unroll
        for (int i = 0; i < RBW; i++) {
            const int m = 16 * (mb0 + i) + (lane & 15);
            if (m >= M) continue;
            kr_half* dst = out + (size_t)m * (size_t)ldo + n;
            if (vec && n + 3 < N) {
                kr_half4 h;
                #pragma unroll
                for (int r = 0; r < 4; r++) h[r] = kr_f16(tot[i][r]);
                *reinterpret_cast<kr_half4*>(dst) = h;
            } else {
                #pragma unroll
                for (int r = 0; r < 4; r++)
                    if (n + r < N) dst[r] = kr_f16(tot[i][r]);
            }
        }
    }
}

// Pack Wt [N, K] (row stride ld) into the fragment layout; rows N..N16-1 are zero.
__global__ void pack_frag_kernel(const kr_half* __restrict__ Wt, long long ld, int N, int K,
                                 kr_half* __restrict__ out) {
    const long long N16 = kr_frag_rows(N);
    const long long chunks = N16 * (K / 8);   // 8-half groups
    for (long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x; c < chunks;
         c += (long long)gridDim.x * blockDim.x) {
        const long long r = c / (K / 8), k = (c % (K / 8)) * 8;
        kr_half8 v = kr_half8{0, 0, 0, 0, 0, 0, 0, 0};
        if (r < N) v = *reinterpret_cast<const kr_half8*>(Wt + r * ld + k);
        *reinterpret_cast<kr_half8*>(out + kr_frag_index(r, k, K)) = v;
    }
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

bool kr_gemm_head_small_ok(int M, int N, int K) {
    return M >= 1 && M <= 512 && N >= 1 && (K == 256 || K == 512 || K == 768);
}

int kr_gemm_head_small(const kr_half* Af, const kr_half* Wf, int M, int N, int K, kr_half* out,
                       long long ldo, hipStream_t s) {
    KR_REQUIRE(Af && Wf && out, "head: null pointer");
    KR_REQUIRE(kr_gemm_head_small_ok(M, N, K), "head: unsupported M=%d N=%d K=%d", M, N, K);
    KR_REQUIRE(ldo >= N, "head: ldo %lld < N %d", ldo, N);
    KR_REQUIRE(((uintptr_t)Af & 15) == 0 && ((uintptr_t)Wf & 15) == 0,
               "head: operands must be 16-byte aligned");
    const int vec = (ldo & 3) == 0 && ((uintptr_t)out & 7) == 0;
    const int nb = (N + 15) / 16;
    constexpr int R = kHeadRBW;
    // row groups of 64 R rows, and column runs: one workgroup per CU
    const int mh = (M + 64 * R - 1) / (64 * R);
    int ncr = nb < 256 / mh ? nb : 256 / mh;
    // a multiple of 8 runs puts the groups of a run on one XCD; measured on
    // MI355X at three row groups (85 runs -> 80): decode +2.7% at B = 320,
    // +1.1% at B = 384 (A B twice, one box)
    if (ncr >= 8) ncr &= ~7;
    const int grid = ncr * mh;
    switch (K) {
        case 256: gemm_head_small_kernel<8, R><<<grid, 256, 0, s>>>(Af, Wf, out, ldo, M, N, vec, mh); break;
        case 512: gemm_head_small_kernel<16, R><<<grid, 256, 0, s>>>(Af, Wf, out, ldo, M, N, vec, mh); break;
        default: gemm_head_small_kernel<24, R><<<grid, 256, 0, s>>>(Af, Wf, out, ldo, M, N, vec, mh); break;
    }
    KR_LAUNCHED();
    return KR_OK;
}

int check_args(const kr_gemm_args& g, int ep) {
    KR_REQUIRE(g.A && (g.Wt || g.Wf) && g.out, "gemm: null pointer");
    KR_REQUIRE(g.M >= 0 && g.N >= 1 && g.K >= kKS && g.K % kKS == 0,
               "gemm: unsupported shape M=%d N=%d K=%d (K must be a multiple of %d)", g.M, g.N,
               g.K, kKS);
    KR_REQUIRE(g.a_frag || (g.lda % 8 == 0 && g.lda >= g.K), "gemm: lda must be >= K, multiple of 8");
    KR_REQUIRE(!g.Wt || (g.ldw % 8 == 0 && g.ldw >= g.K), "gemm: ldw must be >= K, multiple of 8");
    KR_REQUIRE(((uintptr_t)g.A & 15) == 0 && ((uintptr_t)g.Wt & 15) == 0 &&
                   ((uintptr_t)g.Wf & 15) == 0,
               "gemm: A, Wt and Wf must be 16-byte aligned");
    KR_REQUIRE(g.out_frag || g.ldo >= g.N, "gemm: ldo < N");
    KR_REQUIRE(!g.a_frag || g.Wf, "gemm: fragment-packed A needs fragment-packed W");
    KR_REQUIRE(!g.out_frag || (g.N % 32 == 0 && ep != KR_EP_F32 && ep != KR_EP_RESID &&
                               ep != KR_EP_GATED && ((uintptr_t)g.out & 7) == 0),
               "gemm: fragment-packed output needs N %% 32 == 0 and an elementwise fp16 epilogue");
    KR_REQUIRE(ep >= KR_EP_F32 && ep <= KR_EP_GATED, "gemm: unknown epilogue %d", ep);
    KR_REQUIRE(!g.i8 || ((g.sa || g.a_q16) && g.sw && (g.a_frag || g.lda % 16 == 0) &&
                         (!g.Wt || g.ldw % 16 == 0)),
               "gemm: int8 needs scales and 16-byte aligned rows (lda/ldw multiples of 16)");
    KR_REQUIRE((ep != KR_EP_RESID && ep != KR_EP_GATED) || g.res, "gemm: residual missing");
    KR_REQUIRE(ep != KR_EP_GATED || g.gate, "gemm: gate missing");
    return KR_OK;
}

int kr_gemm_panel_ns(const kr_gemm_args* jobs, int njobs) {
    if (njobs < 1 || njobs > KR_GEMM_MAX_JOBS || jobs[0].K < kKS || jobs[0].K / kKS > 16) return 0;
    kr_gemm_multi mj{};
    mj.njobs = njobs;
    for (int j = 0; j < njobs; j++) mj.job[j] = jobs[j];
    return choose_small_shape(mj).NS;
}

int kr_gemm_launch_multi(const kr_gemm_args* jobs, const int* eps, int njobs, hipStream_t s) {
    KR_REQUIRE(njobs >= 1 && njobs <= KR_GEMM_MAX_JOBS, "gemm: bad job count %d", njobs);
    for (int j = 0; j < njobs; j++) {
        const int rc = check_args(jobs[j], eps[j]);
        if (rc) return rc;
    }
    const int M = jobs[0].M, K = jobs[0].K;
    bool same = true, small_n = true, frag = jobs[0].a_frag != 0, any_frag = false;
    const bool i8 = jobs[0].i8 != 0, qa = jobs[0].a_q16 != 0;
    for (int j = 1; j < njobs; j++)
        same = same && jobs[j].M == M && jobs[j].K == K && (jobs[j].a_frag != 0) == frag &&
               (jobs[j].i8 != 0) == i8 && (jobs[j].a_q16 != 0) == qa;
    for (int j = 0; j < njobs; j++)
        KR_REQUIRE(!jobs[j].a_q16 || (jobs[j].i8 && jobs[j].a_frag && jobs[j].Wf),
                   "gemm: on-load quantisation needs int8 weights and fragment-packed operands");
    for (int j = 0; j < njobs; j++) {
        small_n = small_n && jobs[j].N < KR_GEMM_SMALL_MAX_N;
        any_frag = any_frag || jobs[j].a_frag || jobs[j].out_frag;
    }
    if (M == 0) return KR_OK;
    const bool small = M <= KR_GEMM_SMALL_M && same && small_n;
    KR_REQUIRE(small || !any_frag, "gemm: fragment-packed operands need the small-M path "
               "(M <= %d, N < %d, one M/K/layout per launch)", KR_GEMM_SMALL_M, KR_GEMM_SMALL_MAX_N);
    if (small) {
        KR_REQUIRE(K / kKS <= 16, "gemm: K=%d too large for the small-M path", K);
        kr_gemm_multi mj{};
        mj.njobs = njobs;
        for (int j = 0; j < njobs; j++) { mj.job[j] = jobs[j]; mj.ep[j] = eps[j]; }
        if (qa) return launch_small<true, true, true>(mj, s);
        if (frag) return i8 ? launch_small<true, true>(mj, s) : launch_small<true, false>(mj, s);
        // row-major A: fragment weights are not used, the row-major copy must exist
        for (int j = 0; j < njobs; j++) KR_REQUIRE(jobs[j].Wt, "gemm: row-major W missing");
        return i8 ? launch_small<false, true>(mj, s) : launch_small<false, false>(mj, s);
    }
    for (int j = 0; j < njobs; j++) {
        const kr_gemm_args& g = jobs[j];
        KR_REQUIRE(g.Wt, "gemm: row-major W missing");
        int rc;
        if (g.i8) {
            // the 256 x 256 kernel pays where a tile has many K steps or the
            // product many column tiles; measured on MI355X at M = 262144:
            // ffn K (K = 768, N = 3072) -4%, ffn V (K = 3072, N = 768)
            // -1.5%, the 768 x 768 products +7 to +14% (six K steps per
            // tile with one in flight)
            if (g.M >= 4096 && (g.N >= 2048 || g.K >= 2048) && g.K % 128 == 0 &&
                g.lda % 16 == 0 && g.ldw % 16 == 0 && ((uintptr_t)g.A & 15) == 0 &&
                ((uintptr_t)g.Wt & 15) == 0)
                rc = kr_gemm_launch_wide(g, eps[j], s);
            else if (g.M >= 4096 && (g.K >> 1) % 64 == 0) rc = launch_big<true>(g, eps[j], s);
            else if (g.M >= 4096) rc = launch_tile<128, 128, true>(g, eps[j], s);
            else rc = launch_tile<64, 64, true>(g, eps[j], s);
        } else if (g.K % 256 == 0 && (g.M >= 4096 || (g.M >= 128 && g.N >= KR_GEMM_SMALL_MAX_N))) {
            // large M, or the head at decode batch sizes: the persistent
            // 256 x 128 kernel (vector epilogue when the output row stride is
            // a multiple of 4 elements)
            rc = launch_big<false>(g, eps[j], s);
        } else if (g.M >= 4096) {
            rc = launch_tile<128, 128, false>(g, eps[j], s);
        } else if (g.M > KR_GEMM_SMALL_M) {
            rc = launch_tile<64, 64, false>(g, eps[j], s);
        } else {
            rc = launch_tile<64, 128, false>(g, eps[j], s);   // small M, huge N (the head)
        }
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

size_t kr_fragment_bytes(int N, int K) {
    if (N < 1 || K < 32 || K % 32) return 0;
    return (size_t)kr_frag_rows(N) * (size_t)K * 2;
}

int kr_pack_fragments(const uint16_t* Wt, long long ld, int N, int K, uint16_t* out, void* stream) {
    KR_REQUIRE(Wt && out && N >= 1 && K >= 32 && K % 32 == 0 && ld >= K && ld % 8 == 0,
               "kr_pack_fragments: bad args (K must be a multiple of 32)");
    KR_REQUIRE(((uintptr_t)Wt & 15) == 0 && ((uintptr_t)out & 15) == 0,
               "kr_pack_fragments: pointers must be 16-byte aligned");
    pack_frag_kernel<<<512, 256, 0, kr_stream(stream)>>>(reinterpret_cast<const kr_half*>(Wt), ld,
                                                         N, K, reinterpret_cast<kr_half*>(out));
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

int kr_det_matmul_packed_multi(const kr_packed_job* jobs, int n_jobs, int M, int K,
                               void* stream) {
    KR_REQUIRE(jobs && n_jobs >= 1 && n_jobs <= KR_GEMM_MAX_JOBS,
               "kr_det_matmul_packed_multi: 1..%d jobs", KR_GEMM_MAX_JOBS);
    KR_REQUIRE(M >= 0 && M <= KR_GEMM_SMALL_M && K > 0,
               "kr_det_matmul_packed_multi: M=%d K=%d (M <= %d)", M, K, KR_GEMM_SMALL_M);
    kr_gemm_args g[KR_GEMM_MAX_JOBS] = {};
    int eps[KR_GEMM_MAX_JOBS] = {};
    for (int j = 0; j < n_jobs; j++) {
        const kr_packed_job& p = jobs[j];
        KR_REQUIRE(p.xf && p.Wf && p.out, "kr_det_matmul_packed_multi: null pointer in job %d", j);
        g[j].A = reinterpret_cast<const kr_half*>(p.xf);
        g[j].lda = K;
        g[j].Wf = reinterpret_cast<const kr_half*>(p.Wf);
        g[j].out = p.out;
        g[j].ldo = p.ldo;
        g[j].res = reinterpret_cast<const kr_half*>(p.res);
        g[j].gate = reinterpret_cast<const kr_half*>(p.gate);
        g[j].M = M;
        g[j].N = p.N;
        g[j].K = K;
        g[j].a_frag = 1;
        g[j].out_frag = p.out_packed ? 1 : 0;
        eps[j] = p.epilogue;
    }
    return kr_gemm_launch_multi(g, eps, n_jobs, kr_stream(stream));
}

int kr_det_matmul_packed(const uint16_t* xf, int M, int K, const uint16_t* Wf, int N, void* out,
                         long long ldo, int epilogue, const uint16_t* res, const uint16_t* gate,
                         int out_packed, void* stream) {
    kr_gemm_args g{};
    g.A = reinterpret_cast<const kr_half*>(xf);
    g.lda = K;
    g.Wf = reinterpret_cast<const kr_half*>(Wf);
    g.out = out;
    g.ldo = ldo;
    g.res = reinterpret_cast<const kr_half*>(res);
    g.gate = reinterpret_cast<const kr_half*>(gate);
    g.M = M;
    g.N = N;
    g.K = K;
    g.a_frag = 1;
    g.out_frag = out_packed ? 1 : 0;
    return kr_gemm_launch(g, epilogue, kr_stream(stream));
}

}  // extern "C"
