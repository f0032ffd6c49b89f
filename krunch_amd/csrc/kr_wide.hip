// The 256 x 256 persistent GEMM and the large-M head entry point.
#include <stdint.h>
#include <algorithm>
#include <type_traits>

#include "kr_gemm.h"
#include "kr_gemm_epilogue.h"
#include "kr_math.h"

// ---------------------------------------------------------------------------
// 256 x 256 persistent GEMM for products without slice partials: the head
// (fp16, under its one-chain contract, kr_gemm.h) and the w8a8 products
// (int8, exact int32 sums). A file of its own: every kernel added to
// kr_gemm.hip's code object moves the others (its metadata grows ahead of
// the code), and measured on MI355X (A B C on one box) the head kernel added
// there moved the decode step's panel kernels by 13 KB, which then ran up to
// 6% slower (w8a8 decode -3%).
//
// Without slice partials a wave's 64 x 128 output block needs 128
// accumulator registers, so a 512-thread workgroup takes 256 x 256 tiles:
// (256 + 256) rows x 128 bytes per K step (64 fp16 or 128 int8 k), two
// 64 KB stages, one step in flight. A step costs 512 L2 line requests for
// twice the MACs of the 256 x 128 kernel's 384; the copies, not the MFMAs,
// set the time of both (timing copies on MI355X: without the copies a launch
// took 27% less; without the MFMAs, the fragment reads or the per-step
// barrier 0-3% less). The fp16 head at 8192 x 50277 x 768: 0.94-0.97 PF/s
// against 0.78-0.82 for the 256 x 128 slice-contract kernel.
// Copies: wave w < 4 copies A rows, w >= 4 W rows, 8 rows x 128 bytes per
// instruction (the swizzled stage layout big_pos), from a wave-uniform base
// plus a 32-bit byte offset (kr_gemm_launch_wide keeps every offset below 2^31).
// ---------------------------------------------------------------------------
namespace {

constexpr int kWideStageUnits = 512 * 8;      // 16-byte units per 64 KB stage

__device__ __forceinline__ void wide_copy(const void* base, unsigned off, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds), "v"(off), "s"(base) : "memory", "m0");
}

__device__ __forceinline__ bool wide_tile(int M, int N, int vb, int group_m, int& m_t, int& n_t) {
    const int gy = (M + 255) / 256, gx = (N + 255) / 256;
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

template <int EP, bool I8>
__global__ void __launch_bounds__(512, 1) gemm_wide_kernel(kr_gemm_args g, int n_virtual,
                                                           int group_m) {
    __shared__ __attribute__((aligned(1024))) kr_half8 ring[2 * kWideStageUnits];
    typedef typename std::conditional<I8, kr_int4, kr_float4>::type Acc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;        // 4 x 2 waves of 64 x 128
    const int G = gridDim.x;
    const int M = g.M, N = g.N;
    const int KS = (I8 ? g.K >> 1 : g.K) / 64;     // 64-half (128-byte) K steps
    const unsigned ring_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)ring;
    const bool a_wave = wave < 4;
    const kr_half* base = a_wave ? g.A : g.Wt;
    const long long ld16 = a_wave ? (I8 ? g.lda >> 1 : g.lda) : (I8 ? g.ldw >> 1 : g.ldw);
    const int lim = a_wave ? M : N;
    // copy i of this wave, tile rows from r0 of its operand: stage rows
    // 8 (8 w + i) .. + 7 (W rows after the 256 A rows), lane l moving chunk
    // (l % 8) ^ ((row / 2) % 8) of row 8 (8 w + i) % 256 + l / 8
    auto issue = [&](int r0, int ks, int q) {
        const unsigned so = ring_base + (unsigned)((q & 1) * kWideStageUnits * 16);
        #pragma unroll
        for (int i = 0; i < 8; i++) {
            const int crow = 8 * ((wave * 8 + i) & 31) + (lane >> 3);
            const int ckc = (lane & 7) ^ ((crow >> 1) & 7);
            const unsigned off = (unsigned)((long long)min(r0 + crow, lim - 1) * ld16 * 2) +
                                 (unsigned)(ckc * 16 + ks * 128);
            wide_copy(base, off, so + (unsigned)((wave * 8 + i) * 1024));
        }
    };
    int vb = blockIdx.x, m_t, n_t;
    if (!wide_tile(M, N, vb, group_m, m_t, n_t)) return;
    int r0 = a_wave ? m_t * 256 : n_t * 256, nr0 = 0;
    int q = 0;
    issue(r0, 0, 0);
    int stores_behind = 0;   // vector stores of the previous tile, behind this tile's first copies
    const uintptr_t ovec = EP == KR_EP_F32 ? 15 : 7;
    const bool vec_ok = (g.ldo & 3) == 0 && ((uintptr_t)g.out & ovec) == 0 &&
                        ((EP != KR_EP_RESID && EP != KR_EP_GATED) || ((uintptr_t)g.res & 7) == 0) &&
                        (EP != KR_EP_GATED || ((uintptr_t)g.gate & 7) == 0);
    const int lr = lane & 15, lq = lane >> 4;
    while (true) {
        const int m0 = m_t * 256, n0 = n_t * 256;
        int nm_t = 0, nn_t = 0;
        const bool has_next = vb + G < n_virtual && wide_tile(M, N, vb + G, group_m, nm_t, nn_t);
        if (has_next) nr0 = a_wave ? nm_t * 256 : nn_t * 256;
        Acc acc[4][8];
        #pragma unroll
        for (int i = 0; i < 4; i++)
            #pragma unroll
            for (int t = 0; t < 8; t++) acc[i][t] = Acc{0, 0, 0, 0};
        #pragma unroll 1
        for (int ks = 0; ks < KS; ks++, q++) {
            // step q's copies are in once at most the previous tile's stores
            // (issued after them, counted in a tile's first step) remain
            if (ks == 0 && stores_behind == 32) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();   // every wave's copies of step q are in; step q-1's stage is free
            if (ks + 1 < KS) issue(r0, ks + 1, q + 1);
            else if (has_next) issue(nr0, 0, q + 1);
            const kr_half8* As = ring + (q & 1) * kWideStageUnits;
            const kr_half8* Ws = As + 256 * 8;
            #pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                kr_half8 a[4];
                #pragma unroll
                for (int i = 0; i < 4; i++) a[i] = As[big_pos(64 * wm + 16 * i + lr, 4 * kb + lq)];
                #pragma unroll
                for (int th = 0; th < 2; th++) {
                    // four weight fragments at a time (register budget)
                    __builtin_amdgcn_sched_barrier(0);
                    kr_half8 w[4];
                    #pragma unroll
                    for (int t = 0; t < 4; t++)
                        w[t] = Ws[big_pos(128 * wn + 16 * (4 * th + t) + lr, 4 * kb + lq)];
                    __builtin_amdgcn_sched_barrier(0);
                    #pragma unroll
                    for (int i = 0; i < 4; i++)
                        #pragma unroll
                        for (int t = 0; t < 4; t++) {
                            Acc& c = acc[i][4 * th + t];
                            if constexpr (I8)
                                c = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(w[t]), as_i4(a[i]), c, 0, 0, 0);
                            else
                                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[t], a[i], c, 0, 0, 0);
                        }
                }
            }
        }
        // lane: row 64 wm + 16 i + lane % 16, columns 128 wn + 16 t + 4 (lane / 16) .. + 3;
        // int8: dequantised (float(acc) * sa[m]) * sw[n], then the epilogue
        const bool full = m0 + 256 <= M && n0 + 256 <= N;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + 64 * wm + 16 * i + lr;
            if (!full && m >= M) continue;
            float sa = 1.0f;
            if constexpr (I8) sa = g.sa[m];
            #pragma unroll
            for (int t = 0; t < 8; t++) {
                const int n = n0 + 128 * wn + 16 * t + 4 * lq;
                kr_float4 v;
                if constexpr (I8) {
                    #pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = __fmul_rn(__fmul_rn((float)acc[i][t][r], sa), g.sw[min(n + r, N - 1)]);
                } else {
                    v = acc[i][t];
                }
                store_row4<EP, I8>(g, m, n, v, vec_ok && n + 3 < N);
            }
        }
        if (!has_next) break;
        // a whole tile with vector access ends in exactly 32 stores per wave
        stores_behind = full && vec_ok ? 32 : 0;
        vb += G;
        m_t = nm_t;
        n_t = nn_t;
        r0 = nr0;
    }
}

}  // namespace

// Row tiles per group of the 256 x 256 kernel's tile order: about 1.25 MB of
// A panels per group (3 at a 768-wide fp16 head: measured fastest on MI355X,
// 652-668 us per 8192-row launch; 1: 687-709, 5: 669-673, 8: 703-707).
static int wide_group_m(long long row_bytes) {
    const long long g = (5ll << 18) / (256 * row_bytes);
    return (int)std::min<long long>(8, std::max<long long>(1, g));
}

// The 256 x 256 kernel on g (head: EP_F16, fp16; else int8 operands), A in
// row blocks whose 32-bit byte offsets stay below 2^31 (a row's result does
// not depend on how many rows share the launch).
int kr_gemm_launch_wide(const kr_gemm_args& g0, int ep, hipStream_t s) {
    const bool i8 = g0.i8 != 0;
    const long long lda_b = i8 ? g0.lda : g0.lda * 2, ldw_b = i8 ? g0.ldw : g0.ldw * 2;
    KR_REQUIRE(g0.Wt && (long long)g0.N * ldw_b < (1ll << 31), "gemm: weights of 2 GB or more");
    KR_REQUIRE((i8 ? g0.K : 2 * g0.K) % 128 == 0, "gemm: K=%d is not a whole number of 128-byte steps", g0.K);
    KR_REQUIRE(i8 || ep == KR_EP_F16, "gemm: the fp16 256 x 256 kernel is the head's (fp16 out)");
    const long long rows_max = ((1ll << 31) / lda_b) / 256 * 256;
    KR_REQUIRE(rows_max >= 256, "gemm: lda %lld too large", g0.lda);
    const int gm = wide_group_m(i8 ? g0.K : 2ll * g0.K);
    const size_t out_elem = ep == KR_EP_F32 ? 4 : 2;
    for (long long r0 = 0; r0 < g0.M; r0 += rows_max) {
        kr_gemm_args g = g0;
        g.M = (int)std::min<long long>(rows_max, g0.M - r0);
        g.A = reinterpret_cast<const kr_half*>(reinterpret_cast<const char*>(g0.A) + r0 * lda_b);
        g.out = static_cast<char*>(g0.out) + (size_t)r0 * (size_t)g0.ldo * out_elem;
        if (g0.res) g.res = g0.res + (size_t)r0 * (size_t)g0.ldo;
        if (g0.gate) g.gate = g0.gate + (size_t)r0 * (size_t)g0.ldo;
        if (g0.sa) g.sa = g0.sa + r0;
        const long long T = (long long)((g.N + 255) / 256) * ((g.M + 255) / 256);
        const int n_virtual = (int)((T + 7) / 8 * 8);
        const int grid = n_virtual < 256 ? n_virtual : 256;   // one workgroup per CU
        if (!i8) {
            gemm_wide_kernel<KR_EP_F16, false><<<grid, 512, 0, s>>>(g, n_virtual, gm);
        } else {
            switch (ep) {
                case KR_EP_F32: gemm_wide_kernel<KR_EP_F32, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                case KR_EP_F16: gemm_wide_kernel<KR_EP_F16, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                case KR_EP_SIGMOID: gemm_wide_kernel<KR_EP_SIGMOID, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                case KR_EP_RELUSQ: gemm_wide_kernel<KR_EP_RELUSQ, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                case KR_EP_RESID: gemm_wide_kernel<KR_EP_RESID, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                case KR_EP_GATED: gemm_wide_kernel<KR_EP_GATED, true><<<grid, 512, 0, s>>>(g, n_virtual, gm); break;
                default: return kr_fail(KR_EINVAL, "unknown epilogue %d", ep);
            }
        }
        KR_LAUNCHED();
    }
    return KR_OK;
}

int kr_gemm_head_big(const kr_half* A, long long lda, const kr_half* Wt, long long ldw, int M,
                     int N, int K, kr_half* out, long long ldo, hipStream_t s) {
    KR_REQUIRE(A && Wt && out, "head: null pointer");
    KR_REQUIRE(M >= 0 && N >= 1 && K >= 64 && K % 64 == 0,
               "head: unsupported M=%d N=%d K=%d (K must be a multiple of 64)", M, N, K);
    KR_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0,
               "head: lda %lld / ldw %lld must be >= K and multiples of 8", lda, ldw);
    KR_REQUIRE(ldo >= N, "head: ldo %lld < N %d", ldo, N);
    KR_REQUIRE(((uintptr_t)A & 15) == 0 && ((uintptr_t)Wt & 15) == 0,
               "head: operands must be 16-byte aligned");
    if (M == 0) return KR_OK;
    kr_gemm_args g{};
    g.A = A;
    g.lda = lda;
    g.Wt = Wt;
    g.ldw = ldw;
    g.out = out;
    g.ldo = ldo;
    g.M = M;
    g.N = N;
    g.K = K;
    return kr_gemm_launch_wide(g, KR_EP_F16, s);
}

