// MFMA fp16 GEMM with fused epilogues (declarations shared by the layer driver).
#pragma once
#include "kr_common.h"

// Epilogues applied to the fp32 accumulator `acc` of C = A @ W.
enum kr_epilogue : int {
    KR_EP_F32 = 0,      // out(f32) = acc                               (k, v of time mix)
    KR_EP_F16 = 1,      // out(f16) = fp16(acc)                         (head logits)
    KR_EP_SIGMOID = 2,  // out(f16) = fp16(sigmoid(fp16(acc)))          (receptances)
    KR_EP_RELUSQ = 3,   // out(f16) = fp16(relu(fp16(acc))^2)           (channel-mix key)
    KR_EP_RESID = 4,    // out(f16) = fp16(res + fp16(acc))             (time-mix output)
    KR_EP_GATED = 5,    // out(f16) = fp16(res + fp16(gate * fp16(acc))) (channel-mix output)
};

struct kr_gemm_args {
    const kr_half* A;   // [M, K] row-major, row stride lda (or fragment-packed, a_frag)
    long long lda;
    const kr_half* Wt;  // [N, K] row-major (W transposed), row stride ldw
    long long ldw;
    void* out;          // [M, N], row stride ldo (f32 or f16 per epilogue; or fragment-packed)
    long long ldo;
    const kr_half* res;   // [M, N] stride ldo (RESID, GATED); may alias out
    const kr_half* gate;  // [M, N] stride ldo (GATED)
    int M, N, K;
    const kr_half* Wf;  // W^T fragment-packed (kr_frag_index), or null; small-M path only
    int a_frag;         // A is fragment-packed (small-M path only; needs Wf)
    int out_frag;       // fp16 output written fragment-packed as a K = N operand
    // w8a8: A and W^T hold int8 (pointers reinterpreted; lda/ldw in bytes),
    // acc = exact int32 sum, value = (float(acc) * sa[m]) * sw[n], then the epilogue.
    int i8;
    const float* sa;    // [M] per-row (per-token) activation scales
    const float* sw;    // [N] per-output-channel weight scales
    // w8a8, small-M fragment path only: A holds fp16 in the fp16 fragment
    // layout (kr_frag_index) and each workgroup quantises its rows on load by
    // the rule below, scales included (sa is not read). Same bits as
    // quantising with kr_quantize_rows first.
    int a_q16;
};

// w8a8 quantisation rule, one scale per row (weights: rows of W^T; activations:
// rows = tokens):
//   amax = max_k |x[k]|;  s = amax / 127;  inv = 127 / amax   (IEEE fp32
//   divides; s = inv = 1 when amax = 0)
//   q[k] = the integer nearest to the exact product x[k] * inv, ties to even
// (|q| <= 127 since |x| <= amax). kr_q8_bits computes it with one FMA:
// x * inv + 1.5 * 2^23 lies in [2^23, 2^24), where float32 spacing is 1, so
// the FMA's single rounding is the integer rounding of x * inv, and the
// result's bits are 0x4B400000 + q: their low byte is q as two's complement.
__device__ __forceinline__ float kr_q8_inv(float amax) { return amax > 0.0f ? 127.0f / amax : 1.0f; }
__device__ __forceinline__ float kr_q8_scale(float amax) { return amax > 0.0f ? amax / 127.0f : 1.0f; }
__device__ __forceinline__ uint32_t kr_q8_bits(float x, float inv) {
    return __float_as_uint(__builtin_fmaf(x, inv, 12582912.0f));
}
// q of x0..x3 packed into bytes 0..3 (v_perm_b32 picks the low bytes).
__device__ __forceinline__ uint32_t kr_q8_pack4(float x0, float x1, float x2, float x3, float inv) {
    const uint32_t lo = __builtin_amdgcn_perm(kr_q8_bits(x1, inv), kr_q8_bits(x0, inv), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(kr_q8_bits(x3, inv), kr_q8_bits(x2, inv), 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Fragment-packed layout of an [R, K] fp16 operand (K % 32 == 0, R padded to
// a multiple of 16): the 16 x 32 block (R/16 = rb, K/32 = kb) is one
// contiguous 1 KB run at block index rb * (K/32) + kb, stored in the order
// the v_mfma_f32_16x16x32_f16 operand registers want it: lane
// l = (r % 16) + 16 * ((k % 32) / 8) holds the 8 halves k % 8 = 0..7. One
// wave's operand load is then a single fully coalesced 1 KB read.
__host__ __device__ inline size_t kr_frag_index(long long r, long long k, long long K) {
    return ((size_t)((r >> 4) * (K >> 5) + (k >> 5)) * 64 +
            (size_t)((r & 15) + 16 * ((k & 31) >> 3))) * 8 + (size_t)(k & 7);
}
// int8 operands use the same bytes per block: a 16 x 64 int8 block is the
// 16 x 32 block of the 16-bit view (byte pairs), so lane r%16 + 16*((k%64)/16)
// holds the 16 consecutive k of one row - the v_mfma_i32_16x16x64_i8 operand.
__host__ __device__ inline size_t kr_frag_index_i8(long long r, long long k, long long K) {
    return 2 * kr_frag_index(r, k >> 1, K >> 1) + (size_t)(k & 1);
}
// Rows of a fragment-packed operand with R logical rows (multiple of 16).
__host__ __device__ inline long long kr_frag_rows(long long R) { return (R + 15) / 16 * 16; }

// The canonical reduction is split-K over 256-wide slices of K (K % 256 == 0).
#define KR_GEMM_KSPLIT 256
#define KR_GEMM_MAX_JOBS 3
// Products with M <= KR_GEMM_SMALL_M (and N < 16384) take the small-M kernel,
// which also reads and writes fragment-packed operands.
#define KR_GEMM_SMALL_M 512
#define KR_GEMM_SMALL_MAX_N 16384

// Up to three products with the same M and K in one launch.
struct kr_gemm_multi {
    kr_gemm_args job[KR_GEMM_MAX_JOBS];
    int ep[KR_GEMM_MAX_JOBS];
    int tiles[KR_GEMM_MAX_JOBS];
    int njobs;
    // decode-step timing (null otherwise): wave w of workgroup b stores its
    // start and end times (the 100 MHz steady counter) at stamps[16 b + w]
    unsigned long long* stamps;
};

// Launch C = A @ W (W given transposed), kernel and tile shape chosen from M.
// Reduction contract (fp16), whatever the kernel: for every output element,
//   P_s = chain of v_mfma_f32_16x16x32_f16 over k = 256s, 256s+32, ..., 256s+224
//         starting from zero (s = 0 .. K/256 - 1),
//   acc = P_0; acc = acc + P_1; ...; acc = acc + P_{S-1}   (fp32 adds, in order),
// then the epilogue. A row therefore gets identical bits for any M. The int8
// path accumulates exactly in int32, so any order gives the same bits.
int kr_gemm_launch(const kr_gemm_args& g, int epilogue, hipStream_t stream);

// Kernel timing for the decode-step profiler: the next small-M panel launch
// on this host thread (kr_gemm_launch / kr_gemm_launch_multi choosing
// gemm_panel_kernel) with at most max_groups workgroups gets `stamps`
// (2 x KR_STAMP_WAVES x max_groups u64, see kr_gemm_multi) and stores each
// wave's start and end times there, also when it is captured in a graph
// (then at every replay). Arm with a buffer, disarm with nullptr.
// kr_gemm_timed_launch_taken(): the grid size of the panel launch that took
// the buffer since it was armed; 0 if none came; minus the grid size if one
// came with more than max_groups workgroups (it ran untimed).
// With start / stop events as well (an eager launch; not under stream
// capture) the launch goes through hipExtLaunchKernel, whose events take the
// dispatch's own start and end times.
constexpr int KR_STAMP_WAVES = 16;
void kr_gemm_time_next_panel(unsigned long long* stamps, int max_groups,
                             hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
int kr_gemm_timed_launch_taken();
// Several products; on the small-M path those sharing M and K run in one
// launch (independent outputs), otherwise they are launched in order.
// Width (in 16-column panels) of the column groups the small-M fragment
// kernel uses for these jobs launched together. When a job has a multiple of 8
// groups, XCD x takes its groups x, x + 8, ... (workgroups are dealt to the
// XCDs round robin), so a caller can stage each XCD's weight panels in that
// XCD's L2 ahead of the launch.
int kr_gemm_panel_ns(const kr_gemm_args* jobs, int njobs);

int kr_gemm_launch_multi(const kr_gemm_args* jobs, const int* epilogues, int njobs,
                         hipStream_t stream);

// The head (logits = fp16(LN_out(x) @ head)) has a reduction contract of
// its own, which the two head kernels below share and no other product uses:
//   acc = chain of v_mfma_f32_16x16x32_f16 over k = 0, 32, ..., K - 32 from
//         zero (one chain, no slice partials), out = fp16(acc).
// A row's logits are therefore the same bits for any M and either kernel.
// The decode head holds the whole K of its rows in one wave, so one chain
// costs it nothing; the large-M head gains a 256 x 256 tile from the
// registers the slice partials would take.

// out[M, N] (row stride ldo) = fp16(A @ W) for the small-M head (M <= 512,
// K in {256, 512, 768}): A fragment-packed [M rows padded to 16, K], W^T
// fragment-packed [N padded to 16, K].
bool kr_gemm_head_small_ok(int M, int N, int K);
int kr_gemm_head_small(const kr_half* Af, const kr_half* Wf, int M, int N, int K, kr_half* out,
                       long long ldo, hipStream_t stream);
// The same product for any M: A [M, K] row-major (row stride lda), W^T [N, K]
// row-major (row stride ldw); K % 64 == 0, lda and ldw multiples of 8,
// A and Wt 16-byte aligned, N * ldw * 2 < 2^31.
int kr_gemm_head_big(const kr_half* A, long long lda, const kr_half* Wt, long long ldw, int M,
                     int N, int K, kr_half* out, long long ldo, hipStream_t stream);
// The 256 x 256 persistent kernel (kr_wide.hip) on one product without slice
// partials: the head (KR_EP_F16, fp16 operands) or any epilogue on int8
// operands (w8a8, exact int32 sums). Needs K a whole number of 128-byte
// steps, 16-byte aligned operand rows, and N * (W^T row bytes) < 2^31.
int kr_gemm_launch_wide(const kr_gemm_args& g, int epilogue, hipStream_t stream);


// Per-row symmetric int8 quantisation of an fp16 [M, K] matrix (kr_quant.hip).
int kr_impl_quantize_rows(const void* x, long long ldx, int M, int K, void* q, float* scales,
                          int packed, hipStream_t s);
