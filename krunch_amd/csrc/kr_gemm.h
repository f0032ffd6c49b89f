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
    const kr_half* A;   // [M, K] row-major, row stride lda
    long long lda;
    const kr_half* Wt;  // [N, K] row-major (W transposed), row stride ldw
    long long ldw;
    void* out;          // [M, N], row stride ldo (f32 or f16 per epilogue)
    long long ldo;
    const kr_half* res;   // [M, N] stride ldo (RESID, GATED); may alias out
    const kr_half* gate;  // [M, N] stride ldo (GATED)
    int M, N, K;
};

// The canonical reduction is split-K over 256-wide slices of K (K % 256 == 0).
#define KR_GEMM_KSPLIT 256
#define KR_GEMM_MAX_JOBS 3

// Up to three products with the same M and K in one launch.
struct kr_gemm_multi {
    kr_gemm_args job[KR_GEMM_MAX_JOBS];
    int ep[KR_GEMM_MAX_JOBS];
    int tiles[KR_GEMM_MAX_JOBS];
    int njobs;
};

// Launch C = A @ W (W given transposed), kernel and tile shape chosen from M.
// Reduction contract, whatever the kernel: for every output element,
//   P_s = chain of v_mfma_f32_16x16x32_f16 over k = 256s, 256s+32, ..., 256s+224
//         starting from zero (s = 0 .. K/256 - 1),
//   acc = P_0; acc = acc + P_1; ...; acc = acc + P_{S-1}   (fp32 adds, in order),
// then the epilogue. A row therefore gets identical bits for any M.
int kr_gemm_launch(const kr_gemm_args& g, int epilogue, hipStream_t stream);
// Several products; on the small-M path those sharing M and K run in one
// launch (independent outputs), otherwise they are launched in order.
int kr_gemm_launch_multi(const kr_gemm_args* jobs, const int* epilogues, int njobs,
                         hipStream_t stream);

