/* Oracle (TEST INFRASTRUCTURE ONLY): y = x @ W in float32 with one fixed
 * summation order per output, y[m][n] = (((0 + x[m][0]*W[0][n]) + x[m][1]*W[1][n])
 * + ...) over k = 0..K-1, every product and sum rounded on its own
 * (-ffp-contract=off, no fast-math). The order depends on nothing but k, so a
 * row's result is the same whichever rows share the call: the CPU restatement
 * of the forward is then packed == stepped bit for bit, as the reference's
 * deterministic GEMM makes its GPU path (layer_cpp.cpp:206-290,
 * det_matmul_tc*.cu), and a CPU compress/decompress round trip is byte-exact.
 *
 * Blocking only changes which outputs are in flight together (8 rows x 64
 * columns accumulate in a local array, the column loop vectorises across n);
 * rows or column blocks are shared out over OpenMP threads.
 */
#include <stddef.h>
#include <string.h>

#define RB 8
#define NB 64

static void block(const float* x, int K, const float* W, int N, float* y, int m0, int rows,
                  int n0, int cols) {
    float acc[RB][NB];
    memset(acc, 0, sizeof acc);
    for (int k = 0; k < K; k++) {
        const float* w = W + (size_t)k * N + n0;
        for (int r = 0; r < rows; r++) {
            const float a = x[(size_t)(m0 + r) * K + k];
            float* c = acc[r];
            for (int j = 0; j < cols; j++) c[j] = c[j] + a * w[j];
        }
    }
    for (int r = 0; r < rows; r++) memcpy(y + (size_t)(m0 + r) * N + n0, acc[r], sizeof(float) * cols);
}

void orc_gemm_rows(const float* x, int M, int K, const float* W, int N, float* y) {
    const int mb = (M + RB - 1) / RB, nb = (N + NB - 1) / NB;
    const long tiles = (long)mb * nb;
#pragma omp parallel for schedule(dynamic, 1)
    for (long t = 0; t < tiles; t++) {
        const int bm = (int)(t / nb), bn = (int)(t % nb);
        const int m0 = bm * RB, n0 = bn * NB;
        const int rows = M - m0 < RB ? M - m0 : RB;
        const int cols = N - n0 < NB ? N - n0 : NB;
        block(x, K, W, N, y, m0, rows, n0, cols);
    }
}
