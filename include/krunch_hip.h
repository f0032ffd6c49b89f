/*
 * krunch_hip.h — C ABI of libkrunch_hip.so, the MI355X (gfx950) engine for
 * krunch's batched RWKV-4 compress/decompress path.
 *
 * Conventions (all entry points):
 *   - device pointers and plain sizes only; `stream` is a hipStream_t (NULL =
 *     the default stream); launches are asynchronous, nothing synchronises
 *     unless stated;
 *   - return 0 on success, a negative code on failure; kr_last_error() gives
 *     the message (thread-local);
 *   - the caller owns every buffer; coder states and RNN states are mutated
 *     in place (as the reference's ops do, krunch_ac/cuda/main.cpp:111-130);
 *   - fp16 tensors are passed as uint16_t bit patterns;
 *   - cdf_precision is log2 of the CDF total (24 in the reference,
 *     krunch_ac/cdf.py:18-19; range_coder.cuh:19-20).
 *
 * Each declaration names the reference interface it replaces.
 */
#ifndef KRUNCH_HIP_H
#define KRUNCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- errors */
const char* kr_last_error(void);
int kr_abi_version(void);

/* ------------------------------------------------------------ range coder
 * Coder state: 4 x uint32 per stream, {low, high, pending, bit_offset} for
 * encoding and {low, high, value, bit_offset} for decoding
 * (range_coder.cuh:24-40). Encoders start from {0, 0xFFFFFFFF, 0, 0} and OR
 * bits into a zero-filled output buffer; out_cap bounds every write (an
 * overflow sets *err_flag, which may be NULL). Decoders read zero bits past
 * the end of a stream: in_len bounds the whole input buffer, byte_limits
 * (nullable) each stream's own length. base_byte_offsets (nullable where
 * noted) gives each stream's first byte.
 */

/* replaces krunch_ac_cuda.encode_step (main.cpp encode_step; encode_kernel.cu:53-101):
 * N rows of one stream, full CDF rows of cdf_stride int32 entries. */
int kr_encode_step(const int32_t* cdf, int cdf_stride, const int32_t* symbols, int N,
                   uint8_t* output_buf, uint32_t out_cap, uint32_t* state, int cdf_precision,
                   uint32_t* err_flag, void* stream);

/* replaces krunch_ac_cuda.encode_finalize (encode_kernel.cu:106-119). */
int kr_encode_finalize(uint8_t* output_buf, uint32_t out_cap, uint32_t* state,
                       uint32_t* err_flag, void* stream);

/* replaces krunch_ac_cuda.encode_step_batched (encode_kernel.cu:148-197):
 * one symbol per stream, CDF rows [B, V+1]. */
int kr_encode_step_batched(const int32_t* cdfs, int V, const int32_t* symbols,
                           uint8_t* output_buf, uint32_t out_cap,
                           const int32_t* base_byte_offsets, uint32_t* states, int B,
                           int cdf_precision, uint32_t* err_flag, void* stream);

/* Fused-compress form of encode_step_batched over T steps: pairs[b*pair_stride+t]
 * = (cdf[sym], cdf[sym+1]) as produced by kr_softmax_cdf_pairs; stream b encodes
 * its first n_valid[b] rows (n_valid nullable = T). No reference counterpart: the
 * reference writes full [rows, V+1] CDFs and reads two entries per row
 * (cpp_path.py:499-500 + encode_kernel.cu:110-111). */
int kr_encode_pairs_batched(const uint32_t* pairs, int T, long long pair_stride,
                            const int32_t* n_valid, uint8_t* output_buf, uint32_t out_cap,
                            const int32_t* base_byte_offsets, uint32_t* states, int B,
                            int cdf_precision, uint32_t* err_flag, void* stream);

/* replaces krunch_ac_cuda.encode_finalize_batched (encode_kernel.cu:199-215);
 * base_byte_offsets nullable (all streams at offset 0 is then B = 1). */
int kr_encode_finalize_batched(uint8_t* output_buf, uint32_t out_cap,
                               const int32_t* base_byte_offsets, uint32_t* states, int B,
                               uint32_t* err_flag, void* stream);

/* replaces krunch_ac_cuda.decode_init_batched and, with B = 1 and NULL offsets,
 * decode_init (decode_kernel.cu:28-45,138-157). */
int kr_decode_init_batched(const uint8_t* input_buf, uint32_t in_len,
                           const int32_t* base_byte_offsets, const int32_t* byte_limits,
                           uint32_t* states, int B, void* stream);

/* replaces krunch_ac_cuda.decode_step_batched and, with B = 1, decode_step
 * (decode_kernel.cu:50-110,159-216): CDF rows [B, V+1] -> out_syms [B]. */
int kr_decode_step_batched(const int32_t* cdfs, int V, const uint8_t* input_buf,
                           uint32_t in_len, const int32_t* base_byte_offsets,
                           const int32_t* byte_limits, uint32_t* states, int32_t* out_syms,
                           int B, int cdf_precision, void* stream);

/* -------------------------------------------------------------------- CDF
 * One 1024-thread workgroup per row. V <= 65032 or V = 65536: a row is held
 * in registers as at most 512 leaves of numpy's pairwise summation, and
 * V in 65033..65535 needs 513 (KR_EUNSUPPORTED). Probabilities are
 * renormalised with numpy's float32 summation order, so results are
 * bit-identical to krunch_ac/cdf.py:22-74. Softmax of fp16 logits (row
 * stride ld elements): e = exp(x - max) with a fixed FMA-based routine,
 * q = e * (1 / sum e), then cdf.py on q.
 */

/* replaces krunch_ac.probs_to_cdf (cdf.py:22-74) / probs_to_cdf_gpu
 * (gpu_encode.py:22-48): float probs [N, ld] -> uint32 cdf [N, V+1]. */
int kr_probs_to_cdf(const float* probs, int N, int V, long long ld, uint32_t* cdf_out,
                    int cdf_precision, void* stream);

/* replaces krunch_ac_cuda.det_softmax_cdf (det_softmax_cdf.cu:62-195) and the
 * caller's cumsum (cpp_path.softmax_cdfs_per_row, :490-501): out [N, V+1] int32
 * holds the cumulative CDF (cumulative = 1) or 0 followed by the per-symbol
 * counts (cumulative = 0, the reference op's output). */
int kr_softmax_cdf(const uint16_t* logits, int N, int V, long long ld, int32_t* out,
                   int cumulative, int cdf_precision, void* stream);

/* The softmax probabilities q [N, V] fed to the CDF (test and inspection aid;
 * the reference's torch.softmax in inference.py:254 plays this role). */
int kr_softmax_probs(const uint16_t* logits, int N, int V, long long ld, float* probs,
                     void* stream);

/* Fused compress stage: per row only the interval of symbols[row],
 * pairs[row] = (cdf[sym], cdf[sym+1]) — replaces det_softmax_cdf + cumsum +
 * the coder's two reads (cpp_path.py:499-500, encode_kernel.cu:110-111). */
int kr_softmax_cdf_pairs(const uint16_t* logits, int N, int V, long long ld,
                         const int32_t* symbols, uint32_t* pairs, int cdf_precision,
                         void* stream);

/* Fused decompress stage for B streams (one row of logits each): CDF, search
 * for the decoder target, range decode; writes out_syms[b] and, if tokens is
 * given, tokens[b*tok_stride + tok_count[b]++]. Streams with
 * tok_count[b] >= n_tokens[b] are skipped (n_tokens nullable). Replaces
 * softmax_cdfs_per_row + decode_step_batched (inference.py:427-431). */
int kr_softmax_cdf_decode(const uint16_t* logits, int B, int V, long long ld,
                          const uint8_t* input_buf, uint32_t in_len,
                          const int32_t* base_byte_offsets, const int32_t* byte_limits,
                          uint32_t* states, int32_t* out_syms, int32_t* tokens,
                          long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                          int cdf_precision, void* stream);

/* ------------------------------------------------------------ GEMM / model
 * Matrices of the model are stored transposed, [out, in] (K contiguous).
 * Every output element is reduced the same way whatever M or the kernel:
 * P_s = chain of v_mfma_f32_16x16x32_f16 over the 256-wide K slice s (from
 * zero), acc = P_0 + P_1 + ... added left to right in fp32; so a row's
 * result does not depend on how many rows share the call (K % 256 == 0).
 */

/* W [K, N] (row stride ldw) -> Wt [N, K] (row stride ldt), fp16. */
int kr_transpose_f16(const uint16_t* W, long long ldw, int K, int N, uint16_t* Wt,
                     long long ldt, void* stream);

/* replaces krunch_ac_cuda.det_matmul (layer_cpp.cpp:728-822, det_matmul_tc*.cu):
 * out = epilogue(x [M,K] @ W) with W given as Wt [N, ldw]. epilogue: 0 fp32 out,
 * 1 fp16 out, 2 fp16 sigmoid, 3 fp16 relu^2, 4 fp16 res + acc, 5 fp16
 * res + gate * acc (res/gate [M, ldo] fp16, res may alias out). */
int kr_det_matmul(const uint16_t* x, int M, int K, const uint16_t* Wt, long long ldw, int N,
                  void* out, long long ldo, int epilogue, const uint16_t* res,
                  const uint16_t* gate, void* stream);

/* Fragment-packed copy of Wt [N, K] (row stride ld) for the small-M GEMM: each
 * 16-row x 32-column block is one contiguous 1 KB run in MFMA operand order
 * (no reference counterpart: the reference's WMMA kernels read row-major
 * weights, layer_cpp.cpp:206-290). Output holds kr_fragment_bytes(N, K) bytes,
 * rows padded to a multiple of 16 with zeros; K % 32 == 0. */
size_t kr_fragment_bytes(int N, int K);
int kr_pack_fragments(const uint16_t* Wt, long long ld, int N, int K, uint16_t* out,
                      void* stream);

/* kr_det_matmul on fragment-packed operands (the stepped decode's GEMM): xf is
 * x [M, K] packed by kr_pack_fragments (rows padded to 16), Wf is Wt [N, K]
 * packed; M <= 512, N < 16384. out_packed = 1 writes an fp16 result packed as
 * an [M, N] operand of the next product (elementwise fp16 epilogues only,
 * N % 32 == 0). Same bits as kr_det_matmul on the unpacked operands. */
int kr_det_matmul_packed(const uint16_t* xf, int M, int K, const uint16_t* Wf, int N, void* out,
                         long long ldo, int epilogue, const uint16_t* res, const uint16_t* gate,
                         int out_packed, void* stream);

/* Up to three kr_det_matmul_packed products sharing M and K in one launch of
 * the small-M kernel (independent outputs, same bits as separate calls): the
 * stepped layer runs its channel-mix R (sigmoid) and K (relu^2, packed
 * output) products this way. No reference counterpart: the reference runs
 * them as two matmuls (layer_cpp.cpp:623-628). M <= 512. */
typedef struct kr_packed_job {
    const uint16_t* xf;          /* x [M, K] fragment-packed */
    const uint16_t* Wf;          /* Wt [N, K] fragment-packed */
    int N;
    void* out;                   /* as kr_det_matmul_packed */
    long long ldo;
    int epilogue;
    const uint16_t* res;
    const uint16_t* gate;
    int out_packed;
} kr_packed_job;
int kr_det_matmul_packed_multi(const kr_packed_job* jobs, int n_jobs, int M, int K, void* stream);

/* w8a8 (the reference only sketches an int8 path,
 * docs/INT8_WEIGHTS_DESIGN.md): symmetric int8 with one fp32 scale per row,
 * amax = max|x|, s = amax / 127, inv = 127 / amax (both 1 when the row is
 * zero; IEEE float32 divides), q = the exact product x * inv rounded to the
 * nearest integer, ties to even (|q| <= 127).
 * Rows are tokens for activations and output channels (rows of Wt) for
 * weights. q is [M, K] row-major, or fragment-packed (packed = 1, rows padded
 * to 16, kr_quant_bytes) for the small-M GEMM; K % 64 == 0. */
size_t kr_quant_bytes(int M, int K, int packed);
int kr_quantize_rows(const uint16_t* x, long long ldx, int M, int K, int8_t* q, float* scales,
                     int packed, void* stream);

/* int8 GEMM: acc = sum_k xq[m,k] * wq[n,k] exactly in int32, value =
 * (float(acc) * sa[m]) * sw[n], then the epilogue of kr_det_matmul. packed = 1:
 * xq and wq fragment-packed (wq packed by kr_pack_fragments on its 16-bit
 * view, K/2 columns), M <= 512; packed = 0: both row-major [*, K];
 * packed = 2: as 1, but xq points to fp16 activations, fragment-packed
 * (kr_pack_fragments layout), which the product quantises per row on load
 * by the rule above (sa is not read and may be null) - for finite
 * activations, the same bits as kr_quantize_rows followed by packed = 1, in
 * one launch (the row maximum compares fp16 bit patterns, so a NaN in a row
 * gives that row a NaN scale, where kr_quantize_rows' fmaxf skips it). */
int kr_det_matmul_i8(const int8_t* xq, const float* sa, int M, int K, const int8_t* wq,
                     const float* sw, int N, void* out, long long ldo, int epilogue,
                     const uint16_t* res, const uint16_t* gate, int packed, void* stream);

/* w8a8 copy of one matrix (kr_quantize_rows on Wt: one scale per output channel). */
typedef struct kr_matrix_q8 {
    const int8_t* q;                      /* [N, K] row-major int8 (rows = output channels) */
    const int8_t* qf;                     /* the same fragment-packed (16-bit view, K/2 columns) */
    const float* scale;                   /* [N] */
} kr_matrix_q8;

typedef struct kr_layer_q8 {
    kr_matrix_q8 K, V, R, O, fK, fV, fR;
} kr_layer_q8;

typedef struct kr_layer_weights {
    const void *ln1_w, *ln1_b;            /* fp16 [C] */
    const void *tm_k, *tm_v, *tm_r;       /* fp16 [C] */
    const float *decay;                   /* fp32 [C], w = -exp(time_decay_raw) */
    const float *first;                   /* fp32 [C], u = time_first */
    const void *Kt, *Vt, *Rt, *Ot;        /* fp16 [C, C] */
    const void *ln2_w, *ln2_b;            /* fp16 [C] */
    const void *ftm_k, *ftm_r;            /* fp16 [C] */
    const void *fKt;                      /* fp16 [F, C] */
    const void *fVt;                      /* fp16 [C, F] */
    const void *fRt;                      /* fp16 [C, C] */
    /* Fragment-packed copies of the seven matrices above (kr_pack_fragments),
     * read by the small-M (B*T <= 512) path; all NULL = use the row-major ones. */
    const void *Kf, *Vf, *Rf, *Of, *fKf, *fVf, *fRf;
    /* w8a8 codec: int8 copies of the seven matrices; the
     * layer then runs its GEMMs on int8 MFMA with per-token activation
     * quantisation. NULL = fp16 codec. The head stays fp16 either way. */
    const kr_layer_q8* q8;
} kr_layer_weights;

typedef struct kr_model_weights {
    int n_layer, C, F, V;                 /* C in {256,512,768,1024}, F % 64 == 0, V <= 65536 */
    const void* emb;                      /* fp16 [V, C] */
    const void *ln_out_w, *ln_out_b;      /* fp16 [C] */
    const void* headT;                    /* fp16 [V, C] */
    const kr_layer_weights* layers;       /* host array, n_layer entries */
    /* Fragment-packed copy of headT (kr_pack_fragments), read by the decode
     * head (M <= 512 rows, C <= 768); NULL = the row-major head. */
    const void* headF;
} kr_model_weights;

/* w = -exp(raw) for the WKV decay (the rwkv loader's transform the reference
 * relies on, wkv_kernel.cu:41-45). */
int kr_prepare_decay(const float* raw, float* out, int n, void* stream);

/* RNN state of B streams for n_layer layers in one buffer; per layer
 * [att_xx fp16 | ffn_xx fp16 | aa | bb | pp fp32], each [B, C]
 * (cpp_path.fresh_state_batched, cpp_path.py:412-425). */
size_t kr_state_bytes(int n_layer, int B, int C);
/* att_xx = ffn_xx = aa = bb = 0, pp = -1e30 (fill kernel, graph-safe). */
int kr_state_init(void* state, int n_layer, int B, int C, void* stream);

/* Scratch needed by the layer stack for M = B*T rows. */
size_t kr_forward_workspace_bytes(long long M, int C, int F);

/* replaces krunch_ac_cuda.rwkv4_layer_step_cpp / _t1 (layer_cpp.cpp:294-637):
 * one layer over x [B*T, C] fp16 in place, state tensors [B, C] mutated. */
int kr_layer_step(const kr_layer_weights* L, int C, int F, void* x, int B, int T,
                  void* att_xx, float* aa, float* bb, float* pp, void* ffn_xx, void* ws,
                  size_t ws_bytes, void* stream);

/* kr_layer_step without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace is a static device array of KR_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends; nothing is allocated or freed. A call whose
 * kr_forward_workspace_bytes(B*T, C, F) exceeds it fails (KR_EINVAL): at
 * C = 768, F = 3072 that is B*T <= 1024 rows. Every call on one GPU shares
 * the array, so calls that overlap on one GPU (other streams or threads)
 * race; consecutive calls on one stream do not. Same kernels and bits as
 * kr_layer_step. */
#define KR_NOALLOC_SCRATCH_BYTES (32u << 20)
int kr_layer_step_noalloc(const kr_layer_weights* L, int C, int F, void* x, int B, int T,
                          void* att_xx, float* aa, float* bb, float* pp, void* ffn_xx,
                          void* stream);

/* Layer phase profiler; replaces the reference's KRUNCH_PHASE_PROFILE
 * profiler with read_phase_times / reset_phase_times (layer_cpp.cpp:111-157,
 * 825-836). When on, every kr_layer_step call (outside stream capture)
 * records HIP events between its phases on its stream, waits for the last one
 * and adds the elapsed milliseconds to running sums. The phases (this build's
 * kernel split; a fused launch leaves the phase it absorbed empty) are
 * kr_phase_name(0..kr_phase_count()-1): ln1_mix, kvr_matmul, wkv,
 * ow_matmul_residual, ln2_mix, ffn_rk_matmul, ffn_v_matmul_residual.
 * kr_phase_profile(1 / 0) turns it on / off and returns the previous state
 * (-1 only queries); KRUNCH_PHASE_PROFILE=1 turns it on at first use. */
int kr_phase_profile(int enable);
int kr_phase_count(void);
const char* kr_phase_name(int i);
int kr_read_phase_times(double* ms, int n, long long* call_count);
int kr_reset_phase_times(void);

/* Decode-step timing, the same profiler's role (layer_cpp.cpp:111-157) for
 * the stepped decode. kr_step_timing(p) with p = 3 (ow_matmul_residual),
 * 5 (ffn_rk_matmul) or 6 (ffn_v_matmul_residual) times that phase's product
 * in every layer of every later decode step (kr_decode_step, kr_decode_run,
 * graph or eager): each of its waves stores its start and end on the GPU's
 * 100 MHz steady counter (a vector store per wave, also at every replay of a
 * captured graph), and in eager steps the launch goes through
 * hipExtLaunchKernel with two HIP events that take its dispatch's start and
 * end. Nothing else in the step changes. p = -1 turns it off; *previous
 * (nullable) receives the earlier setting. kr_step_timing_read waits for the
 * device and writes, for layers 0 .. n_read - 1 of the last timed step
 * (n_read = min(n, layers)), the launch's event duration (-1 for a graph
 * step) and its wave span (last wave end minus first wave start), in
 * microseconds; it fails if no timed step ran since the last reading. */
int kr_step_timing(int phase, int* previous);
int kr_step_timing_read(double* launch_us, double* span_us, int n, int* n_read);

/* replaces launch_krunch_wkv_forward (wkv_kernel.cu:75-92), fused with the
 * receptance: ry = fp16(r * fp16(y)); k, v fp32 [B*T, C], r/ry fp16. */
int kr_wkv(int B, int T, int C, const float* decay, const float* first, const float* k,
           const float* v, const uint16_t* r, float* aa, float* bb, float* pp, uint16_t* ry,
           void* stream);

/* All layers over x [B*T, C] (cpp_path.forward_packed_window's layer loop,
 * :155-160; forward_stepped_batched's with T = 1, :451-456). */
int kr_forward_layers(const kr_model_weights* m, void* x, int B, int T, void* state, void* ws,
                      size_t ws_bytes, void* stream);

/* x[row] = emb[ids[row]] (cpp_path.py:154,450). */
int kr_embed(const kr_model_weights* m, const int32_t* ids, int M, void* x, void* stream);

/* logits [M, ld] fp16 = LN_out(x) @ head (cpp_path.py:161-163); xn: [M, C] scratch.
 * The head has a reduction of its own: for every logit one chain of
 * v_mfma_f32_16x16x32_f16 over the whole K = C from zero, then fp16; the
 * same bits for any M, with or without headF (decode and compress agree). */
int kr_head_logits(const kr_model_weights* m, const void* x, int M, void* xn, void* logits,
                   long long ld, void* stream);

/* One packed compress window for B streams x T tokens (rows b*T + t): embed,
 * layers, then per block of head_rows rows head logits -> softmax -> symbol
 * interval into pairs [B*T, 2]. Replaces the per-window body of
 * InferenceEngine._compress_chunk_cpp (inference.py:331-338). Encode the pairs
 * with kr_encode_pairs_batched. */
int kr_compress_window(const kr_model_weights* m, const int32_t* inputs, const int32_t* targets,
                       int B, int T, void* state, void* x, void* ws, size_t ws_bytes,
                       void* logits, long long ld, int head_rows, uint32_t* pairs,
                       int cdf_precision, void* stream);

/* One stepped decompress step for B streams: embed syms, layers (T = 1), head,
 * fused CDF + range decode; syms is read (previous tokens) and overwritten
 * (decoded tokens). Replaces one iteration of the loop in
 * _decompress_chunks_batched_cpp (inference.py:427-434). */
int kr_decode_step(const kr_model_weights* m, int B, void* state, int32_t* syms, void* x,
                   void* ws, size_t ws_bytes, void* logits, long long ld,
                   const uint8_t* input_buf, uint32_t in_len, const int32_t* base_byte_offsets,
                   const int32_t* byte_limits, uint32_t* ac_states, int32_t* tokens,
                   long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                   int cdf_precision, void* stream);

/* n_steps decode steps. The B streams are split into n_groups groups of
 * ceil(B/n_groups) streams with independent workspaces (ws_bytes >=
 * kr_decode_workspace_bytes); with use_graph one step is captured into a HIP
 * graph whose groups are parallel branches, so their latency-bound kernels
 * overlap, and the graph is replayed n_steps times (the reference's graph
 * path, cpp_path.py:229-276). With one group, the graph's decode kernel also
 * runs layer 0's LN1-mix of each decoded symbol for the next step (a first-
 * step graph and a later-steps graph); the state, tokens and coder state it
 * leaves are those of the eager path (use_graph = 0), x and ws are scratch.
 * Synchronous with respect to the work it enqueues. */
size_t kr_decode_workspace_bytes(int B, int n_groups, int C, int F);
int kr_decode_run(const kr_model_weights* m, int B, void* state, int32_t* syms, void* x,
                  void* ws, size_t ws_bytes, void* logits, long long ld,
                  const uint8_t* input_buf, uint32_t in_len, const int32_t* base_byte_offsets,
                  const int32_t* byte_limits, uint32_t* ac_states, int32_t* tokens,
                  long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                  int cdf_precision, int n_steps, int n_groups, int use_graph, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KRUNCH_HIP_H */
