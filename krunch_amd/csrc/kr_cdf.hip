// Row-wise probabilities -> integer CDF on the GPU, bit-exact with the spec
// krunch_ac/cdf.py:22-74, optionally preceded by the deterministic softmax
// of fp16 logits (the role of det_softmax_cdf.cu:62-185 in the reference).
//
// One 1024-thread workgroup per row. The row's values live in registers in
// the layout of numpy's float32 pairwise summation: the row is split into
// 8192-element blocks, each block recursively halved (split rounded down to a
// multiple of 8) into leaves of <= 128 elements; a leaf is summed by 8
// interleaved accumulators (element i goes to accumulator i % 8), the 8
// accumulators are combined as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) and the
// len % 8 tail is added in order. One group of 8 lanes owns one leaf (lane j
// holds accumulator j's elements plus tail element j), so the 8-way combine
// is an xor-butterfly over lanes 1, 2, 4. Inner nodes of the recursion are
// combined level by level in LDS from a host-built plan; block sums are added
// left to right onto 0. The result equals numpy's `p.sum(axis=1)` bit for
// bit, which cdf.py uses to renormalise.
//
// Modes: materialise the CDF (or per-symbol counts, the reference's
// det_softmax_cdf output), write the probabilities, emit only the
// (cdf[sym], cdf[sym+1]) interval of a given symbol per row (compress), or
// find the symbol whose interval contains a range decoder's target and
// advance the decoder (decompress, fused).
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <vector>
#include <algorithm>

#include "kr_math.h"
#include "kr_rc_device.h"
#include "kr_rowops.h"
#include "kr_wave.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kLeavesPerIt = kWaves * 8;     // 128 leaves per register slice
constexpr int kMaxIt = 4;                    // up to 512 leaves: V <= 65536
constexpr int kMaxLeaves = kMaxIt * kLeavesPerIt;
constexpr int kMaxNodes = 2 * kMaxLeaves;
constexpr int kMaxLevels = 16;               // tree height above the leaves
constexpr int kMaxBlocks = 8;                // 8192-element blocks: V <= 65536

enum : int { IN_LOGITS_F16 = 0, IN_PROBS_F32 = 1 };
enum : int { M_CDF = 0, M_COUNTS = 1, M_PROBS = 2, M_PAIRS = 3, M_DECODE = 4 };

struct PlanArgs {
    const int2* leaves;      // (start, len), index order
    const int2* inner;       // (left, right) node ids, grouped by level
    const int* level_start;  // n_levels + 1 offsets into inner
    const int* roots;        // node id of each 8192-block
    const int* wave_root;    // [kMaxIt * kWaves]: node id of the 8-leaf subtree a wave sums itself, or -1
    int V, n_leaves, n_inner, n_levels, n_blocks;
};

struct DecodeArgs {
    const uint8_t* in;
    uint32_t in_len;
    const int32_t* base;      // per-stream byte offset (nullable -> 0)
    const int32_t* limits;    // per-stream byte length (nullable)
    kr_rc_state* states;
    int32_t* out_syms;        // [B] symbol decoded this step
    int32_t* tokens;          // [B, tok_stride] decoded tokens (nullable)
    long long tok_stride;
    int32_t* tok_count;       // [B] tokens written so far (nullable)
    const int32_t* n_tokens;  // [B] stream length; finished streams are skipped (nullable)
    const kr_embed_mix* em;   // layer 0's LN1-mix of the decoded token (device; nullable)
};

struct RowShared {
    float node[kMaxNodes];
    int2 inner[kMaxLeaves];                  // the summation plan, copied once
    int level_start[kMaxLevels + 1];
    int roots[kMaxBlocks];
    int wave_root[kMaxIt * kWaves];
    int leaf_count[kMaxLeaves];
    int leaf_buf[128];
    float redf[kWaves];
    float redp[kWaves];
    int redi[kWaves];
    int redi2[kWaves];
    int redi3[kWaves];
    int redL[kWaves];
    float total;
    int amax, deficit, amax_leaf, hit_leaf, hit_start, hit_len;
    uint32_t target, hit_prefix;
    kr_rc_state dstate;       // decoder state (decode mode)
    kr_bit_window win;        // stream bits of this step (decode mode)
};

__device__ __forceinline__ float wave_max(float v) {
    return kr_wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ int wave_isum(int v) {
    return kr_wave_reduce(v, [](int a, int b) { return a + b; });
}
// (value desc, index asc) total order: the first maximum wins.
__device__ __forceinline__ bool better(float pv, int pi, float bv, int bi) {
    return pv > bv || (pv == bv && pi < bi);
}

// fp16 logits rows are first copied into LDS with 16-byte loads, then read in
// the scattered leaf layout from there: the leaf layout read straight from
// global memory requests every cache line about ten times. Element i sits at
// stage[pad + i + skew(i)]: pad makes the copied 16-byte chunks aligned, and
// skew adds 8 halves (16 bytes, 4 banks) per 128 elements past the unaligned
// head. Inside a full 8192-element block every leaf is 128 elements long, so
// without the skew the 8 leaves one gather instruction reads (8 lanes each)
// start 256 bytes apart, on the same 4 banks: an 8-way bank conflict.
// The last 136 halves are room for the gather's reads past the end of a leaf
// (up to 135 halves past a leaf's first staged element), discarded after.
constexpr int kStageMax = 65536 + 8 * (65536 / 128) + 16 + 136;

struct StageMap {
    int pad, head;
    __device__ __forceinline__ int at(int i) const {
        return pad + i + (i >= head ? ((i - head) >> 7) << 3 : 0);
    }
};

template <int IN>
__device__ __forceinline__ float load_val(const void* row, const kr_half* stage, StageMap sm, int i) {
    if constexpr (IN == IN_LOGITS_F16) return (float)stage[sm.at(i)];
    else return reinterpret_cast<const float*>(row)[i];
}

// A row's values in flight to the stage: every load of the row is issued
// before any is written (V <= 65536 is at most 8 chunks of 8 per thread), so
// staging costs one memory round trip, not one per chunk.
constexpr int kStageChunks = 8;
struct StagedRow {
    kr_half8 c[kStageChunks];
    kr_half h0, h1;   // this thread's element of the unaligned head / of the tail
};

// Load V fp16 values at rp (2-byte aligned) for the stage (see StageMap).
__device__ __forceinline__ StageMap stage_row_load(const kr_half* __restrict__ rp, int V, int tid,
                                                   StagedRow& r) {
    const int head = min((int)(((16 - ((uintptr_t)rp & 15)) & 15) >> 1), V);
    const int pad = (8 - head) & 7;
    const int nchunks = (V - head) / 8;
    #pragma unroll
    for (int u = 0; u < kStageChunks; u++) {
        const int c = tid + u * kThreads;
        if (c < nchunks) r.c[u] = *reinterpret_cast<const kr_half8*>(rp + head + 8 * c);
    }
    const int tail0 = head + 8 * nchunks;
    if (tid < head) r.h0 = rp[tid];
    if (tid >= 8 && tid - 8 < V - tail0) r.h1 = rp[tail0 + tid - 8];
    return StageMap{pad, head};
}

// Write what stage_row_load loaded into the stage.
__device__ __forceinline__ void stage_row_store(int V, kr_half* stage, int tid, StageMap sm,
                                                const StagedRow& r) {
    const int nchunks = (V - sm.head) / 8;
    #pragma unroll
    for (int u = 0; u < kStageChunks; u++) {
        const int c = tid + u * kThreads;
        if (c < nchunks)
            *reinterpret_cast<kr_half8*>(stage + sm.pad + sm.head + 8 * c + ((c >> 4) << 3)) = r.c[u];
    }
    const int tail0 = sm.head + 8 * nchunks;
    if (tid < sm.head) stage[sm.at(tid)] = r.h0;
    if (tid >= 8 && tid - 8 < V - tail0) stage[sm.at(tail0 + tid - 8)] = r.h1;
}

// Copy V fp16 values at rp (2-byte aligned) into the stage (see StageMap).
__device__ __forceinline__ StageMap stage_row(const kr_half* __restrict__ rp, int V, kr_half* stage,
                                              int tid) {
    StagedRow r;
    const StageMap sm = stage_row_load(rp, V, tid, r);
    stage_row_store(V, stage, tid, sm, r);
    return sm;
}

// The summation plan into LDS: all loads issued before the LDS writes.
__device__ __forceinline__ void copy_plan(const PlanArgs& P, RowShared& sh, int tid) {
    const bool a = tid < P.n_inner, b = tid <= P.n_levels, c = tid < P.n_blocks,
               d = tid < kMaxIt * kWaves;
    int2 vi = make_int2(0, 0);
    int vl = 0, vr = 0, vw = 0;
    if (a) vi = P.inner[tid];
    if (b) vl = P.level_start[tid];
    if (c) vr = P.roots[tid];
    if (d) vw = P.wave_root[tid];
    if (a) sh.inner[tid] = vi;
    if (b) sh.level_start[tid] = vl;
    if (c) sh.roots[tid] = vr;
    if (d) sh.wave_root[tid] = vw;
    for (int i = tid + kThreads; i < P.n_inner; i += kThreads) sh.inner[i] = P.inner[i];
}

// a / b correctly rounded (IEEE binary32, round to nearest), given
// y = RN(1 / b): Markstein's correction q + (a - b q) y of the faithful
// quotient q = RN(a y), with the residual exact by FMA. Equal to the
// division for normal operands and quotients (checked against a / b over
// ~10^9 operand pairs, every mantissa of several b near 1); three
// instructions instead of the full division sequence.
__device__ __forceinline__ float div_by(float a, float b, float y) {
    const float q = __fmul_rn(a, y);
    return __builtin_fmaf(__builtin_fmaf(-q, b, a), y, q);
}

__device__ __forceinline__ int leaf_full(int len) { return len >= 8 ? (len >> 3) : 0; }
__device__ __forceinline__ int leaf_rem(int len) { return len >= 8 ? (len & 7) : len; }

// The value of v in lane (lane + T) of the same 16-lane row (DPP row_shl:T).
// Read only by lanes at offset 0 or 8 of a row with T <= 7, whose source
// lanes lie inside the row.
template <int T>
__device__ __forceinline__ float row_shl(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 0x100 + T, 0xF, 0xF, false));
}

// Sum of all held values in numpy's order (see file header). Every thread
// returns the same value. Slots that hold no element of the row carry +0.0
// and are added unconditionally: x + 0.0 == x for every x except -0.0, and
// a signed zero can only decide the sign of a partial sum that is exactly
// zero, which then adds exactly into any nonzero sum, so only an all-zero
// row can differ (in the sign of its zero total).
// act[it]: the wave holds leaves in register slice it; tail[it]: some leaf
// of the wave's slice has a len % 8 tail (both wave-uniform).
__device__ float row_sum_numpy(const float (&v)[kMaxIt][17], const int (&len)[kMaxIt],
                               const bool (&act)[kMaxIt], const bool (&tail)[kMaxIt],
                               const PlanArgs& P, RowShared& sh, int lane, int wave) {
    const int grp = lane >> 3, j = lane & 7;
    #pragma unroll
    for (int it = 0; it < kMaxIt; it++) {
        if (!act[it]) continue;
        float r = v[it][0];
        #pragma unroll
        for (int k = 1; k < 16; k++) r = r + v[it][k];
        r = r + kr_xor<1>(r);
        r = r + kr_xor<2>(r);
        r = r + kr_xor<4>(r);
        // the len % 8 tail elements, in order, onto lane 0 of the group
        float res = len[it] >= 8 ? r : -0.0f;
        if (tail[it]) {
            const float t = v[it][16];
            res = res + t;
            res = res + row_shl<1>(t);
            res = res + row_shl<2>(t);
            res = res + row_shl<3>(t);
            res = res + row_shl<4>(t);
            res = res + row_shl<5>(t);
            res = res + row_shl<6>(t);
        }
        const int L = it * kLeavesPerIt + wave * 8 + grp;
        const int wr = sh.wave_root[it * kWaves + wave];   // wave-uniform
        if (wr >= 0) {
            // The wave's 8 leaves form a perfect subtree of the plan: its
            // three levels are the pairs (lane, lane ^ 8), ^ 16, ^ 32 of the
            // groups' lane 0 (left + right == right + left in IEEE).
            res = res + kr_xor<8>(res);
            res = res + kr_xor<16>(res);
            res = res + kr_xor<32>(res);
            if (lane == 0) sh.node[wr] = res;
        } else if (j == 0 && L < P.n_leaves) {
            sh.node[L] = res;
        }
    }
    __syncthreads();
    // Inner nodes level by level, then the blocks left to right, by wave 0
    // alone: a wave's LDS accesses execute in program order, so each level
    // reads the previous one's writes without a workgroup barrier. The next
    // level's child pairs are read ahead (levels hold <= 64 nodes at V <=
    // 65536; a larger level takes the loop).
    if (wave == 0) {
        int s = sh.level_start[0];
        int e = P.n_levels > 0 ? sh.level_start[1] : s;
        int2 ch = lane < e - s ? sh.inner[s + lane] : make_int2(0, 0);
        for (int lev = 0; lev < P.n_levels; lev++) {
            const int e2 = lev + 1 < P.n_levels ? sh.level_start[lev + 2] : e;
            const int2 nxt = lane < e2 - e ? sh.inner[e + lane] : make_int2(0, 0);
            if (lane < e - s) sh.node[P.n_leaves + s + lane] = sh.node[ch.x] + sh.node[ch.y];
            for (int idx = s + 64 + lane; idx < e; idx += 64) {
                const int2 c2 = sh.inner[idx];
                sh.node[P.n_leaves + idx] = sh.node[c2.x] + sh.node[c2.y];
            }
            __builtin_amdgcn_wave_barrier();
            ch = nxt;
            s = e;
            e = e2;
        }
        if (lane == 0) {
            float acc = 0.0f;
            for (int b = 0; b < P.n_blocks; b++) acc = acc + sh.node[sh.roots[b]];
            sh.total = acc;
        }
    }
    __syncthreads();
    return sh.total;
}

// Element index of slot k (0..16) of a leaf (start, len) held by lane j.
__device__ __forceinline__ int slot_index(int start, int len, int j, int k) {
    return k < 16 ? start + j + 8 * k : start + 8 * leaf_full(len) + j;
}

// floor(p * scale) as an int. From logits p >= 0 (or NaN), and truncation is
// the floor there: one conversion instead of a floor and a conversion.
template <int IN>
__device__ __forceinline__ int scaled_floor(float p, float scale) {
    if constexpr (IN == IN_LOGITS_F16) return (int)__fmul_rn(p, scale);
    else return (int)floorf(__fmul_rn(p, scale));
}

// 16-byte asynchronous copy global -> LDS: lane l writes LDS byte address
// lds + 16 l. The compiler does not count it: readers wait with an explicit
// s_waitcnt vmcnt(0) and a barrier.
__device__ __forceinline__ void lds_copy16(const void* src, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :: "s"(lds), "v"(src) : "memory", "m0");
}

// stage_row's layout for a 16-byte-aligned row whose last chunk of 8 lies
// inside its allocation (row stride a multiple of 8): chunk c at 16-byte unit
// c + c / 16, so unit 17 s + t holds chunk 16 s + t for t < 16 and unit
// 17 s + 16 is the skew gap. Each wave copy fills 64 consecutive units; a gap
// lane re-reads its neighbour's chunk (same cache line) and lanes past the
// row re-read the last chunk. Values past V (the row's padding) are never
// gathered as elements. The copies are left in flight.
__device__ __forceinline__ void stage_row_async(const kr_half* rp, int V, unsigned stage_lds,
                                                int lane, int wave) {
    const int nch = (V + 7) >> 3;
    const int last = nch - 1 + ((nch - 1) >> 4);           // unit of the last chunk
    // q is wave-uniform (the LDS base goes through an SGPR into M0)
    for (int q = __builtin_amdgcn_readfirstlane(wave); 64 * q <= last; q += kWaves) {
        const int u = 64 * q + lane;
        const int s = (u * 61681) >> 20;                    // u / 17 for u < 20000
        const int c = min(16 * s + min(u - 17 * s, 15), nch - 1);
        lds_copy16(rp + 8 * c, stage_lds + 1024u * (unsigned)q);
    }
}

// One row of the CDF stage. async_stage: the row is already being copied
// into the stage (stage_row_async) and, once it is gathered, the copy of
// next_row (>= 0) is started, to land while this row is computed.
template <int IN, int MODE>
__device__ __forceinline__ void cdf_row(const void* __restrict__ input, long long ld, int row,
                                        int next_row, const PlanArgs& P, int prec,
                                        void* __restrict__ out, long long out_ld,
                                        const int32_t* __restrict__ symbols, const DecodeArgs& D,
                                        RowShared& sh, kr_half* stage, unsigned stage_lds,
                                        bool async_stage) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 3, j = lane & 7;
    const int V = P.V;

    const char* rowp;
    if constexpr (IN == IN_LOGITS_F16)
        rowp = reinterpret_cast<const char*>(input) + (size_t)row * (size_t)ld * 2;
    else
        rowp = reinterpret_cast<const char*>(input) + (size_t)row * (size_t)ld * 4;

    // Decode: the decoder state and the stream bits this step will consume
    // (lane 0), the logits row and the summation plan are all requested
    // before anything waits, so the prologue costs about two memory round
    // trips (state, then the bits at its offset). Loads retire in order: the
    // state goes out first so that waiting for it does not wait for the row.
    kr_rc_state dst{};
    kr_bit_window win{};
    StageMap pad{0, 0};
    if constexpr (MODE == M_DECODE) {
        static_assert(IN == IN_LOGITS_F16, "decode reads fp16 logits");
        uint32_t o = 0, lim_cap = 0xFFFFFFFFu;
        if (tid == 0) {
            dst = D.states[row];
            o = D.base ? (uint32_t)D.base[row] : 0u;
            if (D.limits) lim_cap = (uint32_t)D.limits[row];
        }
        StagedRow staged;
        pad = stage_row_load(reinterpret_cast<const kr_half*>(rowp), V, tid, staged);
        // Finished streams decode nothing this step (uniform per workgroup);
        // layer 0 still takes their last symbol, as its own LN1-mix would
        // (after the staged row has left the registers it holds).
        const bool finished = D.n_tokens && D.tok_count && D.tok_count[row] >= D.n_tokens[row];
        if (!finished && tid == 0) {
            uint32_t lim = D.in_len > o ? D.in_len - o : 0u;
            if (lim_cap < lim) lim = lim_cap;
            win.open(D.in + (o < D.in_len ? o : 0u), lim, dst.bit_offset);
        }
        copy_plan(P, sh, tid);
        stage_row_store(V, stage, tid, pad, staged);
        if (finished) {
            if (D.em && wave == 0) embed_mix(*D.em, (size_t)row, D.out_syms[row], lane);
            return;
        }
    }

    if constexpr (IN == IN_LOGITS_F16) {
        if constexpr (MODE != M_DECODE) {
            if (async_stage) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            else pad = stage_row(reinterpret_cast<const kr_half*>(rowp), V, stage, tid);
        }
        if constexpr (MODE == M_DECODE) {
            if (tid == 0) {   // parked in LDS until the symbol is known
                sh.dstate = dst;
                sh.win = win;
                sh.target = kr_rc_target(dst.low, dst.high, dst.pending_or_value, prec);
                sh.hit_leaf = -1;
            }
        }
        __syncthreads();
    }

    // ---- gather the row into registers, leaf layout; slots that hold no
    // element get -inf (softmax input, and the argmax of probabilities) ----
    float v[kMaxIt][17];
    int start[kMaxIt], len[kMaxIt];
    // Slices past the row's leaves (a whole wave's, e.g. the last slice for
    // most waves at V = 50277) and tail slots of full leaves are skipped in
    // every phase: their slots would only carry zeros.
    bool act[kMaxIt], tail[kMaxIt];
    #pragma unroll
    for (int it = 0; it < kMaxIt; it++) {
        const int L = it * kLeavesPerIt + wave * 8 + grp;
        act[it] = it * kLeavesPerIt + wave * 8 < P.n_leaves;
        int2 lf = make_int2(0, 0);
        if (L < P.n_leaves) lf = P.leaves[L];
        start[it] = lf.x;
        len[it] = lf.y;
        const int nf = leaf_full(lf.y), rm = leaf_rem(lf.y);
        tail[it] = __ballot(j < rm) != 0;
        if constexpr (IN == IN_LOGITS_F16) {
            // A leaf inside one 128-element skew segment (every leaf of a
            // full 8192-element block) reads at one constant offset. Slots
            // past the leaf read other staged values (the stage has room
            // for them) that the select then discards.
            const int s0 = pad.at(lf.x) - lf.x;
            if (lf.y == 0 || pad.at(lf.x + lf.y - 1) - (lf.x + lf.y - 1) == s0) {
                const kr_half* sp = stage + lf.x + s0;
                if (lf.y == 128) {   // a full leaf: 16 slots of 8, no tail
                    #pragma unroll
                    for (int k = 0; k < 16; k++) v[it][k] = (float)sp[j + 8 * k];
                    v[it][16] = -INFINITY;
                    continue;
                }
                #pragma unroll
                for (int k = 0; k < 16; k++) {
                    const float x = (float)sp[j + 8 * k];
                    v[it][k] = k < nf ? x : -INFINITY;
                }
                const float x = (float)sp[8 * nf + j];
                v[it][16] = j < rm ? x : -INFINITY;
                continue;
            }
        }
        #pragma unroll
        for (int k = 0; k < 16; k++)
            v[it][k] = k < nf ? load_val<IN>(rowp, stage, pad, lf.x + j + 8 * k) : -INFINITY;
        v[it][16] = j < rm ? load_val<IN>(rowp, stage, pad, lf.x + 8 * nf + j) : -INFINITY;
    }

    // ---- row max (exact, order-free): of the logits, or of the probabilities ----
    float m = -INFINITY;
    #pragma unroll
    for (int it = 0; it < kMaxIt; it++)
        if (act[it]) {
            #pragma unroll
            for (int k = 0; k < 17; k++) m = fmaxf(m, v[it][k]);
        }
    m = wave_max(m);
    if (lane == 0) sh.redf[wave] = m;
    __syncthreads();
    // every wave has gathered: the stage is free for the next row
    if (IN == IN_LOGITS_F16 && async_stage && next_row >= 0)
        stage_row_async(reinterpret_cast<const kr_half*>(input) + (size_t)next_row * (size_t)ld, V,
                        stage_lds, lane, wave);
    m = sh.redf[0];
    #pragma unroll
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, sh.redf[w]);

    // qmax: the largest value the CDF stage divides; p = q / denom is
    // nondecreasing in q, so the largest p is qmax / denom.
    float inv_S = 1.0f, qmax;
    if constexpr (IN == IN_LOGITS_F16) {
        // ---- e = kexp(x - m); S = numpy-order sum; q = e * (1/S) ----
        #pragma unroll
        for (int it = 0; it < kMaxIt; it++)
            if (act[it]) {
                #pragma unroll
                for (int k = 0; k < 16; k++) v[it][k] = kr_kexp(__fsub_rn(v[it][k], m));
                v[it][16] = tail[it] ? kr_kexp(__fsub_rn(v[it][16], m)) : 0.0f;
            }
        const float S = row_sum_numpy(v, len, act, tail, P, sh, lane, wave);
        inv_S = 1.0f / S;
        #pragma unroll
        for (int it = 0; it < kMaxIt; it++)
            if (act[it]) {
                #pragma unroll
                for (int k = 0; k < 16; k++) v[it][k] = __fmul_rn(v[it][k], inv_S);
                if (tail[it]) v[it][16] = __fmul_rn(v[it][16], inv_S);
            }
        // every e <= kexp(0) = 1, reached at the maximum logit
        qmax = inv_S;
    } else {
        qmax = m;
        #pragma unroll
        for (int it = 0; it < kMaxIt; it++)
            if (act[it]) {
                #pragma unroll
                for (int k = 0; k < 17; k++) if (v[it][k] == -INFINITY) v[it][k] = 0.0f;
            }
    }

    if constexpr (MODE == M_PROBS) {
        float* o = reinterpret_cast<float*>(out) + (size_t)row * (size_t)out_ld;
        #pragma unroll
        for (int it = 0; it < kMaxIt; it++) {
            const int nf = leaf_full(len[it]), rm = leaf_rem(len[it]);
            #pragma unroll
            for (int k = 0; k < 16; k++)
                if (k < nf) o[start[it] + j + 8 * k] = v[it][k];
            if (j < rm) o[start[it] + 8 * nf + j] = v[it][16];
        }
        return;
    }

    // ---- cdf.py: p = q / max(sum(q), 1e-30) ----
    const float P_sum = row_sum_numpy(v, len, act, tail, P, sh, lane, wave);
    const float denom = fmaxf(P_sum, 1e-30f);
    const float rdenom = 1.0f / denom;
    const float scale = (float)((1 << prec) - V);
    const float pmax = div_by(qmax, denom, rdenom);

    // ---- c = floor(p * scale) + 1 per element. Per leaf slice a lane keeps
    // the sum of floor(p * scale) over its slots (an empty slot holds q = 0,
    // so it adds 0) and adds its element count afterwards. The first maximum
    // of p is the lowest index with p == pmax: slots are visited from the
    // highest index down and the last hit is kept. With logits pmax > 0, so
    // an empty slot (p = 0) never hits; probabilities check occupancy. ----
    int lsum[kMaxIt];
    int bslot = -1;                       // 32 * it + k of the first maximum held
    int32_t* orow = nullptr;
    if constexpr (MODE == M_CDF || MODE == M_COUNTS)
        orow = reinterpret_cast<int32_t*>(out) + (size_t)row * (size_t)out_ld;
    // A lane only notes, per register slice, whether any of its slots holds
    // p == pmax (one compare per element, the flags kept as lane masks); the
    // lanes that do (a few per row) find their lowest such slot afterwards,
    // in the lowest flagged slice only.
    bool any_hit[kMaxIt];
    auto is_hit = [&](int it, int k, float p) {
        bool hit = p == pmax;
        if constexpr (IN == IN_PROBS_F32) {
            const int nf = leaf_full(len[it]), rm = leaf_rem(len[it]);
            hit = hit && (k < 16 ? (k < nf) : (j < rm));
        }
        return hit;
    };
    #pragma unroll
    for (int it = kMaxIt - 1; it >= 0; it--) {
        const int nf = leaf_full(len[it]), rm = leaf_rem(len[it]);
        int ls = 0;
        lsum[it] = 0;
        any_hit[it] = false;
        if (!act[it]) continue;
        #pragma unroll
        for (int k = 16; k >= 0; k--) {
            if (k == 16 && !tail[it]) continue;   // no lane holds a tail element
            const float p = div_by(v[it][k], denom, rdenom);
            const int f = scaled_floor<IN>(p, scale);
            ls += f;
            if constexpr (MODE == M_CDF || MODE == M_COUNTS) {
                const bool live = k < 16 ? (k < nf) : (j < rm);
                if (live) orow[slot_index(start[it], len[it], j, k) + 1] = f + 1;
            }
            any_hit[it] = any_hit[it] || is_hit(it, k, p);
        }
        lsum[it] = ls + nf + (j < rm ? 1 : 0);
    }
    // a lane's lowest indices are in its lowest slice: the first flagged
    // slice holds its first maximum; slots from the highest index down, the
    // last hit kept
    #pragma unroll
    for (int it = 0; it < kMaxIt; it++) {
        const bool first = any_hit[it] && bslot < 0;
        if (first) {
            #pragma unroll
            for (int k = 16; k >= 0; k--) {
                if (k == 16 && !tail[it]) continue;
                if (is_hit(it, k, div_by(v[it][k], denom, rdenom))) bslot = 32 * it + k;
            }
        }
    }
    int key = 0x7fffffff;                 // (index << 9) | leaf of that maximum
    if (bslot >= 0) {
        const int bi = bslot >> 5, bk = bslot & 31;
        int st = start[0], ln = len[0];
        #pragma unroll
        for (int it = 1; it < kMaxIt; it++)
            if (bi == it) { st = start[it]; ln = len[it]; }
        key = (slot_index(st, ln, j, bk) << 9) | (bi * kLeavesPerIt + wave * 8 + grp);
    }

    int csum = 0, cpre = 0, csym = 0;
    int sym = -1;
    if constexpr (MODE == M_PAIRS) sym = symbols[row];
    #pragma unroll
    for (int it = 0; it < kMaxIt; it++) {
        csum += lsum[it];
        if constexpr (MODE == M_PAIRS) {
            if (start[it] + len[it] <= sym) {
                cpre += lsum[it];
            } else if (start[it] <= sym) {   // the leaf that holds the symbol
                const int nf = leaf_full(len[it]), rm = leaf_rem(len[it]);
                #pragma unroll
                for (int k = 0; k < 17; k++) {
                    const bool live = k < 16 ? (k < nf) : (j < rm);
                    const int idx = slot_index(start[it], len[it], j, k);
                    const int c = scaled_floor<IN>(div_by(v[it][k], denom, rdenom), scale) + 1;
                    if (live && idx < sym) cpre += c;
                    if (live && idx == sym) csym = c;
                }
            }
        }
        if constexpr (MODE == M_DECODE) {
            int lc = lsum[it];
            lc += kr_xor<1>(lc);
            lc += kr_xor<2>(lc);
            lc += kr_xor<4>(lc);
            const int L = it * kLeavesPerIt + wave * 8 + grp;
            if (j == 0 && L < P.n_leaves) sh.leaf_count[L] = lc;
        }
    }

    // ---- argmax (lowest key) and integer sums across the workgroup ----
    key = kr_wave_reduce(key, [](int a, int b) { return a < b ? a : b; });
    csum = wave_isum(csum);
    if constexpr (MODE == M_PAIRS) {
        cpre = wave_isum(cpre);
        csym = wave_isum(csym);
    }
    if (lane == 0) {
        sh.redi[wave] = key;
        sh.redi2[wave] = csum;
        if constexpr (MODE == M_PAIRS) sh.redi3[wave] = cpre;
        if constexpr (MODE == M_PAIRS) sh.redL[wave] = csym;
    }
    __syncthreads();
    if (tid == 0) {
        int gk = sh.redi[0], gs = sh.redi2[0];
        for (int w = 1; w < kWaves; w++) {
            gk = min(gk, sh.redi[w]);
            gs += sh.redi2[w];
        }
        // A row with no maximum (NaN input) has no argmax; bin 0 then takes
        // the deficit so every index stays in bounds.
        int gi = gk >> 9, gL = gk & 511;
        if (gk == 0x7fffffff || gi >= V) { gi = 0; gL = 0; }
        const int deficit = (1 << prec) - gs;
        sh.amax = gi;
        sh.deficit = deficit;
        sh.amax_leaf = gL;
        if constexpr (MODE == M_CDF || MODE == M_COUNTS) {
            orow[gi + 1] += deficit;
            orow[0] = 0;
        }
        if constexpr (MODE == M_PAIRS) {
            int pre = 0, cs = 0;
            for (int w = 0; w < kWaves; w++) { pre += sh.redi3[w]; cs += sh.redL[w]; }
            const uint32_t lo = (uint32_t)(pre + (gi < sym ? deficit : 0));
            const uint32_t wdt = (uint32_t)(cs + (gi == sym ? deficit : 0));
            reinterpret_cast<uint2*>(out)[row] = make_uint2(lo, lo + wdt);
        }
        if constexpr (MODE == M_DECODE) sh.leaf_count[gL] += deficit;
    }
    if constexpr (MODE == M_PAIRS || MODE == M_COUNTS) return;

    if constexpr (MODE == M_CDF) {
        // Inclusive scan of counts over contiguous per-thread segments.
        __syncthreads();
        const int seg = (V + kThreads - 1) / kThreads;
        const int i0 = min(V, tid * seg), i1 = min(V, i0 + seg);
        int local = 0;
        for (int i = i0; i < i1; i++) local += orow[i + 1];
        int incl = local;
        for (int o = 1; o < 64; o <<= 1) {
            const int up = __shfl_up(incl, o);
            if (lane >= o) incl += up;
        }
        if (lane == 63) sh.redi[wave] = incl;
        __syncthreads();
        int base = incl - local;
        for (int w = 0; w < wave; w++) base += sh.redi[w];
        for (int i = i0; i < i1; i++) {
            base += orow[i + 1];
            orow[i + 1] = base;
        }
        return;
    }

    if constexpr (MODE == M_DECODE) {
        __syncthreads();
        const uint32_t target = sh.target;
        if (wave == 0) {
            // exclusive scan over leaf totals; 8 consecutive leaves per lane
            int loc[8];
            int s = 0;
            #pragma unroll
            for (int q = 0; q < 8; q++) {
                const int L = lane * 8 + q;
                loc[q] = L < P.n_leaves ? sh.leaf_count[L] : 0;
                s += loc[q];
            }
            int incl = s;
            for (int o = 1; o < 64; o <<= 1) {
                const int up = __shfl_up(incl, o);
                if (lane >= o) incl += up;
            }
            uint32_t run = (uint32_t)(incl - s);
            #pragma unroll
            for (int q = 0; q < 8; q++) {
                const int L = lane * 8 + q;
                if (L < P.n_leaves && run <= target && target < run + (uint32_t)loc[q]) {
                    sh.hit_leaf = L;
                    sh.hit_prefix = run;
                }
                run += (uint32_t)loc[q];
            }
        }
        __syncthreads();
        const int Lstar = sh.hit_leaf;
        const int gi = sh.amax, deficit = sh.deficit;
        // The owning lanes recompute the hit leaf's counts from the q values
        // they hold (same operations, same bits) instead of keeping every count.
        #pragma unroll
        for (int it = 0; it < kMaxIt; it++) {
            const int L = it * kLeavesPerIt + wave * 8 + grp;
            if (L == Lstar) {
                const int nf = leaf_full(len[it]), rm = leaf_rem(len[it]);
                #pragma unroll
                for (int k = 0; k < 17; k++) {
                    const bool live = k < 16 ? (k < nf) : (j < rm);
                    const int off = k < 16 ? j + 8 * k : 8 * nf + j;
                    if (live) {
                        const float p = div_by(v[it][k], denom, rdenom);
                        const int c = scaled_floor<IN>(p, scale) + 1;
                        sh.leaf_buf[off] = c + (start[it] + off == gi ? deficit : 0);
                    }
                }
                if (j == 0) { sh.hit_start = start[it]; sh.hit_len = len[it]; }
            }
        }
        __syncthreads();
        if (D.em && wave >= 4) {
            // layer 0's K, V, R and output projection weights into this XCD's
            // L2 (workgroup row runs on XCD row % 8) while wave 0 searches
            // and mixes: 3 staging blocks of 4 waves per row
            const int k = (row >> 3) * 3 + ((wave - 4) >> 2);
            if (k < (D.em->pf.blocks >> 3)) prefetch_panels(D.em->pf, 8 * k + (row & 7), tid & 255);
        }
        if (wave == 0) {
            // Symbol search inside the hit leaf (<= 128 counts): two counts
            // per lane, an inclusive scan, and the first lane whose range
            // holds the target. A valid CDF always contains the target; the
            // guard keeps a corrupt stream from reading unset LDS.
            const bool hit = Lstar >= 0;
            const int s0 = hit ? sh.hit_start : V - 1, n = hit ? sh.hit_len : 0;
            const uint32_t base_run = hit ? sh.hit_prefix : (1u << prec) - 1u;
            const uint32_t c0 = 2 * lane < n ? (uint32_t)sh.leaf_buf[2 * lane] : 0u;
            const uint32_t c1 = 2 * lane + 1 < n ? (uint32_t)sh.leaf_buf[2 * lane + 1] : 0u;
            uint32_t incl = c0 + c1;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t up = __shfl_up(incl, o);
                if (lane >= o) incl += up;
            }
            const uint32_t run0 = base_run + incl - (c0 + c1);   // before this lane's pair
            const bool h0 = 2 * lane < n && target < run0 + c0;
            const bool h1 = 2 * lane + 1 < n && !h0 && target < run0 + c0 + c1;
            const unsigned long long ball = __ballot(h0 || h1);
            const int src_lane = ball ? __ffsll(ball) - 1 : 0;
            const int s_l = h0 ? s0 + 2 * lane : s0 + 2 * lane + 1;
            const uint32_t lo_l = h0 ? run0 : run0 + c0;
            const uint32_t hi_l = h0 ? run0 + c0 : run0 + c0 + c1;
            int s = __shfl(s_l, src_lane);
            uint32_t clo = __shfl(lo_l, src_lane), chi = __shfl(hi_l, src_lane);
            if (!ball) {   // no hit: the last symbol of the leaf, or V-1 with [2^p-1, 2^p)
                s = hit ? s0 + n - 1 : V - 1;
                clo = base_run;
                chi = hit ? base_run : (1u << prec);
            }
            if (lane == 0) {
                kr_rc_state st = sh.dstate;
                kr_bit_window wnd = sh.win;
                kr_rc_consume(st.low, st.high, st.pending_or_value, clo, chi, prec, wnd);
                st.bit_offset = wnd.pos;
                D.states[row] = st;
                D.out_syms[row] = s;
                if (D.tokens) {
                    const int cnt = D.tok_count ? D.tok_count[row] : 0;
                    if (cnt >= 0 && cnt < D.tok_stride)
                        D.tokens[(size_t)row * (size_t)D.tok_stride + cnt] = s;
                    if (D.tok_count) D.tok_count[row] = cnt + 1;
                }
            }
            if (D.em) embed_mix(*D.em, (size_t)row, s, lane);   // s is wave-uniform
        }
    }
}

template <int IN, int MODE>
__global__ void __launch_bounds__(kThreads)
row_cdf_kernel(const void* __restrict__ input, long long ld, int n_rows, PlanArgs P, int prec,
               void* __restrict__ out, long long out_ld, const int32_t* __restrict__ symbols,
               DecodeArgs D, int async_stage) {
    __shared__ RowShared sh;
    __shared__ __attribute__((aligned(16))) kr_half stage[IN == IN_LOGITS_F16 ? kStageMax : 8];
    const int tid = threadIdx.x;
    if constexpr (MODE != M_DECODE) copy_plan(P, sh, tid);   // decode copies it after its first loads
    const unsigned stage_lds = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)stage;
    if constexpr (MODE == M_PAIRS && IN == IN_LOGITS_F16) {
        const int G = (int)gridDim.x;
        int row = (int)blockIdx.x;
        if (async_stage && row < n_rows)
            stage_row_async(reinterpret_cast<const kr_half*>(input) + (size_t)row * (size_t)ld, P.V,
                            stage_lds, tid & 63, tid >> 6);
        for (; row < n_rows; row += G)
            cdf_row<IN, MODE>(input, ld, row, row + G < n_rows ? row + G : -1, P, prec, out, out_ld,
                              symbols, D, sh, stage, stage_lds, async_stage != 0);
    } else {
        cdf_row<IN, MODE>(input, ld, (int)blockIdx.x, -1, P, prec, out, out_ld, symbols, D, sh,
                          stage, stage_lds, false);
    }
}

// ---------------------------------------------------------------------------
// Host: summation plans per (device, V)
// ---------------------------------------------------------------------------
struct DevPlan {
    PlanArgs args;
    void* mem;
};

std::mutex g_plan_mu;
std::map<std::pair<int, int>, DevPlan> g_plans;

struct BuildNode { bool leaf; int id; };

// The plan of numpy's pairwise summation of a row of V elements: leaves
// (start, len) in index order, inner nodes (left, right) grouped by level,
// the root of each 8192-element block, and for each (register slice, wave)
// the node whose 8-leaf subtree that wave sums in registers (-1: none).
// Node ids: leaves 0..NL-1, then the LDS-summed inner nodes in level order,
// then the wave-summed subtree roots. Returns the number of levels.
int build_plan(int V, std::vector<int2>& leaves, std::vector<int2>& inner_out,
               std::vector<int>& level_start, std::vector<int>& roots, std::vector<int>& wave_root) {
    struct Inner { BuildNode l, r; };
    std::vector<Inner> inner;
    // recursive split, numpy pairwise rule
    struct Rec {
        std::vector<int2>& leaves;
        std::vector<Inner>& inner;
        BuildNode go(int start, int n) {
            if (n <= 128) {
                leaves.push_back(make_int2(start, n));
                return BuildNode{true, (int)leaves.size() - 1};
            }
            int half = n / 2;
            half -= half % 8;
            const BuildNode l = go(start, half);
            const BuildNode r = go(start + half, n - half);
            inner.push_back(Inner{l, r});
            return BuildNode{false, (int)inner.size() - 1};
        }
    } rec{leaves, inner};
    std::vector<BuildNode> block_roots;
    for (int s = 0; s < V; s += 8192) block_roots.push_back(rec.go(s, std::min(8192, V - s)));
    const int NL = (int)leaves.size(), NI = (int)inner.size();
    auto key = [](BuildNode n) { return n.leaf ? (long long)n.id : -(long long)n.id - 1; };
    std::map<std::pair<long long, long long>, int> by_children;
    for (int i = 0; i < NI; i++) by_children[{key(inner[i].l), key(inner[i].r)}] = i;
    auto find = [&](BuildNode a, BuildNode b) -> int {
        auto f = by_children.find({key(a), key(b)});
        return f == by_children.end() ? -1 : f->second;
    };
    // 0: summed in LDS, 1: inside a wave subtree, 2: root of a wave subtree
    std::vector<int> kind(NI, 0);
    std::vector<int> wave_node(kMaxIt * kWaves, -1);
    for (int it = 0; it < kMaxIt; it++)
        for (int w = 0; w < kWaves; w++) {
            const int L0 = it * kLeavesPerIt + w * 8;
            if (L0 + 7 >= NL) continue;
            int lvl[4], cnt = 4;
            bool ok = true;
            std::vector<int> internal;
            for (int k = 0; k < 4 && ok; k++)
                ok = (lvl[k] = find(BuildNode{true, L0 + 2 * k}, BuildNode{true, L0 + 2 * k + 1})) >= 0;
            while (ok && cnt > 1) {
                for (int k = 0; k < cnt / 2 && ok; k++) {
                    internal.push_back(lvl[2 * k]);
                    internal.push_back(lvl[2 * k + 1]);
                    ok = (lvl[k] = find(BuildNode{false, lvl[2 * k]}, BuildNode{false, lvl[2 * k + 1]})) >= 0;
                }
                cnt /= 2;
            }
            if (!ok) continue;   // only a complete subtree of 8 leaves counts
            for (int n : internal) kind[n] = 1;
            kind[lvl[0]] = 2;
            wave_node[it * kWaves + w] = lvl[0];
        }
    // levels of the LDS-summed nodes (leaves and wave roots are level 0)
    std::vector<int> level(NI, -1);
    std::function<int(BuildNode)> lev_of = [&](BuildNode n) -> int {
        if (n.leaf || kind[n.id] == 2) return 0;
        if (level[n.id] >= 0) return level[n.id];
        return level[n.id] = 1 + std::max(lev_of(inner[n.id].l), lev_of(inner[n.id].r));
    };
    std::vector<int> order;
    for (int i = 0; i < NI; i++)
        if (kind[i] == 0) { lev_of(BuildNode{false, i}); order.push_back(i); }
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return level[a] < level[b]; });
    std::vector<int> id(NI, -1);
    for (int i = 0; i < (int)order.size(); i++) id[order[i]] = NL + i;
    int next = NL + (int)order.size();
    for (int i = 0; i < NI; i++) if (kind[i] == 2) id[i] = next++;
    auto ident = [&](BuildNode n) { return n.leaf ? n.id : id[n.id]; };
    inner_out.resize(order.size());
    int max_l = 0;
    for (int i = 0; i < (int)order.size(); i++) {
        inner_out[i] = make_int2(ident(inner[order[i]].l), ident(inner[order[i]].r));
        max_l = std::max(max_l, level[order[i]]);
    }
    level_start.assign(max_l + 1, 0);
    {
        int idx = 0;
        for (int h = 1; h <= max_l; h++) {
            level_start[h - 1] = idx;
            while (idx < (int)order.size() && level[order[idx]] == h) idx++;
        }
        level_start[max_l] = idx;
    }
    for (auto& r : block_roots) roots.push_back(ident(r));
    wave_root.assign(kMaxIt * kWaves, -1);
    for (int x = 0; x < kMaxIt * kWaves; x++)
        if (wave_node[x] >= 0) wave_root[x] = id[wave_node[x]];
    return max_l;
}

int get_plan(int V, PlanArgs* out) {
    int dev = 0;
    KR_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_plan_mu);
    auto it = g_plans.find({dev, V});
    if (it != g_plans.end()) { *out = it->second.args; return KR_OK; }
    std::vector<int2> leaves, inner;
    std::vector<int> level_start, roots, wave_root;
    const int n_levels = build_plan(V, leaves, inner, level_start, roots, wave_root);
    if ((int)leaves.size() > kMaxLeaves || n_levels > kMaxLevels || (int)roots.size() > kMaxBlocks)
        return kr_fail(KR_EUNSUPPORTED,
                       "vocabulary %d needs %d summation leaves, %d levels (max %d, %d)", V,
                       (int)leaves.size(), n_levels, kMaxLeaves, kMaxLevels);
    const size_t nb = sizeof(int2) * (leaves.size() + inner.size()) +
                      sizeof(int) * (level_start.size() + roots.size() + wave_root.size());
    std::vector<char> host(nb);
    char* p = host.data();
    auto put = [&](const void* src, size_t bytes) { std::memcpy(p, src, bytes); p += bytes; };
    put(leaves.data(), sizeof(int2) * leaves.size());
    put(inner.data(), sizeof(int2) * inner.size());
    put(level_start.data(), sizeof(int) * level_start.size());
    put(roots.data(), sizeof(int) * roots.size());
    put(wave_root.data(), sizeof(int) * wave_root.size());
    void* mem = nullptr;
    KR_HIP(hipMalloc(&mem, nb));
    KR_HIP(hipMemcpy(mem, host.data(), nb, hipMemcpyHostToDevice));
    char* d = static_cast<char*>(mem);
    PlanArgs a;
    a.leaves = reinterpret_cast<const int2*>(d);
    d += sizeof(int2) * leaves.size();
    a.inner = reinterpret_cast<const int2*>(d);
    d += sizeof(int2) * inner.size();
    a.level_start = reinterpret_cast<const int*>(d);
    d += sizeof(int) * level_start.size();
    a.roots = reinterpret_cast<const int*>(d);
    d += sizeof(int) * roots.size();
    a.wave_root = reinterpret_cast<const int*>(d);
    a.V = V;
    a.n_leaves = (int)leaves.size();
    a.n_inner = (int)inner.size();
    a.n_levels = n_levels;
    a.n_blocks = (int)roots.size();
    g_plans[{dev, V}] = DevPlan{a, mem};
    *out = a;
    return KR_OK;
}

int check_common(int N, int V, int prec) {
    KR_REQUIRE(N >= 0, "bad row count %d", N);
    KR_REQUIRE(V >= 1 && V <= 65536, "vocabulary %d out of range [1, 65536]", V);
    KR_REQUIRE(prec >= 1 && prec <= 30 && V < (1 << prec), "cdf_precision %d invalid for V=%d",
               prec, V);
    return KR_OK;
}

template <int IN, int MODE>
int launch_rows(const void* in, long long ld, int N, int V, int prec, void* out,
                long long out_ld, const int32_t* symbols, const DecodeArgs& D, void* stream) {
    int rc = check_common(N, V, prec);
    if (rc) return rc;
    if (N == 0) return KR_OK;
    PlanArgs P;
    rc = get_plan(V, &P);
    if (rc) return rc;
    // Pairs (many rows): one persistent workgroup per CU (the stage fills
    // most of a CU's LDS), each copying its next row in while it computes
    // the current one. That needs rows whose 16-byte chunks all lie inside
    // the allocation: 16-byte-aligned rows and a stride that is a multiple of 8.
    int grid = N, async = 0;
    if (MODE == M_PAIRS && IN == IN_LOGITS_F16 && ((uintptr_t)in & 15) == 0 && ld % 8 == 0) {
        int dev = 0, cus = 0;
        KR_HIP(hipGetDevice(&dev));
        KR_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        grid = std::min(N, std::max(cus, 1));
        async = 1;
    }
    row_cdf_kernel<IN, MODE><<<grid, kThreads, 0, kr_stream(stream)>>>(in, ld, N, P, prec, out,
                                                                        out_ld, symbols, D, async);
    KR_LAUNCHED();
    return KR_OK;
}

}  // namespace

// kr_softmax_cdf_decode, plus (em non-null) layer 0's LN1-mix of each decoded
// token; em is a device copy of a kr_embed_mix (kr_model.h) that
// kr_impl_embed_mix_args filled.
int kr_impl_cdf_decode(const uint16_t* logits, int B, int V, long long ld,
                       const uint8_t* input_buf, uint32_t in_len,
                       const int32_t* base_byte_offsets, const int32_t* byte_limits,
                       uint32_t* states, int32_t* out_syms, int32_t* tokens,
                       long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                       int cdf_precision, const kr_embed_mix* em, void* stream) {
    KR_REQUIRE(logits && input_buf && states && out_syms, "kr_softmax_cdf_decode: null pointer");
    KR_REQUIRE(ld >= V, "kr_softmax_cdf_decode: ld %lld < V %d", ld, V);
    KR_REQUIRE(!tokens || tok_stride >= 1, "kr_softmax_cdf_decode: bad tok_stride");
    DecodeArgs D;
    D.in = input_buf;
    D.in_len = in_len;
    D.base = base_byte_offsets;
    D.limits = byte_limits;
    D.states = reinterpret_cast<kr_rc_state*>(states);
    D.out_syms = out_syms;
    D.tokens = tokens;
    D.tok_stride = tok_stride;
    D.tok_count = tok_count;
    D.n_tokens = n_tokens;
    D.em = em;
    return launch_rows<IN_LOGITS_F16, M_DECODE>(logits, ld, B, V, cdf_precision, nullptr, 0,
                                                nullptr, D, stream);
}

extern "C" {

int kr_probs_to_cdf(const float* probs, int N, int V, long long ld, uint32_t* cdf_out,
                    int cdf_precision, void* stream) {
    KR_REQUIRE(probs && cdf_out, "kr_probs_to_cdf: null pointer");
    KR_REQUIRE(ld >= V, "kr_probs_to_cdf: ld %lld < V %d", ld, V);
    return launch_rows<IN_PROBS_F32, M_CDF>(probs, ld, N, V, cdf_precision, cdf_out, V + 1,
                                            nullptr, DecodeArgs{}, stream);
}

int kr_softmax_cdf(const uint16_t* logits, int N, int V, long long ld, int32_t* out,
                   int cumulative, int cdf_precision, void* stream) {
    KR_REQUIRE(logits && out, "kr_softmax_cdf: null pointer");
    KR_REQUIRE(ld >= V, "kr_softmax_cdf: ld %lld < V %d", ld, V);
    if (cumulative)
        return launch_rows<IN_LOGITS_F16, M_CDF>(logits, ld, N, V, cdf_precision, out, V + 1,
                                                 nullptr, DecodeArgs{}, stream);
    return launch_rows<IN_LOGITS_F16, M_COUNTS>(logits, ld, N, V, cdf_precision, out, V + 1,
                                                nullptr, DecodeArgs{}, stream);
}

int kr_softmax_probs(const uint16_t* logits, int N, int V, long long ld, float* probs,
                     void* stream) {
    KR_REQUIRE(logits && probs, "kr_softmax_probs: null pointer");
    KR_REQUIRE(ld >= V, "kr_softmax_probs: ld %lld < V %d", ld, V);
    return launch_rows<IN_LOGITS_F16, M_PROBS>(logits, ld, N, V, KR_CDF_PRECISION_DEFAULT, probs,
                                               V, nullptr, DecodeArgs{}, stream);
}

int kr_softmax_cdf_pairs(const uint16_t* logits, int N, int V, long long ld,
                         const int32_t* symbols, uint32_t* pairs, int cdf_precision,
                         void* stream) {
    KR_REQUIRE(logits && symbols && pairs, "kr_softmax_cdf_pairs: null pointer");
    KR_REQUIRE(ld >= V, "kr_softmax_cdf_pairs: ld %lld < V %d", ld, V);
    return launch_rows<IN_LOGITS_F16, M_PAIRS>(logits, ld, N, V, cdf_precision, pairs, 2,
                                               symbols, DecodeArgs{}, stream);
}

int kr_softmax_cdf_decode(const uint16_t* logits, int B, int V, long long ld,
                          const uint8_t* input_buf, uint32_t in_len,
                          const int32_t* base_byte_offsets, const int32_t* byte_limits,
                          uint32_t* states, int32_t* out_syms, int32_t* tokens,
                          long long tok_stride, int32_t* tok_count, const int32_t* n_tokens,
                          int cdf_precision, void* stream) {
    return kr_impl_cdf_decode(logits, B, V, ld, input_buf, in_len, base_byte_offsets, byte_limits,
                              states, out_syms, tokens, tok_stride, tok_count, n_tokens,
                              cdf_precision, nullptr, stream);
}

}  // extern "C"
