// Host-side descriptors of the RWKV-4 weights (public: include/krunch_hip.h)
// and the per-layer view of the recurrent state used by the layer driver.
#pragma once
#include "kr_common.h"
#include "krunch_hip.h"

// Recurrent state of B streams for one layer (device pointers, [B, C]).
struct kr_layer_state {
    void* att_xx;   // fp16
    float* aa;      // fp32
    float* bb;      // fp32
    float* pp;      // fp32
    void* ffn_xx;   // fp16
};

// Weight panels to pull into each XCD's L2 while a latency-bound kernel runs:
// region r holds n_groups column groups of group_bytes each (fragment-packed
// weights, one group per workgroup column group of the product that follows);
// the staging threads of XCD x read groups x, x + 8, ..., the ones that XCD's
// workgroups will multiply by.
struct PrefetchSet {
    const char* base[4];
    long long group_bytes[4];
    int n_groups[4];
    int n;                     // regions
    int blocks;                // staging blocks of 256 threads (a multiple of 8)
};

// Layer 0's LN1-mix of the token a decode step has just decoded, run by the
// decode kernel's workgroup of that stream (one wave), so the next step
// starts at layer 0's K, V, R products. Row b of the next step:
//   xw[b]  = emb[id]                                  (the residual stream)
//   xx     = LN1(emb[id]);  sx = src[b]               (the carried row)
//   out[m] = mix(xx, sx) with tm[m], fragment-packed  (K, V, R operands;
//            w8a8: q[m], qs[m], quantised per row)
//   state[b] = sx;  pend[b] = xx
// The carried row is committed one step late: after a step, state holds the
// row of the token that step consumed (what the layer's own LN1-mix would
// leave), and pend the row of the token just decoded, which the next step's
// decode kernel reads as src. The first step of a run reads src = state.
// The bits are those of ln_mix_kernel on the same row.
struct kr_embed_mix {
    const kr_half* emb;
    int V;
    int C;                     // 0: no layer-0 work in the decode kernel
    const kr_half* ln_w;
    const kr_half* ln_b;
    const kr_half* tm[3];
    kr_half* out[3];
    int8_t* q[3];              // w8a8 layer 0 (q[0] non-null): int8 mixes instead of out[]
    float* qs[3];              // and their row scales (kr_quantize_rows rule)
    const kr_half* src;        // [B, C]
    kr_half* state;            // [B, C] layer 0's att_xx
    kr_half* pend;             // [B, C]
    kr_half* xw;               // [B, C]
    PrefetchSet pf;            // layer 0's K, V, R and output projection weights (blocks 0: none)
};
