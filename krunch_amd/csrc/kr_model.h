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
