// Device-side plan of the persistent decode-step kernel (decode_persistent.hip),
// built on the host by the C ABI (capi.hip) from vte_decode_model and the
// workspace layout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vte_amd.h"

#define VTE_DECODE_MAX_SPLITS 128  // attention splits per KV head

typedef vte_decode_layer VtePdLayer;

struct VtePdPlan {
    const VtePdLayer* layers;  // device copy in the workspace
    int n_layers, hidden, ffn, n_q, n_kv, vocab;
    float eps, scale;
    const int* kv_offset;
    const __half* x;           // the token's embedding (layer 0 input, plain fp16)
    const __half* rope_cos;
    const __half* rope_sin;
    const void* output_norm;
    const void* lm_head;
    int fmt_lm;
    float* logits;
    // flagged words (fp16 | tag << 16): layer output, q, new K/V row, attention
    // output, post-attention hidden, SwiGLU output
    uint32_t *ll_h, *ll_q, *ll_kv, *ll_att, *ll_hm, *ll_act;
    uint64_t* part;            // attention records (fp32 | tag << 32) [n_q][MAX_SPLITS][130]
    uint32_t* ctrl;            // [0] epoch, [1] finished blocks, [2] error flags
    int r_qk, r_v, r_o, r_gu, r_d, r_lm;  // rows per tile of each stage
    int split_min;             // smallest attention split (rows)
    unsigned long long timeout_ticks;     // per-block wait deadline (100 MHz clock)
};

namespace vte {
size_t decode_persistent_lds(int hidden, int ffn, int q_dim);
hipError_t decode_persistent_launch(const VtePdPlan& P, int blocks, size_t lds, hipStream_t st);
int decode_persistent_occupancy(const VtePdPlan& P, size_t lds);
}  // namespace vte
