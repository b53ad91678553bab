// Device-side plan of the persistent decode-step kernel (decode_persistent.hip),
// built on the host by the C ABI (capi.hip) from vte_decode_model and the
// workspace layout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vte_amd.h"

#define VTE_DECODE_MAX_SPLITS 128  // attention splits per KV head
#define VTE_PD_UPT_GU 8            // weight units per thread of a gate/up tile
#define VTE_PD_UPT_QKV 2           // weight units per thread of a q/k/v tile
#define VTE_PB_MAX_B 16            // sequences of the batched persistent step (one MFMA column tile)
#define VTE_PB_MAX_K 1536          // longest activation row the batched step stages per block
#define VTE_PB_MAX_SLICES 16       // down-projection slices of the batched step

typedef vte_decode_layer VtePdLayer;

struct VtePdPlan {
    const VtePdLayer* layers;  // device copy in the workspace
    int n_layers, hidden, ffn, n_q, n_kv;
    float eps, scale;
    const int* kv_offset;
    int max_seq;               // rows of the K/V caches and RoPE tables: kv_offset[0] must lie in [0, max_seq)
    const __half* x;           // the token's embedding (layer 0 input, plain fp16)
    const __half* rope_cos;
    const __half* rope_sin;
    __half* h_out;             // the last layer's output (plain fp16 [hidden], read by the LM head launch)
    // flagged words (fp16 | tag << 16): layer output, q, new K/V row, attention
    // output, post-attention hidden, SwiGLU output
    uint32_t *ll_h, *ll_q, *ll_kv, *ll_att, *ll_hm, *ll_act;
    uint64_t* part;            // attention records (fp32 | tag << 32) [n_q][MAX_SPLITS][130]
    uint64_t* ll_dn;           // down partial sums (fp32 | tag << 32) [ffn / 256][hidden]
    uint32_t* ctrl;            // [0] epoch, [1] finished blocks, [2] error flags (1: a wait timed out, 2: position out of range)
    int r_qk, r_v, r_o, r_gu;  // rows per tile of the q/k, v, o-proj and gate/up stages
    int r_dn;                  // rows per down-partial tile (one 256-wide slice of the ffn activations)
    int r_red;                 // rows each block reduces over the down partials
    int split_min;             // smallest attention split (rows)
    unsigned long long timeout_ticks;     // per-block wait deadline (100 MHz clock)
};

// Device-side plan of the batched persistent step (decode_persistent_mm.hip):
// B <= 16 sequences, every activation buffer [B][...] (sequence-major).
struct VtePbPlan {
    const VtePdLayer* layers;
    int n_layers, hidden, ffn, n_q, n_kv, B;
    float eps, scale;
    const int* kv_offset;      // [B] positions, each in [0, max_seq)
    int max_seq;
    long long kv_batch_stride; // elements between two sequences' caches (layer.k_cache + m * stride)
    const __half* x;           // [B][hidden] embeddings (layer 0 input, plain fp16)
    const __half* rope_cos;
    const __half* rope_sin;
    __half* h_out;             // [B][hidden] the last layer's output (plain fp16)
    uint32_t *ll_h, *ll_q, *ll_kv, *ll_att, *ll_hm, *ll_act;  // flagged fp16 words, [B][...] each (ll_kv: [B][2 * kv_dim]; ll_act: [slice][B][slice width])
    uint64_t* part;            // attention records (fp32 | tag << 32) [B][n_q][MAX_SPLITS][130]
    uint64_t* ll_dn;           // down partial sums (fp32 | tag << 32) [slices][B][hidden]
    uint32_t* ctrl;            // as VtePdPlan::ctrl
    int sl_sb;                 // super-blocks of the ffn activations per down slice
    int split_min;
    uint32_t* trace;           // stage clocks [block][layer][8] (probe builds with VTE_PB_TRACE; else unused)
    unsigned long long timeout_ticks;
};

namespace vte {
size_t decode_persistent_lds(int hidden, int ffn, int q_dim);
hipError_t decode_persistent_launch(const VtePdPlan& P, int blocks, size_t lds, hipStream_t st);
int decode_persistent_occupancy(const VtePdPlan& P, size_t lds);
size_t decode_persistent_mm_lds(int hidden, int q_dim, int slice);
hipError_t decode_persistent_mm_launch(const VtePbPlan& P, int blocks, size_t lds, hipStream_t st);
int decode_persistent_mm_occupancy(size_t lds);
}  // namespace vte
