/*
 * libvte_amd.so — C ABI of the MI355X (gfx950) decode hot path.
 *
 * Plain pointers, sizes and a hipStream_t passed as void* (NULL = the null
 * stream).  Every device pointer is a device address the caller owns (e.g. a
 * slice of one slab allocation); no entry point allocates or frees device
 * memory, and every launch is asynchronous on `stream`.
 *
 * Return value: 0 on success, VTE_EINVAL (-1) when host-side validation
 * rejects an argument (nothing is launched), otherwise the hipError_t of the
 * failed launch.  vte_last_error() returns the message of the last failure.
 *
 * Codes:  dtype  VTE_F32 = 0, VTE_F16 = 1
 *         fmt    VTE_Q4_K = 4 (144 B / 256 elements), VTE_Q6_K = 6 (210 B / 256),
 *                VTE_Q8_0 = 8 (34 B / 32)
 * Weight matrices are raw GGUF super-block rows: row r of an N x K matrix
 * starts at byte r * (K / block_elems) * block_bytes.
 *
 * Each declaration names the reference interface it replaces
 * (kyuubyN/VTE, paths relative to the repository root).  The same kernels are
 * also exported under the reference's own kernel symbols from the code object
 * vte_kernels_gfx950.hsaco (hipModuleGetFunction drop-in): gemv_q4k_kernel,
 * gemv_q6k_kernel, gemv_q8_0_kernel, kv_cache_append_kernel,
 * flash_attention_split_kv_partial_kernel, flash_attention_split_kv_reduce_kernel,
 * rmsnorm_kernel, rope_kernel, swiglu_kernel, add_kernel,
 * embedding_lookup_q6k_kernel, embedding_lookup_q4k_kernel,
 * embedding_lookup_q8_0_kernel.  Beside them the code object holds the
 * fp32-I/O siblings gemv_q4k_f32_kernel, gemv_q6k_f32_kernel,
 * gemv_q8_0_f32_kernel (same 10 arguments and geometry, fp32 input, bias,
 * residual and output) and the batched MFMA GEMMs gemm_q4k_mfma_kernel,
 * gemm_q6k_mfma_kernel (the same 10 arguments, fp16 I/O; grid
 * (ceil(out_features/32), ceil(batch*seq_len/16)), block 512) that the
 * reference's dispatch can select from batch 8 (no reference counterpart:
 * its batched executor re-runs the GEMV per row, batched_hip_graph_executor.py:231-251).
 */
#ifndef VTE_AMD_H
#define VTE_AMD_H

#ifdef __cplusplus
extern "C" {
#endif

#define VTE_EINVAL (-1)
#define VTE_F32 0
#define VTE_F16 1
#define VTE_Q4_K 4
#define VTE_Q6_K 6
#define VTE_Q8_0 8

/* Message of the last failed call (thread-unsafe static buffer).
 * Replaces: HIPRuntimeError text, vte/bridge/hip_runtime.py:342-344. */
const char* vte_last_error(void);

/* ABI revision of this header (1). */
int vte_abi_version(void);

/* CU count, HBM bytes and gfx arch name of `device`.
 * Replaces: HIPRuntime.get_num_cus / get_gpu_architecture, vte/bridge/hip_runtime.py. */
int vte_device_info(int device, int* n_cu, long long* total_mem, char* arch, int arch_len);

/* y[m][n] = ((sum_k W[n][k] x[m][k]) + bias[n]) * residual_scale + residual[m][n]
 * for m < M (batch rows), fp32 accumulation.  x [M][K] in in_dtype, y [M][N]
 * in out_dtype; bias fp16/f32 [N] and residual [M][N] (out_dtype) nullable.
 * fmt Q4_K / Q6_K / Q8_0; K a multiple of 256 (Q8_0: 32).  M <= 4 runs the
 * persistent bandwidth kernel, larger M the wave-per-row kernel.
 * Replaces: gemv_q4k_kernel (vte/compiler/templates/rdna/gemv_q4k.hip.template:56-168),
 *           gemv_q6k_kernel (gemv_q6k.hip.template:25-104),
 *           gemv_q8_0_kernel (gemv_q8_0.hip.template:26-93),
 *           launch geometry vte/core/fallback_executor.py:140-148,
 *           arguments vte/core/kernel_arg_builder.py:327-386. */
int vte_gemv(int fmt, int in_dtype, int out_dtype, const void* x, const void* w, void* y, int M, int K, int N,
             const void* bias, const void* residual, float residual_scale, void* stream);

/* Same contract as vte_gemv, batched (M >= 8) on MFMA: super-blocks are
 * dequantised to fp16 in registers and multiplied with
 * mfma_f32_16x16x32_f16, fp32 accumulation.  Q4_K and Q6_K.
 * Replaces: the per-row GEMV launches with grid.y = batch of
 * vte/core/batched_hip_graph_executor.py:231-251 (the reference has no MFMA path). */
int vte_gemm_mfma(int fmt, int in_dtype, int out_dtype, const void* x, const void* w, void* y, int M, int K,
                  int N, const void* bias, const void* residual, float residual_scale, void* stream);

/* Split-K partial sums for batched projections (M >= 3; above 32 columns with
 * at most 8 super-blocks per split one weight-stationary launch, same
 * results), Q4_K / Q6_K, fp16 x:
 *   part[s][m][n] = sum over split s's super-blocks of dequant(W[n, k]) * x[m, k]
 * (fp32, no bias / scale / residual; 1 <= splits <= 8 and splits <= K / 256).
 * vte_add_rmsnorm adds the splits to the residual.
 * Replaces: split_k_qkv_pass1_kernel (split_k_qkv_pass1.hip.template:29-79), the
 *           reference's split-K pass writing per-split sums to a scratchpad. */
int vte_gemm_mfma_splitk(int fmt, const void* x, const void* w, float* part, int M, int K, int N, int splits,
                         void* stream);

/* Dequantise n_elements (a multiple of the block size) to fp32, bit-exact with
 * the reference's NumPy dequantiser.
 * Replaces: dequantize_q4_k / dequantize_q6_k / dequantize_q8_0
 *           (vte/compiler/dequantizer.py:26-70, 129-169, 172-196). */
int vte_dequantize(int fmt, const void* src, float* dst, long long n_elements, void* stream);

/* Floats of split-KV scratch (part_m + part_l + part_o) for a shape. */
long long vte_attn_scratch_floats(int batch, int n_q, int max_splits);

/* Split-KV flash decoding with log-sum-exp combine, ragged batches.
 * q [B][n_q][128] (dtype), caches fp16 [B][max_seq][n_kv][128] with
 * kv_batch_stride elements between sequences, out [B][n_q][128] (dtype).
 * Sequence b attends to positions 0..kv_offset[b] (device int array), split
 * tokens per partial block (multiple of 32), max_splits >= ceil(max_seq/split)
 * (at most 4096).  part_m/part_l [B][n_q][max_splits], part_o
 * [B][n_q][max_splits][128] fp32 scratch.  counters: NULL = separate combine
 * launch; else 1 + B*n_kv ints, zeroed before the first call and then owned
 * by the kernel: counters[0] is a sticky error word (nonzero once a combining
 * block gave up waiting on a split's records: that launch's outputs are
 * invalid), counters[1 + b*n_kv + kvh] the per-group epochs; the combine
 * then runs inside the partial kernel
 * (max_splits <= 512, split > 32): part_o then holds flagged records and must
 * hold B*n_q*max_splits*260 floats, zeroed before the first call.
 * out NULL (with counters NULL): only the partials are written, for
 * vte_attn_out_gemv to combine.  kv_batch_stride 0 with B > 1: every column
 * reads the same cache (prompt tokens of one sequence, each at its own
 * kv_offset); two columns then share each K/V tile load, same results.
 * Replaces: SplitKVAttentionDispatcher launches (vte/core/split_kv_attention.py:187-217),
 *           flash_attention_split_kv_partial_kernel (flash_attention_split_kv_partial.hip.template:31-120),
 *           flash_attention_split_kv_reduce_kernel (flash_attention_split_kv_reduce.hip.template:14-67). */
int vte_attn_split_kv(int dtype, const void* q, const void* k_cache, const void* v_cache, float* part_m,
                      float* part_l, float* part_o, void* out, int batch, int n_q, int n_kv, int head_dim,
                      float scale, const int* kv_offset, int kv_batch_stride, int split, int max_splits,
                      int* counters, void* stream);

/* k_cache[b][kv_offset[b]] = k[b], v_cache likewise (fp16 [B][n_kv][head_dim]).
 * Replaces: kv_cache_append_kernel (kv_cache_append.hip.template:13-39). */
int vte_kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int batch, int n_kv, int head_dim,
                  const int* kv_offset, int kv_batch_stride, void* stream);

/* out = fp16(x * rsqrt(mean(x^2) + eps) * w), rows x hidden, fp16.
 * Replaces: rmsnorm_kernel (rmsnorm.hip.template:6-117). */
int vte_rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps, void* stream);

/* x_out = fp16(x + sum_s part[s]) and xn = fp16(x_out * rsqrt(mean(x_out^2) + eps) * w)
 * for part [n_parts][rows][hidden] fp32 (1 <= n_parts <= 8), hidden % 8 == 0,
 * hidden <= 8192; x_out may equal x.
 * Replaces: add_kernel (add.hip.template:4-17) as the residual add of the
 *           projection, followed by rmsnorm_kernel (rmsnorm.hip.template:6-117);
 *           the split sum is split_k_qkv_pass2.hip.template:25-137's reduction. */
int vte_add_rmsnorm(const void* x, const float* part, int n_parts, const void* w, void* x_out, void* xn, int rows,
                    int hidden, float eps, void* stream);

/* In-place rotary embedding of q [B][seq][n_q][hd] and k [B][seq][n_kv][hd]
 * at positions kv_offset[b] + s, fp16 cos/sin caches [max_seq][hd].
 * rope_type 0 = NORM (adjacent pairs), 1 = NEOX (i, i + hd/2), 2 = partial
 * NEOX over rotary_dim.
 * Replaces: rope_kernel (rope.hip.template:17-137; NEOX at :82-97). */
int vte_rope(void* q, void* k, const void* cos_cache, const void* sin_cache, int batch, int seq_len, int n_q,
             int n_kv, int head_dim, const int* kv_offset, int rope_type, int rotary_dim, void* stream);

/* out = fp16(silu(gate) * up), n fp16 elements.
 * Replaces: swiglu_kernel (swiglu.hip.template:4-26). */
int vte_swiglu(const void* gate, const void* up, void* out, int n, void* stream);

/* out = fp16(residual + scale * input), n fp16 elements.
 * Replaces: add_kernel (add.hip.template:4-17). */
int vte_add(const void* residual, const void* input, void* out, int n, float scale, void* stream);

/* out[t] = fp16(dequant(table row tokens[t]) * scale), Q6_K table [vocab][hidden].
 * Replaces: embedding_lookup_q6k_kernel (embedding_lookup_q6k.hip.template:17-58). */
int vte_embedding_q6k(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                      void* stream);

/* The same from a Q4_K table [vocab][hidden] (hidden a multiple of 256; the
 * untied embedding of Qwen2.5-7B).
 * Replaces: embedding_lookup_q4k_kernel (embedding_lookup_q4k.hip.template:26-75). */
int vte_embedding_q4k(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                      void* stream);

/* The same from a Q8_0 table [vocab][hidden] (hidden a multiple of 32; tied
 * Q8_0 embeddings, scale 12 for Granite).
 * Replaces: embedding_lookup_q8_0_kernel (embedding_lookup_q8_0.hip.template:15-46). */
int vte_embedding_q8_0(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                       void* stream);

/* Bytes of device scratch (8-byte aligned) vte_topk needs for `rows` rows. */
long long vte_topk_scratch_bytes(int rows);

/* Per row of fp32 logits [rows][vocab] (vocab <= 262144): the k (1..64)
 * largest values in descending order, ties broken by the lower index, with
 * their indices.
 * Replaces: the argpartition top-k of Sampler.sample (vte/core/sampler.py:54-129)
 *           and topk_reduce_greedy_kernel (topk_reduce_greedy.hip.template:52-83). */
int vte_topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
             void* stream);

/* vte_topk without a workspace argument and without allocating: the
 * candidate buffer is a fixed device array inside the library (one per GPU,
 * 64 rows = 4.2 MB, held until the process ends).  rows must be <= 64 (else
 * -1 and a message).  Calls that overlap on one GPU race on that array.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). */
int vte_topk_noalloc(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* stream);

/* Greedy decoding on the device (temperature 0, no repetition penalty): for
 * each row b, tok = top_idx[b*k] (the top-1 candidate of vte_topk: the
 * largest logit, lowest id among equal ones), tokens[b] = tok, kv_offset[b] =
 * min(kv_offset[b] + 1, max_pos), history[*step][b] = tok while *step <
 * history_steps; then *step += 1.  Appended to a captured decode step, the
 * next replay decodes the next token with no host round trip.
 * Replaces: the greedy pick of topk_reduce_greedy_kernel
 *           (topk_reduce_greedy.hip.template:52-83) and the host loop that feeds
 *           the picked token back (vte/core/model.py:1039-1044 with
 *           Sampler.pick_greedy_from_gpu_candidates, vte/core/sampler.py:163-233). */
int vte_greedy_advance(const int* top_idx, int k, int rows, int* tokens, int* kv_offset, int max_pos, int* history,
                       int history_steps, int* step, void* stream);

/* vte_topk over the tokens NOT in each row's exclusion list, plus the exact
 * logits of the excluded tokens.  excl_ids [rows][max_excl]: sorted token ids
 * (the repetition window of the sampler, max_excl <= 4096; the reference uses
 * 512); excl_cnt [rows]: how many of them are valid.  Both are read on the
 * device, so a captured graph sees the values staged before each replay.
 * gathered [rows][max_excl]: logits[row][excl_ids[row][i]] for i < excl_cnt[row].
 * Since the repetition penalty only lowers logits, the top-k of the penalised
 * row is contained in the k returned candidates plus the penalised gathered
 * values.  Needs vocab - max_excl >= k.
 * Replaces: topk_reduce_greedy_kernel's exclusion and gather
 *           (topk_reduce_greedy.hip.template:40-83) and the buffers of
 *           TopKLogitsReducer (vte/core/topk_logits_reducer.py:79-125). */
int vte_topk_exclude(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
                     const int* excl_ids, const int* excl_cnt, int max_excl, float* gathered, void* stream);

/* One launch: RMSNorm(x) -> q/k/v projections (+bias) -> NEOX RoPE on q and k
 * -> q to q_out [B][n_q*128], k and v appended to the caches at kv_offset[b].
 * Same rounding points as the unfused nodes.  head_dim 128, q/k Q4_K, v Q4_K
 * or Q6_K.  norm_w NULL: x is already normalised (fp16) and is used as is.
 * With norm_w: batch 1..4 on the VALU mat-vec (norm fused in).  NULL norm_w:
 * batch 1..2 on the VALU mat-vec, batch 3..4096 on MFMA (launches of 32
 * sequences; above 32 one weight-stationary launch, same results); above
 * batch 4 norm_w must be NULL (RMSNorm runs before).
 * Replaces: the rmsnorm -> q/k/v gemv -> rope -> kv_cache_append nodes
 *           (vte/compiler/qwen_compute.py:100-282) and their fused forms
 *           FusedQKVDispatcher (vte/core/fused_qkv_dispatch.py:12-198),
 *           fused_norm_matmul_rope_kernel (fused_norm_matmul_rope.hip.template:34-199). */
int vte_attn_in(const void* x, const void* norm_w, float eps, const void* wq, const void* q_bias, int fmt_q,
                const void* wk, const void* k_bias, int fmt_k, const void* wv, const void* v_bias, int fmt_v,
                void* q_out, void* k_cache, void* v_cache, const int* kv_offset, int kv_batch_stride,
                const void* rope_cos, const void* rope_sin, int batch, int hidden, int n_q, int n_kv, int head_dim,
                void* stream);

/* One launch: RMSNorm(x) -> gate and up projections -> fp16(silu(g) * u),
 * out [B][ffn], Q4_K gate/up.  norm_w NULL: x is already normalised.
 * With norm_w: batch 1..4 on the VALU mat-vec.  NULL norm_w: batch 1..2 on
 * the VALU mat-vec, 3..4096 on MFMA; above batch 4 norm_w must be NULL.
 * Replaces: FusedFFNDispatcher (vte/core/fused_qkv_dispatch.py:200-270) with
 *           fused_gate_up_silu_kernel (fused_rmsnorm_gate_up_silu.hip.template:66-111). */
int vte_ffn_in(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up, int fmt,
               void* out, int batch, int hidden, int ffn, void* stream);

/* One launch: RMSNorm(x) followed by the vte_gemv contract (the LM head with
 * out_dtype f32).  batch 1..4; Q4_K, Q6_K or Q8_0 (tied Q8_0 tables).
 * Replaces: the output_norm + LM-head capture (vte/core/hip_graph_executor.py:429-474). */
int vte_norm_gemv(const void* x, const void* norm_w, float eps, const void* w, int fmt, void* out, int out_dtype,
                  const void* bias, const void* residual, float residual_scale, int batch, int K, int N,
                  void* stream);

/* Attention output projection with the split-KV combine fused in:
 * out[b][n] = fp16(sum_k W[n][k] a[b][k] * residual_scale + residual[b][n]),
 * a[b][h*128 + d] = fp16(log-sum-exp combine of the partials of
 * vte_attn_split_kv for sequence b, head h), K = n_q * 128, N outputs,
 * fp16 residual nullable.  batch 1..4, max_splits <= 64, Q4_K or Q6_K.
 * Replaces: flash_attention_split_kv_reduce_kernel (flash_attention_split_kv_reduce.hip.template:14-67)
 *           followed by the o-proj gemv with residual (vte/compiler/qwen_compute.py:100-282). */
int vte_attn_out_gemv(const float* part_m, const float* part_l, const float* part_o, const int* kv_offset, int batch,
                      int n_q, int max_splits, int split, const void* w, int fmt, void* out, const void* residual,
                      float residual_scale, int N, void* stream);

/* dst[i] = fp16(scale * N(0,1)) from a counter-based generator (synthetic KV
 * prefixes); no reference counterpart (test and benchmark input). */
int vte_fill_normal_f16(void* dst, long long n, unsigned long long seed, float scale, void* stream);

/* ---- Persistent decode step (batch 1) ----
 * The whole Qwen2-shaped decode step of one sequence (every layer's
 * RMSNorm, q/k/v + bias + RoPE + K/V append, split-KV attention, o-proj +
 * residual, RMSNorm, gate/up + SwiGLU, down + residual) as ONE kernel launch
 * of one block per CU, then the output norm and the LM head as a second
 * launch (the fused norm + mat-vec of vte_norm_gemv).  Blocks hand
 * activations to each other through flagged words in the workspace instead
 * of kernel boundaries.
 * Limits: head_dim 128, n_q / n_kv <= 8, hidden, ffn and n_q * 128 multiples
 * of 256 and <= 10240 (hidden <= 8192); q/k/o/gate/up Q4_K, v and down Q4_K
 * or Q6_K, LM head Q4_K, Q6_K or Q8_0; the KV cache of one sequence [max_seq][n_kv][128] fp16 per
 * layer.  Replaces: the batch-1 capture of vte/core/hip_graph_executor.py:504-738
 * (nodes of vte/compiler/qwen_compute.py:100-282) up to the LM-head logits. */
typedef struct vte_decode_layer {
    const void *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down; /* raw GGUF rows */
    const void *q_bias, *k_bias, *v_bias;                    /* fp16, nullable */
    const void *attn_norm, *ffn_norm;                        /* fp16 [hidden] */
    void *k_cache, *v_cache;                                 /* fp16 [max_seq][n_kv][128] */
    int fmt_q, fmt_k, fmt_v, fmt_o, fmt_gate_up, fmt_down;
} vte_decode_layer;

typedef struct vte_decode_model {
    int n_layers, hidden, ffn, n_q, n_kv, head_dim, vocab, max_seq;
    float eps;
    const void *rope_cos, *rope_sin; /* fp16 [max_seq][128] (rope_cache_builder.py layout) */
    const void *output_norm;         /* fp16 [hidden] */
    const void *lm_head;             /* raw GGUF rows [vocab][hidden] */
    int fmt_lm;
} vte_decode_model;

/* Device workspace bytes the step needs (flagged activation buffers,
 * attention partials, down-projection partial sums, the last layer's output,
 * the layer table and a control word block). */
long long vte_decode_workspace_bytes(const vte_decode_model* m);

/* Validate the model, copy the layer table into the workspace and clear its
 * control words (synchronous on `stream`; not capturable).  Once per
 * workspace, before the first vte_decode_step. */
int vte_decode_setup(const vte_decode_model* m, const vte_decode_layer* layers, void* workspace,
                     long long workspace_bytes, void* stream);

/* One step: x = the token's embedding (fp16 [hidden]), kv_offset[0] = its
 * position (read on the device; rows 0..kv_offset-1 of every cache hold the
 * prefix, row kv_offset is written), logits fp32 [vocab].  Capturable.
 * Steps on one workspace must not overlap. */
int vte_decode_step(const vte_decode_model* m, void* workspace, const int* kv_offset, const void* x, float* logits,
                    void* stream);

/* Synchronous read of the workspace's error flags: bit 0 = a block waited
 * past its deadline (a step whose blocks could not all be resident); bit 1 =
 * kv_offset[0] was outside [0, max_seq) (the step wrote nothing, its logits
 * are invalid). */
int vte_decode_status(void* workspace, int* flags);

/* Batched persistent step (csrc/decode_persistent_mm.hip): the layers of a
 * decode step for `batch` <= 16 sequences, each at its own position, as one
 * launch; replaces the per-layer launches of the batched graph
 * (vte/core/batched_hip_graph_executor.py:231-292, execute_decode_batch at
 * :287-292) up to the LM head.  Supports hidden and n_q*128 up to 1536, every
 * projection Q4_K or Q6_K.  Workspace bytes for `batch` sequences (-1: shape
 * not supported). */
long long vte_decode_batch_workspace_bytes(const vte_decode_model* m, int batch);

/* As vte_decode_setup, for the batched workspace (synchronous, once). */
int vte_decode_batch_setup(const vte_decode_model* m, const vte_decode_layer* layers, int batch, void* workspace,
                           long long workspace_bytes, void* stream);

/* One batched step: x = the embeddings fp16 [batch][hidden]; kv_offset[b]
 * (device) = sequence b's position, its cache at layer.k_cache + b *
 * kv_batch_stride (elements); h_out = the last layer's output fp16
 * [batch][hidden] (the caller runs the output norm and LM head).  Capturable;
 * error flags through vte_decode_status (bit 1: a position outside
 * [0, max_seq), nothing written).  Steps on one workspace must not overlap. */
int vte_decode_batch_step(const vte_decode_model* m, void* workspace, int batch, long long kv_batch_stride,
                          const int* kv_offset, const void* x, void* h_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VTE_AMD_H */
