// C ABI of libvte_amd.so: plain pointers, sizes and a hipStream_t passed as
// void*.  Every entry point validates shapes on the host before launching, so
// a kernel never runs with a geometry it does not support.  Return value: 0 on
// success, VTE_EINVAL (-1) for a rejected argument, otherwise the hipError_t
// of the failed launch; vte_last_error() gives the message.  Declarations and
// reference citations: include/vte_amd.h (included, so the compiler checks
// every definition against its declaration).
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/vte_amd.h"
#include "vte_common.h"
#include "fused_kernels.h"
#include "decode_persistent.h"
#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace vte {
template <typename TI, typename TO>
hipError_t gemv_valu(int fmt, const void* x, const void* w, void* y, int M, int K, int N, const void* bias,
                     const void* residual, float rs, hipStream_t st);
hipError_t gemm_mfma(int fmt, int in_dt, int out_dt, const void* x, const void* w, void* y, int M, int K, int N,
                     const void* bias, const void* residual, float rs, hipStream_t st);
hipError_t attn_out_mv(const float* part_m, const float* part_l, const float* part_o, const int* kv_offset, int M,
                       int n_q, int max_splits, int split, const void* w, int fmt, void* out, const void* residual,
                       float rs, int N, hipStream_t st);
hipError_t stream_mv(int fmt, bool in_f32, bool out_f32, const void* x, const void* w, void* y, int M, int K, int N,
                     const void* bias, const void* residual, float rs, hipStream_t st);
hipError_t dequantize(int fmt, const void* src, float* dst, long long n_elements, hipStream_t st);
template <typename TQ, typename TO>
hipError_t attn_split_kv(const void* q, const void* k_cache, const void* v_cache, float* part_m, float* part_l,
                         float* part_o, void* out, int B, int n_q, int n_kv, float scale, const int* kv_offset,
                         int kv_batch_stride, int split, int max_splits, int* counters, hipStream_t st);
hipError_t kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int B, int n_kv, int head_dim,
                     const int* kv_offset, int kv_batch_stride, hipStream_t st);
hipError_t rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps, hipStream_t st);
hipError_t add_rmsnorm(const void* x, const float* part, int n_parts, const void* w, void* x_out, void* xn,
                       int rows, int hidden, float eps, hipStream_t st);
hipError_t gemm_mfma_splitk(int fmt, const void* x, const void* w, float* part, int M, int K, int N, int splits,
                            hipStream_t st);
hipError_t rope(void* q, void* k, const void* cosc, const void* sinc, int B, int seq_len, int n_q, int n_kv,
                int head_dim, const int* kv_offset, int rope_type, int rotary_dim, hipStream_t st);
hipError_t swiglu(const void* g, const void* u, void* out, int n, hipStream_t st);
hipError_t add(const void* r, const void* in, void* out, int n, float scale, hipStream_t st);
hipError_t embedding(int fmt, const int* tokens, const void* table, void* out, int n_tokens, int hidden,
                     float scale, hipStream_t st);
size_t topk_scratch_bytes(int rows);
hipError_t greedy_advance(const int* top_idx, int k, int rows, int* tokens, int* kv_offset, int max_pos,
                          int* history, int hist_steps, int* step, hipStream_t st);
hipError_t topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
                hipStream_t st, const int* excl_ids, const int* excl_cnt, int max_excl, float* gathered);
int topk_noalloc_max_rows();
hipError_t topk_noalloc(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx,
                        hipStream_t st);
hipError_t fill_normal_f16(void* dst, long long n, unsigned long long seed, float scale, hipStream_t st);
hipError_t attn_in(const void* x, const void* norm_w, float eps, const void* wq, const void* q_bias, int fmt_q,
                   const void* wk, const void* k_bias, int fmt_k, const void* wv, const void* v_bias, int fmt_v,
                   void* q_out, void* k_cache, void* v_cache, const int* kv_offset, int kv_batch_stride,
                   const void* rope_cos, const void* rope_sin, int M, int K, int n_q, int n_kv, hipStream_t st);
hipError_t ffn_in(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up, int fmt,
                  void* out, int M, int K, int ffn, hipStream_t st);
hipError_t qkv_mm(const void* xn, const void* wq, const void* q_bias, int fmt_q, const void* wk, const void* k_bias,
                  int fmt_k, const void* wv, const void* v_bias, int fmt_v, void* q_out, void* k_cache, void* v_cache,
                  const int* kv_offset, int kv_batch_stride, const void* rope_cos, const void* rope_sin, int B, int K,
                  int n_q, int n_kv, hipStream_t st);
hipError_t gate_up_mm(const void* xn, const void* w_gate, const void* w_up, int fmt, void* out, int B, int K, int ffn,
                      hipStream_t st);
hipError_t norm_mv(const void* x, const void* norm_w, float eps, const void* w, int fmt, void* out, bool out_f32,
                   const void* bias, const void* residual, float rs, int M, int K, int N, hipStream_t st);
}  // namespace vte

static thread_local char g_err[512] = "";

static int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return VTE_EINVAL;
}

static int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    snprintf(g_err, sizeof(g_err), "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return (int)e;
}

#define REQUIRE(cond, ...) \
    do {                   \
        if (!(cond)) return fail(__VA_ARGS__); \
    } while (0)

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

static int check_gemv(int fmt, int in_dt, int out_dt, const void* x, const void* w, void* y, int M, int K, int N) {
    REQUIRE(fmt == 4 || fmt == 6 || fmt == 8, "gemv: unknown format %d (4=Q4_K, 6=Q6_K, 8=Q8_0)", fmt);
    REQUIRE(in_dt == VTE_F32 || in_dt == VTE_F16, "gemv: in_dtype must be 0 (f32) or 1 (f16)");
    REQUIRE(out_dt == VTE_F32 || out_dt == VTE_F16, "gemv: out_dtype must be 0 (f32) or 1 (f16)");
    REQUIRE(x && w && y, "gemv: null input/weight/output pointer");
    REQUIRE(M >= 1 && N >= 1 && K >= 1, "gemv: empty shape M=%d K=%d N=%d", M, K, N);
    REQUIRE(K % ((fmt == 8) ? 32 : 256) == 0, "gemv: in_features %d not a multiple of the block size", K);
    REQUIRE(K <= 65536, "gemv: in_features %d exceeds 65536", K);
    REQUIRE(aligned(x, 16), "gemv: input must be 16-byte aligned");
    REQUIRE(aligned(w, 16), "gemv: weight must be 16-byte aligned");
    return 0;
}

extern "C" {

const char* vte_last_error(void) { return g_err; }

int vte_abi_version(void) { return 1; }

int vte_device_info(int device, int* n_cu, long long* total_mem, char* arch, int arch_len) {
    REQUIRE(n_cu && total_mem && arch && arch_len > 0, "device_info: null pointer");
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return hip_status(e, "hipGetDeviceProperties");
    *n_cu = p.multiProcessorCount;
    *total_mem = (long long)p.totalGlobalMem;
    snprintf(arch, (size_t)arch_len, "%s", p.gcnArchName);
    return 0;
}

int vte_gemv(int fmt, int in_dtype, int out_dtype, const void* x, const void* w, void* y, int M, int K, int N,
             const void* bias, const void* residual, float residual_scale, void* stream) {
    int rc = check_gemv(fmt, in_dtype, out_dtype, x, w, y, M, K, N);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    e = vte::stream_mv(fmt, in_dtype == VTE_F32, out_dtype == VTE_F32, x, w, y, M, K, N, bias, residual,
                       residual_scale, st);
    if (e != hipErrorNotSupported) return hip_status(e, "vte_gemv launch");
    if (in_dtype == VTE_F32 && out_dtype == VTE_F32)
        e = vte::gemv_valu<float, float>(fmt, x, w, y, M, K, N, bias, residual, residual_scale, st);
    else if (in_dtype == VTE_F16 && out_dtype == VTE_F16)
        e = vte::gemv_valu<__half, __half>(fmt, x, w, y, M, K, N, bias, residual, residual_scale, st);
    else if (in_dtype == VTE_F16 && out_dtype == VTE_F32)
        e = vte::gemv_valu<__half, float>(fmt, x, w, y, M, K, N, bias, residual, residual_scale, st);
    else
        return fail("gemv: f32 input with f16 output is not provided");
    return hip_status(e, "vte_gemv launch");
}

int vte_gemm_mfma(int fmt, int in_dtype, int out_dtype, const void* x, const void* w, void* y, int M, int K,
                  int N, const void* bias, const void* residual, float residual_scale, void* stream) {
    int rc = check_gemv(fmt, in_dtype, out_dtype, x, w, y, M, K, N);
    if (rc) return rc;
    REQUIRE(fmt == 4 || fmt == 6, "gemm_mfma: Q4_K and Q6_K only");
    REQUIRE(!(in_dtype == VTE_F32 && out_dtype == VTE_F16), "gemm_mfma: f32 input with f16 output is not provided");
    return hip_status(vte::gemm_mfma(fmt, in_dtype, out_dtype, x, w, y, M, K, N, bias, residual, residual_scale,
                                     (hipStream_t)stream),
                      "vte_gemm_mfma launch");
}

int vte_gemm_mfma_splitk(int fmt, const void* x, const void* w, float* part, int M, int K, int N, int splits,
                         void* stream) {
    int rc = check_gemv(fmt, VTE_F16, VTE_F32, x, w, part, M, K, N);
    if (rc) return rc;
    REQUIRE(fmt == 4 || fmt == 6, "gemm_mfma_splitk: Q4_K and Q6_K only");
    REQUIRE(splits >= 1 && splits <= 8 && splits <= K / 256, "gemm_mfma_splitk: splits %d outside 1..min(8, K/256)",
            splits);
    return hip_status(vte::gemm_mfma_splitk(fmt, x, w, part, M, K, N, splits, (hipStream_t)stream),
                      "vte_gemm_mfma_splitk launch");
}

int vte_dequantize(int fmt, const void* src, float* dst, long long n_elements, void* stream) {
    REQUIRE(fmt == 4 || fmt == 6 || fmt == 8, "dequantize: unknown format %d", fmt);
    REQUIRE(src && dst, "dequantize: null pointer");
    REQUIRE(n_elements > 0 && n_elements % ((fmt == 8) ? 32 : 256) == 0,
            "dequantize: n_elements %lld not a positive multiple of the block size", n_elements);
    REQUIRE(n_elements / 256 < (1LL << 31), "dequantize: too many elements");
    return hip_status(vte::dequantize(fmt, src, dst, n_elements, (hipStream_t)stream), "vte_dequantize launch");
}

long long vte_attn_scratch_floats(int batch, int n_q, int max_splits) {
    // part_m + part_l + part_o
    return (long long)batch * n_q * max_splits * (2 + 128);
}

int vte_attn_split_kv(int dtype, const void* q, const void* k_cache, const void* v_cache, float* part_m,
                      float* part_l, float* part_o, void* out, int batch, int n_q, int n_kv, int head_dim,
                      float scale, const int* kv_offset, int kv_batch_stride, int split, int max_splits,
                      int* counters, void* stream) {
    REQUIRE(dtype == VTE_F32 || dtype == VTE_F16, "attn: dtype must be 0 (f32) or 1 (f16)");
    REQUIRE(q && k_cache && v_cache && part_m && part_l && part_o && kv_offset, "attn: null pointer");
    REQUIRE(out != nullptr || counters == nullptr, "attn: the in-kernel combine needs an output");
    REQUIRE(head_dim == 128, "attn: head_dim %d unsupported (128 only)", head_dim);
    REQUIRE(batch >= 1 && n_kv >= 1 && n_q >= n_kv && n_q % n_kv == 0, "attn: bad head counts %d/%d", n_q, n_kv);
    REQUIRE(n_q / n_kv <= 8, "attn: GQA group %d > 8 unsupported", n_q / n_kv);
    REQUIRE(split >= 32 && split % 32 == 0, "attn: split %d must be a positive multiple of 32", split);
    REQUIRE(max_splits >= 1 && max_splits <= 4096, "attn: max_splits %d out of range (1..4096)", max_splits);
    REQUIRE(counters == nullptr || max_splits <= 512, "attn: in-kernel combine supports at most 512 splits");
    REQUIRE(counters == nullptr || split > 32, "attn: in-kernel combine needs splits of more than 32 tokens");
    REQUIRE(aligned(k_cache, 16) && aligned(v_cache, 16), "attn: KV cache must be 16-byte aligned");
    REQUIRE(aligned(q, 16), "attn: q must be 16-byte aligned");
    REQUIRE(kv_batch_stride % 8 == 0, "attn: kv_batch_stride must keep rows 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = (dtype == VTE_F32)
                       ? vte::attn_split_kv<float, float>(q, k_cache, v_cache, part_m, part_l, part_o, out, batch,
                                                          n_q, n_kv, scale, kv_offset, kv_batch_stride, split,
                                                          max_splits, counters, st)
                       : vte::attn_split_kv<__half, __half>(q, k_cache, v_cache, part_m, part_l, part_o, out,
                                                            batch, n_q, n_kv, scale, kv_offset, kv_batch_stride,
                                                            split, max_splits, counters, st);
    return hip_status(e, "vte_attn_split_kv launch");
}

int vte_add_rmsnorm(const void* x, const float* part, int n_parts, const void* w, void* x_out, void* xn, int rows,
                    int hidden, float eps, void* stream) {
    REQUIRE(x && part && w && x_out && xn, "add_rmsnorm: null pointer");
    REQUIRE(rows >= 1 && n_parts >= 1 && n_parts <= 8, "add_rmsnorm: rows %d / n_parts %d", rows, n_parts);
    REQUIRE(hidden >= 8 && hidden % 8 == 0 && hidden <= 8192, "add_rmsnorm: hidden %d not a multiple of 8 in 8..8192",
            hidden);
    REQUIRE(aligned(x, 16) && aligned(part, 16) && aligned(w, 16) && aligned(x_out, 16) && aligned(xn, 16),
            "add_rmsnorm: 16-byte alignment required");
    return hip_status(vte::add_rmsnorm(x, part, n_parts, w, x_out, xn, rows, hidden, eps, (hipStream_t)stream),
                      "vte_add_rmsnorm launch");
}

int vte_kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int batch, int n_kv, int head_dim,
                  const int* kv_offset, int kv_batch_stride, void* stream) {
    REQUIRE(k && v && k_cache && v_cache && kv_offset, "kv_append: null pointer");
    REQUIRE(batch >= 1 && n_kv >= 1 && head_dim >= 1 && head_dim <= 1024, "kv_append: bad shape");
    return hip_status(vte::kv_append(k, v, k_cache, v_cache, batch, n_kv, head_dim, kv_offset, kv_batch_stride,
                                     (hipStream_t)stream),
                      "vte_kv_append launch");
}

int vte_rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps, void* stream) {
    REQUIRE(x && w && out, "rmsnorm: null pointer");
    REQUIRE(rows >= 1 && hidden >= 1, "rmsnorm: empty shape");
    REQUIRE(hidden % 8 != 0 || (aligned(x, 16) && aligned(w, 16) && aligned(out, 16)),
            "rmsnorm: 16-byte alignment required");
    return hip_status(vte::rmsnorm(x, w, out, rows, hidden, eps, (hipStream_t)stream), "vte_rmsnorm launch");
}

int vte_rope(void* q, void* k, const void* cos_cache, const void* sin_cache, int batch, int seq_len, int n_q,
             int n_kv, int head_dim, const int* kv_offset, int rope_type, int rotary_dim, void* stream) {
    REQUIRE(q && k && cos_cache && sin_cache && kv_offset, "rope: null pointer");
    REQUIRE(batch >= 1 && seq_len >= 1 && n_q >= n_kv && n_kv >= 1 && head_dim % 2 == 0, "rope: bad shape");
    REQUIRE(rope_type >= 0 && rope_type <= 2, "rope: rope_type %d unknown", rope_type);
    REQUIRE(rope_type != 2 || (rotary_dim > 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0),
            "rope: bad rotary_dim %d", rotary_dim);
    return hip_status(vte::rope(q, k, cos_cache, sin_cache, batch, seq_len, n_q, n_kv, head_dim, kv_offset,
                                rope_type, rotary_dim, (hipStream_t)stream),
                      "vte_rope launch");
}

int vte_swiglu(const void* gate, const void* up, void* out, int n, void* stream) {
    REQUIRE(gate && up && out && n >= 1, "swiglu: bad arguments");
    return hip_status(vte::swiglu(gate, up, out, n, (hipStream_t)stream), "vte_swiglu launch");
}

int vte_add(const void* residual, const void* input, void* out, int n, float scale, void* stream) {
    REQUIRE(residual && input && out && n >= 1, "add: bad arguments");
    return hip_status(vte::add(residual, input, out, n, scale, (hipStream_t)stream), "vte_add launch");
}

static int embedding_call(int fmt, const char* name, const int* tokens, const void* table, void* out, int n_tokens,
                          int hidden, float scale, void* stream) {
    const int qb = fmt == 8 ? 32 : 256;
    REQUIRE(tokens && table && out && n_tokens >= 1 && hidden >= 1, "%s: bad arguments", name);
    REQUIRE(hidden % qb == 0, "%s: hidden %d not a multiple of %d", name, hidden, qb);
    REQUIRE((long long)n_tokens * hidden <= 0x7fffffffLL, "%s: %d tokens x %d too large", name, n_tokens, hidden);
    return hip_status(vte::embedding(fmt, tokens, table, out, n_tokens, hidden, scale, (hipStream_t)stream), name);
}

int vte_embedding_q6k(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                      void* stream) {
    return embedding_call(6, "vte_embedding_q6k", tokens, table, out, n_tokens, hidden, scale, stream);
}

int vte_embedding_q4k(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                      void* stream) {
    return embedding_call(4, "vte_embedding_q4k", tokens, table, out, n_tokens, hidden, scale, stream);
}

int vte_embedding_q8_0(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                       void* stream) {
    return embedding_call(8, "vte_embedding_q8_0", tokens, table, out, n_tokens, hidden, scale, stream);
}

long long vte_topk_scratch_bytes(int rows) { return (long long)vte::topk_scratch_bytes(rows); }

int vte_topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
             void* stream) {
    REQUIRE(logits && out_val && out_idx && scratch, "topk: null pointer");
    REQUIRE(rows >= 1 && k >= 1 && k <= 64 && vocab >= k, "topk: need 1 <= k <= min(64, vocab)");
    REQUIRE(rows <= 65535, "topk: rows %d out of range", rows);
    REQUIRE(vocab <= 262144, "topk: vocab %d above 262144", vocab);
    REQUIRE(aligned(scratch, 8), "topk: scratch must be 8-byte aligned");
    return hip_status(vte::topk(logits, rows, vocab, k, out_val, out_idx, scratch, (hipStream_t)stream, nullptr,
                                nullptr, 0, nullptr),
                      "vte_topk launch");
}

int vte_greedy_advance(const int* top_idx, int k, int rows, int* tokens, int* kv_offset, int max_pos, int* history,
                       int history_steps, int* step, void* stream) {
    REQUIRE(top_idx && tokens && kv_offset && step, "greedy_advance: null pointer");
    REQUIRE(k >= 1 && rows >= 1 && rows <= 65535 && max_pos >= 0, "greedy_advance: bad shape");
    REQUIRE(history != nullptr || history_steps == 0, "greedy_advance: history steps without a history buffer");
    return hip_status(vte::greedy_advance(top_idx, k, rows, tokens, kv_offset, max_pos, history, history_steps, step,
                                          (hipStream_t)stream),
                      "vte_greedy_advance launch");
}

int vte_topk_noalloc(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* stream) {
    REQUIRE(logits && out_val && out_idx, "topk_noalloc: null pointer");
    REQUIRE(rows >= 1 && k >= 1 && k <= 64 && vocab >= k, "topk_noalloc: need 1 <= k <= min(64, vocab)");
    REQUIRE(rows <= vte::topk_noalloc_max_rows(),
            "topk_noalloc: %d rows exceed the library's fixed scratch of %d rows (use vte_topk with a workspace)",
            rows, vte::topk_noalloc_max_rows());
    REQUIRE(vocab <= 262144, "topk_noalloc: vocab %d above 262144", vocab);
    return hip_status(vte::topk_noalloc(logits, rows, vocab, k, out_val, out_idx, (hipStream_t)stream),
                      "vte_topk_noalloc launch");
}

int vte_topk_exclude(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
                     const int* excl_ids, const int* excl_cnt, int max_excl, float* gathered, void* stream) {
    REQUIRE(logits && out_val && out_idx && scratch && excl_ids && excl_cnt && gathered, "topk_exclude: null pointer");
    REQUIRE(rows >= 1 && k >= 1 && k <= 64 && vocab >= k, "topk_exclude: need 1 <= k <= min(64, vocab)");
    REQUIRE(rows <= 65535, "topk_exclude: rows %d out of range", rows);
    REQUIRE(vocab <= 262144, "topk_exclude: vocab %d above 262144", vocab);
    REQUIRE(max_excl >= 1 && max_excl <= 4096, "topk_exclude: max_excl %d outside 1..4096", max_excl);
    REQUIRE(vocab - max_excl >= k, "topk_exclude: vocab %d leaves fewer than k outside %d exclusions", vocab, max_excl);
    REQUIRE(aligned(scratch, 8), "topk_exclude: scratch must be 8-byte aligned");
    return hip_status(vte::topk(logits, rows, vocab, k, out_val, out_idx, scratch, (hipStream_t)stream, excl_ids,
                                excl_cnt, max_excl, gathered),
                      "vte_topk_exclude launch");
}

int vte_attn_in(const void* x, const void* norm_w, float eps, const void* wq, const void* q_bias, int fmt_q,
                const void* wk, const void* k_bias, int fmt_k, const void* wv, const void* v_bias, int fmt_v,
                void* q_out, void* k_cache, void* v_cache, const int* kv_offset, int kv_batch_stride,
                const void* rope_cos, const void* rope_sin, int batch, int hidden, int n_q, int n_kv, int head_dim,
                void* stream) {
    REQUIRE(x && wq && wk && wv && q_out && k_cache && v_cache && kv_offset && rope_cos && rope_sin,
            "attn_in: null pointer");
    REQUIRE(head_dim == 128, "attn_in: head_dim must be 128");
    REQUIRE(batch >= 1 && batch <= 4096, "attn_in: batch %d outside 1..4096", batch);
    REQUIRE(batch <= 4 || norm_w == nullptr,
            "attn_in: batch %d > 4 takes RMSNorm-ed activations (norm_w must be NULL)", batch);
    REQUIRE(hidden % 256 == 0 && hidden <= 8192, "attn_in: hidden %d unsupported", hidden);
    REQUIRE(fmt_q == 4 && fmt_k == 4 && (fmt_v == 4 || fmt_v == 6), "attn_in: q/k must be Q4_K, v Q4_K or Q6_K");
    REQUIRE(n_kv >= 1 && n_q >= n_kv && n_q % n_kv == 0, "attn_in: bad head counts");
    REQUIRE(aligned(x, 16) && aligned(norm_w, 16) && aligned(wq, 16) && aligned(wk, 16) && aligned(wv, 16),
            "attn_in: 16-byte alignment");
    hipError_t e;
    if (norm_w != nullptr || batch <= 2)  // fused mat-vec; batch >= 3 on normalised activations: MFMA
        e = vte::attn_in(x, norm_w, eps, wq, q_bias, fmt_q, wk, k_bias, fmt_k, wv, v_bias, fmt_v, q_out, k_cache,
                         v_cache, kv_offset, kv_batch_stride, rope_cos, rope_sin, batch, hidden, n_q, n_kv,
                         (hipStream_t)stream);
    else
        e = vte::qkv_mm(x, wq, q_bias, fmt_q, wk, k_bias, fmt_k, wv, v_bias, fmt_v, q_out, k_cache, v_cache,
                        kv_offset, kv_batch_stride, rope_cos, rope_sin, batch, hidden, n_q, n_kv, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("attn_in: shape does not fit the fused kernel's LDS plan");
    return hip_status(e, "vte_attn_in launch");
}

int vte_ffn_in(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up, int fmt,
               void* out, int batch, int hidden, int ffn, void* stream) {
    REQUIRE(x && w_gate && w_up && out, "ffn_in: null pointer");
    REQUIRE(fmt == 4, "ffn_in: gate/up must be Q4_K");
    REQUIRE(batch >= 1 && batch <= 4096, "ffn_in: batch %d outside 1..4096", batch);
    REQUIRE(batch <= 4 || norm_w == nullptr,
            "ffn_in: batch %d > 4 takes RMSNorm-ed activations (norm_w must be NULL)", batch);
    REQUIRE(hidden % 256 == 0 && hidden <= 8192 && ffn >= 1, "ffn_in: bad shape");
    REQUIRE(aligned(x, 16) && aligned(norm_w, 16) && aligned(w_gate, 16) && aligned(w_up, 16),
            "ffn_in: 16-byte alignment");
    hipError_t e = norm_w != nullptr || batch <= 2
                       ? vte::ffn_in(x, norm_w, eps, w_gate, w_up, fmt, out, batch, hidden, ffn, (hipStream_t)stream)
                       : vte::gate_up_mm(x, w_gate, w_up, fmt, out, batch, hidden, ffn, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("ffn_in: shape does not fit the fused kernel's LDS plan");
    return hip_status(e, "vte_ffn_in launch");
}

int vte_norm_gemv(const void* x, const void* norm_w, float eps, const void* w, int fmt, void* out, int out_dtype,
                  const void* bias, const void* residual, float residual_scale, int batch, int K, int N,
                  void* stream) {
    REQUIRE(x && norm_w && w && out, "norm_gemv: null pointer");
    REQUIRE(fmt == 4 || fmt == 6 || fmt == 8, "norm_gemv: Q4_K, Q6_K or Q8_0");
    REQUIRE(out_dtype == VTE_F32 || out_dtype == VTE_F16, "norm_gemv: bad out dtype");
    REQUIRE(batch >= 1 && batch <= 4, "norm_gemv: batch %d outside 1..4", batch);
    REQUIRE(K % 256 == 0 && K <= 8192 && N >= 1, "norm_gemv: bad shape");
    REQUIRE(aligned(x, 16) && aligned(norm_w, 16) && aligned(w, 16), "norm_gemv: 16-byte alignment");
    hipError_t e = vte::norm_mv(x, norm_w, eps, w, fmt, out, out_dtype == VTE_F32, bias, residual, residual_scale,
                                batch, K, N, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("norm_gemv: shape does not fit the fused kernel's LDS plan");
    return hip_status(e, "vte_norm_gemv launch");
}

int vte_attn_out_gemv(const float* part_m, const float* part_l, const float* part_o, const int* kv_offset, int batch,
                      int n_q, int max_splits, int split, const void* w, int fmt, void* out, const void* residual,
                      float residual_scale, int N, void* stream) {
    REQUIRE(part_m && part_l && part_o && kv_offset && w && out, "attn_out_gemv: null pointer");
    REQUIRE(fmt == 4 || fmt == 6, "attn_out_gemv: Q4_K or Q6_K");
    REQUIRE(batch >= 1 && batch <= 4, "attn_out_gemv: batch %d outside 1..4", batch);
    REQUIRE(n_q >= 1 && (n_q * 128) % 256 == 0 && n_q * 128 <= 8192 && N >= 1, "attn_out_gemv: bad shape");
    REQUIRE(max_splits >= 1 && max_splits <= 64, "attn_out_gemv: max_splits %d outside 1..64", max_splits);
    REQUIRE(split >= 1, "attn_out_gemv: split must be positive");
    REQUIRE(aligned(part_o, 16) && aligned(w, 16), "attn_out_gemv: 16-byte alignment");
    hipError_t e = vte::attn_out_mv(part_m, part_l, part_o, kv_offset, batch, n_q, max_splits, split, w, fmt, out,
                                    residual, residual_scale, N, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("attn_out_gemv: shape does not fit the kernel's LDS plan");
    return hip_status(e, "vte_attn_out_gemv launch");
}

int vte_fill_normal_f16(void* dst, long long n, unsigned long long seed, float scale, void* stream) {
    REQUIRE(dst && n >= 1 && n / 256 < (1LL << 31), "fill_normal_f16: bad arguments");
    return hip_status(vte::fill_normal_f16(dst, n, seed, scale, (hipStream_t)stream), "vte_fill_normal_f16 launch");
}

}  // extern "C"

// ------------------------------------------------------------------ persistent decode step

namespace {
struct PdLayout {
    size_t ctrl, layers, ll_h, ll_q, ll_kv, ll_att, ll_hm, ll_act, part, ll_dn, h_out, total;
};
size_t pd_align(size_t x) { return (x + 255) & ~(size_t)255; }
PdLayout pd_layout(const vte_decode_model* m) {
    PdLayout L;
    const size_t qd = (size_t)m->n_q * 128, kvd = (size_t)m->n_kv * 128;
    size_t o = 0;
    L.ctrl = o; o = pd_align(o + 256);
    L.layers = o; o = pd_align(o + (size_t)m->n_layers * sizeof(vte_decode_layer));
    L.ll_h = o; o = pd_align(o + (size_t)m->hidden * 4);
    L.ll_q = o; o = pd_align(o + qd * 4);
    L.ll_kv = o; o = pd_align(o + 2 * kvd * 4);
    L.ll_att = o; o = pd_align(o + qd * 4);
    L.ll_hm = o; o = pd_align(o + (size_t)m->hidden * 4);
    L.ll_act = o; o = pd_align(o + (size_t)m->ffn * 4);
    L.part = o; o = pd_align(o + (size_t)m->n_q * VTE_DECODE_MAX_SPLITS * 130 * 8);
    L.ll_dn = o; o = pd_align(o + (size_t)(m->ffn / 256) * m->hidden * 8);
    L.h_out = o; o = pd_align(o + (size_t)m->hidden * 2);
    L.total = o;
    return L;
}
int pd_check_model(const vte_decode_model* m, bool pointers = true) {
    REQUIRE(m != nullptr, "decode: null model");
    REQUIRE(m->n_layers >= 1 && m->n_layers <= 1024, "decode: n_layers %d", m->n_layers);
    REQUIRE(m->head_dim == 128, "decode: head_dim must be 128");
    REQUIRE(m->n_kv >= 1 && m->n_q % m->n_kv == 0 && m->n_q / m->n_kv <= 8, "decode: n_q / n_kv must be <= 8");
    const int qd = m->n_q * 128;
    REQUIRE(m->hidden % 256 == 0 && m->hidden <= 10240 && m->ffn % 256 == 0 && m->ffn <= 10240 && qd % 256 == 0 &&
                qd <= 10240, "decode: hidden, ffn and n_q*128 must be multiples of 256 up to 10240");
    REQUIRE(fmv_ro(m->hidden) == fmv_ro(qd), "decode: hidden %d and q_dim %d need the same unit mapping", m->hidden, qd);
    REQUIRE(m->hidden <= 8192, "decode: hidden %d above the LM head's 8192", m->hidden);
    REQUIRE(m->vocab >= 1 && m->max_seq >= 1, "decode: vocab / max_seq");
    if (!pointers) return 0;
    REQUIRE(m->fmt_lm == 4 || m->fmt_lm == 6 || m->fmt_lm == 8, "decode: LM head must be Q4_K, Q6_K or Q8_0");
    REQUIRE(m->rope_cos && m->rope_sin && m->output_norm && m->lm_head, "decode: null model pointer");
    REQUIRE(aligned(m->output_norm, 16) && aligned(m->lm_head, 16), "decode: 16-byte alignment");
    return 0;
}
int pd_cap(int K, int upt) {  // rows a tile of K-long rows can hold at `upt` units per thread
    const int per_row = (K / 256) * 4;
    return fmv_ro(K) ? (ROWS_THREADS / per_row) * upt : (upt * ROWS_THREADS) / per_row;
}
int g_pd_cus[64] = {0};
}  // namespace

long long vte_decode_workspace_bytes(const vte_decode_model* m) {
    if (pd_check_model(m, false)) return -1;
    return (long long)pd_layout(m).total;
}

int vte_decode_setup(const vte_decode_model* m, const vte_decode_layer* layers, void* ws, long long ws_bytes,
                     void* stream) {
    int rc = pd_check_model(m);
    if (rc) return rc;
    REQUIRE(layers && ws, "decode_setup: null pointer");
    REQUIRE(aligned(ws, 256), "decode_setup: workspace must be 256-byte aligned");
    const PdLayout L = pd_layout(m);
    REQUIRE(ws_bytes >= (long long)L.total, "decode_setup: workspace %lld < %zu bytes", ws_bytes, L.total);
    for (int l = 0; l < m->n_layers; ++l) {
        const vte_decode_layer& y = layers[l];
        REQUIRE(y.wq && y.wk && y.wv && y.wo && y.w_gate && y.w_up && y.w_down && y.attn_norm && y.ffn_norm &&
                    y.k_cache && y.v_cache, "decode_setup: layer %d: null pointer", l);
        REQUIRE(y.fmt_q == 4 && y.fmt_k == 4 && y.fmt_o == 4 && y.fmt_gate_up == 4 &&
                    (y.fmt_v == 4 || y.fmt_v == 6) && (y.fmt_down == 4 || y.fmt_down == 6),
                "decode_setup: layer %d: q/k/o/gate/up Q4_K, v and down Q4_K or Q6_K", l);
        REQUIRE(aligned(y.wq, 16) && aligned(y.wk, 16) && aligned(y.wv, 16) && aligned(y.wo, 16) &&
                    aligned(y.w_gate, 16) && aligned(y.w_up, 16) && aligned(y.w_down, 16) &&
                    aligned(y.attn_norm, 16) && aligned(y.ffn_norm, 16) && aligned(y.k_cache, 16) &&
                    aligned(y.v_cache, 16), "decode_setup: layer %d: 16-byte alignment", l);
    }
    hipStream_t st = (hipStream_t)stream;
    uint8_t* base = static_cast<uint8_t*>(ws);
    hipError_t e = hipMemsetAsync(base, 0, L.total, st);
    if (e != hipSuccess) return hip_status(e, "decode_setup memset");
    const uint32_t ctrl[4] = {1u, 0u, 0u, 0u};  // epoch starts at 1: no tag matches the cleared words
    e = hipMemcpyAsync(base + L.ctrl, ctrl, sizeof(ctrl), hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + L.layers, layers, (size_t)m->n_layers * sizeof(vte_decode_layer),
                           hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return hip_status(e, "decode_setup copy");
}

int vte_decode_step(const vte_decode_model* m, void* ws, const int* kv_offset, const void* x, float* logits,
                    void* stream) {
    int rc = pd_check_model(m);
    if (rc) return rc;
    REQUIRE(ws && kv_offset && x && logits, "decode_step: null pointer");
    REQUIRE(aligned(ws, 256) && aligned(x, 16), "decode_step: alignment");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    REQUIRE(dev >= 0 && dev < 64, "decode_step: device %d", dev);
    if (g_pd_cus[dev] == 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_status(e, "hipDeviceGetAttribute");
        g_pd_cus[dev] = n;
    }
    const int blocks = g_pd_cus[dev];  // one 256-thread block per CU
    const PdLayout L = pd_layout(m);
    uint8_t* base = static_cast<uint8_t*>(ws);
    VtePdPlan P{};
    P.layers = reinterpret_cast<const VtePdLayer*>(base + L.layers);
    P.n_layers = m->n_layers;
    P.hidden = m->hidden;
    P.ffn = m->ffn;
    P.n_q = m->n_q;
    P.n_kv = m->n_kv;
    P.eps = m->eps;
    P.scale = 1.0f / sqrtf(128.0f);
    P.kv_offset = kv_offset;
    P.max_seq = m->max_seq;
    P.x = static_cast<const __half*>(x);
    P.rope_cos = static_cast<const __half*>(m->rope_cos);
    P.rope_sin = static_cast<const __half*>(m->rope_sin);
    P.h_out = reinterpret_cast<__half*>(base + L.h_out);
    P.ll_h = reinterpret_cast<uint32_t*>(base + L.ll_h);
    P.ll_q = reinterpret_cast<uint32_t*>(base + L.ll_q);
    P.ll_kv = reinterpret_cast<uint32_t*>(base + L.ll_kv);
    P.ll_att = reinterpret_cast<uint32_t*>(base + L.ll_att);
    P.ll_hm = reinterpret_cast<uint32_t*>(base + L.ll_hm);
    P.ll_act = reinterpret_cast<uint32_t*>(base + L.ll_act);
    P.part = reinterpret_cast<uint64_t*>(base + L.part);
    P.ll_dn = reinterpret_cast<uint64_t*>(base + L.ll_dn);
    P.ctrl = reinterpret_cast<uint32_t*>(base + L.ctrl);
    const int H = m->hidden, F = m->ffn, qd = m->n_q * 128, kvd = m->n_kv * 128;
    // rows per tile: RoPE tiles a power of two (pairs d, d + 64 of one head);
    // otherwise about one tile per block, within the stage's units per thread
    int r = 2;
    while (r * 2 <= std::min(pd_cap(H, VTE_PD_UPT_QKV), 128)) r *= 2;
    P.r_qk = r;
    P.r_v = std::max(1, pd_cap(H, VTE_PD_UPT_QKV));
    P.r_o = std::max(1, std::min(pd_cap(qd, 1), (H + blocks - 1) / blocks));
    // gate/up: about one tile per block, none on the last n_q blocks (they run
    // the attention combine, so their o-proj is the stage's critical path)
    const int gu_blocks = std::max(1, blocks - m->n_q);
    P.r_gu = std::min(pd_cap(H, VTE_PD_UPT_GU) & ~1, 2 * ((F + gu_blocks - 1) / gu_blocks));
    // down: F / 256 slices; about blocks / slices row tiles each, of at most
    // 256 rows (4 units per row, 64 rows per pass of the 256 threads, 4 passes)
    const int nsl = F / 256;
    P.r_dn = std::min(256, (H + std::max(1, blocks / nsl) - 1) / std::max(1, blocks / nsl));
    P.r_red = (H + blocks - 1) / blocks;
    REQUIRE(P.r_qk >= 2 && P.r_gu >= 2 && P.r_dn >= 1, "decode_step: tile plan does not fit");
    REQUIRE(P.r_red <= ROWS_THREADS, "decode_step: %d reduce rows per block exceed %d threads (hidden %d on %d CUs)",
            P.r_red, ROWS_THREADS, H, blocks);
    REQUIRE(kvd % P.r_qk == 0 && qd % P.r_qk == 0, "decode_step: RoPE tiles");
    static const int split_env = [] {
        const char* s = getenv("VTE_PD_SPLIT");  // tuning: smallest attention split (multiple of 32)
        return s ? atoi(s) : 0;
    }();
    P.split_min = split_env >= 32 ? split_env / 32 * 32 : 128;
    P.timeout_ticks = 20000000ull;  // 0.2 s
    const size_t lds = std::max(vte::decode_persistent_lds(H, F, qd), (size_t)P.r_red * nsl * 4);
    const int occ = vte::decode_persistent_occupancy(P, lds);
    REQUIRE(occ >= 1, "decode_step: the kernel does not fit on a CU (occupancy %d)", occ);
    e = vte::decode_persistent_launch(P, blocks, lds, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("decode_step: unsupported shape");
    if (e != hipSuccess) return hip_status(e, "vte_decode_step launch");
    // output norm + LM head over the last layer's output, as the graph path's
    e = vte::norm_mv(P.h_out, m->output_norm, m->eps, m->lm_head, m->fmt_lm, logits, true, nullptr, nullptr, 1.f, 1, H,
                     m->vocab, (hipStream_t)stream);
    if (e == hipErrorNotSupported) return fail("decode_step: the LM head does not fit the fused kernel");
    return hip_status(e, "vte_decode_step LM head launch");
}

int vte_decode_status(void* ws, int* flags) {
    REQUIRE(ws && flags, "decode_status: null pointer");
    uint32_t c[4];
    hipError_t e = hipMemcpy(c, ws, sizeof(c), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_status(e, "decode_status copy");
    *flags = (int)c[2];
    return 0;
}

// ------------------------------------------------------------------ batched persistent decode step

namespace {
struct PbLayout {
    size_t ctrl, layers, ll_h, ll_q, ll_kv, ll_att, ll_hm, ll_act, part, ll_dn, trace, total;
    int sl_sb, nsl;
};
PbLayout pb_layout(const vte_decode_model* m, int B) {
    PbLayout L;
    const size_t qd = (size_t)m->n_q * 128, kvd = (size_t)m->n_kv * 128, H = m->hidden, F = m->ffn;
    const int nsb = m->ffn / 256;
    L.sl_sb = std::max(1, (nsb + 7) / 8);  // about 8 slices of the ffn activations
    L.nsl = (nsb + L.sl_sb - 1) / L.sl_sb;
    size_t o = 0;
    L.ctrl = o; o = pd_align(o + 256);
    L.layers = o; o = pd_align(o + (size_t)m->n_layers * sizeof(vte_decode_layer));
    L.ll_h = o; o = pd_align(o + B * H * 4);
    L.ll_q = o; o = pd_align(o + B * qd * 4);
    L.ll_kv = o; o = pd_align(o + B * 2 * kvd * 4);
    L.ll_att = o; o = pd_align(o + B * qd * 4);
    L.ll_hm = o; o = pd_align(o + B * H * 4);
    L.ll_act = o; o = pd_align(o + B * F * 4);
    L.part = o; o = pd_align(o + (size_t)B * m->n_q * VTE_DECODE_MAX_SPLITS * 130 * 8);
    L.ll_dn = o; o = pd_align(o + (size_t)L.nsl * B * H * 8);
    // The kernel's staging reads whole rounds of 256 x 24 word pairs (48 KB)
    // past the end of a flagged input without a bounds test: every staged
    // buffer (ll_h, ll_att, ll_hm, ll_act) is followed by at least that much
    // workspace (the attention records alone hold >= 133 KB).
#ifdef VTE_PB_TRACE
    L.trace = o; o = pd_align(o + (size_t)1024 * m->n_layers * 16 * 4);
#else
    L.trace = 0;
#endif
    L.total = o;
    return L;
}
int pb_check_model(const vte_decode_model* m, int B, bool pointers = true) {
    REQUIRE(m != nullptr, "decode_batch: null model");
    REQUIRE(B >= 1 && B <= VTE_PB_MAX_B, "decode_batch: batch %d outside [1, %d]", B, VTE_PB_MAX_B);
    REQUIRE(m->n_layers >= 1 && m->n_layers <= 1024, "decode_batch: n_layers %d", m->n_layers);
    REQUIRE(m->head_dim == 128, "decode_batch: head_dim must be 128");
    REQUIRE(m->n_kv >= 1 && m->n_q % m->n_kv == 0 && m->n_q / m->n_kv <= 8, "decode_batch: n_q / n_kv must be <= 8");
    const int qd = m->n_q * 128;
    REQUIRE(m->hidden % 256 == 0 && m->hidden <= VTE_PB_MAX_K && qd % 256 == 0 && qd <= VTE_PB_MAX_K &&
                m->ffn % 256 == 0, "decode_batch: hidden and n_q*128 multiples of 256 up to %d, ffn a multiple of 256",
            VTE_PB_MAX_K);
    const PbLayout L = pb_layout(m, B);
    REQUIRE(L.sl_sb * 256 <= VTE_PB_MAX_K && L.nsl <= VTE_PB_MAX_SLICES, "decode_batch: ffn %d too long", m->ffn);
    REQUIRE(m->max_seq >= 1, "decode_batch: max_seq");
    REQUIRE(L.ll_dn - L.ll_act >= (size_t)B * m->ffn * 4 + 48 * 1024, "decode_batch: workspace tail");
    if (!pointers) return 0;
    REQUIRE(m->rope_cos && m->rope_sin, "decode_batch: null RoPE tables");
    return 0;
}
}  // namespace

long long vte_decode_batch_workspace_bytes(const vte_decode_model* m, int batch) {
    if (pb_check_model(m, batch, false)) return -1;
    return (long long)pb_layout(m, batch).total;
}

int vte_decode_batch_setup(const vte_decode_model* m, const vte_decode_layer* layers, int batch, void* ws,
                           long long ws_bytes, void* stream) {
    int rc = pb_check_model(m, batch);
    if (rc) return rc;
    REQUIRE(layers && ws, "decode_batch_setup: null pointer");
    REQUIRE(aligned(ws, 256), "decode_batch_setup: workspace must be 256-byte aligned");
    const PbLayout L = pb_layout(m, batch);
    REQUIRE(ws_bytes >= (long long)L.total, "decode_batch_setup: workspace %lld < %zu bytes", ws_bytes, L.total);
    for (int l = 0; l < m->n_layers; ++l) {
        const vte_decode_layer& y = layers[l];
        REQUIRE(y.wq && y.wk && y.wv && y.wo && y.w_gate && y.w_up && y.w_down && y.attn_norm && y.ffn_norm &&
                    y.k_cache && y.v_cache, "decode_batch_setup: layer %d: null pointer", l);
        const int f[6] = {y.fmt_q, y.fmt_k, y.fmt_v, y.fmt_o, y.fmt_gate_up, y.fmt_down};
        for (int i = 0; i < 6; ++i)
            REQUIRE(f[i] == 4 || f[i] == 6, "decode_batch_setup: layer %d: projections must be Q4_K or Q6_K", l);
        REQUIRE(aligned(y.wq, 16) && aligned(y.wk, 16) && aligned(y.wv, 16) && aligned(y.wo, 16) &&
                    aligned(y.w_gate, 16) && aligned(y.w_up, 16) && aligned(y.w_down, 16) &&
                    aligned(y.attn_norm, 16) && aligned(y.ffn_norm, 16) && aligned(y.k_cache, 16) &&
                    aligned(y.v_cache, 16), "decode_batch_setup: layer %d: 16-byte alignment", l);
    }
    hipStream_t st = (hipStream_t)stream;
    uint8_t* base = static_cast<uint8_t*>(ws);
    hipError_t e = hipMemsetAsync(base, 0, L.total, st);
    if (e != hipSuccess) return hip_status(e, "decode_batch_setup memset");
    const uint32_t ctrl[4] = {1u, 0u, 0u, 0u};  // epoch starts at 1: no tag matches the cleared words
    e = hipMemcpyAsync(base + L.ctrl, ctrl, sizeof(ctrl), hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + L.layers, layers, (size_t)m->n_layers * sizeof(vte_decode_layer),
                           hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return hip_status(e, "decode_batch_setup copy");
}

int vte_decode_batch_step(const vte_decode_model* m, void* ws, int batch, long long kv_batch_stride,
                          const int* kv_offset, const void* x, void* h_out, void* stream) {
    int rc = pb_check_model(m, batch);
    if (rc) return rc;
    REQUIRE(ws && kv_offset && x && h_out, "decode_batch_step: null pointer");
    REQUIRE(aligned(ws, 256) && aligned(x, 16) && aligned(h_out, 16), "decode_batch_step: alignment");
    REQUIRE(kv_batch_stride >= (long long)m->max_seq * m->n_kv * 128 || batch == 1,
            "decode_batch_step: kv_batch_stride %lld below one sequence's cache", kv_batch_stride);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    REQUIRE(dev >= 0 && dev < 64, "decode_batch_step: device %d", dev);
    if (g_pd_cus[dev] == 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_status(e, "hipDeviceGetAttribute");
        g_pd_cus[dev] = n;
    }
    const int blocks = g_pd_cus[dev];  // one 256-thread block per CU
    const PbLayout L = pb_layout(m, batch);
    const int H = m->hidden, qd = m->n_q * 128, kvd = m->n_kv * 128;
    // every q/k/v tile on its own block, the reduce outputs within one pass of the threads
    REQUIRE(qd / 16 + 2 * (kvd / 16) <= blocks, "decode_batch_step: %d q/k/v tiles exceed %d blocks",
            qd / 16 + 2 * (kvd / 16), blocks);
    REQUIRE((batch * H + blocks - 1) / blocks <= 256, "decode_batch_step: %d outputs per block in the reduce",
            (batch * H + blocks - 1) / blocks);
    uint8_t* base = static_cast<uint8_t*>(ws);
    VtePbPlan P{};
    P.layers = reinterpret_cast<const VtePdLayer*>(base + L.layers);
    P.n_layers = m->n_layers;
    P.hidden = H;
    P.ffn = m->ffn;
    P.n_q = m->n_q;
    P.n_kv = m->n_kv;
    P.B = batch;
    P.eps = m->eps;
    P.scale = 1.0f / sqrtf(128.0f);
    P.kv_offset = kv_offset;
    P.max_seq = m->max_seq;
    P.kv_batch_stride = kv_batch_stride;
    P.x = static_cast<const __half*>(x);
    P.rope_cos = static_cast<const __half*>(m->rope_cos);
    P.rope_sin = static_cast<const __half*>(m->rope_sin);
    P.h_out = static_cast<__half*>(h_out);
    P.ll_h = reinterpret_cast<uint32_t*>(base + L.ll_h);
    P.ll_q = reinterpret_cast<uint32_t*>(base + L.ll_q);
    P.ll_kv = reinterpret_cast<uint32_t*>(base + L.ll_kv);
    P.ll_att = reinterpret_cast<uint32_t*>(base + L.ll_att);
    P.ll_hm = reinterpret_cast<uint32_t*>(base + L.ll_hm);
    P.ll_act = reinterpret_cast<uint32_t*>(base + L.ll_act);
    P.part = reinterpret_cast<uint64_t*>(base + L.part);
    P.ll_dn = reinterpret_cast<uint64_t*>(base + L.ll_dn);
    P.ctrl = reinterpret_cast<uint32_t*>(base + L.ctrl);
    P.sl_sb = L.sl_sb;
    P.trace = L.trace ? reinterpret_cast<uint32_t*>(base + L.trace) : nullptr;
    P.split_min = 128;
    P.timeout_ticks = 20000000ull;  // 0.2 s
    const size_t lds = vte::decode_persistent_mm_lds(H, qd, L.sl_sb * 256);
    const int occ = vte::decode_persistent_mm_occupancy(lds);
    REQUIRE(occ >= 1, "decode_batch_step: the kernel does not fit on a CU (occupancy %d)", occ);
    e = vte::decode_persistent_mm_launch(P, blocks, lds, (hipStream_t)stream);
    return hip_status(e, "vte_decode_batch_step launch");
}
