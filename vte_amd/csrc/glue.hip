// Decode-step glue kernels (fp16 storage, fp32 math), gfx950.
//
// Reference contracts (same symbol names and argument lists, so a code object
// built from this file drops into hipModuleGetFunction lookups):
//   rmsnorm_kernel               vte/compiler/templates/rdna/rmsnorm.hip.template:6-117
//   rope_kernel                  vte/compiler/templates/rdna/rope.hip.template:17-137
//   swiglu_kernel                vte/compiler/templates/rdna/swiglu.hip.template:4-26
//   add_kernel                   vte/compiler/templates/rdna/add.hip.template:4-17
//   embedding_lookup_q6k_kernel  vte/compiler/templates/rdna/embedding_lookup_q6k.hip.template:17-58
// plus a top-k selector over fp32 logits for on-device sampling candidates.
#include "vte_common.h"

// ---------------------------------------------------------------------------
// RMSNorm: out = x * rsqrt(mean(x^2) + eps) * w.  grid (rows), block (256).
// Hidden sizes that are multiples of 8 use 16-byte loads.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rmsnorm_kernel(const __half* __restrict__ x,
                                                                 const __half* __restrict__ weight,
                                                                 __half* __restrict__ output, int hidden_size,
                                                                 float eps) {
    __shared__ float part[16];
    const int row = blockIdx.x, tid = threadIdx.x;
    const __half* xr = x + (size_t)row * hidden_size;
    __half* orow = output + (size_t)row * hidden_size;
    float ss = 0.f;
    const int nv = (hidden_size % 8 == 0) ? hidden_size / 8 : 0;
    for (int i = tid; i < nv; i += blockDim.x) {
        const uint4 v = reinterpret_cast<const uint4*>(xr)[i];
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = h2f_bits(w4[j]), b = h2f_bits(w4[j] >> 16);
            ss = fmaf(a, a, ss);
            ss = fmaf(b, b, ss);
        }
    }
    for (int i = nv * 8 + tid; i < hidden_size; i += blockDim.x) {
        const float a = __half2float(xr[i]);
        ss = fmaf(a, a, ss);
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    const int nw = (blockDim.x + 63) >> 6;
    for (int w = 0; w < nw; ++w) tot += part[w];
    const float inv = rsqrtf(tot / (float)hidden_size + eps);
    for (int i = tid; i < hidden_size; i += blockDim.x)
        orow[i] = __float2half(__half2float(xr[i]) * inv * __half2float(weight[i]));
}

// ---------------------------------------------------------------------------
// RoPE, in place on q [B][seq][n_q][hd] and k [B][seq][n_kv][hd] at position
// kv_offset[b] + token.  rope_type 0 = NEOX rotate-half (Qwen2), 1 = adjacent
// pairs, 2 = NEOX over the first rotary_dim channels.  Tables are fp16
// [pos][hd] (type 2: [pos][rotary_dim]), both halves duplicated
// (vte/compiler/rope_cache_builder.py:54-90).
// grid (ceil(seq*n_q*hd/256), B), block 256.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_pair(__half* v, int idx, int head_offset, int pos, const __half* cosc,
                                          const __half* sinc, int head_dim, int rope_type, int rotary_dim) {
    const int half_dim = head_dim / 2;
    if (rope_type == 1) {
        if ((head_offset & 1) == 0) {
            const int i = head_offset / 2;
            const float x0 = __half2float(v[idx]), x1 = __half2float(v[idx + 1]);
            const float c = __half2float(cosc[(size_t)pos * head_dim + i]);
            const float s = __half2float(sinc[(size_t)pos * head_dim + i]);
            v[idx] = __float2half(x0 * c - x1 * s);
            v[idx + 1] = __float2half(x0 * s + x1 * c);
        }
    } else if (rope_type == 2) {
        const int hr = rotary_dim / 2;
        if (head_offset < hr) {
            const float a = __half2float(v[idx]), b = __half2float(v[idx + hr]);
            const float c = __half2float(cosc[(size_t)pos * rotary_dim + head_offset]);
            const float s = __half2float(sinc[(size_t)pos * rotary_dim + head_offset]);
            v[idx] = __float2half(a * c - b * s);
            v[idx + hr] = __float2half(a * s + b * c);
        }
    } else if (head_offset < half_dim) {
        const float a = __half2float(v[idx]), b = __half2float(v[idx + half_dim]);
        const float c = __half2float(cosc[(size_t)pos * head_dim + head_offset]);
        const float s = __half2float(sinc[(size_t)pos * head_dim + head_offset]);
        v[idx] = __float2half(a * c - b * s);
        v[idx + half_dim] = __float2half(a * s + b * c);
    }
}

extern "C" __global__ __launch_bounds__(256) void rope_kernel(__half* __restrict__ q, __half* __restrict__ k,
                                                              const __half* __restrict__ cos_cache,
                                                              const __half* __restrict__ sin_cache, int seq_len,
                                                              int num_q_heads, int num_kv_heads, int head_dim,
                                                              const int* __restrict__ kv_cache_offset_ptr,
                                                              int rope_type, int rotary_dim) {
    const int b = blockIdx.y;
    const int nq = seq_len * num_q_heads * head_dim;
    const int nk = seq_len * num_kv_heads * head_dim;
    __half* qb = q + (size_t)b * nq;
    __half* kb = k + (size_t)b * nk;
    const int off = kv_cache_offset_ptr[b];
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < nq)
        rope_pair(qb, idx, idx % head_dim, off + idx / (num_q_heads * head_dim), cos_cache, sin_cache, head_dim,
                  rope_type, rotary_dim);
    if (idx < nk)
        rope_pair(kb, idx, idx % head_dim, off + idx / (num_kv_heads * head_dim), cos_cache, sin_cache,
                  head_dim, rope_type, rotary_dim);
}

// ---------------------------------------------------------------------------
// SwiGLU: out = silu(g) * u, silu(g) = g / (1 + exp(-g)).   grid ceil(n/256).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void swiglu_kernel(const __half* __restrict__ gate,
                                                                const __half* __restrict__ up,
                                                                __half* __restrict__ out, int total_elements) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_elements) return;
    const float g = __half2float(gate[i]);
    const float u = __half2float(up[i]);
    const float sig = 1.0f / (1.0f + expf(-g));
    out[i] = __float2half(g * sig * u);
}

// add: out = residual + scale * in.
extern "C" __global__ __launch_bounds__(256) void add_kernel(const __half* __restrict__ residual,
                                                             const __half* __restrict__ input,
                                                             __half* __restrict__ output, int n,
                                                             float residual_scale) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        output[i] = __float2half(__half2float(residual[i]) + residual_scale * __half2float(input[i]));
}

// ---------------------------------------------------------------------------
// Embedding lookup from a raw Q6_K table: out[s][d] = fp16(dequant(W[tok[s]])[d] * scale).
// grid ceil(seq*hidden/256), block 256.  Same rounding as the Q6_K dequantiser.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void embedding_lookup_q6k_kernel(
    const int* __restrict__ token_ids, const void* __restrict__ embed_weight, __half* __restrict__ output,
    int seq_len, int hidden_size, float embedding_scale) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq_len * hidden_size) return;
    const int s = idx / hidden_size, dcol = idx % hidden_size;
    const int tok = token_ids[s];
    const uint8_t* blk = (const uint8_t*)embed_weight + ((size_t)tok * (hidden_size / QK_K) + dcol / QK_K) * Q6K_BYTES;
    const int e = dcol % QK_K;
    const int half = e >> 7, g = (e >> 5) & 3, l = e & 31;
    const uint8_t qlb = blk[64 * half + l + ((g & 1) ? 32 : 0)];
    const int nib = (g < 2) ? (qlb & 0x0F) : (qlb >> 4);
    const int q = (nib | (((blk[128 + 32 * half + l] >> (2 * g)) & 3) << 4)) - 32;
    const int8_t sc = (int8_t)blk[192 + 8 * half + (l >> 4) + 2 * g];
    const float d = h2f_bits(blk[208] | (blk[209] << 8));
    const float w = __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
    output[idx] = __float2half(w * embedding_scale);
}

// ---------------------------------------------------------------------------
// Top-k over fp32 logits, k <= 64, exact, ordered by (value desc, index asc):
// the order np.lexsort((index, -value)) gives.  Two launches:
//  1. grid (TOPK_P, rows), 4 waves per block: each wave keeps the top 64 of its
//     slice as a bitonic-sorted 64-lane list, merging in one 64-element group
//     at a time (sort the group, take max(list[l], group[63 - l]) which is
//     bitonic and holds the top 64 of the union, then a bitonic merge);
//  2. one block per row merges the TOPK_P * 4 lists the same way and writes
//     the first k entries.
// Padding entries are (-inf, INT_MAX) so they rank after every real logit.
// ---------------------------------------------------------------------------
#define TOPK_P 64
#define TOPK_WAVES 4

__device__ __forceinline__ bool tk_better(float a, int ia, float b, int ib) {
    return a > b || (a == b && ia < ib);
}

// One compare-exchange stage of a bitonic network across the wave.
__device__ __forceinline__ void tk_stage(float& v, int& ix, int lane, int stride, bool desc) {
    const float ov = __shfl_xor(v, stride, 64);
    const int oi = __shfl_xor(ix, stride, 64);
    const bool lower = (lane & stride) == 0;
    const bool ob = tk_better(ov, oi, v, ix);
    if ((lower == desc) ? ob : (!ob && !(ov == v && oi == ix))) { v = ov; ix = oi; }
}

__device__ __forceinline__ void tk_sort64(float& v, int& ix, int lane) {
    for (int size = 2; size <= 64; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) tk_stage(v, ix, lane, stride, (lane & size) == 0);
}

// (v, ix): sorted top list; (gv, gi): another sorted list -> top 64 of the union, sorted.
__device__ __forceinline__ void tk_merge64(float& v, int& ix, float gv, int gi, int lane) {
    const float rv = __shfl(gv, 63 - lane, 64);
    const int ri = __shfl(gi, 63 - lane, 64);
    if (tk_better(rv, ri, v, ix)) { v = rv; ix = ri; }
    for (int stride = 32; stride > 0; stride >>= 1) tk_stage(v, ix, lane, stride, true);
}

__global__ __launch_bounds__(64 * TOPK_WAVES) void topk_partial_kernel(const float* __restrict__ logits, int vocab,
                                                                         float* __restrict__ sv, int* __restrict__ si) {
    const int row = blockIdx.y, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int gw = blockIdx.x * TOPK_WAVES + wv, nw = TOPK_P * TOPK_WAVES;
    const int per = ((vocab + nw - 1) / nw + 63) & ~63;
    const int lo = gw * per, hi = min(lo + per, vocab);
    const float* r = logits + (size_t)row * vocab;
    float v = -INFINITY;
    int ix = 0x7fffffff;
    for (int base = lo; base < hi; base += 64) {
        const int i = base + lane;
        float gv = (i < hi) ? r[i] : -INFINITY;
        int gi = (i < hi) ? i : 0x7fffffff;
        tk_sort64(gv, gi, lane);
        if (base == lo) { v = gv; ix = gi; }
        else tk_merge64(v, ix, gv, gi, lane);
    }
    const size_t o = ((size_t)row * nw + gw) * 64 + lane;
    sv[o] = v;
    si[o] = ix;
}

__global__ __launch_bounds__(64 * TOPK_WAVES) void topk_final_kernel(const float* __restrict__ sv,
                                                                       const int* __restrict__ si, int k,
                                                                       float* __restrict__ out_val,
                                                                       int* __restrict__ out_idx) {
    __shared__ float lv[TOPK_WAVES][64];
    __shared__ int li[TOPK_WAVES][64];
    const int row = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nl = TOPK_P * TOPK_WAVES;
    const size_t base = (size_t)row * nl * 64;
    float v = sv[base + (size_t)wv * 64 + lane];
    int ix = si[base + (size_t)wv * 64 + lane];
    for (int l = wv + TOPK_WAVES; l < nl; l += TOPK_WAVES)
        tk_merge64(v, ix, sv[base + (size_t)l * 64 + lane], si[base + (size_t)l * 64 + lane], lane);
    lv[wv][lane] = v;
    li[wv][lane] = ix;
    __syncthreads();
    if (wv == 0) {
        for (int w = 1; w < TOPK_WAVES; ++w) tk_merge64(v, ix, lv[w][lane], li[w][lane], lane);
        if (lane < k) {
            out_val[(size_t)row * k + lane] = v;
            out_idx[(size_t)row * k + lane] = ix;
        }
    }
}

// ---------------------------------------------------------------------------
// Seeded device-side fill of fp16 memory with scale * N(0,1) (counter-based
// splitmix64 hash + Box-Muller).  Used to lay down synthetic KV prefixes of
// up to gigabytes without a host round trip; not part of any parity path.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_f16_kernel(__half* __restrict__ dst, long long n,
                                                              unsigned long long seed, float scale) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t h = splitmix64(seed * 0x2545F4914F6CDD1Dull + (uint64_t)i);
    const float u1 = ((float)((h >> 40) & 0xFFFFFF) + 1.0f) * (1.0f / 16777217.0f);
    const float u2 = (float)((h >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    dst[i] = __float2half(scale * r * cosf(6.28318530718f * u2));
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace vte {

hipError_t fill_normal_f16(void* dst, long long n, unsigned long long seed, float scale, hipStream_t st) {
    hipLaunchKernelGGL(fill_normal_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (__half*)dst, n,
                       seed, scale);
    return hipGetLastError();
}

hipError_t rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, st, (const __half*)x, (const __half*)w,
                       (__half*)out, hidden, eps);
    return hipGetLastError();
}

hipError_t rope(void* q, void* k, const void* cosc, const void* sinc, int B, int seq_len, int n_q, int n_kv,
                int head_dim, const int* kv_offset, int rope_type, int rotary_dim, hipStream_t st) {
    const int n = seq_len * n_q * head_dim;
    hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256, B), dim3(256), 0, st, (__half*)q, (__half*)k,
                       (const __half*)cosc, (const __half*)sinc, seq_len, n_q, n_kv, head_dim, kv_offset,
                       rope_type, rotary_dim);
    return hipGetLastError();
}

hipError_t swiglu(const void* g, const void* u, void* out, int n, hipStream_t st) {
    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, st, (const __half*)g, (const __half*)u,
                       (__half*)out, n);
    return hipGetLastError();
}

hipError_t add(const void* r, const void* in, void* out, int n, float scale, hipStream_t st) {
    hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, st, (const __half*)r, (const __half*)in,
                       (__half*)out, n, scale);
    return hipGetLastError();
}

hipError_t embedding_q6k(const int* tokens, const void* table, void* out, int n_tokens, int hidden, float scale,
                         hipStream_t st) {
    const int n = n_tokens * hidden;
    hipLaunchKernelGGL(embedding_lookup_q6k_kernel, dim3((n + 255) / 256), dim3(256), 0, st, tokens, table,
                       (__half*)out, n_tokens, hidden, scale);
    return hipGetLastError();
}

size_t topk_scratch_bytes(int rows) { return (size_t)rows * TOPK_P * TOPK_WAVES * 64 * (sizeof(float) + sizeof(int)); }

hipError_t topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* scratch,
                hipStream_t st) {
    float* sv = (float*)scratch;
    int* si = (int*)((char*)scratch + (size_t)rows * TOPK_P * TOPK_WAVES * 64 * sizeof(float));
    hipLaunchKernelGGL(topk_partial_kernel, dim3(TOPK_P, rows), dim3(64 * TOPK_WAVES), 0, st, logits, vocab, sv, si);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(topk_final_kernel, dim3(rows), dim3(64 * TOPK_WAVES), 0, st, sv, si, k, out_val, out_idx);
    return hipGetLastError();
}

}  // namespace vte
