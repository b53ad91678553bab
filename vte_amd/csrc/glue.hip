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
// Top-k over fp32 logits (one 1024-thread block per row).  Exact radix select
// on order-preserving 32-bit keys (4 passes of 8 bits), then a gather that
// keeps every key above the threshold and the lowest-index ties at it, then a
// bitonic sort (value descending, index ascending).  k <= 64.
// out_val / out_idx: [rows][k].
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f2key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(1024) void topk_rows_kernel(const float* __restrict__ logits, int vocab, int k,
                                                         float* __restrict__ out_val, int* __restrict__ out_idx) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel_prefix, sel_need;
    __shared__ int wave_cnt[16];
    __shared__ int n_above;
    __shared__ float cand_v[64];
    __shared__ int cand_i[64];
    const float* row = logits + (size_t)blockIdx.x * vocab;
    const int tid = threadIdx.x;
    if (tid == 0) { sel_prefix = 0; sel_need = (uint32_t)k; n_above = 0; }
    if (tid < 64) { cand_v[tid] = -INFINITY; cand_i[tid] = 0x7fffffff; }
    __syncthreads();
    // radix select of the k-th largest key
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 256; i += blockDim.x) hist[i] = 0;
        __syncthreads();
        const uint32_t prefix = sel_prefix;
        const uint32_t pmask = (pass == 0) ? 0u : (0xFFFFFFFFu << (shift + 8));
        for (int i = tid; i < vocab; i += blockDim.x) {
            const uint32_t key = f2key(row[i]);
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t need = sel_need, cum = 0;
            int bin = 255;
            for (; bin > 0; --bin) {
                if (cum + hist[bin] >= need) break;
                cum += hist[bin];
            }
            sel_prefix = prefix | ((uint32_t)bin << shift);
            sel_need = need - cum;
        }
        __syncthreads();
    }
    const uint32_t thr = sel_prefix;   // exact key of the k-th largest value
    const int ties_needed = (int)sel_need;
    // gather: keys above thr (fewer than k of them) go in any order; ties at thr
    // are ranked by index through a block-wide scan over contiguous ranges.
    const int per = (vocab + blockDim.x - 1) / blockDim.x;
    const int lo = tid * per, hi = min(lo + per, vocab);
    int my_ties = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t key = f2key(row[i]);
        if (key > thr) {
            const int slot = atomicAdd(&n_above, 1);
            cand_v[slot] = row[i];
            cand_i[slot] = i;
        } else if (key == thr) {
            ++my_ties;
        }
    }
    // exclusive scan of my_ties across the block (wave scan + wave totals)
    int incl = my_ties;
    const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    if (lane == 63) wave_cnt[wv] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += wave_cnt[w];
    int rank = base + incl - my_ties;
    const int above = k - ties_needed;
    if (my_ties > 0 && rank < ties_needed) {
        for (int i = lo; i < hi && rank < ties_needed; ++i) {
            if (f2key(row[i]) == thr) {
                cand_v[above + rank] = row[i];
                cand_i[above + rank] = i;
                ++rank;
            }
        }
    }
    __syncthreads();
    // bitonic sort of 64 candidates in wave 0: value desc, index asc
    if (tid < 64) {
        float v = cand_v[tid];
        int ix = cand_i[tid];
        for (int size = 2; size <= 64; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const float ov = __shfl_xor(v, stride, 64);
                const int oi = __shfl_xor(ix, stride, 64);
                const bool up = ((tid & size) == 0);          // block sorted "descending-first"
                const bool lower = ((tid & stride) == 0);
                const bool other_first = (ov > v) || (ov == v && oi < ix);
                const bool take = (lower == up) ? other_first : !other_first;
                if (take) { v = ov; ix = oi; }
            }
        }
        if (tid < k) {
            out_val[(size_t)blockIdx.x * k + tid] = v;
            out_idx[(size_t)blockIdx.x * k + tid] = ix;
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

hipError_t topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, hipStream_t st) {
    hipLaunchKernelGGL(topk_rows_kernel, dim3(rows), dim3(1024), 0, st, logits, vocab, k, out_val, out_idx);
    return hipGetLastError();
}

}  // namespace vte
