// Decode-step glue kernels (fp16 storage, fp32 math), gfx950.
//
// Reference contracts (same symbol names and argument lists, so a code object
// built from this file drops into hipModuleGetFunction lookups):
//   rmsnorm_kernel               vte/compiler/templates/rdna/rmsnorm.hip.template:6-117
//   rope_kernel                  vte/compiler/templates/rdna/rope.hip.template:17-137
//   swiglu_kernel                vte/compiler/templates/rdna/swiglu.hip.template:4-26
//   add_kernel                   vte/compiler/templates/rdna/add.hip.template:4-17
//   embedding_lookup_q6k_kernel  vte/compiler/templates/rdna/embedding_lookup_q6k.hip.template:17-58
//   embedding_lookup_q4k_kernel  vte/compiler/templates/rdna/embedding_lookup_q4k.hip.template:26-75
//   embedding_lookup_q8_0_kernel vte/compiler/templates/rdna/embedding_lookup_q8_0.hip.template:15-46
// plus a top-k selector over fp32 logits for on-device sampling candidates.
#include <mutex>

#include "quant.h"

// ---------------------------------------------------------------------------
// RMSNorm: out = x * rsqrt(mean(x^2) + eps) * w.  grid (rows), block (256).
// Hidden sizes that are multiples of 8 and at most 8 * 4 * 256 keep their
// 16-byte chunks (and the matching weight chunks, requested together) in
// registers, so a row costs one memory round trip; other sizes take the
// element loop.
// ---------------------------------------------------------------------------
#define RMS_CH 4  // 16-byte chunks per thread on the register path
extern "C" __global__ __launch_bounds__(256) void rmsnorm_kernel(const __half* __restrict__ x,
                                                                 const __half* __restrict__ weight,
                                                                 __half* __restrict__ output, int hidden_size,
                                                                 float eps) {
    __shared__ float part[16];
    const int row = blockIdx.x, tid = threadIdx.x;
    const __half* xr = x + (size_t)row * hidden_size;
    __half* orow = output + (size_t)row * hidden_size;
    const int nv = hidden_size / 8;
    const bool regs = hidden_size % 8 == 0 && nv <= RMS_CH * 256;
    uint4 xv[RMS_CH], wv[RMS_CH];
    float ss = 0.f;
    if (regs) {
#pragma unroll
        for (int j = 0; j < RMS_CH; ++j) {
            const int c = min(tid + 256 * j, nv - 1);
            xv[j] = reinterpret_cast<const uint4*>(xr)[c];
            wv[j] = reinterpret_cast<const uint4*>(weight)[c];
        }
#pragma unroll
        for (int j = 0; j < RMS_CH; ++j) {
            if (tid + 256 * j >= nv) continue;
            const uint32_t w4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = h2f_bits(w4[i]), b = h2f_bits(w4[i] >> 16);
                ss = fmaf(a, a, ss);
                ss = fmaf(b, b, ss);
            }
        }
    } else {
        for (int i = tid; i < hidden_size; i += blockDim.x) {
            const float a = __half2float(xr[i]);
            ss = fmaf(a, a, ss);
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    const int nw = (blockDim.x + 63) >> 6;
    for (int w = 0; w < nw; ++w) tot += part[w];
    const float inv = rsqrtf(tot / (float)hidden_size + eps);
    if (regs) {
#pragma unroll
        for (int j = 0; j < RMS_CH; ++j) {
            const int c = tid + 256 * j;
            if (c >= nv) continue;
            const uint32_t xa[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const uint32_t wa[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const __half lo = __float2half(h2f_bits(xa[i]) * inv * h2f_bits(wa[i]));
                const __half hi = __float2half(h2f_bits(xa[i] >> 16) * inv * h2f_bits(wa[i] >> 16));
                o[i] = (uint32_t)__half_as_ushort(lo) | ((uint32_t)__half_as_ushort(hi) << 16);
            }
            reinterpret_cast<uint4*>(orow)[c] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else {
        for (int i = tid; i < hidden_size; i += blockDim.x)
            orow[i] = __float2half(__half2float(xr[i]) * inv * __half2float(weight[i]));
    }
}

// ---------------------------------------------------------------------------
// Residual add of split-K partial sums, then RMSNorm (grid rows, block 256):
//   x_out = fp16(x + sum_s part[s])        (the projection + residual store)
//   xn    = fp16(x_out * rsqrt(mean(x_out^2) + eps) * w)
// part is [n_parts][rows][hidden] fp32, summed in split order.  The sums
// replace the residual epilogue of the projection and the following RMSNorm
// node (reference: add_kernel, add.hip.template:4-17, then rmsnorm.hip.template:6-117),
// one launch for both.  hidden % 8 == 0 and hidden <= 8 * 4 * 256;
// x_out may alias x (each thread reads its chunks before writing them).
// ---------------------------------------------------------------------------
#define ADDN_MAX_PARTS 8
template <int CH>  // 16-byte chunks per thread: ceil(hidden / 8 / 256)
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const __half* x,
                                                                     const float* __restrict__ part, int n_parts,
                                                                     const __half* __restrict__ weight,
                                                                     __half* x_out, __half* __restrict__ xn,
                                                                     int rows, int hidden, float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int nv = hidden / 8;
    const size_t ro = (size_t)row * hidden;
    const size_t ps = (size_t)rows * hidden;
    uint4 xv[CH], wv[CH];
    float acc[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int c = min(tid + 256 * j, nv - 1);
        xv[j] = reinterpret_cast<const uint4*>(x + ro)[c];
        wv[j] = reinterpret_cast<const uint4*>(weight)[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    }
    // CH == 1: every split's loads are issued unconditionally (clamped split
    // index, masked add), so they all travel in one memory round trip
#pragma unroll
    for (int s = 0; s < ADDN_MAX_PARTS; ++s) {
        if (CH > 1 && s >= n_parts) break;
        const bool use = s < n_parts;
        const float* pr = part + min(s, n_parts - 1) * ps + ro;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int c = min(tid + 256 * j, nv - 1);
            const float4 a = reinterpret_cast<const float4*>(pr)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(pr)[2 * c + 1];
            acc[j][0] += use ? a.x : 0.f; acc[j][1] += use ? a.y : 0.f;
            acc[j][2] += use ? a.z : 0.f; acc[j][3] += use ? a.w : 0.f;
            acc[j][4] += use ? b.x : 0.f; acc[j][5] += use ? b.y : 0.f;
            acc[j][6] += use ? b.z : 0.f; acc[j][7] += use ? b.w : 0.f;
        }
    }
    float ss = 0.f;
    uint32_t xo[CH][4];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const uint32_t w4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const __half lo = __float2half(acc[j][2 * i] + h2f_bits(w4[i]));
            const __half hi = __float2half(acc[j][2 * i + 1] + h2f_bits(w4[i] >> 16));
            xo[j][i] = (uint32_t)__half_as_ushort(lo) | ((uint32_t)__half_as_ushort(hi) << 16);
            const float a = __half2float(lo), b = __half2float(hi);
            if (tid + 256 * j < nv) {
                ss = fmaf(a, a, ss);
                ss = fmaf(b, b, ss);
            }
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float inv = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)hidden + eps);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int c = tid + 256 * j;
        if (c >= nv) continue;
        const uint32_t wa[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const __half lo = __float2half(h2f_bits(xo[j][i]) * inv * h2f_bits(wa[i]));
            const __half hi = __float2half(h2f_bits(xo[j][i] >> 16) * inv * h2f_bits(wa[i] >> 16));
            o[i] = (uint32_t)__half_as_ushort(lo) | ((uint32_t)__half_as_ushort(hi) << 16);
        }
        reinterpret_cast<uint4*>(x_out + ro)[c] = make_uint4(xo[j][0], xo[j][1], xo[j][2], xo[j][3]);
        reinterpret_cast<uint4*>(xn + ro)[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
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
// Embedding lookup from a raw quantised table (the weights stay in their GGUF
// blocks; only the looked-up rows are dequantised):
//   out[s][d] = fp16(dequant(W[tok[s]])[d] * scale),
// dequant with the exact dequantiser's rounding.  grid ceil(seq*hidden/256),
// block 256, one element per thread (a few KB per token: off the hot path).
// ---------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ void embedding_elem(const int* __restrict__ token_ids, const void* __restrict__ table,
                                               __half* __restrict__ output, int seq_len, int hidden, float scale) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq_len * hidden) return;
    const int s = idx / hidden, dcol = idx % hidden;
    const size_t tok = (size_t)token_ids[s];
    constexpr int QB = FMT == 8 ? QK8_0 : QK_K;
    constexpr int BYTES = FMT == 4 ? Q4K_BYTES : FMT == 6 ? Q6K_BYTES : Q80_BYTES;
    const uint8_t* blk = (const uint8_t*)table + (tok * (hidden / QB) + dcol / QB) * BYTES;
    const int e = dcol % QB;
    const float w = FMT == 4 ? q4k_elem_exact(blk, e) : FMT == 6 ? q6k_elem_exact(blk, e) : q80_elem_exact(blk, e);
    float v = __fmul_rn(w, scale);
    // keep the product and the fp16 rounding apart: fused into one mixed
    // fma with a +0 addend they would turn a -0 product into +0
    asm volatile("" : "+v"(v));
    output[idx] = __float2half(v);
}

// embedding_lookup_q6k.hip.template:17-58 (Qwen2.5-1.5B: tied to the LM head)
extern "C" __global__ __launch_bounds__(256) void embedding_lookup_q6k_kernel(
    const int* __restrict__ token_ids, const void* __restrict__ embed_weight, __half* __restrict__ output,
    int seq_len, int hidden_size, float embedding_scale) {
    embedding_elem<6>(token_ids, embed_weight, output, seq_len, hidden_size, embedding_scale);
}
// embedding_lookup_q4k.hip.template:26-75 (Qwen2.5-7B: untied, Q4_K table)
extern "C" __global__ __launch_bounds__(256) void embedding_lookup_q4k_kernel(
    const int* __restrict__ token_ids, const void* __restrict__ embed_weight, __half* __restrict__ output,
    int seq_len, int hidden_size, float embedding_scale) {
    embedding_elem<4>(token_ids, embed_weight, output, seq_len, hidden_size, embedding_scale);
}
// embedding_lookup_q8_0.hip.template:15-46 (tied Q8_0 tables; scale 12 for Granite)
extern "C" __global__ __launch_bounds__(256) void embedding_lookup_q8_0_kernel(
    const int* __restrict__ token_ids, const void* __restrict__ embed_weight, __half* __restrict__ output,
    int seq_len, int hidden_size, float embedding_scale) {
    embedding_elem<8>(token_ids, embed_weight, output, seq_len, hidden_size, embedding_scale);
}

// ---------------------------------------------------------------------------
// Top-k over fp32 logits, k <= 64, exact, ordered by (value desc, index asc):
// the order np.lexsort((index, -value)) gives.  Two launches:
//  1. grid (TOPK_P, rows): each block takes a slice (at most TOPK_SLICE
//     logits) into registers, 16 per thread.  T, the smallest of the four
//     waves' ceil(k/4)-th largest per-thread maxima, has at least k entries
//     >= T in the slice, so the slice's top k are among the entries >= T;
//     when those number at most TOPK_CAP they are the block's candidates.
//     Otherwise (heavy ties) the block
//     selects its 64 best exactly by radix selection in LDS (11/11/10-bit
//     digit histograms) and keeps the lowest-indexed ties.
//  2. one block per row thresholds the <= TOPK_P * TOPK_CAP candidates the same
//     way; when at most 256 survive, each survivor's rank is the number of
//     survivors ordered before it, else the exact radix selection runs on all
//     candidates.
// Keys map fp32 to an order-preserving uint32 (-0.0 taken as +0.0, as the
// reference's comparison does).
// ---------------------------------------------------------------------------
#define TOPK_P 64
#define TOPK_SLICE 4096
#define TOPK_CAP 128  // candidate slots per slice
#define TOPK_THREADS 256
#define TOPK_BINS 2048

__device__ __forceinline__ uint32_t tk_key(float v) {
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float tk_val(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Block-wide exclusive scan of one int per thread (TOPK_THREADS threads).
__device__ __forceinline__ int tk_excl_scan(int v, int* wsum, int& total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    int base = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < TOPK_THREADS / 64; ++w) {
        base += (w < wv) ? wsum[w] : 0;
        total += wsum[w];
    }
    __syncthreads();
    return base + x - v;
}

struct TkShared {
    int hist[TOPK_BINS];
    int wsum[TOPK_THREADS / 64];
    int sel_digit, sel_need;
};

// Key of rank `need` (1 = largest) among keys[0..n): returns it and the number
// of entries equal to it that belong to the top `need` (in index order).
__device__ uint32_t tk_radix_select(const uint32_t* keys, int n, int need, TkShared& sh, int& need_eq) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0, mask = 0;
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        const int shift = shifts[r], nb = 1 << widths[r];
        for (int i = tid; i < nb; i += TOPK_THREADS) sh.hist[i] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += TOPK_THREADS) {
            const uint32_t k = keys[i];
            if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & (nb - 1)], 1);
        }
        __syncthreads();
        if (tid < 64) {
            // lane l owns nb/64 consecutive bins, lanes ordered from the top digit down
            const int per = nb >> 6;
            const int top = nb - 1 - lane * per;
            int s = 0;
            for (int j = 0; j < per; ++j) s += sh.hist[top - j];
            int incl = s;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (lane >= o) incl += y;
            }
            const int excl = incl - s;
            if (excl < need && need <= incl) {  // exactly one lane
                int c = excl;
                for (int j = 0; j < per; ++j) {
                    const int h = sh.hist[top - j];
                    if (need <= c + h) {
                        sh.sel_digit = top - j;
                        sh.sel_need = need - c;
                        break;
                    }
                    c += h;
                }
            }
        }
        __syncthreads();
        prefix |= (uint32_t)sh.sel_digit << shift;
        mask |= (uint32_t)(nb - 1) << shift;
        need = sh.sel_need;
        __syncthreads();
    }
    need_eq = need;
    return prefix;
}

// Keep keys[i] > T plus the first need_eq entries equal to T (positions in
// ascending order); returns the number kept (= min(64, n) by construction)
// and writes the kept positions, in order, to out_pos.
__device__ int tk_compact(const uint32_t* keys, int n, uint32_t T, int need_eq, int* out_pos, TkShared& sh) {
    const int tid = threadIdx.x;
    const int per = (n + TOPK_THREADS - 1) / TOPK_THREADS;
    const int lo = min(n, tid * per), hi = min(n, lo + per);
    int eq = 0;
    for (int i = lo; i < hi; ++i) eq += keys[i] == T;
    int tot;
    const int eq_before = tk_excl_scan(eq, sh.wsum, tot);
    int keep = 0, e = eq_before;
    for (int i = lo; i < hi; ++i) {
        const uint32_t k = keys[i];
        if (k > T) ++keep;
        else if (k == T) { keep += e < need_eq; ++e; }
    }
    const int base = tk_excl_scan(keep, sh.wsum, tot);
    int o = base;
    e = eq_before;
    for (int i = lo; i < hi; ++i) {
        const uint32_t k = keys[i];
        bool take = k > T;
        if (k == T) { take = e < need_eq; ++e; }
        if (take) out_pos[o++] = i;
    }
    __syncthreads();
    return tot;
}

// A candidate in one 8-byte word: key in the high half, index in the low half.
__device__ __forceinline__ uint64_t tk_pack(uint32_t key, int idx) {
    return ((uint64_t)key << 32) | (uint32_t)idx;
}

// Output order: a before b when its key is larger, or equal with a smaller index.
__device__ __forceinline__ bool tk_before(uint32_t a, int ia, uint32_t b, int ib) {
    return a > b || (a == b && ia < ib);
}

// r-th largest (1-based) of the wave's 64 values, by deciding its bits from
// the top: the largest t with #{v >= t} >= r.  Ballots and scalar popcounts.
__device__ __forceinline__ uint32_t tk_wave_kth(uint32_t v, int r) {
    uint32_t t = 0;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t trial = t | (1u << b);
        if (__popcll(__ballot(v >= trial)) >= r) t = trial;
    }
    return t;
}

// Threshold from the per-thread values `tm` (thread maxima): the smallest of
// the four waves' ceil(kth/4)-th largest, so at least kth values are >= it.
// Ends with a barrier.
__device__ __forceinline__ uint32_t tk_block_threshold(uint32_t tm, int kth, uint32_t* wt) {
    const uint32_t t = tk_wave_kth(tm, (kth + 3) >> 2);
    if ((threadIdx.x & 63) == 0) wt[threadIdx.x >> 6] = t;
    __syncthreads();
    return min(min(wt[0], wt[1]), min(wt[2], wt[3]));
}

#define TKR (TOPK_SLICE / TOPK_THREADS)  // slice entries per thread

// Exclusion list of a row (sorted token ids, the repetition window of the
// sampler): ids [rows][max_excl], counts [rows] in device memory so a captured
// graph reads the values staged before each replay.  Excluded entries take key
// 0 (below every finite and infinite logit) in the selection, and the block
// whose slice holds an excluded id writes that id's exact logit to
// gathered[row][i] (topk_reduce_greedy.hip.template:52-83 does the same for its
// per-thread maxima: the penalty only lowers logits, so the best tokens after
// it are the best non-excluded ones or excluded ones at their exact values).
struct TkExclude {
    const int* ids;
    const int* cnt;   // null: no exclusion
    int max_excl;
    float* gathered;
};

__global__ __launch_bounds__(TOPK_THREADS) void topk_partial_kernel(const float* __restrict__ logits, int vocab,
                                                                      int slice, int k,
                                                                      uint64_t* __restrict__ cand,
                                                                      int* __restrict__ cand_cnt, TkExclude ex) {
    __shared__ uint32_t keys[TOPK_SLICE];
    __shared__ int pos[64];
    __shared__ TkShared sh;
    __shared__ uint32_t wt[TOPK_THREADS / 64];
    __shared__ uint32_t xmask[TOPK_SLICE / 32];
    const int row = blockIdx.y, p = blockIdx.x, tid = threadIdx.x;
    const int lo = p * slice, n = max(0, min(slice, vocab - lo));
    const float* r = logits + (size_t)row * vocab + lo;
    // entry j * 256 + tid of the slice in register j (all loads issued at once)
    uint32_t kr[TKR];
    float v[TKR];
#pragma unroll
    for (int j = 0; j < TKR; ++j) {
        const int i = j * TOPK_THREADS + tid;
        v[j] = r[i < n ? i : 0];
    }
    const int n_ex = ex.cnt != nullptr ? min(ex.cnt[row], ex.max_excl) : 0;
    if (n_ex > 0) {  // uniform per block: mark the slice's excluded entries, gather their logits
        for (int w = tid; w < TOPK_SLICE / 32; w += TOPK_THREADS) xmask[w] = 0u;
        __syncthreads();
        const int* ids = ex.ids + (size_t)row * ex.max_excl;
        for (int i = tid; i < n_ex; i += TOPK_THREADS) {
            const int id = ids[i];
            if (id >= lo && id < lo + n) {
                atomicOr(&xmask[(id - lo) >> 5], 1u << ((id - lo) & 31));
                ex.gathered[(size_t)row * ex.max_excl + i] = r[id - lo];
            }
        }
        __syncthreads();
    }
    uint32_t tm = 0;
#pragma unroll
    for (int j = 0; j < TKR; ++j) {
        const int i = j * TOPK_THREADS + tid;
        const bool xd = n_ex > 0 && ((xmask[i >> 5] >> (i & 31)) & 1u);
        const bool ok = i < n;
        kr[j] = ok && !xd ? tk_key(v[j]) : 0u;
        tm = ok ? max(tm, kr[j]) : tm;
    }
    const size_t o = ((size_t)row * gridDim.x + p) * TOPK_CAP;
    if (n <= 64) {
        if (tid < n) cand[o + tid] = tk_pack(kr[0], lo + tid);
        if (tid == 0) cand_cnt[(size_t)row * gridDim.x + p] = n;
        return;
    }
    // n > 64 >= k: every wave's ceil(k/4) largest maxima are entries' keys
    const uint32_t T = tk_block_threshold(tm, k, wt);
    int c = 0;
#pragma unroll
    for (int j = 0; j < TKR; ++j) c += (j * TOPK_THREADS + tid < n && kr[j] >= T) ? 1 : 0;
    int total;
    int base = tk_excl_scan(c, sh.wsum, total);
    if (total <= TOPK_CAP) {
#pragma unroll
        for (int j = 0; j < TKR; ++j) {
            const int i = j * TOPK_THREADS + tid;
            if (i < n && kr[j] >= T) {
                cand[o + base] = tk_pack(kr[j], lo + i);
                ++base;
            }
        }
        if (tid == 0) cand_cnt[(size_t)row * gridDim.x + p] = total;
        return;
    }
    // many entries tie at the top: exact selection of the slice's best 64
#pragma unroll
    for (int j = 0; j < TKR; ++j) {
        const int i = j * TOPK_THREADS + tid;
        if (i < n) keys[i] = kr[j];
    }
    __syncthreads();
    int need_eq;
    const uint32_t T64 = tk_radix_select(keys, n, 64, sh, need_eq);
    const int kept = tk_compact(keys, n, T64, need_eq, pos, sh);
    if (tid < kept) cand[o + tid] = tk_pack(keys[pos[tid]], lo + pos[tid]);
    if (tid == 0) cand_cnt[(size_t)row * gridDim.x + p] = kept;
}

// Bitonic network over 64 lanes on (key desc, index asc).
__device__ __forceinline__ void tk_sort64(uint32_t& k, int& ix, int lane) {
    for (int size = 2; size <= 64; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t ok = __shfl_xor(k, stride, 64);
            const int oi = __shfl_xor(ix, stride, 64);
            const bool lower = (lane & stride) == 0;
            const bool desc = (lane & size) == 0;
            const bool other_first = tk_before(ok, oi, k, ix);
            if ((lower == desc) == other_first) { k = ok; ix = oi; }
        }
}

__global__ __launch_bounds__(TOPK_THREADS) void topk_final_kernel(const uint64_t* __restrict__ cand,
                                                                    const int* __restrict__ cand_cnt, int P, int k,
                                                                    float* __restrict__ out_val,
                                                                    int* __restrict__ out_idx) {
    constexpr int NS = TOPK_P * TOPK_CAP / TOPK_THREADS;  // candidate slots per thread
    static_assert(TOPK_THREADS == 2 * TOPK_CAP && NS <= 32, "slot map: two slices per round, <= 32 slots");
    __shared__ uint32_t keys[TOPK_P * TOPK_CAP];
    __shared__ int idx[TOPK_P * TOPK_CAP];
    __shared__ int offs[TOPK_P + 1];
    __shared__ int pos[64];
    __shared__ TkShared sh;
    __shared__ uint32_t sk[TOPK_THREADS];
    __shared__ int si[TOPK_THREADS];
    __shared__ uint32_t wt[TOPK_THREADS / 64];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    // every slot's candidate and its slice's count requested at once; slots
    // past their slice's count are invalid (no compaction on the common path).
    // Slot j of a thread: slice 2j + tid / 128, offset (tid + 37 j) mod 128,
    // so each thread sees low offsets (the filled ones) of many slices.
    const size_t rb = (size_t)row * P * TOPK_CAP;
    uint32_t ck[NS];
    int cx[NS];
    uint32_t cvm = 0;  // bit j: slot j valid
    uint32_t tm = 0;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int seg = 2 * j + (tid >> 7), off = ((tid & 127) + 37 * j) & 127;
        const int segc = min(seg, P - 1);
        const uint64_t c = cand[rb + (size_t)segc * TOPK_CAP + off];
        const int cnt = cand_cnt[(size_t)row * P + segc];
        const bool ok = seg < P && off < cnt;
        ck[j] = ok ? (uint32_t)(c >> 32) : 0u;
        cx[j] = ok ? (int)(uint32_t)c : 0x7fffffff;
        cvm |= ok ? (1u << j) : 0u;
        tm = ok ? max(tm, ck[j]) : tm;
    }
    // total candidates (each wave sums the slice counts itself)
    const int n = (int)wave_sum((float)(lane < P ? cand_cnt[(size_t)row * P + lane] : 0));
    // n > 256: every thread holds a candidate, so each wave's ceil(k/4)
    // largest maxima are candidates' keys and at least k candidates are >= T
    const uint32_t T = n > TOPK_THREADS ? tk_block_threshold(tm, k, wt) : 0u;
    int c = 0;
#pragma unroll
    for (int j = 0; j < NS; ++j) c += ((cvm >> j) & 1u) && ck[j] >= T ? 1 : 0;
    int total;
    int base = tk_excl_scan(c, sh.wsum, total);
    if (total <= TOPK_THREADS) {
        // survivors -> LDS; each one's rank = survivors ordered before it,
        // counted by g = 256 / (survivor slots) threads over 1/g of them each
        __shared__ int rk[TOPK_THREADS];
        rk[tid] = 0;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            if (((cvm >> j) & 1u) && ck[j] >= T) {
                sk[base] = ck[j];
                si[base] = cx[j];
                ++base;
            }
        }
        __syncthreads();
        const int per = total <= 64 ? 64 : (total <= 128 ? 128 : TOPK_THREADS);
        const int g = TOPK_THREADS / per, sv = tid % per, q = tid / per;
        if (sv < total) {
            const uint32_t kk = sk[sv];
            const int ix = si[sv];
            const int j0 = (total * q) / g, j1 = (total * (q + 1)) / g;
            int rank = 0;
#pragma unroll 8
            for (int j = j0; j < j1; ++j) rank += tk_before(sk[j], si[j], kk, ix) ? 1 : 0;
            if (g > 1) atomicAdd(&rk[sv], rank);
            else rk[sv] = rank;
        }
        __syncthreads();
        if (tid < total) {
            const int rank = rk[tid];
            if (rank < k) {
                out_val[(size_t)row * k + rank] = tk_val(sk[tid]);
                out_idx[(size_t)row * k + rank] = si[tid];
            }
        }
        return;
    }
    // many ties at the top: compact every candidate into keys[0 .. n) ...
    if (tid < 64) {
        const int cc = tid < P ? cand_cnt[(size_t)row * P + tid] : 0;
        int incl = cc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        offs[tid] = incl - cc;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const int seg = 2 * j + (tid >> 7), off = ((tid & 127) + 37 * j) & 127;
        if ((cvm >> j) & 1u) {
            keys[offs[seg] + off] = ck[j];
            idx[offs[seg] + off] = cx[j];
        }
    }
    __syncthreads();
    // ... and select exactly by radix over all of them
    int need_eq;
    const uint32_t T64 = tk_radix_select(keys, n, 64, sh, need_eq);
    const int kept = tk_compact(keys, n, T64, need_eq, pos, sh);
    if (tid < 64) {
        uint32_t kk = 0;
        int ix = 0x7fffffff;
        if (tid < kept) { kk = keys[pos[tid]]; ix = idx[pos[tid]]; }
        tk_sort64(kk, ix, lane);
        if (lane < k) {
            out_val[(size_t)row * k + lane] = tk_val(kk);
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

hipError_t add_rmsnorm(const void* x, const float* part, int n_parts, const void* w, void* x_out, void* xn,
                      int rows, int hidden, float eps, hipStream_t st) {
    const int ch = (hidden / 8 + 255) / 256;
#define ADDN_LAUNCH(C)                                                                                            \
    hipLaunchKernelGGL(add_rmsnorm_kernel<C>, dim3(rows), dim3(256), 0, st, (const __half*)x, part, n_parts,     \
                       (const __half*)w, (__half*)x_out, (__half*)xn, rows, hidden, eps)
    if (ch == 1) ADDN_LAUNCH(1);
    else if (ch == 2) ADDN_LAUNCH(2);
    else if (ch == 3) ADDN_LAUNCH(3);
    else ADDN_LAUNCH(4);
#undef ADDN_LAUNCH
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

hipError_t embedding(int fmt, const int* tokens, const void* table, void* out, int n_tokens, int hidden,
                     float scale, hipStream_t st) {
    const int n = n_tokens * hidden;
    auto* k = fmt == 4 ? embedding_lookup_q4k_kernel : fmt == 6 ? embedding_lookup_q6k_kernel
                                                                 : embedding_lookup_q8_0_kernel;
    hipLaunchKernelGGL(k, dim3((n + 255) / 256), dim3(256), 0, st, tokens, table, (__half*)out, n_tokens, hidden,
                       scale);
    return hipGetLastError();
}

// Greedy decoding without a host round trip: the next token of row b is its
// top-1 candidate (out_idx[b][0]: the largest logit, the lowest id among
// equal ones, as np.argmax picks it); it becomes row b's token of the next
// step (tokens[b]), its position advances by one (kv_offset[b], held at
// max_pos), and it is recorded in history[step][b] (while step < hist_steps).
// One block; every thread reads the step counter before thread 0 advances it.
__global__ void greedy_advance_kernel(const int* __restrict__ top_idx, int k, int rows, int* __restrict__ tokens,
                                      int* __restrict__ kv_offset, int max_pos, int* __restrict__ history,
                                      int hist_steps, int* __restrict__ step) {
    __shared__ int s_step;
    if (threadIdx.x == 0) s_step = *step;
    __syncthreads();
    const int s = s_step;
    for (int b = threadIdx.x; b < rows; b += blockDim.x) {
        const int tok = top_idx[(size_t)b * k];
        tokens[b] = tok;
        kv_offset[b] = min(kv_offset[b] + 1, max_pos);
        if (s < hist_steps) history[(size_t)s * rows + b] = tok;
    }
    __syncthreads();
    if (threadIdx.x == 0) *step = s + 1;
}

hipError_t greedy_advance(const int* top_idx, int k, int rows, int* tokens, int* kv_offset, int max_pos,
                          int* history, int hist_steps, int* step, hipStream_t st) {
    hipLaunchKernelGGL(greedy_advance_kernel, dim3(1), dim3(256), 0, st, top_idx, k, rows, tokens, kv_offset, max_pos,
                       history, hist_steps, step);
    return hipGetLastError();
}

size_t topk_scratch_bytes(int rows) { return (size_t)rows * TOPK_P * (TOPK_CAP * 8 + 4); }

hipError_t topk(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx, void* work,
                hipStream_t st, const int* excl_ids, const int* excl_cnt, int max_excl, float* gathered) {
    if (vocab > TOPK_P * TOPK_SLICE) return hipErrorInvalidValue;
    // as many slices as needed, each at most TOPK_SLICE, at most TOPK_P of them
    int P = (vocab + 2047) / 2048;
    if (P > TOPK_P) P = TOPK_P;
    const int slice = (vocab + P - 1) / P;
    uint64_t* cand = (uint64_t*)work;
    int* cc = (int*)((char*)work + (size_t)rows * TOPK_P * TOPK_CAP * 8);
    const TkExclude ex{excl_ids, excl_cnt, max_excl, gathered};
    hipLaunchKernelGGL(topk_partial_kernel, dim3(P, rows), dim3(TOPK_THREADS), 0, st, logits, vocab, slice, k, cand,
                       cc, ex);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(topk_final_kernel, dim3(rows), dim3(TOPK_THREADS), 0, st, cand, cc, P, k, out_val, out_idx);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Allocation-free top-k: the candidate buffer lives in a file-scope device
// array of TOPK_NOALLOC_MAX_ROWS rows (4.2 MB, held by every GPU the library
// runs on until the process ends).  Host code never passes `scratch` itself
// (its name is a host-side stand-in, not a device address): the device
// address is looked up once per device with hipGetSymbolAddress and kept.
// Every call on one GPU shares that GPU's array, so calls that overlap on one
// GPU (two streams, two threads) race.  The kernels need no clearing: every
// slice writes its candidate count before the final pass reads it.
// ---------------------------------------------------------------------------
#define TOPK_NOALLOC_MAX_ROWS 64
#define TOPK_NOALLOC_BYTES ((size_t)TOPK_NOALLOC_MAX_ROWS * TOPK_P * (TOPK_CAP * 8 + 4))
static __device__ __align__(256) uint8_t scratch[TOPK_NOALLOC_BYTES];

#define TOPK_NOALLOC_MAX_DEVICES 64
static void* g_scratch_ptr[TOPK_NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

int topk_noalloc_max_rows() { return TOPK_NOALLOC_MAX_ROWS; }

// Device address of this device's `scratch` (looked up on the first call
// per device, with that device current).
hipError_t topk_noalloc_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= TOPK_NOALLOC_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

hipError_t topk_noalloc(const float* logits, int rows, int vocab, int k, float* out_val, int* out_idx,
                        hipStream_t st) {
    if (rows > TOPK_NOALLOC_MAX_ROWS) return hipErrorInvalidValue;
    void* work = nullptr;
    const hipError_t e = topk_noalloc_scratch(&work);
    if (e != hipSuccess) return e;
    return topk(logits, rows, vocab, k, out_val, out_idx, work, st, nullptr, nullptr, 0, nullptr);
}

}  // namespace vte
