// Planned quantised mat-vec: one persistent launch computes several weight
// segments against the same activations with per-segment epilogues, fusing the
// decode-step glue into the GEMV (gfx950).
//
// Reference nodes replaced, per layer (vte/compiler/qwen_compute.py:100-282,
// captured in vte/core/hip_graph_executor.py:504-738):
//   rmsnorm -> gemv q/k/v (+bias) -> rope -> kv_cache_append     => one launch
//   rmsnorm -> gemv gate/up -> swiglu                            => one launch
//   rmsnorm(output_norm) -> LM-head gemv                         => one launch
// with the same rounding points as those nodes: normalised activations,
// projections (+bias), rotated q/k and the SwiGLU output are fp16 values,
// computed in fp32 from fp16 inputs:
//   rmsnorm   fp16(x * rsqrt(mean(x^2) + eps) * w)            rmsnorm.hip.template:19-71
//   rope      fp16(a*c - b*s), fp16(a*s + b*c) on (d, d+64)    rope.hip.template:82-97
//   swiglu    fp16(g / (1 + exp(-g)) * u)                      swiglu.hip.template:11-25
//
// Row tiles: plain tiles are R consecutive rows; paired tiles are R/2 rows
// plus R/2 partner rows (RoPE: d and d + 64 of the same head; SwiGLU: the same
// row of the gate and up matrices), so a pair's two dot products finish in
// the same block.  Dot products use the engine in rows.h.
#include <cstring>

#include "rows.h"

#define FMV_MAX_SEG 3
#define FMV_Q6_CHUNKS 8   // 16-byte chunks per thread for a staged Q6_K tile
#define FMV_Q4_UNITS 2    // Q4_K units per thread per tile
#define FMV_MAX_R 32

enum FmvMode : int {
    FMV_STORE_F16 = 0,   // out[m][row] = fp16((acc + bias) * rs + residual)
    FMV_STORE_F32 = 1,   // same, fp32 output (logits)
    FMV_ROPE_Q = 2,      // fp16(acc + bias), rotated, -> out (q buffer [m][rows])
    FMV_ROPE_KCACHE = 3, // fp16(acc + bias), rotated, -> k_cache at kv_offset[m]
    FMV_VCACHE = 4,      // fp16(acc + bias) -> v_cache at kv_offset[m]
    FMV_SWIGLU = 5,      // rows of w (gate) and w2 (up): out[m][j] = fp16(silu(g) * u)
};

struct FmvSeg {
    const uint8_t* w;      // weight rows (gate for SwiGLU)
    const uint8_t* w2;     // up rows (SwiGLU only)
    void* out;
    const __half* bias;    // nullable, fp16 [n_rows]
    const __half* residual;  // nullable, fp16 [M][n_rows]
    int fmt;               // 4 = Q4_K, 6 = Q6_K
    int n_rows;            // output rows of this segment
    int R;                 // rows per tile (paired modes: even, R/2 divides 64 for RoPE)
    int mode;
    int tiles;
};

struct FmvPlan {
    FmvSeg seg[FMV_MAX_SEG];
    int nseg;
    int K;
    int M;
    const __half* norm_w;  // nullable: RMSNorm prologue on the activations
    float eps;
    float rs;              // residual scale of store epilogues
    const __half* rope_cos;
    const __half* rope_sin;
    const int* kv_offset;
    __half* k_cache;
    __half* v_cache;
    int kv_batch_stride;
    int n_kv;
};

struct FmvTile {
    int seg, t;
};

__device__ __forceinline__ FmvTile fmv_tile(const FmvPlan& P, int g) {
    FmvTile r{-1, 0};
    for (int s = 0; s < P.nseg; ++s) {
        if (g < P.seg[s].tiles) { r.seg = s; r.t = g; return r; }
        g -= P.seg[s].tiles;
    }
    return r;
}

__device__ __forceinline__ bool fmv_paired(int mode) {
    return mode == FMV_ROPE_Q || mode == FMV_ROPE_KCACHE || mode == FMV_SWIGLU;
}

// Local row lr of tile t -> (matrix base, global row).  Returns rows in tile.
__device__ __forceinline__ int fmv_rows(const FmvSeg& S, int t) {
    if (!fmv_paired(S.mode)) return min(S.R, S.n_rows - t * S.R);
    if (S.mode == FMV_SWIGLU) return 2 * min(S.R / 2, S.n_rows - t * (S.R / 2));
    return S.R;
}

// For paired modes the "first" rows of tile t start at j0 and the partner of
// local row i < R/2 is local row i + R/2.
__device__ __forceinline__ void fmv_row(const FmvSeg& S, int t, int lr, const uint8_t*& base, int& row) {
    const int h = S.R / 2;
    if (!fmv_paired(S.mode)) { base = S.w; row = t * S.R + lr; return; }
    if (S.mode == FMV_SWIGLU) {
        const int nf = min(h, S.n_rows - t * h);  // rows per half in this tile
        const int j0 = t * h;
        if (lr < nf) { base = S.w; row = j0 + lr; } else { base = S.w2; row = j0 + lr - nf; }
        return;
    }
    const int tiles_per_head = 64 / h;
    const int head = t / tiles_per_head, j0 = (t % tiles_per_head) * h;
    base = S.w;
    row = head * 128 + j0 + (lr < h ? lr : lr - h + 64);
}

template <int NC>
__global__ __launch_bounds__(ROWS_THREADS) void fused_mv_kernel(const __half* __restrict__ x, FmvPlan P) {
    extern __shared__ uint4 smem_fmv[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem_fmv);
    const int K = P.K, M = P.M;
    const int n_sb = K / QK_K;
    const int per_row = n_sb * 4;
    const int ldx = xpad_len(K);
    // LDS plan: x [NC][ldx] fp16 | s16 [NC][K/16] | part [NC][FMV_MAX_R*per_row] | rsum [NC][FMV_MAX_R] |
    //           norm weights [ldx] fp16 (with a norm) | stage
    _Float16* xs = reinterpret_cast<_Float16*>(lds);
    size_t o = ((size_t)NC * ldx * 2 + 15) & ~(size_t)15;
    float* s16 = reinterpret_cast<float*>(lds + o);
    o += (size_t)NC * (K / 16) * 4;
    o = (o + 15) & ~(size_t)15;
    float* part = reinterpret_cast<float*>(lds + o);
    const int ustride = FMV_MAX_R * per_row;
    o += (size_t)NC * ustride * 4;
    float* rsum = reinterpret_cast<float*>(lds + o);
    o += (size_t)NC * FMV_MAX_R * 4;
    o = (o + 15) & ~(size_t)15;
    _Float16* wn_s = reinterpret_cast<_Float16*>(lds + o);
    if (P.norm_w != nullptr) o += ((size_t)ldx * 2 + 15) & ~(size_t)15;
    uint8_t* stage = lds + o;
    __shared__ float red[4][NC];
    __shared__ int pos_s[NC];  // kv_offset[m], read once per block

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int total = 0;
    for (int s = 0; s < P.nseg; ++s) total += P.seg[s].tiles;
    const int G = gridDim.x;

    Q4KUnitData cur[FMV_Q4_UNITS], nxt[FMV_Q4_UNITS];
    uint4 chunk[FMV_Q6_CHUNKS];
    auto load_tile = [&](int g, Q4KUnitData (&q4)[FMV_Q4_UNITS]) {
        if (g >= total) return;
        const FmvTile T = fmv_tile(P, g);
        const FmvSeg& S = P.seg[T.seg];
        const int nr = fmv_rows(S, T.t);
        if (S.fmt == 4) {
            const float inv = 1.0f / (float)n_sb;
#pragma unroll
            for (int j = 0; j < FMV_Q4_UNITS; ++j) {
                const int u = tid + j * ROWS_THREADS;
                if (u < nr * per_row) {
                    const int sbg = u >> 2;
                    const int lr = (int)(((float)sbg + 0.5f) * inv);
                    const uint8_t* base;
                    int row;
                    fmv_row(S, T.t, lr, base, row);
                    q4[j] = q4k_unit_load(base + ((size_t)row * n_sb + (sbg - lr * n_sb)) * Q4K_BYTES, u & 3);
                }
            }
        } else {  // Q6_K plain tile: contiguous rows, stage the aligned byte range
            const uintptr_t a = reinterpret_cast<uintptr_t>(S.w + (size_t)T.t * S.R * n_sb * Q6K_BYTES);
            const uintptr_t a0 = a & ~(uintptr_t)15;
            const int nchunk = (int)((a + (size_t)nr * n_sb * Q6K_BYTES - a0 + 15) >> 4);
#pragma unroll
            for (int j = 0; j < FMV_Q6_CHUNKS; ++j) {
                const int c = tid + j * ROWS_THREADS;
                if (c < nchunk) chunk[j] = ldg_stream16(reinterpret_cast<const uint8_t*>(a0) + 16 * (size_t)c);
            }
        }
    };
    auto store_stage = [&](int g) {
        if (g >= total) return;
        const FmvTile T = fmv_tile(P, g);
        const FmvSeg& S = P.seg[T.seg];
        if (S.fmt != 6) return;
        const int nr = fmv_rows(S, T.t);
        const uintptr_t a = reinterpret_cast<uintptr_t>(S.w + (size_t)T.t * S.R * n_sb * Q6K_BYTES);
        const uintptr_t a0 = a & ~(uintptr_t)15;
        const int nchunk = (int)((a + (size_t)nr * n_sb * Q6K_BYTES - a0 + 15) >> 4);
#pragma unroll
        for (int j = 0; j < FMV_Q6_CHUNKS; ++j) {
            const int c = tid + j * ROWS_THREADS;
            if (c < nchunk) reinterpret_cast<uint4*>(stage)[c] = chunk[j];
        }
    };

    int g = blockIdx.x;
    if (tid < M && P.kv_offset != nullptr) pos_s[tid] = P.kv_offset[tid];
    load_tile(g, cur);
    // ---- activations: fp16 [M][K] -> LDS, optional RMSNorm ----
    stage_act<NC>(x, false, M, K, xs, P.norm_w, wn_s);
    store_stage(g);
    __syncthreads();
    if (P.norm_w != nullptr) {
        float ss[NC];
#pragma unroll
        for (int m = 0; m < NC; ++m) ss[m] = 0.f;
        for (int e = tid; e < K; e += ROWS_THREADS) {
#pragma unroll
            for (int m = 0; m < NC; ++m) {
                const float v = (float)xs[m * ldx + xpad(e)];
                ss[m] = fmaf(v, v, ss[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < NC; ++m) {
            ss[m] = wave_sum(ss[m]);
            if (lane == 0) red[wv][m] = ss[m];
        }
        __syncthreads();
        float inv[NC];
#pragma unroll
        for (int m = 0; m < NC; ++m)
            inv[m] = rsqrtf((red[0][m] + red[1][m] + red[2][m] + red[3][m]) / (float)K + P.eps);
        for (int e = tid; e < K; e += ROWS_THREADS) {
            const float wn = (float)wn_s[xpad(e)];
#pragma unroll
            for (int m = 0; m < NC; ++m) {
                _Float16& xv = xs[m * ldx + xpad(e)];
                xv = (_Float16)((float)xv * inv[m] * wn);
            }
        }
        __syncthreads();
    }
    act_sums<NC>(ActLDS{xs, s16}, K);
    __syncthreads();

    for (; g < total; g += G) {
        const FmvTile T = fmv_tile(P, g);
        const FmvSeg& S = P.seg[T.seg];
        const int nr = fmv_rows(S, T.t);
        const int units = nr * per_row;
        const int gn = g + G;
        load_tile(gn, nxt);
        const float inv_nsb = 1.0f / (float)n_sb;
        if (S.fmt == 4) {
#pragma unroll
            for (int j = 0; j < FMV_Q4_UNITS; ++j) {
                const int u = tid + j * ROWS_THREADS;
                if (u >= units) break;
                const int sbg = u >> 2, q = u & 3;
                const int lr = (int)(((float)sbg + 0.5f) * inv_nsb);
                const int sb = sbg - lr * n_sb;
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * ustride + u] = q4k_unit_dot(cur[j], q, xs + (size_t)m * ldx + xpad(sb * QK_K + 64 * q),
                                                         s16 + m * (K / 16) + sb * 16 + 4 * q);
            }
        } else {
            const uint8_t* rows_lds =
                stage + (reinterpret_cast<uintptr_t>(S.w + (size_t)T.t * S.R * n_sb * Q6K_BYTES) & 15);
            for (int u = tid; u < units; u += ROWS_THREADS) {
                const int sbg = u >> 2, q = u & 3;
                const int lr = (int)(((float)sbg + 0.5f) * inv_nsb);
                const int sb = sbg - lr * n_sb;
                const uint8_t* blk = rows_lds + (size_t)sbg * Q6K_BYTES;
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * ustride + u] = q6k_unit_dot(blk, q >> 1, (q & 1) * 16, xs + (size_t)m * ldx + xpad(sb * QK_K),
                                                         s16 + m * (K / 16) + sb * 16);
            }
        }
        __syncthreads();
        for (int i = tid; i < NC * nr; i += ROWS_THREADS) {
            const int m = i / nr, r = i - m * nr;
            const float4* p = reinterpret_cast<const float4*>(part + m * ustride + r * per_row);
            float sacc = 0.f;
            for (int j = 0; j < per_row / 4; ++j) {
                const float4 v = p[j];
                sacc += (v.x + v.y) + (v.z + v.w);
            }
            rsum[m * FMV_MAX_R + r] = sacc;
        }
        store_stage(gn);
        __syncthreads();
        // ---- epilogue ----
        if (!fmv_paired(S.mode)) {
            for (int i = tid; i < M * nr; i += ROWS_THREADS) {
                const int m = i / nr, r = i - m * nr;
                const uint8_t* base;
                int row;
                fmv_row(S, T.t, r, base, row);
                float v = rsum[m * FMV_MAX_R + r];
                if (S.bias) v += __half2float(S.bias[row]);
                if (S.mode == FMV_VCACHE) {
                    const int pos = pos_s[m];
                    P.v_cache[(size_t)m * P.kv_batch_stride + ((size_t)pos * P.n_kv + row / 128) * 128 + (row % 128)] =
                        __float2half(v);
                    continue;
                }
                v *= P.rs;
                const size_t oi = (size_t)m * S.n_rows + row;
                if (S.residual) v += __half2float(S.residual[oi]);
                if (S.mode == FMV_STORE_F32) reinterpret_cast<float*>(S.out)[oi] = v;
                else reinterpret_cast<__half*>(S.out)[oi] = __float2half(v);
            }
        } else {
            const int hp = nr / 2;
            for (int i = tid; i < M * hp; i += ROWS_THREADS) {
                const int m = i / hp, r = i - m * hp;
                const uint8_t* base;
                int row1, row2;
                fmv_row(S, T.t, r, base, row1);
                fmv_row(S, T.t, r + hp, base, row2);
                float a = rsum[m * FMV_MAX_R + r], bv = rsum[m * FMV_MAX_R + r + hp];
                if (S.mode == FMV_SWIGLU) {
                    const float gg = __half2float(__float2half(a));
                    const float uu = __half2float(__float2half(bv));
                    const float sig = 1.0f / (1.0f + expf(-gg));
                    reinterpret_cast<__half*>(S.out)[(size_t)m * S.n_rows + row1] = __float2half(gg * sig * uu);
                    continue;
                }
                if (S.bias) { a += __half2float(S.bias[row1]); bv += __half2float(S.bias[row2]); }
                const float x1 = __half2float(__float2half(a)), x2 = __half2float(__float2half(bv));
                const int pos = pos_s[m];
                const int d = row1 % 128;
                const float c = __half2float(P.rope_cos[(size_t)pos * 128 + d]);
                const float sn = __half2float(P.rope_sin[(size_t)pos * 128 + d]);
                const __half o1 = __float2half(x1 * c - x2 * sn), o2 = __float2half(x1 * sn + x2 * c);
                if (S.mode == FMV_ROPE_Q) {
                    __half* q = reinterpret_cast<__half*>(S.out) + (size_t)m * S.n_rows;
                    q[row1] = o1;
                    q[row2] = o2;
                } else {
                    __half* kc = P.k_cache + (size_t)m * P.kv_batch_stride + ((size_t)pos * P.n_kv + row1 / 128) * 128;
                    kc[d] = o1;
                    kc[d + 64] = o2;
                }
            }
        }
        // the next tile's Q4_K units (if it is a Q4_K tile) become current
#pragma unroll
        for (int j = 0; j < FMV_Q4_UNITS; ++j) cur[j] = nxt[j];
    }
}

namespace vte {

static int fmv_num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    }
    return n;
}

size_t fmv_lds_bytes(int NC, int K, bool has_q6, bool has_norm) {
    const int per_row = (K / 256) * 4;
    size_t o = ((size_t)NC * xpad_len(K) * 2 + 15) & ~(size_t)15;
    o += (size_t)NC * (K / 16) * 4;
    o = (o + 15) & ~(size_t)15;
    o += (size_t)NC * FMV_MAX_R * per_row * 4;
    o += (size_t)NC * FMV_MAX_R * 4;
    o = (o + 15) & ~(size_t)15;
    if (has_norm) o += ((size_t)xpad_len(K) * 2 + 15) & ~(size_t)15;
    if (has_q6) o += (size_t)ROWS_THREADS * FMV_Q6_CHUNKS * 16;
    return o;
}

// Rows per tile for a segment (0 if the shape cannot be tiled).
int fmv_rows_per_tile(int fmt, int mode, int K, int n_rows) {
    const int n_sb = K / 256;
    if (fmt == 4) {
        int R = ROWS_THREADS * FMV_Q4_UNITS / (n_sb * 4);
        if (R > FMV_MAX_R) R = FMV_MAX_R;
        if (mode == FMV_ROPE_Q || mode == FMV_ROPE_KCACHE) {  // R/2 must divide 64
            int h = 1;
            while (2 * h <= R / 2 && 64 % (2 * h) == 0) h *= 2;
            return 2 * h;
        }
        if (mode == FMV_SWIGLU) return R >= 2 ? (R & ~1) : 0;
        return R >= 1 ? R : 0;
    }
    if (mode != FMV_STORE_F16 && mode != FMV_STORE_F32 && mode != FMV_VCACHE) return 0;  // Q6_K: plain tiles only
    int R = (int)(((size_t)ROWS_THREADS * FMV_Q6_CHUNKS * 16 - 48) / ((size_t)n_sb * Q6K_BYTES));
    if (R > FMV_MAX_R) R = FMV_MAX_R;
    (void)n_rows;
    return R;
}

hipError_t fused_mv(const __half* x, FmvPlan plan, hipStream_t st) {
    bool has_q6 = false;
    int total = 0;
    for (int s = 0; s < plan.nseg; ++s) {
        FmvSeg& S = plan.seg[s];
        if (S.R <= 0) return hipErrorInvalidValue;
        if (S.fmt == 6) has_q6 = true;
        if (S.mode == FMV_SWIGLU) S.tiles = (S.n_rows + S.R / 2 - 1) / (S.R / 2);
        else if (S.mode == FMV_ROPE_Q || S.mode == FMV_ROPE_KCACHE) S.tiles = S.n_rows / S.R;
        else S.tiles = (S.n_rows + S.R - 1) / S.R;
        total += S.tiles;
    }
    const int NC = plan.M <= 1 ? 1 : (plan.M <= 2 ? 2 : 4);
    const size_t lds = fmv_lds_bytes(NC, plan.K, has_q6, plan.norm_w != nullptr);
    if (plan.norm_w != nullptr && (reinterpret_cast<uintptr_t>(plan.norm_w) & 15)) return hipErrorInvalidValue;
    if (lds > 65536 || plan.M > 4) return hipErrorNotSupported;
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (plan.K & 7)) return hipErrorInvalidValue;  // 16-byte staging
    int blocks = 0;
    hipError_t e;
    if (NC == 1) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, (const void*)fused_mv_kernel<1>, ROWS_THREADS, lds);
    else if (NC == 2) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, (const void*)fused_mv_kernel<2>, ROWS_THREADS, lds);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, (const void*)fused_mv_kernel<4>, ROWS_THREADS, lds);
    if (e != hipSuccess || blocks <= 0) blocks = 1;
    int grid = fmv_num_cus() * blocks;
    if (grid > total) grid = total;
    if (NC == 1) hipLaunchKernelGGL(fused_mv_kernel<1>, dim3(grid), dim3(ROWS_THREADS), lds, st, x, plan);
    else if (NC == 2) hipLaunchKernelGGL(fused_mv_kernel<2>, dim3(grid), dim3(ROWS_THREADS), lds, st, x, plan);
    else hipLaunchKernelGGL(fused_mv_kernel<4>, dim3(grid), dim3(ROWS_THREADS), lds, st, x, plan);
    return hipGetLastError();
}

static FmvPlan plan_base(int M, int K, const void* norm_w, float eps) {
    FmvPlan P;
    memset(&P, 0, sizeof(P));
    P.M = M;
    P.K = K;
    P.norm_w = (const __half*)norm_w;
    P.eps = eps;
    P.rs = 1.0f;
    return P;
}

static FmvSeg seg(const void* w, const void* w2, void* out, const void* bias, const void* residual, int fmt,
                  int n_rows, int mode, int K) {
    FmvSeg S;
    S.w = (const uint8_t*)w;
    S.w2 = (const uint8_t*)w2;
    S.out = out;
    S.bias = (const __half*)bias;
    S.residual = (const __half*)residual;
    S.fmt = fmt;
    S.n_rows = n_rows;
    S.mode = mode;
    S.R = fmv_rows_per_tile(fmt, mode, K, n_rows);
    S.tiles = 0;
    return S;
}

hipError_t attn_in(const void* x, const void* norm_w, float eps, const void* wq, const void* q_bias, int fmt_q,
                   const void* wk, const void* k_bias, int fmt_k, const void* wv, const void* v_bias, int fmt_v,
                   void* q_out, void* k_cache, void* v_cache, const int* kv_offset, int kv_batch_stride,
                   const void* rope_cos, const void* rope_sin, int M, int K, int n_q, int n_kv, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.seg[0] = seg(wq, nullptr, q_out, q_bias, nullptr, fmt_q, n_q * 128, FMV_ROPE_Q, K);
    P.seg[1] = seg(wk, nullptr, nullptr, k_bias, nullptr, fmt_k, n_kv * 128, FMV_ROPE_KCACHE, K);
    P.seg[2] = seg(wv, nullptr, nullptr, v_bias, nullptr, fmt_v, n_kv * 128, FMV_VCACHE, K);
    P.nseg = 3;
    P.rope_cos = (const __half*)rope_cos;
    P.rope_sin = (const __half*)rope_sin;
    P.kv_offset = kv_offset;
    P.k_cache = (__half*)k_cache;
    P.v_cache = (__half*)v_cache;
    P.kv_batch_stride = kv_batch_stride;
    P.n_kv = n_kv;
    return fused_mv((const __half*)x, P, st);
}

hipError_t ffn_in(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up, int fmt,
                  void* out, int M, int K, int ffn, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.seg[0] = seg(w_gate, w_up, out, nullptr, nullptr, fmt, ffn, FMV_SWIGLU, K);
    P.nseg = 1;
    return fused_mv((const __half*)x, P, st);
}

hipError_t norm_mv(const void* x, const void* norm_w, float eps, const void* w, int fmt, void* out, bool out_f32,
                   const void* bias, const void* residual, float rs, int M, int K, int N, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.rs = rs;
    P.seg[0] = seg(w, nullptr, out, bias, residual, fmt, N, out_f32 ? FMV_STORE_F32 : FMV_STORE_F16, K);
    P.nseg = 1;
    return fused_mv((const __half*)x, P, st);
}

}  // namespace vte
