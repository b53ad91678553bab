// Quantised mat-vec for batch 1..4 (gfx950), the bandwidth kernel of the
// decode step.  One launch computes up to three weight segments against the
// same activations, each with its own epilogue, so the decode-step glue is
// fused into the GEMV:
//
//   rmsnorm -> gemv q/k/v (+bias) -> rope -> kv_cache_append     => one launch
//   rmsnorm -> gemv gate/up -> swiglu                            => one launch
//   rmsnorm(output_norm) -> LM-head gemv                         => one launch
//   gemv (+bias, *scale, +residual), e.g. o-proj / down          => one launch
//
// (reference nodes: vte/compiler/qwen_compute.py:100-282, captured by
// vte/core/hip_graph_executor.py:504-738), with the same rounding points as
// those nodes: normalised activations, projections (+bias), rotated q/k and
// the SwiGLU output are fp16 values computed in fp32 from fp16 inputs:
//   rmsnorm   fp16(x * rsqrt(mean(x^2) + eps) * w)            rmsnorm.hip.template:19-71
//   rope      fp16(a*c - b*s), fp16(a*s + b*c) on (d, d+64)    rope.hip.template:82-97
//   swiglu    fp16(g / (1 + exp(-g)) * u)                      swiglu.hip.template:11-25
//
// One block (256 threads) per tile, one work unit (64 weights sharing a scale
// pair) per thread.  A tile is R rows whose units fill the block -- plain
// tiles are consecutive rows; paired tiles are R/2 rows plus their partner
// rows (RoPE d and d + 64 of one head, or gate row j and up row j), so a
// pair's two dot products finish in the same block.  Everything a block reads
// is requested up front -- its weights (straight into registers: no LDS copy,
// no pipeline), the epilogue operands and the activations -- so a block costs
// one memory latency plus its arithmetic, and the GPU overlaps many blocks
// (low register and LDS use keep several blocks resident per CU).  Partials
// meet in LDS and each output is summed in a fixed order (graph replays are
// bit for bit reproducible).
#pragma once
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "rows.h"

#define TMV_MAX_SEG 3
#define TMV_MAX_R 64


enum FmvMode : int {
    FMV_STORE_F16 = 0,   // out[m][row] = fp16((acc + bias) * rs + residual)
    FMV_STORE_F32 = 1,   // same, fp32 output
    FMV_ROPE_Q = 2,      // fp16(acc + bias), rotated, -> out (q buffer [m][rows])
    FMV_ROPE_KCACHE = 3, // fp16(acc + bias), rotated, -> k_cache at kv_offset[m]
    FMV_VCACHE = 4,      // fp16(acc + bias) -> v_cache at kv_offset[m]
    FMV_SWIGLU = 5,      // rows of w (gate) and w2 (up): out[m][j] = fp16(silu(g) * u)
};

struct FmvSeg {
    const uint8_t* w;        // weight rows (gate for SwiGLU)
    const uint8_t* w2;       // up rows (SwiGLU only)
    void* out;
    const void* bias;        // nullable, [n_rows] in the output type (fp16 for fused modes)
    const void* residual;    // nullable, [M][n_rows] in the output type
    int fmt;                 // 4 = Q4_K, 6 = Q6_K
    int n_rows;              // output rows of this segment
    int R;                   // rows per tile (paired modes: even; RoPE: R/2 a power of two dividing 64)
    int mode;
    int tiles;
    int row_bytes;
};

struct FmvPlan {
    FmvSeg seg[TMV_MAX_SEG];
    int nseg;
    int total;               // tiles over all segments (= blocks)
    int K;
    int M;
    int x_f32;               // activations fp32 (else fp16)
    const __half* norm_w;    // nullable: RMSNorm prologue on the activations
    float eps;
    float rs;                // residual scale of store epilogues
    const __half* rope_cos;
    const __half* rope_sin;
    const int* kv_offset;
    __half* k_cache;
    __half* v_cache;
    int kv_batch_stride;
    int n_kv;
    // activations from split-KV partials (log-sum-exp combine in the prologue)
    const float* att_m;      // nullable: [M][att_nq][att_S] running maxima
    const float* att_l;      // [M][att_nq][att_S] denominators
    const float* att_o;      // [M][att_nq][att_S][128] unnormalised outputs
    int att_nq, att_S, att_split;
    int wfirst;              // launch the weights-first form (fused_mv_kernel WF) when it exists
};

__host__ __device__ __forceinline__ bool fmv_paired(int mode) {
    return mode == FMV_ROPE_Q || mode == FMV_ROPE_KCACHE || mode == FMV_SWIGLU;
}

// Tile g: its segment's parameters, rows and row bases (A: local rows
// [0, hA), B: local rows [hA, nr)).  Segments are selected with a fixed
// if-chain (an indexed struct access would reload the kernel argument).
struct TileGeo {
    int nr, hA, j0;
    const uint8_t* bA;
    const uint8_t* bB;
    int fmt, mode, rb, n_rows;
    void* out;
    const void* bias;
    const void* residual;
};

__device__ __forceinline__ void geo_from_seg(const FmvSeg& S, int g, TileGeo& T) {
    const int rb = S.row_bytes;
    T.fmt = S.fmt;
    T.mode = S.mode;
    T.rb = rb;
    T.n_rows = S.n_rows;
    T.out = S.out;
    T.bias = S.bias;
    T.residual = S.residual;
    if (!fmv_paired(S.mode)) {
        T.j0 = g * S.R;
        T.nr = min(S.R, S.n_rows - T.j0);
        T.hA = T.nr;
        T.bA = S.w + (size_t)T.j0 * rb;
        T.bB = T.bA;
    } else if (S.mode == FMV_SWIGLU) {
        const int h = S.R >> 1;
        T.j0 = g * h;
        const int nf = min(h, S.n_rows - T.j0);
        T.hA = nf;
        T.nr = 2 * nf;
        T.bA = S.w + (size_t)T.j0 * rb;
        T.bB = S.w2 + (size_t)T.j0 * rb;
    } else {  // RoPE pairs (d, d + 64) of one 128-wide head
        const int h = S.R >> 1;
        const int lh = 31 - __builtin_clz(h);  // log2 h
        const int ltph = 6 - lh;               // log2 of tiles per head
        T.j0 = ((g >> ltph) << 7) + ((g & ((1 << ltph) - 1)) << lh);
        T.hA = h;
        T.nr = S.R;
        T.bA = S.w + (size_t)T.j0 * rb;
        T.bB = S.w + (size_t)(T.j0 + 64) * rb;
    }
}

__device__ __forceinline__ TileGeo tile_geo(const FmvPlan& P, int g) {
    TileGeo T;
    const int t0 = P.seg[0].tiles, t1 = P.seg[1].tiles;
    if (P.nseg == 1 || g < t0) geo_from_seg(P.seg[0], g, T);
    else if (P.nseg == 2 || g < t0 + t1) geo_from_seg(P.seg[1], g - t0, T);
    else geo_from_seg(P.seg[2], g - t0 - t1, T);
    return T;
}

// 16 bytes from a global address of any alignment (Q6_K blocks are 2-byte
// aligned); the hardware handles the misaligned vector load.
__device__ __forceinline__ uint4 ldg_u16b(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// Q6_K unit (h, l16) from registers: 64 weights at 128h + l16 + i + 32g
// (i < 16, g < 4).  la/lb: ql[64h + l16 ..], ql[64h + 32 + l16 ..]; hq:
// qh[32h + l16 ..]; sc8: bytes 192 + 8h .. +7; d: fp16 bits.  x[2g], x[2g+1]:
// the 16 activations of group g (xperm layout); X[g]: their sum.
__device__ __forceinline__ float q6k_unit_dot_x(const uint4& la4, const uint4& lb4, const uint4& hq4, uint2 sc8,
                                                uint32_t dbits, int l16, const uint4 (&x)[8], const float (&X)[4]) {
    const float d = h2f_bits(dbits);
    const uint32_t la[4] = {la4.x, la4.y, la4.z, la4.w};
    const uint32_t lb[4] = {lb4.x, lb4.y, lb4.z, lb4.w};
    const uint32_t hw[4] = {hq4.x, hq4.y, hq4.z, hq4.w};
    const uint64_t scw = ((uint64_t)sc8.y << 32) | sc8.x;
    const int c = l16 >> 4;
    float r = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 x0 = x[2 * g], x1 = x[2 * g + 1];
        float S = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t l = (g & 1) ? lb[i] : la[i];
            const uint32_t nib = (g < 2) ? (l & 0x0F0F0F0Fu) : ((l >> 4) & 0x0F0F0F0Fu);
            const uint32_t u = nib | (((hw[i] >> (2 * g)) & 0x03030303u) << 4);
            const uint4 xv = (i < 2) ? x0 : x1;
            const uint32_t x02 = (i & 1) ? xv.z : xv.x;
            const uint32_t x13 = (i & 1) ? xv.w : xv.y;
            S = dot4_codes(u, x02, x13, S);
        }
        const int8_t sc = (int8_t)((scw >> (8 * (c + 2 * g))) & 0xFF);
        r = fmaf(d * (float)sc, fmaf(-1056.f, X[g], S), r);
    }
    return r;
}

// Q8_0 unit: two 32-weight blocks (codes qa / qb, fp16 scales in the low /
// high half of dbits) against the 64 activations x (xperm layout) with
// per-16 sums s16.  Signed codes become 128 + q by flipping the sign bit, so
//   sum_i q_i x_i = S - 1152 X,   S = sum (1152 + q_i) x_i (fp16 1024 + (128 + q)),
// and the unit's value is d_a (S_a - 1152 X_a) + d_b (S_b - 1152 X_b), the
// reference's w = d * q (vte/compiler/dequantizer.py:172-196) summed in fp32.
__device__ __forceinline__ float q80_unit_dot_x(const uint4& a0, const uint4& a1, const uint4& b0, const uint4& b1,
                                                uint32_t dbits, const uint4 (&x)[8], const float (&s16)[4]) {
    const uint32_t qa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const uint32_t qb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    float Sa[2] = {0.f, 0.f}, Sb[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // code word j: elements 4j .. 4j+3 of each block
        const uint4 xa = x[j >> 1], xb = x[4 + (j >> 1)];
        const uint32_t xa02 = (j & 1) ? xa.z : xa.x, xa13 = (j & 1) ? xa.w : xa.y;
        const uint32_t xb02 = (j & 1) ? xb.z : xb.x, xb13 = (j & 1) ? xb.w : xb.y;
        Sa[j & 1] = dot4_codes(qa[j] ^ 0x80808080u, xa02, xa13, Sa[j & 1]);
        Sb[j & 1] = dot4_codes(qb[j] ^ 0x80808080u, xb02, xb13, Sb[j & 1]);
    }
    const float r = h2f_bits(dbits) * fmaf(-1152.f, s16[0] + s16[1], Sa[0] + Sa[1]);
    return fmaf(h2f_bits(dbits >> 16), fmaf(-1152.f, s16[2] + s16[3], Sb[0] + Sb[1]), r);
}

// Activations of a Q6_K unit (h, l16) from LDS: xsb -> the super-block's x
// (padded xperm layout), s16sb -> its per-16 sums.
__device__ __forceinline__ void q6k_unit_x(const _Float16* xsb, const float* s16sb, int h, int l16, uint4 (&x)[8],
                                           float (&X)[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4* xp = reinterpret_cast<const uint4*>(xsb + xpad(128 * h + l16 + 32 * g));
        x[2 * g] = xp[0];
        x[2 * g + 1] = xp[1];
        X[g] = s16sb[(128 * h + l16 + 32 * g) >> 4];
    }
}

// Scalar global loads through the global address space (a generic pointer
// would make them flat loads, which also count against the LDS counter).
__device__ __forceinline__ uint32_t ldg_b16(const void* p, size_t i) {
    return ((__attribute__((address_space(1))) const uint16_t*)p)[i];
}
__device__ __forceinline__ uint32_t ldg_b32(const void* p, size_t i) {
    return ((__attribute__((address_space(1))) const uint32_t*)p)[i];
}

__device__ __forceinline__ float row_sum(const float* p, int per_row) {
    const float4* v = reinterpret_cast<const float4*>(p);
    float a = 0.f, b = 0.f;
    int j = 0;
    for (; j + 2 <= per_row / 4; j += 2) {
        const float4 x = v[j], y = v[j + 1];
        a += (x.x + x.y) + (x.z + x.w);
        b += (y.x + y.y) + (y.z + y.w);
    }
    if (j < per_row / 4) {
        const float4 x = v[j];
        a += (x.x + x.y) + (x.z + x.w);
    }
    return a + b;
}

// Activations = the split-KV attention output, combined here from the
// partials: x[m][h*128 + d] = fp16(sum_s w_s o_s[d] / sum_s w_s l_s) with
// w_s = exp(m_s - max_s m_s) over the splits of sequence m (those below its
// length); the same terms as the separate combine kernel.  `wb` holds
// [NC][att_nq][att_S] floats of LDS.
#define TMV_ATT_MAX_S 64
template <int NC>
__device__ __forceinline__ void stage_combine(const FmvPlan& P, _Float16* xs, float* wb, const int* pos_s, int tid) {
    const int M = P.M, nq = P.att_nq, S = P.att_S, K = P.K, ldx = xpad_len(K);
    const int per_col = nq * S;
    for (int i = tid; i < M * per_col; i += ROWS_THREADS) {
        const int m = i / per_col, sidx = i - m * per_col, sp = sidx % S;
        const int ns = (pos_s[m] + 1 + P.att_split - 1) / P.att_split;
        wb[i] = sp < ns ? P.att_m[(size_t)m * per_col + sidx] : -INFINITY;
    }
    __syncthreads();
    if (tid < M * nq) {  // per (sequence, head): normalised split weights
        const int m = tid / nq;
        const int ns = (pos_s[m] + 1 + P.att_split - 1) / P.att_split;
        float* w = wb + (size_t)tid * S;
        const float* l = P.att_l + (size_t)tid * S;
        float mx = -INFINITY;
        for (int sp = 0; sp < ns; ++sp) mx = fmaxf(mx, w[sp]);
        float L = 0.f;
        for (int sp = 0; sp < ns; ++sp) {
            const float e = __expf(w[sp] - mx);
            w[sp] = e;
            L = fmaf(l[sp], e, L);
        }
        const float inv = 1.0f / fmaxf(L, 1e-20f);
        for (int sp = 0; sp < ns; ++sp) w[sp] *= inv;
    }
    __syncthreads();
    for (int j = tid; j < M * K; j += ROWS_THREADS) {
        const int m = j / K, e = j - m * K, h = e >> 7, d = e & 127;
        const int ns = (pos_s[m] + 1 + P.att_split - 1) / P.att_split;
        const float* w = wb + ((size_t)m * nq + h) * S;
        const float* o = P.att_o + (((size_t)m * nq + h) * S) * 128 + d;
        float acc = 0.f;
        int sp = 0;
        for (; sp + 8 <= ns; sp += 8) {
            float v[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = o[(size_t)(sp + t) * 128];
#pragma unroll
            for (int t = 0; t < 8; ++t) acc = fmaf(v[t], w[sp + t], acc);
        }
        for (; sp < ns; ++sp) acc = fmaf(o[(size_t)sp * 128], w[sp], acc);
        xs[(size_t)m * ldx + xpad(xperm(e))] = (_Float16)acc;
    }
    for (int j = tid; j < (NC - M) * K; j += ROWS_THREADS) {  // padding columns
        const int m = M + j / K, e = j % K;
        xs[(size_t)m * ldx + xpad(xperm(e))] = (_Float16)0.f;
    }
}

// The same combine with every global load of a column issued before its
// results are needed (K = KC a multiple of 256 known at compile time): thread
// tid owns dims tid + 256 j; the partial outputs of those dims for the
// first CMB_SC splits, and the split statistics (one (head, split) per
// thread, into LDS), are requested together; after a barrier one thread per
// head turns the statistics into normalised weights; after another the
// thread combines its dims (further rounds of CMB_SC splits if S is larger).
// `wb` holds 2 * att_nq * att_S floats (maxima, then denominators).
#define CMB_SC 9
template <int NC, int KC>
__device__ __forceinline__ void stage_combine_fast(const FmvPlan& P, _Float16* xs, float* wb, const int* pos_s,
                                                   int tid) {
    constexpr int DPT = KC / ROWS_THREADS;
    const int M = NC == 1 ? 1 : P.M, nq = P.att_nq, S = P.att_S, ldx = xpad_len(KC);
    const int per_col = nq * S;
    float* wm = wb;
    float* wl = wb + per_col;
    for (int m = 0; m < M; ++m) {
        const int ns = (pos_s[m] + 1 + P.att_split - 1) / P.att_split;
        const float* om = P.att_o + (size_t)m * per_col * 128;
        float ov[DPT][CMB_SC];
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int d = tid + ROWS_THREADS * j, h = d >> 7;
#pragma unroll
            for (int c = 0; c < CMB_SC; ++c)
                ov[j][c] = om[((size_t)h * S + min(c, S - 1)) * 128 + (d & 127)];
        }
        for (int i = tid; i < per_col; i += ROWS_THREADS) {
            const bool ok = i % S < ns;
            const float mv = P.att_m[(size_t)m * per_col + i], lv = P.att_l[(size_t)m * per_col + i];
            wm[i] = ok ? mv : -INFINITY;
            wl[i] = ok ? lv : 0.f;
        }
        __syncthreads();
        if (tid < nq) {  // head tid: w_s = exp(m_s - max) / sum_s l_s exp(m_s - max)
            float* w = wm + tid * S;
            const float* l = wl + tid * S;
            float mx = -INFINITY;
            for (int sp = 0; sp < ns; ++sp) mx = fmaxf(mx, w[sp]);
            float L = 0.f;
            for (int sp = 0; sp < ns; ++sp) {
                const float e = __expf(w[sp] - mx);
                w[sp] = e;
                L = fmaf(l[sp], e, L);
            }
            const float inv = 1.0f / fmaxf(L, 1e-20f);
            for (int sp = 0; sp < ns; ++sp) w[sp] *= inv;
        }
        __syncthreads();
        float acc[DPT];
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int h = (tid + ROWS_THREADS * j) >> 7;
            acc[j] = 0.f;
#pragma unroll
            for (int c = 0; c < CMB_SC; ++c) acc[j] = c < ns ? fmaf(ov[j][c], wm[h * S + c], acc[j]) : acc[j];
        }
        for (int c0 = CMB_SC; c0 < ns; c0 += CMB_SC) {  // caches of more than CMB_SC splits
#pragma unroll
            for (int j = 0; j < DPT; ++j) {
                const int d = tid + ROWS_THREADS * j, h = d >> 7;
#pragma unroll
                for (int c = 0; c < CMB_SC; ++c)
                    ov[j][c] = om[((size_t)h * S + min(c0 + c, S - 1)) * 128 + (d & 127)];
            }
#pragma unroll
            for (int j = 0; j < DPT; ++j) {
                const int h = (tid + ROWS_THREADS * j) >> 7;
#pragma unroll
                for (int c = 0; c < CMB_SC; ++c)
                    acc[j] = c0 + c < ns ? fmaf(ov[j][c], wm[h * S + min(c0 + c, S - 1)], acc[j]) : acc[j];
            }
        }
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int e = tid + ROWS_THREADS * j;
            xs[(size_t)m * ldx + xpad(xperm(e))] = (_Float16)acc[j];
        }
        if (m + 1 < M) __syncthreads();  // wm / wl are reused by the next column
    }
    for (int j = tid; j < (NC - M) * KC; j += ROWS_THREADS) {  // padding columns
        const int m = M + j / KC, e = j % KC;
        xs[(size_t)m * ldx + xpad(xperm(e))] = (_Float16)0.f;
    }
}

// 32-bit aligned load holding element i of an fp16 (f32 = false) or fp32
// array; returns the element's bits (0 for a null array).  The load is
// unconditional (a null array reads `dummy`), which keeps the vector-memory
// counter the same on every path.
__device__ __forceinline__ uint32_t ld_elem_bits(const void* a, const void* dummy, size_t i, bool f32) {
    const uint8_t* base = reinterpret_cast<const uint8_t*>(a != nullptr ? a : dummy);
    const size_t byte = a != nullptr ? (f32 ? 4 * i : 2 * i) : 0;
    const uint32_t w = ldg_b32(base + (byte & ~(size_t)3), 0);
    const uint32_t v = f32 ? w : ((w >> (8 * (byte & 2))) & 0xFFFFu);
    return a != nullptr ? v : 0u;
}

// Sum of the 8 fp16 values of a 16-byte chunk, in fp32.
__device__ __forceinline__ float chunk_sum(const uint32_t (&h)[4]) {
    float a = rdot2(h[0], 0x3C003C00u, 0.f);
    a = rdot2(h[1], 0x3C003C00u, a);
    a = rdot2(h[2], 0x3C003C00u, a);
    return rdot2(h[3], 0x3C003C00u, a);
}
// Sum of squares of the 8 fp16 values of a chunk, in fp32.
__device__ __forceinline__ float chunk_sumsq(const uint32_t (&h)[4]) {
    float a = rdot2(h[0], h[0], 0.f);
    a = rdot2(h[1], h[1], a);
    a = rdot2(h[2], h[2], a);
    return rdot2(h[3], h[3], a);
}
// value of the lane with the neighbouring index (lane ^ 1)
__device__ __forceinline__ float lane_pair(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
// Chunk (8 fp16, as 4 words) -> fp16(x * inv * w) with w the matching norm weights.
__device__ __forceinline__ void chunk_norm(uint32_t (&h)[4], const uint4& w, float inv) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 lo = (_Float16)(h2f_bits(h[i]) * inv * h2f_bits(ww[i]));
        const _Float16 hi = (_Float16)(h2f_bits(h[i] >> 16) * inv * h2f_bits(ww[i] >> 16));
        h[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
}

// Activation chunks of one staging round: chunk c = c0 + 256 j + tid holds
// x[c / per_col][8 (c % per_col) ..] (columns >= M read as zero) as fp16 words.
template <bool F32, int XR>
struct XChunks {
    uint32_t h[XR][4];
    uint4 w[XR];  // matching norm weights (with a norm)
};

template <int NC, bool F32, int XR>
__device__ __forceinline__ void xr_load(const FmvPlan& P, const void* __restrict__ x, int K, int c0, bool norm,
                                        XChunks<F32, XR>& r, int tid) {
    const int per_col = K / 8;
    const int M = NC == 1 ? 1 : P.M;
    const uint4* nv = reinterpret_cast<const uint4*>(norm ? (const void*)P.norm_w : x);
    uint4 raw[XR][F32 ? 2 : 1];
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = c0 + j * ROWS_THREADS + tid;
        const int m = NC == 1 ? 0 : c / per_col;
        const bool ok = c < NC * per_col && m < M;
        const int cc = ok ? c : 0;
        if (c0 + j * ROWS_THREADS >= NC * per_col) {  // uniform: no lane of this slot has a chunk
            raw[j][0] = raw[j][F32 ? 1 : 0] = r.w[j] = make_uint4(0, 0, 0, 0);
            continue;
        }
        if (F32) {
            const uint4* p = reinterpret_cast<const uint4*>(x) + 2 * (size_t)cc;
            raw[j][0] = p[0];
            raw[j][1] = p[1];
        } else {
            raw[j][0] = reinterpret_cast<const uint4*>(x)[cc];
        }
        r.w[j] = nv[ok ? c - m * per_col : 0];  // unconditional (re-reads x without a norm)
    }
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = c0 + j * ROWS_THREADS + tid;
        const int m = NC == 1 ? 0 : c / per_col;
        const bool ok = c < NC * per_col && m < M;
        if (F32) {
            const uint32_t w[8] = {raw[j][0].x, raw[j][0].y, raw[j][0].z, raw[j][0].w,
                                   raw[j][1].x, raw[j][1].y, raw[j][1].z, raw[j][1].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 lo = (_Float16)__uint_as_float(w[2 * i]);
                const _Float16 hi = (_Float16)__uint_as_float(w[2 * i + 1]);
                r.h[j][i] = ok ? ((uint32_t)__builtin_bit_cast(uint16_t, lo) |
                                  ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16)) : 0u;
            }
        } else {
            r.h[j][0] = ok ? raw[j][0].x : 0u;
            r.h[j][1] = ok ? raw[j][0].y : 0u;
            r.h[j][2] = ok ? raw[j][0].z : 0u;
            r.h[j][3] = ok ? raw[j][0].w : 0u;
        }
    }
}

// Store a round's chunks (fp16) to the padded LDS layout and, when `sums`,
// their per-16 sums (chunks c and c ^ 1 sit in lanes tid and tid ^ 1).
// sums == false stores raw chunks in natural order (to be normalised in LDS).
template <int NC, bool F32, int XR>
__device__ __forceinline__ void xr_store(int K, int c0, const XChunks<F32, XR>& r, _Float16* xs, float* s16,
                                         bool sums, int tid) {
    const int per_col = K / 8, ldx = xpad_len(K);
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = c0 + j * ROWS_THREADS + tid;
        const int m = NC == 1 ? 0 : c / per_col;
        const int cl = c - m * per_col;
        float s = 0.f;
        if (sums) {
            s = chunk_sum(r.h[j]);
            s += lane_pair(s);
        }
        if (c < NC * per_col) {
            uint32_t h0 = r.h[j][0], h1 = r.h[j][1], h2 = r.h[j][2], h3 = r.h[j][3];
            if (sums) {  // final values: the xperm layout; raw chunks (sums == false) stay in natural order
                xperm_words(h0, h1);
                xperm_words(h2, h3);
            }
            *reinterpret_cast<uint4*>(xs + (size_t)m * ldx + xpad(8 * cl)) = make_uint4(h0, h1, h2, h3);
            if (sums && (cl & 1) == 0) s16[m * (K / 16) + (cl >> 1)] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// Per-tile pieces of the kernel: weight loads, epilogue operands, unit dots,
// epilogue; and the block prologue (activation staging)
// ---------------------------------------------------------------------------

// This thread's UPT work units of a tile, loaded straight into registers.
template <int UPT>
struct TileW {
    uint4 w0[UPT], w1[UPT], w2[UPT], w3[UPT];  // w3: Q8_0 only
    uint2 sc8[UPT];
    uint32_t dbits[UPT];
    int usb[UPT];
};

// Unit mapping of a tile (R rows of per_row units):
//  flat (RO false): unit i of this thread is u = tid + 256 i, row u / per_row;
//  range-owned (RO true): thread tid = rg * per_row + kr keeps unit range kr
//    (one 64-weight column slice) for rows rg + G * i, G = 256 / per_row, so
//    its 64 activations are read once and serve all UPT units.
struct UnitPos {
    int lr, kr;  // local row, unit index within the row
};
template <int UPT, bool RO>
__device__ __forceinline__ UnitPos unit_pos(int tid, int i, int per_row) {
    UnitPos p;
    if (RO) {
        const int G = ROWS_THREADS / per_row;
        const int rg = (int)(((float)tid + 0.5f) * (1.0f / (float)per_row));
        p.kr = tid - rg * per_row;
        p.lr = rg < G ? rg + G * i : 0x7fffffff;  // threads past G * per_row hold no unit
    } else {
        const int u = tid + i * ROWS_THREADS;
        const int sbg = u >> 2;
        const int n_sb = per_row >> 2;
        p.lr = (int)(((float)sbg + 0.5f) * (1.0f / (float)n_sb));
        p.kr = u - p.lr * per_row;
    }
    return p;
}

template <int UPT, int FMT, bool RO>
__device__ __forceinline__ void tile_w_issue(TileW<UPT>& W, const TileGeo& T, int n_sb, int per_row, int tid) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        const UnitPos up = unit_pos<UPT, RO>(tid, i, per_row);
        // past the tile's end: re-read its last row
        const int lr = min(up.lr, T.nr - 1);
        const int sb = up.kr >> 2, q = up.kr & 3;
        W.usb[i] = sb;
        const uint8_t* rowp = lr < T.hA ? T.bA + (size_t)lr * T.rb : T.bB + (size_t)(lr - T.hA) * T.rb;
        if (FMT == 4) {
            const uint8_t* blk = rowp + sb * Q4K_BYTES;
            W.w0[i] = ldg_g16(blk);
            W.w1[i] = ldg_g16(blk + 16 + 32 * q);
            W.w2[i] = ldg_g16(blk + 32 + 32 * q);
        } else if (FMT == 8) {  // unit = Q8_0 blocks 2 kr, 2 kr + 1 (68 bytes, 2-byte aligned)
            const uint8_t* blk = rowp + (size_t)up.kr * (2 * Q80_BYTES);
            W.w0[i] = ldg_u16b(blk + 2);
            W.w1[i] = ldg_u16b(blk + 18);
            W.w2[i] = ldg_u16b(blk + Q80_BYTES + 2);
            W.w3[i] = ldg_u16b(blk + Q80_BYTES + 18);
            W.dbits[i] = ldg_b16(blk, 0) | (ldg_b16(blk + Q80_BYTES, 0) << 16);
        } else {
            const uint8_t* blk = rowp + sb * Q6K_BYTES;
            const int h = q >> 1, l16 = (q & 1) * 16;
            W.w0[i] = ldg_u16b(blk + 64 * h + l16);
            W.w1[i] = ldg_u16b(blk + 64 * h + 32 + l16);
            W.w2[i] = ldg_u16b(blk + 128 + 32 * h + l16);
            __builtin_memcpy(&W.sc8[i], blk + 192 + 8 * h, 8);
            W.dbits[i] = ldg_b16(blk + 208, 0);
        }
    }
}

// Epilogue operands of this thread's output (column em, row row1) of a tile.
struct TileE {
    int em, row1;
    bool eth;
    uint32_t b1, b2, res, cb, sbits;
};

// Output slot and bias / residual (unconditional loads: read as 0 when absent).
template <int NC>
__device__ __forceinline__ void tile_e_issue(TileE& E, const FmvPlan& P, const TileGeo& T, int M, const void* dummy,
                                             int tid) {
    const bool paired = fmv_paired(T.mode);
    const int nout = paired ? T.hA : T.nr;  // outputs (per column) of the tile
    E.eth = tid < M * nout;                 // M * nout <= 256 (checked on the host)
    const int tt = E.eth ? tid : 0;
    // tt / nout for tt < 256, nout <= 256: the float quotient is exact enough
    E.em = NC == 1 ? 0 : (int)(((float)tt + 0.5f) * (1.0f / (float)nout));
    E.row1 = T.j0 + (tt - E.em * nout);
    const bool f32o = T.mode == FMV_STORE_F32;
    E.b1 = ld_elem_bits(T.bias, dummy, E.row1, f32o);
    E.b2 = ld_elem_bits(paired ? T.bias : nullptr, dummy, E.row1 + 64, false);
    E.res = ld_elem_bits(T.residual, dummy, (size_t)E.em * T.n_rows + E.row1, f32o);
}

// cos/sin of the output's position (read as 0 when the mode has no rotation).
__device__ __forceinline__ void tile_e_rope(TileE& E, const FmvPlan& P, const TileGeo& T, int pos,
                                            const void* dummy) {
    const bool rope = T.mode == FMV_ROPE_Q || T.mode == FMV_ROPE_KCACHE;
    const size_t ci = rope ? (size_t)pos * 128 + (E.row1 & 127) : 0;
    E.cb = ld_elem_bits(rope ? (const void*)P.rope_cos : nullptr, dummy, ci, false);
    E.sbits = ld_elem_bits(rope ? (const void*)P.rope_sin : nullptr, dummy, ci, false);
}

// The units' partials for every column -> part[m * pstride + unit].
template <int NC, int UPT, int FMT, bool RO>
__device__ __forceinline__ void tile_dot(const TileW<UPT>& W, int nr, int per_row, int K, const _Float16* xs,
                                         const float* s16, float* part, int pstride, int tid) {
    const int ldx = xpad_len(K);
    uint4 x[NC][8];
    float xs16[NC][4];
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        const UnitPos up = unit_pos<UPT, RO>(tid, i, per_row);
        const int q = up.kr & 3, sb = up.kr >> 2;
        const int h = q >> 1, l16 = (q & 1) * 16;
        if (!RO || i == 0) {  // range-owned: the unit range, hence x, is the same for every i
#pragma unroll
            for (int m = 0; m < NC; ++m) {
                if (FMT == 4 || FMT == 8)
                    q4k_unit_x(xs + (size_t)m * ldx + xpad(sb * QK_K + 64 * q), s16 + m * (K / 16) + sb * 16 + 4 * q,
                               x[m], xs16[m]);
                else
                    q6k_unit_x(xs + (size_t)m * ldx + xpad(sb * QK_K), s16 + m * (K / 16) + sb * 16, h, l16, x[m],
                               xs16[m]);
            }
        }
        if (up.lr < nr) {
            const int u = up.lr * per_row + up.kr;
            if (FMT == 4) {
                const Q4KUnitData d{W.w0[i], W.w1[i], W.w2[i]};
#pragma unroll
                for (int m = 0; m < NC; ++m) part[m * pstride + u] = q4k_unit_dot_x(d, q, x[m], xs16[m]);
            } else if (FMT == 8) {
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * pstride + u] = q80_unit_dot_x(W.w0[i], W.w1[i], W.w2[i], W.w3[i], W.dbits[i], x[m],
                                                           xs16[m]);
            } else {
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * pstride + u] = q6k_unit_dot_x(W.w0[i], W.w1[i], W.w2[i], W.sc8[i], W.dbits[i], l16,
                                                           x[m], xs16[m]);
            }
        }
    }
}

// One output per thread (threads with E.eth): row sums of the partials and
// the mode's epilogue.
template <int NC>
__device__ __forceinline__ void tile_epilogue(const FmvPlan& P, const TileGeo& T, const TileE& E, const float* part,
                                              int pstride, int per_row, const int* pos_s) {
    if (!E.eth) return;
    const int em = E.em, row1 = E.row1;
    const int er = row1 - T.j0;
    const bool f32o = T.mode == FMV_STORE_F32;
    if (!fmv_paired(T.mode)) {
        float v = row_sum(part + em * pstride + er * per_row, per_row) +
                  (f32o ? __uint_as_float(E.b1) : h2f_bits(E.b1));
        if (T.mode == FMV_VCACHE) {
            P.v_cache[(size_t)em * P.kv_batch_stride + ((size_t)pos_s[em] * P.n_kv + row1 / 128) * 128 +
                      (row1 % 128)] = __float2half(v);
            return;
        }
        v = v * P.rs + (f32o ? __uint_as_float(E.res) : h2f_bits(E.res));
        const size_t oi = (size_t)em * T.n_rows + row1;
        if (f32o) reinterpret_cast<float*>(T.out)[oi] = v;
        else reinterpret_cast<__half*>(T.out)[oi] = __float2half(v);
        return;
    }
    const float a = row_sum(part + em * pstride + er * per_row, per_row);
    const float bv = row_sum(part + em * pstride + (er + T.hA) * per_row, per_row);
    if (T.mode == FMV_SWIGLU) {
        const float gg = __half2float(__float2half(a));
        const float uu = __half2float(__float2half(bv));
        const float sig = 1.0f / (1.0f + expf(-gg));
        reinterpret_cast<__half*>(T.out)[(size_t)em * T.n_rows + row1] = __float2half(gg * sig * uu);
        return;
    }
    const float x1 = __half2float(__float2half(a + h2f_bits(E.b1)));
    const float x2 = __half2float(__float2half(bv + h2f_bits(E.b2)));
    const float c = h2f_bits(E.cb), sn = h2f_bits(E.sbits);
    const __half o1 = __float2half(x1 * c - x2 * sn), o2 = __float2half(x1 * sn + x2 * c);
    if (T.mode == FMV_ROPE_Q) {
        __half* qo = reinterpret_cast<__half*>(T.out) + (size_t)em * T.n_rows;
        qo[row1] = o1;
        qo[row1 + 64] = o2;
    } else {
        const int d = row1 & 127;
        __half* kc = P.k_cache + (size_t)em * P.kv_batch_stride + ((size_t)pos_s[em] * P.n_kv + row1 / 128) * 128;
        kc[d] = o1;
        kc[d + 64] = o2;
    }
}

// LDS layout of a block: x [NC][ldx] fp16 | s16 [NC][K/16] | part [NC][UPT * 256]
// | combine weights (attention-output source only).
struct FmvLDS {
    _Float16* xs;
    float* s16;
    float* part;
};

__device__ __forceinline__ FmvLDS fmv_lds(uint8_t* lds, int NC, int K, int UPT) {
    FmvLDS L;
    L.xs = reinterpret_cast<_Float16*>(lds);
    size_t o = ((size_t)NC * xpad_len(K) * 2 + 15) & ~(size_t)15;
    L.s16 = reinterpret_cast<float*>(lds + o);
    o += (size_t)NC * (K / 16) * 4;
    o = (o + 15) & ~(size_t)15;
    L.part = reinterpret_cast<float*>(lds + o);
    return L;
}

// Block prologue: kv offsets -> pos_s, activations (RMSNorm-ed when the plan
// has a norm, or combined from split-KV partials) and their per-16 sums into
// LDS.  The activations are requested first; `issue()` runs right after the
// first barrier (the activations are in), so the caller's weight loads do not
// queue ahead of them; the normalisation then runs while those are in flight.
// Ends with a barrier.
template <int NC, bool F32, int KC, bool ATT, typename IssueFn>
__device__ __forceinline__ void fmv_prologue(const void* __restrict__ x, const FmvPlan& P, const FmvLDS& L,
                                             float* wb, float (*red)[NC], int* pos_s, IssueFn issue) {
    const int K = KC > 0 ? KC : P.K, M = NC == 1 ? 1 : P.M;
    const int ldx = xpad_len(K);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    constexpr bool att_src = ATT;  // the launcher sets ATT exactly when P.att_o != nullptr
    const bool norm = P.norm_w != nullptr;
    const void* dummy = P.seg[0].w;
    const int pos_reg = (int)ld_elem_bits(P.kv_offset, dummy, min(tid, M - 1), true);

    constexpr int XR = F32 ? 4 : 8;
    const int nchx = NC * (K / 8);
    const bool one_round = nchx <= XR * ROWS_THREADS;
    XChunks<F32, XR> xr;
    float ss[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) ss[m] = 0.f;
    if (!att_src) {
        for (int c0 = 0; c0 < nchx; c0 += XR * ROWS_THREADS) {
            xr_load<NC, F32, XR>(P, x, K, c0, norm, xr, tid);
            if (norm) {
#pragma unroll
                for (int j = 0; j < XR; ++j) {
                    const int c = c0 + j * ROWS_THREADS + tid;
                    const int m = NC == 1 ? 0 : c / (K / 8);
                    const float q = chunk_sumsq(xr.h[j]);
#pragma unroll
                    for (int mm = 0; mm < NC; ++mm) ss[mm] += (m == mm) ? q : 0.f;
                }
                // one round: the chunks stay in registers until the scale is known
                if (!one_round) xr_store<NC, F32, XR>(K, c0, xr, L.xs, L.s16, false, tid);
            } else {
                xr_store<NC, F32, XR>(K, c0, xr, L.xs, L.s16, true, tid);
            }
        }
        if (norm) {
#pragma unroll
            for (int m = 0; m < NC; ++m) {
                ss[m] = wave_sum(ss[m]);
                if (lane == 0) red[wv][m] = ss[m];
            }
        }
    }
    if (tid < M) pos_s[tid] = pos_reg;
    __syncthreads();
    issue();

    if constexpr (att_src) {
        if constexpr (KC > 0 && KC % ROWS_THREADS == 0) stage_combine_fast<NC, KC>(P, L.xs, wb, pos_s, tid);
        else stage_combine<NC>(P, L.xs, wb, pos_s, tid);
        __syncthreads();
        act_sums<NC>(ActLDS{L.xs, L.s16}, K);
    } else if (norm) {
        float inv[NC];
#pragma unroll
        for (int m = 0; m < NC; ++m)
            inv[m] = rsqrtf((red[0][m] + red[1][m] + red[2][m] + red[3][m]) / (float)K + P.eps);
        if (one_round) {
#pragma unroll
            for (int j = 0; j < XR; ++j) {
                const int c = j * ROWS_THREADS + tid;
                const int m = NC == 1 ? 0 : c / (K / 8);
                float iv = inv[0];
#pragma unroll
                for (int mm = 1; mm < NC; ++mm) iv = (m == mm) ? inv[mm] : iv;
                chunk_norm(xr.h[j], xr.w[j], iv);
            }
            xr_store<NC, F32, XR>(K, 0, xr, L.xs, L.s16, true, tid);
        } else {  // raw chunks are in LDS: scale them there
            const int per_col = K / 8;
            const uint4* nv = reinterpret_cast<const uint4*>(P.norm_w);
            for (int c = tid; c - tid < nchx; c += ROWS_THREADS) {
                const bool ok = c < nchx;
                const int m = ok ? c / per_col : 0, cl = ok ? c - m * per_col : 0;
                float iv = inv[0];
#pragma unroll
                for (int mm = 1; mm < NC; ++mm) iv = (m == mm) ? inv[mm] : iv;
                uint4* px = reinterpret_cast<uint4*>(L.xs + (size_t)m * ldx + xpad(8 * cl));
                const uint4 v = *px;
                uint32_t h[4] = {v.x, v.y, v.z, v.w};
                chunk_norm(h, nv[cl], iv);
                float s = chunk_sum(h);
                s += lane_pair(s);
                xperm_words(h[0], h[1]);
                xperm_words(h[2], h[3]);
                if (ok) {
                    *px = make_uint4(h[0], h[1], h[2], h[3]);
                    if ((cl & 1) == 0) L.s16[m * (K / 16) + (cl >> 1)] = s;
                }
            }
        }
    }
    __syncthreads();
}

// One tile per block (grid = tiles): everything a block reads is requested
// up front, so a block costs about one memory latency plus its arithmetic.
template <int NC, bool F32, int UPT, int FMT, int KC, bool RO, bool ATT, bool WF>
__device__ __forceinline__ void tmv_body(const void* __restrict__ x, const FmvPlan& P, const TileGeo& T,
                                         uint8_t* lds, float (*red)[NC], int* pos_s) {
    const int K = KC > 0 ? KC : P.K, M = NC == 1 ? 1 : P.M;
    const int n_sb = K / QK_K, per_row = n_sb * 4;
    const FmvLDS L = fmv_lds(lds, NC, K, UPT);
    const int pstride = UPT * ROWS_THREADS;
    float* wb = L.part + (size_t)NC * pstride;
    const int tid = threadIdx.x;
    const void* dummy = P.seg[0].w;
    TileE E;
    tile_e_issue<NC>(E, P, T, M, dummy, tid);
    TileW<UPT> W;
    if constexpr (WF) tile_w_issue<UPT, FMT, RO>(W, T, n_sb, per_row, tid);
    fmv_prologue<NC, F32, KC, ATT>(x, P, L, wb, red, pos_s, [&]() {
        if constexpr (!WF) tile_w_issue<UPT, FMT, RO>(W, T, n_sb, per_row, tid);
        tile_e_rope(E, P, T, pos_s[E.em], dummy);  // kv offsets are in LDS after the first barrier
    });
    tile_dot<NC, UPT, FMT, RO>(W, T.nr, per_row, K, L.xs, L.s16, L.part, pstride, tid);
    __syncthreads();
    tile_epilogue<NC>(P, T, E, L.part, pstride, per_row, pos_s);
}

// KC: the activation length K when fixed at compile time (0: P.K), so the
// staging, norm and row-sum loops have constant trip counts and no divisions.
// RO: range-owned unit mapping (see unit_pos).
// ATT: activations combined from split-KV partials (a separate instantiation:
// the combine's registers would otherwise lower every mat-vec's occupancy).
// WF: the tile's weight loads are issued before the activation loads (one
// memory round trip per block instead of two, but the activations then queue
// behind the weights): faster for launches of many tiles (the LM head),
// slower for the short launches of the decode step.
template <int NC, bool F32, int UPT, int KC, bool RO, bool ATT = false, bool WF = false>
__global__ __launch_bounds__(ROWS_THREADS) void fused_mv_kernel(const void* __restrict__ x, FmvPlan P) {
    extern __shared__ uint4 smem_fmv[];
    __shared__ float red[4][NC];
    __shared__ int pos_s[NC];
    const TileGeo T = tile_geo(P, blockIdx.x);
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem_fmv);
    if (T.fmt == 4) tmv_body<NC, F32, UPT, 4, KC, RO, ATT, WF>(x, P, T, lds, red, pos_s);
    else if (ATT || WF || T.fmt == 6) tmv_body<NC, F32, UPT, 6, KC, RO, ATT, WF>(x, P, T, lds, red, pos_s);
    else tmv_body<NC, F32, UPT, 8, KC, RO, ATT, WF>(x, P, T, lds, red, pos_s);
}

// Range-owned mapping when a row's units fill the block's threads with at
// most 1/16 of them idle (e.g. K = 1536: 24 units per row, 240 of 256
// threads); otherwise (e.g. K = 8960) the flat mapping.
__host__ __device__ inline bool fmv_ro(int K) {
    const int per_row = (K / QK_K) * 4;
    return per_row <= 64 && (ROWS_THREADS % per_row) * 16 <= ROWS_THREADS;
}

template <int NC, bool F32, int KC, bool RO>
static void fmv_launch_k(int upt, int total, size_t lds, hipStream_t st, const void* x, const FmvPlan& plan) {
    const dim3 g(total), b(ROWS_THREADS);
    if constexpr (!F32 && KC != 8960) {  // attention-output activations (o-proj): fp16 path, K = q_dim
        if (plan.att_o != nullptr) {
            if (upt == 4) hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 4, KC, RO, true>), g, b, lds, st, x, plan);
            else if (upt == 2) hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 2, KC, RO, true>), g, b, lds, st, x, plan);
            else hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 1, KC, RO, true>), g, b, lds, st, x, plan);
            return;
        }
    }
    if constexpr (KC == 1536 && RO) {  // weights-first form for launches of many tiles
        if (upt == 4 && plan.wfirst) {
            hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 4, KC, RO, false, true>), g, b, lds, st, x, plan);
            return;
        }
    }
    if (upt == 4) hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 4, KC, RO>), g, b, lds, st, x, plan);
    else if (upt == 2) hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 2, KC, RO>), g, b, lds, st, x, plan);
    else hipLaunchKernelGGL((fused_mv_kernel<NC, F32, 1, KC, RO>), g, b, lds, st, x, plan);
}

// Launch of one tile per block for fp32 activations (fused_f32.hip).
namespace vte {
void fmv_launch_x32(int NC, int upt, int total, size_t lds, hipStream_t st, const void* x, const FmvPlan& plan);
}

