// Batched (3 or more columns) projections with the decode-step glue fused in, on MFMA
// (gfx950).  One launch per group of projections that read the same
// (already RMSNorm-ed, fp16) activations:
//
//   q/k/v (+bias) -> RoPE(q, k) -> K/V cache append       => one launch
//   gate/up -> SwiGLU                                       => one launch
//
// (reference nodes: vte/compiler/qwen_compute.py:100-282, captured by
// vte/core/hip_graph_executor.py:504-738), with the rounding points of those
// nodes: projections (+bias) and rotated q/k are fp16 values computed in fp32,
// SwiGLU is fp16(g / (1 + exp(-g)) * u) on fp16 g and u
// (rope.hip.template:82-97, swiglu.hip.template:11-25).
//
// Tiles are 16 * RT weight rows; paired tiles hold 8 * RT rows and their
// partners (RoPE: d and d + 64 of one head; SwiGLU: gate row j and up row j),
// so a pair's two sums finish in the same block.  The weight operand of each
// lane comes from its tile row's weight row; everything else is the batched
// MFMA GEMM (waves split K, partial C tiles summed through LDS), whose k-slot
// map, exact operands and per-super-block scaling it shares (mfma_deq.h).
#include <cstdlib>
#include <cstring>

#include "mfma_deq.h"

#define MM_MAX_SEG 3


enum MmMode : int {
    MM_STORE = 0,        // out[m][row] = fp16(acc + bias)
    MM_ROPE_Q = 2,       // fp16(acc + bias), rotated -> out (q [m][rows])
    MM_ROPE_KCACHE = 3,  // fp16(acc + bias), rotated -> k_cache at kv_offset[m]
    MM_VCACHE = 4,       // fp16(acc + bias) -> v_cache at kv_offset[m]
    MM_SWIGLU = 5,       // gate rows of w, up rows of w2: out[m][j] = fp16(silu(g) * u)
};

struct MmSeg {
    const uint8_t* w;
    const uint8_t* w2;   // up rows (SwiGLU)
    __half* out;
    const __half* bias;  // nullable
    int fmt;             // 4 = Q4_K, 6 = Q6_K
    int n_rows;          // output rows (SwiGLU: outputs, i.e. gate rows)
    int mode;
    int tiles;
    int row_bytes;
};

struct MmPlan {
    MmSeg seg[MM_MAX_SEG];
    int nseg;
    int K, M;            // activations [M][K] fp16, M <= 16 * NT in one launch
    const __half* x;
    const __half* rope_cos;
    const __half* rope_sin;
    const int* kv_offset;  // [M] positions of this launch's columns
    __half* k_cache;       // sequence m at k_cache + m * kv_batch_stride
    __half* v_cache;
    int kv_batch_stride;
    int n_kv;
};

__host__ __device__ __forceinline__ bool mm_paired(int mode) {
    return mode == MM_ROPE_Q || mode == MM_ROPE_KCACHE || mode == MM_SWIGLU;
}

// Tile of a block: `pr` pairs (paired) or 16*RT rows starting at j0.
struct MmTile {
    const MmSeg* S;
    int j0;      // first row (paired: first A row)
    int nvalid;  // valid rows (not paired) or pairs (paired)
};

template <int RT>
__device__ __forceinline__ MmTile mm_tile(const MmPlan& P, int g) {
    MmTile T;
    const int t0 = P.seg[0].tiles, t1 = P.seg[1].tiles;
    int s = 0;
    if (P.nseg > 1 && g >= t0) {
        g -= t0;
        s = 1;
        if (P.nseg > 2 && g >= t1) {
            g -= t1;
            s = 2;
        }
    }
    const MmSeg& S = P.seg[s];
    T.S = &P.seg[s];
    if (!mm_paired(S.mode)) {
        T.j0 = g * 16 * RT;
        T.nvalid = min(16 * RT, S.n_rows - T.j0);
    } else if (S.mode == MM_SWIGLU) {
        T.j0 = g * 8 * RT;
        T.nvalid = min(8 * RT, S.n_rows - T.j0);
    } else {  // RoPE: 8 * RT pairs (d, d + 64) of one 128-row head
        const int tph = 64 / (8 * RT);  // tiles per head
        T.j0 = (g / tph) * 128 + (g % tph) * 8 * RT;
        T.nvalid = 8 * RT;
    }
    return T;
}

// Weight row of tile row rr (past the valid rows: a valid row, results unused).
template <int RT>
__device__ __forceinline__ const uint8_t* mm_row(const MmTile& T, int rr) {
    const MmSeg& S = *T.S;
    if (!mm_paired(S.mode)) return S.w + (size_t)(T.j0 + min(rr, T.nvalid - 1)) * S.row_bytes;
    const int p = rr % (8 * RT), pc = min(p, T.nvalid - 1);
    if (rr < 8 * RT) return S.w + (size_t)(T.j0 + pc) * S.row_bytes;
    if (S.mode == MM_SWIGLU) return S.w2 + (size_t)(T.j0 + pc) * S.row_bytes;
    return S.w + (size_t)(T.j0 + 64 + pc) * S.row_bytes;
}

template <int FMT, int RT, int NT, int NW>
__device__ __forceinline__ void mm_body(const MmPlan& P, const MmTile& T, float (*red)[RT][NT][4][64],
                                        float (*xl)[NT * 128]) {
    constexpr bool XM = NT > 1;  // minimum-term form (q4_xmin)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int K = P.K, M = P.M, n_sb = K / QK_K;
    const int sb0 = (n_sb * wv) / NW, sb1 = (n_sb * (wv + 1)) / NW;
    const __half* x = P.x;

    floatx4_t acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    const uint8_t* rowp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) rowp[rt] = mm_row<RT>(T, rt * 16 + col);

    for (int sb = sb0; sb < sb1; ++sb) {
        half8_t bx[8][NT];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int kb = sb * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int m = nt * 16 + col;
                bx[t][nt] = load_x8<__half>(x + (size_t)(m < M ? m : 0) * K + kb, m < M);
            }
        }
        // weights requested before the minimum-term LDS round trip, whose
        // memory clobber would otherwise hold them back
        typename SbRaw<FMT>::Raw raw[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            sb_load(rowp[rt] + (size_t)sb * (FMT == 4 ? Q4K_BYTES : Q6K_BYTES), grp, raw[rt]);
        XMin<NT, XM> xm;
        sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            typename SbRaw<FMT>::Ops ops;
            sb_ops<XM>(raw[rt], grp, ops);
            sb_mfma<NT>(ops, bx, xm, acc[rt]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wv][rt][nt][i][lane] = acc[rt][nt][i];
}

// Sum over the NW waves of tile row rr, batch column mc (C layout: lane
// (row rw, grp) holds batch columns 4*grp+i of a 16-column tile).
template <int RT, int NT, int NW>
__device__ __forceinline__ float mm_sum(float (*red)[RT][NT][4][64], int rr, int mc) {
    const int rt = rr >> 4, rw = rr & 15, nt = mc >> 4, cc = mc & 15;
    const int ln = c_lane(rw, cc), i = c_reg(cc);
    float s = 0.f;
#pragma unroll
    for (int wq = 0; wq < NW; ++wq) s += red[wq][rt][nt][i][ln];
    return s;
}

__device__ __forceinline__ float mm_bias(const __half* b, int row) { return b ? __half2float(b[row]) : 0.f; }

// Epilogue of one C tile group: batch columns cb .. cb + mcount - 1 of the
// launch (column m reads kv_offset[m] and writes row m of the outputs).
template <int RT, int NT, int NW>
__device__ __forceinline__ void mm_epilogue(const MmPlan& P, const MmTile& T, float (*red)[RT][NT][4][64], int cb,
                                            int mcount) {
    const MmSeg& S = *T.S;
    if (!mm_paired(S.mode)) {
        for (int o = threadIdx.x; o < 16 * RT * 16 * NT; o += blockDim.x) {
            const int rr = o / (16 * NT), mc = o % (16 * NT);
            if (rr >= T.nvalid || mc >= mcount) continue;
            const int row = T.j0 + rr, m = cb + mc;
            const __half v = __float2half(mm_sum<RT, NT, NW>(red, rr, mc) + mm_bias(S.bias, row));
            if (S.mode == MM_VCACHE) {
                const int pos = P.kv_offset[m];
                P.v_cache[(size_t)m * P.kv_batch_stride + ((size_t)pos * P.n_kv + row / 128) * 128 + (row % 128)] = v;
            } else {
                S.out[(size_t)m * S.n_rows + row] = v;
            }
        }
        return;
    }
    for (int o = threadIdx.x; o < 8 * RT * 16 * NT; o += blockDim.x) {
        const int p = o / (16 * NT), mc = o % (16 * NT);
        if (p >= T.nvalid || mc >= mcount) continue;
        const float a = mm_sum<RT, NT, NW>(red, p, mc), b = mm_sum<RT, NT, NW>(red, p + 8 * RT, mc);
        const int row = T.j0 + p, m = cb + mc;
        if (S.mode == MM_SWIGLU) {
            const float g = __half2float(__float2half(a)), u = __half2float(__float2half(b));
            S.out[(size_t)m * S.n_rows + row] = __float2half(g / (1.0f + expf(-g)) * u);
            continue;
        }
        const float x1 = __half2float(__float2half(a + mm_bias(S.bias, row)));
        const float x2 = __half2float(__float2half(b + mm_bias(S.bias, row + 64)));
        const int pos = P.kv_offset[m], d = row & 127;
        const float c = __half2float(P.rope_cos[(size_t)pos * 128 + d]);
        const float sn = __half2float(P.rope_sin[(size_t)pos * 128 + d]);
        const __half o1 = __float2half(x1 * c - x2 * sn), o2 = __float2half(x1 * sn + x2 * c);
        if (S.mode == MM_ROPE_Q) {
            S.out[(size_t)m * S.n_rows + row] = o1;
            S.out[(size_t)m * S.n_rows + row + 64] = o2;
        } else {
            __half* kc = P.k_cache + (size_t)m * P.kv_batch_stride + ((size_t)pos * P.n_kv + row / 128) * 128;
            kc[d] = o1;
            kc[d + 64] = o2;
        }
    }
}

// NW waves per block split K (6 for K = 1536: one super-block each).
template <int RT, int NT, int NW>
__global__ __launch_bounds__(64 * NW) void fused_mm_kernel(MmPlan P) {
    __shared__ float red[NW][RT][NT][4][64];
    __shared__ float xl[NW][NT * 128];  // minimum-term scratch per wave (q4_xmin)
    const MmTile T = mm_tile<RT>(P, blockIdx.x);
    const MmSeg& S = *T.S;
    if (S.fmt == 4) mm_body<4, RT, NT, NW>(P, T, red, xl);
    else mm_body<6, RT, NT, NW>(P, T, red, xl);
    __syncthreads();

    mm_epilogue<RT, NT, NW>(P, T, red, 0, P.M);
}


// Weight-stationary form for long batches (prefill chunks), K = 6 super-blocks:
// wave w decodes super-block w of its tile rows once, keeps the weight
// operands in registers and runs them against the block's columns
// [blockIdx.y * cols, ...) 16 * NT at a time; the next columns' activations
// are requested before the epilogue of the current ones.  Each C tile sums
// its eight k-steps in the same order as fused_mm_kernel, so both forms give
// the same bits.
template <int FMT, int RT, int NT>
__device__ __forceinline__ void mm_ws_body(const MmPlan& P, const MmTile& T, float (*red)[RT][NT][4][64],
                                           float (*xl)[NT * 128], int c0,
                                           int c1) {
    constexpr bool XM = true;  // minimum-term form (q4_xmin)
    constexpr int NW = 6;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int K = P.K;
    typename SbRaw<FMT>::Ops ops[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint8_t* rowp = mm_row<RT>(T, rt * 16 + col);
        typename SbRaw<FMT>::Raw raw;
        sb_load(rowp + (size_t)wv * (FMT == 4 ? Q4K_BYTES : Q6K_BYTES), grp, raw);
        sb_ops<XM>(raw, grp, ops[rt]);
    }
    half8_t bx[8][NT];
    auto load_b = [&](int m0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int kb = wv * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int m = m0 + nt * 16 + col;
                bx[t][nt] = load_x8<__half>(P.x + (size_t)(m < c1 ? m : c0) * K + kb, m < c1);
            }
        }
    };
    load_b(c0);
    for (int m0 = c0; m0 < c1; m0 += 16 * NT) {
        floatx4_t acc[RT][NT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        XMin<NT, XM> xm;
        sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sb_mfma<NT>(ops[rt], bx, xm, acc[rt]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wv][rt][nt][i][lane] = acc[rt][nt][i];
        if (m0 + 16 * NT < c1) load_b(m0 + 16 * NT);
        __syncthreads();
        mm_epilogue<RT, NT, NW>(P, T, red, m0, min(16 * NT, c1 - m0));
        __syncthreads();
    }
}

template <int RT, int NT>
__global__ __launch_bounds__(64 * 6) void fused_mm_ws_kernel(MmPlan P, int cols) {
    __shared__ float red[6][RT][NT][4][64];
    __shared__ float xl[6][NT * 128];
    const MmTile T = mm_tile<RT>(P, blockIdx.x);
    const int c0 = blockIdx.y * cols, c1 = min(P.M, c0 + cols);
    if (c0 >= c1) return;
    if (T.S->fmt == 4) mm_ws_body<4, RT, NT>(P, T, red, xl, c0, c1);
    else mm_ws_body<6, RT, NT>(P, T, red, xl, c0, c1);
}

namespace vte {

static MmSeg mm_seg(const void* w, const void* w2, void* out, const void* bias, int fmt, int n_rows, int mode, int K,
                    int RT) {
    MmSeg S;
    memset(&S, 0, sizeof(S));
    S.w = (const uint8_t*)w;
    S.w2 = (const uint8_t*)w2;
    S.out = (__half*)out;
    S.bias = (const __half*)bias;
    S.fmt = fmt;
    S.n_rows = n_rows;
    S.mode = mode;
    S.row_bytes = (K / QK_K) * (fmt == 4 ? Q4K_BYTES : Q6K_BYTES);
    if (mode == MM_SWIGLU) S.tiles = (n_rows + 8 * RT - 1) / (8 * RT);
    else if (mode == MM_ROPE_Q || mode == MM_ROPE_KCACHE) S.tiles = n_rows / (8 * RT) / 2;
    else S.tiles = (n_rows + 16 * RT - 1) / (16 * RT);
    return S;
}

static int mm_env(const char* name, int dflt) {
    const char* v = getenv(name);
    return v ? atoi(v) : dflt;
}

// Runs the plan over the batch: in chunks of 32 columns (one launch each), or
// in one weight-stationary launch when the batch is longer than 32 columns.
template <int RT>
static hipError_t mm_run(MmPlan P, int B, size_t out_ld_elems[MM_MAX_SEG], hipStream_t st) {
    int total = 0;
    for (int s = 0; s < P.nseg; ++s) total += P.seg[s].tiles;
    const __half* x0 = P.x;
    const int* ko0 = P.kv_offset;
    __half* out0[MM_MAX_SEG];
    for (int s = 0; s < P.nseg; ++s) out0[s] = P.seg[s].out;
    __half* kc0 = P.k_cache;
    __half* vc0 = P.v_cache;
    if constexpr (RT == 4) if (B > 32 && P.K == 6 * QK_K && mm_env("VTE_MM_WS", 1)) {
        // 64 rows per block, 16 columns at a time: one block per CU
        const int g = ws_column_groups(total, B, device_cus());
        const int cols = ((B + 31) / 32 + g - 1) / g * 32, gy = (B + cols - 1) / cols;
        P.M = B;
        hipLaunchKernelGGL((fused_mm_ws_kernel<RT, 1>), dim3(total, gy), dim3(64 * 6), 0, st, P, cols);
        return hipGetLastError();
    }
    if constexpr (RT <= 2) if (B > 32 && P.K == 6 * QK_K && mm_env("VTE_MM_WS", 1)) {
        // two 6-wave blocks fit per CU
        const int g = ws_column_groups(total, B, 2 * device_cus());
        const int cols = ((B + 31) / 32 + g - 1) / g * 32, gy = (B + cols - 1) / cols;
        P.M = B;
        hipLaunchKernelGGL((fused_mm_ws_kernel<RT, 2>), dim3(total, gy), dim3(64 * 6), 0, st, P, cols);
        return hipGetLastError();
    }
    for (int m0 = 0; m0 < B; m0 += 32) {
        const int mc = B - m0 < 32 ? B - m0 : 32;
        P.M = mc;
        P.x = x0 + (size_t)m0 * P.K;
        P.kv_offset = ko0 ? ko0 + m0 : nullptr;
        for (int s = 0; s < P.nseg; ++s) P.seg[s].out = out0[s] ? out0[s] + (size_t)m0 * out_ld_elems[s] : nullptr;
        P.k_cache = kc0 ? kc0 + (size_t)m0 * P.kv_batch_stride : nullptr;
        P.v_cache = vc0 ? vc0 + (size_t)m0 * P.kv_batch_stride : nullptr;
        // batches above 16 columns take the two-tile form for every chunk, a
        // short tail included, so all their columns share the minimum-term
        // form (and the bits) of the weight-stationary launch
        if (P.K == 6 * QK_K) {
            if (B > 16) hipLaunchKernelGGL((fused_mm_kernel<RT, 2, 6>), dim3(total), dim3(64 * 6), 0, st, P);
            else hipLaunchKernelGGL((fused_mm_kernel<RT, 1, 6>), dim3(total), dim3(64 * 6), 0, st, P);
        } else {
            if (B > 16) hipLaunchKernelGGL((fused_mm_kernel<RT, 2, MF_WAVES>), dim3(total), dim3(64 * MF_WAVES), 0, st, P);
            else hipLaunchKernelGGL((fused_mm_kernel<RT, 1, MF_WAVES>), dim3(total), dim3(64 * MF_WAVES), 0, st, P);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// q/k/v projections of RMSNorm-ed fp16 activations xn [B][K] with bias, RoPE
// on q and k, and the K/V rows written at kv_offset[b]; q_out [B][n_q*128].
hipError_t qkv_mm(const void* xn, const void* wq, const void* q_bias, int fmt_q, const void* wk, const void* k_bias,
                  int fmt_k, const void* wv, const void* v_bias, int fmt_v, void* q_out, void* k_cache, void* v_cache,
                  const int* kv_offset, int kv_batch_stride, const void* rope_cos, const void* rope_sin, int B, int K,
                  int n_q, int n_kv, hipStream_t st) {
    // 64 rows per block from 129 columns (2048-token prefill in chunks of 512:
    // 38.5 -> 37.2 ms; chunks of 64-128 are faster with 16)
    const int RT = mm_env("VTE_MM_RT_QKV", B > 128 ? 4 : 1);
    MmPlan P;
    memset(&P, 0, sizeof(P));
    P.K = K;
    P.x = (const __half*)xn;
    P.seg[0] = mm_seg(wq, nullptr, q_out, q_bias, fmt_q, n_q * 128, MM_ROPE_Q, K, RT);
    P.seg[1] = mm_seg(wk, nullptr, nullptr, k_bias, fmt_k, n_kv * 128, MM_ROPE_KCACHE, K, RT);
    P.seg[2] = mm_seg(wv, nullptr, nullptr, v_bias, fmt_v, n_kv * 128, MM_VCACHE, K, RT);
    P.nseg = 3;
    P.rope_cos = (const __half*)rope_cos;
    P.rope_sin = (const __half*)rope_sin;
    P.kv_offset = kv_offset;
    P.k_cache = (__half*)k_cache;
    P.v_cache = (__half*)v_cache;
    P.kv_batch_stride = kv_batch_stride;
    P.n_kv = n_kv;
    size_t ld[MM_MAX_SEG] = {(size_t)n_q * 128, 0, 0};
    return RT == 4 ? mm_run<4>(P, B, ld, st) : RT == 2 ? mm_run<2>(P, B, ld, st) : mm_run<1>(P, B, ld, st);
}

// out [B][ffn] = fp16(silu(W_gate xn) * (W_up xn)) for RMSNorm-ed fp16 xn [B][K].
hipError_t gate_up_mm(const void* xn, const void* w_gate, const void* w_up, int fmt, void* out, int B, int K, int ffn,
                      hipStream_t st) {
    // 16 gate/up pairs per block (half the blocks of 8, activations read half
    // as often); 24 for 17-32 columns (measured: batch 32 2.26 -> 2.18 ms per
    // step, batch 8-16 slightly slower); 32 in the weight-stationary form above
    // 32 columns (one block per CU, but each activation chunk serves twice
    // the rows: 2048-token prefill 51.9 -> 47.9 ms)
    int RT = mm_env("VTE_MM_RT_FFN", B > 32 ? 4 : B > 16 ? 3 : 2);
    if (B > 32 && RT == 3) RT = 2;
    MmPlan P;
    memset(&P, 0, sizeof(P));
    P.K = K;
    P.x = (const __half*)xn;
    P.seg[0] = mm_seg(w_gate, w_up, out, nullptr, fmt, ffn, MM_SWIGLU, K, RT);
    P.nseg = 1;
    size_t ld[MM_MAX_SEG] = {(size_t)ffn, 0, 0};
    return RT == 4   ? mm_run<4>(P, B, ld, st)
           : RT == 3 ? mm_run<3>(P, B, ld, st)
           : RT == 2 ? mm_run<2>(P, B, ld, st)
                     : mm_run<1>(P, B, ld, st);
}

}  // namespace vte
