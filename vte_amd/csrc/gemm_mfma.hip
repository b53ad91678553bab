// Batched decode GEMM over raw Q4_K / Q6_K super-blocks on MFMA, gfx950.
//
//   Y[m, r] = ((sum_k dequant(W[r, k]) * X[m, k] + bias[r]) * rs) + residual[m, r]
//
// Same contract as the GEMV (vte/compiler/templates/rdna/gemv_q4k.hip.template:56-168);
// the reference re-reads W once per batch row (grid.y = batch), this kernel
// reads it once per 32-column batch tile.
//
// Design:
//  * v_mfma_f32_16x16x32_f16: M = 16 weight rows, N = 16 batch columns,
//    K = 32.  A block of 8 waves owns RT x 16 rows; each wave takes a
//    contiguous range of super-blocks (split-K inside the block) and the
//    partial C tiles are summed through LDS before the epilogue.
//  * Weights are dequantised in registers to fp16 with packed fp16 math
//    (nibble -> 0x64xx magic -> exact subtract -> v_pk_fma_f16), so only the
//    final weight carries an fp16 rounding; activations go to fp16; the MFMA
//    accumulates in fp32.
//  * K-slot permutation: MFMA pairs A and B by (lane group, slot), so any
//    bijection of super-block elements to (k-step, group, slot) is valid as
//    long as A and B use the same one.  The map is chosen so each lane's 8
//    slots are 8 contiguous elements sharing one sub-block scale:
//      Q4_K step t, group g: qs chunk c = g + 4*(t>>2), nibble (t>>1)&1, half t&1
//      Q6_K step t, group g: half h = t>>2, quarter q = t&3, l = 8g .. 8g+7
//  * Q4_K rows are 16-byte aligned and Q6_K rows 2-byte aligned; both load
//    straight from HBM (unaligned 8-byte loads stream at full speed).
#include "mfma_deq.h"

template <typename TI, typename TO, int FMT, int RT, int NT>
__global__ __launch_bounds__(512) void gemm_mfma_kernel(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                                        TO* __restrict__ y, int M, int K, int N,
                                                        const TO* __restrict__ bias, const TO* __restrict__ residual,
                                                        float rs, size_t split_stride) {
    __shared__ float red[MF_WAVES][RT][NT][4][64];

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int n_sb = K / QK_K;
    const int bpr = (FMT == 4) ? Q4K_BYTES : Q6K_BYTES;
    const size_t row_bytes = (size_t)n_sb * bpr;
    const int row0 = blockIdx.x * (16 * RT);
    // split-K over blockIdx.y: this block's super-block range, then each
    // wave's contiguous share of it; split s writes its sums at y + s * split_stride
    const int kb0 = (n_sb * (int)blockIdx.y) / (int)gridDim.y, kb1 = (n_sb * ((int)blockIdx.y + 1)) / (int)gridDim.y;
    const int sb0 = kb0 + ((kb1 - kb0) * wv) / MF_WAVES, sb1 = kb0 + ((kb1 - kb0) * (wv + 1)) / MF_WAVES;
    y += blockIdx.y * split_stride;

    floatx4_t acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};


    for (int sb = sb0; sb < sb1; ++sb) {
        // ---- B operand (activations) for the 8 k-steps ----
        half8_t bx[8][NT];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int kb = sb * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int m = nt * 16 + col;
                bx[t][nt] = load_x8<TI>(x + (size_t)(m < M ? m : 0) * K + kb, m < M);
            }
        }
        if (FMT == 4) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int r = min(row0 + rt * 16 + col, N - 1);
                const uint8_t* blk = w + (size_t)r * row_bytes + (size_t)sb * Q4K_BYTES;
                const uint4 h = *reinterpret_cast<const uint4*>(blk);
                uint4 qc[2];
                qc[0] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * grp);
                qc[1] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * (grp + 4));
                Q4KLaneScale s[2];
                s[0] = q4k_lane_scale(h, grp >> 1);
                s[1] = q4k_lane_scale(h, 2 + (grp >> 1));
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int ci = t >> 2, part = (t >> 1) & 1, e = t & 1;
                    const uint32_t wa = (e == 0) ? ((ci == 0) ? qc[0].x : qc[1].x) : ((ci == 0) ? qc[0].z : qc[1].z);
                    const uint32_t wb = (e == 0) ? ((ci == 0) ? qc[0].y : qc[1].y) : ((ci == 0) ? qc[0].w : qc[1].w);
                    const uint32_t u0 = part ? ((wa >> 4) & 0x0F0F0F0Fu) : (wa & 0x0F0F0F0Fu);
                    const uint32_t u1 = part ? ((wb >> 4) & 0x0F0F0F0Fu) : (wb & 0x0F0F0F0Fu);
                    const float dd = part ? s[ci].d_hi : s[ci].d_lo;
                    const float mm = part ? s[ci].m_hi : s[ci].m_lo;
                    const half2_t d2 = {(_Float16)dd, (_Float16)dd};
                    const half2_t m2 = {(_Float16)mm, (_Float16)mm};
                    const half8_t a = deq8(u0, u1, (_Float16)0.0f, d2, m2);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bx[t][nt], acc[rt][nt], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                half8_t av[8];
                q6k_a_operands(w + (size_t)min(row0 + rt * 16 + col, N - 1) * row_bytes + (size_t)sb * Q6K_BYTES, grp, av);
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[t], bx[t][nt], acc[rt][nt], 0, 0, 0);
            }
        }
    }

    // ---- split-K reduction across the 8 waves, then the epilogue ----
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wv][rt][nt][i][lane] = acc[rt][nt][i];
    __syncthreads();
    // C layout: lane (col, grp) holds rows 4*grp+i of the tile, batch column col.
    for (int o = threadIdx.x; o < RT * 16 * NT * 16; o += blockDim.x) {
        const int rr = o / (NT * 16), mc = o % (NT * 16);
        const int rt = rr >> 4, rw = rr & 15, nt = mc >> 4, cc = mc & 15;
        const int ln = cc + 16 * (rw >> 2), i = rw & 3;
        float s = 0.f;
#pragma unroll
        for (int wq = 0; wq < MF_WAVES; ++wq) s += red[wq][rt][nt][i][ln];
        const int row = row0 + rr;
        if (row < N && mc < M) gemv_store<TO>(y, bias, residual, rs, row, mc, N, s);
    }
}

namespace vte {

template <typename TI, typename TO, int FMT, int RT, int NT>
static void launch_tile(const TI* x, const void* w, TO* y, int M, int K, int N, const void* bias,
                        const TO* residual, float rs, hipStream_t st, int splits = 1, size_t split_stride = 0) {
    hipLaunchKernelGGL((gemm_mfma_kernel<TI, TO, FMT, RT, NT>), dim3((N + 16 * RT - 1) / (16 * RT), splits),
                       dim3(64 * MF_WAVES), 0, st, x, (const uint8_t*)w, y, M, K, N, (const TO*)bias, residual, rs,
                       split_stride);
}

// Batch columns are processed in chunks of 32 (two 16-wide MFMA N tiles).
// Tall matrices (N >= 4096) use 32-row tiles.
template <typename TI, typename TO, int FMT>
static hipError_t launch_mfma(const void* x, const void* w, void* y, int M, int K, int N, const void* bias,
                              const void* residual, float rs, hipStream_t st) {
    const bool tall = N >= 4096;
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = (M - m0 < 32) ? (M - m0) : 32;
        const TI* xs = (const TI*)x + (size_t)m0 * K;
        TO* ys = (TO*)y + (size_t)m0 * N;
        const TO* rp = residual ? (const TO*)residual + (size_t)m0 * N : nullptr;
        if (mc > 16) {
            if (tall) launch_tile<TI, TO, FMT, 2, 2>(xs, w, ys, mc, K, N, bias, rp, rs, st);
            else launch_tile<TI, TO, FMT, 1, 2>(xs, w, ys, mc, K, N, bias, rp, rs, st);
        } else {
            if (tall) launch_tile<TI, TO, FMT, 2, 1>(xs, w, ys, mc, K, N, bias, rp, rs, st);
            else launch_tile<TI, TO, FMT, 1, 1>(xs, w, ys, mc, K, N, bias, rp, rs, st);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Split-K partial sums: part[s][m][n] (fp32) = sum over split s's share of the
// super-blocks of dequant(W[n, k]) * x[m, k]; no bias, scale or residual (the
// consumer adds the splits).  Splits multiply the blocks of a short-and-wide
// problem (down projection: K = 8960, N = 1536) so the whole chip streams W.
template <int FMT>
static hipError_t launch_splitk(const void* x, const void* w, float* part, int M, int K, int N, int splits,
                                hipStream_t st) {
    const size_t ss = (size_t)M * N;
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = (M - m0 < 32) ? (M - m0) : 32;
        const __half* xs = (const __half*)x + (size_t)m0 * K;
        float* ps = part + (size_t)m0 * N;
        if (mc > 16) launch_tile<__half, float, FMT, 1, 2>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
        else launch_tile<__half, float, FMT, 1, 1>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t gemm_mfma_splitk(int fmt, const void* x, const void* w, float* part, int M, int K, int N, int splits,
                            hipStream_t st) {
    if (fmt == 4) return launch_splitk<4>(x, w, part, M, K, N, splits, st);
    return launch_splitk<6>(x, w, part, M, K, N, splits, st);
}

hipError_t gemm_mfma(int fmt, int in_dt, int out_dt, const void* x, const void* w, void* y, int M, int K, int N,
                     const void* bias, const void* residual, float rs, hipStream_t st) {
    // dtype codes: 0 = f32, 1 = f16
    if (fmt == 4) {
        if (in_dt == 0) return launch_mfma<float, float, 4>(x, w, y, M, K, N, bias, residual, rs, st);
        if (out_dt == 1) return launch_mfma<__half, __half, 4>(x, w, y, M, K, N, bias, residual, rs, st);
        return launch_mfma<__half, float, 4>(x, w, y, M, K, N, bias, residual, rs, st);
    }
    if (in_dt == 0) return launch_mfma<float, float, 6>(x, w, y, M, K, N, bias, residual, rs, st);
    if (out_dt == 1) return launch_mfma<__half, __half, 6>(x, w, y, M, K, N, bias, residual, rs, st);
    return launch_mfma<__half, float, 6>(x, w, y, M, K, N, bias, residual, rs, st);
}

}  // namespace vte
