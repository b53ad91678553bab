// Batched decode GEMM over raw Q4_K / Q6_K super-blocks on MFMA, gfx950.
//
//   Y[m, r] = ((sum_k dequant(W[r, k]) * X[m, k] + bias[r]) * rs) + residual[m, r]
//
// Same contract as the GEMV (vte/compiler/templates/rdna/gemv_q4k.hip.template:56-168);
// the reference re-reads W once per batch row (grid.y = batch), this kernel
// reads it once per 32-column batch tile (and the weight-stationary split-K
// form once per column group of up to hundreds of columns).
//
// Design:
//  * v_mfma_f32_16x16x32_f16 with exact integer weight operands and the
//    super-block scales applied in fp32 once per super-block (mfma_deq.h:
//    sb_mfma).  A block of 8 waves owns RT x 16 rows; each wave takes a
//    contiguous range of super-blocks (split-K inside the block) and the
//    partial C tiles are summed through LDS in wave order before the epilogue.
//  * Q4_K rows are 16-byte aligned and Q6_K rows 2-byte aligned; both load
//    straight from HBM (unaligned 8-byte loads stream at full speed).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "mfma_deq.h"

// Body of one block: row tile blockIdx.x, split `split` of `nsplit` (split-K
// partial sums at y + split * split_stride).
template <typename TI, typename TO, int FMT, int RT, int NT, int NW>
__device__ __forceinline__ void gemm_mfma_body(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                               TO* __restrict__ y, int M, int K, int N, const TO* __restrict__ bias,
                                               const TO* __restrict__ residual, float rs, size_t split_stride,
                                               int split, int nsplit, float (*red)[RT][NT][4][64],
                                               float (*xl)[NT * 128]) {
    constexpr bool XM = NT > 1;  // minimum-term form (q4_xmin)

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int n_sb = K / QK_K;
    const int bpr = (FMT == 4) ? Q4K_BYTES : Q6K_BYTES;
    const size_t row_bytes = (size_t)n_sb * bpr;
    const int row0 = blockIdx.x * (16 * RT);
    // split-K over blockIdx.y: this block's super-block range, then each
    // wave's contiguous share of it; split s writes its sums at y + s * split_stride
    const int kb0 = (n_sb * split) / nsplit, kb1 = (n_sb * (split + 1)) / nsplit;
    const int sb0 = kb0 + ((kb1 - kb0) * wv) / NW, sb1 = kb0 + ((kb1 - kb0) * (wv + 1)) / NW;
    y += split * split_stride;

    floatx4_t acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    for (int sb = sb0; sb < sb1; ++sb) {
        // ---- A operands (activations) for the 8 k-steps ----
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
        // weights requested before the minimum-term LDS round trip, whose
        // memory clobber would otherwise hold them back
        typename SbRaw<FMT>::Raw raw[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int r = min(row0 + rt * 16 + col, N - 1);
            sb_load(w + (size_t)r * row_bytes + (size_t)sb * bpr, grp, raw[rt]);
        }
        XMin<NT, XM> xm;
        sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            typename SbRaw<FMT>::Ops ops;
            sb_ops<XM>(raw[rt], grp, ops);
            sb_mfma<NT>(ops, bx, xm, acc[rt]);
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
    // C layout: lane (row rw, grp) holds batch columns 4*grp + i of the tile.
    for (int o = threadIdx.x; o < RT * 16 * NT * 16; o += blockDim.x) {
        const int rr = o / (NT * 16), mc = o % (NT * 16);
        const int rt = rr >> 4, rw = rr & 15, nt = mc >> 4, cc = mc & 15;
        const int ln = c_lane(rw, cc), i = c_reg(cc);
        float s = 0.f;
#pragma unroll
        for (int wq = 0; wq < NW; ++wq) s += red[wq][rt][nt][i][ln];
        const int row = row0 + rr;
        if (row < N && mc < M) gemv_store<TO>(y, bias, residual, rs, row, mc, N, s);
    }
}

// NW waves per block split K (6 when K = 1536: one super-block each).
template <typename TI, typename TO, int FMT, int RT, int NT, int NW = MF_WAVES>
__global__ __launch_bounds__(64 * NW) void gemm_mfma_kernel(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                                        TO* __restrict__ y, int M, int K, int N,
                                                        const TO* __restrict__ bias, const TO* __restrict__ residual,
                                                        float rs, size_t split_stride) {
    __shared__ float red[NW][RT][NT][4][64];
    __shared__ float xl[NW][NT * 128];  // minimum-term scratch per wave (q4_xmin)
    gemm_mfma_body<TI, TO, FMT, RT, NT, NW>(x, w, y, M, K, N, bias, residual, rs, split_stride, (int)blockIdx.y,
                                            (int)gridDim.y, red, xl);
}

// Batched MFMA GEMM behind the reference GEMV's 10-argument ABI (fp16 I/O,
// argument list of gemv_q4k.hip.template:56-67), for callers that select a
// batched symbol at batch >= 8: rows = batch * seq_len columns of the input.
// Launch geometry differs from the GEMV's: grid (ceil(out_features / 32),
// ceil(batch * seq_len / 16), 1), block (512, 1, 1); blockIdx.y picks 16
// columns.  in_features must be a multiple of 256.
template <int FMT>
__device__ __forceinline__ void gemm_ref_abi(const void* input_ptr, const void* weight_ptr, void* output_ptr, int batch,
                                             int seq_len, int in_features, int out_features, const void* bias_ptr,
                                             const void* residual_ptr, float residual_scale) {
    __shared__ float red[MF_WAVES][2][1][4][64];
    __shared__ float xl[MF_WAVES][128];
    const int cols = batch * seq_len, c0 = (int)blockIdx.y * 16;
    if (c0 >= cols) return;
    const __half* x = static_cast<const __half*>(input_ptr) + (size_t)c0 * in_features;
    __half* y = static_cast<__half*>(output_ptr) + (size_t)c0 * out_features;
    const __half* res = residual_ptr ? static_cast<const __half*>(residual_ptr) + (size_t)c0 * out_features : nullptr;
    gemm_mfma_body<__half, __half, FMT, 2, 1, MF_WAVES>(x, static_cast<const uint8_t*>(weight_ptr), y,
                                                        min(16, cols - c0), in_features, out_features,
                                                        static_cast<const __half*>(bias_ptr), res, residual_scale, 0,
                                                        0, 1, red, xl);
}
extern "C" __global__ __launch_bounds__(64 * MF_WAVES) void gemm_q4k_mfma_kernel(
    const void* input_ptr, const void* weight_ptr, void* output_ptr, int batch, int seq_len, int in_features,
    int out_features, const void* bias_ptr, const void* residual_ptr, float residual_scale) {
    gemm_ref_abi<4>(input_ptr, weight_ptr, output_ptr, batch, seq_len, in_features, out_features, bias_ptr,
                    residual_ptr, residual_scale);
}
extern "C" __global__ __launch_bounds__(64 * MF_WAVES) void gemm_q6k_mfma_kernel(
    const void* input_ptr, const void* weight_ptr, void* output_ptr, int batch, int seq_len, int in_features,
    int out_features, const void* bias_ptr, const void* residual_ptr, float residual_scale) {
    gemm_ref_abi<6>(input_ptr, weight_ptr, output_ptr, batch, seq_len, in_features, out_features, bias_ptr,
                    residual_ptr, residual_scale);
}


// Weight-stationary split-K for long batches (prefill chunks): as
// gemm_mfma_kernel with fp16 activations and fp32 partial sums, when no wave
// owns more than one super-block of its block's range.  Each wave dequantises
// its super-block of the 16 tile rows once and runs it against the block's
// columns [blockIdx.z * cols, ...), 16 * NT at a time, requesting the next
// columns' activations before the epilogue; the k-steps and the wave sum keep
// the order of gemm_mfma_kernel, so the partial sums have the same bits.
template <int FMT, int RT, int NT>
__global__ __launch_bounds__(64 * MF_WAVES) void gemm_ws_splitk_kernel(const __half* __restrict__ x,
                                                                     const uint8_t* __restrict__ w,
                                                                     float* __restrict__ part, int M, int K, int N,
                                                                     size_t split_stride, int cols) {
    constexpr bool XM = true;  // minimum-term form (q4_xmin)
    constexpr int NW = MF_WAVES;
    __shared__ float red[NW][RT][NT][4][64];
    __shared__ float xl[NW][NT * 128];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int n_sb = K / QK_K;
    const size_t row_bytes = (size_t)n_sb * (FMT == 4 ? Q4K_BYTES : Q6K_BYTES);
    const int row0 = blockIdx.x * 16 * RT;
    const int kb0 = (n_sb * (int)blockIdx.y) / (int)gridDim.y, kb1 = (n_sb * ((int)blockIdx.y + 1)) / (int)gridDim.y;
    const int sb0 = kb0 + ((kb1 - kb0) * wv) / NW, sb1 = kb0 + ((kb1 - kb0) * (wv + 1)) / NW;
    const bool has = sb1 > sb0;
    const int c0 = blockIdx.z * cols, c1 = min(M, c0 + cols);
    if (c0 >= c1) return;
    float* y = part + blockIdx.y * split_stride;

    typename SbRaw<FMT>::Ops ops[RT];
    if (has) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint8_t* blk = w + (size_t)min(row0 + rt * 16 + col, N - 1) * row_bytes;
            typename SbRaw<FMT>::Raw raw;
            sb_load(blk + (size_t)sb0 * (FMT == 4 ? Q4K_BYTES : Q6K_BYTES), grp, raw);
            sb_ops<XM>(raw, grp, ops[rt]);
        }
    }
    half8_t bx[8][NT];
    auto load_b = [&](int m0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int kb = sb0 * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int m = m0 + nt * 16 + col;
                bx[t][nt] = load_x8<__half>(x + (size_t)(m < c1 ? m : c0) * K + kb, has && m < c1);
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
        if (has) {
            XMin<NT, XM> xm;
            sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sb_mfma<NT>(ops[rt], bx, xm, acc[rt]);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wv][rt][nt][i][lane] = acc[rt][nt][i];
        if (m0 + 16 * NT < c1) load_b(m0 + 16 * NT);
        __syncthreads();
        const int mcount = min(16 * NT, c1 - m0);
        for (int o = threadIdx.x; o < 16 * RT * NT * 16; o += blockDim.x) {
            const int rr = o / (NT * 16), mc = o % (NT * 16);
            const int rt = rr >> 4, rw = rr & 15, nt = mc >> 4, cc = mc & 15;
            const int ln = c_lane(rw, cc), i = c_reg(cc);
            float s = 0.f;
#pragma unroll
            for (int wq = 0; wq < NW; ++wq) s += red[wq][rt][nt][i][ln];
            const int row = row0 + rr;
            if (row < N && mc < mcount) y[(size_t)(m0 + mc) * N + row] = s;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Streaming batched GEMM for tall matrices at K = 1536 (the LM head at batch
// >= 8).  Persistent 8-wave blocks, two per CU; the batch's activations are staged once
// per block in LDS as fp16 rows padded by 16 bytes (the 16 lanes of an MFMA
// B-operand read hit distinct banks); each wave then owns whole 16-row
// tiles: it requests the raw bytes of its rows' super-blocks (16-byte loads),
// turns them into exact weight operands and runs the K loop with the
// activation operands read from LDS, so a tile needs no cross-wave reduction and no
// barrier, and the waves of a CU keep their loads in flight independently
// (three super-blocks ahead).  Measured at batch 16 on 151936 x 1536 Q6_K:
// 71 us, its waves waiting on memory for more than half of their cycles.
// ---------------------------------------------------------------------------
#define GS_K 1536
#define GS_NSB (GS_K / QK_K)
#define GS_LDX (GS_K + 8)  // halves per staged activation row

// OT (one tile): a wave owns exactly one 16-row tile (grid = tiles / WPB,
// the hardware balances the blocks) and requests all six of its super-blocks
// at once.
template <typename TI, typename TO, int FMT, int NT, int WPB, bool OT = false>
__global__ __launch_bounds__(64 * WPB, (OT && NT == 1) ? 4 : 2) void gemm_stream_kernel(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                                          TO* __restrict__ y, int M, int N, const TO* __restrict__ bias,
                                                          const TO* __restrict__ residual, float rs) {
    constexpr bool XM = NT > 1;  // minimum-term form (q4_xmin)
    extern __shared__ uint4 gs_smem[];
    __shared__ float xl[WPB][NT * 128];
    _Float16* xs = reinterpret_cast<_Float16*>(gs_smem);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    constexpr int CPR = GS_K / 8;  // 8-element chunks per row
    constexpr int BPB = FMT == 4 ? Q4K_BYTES : Q6K_BYTES;
    const size_t row_bytes = (size_t)GS_NSB * BPB;
    const int ntiles = (N + 15) / 16;
    using Raw = typename SbRaw<FMT>::Raw;
    Raw r[OT ? GS_NSB : 1];
    const int ot_tile = blockIdx.x * WPB + wv;
    if constexpr (OT) {
        // The block's activation chunks, then the tile's weights, all requested
        // at once; the chunks (requested first: the load counter is in order)
        // go to LDS as soon as they arrive, while the weights are in flight.
        constexpr int XPT = 16 * NT * CPR / (64 * WPB);  // chunks per thread
        static_assert(XPT * 64 * WPB == 16 * NT * CPR, "activation chunks fill the block");
        half8_t xv[XPT];
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int i = tid + j * 64 * WPB, m = i / CPR, c = i - m * CPR;
            xv[j] = load_x8<TI>(x + (size_t)(m < M ? m : 0) * GS_K + 8 * c, m < M);
        }
        const uint8_t* rowp = w + (size_t)min(min(ot_tile, ntiles - 1) * 16 + col, N - 1) * row_bytes;
#pragma unroll
        for (int sb = 0; sb < GS_NSB; ++sb) sb_load(rowp + sb * BPB, grp, r[sb]);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the LDS stores (not sunk into the K loop)
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int i = tid + j * 64 * WPB, m = i / CPR, c = i - m * CPR;
            *reinterpret_cast<half8_t*>(xs + m * GS_LDX + 8 * c) = xv[j];
        }
    }
    for (int i = tid; i < (OT ? 0 : 16 * NT * CPR); i += 64 * WPB) {
        const int m = i / CPR, c = i - m * CPR;
        const half8_t v = load_x8<TI>(x + (size_t)(m < M ? m : 0) * GS_K + 8 * c, m < M);
        *reinterpret_cast<half8_t*>(xs + m * GS_LDX + 8 * c) = v;
    }
    __syncthreads();
    if constexpr (OT) {
        // no early exit for waves past the last tile (they recompute it and
        // store nothing), so the weight loads above stay where they are
        const int tile = ot_tile;
        floatx4_t acc[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sb = 0; sb < GS_NSB; ++sb) {
            typename SbRaw<FMT>::Ops ops;
            sb_ops<XM>(r[sb], grp, ops);
            half8_t bx[8][NT];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int kb = sb * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    bx[t][nt] = *reinterpret_cast<const half8_t*>(xs + (nt * 16 + col) * GS_LDX + kb);
            }
            XMin<NT, XM> xm;
            sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
            sb_mfma<NT>(ops, bx, xm, acc);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rr = tile * 16 + col, m = nt * 16 + 4 * grp + i;
                if (tile < ntiles && rr < N && m < M) gemv_store<TO>(y, bias, residual, rs, rr, m, N, acc[nt][i]);
            }
        return;
    }
    for (int tile = blockIdx.x * WPB + wv; tile < ntiles; tile += gridDim.x * WPB) {
        const uint8_t* rowp = w + (size_t)min(tile * 16 + col, N - 1) * row_bytes;
        auto load = [&](int sb, Raw& r) { sb_load(rowp + sb * BPB, grp, r); };
        Raw cur, nxt, nx2;
        load(0, cur);
        load(1, nxt);
        load(2, nx2);
        floatx4_t acc[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        // three super-blocks in flight per wave while sb is multiplied
#pragma unroll 1
        for (int sb = 0; sb < GS_NSB; ++sb) {
            typename SbRaw<FMT>::Ops ops;
            sb_ops<XM>(cur, grp, ops);
            cur = nxt;
            nxt = nx2;
            load(min(sb + 3, GS_NSB - 1), nx2);
            half8_t bx[8][NT];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int kb = sb * QK_K + kslot_base<FMT>(t, grp);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    bx[t][nt] = *reinterpret_cast<const half8_t*>(xs + (nt * 16 + col) * GS_LDX + kb);
            }
            XMin<NT, XM> xm;
            sb_xmin<FMT, NT, XM>(bx, xl[wv], xm);
            sb_mfma<NT>(ops, bx, xm, acc);
        }
        // C layout: lane (col, grp) holds batch columns 4*grp + i of weight row col
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = tile * 16 + col, m = nt * 16 + 4 * grp + i;
                if (r < N && m < M) gemv_store<TO>(y, bias, residual, rs, r, m, N, acc[nt][i]);
            }
    }
}

namespace vte {

template <typename TI, typename TO, int FMT, int RT, int NT>
static void launch_tile(const TI* x, const void* w, TO* y, int M, int K, int N, const void* bias,
                        const TO* residual, float rs, hipStream_t st, int splits = 1, size_t split_stride = 0) {
    const dim3 g((N + 16 * RT - 1) / (16 * RT), splits);
    if (K == 6 * QK_K && splits == 1)
        hipLaunchKernelGGL((gemm_mfma_kernel<TI, TO, FMT, RT, NT, 6>), g, dim3(64 * 6), 0, st, x, (const uint8_t*)w, y,
                           M, K, N, (const TO*)bias, residual, rs, split_stride);
    else
        hipLaunchKernelGGL((gemm_mfma_kernel<TI, TO, FMT, RT, NT>), g, dim3(64 * MF_WAVES), 0, st, x,
                           (const uint8_t*)w, y, M, K, N, (const TO*)bias, residual, rs, split_stride);
}

// Batch columns are processed in chunks of 32 (two 16-wide MFMA N tiles).
// Tall matrices (N >= 4096) use 32-row tiles.
static int gs_num_cus() { return device_cus(); }

// Whether the device grants the streaming kernel's dynamic LDS (staged
// activations of up to 32 batch columns).
static bool gs_lds_ok(int M) {
    static int max_lds = 0;
    if (max_lds == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            max_lds = 65536;
    }
    return (M > 16 ? 32 : 16) * GS_LDX * 2 <= max_lds;
}

// The streaming kernel for K = 1536 and N >= 16384 (one launch per 32 batch columns).
template <typename TI, typename TO, int FMT>
static hipError_t launch_stream(const void* x, const void* w, void* y, int M, int N, const void* bias,
                                const void* residual, float rs, hipStream_t st) {
    constexpr int WPB = 8;  // 8-wave blocks, two per CU
    static const int bpc = getenv("VTE_GS_BPC") ? atoi(getenv("VTE_GS_BPC")) : 2;
    static const bool gs_ot = getenv("VTE_GS_OT") ? atoi(getenv("VTE_GS_OT")) != 0 : true;
    const int ntiles = (N + 15) / 16;
    const int grid = std::min((ntiles + WPB - 1) / WPB, gs_num_cus() * bpc);
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = (M - m0 < 32) ? (M - m0) : 32;
        const TI* xs = (const TI*)x + (size_t)m0 * GS_K;
        TO* ys = (TO*)y + (size_t)m0 * N;
        const TO* rp = residual ? (const TO*)residual + (size_t)m0 * N : nullptr;
#define GS_LAUNCH(NT_, W_, OT_, G_)                                                                                \
    hipLaunchKernelGGL((gemm_stream_kernel<TI, TO, FMT, NT_, W_, OT_>), dim3(G_), dim3(64 * W_), 16 * NT_ * GS_LDX * 2, \
                       st, xs, (const uint8_t*)w, ys, mc, N, (const TO*)bias, rp, rs)
        const int ot = (ntiles + WPB - 1) / WPB;
        if (gs_ot) {
            if (M > 16) GS_LAUNCH(2, WPB, true, ot);
            else GS_LAUNCH(1, WPB, true, ot);
        } else {
            if (M > 16) GS_LAUNCH(2, WPB, false, grid);  // a 16-column tail of a longer batch too (one minimum-term form)
            else GS_LAUNCH(1, WPB, false, grid);
        }
#undef GS_LAUNCH
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <typename TI, typename TO, int FMT>
static hipError_t launch_mfma(const void* x, const void* w, void* y, int M, int K, int N, const void* bias,
                              const void* residual, float rs, hipStream_t st) {
    if (K == GS_K && N >= 16384 && gs_lds_ok(M)) return launch_stream<TI, TO, FMT>(x, w, y, M, N, bias, residual, rs, st);
    const bool tall = N >= 4096;
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = (M - m0 < 32) ? (M - m0) : 32;
        const TI* xs = (const TI*)x + (size_t)m0 * K;
        TO* ys = (TO*)y + (size_t)m0 * N;
        const TO* rp = residual ? (const TO*)residual + (size_t)m0 * N : nullptr;
        if (M > 16) {  // also a tail of 16 or fewer: every column of a batch gets one minimum-term form
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
// true when the environment variable is set to 0 (switches a launch form off)
static bool getenv_off(const char* name) {
    const char* v = getenv(name);
    return v != nullptr && atoi(v) == 0;
}

template <int FMT>
static hipError_t launch_splitk(const void* x, const void* w, float* part, int M, int K, int N, int splits,
                                hipStream_t st) {
    const size_t ss = (size_t)M * N;
    const int n_sb = K / QK_K;
    if (M > 32 && (n_sb + splits - 1) / splits <= MF_WAVES && !getenv_off("VTE_MM_WS")) {
        // one launch; two 8-wave blocks fit per CU
        if (getenv_off("VTE_MM_WS_RT4")) {  // 16 rows per block, 32 columns at a time
            const int tiles = (N + 15) / 16;
            const int g = ws_column_groups(tiles * splits, M, 2 * device_cus());
            const int cols = ((M + 31) / 32 + g - 1) / g * 32, gz = (M + cols - 1) / cols;
            hipLaunchKernelGGL((gemm_ws_splitk_kernel<FMT, 1, 2>), dim3(tiles, splits, gz), dim3(64 * MF_WAVES), 0,
                               st, (const __half*)x, (const uint8_t*)w, part, M, K, N, ss, cols);
        } else {  // 64 rows per block, 16 columns at a time: each activation chunk serves 4x the rows
            const int tiles = (N + 63) / 64;
            const int g = ws_column_groups(tiles * splits, M, device_cus());
            const int cols = ((M + 31) / 32 + g - 1) / g * 32, gz = (M + cols - 1) / cols;
            hipLaunchKernelGGL((gemm_ws_splitk_kernel<FMT, 4, 1>), dim3(tiles, splits, gz), dim3(64 * MF_WAVES), 0,
                               st, (const __half*)x, (const uint8_t*)w, part, M, K, N, ss, cols);
        }
        return hipGetLastError();
    }
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = (M - m0 < 32) ? (M - m0) : 32;
        const __half* xs = (const __half*)x + (size_t)m0 * K;
        float* ps = part + (size_t)m0 * N;
        // 32-row tiles above 8 columns (measured per decode step: batch 32
        // 2.18 -> 2.08 ms, batch 16 1.544 -> 1.536 ms; batch 8 faster with 16 rows)
        static const int rt_env = [] { const char* v = getenv("VTE_SPLITK_RT"); return v ? atoi(v) : 0; }();
        const int rt = rt_env > 0 ? rt_env : (mc > 8 ? 2 : 1);
        if (rt == 4) {
            if (M > 16) launch_tile<__half, float, FMT, 4, 2>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
            else launch_tile<__half, float, FMT, 4, 1>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
        } else if (rt == 2) {
            if (M > 16) launch_tile<__half, float, FMT, 2, 2>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
            else launch_tile<__half, float, FMT, 2, 1>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
        } else if (M > 16) launch_tile<__half, float, FMT, 1, 2>(xs, w, ps, mc, K, N, nullptr, nullptr, 1.f, st, splits, ss);
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
