// Batch 1..4 quantised mat-vec over raw GGUF Q4_K / Q6_K rows, gfx950: the
// bandwidth-oriented GEMV of the decode step and of the benchmark configs.
//
// Reference contract: vte/compiler/templates/rdna/gemv_q4k.hip.template:56-168 and
// gemv_q6k.hip.template:25-104 (y = W x, fp32 accumulation, bias / residual
// epilogue).  The row-dot engine (work units, packed-fp16 inner product,
// deterministic row reduction) is rows.h.
//
// Persistent: grid = CUs x resident blocks, each block walks tiles of R rows.
// Per block (256 threads):
//  1. the activations are staged once into LDS as fp16 with their per-16 sums;
//  2. per tile, the next tile's weights are loaded while the current one is
//     consumed: Q4_K units straight into registers, Q6_K rows as 16-byte
//     aligned chunks that go through LDS (Q6_K blocks are 2-byte aligned);
//  3. each thread computes the partial of its units, rows are summed with one
//     thread per (column, row) and the epilogue applies bias, residual scale
//     and residual.
#include "rows.h"

#define QMV_MAX_LDS 65536
#define Q6_STAGE_PER_THREAD 8  // 16-byte chunks per thread per Q6_K tile (32 KiB)
#define Q4_UNITS_PER_THREAD 2  // Q4_K units per thread per tile

struct QmvLayout {
    size_t off_s16, off_part, off_stage, total;
};

__host__ __device__ inline QmvLayout qmv_layout(int fmt, int NC, int K, int R) {
    QmvLayout L;
    const int n_sb = K / 256;
    size_t o = (size_t)NC * xpad_len(K) * 2;             // x fp16 (padded layout)
    o = (o + 15) & ~(size_t)15;
    L.off_s16 = o; o += (size_t)NC * (K / 16) * 4;       // per-16 sums
    o = (o + 15) & ~(size_t)15;
    L.off_part = o; o += (size_t)NC * R * n_sb * 4 * 4;  // unit partials
    o = (o + 15) & ~(size_t)15;
    L.off_stage = o;
    if (fmt == 6) o += (size_t)R * n_sb * 210 + 48;      // Q6_K rows + alignment slack
    L.total = o;
    return L;
}

// Persistent: block b handles row tiles b, b + gridDim.x, ...; R rows per tile.
// The activation is staged once per block; the next tile's weights are in
// flight (registers) while the current tile is computed.
template <int NC, int FMT, typename TO>
__global__ __launch_bounds__(ROWS_THREADS) void qmv_kernel(const void* __restrict__ x, int x_f32,
                                                           const uint8_t* __restrict__ w, TO* __restrict__ y, int M,
                                                           int K, int N, const TO* __restrict__ bias,
                                                           const TO* __restrict__ residual, float rs, int R,
                                                           int n_tiles) {
    extern __shared__ uint4 smem_qmv[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(smem_qmv);
    const QmvLayout L = qmv_layout(FMT, NC, K, R);
    _Float16* xs = reinterpret_cast<_Float16*>(lds);
    float* s16 = reinterpret_cast<float*>(lds + L.off_s16);
    float* part = reinterpret_cast<float*>(lds + L.off_part);
    uint8_t* stage = lds + L.off_stage;

    const int tid = threadIdx.x;
    const int n_sb = K / QK_K;
    const int per_row = n_sb * 4;
    const float inv_nsb = 1.0f / (float)n_sb;
    const int ustride = R * per_row;  // partial stride per column
    const size_t RB = (size_t)n_sb * ((FMT == 4) ? Q4K_BYTES : Q6K_BYTES);
    const int G = gridDim.x;

    Q4KUnitData cur[Q4_UNITS_PER_THREAD], nxt[Q4_UNITS_PER_THREAD];
    uint4 chunk[Q6_STAGE_PER_THREAD];
    // issue the loads of tile t into the given registers
    auto load_tile = [&](int t, Q4KUnitData (&q4)[Q4_UNITS_PER_THREAD]) {
        if (t >= n_tiles) return;
        const int nr = min(R, N - t * R);
        const uint8_t* wb = w + (size_t)t * R * RB;
        if (FMT == 4) {
#pragma unroll
            for (int j = 0; j < Q4_UNITS_PER_THREAD; ++j) {
                const int u = tid + j * ROWS_THREADS;
                if (u < nr * per_row) q4[j] = q4k_unit_load(wb + (size_t)(u >> 2) * Q4K_BYTES, u & 3);
            }
        } else {
            const uintptr_t a = reinterpret_cast<uintptr_t>(wb);
            const uintptr_t a0 = a & ~(uintptr_t)15;
            const int nchunk = (int)((a + (size_t)nr * RB - a0 + 15) >> 4);
#pragma unroll
            for (int j = 0; j < Q6_STAGE_PER_THREAD; ++j) {
                const int c = tid + j * ROWS_THREADS;
                if (c < nchunk) chunk[j] = ldg_stream16(reinterpret_cast<const uint8_t*>(a0) + 16 * (size_t)c);
            }
        }
    };
    auto store_stage = [&](int t) {  // Q6_K: registers of tile t -> LDS
        if (t >= n_tiles) return;
        const int nr = min(R, N - t * R);
        const uintptr_t a = reinterpret_cast<uintptr_t>(w + (size_t)t * R * RB);
        const uintptr_t a0 = a & ~(uintptr_t)15;
        const int nchunk = (int)((a + (size_t)nr * RB - a0 + 15) >> 4);
#pragma unroll
        for (int j = 0; j < Q6_STAGE_PER_THREAD; ++j) {
            const int c = tid + j * ROWS_THREADS;
            if (c < nchunk) reinterpret_cast<uint4*>(stage)[c] = chunk[j];
        }
    };

    int t = blockIdx.x;
    load_tile(t, cur);
    // activations -> LDS fp16, then per-16 sums
    const int ldx = xpad_len(K);
    stage_act<NC>(x, x_f32 != 0, M, K, xs);
    if (FMT == 6) store_stage(t);
    __syncthreads();
    act_sums<NC>(ActLDS{xs, s16}, K);
    __syncthreads();

    for (; t < n_tiles; t += G) {
        const int nr = min(R, N - t * R);
        const int units = nr * per_row;
        const int tn = t + G;
        load_tile(tn, nxt);  // next tile in flight during this tile's math
        const uint8_t* rows_lds =
            stage + (reinterpret_cast<uintptr_t>(w + (size_t)t * R * RB) & 15);
#pragma unroll
        for (int j = 0; j < ((FMT == 4) ? Q4_UNITS_PER_THREAD : (Q6_STAGE_PER_THREAD * 16 / 52 + 1)); ++j) {
            const int u = tid + j * ROWS_THREADS;
            if (u >= units) break;
            const int sbg = u >> 2, q = u & 3;
            const int rl = (int)(((float)sbg + 0.5f) * inv_nsb);
            const int sb = sbg - rl * n_sb;
            if (FMT == 4) {
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * ustride + u] = q4k_unit_dot(cur[j], q, xs + (size_t)m * ldx + xpad(sb * QK_K + 64 * q),
                                                         s16 + m * (K / 16) + sb * 16 + 4 * q);
            } else {
                const uint8_t* blk = rows_lds + (size_t)sbg * Q6K_BYTES;
                const int h = q >> 1, l16 = (q & 1) * 16;
#pragma unroll
                for (int m = 0; m < NC; ++m)
                    part[m * ustride + u] = q6k_unit_dot(blk, h, l16, xs + (size_t)m * ldx + xpad(sb * QK_K),
                                                         s16 + m * (K / 16) + sb * 16);
            }
        }
        __syncthreads();
        // row sums: one thread per (column, row)
        for (int i = tid; i < NC * nr; i += ROWS_THREADS) {
            const int m = i / nr, r = i - m * nr;
            const float4* p = reinterpret_cast<const float4*>(part + m * ustride + r * per_row);
            float s = 0.f;
            for (int j = 0; j < per_row / 4; ++j) {
                const float4 v = p[j];
                s += (v.x + v.y) + (v.z + v.w);
            }
            if (m < M) gemv_store<TO>(y, bias, residual, rs, t * R + r, m, N, s);
        }
        if (FMT == 6) store_stage(tn);
        __syncthreads();
        if (FMT == 4) {
#pragma unroll
            for (int j = 0; j < Q4_UNITS_PER_THREAD; ++j) cur[j] = nxt[j];
        }
    }
}

namespace vte {

static int num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    }
    return n;
}

// Rows per tile: Q4_K at most Q4_UNITS_PER_THREAD units per thread; Q6_K a
// staged tile within the per-thread chunk budget.
static int qmv_rows(int fmt, int NC, int K) {
    const int n_sb = K / 256;
    int R;
    if (fmt == 4) {
        R = ROWS_THREADS * Q4_UNITS_PER_THREAD / (n_sb * 4);
    } else {
        R = (int)(((size_t)ROWS_THREADS * Q6_STAGE_PER_THREAD * 16 - 48) / ((size_t)n_sb * 210));
        // Q6_K unit loop bound: units per thread per tile must not exceed the unrolled count
        while (R > 1 && R * n_sb * 4 > ROWS_THREADS * (Q6_STAGE_PER_THREAD * 16 / 52 + 1)) --R;
    }
    if (R < 1) R = 1;
    while (R > 1 && qmv_layout(fmt, NC, K, R).total > QMV_MAX_LDS) --R;
    return R;
}

template <int NC, int FMT, typename TO>
static hipError_t qmv_go(const void* x, bool x_f32, const void* w, void* y, int M, int K, int N, const void* bias,
                         const void* residual, float rs, hipStream_t st) {
    const int R = qmv_rows(FMT, NC, K);
    const QmvLayout L = qmv_layout(FMT, NC, K, R);
    if (L.total > QMV_MAX_LDS) return hipErrorNotSupported;
    if (FMT == 4 && R * (K / 256) * 4 > ROWS_THREADS * Q4_UNITS_PER_THREAD) return hipErrorNotSupported;
    if (FMT == 6 && ((size_t)R * (K / 256) * 210 + 48) > (size_t)ROWS_THREADS * Q6_STAGE_PER_THREAD * 16)
        return hipErrorNotSupported;
    // staging reads x in 16-byte chunks
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (K & 7)) return hipErrorNotSupported;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, (const void*)qmv_kernel<NC, FMT, TO>, ROWS_THREADS,
                                                     L.total) != hipSuccess || blocks <= 0)
        blocks = 1;
    const int n_tiles = (N + R - 1) / R;
    int grid = num_cus() * blocks;
    if (grid > n_tiles) grid = n_tiles;
    hipLaunchKernelGGL((qmv_kernel<NC, FMT, TO>), dim3(grid), dim3(ROWS_THREADS), L.total, st, x, (int)x_f32,
                       (const uint8_t*)w, (TO*)y, M, K, N, (const TO*)bias, (const TO*)residual, rs, R, n_tiles);
    return hipGetLastError();
}

template <int FMT, typename TO>
static hipError_t qmv_nc(const void* x, bool x_f32, const void* w, void* y, int M, int K, int N, const void* bias,
                         const void* residual, float rs, hipStream_t st) {
    if (M <= 1) return qmv_go<1, FMT, TO>(x, x_f32, w, y, M, K, N, bias, residual, rs, st);
    if (M <= 2) return qmv_go<2, FMT, TO>(x, x_f32, w, y, M, K, N, bias, residual, rs, st);
    if (M <= 4) return qmv_go<4, FMT, TO>(x, x_f32, w, y, M, K, N, bias, residual, rs, st);
    return hipErrorNotSupported;
}

// Returns hipErrorNotSupported (nothing launched) when the shape does not fit
// this kernel (M > 4 or an LDS plan above 64 KiB); callers fall back.
hipError_t qmv(int fmt, bool in_f32, bool out_f32, const void* x, const void* w, void* y, int M, int K, int N,
               const void* bias, const void* residual, float rs, hipStream_t st) {
    if (fmt == 4)
        return out_f32 ? qmv_nc<4, float>(x, in_f32, w, y, M, K, N, bias, residual, rs, st)
                       : qmv_nc<4, __half>(x, in_f32, w, y, M, K, N, bias, residual, rs, st);
    if (fmt == 6)
        return out_f32 ? qmv_nc<6, float>(x, in_f32, w, y, M, K, N, bias, residual, rs, st)
                       : qmv_nc<6, __half>(x, in_f32, w, y, M, K, N, bias, residual, rs, st);
    return hipErrorNotSupported;
}

}  // namespace vte
