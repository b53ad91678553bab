// Fused dequant-GEMV over raw GGUF Q4_K / Q6_K / Q8_0 super-blocks, gfx950.
//
//   y[m, r] = ((sum_k dequant(W[r, k]) * x[m, k] + bias[r]) * rs) + residual[m, r]
//
// Reference contract: vte/compiler/templates/rdna/gemv_q4k.hip.template:56-168,
// gemv_q6k.hip.template:25-104, gemv_q8_0.hip.template:26-93 (10-argument ABI,
// fp16 activations, fp32 accumulator, bias/residual epilogue).
//
// MI355X design (one wave64 per output row, four rows per 256-thread block):
//  * Q4_K rows are 16-byte aligned (144 = 9 x 16), so each lane issues 16-byte
//    loads straight from HBM: lane = (super-block slot s = lane>>3, qs chunk
//    c = lane&7); the 8 lanes of a slot read 128 contiguous bytes of qs plus one
//    shared 16-byte header (a single cache line request for the 8 lanes).
//  * Q6_K (210 B) and Q8_0 (34 B) blocks are only 2-byte aligned, so a wave
//    stages its row through LDS with 16-byte aligned, fully coalesced loads and
//    decodes from LDS with 16-bit reads.
//  * The sub-block scales are factored out of the inner product:
//      sum_i (d*sc*q_i - dmin*m) x_i = (d*sc) * sum_i q_i x_i - (dmin*m) * sum_i x_i
//    so the inner loop is one int->float convert and one FMA per weight.
//  * fp32 accumulation; a 64-lane butterfly reduction per row.
#include "quant.h"
#include "ref_mv.h"

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------

// One wave computes NC output columns of row `row`.  x points at column 0;
// columns are ldx elements apart.
template <typename TI, int NC>
__device__ __forceinline__ void q4k_row_dot(const uint8_t* __restrict__ row_ptr, const TI* __restrict__ x,
                                            int ldx, int n_sb, int lane, float (&acc)[NC]) {
    const int slot = lane >> 3;
    const int c = lane & 7;
    const int mblk = c >> 1;
    const int off16 = (c & 1) * 16;
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = 0.f;

    for (int sb = slot; sb < n_sb; sb += 8) {
        const uint8_t* blk = row_ptr + (size_t)sb * Q4K_BYTES;
        const uint4 h = *reinterpret_cast<const uint4*>(blk);
        const uint4 qv = *reinterpret_cast<const uint4*>(blk + 16 + mblk * 32 + off16);
        const Q4KLaneScale s = q4k_lane_scale(h, mblk);
        const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
        float qlo[16], qhi[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = w[i] & 0x0F0F0F0Fu;
            const uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                qlo[4 * i + b] = (float)((lo >> (8 * b)) & 0xFFu);
                qhi[4 * i + b] = (float)((hi >> (8 * b)) & 0xFFu);
            }
        }
        const int xb = sb * QK_K + 64 * mblk + off16;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            float xl[16], xh[16];
            ld_act16<TI>(x + (size_t)j * ldx + xb, xl);
            ld_act16<TI>(x + (size_t)j * ldx + xb + 32, xh);
            float dl = 0.f, dh = 0.f, sl = 0.f, shh = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                dl = fmaf(qlo[i], xl[i], dl);
                dh = fmaf(qhi[i], xh[i], dh);
                sl += xl[i];
                shh += xh[i];
            }
            acc[j] += s.d_lo * dl - s.m_lo * sl + s.d_hi * dh - s.m_hi * shh;
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = wave_sum(acc[j]);
}

// ---------------------------------------------------------------------------
// Q6_K (LDS-staged)
// ---------------------------------------------------------------------------

// Cooperative 16-byte aligned copy of [src, src+nbytes) into LDS.  Returns the
// LDS address of src.  `stage` must hold nbytes + 32 bytes.
__device__ __forceinline__ const uint8_t* wave_stage(const uint8_t* __restrict__ src, size_t nbytes,
                                                     uint8_t* stage, int lane) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const uintptr_t a0 = a & ~(uintptr_t)15;
    const uintptr_t a1 = (a + nbytes + 15) & ~(uintptr_t)15;
    const int nchunks = (int)((a1 - a0) >> 4);
    const uint4* g = reinterpret_cast<const uint4*>(a0);
    uint4* l = reinterpret_cast<uint4*>(stage);
    for (int i = lane; i < nchunks; i += VTE_WAVE) l[i] = g[i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    __builtin_amdgcn_wave_barrier();
    return stage + (a - a0);
}

// Lane unit = (super-block slot sbs = lane>>4, half h, l4): 16 weights at
// positions 128h + l4 + i + 32g (i<4, g<4) of super-block sb; see
// vte/compiler/dequantizer.py:150-166 for the element map.
template <typename TI, int NC>
__device__ __forceinline__ void q6k_row_dot(const uint8_t* __restrict__ row, const TI* __restrict__ x,
                                            int ldx, int n_sb, int lane, float (&acc)[NC]) {
    const int slot = lane >> 4;
    const int u = lane & 15;
    const int h = u >> 3;
    const int l4 = (u & 7) * 4;
    const int is = l4 >> 4;
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = 0.f;
    for (int sb = slot; sb < n_sb; sb += 4) {
        const uint8_t* blk = row + sb * Q6K_BYTES;
        const uint32_t qa = lds_u32_a2(blk + 64 * h + l4);
        const uint32_t qb = lds_u32_a2(blk + 64 * h + 32 + l4);
        const uint32_t qh = lds_u32_a2(blk + 128 + 32 * h + l4);
        const float d = h2f_bits(lds_u16(blk + 208));
        const uint8_t* scp = blk + 192 + 8 * h + is;
        float dsc[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) dsc[g] = d * (float)(int8_t)scp[2 * g];
        uint32_t qw[4];
        qw[0] = (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
        qw[1] = (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
        qw[2] = ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
        qw[3] = ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
        const int xb = sb * QK_K + 128 * h + l4;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const TI* xj = x + (size_t)j * ldx + xb;
            float part = 0.f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float dot = 0.f, sx = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float xv = ld_act<TI>(xj + 32 * g + i);
                    dot = fmaf((float)((qw[g] >> (8 * i)) & 0xFFu), xv, dot);
                    sx += xv;
                }
                part = fmaf(dsc[g], dot - 32.f * sx, part);
            }
            acc[j] += part;
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = wave_sum(acc[j]);
}

// ---------------------------------------------------------------------------
// Q8_0 (LDS-staged)
// ---------------------------------------------------------------------------

template <typename TI, int NC>
__device__ __forceinline__ void q80_row_dot(const uint8_t* __restrict__ row, const TI* __restrict__ x,
                                            int ldx, int n_blk, int lane, float (&acc)[NC]) {
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = 0.f;
    for (int b = lane; b < n_blk; b += VTE_WAVE) {
        const uint8_t* blk = row + b * Q80_BYTES;
        const float d = h2f_bits(lds_u16(blk));
        uint32_t qw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) qw[i] = lds_u32_a2(blk + 2 + 4 * i);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const TI* xj = x + (size_t)j * ldx + b * QK8_0;
            float v[16];
            float dot = 0.f;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                ld_act16<TI>(xj + 16 * half, v);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int e = 16 * half + i;
                    const int q = (int)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xFFu);
                    dot = fmaf((float)q, v[i], dot);
                }
            }
            acc[j] = fmaf(d, dot, acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = wave_sum(acc[j]);
}

// ---------------------------------------------------------------------------
// Kernels: native launch (4 rows per 256-thread block, NC columns per pass)
// ---------------------------------------------------------------------------

#define GEMV_WAVES 4

template <typename TI, typename TO, int NC>
__global__ __launch_bounds__(256) void gemv_q4k_rows(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                                     TO* __restrict__ y, int M, int K, int N,
                                                     const TO* __restrict__ bias, const TO* __restrict__ residual,
                                                     float rs) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6);
    if (row >= N) return;
    const int n_sb = K / QK_K;
    const uint8_t* rp = w + (size_t)row * n_sb * Q4K_BYTES;
    for (int m0 = 0; m0 < M; m0 += NC) {
        float acc[NC];
        q4k_row_dot<TI, NC>(rp, x + (size_t)m0 * K, K, n_sb, lane, acc);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (m0 + j < M) gemv_store<TO>(y, bias, residual, rs, row, m0 + j, N, acc[j]);
        }
    }
}

template <typename TI, typename TO, int NC, int FMT>
__global__ __launch_bounds__(256) void gemv_staged_rows(const TI* __restrict__ x, const uint8_t* __restrict__ w,
                                                        TO* __restrict__ y, int M, int K, int N,
                                                        const TO* __restrict__ bias,
                                                        const TO* __restrict__ residual, float rs,
                                                        int stage_bytes) {
    extern __shared__ uint4 smem_u4[];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int row = blockIdx.x * GEMV_WAVES + wv;
    if (row >= N) return;
    uint8_t* stage = reinterpret_cast<uint8_t*>(smem_u4) + (size_t)wv * stage_bytes;
    const int n_blk = (FMT == 6) ? K / QK_K : K / QK8_0;
    const size_t rb = (size_t)n_blk * ((FMT == 6) ? Q6K_BYTES : Q80_BYTES);
    const uint8_t* rl = wave_stage(w + (size_t)row * rb, rb, stage, lane);
    for (int m0 = 0; m0 < M; m0 += NC) {
        float acc[NC];
        if (FMT == 6) q6k_row_dot<TI, NC>(rl, x + (size_t)m0 * K, K, n_blk, lane, acc);
        else q80_row_dot<TI, NC>(rl, x + (size_t)m0 * K, K, n_blk, lane, acc);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (m0 + j < M) gemv_store<TO>(y, bias, residual, rs, row, m0 + j, N, acc[j]);
        }
    }
}

// ---------------------------------------------------------------------------
// Reference-ABI kernels (drop-in for hipModuleGetFunction by name).
// grid (out_features, batch*seq_len, 1), block (64,1,1), fp16 in/out
// (vte/core/fallback_executor.py:140-148, kernel_arg_builder.py:32-43).
// Rows of 64-multiple lengths up to 16384 run on ref_mv.h (several rows per
// working block); other lengths one row per wave.
// ---------------------------------------------------------------------------

// Rows the batched-row mat-vec (ref_mv.h) does not serve (K not a multiple of
// 64 or above 16384): one row per wave straight from global memory.
template <typename T, int FMT>
__device__ __forceinline__ void ref_gemv_row(const void* __restrict__ input_ptr, const void* __restrict__ weight_ptr,
                                             void* __restrict__ output_ptr, int batch, int seq_len, int in_features,
                                             int out_features, const void* __restrict__ bias_ptr,
                                             const void* __restrict__ residual_ptr, float residual_scale) {
    const int row = blockIdx.x, m = blockIdx.y;
    if (row >= out_features || m >= batch * seq_len) return;
    const int n_blk = FMT == 8 ? in_features / QK8_0 : in_features / QK_K;
    const size_t rb = (size_t)n_blk * (FMT == 4 ? Q4K_BYTES : FMT == 6 ? Q6K_BYTES : Q80_BYTES);
    const uint8_t* rp = (const uint8_t*)weight_ptr + (size_t)row * rb;
    const T* xm = (const T*)input_ptr + (size_t)m * in_features;
    float acc[1];
    if constexpr (FMT == 4) q4k_row_dot<T, 1>(rp, xm, in_features, n_blk, threadIdx.x, acc);
    else if constexpr (FMT == 6) q6k_row_dot<T, 1>(rp, xm, in_features, n_blk, threadIdx.x, acc);
    else q80_row_dot<T, 1>(rp, xm, in_features, n_blk, threadIdx.x, acc);
    if (threadIdx.x == 0)
        gemv_store<T>((T*)output_ptr, (const T*)bias_ptr, (const T*)residual_ptr, residual_scale, row, m, out_features,
                      acc[0]);
}

template <typename T, int FMT>
__device__ __forceinline__ void ref_gemv(const void* __restrict__ input_ptr, const void* __restrict__ weight_ptr,
                                         void* __restrict__ output_ptr, int batch, int seq_len, int in_features,
                                         int out_features, const void* __restrict__ bias_ptr,
                                         const void* __restrict__ residual_ptr, float residual_scale) {
    __shared__ float part[64];
    // Q4_K rows of at most 4096 weights in matrices below 32768 rows: the
    // one-row-per-wave kernel is 0.2-0.8 us faster per launch (its 16-byte
    // aligned rows need no LDS; measured 8960x1536 8.97 / 9.20 us, 1536x1536
    // 8.67 / 9.46 us); every other shape gains from several rows per block
    if (ref_mv_ok(in_features) && (FMT != 4 || in_features > 4096 || out_features >= 32768))
        ref_mv_dispatch<T, FMT>((const T*)input_ptr, (const uint8_t*)weight_ptr, (T*)output_ptr, batch * seq_len,
                                in_features, out_features, (const T*)bias_ptr, (const T*)residual_ptr, residual_scale,
                                part);
    else
        ref_gemv_row<T, FMT>(input_ptr, weight_ptr, output_ptr, batch, seq_len, in_features, out_features, bias_ptr,
                             residual_ptr, residual_scale);
}

#define REF_GEMV_ARGS                                                                                          \
    const void* __restrict__ input_ptr, const void* __restrict__ weight_ptr, void* __restrict__ output_ptr,   \
        int batch, int seq_len, int in_features, int out_features, const void* __restrict__ bias_ptr,         \
        const void* __restrict__ residual_ptr, float residual_scale
#define REF_GEMV_PASS \
    input_ptr, weight_ptr, output_ptr, batch, seq_len, in_features, out_features, bias_ptr, residual_ptr, residual_scale

// fp16 I/O: the reference's symbols.
extern "C" __global__ __launch_bounds__(64) void gemv_q4k_kernel(REF_GEMV_ARGS) { ref_gemv<__half, 4>(REF_GEMV_PASS); }
extern "C" __global__ __launch_bounds__(64) void gemv_q6k_kernel(REF_GEMV_ARGS) { ref_gemv<__half, 6>(REF_GEMV_PASS); }
extern "C" __global__ __launch_bounds__(64) void gemv_q8_0_kernel(REF_GEMV_ARGS) { ref_gemv<__half, 8>(REF_GEMV_PASS); }
// fp32 I/O siblings (same argument list and geometry; input, output, bias and
// residual fp32): the BASELINE GEMV configs take fp32 activations.
extern "C" __global__ __launch_bounds__(64) void gemv_q4k_f32_kernel(REF_GEMV_ARGS) { ref_gemv<float, 4>(REF_GEMV_PASS); }
extern "C" __global__ __launch_bounds__(64) void gemv_q6k_f32_kernel(REF_GEMV_ARGS) { ref_gemv<float, 6>(REF_GEMV_PASS); }
extern "C" __global__ __launch_bounds__(64) void gemv_q8_0_f32_kernel(REF_GEMV_ARGS) { ref_gemv<float, 8>(REF_GEMV_PASS); }

// ---------------------------------------------------------------------------
// Exact dequantisers (bit-exact with the NumPy reference: no FMA contraction).
// vte/compiler/dequantizer.py:26-70, 129-169, 172-196.
// ---------------------------------------------------------------------------

extern "C" __global__ __launch_bounds__(256) void dequantize_q4k_kernel(const void* __restrict__ src,
                                                                        float* __restrict__ dst,
                                                                        long long n_blocks) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_blocks * QK_K) return;
    dst[idx] = q4k_elem_exact((const uint8_t*)src + (idx >> 8) * Q4K_BYTES, (int)(idx & 255));
}

extern "C" __global__ __launch_bounds__(256) void dequantize_q6k_kernel(const void* __restrict__ src,
                                                                        float* __restrict__ dst,
                                                                        long long n_blocks) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_blocks * QK_K) return;
    dst[idx] = q6k_elem_exact((const uint8_t*)src + (idx >> 8) * Q6K_BYTES, (int)(idx & 255));
}

extern "C" __global__ __launch_bounds__(256) void dequantize_q8_0_kernel(const void* __restrict__ src,
                                                                         float* __restrict__ dst,
                                                                         long long n_blocks) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_blocks * QK8_0) return;
    dst[idx] = q80_elem_exact((const uint8_t*)src + (idx >> 5) * Q80_BYTES, (int)(idx & 31));
}

// ---------------------------------------------------------------------------
// Host launchers (C++ linkage; the C ABI lives in capi.hip)
// ---------------------------------------------------------------------------

namespace vte {

template <typename TI, typename TO, int NC>
static hipError_t launch_rows(int fmt, const void* x, const void* w, void* y, int M, int K, int N,
                              const void* bias, const void* residual, float rs, hipStream_t st) {
    dim3 grid((N + GEMV_WAVES - 1) / GEMV_WAVES), block(64 * GEMV_WAVES);
    if (fmt == 4) {
        hipLaunchKernelGGL((gemv_q4k_rows<TI, TO, NC>), grid, block, 0, st, (const TI*)x, (const uint8_t*)w,
                           (TO*)y, M, K, N, (const TO*)bias, (const TO*)residual, rs);
    } else {
        const size_t rb = (fmt == 6) ? (size_t)(K / QK_K) * Q6K_BYTES : (size_t)(K / QK8_0) * Q80_BYTES;
        const int stage = (int)((rb + 32 + 15) & ~(size_t)15);
        const size_t lds = (size_t)stage * GEMV_WAVES;
        if (fmt == 6)
            hipLaunchKernelGGL((gemv_staged_rows<TI, TO, NC, 6>), grid, block, lds, st, (const TI*)x,
                               (const uint8_t*)w, (TO*)y, M, K, N, (const TO*)bias, (const TO*)residual, rs,
                               stage);
        else
            hipLaunchKernelGGL((gemv_staged_rows<TI, TO, NC, 8>), grid, block, lds, st, (const TI*)x,
                               (const uint8_t*)w, (TO*)y, M, K, N, (const TO*)bias, (const TO*)residual, rs,
                               stage);
    }
    return hipGetLastError();
}

template <typename TI, typename TO>
hipError_t gemv_valu(int fmt, const void* x, const void* w, void* y, int M, int K, int N, const void* bias,
                     const void* residual, float rs, hipStream_t st) {
    if (M == 1) return launch_rows<TI, TO, 1>(fmt, x, w, y, M, K, N, bias, residual, rs, st);
    if (M == 2) return launch_rows<TI, TO, 2>(fmt, x, w, y, M, K, N, bias, residual, rs, st);
    return launch_rows<TI, TO, 4>(fmt, x, w, y, M, K, N, bias, residual, rs, st);
}

template hipError_t gemv_valu<float, float>(int, const void*, const void*, void*, int, int, int, const void*,
                                            const void*, float, hipStream_t);
template hipError_t gemv_valu<__half, __half>(int, const void*, const void*, void*, int, int, int,
                                              const void*, const void*, float, hipStream_t);
template hipError_t gemv_valu<__half, float>(int, const void*, const void*, void*, int, int, int, const void*,
                                             const void*, float, hipStream_t);

hipError_t dequantize(int fmt, const void* src, float* dst, long long n_elements, hipStream_t st) {
    const long long per = (fmt == 8) ? QK8_0 : QK_K;
    const long long nb = n_elements / per;
    const long long total = nb * per;
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    if (fmt == 4) hipLaunchKernelGGL(dequantize_q4k_kernel, grid, block, 0, st, src, dst, nb);
    else if (fmt == 6) hipLaunchKernelGGL(dequantize_q6k_kernel, grid, block, 0, st, src, dst, nb);
    else hipLaunchKernelGGL(dequantize_q8_0_kernel, grid, block, 0, st, src, dst, nb);
    return hipGetLastError();
}

}  // namespace vte
