// Mat-vec behind the reference's GEMV ABI (gfx950, wave64).
//
// The ABI fixes the launch: grid (out_features, batch * seq_len), one
// 64-thread block per output row (vte/core/fallback_executor.py:140-148).  A
// wave that walks one row super-block by super-block keeps few loads in
// flight and fetches the row's activations again for every row; here the
// work of a block is laid out for the wave instead:
//  * work unit = 64 weights sharing one scale pair (rows.h), a row holds
//    U = K / 64 of them; the lanes form G = 64 / U row groups when U < 64
//    (U = 24 at K = 1536: two groups of 24 lanes) and a lane takes units
//    li, li + 64, ... of its group's row otherwise;
//  * a lane loads the activations of its units once (global -> registers, in
//    the paired fp16 layout and per-16 sums of the fused mat-vec) and keeps
//    them for every row it visits;
//  * block b takes R consecutive rows (R a multiple of G, larger for tall
//    matrices so the activations are fetched once per R rows); blocks past
//    ceil(N / R) leave at once.  The grid must hold at least ceil(N / R)
//    blocks in x, which the ABI's grid (N blocks) does;
//  * every weight load of a row is issued before its products, and the next
//    row's loads before this row's products;
//  * the unit products are the fused mat-vec's (rows.h, fused_kernels.h):
//    codes as fp16 (1024 + q) against fp16 activations with fp32 sums, the
//    scales applied per sub-block in fp32; the lanes' sums meet in LDS.
// fp32 activations (the `_f32` siblings) are rounded to fp16 on load, as in
// the fused mat-vec's staging.
#pragma once
#include "fused_kernels.h"

#define REF_MV_MAX_K 16384

// 16 activations from global memory as the paired fp16 words of the fused
// layout (two chunks of 4 words) and their fp32 sum.
template <typename T>
__device__ __forceinline__ void ref_x16(const T* p, uint4& a, uint4& b, float& s);
template <>
__device__ __forceinline__ void ref_x16<__half>(const __half* p, uint4& a, uint4& b, float& s) {
    const uint4 u = ldg_g16(p), v = ldg_g16(p + 8);
    uint32_t h0[4] = {u.x, u.y, u.z, u.w}, h1[4] = {v.x, v.y, v.z, v.w};
    s = chunk_sum(h0) + chunk_sum(h1);
    xperm_words(h0[0], h0[1]);
    xperm_words(h0[2], h0[3]);
    xperm_words(h1[0], h1[1]);
    xperm_words(h1[2], h1[3]);
    a = make_uint4(h0[0], h0[1], h0[2], h0[3]);
    b = make_uint4(h1[0], h1[1], h1[2], h1[3]);
}
template <>
__device__ __forceinline__ void ref_x16<float>(const float* p, uint4& a, uint4& b, float& s) {
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 f = ldg_g16(p + 4 * i);
        const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(f.x)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(f.y)) << 16);
        const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(f.z)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(f.w)) << 16);
        h[2 * i] = lo;
        h[2 * i + 1] = hi;
    }
    uint32_t h0[4] = {h[0], h[1], h[2], h[3]}, h1[4] = {h[4], h[5], h[6], h[7]};
    s = chunk_sum(h0) + chunk_sum(h1);
    xperm_words(h0[0], h0[1]);
    xperm_words(h0[2], h0[3]);
    xperm_words(h1[0], h1[1]);
    xperm_words(h1[2], h1[3]);
    a = make_uint4(h0[0], h0[1], h0[2], h0[3]);
    b = make_uint4(h1[0], h1[1], h1[2], h1[3]);
}

// Activations of unit kr of column xm: four runs of 16 elements (Q4_K and
// Q8_0: the unit's 64 consecutive elements; Q6_K unit (h, l16) of super-block
// sb: 128 h + l16 + 32 g, g < 4), as x[2g], x[2g + 1] with sums s[g].
template <typename T, int FMT>
__device__ __forceinline__ void ref_unit_x(const T* xm, int kr, uint4 (&x)[8], float (&s)[4]) {
    const int sb = kr >> 2, q = kr & 3;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int e = FMT == 6 ? sb * QK_K + 128 * (q >> 1) + (q & 1) * 16 + 32 * g : 64 * kr + 16 * g;
        ref_x16<T>(xm + e, x[2 * g], x[2 * g + 1], s[g]);
    }
}

// Raw bytes of one unit of a row (the loads of tile_w_issue for one unit).
struct RefW {
    uint4 a, b, c, d;
    uint2 sc8;
    uint32_t dbits;
};
template <int FMT>
__device__ __forceinline__ void ref_unit_w(const uint8_t* rowp, int kr, RefW& w) {
    const int sb = kr >> 2, q = kr & 3;
    if (FMT == 4) {
        const uint8_t* blk = rowp + (size_t)sb * Q4K_BYTES;  // rows and blocks 16-byte aligned
        w.a = ldg_g16(blk);
        w.b = ldg_g16(blk + 16 + 32 * q);
        w.c = ldg_g16(blk + 32 + 32 * q);
    } else if (FMT == 8) {  // blocks 2 kr, 2 kr + 1 (2-byte aligned)
        const uint8_t* blk = rowp + (size_t)kr * (2 * Q80_BYTES);
        w.a = ldg_u16b(blk + 2);
        w.b = ldg_u16b(blk + 18);
        w.c = ldg_u16b(blk + Q80_BYTES + 2);
        w.d = ldg_u16b(blk + Q80_BYTES + 18);
        w.dbits = ldg_b16(blk, 0) | (ldg_b16(blk + Q80_BYTES, 0) << 16);
    } else {
        const uint8_t* blk = rowp + (size_t)sb * Q6K_BYTES;
        const int h = q >> 1, l16 = (q & 1) * 16;
        w.a = ldg_u16b(blk + 64 * h + l16);
        w.b = ldg_u16b(blk + 64 * h + 32 + l16);
        w.c = ldg_u16b(blk + 128 + 32 * h + l16);
        __builtin_memcpy(&w.sc8, blk + 192 + 8 * h, 8);
        w.dbits = ldg_b16(blk + 208, 0);
    }
}
template <int FMT>
__device__ __forceinline__ float ref_unit_dot(const RefW& w, int kr, const uint4 (&x)[8], const float (&s)[4]) {
    const int q = kr & 3;
    if (FMT == 4) return q4k_unit_dot_x(Q4KUnitData{w.a, w.b, w.c}, q, x, s);
    if (FMT == 8) return q80_unit_dot_x(w.a, w.b, w.c, w.d, w.dbits, x, s);
    return q6k_unit_dot_x(w.a, w.b, w.c, w.sc8, w.dbits, (q & 1) * 16, x, s);
}

__host__ __device__ __forceinline__ int ref_mv_groups(int K) {
    const int U = K / 64;
    return U < 64 ? 64 / U : 1;
}
// Rows per block: about N / 4096 (at least G, at most 16, a multiple of G);
// one row for K > 4096.
__host__ __device__ __forceinline__ int ref_mv_rows(int N, int K) {
    const int G = ref_mv_groups(K);
    if (K > 64 * 64) return 1;
    int r = N / 4096;
    r = r < 1 ? 1 : (r > 16 ? 16 : r);
    return (r + G - 1) / G * G;
}
// Shapes this mat-vec serves (the others keep the one-row-per-wave kernels).
__host__ __device__ __forceinline__ bool ref_mv_ok(int K) {
    return K % 64 == 0 && K >= 64 && K <= REF_MV_MAX_K;
}

template <typename T, int FMT, int UPL>
__device__ __forceinline__ void ref_mv(const T* __restrict__ x, const uint8_t* __restrict__ w, T* __restrict__ y,
                                       int M, int K, int N, const T* __restrict__ bias,
                                       const T* __restrict__ residual, float rs, float* part) {
    const int m = blockIdx.y;
    const int U = K / 64, G = ref_mv_groups(K), LG = U < 64 ? U : 64;
    const int R = ref_mv_rows(N, K), r0 = blockIdx.x * R;
    if (m >= M || r0 >= N) return;
    const int lane = threadIdx.x, grp = lane / LG, li = lane - grp * LG;
    const bool act = grp < G;
    const size_t rb = FMT == 4 ? (size_t)(K / QK_K) * Q4K_BYTES
                    : FMT == 6 ? (size_t)(K / QK_K) * Q6K_BYTES : (size_t)(K / QK8_0) * Q80_BYTES;
    const T* xm = x + (size_t)m * K;
    // units li + LG j of the row (j < UPL): present when below U
    bool has[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) has[j] = act && li + LG * j < U;
    RefW W[UPL];
    auto issue = [&](int row, RefW (&dst)[UPL]) {
        const uint8_t* rowp = w + (size_t)(row < N ? row : N - 1) * rb;
#pragma unroll
        for (int j = 0; j < UPL; ++j)
            if (has[j]) ref_unit_w<FMT>(rowp, li + LG * j, dst[j]);
    };
    issue(r0 + grp, W);
    uint4 xv[UPL][8];
    float xs[UPL][4];
#pragma unroll
    for (int j = 0; j < UPL; ++j)
        if (has[j]) ref_unit_x<T, FMT>(xm, li + LG * j, xv[j], xs[j]);
    for (int it = 0; it < R; it += G) {
        const int row = r0 + it + grp;
        RefW Wn[UPL];
        const bool more = it + G < R && r0 + it + G < N;
        if (more) issue(row + G, Wn);
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j)
            if (has[j]) acc += ref_unit_dot<FMT>(W[j], li + LG * j, xv[j], xs[j]);
        part[lane] = acc;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (lane < G && r0 + it + lane < N) {
            float s = 0.f;
            for (int i = 0; i < LG; ++i) s += part[lane * LG + i];
            gemv_store<T>(y, bias, residual, rs, r0 + it + lane, m, N, s);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (!more) break;
#pragma unroll
        for (int j = 0; j < UPL; ++j) W[j] = Wn[j];
    }
}

// Rows of more than 64 units (K > 4096): one row per block, the lane's units
// lane, lane + 64, ... walked with the next unit's weights requested before
// the current unit's activations (L2 hits) and products.
template <typename T, int FMT>
__device__ __forceinline__ void ref_mv_long(const T* __restrict__ x, const uint8_t* __restrict__ w, T* __restrict__ y,
                                            int M, int K, int N, const T* __restrict__ bias,
                                            const T* __restrict__ residual, float rs, float* part) {
    const int m = blockIdx.y, row = blockIdx.x;
    if (m >= M || row >= N) return;
    const int U = K / 64, lane = threadIdx.x;
    const size_t rb = FMT == 4 ? (size_t)(K / QK_K) * Q4K_BYTES
                    : FMT == 6 ? (size_t)(K / QK_K) * Q6K_BYTES : (size_t)(K / QK8_0) * Q80_BYTES;
    const uint8_t* rowp = w + (size_t)row * rb;
    const T* xm = x + (size_t)m * K;
    RefW W;
    ref_unit_w<FMT>(rowp, lane, W);  // U > 64: every lane has a first unit
    float acc = 0.f;
    for (int kr = lane; kr < U; kr += 64) {
        const bool more = kr + 64 < U;
        RefW Wn;
        if (more) ref_unit_w<FMT>(rowp, kr + 64, Wn);
        uint4 xv[8];
        float xs[4];
        ref_unit_x<T, FMT>(xm, kr, xv, xs);
        acc += ref_unit_dot<FMT>(W, kr, xv, xs);
        if (!more) break;
        W = Wn;
    }
    acc = wave_sum(acc);
    if (lane == 0) gemv_store<T>(y, bias, residual, rs, row, m, N, acc);
}

template <typename T, int FMT>
__device__ __forceinline__ void ref_mv_dispatch(const T* x, const uint8_t* w, T* y, int M, int K, int N, const T* bias,
                                                const T* residual, float rs, float* part) {
    if (K <= 64 * 64) ref_mv<T, FMT, 1>(x, w, y, M, K, N, bias, residual, rs, part);
    else ref_mv_long<T, FMT>(x, w, y, M, K, N, bias, residual, rs, part);
}
