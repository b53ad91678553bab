// Quantised row-dot pieces shared by the mat-vec kernels (gfx950, wave64).
//
// Work unit = 64 weights of one row that share one scale pair:
//   Q4_K: (super-block, group mblk): 32 qs bytes at 16 + 32*mblk, both nibble
//         halves (sub-blocks 2*mblk and 2*mblk + 1) -> 2 x 16-byte loads plus
//         the 16-byte header (the 4 lanes of a super-block hit one line).
//   Q6_K: (super-block, half h, l16): ql[64h + l16 .. +15], ql[64h + 32 + l16 ..],
//         qh[32h + l16 ..], four scales and d (unaligned 16-byte loads:
//         Q6_K blocks are only 2-byte aligned).
//
// Inner product: codes become fp16 (1024 + u) by placing them under the
// exponent of 1024 (0x6400), and v_dot2_f32_f16 accumulates two of them
// against two fp16 activations in fp32; per sub-block
//   sum_i w_i x_i = a * (S - c * X) - b * X,   S = sum (1024 + u_i) x_i,  X = sum x_i
// with (a, b, c) = (d*sc, dmin*m, 1024) for Q4_K and (d*sc, 0, 1056) for Q6_K.
// X comes from per-16-element sums of x precomputed at staging time.
//
// Activation layout in LDS: each group of four elements is stored as
// [x0, x2, x1, x3] (xperm), so one 32-bit word pairs the activations of code
// bytes 0 and 2, or 1 and 3, of a code word.  A Q4_K word w then needs one
// v_and_or_b32 per pair of codes: (w & 0x000F000F) | 0x64006400 is the fp16
// pair (1024 + lo0, 1024 + lo2), (w & 0x00F000F0) | 0x64006400 the pair
// (1024 + 16 hi0, 1024 + 16 hi2); the same on w >> 8 gives bytes 1 and 3.
#pragma once
#include "quant.h"

typedef _Float16 rh2_t __attribute__((ext_vector_type(2)));

#define ROWS_THREADS 256

__device__ __forceinline__ float rdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(rh2_t, a), __builtin_bit_cast(rh2_t, b), c, false);
}
// fp16 pairs (1024 + byte0, 1024 + byte2) and (1024 + byte1, 1024 + byte3) of t
__device__ __forceinline__ uint32_t rmagic02(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04020400u); }
__device__ __forceinline__ uint32_t rmagic13(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04030401u); }

// 4 bytes of codes (each < 256) in t against 4 activations in the xperm
// layout (words (x0, x2) and (x1, x3)).
__device__ __forceinline__ float dot4_codes(uint32_t t, uint32_t x02, uint32_t x13, float acc) {
    acc = rdot2(rmagic02(t), x02, acc);
    return rdot2(rmagic13(t), x13, acc);
}

// LDS layout for one block's activations: NC fp16 columns of length K and the
// per-16-element sums of each column (float).  Element e of a column lives at
// xpad(xperm(e)), xpad(p) = p + 8 * (p / 64): a 16-byte pad after every 128
// bytes, so the 16-byte reads of lanes whose units sit 64 or 128 elements
// apart fall in different LDS banks instead of all hitting the same one.
__host__ __device__ __forceinline__ int xpad(int e) { return e + ((e >> 6) << 3); }
__host__ __device__ __forceinline__ int xpad_len(int K) { return xpad(K); }
__host__ __device__ __forceinline__ int xperm(int e) { return (e & ~3) | ((e & 1) << 1) | ((e >> 1) & 1); }

// Two natural-order words (x0, x1), (x2, x3) -> the xperm words (x0, x2), (x1, x3).
__device__ __forceinline__ void xperm_words(uint32_t& a, uint32_t& b) {
    const uint32_t p = __builtin_amdgcn_perm(b, a, 0x05040100u);
    const uint32_t q = __builtin_amdgcn_perm(b, a, 0x07060302u);
    a = p;
    b = q;
}

struct ActLDS {
    _Float16* x;   // [NC][xpad_len(K)]
    float* s16;    // [NC][K/16]
};

// After x is in LDS (and a barrier), fill the per-16 sums (the xperm order
// does not change a 16-element sum).  Caller places a barrier afterwards.
template <int NC>
__device__ __forceinline__ void act_sums(ActLDS a, int K) {
    const int nseg = K / 16;
    const int ld = xpad_len(K);
    for (int i = threadIdx.x; i < NC * nseg; i += blockDim.x) {
        const int m = i / nseg, s = i % nseg;
        const uint4* p = reinterpret_cast<const uint4*>(a.x + (size_t)m * ld + xpad(16 * s));
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint4 v = p[j];
            acc = rdot2(v.x, 0x3C003C00u, acc);
            acc = rdot2(v.y, 0x3C003C00u, acc);
            acc = rdot2(v.z, 0x3C003C00u, acc);
            acc = rdot2(v.w, 0x3C003C00u, acc);
        }
        a.s16[i] = acc;
    }
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------
struct Q4KUnitData {
    uint4 h, q0, q1;
};

// Partial dot of one unit: x -> the 64 activations x[64*mblk ..] of the
// super-block in the xperm layout (8 words of 16 bytes), s -> their four
// per-16 sums.  Four accumulators keep the dependent chains short.
__device__ __forceinline__ float q4k_unit_dot_x(const Q4KUnitData& u, int mblk, const uint4 (&x)[8],
                                                const float (&s16)[4]) {
    const Q4KLaneScale s = q4k_lane_scale(u.h, mblk);
    const uint32_t w[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
    // 0x64006400 in a VGPR: VOP3 instructions take no literal on this target,
    // so (w & mask) | magic is one v_and_or_b32 only with the mask in an SGPR
    // and the magic in a VGPR
    uint32_t mg;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mg));
    float Sl[2] = {0.f, 0.f}, Sh[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 xl = x[i];      // x[8i .. 8i+7] of the low-nibble sub-block
        const uint4 xh = x[4 + i];  // x[32 + 8i ..] of the high-nibble sub-block
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t a = w[2 * i + j], b = a >> 8;
            const uint32_t xl02 = j ? xl.z : xl.x, xl13 = j ? xl.w : xl.y;
            const uint32_t xh02 = j ? xh.z : xh.x, xh13 = j ? xh.w : xh.y;
            Sl[j] = rdot2((a & 0x000F000Fu) | mg, xl02, Sl[j]);
            Sl[j] = rdot2((b & 0x000F000Fu) | mg, xl13, Sl[j]);
            Sh[j] = rdot2((a & 0x00F000F0u) | mg, xh02, Sh[j]);
            Sh[j] = rdot2((b & 0x00F000F0u) | mg, xh13, Sh[j]);
        }
    }
    const float S_l = Sl[0] + Sl[1];
    const float S_h = Sh[0] + Sh[1];  // sum (1024 + 16 u) x
    const float sx_lo = s16[0] + s16[1], sx_hi = s16[2] + s16[3];
    float r = s.d_lo * fmaf(-1024.f, sx_lo, S_l);
    r = fmaf(-s.m_lo, sx_lo, r);
    r = fmaf(s.d_hi * 0.0625f, fmaf(-1024.f, sx_hi, S_h), r);
    return fmaf(-s.m_hi, sx_hi, r);
}

// Activations of a Q4_K unit from LDS: xu -> x[64*mblk ..] (one unpadded
// 64-element run of the padded layout), s16 -> its four per-16 sums.
__device__ __forceinline__ void q4k_unit_x(const _Float16* xu, const float* s16, uint4 (&x)[8], float (&s)[4]) {
    const uint4* xp = reinterpret_cast<const uint4*>(xu);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = xp[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = s16[i];
}
