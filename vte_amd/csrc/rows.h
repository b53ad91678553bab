// Block-level quantised row-dot engine (gfx950, 256-thread blocks).
//
// A block computes, for rows [r0, r0 + R) of a raw GGUF matrix and NC
// activation columns held in LDS as fp16, the fp32 dot products
// out[m][r] = sum_k dequant(W[r0 + r, k]) * x[m][k].
//
// Work unit = 64 weights that share one scale pair:
//   Q4_K: (super-block, group mblk): 32 qs bytes at 16 + 32*mblk, both nibble
//         halves (sub-blocks 2*mblk and 2*mblk + 1) -> 2 x 16-byte loads plus
//         the 16-byte header (the 4 lanes of a super-block hit one line).
//   Q6_K: (super-block, half h, l16): ql[64h + l16 .. +15], ql[64h + 32 + l16 ..],
//         qh[32h + l16 ..] and four scales; read from an LDS copy of the
//         block's rows because Q6_K blocks are only 2-byte aligned.
// Units are laid out flat over the block's rows (rows are contiguous runs of
// super-blocks), so every wave load is contiguous whatever K is.  Each unit's
// partial goes to LDS and rows are summed deterministically by whole waves
// (no float atomics: graph replays reproduce bit for bit).
//
// Inner product: 4/6-bit codes become fp16 (1024 + u) with one v_perm_b32 per
// pair and v_dot2_f32_f16 accumulates against fp16 x in fp32; per sub-block
//   sum_i w_i x_i = a * (S - c * X) - b * X,   S = sum (1024 + u_i) x_i,  X = sum x_i
// with (a, b, c) = (d*sc, dmin*m, 1024) for Q4_K and (d*sc, 0, 1056) for Q6_K.
// X comes from per-16-element sums of x precomputed at staging time.
#pragma once
#include "quant.h"

typedef _Float16 rh2_t __attribute__((ext_vector_type(2)));

#define ROWS_THREADS 256

__device__ __forceinline__ float rdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(rh2_t, a), __builtin_bit_cast(rh2_t, b), c, false);
}
__device__ __forceinline__ uint32_t rmagic01(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u); }
__device__ __forceinline__ uint32_t rmagic23(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u); }

// 4 bytes of codes (each < 256) in t against 4 fp16 activations (two words).
__device__ __forceinline__ float dot4_codes(uint32_t t, uint32_t x01, uint32_t x23, float acc) {
    acc = rdot2(rmagic01(t), x01, acc);
    return rdot2(rmagic23(t), x23, acc);
}

// LDS layout for one block's activations: NC fp16 columns of length K and the
// per-16-element sums of each column (float).  Element e of a column lives at
// xpad(e) = e + 8 * (e / 64): a 16-byte pad after every 128 bytes, so the
// 16-byte reads of lanes whose units sit 64 or 128 elements apart fall in
// different LDS banks instead of all hitting the same one.
__host__ __device__ __forceinline__ int xpad(int e) { return e + ((e >> 6) << 3); }
__host__ __device__ __forceinline__ int xpad_len(int K) { return xpad(K); }

struct ActLDS {
    _Float16* x;   // [NC][xpad_len(K)]
    float* s16;    // [NC][K/16]
};

// Stage NC activation columns ([M][K], fp32 or fp16; columns >= M are zero)
// into the padded fp16 LDS layout, plus optionally one more fp16 vector of K
// elements (`extra`, e.g. RMSNorm weights) into `extra_dst` with the same
// layout.  Each thread issues up to 8 independent 16-byte loads before it
// stores any, so the staging costs one memory latency rather than one per
// element.  Chunks of 8 elements stay contiguous in the padded layout (pads
// fall every 64 elements).
template <int NC>
__device__ __forceinline__ void stage_act(const void* __restrict__ x, bool x_f32, int M, int K, _Float16* xs,
                                          const __half* __restrict__ extra = nullptr, _Float16* extra_dst = nullptr) {
    const int ldx = xpad_len(K);
    const int per_col = K / 8;
    const int ncol = NC + (extra != nullptr ? 1 : 0);
    const int nch = ncol * per_col;
    for (int c0 = 0; c0 < nch; c0 += 8 * ROWS_THREADS) {
        uint4 v[8][2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = c0 + j * ROWS_THREADS + threadIdx.x;
            const int m = c / per_col;
            if (c < nch) {
                if (m == NC) {
                    v[j][0] = reinterpret_cast<const uint4*>(extra)[c - NC * per_col];
                } else if (m < M) {
                    if (x_f32) {
                        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(x) + (size_t)c * 8);
                        v[j][0] = p[0];
                        v[j][1] = p[1];
                    } else {
                        v[j][0] = reinterpret_cast<const uint4*>(x)[c];
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = c0 + j * ROWS_THREADS + threadIdx.x;
            if (c >= nch) break;
            const int m = c / per_col, e = (c - m * per_col) * 8;
            if (m == NC) {
                *reinterpret_cast<uint4*>(extra_dst + xpad(e)) = v[j][0];
                continue;
            }
            uint4 o = make_uint4(0, 0, 0, 0);
            if (m < M) {
                if (x_f32) {
                    const float* f = reinterpret_cast<const float*>(&v[j][0]);
                    _Float16 hh[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) hh[i] = (_Float16)f[i];
                    o = *reinterpret_cast<const uint4*>(hh);
                } else {
                    o = v[j][0];
                }
            }
            *reinterpret_cast<uint4*>(xs + (size_t)m * ldx + xpad(e)) = o;
        }
    }
}

// After x is in LDS (and a barrier), fill the per-16 sums.  Caller places a
// barrier afterwards.
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

__device__ __forceinline__ Q4KUnitData q4k_unit_load(const uint8_t* __restrict__ blk, int mblk) {
    Q4KUnitData d;
    d.h = ldg_stream16(blk);
    d.q0 = ldg_stream16(blk + 16 + 32 * mblk);
    d.q1 = ldg_stream16(blk + 32 + 32 * mblk);
    return d;
}

// Partial dot of one unit: xu -> the 64 fp16 activations x[64*mblk ..] of the
// super-block (one unpadded 64-element run of the padded layout), s16 -> their
// four per-16 sums.
__device__ __forceinline__ float q4k_unit_dot(const Q4KUnitData& u, int mblk, const _Float16* xu, const float* s16) {
    const Q4KLaneScale s = q4k_lane_scale(u.h, mblk);
    const uint4* xp = reinterpret_cast<const uint4*>(xu);
    const uint32_t w[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
    float S_l = 0.f, S_h = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 xl = xp[i];      // x[8i .. 8i+7] of the low-nibble sub-block
        const uint4 xh = xp[4 + i];  // x[32 + 8i ..] of the high-nibble sub-block
        const uint32_t lo0 = w[2 * i] & 0x0F0F0F0Fu, lo1 = w[2 * i + 1] & 0x0F0F0F0Fu;
        const uint32_t hi0 = (w[2 * i] >> 4) & 0x0F0F0F0Fu, hi1 = (w[2 * i + 1] >> 4) & 0x0F0F0F0Fu;
        S_l = dot4_codes(lo0, xl.x, xl.y, S_l);
        S_l = dot4_codes(lo1, xl.z, xl.w, S_l);
        S_h = dot4_codes(hi0, xh.x, xh.y, S_h);
        S_h = dot4_codes(hi1, xh.z, xh.w, S_h);
    }
    const float sx_lo = s16[0] + s16[1], sx_hi = s16[2] + s16[3];
    float r = s.d_lo * fmaf(-1024.f, sx_lo, S_l);
    r = fmaf(-s.m_lo, sx_lo, r);
    r = fmaf(s.d_hi, fmaf(-1024.f, sx_hi, S_h), r);
    return fmaf(-s.m_hi, sx_hi, r);
}

// ---------------------------------------------------------------------------
// Q6_K (from an LDS copy of the rows; blocks are 2-byte aligned)
// ---------------------------------------------------------------------------
// Four little-endian dwords starting at a 2-byte aligned LDS address: five
// 4-byte aligned LDS reads (the pointer is cast to the LDS address space, so
// they are ds_read instructions, which the compiler may pair into
// ds_read2_b32 -- each still naturally aligned, as misaligned wide LDS reads
// stall) and byte alignment in registers (the shift is 0 or 2).
typedef __attribute__((address_space(3))) const uint32_t lds_u32_t;
__device__ __forceinline__ void lds_16b_a2(const uint8_t* p, uint32_t (&o)[4]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    lds_u32_t* q = (lds_u32_t*)(reinterpret_cast<const uint8_t*>(a & ~(uintptr_t)3));
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t d[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) d[i] = q[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// unit (h, l16) of a super-block: 64 weights at 128h + l16 + i + 32g
// (i < 16, g < 4).  xsb -> the super-block's x in the padded layout
// (element e at xpad(e)), s16sb -> its per-16 sums.
__device__ __forceinline__ float q6k_unit_dot(const uint8_t* blk, int h, int l16, const _Float16* xsb,
                                              const float* s16sb) {
    const float d = h2f_bits(*reinterpret_cast<const uint16_t*>(blk + 208));
    const uint8_t* qa = blk + 64 * h + l16;
    const uint8_t* qhp = blk + 128 + 32 * h + l16;
    uint32_t la[4], lb[4], hw[4];
    lds_16b_a2(qa, la);
    lds_16b_a2(qa + 32, lb);
    lds_16b_a2(qhp, hw);
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * h + (l16 >> 4));
    float r = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4* xp = reinterpret_cast<const uint4*>(xsb + xpad(128 * h + l16 + 32 * g));
        const uint4 x0 = xp[0], x1 = xp[1];
        float S = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t l = (g & 1) ? lb[i] : la[i];
            const uint32_t nib = (g < 2) ? (l & 0x0F0F0F0Fu) : ((l >> 4) & 0x0F0F0F0Fu);
            const uint32_t u = nib | (((hw[i] >> (2 * g)) & 0x03030303u) << 4);
            const uint4 xv = (i < 2) ? x0 : x1;
            const uint32_t x01 = (i & 1) ? xv.z : xv.x;
            const uint32_t x23 = (i & 1) ? xv.w : xv.y;
            S = dot4_codes(u, x01, x23, S);
        }
        const float X = s16sb[(128 * h + l16 + 32 * g) >> 4];
        r = fmaf(d * (float)sc[2 * g], fmaf(-1056.f, X, S), r);
    }
    return r;
}
