// Shared GGUF block decoding helpers.
#pragma once
#include "vte_common.h"

// Scales of the two sub-blocks a lane touches.  A lane owns qs chunk c (16 B):
// mblk = c>>1, low nibbles belong to sub-block 2*mblk, high nibbles to
// 2*mblk+1.  Branch-free restatement of get_scale_min_k4
// (vte/compiler/dequantizer.py:6-23) on the three scale words.
struct Q4KLaneScale { float d_lo, m_lo, d_hi, m_hi; };
// The same four 6-bit values as integers: scales and mins of sub-blocks 2*mblk, 2*mblk+1.
struct Q4KLaneInts { uint32_t sc0, mn0, sc1, mn1; };

__device__ __forceinline__ Q4KLaneInts q4k_lane_ints(uint4 h, int mblk) {
    const int sh = (mblk & 1) * 16;
    const uint32_t a = h.y >> sh;  // bytes j, j+1        (j = 2*(mblk&1))
    const uint32_t b = h.z >> sh;  // bytes j+4, j+5
    const uint32_t c = h.w >> sh;  // bytes j+8, j+9
    uint32_t sc0, sc1, mn0, mn1;
    if (mblk < 2) {
        sc0 = a & 63; sc1 = (a >> 8) & 63;
        mn0 = b & 63; mn1 = (b >> 8) & 63;
    } else {
        sc0 = (c & 15) | (((a >> 6) & 3) << 4);
        sc1 = ((c >> 8) & 15) | (((a >> 14) & 3) << 4);
        mn0 = ((c >> 4) & 15) | (((b >> 6) & 3) << 4);
        mn1 = ((c >> 12) & 15) | (((b >> 14) & 3) << 4);
    }
    return Q4KLaneInts{sc0, mn0, sc1, mn1};
}

__device__ __forceinline__ Q4KLaneScale q4k_lane_scale(uint4 h, int mblk) {
    const float d = h2f_bits(h.x);
    const float dmin = h2f_bits(h.x >> 16);
    const Q4KLaneInts i = q4k_lane_ints(h, mblk);
    Q4KLaneScale s;
    s.d_lo = d * (float)i.sc0; s.m_lo = dmin * (float)i.mn0;
    s.d_hi = d * (float)i.sc1; s.m_hi = dmin * (float)i.mn1;
    return s;
}

// 32-bit little-endian read from a 2-byte aligned LDS address.
__device__ __forceinline__ uint32_t lds_u32_a2(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}


// Element e of one block, dequantised exactly as the NumPy dequantiser
// computes it (fp32, every product and difference rounded on its own: no
// FMA contraction).  vte/compiler/dequantizer.py:6-70 (Q4_K), 129-169 (Q6_K),
// 172-196 (Q8_0).
__device__ __forceinline__ float q4k_elem_exact(const uint8_t* blk, int e) {
    const float d = h2f_bits(blk[0] | (blk[1] << 8));
    const float dmin = h2f_bits(blk[2] | (blk[3] << 8));
    const uint8_t* s = blk + 4;
    const int mblk = e >> 6, hi = (e >> 5) & 1, i = e & 31;
    const int j = 2 * mblk + hi;  // sub-block: low nibbles 2*mblk, high nibbles 2*mblk+1
    int sc, mn;
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const uint8_t q = blk[16 + 32 * mblk + i];
    const int nib = hi ? (q >> 4) : (q & 0x0F);
    return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)nib), __fmul_rn(dmin, (float)mn));
}
__device__ __forceinline__ float q6k_elem_exact(const uint8_t* blk, int e) {
    const int half = e >> 7, g = (e >> 5) & 3, l = e & 31;
    const uint8_t qlb = blk[64 * half + l + ((g & 1) ? 32 : 0)];
    const int nib = (g < 2) ? (qlb & 0x0F) : (qlb >> 4);
    const int q = (nib | (((blk[128 + 32 * half + l] >> (2 * g)) & 3) << 4)) - 32;
    const int8_t sc = (int8_t)blk[192 + 8 * half + (l >> 4) + 2 * g];
    const float d = h2f_bits(blk[208] | (blk[209] << 8));
    return __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
}
__device__ __forceinline__ float q80_elem_exact(const uint8_t* blk, int i) {
    return __fmul_rn(h2f_bits(blk[0] | (blk[1] << 8)), (float)(int8_t)blk[2 + i]);
}
