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

