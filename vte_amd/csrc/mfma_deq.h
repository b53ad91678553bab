// Weight dequantisation into MFMA A operands (Q4_K / Q6_K super-blocks to
// fp16) and the k-slot map shared by the batched MFMA kernels, gfx950.
//
//  * v_mfma_f32_16x16x32_f16: M = 16 weight rows, N = 16 batch columns, K = 32.
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
#pragma once
#include <cstdlib>
#include "quant.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

union H8 {
    half8_t v;
    uint32_t u[4];
    half2_t h2[4];
};

#define MF_WAVES 8

// bytes b0..b3 of `u` (each < 256, here 6-bit values) -> two fp16 pairs 1024+b.
__device__ __forceinline__ void bytes_to_f16magic(uint32_t u, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// 8 nibble/6-bit values in the bytes of (u0, u1) -> 8 fp16 weights (q - bias) * d - m.
__device__ __forceinline__ half8_t deq8(uint32_t u0, uint32_t u1, _Float16 sub, half2_t d2, half2_t m2) {
    H8 r;
    bytes_to_f16magic(u0, r.u[0], r.u[1]);
    bytes_to_f16magic(u1, r.u[2], r.u[3]);
    const half2_t off = {(_Float16)(1024.0f) + sub, (_Float16)(1024.0f) + sub};
#pragma unroll
    for (int i = 0; i < 4; ++i) r.h2[i] = (r.h2[i] - off) * d2 - m2;
    return r.v;
}

template <typename TI>
__device__ __forceinline__ half8_t load_x8(const TI* p, bool valid);
template <>
__device__ __forceinline__ half8_t load_x8<__half>(const __half* p, bool valid) {
    if (!valid) return half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    return *reinterpret_cast<const half8_t*>(p);
}
template <>
__device__ __forceinline__ half8_t load_x8<float>(const float* p, bool valid) {
    half8_t r = {0, 0, 0, 0, 0, 0, 0, 0};
    if (!valid) return r;
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    r[0] = (_Float16)a.x; r[1] = (_Float16)a.y; r[2] = (_Float16)a.z; r[3] = (_Float16)a.w;
    r[4] = (_Float16)b.x; r[5] = (_Float16)b.y; r[6] = (_Float16)b.z; r[7] = (_Float16)b.w;
    return r;
}

// Element offset (within a super-block) of step t, group g.
template <int FMT>
__device__ __forceinline__ int kslot_base(int t, int g) {
    if (FMT == 4) {
        const int c = g + 4 * (t >> 2);
        return 64 * (c >> 1) + 16 * (c & 1) + 32 * ((t >> 1) & 1) + 8 * (t & 1);
    } else {
        return 128 * (t >> 2) + 32 * (t & 3) + 8 * g;
    }
}


// The eight MFMA A operands (k-steps t = 4*hh + q) of one lane for a Q6_K
// super-block read straight from global memory: the lane's 8-byte slices of
// ql, qh and the scales of each half.  Q6_K blocks are only 2-byte aligned;
// the unaligned 8-byte loads stream as fast as aligned ones on gfx950.
__device__ __forceinline__ uint2 q6_ld8(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
// A lane's raw bytes of one Q6_K super-block (both halves), loaded ahead of
// the dequantisation so several super-blocks can be in flight.
struct Q6Raw {
    uint2 qa[2], qb[2], qh[2], sc[2];
    uint32_t d;
};
__device__ __forceinline__ void q6_raw_load(const uint8_t* blk, int grp, Q6Raw& r) {
    r.d = ((const __attribute__((address_space(1))) uint16_t*)(blk + 208))[0];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        r.qa[hh] = q6_ld8(blk + 64 * hh + 8 * grp);
        r.qb[hh] = q6_ld8(blk + 64 * hh + 32 + 8 * grp);
        r.qh[hh] = q6_ld8(blk + 128 + 32 * hh + 8 * grp);
        r.sc[hh] = q6_ld8(blk + 192 + 8 * hh);
    }
}
__device__ __forceinline__ void q6_raw_operands(const Q6Raw& r, int grp, half8_t (&a)[8]) {
    const float d = h2f_bits(r.d);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const uint2 qa = r.qa[hh], qb = r.qb[hh], qh = r.qh[hh], scw = r.sc[hh];
        const uint64_t sc = ((uint64_t)scw.y << 32) | scw.x;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t u0, u1;
            if (q == 0) {
                u0 = (qa.x & 0x0F0F0F0Fu) | ((qh.x << 4) & 0x30303030u);
                u1 = (qa.y & 0x0F0F0F0Fu) | ((qh.y << 4) & 0x30303030u);
            } else if (q == 1) {
                u0 = (qb.x & 0x0F0F0F0Fu) | ((qh.x << 2) & 0x30303030u);
                u1 = (qb.y & 0x0F0F0F0Fu) | ((qh.y << 2) & 0x30303030u);
            } else if (q == 2) {
                u0 = ((qa.x >> 4) & 0x0F0F0F0Fu) | (qh.x & 0x30303030u);
                u1 = ((qa.y >> 4) & 0x0F0F0F0Fu) | (qh.y & 0x30303030u);
            } else {
                u0 = ((qb.x >> 4) & 0x0F0F0F0Fu) | ((qh.x >> 2) & 0x30303030u);
                u1 = ((qb.y >> 4) & 0x0F0F0F0Fu) | ((qh.y >> 2) & 0x30303030u);
            }
            const int8_t scq = (int8_t)((sc >> (8 * ((grp >> 1) + 2 * q))) & 0xFF);
            const float dsc = d * (float)scq;
            const half2_t d2 = {(_Float16)dsc, (_Float16)dsc};
            const half2_t z2 = {(_Float16)0.0f, (_Float16)0.0f};
            a[4 * hh + q] = deq8(u0, u1, (_Float16)32.0f, d2, z2);
        }
    }
}

__device__ __forceinline__ void q6k_a_operands(const uint8_t* blk, int grp, half8_t (&a)[8]) {
    Q6Raw r;
    q6_raw_load(blk, grp, r);
    q6_raw_operands(r, grp, a);
}

// Q4_K: the header and the lane's two 16-byte code chunks; operands for the
// k-slot map of kslot_base<4>.
struct Q4Raw {
    uint4 h, q0, q1;
};
__device__ __forceinline__ void q4_raw_load(const uint8_t* blk, int grp, Q4Raw& r) {
    r.h = *reinterpret_cast<const uint4*>(blk);
    r.q0 = *reinterpret_cast<const uint4*>(blk + 16 + 16 * grp);
    r.q1 = *reinterpret_cast<const uint4*>(blk + 16 + 16 * (grp + 4));
}
__device__ __forceinline__ void q4_raw_operands(const Q4Raw& r, int grp, half8_t (&a)[8]) {
    Q4KLaneScale s[2];
    s[0] = q4k_lane_scale(r.h, grp >> 1);
    s[1] = q4k_lane_scale(r.h, 2 + (grp >> 1));
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int ci = t >> 2, part = (t >> 1) & 1, e = t & 1;
        const uint4 qc = ci == 0 ? r.q0 : r.q1;
        const uint32_t wa = e == 0 ? qc.x : qc.z, wb = e == 0 ? qc.y : qc.w;
        const uint32_t u0 = part ? ((wa >> 4) & 0x0F0F0F0Fu) : (wa & 0x0F0F0F0Fu);
        const uint32_t u1 = part ? ((wb >> 4) & 0x0F0F0F0Fu) : (wb & 0x0F0F0F0Fu);
        const float dd = part ? s[ci].d_hi : s[ci].d_lo;
        const float mm = part ? s[ci].m_hi : s[ci].m_lo;
        const half2_t d2 = {(_Float16)dd, (_Float16)dd};
        const half2_t m2 = {(_Float16)mm, (_Float16)mm};
        a[t] = deq8(u0, u1, (_Float16)0.0f, d2, m2);
    }
}

// Column groups for a weight-stationary launch of `tiles` row tiles over M
// batch columns, 32 at a time: each group re-reads and re-dequantises the
// weights, each block walks its group's 32-column chunks one after another,
// and `slots` blocks run at once.  Picks the group count with the least
// (rounds of blocks) x (chunks per block), weighted by 1 + groups / 16 for
// the repeated weight reads.
static inline int ws_column_groups(int tiles, int M, int slots) {
    const int chunks = (M + 31) / 32;
    if (const char* v = getenv("VTE_WS_GROUPS")) {  // tuning: pin the group count
        const int g = atoi(v);
        if (g >= 1) return g < chunks ? g : chunks;
    }
    int best = 1;
    double best_cost = 1e30;
    for (int g = 1; g <= chunks; ++g) {
        const int per = (chunks + g - 1) / g;
        const int used = (chunks + per - 1) / per;  // groups that hold columns
        const int rounds = (tiles * used + slots - 1) / slots;
        const double cost = (double)rounds * per * (1.0 + used / 16.0);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = used;
        }
    }
    return best;
}

// Compute units of the current device (cached after the first query).
static inline int device_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    }
    return n;
}
