// Quantised weights as exact MFMA operands (Q4_K / Q6_K super-blocks) and the
// k-slot map shared by the batched MFMA kernels, gfx950.
//
//  * v_mfma_f32_16x16x32_f16 with the activations as the A operand (M = 16
//    batch columns) and the weights as the B operand (N = 16 weight rows),
//    K = 32: C[m][n] lands in lane (n, g) as batch columns 4g .. 4g+3 of
//    weight row n, the lane that loaded row n's super-block, so the
//    super-block scales apply lane-locally.
//  * Exact weight operands: a super-block's weights are d * (sc_j * q) -
//    dmin * m_j (Q4_K) or d * (sc_j * (q - 32)) (Q6_K), with 4/6-bit codes
//    q and 6/8-bit sub-block scales sc_j, m_j.  The operands are the integer
//    products sc_j * q (<= 945) and sc_j * (q - 32) (exact in fp16 while
//    |sc_j| <= 64, one rounding of an integer product beyond), made with
//    packed fp16 math from the code bytes (nibble -> 0x64xx magic = 1024 + q);
//    the Q4_K minimum term is either one MFMA per k-step of the activations
//    against the splat 6-bit minimum (launches of at most 16 columns) or one
//    MFMA of the activations' sub-block sums (formed once per super-block and
//    wave, q4_xmin) against the row's eight minima (longer batches).  The MFMA sums a super-block in fp32 and the fp32
//    scales d, dmin are applied once per super-block (sb_mfma).  The weights
//    therefore enter the sums exactly as the reference's fp32 dequantisation
//    defines them (vte/compiler/dequantizer.py:26-70, 129-169); only the fp16
//    activations and the fp32 sums round.
//  * K-slot permutation: MFMA pairs A and B by (lane group, slot), so any
//    bijection of super-block elements to (k-step, group, slot) is valid as
//    long as A and B use the same one.  The map is chosen so each lane's 8
//    slots are 8 contiguous elements sharing one sub-block scale:
//      Q4_K step t, group g: qs chunk c = g + 4*(t>>2), nibble (t>>1)&1, half t&1
//           (sub-block 2 * ((g>>1) + 2*(t>>2)) + ((t>>1)&1); steps 2s, 2s+1 share one)
//      Q6_K step t, group g: half h = g>>1, quarter q = t>>1, l = 16 (g&1) + 8 (t&1) .. +7
//           (16-element sub-block 8h + 2q + (g&1)); a lane's codes for all 8
//           steps come from three 16-byte runs of its row's block (ql, ql + 32, qh)
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

// bytes b0..b3 of `u` (each < 256) -> two fp16 pairs 1024+b.
__device__ __forceinline__ void bytes_to_f16magic(uint32_t u, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// 8 codes in the bytes of (u0, u1) -> 8 fp16 values (1024 + q) * s + c: with
// c = -1024 s the exact integer q * s, with c = -1056 s the integer (q - 32) * s.
__device__ __forceinline__ half8_t codes8(uint32_t u0, uint32_t u1, half2_t s2, half2_t c2) {
    H8 r;
    bytes_to_f16magic(u0, r.u[0], r.u[1]);
    bytes_to_f16magic(u1, r.u[2], r.u[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.h2[i] = __builtin_elementwise_fma(r.h2[i], s2, c2);  // one rounding: exact
    return r.v;
}

__device__ __forceinline__ half2_t splat2(float v) { return half2_t{(_Float16)v, (_Float16)v}; }

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
        return 128 * (g >> 1) + 32 * (t >> 1) + 16 * (g & 1) + 8 * (t & 1);
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
    uint4 la, lb, hq;  // ql[64h + 16j ..], ql[64h + 32 + 16j ..], qh[32h + 16j ..] (h = g>>1, j = g&1)
    uint2 sc;          // scales 8h .. 8h+7
    uint32_t d;
};
__device__ __forceinline__ uint4 q6_ld16(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ void q6_raw_load(const uint8_t* blk, int grp, Q6Raw& r) {
    const int h = grp >> 1, j = grp & 1;
    r.la = q6_ld16(blk + 64 * h + 16 * j);
    r.lb = q6_ld16(blk + 64 * h + 32 + 16 * j);
    r.hq = q6_ld16(blk + 128 + 32 * h + 16 * j);
    r.sc = q6_ld8(blk + 192 + 8 * h);
    r.d = ((const __attribute__((address_space(1))) uint16_t*)(blk + 208))[0];
}
// Exact operands of one super-block for one lane: the 8 k-steps' weight
// operands and the fp32 scales (Q4_K: also the 4 sub-block minima, splat).
struct Q6Ops {
    half8_t w[8];
    float d;
};
struct Q4Ops {
    half8_t w[8];
    half8_t mins;   // XM: lane groups 0-1 the row's eight sub-block minima m_0..m_7, groups 2-3 zero
    uint32_t mnb;   // !XM: byte s = m_j of the lane's sub-block of steps 2s, 2s+1
    float d, dmin;
};

__device__ __forceinline__ void q6_exact_operands(const Q6Raw& r, int grp, Q6Ops& o) {
    o.d = h2f_bits(r.d);
    const uint32_t la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
    const uint32_t lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
    const uint32_t hq[4] = {r.hq.x, r.hq.y, r.hq.z, r.hq.w};
    const uint64_t sc = ((uint64_t)r.sc.y << 32) | r.sc.x;
    const int j = grp & 1;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int q = t >> 1, w0 = 2 * (t & 1);  // quarter; first code word of the step's 8 codes
        uint32_t u[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t l = (q & 1) ? lb[w0 + e] : la[w0 + e];
            const uint32_t nib = (q < 2) ? (l & 0x0F0F0F0Fu) : ((l >> 4) & 0x0F0F0F0Fu);
            u[e] = nib | (((hq[w0 + e] >> (2 * q)) & 0x03030303u) << 4);
        }
        const float scq = (float)(int8_t)((sc >> (8 * (2 * q + j))) & 0xFF);
        // (1024 + u) - 1056 = u - 32 exactly, then one multiply by the integer scale
        H8 v;
        bytes_to_f16magic(u[0], v.u[0], v.u[1]);
        bytes_to_f16magic(u[1], v.u[2], v.u[3]);
        const half2_t off = splat2(-1056.0f), s2 = splat2(scq);
#pragma unroll
        for (int i = 0; i < 4; ++i) v.h2[i] = (v.h2[i] + off) * s2;
        o.w[t] = v.v;
    }
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
template <bool XM>
__device__ __forceinline__ void q4_exact_operands(const Q4Raw& r, int grp, Q4Ops& o) {
    o.d = h2f_bits(r.h.x);
    o.dmin = h2f_bits(r.h.x >> 16);
    Q4KLaneInts s[2];
    s[0] = q4k_lane_ints(r.h, grp >> 1);
    s[1] = q4k_lane_ints(r.h, 2 + (grp >> 1));
    if constexpr (!XM) {
        o.mnb = s[0].mn0 | (s[0].mn1 << 8) | (s[1].mn0 << 16) | (s[1].mn1 << 24);
    } else {
        half8_t mv;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const Q4KLaneInts v = q4k_lane_ints(r.h, mb);
            mv[2 * mb] = grp < 2 ? (_Float16)(float)v.mn0 : (_Float16)0.0f;
            mv[2 * mb + 1] = grp < 2 ? (_Float16)(float)v.mn1 : (_Float16)0.0f;
        }
        o.mins = mv;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int ci = t >> 2, part = (t >> 1) & 1, e = t & 1;
        const uint4 qc = ci == 0 ? r.q0 : r.q1;
        const uint32_t wa = e == 0 ? qc.x : qc.z, wb = e == 0 ? qc.y : qc.w;
        const uint32_t u0 = part ? ((wa >> 4) & 0x0F0F0F0Fu) : (wa & 0x0F0F0F0Fu);
        const uint32_t u1 = part ? ((wb >> 4) & 0x0F0F0F0Fu) : (wb & 0x0F0F0F0Fu);
        const float sc = (float)(part ? s[ci].sc1 : s[ci].sc0);
        o.w[t] = codes8(u0, u1, splat2(sc), splat2(-1024.0f * sc));
    }
}

// Sub-block sums of the activations of one super-block, X[m][j] = sum of
// x[m][k] over sub-block j (Q4_K: 8 sub-blocks of 32), for the minimum term
// dmin * sum_j m_j X[m][j], which is the same for every weight row of the
// tile and so is formed once per super-block and wave: eight MFMAs of the
// activation operands against 0/1 sub-block indicators (exact fp32 sums),
// then, through the wave's LDS scratch `xl` [NT][16][8], the A-operand layout
// with X split into fp16 hi (lane group 0) and lo (group 1) parts, so the
// single MFMA against the row minima (Q4Ops::mins) sums hi + lo to ~2^-22.
// This form (XM) pays off where several row tiles or column tiles share the
// sums (weight-stationary and multi-tile launches).  With one row tile and
// one column tile per super-block and wave (the batched decode launches) its
// serial chain (indicator MFMAs, LDS round trip) lies on the critical path,
// and the !XM form instead adds one MFMA per k-step of the activations
// against the splat minimum of the step's sub-block, independent of the
// weight MFMAs.  The two forms round the minimum term differently (both sum
// in fp32; results agree to fp32 rounding, not bit for bit).
template <int NT, bool XM>
struct XMin {
    half8_t xa[NT];
};
template <int NT>
struct XMin<NT, false> {};
template <int NT>
__device__ __forceinline__ void q4_xmin(const half8_t (&bx)[8][NT], float* xl, XMin<NT, true>& xm) {
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    floatx4_t cx[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) cx[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int sub = 2 * ((grp >> 1) + 2 * (t >> 2)) + ((t >> 1) & 1);  // sub-block of step t, group grp
        const _Float16 one = col == sub ? (_Float16)1.0f : (_Float16)0.0f;
        const half8_t ind = {one, one, one, one, one, one, one, one};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) cx[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[t][nt], ind, cx[nt], 0, 0, 0);
    }
    // C layout: lane (j, grp) holds X[4 grp + i][j]
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (col < 8) xl[(nt * 16 + 4 * grp + i) * 8 + col] = cx[nt][i];
    // a wave's LDS operations complete in order: wait for the stores (LDS
    // counter only, the weight prefetches stay in flight) before the reads
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float4 a = *reinterpret_cast<const float4*>(xl + (nt * 16 + col) * 8);
        const float4 b = *reinterpret_cast<const float4*>(xl + (nt * 16 + col) * 8 + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        half8_t h;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const _Float16 hi = (_Float16)v[j];
            const _Float16 lo = (_Float16)(v[j] - (float)hi);
            h[j] = grp == 0 ? hi : (grp == 1 ? lo : (_Float16)0.0f);
        }
        xm.xa[nt] = h;
    }
    asm volatile("" ::: "memory");  // xl is rewritten by the next call
}

// One super-block of MFMA work for NT 16-column activation tiles bx[t][nt]
// (A operands, k-slot map of the format) against one lane's exact weight
// operands: acc[nt] += d * sum(w x) [- dmin * sum_j m_j X_j], the sums in fp32
// over the super-block's 8 k-steps in order.  Every batched kernel goes
// through these functions, so for a given minimum-term form (XM) a weight
// row's result depends only on which super-blocks a wave sums (and the order
// the waves' partials are added), not on the kernel or the number of columns.
template <int NT, bool XM>
__device__ __forceinline__ void sb_mfma(const Q6Ops& o, const half8_t (&bx)[8][NT], const XMin<NT, XM>&,
                                        floatx4_t (&acc)[NT]) {
    floatx4_t aw[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) aw[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) aw[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[t][nt], o.w[t], aw[nt], 0, 0, 0);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] = fmaf(o.d, aw[nt][i], acc[nt][i]);
}
template <int NT>
__device__ __forceinline__ void sb_mfma(const Q4Ops& o, const half8_t (&bx)[8][NT], const XMin<NT, true>& xm,
                                        floatx4_t (&acc)[NT]) {
    floatx4_t aw[NT], am[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        aw[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        am[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xm.xa[nt], o.mins, floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) aw[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[t][nt], o.w[t], aw[nt], 0, 0, 0);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] = fmaf(-o.dmin, am[nt][i], fmaf(o.d, aw[nt][i], acc[nt][i]));
}

template <int NT>
__device__ __forceinline__ void sb_mfma(const Q4Ops& o, const half8_t (&bx)[8][NT], const XMin<NT, false>&,
                                        floatx4_t (&acc)[NT]) {
    floatx4_t aw[NT], am[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) aw[nt] = am[nt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const _Float16 m = (_Float16)(float)((o.mnb >> (8 * (t >> 1))) & 0xFFu);
        const half8_t mv = {m, m, m, m, m, m, m, m};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            aw[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[t][nt], o.w[t], aw[nt], 0, 0, 0);
            am[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[t][nt], mv, am[nt], 0, 0, 0);
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] = fmaf(-o.dmin, am[nt][i], fmaf(o.d, aw[nt][i], acc[nt][i]));
}

// The minimum-term sums where the format has one (Q4_K), else nothing.
template <int FMT, int NT, bool XM>
__device__ __forceinline__ void sb_xmin(const half8_t (&bx)[8][NT], float* xl, XMin<NT, XM>& xm) {
    if constexpr (FMT == 4 && XM) q4_xmin<NT>(bx, xl, xm);
}

// Raw bytes -> operands for either format.
template <int FMT> struct SbRaw;
template <> struct SbRaw<4> { using Raw = Q4Raw; using Ops = Q4Ops; };
template <> struct SbRaw<6> { using Raw = Q6Raw; using Ops = Q6Ops; };
__device__ __forceinline__ void sb_load(const uint8_t* blk, int grp, Q4Raw& r) { q4_raw_load(blk, grp, r); }
__device__ __forceinline__ void sb_load(const uint8_t* blk, int grp, Q6Raw& r) { q6_raw_load(blk, grp, r); }
template <bool XM>
__device__ __forceinline__ void sb_ops(const Q4Raw& r, int grp, Q4Ops& o) { q4_exact_operands<XM>(r, grp, o); }
template <bool XM>
__device__ __forceinline__ void sb_ops(const Q6Raw& r, int grp, Q6Ops& o) { q6_exact_operands(r, grp, o); }

// C tile element of weight row rw (0..15) and batch column cc (0..15): lane
// rw + 16 * (cc / 4), register cc % 4.
__device__ __forceinline__ int c_lane(int rw, int cc) { return rw + 16 * (cc >> 2); }
__device__ __forceinline__ int c_reg(int cc) { return cc & 3; }

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
