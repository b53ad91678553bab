// Split-KV attention building blocks shared by the attention kernels and the
// persistent decode-step kernel (gfx950, wave64): one wave's 32-token K/V
// tile, the MFMA score / online-softmax / P.V step over it, and
// device-coherent float accesses.  Algorithm: online softmax per chunk as in
// vte/compiler/templates/rdna/flash_attention_split_kv_partial.hip.template:31-120.
#pragma once
#include "vte_common.h"
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

#define ATT_D 128
#define ATT_WAVES 4
#define ATT_TILE 32  // tokens per wave step (two 16-token MFMA tiles)
#define ATT_MAXG 8   // query heads per KV head served by one block
#define ATT_MAX_COMBINE 512  // splits per sequence the in-kernel combine handles
#define ATT_MAX_SPLITS 4096  // splits per sequence the separate combine handles
#define ATT_REC (ATT_D + 2)  // 64-bit words of a flagged split record: m, l, o[128]
#define ATT_VT_STRIDE 36     // halves per row of the transposed V tile (32 tokens + pad)

// Device-coherent float store / load (relaxed device-scope atomics: on this
// multi-XCD part they write through / read past the XCD's L2), and a wait for
// this wave's outstanding stores to complete.
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Flagged fp32 word (value | tag << 32): one 64-bit device-coherent store or
// load, so a reader that sees the tag sees the value written with it.
__device__ __forceinline__ void st_flag32(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// The value of a flagged word once it carries `tag` (polls; gives up after
// `limit` polls and returns what it holds, so a kernel never hangs).
__device__ __forceinline__ float wait_flag32(const uint64_t* p, uint32_t tag, int limit = 1 << 18) {
    uint64_t w = __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = 0; (uint32_t)(w >> 32) != tag && i < limit; ++i)
        w = __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __uint_as_float((uint32_t)w);
}
// N flagged words p[0], p[stride], ... (slots from `n` on re-read word n - 1)
// requested together and re-polled until each carries `tag` (one round trip
// when they are already there).  Returns false when it gave up after `limit`
// polls (the values are then stale).
template <int N>
__device__ __forceinline__ bool wait_flag32_n(const uint64_t* p, size_t stride, uint32_t tag, float (&v)[N],
                                              int n = N, int limit = 1 << 18) {
    uint64_t w[N];
    const uint64_t* q[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
        q[j] = p + (size_t)min(j, n - 1) * stride;
        w[j] = __hip_atomic_load(const_cast<uint64_t*>(q[j]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    for (int i = 0; i < limit; ++i) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const bool ok = (uint32_t)(w[j] >> 32) == tag;
            all = all && ok;
            if (!ok) w[j] = __hip_atomic_load(const_cast<uint64_t*>(q[j]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (all) break;
    }
    bool done = true;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        v[j] = __uint_as_float((uint32_t)w[j]);
        done = done && (uint32_t)(w[j] >> 32) == tag;
    }
    return done;
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// One wave's 32-token tile: K rows (MFMA A operands, two 16-token halves) and
// V rows (two fp16 per lane: d = 2 lane, 2 lane + 1).  Rows past `rmax` read
// row `rmax` instead (results for them are masked).
struct AttTile {
    half8_t ka[2][ATT_D / 32];
    uint32_t vv[ATT_TILE];
};

__device__ __forceinline__ void att_load_tile(AttTile& T, const __half* kb, const __half* vb, size_t row_stride,
                                              int t0, int rmax, int col, int grp, int lane) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int tok = min(t0 + 16 * tt + col, rmax);
        const __half* kr = kb + (size_t)tok * row_stride;
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s) T.ka[tt][s] = *reinterpret_cast<const half8_t*>(kr + 32 * s + 8 * grp);
    }
#pragma unroll
    for (int t = 0; t < ATT_TILE; ++t) {
        const int tok = min(t0 + t, rmax);
        T.vv[t] = *reinterpret_cast<const uint32_t*>(vb + (size_t)tok * row_stride + 2 * lane);
    }
}

// Eight consecutive query elements as fp16 (16- or 32-byte loads).
__device__ __forceinline__ half8_t att_load_q8(const __half* p) { return *reinterpret_cast<const half8_t*>(p); }
__device__ __forceinline__ half8_t att_load_q8(const float* p) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], c = reinterpret_cast<const float4*>(p)[1];
    return half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                   (_Float16)c.x, (_Float16)c.y, (_Float16)c.z, (_Float16)c.w};
}

// One 32-token tile of a wave: scores (MFMA), online softmax, P.V (MFMA)
// into the running (m_run, l_run, o_acc).  `vt` is the wave's LDS tile for
// the transposed V.  FIRST: the wave's first tile (nothing to rescale; the
// P.V products start from zero).
template <bool FIRST>
__device__ __forceinline__ void att_tile_step(AttTile& T, int t0, int t_end, const half8_t (&qb)[ATT_D / 32],
                                              float scale, float& m_run, float& l_run,
                                              floatx4_t (&o_acc)[ATT_D / 16],
                                              uint32_t (*vt)[ATT_VT_STRIDE / 2], int lane, int col, int grp,
                                              int t_end_col) {
    // t_end: end of the tokens any query slot reads (V rows past it are
    // zeroed); t_end_col: end for this lane's query slot (scores past it -inf)
    // rows at or past the end contribute p = 0; zero their V so that
    // whatever the rows hold cannot turn 0 * V into NaN (tail tile only)
    if (t0 + ATT_TILE > t_end) {
#pragma unroll
        for (int t = 0; t < ATT_TILE; ++t) T.vv[t] = (t0 + t < t_end) ? T.vv[t] : 0u;
    }
    // ---- scores for 32 tokens: two 16x16 S^T tiles ----
    floatx4_t acc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        acc[tt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s)
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.ka[tt][s], qb[s], acc[tt], 0, 0, 0);
    }
    // ---- V^T into LDS: dword (V[t][d], V[t+1][d]) at vt[d][t/2] ----
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < ATT_TILE; t += 2) {
        vt[2 * lane][t / 2] = __builtin_amdgcn_perm(T.vv[t + 1], T.vv[t], 0x05040100u);
        vt[2 * lane + 1][t / 2] = __builtin_amdgcn_perm(T.vv[t + 1], T.vv[t], 0x07060302u);
    }
    // lane holds S^T[token = t0 + 16*tt + 4*grp + i][head = col]
    float sc[2][4];
    float tmax = -1e30f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = t0 + 16 * tt + 4 * grp + i;
            float sv = acc[tt][i] * scale;
            sv = (tok < t_end_col) ? sv : -INFINITY;
            sc[tt][i] = sv;
            tmax = fmaxf(tmax, sv);
        }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = FIRST ? tmax : fmaxf(m_run, tmax);
    const float corr = FIRST ? 0.f : __expf(m_run - m_new);
    // A operand of P.V: P[head = col][token slots (grp, j)], j < 4 -> tile 0, j >= 4 -> tile 1
    half8_t pa;
    float psum = 0.f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pv = __expf(sc[tt][i] - m_new);
            psum += pv;
            pa[4 * tt + i] = (_Float16)pv;
        }
    l_run = FIRST ? psum : l_run * corr + psum;
    m_run = m_new;
    // rescale O rows (heads 4*grp + i) by their corr, held by lanes 4*grp + i
    float cr[4];
    if (!FIRST) {
#pragma unroll
        for (int i = 0; i < 4; ++i) cr[i] = __shfl(corr, 4 * grp + i, 64);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt) {
        if (!FIRST) {
#pragma unroll
            for (int i = 0; i < 4; ++i) o_acc[dt][i] *= cr[i];
        }
        // B operand: V[token slots][d = 16*dt + col]
        const uint32_t* vr = &vt[16 * dt + col][0];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr + 2 * grp);       // tokens 4g .. 4g+3
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 8 + 2 * grp);   // tokens 16+4g ..
        const half8_t vb8 = __builtin_bit_cast(half8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
        o_acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb8, FIRST ? floatx4_t{0.f, 0.f, 0.f, 0.f} : o_acc[dt],
                                                           0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
}

