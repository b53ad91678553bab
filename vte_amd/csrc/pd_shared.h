// Pieces shared by the persistent decode-step kernels (batch 1:
// decode_persistent.hip; batches of up to 16 columns: decode_persistent_mm.hip):
// flagged words handed between blocks, bounded waits, and the split-KV
// attention items and their log-sum-exp combine for one sequence.
//
// A flagged word carries its value and the tag of the layer that wrote it
// (fp16 | tag << 16, or fp32 | tag << 32), stored with a device-coherent store
// and polled with device-coherent loads until the tag is the current one, so
// one memory round trip hands a value over: no counters, fences or L2
// writeback.
#pragma once
#include "attn_tile.h"
#include "decode_persistent.h"

namespace {

constexpr int PD_MS = VTE_DECODE_MAX_SPLITS;  // attention splits per KV head
constexpr int PD_PW = ATT_D + 2;              // words of one (head, split) record: m, l, o[128]
constexpr int PD_T = 256;                     // threads per block

// One sequence's view for the attention stages: its cache rows, its q and new
// K/V words, its attention output words and its split records.
struct PdSeqAttn {
    int n_q, n_kv;
    float scale;
    const __half* k_cache;   // [max_seq][n_kv][128] of this sequence
    const __half* v_cache;
    const uint32_t* ll_q;    // flagged q [n_q * 128]
    const uint32_t* ll_kv;   // flagged new K [n_kv * 128] then V
    uint32_t* ll_att;        // flagged attention output [n_q * 128]
    uint64_t* part;          // split records [n_q][PD_MS][PD_PW]
};

// ---------------------------------------------------------------- flagged words
__device__ __forceinline__ uint64_t pd_now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint64_t ld_c64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_c32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
__device__ __forceinline__ uint32_t ll16(uint32_t hbits, uint32_t tag) { return (hbits & 0xFFFFu) | (tag << 16); }
__device__ __forceinline__ uint64_t ll32(float v, uint32_t tag32) {
    return (uint64_t)__float_as_uint(v) | ((uint64_t)tag32 << 32);
}
// both 16-bit-payload words of a 64-bit load carry `tag`
__device__ __forceinline__ bool ok2(uint64_t w, uint32_t tag) {
    return ((uint32_t)(w >> 16) & 0xFFFFu) == tag && (uint32_t)(w >> 48) == tag;
}
// the fp16 pair of a 64-bit load of two flagged words
__device__ __forceinline__ uint32_t pair2(uint64_t w) {
    return ((uint32_t)w & 0xFFFFu) | (((uint32_t)(w >> 32) & 0xFFFFu) << 16);
}

struct PdClock {
    uint64_t deadline;
    uint32_t* err;
};
// True once the deadline has passed (checked every 16 polls); records the error.
__device__ __forceinline__ bool pd_expired(const PdClock& ck, int& spins) {
    if ((++spins & 15) != 0) return false;
    if (pd_now() < ck.deadline) return false;
    __hip_atomic_fetch_or(ck.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// One flagged fp16 word (value bits), waited for.
__device__ __forceinline__ uint32_t pd_wait16(const uint32_t* p, uint32_t tag, const PdClock& ck) {
    uint32_t w = ld_c32(p);
    int spins = 0;
    while ((w >> 16) != tag && !pd_expired(ck, spins)) w = ld_c32(p);
    return w & 0xFFFFu;
}
// One flagged fp32 word, waited for.
__device__ __forceinline__ float pd_wait32(const uint64_t* p, uint32_t tag32, const PdClock& ck) {
    uint64_t w = ld_c64(p);
    int spins = 0;
    while ((uint32_t)(w >> 32) != tag32 && !pd_expired(ck, spins)) w = ld_c64(p);
    return __uint_as_float((uint32_t)w);
}

// Chunks c = tid + 256 j (j < NJ, c < nch) of 8 flagged fp16 words each, all
// requested together and re-polled until every flag matches: h[j] = the 8
// values as 4 fp16 pairs (natural order; zero past nch).
template <int NJ>
__device__ __forceinline__ void pd_wait_chunks(const uint32_t* src, uint32_t tag, int nch, uint32_t (&h)[NJ][4],
                                               const PdClock& ck) {
    const int tid = threadIdx.x;
    uint64_t w[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = tid + PD_T * j;
        const uint64_t* p = reinterpret_cast<const uint64_t*>(src + 8 * (size_t)(c < nch ? c : 0));
#pragma unroll
        for (int i = 0; i < 4; ++i) w[j][i] = c < nch ? ld_c64(p + i) : ((uint64_t)tag << 48 | (uint64_t)tag << 16);
    }
    int spins = 0;
    while (true) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = tid + PD_T * j;
            const bool okj = ok2(w[j][0], tag) && ok2(w[j][1], tag) && ok2(w[j][2], tag) && ok2(w[j][3], tag);
            all = all && okj;
            if (!okj && c < nch) {
                const uint64_t* p = reinterpret_cast<const uint64_t*>(src + 8 * (size_t)c);
#pragma unroll
                for (int i = 0; i < 4; ++i) w[j][i] = ld_c64(p + i);
            }
        }
        if (all || pd_expired(ck, spins)) break;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const bool in = tid + PD_T * j < nch;
#pragma unroll
        for (int i = 0; i < 4; ++i) h[j][i] = in ? pair2(w[j][i]) : 0u;
    }
}

// ------------------------------------------------------------------ attention
struct PdAttLDS {
    union {
        uint32_t vt[ATT_WAVES][ATT_D][ATT_VT_STRIDE / 2];
        float o[ATT_WAVES][16][ATT_D + 4];
        struct {
            float wm[PD_MS], wl[PD_MS], oh[PD_T];
        } c;
    } u;
    float m_sh[ATT_WAVES][16], l_sh[ATT_WAVES][16];
    float sc[4];
    alignas(16) uint32_t q[ATT_MAXG * ATT_D / 2];  // the KV group's q as fp16 pairs [head][dim / 2] (S2)
};

// S2: partials of split c (rows [c*split, min((c+1)*split, pos))) of KV head kvh.
// One word of every 128-byte line of the wave's first K/V tile of split c of
// KV head kvh (cached rows, written by earlier launches): requested while the
// layer's first stage runs, so the split's tile loads hit the L2.
__device__ __forceinline__ uint2 pd_attn_touch(const PdSeqAttn& SA, int kvh, int c, int split,
                                               int pos) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t_begin = c * split, t_end = min(t_begin + split, pos);
    const int tok = min(t_begin + wv * ATT_TILE + (lane >> 1), t_end - 1);  // 32 rows, two 128-byte lines each
    const size_t off = ((size_t)tok * SA.n_kv + kvh) * ATT_D + (size_t)(lane & 1) * 64;
    return make_uint2(*reinterpret_cast<const uint32_t*>(SA.k_cache + off),
                      *reinterpret_cast<const uint32_t*>(SA.v_cache + off));
}

__device__ __forceinline__ void pd_attn_item(const PdSeqAttn& SA, int kvh, int c, int split, int pos,
                             uint32_t tag, uint32_t tag32, PdAttLDS& A, const PdClock& ck) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;
    const int G = SA.n_q / SA.n_kv;
    const int t_begin = c * split, t_end = min(t_begin + split, pos);
    const size_t row_stride = (size_t)SA.n_kv * ATT_D;
    const __half* kb = SA.k_cache + (size_t)kvh * ATT_D;
    const __half* vb = SA.v_cache + (size_t)kvh * ATT_D;
    AttTile T;
    int t0 = t_begin + wv * ATT_TILE;
    att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);  // cached rows: written by earlier launches

    // Q^T of the group's heads (B operand, heads past G zero).  The block
    // polls the group's G * 128 flagged q words together (two 64-bit pairs
    // per thread at most, G <= 8) and stages them in LDS as fp16 pairs
    // [head][dim / 2]; each wave then reads its operands from there.
    {
        const uint64_t* qg = reinterpret_cast<const uint64_t*>(SA.ll_q + (size_t)kvh * G * ATT_D);
        const int npair = G * ATT_D / 2, t = threadIdx.x;
        const bool h0 = t < npair, h1 = t + PD_T < npair;
        const uint64_t dflt = (uint64_t)tag << 48 | (uint64_t)tag << 16;
        uint64_t w0 = h0 ? ld_c64(qg + t) : dflt, w1 = h1 ? ld_c64(qg + t + PD_T) : dflt;
        int spins = 0;
        while (true) {
            const bool ok0 = ok2(w0, tag), ok1 = ok2(w1, tag);
            if ((ok0 && ok1) || pd_expired(ck, spins)) break;
            if (!ok0) w0 = ld_c64(qg + t);
            if (!ok1) w1 = ld_c64(qg + t + PD_T);
        }
        if (h0) A.q[t] = pair2(w0);
        if (h1) A.q[t + PD_T] = pair2(w1);
    }
    __syncthreads();
    half8_t qb[ATT_D / 32];
    {
        const bool slot = col < G;
        const uint32_t* qs = A.q + (size_t)(slot ? col : 0) * (ATT_D / 2) + 4 * grp;
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s) {
            const uint4 u = *reinterpret_cast<const uint4*>(qs + 16 * s);
            qb[s] = slot ? __builtin_bit_cast(half8_t, u) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    float m_run = -1e30f, l_run = 0.f;
    floatx4_t o_acc[ATT_D / 16];
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt) o_acc[dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    if (t0 < t_end)
        att_tile_step<true>(T, t0, t_end, qb, SA.scale, m_run, l_run, o_acc, A.u.vt[wv], lane, col, grp, t_end);
    for (t0 += ATT_WAVES * ATT_TILE; t0 < t_end; t0 += ATT_WAVES * ATT_TILE) {
        att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);
        att_tile_step<false>(T, t0, t_end, qb, SA.scale, m_run, l_run, o_acc, A.u.vt[wv], lane, col, grp, t_end);
    }
    // the four waves' (m, l, O) -> one record per head, flagged
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (grp == 0) {
        A.m_sh[wv][col] = m_run;
        A.l_sh[wv][col] = l_run;
    }
    __syncthreads();
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) A.u.o[wv][4 * grp + i][16 * dt + col] = o_acc[dt][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * ATT_D; idx += PD_T) {
        const int h = idx / ATT_D, d = idx % ATT_D;
        float M = -1e30f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, A.m_sh[w][h]);
        float Ls = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; ++w) {
            const float e = __expf(A.m_sh[w][h] - M);
            Ls = fmaf(A.l_sh[w][h], e, Ls);
            O = fmaf(A.u.o[w][h][d], e, O);
        }
        uint64_t* rec = SA.part + ((size_t)(kvh * G + h) * PD_MS + c) * PD_PW;
        st_c64(rec + 2 + d, ll32(O, tag32));
        if (d == 0) {
            st_c64(rec, ll32(M, tag32));
            st_c64(rec + 1, ll32(Ls, tag32));
        }
    }
    __syncthreads();  // LDS reused by the next item / stage
}

// S3: attention output of query head qh = LSE combine of its ns split records
// and the new token's row (score q . k_new, value v_new), -> flagged fp16.
// The block takes dims part * 128/np .. of the head (np blocks per head for
// long caches): threads (dim, group g) sum the splits g, g + TPD, ... and
// the groups' sums are added in group order.
__device__ __forceinline__ void pd_attn_combine(const PdSeqAttn& SA, int qh, int part, int np, int ns, uint32_t tag,
                                                uint32_t tag32, PdAttLDS& A, const PdClock& ck) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int G = SA.n_q / SA.n_kv, kvh = qh / G, kv_dim = SA.n_kv * ATT_D;
    const uint64_t* recs = SA.part + (size_t)qh * PD_MS * PD_PW;
    const int DQ = ATT_D / np, TPD = PD_T / DQ;
    const int dd = tid % DQ, g = tid / DQ, d = part * DQ + dd;
    // every word this thread needs is requested before any is waited for: o[d]
    // of its first 8 splits, the split's (m, l), q and k_new (waves 2-3), v_new
    uint64_t ow[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = g + TPD * j;
        ow[j] = c < ns ? ld_c64(recs + (size_t)c * PD_PW + 2 + d) : ((uint64_t)tag32 << 32);
    }
    uint64_t wm = (uint64_t)tag32 << 32, wl = (uint64_t)tag32 << 32;
    if (tid < ns) {
        wm = ld_c64(recs + (size_t)tid * PD_PW);
        wl = ld_c64(recs + (size_t)tid * PD_PW + 1);
    }
    const int dq = tid & 127;
    const uint32_t* pq = SA.ll_q + (size_t)qh * ATT_D + dq;
    const uint32_t* pk = SA.ll_kv + (size_t)kvh * ATT_D + dq;
    const uint32_t* pv = SA.ll_kv + kv_dim + (size_t)kvh * ATT_D + d;
    uint32_t wq = tid >= 128 ? ld_c32(pq) : (tag << 16), wk = tid >= 128 ? ld_c32(pk) : (tag << 16);
    uint32_t wvn = tid < DQ ? ld_c32(pv) : (tag << 16);
    {  // one poll loop over all of them: a single round trip once the last record lands
        int spins = 0;
        while (true) {
            bool ok = (wq >> 16) == tag && (wk >> 16) == tag && (wvn >> 16) == tag &&
                      (uint32_t)(wm >> 32) == tag32 && (uint32_t)(wl >> 32) == tag32;
#pragma unroll
            for (int j = 0; j < 8; ++j) ok = ok && (uint32_t)(ow[j] >> 32) == tag32;
            if (ok || pd_expired(ck, spins)) break;
            if ((uint32_t)(wm >> 32) != tag32) wm = ld_c64(recs + (size_t)tid * PD_PW);
            if ((uint32_t)(wl >> 32) != tag32) wl = ld_c64(recs + (size_t)tid * PD_PW + 1);
            if ((wq >> 16) != tag) wq = ld_c32(pq);
            if ((wk >> 16) != tag) wk = ld_c32(pk);
            if ((wvn >> 16) != tag) wvn = ld_c32(pv);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if ((uint32_t)(ow[j] >> 32) != tag32) ow[j] = ld_c64(recs + (size_t)(g + TPD * j) * PD_PW + 2 + d);
        }
    }
    if (tid < ns) {
        A.u.c.wm[tid] = __uint_as_float((uint32_t)wm);
        A.u.c.wl[tid] = __uint_as_float((uint32_t)wl);
    }
    if (tid >= 128) {  // waves 2-3: q . k_new
        const float s = wave_sum(h2f_bits(wq & 0xFFFFu) * h2f_bits(wk & 0xFFFFu));
        if (lane == 0) A.sc[wv - 2] = s;
    }
    const float vnew = h2f_bits(wvn & 0xFFFFu);
    __syncthreads();
    if (wv == 0) {  // maximum, split weights exp(m_c - M) and the denominator
        const float snew = (A.sc[0] + A.sc[1]) * SA.scale;
        float M = snew;
        for (int c = lane; c < ns; c += 64) M = fmaxf(M, A.u.c.wm[c]);
        M = wave_max(M);
        float Ls = 0.f;
        for (int c = lane; c < ns; c += 64) {
            const float e = __expf(A.u.c.wm[c] - M);
            A.u.c.wm[c] = e;
            Ls = fmaf(A.u.c.wl[c], e, Ls);
        }
        Ls = wave_sum(Ls);
        const float enew = __expf(snew - M);
        if (lane == 0) {
            A.sc[2] = enew;
            A.sc[3] = Ls + enew;
        }
    }
    __syncthreads();
    // O[d] = sum_c w_c o_c[d] + e_new v_new[d]
    float O = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = g + TPD * j;
        if (c < ns) O = fmaf(__uint_as_float((uint32_t)ow[j]), A.u.c.wm[c], O);
    }
    // further splits (long caches) in batches of 16 per thread: all 16 words
    // requested at once and re-polled together, one round trip per batch
    for (int c = g + 8 * TPD; c < ns; c += 16 * TPD) {
        uint64_t w[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int cj = c + TPD * j;
            w[j] = cj < ns ? ld_c64(recs + (size_t)cj * PD_PW + 2 + d) : ((uint64_t)tag32 << 32);
        }
        int spins = 0;
        while (true) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < 16; ++j) ok = ok && (uint32_t)(w[j] >> 32) == tag32;
            if (ok || pd_expired(ck, spins)) break;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if ((uint32_t)(w[j] >> 32) != tag32) w[j] = ld_c64(recs + (size_t)(c + TPD * j) * PD_PW + 2 + d);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (c + TPD * j < ns) O = fmaf(__uint_as_float((uint32_t)w[j]), A.u.c.wm[c + TPD * j], O);
    }
    A.u.c.oh[tid] = O;
    __syncthreads();
    if (tid < DQ) {
        float S = 0.f;
        for (int k = 0; k < TPD; ++k) S += A.u.c.oh[k * DQ + tid];
        S = fmaf(A.sc[2], vnew, S);
        st_c32(SA.ll_att + (size_t)qh * ATT_D + d, ll16(f16_bits(S / fmaxf(A.sc[3], 1e-20f)), tag));
    }
    __syncthreads();
}

}  // namespace
