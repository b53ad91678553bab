// Persistent decode step for one sequence (batch 1), gfx950.
//
// The whole 28-layer step (vte/compiler/qwen_compute.py:100-282, captured node
// by node by vte/core/hip_graph_executor.py:504-738) runs as ONE launch of one
// 256-thread block per CU.  Per layer the blocks pass through six stages:
//
//   S1  RMSNorm + q/k/v mat-vec + bias + RoPE + K/V append     (row tiles)
//   S2  split-KV attention partials over the cached rows        (KV head, split)
//   S3  log-sum-exp combine + the new token's own row           (query head)
//   S4  o-proj mat-vec + residual                               (row tiles)
//   S5  RMSNorm + gate/up mat-vec + SwiGLU                      (row-pair tiles)
//   S6  down mat-vec + residual                                 (row tiles)
//
// then RMSNorm + LM head.  A stage needs the whole output of the one before
// it, which in a graph costs a kernel boundary (~2 us on this part) plus the
// next kernel's activation fetch before its weights are even requested.  Here
// every value handed from one block to another is stored as a flagged word
// (fp16 | tag << 16, or fp32 | tag << 32 for the attention partials) with
// device-coherent stores, and the consumer polls the words themselves with
// device-coherent loads until every flag carries the current tag: one memory
// round trip, no counters, no fences, no L2 writeback.  Before it waits, a
// block has already requested its weight tile of the stage (weights do not
// depend on the activations), so the weight stream overlaps the handoff.
//
// Tags: a device-resident epoch, incremented by the last block to finish,
// makes tag = (epoch << 5 | layer) unique per launch and layer, so the
// flagged buffers are reused across layers and launches without clearing.
// A word of a previous layer or launch never carries the current tag.
// Reuse is safe because every stage waits on all of its predecessor's output,
// so by the time any block writes a buffer again, every reader of its previous
// contents has finished (the chain of full dependencies in between).
//
// All blocks must be resident at once (grid = CU count, one block per CU;
// the host checks the occupancy).  Every wait is bounded: past a deadline a
// block records an error flag and proceeds, so the kernel always drains.
//
// Arithmetic is the fused mat-vec's (fused_kernels.h: same unit dot products,
// same row sums, same RMSNorm and epilogue rounding points), so every
// projection gives the same bits as the graph path; attention splits differ
// (the new token is folded in by the combine) and agree to fp32 rounding.
#include <cstdio>

#include "fused_kernels.h"
#include "attn_tile.h"
#include "decode_persistent.h"

namespace {

constexpr int PD_MS = VTE_DECODE_MAX_SPLITS;  // attention splits per KV head
constexpr int PD_PW = ATT_D + 2;              // words of one (head, split) record: m, l, o[128]
constexpr int PD_T = ROWS_THREADS;            // threads per block

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

// ------------------------------------------------------------- activation staging
// The K activations of a stage into LDS in the fused mat-vec layout (padded
// xperm order + per-16 sums), RMS-normalised when norm_w is set, with the
// arithmetic of fmv_prologue (same chunk-to-thread map, so the same sums).
// src: flagged words (ll) or a plain fp16 vector.  Ends with a barrier.
template <int NJ>
__device__ __forceinline__ void pd_stage_x_nj(const void* src, bool ll, uint32_t tag, const __half* norm_w, float eps, int K,
                              const FmvLDS& L, float* red, const PdClock& ck) {
    const int nch = K / 8, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ldx = xpad_len(K);
    uint32_t h[NJ][4];
    if (ll) {
        pd_wait_chunks<NJ>(reinterpret_cast<const uint32_t*>(src), tag, nch, h, ck);
    } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = tid + PD_T * j;
            const uint4 v = c < nch ? reinterpret_cast<const uint4*>(src)[c] : make_uint4(0, 0, 0, 0);
            h[j][0] = v.x; h[j][1] = v.y; h[j][2] = v.z; h[j][3] = v.w;
        }
    }
    if (norm_w != nullptr) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) ss += chunk_sumsq(h[j]);
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float inv = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
        const uint4* nv = reinterpret_cast<const uint4*>(norm_w);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = tid + PD_T * j;
            chunk_norm(h[j], nv[c < nch ? c : 0], inv);
        }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = tid + PD_T * j;
        float s = chunk_sum(h[j]);
        s += lane_pair(s);
        if (c < nch) {
            uint32_t h0 = h[j][0], h1 = h[j][1], h2 = h[j][2], h3 = h[j][3];
            xperm_words(h0, h1);
            xperm_words(h2, h3);
            *reinterpret_cast<uint4*>(L.xs + xpad(8 * c)) = make_uint4(h0, h1, h2, h3);
            if ((c & 1) == 0) L.s16[c >> 1] = s;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void pd_stage_x(const void* src, bool ll, uint32_t tag, const __half* norm_w, float eps,
                                           int K, const FmvLDS& L, float* red, const PdClock& ck) {
    const int nch = K / 8;
    if (nch <= PD_T) pd_stage_x_nj<1>(src, ll, tag, norm_w, eps, K, L, red, ck);
    else if (nch <= 2 * PD_T) pd_stage_x_nj<2>(src, ll, tag, norm_w, eps, K, L, red, ck);
    else pd_stage_x_nj<5>(src, ll, tag, norm_w, eps, K, L, red, ck);  // K <= 10240 (checked on the host)
}

// ------------------------------------------------------------------ mat-vec stages
struct PdStage {
    FmvSeg seg[3];
    int nseg, total, K;
};

__device__ __forceinline__ TileGeo pd_geo(const PdStage& S, int g) {
    TileGeo T;
    const int t0 = S.seg[0].tiles, t1 = S.seg[1].tiles;
    if (S.nseg == 1 || g < t0) geo_from_seg(S.seg[0], g, T);
    else if (S.nseg == 2 || g < t0 + t1) geo_from_seg(S.seg[1], g - t0, T);
    else geo_from_seg(S.seg[2], g - t0 - t1, T);
    return T;
}

__device__ __forceinline__ int pd_block_bytes(int fmt) { return fmt == 4 ? Q4K_BYTES : Q6K_BYTES; }

__device__ __forceinline__ FmvSeg pd_seg(const uint8_t* w, const uint8_t* w2, const void* bias, int fmt, int n_rows,
                                         int R, int mode, int K) {
    FmvSeg s;
    s.w = w;
    s.w2 = w2;
    s.out = nullptr;
    s.bias = bias;
    s.residual = nullptr;
    s.fmt = fmt;
    s.n_rows = n_rows;
    s.R = R;
    s.mode = mode;
    // SwiGLU tiles: R / 2 gate rows (n_rows counts gate rows); RoPE tiles: R
    // rows of the n_rows (R / 2 rotation pairs); plain tiles: R rows
    const int per_tile = mode == FMV_SWIGLU ? R / 2 : R;
    s.tiles = (n_rows + per_tile - 1) / per_tile;
    s.row_bytes = (K / QK_K) * pd_block_bytes(fmt);
    return s;
}

template <int UPT, bool RO>
__device__ __forceinline__ void pd_issue(TileW<UPT>& W, const TileGeo& T, int K) {
    const int n_sb = K / QK_K, per_row = n_sb * 4;
    if (T.fmt == 4) tile_w_issue<UPT, 4, RO>(W, T, n_sb, per_row, threadIdx.x);
    else tile_w_issue<UPT, 6, RO>(W, T, n_sb, per_row, threadIdx.x);
}

template <int UPT, bool RO>
__device__ __forceinline__ void pd_dot(const TileW<UPT>& W, const TileGeo& T, int K, const FmvLDS& L) {
    const int per_row = (K / QK_K) * 4;
    if (T.fmt == 4) tile_dot<1, UPT, 4, RO>(W, T.nr, per_row, K, L.xs, L.s16, L.part, UPT * PD_T, threadIdx.x);
    else tile_dot<1, UPT, 6, RO>(W, T.nr, per_row, K, L.xs, L.s16, L.part, UPT * PD_T, threadIdx.x);
}

// Where a stage's outputs go.
struct PdOut {
    uint32_t tag;
    uint32_t* ll;             // flagged output words (q, attention-free stores)
    uint32_t* ll_kv;          // flagged new K (rows 0..kv_dim) and V (kv_dim..) of this token
    const void* res;          // residual: flagged words (res_ll) or plain fp16
    bool res_ll;
    uint32_t res_tag;
    __half* k_cache;          // this layer's cache row `pos`
    __half* v_cache;
    int kv_dim;
    int pos;
    const __half* cosp;       // RoPE tables at row `pos`
    const __half* sinp;
    float* logits;
};

// One output per thread, as tile_epilogue (batch 1) with flagged stores.
__device__ __forceinline__ void pd_epilogue(const TileGeo& T, const float* part, int per_row, const PdOut& o,
                                            const PdClock& ck) {
    const bool paired = fmv_paired(T.mode);
    const int t = threadIdx.x;
    if (t >= (paired ? T.hA : T.nr)) return;
    const int row1 = T.j0 + t;
    if (!paired) {
        const uint32_t b1 = T.bias != nullptr ? ldg_b16(T.bias, row1) : 0u;
        float v = row_sum(part + t * per_row, per_row);
        if (T.mode == FMV_STORE_F32) {
            o.logits[row1] = (v + 0.f) * 1.f + 0.f;
            return;
        }
        v += h2f_bits(b1);
        if (T.mode == FMV_VCACHE) {
            const uint32_t hb = f16_bits(v);
            reinterpret_cast<uint16_t*>(o.v_cache)[(size_t)o.pos * o.kv_dim + row1] = (uint16_t)hb;
            st_c32(o.ll_kv + o.kv_dim + row1, ll16(hb, o.tag));
            return;
        }
        // FMV_STORE_F16: fp16((acc + bias) * 1 + residual[row])
        const uint32_t rb = o.res_ll ? pd_wait16(reinterpret_cast<const uint32_t*>(o.res) + row1, o.res_tag, ck)
                                     : (uint32_t)reinterpret_cast<const uint16_t*>(o.res)[row1];
        v = v * 1.f + h2f_bits(rb);
        st_c32(o.ll + row1, ll16(f16_bits(v), o.tag));
        return;
    }
    const float a = row_sum(part + t * per_row, per_row);
    const float bv = row_sum(part + (t + T.hA) * per_row, per_row);
    if (T.mode == FMV_SWIGLU) {
        const float gg = __half2float(__float2half(a));
        const float uu = __half2float(__float2half(bv));
        const float sig = 1.0f / (1.0f + expf(-gg));
        st_c32(o.ll + row1, ll16(f16_bits(gg * sig * uu), o.tag));
        return;
    }
    const uint32_t b1 = T.bias != nullptr ? ldg_b16(T.bias, row1) : 0u;
    const uint32_t b2 = T.bias != nullptr ? ldg_b16(T.bias, row1 + 64) : 0u;
    const float x1 = __half2float(__float2half(a + h2f_bits(b1)));
    const float x2 = __half2float(__float2half(bv + h2f_bits(b2)));
    const int d = row1 & 127;
    const float c = __half2float(o.cosp[d]), sn = __half2float(o.sinp[d]);
    const uint32_t o1 = f16_bits(x1 * c - x2 * sn), o2 = f16_bits(x1 * sn + x2 * c);
    if (T.mode == FMV_ROPE_Q) {
        st_c32(o.ll + row1, ll16(o1, o.tag));
        st_c32(o.ll + row1 + 64, ll16(o2, o.tag));
    } else {  // FMV_ROPE_KCACHE
        uint16_t* kc = reinterpret_cast<uint16_t*>(o.k_cache) + (size_t)o.pos * o.kv_dim + (row1 - d);
        kc[d] = (uint16_t)o1;
        kc[d + 64] = (uint16_t)o2;
        st_c32(o.ll_kv + row1, ll16(o1, o.tag));
        st_c32(o.ll_kv + row1 + 64, ll16(o2, o.tag));
    }
}

// A mat-vec stage: this block's tiles g = blockIdx.x + i * gridDim.x.  The
// first tile's weights (W, T) were requested by pd_begin before the caller
// waited on anything; PF: the next tile's weights are requested before the
// current tile's dot products (stages of several tiles per block).
template <int UPT, bool RO>
__device__ __forceinline__ void pd_begin(const PdStage& S, TileW<UPT>& W, TileGeo& T) {
    if ((int)blockIdx.x < S.total) {
        T = pd_geo(S, blockIdx.x);
        pd_issue<UPT, RO>(W, T, S.K);
    }
}

template <int UPT, bool RO, bool PF>
__device__ __forceinline__ void pd_run(const PdStage& S, TileW<UPT>& W, TileGeo& T, const void* src, bool ll, uint32_t in_tag,
                       const __half* norm_w, float eps, uint8_t* lds, float* red, const PdOut& o, const PdClock& ck) {
    if ((int)blockIdx.x >= S.total) return;
    const int K = S.K, per_row = (K / QK_K) * 4;
    const FmvLDS L = fmv_lds(lds, 1, K, UPT);
    pd_stage_x(src, ll, in_tag, norm_w, eps, K, L, red, ck);
    for (int g = blockIdx.x; g < S.total; g += gridDim.x) {
        const int gn = g + gridDim.x;
        TileW<UPT> Wn;
        TileGeo Tn;
        if (PF && gn < S.total) {
            Tn = pd_geo(S, gn);
            pd_issue<UPT, RO>(Wn, Tn, K);
        }
        pd_dot<UPT, RO>(W, T, K, L);
        __syncthreads();
        pd_epilogue(T, L.part, per_row, o, ck);
        __syncthreads();
        if (gn < S.total) {
            if (PF) {
                W = Wn;
                T = Tn;
            } else {
                T = pd_geo(S, gn);
                pd_issue<UPT, RO>(W, T, K);
            }
        }
    }
}

// One mat-vec stage as its own (non-inlined) function: the weight registers
// live in its frame only, so the kernel's other stages do not share their
// register budget with them.  The first tile's weights are requested before
// the input is waited for.
template <int UPT, bool RO, bool PF>
__device__ __forceinline__ void pd_mv(const PdStage& S, const void* src, bool ll, uint32_t in_tag, const __half* norm_w,
                                   float eps, uint8_t* lds, float* red, const PdOut& o, const PdClock& ck) {
    TileW<UPT> W;
    TileGeo T;
    pd_begin<UPT, RO>(S, W, T);
    pd_run<UPT, RO, PF>(S, W, T, src, ll, in_tag, norm_w, eps, lds, red, o, ck);
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
};

// S2: partials of split c (rows [c*split, min((c+1)*split, pos))) of KV head kvh.
__device__ __forceinline__ void pd_attn_item(const VtePdPlan& P, const VtePdLayer& Ly, int kvh, int c, int split, int pos,
                             uint32_t tag, uint32_t tag32, PdAttLDS& A, const PdClock& ck) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;
    const int G = P.n_q / P.n_kv;
    const int t_begin = c * split, t_end = min(t_begin + split, pos);
    const size_t row_stride = (size_t)P.n_kv * ATT_D;
    const __half* kb = reinterpret_cast<const __half*>(Ly.k_cache) + (size_t)kvh * ATT_D;
    const __half* vb = reinterpret_cast<const __half*>(Ly.v_cache) + (size_t)kvh * ATT_D;
    AttTile T;
    int t0 = t_begin + wv * ATT_TILE;
    att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);  // cached rows: written by earlier launches

    // Q^T of the group's heads (B operand, heads past G zero) from the flagged q words
    half8_t qb[ATT_D / 32];
    {
        const bool slot = col < G;
        const uint32_t* qp = P.ll_q + (size_t)(kvh * G + (slot ? col : 0)) * ATT_D + 8 * grp;
        uint64_t w[ATT_D / 32][4];
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[s][i] = slot ? ld_c64(reinterpret_cast<const uint64_t*>(qp + 32 * s) + i)
                               : ((uint64_t)tag << 48 | (uint64_t)tag << 16);
        int spins = 0;
        while (true) {
            bool all = true;
#pragma unroll
            for (int s = 0; s < ATT_D / 32; ++s)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool ok = ok2(w[s][i], tag);
                    all = all && ok;
                    if (!ok) w[s][i] = ld_c64(reinterpret_cast<const uint64_t*>(qp + 32 * s) + i);
                }
            if (all || pd_expired(ck, spins)) break;
        }
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s) {
            const uint4 u = make_uint4(pair2(w[s][0]), pair2(w[s][1]), pair2(w[s][2]), pair2(w[s][3]));
            qb[s] = slot ? __builtin_bit_cast(half8_t, u) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    float m_run = -1e30f, l_run = 0.f;
    floatx4_t o_acc[ATT_D / 16];
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt) o_acc[dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    if (t0 < t_end)
        att_tile_step<true>(T, t0, t_end, qb, P.scale, m_run, l_run, o_acc, A.u.vt[wv], lane, col, grp, t_end);
    for (t0 += ATT_WAVES * ATT_TILE; t0 < t_end; t0 += ATT_WAVES * ATT_TILE) {
        att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);
        att_tile_step<false>(T, t0, t_end, qb, P.scale, m_run, l_run, o_acc, A.u.vt[wv], lane, col, grp, t_end);
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
        uint64_t* rec = P.part + ((size_t)(kvh * G + h) * PD_MS + c) * PD_PW;
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
__device__ __forceinline__ void pd_attn_combine(const VtePdPlan& P, int qh, int ns, uint32_t tag, uint32_t tag32, PdAttLDS& A,
                                const PdClock& ck) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int G = P.n_q / P.n_kv, kvh = qh / G, kv_dim = P.n_kv * ATT_D;
    const uint64_t* recs = P.part + (size_t)qh * PD_MS * PD_PW;
    float vnew = 0.f;
    if (tid < ns) {
        A.u.c.wm[tid] = pd_wait32(recs + (size_t)tid * PD_PW, tag32, ck);
        A.u.c.wl[tid] = pd_wait32(recs + (size_t)tid * PD_PW + 1, tag32, ck);
    }
    if (tid >= 128) {  // waves 2-3: q . k_new
        const int d = tid - 128;
        const float qv = h2f_bits(pd_wait16(P.ll_q + (size_t)qh * ATT_D + d, tag, ck));
        const float kv = h2f_bits(pd_wait16(P.ll_kv + (size_t)kvh * ATT_D + d, tag, ck));
        const float s = wave_sum(qv * kv);
        if (lane == 0) A.sc[wv - 2] = s;
    } else {
        vnew = h2f_bits(pd_wait16(P.ll_kv + kv_dim + (size_t)kvh * ATT_D + tid, tag, ck));
    }
    __syncthreads();
    if (wv == 0) {  // maximum, split weights exp(m_c - M) and the denominator
        const float snew = (A.sc[0] + A.sc[1]) * P.scale;
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
    // O[d] = sum_c w_c o_c[d] + e_new v_new[d]: threads (d, half) take every other split
    const int d = tid & 127, hf = tid >> 7;
    float O = 0.f;
    int c = hf;
    for (; c + 14 < ns; c += 16) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = pd_wait32(recs + (size_t)(c + 2 * j) * PD_PW + 2 + d, tag32, ck);
#pragma unroll
        for (int j = 0; j < 8; ++j) O = fmaf(v[j], A.u.c.wm[c + 2 * j], O);
    }
    for (; c < ns; c += 2) O = fmaf(pd_wait32(recs + (size_t)c * PD_PW + 2 + d, tag32, ck), A.u.c.wm[c], O);
    if (hf) A.u.c.oh[d] = O;
    __syncthreads();
    if (!hf) {
        O = O + A.u.c.oh[d];
        O = fmaf(A.sc[2], vnew, O);
        st_c32(P.ll_att + (size_t)qh * ATT_D + d, ll16(f16_bits(O / fmaxf(A.sc[3], 1e-20f)), tag));
    }
    __syncthreads();
}

// ------------------------------------------------------------------ the kernel
constexpr int UPT_QKV = 1, UPT_O = 1, UPT_GU = 4, UPT_D = 4, UPT_LM = 4;

template <bool RO_H, bool RO_F>
__global__ __launch_bounds__(PD_T, 1) void decode_persistent_kernel(VtePdPlan P) {
    extern __shared__ uint4 pd_smem[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(pd_smem);
    __shared__ PdAttLDS A;
    __shared__ float red[4];
    const uint32_t epoch = ld_c32(P.ctrl);
    const int pos = P.kv_offset[0];
    const PdClock ck{pd_now() + P.timeout_ticks, P.ctrl + 2};
    const int H = P.hidden, F = P.ffn, qd = P.n_q * ATT_D, kvd = P.n_kv * ATT_D;
    const int G = gridDim.x, b = blockIdx.x;
    // attention geometry: ns splits of the pos cached rows, at most PD_MS per KV head
    const int split = max(P.split_min, ((pos + PD_MS - 1) / PD_MS + ATT_TILE - 1) / ATT_TILE * ATT_TILE);
    const int ns = (pos + split - 1) / split;
    const __half* cosp = P.rope_cos + (size_t)pos * ATT_D;
    const __half* sinp = P.rope_sin + (size_t)pos * ATT_D;

    for (int l = 0; l < P.n_layers; ++l) {
        const VtePdLayer& Ly = P.layers[l];
        const uint32_t tag32 = (epoch << 5) | (uint32_t)l, tag = tag32 & 0xFFFFu;
        const uint32_t ptag = ((epoch << 5) | (uint32_t)(l - 1)) & 0xFFFFu;  // the previous layer's
        const bool first = l == 0;
        const void* hin = first ? (const void*)P.x : (const void*)P.ll_h;
        PdOut o{};
        o.pos = pos;
        o.kv_dim = kvd;
        o.cosp = cosp;
        o.sinp = sinp;
        o.k_cache = reinterpret_cast<__half*>(Ly.k_cache);
        o.v_cache = reinterpret_cast<__half*>(Ly.v_cache);
        o.ll_kv = P.ll_kv;
        o.tag = tag;

        // ---- S1: norm + q/k/v + bias + RoPE + K/V append ----
        {
            PdStage S;
            S.K = H;
            S.nseg = 3;
            S.seg[0] = pd_seg((const uint8_t*)Ly.wq, nullptr, Ly.q_bias, Ly.fmt_q, qd, P.r_qk, FMV_ROPE_Q, H);
            S.seg[1] = pd_seg((const uint8_t*)Ly.wk, nullptr, Ly.k_bias, Ly.fmt_k, kvd, P.r_qk, FMV_ROPE_KCACHE, H);
            S.seg[2] = pd_seg((const uint8_t*)Ly.wv, nullptr, Ly.v_bias, Ly.fmt_v, kvd, P.r_v, FMV_VCACHE, H);
            S.total = S.seg[0].tiles + S.seg[1].tiles + S.seg[2].tiles;
            o.ll = P.ll_q;
            pd_mv<UPT_QKV, RO_H, false>(S, hin, !first, ptag, (const __half*)Ly.attn_norm, P.eps, lds, red, o,
                                         ck);
        }
        PdStage So;
        So.K = qd;
        So.nseg = 1;
        So.seg[0] = pd_seg((const uint8_t*)Ly.wo, nullptr, nullptr, Ly.fmt_o, H, P.r_o, FMV_STORE_F16, qd);
        So.total = So.seg[0].tiles;

        // ---- S2: split-KV partials (blocks 0 .. n_kv*ns-1) ----
        for (int it = b; it < P.n_kv * ns; it += G) pd_attn_item(P, Ly, it / ns, it % ns, split, pos, tag, tag32, A, ck);
        // ---- S3: combine per query head (the last n_q blocks) ----
        for (int qh = G - 1 - b; qh >= 0 && qh < P.n_q; qh += G) pd_attn_combine(P, qh, ns, tag, tag32, A, ck);

        // ---- S4: o-proj + residual ----
        o.ll = P.ll_hm;
        o.res = hin;
        o.res_ll = !first;
        o.res_tag = ptag;
        pd_mv<UPT_O, RO_H, false>(So, P.ll_att, true, tag, nullptr, P.eps, lds, red, o, ck);

        // ---- S5: norm + gate/up + SwiGLU ----
        {
            PdStage S;
            S.K = H;
            S.nseg = 1;
            S.seg[0] = pd_seg((const uint8_t*)Ly.w_gate, (const uint8_t*)Ly.w_up, nullptr, Ly.fmt_gate_up, F, P.r_gu,
                              FMV_SWIGLU, H);
            S.total = S.seg[0].tiles;
            o.ll = P.ll_act;
            pd_mv<UPT_GU, RO_H, true>(S, P.ll_hm, true, tag, (const __half*)Ly.ffn_norm, P.eps, lds, red, o,
                                        ck);
        }
        // ---- S6: down + residual ----
        {
            PdStage S;
            S.K = F;
            S.nseg = 1;
            S.seg[0] = pd_seg((const uint8_t*)Ly.w_down, nullptr, nullptr, Ly.fmt_down, H, P.r_d, FMV_STORE_F16, F);
            S.total = S.seg[0].tiles;
            o.ll = P.ll_h;
            o.res = P.ll_hm;
            o.res_ll = true;
            o.res_tag = tag;
            pd_mv<UPT_D, RO_F, false>(S, P.ll_act, true, tag, nullptr, P.eps, lds, red, o, ck);
        }
    }
    // ---- output norm + LM head -> fp32 logits ----
    {
        const uint32_t ltag = ((epoch << 5) | (uint32_t)(P.n_layers - 1)) & 0xFFFFu;
        PdStage S;
        S.K = H;
        S.nseg = 1;
        S.seg[0] = pd_seg((const uint8_t*)P.lm_head, nullptr, nullptr, P.fmt_lm, P.vocab, P.r_lm, FMV_STORE_F32, H);
        S.total = S.seg[0].tiles;
        PdOut o{};
        o.logits = P.logits;
        pd_mv<UPT_LM, RO_H, true>(S, P.ll_h, true, ltag, (const __half*)P.output_norm, P.eps, lds, red, o, ck);
    }
    // ---- the last block to finish advances the epoch (read by every block at its start) ----
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(P.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)G - 1) {
            st_c32(P.ctrl + 1, 0u);
            st_c32(P.ctrl, epoch + 1u);
        }
    }
}

}  // namespace

namespace vte {

size_t decode_persistent_lds(int hidden, int ffn, int q_dim) {
    const int K = std::max(std::max(hidden, ffn), q_dim);
    size_t o = ((size_t)xpad_len(K) * 2 + 15) & ~(size_t)15;
    o += (size_t)(K / 16) * 4;
    o = (o + 15) & ~(size_t)15;
    return o + (size_t)UPT_GU * ROWS_THREADS * 4;
}

hipError_t decode_persistent_launch(const VtePdPlan& P, int blocks, size_t lds, hipStream_t st) {
    const bool ro_h = fmv_ro(P.hidden) && fmv_ro(P.n_q * ATT_D);
    const bool ro_f = fmv_ro(P.ffn);
    if (fmv_ro(P.hidden) != fmv_ro(P.n_q * ATT_D)) return hipErrorNotSupported;
    if (ro_h && ro_f) hipLaunchKernelGGL((decode_persistent_kernel<true, true>), dim3(blocks), dim3(PD_T), lds, st, P);
    else if (ro_h) hipLaunchKernelGGL((decode_persistent_kernel<true, false>), dim3(blocks), dim3(PD_T), lds, st, P);
    else if (ro_f) hipLaunchKernelGGL((decode_persistent_kernel<false, true>), dim3(blocks), dim3(PD_T), lds, st, P);
    else hipLaunchKernelGGL((decode_persistent_kernel<false, false>), dim3(blocks), dim3(PD_T), lds, st, P);
    return hipGetLastError();
}

int decode_persistent_occupancy(const VtePdPlan& P, size_t lds) {
    const bool ro_h = fmv_ro(P.hidden), ro_f = fmv_ro(P.ffn);
    int n = 0;
    hipError_t e;
    if (ro_h && ro_f) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<true, true>, PD_T, lds);
    else if (ro_h) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<true, false>, PD_T, lds);
    else if (ro_f) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<false, true>, PD_T, lds);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<false, false>, PD_T, lds);
    return e == hipSuccess ? n : -1;
}

}  // namespace vte
