// Persistent decode step for one sequence (batch 1), gfx950.
//
// The whole 28-layer step (vte/compiler/qwen_compute.py:100-282, captured node
// by node by vte/core/hip_graph_executor.py:504-738) runs as ONE launch of one
// 256-thread block per CU.  Per layer the blocks pass through seven stages:
//
//   S1  RMSNorm + q/k/v mat-vec + bias + RoPE + K/V append     (row tiles)
//   S2  split-KV attention partials over the cached rows        (KV head, split;
//       on the blocks after the S1 tiles)
//   S3  log-sum-exp combine + the new token's own row           (query head)
//   S4  o-proj mat-vec + residual                               (row tiles)
//   S5  RMSNorm + gate/up mat-vec + SwiGLU                      (row-pair tiles)
//   S6a down partial sums over one 256-wide slice of the        (slice, row tiles)
//       SwiGLU output each
//   S7  sum of the partials + residual                          (row ranges)
//
// The LM head follows as a separate launch (the graph path's norm + mat-vec
// kernel) over the last layer's output.  Most stages need the whole output of
// the one before them, which in a graph costs a kernel boundary (~2 us on this part) plus the
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
// makes tag = epoch * n_layers + layer consecutive over the layers of
// successive launches, so the flagged buffers are reused across layers and
// launches without clearing: a word not yet written in this layer still
// holds the previous layer's tag, one less than the current one (also in the
// 16 bits of the fp16 words' tags).
// Reuse is safe because between a buffer's readers and its next writer there
// is always a stage that waits on all of its predecessor's output (S6a reads
// one slice, but S7 waits on every S6a tile and S1 on every S7 row), so by
// the time any block writes a buffer again, every reader of its previous
// contents has finished.
//
// All blocks must be resident at once (grid = CU count, one block per CU;
// the host checks the occupancy).  Every wait is bounded: past a deadline a
// block records an error flag and proceeds, so the kernel always drains.
//
// Arithmetic is the fused mat-vec's (fused_kernels.h: same unit dot products,
// same row sums, same RMSNorm and epilogue rounding points), so q/k/v, o-proj
// and gate/up give the same bits as the graph path on the same inputs; the
// down projection sums per 256-column slice first and the attention splits
// differ (the new token is folded in by the combine): both agree to fp32
// rounding.

#include "fused_kernels.h"
#include "attn_tile.h"
#include "decode_persistent.h"

namespace {

constexpr int PD_MS = VTE_DECODE_MAX_SPLITS;  // attention splits per KV head
constexpr int PD_PW = ATT_D + 2;              // words of one (head, split) record: m, l, o[128]
constexpr int PD_T = ROWS_THREADS;            // threads per block
constexpr int UPT_QKV = VTE_PD_UPT_QKV, UPT_O = 1, UPT_GU = VTE_PD_UPT_GU, UPT_D = 4;  // weight units per thread of each stage

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
};

// Epilogue operands of this thread's output (bias of the row and of its RoPE
// partner, cos / sin of its dimension) as raw fp16 bits, requested together
// with the tile's weights so the epilogue waits on none of them.
struct PdPre {
    uint32_t b1, b2, c, s, r;  // r: the residual word (flagged or plain fp16 bits)
};
__device__ __forceinline__ PdPre pd_pre(const TileGeo& T, const PdOut& o) {
    PdPre p{0u, 0u, 0u, 0u, 0u};
    const bool paired = fmv_paired(T.mode);
    const int t = threadIdx.x;
    if (t >= (paired ? T.hA : T.nr) || T.mode == FMV_SWIGLU) return p;
    const int row1 = T.j0 + t;
    if (T.bias != nullptr) {
        p.b1 = ldg_b16(T.bias, row1);
        if (paired) p.b2 = ldg_b16(T.bias, row1 + 64);
    }
    if (T.mode == FMV_ROPE_Q || T.mode == FMV_ROPE_KCACHE) {
        p.c = ldg_b16(o.cosp, row1 & 127);
        p.s = ldg_b16(o.sinp, row1 & 127);
    }
    if (T.mode == FMV_STORE_F16)
        p.r = o.res_ll ? ld_c32(reinterpret_cast<const uint32_t*>(o.res) + row1)
                       : (uint32_t)reinterpret_cast<const uint16_t*>(o.res)[row1];
    return p;
}

// One output per thread, as tile_epilogue (batch 1) with flagged stores.
__device__ __forceinline__ void pd_epilogue(const TileGeo& T, const float* part, int per_row, const PdOut& o,
                                            const PdPre& pre, const PdClock& ck) {
    const bool paired = fmv_paired(T.mode);
    const int t = threadIdx.x;
    if (t >= (paired ? T.hA : T.nr)) return;
    const int row1 = T.j0 + t;
    if (!paired) {
        float v = row_sum(part + t * per_row, per_row);
        v += h2f_bits(pre.b1);
        if (T.mode == FMV_VCACHE) {
            const uint32_t hb = f16_bits(v);
            reinterpret_cast<uint16_t*>(o.v_cache)[(size_t)o.pos * o.kv_dim + row1] = (uint16_t)hb;
            st_c32(o.ll_kv + o.kv_dim + row1, ll16(hb, o.tag));
            return;
        }
        // FMV_STORE_F16: fp16((acc + bias) * 1 + residual[row])
        uint32_t rb = pre.r;
        if (o.res_ll) {  // requested with the weights; re-polled only if it was not yet written
            int spins = 0;
            while ((rb >> 16) != o.res_tag && !pd_expired(ck, spins))
                rb = ld_c32(reinterpret_cast<const uint32_t*>(o.res) + row1);
            rb &= 0xFFFFu;
        }
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
    const float x1 = __half2float(__float2half(a + h2f_bits(pre.b1)));
    const float x2 = __half2float(__float2half(bv + h2f_bits(pre.b2)));
    const int d = row1 & 127;
    const float c = h2f_bits(pre.c), sn = h2f_bits(pre.s);
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
__device__ __forceinline__ void pd_begin(const PdStage& S, TileW<UPT>& W, TileGeo& T, PdPre& pre, const PdOut& o) {
    if ((int)blockIdx.x < S.total) {
        T = pd_geo(S, blockIdx.x);
        pd_issue<UPT, RO>(W, T, S.K);
        pre = pd_pre(T, o);
    }
}

template <int UPT, bool RO, bool PF>
__device__ __forceinline__ void pd_run(const PdStage& S, TileW<UPT>& W, TileGeo& T, PdPre& pre, const void* src,
                                       bool ll, uint32_t in_tag, const __half* norm_w, float eps, uint8_t* lds,
                                       float* red, const PdOut& o, const PdClock& ck) {
    if ((int)blockIdx.x >= S.total) return;
    const int K = S.K, per_row = (K / QK_K) * 4;
    const FmvLDS L = fmv_lds(lds, 1, K, UPT);
    pd_stage_x(src, ll, in_tag, norm_w, eps, K, L, red, ck);
    for (int g = blockIdx.x; g < S.total; g += gridDim.x) {
        const int gn = g + gridDim.x;
        TileW<UPT> Wn;
        TileGeo Tn;
        PdPre pn;
        if (PF && gn < S.total) {
            Tn = pd_geo(S, gn);
            pd_issue<UPT, RO>(Wn, Tn, K);
            pn = pd_pre(Tn, o);
        }
        pd_dot<UPT, RO>(W, T, K, L);
        __syncthreads();
        pd_epilogue(T, L.part, per_row, o, pre, ck);
        __syncthreads();
        if (gn < S.total) {
            if (PF) {
                W = Wn;
                T = Tn;
                pre = pn;
            } else {
                T = pd_geo(S, gn);
                pd_issue<UPT, RO>(W, T, K);
                pre = pd_pre(T, o);
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
    PdPre pre;
    pd_begin<UPT, RO>(S, W, T, pre, o);
    pd_run<UPT, RO, PF>(S, W, T, pre, src, ll, in_tag, norm_w, eps, lds, red, o, ck);
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
__device__ __forceinline__ uint2 pd_attn_touch(const VtePdPlan& P, const VtePdLayer& Ly, int kvh, int c, int split,
                                               int pos) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t_begin = c * split, t_end = min(t_begin + split, pos);
    const int tok = min(t_begin + wv * ATT_TILE + (lane >> 1), t_end - 1);  // 32 rows, two 128-byte lines each
    const size_t off = ((size_t)tok * P.n_kv + kvh) * ATT_D + (size_t)(lane & 1) * 64;
    return make_uint2(*reinterpret_cast<const uint32_t*>(reinterpret_cast<const __half*>(Ly.k_cache) + off),
                      *reinterpret_cast<const uint32_t*>(reinterpret_cast<const __half*>(Ly.v_cache) + off));
}

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

    // Q^T of the group's heads (B operand, heads past G zero).  The block
    // polls the group's G * 128 flagged q words together (two 64-bit pairs
    // per thread at most, G <= 8) and stages them in LDS as fp16 pairs
    // [head][dim / 2]; each wave then reads its operands from there.
    {
        const uint64_t* qg = reinterpret_cast<const uint64_t*>(P.ll_q + (size_t)kvh * G * ATT_D);
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
// The block takes dims part * 128/np .. of the head (np blocks per head for
// long caches): threads (dim, group g) sum the splits g, g + TPD, ... and
// the groups' sums are added in group order.
__device__ __forceinline__ void pd_attn_combine(const VtePdPlan& P, int qh, int part, int np, int ns, uint32_t tag,
                                                uint32_t tag32, PdAttLDS& A, const PdClock& ck) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int G = P.n_q / P.n_kv, kvh = qh / G, kv_dim = P.n_kv * ATT_D;
    const uint64_t* recs = P.part + (size_t)qh * PD_MS * PD_PW;
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
    const uint32_t* pq = P.ll_q + (size_t)qh * ATT_D + dq;
    const uint32_t* pk = P.ll_kv + (size_t)kvh * ATT_D + dq;
    const uint32_t* pv = P.ll_kv + kv_dim + (size_t)kvh * ATT_D + d;
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
        st_c32(P.ll_att + (size_t)qh * ATT_D + d, ll16(f16_bits(S / fmaxf(A.sc[3], 1e-20f)), tag));
    }
    __syncthreads();
}

// ------------------------------------------------------------------ down
// S6a: tile g covers rows j0 .. j0 + r_dn of w_down over the 256 columns of
// slice s = g / rt (one super-block per row), so a block waits only on the 256
// SwiGLU words of its slice (written by the few blocks whose gate/up tiles
// cover it) instead of all ffn of them.  Each row's partial sum (the same
// per-unit dot products and the row_sum order of the fused mat-vec, over 4
// units) goes out as a flagged fp32 word.
template <int FMT>
__device__ __forceinline__ void pd_down_tile(const VtePdPlan& P, const VtePdLayer& Ly, int g, int rt, uint32_t tag,
                                             uint32_t tag32, const FmvLDS& L, float* red, const PdClock& ck) {
    const int H = P.hidden, n_sb = P.ffn / QK_K;
    const int s = g / rt, rtile = g - s * rt;
    const int bpb = FMT == 4 ? Q4K_BYTES : Q6K_BYTES;
    TileGeo T;
    T.fmt = FMT;
    T.mode = FMV_STORE_F16;
    T.rb = n_sb * bpb;
    T.n_rows = H;
    T.j0 = rtile * P.r_dn;
    T.nr = min(P.r_dn, H - T.j0);
    T.hA = T.nr;
    T.bA = reinterpret_cast<const uint8_t*>(Ly.w_down) + (size_t)T.j0 * T.rb + (size_t)s * bpb;
    T.bB = T.bA;
    T.out = nullptr;
    T.bias = nullptr;
    T.residual = nullptr;
    TileW<UPT_D> W;
    tile_w_issue<UPT_D, FMT, true>(W, T, 1, 4, threadIdx.x);  // before the wait: the weights do not depend on it
    pd_stage_x_nj<1>(P.ll_act + (size_t)s * QK_K, true, tag, nullptr, 0.f, QK_K, L, red, ck);
    tile_dot<1, UPT_D, FMT, true>(W, T.nr, 4, QK_K, L.xs, L.s16, L.part, UPT_D * PD_T, threadIdx.x);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < T.nr) st_c64(P.ll_dn + (size_t)s * H + T.j0 + t, ll32(row_sum(L.part + t * 4, 4), tag32));
    __syncthreads();
}

__device__ __forceinline__ void pd_down_part(const VtePdPlan& P, const VtePdLayer& Ly, uint32_t tag, uint32_t tag32,
                                             uint8_t* lds, float* red, const PdClock& ck) {
    const int nsl = P.ffn / QK_K, rt = (P.hidden + P.r_dn - 1) / P.r_dn, total = nsl * rt;
    const FmvLDS L = fmv_lds(lds, 1, QK_K, UPT_D);
    for (int g = blockIdx.x; g < total; g += gridDim.x) {
        if (Ly.fmt_down == 4) pd_down_tile<4>(P, Ly, g, rt, tag, tag32, L, red, ck);
        else pd_down_tile<6>(P, Ly, g, rt, tag, tag32, L, red, ck);
    }
}

// S7: rows r0 .. r0 + r_red of the layer output = fp16(sum over the slices,
// in slice order, + the post-attention residual): flagged for the next
// layer, plain into h_out after the last layer.
__device__ __forceinline__ void pd_down_reduce(const VtePdPlan& P, uint32_t tag, uint32_t tag32, bool last,
                                               uint8_t* lds, const PdClock& ck) {
    const int H = P.hidden, nsl = P.ffn / QK_K;
    const int r0 = blockIdx.x * P.r_red, nrw = min(P.r_red, H - r0);
    if (nrw <= 0) return;
    float* pp = reinterpret_cast<float*>(lds);  // [nrw][nsl]
    const int t = threadIdx.x;
    uint32_t rw = t < nrw ? ld_c32(P.ll_hm + r0 + t) : 0u;  // the residual, requested before the partials
    for (int i = threadIdx.x; i < nrw * nsl; i += PD_T) {
        const int row = i / nsl, k = i - row * nsl;
        pp[i] = pd_wait32(P.ll_dn + (size_t)k * H + r0 + row, tag32, ck);
    }
    __syncthreads();
    if (t < nrw) {
        float v = 0.f;
        for (int k = 0; k < nsl; ++k) v += pp[t * nsl + k];
        int spins = 0;
        while ((rw >> 16) != tag && !pd_expired(ck, spins)) rw = ld_c32(P.ll_hm + r0 + t);
        v = v * 1.f + h2f_bits(rw & 0xFFFFu);
        const uint32_t hb = f16_bits(v);
        st_c32(P.ll_h + r0 + t, ll16(hb, tag));
        if (last) reinterpret_cast<uint16_t*>(P.h_out)[r0 + t] = (uint16_t)hb;
    }
    __syncthreads();
}

// ------------------------------------------------------------------ L2 warm-up
// While the attention stages run on a few blocks, the HBM stream is idle.  A
// block then requests one word of every 128-byte line of its gate/up tile and
// of its down tile (before the o-proj wait), so those weights sit in its XCD's
// L2 (and the MALL) when their stages request them.  The words are held in
// registers until the o-proj wait has covered them (loads complete in order),
// so the warm-up never makes the block wait longer than it waits anyway.
struct PdTouch {
    uint32_t v[7];
};
__device__ __forceinline__ uint32_t pd_ld_word(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)3);
}
// gate rows then up rows of this block's SwiGLU tile: two contiguous ranges
__device__ __forceinline__ void pd_touch_gu(const PdStage& S5, PdTouch& t) {
    const int tid = threadIdx.x, b = blockIdx.x;
    if (b >= S5.total) return;
    const TileGeo T = pd_geo(S5, b);
    const int bytes = T.hA * T.rb;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int off = (tid + PD_T * i) * 128;
        if (off < bytes) {
            t.v[2 * i] = pd_ld_word(T.bA + off);
            t.v[2 * i + 1] = pd_ld_word(T.bB + off);
        }
    }
}
// one super-block of each row of this block's down tile (up to three lines)
__device__ __forceinline__ void pd_touch_down(const VtePdPlan& P, const VtePdLayer& Ly, PdTouch& t) {
    const int tid = threadIdx.x, b = blockIdx.x;
    const int nsl = P.ffn / QK_K, rt = (P.hidden + P.r_dn - 1) / P.r_dn;
    if (b >= nsl * rt) return;
    const int s = b / rt, j0 = (b - s * rt) * P.r_dn, nr = min(P.r_dn, P.hidden - j0);
    const int bpb = Ly.fmt_down == 4 ? Q4K_BYTES : Q6K_BYTES, rb = nsl * bpb;
    if (tid < nr) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(Ly.w_down) + (size_t)(j0 + tid) * rb + (size_t)s * bpb;
        t.v[4] = pd_ld_word(p);
        t.v[5] = pd_ld_word(p + bpb / 2);
        t.v[6] = pd_ld_word(p + bpb - 4);
    }
}
__device__ __forceinline__ void pd_touch_done(const PdTouch& t) {
    asm volatile("" ::"v"(t.v[0]), "v"(t.v[1]), "v"(t.v[2]), "v"(t.v[3]), "v"(t.v[4]), "v"(t.v[5]), "v"(t.v[6]));
}

// ------------------------------------------------------------------ the kernel

template <bool RO_H>
__global__ __launch_bounds__(PD_T, 1) void decode_persistent_kernel(VtePdPlan P) {
    extern __shared__ uint4 pd_smem[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(pd_smem);
    __shared__ PdAttLDS A;
    __shared__ float red[4];
    const uint32_t epoch = ld_c32(P.ctrl);
    const int pos = P.kv_offset[0];
    if (pos < 0 || pos >= P.max_seq) {  // every block sees the same value: none writes, none waits
        if (blockIdx.x == 0 && threadIdx.x == 0) __hip_atomic_fetch_or(P.ctrl + 2, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const PdClock ck{pd_now() + P.timeout_ticks, P.ctrl + 2};
    const int H = P.hidden, F = P.ffn, qd = P.n_q * ATT_D, kvd = P.n_kv * ATT_D;
    const int G = gridDim.x, b = blockIdx.x;
    // attention geometry: ns splits of the pos cached rows, at most PD_MS per KV head
    const int split = max(P.split_min, ((pos + PD_MS - 1) / PD_MS + ATT_TILE - 1) / ATT_TILE * ATT_TILE);
    const int ns = (pos + split - 1) / split;
    // combine blocks per query head: enough that a thread's first 8 records cover every split
    const int np3 = ns <= 16 ? 1 : ns <= 32 ? 2 : ns <= 64 ? 4 : 8;
    const __half* cosp = P.rope_cos + (size_t)pos * ATT_D;
    const __half* sinp = P.rope_sin + (size_t)pos * ATT_D;
    for (int l = 0; l < P.n_layers; ++l) {
        const VtePdLayer& Ly = P.layers[l];
        const uint32_t tag32 = epoch * (uint32_t)P.n_layers + (uint32_t)l, tag = tag32 & 0xFFFFu;
        const uint32_t ptag = (tag32 - 1u) & 0xFFFFu;  // the previous layer's
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
        PdStage S1;
        S1.K = H;
        S1.nseg = 3;
        S1.seg[0] = pd_seg((const uint8_t*)Ly.wq, nullptr, Ly.q_bias, Ly.fmt_q, qd, P.r_qk, FMV_ROPE_Q, H);
        S1.seg[1] = pd_seg((const uint8_t*)Ly.wk, nullptr, Ly.k_bias, Ly.fmt_k, kvd, P.r_qk, FMV_ROPE_KCACHE, H);
        S1.seg[2] = pd_seg((const uint8_t*)Ly.wv, nullptr, Ly.v_bias, Ly.fmt_v, kvd, P.r_v, FMV_VCACHE, H);
        S1.total = S1.seg[0].tiles + S1.seg[1].tiles + S1.seg[2].tiles;
        // attention items run on the blocks after the S1 tiles (item it on block
        // (S1.total + it) mod G), which request their first split's cached K/V
        // rows toward the L2 now, while the q/k/v stage runs elsewhere
        const int n_items = P.n_kv * ns, it0 = (b - S1.total % G + G) % G;
        const uint2 katt = it0 < n_items && b >= S1.total ? pd_attn_touch(P, Ly, it0 / ns, it0 % ns, split, pos)
                                                          : make_uint2(0u, 0u);
        o.ll = P.ll_q;
        pd_mv<UPT_QKV, RO_H, false>(S1, hin, !first, ptag, (const __half*)Ly.attn_norm, P.eps, lds, red, o, ck);
        PdStage So;
        So.K = qd;
        So.nseg = 1;
        So.seg[0] = pd_seg((const uint8_t*)Ly.wo, nullptr, nullptr, Ly.fmt_o, H, P.r_o, FMV_STORE_F16, qd);
        So.total = So.seg[0].tiles;

        // ---- S2: split-KV partials ----
        asm volatile("" ::"v"(katt.x), "v"(katt.y));
        for (int it = it0; it < n_items; it += G) pd_attn_item(P, Ly, it / ns, it % ns, split, pos, tag, tag32, A, ck);
        // ---- S3: combine per query head (the last n_q * np3 blocks) ----
        // (np3 blocks per head when the splits are many: fewer rounds per thread)
        for (int i = G - 1 - b; i >= 0 && i < P.n_q * np3; i += G)
            pd_attn_combine(P, i / np3, i % np3, np3, ns, tag, tag32, A, ck);
        PdStage S5;
        S5.K = H;
        S5.nseg = 1;
        S5.seg[0] = pd_seg((const uint8_t*)Ly.w_gate, (const uint8_t*)Ly.w_up, nullptr, Ly.fmt_gate_up, F, P.r_gu,
                           FMV_SWIGLU, H);
        S5.total = S5.seg[0].tiles;
        // ---- S4: o-proj + residual; the combine blocks (its critical path) skip the warm-up ----
        o.ll = P.ll_hm;
        o.res = hin;
        o.res_ll = !first;
        o.res_tag = ptag;
        {
            TileW<UPT_O> W;
            TileGeo T;
            PdPre pre;
            pd_begin<UPT_O, RO_H>(So, W, T, pre, o);
            PdTouch tw;
#pragma unroll
            for (int i = 0; i < 7; ++i) tw.v[i] = 0u;
            if (G - 1 - b >= P.n_q * np3) {
                pd_touch_gu(S5, tw);
                pd_touch_down(P, Ly, tw);
            }
            pd_run<UPT_O, RO_H, false>(So, W, T, pre, P.ll_att, true, tag, nullptr, P.eps, lds, red, o, ck);
            pd_touch_done(tw);
        }
        // ---- S5: norm + gate/up + SwiGLU ----
        o.ll = P.ll_act;
        pd_mv<UPT_GU, RO_H, false>(S5, P.ll_hm, true, tag, (const __half*)Ly.ffn_norm, P.eps, lds, red, o, ck);
        // ---- S6a: down partials; S7: their sum + residual -> the layer output ----
        pd_down_part(P, Ly, tag, tag32, lds, red, ck);
        pd_down_reduce(P, tag, tag32, l == P.n_layers - 1, lds, ck);
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
    const bool ro_h = fmv_ro(P.hidden);
    if (ro_h != fmv_ro(P.n_q * ATT_D)) return hipErrorNotSupported;
    if (ro_h) hipLaunchKernelGGL((decode_persistent_kernel<true>), dim3(blocks), dim3(PD_T), lds, st, P);
    else hipLaunchKernelGGL((decode_persistent_kernel<false>), dim3(blocks), dim3(PD_T), lds, st, P);
    return hipGetLastError();
}

int decode_persistent_occupancy(const VtePdPlan& P, size_t lds) {
    int n = 0;
    const hipError_t e =
        fmv_ro(P.hidden) ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<true>, PD_T, lds)
                         : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_kernel<false>, PD_T, lds);
    return e == hipSuccess ? n : -1;
}

}  // namespace vte
