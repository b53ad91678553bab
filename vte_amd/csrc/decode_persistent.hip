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
#include "pd_shared.h"

namespace {

static_assert(PD_T == ROWS_THREADS, "the mat-vec stages assume one unit layout per 256 threads");
constexpr int UPT_QKV = VTE_PD_UPT_QKV, UPT_O = 1, UPT_GU = VTE_PD_UPT_GU, UPT_D = 4;  // weight units per thread of each stage

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
    const PdSeqAttn SA{P.n_q, P.n_kv, P.scale, nullptr, nullptr, P.ll_q, P.ll_kv, P.ll_att, P.part};
    const __half* cosp = P.rope_cos + (size_t)pos * ATT_D;
    const __half* sinp = P.rope_sin + (size_t)pos * ATT_D;
    for (int l = 0; l < P.n_layers; ++l) {
        const VtePdLayer& Ly = P.layers[l];
        PdSeqAttn SL = SA;
        SL.k_cache = reinterpret_cast<const __half*>(Ly.k_cache);
        SL.v_cache = reinterpret_cast<const __half*>(Ly.v_cache);
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
        const uint2 katt = it0 < n_items && b >= S1.total ? pd_attn_touch(SL, it0 / ns, it0 % ns, split, pos)
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
        for (int it = it0; it < n_items; it += G) pd_attn_item(SL, it / ns, it % ns, split, pos, tag, tag32, A, ck);
        // ---- S3: combine per query head (the last n_q * np3 blocks) ----
        // (np3 blocks per head when the splits are many: fewer rounds per thread)
        for (int i = G - 1 - b; i >= 0 && i < P.n_q * np3; i += G)
            pd_attn_combine(SL, i / np3, i % np3, np3, ns, tag, tag32, A, ck);
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
