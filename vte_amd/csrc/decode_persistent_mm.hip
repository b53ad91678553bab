// Persistent decode step for a batch of up to 16 sequences, gfx950.
//
// The batched decode step (vte/core/batched_hip_graph_executor.py:231-292:
// the layers of qwen_compute.py:100-282 with grid.y = batch) as ONE launch of
// one 256-thread block per CU, each sequence at its own position (ragged
// caches).  The stages of a layer are the batch-1 persistent step's
// (decode_persistent.hip), with the projections on MFMA: a stage's
// activations for all B columns are staged once per block into LDS as fp16
// [16][K] (RMS-normalised where the stage starts with a norm) and the block's
// tiles of 16 weight rows run the exact-operand super-block MFMAs of the
// batched kernels (mfma_deq.h) over them, the 4 waves splitting K and each
// wave requesting every tile's weights of a super-block at once:
//
//   S1  RMSNorm + q/k/v + bias + RoPE + K/V append       one 16-row tile per block (q, k: 8 RoPE pairs)
//   S2  split-KV attention partials                       (sequence, KV head, split) items
//   S3  log-sum-exp combine + the new token's own row     (sequence, query head) items
//   S4  o-proj + residual                                 16-row tiles
//   S5  RMSNorm + gate/up + SwiGLU                        tiles of 8 gate + 8 up rows, up to 5 per block
//   S6a down partial sums over one slice of sl_sb         (slice, 16-row tile)
//       super-blocks of the SwiGLU output
//   S7  sum of the slice partials + residual              B * hidden outputs spread over the blocks
//
// Values cross blocks as flagged words (pd_shared.h): fp16 | tag << 16 for
// activations, fp32 | tag << 32 for attention records and down partials, the
// tag consecutive over layers and launches (epoch * n_layers + layer), so the
// buffers are reused without clearing; the same stage order as the batch-1
// step makes the reuse safe (each buffer's next writer runs after a stage
// that waited on all of its readers' outputs).  Every wait is bounded (error
// flag, then the kernel drains).  A block waiting on a stage first spins on a
// few words of its input (every 16th of the last column), then requests the
// whole input in coalesced 64-bit loads.
//
// The LM head is not part of this launch: the last layer's output goes to a
// plain fp16 [B][hidden] buffer for the caller's norm + LM-head launches.
//
// Numerics: the batched path's (fp16 activations, exact integer weight
// operands, fp32 sums, the same fp16 rounding points); sums over K are split
// over 4 waves instead of the graph kernels' 6 or 8 and the down projection
// sums slice by slice, so results agree with the graph path to fp32 rounding.
//
// Measured on the 1.5B shape at batch 16 (2048-row caches): 2.08 ms per step
// against 1.54 ms for the batched graph, so the graph stays the default and
// this step is opt-in.  Per layer ~70 us against ~55 us; stage clocks of a
// probe build (VTE_PB_TRACE) put most of it in the hand-offs of the 96 KB
// activation blocks: a consumer sees the producing stage's last words within
// ~0.2 us, but then needs two rounds of device-coherent loads of freshly
// written lines (~1.8 us each; one round of all 48 pairs per thread does not
// fit the registers beside their addresses) plus its LDS writes, 5-6 us in
// all; and in the gate/up and down stages, whose 4 waves per CU (one block
// per CU) hide less memory latency than the graph kernels' 12.

#include "fused_kernels.h"
#include "mfma_deq.h"
#include "decode_persistent.h"
#include "pd_shared.h"

namespace {

#ifdef VTE_PB_TRACE  // probe builds only: per-block stage clocks after the workspace
#define PB_STAMP(k) \
    if (tid == 0) P.trace[(size_t)(b * P.n_layers + l) * 16 + (k)] = (uint32_t)pd_now()
#else
#define PB_STAMP(k)
#endif

constexpr int PB_NW = 4;     // waves per block
constexpr int PB_RT_GU = 5;  // gate/up tiles a block runs together (1120 tiles of the 1.5B shape on 256 blocks: <= 5)
constexpr int PB_RT_DN = 3;  // down row tiles a block runs together
constexpr int PB_MAXK = VTE_PB_MAX_K;  // longest activation row a stage stages (hidden, q_dim, down slice)
constexpr int PB_NP = 16 * PB_MAXK / 2 / PD_T;  // word pairs per thread of a full staging
constexpr int PB_NR = PB_NP / 2;                 // pairs per thread in flight per round

// Device-coherent 64-bit load through a global-address-space pointer (so a
// wave's loads share one base register and an immediate offset).
typedef __attribute__((address_space(1))) uint64_t pb_g64;
__device__ __forceinline__ uint64_t pb_ld64(const uint32_t* p) {
    return __hip_atomic_load((pb_g64*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__host__ __device__ constexpr int pb_ldx(int K) { return K + 8; }  // LDS row stride (halves): conflict-free column reads

// ---------------------------------------------------------------- staging
// Columns m < B of K flagged fp16 words each, contiguous ([B][K] at src)
// -> LDS xs[m][0..K) as fp16, every word requested at once and re-polled
// until all carry `tag`.  With norm_w: each column RMS-normalised,
// fp16(x * rsqrt(mean(x^2) + eps) * w), its sum of squares in a fixed order.
// ll = false: plain fp16 source (the layer-0 input).  Ends with a barrier.
__device__ __forceinline__ void pb_stage(const void* src, bool ll, int K, int B, uint32_t tag,
                                         const __half* norm_w, float eps, __half* xs, float* inv,
                                         const PdClock& ck) {
    const int tid = threadIdx.x, cpc = K / 8, nch = B * cpc, ld = pb_ldx(K);
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
    if (ll) {
        // first every 16th word of the last column, one per thread: a block
        // waiting on a stage that has not finished spins on these few words
        // instead of re-requesting the whole input (which would also slow
        // down the blocks producing it)
        if (tid < K / 16) {
            const uint32_t* p = s32 + (size_t)(B - 1) * K + 16 * tid;
            uint32_t v = ld_c32(p);
            int spins = 0;
            while ((v >> 16) != tag && !pd_expired(ck, spins)) v = ld_c32(p);
        }
        __syncthreads();
    }
    // the input is [B][K] contiguous: word pair f = tid + 256 j, so each
    // wave-wide load covers 512 contiguous bytes; pair f is column m = f / cpp
    const int cpp = K / 2, npair = B * cpp;
    const float rcpp = 1.0f / (float)cpp;
    // in rounds of PB_NR pairs per thread (the round's loads all in flight)
    for (int r0 = 0; r0 < PB_NP; r0 += PB_NR) {
        if (r0 * PD_T >= npair) break;
        uint64_t w[PB_NR];
        if (ll) {
            // straight-line loads without a bounds test (one address register):
            // pairs past npair read the workspace buffer that follows this one
            // (every flagged input has one) and count as ready
#pragma unroll
            for (int j = 0; j < PB_NR; ++j) w[j] = pb_ld64((s32 + 2 * PD_T * (r0 + j)) + (uint32_t)(2 * tid));
            int spins = 0;
            while (true) {
                bool all = true;
#pragma unroll
                for (int j = 0; j < PB_NR; ++j) {
                    const bool okj = ok2(w[j], tag) || tid + PD_T * (r0 + j) >= npair;
                    all = all && okj;
                    if (!okj) w[j] = pb_ld64((s32 + 2 * PD_T * (r0 + j)) + (uint32_t)(2 * tid));
                }
                if (all || pd_expired(ck, spins)) break;
            }
        } else {  // the layer-0 input (a caller's buffer): bounded reads
#pragma unroll
            for (int j = 0; j < PB_NR; ++j) {
                const int f = tid + PD_T * (r0 + j);
                const uint32_t h = f < npair ? reinterpret_cast<const uint32_t*>(src)[f] : 0u;
                w[j] = (uint64_t)(h & 0xFFFFu) | ((uint64_t)(h >> 16) << 32);
            }
        }
#pragma unroll
        for (int j = 0; j < PB_NR; ++j) {
            const int f = tid + PD_T * (r0 + j);
            if (f < npair) {
                const int m = (int)(((float)f + 0.5f) * rcpp);  // exact for f < 2^20
                *reinterpret_cast<uint32_t*>(xs + 2 * f + 8 * m) = pair2(w[j]);  // m * (K + 8) + 2 (f - m cpp)
            }
        }
    }
    __syncthreads();
    if (norm_w == nullptr) return;
    // per column: 16 threads sum strided 8-element chunks, then a 16-lane tree
    {
        const int m = tid >> 4, r = tid & 15;
        float ss = 0.f;
        if (m < B) {
            for (int k = 8 * r; k < K; k += 128) {
                const uint4 v = *reinterpret_cast<const uint4*>(xs + (size_t)m * ld + k);
                const uint32_t h[4] = {v.x, v.y, v.z, v.w};
                ss += chunk_sumsq(h);
            }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
        if (r == 0 && m < B) inv[m] = rsqrtf(ss / (float)K + eps);
    }
    __syncthreads();
    const uint4* nv = reinterpret_cast<const uint4*>(norm_w);
    for (int c = tid; c < nch; c += PD_T) {
        const int m = c / cpc, k = (c - m * cpc) * 8;
        uint4* p = reinterpret_cast<uint4*>(xs + (size_t)m * ld + k);
        const uint4 v = *p;
        uint32_t h[4] = {v.x, v.y, v.z, v.w};
        chunk_norm(h, nv[k / 8], inv[m]);
        *p = make_uint4(h[0], h[1], h[2], h[3]);
    }
    __syncthreads();
}

// ---------------------------------------------------------------- MFMA tiles
// A block's tiles of a stage (up to RT, 16 weight rows each) run together:
// the 4 waves split the super-blocks, and per super-block a wave requests the
// raw weights of every tile at once before its MFMAs, so one memory round
// trip serves all the block's tiles.  rowp[rt]: the weight row of this
// lane's MFMA column (lane & 15) in tile rt, at the stage's first
// super-block.  red: [PB_NW][RT][4][64] partial C tiles, summed over the
// waves in wave order by pb_sum.
template <int FMT, int RT>
__device__ __forceinline__ void pb_mma(const uint8_t* const (&rowp)[RT], int n_sb, const __half* xs, int ld, int B,
                                       float* red) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, col = lane & 15, grp = lane >> 4;
    const int sb0 = (n_sb * wv) / PB_NW, sb1 = (n_sb * (wv + 1)) / PB_NW;
    floatx4_t acc[RT][1];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt][0] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    const __half* xc = xs + (size_t)(col < B ? col : 0) * ld;
    for (int sb = sb0; sb < sb1; ++sb) {
        typename SbRaw<FMT>::Raw raw[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sb_load(rowp[rt] + (size_t)sb * (FMT == 4 ? Q4K_BYTES : Q6K_BYTES), grp, raw[rt]);
        half8_t bx[8][1];
#pragma unroll
        for (int t = 0; t < 8; ++t) bx[t][0] = load_x8<__half>(xc + sb * QK_K + kslot_base<FMT>(t, grp), col < B);
        XMin<1, false> xm;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            typename SbRaw<FMT>::Ops ops;
            sb_ops<false>(raw[rt], grp, ops);
            sb_mfma<1>(ops, bx, xm, acc[rt]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wv * RT + rt) * 4 + i) * 64 + lane] = acc[rt][0][i];
}

// Tile rt's result for weight row rr (0..15) and batch column m.
template <int RT>
__device__ __forceinline__ float pb_sum(const float* red, int rt, int rr, int m) {
    const int ln = c_lane(rr, m), i = c_reg(m);
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < PB_NW; ++w) s += red[((w * RT + rt) * 4 + i) * 64 + ln];
    return s;
}

// The block's tiles t < nt of a stage in groups of RT (rows of tiles past nt
// repeat the last tile; their results are not stored), each group's results
// handed to out(t, red) after a barrier.
template <int FMT, int RT, typename RowF, typename OutF>
__device__ __forceinline__ void pb_tiles(int nt, int n_sb, RowF rowp, const __half* xs, int ld, int B, float* red,
                                         OutF out) {
    for (int t0 = 0; t0 < nt; t0 += RT) {
        const uint8_t* rp[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) rp[rt] = rowp(min(t0 + rt, nt - 1));
        pb_mma<FMT, RT>(rp, n_sb, xs, ld, B, red);
        __syncthreads();
        out(t0, min(RT, nt - t0));
        __syncthreads();
    }
}

__device__ __forceinline__ int pb_bpb(int fmt) { return fmt == 4 ? Q4K_BYTES : Q6K_BYTES; }

// S5 on one block: its ntl tiles (8 gate + 8 up rows each).
template <int FMT, typename RowF>
__device__ __forceinline__ void pb_gate_up(const VtePbPlan& P, RowF rowp, int ntl, int n_sb, int b, int G, int Bn,
                                           uint32_t tag, const VtePdLayer& Ly, __half* xs, float* inv, float* red,
                                           const PdClock& ck) {
    const int H = P.hidden, F = P.ffn, tid = threadIdx.x;
    pb_tiles<FMT, PB_RT_GU>(ntl, n_sb, rowp, xs, pb_ldx(H), Bn, red, [=](int t0, int nt) {
        for (int o = tid; o < nt * 8 * Bn; o += PD_T) {
            const int t = o / (8 * Bn), r = o - t * 8 * Bn, p = r & 7, m = r >> 3;
            const float gg = __half2float(__float2half(pb_sum<PB_RT_GU>(red, t, p, m)));
            const float uu = __half2float(__float2half(pb_sum<PB_RT_GU>(red, t, p + 8, m)));
            // slice-major [slice][m][slice width]: each down slice reads one contiguous block
            const int row = (b + G * (t0 + t)) * 8 + p, SW = P.sl_sb * QK_K, sl = row / SW;
            const int sw = min(SW, F - sl * SW);
            st_c32(P.ll_act + (size_t)sl * SW * Bn + (size_t)m * sw + (row - sl * SW),
                   ll16(f16_bits(gg / (1.0f + expf(-gg)) * uu), tag));
        }
    });
}

// S6a on one block: slice s's partial sums for its row tiles jb + bps k.
template <int FMT, typename RowF>
__device__ __forceinline__ void pb_down(const VtePbPlan& P, RowF rowp, int ntl, int nsb, int s, int sb0, int jb,
                                        int bps, int Bn, uint32_t tag, uint32_t tag32, __half* xs, float* inv,
                                        float* red, const PdClock& ck) {
    const int H = P.hidden, F = P.ffn, tid = threadIdx.x, sw = nsb * QK_K;
    pb_tiles<FMT, PB_RT_DN>(ntl, nsb, rowp, xs, pb_ldx(sw), Bn, red, [=](int t0, int nt) {
        for (int o = tid; o < nt * 16 * Bn; o += PD_T) {
            const int t = o / (16 * Bn), r = o - t * 16 * Bn, p = r & 15, m = r >> 4;
            st_c64(P.ll_dn + ((size_t)s * Bn + m) * H + (jb + bps * (t0 + t)) * 16 + p,
                   ll32(pb_sum<PB_RT_DN>(red, t, p, m), tag32));
        }
    });
}

// ---------------------------------------------------------------- the kernel
struct PbSeqs {
    int pos[16], split[16], ns[16], it0[16];  // it0: first attention item of each sequence
    int n_items, ns_max, bad;
};

__global__ __launch_bounds__(PD_T, 1) void decode_persistent_mm_kernel(VtePbPlan P) {
    extern __shared__ uint4 pb_smem[];
    __shared__ PdAttLDS A;
    __shared__ float red[PB_NW * PB_RT_GU * 4 * 64];
    __shared__ float inv[16];
    __shared__ PbSeqs Q;  // per-sequence attention geometry
    const int tid = threadIdx.x, G = gridDim.x, b = blockIdx.x, Bn = P.B;
    const uint32_t epoch = ld_c32(P.ctrl);
    if (tid == 0) {
        int n = 0, mx = 0, bad = 0;
        for (int m = 0; m < 16; ++m) {
            const int pos = m < Bn ? P.kv_offset[m] : 0;
            bad |= pos < 0 || pos >= P.max_seq;
            const int sp = max(P.split_min, ((pos + PD_MS - 1) / PD_MS + ATT_TILE - 1) / ATT_TILE * ATT_TILE);
            Q.pos[m] = pos;
            Q.split[m] = sp;
            Q.ns[m] = m < Bn ? (pos + sp - 1) / sp : 0;
            Q.it0[m] = n;
            n += P.n_kv * Q.ns[m];
            mx = max(mx, Q.ns[m]);
        }
        Q.n_items = n;
        Q.ns_max = mx;
        Q.bad = bad;
    }
    __syncthreads();
    if (Q.bad) {  // every block sees the same positions: none writes, none waits
        if (b == 0 && tid == 0) __hip_atomic_fetch_or(P.ctrl + 2, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const PdClock ck{pd_now() + P.timeout_ticks, P.ctrl + 2};
    __half* xs = reinterpret_cast<__half*>(pb_smem);
    const int H = P.hidden, F = P.ffn, qd = P.n_q * ATT_D, kvd = P.n_kv * ATT_D;
    const int nsb_f = F / QK_K, nsl = (nsb_f + P.sl_sb - 1) / P.sl_sb;
    const int np3 = Q.ns_max <= 16 ? 1 : Q.ns_max <= 32 ? 2 : Q.ns_max <= 64 ? 4 : 8;
    // tiles: S1 q (8 RoPE pairs) + k (8 pairs) + v (16 rows); S4 16 rows; S5 16 gate + 16 up rows
    const int t_q = qd / 16, t_k = kvd / 16, t_v = kvd / 16, t_s1 = t_q + t_k + t_v;
    const int t_o = H / 16, t_gu = F / 8, t_dn_rows = H / 16;
    const int bps = max(1, G / nsl);  // blocks per down slice
    for (int l = 0; l < P.n_layers; ++l) {
        const VtePdLayer& Ly = P.layers[l];
        const uint32_t tag32 = epoch * (uint32_t)P.n_layers + (uint32_t)l, tag = tag32 & 0xFFFFu;
        const uint32_t ptag = (tag32 - 1u) & 0xFFFFu;
        const bool first = l == 0;
        const void* hin = first ? (const void*)P.x : (const void*)P.ll_h;
        const __half* kc = reinterpret_cast<const __half*>(Ly.k_cache);
        const __half* vc = reinterpret_cast<const __half*>(Ly.v_cache);

        PB_STAMP(0);
        // ---- S1: norm + q/k/v + bias + RoPE + K/V append ----
        if (b < t_s1) {
            const int g = b;  // t_s1 <= G (checked on the host)
            const int seg = g < t_q ? 0 : g < t_q + t_k ? 1 : 2;
            const int fmt = seg == 0 ? Ly.fmt_q : seg == 1 ? Ly.fmt_k : Ly.fmt_v;
            const uint8_t* wbase = (const uint8_t*)(seg == 0 ? Ly.wq : seg == 1 ? Ly.wk : Ly.wv);
            const __half* bias = (const __half*)(seg == 0 ? Ly.q_bias : seg == 1 ? Ly.k_bias : Ly.v_bias);
            const int gi = seg == 0 ? g : seg == 1 ? g - t_q : g - t_q - t_k;
            // RoPE tiles: rows j0 .. j0 + 7 and their partners j0 + 64 ..; V: rows j0 .. j0 + 15
            const int j0 = seg < 2 ? (gi / 8) * 128 + (gi % 8) * 8 : gi * 16;
            const int rb = (H / QK_K) * pb_bpb(fmt), col = tid & 15;
            const int wrow = seg < 2 ? j0 + (col & 7) + (col >> 3) * 64 : j0 + col;
            const uint8_t* rp1[1] = {wbase + (size_t)wrow * rb};
            if (fmt == 4) {
                pb_stage(hin, !first, H, Bn, ptag, (const __half*)Ly.attn_norm, P.eps, xs, inv, ck);
                PB_STAMP(8);
                pb_mma<4, 1>(rp1, H / QK_K, xs, pb_ldx(H), Bn, red);
            } else {
                pb_stage(hin, !first, H, Bn, ptag, (const __half*)Ly.attn_norm, P.eps, xs, inv, ck);
                pb_mma<6, 1>(rp1, H / QK_K, xs, pb_ldx(H), Bn, red);
            }
            __syncthreads();
            if (seg < 2) {
                if (tid < 8 * Bn) {
                    const int p = tid & 7, m = tid >> 3, row = j0 + p, d = row & 127;
                    const float x1 = __half2float(__float2half(pb_sum<1>(red, 0, p, m) + (bias ? __half2float(bias[row]) : 0.f)));
                    const float x2 =
                        __half2float(__float2half(pb_sum<1>(red, 0, p + 8, m) + (bias ? __half2float(bias[row + 64]) : 0.f)));
                    const int pos = Q.pos[m];
                    const float c = __half2float(P.rope_cos[(size_t)pos * ATT_D + d]);
                    const float sn = __half2float(P.rope_sin[(size_t)pos * ATT_D + d]);
                    const uint32_t o1 = f16_bits(x1 * c - x2 * sn), o2 = f16_bits(x1 * sn + x2 * c);
                    if (seg == 0) {
                        st_c32(P.ll_q + (size_t)m * qd + row, ll16(o1, tag));
                        st_c32(P.ll_q + (size_t)m * qd + row + 64, ll16(o2, tag));
                    } else {
                        uint16_t* kr = reinterpret_cast<uint16_t*>(Ly.k_cache) + (size_t)m * P.kv_batch_stride +
                                       ((size_t)pos * P.n_kv + row / 128) * 128;
                        kr[d] = (uint16_t)o1;
                        kr[d + 64] = (uint16_t)o2;
                        st_c32(P.ll_kv + (size_t)m * 2 * kvd + row, ll16(o1, tag));
                        st_c32(P.ll_kv + (size_t)m * 2 * kvd + row + 64, ll16(o2, tag));
                    }
                }
            } else if (tid < 16 * Bn) {
                const int p = tid & 15, m = tid >> 4, row = j0 + p;
                const uint32_t hb = f16_bits(pb_sum<1>(red, 0, p, m) + (bias ? __half2float(bias[row]) : 0.f));
                const int pos = Q.pos[m];
                reinterpret_cast<uint16_t*>(Ly.v_cache)[(size_t)m * P.kv_batch_stride +
                                                        ((size_t)pos * P.n_kv + row / 128) * 128 + (row & 127)] =
                    (uint16_t)hb;
                st_c32(P.ll_kv + (size_t)m * 2 * kvd + kvd + row, ll16(hb, tag));
            }
            __syncthreads();
        }

        PB_STAMP(1);
        // ---- S2: split-KV partials, items after the S1 blocks ----
        for (int it = (b - t_s1 % G + G) % G; it < Q.n_items; it += G) {
            int m = 0;
            while (m + 1 < Bn && Q.it0[m + 1] <= it) ++m;
            const int r = it - Q.it0[m], kvh = r / Q.ns[m], c = r - kvh * Q.ns[m];
            const PdSeqAttn SA{P.n_q, P.n_kv, P.scale, kc + (size_t)m * P.kv_batch_stride,
                               vc + (size_t)m * P.kv_batch_stride, P.ll_q + (size_t)m * qd,
                               P.ll_kv + (size_t)m * 2 * kvd, P.ll_att + (size_t)m * qd,
                               P.part + (size_t)m * P.n_q * PD_MS * PD_PW};
            pd_attn_item(SA, kvh, c, Q.split[m], Q.pos[m], tag, tag32, A, ck);
        }
        PB_STAMP(2);
        // ---- S3: combine per (sequence, query head), on the last blocks ----
        for (int i = G - 1 - b; i >= 0 && i < Bn * P.n_q * np3; i += G) {
            const int m = i / (P.n_q * np3), r = i - m * P.n_q * np3;
            const PdSeqAttn SA{P.n_q, P.n_kv, P.scale, kc + (size_t)m * P.kv_batch_stride,
                               vc + (size_t)m * P.kv_batch_stride, P.ll_q + (size_t)m * qd,
                               P.ll_kv + (size_t)m * 2 * kvd, P.ll_att + (size_t)m * qd,
                               P.part + (size_t)m * P.n_q * PD_MS * PD_PW};
            pd_attn_combine(SA, r / np3, r % np3, np3, Q.ns[m], tag, tag32, A, ck);
        }

        PB_STAMP(3);
        // ---- S4: o-proj + residual ----
        for (int g = b; g < t_o; g += G) {
            const int j0 = g * 16, rb = (qd / QK_K) * pb_bpb(Ly.fmt_o);
            const uint8_t* rp1[1] = {(const uint8_t*)Ly.wo + (size_t)(j0 + (tid & 15)) * rb};
            // residual word of this thread's output, requested before the wait
            const int p = tid & 15, m = tid >> 4, row = j0 + p;
            uint32_t rw = 0u;
            if (m < Bn)
                rw = first ? (uint32_t)reinterpret_cast<const uint16_t*>(P.x)[(size_t)m * H + row]
                           : ld_c32(P.ll_h + (size_t)m * H + row);
            if (Ly.fmt_o == 4) {
                pb_stage(P.ll_att, true, qd, Bn, tag, nullptr, 0.f, xs, inv, ck);
                PB_STAMP(9);
                pb_mma<4, 1>(rp1, qd / QK_K, xs, pb_ldx(qd), Bn, red);
            } else {
                pb_stage(P.ll_att, true, qd, Bn, tag, nullptr, 0.f, xs, inv, ck);
                pb_mma<6, 1>(rp1, qd / QK_K, xs, pb_ldx(qd), Bn, red);
            }
            __syncthreads();
            if (m < Bn) {
                if (!first) {
                    int spins = 0;
                    while ((rw >> 16) != ptag && !pd_expired(ck, spins)) rw = ld_c32(P.ll_h + (size_t)m * H + row);
                }
                const float v = pb_sum<1>(red, 0, p, m) * 1.f + h2f_bits(rw & 0xFFFFu);
                st_c32(P.ll_hm + (size_t)m * H + row, ll16(f16_bits(v), tag));
            }
            __syncthreads();
        }

        PB_STAMP(4);
        // ---- S5: norm + gate/up + SwiGLU, tiles of 8 gate + 8 up rows (tiles g = b + G k) ----
        if (b < t_gu) {
            const int rb = (H / QK_K) * pb_bpb(Ly.fmt_gate_up), n_sb = H / QK_K, col = tid & 15;
            const uint8_t* wsel = (const uint8_t*)(col < 8 ? Ly.w_gate : Ly.w_up);
            auto rowp = [=](int t) { return wsel + (size_t)((b + G * t) * 8 + (col & 7)) * rb; };
            const int ntl = (t_gu - b + G - 1) / G;
            pb_stage(P.ll_hm, true, H, Bn, tag, (const __half*)Ly.ffn_norm, P.eps, xs, inv, ck);
            PB_STAMP(10);
            if (Ly.fmt_gate_up == 4) pb_gate_up<4>(P, rowp, ntl, n_sb, b, G, Bn, tag, Ly, xs, inv, red, ck);
            else pb_gate_up<6>(P, rowp, ntl, n_sb, b, G, Bn, tag, Ly, xs, inv, red, ck);
        }

        PB_STAMP(5);
        // ---- S6a: down partials over slice s of sl_sb super-blocks (row tiles jb + bps k) ----
        {
            const int s = b / bps, jb = b - s * bps;
            if (s < nsl) {
                const int sb0 = s * P.sl_sb, nsb = min(P.sl_sb, nsb_f - sb0), col = tid & 15;
                const int bpb = pb_bpb(Ly.fmt_down), rb = nsb_f * bpb;
                const uint8_t* wd = (const uint8_t*)Ly.w_down + (size_t)sb0 * bpb;
                auto rowp = [=](int t) { return wd + (size_t)((jb + bps * t) * 16 + col) * rb; };
                const int ntl = (t_dn_rows - jb + bps - 1) / bps;
                pb_stage(P.ll_act + (size_t)sb0 * QK_K * Bn, true, nsb * QK_K, Bn, tag, nullptr, 0.f, xs, inv, ck);
                PB_STAMP(11);
                if (Ly.fmt_down == 4) pb_down<4>(P, rowp, ntl, nsb, s, sb0, jb, bps, Bn, tag, tag32, xs, inv, red, ck);
                else pb_down<6>(P, rowp, ntl, nsb, s, sb0, jb, bps, Bn, tag, tag32, xs, inv, red, ck);
            }
        }

        PB_STAMP(6);
        // ---- S7: sum of the slice partials (slice order) + residual ----
        {
            const int per = (Bn * H + G - 1) / G, o = b * per + tid;
            if (tid < per && o < Bn * H) {
                const int m = o / H, row = o - m * H;
                uint64_t pw[16];
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    pw[s] = s < nsl ? ld_c64(P.ll_dn + ((size_t)s * Bn + m) * H + row) : ((uint64_t)tag32 << 32);
                uint32_t rw = ld_c32(P.ll_hm + (size_t)m * H + row);
                int spins = 0;
                while (true) {
                    bool ok = (rw >> 16) == tag;
#pragma unroll
                    for (int s = 0; s < 16; ++s) ok = ok && (uint32_t)(pw[s] >> 32) == tag32;
                    if (ok || pd_expired(ck, spins)) break;
                    if ((rw >> 16) != tag) rw = ld_c32(P.ll_hm + (size_t)m * H + row);
#pragma unroll
                    for (int s = 0; s < 16; ++s)
                        if (s < nsl && (uint32_t)(pw[s] >> 32) != tag32) pw[s] = ld_c64(P.ll_dn + ((size_t)s * Bn + m) * H + row);
                }
                float v = 0.f;
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    if (s < nsl) v += __uint_as_float((uint32_t)pw[s]);
                v = v * 1.f + h2f_bits(rw & 0xFFFFu);
                const uint32_t hb = f16_bits(v);
                st_c32(P.ll_h + (size_t)m * H + row, ll16(hb, tag));
                if (l == P.n_layers - 1) reinterpret_cast<uint16_t*>(P.h_out)[(size_t)m * H + row] = (uint16_t)hb;
            }
        }
        PB_STAMP(7);
    }
    // ---- the last block to finish advances the epoch ----
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(P.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)G - 1) {
            st_c32(P.ctrl + 1, 0u);
            st_c32(P.ctrl, epoch + 1u);
        }
    }
}

}  // namespace

namespace vte {

size_t decode_persistent_mm_lds(int hidden, int q_dim, int slice) {
    const int K = std::max(std::max(hidden, q_dim), slice);
    return (size_t)16 * pb_ldx(K) * 2;
}

hipError_t decode_persistent_mm_launch(const VtePbPlan& P, int blocks, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL(decode_persistent_mm_kernel, dim3(blocks), dim3(PD_T), lds, st, P);
    return hipGetLastError();
}

int decode_persistent_mm_occupancy(size_t lds) {
    int n = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_persistent_mm_kernel, PD_T, lds);
    return e == hipSuccess ? n : -1;
}

}  // namespace vte
