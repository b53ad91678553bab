// Split-KV flash-decoding attention over an fp16 KV cache, gfx950.
//
// Reference algorithm: vte/compiler/templates/rdna/kv_cache_append.hip.template:13-39,
// flash_attention_split_kv_partial.hip.template:31-120 (online softmax per chunk,
// partial m / l / o) and flash_attention_split_kv_reduce.hip.template:14-67
// (log-sum-exp combine).  KV layout is the reference's:
//   cache[b * kv_batch_stride + (pos * n_kv + kv_head) * head_dim + d]   (fp16)
// and the current position of sequence b is kv_offset[b] (positions 0..kv_offset
// are valid), read from device memory so one captured graph serves every step.
//
// MI355X design of the partial pass (one 256-thread block per (split, kv head, b)):
//  * GQA-aware: the block serves all G = n_q / n_kv query heads of its KV head,
//    so every K/V byte is read from HBM once (the reference reads it G times).
//  * Scores S^T[token][head] = K . Q^T come from MFMA 16x16x32 f16: K rows are
//    loaded straight into the A operand (16-byte loads), Q^T (padded to 16 heads)
//    is a per-block constant B operand.  fp32 accumulation.
//  * Online softmax on the MFMA C registers (one head per lane column).  P.V is
//    a second MFMA: P (fp16) is already in the A-operand layout in registers,
//    V rows are loaded coalesced and transposed through LDS (v_perm pairs) so
//    each lane reads its 8 B-operand tokens of one dimension with two 8-byte
//    LDS reads.  Both products accumulate in fp32.
//  * Ragged batches: per-sequence split count ceil((kv_offset[b]+1) / split);
//    blocks past a sequence's last split exit at once, and the combine reads
//    only that sequence's splits, so each sequence's result is independent of
//    the batch it sits in.
#include <cstdlib>
#include "vte_common.h"

#include "attn_tile.h"


// ---------------------------------------------------------------------------
// KV append (reference ABI, vte/compiler/templates/rdna/kv_cache_append.hip.template:13-39)
// grid (batch, n_kv), block (head_dim)
// ---------------------------------------------------------------------------
extern "C" __global__ void kv_cache_append_kernel(const __half* __restrict__ k, const __half* __restrict__ v,
                                                  __half* __restrict__ k_cache, __half* __restrict__ v_cache,
                                                  int num_kv_heads, int head_dim,
                                                  const int* __restrict__ kv_cache_offset_ptr,
                                                  int kv_batch_stride) {
    const int b = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    if (t >= head_dim) return;
    const int pos = kv_cache_offset_ptr[b];
    const size_t src = ((size_t)b * num_kv_heads + h) * head_dim + t;
    const size_t dst = (size_t)b * kv_batch_stride + ((size_t)pos * num_kv_heads + h) * head_dim + t;
    k_cache[dst] = k[src];
    v_cache[dst] = v[src];
}

// ---------------------------------------------------------------------------
// Native partial pass
// ---------------------------------------------------------------------------

// Partials of one split of one (sequence, KV head): grid (max_splits, n_kv, B),
// four waves, each taking 32-token tiles, the first TPW of them (1 or 2)
// loaded together.  SPEC: those tiles' K/V rows are requested before the
// sequence length is known (rows up to the split's
// end, which the host checked lie inside the sequence's cache), so the
// length and the first tile arrive in one memory round trip; rows at or past
// the length are masked (scores -inf, V zero).
// QC = 2: the block serves query columns 2z and 2z + 1, which read the same
// cache (kv_batch_stride 0: prompt tokens of one sequence), so each K/V tile
// is loaded once for both: MFMA N slots 0..G-1 are column 2z's heads and
// G..2G-1 column 2z + 1's, each slot masked at its own column's length.
template <typename TQ, typename TO, bool SPEC, int TPW, int QC = 1>
__global__ __launch_bounds__(256, TPW == 2 ? 1 : 3) void attn_partial_gqa(
    const TQ* __restrict__ q,            // [B][n_q][D]
    const __half* __restrict__ k_cache, const __half* __restrict__ v_cache,
    float* __restrict__ part_m, float* __restrict__ part_l, float* __restrict__ part_o,
    int n_q, int n_kv, float scale, const int* __restrict__ kv_offset, int kv_batch_stride,
    int split, int max_splits, int* __restrict__ counters, TO* __restrict__ out, int n_cols) {
    // TPW == 0: one 32-token split per wave (split == 32), no block combine
    constexpr bool PW = TPW == 0;
    static_assert(QC == 1 || (!PW && !SPEC), "two query columns per block: block-combined, non-speculative splits");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int sp = PW ? blockIdx.x * ATT_WAVES + wv : blockIdx.x, kvh = blockIdx.y, b = QC * blockIdx.z;
    if (PW && sp >= max_splits) return;
    const int t_begin = sp * split;
    const int G = n_q / n_kv;
    const int col = lane & 15;   // head (MFMA N index) / token row (A operand)
    const int grp = lane >> 4;   // 0..3
    const size_t row_stride = (size_t)n_kv * ATT_D;  // elements between consecutive positions
    const __half* kb = k_cache + (size_t)b * kv_batch_stride + (size_t)kvh * ATT_D;
    const __half* vb = v_cache + (size_t)b * kv_batch_stride + (size_t)kvh * ATT_D;
    const int len_raw = QC == 1 ? kv_offset[b] : max(kv_offset[b], kv_offset[min(b + 1, n_cols - 1)]);
    // in-kernel combine: this launch's record tag (the group's epoch + 1)
    // (counters[0]: sticky error word; counters[1 + b * n_kv + kvh]: the group's epoch)
    const uint32_t tag = counters != nullptr ? (uint32_t)counters[1 + (size_t)b * n_kv + kvh] + 1u : 0u;
    AttTile T, T1;
    int t0 = PW ? t_begin : t_begin + wv * ATT_TILE;
    if (SPEC) {
        att_load_tile(T, kb, vb, row_stride, t0, t_begin + split - 1, col, grp, lane);
        if (TPW == 2)
            att_load_tile(T1, kb, vb, row_stride, t0 + ATT_WAVES * ATT_TILE, t_begin + split - 1, col, grp, lane);
    }

    // B operand: Q^T for this KV head's G query heads, fp16, zero-padded to 16.
    // Rows past G read head G-1 and are zeroed by a select (no branch).
    half8_t qb[ATT_D / 32];
    // this lane's query slot: column b + qc, head hs of the group
    const int qc = QC == 1 ? 0 : min(col / G, QC - 1), hs = QC == 1 ? min(col, G - 1) : col - qc * G;
    const int bq = QC == 1 ? b : min(b + qc, n_cols - 1);
    const bool slot_ok = QC == 1 ? col < G : (col < QC * G && hs < G && b + qc < n_cols);
    {
        const int qh = kvh * G + min(hs, G - 1);
        const TQ* qp = q + ((size_t)bq * n_q + qh) * ATT_D;
#pragma unroll
        for (int s = 0; s < ATT_D / 32; ++s) {
            const half8_t v = att_load_q8(qp + 32 * s + 8 * grp);
            qb[s] = slot_ok ? v : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    const int len = len_raw + 1;
    if (t_begin >= len) return;  // past this sequence's last split (PW: this wave's)
    const int t_end = min(t_begin + split, len);
    const int t_end_col = QC == 1 ? t_end : min(t_begin + split, kv_offset[bq] + 1);

    // V tile of a wave, transposed: vt[d][t] (fp16, rows of 36 halves so the
    // 8-byte reads of 16 consecutive d rows hit distinct LDS banks)
    // Phases use disjoint LDS lifetimes: the V^T tiles (tile loop), the
    // per-wave O rows (block combine) and the split weights (LSE combine).
    union AttnLDS {
        uint32_t vt[ATT_WAVES][ATT_D][ATT_VT_STRIDE / 2];
        float o[ATT_WAVES][16][ATT_D + 4];  // heads >= G hold zeros (unconditional stores)
        float w[ATT_MAXG][ATT_MAX_COMBINE];
    };
    __shared__ AttnLDS lds;
    __shared__ float m_sh[ATT_WAVES][16], l_sh[ATT_WAVES][16];
    auto& vt_sh = lds.vt;
    auto& o_sh = lds.o;

    float m_run = -1e30f;  // running max of head `col` (identical across grp)
    float l_run = 0.f;     // per-lane partial denominator of head `col`
    // O[h][d] in the MFMA C layout: lane (col, grp) holds heads 4*grp + i, dim 16*dt + col
    floatx4_t o_acc[ATT_D / 16];
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt) o_acc[dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    if (!SPEC) {
        att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);
        if (TPW == 2) att_load_tile(T1, kb, vb, row_stride, t0 + ATT_WAVES * ATT_TILE, t_end - 1, col, grp, lane);
    }
    if (t0 < t_end) att_tile_step<true>(T, t0, t_end, qb, scale, m_run, l_run, o_acc, vt_sh[wv], lane, col, grp, t_end_col);
    if (PW) {  // the wave's split is done: its statistics and outputs are the partials
        l_run += __shfl_xor(l_run, 16, 64);
        l_run += __shfl_xor(l_run, 32, 64);
        const size_t st0 = ((size_t)b * n_q + kvh * G) * max_splits + sp;
        if (grp == 0 && col < G) {
            part_m[st0 + (size_t)col * max_splits] = m_run;
            part_l[st0 + (size_t)col * max_splits] = l_run;
        }
#pragma unroll
        for (int dt = 0; dt < ATT_D / 16; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int h = 4 * grp + i;
                if (h < G) part_o[(st0 + (size_t)h * max_splits) * ATT_D + 16 * dt + col] = o_acc[dt][i];
            }
        return;
    }
    t0 += ATT_WAVES * ATT_TILE;
    if (TPW == 2) {
        if (t0 < t_end) att_tile_step<false>(T1, t0, t_end, qb, scale, m_run, l_run, o_acc, vt_sh[wv], lane, col, grp, t_end_col);
        t0 += ATT_WAVES * ATT_TILE;
    }
    for (; t0 < t_end; t0 += ATT_WAVES * ATT_TILE) {
        att_load_tile(T, kb, vb, row_stride, t0, t_end - 1, col, grp, lane);
        att_tile_step<false>(T, t0, t_end, qb, scale, m_run, l_run, o_acc, vt_sh[wv], lane, col, grp, t_end_col);
    }

    // ---- combine the four waves of this block ----
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (grp == 0) { m_sh[wv][col] = m_run; l_sh[wv][col] = l_run; }
    __syncthreads();  // every wave is done with its V^T tile (o_sh overlays it)
#pragma unroll
    for (int dt = 0; dt < ATT_D / 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o_sh[wv][4 * grp + i][16 * dt + col] = o_acc[dt][i];
    __syncthreads();
    // thread -> (query slot h, dim): 256 threads cover 2 slots x 128 dims per pass
    for (int idx = threadIdx.x; idx < QC * G * ATT_D; idx += 256) {
        const int h = idx / ATT_D, d = idx % ATT_D;
        const int bc = b + h / G;  // the slot's query column
        if (QC > 1 && bc >= n_cols) break;
        float M = -1e30f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, m_sh[w][h]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; ++w) {
            const float c = __expf(m_sh[w][h] - M);
            L = fmaf(l_sh[w][h], c, L);
            O = fmaf(o_sh[w][h][d], c, O);
        }
        const int qh = kvh * G + h % G;
        const size_t st = ((size_t)bc * n_q + qh) * max_splits + sp;
        if (counters != nullptr) {  // flagged record, read back by the combining blocks
            uint64_t* rec = reinterpret_cast<uint64_t*>(part_o) + st * ATT_REC;
            st_flag32(rec + 2 + d, O, tag);
            if (d == 0) {
                st_flag32(rec, M, tag);
                st_flag32(rec + 1, L, tag);
            }
        } else {
            part_o[st * ATT_D + d] = O;
            if (d == 0) { part_m[st] = M; part_l[st] = L; }
        }
    }
    if (QC > 1 || counters == nullptr) return;  // separate combine launch

    // ---- the last G splits of this (sequence, KV head) combine one head each ----
    // Every split stored its records as flagged words (value | tag << 32,
    // device-coherent stores); a combining block polls the records of its head
    // until each carries this launch's tag: one memory round trip after the
    // last split, no completion counter, no fence.  The tag is the group's
    // epoch (counters[b][kvh], read by every block at its start) plus one; the
    // block combining head 0 advances the epoch once it has seen every split's
    // records (so every block of the group has read it), which makes the next
    // replay of a captured graph use a new tag.  Combining blocks are the
    // group's highest split indices, dispatched after the splits they wait for.
    const int ns = (len + split - 1) / split;
    const int r = ns - 1 - sp;
    if (r >= G) return;
    auto& wsh = lds.w;  // o_sh is dead once the records are stored
    __shared__ float Msh, Lsh;
    __shared__ float oh[ATT_D];
    for (int h = r; h < G; h += ns) {
        const int qh = kvh * G + h;
        const uint64_t* recs = reinterpret_cast<const uint64_t*>(part_o) + ((size_t)b * n_q + qh) * max_splits * ATT_REC;
        __syncthreads();  // LDS of the previous head
        for (int c = threadIdx.x; c < ns; c += 256) {
            float ml[2];
            if (!wait_flag32_n<2>(recs + (size_t)c * ATT_REC, 1, tag, ml))
                __hip_atomic_fetch_or(counters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wsh[0][c] = ml[0];
            wsh[1][c] = ml[1];
        }
        __syncthreads();
        if (wv == 0) {  // maximum, split weights exp(m_c - M) and the denominator
            float M = -1e30f;
            for (int c = lane; c < ns; c += 64) M = fmaxf(M, wsh[0][c]);
            M = wave_max(M);
            float Ls = 0.f;
            for (int c = lane; c < ns; c += 64) {
                const float wgt = __expf(wsh[0][c] - M);
                wsh[0][c] = wgt;
                Ls = fmaf(wsh[1][c], wgt, Ls);
            }
            Ls = wave_sum(Ls);
            if (lane == 0) { Msh = M; Lsh = Ls; }
        }
        __syncthreads();
        // threads (d, half): half 0 takes the even splits, half 1 the odd ones
        const int d = threadIdx.x & (ATT_D - 1), hf = threadIdx.x >> 7;
        const uint64_t* po = recs + 2 + d;
        float O = 0.f;
        for (int c = hf; c < ns; c += 16) {  // 8 splits per round, all requested together
            const int nj = min(8, (ns - c + 1) / 2);  // splits c, c + 2, ... below ns (slots past nj re-read the last)
            float v[8];
            if (!wait_flag32_n<8>(po + (size_t)c * ATT_REC, 2 * ATT_REC, tag, v, nj))
                __hip_atomic_fetch_or(counters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int j = 0; j < 8; ++j) O = j < nj ? fmaf(v[j], wsh[0][c + 2 * j], O) : O;
        }
        if (hf) oh[d] = O;
        __syncthreads();
        if (!hf) st_act<TO>(out + ((size_t)b * n_q + qh) * ATT_D + d, (O + oh[d]) / fmaxf(Lsh, 1e-20f));
    }
    if (r == 0 && threadIdx.x == 0)
        __hip_atomic_store(counters + 1 + (size_t)b * n_kv + kvh, (int)tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LSE combine for many splits (> 128): grid (n_q, B, 4 dim quarters), block
// 256 = 32 dims x 8 split groups.  Every block computes the split weights of
// its (head, sequence) (one split per thread, block max and sum); a thread
// then accumulates its dim over the splits g, g + 8, ... with 16 of them
// requested per round, the first round before the weights are known; the 8
// group sums meet in LDS.
#define CMBW_R 16
template <typename TO>
__global__ __launch_bounds__(256) void attn_combine_wide(const float* __restrict__ part_m,
                                                         const float* __restrict__ part_l,
                                                         const float* __restrict__ part_o, TO* __restrict__ out,
                                                         int n_q, const int* __restrict__ kv_offset, int split,
                                                         int max_splits) {
    __shared__ float w_sh[ATT_MAX_SPLITS];
    __shared__ float red[2][4];
    __shared__ float osum[8][33];
    const int qh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int dl = tid & 31, g = tid >> 5, d = blockIdx.z * 32 + dl;
    const int len = kv_offset[b] + 1;
    const int ns = (len + split - 1) / split;
    const size_t base = ((size_t)b * n_q + qh) * max_splits;
    const float* po = part_o + base * ATT_D + d;
    float ov[CMBW_R];
#pragma unroll
    for (int i = 0; i < CMBW_R; ++i) ov[i] = po[(size_t)min(g + 8 * i, ns - 1) * ATT_D];
    float mloc = -INFINITY;
    for (int c = tid; c < ns; c += 256) {
        const float m = part_m[base + c];
        w_sh[c] = m;
        mloc = fmaxf(mloc, m);
    }
    mloc = wave_max(mloc);
    if (lane == 0) red[0][wv] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float lloc = 0.f;
    for (int c = tid; c < ns; c += 256) {
        const float w = __expf(w_sh[c] - M);
        w_sh[c] = w;
        lloc = fmaf(part_l[base + c], w, lloc);
    }
    lloc = wave_sum(lloc);
    if (lane == 0) red[1][wv] = lloc;
    __syncthreads();
    const float L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    float O = 0.f;
#pragma unroll
    for (int i = 0; i < CMBW_R; ++i) {
        const int c = g + 8 * i;
        O = c < ns ? fmaf(ov[i], w_sh[min(c, ns - 1)], O) : O;
    }
    for (int c0 = 8 * CMBW_R; c0 < ns; c0 += 8 * CMBW_R) {
#pragma unroll
        for (int i = 0; i < CMBW_R; ++i) ov[i] = po[(size_t)min(c0 + g + 8 * i, ns - 1) * ATT_D];
#pragma unroll
        for (int i = 0; i < CMBW_R; ++i) {
            const int c = c0 + g + 8 * i;
            O = c < ns ? fmaf(ov[i], w_sh[min(c, ns - 1)], O) : O;
        }
    }
    osum[g][dl] = O;
    __syncthreads();
    if (g == 0) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) t += osum[j][dl];
        st_act<TO>(out + ((size_t)b * n_q + qh) * ATT_D + d, t / fmaxf(L, 1e-20f));
    }
}

// ---------------------------------------------------------------------------
// Reference-ABI split-KV kernels (hipModuleGetFunction drop-in).
// Chunk size is a compile-time constant as in the reference template
// (flash_attention_split_kv_partial.hip.template:29).
// ---------------------------------------------------------------------------
#ifndef SPLIT_KV_CHUNK_SIZE
#define SPLIT_KV_CHUNK_SIZE 32
#endif

// grid (batch, n_q, max_chunks), block (head_dim <= 256); one lane per dim,
// scores reduced with a wave butterfly plus a 4-entry LDS exchange.
extern "C" __global__ __launch_bounds__(256) void flash_attention_split_kv_partial_kernel(
    const __half* __restrict__ q, const __half* __restrict__ k_cache, const __half* __restrict__ v_cache,
    float* __restrict__ partial_m, float* __restrict__ partial_l, float* __restrict__ partial_o,
    int num_q_heads, int num_kv_heads, int head_dim, float scale, const int* __restrict__ kv_cache_offset_ptr,
    int kv_batch_stride, int max_chunks) {
    __shared__ float red[4];
    const int b = blockIdx.x, qh = blockIdx.y, chunk = blockIdx.z, tid = threadIdx.x;
    const int total = kv_cache_offset_ptr[b] + 1;
    const int st = (b * num_q_heads + qh) * max_chunks + chunk;
    const int start = chunk * SPLIT_KV_CHUNK_SIZE;
    if (start >= total) {
        if (tid == 0) { partial_m[st] = -1e30f; partial_l[st] = 0.f; }
        if (tid < head_dim) partial_o[(size_t)st * head_dim + tid] = 0.f;
        return;
    }
    const int end = min(start + SPLIT_KV_CHUNK_SIZE, total);
    const int kvh = qh / (num_q_heads / num_kv_heads);
    const bool act = tid < head_dim;
    const float qv = act ? __half2float(q[((size_t)b * num_q_heads + qh) * head_dim + tid]) : 0.f;
    const __half* kc = k_cache + (size_t)b * kv_batch_stride;
    const __half* vc = v_cache + (size_t)b * kv_batch_stride;
    const int nw = (blockDim.x + 63) >> 6;
    float m = -1e30f, l = 0.f, o = 0.f;
    for (int j = start; j < end; ++j) {
        const size_t base = ((size_t)j * num_kv_heads + kvh) * head_dim;
        float part = act ? qv * __half2float(kc[base + tid]) : 0.f;
        part = wave_sum(part);
        if ((tid & 63) == 0) red[tid >> 6] = part;
        __syncthreads();
        float s = 0.f;
        for (int w = 0; w < nw; ++w) s += red[w];
        __syncthreads();
        s *= scale;
        const float mn = fmaxf(m, s);
        const float c = __expf(m - mn);
        const float p = __expf(s - mn);
        l = l * c + p;
        o = o * c + p * (act ? __half2float(vc[base + tid]) : 0.f);
        m = mn;
    }
    if (tid == 0) { partial_m[st] = m; partial_l[st] = l; }
    if (act) partial_o[(size_t)st * head_dim + tid] = o;
}

// grid (batch, n_q), block (head_dim); dynamic LDS unused (kept for ABI parity).
extern "C" __global__ __launch_bounds__(256) void flash_attention_split_kv_reduce_kernel(
    const float* __restrict__ partial_m, const float* __restrict__ partial_l,
    const float* __restrict__ partial_o, __half* __restrict__ output, int num_q_heads, int head_dim,
    int max_chunks) {
    const int b = blockIdx.x, qh = blockIdx.y, tid = threadIdx.x;
    const int base = (b * num_q_heads + qh) * max_chunks;
    float M = -1e30f;
    for (int c = 0; c < max_chunks; ++c) M = fmaxf(M, partial_m[base + c]);
    float L = 0.f, O = 0.f;
    for (int c = 0; c < max_chunks; ++c) {
        const float w = __expf(partial_m[base + c] - M);
        L += partial_l[base + c] * w;
        if (tid < head_dim) O += partial_o[((size_t)base + c) * head_dim + tid] * w;
    }
    if (tid < head_dim) output[((size_t)b * num_q_heads + qh) * head_dim + tid] = __float2half(O / fmaxf(L, 1e-20f));
}

// LSE combine for max_splits <= 128 in one memory round trip: every load
// (length, split statistics, partial outputs of all max_splits splits) is
// issued before any result is needed; splits at or past the sequence's
// split count are masked by selects, so stale scratch cannot leak in.  Each
// wave reduces the split statistics on its own (lane c holds splits c and
// c + 64), so there is no barrier.  grid (n_q, B), block 128 (one thread per dim).
template <typename TO, int NSMAX>
__global__ __launch_bounds__(128) void attn_combine_small(const float* __restrict__ part_m,
                                                          const float* __restrict__ part_l,
                                                          const float* __restrict__ part_o, TO* __restrict__ out,
                                                          int n_q, const int* __restrict__ kv_offset, int split,
                                                          int max_splits) {
    constexpr int PL = NSMAX > 64 ? 2 : 1;  // splits per lane
    const int qh = blockIdx.x, b = blockIdx.y, d = threadIdx.x, lane = d & 63;
    const size_t base = ((size_t)b * n_q + qh) * max_splits;
    const int len_raw = kv_offset[b];
    float m_l[PL], l_l[PL];
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        const int cl = min(lane + 64 * j, max_splits - 1);
        m_l[j] = part_m[base + cl];
        l_l[j] = part_l[base + cl];
    }
    const float* po = part_o + base * ATT_D + d;
    float o[NSMAX];
#pragma unroll
    for (int c = 0; c < NSMAX; ++c) o[c] = po[(size_t)min(c, max_splits - 1) * ATT_D];
    const int ns = (len_raw + 1 + split - 1) / split;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        m_l[j] = lane + 64 * j < ns ? m_l[j] : -INFINITY;
        mx = fmaxf(mx, m_l[j]);
    }
    const float M = wave_max(mx);
    float w[PL], ls = 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
        w[j] = lane + 64 * j < ns ? __expf(m_l[j] - M) : 0.f;
        ls += lane + 64 * j < ns ? l_l[j] * w[j] : 0.f;
    }
    const float L = wave_sum(ls);
    float O = 0.f;
#pragma unroll
    for (int c = 0; c < NSMAX; ++c) {
        const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[c >> 6]), c & 63));
        O = c < ns ? fmaf(o[c], wc, O) : O;
    }
    st_act<TO>(out + ((size_t)b * n_q + qh) * ATT_D + d, O / fmaxf(L, 1e-20f));
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace vte {

// true when the environment variable is set to 0 (switches a launch form off)
static bool getenv_off_att(const char* name) {
    const char* v = getenv(name);
    return v != nullptr && atoi(v) == 0;
}

template <typename TQ, typename TO>
hipError_t attn_split_kv(const void* q, const void* k_cache, const void* v_cache, float* part_m, float* part_l,
                         float* part_o, void* out, int B, int n_q, int n_kv, float scale, const int* kv_offset,
                         int kv_batch_stride, int split, int max_splits, int* counters, hipStream_t st) {
    dim3 g1(max_splits, n_kv, B), b1(256);
    // positions every split may read ahead of knowing the length: all of
    // max_splits * split must lie inside one sequence's kv_batch_stride
    const long long rows_cap = kv_batch_stride / ((long long)n_kv * ATT_D);
    const bool spec = (long long)max_splits * split <= rows_cap;
#define ATT_LAUNCH_Q(SP, TP, QC)                                                                               \
    hipLaunchKernelGGL((attn_partial_gqa<TQ, TO, SP, TP, QC>), g1, b1, 0, st, (const TQ*)q, (const __half*)k_cache, \
                       (const __half*)v_cache, part_m, part_l, part_o, n_q, n_kv, scale, kv_offset, kv_batch_stride, \
                       split, max_splits, counters, (TO*)out, B)
#define ATT_LAUNCH_P(SP, TP) ATT_LAUNCH_Q(SP, TP, 1)
    const bool two = split >= 2 * ATT_WAVES * ATT_TILE;  // two tiles per wave loaded together
    const int G = n_q / n_kv;
    if (kv_batch_stride == 0 && B > 1 && counters == nullptr && split != ATT_TILE && 2 * G <= 16 &&
        !getenv_off_att("VTE_ATT_QC")) {
        // every column reads one cache (prompt tokens of one sequence): two
        // query columns per block share each K/V tile
        g1.z = (B + 1) / 2;
        if (two) ATT_LAUNCH_Q(false, 2, 2);
        else ATT_LAUNCH_Q(false, 1, 2);
    } else if (split == ATT_TILE) {  // one split per wave: a block takes four consecutive splits
        g1.x = (max_splits + ATT_WAVES - 1) / ATT_WAVES;
        if (spec) ATT_LAUNCH_P(true, 0);
        else ATT_LAUNCH_P(false, 0);
    } else if (spec) {
        if (two) ATT_LAUNCH_P(true, 2);
        else ATT_LAUNCH_P(true, 1);
    } else {
        if (two) ATT_LAUNCH_P(false, 2);
        else ATT_LAUNCH_P(false, 1);
    }
#undef ATT_LAUNCH_P
#undef ATT_LAUNCH_Q
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || counters != nullptr || out == nullptr) return e;  // out == nullptr: partials only
    dim3 g2(n_q, B), b2(ATT_D);
    if (max_splits <= 16)
        hipLaunchKernelGGL((attn_combine_small<TO, 16>), g2, b2, 0, st, part_m, part_l, part_o, (TO*)out, n_q,
                           kv_offset, split, max_splits);
    else if (max_splits <= 32)
        hipLaunchKernelGGL((attn_combine_small<TO, 32>), g2, b2, 0, st, part_m, part_l, part_o, (TO*)out, n_q,
                           kv_offset, split, max_splits);
    else if (max_splits <= 64)
        hipLaunchKernelGGL((attn_combine_small<TO, 64>), g2, b2, 0, st, part_m, part_l, part_o, (TO*)out, n_q,
                           kv_offset, split, max_splits);
    else if (max_splits <= 128)
        hipLaunchKernelGGL((attn_combine_small<TO, 128>), g2, b2, 0, st, part_m, part_l, part_o, (TO*)out, n_q,
                           kv_offset, split, max_splits);
    else
        hipLaunchKernelGGL((attn_combine_wide<TO>), dim3(n_q, B, ATT_D / 32), dim3(256), 0, st, part_m, part_l, part_o,
                           (TO*)out, n_q, kv_offset, split, max_splits);
    return hipGetLastError();
}

template hipError_t attn_split_kv<float, float>(const void*, const void*, const void*, float*, float*, float*,
                                                void*, int, int, int, float, const int*, int, int, int, int*,
                                                hipStream_t);
template hipError_t attn_split_kv<__half, __half>(const void*, const void*, const void*, float*, float*, float*,
                                                  void*, int, int, int, float, const int*, int, int, int, int*,
                                                  hipStream_t);

hipError_t kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int B, int n_kv, int head_dim,
                     const int* kv_offset, int kv_batch_stride, hipStream_t st) {
    hipLaunchKernelGGL(kv_cache_append_kernel, dim3(B, n_kv), dim3(head_dim), 0, st, (const __half*)k,
                       (const __half*)v, (__half*)k_cache, (__half*)v_cache, n_kv, head_dim, kv_offset,
                       kv_batch_stride);
    return hipGetLastError();
}

}  // namespace vte

