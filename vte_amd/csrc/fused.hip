// Host side of the fused quantised mat-vec (batch 1..4): plan completion,
// tile geometry, launch selection and the C++ entry points used by capi.hip.
// The kernels are in fused_kernels.h; fp32-activation instantiations are
// compiled in fused_f32.hip.
#include "fused_kernels.h"

namespace vte {

static size_t fmv_max_lds() {
    static size_t n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        n = (size_t)v;
    }
    return n;
}

static size_t fmv_lds_bytes(int NC, int K, int upt, int att_rows) {
    size_t o = ((size_t)NC * xpad_len(K) * 2 + 15) & ~(size_t)15;
    o += (size_t)NC * (K / 16) * 4;
    o = (o + 15) & ~(size_t)15;
    o += (size_t)NC * upt * ROWS_THREADS * 4;
    o += (size_t)att_rows * 4;
    return o;
}

// Rows per tile: as many as fill the block with one unit per thread (0 if a
// single row has more units than threads).  RoPE tiles take a power-of-two
// number of rows per half so tiles never straddle a head.
static int fmv_rows_per_tile(int mode, int K, int upt) {
    const int per_row = (K / QK_K) * 4;
    // range-owned tiles: 256 / per_row row groups of upt rows
    const int R = fmv_ro(K) ? (ROWS_THREADS / per_row) * upt : upt * ROWS_THREADS / per_row;
    if (R < 1) return 0;
    if (mode == FMV_SWIGLU) return R >= 2 ? std::min(R & ~1, TMV_MAX_R) : 0;
    if (mode == FMV_ROPE_Q || mode == FMV_ROPE_KCACHE) {
        int h = 1;
        while (4 * h <= R && 2 * h <= 64) h *= 2;
        return R >= 2 ? 2 * h : 0;
    }
    return std::min(R, TMV_MAX_R);
}

// Compile-time K for the shapes of the 1.5B decode step (hidden 1536, FFN
// 8960); any other K takes the runtime-K kernels.
template <int NC>
static void fmv_launch_x16(int upt, int total, size_t lds, hipStream_t st, const void* x, const FmvPlan& plan) {
    if (plan.K == 1536) fmv_launch_k<NC, false, 1536, true>(upt, total, lds, st, x, plan);
    else if (plan.K == 8960) fmv_launch_k<NC, false, 8960, false>(upt, total, lds, st, x, plan);
    else if (fmv_ro(plan.K)) fmv_launch_k<NC, false, 0, true>(upt, total, lds, st, x, plan);
    else fmv_launch_k<NC, false, 0, false>(upt, total, lds, st, x, plan);
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

static int fmv_num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    }
    return n;
}

// Fills in a plan's per-segment geometry for `upt` units per thread.
// Returns hipSuccess, hipErrorNotSupported (the shape does not fit this upt)
// or hipErrorInvalidValue.
static hipError_t fmv_complete(const FmvPlan& plan, int upt, FmvPlan& P) {
    const int n_sb = plan.K / QK_K;
    P = plan;
    int total = 0;
    for (int s = 0; s < P.nseg; ++s) {
        FmvSeg& S = P.seg[s];
        if (S.fmt != 4 && S.fmt != 6 && S.fmt != 8) return hipErrorInvalidValue;
        if (fmv_paired(S.mode) && S.fmt != 4) return hipErrorInvalidValue;
        if (S.fmt == 8 && P.att_o != nullptr) return hipErrorNotSupported;
        S.row_bytes = S.fmt == 8 ? (P.K / QK8_0) * Q80_BYTES : n_sb * (S.fmt == 4 ? Q4K_BYTES : Q6K_BYTES);
        S.R = fmv_rows_per_tile(S.mode, P.K, upt);
        if (S.R <= 0 || P.M * S.R > ROWS_THREADS) return hipErrorNotSupported;
        if (S.mode == FMV_SWIGLU) {
            S.tiles = (S.n_rows + S.R / 2 - 1) / (S.R / 2);
        } else if (S.mode == FMV_ROPE_Q || S.mode == FMV_ROPE_KCACHE) {
            if (S.n_rows % 128 != 0) return hipErrorInvalidValue;
            S.tiles = S.n_rows / S.R;
        } else {
            S.tiles = (S.n_rows + S.R - 1) / S.R;
        }
        total += S.tiles;
    }
    P.total = total;
    return hipSuccess;
}

// Completes the plan (units per thread, rows per tile, tile counts) and
// launches one block per tile.  Units per thread (1, 2 or 4) are as many as
// keep at least two tiles per CU: larger tiles spread the per-block prologue
// (activation staging, RMSNorm) over more weights.
hipError_t fused_mv(const void* x, FmvPlan plan, hipStream_t st) {
    if (plan.M < 1 || plan.M > 4 || plan.nseg < 1 || plan.nseg > TMV_MAX_SEG) return hipErrorNotSupported;
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (plan.K % QK_K) != 0) return hipErrorInvalidValue;
    if (plan.norm_w != nullptr && (reinterpret_cast<uintptr_t>(plan.norm_w) & 15)) return hipErrorInvalidValue;
    const int NC = plan.M <= 1 ? 1 : (plan.M <= 2 ? 2 : 4);
    const int att_rows = plan.att_o != nullptr ? 2 * plan.M * plan.att_nq * plan.att_S : 0;
    static int upt_force = -1;  // VTE_FMV_UPT=1|2|4 pins units per thread (tuning)
    if (upt_force < 0) upt_force = env_int("VTE_FMV_UPT", 0);
    static int wfirst = -2;     // VTE_FMV_WFIRST=0|1 forces the weights-first form off / on (tuning)
    if (wfirst == -2) wfirst = env_int("VTE_FMV_WFIRST", -1);
    for (int upt : {4, 2, 1}) {
        if (upt_force > 0 && upt != upt_force) continue;
        FmvPlan P;
        const hipError_t e = fmv_complete(plan, upt, P);
        if (e == hipErrorInvalidValue) return e;
        if (e != hipSuccess) continue;
        if (upt_force <= 0 && upt > 1 && P.total < 2 * fmv_num_cus()) continue;
        const size_t lds = fmv_lds_bytes(NC, P.K, upt, att_rows);
        if (lds + 64 > fmv_max_lds()) continue;
        // weights first when the launch has many rounds of tiles (measured: Q6_K
        // LM head 151936 x 1536 46.7 -> 41.6 us; the decode step's launches of
        // at most a few tiles per CU are faster with the activations first)
        P.wfirst = wfirst >= 0 ? wfirst : (P.total >= 8 * fmv_num_cus() ? 1 : 0);
        for (int s = 0; s < P.nseg; ++s)
            if (P.seg[s].fmt == 8) P.wfirst = 0;  // the weights-first form has no Q8_0 instantiation
        if (P.x_f32) {
            fmv_launch_x32(NC, upt, P.total, lds, st, x, P);
        } else {
            if (NC == 1) fmv_launch_x16<1>(upt, P.total, lds, st, x, P);
            else if (NC == 2) fmv_launch_x16<2>(upt, P.total, lds, st, x, P);
            else fmv_launch_x16<4>(upt, P.total, lds, st, x, P);
        }
        return hipGetLastError();
    }
    return hipErrorNotSupported;
}

static FmvPlan plan_base(int M, int K, const void* norm_w, float eps) {
    FmvPlan P;
    memset(&P, 0, sizeof(P));
    P.M = M;
    P.K = K;
    P.norm_w = (const __half*)norm_w;
    P.eps = eps;
    P.rs = 1.0f;
    return P;
}

static FmvSeg seg(const void* w, const void* w2, void* out, const void* bias, const void* residual, int fmt,
                  int n_rows, int mode) {
    FmvSeg S;
    memset(&S, 0, sizeof(S));
    S.w = (const uint8_t*)w;
    S.w2 = (const uint8_t*)w2;
    S.out = out;
    S.bias = bias;
    S.residual = residual;
    S.fmt = fmt;
    S.n_rows = n_rows;
    S.mode = mode;
    return S;
}

hipError_t attn_in(const void* x, const void* norm_w, float eps, const void* wq, const void* q_bias, int fmt_q,
                   const void* wk, const void* k_bias, int fmt_k, const void* wv, const void* v_bias, int fmt_v,
                   void* q_out, void* k_cache, void* v_cache, const int* kv_offset, int kv_batch_stride,
                   const void* rope_cos, const void* rope_sin, int M, int K, int n_q, int n_kv, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.seg[0] = seg(wq, nullptr, q_out, q_bias, nullptr, fmt_q, n_q * 128, FMV_ROPE_Q);
    P.seg[1] = seg(wk, nullptr, nullptr, k_bias, nullptr, fmt_k, n_kv * 128, FMV_ROPE_KCACHE);
    P.seg[2] = seg(wv, nullptr, nullptr, v_bias, nullptr, fmt_v, n_kv * 128, FMV_VCACHE);
    P.nseg = 3;
    P.rope_cos = (const __half*)rope_cos;
    P.rope_sin = (const __half*)rope_sin;
    P.kv_offset = kv_offset;
    P.k_cache = (__half*)k_cache;
    P.v_cache = (__half*)v_cache;
    P.kv_batch_stride = kv_batch_stride;
    P.n_kv = n_kv;
    return fused_mv(x, P, st);
}

hipError_t ffn_in(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up, int fmt,
                  void* out, int M, int K, int ffn, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.seg[0] = seg(w_gate, w_up, out, nullptr, nullptr, fmt, ffn, FMV_SWIGLU);
    P.nseg = 1;
    return fused_mv(x, P, st);
}

hipError_t norm_mv(const void* x, const void* norm_w, float eps, const void* w, int fmt, void* out, bool out_f32,
                   const void* bias, const void* residual, float rs, int M, int K, int N, hipStream_t st) {
    FmvPlan P = plan_base(M, K, norm_w, eps);
    P.rs = rs;
    P.seg[0] = seg(w, nullptr, out, bias, residual, fmt, N, out_f32 ? FMV_STORE_F32 : FMV_STORE_F16);
    P.nseg = 1;
    return fused_mv(x, P, st);
}

// y = W · combine(split-KV partials) + residual for batch 1..4 (fp16 output):
// the attention output projection with the log-sum-exp combine in its
// prologue.  hipErrorNotSupported when there are more than TMV_ATT_MAX_S splits.
hipError_t attn_out_mv(const float* part_m, const float* part_l, const float* part_o, const int* kv_offset, int M,
                       int n_q, int max_splits, int split, const void* w, int fmt, void* out, const void* residual,
                       float rs, int N, hipStream_t st) {
    if (max_splits > TMV_ATT_MAX_S || split < 1) return hipErrorNotSupported;
    FmvPlan P = plan_base(M, n_q * 128, nullptr, 0.f);
    P.rs = rs;
    P.kv_offset = kv_offset;
    P.att_m = part_m;
    P.att_l = part_l;
    P.att_o = part_o;
    P.att_nq = n_q;
    P.att_S = max_splits;
    P.att_split = split;
    P.seg[0] = seg(w, nullptr, out, nullptr, residual, fmt, N, FMV_STORE_F16);
    P.nseg = 1;
    return fused_mv(part_o, P, st);
}

// Plain y = (W x + bias) * rs + residual for batch 1..4 (no norm); x fp32 or
// fp16, y / bias / residual in the output type.  hipErrorNotSupported (nothing
// launched) when the shape does not fit: rows longer than 256 units (K > 16384).
hipError_t stream_mv(int fmt, bool in_f32, bool out_f32, const void* x, const void* w, void* y, int M, int K, int N,
                     const void* bias, const void* residual, float rs, hipStream_t st) {
    if (fmt != 4 && fmt != 6 && fmt != 8) return hipErrorNotSupported;
    if (M > 4 || K % QK_K != 0) return hipErrorNotSupported;
    FmvPlan P = plan_base(M, K, nullptr, 0.f);
    P.x_f32 = in_f32 ? 1 : 0;
    P.rs = rs;
    P.seg[0] = seg(w, nullptr, y, bias, residual, fmt, N, out_f32 ? FMV_STORE_F32 : FMV_STORE_F16);
    P.nseg = 1;
    return fused_mv(x, P, st);
}

}  // namespace vte

