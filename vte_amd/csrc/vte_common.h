// Shared device helpers for the gfx950 (CDNA4, wave64) decode-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define VTE_WAVE 64

// GGUF block geometry (bytes per block / elements per block).
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define Q80_BYTES 34
#define QK_K 256
#define QK8_0 32

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }
__device__ __forceinline__ float h2f_bits(uint32_t bits16) {
    __half_raw r;
    r.x = (unsigned short)(bits16 & 0xFFFFu);
    return __half2float(__half(r));
}

// 16-byte weight load.  The pointer is cast to the global address space so the load is a
// global_load (vector-memory counter only) even when the address went
// through integer arithmetic; a flat load would also count against the LDS
// counter and force waits on unrelated LDS accesses.
typedef unsigned int vte_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const vte_u32x4 vte_g_u32x4;
// Plain (temporal) loads: measured faster than non-temporal ones for the
// quantised weight streams (Q4_K 8960x1536 GEMV 5.5 -> 5.2 us, Q6_K LM head
// 45 -> 43 us; non-temporal Q6_K loads 63 us).
__device__ __forceinline__ uint4 ldg_g16(const void* p) {
    const vte_u32x4 v = *((vte_g_u32x4*)(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Activation loads: the same kernels serve fp16 (reference ABI) and fp32
// (benchmark configs) activations.
template <typename T> __device__ __forceinline__ float ld_act(const T* p);
template <> __device__ __forceinline__ float ld_act<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld_act<__half>(const __half* p) { return __half2float(*p); }

template <typename T> __device__ __forceinline__ void st_act(T* p, float v);
template <> __device__ __forceinline__ void st_act<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void st_act<__half>(__half* p, float v) { *p = __float2half(v); }

// Load 16 consecutive activations starting at p (16-element aligned).
template <typename T> __device__ __forceinline__ void ld_act16(const T* p, float (&v)[16]);
template <> __device__ __forceinline__ void ld_act16<float>(const float* p, float (&v)[16]) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 t = q[i];
        v[4 * i + 0] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}
template <> __device__ __forceinline__ void ld_act16<__half>(const __half* p, float (&v)[16]) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint4 t = q[i];
        uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[8 * i + 2 * j + 0] = h2f_bits(w[j]);
            v[8 * i + 2 * j + 1] = h2f_bits(w[j] >> 16);
        }
    }
}

// Full-wave reductions (all 64 lanes active); every lane receives the result.
// Within each row of 16 lanes: DPP quad permutes [1,0,3,2] and [2,3,0,1],
// then row_half_mirror and row_mirror (each pairs a lane with one in the
// other half); the four row results are read into scalars.  No LDS traffic.
#define VTE_DPP_F(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, false))
__device__ __forceinline__ float wave_rows4(float v, int r) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += VTE_DPP_F(v, 0xB1);
    v += VTE_DPP_F(v, 0x4E);
    v += VTE_DPP_F(v, 0x141);
    v += VTE_DPP_F(v, 0x140);
    return (wave_rows4(v, 0) + wave_rows4(v, 1)) + (wave_rows4(v, 2) + wave_rows4(v, 3));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, VTE_DPP_F(v, 0xB1));
    v = fmaxf(v, VTE_DPP_F(v, 0x4E));
    v = fmaxf(v, VTE_DPP_F(v, 0x141));
    v = fmaxf(v, VTE_DPP_F(v, 0x140));
    return fmaxf(fmaxf(wave_rows4(v, 0), wave_rows4(v, 1)), fmaxf(wave_rows4(v, 2), wave_rows4(v, 3)));
}

// GEMV epilogue shared by every format, same order as the reference:
// ((acc + bias[row]) * residual_scale) + residual[m,row]; bias and residual
// share the output type (fp16 in the reference ABI).
template <typename TO>
__device__ __forceinline__ void gemv_store(TO* out, const TO* bias, const TO* residual, float rs,
                                           int row, int m, int n_rows, float acc) {
    if (bias) acc += ld_act<TO>(bias + row);
    acc *= rs;
    size_t o = (size_t)m * n_rows + row;
    if (residual) acc += ld_act<TO>(residual + o);
    st_act<TO>(out + o, acc);
}
