// Weight dequantisation into MFMA A operands (Q4_K / Q6_K super-blocks to
// fp16) and the k-slot map shared by the batched MFMA kernels, gfx950.
//
//  * v_mfma_f32_16x16x32_f16: M = 16 weight rows, N = 16 batch columns, K = 32.
//  * Weights are dequantised in registers to fp16 with packed fp16 math
//    (nibble -> 0x64xx magic -> exact subtract -> v_pk_fma_f16), so only the
//    final weight carries an fp16 rounding; activations go to fp16; the MFMA
//    accumulates in fp32.
//  * K-slot permutation: MFMA pairs A and B by (lane group, slot), so any
//    bijection of super-block elements to (k-step, group, slot) is valid as
//    long as A and B use the same one.  The map is chosen so each lane's 8
//    slots are 8 contiguous elements sharing one sub-block scale:
//      Q4_K step t, group g: qs chunk c = g + 4*(t>>2), nibble (t>>1)&1, half t&1
//      Q6_K step t, group g: half h = t>>2, quarter q = t&3, l = 8g .. 8g+7
#pragma once
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
#define Q6_SLOT 224  // LDS bytes per staged Q6_K block row (14 aligned chunks)

// bytes b0..b3 of `u` (each < 256, here 6-bit values) -> two fp16 pairs 1024+b.
__device__ __forceinline__ void bytes_to_f16magic(uint32_t u, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// 8 nibble/6-bit values in the bytes of (u0, u1) -> 8 fp16 weights (q - bias) * d - m.
__device__ __forceinline__ half8_t deq8(uint32_t u0, uint32_t u1, _Float16 sub, half2_t d2, half2_t m2) {
    H8 r;
    bytes_to_f16magic(u0, r.u[0], r.u[1]);
    bytes_to_f16magic(u1, r.u[2], r.u[3]);
    const half2_t off = {(_Float16)(1024.0f) + sub, (_Float16)(1024.0f) + sub};
#pragma unroll
    for (int i = 0; i < 4; ++i) r.h2[i] = (r.h2[i] - off) * d2 - m2;
    return r.v;
}

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
        return 128 * (t >> 2) + 32 * (t & 3) + 8 * g;
    }
}

