// Measurement kernels of the per-launch GEMV bandwidth method
// (tools/bench_gemv_q4k_bandwidth.py:74-110, run_trial at :166-200): the
// dispatch floor is the event-bracketed time of an empty kernel, and the
// bandwidth a GEMV reaches is compared with a plain read of the same weight
// rows launched with the GEMV ABI's geometry (one 64-thread block per row).
// Only the benchmark loads them; no decode path calls them.
#include "vte_common.h"

extern "C" __global__ void vte_null_kernel() {}

// Block r reads row r (row_bytes bytes at src + r * row_bytes) in 16-byte
// loads, the row's dword tail in 4-byte loads, and writes one word derived
// from every loaded byte so no load is dropped.  Rows of Q6_K matrices
// (210-byte blocks) are only 4-byte aligned; the vector loads take any
// alignment.
extern "C" __global__ __launch_bounds__(64) void vte_read_rows_kernel(const void* src, void* dst, int row_bytes) {
    const uint8_t* row = reinterpret_cast<const uint8_t*>(src) + (size_t)blockIdx.x * row_bytes;
    const int nv = row_bytes >> 4, t = threadIdx.x;
    uint32_t acc = 0u;
    for (int i = t; i < nv; i += 64) {
        uint4 v;
        __builtin_memcpy(&v, row + 16 * (size_t)i, 16);
        acc += v.x ^ (v.y + v.z) ^ v.w;
    }
    for (int i = 16 * nv + 4 * t; i + 4 <= row_bytes; i += 256) {
        uint32_t w;
        __builtin_memcpy(&w, row + i, 4);
        acc += w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (t == 0) reinterpret_cast<uint32_t*>(dst)[blockIdx.x] = acc;
}
