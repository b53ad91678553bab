// Single translation unit for the standalone code object (--genco): the
// reference-named extern "C" kernels of the GEMV, attention and glue sources
// (plus their fp32 GEMV siblings, the batched MFMA GEMM symbols and two
// measurement kernels of the benchmark),
// loadable with hipModuleLoad / hipModuleGetFunction.
#include "gemv.hip"
#include "attention.hip"
#include "glue.hip"
#include "gemm_mfma.hip"
#include "bench_kernels.hip"
