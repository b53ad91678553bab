// fp32-activation instantiations of the fused quantised mat-vec (the
// standalone GEMV configs take fp32 x); compiled apart from the fp16 ones so
// the two halves build in parallel.
#include "fused_kernels.h"

namespace vte {

template <int NC>
static void launch_nc(int upt, int total, size_t lds, hipStream_t st, const void* x, const FmvPlan& plan) {
    if (plan.K == 1536) fmv_launch_k<NC, true, 1536, true>(upt, total, lds, st, x, plan);
    else if (plan.K == 8960) fmv_launch_k<NC, true, 8960, false>(upt, total, lds, st, x, plan);
    else if (fmv_ro(plan.K)) fmv_launch_k<NC, true, 0, true>(upt, total, lds, st, x, plan);
    else fmv_launch_k<NC, true, 0, false>(upt, total, lds, st, x, plan);
}

void fmv_launch_x32(int NC, int upt, int total, size_t lds, hipStream_t st, const void* x, const FmvPlan& plan) {
    if (NC == 1) launch_nc<1>(upt, total, lds, st, x, plan);
    else if (NC == 2) launch_nc<2>(upt, total, lds, st, x, plan);
    else launch_nc<4>(upt, total, lds, st, x, plan);
}

}  // namespace vte
