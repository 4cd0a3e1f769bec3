// Instantiations of the FP8 GEMM kernel for one scaling mode.
#include "gemm_kernel.h"

namespace pta {
namespace gemm_detail {
int dispatch_row(const GemmArgs &g, int fa, int fb, int out_dt, hipStream_t st) {
    return dispatch_fmt<SM_ROW, false, false>(g, fa, fb, out_dt, st);
}
} // namespace gemm_detail
} // namespace pta
