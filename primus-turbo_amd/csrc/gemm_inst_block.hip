// Instantiations of the FP8 GEMM kernel for blockwise scaling.
#include "gemm_kernel.h"

namespace pta {
namespace gemm_detail {
int dispatch_block(const GemmArgs &g, bool a2d, bool b2d, int fa, int fb, int out_dt, hipStream_t st) {
    if (!a2d && b2d) return dispatch_fmt<SM_BLOCK, false, true>(g, fa, fb, out_dt, st);
    if (!a2d && !b2d) return dispatch_fmt<SM_BLOCK, false, false>(g, fa, fb, out_dt, st);
    return dispatch_fmt<SM_BLOCK, true, false>(g, fa, fb, out_dt, st);
}
} // namespace gemm_detail
} // namespace pta
