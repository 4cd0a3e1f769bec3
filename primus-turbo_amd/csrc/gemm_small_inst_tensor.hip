// Instantiations of the small-problem FP8 GEMM for one scaling mode.
#include "gemm_small.h"

namespace pta {
namespace gemm_small {
int dispatch_small_tensor(const SmallArgs &g, bool akm, bool bkm, int fa, int fb, int out_dt, hipStream_t st) {
    return small_layouts<SM_TENSOR>(g, akm, bkm, fa, fb, out_dt, st);
}
} // namespace gemm_small
} // namespace pta
