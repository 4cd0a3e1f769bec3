// Instantiations of the small-problem FP8 GEMM for MX scaling (NT only).
#include "gemm_small.h"

namespace pta {
namespace gemm_small {
int dispatch_small_mx(const SmallArgs &g, int fa, int fb, int out_dt, hipStream_t st) {
    return small_fmt<SM_MX, false, false>(g, fa, fb, out_dt, st);
}
} // namespace gemm_small
} // namespace pta
