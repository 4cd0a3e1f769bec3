// Streaming probe for bench.py, built into its own library
// (libpta_stream_probe.so, not the product library): the memory ceiling the
// quantize kernels are measured against.  A quantizer reads each input byte
// once and writes each output byte once, so its bound is what a plain stream
// of the same pattern reaches: "copy" (read and write equal bytes, as the
// dual / segment / MX kernels do) or "read 2, write 1" (a bf16 -> fp8 cast:
// the 128x128 weight and rowwise kernels).  The kernel has no arithmetic
// beyond folding the loaded words into the stored ones: 16-byte loads and
// stores per lane, two positions' loads in flight before their stores, one
// position pair per lane (the grid covers the data; measured against 4 and 8
// positions in flight and grids capped at 1024-8192 workgroups: this form was
// the fastest or within 2% at 34 MB - 960 MB), optionally non-temporal.
//
// C ABI (no counterpart in the reference):
//   int pta_bench_stream_probe(const void *src, void *dst, int64_t write_bytes,
//                              int read_ratio, int nontemporal, hipStream_t);
// streams write_bytes (a multiple of 16) into dst while reading
// read_ratio * write_bytes from src (1: a copy; 2: two 16-byte loads folded
// by XOR into each 16-byte store).  Returns 0, 1 for bad arguments or 2 when
// the launch fails.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
using v4u = unsigned int __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ v4u ld16(const v4u *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ __forceinline__ void st16(v4u *p, v4u v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

constexpr int SP_THREADS = 256;
constexpr int SP_UNROLL  = 2;

// dst[i] = fold of src[RATIO i .. RATIO i + RATIO - 1], i < n16
template <int RATIO, bool NT>
__global__ __launch_bounds__(SP_THREADS) void stream_probe_kernel(const v4u *src, v4u *dst, int64_t n16) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * SP_THREADS;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * SP_THREADS + threadIdx.x; base < n16;
         base += SP_UNROLL * stride) {
        v4u v[SP_UNROLL][RATIO];
#pragma unroll
        for (int u = 0; u < SP_UNROLL; ++u) {
            const int64_t i = base + u * stride;
            if (i < n16) {
#pragma unroll
                for (int r = 0; r < RATIO; ++r) v[u][r] = ld16<NT>(src + i * RATIO + r);
            }
        }
#pragma unroll
        for (int u = 0; u < SP_UNROLL; ++u) {
            const int64_t i = base + u * stride;
            if (i < n16) {
                v4u w = v[u][0];
#pragma unroll
                for (int r = 1; r < RATIO; ++r) w ^= v[u][r];
                st16<NT>(dst + i, w);
            }
        }
    }
}

template <int RATIO, bool NT>
int probe_launch(const void *src, void *dst, int64_t n16, hipStream_t st) {
    // one pass: every lane owns SP_UNROLL positions (the loop covers sizes
    // beyond a 2^31-workgroup grid)
    const int64_t  per  = int64_t(SP_THREADS) * SP_UNROLL;
    const int64_t  want = (n16 + per - 1) / per;
    const uint32_t grid = static_cast<uint32_t>(want < (int64_t(1) << 30) ? want : (int64_t(1) << 30));
    stream_probe_kernel<RATIO, NT><<<grid, SP_THREADS, 0, st>>>(static_cast<const v4u *>(src), static_cast<v4u *>(dst),
                                                               n16);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
} // namespace

extern "C" int pta_bench_stream_probe(const void *src, void *dst, int64_t write_bytes, int read_ratio,
                                      int nontemporal, hipStream_t st) {
    if (!src || !dst || write_bytes < 0 || write_bytes % 16 != 0) return 1;
    if ((read_ratio != 1 && read_ratio != 2) || !aligned16(src) || !aligned16(dst)) return 1;
    if (write_bytes == 0) return 0;
    const int64_t n16 = write_bytes / 16;
    if (read_ratio == 1)
        return nontemporal ? probe_launch<1, true>(src, dst, n16, st) : probe_launch<1, false>(src, dst, n16, st);
    return nontemporal ? probe_launch<2, true>(src, dst, n16, st) : probe_launch<2, false>(src, dst, n16, st);
}
