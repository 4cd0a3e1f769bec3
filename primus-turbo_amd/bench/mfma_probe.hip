// Matrix-pipe probe for bench.py, built into its own library
// (libpta_mfma_probe.so, not the product library): the compute ceiling the
// scaled GEMM kernels are measured against.  Each workgroup has the GEMM's
// shape of work (8 waves, two per SIMD, each wave a 64x128 block of C as 4x8
// tiles of v_mfma_f32_16x16x128_f8f6f4), but its operands stay in registers:
// no global or LDS traffic in the loop.  What the variants add per MFMA is
// what each scale granularity costs the GEMM's main loop:
//   0  MFMA only, accumulating in place (tensorwise / rowwise: scales go in
//      the epilogue);
//   1  MFMA into a fresh partial plus 4 FMAs, acc += p * s_row (blockwise
//      1x128 x 128x128: one scale per row and K block);
//   2  the same plus 4 multiplies, acc += p * (s_row * s_col) (blockwise
//      1x128 x 1x128, the wgrad's scales);
//   3  the scaled MFMA with per-lane E8M0 exponents (MX), accumulating in
//      place.
// Per wave and iteration: 32 MFMAs = 64 x 128 x 128 MACs.
//
// C ABI (no counterpart in the reference):
//   int pta_bench_mfma_probe(int variant, int iters, int workgroups,
//                            const void *operands, float *out, hipStream_t);
// operands: 4096 x 32 bytes of fp8 (e4m3) operand data; out: workgroups x 512
// floats (a fold of each lane's accumulators, so nothing is optimised away).
// Returns 0, 1 for bad arguments or 2 when the launch fails.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
typedef int   v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int MP_THREADS = 512;

template <int V>
__global__ __launch_bounds__(MP_THREADS) void mfma_probe_kernel(const int *ops, float *out, int iters) {
    const int  lane = threadIdx.x & 63;
    const int *src  = ops + (threadIdx.x % 4096) * 8;
    v8i        a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) a[i][e] = src[(i * 8 + e) % 32];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) b[j][e] = src[(j * 8 + e + 3) % 32];
    v4f acc[8][4];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};
    float sr[4], sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sr[i] = 1.0f + 0.001f * static_cast<float>(lane + i);
        sc[i] = 1.0f - 0.001f * static_cast<float>(lane + 2 * i);
    }
    const int ea = 127 + (lane & 1), eb = 127 - (lane & 1); // E8M0 exponents 2^0, 2^+-1
    v4f       p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p[u] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
        // opaque updates in place (no instructions): the row scales change per
        // iteration (K block), the column scales per B fragment, and every MFMA
        // gets operands the compiler cannot prove equal to another's
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(sr[i]));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            asm volatile("" : "+v"(b[j & 1]));
            if constexpr (V == 2) asm volatile("" : "+v"(sc[0]), "+v"(sc[1]), "+v"(sc[2]), "+v"(sc[3]));
            const v8i bf = b[j & 1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = j * 4 + i;
                if constexpr (V == 0) {
                    acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, a[i], acc[j][i], 0, 0, 0, 0, 0, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                } else if constexpr (V == 3) {
                    acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, a[i], acc[j][i], 0, 0, 0, eb, 0, ea);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                } else {
                    // fresh partial; the tile issued two MFMAs earlier is scaled
                    // behind it (the partial of the previous iteration's last
                    // two tiles wraps round)
                    p[tt & 3]   = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, a[i], v4f{0.f, 0.f, 0.f, 0.f},
                                                                                  0, 0, 0, 0, 0, 0);
                    const int q = (tt + 30) & 31, iq = q & 3;
                    if constexpr (V == 1) {
                        acc[q >> 2][iq] += p[q & 3] * sr[iq];
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[q >> 2][iq][r] += p[q & 3][r] * (sr[iq] * sc[r]);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                    }
                }
            }
        }
    }
    float res = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) res += acc[j][i][0] + acc[j][i][1] + acc[j][i][2] + acc[j][i][3];
#pragma unroll
    for (int u = 0; u < 4; ++u) res += p[u][0] + p[u][3];
    out[static_cast<int64_t>(blockIdx.x) * MP_THREADS + threadIdx.x] = res;
}
} // namespace

extern "C" int pta_bench_mfma_probe(int variant, int iters, int workgroups, const void *operands, float *out,
                                    hipStream_t stream) {
    if (variant < 0 || variant > 3 || iters < 1 || workgroups < 1 || operands == nullptr || out == nullptr) return 1;
    const int *ops = static_cast<const int *>(operands);
    switch (variant) {
    case 0: mfma_probe_kernel<0><<<workgroups, MP_THREADS, 0, stream>>>(ops, out, iters); break;
    case 1: mfma_probe_kernel<1><<<workgroups, MP_THREADS, 0, stream>>>(ops, out, iters); break;
    case 2: mfma_probe_kernel<2><<<workgroups, MP_THREADS, 0, stream>>>(ops, out, iters); break;
    default: mfma_probe_kernel<3><<<workgroups, MP_THREADS, 0, stream>>>(ops, out, iters); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
