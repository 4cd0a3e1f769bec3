// Tensorwise / rowwise / MXFP8 quantization, dequantization and byte
// transposes for gfx950.
//
// Scale arithmetic follows the reference's HIP kernels:
//   amax -> scale, eps 1e-12  csrc/include/primus_turbo/device/quant_utils.cuh:53-72
//   quant op                  csrc/include/primus_turbo/device/quant_utils.cuh:31-38
//   rowwise (row-major)       csrc/kernels/quantization/quantization_rowwise.cu:57-135
//   rowwise (other axis)      csrc/kernels/quantization/quantization_rowwise.cu:186-235
// The MX rule (kernel source absent from the reference snapshot) follows the
// constants of csrc/include/primus_turbo/quantization.h:85-102 and the
// reference's MX round-trip test (tests/pytorch/ops/test_quantization.py:
// 304-460), which rules out saturating block maxima:
//   E = floor(log2 amax) - emax_elem, plus 1 when amax * 2^-E > fp8_max,
//   e8m0 = clamp(E + 127, 0, 254), q = fp8(x * 2^(127 - e8m0)).
#include "common.h"

#include <mutex>

namespace pta {
namespace {

// Max of two partial maxima of |x|.  They start from +0, so they are +0 ..
// +inf, or NaN where the NaN-propagating max built them from a NaN input.
// Their bit patterns order as the values do and every NaN pattern lies above
// +inf's, so the integer max is exact and keeps a NaN; it needs none of the
// NaN-quieting the compiler puts in front of a float max of a lane-exchanged
// operand.
__device__ __forceinline__ float amax2(float a, float b) {
    return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}
__device__ __forceinline__ float amax_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return amax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float amax_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return amax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// |x| with a signalling NaN first quieted.  v_max / v_max3 of a signalling
// NaN return NaN, and the next NaN-dropping max then drops that NaN together
// with the running maximum it replaced; after the quieting every NaN is
// dropped, as the reference's fmaxf drops it.
__device__ __forceinline__ float absq(float x) { return fabsf(__builtin_canonicalizef(x)); }
// the same from an opaque copy of x: each pass forms its quieted values where
// it uses them, instead of the compiler holding one pass's 64 for the next
// (+56 VGPRs in the dual kernel, +7 in the MX kernel)
__device__ __forceinline__ float absq_fresh(float x) {
    asm volatile("" : "+v"(x));
    return fabsf(__builtin_canonicalizef(x));
}

// NaN-propagating max of |x| (v_maximum3_f32): NaN when an input is NaN,
// the NaN-dropping amax otherwise; special: +inf or NaN
__device__ __forceinline__ float pmax_abs(float a, float x) { return __builtin_elementwise_maximum(a, fabsf(x)); }
__device__ __forceinline__ bool  special_amax(float a) { return __float_as_uint(a) >= 0x7f800000u; }

// wave max of partial maxima of |x| (integer max, exact as for amax2)
__device__ __forceinline__ float amax_wave(float v) {
    v = amax2(v, dpp_f<PTA_DPP_QUAD_XOR1>(v));
    v = amax2(v, dpp_f<PTA_DPP_QUAD_XOR2>(v));
    v = amax2(v, dpp_f<PTA_DPP_ROW_HALF_MIRROR>(v));
    v = amax2(v, dpp_f<PTA_DPP_ROW_MIRROR>(v));
    return amax_xor32(amax_xor16(v));
}

// Cast of four values already scaled into range, without the clamp: used
// where no input is NaN or infinite, so that |x| <= amax and |x * scale| <=
// max (1 + 2^-23), whose round-to-nearest-even cast is the clamped cast's byte.
template <int FMT>
__device__ __forceinline__ uint32_t cast4(float a, float b, float c, float d) {
    uint32_t w;
    if constexpr (FMT == PTA_E4M3) {
        w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    } else {
        w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
    }
    return w;
}


constexpr int NT = 256;

// ---------------------------------------------------------------------------
// TENSORWISE
// ---------------------------------------------------------------------------
constexpr int TW_MAX_PARTS = 2048;

// pass 1: per-block partial amax (16 elements per lane per iteration)
template <int IN_DT, bool VEC>
__global__ __launch_bounds__(NT) void tw_amax_kernel(const void *x, int64_t n, float *partial) {
    float         a      = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * NT * 16;
    for (int64_t base = (static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x) * 16; base < n;
         base += stride) {
        if (VEC && base + 16 <= n) {
            float v[8], w[8];
            load8<IN_DT>(x, base, v);
            load8<IN_DT>(x, base + 8, w);
#pragma unroll
            for (int j = 0; j < 8; ++j) a = fmaxf(a, fmaxf(absq(v[j]), absq(w[j])));
        } else {
            for (int j = 0; j < 16; ++j)
                if (base + j < n) a = fmaxf(a, absq(load_scalar<IN_DT>(x, base + j)));
        }
    }
    a = max64(a);
    __shared__ float s[NT / 64];
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
}

// pass 2: every block reduces the partials (tiny, L2-resident), then quantizes
template <int IN_DT, int FMT, bool VEC>
__global__ __launch_bounds__(NT) void tw_quant_kernel(const void *x, int64_t n, const float *partial,
                                                       int nparts, const float *scale_in,
                                                       uint8_t *q, float *scale_inv) {
    __shared__ float s_scale;
    if (threadIdx.x < 64) {
        float sc;
        if (scale_in != nullptr) {
            sc = scale_in[0];
        } else {
            float a = 0.0f;
            for (int i = threadIdx.x; i < nparts; i += 64) a = fmaxf(a, partial[i]);
            a  = max64(a);
            sc = scale_from_amax<FMT>(a, 1e-12f);
        }
        if (threadIdx.x == 0) {
            s_scale = sc;
            if (blockIdx.x == 0) scale_inv[0] = 1.0f / sc;
        }
    }
    __syncthreads();
    const float   sc     = s_scale;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * NT * 16;
    for (int64_t base = (static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x) * 16; base < n;
         base += stride) {
        if (VEC && base + 16 <= n) {
            float v[16];
            float a[8], b[8];
            load8<IN_DT>(x, base, a);
            load8<IN_DT>(x, base + 8, b);
#pragma unroll
            for (int j = 0; j < 8; ++j) { v[j] = a[j]; v[j + 8] = b[j]; }
            *reinterpret_cast<uint4 *>(q + base) =
                make_uint4(quant4<FMT>(v, sc), quant4<FMT>(v + 4, sc), quant4<FMT>(v + 8, sc),
                           quant4<FMT>(v + 12, sc));
        } else {
            for (int j = 0; j < 16; ++j)
                if (base + j < n) q[base + j] = cvt1_fp8<FMT>(qclamp<FMT>(load_scalar<IN_DT>(x, base + j), sc));
        }
    }
}

int tw_grid(int64_t n) {
    int64_t g = cdiv(n, static_cast<int64_t>(NT) * 16 * 4);
    if (g < 1) g = 1;
    if (g > TW_MAX_PARTS) g = TW_MAX_PARTS;
    return static_cast<int>(g);
}

// One launch for tensors of up to TW_FUSED_MAX elements: each thread keeps its
// IT x 16 elements in registers, the workgroups publish their partial amax,
// wait until every workgroup has published, reduce all partials and cast from
// the registers: one read of x instead of two, one launch instead of two.
// Publication: partial[b], then, once that store has completed, tag[b] = this
// call's 64-bit tag, both device-coherent; thread i of every workgroup polls
// tag[i] with device-coherent loads and then reads partial[i] the same way.
// The tag is unique per call, so a workspace that holds an earlier call's tags
// needs no clearing, and calls on different streams use their own workspaces.
// At most TW_FUSED_GRID workgroups of 256 threads and little LDS (half the
// CUs of an MI355X at one workgroup each): on an otherwise idle GPU they are
// all resident together; concurrent work on other streams that holds the CUs
// for long can keep some of them from starting.  A poll that has not seen
// every tag after TW_SPIN_LIMIT rounds gives up: the call's scale becomes NaN
// and the call's tag goes into the status word at TW_STATUS_OFFSET of the
// workspace (pta_last_wait_status), so a failure shows instead of hanging.  A
// tag fixed at graph capture would repeat on every replay, so captured calls
// use the two-launch form.
constexpr int      TW_FUSED_GRID = 128; // workgroups at most (<= NT: one partial per thread;
                                        // 256 measured slower than the two-launch form)
constexpr int64_t  TW_FUSED_MAX  = int64_t(TW_FUSED_GRID) * NT * 16 * 4;
constexpr unsigned TW_SPIN_LIMIT = 1u << 22;
constexpr size_t   TW_TAG_OFFSET = TW_FUSED_GRID * sizeof(float); // tags after the partials
constexpr size_t   TW_STATUS_OFFSET = TW_TAG_OFFSET + TW_FUSED_GRID * sizeof(uint64_t); // then the status word
static_assert(TW_STATUS_OFFSET + sizeof(uint64_t) <= TW_MAX_PARTS * sizeof(float),
              "partials, tags and the status word fit the tensorwise workspace");

template <int IN_DT, int FMT, int IT>
__global__ __launch_bounds__(NT) void tw_fused_kernel(const void *x, int64_t n, uint8_t *q, float *scale_inv,
                                                      float *partial, uint64_t *tags, uint64_t tag,
                                                      uint64_t expect, unsigned spin_limit, uint64_t *status) {
    const int     tid    = static_cast<int>(threadIdx.x);
    const int     b      = static_cast<int>(blockIdx.x);
    const int     g      = static_cast<int>(gridDim.x);
    const int64_t stride = static_cast<int64_t>(g) * NT * 16;
    const int64_t base0  = (static_cast<int64_t>(b) * NT + tid) * 16;
    float         v[IT][16];
    float         a = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t base = base0 + it * stride;
        if (base + 16 <= n) {
            float lo[8], hi[8];
            load8<IN_DT>(x, base, lo);
            load8<IN_DT>(x, base + 8, hi);
#pragma unroll
            for (int j = 0; j < 8; ++j) { v[it][j] = lo[j]; v[it][j + 8] = hi[j]; }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[it][j] = base + j < n ? load_scalar<IN_DT>(x, base + j) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) a = fmaxf(a, absq(v[it][j]));
    }
    __shared__ float s[NT / 64];
    a = max64(a);
    if ((tid & 63) == 0) s[tid >> 6] = a;
    __syncthreads();
    if (tid == 0) {
        // device-coherent stores; the tag goes out once the partial's store
        // has completed (no release fence: that would write back all of L2)
        __hip_atomic_store(&partial[b], fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __hip_atomic_store(&tags[b], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float pa   = 0.0f;
    bool  seen = true;
    if (tid < g) {
        unsigned k = 0;
        // device-coherent polls; the partial is read (device-coherent) only
        // after its tag has been seen
        while (__hip_atomic_load(&tags[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != expect &&
               k < spin_limit) {
            ++k;
            __builtin_amdgcn_s_sleep(2);
        }
        asm volatile("" ::: "memory");
        seen = k < spin_limit;
        pa   = __hip_atomic_load(&partial[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool all_seen = __syncthreads_and(seen);
    if (!all_seen && tid == 0) __hip_atomic_store(status, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pa = max64(pa);
    if ((tid & 63) == 0) s[tid >> 6] = pa; // s[] free again: every read of it precedes __syncthreads_and
    __syncthreads();
    const float amax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    const float sc   = all_seen ? scale_from_amax<FMT>(amax, 1e-12f) : __builtin_nanf("");
    if (b == 0 && tid == 0) scale_inv[0] = 1.0f / sc;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t base = base0 + it * stride;
        if (base + 16 <= n) {
            *reinterpret_cast<uint4 *>(q + base) = make_uint4(quant4<FMT>(v[it], sc), quant4<FMT>(v[it] + 4, sc),
                                                              quant4<FMT>(v[it] + 8, sc), quant4<FMT>(v[it] + 12, sc));
        } else {
            for (int j = 0; j < 16; ++j)
                if (base + j < n) q[base + j] = cvt1_fp8<FMT>(qclamp<FMT>(v[it][j], sc));
        }
    }
}

template <int IN_DT, int FMT>
int tw_fused_launch(const void *x, int64_t n, uint8_t *q, float *scale_inv, float *parts, hipStream_t st) {
    const int64_t per  = static_cast<int64_t>(NT) * 16;
    const int     it   = n <= per * TW_FUSED_GRID ? 1 : n <= 2 * per * TW_FUSED_GRID ? 2 : 4;
    const int     g    = static_cast<int>(std::max<int64_t>(1, cdiv(n, per * it)));
    uint8_t       *wsb    = reinterpret_cast<uint8_t *>(parts);
    uint64_t      *tags   = reinterpret_cast<uint64_t *>(wsb + TW_TAG_OFFSET);
    uint64_t      *status = reinterpret_cast<uint64_t *>(wsb + TW_STATUS_OFFSET);
    const uint64_t tag    = next_call_tag();
    const WaitPlan w      = wait_plan(tag, TW_SPIN_LIMIT);
    record_wait(tag, static_cast<int64_t>(TW_STATUS_OFFSET));
#define PTA_TW_GO(IT)                                                                              \
    tw_fused_kernel<IN_DT, FMT, IT><<<g, NT, 0, st>>>(x, n, q, scale_inv, parts, tags, tag, w.expect, w.spin_limit, status)
    if (it == 1) PTA_TW_GO(1);
    else if (it == 2) PTA_TW_GO(2);
    else PTA_TW_GO(4);
#undef PTA_TW_GO
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

// ---------------------------------------------------------------------------
// ROWWISE along the last axis: one wave per row (len <= 4096) or one
// workgroup per row (len <= 16384); values stay in VGPRs (single HBM read).
// Longer rows fall back to two sweeps of the row.
// ---------------------------------------------------------------------------
template <int IN_DT, int FMT, bool VEC, int CPT, bool WAVE_PER_ROW>
__global__ __launch_bounds__(NT) void rw_last_kernel(const void *x, int64_t rows, int64_t len,
                                                      const float *scale_in, uint8_t *q,
                                                      float *scale_inv) {
    constexpr int LANES = WAVE_PER_ROW ? 64 : NT;
    const int64_t row   = WAVE_PER_ROW ? static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)
                                       : static_cast<int64_t>(blockIdx.x);
    const int     l     = WAVE_PER_ROW ? (threadIdx.x & 63) : threadIdx.x;
    if (WAVE_PER_ROW && row >= rows) return; // whole wave exits together
    const int64_t off = row * len;

    // 16-bit inputs of a vector launch stay packed (8 VGPRs per 16
    // values instead of 16) and are widened again in each pass that uses
    // them: the kernel then fits 8 waves per SIMD
    constexpr bool PACK = VEC && IN_DT != PTA_F32;
    float    v[PACK ? 1 : CPT][16];
    uint32_t raw[PACK ? CPT : 1][8];
    auto get16 = [&](int c, float (&o)[16]) {
        if constexpr (PACK) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if constexpr (IN_DT == PTA_BF16) {
                    o[2 * i]     = __uint_as_float(raw[c][i] << 16);
                    o[2 * i + 1] = __uint_as_float(raw[c][i] & 0xffff0000u);
                } else {
                    o[2 * i]     = f16_bits_to_f32(raw[c][i] & 0xffffu);
                    o[2 * i + 1] = f16_bits_to_f32(raw[c][i] >> 16);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) o[j] = v[c][j];
        }
    };
    // the packed words are opaque between passes, so the widened values are
    // not kept live from one pass to the next
    auto fence_raw = [&]() {
        if constexpr (PACK) {
#pragma unroll
            for (int c = 0; c < CPT; ++c)
#pragma unroll
                for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(raw[c][i]));
        }
    };
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int64_t base = (static_cast<int64_t>(c) * LANES + l) * 16;
        if constexpr (PACK) {
            const uint16_t *xs = reinterpret_cast<const uint16_t *>(x) + off + base;
            if (VEC && base + 16 <= len) {
                const uint4 lo = *reinterpret_cast<const uint4 *>(xs), hi = *reinterpret_cast<const uint4 *>(xs + 8);
                raw[c][0] = lo.x; raw[c][1] = lo.y; raw[c][2] = lo.z; raw[c][3] = lo.w;
                raw[c][4] = hi.x; raw[c][5] = hi.y; raw[c][6] = hi.z; raw[c][7] = hi.w;
            } else {
                // +0 past the row's end
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t e0 = base + 2 * i < len ? xs[2 * i] : 0u;
                    const uint32_t e1 = base + 2 * i + 1 < len ? xs[2 * i + 1] : 0u;
                    raw[c][i] = e0 | (e1 << 16);
                }
            }
        } else if (VEC && base + 16 <= len) {
            float p[8], r[8];
            load8<IN_DT>(x, off + base, p);
            load8<IN_DT>(x, off + base + 8, r);
#pragma unroll
            for (int j = 0; j < 8; ++j) { v[c][j] = p[j]; v[c][j + 8] = r[j]; }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[c][j] = base + j < len ? load_scalar<IN_DT>(x, off + base + j) : 0.0f;
        }
        float t[16];
        get16(c, t);
#pragma unroll
        for (int j = 0; j < 16; ++j) a = pmax_abs(a, t[j]);
    }
    // a row with NaN or infinity (NaN-propagating amax) recomputes the
    // reference's NaN-dropping amax and keeps the clamped cast; a given scale
    // keeps it too.  The decision is uniform over the row's lanes.
    float sc;
    bool  clamped = true;
    if (scale_in != nullptr) {
        sc = scale_in[row];
    } else {
        auto row_max = [&](float m) -> float {
            m = amax_wave(m);
            if constexpr (!WAVE_PER_ROW) {
                __shared__ float s[NT / 64];
                __syncthreads(); // reads of a first pass are done
                if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
                __syncthreads();
                m = amax2(amax2(s[0], s[1]), amax2(s[2], s[3]));
            }
            return m;
        };
        a       = row_max(a);
        clamped = special_amax(a);
        if (clamped) {
            fence_raw();
            a = 0.0f;
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
                float t[16];
                get16(c, t);
#pragma unroll
                for (int j = 0; j < 16; ++j) a = fmaxf(a, absq(t[j]));
            }
            a = row_max(a);
        }
        sc = scale_from_amax<FMT>(a, 1e-12f);
    }
    if (l == 0) scale_inv[row] = 1.0f / sc;
    fence_raw();
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int64_t base = (static_cast<int64_t>(c) * LANES + l) * 16;
        float t[16];
        get16(c, t);
        if (VEC && base + 16 <= len) {
            uint4 w;
            if (clamped) {
                w = make_uint4(quant4<FMT>(&t[0], sc), quant4<FMT>(&t[4], sc), quant4<FMT>(&t[8], sc),
                               quant4<FMT>(&t[12], sc));
            } else {
                const float *x = t;
                w = make_uint4(cast4<FMT>(x[0] * sc, x[1] * sc, x[2] * sc, x[3] * sc),
                               cast4<FMT>(x[4] * sc, x[5] * sc, x[6] * sc, x[7] * sc),
                               cast4<FMT>(x[8] * sc, x[9] * sc, x[10] * sc, x[11] * sc),
                               cast4<FMT>(x[12] * sc, x[13] * sc, x[14] * sc, x[15] * sc));
            }
            *reinterpret_cast<uint4 *>(q + off + base) = w;
        } else {
            for (int j = 0; j < 16; ++j)
                if (base + j < len) q[off + base + j] = cvt1_fp8<FMT>(qclamp<FMT>(t[j], sc));
        }
    }
}

template <int IN_DT, int FMT>
__global__ __launch_bounds__(NT) void rw_last_long_kernel(const void *x, int64_t len,
                                                           const float *scale_in, uint8_t *q,
                                                           float *scale_inv) {
    const int64_t row = blockIdx.x;
    const int64_t off = row * len;
    float         sc;
    if (scale_in != nullptr) {
        sc = scale_in[row];
    } else {
        float a = 0.0f;
        for (int64_t i = threadIdx.x; i < len; i += NT) a = fmaxf(a, absq(load_scalar<IN_DT>(x, off + i)));
        a = max64(a);
        __shared__ float s[NT / 64];
        if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = a;
        __syncthreads();
        a  = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        sc = scale_from_amax<FMT>(a, 1e-12f);
    }
    if (threadIdx.x == 0) scale_inv[row] = 1.0f / sc;
    for (int64_t i = threadIdx.x; i < len; i += NT)
        q[off + i] = cvt1_fp8<FMT>(qclamp<FMT>(load_scalar<IN_DT>(x, off + i), sc));
}

// ---------------------------------------------------------------------------
// ROWWISE along a non-last axis: x[outer, len, inner] -> scale per (o, n).
// pass 1: partial column amax over chunks of RW_CH rows;
// pass 2: finalize scale / scale_inv per column;
// pass 3: quantize.
// ---------------------------------------------------------------------------
constexpr int RW_CH = 64;

template <int IN_DT>
__global__ __launch_bounds__(NT) void rw_col_partial_kernel(const void *x, int64_t len, int64_t inner,
                                                             float *partial, int64_t nchunk) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
    const int64_t c = blockIdx.y, o = blockIdx.z;
    if (n >= inner) return;
    const int64_t r0 = c * RW_CH, r1 = r0 + RW_CH < len ? r0 + RW_CH : len;
    float         a  = 0.0f;
    for (int64_t r = r0; r < r1; ++r) a = fmaxf(a, absq(load_scalar<IN_DT>(x, (o * len + r) * inner + n)));
    partial[(o * nchunk + c) * inner + n] = a;
}

template <int FMT>
__global__ __launch_bounds__(NT) void rw_col_finalize_kernel(const float *partial, int64_t nchunk,
                                                              int64_t inner, const float *scale_in,
                                                              float *scale, float *scale_inv) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
    const int64_t o = blockIdx.y;
    if (n >= inner) return;
    float sc;
    if (scale_in != nullptr) {
        sc = scale_in[o * inner + n];
    } else {
        float a = 0.0f;
        for (int64_t c = 0; c < nchunk; ++c) a = fmaxf(a, partial[(o * nchunk + c) * inner + n]);
        sc = scale_from_amax<FMT>(a, 1e-12f);
    }
    scale[o * inner + n]     = sc;
    scale_inv[o * inner + n] = 1.0f / sc;
}

template <int IN_DT, int FMT>
__global__ __launch_bounds__(NT) void rw_col_quant_kernel(const void *x, int64_t len, int64_t inner,
                                                           const float *scale, uint8_t *q) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
    const int64_t c = blockIdx.y, o = blockIdx.z;
    if (n >= inner) return;
    const float   sc = scale[o * inner + n];
    const int64_t r0 = c * RW_CH, r1 = r0 + RW_CH < len ? r0 + RW_CH : len;
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t i = (o * len + r) * inner + n;
        q[i]            = cvt1_fp8<FMT>(qclamp<FMT>(load_scalar<IN_DT>(x, i), sc));
    }
}

// ---------------------------------------------------------------------------
// MXFP8: tile of 64 rows x 64 cols per workgroup (input x[G, M, N]).
// Rowwise: lane t owns row t>>2 ... using 4 lanes per 64-col row, 16 cols each.
// Colwise: the tile is staged in LDS and lane t owns column t>>2, 16 rows.
// ---------------------------------------------------------------------------
// Shared exponent of a block: E = floor(log2 amax) - emax, plus 1 when the
// block maximum would saturate (amax * 2^-E > fp8_max).  Both fp8 maxima are
// 1.75 * 2^emax, so for a normal amax the bump is "mantissa above 1.75"; a
// subnormal amax clamps to 0 either way.  Biased: e8m0 = clamp(E + 127, 0, 254).
template <int FMT> __device__ __forceinline__ int mx_e8m0(float amax) {
    constexpr int  emax = FMT == PTA_E4M3 ? 8 : 15;
    const uint32_t bits = __float_as_uint(amax);
    const int      be   = static_cast<int>((bits >> 23) & 0xffu);
    int            e    = be - emax + ((be != 0 && (bits & 0x7fffffu) > 0x600000u) ? 1 : 0);
    e                   = e < 0 ? 0 : (e > 254 ? 254 : e);
    return amax > 0.0f ? e : 0;
}
__device__ __forceinline__ float mx_qscale(int e8m0) {
    return __uint_as_float(static_cast<uint32_t>(254 - e8m0) << 23); // 2^(127 - e8m0)
}

// MXFP8: one workgroup (4 waves) per 128 x 128 tile of x[g]; lane t owns rows
// 4*(t>>3) .. +3 and columns 16*(t&7) .. +15, so one wave holds 32 consecutive
// rows, i.e. exactly one 32-row column block, and a lane pair (t, t^1) one
// 32-column row block:
//   row amax (1 x 32)  = lane max, then the pair (DPP quad xor 1);
//   col amax (32 x 1)  = max over the lane's 4 rows, then lanes ^8, ^16, ^32;
//   2-D amax (32 x 32) = the row maxima reduced like a column.
// Row output q_row[g*M + m, N_pad] (16-byte stores), colwise output written
// transposed q_col[g*N + n, M_pad] through an LDS byte transpose; padded
// elements are zero and so are their exponents.
struct MXArgs {
    const void *x;
    int64_t     M, N, M_pad, N_pad;
    uint8_t    *q_row, *e_row, *q_col, *e_col;
    int         use2d_row, use2d_col, vec;
    // exponent layout: 0 = [rows, cols/32]; 1 = K-block major [cols/128][rows][4]
    // with erows_row / erows_col rows in the rowwise / colwise arrays
    int         ekmaj;
    int64_t     erows_row, erows_col;
    // grouped rows (x[M, N] split by goffs[G+1]): tiles live in the 128-padded
    // colwise space offs_col; the rowwise output places group g at offs_row[g]
    const int64_t *goffs, *offs_row, *offs_col;
    int64_t        G;
};

// 16-byte store, optionally non-temporal
template <bool NT> __device__ __forceinline__ void st_u4(uint8_t *p, uint4 v) {
    if constexpr (NT) {
        typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(v4u_t{v.x, v.y, v.z, v.w}, reinterpret_cast<v4u_t *>(p));
    } else {
        *reinterpret_cast<uint4 *>(p) = v;
    }
}

// MX tile kernel STREAM mode: 0 plain accesses; 1 non-temporal loads (inputs of
// 192 MiB or more whose fp8 outputs fit the 256 MB MALL); 2 non-temporal
// stores with plain loads (such inputs with larger outputs; both hints
// together were slower on the blockwise kernels)
inline int mx_stream_mode(bool vec, int64_t in_bytes, int64_t out_bytes) {
    if (!vec || in_bytes < (192ll << 20)) return 0;
    return out_bytes >= (256ll << 20) ? 2 : 1;
}

// Two neighbouring tiles of a tile row per workgroup (512-byte row segments)
// for inputs of 128 MiB or more with an even tile count per row.  Measured
// (MX dual, paired against one tile per workgroup): 56 MiB +6.8%, 112 MiB
// +0.4%, 128 MiB -5.9%, 168 MiB -4.1%, 470 MiB -3.3%.
inline bool mx_pair_tiles(bool vec, int64_t in_bytes, int64_t n_pad) {
    return vec && in_bytes >= (128ll << 20) && (n_pad / 128) % 2 == 0;
}

// TPW: tiles per workgroup.  With 2 (large tensors: mx_pair_tiles), the two
// 256-lane halves take neighbouring tiles of one tile row, so the workgroup
// reads 512-byte row segments; every barrier below is taken by both halves.
template <int IN_DT, int FMT, bool ROW, bool COL, int STREAM, bool GROUPED, int TPW>
__global__ __launch_bounds__(NT * TPW) void mx_tile_kernel(const MXArgs a) {
    const int     half = TPW == 2 ? static_cast<int>(threadIdx.x >> 8) : 0;
    const int     t    = static_cast<int>(threadIdx.x) & (NT - 1);
    const int     wave = t >> 6;
    const int     cseg = t & 7;
    const int     rgrp = t >> 3;
    // consecutive workgroups walk the column tiles of one tile row, so the
    // workgroups that run together stream whole rows (MX dual quantize of
    // 28672 x 8192: 246 -> 205 us; 8192 x 8192: 55.7 -> 54.2 us)
    const int64_t M = a.M, N = a.N;
    // 32-bit index arithmetic (at most 2^31 - 1 tiles per launch)
    const uint32_t tiles_n = static_cast<uint32_t>(a.N_pad / 128);
    const uint32_t bx = blockIdx.x * TPW + half;
    const int64_t  tm = bx / tiles_n, tn = bx % tiles_n, g = blockIdx.z;
    const int64_t n0 = tn * 128 + cseg * 16;
    const char   *xb = reinterpret_cast<const char *>(a.x) + g * M * N * InTraits<IN_DT>::bytes;

    // local row lr of this tile: x row xr0 + lr if lr < nval, rowwise output
    // row orow0 + lr if lr < nout (rows nval .. nout - 1 are zero padding)
    int64_t xr0, nval, orow0, nout;
    if constexpr (GROUPED) {
        const int64_t pad0 = tm * 128;
        if (pad0 >= a.offs_col[a.G]) return;
        int64_t lo = 0, hi = a.G - 1; // last group whose padded range starts at or before pad0
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (a.offs_col[mid] <= pad0) lo = mid;
            else hi = mid - 1;
        }
        const int64_t li0 = pad0 - a.offs_col[lo];
        const int64_t len = a.goffs[lo + 1] - a.goffs[lo];
        xr0   = a.goffs[lo] + li0;
        nval  = len - li0;
        orow0 = a.offs_row[lo] + li0;
        nout  = (len + 31) / 32 * 32 - li0;
    } else {
        xr0   = tm * 128;
        nval  = M - tm * 128;
        orow0 = g * M + tm * 128;
        nout  = nval;
    }

    float v[4][16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m  = xr0 + rgrp * 4 + i;
        const bool    ok = rgrp * 4 + i < nval && n0 < N; // N % 32 == 0: all 16 columns in or out
        if (a.vec) {
            float lo[8] = {0, 0, 0, 0, 0, 0, 0, 0}, hi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (ok) {
                load8<IN_DT, STREAM == 1>(xb, m * N + n0, lo);
                load8<IN_DT, STREAM == 1>(xb, m * N + n0 + 8, hi);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[i][j]     = lo[j];
                v[i][j + 8] = hi[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[i][j] = ok ? load_scalar<IN_DT>(xb, m * N + n0 + j) : 0.0f;
        }
    }

    // 1 x 32 row maxima and the lane's share of the 32 x 32 block maxima (the
    // 2-D variants).  First NaN-propagating: a wave (one 32-row block) with no
    // NaN or infinity casts without the clamp, since the E8M0 scale brings
    // every finite value within +-max (|x| 2^(127 - e) <= 1.75 2^emax); a wave
    // with one recomputes the reference's NaN-dropping maxima and clamps.
    float blk = 0.0f;
    float ra[4];
    auto  row_maxima = [&](bool propagate) {
        blk = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) m = propagate ? pmax_abs(m, v[i][j]) : fmaxf(m, absq_fresh(v[i][j]));
            m     = amax2(m, dpp_f<PTA_DPP_QUAD_XOR1>(m));
            ra[i] = m;
            blk   = amax2(blk, m);
        }
    };
    row_maxima(true);
    const bool wave_special = __ballot(special_amax(blk)) != 0;
    if (wave_special) row_maxima(false);
    if (a.use2d_row || a.use2d_col) {
        blk = amax2(blk, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(blk), 0x128, 0xf, 0xf, false)));
        blk = amax_xor32(amax_xor16(blk));
    }

    // The tile's exponents are staged in LDS and stored as one dword per row
    // (rowwise: the tile's 4 column blocks; colwise: its 4 row blocks):
    // scattered single-byte stores cost a third of the kernel's time.
    __shared__ uint32_t s_exp_[TPW][2][128];
    auto &s_exp = s_exp_[half];
    if constexpr (ROW) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lr = rgrp * 4 + i;
            if (lr >= nout) continue;
            const int64_t orow = orow0 + lr;
            const int     e    = mx_e8m0<FMT>(a.use2d_row ? blk : ra[i]);
            const float   sc   = mx_qscale(e);
            uint8_t      *dst  = a.q_row + orow * a.N_pad + n0;
            const float  *x    = v[i];
            st_u4<STREAM == 2>(dst,
                wave_special ? make_uint4(quant4<FMT>(&x[0], sc), quant4<FMT>(&x[4], sc), quant4<FMT>(&x[8], sc),
                                          quant4<FMT>(&x[12], sc))
                             : make_uint4(cast4<FMT>(x[0] * sc, x[1] * sc, x[2] * sc, x[3] * sc),
                                          cast4<FMT>(x[4] * sc, x[5] * sc, x[6] * sc, x[7] * sc),
                                          cast4<FMT>(x[8] * sc, x[9] * sc, x[10] * sc, x[11] * sc),
                                          cast4<FMT>(x[12] * sc, x[13] * sc, x[14] * sc, x[15] * sc)));
            if ((cseg & 1) == 0) reinterpret_cast<uint8_t *>(&s_exp[0][lr])[cseg >> 1] = static_cast<uint8_t>(e);
        }
    }

    if constexpr (COL) {
        __shared__ uint32_t s_tr_[TPW][128][128 / 4 + 1]; // transposed bytes, padded
        auto &s_tr = s_tr_[half];
        const int64_t       eb_col = a.M_pad / 32;
        // A wave holds one 32-row block; lanes l, l ^ 8, l ^ 16, l ^ 32, ... (the
        // same cseg) hold its 8 row groups of the same 16 columns.  Column j's
        // block maximum is reduced by a transposing butterfly that halves the
        // values per lane at each step: permlane32 and permlane16 swaps (with
        // two different operands a swap hands the lower half / even rows the
        // pair's first operand and the others the second, so no selects), then
        // a row_ror:8 DPP step.  Lane l ends with 2 columns,
        // jc = 8 (l >= 32) + 4 ((l >> 4) & 1) + 2 ((l >> 3) & 1) + t, computes
        // their exponents, and the reverse steps broadcast the scales back.
        const int l    = t & 63;
        const int jc0  = 8 * (l >> 5) + 4 * ((l >> 4) & 1) + 2 * ((l >> 3) & 1);
        float     sc16[16];
        int       e2[2];
        if (!a.use2d_col) {
            // from +0: a column of NaN gives 0, never NaN (amax2); quieted
            // inputs where the wave holds NaN or infinity
            float ca[16];
            if (wave_special) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    ca[j] = fmaxf(fmaxf(0.0f, absq_fresh(v[0][j])), fmaxf(absq_fresh(v[1][j]), fmaxf(absq_fresh(v[2][j]), absq_fresh(v[3][j]))));
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    ca[j] = fmaxf(fmaxf(0.0f, fabsf(v[0][j])), fmaxf(fabsf(v[1][j]), fmaxf(fabsf(v[2][j]), fabsf(v[3][j]))));
            }
            float b8[8], b4[4], b2[2];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(ca[k]), __float_as_uint(ca[k + 8]), false, false);
                b8[k] = amax2(__uint_as_float(r[0]), __uint_as_float(r[1])); // column 8 (l >= 32) + k
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(b8[k]), __float_as_uint(b8[k + 4]), false, false);
                b4[k] = amax2(__uint_as_float(r[0]), __uint_as_float(r[1])); // + 4 ((l >> 4) & 1)
            }
            const bool hi8 = (l & 8) != 0;
#pragma unroll
            for (int k = 0; k < 2; ++k)
                b2[k] = amax2(hi8 ? b4[2 + k] : b4[k],
                              __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(hi8 ? b4[k] : b4[2 + k]), 0x128, 0xf, 0xf, false)));
            float s2[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                e2[k] = mx_e8m0<FMT>(b2[k]);
                s2[k] = mx_qscale(e2[k]);
            }
            // reverse: the row_ror:8 partner's pair, then the swaps with equal
            // operands return (even row's, odd row's) and (lower half's, upper half's)
            const float p0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s2[0]), 0x128, 0xf, 0xf, false));
            const float p1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s2[1]), 0x128, 0xf, 0xf, false));
            b4[0] = hi8 ? p0 : s2[0];
            b4[1] = hi8 ? p1 : s2[1];
            b4[2] = hi8 ? s2[0] : p0;
            b4[3] = hi8 ? s2[1] : p1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(b4[k]), __float_as_uint(b4[k]), false, false);
                b8[k]     = __uint_as_float(r[0]);
                b8[k + 4] = __uint_as_float(r[1]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(b8[k]), __float_as_uint(b8[k]), false, false);
                sc16[k]     = __uint_as_float(r[0]);
                sc16[k + 8] = __uint_as_float(r[1]);
            }
        } else {
            const int   e = mx_e8m0<FMT>(blk);
            const float s = mx_qscale(e);
            e2[0] = e2[1] = e;
#pragma unroll
            for (int j = 0; j < 16; ++j) sc16[j] = s;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) reinterpret_cast<uint8_t *>(&s_exp[1][cseg * 16 + jc0 + k])[wave] = static_cast<uint8_t>(e2[k]);
        if (wave_special) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s_tr[cseg * 16 + j][rgrp] = qpack4<FMT>(v[0][j], v[1][j], v[2][j], v[3][j], sc16[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                s_tr[cseg * 16 + j][rgrp] = cast4<FMT>(v[0][j] * sc16[j], v[1][j] * sc16[j], v[2][j] * sc16[j], v[3][j] * sc16[j]);
        }
        __syncthreads();
        if (t < 128 && tn * 128 + t < N) {
            const int64_t n = g * N + tn * 128 + t;
            uint8_t *d = a.ekmaj ? a.e_col + (tm * a.erows_col + n) * 4 : a.e_col + n * eb_col + tm * 4;
            *reinterpret_cast<uint32_t *>(d) = s_exp[1][t];
        }
        // 128 output rows (n) x 128 bytes (m) in 16-byte chunks
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int     c  = it * NT + t;
            const int     nl = c >> 3;
            const int     mc = (c & 7) * 16;
            const int64_t n  = tn * 128 + nl;
            if (n >= N) continue;
            const uint32_t *src = &s_tr[nl][mc >> 2];
            st_u4<STREAM == 2>(a.q_col + (g * N + n) * a.M_pad + tm * 128 + mc, make_uint4(src[0], src[1], src[2], src[3]));
        }
    }
    if constexpr (ROW) {
        if constexpr (!COL) __syncthreads();
        // exponent bytes of the tile's 4 column blocks, one dword per output row
        if (t < 128 && t < nout) {
            const int64_t r = orow0 + t;
            uint8_t *d = a.ekmaj ? a.e_row + (tn * a.erows_row + r) * 4 : a.e_row + r * (a.N_pad / 32) + tn * 4;
            *reinterpret_cast<uint32_t *>(d) = s_exp[0][t];
        }
    }
}

// ---------------------------------------------------------------------------
// Dequantization kernels
// ---------------------------------------------------------------------------
template <int FMT> __device__ __forceinline__ float fp8_to_f32(uint32_t b) {
    // exact decode of an OCP fp8 byte (gfx950 v_cvt_f32_fp8 / v_cvt_f32_bf8)
    if constexpr (FMT == PTA_E4M3) return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(b), 0);
    else return __builtin_amdgcn_cvt_f32_bf8(static_cast<int>(b), 0);
}

template <int OUT_DT> __device__ __forceinline__ void store_out(void *y, int64_t i, float v) {
    if constexpr (OUT_DT == PTA_F32) reinterpret_cast<float *>(y)[i] = v;
    else if constexpr (OUT_DT == PTA_BF16) reinterpret_cast<uint16_t *>(y)[i] = f32_to_bf16_bits(v);
    else reinterpret_cast<uint16_t *>(y)[i] = f32_to_f16_bits(v);
}

// mode: 0 tensor, 1 rowwise [outer,len,inner], 2 block axis0, 3 block axis1, 4 block 2d, 5 mx,
// 6 grouped mx rowwise (padded rows -> packed rows), 7 grouped mx colwise (transposed padded
// columns -> packed rows)
struct DQArgs {
    const uint8_t *q;
    const float   *s;
    const uint8_t *e;
    void          *y;
    int64_t        n;
    int64_t        d0, d1, d2; // mode-specific dims
    int64_t        block;
    int            transpose_out;
    const int64_t *goffs, *goffs_pad; // grouped modes: [G+1] true / padded row offsets
    int64_t        G;
};

// group of packed row r: the g with goffs[g] <= r < goffs[g+1] (binary search)
__device__ __forceinline__ int64_t find_group(const int64_t *offs, int64_t G, int64_t r) {
    int64_t lo = 0, hi = G; // invariant: offs[lo] <= r < offs[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (offs[mid] <= r) lo = mid;
        else hi = mid;
    }
    return lo;
}

template <int FMT, int OUT_DT, int MODE>
__global__ __launch_bounds__(NT) void dequant_kernel(DQArgs a) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * NT;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x; i < a.n; i += stride) {
        float sc;
        if constexpr (MODE == 0) {
            sc = a.s[0];
        } else if constexpr (MODE == 1) { // [outer, len, inner]
            const int64_t inner = a.d2, len = a.d1;
            const int64_t o = i / (len * inner), nn = i % inner;
            sc = a.s[o * inner + nn];
        } else if constexpr (MODE == 2) { // [M, N], s[ceil(M/b), N]
            const int64_t N = a.d1;
            sc = a.s[(i / N) / a.block * N + (i % N)];
        } else if constexpr (MODE == 3) { // [M, N], s[M, ceil(N/b)]
            const int64_t N = a.d1, nb = (N + a.block - 1) / a.block;
            sc = a.s[(i / N) * nb + (i % N) / a.block];
        } else if constexpr (MODE == 4) { // [B, M, N], s[B, mb, nb]
            const int64_t M = a.d1, N = a.d2;
            const int64_t mb = (M + a.block - 1) / a.block, nb = (N + a.block - 1) / a.block;
            const int64_t b = i / (M * N), r = (i / N) % M, c = i % N;
            sc = a.s[(b * mb + r / a.block) * nb + c / a.block];
        } else if constexpr (MODE == 5) { // MX: q[R, C], e[R, C/32]
            const int64_t C = a.d1;
            const int64_t r = i / C, c = i % C;
            sc = __uint_as_float(static_cast<uint32_t>(a.e[r * (C / 32) + c / 32]) << 23);
        }
        if constexpr (MODE == 6) { // y[total_M, C] from q[padded rows, C], e[padded rows, C/32]
            const int64_t C = a.d1;
            const int64_t r = i / C, c = i % C;
            const int64_t g  = find_group(a.goffs, a.G, r);
            const int64_t sr = r - a.goffs[g] + a.goffs_pad[g];
            sc = __uint_as_float(static_cast<uint32_t>(a.e[sr * (C / 32) + c / 32]) << 23);
            store_out<OUT_DT>(a.y, i, fp8_to_f32<FMT>(a.q[sr * C + c]) * sc);
            continue;
        } else if constexpr (MODE == 7) { // y[total_M, R] from q[R, Cq] (columns padded per group)
            const int64_t R = a.d0, Cq = a.d1;
            const int64_t m = i / R, n = i % R;
            const int64_t g  = find_group(a.goffs, a.G, m);
            const int64_t sc_col = m - a.goffs[g] + a.goffs_pad[g];
            sc = __uint_as_float(static_cast<uint32_t>(a.e[n * (Cq / 32) + sc_col / 32]) << 23);
            store_out<OUT_DT>(a.y, i, fp8_to_f32<FMT>(a.q[n * Cq + sc_col]) * sc);
            continue;
        }
        const float v = fp8_to_f32<FMT>(a.q[i]) * sc;
        if constexpr (MODE == 5) {
            if (a.transpose_out) {
                const int64_t R = a.d0, C = a.d1;
                store_out<OUT_DT>(a.y, (i % C) * R + i / C, v);
                continue;
            }
        }
        store_out<OUT_DT>(a.y, i, v);
    }
}

template <int MODE> int launch_dequant(const DQArgs &a, int fmt, int out_dt, hipStream_t st) {
    if (a.n == 0) return PTA_OK;
    int64_t g = cdiv(a.n, NT);
    if (g > 65536) g = 65536;
    const dim3 grid(static_cast<uint32_t>(g));
#define PTA_DQ(F, O) dequant_kernel<F, O, MODE><<<grid, NT, 0, st>>>(a)
#define PTA_DQ_O(F)                                                                                \
    if (out_dt == PTA_BF16) PTA_DQ(F, PTA_BF16);                                                   \
    else if (out_dt == PTA_F16) PTA_DQ(F, PTA_F16);                                                \
    else PTA_DQ(F, PTA_F32)
    if (fmt == PTA_E4M3) { PTA_DQ_O(PTA_E4M3); }
    else { PTA_DQ_O(PTA_E5M2); }
#undef PTA_DQ_O
#undef PTA_DQ
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

// ---------------------------------------------------------------------------
// byte transpose x[B, M, N] -> y[B, N, M], 64 x 64 tiles
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void transpose_u8_kernel(const uint8_t *x, int64_t M, int64_t N, uint8_t *y) {
    __shared__ uint8_t s[64][68];
    const int64_t b = blockIdx.z, m0 = static_cast<int64_t>(blockIdx.y) * 64, n0 = static_cast<int64_t>(blockIdx.x) * 64;
    const uint8_t *xb = x + b * M * N;
    uint8_t       *yb = y + b * M * N;
    const int      t  = threadIdx.x;
    // read: 64 rows x 64 bytes; lane t: row t>>2, 16 bytes at (t&3)*16
    {
        const int     r = t >> 2, c = (t & 3) * 16;
        const int64_t m = m0 + r;
        for (int j = 0; j < 16; ++j) {
            const int64_t n = n0 + c + j;
            s[r][c + j] = (m < M && n < N) ? xb[m * N + n] : 0;
        }
    }
    __syncthreads();
    {
        const int     r = t >> 2, c = (t & 3) * 16; // r: output row (n), c: output col (m)
        const int64_t n = n0 + r;
        if (n < N) {
            for (int j = 0; j < 16; ++j) {
                const int64_t m = m0 + c + j;
                if (m < M) yb[n * M + m] = s[c + j][r];
            }
        }
    }
}

template <int IN_DT, int FMT>
int tw_launch(const void *x, int64_t n, const float *scale, uint8_t *q, float *scale_inv,
              float *parts, bool vec, hipStream_t st) {
    if (scale == nullptr && vec && n > 0 && n <= TW_FUSED_MAX) {
        // a captured call would replay its tag: under stream capture the
        // two-launch form below is used
        if (!stream_capturing(st)) return tw_fused_launch<IN_DT, FMT>(x, n, q, scale_inv, parts, st);
    }
    const int g = tw_grid(n);
    if (scale == nullptr) {
        if (vec) tw_amax_kernel<IN_DT, true><<<g, NT, 0, st>>>(x, n, parts);
        else tw_amax_kernel<IN_DT, false><<<g, NT, 0, st>>>(x, n, parts);
        PTA_CHECK_LAUNCH();
    }
    if (vec) tw_quant_kernel<IN_DT, FMT, true><<<g, NT, 0, st>>>(x, n, parts, g, scale, q, scale_inv);
    else tw_quant_kernel<IN_DT, FMT, false><<<g, NT, 0, st>>>(x, n, parts, g, scale, q, scale_inv);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

template <int IN_DT, int FMT>
int rw_last_launch(const void *x, int64_t rows, int64_t len, const float *scale, uint8_t *q,
                   float *scale_inv, bool vec, hipStream_t st) {
    const int64_t cpt64 = cdiv(len, 64 * 16);
    if (cpt64 <= 4) {
        const dim3 grid(static_cast<uint32_t>(cdiv(rows, 4)));
#define PTA_RW_W(C)                                                                                \
    if (vec) rw_last_kernel<IN_DT, FMT, true, C, true><<<grid, NT, 0, st>>>(x, rows, len, scale, q, scale_inv); \
    else rw_last_kernel<IN_DT, FMT, false, C, true><<<grid, NT, 0, st>>>(x, rows, len, scale, q, scale_inv)
        if (cpt64 == 1) { PTA_RW_W(1); }
        else if (cpt64 == 2) { PTA_RW_W(2); }
        else { PTA_RW_W(4); }
#undef PTA_RW_W
    } else if (cdiv(len, NT * 16) <= 4) {
        const int64_t cpt = cdiv(len, NT * 16);
        const dim3    grid(static_cast<uint32_t>(rows));
#define PTA_RW_B(C)                                                                                \
    if (vec) rw_last_kernel<IN_DT, FMT, true, C, false><<<grid, NT, 0, st>>>(x, rows, len, scale, q, scale_inv); \
    else rw_last_kernel<IN_DT, FMT, false, C, false><<<grid, NT, 0, st>>>(x, rows, len, scale, q, scale_inv)
        if (cpt <= 2) { PTA_RW_B(2); }
        else { PTA_RW_B(4); }
#undef PTA_RW_B
    } else {
        rw_last_long_kernel<IN_DT, FMT><<<static_cast<uint32_t>(rows), NT, 0, st>>>(x, len, scale, q, scale_inv);
    }
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

template <int IN_DT, int FMT>
int rw_col_launch(const void *x, int64_t outer, int64_t len, int64_t inner, const float *scale_in,
                  uint8_t *q, float *scale_inv, float *ws, hipStream_t st) {
    const int64_t nchunk  = cdiv(len, RW_CH);
    float        *scale   = ws;
    float        *partial = ws + outer * inner;
    const dim3    g3(static_cast<uint32_t>(cdiv(inner, NT)), static_cast<uint32_t>(nchunk),
                     static_cast<uint32_t>(outer));
    if (scale_in == nullptr) {
        rw_col_partial_kernel<IN_DT><<<g3, NT, 0, st>>>(x, len, inner, partial, nchunk);
        PTA_CHECK_LAUNCH();
    }
    rw_col_finalize_kernel<FMT><<<dim3(static_cast<uint32_t>(cdiv(inner, NT)), static_cast<uint32_t>(outer)), NT, 0, st>>>(
        partial, nchunk, inner, scale_in, scale, scale_inv);
    PTA_CHECK_LAUNCH();
    rw_col_quant_kernel<IN_DT, FMT><<<g3, NT, 0, st>>>(x, len, inner, scale, q);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

int check_in(const void *x, int in_dtype, int fmt) {
    PTA_CHECK_ARG(x != nullptr, "input pointer is NULL");
    PTA_CHECK_ARG(in_dtype == PTA_BF16 || in_dtype == PTA_F16 || in_dtype == PTA_F32,
                  "unsupported input dtype code %d", in_dtype);
    PTA_CHECK_ARG(fmt == PTA_E4M3 || fmt == PTA_E5M2, "unsupported fp8 format code %d", fmt);
    return PTA_OK;
}

#define PTA_DISPATCH_IN_FMT(in_dtype, fmt, FN, ...)                                                \
    [&]() -> int {                                                                                 \
        if (in_dtype == PTA_BF16) return fmt == PTA_E4M3 ? FN<PTA_BF16, PTA_E4M3>(__VA_ARGS__)    \
                                                         : FN<PTA_BF16, PTA_E5M2>(__VA_ARGS__);   \
        if (in_dtype == PTA_F16) return fmt == PTA_E4M3 ? FN<PTA_F16, PTA_E4M3>(__VA_ARGS__)      \
                                                        : FN<PTA_F16, PTA_E5M2>(__VA_ARGS__);     \
        return fmt == PTA_E4M3 ? FN<PTA_F32, PTA_E4M3>(__VA_ARGS__) : FN<PTA_F32, PTA_E5M2>(__VA_ARGS__); \
    }()

template <int IN_DT, int FMT>
int mx_launch(const void *x, int64_t G, int64_t M, int64_t N, uint8_t *q_row, uint8_t *e_row,
              int u2r, uint8_t *q_col, uint8_t *e_col, int u2c, int layout, hipStream_t st) {
    MXArgs a{};
    a.x = x; a.M = M; a.N = N;
    a.M_pad = cdiv(M, 128) * 128;
    a.N_pad = cdiv(N, 128) * 128;
    a.q_row = q_row; a.e_row = e_row; a.q_col = q_col; a.e_col = e_col;
    a.use2d_row = u2r; a.use2d_col = u2c;
    a.ekmaj = layout == PTA_MX_EXP_KMAJOR;
    a.erows_row = G * M; a.erows_col = G * N;
    a.vec = aligned16(x) ? 1 : 0;
    PTA_CHECK_ARG((a.M_pad / 128) * (a.N_pad / 128) <= 0x7fffffffll, "tensor too large: more than 2^31 - 1 tiles of 128 x 128");
    const dim3 grid(static_cast<uint32_t>((a.M_pad / 128) * (a.N_pad / 128)), 1, static_cast<uint32_t>(G));
    const int64_t in_bytes = G * M * N * InTraits<IN_DT>::bytes;
    const int     mode     = mx_stream_mode(a.vec != 0, in_bytes, G * M * N * ((q_row ? 1 : 0) + (q_col ? 1 : 0)));
    const bool    pair     = mx_pair_tiles(a.vec != 0, in_bytes, a.N_pad);
    const dim3    grid2(grid.x / 2, grid.y, grid.z);
#define PTA_MX_GO(R, C)                                                                            \
    if (mode == 2 && pair) mx_tile_kernel<IN_DT, FMT, R, C, 2, false, 2><<<grid2, 2 * NT, 0, st>>>(a); \
    else if (mode == 2) mx_tile_kernel<IN_DT, FMT, R, C, 2, false, 1><<<grid, NT, 0, st>>>(a);     \
    else if (mode == 1 && pair) mx_tile_kernel<IN_DT, FMT, R, C, 1, false, 2><<<grid2, 2 * NT, 0, st>>>(a); \
    else if (mode == 1) mx_tile_kernel<IN_DT, FMT, R, C, 1, false, 1><<<grid, NT, 0, st>>>(a);     \
    else if (pair) mx_tile_kernel<IN_DT, FMT, R, C, 0, false, 2><<<grid2, 2 * NT, 0, st>>>(a);     \
    else mx_tile_kernel<IN_DT, FMT, R, C, 0, false, 1><<<grid, NT, 0, st>>>(a);
    if (q_row && q_col) { PTA_MX_GO(true, true) }
    else if (q_row) { PTA_MX_GO(true, false) }
    else { PTA_MX_GO(false, true) }
#undef PTA_MX_GO
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

template <int IN_DT, int FMT>
int mx_grouped_launch(const void *x, int64_t M, int64_t N, int64_t G, const int64_t *goffs,
                      const int64_t *offs_row, const int64_t *offs_col, uint8_t *q_row, uint8_t *e_row,
                      uint8_t *q_col, uint8_t *e_col, int u2r, int u2c, hipStream_t st) {
    MXArgs a{};
    a.x = x; a.M = M; a.N = N;
    a.M_pad = cdiv(M + G * 128, 128) * 128; // colwise output columns
    a.N_pad = cdiv(N, 128) * 128;
    a.q_row = q_row; a.e_row = e_row; a.q_col = q_col; a.e_col = e_col;
    a.use2d_row = u2r; a.use2d_col = u2c;
    a.vec = aligned16(x) ? 1 : 0;
    a.goffs = goffs; a.offs_row = offs_row; a.offs_col = offs_col; a.G = G;
    PTA_CHECK_ARG((a.M_pad / 128) * (a.N_pad / 128) <= 0x7fffffffll, "tensor too large: more than 2^31 - 1 tiles of 128 x 128");
    const dim3 grid(static_cast<uint32_t>((a.M_pad / 128) * (a.N_pad / 128)), 1, 1);
    const int64_t in_bytes = M * N * InTraits<IN_DT>::bytes;
    const int     mode     = mx_stream_mode(a.vec != 0, in_bytes, M * N * ((q_row ? 1 : 0) + (q_col ? 1 : 0)));
    const bool    pair     = mx_pair_tiles(a.vec != 0, in_bytes, a.N_pad);
    const dim3    grid2(grid.x / 2, grid.y, grid.z);
#define PTA_MX_GO(R, C)                                                                            \
    if (mode == 2 && pair) mx_tile_kernel<IN_DT, FMT, R, C, 2, true, 2><<<grid2, 2 * NT, 0, st>>>(a); \
    else if (mode == 2) mx_tile_kernel<IN_DT, FMT, R, C, 2, true, 1><<<grid, NT, 0, st>>>(a);      \
    else if (mode == 1 && pair) mx_tile_kernel<IN_DT, FMT, R, C, 1, true, 2><<<grid2, 2 * NT, 0, st>>>(a); \
    else if (mode == 1) mx_tile_kernel<IN_DT, FMT, R, C, 1, true, 1><<<grid, NT, 0, st>>>(a);      \
    else if (pair) mx_tile_kernel<IN_DT, FMT, R, C, 0, true, 2><<<grid2, 2 * NT, 0, st>>>(a);      \
    else mx_tile_kernel<IN_DT, FMT, R, C, 0, true, 1><<<grid, NT, 0, st>>>(a);
    if (q_row && q_col) { PTA_MX_GO(true, true) }
    else if (q_row) { PTA_MX_GO(true, false) }
    else { PTA_MX_GO(false, true) }
#undef PTA_MX_GO
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

} // namespace
} // namespace pta

using namespace pta;

extern "C" size_t pta_quantize_fp8_tensorwise_workspace_size(int64_t) {
    return TW_MAX_PARTS * sizeof(float);
}

extern "C" int pta_quantize_fp8_tensorwise(const void *x, int in_dtype, int64_t n, const float *scale,
                                           void *q, int fmt, float *scale_inv, void *workspace,
                                           size_t workspace_bytes, pta_stream_t stream) {
    clear_error();
    if (int rc = check_in(x, in_dtype, fmt)) return rc;
    PTA_CHECK_ARG(q && scale_inv && n >= 0, "bad arguments");
    PTA_CHECK_ARG(scale != nullptr || (workspace && workspace_bytes >= TW_MAX_PARTS * sizeof(float)),
                  "workspace of %zu bytes required", (size_t)(TW_MAX_PARTS * sizeof(float)));
    const bool vec = aligned16(x) && aligned16(q);
    return PTA_DISPATCH_IN_FMT(in_dtype, fmt, tw_launch, x, n, scale, static_cast<uint8_t *>(q),
                               scale_inv, static_cast<float *>(workspace), vec, as_stream(stream));
}

extern "C" size_t pta_quantize_fp8_rowwise_workspace_size(int64_t outer, int64_t len, int64_t inner) {
    if (inner == 1) return 0;
    return static_cast<size_t>(outer * inner * (1 + cdiv(len, RW_CH))) * sizeof(float);
}

extern "C" int pta_quantize_fp8_rowwise(const void *x, int in_dtype, int64_t outer, int64_t len,
                                        int64_t inner, const float *scale, void *q, int fmt,
                                        float *scale_inv, void *workspace, size_t workspace_bytes,
                                        pta_stream_t stream) {
    clear_error();
    if (int rc = check_in(x, in_dtype, fmt)) return rc;
    PTA_CHECK_ARG(q && scale_inv && outer >= 0 && len >= 0 && inner >= 1, "bad arguments");
    if (outer == 0 || len == 0) return PTA_OK;
    hipStream_t st = as_stream(stream);
    if (inner == 1) {
        PTA_CHECK_ARG(outer <= 0x7fffffffLL, "too many rows");
        const bool vec = aligned16(x) && aligned16(q) && (len % 16 == 0);
        return PTA_DISPATCH_IN_FMT(in_dtype, fmt, rw_last_launch, x, outer, len, scale,
                                   static_cast<uint8_t *>(q), scale_inv, vec, st);
    }
    const size_t need = pta_quantize_fp8_rowwise_workspace_size(outer, len, inner);
    PTA_CHECK_ARG(workspace && workspace_bytes >= need, "workspace of %zu bytes required", need);
    PTA_CHECK_ARG(outer <= 65535 && cdiv(len, RW_CH) <= 65535, "shape too large");
    return PTA_DISPATCH_IN_FMT(in_dtype, fmt, rw_col_launch, x, outer, len, inner, scale,
                               static_cast<uint8_t *>(q), scale_inv,
                               static_cast<float *>(workspace), st);
}

extern "C" int pta_quantize_mxfp8(const void *x, int in_dtype, int64_t G, int64_t M, int64_t N,
                                  void *q_row, uint8_t *e_row, int use_2d_row, void *q_col,
                                  uint8_t *e_col, int use_2d_col, int fmt, int layout, pta_stream_t stream) {
    clear_error();
    if (int rc = check_in(x, in_dtype, fmt)) return rc;
    PTA_CHECK_ARG(in_dtype != PTA_F32, "MXFP8 quantization takes bf16 or fp16 input");
    PTA_CHECK_ARG(G >= 1 && M >= 0 && N >= 0 && G <= 65535, "bad shape");
    PTA_CHECK_ARG(N % 32 == 0, "N must be divisible by 32");
    PTA_CHECK_ARG((q_row == nullptr) == (e_row == nullptr), "q_row/e_row must both be set or NULL");
    PTA_CHECK_ARG((q_col == nullptr) == (e_col == nullptr), "q_col/e_col must both be set or NULL");
    PTA_CHECK_ARG(q_row || q_col, "no output requested");
    PTA_CHECK_ARG(layout == 0 || layout == PTA_MX_EXP_KMAJOR, "unknown exponent layout %d", layout);
    PTA_CHECK_ARG((!q_row || aligned16(q_row)) && (!q_col || aligned16(q_col)), "outputs must be 16-byte aligned");
    if (M == 0 || N == 0) return PTA_OK;
    return PTA_DISPATCH_IN_FMT(in_dtype, fmt, mx_launch, x, G, M, N, static_cast<uint8_t *>(q_row),
                               e_row, use_2d_row, static_cast<uint8_t *>(q_col), e_col, use_2d_col,
                               layout, as_stream(stream));
}

extern "C" int pta_grouped_quantize_mxfp8(const void *x, int in_dtype, int64_t M, int64_t N, int64_t G,
                                          const int64_t *group_lens, const int64_t *group_offs,
                                          void *q_row, uint8_t *e_row, int use_2d_row, int64_t *lens_row,
                                          int64_t *offs_row, void *q_col, uint8_t *e_col, int use_2d_col,
                                          int64_t *lens_col, int64_t *offs_col, int fmt,
                                          pta_stream_t stream) {
    clear_error();
    if (int rc = check_in(x, in_dtype, fmt)) return rc;
    PTA_CHECK_ARG(in_dtype != PTA_F32, "MXFP8 quantization takes bf16 or fp16 input");
    PTA_CHECK_ARG(G >= 1 && M >= 0 && N >= 0, "bad shape");
    PTA_CHECK_ARG(N % 32 == 0, "N must be divisible by 32");
    PTA_CHECK_ARG(group_lens && group_offs && lens_row && offs_row && lens_col && offs_col,
                  "group arrays must be set");
    PTA_CHECK_ARG((q_row == nullptr) == (e_row == nullptr), "q_row/e_row must both be set or NULL");
    PTA_CHECK_ARG((q_col == nullptr) == (e_col == nullptr), "q_col/e_col must both be set or NULL");
    PTA_CHECK_ARG(q_row || q_col, "no output requested");
    PTA_CHECK_ARG((!q_row || aligned16(q_row)) && (!q_col || aligned16(q_col)), "outputs must be 16-byte aligned");
    PTA_CHECK_ARG(!use_2d_row && !use_2d_col, "2-D exponent blocks are not supported for grouped rows");
    if (int rc = pta_grouped_compute_padded_layout(group_lens, lens_row, offs_row, G, 32, stream)) return rc;
    if (int rc = pta_grouped_compute_padded_layout(group_lens, lens_col, offs_col, G, 128, stream)) return rc;
    if (M == 0 || N == 0) return PTA_OK;
    return PTA_DISPATCH_IN_FMT(in_dtype, fmt, mx_grouped_launch, x, M, N, G, group_offs, offs_row, offs_col,
                               static_cast<uint8_t *>(q_row), e_row, static_cast<uint8_t *>(q_col), e_col,
                               use_2d_row, use_2d_col, as_stream(stream));
}

extern "C" int pta_dequantize_fp8_tensorwise(const void *q, int fmt, int64_t n, const float *scale_inv,
                                             void *y, int out_dtype, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(q && y && scale_inv && n >= 0, "bad arguments");
    DQArgs a{};
    a.q = static_cast<const uint8_t *>(q); a.s = scale_inv; a.y = y; a.n = n;
    return launch_dequant<0>(a, fmt, out_dtype, as_stream(stream));
}

extern "C" int pta_dequantize_fp8_rowwise(const void *q, int fmt, int64_t outer, int64_t len,
                                          int64_t inner, const float *scale_inv, void *y,
                                          int out_dtype, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(q && y && scale_inv && outer >= 0 && len >= 0 && inner >= 1, "bad arguments");
    DQArgs a{};
    a.q = static_cast<const uint8_t *>(q); a.s = scale_inv; a.y = y;
    a.n = outer * len * inner; a.d0 = outer; a.d1 = len; a.d2 = inner;
    return launch_dequant<1>(a, fmt, out_dtype, as_stream(stream));
}

extern "C" int pta_dequantize_fp8_blockwise(const void *q, int fmt, int64_t B, int64_t M, int64_t N,
                                            int64_t block, int mode, const float *scale_inv, void *y,
                                            int out_dtype, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(q && y && scale_inv && B >= 1 && M >= 0 && N >= 0 && block > 0, "bad arguments");
    DQArgs a{};
    a.q = static_cast<const uint8_t *>(q); a.s = scale_inv; a.y = y; a.block = block;
    a.n = B * M * N; a.d0 = B; a.d1 = M; a.d2 = N;
    hipStream_t st = as_stream(stream);
    if (mode == 0) { a.d1 = N; return launch_dequant<2>(a, fmt, out_dtype, st); }
    if (mode == 1) { a.d1 = N; return launch_dequant<3>(a, fmt, out_dtype, st); }
    PTA_CHECK_ARG(mode == 2, "mode must be 0, 1 or 2");
    return launch_dequant<4>(a, fmt, out_dtype, st);
}

extern "C" int pta_dequantize_mxfp8(const void *q, int fmt, int64_t R, int64_t C, const uint8_t *e8m0,
                                    int transpose_out, void *y, int out_dtype, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(q && y && e8m0 && R >= 0 && C >= 0 && C % 32 == 0, "bad arguments");
    DQArgs a{};
    a.q = static_cast<const uint8_t *>(q); a.e = e8m0; a.y = y;
    a.n = R * C; a.d0 = R; a.d1 = C; a.transpose_out = transpose_out;
    return launch_dequant<5>(a, fmt, out_dtype, as_stream(stream));
}

extern "C" int pta_grouped_dequantize_mxfp8(const void *q, int fmt, int64_t R, int64_t C,
                                            const uint8_t *e8m0, int colwise, const int64_t *group_offs,
                                            const int64_t *group_offs_padded, int64_t G, int64_t total_M,
                                            void *y, int out_dtype, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(q && y && e8m0 && group_offs && group_offs_padded, "pointers must be set");
    PTA_CHECK_ARG(R >= 0 && C >= 0 && C % 32 == 0 && G >= 1 && total_M >= 0, "bad shape");
    DQArgs a{};
    a.q = static_cast<const uint8_t *>(q); a.e = e8m0; a.y = y;
    a.d0 = R; a.d1 = C; a.goffs = group_offs; a.goffs_pad = group_offs_padded; a.G = G;
    if (!colwise) {
        a.n = total_M * C;
        return launch_dequant<6>(a, fmt, out_dtype, as_stream(stream));
    }
    a.n = total_M * R;
    return launch_dequant<7>(a, fmt, out_dtype, as_stream(stream));
}

// E8M0 scale shuffle (16 x 16 MFMA layout) of x[M, N] into y[M_pad, N_pad]
// (M_pad = roundup(M, 256), N_pad = roundup(N, 8)): the padded array is cut
// into 32 x 8 tiles stored one after another (row-major over tiles), and inside
// a tile the byte of row 16*h + r, column 4*q + c goes to offset
// 64*c + 4*r + 2*q + h.  One thread writes one output dword: the four bytes
// of rows r, r + 16 and columns c, c + 4 of its tile; bytes outside x are 0.
__global__ __launch_bounds__(NT) void shuffle_e8m0_kernel(const uint8_t *x, int64_t M, int64_t N, uint8_t *y,
                                                          int64_t n_dwords, int64_t tiles_per_row) {
    const int64_t d = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
    if (d >= n_dwords) return;
    const int64_t tile = d >> 6;
    const int     w    = static_cast<int>(d & 63);
    const int     c = w >> 4, r = w & 15;
    const int64_t row0 = (tile / tiles_per_row) * 32 + r, col0 = (tile % tiles_per_row) * 8 + c;
    auto at = [&](int64_t rr, int64_t cc) -> uint32_t { return rr < M && cc < N ? x[rr * N + cc] : 0u; };
    const uint32_t v = at(row0, col0) | (at(row0 + 16, col0) << 8) | (at(row0, col0 + 4) << 16) |
                       (at(row0 + 16, col0 + 4) << 24);
    reinterpret_cast<uint32_t *>(y)[d] = v;
}

extern "C" int pta_shuffle_e8m0_scale(const uint8_t *x, int64_t M, int64_t N, uint8_t *y, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(x && y && M >= 0 && N >= 0, "bad arguments");
    PTA_CHECK_ARG((reinterpret_cast<uintptr_t>(y) & 3) == 0, "output must be 4-byte aligned");
    const int64_t Mp = cdiv(M, 256) * 256, Np = cdiv(N, 8) * 8;
    const int64_t n_dwords = Mp * Np / 4;
    if (n_dwords == 0) return PTA_OK;
    shuffle_e8m0_kernel<<<static_cast<uint32_t>(cdiv(n_dwords, NT)), NT, 0, as_stream(stream)>>>(x, M, N, y, n_dwords,
                                                                                                 Np / 8);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" int pta_transpose_u8(const void *x, int64_t B, int64_t M, int64_t N, void *y,
                                pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(x && y && B >= 1 && M >= 0 && N >= 0 && B <= 65535, "bad arguments");
    if (M == 0 || N == 0) return PTA_OK;
    const dim3 grid(static_cast<uint32_t>(cdiv(N, 64)), static_cast<uint32_t>(cdiv(M, 64)),
                    static_cast<uint32_t>(B));
    transpose_u8_kernel<<<grid, NT, 0, as_stream(stream)>>>(static_cast<const uint8_t *>(x), M, N,
                                                            static_cast<uint8_t *>(y));
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free tensorwise quantization.  This entry point has no
// counterpart in the reference: it serves callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  The amax pass's partial maxima (at most TW_MAX_PARTS
// floats for any n) live in `scratch`, a file-scope device array of
// TW_MAX_PARTS * 4 = 8 KiB that every GPU the library runs on holds until the
// process ends.  The amax kernel writes every partial the quant kernel reads,
// so nothing has to start at zero.  All calls on one GPU share that GPU's
// array: calls that overlap on one GPU (different streams, or host threads
// without ordering) race on it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[pta::TW_MAX_PARTS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex    g_scratch_mu;
float        *g_scratch_ptr[kMaxDevices] = {}; // device address of `scratch` per device

// Device address of this GPU's `scratch`, looked up once per device with that
// device current.  The array's name in host code is only a stand-in for the
// symbol; kernels and copies get this pointer instead.
int scratch_for_current_device(float **out) {
    int dev = -1;
    PTA_CHECK_HIP(hipGetDevice(&dev));
    PTA_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device index %d outside the supported range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        PTA_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        PTA_CHECK_ARG(p != nullptr, "no device address for the scratch array on device %d", dev);
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    *out = g_scratch_ptr[dev];
    return PTA_OK;
}
} // namespace

static_assert(sizeof(float) * pta::TW_MAX_PARTS == PTA_TENSORWISE_NOALLOC_SCRATCH_BYTES,
              "the header states the scratch size");

extern "C" int pta_quantize_fp8_tensorwise_noalloc(const void *x, int in_dtype, int64_t n, const float *scale,
                                                   void *q, int fmt, float *scale_inv, pta_stream_t stream) {
    clear_error();
    if (int rc = check_in(x, in_dtype, fmt)) return rc;
    PTA_CHECK_ARG(q && scale_inv && n >= 0, "bad arguments");
    float *parts = nullptr;
    if (scale == nullptr) {
        // the amax pass writes one partial per workgroup: tw_grid(n) <= TW_MAX_PARTS
        const int g = tw_grid(n);
        PTA_CHECK_ARG(g <= TW_MAX_PARTS, "tensorwise amax needs %d partials, the scratch holds %d", g,
                      TW_MAX_PARTS);
        if (int rc = scratch_for_current_device(&parts)) return rc;
    }
    const bool vec = aligned16(x) && aligned16(q);
    return PTA_DISPATCH_IN_FMT(in_dtype, fmt, tw_launch, x, n, scale, static_cast<uint8_t *>(q), scale_inv, parts,
                               vec, as_stream(stream));
}
