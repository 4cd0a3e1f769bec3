// Shared host/device helpers for the gfx950 FP8 linear-path library.
//
// Everything here is MI355X-specific: wave64, OCP fp8 conversion through
// v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 (round-to-nearest-even), DPP lane
// exchanges for reductions.  No CUDA shims, no multi-architecture paths.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "primus_turbo_amd.h"

namespace pta {

// ---------------------------------------------------------------------------
// error reporting (thread-local message, int status codes at the C boundary)
// ---------------------------------------------------------------------------
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define PTA_CHECK_ARG(cond, ...)                                                                   \
    do {                                                                                           \
        if (!(cond)) {                                                                             \
            ::pta::set_error(__VA_ARGS__);                                                         \
            return PTA_ERR_INVALID_ARG;                                                            \
        }                                                                                          \
    } while (0)

#define PTA_CHECK_HIP(expr)                                                                        \
    do {                                                                                           \
        hipError_t _e = (expr);                                                                    \
        if (_e != hipSuccess) {                                                                    \
            ::pta::set_error("HIP error '%s' at %s:%d", hipGetErrorString(_e), __FILE__,          \
                             __LINE__);                                                            \
            return PTA_ERR_HIP;                                                                    \
        }                                                                                          \
    } while (0)

#define PTA_CHECK_LAUNCH() PTA_CHECK_HIP(hipGetLastError())

inline hipStream_t as_stream(pta_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline float fp8_max_host(int fmt) { return fmt == PTA_E5M2 ? 57344.0f : 448.0f; }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 64-bit tag unique per call within the process (a per-process salt from the
// process id and start time, xor a counter): kernels whose workgroups hand data
// to each other through a caller's workspace mark each handover with it, so a
// workspace holding an earlier call's tags needs no clearing.
uint64_t next_call_tag();

// true when work submitted to st is being recorded into a graph (a recorded
// call tag would repeat on every replay)
bool stream_capturing(hipStream_t st);

// Bounded cross-workgroup waits (the single-launch tensorwise quantize, the
// K split of the GEMM).  A waiting workgroup polls for `expect` at most
// `spin_limit` times; if it gives up, its result becomes NaN and it writes the
// call's tag into a status word of the caller's workspace.  wait_plan() gives
// the values for a call published under `tag` (normally expect == tag; the
// test hook pta_test_force_wait_giveup makes every wait poll a tag that is
// never published, with a short limit).  record_wait() notes, per host
// thread, the tag and the status word's workspace byte offset of the current
// call; clear_error() resets it to "no bounded wait".
struct WaitPlan {
    uint64_t expect;
    uint32_t spin_limit;
};
WaitPlan wait_plan(uint64_t tag, uint32_t default_limit);
void     record_wait(uint64_t tag, int64_t status_offset);

// compute units of the current device (cached per device)
int device_cu_count();

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    _Float16 h;
    uint16_t s = static_cast<uint16_t>(b);
    __builtin_memcpy(&h, &s, 2);
    return static_cast<float>(h);
}

// Convert an fp32 value to bf16 bits with round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    // The value is an fp32 result that then rounds to fp16: the opaque copy keeps the compiler from
    // fusing the product that made it into v_fma_mix / v_mad_mix, whose single rounding straight to
    // fp16 differs from fp32-then-fp16 on products that round onto an fp16 midpoint.
    asm volatile("" : "+v"(f));
    _Float16 h = static_cast<_Float16>(f);
    uint16_t s;
    __builtin_memcpy(&s, &h, 2);
    return s;
}

// Load 8 consecutive input elements as fp32 (16-byte aligned source for 16-bit
// types, two 16-byte loads for fp32).
template <int IN_DT> struct InTraits;
template <> struct InTraits<PTA_BF16> {
    static constexpr int bytes = 2;
};
template <> struct InTraits<PTA_F16> {
    static constexpr int bytes = 2;
};
template <> struct InTraits<PTA_F32> {
    static constexpr int bytes = 4;
};

template <int IN_DT>
__device__ __forceinline__ float load_scalar(const void *base, int64_t idx) {
    if constexpr (IN_DT == PTA_F32) {
        return reinterpret_cast<const float *>(base)[idx];
    } else if constexpr (IN_DT == PTA_BF16) {
        return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(base)[idx]);
    } else {
        return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(base)[idx]);
    }
}

// 8 elements from a 16-byte-aligned address (two dwordx4 for fp32).
// STREAM: non-temporal loads (data read once and larger than the caches).
template <int IN_DT, bool STREAM = false>
__device__ __forceinline__ void load8(const void *base, int64_t idx, float (&v)[8]) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    auto ld = [](const void *p) -> v4u {
        if constexpr (STREAM) return __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
        else return *reinterpret_cast<const v4u *>(p);
    };
    if constexpr (IN_DT == PTA_F32) {
        const float *p = reinterpret_cast<const float *>(base) + idx;
        const v4u    a = ld(p), b = ld(p + 4);
        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
        v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
    } else {
        const v4u w     = ld(reinterpret_cast<const uint16_t *>(base) + idx);
        uint32_t  ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (IN_DT == PTA_BF16) {
                v[2 * i]     = __uint_as_float(ws[i] << 16);
                v[2 * i + 1] = __uint_as_float(ws[i] & 0xffff0000u);
            } else {
                v[2 * i]     = f16_bits_to_f32(ws[i] & 0xffffu);
                v[2 * i + 1] = f16_bits_to_f32(ws[i] >> 16);
            }
        }
    }
}

// Pack four fp32 values (already clamped to the format's range) into four OCP
// fp8 bytes with round-to-nearest-even.  FMT: PTA_E4M3 or PTA_E5M2.
template <int FMT> __device__ __forceinline__ uint32_t cvt4_fp8(float a, float b, float c, float d) {
    int w;
    if constexpr (FMT == PTA_E4M3) {
        w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    } else {
        w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
    }
    return static_cast<uint32_t>(w);
}

template <int FMT> __device__ __forceinline__ uint8_t cvt1_fp8(float a) {
    return static_cast<uint8_t>(cvt4_fp8<FMT>(a, 0.f, 0.f, 0.f) & 0xffu);
}

template <int FMT> __device__ __forceinline__ constexpr float fp8_max() {
    return FMT == PTA_E4M3 ? 448.0f : 57344.0f;
}

// quant op of the reference: clamp(x * scale, -max, max) through fminf / fmaxf,
// which send NaN to +max.  Computed as -med3(x * -scale, -max, max): one
// v_med3_f32 instead of a min and a max.  x * -scale = -(x * scale) exactly (RNE
// is sign-symmetric), so for every non-NaN input the result is the reference's
// clamp, -0 included; a NaN product is always a quiet NaN (an sNaN input is
// quieted by the multiply), which v_med3_f32 sends to -max (measured on gfx950
// for both signs), so the negation gives the reference's +max.  The two
// negations fold into source modifiers of the multiply and of the conversion.
template <int FMT> __device__ __forceinline__ float qclamp(float x, float scale) {
    return -__builtin_amdgcn_fmed3f(x * -scale, -fp8_max<FMT>(), fp8_max<FMT>());
}

// Four quantized values packed as four fp8 bytes (element 0 in the low byte):
// each value is -med3(x * -s, -max, max) as in qclamp; the four negations are
// one xor of the bytes' sign bits after the conversion (fp8 negation flips bit 7,
// for zeros and the clamped maxima as for every other value).  The first
// conversion's tied operand is its own first input, whose register is then
// reused for the result (no zero-initialised register).
template <int FMT>
__device__ __forceinline__ uint32_t qpack4s(float x0, float x1, float x2, float x3, float s0, float s1, float s2,
                                            float s3) {
    constexpr float M = fp8_max<FMT>();
    const float     a = __builtin_amdgcn_fmed3f(x0 * -s0, -M, M), b = __builtin_amdgcn_fmed3f(x1 * -s1, -M, M);
    const float     c = __builtin_amdgcn_fmed3f(x2 * -s2, -M, M), d = __builtin_amdgcn_fmed3f(x3 * -s3, -M, M);
    int             w;
    if constexpr (FMT == PTA_E4M3) {
        w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    } else {
        w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, __float_as_int(a), false);
        w = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
    }
    return static_cast<uint32_t>(w) ^ 0x80808080u;
}

template <int FMT>
__device__ __forceinline__ uint32_t qpack4(float x0, float x1, float x2, float x3, float scale) {
    return qpack4s<FMT>(x0, x1, x2, x3, scale, scale, scale, scale);
}

template <int FMT>
__device__ __forceinline__ uint32_t quant4(const float *v, float scale) {
    return qpack4<FMT>(v[0], v[1], v[2], v[3], scale);
}

// ---- DPP lane exchange (wave64, rows of 16 lanes) ---------------------------
// ctrl values from the GCN/CDNA DPP encoding.
#define PTA_DPP_QUAD_XOR1 0xB1
#define PTA_DPP_QUAD_XOR2 0x4E
#define PTA_DPP_ROW_HALF_MIRROR 0x141
#define PTA_DPP_ROW_MIRROR 0x140

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// max over groups of 8 consecutive lanes (result in every lane of the group)
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<PTA_DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f<PTA_DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f<PTA_DPP_ROW_HALF_MIRROR>(v));
    return v;
}

// max over groups of 16 consecutive lanes
__device__ __forceinline__ float max16(float v) {
    v = max8(v);
    v = fmaxf(v, dpp_f<PTA_DPP_ROW_MIRROR>(v));
    return v;
}

// max(v, v of lane ^ 16) and max(v, v of lane ^ 32) on the VALU: with both
// operands equal, v_permlane16_swap leaves rows (r0, r0, r2, r2) in one result
// and (r1, r1, r3, r3) in the other (rows of 16 lanes); v_permlane32_swap does
// the same with the two halves of the wave.
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// max over the whole wave (result valid in every lane)
__device__ __forceinline__ float max64(float v) {
    v = max16(v);
    v = max_xor16(v);
    v = max_xor32(v);
    return v;
}

// scale = max / fmaxf(amax, eps) and its inverse 1/scale, both IEEE divisions
// (hipcc emits correctly rounded fp32 division unless fast-math is requested,
// and this library is never built with fast-math).
template <int FMT> __device__ __forceinline__ float scale_from_amax(float amax, float eps) {
    return fp8_max<FMT>() / fmaxf(amax, eps);
}

// Wave-uniform helpers
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & 63; }

} // namespace pta
