/*
 * CPU oracle for the FP8 linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain scalar C, the arithmetic of the reference's
 * quantization kernels so that the HIP kernels under primus-turbo_amd/csrc can
 * be checked byte-for-byte.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never does.
 *
 * Conventions shared by every function below:
 *   - in_dt: 0 = fp32, 1 = fp16, 2 = bf16 (input element type)
 *   - fmt  : 0 = OCP e4m3fn (max 448), 1 = OCP e5m2 (max 57344)
 *   - all scale arithmetic is IEEE-754 binary32 with round-to-nearest-even;
 *     this file must be compiled without -ffast-math and with
 *     -ffp-contract=off so that no multiply/add pair is fused.
 *
 * Reference formulas restated here (paths relative to the reference root):
 *   amax -> scale      csrc/include/primus_turbo/device/quant_utils.cuh:53-72
 *   quant op           csrc/include/primus_turbo/device/quant_utils.cuh:31-38
 *   AbsMax (NaN-free)  csrc/include/primus_turbo/device/reduce.cuh:100-116
 *   fp8 max per dtype  csrc/pytorch/quantization/quantization.cpp:21-35
 *   fp32 -> fp8 cast   csrc/include/primus_turbo/float8.h:83-93 (HIP
 *                      __hip_fp8_e4m3 ctor == v_cvt_pk_fp8_f32 on gfx950, RNE)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define OR_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* scalar helpers                                                             */
/* ------------------------------------------------------------------------- */
static inline float u32_as_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_as_u32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int      exp  = (h >> 10) & 0x1f;
    const uint32_t man  = h & 0x3ff;
    if (exp == 0x1f) return u32_as_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24 exactly representable */
        float v = (float)man * u32_as_f32(0x33800000u); /* 2^-24 */
        return sign ? -v : v;
    }
    return u32_as_f32(sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13));
}

static inline float load_in(const void *x, int in_dt, int64_t i) {
    switch (in_dt) {
    case 0: return ((const float *)x)[i];
    case 1: return half_to_float(((const uint16_t *)x)[i]);
    default: return u32_as_f32((uint32_t)((const uint16_t *)x)[i] << 16);
    }
}

static inline float fp8_max_of(int fmt) { return fmt == 0 ? 448.0f : 57344.0f; }

/*
 * fp32 -> OCP fp8 with round-to-nearest-even, written from the OCP 8-bit
 * floating point specification (v1.0):
 *   e4m3fn: bias 7, no infinities, S.1111.111 is NaN, max normal 448,
 *           min subnormal 2^-9.
 *   e5m2  : bias 15, IEEE-like (inf = S.11111.00), max normal 57344,
 *           min subnormal 2^-16.
 * Values whose rounded magnitude exceeds the max normal become NaN (e4m3fn)
 * or infinity (e5m2) -- the non-saturating behaviour of torch's casts.  The
 * quantizers below always clamp to +-max first, so this path is only hit by
 * the exhaustive conversion tests.
 */
OR_EXPORT uint8_t or_fp8_from_float(float v, int fmt) {
    const int mbits = fmt == 0 ? 3 : 2;
    const int bias  = fmt == 0 ? 7 : 15;
    const uint32_t u    = f32_as_u32(v);
    const uint8_t  sign = (uint8_t)((u >> 31) << 7);
    const uint8_t  nan  = fmt == 0 ? 0x7f : 0x7e;
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) return (uint8_t)(sign | nan);
        return fmt == 0 ? (uint8_t)(sign | 0x7f) : (uint8_t)(sign | 0x7c);
    }
    const double a = fabs((double)v);
    if (a == 0.0) return sign;
    /* quantum of the fp8 grid at this magnitude */
    int e2;
    frexp(a, &e2); /* a = f * 2^e2, f in [0.5, 1) -> floor(log2 a) = e2 - 1 */
    int e = e2 - 1;
    const int emin = 1 - bias;
    if (e < emin) e = emin; /* subnormal range shares the min exponent quantum */
    const double q = ldexp(1.0, e - mbits);
    /* a / q is exact in double (power-of-two divide); round half to even */
    const double r  = a / q;
    double       fl = floor(r);
    const double fr = r - fl;
    if (fr > 0.5 || (fr == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
    const double rounded = fl * q;
    const double maxv    = fmt == 0 ? 448.0 : 57344.0;
    if (rounded > maxv) {
        return fmt == 0 ? (uint8_t)(sign | nan) : (uint8_t)(sign | 0x7c);
    }
    if (rounded == 0.0) return sign;
    int re2;
    frexp(rounded, &re2);
    int re = re2 - 1;
    if (re < emin) {
        /* subnormal: mantissa = rounded / 2^(emin - mbits) */
        const int m = (int)(rounded / ldexp(1.0, emin - mbits));
        return (uint8_t)(sign | m);
    }
    const int m = (int)(rounded / ldexp(1.0, re - mbits)) - (1 << mbits);
    return (uint8_t)(sign | ((re + bias) << mbits) | m);
}

OR_EXPORT float or_fp8_to_float(uint8_t b, int fmt) {
    const int mbits = fmt == 0 ? 3 : 2;
    const int ebits = fmt == 0 ? 4 : 5;
    const int bias  = fmt == 0 ? 7 : 15;
    const int s     = b >> 7;
    const int e     = (b >> mbits) & ((1 << ebits) - 1);
    const int m     = b & ((1 << mbits) - 1);
    double    v;
    if (fmt == 0 && e == 15 && m == 7) return NAN;
    if (fmt == 1 && e == 31) return m ? NAN : (s ? -INFINITY : INFINITY);
    if (e == 0) v = ldexp((double)m, 1 - bias - mbits);
    else v = ldexp((double)((1 << mbits) + m), e - bias - mbits);
    return (float)(s ? -v : v);
}

/* AbsMax op of the reference: fmaxf(fabsf(a), fabsf(b)) -- every NaN is
 * dropped, signalling ones included (CUDA's fmaxf returns the other operand for
 * any NaN).  glibc's fmaxf, like IEEE 754-2008 maxNum, returns NaN for a
 * signalling NaN, so the NaN test comes first here. */
static inline float absmax(float acc, float x) { return isnan(x) ? acc : fmaxf(acc, fabsf(x)); }

/* quant op: clamp(x * scale) to [-max, max] (fmin/fmax map NaN to +max), cast. */
static inline uint8_t quant_one(float x, float scale, int fmt) {
    const float m = fp8_max_of(fmt);
    const float v = x * scale;
    return or_fp8_from_float(fmaxf(fminf(v, m), -m), fmt);
}

/* scale = max / fmaxf(amax, eps); scale_inv = 1 / scale (two IEEE divides). */
static inline void scale_pair(float amax, float eps, int fmt, float *scale, float *scale_inv) {
    const float s = fp8_max_of(fmt) / fmaxf(amax, eps);
    *scale        = s;
    *scale_inv    = 1.0f / s;
}

/* ------------------------------------------------------------------------- */
/* TENSORWISE: csrc/pytorch/quantization/quantization.cpp:42-88              */
/* eps 1e-12 (quantization.h default for compute_scale_from_amax)            */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_quant_tensorwise(const void *x, int in_dt, int64_t n, int fmt, uint8_t *q,
                                   float *scale_inv_out) {
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) amax = absmax(amax, load_in(x, in_dt, i));
    float scale, sinv;
    scale_pair(amax, 1e-12f, fmt, &scale, &sinv);
    for (int64_t i = 0; i < n; ++i) q[i] = quant_one(load_in(x, in_dt, i), scale, fmt);
    *scale_inv_out = sinv;
}

/* ------------------------------------------------------------------------- */
/* ROWWISE: quantization.cpp:108-206, quantization_rowwise.cu:57-135,186-235  */
/* x viewed as [B, L, N]; one scale per (b, n), reduced over L (the axis).   */
/* axis == last dim  <=>  N == 1.  eps 1e-12 (quantization_rowwise.cu:71).   */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_quant_rowwise(const void *x, int in_dt, int64_t B, int64_t L, int64_t N,
                                int fmt, uint8_t *q, float *scale_inv_out) {
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t n = 0; n < N; ++n) {
            float amax = 0.0f;
            for (int64_t l = 0; l < L; ++l) amax = absmax(amax, load_in(x, in_dt, (b * L + l) * N + n));
            float scale, sinv;
            scale_pair(amax, 1e-12f, fmt, &scale, &sinv);
            for (int64_t l = 0; l < L; ++l) {
                const int64_t i = (b * L + l) * N + n;
                q[i]            = quant_one(load_in(x, in_dt, i), scale, fmt);
            }
            scale_inv_out[b * N + n] = sinv;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* BLOCKWISE 1-D (1 x bs along axis 1, or bs x 1 along axis 0)               */
/* primus_turbo/triton/quantization/quant_blockwise.py:11-62 (eps 1e-4);     */
/* masked tail elements are 0 and take part in the amax.                     */
/* axis 1: s[M, ceil(N/bs)];  axis 0: s[ceil(M/bs), N].                       */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_quant_block1d(const void *x, int in_dt, int64_t M, int64_t N, int64_t bs,
                                int axis, int fmt, uint8_t *q, float *s) {
    if (axis == 1) {
        const int64_t nb = (N + bs - 1) / bs;
        for (int64_t m = 0; m < M; ++m)
            for (int64_t j = 0; j < nb; ++j) {
                const int64_t n0 = j * bs, n1 = (n0 + bs < N) ? n0 + bs : N;
                float         amax = 0.0f;
                for (int64_t n = n0; n < n1; ++n) amax = absmax(amax, load_in(x, in_dt, m * N + n));
                float scale, sinv;
                scale_pair(amax, 1e-4f, fmt, &scale, &sinv);
                for (int64_t n = n0; n < n1; ++n) q[m * N + n] = quant_one(load_in(x, in_dt, m * N + n), scale, fmt);
                s[m * nb + j] = sinv;
            }
    } else {
        const int64_t mb = (M + bs - 1) / bs;
        for (int64_t i = 0; i < mb; ++i)
            for (int64_t n = 0; n < N; ++n) {
                const int64_t m0 = i * bs, m1 = (m0 + bs < M) ? m0 + bs : M;
                float         amax = 0.0f;
                for (int64_t m = m0; m < m1; ++m) amax = absmax(amax, load_in(x, in_dt, m * N + n));
                float scale, sinv;
                scale_pair(amax, 1e-4f, fmt, &scale, &sinv);
                for (int64_t m = m0; m < m1; ++m) q[m * N + n] = quant_one(load_in(x, in_dt, m * N + n), scale, fmt);
                s[i * N + n] = sinv;
            }
    }
}

/* ------------------------------------------------------------------------- */
/* BLOCKWISE 2-D weight (bs x bs tiles), quantization_blockwise.cu:246-332   */
/* and quant_blockwise.py:118-155.  w[B, M, N] -> s[B, ceil(M/bs), ceil(N/bs)] */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_quant_block_weight(const void *x, int in_dt, int64_t B, int64_t M, int64_t N,
                                     int64_t bs, int fmt, uint8_t *q, float *s) {
    const int64_t mb = (M + bs - 1) / bs, nb = (N + bs - 1) / bs;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t i = 0; i < mb; ++i)
            for (int64_t j = 0; j < nb; ++j) {
                const int64_t m0 = i * bs, m1 = (m0 + bs < M) ? m0 + bs : M;
                const int64_t n0 = j * bs, n1 = (n0 + bs < N) ? n0 + bs : N;
                float         amax = 0.0f;
                for (int64_t m = m0; m < m1; ++m)
                    for (int64_t n = n0; n < n1; ++n) amax = absmax(amax, load_in(x, in_dt, (b * M + m) * N + n));
                float scale, sinv;
                scale_pair(amax, 1e-4f, fmt, &scale, &sinv);
                for (int64_t m = m0; m < m1; ++m)
                    for (int64_t n = n0; n < n1; ++n) {
                        const int64_t k = (b * M + m) * N + n;
                        q[k]            = quant_one(load_in(x, in_dt, k), scale, fmt);
                    }
                s[(b * mb + i) * nb + j] = sinv;
            }
}

/* ------------------------------------------------------------------------- */
/* Grouped segment row + col quant, quantization_blockwise.cu:16-213 and      */
/* quant_blockwise.py:237-327.  bs = 128.                                     */
/*   row : 1 x bs scales over valid rows; q_row[M, N];                        */
/*         s_row stored transposed ("pshuffled") as [ceil(N/bs), M].          */
/*   col : each group is padded to a multiple of bs rows (pad rows are 0);    */
/*         q_col_pad[M + G*bs, N] (rows >= padded total are not written),     */
/*         s_col_pad[ceil((M + G*bs)/bs), N] (rows >= padded tiles untouched). */
/*   vk_lens[G] = roundup(len_g, bs); vk_offs[G+1] = exclusive prefix sum.    */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_quant_block_segment(const void *x, int in_dt, int64_t M, int64_t N, int64_t G,
                                      const int64_t *group_lens, int64_t bs, int fmt, uint8_t *q_row,
                                      uint8_t *q_col_pad, float *s_row_t, float *s_col_pad,
                                      int64_t *vk_lens, int64_t *vk_offs) {
    const int64_t nb  = (N + bs - 1) / bs;
    int64_t       off = 0, poff = 0;
    vk_offs[0]        = 0;
    for (int64_t g = 0; g < G; ++g) {
        const int64_t len  = group_lens[g];
        const int64_t plen = (len + bs - 1) / bs * bs;
        vk_lens[g]         = plen;
        vk_offs[g + 1]     = poff + plen;
        /* row direction: plain 1 x bs blocks on each valid row */
        for (int64_t r = 0; r < len; ++r) {
            const int64_t m = off + r;
            for (int64_t j = 0; j < nb; ++j) {
                const int64_t n0 = j * bs, n1 = (n0 + bs < N) ? n0 + bs : N;
                float         amax = 0.0f;
                for (int64_t n = n0; n < n1; ++n) amax = absmax(amax, load_in(x, in_dt, m * N + n));
                float scale, sinv;
                scale_pair(amax, 1e-4f, fmt, &scale, &sinv);
                for (int64_t n = n0; n < n1; ++n) q_row[m * N + n] = quant_one(load_in(x, in_dt, m * N + n), scale, fmt);
                s_row_t[j * M + m] = sinv;
            }
        }
        /* col direction: bs x 1 blocks over the zero-padded segment */
        for (int64_t t = 0; t < plen / bs; ++t) {
            const int64_t prow0 = poff + t * bs;
            for (int64_t n = 0; n < N; ++n) {
                float amax = 0.0f;
                for (int64_t r = 0; r < bs; ++r) {
                    const int64_t lr = t * bs + r;
                    if (lr < len) amax = absmax(amax, load_in(x, in_dt, (off + lr) * N + n));
                }
                float scale, sinv;
                scale_pair(amax, 1e-4f, fmt, &scale, &sinv);
                for (int64_t r = 0; r < bs; ++r) {
                    const int64_t lr = t * bs + r;
                    const float   v  = lr < len ? load_in(x, in_dt, (off + lr) * N + n) : 0.0f;
                    q_col_pad[(prow0 + r) * N + n] = quant_one(v, scale, fmt);
                }
                s_col_pad[(prow0 / bs) * N + n] = sinv;
            }
        }
        off += len;
        poff += plen;
    }
}

/* ------------------------------------------------------------------------- */
/* MXFP8 (block 32, E8M0 shared exponent).                                    */
/* The reference's quantize kernel source is absent from the snapshot; the   */
/* surviving constants (csrc/include/primus_turbo/quantization.h:85-102:      */
/* FP8E4M3_TARGET_MAX_POW2 = 8, FP8E5M2_TARGET_MAX_POW2 = 15, the mantissa    */
/* widths and E8M0_EXPONENT_BIAS = 127) and the reference's own round-trip   */
/* test (tests/pytorch/ops/test_quantization.py:304-460, rtol = atol = 0.1    */
/* against the dequantized value) fix the rule restated here:                 */
/*   E     = floor(log2(amax)) - emax_elem,                                   */
/*           plus 1 when amax * 2^-E > fp8_max (the block maximum would       */
/*           otherwise saturate: mantissa of amax above 1.75)                 */
/*   e8m0  = clamp(E + 127, 0, 254)        (amax == 0 -> 0)                   */
/*   q     = cast(clamp(x * 2^(127 - e8m0), +-max))                           */
/* The plain OCP floor rule (no bump) saturates every block whose amax       */
/* mantissa exceeds 1.75 and fails that test at its 1024 x 1024 sizes.       */
/* decode: scale = bits(e8m0 << 23) (csrc/include/primus_turbo/device/        */
/* utils.cuh:117-120), so e8m0 == 0 decodes to 0.0.                           */
/* Layouts (quantization.cpp:736-858): row q[G*M, N_pad] s[G*M, N_pad/32];    */
/* col q[G*N, M_pad] s[G*N, M_pad/32] (transposed); pads are 128 and padded   */
/* elements are 0.  use_2d_block shares one exponent per 32 x 32 tile.        */
/* ------------------------------------------------------------------------- */
static inline int mx_e8m0_of(float amax, int fmt) {
    const int   emax = fmt == 0 ? 8 : 15;
    const float fmax = fmt == 0 ? 448.0f : 57344.0f;
    if (!(amax > 0.0f)) return 0;
    if (isinf(amax)) return 255 - emax; /* biased exponent field 255, no bump */
    int e2;
    frexpf(amax, &e2);                 /* amax = f * 2^e2, f in [0.5, 1) */
    int E = (e2 - 1) - emax;           /* floor(log2 amax) - emax */
    if (ldexpf(amax, -E) > fmax) E += 1; /* exact: a power-of-two scaling */
    int e = E + 127;
    if (e < 0) e = 0;
    if (e > 254) e = 254;
    return e;
}

static inline float mx_quant_scale(int e8m0) {
    /* 2^(127 - e8m0); e8m0 <= 253 for any finite fp32 amax so this is normal */
    return ldexpf(1.0f, 127 - e8m0);
}

OR_EXPORT int or_mx_e8m0(float amax, int fmt) { return mx_e8m0_of(amax, fmt); }

/* direction: 1 = rowwise (blocks along N), 0 = colwise (blocks along M, output transposed) */
OR_EXPORT void or_quant_mx(const void *x, int in_dt, int64_t G, int64_t M, int64_t N, int direction,
                           int use_2d, int fmt, uint8_t *q, uint8_t *e) {
    const int64_t M_pad = (M + 127) / 128 * 128, N_pad = (N + 127) / 128 * 128;
    for (int64_t g = 0; g < G; ++g) {
        const int64_t base = g * M * N;
#define XV(m, n) (((m) < M && (n) < N) ? load_in(x, in_dt, base + (m) * N + (n)) : 0.0f)
        if (direction == 1) {
            const int64_t nsb = N_pad / 32;
            for (int64_t m = 0; m < M; ++m)
                for (int64_t j = 0; j < nsb; ++j) {
                    float amax = 0.0f;
                    if (use_2d) {
                        const int64_t m0 = m / 32 * 32;
                        for (int64_t mm = m0; mm < m0 + 32; ++mm)
                            for (int64_t n = j * 32; n < j * 32 + 32; ++n) amax = absmax(amax, XV(mm, n));
                    } else {
                        for (int64_t n = j * 32; n < j * 32 + 32; ++n) amax = absmax(amax, XV(m, n));
                    }
                    const int   ex = mx_e8m0_of(amax, fmt);
                    const float sc = mx_quant_scale(ex);
                    for (int64_t n = j * 32; n < j * 32 + 32; ++n)
                        q[(g * M + m) * N_pad + n] = quant_one(XV(m, n), sc, fmt);
                    e[(g * M + m) * nsb + j] = (uint8_t)ex;
                }
        } else {
            const int64_t msb = M_pad / 32;
            for (int64_t n = 0; n < N; ++n)
                for (int64_t i = 0; i < msb; ++i) {
                    float amax = 0.0f;
                    if (use_2d) {
                        const int64_t n0 = n / 32 * 32;
                        for (int64_t m = i * 32; m < i * 32 + 32; ++m)
                            for (int64_t nn = n0; nn < n0 + 32; ++nn) amax = absmax(amax, XV(m, nn));
                    } else {
                        for (int64_t m = i * 32; m < i * 32 + 32; ++m) amax = absmax(amax, XV(m, n));
                    }
                    const int   ex = mx_e8m0_of(amax, fmt);
                    const float sc = mx_quant_scale(ex);
                    for (int64_t m = i * 32; m < i * 32 + 32; ++m)
                        q[(g * N + n) * M_pad + m] = quant_one(XV(m, n), sc, fmt);
                    e[(g * N + n) * msb + i] = (uint8_t)ex;
                }
        }
#undef XV
    }
}

/* ------------------------------------------------------------------------- */
/* Dequantization: y = float(q) * scale_inv (quantization_tensorwise.cu:     */
/* 38-45, quant_blockwise.py:162-234, dequantization_mxfp8.cu:26-111).        */
/* Output is fp32 here; callers round to their output dtype.                  */
/* ------------------------------------------------------------------------- */
OR_EXPORT void or_dequant_fp8(const uint8_t *q, int64_t n, int fmt, const float *scale_per_elem,
                              float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_fp8_to_float(q[i], fmt) * scale_per_elem[i];
}

OR_EXPORT float or_e8m0_to_scale(uint8_t e) { return u32_as_f32((uint32_t)e << 23); }
