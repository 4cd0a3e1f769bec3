// Driver for the reference's own HIP quantization, MX dequantization, transpose
// and MoE permutation kernels --
// TEST INFRASTRUCTURE ONLY.
//
// oracle/Makefile.ref compiles this file together with the reference's kernel
// sources, where they lie under /root/reference/csrc, into oracle/_ref/libref_quant.so.
// The extern "C" functions below replay the host-side sequence of the
// reference's native ops (csrc/pytorch/quantization/quantization.cpp:42-206,
// 1382-1476; csrc/pytorch/moe_permute/moe_permute.cpp:39-276) on
// caller-provided device buffers, so GPU parity tests can compare the bytes
// and scales of this repository's kernels with the reference's.
// Input is bf16; fmt 0 = e4m3fn, 1 = e5m2.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "primus_turbo/moe_permute.h"
#include "primus_turbo/quantization.h"
#include "primus_turbo/reduce.h"
#include "primus_turbo/shuffle.h"
#include "primus_turbo/transpose.h"

using namespace primus_turbo;
using bf16 = dtype::bfloat16;

namespace {
float fp8_max(int fmt) { return fmt == 0 ? 448.0f : 57344.0f; }
} // namespace

extern "C" {

// bytes of workspace needed by ref_quant_tensorwise (amax, scale, reduce scratch)
int64_t ref_tensorwise_ws_bytes(int64_t n) {
    return 256 + get_reduce_row_workspace_sizes<float>(1, n);
}

// quantization.cpp:42-88 (no precomputed scale)
int ref_quant_tensorwise(const void *x, int64_t n, int fmt, void *q, float *scale_inv, void *ws,
                         void *stream_) {
    hipStream_t st     = reinterpret_cast<hipStream_t>(stream_);
    float      *amax   = reinterpret_cast<float *>(ws);
    float      *scale  = amax + 1;
    void       *rws    = reinterpret_cast<char *>(ws) + 256;
    const int64_t rsz  = get_reduce_row_workspace_sizes<float>(1, n);
    reduce_row<bf16, float, float>(PrimusTurboReduceOp::REDUCE_ABS_MAX, reinterpret_cast<const bf16 *>(x),
                                   amax, 1, n, rsz, rws, st);
    compute_scale_from_amax<float>(amax, fp8_max(fmt), scale, scale_inv, 1, st);
    if (fmt == 0)
        quantize_tensorwise_impl<bf16, dtype::float8_e4m3>(reinterpret_cast<const bf16 *>(x), scale,
                                                           reinterpret_cast<dtype::float8_e4m3 *>(q), n, st);
    else
        quantize_tensorwise_impl<bf16, dtype::float8_e5m2>(reinterpret_cast<const bf16 *>(x), scale,
                                                           reinterpret_cast<dtype::float8_e5m2 *>(q), n, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// quantization.cpp:155-167 (row-major: axis is the last dim); scale buffer [outer]
int ref_quant_rowwise_last(const void *x, int64_t outer, int64_t inner, int fmt, void *q, float *scale,
                           float *scale_inv, void *stream_) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream_);
    if (fmt == 0)
        quantize_rowwise_row_major_impl<bf16, dtype::float8_e4m3, float, false>(
            reinterpret_cast<const bf16 *>(x), scale, scale_inv, reinterpret_cast<dtype::float8_e4m3 *>(q),
            outer, inner, st);
    else
        quantize_rowwise_row_major_impl<bf16, dtype::float8_e5m2, float, false>(
            reinterpret_cast<const bf16 *>(x), scale, scale_inv, reinterpret_cast<dtype::float8_e5m2 *>(q),
            outer, inner, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int64_t ref_rowwise_col_ws_bytes(int64_t B, int64_t M, int64_t N) {
    return 256 + B * N * 4 + get_reduce_col_workspace_sizes<float>(B, M, N);
}

// quantization.cpp:168-201 (x viewed [B, M, N], reduced over M); scale buffers [B*N]
int ref_quant_rowwise_col(const void *x, int64_t B, int64_t M, int64_t N, int fmt, void *q, float *scale,
                          float *scale_inv, void *ws, void *stream_) {
    hipStream_t   st   = reinterpret_cast<hipStream_t>(stream_);
    float        *amax = reinterpret_cast<float *>(reinterpret_cast<char *>(ws) + 256);
    void         *rws  = reinterpret_cast<char *>(ws) + 256 + B * N * 4;
    const int64_t rsz  = get_reduce_col_workspace_sizes<float>(B, M, N);
    reduce_col<bf16, float, float>(PrimusTurboReduceOp::REDUCE_ABS_MAX, reinterpret_cast<const bf16 *>(x), amax,
                                   B, M, N, rsz, rws, st);
    compute_scale_from_amax<float>(amax, fp8_max(fmt), scale, scale_inv, B * N, st);
    if (fmt == 0)
        quantize_rowwise_col_major_impl<bf16, dtype::float8_e4m3, float>(
            reinterpret_cast<const bf16 *>(x), scale, scale_inv, reinterpret_cast<dtype::float8_e4m3 *>(q), B, M,
            N, st);
    else
        quantize_rowwise_col_major_impl<bf16, dtype::float8_e5m2, float>(
            reinterpret_cast<const bf16 *>(x), scale, scale_inv, reinterpret_cast<dtype::float8_e5m2 *>(q), B, M,
            N, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// quantization.cpp:1442-1476
int ref_quant_weight(const void *w, int64_t B, int64_t M, int64_t N, int fmt, void *q, float *s, void *stream_) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream_);
    if (fmt == 0)
        quantize_blockwise_for_weight_impl<bf16, dtype::float8_e4m3>(
            reinterpret_cast<const bf16 *>(w), reinterpret_cast<dtype::float8_e4m3 *>(q), s, B, M, N, fp8_max(fmt),
            st);
    else
        quantize_blockwise_for_weight_impl<bf16, dtype::float8_e5m2>(
            reinterpret_cast<const bf16 *>(w), reinterpret_cast<dtype::float8_e5m2 *>(q), s, B, M, N, fp8_max(fmt),
            st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// quantization.cpp:1382-1439
int ref_quant_segment(const void *x, int64_t M, int64_t N, int64_t G, const int64_t *group_lens,
                      const int64_t *group_offs, int fmt, void *q_row, void *q_col, float *s_row, float *s_col,
                      int64_t *vk_lens, int64_t *vk_offs, void *stream_) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream_);
    compute_padded_group_offs<int64_t>(group_lens, vk_lens, vk_offs, G, 128, st);
    const int64_t Mpad = M + G * 128;
    if (fmt == 0)
        quantize_blockwise_segment_m_row_col_impl<bf16, dtype::float8_e4m3>(
            reinterpret_cast<const bf16 *>(x), reinterpret_cast<dtype::float8_e4m3 *>(q_row),
            reinterpret_cast<dtype::float8_e4m3 *>(q_col), s_row, s_col, group_offs, vk_offs, M, N, Mpad,
            static_cast<int>(G), fp8_max(fmt), st);
    else
        quantize_blockwise_segment_m_row_col_impl<bf16, dtype::float8_e5m2>(
            reinterpret_cast<const bf16 *>(x), reinterpret_cast<dtype::float8_e5m2 *>(q_row),
            reinterpret_cast<dtype::float8_e5m2 *>(q_col), s_row, s_col, group_offs, vk_offs, M, N, Mpad,
            static_cast<int>(G), fp8_max(fmt), st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// E8M0 scale shuffle of x[M, N] into y[roundup(M,256), roundup(N,8)] with the
// reference's 16x16 layout (csrc/kernels/shuffle/shuffle.cu:12-73,125-139;
// host padding as csrc/pytorch/shuffle/shuffle_meta.cpp:13-29).
int ref_shuffle_e8m0(const void *x, int64_t M, int64_t N, void *y, void *stream) {
    const int64_t Mp = (M + 255) / 256 * 256, Np = (N + 7) / 8 * 8;
    shuffle_e8m0_scale(reinterpret_cast<uint8_t *>(const_cast<void *>(x)), reinterpret_cast<uint8_t *>(y), 16, 16,
                       M, N, Mp, Np, reinterpret_cast<hipStream_t>(stream));
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// MoE permutation (csrc/pytorch/moe_permute/moe_permute.cpp:39-276), on
// caller-allocated outputs.  kind 0 = bool routing map, 1 = int32, 2 = int64
// top-k indices.  num_dispatched must be zeroed by the caller (the reference
// allocates it with at::zeros, moe_permute.cpp:76).
int ref_moe_preprocess(const void *map, int kind, int64_t T, int E, int topk, int pad, int64_t cap,
                       int probs_topk_stride, int *row_id_map, int64_t *tpe, int *overflow, int *ndisp,
                       void *stream) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (kind == 0)
        permute_preprocessing_impl<bool>(reinterpret_cast<const bool *>(map), topk, ndisp, E, (int)T, pad, tpe,
                                         row_id_map, overflow, cap, probs_topk_stride, st);
    else if (kind == 1)
        permute_preprocessing_impl<int>(reinterpret_cast<const int *>(map), topk, ndisp, E, (int)T, pad, tpe,
                                        row_id_map, overflow, cap, probs_topk_stride, st);
    else
        permute_preprocessing_impl<int64_t>(reinterpret_cast<const int64_t *>(map), topk, ndisp, E, (int)T, pad,
                                            tpe, row_id_map, overflow, cap, probs_topk_stride, st);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// permute (moe_permute.cpp:108-204): elem_bytes 1 (fp8, optional scaling
// factors) or 2; rim_rows = row_id_map.size(0).
int ref_moe_permute(const void *tokens, void *out, int elem_bytes, const float *sf, float *osf, const float *probs,
                    float *oprobs, const int *row_id_map, const int *ndisp, int pad, int E, int H, int spt,
                    int rim_rows, int probs_stride, void *stream) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (elem_bytes == 1)
        permute_impl<uint8_t, float, float>(reinterpret_cast<const uint8_t *>(tokens), reinterpret_cast<uint8_t *>(out),
                                            sf, osf, probs, oprobs, row_id_map, ndisp, pad, E, H, spt, rim_rows,
                                            probs_stride, st);
    else
        permute_impl<uint16_t, float, float>(reinterpret_cast<const uint16_t *>(tokens),
                                             reinterpret_cast<uint16_t *>(out), nullptr, nullptr, probs, oprobs,
                                             row_id_map, ndisp, pad, E, H, spt, rim_rows, probs_stride, st);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// unpermute (moe_permute.cpp:214-276): is_bf16 1 = bfloat16, 0 = float16; T = output rows.
int ref_moe_unpermute(const void *perm, void *out, int is_bf16, const float *pprobs, float *oprobs,
                      const int *row_id_map, const int *ndisp, int E, int H, int T, int probs_stride, void *stream) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (is_bf16)
        unpermute_impl<dtype::bfloat16, float>(reinterpret_cast<const dtype::bfloat16 *>(perm),
                                               reinterpret_cast<dtype::bfloat16 *>(out), pprobs, oprobs, row_id_map,
                                               ndisp, E, H, T, probs_stride, st);
    else
        unpermute_impl<dtype::float16, float>(reinterpret_cast<const dtype::float16 *>(perm),
                                              reinterpret_cast<dtype::float16 *>(out), pprobs, oprobs, row_id_map,
                                              ndisp, E, H, T, probs_stride, st);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// MX dequantize of a 2-D q[rows, cols] with E8M0 e[e_rows, e_cols] (row-major),
// replaying dequantize_mxfp8 (csrc/pytorch/quantization/quantization.cpp:283-357):
// rowwise writes y[rows, cols]; colwise (axis 0) writes the transpose
// y[cols, rows].  out_dt 0 = fp32, 2 = bf16 (the C ABI's type codes).
int ref_dequant_mxfp8(const void *q, int fmt, int64_t rows, int64_t cols, const uint8_t *e, int64_t e_rows,
                      int64_t e_cols, int rowwise, void *y, int out_dt, void *stream) {
    hipStream_t   st  = reinterpret_cast<hipStream_t>(stream);
    const int64_t ys0 = rowwise ? cols : rows; // output_2d.stride(0)
#define PTA_REF_DQ(OT, QT)                                                                                    \
    dequantize_mxfp8_impl<OT, QT>(reinterpret_cast<const QT *>(q), reinterpret_cast<OT *>(y), cols, 1, ys0, 1, \
                                  static_cast<int>(rows), static_cast<int>(cols), e, e_cols, 1,               \
                                  static_cast<int>(e_rows), static_cast<int>(e_cols), 32, rowwise != 0, st)
    if (out_dt == 2) {
        if (fmt == 0) PTA_REF_DQ(dtype::bfloat16, dtype::float8_e4m3);
        else PTA_REF_DQ(dtype::bfloat16, dtype::float8_e5m2);
    } else {
        if (fmt == 0) PTA_REF_DQ(dtype::float32, dtype::float8_e4m3);
        else PTA_REF_DQ(dtype::float32, dtype::float8_e5m2);
    }
#undef PTA_REF_DQ
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// transpose_2d (csrc/pytorch/transpose/transpose.cpp): x[batch, M, N] -> y[batch, N, M]
int ref_transpose_2d(const void *x, void *y, int64_t batch, int64_t M, int64_t N, int64_t itemsize, void *stream) {
    transpose_2d_impl(x, y, batch, M, N, itemsize, reinterpret_cast<hipStream_t>(stream));
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

} // extern "C"
