/*
 * primus_turbo_amd.h -- C ABI of the MI355X (gfx950) FP8 linear-path library
 * (libprimus_turbo_amd.so).
 *
 * Every entry point takes raw device pointers, int64 sizes, small integer
 * type codes and a HIP stream (hipStream_t passed as void*).  The caller owns
 * every buffer: outputs and workspaces are allocated by the caller (the
 * library never allocates, frees or synchronises the host).  All work is
 * enqueued on the given stream; nothing is read back to the host.  Each call
 * returns PTA_OK or a negative error code; pta_last_error() returns a
 * thread-local message describing the last failure.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the Primus-Turbo repository root).  The reference's native ops are
 * TORCH_LIBRARY schemas (csrc/pytorch/bindings_pytorch.cpp:13-130) that
 * allocate their outputs with at::empty; here the equivalent Python layer
 * allocates and passes pointers in.
 */
#ifndef PRIMUS_TURBO_AMD_H
#define PRIMUS_TURBO_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define PTA_OK 0
#define PTA_ERR_INVALID_ARG (-1)
#define PTA_ERR_HIP (-2)
#define PTA_ERR_UNSUPPORTED (-3)

/* ---- element type codes ---------------------------------------------------- */
#define PTA_F32 0
#define PTA_F16 1
#define PTA_BF16 2

/* ---- fp8 formats (OCP, gfx950) --------------------------------------------- */
#define PTA_E4M3 0 /* torch.float8_e4m3fn, max 448   */
#define PTA_E5M2 1 /* torch.float8_e5m2,   max 57344 */

/* ---- scaling granularity: values equal ScalingGranularity.<X>.value --------
 * (primus_turbo/pytorch/core/low_precision.py:125-133, enum auto() from 1) */
#define PTA_TENSORWISE 1
#define PTA_ROWWISE 2
#define PTA_BLOCKWISE 3
#define PTA_MX_BLOCKWISE 4

typedef void *pta_stream_t; /* hipStream_t */

/* Thread-local description of the last error (empty string if none). */
const char *pta_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int pta_abi_version(void);

/* Bounded cross-workgroup waits.  Two kernels hand data from one workgroup to
 * another through the caller's workspace: the single-launch tensorwise
 * quantize (pta_quantize_fp8_tensorwise and _noalloc, up to 2^21 elements,
 * not under stream capture: every workgroup waits for all others' partial
 * maxima) and the K split of the dense GEMM (pta_gemm_fp8 and
 * pta_gemm_fp8_nt_strided_ws: the second half of a tile waits for the
 * first).  Each wait is bounded: if it gives up (some workgroups could not
 * start, e.g. because concurrent work on other streams held the CUs), the
 * affected outputs become NaN and the kernel writes the call's 64-bit tag
 * into a status word of the workspace.  No counterpart in the reference.
 *
 * pta_last_wait_status: for the last entry-point call made on this host
 * thread, *tag = that call's tag and *status_offset = the status word's byte
 * offset in the workspace it was given (8-byte aligned), or -1 when that call
 * launched no bounded wait.  After the stream has finished the call, the
 * uint64 at workspace + *status_offset equals *tag if and only if a wait gave
 * up.  (The workspace is not cleared: any other value means success.) */
int pta_last_wait_status(uint64_t *tag, int64_t *status_offset);
/* Test hook, no counterpart in the reference: on != 0 makes every bounded
 * wait launched from now on (any thread) poll for a tag that is never
 * published, with a short limit, so each one gives up quickly and every
 * kernel still exits; 0 restores normal waits.  For tests of the give-up
 * path only. */
void pta_test_force_wait_giveup(int on);

/* ============================================================================
 * Quantization
 * ========================================================================== */

/* Workspace bytes needed by pta_quantize_fp8_tensorwise for n elements. */
size_t pta_quantize_fp8_tensorwise_workspace_size(int64_t n);

/* Tensorwise: amax = max|x| (NaN ignored), scale = fp8_max / max(amax, 1e-12),
 * q = fp8(clamp(x * scale)), *scale_inv = 1 / scale.  If scale is non-NULL it
 * is a device scalar used instead of the amax-derived one.  Up to 2^21
 * elements (16-byte aligned x and q, stream not capturing) this is one launch
 * whose workgroups exchange partial maxima through the workspace; if that
 * exchange does not complete, *scale_inv is NaN.  Otherwise two launches.
 * Replaces quantize_fp8_tensorwise (csrc/pytorch/quantization/quantization.cpp:42-88). */
int pta_quantize_fp8_tensorwise(const void *x, int in_dtype, int64_t n, const float *scale,
                                void *q, int fmt, float *scale_inv, void *workspace,
                                size_t workspace_bytes, pta_stream_t stream);

/* Allocation-free variant of pta_quantize_fp8_tensorwise (same arguments
 * without the workspace, same results).  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The amax
 * pass keeps its partial maxima (at most 2048 floats for any n) in a static
 * device array of PTA_TENSORWISE_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends; the call itself allocates nothing.  Calls that overlap on one
 * GPU share that array and race. */
#define PTA_TENSORWISE_NOALLOC_SCRATCH_BYTES 8192
int pta_quantize_fp8_tensorwise_noalloc(const void *x, int in_dtype, int64_t n, const float *scale,
                                        void *q, int fmt, float *scale_inv, pta_stream_t stream);

/* Workspace bytes needed by pta_quantize_fp8_rowwise. */
size_t pta_quantize_fp8_rowwise_workspace_size(int64_t outer, int64_t len, int64_t inner);

/* Rowwise: x viewed as [outer, len, inner]; one scale per (outer, inner) slice
 * reduced over `len` (the quantization axis), eps 1e-12.  scale_inv has
 * outer*inner entries.  If scale is non-NULL (outer*inner entries) it is used
 * instead of the amax-derived one.
 * Replaces quantize_fp8_rowwise (csrc/pytorch/quantization/quantization.cpp:108-206). */
int pta_quantize_fp8_rowwise(const void *x, int in_dtype, int64_t outer, int64_t len,
                             int64_t inner, const float *scale, void *q, int fmt, float *scale_inv,
                             void *workspace, size_t workspace_bytes, pta_stream_t stream);

/* Blockwise 1-D: axis 1 -> 1 x block along N, s[M, ceil(N/block)];
 * axis 0 -> block x 1 along M, s[ceil(M/block), N]; eps 1e-4.
 * Replaces quant_fp8_blockwise_impl
 * (primus_turbo/pytorch/kernels/quantization/quantization_impl.py:74-118). */
int pta_quantize_fp8_blockwise(const void *x, int in_dtype, int64_t M, int64_t N, int64_t block,
                               int axis, void *q, float *s, int fmt, pta_stream_t stream);

/* Layout flags of pta_quantize_fp8_blockwise_dual. */
#define PTA_DUAL_COL_TRANSPOSED 1   /* q_col written as [N, roundup(M, 128)], zero padded */
#define PTA_DUAL_ROW_SCALE_KMAJOR 2 /* s_row written as [ceil(N/block), M] */

/* Blockwise dual (one read of x): row-scaled q_row[M,N] + s_row[M, ceil(N/block)]
 * and col-scaled q_col + s_col[ceil(M/block), N].  Without flags q_col is
 * [M, N] and s_row is [M, ceil(N/block)] (the reference layouts).
 * PTA_DUAL_COL_TRANSPOSED writes q_col as [N, M_pad], M_pad = roundup(M, 128),
 * zero padded (K-contiguous operand for the NT wgrad GEMM);
 * PTA_DUAL_ROW_SCALE_KMAJOR stores s_row(m, kb) at s_row[kb * M + m], so a GEMM
 * reading the scales of one K block for consecutive rows touches consecutive
 * words.  Either output pair may be NULL.
 * Replaces quant_fp8_blockwise_dual_impl (quantization_impl.py:229-274). */
int pta_quantize_fp8_blockwise_dual(const void *x, int in_dtype, int64_t M, int64_t N,
                                    int64_t block, void *q_row, float *s_row, void *q_col,
                                    float *s_col, int layout, int fmt, pta_stream_t stream);

/* Blockwise 2-D weight quant: w[B, M, N] -> q[B, M, N],
 * s[B, ceil(M/block), ceil(N/block)], one scale per block x block tile.
 * If q_t is non-NULL the same bytes are also written transposed as
 * [B, N, M_pad], M_pad = roundup(M, 128), padding bytes zero.
 * Replaces quantize_fp8_blockwise_for_weight (quantization.cpp:1442-1476). */
int pta_quantize_fp8_blockwise_for_weight(const void *w, int in_dtype, int64_t B, int64_t M,
                                          int64_t N, int64_t block, void *q, float *s, void *q_t,
                                          int fmt, pta_stream_t stream);

/* layout flag of pta_quantize_fp8_blockwise_segment_m_row_col: q_col_pad is
 * written transposed, [N, roundup(M, 128) + 128 * G] (column m = padded row m,
 * zero bytes in padding rows), K-contiguous for the variable-K wgrad GEMM */
#define PTA_SEGMENT_COL_TRANSPOSED 1

/* Grouped segment row + col quant (block 128): rows of x[M, N] belong to G
 * groups (group_offs[G+1], device).  Produces q_row[M,N], s_row_t[ceil(N/128), M]
 * (transposed row scales), the 128-padded column-quantized q_col_pad[M+G*128, N]
 * (or its transpose, see PTA_SEGMENT_COL_TRANSPOSED) with
 * s_col_pad[ceil((M+G*128)/128), N], and vk_lens[G] / vk_offs[G+1] (group
 * lengths rounded up to 128 and their prefix sum).  All on device.
 * Replaces quantize_fp8_blockwise_segment_m_row_col (quantization.cpp:1382-1439). */
int pta_quantize_fp8_blockwise_segment_m_row_col(const void *x, int in_dtype, int64_t M,
                                                 int64_t N, int64_t G, const int64_t *group_lens,
                                                 const int64_t *group_offs, int64_t block,
                                                 void *q_row, void *q_col_pad, float *s_row_t,
                                                 float *s_col_pad, int64_t *vk_lens,
                                                 int64_t *vk_offs, int fmt, int layout,
                                                 pta_stream_t stream);

/* Exponent layout of pta_quantize_mxfp8: 0 = [rows, cols_pad/32] (the
 * reference's); PTA_MX_EXP_KMAJOR = K-block major [cols_pad/128][rows][4]: the
 * four exponents of one 128-column block of a row are one dword and the
 * dwords of consecutive rows are contiguous (a GEMM staging the exponents of
 * one K block for 64 rows then reads 256 contiguous bytes). */
#define PTA_MX_EXP_KMAJOR 1

/* MXFP8 (block 32, E8M0): x[G, M, N].  Rowwise output q_row[G*M, N_pad],
 * e_row[G*M, N_pad/32]; colwise output (transposed) q_col[G*N, M_pad],
 * e_col[G*N, M_pad/32]; pads are 128 and padded elements are 0.  Either pair
 * may be NULL.  use_2d_* shares one exponent per 32 x 32 tile.  `layout`
 * selects the exponent layout (0 or PTA_MX_EXP_KMAJOR).
 * Replaces quantize_mxfp8 / quantize_mxfp8_dual (quantization.cpp:736-967). */
int pta_quantize_mxfp8(const void *x, int in_dtype, int64_t G, int64_t M, int64_t N, void *q_row,
                       uint8_t *e_row, int use_2d_row, void *q_col, uint8_t *e_col, int use_2d_col,
                       int fmt, int layout, pta_stream_t stream);

/* Grouped MXFP8 (block 32, E8M0) of x[M, N] whose rows are split into G
 * groups by group_offs[G+1] (device).  Each group is zero-padded along M to
 * 32 rows for the rowwise output and to 128 for the colwise output; the padded
 * lengths and offsets are written to lens_row / offs_row (32) and lens_col /
 * offs_col (128) on the device.  Rowwise: q_row[M_pad_row, N_pad] with group
 * g at rows offs_row[g] .. offs_row[g+1], e_row[M_pad_row, N_pad/32],
 * M_pad_row = roundup(M + 32 G, 32).  Colwise (transposed): q_col[N, M_pad_col]
 * with group g at columns offs_col[g] .., e_col[N, M_pad_col/32],
 * M_pad_col = roundup(M + 128 G, 128).  Padding inside a group's padded range
 * is zero (bytes and exponents); rows / columns past the last group are not
 * written.  Either output pair may be NULL; 2-D exponent blocks are rejected.
 * Replaces grouped_quantize_mxfp8 / grouped_quantize_mxfp8_dual
 * (csrc/pytorch/quantization/quantization.cpp:969-1195). */
int pta_grouped_quantize_mxfp8(const void *x, int in_dtype, int64_t M, int64_t N, int64_t G,
                               const int64_t *group_lens, const int64_t *group_offs, void *q_row,
                               uint8_t *e_row, int use_2d_row, int64_t *lens_row, int64_t *offs_row,
                               void *q_col, uint8_t *e_col, int use_2d_col, int64_t *lens_col,
                               int64_t *offs_col, int fmt, pta_stream_t stream);

/* ============================================================================
 * Dequantization: y = out_dtype(float(q) * scale_inv)
 * ========================================================================== */

/* Replaces dequantize_fp8_tensorwise (quantization.cpp:207+). */
int pta_dequantize_fp8_tensorwise(const void *q, int fmt, int64_t n, const float *scale_inv,
                                  void *y, int out_dtype, pta_stream_t stream);

/* q viewed as [outer, len, inner], scale_inv[outer*inner].
 * Replaces dequantize_fp8_rowwise (quantization.cpp). */
int pta_dequantize_fp8_rowwise(const void *q, int fmt, int64_t outer, int64_t len, int64_t inner,
                               const float *scale_inv, void *y, int out_dtype, pta_stream_t stream);

/* mode 0: block x 1 (axis 0), mode 1: 1 x block (axis 1), mode 2: 2-D weight
 * tiles over [B, M, N].  Replaces dequant_fp8_blockwise(_for_weight)_impl
 * (quantization_impl.py:139-226). */
int pta_dequantize_fp8_blockwise(const void *q, int fmt, int64_t B, int64_t M, int64_t N,
                                 int64_t block, int mode, const float *scale_inv, void *y,
                                 int out_dtype, pta_stream_t stream);

/* MX dequant of q[R, C] with e8m0[R, C/32] along rows; transpose_out = 1 writes
 * y as [C, R] (the colwise direction).  Replaces dequantize_mxfp8
 * (csrc/kernels/quantization/dequantization_mxfp8.cu:26-111). */
int pta_dequantize_mxfp8(const void *q, int fmt, int64_t R, int64_t C, const uint8_t *e8m0,
                         int transpose_out, void *y, int out_dtype, pta_stream_t stream);

/* Grouped MX dequant back to packed rows y[total_M, *].  colwise = 0: q[R, C]
 * holds each group's rows at padded offsets (group_offs_padded), e8m0[R, C/32];
 * y is [total_M, C].  colwise = 1: q[R, C] is the transposed colwise copy
 * whose columns are the padded rows, e8m0[R, C/32]; y is [total_M, R].
 * Packed row r of group g (group_offs[g] <= r < group_offs[g+1]) reads padded
 * row r - group_offs[g] + group_offs_padded[g].  Offsets stay on the device.
 * Replaces grouped_dequantize_mxfp8 (csrc/pytorch/quantization/quantization.cpp:360-425). */
int pta_grouped_dequantize_mxfp8(const void *q, int fmt, int64_t R, int64_t C, const uint8_t *e8m0,
                                 int colwise, const int64_t *group_offs,
                                 const int64_t *group_offs_padded, int64_t G, int64_t total_M,
                                 void *y, int out_dtype, pta_stream_t stream);

/* ============================================================================
 * Layout helpers
 * ========================================================================== */

/* E8M0 scale shuffle into the 16 x 16 MFMA layout: x[M, N] -> y[M_pad, N_pad],
 * M_pad = roundup(M, 256), N_pad = roundup(N, 8), zero padded; 32 x 8 tiles,
 * byte (16 h + r, 4 q + c) of a tile at offset 64 c + 4 r + 2 q + h.
 * Replaces shuffle_scale(scale, [16, 16]) (csrc/kernels/shuffle/shuffle.cu:12-73,
 * csrc/pytorch/shuffle/shuffle.cpp) and the shuffle_scale option of the MXFP8
 * quantizers. */
int pta_shuffle_e8m0_scale(const uint8_t *x, int64_t M, int64_t N, uint8_t *y, pta_stream_t stream);

/* Byte transpose x[B, M, N] -> y[B, N, M].  Replaces transpose_2d
 * (csrc/pytorch/transpose/transpose.cpp) for fp8 tensors. */
int pta_transpose_u8(const void *x, int64_t B, int64_t M, int64_t N, void *y, pta_stream_t stream);

/* offs[0] = 0, offs[i+1] = offs[i] + lens[i] (int64, device).
 * Replaces grouped_gemm_compute_offs (csrc/pytorch/grouped_gemm/ck_grouped_gemm.cpp:63-80). */
int pta_grouped_compute_offs(const int64_t *lens, int64_t *offs, int64_t G, pta_stream_t stream);

/* lens_padded[g] = roundup(lens[g], align) (skipped when NULL), offs_padded =
 * their exclusive prefix sum [G+1] (int64, device).  Replaces
 * compute_padded_layout_gpu (called at csrc/pytorch/quantization/quantization.cpp:1047). */
int pta_grouped_compute_padded_layout(const int64_t *lens, int64_t *lens_padded, int64_t *offs_padded,
                                      int64_t G, int64_t align, pta_stream_t stream);

/* padded_offs[0] = 0, padded_offs[g+1] = padded_offs[g] + roundup(offs[g+1] - offs[g], align)
 * (int64, device).  Replaces the padded-offset computation of
 * csrc/kernels/quantization/quantization_blockwise.cu:16-51. */
int pta_grouped_compute_padded_offs(const int64_t *offs, int64_t *padded_offs, int64_t G,
                                    int64_t align, pta_stream_t stream);

/* ============================================================================
 * GEMM
 * ========================================================================== */

/* C = op(A) @ op(B) with fp32 accumulation and fp8 inputs, output in c_dtype
 * (PTA_BF16 / PTA_F16 / PTA_F32).  Logical shapes: op(A) [M,K], op(B) [K,N];
 * trans_c = 1 stores C^T ([N, M]).
 * granularity: PTA_TENSORWISE (a_scale, b_scale device scalars),
 *              PTA_ROWWISE   (a_scale[M], b_scale[N]),
 *              PTA_BLOCKWISE (see below),
 *              PTA_MX_BLOCKWISE (NT only: e8m0 a_scale[M, K/32], b_scale[N, K/32]).
 * Blockwise scale layouts are those of the reference Triton wrapper
 * (primus_turbo/triton/gemm/gemm_fp8_kernel.py:1013-1154):
 *   NT: A[M,K] a_scale[M,K/128];  B[N,K] b_scale[N/128,K/128]
 *   NN: A[M,K] a_scale[M,K/128];  B[K,N] b_scale[K/128,N/128]
 *   TN: A[K,M] a_scale[K/128,M];  B[K,N] b_scale[K/128,N]
 * workspace may be NULL when pta_gemm_fp8_workspace_size() returns 0 for
 * these arguments.  The workspace holds the NN / TN operand transposes and,
 * for problems of at most half a round of 256 x 256 tiles with K >= 4096 (at
 * most a quarter round: K >= 3072) and K % 128 == 0, the fp32 partial tiles of
 * the K split (each tile then runs as two half-K workgroups; not under stream
 * capture).  Replaces gemm_fp8_impl
 * (primus_turbo/pytorch/kernels/gemm/gemm_fp8_impl.py:438-467) and the native
 * hipblaslt/ck/turbo_gemm_fp8 ops behind it. */
size_t pta_gemm_fp8_workspace_size(int64_t M, int64_t N, int64_t K, int trans_a, int trans_b,
                                   int granularity);
int pta_gemm_fp8(const void *a, int a_fmt, const void *a_scale, int trans_a, const void *b,
                 int b_fmt, const void *b_scale, int trans_b, void *c, int c_dtype, int trans_c,
                 int64_t M, int64_t N, int64_t K, int granularity, void *workspace,
                 size_t workspace_bytes, pta_stream_t stream);

/* Kernel-level NT entry: C[m, n] = sum_k A[m, k] * B[n, k] with explicit row
 * strides and explicit scale addressing.  Blockwise scales are read as
 * a_scale[r * sa_m + kb * sa_k] with r = m (or m / 128 when a_scale_2d) and
 * kb = k / 128; likewise for B.  MX scales are e8m0 bytes at
 * a_scale[m * sa_m + (k / 128) * sa_k + (k / 32) % 4] (row-major
 * [rows, K/32]: sa_m = K/32, sa_k = 4, where sa_k = 0 is read as 4;
 * PTA_MX_EXP_KMAJOR: sa_m = 4, sa_k = 4 * rows); sa_m and sa_k must be
 * multiples of 4.  *_scale_bytes bound the scale arrays.  This has
 * no single counterpart in the reference; it is the kernel interface below
 * gemm_fp8_impl that the autograd functions use to consume transposed
 * quantized copies without extra layout passes. */
int pta_gemm_fp8_nt_strided(const void *a, int a_fmt, int64_t lda, const void *b, int b_fmt,
                            int64_t ldb, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                            int64_t K, int granularity, const void *a_scale, int64_t sa_m,
                            int64_t sa_k, int a_scale_2d, int64_t a_scale_bytes,
                            const void *b_scale, int64_t sb_m, int64_t sb_k, int b_scale_2d,
                            int64_t b_scale_bytes, pta_stream_t stream);

/* pta_gemm_fp8_nt_strided with the kernel choice of pta_gemm_fp8: problems of
 * fewer than 72 tiles of 256 x 256 run on the small-tile kernel (results bit
 * for bit those of the 256 x 256 kernel; blockwise problems it would run on
 * 128 x 128 tiles stay on the 256 x 256 kernel), and problems of at most half
 * a round of tiles with K >= 4096 (a quarter round: K >= 3072) and
 * K % 128 == 0 take the K split, whose
 * fp32 partial tiles and per-call tags live in the workspace (not under
 * stream capture; two calls in flight must not share one workspace).  The
 * workspace size depends on the shape, the granularity, the row strides and
 * the scale extents: pta_gemm_fp8_nt_strided_ws_size(); workspace may be NULL
 * when that is 0.
 * The strided entry above always runs the 256 x 256 kernel.  Like it, this has
 * no single counterpart in the reference: it is what the autograd functions
 * below gemm_fp8_impl call. */
size_t pta_gemm_fp8_nt_strided_ws_size(int64_t M, int64_t N, int64_t K, int granularity, int64_t lda,
                                       int64_t ldb, int64_t a_scale_bytes, int64_t b_scale_bytes);
int pta_gemm_fp8_nt_strided_ws(const void *a, int a_fmt, int64_t lda, const void *b, int b_fmt,
                               int64_t ldb, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                               int64_t K, int granularity, const void *a_scale, int64_t sa_m,
                               int64_t sa_k, int a_scale_2d, int64_t a_scale_bytes,
                               const void *b_scale, int64_t sb_m, int64_t sb_k, int b_scale_2d,
                               int64_t b_scale_bytes, void *workspace, size_t workspace_bytes,
                               pta_stream_t stream);

/* Grouped GEMM over G groups of rows of A (M-grouped, forward / dgrad):
 * out[offs[g]:offs[g+1]] = A[offs[g]:offs[g+1]] @ op(B[g]), B[G, N, K]
 * (trans_b = 1) or [G, K, N].  group_offs[G+1] on device, never read by the host.
 * group_offs_out (may be NULL): when set, A's rows follow the padded layout
 * group_offs and group g's output rows are written packed at
 * out[group_offs_out[g] : group_offs_out[g+1]] (only that many rows of the
 * group are computed into out) -- the MX grouped forward reads 32-padded rows
 * this way (ops/grouped_gemm_fp8.py:692-707 of the reference).
 * Rows [offs_out[G], M_total) of out are set to 0 (offs_out = group_offs_out
 * or group_offs).
 * Blockwise: a_scale transposed [K/128, M_total], b_scale[G, N/128, K/128]
 * (trans_b = 1) or [G, K/128, N/128].  Tensorwise: device scalars.
 * Rowwise: a_scale[M_total], b_scale[G, N].
 * Replaces grouped_gemm_fp8_impl
 * (primus_turbo/pytorch/kernels/grouped_gemm/grouped_gemm_fp8_impl.py:817-859). */
size_t pta_grouped_gemm_fp8_workspace_size(int64_t M_total, int64_t N, int64_t K, int64_t G,
                                           int trans_b, int granularity);
int pta_grouped_gemm_fp8(const void *a, int a_fmt, const void *a_scale, const void *b, int b_fmt,
                         const void *b_scale, int trans_b, const int64_t *group_offs,
                         const int64_t *group_offs_out, int64_t G, int64_t M_total, int64_t N,
                         int64_t K, void *out, int c_dtype, int granularity, int num_cu,
                         void *workspace, size_t workspace_bytes, pta_stream_t stream);

/* Variable-K grouped GEMM (wgrad): for each g,
 * out[g] = op_c( lhs[seg_g]^T @ rhs[seg_g] ) with seg_g = rows
 * [group_offs[g], group_offs[g+1]) of lhs[M_total, OUT_M] and rhs[M_total, OUT_N];
 * out[G, OUT_M, OUT_N] (trans_c = 0) or [G, OUT_N, OUT_M] (trans_c = 1).
 * Blockwise: segments are 128-aligned (group_offs multiples of 128),
 * lhs_scale[M_total/128, OUT_M], rhs_scale[M_total/128, OUT_N].  Tensorwise:
 * device scalars, any group sizes.  Empty groups produce zero output.  Replaces grouped_gemm_fp8_variable_k_impl
 * (grouped_gemm_fp8_impl.py:862-901). */
size_t pta_grouped_gemm_fp8_variable_k_workspace_size(int64_t M_total, int64_t OUT_M,
                                                      int64_t OUT_N, int64_t G, int granularity);
int pta_grouped_gemm_fp8_variable_k(const void *lhs, int lhs_fmt, const void *lhs_scale,
                                    const void *rhs, int rhs_fmt, const void *rhs_scale,
                                    const int64_t *group_offs, int64_t G, int64_t M_total,
                                    int64_t OUT_M, int64_t OUT_N, void *out, int c_dtype,
                                    int trans_c, int granularity, int num_cu, void *workspace,
                                    size_t workspace_bytes, pta_stream_t stream);

/* Variable-K grouped GEMM on operands already transposed and padded per
 * group (wgrad): out[g] = op_c( lhs_t[:, seg_g] @ rhs_t[:, seg_g]^T ) with
 * lhs_t[OUT_M, K_pad], rhs_t[OUT_N, K_pad], seg_g = columns
 * [group_offs[g], group_offs[g+1]) (multiples of 128); out[G, OUT_M, OUT_N]
 * (trans_c = 0) or [G, OUT_N, OUT_M].  Empty groups give zero slices.
 * Scales: MX_BLOCKWISE E8M0 lhs_scale[OUT_M, K_pad/32], rhs_scale[OUT_N, K_pad/32];
 * BLOCKWISE fp32 lhs_scale[K_pad/128, OUT_M], rhs_scale[K_pad/128, OUT_N]
 * (the segment quant's column scales).
 * Replaces the MX call of grouped_gemm_fp8_variable_k_impl
 * (primus_turbo/pytorch/ops/grouped_gemm_fp8.py:760-775) and, for BLOCKWISE,
 * grouped_gemm_fp8_variable_k_impl on the segment quant's column copies
 * (grouped_gemm_fp8.py:186-200) without transposing them first. */
int pta_grouped_gemm_fp8_variable_k_nt(const void *lhs_t, int lhs_fmt, const void *lhs_scale,
                                       const void *rhs_t, int rhs_fmt, const void *rhs_scale,
                                       const int64_t *group_offs, int64_t G, int64_t K_pad,
                                       int64_t OUT_M, int64_t OUT_N, void *out, int c_dtype,
                                       int trans_c, int granularity, pta_stream_t stream);

/* ============================================================================
 * MoE token permutation (expert-major packing for grouped_gemm_fp8)
 * ========================================================================== */

/* expert_map kinds: bool routing map [T, E], or top-k expert indices [T, topk] */
#define PTA_MOE_MAP_BOOL 0
#define PTA_MOE_MAP_I32 1
#define PTA_MOE_MAP_I64 2

/* Workspace bytes needed by pta_moe_permute_preprocess. */
size_t pta_moe_permute_preprocess_workspace_size(int64_t num_tokens, int num_local_experts);

/* Slot assignment.  Each (token t, local expert e) pair routed by expert_map
 * gets the 1-based row slot = 1 + (tokens before t routed to e) + (sum over
 * e' < e of the counts of e' rounded up to pad_multiple).  row_id_map
 * [num_tokens + pad_multiple, 2E + 1] int32: row t holds its slots in
 * ascending e at [0, n), the aux value (e, or with probs_topk_stride > 0 the
 * first k with expert_map[t, k] == e) at [E, E + n) and n at [2E]; padding row
 * num_tokens + i holds the negated slot of the i-th padding row of each expert
 * that has one.  Entries past n are left unwritten.  Slots above
 * num_permuted_tokens (when > 0) are dropped and set *overflow_flag = 1.
 * tokens_per_expert[E] int64 = padded counts (clipped by the cap);
 * *num_dispatched = tokens routed to at least one local expert.  Index maps
 * ignore entries outside [0, E) (after conversion to int32).  E <= 511.
 * Replaces permute_preprocessing (csrc/pytorch/moe_permute/moe_permute.cpp:39-97,
 * kernel csrc/kernels/moe_permute/moe_permute.cu:82-340). */
int pta_moe_permute_preprocess(const void *expert_map, int map_kind, int64_t num_tokens,
                               int num_local_experts, int num_topk, int pad_multiple,
                               int64_t num_permuted_tokens, int probs_topk_stride, int32_t *row_id_map,
                               int64_t *tokens_per_expert, int32_t *overflow_flag,
                               int32_t *num_dispatched, void *workspace, size_t workspace_bytes,
                               pta_stream_t stream);

/* Scatter: for every row r < min(*num_dispatched + pad_multiple, row_id_map_rows)
 * and each of its n slots d: permuted[d - 1] = tokens[r] (d > 0, r a real
 * token) or zeros (d < 0, or r >= *num_dispatched: a padding row).  Rows are
 * hidden * elem_bytes bytes (elem_bytes 1 for fp8, 2 for bf16/fp16; a
 * multiple of 16).  Optional per-token fp32 scaling factors
 * [num_tokens, scales_per_token] and probs [num_tokens, probs_stride or E]
 * (indexed by the aux value) follow the same rows.  Slots outside
 * [1, num_permuted] are skipped.
 * Replaces permute (csrc/pytorch/moe_permute/moe_permute.cpp:108-204,
 * kernel csrc/kernels/moe_permute/moe_permute.cu:437-505). */
int pta_moe_permute(const void *tokens, int64_t num_tokens, int elem_bytes, int64_t hidden,
                    void *permuted, int64_t num_permuted, const int32_t *row_id_map,
                    int64_t row_id_map_rows, const int32_t *num_dispatched, int pad_multiple,
                    int num_local_experts, const float *scaling_factor,
                    float *permuted_scaling_factor, int scales_per_token, const float *probs,
                    float *permuted_probs, int probs_stride, pta_stream_t stream);

/* Gather-reduce: for t < min(*num_dispatched, num_tokens), tokens[t] =
 * dtype(sum in fp32, in row_id_map order, of permuted[d - 1] over the row's
 * positive slots d); with one expert and a probs width of 1 the single row is
 * copied bit for bit.  dtype is PTA_BF16 or PTA_F16, hidden % 8 == 0.
 * probs[t, :] (width probs_stride or E) = permuted_probs[d - 1] at the aux
 * column of each positive slot, 0 elsewhere.  Rows *num_dispatched <= t <
 * num_tokens are written as zeros (tokens and probs).
 * Replaces unpermute (csrc/pytorch/moe_permute/moe_permute.cpp:214-276,
 * kernels csrc/kernels/moe_permute/moe_permute.cu:507-602). */
int pta_moe_unpermute(const void *permuted, int64_t num_permuted, int dtype, int64_t hidden,
                      void *tokens, int64_t num_tokens, const int32_t *row_id_map,
                      const int32_t *num_dispatched, int num_local_experts,
                      const float *permuted_probs, float *probs, int probs_stride,
                      pta_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PRIMUS_TURBO_AMD_H */
