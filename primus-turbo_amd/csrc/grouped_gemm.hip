// Host side of the grouped FP8 GEMMs (MoE experts) on gfx950.
//
// M-grouped (forward / dgrad): one launch whose grid is an upper bound on the
// number of (group, m-tile, n-tile) work items; each workgroup locates its
// group by walking the device-resident group offsets, so the host never reads
// group sizes (no device -> host sync, graph-capturable).  Empty groups own no
// tiles.  K-grouped (variable-K wgrad): grid.y runs over groups; a group with
// no rows writes a zero slice.
// Semantics follow primus_turbo/pytorch/kernels/grouped_gemm/grouped_gemm_fp8_impl.py:
// 817-901 and the tail zeroing of grouped_gemm_kernel.py:1276-1310.
#include "gemm_kernel.h"

namespace pta {
using namespace gemm_detail;

namespace {

// rows [group_offs[G], M_total) of out := 0
__global__ __launch_bounds__(256) void zero_tail_kernel(const int64_t *offs, int64_t G, int64_t M_total,
                                                        int64_t row_bytes, uint8_t *out) {
    const int64_t start = offs[G];
    const int64_t begin = start * row_bytes, end = M_total * row_bytes;
    for (int64_t i = begin + (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 16; i < end;
         i += static_cast<int64_t>(gridDim.x) * 256 * 16) {
        if (i + 16 <= end && ((reinterpret_cast<uintptr_t>(out + i) & 15) == 0)) {
            *reinterpret_cast<uint4 *>(out + i) = make_uint4(0, 0, 0, 0);
        } else {
            for (int64_t j = i; j < i + 16 && j < end; ++j) out[j] = 0;
        }
    }
}

// y[c, poffs[g] + r] = x[offs[g] + r, c] for r < len_g, 0 for len_g <= r < plen_g:
// the token (K) axis of each group is moved to a 128-aligned column range of a
// K-contiguous operand.  grid: (ceil(C/64), ceil(Mp/64)), Mp = M_total + 128*G.
__global__ __launch_bounds__(256) void segment_transpose_kernel(const uint8_t *x, int64_t M_total, int64_t C,
                                                                const int64_t *offs, const int64_t *poffs,
                                                                int64_t G, int64_t ldy, uint8_t *y) {
    __shared__ uint8_t s[64][68];
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t p0 = static_cast<int64_t>(blockIdx.y) * 64; // padded column block
    const int64_t Mp = poffs[G];
    if (p0 >= Mp) return;
    const int t = threadIdx.x;
    // gather: local padded column p0 + r -> source token row (or -1 for padding)
    {
        const int     r  = t >> 2, cc = (t & 3) * 16;
        const int64_t p  = p0 + r;
        int64_t       src = -1;
        if (p < Mp) {
            int64_t lo = 0, hi = G - 1; // last g with poffs[g] <= p
            while (lo < hi) {
                const int64_t mid = (lo + hi + 1) >> 1;
                if (poffs[mid] <= p) lo = mid;
                else hi = mid - 1;
            }
            const int64_t rr = p - poffs[lo];
            if (rr < offs[lo + 1] - offs[lo]) src = offs[lo] + rr;
        }
        for (int j = 0; j < 16; ++j) {
            const int64_t c = c0 + cc + j;
            s[r][cc + j]    = (src >= 0 && c < C) ? x[src * C + c] : 0;
        }
    }
    __syncthreads();
    {
        const int     r = t >> 2, cc = (t & 3) * 16; // r: output row (c), cc: column chunk
        const int64_t c = c0 + r;
        if (c < C) {
            for (int j = 0; j < 16; ++j) {
                const int64_t p = p0 + cc + j;
                if (p < Mp) y[c * ldy + p] = s[cc + j][r];
            }
        }
    }
}

int gran_sm(int gran) {
    switch (gran) {
    case PTA_TENSORWISE: return SM_TENSOR;
    case PTA_ROWWISE: return SM_ROW;
    case PTA_BLOCKWISE: return SM_BLOCK;
    case PTA_MX_BLOCKWISE: return SM_MX;
    default: return -1;
    }
}

// Compute units of the current device (cached per device id).
int cu_count() {
    static int cached[64] = {0};
    int        dev        = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n; // benign race: every writer stores the same value
    }
    return cached[dev];
}

int run(GemmArgs &g, int sm, bool a2d, bool b2d, int fa, int fb, int out_dt, hipStream_t st) {
    if (sm == SM_TENSOR) return dispatch_tensor(g, fa, fb, out_dt, st);
    if (sm == SM_ROW) return dispatch_row(g, fa, fb, out_dt, st);
    if (sm == SM_MX) return dispatch_mx(g, fa, fb, out_dt, st);
    return dispatch_block(g, a2d, b2d, fa, fb, out_dt, st);
}

} // namespace
} // namespace pta

using namespace pta;

extern "C" size_t pta_grouped_gemm_fp8_workspace_size(int64_t /*M_total*/, int64_t N, int64_t K,
                                                      int64_t G, int trans_b, int /*granularity*/) {
    return trans_b ? 0 : static_cast<size_t>(cdiv(G * N * K, 256) * 256);
}

extern "C" int pta_grouped_gemm_fp8(const void *a, int a_fmt, const void *a_scale, const void *b,
                                    int b_fmt, const void *b_scale, int trans_b,
                                    const int64_t *group_offs, const int64_t *group_offs_out, int64_t G,
                                    int64_t M_total, int64_t N, int64_t K, void *out, int c_dtype,
                                    int granularity, int num_cu, void *workspace, size_t workspace_bytes,
                                    pta_stream_t stream) {
    clear_error();
    const int sm = gran_sm(granularity);
    PTA_CHECK_ARG(sm >= 0, "unknown granularity %d", granularity);
    PTA_CHECK_ARG(num_cu >= 0, "num_cu must be >= 0 (0: all compute units)");
    PTA_CHECK_ARG(a && b && out && a_scale && b_scale && group_offs, "NULL pointer argument");
    PTA_CHECK_ARG(G >= 1 && M_total >= 0 && N >= 0 && K >= 0, "bad shape");
    PTA_CHECK_ARG(K % 16 == 0, "K must be a multiple of 16");
    PTA_CHECK_ARG(c_dtype == PTA_BF16 || c_dtype == PTA_F16 || c_dtype == PTA_F32, "unsupported output dtype");
    if (sm == SM_MX) PTA_CHECK_ARG(trans_b && K % 128 == 0, "MX grouped GEMM needs trans_b and K %% 128 == 0");
    if (M_total == 0 || N == 0) return PTA_OK;
    hipStream_t  st = as_stream(stream);
    const size_t eb = c_dtype == PTA_F32 ? 4 : 2;
    const size_t need = pta_grouped_gemm_fp8_workspace_size(M_total, N, K, G, trans_b, granularity);
    PTA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace), "workspace of %zu bytes required", need);

    const uint8_t *bp = static_cast<const uint8_t *>(b);
    if (!trans_b) { // B[g] stored [K, N]: transpose every group to [N, K]
        if (int rc = pta_transpose_u8(b, G, K, N, workspace, stream)) return rc;
        bp = static_cast<const uint8_t *>(workspace);
    }
    GemmArgs g{};
    g.a = static_cast<const uint8_t *>(a); g.b = bp; g.c = out;
    g.M = M_total; g.N = N; g.K = K; g.lda = K; g.ldb = K; g.ldc = N;
    g.sa = a_scale; g.sb = b_scale;
    g.group_mode = 1; g.group_offs = group_offs; g.group_offs_out = group_offs_out; g.G = G;
    g.b_gstride = N * K;
    g.aligned_c = ((N * static_cast<int64_t>(eb)) % 16 == 0) && aligned16(out);
    g.group_m = 1;
    const int64_t kb = cdiv(K, 128);
    bool          b2d = false;
    if (sm == SM_BLOCK) {
        g.sa_m = 1; g.sa_k = M_total; g.sa_bytes = kb * M_total * 4; // a_scale [K/128, M_total]
        b2d = true;
        if (trans_b) { g.sb_m = kb; g.sb_k = 1; }           // [G, N/128, K/128]
        else { g.sb_m = 1; g.sb_k = cdiv(N, 128); }          // [G, K/128, N/128]
        g.sb_gstride = cdiv(N, 128) * kb * 4;
        g.sb_bytes   = g.sb_gstride;
    } else if (sm == SM_ROW) {
        g.sa_bytes = M_total * 4; g.sb_bytes = N * 4; g.sb_gstride = N * 4; // b_scale [G, N]
    } else if (sm == SM_MX) {
        g.sa_m = K / 32; g.sb_m = K / 32; g.sa_k = 4; g.sb_k = 4; g.sa_bytes = M_total * (K / 32);
        g.sb_gstride = N * (K / 32); g.sb_bytes = g.sb_gstride;
    } else {
        g.sa_bytes = 4; g.sb_bytes = 4; g.sb_gstride = 0; // one scalar shared by all groups
    }
    // tile-list upper bound: every group may add one partial tile; rows rounded
    // up to a multiple of 32 for the kernel's XCD-aware tile order.  Persistent
    // grid: one workgroup per CU (the tile uses most of a CU's LDS), or
    // num_cu of them, which leaves the other CUs free for concurrent work.
    g.tiles_n    = static_cast<int>(cdiv(N, BN));
    g.tiles_m    = static_cast<int>(cdiv(cdiv(M_total, BM) + G, 32) * 32);
    const int cu = cu_count();
    g.persistent = num_cu > 0 && num_cu < cu ? num_cu : cu;
    if (int rc = run(g, sm, false, b2d, a_fmt, b_fmt, c_dtype, st)) return rc;
    zero_tail_kernel<<<64, 256, 0, st>>>(group_offs_out ? group_offs_out : group_offs, G, M_total,
                                         N * static_cast<int64_t>(eb), static_cast<uint8_t *>(out));
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" size_t pta_grouped_gemm_fp8_variable_k_workspace_size(int64_t M_total, int64_t OUT_M,
                                                                 int64_t OUT_N, int64_t G,
                                                                 int /*granularity*/) {
    const int64_t Mp = M_total + 128 * G;
    return static_cast<size_t>(cdiv(Mp * OUT_M, 256) * 256 + cdiv(Mp * OUT_N, 256) * 256 +
                               cdiv((G + 1) * 8, 256) * 256);
}

extern "C" int pta_grouped_gemm_fp8_variable_k(const void *lhs, int lhs_fmt, const void *lhs_scale,
                                               const void *rhs, int rhs_fmt, const void *rhs_scale,
                                               const int64_t *group_offs, int64_t G, int64_t M_total,
                                               int64_t OUT_M, int64_t OUT_N, void *out, int c_dtype,
                                               int trans_c, int granularity, int num_cu,
                                               void *workspace, size_t workspace_bytes,
                                               pta_stream_t stream) {
    clear_error();
    (void)num_cu;
    const int sm = gran_sm(granularity);
    PTA_CHECK_ARG(sm == SM_BLOCK || sm == SM_TENSOR || sm == SM_ROW,
                  "variable-K grouped GEMM supports BLOCKWISE, ROWWISE and TENSORWISE");
    PTA_CHECK_ARG(lhs && rhs && out && lhs_scale && rhs_scale && group_offs, "NULL pointer argument");
    PTA_CHECK_ARG(G >= 1 && M_total >= 0 && OUT_M >= 0 && OUT_N >= 0, "bad shape");
    PTA_CHECK_ARG(c_dtype == PTA_BF16 || c_dtype == PTA_F16 || c_dtype == PTA_F32, "unsupported output dtype");
    PTA_CHECK_ARG(G <= 65535, "too many groups");
    if (OUT_M == 0 || OUT_N == 0) return PTA_OK;
    hipStream_t   st = as_stream(stream);
    const size_t  eb = c_dtype == PTA_F32 ? 4 : 2;
    const size_t  need = pta_grouped_gemm_fp8_variable_k_workspace_size(M_total, OUT_M, OUT_N, G, granularity);
    PTA_CHECK_ARG(workspace_bytes >= need && workspace, "workspace of %zu bytes required", need);
    const int64_t Mp = M_total + 128 * G;
    uint8_t *lt = static_cast<uint8_t *>(workspace);
    uint8_t *rt = lt + cdiv(Mp * OUT_M, 256) * 256;
    int64_t *po = reinterpret_cast<int64_t *>(rt + cdiv(Mp * OUT_N, 256) * 256);
    // 128-aligned per-group column ranges (blockwise offsets are already aligned,
    // so for them this is a plain transpose)
    if (int rc = pta_grouped_compute_padded_offs(group_offs, po, G, 128, stream)) return rc;
    {
        const dim3 gl(static_cast<uint32_t>(cdiv(OUT_M, 64)), static_cast<uint32_t>(cdiv(Mp, 64)));
        segment_transpose_kernel<<<gl, 256, 0, st>>>(static_cast<const uint8_t *>(lhs), M_total, OUT_M,
                                                      group_offs, po, G, Mp, lt);
        PTA_CHECK_LAUNCH();
        const dim3 gr(static_cast<uint32_t>(cdiv(OUT_N, 64)), static_cast<uint32_t>(cdiv(Mp, 64)));
        segment_transpose_kernel<<<gr, 256, 0, st>>>(static_cast<const uint8_t *>(rhs), M_total, OUT_N,
                                                      group_offs, po, G, Mp, rt);
        PTA_CHECK_LAUNCH();
    }
    // NT problem per group: C[m, n] = sum_{k in seg} lhsT[m, k] rhsT[n, k]
    GemmArgs   g{};
    const bool swap = trans_c != 0; // C^T: exchange the operands
    g.a = swap ? rt : lt; g.b = swap ? lt : rt;
    g.M = swap ? OUT_N : OUT_M; g.N = swap ? OUT_M : OUT_N; g.K = Mp;
    g.lda = Mp; g.ldb = Mp; g.ldc = g.N;
    g.sa = swap ? rhs_scale : lhs_scale; g.sb = swap ? lhs_scale : rhs_scale;
    g.group_mode = 2; g.group_offs = po; g.G = G;
    g.c = out; g.c_gstride = OUT_M * OUT_N * static_cast<int64_t>(eb);
    g.aligned_c = ((g.N * static_cast<int64_t>(eb)) % 16 == 0) && aligned16(out);
    g.group_m = 4;
    g.tiles_m = static_cast<int>(cdiv(g.M, BM));
    g.tiles_n = static_cast<int>(cdiv(g.N, BN));
    if (sm == SM_BLOCK) { // scales [M_total/128, OUT_*]: global K block index == padded index
        g.sa_m = 1; g.sa_k = g.M; g.sa_bytes = cdiv(M_total, 128) * g.M * 4;
        g.sb_m = 1; g.sb_k = g.N; g.sb_bytes = cdiv(M_total, 128) * g.N * 4;
    } else if (sm == SM_ROW) { // per-column scales shared by all groups
        g.sa_bytes = g.M * 4; g.sb_bytes = g.N * 4;
    } else {
        g.sa_bytes = 4; g.sb_bytes = 4;
    }
    const int fa = swap ? rhs_fmt : lhs_fmt, fb = swap ? lhs_fmt : rhs_fmt;
    return run(g, sm, false, false, fa, fb, c_dtype, st);
}

extern "C" int pta_grouped_gemm_fp8_variable_k_nt(const void *lhs_t, int lhs_fmt, const void *lhs_scale,
                                                  const void *rhs_t, int rhs_fmt, const void *rhs_scale,
                                                  const int64_t *group_offs, int64_t G, int64_t K_pad,
                                                  int64_t OUT_M, int64_t OUT_N, void *out, int c_dtype,
                                                  int trans_c, int granularity, pta_stream_t stream) {
    clear_error();
    const int sm = gran_sm(granularity);
    PTA_CHECK_ARG(sm == SM_MX || sm == SM_BLOCK, "the pre-transposed variable-K entry supports MX_BLOCKWISE and BLOCKWISE");
    PTA_CHECK_ARG(lhs_t && rhs_t && out && lhs_scale && rhs_scale && group_offs, "NULL pointer argument");
    PTA_CHECK_ARG(G >= 1 && G <= 65535 && K_pad >= 0 && OUT_M >= 0 && OUT_N >= 0, "bad shape");
    PTA_CHECK_ARG(K_pad % 128 == 0, "K_pad must be a multiple of 128");
    PTA_CHECK_ARG(c_dtype == PTA_BF16 || c_dtype == PTA_F16 || c_dtype == PTA_F32, "unsupported output dtype");
    PTA_CHECK_ARG(aligned16(lhs_t) && aligned16(rhs_t), "operands must be 16-byte aligned");
    if (OUT_M == 0 || OUT_N == 0) return PTA_OK;
    hipStream_t  st = as_stream(stream);
    const size_t eb = c_dtype == PTA_F32 ? 4 : 2;
    // NT problem per group: C[m, n] = sum_{k in segment g} lhs_t[m, k] rhs_t[n, k];
    // segment offsets are multiples of 128, so K block kb of a segment is
    // global K block (offset / 128 + kb) of the padded layout: the exponent
    // bytes 4 kb + (0..3) (MX) or the scale row kb (blockwise column scales)
    GemmArgs   g{};
    const bool swap = trans_c != 0;
    g.a = static_cast<const uint8_t *>(swap ? rhs_t : lhs_t);
    g.b = static_cast<const uint8_t *>(swap ? lhs_t : rhs_t);
    g.M = swap ? OUT_N : OUT_M; g.N = swap ? OUT_M : OUT_N; g.K = K_pad;
    g.lda = K_pad; g.ldb = K_pad; g.ldc = g.N;
    g.sa = swap ? rhs_scale : lhs_scale; g.sb = swap ? lhs_scale : rhs_scale;
    if (sm == SM_MX) {
        g.sa_m = K_pad / 32; g.sb_m = K_pad / 32; g.sa_k = 4; g.sb_k = 4;
        g.sa_bytes = g.M * (K_pad / 32); g.sb_bytes = g.N * (K_pad / 32);
    } else { // fp32 [K_pad/128, rows]
        g.sa_m = 1; g.sa_k = g.M; g.sa_bytes = (K_pad / 128) * g.M * 4;
        g.sb_m = 1; g.sb_k = g.N; g.sb_bytes = (K_pad / 128) * g.N * 4;
    }
    g.group_mode = 2; g.group_offs = group_offs; g.G = G;
    g.c = out; g.c_gstride = OUT_M * OUT_N * static_cast<int64_t>(eb);
    g.aligned_c = ((g.N * static_cast<int64_t>(eb)) % 16 == 0) && aligned16(out);
    g.group_m = 4;
    g.tiles_m = static_cast<int>(cdiv(g.M, BM));
    g.tiles_n = static_cast<int>(cdiv(g.N, BN));
    const int fa = swap ? rhs_fmt : lhs_fmt, fb = swap ? lhs_fmt : rhs_fmt;
    return run(g, sm, false, false, fa, fb, c_dtype, st);
}
