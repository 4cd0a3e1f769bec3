// Host side of the dense FP8 GEMM: layout reduction to NT and scale-stride
// bookkeeping (the kernel itself lives in gemm_kernel.h).
#include "gemm_kernel.h"
#include "gemm_small.h"

// Problems with fewer 256 x 256 tiles than this run on the 64 x 64-tile kernel
// (gemm_small.h), which also reads K-major operands without a transpose pass.
// Measured crossovers on MI355X: NT 2048^3 (64 tiles) 21 us small vs 24 us
// large, 1536 x 4096 x 4096 (96 tiles) 47 vs 44; with a K-major operand the
// large kernel also pays the transpose (1024 x 4096 x 4096 NN: 74 vs 125).
#ifndef PTA_SMALL_MAX_TILES
#define PTA_SMALL_MAX_TILES 72
#endif
#ifndef PTA_SMALL_MAX_TILES_KMAJOR
#define PTA_SMALL_MAX_TILES_KMAJOR 100
#endif
// Tile of the small kernel: 128 x 128 when that still gives this many tiles,
// else 64 x 64 when that does, else 32 x 64 (about one tile per CU or more).
#ifndef PTA_SMALL_T128_MIN
#define PTA_SMALL_T128_MIN 240
#endif
#ifndef PTA_SMALL_T64_MIN
#define PTA_SMALL_T64_MIN 240
#endif
#ifndef PTA_SMALL_FORCE_TILE
#define PTA_SMALL_FORCE_TILE -1
#endif
// Shortest K for the K split of small problems (see split_tiles): up to half
// a round of tiles, and up to a quarter round.
#ifndef PTA_SPLIT_MIN_K
#define PTA_SPLIT_MIN_K 4096
#endif
#ifndef PTA_SPLIT_MIN_K_QUARTER
#define PTA_SPLIT_MIN_K_QUARTER 3072
#endif

namespace pta {
using namespace gemm_detail;

// K split for problems of at most half a round of tiles (one 256 x 256 tile
// per CU and round) and K >= 4096, or at most a quarter round and K >= 3072:
// every tile runs as two half-K workgroups whose fp32 partials meet in the
// workspace, so twice as many CUs work.  The hand-over (256 KB written and
// read per tile) costs a fixed ~6-10 us, so a shorter K runs whole
// (kernel-trace medians, split / whole; 108 tiles: K = 2048 1.22-1.27, 3072
// 1.01-1.04, 4096 0.92-0.98, 6144 0.78-0.80; 128 tiles: 2048 1.14-1.22, 3072
// 0.99-1.00; 64 tiles: 2048 1.02-1.03, 3072 0.84, 4096 0.78-0.81).  Splitting
// the last round of larger problems measured no faster (headline
// 4096x18432x7168: +1%), so those run whole.  Returns the number of split
// tiles (0: none).
int64_t split_tiles(int64_t tiles, int64_t K, int cus) {
    if (K % BK != 0 || tiles <= 0 || cus <= 0 || 2 * tiles > cus) return 0;
    const int64_t kmin = 4 * tiles <= cus ? PTA_SPLIT_MIN_K_QUARTER : PTA_SPLIT_MIN_K;
    return K >= kmin ? tiles : 0;
}

constexpr int64_t SPLIT_TILE_BYTES = int64_t(BM) * BN * 4;

// byte offset of the status word in a K-split workspace for `n` split tiles
// (after the fp32 partial tiles and one tag each)
int64_t split_status_offset(int64_t n) { return n * SPLIT_TILE_BYTES + cdiv(n * 8, 256) * 256; }

// workspace bytes for `n` split tiles (partial tiles, tags, status word)
int64_t split_ws_bytes(int64_t n) { return n > 0 ? split_status_offset(n) + 256 : 0; }

// Entry used by the dense and grouped front ends: NT problem fully described.
// split_ws: workspace of split_ws_bytes(split_tiles(...)) bytes, or NULL (no
// K split); split_ws_offset: its byte offset in the caller's workspace.
int gemm_nt_launch(const uint8_t *a, int fa, int64_t lda, const uint8_t *b, int fb, int64_t ldb,
                   void *c, int out_dt, int64_t ldc, int64_t M, int64_t N, int64_t K, int sm,
                   bool a2d, bool b2d, const void *sa, int64_t sa_m, int64_t sa_k, int64_t sa_bytes,
                   const void *sb, int64_t sb_m, int64_t sb_k, int64_t sb_bytes, hipStream_t st,
                   uint8_t *split_ws = nullptr, int64_t split_ws_offset = 0) {
    GemmArgs g{};
    g.a = a; g.b = b; g.c = c; g.M = M; g.N = N; g.K = K; g.lda = lda; g.ldb = ldb; g.ldc = ldc;
    g.sa = sa; g.sb = sb; g.sa_m = sa_m; g.sa_k = sa_k; g.sb_m = sb_m; g.sb_k = sb_k;
    g.sa_bytes = sa_bytes; g.sb_bytes = sb_bytes;
    if (sm == SM_MX) { // row-major exponents unless a K-block stride is given
        if (g.sa_k == 0) g.sa_k = 4;
        if (g.sb_k == 0) g.sb_k = 4;
    }
    g.tiles_m = static_cast<int>(cdiv(M, BM));
    g.tiles_n = static_cast<int>(cdiv(N, BN));
    g.group_m = 4;
    g.aligned_c = ((ldc * (out_dt == PTA_F32 ? 4 : 2)) % 16 == 0) && aligned16(c);
    if (split_ws != nullptr && !stream_capturing(st)) {
        // a graph would replay the call tag, so captured calls do not split
        const int64_t ns = split_tiles(int64_t(g.tiles_m) * g.tiles_n, K, device_cu_count());
        if (ns > 0) {
            const uint64_t tag = next_call_tag();
            const WaitPlan w   = wait_plan(tag, SPLIT_SPIN_LIMIT);
            g.split_count  = static_cast<int>(ns);
            g.split_ws     = reinterpret_cast<float *>(split_ws);
            g.split_tags   = reinterpret_cast<uint64_t *>(split_ws + ns * SPLIT_TILE_BYTES);
            g.split_tag    = tag;
            g.split_expect = w.expect;
            g.split_spin   = w.spin_limit;
            g.split_status = reinterpret_cast<uint64_t *>(split_ws + split_status_offset(ns));
            record_wait(g.split_tag, split_ws_offset + split_status_offset(ns));
        }
    }
    if (sm == SM_TENSOR) return dispatch_tensor(g, fa, fb, out_dt, st);
    if (sm == SM_ROW) return dispatch_row(g, fa, fb, out_dt, st);
    if (sm == SM_MX) return dispatch_mx(g, fa, fb, out_dt, st);
    if (a2d && b2d) {
        set_error("blockwise GEMM with 2-D scales on both operands is not supported");
        return PTA_ERR_UNSUPPORTED;
    }
    return dispatch_block(g, a2d, b2d, fa, fb, out_dt, st);
}

} // namespace pta

using namespace pta;

namespace {
int gran_to_sm(int gran) {
    switch (gran) {
    case PTA_TENSORWISE: return SM_TENSOR;
    case PTA_ROWWISE: return SM_ROW;
    case PTA_BLOCKWISE: return SM_BLOCK;
    case PTA_MX_BLOCKWISE: return SM_MX;
    default: return -1;
    }
}

// zero fill of an empty-K product (a kernel, not a memset, so that it may be
// recorded into a graph)
__global__ void zero_fill_kernel(uint8_t *c, int64_t bytes) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride) c[i] = 0;
}

int small_dispatch(gemm_small::SmallArgs &g, bool akm, bool bkm, int fa, int fb, int c_dtype, int sm,
                   hipStream_t st);

// pta_gemm_fp8 on the small-tile kernel: operands read in place (K-major for
// trans_a A and for non-trans_b B), scale strides as the reference's layouts
// give them, C^T by exchanging the operands.
int gemm_small_nt(const void *a, int a_fmt, const void *a_scale, int trans_a, const void *b, int b_fmt,
                  const void *b_scale, int trans_b, void *c, int c_dtype, int trans_c, int64_t M, int64_t N,
                  int64_t K, int sm, hipStream_t st) {
    using gemm_small::SmallArgs;
    const int64_t kb = cdiv(K, 128);
    SmallArgs     g{};
    g.a = static_cast<const uint8_t *>(a); g.b = static_cast<const uint8_t *>(b); g.c = c;
    g.M = M; g.N = N; g.K = K;
    g.lda = trans_a ? M : K; // A [K, M] or [M, K]
    g.ldb = trans_b ? K : N; // B [N, K] or [K, N]
    g.ldc = N;
    g.sa = a_scale; g.sb = b_scale;
    g.sa_bytes = 4; g.sb_bytes = 4;
    if (sm == SM_ROW) { g.sa_bytes = M * 4; g.sb_bytes = N * 4; }
    if (sm == SM_BLOCK) {
        // A: [M, K/128] or [K/128, M]; B: [N/128, K/128] (NT), [K/128, N/128] (NN), [K/128, N] (TN)
        if (!trans_a) { g.sa_m = kb; g.sa_k = 1; } else { g.sa_m = 1; g.sa_k = M; }
        if (trans_b) { g.b2d = 1; g.sb_m = kb; g.sb_k = 1; }
        else if (!trans_a) { g.b2d = 1; g.sb_m = 1; g.sb_k = cdiv(N, 128); }
        else { g.b2d = 0; g.sb_m = 1; g.sb_k = N; }
        g.sa_bytes = M * kb * 4;
        g.sb_bytes = (g.b2d ? cdiv(N, 128) : N) * kb * 4;
    }
    if (sm == SM_MX) {
        g.sa_m = K / 32; g.sb_m = K / 32; g.sa_k = 4; g.sb_k = 4;
        g.sa_bytes = M * (K / 32); g.sb_bytes = N * (K / 32);
    }
    bool akm = trans_a != 0, bkm = trans_b == 0;
    int  fa = a_fmt, fb = b_fmt;
    if (trans_c) { // C^T[n, m] = sum_k B(n, k) A(m, k)
        std::swap(g.a, g.b); std::swap(g.lda, g.ldb); std::swap(g.M, g.N);
        std::swap(g.sa, g.sb); std::swap(g.sa_m, g.sb_m); std::swap(g.sa_k, g.sb_k);
        std::swap(g.sa_bytes, g.sb_bytes); std::swap(g.a2d, g.b2d);
        std::swap(akm, bkm); std::swap(fa, fb);
        g.ldc = M;
    }
    return small_dispatch(g, akm, bkm, fa, fb, c_dtype, sm, st);
}

// Tile choice, tile order and launch of the small-tile kernel for a problem
// in the NT view (g without tile, tiles_*, group_m and aligned_c).
int small_dispatch(gemm_small::SmallArgs &g, bool akm, bool bkm, int fa, int fb, int c_dtype, int sm,
                   hipStream_t st) {
    // the largest tile whose grid still covers the CUs (a K-major operand's
    // row stride must be a multiple of the tile's bytes per K row and thread)
    using gemm_small::TILE_32x64;
    using gemm_small::TILE_64x64;
    using gemm_small::TILE_128x128;
    const int64_t t128 = cdiv(g.M, 128) * cdiv(g.N, 128), t64 = cdiv(g.M, 64) * cdiv(g.N, 64);
    const bool    ok128 = (!akm || g.lda % 16 == 0) && (!bkm || g.ldb % 16 == 0);
    g.tile = (t128 >= PTA_SMALL_T128_MIN && ok128) ? TILE_128x128 : (t64 >= PTA_SMALL_T64_MIN ? TILE_64x64 : TILE_32x64);
#if PTA_SMALL_FORCE_TILE >= 0
    g.tile = PTA_SMALL_FORCE_TILE;
    if (g.tile == TILE_128x128 && !ok128) g.tile = TILE_64x64;
#endif
    const int tbm = g.tile == TILE_128x128 ? 128 : (g.tile == TILE_64x64 ? 64 : 32);
    const int tbn = g.tile == TILE_128x128 ? 128 : 64;
    g.tiles_m = static_cast<int>(cdiv(g.M, tbm));
    g.tiles_n = static_cast<int>(cdiv(g.N, tbn));
    // about square per-XCD tile blocks: group_m = 2^floor(log2(sqrt(tiles / 8)))
    g.group_m = 1;
    while (4 * g.group_m * g.group_m * 8 <= int64_t(g.tiles_m) * g.tiles_n && 2 * g.group_m <= g.tiles_m) g.group_m *= 2;
    g.aligned_c = ((g.ldc * (c_dtype == PTA_F32 ? 4 : 2)) % 16 == 0) && aligned16(g.c);
    switch (sm) {
    case SM_TENSOR: return gemm_small::dispatch_small_tensor(g, akm, bkm, fa, fb, c_dtype, st);
    case SM_ROW: return gemm_small::dispatch_small_row(g, akm, bkm, fa, fb, c_dtype, st);
    case SM_BLOCK: return gemm_small::dispatch_small_block(g, akm, bkm, fa, fb, c_dtype, st);
    default: return gemm_small::dispatch_small_mx(g, fa, fb, c_dtype, st);
    }
}
} // namespace

// K-contiguous blockwise problems that the small-tile kernel would run on
// 128 x 128 tiles are faster on the 256 x 256 kernel (2048^3: 24.7 against
// 31.6 us, 2048 x 2048 x 1024: 15.6 against 19.9; tensorwise and MX are not:
// 21.3 against 19.7 and 23.9 against 24.5 us at 2048^3).
static bool block_on_128_tiles(int64_t M, int64_t N, int sm) {
    return sm == SM_BLOCK && cdiv(M, 128) * cdiv(N, 128) >= PTA_SMALL_T128_MIN;
}

// Whether pta_gemm_fp8 takes the small-tile kernel: few large tiles, K-major
// operands with a row stride that is a multiple of 8 (8-byte K-row loads), and
// every operand offset of the kernel within 32 bits.
static bool small_path(int64_t M, int64_t N, int64_t K, int trans_a, int trans_b, int sm) {
    const bool    kmajor = trans_a || !trans_b;
    const int64_t tiles  = cdiv(M, BM) * cdiv(N, BN);
    if (tiles >= (kmajor ? PTA_SMALL_MAX_TILES_KMAJOR : PTA_SMALL_MAX_TILES)) return false;
    // K-contiguous operands, a quarter of a round of 256 x 256 tiles or more
    // and a long K: the large tiles with the K split are faster (blockwise
    // 1024x4096x4096: 62 -> 45 us; at K = 2048 or with fewer tiles they are not)
    if (!kmajor && tiles >= 48 && K >= 4096 && K % 128 == 0) return false;
    if (!kmajor && block_on_128_tiles(M, N, sm)) return false;
    const int64_t lim = int64_t(1) << 30;
    if (trans_a ? (M % 8 != 0 || (K + 1024) * M >= lim) : 64 * K >= lim) return false;
    if (!trans_b ? (N % 8 != 0 || (K + 1024) * N >= lim) : 64 * K >= lim) return false;
    return true;
}

extern "C" size_t pta_gemm_fp8_workspace_size(int64_t M, int64_t N, int64_t K, int trans_a,
                                              int trans_b, int granularity) {
    if (small_path(M, N, K, trans_a, trans_b, gran_to_sm(granularity))) return 0;
    size_t ws = 0;
    if (trans_a) ws += static_cast<size_t>(cdiv(M * K, 256) * 256);
    if (!trans_b) ws += static_cast<size_t>(cdiv(N * K, 256) * 256);
    ws += static_cast<size_t>(split_ws_bytes(split_tiles(cdiv(M, BM) * cdiv(N, BN), K, device_cu_count())));
    return ws;
}

extern "C" int pta_gemm_fp8(const void *a, int a_fmt, const void *a_scale, int trans_a, const void *b,
                            int b_fmt, const void *b_scale, int trans_b, void *c, int c_dtype,
                            int trans_c, int64_t M, int64_t N, int64_t K, int granularity,
                            void *workspace, size_t workspace_bytes, pta_stream_t stream) {
    clear_error();
    const int sm = gran_to_sm(granularity);
    PTA_CHECK_ARG(sm >= 0, "unknown granularity %d", granularity);
    PTA_CHECK_ARG(a && b && c && a_scale && b_scale, "NULL pointer argument");
    PTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "negative shape");
    PTA_CHECK_ARG((a_fmt == PTA_E4M3 || a_fmt == PTA_E5M2) && (b_fmt == PTA_E4M3 || b_fmt == PTA_E5M2),
                  "unsupported fp8 format");
    PTA_CHECK_ARG(c_dtype == PTA_BF16 || c_dtype == PTA_F16 || c_dtype == PTA_F32, "unsupported output dtype");
    PTA_CHECK_ARG(K % 16 == 0, "K must be a multiple of 16 (got %lld)", (long long)K);
    PTA_CHECK_ARG(!(trans_a && trans_b), "the TT layout is not supported");
    if (sm == SM_MX) {
        PTA_CHECK_ARG(!trans_a && trans_b, "MX_BLOCKWISE supports the NT layout only");
        PTA_CHECK_ARG(K % 128 == 0, "MX_BLOCKWISE needs K %% 128 == 0");
    }
    if (M == 0 || N == 0) return PTA_OK;
    PTA_CHECK_ARG(aligned16(a) && aligned16(b), "A and B must be 16-byte aligned");
    hipStream_t st = as_stream(stream);
    if (K == 0) {
        const size_t eb = c_dtype == PTA_F32 ? 4 : 2;
        zero_fill_kernel<<<256, 256, 0, st>>>(static_cast<uint8_t *>(c), M * N * static_cast<int64_t>(eb));
        PTA_CHECK_LAUNCH();
        return PTA_OK;
    }
    const size_t need = pta_gemm_fp8_workspace_size(M, N, K, trans_a, trans_b, granularity);
    PTA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                  "workspace of %zu bytes required", need);
    if (small_path(M, N, K, trans_a, trans_b, sm))
        return gemm_small_nt(a, a_fmt, a_scale, trans_a, b, b_fmt, b_scale, trans_b, c, c_dtype, trans_c, M, N, K,
                             sm, st);

    // ---- reduce to NT: A' [M, K] K-contiguous, B' [N, K] K-contiguous ------
    const uint8_t *ap = static_cast<const uint8_t *>(a);
    const uint8_t *bp = static_cast<const uint8_t *>(b);
    uint8_t       *wsp = static_cast<uint8_t *>(workspace);
    if (trans_a) { // A stored [K, M]
        if (int rc = pta_transpose_u8(a, 1, K, M, wsp, stream)) return rc;
        ap = wsp;
        wsp += cdiv(M * K, 256) * 256;
    }
    if (!trans_b) { // B stored [K, N]
        if (int rc = pta_transpose_u8(b, 1, K, N, wsp, stream)) return rc;
        bp = wsp;
        wsp += cdiv(N * K, 256) * 256;
    }
    // what remains of the workspace holds the K split's partial tiles
    uint8_t      *split_ws  = split_tiles(cdiv(M, BM) * cdiv(N, BN), K, device_cu_count()) > 0 ? wsp : nullptr;
    const int64_t split_off = workspace != nullptr ? wsp - static_cast<uint8_t *>(workspace) : 0;
    // scale strides in the NT view
    bool    a2d = false, b2d = false;
    int64_t sa_m = 0, sa_k = 0, sb_m = 0, sb_k = 0;
    const int64_t kb = cdiv(K, 128);
    if (sm == SM_BLOCK) {
        if (!trans_a) { sa_m = kb; sa_k = 1; }     // [M, K/128]
        else { sa_m = 1; sa_k = M; }               // [K/128, M]
        if (trans_b) { b2d = true; sb_m = kb; sb_k = 1; }                 // [N/128, K/128]
        else if (!trans_a) { b2d = true; sb_m = 1; sb_k = cdiv(N, 128); } // NN: [K/128, N/128]
        else { b2d = false; sb_m = 1; sb_k = N; }                         // TN: [K/128, N]
    } else if (sm == SM_MX) {
        sa_m = K / 32; sb_m = K / 32; sa_k = 4; sb_k = 4;
    }
    // extent of each scale array in bytes
    int64_t sa_bytes = 4, sb_bytes = 4;
    if (sm == SM_ROW) { sa_bytes = M * 4; sb_bytes = N * 4; }
    if (sm == SM_BLOCK) {
        sa_bytes = M * kb * 4;
        sb_bytes = (b2d ? cdiv(N, 128) : N) * kb * 4;
    }
    if (sm == SM_MX) { sa_bytes = M * (K / 32); sb_bytes = N * (K / 32); }
    if (!trans_c) {
        return gemm_nt_launch(ap, a_fmt, K, bp, b_fmt, K, c, c_dtype, N, M, N, K, sm, a2d, b2d,
                              a_scale, sa_m, sa_k, sa_bytes, b_scale, sb_m, sb_k, sb_bytes, st, split_ws,
                              split_off);
    }
    // C^T[n, m] = sum_k B'[n,k] A'[m,k]: swap the operands
    return gemm_nt_launch(bp, b_fmt, K, ap, a_fmt, K, c, c_dtype, M, N, M, K, sm, b2d, a2d,
                          b_scale, sb_m, sb_k, sb_bytes, a_scale, sa_m, sa_k, sa_bytes, st, split_ws, split_off);
}

// Whether the kernel-choosing strided entry takes the small-tile kernel: the
// NT rule of small_path, with the operands' row strides (and the scale
// extents) in 32-bit reach of the small kernel's buffer offsets.
static bool strided_small_path(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t sa_bytes,
                               int64_t sb_bytes, int sm) {
    const int64_t tiles = cdiv(M, BM) * cdiv(N, BN);
    if (tiles >= PTA_SMALL_MAX_TILES) return false;
    if (tiles >= 48 && K >= 4096 && K % 128 == 0) return false; // the K split is faster there
    if (block_on_128_tiles(M, N, sm)) return false;
    const int64_t lim = int64_t(1) << 30;
    return 64 * lda < lim && 64 * ldb < lim && sa_bytes < 2 * lim && sb_bytes < 2 * lim;
}

static size_t strided_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t sa_bytes,
                               int64_t sb_bytes, int sm) {
    if (strided_small_path(M, N, K, lda, ldb, sa_bytes, sb_bytes, sm)) return 0;
    return static_cast<size_t>(split_ws_bytes(split_tiles(cdiv(M, BM) * cdiv(N, BN), K, device_cu_count())));
}

// choose: pick the small-tile kernel or the K split as pta_gemm_fp8 does
// (workspace of strided_ws_bytes); otherwise always the 256 x 256 kernel.
static int nt_strided(const void *a, int a_fmt, int64_t lda, const void *b, int b_fmt, int64_t ldb, void *c,
                      int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K, int granularity,
                      const void *a_scale, int64_t sa_m, int64_t sa_k, int a_scale_2d, int64_t a_scale_bytes,
                      const void *b_scale, int64_t sb_m, int64_t sb_k, int b_scale_2d, int64_t b_scale_bytes,
                      bool choose, void *workspace, size_t workspace_bytes, pta_stream_t stream) {
    clear_error();
    const int sm = gran_to_sm(granularity);
    PTA_CHECK_ARG(sm >= 0, "unknown granularity %d", granularity);
    PTA_CHECK_ARG(a && b && c && a_scale && b_scale, "NULL pointer argument");
    PTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && lda >= K && ldb >= K && ldc >= N, "bad shape / strides");
    PTA_CHECK_ARG((a_fmt == PTA_E4M3 || a_fmt == PTA_E5M2) && (b_fmt == PTA_E4M3 || b_fmt == PTA_E5M2),
                  "unsupported fp8 format");
    PTA_CHECK_ARG(c_dtype == PTA_BF16 || c_dtype == PTA_F16 || c_dtype == PTA_F32, "unsupported output dtype");
    PTA_CHECK_ARG(K % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0, "K and row strides must be multiples of 16");
    PTA_CHECK_ARG(aligned16(a) && aligned16(b), "A and B must be 16-byte aligned");
    PTA_CHECK_ARG(!(a_scale_2d && b_scale_2d), "2-D scales on both operands are not supported");
    if (sm == SM_MX) {
        PTA_CHECK_ARG(K % 128 == 0, "MX_BLOCKWISE needs K %% 128 == 0");
        PTA_CHECK_ARG(sa_m % 4 == 0 && sa_k % 4 == 0 && sb_m % 4 == 0 && sb_k % 4 == 0 && sa_m >= 0 &&
                          sa_k >= 0 && sb_m >= 0 && sb_k >= 0,
                      "MX exponent strides must be non-negative multiples of 4");
        const int64_t nkb = K / 128, ska = sa_k ? sa_k : 4, skb = sb_k ? sb_k : 4;
        PTA_CHECK_ARG(M == 0 || N == 0 || ((M - 1) * sa_m + (nkb - 1) * ska + 4 <= a_scale_bytes &&
                                           (N - 1) * sb_m + (nkb - 1) * skb + 4 <= b_scale_bytes),
                      "MX exponent arrays are smaller than the strides address");
    }
    if (M == 0 || N == 0 || K == 0) {
        PTA_CHECK_ARG(K != 0 || M == 0 || N == 0, "K == 0 is not supported by the strided entry");
        return PTA_OK;
    }
    hipStream_t st       = as_stream(stream);
    uint8_t    *split_ws = nullptr;
    if (choose) {
        const size_t need = strided_ws_bytes(M, N, K, lda, ldb, a_scale_bytes, b_scale_bytes, sm);
        PTA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                      "workspace of %zu bytes required", need);
        if (strided_small_path(M, N, K, lda, ldb, a_scale_bytes, b_scale_bytes, sm)) {
            gemm_small::SmallArgs g{};
            g.a = static_cast<const uint8_t *>(a); g.b = static_cast<const uint8_t *>(b); g.c = c;
            g.M = M; g.N = N; g.K = K; g.lda = lda; g.ldb = ldb; g.ldc = ldc;
            g.sa = a_scale; g.sb = b_scale; g.sa_m = sa_m; g.sa_k = sa_k; g.sb_m = sb_m; g.sb_k = sb_k;
            g.sa_bytes = a_scale_bytes; g.sb_bytes = b_scale_bytes;
            g.a2d = a_scale_2d != 0; g.b2d = b_scale_2d != 0;
            if (sm == SM_MX) { // row-major exponents unless a K-block stride is given
                if (g.sa_k == 0) g.sa_k = 4;
                if (g.sb_k == 0) g.sb_k = 4;
            }
            return small_dispatch(g, false, false, a_fmt, b_fmt, c_dtype, sm, st);
        }
        if (need > 0) split_ws = static_cast<uint8_t *>(workspace);
    }
    return gemm_nt_launch(static_cast<const uint8_t *>(a), a_fmt, lda, static_cast<const uint8_t *>(b), b_fmt,
                          ldb, c, c_dtype, ldc, M, N, K, sm, a_scale_2d != 0, b_scale_2d != 0, a_scale, sa_m,
                          sa_k, a_scale_bytes, b_scale, sb_m, sb_k, b_scale_bytes, st, split_ws);
}

extern "C" int pta_gemm_fp8_nt_strided(const void *a, int a_fmt, int64_t lda, const void *b, int b_fmt,
                                       int64_t ldb, void *c, int c_dtype, int64_t ldc, int64_t M,
                                       int64_t N, int64_t K, int granularity, const void *a_scale,
                                       int64_t sa_m, int64_t sa_k, int a_scale_2d,
                                       int64_t a_scale_bytes, const void *b_scale, int64_t sb_m,
                                       int64_t sb_k, int b_scale_2d, int64_t b_scale_bytes,
                                       pta_stream_t stream) {
    return nt_strided(a, a_fmt, lda, b, b_fmt, ldb, c, c_dtype, ldc, M, N, K, granularity, a_scale, sa_m, sa_k,
                      a_scale_2d, a_scale_bytes, b_scale, sb_m, sb_k, b_scale_2d, b_scale_bytes, false, nullptr,
                      0, stream);
}

extern "C" size_t pta_gemm_fp8_nt_strided_ws_size(int64_t M, int64_t N, int64_t K, int granularity, int64_t lda,
                                                  int64_t ldb, int64_t a_scale_bytes, int64_t b_scale_bytes) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return strided_ws_bytes(M, N, K, lda, ldb, a_scale_bytes, b_scale_bytes, gran_to_sm(granularity));
}

extern "C" int pta_gemm_fp8_nt_strided_ws(const void *a, int a_fmt, int64_t lda, const void *b, int b_fmt,
                                          int64_t ldb, void *c, int c_dtype, int64_t ldc, int64_t M,
                                          int64_t N, int64_t K, int granularity, const void *a_scale,
                                          int64_t sa_m, int64_t sa_k, int a_scale_2d,
                                          int64_t a_scale_bytes, const void *b_scale, int64_t sb_m,
                                          int64_t sb_k, int b_scale_2d, int64_t b_scale_bytes,
                                          void *workspace, size_t workspace_bytes, pta_stream_t stream) {
    return nt_strided(a, a_fmt, lda, b, b_fmt, ldb, c, c_dtype, ldc, M, N, K, granularity, a_scale, sa_m, sa_k,
                      a_scale_2d, a_scale_bytes, b_scale, sb_m, sb_k, b_scale_2d, b_scale_bytes, true, workspace,
                      workspace_bytes, stream);
}
