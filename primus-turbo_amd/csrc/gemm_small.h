// Small- and mid-size FP8 GEMM for gfx950 (MI355X).
//
// The large-tile kernel (gemm_kernel.h) gives each workgroup a 256 x 256 tile
// and walks K serially; a problem with few such tiles (512 x 1024, say: 8
// tiles) leaves most of the 256 CUs idle and is bound by the latency of its
// long K loop.  Here a workgroup of four waves (2 x 2) owns a 32 x 64, 64 x 64
// or 128 x 128 tile (chosen per problem so the grid covers the CUs), and
// either operand may be read K-contiguous ([rows, K]) or K-major ([K, rows]):
// a K-major tile is transposed in registers (4 x 4 byte blocks, v_perm) on its
// way into LDS, so the NN and TN layouts need no separate transpose pass.
//
// Pipeline, per thread: RING K blocks (128 deep) of both operands and their
// scales are in flight in registers at once (buffer loads; blocks past K and
// rows past the operand's extent read as zeros).  Each block is written to one
// of two LDS stages, one barrier per block, and consumed by the wave's grid of
// v_mfma 16x16x128 with the fragment conventions of the large-tile kernel: the
// MFMA is issued with the B tile first, so lane l holds C[m = l%16][n =
// 4*(l/16) .. +3] of each 16 x 16 sub-tile.
//
// Scaling granularities as in the large-tile kernel (gemm_fp8_kernel.py
// :164-167, :524-528, :934-964 of the reference; MX with per-32-K E8M0
// exponents on the scaled MFMA): TENSORWISE / ROWWISE scale in the epilogue,
// BLOCKWISE scales each K block's MFMA partial into the fp32 accumulator, MX
// passes the exponents to the MFMA.
#pragma once
#include "gemm_kernel.h"

namespace pta {
namespace gemm_small {
using gemm_detail::frag;
using gemm_detail::rsrc_t;
using gemm_detail::SM_BLOCK;
using gemm_detail::SM_MX;
using gemm_detail::SM_ROW;
using gemm_detail::SM_TENSOR;
using gemm_detail::store4;
using gemm_detail::v4f;
using gemm_detail::v8i;

constexpr int SBK   = 128; // K block
constexpr int SNTHR = 256; // four waves, 2 x 2 over the tile
constexpr int RING  = 2;   // K blocks in flight per thread (2, 4 and 8 measured: 2 is best)

// Workgroup tile shapes.  Per wave (SBM/2) x (SBN/2) of C = STM x STN MFMA
// sub-tiles; per thread and K block, SBM/2 bytes of A and SBN/2 bytes of B.
enum : int { TILE_32x64 = 0, TILE_64x64 = 1, TILE_128x128 = 2 };
template <int TILE>
struct STile {
    static constexpr int BM  = TILE == TILE_128x128 ? 128 : (TILE == TILE_64x64 ? 64 : 32);
    static constexpr int BN  = TILE == TILE_128x128 ? 128 : 64;
    static constexpr int WTM = BM / 2, WTN = BN / 2;
    static constexpr int STM = WTM / 16, STN = WTN / 16;
    static constexpr int A_BYTES = BM * SBK, B_BYTES = BN * SBK;
    static constexpr int STAGE   = A_BYTES + B_BYTES;
};

// Problem in the NT view: C[m, n] = sum_k A(m, k) B(n, k), with A(m, k) at
// a[m * lda + k] (K-contiguous) or a[k * lda + m] (K-major), likewise B.
struct SmallArgs {
    const uint8_t *a, *b;
    void          *c;
    int64_t        M, N, K, lda, ldb, ldc;
    const void    *sa, *sb;
    // blockwise: scale(r, kb) at s[idx(r) * s_m + kb * s_k] with idx(r) = r / 128
    // for a 2-D (128 x 128 block) operand, r otherwise; MX: exponent byte of
    // row r, 32-K block q at s[r * s_m + (q / 4) * s_k + q % 4]
    int64_t        sa_m, sa_k, sb_m, sb_k, sa_bytes, sb_bytes;
    int            a2d, b2d;
    int            tile;    // TILE_* of this launch
    int            tiles_m, tiles_n;
    int            group_m; // tile rows per group of the tile order
    int            aligned_c;
};

// LDS layout of an operand tile: row r (an m or n) holds its 128 K bytes as
// eight 16-byte chunks, chunk c stored at position c ^ ((r ^ (r >> 3)) & 7).
// The 16 rows of an MFMA fragment read see distinct chunk positions within
// every 8 aligned rows, and the column writes of the K-major transpose (rows
// 4 to 16 apart) spread over the chunk positions as well.
__device__ __forceinline__ int soff(int row, int ch) { return row * SBK + ((ch ^ ((row ^ (row >> 3)) & 7)) << 4); }

// 32-bit offset that lies past any descriptor extent this kernel builds
constexpr int OOB = 0x7ffffff0;

// Buffer descriptor from wave-uniform values, built from scalar registers
// (readfirstlane) so that loads through it need no per-lane waterfall loop.
__device__ __forceinline__ rsrc_t tile_rsrc(const uint8_t *p, int64_t bytes) {
    const uint64_t a  = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void *u = reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0),
                                             __builtin_amdgcn_readfirstlane(static_cast<int32_t>(bytes)), 0x00020000);
}

// Operand tile of R rows starting at row r0: base pointer and extent.  A
// K-contiguous tile ends after its last valid row's K bytes; a K-major tile
// after the last K row's bytes up to the operand's row count rounded to 16
// (the row loads of up to 16 bytes stay whole; the host guarantees
// ld % 16 == 0 for a K-major operand, and rows <= ld).
template <bool KM, int R>
__device__ __forceinline__ rsrc_t operand_rsrc(const uint8_t *p, int64_t ld, int64_t r0, int64_t rows, int64_t K) {
    if constexpr (!KM) {
        const int64_t valid = min<int64_t>(rows - r0, R);
        return tile_rsrc(p + r0 * ld, (valid - 1) * ld + K);
    } else {
        const int64_t end = min<int64_t>((rows + 15) & ~int64_t(15), ld);
        return tile_rsrc(p + r0, (K - 1) * ld + end - r0);
    }
}

// One K block of an R-row operand tile, R/2 bytes per thread.
//   K-contiguous: rows t/8 + 32 q, 16-byte chunk t%8 of each.
//   K-major: K rows k0 + 4(t/8) .. +3, tile rows (R/8)(t%8) .. +R/8-1 of each.
template <bool KM, int R>
__device__ __forceinline__ void load_operand(rsrc_t r, int ld, int k0, int K, uint32_t (&v)[R / 8]) {
    const int t = threadIdx.x;
    if constexpr (!KM) {
        const int c = t & 7, row = t >> 3;
#pragma unroll
        for (int q = 0; q < R / 32; ++q) {
            int off = (row + 32 * q) * ld + k0 + 16 * c;
            if (k0 + 16 * c >= K) off = OOB; // past K: zeros (not the next row's bytes)
            const uint4 x = gemm_detail::bload16(r, off, 0);
            v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
        }
    } else {
        constexpr int W = R / 8; // bytes per K row and thread
        const int     rg = t & 7, kg = t >> 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // K rows past K start beyond the extent and read as zeros
            const int off = (k0 + 4 * kg + j) * ld + W * rg;
            if constexpr (W == 4) {
                v[j] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
            } else if constexpr (W == 8) {
                const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
                v[2 * j] = x.x; v[2 * j + 1] = x.y;
            } else {
                const uint4 x = gemm_detail::bload16(r, off, 0);
                v[4 * j] = x.x; v[4 * j + 1] = x.y; v[4 * j + 2] = x.z; v[4 * j + 3] = x.w;
            }
        }
    }
}

// Store one K block of an operand tile into LDS at T (see soff for the layout).
template <bool KM, int R>
__device__ __forceinline__ void write_operand(uint8_t *T, const uint32_t (&v)[R / 8]) {
    const int t = threadIdx.x;
    if constexpr (!KM) {
        const int c = t & 7, row = t >> 3;
#pragma unroll
        for (int q = 0; q < R / 32; ++q)
            *reinterpret_cast<uint4 *>(T + soff(row + 32 * q, c)) = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
        // v[j * H + h] holds K row kk + j, tile rows W rg + 4h .. +3 (one byte
        // each); transpose each 4 x 4 byte block so that a dword holds K
        // kk .. kk+3 of one row
        constexpr int W = R / 8, H = W / 4;
        const int     rg = t & 7, kk = 4 * (t >> 3);
        const int     ch = kk >> 4, w = kk & 15;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint32_t a = v[h], b = v[H + h], c = v[2 * H + h], d = v[3 * H + h];
            const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u); // a0 b0 a1 b1
            const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u); // a2 b2 a3 b3
            const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
            const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
            const uint32_t col[4] = {__builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u),  // a0 b0 c0 d0
                                     __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u),  // a1 b1 c1 d1
                                     __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u),
                                     __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u)};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<uint32_t *>(T + soff(W * rg + 4 * h + i, ch) + w) = col[i];
        }
    }
}

// Registers of one in-flight K block.
template <class TL>
struct Slot {
    uint32_t a[TL::BM / 8], b[TL::BN / 8];
    float    sa[TL::STM];      // BLOCKWISE: A scale of the lane's row in sub-tile i
    float    sb[TL::STN][4];   // BLOCKWISE: B scales of the lane's four columns in sub-tile j
    int      ea[TL::STM], eb[TL::STN]; // MX: exponent bytes of the lane's A / B rows
};

template <int SM, int FA, int FB, int OUT_DT, bool AKM, bool BKM, int TILE>
__global__ __launch_bounds__(SNTHR) void gemm_small_kernel(const SmallArgs g) {
    using TL = STile<TILE>;
    constexpr int SBM = TL::BM, SBN = TL::BN, WTM = TL::WTM, WTN = TL::WTN, STM = TL::STM, STN = TL::STN;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * TL::STAGE];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fg = lane >> 4;

    // Workgroups are dispatched round-robin over the 8 XCDs, and each XCD's
    // L2 starts the launch cold: its tiles are fetched from the memory-side
    // cache.  XCD x takes tile ids [x T/8, (x+1) T/8), and ids walk groups of
    // group_m tile rows column by column, so one XCD's tiles form a compact
    // block (group_m x T/(8 group_m)) and share A rows and B rows.
    int       id    = static_cast<int>(blockIdx.x);
    const int total = g.tiles_m * g.tiles_n;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    const int per_group = g.group_m * g.tiles_n;
    const int first_m   = id / per_group * g.group_m;
    const int gsz       = min(g.tiles_m - first_m, g.group_m);
    const int64_t m0 = static_cast<int64_t>(first_m + (id % per_group) % gsz) * SBM;
    const int64_t n0 = static_cast<int64_t>((id % per_group) / gsz) * SBN;
    const int64_t M = g.M, N = g.N, K = g.K;
    const int     nk = static_cast<int>((K + SBK - 1) / SBK);
    const int     Ki = static_cast<int>(K);

    const rsrc_t rA = operand_rsrc<AKM, SBM>(g.a, g.lda, m0, M, K);
    const rsrc_t rB = operand_rsrc<BKM, SBN>(g.b, g.ldb, n0, N, K);
    const int    lda = static_cast<int>(g.lda), ldb = static_cast<int>(g.ldb);

    // scale addressing: the lane's rows m (one per A sub-tile) and columns n
    // (four per B sub-tile), clamped into the operand so every read is in range
    const rsrc_t rSA = tile_rsrc(static_cast<const uint8_t *>(g.sa), g.sa_bytes);
    const rsrc_t rSB = tile_rsrc(static_cast<const uint8_t *>(g.sb), g.sb_bytes);
    int          sa_vo[STM], sb_vo[STN][4];
#pragma unroll
    for (int i = 0; i < STM; ++i) {
        const int64_t m = min<int64_t>(m0 + wm * WTM + 16 * i + fr, M - 1);
        if constexpr (SM == SM_BLOCK) sa_vo[i] = static_cast<int>((g.a2d ? (m >> 7) : m) * g.sa_m) * 4;
        else if constexpr (SM == SM_MX) sa_vo[i] = static_cast<int>(m * g.sa_m) + fg;
    }
#pragma unroll
    for (int j = 0; j < STN; ++j) {
        if constexpr (SM == SM_BLOCK) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t nc = min<int64_t>(n0 + wn * WTN + 16 * j + 4 * fg + r, N - 1);
                sb_vo[j][r] = static_cast<int>((g.b2d ? (nc >> 7) : nc) * g.sb_m) * 4;
            }
        } else if constexpr (SM == SM_MX) {
            const int64_t n = min<int64_t>(n0 + wn * WTN + 16 * j + fr, N - 1);
            sb_vo[j][0] = static_cast<int>(n * g.sb_m) + fg;
        }
    }

    auto load_slot = [&](int kb, Slot<TL> &s) {
        const int k0 = kb * SBK;
        load_operand<AKM, SBM>(rA, lda, k0, Ki, s.a);
        load_operand<BKM, SBN>(rB, ldb, k0, Ki, s.b);
        if constexpr (SM == SM_BLOCK) {
            const int ka = static_cast<int>(kb * g.sa_k) * 4, kbb = static_cast<int>(kb * g.sb_k) * 4;
#pragma unroll
            for (int i = 0; i < STM; ++i) s.sa[i] = gemm_detail::bload_f32(rSA, sa_vo[i], ka);
#pragma unroll
            for (int j = 0; j < STN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) s.sb[j][r] = gemm_detail::bload_f32(rSB, sb_vo[j][r], kbb);
        } else if constexpr (SM == SM_MX) {
            const int ka = static_cast<int>(kb * g.sa_k), kbb = static_cast<int>(kb * g.sb_k);
#pragma unroll
            for (int i = 0; i < STM; ++i) s.ea[i] = gemm_detail::bload_u8(rSA, sa_vo[i], ka);
#pragma unroll
            for (int j = 0; j < STN; ++j) s.eb[j] = gemm_detail::bload_u8(rSB, sb_vo[j][0], kbb);
        }
    };

    // fragment offsets: rows wm*WTM + 16 i + fr of A, wn*WTN + 16 j + fr of B
    int aoff[STM][2], boff[STN][2];
#pragma unroll
    for (int i = 0; i < STM; ++i) {
        aoff[i][0] = soff(wm * WTM + 16 * i + fr, fg);
        aoff[i][1] = soff(wm * WTM + 16 * i + fr, 4 + fg);
    }
#pragma unroll
    for (int j = 0; j < STN; ++j) {
        boff[j][0] = TL::A_BYTES + soff(wn * WTN + 16 * j + fr, fg);
        boff[j][1] = TL::A_BYTES + soff(wn * WTN + 16 * j + fr, 4 + fg);
    }

    v4f acc[STN][STM];
#pragma unroll
    for (int j = 0; j < STN; ++j)
#pragma unroll
        for (int i = 0; i < STM; ++i) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};

    // Epilogue scales, read now: issued ahead of the operand loads, they are
    // long in registers when the epilogue needs them (a read there would cost
    // one more memory round trip).  Volatile: kept here, not sunk past the loop.
    constexpr int VOL = static_cast<int>(1u << 31);
    float ts = 1.0f, ra[STM] = {}, rb[STN][4] = {};
    if constexpr (SM == SM_TENSOR) {
        ts = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSA, 0, 0, VOL)) *
             __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, 0, 0, VOL));
    } else if constexpr (SM == SM_ROW) {
#pragma unroll
        for (int i = 0; i < STM; ++i) {
            const int m = static_cast<int>(min<int64_t>(m0 + wm * WTM + 16 * i + fr, M - 1));
            ra[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSA, 4 * m, 0, VOL));
        }
#pragma unroll
        for (int j = 0; j < STN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = static_cast<int>(min<int64_t>(n0 + wn * WTN + 16 * j + 4 * fg + r, N - 1));
                rb[j][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rSB, 4 * n, 0, VOL));
            }
    }

    // Block kb is consumed in iteration kb: its fragments are read from LDS
    // stage kb & 1, block kb + 1 is written from its ring slot into the other
    // stage while the MFMAs of block kb run, and one barrier per block then
    // publishes it.  The other stage is free: every wave read it (block kb - 1)
    // before the previous barrier.
    //
    // One loop issues every load, one slot per iteration in the same order on
    // every path (blocks past K load zeros, their compute is skipped), so the
    // compiler's wait counts see a fixed distance of RING - 1 slots between a
    // slot's loads and their use.  Its first pass (kb0 = -RING) fills the ring
    // and writes block 0: the slots keep one set of registers throughout, with
    // no peeled prologue whose register copies would wait for loads in flight.
    Slot<TL> ring[RING];
    float    sa[STM] = {}, sb[STN][4] = {}; // scales of the block being consumed
    int      ea[STM] = {}, eb[STN] = {};
    int      kb_first = -RING;
    asm volatile("" : "+s"(kb_first)); // opaque start: not peeled
    for (int kb0 = kb_first; kb0 < nk; kb0 += RING) {
#pragma unroll
        for (int s = 0; s < RING; ++s) {
            const int  kb    = kb0 + s;   // kb0 is a multiple of RING: slot kb % RING == s
            const int  sn    = (s + 1) % RING;
            const bool live  = kb >= 0 && kb < nk;
            const bool wlive = kb >= -1 && kb + 1 < nk;
            const uint8_t *S = smem + (s & 1) * TL::STAGE;
            uint8_t       *W = smem + ((s + 1) & 1) * TL::STAGE;
            v8i af[STM];
            if (live) {
#pragma unroll
                for (int i = 0; i < STM; ++i) af[i] = frag(S, aoff[i][0], aoff[i][1]);
            }
            // scales of block kb leave slot s before it is refilled
            float csa[STM], csb[STN][4];
            int   cea[STM], ceb[STN];
#pragma unroll
            for (int i = 0; i < STM; ++i) { csa[i] = sa[i]; cea[i] = ea[i]; }
#pragma unroll
            for (int j = 0; j < STN; ++j) {
                ceb[j] = eb[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) csb[j][r] = sb[j][r];
            }
            if (wlive) {
                write_operand<AKM, SBM>(W, ring[sn].a);
                write_operand<BKM, SBN>(W + TL::A_BYTES, ring[sn].b);
                if constexpr (SM == SM_BLOCK) {
#pragma unroll
                    for (int i = 0; i < STM; ++i) sa[i] = ring[sn].sa[i];
#pragma unroll
                    for (int j = 0; j < STN; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) sb[j][r] = ring[sn].sb[j][r];
                } else if constexpr (SM == SM_MX) {
#pragma unroll
                    for (int i = 0; i < STM; ++i) ea[i] = ring[sn].ea[i];
#pragma unroll
                    for (int j = 0; j < STN; ++j) eb[j] = ring[sn].eb[j];
                }
            }
            load_slot(kb + RING, ring[s]);
            if (live) {
#pragma unroll
                for (int j = 0; j < STN; ++j) {
                    const v8i bf = frag(S, boff[j][0], boff[j][1]);
#pragma unroll
                    for (int i = 0; i < STM; ++i) {
                        if constexpr (SM == SM_BLOCK) {
                            const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                bf, af[i], v4f{0.f, 0.f, 0.f, 0.f}, FB, FA, 0, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[j][i][r] += p[r] * (csa[i] * csb[j][r]);
                        } else if constexpr (SM == SM_MX) {
                            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                bf, af[i], acc[j][i], FB, FA, 0, ceb[j], 0, cea[i]);
                        } else {
                            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                bf, af[i], acc[j][i], FB, FA, 0, 0, 0, 0);
                        }
                    }
                }
            }
            if (wlive) __syncthreads();
        }
    }

    // ---- epilogue: scale and store, 4 consecutive n per lane and sub-tile ----
#pragma unroll
    for (int j = 0; j < STN; ++j) {
        const int64_t n = n0 + wn * WTN + 16 * j + 4 * fg;
#pragma unroll
        for (int i = 0; i < STM; ++i) {
            const int64_t m = m0 + wm * WTM + 16 * i + fr;
            if (m >= M || n >= N) continue;
            float x[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[j][i][r];
                if constexpr (SM == SM_TENSOR) v = v * ts;
                if constexpr (SM == SM_ROW) v = v * ra[i] * rb[j][r];
                x[r] = v;
            }
            const bool full = g.aligned_c && (n + 4 <= N);
            store4<OUT_DT>(g.c, m * g.ldc + n, x[0], x[1], x[2], x[3], full, static_cast<int>(min<int64_t>(4, N - n)));
        }
    }
}

template <int SM, bool AKM, bool BKM, int FA, int FB, int OUT_DT>
int launch_small(const SmallArgs &g, hipStream_t st) {
    const uint32_t grid = static_cast<uint32_t>(g.tiles_m) * static_cast<uint32_t>(g.tiles_n);
    switch (g.tile) {
    case TILE_32x64: gemm_small_kernel<SM, FA, FB, OUT_DT, AKM, BKM, TILE_32x64><<<grid, SNTHR, 0, st>>>(g); break;
    case TILE_64x64: gemm_small_kernel<SM, FA, FB, OUT_DT, AKM, BKM, TILE_64x64><<<grid, SNTHR, 0, st>>>(g); break;
    default: gemm_small_kernel<SM, FA, FB, OUT_DT, AKM, BKM, TILE_128x128><<<grid, SNTHR, 0, st>>>(g); break;
    }
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

template <int SM, bool AKM, bool BKM>
int small_fmt(const SmallArgs &g, int fa, int fb, int out_dt, hipStream_t st) {
#define PTA_S_OUT(FA_, FB_)                                                                        \
    if (out_dt == PTA_BF16) return launch_small<SM, AKM, BKM, FA_, FB_, PTA_BF16>(g, st);          \
    if (out_dt == PTA_F16) return launch_small<SM, AKM, BKM, FA_, FB_, PTA_F16>(g, st);            \
    return launch_small<SM, AKM, BKM, FA_, FB_, PTA_F32>(g, st);
    if (fa == PTA_E4M3 && fb == PTA_E4M3) { PTA_S_OUT(0, 0) }
    if (fa == PTA_E4M3 && fb == PTA_E5M2) { PTA_S_OUT(0, 1) }
    if (fa == PTA_E5M2 && fb == PTA_E4M3) { PTA_S_OUT(1, 0) }
    PTA_S_OUT(1, 1)
#undef PTA_S_OUT
}

// the operand layouts of one scale mode: NT reads both operands K-contiguous,
// NN a K-major B, TN both K-major, and C^T exchanges the operands
template <int SM>
int small_layouts(const SmallArgs &g, bool akm, bool bkm, int fa, int fb, int out_dt, hipStream_t st) {
    if (akm && bkm) return small_fmt<SM, true, true>(g, fa, fb, out_dt, st);
    if (akm) return small_fmt<SM, true, false>(g, fa, fb, out_dt, st);
    if (bkm) return small_fmt<SM, false, true>(g, fa, fb, out_dt, st);
    return small_fmt<SM, false, false>(g, fa, fb, out_dt, st);
}

// one translation unit per scale mode (parallel builds)
int dispatch_small_tensor(const SmallArgs &g, bool akm, bool bkm, int fa, int fb, int out_dt, hipStream_t st);
int dispatch_small_row(const SmallArgs &g, bool akm, bool bkm, int fa, int fb, int out_dt, hipStream_t st);
int dispatch_small_block(const SmallArgs &g, bool akm, bool bkm, int fa, int fb, int out_dt, hipStream_t st);
int dispatch_small_mx(const SmallArgs &g, int fa, int fb, int out_dt, hipStream_t st);

} // namespace gemm_small
} // namespace pta
