// Blockwise FP8 quantization on gfx950: 1 x 128 (row), 128 x 1 (col), dual,
// 128 x 128 weight tiles and the grouped "segment" variant.
//
// One workgroup (4 waves, 256 lanes) owns a 128 x 128 input tile.  Lane t owns
// 4 consecutive rows (4*(t>>3) .. +3) of a 16-column segment (16*(t&7) .. +15):
//   * bf16 input is read once with 16-byte loads (a wave covers 8 rows x 256 B);
//   * row amax = max over the lane's 16 values, then a transposing butterfly
//     over the 8 lanes of the row group (3 DPP steps, no LDS) that leaves each
//     lane one row's amax, so each lane divides once; a DPP broadcast hands
//     every lane its 4 rows' scales;
//   * col amax = max over the lane's 4 rows, then rotate-by-8 DPP inside each
//     16-lane row, then a 16 x 128 LDS table reduced by 128 lanes;
//   * the partial maxima are combined with integer max (exact: they are
//     non-negative and NaN-free);
//   * all 64 values stay in VGPRs between the reductions and the casts.
// Scale arithmetic follows the reference exactly (eps 1e-4, IEEE divides):
//   primus_turbo/triton/quantization/quant_blockwise.py:11-18 (1-D / dual)
//   csrc/kernels/quantization/quantization_blockwise.cu:298-308 (weight)
//   csrc/kernels/quantization/quantization_blockwise.cu:58-213 (segment)
#include "common.h"

namespace pta {

namespace {

constexpr int TILE = 128;
constexpr int NT   = 256;

enum : int {
    QB_ROW     = 1,  // 1 x 128 scales, q_row [M, N]
    QB_COL     = 2,  // 128 x 1 scales, q_col [M, N] or transposed
    QB_COL_T   = 4,  // q_col written as [N, M]
    QB_W2D     = 8,  // one scale per 128 x 128 tile (weight)
    QB_W2D_T   = 16, // weight bytes also written transposed [N, M]
    QB_SEGMENT = 32, // grouped rows: tile index is in 128-padded segment space
};

struct QBArgs {
    const void *x;
    int64_t     M, N;      // input rows / cols (per batch for W2D)
    int64_t     batch_stride_x;
    uint8_t    *q_row;     // ROW / W2D output
    float      *s_row;     // ROW: s_row[r * srow_m + kb * srow_k]
    int64_t     srow_m, srow_k;
    uint8_t    *q_col;     // COL output
    int64_t     ldt_col;   // COL_T: row stride of the transposed q_col [N, ldt_col]
    float      *s_col;     // COL: [mb, N]
    uint8_t    *q_t;       // W2D_T output
    float      *s_w;       // W2D: [B, mb, nb]
    // segment mode
    const int64_t *group_offs;  // [G+1]
    const int64_t *padded_offs; // [G+1]
    int64_t        G;
};

// Max of two partial maxima of |x|.  They start from +0, so they are +0 ..
// +inf, or NaN where the NaN-propagating max built them from a NaN input.
// Their bit patterns order as the values do and every NaN pattern lies above
// +inf's, so the integer max is exact and keeps a NaN; it needs none of the
// NaN-quieting the compiler puts in front of a float max of a lane-exchanged
// operand.
__device__ __forceinline__ float amax2(float a, float b) {
    return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// Cast of four values already scaled into range: no clamp.  Used where no
// input of the wave (or tile) is NaN or infinite: then |x| <= amax and the
// scale is max / amax rounded, so |x * scale| <= max (1 + 2^-23) and the
// round-to-nearest-even cast gives exactly the byte the clamped cast gives.
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

// NaN-propagating max of |x| (v_maximum3_f32): the partial maxima it builds
// are NaN when an input is NaN and equal the NaN-dropping amax otherwise.
__device__ __forceinline__ float pmax_abs(float a, float x) { return __builtin_elementwise_maximum(a, fabsf(x)); }

// special: the bit pattern of a non-negative partial maximum that is +inf or NaN
__device__ __forceinline__ bool special_amax(float a) { return __float_as_uint(a) >= 0x7f800000u; }

// wave max of partial maxima (integer max, exact as for amax2)
__device__ __forceinline__ float amax_wave(float v) {
    v = amax2(v, dpp_f<PTA_DPP_QUAD_XOR1>(v));
    v = amax2(v, dpp_f<PTA_DPP_QUAD_XOR2>(v));
    v = amax2(v, dpp_f<PTA_DPP_ROW_HALF_MIRROR>(v));
    v = amax2(v, dpp_f<PTA_DPP_ROW_MIRROR>(v));
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v      = amax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r      = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
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

// DPP controls beside the ones common to every kernel: broadcast lane 0 / lane
// 1 of each quad, rotate a 16-lane row by 8
constexpr int DPP_QUAD_BCAST0 = 0x00, DPP_QUAD_BCAST1 = 0x55, DPP_ROW_ROR8 = 0x128;

// 16-byte output store; non-temporal for streamed (larger than the MALL) inputs,
// whose outputs do not stay resident either.
template <bool NT_ST>
__device__ __forceinline__ void st16(void *dst, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = {a, b, c, d};
    if constexpr (NT_ST) __builtin_nontemporal_store(v, reinterpret_cast<v4u *>(dst));
    else *reinterpret_cast<v4u *>(dst) = v;
}

// STREAM: 0 plain accesses, 1 non-temporal input loads, 2 non-temporal output stores (plain loads).
// TPW: tiles per workgroup.  With 2, the workgroup's two halves (256 lanes
// each) take two neighbouring tiles of one tile row (row-major order) or one
// tile column (column-major order), so the workgroup reads 512-byte row
// segments; both halves run the same barriers (the tile-dependent branch of
// the weight mode is taken by both when either tile needs it).
template <int IN_DT, int FMT, int MODE, bool VEC, int STREAM, int TPW>
__global__ __launch_bounds__(NT * TPW) void quant_block_tile_kernel(QBArgs args) {
    const int     half  = TPW == 2 ? static_cast<int>(threadIdx.x >> 8) : 0;
    const int     t     = static_cast<int>(threadIdx.x) & (NT - 1);
    const int     lane  = t & 63;
    const int     wave  = t >> 6;
    const int     cseg  = t & 7;
    const int     rgrp  = t >> 3;
    // Tile order over the flat index (2^31 - 1 tiles at most).  Row-major:
    // consecutive workgroups walk the column tiles of one tile row, so the
    // workgroups that run together stream whole input rows.  Column-major:
    // they walk the tile rows of one column tile, so the transposed copy's
    // rows are written contiguously.  Measured (one box, alternating):
    // segment quant 388 us row-major / 404 column-major, 128 x 128 weight
    // 77.1 / 78.6; weight + transposed copy of 32 experts 376 / 363, headline
    // activation dual 22.4 / 21.9: the modes that write a transposed copy of
    // a non-grouped tensor take the column-major order.
    constexpr bool COLMAJOR = (MODE & QB_SEGMENT) == 0 && (MODE & (QB_COL_T | QB_W2D_T)) != 0;
    const int64_t M = args.M, N = args.N;
    // 32-bit index arithmetic: the launch holds at most 2^31 - 1 tiles (a
    // 64-bit division costs ~150 instructions ahead of the first load)
    const uint32_t tiles_n = static_cast<uint32_t>((N + TILE - 1) / TILE);
    const uint32_t tiles_m = gridDim.x * TPW / tiles_n;
    const uint32_t bx      = blockIdx.x * TPW + half;
    const int64_t  tm      = COLMAJOR ? bx % tiles_m : bx / tiles_n; // tile row (padded space for SEGMENT)
    const int64_t  tn      = COLMAJOR ? bx / tiles_m : bx % tiles_n;
    const int64_t batch = blockIdx.z;
    const int64_t n0 = tn * TILE + cseg * 16;

    // ---- map tile rows to input rows -------------------------------------
    int64_t row_base;      // input row of local row 0
    int64_t row_lo, row_hi; // valid input rows [row_lo, row_hi)
    int64_t pad_row0 = tm * TILE;
    if constexpr ((MODE & QB_SEGMENT) != 0) {
        const int64_t M_padded = args.padded_offs[args.G];
        if (pad_row0 >= M_padded) return;
        // the last g with padded_offs[g] <= pad_row0 owns a non-empty segment.
        // The offsets are non-decreasing, so the lanes' comparisons over 64
        // consecutive groups form a prefix and one ballot counts it: one round
        // of loads per 64 groups instead of a chain of dependent ones.
        int64_t g = 0;
        for (int64_t q0 = 0; q0 < args.G; q0 += 64) {
            const int64_t  q    = q0 + lane;
            const bool     le   = q < args.G && args.padded_offs[q] <= pad_row0;
            const int      cnt  = __popcll(__ballot(le));
            if (cnt > 0) g = q0 + cnt - 1;
            if (cnt < 64) break;
        }
        const int64_t orig_start = args.group_offs[g];
        const int64_t orig_end   = args.group_offs[g + 1];
        const int64_t pad_start  = args.padded_offs[g];
        row_base = orig_start + (pad_row0 - pad_start);
        row_lo   = orig_start;
        row_hi   = orig_end < M ? orig_end : M;
    } else {
        row_base = pad_row0;
        row_lo   = 0;
        row_hi   = M;
    }

    const char *xb = reinterpret_cast<const char *>(args.x) +
                     batch * args.batch_stride_x * InTraits<IN_DT>::bytes;

    // The lane's 4 x 16 inputs are loaded packed (8 VGPRs per row for 16-bit
    // types) and widened to fp32 where used.
    constexpr int CH = InTraits<IN_DT>::bytes; // 16-byte chunks per 16 elements
    uint4 raw[4][CH];
    bool  rvalid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = row_base + rgrp * 4 + i;
        rvalid[i]       = (r >= row_lo) && (r < row_hi);
        if (VEC) {
            // conditional global loads.  (Loads through a buffer resource that
            // spans the tile's valid rows, out-of-range rows reading as zero,
            // issue all eight back to back with no branches, and measured 1-3%
            // slower on the large streamed tensors, no faster on the rest.)
            typedef unsigned int v4u __attribute__((ext_vector_type(4)));
            const bool   ok = rvalid[i] && n0 + 16 <= N;
            const v4u   *p  = reinterpret_cast<const v4u *>(xb + (r * N + n0) * InTraits<IN_DT>::bytes);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                v4u w = v4u{0u, 0u, 0u, 0u};
                if (ok) {
                    if constexpr (STREAM == 1) w = __builtin_nontemporal_load(p + c);
                    else w = p[c];
                }
                raw[i][c] = make_uint4(w.x, w.y, w.z, w.w);
            }
        } else {
            // scalar path: widen then re-pack into the raw layout
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                uint32_t wd[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (IN_DT == PTA_F32) {
                        const int j = 4 * c + k;
                        wd[k] = (rvalid[i] && n0 + j < N) ? __float_as_uint(load_scalar<IN_DT>(xb, r * N + n0 + j)) : 0u;
                    } else {
                        const int  j0 = 8 * c + 2 * k;
                        const auto rd = [&](int j) -> uint32_t {
                            return (rvalid[i] && n0 + j < N) ? reinterpret_cast<const uint16_t *>(xb)[r * N + n0 + j] : 0u;
                        };
                        wd[k] = rd(j0) | (rd(j0 + 1) << 16);
                    }
                }
                raw[i][c] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
            }
        }
    }
    // element (i, j) of the lane's 4 x 16 block as fp32
    auto V = [&](int i, int j) -> float {
        if constexpr (IN_DT == PTA_F32) {
            const uint4    w  = raw[i][j >> 2];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
            return __uint_as_float(ws[j & 3]);
        } else {
            const uint4    w  = raw[i][j >> 3];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
            const uint32_t d  = ws[(j >> 1) & 3];
            if constexpr (IN_DT == PTA_BF16) return __uint_as_float((j & 1) ? (d & 0xffff0000u) : (d << 16));
            else return f16_bits_to_f32((j & 1) ? (d >> 16) : (d & 0xffffu));
        }
    };
    auto Q4 = [&](int i, int j, float sc) -> uint32_t {
        return qpack4<FMT>(V(i, j), V(i, j + 1), V(i, j + 2), V(i, j + 3), sc);
    };
    auto F4 = [&](int i, int j, float sc) -> uint32_t {
        return cast4<FMT>(V(i, j) * sc, V(i, j + 1) * sc, V(i, j + 2) * sc, V(i, j + 3) * sc);
    };
    // NaN or infinity among this wave's inputs: those waves take the
    // reference's NaN-dropping amax and the clamped cast, the rest the plain
    // cast (modes without a row pass keep the clamped cast throughout)
    bool wave_special = (MODE & (QB_ROW | QB_W2D)) == 0;

    __shared__ float    s_part_[TPW][16][TILE]; // col partial maxima (16 lane-rows x 128 cols)
    __shared__ float    s_cscale_[TPW][TILE];
    __shared__ float    s_wmax_[TPW][8];
    __shared__ uint32_t s_tr_[TPW][TILE][TILE / 4 + 1]; // transposed bytes, padded
    auto &s_part = s_part_[half];
    auto &s_cscale = s_cscale_[half];
    auto &s_wmax = s_wmax_[half];
    auto &s_tr = s_tr_[half];

    // ---- row direction ----------------------------------------------------
    if constexpr ((MODE & QB_ROW) != 0) {
        // The 8 lanes of a row group hold the same 4 rows.  A transposing
        // butterfly (partners 7 - c, c ^ 1, c ^ 2; c = cseg) leaves lane c with
        // the amax of one row, R(c) = 2 (c >= 4) + (c & 1), so each lane divides
        // once instead of once per row.
        const bool lo = cseg < 4, odd = (cseg & 1) != 0;
        auto row_amax = [&](const float (&a)[4]) -> float {
            float k0 = lo ? a[0] : a[2], k1 = lo ? a[1] : a[3];
            k0       = amax2(k0, dpp_f<PTA_DPP_ROW_HALF_MIRROR>(lo ? a[2] : a[0]));
            k1       = amax2(k1, dpp_f<PTA_DPP_ROW_HALF_MIRROR>(lo ? a[3] : a[1]));
            float am = odd ? k1 : k0;
            am       = amax2(am, dpp_f<PTA_DPP_QUAD_XOR1>(odd ? k0 : k1));
            return amax2(am, dpp_f<PTA_DPP_QUAD_XOR2>(am));
        };
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) a[i] = pmax_abs(a[i], V(i, j));
        }
        float am     = row_amax(a);
        wave_special = __ballot(special_amax(am)) != 0;
        if (wave_special) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) a[i] = fmaxf(a[i], absq(V(i, j)));
            }
            am = row_amax(a);
        }
        const float sc_own = scale_from_amax<FMT>(am, 1e-4f);
        {
            // lanes 0, 1, 4, 5 of the group store rows 0 .. 3's inverse scales
            const int64_t r = row_base + rgrp * 4 + (lo ? 0 : 2) + (odd ? 1 : 0);
            if ((cseg & 2) == 0 && r >= row_lo && r < row_hi) args.s_row[r * args.srow_m + tn * args.srow_k] = 1.0f / sc_own;
        }
        // every lane of the group takes the 4 rows' scales: lanes 0 / 1 of each
        // quad hold rows 0 / 1 (first quad) or 2 / 3 (second quad)
        const float x = dpp_f<DPP_QUAD_BCAST0>(sc_own), y = dpp_f<DPP_QUAD_BCAST1>(sc_own);
        const float xm = dpp_f<PTA_DPP_ROW_HALF_MIRROR>(x), ym = dpp_f<PTA_DPP_ROW_HALF_MIRROR>(y);
        const float sc[4] = {lo ? x : xm, lo ? y : ym, lo ? xm : x, lo ? ym : y};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t r = row_base + rgrp * 4 + i;
            if (rvalid[i]) {
                uint32_t w[4];
                if (wave_special) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) w[k] = Q4(i, 4 * k, sc[i]);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) w[k] = F4(i, 4 * k, sc[i]);
                }
                uint8_t *dst = args.q_row + r * N + n0;
                if (VEC && n0 + 16 <= N) {
                    st16<(STREAM == 2)>(dst, w[0], w[1], w[2], w[3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        if (n0 + j < N) dst[j] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
                }
            }
        }
    }

    // ---- column direction -------------------------------------------------
    if constexpr ((MODE & QB_COL) != 0) {
        // column maxima from +0, so that a column of NaN gives 0 and never NaN
        // (amax2); quieted inputs where the wave holds NaN or infinity.  Lanes l
        // and l ^ 8 share a column segment inside each 16-lane row.
        float ca[16];
        if (wave_special) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                ca[j] = fmaxf(fmaxf(0.0f, absq_fresh(V(0, j))), fmaxf(absq_fresh(V(1, j)), fmaxf(absq_fresh(V(2, j)), absq_fresh(V(3, j)))));
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                ca[j] = fmaxf(fmaxf(0.0f, fabsf(V(0, j))), fmaxf(fabsf(V(1, j)), fmaxf(fabsf(V(2, j)), fabsf(V(3, j)))));
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) ca[j] = amax2(ca[j], dpp_f<DPP_ROW_ROR8>(ca[j]));
        if ((lane & 15) < 8) {
            const int prow = wave * 4 + (lane >> 4);
#pragma unroll
            for (int j = 0; j < 16; ++j) s_part[prow][cseg * 16 + j] = ca[j];
        }
        __syncthreads();
        if (t < TILE) {
            float a = 0.0f;
#pragma unroll
            for (int p = 0; p < 16; ++p) a = amax2(a, s_part[p][t]);
            const float sc = scale_from_amax<FMT>(a, 1e-4f);
            s_cscale[t]    = sc;
            const int64_t n = tn * TILE + t;
            if (n < N) args.s_col[tm * N + n] = 1.0f / sc;
        }
        __syncthreads();
        float cs[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) cs[j] = s_cscale[cseg * 16 + j];

        if constexpr ((MODE & QB_COL_T) == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t prow = pad_row0 + rgrp * 4 + i; // output row (padded space)
                bool          ok;
                if constexpr ((MODE & QB_SEGMENT) != 0) ok = prow < args.padded_offs[args.G];
                else ok = rvalid[i];
                if (!ok) continue;
                uint32_t w[4];
                if (wave_special) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        w[k] = qpack4s<FMT>(V(i, 4 * k), V(i, 4 * k + 1), V(i, 4 * k + 2), V(i, 4 * k + 3), cs[4 * k],
                                            cs[4 * k + 1], cs[4 * k + 2], cs[4 * k + 3]);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        w[k] = cast4<FMT>(V(i, 4 * k) * cs[4 * k], V(i, 4 * k + 1) * cs[4 * k + 1],
                                          V(i, 4 * k + 2) * cs[4 * k + 2], V(i, 4 * k + 3) * cs[4 * k + 3]);
                }
                uint8_t *dst = args.q_col + prow * N + n0;
                if (VEC && n0 + 16 <= N) {
                    st16<(STREAM == 2)>(dst, w[0], w[1], w[2], w[3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        if (n0 + j < N) dst[j] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
                }
            }
        } else {
            // transposed output q_col[N, M]: stage bytes column-major in LDS
            if (wave_special) {
#pragma unroll
                for (int j = 0; j < 16; ++j) s_tr[cseg * 16 + j][rgrp] = qpack4<FMT>(V(0, j), V(1, j), V(2, j), V(3, j), cs[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    s_tr[cseg * 16 + j][rgrp] = cast4<FMT>(V(0, j) * cs[j], V(1, j) * cs[j], V(2, j) * cs[j], V(3, j) * cs[j]);
            }
            __syncthreads();
            // 128 output rows (n) x 128 bytes (m): 16-byte chunks; the row stride
            // ldt_col is a multiple of 128 and the padding bytes (rows past M, or
            // past a group's rows in segment mode) are zero
            const int64_t ldt = args.ldt_col;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int     c   = it * NT + t;
                const int     nl  = c >> 3;
                const int     mc  = (c & 7) * 16;
                const int64_t n   = tn * TILE + nl;
                const int64_t m   = tm * TILE + mc;
                if (n >= N) continue;
                const uint32_t *src = &s_tr[nl][mc >> 2];
                st16<(STREAM == 2)>(args.q_col + n * ldt + m, src[0], src[1], src[2], src[3]);
            }
        }
    }

    // ---- 128 x 128 weight tile --------------------------------------------
    if constexpr ((MODE & QB_W2D) != 0) {
        // one scale for the tile: NaN-propagating amax first; a tile with NaN
        // or infinity recomputes the reference's NaN-dropping amax and takes
        // the clamped cast (the decision is the same in all four waves)
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) a = pmax_abs(a, V(i, j));
        a = amax_wave(a);
        if (lane == 0) s_wmax[wave] = a;
        __syncthreads();
        a            = amax2(amax2(s_wmax[0], s_wmax[1]), amax2(s_wmax[2], s_wmax[3]));
        wave_special = special_amax(a);
        if constexpr (TPW == 2) {
            // the branch below holds a barrier: both tiles take it when either needs it
            // (the clamped cast is exact for any tile)
            const auto &o = s_wmax_[half ^ 1];
            wave_special  = wave_special || special_amax(amax2(amax2(o[0], o[1]), amax2(o[2], o[3])));
        }
        if (wave_special) {
            a = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 16; ++j) a = fmaxf(a, absq(V(i, j)));
            a = amax_wave(a);
            if (lane == 0) s_wmax[4 + wave] = a;
            __syncthreads();
            a = amax2(amax2(s_wmax[4], s_wmax[5]), amax2(s_wmax[6], s_wmax[7]));
        }
        const float   sc  = scale_from_amax<FMT>(a, 1e-4f);
        const int64_t mb  = (M + TILE - 1) / TILE, nb = (N + TILE - 1) / TILE;
        if (t == 0) args.s_w[(batch * mb + tm) * nb + tn] = 1.0f / sc;
        uint8_t *qb = args.q_row + batch * M * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t r = row_base + rgrp * 4 + i;
            uint32_t      w[4];
            if (wave_special) {
#pragma unroll
                for (int k = 0; k < 4; ++k) w[k] = Q4(i, 4 * k, sc);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) w[k] = F4(i, 4 * k, sc);
            }
            if (!rvalid[i]) continue;
            uint8_t *dst = qb + r * N + n0;
            if (VEC && n0 + 16 <= N) {
                st16<(STREAM == 2)>(dst, w[0], w[1], w[2], w[3]);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (n0 + j < N) dst[j] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
            }
        }
        if constexpr ((MODE & QB_W2D_T) != 0) {
            // transposed copy [B, N, M] through LDS.  The bytes are quantized
            // again rather than byte-transposed from the row words (8 v_perm per
            // 16 bytes): the transpose frees 13 VGPRs, the fifth resident
            // workgroup per CU that buys makes the 940 MB expert stream 2.5%
            // slower, and at four workgroups both forms take the same time.
            // The clamped cast throughout: with the plain cast here the
            // compiler holds 147 VGPRs (three workgroups per CU).
#pragma unroll
            for (int j = 0; j < 16; ++j) s_tr[cseg * 16 + j][rgrp] = qpack4<FMT>(V(0, j), V(1, j), V(2, j), V(3, j), sc);
            __syncthreads();
            const int64_t ldt = (M + TILE - 1) / TILE * TILE; // padded rows are zero
            uint8_t      *qt  = args.q_t + batch * N * ldt;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int     c  = it * NT + t;
                const int     nl = c >> 3;
                const int     mc = (c & 7) * 16;
                const int64_t n  = tn * TILE + nl;
                const int64_t m  = tm * TILE + mc;
                if (n >= N) continue;
                const uint32_t *src = &s_tr[nl][mc >> 2];
                st16<(STREAM == 2)>(qt + n * ldt + m, src[0], src[1], src[2], src[3]);
            }
        }
    }
}

// vk_lens[g] = roundup(lens[g], 128); vk_offs = exclusive prefix sum (single workgroup)
__global__ __launch_bounds__(256) void padded_offs_kernel(const int64_t *lens, int64_t *vk_lens,
                                                          int64_t *vk_offs, int64_t G, int64_t align) {
    __shared__ int64_t s_carry;
    if (threadIdx.x == 0) {
        s_carry    = 0;
        vk_offs[0] = 0;
    }
    __syncthreads();
    for (int64_t base = 0; base < G; base += 256) {
        const int64_t g   = base + threadIdx.x;
        const int64_t len = g < G ? lens[g] : 0;
        const int64_t p   = (len + align - 1) / align * align;
        // inclusive scan within the block (Hillis-Steele over LDS)
        __shared__ int64_t s_scan[256];
        s_scan[threadIdx.x] = p;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            const int64_t add = threadIdx.x >= off ? s_scan[threadIdx.x - off] : 0;
            __syncthreads();
            s_scan[threadIdx.x] += add;
            __syncthreads();
        }
        const int64_t carry = s_carry;
        if (g < G) {
            if (vk_lens) vk_lens[g] = p;
            vk_offs[g + 1] = carry + s_scan[threadIdx.x];
        }
        __syncthreads();
        if (threadIdx.x == 255) s_carry = carry + s_scan[255];
        __syncthreads();
    }
}

// padded_offs[g] = sum_{q<g} roundup(offs[q+1] - offs[q], align)
__global__ __launch_bounds__(256) void offs_to_padded_offs_kernel(const int64_t *offs, int64_t *poffs,
                                                                  int64_t G, int64_t align) {
    __shared__ int64_t s_scan[256];
    __shared__ int64_t s_carry;
    if (threadIdx.x == 0) {
        s_carry  = 0;
        poffs[0] = 0;
    }
    __syncthreads();
    for (int64_t base = 0; base < G; base += 256) {
        const int64_t g   = base + threadIdx.x;
        const int64_t len = g < G ? offs[g + 1] - offs[g] : 0;
        s_scan[threadIdx.x] = (len + align - 1) / align * align;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            const int64_t add = threadIdx.x >= off ? s_scan[threadIdx.x - off] : 0;
            __syncthreads();
            s_scan[threadIdx.x] += add;
            __syncthreads();
        }
        const int64_t carry = s_carry;
        if (g < G) poffs[g + 1] = carry + s_scan[threadIdx.x];
        __syncthreads();
        if (threadIdx.x == 255) s_carry = carry + s_scan[255];
        __syncthreads();
    }
}

// Inputs larger than this cannot stay resident in the 256 MB MALL.  They are
// quantized two tiles per workgroup.  Outputs larger than the MALL are stored
// non-temporally with plain loads: on the 470-1000 MB outputs of the grouped
// configuration that is 4-6% faster than both hints and 3% faster than none
// (the hints were 3-10% slower on outputs that fit).  When the outputs fit,
// the 128 x 128 weight mode reads with plain loads (2.7% faster than the load
// hint on the 264 MB headline weight, once tiles were paired) and the 1-D
// modes with non-temporal loads (1.6-2.2% faster at 28672 x 8192).
constexpr int64_t STREAM_BYTES    = 192ll << 20;
constexpr int64_t NT_STORE_BYTES  = 256ll << 20;

// flat count of the 128 x 128 tiles of a rows x cols tensor (the kernel takes
// consecutive indices along a tile row); launch_tile rejects counts past
// 2^31 - 1, which come back as UINT32_MAX
uint32_t tile_grid(int64_t rows, int64_t cols) {
    const int64_t t = cdiv(rows, static_cast<int64_t>(TILE)) * cdiv(cols, static_cast<int64_t>(TILE));
    return t > 0x7fffffffll ? 0xffffffffu : static_cast<uint32_t>(t);
}

template <int MODE>
int launch_tile(const QBArgs &a, int in_dtype, int fmt, dim3 grid, bool vec, hipStream_t st) {
    PTA_CHECK_ARG(grid.x <= 0x7fffffffu, "tensor too large: more than 2^31 - 1 tiles of 128 x 128");
    if (grid.x == 0) return PTA_OK;
    const int64_t elems    = static_cast<int64_t>(grid.z) * a.M * a.N;
    const int64_t in_bytes = elems * (in_dtype == PTA_F32 ? 4 : 2);
    // fp8 byte outputs written by this mode
    const int64_t nq        = ((MODE & (QB_ROW | QB_W2D)) ? 1 : 0) + ((MODE & QB_COL) ? 1 : 0) + ((MODE & QB_W2D_T) ? 1 : 0);
    const bool    stream    = vec && in_bytes >= STREAM_BYTES;
    const bool    nt_store  = stream && elems * nq >= NT_STORE_BYTES;
    // the load hint for the 1-D modes whose outputs fit the MALL (row-only / column-only
    // 28672 x 8192: 1.6% / 2.2% faster); the 128 x 128 weight mode reads faster without it
    const bool    nt_load   = stream && !nt_store && (MODE & QB_W2D) == 0;
    // two tiles per workgroup for the large (streamed) tensors when the tile
    // order pairs neighbours within one tile row (row-major) or column
    constexpr bool COLMAJOR = (MODE & QB_SEGMENT) == 0 && (MODE & (QB_COL_T | QB_W2D_T)) != 0;
    const uint32_t tiles_n  = static_cast<uint32_t>(cdiv(a.N, static_cast<int64_t>(TILE)));
    const bool     pair     = stream && (COLMAJOR ? (grid.x / tiles_n) % 2 == 0 : tiles_n % 2 == 0);
    const dim3     grid2(grid.x / 2, grid.y, grid.z);
#define PTA_QB_LAUNCH(IDT, F, V, S)                                                                \
    do {                                                                                           \
        if constexpr (V) {                                                                         \
            if (pair) {                                                                            \
                quant_block_tile_kernel<IDT, F, MODE, V, S, 2><<<grid2, 2 * NT, 0, st>>>(a);       \
                break;                                                                             \
            }                                                                                      \
        }                                                                                          \
        quant_block_tile_kernel<IDT, F, MODE, V, S, 1><<<grid, NT, 0, st>>>(a);                    \
    } while (0)
#define PTA_QB_FMT(IDT, V, S)                                                                      \
    if (fmt == PTA_E4M3) PTA_QB_LAUNCH(IDT, PTA_E4M3, V, S);                                       \
    else PTA_QB_LAUNCH(IDT, PTA_E5M2, V, S)
#define PTA_QB_VEC(IDT)                                                                            \
    if (nt_store) { PTA_QB_FMT(IDT, true, 2); }                                                    \
    else if (nt_load) { PTA_QB_FMT(IDT, true, 1); }                                                \
    else if (vec) { PTA_QB_FMT(IDT, true, 0); }                                                    \
    else { PTA_QB_FMT(IDT, false, 0); }
    if (in_dtype == PTA_BF16) { PTA_QB_VEC(PTA_BF16) }
    else if (in_dtype == PTA_F16) { PTA_QB_VEC(PTA_F16) }
    else { PTA_QB_VEC(PTA_F32) }
#undef PTA_QB_VEC
#undef PTA_QB_FMT
#undef PTA_QB_LAUNCH
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

bool vec_ok(const void *x, int in_dtype, int64_t N, std::initializer_list<const void *> outs) {
    const int64_t eb = in_dtype == PTA_F32 ? 4 : 2;
    if (!aligned16(x) || (N * eb) % 16 != 0 || N % 16 != 0) return false;
    for (const void *p : outs)
        if (p && !aligned16(p)) return false;
    return true;
}

int check_common(const void *x, int in_dtype, int fmt, int64_t block) {
    PTA_CHECK_ARG(x != nullptr, "input pointer is NULL");
    PTA_CHECK_ARG(in_dtype == PTA_BF16 || in_dtype == PTA_F16 || in_dtype == PTA_F32,
                  "unsupported input dtype code %d", in_dtype);
    PTA_CHECK_ARG(fmt == PTA_E4M3 || fmt == PTA_E5M2, "unsupported fp8 format code %d", fmt);
    PTA_CHECK_ARG(block == TILE, "block size %lld unsupported: only 128 is implemented",
                  (long long)block);
    return PTA_OK;
}

} // namespace
} // namespace pta

using namespace pta;

extern "C" int pta_quantize_fp8_blockwise(const void *x, int in_dtype, int64_t M, int64_t N,
                                          int64_t block, int axis, void *q, float *s, int fmt,
                                          pta_stream_t stream) {
    clear_error();
    if (int rc = check_common(x, in_dtype, fmt, block)) return rc;
    PTA_CHECK_ARG(M >= 0 && N >= 0, "negative shape");
    PTA_CHECK_ARG(axis == 0 || axis == 1, "axis must be 0 or 1");
    if (M == 0 || N == 0) return PTA_OK;
    QBArgs a{};
    a.x = x; a.M = M; a.N = N;
    dim3 grid(tile_grid(M, N), 1, 1);
    const bool v = vec_ok(x, in_dtype, N, {q});
    if (axis == 1) {
        a.q_row = static_cast<uint8_t *>(q); a.s_row = s;
        a.srow_m = cdiv(N, TILE); a.srow_k = 1;
        return launch_tile<QB_ROW>(a, in_dtype, fmt, grid, v, as_stream(stream));
    }
    a.q_col = static_cast<uint8_t *>(q); a.s_col = s;
    return launch_tile<QB_COL>(a, in_dtype, fmt, grid, v, as_stream(stream));
}

extern "C" int pta_quantize_fp8_blockwise_dual(const void *x, int in_dtype, int64_t M, int64_t N,
                                               int64_t block, void *q_row, float *s_row,
                                               void *q_col, float *s_col, int layout,
                                               int fmt, pta_stream_t stream) {
    clear_error();
    if (int rc = check_common(x, in_dtype, fmt, block)) return rc;
    PTA_CHECK_ARG(M >= 0 && N >= 0, "negative shape");
    PTA_CHECK_ARG((q_row == nullptr) == (s_row == nullptr), "q_row/s_row must both be set or NULL");
    PTA_CHECK_ARG((q_col == nullptr) == (s_col == nullptr), "q_col/s_col must both be set or NULL");
    PTA_CHECK_ARG(q_row || q_col, "no output requested");
    PTA_CHECK_ARG((layout & ~(PTA_DUAL_COL_TRANSPOSED | PTA_DUAL_ROW_SCALE_KMAJOR)) == 0, "unknown layout flags");
    if (M == 0 || N == 0) return PTA_OK;
    const bool col_transposed = (layout & PTA_DUAL_COL_TRANSPOSED) != 0;
    QBArgs     a{};
    a.x = x; a.M = M; a.N = N;
    a.q_row = static_cast<uint8_t *>(q_row); a.s_row = s_row;
    if (layout & PTA_DUAL_ROW_SCALE_KMAJOR) { a.srow_m = 1; a.srow_k = M; }
    else { a.srow_m = cdiv(N, TILE); a.srow_k = 1; }
    a.q_col = static_cast<uint8_t *>(q_col); a.s_col = s_col;
    a.ldt_col = cdiv(M, TILE) * TILE;
    dim3       grid(tile_grid(M, N), 1, 1);
    PTA_CHECK_ARG(!col_transposed || aligned16(q_col), "transposed q_col must be 16-byte aligned");
    const bool v = vec_ok(x, in_dtype, N, {q_row, col_transposed ? nullptr : q_col});
    hipStream_t st = as_stream(stream);
    if (q_row && q_col) {
        return col_transposed ? launch_tile<QB_ROW | QB_COL | QB_COL_T>(a, in_dtype, fmt, grid, v, st)
                              : launch_tile<QB_ROW | QB_COL>(a, in_dtype, fmt, grid, v, st);
    }
    if (q_row) return launch_tile<QB_ROW>(a, in_dtype, fmt, grid, v, st);
    return col_transposed ? launch_tile<QB_COL | QB_COL_T>(a, in_dtype, fmt, grid, v, st)
                          : launch_tile<QB_COL>(a, in_dtype, fmt, grid, v, st);
}

extern "C" int pta_quantize_fp8_blockwise_for_weight(const void *w, int in_dtype, int64_t B,
                                                     int64_t M, int64_t N, int64_t block, void *q,
                                                     float *s, void *q_t, int fmt,
                                                     pta_stream_t stream) {
    clear_error();
    if (int rc = check_common(w, in_dtype, fmt, block)) return rc;
    PTA_CHECK_ARG(B >= 0 && M >= 0 && N >= 0, "negative shape");
    PTA_CHECK_ARG(q != nullptr && s != nullptr, "q and s must be set");
    if (B == 0 || M == 0 || N == 0) return PTA_OK;
    PTA_CHECK_ARG(B <= 65535, "batch too large");
    QBArgs a{};
    a.x = w; a.M = M; a.N = N; a.batch_stride_x = M * N;
    a.q_row = static_cast<uint8_t *>(q); a.s_w = s; a.q_t = static_cast<uint8_t *>(q_t);
    dim3 grid(tile_grid(M, N), 1, static_cast<uint32_t>(B));
    PTA_CHECK_ARG(!q_t || aligned16(q_t), "q_t must be 16-byte aligned");
    const bool v = vec_ok(w, in_dtype, N, {q}) && (M * N * (in_dtype == PTA_F32 ? 4 : 2)) % 16 == 0;
    hipStream_t st = as_stream(stream);
    if (q_t) return launch_tile<QB_W2D | QB_W2D_T>(a, in_dtype, fmt, grid, v, st);
    return launch_tile<QB_W2D>(a, in_dtype, fmt, grid, v, st);
}

extern "C" int pta_quantize_fp8_blockwise_segment_m_row_col(
    const void *x, int in_dtype, int64_t M, int64_t N, int64_t G, const int64_t *group_lens,
    const int64_t *group_offs, int64_t block, void *q_row, void *q_col_pad, float *s_row_t,
    float *s_col_pad, int64_t *vk_lens, int64_t *vk_offs, int fmt, int layout, pta_stream_t stream) {
    clear_error();
    if (int rc = check_common(x, in_dtype, fmt, block)) return rc;
    PTA_CHECK_ARG(M >= 0 && N >= 0 && G >= 1, "bad shape");
    PTA_CHECK_ARG(layout == 0 || layout == PTA_SEGMENT_COL_TRANSPOSED, "unknown layout %d", layout);
    PTA_CHECK_ARG(group_lens && group_offs && vk_offs && vk_lens, "group arrays must be set");
    PTA_CHECK_ARG(q_row && q_col_pad && s_row_t && s_col_pad, "outputs must be set");
    hipStream_t st = as_stream(stream);
    padded_offs_kernel<<<1, 256, 0, st>>>(group_lens, vk_lens, vk_offs, G, TILE);
    PTA_CHECK_LAUNCH();
    if (N == 0) return PTA_OK;
    const int64_t M_pad_max = M + G * TILE;
    QBArgs        a{};
    a.x = x; a.M = M; a.N = N;
    a.q_row = static_cast<uint8_t *>(q_row); a.s_row = s_row_t;
    a.srow_m = 1; a.srow_k = M;
    a.q_col = static_cast<uint8_t *>(q_col_pad); a.s_col = s_col_pad;
    a.ldt_col = cdiv(M, TILE) * TILE + G * TILE;
    a.group_offs = group_offs; a.padded_offs = vk_offs; a.G = G;
    dim3 grid(tile_grid(M_pad_max, N), 1, 1);
    if (layout == PTA_SEGMENT_COL_TRANSPOSED) {
        // q_col [N, roundup(M, 128) + 128 G]: column m of the transposed copy is
        // row m of the padded layout (16-byte chunks, zero padding rows)
        PTA_CHECK_ARG(aligned16(q_col_pad), "transposed q_col must be 16-byte aligned");
        const bool v = vec_ok(x, in_dtype, N, {q_row});
        return launch_tile<QB_ROW | QB_COL | QB_COL_T | QB_SEGMENT>(a, in_dtype, fmt, grid, v, st);
    }
    const bool v = vec_ok(x, in_dtype, N, {q_row, q_col_pad});
    return launch_tile<QB_ROW | QB_COL | QB_SEGMENT>(a, in_dtype, fmt, grid, v, st);
}

extern "C" int pta_grouped_compute_padded_offs(const int64_t *offs, int64_t *padded_offs, int64_t G,
                                               int64_t align, pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(offs && padded_offs && G >= 0 && align >= 1, "bad arguments");
    offs_to_padded_offs_kernel<<<1, 256, 0, as_stream(stream)>>>(offs, padded_offs, G, align);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" int pta_grouped_compute_padded_layout(const int64_t *lens, int64_t *lens_padded,
                                                 int64_t *offs_padded, int64_t G, int64_t align,
                                                 pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(lens && offs_padded && G >= 0 && align >= 1, "bad arguments");
    padded_offs_kernel<<<1, 256, 0, as_stream(stream)>>>(lens, lens_padded, offs_padded, G, align);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" int pta_grouped_compute_offs(const int64_t *lens, int64_t *offs, int64_t G,
                                        pta_stream_t stream) {
    clear_error();
    PTA_CHECK_ARG(lens && offs && G >= 0, "bad arguments");
    padded_offs_kernel<<<1, 256, 0, as_stream(stream)>>>(lens, nullptr, offs, G, 1);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}
