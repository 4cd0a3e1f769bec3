// MoE token permutation on gfx950: routing preprocessing (per-expert slots in
// token order, per-expert padding, row_id_map), the scatter of token rows into
// the expert-major packed layout that grouped_gemm_fp8 consumes, and its
// fp32-accumulated inverse.
//
// Semantics are those of the reference's csrc/kernels/moe_permute/moe_permute.cu:
// permute_preprocessing_kernel (:82-340), permute_kernel (:437-505) and
// unpermute_kernel / unpermute_kernel_e1 (:507-602).  row_id_map keeps the
// reference's [T + pad_multiple, 2E + 1] int32 layout so that the reference's
// Python layer and token dispatcher can consume it unchanged:
//   row t     : [0, n) 1-based destination rows of the kept (t, e) pairs in
//               ascending e, [E, E + n) the aux value (e, or the first k with
//               topk_idx[t, k] == e for topk-aligned probs), [2E] = n;
//   row T + i : padding rows, destinations stored negated.
//
// MI355X design:
// * The preprocessing is three stream-ordered launches (per-tile counts, a
//   per-expert scan over tiles, slot assignment) instead of a single
//   decoupled-lookback pass.  It needs no zero-initialised, cached or
//   double-buffered flag workspace: the caller's workspace is overwritten on
//   every call and nothing is allocated, so the sequence is graph-capturable.
// * A tile is one wave of 64 tokens: the rank of a token among the tile's
//   tokens routed to expert e is one ballot + popcount.  Each lane keeps its
//   token's expert bitmap (up to 512 experts) in its own LDS column.
// * Scatter / gather: a token row is spread over 64-256 threads (whole waves)
//   with four 16-byte pieces per thread in flight; the gather reads four
//   source rows at a time before accumulating them in row order.  Rows written
//   exactly once use non-temporal stores; the gather reads its source rows
//   non-temporally too.
#include "common.h"

#include <climits>

namespace pta {
namespace {

constexpr int MP_TILE  = 64;  // tokens per tile (one per lane)
constexpr int MP_MAX_E = 511; // experts per call (the reference's bound, moe_permute.cu:387-388)
constexpr int MP_WORDS = 16;  // 512-bit expert bitmap per token

typedef unsigned int mp_v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

__device__ __forceinline__ int pad_up(int v, int m) { return m > 0 ? (v + m - 1) / m * m : v; }

// Four 0/1 bytes of a bool routing row -> four bits (a byte counts as routed
// when it is non-zero).
__device__ __forceinline__ uint32_t bytes4_to_bits(uint32_t v) {
    v |= v >> 4;
    v |= v >> 2;
    v |= v >> 1;
    v &= 0x01010101u;
    return (v | (v >> 7) | (v >> 14) | (v >> 21)) & 0xFu;
}

// Expert bitmap of token t (the calling lane's) into s_bm[w * 64 + lane], w < nw.
// Index maps convert each entry to int before the range test, as the reference
// does (moe_permute.cu:58-60), so int64 entries are truncated to 32 bits.
template <int KIND>
__device__ __forceinline__ void load_bitmap(const void *map, int64_t T, int E, int topk, int64_t t,
                                            uint32_t *s_bm, int nw) {
    const int  lane  = threadIdx.x & 63;
    const bool valid = t < T;
    if constexpr (KIND == PTA_MOE_MAP_BOOL) {
        const uint8_t *row = reinterpret_cast<const uint8_t *>(map) + t * E;
        const bool     dw  = (E & 3) == 0;
        for (int w = 0; w < nw; ++w) {
            uint32_t  bits = 0;
            const int e0 = w * 32, e1 = min(E, e0 + 32);
            if (valid) {
                if (dw) {
                    for (int e = e0; e < e1; e += 4)
                        bits |= bytes4_to_bits(*reinterpret_cast<const uint32_t *>(row + e)) << (e - e0);
                } else {
                    for (int e = e0; e < e1; ++e) bits |= (row[e] != 0 ? 1u : 0u) << (e - e0);
                }
            }
            s_bm[w * 64 + lane] = bits;
        }
    } else {
        for (int w = 0; w < nw; ++w) s_bm[w * 64 + lane] = 0;
        if (valid) {
            for (int k = 0; k < topk; ++k) {
                int e;
                if constexpr (KIND == PTA_MOE_MAP_I32)
                    e = reinterpret_cast<const int32_t *>(map)[t * topk + k];
                else
                    e = static_cast<int>(reinterpret_cast<const int64_t *>(map)[t * topk + k]);
                if (e >= 0 && e < E) s_bm[(e >> 5) * 64 + lane] |= 1u << (e & 31);
            }
        }
    }
}

// counts[tile][e] = tokens of the tile routed to e; counts[tile][E] = tokens of
// the tile routed to at least one local expert.
template <int KIND>
__global__ __launch_bounds__(64) void mp_count_kernel(const void *map, int64_t T, int E, int topk,
                                                      int32_t *counts) {
    __shared__ uint32_t s_bm[MP_WORDS * 64];
    const int           lane = threadIdx.x;
    const int64_t       tile = blockIdx.x;
    const int           nw   = (E + 31) >> 5;
    load_bitmap<KIND>(map, T, E, topk, tile * MP_TILE + lane, s_bm, nw);
    int32_t *row  = counts + tile * (E + 1);
    uint32_t any  = 0;
    int      keep = 0;
    for (int w = 0; w < nw; ++w) {
        const uint32_t bits = s_bm[w * 64 + lane];
        any |= bits;
        const int nb = min(32, E - w * 32);
        for (int b = 0; b < nb; ++b) {
            const int e = w * 32 + b;
            const int c = __popcll(__ballot((bits >> b) & 1u));
            if ((e & 63) == lane) keep = c;
            if ((e & 63) == 63 || e == E - 1) {
                if (lane <= (e & 63)) row[(e & ~63) + lane] = keep;
            }
        }
    }
    const int nd = __popcll(__ballot(any != 0));
    if (lane == 0) row[E] = nd;
}

// Column c of counts[ntiles][E + 1] := exclusive prefix over tiles;
// totals[c] = column sum.  Block c owns column c.  Also clears the overflow flag.
__global__ __launch_bounds__(256) void mp_scan_kernel(int32_t *counts, int64_t ntiles, int W,
                                                      int32_t *totals, int32_t *overflow_flag) {
    __shared__ int s_wsum[4];
    const int      c    = blockIdx.x;
    const int      lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int            carry = 0;
    for (int64_t base = 0; base < ntiles; base += 256) {
        const int64_t i    = base + threadIdx.x;
        const int     v    = i < ntiles ? counts[i * W + c] : 0;
        const int     incl = wave_incl_scan(v);
        if (lane == 63) s_wsum[wave] = incl;
        __syncthreads();
        int before = carry;
        for (int q = 0; q < wave; ++q) before += s_wsum[q];
        const int chunk = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
        if (i < ntiles) counts[i * W + c] = before + incl - v;
        carry += chunk;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        totals[c] = carry;
        if (c == 0) *overflow_flag = 0;
    }
}

// Blocks [0, ntiles): slots of the tile's tokens.  Block ntiles: padding rows,
// tokens_per_expert and the dispatched-token count.
template <int KIND>
__global__ __launch_bounds__(64) void mp_assign_kernel(const void *map, int64_t T, int E, int topk,
                                                       int pad_multiple, int npt, int probs_topk_stride,
                                                       const int32_t *counts, const int32_t *totals,
                                                       int64_t ntiles, int32_t *rim,
                                                       int64_t *tokens_per_expert,
                                                       int32_t *overflow_flag, int32_t *num_dispatched) {
    __shared__ uint32_t s_bm[MP_WORDS * 64];
    __shared__ int      s_base[MP_MAX_E + 1]; // padded exclusive prefix over experts
    __shared__ int      s_cnt[MP_MAX_E + 1];  // tokens routed to each expert
    const int           lane = threadIdx.x;
    const int64_t       tile = blockIdx.x;
    const int           W    = 2 * E + 1;

    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
        const int e      = e0 + lane;
        const int cnt    = e < E ? totals[e] : 0;
        const int padded = pad_up(cnt, pad_multiple);
        const int incl   = wave_incl_scan(padded);
        if (e < E) {
            s_base[e] = carry + incl - padded;
            s_cnt[e]  = cnt;
        }
        carry += __shfl(incl, 63, 64);
    }
    __syncthreads();

    bool ovf = false;
    if (tile == ntiles) {
        // padding row T + i: the i-th padding slot of every expert that has one
        for (int i = lane; i < pad_multiple; i += 64) {
            int32_t *row = rim + (T + i) * W;
            int      n   = 0;
            for (int e = 0; e < E; ++e) {
                const int cnt = s_cnt[e];
                if (i >= pad_up(cnt, pad_multiple) - cnt) continue;
                const int v = cnt + s_base[e] + i + 1;
                if (v > npt) {
                    ovf = true;
                    continue;
                }
                row[n]     = -v;
                row[E + n] = e;
                ++n;
            }
            row[2 * E] = n;
        }
        for (int e = lane; e < E; e += 64) {
            const int padded = pad_up(s_cnt[e], pad_multiple);
            const int over   = padded + s_base[e] - npt;
            tokens_per_expert[e] = over < 0 ? padded : max(0, padded - over);
        }
        if (lane == 0) *num_dispatched = totals[E];
        if (ovf) *overflow_flag = 1;
        return;
    }

    const int32_t *tb = counts + tile * (E + 1);
    for (int e = lane; e < E; e += 64) s_base[e] += tb[e];
    const int64_t t  = tile * MP_TILE + lane;
    const int     nw = (E + 31) >> 5;
    load_bitmap<KIND>(map, T, E, topk, t, s_bm, nw);
    __syncthreads();

    const uint64_t below = (1ull << lane) - 1ull;
    int32_t       *row   = rim + t * W;
    int            n     = 0;
    for (int w = 0; w < nw; ++w) {
        const uint32_t bits = s_bm[w * 64 + lane];
        const int      nb   = min(32, E - w * 32);
        for (int b = 0; b < nb; ++b) {
            const bool     r = (bits >> b) & 1u;
            const uint64_t m = __ballot(r);
            if (m == 0) continue;
            if (r) {
                const int e    = w * 32 + b;
                const int slot = s_base[e] + __popcll(m & below) + 1;
                if (slot > npt) {
                    ovf = true;
                } else {
                    int aux = e;
                    if constexpr (KIND != PTA_MOE_MAP_BOOL) {
                        if (probs_topk_stride > 0) {
                            for (int k = 0; k < topk; ++k) {
                                int ek;
                                if constexpr (KIND == PTA_MOE_MAP_I32)
                                    ek = reinterpret_cast<const int32_t *>(map)[t * topk + k];
                                else
                                    ek = static_cast<int>(reinterpret_cast<const int64_t *>(map)[t * topk + k]);
                                if (ek == e) {
                                    aux = k;
                                    break;
                                }
                            }
                        }
                    }
                    row[n]     = slot;
                    row[E + n] = aux;
                    ++n;
                }
            }
        }
    }
    if (t < T) row[2 * E] = n;
    if (ovf) *overflow_flag = 1;
}

// Token rows are spread over TPT = 2^tpt_log2 threads (64..256, whole waves),
// 256 / TPT rows per block, MP_CPT 16-byte pieces per thread in flight.
constexpr int MP_CPT = 4;

__device__ __forceinline__ mp_v4u ld_nt(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const mp_v4u *>(p));
}

// Rows [nd, nd + pad_multiple) of row_id_map are padding rows (their
// destinations receive zeros), as in the reference.
__global__ __launch_bounds__(256) void mp_permute_kernel(
    const uint8_t *tokens, int64_t T, int64_t row_bytes, uint8_t *out, int64_t P, const int32_t *rim,
    int64_t rim_rows, const int32_t *ndisp_ptr, int pad_multiple, int E, const float *sf, float *osf,
    int spt, const float *probs, float *oprobs, int pstride, int tpt_log2) {
    __shared__ int s_dst[4][MP_MAX_E + 1];
    const int      tpt  = 1 << tpt_log2;
    const int      sub  = threadIdx.x >> tpt_log2;
    const int      lt   = threadIdx.x & (tpt - 1);
    const int64_t  tok  = static_cast<int64_t>(blockIdx.x) * (256 >> tpt_log2) + sub;
    const int      nd   = *ndisp_ptr;
    const bool     active = tok < min(static_cast<int64_t>(nd) + pad_multiple, rim_rows);
    const int32_t *row  = rim + tok * (2 * E + 1);
    const int      n    = active ? min(max(row[2 * E], 0), E) : 0;
    int           *dst  = s_dst[sub];
    for (int j = lt; j < n; j += tpt) dst[j] = row[j];
    __syncthreads();
    if (!active) return;
    const bool     src    = tok < nd && tok < T;
    const int64_t  nchunk = row_bytes >> 4;
    const mp_v4u   zero   = {0u, 0u, 0u, 0u};
    const uint8_t *in     = tokens + tok * row_bytes;
    for (int64_t c0 = lt; c0 < nchunk; c0 += static_cast<int64_t>(tpt) * MP_CPT) {
        mp_v4u v[MP_CPT];
#pragma unroll
        for (int u = 0; u < MP_CPT; ++u) {
            const int64_t c = c0 + static_cast<int64_t>(u) * tpt;
            // plain loads: a non-temporal read of the source rows measured 10-15% slower here
            v[u]            = (src && c < nchunk) ? *reinterpret_cast<const mp_v4u *>(in + c * 16) : zero;
        }
        for (int q = 0; q < n; ++q) {
            const int     d = __builtin_amdgcn_readfirstlane(dst[q]);
            const int64_t r = d > 0 ? d - 1 : -static_cast<int64_t>(d) - 1;
            if (d == 0 || r >= P) continue;
            uint8_t *o = out + r * row_bytes;
#pragma unroll
            for (int u = 0; u < MP_CPT; ++u) {
                const int64_t c = c0 + static_cast<int64_t>(u) * tpt;
                if (c < nchunk) __builtin_nontemporal_store(d > 0 ? v[u] : zero, reinterpret_cast<mp_v4u *>(o + c * 16));
            }
        }
    }
    if (osf != nullptr) {
        for (int q = 0; q < n; ++q) {
            const int     d = __builtin_amdgcn_readfirstlane(dst[q]);
            const int64_t r = d > 0 ? d - 1 : -static_cast<int64_t>(d) - 1;
            if (d == 0 || r >= P) continue;
            for (int s = lt; s < spt; s += tpt) osf[r * spt + s] = (d > 0 && src) ? sf[tok * spt + s] : 0.0f;
        }
    }
    if (oprobs != nullptr) {
        for (int j = lt; j < n; j += tpt) {
            const int     d   = dst[j];
            const int     aux = row[E + j];
            const int64_t r   = d > 0 ? d - 1 : -static_cast<int64_t>(d) - 1;
            if (d == 0 || r >= P) continue;
            const bool ok = d > 0 && src && aux >= 0 && aux < pstride;
            oprobs[r]     = ok ? probs[tok * pstride + aux] : 0.0f;
        }
    }
}

template <int DT>
__device__ __forceinline__ void acc8(float (&a)[8], const mp_v4u &v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = v[i];
        if constexpr (DT == PTA_BF16) {
            a[2 * i] += bf16_bits_to_f32(w & 0xffffu);
            a[2 * i + 1] += bf16_bits_to_f32(w >> 16);
        } else {
            a[2 * i] += f16_bits_to_f32(w & 0xffffu);
            a[2 * i + 1] += f16_bits_to_f32(w >> 16);
        }
    }
}

template <int DT>
__device__ __forceinline__ mp_v4u round8(const float (&a)[8]) {
    mp_v4u r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        if constexpr (DT == PTA_BF16) {
            lo = f32_to_bf16_bits(a[2 * i]);
            hi = f32_to_bf16_bits(a[2 * i + 1]);
        } else {
            lo = f32_to_f16_bits(a[2 * i]);
            hi = f32_to_f16_bits(a[2 * i + 1]);
        }
        r[i] = lo | (hi << 16);
    }
    return r;
}

// Token t < nd: out[t] = round(sum over the row's positive slots, in row
// order, of fp32(permuted[slot - 1])), starting from +0.0; tokens
// nd <= t < T get zero rows (and zero probs), so no output row is left
// unwritten when fewer tokens were dispatched than restored.  copy_rows (one
// expert, probs width 1) copies the single source row bit for bit instead, as
// the reference's unpermute_kernel_e1 does.  Row layout over threads as in
// mp_permute_kernel; sources are read MP_GRP rows at a time.
constexpr int MP_GRP = 4;

template <int DT>
__global__ __launch_bounds__(256) void mp_unpermute_kernel(const uint8_t *perm, int64_t P, int64_t H,
                                                           uint8_t *out, int64_t T, const int32_t *rim,
                                                           const int32_t *ndisp_ptr, int E,
                                                           const float *pprobs, float *oprobs,
                                                           int pstride, int copy_rows, int tpt_log2) {
    __shared__ int s_src[4][MP_MAX_E + 1];
    __shared__ int s_aux[4][MP_MAX_E + 1];
    const int      tpt    = 1 << tpt_log2;
    const int      sub    = threadIdx.x >> tpt_log2;
    const int      lt     = threadIdx.x & (tpt - 1);
    const int64_t  tok    = static_cast<int64_t>(blockIdx.x) * (256 >> tpt_log2) + sub;
    const bool     active = tok < min(static_cast<int64_t>(*ndisp_ptr), T);
    const int32_t *row    = rim + tok * (2 * E + 1);
    const int      n      = active ? min(max(row[2 * E], 0), E) : 0;
    int           *src    = s_src[sub];
    int           *aux    = s_aux[sub];
    for (int j = lt; j < n; j += tpt) {
        const int s = row[j];
        src[j]      = (s > 0 && s <= P) ? s : 0; // slots outside the permuted rows read nothing
        aux[j]      = row[E + j];
    }
    __syncthreads();
    if (tok >= T) return; // inactive tokens below T fall through with n = 0: zero rows

    const int64_t rb     = H * 2;
    const int64_t nchunk = rb >> 4;
    uint8_t      *orow   = out + tok * rb;
    const mp_v4u  zero   = {0u, 0u, 0u, 0u};
    if (copy_rows) {
        const int s = n > 0 ? __builtin_amdgcn_readfirstlane(src[0]) : 0;
        for (int64_t c = lt; c < nchunk; c += tpt) {
            const mp_v4u v = s > 0 ? ld_nt(perm + (s - 1) * rb + c * 16) : zero;
            __builtin_nontemporal_store(v, reinterpret_cast<mp_v4u *>(orow + c * 16));
        }
    } else {
        for (int64_t c0 = lt; c0 < nchunk; c0 += static_cast<int64_t>(tpt) * MP_CPT) {
            float a[MP_CPT][8];
#pragma unroll
            for (int u = 0; u < MP_CPT; ++u)
#pragma unroll
                for (int i = 0; i < 8; ++i) a[u][i] = 0.0f;
            for (int q0 = 0; q0 < n; q0 += MP_GRP) {
                mp_v4u v[MP_GRP][MP_CPT];
                int    s[MP_GRP];
#pragma unroll
                for (int g = 0; g < MP_GRP; ++g) {
                    s[g] = q0 + g < n ? __builtin_amdgcn_readfirstlane(src[q0 + g]) : 0;
#pragma unroll
                    for (int u = 0; u < MP_CPT; ++u) {
                        const int64_t c = c0 + static_cast<int64_t>(u) * tpt;
                        v[g][u]         = (s[g] > 0 && c < nchunk) ? ld_nt(perm + (s[g] - 1) * rb + c * 16) : zero;
                    }
                }
#pragma unroll
                for (int g = 0; g < MP_GRP; ++g)
                    if (s[g] > 0)
#pragma unroll
                        for (int u = 0; u < MP_CPT; ++u) acc8<DT>(a[u], v[g][u]);
            }
#pragma unroll
            for (int u = 0; u < MP_CPT; ++u) {
                const int64_t c = c0 + static_cast<int64_t>(u) * tpt;
                if (c < nchunk) __builtin_nontemporal_store(round8<DT>(a[u]), reinterpret_cast<mp_v4u *>(orow + c * 16));
            }
        }
    }
    if (oprobs != nullptr) {
        for (int p = lt; p < pstride; p += tpt) {
            float v = 0.0f;
            for (int q = 0; q < n; ++q) {
                const int s = src[q];
                if (s > 0 && aux[q] == p) v = pprobs[s - 1];
            }
            oprobs[tok * pstride + p] = v;
        }
    }
}

// log2 of the threads per token row: enough for MP_CPT pieces each, 64..256.
int mp_tpt_log2(int64_t nchunk) {
    int l = 6;
    while (l < 8 && (static_cast<int64_t>(1) << l) * MP_CPT < nchunk) ++l;
    return l;
}

} // namespace
} // namespace pta

using namespace pta;

extern "C" size_t pta_moe_permute_preprocess_workspace_size(int64_t num_tokens, int num_local_experts) {
    if (num_tokens < 0 || num_local_experts <= 0) return 0;
    return static_cast<size_t>(cdiv(num_tokens, MP_TILE) + 1) * (num_local_experts + 1) * sizeof(int32_t);
}

extern "C" int pta_moe_permute_preprocess(const void *expert_map, int map_kind, int64_t num_tokens,
                                          int num_local_experts, int num_topk, int pad_multiple,
                                          int64_t num_permuted_tokens, int probs_topk_stride,
                                          int32_t *row_id_map, int64_t *tokens_per_expert,
                                          int32_t *overflow_flag, int32_t *num_dispatched, void *workspace,
                                          size_t workspace_bytes, pta_stream_t stream) {
    clear_error();
    const int     E = num_local_experts;
    const int64_t T = num_tokens;
    PTA_CHECK_ARG(map_kind == PTA_MOE_MAP_BOOL || map_kind == PTA_MOE_MAP_I32 || map_kind == PTA_MOE_MAP_I64,
                  "expert_map must be bool or int or int64 (kind %d)", map_kind);
    PTA_CHECK_ARG(E > 0, "num_local_experts must be > 0");
    PTA_CHECK_ARG(E <= MP_MAX_E, "num_local_experts must be < 512 (got %d)", E);
    PTA_CHECK_ARG(T >= 0 && pad_multiple >= 0, "negative size");
    PTA_CHECK_ARG(T + pad_multiple < INT_MAX, "too many tokens for int32 row ids");
    PTA_CHECK_ARG(map_kind == PTA_MOE_MAP_BOOL || num_topk > 0, "index expert_map needs num_topk > 0");
    if (map_kind == PTA_MOE_MAP_BOOL) {
        PTA_CHECK_ARG(probs_topk_stride == 0,
                      "probs_topk_stride > 0 (topk-aligned probs) requires the topk_idx expert_map; "
                      "routing_map mode only supports multihot probs");
    } else {
        PTA_CHECK_ARG(probs_topk_stride == 0 || probs_topk_stride == num_topk,
                      "probs_topk_stride must be 0 (multihot probs) or equal to num_topk");
    }
    PTA_CHECK_ARG(row_id_map && tokens_per_expert && overflow_flag && num_dispatched && workspace,
                  "null pointer");
    PTA_CHECK_ARG(T == 0 || expert_map, "null expert_map");
    PTA_CHECK_ARG(workspace_bytes >= pta_moe_permute_preprocess_workspace_size(T, E), "workspace too small");
    const int64_t ntiles = cdiv(T, MP_TILE);
    int32_t      *counts = reinterpret_cast<int32_t *>(workspace);
    int32_t      *totals = counts + ntiles * (E + 1);
    const int     npt    = num_permuted_tokens <= 0 || num_permuted_tokens > INT_MAX
                               ? INT_MAX
                               : static_cast<int>(num_permuted_tokens);
    hipStream_t st = as_stream(stream);
#define PTA_MP_LAUNCH(K)                                                                           \
    do {                                                                                           \
        if (ntiles > 0) mp_count_kernel<K><<<ntiles, 64, 0, st>>>(expert_map, T, E, num_topk, counts); \
        mp_scan_kernel<<<E + 1, 256, 0, st>>>(counts, ntiles, E + 1, totals, overflow_flag);      \
        mp_assign_kernel<K><<<ntiles + 1, 64, 0, st>>>(expert_map, T, E, num_topk, pad_multiple, npt, \
                                                      probs_topk_stride, counts, totals, ntiles,  \
                                                      row_id_map, tokens_per_expert, overflow_flag, \
                                                      num_dispatched);                             \
    } while (0)
    if (map_kind == PTA_MOE_MAP_BOOL) PTA_MP_LAUNCH(PTA_MOE_MAP_BOOL);
    else if (map_kind == PTA_MOE_MAP_I32) PTA_MP_LAUNCH(PTA_MOE_MAP_I32);
    else PTA_MP_LAUNCH(PTA_MOE_MAP_I64);
#undef PTA_MP_LAUNCH
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" int pta_moe_permute(const void *tokens, int64_t num_tokens, int elem_bytes, int64_t hidden,
                               void *permuted, int64_t num_permuted, const int32_t *row_id_map,
                               int64_t row_id_map_rows, const int32_t *num_dispatched, int pad_multiple,
                               int num_local_experts, const float *scaling_factor,
                               float *permuted_scaling_factor, int scales_per_token, const float *probs,
                               float *permuted_probs, int probs_stride, pta_stream_t stream) {
    clear_error();
    const int E = num_local_experts;
    PTA_CHECK_ARG(elem_bytes == 1 || elem_bytes == 2, "token elements must be 1 or 2 bytes (got %d)", elem_bytes);
    PTA_CHECK_ARG(E > 0 && E <= MP_MAX_E, "num_local_experts must be in [1, 511]");
    PTA_CHECK_ARG(hidden >= 0 && num_tokens >= 0 && num_permuted >= 0 && row_id_map_rows >= 0 && pad_multiple >= 0,
                  "negative size");
    PTA_CHECK_ARG((hidden * elem_bytes) % 16 == 0,
                  "hidden_size must be a multiple of %d for %d-byte elements", 16 / elem_bytes, elem_bytes);
    PTA_CHECK_ARG(probs_stride >= 0, "probs_stride must be >= 0");
    if (num_permuted == 0 || row_id_map_rows == 0) return PTA_OK;
    PTA_CHECK_ARG(tokens && permuted && row_id_map && num_dispatched, "null pointer");
    PTA_CHECK_ARG(aligned16(tokens) && aligned16(permuted), "token buffers must be 16-byte aligned");
    PTA_CHECK_ARG((scaling_factor == nullptr) == (permuted_scaling_factor == nullptr),
                  "scaling_factor and permuted_scaling_factor go together");
    PTA_CHECK_ARG(scaling_factor == nullptr || scales_per_token > 0, "scales_per_token must be > 0");
    PTA_CHECK_ARG((probs == nullptr) == (permuted_probs == nullptr), "probs and permuted_probs go together");
    const int pstride = probs_stride > 0 ? probs_stride : E;
    const int tl      = mp_tpt_log2(hidden * elem_bytes / 16);
    mp_permute_kernel<<<cdiv(row_id_map_rows, 256 >> tl), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<const uint8_t *>(tokens), num_tokens, hidden * elem_bytes,
        reinterpret_cast<uint8_t *>(permuted), num_permuted, row_id_map, row_id_map_rows, num_dispatched,
        pad_multiple, E, scaling_factor, permuted_scaling_factor, scales_per_token, probs, permuted_probs,
        pstride, tl);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}

extern "C" int pta_moe_unpermute(const void *permuted, int64_t num_permuted, int dtype, int64_t hidden,
                                 void *tokens, int64_t num_tokens, const int32_t *row_id_map,
                                 const int32_t *num_dispatched, int num_local_experts,
                                 const float *permuted_probs, float *probs, int probs_stride,
                                 pta_stream_t stream) {
    clear_error();
    const int E = num_local_experts;
    PTA_CHECK_ARG(dtype == PTA_BF16 || dtype == PTA_F16, "unpermute: permuted_tokens must be bfloat16 or float16");
    PTA_CHECK_ARG(E > 0 && E <= MP_MAX_E, "num_local_experts must be in [1, 511]");
    PTA_CHECK_ARG(hidden >= 0 && num_tokens >= 0 && num_permuted >= 0, "negative size");
    PTA_CHECK_ARG(hidden % 8 == 0, "unpermute: hidden_size must be a multiple of 8");
    PTA_CHECK_ARG(probs_stride >= 0, "probs_stride must be >= 0");
    // an empty permuted operand may come with a NULL probs pointer (no row to read)
    PTA_CHECK_ARG(permuted_probs == nullptr ? (probs == nullptr || num_permuted == 0) : probs != nullptr,
                  "permuted_probs and probs go together");
    if (num_tokens == 0) return PTA_OK;
    PTA_CHECK_ARG(tokens && row_id_map && num_dispatched && (permuted || num_permuted == 0), "null pointer");
    PTA_CHECK_ARG(aligned16(tokens) && (permuted == nullptr || aligned16(permuted)),
                  "token buffers must be 16-byte aligned");
    const int pstride = probs_stride > 0 ? probs_stride : E;
    const int copy    = (E == 1 && pstride == 1) ? 1 : 0;
    const int tl      = mp_tpt_log2(hidden * 2 / 16);
    const dim3 grid(static_cast<unsigned>(cdiv(num_tokens, 256 >> tl)));
    if (dtype == PTA_BF16)
        mp_unpermute_kernel<PTA_BF16><<<grid, 256, 0, as_stream(stream)>>>(
            reinterpret_cast<const uint8_t *>(permuted), num_permuted, hidden, reinterpret_cast<uint8_t *>(tokens),
            num_tokens, row_id_map, num_dispatched, E, permuted_probs, probs, pstride, copy, tl);
    else
        mp_unpermute_kernel<PTA_F16><<<grid, 256, 0, as_stream(stream)>>>(
            reinterpret_cast<const uint8_t *>(permuted), num_permuted, hidden, reinterpret_cast<uint8_t *>(tokens),
            num_tokens, row_id_map, num_dispatched, E, permuted_probs, probs, pstride, copy, tl);
    PTA_CHECK_LAUNCH();
    return PTA_OK;
}
