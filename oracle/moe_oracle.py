"""CPU oracle for MoE token permute / unpermute -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``primus-turbo_amd/primus_turbo``) never imports it.

numpy restatement of the reference's three MoE permutation kernels
(csrc/kernels/moe_permute/moe_permute.cu):

* ``preprocess``  -- permute_preprocessing_kernel (:82-340): per-expert slot
  assignment in token order, per-expert padding to ``pad_multiple``, the
  ``row_id_map`` [T + pad_multiple, 2E + 1] int32 layout, the overflow cap and
  ``tokens_per_expert``;
* ``permute``     -- permute_kernel (:437-505): scatter of each token row to
  its destination rows (zeros into padding rows), plus the per-token scaling
  factors and probs;
* ``unpermute``   -- unpermute_kernel / unpermute_kernel_e1 (:507-602): fp32
  sum of the routed rows in row_id_map order, rounded once to bf16/fp16.

Entries of ``row_id_map`` past a row's count are never written by the
reference (it allocates the map with at::empty), so ``preprocess`` returns a
mask of the defined entries next to the map.  Pinning of each function is
documented in ``tests/test_moe_oracle.py``.
"""

from __future__ import annotations

import numpy as np

INT_MAX = 2**31 - 1
KIND_BOOL, KIND_I32, KIND_I64 = 0, 1, 2


def routed_mask(expert_map: np.ndarray, kind: int, E: int) -> np.ndarray:
    """[T, E] bool: token t is routed to local expert e.

    Index maps keep entries in [0, E) after the kernel's int conversion
    (moe_permute.cu:58-60: ``const int e = topk_idx[...]``, i.e. int64 values
    are truncated to int32); the bool map is used as is (:41-42)."""
    T = expert_map.shape[0]
    if kind == KIND_BOOL:
        return np.asarray(expert_map, dtype=bool).reshape(T, E).copy()
    idx = np.asarray(expert_map).astype(np.int64).astype(np.int32).astype(np.int64)
    m = np.zeros((T, E), dtype=bool)
    valid = (idx >= 0) & (idx < E)
    t = np.repeat(np.arange(T), idx.shape[1]).reshape(idx.shape)
    m[t[valid], idx[valid]] = True
    return m


def preprocess(expert_map, kind, E, topk, pad_multiple, num_permuted_tokens=-1, probs_topk_stride=0):
    """Returns (row_id_map, defined_mask, tokens_per_expert int64[E], overflow_flag, num_dispatched).

    Follows permute_preprocessing_kernel (moe_permute.cu:82-340):
    * slot of (t, e) = 1 + number of tokens t' < t routed to e (:156-167),
      plus the exclusive prefix over experts of the padded per-expert counts
      (:207-224, :230-241);
    * slots above the cap ``npt`` (INT_MAX when num_permuted_tokens <= 0) set
      the overflow flag and are dropped from the row (:230-240);
    * row t holds its kept slots in ascending expert order at [0, n), the aux
      value (expert id, or the first k with topk_idx[t, k] == e for
      topk-aligned probs) at [E, E + n) and n at [2E] (:242-267);
    * padding row T + i holds, for each expert with more than i padding slots,
      the negative 1-based slot -(count_e + prefix_e + i + 1) (:289-307);
    * tokens_per_expert = padded count, clipped by the cap (:309-315);
    * num_dispatched = number of tokens routed to at least one local expert.
    """
    expert_map = np.asarray(expert_map)
    T = expert_map.shape[0]
    routed = routed_mask(expert_map, kind, E)
    npt = INT_MAX if num_permuted_tokens <= 0 else int(num_permuted_tokens)
    counts = routed.sum(axis=0).astype(np.int64)
    padded = ((counts + pad_multiple - 1) // pad_multiple) * pad_multiple if pad_multiple > 0 else counts.copy()
    prefix = np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int64)
    rank = np.cumsum(routed, axis=0).astype(np.int64)  # 1-based rank where routed
    slot = rank + prefix[None, :]
    keep = routed & (slot <= npt)
    overflow = int(bool((routed & (slot > npt)).any()))

    aux = np.broadcast_to(np.arange(E, dtype=np.int64), (T, E)).copy()
    if kind != KIND_BOOL and probs_topk_stride > 0:
        idx = expert_map.astype(np.int64).astype(np.int32).astype(np.int64)
        for k in range(idx.shape[1] - 1, -1, -1):  # the first matching k wins
            v = (idx[:, k] >= 0) & (idx[:, k] < E)
            aux[np.nonzero(v)[0], idx[v, k]] = k

    W = 2 * E + 1
    rim = np.zeros((T + pad_multiple, W), dtype=np.int32)
    defined = np.zeros((T + pad_multiple, W), dtype=bool)
    n = keep.sum(axis=1)
    pos = np.cumsum(keep, axis=1) - 1
    ts, es = np.nonzero(keep)
    rim[ts, pos[ts, es]] = slot[ts, es]
    rim[ts, E + pos[ts, es]] = aux[ts, es]
    defined[ts, pos[ts, es]] = True
    defined[ts, E + pos[ts, es]] = True
    rim[:T, 2 * E] = n
    defined[:T, 2 * E] = True

    num_padded = padded - counts
    for i in range(pad_multiple):
        r = T + i
        k = 0
        for e in range(E):
            if i >= num_padded[e]:
                continue
            v = counts[e] + prefix[e] + i + 1
            if v > npt:
                overflow = 1
                continue
            rim[r, k] = -v
            rim[r, E + k] = e
            defined[r, k] = defined[r, E + k] = True
            k += 1
        rim[r, 2 * E] = k
        defined[r, 2 * E] = True

    over = padded + prefix - npt
    tpe = np.where(over < 0, padded, np.maximum(0, padded - over)).astype(np.int64)
    num_dispatched = int(routed.any(axis=1).sum())
    return rim, defined, tpe, overflow, num_dispatched


def permute(tokens, rim, num_dispatched, pad_multiple, E, num_permuted, scaling_factor=None, probs=None,
            probs_stride=0):
    """Scatter of permute_kernel (moe_permute.cu:437-505) on raw element arrays.

    tokens: [T, H] array of any element type (copied bit for bit).  Rows
    [num_dispatched, num_dispatched + pad_multiple) of row_id_map are padding
    rows: their destinations receive zeros.  Returns (out, written_rows,
    out_scaling_factor, out_probs); rows never written are flagged False in
    written_rows (the reference leaves them uninitialised)."""
    tokens = np.asarray(tokens)
    T, H = tokens.shape
    out = np.zeros((num_permuted, H), dtype=tokens.dtype)
    written = np.zeros(num_permuted, dtype=bool)
    spt = 0 if scaling_factor is None else scaling_factor.shape[1]
    osf = None if scaling_factor is None else np.zeros((num_permuted, spt), dtype=np.float32)
    opr = None if probs is None else np.zeros(num_permuted, dtype=np.float32)
    pstride = probs_stride if probs_stride > 0 else E
    rows = min(num_dispatched + pad_multiple, rim.shape[0])
    for t in range(rows):
        pad = t >= num_dispatched
        n = int(rim[t, 2 * E])
        for j in range(n):
            d = int(rim[t, j])
            real = d > 0
            r = d - 1 if real else -d - 1
            if not (0 <= r < num_permuted):
                continue
            src = real and not pad
            out[r] = tokens[t] if src else 0
            written[r] = True
            if osf is not None:
                osf[r] = scaling_factor[t] if src else 0.0
            if opr is not None:
                opr[r] = probs.reshape(-1)[t * pstride + int(rim[t, E + j])] if src else 0.0
    return out, written, osf, opr


def unpermute(permuted_f32, rim, num_dispatched, E, T, probs_stride=0, permuted_probs=None):
    """fp32 sums of unpermute_kernel (moe_permute.cu:543-602), before the final rounding.

    permuted_f32: [P, H] exact fp32 values of the bf16/fp16 rows.  Row t <
    num_dispatched is the fp32 sum, in row_id_map order starting from +0.0, of
    the rows with a positive slot.  For E == 1 with a probs row width of 1 the
    reference copies the row instead (unpermute_kernel_e1, :507-541), which
    differs from the sum only for -0.0; ``copy_rows`` marks that case.
    Returns (sums [T, H] float32, rows_written bool[T], out_probs or None, copy_rows)."""
    permuted_f32 = np.asarray(permuted_f32, dtype=np.float32)
    H = permuted_f32.shape[1]
    pstride = probs_stride if probs_stride > 0 else E
    copy_rows = E == 1 and pstride == 1
    acc = np.zeros((T, H), dtype=np.float32)
    done = np.zeros(T, dtype=bool)
    oprobs = None if permuted_probs is None else np.zeros((T, pstride), dtype=np.float32)
    nd = min(num_dispatched, T)
    done[:nd] = True
    for t in range(nd):
        n = int(rim[t, 2 * E])
        if copy_rows:
            s = int(rim[t, 0]) if n > 0 else 0
            if s > 0:
                acc[t] = permuted_f32[s - 1]
            if oprobs is not None:
                oprobs[t, 0] = permuted_probs[s - 1] if s > 0 else 0.0
            continue
        a = np.zeros(H, dtype=np.float32)
        for j in range(n):
            s = int(rim[t, j])
            if s > 0:
                a = (a + permuted_f32[s - 1]).astype(np.float32)
                if oprobs is not None:
                    oprobs[t, int(rim[t, E + j])] = permuted_probs[s - 1]
        acc[t] = a
    return acc, done, oprobs, copy_rows


def round_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 round-to-nearest-even, returned as float32 (numpy's cast is RNE)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
