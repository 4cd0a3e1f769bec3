"""Pins the MoE permutation oracle (oracle/moe_oracle.py) on the CPU.

Each check comes from outside the oracle's own formulation:
* the expert-major order of the reference's test reference
  (tests/pytorch/ref/permuatation_ref.py:10-33: masked_select over the
  transposed routing map) -- restated here with torch ops;
* the per-expert padding layout the reference's tests expect
  (tests/pytorch/ops/test_moe_permute.py:44-73, "expected_permuted_layout");
* the overflow-flag table of test_moe_permute.py:177-229 (golden outcomes);
* scatter_add for unpermute (permuatation_ref.py:36-72) on integer-valued
  rows, where fp32 sums are exact in any order;
* equivalence of the bool and top-k index forms of the same routing.
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as MO


def _routing(T, E, topk, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.argsort(torch.rand(T, E, generator=g), dim=1)
    rm = torch.zeros(T, E, dtype=torch.bool)
    rm.scatter_(1, perm[:, :topk], True)
    return rm


def _topk_idx(rm, topk, dtype=torch.int64):
    T, E = rm.shape
    ids = torch.arange(E).unsqueeze(0).expand(T, -1)
    return ids[rm].view(T, topk).to(dtype)


def _mask_map_order(rm):
    """sorted token indices of the reference test ref (masked_select on rm.T)."""
    T, E = rm.shape
    tok = torch.arange(T).unsqueeze(0).expand(E, -1)
    return tok.masked_select(rm.T.contiguous()).numpy()


def _expected_layout(rm, pad):
    """(src_token, src_expert) per permuted row, -1 for padding rows."""
    T, E = rm.shape
    real = rm.sum(0).tolist()
    padded = [((r + pad - 1) // pad) * pad for r in real] if pad > 0 else list(real)
    st = np.full(sum(padded), -1, np.int64)
    se = np.full(sum(padded), -1, np.int64)
    off = 0
    for e in range(E):
        idx = rm[:, e].nonzero(as_tuple=True)[0].numpy()
        st[off:off + len(idx)] = idx
        se[off:off + len(idx)] = e
        off += padded[e]
    return st, se


@pytest.mark.parametrize("topk", [1, 2, 4, 8])
@pytest.mark.parametrize("kind", [MO.KIND_BOOL, MO.KIND_I32, MO.KIND_I64])
def test_permute_order_matches_mask_map_reference(topk, kind):
    T, E, H = 300, 16, 8
    rm = _routing(T, E, topk, seed=topk)
    em = rm.numpy() if kind == MO.KIND_BOOL else _topk_idx(rm, topk).numpy()
    rim, defined, tpe, ovf, nd = MO.preprocess(em, kind, E, topk, 0)
    assert ovf == 0 and nd == T
    assert np.array_equal(tpe, rm.sum(0).numpy())
    x = np.arange(T * H, dtype=np.int32).reshape(T, H)
    P = int(tpe.sum())
    out, written, _, _ = MO.permute(x, rim, nd, 0, E, P)
    assert written.all()
    assert np.array_equal(out, x[_mask_map_order(rm)])


@pytest.mark.parametrize("pad", [8, 16, 64])
@pytest.mark.parametrize("topk", [1, 2, 4])
def test_padding_layout(pad, topk):
    T, E, H = 257, 8, 4
    rm = _routing(T, E, topk, seed=100 + pad)
    rim, defined, tpe, ovf, nd = MO.preprocess(rm.numpy(), MO.KIND_BOOL, E, 0, pad)
    base = rm.sum(0).numpy()
    assert np.array_equal(tpe, ((base + pad - 1) // pad) * pad)
    assert (tpe % pad == 0).all() and ovf == 0
    st, se = _expected_layout(rm, pad)
    x = np.arange(1, T * H + 1, dtype=np.int32).reshape(T, H)
    probs = np.random.default_rng(pad).random((T, E)).astype(np.float32)
    out, written, _, opr = MO.permute(x, rim, nd, pad, E, int(tpe.sum()), probs=probs)
    assert written.all()
    real = st >= 0
    assert np.array_equal(out[real], x[st[real]])
    assert (out[~real] == 0).all()
    assert np.array_equal(opr[real], probs[st[real], se[real]])
    assert (opr[~real] == 0).all()


@pytest.mark.parametrize(
    "pad,cap_kind,expected",
    [
        (0, "uncapped", 0), (0, ("real", 0), 0), (0, ("real", +256), 0), (0, "half", 1), (0, "tiny", 1),
        (8, ("padded", 0), 0), (8, ("padded", +8), 0), (8, ("real", 0), 1), (8, "half", 1),
        (64, ("padded", 0), 0), (64, ("real", 0), 1),
    ],
)
def test_overflow_table(pad, cap_kind, expected):
    T, E, topk = 1024, 8, 2
    rm = _routing(T, E, topk, seed=4321)
    per = rm.sum(0).numpy()
    real = int(per.sum())
    padded = int((((per + pad - 1) // pad) * pad).sum()) if pad > 0 else real
    if cap_kind == "uncapped":
        cap = -1
    elif cap_kind == "half":
        cap = real // 2
    elif cap_kind == "tiny":
        cap = 1
    else:
        base, delta = cap_kind
        cap = (real if base == "real" else padded) + delta
    rim, defined, tpe, ovf, nd = MO.preprocess(rm.numpy(), MO.KIND_BOOL, E, 0, pad, cap)
    assert ovf == expected
    if cap > 0:
        # every kept slot fits under the cap and tokens_per_expert sums to min(cap, padded)
        assert int(tpe.sum()) == min(cap, padded)
        n = rim[:T, 2 * E]
        for t in range(T):
            assert (rim[t, :n[t]] <= cap).all()


def test_unpermute_is_scatter_add():
    T, E, topk, H = 200, 8, 3, 16
    rm = _routing(T, E, topk, seed=5)
    rim, defined, tpe, ovf, nd = MO.preprocess(rm.numpy(), MO.KIND_BOOL, E, 0, 0)
    P = int(tpe.sum())
    g = np.random.default_rng(1).integers(-64, 64, size=(P, H)).astype(np.float32)
    sums, done, _, _ = MO.unpermute(g, rim, nd, E, T)
    ref = torch.zeros(T, H).scatter_add_(0, torch.from_numpy(_mask_map_order(rm)).unsqueeze(1).expand(-1, H),
                                         torch.from_numpy(g))
    assert done.all()
    assert np.array_equal(sums, ref.numpy())
    # unpermute(permute(x)) = topk * x on integer rows
    x = np.random.default_rng(2).integers(-8, 8, size=(T, H)).astype(np.float32)
    out, _, _, _ = MO.permute(x, rim, nd, 0, E, P)
    back, _, _, _ = MO.unpermute(out, rim, nd, E, T)
    assert np.array_equal(back, topk * x)


def test_index_and_bool_maps_agree_and_topk_aux():
    T, E, topk = 150, 32, 4
    rm = _routing(T, E, topk, seed=9)
    a = MO.preprocess(rm.numpy(), MO.KIND_BOOL, E, 0, 16)
    idx = _topk_idx(rm, topk, torch.int32).numpy()
    # shuffle the k order so aux (first matching k) is not sorted
    rng = np.random.default_rng(3)
    idx = np.take_along_axis(idx, np.argsort(rng.random(idx.shape), axis=1), axis=1)
    b = MO.preprocess(idx, MO.KIND_I32, E, topk, 16)
    c = MO.preprocess(idx, MO.KIND_I32, E, topk, 16, probs_topk_stride=topk)
    for x, y in zip(a[2:], b[2:]):
        assert np.array_equal(x, y)
    W = 2 * E + 1
    assert np.array_equal(a[0][a[1]], b[0][b[1]])
    n = c[0][:T, 2 * E]
    for t in range(T):
        for j in range(n[t]):
            e = b[0][t, E + j]
            k = c[0][t, E + j]
            assert idx[t, k] == e
    assert W == c[0].shape[1]


def test_unrouted_and_out_of_range_indices():
    T, E, topk = 70, 4, 2
    idx = np.full((T, topk), -1, np.int64)
    idx[:50, 0] = np.arange(50) % E
    idx[:50, 1] = 7  # outside [0, E): ignored
    rim, defined, tpe, ovf, nd = MO.preprocess(idx, MO.KIND_I64, E, topk, 0)
    assert nd == 50
    assert np.array_equal(tpe, np.bincount(np.arange(50) % E, minlength=E))
    assert (rim[50:T, 2 * E] == 0).all()


def test_unpermute_negative_zero_rule():
    """fp32 sums start at +0.0 (so -0.0 rows come back +0.0) except in the
    single-expert copy kernel (moe_permute.cu:507-541 vs :543-602)."""
    rm = np.ones((2, 1), bool)
    rim, _, tpe, _, nd = MO.preprocess(rm, MO.KIND_BOOL, 1, 0, 0)
    g = np.array([[-0.0, 1.0], [2.0, -0.0]], np.float32)
    s, _, _, copy = MO.unpermute(g, rim, nd, 1, 2)
    assert copy and np.signbit(s[0, 0]) and np.signbit(s[1, 1])
    rm2 = np.zeros((2, 2), bool)
    rm2[:, 0] = True
    rim2, _, _, _, nd2 = MO.preprocess(rm2, MO.KIND_BOOL, 2, 0, 0)
    s2, _, _, copy2 = MO.unpermute(g, rim2, nd2, 2, 2)
    assert not copy2 and not np.signbit(s2[0, 0]) and not np.signbit(s2[1, 1])
