"""GPU parity of the MoE permutation path (moe_permute / moe_unpermute).

Kernel level: row_id_map, tokens_per_expert, overflow flag, dispatched count,
permuted rows (bytes), scaling factors, probs and unpermuted sums are compared
bit for bit with the oracle (oracle/moe_oracle.py) and, when oracle/_ref was
built, with the reference's own kernels (csrc/kernels/moe_permute/moe_permute.cu)
on the same inputs.  API level: the reference's own test cases
(tests/pytorch/ops/test_moe_permute.py) restated.
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as MO
from oracle import oracle as O
from tests.helpers import assert_bytes_equal, randn, ref_lib, stream

pytestmark = pytest.mark.gpu

KIND = {torch.bool: MO.KIND_BOOL, torch.int32: MO.KIND_I32, torch.int64: MO.KIND_I64}


def _impl():
    from primus_turbo.pytorch.kernels.moe import moe_permute_impl as I

    return I


def _routing(T, E, topk, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.argsort(torch.rand(T, E, generator=g), dim=1)
    rm = torch.zeros(T, E, dtype=torch.bool)
    rm.scatter_(1, perm[:, :topk], True)
    return rm


def _expert_map(rm, topk, dtype, shuffle_seed=None):
    if dtype == torch.bool:
        return rm
    T, E = rm.shape
    idx = torch.arange(E).unsqueeze(0).expand(T, -1)[rm].view(T, topk)
    if shuffle_seed is not None:  # arbitrary k order: exercises the topk-aligned aux value
        g = torch.Generator().manual_seed(shuffle_seed)
        idx = torch.gather(idx, 1, torch.argsort(torch.rand(T, topk, generator=g), dim=1))
    return idx.to(dtype)


def _cmp_preprocess(got, exp, what):
    rim, tpe, ovf, nd = got
    erim, edef, etpe, eovf, end_ = exp
    rim = rim.cpu().numpy()
    assert rim.shape == erim.shape, what
    assert_bytes_equal(rim[edef], erim[edef], f"{what}: row_id_map")
    assert np.array_equal(tpe.cpu().numpy(), etpe), f"{what}: tokens_per_expert"
    assert int(ovf.item()) == eovf, f"{what}: overflow"
    assert int(nd.item()) == end_, f"{what}: num_dispatched"


PRE_CASES = [
    # (map dtype, E, topk, T, pad_multiple, cap, topk-aligned probs)
    (torch.bool, 16, 4, 4096, 0, -1, False),
    (torch.int32, 16, 8, 4096, 0, -1, True),
    (torch.int64, 16, 2, 4096, 0, -1, True),
    (torch.bool, 8, 2, 1000, 16, -1, False),
    (torch.int32, 32, 4, 777, 64, -1, True),
    (torch.bool, 1, 1, 300, 8, -1, False),
    (torch.int64, 256, 8, 3000, 128, -1, True),
    (torch.bool, 511, 3, 200, 16, -1, False),
    (torch.bool, 5, 2, 70000, 0, -1, False),      # many tiles: multi-chunk scan
    (torch.int32, 64, 6, 70001, 32, -1, False),
    (torch.bool, 8, 2, 1024, 8, 1100, False),      # cap: overflow
    (torch.bool, 8, 2, 1024, 0, 1, False),
    (torch.int32, 8, 2, 1024, 64, 512, True),
]


@pytest.mark.parametrize("case", PRE_CASES, ids=[f"{c[0]}-E{c[1]}-k{c[2]}-T{c[3]}-p{c[4]}-c{c[5]}" for c in PRE_CASES])
def test_preprocess_vs_oracle_and_reference(case):
    dt, E, topk, T, pad, cap, aligned = case
    I = _impl()
    rm = _routing(T, E, topk, seed=T + E)
    em = _expert_map(rm, topk, dt, shuffle_seed=7 if aligned else None)
    pts = topk if aligned else 0
    kt = 0 if dt == torch.bool else topk
    emc = em.cuda()
    print(f"preprocess {case}", flush=True)
    got = I.permute_preprocessing_impl(emc, E, kt, pad, cap, pts)
    exp = MO.preprocess(em.numpy(), KIND[dt], E, kt, pad, cap, pts)
    _cmp_preprocess(got, exp, f"oracle {case}")
    R = ref_lib()
    if R is not None and R.ref_moe_preprocess is not None:
        rim = torch.empty_like(got[0])
        tpe = torch.empty_like(got[1])
        ovf = torch.empty_like(got[2])
        nd = torch.zeros_like(got[3])
        assert R.ref_moe_preprocess(emc.data_ptr(), KIND[dt], T, E, kt, pad, cap, pts, rim.data_ptr(),
                                    tpe.data_ptr(), ovf.data_ptr(), nd.data_ptr(), stream()) == 0
        torch.cuda.synchronize()
        _cmp_preprocess((rim, tpe, ovf, nd), exp, f"reference kernel {case}")


def test_preprocess_unrouted_tail_and_bad_indices():
    """Tokens past the dispatched prefix carry -1 indices; out-of-range
    indices are ignored; int64 entries are read as int32 (moe_permute.cu:58)."""
    T, E, topk = 500, 8, 2
    idx = torch.full((T, topk), -1, dtype=torch.int64)
    g = torch.Generator().manual_seed(3)
    idx[:400, 0] = torch.randint(0, E, (400,), generator=g)
    idx[:400, 1] = torch.randint(0, 2 * E, (400,), generator=g)
    idx[5, 1] = (1 << 32) + 3
    I = _impl()
    got = I.permute_preprocessing_impl(idx.cuda(), E, topk, 16, -1, 0)
    _cmp_preprocess(got, MO.preprocess(idx.numpy(), MO.KIND_I64, E, topk, 16), "unrouted tail")


def _perm_case(dt_tok, E, topk, T, H, pad, with_probs, aligned, fp8_spt=0):
    I = _impl()
    rm = _routing(T, E, topk, seed=11 * T + E)
    em = _expert_map(rm, topk, torch.int32 if aligned else torch.bool, shuffle_seed=5 if aligned else None)
    kt = topk if aligned else 0
    pts = topk if aligned else 0
    rim, tpe, ovf, nd = I.permute_preprocessing_impl(em.cuda(), E, kt, pad, -1, pts)
    P = int(tpe.sum().item())
    if dt_tok == torch.uint8:
        tok = torch.randint(0, 256, (T, H), dtype=torch.uint8)
    else:
        tok = randn((T, H), dtype=dt_tok, seed=T)
    width = pts if pts > 0 else E
    probs = torch.rand((T, width), generator=torch.Generator().manual_seed(1)) if with_probs else None
    sf = torch.rand((T, fp8_spt), generator=torch.Generator().manual_seed(2)) if fp8_spt else None
    tc = tok.cuda()
    out = torch.empty((P, H), dtype=tok.dtype, device="cuda")
    osf = torch.empty((P, fp8_spt), device="cuda") if fp8_spt else None
    opr = torch.empty((P,), device="cuda") if with_probs else None
    I.permute_impl(tc, out, sf.cuda() if sf is not None else None, osf, probs.cuda() if with_probs else None, opr,
                   rim, nd, pad, E, H, fp8_spt, dt_tok == torch.uint8, with_probs, P, pts)
    raw = tok.view(torch.uint8).numpy() if dt_tok == torch.uint8 else tok.view(torch.int16).numpy()
    eo, written, eosf, eopr = MO.permute(raw, rim.cpu().numpy(), int(nd.item()), pad, E, P,
                                         scaling_factor=sf.numpy() if sf is not None else None,
                                         probs=probs.numpy() if with_probs else None, probs_stride=pts)
    assert written.all()
    return dict(rim=rim, nd=nd, tpe=tpe, P=P, tok=tc, out=out, osf=osf, opr=opr, eo=eo, eosf=eosf, eopr=eopr,
                probs=probs, sf=sf, pts=pts)


PERM_CASES = [
    (torch.bfloat16, 16, 4, 512, 4096, 0, False, False),
    (torch.bfloat16, 16, 8, 300, 7168, 16, True, True),
    (torch.float16, 8, 2, 1000, 64, 64, True, False),
    (torch.bfloat16, 1, 1, 129, 256, 8, True, False),
    (torch.bfloat16, 64, 6, 257, 2048, 128, True, True),
]


@pytest.mark.parametrize("case", PERM_CASES, ids=[f"{c[0]}-E{c[1]}-k{c[2]}-T{c[3]}-H{c[4]}-p{c[5]}" for c in PERM_CASES])
def test_permute_vs_oracle_and_reference(case):
    dt, E, topk, T, H, pad, with_probs, aligned = case
    print(f"permute {case}", flush=True)
    r = _perm_case(dt, E, topk, T, H, pad, with_probs, aligned)
    assert_bytes_equal(r["out"].cpu().view(torch.int16).numpy(), r["eo"], "permuted tokens")
    if with_probs:
        assert_bytes_equal(r["opr"].cpu().numpy().view(np.uint32), r["eopr"].view(np.uint32), "permuted probs")
    R = ref_lib()
    if R is not None and R.ref_moe_preprocess is not None:
        out = torch.empty_like(r["out"])
        opr = torch.empty_like(r["opr"]) if with_probs else None
        assert R.ref_moe_permute(r["tok"].data_ptr(), out.data_ptr(), 2, None, None,
                                 r["probs"].cuda().data_ptr() if with_probs else None,
                                 opr.data_ptr() if with_probs else None, r["rim"].data_ptr(), r["nd"].data_ptr(),
                                 pad, E, H, 0, r["rim"].shape[0], r["pts"], stream()) == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), r["out"].view(torch.int16)), "vs reference permute"
        if with_probs:
            assert torch.equal(opr, r["opr"]), "vs reference permuted probs"


@pytest.mark.parametrize("pad", [0, 32])
def test_permute_fp8_with_scaling_factors(pad):
    E, topk, T, H, spt = 16, 4, 700, 7168, 56
    print(f"permute fp8 pad={pad}", flush=True)
    r = _perm_case(torch.uint8, E, topk, T, H, pad, False, False, fp8_spt=spt)
    assert_bytes_equal(r["out"].cpu().numpy(), r["eo"], "permuted fp8 bytes")
    assert_bytes_equal(r["osf"].cpu().numpy().view(np.uint32), r["eosf"].view(np.uint32), "permuted scales")
    R = ref_lib()
    if R is not None and R.ref_moe_preprocess is not None:
        out = torch.empty_like(r["out"])
        osf = torch.empty_like(r["osf"])
        assert R.ref_moe_permute(r["tok"].data_ptr(), out.data_ptr(), 1, r["sf"].cuda().data_ptr(), osf.data_ptr(),
                                 None, None, r["rim"].data_ptr(), r["nd"].data_ptr(), pad, E, H, spt,
                                 r["rim"].shape[0], 0, stream()) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, r["out"]) and torch.equal(osf, r["osf"]), "vs reference fp8 permute"


UNP_CASES = [
    (torch.bfloat16, 16, 4, 512, 4096, 0, False, False),
    (torch.bfloat16, 16, 8, 300, 7168, 16, True, True),
    (torch.float16, 8, 3, 1000, 72, 64, True, False),
    (torch.bfloat16, 1, 1, 130, 512, 0, True, False),   # single-expert copy kernel
    (torch.bfloat16, 64, 20, 257, 1024, 128, True, True),  # > 4 sources per token
]


@pytest.mark.parametrize("case", UNP_CASES, ids=[f"{c[0]}-E{c[1]}-k{c[2]}-T{c[3]}-H{c[4]}-p{c[5]}" for c in UNP_CASES])
def test_unpermute_vs_oracle_and_reference(case):
    dt, E, topk, T, H, pad, with_probs, aligned = case
    I = _impl()
    print(f"unpermute {case}", flush=True)
    r = _perm_case(dt, E, topk, T, H, pad, with_probs, aligned)
    P = r["P"]
    perm = randn((P, H), dtype=dt, seed=P)
    perm.view(-1)[::97] = -0.0  # negative zeros: summed rows drop the sign, the copy kernel keeps it
    pp = torch.rand(P, generator=torch.Generator().manual_seed(9)) if with_probs else None
    width = r["pts"] if r["pts"] > 0 else E
    out = torch.empty((T, H), dtype=dt, device="cuda")
    oprobs = torch.empty((T, width), device="cuda") if with_probs else None
    pc = perm.cuda()
    I.unpermute_impl(pc, out, pp.cuda() if with_probs else None, oprobs, r["rim"], r["nd"], E, H, with_probs,
                     r["pts"])
    sums, done, eprobs, _ = MO.unpermute(O.to_float32(perm), r["rim"].cpu().numpy(), int(r["nd"].item()), E, T,
                                         probs_stride=r["pts"], permuted_probs=pp.numpy() if with_probs else None)
    assert done.all()
    exp = O.bf16_round(sums) if dt == torch.bfloat16 else MO.round_f16(sums)
    got = out.float().cpu().numpy()
    assert_bytes_equal(got.view(np.uint32), exp.view(np.uint32), "unpermuted rows")
    if with_probs:
        assert_bytes_equal(oprobs.cpu().numpy().view(np.uint32), eprobs.view(np.uint32), "unpermuted probs")
    R = ref_lib()
    if R is not None and R.ref_moe_preprocess is not None:
        rout = torch.empty_like(out)
        rpr = torch.empty_like(oprobs) if with_probs else None
        assert R.ref_moe_unpermute(pc.data_ptr(), rout.data_ptr(), int(dt == torch.bfloat16),
                                   pp.cuda().data_ptr() if with_probs else None,
                                   rpr.data_ptr() if with_probs else None, r["rim"].data_ptr(), r["nd"].data_ptr(),
                                   E, H, T, r["pts"], stream()) == 0
        torch.cuda.synchronize()
        assert torch.equal(rout.view(torch.int16), out.view(torch.int16)), "vs reference unpermute"
        if with_probs:
            assert torch.equal(rpr, oprobs), "vs reference unpermuted probs"


# ---------------------------------------------------------------------------
# API level: the reference's own test cases (tests/pytorch/ops/test_moe_permute.py)
# ---------------------------------------------------------------------------


def _ops():
    import primus_turbo.pytorch as turbo

    return turbo.ops.moe_permute, turbo.ops.moe_unpermute


def _mask_map_ref(tokens, rm):
    """torch restatement of pytorch_permute_mask_map (permuatation_ref.py:10-33)."""
    T, E = rm.shape
    idx = torch.arange(T, device=rm.device).unsqueeze(0).expand(E, -1).masked_select(rm.T.contiguous())
    return tokens.index_select(0, idx), idx


def _tol(dt):
    return dict(atol=1e-2, rtol=1e-2) if dt == torch.bfloat16 else dict(atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("num_topk", [1, 2, 4, 8])
@pytest.mark.parametrize("kind", [torch.bool, torch.int32, torch.int64])
def test_moe_permutation_fwd_bwd(num_topk, kind):
    moe_permute, moe_unpermute = _ops()
    T, E, H = 4096, 16, 4096
    rm = _routing(T, E, num_topk, seed=1234).cuda()
    em = _expert_map(rm.cpu(), num_topk, kind).cuda()
    base = randn((T, H), seed=1).cuda()
    tok_ref = base.detach().float().requires_grad_(True)
    tok = base.detach().clone().requires_grad_(True)
    ref_perm, idx = _mask_map_ref(tok_ref, rm)
    grad_perm = randn(tuple(ref_perm.shape), seed=2).cuda()
    ref_perm.backward(grad_perm.float())
    perm, rim, tpe, ovf, nd, _, _ = moe_permute(tok, em, num_local_experts=E,
                                                num_topk=0 if kind == torch.bool else num_topk,
                                                probs_layout="routing_map")
    assert int(ovf.item()) == 0 and int(nd.item()) == T
    assert torch.equal(tpe.cpu(), rm.sum(0).to(torch.int64).cpu())
    perm.backward(grad_perm)
    assert torch.equal(perm, ref_perm.detach().bfloat16())
    torch.testing.assert_close(tok.grad.float(), tok_ref.grad, **_tol(torch.bfloat16))
    # unpermute forward / backward vs scatter_add in fp32
    unp_in = perm.detach().clone().requires_grad_(True)
    out, _ = moe_unpermute(unp_in, rim, nd, restore_shape=tok.shape, num_local_experts=E)
    ref_out = torch.zeros(T, H, device="cuda").scatter_add_(0, idx.unsqueeze(1).expand(-1, H), perm.float())
    torch.testing.assert_close(out.float(), ref_out, **_tol(torch.bfloat16))
    grad_unp = randn((T, H), seed=3).cuda()
    out.backward(grad_unp)
    assert torch.equal(unp_in.grad, grad_unp.index_select(0, idx))


@pytest.mark.parametrize("num_topk", [1, 2, 4])
@pytest.mark.parametrize("pad", [8, 16, 64])
def test_moe_permute_pad_multiple(num_topk, pad):
    moe_permute, _ = _ops()
    T, E, H = 1024, 8, 64
    rm = _routing(T, E, num_topk, seed=1234).cuda()
    tok = randn((T, H)).cuda()
    _, _, base, _, _, _, _ = moe_permute(tok, rm, num_local_experts=E, pad_multiple=0, probs_layout="routing_map")
    _, _, padded, _, _, _, _ = moe_permute(tok, rm, num_local_experts=E, pad_multiple=pad,
                                           probs_layout="routing_map")
    assert torch.equal(padded, ((base + pad - 1) // pad) * pad)
    assert (padded % pad == 0).all()


@pytest.mark.parametrize(
    "pad,cap_kind,expected",
    [
        (0, "uncapped", 0), (0, ("real", 0), 0), (0, ("real", +256), 0), (0, "half", 1), (0, "tiny", 1),
        (8, ("padded", 0), 0), (8, ("padded", +8), 0), (8, ("real", 0), 1), (8, "half", 1),
        (64, ("padded", 0), 0), (64, ("real", 0), 1),
    ],
)
def test_overflow_flag(pad, cap_kind, expected):
    moe_permute, _ = _ops()
    T, E, topk, H = 1024, 8, 2, 64
    rm = _routing(T, E, topk, seed=4321).cuda()
    per = rm.sum(0)
    real = int(per.sum().item())
    padded = int((((per + pad - 1) // pad) * pad).sum().item()) if pad > 0 else real
    if cap_kind == "uncapped":
        cap = -1
    elif cap_kind == "half":
        cap = real // 2
    elif cap_kind == "tiny":
        cap = 1
    else:
        b, d = cap_kind
        cap = (real if b == "real" else padded) + d
    _, _, _, ovf, _, _, _ = moe_permute(randn((T, H)).cuda(), rm, num_local_experts=E, pad_multiple=pad,
                                        num_permuted_tokens=cap, probs_layout="routing_map")
    assert int(ovf.item()) == expected


@pytest.mark.parametrize("with_probs", [False, True])
@pytest.mark.parametrize("pad", [0, 8])
def test_moe_permute_empty_input(with_probs, pad):
    moe_permute, moe_unpermute = _ops()
    E, H = 8, 64
    rm = torch.zeros((0, E), dtype=torch.bool, device="cuda")
    tok = torch.randn((0, H), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    probs = torch.zeros((0, E), device="cuda", requires_grad=True) if with_probs else None
    perm, rim, tpe, ovf, nd, _, pp = moe_permute(tok, rm, num_local_experts=E, pad_multiple=pad, probs=probs,
                                                 probs_layout="routing_map")
    assert perm.shape == (0, H) and tpe.shape == (E,) and int(tpe.sum().item()) == 0
    assert int(ovf.item()) == 0 and int(nd.item()) == 0
    assert rim.shape == (pad, 2 * E + 1)
    assert (pp is not None and pp.numel() == 0) if with_probs else pp is None
    if with_probs:
        torch.autograd.backward([perm, pp], [torch.zeros_like(perm), torch.zeros_like(pp)])
        assert probs.grad is not None and probs.grad.shape == (0, E)
    else:
        perm.backward(torch.zeros_like(perm))
    assert tok.grad is not None and tok.grad.shape == (0, H)
    p0 = torch.zeros((0, H), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    u, _ = moe_unpermute(p0, rim, nd, restore_shape=tok.shape, num_local_experts=E)
    assert u.shape == (0, H)
    u.backward(torch.zeros_like(u))
    assert p0.grad is not None and p0.grad.shape == (0, H)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64, torch.bool])
@pytest.mark.parametrize("with_probs", [False, True])
def test_moe_unpermute_nothing_routed_is_zero(dtype, with_probs):
    """Every token routes outside [0, E) (or to no local expert): nothing is
    dispatched, the permuted operand is empty, and the unpermuted tokens (and
    probs) must come back exactly zero -- not whatever the allocator held.
    The caching allocator is filled with a non-zero pattern first, so an
    unwritten output row cannot pass by landing on a zeroed page."""
    moe_permute, moe_unpermute = _ops()
    T, E, H, k = 300, 8, 256, 2
    if dtype == torch.bool:
        em = torch.zeros((T, E), dtype=torch.bool, device="cuda")
    else:
        em = torch.randint(E, 3 * E, (T, k), dtype=dtype, device="cuda")
        em[::3, 0] = -1
    layout = "routing_map" if dtype == torch.bool else "topk"
    tok = randn((T, H)).cuda()
    probs = torch.rand((T, E if dtype == torch.bool else k), device="cuda") if with_probs else None
    perm, rim, tpe, ovf, nd, _, pp = moe_permute(tok, em, num_local_experts=E, num_topk=0 if dtype == torch.bool else k,
                                                 probs=probs, probs_layout=layout)
    assert perm.shape == (0, H) and int(tpe.sum().item()) == 0 and int(nd.item()) == 0
    junk = torch.full((8 << 20,), 0x3F80, dtype=torch.int16, device="cuda")  # bf16 1.0 everywhere
    del junk
    u, up = moe_unpermute(perm, rim, nd, restore_shape=tok.shape, num_local_experts=E, permuted_probs=pp,
                          probs_topk_stride=0 if dtype == torch.bool else k)
    torch.cuda.synchronize()
    assert u.shape == (T, H) and torch.count_nonzero(u).item() == 0
    if with_probs:
        assert torch.count_nonzero(up).item() == 0


def _layout(rm, pad):
    T, E = rm.shape
    real = rm.sum(0).tolist()
    padded = [((r + pad - 1) // pad) * pad for r in real] if pad > 0 else list(real)
    st = torch.full((sum(padded),), -1, dtype=torch.long, device=rm.device)
    se = torch.full((sum(padded),), -1, dtype=torch.long, device=rm.device)
    off = 0
    for e in range(E):
        if real[e] > 0:
            st[off:off + real[e]] = rm[:, e].nonzero(as_tuple=True)[0]
            se[off:off + real[e]] = e
        off += padded[e]
    return st, se


@pytest.mark.parametrize("num_topk", [1, 2, 4])
@pytest.mark.parametrize("pad", [0, 16])
def test_moe_permute_with_probs_fwd_bwd(num_topk, pad):
    moe_permute, _ = _ops()
    T, E, H = 256, 8, 128
    rm = _routing(T, E, num_topk, seed=7).cuda()
    tok = randn((T, H)).cuda().requires_grad_(True)
    probs = (torch.rand((T, E), device="cuda") * rm.float()).requires_grad_(True)
    perm, rim, _, ovf, _, _, pp = moe_permute(tok, rm, num_local_experts=E, pad_multiple=pad, probs=probs,
                                              probs_layout="routing_map")
    assert int(ovf.item()) == 0 and pp.dtype == torch.float32 and pp.shape[0] == perm.shape[0]
    st, se = _layout(rm, pad)
    real = st >= 0
    exp = torch.zeros(st.numel(), device="cuda")
    exp[real] = probs.detach()[st[real], se[real]]
    assert torch.equal(pp, exp)
    gp = torch.randn_like(perm)
    gpp = torch.randn_like(pp)
    torch.autograd.backward([perm, pp], [gp, gpp])
    eg = torch.zeros_like(probs)
    eg[st[real], se[real]] = gpp[real]
    assert torch.equal(probs.grad, eg)
    assert tok.grad is not None and tok.grad.shape == tok.shape


@pytest.mark.parametrize("num_topk", [2, 8])
def test_moe_permute_topk_probs_layout(num_topk):
    """probs_layout='topk': probs [T, topk] follow the k of each (token, expert)."""
    moe_permute, moe_unpermute = _ops()
    T, E, H = 333, 32, 256
    rm = _routing(T, E, num_topk, seed=17)
    idx = _expert_map(rm, num_topk, torch.int64, shuffle_seed=3)
    probs = torch.rand((T, num_topk), device="cuda")
    perm, rim, tpe, ovf, nd, _, pp = moe_permute(randn((T, H)).cuda(), idx.cuda(), num_local_experts=E,
                                                 num_topk=num_topk, probs=probs, probs_layout="topk")
    st, se = _layout(rm.cuda(), 0)
    k_of = torch.full((T, E), -1, dtype=torch.long)
    for k in range(num_topk):
        k_of[torch.arange(T), idx[:, k]] = k
    k_of = k_of.cuda()
    assert torch.equal(pp, probs[st, k_of[st, se]])
    up, uprobs = moe_unpermute(perm, rim, nd, restore_shape=(T, H), num_local_experts=E, permuted_probs=pp,
                               probs_topk_stride=num_topk)
    assert torch.equal(uprobs, probs)


def test_moe_unpermute_with_probs_fwd_bwd():
    moe_permute, moe_unpermute = _ops()
    T, E, topk, H = 256, 8, 2, 128
    rm = _routing(T, E, topk, seed=11).cuda()
    tok = randn((T, H)).cuda()
    probs = torch.rand((T, E), device="cuda") * rm.float()
    perm, rim, _, _, nd, _, pp = moe_permute(tok, rm, num_local_experts=E, probs=probs, probs_layout="routing_map")
    pp = pp.detach().clone().requires_grad_(True)
    pin = perm.detach().clone().requires_grad_(True)
    ut, up = moe_unpermute(pin, rim, nd, restore_shape=tok.shape, num_local_experts=E, permuted_probs=pp)
    assert up.shape == (T, E)
    assert torch.equal(up, probs)
    gu = torch.randn_like(ut)
    gup = torch.randn_like(up)
    torch.autograd.backward([ut, up], [gu, gup])
    st, se = _layout(rm, 0)
    assert torch.equal(pp.grad, gup[st, se])
    assert torch.equal(pin.grad, gu[st])


@pytest.mark.parametrize("num_topk", [1, 4])
def test_moe_permute_fp16_fwd_bwd(num_topk):
    moe_permute, moe_unpermute = _ops()
    T, E, H = 1024, 8, 256
    rm = _routing(T, E, num_topk, seed=21).cuda()
    base = randn((T, H), dtype=torch.float16, seed=4).cuda()
    tok = base.clone().requires_grad_(True)
    perm, rim, _, ovf, nd, _, _ = moe_permute(tok, rm, num_local_experts=E, probs_layout="routing_map")
    ref_perm, idx = _mask_map_ref(base, rm)
    assert torch.equal(perm, ref_perm)
    g = torch.randn_like(perm)
    perm.backward(g)
    ref_grad = torch.zeros(T, H, device="cuda").scatter_add_(0, idx.unsqueeze(1).expand(-1, H), g.float())
    torch.testing.assert_close(tok.grad.float(), ref_grad, **_tol(torch.float16))
    out, _ = moe_unpermute(perm, rim, nd, restore_shape=tok.shape, num_local_experts=E)
    assert out.dtype == torch.float16
    torch.testing.assert_close(out.float(), num_topk * base.float(), **_tol(torch.float16))


@pytest.mark.parametrize("num_topk", [1, 2, 4])
@pytest.mark.parametrize("pad", [8, 64])
def test_moe_permute_pad_multiple_fwd_bwd(num_topk, pad):
    moe_permute, moe_unpermute = _ops()
    T, E, H = 512, 8, 128
    rm = _routing(T, E, num_topk, seed=33).cuda()
    base = randn((T, H), seed=5).cuda()
    t0 = base.clone().requires_grad_(True)
    p0, r0, _, _, n0, _, _ = moe_permute(t0, rm, num_local_experts=E, pad_multiple=0, probs_layout="routing_map")
    g0 = torch.randn_like(p0)
    p0.backward(g0)
    u0_in = p0.detach().clone().requires_grad_(True)
    u0, _ = moe_unpermute(u0_in, r0, n0, restore_shape=t0.shape, num_local_experts=E)
    gu = torch.randn_like(u0)
    u0.backward(gu)

    t1 = base.clone().requires_grad_(True)
    p1, r1, tpe1, _, n1, _, _ = moe_permute(t1, rm, num_local_experts=E, pad_multiple=pad,
                                            probs_layout="routing_map")
    st, _ = _layout(rm, pad)
    real = st >= 0
    assert p1.shape[0] == st.numel() and int(tpe1.sum().item()) == p1.shape[0]
    assert torch.equal(p1[real], p0.detach())
    assert (p1[~real] == 0).all()
    g1 = torch.zeros_like(p1)
    g1[real] = g0
    p1.backward(g1)
    assert torch.equal(t1.grad, t0.grad)
    u1_in = p1.detach().clone().requires_grad_(True)
    u1, _ = moe_unpermute(u1_in, r1, n1, restore_shape=t1.shape, num_local_experts=E, pad_multiple=pad)
    assert u1.shape == (T, H) and torch.equal(u1, u0)
    u1.backward(gu)
    assert torch.equal(u1_in.grad[real], u0_in.grad)
    assert (u1_in.grad[~real] == 0).all()
