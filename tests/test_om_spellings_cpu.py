"""Host logic of the om executor's score spellings and of the causal fold.

The plan side of the widened om boundary, on the CPU:

* each score spelling catopt's laws deliver parses into ``(q, k, scale,
  mask / bias)`` — the sdpa-cat right-hand sides (``mul(q, fill(q, SC))``,
  key-axis ``concat`` of products, ``add(·, attnbias(m))``), and
  ``split`` / ``slice`` blocks of any of them;
* the two integer facts a kernel launch relies on are pinned against the
  bindings themselves, evaluated on the host: a block of a score is the
  product of the operand blocks (``_push_block``), and a block of the causal
  generator keeps exactly ``j <= i + off`` with the offset the plan derives
  (``_cmask_causal_off``), brute force over split sizes, indices, axes and
  generator offsets;
* weight-only masks are classified at construction (triangle → causal,
  other planes → keep-mask / bias, per-batch planes → the score path);
* ``specialize_causal`` mirrors the reference's own test
  (tests/test_optimize_edges.py:136-190 of luisfuturist/catopt).
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.bindings import HIP_BINDINGS
from catopt_amd.evaluator import eval_term
from catopt_amd.executors import HipOMModule
from catopt_amd.executors.om import (_block_start, _cmask_causal_off, _push_block, _qk_parts, mask_kwargs,
                                     parse_score)
from catopt_amd.folds import eval_const, is_causal_keep_mask, specialize_causal
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from tests.cpu_table import cpu_table

mk = Op.make
NEG_INF = Const(float("-inf"))


def _np(t):
    return t.detach().double().cpu().numpy()


def _host_eval(t, env, params=None):
    return eval_term(t, env, params or {}, cpu_table())


def _qkt(q, k):
    return mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))


def _cat_scores(q, ks, sc):
    qs = mk("mul", q, mk("fill", q, value=sc))
    return mk("concat", *[_qkt(qs, k) for k in ks], dim=-1)


# ------------------------------------------------------------------ parsing


def test_sdpa_cat_spelling_parses_to_one_product():
    q = Var("q", TensorType((1, 2, 16, 64)))
    k1, k2 = Var("k1", TensorType((1, 2, 8, 64))), Var("k2", TensorType((1, 2, 24, 64)))
    s = _cat_scores(q, [k1, k2], 0.125)
    sc = parse_score(mk("masked_fill", s, mk("cmask", s), NEG_INF))
    assert sc["q"] is q and sc["k"] == mk("concat", k1, k2, dim=-2)
    assert math.isclose(sc["scale"], 0.125) and sc["bias"] is None
    assert _cmask_causal_off(sc["mask"]) == 0
    # the attn_mask right-hand side: add(cat scores, attnbias(m)), either order
    m = Var("m", TensorType((16, 32)))
    for t in (mk("add", s, mk("attnbias", m)), mk("add", mk("attnbias", m), s)):
        sc = parse_score(t)
        assert sc["bias"] == mk("attnbias", m) and sc["mask"] is None and math.isclose(sc["scale"], 0.125)


def test_concat_of_products_with_different_queries_or_scales_does_not_parse():
    q1, q2, k1, k2 = (Var(n, TensorType((4, 8))) for n in ("q1", "q2", "k1", "k2"))
    assert _qk_parts(mk("concat", _qkt(q1, k1), _qkt(q2, k2), dim=-1)) is None
    mixed = mk("concat", _qkt(q1, k1), mk("mul", _qkt(q1, k2), Const(2.0)), dim=-1)
    assert _qk_parts(mixed) is None
    assert _qk_parts(mk("concat", _qkt(q1, k1), _qkt(q1, k2), dim=-2)) is None  # a query-axis concat
    # a finite fill of q is a scale; a fill with a non-numeric value is not
    assert _qk_parts(_qkt(mk("mul", q1, mk("fill", q1, value="SC")), k1))["q"] != q1


@pytest.mark.parametrize("op", ["split", "slice"])
@pytest.mark.parametrize("axis", [-1, -2])
def test_a_score_block_is_the_product_of_operand_blocks(op, axis):
    # the block _push_block builds, evaluated by the bindings, equals the
    # block of the evaluated score: pins the axis and attr mapping
    g = torch.Generator().manual_seed(3)
    q = Var("q", TensorType((2, 3, 12, 8)))
    k1, k2 = Var("k1", TensorType((2, 3, 8, 8))), Var("k2", TensorType((2, 3, 12, 8)))
    env = {n: torch.randn(sh, generator=g, dtype=torch.float64)
           for n, sh in (("q", (2, 3, 12, 8)), ("k1", (2, 3, 8, 8)), ("k2", (2, 3, 12, 8)))}
    S = _cat_scores(q, [k1, k2], 0.5)
    ext = 20 if axis == -1 else 12
    if op == "split":
        cases = [dict(sizes=(5, ext - 5), index=i) for i in (0, 1)] + [dict(sizes=4, index=2)]
        blocks = [mk("split", S, dim=axis, **c) for c in cases]
    else:
        dim = 4 + axis  # the slice binding takes a non-negative dim
        blocks = [mk("slice", S, dim=dim, start=a, end=b) for a, b in ((0, 5), (3, 11), (7, ext))]
    for blk in blocks:
        p = _qk_parts(blk)
        assert p is not None, blk
        want = _host_eval(blk, env)
        qv, kv = _host_eval(p["q"], env), _host_eval(p["k"], env)
        got = p["scale"] * (qv @ kv.transpose(-2, -1))
        assert got.shape == want.shape and torch.allclose(got, want, rtol=1e-12, atol=1e-12), blk


@pytest.mark.parametrize("T,K", [(9, 9), (7, 13), (12, 5)])
def test_cmask_block_offsets_brute_force(T, K):
    # every split / slice block of cmask(x, off), along keys, queries or both,
    # evaluated by the bindings, keeps exactly j <= i + result
    x = Var("x", TensorType((2, T, K)))
    xv = torch.zeros(2, T, K)
    checked = 0
    for off in (-3, 0, 2):
        base = mk("cmask", x, off=off) if off else mk("cmask", x)
        for kcut, qcut in itertools.product(range(0, K, 3), range(0, T, 4)):
            t = base
            if kcut:
                t = mk("split", t, sizes=(kcut, K - kcut), dim=-1, index=1)
            if qcut:
                t = mk("slice", t, dim=1, start=qcut, end=T)  # rank 3: dim 1 is the query axis
            res = _cmask_causal_off(t)
            masked = _host_eval(t, {"x": xv})[0]
            i = torch.arange(masked.shape[0])[:, None]
            j = torch.arange(masked.shape[1])[None, :]
            assert torch.equal(masked, ~(j <= i + res)), (off, kcut, qcut, res)
            checked += 1
    assert checked >= 18
    # a planted mistake: the key start counted with the wrong sign fails
    t = mk("split", mk("cmask", x), sizes=(3, K - 3), dim=-1, index=1)
    masked = _host_eval(t, {"x": xv})[0]
    i = torch.arange(T)[:, None]
    j = torch.arange(K - 3)[None, :]
    assert not torch.equal(masked, ~(j <= i + 3))


def test_block_start_reads_split_sizes_and_rejects_other_axes():
    x = Var("x", TensorType((2, 4, 10)))
    assert _block_start(mk("split", x, sizes=(3, 3, 4), dim=-1, index=2))[1:] == (-1, 6)
    assert _block_start(mk("split", x, sizes=4, dim=1, index=1))[1:] == (-2, 4)
    assert _block_start(mk("split", x, sizes=(1, 1), dim=0, index=1)) is None  # a batch axis
    assert _block_start(mk("slice", x, dim=2, start=2, end=8, step=2)) is None  # strided
    # a negative slice dim is axis 0 in the slice binding: not a score axis here
    assert _block_start(mk("slice", x, dim=-1, start=2, end=8)) is None
    y = Var("y", TensorType((4, 10)))
    assert _block_start(mk("slice", y, dim=-1, start=2, end=4))[1:] == (-2, 2)


def test_push_block_builds_operand_blocks():
    q = Var("q", TensorType((2, 6, 8)))
    blk = mk("split", mk("matmul", q, q), sizes=(2, 4), dim=-2, index=1)
    assert _push_block(blk, q) == mk("split", q, sizes=(2, 4), dim=-2, index=1)
    blk = mk("slice", mk("matmul", q, q), dim=2, start=1, end=5)
    assert _push_block(blk, q) == mk("slice", q, dim=1, start=1, end=5)


# ------------------------------------------------------------- plan classes


def _bias_form(m_term, T=16, d=64, blocks=None):
    q, k, v = (Var(n, TensorType((1, 2, T, d))) for n in "qkv")
    S = mk("mul", _qkt(q, k), Const(1 / 8.0))
    if blocks is None:
        root = mk("om_apply", mk("om_elem", mk("add", S, mk("attnbias", m_term)), v))
        return IR(root, [q, k, v] + ([m_term] if isinstance(m_term, Var) else []))
    leaves = []
    for i in range(len(blocks)):
        s_i = mk("split", S, sizes=blocks, dim=-1, index=i)
        b_i = mk("split", mk("attnbias", m_term), sizes=blocks, dim=-1, index=i)
        leaves.append(mk("om_elem", mk("add", s_i, b_i), mk("split", v, sizes=blocks, dim=-2, index=i)))
    tree = leaves[0]
    for lf in leaves[1:]:
        tree = mk("om_compose", tree, lf)
    return IR(mk("om_apply", tree), [q, k, v] + ([m_term] if isinstance(m_term, Var) else []))


def _kinds(mod):
    return [(lf["kind"], lf.get("mask_kind")) for lf in mod._plan["leaves"]]


def test_attnbias_masks_classify_at_construction():
    T = 16
    m = Param("m", TensorType((T, T)))
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    g = torch.Generator().manual_seed(5)
    rand_keep = torch.rand(T, T, generator=g) < 0.6
    rand_bias = torch.randn(T, T, generator=g, dtype=torch.float64)
    zero_inf = torch.zeros(T, T, dtype=torch.float64).masked_fill(~tril, float("-inf"))
    cases = [
        (tril, [("attn", "causal")]),
        (rand_keep, [("attn", "bool_const")]),
        (zero_inf, [("attn", "causal")]),
        (rand_bias, [("attn", "bias_const")]),
    ]
    for val, want in cases:
        mod = HipOMModule(_bias_form(m), {"m": val}, ops=cpu_table())
        assert _kinds(mod) == want, val.dtype
    lf = HipOMModule(_bias_form(m), {"m": rand_keep}, ops=cpu_table())._plan["leaves"][0]
    assert torch.equal(lf["keep"], rand_keep)
    lf = HipOMModule(_bias_form(m), {"m": rand_bias}, ops=cpu_table())._plan["leaves"][0]
    assert torch.equal(lf["bias_plane"], rand_bias.float())
    # a per-(batch, head) bias differs over the leading axes: the score path
    per_head = torch.randn(1, 2, T, T, generator=g, dtype=torch.float64)
    mh = Param("m", TensorType((1, 2, T, T)))
    assert _kinds(HipOMModule(_bias_form(mh), {"m": per_head}, ops=cpu_table())) == [("scores", None)]
    # an input mask is read per call
    mv = Var("m", TensorType((T, T)))
    assert _kinds(HipOMModule(_bias_form(mv), {}, ops=cpu_table())) == [("attn", "bias_runtime")]


def test_split_attnbias_blocks_fold_to_their_planes():
    T = 16
    m = Param("m", TensorType((T, T)))
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    mod = HipOMModule(_bias_form(m, blocks=(6, 10)), {"m": tril}, ops=cpu_table())
    lfs = mod._plan["leaves"]
    # block 0 keeps keys 0..5 of each row: j <= i; block 1 starts at key 6: j <= i - 6
    assert [(lf["kind"], lf["mask_kind"], lf.get("causal_off")) for lf in lfs] == \
        [("attn", "causal", 0), ("attn", "causal", -6)]
    g = torch.Generator().manual_seed(1)
    keep = torch.rand(T, T, generator=g) < 0.5
    lfs = HipOMModule(_bias_form(m, blocks=(6, 10)), {"m": keep}, ops=cpu_table())._plan["leaves"]
    assert torch.equal(lfs[0]["keep"], keep[:, :6]) and torch.equal(lfs[1]["keep"], keep[:, 6:])


def test_runtime_mask_kwargs_take_one_shared_plane():
    T = 8
    lf = {"mask_kind": "bias_runtime", "bias_term": "b", "attnbias": True}
    keep = torch.rand(T, T) < 0.5
    assert torch.equal(mask_kwargs(lf, lambda t: keep.expand(2, 3, T, T), T, T)["mask"], keep)
    bias = torch.randn(T, T)
    assert torch.equal(mask_kwargs(lf, lambda t: bias, T, T)["bias"], bias)
    assert mask_kwargs(lf, lambda t: torch.randn(2, T, T), T, T) is None  # differs over the batch
    lf2 = dict(lf, attnbias=False)
    assert mask_kwargs(lf2, lambda t: keep, T, T) is None  # add(s, bool) is not a mask
    lf3 = {"mask_kind": "runtime", "mask": "m"}
    assert torch.equal(mask_kwargs(lf3, lambda t: ~keep, T, T)["mask"], keep)
    # a key-padding plane (one query row) broadcasts over the score's rows
    pad = torch.tensor([[True, True, True, False, False, False, False, False]])
    got = mask_kwargs(lf3, lambda t: ~pad.reshape(1, 1, 1, T), T, T)["mask"]
    assert got.shape == (T, T) and torch.equal(got, pad.expand(T, T))
    # planes that do not broadcast to the score's (Tq, Tk) take the score path
    assert mask_kwargs(lf3, lambda t: ~keep[:4], T, T) is None
    assert mask_kwargs(lf, lambda t: torch.randn(T, T + 1), T, T) is None


def test_const_planes_fit_the_score_shape_at_call_time():
    """A weight-only plane with one query row is never read as a triangle of
    that one row: a 0/-inf bias keeping keys 0..2 of 8 keeps keys 0..2 for
    every query row, and a (T, T) triangle is causal only for a (T, T)
    score."""
    from catopt_amd.executors.om import _bias_const, _keep_const
    T = 8
    bias = torch.full((1, 1, 1, T), float("-inf"))
    bias[..., :3] = 0.0
    lf: dict = {}
    _bias_const(lf, bias)
    kw = mask_kwargs(lf, None, T, T)
    assert "causal" not in kw and torch.equal(kw["mask"], (bias[0, 0] == 0).expand(T, T))
    assert mask_kwargs(lf, None, 1, T) == {"causal": True, "causal_off": 2}  # one row: the same set
    tri = torch.ones(T, T, dtype=torch.bool).tril()
    lf = {}
    _keep_const(lf, tri)
    assert lf["mask_kind"] == "causal" and mask_kwargs(lf, None, T, T) == {"causal": True, "causal_off": 0}
    assert mask_kwargs(lf, None, T, T + 1) is None  # the plane is (T, T)
    lf = {}
    _keep_const(lf, torch.rand(T, 1) < 0.5)  # a row mask broadcasts over the keys
    assert mask_kwargs(lf, None, T, 5)["mask"].shape == (T, 5)
    lf = {}
    _bias_const(lf, torch.randn(1, T))
    assert lf["mask_kind"] == "bias_const" and mask_kwargs(lf, None, 3, T)["bias"].shape == (3, T)


def test_every_om_tree_plans_and_host_calls_run_the_generic_module():
    # explicit-score leaves and packaged carriers plan as well (the
    # reference's slice / stack modes); host inputs run the generic module
    T, d = 6, 4
    s1, s2 = Var("s1", TensorType((T, 3))), Var("s2", TensorType((T, 5)))
    v1, v2 = Var("v1", TensorType((3, d))), Var("v2", TensorType((5, d)))
    mm, ll, aa = Var("m", TensorType((T, 1))), Var("l", TensorType((T, 1))), Var("a", TensorType((T, d)))
    tree = mk("om_compose", mk("om_compose", mk("om_elem", s1, v1), mk("om", mm, ll, aa)), mk("om_elem", s2, v2))
    ir = IR(mk("om_apply", tree), [s1, v1, s2, v2, mm, ll, aa])
    mod = HipOMModule(ir, {}, ops=cpu_table())
    assert mod.leaf_kinds == ["scores", "om", "scores"]
    g = np.random.default_rng(0)
    xs = [g.standard_normal(sh) for sh in ((T, 3), (3, d), (T, 5), (5, d))]
    xs[0][2] = -np.inf  # a fully masked row in one block
    f0 = oracle.om_elem(g.standard_normal((T, 2)), g.standard_normal((2, d)))
    ins = [torch.from_numpy(a) for a in xs] + [torch.from_numpy(a) for a in f0]
    out = mod(*ins)
    assert mod.fallbacks == 1
    ref = oracle.om_apply(oracle.om_compose(oracle.om_compose(oracle.om_elem(xs[0], xs[1]), f0),
                                            oracle.om_elem(xs[2], xs[3])))
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]


# ------------------------------------------------------- specialize_causal


def _T(*shape):
    return TensorType(tuple(shape))


def test_is_causal_keep_mask_cases():
    T = 4
    tril = torch.tril(torch.ones(T, T, dtype=torch.bool))
    assert is_causal_keep_mask(tril, (2, T, T))
    add = torch.zeros(T, T).masked_fill(~tril, float("-inf"))
    assert is_causal_keep_mask(add, (2, T, T))
    assert not is_causal_keep_mask(tril, (T,))
    assert not is_causal_keep_mask(torch.ones(T, T + 1, dtype=torch.bool), (2, T, T + 1))
    assert not is_causal_keep_mask(tril, (2, T + 1, T + 1))
    assert not is_causal_keep_mask(torch.rand(T, T, generator=torch.Generator().manual_seed(0)) > 0.5, (2, T, T))
    assert not is_causal_keep_mask(torch.ones(T, dtype=torch.bool), (2, T, T))
    # q's shape unknown: a square mask of T > 1 fixes Tq = Tk = T; T = 1 does not
    assert is_causal_keep_mask(tril, None)
    assert not is_causal_keep_mask(torch.ones(1, 1, dtype=torch.bool), None)


def test_specialize_causal_drops_param_tril_mask():
    ops = cpu_table()
    q, k, v = (Var(n, _T(1, 4, 4)) for n in "qkv")
    mp = Param("mask", _T(4, 4))
    env = {"mask": torch.tril(torch.ones(4, 4, dtype=torch.bool))}
    sdpa = mk("sdpa", q, k, v, mp)
    memo: dict = {}
    out = specialize_causal(sdpa, env, memo, ops=ops)
    assert out.attrs.get("arg5") is True and len(out.args) == 3 and memo.get("_hit") is True
    sdpa2 = mk("sdpa", q, k, v, mp, arg5=True)  # already causal
    assert len(specialize_causal(sdpa2, env, ops=ops).args) == 4
    out3 = specialize_causal(sdpa, {"mask": torch.ones(4, 4, dtype=torch.bool)}, ops=ops)
    assert len(out3.args) == 4 and not out3.attrs.get("arg5")
    mv = Var("m", _T(4, 4))  # a runtime mask cannot be folded
    memo4: dict = {}
    assert len(specialize_causal(mk("sdpa", q, k, v, mv), env, memo4, ops=ops).args) == 4
    assert "_hit" not in memo4
    leaf = Var("x", _T(2))
    assert specialize_causal(leaf, env, ops=ops) is leaf
    memo5: dict = {}
    assert specialize_causal(sdpa, env, memo5, ops=ops) is specialize_causal(sdpa, env, memo5, ops=ops)


def test_specialize_causal_evaluates_parameter_only_subtrees_and_rewrites_inside():
    ops = cpu_table()
    q, k, v = (Var(n, _T(1, 4, 4)) for n in "qkv")
    mp = Param("mask", _T(4, 4))
    env = {"mask": torch.ones(4, 4, dtype=torch.bool).triu(1)}  # the masked set
    keep = mk("logical_not", mp)
    body = mk("add", mk("sdpa", q, k, v, keep), q)
    out = specialize_causal(body, env, ops=ops)
    assert out.op == "add" and out.args[0].attrs.get("arg5") is True and len(out.args[0].args) == 3
    # a subtree that raises, or an unbound Param, is not foldable
    assert eval_const(mk("reshape", mp, shape=(3, 3)), env, ops) is None
    assert eval_const(Param("gone", _T(2)), env, ops) is None
    assert eval_const(mk("logical_not", Var("x", _T(4, 4))), env, ops) is None
    assert torch.equal(eval_const(keep, env, ops), ~env["mask"])


def test_torch_sdpa_gives_zero_rows_where_every_key_is_masked():
    # the fused sdpa binding's empty-row value (0, not om_apply's NaN) is
    # torch's own: checked here on the host op
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 1, 4, 8, generator=g) for _ in range(3))
    m = torch.ones(4, 4, dtype=torch.bool)
    m[2] = False
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=m)
    assert torch.equal(out[0, 0, 2], torch.zeros(8)) and torch.isfinite(out).all()
    assert HIP_BINDINGS["sdpa"] is not None
