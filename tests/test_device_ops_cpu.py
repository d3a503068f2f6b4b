"""The device ops of the op table (CPU): names, operand order and attr
plumbing of the bindings beyond the delivered forms, after the reference's
core table (packages/catopt-torch/src/catopt_torch/torch_bridge.py:1146-1902
of luisfuturist/catopt).

The bindings run torch's op where the operands live, so these run on host
tensors.  Each case checks what an attr changes against numpy (the closed
form, with the attr's value mattering: a non-default ``eps``, ``beta``,
``correction``, ``diagonal``, ``dim`` …), and the sink's feasibility bound
covers every name of the reference's core table but the two that need code
absent from this image.
"""

from __future__ import annotations

import math
import re

import numpy as np
import pytest
import torch

from catopt_amd.bindings import HIP_BINDINGS
from catopt_amd.device_ops import DEVICE_OPS
from catopt_amd.evaluator import HipIRModule
from catopt_amd.ir import IR, Const, Op, TensorType, Var
from tests.cpu_table import cpu_table

mk = Op.make
B = HIP_BINDINGS

# The reference core table's names (torch_bridge.py:1146-1902), as data.
CORE_NAMES = """
matmul add mul div sub rsub neg silu relu relu_ sigmoid tanh gelu exp pow square sqrt rsqrt sum mean amax amin max
min var_mean std_mean transpose reshape contiguous sdpa broadcast linear conv2d max_pool2d adaptive_avg_pool2d
concat pack chunk split dropout to clone getitem unbind stack expand flatten slice unsqueeze squeeze select embedding
index_select type_as cos sin float alias softmax rms_norm layer_norm broadcast_to repeat unflatten permute movedim
flip roll expand_as narrow gather take_along_dim scatter scatter_add scatter_reduce index_add index index_put
slice_scatter select_scatter argmax argmin prod var std any all nansum nanmean count_nonzero cumsum cumprod
logcumsumexp cummax cummin median kthvalue argsort topk sort mode linalg_vector_norm diag_sum clamp clamp_min
clamp_max hardtanh leaky_relu elu celu softplus softsign hardswish hardsigmoid mish relu6 glu prelu maximum minimum
fmax fmin fmod remainder xlogy atan2 heaviside isclose lerp addcmul addcdiv logical_and logical_or logical_xor
bitwise_and bitwise_or log_softmax abs sign floor ceil round frac trunc log log2 log10 log1p exp2 expm1 erf erfc
erfinv gammaln digamma i0 sinc reciprocal nan_to_num isnan isinf isfinite isposinf isneginf asin acos atan sinh cosh
asinh acosh atanh triu tril pad one_hot batch_norm group_norm instance_norm upsample_nearest2d upsample_bilinear2d
conv1d searchsorted nonzero outer einsum tensor_split unfold pixel_shuffle pixel_unshuffle hstack vstack arange zeros
ones empty randn rand full zeros_like ones_like full_like new_zeros new_ones new_empty new_full int long double half
bfloat16 bool byte char short detach detach_ _assert_tensor_metadata copy item numel masked_fill eq ne lt le gt ge
logical_not where aff aff_compose apply om om_elem om_compose om_apply aff_diag affd_compose applyd
""".split()
UNBOUND = {"deform_conv2d", "lstm.input"}  # torchvision / the recurrent kernel: absent here


def _x(*shape, seed=0):
    return torch.from_numpy(np.random.default_rng(seed).standard_normal(shape))


def test_every_core_name_is_bound():
    missing = [n for n in CORE_NAMES if n not in B]
    assert missing == []
    assert not UNBOUND & set(B)


def test_the_sink_bound_covers_the_device_ops():
    from catopt_amd.sink import HipSink

    assert set(DEVICE_OPS) <= HipSink().supported_ops


@pytest.mark.parametrize("name", sorted(n for n in DEVICE_OPS if re.fullmatch(
    r"abs|sign|floor|ceil|frac|trunc|log1p|exp2|expm1|erf|erfc|sin|cos|atan|sinh|cosh|asinh|reciprocal|sinc", n)))
def test_unary_ops_against_numpy(name):
    x = _x(5, 7, seed=hash(name) % 1000)
    npf = {"exp2": np.exp2, "expm1": np.expm1, "log1p": lambda v: np.log1p(np.abs(v)),
           "erf": np.vectorize(math.erf), "erfc": np.vectorize(math.erfc), "frac": lambda v: v - np.trunc(v),
           "reciprocal": lambda v: 1.0 / v, "sinc": np.sinc, "asinh": np.arcsinh, "atan": np.arctan}
    arg = x.abs() if name == "log1p" else x
    ref = npf.get(name, getattr(np, name, None))(x.numpy())
    np.testing.assert_allclose(B[name](arg).numpy(), ref, rtol=1e-12, atol=1e-12)


def test_clamp_family_reads_min_and_max():
    x = _x(40)
    np.testing.assert_array_equal(B["clamp"](x, min=-0.5, max=0.25).numpy(), np.clip(x.numpy(), -0.5, 0.25))
    np.testing.assert_array_equal(B["clamp"](x, -0.5).numpy(), np.maximum(x.numpy(), -0.5))
    np.testing.assert_array_equal(B["clamp_min"](x, min=0.1).numpy(), np.maximum(x.numpy(), 0.1))
    np.testing.assert_array_equal(B["clamp_max"](x, torch.tensor(0.2, dtype=torch.float64)).numpy(), np.minimum(x.numpy(), 0.2))
    np.testing.assert_array_equal(B["hardtanh"](x, min=-0.3, max=0.4).numpy(), np.clip(x.numpy(), -0.3, 0.4))


def test_activation_attrs():
    x = _x(50) * 4
    xn = x.numpy()
    beta, thr = 2.0, 3.0
    sp = np.where(beta * xn > thr, xn, np.log1p(np.exp(beta * xn)) / beta)
    np.testing.assert_allclose(B["softplus"](x, beta=beta, threshold=thr).numpy(), sp, rtol=1e-12)
    np.testing.assert_allclose(B["leaky_relu"](x, negative_slope=0.2).numpy(), np.where(xn > 0, xn, 0.2 * xn))
    np.testing.assert_allclose(B["leaky_relu"](x, torch.tensor(0.3, dtype=torch.float64)).numpy(), np.where(xn > 0, xn, 0.3 * xn))
    elu = 1.5 * np.where(2 * xn > 0, 2 * xn, 0.7 * np.expm1(2 * xn))
    np.testing.assert_allclose(B["elu"](x, alpha=0.7, scale=1.5, input_scale=2.0).numpy(), elu, rtol=1e-12)
    np.testing.assert_allclose(B["relu6"](x).numpy(), np.clip(xn, 0, 6))
    np.testing.assert_allclose(B["softsign"](x).numpy(), xn / (1 + np.abs(xn)), rtol=1e-12)


def test_comparisons_and_binary_ops():
    x, y = _x(6, 5, seed=1), _x(6, 5, seed=2)
    xn, yn = x.numpy(), y.numpy()
    for name, f in (("lt", np.less), ("le", np.less_equal), ("gt", np.greater), ("ge", np.greater_equal),
                    ("maximum", np.maximum), ("minimum", np.minimum), ("atan2", np.arctan2), ("fmod", np.fmod),
                    ("remainder", np.mod), ("outer", None)):
        if name == "outer":
            np.testing.assert_allclose(B[name](x[0], y[0]).numpy(), np.outer(xn[0], yn[0]))
            continue
        np.testing.assert_allclose(B[name](x, y).numpy(), f(xn, yn), rtol=1e-12, atol=1e-15)
    assert torch.equal(B["gt"](x, torch.tensor(0.0)), x > 0)  # an evaluated Const operand
    w = torch.tensor(0.25)
    np.testing.assert_allclose(B["lerp"](x, y, w).numpy(), xn + 0.25 * (yn - xn), rtol=1e-12)
    np.testing.assert_allclose(B["addcmul"](x, x, y, value=0.5).numpy(), xn + 0.5 * xn * yn, rtol=1e-12)
    np.testing.assert_allclose(B["addcdiv"](x, x, y, value=2).numpy(), xn + 2 * xn / yn, rtol=1e-12)


def test_reductions_read_dim_keepdim_and_correction():
    x = _x(4, 6, 5, seed=3)
    xn = x.numpy()
    np.testing.assert_allclose(B["var"](x, dim=1, correction=0).numpy(), xn.var(1, ddof=0), rtol=1e-12)
    np.testing.assert_allclose(B["std"](x, dim=(0, 2), keepdim=True).numpy(),
                               xn.std((0, 2), ddof=1, keepdims=True), rtol=1e-12)
    v, m = B["var_mean"](x, dim=2, correction=2)
    np.testing.assert_allclose(v.numpy(), xn.var(2, ddof=2), rtol=1e-12)
    np.testing.assert_allclose(m.numpy(), xn.mean(2), rtol=1e-12)
    np.testing.assert_allclose(B["prod"](x, dim=-1).numpy(), xn.prod(-1), rtol=1e-12)
    np.testing.assert_allclose(B["amin"](x, dim=0, keepdim=True).numpy(), xn.min(0, keepdims=True))
    assert float(B["max"](x)) == xn.max()  # no dim: the whole-tensor value
    vals, idx = B["max"](x, dim=1)
    np.testing.assert_array_equal(vals.numpy(), xn.max(1))
    np.testing.assert_array_equal(idx.numpy(), xn.argmax(1))
    np.testing.assert_array_equal(B["argmin"](x, dim=2).numpy(), xn.argmin(2))
    assert int(B["argmax"](x)) == int(xn.argmax())
    np.testing.assert_allclose(B["linalg_vector_norm"](x, ord=1, dim=-1).numpy(), np.abs(xn).sum(-1), rtol=1e-12)
    assert float(B["diag_sum"](x[0, :5])) == pytest.approx(np.trace(xn[0, :5]))
    np.testing.assert_array_equal(B["count_nonzero"](B["gt"](x, torch.tensor(0.0)), dim=1).numpy(), (xn > 0).sum(1))


def test_cumulative_and_ordering_ops():
    x = _x(3, 8, seed=4)
    xn = x.numpy()
    np.testing.assert_allclose(B["cumsum"](x, dim=1).numpy(), np.cumsum(xn, 1), rtol=1e-12)
    np.testing.assert_allclose(B["cumprod"](x, dim=0).numpy(), np.cumprod(xn, 0), rtol=1e-12)
    np.testing.assert_allclose(B["logcumsumexp"](x, dim=1).numpy(), np.logaddexp.accumulate(xn, 1), rtol=1e-12)
    np.testing.assert_array_equal(B["cummax"](x, dim=1)[0].numpy(), np.maximum.accumulate(xn, 1))
    np.testing.assert_array_equal(B["sort"](x, dim=1, descending=True)[0].numpy(), -np.sort(-xn, 1))
    np.testing.assert_array_equal(B["argsort"](x, dim=1).numpy(), np.argsort(xn, 1, kind="stable"))
    top = B["topk"](x, k=3, dim=1)[0].numpy()
    np.testing.assert_array_equal(top, -np.sort(-xn, 1)[:, :3])
    np.testing.assert_array_equal(B["kthvalue"](x, k=2, dim=1)[0].numpy(), np.sort(xn, 1)[:, 1])


def test_norms_read_their_shape_and_eps():
    x, w, b = _x(3, 4, 8, seed=5), _x(8, seed=6), _x(8, seed=7)
    xn = x.numpy()
    eps = 0.3  # large enough that a dropped eps fails
    mu, var = xn.mean(-1, keepdims=True), xn.var(-1, keepdims=True)
    ref = (xn - mu) / np.sqrt(var + eps) * w.numpy() + b.numpy()
    np.testing.assert_allclose(B["layer_norm"](x, w, b, dim=[8], eps=eps).numpy(), ref, rtol=1e-10)
    ref2 = (xn - xn.mean((-2, -1), keepdims=True)) / np.sqrt(xn.var((-2, -1), keepdims=True) + 1e-5)
    np.testing.assert_allclose(B["layer_norm"](x, normalized_shape=(4, 8)).numpy(), ref2, rtol=1e-9)
    g = x.reshape(3, 4, 2, 4)  # (N, C=4, 2, 4), two groups of two channels
    gn = g.numpy().reshape(3, 2, -1)
    gref = ((gn - gn.mean(-1, keepdims=True)) / np.sqrt(gn.var(-1, keepdims=True) + 0.1)).reshape(3, 4, 2, 4)
    np.testing.assert_allclose(B["group_norm"](g, num_groups=2, eps=0.1).numpy(), gref, rtol=1e-9)
    rm, rv, bw, bb = _x(4, seed=8), _x(4, seed=9).abs() + 0.5, _x(4, seed=10), _x(4, seed=11)
    bref = (g.numpy() - rm.numpy()[:, None, None]) / np.sqrt(rv.numpy()[:, None, None] + 1e-5) \
        * bw.numpy()[:, None, None] + bb.numpy()[:, None, None]
    np.testing.assert_allclose(B["batch_norm"](g, bw, bb, rm, rv).numpy(), bref, rtol=1e-9)


def test_masks_padding_and_encodings():
    x = _x(5, 5, seed=12)
    np.testing.assert_array_equal(B["triu"](x, diagonal=1).numpy(), np.triu(x.numpy(), 1))
    np.testing.assert_array_equal(B["tril"](x, diagonal=-1).numpy(), np.tril(x.numpy(), -1))
    p = B["pad"](x, pad=[1, 2], value=9.0).numpy()
    np.testing.assert_array_equal(p, np.pad(x.numpy(), ((0, 0), (1, 2)), constant_values=9.0))
    oh = B["one_hot"](torch.tensor([0, 3, 1]), num_classes=5).numpy()
    np.testing.assert_array_equal(oh, np.eye(5, dtype=np.int64)[[0, 3, 1]])
    np.testing.assert_array_equal(B["embedding"](x, torch.tensor([4, 0])).numpy(), x.numpy()[[4, 0]])


def test_layout_and_indexing():
    x = _x(2, 3, 4, seed=13)
    xn = x.numpy()
    np.testing.assert_array_equal(B["permute"](x, dims=[2, 0, 1]).numpy(), xn.transpose(2, 0, 1))
    np.testing.assert_array_equal(B["permute"](x).numpy(), xn.transpose(2, 1, 0))  # no dims: reversed
    np.testing.assert_array_equal(B["movedim"](x, source=0, destination=2).numpy(), np.moveaxis(xn, 0, 2))
    np.testing.assert_array_equal(B["flip"](x, dims=[1]).numpy(), xn[:, ::-1])
    np.testing.assert_array_equal(B["roll"](x, shifts=1, dims=2).numpy(), np.roll(xn, 1, 2))
    np.testing.assert_array_equal(B["narrow"](x, dim=2, start=1, length=2).numpy(), xn[:, :, 1:3])
    np.testing.assert_array_equal(B["unbind"](x, dim=1, index=2).numpy(), xn[:, 2])
    np.testing.assert_array_equal(B["repeat"](x, shape=[1, 2, 1]).numpy(), np.tile(xn, (1, 2, 1)))
    np.testing.assert_array_equal(B["broadcast_to"](x[:, :1], shape=[2, 3, 4]).numpy(),
                                  np.broadcast_to(xn[:, :1], (2, 3, 4)))
    np.testing.assert_array_equal(B["unflatten"](x, dim=2, sizes=[2, 2]).numpy(), xn.reshape(2, 3, 2, 2))
    np.testing.assert_array_equal(B["index_select"](x, dim=1, index=(2, 0)).numpy(), xn[:, [2, 0]])
    np.testing.assert_array_equal(B["index_select"](x, torch.tensor([1]), dim=2).numpy(), xn[:, :, [1]])
    idx = torch.tensor([[[3, 0, 1, 2]] * 3] * 2)
    np.testing.assert_array_equal(B["gather"](x, idx, dim=2).numpy(), np.take_along_axis(xn, idx.numpy(), 2))
    i0 = torch.tensor([1, 0])
    np.testing.assert_array_equal(B["index"](x, i0, layout=(False, True)).numpy(), xn[:, [1, 0]])
    put = B["index_put"](x, i0, torch.tensor(7.0, dtype=x.dtype), layout=(False, True)).numpy()
    want = xn.copy()
    want[:, [1, 0]] = 7.0
    np.testing.assert_array_equal(put, want)
    sa = B["scatter_add"](torch.zeros(2, 3, 4, dtype=x.dtype), idx, x, dim=2).numpy()
    ref = np.zeros_like(xn)
    np.put_along_axis(ref, idx.numpy(), xn, 2)  # idx is a permutation per row: add == put
    np.testing.assert_array_equal(sa, ref)
    sl = B["slice_scatter"](x, torch.zeros(2, 3, 2, dtype=x.dtype), dim=2, start=1, end=3).numpy()
    assert (sl[:, :, 1:3] == 0).all() and np.array_equal(sl[:, :, 0], xn[:, :, 0])
    ss = B["searchsorted"](torch.tensor([0.0, 1.0, 2.0]), torch.tensor([1.0, 1.5]), right=True).numpy()
    np.testing.assert_array_equal(ss, np.searchsorted([0.0, 1.0, 2.0], [1.0, 1.5], side="right"))


def test_creators_and_casts():
    assert B["zeros"](shape=[2, 3]).shape == (2, 3)
    f = B["full"](torch.tensor(2.5), shape=[2])
    assert f.tolist() == [2.5, 2.5]
    assert B["arange"](torch.tensor(1), torch.tensor(7), torch.tensor(2)).tolist() == [1, 3, 5]
    assert B["arange"](arg0=0, arg1=3).tolist() == [0, 1, 2]
    x = _x(3)
    assert B["zeros_like"](x, dtype="float32").dtype == torch.float32
    assert B["full_like"](x, torch.tensor(4.0)).tolist() == [4.0] * 3
    nf = B["new_full"](x, torch.tensor(1.5), shape=[2])
    assert nf.tolist() == [1.5, 1.5] and nf.dtype == x.dtype
    assert B["float"](torch.tensor([1, 2])).dtype == torch.float32
    assert B["float"](x, dtype="bfloat16").dtype == torch.bfloat16
    for n, dt in (("int", torch.int32), ("long", torch.int64), ("half", torch.float16), ("bool", torch.bool)):
        assert B[n](x).dtype == dt
    assert torch.equal(B["copy"](torch.zeros(2, 3), torch.arange(3.0)), torch.arange(3.0).expand(2, 3))
    assert B["numel"](torch.zeros(2, 5)) == 10


def test_device_ops_through_the_generic_evaluator():
    """A term that mixes the new ops with the existing ones evaluates as
    the same numpy composition (attrs travel through the IR)."""
    x = Var("x", TensorType((4, 6)))
    t = mk("cumsum", mk("clamp", mk("layer_norm", x, dim=[6], eps=0.5), min=-0.5, max=0.75), dim=1)
    t = mk("where", mk("gt", t, Const(0.0)), t, mk("softplus", t, beta=2.0))
    mod = HipIRModule(IR(t, [x]), {}, ops=cpu_table())
    xv = _x(4, 6, seed=14)
    xn = xv.numpy()
    ln = (xn - xn.mean(-1, keepdims=True)) / np.sqrt(xn.var(-1, keepdims=True) + 0.5)
    c = np.cumsum(np.clip(ln, -0.5, 0.75), 1)
    ref = np.where(c > 0, c, np.log1p(np.exp(2 * c)) / 2)
    np.testing.assert_allclose(mod(xv).numpy(), ref, rtol=1e-10)
