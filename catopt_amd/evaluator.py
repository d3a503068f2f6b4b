"""The generic executor: a slot-tape evaluator over HIP bindings.

``HipIRModule`` is the counterpart of the reference's ``IRModule``
(luisfuturist/catopt ``packages/catopt-torch/src/catopt_torch/torch_bridge.py``:
class at :2386-2874, ``_EvalPlan`` slot tape at :2077-2269,
``_fold_weight_chains`` at :2456-2686).  It is what ``HipSink.lower`` returns
and what every planned executor embeds as ``eval_mod`` — the complete
fallback for terms whose root does not match a planned pattern.

Construction does three things, in order:

1. **Weight fold** (a construction-time pass, as ``_fold_weight_chains``):
   every subterm whose leaves are only Params and Consts is evaluated once
   and replaced by a fused Param.  ``matmul(Param, Param)`` folds through the
   HIP GEMM; the shallow elementwise/view/reduction list folds when all of
   its operands already are leaves.  The carrier generators (``decay``,
   ``decay_vec``, ``cmask``) and the slice/gather family are not folded,
   exactly as in the reference.
2. **Epilogue fusion** (this package's lowering choice, no reference
   counterpart): patterns whose intermediate would otherwise round-trip
   HBM become one kernel —
   * ``add(linear(x, W, b), c)`` chains with Param addends: the addends are
     folded into the GEMM's bias (the ``ASSOC_LINEAR_BIAS`` RHS spine,
     ``laws/tensor.py:1374-1394``);
   * ``mul(silu(chunk(L, 2, -1, 0)), chunk(L, 2, -1, 1))`` with
     ``L = linear(h, W)`` (the ``SWIGLU_FUSE`` RHS, ``laws/tensor.py:1485-1519``),
     its ``split`` spelling, and ``glu(linear(h, W))`` (``GLU_FOLD``,
     ``laws/tensor.py:585-601``): one GEMM with the gate applied in
     registers;
   * ``mul(silu(linear(h, A)), linear(h, B))`` with Param ``A``, ``B``: the
     concat ``[A; B]`` is built once and takes the same path.
3. **Tape build**: the folded, fused DAG is laid out in post-order as
   ``(op, operand refs, attrs)`` steps.  Bindings are resolved per call from
   the op table, so a binding registered after construction applies.  A
   missing binding raises ``ValueError`` (torch_bridge.py:2241-2244).

Params are registered as buffers, so ``module.to(device)`` moves them.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from . import _lib as L
from . import kernels as K
from .bindings import HipOpTable, attr_of, scalar_value
from .graphs import global_module_hooks, record_graph, signature
from .ir import IR, Const, Op, Param, TensorType, Var, is_op, postorder

__all__ = ["HipIRModule", "FOLD_OPS", "eval_term"]

#: Ops folded at construction when every operand is a Param/Const
#: (torch_bridge.py:2477-2684 lists the same families; the carrier
#: generators and slice/gather views stay out).
FOLD_OPS = frozenset({
    "add", "mul", "sub", "div", "neg", "square", "sqrt", "rsqrt", "sigmoid", "silu", "tanh",
    "gelu", "exp", "pow", "concat", "relu", "glu", "softmax", "sum", "mean", "amax",
    "transpose", "permute", "reshape", "view", "unsqueeze", "squeeze", "flatten", "tril",
    "contiguous", "to", "alias", "clone", "dropout", "logical_not", "eq", "ne", "where",
})

class _BufferParams:
    """Param name -> the module buffer holding its value, read at lookup
    (no per-call copy of the map)."""

    __slots__ = ("_bufs", "_names")

    def __init__(self, bufs: dict, names: dict) -> None:
        self._bufs, self._names = bufs, names

    def __getitem__(self, name: str) -> torch.Tensor:
        return self._bufs[self._names[name]]

    def __contains__(self, name: object) -> bool:
        return name in self._names

    def get(self, name: str, default: Any = None) -> Any:
        attr = self._names.get(name)
        return default if attr is None else self._bufs[attr]

    def keys(self):
        return self._names.keys()

    def items(self):
        return ((n, self._bufs[a]) for n, a in self._names.items())

    def __iter__(self):
        return iter(self._names)

    def __len__(self) -> int:
        return len(self._names)


def _is_param(t: Any) -> bool:
    return isinstance(t, Param) or (not is_op(t) and hasattr(t, "name") and type(t).__name__ == "Param")


def _is_var(t: Any) -> bool:
    return isinstance(t, Var) or (not is_op(t) and hasattr(t, "name") and type(t).__name__ == "Var")


def _is_const(t: Any) -> bool:
    return isinstance(t, Const) or (not is_op(t) and hasattr(t, "value") and type(t).__name__ == "Const")


def _mk(op: str, *args: Any, **attrs: Any) -> Op:
    return Op.make(op, *args, **attrs)


def eval_term(t: Any, env: dict, params: dict, ops: HipOpTable, memo: dict | None = None,
              default: Any = None) -> Any:
    """Evaluate ``t`` against ``env`` (Var name -> value) and ``params``.

    Iterative post-order with a content-keyed memo, so shared subterms run
    once and deep chains do not recurse.  A Var missing from ``env``
    evaluates to ``default`` (the single-input ``self`` fallback of
    ``IRModule``); a Const is a 0-dim tensor (torch_bridge.py:2335-2336).
    """
    memo = {} if memo is None else memo

    def leaf(a):
        if _is_var(a):
            return env.get(a.name, default)
        if _is_param(a):
            try:
                return params[a.name]
            except KeyError:
                raise KeyError(f"no value bound for Param {a.name!r}") from None
        if _is_const(a):
            return torch.tensor(a.value)
        raise TypeError(f"unknown term leaf {a!r}")

    if not is_op(t):
        return leaf(t)
    for node in postorder(t):
        if node in memo:
            continue
        fn = ops[node.op]
        vals = [memo[a] if is_op(a) else leaf(a) for a in node.args]
        memo[node] = fn(*vals, **node.attrs)
    return memo[t]


# ------------------------------------------------------------------ fused ops


def _hip_linear(x, w, b=None, **kw):
    if x.device.type != "cuda":
        raise ValueError("the fused linear runs on the ROCm device only")
    return K.linear(x, w, b)


def _hip_swiglu(x, w, **kw):
    return K.linear(x, w, epilogue=L.EPI_SILU_MUL)


def _hip_glu(x, w, **kw):
    return K.linear(x, w, epilogue=L.EPI_GLU)


FUSED_BINDINGS = {
    "hip_linear": _hip_linear,
    "hip_swiglu": _hip_swiglu,
    "hip_glu": _hip_glu,
}


# -------------------------------------------------------------------- module


class HipIRModule(nn.Module):
    """Generic executor for any IR term (see the module docstring)."""

    is_batched = False

    def __init__(self, ir: IR, param_values: dict | None = None, *, ops: HipOpTable | None = None,
                 device: Any = None, fold: bool = True, fuse: bool = True) -> None:
        super().__init__()
        self._ir = ir
        self._inputs = list(ir.inputs)
        self.ops = ops if ops is not None else HipOpTable()
        self.stats: dict = {"folded": 0, "fused": {}}
        self._buf_names: dict[str, str] = {}
        values = dict(param_values or {})
        for p in ir.params.values() if isinstance(ir.params, dict) else ir.params:
            shape = getattr(getattr(p, "typ", None), "shape", None)
            if p.name not in values and shape is not None:
                # no value given: a random init, unknown extents taken as 1
                # (torch_bridge.py:2722-2764); a Param of unknown rank stays
                # unbound and raises when evaluated
                values[p.name] = torch.randn(*[1 if d is None else int(d) for d in shape]) * 0.02
        for name, v in values.items():
            t = torch.as_tensor(v)
            if device is not None:
                t = t.to(device)
            self._set_param(name, t.detach())
        self._fold_memo: dict = {}
        root = ir.root
        if fold:
            root = self._fold_weight_chains(root)
        if fuse:
            root = self._fuse(root)
        self._root = root
        self._prune()
        self._tape = _Tape(root)
        self._graph = None  # set by capture_cuda_graph (a plain attribute: forward reads it per call)

    def __call__(self, *xs: Any) -> Any:
        # nn.Module's call path (hook dispatch) costs microseconds per call,
        # the same order as the small kernels a step launches; without hooks
        # it only calls forward
        if self._forward_hooks or self._forward_pre_hooks or global_module_hooks():
            return super().__call__(*xs)
        return self.forward(*xs)

    # -- parameters -------------------------------------------------------

    def _set_param(self, name: str, t: torch.Tensor) -> None:
        attr = self._buf_names.get(name)
        if attr is None:
            self._nbuf = getattr(self, "_nbuf", 0) + 1
            attr = f"p{self._nbuf}_" + "".join(c if c.isalnum() else "_" for c in name)[:40]
            self._buf_names[name] = attr
        self.register_buffer(attr, t, persistent=False)

    @property
    def _param_map(self) -> "_BufferParams":
        # re-read per call (the reference's contract: a replaced buffer is
        # picked up), straight from the buffer dict rather than through
        # nn.Module.__getattr__, which costs microseconds per name
        return _BufferParams(self._buffers, self._buf_names)

    # The parameters live in non-persistent buffers under attribute-safe
    # names; the state dict speaks the IR's Param names instead, as the
    # reference's modules do (torch_bridge.py:2722-2764: one entry per live
    # Param, fused ones included).  Loading copies into the existing buffers,
    # so a captured graph, which baked their addresses, sees the new values.

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        for name, attr in self._buf_names.items():
            t = self._buffers[attr]
            destination[prefix + name] = t if keep_vars else t.detach()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        for name, attr in self._buf_names.items():
            key = prefix + name
            if key not in state_dict:
                missing_keys.append(key)
                continue
            buf, v = self._buffers[attr], state_dict[key]
            if not isinstance(v, torch.Tensor) or tuple(v.shape) != tuple(buf.shape):
                error_msgs.append(f"size mismatch for {key}: copying a param with shape "
                                  f"{tuple(getattr(v, 'shape', ()))}, the shape in current model is "
                                  f"{tuple(buf.shape)}.")
                continue
            with torch.no_grad():
                buf.copy_(v)
        if strict:
            for key in state_dict:
                if key.startswith(prefix):
                    head = key[len(prefix):].split(".", 1)
                    if (head[0] not in self._modules) if len(head) > 1 else (head[0] not in self._buf_names):
                        unexpected_keys.append(key)

    def _pv(self, t: Any) -> torch.Tensor | None:
        if _is_param(t) and t.name in self._buf_names:
            return self._buffers[self._buf_names[t.name]]
        return None

    def _new_param(self, value: torch.Tensor) -> Param:
        self._nfused = getattr(self, "_nfused", 0) + 1
        name = f"fused_{self._nfused}"
        while name in self._buf_names:
            name += "_"
        self._set_param(name, value.detach())
        return Param(name, TensorType(tuple(int(d) for d in value.shape)))

    def _prune(self) -> None:
        live = {a.name for n in postorder(self._root) for a in n.args if _is_param(a)}
        if _is_param(self._root):
            live.add(self._root.name)
        for name in [n for n in self._buf_names if n not in live]:
            delattr(self, self._buf_names.pop(name))

    # -- construction passes ------------------------------------------------

    def _fold_weight_chains(self, root: Any) -> Any:
        """Bottom-up replacement of weight-only subtrees by fused Params."""
        if not is_op(root):
            return root
        for node in postorder(root):
            if node in self._fold_memo:
                continue
            args = tuple(self._fold_memo.get(a, a) if is_op(a) else a for a in node.args)
            new = _mk(node.op, *args, **dict(node.attrs)) if args != node.args else node
            folded = new
            leafy = all(_is_param(a) or _is_const(a) for a in args)
            if leafy and any(_is_param(a) for a in args):
                fold_it = (new.op == "matmul" and all(_is_param(a) for a in args)) or new.op in FOLD_OPS
                if fold_it:
                    vals = [self._pv(a) if _is_param(a) else torch.tensor(a.value) for a in args]
                    try:
                        with torch.no_grad():
                            out = self.ops[new.op](*vals, **new.attrs)
                    except Exception:  # a fold that cannot run stays a runtime op
                        out = None
                    if isinstance(out, torch.Tensor):
                        folded = self._new_param(out)
                        self.stats["folded"] += 1
            self._fold_memo[node] = folded
        return self._fold_memo[root]

    def _count(self, kind: str) -> None:
        self.stats["fused"][kind] = self.stats["fused"].get(kind, 0) + 1

    def _fuse(self, root: Any) -> Any:
        """Rewrite the epilogue patterns of the module docstring bottom-up."""
        if not is_op(root):
            return root
        memo: dict = {}
        for node in postorder(root):
            args = tuple(memo.get(a, a) if is_op(a) else a for a in node.args)
            new = _mk(node.op, *args, **dict(node.attrs)) if args != node.args else node
            memo[node] = self._fuse_one(new)
        return memo[root]

    def _vec_param(self, t: Any, n: int, dtype: torch.dtype) -> torch.Tensor | None:
        v = self._pv(t)
        if v is None or v.dim() != 1 or v.shape[0] != n or v.dtype != dtype:
            return None
        return v

    def _fuse_one(self, t: Op) -> Any:
        # linear(x, W[, b]) with Param weight/bias on the device -> hip_linear
        if t.op == "linear" and len(t.args) in (2, 3) and _is_param(t.args[1]):
            w = self._pv(t.args[1])
            if w is not None and w.dim() == 2 and w.dtype in (torch.float32, torch.bfloat16):
                b = t.args[2] if len(t.args) == 3 else t.attrs.get("bias")
                if b is None or _is_param(b):
                    bv = None if b is None else self._vec_param(b, w.shape[0], w.dtype)
                    if b is None or bv is not None:
                        self._count("linear")
                        return _mk("hip_linear", *( (t.args[0], t.args[1]) if b is None else (t.args[0], t.args[1], b)))
        # add(hip_linear(...), c) / add(c, hip_linear(...)) with a Param vector c
        if t.op == "add" and len(t.args) == 2:
            for lin, c in ((t.args[0], t.args[1]), (t.args[1], t.args[0])):
                if is_op(lin, "hip_linear") and _is_param(c) and _is_param(lin.args[1]):
                    w = self._pv(lin.args[1])
                    cv = self._vec_param(c, w.shape[0], w.dtype)
                    if cv is None:
                        continue
                    with torch.no_grad():
                        if len(lin.args) == 3:
                            bias = (self._pv(lin.args[2]).float() + cv.float()).to(w.dtype)
                        else:
                            bias = cv.clone()
                    self._count("bias_add")
                    return _mk("hip_linear", lin.args[0], lin.args[1], self._new_param(bias))
        # glu(hip_linear(h, W)) over the last axis -> hip_glu
        if t.op == "glu" and len(t.args) == 1 and int(attr_of(t.attrs, "dim", default=-1)) == -1:
            lin = t.args[0]
            if is_op(lin, "hip_linear") and len(lin.args) == 2 and self._pv(lin.args[1]).dtype == torch.bfloat16:
                self._count("glu")
                return _mk("hip_glu", lin.args[0], lin.args[1])
        # mul(silu(half0(L)), half1(L)) -> hip_swiglu; mul(silu(lin A), lin B) -> concat + hip_swiglu
        if t.op == "mul" and len(t.args) == 2:
            for s, u in ((t.args[0], t.args[1]), (t.args[1], t.args[0])):
                if not is_op(s, "silu", 1):
                    continue
                g = s.args[0]
                lin_g, ix_g = self._half_of_linear(g)
                lin_u, ix_u = self._half_of_linear(u)
                if lin_g is not None and lin_g is lin_u and (ix_g, ix_u) == (0, 1):
                    w = self._pv(lin_g.args[1])
                    if w.dtype == torch.bfloat16:
                        self._count("swiglu")
                        return _mk("hip_swiglu", lin_g.args[0], lin_g.args[1])
                if is_op(g, "hip_linear", 2) and is_op(u, "hip_linear", 2) and g.args[0] == u.args[0]:
                    wa, wb = self._pv(g.args[1]), self._pv(u.args[1])
                    if wa.shape == wb.shape and wa.dtype == wb.dtype == torch.bfloat16:
                        with torch.no_grad():
                            wcat = torch.cat([wa, wb], 0).contiguous()
                        self._count("swiglu_concat")
                        return _mk("hip_swiglu", g.args[0], self._new_param(wcat))
        return t

    def _half_of_linear(self, t: Any) -> tuple:
        """``(L, i)`` when ``t`` is half ``i`` of ``L = hip_linear(h, W)``
        along the last axis (``chunk(L, 2, -1, i)`` or the equal ``split``)."""
        if not is_op(t) or len(t.args) != 1:
            return None, None
        lin = t.args[0]
        if not is_op(lin, "hip_linear", 2):
            return None, None
        w = self._pv(lin.args[1])
        n = w.shape[0]
        dim = int(attr_of(t.attrs, "dim", default=-1))
        if dim != -1 or n % 2:
            return None, None
        if t.op == "chunk" and int(attr_of(t.attrs, "chunks", default=2)) == 2:
            return lin, int(attr_of(t.attrs, "index", default=0))
        if t.op == "split":
            sz = attr_of(t.attrs, "sizes", "split_size", default=None)
            halves = (list(sz) == [n // 2, n // 2]) if isinstance(sz, (list, tuple)) else sz == n // 2
            if halves:
                return lin, int(attr_of(t.attrs, "index", default=0))
        return None, None

    # -- execution ------------------------------------------------------------

    def _env(self, xs: tuple) -> tuple[Any, dict]:
        x = xs[0] if xs else None
        env = {"self": x}
        for i, v in enumerate(self._inputs):
            env[v.name] = xs[i] if i < len(xs) else x
        return x, env

    def _eval(self, t: Any, env: dict, x: Any, memo: dict) -> Any:
        """Evaluate a subterm (used by the planned executors for their leaves)."""
        ops = self._bindings()
        return eval_term(t, env, self._param_map, ops, memo, default=x)

    def _eval_fast(self, t: Any, env: dict, x: Any) -> Any:
        return self._eval(t, env, x, {})

    def _bindings(self) -> HipOpTable:
        tab = HipOpTable(FUSED_BINDINGS)
        tab.register(torch_bindings=self.ops.torch_bindings)
        return tab

    def _forward_impl(self, *xs: Any) -> Any:
        x, env = self._env(xs)
        return self._tape.run(env, x, self._param_map, self.ops)

    def forward(self, *xs: Any) -> Any:
        g = getattr(self, "_graph", None)
        if g is not None and signature(xs) == self._graph_sig:
            for dst, src in zip(self._graph_inputs, xs):
                dst.copy_(src)
            g.replay()
            return self._graph_out
        return self._forward_impl(*xs)

    # -- hipGraph capture (the generic tape records like a planned executor) --

    @property
    def _plan(self) -> dict:
        return {"tape": self._tape}

    @property
    def is_graph_captured(self) -> bool:
        return getattr(self, "_graph", None) is not None

    def capture_cuda_graph(self, *example_inputs: torch.Tensor, warmup: int = 3) -> "HipIRModule":
        """Record the forward into a hipGraph; returns ``self`` (a no-op
        without a device)."""
        if not torch.cuda.is_available():
            return self
        self._graph, self._graph_inputs, self._graph_out, self._graph_sig = record_graph(
            self._forward_impl, example_inputs, warmup)
        return self

    def drop_cuda_graph(self) -> None:
        self._graph = None
        self._graph_inputs, self._graph_out, self._graph_sig = [], None, None


class _Tape:
    """Post-order slot tape of a term: one step per distinct Op node.

    Operand refs are ``(kind, payload)`` with kind ``s`` (slot), ``v``
    (Var name), ``p`` (Param name) or ``c`` (Const value).  Each slot is
    released after its last use, so peak memory follows the live set
    rather than the whole graph.
    """

    def __init__(self, root: Any) -> None:
        self.root_leaf = None if is_op(root) else root
        nodes = postorder(root) if is_op(root) else []
        index = {n: i for i, n in enumerate(nodes)}
        self.steps = []
        last_use: dict[int, int] = {}
        for i, n in enumerate(nodes):
            refs = []
            for a in n.args:
                if is_op(a):
                    refs.append(("s", index[a]))
                    last_use[index[a]] = i
                elif _is_var(a):
                    refs.append(("v", a.name))
                elif _is_param(a):
                    refs.append(("p", a.name))
                elif _is_const(a):
                    refs.append(("c", a.value))
                else:
                    raise TypeError(f"unknown term leaf {a!r}")
            self.steps.append((n.op, tuple(refs), dict(n.attrs)))
        self.release = [[] for _ in nodes]
        for s, i in last_use.items():
            if s != len(nodes) - 1:
                self.release[i].append(s)

    def run(self, env: dict, x: Any, params: dict, ops: HipOpTable) -> Any:
        if self.root_leaf is not None:
            return eval_term(self.root_leaf, env, params, ops, default=x)
        slots: list = [None] * len(self.steps)
        for i, (op, refs, attrs) in enumerate(self.steps):
            fn = ops.torch_bindings.get(op) or FUSED_BINDINGS.get(op)
            if fn is None:
                raise ValueError(f"No HIP binding for op {op!r}")
            vals = []
            for kind, p in refs:
                if kind == "s":
                    vals.append(slots[p])
                elif kind == "v":
                    vals.append(env.get(p, x))
                elif kind == "p":
                    vals.append(params[p])
                else:
                    vals.append(torch.tensor(p))
            slots[i] = fn(*vals, **attrs)
            for s in self.release[i]:
                slots[s] = None
        return slots[-1]


def const_scale(t: Any) -> float | None:
    """The number of a ``Const`` (or ``None``)."""
    return scalar_value(t)
