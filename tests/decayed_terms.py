"""The chunked decayed-retention term family, spelled for the executor tests.

catopt's lowering tests build this family by hand (tests/test_decayed_lower.py
:52-205 of luisfuturist/catopt): q/k/v projections ``linear(x, W, b)`` of one
input, a decay base γ, ``K`` arms of ``C`` rows, each arm an intra element
``om_decayed(q_i k_iᵀ, decay(γ, C), v_i) / S`` plus ``i`` decay-gated pair
products over the earlier chunks.  :class:`DecayedTerms` spells every arm
with knobs for

* the spellings that extraction can deliver for the same function: the row
  gate outside the ``div``, on its right, or inside it (``gate``); the state
  half as ``(k_j ⊙ η)ᵀ`` or ``k_jᵀ ⊙ η`` (``state``); the pair product right-
  or left-associated, or as the law's score block (``assoc``); the key block
  as ``split(transpose(k))`` or ``transpose(split(k))`` (``keys``);
* the variants that denote another function: no row gate, an ungated or
  non-key state half, a second decay base, a gated intra element, a score
  that is not one product.

Every term is an ordinary IR; the tests evaluate it as written through the
generic module (on the CPU op table or on the GPU) to pin what it denotes.
"""

from __future__ import annotations

import torch

from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var

mk = Op.make

SAME_FUNCTION = {
    "gate": ("row", "row_rev", "row_in"),
    "state": ("parsed", "parsed_rev", "colscale"),
    "assoc": ("right", "left", "law"),
    "keys": ("split_t", "t_split"),
}


class DecayedTerms:
    """A ``K``-arm chunked decayed term over ``x (B, [H,] K*C, D)``.

    ``heads``: ``None`` for a scalar decay base and a 3-D input (every batch
    row one sequence), or ``H`` for a per-head base ``γ (H,)`` and a 4-D input.
    """

    def __init__(self, B: int = 2, K: int = 3, C: int = 16, D: int = 32, heads: int | None = None,
                 scale: float = 2.0) -> None:
        self.B, self.K, self.C, self.D, self.H = B, K, C, D, heads
        self.T = K * C
        self.SZ = [C] * K
        lead = (B,) if heads is None else (B, heads)
        self.x = Var("x", TensorType((*lead, self.T, D)))
        self.w = {n: Param(f"w{n}", TensorType((D, D))) for n in "qkv"}
        self.b = {n: Param(f"b{n}", TensorType((D,))) for n in "qkv"}
        gshape = () if heads is None else (heads,)
        self.g = Param("g", TensorType(gshape))
        self.g2 = Param("g2", TensorType(gshape))
        self.S = Const(float(scale))
        self.scale = float(scale)
        self.q, self.k, self.v = (mk("linear", self.x, self.w[n], self.b[n]) for n in "qkv")

    # ------------------------------------------------------------ blocks
    def _split(self, t, i, dim=-2):
        return mk("split", t, dim=dim, index=i, sizes=self.SZ)

    def qi(self, i):
        return self._split(self.q, i)

    def ki(self, i):
        return self._split(self.k, i)

    def vi(self, i):
        return self._split(self.v, i)

    def kti(self, i, keys="split_t"):
        if keys == "split_t":
            return self._split(mk("transpose", self.k, dim0=-1, dim1=-2), i, dim=-1)
        return mk("transpose", self.ki(i), dim0=-1, dim1=-2)

    def law_block(self, i, j):
        s = mk("matmul", self.q, mk("transpose", self.k, dim0=-2, dim1=-1))
        return self._split(self._split(s, i, -2), j, -1)

    def dv(self, *, sign=1, offset=0, g=None):
        return mk("decay_vec", self.g if g is None else g, t=self.C, sign=sign, offset=offset)

    def row(self, offset, g=None):
        return mk("unsqueeze", self.dv(offset=offset, g=g), dim=-1)

    def decay(self, g=None):
        return mk("decay", self.g if g is None else g, t=self.C)

    # ------------------------------------------------------------ summands
    def state_half(self, j, state="parsed", keys="split_t"):
        """``A_j`` of the pair product ``q_i @ (A_j @ v_j)``."""
        if state == "parsed":
            return mk("transpose", mk("mul", self.ki(j), mk("unsqueeze", self.dv(sign=-1), dim=-1)),
                      dim0=-1, dim1=-2)
        if state == "parsed_rev":
            return mk("transpose", mk("mul", mk("unsqueeze", self.dv(sign=-1), dim=-1), self.ki(j)),
                      dim0=-1, dim1=-2)
        if state == "colscale":
            return mk("mul", self.kti(j, keys), mk("unsqueeze", self.dv(sign=-1), dim=-2))
        if state == "no_mul":  # ungated: another function
            return mk("transpose", self.ki(j), dim0=-1, dim1=-2)
        if state == "add":  # not a gated key transpose: another function
            return mk("transpose", mk("add", self.ki(j), self.ki(j)), dim0=-1, dim1=-2)
        raise ValueError(state)

    def pair(self, i, j, *, state="parsed", assoc="right", keys="split_t"):
        if assoc == "right":
            return mk("matmul", self.qi(i), mk("matmul", self.state_half(j, state, keys), self.vi(j)))
        if assoc == "left":
            return mk("matmul", mk("matmul", self.qi(i), self.state_half(j, state, keys)), self.vi(j))
        if assoc == "law":
            col = mk("unsqueeze", self.dv(sign=-1), dim=-2)
            return mk("matmul", mk("mul", self.law_block(i, j), col), self.vi(j))
        raise ValueError(assoc)

    def cross(self, i, j, *, gate="row", **kw):
        body = self.pair(i, j, **kw)
        row = self.row((i - j) * self.C)
        if gate == "row":
            return mk("mul", row, mk("div", body, self.S))
        if gate == "row_rev":
            return mk("mul", mk("div", body, self.S), row)
        if gate == "row_in":
            return mk("div", mk("mul", row, body), self.S)
        if gate == "none":  # no row gate: another function
            return mk("div", body, self.S)
        raise ValueError(gate)

    def intra(self, i, *, keys="split_t", score=None, decay=None, law=False):
        sc = score if score is not None else (
            self.law_block(i, i) if law else mk("matmul", self.qi(i), self.kti(i, keys)))
        return mk("div", mk("om_decayed", sc, decay if decay is not None else self.decay(), self.vi(i)), self.S)

    def arm(self, i, *, gate="row", state="parsed", assoc="right", keys="split_t", row=False,
            decay=None, score=None):
        t = self.intra(i, keys=keys, score=score, decay=decay, law=assoc == "law")
        if row:  # a gated intra element: another function
            t = mk("mul", self.row(self.C), t)
        for j in range(i):
            t = mk("add", t, self.cross(i, j, gate=gate, state=state, assoc=assoc, keys=keys))
        return t

    def root(self, **kw):
        return mk("concat", *[self.arm(i, **kw) for i in range(self.K)], dim=-2)

    def ir(self, root) -> IR:
        return IR(root, [self.x])

    # ------------------------------------------------------------ values
    def values(self, *, dtype=torch.float64, seed=0, gammas=(0.9, 0.8), gamma_dtype=None):
        """Parameter values and an input: weights of scale ``1/√D`` so the
        projections stay O(1); ``g`` and ``g2`` from ``gammas`` (per head: a
        spread of rates starting there), in ``gamma_dtype`` (default ``dtype``)."""
        gen = torch.Generator().manual_seed(seed)
        r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
        D = self.D
        vals = {}
        for n in "qkv":
            vals[f"w{n}"] = (r(D, D) / D ** 0.5).to(dtype)
            vals[f"b{n}"] = (0.1 * r(D)).to(dtype)
        for name, g0 in zip(("g", "g2"), gammas):
            gd = gamma_dtype or dtype
            if self.H is None:
                vals[name] = torch.tensor(g0, dtype=gd)
            else:
                vals[name] = torch.tensor([g0 + (1 - g0) * h / (2 * self.H) for h in range(self.H)], dtype=gd)
        lead = (self.B,) if self.H is None else (self.B, self.H)
        x = r(*lead, self.T, D).to(dtype)
        return vals, x

    def projections(self, vals, x):
        """``q, k, v`` in float64 from the same (possibly rounded) values."""
        f = lambda n: x.double() @ vals[f"w{n}"].double().T + vals[f"b{n}"].double()  # noqa: E731
        return f("q"), f("k"), f("v")
