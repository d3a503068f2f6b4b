"""CPU oracle for the catopt delivered-form path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (``ref``), the arithmetic of the reference's
delivered modules (luisfuturist/catopt: the torch bindings and carrier executors the
lowering path runs).  Each function cites the reference file:line it
follows.  It is the *checker*: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it.  The product path
(``catopt_amd``) never imports, calls or links anything here.

Pinning (see tests/test_oracle.py): every function below is checked against
an independent closed form, a torch library routine (``F.rms_norm``,
``F.scaled_dot_product_attention``), brute force on tiny inputs, or an
algebraic identity chosen so that a dropped term, a wrong sign or index, or
a transposed operand fails.  No function is "parity unpinned".

``torch_cpu`` holds the same forms as eager torch ops on the host CPU, the
reference's own execution style, for the CPU baseline ``bench.py`` times; each
is pinned against the numpy functions here.
"""

from . import torch_cpu  # noqa: F401  (the delivered forms as eager torch ops on the host CPU)
from .ref import *  # noqa: F401,F403
