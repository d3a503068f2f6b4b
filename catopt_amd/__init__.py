"""catopt_amd — MI355X (gfx950) executor for the forms catopt's search delivers.

Host side in Python on PyTorch-ROCm; device side hand-written HIP kernels in
``csrc/`` reached through the C ABI of ``include/catopt_hip.h``
(``libcatopt_hip.so``, loaded by :mod:`catopt_amd._lib`).
"""

__version__ = "0.1.0"
