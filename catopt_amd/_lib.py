"""ctypes binding of ``libcatopt_hip.so`` (the C ABI in ``include/catopt_hip.h``).

The library is loaded lazily on first use.  A missing or mismatched library
is an error, never a silent fallback: the executors in this package have no
CPU path for the delivered forms.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libcatopt_hip.so")
ABI_VERSION = 1

# enum values mirrored from include/catopt_hip.h
OK, E_INVAL, E_UNSUPPORTED, E_HIP, E_WORKSPACE = 0, 1, 2, 3, 4
F32, BF16 = 0, 1
EPI_NONE, EPI_BIAS, EPI_BIAS_ADD2, EPI_SILU_MUL, EPI_GLU = 0, 1, 2, 3, 4
MASK_NONE, MASK_CAUSAL, MASK_BOOL, MASK_BIAS = 0, 1, 2, 3
SCAN_AUTO, SCAN_STREAM, SCAN_CHUNKED = 0, 1, 2

_i32, _i64, _f32, _p = C.c_int32, C.c_int64, C.c_float, C.c_void_p
_pi64 = C.POINTER(C.c_int64)

#: name -> (restype, argtypes); the exported surface of the header.
SIGNATURES: dict[str, tuple] = {
    "catopt_hip_abi_version": (_i32, []),
    "catopt_hip_strerror": (C.c_char_p, [_i32]),
    "catopt_hip_last_hip_error": (_i32, []),
    "catopt_hip_rmsnorm": (_i32, [_i32, _i64, _i64, _p, _i64, _p, _f32, _p, _i64, _p]),
    "catopt_hip_linear": (
        _i32,
        [_i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _p, _i32, _p, _i64, _p],
    ),
    "catopt_hip_matmul": (
        _i32,
        [_i32, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _i64, _i32, _p, _i64, _i64, _p],
    ),
    "catopt_hip_attn_fwd": (
        _i32,
        [_i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _pi64, _p, _pi64, _p, _pi64,
         _f32, _i32, _i64, _p, _i64, _i32, _p, _pi64, _p, _p, _p],
    ),
    "catopt_hip_om_rows": (_i32, [_i32, _i64, _i64, _p, _i64, _i32, _p, _p, _p, _i64, _p]),
    "catopt_hip_omd_fold_apply": (_i32, [_i64, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p]),
    "catopt_hip_om_compose": (_i32, [_i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "catopt_hip_retention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "catopt_hip_retention_fwd": (
        _i32,
        [_i32, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _f32, _p, _p, _i64, _p],
    ),
    "catopt_hip_decay": (_i32, [_i64, _i64, _p, _p, _p]),
    "catopt_hip_decay_vec": (_i32, [_i64, _i64, _i64, _i64, _p, _p, _p]),
    "catopt_hip_hbm_read": (_i32, [_p, _i64, _p, _p]),
    "catopt_hip_scan_workspace_bytes": (_i64, [_i64, _i64]),
    "catopt_hip_affd_scan_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32]),
    "catopt_hip_ssm_scan_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "catopt_hip_affd_scan": (
        _i32,
        [_i64, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i32, _p, _p, _p, _i64, _p],
    ),
    "catopt_hip_affd_scan_noalloc_max_bytes": (_i64, []),
    "catopt_hip_affd_scan_noalloc": (
        _i32,
        [_i64, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i32, _p, _p, _p],
    ),
    "catopt_hip_ssm_scan": (
        _i32,
        [_i64, _i64, _i64, _i64, _p, _i32, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p, _i64, _p],
    ),
    "catopt_hip_attn_carrier_f32": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _f32, _p, _p, _p, _i64,
         _i64, _p],
    ),
    "catopt_hip_attn_carrier_f32_masked": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _f32, _i32, _i64, _p,
         _i64, _p, _p, _p, _i64, _i64, _p],
    ),
    "catopt_hip_aff_scan_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i64]),
    "catopt_hip_aff_scan": (
        _i32,
        [_i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i32, _p, _p, _p, _i64, _p],
    ),
    "catopt_hip_affd_compose_slots": (_i32, [_i64, _i64, _p, _p, _p, _p, _i64, _i64, _p]),
    "catopt_hip_aff_compose_slots": (_i32, [_i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p]),
    "catopt_hip_silu": (_i32, [_i32, _i64, _p, _p, _p]),
    "catopt_hip_silu_mul": (_i32, [_i32, _i64, _p, _p, _p, _p]),
}


class HipExtensionMissing(RuntimeError):
    """The compiled HIP library is absent or does not match this package."""


class HipKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, hip_error: int = 0) -> None:
        self.fn, self.status, self.hip_error = fn, status, hip_error
        text = _lib.catopt_hip_strerror(status).decode() if _lib is not None else str(status)
        extra = f" (hipError_t {hip_error})" if status == E_HIP else ""
        super().__init__(f"{fn} failed: {text}{extra}")


_lib: C.CDLL | None = None
_lock = threading.Lock()


def load(path: Path | str | None = None) -> C.CDLL:
    """Load (once) and type the library; raise :class:`HipExtensionMissing` if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        # torch ships its own HIP runtime under the same soname as ROCm's; it
        # must be loaded first so that this library binds to that instance
        # (one runtime per process: torch's streams and allocations are then
        # valid here).  Loading this library first pulls in /opt/rocm's copy
        # and the two runtimes disagree (hipErrorNoDevice on launch).
        import torch  # noqa: F401

        if not p.exists():
            raise HipExtensionMissing(
                f"{p} not found: build it with `python -m catopt_amd.build` "
                "(hipcc, gfx950); there is no CPU fallback for the delivered forms"
            )
        try:
            lib = C.CDLL(str(p))
        except OSError as exc:
            raise HipExtensionMissing(f"cannot load {p}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise HipExtensionMissing(f"{p} does not export {name}") from exc
            fn.restype = res
            fn.argtypes = args
        ver = lib.catopt_hip_abi_version()
        if ver != ABI_VERSION:
            raise HipExtensionMissing(f"{p} ABI version {ver} != expected {ABI_VERSION}")
        _lib = lib
        return lib


_calls = 0  # library entry points that returned OK in this process


def check(fn: str, status: int) -> None:
    """Raise :class:`HipKernelError` for a non-zero status; count the call
    otherwise (:func:`call_count`)."""
    global _calls
    if status != OK:
        hip = _lib.catopt_hip_last_hip_error() if _lib is not None else 0
        raise HipKernelError(fn, status, hip)
    _calls += 1


def call_count() -> int:
    """Number of successful launching entry-point calls so far (a host-side
    counter; graph replays launch without calling in and are not counted)."""
    return _calls


def i64_array(vals) -> C.Array:
    """A host int64 array (for the stride triples of catopt_hip_attn_fwd)."""
    arr = (C.c_int64 * len(vals))(*[int(v) for v in vals])
    return arr
