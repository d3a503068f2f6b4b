"""The C ABI library loads and exports what ``include/catopt_hip.h`` declares (CPU only).

No compute call is made here: only the version/strerror/workspace queries
and argument checks that every entry point performs on the host before it
touches the HIP runtime.
"""

from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from catopt_amd import _lib as L

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared() -> set[str]:
    names: set[str] = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(catopt_hip_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    if not L.LIB_PATH.exists():  # built by __graft_entry__.build(); build here only if absent
        from catopt_amd import build

        build.build()
    return L.load()


def test_header_and_binding_agree():
    declared = _declared()
    assert declared, "no catopt_hip_* declarations found"
    assert declared == set(L.SIGNATURES), declared ^ set(L.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    exported = set(re.findall(r"\b(catopt_hip_\w+)$", out.stdout, flags=re.M))
    missing = _declared() - exported
    assert not missing, missing
    for name in _declared():
        assert getattr(lib, name) is not None


def test_version_and_status_text(lib):
    assert lib.catopt_hip_abi_version() == L.ABI_VERSION
    assert lib.catopt_hip_strerror(L.OK) == b"ok"
    assert lib.catopt_hip_strerror(L.E_WORKSPACE) == b"workspace too small"
    assert lib.catopt_hip_strerror(99) == b"unknown status"
    assert lib.catopt_hip_last_hip_error() == 0


def test_workspace_queries(lib):
    # retention: two 64 KB fp32 state pieces per (b·h, segment) before the
    # output pass, segments chosen from the CU count (without a device, the
    # bound: 8 segments); head dims are multiples of 8 up to 128, chunk 64
    piece = 128 * 128 * 4
    ws = lib.catopt_hip_retention_workspace_bytes(4, 16, 8192, 128, 64)
    assert ws % (4 * 16 * 2 * piece) == 0 and 0 < ws <= 4 * 16 * 2 * 8 * piece
    assert lib.catopt_hip_retention_workspace_bytes(1, 1, 1024, 96, 64) > 0
    assert lib.catopt_hip_retention_workspace_bytes(1, 1, 64, 96, 64) == 0  # one chunk: one segment
    assert lib.catopt_hip_retention_workspace_bytes(64, 16, 64, 128, 64) == 0  # one segment: no pieces
    assert lib.catopt_hip_retention_workspace_bytes(1, 1, 64, 100, 64) == -1
    assert lib.catopt_hip_retention_workspace_bytes(1, 1, 64, 136, 64) == -1
    assert lib.catopt_hip_retention_workspace_bytes(1, 1, 64, 128, 32) == -1
    assert lib.catopt_hip_scan_workspace_bytes(10, 3) == 2 * 10 * 3 * 4
    assert lib.catopt_hip_scan_workspace_bytes(-1, 3) == -1
    # schedule-resolved queries: streaming reads no workspace; AUTO goes
    # chunk-parallel only when the lanes do not fill the GPU (131072 lanes)
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 10, 3, L.SCAN_STREAM) == 0
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 10, 3, L.SCAN_CHUNKED) == 2 * 10 * 3 * 4
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 10, 3, L.SCAN_AUTO) == 2 * 10 * 3 * 4
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 10, 1, L.SCAN_AUTO) == 0
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 1 << 20, 3, L.SCAN_AUTO) == 0
    assert lib.catopt_hip_affd_scan_workspace_bytes(100, 10, 3, 7) == -1
    # C5 (B=16, D=2048, N=16, 128 chunks) streams: no 512 MiB workspace
    assert lib.catopt_hip_ssm_scan_workspace_bytes(16, 16384, 2048, 16, 128, L.SCAN_AUTO) == 0
    assert lib.catopt_hip_ssm_scan_workspace_bytes(16, 16384, 2048, 16, 128, L.SCAN_CHUNKED) == \
        2 * 16 * 2048 * 16 * 128 * 4
    assert lib.catopt_hip_ssm_scan_workspace_bytes(1, 512, 64, 16, 23, L.SCAN_AUTO) == 2 * 64 * 16 * 23 * 4
    assert lib.catopt_hip_ssm_scan_workspace_bytes(1, 512, 64, 12, 23, L.SCAN_AUTO) == -1
    # dense scan: chunk maps (G·d², 256-byte rounded) + offsets (P·d) + carries (P·d·k), per chunk
    up = lambda n: -(-n // 64) * 64  # noqa: E731
    assert lib.catopt_hip_aff_scan_workspace_bytes(4, 16, 2, 1, 3) == 4 * (up(3 * 256) + up(3 * 64) + up(3 * 128))
    assert lib.catopt_hip_aff_scan_workspace_bytes(4, 16, 2, 0, 3) == 4 * (up(3 * 4 * 256) + up(3 * 64) + up(3 * 128))
    assert lib.catopt_hip_aff_scan_workspace_bytes(-1, 16, 1, 1, 3) == -1


def test_host_argument_checks(lib):
    # Each of these is rejected before any HIP call (bad sizes or enums).
    assert lib.catopt_hip_rmsnorm(L.BF16, -1, 8, None, 8, None, 1e-6, None, 8, None) == L.E_INVAL
    assert lib.catopt_hip_rmsnorm(L.BF16, 4, 8, None, 4, None, 1e-6, None, 8, None) == L.E_INVAL
    assert lib.catopt_hip_rmsnorm(L.BF16, 0, 8, None, 8, None, 1e-6, None, 8, None) == L.OK
    assert lib.catopt_hip_linear(L.BF16, 4, 4, 4, None, 4, None, 4, None, None, 9, None, 4, None) == L.E_INVAL
    assert lib.catopt_hip_linear(7, 4, 4, 4, None, 4, None, 4, None, None, 0, None, 4, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_linear(L.F32, 0, 4, 4, None, 4, None, 4, None, None, 0, None, 4, None) == L.OK
    # retention: a head dim off the multiples of 8 is outside the kernel; a
    # ragged T is inside it (rows past T load as zeros), so null operands
    # are the error there
    assert lib.catopt_hip_retention_fwd(L.BF16, 1, 1, 100, 100, 64, None, None, None, None, 1.0,
                                        None, None, 0, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_retention_fwd(L.BF16, 1, 1, 100, 128, 64, None, None, None, None, 1.0,
                                        None, None, 0, None) == L.E_INVAL
    # fp32: head dims are multiples of 4 (100 is one), up to 128; chunk 64 only
    assert lib.catopt_hip_retention_fwd(L.F32, 1, 1, 100, 100, 64, None, None, None, None, 1.0,
                                        None, None, 0, None) == L.E_INVAL
    for d, chunk in ((102, 64), (132, 64), (128, 128)):
        assert lib.catopt_hip_retention_fwd(L.F32, 1, 1, 100, d, chunk, None, None, None, None, 1.0,
                                            None, None, 0, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_retention_fwd(L.F32, 1, 1, 0, 128, 64, None, None, None, None, 1.0,
                                        None, None, 0, None) == L.OK
    zeros = (C.c_int64 * 3)(0, 0, 0)
    assert lib.catopt_hip_attn_fwd(L.BF16, 1, 1, 8, 8, 96, 96, None, zeros, None, zeros, None, zeros,
                                   1.0, L.MASK_CAUSAL, 0, None, 0, 1, None, zeros, None, None,
                                   None) in (L.E_UNSUPPORTED, L.E_INVAL)
    table = (C.c_int64 * 2)(0, 4)
    assert lib.catopt_hip_affd_scan(4, 8, None, 8, None, 8, None, table, 1, 7, None, None, None, 0,
                                    None) == L.E_INVAL
    # dense scan: bad schedule, d beyond the MFMA tiles, k < 1, negative stride
    args = (None, 0, 0, None, 16, 0, None, table, 1)
    assert lib.catopt_hip_aff_scan(4, 2, 16, 1, *args, 7, None, None, None, 0, None) == L.E_INVAL
    assert lib.catopt_hip_aff_scan(4, 2, 65, 1, *args, 0, None, None, None, 0, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_aff_scan(4, 2, 16, 0, *args, 0, None, None, None, 0, None) == L.E_INVAL
    assert lib.catopt_hip_aff_scan(4, 2, 16, 1, None, -1, 0, None, 16, 0, None, table, 1, 0, None, None,
                                   None, 0, None) == L.E_INVAL
    # fp32 carrier: dk / dv beyond the templates, bad leading dimension
    assert lib.catopt_hip_attn_carrier_f32(1, 4, 4, 129, 8, None, 0, 129, None, 0, 129, None, 0, 8, 1.0,
                                           None, None, None, 0, 8, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_attn_carrier_f32(1, 4, 4, 16, 300, None, 0, 16, None, 0, 16, None, 0, 300, 1.0,
                                           None, None, None, 0, 300, None) == L.E_UNSUPPORTED
    assert lib.catopt_hip_attn_carrier_f32(1, 4, 4, 16, 8, None, 0, 8, None, 0, 16, None, 0, 8, 1.0,
                                           None, None, None, 0, 8, None) == L.E_INVAL
    # masked fp32 carrier: unknown mode, a plane mode without a plane, a row
    # stride below Tk, a misaligned bias (all rejected before any launch;
    # the operand addresses are never read)
    fake = 4096

    def masked(mode, mask, ld, dk=16):
        return lib.catopt_hip_attn_carrier_f32_masked(1, 4, 4, dk, 8, fake, 0, dk, fake, 0, dk, fake, 0, 8, 1.0,
                                                      mode, 0, mask, ld, fake, fake, fake, 0, 8, None)

    assert masked(7, None, 0) == L.E_INVAL
    assert masked(-1, None, 0) == L.E_INVAL
    assert masked(L.MASK_BOOL, None, 4) == L.E_INVAL
    assert masked(L.MASK_BIAS, fake, 3) == L.E_INVAL
    assert masked(L.MASK_BIAS, fake + 2, 4) == L.E_INVAL
    assert masked(L.MASK_CAUSAL, None, 0, dk=129) == L.E_UNSUPPORTED
