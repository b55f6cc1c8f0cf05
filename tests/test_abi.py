"""The C-ABI library loads and exports every symbol its header declares (CPU).

No kernel is launched here: only host functions (workspace sizing, error
strings, argument validation that returns before any HIP call).
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from ace_kernels import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "ace_hip.h"


def _declared() -> list:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ace_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_exports() -> None:
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.ace_abi_version() == _lib.ABI_VERSION


def test_error_strings() -> None:
    lib = _lib.lib()
    assert lib.ace_error_string(0) == b"success"
    assert b"invalid" in lib.ace_error_string(1)
    assert b"workspace" in lib.ace_error_string(3)


def test_workspace_sizes() -> None:
    lib = _lib.lib()
    small = lib.ace_workspace_bytes(1, 4, 512, 20, _lib.HARD, _lib.F32, 1, 0)
    big = lib.ace_workspace_bytes(2, 4, 128 ** 3, 20, _lib.HARD, _lib.F32, 1, 0)
    assert 0 < small < big
    # counters on their own 256-byte lines plus <= 16 replicas of the final
    # sums: small, and not voxel-sized
    assert big < 1 << 20
    reset = lib.ace_workspace_reset_bytes(2, 4, 128 ** 3, 20, _lib.HARD, _lib.F32, 1, 0)
    assert 0 < reset <= big and reset % 256 == 0
    assert lib.ace_workspace_bytes(0, 4, 512, 20, 0, 0, 1, 0) == 0


def test_invalid_arguments_rejected_before_launch() -> None:
    lib = _lib.lib()
    args = [None, _lib.F32, None, _lib.TARGET_LABELS_I64, 2, 4, 64, 20, _lib.HARD, _lib.ACT_SOFTMAX,
            1, 1, _lib.RED_MEAN, 0, 0.01, None, None, None, None, 0, None, None, None, None, None, None, None]
    assert lib.ace_forward(*args) == 1  # null x
    bwd = [None, _lib.F32, None, 0, 2, 4, 64, 20, _lib.HARD, 1, 1, 0, None, None, None, None, None, None, 0, None, None]
    assert lib.ace_backward(*bwd) == 1


def test_missing_library_fails_loudly(monkeypatch: pytest.MonkeyPatch, tmp_path: Path) -> None:
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    _lib.lib.cache_clear()
    try:
        with pytest.raises(_lib.AceLibraryError, match="not built"):
            _lib.lib()
    finally:
        monkeypatch.undo()
        _lib.lib.cache_clear()


def test_level_entry_points_validate_before_launch() -> None:
    """ace_forward_levels / ace_backward_levels reject bad level counts, null
    per-level pointers and configurations without a fast kernel before any
    HIP call (none of these reach the GPU)."""
    import ctypes

    lib = _lib.lib()
    vox = (ctypes.c_int64 * 2)(4096, 512)
    one = lib.ace_workspace_bytes_levels(1, vox, 2, 4, 20, _lib.HARD, _lib.F32, 1)
    two = lib.ace_workspace_bytes_levels(2, vox, 2, 4, 20, _lib.HARD, _lib.F32, 1)
    assert 0 < one < two and one % 256 == 0 and two % 256 == 0
    assert lib.ace_workspace_bytes_levels(0, vox, 2, 4, 20, _lib.HARD, _lib.F32, 1) == 0
    assert lib.ace_workspace_bytes_levels(5, vox, 2, 4, 20, _lib.HARD, _lib.F32, 1) == 0
    fwd = (_lib.AceFwdLevel * 2)()
    common = [_lib.F32, 2, 4, 20, _lib.HARD, 1, 1, _lib.RED_MEAN, 0, 0.01, None, None, None]
    assert lib.ace_forward_levels(0, fwd, *common, None, 0, None) == 1      # no levels
    assert lib.ace_forward_levels(5, fwd, *common, None, 0, None) == 1      # above the maximum
    assert lib.ace_forward_levels(2, fwd, *common, None, 0, None) == 1      # null workspace
    c5 = [_lib.F32, 2, 5, 20, _lib.HARD, 1, 1, _lib.RED_MEAN, 0, 0.01, None, None, None]
    assert lib.ace_forward_levels(2, fwd, *c5, 1, 1 << 20, None) == 2      # C = 5: no fast kernel
    bwd = (_lib.AceBwdLevel * 2)()
    assert lib.ace_backward_levels(0, bwd, _lib.F32, 2, 4, 20, _lib.HARD, 1, 0, 0, None, None,
                                   None) == 1
    assert lib.ace_backward_levels(2, bwd, _lib.F32, 2, 16, 20, _lib.HARD, 1, 0, 0, None, None,
                                   None) == 1                              # null bin table


def _noalloc_args(x, target, batch, voxels, binning, num_bins, table, centre, outputs):
    return [x, _lib.F32, target, _lib.TARGET_LABELS_I64, batch, 4, voxels, num_bins, binning,
            _lib.ACT_SOFTMAX, 1, 1, _lib.RED_MEAN, 0, 0.01, None, table, centre, *outputs, None, None]


def test_noalloc_validates_and_rejects_oversize_before_launch() -> None:
    """ace_forward_noalloc returns before any HIP call on invalid arguments
    and on problems whose workspace exceeds its scratch (the pointers below
    are never dereferenced on the host, and nothing is launched)."""
    lib = _lib.lib()
    assert b"scratch" in lib.ace_error_string(_lib.ESCRATCH)
    fake = 256  # non-null stand-ins: validation only checks for null
    outs = [fake] * 5
    assert lib.ace_forward_noalloc(*_noalloc_args(None, fake, 2, 64, _lib.HARD, 20, fake, None, outs)) == 1
    assert lib.ace_forward_noalloc(*_noalloc_args(fake, fake, 2, 64, _lib.SOFT, 20, fake, None, outs)) == 1
    # 200 batch indices of 50-bin soft moments: > 1 MiB of final sums
    big = lib.ace_workspace_bytes(200, 4, 64, 50, _lib.SOFT, _lib.F32, 1, 0)
    assert big > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.ace_forward_noalloc(*_noalloc_args(fake, fake, 200, 64, _lib.SOFT, 50, fake, fake, outs))
    assert rc == _lib.ESCRATCH
    # the benchmark configurations fit
    for args in [(2, 4, 128 ** 3, 20, _lib.HARD), (2, 4, 128 ** 3, 20, _lib.SOFT),
                 (1, 16, 128 ** 3, 20, _lib.HARD), (32, 4, 512 ** 2, 50, _lib.SOFT)]:
        b, c, n, k, binning = args
        assert lib.ace_workspace_bytes(b, c, n, k, binning, _lib.F32, 1, 0) <= _lib.NOALLOC_SCRATCH_BYTES


def test_noalloc_source_calls_no_allocator() -> None:
    """The allocation-free forward's host code names no allocating routine."""
    src = (Path(__file__).resolve().parents[1] / "ace-kernels_amd" / "csrc" / "ace_abi.hip").read_text()
    start = src.index("// ---------------------------------------------- allocation-free forward")
    end = src.index("int ace_set_launch_events")
    body = src[start:end]
    for name in ("hipMalloc", "hipFree", "hipHostMalloc", "hipMallocAsync", "hipExtMalloc", "malloc(", "new "):
        assert name not in body, name
    assert "hipGetSymbolAddress" in body and "HIP_SYMBOL(scratch)" in body


def test_no_environment_knobs() -> None:
    """The library reads no environment variable: the launch geometry and
    the loss block's wait depend on the call's arguments alone.  The forward's
    give-up path is reached through ace_set_test_hooks, which checks its
    arguments and restores the defaults for negative values."""
    csrc = Path(__file__).resolve().parents[1] / "ace-kernels_amd" / "csrc"
    for src in sorted(csrc.glob("*.hip")) + sorted(csrc.glob("*.hpp")):
        assert "getenv" not in src.read_text(), src.name
    lib = _lib.lib()
    assert lib.ace_set_test_hooks((1 << 20) + 1, 0) == 1
    assert lib.ace_set_test_hooks(0, (1 << 16) + 1) == 1
    assert lib.ace_set_test_hooks(0, 2000) == 0
    assert lib.ace_set_test_hooks(-1, -1) == 0


def test_f64_forward_refuses_lds_beside_its_static_arrays() -> None:
    """ace_forward_f64 refuses, before any HIP call, a layout whose dynamic
    LDS fits the 160 KiB workgroup alone but not beside the kernel's static
    arrays (64 doubles and an int, 528 bytes).  Its dynamic LDS at hard
    binning with C' = 2 is the larger of the wave histograms and the
    epilogue's layout (tables, 4 C'K doubles, C'K flag bytes), so K near 2210
    lands in that band.  Only refused configurations are called here (fake
    pointers)."""
    lib = _lib.lib()
    fake = 256
    limit, static = 160 * 1024, 64 * 8 + 16

    def dyn_lds(k):
        ck = 2 * k
        tab = (k * 8 + 15) // 16 * 16
        nv = 3 * ck
        waves = next((w for w in (4, 2, 1) if tab + w * nv * 8 <= limit - static), 1)
        epi = tab + 4 * ck * 8 + (ck + 15) // 16 * 16
        return max(tab + waves * nv * 8, epi)

    band = [k for k in range(1500, 3000) if limit - static < dyn_lds(k) <= limit]
    assert band, "no bin count in the band"
    for k in band + [k for k in range(1500, 3000) if dyn_lds(k) > limit][:3]:
        args = [fake, fake, _lib.TARGET_LABELS_I64, 2, 2, 64, k, _lib.HARD, _lib.ACT_SOFTMAX,
                1, 1, _lib.RED_MEAN, 0, 0.01, None, fake, None, fake, 1 << 40, fake, fake, fake, fake,
                fake, None, None]
        assert lib.ace_forward_f64(*args) == 2, k  # ACE_EUNSUPPORTED


def test_f64_entry_points_validate_before_launch() -> None:
    """ace_forward_f64 / ace_backward_f64 reject bad arguments before any HIP
    call; ace_workspace_bytes sizes their workspace for x_dtype ACE_F64."""
    lib = _lib.lib()
    fake = 256
    fwd = [None, fake, _lib.TARGET_LABELS_I64, 2, 4, 64, 20, _lib.HARD, _lib.ACT_SOFTMAX,
           1, 1, _lib.RED_MEAN, 0, 0.01, None, fake, None, fake, 1 << 20, fake, fake, fake, fake,
           fake, None, None]
    assert lib.ace_forward_f64(*fwd) == 1  # null x
    fwd[0] = fake
    fwd[2] = _lib.TARGET_ONEHOT_F32  # float64 path takes labels or a float64 one-hot
    assert lib.ace_forward_f64(*fwd) == 1
    fwd[2] = _lib.TARGET_LABELS_I64
    fwd[4] = 65
    assert lib.ace_forward_f64(*fwd) == 2  # C > 64
    fwd[4] = 4
    fwd[18] = 16  # workspace too small
    assert lib.ace_forward_f64(*fwd) == 3
    bwd = [None, None, _lib.TARGET_LABELS_I64, 2, 4, 64, 20, _lib.HARD, _lib.ACT_SOFTMAX, 1, 0,
           fake, None, fake, None, fake, fake, 0, fake, None]
    assert lib.ace_backward_f64(*bwd) == 1  # null x
    ws = lib.ace_workspace_bytes(2, 4, 128 ** 3, 20, _lib.HARD, _lib.F64, 1, 0)
    assert ws > lib.ace_workspace_bytes(2, 4, 128 ** 3, 20, _lib.HARD, _lib.F32, 1, 0) > 0
    assert ws % 256 == 0


def test_autograd_module_loads_and_builds_signatures() -> None:
    """The C++ loss call (``_ace_autograd``) loads beside the library, is
    wired to its entry points, and builds a signature on the host; the
    no-GPU check of its calls is that the extension module carries them."""
    mod = _lib.autograd()
    for name in ("make_signature", "set_entry_points", "ace_loss", "Signature"):
        assert hasattr(mod, name), name
    sig = mod.make_signature(_lib.F32, _lib.TARGET_LABELS_I64, 2, 4, 64, 20, _lib.HARD, _lib.ACT_SOFTMAX,
                             1, 1, _lib.RED_MEAN, 0, 0.01, 0, 1 << 20, 0, 2 << 20, 1 << 16,
                             2 * 160 + 8 + 8, 640, 1280, 1312, True, False, [])
    assert isinstance(sig, mod.Signature)


def test_autograd_source_reaches_kernels_through_the_c_abi() -> None:
    """The C++ loss call includes the C-ABI header and launches nothing itself."""
    src = (Path(__file__).resolve().parents[1] / "ace-kernels_amd" / "csrc" / "ace_autograd.cpp").read_text()
    assert '#include "ace_hip.h"' in src
    for name in ("hipLaunchKernel", "<<<", "hipMalloc", "hipMemset"):
        assert name not in src, name


def test_probabilities_hook_checks_its_arguments() -> None:
    """ace_probabilities validates before any HIP call: bad sizes, dtype or
    activation and null pointers are ACE_EINVAL, C > 64 ACE_EUNSUPPORTED, and
    an empty problem launches nothing (ACE_OK with null pointers)."""
    lib = _lib.lib()
    fake = 256
    assert lib.ace_probabilities(fake, _lib.F32, 1, 0, 8, _lib.ACT_SOFTMAX, fake, None) == _lib.EINVAL
    assert lib.ace_probabilities(fake, _lib.F32, -1, 4, 8, _lib.ACT_SOFTMAX, fake, None) == _lib.EINVAL
    assert lib.ace_probabilities(fake, _lib.F32, 1, 4, 8, 3, fake, None) == _lib.EINVAL
    assert lib.ace_probabilities(fake, _lib.F32, 1, 65, 8, _lib.ACT_SOFTMAX, fake, None) == _lib.EUNSUPPORTED
    assert lib.ace_probabilities(None, _lib.F32, 1, 4, 8, _lib.ACT_SOFTMAX, fake, None) == _lib.EINVAL
    assert lib.ace_probabilities(fake, _lib.F32, 1, 4, 8, _lib.ACT_SOFTMAX, None, None) == _lib.EINVAL
    assert lib.ace_probabilities(fake, _lib.F64, 1, 4, 8, _lib.ACT_SOFTMAX, fake, None) == _lib.EINVAL
    assert lib.ace_probabilities(None, _lib.F32, 0, 4, 8, _lib.ACT_SOFTMAX, None, None) == 0
