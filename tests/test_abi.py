"""The C-ABI library loads and exports every declared entry point (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = (ROOT / "include" / "hsmoe.h").read_text()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*|void)\s+(hsmoe_\w+)\(", text, re.M)))


def test_header_and_binding_agree():
    from home_seek_amd import _lib
    assert set(_declared()) == set(_lib.exported_symbols())


def test_library_exports_every_symbol():
    handle = ctypes.CDLL(str(ROOT / "home-seek_amd" / "libhsmoe.so"))
    for name in _declared():
        assert hasattr(handle, name), name


def test_version_and_error_paths():
    from home_seek_amd import _lib
    L = _lib.lib()
    assert L.hsmoe_version() == 1
    rc = L.hsmoe_fp4_dequant_bf16(None, None, 0, 1, 32, 16, 1, None, 32, None)
    assert rc == -1 and b"null" in L.hsmoe_last_error()
    rc = L.hsmoe_moe_decode(1, 9, 512, 512, 1, 1, 6, 1, 256, 0, None, 10.0, None, 1, 1, 1 << 20, None)
    assert rc == -2 and b"m <= 8" in L.hsmoe_last_error()
    rc = L.hsmoe_lm_head_accept(4096, 4096, 3, 4096, 129280, 4096, None, 4096, 4096, None, 0, None)
    assert rc == -4
    with pytest.raises(_lib.HsmoeError):
        _lib.check(rc, "lm_head")


def test_layer_entry_point_rejects_bad_arguments():
    """Argument and shape errors of the fused layer entry point are reported
    before anything is launched (no GPU needed)."""
    from home_seek_amd import _lib
    L = _lib.lib()
    rc = L.hsmoe_moe_layer_decode(4096, 1, 4096, 2048, None, None, 256, 6, 1.5, 4096, 0, None, 10.0, 4096, 4096,
                                  None, 4096, None, 4096, 1 << 24, None)
    assert rc == -1 and b"null" in L.hsmoe_last_error()
    rc = L.hsmoe_moe_layer_decode(4096, 9, 4096, 2048, 4096, None, 256, 6, 1.5, 4096, 0, None, 10.0, 4096, 4096,
                                  None, 4096, None, 4096, 1 << 24, None)
    assert rc == -2 and b"m <= 8" in L.hsmoe_last_error()
    rc = L.hsmoe_moe_layer_decode(4096, 1, 4096, 2048, 4096, None, 256, 6, 1.5, 4096, 0, None, 10.0, 4096, 4096,
                                  None, 4096, None, 4096, 64, None)
    assert rc == -4
    assert L.hsmoe_moe_layer_workspace_size(1, 4096, 2048, 256, 6) > 0


def test_norm_tail_entry_points_check_the_tail():
    """The _norm entry points check their norm tail before anything is launched."""
    from home_seek_amd import _lib
    L = _lib.lib()
    args = (4096, 1, 4096, 2048, 4096, None, 256, 6, 1.5, 4096, 0, None, 10.0, 4096, 4096, None, None, None)
    rc = L.hsmoe_moe_layer_decode_norm(*args, None, 4096, 1 << 24, None)
    assert rc == -1 and b"norm tail" in L.hsmoe_last_error()
    overlapping = _lib.NormTail(1 << 20, None, 1 << 21, 1e-6, 1 << 22, 4096)  # norm_out on x
    rc = L.hsmoe_moe_layer_decode_norm(*args, ctypes.addressof(overlapping), 4096, 1 << 24, None)
    assert rc == -1 and b"overlap" in L.hsmoe_last_error()
    tail = _lib.NormTail(1 << 20, None, 1 << 21, 1e-6, 1 << 22, 1 << 23)
    rc = L.hsmoe_moe_layer_decode_norm(*args, ctypes.addressof(tail), 4096, 64, None)
    assert rc == -4
    rc = L.hsmoe_moe_layer_decode_routed_norm(4096, 1, 4096, 2048, 4096, None, 0, None, 1.0, 6, 4096, 256, 0, None,
                                              10.0, None, None, ctypes.addressof(overlapping), 4096, 1 << 24, None)
    assert rc == -1 and b"overlap" in L.hsmoe_last_error()
    rc = L.hsmoe_moe_layer_decode(*args, 4096, 1 << 24, None)  # without a tail an output is still required
    assert rc == -1 and b"no output" in L.hsmoe_last_error()
