"""The C-ABI library without a GPU: it loads, exports every function include/bh_hex.h declares,
and rejects bad arguments on the host (status codes and messages) before touching the device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from blackhole_runtime import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "bh_hex.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(bh_hex_\w+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.bh_hex_abi_version() == _lib.ABI_VERSION
    # the thread's last error message (empty in a fresh process; a test that provoked a refusal
    # earlier in the same process leaves its message)
    assert isinstance(lib.bh_hex_last_error(), bytes)


def test_struct_layouts_match_header():
    # bh_hex_proj: 4 pointers, 4 int64 strides, int32 block (+ padding); bh_hex_tile: 3 int32
    assert ctypes.sizeof(_lib.HexProj) == 72 and _lib.HexProj.block.offset == 64
    assert ctypes.sizeof(_lib.HexTile) == 12


def test_align_max_blocks_formula():
    lib = _lib.load()
    for S, n, bm in ((0, 8, 16), (8, 4, 4), (128, 96, 16), (32768, 96, 64), (5, 100, 16)):
        assert lib.bh_hex_align_max_blocks(S, n, bm) == -(-S // bm) + min(n, S)
    assert lib.bh_hex_align_max_blocks(4, 4, 0) == -1


def test_align_workspace_sizes_and_errors():
    """bh_hex_align_ws: ceil(S / 1024) counts per expert above 4096 slots, none up to 4096; a
    null or short workspace is refused before anything is launched."""
    lib = _lib.load()
    assert lib.bh_hex_align_workspace(4096, 96) == 0
    assert lib.bh_hex_align_workspace(4097, 96) == 5 * 96
    assert lib.bh_hex_align_workspace(32768, 96) == 32 * 96
    assert lib.bh_hex_align_workspace(-1, 96) == -1 and lib.bh_hex_align_workspace(8, 0) == -1
    fake = ctypes.c_void_p(16)          # never dereferenced: the checks return first
    _status(lib.bh_hex_align_ws(fake, _lib.I64, 8192, 96, None, 128, None, 0, fake, fake, fake, None),
            _lib.ERR_VALUE, "null workspace")
    _status(lib.bh_hex_align_ws(fake, _lib.I64, 8192, 96, None, 128, fake, 8 * 96 - 1, fake, fake, fake, None),
            _lib.ERR_VALUE, "workspace too small")
    _status(lib.bh_hex_align_ws(fake, _lib.I64, 8192, 96, None, 0, fake, 8 * 96, fake, fake, fake, None),
            _lib.ERR_VALUE, "block_m")


def _workspace(lib, *args):
    nc, npart = ctypes.c_int64(), ctypes.c_int64()
    rc = lib.bh_hex_moe_workspace(*args, ctypes.byref(nc), ctypes.byref(npart))
    return rc, nc.value, npart.value


def test_workspace_sizes():
    lib = _lib.load()
    assert _workspace(lib, -1, 64, 64, 16, 1)[0] == _lib.ERR_VALUE
    assert _workspace(lib, 4, 64, 64, 24, 1)[0] == _lib.ERR_UNSUPPORTED
    rc, nc, npart = _workspace(lib, 104, 768, 2048, 16, 1)
    assert rc == _lib.OK and nc == 104 * 3 * 16 and npart > 0
    rc, nc2, npart2 = _workspace(lib, 104, 768, 2048, 64, 1)
    assert nc2 == nc and npart2 > npart          # partial tiles grow with block_m
    assert _workspace(lib, 104, 768, 2048, 128, 1) == (_lib.OK, 0, 0)   # the prefill kernels need none


def _status(rc, code, pattern):
    lib = _lib.load()
    assert rc == code
    assert re.search(pattern, lib.bh_hex_last_error().decode())


def test_host_side_errors():
    lib = _lib.load()
    _status(lib.bh_hex_align(None, _lib.I64, 8, 4, 0, None, None, None, None), _lib.ERR_VALUE, "block_m")
    _status(lib.bh_hex_align(None, _lib.F32, 8, 4, 16, None, None, None, None), _lib.ERR_UNSUPPORTED, "ids dtype")
    _status(lib.bh_hex_align(None, _lib.I64, 8, 5000, 16, None, None, None, None), _lib.ERR_UNSUPPORTED, "experts")
    _status(lib.bh_hex_direct(None, _lib.I32, -1, 16, None, None, None, None), _lib.ERR_VALUE, "slot count")
    _status(lib.bh_hex_route_topk(None, _lib.F32, 8, 2, 8, 9, 1, None, None, _lib.I64, None), _lib.ERR_VALUE, "k must")
    _status(lib.bh_hex_route_topk(None, _lib.F32, 8, 2, 2000, 8, 1, None, None, _lib.I64, None),
            _lib.ERR_UNSUPPORTED, "experts")
    w = _lib.HexProj(16, 16, 16, 16, 0, 0, 0, 0, 32)
    _status(lib.bh_hex_dequant(ctypes.byref(w), 5, 1, 1, 64, None, 16, _lib.F32, 0, 0, 0, 0, None),
            _lib.ERR_UNSUPPORTED, "bits")
    _status(lib.bh_hex_dequant(ctypes.byref(w), 4, 1, 1, 48, None, 16, _lib.F32, 0, 64, 0, 0, None),
            _lib.ERR_ASSERT, "multiple of 32")
    bad = _lib.HexProj(16, 16, 16, 16, 0, 0, 0, 0, 48)
    _status(lib.bh_hex_dequant(ctypes.byref(bad), 4, 1, 1, 96, None, 16, _lib.F32, 0, 96, 0, 0, None),
            _lib.ERR_VALUE, "scale block")
    for bad in (_lib.HexTile(16, 32, 1), _lib.HexTile(32, 256, 2)):
        _status(lib.bh_hex_moe_glu(16, _lib.BF16, 64, 16, 64, ctypes.byref(w), ctypes.byref(w), 4, 64, 64,
                                   16, 16, 1, 16, 16, 4, 4, 1, ctypes.byref(bad), None, 0, None, 0, None),
                _lib.ERR_UNSUPPORTED, "block_n must be 256")
    tile = _lib.HexTile(16, 256, 1)
    _status(lib.bh_hex_moe_glu(16, _lib.F32, 64, 16, 64, ctypes.byref(w), ctypes.byref(w), 4, 64, 64,
                               16, 16, 1, 16, 16, 4, 4, 1, ctypes.byref(tile), None, 0, None, 0, None),
            _lib.ERR_UNSUPPORTED, "BF16 or F16")
    # a plan with blocks needs the workspace (checked before anything reaches the device)
    w32 = _lib.HexProj(16, 16, 16, 16, 0, 4, 0, 1, 32)
    _status(lib.bh_hex_moe_glu(16, _lib.BF16, 64, 16, 64, ctypes.byref(w32), ctypes.byref(w32), 4, 64, 64,
                               16, 16, 1, 16, 16, 4, 4, 1, ctypes.byref(tile), None, 0, None, 0, None),
            _lib.ERR_VALUE, "workspace")
    # the 128-slot kernels step through the inputs 128 at a time
    _status(lib.bh_hex_moe_glu(16, _lib.BF16, 64, 16, 64, ctypes.byref(w32), ctypes.byref(w32), 4, 64, 64,
                               16, 16, 1, 16, 16, 4, 4, 1, ctypes.byref(_lib.HexTile(128, 256, 1)), None, 0, None, 0,
                               None),
            _lib.ERR_UNSUPPORTED, r"n_in % 128")
    _status(lib.bh_hex_moe_reduce(16, _lib.F32, 6, 16, _lib.I64, 4, 2, 2, 6, 16, _lib.BF16, 6, None),
            _lib.ERR_UNSUPPORTED, "H % 4")
    _status(lib.bh_hex_moe_reduce(16, _lib.I32, 8, 16, _lib.I64, 4, 2, 2, 8, 16, _lib.BF16, 8, None),
            _lib.ERR_UNSUPPORTED, "y dtype")
    # y is float32 or the activation dtype
    _status(lib.bh_hex_moe_down(16, _lib.BF16, 64, 16, _lib.F16, 64, ctypes.byref(w32), 4, 64, 64, 16, 16, 1, 16, 16,
                                4, 4, 16, ctypes.byref(tile), None, 0, None, 0, None),
            _lib.ERR_UNSUPPORTED, "y dtype")


def test_check_maps_status_to_reference_exceptions():
    lib = _lib.load()
    lib.bh_hex_align(None, _lib.I64, 8, 4, 0, None, None, None, None)
    with pytest.raises(ValueError, match="block_m"):
        _lib.check(_lib.ERR_VALUE, "x")
    with pytest.raises(AssertionError):
        _lib.check(_lib.ERR_ASSERT, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_HIP, "x")
