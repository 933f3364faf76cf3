"""CPU-side checks of the C-ABI library: it loads, exports exactly what
include/xnq.h declares, and its host-only validation behaves like xn's
(no kernel is launched here; there is no GPU in this container)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "xnq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xnq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from xn_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libxnq.so is not built: run __graft_entry__.build()")
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    from xn_amd import _lib

    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_sizes_match_ggml(lib):
    from xn_amd import GgmlDType

    for dt in GgmlDType:
        if lib.xnq_type_size(int(dt)):
            assert lib.xnq_type_size(int(dt)) == dt.type_size()
            assert lib.xnq_block_size(int(dt)) == dt.block_size()
    assert lib.xnq_abi_version() == 5


def test_host_validation(lib):
    from xn_amd._lib import XnqError, check

    out = ctypes.c_void_p()
    # unknown dtype id (mod.rs:114)
    st = lib.xnq_qtensor_upload(0, 99, None, 1, 256, None, ctypes.byref(out))
    assert st == 1 and b"unknown dtype" in lib.xnq_last_error()
    # dtype without a device implementation (lib.rs:284-287)
    st = lib.xnq_qtensor_upload(0, 30, None, 1, 256, None, ctypes.byref(out))
    assert st == 2 and b"not supported" in lib.xnq_last_error()
    # last dim not divisible by the block size (mod.rs:262-274)
    st = lib.xnq_qtensor_upload(0, 12, None, 1, 100, None, ctypes.byref(out))
    assert st == 1 and b"divisible" in lib.xnq_last_error()
    with pytest.raises(XnqError):
        check(lib.xnq_set_route(7))
    assert lib.xnq_lhs_workspace_size(12, 4, 4096) >= 4 * 4096 + 4 * 16 * 4 + 4 * 256 * 2


def test_product_does_not_import_oracle():
    """The shipped package never reaches into the test oracle."""
    for dirpath, _, files in os.walk(os.path.join(ROOT, "xn_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), os.path.join(dirpath, f)


def test_capture_needs_a_stream(lib):
    # the null stream cannot be captured (cuda_backend/mod.rs:264 captures the device stream)
    assert lib.xnq_capture_begin(None) == 1
    assert b"null stream" in lib.xnq_last_error()
    assert lib.xnq_graph_launch(None, None) == 1
