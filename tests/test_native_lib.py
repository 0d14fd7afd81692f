"""The C-ABI library loads and exports every entry point include/*.h declares (no GPU needed)."""
import ctypes
import glob
import os
import re

from tests.conftest import ROOT


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for mt in re.finditer(r"\b(?:int|const char \*|void)\s*\*?\s*(mps_[a-z0-9_]+)\s*\(", text):
            names.add(mt.group(1))
    return names


def test_header_declares_entry_points():
    names = _declared()
    for required in ("mps_fp8_decode", "mps_fp8_plan_create", "mps_fp8_plan_decode", "mps_last_error",
                     "mps_clock_rate_khz", "mps_fp8_encode", "mps_awq_decode", "mps_awq_encode"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from mpserve_amd import _native

    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_product_library_has_no_item_trace():
    """The item and record traces exist only in instrumented builds
    (--define MPS_TRACE_ITEMS=1); the product library carries none of them."""
    from mpserve_amd import _native

    lib = ctypes.CDLL(_native.LIB_PATH)
    for name in ("mps_item_trace_clear", "mps_item_trace_read", "mps_awq_trace_clear", "mps_awq_trace_read"):
        assert not hasattr(lib, name), name


def test_last_error_is_empty_string_initially():
    from mpserve_amd import _native

    assert isinstance(_native.lib().mps_last_error(), bytes)
