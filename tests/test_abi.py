"""CPU-side checks of the C ABI boundary: the library loads, exports every
entry point include/tensorium_hip.h declares, the Python mirror binds exactly
those, and calls made before tnh_init fail with a status and a message
instead of touching a device."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tensorium_hip.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(tnh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "tnh_sgemm" in names and "tnh_conv2d_fwd" in names and len(names) >= 30


def test_library_exports_every_declared_symbol():
    from tensorium_amd import nnhip

    L = C.CDLL(nnhip.LIB_PATH)
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_python_mirror_binds_exactly_the_header():
    from tensorium_amd import nnhip

    assert sorted(nnhip.exported_symbols()) == declared()


def test_calls_before_init_report_not_initialized():
    from tensorium_amd import nnhip

    L = nnhip.lib()
    st = L.tnh_sgemm(0, 0, 4, 4, 4, 1.0, None, 0, 4, None, 0, 4, 0.0, None, 0, 4)
    assert st == 1  # TNH_ERR_NOT_INITIALIZED
    assert b"tnh_init" in L.tnh_last_error()
    with pytest.raises(nnhip.TNHError):
        nnhip.call("tnh_fill", 4, None, 0, 1.0, 1)


def test_device_count_without_gpu_is_an_error_not_a_crash():
    from tensorium_amd import nnhip

    n = C.c_int32(-1)
    st = nnhip.lib().tnh_device_count(C.byref(n))
    assert st in (0, 3) and n.value >= 0


def test_oracle_is_not_linked_into_the_product():
    """The product library must not depend on the CPU oracle."""
    from tensorium_amd import nnhip

    data = open(nnhip.LIB_PATH, "rb").read()
    assert b"librefcpu" not in data and b"ref_sgemm" not in data


def test_runners_and_mirror_import_without_torch():
    """The Python mirror, the darknet network runner and the config-3 trainer
    run on the library's own memory: importing them loads no torch (the tests
    and bench.py use torch only as plumbing around them)."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); "
            "import tensorium_amd.nnhip, tensorium_amd.darknet, tensorium_amd.trainnet, tensorium_amd.weights; "
            "print('torch' in sys.modules)" % root)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-500:]
    assert r.stdout.strip() == "False"
