import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")
    config.addinivalue_line("markers", "slow: long CPU test")


@pytest.fixture(scope="session")
def oracle_lib():
    """The oracle's digest library (oracle/Makefile), built if missing."""
    import ctypes
    so = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "liboracle.so"], check=True, capture_output=True)
    lib = ctypes.CDLL(so)
    lib.pd_digest.restype = ctypes.c_uint64
    lib.pd_digest.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64]
    lib.pd_eval.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32), ctypes.c_size_t]
    lib.pd_eval.restype = ctypes.c_int
    lib.pd_eval_f64.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.pd_eval_f64.restype = ctypes.c_int
    return lib


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "digests.json")) as f:
        return json.load(f)
