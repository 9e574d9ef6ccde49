"""The C-ABI library loads on the CPU and exports every entry point that
include/anedvd_moe.h declares (no GPU call is made here)."""
import ctypes
import os
import re

from anedvd_amd import moe
from tests.conftest import ROOT


def declared_functions():
    text = open(os.path.join(ROOT, "include", "anedvd_moe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(anedvd_\w+)\s*\(", text)))


def test_header_and_wrapper_agree():
    assert declared_functions() == sorted(moe.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(moe.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.anedvd_moe_abi_version() == 5


def test_open_without_a_device_fails_cleanly():
    if os.path.exists("/dev/kfd"):
        return
    try:
        moe.MoeContext(0)
    except moe.MoeError as e:
        assert e.name == "NoDevice"
    else:
        raise AssertionError("opening a context without a GPU must fail")
