"""The C ABI of include/dolittle_hip.h: libdlhip.so loads on a machine
without a GPU and exports every declared function, and the Python mirror
binds each of them (no compute call is made)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "dolittle_amd", "libdlhip.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        from dolittle_amd import build
        build.build()
    from dolittle_amd import _lib
    return _lib


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_every_declared_function_is_exported(lib):
    declared = set(lib.header_functions())
    assert len(declared) > 60
    missing = declared - exported(LIB)
    assert not missing, sorted(missing)


def test_every_declared_function_has_a_binding(lib):
    declared = set(lib.header_functions()) - {"dl_last_error"}  # bound with a char* result
    assert declared <= set(lib.SIGNATURES), sorted(declared - set(lib.SIGNATURES))
    lib.load()
    assert lib.missing_exports() == []


def test_library_loads_without_a_device(lib):
    handle = lib.load()
    assert handle.dl_last_error is not None
    from dolittle_amd import DeviceError, InvalidArgument
    import ctypes as C
    # Argument validation runs before any device call.
    with pytest.raises((InvalidArgument, DeviceError)):
        lib.call("dl_sampler_required_bytes", 0, C.byref(C.c_uint64(0)))
