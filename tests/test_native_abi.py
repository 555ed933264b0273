"""The C ABI library loads and exports every symbol include/mfft.h declares
(CPU only: no compute calls).  Also checks that the ctypes structs match the
header's layout, and that invalid arguments are rejected before any device
work (these checks run on the host side of mfft_plan_create)."""
import ctypes
import os
import re

import pytest

from kunlunxin_fft_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mfft.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|void)\s+\**(mfft_\w+)\s*\(", src, re.M)))


def test_header_declares_what_the_binding_expects():
    assert _declared() == sorted(native.EXPORTS)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(native.LIB_PATH):
        pytest.fail("libmfft.so not built: run __graft_entry__.build()")
    lib = native.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.mfft_abi_version() == 2


def test_struct_layouts():
    # int64 x3, int32 x8, int64 x5, double
    assert ctypes.sizeof(native.PlanInfo) == 3 * 8 + 8 * 4 + 5 * 8 + 8
    assert ctypes.sizeof(native.DeviceProps) == 256 + 256 + 4 * 2 + 8 * 3 + 4 * 8


@pytest.mark.parametrize("kwargs,match", [
    (dict(n=12, batch=1), "power of two"),
    (dict(n=16, batch=0), "batch"),
    (dict(n=1 << 21, batch=1), "maximum"),
    (dict(n=16, batch=1, transform_type="r2c", transform_direction="inverse"), "forward"),
    (dict(n=16, batch=1, transform_type="c2r", transform_direction="forward"), "inverse"),
    (dict(n=16, batch=1, flow=native.FLOW_FOUR_STEP), "FOUR_STEP"),
    (dict(n=1 << 16, batch=1, flow=native.FLOW_LDS_FUSED), "LDS_FUSED"),
    (dict(n=1 << 17, batch=1, transform_type="r2c", flow=native.FLOW_LDS_FUSED), "LDS_FUSED"),
    (dict(n=1 << 16, batch=1, transform_type="r2c", flow=native.FLOW_LDS_FUSED, params=(16,)), "LDS_FUSED"),
    (dict(n=2, batch=1, flow=native.FLOW_RADIX4_DIT), "core length"),
    (dict(n=64, batch=1, flow=native.FLOW_RADIX2_DIT, params=(32,)), "threads per block"),
    (dict(n=64, batch=1, flow=99), "unknown flow"),
    # a launch of 2^32 work-items or more does not fit one dispatch
    (dict(n=1024, batch=1 << 23, flow=native.FLOW_RADIX2_DIT), "dispatch"),
    (dict(n=1024, batch=1 << 26, flow=native.FLOW_LDS_FUSED), "dispatch"),
    (dict(n=1 << 20, batch=1 << 17, flow=native.FLOW_FOUR_STEP, params=(1024,)), "dispatch"),
    (dict(n=1 << 14, batch=1 << 23, flow=native.FLOW_DENSE_MFMA), "dispatch"),
    # the stitch launch, not the 4-point core, is the one that would not fit:
    # one thread per mirror pair (3 a row at n = 8) past the limit, while the
    # radix-2 stages (2 threads a row) still fit
    (dict(n=8, batch=0x55555556, transform_type="r2c", flow=native.FLOW_RADIX2_DIT), "dispatch"),
])
def test_plan_create_rejects_before_device_work(kwargs, match):
    if not os.path.exists(native.LIB_PATH):
        pytest.fail("libmfft.so not built")
    with pytest.raises(ValueError, match=match):
        native.NativePlan(**kwargs)


def test_execute_rejects_null_plan():
    lib = native.load()
    assert lib.mfft_execute(None, None, None, None) == native.ERR_VALUE
    assert b"plan" in lib.mfft_last_error()
    assert lib.mfft_execute_ws(None, None, None, None, 0, None) == native.ERR_VALUE
    assert lib.mfft_plan_workspace_size(None, None) == native.ERR_VALUE
    assert lib.mfft_plan_destroy(None) == 0


def test_plan_create_ex_rejects_unknown_flags():
    lib = native.load()
    h = ctypes.c_void_p()
    arr = (ctypes.c_int32 * native.MAX_PARAMS)()
    rc = lib.mfft_plan_create_ex(ctypes.byref(h), 1024, 1, native.C2C, native.FORWARD, native.NORM_IDS["backward"],
                                 native.FLOW_AUTO, arr, 0, 2)
    assert rc == native.ERR_VALUE and b"flags" in lib.mfft_last_error() and not h.value


def test_standalone_kernels_refuse_oversized_batches():
    """mfft_bit_reverse_permute and mfft_twiddle_transpose validate their
    sizes before any device work: at most 2^40 bytes, and no launch of 2^32
    work-items or more (the pointers are never touched)."""
    lib = native.load()
    a, b = ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 40)
    assert lib.mfft_bit_reverse_permute(a, b, 1024, 1 << 28, None) == native.ERR_VALUE
    assert b"too large" in lib.mfft_last_error()
    assert lib.mfft_bit_reverse_permute(a, b, 1024, 1 << 22, None) == native.ERR_UNSUPPORTED
    assert b"2^32" in lib.mfft_last_error()
    # 16 x 16 matrices fill a quarter of a 32 x 32 tile: 256 threads per 256 values
    assert lib.mfft_twiddle_transpose(a, b, 16, 16, 1 << 24, native.FORWARD, None) == native.ERR_UNSUPPORTED
    assert b"2^32" in lib.mfft_last_error()


def test_stream_copy_validates_before_device_work():
    """mfft_stream_copy (the bench's copy ceiling) refuses NULL, sizes that
    are not a multiple of 16, misaligned or overlapping buffers, and copies
    whose launch would reach 2^32 work-items, before touching the pointers."""
    lib = native.load()
    a, b = ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 41)
    assert lib.mfft_stream_copy(None, b, 16, None) == native.ERR_VALUE
    assert lib.mfft_stream_copy(a, b, 24, None) == native.ERR_VALUE
    assert b"multiple of 16" in lib.mfft_last_error()
    assert lib.mfft_stream_copy(a, b, -16, None) == native.ERR_VALUE
    assert lib.mfft_stream_copy(ctypes.c_void_p((1 << 20) + 8), b, 16, None) == native.ERR_VALUE
    assert b"aligned" in lib.mfft_last_error()
    assert lib.mfft_stream_copy(a, ctypes.c_void_p((1 << 20) + 16), 64, None) == native.ERR_VALUE
    assert b"overlap" in lib.mfft_last_error()
    assert lib.mfft_stream_copy(a, b, (1 << 40) + 16, None) == native.ERR_VALUE
    assert lib.mfft_stream_copy(a, b, 1 << 39, None) == native.ERR_UNSUPPORTED
    assert b"2^32" in lib.mfft_last_error()
