"""ctypes binding of the C ABI in ``include/mfft.h`` (libmfft.so, built in-tree).

This is the only place Python touches the native library.  There is no CPU
fallback: if ``libmfft.so`` is missing or cannot load, every entry point
raises ``RuntimeError`` -- the FFT runs on the GPU or not at all.

Load order matters on ROCm: import torch first, so the HIP runtime torch
ships (SONAME ``libamdhip64.so.7``) is already in the process and the
library binds to that same runtime instead of loading a second one.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmfft.so")

# enums of include/mfft.h
C2C, R2C, C2R = 0, 1, 2
FORWARD, INVERSE = 0, 1
NORM_IDS = {"none": 0, "forward": 1, "backward": 2, "ortho": 3}
TYPE_IDS = {"c2c": C2C, "r2c": R2C, "c2r": C2R}
DIR_IDS = {"forward": FORWARD, "inverse": INVERSE}
FLOW_AUTO, FLOW_RADIX2_DIT, FLOW_RADIX2_DIF, FLOW_RADIX4_DIT, FLOW_RADIX4_DIF, \
    FLOW_LDS_FUSED, FLOW_FOUR_STEP, FLOW_DENSE_MFMA = range(8)
FLOW_NAMES = {
    FLOW_AUTO: "auto", FLOW_RADIX2_DIT: "radix2-dit", FLOW_RADIX2_DIF: "radix2-dif",
    FLOW_RADIX4_DIT: "radix4-dit", FLOW_RADIX4_DIF: "radix4-dif",
    FLOW_LDS_FUSED: "lds-fused", FLOW_FOUR_STEP: "four-step", FLOW_DENSE_MFMA: "dense-mfma",
}
MAX_MFMA_CORE = 1 << 14
ERR_VALUE, ERR_TYPE, ERR_RUNTIME, ERR_UNSUPPORTED = 1, 2, 3, 4
MAX_PARAMS = 4

# Every symbol include/mfft.h declares (checked by the host tests).
EXPORTS = (
    "mfft_plan_create", "mfft_execute", "mfft_execute_timed", "mfft_plan_destroy", "mfft_plan_query",
    "mfft_bit_reverse_permute", "mfft_device_props_get", "mfft_last_error",
    "mfft_abi_version", "mfft_plan_sync_overruns", "mfft_plan_create_ex", "mfft_plan_workspace_size",
    "mfft_execute_ws", "mfft_execute_noalloc", "mfft_twiddle_transpose", "mfft_stream_copy",
    "mfft_r2c_stitch", "mfft_c2r_pre", "mfft_c2r_unpack",
)
PLAN_CALLER_WORKSPACE = 1


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int64), ("batch", ctypes.c_int64), ("core_n", ctypes.c_int64),
        ("transform_type", ctypes.c_int32), ("transform_direction", ctypes.c_int32),
        ("norm", ctypes.c_int32), ("flow", ctypes.c_int32), ("device", ctypes.c_int32),
        ("launches", ctypes.c_int32), ("elems_per_thread", ctypes.c_int32),
        ("threads_per_block", ctypes.c_int32),
        ("n1", ctypes.c_int64), ("n2", ctypes.c_int64), ("chunk_rows", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64), ("table_bytes", ctypes.c_int64),
        ("scale", ctypes.c_double),
    ]


class DeviceProps(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256), ("gcn_arch_name", ctypes.c_char * 256),
        ("multiprocessor_count", ctypes.c_int32), ("warp_size", ctypes.c_int32),
        ("shared_mem_per_block", ctypes.c_int64), ("shared_mem_per_multiprocessor", ctypes.c_int64),
        ("total_global_mem", ctypes.c_int64), ("clock_rate_khz", ctypes.c_int32),
        ("memory_clock_rate_khz", ctypes.c_int32), ("memory_bus_width", ctypes.c_int32),
        ("l2_cache_size", ctypes.c_int32), ("driver_version", ctypes.c_int32),
        ("runtime_version", ctypes.c_int32), ("abi_version", ctypes.c_int32),
    ]


_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libmfft.so (once).  Raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"native FFT library missing: {LIB_PATH} -- build it with "
                "`python kunlunxin-fft_amd/build.py` (or __graft_entry__.build()); "
                "there is no CPU fallback")
        try:
            import torch  # noqa: F401  (binds the library to torch's HIP runtime)
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.mfft_plan_create.argtypes = [ctypes.POINTER(vp), i64, i64, i32, i32, i32, i32,
                                         ctypes.POINTER(ctypes.c_int32), i32]
        lib.mfft_plan_create.restype = i32
        lib.mfft_plan_create_ex.argtypes = [ctypes.POINTER(vp), i64, i64, i32, i32, i32, i32,
                                            ctypes.POINTER(ctypes.c_int32), i32, i32]
        lib.mfft_plan_create_ex.restype = i32
        lib.mfft_execute.argtypes = [vp, vp, vp, vp]
        lib.mfft_execute.restype = i32
        lib.mfft_plan_workspace_size.argtypes = [vp, ctypes.POINTER(i64)]
        lib.mfft_plan_workspace_size.restype = i32
        lib.mfft_execute_ws.argtypes = [vp, vp, vp, vp, i64, vp]
        lib.mfft_execute_ws.restype = i32
        lib.mfft_execute_noalloc.argtypes = [vp, vp, vp, vp]
        lib.mfft_execute_noalloc.restype = i32
        lib.mfft_execute_timed.argtypes = [vp, vp, vp, vp, i64, vp, ctypes.POINTER(ctypes.c_float), i32,
                                           ctypes.POINTER(i32)]
        lib.mfft_execute_timed.restype = i32
        lib.mfft_plan_destroy.argtypes = [vp]
        lib.mfft_plan_destroy.restype = i32
        lib.mfft_plan_query.argtypes = [vp, ctypes.POINTER(PlanInfo)]
        lib.mfft_plan_query.restype = i32
        lib.mfft_plan_sync_overruns.argtypes = [vp, ctypes.POINTER(ctypes.c_int64)]
        lib.mfft_plan_sync_overruns.restype = i32
        lib.mfft_bit_reverse_permute.argtypes = [vp, vp, i64, i64, vp]
        lib.mfft_bit_reverse_permute.restype = i32
        for nm in ("mfft_r2c_stitch", "mfft_c2r_unpack"):
            getattr(lib, nm).argtypes = [vp, vp, i64, i64, ctypes.c_float, vp]
            getattr(lib, nm).restype = i32
        lib.mfft_c2r_pre.argtypes = [vp, vp, i64, i64, vp]
        lib.mfft_c2r_pre.restype = i32
        lib.mfft_twiddle_transpose.argtypes = [vp, vp, i64, i64, i64, i32, vp]
        lib.mfft_twiddle_transpose.restype = i32
        lib.mfft_stream_copy.argtypes = [vp, vp, i64, vp]
        lib.mfft_stream_copy.restype = i32
        lib.mfft_device_props_get.argtypes = [i32, ctypes.POINTER(DeviceProps)]
        lib.mfft_device_props_get.restype = i32
        lib.mfft_last_error.argtypes = []
        lib.mfft_last_error.restype = ctypes.c_char_p
        lib.mfft_abi_version.argtypes = []
        lib.mfft_abi_version.restype = i32
        _lib = lib
    return _lib


def check(rc: int) -> None:
    """Map a C return code onto the reference's exception classes."""
    if rc == 0:
        return
    msg = (load().mfft_last_error() or b"").decode(errors="replace")
    if rc in (ERR_VALUE, ERR_UNSUPPORTED):
        raise ValueError(msg)
    if rc == ERR_TYPE:
        raise TypeError(msg)
    raise RuntimeError(msg or f"libmfft error {rc}")


class NativePlan:
    """Owner of one ``mfft_plan*``; destroyed with the object."""

    __slots__ = ("_h", "info", "ws_bytes", "__weakref__")

    def __init__(self, n: int, batch: int, transform_type: str = "c2c",
                 transform_direction: str = "forward", norm: str = "backward",
                 flow: int = FLOW_AUTO, params=(), caller_workspace: bool = False):
        lib = load()
        if transform_type not in TYPE_IDS:
            raise ValueError(f"unsupported transform_type {transform_type!r}")
        if transform_direction not in DIR_IDS:
            raise ValueError(f"unsupported transform_direction {transform_direction!r}")
        if norm not in NORM_IDS:
            raise ValueError(f"unsupported norm {norm!r}")
        params = [int(p) for p in params]
        if len(params) > MAX_PARAMS:
            raise ValueError(f"at most {MAX_PARAMS} flow params, got {len(params)}")
        arr = (ctypes.c_int32 * MAX_PARAMS)(*(params + [0] * (MAX_PARAMS - len(params))))
        h = ctypes.c_void_p()
        self._h = None
        check(lib.mfft_plan_create_ex(ctypes.byref(h), int(n), int(batch), TYPE_IDS[transform_type],
                                      DIR_IDS[transform_direction], NORM_IDS[norm], int(flow),
                                      arr, len(params), PLAN_CALLER_WORKSPACE if caller_workspace else 0))
        self._h = h
        info = PlanInfo()
        check(lib.mfft_plan_query(self._h, ctypes.byref(info)))
        self.info = info
        self.ws_bytes = self.workspace_size()

    def execute(self, in_ptr: int, out_ptr: int, stream_ptr: int) -> None:
        # plain ints convert through the c_void_p argtypes
        rc = _lib.mfft_execute(self._h, in_ptr, out_ptr, stream_ptr)
        if rc:
            check(rc)

    def execute_noalloc(self, in_ptr: int, out_ptr: int, stream_ptr: int) -> None:
        """Execute with the library's static scratch (mfft_execute_noalloc):
        no allocation; calls that overlap on one device race."""
        check(_lib.mfft_execute_noalloc(self._h, in_ptr, out_ptr, stream_ptr))

    def workspace_size(self) -> int:
        """Bytes of workspace an execute of this plan needs (0: none)."""
        k = ctypes.c_int64(0)
        check(_lib.mfft_plan_workspace_size(self._h, ctypes.byref(k)))
        return int(k.value)

    def execute_ws(self, in_ptr: int, out_ptr: int, ws_ptr: int, ws_bytes: int, stream_ptr: int) -> None:
        """Execute with the caller's workspace (256-byte aligned device memory
        of at least workspace_size() bytes) instead of the plan's own."""
        check(_lib.mfft_execute_ws(self._h, in_ptr, out_ptr, ws_ptr, int(ws_bytes), stream_ptr))

    def execute_timed(self, in_ptr: int, out_ptr: int, stream_ptr: int, cap: int = 64,
                      ws_ptr: int = 0, ws_bytes: int = 0) -> list:
        """Execute once (with the caller's workspace when ws_ptr is given) and
        return each kernel launch's duration in ms (HIP events on the same
        stream; waits for the stream)."""
        ms = (ctypes.c_float * cap)()
        k = ctypes.c_int(0)
        check(_lib.mfft_execute_timed(self._h, ctypes.c_void_p(in_ptr), ctypes.c_void_p(out_ptr),
                                      ctypes.c_void_p(ws_ptr or None), int(ws_bytes),
                                      ctypes.c_void_p(stream_ptr), ms, cap, ctypes.byref(k)))
        return [float(ms[i]) for i in range(k.value)]

    def sync_overruns(self) -> int:
        """Fused four-step schedule: pass-2 waits that hit their poll limit
        over this plan's launches so far (0 unless something is wrong)."""
        k = ctypes.c_int64(0)
        check(_lib.mfft_plan_sync_overruns(self._h, ctypes.byref(k)))
        return int(k.value)

    @property
    def flow_name(self) -> str:
        return FLOW_NAMES.get(self.info.flow, str(self.info.flow))

    def close(self) -> None:
        """Destroy the native plan now.  The caller makes sure no execute of
        it is still pending (mfft_plan_destroy does not synchronise)."""
        h, self._h = self._h, None
        if h is not None and _lib is not None:
            _lib.mfft_plan_destroy(h)

    def __del__(self):
        # Never destroy from here: a collection can run while kernels that
        # read the plan's tables are still queued, or inside a graph capture.
        # The handle waits in a list that release_retired() empties at a
        # point the owner chooses (after synchronising the device).
        h, self._h = getattr(self, "_h", None), None
        if h is not None and _RETIRED is not None:  # None at interpreter shutdown
            _RETIRED.append((h, int(self.info.device) if hasattr(self, "info") else 0))


# Native plans dropped by their owners, not yet destroyed: (handle, device).
# __del__ only appends (atomic under the GIL, and it must not wait on a lock
# a collection could interrupt); release_retired takes items out under
# _RETIRED_LOCK, from the front, so two threads releasing at once never
# take (and destroy) the same handle, and handles appended meanwhile stay.
_RETIRED: list = []
_RETIRED_LOCK = threading.Lock()


def retired_count() -> int:
    return len(_RETIRED)


def release_retired(sync=None) -> int:
    """Destroy every retired plan; ``sync(device)`` is called once per
    device first, to make sure none of their executes is pending.  Returns
    how many plans were destroyed.  Safe to call from several threads."""
    if not _RETIRED or _lib is None:
        return 0
    with _RETIRED_LOCK:
        items = _RETIRED[:]
        del _RETIRED[:len(items)]
    if not items:
        return 0
    if sync is not None:
        for dev in sorted({d for _, d in items}):
            sync(dev)
    for h, _ in items:
        _lib.mfft_plan_destroy(h)
    return len(items)


def r2c_stitch(z_ptr: int, x_ptr: int, n: int, batch: int, scale: float, stream_ptr: int) -> None:
    check(load().mfft_r2c_stitch(ctypes.c_void_p(z_ptr), ctypes.c_void_p(x_ptr), int(n), int(batch),
                                 float(scale), ctypes.c_void_p(stream_ptr)))


def c2r_pre(x_ptr: int, z_ptr: int, n: int, batch: int, stream_ptr: int) -> None:
    check(load().mfft_c2r_pre(ctypes.c_void_p(x_ptr), ctypes.c_void_p(z_ptr), int(n), int(batch),
                              ctypes.c_void_p(stream_ptr)))


def c2r_unpack(u_ptr: int, out_ptr: int, n: int, batch: int, scale: float, stream_ptr: int) -> None:
    check(load().mfft_c2r_unpack(ctypes.c_void_p(u_ptr), ctypes.c_void_p(out_ptr), int(n), int(batch),
                                 float(scale), ctypes.c_void_p(stream_ptr)))


def bit_reverse_permute(in_ptr: int, out_ptr: int, n: int, batch: int, stream_ptr: int) -> None:
    check(load().mfft_bit_reverse_permute(ctypes.c_void_p(in_ptr), ctypes.c_void_p(out_ptr),
                                          int(n), int(batch), ctypes.c_void_p(stream_ptr)))


def twiddle_transpose(in_ptr: int, out_ptr: int, rows: int, cols: int, batch: int, direction: str,
                      stream_ptr: int) -> None:
    """out[c][r] = in[r][c] * W_(rows*cols)^(-+ r c) per rows x cols matrix."""
    check(load().mfft_twiddle_transpose(ctypes.c_void_p(in_ptr), ctypes.c_void_p(out_ptr), int(rows), int(cols),
                                        int(batch), DIR_IDS[direction], ctypes.c_void_p(stream_ptr)))


def stream_copy(in_ptr: int, out_ptr: int, nbytes: int, stream_ptr: int) -> None:
    """out = in over nbytes (measurement only: the streaming-copy ceiling)."""
    check(load().mfft_stream_copy(ctypes.c_void_p(in_ptr), ctypes.c_void_p(out_ptr), int(nbytes),
                                  ctypes.c_void_p(stream_ptr)))


def device_props(device: int = 0) -> dict:
    p = DeviceProps()
    check(load().mfft_device_props_get(int(device), ctypes.byref(p)))
    d = {f: getattr(p, f) for f, _ in DeviceProps._fields_}
    d["name"] = p.name.decode(errors="replace")
    d["gcn_arch_name"] = p.gcn_arch_name.decode(errors="replace")
    return d
