"""Tensor-level runners: the reference's runner names over the native flows.

``execute_fft_plan`` dispatches by ``plan.executed`` exactly like the
reference (entry.py:549-550: ``getattr(runner, plan.executed)``); here the
name selects a native flow of ``libmfft.so`` and the plan's parameters:

===========================================  ==============================  =========
runner name (reference file:line)            native flow                     params
===========================================  ==============================  =========
fft_dit, fft_dit_batch (runner.py:118, 781)  RADIX2_DIT (M0, bitrev fold)    block
fft_dif, fft_dif_batch (runner.py:165, 839)  RADIX2_DIF (M0, bitrev fold)    block
fft_dit_radix4(_batch) (runner.py:1399,1112) RADIX4_DIT (M5, digit-rev fold) block
fft_dif_radix4(_batch) (runner.py:1473,1193) RADIX4_DIF (M5)                 block
fft_lds_fused(_batch)                        LDS_FUSED (single pass)         elems
fft_four_step(_batch)                        FOUR_STEP (two passes)          n1, chunk_rows, schedule
fft_dit_fused (runner.py:209)                LDS_FUSED / FOUR_STEP (auto)    --
fft_{dit,dif}_matrix(_batch) (runner.py:379) DENSE_MFMA (core 2..16384)      --
fft_{dit,dif}_grouped (runner.py:505)        LDS_FUSED / FOUR_STEP (auto)    --
run_hybrid (adapter_hybrid.py:224)           FOUR_STEP (n1 = N/tile)         tile
===========================================  ==============================  =========

The M2 names (the reference's dense-dot matrix flow) run the dense-dot core
on the fp32 matrix cores, every butterfly a DFT-8 matrix product (cores of
2..16384 points; longer ones go to the library's choice).  The M1/M3 names
exist so a plan naming them still runs: on MI355X the stages they fuse (in
global memory, or as XOR-gather maps) all run inside one LDS-resident
kernel, or the four-step for core lengths above 32768.

Every transform semantic -- C2C forward/inverse with its norm, R2C and C2R
-- is one native plan: the conjugation, the norm scale and the real-FFT
pack/stitch/pre-twiddle are fused into the kernels, so a call is one
allocation of the output plus one ``mfft_execute``.  Native plans are cached
by shape/semantics/flow/device.
"""
from __future__ import annotations

import math
import random
import threading
import time
import weakref
from collections import OrderedDict

import torch

from . import native
from .context import (  # noqa: F401  (re-exported)
    current_device_index, device_context, device_name, device_ready, xpu_context,
)
from .validate import log2_exact, validate_batch_input, validate_input, validate_tensor, validate_twiddle

from .flows import DEFAULT_STAGE_BLOCK, RUNNER_FLOWS, flow_params  # noqa: F401  (re-exported)


# Native plans, cached by (flow, params, shape, semantics, device).  They are
# created with a caller-owned workspace: a plan holds only its twiddle tables
# (a few KB to a few hundred KB), and every execute that needs scratch takes
# it from torch's stream-ordered allocator on the stream it runs on, so one
# cached plan can run on several streams at once.
_NATIVE: "OrderedDict[tuple, native.NativePlan]" = OrderedDict()
_NATIVE_LOCK = threading.Lock()
NATIVE_CACHE_SIZE = 256
# Dropped native plans are destroyed in a batch once this many wait (never
# inside a graph capture, and automatically only in a single-threaded
# process), after one synchronisation of their devices.
RETIRED_FLUSH = 64


def _sync_device(dev: int) -> None:
    torch.cuda.synchronize(dev)


def release_retired_plans() -> int:
    """Destroy the native plans dropped so far (evicted from the cache, or
    whose owners went away), after synchronising their devices.  A no-op
    inside a graph capture.  Returns how many were destroyed."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return 0
    return native.release_retired(_sync_device)


def get_native_plan(executed: str, n: int, batch: int, transform_type: str,
                    transform_direction: str, norm: str, block, params: dict,
                    device_index: int) -> native.NativePlan:
    """Cached native plan for one (runner, shape, semantics, params, device)."""
    flow, prm = flow_params(executed, n, transform_type, block, params)
    key = (flow, prm, int(n), int(batch), transform_type, transform_direction, norm, int(device_index))
    with _NATIVE_LOCK:
        p = _NATIVE.get(key)
        if p is not None:
            _NATIVE.move_to_end(key)
            return p
    # Destroying retired plans synchronises their devices, which would break
    # a graph capture in progress on any thread of the process.  This call
    # can see only its own thread's capture, so it flushes only when it is
    # the process's one Python thread; a multi-threaded caller flushes at
    # points of its choosing (release_retired_plans / clear_native_cache).
    if native.retired_count() >= RETIRED_FLUSH and threading.active_count() == 1:
        release_retired_plans()
    with device_context(device_index):
        p = native.NativePlan(n, batch, transform_type, transform_direction, norm, flow, prm,
                              caller_workspace=True)
    with _NATIVE_LOCK:
        _NATIVE[key] = p
        while len(_NATIVE) > NATIVE_CACHE_SIZE:
            _NATIVE.popitem(last=False)  # retired when its last user lets go
    return p


def clear_native_cache() -> None:
    """Drop every cached native plan and destroy those no caller holds."""
    with _NATIVE_LOCK:
        _NATIVE.clear()
    release_retired_plans()


def output_spec(transform_type: str, n: int, batch: int):
    """(shape, dtype) of a plan's output; rank-1 for batch 1 (entry.py:488-493)."""
    if transform_type == "r2c":
        last, dt = n // 2 + 1, torch.complex64
    elif transform_type == "c2r":
        last, dt = n, torch.float32
    else:
        last, dt = n, torch.complex64
    return ((last,) if batch == 1 else (batch, last)), dt


# torch's raw current-stream and current-device queries (the public
# torch.cuda.current_stream builds a Stream object per call, ~1.7 us)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_raw_device = getattr(torch._C, "_cuda_getDevice", None)


def stream_handle(dev: int) -> int:
    """hipStream_t of torch's current stream on device ``dev``."""
    if _raw_stream is not None:
        return _raw_stream(dev)
    return torch.cuda.current_stream(dev).cuda_stream


def current_device() -> int:
    return _raw_device() if _raw_device is not None else torch.cuda.current_device()


def workspace_for(nplan: native.NativePlan, device) -> "torch.Tensor | None":
    """Scratch for one execute of ``nplan`` from torch's caching allocator
    (512-byte aligned, ordered on the current stream), or None."""
    if not nplan.ws_bytes:
        return None
    return torch.empty(nplan.ws_bytes, dtype=torch.uint8, device=device)


def launch(nplan: native.NativePlan, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Enqueue one execute on x's device and current stream.  A plan that
    needs scratch gets it per call on that stream: the block returns to the
    allocator when this call returns, and the allocator hands it out again
    only to work ordered after this execute on the same stream."""
    dev = x.get_device()
    stream = stream_handle(dev)
    if nplan.ws_bytes:
        ws = torch.empty(nplan.ws_bytes, dtype=torch.uint8, device=x.device)
        if current_device() == dev:
            nplan.execute_ws(x.data_ptr(), out.data_ptr(), ws.data_ptr(), nplan.ws_bytes, stream)
        else:
            with device_context(dev):
                nplan.execute_ws(x.data_ptr(), out.data_ptr(), ws.data_ptr(), nplan.ws_bytes, stream)
        return out
    if current_device() == dev:
        nplan.execute(x.data_ptr(), out.data_ptr(), stream)
    else:
        with device_context(dev):
            nplan.execute(x.data_ptr(), out.data_ptr(), stream)
    return out


def run(executed: str, x: torch.Tensor, batch: int, n: int, transform_type: str = "c2c",
        transform_direction: str = "forward", norm: str = "backward", block=None,
        params: dict | None = None) -> torch.Tensor:
    """Run one transform of ``x`` through the named runner; returns a new tensor."""
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    nplan = get_native_plan(executed, n, batch, transform_type, transform_direction, norm,
                            block, params or {}, dev)
    shape, dt = output_spec(transform_type, n, batch)
    out = torch.empty(shape, dtype=dt, device=x.device)
    return launch(nplan, x, out)


# ---------------- reference runner entry points (forward C2C) ----------------

# Largest deviation of a caller's table from exp(-2*pi*i*idx/N) that still
# counts as those roots: the reference builds them from a float32 angle
# (runner.py:93-97), which is off by up to ~2e-7 at N = 2^20.
TWIDDLE_TOL = 1e-6
# tables already checked: (ptrs, versions, n, device) -> weak references to
# the two tensors, so that a later table at a reused address is not taken
# for the one that was checked
_TWIDDLE_OK: dict = {}


def check_twiddle(twiddle, x) -> None:
    """The reference's twiddle= contract for the stage runners: validate the
    table (validate.py:71-84), then require that it holds the forward roots
    exp(-2*pi*i*idx/N), idx < N/2.  Every native plan computes with its own
    table of those roots (built once per plan); any other table would ask
    for a different transform, which the library does not run, so it raises
    ValueError instead of silently using its own.  The value check costs one
    device round trip per distinct table and is then remembered for the same
    two tensor objects at the same version (an in-place write bumps it)."""
    if twiddle is None:
        return
    n = x.numel() if x.dim() == 1 else int(x.shape[-1])
    validate_twiddle(twiddle, n, x.device)
    wr, wi = twiddle
    key = (wr.data_ptr(), wi.data_ptr(), wr._version, wi._version, n, str(x.device))
    seen = _TWIDDLE_OK.get(key)
    if seen is not None and seen[0]() is wr and seen[1]() is wi:
        return
    idx = torch.arange(n >> 1, dtype=torch.float64, device=x.device)
    ang = -2.0 * math.pi * idx / n
    dev = max(float((wr.double() - torch.cos(ang)).abs().max().item()) if n > 1 else 0.0,
              float((wi.double() - torch.sin(ang)).abs().max().item()) if n > 1 else 0.0)
    if not dev <= TWIDDLE_TOL:
        raise ValueError(f"twiddle table differs from exp(-2*pi*i*idx/{n}) by up to {dev:.3e} "
                         f"(> {TWIDDLE_TOL:g}): only the forward roots are supported (every plan "
                         "builds and keeps its own table of them)")
    if len(_TWIDDLE_OK) > 64:
        _TWIDDLE_OK.clear()
    _TWIDDLE_OK[key] = (weakref.ref(wr), weakref.ref(wi))


def _single(name, x, block, params=None, twiddle=None):
    validate_input(x, "x", block=block)
    check_twiddle(twiddle, x)
    return run(name, x, 1, x.numel(), block=block, params=params, norm="backward")


def _batched(name, x, block, params=None, twiddle=None, variant=None, spread_only=False):
    """A runner over a (B, N) batch: the reference's batch contract
    (runner.py:757-778: rank-2 contiguous complex64 on the GPU, N and B
    powers of two, variant 'spread' or 'folded'), then the native flow.
    ``spread_only``: the reference lowers only 'spread' for this runner
    (radix-4 and matrix batches) and refuses 'folded' with ValueError."""
    if variant is not None:
        _check_variant(variant)
    if spread_only and variant != "spread":
        raise ValueError(f"{name} lowers variant='spread' only (as the reference); got variant={variant!r}")
    validate_batch_input(x, "x", block=block)
    b, n = int(x.shape[0]), int(x.shape[1])
    log2_exact(b)
    check_twiddle(twiddle, x)
    y = run(name, x, b, n, block=block, params=params, norm="backward")
    return y.reshape(b, n)


# Every runner keeps the reference's signature (src/xpu/runner.py:118-1472):
# the same positional order, keywords and defaults, block=1024 included.
# ``block`` sizes the global-stage flows' workgroups; the single-pass,
# four-step and matrix-core flows size their own launches and only check
# that it is a power of two.  ``tile``/``rows``/``glog``/``maxp``/``cells``/
# ``packets`` shape the reference's Triton programs and have no counterpart
# in the HIP kernels; they are accepted and ignored.  ``variant`` is
# 'spread' or 'folded' (the batch always folds into one 1-D grid here; both
# compute the same values), except for the radix-4 and matrix batches,
# which take 'spread' only, as in the reference.  ``twiddle`` must hold the
# forward roots (check_twiddle).  The runner functions take power-of-two
# batches, as the reference's do; plans (``execute_fft_plan``) run any
# B >= 1.

def fft_dit(x, block: int = 1024, twiddle=None):
    """M0 radix-2 DIT: log2(N) stage launches, bit reversal folded into stage 0
    (reference runner.py:118)."""
    return _single("fft_dit", x, block, twiddle=twiddle)


def fft_dif(x, block: int = 1024, twiddle=None):
    """M0 radix-2 DIF: log2(N) stage launches, bit reversal folded into the
    last (reference runner.py:166)."""
    return _single("fft_dif", x, block, twiddle=twiddle)


def fft_dit_batch(x, block: int = 1024, variant: str = "spread", twiddle=None):
    """M4: M0 over a (B, N) batch, one launch per stage (reference runner.py:781)."""
    return _batched("fft_dit_batch", x, block, twiddle=twiddle, variant=variant)


def fft_dif_batch(x, block: int = 1024, variant: str = "spread", twiddle=None):
    """M4 DIF mirror (reference runner.py:844)."""
    return _batched("fft_dif_batch", x, block, twiddle=twiddle, variant=variant)


def fft_dit_radix4(x, block: int = 1024, twiddle=None):
    """M5 radix-4 DIT (radix-2 tail for odd log2 N), digit reversal folded in
    (reference runner.py:1399)."""
    if isinstance(x, torch.Tensor) and x.numel() < 4:
        raise ValueError(f"radix-4 requires N >= 4, got N={x.numel()}")
    return _single("fft_dit_radix4", x, block, twiddle=twiddle)


def fft_dif_radix4(x, block: int = 1024, twiddle=None):
    """M5 radix-4 DIF (reference runner.py:1472)."""
    if isinstance(x, torch.Tensor) and x.numel() < 4:
        raise ValueError(f"radix-4 requires N >= 4, got N={x.numel()}")
    return _single("fft_dif_radix4", x, block, twiddle=twiddle)


def fft_dit_radix4_batch(x, block: int = 1024, variant: str = "spread", twiddle=None):
    """M5 batch (reference runner.py:1112)."""
    return _batched("fft_dit_radix4_batch", x, block, twiddle=twiddle, variant=variant, spread_only=True)


def fft_dif_radix4_batch(x, block: int = 1024, variant: str = "spread", twiddle=None):
    """M5 batch DIF (reference runner.py:1193)."""
    return _batched("fft_dif_radix4_batch", x, block, twiddle=twiddle, variant=variant, spread_only=True)


def fft_lds_fused(x, elems: int = 0, twiddle=None, *, stagger: int = 0, stage: int = 0):
    """Single-pass LDS-resident Stockham FFT (core length <= 32768); the
    keywords are the LDS_FUSED flow parameters of include/mfft.h (elements
    per thread, start stagger, staged form), 0 = the library's default."""
    return _single("fft_lds_fused", x, None, {"elems": elems, "stagger": stagger, "stage": stage}, twiddle=twiddle)


def fft_lds_fused_batch(x, elems: int = 0, twiddle=None, *, stagger: int = 0, stage: int = 0):
    return _batched("fft_lds_fused_batch", x, None, {"elems": elems, "stagger": stagger, "stage": stage},
                    twiddle=twiddle)


def _four_step_params(n1, chunk_rows, schedule, allow_fused_schedule) -> dict:
    if schedule == 2 and not allow_fused_schedule:
        raise ValueError("schedule=2 (both passes in one launch) needs allow_fused_schedule=True: when one of "
                         "its bounded waits gives up, the launch writes NaN and the execute still returns "
                         "success; the caller must check NativePlan.sync_overruns() (mfft_plan_sync_overruns) "
                         "after synchronising")
    return {"n1": n1, "chunk_rows": chunk_rows, "schedule": schedule}


def fft_four_step(x, n1: int = 0, chunk_rows: int = 0, schedule: int = 0, twiddle=None, *,
                  allow_fused_schedule: bool = False):
    """Two-pass four-step FFT (column pass + twiddle, in-place row pass).
    ``schedule=2`` (one fused launch) only with ``allow_fused_schedule=True``."""
    return _single("fft_four_step", x, None, _four_step_params(n1, chunk_rows, schedule, allow_fused_schedule),
                   twiddle=twiddle)


def fft_four_step_batch(x, n1: int = 0, chunk_rows: int = 0, schedule: int = 0, twiddle=None, *,
                        allow_fused_schedule: bool = False):
    return _batched("fft_four_step_batch", x, None,
                    _four_step_params(n1, chunk_rows, schedule, allow_fused_schedule), twiddle=twiddle)


def fft_dit_fused(x, block: int = 1024, tile: int = 64, twiddle=None):
    """Reference M1 name (runner.py:209): all stages fused on chip (LDS
    kernel, four-step above 32768 points)."""
    _check_pow2_block(block)
    return _single("fft_dit_fused", x, None, twiddle=twiddle)


def fft_dit_matrix(x, block: int = 1024, tile: int = 64, rows: int = 8, twiddle=None):
    """Reference M2 name (runner.py:379): the dense-dot core on the fp32
    matrix cores (cores of 2..16384 points; the library's choice above)."""
    _check_pow2_block(block)
    return _single("fft_dit_matrix", x, None, twiddle=twiddle)


def fft_dif_matrix(x, block: int = 1024, tile: int = 64, rows: int = 8, twiddle=None):
    """Reference M2 DIF name (runner.py:445)."""
    _check_pow2_block(block)
    return _single("fft_dif_matrix", x, None, twiddle=twiddle)


def fft_dit_matrix_batch(x, block: int = 1024, tile: int = 64, rows: int = 8, variant: str = "spread",
                         twiddle=None):
    """Reference M2 batch name (runner.py:956)."""
    _check_pow2_block(block)
    return _batched("fft_dit_matrix_batch", x, None, twiddle=twiddle, variant=variant, spread_only=True)


def fft_dif_matrix_batch(x, block: int = 1024, tile: int = 64, rows: int = 8, variant: str = "spread",
                         twiddle=None):
    """Reference M2 batch DIF name (runner.py:1038)."""
    _check_pow2_block(block)
    return _batched("fft_dif_matrix_batch", x, None, twiddle=twiddle, variant=variant, spread_only=True)


def fft_dit_matrix_packet_batch(x, block: int = 1024, tile: int = 64, rows: int = 8, packets: int = 2,
                                twiddle=None):
    """Reference M2 packet-loop name (runner.py:1271, experimental there):
    the same dense-dot matrix-core flow as fft_dit_matrix_batch, with the
    reference's checks of ``packets`` (a power of two, at most 2, dividing
    B), which only concern its Triton program."""
    _check_pow2_block(block)
    if isinstance(x, torch.Tensor) and x.dim() == 2:
        b = int(x.shape[0])
        if packets < 1 or (packets & (packets - 1)) != 0:
            raise ValueError(f"packets must be a power of two, got {packets}")
        if packets > 2:
            raise ValueError(f"packets={packets} exceeds the reference program's ceiling of 2")
        if b % packets != 0:
            raise ValueError(f"packets={packets} must divide batch B={b}")
    return _batched("fft_dit_matrix_batch", x, None, twiddle=twiddle)


def fft_dit_grouped(x, block: int = 1024, tile: int = 64, rows: int = 8,
                    glog: int = 2, maxp: int = 4096, cells: int = 1, twiddle=None):
    """Reference M3 name (runner.py:603): runs the LDS / four-step kernels."""
    _check_pow2_block(block)
    return _single("fft_dit_grouped", x, None, twiddle=twiddle)


def fft_dif_grouped(x, block: int = 1024, tile: int = 64, rows: int = 8,
                    glog: int = 2, maxp: int = 4096, cells: int = 1, twiddle=None):
    """Reference M3 DIF name (runner.py:685)."""
    _check_pow2_block(block)
    return _single("fft_dif_grouped", x, None, twiddle=twiddle)


def _check_variant(variant: str) -> None:
    if variant not in ("spread", "folded"):
        raise ValueError(f"variant must be 'spread' or 'folded', got {variant!r}")


def _check_pow2_block(block) -> None:
    if block is not None:
        log2_exact(block)


def bit_reverse_permute(x, block: int = 1024):
    """Y[r][bit_reverse(i)] = X[r][i] (reference runner.py:1542-1552), on a
    rank-1 (N,) or rank-2 (B, N) complex64 tensor; ``block`` must be a power
    of two (the kernel sizes its own launch)."""
    if isinstance(x, torch.Tensor) and x.dim() == 1:
        validate_input(x, "x", block=block, require_complex=True)
    else:
        validate_tensor(x, "x", dtype=torch.complex64, block=block)
    n = int(x.shape[-1])
    log2_exact(n)
    b = 1 if x.dim() == 1 else int(x.shape[0])
    out = torch.empty_like(x)
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    with device_context(dev):
        native.bit_reverse_permute(x.data_ptr(), out.data_ptr(), n, b, stream_handle(dev))
    return out


# ---------------- dedicated real-flow epilogues (runner.py:1640-1834) ----------------
# The plans fuse the R2C stitch and the C2R pre-twiddle into their kernels;
# these runners expose the same steps on their own, for a caller that runs
# the half-length core itself (mfft_r2c_stitch / mfft_c2r_pre /
# mfft_c2r_unpack: one launch each, no plan, no allocation but the output).


def _validate_real_half(x, n: int, bins: int, name: str) -> None:
    """The epilogues' shared contract (reference runner.py:1661-1678)."""
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(x).__name__}")
    if x.dtype != torch.complex64:
        raise TypeError(f"{name} must be complex64, got {x.dtype}")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (device='cuda'), got {x.device}")
    if x.dim() not in (1, 2):
        raise ValueError(f"{name} must be rank-1 or rank-2, got dim={x.dim()}")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    log2_exact(n)
    if n < 4:
        raise ValueError(f"dedicated real flow needs N >= 4, got {n}")
    if x.shape[-1] != bins:
        raise ValueError(f"{name} last dim {x.shape[-1]} != expected {bins}")


def _epilogue_block(block) -> int:
    if not isinstance(block, int) or block <= 0 or (block & (block - 1)):
        raise ValueError(f"block must be a positive power of two, got {block!r}")
    return block


def _epilogue(fn, x, out, n):
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    rows = 1 if x.dim() == 1 else int(x.shape[0])
    with device_context(dev):
        fn(x.data_ptr(), out.data_ptr(), n, rows, stream_handle(dev))
    return out


def r2c_stitch(z, n: int, scale: float = 1.0, block: int = 1024):
    """R2C epilogue: ``z``, the unnormalised N/2-point FFT of the packed
    pairs x[2k] + i x[2k+1] (``(N/2,)`` or ``(B, N/2)``), to the real input's
    ``(N/2+1,)`` / ``(B, N/2+1)`` spectrum times ``scale``, with the
    imaginary parts of bins 0 and N/2 exactly 0 (reference runner.py:1687)."""
    _validate_real_half(z, n, n >> 1, "z")
    scale = float(scale)
    _epilogue_block(block)
    out = torch.empty((*z.shape[:-1], (n >> 1) + 1), dtype=torch.complex64, device=z.device)
    return _epilogue(lambda i, o, nn, r, st: native.r2c_stitch(i, o, nn, r, scale, st), z, out, n)


def c2r_pre(xh, n: int, block: int = 1024):
    """C2R prologue: the half spectrum ``(N/2+1,)`` / ``(B, N/2+1)``
    (imaginary parts of bins 0 and N/2 ignored) to the ``(N/2,)`` /
    ``(B, N/2)`` input of the half-length core (reference runner.py:1718)."""
    _validate_real_half(xh, n, (n >> 1) + 1, "xh")
    _epilogue_block(block)
    out = torch.empty((*xh.shape[:-1], n >> 1), dtype=torch.complex64, device=xh.device)
    return _epilogue(native.c2r_pre, xh, out, n)


def c2r_unpack(u, n: int, scale: float = 1.0, block: int = 1024):
    """C2R epilogue: ``u``, the unnormalised forward N/2-point FFT of
    :func:`c2r_pre`'s output, to the real samples ``(N,)`` / ``(B, N)``
    float32 times ``scale`` (2 x the norm's inverse scale, e.g. 2/N for
    ``backward``); ``u`` is read in mirror order, which turns the forward
    core into the inverse (reference runner.py:1744)."""
    _validate_real_half(u, n, n >> 1, "u")
    scale = float(scale)
    _epilogue_block(block)
    out = torch.empty((*u.shape[:-1], n), dtype=torch.float32, device=u.device)
    return _epilogue(lambda i, o, nn, r, st: native.c2r_unpack(i, o, nn, r, scale, st), u, out, n)


# Host references of the three epilogues (the reference's *_ref functions,
# runner.py:1776-1834): the same formulas in torch complex arithmetic, on
# any device, with the roots in float64.  They are what the reference's
# host tests check the epilogues against; no execute path calls them.

def _roots(n: int, count: int, sign: float, device):
    k = torch.arange(count, dtype=torch.float64, device=device)
    return torch.polar(torch.ones_like(k), sign * 2.0 * math.pi * k / n).to(torch.complex64)


def r2c_stitch_ref(z, n: int, scale: float = 1.0):
    """X[k] = A - i w^k C for k in [0, N/2], A = (Z[k] + conj Z[-k]) / 2,
    C = (Z[k] - conj Z[-k]) / 2 (indices mod N/2), w = exp(-2 pi i / N);
    imaginary parts of bins 0 and N/2 set to 0; times ``scale``."""
    h = n >> 1
    if z.shape[-1] != h:
        raise ValueError(f"z last dim {z.shape[-1]} != N/2 ({h})")
    k = torch.arange(h + 1, device=z.device)
    zk, zj = z[..., k % h], z[..., (h - k) % h].conj()
    x = 0.5 * (zk + zj) - 1j * _roots(n, h + 1, -1.0, z.device) * (0.5 * (zk - zj))
    edge = (k == 0) | (k == h)
    x = torch.complex(x.real, torch.where(edge, torch.zeros_like(x.imag), x.imag))
    return x * scale


def c2r_pre_ref(xh, n: int):
    """Z[k] = A + i w^-k C for k in [0, N/2), A = (X[k] + conj X[N/2-k]) / 2,
    C = (X[k] - conj X[N/2-k]) / 2, w = exp(-2 pi i / N), with the
    imaginary parts of X[0] and X[N/2] taken as 0."""
    h = n >> 1
    if xh.shape[-1] != h + 1:
        raise ValueError(f"xh last dim {xh.shape[-1]} != N/2+1 ({h + 1})")
    x = xh.clone()
    x[..., 0] = x[..., 0].real.to(x.dtype)
    x[..., h] = x[..., h].real.to(x.dtype)
    k = torch.arange(h, device=xh.device)
    xk, xj = x[..., k], x[..., h - k].conj()
    return 0.5 * (xk + xj) + 1j * _roots(n, h, 1.0, xh.device) * (0.5 * (xk - xj))


def c2r_unpack_ref(u, n: int, scale: float = 1.0):
    """out[2k] + i out[2k+1] = scale * U[(N/2 - k) mod N/2]."""
    h = n >> 1
    if u.shape[-1] != h:
        raise ValueError(f"u last dim {u.shape[-1]} != N/2 ({h})")
    k = torch.arange(h, device=u.device)
    v = (u[..., (h - k) % h] * scale).contiguous()
    return torch.view_as_real(v).reshape(*u.shape[:-1], n)


def twiddle_tables(n: int, device):
    """Planar (cos, sin) float32 of exp(-2*pi*i*idx/n), idx in [0, n/2)
    (reference runner.py:93-97); computed in float64 and rounded once.
    The native plans build their own tables; this is an inspection helper."""
    log2_exact(n)
    idx = torch.arange(n >> 1, dtype=torch.float64)
    ang = -2.0 * math.pi * idx / n
    return (torch.cos(ang).to(torch.float32).to(device), torch.sin(ang).to(torch.float32).to(device))


def _sync() -> None:
    if device_ready():
        torch.cuda.synchronize()


def time_call(fn, warmup: int = 5, iters: int = 20) -> float:
    """Median API wall time in ms of ``fn()`` (reference runner.py:1560-1573):
    ``warmup`` untimed calls, then ``iters`` calls each followed by a device
    synchronisation; includes the host path, allocation and the sync."""
    for _ in range(warmup):
        fn()
    _sync()
    samples = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        _sync()
        samples.append((time.perf_counter() - t0) * 1e3)
    samples.sort()
    return samples[len(samples) // 2]


def _stats(xs):
    if not xs:
        return None
    xs = sorted(xs)
    return {"median": xs[len(xs) // 2], "min": xs[0], "p10": xs[max(0, int(0.10 * len(xs)))],
            "p90": xs[min(len(xs) - 1, int(0.90 * len(xs)))], "trials": len(xs)}


def time_call_detailed(fn, warmup: int = 10, trials: int = 50, seed: int = 0) -> dict:
    """The reference's trial protocol (runner.py:1576-1635): ``warmup``
    untimed calls, then ``trials`` calls in an order shuffled by
    ``random.Random(seed)``, each bracketed by HIP events on the current
    stream and a device synchronisation.  Returns ``{"api_ms": stats,
    "kernel_ms": stats, "metric_note": str}`` with stats = ``{median, min,
    p10, p90, trials}``; ``kernel_ms`` keeps only positive event times and
    is None when there are none (or no GPU)."""
    for _ in range(warmup):
        fn()
    _sync()
    use_events = device_ready()
    order = list(range(trials))
    random.Random(seed).shuffle(order)
    api, kern = [], []
    for _ in order:
        if use_events:
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            api.append((time.perf_counter() - t0) * 1e3)
            kt = s.elapsed_time(e)
            if kt > 0:
                kern.append(kt)
        else:
            t0 = time.perf_counter()
            fn()
            _sync()
            api.append((time.perf_counter() - t0) * 1e3)
    return {"api_ms": _stats(api), "kernel_ms": _stats(kern),
            "metric_note": ("api_ms = synchronized wall time (host path + allocation + launch + sync); "
                            "kernel_ms = HIP event elapsed time on the current stream (device time) when "
                            "events report > 0, else null")}


def time_native_graph(nplan: native.NativePlan, x: torch.Tensor, out: torch.Tensor, ws, reps: int = 20,
                      rounds: int = 5) -> float:
    """Median device time (ms) of one execute of ``nplan``: ``reps`` executes
    recorded into one HIP graph on a side stream, the graph replayed
    ``rounds`` times between HIP events on the current stream.

    For launch-bound shapes (a few microseconds per execute) a host loop of
    enqueues measures the host's enqueue rate instead: the GPU idles between
    kernels whenever one enqueue takes longer than one kernel.  Replaying a
    graph launches the executes back to back.  An execute records only
    kernel launches (no allocation, memset or host sync), so it captures as
    is; ``ws`` (or None) must be allocated before the call."""
    dev = x.device
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    wp = ws.data_ptr() if ws is not None else 0
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        for _ in range(2):
            nplan.execute_ws(x.data_ptr(), out.data_ptr(), wp, nplan.ws_bytes, side.cuda_stream)
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(reps):
                nplan.execute_ws(x.data_ptr(), out.data_ptr(), wp, nplan.ws_bytes, side.cuda_stream)
    torch.cuda.synchronize(dev)
    cur = torch.cuda.current_stream(dev)
    graph.replay()
    res = []
    for _ in range(rounds):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(cur)
        graph.replay()
        e.record(cur)
        e.synchronize()
        res.append(s.elapsed_time(e) / reps)
    del graph
    res.sort()
    return res[len(res) // 2]
