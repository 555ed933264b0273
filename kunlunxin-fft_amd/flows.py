"""Runner name -> native flow and parameters (host-only: no torch import).

``execute_fft_plan`` dispatches by ``plan.executed`` as the reference does
(entry.py:549-550, ``getattr(runner, plan.executed)``); here the name
selects a flow of ``libmfft.so`` and ``flow_params`` maps the plan's
parameters onto that flow's native parameters (the C ABI's ``params``
array, include/mfft.h).  Kept apart from ``runner`` so that host code (the
launch ledger, the selector's tooling) can resolve a plan without torch.
"""
from __future__ import annotations

from . import native
from .validate import log2_exact

DEFAULT_STAGE_BLOCK = 256

# runner name -> (native flow, parameter kind)
RUNNER_FLOWS = {
    "fft_dit": (native.FLOW_RADIX2_DIT, "block"),
    "fft_dit_batch": (native.FLOW_RADIX2_DIT, "block"),
    "fft_dif": (native.FLOW_RADIX2_DIF, "block"),
    "fft_dif_batch": (native.FLOW_RADIX2_DIF, "block"),
    "fft_dit_radix4": (native.FLOW_RADIX4_DIT, "block"),
    "fft_dit_radix4_batch": (native.FLOW_RADIX4_DIT, "block"),
    "fft_dif_radix4": (native.FLOW_RADIX4_DIF, "block"),
    "fft_dif_radix4_batch": (native.FLOW_RADIX4_DIF, "block"),
    "fft_lds_fused": (native.FLOW_LDS_FUSED, "lds"),
    "fft_lds_fused_batch": (native.FLOW_LDS_FUSED, "lds"),
    "fft_four_step": (native.FLOW_FOUR_STEP, "fourstep"),
    "fft_four_step_batch": (native.FLOW_FOUR_STEP, "fourstep"),
    "fft_dit_fused": (native.FLOW_AUTO, "none"),
    "fft_dit_matrix": (native.FLOW_DENSE_MFMA, "dense"),
    "fft_dif_matrix": (native.FLOW_DENSE_MFMA, "dense"),
    "fft_dit_matrix_batch": (native.FLOW_DENSE_MFMA, "dense"),
    "fft_dif_matrix_batch": (native.FLOW_DENSE_MFMA, "dense"),
    "fft_dit_grouped": (native.FLOW_AUTO, "none"),
    "fft_dif_grouped": (native.FLOW_AUTO, "none"),
    "run_hybrid": (native.FLOW_FOUR_STEP, "hybrid"),
}


def flow_params(executed: str, n: int, transform_type: str, block, params: dict) -> tuple:
    """(flow id, native params) for one runner name and plan parameters."""
    if executed not in RUNNER_FLOWS:
        raise ValueError(f"unknown runner {executed!r}")
    flow, kind = RUNNER_FLOWS[executed]
    params = params or {}
    core = n // 2 if transform_type in ("r2c", "c2r") else n
    # A legacy table entry measured on the c2c core of length n also answers
    # r2c/c2r, whose core is n/2: keep its flow where the flow can run that
    # core, else let the library pick (LDS up to 32768, four-step above).
    if kind == "lds":
        # LDS kernel limits: core <= 32768; 32 elements per thread from 1024
        # points; >= 16 from 8192 points
        e = int(params.get("elems", 0))
        logc = core.bit_length() - 1
        if core > 32768:
            return native.FLOW_AUTO, ()
        if e == 32 and logc < 10:
            e = 0
        # r2c cores below 32768 run with 16 elements per thread: the
        # 32-element kernel stitches through the output row (one more pass
        # over it, measured 1.3-1.8x slower there); at 32768 it is the only
        # single-pass form
        if e == 32 and transform_type == "r2c" and logc < 15:
            e = 16
        # c2r cores below 32768 run with 16 elements per thread: they load
        # each bin once and pair it with its mirror bin through LDS, where the
        # 32-element kernel (no registers to spare for the pairs) loads every
        # bin twice (measured 1.3-1.5x slower at 2^10-2^14 points)
        if e == 32 and transform_type == "c2r" and logc < 15:
            e = 16
        if logc >= 13 and 0 < e < 16:
            e = 0
        if logc == 15:
            e = 0
        # the staged form: fewer than 16 threads per transform of the core
        # (the elements per thread the library resolves e = 0 to, below 2^15:
        # 16 up to 16 points, 8 up to 64, else 16)
        stage = int(params.get("stage", 0))
        if stage:
            eff = e or (16 if logc <= 4 else 8 if logc <= 6 else 16)
            if eff == 32 or logc - min(eff.bit_length() - 1, logc) >= 4:
                stage = 0
        if stage:
            return flow, (e, int(params.get("stagger", 0)), 1)
        return flow, (e, int(params.get("stagger", 0)))
    if kind == "fourstep":
        n1 = int(params.get("n1", 0))
        if core < 256:
            return native.FLOW_AUTO, ()
        if n1 and (core % n1 or not 16 <= core // n1 <= 1024 or not 16 <= n1 <= 1024):
            n1 = 0
        sched = int(params.get("schedule", 0))
        if sched == 2:
            l1 = (n1 or (1 << ((core.bit_length() - 1) // 2))).bit_length() - 1
            l2 = core.bit_length() - 1 - l1
            if not (7 <= l1 <= 9 and 7 <= l2 <= 9 and abs(l1 - l2) <= 1):
                sched = 0  # a real flow's half-length core outside the fused range
        # params[3]: the pass-2 row order (schedules 0, 1, 3), the queue lag (schedule 2)
        last = int(params.get("lag", 0)) if sched == 2 else int(params.get("pass2_order", 0))
        return flow, (n1, int(params.get("chunk_rows", 0)), sched, last)
    if kind == "block":
        # a stage flow needs at least one stage (radix-4: one radix-4 stage);
        # shorter cores (N=1 c2c, N=2 real) run in the single-pass kernel
        if core < (4 if flow in (native.FLOW_RADIX4_DIT, native.FLOW_RADIX4_DIF) else 2):
            return native.FLOW_AUTO, ()
        b = int(block or DEFAULT_STAGE_BLOCK)
        log2_exact(b)
        # the reference's block counts elements per Triton program (any power
        # of two; its sweeps run up to 2048); here it is threads per
        # workgroup, 64 (one wave) to 1024: other powers of two clamp
        return flow, (min(max(b, 64), 1024),)
    if kind == "dense":
        # the dense-dot matrix-core flow runs cores of 2 .. 16384 points;
        # other lengths leave the flow to the library
        if not 2 <= core <= native.MAX_MFMA_CORE:
            return native.FLOW_AUTO, ()
        return flow, ()
    if kind == "hybrid":
        tile = int(params.get("tile", 0))
        n1 = core // tile if tile and core % tile == 0 else 0
        return flow, (n1, 0)
    return flow, ()


