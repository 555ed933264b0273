"""Four-step compositions around an exchangeable sub-FFT core
(reference src/xpu/adapter_hybrid.py:60-108 HybridPlan / plan_hybrid,
:224-302 run_hybrid, :318-323 _core_fft_1d; the diagnostics plan_ledger,
summarize_samples, time_cell and profile_hybrid, :273-430).

N = tile * t2 (t2 = N / tile), digits m = m1 * tile + m0, k = k_t + t2 * k_r:

1. gather  x.reshape(t2, tile).T -> (m0, m1)           [framework copy]
2. core    row FFTs of length t2 over m1 -> (m0, k_t)
3. boundary  transpose and twiddle W_N^(k_t m0) -> (k_t, m0)   [one HIP pass]
4. core    row FFTs of length tile over m0 -> (k_t, k_r)
5. scatter (k_t, k_r) -> X[k_t + t2 k_r]                [framework copy]

``core`` names the processing unit of steps 2 and 4 (the external-core
registry, config/external_cores.json):

* ``"vendor"``: rocFFT through ``torch.fft`` -- the reference's "A1P1"
  materialized external sub-transform.  Steps 1 and 5 are torch copies, as in
  the reference; step 3 is this library's ``mfft_twiddle_transpose`` kernel.
* ``"local"``: this library's own four-step (one native plan, both passes
  fused with the twiddle and the transposes), n1 = t2.  The reference's
  name for its in-library core, ``"triton"``, selects it too.

A composition only ever runs when a composition table promotes it for an
exact shape (``composition.composition_select``), or when a caller builds a
plan with ``plan_hybrid`` and calls ``run_hybrid`` itself.
"""
from __future__ import annotations

from dataclasses import dataclass, field

CORES = ("vendor", "local")


@dataclass
class HybridPlan:
    """A composition of one shape; the core is a parameter of the plan."""

    n: int
    batch: int
    tile: int
    direction: str = "dit"
    core: str = "vendor"
    transform_direction: str = "forward"
    norm: str = "backward"
    stage2_len: int = field(init=False)

    def __post_init__(self):
        # the reference's order of checks and key phrases (adapter_hybrid.py:82-90)
        if self.direction != "dit":
            raise ValueError("the composition covers DIT only (the DIT decomposition)")
        if self.tile <= 0 or self.n % self.tile:
            raise ValueError(f"tile {self.tile} must divide N={self.n}")
        if self.n <= 0 or (self.n & (self.n - 1)) or (self.tile & (self.tile - 1)):
            raise ValueError("N and tile must be powers of two")
        # the reference's in-library core is its Triton one; here it is this library's own
        if self.core == "triton":
            self.core = "local"
        if self.core not in CORES:
            raise ValueError(f"unknown core {self.core!r}; known: {CORES} (and 'triton', an alias of 'local')")
        if self.transform_direction not in ("forward", "inverse"):
            raise ValueError(f"bad transform_direction {self.transform_direction!r}")
        self.stage2_len = self.n // self.tile
        if self.core == "local" and not (16 <= self.tile <= 1024 and 16 <= self.stage2_len <= 1024):
            raise ValueError("the local core needs tile and N/tile in [16, 1024]")


def plan_hybrid(n: int, batch: int, tile: int = 64, core: str = "vendor", transform_direction: str = "forward",
                norm: str = "backward") -> HybridPlan:
    return HybridPlan(n=n, batch=batch, tile=tile, core=core, transform_direction=transform_direction, norm=norm)


def _checked_batch(x, plan: HybridPlan) -> int:
    import torch

    from .validate import validate_tensor

    validate_tensor(x, "x", dtype=torch.complex64, ranks=(1, 2), last=plan.n)
    b = 1 if x.dim() == 1 else int(x.shape[0])
    if b != plan.batch:
        raise ValueError(f"plan batch {plan.batch} != input batch {b}")
    return b


def _vendor_steps(x, plan: HybridPlan, b: int, lap=None):
    """Steps 1-5 around the vendor core; ``lap(name)``, when given, is
    called after each step (profile_hybrid's phase clock)."""
    import torch

    from . import native
    from .entry import norm_scale
    from .runner import stream_handle

    n, tile, t2 = plan.n, plan.tile, plan.stage2_len
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    inverse = plan.transform_direction == "inverse"
    sub = torch.fft.ifft if inverse else torch.fft.fft
    sub_norm = "forward" if inverse else "backward"  # unnormalised sub-transforms either way
    lap = lap or (lambda name, t=None: None)
    with torch.cuda.device(dev):
        blocks = x.reshape(b, t2, tile).permute(0, 2, 1).contiguous()            # (b, tile, t2)
        lap("gather", blocks)
        stage1 = sub(blocks, dim=-1, norm=sub_norm)                               # (b, tile, t2): (m0, k_t)
        lap("stage1_core", stage1)
        grid = torch.empty((b, t2, tile), dtype=torch.complex64, device=x.device)
        native.twiddle_transpose(stage1.data_ptr(), grid.data_ptr(), tile, t2, b, plan.transform_direction,
                                 stream_handle(dev))                              # (b, t2, tile): (k_t, m0)
        lap("twiddle_transpose", grid)
        stage2 = sub(grid, dim=-1, norm=sub_norm)                                 # (k_t, k_r)
        lap("stage2_core", stage2)
        out = stage2.permute(0, 2, 1).reshape(x.shape)                            # X[k_t + t2 k_r]
        scale = norm_scale(n, plan.transform_direction, plan.norm)
        if scale != 1.0:
            out = out * scale
        out = out.contiguous()
        lap("scatter", out)
        return out


def run_hybrid(x, plan: HybridPlan):
    """Execute a composition on a (B, N) or (N,) complex64 GPU tensor;
    returns a new tensor of the same shape."""
    import torch

    from .runner import get_native_plan, launch

    b = _checked_batch(x, plan)
    if plan.core == "local":
        dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
        nplan = get_native_plan("run_hybrid", plan.n, b, "c2c", plan.transform_direction, plan.norm, None,
                                {"tile": plan.tile}, dev)
        return launch(nplan, x, torch.empty_like(x))
    return _vendor_steps(x, plan, b)


def plan_ledger(plan: HybridPlan) -> dict:
    """Analytic call and boundary accounting of one composition (reference
    adapter_hybrid.py:273-315): the sub-FFT rows and lengths of each stage,
    the host API calls and launches where they are known, and the bytes
    each framework-owned boundary moves (read + write, complex64).  Not
    measured; rocFFT's launches inside ``torch.fft`` are opaque and stay
    None."""
    n, b, tile, t2 = plan.n, plan.batch, plan.tile, plan.stage2_len
    elem = 8
    rows = {"stage1": b * tile, "stage1_len": t2, "stage2": b * t2, "stage2_len": tile}
    if plan.core == "local":
        return {
            "core": "local", "core_calls": rows, "core_api_calls": 1, "core_launches_est": 2,
            "materialized_boundaries": [
                {"op": "pass 1: column FFTs of length N/tile, twiddle, transposed store (native)",
                 "bytes_est": 2 * b * n * elem},
                {"op": "pass 2: row FFTs of length tile in place (native)", "bytes_est": 2 * b * n * elem}],
            "gm_bytes_framework_est": 0,
            "gm_bytes_core_est": 4 * b * n * elem,
            "sync_points_per_timed_call": 1, "element_bytes_assumed": elem,
            "twiddle_and_row_tables": "native plan tables (uploaded once per plan)",
            "buffers": "none: the second pass runs in place in the output",
        }
    from .entry import norm_scale

    scaled = norm_scale(n, plan.transform_direction, plan.norm) != 1.0
    boundaries = [
        {"op": "gather x.reshape(t2, tile).T -> blocks (torch copy)", "bytes_est": 2 * b * n * elem},
        {"op": "twiddle + transpose -> grid (mfft_twiddle_transpose, roots computed in the kernel)",
         "bytes_est": 2 * b * n * elem},
        {"op": "digit-reversal transpose -> out (torch copy)", "bytes_est": 2 * b * n * elem},
    ]
    if scaled:
        boundaries.append({"op": "normalization scale (torch multiply)", "bytes_est": 2 * b * n * elem})
    return {
        "core": "vendor", "core_calls": rows,
        "core_api_calls": 2,  # one batched torch.fft call per stage
        "core_launches_est": None,  # inside rocFFT: opaque
        "materialized_boundaries": boundaries,
        "gm_bytes_framework_est": sum(x["bytes_est"] for x in boundaries),
        "sync_points_per_timed_call": 1, "element_bytes_assumed": elem,
        "twiddle_and_row_tables": "none held: the boundary kernel computes its roots",
        "buffers": "per call (torch's caching allocator); the output is fresh per call",
    }


def summarize_samples(samples: list) -> dict:
    """p50, MAD, p95, max and outliers of timing samples (reference
    adapter_hybrid.py:326-350, same keys and rules): the median of an even
    count is the mean of the middle two; an outlier exceeds p50 + 3 MAD, or
    1.5 p50 when the MAD is 0; p95 is the sample at round(0.95 (n - 1))."""
    if not samples:
        return {"n": 0}
    s = sorted(float(v) for v in samples)
    n = len(s)

    def median(xs):
        return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])

    p50 = median(s)
    mad = median(sorted(abs(v - p50) for v in s))
    thr = p50 + 3.0 * mad if mad > 0 else 1.5 * p50
    out = [v for v in s if v > thr]
    return {"n": n, "p50": p50, "mad": mad, "p95": s[min(n - 1, int(round(0.95 * (n - 1))))], "max": s[-1],
            "outlier_count": len(out), "outlier_values": out, "outlier_threshold": thr}


def time_cell(fn, x, warmup: int, trials: int):
    """(first_ms, stats): the first call alone (plan creation and table
    upload included), then ``summarize_samples`` of ``trials`` calls after
    ``warmup``, each between two device synchronizes (reference
    adapter_hybrid.py:353-374)."""
    import time

    import torch

    dev = x.device
    t0 = time.perf_counter()
    fn(x)
    torch.cuda.synchronize(dev)
    first_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        fn(x)
    torch.cuda.synchronize(dev)
    samples = []
    for _ in range(trials):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        fn(x)
        torch.cuda.synchronize(dev)
        samples.append((time.perf_counter() - t0) * 1e3)
    return first_ms, summarize_samples(samples)


def profile_hybrid(x, plan: HybridPlan):
    """``(out, phases)``: ``run_hybrid``'s result and the wall time of each
    of its phases, with a device synchronize after each (reference
    adapter_hybrid.py:377-430; diagnostic only, slower than the steady
    path).  Vendor core: gather, stage-1 core, twiddle-transpose, stage-2
    core and scatter, the contiguity of every materialised core input and
    output, and ``hidden_copies`` (core inputs that were not contiguous).
    Local core: one phase, the native four-step, which does all five steps
    in its two passes."""
    import time

    import torch

    b = _checked_batch(x, plan)
    dev = x.device
    phases: dict = {"core": plan.core}
    if plan.core == "local":
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        out = run_hybrid(x, plan)
        torch.cuda.synchronize(dev)
        phases["fused_four_step_ms"] = (time.perf_counter() - t0) * 1e3
        phases["hidden_copies"] = []
        return out, phases
    clock = [None]
    # the reference's names for the tensors each phase hands on
    handed = {"gather": "stage1_in_contiguous", "stage1_core": "stage1_out_contiguous",
              "twiddle_transpose": "stage2_in_contiguous", "stage2_core": "stage2_out_contiguous"}

    def lap(name, t):
        torch.cuda.synchronize(dev)
        now = time.perf_counter()
        phases[f"{name}_ms"] = (now - clock[0]) * 1e3
        clock[0] = now
        if name in handed:
            phases[handed[name]] = bool(t.is_contiguous())

    torch.cuda.synchronize(dev)
    clock[0] = time.perf_counter()
    out = _vendor_steps(x, plan, b, lap)
    phases["hidden_copies"] = [k for k in ("stage1_in", "stage2_in") if not phases[f"{k}_contiguous"]]
    return out, phases
