"""Four-step compositions around an exchangeable sub-FFT core
(reference src/xpu/adapter_hybrid.py:60-108 HybridPlan / plan_hybrid,
:224-302 run_hybrid, :318-323 _core_fft_1d).

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


def run_hybrid(x, plan: HybridPlan):
    """Execute a composition on a (B, N) or (N,) complex64 GPU tensor;
    returns a new tensor of the same shape."""
    import torch

    from . import native
    from .entry import norm_scale
    from .runner import get_native_plan, launch, stream_handle
    from .validate import validate_tensor

    validate_tensor(x, "x", dtype=torch.complex64, ranks=(1, 2), last=plan.n)
    b = 1 if x.dim() == 1 else int(x.shape[0])
    if b != plan.batch:
        raise ValueError(f"plan batch {plan.batch} != input batch {b}")
    n, tile, t2 = plan.n, plan.tile, plan.stage2_len
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    if plan.core == "local":
        nplan = get_native_plan("run_hybrid", n, b, "c2c", plan.transform_direction, plan.norm, None,
                                {"tile": tile}, dev)
        return launch(nplan, x, torch.empty_like(x))
    inverse = plan.transform_direction == "inverse"
    sub = torch.fft.ifft if inverse else torch.fft.fft
    sub_norm = "forward" if inverse else "backward"  # unnormalised sub-transforms either way
    with torch.cuda.device(dev):
        blocks = x.reshape(b, t2, tile).permute(0, 2, 1).contiguous()            # (b, tile, t2)
        stage1 = sub(blocks, dim=-1, norm=sub_norm)                               # (b, tile, t2): (m0, k_t)
        grid = torch.empty((b, t2, tile), dtype=torch.complex64, device=x.device)
        native.twiddle_transpose(stage1.data_ptr(), grid.data_ptr(), tile, t2, b, plan.transform_direction,
                                 stream_handle(dev))                              # (b, t2, tile): (k_t, m0)
        stage2 = sub(grid, dim=-1, norm=sub_norm)                                 # (k_t, k_r)
        out = stage2.permute(0, 2, 1).reshape(x.shape)                            # X[k_t + t2 k_r]
        scale = norm_scale(n, plan.transform_direction, plan.norm)
        if scale != 1.0:
            out = out * scale
        return out.contiguous()
