"""GPU parity: every native flow against the CPU oracle (float64), through the
C ABI (via the package's plan API or the ctypes NativePlan).

Gate (north star): relative L2 error <= 1e-5 against the float64 oracle, and
the reference's peak-normalised worst-element error (max_rel_error) <= 1e-5
(the reference's own worst published figure is ~1.2e-6; its gate 1e-4).
At the benchmark's full sizes the C oracle is checked on a subset of rows and
numpy's float64 FFT on all rows, plus size-independent properties (round
trip, Parseval, linearity).
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import (
    DeviceProfile, ExecutionPlan, execute_fft_plan, native, plan_fft, run_fft,
)
from kunlunxin_fft_amd.entry import _resolve
from kunlunxin_fft_amd.runner import bit_reverse_permute, run

pytestmark = pytest.mark.gpu

RTOL_L2 = 1e-5
RTOL_MAX = 1e-5


def seeded_c64(n, b, session=0):
    """scripts/issue10_wp3_holdout.py:127-140 input protocol."""
    rng = np.random.default_rng(102026 + 100000 * session + 10 * n + b)
    x = (rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))).astype(np.complex64)
    return x[0] if b == 1 else x


def seeded_f32(n, b, session=0):
    rng = np.random.default_rng(102026 + 100000 * session + 10 * n + b)
    x = rng.standard_normal((b, n)).astype(np.float32)
    return x[0] if b == 1 else x


def mkplan(executed, n, b, tt="c2c", td="forward", norm="backward", params=None, block=256):
    return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed=executed, block=block,
                         flow_id="test", flow_realization="test", processing_unit="test",
                         params=params or {}, transform_type=tt, transform_direction=td, norm=norm)


def check(got, ref, label):
    l2 = oracle.rel_l2(got, ref)
    mx = oracle.max_rel_error(got, ref)
    assert l2 <= RTOL_L2 and mx <= RTOL_MAX, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"
    return l2, mx


def np_ref(x, td, norm):
    n = x.shape[-1]
    if td == "forward":
        return np.fft.fft(x.astype(np.complex128), norm="backward" if norm == "none" else norm)
    if norm in ("none", "forward"):
        return np.fft.ifft(x.astype(np.complex128), norm="backward") * n
    return np.fft.ifft(x.astype(np.complex128), norm=norm)


def test_single_hip_runtime_in_process(gpu):
    """The library must bind to torch's HIP runtime, not load a second one."""
    torch.zeros(1, device=gpu)
    native.load()
    maps = open("/proc/self/maps").read()
    paths = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len(paths) == 1, paths


# ---------------------------------------------------------------- C2C flows
FLOW_CASES = []
for name in ("fft_dit", "fft_dif"):
    FLOW_CASES += [(name, n) for n in (2, 8, 64, 1024, 4096, 1 << 15)]
for name in ("fft_dit_radix4", "fft_dif_radix4"):
    FLOW_CASES += [(name, n) for n in (4, 8, 32, 256, 2048, 1 << 15)]
FLOW_CASES += [("fft_lds_fused", n) for n in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384,
                                             32768)]
FLOW_CASES += [("fft_four_step", n) for n in (256, 1024, 4096, 1 << 14, 1 << 16, 1 << 18, 1 << 20)]


# batch 3 below 2^18 points (the large-N batches are the config tests' cases)
@pytest.mark.parametrize("name,n,b", [(name, n, b) for b in (1, 3) for name, n in FLOW_CASES
                                      if b == 1 or n < (1 << 18)])
def test_c2c_forward_matches_oracle(gpu, name, n, b):
    x = seeded_c64(n, b)
    bname = name + "_batch" if b > 1 else name
    y = execute_fft_plan(mkplan(bname, n, b), torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = oracle.fft_dit(x) if n <= (1 << 16) else np.fft.fft(x.astype(np.complex128))
    check(y, ref, f"{bname} N={n} B={b}")


@pytest.mark.parametrize("name", ["fft_dit", "fft_dif", "fft_dit_radix4", "fft_dif_radix4",
                                  "fft_lds_fused", "fft_four_step"])
@pytest.mark.parametrize("norm", ["none", "forward", "backward", "ortho"])
@pytest.mark.parametrize("td", ["forward", "inverse"])
def test_c2c_all_norms(gpu, name, norm, td):
    n, b = 1024, 5
    x = seeded_c64(n, b, session=1)
    y = execute_fft_plan(mkplan(name + "_batch", n, b, td=td, norm=norm),
                         torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.c2c(x, td, norm), f"{name} {td} {norm}")


@pytest.mark.parametrize("elems,n", [(e, n) for e in (4, 8) for n in (8, 16, 32, 64, 128, 256, 512, 1024, 2048,
                                                                    4096, 8192)]
                         + [(16, n) for n in (32, 256, 2048, 4096)]
                         + [(32, n) for n in (1024, 2048, 4096, 8192, 16384, 32768)] + [(16, 16384)])
def test_lds_elems_axis_neutral(gpu, elems, n):
    x = seeded_c64(n, 7)
    y = execute_fft_plan(mkplan("fft_lds_fused_batch", n, 7, params={"elems": elems}),
                         torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.fft_dit(x), f"lds elems={elems} N={n}")


@pytest.mark.parametrize("elems", [4, 8])
@pytest.mark.parametrize("n", [64, 1024, 2048])
@pytest.mark.parametrize("b", [1, 5])
def test_lds_small_elems_inverse_and_real(gpu, elems, n, b):
    """The latency kernels (4 and 8 elements per thread) in the inverse
    direction (conjugated roots) and in the fused R2C/C2R modes; at 8
    elements, N = 1024 and 2048 pair the mirror bins across lanes (a
    512- or 1024-point core, whole waves per transform)."""
    x = seeded_c64(n, b, session=3)
    sfx = "_batch" if b > 1 else ""
    p = {"elems": elems}
    y = execute_fft_plan(mkplan("fft_lds_fused" + sfx, n, b, td="inverse", norm="ortho", params=p),
                         torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.c2c(x, "inverse", "ortho"), f"lds elems={elems} N={n} B={b} inverse")
    r = seeded_f32(n, b, session=3)
    z = execute_fft_plan(mkplan("fft_lds_fused" + sfx, n, b, tt="r2c", params=p), torch.from_numpy(r).to(gpu))
    check(z.cpu().numpy(), np.fft.rfft(r.astype(np.float64)), f"lds elems={elems} N={n} B={b} r2c")
    back = execute_fft_plan(mkplan("fft_lds_fused" + sfx, n, b, tt="c2r", td="inverse", params=p), z)
    check(back.cpu().numpy(), r.astype(np.float64), f"lds elems={elems} N={n} B={b} c2r round trip")


@pytest.mark.parametrize("n,b,stg", [(1 << 15, 600, 4), (1 << 14, 1100, 2), (1 << 15, 300, 4)])
def test_lds_start_stagger_neutral(gpu, n, b, stg):
    """The start stagger only delays workgroups: results equal the
    unstaggered kernel's bit for bit (B=600 and 1100 run it over two or more
    waves of workgroups; B=300 leaves it off)."""
    x = torch.from_numpy(seeded_c64(n, b, session=5)).to(gpu)
    y0 = execute_fft_plan(mkplan("fft_lds_fused_batch", n, b, params={"elems": 32}), x)
    y1 = execute_fft_plan(mkplan("fft_lds_fused_batch", n, b, params={"elems": 32, "stagger": stg}), x)
    assert torch.equal(y0, y1)
    rows = [0, b // 2, b - 1]
    check(y1[rows].cpu().numpy(), np.fft.fft(x[rows].cpu().numpy().astype(np.complex128)), f"stagger N={n} B={b}")
    # c2r with a 2^15-point core (the fused pre-twiddle mode)
    if n == 1 << 15 and b == 600:
        h = torch.from_numpy(seeded_c64(n + 1, b, session=6)).to(gpu)  # n + 1 bins of a 2n-point c2r
        r0 = execute_fft_plan(mkplan("fft_lds_fused_batch", 2 * n, b, tt="c2r", td="inverse",
                                     params={"elems": 32}), h)
        r1 = execute_fft_plan(mkplan("fft_lds_fused_batch", 2 * n, b, tt="c2r", td="inverse",
                                     params={"elems": 32, "stagger": stg}), h)
        assert torch.equal(r0, r1)


@pytest.mark.parametrize("n,n1", [(256, 16), (512, 32), (1 << 12, 16), (1 << 12, 256), (1 << 16, 64),
                                  (1 << 16, 1024), (1 << 20, 1024), (1 << 14, 512)])
@pytest.mark.parametrize("chunk", [0, 2])
def test_four_step_split_and_chunk_neutral(gpu, n, n1, chunk):
    b = 3 if n <= (1 << 16) else 2
    x = seeded_c64(n, b, session=2)
    y = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params={"n1": n1, "chunk_rows": chunk}),
                         torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np.fft.fft(x.astype(np.complex128)), f"four-step N={n} n1={n1} chunk={chunk}")


@pytest.mark.parametrize("tt", ["r2c", "c2r"])
@pytest.mark.parametrize("n,n1,b,chunk", [(1 << 12, 32, 5, 2), (1 << 17, 256, 7, 3), (1 << 20, 1024, 3, 1)])
@pytest.mark.parametrize("sched", [0, 1])
def test_real_four_step_chunk_interleaved(gpu, tt, n, n1, b, chunk, sched):
    """A real transform over a chunked four-step core runs chunk by chunk,
    the last chunk ragged: with schedule 0 the stitch (r2c) or pre-twiddle
    (c2r) is inside the two passes (two launches per chunk); with the
    persistent schedule it is a separate launch between the core's chunks
    (three per chunk).  Every row takes the same arithmetic as without
    chunks, so the results are bit-identical."""
    td = "forward" if tt == "r2c" else "inverse"
    rng = np.random.default_rng(7100 + n + b)
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
        ref = np.fft.rfft(h.astype(np.float64), norm="ortho")
        out = lambda: torch.empty((b, n // 2 + 1), dtype=torch.complex64, device=gpu)
    else:
        m = n // 2 + 1
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
        ref = np.fft.irfft(h.astype(np.complex128), n=n, norm="ortho")
        out = lambda: torch.empty((b, n), dtype=torch.float32, device=gpu)
    x = torch.from_numpy(h).to(gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    ys = []
    for ch in (0, chunk):
        p = native.NativePlan(n, b, tt, td, "ortho", native.FLOW_FOUR_STEP, (n1, ch, sched))
        chunks = -(-b // ch) if ch else 1
        assert p.info.launches == (2 if sched == 0 else 3) * chunks
        y = out()
        ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=gpu)
        p.execute_ws(x.data_ptr(), y.data_ptr(), ws.data_ptr(), p.ws_bytes, st)
        ys.append(y)
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1])
    check(ys[1].cpu().numpy(), ref, f"{tt} four-step N={n} n1={n1} B={b} chunk={chunk}")


@pytest.mark.parametrize("n,n1", [(1 << 12, 64), (1 << 16, 256), (1 << 18, 512), (1 << 20, 1024)])
@pytest.mark.parametrize("chunk,sched", [(0, 0), (2, 0), (0, 1), (3, 1)])
def test_four_step_reverse_pass2_order(gpu, n, n1, chunk, sched):
    """pass2_order 1 (pass 2 walks the batch rows last-written first) only
    reorders whole rows between workgroups: results equal the forward
    order's bit for bit, chunked or not, per-group or persistent."""
    b = 7 if n <= (1 << 16) else 3
    x = torch.from_numpy(seeded_c64(n, b, session=7)).to(gpu)
    base = {"n1": n1, "chunk_rows": chunk, "schedule": sched}
    y0 = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params=base), x)
    y1 = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params={**base, "pass2_order": 1}), x)
    assert torch.equal(y0, y1)
    check(y1.cpu().numpy(), np.fft.fft(x.cpu().numpy().astype(np.complex128)), f"reverse N={n} chunk={chunk}")
    yi = execute_fft_plan(mkplan("fft_four_step_batch", n, b, td="inverse", norm="ortho",
                                 params={**base, "pass2_order": 1}), x)
    check(yi.cpu().numpy(), np_ref(x.cpu().numpy(), "inverse", "ortho"), f"reverse inverse N={n}")


@pytest.mark.parametrize("n,n1", [(256, 16), (1 << 10, 32), (1 << 12, 64), (1 << 14, 128), (1 << 15, 128),
                                  (1 << 15, 256), (1 << 16, 256), (1 << 17, 256), (1 << 17, 512),
                                  (1 << 18, 512), (1 << 19, 512), (1 << 19, 1024), (1 << 20, 1024)])
@pytest.mark.parametrize("b,chunk", [(5, 0), (7, 3), (1, 0)])
def test_four_step_persistent(gpu, n, n1, b, chunk):
    """Schedule 1: persistent workgroups walk the column groups with a grid
    stride and prefetch the next group; batches and chunks whose group count
    is not a multiple of the grid leave some workgroups one group short."""
    if n >= (1 << 19):
        b = min(b, 3)
    x = seeded_c64(n, b, session=4)
    td = "inverse" if chunk == 3 else "forward"
    norm = "ortho" if chunk == 3 else "backward"
    plan = mkplan("fft_four_step_batch", n, b, td=td, norm=norm,
                  params={"n1": n1, "chunk_rows": chunk, "schedule": 1})
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np_ref(x, td, norm), f"persistent four-step N={n} n1={n1} B={b} chunk={chunk} {td}")


@pytest.mark.parametrize("n,n1", [(256, 16), (1 << 10, 32), (1 << 10, 64), (1 << 12, 64), (1 << 14, 128),
                                  (1 << 15, 256), (1 << 16, 256), (1 << 17, 256), (1 << 17, 512),
                                  (1 << 18, 512), (1 << 19, 512), (1 << 19, 1024), (1 << 20, 1024)])
@pytest.mark.parametrize("b,chunk,rev", [(1, 0, 0), (5, 0, 1), (7, 3, 0), (64, 0, 0)])
def test_four_step_narrow(gpu, n, n1, b, chunk, rev):
    """Schedule 3: 4-column groups with at most 16 elements per thread (the
    pass tables built for that), over ragged and chunked batches, both row
    orders of pass 2, both directions."""
    if n >= (1 << 18):
        b = min(b, 3)
    x = seeded_c64(n, b, session=5)
    td = "inverse" if rev else "forward"
    norm = "ortho" if chunk == 3 else "backward"
    plan = mkplan("fft_four_step_batch" if b > 1 else "fft_four_step", n, b, td=td, norm=norm,
                  params={"n1": n1, "chunk_rows": chunk, "schedule": 3, "pass2_order": rev})
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np_ref(x, td, norm), f"narrow four-step N={n} n1={n1} B={b} chunk={chunk} rev={rev} {td}")


@pytest.mark.parametrize("tt", ["r2c", "c2r"])
@pytest.mark.parametrize("n,b,chunk", [(1 << 17, 1, 0), (1 << 20, 2, 0), (1 << 18, 5, 2), (4096, 3, 0)])
def test_four_step_narrow_real(gpu, tt, n, b, chunk):
    """Schedule 3 under a real transform: the half-length core on the narrow
    passes, the stitch / pre-twiddle as its own launch (chunk by chunk when
    chunked)."""
    plan = mkplan("fft_four_step_batch" if b > 1 else "fft_four_step", n, b, tt=tt,
                  td="inverse" if tt == "c2r" else "forward", params={"chunk_rows": chunk, "schedule": 3})
    if tt == "r2c":
        r = seeded_f32(n, b, session=6)
        y = execute_fft_plan(plan, torch.from_numpy(r).to(gpu)).cpu().numpy()
        check(y, np.fft.rfft(r.astype(np.float64)), f"narrow r2c N={n} B={b} chunk={chunk}")
    else:
        rng = np.random.default_rng(n + b)
        h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
        h = h[0] if b == 1 else h
        y = execute_fft_plan(plan, torch.from_numpy(h).to(gpu)).cpu().numpy()
        check(y, np.fft.irfft(h.astype(np.complex128), n=n), f"narrow c2r N={n} B={b} chunk={chunk}")


FUSED_SPLITS = [(1 << 14, 128), (1 << 15, 128), (1 << 15, 256), (1 << 16, 256), (1 << 17, 256),
                (1 << 17, 512), (1 << 18, 512)]


@pytest.mark.parametrize("n,n1", FUSED_SPLITS)
@pytest.mark.parametrize("b,chunk", [(1, 0), (5, 0), (13, 0), (19, 4), (64, 0)])
def test_four_step_fused(gpu, n, n1, b, chunk):
    """Schedule 2: both passes in one launch, each transform's pass 2 waiting
    for its pass-1 groups on the same XCD.  Batches below 8 leave XCDs with
    no transform; 13 and 19 rows give the XCDs unequal shares; chunks re-run
    the launch with its counters cleared.  No pass-2 wait may give up."""
    if n >= (1 << 18):
        b = min(b, 19)
    x = seeded_c64(n, b, session=6)
    td = "inverse" if chunk else "forward"
    norm = "forward" if chunk else "backward"
    plan = mkplan("fft_four_step_batch", n, b, td=td, norm=norm,
                  params={"n1": n1, "chunk_rows": chunk, "schedule": 2})
    xd = torch.from_numpy(x).to(gpu)
    y = execute_fft_plan(plan, xd).cpu().numpy()
    check(y, np_ref(x, td, norm), f"fused four-step N={n} n1={n1} B={b} chunk={chunk} {td}")
    y2 = execute_fft_plan(plan, xd).cpu().numpy()  # second launch on the same counters
    np.testing.assert_array_equal(y2, y)
    nplan, _ = _resolve(plan, 0)
    assert nplan.sync_overruns() == 0


@pytest.mark.parametrize("lag,take,ring,bpc", [(1, 1, 0, 0), (1, 8, 0, 0), (3, 2, 0, 0), (12, 4, 0, 0),
                                                (63, 64, 0, 0), (1, 1, 2, 1), (2, 2, 6, 2), (3, 1, 4, 3),
                                                (1, 2, 2, 0), (4, 2, 9, 1)])
def test_four_step_fused_queue_settings(gpu, lag, take, ring, bpc):
    """The fused schedule's queue lag (params[3] bits 0-7), items per dequeue
    (bits 8-15), Z slots per XCD (bits 16-23, at least lag + 1) and blocks
    per CU (bits 24-30) only reorder work and move Z: results are bitwise the
    same as the default settings, including lags beyond the transforms of a
    slot and rings as small as lag + 1 (pass 1 then waits for its slot)."""
    n, b = 1 << 16, 21
    x = torch.from_numpy(seeded_c64(n, b, session=7)).to(gpu)
    ref = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params={"n1": 256, "schedule": 2}), x)
    word = lag | (take << 8) | (ring << 16) | (bpc << 24)
    p = native.NativePlan(n, b, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2, word))
    y = torch.empty_like(x)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y, ref) and p.sync_overruns() == 0


def test_four_step_schedules_agree(gpu):
    """All three schedules run the same butterflies and twiddles (only the
    compiler's instruction choices may differ): outputs agree to 1e-6."""
    n, b = 1 << 18, 40
    x = torch.from_numpy(seeded_c64(n, b, session=5)).to(gpu)
    y0 = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params={"n1": 512}), x)
    for sched in (1, 2):
        y1 = execute_fft_plan(mkplan("fft_four_step_batch", n, b, params={"n1": 512, "schedule": sched}), x)
        d = (torch.linalg.vector_norm(y1 - y0) / torch.linalg.vector_norm(y0)).item()
        assert d <= 1e-6, f"schedule {sched} differs: rel L2 {d:.3e}"


@pytest.mark.parametrize("sched", [1, 2])
def test_four_step_schedule_real(gpu, sched):
    n, b = 1 << 17, 6
    xr = seeded_f32(n, b)
    p = {"n1": 256, "chunk_rows": 4, "schedule": sched}
    X = execute_fft_plan(mkplan("fft_four_step_batch", n, b, tt="r2c", params=p), torch.from_numpy(xr).to(gpu))
    check(X.cpu().numpy(), oracle.r2c_dedicated(xr), f"schedule {sched} r2c")
    y = execute_fft_plan(mkplan("fft_four_step_batch", n, b, tt="c2r", td="inverse", params=p), X).cpu().numpy()
    check(y, xr.astype(np.float64), f"schedule {sched} r2c->c2r round trip")


def test_four_step_fused_range(gpu):
    """The fused schedule takes n1, n2 in [128, 512] within a factor 2; plan
    creation rejects other splits (no launch)."""
    with pytest.raises(ValueError, match="fused"):
        native.NativePlan(1 << 20, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (1024, 0, 2))
    with pytest.raises(ValueError, match="fused"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (128, 0, 2))
    p = native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2))
    assert p.info.n1 == 256 and p.info.launches == 2 and p.sync_overruns() == 0
    with pytest.raises(ValueError, match="schedule"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 4))
    with pytest.raises(ValueError, match="lag"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2, 65))
    with pytest.raises(ValueError, match="dequeue"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2, 65 << 8))
    # a ring smaller than lag + 1, or beyond 64 slots; more than 16 blocks per CU
    with pytest.raises(ValueError, match="Z slots"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP,
                          (256, 0, 2, 3 | (3 << 16)))
    with pytest.raises(ValueError, match="Z slots"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2, 65 << 16))
    with pytest.raises(ValueError, match="blocks per CU"):
        native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP, (256, 0, 2, 17 << 24))
    # the ring lives in the workspace: num_xcc x slots x N complex values
    q = native.NativePlan(1 << 16, 2, "c2c", "forward", "backward", native.FLOW_FOUR_STEP,
                          (256, 0, 2, 1 | (5 << 16)), caller_workspace=True)
    assert q.workspace_size() >= 8 * 5 * (1 << 16) * 8


# ---------------------------------------------------------------- real flows
REAL_CASES = [("fft_lds_fused", n) for n in (2, 4, 8, 64, 256, 4096, 8192, 16384, 32768, 65536)]
REAL_CASES += [("fft_four_step", n) for n in (512, 1 << 15, 1 << 20)]
REAL_CASES += [("fft_dit", n) for n in (4, 256, 4096)] + [("fft_dif_radix4", n) for n in (8, 256)]


@pytest.mark.parametrize("name,n", REAL_CASES)
@pytest.mark.parametrize("norm", ["backward", "ortho", "forward", "none"])
def test_r2c_c2r_match_oracle(gpu, name, n, norm):
    b = 4 if n <= (1 << 15) else 1
    xr = seeded_f32(n, b)
    bname = name + ("_batch" if b > 1 else "")
    X = execute_fft_plan(mkplan(bname, n, b, tt="r2c", norm=norm), torch.from_numpy(xr).to(gpu))
    check(X.cpu().numpy(), oracle.r2c_dedicated(xr, norm), f"r2c {name} N={n} {norm}")
    Xh = np.ascontiguousarray(oracle.r2c_dedicated(xr, "backward").astype(np.complex64))
    y = execute_fft_plan(mkplan(bname, n, b, tt="c2r", td="inverse", norm=norm),
                         torch.from_numpy(Xh).to(gpu)).cpu().numpy()
    check(y, oracle.c2r_dedicated(Xh, n, norm), f"c2r {name} N={n} {norm}")


@pytest.mark.parametrize("elems,n", [(e, n) for e in (4, 8, 16) for n in (16, 64, 512, 2048, 8192)] + [(8, 1024)]
                         + [(16, 1 << 14), (16, 1 << 15), (32, 1 << 12), (32, 1 << 15), (32, 1 << 16)])
@pytest.mark.parametrize("b", [1, 3, 37])
def test_c2r_mirror_pairs(gpu, elems, n, b):
    """Fused C2R: each bin is loaded once and meets its mirror bin n/2 - k
    from the partner lane (8, 16 or 32 elements per thread and whole waves per
    transform) or through LDS (the other forms), bin 0
    pairs with bin n/2, and the DC/Nyquist imaginary parts are ignored.
    Ragged batches leave rows of a multi-transform block inactive."""
    rng = np.random.default_rng(4000 + n + b + elems)
    m = n // 2 + 1
    h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
    ref = np.fft.irfft(h.astype(np.complex128), n=n)  # ignores the DC and Nyquist imaginary parts
    p = mkplan("fft_lds_fused" + ("_batch" if b > 1 else ""), n, b, tt="c2r", td="inverse",
               params={"elems": elems})
    y = execute_fft_plan(p, torch.from_numpy(h if b > 1 else h[0]).to(gpu)).cpu().numpy()
    check(y.reshape(b, n), ref, f"c2r elems={elems} N={n} B={b}")


@pytest.mark.parametrize("n", [1 << k for k in range(11, 17)])
@pytest.mark.parametrize("b", [1, 5, 11])
def test_r2c_32_elements_stitch_through_output(gpu, n, b):
    """R2C with 32 elements per thread (the split exchange).  From a
    2048-point core the remainder radix runs first, so the last pass has the
    full radix 32 and the stitch runs in registers, each bin's mirror coming
    from the partner lane; the 1024-point core (32 lanes per transform, two
    transforms per wave) sends its outputs to the output row, then each
    thread turns disjoint mirror pairs into bins in place.  Ragged batches
    leave rows of a multi-transform block inactive."""
    rng = np.random.default_rng(6000 + n + b)
    h = rng.standard_normal((b, n)).astype(np.float32)
    p = native.NativePlan(n, b, "r2c", "forward", "ortho", native.FLOW_LDS_FUSED, (32,))
    x = torch.from_numpy(h).to(gpu)
    y = torch.full((b, n // 2 + 1), float("nan"), dtype=torch.complex64, device=gpu)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    check(y.cpu().numpy(), np.fft.rfft(h.astype(np.float64), norm="ortho"), f"r2c e32 N={n} B={b}")


@pytest.mark.parametrize("n", [1 << k for k in range(11, 17)])
@pytest.mark.parametrize("b", [1, 5, 11])
def test_c2r_32_elements_lane_pairs(gpu, n, b):
    """C2R with 32 elements per thread through the C ABI (the Python runner
    maps 32 to 16 below a 32768-point core).  From a 2048-point core each
    wave holds the indices j and T - j in lanes l and l ^ 32, so every bin is
    loaded once and its mirror comes from the partner lane (bin 0 pairs with
    bin n/2, loaded by the j = 0 lane; j = T/2 and j = 0 pair with
    themselves); the 1024-point core (one transform per 32 lanes) loads both
    bins.  The DC and Nyquist imaginary parts are nonzero and ignored."""
    rng = np.random.default_rng(6500 + n + b)
    m = n // 2 + 1
    h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
    p = native.NativePlan(n, b, "c2r", "inverse", "backward", native.FLOW_LDS_FUSED, (32,))
    x = torch.from_numpy(h).to(gpu)
    y = torch.full((b, n), float("nan"), dtype=torch.float32, device=gpu)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    check(y.cpu().numpy(), np.fft.irfft(h.astype(np.complex128), n=n), f"c2r e32 N={n} B={b}")


@pytest.mark.parametrize("name", ["fft_lds_fused", "fft_four_step", "fft_dit"])
def test_c2r_ignores_dc_nyquist_imag(gpu, golden, name):
    n = 256
    h = golden[f"irfft_in_{n}"].astype(np.complex64)
    if name == "fft_four_step":
        n2 = 1024
        rng = np.random.default_rng(1)
        h = (rng.standard_normal(n2 // 2 + 1) + 1j * rng.standard_normal(n2 // 2 + 1)).astype(np.complex64)
        ref = np.fft.irfft(h.astype(np.complex128), n=n2)
        n = n2
    else:
        ref = golden[f"irfft_out_{n}"]
    y = execute_fft_plan(mkplan(name, n, 1, tt="c2r", td="inverse"), torch.from_numpy(h).to(gpu)).cpu().numpy()
    check(y, ref, f"c2r DC/Nyquist {name}")


# ------------------------------------ the reference's benchmark configurations
def test_config1_n2048_b1(gpu, golden):
    x = golden["c1_in"]
    plan = plan_fft("dit", 2048, profile_hash=DeviceProfile.load().hash())
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, golden["c1_out"], f"C1 via {plan.executed}")
    check(y, oracle.fft_dit(x), "C1 vs C oracle")
    if oracle.reference_lib() is not None:
        check(y, oracle.reference_fft(x), "C1 vs reference build")


@pytest.mark.parametrize("n", [1024, 2048])
@pytest.mark.parametrize("b", [16, 64])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_config2_batched(gpu, n, b, direction):
    x = seeded_c64(n, b)
    plan = plan_fft(direction, n, batch=b, profile_hash=DeviceProfile.load().hash())
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.fft_dit(x), f"C2 N={n} B={b} via {plan.executed}")
    y2 = execute_fft_plan(mkplan("fft_lds_fused_batch", n, b), torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y2, oracle.fft_dit(x), f"C2 LDS N={n} B={b}")


@pytest.mark.parametrize("n", [256, 4096])
@pytest.mark.parametrize("b", [1, 64])
@pytest.mark.parametrize("norm", ["none", "forward", "backward", "ortho"])
def test_config3_inverse_and_real_round_trip(gpu, n, b, norm):
    prof = DeviceProfile.load().hash()
    x = seeded_c64(n, b)
    inv = plan_fft("dit", n, batch=b, profile_hash=prof, transform_direction="inverse", norm=norm)
    y = execute_fft_plan(inv, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np_ref(x, "inverse", norm), f"C3 inverse N={n} B={b} {norm}")
    xr = seeded_f32(n, b)
    r2c = plan_fft("dit", n, batch=b, profile_hash=prof, transform_type="r2c", norm=norm)
    c2r = plan_fft("dit", n, batch=b, profile_hash=prof, transform_type="c2r", norm=norm)
    X = execute_fft_plan(r2c, torch.from_numpy(xr).to(gpu))
    npn = "backward" if norm == "none" else norm
    check(X.cpu().numpy(), np.fft.rfft(xr.astype(np.float64), norm=npn), f"C3 r2c N={n} B={b} {norm}")
    back = execute_fft_plan(c2r, X).cpu().numpy()
    # c2r(r2c(x)) = x * (fwd scale * inv scale * n)
    k = {"none": n, "forward": 1.0, "backward": 1.0, "ortho": 1.0}[norm]
    check(back, xr.astype(np.float64) * k, f"C3 round trip N={n} B={b} {norm}")


def test_config4_n2p20_b1(gpu):
    n = 1 << 20
    x = seeded_c64(n, 1)
    plan = plan_fft("dit", n, profile_hash=DeviceProfile.load().hash())
    xd = torch.from_numpy(x).to(gpu)
    y = execute_fft_plan(plan, xd)
    check(y.cpu().numpy(), oracle.fft_dit(x), f"C4 N=2^20 via {plan.executed}")
    inv = plan_fft("dit", n, profile_hash=DeviceProfile.load().hash(), transform_direction="inverse")
    back = execute_fft_plan(inv, y).cpu().numpy()
    check(back, x.astype(np.complex128), "C4 round trip")


def test_config4_n2p16_b256(gpu):
    n, b = 1 << 16, 256
    x = seeded_c64(n, b)
    plan = plan_fft("dit", n, batch=b, profile_hash=DeviceProfile.load().hash())
    xd = torch.from_numpy(x).to(gpu)
    y = execute_fft_plan(plan, xd).cpu().numpy()
    check(y[:4], oracle.fft_dit(x[:4]), f"C4 N=2^16 B=256 rows 0-3 vs C oracle ({plan.executed})")
    check(y, np.fft.fft(x.astype(np.complex128)), "C4 N=2^16 B=256 vs numpy")
    # Parseval per row: sum |X|^2 = N * sum |x|^2
    ex = (np.abs(x.astype(np.complex128)) ** 2).sum(axis=1) * n
    ey = (np.abs(y.astype(np.complex128)) ** 2).sum(axis=1)
    assert np.abs(ey / ex - 1).max() < 1e-5


@pytest.mark.parametrize("n", [1 << k for k in range(4, 15)])
@pytest.mark.parametrize("b", [1, 16, 64, 256])
def test_config5_selector_and_m0_cells(gpu, n, b):
    """All 44 cells of the selector sweep: the selected plan and the M0
    incumbent (fft_dit / fft_dit_batch) against the C oracle (numpy for the
    cells above 2^20 points)."""
    prof = DeviceProfile.load().hash()
    x = seeded_c64(n, b)
    xd = torch.from_numpy(x).to(gpu)
    ref = oracle.fft_dit(x) if n * b <= (1 << 20) else np.fft.fft(x.astype(np.complex128))
    plan = plan_fft("dit", n, batch=b, profile_hash=prof)
    check(execute_fft_plan(plan, xd).cpu().numpy(), ref, f"C5 N={n} B={b} selector ({plan.executed})")
    m0 = mkplan("fft_dit" if b == 1 else "fft_dit_batch", n, b)
    check(execute_fft_plan(m0, xd).cpu().numpy(), ref, f"C5 N={n} B={b} M0")


@pytest.mark.parametrize("n", [16, 256, 4096, 16384])
@pytest.mark.parametrize("b", [1, 64])
@pytest.mark.parametrize("tt,td,norm", [("c2c", "inverse", "ortho"), ("r2c", "forward", "forward"),
                                        ("c2r", "inverse", "none")])
def test_config5_cells_other_semantics(gpu, n, b, tt, td, norm):
    """The C2C entries of the config-5 sweep also answer the other
    semantics (legacy entries carry no semantic triple): the selected plan
    runs inverse, R2C and C2R with any norm on the cell's shape."""
    prof = DeviceProfile.load().hash()
    plan = plan_fft("dit", n, batch=b, profile_hash=prof, transform_type=tt, transform_direction=td, norm=norm)
    assert not plan.fallback
    rng = np.random.default_rng(8000 + n + b)
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
        ref = np.fft.rfft(h.astype(np.float64), norm=norm)
    elif tt == "c2r":
        h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
        ref = np.fft.irfft(h.astype(np.complex128), n=n, norm="forward")  # "none" on the inverse: no 1/N
    else:
        h = seeded_c64(n, b, session=11).reshape(b, n)
        ref = np_ref(h, td, norm)
    y = execute_fft_plan(plan, torch.from_numpy(h if b > 1 else h[0]).to(gpu)).cpu().numpy()
    check(y.reshape(ref.shape), ref, f"C5 {tt} {td} {norm} N={n} B={b} ({plan.executed})")


def _real_entries():
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "..", "kunlunxin-fft_amd", "config", "selector_table.json")
    t = json.load(open(path))
    return [(e["N"], e["batch"], e["transform_type"], e["transform_direction"], e["executed"])
            for e in t["entries"] if "transform_type" in e]


@pytest.mark.parametrize("n,b,tt,td,executed", _real_entries())
def test_selector_real_entries(gpu, n, b, tt, td, executed):
    """The exact-semantic R2C / C2R entries of the shipped table: plan_fft
    resolves them (not the C2C entry of the same cell), and the selected
    plan is correct on the first, a middle and the last row."""
    plan = plan_fft("dit", n, batch=b, profile_hash=DeviceProfile.load().hash(), transform_type=tt,
                    transform_direction=td)
    assert plan.executed == executed and plan.transform_type == tt and not plan.fallback
    rng = np.random.default_rng(5000 + n)
    if tt == "r2c":
        x = torch.randn((b, n), dtype=torch.float32, device=gpu, generator=torch.Generator(gpu).manual_seed(n))
    else:
        x = torch.randn((b, n // 2 + 1), dtype=torch.complex64, device=gpu,
                        generator=torch.Generator(gpu).manual_seed(n))
    y = execute_fft_plan(plan, x if b > 1 else x[0]).reshape(b, -1)
    rows = sorted({0, int(rng.integers(0, b)), b - 1})
    h = x[rows].cpu().numpy()
    ref = np.fft.rfft(h.astype(np.float64)) if tt == "r2c" else np.fft.irfft(h.astype(np.complex128), n=n)
    check(y[rows].cpu().numpy(), ref, f"selector {tt} N={n} B={b} ({executed})")
    del x, y


# --------------------------------------------------------- properties, KATs
@pytest.mark.parametrize("name", ["fft_lds_fused", "fft_four_step", "fft_dit_radix4"])
def test_linearity(gpu, name):
    n, b = 4096, 4
    a = seeded_c64(n, b)
    c = seeded_c64(n, b, session=3)
    alpha = 0.75 - 0.25j
    mix = (alpha * a.astype(np.complex128) + c).astype(np.complex64)
    p = mkplan(name + "_batch", n, b)
    run_ = lambda h: execute_fft_plan(p, torch.from_numpy(h).to(gpu)).cpu().numpy().astype(np.complex128)
    check(run_(mix), alpha * run_(a) + run_(c), f"linearity {name}")


@pytest.mark.parametrize("n", [1 << k for k in range(10, 21)])
def test_roofline_rows_full_size(gpu, n):
    """The bench's rows at full size (B = max(64, 2^25/N), 256 MiB in and out
    per N) through the selected plans: sampled rows against numpy float64,
    the forward -> inverse round trip and Parseval's identity over the whole
    batch (both size-independent)."""
    b = max(64, (1 << 25) // n)
    prof = DeviceProfile.load().hash()
    g = torch.Generator(gpu).manual_seed(n)
    x = torch.randn((b, n), dtype=torch.complex64, device=gpu, generator=g)
    fwd = plan_fft("dit", n, batch=b, profile_hash=prof)
    inv = plan_fft("dit", n, batch=b, profile_hash=prof, transform_direction="inverse")
    assert not fwd.fallback and not inv.fallback
    y = execute_fft_plan(fwd, x)
    rows = [0, b // 2 + 1, b - 1]
    check(y[rows].cpu().numpy(), np.fft.fft(x[rows].cpu().numpy().astype(np.complex128)),
          f"full-size N={n} B={b} ({fwd.executed})")
    # Parseval: sum |Y|^2 = N sum |x|^2 (float64 sums on the device)
    ex = torch.sum(torch.abs(x.to(torch.complex128)) ** 2).item()
    ey = torch.sum(torch.abs(y.to(torch.complex128)) ** 2).item()
    assert abs(ey / (n * ex) - 1.0) <= 1e-5, f"Parseval N={n}: {ey / (n * ex) - 1.0:.3e}"
    z = execute_fft_plan(inv, y)  # backward norm: the inverse carries 1/N
    d = (torch.linalg.vector_norm((z - x).to(torch.complex128)) /
         torch.linalg.vector_norm(x.to(torch.complex128))).item()
    assert d <= 1e-5, f"round trip N={n}: rel L2 {d:.3e}"


def test_known_signals(gpu, golden):
    for name in ("fft_dit", "fft_lds_fused", "fft_four_step"):
        for kin, kout in (("impulse256_in", "impulse256_out"), ("tone256_in", "tone256_out")):
            x = golden[kin].astype(np.complex64)
            y = execute_fft_plan(mkplan(name, 256, 1), torch.from_numpy(x).to(gpu)).cpu().numpy()
            assert np.abs(y - golden[kout]).max() < 1e-4, (name, kin)
        s = golden["sentinel1024_in"].astype(np.complex64)
        y = execute_fft_plan(mkplan(name, 1024, 1), torch.from_numpy(s).to(gpu)).cpu().numpy()
        dc = golden["sentinel1024_dc"][0]
        assert abs(y[0] - dc) < 1e-2 * abs(dc) and np.isfinite(y).all() and not np.array_equal(y, s)


@pytest.mark.parametrize("n", [8, 16, 64, 256, 1024, 4096])
def test_fft_check_kat(gpu, golden, n):
    x = golden[f"kat_in_{n}"].astype(np.complex64)
    for name in ("fft_dit", "fft_dif", "fft_dit_radix4", "fft_dif_radix4", "fft_lds_fused"):
        y = execute_fft_plan(mkplan(name, n, 1), torch.from_numpy(x).to(gpu)).cpu().numpy()
        check(y, golden[f"kat_out_{n}"], f"KAT {name} N={n}")


def test_bit_reverse_permute(gpu, golden):
    n = 64
    x = torch.complex(torch.arange(n, dtype=torch.float32), torch.arange(n, dtype=torch.float32) * 0.5).to(gpu)
    y = bit_reverse_permute(x).cpu()
    expect = [oracle.bit_reverse(i, 6) for i in range(n)]
    assert torch.equal(y.real.to(torch.int64)[expect], x.real.cpu().to(torch.int64))
    x8 = torch.arange(8, dtype=torch.float32).to(torch.complex64).to(gpu)
    y8 = bit_reverse_permute(x8).cpu().real.to(torch.int64).tolist()
    assert [y8.index(i) for i in range(8)] == list(golden["bitrev8"])


@pytest.mark.parametrize("nbytes", [16, 4096, 32768, 32768 + 48, (64 << 20) + 16 * 777])
def test_stream_copy_is_exact(gpu, nbytes):
    """The bench's streaming copy moves every byte, including a tail shorter
    than one 32 KiB block, and writes nothing past the end."""
    from kunlunxin_fft_amd import native

    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=gpu)
    dst = torch.full((nbytes + 4096,), 7, dtype=torch.uint8, device=gpu)
    native.stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize(gpu)
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 7).all())


def test_reexecution_is_bitwise_stable_and_one_shot_matches(gpu):
    prof = DeviceProfile.load().hash()
    for n, b in ((128, 1), (2048, 16), (1 << 16, 2)):
        x = torch.from_numpy(seeded_c64(n, b)).to(gpu)
        plan = plan_fft("dit", n, batch=b, profile_hash=prof)
        y1 = execute_fft_plan(plan, x)
        y2 = execute_fft_plan(plan, x)
        assert torch.equal(y1, y2)
        y3, rep = run_fft(x, "dit", profile_hash=prof)
        assert torch.equal(y1, y3) and rep.executed == plan.executed


def test_run_fft_squeezes_and_infers_c2r_length(gpu):
    x = torch.from_numpy(seeded_c64(256, 1)).to(gpu).unsqueeze(0)
    y, rep = run_fft(x, "dit")
    assert y.shape == (1, 256) and rep.batch == 1
    h = torch.from_numpy(oracle.r2c_dedicated(seeded_f32(256, 1)).astype(np.complex64)).to(gpu)
    r, rep = run_fft(h, "dit", transform_type="c2r")
    assert r.shape == (256,) and rep.n == 256 and r.dtype == torch.float32


def test_input_validation_raises_before_launch(gpu):
    p = mkplan("fft_lds_fused", 16, 1)
    good = torch.ones(16, dtype=torch.complex64, device=gpu)
    with pytest.raises(TypeError):
        execute_fft_plan(p, good.real.contiguous())
    with pytest.raises(ValueError):
        execute_fft_plan(p, good.reshape(4, 4))
    with pytest.raises(ValueError):
        execute_fft_plan(p, torch.ones(32, dtype=torch.complex64, device=gpu)[::2])
    with pytest.raises(ValueError):
        execute_fft_plan(p, torch.ones(16, dtype=torch.complex64))
    with pytest.raises(TypeError):
        execute_fft_plan(p, np.ones(16, np.complex64))
    from kunlunxin_fft_amd.runner import fft_dit

    with pytest.raises(ValueError):
        fft_dit(torch.ones(12, dtype=torch.complex64, device=gpu))


@pytest.mark.parametrize("tt", ["r2c", "c2r"])
def test_real_m0_for_a_huge_odd_batch_of_short_rows(gpu, tt):
    """M0 (the closed fallback) on real rows: its stitch / pre-twiddle runs
    one thread per mirror pair over the flat batch, so N = 16 at
    B = 3 * 2^23 + 1 (past 2^24 rows, where a block per row would need more
    than one dispatch's 2^32 work-items) plans and matches numpy on the
    first, a middle and the last rows."""
    n, b = 16, 3 * (1 << 23) + 1
    td = "inverse" if tt == "c2r" else "forward"
    plan = mkplan("fft_dit_batch", n, b, tt=tt, td=td)
    print(f"huge odd batch {tt}: N={n} B={b}", flush=True)
    g = torch.Generator(gpu).manual_seed(11)
    if tt == "r2c":
        x = torch.randn((b, n), dtype=torch.float32, device=gpu, generator=g)
    else:
        x = torch.randn((b, n // 2 + 1), dtype=torch.complex64, device=gpu, generator=g)
    y = execute_fft_plan(plan, x)
    rows = [0, 1, b // 2, (1 << 24) - 1, 1 << 24, b - 1]
    xs = x[rows].cpu().numpy()
    ref = np.fft.rfft(xs.astype(np.float64)) if tt == "r2c" else np.fft.irfft(xs.astype(np.complex128), n=n)
    check(y[rows].cpu().numpy(), ref, f"M0 {tt} N={n} B={b}")
    del x, y


ROUND_CASES = [(16, 3, "c2c"), (1024, 100, "c2c"), (1024, 1000, "r2c"), (4096, 100, "c2r"), (1 << 15, 5, "c2c"),
               (1 << 16, 7, "r2c"), (1 << 18, 3, "c2r"), (1 << 20, 3, "c2c"), (256, 70000, "c2c"),
               (1 << 20, 5000, "c2c")]


@pytest.mark.parametrize("n,b,tt", ROUND_CASES, ids=[f"N{n}-B{b}-{tt}" for n, b, tt in ROUND_CASES])
def test_batch_without_exact_key_runs_the_rounded_decision(gpu, n, b, tt):
    """plan_fft for a batch the table holds no key for (not a power of two,
    or past its 2^32-element grid: N = 2^20, B = 5000) takes the decision of
    the next power-of-two batch of the same N and semantic (or the largest
    one), and runs it correctly on the ragged batch: the first, a middle and
    the last rows against numpy."""
    from kunlunxin_fft_amd.selector import default_table, find_entry, rounded_batch

    td = "inverse" if tt == "c2r" else "forward"
    prof = DeviceProfile.load().hash()
    plan = plan_fft("dit", n, batch=b, transform_type=tt, transform_direction=td, profile_hash=prof)
    t = default_table()
    rb = rounded_batch(t, n, b, "dit", tt, td, "backward")
    e = find_entry(t, n, rb, "dit", tt, td, "backward")
    assert not plan.fallback and plan.selection_source == "table" and f"batch={rb}" in plan.reason, plan.reason
    assert plan.executed == e["executed"] and plan.params["table_batch"] == rb
    print(f"rounded batch: N={n} B={b} {tt} -> table batch {rb} ({plan.executed})", flush=True)
    g = torch.Generator(gpu).manual_seed(n + b)
    if tt == "r2c":
        x = torch.randn((b, n), dtype=torch.float32, device=gpu, generator=g)
    elif tt == "c2r":
        x = torch.randn((b, n // 2 + 1), dtype=torch.complex64, device=gpu, generator=g)
    else:
        x = torch.randn((b, n), dtype=torch.complex64, device=gpu, generator=g)
    y = execute_fft_plan(plan, x)
    rows = sorted({0, b // 2, b - 1})
    h = x[rows].cpu().numpy()
    if tt == "r2c":
        ref = np.fft.rfft(h.astype(np.float64))
    elif tt == "c2r":
        ref = np.fft.irfft(h.astype(np.complex128), n=n)
    else:
        ref = np.fft.fft(h.astype(np.complex128))
    check(y[rows].cpu().numpy(), ref, f"rounded N={n} B={b} {tt}")
    del x, y


def test_native_rejects_oversized_batch(gpu):
    """Plans cover at most 2^40 bytes of complex64 rows (no byte count can
    overflow), and no launch of 2^32 work-items or more (one dispatch's
    limit): at n = 1024 the LDS kernel runs 64 threads per transform, so 2^27
    rows are refused and the largest batch whose launch fits still plans."""
    for n in (1, 1024, 1 << 20):
        with pytest.raises(ValueError, match="2\\^40"):
            native.NativePlan(n, ((1 << 37) // n) + 1)
    with pytest.raises(ValueError, match="dispatch"):
        native.NativePlan(1024, (1 << 37) // 1024, flow=native.FLOW_LDS_FUSED)
    big = ((1 << 32) - 1 - 1024) // 64
    assert native.NativePlan(1024, big, flow=native.FLOW_LDS_FUSED).info.batch == big


def test_native_rejects_overlap_and_misalignment(gpu):
    np_ = native.NativePlan(64, 2, flow=native.FLOW_LDS_FUSED)
    buf = torch.zeros(4 * 64, dtype=torch.complex64, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    with pytest.raises(ValueError, match="overlap"):
        np_.execute(buf.data_ptr(), buf.data_ptr() + 8 * 64, stream)
    with pytest.raises(ValueError, match="aligned"):
        np_.execute(buf.data_ptr() + 4, buf.data_ptr() + 8 * 200, stream)
    assert np_.info.launches == 1 and np_.info.workspace_bytes == 0


def test_runs_on_a_side_stream(gpu):
    n, b = 4096, 8
    x = torch.from_numpy(seeded_c64(n, b)).to(gpu)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y = run("fft_lds_fused_batch", x, b, n)
    s.synchronize()
    check(y.cpu().numpy(), oracle.fft_dit(seeded_c64(n, b)), "side stream")


def test_plan_reuse_checks_every_call(gpu):
    """Repeat executes of one plan (the cached per-plan fast path) give the
    checked first call's result, follow the current stream, and still raise
    the reference's errors for any input that does not match the plan."""
    n, b = 2048, 4
    h = seeded_c64(n, b)
    x = torch.from_numpy(h).to(gpu)
    plan = plan_fft("dit", n, batch=b, profile_hash=DeviceProfile.load().hash())
    y0 = execute_fft_plan(plan, x).cpu().numpy()
    y1 = execute_fft_plan(plan, x).cpu().numpy()
    assert np.array_equal(y0, y1)
    check(y1, oracle.fft_dit(h), "plan reuse")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y2 = execute_fft_plan(plan, x)
    s.synchronize()
    assert np.array_equal(y2.cpu().numpy(), y0)
    with pytest.raises(ValueError, match="shape"):
        execute_fft_plan(plan, x[:2])
    with pytest.raises(TypeError):
        execute_fft_plan(plan, x.to(torch.complex128))
    with pytest.raises(ValueError, match="contiguous"):
        execute_fft_plan(plan, torch.from_numpy(np.ascontiguousarray(h.T)).to(gpu).T)
    with pytest.raises(ValueError, match="GPU"):
        execute_fft_plan(plan, torch.from_numpy(h))
    with pytest.raises(TypeError):
        execute_fft_plan(plan, h)
    assert np.array_equal(execute_fft_plan(plan, x).cpu().numpy(), y0)


def test_plan_info_reports_flows(gpu):
    assert native.NativePlan(4096, 4).flow_name == "lds-fused"
    fs = native.NativePlan(1 << 16, 4)
    assert fs.flow_name == "four-step" and fs.info.launches == 2 and fs.info.workspace_bytes == 0
    r2 = native.NativePlan(1024, 2, flow=native.FLOW_RADIX2_DIT)
    assert r2.info.launches == 10 and r2.info.workspace_bytes == 2 * 1024 * 8


# ------------------------------------------- real transforms fused into the four-step
REAL4_SPLITS = [(512, 16), (1 << 11, 32), (1 << 13, 64), (1 << 12, 16), (1 << 12, 128), (1 << 15, 16),
                (1 << 15, 1024), (1 << 15, 128),
                (1 << 17, 256), (1 << 18, 512), (1 << 19, 1024), (1 << 20, 512), (1 << 20, 1024)]


@pytest.mark.parametrize("n,n1", REAL4_SPLITS)
@pytest.mark.parametrize("b,chunk", [(1, 0), (3, 0), (5, 2)])
def test_real_four_step_fused(gpu, n, n1, b, chunk):
    """R2C with the stitch in pass 2 and C2R with the pre-twiddle in pass 1
    (schedule 0): every split of the half-length core, the smallest column
    groups (16 columns = 8 mirror pairs, pair 0 = columns 0 and n/2 of the
    grid), ragged chunks, against numpy rfft / irfft; the plan makes two
    launches per chunk and C2R takes no workspace."""
    if n >= (1 << 19):
        b, chunk = min(b, 3), min(chunk, 2)
    xr = seeded_f32(n, b, session=12)
    norm = "ortho" if chunk else "backward"
    p = {"n1": n1, "chunk_rows": chunk}
    r2c = mkplan("fft_four_step_batch" if b > 1 else "fft_four_step", n, b, tt="r2c", norm=norm, params=p)
    X = execute_fft_plan(r2c, torch.from_numpy(xr).to(gpu))
    check(X.cpu().numpy(), np.fft.rfft(xr.astype(np.float64), norm=norm), f"fused r2c N={n} n1={n1} B={b} c={chunk}")
    c2r = mkplan("fft_four_step_batch" if b > 1 else "fft_four_step", n, b, tt="c2r", td="inverse", norm=norm,
                 params=p)
    h = X.cpu().numpy().astype(np.complex128)
    y = execute_fft_plan(c2r, X).cpu().numpy()
    check(y, np.fft.irfft(h, n=n, norm=norm), f"fused c2r N={n} n1={n1} B={b} c={chunk}")
    nr, _ = _resolve(r2c, 0)
    nc, _ = _resolve(c2r, 0)
    chunks = -(-b // chunk) if chunk else 1
    assert nr.info.launches == 2 * chunks and nc.info.launches == 2 * chunks
    assert nc.ws_bytes == 0 and nr.ws_bytes == 8 * (n // 2) * b


@pytest.mark.parametrize("n,n1", [(1 << 12, 64), (1 << 17, 256)])
def test_real_four_step_fused_hermitian_edges(gpu, n, n1):
    """C2R ignores the imaginary parts of bins 0 and n/2 (fused pre-twiddle
    path), and special inputs (impulse, constant) stay exact."""
    b = 2
    rng = np.random.default_rng(99)
    h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
    c2r = mkplan("fft_four_step_batch", n, b, tt="c2r", td="inverse", params={"n1": n1})
    y = execute_fft_plan(c2r, torch.from_numpy(h).to(gpu)).cpu().numpy()
    h2 = h.copy()
    h2[:, 0] = h2[:, 0].real
    h2[:, -1] = h2[:, -1].real
    check(y, np.fft.irfft(h2.astype(np.complex128), n=n), f"fused c2r edges N={n}")
    r2c = mkplan("fft_four_step_batch", n, b, tt="r2c", params={"n1": n1})
    imp = np.zeros((b, n), np.float32)
    imp[:, 0] = 1.0
    X = execute_fft_plan(r2c, torch.from_numpy(imp).to(gpu)).cpu().numpy()
    np.testing.assert_allclose(X, np.ones((b, n // 2 + 1)), atol=1e-6)
    const = np.full((b, n), 3.0, np.float32)
    X = execute_fft_plan(r2c, torch.from_numpy(const).to(gpu)).cpu().numpy()
    ref = np.zeros((b, n // 2 + 1), np.complex128)
    ref[:, 0] = 3.0 * n
    assert np.abs(X - ref).max() <= 1e-5 * 3.0 * n
