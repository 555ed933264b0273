"""mfft_execute_noalloc: the allocation-free execute over the library's
static scratch, through the C ABI (ctypes), against mfft_execute_ws with a
torch-allocated workspace -- the same kernels, so the results must be
bit-identical.  Two calls in a row share the static buffer, the second with
a smaller input; among them the fused four-step schedule, whose scratch
carries state (launch counters, cleared by a fill kernel at the start of
every call, and its ring of Z slots).  The same executes recorded into a HIP
graph and replayed, with new inputs and eager work between replays, match
eager executes every time.  A plan needing more scratch than the buffer is
refused before any launch."""
import numpy as np
import pytest
import torch

from kunlunxin_fft_amd import native

pytestmark = pytest.mark.gpu

LIMIT = 32 << 20  # MFFT_NOALLOC_SCRATCH_BYTES
# fused-schedule queue settings (params[3]): lag 2, 2 items per dequeue, 6 Z
# slots per XCD, 2 blocks per CU -- a ring of 8 XCDs x 6 x N complex64 that
# fits the static buffer at N = 2^16 (24 MiB)
FUSED_WORD = 2 | (2 << 8) | (6 << 16) | (2 << 24)

# (n, batch, transform, direction, flow, params): the second of each pair is smaller
PAIRS = [
    ((4096, 64, "c2c", "forward", native.FLOW_RADIX2_DIT, (256,)),
     (1024, 8, "c2c", "forward", native.FLOW_RADIX2_DIT, (256,))),
    ((1 << 18, 4, "r2c", "forward", native.FLOW_FOUR_STEP, (256,)),
     (1 << 17, 3, "r2c", "forward", native.FLOW_FOUR_STEP, (256,))),
    ((2048, 16, "c2r", "inverse", native.FLOW_RADIX4_DIT, ()),
     (512, 5, "c2r", "inverse", native.FLOW_RADIX4_DIT, ())),
    ((1 << 14, 256, "c2c", "inverse", native.FLOW_RADIX4_DIF, ()),
     (1 << 12, 4, "c2c", "inverse", native.FLOW_RADIX4_DIF, ())),
    ((2048, 16, "c2c", "forward", native.FLOW_LDS_FUSED, ()),
     (256, 3, "c2c", "forward", native.FLOW_LDS_FUSED, ())),
    # the fused schedule (params[2] = 2): counters + Z ring in the static buffer
    ((1 << 16, 8, "c2c", "forward", native.FLOW_FOUR_STEP, (256, 0, 2, FUSED_WORD)),
     (1 << 15, 3, "c2c", "inverse", native.FLOW_FOUR_STEP, (128, 0, 2, FUSED_WORD))),
    # the narrow schedule (params[2] = 3): a real transform's pre-twiddle
    # runs as its own launch, out of the static buffer
    ((1 << 18, 2, "c2r", "inverse", native.FLOW_FOUR_STEP, (0, 0, 3)),
     (1 << 16, 1, "c2r", "inverse", native.FLOW_FOUR_STEP, (0, 0, 3))),
]


def _io(n, b, tt, gpu, seed):
    rng = np.random.default_rng(seed)
    if tt == "r2c":
        x = torch.from_numpy(rng.standard_normal((b, n)).astype(np.float32)).to(gpu)
        shape, dt = (b, n // 2 + 1), torch.complex64
    else:
        m = n // 2 + 1 if tt == "c2r" else n
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
        x = torch.from_numpy(h).to(gpu)
        shape, dt = ((b, n), torch.float32) if tt == "c2r" else ((b, n), torch.complex64)
    return x, torch.empty(shape, dtype=dt, device=gpu), torch.empty(shape, dtype=dt, device=gpu)


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0][2]}-flow{p[0][4]}-N{p[0][0]}")
def test_noalloc_matches_execute_ws(gpu, pair):
    st = torch.cuda.current_stream(gpu).cuda_stream
    for k, (n, b, tt, td, flow, prm) in enumerate(pair):
        print(f"noalloc case {tt} {td} flow={flow} N={n} B={b} call={k}", flush=True)
        p = native.NativePlan(n, b, tt, td, "backward", flow, prm, caller_workspace=True)
        assert p.ws_bytes <= LIMIT
        x, y_ref, y = _io(n, b, tt, gpu, seed=100 + 7 * k + n)
        ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=gpu)
        p.execute_ws(x.data_ptr(), y_ref.data_ptr(), ws.data_ptr() if p.ws_bytes else 0, p.ws_bytes, st)
        y.fill_(float("nan"))
        p.execute_noalloc(x.data_ptr(), y.data_ptr(), st)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"call {k}: N={n} B={b} {tt}"
        assert torch.isfinite(torch.view_as_real(y) if y.is_complex() else y).all()
        assert p.sync_overruns() == 0


GRAPH_CASES = [
    (4096, 16, "c2c", "forward", native.FLOW_RADIX2_DIT, (256,)),
    (1 << 17, 2, "r2c", "forward", native.FLOW_FOUR_STEP, (256,)),
    (1 << 16, 4, "c2c", "forward", native.FLOW_FOUR_STEP, (256, 0, 2, FUSED_WORD)),
    (1 << 18, 1, "r2c", "forward", native.FLOW_FOUR_STEP, (0, 0, 3)),
]


@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: f"{c[2]}-flow{c[4]}-N{c[0]}-p{len(c[5])}")
def test_noalloc_under_graph_capture(gpu, case):
    """The entry point's purpose: an execute recorded into a HIP graph with
    no allocation.  Three replays, each on a new input copied into the
    captured buffer, with an eager execute_ws of the same input between
    them: every replay's output equals the eager one bit for bit."""
    n, b, tt, td, flow, prm = case
    print(f"noalloc graph case {tt} {td} flow={flow} N={n} B={b} params={prm}", flush=True)
    p = native.NativePlan(n, b, tt, td, "backward", flow, prm, caller_workspace=True)
    assert p.ws_bytes <= LIMIT
    assert p.ws_bytes > 0 or tt == "r2c"  # the stage flow and the fused schedule use scratch
    x, y_ref, y = _io(n, b, tt, gpu, seed=500 + n)
    ws = torch.empty(max(p.ws_bytes, 1), dtype=torch.uint8, device=gpu)
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        p.execute_noalloc(x.data_ptr(), y.data_ptr(), side.cuda_stream)  # first call outside the capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            p.execute_noalloc(x.data_ptr(), y.data_ptr(), side.cuda_stream)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(gpu).cuda_stream
    for r in range(3):
        x2, _, _ = _io(n, b, tt, gpu, seed=600 + 13 * r + n)
        x.copy_(x2)
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        p.execute_ws(x.data_ptr(), y_ref.data_ptr(), ws.data_ptr() if p.ws_bytes else 0, p.ws_bytes, st)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"replay {r}: N={n} B={b} {tt} params={prm}"
    assert p.sync_overruns() == 0
    del graph


def test_noalloc_refuses_plans_beyond_the_static_buffer(gpu):
    """An M0 plan of 4096 x 2048 rows needs 64 MiB of ping-pong scratch: the
    call fails with ValueError before any launch, and the output is untouched."""
    p = native.NativePlan(4096, 2048, "c2c", "forward", "backward", native.FLOW_RADIX2_DIT, (256,),
                          caller_workspace=True)
    assert p.ws_bytes > LIMIT
    x = torch.zeros((2048, 4096), dtype=torch.complex64, device=gpu)
    y = torch.full((2048, 4096), 7.0, dtype=torch.complex64, device=gpu)
    with pytest.raises(ValueError, match="static buffer"):
        p.execute_noalloc(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
