"""HIP graph capture of the execute path: small transforms are launch-bound,
and a caller can record many executes into one graph and replay it.  An
execute only enqueues kernels on the caller's stream (no allocation inside
the library, no host sync, no memset node), so it records as is.  Each replay
is checked against the eager result, with eager work and synchronisation
between replays."""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import DeviceProfile, execute_fft_plan, plan_fft

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,b,tt,td", [(2048, 1, "c2c", "forward"), (1024, 16, "c2c", "inverse"),
                                       (4096, 64, "r2c", "forward"), (1 << 16, 4, "c2c", "forward"),
                                       (256, 8, "c2r", "inverse")])
def test_graph_replay_matches_eager(gpu, n, b, tt, td):
    prof = DeviceProfile.load().hash()
    plan = plan_fft("dit", n, batch=b, profile_hash=prof, transform_type=tt, transform_direction=td)
    g = torch.Generator(gpu).manual_seed(n + b)
    shape = (b, n // 2 + 1) if tt == "c2r" else (b, n)
    dt = torch.float32 if tt == "r2c" else torch.complex64
    if b == 1:
        shape = shape[1:]
    x = torch.randn(shape, dtype=dt, device=gpu, generator=g)
    execute_fft_plan(plan, x)  # resolves the native plan before capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        execute_fft_plan(plan, x)  # warm the side stream's allocator pool
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            outs = [execute_fft_plan(plan, x) for _ in range(4)]
    torch.cuda.synchronize()
    for rep in range(3):
        # new input each time (eager work between replays): a replay that
        # did not re-run the recorded kernels would leave the old results
        x.copy_(torch.randn(shape, dtype=dt, device=gpu, generator=g))
        want = execute_fft_plan(plan, x)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o, want), f"replay {rep} differs from eager"
    ref = {"c2c": lambda h: oracle.c2c(h, td, "backward") if n <= 4096 else np.fft.fft(h.astype(np.complex128)),
           "r2c": lambda h: np.fft.rfft(h.astype(np.float64)),
           "c2r": lambda h: np.fft.irfft(h.astype(np.complex128), n=n)}[tt](x.cpu().numpy())
    assert oracle.rel_l2(outs[-1].cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("name,n,b,params", [("fft_lds_fused", 2048, 1, {}), ("fft_lds_fused_batch", 4096, 64, {}),
                                             ("fft_dit_batch", 1024, 16, {}),
                                             ("fft_four_step_batch", 1 << 14, 16, {"n1": 128}),
                                             ("fft_four_step_batch", 1 << 16, 5, {"n1": 256, "schedule": 2}),
                                             ("fft_dit_matrix_batch", 4096, 16, {})])
def test_graph_timer_leaves_the_eager_result(gpu, name, n, b, params):
    """The table builder's and bench's timer for launch-bound cells
    (runner.time_native_graph) replays a graph of back-to-back executes into
    one output: that output must equal an eager execute bit for bit, for every
    flow the timer meets (stage flow with workspace, LDS, four-step, the fused
    schedule with its counters and Z ring, dense MFMA)."""
    from kunlunxin_fft_amd import runner

    nplan = runner.get_native_plan(name, n, b, "c2c", "forward", "backward", None, params, 0)
    g = torch.Generator(gpu).manual_seed(n + b)
    x = torch.randn((b, n), dtype=torch.complex64, device=gpu, generator=g)
    ref = torch.empty_like(x)
    ws = runner.workspace_for(nplan, gpu)
    nplan.execute_ws(x.data_ptr(), ref.data_ptr(), ws.data_ptr() if ws is not None else 0, nplan.ws_bytes,
                     torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    out = torch.full_like(x, float("nan"))
    ms = runner.time_native_graph(nplan, x, out, ws, reps=8, rounds=3)
    torch.cuda.synchronize()
    assert ms > 0
    assert torch.equal(out, ref)
    check_ref = oracle.c2c(x.cpu().numpy()[:2], "forward", "backward") if n <= 4096 else None
    if check_ref is not None:
        assert oracle.rel_l2(out.cpu().numpy()[:2], check_ref) <= 1e-5
