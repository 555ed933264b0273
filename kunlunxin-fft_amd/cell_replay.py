"""Replay one selector-table cell on the GPU: the plan the table selects for
(N, batch, semantic) and any named alternatives, each run ``--reps`` times
back to back on one stream, with the median HIP-event time of each.  For
checking a table decision outside the builder, for instance under
``rocprofv3 --kernel-trace --stats``, whose per-kernel durations then come
from the same launches.

    python kunlunxin-fft_amd/cell_replay.py --n 16 --batch 2097152 \\
        --runner fft_lds_fused_batch:elems=4 --runner fft_dit_matrix_batch

An alternative is a runner name with optional ``key=value`` plan
parameters after a colon, comma-separated (integers where they parse).
"""
from __future__ import annotations

import argparse
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def parse_runner(text: str):
    name, _, rest = text.partition(":")
    params = {}
    for kv in filter(None, rest.split(",")):
        k, _, v = kv.partition("=")
        params[k] = int(v) if v.lstrip("-").isdigit() else v
    return name, params


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, required=True)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--direction", default="dit")
    ap.add_argument("--transform-type", default="c2c", choices=("c2c", "r2c", "c2r"))
    ap.add_argument("--runner", action="append", default=[], help="NAME[:key=value,...]; repeatable")
    ap.add_argument("--reps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    args = ap.parse_args()

    sys.path.insert(0, os.path.dirname(HERE))
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    import torch

    from kunlunxin_fft_amd.runner import get_native_plan, output_spec, workspace_for

    n, b, tt = args.n, args.batch, args.transform_type
    td = "inverse" if tt == "c2r" else "forward"
    plan = pkg.plan_fft(args.direction, n, batch=b, profile_hash=pkg.DeviceProfile.load().hash(),
                        transform_type=tt, transform_direction=td)
    runs = [("table: " + plan.executed, plan.executed, plan.block, dict(plan.params))]
    for r in args.runner:
        name, params = parse_runner(r)
        runs.append((r, name, 256, params))
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(n + b)
    if tt == "r2c":
        x = torch.randn((b, n), dtype=torch.float32, device=dev, generator=g)
    else:
        x = torch.randn((b, n // 2 + 1 if tt == "c2r" else n), dtype=torch.complex64, device=dev, generator=g)
    stream = torch.cuda.current_stream(dev)
    print(f"N={n} B={b} {tt} {td}: table selects {plan.executed} {plan.params} ({plan.selection_source})",
          flush=True)
    for label, name, block, params in runs:
        nplan = get_native_plan(name, n, b, tt, td, "backward", block, params, 0)
        shape, dt = output_spec(tt, n, b)
        out = torch.empty(shape, dtype=dt, device=dev)
        ws = workspace_for(nplan, dev)
        wp = ws.data_ptr() if ws is not None else 0
        for _ in range(args.warmup):
            nplan.execute_ws(x.data_ptr(), out.data_ptr(), wp, nplan.ws_bytes, stream.cuda_stream)
        ms = []
        for _ in range(args.reps):
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            nplan.execute_ws(x.data_ptr(), out.data_ptr(), wp, nplan.ws_bytes, stream.cuda_stream)
            e.record(stream)
            ms.append((s, e))
        torch.cuda.synchronize(dev)
        med = statistics.median(s.elapsed_time(e) for s, e in ms)
        print(f"  {label:<40} flow {nplan.flow_name:<10} {med * 1e3:9.2f} us per execute "
              f"({nplan.info.launches} launch{'es' if nplan.info.launches != 1 else ''})", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
