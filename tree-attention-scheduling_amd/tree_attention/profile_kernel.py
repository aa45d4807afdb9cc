"""Launch one kernel of a plan repeatedly for profiling (cf. scripts/profile_kernel.py in the reference).

    python -m tree_attention.profile_kernel --shape wide_long --method cube \
        --cost-model mi355x --kernel large256 --iters 20

``--kernel`` is one of ``small``, ``large64``, ``large128``, ``large256``,
``tail`` (the tail items writing partials), ``tailmerge`` (the same items
merging their requests, as in the layer), ``merge``, ``layer`` (the whole attention_matrix call), ``copy`` (a plain
device-to-device copy of ``--copy-mib`` MiB, the reference point that scales
rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes) or ``stream`` (the
library's read-only stream, ``ta_read_stream``, over ``--copy-mib`` MiB: the
read ceiling of the memory-bound kinds).  With ``--kernel stream`` the row
also gives the read rate in GB/s.  K/V rotate over
``--pools`` copies so repeated launches read HBM, not the MALL.  Prints the
mean device time per launch measured with HIP events (launch gaps included)
and, with ``--stamp``, the median of the kernels' own durations (dispatch
begin/end stamps of each launch through ``ta_time_next_launch``).
"""
from __future__ import annotations

import argparse
import json
import statistics

import torch

from . import CostModel, KVTree, schedule, shapes
from . import _native
from .kernels import (CachedDecodePlan, attention_matrix, launch_durations_us, merge, pack_kv, prepare, segment,
                      tail_merge)

KINDS = {"small": _native.TA_SMALL, "large64": _native.TA_LARGE64, "large128": _native.TA_LARGE128,
         "large256": _native.TA_LARGE256, "tail": _native.TA_TAIL}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", default="wide_long",
                    help="a scripts/benchmark.py case, or qwen3_4b (the Qwen3-4B-shaped decode workload's tree)")
    ap.add_argument("--shared-prefix", default=None, metavar="R,ROOT,PRIVATE",
                    help="instead of --shape: R requests on one ROOT-token root with PRIVATE-token tails")
    ap.add_argument("--method", default="cube")
    ap.add_argument("--cost-model", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--kernel", default="layer",
                    choices=sorted(KINDS) + ["tailmerge", "merge", "layer", "copy", "stream"])
    ap.add_argument("--stream-blocks", type=int, default=4096, help="workgroups of --kernel stream")
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--pools", type=int, default=8)
    ap.add_argument("--heads", default="32,8,128")
    ap.add_argument("--tile-rows", type=int, default=256)
    ap.add_argument("--decode", type=int, default=0, metavar="N",
                    help="decode layer: a CachedDecodePlan over the shape's plan with N reserved tail tokens "
                         "per request (scripts/benchmark_decode_plan.py's protocol), updated to --step")
    ap.add_argument("--step", type=int, default=1, help="generated tokens of each tail with --decode")
    ap.add_argument("--stamp", action="store_true",
                    help="also report the median kernel duration from dispatch stamps (library kernels only)")
    ap.add_argument("--param", action="append", default=[],
                    help="CostModel field override, e.g. --param kv_split=1024 (repeatable)")
    args = ap.parse_args(argv)
    hq, hk, d = map(int, args.heads.split(","))
    if args.shared_prefix:
        r, root, private = map(int, args.shared_prefix.split(","))
        spec = shapes.shared_prefix(r, root, private)
        args.shape = f"shared_prefix({r},{root},{private})"
    elif args.shape == "qwen3_4b":  # the Qwen3-4B-shaped decode workload's prompt tree (token sequences)
        spec = None
    else:
        spec = shapes.benchmark_cases()[args.shape]
    tree = KVTree.from_sequences(shapes.qwen3_4b_workload()) if spec is None else shapes.tree(spec)
    model = CostModel.mi355x() if args.cost_model == "mi355x" else CostModel()
    for kv in args.param:
        key, val = kv.split("=")
        setattr(model, key, type(getattr(model, key))(float(val)))
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(101)
    q = torch.randn(len(tree.paths), hq, d, generator=g).bfloat16().to(dev)
    tokens = tree.storage_tokens + len(tree.paths) * args.decode
    tokens = -(-tokens // 8) * 8  # pool capacity a multiple of 8, as the model adapter allocates it
    k = torch.randn(tokens, hk, d, generator=g).bfloat16().to(dev)
    v = torch.randn(tokens, hk, d, generator=g).bfloat16().to(dev)
    kp, vp = pack_kv(k, v)
    pools = [(kp, vp)] + [(kp.clone(), vp.clone()) for _ in range(args.pools - 1)]
    plan = schedule(tree, hq, hk, d, args.method, model)
    if args.decode:
        cached = CachedDecodePlan(plan, q, tree.storage_tokens, args.decode)
        prepared = cached.update(args.step)
        args.shape += f" + {args.decode}-token decode tails at step {args.step}"
    else:
        prepared = prepare(plan, q, args.tile_rows)
    attention_matrix(q, kp, vp, prepared)  # partials exist before a lone merge

    if args.kernel in ("copy", "stream"):
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src) if args.kernel == "copy" else torch.zeros(4 * args.stream_blocks,
                                                                            dtype=torch.int32, device=dev)
        lib = _native.load()

    def launch(i):
        kpi, vpi = pools[i % len(pools)]
        if args.kernel == "copy":
            dst.copy_(src)
        elif args.kernel == "stream":
            _native.check(lib.ta_read_stream(src.data_ptr(), src.numel(), dst.data_ptr(), args.stream_blocks,
                                             torch.cuda.current_stream().cuda_stream))
        elif args.kernel == "layer":
            attention_matrix(q, kpi, vpi, prepared)
        elif args.kernel == "merge":
            merge(prepared)
        elif args.kernel == "tailmerge":
            tail_merge(q, kpi, vpi, prepared)
        else:
            segment(q, kpi, vpi, prepared, KINDS[args.kernel])

    for i in range(3):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.iters):
        launch(i)
    end.record()
    torch.cuda.synchronize()
    row = {"kernel": args.kernel, "shape": args.shape, "method": args.method,
           "params": {f: getattr(model, f) for f in ("kv_split", "max_query_rows")},
           "tile_rows": args.tile_rows, "iters": args.iters, "us_per_launch": start.elapsed_time(end) * 1e3 / args.iters,
           "items": list(prepared.abi.n_items)}
    if args.stamp and args.kernel != "copy":
        row["kernel_us_median"] = statistics.median(launch_durations_us(launch, args.iters))
    if args.kernel == "stream":
        row["bytes"] = src.numel()
        row["read_gbs"] = src.numel() / (row.get("kernel_us_median") or row["us_per_launch"]) / 1e3
    print(json.dumps(row), flush=True)


if __name__ == "__main__":
    main()
