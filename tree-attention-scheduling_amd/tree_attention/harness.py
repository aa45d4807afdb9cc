"""Shared pieces of the benchmark harnesses: KV pool rotation and the fp32 output check.

``rotated_pools`` clones the packed K/V pools until the set spans at least
``min_bytes`` (535 MB by default, above the MI355X's 256 MB MALL), so that
timing loops that rotate over them read HBM rather than the last-level cache.

``reference_fp32`` is per-request softmax attention in fp32 on the device, the
same arithmetic as the reference's reference.py:4-13 (gather the request's
path, GQA by repeating KV heads, softmax(q k^T / sqrt(d)) v, cast to q's
dtype).  The harnesses check every timed configuration against it with the
reference's device tolerance (atol .008 / rtol .03, scripts/benchmark.py:96)
and report the relative L2 error; the CPU oracle comparison of the same shapes
is the GPU test suite's.  Operands are fp32 and contiguous.

``graph_layer_us`` times layers on the device alone: a decode-sized layer
(10-20 us) is shorter than the host's submission of one ``attention_matrix``
call, so a loop of eager calls between two events measures the host.  It
captures ``count`` calls (rotating over the pools) in one HIP graph and times
replays of it, as a decode step that runs ahead of the device sees them.
"""
from __future__ import annotations

import torch

MALL_BYTES = 256 << 20
ROTATION_BYTES = 535_000_000


def rotated_pools(kp: torch.Tensor, vp: torch.Tensor, min_bytes: int = ROTATION_BYTES, max_pools: int = 256):
    """``[(kp, vp), clone, ...]`` spanning at least ``min_bytes`` (at most ``max_pools`` pools)."""
    per = kp.numel() * kp.element_size() + vp.numel() * vp.element_size()
    n = max(1, min(max_pools, -(-min_bytes // max(per, 1))))
    return [(kp, vp)] + [(kp.clone(), vp.clone()) for _ in range(n - 1)]


def pool_bytes(pools) -> int:
    return sum(k.numel() * k.element_size() + v.numel() * v.element_size() for k, v in pools)


def reference_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tree) -> torch.Tensor:
    """Per-request attention of ``q [R, HQ, D]`` over ``k, v [T, HK, D]`` along ``tree.paths``,
    computed in fp32 on q's device, returned in fp32."""
    nreq, hq, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    out = torch.empty(nreq, hq, d, dtype=torch.float32, device=q.device)
    scale = d ** -0.5
    for r, path in enumerate(tree.paths):
        ids = torch.as_tensor(path, dtype=torch.long, device=q.device)
        kr = k.index_select(0, ids).float().permute(1, 2, 0).contiguous()  # [HK, D, T]
        vr = v.index_select(0, ids).float().permute(1, 0, 2).contiguous()  # [HK, T, D]
        qr = q[r].float().reshape(hk, g, d).contiguous()                    # [HK, G, D]
        p = torch.softmax(torch.matmul(qr, kr) * scale, dim=-1)             # [HK, G, T]
        out[r] = torch.matmul(p, vr).reshape(hq, d)
    return out


def check(out: torch.Tensor, ref32: torch.Tensor, what: str) -> dict:
    """Assert ``out`` against the fp32 reference (atol .008 / rtol .03) and return the errors."""
    torch.testing.assert_close(out, ref32.to(out.dtype), atol=0.008, rtol=0.03, msg=lambda m: f"{what}: {m}")
    diff = out.float() - ref32
    return {"max_abs_error": diff.abs().max().item(),
            "rel_l2": (diff.norm() / ref32.norm().clamp_min(1e-30)).item()}


def graph_layer_us(layer, count: int, replays: int = 5) -> float:
    """Mean device time of ``layer(i)``, i = 0..count-1, from replays of one HIP graph of them.

    ``layer`` must neither allocate device memory nor synchronise (``attention_matrix``
    writes the plan's own output buffer).  The graph is captured on a side stream.
    """
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for i in range(min(count, 3)):  # first calls: library and code-object loads
            layer(i)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(count):
            layer(i)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    del graph
    return start.elapsed_time(end) * 1e3 / (replays * count)
