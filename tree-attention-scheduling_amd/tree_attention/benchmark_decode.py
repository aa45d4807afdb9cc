"""Decode-step benchmark of the Qwen3-4B-shaped workload with cached tree-attention plans.

    python -m tree_attention.benchmark_decode [--steps 16] [--layers 36] [--method cube] [--prefill tree]

Counterpart of the reference's scripts/benchmark_decode_plan.py (a cached
prompt plan whose tails grow by one token per step, :21-64) and
scripts/benchmark_qwen.py (the model around it), on one MI355X:

* model: Qwen3-4B-shaped (hidden 2560, 32 query / 8 KV heads, head dim 128,
  FFN 9728, vocabulary 151,936, RoPE theta 1e6), ``--layers`` layers (36 by
  default), random-init bf16 weights (no checkpoint is fetched);
* workload: ``shapes.qwen3_4b_workload`` -- 32 requests over a 2048-token
  prompt, a 4-way branch of 64-token nodes and 8 suffixes of 128 tokens each;
* prefill through the model's own attention, then ``--steps`` greedy decode
  steps of ``CachedPrefixDecoder`` (the prompt is planned once; each step only
  sets the tails' lengths).

Prefill is timed both ways: one full forward per request (the reference
adapter, qwen.py:34-51) and shared-prefix prefill (every tree node once over
its ancestors' cache); it reports both times and, against an fp32 forward of
the same weights (one full prompt per request), the error of each prefill's
last-token logits, so the two bf16 prefills are compared with the truth rather
than with each other.  It then runs the steps twice on two decoders
(prefilled by ``--prefill``) fed the same tokens: with the fused per-layer
decode glue (RoPE, the pool scatters and the Q layout in one launch,
``kernels.decode_append``) and with the eager ops of the reference adapter.
Per step it reports the wall time (device synchronised on both sides) and the
per-layer attention time (HIP events around each ``attention_matrix`` call),
and checks that both decoders produced identical logits.  At the steps
``--check-steps`` (0 and 15 by default) every layer's attention output of the
fused decoder is checked against an fp32 per-request attention over the same
pools and context paths (atol .008 / rtol .03, as scripts/model_checks.py:45-57
does), and the JSON line carries each checked step's per-layer relative L2
error (max and median over the layers); those steps stay out of the timings.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import statistics
import time

import torch

from . import CostModel, shapes
from . import qwen as integration
from .harness import check, reference_fp32


def _model(layers: int, device):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=151_936, hidden_size=2560, intermediate_size=9728, num_hidden_layers=layers,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=4096)
    torch.manual_seed(2027)
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            return Qwen3ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(previous)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--method", default="cube")
    ap.add_argument("--warmup", type=int, default=2, help="decode steps run before the timed ones")
    ap.add_argument("--prefill", default="tree", choices=["tree", "request"], help="prefill of the decoders")
    ap.add_argument("--check-steps", default="0,15", help="steps whose per-layer attention is checked in fp32")
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    model = _model(args.layers, dev)
    sequences = shapes.qwen3_4b_workload()
    budget = args.steps + args.warmup
    prefill_s, prefill_logits = {}, {}
    for mode in ("request", "tree"):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        probe = integration.CachedPrefixDecoder(model, sequences, budget, args.method, CostModel.mi355x(),
                                                prefill=mode)
        torch.cuda.synchronize()
        prefill_s[mode] = time.perf_counter() - t0
        prefill_logits[mode] = probe.logits.float()
        del probe
    prefill_diff = (prefill_logits["tree"] - prefill_logits["request"]).abs().max().item()
    with torch.inference_mode():
        ref_model = _model(args.layers, dev)
        ref_model.float()
        truth = torch.stack([ref_model(torch.tensor([s], device=dev), use_cache=False, logits_to_keep=1).logits[0, -1]
                             for s in sequences])
        del ref_model
        torch.cuda.empty_cache()
    vs_fp32 = {m: {"max_abs": round((l - truth).abs().max().item(), 4),
                   "rel_l2": round(((l - truth).norm() / truth.norm()).item(), 5),
                   "argmax_agree": round((l.argmax(-1) == truth.argmax(-1)).float().mean().item(), 4)}
               for m, l in prefill_logits.items()}
    decoders = {name: integration.CachedPrefixDecoder(model, sequences, budget, args.method, CostModel.mi355x(),
                                                      fused_glue=fused, prefill=args.prefill, graph=graph)
                for name, fused, graph in (("fused", True, False), ("eager", False, False), ("graph", True, True))}
    torch.cuda.synchronize()

    original = integration.attention_matrix
    attn_events = []
    check_steps = {int(x) for x in args.check_steps.split(",") if x.strip()}
    recorded = []  # (q, out, kp, vp) of every layer of a checked step

    def timed_attention(q, kp, vp, prepared):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        out = original(q, kp, vp, prepared)
        stop.record()
        attn_events.append((start, stop))
        if recording:
            recorded.append((q.clone(), out.clone(), kp, vp))
        return out

    def layer_errors(decoder, step):
        """Every recorded layer against fp32 attention along the prompt paths plus the tails so far."""
        tails = [[decoder.prefix_size + r * decoder.max_new_tokens + t for t in range(decoder.generated)]
                 for r in range(len(decoder.sequences))]
        context = type("Context", (), {"paths": [list(p) + t for p, t in zip(decoder.tree.paths, tails)]})
        rel = []
        for layer, (q, out, kp, vp) in enumerate(recorded):
            ref = reference_fp32(q, kp.permute(2, 0, 1), vp.permute(1, 0, 2), context)
            rel.append(check(out, ref, f"step {step} layer {layer} attention")["rel_l2"])
        recorded.clear()
        return {"layers": len(rel), "context_tokens": len(context.paths[0]), "max": round(max(rel), 6),
                "median": round(statistics.median(rel), 6), "per_layer": [round(x, 6) for x in rel]}

    step_ms = {name: [] for name in decoders}
    attn_us = {name: [] for name in decoders if name != "graph"}
    identical = graph_identical = True
    recording = False
    layer_rel_l2 = {}
    integration.attention_matrix = timed_attention
    try:
        for step in range(budget):
            tokens = decoders["fused"].logits.argmax(-1).tolist()
            logits = {}
            for name, decoder in decoders.items():
                recording = name == "fused" and step in check_steps
                attn_events.clear()
                # the graph decoder captures the plain call (no events inside a capture)
                integration.attention_matrix = original if name == "graph" else timed_attention
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                logits[name] = decoder.step(tokens)
                torch.cuda.synchronize()
                dt = (time.perf_counter() - t0) * 1e3
                if recording:
                    recording = False
                    layer_rel_l2[step] = layer_errors(decoder, step)
                elif step >= args.warmup and step not in check_steps:
                    step_ms[name].append(dt)
                    if name in attn_us:
                        attn_us[name].append(statistics.mean(a.elapsed_time(b) * 1e3 for a, b in attn_events))
            identical &= bool(torch.equal(logits["fused"], logits["eager"]))
            graph_identical &= bool(torch.equal(logits["fused"], logits["graph"]))
    finally:
        integration.attention_matrix = original

    cached = decoders["fused"].cached_plan.prepared
    line = {
        "benchmark": "qwen3_4b_shaped_decode",
        "config": {"layers": args.layers, "requests": len(sequences), "prompt_tree_tokens": decoders["fused"].prefix_size,
                   "method": args.method, "cost_model": "mi355x", "steps": args.steps, "warmup": args.warmup,
                   "dtype": "bf16", "weights": "random-init", "prefill": args.prefill,
                   "prompt_tokens": sum(map(len, sequences))},
        "step_ms": {n: round(statistics.median(v), 3) for n, v in step_ms.items()},
        "attention_us_per_layer": {n: round(statistics.median(v), 2) for n, v in attn_us.items()},
        "glue_saving_us_per_layer": round((statistics.median(step_ms["eager"]) - statistics.median(step_ms["fused"]))
                                          * 1e3 / args.layers, 2),
        "fused_equals_eager": identical,
        "graph_equals_fused": graph_identical,
        "graph_speedup": round(statistics.median(step_ms["fused"]) / statistics.median(step_ms["graph"]), 2),
        "timed_steps": len(step_ms["fused"]),
        "attention_rel_l2_vs_fp32": {str(k): v for k, v in sorted(layer_rel_l2.items())},
        "plan": {"jobs": len(cached.jobs), "items": list(cached.abi.n_items), "attached": len(cached.attached)},
        "prefill_s": {m: round(t, 3) for m, t in prefill_s.items()},
        "prefill_speedup": round(prefill_s["request"] / prefill_s["tree"], 2),
        "prefill_logits_max_abs_diff": round(prefill_diff, 4),
        "prefill_logits_vs_fp32": vs_fp32,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
