"""GPU parity of every evaluation configuration against the CPU FP32 oracle.

Each configuration runs under the reference's default ``CostModel()`` and the
MI355X fit (``CostModel.mi355x()``, the parameters bench.py and the model
adapter use), through ``attention_matrix`` (the ``ta_attention_matrix`` C-ABI
entry point), and is checked against ``request_attention``, the restatement of
the reference's reference.py:4-13, computed once per shape on the same
bf16/fp16-valued Q/K/V.  Bars: relative L2 <= 0.3% per layer and the
reference's device tolerance atol .008 / rtol .03 (scripts/benchmark.py:96,
scripts/benchmark_tree_grid.py:40-41).

* CPU-baseline shape: 8 requests, a 1024-token shared root + 64 private tokens
  each, ``request`` and ``cube`` plans, bf16 and fp16.
* Nested unequal-prefix tree (root 4096 -> 8 x 1024 -> 4 x 256, an internal
  terminal, two duplicate paths) under the fitted model, all four methods.
* The 81-shape requests x context x shared fraction x depth factorial
  (``shapes.config_grid``), all four methods under the fitted model; pools are
  rounded up to a multiple of 8 tokens, as the model adapter allocates them.
* The six scripts/benchmark.py:14-23 cases, including ``wide_long`` (the
  128 x 8192 headline) and ``no_share_long`` (128 x 8192, nothing shared),
  under the default and the fitted model.
"""
import sys

import pytest
import torch

from oracle.attention_oracle import relative_l2, request_attention
from tree_attention import CostModel, schedule, shapes
from tree_attention.kernels import attention_matrix, pack_kv, prepare

pytestmark = pytest.mark.gpu
METHODS = ("request", "fixed", "greedy", "cube")
REL_L2 = 3e-3
HEADS = (32, 8, 128)


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def inputs(tree, dtype, seed, align=8):
    g = torch.Generator().manual_seed(seed)
    t = -(-tree.storage_tokens // align) * align
    q = torch.randn(len(tree.paths), HEADS[0], HEADS[2], generator=g).to(dtype)
    k = torch.randn(t, HEADS[1], HEADS[2], generator=g).to(dtype)
    v = torch.randn(t, HEADS[1], HEADS[2], generator=g).to(dtype)
    return q, k, v


def check(out, ref32, what):
    torch.testing.assert_close(out, ref32.to(out.dtype), atol=0.008, rtol=0.03, msg=lambda m: f"{what}: {m}")
    err = relative_l2(out, ref32)
    assert err <= REL_L2, (what, err)
    return err


def run_methods(tree, q, k, v, device, cases, what):
    """Every (method, model) of ``cases`` against the oracle; returns {case: rel-L2}."""
    say(what, "oracle", len(tree.paths), "requests", tree.storage_tokens, "tokens")
    ref = request_attention(q.float(), k.float(), v.float(), tree)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    errs = {}
    for method, model, name in cases:
        say(what, method, name)
        plan = schedule(tree, *HEADS, method, model)
        plan.validate(tree)
        out = attention_matrix(qd, kp, vp, prepare(plan, qd)).cpu()
        errs[(method, name)] = check(out, ref, f"{what}/{method}/{name}")
    say(what, "rel-L2", {f"{m}/{n}": round(e, 6) for (m, n), e in errs.items()})
    return errs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_cpu_baseline_shape(dtype, device):
    """8 x (1024 + 64): per-request and cube plans, default and fitted cost models."""
    tree = shapes.tree(shapes.cpu_baseline_shape())
    assert tree.storage_tokens == 1536 and sum(map(len, tree.paths)) == 8704
    q, k, v = inputs(tree, dtype, 101)
    cases = [(m, model, name) for name, model in (("default", CostModel()), ("mi355x", CostModel.mi355x()))
             for m in ("request", "cube")]
    run_methods(tree, q, k, v, device, cases, f"config1/{dtype}")


def test_nested_unequal_fitted_model(device):
    """The nested unequal-prefix tree under the fitted MI355X model, all four methods."""
    tree = shapes.tree(shapes.nested_unequal())
    assert tree.storage_tokens == 20480 and len(tree.paths) == 35
    q, k, v = inputs(tree, torch.bfloat16, 7)
    run_methods(tree, q, k, v, device, [(m, CostModel.mi355x(), "mi355x") for m in METHODS], "nested")


GRID = list(shapes.config_grid())


@pytest.mark.parametrize("params,spec", GRID, ids=[
    "r{requests}_c{context}_f{fraction}_d{depth}".format(**p) for p, _ in GRID])
def test_config_grid_shape(params, spec, device):
    """One shape of the 81-shape factorial, all four methods under the fitted model
    (scripts/benchmark_tree_grid.py:40-41 checks every grid row against the oracle)."""
    tree = shapes.tree(spec)
    assert len(tree.paths) == params["requests"]
    assert all(len(p) == params["context"] for p in tree.paths)
    q, k, v = inputs(tree, torch.bfloat16, 201)
    run_methods(tree, q, k, v, device, [(m, CostModel.mi355x(), "mi355x") for m in METHODS],
                "grid/r{requests}/c{context}/f{fraction}/d{depth}".format(**params))


@pytest.mark.parametrize("name", ["no_share", "wide", "unequal", "deep", "wide_long", "no_share_long"])
def test_benchmark_case_both_models(name, device):
    """scripts/benchmark.py:14-23's six cases under the default and the fitted model."""
    tree = shapes.tree(shapes.benchmark_cases()[name])
    q, k, v = inputs(tree, torch.bfloat16, 101)
    methods = ("request", "cube") if name.endswith("_long") else METHODS
    cases = [(m, model, mname) for mname, model in (("default", CostModel()), ("mi355x", CostModel.mi355x()))
             for m in methods]
    run_methods(tree, q, k, v, device, cases, f"bench/{name}")
