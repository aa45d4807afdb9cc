"""Extract planner / tree golden values from the reference's published result files.

Reads (text JSON only) ``results/tree_grid_run{1,2,3}.json``,
``results/tree_scan.json``, ``results/benchmark.json``,
``results/npu_correctness.json``, ``results/qwen4b.json`` and
``configs/qwen_workloads.json`` under the reference checkout and writes small
fixtures next to this script.  Run in the build container only:

    python tests/golden/make_result_fixtures.py [/root/reference]
"""
import json
import sys
from pathlib import Path

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent


def load(rel):
    return json.loads((REF / rel).read_text())


def tree_grid():
    runs = [load(f"results/tree_grid_run{i}.json") for i in (1, 2, 3)]
    rows = []
    for i, row in enumerate(runs[0]):
        for other in runs[1:]:
            # the planner is deterministic: every process published the same floats
            assert other[i]["shape"] == row["shape"] and other[i]["method"] == row["method"]
            assert other[i]["estimated_us"] == row["estimated_us"]
            assert other[i]["jobs"] == row["jobs"] and other[i]["logical_jobs"] == row["logical_jobs"]
        rows.append({k: row[k] for k in ("shape", "requests", "storage_tokens", "method",
                                          "jobs", "logical_jobs", "estimated_us")})
    return {"source": "results/tree_grid_run{1,2,3}.json", "rows": rows}


def tree_scan():
    rows = load("results/tree_scan.json")
    return {"source": "results/tree_scan.json", "rows": rows}


def benchmark_cases():
    rows = []
    for row in load("results/benchmark.json"):
        rows.append({k: row[k] for k in ("case", "method", "jobs", "shared_tokens", "logical_tokens")})
    return {"source": "results/benchmark.json", "rows": rows}


def npu_jobs():
    seen = {}
    for row in load("results/npu_correctness.json"):
        seen[(row["case"], row["method"])] = row["jobs"]
    return {"source": "results/npu_correctness.json (kv_split=128, 8 Q / 2 KV heads, d=64)",
            "rows": [{"case": c, "method": m, "logical_jobs": j} for (c, m), j in seen.items()]}


def qwen_trees():
    workloads = load("configs/qwen_workloads.json")["workloads"]
    agg = load("results/qwen4b.json")["results"]
    expected = {}
    for row in agg:
        # allocated = storage + requests * new_tokens (16 per request, 8 requests)
        expected[row["workload"]] = {"allocated_kv_tokens": row["allocated_kv_tokens"],
                                     "physical_kv_tokens": row["physical_kv_tokens"],
                                     "logical_kv_tokens": row["logical_kv_tokens"]}
    return {"source": "configs/qwen_workloads.json + results/qwen4b.json",
            "new_tokens_per_request": 16,
            "workloads": {name: {"sequences": seqs, **expected[name]} for name, seqs in workloads.items()}}


if __name__ == "__main__":
    for name, fn in (("planner_tree_grid.json", tree_grid), ("planner_tree_scan.json", tree_scan),
                     ("benchmark_cases.json", benchmark_cases), ("npu_correctness_jobs.json", npu_jobs),
                     ("qwen_workload_trees.json", qwen_trees)):
        (OUT / name).write_text(json.dumps(fn(), separators=(",", ":")))
        print(name, (OUT / name).stat().st_size)
