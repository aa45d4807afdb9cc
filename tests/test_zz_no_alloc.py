"""ta_attention_matrix_noalloc, the entry point that allocates nothing, against ta_attention_matrix.

Both run the same kernels on the same plan; the no-allocation variant keeps
the partials in the library's fixed per-GPU array instead of the plan's
buffers, so the outputs must be bit-identical.  Two calls in a row, the
second on a smaller layer, plus a third repeating the first: each call's
result must not depend on what the previous one left in the array.
"""
import ctypes
import sys

import pytest
import torch

from tree_attention import CostModel, _native, schedule, shapes
from tree_attention.kernels import pack_kv, prepare

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def _layer(spec, model, seed, device):
    tree = shapes.tree(spec)
    g = torch.Generator().manual_seed(seed)
    t = -(-tree.storage_tokens // 8) * 8
    q = torch.randn(len(tree.paths), 32, 128, generator=g).bfloat16().to(device)
    k = torch.randn(t, 8, 128, generator=g).bfloat16().to(device)
    v = torch.randn(t, 8, 128, generator=g).bfloat16().to(device)
    kp, vp = pack_kv(k, v)
    prepared = prepare(schedule(tree, 32, 8, 128, "cube", model), q)
    return q, kp, vp, prepared


def _call(name, q, kp, vp, abi, out):
    lib = _native.load()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        return getattr(lib, name)(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), kp.shape[2], ctypes.byref(abi),
                                  out.data_ptr(), stream)


def test_noalloc_equals_attention_matrix(device):
    layers = [("headline 128 x 8192", shapes.headline(), CostModel.mi355x(), 101),
              ("wide 32 x 2112 (smaller)", shapes.benchmark_cases()["wide"], CostModel(), 7),
              ("headline again", shapes.headline(), CostModel.mi355x(), 5),
              # more than 16 slots per request, mixed kinds: small + 64-row + tail jobs
              ("unequal, 24 slots", shapes.benchmark_cases()["unequal"], CostModel(), 11),
              # about 50-70 slots per request over several job kinds
              ("nested, 52 slots", shapes.nested_unequal(), CostModel.mi355x(), 13)]
    for name, spec, model, seed in layers:
        q, kp, vp, prepared = _layer(spec, model, seed, device)
        abi = prepared.abi
        need = abi.nslot * abi.hq * abi.d * 2 + abi.nslot * abi.hq * 8
        say("noalloc", name, "slots", abi.nslot, "per request", abi.maxs, "items", list(abi.n_items),
            "attached tails", bool(abi.xtail), "partial bytes", need)
        assert need <= _native.NOALLOC_SCRATCH_BYTES
        # the variant ignores the plan's partial buffers
        bare = _native.TaPlan.from_buffer_copy(abi)
        bare.part, bare.lse = None, None
        a = torch.empty_like(q)
        b = torch.full_like(q, float("nan"))
        assert _call("ta_attention_matrix", q, kp, vp, abi, a) == 0
        assert _call("ta_attention_matrix_noalloc", q, kp, vp, bare, b) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(b.float()).all(), name
        assert torch.equal(a, b), name
        kinds = [k for k in range(_native.TA_NKINDS) if abi.n_items[k] > 0]
        if name.startswith(("wide", "unequal")):
            assert abi.n_items[_native.TA_TAIL] > 0  # the fused tail-merge kernel ran on the array too
        if name.startswith("unequal"):
            assert abi.maxs > 16 and len(kinds) >= 3, (abi.maxs, kinds)
        if name.startswith("nested"):
            assert abi.maxs > 16 and len(kinds) >= 2, (abi.maxs, kinds)


def test_noalloc_on_register_staged_pools(device):
    """Pools whose capacity is not a multiple of 8 run the register-staged kernels and the
    unfused order (every kind writes partials, then all requests merge): the variant keeps
    those partials in the array too.  Mixed kinds with up to 24 slots per request; two calls,
    the second on a smaller layer, each bit-identical to ta_attention_matrix."""
    for name, spec, seed in (("unequal, capacity 8k + 3", shapes.benchmark_cases()["unequal"], 31),
                             ("deep, capacity 8k + 5", shapes.benchmark_cases()["deep"], 32)):
        tree = shapes.tree(spec)
        g = torch.Generator().manual_seed(seed)
        t = -(-tree.storage_tokens // 8) * 8 + (3 if name.startswith("unequal") else 5)
        q = torch.randn(len(tree.paths), 32, 128, generator=g).bfloat16().to(device)
        k = torch.randn(t, 8, 128, generator=g).bfloat16().to(device)
        v = torch.randn(t, 8, 128, generator=g).bfloat16().to(device)
        kp, vp = pack_kv(k, v)
        assert kp.shape[2] % 8 != 0
        prepared = prepare(schedule(tree, 32, 8, 128, "cube", CostModel()), q).for_pools(kp)
        abi = prepared.abi
        assert not abi.xtail
        say("noalloc register-staged", name, "slots", abi.nslot, "per request", abi.maxs, "items",
            list(abi.n_items))
        bare = _native.TaPlan.from_buffer_copy(abi)
        bare.part, bare.lse = None, None
        a = torch.empty_like(q)
        b = torch.full_like(q, float("nan"))
        assert _call("ta_attention_matrix", q, kp, vp, abi, a) == 0
        assert _call("ta_attention_matrix_noalloc", q, kp, vp, bare, b) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(b.float()).all(), name
        assert torch.equal(a, b), name


def test_noalloc_rejects_plans_beyond_its_array(device):
    q, kp, vp, prepared = _layer(shapes.benchmark_cases()["wide"], CostModel(), 3, device)
    big = _native.TaPlan.from_buffer_copy(prepared.abi)
    big.nslot = _native.NOALLOC_SCRATCH_BYTES // (big.hq * big.d * 2) + 1
    out = torch.zeros_like(q)
    assert _call("ta_attention_matrix_noalloc", q, kp, vp, big, out) == _native.TA_ERR_SCRATCH
    torch.cuda.synchronize()
    assert not out.any()  # nothing was launched
    assert b"TA_NOALLOC_SCRATCH_BYTES" in _native.load().ta_error_string(_native.TA_ERR_SCRATCH)


_CAPTURE = """
import ctypes, sys, torch
sys.path[:0] = {paths!r}
from tree_attention import CostModel, _native, shapes
from test_zz_no_alloc import _layer, _call
dev = torch.device("cuda:0")
lib = _native.load()
q, kp, vp, prepared = _layer(shapes.nested_unequal(), CostModel.mi355x(), 21, dev)
ref = torch.empty_like(q)
assert _call("ta_attention_matrix", q, kp, vp, prepared.abi, ref) == 0
bare = _native.TaPlan.from_buffer_copy(prepared.abi)
bare.part, bare.lse = None, None
q2, kp2, vp2, prepared2 = _layer(shapes.benchmark_cases()["unequal"], CostModel(), 22, dev)
ref2 = torch.empty_like(q2)
assert _call("ta_attention_matrix", q2, kp2, vp2, prepared2.abi, ref2) == 0
torch.cuda.synchronize()
out = torch.full_like(q, float("nan"))
graph, side = torch.cuda.CUDAGraph(), torch.cuda.Stream()
print("capture: first ta_attention_matrix_noalloc call of the process", flush=True)
with torch.cuda.graph(graph, stream=side):
    rc = _call("ta_attention_matrix_noalloc", q, kp, vp, bare, out)
assert rc == 0, rc
for rep in range(4):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {{rep}}"
    # eager work between replays: another layer through the same array
    other = torch.full_like(q2, float("nan"))
    assert _call("ta_attention_matrix_noalloc", q2, kp2, vp2, prepared2.abi, other) == 0
    torch.cuda.synchronize()
    assert torch.equal(other, ref2), f"eager {{rep}}"
    print("replay", rep, "equal", flush=True)
print("ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(device):
    """The array's address is looked up on a device's first call; here that call
    is inside a stream capture (a fresh process, so no earlier call set it up).
    Every replay equals ta_attention_matrix bit for bit, with eager calls on
    another layer through the same array between the replays."""
    import subprocess
    from pathlib import Path
    here = Path(__file__).resolve().parent
    paths = [str(here), str(here.parent / "tree-attention-scheduling_amd")]
    say("noalloc capture subprocess: nested 52 slots, 4 replays")
    r = subprocess.run([sys.executable, "-c", _CAPTURE.format(paths=paths)], capture_output=True, text=True,
                       timeout=110)
    say(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert r.stdout.strip().endswith("ok")
