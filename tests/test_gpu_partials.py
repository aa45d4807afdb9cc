"""The fp16 partial rows the GPU writes, read back and checked against exact partials.

The segment kernels store every partial output row as fp16 values of (o / z) * 2^-e, e the
frexp exponent of the row's largest |o / z|, beside an fp32 (log-sum-exp, e) pair; the
reference keeps fp32 partials (kernels.py:140-141).  Here one layer runs on the device, its
partial buffers are copied back, decoded, and compared row by row with the same partials
computed on the CPU in fp64 without rounding.  Two CPU emulations split the device's error:
the kernels' P rounded to bf16 before PV (fp32 partials; test_partial_precision emulates the
whole layer so), and the fp16 storage of the exact partials alone.  The decoded device partials
merged in fp64 on the CPU are then compared with the merge kernel's output.
"""
import math

import pytest
import torch

from oracle.attention_oracle import relative_l2, request_attention
from tree_attention import CostModel, KVTree, schedule, shapes
from tree_attention.kernels import CachedDecodePlan, attention_matrix, pack_kv, prepare

from test_partial_precision import HK, HQ, D, _partials_by_request

pytestmark = pytest.mark.gpu


def _layer(name, device):
    """The headline layer or the Qwen3-4B-shaped decode layer (step 8 of 16), prepared on the device."""
    g = torch.Generator().manual_seed(101)
    tree = shapes.tree(shapes.headline()) if name == "headline" else KVTree.from_sequences(shapes.qwen3_4b_workload())
    decode = 16 if name == "decode" else 0
    t = tree.storage_tokens + decode * len(tree.paths)
    q = torch.randn(len(tree.paths), HQ, D, generator=g).bfloat16()
    k = torch.randn(t, HK, D, generator=g).bfloat16()
    v = torch.randn(t, HK, D, generator=g).bfloat16()
    plan = schedule(tree, HQ, HK, D, "cube", CostModel.mi355x())
    qd = q.to(device)
    if decode:
        prepared = CachedDecodePlan(plan, qd, tree.storage_tokens, decode).update(8)
        paths = [p + tuple(range(tree.storage_tokens + decode * r, tree.storage_tokens + decode * r + 8))
                 for r, p in enumerate(tree.paths)]
    else:
        prepared = prepare(plan, qd)
        paths = tree.paths
    return q, k, v, qd, paths, prepared


def _slots(prepared, nreq):
    """Per request, the partial slot of each entry of ``_partials_by_request`` (job order)."""
    rowbase = prepared.rowbase.cpu().tolist()
    slots = [[] for _ in range(nreq)]
    for j, job in enumerate(prepared.jobs):
        for pos, r in enumerate(job.requests):
            slots[r].append(rowbase[j] + pos)
    return slots


def _partials(q, k, v, toks):
    """Exact (fp64) and bf16-P (fp32) values of one request's partial over ``toks``: (o / z) per
    query head for each, and the exact log-sum-exp."""
    kv_of_head = torch.arange(HQ) // (HQ // HK)
    ids = torch.as_tensor(toks, dtype=torch.long)
    kr = k.index_select(0, ids).double()[:, kv_of_head, :]
    vr = v.index_select(0, ids).double()[:, kv_of_head, :]
    s = torch.einsum("hd,lhd->hl", q.double(), kr) / math.sqrt(D)
    m = s.amax(-1, keepdim=True)
    p = torch.exp(s - m)
    z = p.sum(-1, keepdim=True)
    exact = torch.einsum("hl,lhd->hd", p, vr) / z
    pb = p.float().bfloat16().double()                 # P rounded before PV, z over the rounded P
    emulated = torch.einsum("hl,lhd->hd", pb, vr) / pb.sum(-1, keepdim=True)
    return exact, emulated, (m + torch.log(z)).squeeze(-1)


def _row_order():
    """Head-dim index of each stored element of a partial row: eight-element slice d8 holds
    d = 32 (d8 / 4) + 4 (d8 % 4) + {0..3} and the same + 16 (the order the merge kernel reads)."""
    order = torch.empty(D, dtype=torch.long)
    for d8 in range(D // 8):
        base = 32 * (d8 // 4) + 4 * (d8 % 4)
        for j in range(4):
            order[8 * d8 + j] = base + j
            order[8 * d8 + 4 + j] = base + 16 + j
    assert sorted(order.tolist()) == list(range(D))
    return order


def _fp16_storage(o):
    amax = o.abs().amax(-1, keepdim=True)
    _, e = torch.frexp(amax)
    return torch.ldexp(torch.ldexp(o, -e).half().float(), e)


@pytest.mark.parametrize("name", ["headline", "decode"])
def test_device_partials_against_fp32(name, device, capsys):
    q, k, v, qd, paths, prepared = _layer(name, device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    out = attention_matrix(qd, kp, vp, prepared)
    torch.cuda.synchronize()
    out = out.cpu()
    stored = prepared.part.float().cpu()
    part = torch.empty_like(stored)
    part[..., _row_order()] = stored
    lse = prepared.lse.cpu()
    parts = _partials_by_request(prepared, len(paths))
    slots = _slots(prepared, len(paths))
    num_dev = num_p = num_16 = den = 0.0
    lse_err = 0.0
    merged = torch.empty(len(paths), HQ, D, dtype=torch.float64)
    for r, plist in enumerate(parts):
        assert len(plist) == len(slots[r])
        os_dev, ls_dev = [], []
        for toks, sl in zip(plist, slots[r]):
            exact, emulated, l64 = _partials(q[r], k, v, toks)
            o_dev = torch.ldexp(part[sl], lse[sl, :, 1:2].round().int()).double()
            l_dev = lse[sl, :, 0].double()
            num_dev += float(((o_dev - exact) ** 2).sum())
            num_p += float(((emulated - exact) ** 2).sum())
            num_16 += float(((_fp16_storage(exact.float()).double() - exact) ** 2).sum())
            den += float((exact ** 2).sum())
            lse_err = max(lse_err, float((l_dev - l64).abs().max()))
            os_dev.append(o_dev.double())
            ls_dev.append(l_dev.double())
        w = torch.softmax(torch.stack(ls_dev), dim=0)
        merged[r] = (torch.stack(os_dev) * w[..., None]).sum(0)
    err_dev, err_p, err_16 = (math.sqrt(x / den) for x in (num_dev, num_p, num_16))
    merge_err = relative_l2(out.float(), merged.float())
    ref = request_attention(q.float(), k.float(), v.float(), paths)
    with capsys.disabled():
        print(f"\n{name}: device partials vs exact partials rel-L2 {err_dev:.6f} (emulated: bf16 P "
              f"{err_p:.6f}, fp16 storage {err_16:.6f}), max |lse difference| {lse_err:.2e}; merge kernel vs fp64 merge of the "
              f"device partials {merge_err:.6f}; layer vs oracle {relative_l2(out.float(), ref):.6f}; "
              f"slots/request {max(map(len, slots))}")
    assert err_dev <= 3e-3
    # the device's partials err as the bf16 P and the fp16 storage predict, the storage a small part
    assert err_dev <= 1.3 * math.hypot(err_p, err_16) and err_16 <= 0.25 * err_dev
    assert lse_err <= 4e-3              # z sums the bf16-rounded P: at most about 2^-8 relative
    assert merge_err <= 3e-3            # bf16 output rounding of an fp32 merge
