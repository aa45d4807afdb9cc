"""Qwen3 adapter (reference src/tree_attention/qwen.py) on tiny random models.

The reference's own check (scripts/check_qwen.py:21-57) decodes a tiny random
Qwen3 (2 layers, hidden 128, 4 Q / 2 KV heads, d = 32, fp16) through the
shared pools and compares every step's logits with a full-sequence forward of
the same model at atol .004 / rtol .02.  The CPU tests below run the same
protocol in fp32 with the attention call swapped for the oracle on the pools,
which pins the adapter's pool layout, tail positions, RoPE positions and plan
handling without a GPU; the GPU tests run the HIP kernels.
"""
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import Qwen3Config, Qwen3ForCausalLM  # noqa: E402

import tree_attention.qwen as integration  # noqa: E402
from oracle.attention_oracle import relative_l2, request_attention  # noqa: E402
from tree_attention import KVTree  # noqa: E402

SEQUENCES = [[1, 2, 3, 4, 5], [1, 2, 3, 8], [1, 2, 3, 4, 5], [7, 8, 9, 10, 11, 12]]
METHODS = ("request", "fixed", "greedy", "cube")


def tiny_model(dtype, device):
    torch.manual_seed(2026)
    cfg = Qwen3Config(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=32)
    return Qwen3ForCausalLM(cfg).to(dtype=dtype, device=device).eval()


def context_paths(decoder):
    """Physical positions each request attends to after the last step (model_checks.py:22-26)."""
    if isinstance(decoder, integration.CachedPrefixDecoder):
        return [path + tuple(decoder.prefix_size + r * decoder.max_new_tokens + t for t in range(decoder.generated))
                for r, path in enumerate(decoder.tree.paths)]
    return decoder.tree.paths


def full_forward_logits(model, sequences, device):
    with torch.inference_mode():
        return torch.stack([model(torch.tensor([s], device=device), use_cache=False).logits[0, -1]
                            for s in sequences])


class OracleAttention:
    """Stand-in for ``attention_matrix`` that evaluates the FP32 oracle on the pools."""

    def __init__(self, decoder):
        self.decoder = decoder
        self.calls = 0

    def __call__(self, q, kp, vp, prepared):
        self.calls += 1
        paths = context_paths(self.decoder)
        out = request_attention(q.cpu(), kp.permute(2, 0, 1).cpu(), vp.permute(1, 0, 2).cpu(), KVTree([], paths))
        prepared.out.copy_(out)
        return prepared.out


@pytest.mark.parametrize("cached", [False, True])
@pytest.mark.parametrize("method", METHODS)
def test_decode_matches_full_forward_cpu(method, cached, monkeypatch):
    model = tiny_model(torch.float32, "cpu")
    cls = integration.CachedPrefixDecoder if cached else integration.SharedKVDecoder
    decoder = cls(model, SEQUENCES, 3, method)
    stand_in = OracleAttention(decoder)
    monkeypatch.setattr(integration, "attention_matrix", stand_in)
    torch.testing.assert_close(decoder.logits, full_forward_logits(model, decoder.sequences, "cpu"),
                               atol=1e-4, rtol=1e-4)
    for step in range(3):
        tokens = decoder.logits.argmax(-1).tolist()
        actual = decoder.step(tokens)
        reference = full_forward_logits(model, decoder.sequences, "cpu")
        torch.testing.assert_close(actual, reference, atol=1e-4, rtol=1e-4, msg=lambda m: f"step {step}: {m}")
    assert stand_in.calls == 3 * model.config.num_hidden_layers
    # the original attention forwards are back in place
    for layer, original in zip(model.model.layers, decoder.original):
        assert layer.self_attn.forward == original


def test_pool_layout_and_capacity_cpu(monkeypatch):
    model = tiny_model(torch.float32, "cpu")
    decoder = integration.SharedKVDecoder(model, SEQUENCES, 2, "cube")
    tree = decoder.tree
    assert tree.storage_tokens == 12 and decoder.prefix_size == 12
    assert decoder.capacity == 12 + 4 * 2
    kp, vp = decoder.pools[0]
    alloc = (decoder.capacity + 7) // 8 * 8
    assert kp.shape == (2, 32, alloc) and vp.shape == (2, alloc, 32)
    monkeypatch.setattr(integration, "attention_matrix", OracleAttention(decoder))
    decoder.step([0, 1, 2, 3])
    decoder.step([4, 5, 6, 7])
    # request r's decode tokens sit at prefix + r * max_new + step
    assert [decoder.tree.paths[r][-2:] for r in range(4)] == [(12 + 2 * r, 13 + 2 * r) for r in range(4)]
    with pytest.raises(ValueError, match="max_new_tokens"):
        decoder.step([0, 0, 0, 0])
    cached = integration.CachedPrefixDecoder(model, SEQUENCES, 1, "fixed")
    monkeypatch.setattr(integration, "attention_matrix", OracleAttention(cached))
    cached.step([1, 1, 1, 1])
    with pytest.raises(ValueError, match="max_new_tokens"):
        cached.step([1, 1, 1, 1])


def decoder_state(decoder):
    return ([list(s) for s in decoder.sequences], list(decoder.tree.paths), decoder.used, decoder.generated)


@pytest.mark.parametrize("cached", [False, True])
def test_refused_step_leaves_the_decoder_unchanged_cpu(cached, monkeypatch):
    """A step refused for capacity (max_new_tokens spent, or pool slots past the pools'
    capacity) raises before it appends a token, extends the tree or advances the counters."""
    model = tiny_model(torch.float32, "cpu")
    cls = integration.CachedPrefixDecoder if cached else integration.SharedKVDecoder
    decoder = cls(model, SEQUENCES, 2, "cube")
    monkeypatch.setattr(integration, "attention_matrix", OracleAttention(decoder))
    decoder.step([0, 1, 2, 3])
    before = decoder_state(decoder)
    # pools shorter than the next step's slots (request 3 writes prefix + 3 * 2 + 1 = 19)
    full = decoder.pools
    decoder.pools = [(kp[:, :, :16], vp[:, :16]) for kp, vp in full]
    with pytest.raises(ValueError, match="pool capacity"):
        decoder.step([4, 5, 6, 7])
    assert decoder_state(decoder) == before
    decoder.pools = full
    decoder.step([4, 5, 6, 7])
    before = decoder_state(decoder)
    with pytest.raises(ValueError, match="max_new_tokens"):
        decoder.step([0, 0, 0, 0])
    assert decoder_state(decoder) == before


# prompts with duplicates, a prompt that is a prefix of others and nested branches
TREE_SEQUENCES = SEQUENCES + [[1, 2, 9], [1, 2, 3, 4, 5, 6, 7], [7, 8], [1, 2, 3, 4, 5, 6, 7, 13, 14]]


def test_tree_prefill_matches_request_prefill_cpu():
    """Shared-prefix prefill (every tree node once) gives the pools and last-token logits of the
    reference's one-forward-per-request prefill (qwen.py:34-51), up to fp32 reduction order."""
    model = tiny_model(torch.float32, "cpu")
    a = integration.SharedKVDecoder(model, TREE_SEQUENCES, 2, "cube", prefill="request")
    b = integration.SharedKVDecoder(model, TREE_SEQUENCES, 2, "cube", prefill="tree")
    torch.testing.assert_close(b.logits, full_forward_logits(model, TREE_SEQUENCES, "cpu"), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(b.logits, a.logits, atol=1e-5, rtol=1e-5)
    n = a.prefix_size
    for (ka, va), (kb, vb) in zip(a.pools, b.pools):
        torch.testing.assert_close(kb[..., :n], ka[..., :n], atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(vb[:, :n], va[:, :n], atol=1e-5, rtol=1e-5)
    with pytest.raises(ValueError, match="prefill"):
        integration.SharedKVDecoder(model, SEQUENCES, 2, "cube", prefill="batch")


@pytest.mark.parametrize("seqs", [[[1, 2], [3, 4, 5], [6]], [[9]], [[1, 2, 3], [1, 2, 3]],
                                  [[4, 5], [4, 6, 7], [8, 9], [10]]])
def test_tree_prefill_edge_trees_cpu(seqs):
    """Childless nodes batched straight under the root (an empty cache repeated per row), a
    single one-token prompt and duplicate prompts."""
    model = tiny_model(torch.float32, "cpu")
    a = integration.SharedKVDecoder(model, seqs, 2, "cube", prefill="request")
    b = integration.SharedKVDecoder(model, seqs, 2, "cube", prefill="tree")
    torch.testing.assert_close(b.logits, full_forward_logits(model, seqs, "cpu"), atol=1e-5, rtol=1e-5)
    n = a.prefix_size
    for (ka, va), (kb, vb) in zip(a.pools, b.pools):
        torch.testing.assert_close(kb[..., :n], ka[..., :n], atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(vb[:, :n], va[:, :n], atol=1e-5, rtol=1e-5)


# four childless siblings of lengths 1-3 under one node, next to inner nodes and a lone leaf
BRANCHY = [[5, 6, 1], [5, 6, 2, 3], [5, 6, 4, 4, 4], [5, 6, 7], [5, 9, 9], [8], [5, 6, 2, 3]]


@pytest.mark.parametrize("leaf_batch", [1, 3, 16])
def test_tree_prefill_forwards_cpu(leaf_batch, monkeypatch):
    """Each stored prompt token goes through the model once: inner nodes one forward each,
    childless siblings right-padded in groups of ``leaf_batch``; logits and pools equal
    the per-request prefill's (the reference's: every prompt in full)."""
    model = tiny_model(torch.float32, "cpu")
    shapes_seen = []
    forward = model.forward

    def counting(*args, **kwargs):
        shapes_seen.append(tuple(kwargs["input_ids"].shape))
        return forward(*args, **kwargs)

    monkeypatch.setattr(integration.SharedKVDecoder, "_prefill",
                        lambda self: integration.SharedKVDecoder._prefill_tree(self, leaf_batch))
    monkeypatch.setattr(model, "forward", counting)
    decoder = integration.SharedKVDecoder(model, BRANCHY, 2, "cube", prefill="request")
    nodes = decoder.tree.nodes
    expected = [(1, len(n.tokens)) for n in nodes if n.tokens and n.children]
    for n in nodes:
        leaves = [len(nodes[c].tokens) for c in n.children if not nodes[c].children]
        for i in range(0, len(leaves), leaf_batch):
            group = leaves[i:i + leaf_batch]
            expected.append((len(group), max(group)))
    assert sorted(shapes_seen) == sorted(expected)
    assert sum(len(n.tokens) for n in nodes) == decoder.prefix_size
    monkeypatch.undo()
    reference = integration.SharedKVDecoder(model, BRANCHY, 2, "cube", prefill="request")
    torch.testing.assert_close(decoder.logits, reference.logits, atol=1e-5, rtol=1e-5)
    n = decoder.prefix_size
    for (ka, va), (kb, vb) in zip(reference.pools, decoder.pools):
        torch.testing.assert_close(kb[..., :n], ka[..., :n], atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(vb[:, :n], va[:, :n], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("cached", [False, True])
def test_tree_prefill_decode_matches_full_forward_cpu(cached, monkeypatch):
    model = tiny_model(torch.float32, "cpu")
    cls = integration.CachedPrefixDecoder if cached else integration.SharedKVDecoder
    decoder = cls(model, TREE_SEQUENCES, 3, "cube", prefill="tree")
    monkeypatch.setattr(integration, "attention_matrix", OracleAttention(decoder))
    for step in range(3):
        actual = decoder.step(decoder.logits.argmax(-1).tolist())
        reference = full_forward_logits(model, decoder.sequences, "cpu")
        torch.testing.assert_close(actual, reference, atol=1e-4, rtol=1e-4, msg=lambda m: f"step {step}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_tree_prefill_decode_gpu(dtype, device):
    """Tree prefill on the GPU, then 3 greedy steps of the cached plan on the HIP kernels: logits
    against a full forward at the tolerances of the decode check below."""
    model = tiny_model(dtype, device)
    atol, rtol = (0.004, 0.02) if dtype == torch.float16 else (0.016, 0.02)
    decoder = integration.CachedPrefixDecoder(model, TREE_SEQUENCES, 3, "cube", prefill="tree")
    torch.testing.assert_close(decoder.logits, full_forward_logits(model, TREE_SEQUENCES, device), atol=atol,
                               rtol=rtol)
    for step in range(3):
        actual = decoder.step(decoder.logits.argmax(-1).tolist())
        reference = full_forward_logits(model, decoder.sequences, device)
        torch.testing.assert_close(actual, reference, atol=atol, rtol=rtol, msg=lambda m: f"step {step}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cached", [False, True])
def test_decode_matches_full_forward_gpu(cached, dtype, device):
    """scripts/check_qwen.py protocol on the HIP kernels: 3 greedy steps, all four methods."""
    model = tiny_model(dtype, device)
    cls = integration.CachedPrefixDecoder if cached else integration.SharedKVDecoder
    # fp16: the reference's tolerance.  bf16 (not in the reference's check): its
    # unit roundoff is 8x fp16's; logits of this model are below 1, where one bf16
    # ulp is 0.0039, so four ulps are allowed.
    atol, rtol = (0.004, 0.02) if dtype == torch.float16 else (0.016, 0.02)
    for method in METHODS:
        decoder = cls(model, SEQUENCES, 3, method)
        for step in range(3):
            tokens = decoder.logits.argmax(-1).tolist()
            actual = decoder.step(tokens)
            reference = full_forward_logits(model, decoder.sequences, device)
            torch.testing.assert_close(actual, reference, atol=atol, rtol=rtol,
                                       msg=lambda m: f"{method} step {step}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_decode_glue_equals_eager_glue(dtype, device):
    """The fused per-layer glue (RoPE, pool scatters, Q layout in one launch) gives the
    same logits, bit for bit, as the eager ops of the reference adapter."""
    model = tiny_model(dtype, device)
    for cls in (integration.SharedKVDecoder, integration.CachedPrefixDecoder):
        fused = cls(model, SEQUENCES, 3, "cube", fused_glue=True)
        eager = cls(model, SEQUENCES, 3, "cube", fused_glue=False)
        for _ in range(3):
            tokens = fused.logits.argmax(-1).tolist()
            a, b = fused.step(tokens), eager.step(tokens)
            assert torch.equal(a, b)
        # written pool positions: the prompt tree and each request's generated tail slots
        written = list(range(fused.prefix_size)) + [fused.prefix_size + r * fused.max_new_tokens + t
                                                    for r in range(len(SEQUENCES)) for t in range(fused.generated)]
        idx = torch.tensor(written, device=device)
        for (kp1, vp1), (kp2, vp2) in zip(fused.pools, eager.pools):
            assert torch.equal(kp1.index_select(2, idx), kp2.index_select(2, idx))
            assert torch.equal(vp1.index_select(1, idx), vp2.index_select(1, idx))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,method,prefill", [(torch.float16, "cube", "request"), (torch.bfloat16, "cube", "tree"),
                                                  (torch.bfloat16, "fixed", "request")])
def test_graph_decode_equals_eager_decode(dtype, method, prefill, device):
    """CachedPrefixDecoder(graph=True) captures the first step's forward in a HIP graph and
    replays it: every step's logits and the pools equal the eager decoder's, bit for bit,
    with the host's own work between the replays; the step past max_new_tokens is refused
    and leaves the decoder as it was."""
    model = tiny_model(dtype, device)
    graphed = integration.CachedPrefixDecoder(model, SEQUENCES, 4, method, graph=True, prefill=prefill)
    eager = integration.CachedPrefixDecoder(model, SEQUENCES, 4, method, prefill=prefill)
    kept = []
    for _ in range(4):
        tokens = eager.logits.argmax(-1).tolist()
        a, b = graphed.step(tokens), eager.step(tokens)
        kept.append(a)
        assert torch.equal(a, b)
        torch.cuda.synchronize()
    assert graphed._replay is not None
    # returned logits are the caller's: later replays do not overwrite them
    assert not any(kept[i].data_ptr() == kept[j].data_ptr() for i in range(4) for j in range(i))
    written = list(range(graphed.prefix_size)) + [graphed.prefix_size + r * graphed.max_new_tokens + t
                                                  for r in range(len(SEQUENCES)) for t in range(graphed.generated)]
    idx = torch.tensor(written, device=device)
    for (kp1, vp1), (kp2, vp2) in zip(graphed.pools, eager.pools):
        assert torch.equal(kp1.index_select(2, idx), kp2.index_select(2, idx))
        assert torch.equal(vp1.index_select(1, idx), vp2.index_select(1, idx))
    before = (graphed.generated, [list(s) for s in graphed.sequences])
    with pytest.raises(ValueError):
        graphed.step(eager.logits.argmax(-1).tolist())
    assert (graphed.generated, graphed.sequences) == before


def test_graph_decode_needs_the_gpu_cpu():
    model = tiny_model(torch.float32, torch.device("cpu"))
    with pytest.raises(ValueError):
        integration.CachedPrefixDecoder(model, SEQUENCES, 2, "cube", graph=True)


@pytest.mark.gpu
def test_per_layer_attention_vs_oracle_gpu(device, monkeypatch):
    """scripts/model_checks.py:42-64: every layer's tree attention vs FP32 on the same Q/K/V."""
    model = tiny_model(torch.bfloat16, device)
    decoder = integration.CachedPrefixDecoder(model, SEQUENCES, 4, "cube")
    original = integration.attention_matrix
    errors = []

    def checked(q, kp, vp, prepared):
        actual = original(q, kp, vp, prepared)
        ref = request_attention(q.float().cpu(), kp.permute(2, 0, 1).float().cpu(),
                                vp.permute(1, 0, 2).float().cpu(), KVTree([], context_paths(decoder)))
        errors.append(relative_l2(actual.cpu(), ref))
        torch.testing.assert_close(actual.cpu(), ref.to(actual.dtype), atol=0.008, rtol=0.03)
        return actual

    monkeypatch.setattr(integration, "attention_matrix", checked)
    for _ in range(4):
        decoder.step(decoder.logits.argmax(-1).tolist())
    assert len(errors) == 4 * model.config.num_hidden_layers
    assert max(errors) <= 3e-3, errors


def qwen3_4b_workload(seed=5):
    """The shared workload builder (tree_attention.shapes), which checks the tree."""
    from tree_attention import shapes
    return shapes.qwen3_4b_workload(seed)


@pytest.mark.gpu
def test_qwen3_4b_shaped_per_layer_attention(device, monkeypatch):
    """Qwen3-4B-shaped random-init bf16 decoder (36 layers, hidden 2560, 32Q/8KV, d=128,
    FFN 9728, RoPE theta 1e6): 16 greedy decode steps of the cached plan over the
    2048 + 64 + 128 workload, every layer's attention at steps 0 and 15 against the
    FP32 oracle on the same Q/K/V (scripts/model_checks.py:42-64)."""
    from tree_attention import CostModel

    cfg = Qwen3Config(vocab_size=151_936, hidden_size=2560, intermediate_size=9728, num_hidden_layers=36,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=4096)
    torch.manual_seed(2027)
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(previous)
    print("model built", flush=True)
    sequences = qwen3_4b_workload()
    decoder = integration.CachedPrefixDecoder(model, sequences, 16, "cube", CostModel.mi355x())
    print("prefilled", decoder.prefix_size, "physical prompt tokens", flush=True)
    original = integration.attention_matrix
    errors, checking = [], {"on": False}

    def checked(q, kp, vp, prepared):
        actual = original(q, kp, vp, prepared)
        if checking["on"]:
            ref = request_attention(q.float().cpu(), kp.permute(2, 0, 1).float().cpu(),
                                    vp.permute(1, 0, 2).float().cpu(), KVTree([], context_paths(decoder)))
            errors.append(relative_l2(actual.cpu(), ref))
        return actual

    monkeypatch.setattr(integration, "attention_matrix", checked)
    for step in range(16):
        checking["on"] = step in (0, 15)
        logits = decoder.step(decoder.logits.argmax(-1).tolist())
        assert torch.isfinite(logits).all()
        print("step", step, "max rel-L2 so far", max(errors, default=0.0), flush=True)
    assert len(errors) == 2 * cfg.num_hidden_layers
    assert max(errors) <= 3e-3, max(errors)
