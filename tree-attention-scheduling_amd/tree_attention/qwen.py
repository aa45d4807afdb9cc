"""Qwen3 decoding over shared per-layer KV pools (drop-in for the reference's ``qwen.py``).

``SharedKVDecoder`` (reference src/tree_attention/qwen.py:9-103) and
``CachedPrefixDecoder`` (:106-124) keep their constructor arguments, public
attributes (``tree``, ``sequences``, ``pools``, ``logits``, ``used``,
``prefix_size``, ``generated``, ``max_new_tokens``, ``capacity``) and
``step(token_ids) -> logits``.

Pool layout (the layout the HIP segment kernels read):

* ``pools[layer] = (kp [HK, D, capacity], vp [HK, capacity, D])`` in the
  model dtype; positions ``[0, prefix_size)`` hold the prompt tree in the
  physical order fixed by ``KVTree.from_sequences``; request ``r``'s decode
  tail occupies ``[prefix_size + r * max_new_tokens, prefix_size + (r + 1) *
  max_new_tokens)`` (qwen.py:53-56), so every tail is one contiguous run.

Per decode step each layer's attention forward is swapped for one that writes
the step's RoPE'd K/V into the pools and calls ``attention_matrix`` on them;
the original forwards are restored afterwards.  The RoPE, the two pool
scatters and the Q layout copy run as one HIP launch per layer
(``kernels.decode_append``, bit-identical to the eager ops) for bf16 / fp16
models on the GPU; ``fused_glue=False`` (and fp32 or CPU models) keep the eager
ops.  ``attention_matrix`` is looked
up as this module's global at call time, so a checker may wrap it (the
reference's scripts/model_checks.py:43,59 does).
"""
from __future__ import annotations

from types import MethodType

import torch

from .kernels import CachedDecodePlan, attention_matrix, decode_append, prepare
from .schedule import CostModel, schedule
from .tree import KVTree

try:  # the model's own rotary helper (transformers >= 4.57)
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
except ImportError as exc:  # pragma: no cover - transformers is a hard dependency of this module
    raise ImportError("tree_attention.qwen needs transformers with Qwen3 support") from exc


def _find_leaf(tree: KVTree, request: int) -> int:
    for i, node in enumerate(tree.nodes):
        if request in node.terminal:
            return i
    raise ValueError(f"request {request} has no terminal node")


class SharedKVDecoder:
    """Greedy-decode driver whose attention reads one physical copy of shared prefixes.

    ``sequences`` are token-id lists (one per request).  The prompt of every
    request is prefilled with the model's own attention; afterwards every
    ``step`` appends one token per request and re-plans the whole tree
    (reference qwen.py:58-61,74-103).  ``prefill="request"`` runs one full
    forward per request, as the reference does; ``prefill="tree"`` runs every
    tree node once over its ancestors' cache (``_prefill_tree``).
    """

    def __init__(self, model, sequences, max_new_tokens=32, method="cube", cost_model=None, fused_glue=None,
                 prefill="request"):
        if prefill not in ("request", "tree"):
            raise ValueError("prefill must be 'request' or 'tree'")
        self.model = model
        self.sequences = [list(s) for s in sequences]
        self.tree = KVTree.from_sequences(self.sequences)
        self.method = method
        self.cost_model = cost_model or CostModel()
        self.device = next(model.parameters()).device
        if fused_glue is None:  # the fused launch covers bf16 / fp16 models on the GPU
            fused_glue = self.device.type == "cuda" and model.dtype in (torch.bfloat16, torch.float16)
        self.fused_glue = fused_glue
        cfg = model.config
        self.hq = cfg.num_attention_heads
        self.hk = cfg.num_key_value_heads
        self.dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.original = [layer.self_attn.forward for layer in model.model.layers]
        self.max_new_tokens = max_new_tokens
        self.prefix_size = self.tree.storage_tokens
        self.used = self.prefix_size
        self.capacity = self.prefix_size + len(self.sequences) * max_new_tokens
        self.generated = 0
        dtype = model.dtype
        # pools are allocated 8-token aligned (the kernels' fast path); positions
        # past `capacity` are never written or read
        alloc = (self.capacity + 7) // 8 * 8
        self.pools = [(torch.empty((self.hk, self.dim, alloc), device=self.device, dtype=dtype),
                       torch.empty((self.hk, alloc, self.dim), device=self.device, dtype=dtype))
                      for _ in model.model.layers]
        self.leaves = [_find_leaf(self.tree, r) for r in range(len(self.sequences))]
        self._prefill_tree() if prefill == "tree" else self._prefill()

    # -------------------------------------------------------------- prefill
    @torch.inference_mode()
    def _prefill(self):
        """Run each prompt once and scatter its not-yet-written K/V into the pools (qwen.py:34-51)."""
        written = set()
        last = []
        for r, seq in enumerate(self.sequences):
            out = self.model(torch.tensor([seq], device=self.device), use_cache=True)
            last.append(out.logits[0, -1].clone())
            path = self.tree.paths[r]
            fresh = [i for i, pos in enumerate(path) if pos not in written]
            if fresh:
                src = torch.tensor(fresh, device=self.device)
                dst = torch.tensor([path[i] for i in fresh], device=self.device)
                for (kp, vp), layer in zip(self.pools, out.past_key_values.layers):
                    # cache tensors are [batch, HK, positions, D]
                    kp.index_copy_(2, dst, layer.keys[0].index_select(1, src).transpose(1, 2))
                    vp.index_copy_(1, dst, layer.values[0].index_select(1, src))
            written.update(path)
        self.logits = torch.stack(last)

    @torch.inference_mode()
    def _prefill_tree(self, leaf_batch=16):
        """Prefill every tree node once, in depth-first order, over its ancestors' cached K/V.

        The reference prefills each request's whole prompt and keeps the first
        copy of every shared position (qwen.py:34-51): work grows with the sum
        of the prompt lengths.  Here a node's tokens run through the model once,
        attending to the cache of the chain above it, so work grows with the
        stored tokens.  Childless siblings run together, up to ``leaf_batch``
        per forward, right-padded to the longest over the parent's cache
        repeated per row (causal attention keeps every real token from the pads
        after it).  After a node's subtree the cache is cut back to the node's
        start.  A request's logits are those of the last token of its terminal
        node.  Positions, causal masking and RoPE are those of the full prompt;
        only the floating-point order of the reductions differs from one full
        forward per request.
        """
        from transformers import DynamicCache

        nodes = self.tree.nodes
        last = [None] * len(self.sequences)
        cache = DynamicCache()

        def cut(cache, base):
            held = cache.get_seq_length()
            if base == 0:
                return DynamicCache()
            if held > base:
                cache.crop(base - held)  # drop the tokens after base
            return cache

        stack = [(0, False, 0)]  # (node, subtree done, cache length before the node)
        while stack:
            v, done, base = stack.pop()
            node = nodes[v]
            if done:
                cache = cut(cache, base)
                continue
            if node.tokens:
                cache = self._prefill_nodes([v], base, cache, last)
            stack.append((v, True, base))
            held = base + len(node.tokens)
            leaves = [c for c in node.children if not nodes[c].children]
            for i in range(0, len(leaves), leaf_batch):
                cache = self._prefill_nodes(leaves[i:i + leaf_batch], held, cache, last)
                cache = cut(cache, held)
            for c in reversed(node.children):
                if nodes[c].children:
                    stack.append((c, False, held))
        self.logits = torch.stack(last)

    def _prefill_nodes(self, group, base, cache, last):
        """One forward of sibling nodes ``group`` over a batch-1 cache of ``base`` tokens.

        Writes the nodes' K/V into the pools and their terminal requests' logits
        into ``last``; returns the cache, extended by the group's tokens (batch
        rows = group members; a one-node group leaves it ready for the node's
        children).
        """
        nodes, ids, dev = self.tree.nodes, self.tree.token_ids, self.device
        lens = [len(nodes[c].tokens) for c in group]
        width = max(lens)
        batch = torch.zeros((len(group), width), dtype=torch.long)
        for i, c in enumerate(group):
            batch[i, :lens[i]] = torch.tensor([ids[p] for p in nodes[c].tokens])
        if len(group) > 1:
            cache.batch_repeat_interleave(len(group))
        ends = sorted({n - 1 for n in lens})
        keep = torch.tensor(ends, device=dev)
        out = self.model(input_ids=batch.to(dev), past_key_values=cache, use_cache=True, logits_to_keep=keep)
        cache = out.past_key_values
        for i, c in enumerate(group):
            n = lens[i]
            dst = torch.tensor(nodes[c].tokens, device=dev)
            for (kp, vp), layer in zip(self.pools, cache.layers):
                # cache tensors are [batch, HK, positions, D]; this node's are [base, base + n)
                kp.index_copy_(2, dst, layer.keys[i, :, base:base + n].transpose(1, 2))
                vp.index_copy_(1, dst, layer.values[i, :, base:base + n])
            for r in nodes[c].terminal:
                last[r] = out.logits[i, ends.index(n - 1)].clone()
        if len(group) > 1:
            cache.batch_select_indices(torch.tensor([0], device=dev))
        return cache

    # ------------------------------------------------------------ decoding
    def _step_slots(self, count):
        """Pool slots of this step's tokens: one per request, in its reserved tail (qwen.py:53-56).
        Computes them without changing any state."""
        return [self.prefix_size + r * self.max_new_tokens + self.generated for r in range(count)]

    def _next_positions(self, count):
        slots = self._step_slots(count)
        self.generated += 1
        return slots

    def _check_append(self, count):
        if self.used + count > self.capacity:
            raise ValueError("Decode exceeds allocated max_new_tokens")

    def _prepare_plan(self):
        plan = schedule(self.tree, self.hq, self.hk, self.dim, self.method, self.cost_model)
        shape_of_q = torch.empty((len(self.sequences), self.hq, self.dim), device=self.device,
                                 dtype=self.model.dtype)
        return prepare(plan, shape_of_q)

    def _append(self, token_ids):
        self._check_append(len(token_ids))
        slots = self._next_positions(len(token_ids))
        for seq, tok in zip(self.sequences, token_ids):
            seq.append(tok)
        self.tree.extend_leaves(self.leaves, slots)
        self.used += len(token_ids)
        return slots

    @torch.inference_mode()
    def step(self, token_ids):
        """Append one token per request and return next-token logits ``[R, vocab]`` (qwen.py:74-103)."""
        token_ids = list(token_ids)
        if len(token_ids) != len(self.sequences):
            raise ValueError("step needs exactly one token per request")
        rope_pos = torch.tensor([[len(s)] for s in self.sequences], device=self.device)
        # every check before any state changes: a refused step leaves the decoder as it was
        self._check_append(len(token_ids))
        cap = self.pools[0][0].shape[2]
        planned = self._step_slots(len(token_ids))
        if not all(0 <= p < cap for p in planned):  # host data: the fused kernel would skip them silently
            raise ValueError(f"pool slots {planned} outside the pool capacity {cap}")
        positions = self._append(token_ids)
        slots = torch.tensor(positions, device=self.device, dtype=torch.int32)
        prepared = self._prepare_plan()
        ids = torch.tensor(token_ids, device=self.device)[:, None]
        self.logits = self._forward(ids, rope_pos, slots, prepared)
        return self.logits

    def _forward(self, ids, rope_pos, slots, prepared, **model_kwargs):
        """The model's forward over one token per request, each layer's attention swapped for one
        that writes the step's RoPE'd K/V into pool ``slots`` and attends the pools with
        ``prepared``; returns the logits ``[R, vocab]``."""
        pools = self.pools
        nreq = ids.shape[0]
        fused = self.fused_glue

        def forward(module, hidden_states, position_embeddings, attention_mask=None, **kwargs):
            shape = (*hidden_states.shape[:-1], -1, module.head_dim)
            # projections of this step: [R, 1, heads, D]
            q = module.q_norm(module.q_proj(hidden_states).view(shape))
            k = module.k_norm(module.k_proj(hidden_states).view(shape))
            v = module.v_proj(hidden_states).view(shape)
            kp, vp = pools[module.layer_idx]
            if fused:
                q = decode_append(q, k, v, *position_embeddings, slots, kp, vp)
            else:
                q, k = apply_rotary_pos_emb(q.transpose(1, 2), k.transpose(1, 2), *position_embeddings)
                v = v.transpose(1, 2)
                # q, k, v: [R, heads, 1, D] -> pool slots of this step
                kp.index_copy_(2, slots.long(), k[:, :, 0, :].permute(1, 2, 0))
                vp.index_copy_(1, slots.long(), v[:, :, 0, :].permute(1, 0, 2))
                q = q[:, :, 0, :].contiguous()
            attn = attention_matrix(q, kp, vp, prepared)
            return module.o_proj(attn.reshape(nreq, 1, -1)), None

        layers = self.model.model.layers
        for layer in layers:
            layer.self_attn.forward = MethodType(forward, layer.self_attn)
        try:
            out = self.model(ids, position_ids=rope_pos, use_cache=False, **model_kwargs)
            return out.logits[:, 0]
        finally:
            for layer, original in zip(layers, self.original):
                layer.self_attn.forward = original


class CachedPrefixDecoder(SharedKVDecoder):
    """Plans the prompt tree once; each step only sets the decode-tail lengths (qwen.py:106-124).

    ``graph=True`` (a bf16 / fp16 model on the GPU) runs the first step's forward eagerly, then
    captures it in a HIP graph over fixed input buffers (token ids, RoPE positions, pool slots)
    and the plan's fixed metadata; every later step writes its inputs into those buffers, sets
    the tails' lengths on the device and replays the graph.  The logits are bit-identical to
    the eager steps'; the host no longer launches each of the model's kernels.  The argument
    has no counterpart in the reference.
    """

    def __init__(self, model, sequences, max_new_tokens=32, method="cube", cost_model=None, fused_glue=None,
                 prefill="request", graph=False):
        super().__init__(model, sequences, max_new_tokens, method, cost_model, fused_glue, prefill)
        if graph and not (self.device.type == "cuda" and self.fused_glue):
            raise ValueError("graph=True needs a bfloat16 or float16 model on the GPU (the fused decode glue)")
        prompt_plan = schedule(self.tree, self.hq, self.hk, self.dim, self.method, self.cost_model)
        shape_of_q = torch.empty((len(self.sequences), self.hq, self.dim), device=self.device,
                                 dtype=model.dtype)
        self.cached_plan = CachedDecodePlan(prompt_plan, shape_of_q, self.prefix_size, max_new_tokens)
        self.graph = graph
        self._replay = None  # (graph, ids, positions, slots, logits) once captured

    @torch.inference_mode()
    def step(self, token_ids):
        if not self.graph:
            return super().step(token_ids)
        token_ids = list(token_ids)
        nreq = len(self.sequences)
        if len(token_ids) != nreq:
            raise ValueError("step needs exactly one token per request")
        self._check_append(nreq)
        cap = self.pools[0][0].shape[2]
        planned = self._step_slots(nreq)
        if not all(0 <= p < cap for p in planned):
            raise ValueError(f"pool slots {planned} outside the pool capacity {cap}")
        ids = torch.tensor(token_ids, device=self.device)[:, None]
        rope_pos = torch.tensor([[len(s)] for s in self.sequences], device=self.device)
        slots = torch.tensor(planned, device=self.device, dtype=torch.int32)
        self._append(token_ids)
        prepared = self._prepare_plan()  # the tails' lengths, set on the device in stream order
        # the masks of every layer type, none built: the swapped attention takes none
        no_mask = {t: None for t in set(self.model.config.layer_types)}
        if self._replay is None:
            logits = self._forward(ids, rope_pos, slots, prepared, attention_mask=no_mask)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self._forward(ids, rope_pos, slots, prepared, attention_mask=no_mask)
            self._replay = (graph, ids, rope_pos, slots, out)
        else:
            graph, ids_buf, pos_buf, slots_buf, out = self._replay
            ids_buf.copy_(ids)
            pos_buf.copy_(rope_pos)
            slots_buf.copy_(slots)
            graph.replay()
            logits = out
        self.logits = logits.clone()
        return self.logits

    def _check_append(self, count):
        if self.generated >= self.max_new_tokens:
            raise ValueError("Decode exceeds allocated max_new_tokens")

    def _append(self, token_ids):
        self._check_append(len(token_ids))
        slots = self._next_positions(len(token_ids))
        for seq, tok in zip(self.sequences, token_ids):
            seq.append(tok)
        self.used += len(token_ids)
        return slots

    def _prepare_plan(self):
        return self.cached_plan.update(self.generated)
