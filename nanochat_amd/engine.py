"""KV cache and inference engine with nanochat's interfaces, MI355X-native.

``KVCache`` keeps the surface of nanochat/engine.py:82-137 (attributes
k_cache, v_cache, cache_seqlens, prev_embedding, n_layers, max_seq_len and the
methods reset / get_pos / get_layer_cache / advance / prefill).  The fan-out
copy in ``prefill`` is one HIP launch (nc_kv_fanout) that reads the prefilled
row once and writes it into every destination row, K and V of all layers,
and sets cache_seqlens on the device.

``Engine`` (generate / generate_batch), ``sample_next_token``, ``RowState``
and ``use_calculator`` are the driver of nanochat/engine.py:25-304: one
batch-1 prefill, fan-out to num_samples rows, then the decode loop with the
per-row tool-use state machine.
"""
from __future__ import annotations

import ast
import ctypes
import operator
from collections import deque

import torch
import torch.nn.functional as F

from . import _ext
from . import sampling as gpu_sampling


class KVCache:
    """Preallocated (L, B, T, H_kv, D) K and V caches plus per-row positions.

    Layout and dtype follow nanochat/engine.py:92-104: zero-filled, contiguous,
    layer outermost, so ``get_layer_cache(l)`` returns (B, T, H_kv, D) views
    that flash_attn_with_kvcache updates in place.
    """

    def __init__(self, batch_size, num_heads, seq_len, head_dim, num_layers, device, dtype):
        self.batch_size = batch_size
        self.max_seq_len = seq_len
        self.n_layers = num_layers
        self.n_heads = num_heads
        self.head_dim = head_dim
        shape = (num_layers, batch_size, seq_len, num_heads, head_dim)
        self.k_cache = torch.zeros(shape, device=device, dtype=dtype)
        self.v_cache = torch.zeros(shape, device=device, dtype=dtype)
        self.cache_seqlens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self.prev_embedding = None

    def reset(self):
        """Positions back to 0 (cache bytes are kept), nanochat/engine.py:106-109."""
        self.cache_seqlens.zero_()
        self.prev_embedding = None

    def get_pos(self):
        """Row 0's position (uniform-batch assumption of nanochat/engine.py:111-113).

        On the GPU this host read also carries the kernels' device error flag (the same single
        copy), and a set flag raises RuntimeError here: e.g. an append past the cache length,
        which the reference's slice assignment rejects at the call (flash_attention.py:160-162).
        """
        if self.cache_seqlens.is_cuda:
            vals, bits = _ext.host_values_and_errors(self.cache_seqlens[:1])
            _ext.raise_device_errors(bits, "KV-cache path")
            return vals[0]
        return self.cache_seqlens[0].item()

    def get_layer_cache(self, layer_idx):
        """(k_cache, v_cache) views of one layer, nanochat/engine.py:115-117."""
        return self.k_cache[layer_idx], self.v_cache[layer_idx]

    def advance(self, num_tokens):
        """cache_seqlens += num_tokens on the device, nanochat/engine.py:119-121."""
        self.cache_seqlens += num_tokens

    def prefill(self, other):
        """Copy other's first get_pos() positions into every row of this cache.

        Preconditions and effects of nanochat/engine.py:123-137: this cache is
        empty, layer/head/head_dim match, it is at least as long as `other`;
        afterwards every row holds other's row 0 prefix and cache_seqlens is
        other's position.  K and V of all layers move in one HIP launch.
        """
        assert self.get_pos() == 0, "Cannot prefill a non-empty KV cache"
        assert self.n_layers == other.n_layers and self.n_heads == other.n_heads and self.head_dim == other.head_dim
        assert self.max_seq_len >= other.max_seq_len
        other_pos = other.get_pos()
        if not 0 <= other_pos <= other.max_seq_len:
            raise ValueError(f"KVCache.prefill: source position {other_pos} outside [0, {other.max_seq_len}]")
        src_k, src_v, dst_k, dst_v = other.k_cache, other.v_cache, self.k_cache, self.v_cache
        dev = dst_k.device
        if dev.type != "cuda" or src_k.device != dev:
            raise RuntimeError("KVCache.prefill: the fan-out copy runs on the GPU only (both caches on one GPU)")
        if src_k.dtype != dst_k.dtype:
            raise TypeError(f"KVCache.prefill: cache dtypes differ ({src_k.dtype} vs {dst_k.dtype})")
        for t in (src_k, src_v, dst_k, dst_v):
            if not t.is_contiguous():
                raise ValueError("KVCache.prefill: caches must be contiguous")
        a = _ext.FanoutArgs()
        a.k_src, a.v_src = src_k.data_ptr(), src_v.data_ptr()
        a.k_dst, a.v_dst = dst_k.data_ptr(), dst_v.data_ptr()
        a.dst_seqlens = self.cache_seqlens.data_ptr()
        a.n_layers = self.n_layers
        a.n_rows = self.batch_size
        a.prefix_len = other_pos
        a.row_elems = self.n_heads * self.head_dim
        a.src_stride_l = src_k.stride(0)
        a.dst_stride_l = dst_k.stride(0)
        a.dst_stride_b = dst_k.stride(1)
        a.dtype = _ext.DTYPE_CODE[dst_k.dtype]
        _ext.check(_ext.lib().nc_kv_fanout(ctypes.byref(a), _ext.stream_handle(dev)), "nc_kv_fanout")
        if other.prev_embedding is not None:
            self.prev_embedding = other.prev_embedding.expand(self.batch_size, -1, -1).clone()


# ---------------------------------------------------------------------------
# Engine: the driver of the path (nanochat/engine.py:140-304).  Same
# allocation sizes, dtype rule, fan-out, per-row state machine and stop rules.
# ---------------------------------------------------------------------------
_ARITH = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv}
_UNARY = {ast.UAdd: operator.pos, ast.USub: operator.neg}
_MATH_CHARS = set("0123456789*+-/.() ")
_STRING_CHARS = set("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789'\"()._ ")
_BANNED = ("__", "import", "exec", "eval", "compile", "open", "file", "input", "raw_input", "globals", "locals",
           "vars", "dir", "getattr", "setattr", "delattr", "hasattr")


def _eval_node(node):
    if isinstance(node, ast.Expression):
        return _eval_node(node.body)
    if isinstance(node, ast.Constant) and type(node.value) in (int, float, str):
        return node.value
    if isinstance(node, ast.BinOp) and type(node.op) in _ARITH:
        return _ARITH[type(node.op)](_eval_node(node.left), _eval_node(node.right))
    if isinstance(node, ast.UnaryOp) and type(node.op) in _UNARY:
        return _UNARY[type(node.op)](_eval_node(node.operand))
    if (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute) and node.func.attr == "count"
            and not node.keywords and len(node.args) == 1):
        target, arg = _eval_node(node.func.value), _eval_node(node.args[0])
        if isinstance(target, str) and isinstance(arg, str):
            return target.count(arg)
    raise ValueError("unsupported expression")


def use_calculator(expr):
    """The calculator tool of nanochat/engine.py:46-79: arithmetic (+ - * / and
    parentheses, no power) or a string literal's .count(...); None when the
    expression is not allowed or does not evaluate.  Evaluated by walking the
    parsed expression over that closed set of node types (nothing is exec'd)."""
    expr = expr.replace(",", "")
    if all(c in _MATH_CHARS for c in expr):
        if "**" in expr:
            return None
    else:
        if not all(c in _STRING_CHARS for c in expr):
            return None
        lowered = expr.lower()
        if any(p in lowered for p in _BANNED) or ".count(" not in expr:
            return None
    try:
        return _eval_node(ast.parse(expr, mode="eval"))
    except Exception:
        return None


@torch.inference_mode()
def sample_next_token(logits, rng, temperature=1.0, top_k=None):
    """(B, vocab) logits -> (B, 1) ids; nanochat/engine.py:140-156."""
    assert temperature >= 0.0, "temperature must be non-negative"
    if temperature == 0.0:
        return torch.argmax(logits, dim=-1, keepdim=True)
    if top_k is not None and top_k > 0:
        k = min(top_k, logits.size(-1))
        vals, idx = torch.topk(logits, k, dim=-1)
        probs = F.softmax(vals / temperature, dim=-1)
        choice = torch.multinomial(probs, num_samples=1, generator=rng)
        return idx.gather(1, choice)
    probs = F.softmax(logits / temperature, dim=-1)
    return torch.multinomial(probs, num_samples=1, generator=rng)


class RowState:
    """Per-row generation state (tokens so far, forced tool tokens, python block)."""

    def __init__(self, current_tokens=None):
        self.current_tokens = current_tokens or []
        self.forced_tokens = deque()
        self.in_python_block = False
        self.python_expr_tokens = []
        self.completed = False


class GraphDecodeStep:
    """One decode forward of (B, 1) token ids replayed from a HIP graph.

    The first call runs eagerly on a side stream (library handles and the
    attention workspace of that stream get created); the second captures the
    forward and replays it; later calls only copy the ids in and replay.  The
    forward must not synchronise the host, which holds when the model runs the
    QK prologue inside the attention call (positions come from the device-side
    cache_seqlens; the cache advances in place).  The returned logits are the
    graph's output buffer, overwritten by the next call.
    """

    def __init__(self, model, cache, batch, device):
        self.model, self.cache = model, cache
        self.ids = torch.zeros((batch, 1), dtype=torch.long, device=device)
        self.stream = torch.cuda.Stream(device=device)
        self.graph = None
        self.logits = None
        self.calls = 0

    def __call__(self, ids):
        main = torch.cuda.current_stream()
        self.ids.copy_(ids)
        self.stream.wait_stream(main)
        if self.graph is None and self.calls == 0:
            with torch.cuda.stream(self.stream):
                out = self.model.forward(self.ids, kv_cache=self.cache)[:, -1, :]
        else:
            if self.graph is None:
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph, stream=self.stream):
                    self.logits = self.model.forward(self.ids, kv_cache=self.cache)[:, -1, :]
            with torch.cuda.stream(self.stream):
                self.graph.replay()
            out = self.logits
        main.wait_stream(self.stream)
        self.calls += 1
        return out


class Engine:
    """Batched generation with one prefill and a fanned-out KV cache."""

    def __init__(self, model, tokenizer, use_graph=None, fused_sampling=None, cache_dtype=None):
        self.model = model
        self.tokenizer = tokenizer
        # None: replay decode steps from a HIP graph whenever the model runs the fused QK prologue on the GPU
        self.use_graph = use_graph
        # Sampling on the GPU.  None (default): greedy steps (temperature 0) run the HIP kernel
        # (nc_sample's argmax is bit-identical to torch.argmax) and draws at temperature > 0 run
        # the reference's torch ops, so a seeded run draws the reference's torch.multinomial
        # stream.  True: draws run the kernel too (top_k up to 1024): the same distribution, one
        # torch.rand uniform per row from the same generator, hence a different stream of
        # tokens for a given seed.  False: torch's ops for every step.
        self.fused_sampling = fused_sampling
        # KV-cache dtype; None applies the reference's rule (bf16 on a GPU, fp32 elsewhere,
        # nanochat/engine.py:186).  Tests set float32 to compare with fp32 golden runs.
        self.cache_dtype = cache_dtype

    def _graph_decode(self, device):
        if device.type != "cuda" or not getattr(self.model, "fused_qk_prologue", False):
            return False
        return True if self.use_graph is None else bool(self.use_graph)

    @torch.inference_mode()
    def generate(self, tokens, num_samples=1, max_tokens=None, temperature=1.0, top_k=None, seed=42):
        """Yield (token_column, token_masks) per step; nanochat/engine.py:176-280."""
        assert isinstance(tokens, list) and isinstance(tokens[0], int), "expecting list of ints"
        device = self.model.get_device()
        dtype = torch.bfloat16 if device.type == "cuda" else torch.float32
        if self.cache_dtype is not None:
            dtype = self.cache_dtype
        rng = torch.Generator(device=device)
        rng.manual_seed(seed)
        special = self.tokenizer.encode_special
        python_start, python_end = special("<|python_start|>"), special("<|python_end|>")
        output_start, output_end = special("<|output_start|>"), special("<|output_end|>")
        assistant_end = special("<|assistant_end|>")
        bos = self.tokenizer.get_bos_token_id()

        m = self.model.config
        shape = dict(num_heads=m.n_kv_head, head_dim=m.n_embd // m.n_head, num_layers=m.n_layer)
        prefill_cache = KVCache(batch_size=1, seq_len=len(tokens), device=device, dtype=dtype, **shape)
        ids = torch.tensor([tokens], dtype=torch.long, device=device)
        logits = self.model.forward(ids, kv_cache=prefill_cache)
        logits = logits[:, -1, :].expand(num_samples, -1)

        decode_len = (len(tokens) + max_tokens) if max_tokens is not None else self.model.config.sequence_len
        cache = KVCache(batch_size=num_samples, seq_len=decode_len, device=device, dtype=dtype, **shape)
        cache.prefill(prefill_cache)
        del prefill_cache

        step = GraphDecodeStep(self.model, cache, num_samples, device) if self._graph_decode(device) else None
        if temperature == 0.0:
            fused = device.type == "cuda" and self.fused_sampling is not False
        else:   # draws: the kernel only on request, and for top_k it supports
            fused = (device.type == "cuda" and self.fused_sampling is True
                     and (top_k is None or top_k <= gpu_sampling.MAX_TOP_K))
        sampler = gpu_sampling.sample_next_token if fused else sample_next_token
        rows = [RowState(tokens.copy()) for _ in range(num_samples)]
        generated = 0
        while True:
            if max_tokens is not None and generated >= max_tokens:
                break
            if all(r.completed for r in rows):
                break
            next_ids = sampler(logits, rng, temperature, top_k)[:, 0]
            if next_ids.is_cuda:
                # the per-step host read of the ids also carries the kernels' error flag
                sampled, bits = _ext.host_values_and_errors(next_ids)
                _ext.raise_device_errors(bits, "Engine.generate")
            else:
                sampled = next_ids.tolist()
            column, masks = [], []
            for i, r in enumerate(rows):
                forced = len(r.forced_tokens) > 0
                masks.append(0 if forced else 1)
                tok = r.forced_tokens.popleft() if forced else sampled[i]
                column.append(tok)
                r.current_tokens.append(tok)
                if tok == assistant_end or tok == bos:
                    r.completed = True
                if tok == python_start:
                    r.in_python_block = True
                    r.python_expr_tokens = []
                elif tok == python_end and r.in_python_block:
                    r.in_python_block = False
                    if r.python_expr_tokens:
                        result = use_calculator(self.tokenizer.decode(r.python_expr_tokens))
                        if result is not None:
                            r.forced_tokens.append(output_start)
                            r.forced_tokens.extend(self.tokenizer.encode(str(result)))
                            r.forced_tokens.append(output_end)
                    r.python_expr_tokens = []
                elif r.in_python_block:
                    r.python_expr_tokens.append(tok)
            yield column, masks
            generated += 1
            ids = torch.tensor(column, dtype=torch.long, device=device).unsqueeze(1)
            logits = step(ids) if step is not None else self.model.forward(ids, kv_cache=cache)[:, -1, :]

    def generate_batch(self, tokens, num_samples=1, **kwargs):
        """Final sequences (terminal tokens dropped) and masks; nanochat/engine.py:282-304."""
        assistant_end = self.tokenizer.encode_special("<|assistant_end|>")
        bos = self.tokenizer.get_bos_token_id()
        results = [tokens.copy() for _ in range(num_samples)]
        masks = [[0] * len(tokens) for _ in range(num_samples)]
        completed = [False] * num_samples
        for column, column_masks in self.generate(tokens, num_samples, **kwargs):
            for i, (tok, mask) in enumerate(zip(column, column_masks)):
                if not completed[i]:
                    if tok == assistant_end or tok == bos:
                        completed[i] = True
                    else:
                        results[i].append(tok)
                        masks[i].append(mask)
            if all(completed):
                break
        return results, masks
