"""nanochat's GPT, inference side: the caller of the KV-cache path.

This is the model half of the end-to-end checks (C1 greedy tokens at d12, C3
generate at d24).  It computes exactly what nanochat/gpt.py computes -- the
same parameters, initialisation sequence and float operations in the same
order -- so a CPU run matches the reference bit for bit, and on the GPU its
attention goes through nanochat_amd.flash_attention (libnc_kv.so):

  - CausalSelfAttention with a cache (nanochat/gpt.py:82-126): q/k/v
    projections, gated value embeddings, rotary, QK RMS norm, x1.2, then
    flash_attn_with_kvcache; the last layer advances the cache by T.  On the
    GPU the rotary/norm/x1.2 prologue runs inside the cache call
    (flash_attn_with_kvcache_rope, positions from cache_seqlens) unless
    GPT.fused_qk_prologue is False; on the CPU the op-by-op sequence runs.
  - GPT.forward (nanochat/gpt.py:416-481): rotary offset T0 = kv_cache.get_pos(),
    smear with the cached previous embedding, resid/x0 lambdas, backout at
    n_layer // 2, final norm, lm_head, softcap 15.
  - window sizes (nanochat/gpt.py:285-312) and the naive no-cache generate
    (nanochat/gpt.py:483-512, the reference's own consistency oracle).
Training (loss, optimizer set-up, FLOP counts) is not part of this build.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import linear as small_m
from .common import COMPUTE_DTYPE
from .flash_attention import flash_attn


@dataclass
class GPTConfig:
    sequence_len: int = 2048
    vocab_size: int = 32768
    n_layer: int = 12
    n_head: int = 6
    n_kv_head: int = 6
    n_embd: int = 768
    window_pattern: str = "SSSL"


def rms(x):
    """Parameter-free RMS norm over the last dimension."""
    return F.rms_norm(x, (x.size(-1),))


# Decode-sized block projections (at most 16 rows, K <= 2048, inference) run on the library's
# small-M kernel where it measured faster than the library GEMM (nanochat_amd.linear.
# prefer_for_projection); False keeps F.linear for every projection.
SMALL_M_PROJECTIONS = True


class CastLinear(nn.Linear):
    """Bias-free linear whose fp32 master weight is cast to the activation dtype.

    Without autograd the cast is kept (keyed by dtype and the weight's version
    counter) instead of being redone on every call: the same values, without
    re-reading the fp32 weights each decode step.
    """

    def weight_as(self, dtype):
        """The weight in `dtype` (kept between calls when autograd is off)."""
        if torch.is_grad_enabled() or self.weight.dtype == dtype:
            return self.weight.to(dtype=dtype)
        key = (dtype, self.weight._version, self.weight.data_ptr())
        cached = getattr(self, "_cast", None)
        if cached is None or cached[0] != key:
            cached = (key, self.weight.to(dtype=dtype))
            self._cast = cached
        return cached[1]

    def forward(self, x):
        w = self.weight_as(x.dtype)
        if SMALL_M_PROJECTIONS and small_m.prefer_for_projection(x, w):
            return small_m.linear(x, w)
        return F.linear(x, w)


def carries_value_embedding(layer, n_layer):
    """Alternate layers carry a value embedding; the last layer always does."""
    return layer % 2 == (n_layer - 1) % 2


def rotate_half_pairs(x, cos, sin):
    """Rotary embedding on (B, T, H, D): dims [0, D/2) and [D/2, D) are rotated as pairs."""
    half = x.shape[3] // 2
    a, b = x[..., :half], x[..., half:]
    return torch.cat([a * cos + b * sin, a * (-sin) + b * cos], 3)


def rotary_tables(seq_len, head_dim, base=100000, device=None, dtype=torch.float32):
    """cos/sin tables (seq_len, head_dim/2) of t * base^(-2i/D), built in fp32 and cast to dtype."""
    channels = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device)
    inv_freq = 1.0 / (base ** (channels / head_dim))
    t = torch.arange(seq_len, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def window_sizes(config: GPTConfig):
    """Per-layer (left, right) windows: L = sequence_len, S = ceil(seq/4 to 128); last layer L."""
    pattern = config.window_pattern.upper()
    if not pattern or any(c not in "SL" for c in pattern):
        raise ValueError(f"Invalid window_pattern: {pattern}. Use only S and L.")
    long_w = config.sequence_len
    short_w = -(-long_w // 4 // 128) * 128
    sizes = [(long_w if pattern[i % len(pattern)] == "L" else short_w, 0) for i in range(config.n_layer)]
    sizes[-1] = (long_w, 0)
    return sizes


class FusedRope(NamedTuple):
    """Whole rotary tables handed to attention when the QK prologue runs inside the cache call.

    fuse_qkv: bf16/fp16 layers compute q, k and v with one GEMM against the concatenated
    c_q/c_k/c_v weights; q, k, v are strided views of its output (the cache call takes them as is).
    """
    cos: torch.Tensor
    sin: torch.Tensor
    fuse_qkv: bool = False


class CausalSelfAttention(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.layer_idx = layer_idx
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.head_dim = config.n_embd // config.n_head
        assert config.n_embd % config.n_head == 0
        assert config.n_kv_head <= config.n_head and config.n_head % config.n_kv_head == 0
        self.c_q = CastLinear(config.n_embd, self.n_head * self.head_dim, bias=False)
        self.c_k = CastLinear(config.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_v = CastLinear(config.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_proj = CastLinear(config.n_embd, config.n_embd, bias=False)
        self.ve_gate_channels = 12
        self.ve_gate = (CastLinear(self.ve_gate_channels, self.n_kv_head, bias=False)
                        if carries_value_embedding(layer_idx, config.n_layer) else None)

    def qkv_weight(self, dtype):
        """cat(c_q, c_k, c_v) weights in `dtype` (kept between calls while the weights are unchanged)."""
        mods = (self.c_q, self.c_k, self.c_v)
        key = (dtype,) + tuple((m.weight.data_ptr(), m.weight._version) for m in mods)
        cached = getattr(self, "_qkv", None)
        if torch.is_grad_enabled() or cached is None or cached[0] != key:
            cached = (key, torch.cat([m.weight_as(dtype) for m in mods], dim=0))
            self._qkv = cached
        return cached[1]

    def forward(self, x, ve, cos_sin, window_size, kv_cache):
        B, T, _ = x.size()
        if isinstance(cos_sin, FusedRope) and cos_sin.fuse_qkv and x.dtype in (torch.bfloat16, torch.float16):
            w = self.qkv_weight(x.dtype)
            if SMALL_M_PROJECTIONS and small_m.prefer_for_projection(x, w):
                qkv = small_m.linear(x, w)
            else:
                qkv = F.linear(x, w)
            nq, nk = self.n_head * self.head_dim, self.n_kv_head * self.head_dim
            q = qkv[..., :nq].view(B, T, self.n_head, self.head_dim)
            k = qkv[..., nq:nq + nk].view(B, T, self.n_kv_head, self.head_dim)
            v = qkv[..., nq + nk:].view(B, T, self.n_kv_head, self.head_dim)
        else:
            q = self.c_q(x).view(B, T, self.n_head, self.head_dim)
            k = self.c_k(x).view(B, T, self.n_kv_head, self.head_dim)
            v = self.c_v(x).view(B, T, self.n_kv_head, self.head_dim)
        if ve is not None:
            ve = ve.view(B, T, self.n_kv_head, self.head_dim)
            gate = 3 * torch.sigmoid(self.ve_gate(x[..., :self.ve_gate_channels]))
            v = v + gate.unsqueeze(-1) * ve
        if isinstance(cos_sin, FusedRope):
            # rotary at each row's cache position + QK norm + x1.2 inside the attention call
            k_cache, v_cache = kv_cache.get_layer_cache(self.layer_idx)
            y = flash_attn.flash_attn_with_kvcache_rope(q, k_cache, v_cache, k, v, kv_cache.cache_seqlens,
                                                        cos_sin.cos, cos_sin.sin, causal=True,
                                                        window_size=window_size)
            if self.layer_idx == kv_cache.n_layers - 1:
                kv_cache.advance(T)
            return self.c_proj(y.contiguous().view(B, T, -1))
        cos, sin = cos_sin
        q, k = rotate_half_pairs(q, cos, sin), rotate_half_pairs(k, cos, sin)
        q, k = rms(q), rms(k)
        q = q * 1.2
        k = k * 1.2
        if kv_cache is None:
            y = flash_attn.flash_attn_func(q, k, v, causal=True, window_size=window_size)
        else:
            k_cache, v_cache = kv_cache.get_layer_cache(self.layer_idx)
            y = flash_attn.flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v,
                                                   cache_seqlens=kv_cache.cache_seqlens, causal=True,
                                                   window_size=window_size)
            if self.layer_idx == kv_cache.n_layers - 1:
                kv_cache.advance(T)
        return self.c_proj(y.contiguous().view(B, T, -1))


class MLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.c_fc = CastLinear(config.n_embd, 4 * config.n_embd, bias=False)
        self.c_proj = CastLinear(4 * config.n_embd, config.n_embd, bias=False)

    def forward(self, x):
        return self.c_proj(F.relu(self.c_fc(x)).square())


class Block(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.attn = CausalSelfAttention(config, layer_idx)
        self.mlp = MLP(config)

    def forward(self, x, ve, cos_sin, window_size, kv_cache):
        x = x + self.attn(rms(x), ve, cos_sin, window_size, kv_cache)
        x = x + self.mlp(rms(x))
        return x


class GPT(nn.Module):
    """Build under `torch.device("meta")`, then `to_empty(device=...)` and `init_weights()`."""

    def __init__(self, config: GPTConfig, pad_vocab_size_to: int = 64, compute_dtype=None):
        super().__init__()
        self.config = config
        self.compute_dtype = compute_dtype if compute_dtype is not None else COMPUTE_DTYPE
        self.window_sizes = window_sizes(config)
        padded = -(-config.vocab_size // pad_vocab_size_to) * pad_vocab_size_to
        self.transformer = nn.ModuleDict({
            "wte": nn.Embedding(padded, config.n_embd),
            "h": nn.ModuleList([Block(config, i) for i in range(config.n_layer)]),
        })
        self.lm_head = CastLinear(config.n_embd, padded, bias=False)
        self.resid_lambdas = nn.Parameter(torch.ones(config.n_layer))
        self.x0_lambdas = nn.Parameter(torch.zeros(config.n_layer))
        self.smear_gate = CastLinear(24, 1, bias=False)
        self.smear_lambda = nn.Parameter(torch.zeros(1))
        self.backout_lambda = nn.Parameter(0.2 * torch.ones(1))
        head_dim = config.n_embd // config.n_head
        kv_dim = config.n_kv_head * head_dim
        self.value_embeds = nn.ModuleDict({str(i): nn.Embedding(padded, kv_dim) for i in range(config.n_layer)
                                           if carries_value_embedding(i, config.n_layer)})
        self.rotary_seq_len = config.sequence_len * 10
        cos, sin = self._rotary_tables(self.rotary_seq_len, head_dim)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def _rotary_tables(self, seq_len, head_dim, base=100000, device=None):
        if device is None:
            device = self.transformer.wte.weight.device
        cos, sin = rotary_tables(seq_len, head_dim, base, device, self.compute_dtype)
        return cos[None, :, None, :], sin[None, :, None, :]

    @torch.no_grad()
    def init_weights(self):
        """nanochat's initialisation, same distributions and the same order of RNG draws."""
        torch.nn.init.normal_(self.transformer.wte.weight, mean=0.0, std=0.8)
        torch.nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)
        n_embd = self.config.n_embd
        s = 3 ** 0.5 * n_embd ** -0.5
        for block in self.transformer.h:
            torch.nn.init.uniform_(block.attn.c_q.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_k.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_v.weight, -s, s)
            torch.nn.init.zeros_(block.attn.c_proj.weight)
            torch.nn.init.uniform_(block.mlp.c_fc.weight, -s * 0.4, s * 0.4)
            torch.nn.init.zeros_(block.mlp.c_proj.weight)
        n_layer = self.config.n_layer
        for i in range(n_layer):
            self.resid_lambdas.data[i] = 1.15 - (0.10 * i / max(n_layer - 1, 1))
        for i in range(n_layer):
            self.x0_lambdas.data[i] = 0.20 - (0.15 * i / max(n_layer - 1, 1))
        torch.nn.init.zeros_(self.smear_lambda)
        torch.nn.init.constant_(self.backout_lambda, 0.2)
        torch.nn.init.uniform_(self.smear_gate.weight, 0.0, 0.02)
        for ve in self.value_embeds.values():
            torch.nn.init.uniform_(ve.weight, -s, s)
        for block in self.transformer.h:
            if block.attn.ve_gate is not None:
                torch.nn.init.uniform_(block.attn.ve_gate.weight, 0.0, 0.02)
        cos, sin = self._rotary_tables(self.rotary_seq_len, n_embd // self.config.n_head)
        self.cos, self.sin = cos, sin
        if self.compute_dtype != torch.float16:
            self.transformer.wte.to(dtype=self.compute_dtype)
            for ve in self.value_embeds.values():
                ve.to(dtype=self.compute_dtype)

    def get_device(self):
        return self.transformer.wte.weight.device

    # With a KV cache on the GPU, rotary + QK norm + x1.2 run inside the attention call
    # (flash_attn_with_kvcache_rope), which takes positions from the device-side
    # cache_seqlens: no get_pos() host sync and ~10 fewer launches per layer.  False
    # keeps the reference's op-by-op sequence.
    fused_qk_prologue = True
    # Decode-sized logits heads (CUDA, bf16/fp16, at most 64 rows) run lm_head, the vocabulary
    # slice, the fp32 cast and the softcap as one kernel (nanochat_amd.linear.logits_head).  The
    # logits are the same up to the GEMM's summation order (bf16-rounded as the reference's);
    # False keeps F.linear and torch's softcap.
    fused_logits_head = True
    # With the fused QK prologue, bf16/fp16 attention layers compute q, k, v with one GEMM (three
    # launches become one); False keeps c_q, c_k, c_v as separate F.linear calls.
    fused_qkv_projection = True

    def forward(self, idx, kv_cache=None):
        """Logits (B, T, vocab) in fp32.  With a cache, attention appends into it."""
        B, T = idx.size()
        assert T <= self.cos.size(1), f"Sequence length grew beyond the rotary table: {T} > {self.cos.size(1)}"
        if kv_cache is not None and self.fused_qk_prologue and idx.is_cuda:
            # positions beyond the table set a device flag
            cos_sin = FusedRope(self.cos, self.sin, self.fused_qkv_projection)
        else:
            T0 = 0 if kv_cache is None else kv_cache.get_pos()
            cos_sin = self.cos[:, T0:T0 + T], self.sin[:, T0:T0 + T]
        x = self.transformer.wte(idx)
        x = x.to(self.compute_dtype)
        x = rms(x)
        if kv_cache is None:
            assert T > 1, "no-cache forward needs T > 1"
            gate = self.smear_lambda.to(x.dtype) * torch.sigmoid(self.smear_gate(x[:, 1:, :24]))
            x = torch.cat([x[:, :1], x[:, 1:] + gate * x[:, :-1]], dim=1)
        else:
            prev = kv_cache.prev_embedding
            last = x[:, -1:, :]
            if T > 1:
                gate = self.smear_lambda.to(x.dtype) * torch.sigmoid(self.smear_gate(x[:, 1:, :24]))
                x = torch.cat([x[:, :1], x[:, 1:] + gate * x[:, :-1]], dim=1)
            elif prev is not None:
                gate = self.smear_lambda.to(x.dtype) * torch.sigmoid(self.smear_gate(x[:, :, :24]))
                x = x + gate * prev
            # this step's last (pre-smear) embedding for the next step; a buffer of the same shape is
            # updated in place after its last read, so a graph-captured decode step stays correct
            if prev is not None and prev.shape == last.shape and prev.dtype == last.dtype:
                prev.copy_(last)
            else:
                kv_cache.prev_embedding = last
        x0 = x
        n_layer = self.config.n_layer
        backout_at = n_layer // 2
        x_backout = None
        for i, block in enumerate(self.transformer.h):
            x = self.resid_lambdas[i] * x + self.x0_lambdas[i] * x0
            key = str(i)
            ve = self.value_embeds[key](idx).to(x.dtype) if key in self.value_embeds else None
            x = block(x, ve, cos_sin, self.window_sizes[i], kv_cache)
            if i == backout_at:
                x_backout = x
        if x_backout is not None:
            x = x - self.backout_lambda.to(x.dtype) * x_backout
        x = rms(x)
        softcap = 15
        if self.fused_logits_head and x.is_cuda:
            w = self.lm_head.weight_as(x.dtype)
            if small_m.supported(x, w):
                return small_m.logits_head(x, w, self.config.vocab_size, softcap)
        logits = self.lm_head(x)[..., :self.config.vocab_size].float()
        return softcap * torch.tanh(logits / softcap)

    @torch.inference_mode()
    def generate(self, tokens, max_tokens, temperature=1.0, top_k=None, seed=42):
        """Naive no-cache decoding of one sequence (the reference's consistency oracle)."""
        assert isinstance(tokens, list)
        device = self.get_device()
        rng = None
        if temperature > 0:
            rng = torch.Generator(device=device)
            rng.manual_seed(seed)
        ids = torch.tensor([tokens], dtype=torch.long, device=device)
        for _ in range(max_tokens):
            logits = self.forward(ids)[:, -1, :]
            if top_k is not None and top_k > 0:
                v, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                logits[logits < v[:, [-1]]] = -float("Inf")
            if temperature > 0:
                probs = F.softmax(logits / temperature, dim=-1)
                next_ids = torch.multinomial(probs, num_samples=1, generator=rng)
            else:
                next_ids = torch.argmax(logits, dim=-1, keepdim=True)
            ids = torch.cat((ids, next_ids), dim=1)
            yield next_ids.item()


def build_model(config: GPTConfig, device, compute_dtype=None, seed: int = 0) -> GPT:
    """Meta-construct, allocate on `device`, seed and initialise (nanochat's recipe)."""
    with torch.device("meta"):
        model = GPT(config, compute_dtype=compute_dtype)
    model.to_empty(device=device)
    torch.manual_seed(seed)
    model.init_weights()
    model.eval()
    return model
