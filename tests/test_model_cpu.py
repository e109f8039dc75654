"""The model and engine counterparts (nanochat_amd/gpt.py, nanochat_amd/engine.py)
against golden vectors from nanochat's own GPT (tests/golden/make_c1_golden.py).

Runs on the CPU in fp32 with the oracle's attention and KV cache standing in
for the HIP library, so it pins the caller side of the path -- rotary offset,
QK norm, value embeddings, smear state, backout, softcap, the engine's
prefill / fan-out / decode order -- bit for bit: the K/V cache bytes of every
layer must hash to the reference's.  The GPU run of the same model through
libnc_kv.so is tests/test_gpu_e2e.py.
"""
import hashlib
import json
from types import SimpleNamespace

import pytest
import torch

import nanochat_amd.engine as eng
import nanochat_amd.gpt as gpt
from oracle import kvcache_oracle as orc
from tests.conftest import ROOT

GOLDEN = json.loads((ROOT / "tests" / "golden" / "c1_d12_seed0.json").read_text())
D12 = gpt.GPTConfig(sequence_len=1024, vocab_size=32768, n_layer=12, n_head=6, n_kv_head=6, n_embd=768,
                    window_pattern="L")


def c1_model(variant, device="cpu"):
    model = gpt.build_model(D12, device, compute_dtype=torch.float32, seed=0)
    if variant == "perturbed":
        torch.manual_seed(1)
        with torch.no_grad():
            for block in model.transformer.h:
                torch.nn.init.normal_(block.attn.c_proj.weight, mean=0.0, std=0.02)
                torch.nn.init.normal_(block.mlp.c_proj.weight, mean=0.0, std=0.02)
            model.smear_lambda.fill_(0.5)
    return model


class SpecialTokens:
    """Stand-in tokenizer: nanochat appends 9 special tokens at the end of the vocab."""

    def __init__(self, vocab=32768):
        names = ["<|bos|>", "<|user_start|>", "<|user_end|>", "<|assistant_start|>", "<|assistant_end|>",
                 "<|python_start|>", "<|python_end|>", "<|output_start|>", "<|output_end|>"]
        self.ids = {n: vocab - 9 + i for i, n in enumerate(names)}

    def encode_special(self, s):
        return self.ids[s]

    def get_bos_token_id(self):
        return self.ids["<|bos|>"]

    def encode(self, s, prepend=None):
        return ([prepend] if prepend is not None else []) + [ord(c) for c in s]

    def decode(self, toks):
        return "".join(chr(t) for t in toks if t < 256)


@pytest.fixture
def oracle_path(monkeypatch):
    """Route the model's attention and the engine's cache through the oracle (CPU)."""
    monkeypatch.setattr(gpt, "flash_attn", SimpleNamespace(flash_attn_func=orc.flash_attn_func,
                                                          flash_attn_with_kvcache=orc.flash_attn_with_kvcache))
    monkeypatch.setattr(eng, "KVCache", orc.KVCache)


@pytest.mark.parametrize("variant", ["init", "perturbed"])
def test_c1_cache_bytes_and_tokens_match_reference(oracle_path, variant):
    gold = GOLDEN[variant]
    prompt = GOLDEN["prompt"]
    model = c1_model(variant)
    kw = dict(num_heads=6, head_dim=128, num_layers=12, device="cpu", dtype=torch.float32)
    with torch.inference_mode():
        pre = orc.KVCache(batch_size=1, seq_len=len(prompt), **kw)
        logits = model.forward(torch.tensor([prompt]), kv_cache=pre)[:, -1, :]
        dec = orc.KVCache(batch_size=1, seq_len=len(prompt) + 64, **kw)
        dec.prefill(pre)
        tokens = []
        for step in range(64):
            nxt = torch.argmax(logits, dim=-1, keepdim=True)
            tokens.append(int(nxt[0, 0]))
            if step == 63:
                break
            logits = model.forward(nxt, kv_cache=dec)[:, -1, :]
    assert tokens == gold["tokens"]
    assert dec.cache_seqlens.tolist() == gold["cache_seqlens"]
    for i in range(12):
        assert hashlib.sha256(dec.k_cache[i].numpy().tobytes()).hexdigest() == gold["cache_sha256"]["k"][i], i
        assert hashlib.sha256(dec.v_cache[i].numpy().tobytes()).hexdigest() == gold["cache_sha256"]["v"][i], i
    assert float(logits.double().sum()) == gold["last_logits_sum"]


@pytest.mark.parametrize("variant", ["init", "perturbed"])
def test_c1_engine_generate_matches_reference(oracle_path, variant):
    model = c1_model(variant)
    engine = eng.Engine(model, SpecialTokens())
    out = [col[0] for col, _ in engine.generate(GOLDEN["prompt"], num_samples=1, max_tokens=64, temperature=0.0)]
    assert out == GOLDEN[variant]["tokens"]


def test_c1_naive_generate_matches_reference(oracle_path):
    model = c1_model("perturbed")
    out = list(model.generate(GOLDEN["prompt"], max_tokens=8, temperature=0.0))
    assert out == GOLDEN["perturbed"]["naive_tokens"][:8]


def test_window_sizes_match_oracle_closed_form():
    for seq, pat, n in ((2048, "SSSL", 24), (4096, "SSSL", 26), (1024, "L", 12), (1000, "SL", 5)):
        cfg = gpt.GPTConfig(sequence_len=seq, n_layer=n, window_pattern=pat)
        assert gpt.window_sizes(cfg) == orc.compute_window_sizes(seq, pat, n)


def test_calculator_tool():
    assert eng.use_calculator("2+3*4") == 14
    assert eng.use_calculator("1,000/8") == 125.0
    assert eng.use_calculator("(7-2)*-3") == -15
    assert eng.use_calculator("'strawberry'.count('r')") == 3
    for bad in ("2**10", "__import__('os')", "1/0", "open('x').count('a')", "'a'.upper()", "x.count('a')"):
        assert eng.use_calculator(bad) is None, bad


def test_model_rotary_tables_equal_oracle():
    """nanochat_amd.gpt.rotary_tables (the fused prologue's tables) is the restated gpt.py:268-283."""
    from oracle import kvcache_oracle as orc
    for dtype in (torch.float32, torch.bfloat16):
        c1, s1 = gpt.rotary_tables(300, 128, dtype=dtype)
        c2, s2 = orc.rotary_tables(300, 128, dtype=dtype)
        assert torch.equal(c1, c2) and torch.equal(s1, s2)
