"""Write tests/golden/c1_d12_seed0.json: golden vectors for the C1 end-to-end check.

Runs in the development container only (it needs /root/reference; the GPU box
never runs it).  It imports nanochat's own GPT (nanochat/gpt.py) -- the only
way to pin GPT.forward with a KV cache (rotary offset, QK norm, value
embeddings, smear state, backout, softcap) -- and drives it the way
Engine.generate does (nanochat/engine.py:176-280) with num_samples=1 and
temperature 0.  nanochat/engine.py itself imports a tokenizer stack that is
not installed here, so the KV cache is oracle/kvcache_oracle.KVCache, the
restatement of nanochat/engine.py:82-137.  Attention is the reference's own
SDPA fallback (nanochat/flash_attention.py:155-177; FA3 is absent on CPU).

Config C1: d12 (12 layers, n_embd 768, 6/6 heads x 128, vocab 32768, window
"L", sequence_len 1024), fp32 on CPU, torch.manual_seed(0) before
init_weights, prompt = 64 ids from randint(0, 32768) with generator seed 0,
64 greedy tokens.  Two models:
  "init":      nanochat's init_weights as is (attn/mlp c_proj are zero and
               smear_lambda is 0, so attention cannot change the logits);
  "perturbed": init_weights, then torch.manual_seed(1) and N(0, 0.02) draws
               into every attn.c_proj and mlp.c_proj weight (in layer order,
               attn before mlp) and smear_lambda = 0.5, so attention and the
               smear cache state drive the tokens.
Stored per model: the greedy tokens, the naive no-cache generate tokens
(nanochat/gpt.py:483-512), final cache_seqlens, SHA-256 of every layer's K and
V cache bytes, and the last step's logits (float64 sum and first 8 values).

    python tests/golden/make_c1_golden.py
"""
import hashlib
import json
import os
import sys
from pathlib import Path

os.environ.setdefault("NANOCHAT_DTYPE", "float32")
HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, "/root/reference")
sys.path.insert(0, str(REPO))

import torch  # noqa: E402

from nanochat.gpt import GPT, GPTConfig  # noqa: E402  (reference, read-only mount)
from oracle.kvcache_oracle import KVCache  # noqa: E402

N_PROMPT, N_GEN = 64, 64


def make_model(perturbed: bool) -> GPT:
    cfg = GPTConfig(sequence_len=1024, vocab_size=32768, n_layer=12, n_head=6, n_kv_head=6, n_embd=768,
                    window_pattern="L")
    with torch.device("meta"):
        model = GPT(cfg)
    model.to_empty(device="cpu")
    torch.manual_seed(0)
    model.init_weights()
    if perturbed:
        torch.manual_seed(1)
        with torch.no_grad():
            for block in model.transformer.h:
                torch.nn.init.normal_(block.attn.c_proj.weight, mean=0.0, std=0.02)
                torch.nn.init.normal_(block.mlp.c_proj.weight, mean=0.0, std=0.02)
            model.smear_lambda.fill_(0.5)
    model.eval()
    return model


@torch.inference_mode()
def run(model: GPT, prompt):
    m = model.config
    kw = dict(num_heads=m.n_kv_head, head_dim=m.n_embd // m.n_head, num_layers=m.n_layer, device="cpu",
              dtype=torch.float32)
    pre = KVCache(batch_size=1, seq_len=len(prompt), **kw)
    logits = model.forward(torch.tensor([prompt], dtype=torch.long), kv_cache=pre)[:, -1, :]
    dec = KVCache(batch_size=1, seq_len=len(prompt) + N_GEN, **kw)
    dec.prefill(pre)
    tokens = []
    for step in range(N_GEN):
        nxt = torch.argmax(logits, dim=-1, keepdim=True)
        tokens.append(int(nxt[0, 0]))
        if step == N_GEN - 1:
            break
        logits = model.forward(nxt, kv_cache=dec)[:, -1, :]
    hashes = {
        "k": [hashlib.sha256(dec.k_cache[i].contiguous().numpy().tobytes()).hexdigest() for i in range(m.n_layer)],
        "v": [hashlib.sha256(dec.v_cache[i].contiguous().numpy().tobytes()).hexdigest() for i in range(m.n_layer)],
    }
    naive = list(model.generate(prompt, max_tokens=N_GEN, temperature=0.0))
    return {
        "tokens": tokens,
        "naive_tokens": naive,
        "cache_seqlens": dec.cache_seqlens.tolist(),
        "cache_sha256": hashes,
        "last_logits_sum": float(logits.double().sum()),
        "last_logits_head": [float(x) for x in logits[0, :8]],
    }


def main():
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 32768, (N_PROMPT,), generator=g).tolist()
    out = {"config": "C1 d12 fp32 CPU, seed 0, greedy", "prompt": prompt}
    for name, pert in (("init", False), ("perturbed", True)):
        out[name] = run(make_model(pert), prompt)
        print(name, out[name]["tokens"][:16], "naive == engine:", out[name]["tokens"] == out[name]["naive_tokens"])
    (HERE / "c1_d12_seed0.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
