"""Compute-dtype policy of nanochat (nanochat/common.py:16-31), kept identical.

NANOCHAT_DTYPE ("bfloat16" | "float16" | "float32") wins; otherwise bf16 when
a GPU of capability >= 8.0 is visible (every MI355X: gfx950 reports 9.x),
else fp32.  The KV cache dtype follows a separate rule in Engine.generate:
bf16 on a GPU device, fp32 elsewhere (nanochat/engine.py:186).
"""
import os

import torch

_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def detect_compute_dtype():
    env = os.environ.get("NANOCHAT_DTYPE")
    if env is not None:
        return _DTYPES[env]
    if torch.cuda.is_available() and torch.cuda.get_device_capability() >= (8, 0):
        return torch.bfloat16
    return torch.float32


COMPUTE_DTYPE = detect_compute_dtype()
