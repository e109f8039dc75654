"""nanochat_amd: nanochat's inference KV-cache path on MI355X (gfx950).

Modules
  flash_attention  drop-in ``flash_attn`` namespace (flash_attn_with_kvcache)
  engine           KVCache (fan-out prefill on the GPU)
  _ext             ctypes binding of libnc_kv.so (include/nc_kv.h)
  build            hipcc build of libnc_kv.so
"""
from .flash_attention import flash_attn  # noqa: F401
from .engine import KVCache  # noqa: F401
