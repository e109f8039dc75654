"""ctypes binding of libnc_kv.so (declared in include/nc_kv.h).

Loads the in-tree library built by ``python -m nanochat_amd.build`` and
mirrors its argument structs.  There is no fallback: if the library is
missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

# NANOCHAT_AMD_LIB points at another build of the same library (e.g. a tuning
# variant); by default the in-tree build next to this file is loaded.
LIB_PATH = Path(os.environ.get("NANOCHAT_AMD_LIB", Path(__file__).resolve().parent / "libnc_kv.so"))
ABI_VERSION = 8

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

NC_DEVERR_OVERFLOW = 1
NC_DEVERR_ROPE_RANGE = 2
NC_DEVERR_BATCH_IDX = 4
NC_DEVERR_QLEN = 8
NC_DEVERR_SAMPLE = 16
NC_DEVERR_PAGE = 32
# leading workspace bytes holding split counters: zero before first use, left zero by every call
NC_WORKSPACE_SYNC_BYTES = 65536
# device scratch nc_attn_kvcache_noalloc holds on each GPU (its largest call's workspace)
NC_NOALLOC_SCRATCH_BYTES = 64 << 20
NC_ERR_SCRATCH_LIMIT = 8

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class AppendArgs(ctypes.Structure):
    _fields_ = [
        ("k_cache", _c_void_p), ("v_cache", _c_void_p),
        ("k", _c_void_p), ("v", _c_void_p),
        ("cache_seqlens", _c_void_p), ("error_flag", _c_void_p),
        ("cache_batch_idx", _c_void_p), ("cache_batch", _i64), ("cu_seqlens_q", _c_void_p), ("total_q", _i64),
        ("page_table", _c_void_p), ("page_table_stride", _i64), ("page_size", _i64), ("num_blocks", _i64),
        ("batch", _i64), ("t_new", _i64), ("t_max", _i64), ("n_kv_heads", _i64), ("head_dim", _i64),
        ("kc_stride_b", _i64), ("kc_stride_t", _i64), ("kc_stride_h", _i64),
        ("vc_stride_b", _i64), ("vc_stride_t", _i64), ("vc_stride_h", _i64),
        ("k_stride_b", _i64), ("k_stride_t", _i64), ("k_stride_h", _i64),
        ("v_stride_b", _i64), ("v_stride_t", _i64), ("v_stride_h", _i64),
        ("in_dtype", _i32), ("cache_dtype", _i32),
    ]


class FanoutArgs(ctypes.Structure):
    _fields_ = [
        ("k_src", _c_void_p), ("v_src", _c_void_p),
        ("k_dst", _c_void_p), ("v_dst", _c_void_p),
        ("dst_seqlens", _c_void_p),
        ("n_layers", _i64), ("n_rows", _i64), ("prefix_len", _i64), ("row_elems", _i64),
        ("src_stride_l", _i64), ("dst_stride_l", _i64), ("dst_stride_b", _i64),
        ("dtype", _i32),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", _c_void_p), ("out", _c_void_p),
        ("k_cache", _c_void_p), ("v_cache", _c_void_p),
        ("k", _c_void_p), ("v", _c_void_p),
        ("cache_seqlens", _c_void_p), ("error_flag", _c_void_p),
        ("cache_batch_idx", _c_void_p), ("cache_batch", _i64), ("cu_seqlens_q", _c_void_p), ("total_q", _i64),
        ("page_table", _c_void_p), ("page_table_stride", _i64), ("page_size", _i64), ("num_blocks", _i64),
        ("workspace", _c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("batch", _i64), ("t_new", _i64), ("t_max", _i64),
        ("n_heads", _i64), ("n_kv_heads", _i64), ("head_dim", _i64),
        ("q_stride_b", _i64), ("q_stride_t", _i64), ("q_stride_h", _i64),
        ("kc_stride_b", _i64), ("kc_stride_t", _i64), ("kc_stride_h", _i64),
        ("vc_stride_b", _i64), ("vc_stride_t", _i64), ("vc_stride_h", _i64),
        ("k_stride_b", _i64), ("k_stride_t", _i64), ("k_stride_h", _i64),
        ("v_stride_b", _i64), ("v_stride_t", _i64), ("v_stride_h", _i64),
        ("window_left", _i32), ("causal", _i32),
        ("softmax_scale", ctypes.c_float),
        ("q_dtype", _i32), ("cache_dtype", _i32),
        ("keys_per_split", _i32),
    ]


class QKPrologue(ctypes.Structure):
    _fields_ = [
        ("cos", _c_void_p), ("sin", _c_void_p),
        ("rot_len", _i64), ("rot_dtype", _i32),
        ("qk_scale", ctypes.c_float), ("eps", ctypes.c_float),
    ]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        ("x", _c_void_p), ("w", _c_void_p), ("y", _c_void_p),
        ("workspace", _c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("m", _i64), ("n", _i64), ("k", _i64),
        ("x_stride_m", _i64), ("w_stride_n", _i64), ("y_stride_m", _i64),
        ("dtype", _i32), ("y_dtype", _i32),
        ("softcap", ctypes.c_float),
    ]


class SampleArgs(ctypes.Structure):
    _fields_ = [
        ("logits", _c_void_p), ("uniforms", _c_void_p), ("out", _c_void_p), ("error_flag", _c_void_p),
        ("batch", _i64), ("vocab", _i64), ("logits_stride", _i64),
        ("temperature", ctypes.c_float), ("top_k", _i32),
    ]


# Every function include/nc_kv.h declares, with its ctypes signature.
EXPORTS = {
    "nc_abi_version": (ctypes.c_int, []),
    "nc_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "nc_supports_head_dim": (ctypes.c_int, [_i64]),
    "nc_kv_append": (ctypes.c_int, [ctypes.POINTER(AppendArgs), _c_void_p]),
    "nc_kv_fanout": (ctypes.c_int, [ctypes.POINTER(FanoutArgs), _c_void_p]),
    "nc_attn_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnArgs)]),
    "nc_attn_kvcache": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _c_void_p]),
    "nc_attn_kvcache_noalloc": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _c_void_p]),
    "nc_attn_rope_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnArgs)]),
    "nc_attn_kvcache_rope": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.POINTER(QKPrologue), _c_void_p]),
    "nc_linear_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "nc_linear": (ctypes.c_int, [ctypes.POINTER(LinearArgs), _c_void_p]),
    "nc_sample": (ctypes.c_int, [ctypes.POINTER(SampleArgs), _c_void_p]),
}

_lib = None
_lib_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded libnc_kv.so (raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m nanochat_amd.build` "
                    "(the KV-cache path has no non-HIP implementation)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, argtypes) in EXPORTS.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = argtypes
            if handle.nc_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {handle.nc_abi_version()}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().nc_strerror(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (nc_status {status})")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------------------
# Per-(device, stream) split-K workspace and per-device error flag.  Calls on
# one stream are ordered, so one buffer per stream is reused across calls.
# ---------------------------------------------------------------------------
_workspaces: dict = {}
_error_flags: dict = {}
_retired: list = []  # outgrown workspaces, kept alive for graphs captured with them


def workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    """Split-K / prologue scratch for calls on `stream` (grows, never shrinks).

    Buffers are allocated zeroed (their first NC_WORKSPACE_SYNC_BYTES hold the
    split counters, which the library keeps at zero between calls) and outside
    inference mode (they outlive the call that made them).  A buffer that is
    outgrown is kept alive, not freed: a HIP graph captured with it may still
    be replayed.
    """
    if nbytes == 0:
        return None
    key = (device.index, stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        cap = max(nbytes, 2 * buf.numel() if buf is not None else 0, 1 << 20)
        if buf is not None:
            _retired.append(buf)
        with torch.inference_mode(False):
            buf = torch.zeros(cap, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf


def error_flag(device: torch.device) -> torch.Tensor:
    flag = _error_flags.get(device.index)
    if flag is None:
        with torch.inference_mode(False):
            flag = torch.zeros(1, dtype=torch.int32, device=device)
        _error_flags[device.index] = flag
    return flag


def read_and_clear_device_errors(device: torch.device) -> int:
    """NC_DEVERR_* bits raised by kernels on `device` since the last read (synchronises)."""
    flag = error_flag(device)
    bits = int(flag.item())
    flag.zero_()
    return bits


# What each device error bit means, in the words of the error the reference raises (or would
# raise) for the same input.
DEVICE_ERROR_MESSAGES = (
    (NC_DEVERR_OVERFLOW, "cache_seqlens + T_new exceeds the cache length (the reference's slice "
                         "assignment fails on the size mismatch)"),
    (NC_DEVERR_ROPE_RANGE, "a position is beyond the rotary tables"),
    (NC_DEVERR_BATCH_IDX, "cache_batch_idx holds an index outside the cache's batch dimension"),
    (NC_DEVERR_QLEN, "cu_seqlens_q holds a row outside [0, total_q) or longer than max_seqlen_q"),
    (NC_DEVERR_SAMPLE, "a row of logits has no finite value (torch.multinomial rejects such a row)"),
    (NC_DEVERR_PAGE, "page_table holds a block index outside the cache"),
)


def raise_device_errors(bits: int, where: str) -> None:
    """RuntimeError naming every NC_DEVERR_* bit set in `bits` (nothing if bits == 0)."""
    if bits:
        msgs = [m for b, m in DEVICE_ERROR_MESSAGES if bits & b] or [f"device error bits {bits:#x}"]
        raise RuntimeError(f"{where}: " + "; ".join(msgs))


def host_values_and_errors(t: torch.Tensor) -> tuple[list, int]:
    """t's values on the host together with the device error flag, in ONE device-to-host copy.

    For host synchronisations the caller makes anyway (KVCache.get_pos, the engine's sampled
    ids): the flag rides along, so surfacing kernel errors adds no synchronisation.  A set flag
    is cleared (on the current stream) and its bits returned."""
    flag = error_flag(t.device)
    vals = torch.cat((t.reshape(-1).to(torch.int64), flag.to(torch.int64))).tolist()
    bits = int(vals[-1])
    if bits:
        flag.zero_()
    return vals[:-1], bits
