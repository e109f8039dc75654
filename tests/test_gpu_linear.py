"""GPU parity of the small-M linear kernel (nc_linear) and the fused logits head.

The reference is F.linear(x, W.to(x.dtype)) (nanochat/gpt.py:45-50) and, for the logits head,
softcap * tanh(logits[..., :vocab].float() / softcap) (gpt.py:468-472).  This is floating-point
GEMM work, so the reference is plain torch in fp32/fp64 on the CPU, with two exact pins:
- integer-valued operands whose dot products are exact in fp32 whatever the summation order: the
  bf16/fp16 result must then equal the exact sum rounded to nearest even, bit for bit.  A wrong
  k pairing between x and W, a dropped chunk or a wrong output index breaks it;
- the logits-head epilogue against torch's own op sequence on the same bf16 values, over every
  bf16 bit pattern.
Random operands: max error relative to max |ref| <= 1e-2 (bf16 output rounding is 2^-9).
"""
import ctypes

import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.linear import MAX_M, linear, logits_head, supported
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _int_operands(seed, m, n, k, dtype):
    g = gen(seed)
    x = torch.randint(-3, 4, (m, k), generator=g).to(dtype)
    w = torch.randint(-3, 4, (n, k), generator=g).to(dtype)
    return x, w


@pytest.mark.parametrize("m,n,k", [
    (1, 1, 8), (1, 10, 24), (5, 100, 136), (16, 16, 128), (17, 33, 264), (32, 1280, 1280),
    (32, 5120, 1280), (32, 1280, 5120), (33, 96, 2048), (48, 200, 640), (64, 1280, 1280), (16, 1536, 6144),
    # narrow plan (m <= 32): 8 waves per workgroup, waves with no chunk, a partial last chunk
    (32, 3840, 1280), (9, 2100, 520), (32, 136, 4104), (2, 24, 392),
    # narrow plan with two column tiles per wave (m > 16, wide n), ragged last block
    (20, 4100, 264), (32, 6144, 1536),
    # two column tiles per wave AND K split over two workgroups (ticket merge of the 2-tile partials)
    (32, 5120, 2048), (24, 6144, 2304),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_exact_on_integer_operands(m, n, k, dtype):
    x, w = _int_operands(m * 7919 + n * 31 + k, m, n, k, dtype)
    exact = x.double() @ w.double().T      # |sum| <= 9k < 2^24: exact in fp32 in any order
    want = exact.float().to(dtype)         # one rounding, nearest even
    got = linear(x.to(DEV), w.to(DEV)).cpu()
    assert got.dtype == dtype and got.shape == (m, n)
    assert torch.equal(bits(got), bits(want)), (m, n, k, dtype)


@pytest.mark.parametrize("m,n,k", [(32, 5120, 2048), (24, 6144, 2304)])
def test_two_tile_split_plan_is_the_one_exercised(m, n, k):
    """The shapes above reach the narrow kernel with two 16-column tiles per wave and K split over
    two workgroups: the workspace holds exactly that plan's partials (64 KiB of split counters,
    then blocks x splits x tiles x row tiles x 64 lanes x 4 fp32 values)."""
    lib = _ext.lib()
    blocks, splits, tiles, row_tiles = (n + 31) // 32, 2, 2, (m + 15) // 16
    want = _ext.NC_WORKSPACE_SYNC_BYTES + blocks * splits * tiles * row_tiles * 64 * 4 * 4
    assert lib.nc_linear_workspace_bytes(m, n, k) == want


@pytest.mark.parametrize("m,n,k", [(32, 1280, 1280), (32, 1280, 5120), (7, 333, 1000), (64, 2048, 512)])
def test_linear_fp32_output_exact_on_integer_operands(m, n, k):
    x, w = _int_operands(11 + m + n + k, m, n, k, torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    from nanochat_amd.linear import _call
    got = _call(xd, wd, n, torch.float32, 0.0).cpu()
    assert torch.equal(got, (x.double() @ w.double().T).float())


@pytest.mark.parametrize("m,n,k,dtype", [
    (32, 1280, 1280, torch.bfloat16), (32, 5120, 1280, torch.bfloat16), (32, 1280, 5120, torch.bfloat16),
    (16, 1536, 6144, torch.bfloat16), (1, 32768, 1280, torch.bfloat16), (64, 640, 4096, torch.float16),
    (3, 50, 72, torch.float16),
])
def test_linear_random_matches_fp32(m, n, k, dtype):
    g = gen(m + n + k)
    x = randn((m, k), g, dtype)
    w = (randn((n, k), g) * k ** -0.5).to(dtype)
    ref = x.double() @ w.double().T
    xd, wd = x.to(DEV), w.to(DEV)
    got = linear(xd, wd)
    assert max_rel_err(got, ref) <= 1e-2
    torch_bf = torch.nn.functional.linear(xd, wd)   # the library GEMM the reference runs
    assert max_rel_err(got, torch_bf.float()) <= 1e-2
    again = linear(xd, wd)                           # deterministic: same bits every call
    assert torch.equal(bits(got), bits(again))


def test_linear_3d_and_strided_views():
    g = gen(5)
    B, C, N = 24, 1280, 640
    wide = randn((B, 1, 2 * C), g, torch.bfloat16).to(DEV)
    x = wide[..., C:]                                # row stride 2C, 16-byte aligned
    w = (randn((N, C), g) * C ** -0.5).to(torch.bfloat16).to(DEV)
    got = linear(x, w)
    assert got.shape == (B, 1, N)
    ref = x.double().cpu() @ w.double().cpu().T
    assert max_rel_err(got, ref) <= 1e-2
    assert torch.equal(bits(got), bits(linear(x.contiguous(), w)))


def test_logits_head_equals_torch_softcap_on_same_logits():
    g = gen(9)
    m, vocab, pad, k = 32, 1000, 1024, 1280
    x = randn((m, 1, k), g, torch.bfloat16).to(DEV)
    w = (randn((pad, k), g) * 0.5).to(torch.bfloat16).to(DEV)   # logits well into tanh's curved range
    got = logits_head(x, w, vocab, 15.0)
    assert got.dtype == torch.float32 and got.shape == (m, 1, vocab)
    logits = linear(x, w[:vocab])                    # the same accumulation, rounded to bf16
    want = 15 * torch.tanh(logits.float() / 15)      # gpt.py:470-471 on those values
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,vocab,pad,k,dtype", [(16, 50257, 50304, 768, torch.bfloat16),
                                                 (64, 32768, 32768, 1536, torch.bfloat16),
                                                 (8, 5000, 5056, 512, torch.float16)])
def test_logits_head_vocab_slices_and_dtypes(m, vocab, pad, k, dtype):
    g = gen(m + vocab)
    x = randn((m, k), g, dtype).to(DEV)
    w = (randn((pad, k), g) * 0.3).to(dtype).to(DEV)
    got = logits_head(x, w, vocab, 15.0)
    assert got.shape == (m, vocab) and got.dtype == torch.float32
    want = 15 * torch.tanh(linear(x, w[:vocab]).float() / 15)
    assert torch.equal(got, want)
    ref = 15 * torch.tanh((x.double().cpu() @ w[:vocab].double().cpu().T) / 15)
    assert max_rel_err(got, ref) <= 1e-2


def test_logits_head_epilogue_every_bf16_value():
    # x = [1, 0...], W[n, 0] = the n-th bf16 bit pattern: logits are exactly every bf16 value
    vals = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    w = torch.zeros((1 << 16, 8), dtype=torch.bfloat16)
    w[:, 0] = vals
    x = torch.zeros((1, 8), dtype=torch.bfloat16)
    x[0, 0] = 1.0
    got = logits_head(x.to(DEV), w.to(DEV), 1 << 16, 15.0)[0]
    want = 15 * torch.tanh(vals.to(DEV).float() / 15)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan], want[~nan])


def test_split_counters_return_to_zero_between_linear_and_attention():
    from nanochat_amd.flash_attention import flash_attn
    g = gen(21)
    wk = randn((1280, 5120), g, torch.bfloat16).to(DEV)   # K split over 4 workgroups per column block
    xk = randn((64, 5120), g, torch.bfloat16).to(DEV)
    first = linear(xk, wk)
    first32 = linear(xk[:32], wk)   # narrow kernel, K split over 2 workgroups per 16 columns
    q = randn((8, 1, 16, 128), g, torch.bfloat16).to(DEV)
    kc = randn((8, 4096, 4, 128), g, torch.bfloat16).to(DEV)
    vc = randn((8, 4096, 4, 128), g, torch.bfloat16).to(DEV)
    sl = torch.full((8,), 4000, dtype=torch.int32, device=DEV)
    for _ in range(3):
        flash_attn.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=sl, causal=True)
        assert torch.equal(bits(linear(xk, wk)), bits(first))
        assert torch.equal(bits(linear(xk[:32], wk)), bits(first32))
    torch.cuda.synchronize()
    for buf in list(_ext._workspaces.values()):
        assert int(buf[:_ext.NC_WORKSPACE_SYNC_BYTES].count_nonzero()) == 0


def test_supported_and_rejections():
    w = torch.zeros((16, 64), dtype=torch.bfloat16, device=DEV)
    assert supported(torch.zeros((MAX_M, 64), dtype=torch.bfloat16, device=DEV), w)
    assert not supported(torch.zeros((MAX_M + 1, 64), dtype=torch.bfloat16, device=DEV), w)
    assert not supported(torch.zeros((4, 64), dtype=torch.float32, device=DEV), w.float())
    assert not supported(torch.zeros((4, 12), dtype=torch.bfloat16, device=DEV),
                         torch.zeros((10, 12), dtype=torch.bfloat16, device=DEV))   # K % 8 != 0
    with pytest.raises(ValueError):
        linear(torch.zeros((MAX_M + 1, 64), dtype=torch.bfloat16, device=DEV), w)
    # the C ABI rejects a missing workspace when K is split
    L = _ext.lib()
    m, n, k = 64, 1280, 1280
    assert L.nc_linear_workspace_bytes(m, n, k) > 0
    x = torch.zeros((m, k), dtype=torch.bfloat16, device=DEV)
    ww = torch.zeros((n, k), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    a = _ext.LinearArgs()
    a.x, a.w, a.y = x.data_ptr(), ww.data_ptr(), y.data_ptr()
    a.m, a.n, a.k, a.x_stride_m, a.w_stride_n, a.y_stride_m = m, n, k, k, k, n
    a.dtype = a.y_dtype = _ext.DTYPE_CODE[torch.bfloat16]
    assert L.nc_linear(ctypes.byref(a), _ext.stream_handle(x.device)) == 6   # NC_ERR_WORKSPACE
