"""The allocation-free decode attention entry (ptb_attn_decode_bf16_noalloc) through the C ABI: its
output equals ptb_attn_decode_bf16's with a caller workspace bit for bit (the same kernels, the
records in the static scratch instead), on two calls in a row -- the second with a smaller input, so
it runs over what the first left in the scratch -- and a shape past the scratch is refused before
anything runs."""
import ctypes

import pytest
import torch

from helpers import bits_equal, randn
from ptb_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(nkv, g, s, seed):
    q = randn((nkv, g, 128), seed).to(DEV)
    k = randn((nkv, s, 128), seed + 1).to(DEV)
    v = randn((nkv, s, 128), seed + 2).to(DEV)
    return q, k, v


def _with_workspace(lib, q, k, v, nkv, g, s, scale):
    o = torch.empty_like(q)
    need = lib.ptb_attn_decode_workspace_bytes(nkv, g, s)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
    st = lib.ptb_attn_decode_bf16(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), nkv, g, s, 128, scale,
                                  ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.status_text(st)
    return o


def _no_alloc(lib, q, k, v, nkv, g, s, scale):
    o = torch.empty_like(q)
    st = lib.ptb_attn_decode_bf16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), nkv, g, s, 128,
                                          scale, torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.status_text(st)
    return o


def test_no_alloc_decode_attention_matches_workspace_entry():
    lib = _lib.load()
    scale = 128 ** -0.5
    # the Qwen3-8B decode shape (several key ranges: records in the scratch), then a smaller one
    for nkv, g, s, seed in [(8, 4, 4096, 0), (2, 8, 1536, 10)]:
        assert 0 < lib.ptb_attn_decode_workspace_bytes(nkv, g, s) <= lib.ptb_attn_decode_noalloc_max_bytes()
        q, k, v = _inputs(nkv, g, s, seed)
        want = _with_workspace(lib, q, k, v, nkv, g, s, scale)
        got = _no_alloc(lib, q, k, v, nkv, g, s, scale)
        torch.cuda.synchronize()
        assert bits_equal(got, want), f"noalloc decode attention differs at {nkv}x{g}x{s}"
    # a cache short enough for the single-launch form needs no scratch at all
    q, k, v = _inputs(8, 4, 128, 20)
    assert lib.ptb_attn_decode_workspace_bytes(8, 4, 128) == 0
    assert bits_equal(_no_alloc(lib, q, k, v, 8, 4, 128, scale), _with_workspace(lib, q, k, v, 8, 4, 128, scale))


def test_no_alloc_refuses_shapes_past_the_scratch():
    lib = _lib.load()
    nkv, g, s = 64, 8, 131072
    assert lib.ptb_attn_decode_workspace_bytes(nkv, g, s) > lib.ptb_attn_decode_noalloc_max_bytes()
    p = ctypes.c_void_p(16)   # never dereferenced: the size check comes first
    st = lib.ptb_attn_decode_bf16_noalloc(p, p, p, p, nkv, g, s, 128, 0.088, None)
    assert st == _lib.PTB_ERR_WORKSPACE
