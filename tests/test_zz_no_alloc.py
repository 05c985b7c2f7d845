"""The allocation-free decode attention entry point against the one with caller scratch.

``sfl_decode_attention_static`` keeps the split partials in the library's
static per-GPU buffer; it must give exactly the results of
``sfl_decode_attention`` with torch-allocated scratch (same kernels), on
consecutive calls where the second is smaller and the buffer holds the first
call's contents, and reject a request larger than the buffer before launching.
"""

import pytest
import torch

from oracle.attention import decode_reference
from systems_for_llms_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(batch, q_heads, kv_heads, cap, dim, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((batch, q_heads, dim), generator=g).to(torch.bfloat16)
    k = torch.randn((batch, kv_heads, cap, dim), generator=g).to(torch.bfloat16)
    v = torch.randn((batch, kv_heads, cap, dim), generator=g).to(torch.bfloat16)
    lengths = torch.randint(0, cap + 1, (batch,), generator=g, dtype=torch.int32)
    lengths[0] = cap
    return q, k, v, lengths


def _run(static, q, k, v, lengths, splits):
    batch, q_heads, dim = q.shape
    kv_heads, cap = k.shape[1], k.shape[2]
    out = torch.full_like(q, float("nan"))
    st = _lib.stream_handle()
    args = (batch, q_heads, kv_heads, cap, dim, splits, dim ** -0.5, 1, 1, 1, st)
    if static:
        _lib.call("sfl_decode_attention_static", q.data_ptr(), k.data_ptr(), v.data_ptr(), lengths.data_ptr(),
                  out.data_ptr(), *args)
    else:
        pmax = torch.empty((batch, q_heads, splits), device="cuda")
        psum = torch.empty_like(pmax)
        pout = torch.empty((batch, q_heads, splits, dim), device="cuda")
        _lib.call("sfl_decode_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), lengths.data_ptr(),
                  pmax.data_ptr(), psum.data_ptr(), pout.data_ptr(), out.data_ptr(), *args)
    torch.cuda.synchronize()
    return out


def test_static_scratch_entry_point_matches_caller_scratch():
    # Second call smaller than the first; grouped heads (MFMA kernel) and MHA (VALU kernel).
    for shape, splits in (((6, 32, 4, 1500, 128), 16), ((3, 8, 8, 700, 64), 5), ((2, 16, 2, 300, 64), 3)):
        cpu = _inputs(*shape, seed=sum(shape))
        gpu = [t.cuda() for t in cpu]
        got = _run(True, *gpu, splits)
        want = _run(False, *gpu, splits)
        assert torch.equal(got, want), shape
        torch.testing.assert_close(got.float().cpu(), decode_reference(*cpu), atol=0.02, rtol=0.02)


def test_static_scratch_rejects_requests_beyond_its_size():
    limit = _lib.lib().sfl_decode_attention_static_scratch_bytes()
    assert limit == 16 << 20
    q, k, v, lengths = (t.cuda() for t in _inputs(64, 32, 4, 256, 128, 3))
    out = torch.zeros_like(q)
    with pytest.raises(RuntimeError, match="static buffer"):  # 64*32*128*130*4 bytes > 16 MiB
        _lib.call("sfl_decode_attention_static", q.data_ptr(), k.data_ptr(), v.data_ptr(), lengths.data_ptr(),
                  out.data_ptr(), 64, 32, 4, 256, 128, 128, 128 ** -0.5, 1, 1, 1, _lib.stream_handle())
    assert not out.any()
