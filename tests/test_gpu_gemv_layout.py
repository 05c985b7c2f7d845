"""GPU checks of the decode GEMVs' data layouts (the packed weight tiles and the
activation layout, as documented in include/sfl.h), independent of the model."""

import pytest
import torch

from systems_for_llms_amd import _lib

pytestmark = pytest.mark.gpu


def epl(dtype):
    return 8 if dtype == torch.bfloat16 else 4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [16, 37, 64])
def test_pack_gemv_weights_layout(dtype, n):
    k = 128
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(n)).to(dtype)
    packed = _lib.pack_gemv(w.cuda()).cpu()
    e = epl(dtype)
    tiles = -(-n // 16)
    ref = torch.zeros(tiles * 16, k, dtype=dtype)
    ref[:n] = w
    # [tile, row r, chunk c, group g, e] -> [tile, c, g, r, e]: lane 16*g + r of chunk c
    ref = ref.view(tiles, 16, k // (4 * e), 4, e).permute(0, 2, 3, 1, 4).reshape(-1)
    assert packed.numel() == _lib.lib().sfl_packed_gemv_elems(n, k)
    assert torch.equal(packed, ref)


def unpack_activation(buf, rows, k, code):
    """[ceil(rows/16) * 16 * k] words of the activation layout -> fp32 [rows, k]."""
    blocks = -(-rows // 16)
    if code == _lib.DTYPE_F32X:
        v = buf.view(blocks, k // 16, 4, 16, 4).permute(0, 3, 1, 2, 4).reshape(blocks * 16, k)
    else:
        halves = buf.view(torch.bfloat16).view(blocks, k // 32, 2, 4, 16, 8).float()
        v = (halves[:, :, 0] + halves[:, :, 1]).permute(0, 3, 1, 2, 4).reshape(blocks * 16, k)
    return v[:rows]


@pytest.mark.parametrize("code", [_lib.DTYPE_BF16X2, _lib.DTYPE_F32X])
@pytest.mark.parametrize("batch", [5, 16, 21])
def test_attention_writes_activation_layout(code, batch):
    """Decode attention's layout outputs hold the same values as its fp32 output."""
    g = torch.Generator().manual_seed(batch)
    heads, dim, cap = 4, 64, 100
    kv_dtype = torch.bfloat16 if code == _lib.DTYPE_BF16X2 else torch.float32
    q = torch.randn(batch, heads, dim, generator=g).cuda()
    k = torch.randn(batch, heads, cap, dim, generator=g).to(kv_dtype).cuda()
    v = torch.randn(batch, heads, cap, dim, generator=g).to(kv_dtype).cuda()
    lengths = torch.randint(1, cap + 1, (batch,), generator=g, dtype=torch.int32).cuda()
    k_dim = heads * dim
    for splits in (1, 3):
        pmax = torch.empty(batch * heads * splits, device="cuda")
        psum = torch.empty_like(pmax)
        pout = torch.empty(batch * heads * splits * dim, device="cuda")
        plain = torch.empty(batch, k_dim, device="cuda")
        laid = torch.zeros(-(-batch // 16) * 16 * k_dim, device="cuda")
        for out, out_code in ((plain, 0), (laid, code)):
            _lib.call("sfl_decode_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), lengths.data_ptr(),
                      pmax.data_ptr(), psum.data_ptr(), pout.data_ptr(), out.data_ptr(), batch, heads,
                      heads, cap, dim, splits, dim ** -0.5, _lib.dtype_code(kv_dtype), 0, out_code,
                      _lib.stream_handle())
        torch.cuda.synchronize()
        got = unpack_activation(laid.cpu(), batch, k_dim, code)
        ref = plain.cpu()
        if code == _lib.DTYPE_F32X:
            assert torch.equal(got, ref)
        else:  # hi and lo are truncations: |v - hi - lo| < 2^-7 |v - hi| < 2^-14 |v|
            assert ((got - ref).abs() <= ref.abs() * 2.0 ** -14).all()
