"""GPU checks of the decode-step entry points that update the residual stream in place.

* ``sfl_decode_attention_out_proj``: x += attention(q, k, v) @ W_o^T with the
  attention and the output projection in one kernel (per-head atomics);
* ``sfl_linear_residual`` with K split over several workgroups (atomics);
* the normalized consumers (``sfl_rmsnorm_swiglu``, ``sfl_rmsnorm_lm_head``)
  reading the raw residual stream with their RMSNorm gain.

References are float64 on the CPU, from the same (dtype-rounded) inputs.
"""

import pytest
import torch

from systems_for_llms_amd import _lib
from test_gpu_gemv_layout import unpack_activation

pytestmark = pytest.mark.gpu


def pack_activation(v, code):
    """fp32 [rows, k] -> words of the activation layout (whole blocks of 16 rows)."""
    rows, k = v.shape
    blocks = -(-rows // 16)
    full = torch.zeros(blocks * 16, k)
    full[:rows] = v
    if code == _lib.DTYPE_F32X:
        return full.view(blocks, 16, k // 16, 4, 4).permute(0, 2, 3, 1, 4).reshape(-1)
    bits = full.view(torch.int32)
    hi = (bits & -65536).view(torch.float32)
    lo = ((full - hi).view(torch.int32) & -65536).view(torch.float32)
    halves = torch.stack([hi, lo]).to(torch.bfloat16)  # exact: both are bf16 values
    words = halves.view(2, blocks, 16, k // 32, 4, 8).permute(1, 3, 0, 4, 2, 5).reshape(-1)
    return words.view(torch.float32)


def activation_values(v, code):
    """The values the layout actually holds (bf16: hi + lo of each fp32 value)."""
    return unpack_activation(pack_activation(v, code), v.shape[0], v.shape[1], code)


def rms_normalize(x, g):
    return x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5) * g


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch", [3, 16, 37])  # 37: three 16-row blocks in one launch
@pytest.mark.parametrize("ksplit", [1, 2, 3, 16])
def test_linear_residual_split_k(dtype, batch, ksplit):
    code = _lib.DTYPE_BF16X2 if dtype == torch.bfloat16 else _lib.DTYPE_F32X
    g = torch.Generator().manual_seed(ksplit * 100 + batch)
    n, k = 96, 320  # bf16: 10 chunks, so ksplit 3 leaves a short part and 16 leaves empty parts
    w = torch.randn(n, k, generator=g).to(dtype)
    act = torch.randn(batch, k, generator=g)
    x0 = torch.randn(batch, n, generator=g)
    x = x0.cuda()
    # Keep every device tensor referenced until the launch has run.
    act_d, w_d = pack_activation(act, code).cuda(), _lib.pack_gemv(w.cuda())
    _lib.call("sfl_linear_residual", act_d.data_ptr(), w_d.data_ptr(), x.data_ptr(), batch, n, k, ksplit,
              _lib.dtype_code(dtype), _lib.stream_handle())
    ref = x0.double() + activation_values(act, code).double() @ w.double().T
    torch.testing.assert_close(x.cpu().double(), ref, atol=2e-5, rtol=2e-5)


def test_linear_residual_rejects_bad_split():
    x = torch.zeros(1, 16, device="cuda")
    w = torch.zeros(16 * 32, device="cuda", dtype=torch.bfloat16)
    for ksplit in (0, 17):
        with pytest.raises(RuntimeError, match="ksplit"):
            _lib.call("sfl_linear_residual", w.data_ptr(), w.data_ptr(), x.data_ptr(), 1, 16, 32, ksplit,
                      1, _lib.stream_handle())


def reference_attention(q, k, v, lengths, scale):
    """fp64 softmax attention of q [B, H, D] over keys [0, lengths[b]); empty rows give zeros."""
    b, h, cap, d = k.shape
    s = torch.einsum("bhd,bhtd->bht", q.double(), k.double()) * scale
    valid = torch.arange(cap)[None, :] < lengths[:, None]
    s = s.masked_fill(~valid[:, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1).nan_to_num(0.0)
    return torch.einsum("bht,bhtd->bhd", p, v.double())


@pytest.mark.parametrize("dtype,dim", [(torch.bfloat16, 32), (torch.bfloat16, 64), (torch.bfloat16, 128),
                                       (torch.float32, 16), (torch.float32, 64), (torch.float32, 128)])
@pytest.mark.parametrize("batch,heads", [(1, 2), (5, 4), (16, 16)])
def test_attention_out_proj_matches_reference(dtype, dim, batch, heads):
    g = torch.Generator().manual_seed(dim * 1000 + batch * 10 + heads)
    cap = 300
    d_model = heads * dim
    q = torch.randn(batch, heads, dim, generator=g)
    k = torch.randn(batch, heads, cap, dim, generator=g).to(dtype)
    v = torch.randn(batch, heads, cap, dim, generator=g).to(dtype)
    w_out = (torch.randn(d_model, d_model, generator=g) * d_model ** -0.5).to(dtype)
    lengths = torch.randint(1, cap + 1, (batch,), generator=g, dtype=torch.int32)
    lengths[0] = cap
    if batch > 2:
        lengths[1] = 0  # an empty row adds nothing
    x0 = torch.randn(batch, d_model, generator=g)
    x = x0.cuda()
    scale = dim ** -0.5
    qd, kd, vd, ld, wd = q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), _lib.pack_gemv(w_out.cuda())
    _lib.call("sfl_decode_attention_out_proj", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ld.data_ptr(),
              wd.data_ptr(), x.data_ptr(), batch, heads, cap, dim, scale, _lib.dtype_code(dtype),
              _lib.stream_handle())
    o = reference_attention(q, k, v, lengths.long(), scale).reshape(batch, d_model)
    ref = x0.double() + o @ w_out.double().T
    got = x.cpu().double()
    print(f"{dtype} D={dim} B={batch} H={heads}: max abs err {(got - ref).abs().max().item():.2e}")
    torch.testing.assert_close(got, ref, atol=5e-5, rtol=5e-5)
    if batch > 2:
        torch.testing.assert_close(got[1], x0[1].double(), atol=0, rtol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attention_out_proj_long_ragged_rows(dtype):
    """Rows several key tiles per wave long (head dim 64: the tile loop with one tile of loads ahead),
    lengths on and off the tile and round boundaries, the capacity, 0 and 1."""
    g = torch.Generator().manual_seed(77)
    heads, dim, cap = 4, 64, 2100
    lengths = torch.tensor([cap, 0, 1, 31, 32, 33, 511, 512, 513, 1024, 1537, 2099], dtype=torch.int32)
    batch, d_model = lengths.numel(), heads * dim
    q = torch.randn(batch, heads, dim, generator=g)
    k = torch.randn(batch, heads, cap, dim, generator=g).to(dtype)
    v = torch.randn(batch, heads, cap, dim, generator=g).to(dtype)
    w_out = (torch.randn(d_model, d_model, generator=g) * d_model ** -0.5).to(dtype)
    x0 = torch.randn(batch, d_model, generator=g)
    x = x0.cuda()
    scale = dim ** -0.5
    qd, kd, vd, ld, wd = q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), _lib.pack_gemv(w_out.cuda())
    _lib.call("sfl_decode_attention_out_proj", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ld.data_ptr(),
              wd.data_ptr(), x.data_ptr(), batch, heads, cap, dim, scale, _lib.dtype_code(dtype),
              _lib.stream_handle())
    o = reference_attention(q, k, v, lengths.long(), scale).reshape(batch, d_model)
    ref = x0.double() + o @ w_out.double().T
    got = x.cpu().double()
    print(f"{dtype} long rows: max abs err {(got - ref).abs().max().item():.2e}")
    torch.testing.assert_close(got, ref, atol=5e-5, rtol=5e-5)
    torch.testing.assert_close(got[1], x0[1].double(), atol=0, rtol=0)  # the empty row adds nothing


def test_attention_out_proj_rejects_unsupported_shapes():
    t = torch.zeros(4096, device="cuda")
    args = lambda dim, dtype: (t.data_ptr(),) * 4 + (t.data_ptr(), t.data_ptr(), 1, 2, 8, dim, 0.1, dtype,
                                                      _lib.stream_handle())
    with pytest.raises(RuntimeError, match="head dim"):
        _lib.call("sfl_decode_attention_out_proj", *args(16, 1))  # bf16 needs D >= 32
    with pytest.raises(RuntimeError, match="head dim"):
        _lib.call("sfl_decode_attention_out_proj", *args(48, 0))
    with pytest.raises(RuntimeError, match="dtype"):  # an activation-layout code is no model dtype
        _lib.call("sfl_decode_attention_out_proj", *args(64, _lib.DTYPE_BF16X2))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d_model,batch", [(96, 7), (1024, 7), (96, 40)])  # 40: three row blocks
def test_normalized_consumers_read_raw_x(dtype, d_model, batch):
    """SwiGLU and lm_head scale by the inverse RMS of x and apply the gain themselves."""
    code = _lib.DTYPE_BF16X2 if dtype == torch.bfloat16 else _lib.DTYPE_F32X
    g = torch.Generator().manual_seed(d_model + batch)
    d_ff, vocab = 96, 203
    x = torch.randn(batch, d_model, generator=g) * 3
    gain = (1 + 0.5 * torch.randn(d_model, generator=g)).to(dtype)
    w1 = torch.randn(d_ff, d_model, generator=g).to(dtype)
    w3 = torch.randn(d_ff, d_model, generator=g).to(dtype)
    wh = torch.randn(vocab, d_model, generator=g).to(dtype)
    xd, gd = x.cuda(), gain.cuda()
    w1d, w3d, whd = _lib.pack_gemv(w1.cuda()), _lib.pack_gemv(w3.cuda()), _lib.pack_gemv(wh.cuda())
    h = torch.zeros(-(-batch // 16) * 16 * d_ff, device="cuda")
    st, dc = _lib.stream_handle(), _lib.dtype_code(dtype)
    _lib.call("sfl_rmsnorm_swiglu", xd.data_ptr(), gd.data_ptr(), w1d.data_ptr(), w3d.data_ptr(), h.data_ptr(),
              batch, d_model, d_ff, dc, st)
    tiles = _lib.lib().sfl_lm_head_tiles(vocab)
    logits = torch.zeros(batch, vocab, device="cuda")
    best_val = torch.empty(tiles, batch, device="cuda")
    best_idx = torch.empty(tiles, batch, device="cuda", dtype=torch.int32)
    _lib.call("sfl_rmsnorm_lm_head", xd.data_ptr(), gd.data_ptr(), whd.data_ptr(),
              logits.data_ptr(), vocab, None, 0, best_val.data_ptr(), best_idx.data_ptr(), batch, batch,
              d_model, vocab, dc, st)
    # The kernels' operand is x * g rounded to the activation format, scaled after the dot product.
    xg = activation_values(x * gain.float(), code).double()
    inv = 1 / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-5)
    a1, a3 = inv * (xg @ w1.double().T), inv * (xg @ w3.double().T)
    h_ref = a1 * torch.sigmoid(a1) * a3
    got_h = unpack_activation(h.cpu(), batch, d_ff, code).double()
    # fp32 accumulation (absolute error ~1e-5 of the largest value); bf16 models
    # also store h as hi + lo bf16 halves (relative error below 2^-16).
    h_scale = h_ref.abs().max().item()
    torch.testing.assert_close(got_h, h_ref, atol=1e-5 * h_scale, rtol=5e-5)
    ref_logits = inv * (xg @ wh.double().T)
    # fp32 accumulation over d_model products of magnitude ~3: absolute error ~1e-5 * |logits|max
    scale = ref_logits.abs().max().item()
    torch.testing.assert_close(logits.cpu().double(), ref_logits, atol=1e-5 * scale, rtol=5e-5)
    # Exact check of the normalization against the unfolded form RMSNorm(x) @ W^T.
    unfolded = rms_normalize(x.double(), gain.double()) @ wh.double().T
    assert (logits.cpu().double() - unfolded).abs().max().item() < 1e-2 * unfolded.abs().max().item()


def test_swiglu_rejects_partial_output_chunks():
    """h is written in whole activation-layout chunks: d_ff must be a multiple of 32 (bf16)."""
    t = torch.zeros(1 << 16, device="cuda")
    with pytest.raises(RuntimeError, match="d_ff"):
        _lib.call("sfl_rmsnorm_swiglu", t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(),
                  1, 64, 80, 1, _lib.stream_handle())
