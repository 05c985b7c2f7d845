"""GPU parity of the prefill path (MFMA GEMMs + causal attention; bf16, fp16, fp32) against the oracle."""

import pytest
import torch

from oracle import model as om
from systems_for_llms_amd import _lib
from systems_for_llms_amd.config import ModelConfig, load_model_config
from systems_for_llms_amd.engine import DecodeSession
from systems_for_llms_amd.model import TransformerLM
from systems_for_llms_amd.weights import seeded_prompt, seeded_state_dict

from gates import bf16_gate

pytestmark = pytest.mark.gpu


# K % 64 == 0 takes the 32x32-MFMA kernel (ragged M and N included: rows past
# the matrices read as zeros, stores are masked); other K the 16x16 kernel.
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (37, 100, 72), (128, 128, 64), (300, 520, 200), (64, 3072, 1024),
                                   (300, 520, 256), (5, 10000, 128), (129, 127, 192), (1000, 36, 2752)])
def test_gemm_matches_fp32_matmul(m, n, k, dtype):
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn((m, k), generator=g).to(dtype)
    w = torch.randn((n, k), generator=g).to(dtype)
    ref = a.float() @ w.float().t()
    ga, gw = a.cuda(), w.cuda()  # keep the device copies alive across the launches
    out = torch.zeros((m, n), device="cuda")
    st = _lib.stream_handle()
    code = _lib.dtype_code(dtype)
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, code, 0, 0, st)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-3, rtol=1e-4)
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, code, 0, 1, st)
    torch.testing.assert_close(out.cpu(), 2 * ref, atol=2e-3, rtol=1e-4)
    ob = torch.zeros((m, n), device="cuda", dtype=dtype)
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), ob.data_ptr(), m, n, k, code, code, 0, st)
    # one rounding of the fp32 sums to the output type (bf16: 2^-8, fp16: 2^-11 relative)
    torch.testing.assert_close(ob.float().cpu(), ref.to(dtype).float(), atol=1e-2, rtol=1e-2)


# Grids of >= 320 tiles of 256 x 384 take the 256 x 384 kernel with its ring
# of LDS stages: K of 64 (fewer steps than stages), 192 and 2752 (the model's
# d_ff), ragged M and N. Sampled token rows keep the CPU reference small.
@pytest.mark.parametrize("m,n,k", [(4100, 8200, 64), (4100, 8200, 192), (2304, 14400, 2752)])
def test_gemm_large_grid_matches_fp32_matmul(m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn((m, k), generator=g).bfloat16()
    w = torch.randn((n, k), generator=g).bfloat16()
    rows = torch.cat([torch.arange(0, 40), torch.randint(0, m, (200,), generator=g), torch.arange(m - 40, m)])
    ref = a[rows].float() @ w.float().t()
    ga, gw = a.cuda(), w.cuda()
    out = torch.zeros((m, n), device="cuda")
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 1, 0, 0, _lib.stream_handle())
    torch.testing.assert_close(out[rows.cuda()].cpu(), ref, atol=1e-3 * k ** 0.5, rtol=1e-4)


# The residual form (fp32 C += A W^T) on the same large ragged grids: the
# accumulators start from the old C (loads clamped at the matrix edges), and
# nothing outside C is written (guard rows before and after it).
@pytest.mark.parametrize("m,n,k", [(4100, 8200, 64), (2304, 14400, 2752)])
def test_gemm_large_grid_accumulates_into_fp32(m, n, k):
    g = torch.Generator().manual_seed(m + n + k + 1)
    a = torch.randn((m, k), generator=g).bfloat16()
    w = torch.randn((n, k), generator=g).bfloat16()
    c0 = torch.randn((m, n), generator=g)
    rows = torch.cat([torch.arange(0, 40), torch.randint(0, m, (200,), generator=g), torch.arange(m - 40, m)])
    ref = c0[rows] + a[rows].float() @ w.float().t()
    ga, gw = a.cuda(), w.cuda()
    c = torch.full(((m + 2) * n,), 7.0, device="cuda")
    cv = c[n:n + m * n].view(m, n)  # one guard row before C, one after
    cv.copy_(c0.cuda())
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), cv.data_ptr(), m, n, k, 1, 0, 1, _lib.stream_handle())
    torch.cuda.synchronize()
    torch.testing.assert_close(cv[rows.cuda()].cpu(), ref, atol=1e-3 * k ** 0.5, rtol=1e-4)
    assert bool((c[:n] == 7.0).all()) and bool((c[n + m * n:] == 7.0).all()), "wrote outside C"


def _sample_rows(m, g):
    return torch.cat([torch.arange(0, 40), torch.randint(0, m, (200,), generator=g), torch.arange(m - 40, m)])


def _bf16_out(shape, aligned, dtype=torch.bfloat16):
    """A zeroed 16-bit output on the GPU; ``aligned=False`` starts it 8 bytes past a
    16-byte boundary (the kernels then store 8 bytes per lane instead of 16)."""
    n = 1
    for s in shape:
        n *= s
    off = 0 if aligned else 4
    buf = torch.zeros(n + off, device="cuda", dtype=dtype)
    out = buf[off:].view(shape)
    assert (out.data_ptr() % 16 == 0) == aligned
    return out


# The bf16 epilogues of the 256 x 384 kernel (q/k/v + RoPE + cache write,
# SwiGLU, plain bf16 output) with ragged M (token tiles spanning two batch
# rows), a ragged N, and outputs that are / are not 16-byte aligned.
@pytest.mark.parametrize("aligned,dtype", [(True, torch.bfloat16), (False, torch.bfloat16), (True, torch.float16)])
def test_gemm_large_grid_bf16_epilogues(aligned, dtype):
    """The 16-bit epilogues (q/k/v + RoPE + cache, SwiGLU, plain) on the large-grid kernel, in
    bf16 (16- and 8-byte stores) and fp16."""
    d, h, f, b, t, cap = 1024, 16, 2752, 4, 3000, 3072
    dk, m = d // h, b * t
    g = torch.Generator().manual_seed(11)
    a = torch.randn((m, d), generator=g).to(dtype)
    wqkv = (torch.randn((3 * d, d), generator=g) * 0.03).to(dtype)
    w1 = (torch.randn((f, d), generator=g) * 0.03).to(dtype)
    w3 = (torch.randn((f, d), generator=g) * 0.03).to(dtype)
    w13 = torch.stack([w1.view(f // 8, 8, d), w3.view(f // 8, 8, d)], dim=1).reshape(2 * f, d).contiguous()
    cos, sin = om.rope_tables(10000.0, dk, cap)
    ga, gqkv, g13 = a.cuda(), wqkv.cuda(), w13.cuda()
    gcos, gsin = cos.t().contiguous().cuda(), sin.t().contiguous().cuda()  # feature-major
    q = _bf16_out((b, h, t, dk), aligned, dtype)
    kc, vc = _bf16_out((b, h, cap, dk), aligned, dtype), _bf16_out((b, h, cap, dk), aligned, dtype)
    hid = _bf16_out((m, f), aligned, dtype)
    n_plain = 8200  # 32 x 256 + 8: the last feature block is partial
    wp = (torch.randn((n_plain, d), generator=g) * 0.03).to(dtype)
    gwp = wp.cuda()
    plain = _bf16_out((m, n_plain), aligned, dtype)
    st = _lib.stream_handle()
    code = _lib.dtype_code(dtype)
    _lib.call("sfl_gemm_qkv_rope", ga.data_ptr(), gqkv.data_ptr(), m, t, d, h, gcos.data_ptr(), gsin.data_ptr(),
              q.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, code, st)
    _lib.call("sfl_gemm_swiglu", ga.data_ptr(), g13.data_ptr(), hid.data_ptr(), m, f, d, code, st)
    _lib.call("sfl_gemm", ga.data_ptr(), gwp.data_ptr(), plain.data_ptr(), m, n_plain, d, code, code, 0, st)
    torch.cuda.synchronize()

    rows = _sample_rows(m, g)
    bi, ti = rows // t, rows % t
    proj = a[rows].float() @ wqkv.float().t()  # [R, 3d]
    c, s = cos[ti][:, None, :], sin[ti][:, None, :]

    def rot(x):  # [R, h, dk], each row at its own position
        out = torch.empty_like(x)
        out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
        out[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
        return out
    qr, kr, vr = (proj[:, i * d:(i + 1) * d].view(-1, h, dk) for i in range(3))
    # fp16 has 3 more mantissa bits than bf16: its 1-ulp flips from fp32 reassociation are 8x as frequent.
    ulp, frac = (2 ** -7, 2e-3) if dtype == torch.bfloat16 else (2 ** -10, 1.6e-2)
    _ulp_close("q (RoPE)", q.cpu()[bi, :, ti], om._round(rot(qr), dtype), frac, ulp=ulp)
    _ulp_close("k cache (RoPE)", kc.cpu()[bi, :, ti], om._round(rot(kr), dtype), frac, ulp=ulp)
    _ulp_close("v cache", vc.cpu()[bi, :, ti], om._round(vr, dtype), frac, ulp=ulp)
    assert not kc[:, :, t:].any() and not vc[:, :, t:].any(), "wrote cache rows past the sequence"
    g1, g3 = a[rows].float() @ w1.float().t(), a[rows].float() @ w3.float().t()
    _ulp_close("SwiGLU hidden", hid.cpu()[rows], om._round(g1 * torch.sigmoid(g1) * g3, dtype), frac, ulp=ulp)
    _ulp_close("plain", plain.cpu()[rows], om._round(a[rows].float() @ wp.float().t(), dtype), frac, ulp=ulp)


# Head dims that are not multiples of 32: a 32-feature MFMA block then holds
# two heads (16) or straddles a head boundary (48). The 256 x 384 kernel
# (large grids), the 128 x 128 one, and for d_model 144 (K % 64 != 0, the
# q | k | v boundaries inside a 32-feature block) the 16x16 kernel.
@pytest.mark.parametrize("dk,h,b,t", [(16, 64, 4, 2600), (48, 16, 4, 3500), (16, 8, 2, 100), (48, 3, 3, 70)])
def test_gemm_qkv_rope_head_dims_across_feature_blocks(dk, h, b, t):
    d, m, cap = dk * h, b * t, t + 16
    g = torch.Generator().manual_seed(dk * 1000 + t)
    a = torch.randn((m, d), generator=g).bfloat16()
    wqkv = (torch.randn((3 * d, d), generator=g) * 0.03).bfloat16()
    cos, sin = om.rope_tables(10000.0, dk, cap)
    q = torch.zeros((b, h, t, dk), device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros((b, h, cap, dk), device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    gcos, gsin = cos.t().contiguous().cuda(), sin.t().contiguous().cuda()  # feature-major
    ga, gw = a.cuda(), wqkv.cuda()
    _lib.call("sfl_gemm_qkv_rope", ga.data_ptr(), gw.data_ptr(), m, t, d, h, gcos.data_ptr(), gsin.data_ptr(),
              q.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, 1, _lib.stream_handle())
    torch.cuda.synchronize()
    rows = _sample_rows(m, g) if m > 400 else torch.arange(m)
    bi, ti = rows // t, rows % t
    proj = a[rows].float() @ wqkv.float().t()
    c, s = cos[ti][:, None, :], sin[ti][:, None, :]

    def rot(x):
        out = torch.empty_like(x)
        out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
        out[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
        return out
    qr, kr, vr = (proj[:, i * d:(i + 1) * d].view(-1, h, dk) for i in range(3))
    _ulp_close(f"q (RoPE, dk {dk})", q.cpu()[bi, :, ti], om._round(rot(qr), torch.bfloat16), 2e-3)
    _ulp_close(f"k cache (RoPE, dk {dk})", kc.cpu()[bi, :, ti], om._round(rot(kr), torch.bfloat16), 2e-3)
    _ulp_close(f"v cache (dk {dk})", vc.cpu()[bi, :, ti], om._round(vr, torch.bfloat16), 2e-3)
    assert not kc[:, :, t:].any() and not vc[:, :, t:].any(), "wrote cache rows past the sequence"


# d % 4 == 0 and d <= 2048 take the one-wave-per-row kernel (m not a multiple
# of its 4 rows per workgroup included); other widths the workgroup-per-row one.
@pytest.mark.parametrize("m,d", [(1, 64), (7, 96), (130, 1024), (33, 2048), (5, 2052), (9, 1030)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rmsnorm_rows_matches_reference(m, d, dtype):
    g = torch.Generator().manual_seed(m * d)
    x = torch.randn((m, d), generator=g) * 3
    w = (1 + 0.5 * torch.randn(d, generator=g)).to(dtype)
    xd, wd = x.cuda(), w.cuda()
    out = torch.zeros((m + 1, d), device="cuda", dtype=torch.bfloat16)  # one guard row
    _lib.call("sfl_rmsnorm_rows", xd.data_ptr(), wd.data_ptr(), out.data_ptr(), m, d, _lib.dtype_code(dtype), 1,
              _lib.stream_handle())
    x64 = x.double()
    ref = (x64 / torch.sqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()).float()
    got = out[:m].float().cpu()
    # One bf16 rounding of a value computed in fp32: half an ulp plus fp32 noise.
    torch.testing.assert_close(got, ref, atol=1e-6, rtol=2 ** -8 + 1e-6)
    # Nearly every value is exactly the bf16 rounding of the reference (the rest sit on a rounding tie).
    assert (got == ref.bfloat16().float()).float().mean().item() > 0.99
    assert not out[m].any(), "wrote past the last row"


@pytest.mark.parametrize("m,d", [(1, 64), (7, 96), (130, 1024), (33, 2048)])
def test_rmsnorm_rows_scaled_splits_the_norm(m, d):
    """The folded norm's input side: bf16(x * w) exactly as the CPU rounds it, and 1 / rms(x)."""
    g = torch.Generator().manual_seed(m * d)
    x = 3 * torch.randn((m, d), generator=g)
    w = (1 + 0.5 * torch.randn(d, generator=g)).bfloat16()
    gx, gw = x.cuda(), w.cuda()
    act = torch.full((m + 1, d), 7.0, device="cuda", dtype=torch.bfloat16)
    rsc = torch.full((m + 1,), -1.0, device="cuda")
    _lib.call("sfl_rmsnorm_rows_scaled", gx.data_ptr(), gw.data_ptr(), act.data_ptr(), rsc.data_ptr(), m, d, 1,
              _lib.stream_handle())
    assert torch.equal(act[:m].cpu(), (x * w.float()).bfloat16())
    torch.testing.assert_close(rsc[:m].cpu(), 1 / torch.sqrt((x * x).mean(-1) + om.EPS), rtol=2e-6, atol=0)
    assert bool((act[m] == 7).all()) and rsc[m].item() == -1.0


# The residual GEMM that also prepares the next RMSNorm: x += A W^T, then
# bf16(x * gain) and per-token sums of x^2 over each 128-feature part, on the
# 128 x 128 tiles (ragged features, a last part of 64) and the 256 x 384 tiles
# (ragged tokens and features), with guard rows around every output; N % 8 ==
# 4 takes the 8-byte stores of the norm input instead of 16-byte ones.
@pytest.mark.parametrize("m,n,k", [(200, 192, 320), (300, 196, 64), (1000, 1024, 64), (24577, 1088, 128)])
def test_gemm_residual_norm_and_norm_scale(m, n, k):
    g = torch.Generator().manual_seed(m + n + k + 7)
    a = torch.randn((m, k), generator=g).bfloat16()
    w = torch.randn((n, k), generator=g).bfloat16()
    x0 = torch.randn((m, n), generator=g)
    gain = (1 + 0.5 * torch.randn(n, generator=g)).bfloat16()
    parts = -(-n // 128)
    xg = torch.full((m + 2, n), float("nan"), device="cuda")
    xg[1:-1] = x0.cuda()
    act = torch.full((m + 1, n), 7.0, device="cuda", dtype=torch.bfloat16)
    ss = torch.full((parts * m + 64,), -1.0, device="cuda")
    rsc = torch.full((m + 1,), -1.0, device="cuda")
    ga, gw, gg = a.cuda(), w.cuda(), gain.cuda()
    st = _lib.stream_handle()
    _lib.call("sfl_gemm_residual_norm", ga.data_ptr(), gw.data_ptr(), xg[1:].data_ptr(), m, n, k, gg.data_ptr(),
              act.data_ptr(), ss.data_ptr(), 1, st)
    _lib.call("sfl_norm_scale", ss.data_ptr(), parts, m, n, rsc.data_ptr(), st)
    x1 = xg[1:-1].cpu()
    assert bool(xg[0].isnan().all()) and bool(xg[-1].isnan().all()), "wrote outside x"
    torch.testing.assert_close(x1, x0 + a.float() @ w.float().t(), atol=1e-3 * k ** 0.5, rtol=1e-4)
    assert torch.equal(act[:m].cpu(), (x1 * gain.float()).bfloat16())
    assert bool((act[m] == 7).all())
    sq = torch.nn.functional.pad(x1 * x1, (0, parts * 128 - n)).view(m, parts, 128).sum(-1).t()
    torch.testing.assert_close(ss[:parts * m].view(parts, m).cpu(), sq, rtol=1e-5, atol=1e-6 * sq.max().item())
    assert bool((ss[parts * m:] == -1).all())
    torch.testing.assert_close(rsc[:m].cpu(), 1 / torch.sqrt((x1 * x1).mean(-1) + om.EPS), rtol=1e-5, atol=0)
    assert rsc[m].item() == -1.0


def gpu_model(cfg, sd, dtype=torch.bfloat16):
    model = TransformerLM.from_config(cfg, device="cuda", dtype=dtype)
    model.load_state_dict(sd)
    return model.eval()


def test_tiny_bf16_forward_via_prefill(golden):
    meta, arrays = golden
    # The golden tiny model has 4 heads of 16; two heads of 32 route forward() through prefill.
    cfg = ModelConfig(**{**meta["tiny"]["config"], "num_heads": 2})
    model = gpu_model(cfg, seeded_state_dict(cfg, meta["tiny"]["seed"]))
    assert model._gemm_prefill()
    ids = torch.from_numpy(arrays["tiny_ids"])
    logits = model(ids.cuda()).float().cpu()
    ref = om.forward(seeded_state_dict(cfg, meta["tiny"]["seed"]), cfg, ids)
    err = (logits - ref).abs().max().item()
    print("tiny (2 heads) bf16 prefill max abs err", err)
    assert err <= 2e-2


def test_tiny_golden_bf16_forward_step_path(golden):
    meta, arrays = golden
    cfg = ModelConfig(**meta["tiny"]["config"])
    model = gpu_model(cfg, seeded_state_dict(cfg, meta["tiny"]["seed"]))
    logits = model(torch.from_numpy(arrays["tiny_ids"]).cuda()).float().cpu()
    err = (logits - torch.from_numpy(arrays["tiny_logits_fp32_sdpa"])).abs().max().item()
    print("tiny bf16 prefill max abs err", err)
    assert err <= 2e-2


def format_floor(sd, cfg, seq, prompt, wide=False, fold=False):
    """The bf16-storage floor of a GEMM prefill of ``prompt`` tokens followed by decode steps:
    bf16 weights and KV cache; bf16 GEMM inputs and probabilities over the prompt chunk only.
    ``wide``: the same with float64-accumulated products (the drift yardstick); ``fold``: the
    prefill stored its norm inputs as bf16(x * g) (the folded-norm path)."""
    cache = om.KVCacheOracle(om.round_weights(sd), cfg, seq.shape[0], seq.shape[1], kv_dtype=torch.bfloat16)
    with om.accumulate_in(torch.float64 if wide else None):
        return torch.cat([cache.step(seq[:, :prompt], act_dtype=torch.bfloat16, norm_fold=fold),
                          cache.step(seq[:, prompt:])], dim=1)


def test_config2_prefill_then_decode_teacher_forced():
    """100.3M bf16, batch 8, the whole context of config 2: GEMM prefill of 512 tokens,
    then teacher-forced decode of the remaining 511 positions to ctx 1024."""
    cfg = load_model_config("scale-100m-s1024")
    sd = seeded_state_dict(cfg, 1337)
    ctx = cfg.context_length  # 1024
    seq = seeded_prompt(cfg.vocab_size, 8, ctx, 2027)
    torch.set_num_threads(16)
    ref = om.KVCacheOracle(sd, cfg, 8, ctx).step(seq)
    rw = om.KVCacheOracle(om.round_weights(sd), cfg, 8, ctx).step(seq)
    model = gpu_model(cfg, sd)
    session = DecodeSession(model, 8, ctx, record_logits=True)
    all_logits = session.prefill(seq[:, :512].cuda(), all_logits=True, forced=seq.cuda())
    session.run(ctx - 1 - 512, use_graph=True)  # positions 512 .. ctx - 2 predict tokens 513 .. ctx - 1
    torch.cuda.synchronize()
    assert session.prefill_norm_folded  # d_model and d_ff are multiples of 64
    floor = format_floor(sd, cfg, seq, 512, fold=True)
    wide = format_floor(sd, cfg, seq, 512, wide=True, fold=True)  # the drift over the same rows the gates compare
    unfolded = format_floor(sd, cfg, seq, 512, fold=False)
    pre = all_logits.cpu()
    dec = session.logits[:, 512:ctx - 1].float().cpu()
    bf16_gate("config2 prefill (positions 0..511)", pre, ref[:, :512], floor[:, :512],
              envelope=(floor[:, :512], wide[:, :512]), ref_bf16_weights=rw[:, :512],
              unfolded_floor=unfolded[:, :512])
    bf16_gate(f"config2 decode after prefill (positions 512..{ctx - 2})", dec, ref[:, 512:ctx - 1],
              floor[:, 512:ctx - 1], envelope=(floor[:, 512:ctx - 1], wide[:, 512:ctx - 1]),
              ref_bf16_weights=rw[:, 512:ctx - 1], unfolded_floor=unfolded[:, 512:ctx - 1])
    # The decode head after prefill (fp32 inputs) equals the prefill's own last-position
    # logits (bf16 GEMM inputs) up to the rounding of the final norm's output.
    torch.testing.assert_close(session.logits[:, 511].float().cpu(), pre[:, 511], atol=2e-2, rtol=0)


@pytest.mark.parametrize("fold", [True, False])
def test_pilot_prefill_with_and_without_folded_norms(fold):
    """22.7M pilot model (head dim 32), batch 4, 200 prompt tokens, all-positions logits: the
    prefill with its norms folded into the GEMMs and the one with separate norm passes, each
    against the storage floor of its own rounding points and the fp32 references (the gates
    of config 2)."""
    cfg = load_model_config("pilot-22m-s256")
    sd = seeded_state_dict(cfg, 7)
    seq = seeded_prompt(cfg.vocab_size, 4, 200, 8)
    model = gpu_model(cfg, sd)
    session = DecodeSession(model, 4, 256)
    session.fold_prefill_norm = fold
    got = session.prefill(seq.cuda(), all_logits=True).cpu()
    assert session.prefill_norm_folded == fold  # d_model 512 and d_ff 1344 are multiples of 64
    torch.set_num_threads(16)
    ref = om.KVCacheOracle(sd, cfg, 4, 256).step(seq)
    rw = om.KVCacheOracle(om.round_weights(sd), cfg, 4, 256).step(seq)
    floor = format_floor(sd, cfg, seq, 200, fold=fold)
    wide = format_floor(sd, cfg, seq, 200, wide=True, fold=fold)
    unfolded = format_floor(sd, cfg, seq, 200, fold=False) if fold else None
    bf16_gate(f"pilot prefill, norms {'folded' if fold else 'separate'}", got, ref, floor, envelope=(floor, wide),
              ref_bf16_weights=rw, unfolded_floor=unfolded)


def _ulp_close(name, got, ref, max_frac, cancel=2 ** -17, ulp=2 ** -7):
    """bf16 results that differ only by rare 1-ulp rounding flips.

    One ulp of the larger value, plus ``cancel`` times the tensor's largest
    value for results formed by cancellation, where a difference in the
    inputs can exceed an ulp of the result: RoPE's e*cos - o*sin near zero
    (fp32 reassociation of its inputs), and an attention output near zero,
    where one flipped bf16 probability moves sum(p v) / l by up to 2^-8 |v|.
    """
    got, ref = got.float().cpu(), ref.float().cpu()
    diff = (got - ref).abs()
    frac = (diff > 0).float().mean().item()
    bound = ulp * torch.maximum(got.abs(), ref.abs()) + cancel * ref.abs().max()
    worst = (diff - bound).max().item()
    print(f"{name}: {frac:.5f} of values differ, max-abs {diff.max().item():.3e}")
    assert frac <= max_frac, f"{name}: {frac} of values differ"
    assert worst <= 0, f"{name}: a difference exceeds one ulp"


@pytest.mark.parametrize("config", ["pilot-22m-s256", "scale-100m-s1024", "scale-324m-s4096"])
def test_prefill_layer_stages_match_the_bf16_format_oracle(config):
    """Each stage of one prefill layer, fed the GPU's own inputs, against the bf16-format oracle:
    bf16 outputs equal up to rare 1-ulp flips (fp32 reassociation at a rounding boundary), fp32
    residual updates to fp32 rounding. The attention matches only with its probabilities stored
    in bf16, as the kernel stores them."""
    cfg = load_model_config(config)
    sd = seeded_state_dict(cfg, 1337)
    sdr = om.round_weights(sd)
    b, t = 2, min(512, cfg.context_length)
    ids = seeded_prompt(cfg.vocab_size, b, t, 2027)
    model = gpu_model(cfg, sd)
    session = DecodeSession(model, b, t)
    d, h, f = cfg.d_model, cfg.num_heads, cfg.d_ff
    dk, m = d // h, b * t
    x = torch.empty((m, d), device="cuda")
    act = torch.empty((m, d), device="cuda", dtype=torch.bfloat16)
    q = torch.empty((b, h, t, dk), device="cuda", dtype=torch.bfloat16)
    attn = torch.empty((b, t, h, dk), device="cuda", dtype=torch.bfloat16)
    hid = torch.empty((m, f), device="cuda", dtype=torch.bfloat16)
    blk, kc, vc = model.layers[0], session.k_cache[0], session.v_cache[0]
    gid = ids.cuda().view(-1)
    st = _lib.stream_handle()
    call = _lib.call
    call("sfl_embed_rows", gid.data_ptr(), model.token_embeddings.weight.data_ptr(), x.data_ptr(), m, d, 1, st)
    x0 = x.clone()
    call("sfl_rmsnorm_rows", x.data_ptr(), blk.attn_norm.weight.data_ptr(), act.data_ptr(), m, d, 1, 1, st)
    act1 = act.clone()
    call("sfl_gemm_qkv_rope", act.data_ptr(), session.wqkv[0].data_ptr(), m, t, d, h, session.cos_fm.data_ptr(),
         session.sin_fm.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), session.cap, 1, st)
    from systems_for_llms_amd.attention import causal_prefill
    causal_prefill(q, kc[:, :, :t], vc[:, :, :t], attn.transpose(1, 2))
    call("sfl_gemm", attn.data_ptr(), blk.attn.output_proj.weight.data_ptr(), x.data_ptr(), m, d, d, 1, 0, 1, st)
    x1 = x.clone()
    call("sfl_rmsnorm_rows", x.data_ptr(), blk.ffn_norm.weight.data_ptr(), act.data_ptr(), m, d, 1, 1, st)
    act2 = act.clone()
    call("sfl_gemm_swiglu", act.data_ptr(), session.weights.w13()[0].data_ptr(), hid.data_ptr(), m, f, d, 1, st)
    call("sfl_gemm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m, d, f, 1, 0, 1, st)
    torch.cuda.synchronize()

    torch.set_num_threads(16)
    bf, p = torch.bfloat16, "layers.0."
    cos, sin = om.rope_tables(cfg.rope_theta, dk, cfg.context_length)
    pos = torch.arange(t)
    x0c = x0.cpu()
    assert torch.equal(x0c, sdr["token_embeddings.weight"][ids].reshape(m, d))
    _ulp_close("rmsnorm (attention input)", act1, om._round(om.rmsnorm(x0c, sdr[p + "attn_norm.weight"]), bf), 1e-3)
    a1 = act1.float().cpu().view(b, t, d)

    def proj(name):
        return om._split_heads(om._linear(a1, sdr[p + f"attn.{name}_proj.weight"]), h)
    _ulp_close("q (RoPE)", q, om._round(om.rope(proj("q"), cos, sin, pos), bf), 2e-3)
    _ulp_close("k cache (RoPE)", kc[:, :, :t], om._round(om.rope(proj("k"), cos, sin, pos), bf), 2e-3)
    _ulp_close("v cache", vc[:, :, :t], om._round(proj("v"), bf), 2e-3)
    qg, kg, vg = q.float().cpu(), kc[:, :, :t].float().cpu(), vc[:, :, :t].float().cpu()
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))
    stored = om._round(om._merge_heads(om.attention_core(qg, kg, vg, mask, bf)), bf)
    _ulp_close("attention (bf16 probabilities)", attn.view(b, t, d), stored, 2e-3, cancel=2 ** -8)
    exact_p = om._round(om._merge_heads(om.attention_core(qg, kg, vg, mask)), bf)
    moved = (attn.view(b, t, d).float().cpu() != exact_p).float().mean().item()
    print(f"attention vs exact probabilities: {moved:.4f} of values differ")
    assert moved > 0.05  # the stored-probability format is what the kernel computes
    x1_ref = x0c + om._linear(attn.float().cpu().view(m, d), sdr[p + "attn.output_proj.weight"])
    torch.testing.assert_close(x1.cpu(), x1_ref, atol=1e-5, rtol=1e-5)
    _ulp_close("rmsnorm (SwiGLU input)", act2, om._round(om.rmsnorm(x1.cpu(), sdr[p + "ffn_norm.weight"]), bf), 1e-3)
    a2 = act2.float().cpu()
    g1 = om._linear(a2, sdr[p + "ffn.w1.weight"])
    _ulp_close("SwiGLU hidden", hid, om._round(g1 * torch.sigmoid(g1) * om._linear(a2, sdr[p + "ffn.w3.weight"]), bf),
               2e-3)
    x2_ref = x1.cpu() + om._linear(hid.float().cpu(), sdr[p + "ffn.w2.weight"])
    torch.testing.assert_close(x.cpu(), x2_ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("config", ["pilot-22m-s256", "scale-100m-s1024", "scale-324m-s4096"])
def test_prefill_folded_norm_stages_match_the_bf16_format_oracle(config):
    """Every layer of a prefill with its norms folded into the GEMMs, each stage fed the GPU's own
    inputs: the norm inputs bf16(x * g) bit-exact, the scales 1 / rms(x) and fp32 residual
    updates to fp32 rounding, the scaled GEMM outputs up to rare 1-ulp flips, the attention (head
    dim 32 on the pilot, 64 otherwise) with its probabilities stored in bf16 as the oracle's
    stored-probability floor computes it; with unit scales the scaled GEMMs are the plain ones,
    bit for bit (layer 0)."""
    cfg = load_model_config(config)
    sd = seeded_state_dict(cfg, 1337)
    sdr = om.round_weights(sd)
    b, t = 2, min(512, cfg.context_length)
    ids = seeded_prompt(cfg.vocab_size, b, t, 2027)
    model = gpu_model(cfg, sd)
    session = DecodeSession(model, b, t)
    d, h, f, nl = cfg.d_model, cfg.num_heads, cfg.d_ff, cfg.num_layers
    dk, m, parts = d // h, b * t, -(-d // 128)
    x = torch.empty((m, d), device="cuda")
    act = torch.empty((m, d), device="cuda", dtype=torch.bfloat16)
    q = torch.empty((b, h, t, dk), device="cuda", dtype=torch.bfloat16)
    attn = torch.empty((b, t, h, dk), device="cuda", dtype=torch.bfloat16)
    hid = torch.empty((m, f), device="cuda", dtype=torch.bfloat16)
    ss = torch.empty((parts, m), device="cuda")
    rsc = torch.empty((m,), device="cuda")
    ones = torch.ones((m,), device="cuda")
    w13 = session.weights.w13()
    gid = ids.cuda().view(-1)
    st = _lib.stream_handle()
    call = _lib.call
    from systems_for_llms_amd.attention import causal_prefill

    def qkv(layer, scale):
        kc, vc = session.k_cache[layer], session.v_cache[layer]
        args = (session.wqkv[layer].data_ptr(),) + ((scale.data_ptr(),) if scale is not None else ())
        call("sfl_gemm_qkv_rope_scaled" if scale is not None else "sfl_gemm_qkv_rope", act.data_ptr(), *args, m, t,
             d, h, session.cos_fm.data_ptr(), session.sin_fm.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
             session.cap, 1, st)
        return q.clone(), kc[:, :, :t].clone(), vc[:, :, :t].clone()

    def swiglu(layer, scale):
        if scale is None:
            call("sfl_gemm_swiglu", act.data_ptr(), w13[layer].data_ptr(), hid.data_ptr(), m, f, d, 1, st)
        else:
            call("sfl_gemm_swiglu_scaled", act.data_ptr(), w13[layer].data_ptr(), scale.data_ptr(), hid.data_ptr(), m,
                 f, d, 1, st)
        return hid.clone()

    # The prefill's own launch sequence (engine.DecodeSession.prefill with folded norms), every
    # intermediate kept: layer i's inputs are the GPU's outputs of layer i - 1.
    call("sfl_embed_rows", gid.data_ptr(), model.token_embeddings.weight.data_ptr(), x.data_ptr(), m, d, 1, st)
    call("sfl_rmsnorm_rows_scaled", x.data_ptr(), model.layers[0].attn_norm.weight.data_ptr(), act.data_ptr(),
         rsc.data_ptr(), m, d, 1, st)
    recs = []
    for layer in range(nl):
        blk = model.layers[layer]
        # ss1: the previous w2 GEMM's sums of squares behind r1 (layer 0's scale comes from the norm pass)
        rec = {"x0": x.clone(), "act1": act.clone(), "r1": rsc.clone(), "ss1": ss.clone()}
        if layer == 0:
            plain, unit = qkv(0, None), qkv(0, ones)
            for p_, u_ in zip(plain, unit):
                assert torch.equal(p_, u_), "unit scales change the q/k/v GEMM"
        rec["q"], rec["k"], rec["v"] = qkv(layer, rsc)
        kc, vc = session.k_cache[layer], session.v_cache[layer]
        causal_prefill(q, kc[:, :, :t], vc[:, :, :t], attn.transpose(1, 2))
        rec["attn"] = attn.clone()
        call("sfl_gemm_residual_norm", attn.data_ptr(), blk.attn.output_proj.weight.data_ptr(), x.data_ptr(), m, d,
             d, blk.ffn_norm.weight.data_ptr(), act.data_ptr(), ss.data_ptr(), 1, st)
        rec["x1"], rec["act2"], rec["ss2"] = x.clone(), act.clone(), ss.clone()
        call("sfl_norm_scale", ss.data_ptr(), parts, m, d, rsc.data_ptr(), st)
        rec["r2"] = rsc.clone()
        if layer == 0:
            assert torch.equal(swiglu(0, None), swiglu(0, ones)), "unit scales change the SwiGLU GEMM"
        rec["hid"] = swiglu(layer, rsc)
        if layer + 1 < nl:
            call("sfl_gemm_residual_norm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m, d, f,
                 model.layers[layer + 1].attn_norm.weight.data_ptr(), act.data_ptr(), ss.data_ptr(), 1, st)
            call("sfl_norm_scale", ss.data_ptr(), parts, m, d, rsc.data_ptr(), st)
        else:  # the last layer's w2 only adds into x (the final norm is a separate pass)
            call("sfl_gemm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m, d, f, 1, 0, 1, st)
        torch.cuda.synchronize()
        recs.append({k: v.cpu() for k, v in rec.items()})
    x_end = x.cpu()

    torch.set_num_threads(16)
    bf = torch.bfloat16
    cos, sin = om.rope_tables(cfg.rope_theta, dk, cfg.context_length)
    pos = torch.arange(t)
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))

    def inv_rms(xx):
        return 1 / torch.sqrt((xx * xx).mean(-1) + om.EPS)

    def split_norm(name, xx, gain, act_, ss_, r_):
        assert torch.equal(act_, (xx * gain).bfloat16()), f"{name}: norm input is not bf16(x * g)"
        if ss_ is not None:
            sq = (xx * xx).view(m, parts, 128).sum(-1).t()
            torch.testing.assert_close(ss_, sq, rtol=1e-5, atol=1e-6 * sq.max().item())
        torch.testing.assert_close(r_, inv_rms(xx), rtol=1e-5, atol=0)

    assert torch.equal(recs[0]["x0"], sdr["token_embeddings.weight"][ids].reshape(m, d))
    for layer, rec in enumerate(recs):
        p = f"layers.{layer}."
        tag = f"layer {layer}"
        if layer == 0:
            split_norm(f"{tag} attention norm", rec["x0"], sdr[p + "attn_norm.weight"], rec["act1"], None, rec["r1"])
        a1, s1 = rec["act1"].float().view(b, t, d), rec["r1"].view(b, t, 1)

        def proj(name):
            return om._split_heads(om._linear(a1, sdr[p + f"attn.{name}_proj.weight"]) * s1, h)
        _ulp_close(f"{tag} q (scaled, RoPE)", rec["q"], om._round(om.rope(proj("q"), cos, sin, pos), bf), 2e-3)
        _ulp_close(f"{tag} k cache (scaled, RoPE)", rec["k"], om._round(om.rope(proj("k"), cos, sin, pos), bf), 2e-3)
        _ulp_close(f"{tag} v cache (scaled)", rec["v"], om._round(proj("v"), bf), 2e-3)
        qg, kg, vg = rec["q"].float(), rec["k"].float(), rec["v"].float()
        stored = om._round(om._merge_heads(om.attention_core(qg, kg, vg, mask, bf)), bf)
        _ulp_close(f"{tag} attention (bf16 probabilities, head dim {dk})", rec["attn"].view(b, t, d), stored, 2e-3,
                   cancel=2 ** -8)
        x1c = rec["x1"]
        torch.testing.assert_close(x1c, rec["x0"] + om._linear(rec["attn"].float().view(m, d),
                                                               sdr[p + "attn.output_proj.weight"]),
                                   atol=1e-5, rtol=1e-5)
        split_norm(f"{tag} ffn norm", x1c, sdr[p + "ffn_norm.weight"], rec["act2"], rec["ss2"], rec["r2"])
        a2, s2 = rec["act2"].float(), rec["r2"][:, None]
        g1 = om._linear(a2, sdr[p + "ffn.w1.weight"]) * s2
        g3 = om._linear(a2, sdr[p + "ffn.w3.weight"]) * s2
        _ulp_close(f"{tag} SwiGLU hidden (scaled)", rec["hid"], om._round(g1 * torch.sigmoid(g1) * g3, bf), 2e-3)
        x2c = recs[layer + 1]["x0"] if layer + 1 < nl else x_end
        torch.testing.assert_close(x2c, x1c + om._linear(rec["hid"].float(), sdr[p + "ffn.w2.weight"]), atol=1e-5,
                                   rtol=1e-5)
        if layer + 1 < nl:
            nxt = recs[layer + 1]
            split_norm(f"layer {layer + 1} attention norm", x2c, sdr[f"layers.{layer + 1}.attn_norm.weight"],
                       nxt["act1"], nxt["ss1"], nxt["r1"])


def test_prefill_bf16_logits_are_the_rounded_fp32_logits():
    """The all-positions lm_head stores bf16 directly for forward(): bit-equal to rounding
    the fp32 logits (one round-to-nearest-even of the same fp32 sums); forward() returns them."""
    cfg = ModelConfig(vocab_size=500, context_length=96, d_model=256, num_layers=2, num_heads=4,
                      d_ff=512, rope_theta=10000.0)
    model = gpu_model(cfg, seeded_state_dict(cfg, 23))
    ids = seeded_prompt(cfg.vocab_size, 3, 80, 24).cuda()
    session = DecodeSession(model, 3, 96)
    f32 = session.prefill(ids, all_logits=True)
    b16 = session.prefill(ids, all_logits=True, logits_dtype=torch.bfloat16)
    assert f32.dtype == torch.float32 and b16.dtype == torch.bfloat16
    assert torch.equal(b16, f32.to(torch.bfloat16))
    assert torch.equal(model(ids), b16)
    with pytest.raises(TypeError):
        session.prefill(ids, all_logits=True, logits_dtype=torch.float16)


def test_generate_bf16_uses_prefill_and_matches_step_path():
    cfg = ModelConfig(vocab_size=500, context_length=96, d_model=256, num_layers=2, num_heads=4,
                      d_ff=512, rope_theta=10000.0)
    sd = seeded_state_dict(cfg, 21)
    model = gpu_model(cfg, sd)
    prompt = seeded_prompt(cfg.vocab_size, 4, 40, 22).cuda()
    ids = model.generate(prompt, 50)
    assert ids.shape == (4, 90) and torch.equal(ids[:, :40], prompt)
    assert bool((ids >= 0).all()) and bool((ids < cfg.vocab_size).all())
    # Teacher-forced on these ids, the step path and the oracle agree with the prefill path's choices.
    ref = om.forward(sd, cfg, ids.cpu())
    agree = (ref[:, 39:-1].argmax(-1) == ids[:, 40:].cpu()).float().mean().item()
    print("generate agreement with fp32 oracle (teacher-forced)", agree)
    assert agree >= 0.95


# ---- float32 prefill (fp32 MFMA GEMMs, fp32 causal attention) ----------------------------

@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (37, 100, 72), (300, 520, 200), (129, 127, 4), (64, 10000, 512)])
def test_gemm_f32_matches_fp64_matmul(m, n, k):
    """sfl_gemm on fp32 operands: fp32 products and sums (v_mfma_f32_32x32x2_f32), ragged M, N and K,
    stored and accumulated, against a float64 product rounded to fp32."""
    g = torch.Generator().manual_seed(m * 7 + n + k)
    a = torch.randn((m, k), generator=g)
    w = torch.randn((n, k), generator=g)
    ref = (a.double() @ w.double().t()).float()
    ga, gw = a.cuda(), w.cuda()
    out = torch.full((m, n), float("nan"), device="cuda")
    st = _lib.stream_handle()
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 0, 0, 0, st)
    tol = 2e-6 * k ** 0.5
    torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=1e-5)
    _lib.call("sfl_gemm", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 0, 0, 1, st)
    torch.testing.assert_close(out.cpu(), 2 * ref, atol=2 * tol, rtol=1e-5)


def test_f32_prefill_stages_match_the_oracle():
    """The fp32 q/k/v (+ RoPE + cache), SwiGLU and causal attention stages of a float32 prefill on
    the GPU's own inputs, against the oracle's restatement in float64."""
    b, t, h, dk, f, cap = 3, 150, 4, 32, 320, 160
    d, m = h * dk, b * t
    g = torch.Generator().manual_seed(5)
    a = torch.randn((m, d), generator=g)
    wqkv = torch.randn((3 * d, d), generator=g) * 0.05
    w1, w3 = (torch.randn((f, d), generator=g) * 0.05 for _ in range(2))
    w13 = torch.stack([w1.view(f // 8, 8, d), w3.view(f // 8, 8, d)], dim=1).reshape(2 * f, d).contiguous()
    cos, sin = om.rope_tables(10000.0, dk, cap)
    ga, gqkv, g13 = a.cuda(), wqkv.cuda(), w13.cuda()
    gcos, gsin = cos.t().contiguous().cuda(), sin.t().contiguous().cuda()
    q = torch.zeros((b, h, t, dk), device="cuda")
    kc, vc = torch.zeros((b, h, cap, dk), device="cuda"), torch.zeros((b, h, cap, dk), device="cuda")
    hid = torch.zeros((m, f), device="cuda")
    attn = torch.zeros((b, t, h, dk), device="cuda")
    st = _lib.stream_handle()
    _lib.call("sfl_gemm_qkv_rope", ga.data_ptr(), gqkv.data_ptr(), m, t, d, h, gcos.data_ptr(), gsin.data_ptr(),
              q.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, 0, st)
    _lib.call("sfl_gemm_swiglu", ga.data_ptr(), g13.data_ptr(), hid.data_ptr(), m, f, d, 0, st)
    from systems_for_llms_amd.attention import causal_prefill
    causal_prefill(q, kc[:, :, :t], vc[:, :, :t], attn.transpose(1, 2))
    torch.cuda.synchronize()

    a64 = a.double().view(b, t, d)
    proj = a64 @ wqkv.double().t()
    pos = torch.arange(t)
    qr, kr, vr = (om._split_heads(proj[..., i * d:(i + 1) * d], h) for i in range(3))
    torch.testing.assert_close(q.cpu(), om.rope(qr, cos.double(), sin.double(), pos).float(), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(kc[:, :, :t].cpu(), om.rope(kr, cos.double(), sin.double(), pos).float(), atol=1e-5,
                               rtol=1e-5)
    torch.testing.assert_close(vc[:, :, :t].cpu(), vr.float(), atol=1e-5, rtol=1e-5)
    assert not kc[:, :, t:].any() and not vc[:, :, t:].any(), "wrote cache rows past the sequence"
    g1, g3 = a.double() @ w1.double().t(), a.double() @ w3.double().t()
    torch.testing.assert_close(hid.cpu(), (g1 * torch.sigmoid(g1) * g3).float(), atol=1e-5, rtol=1e-5)
    qg, kg, vg = q.cpu().double(), kc[:, :, :t].cpu().double(), vc[:, :, :t].cpu().double()
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))
    ref = om._merge_heads(om.attention_core(qg, kg, vg, mask)).float()
    torch.testing.assert_close(attn.cpu().view(b, t, d), ref, atol=1e-5, rtol=1e-5)


def test_f32_forward_is_one_prefill_pass_equal_to_the_oracle():
    """A float32 forward() of the config-1 dims (head dim 32) over 200 positions is one prefill pass
    (no per-position decode steps): its logits equal the oracle's fp32 forward, and the decode steps
    that continue from it give the same logits as the step path from position 0."""
    cfg = load_model_config("pilot-22m-s256")
    sd = seeded_state_dict(cfg, 91)
    model = gpu_model(cfg, sd, torch.float32)
    assert model._gemm_prefill()
    ids = seeded_prompt(cfg.vocab_size, 2, 200, 92)
    logits = model(ids.cuda()).cpu()
    assert model._sfl_session.logits is None  # the prefill path records no per-step logits
    ref = om.forward(sd, cfg, ids)
    err = (logits - ref).abs().max().item()
    print(f"fp32 prefill forward vs oracle max-abs {err:.2e}")
    torch.testing.assert_close(logits, ref, atol=2e-5, rtol=1e-4)
    # Decode after the prefill (positions 200..239) against the step path from position 0.
    seq = seeded_prompt(cfg.vocab_size, 2, 240, 93)
    a = DecodeSession(model, 2, 240, record_logits=True)
    a.prefill(seq[:, :200].cuda(), forced=seq.cuda())
    a.run(39, use_graph=True)
    b = DecodeSession(model, 2, 240, record_logits=True)
    b.start(seq.cuda())
    b.run(239, use_graph=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(a.logits[:, 200:239].cpu(), b.logits[:, 200:239].cpu(), atol=2e-5, rtol=1e-4)
