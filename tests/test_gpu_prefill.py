"""GPU parity of the bf16 MFMA prefill path (GEMMs + masked attention) against the oracle."""

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
@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (37, 100, 72), (128, 128, 64), (300, 520, 200), (64, 3072, 1024),
                                   (300, 520, 256), (5, 10000, 128), (129, 127, 192), (1000, 36, 2752)])
def test_gemm_matches_fp32_matmul(m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn((m, k), generator=g).bfloat16()
    w = torch.randn((n, k), generator=g).bfloat16()
    ref = a.float() @ w.float().t()
    ga, gw = a.cuda(), w.cuda()  # keep the device copies alive across the launches
    out = torch.zeros((m, n), device="cuda")
    st = _lib.stream_handle()
    _lib.call("sfl_gemm_bf16", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 0, 0, st)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-3, rtol=1e-4)
    _lib.call("sfl_gemm_bf16", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 0, 1, st)
    torch.testing.assert_close(out.cpu(), 2 * ref, atol=2e-3, rtol=1e-4)
    ob = torch.zeros((m, n), device="cuda", dtype=torch.bfloat16)
    _lib.call("sfl_gemm_bf16", ga.data_ptr(), gw.data_ptr(), ob.data_ptr(), m, n, k, 1, 0, st)
    torch.testing.assert_close(ob.float().cpu(), ref.bfloat16().float(), atol=1e-2, rtol=1e-2)


# Grids of >= 512 tiles of 256 x 256 take the 256 x 256 kernel with its ring
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
    _lib.call("sfl_gemm_bf16", ga.data_ptr(), gw.data_ptr(), out.data_ptr(), m, n, k, 0, 0, _lib.stream_handle())
    torch.testing.assert_close(out[rows.cuda()].cpu(), ref, atol=1e-3 * k ** 0.5, rtol=1e-4)


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
    _lib.call("sfl_rmsnorm_rows", xd.data_ptr(), wd.data_ptr(), out.data_ptr(), m, d, _lib.dtype_code(dtype),
              _lib.stream_handle())
    x64 = x.double()
    ref = (x64 / torch.sqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()).float()
    got = out[:m].float().cpu()
    # One bf16 rounding of a value computed in fp32: half an ulp plus fp32 noise.
    torch.testing.assert_close(got, ref, atol=1e-6, rtol=2 ** -8 + 1e-6)
    # Nearly every value is exactly the bf16 rounding of the reference (the rest sit on a rounding tie).
    assert (got == ref.bfloat16().float()).float().mean().item() > 0.99
    assert not out[m].any(), "wrote past the last row"


def gpu_model(cfg, sd):
    model = TransformerLM.from_config(cfg, device="cuda", dtype=torch.bfloat16)
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


def test_config2_prefill_then_decode_teacher_forced():
    """100.3M bf16, batch 8: GEMM prefill of 512 tokens, then 64 teacher-forced decode positions.

    The floor models the formats the prefill stores: bf16 weights and KV cache,
    and bf16 GEMM inputs (RMSNorm outputs, q, attention output, SwiGLU hidden)
    for the 512 prompt positions; the decode positions keep fp32 inputs.
    """
    cfg = load_model_config("scale-100m-s1024")
    sd = seeded_state_dict(cfg, 1337)
    seq = seeded_prompt(cfg.vocab_size, 8, 576, 2027)
    torch.set_num_threads(16)
    ref = om.KVCacheOracle(sd, cfg, 8, 576).step(seq)
    cache = om.KVCacheOracle(om.round_weights(sd), cfg, 8, 576, kv_dtype=torch.bfloat16)
    floor = torch.cat([cache.step(seq[:, :512], act_dtype=torch.bfloat16), cache.step(seq[:, 512:])], dim=1)
    model = gpu_model(cfg, sd)
    session = DecodeSession(model, 8, 576, record_logits=True)
    all_logits = session.prefill(seq[:, :512].cuda(), all_logits=True, forced=seq.cuda())
    session.run(64, use_graph=True)
    torch.cuda.synchronize()
    pre = all_logits.cpu()
    dec = session.logits[:, 512:575].float().cpu()
    bf16_gate("config2 prefill (positions 0..511)", pre, ref[:, :512], floor[:, :512])
    bf16_gate("config2 decode after prefill (positions 512..574)", dec, ref[:, 512:575], floor[:, 512:575])
    # The decode head after prefill (fp32 inputs) equals the prefill's own last-position
    # logits (bf16 GEMM inputs) up to the rounding of the final norm's output.
    torch.testing.assert_close(session.logits[:, 511].float().cpu(), pre[:, 511], atol=2e-2, rtol=0)


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
