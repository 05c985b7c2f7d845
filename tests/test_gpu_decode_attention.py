"""GPU parity of the split-KV decode attention against the CPU oracle.

Follows the reference's preflight suite (attention_lab/cuda_decode/study.py:73-135):
every dtype, head dim and GQA ratio, lengths around tile boundaries, ragged and
empty rows, several split counts, the maximum split count with a custom scale,
a non-default stream and graph replay after lengths change in place.
Tolerances: bf16 0.02, fp16 0.004 (study.py:65-70), fp32 1e-5.
"""

import pytest
import torch

from oracle.attention import decode_reference

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 0.02, torch.float16: 0.004, torch.float32: 1e-5}


def make_inputs(batch, heads, groups, length, dim, dtype, seed, ragged=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((batch, heads, dim), generator=g).to(dtype)
    shape = (batch, heads // groups, length, dim)
    k = torch.randn(shape, generator=g).to(dtype)
    v = torch.randn(shape, generator=g).to(dtype)
    sizes = [min(length, x) for x in (0, 1, max(1, length // 2), length)] if ragged else [length] * batch
    lengths = torch.tensor(sizes, dtype=torch.int32)
    return q, k, v, lengths


def to_gpu(*xs):
    return [x.cuda() for x in xs]


def check(actual, q, k, v, lengths, dtype, scale=None):
    expected = decode_reference(q, k, v, lengths, scale=scale)
    tol = TOL[dtype]
    torch.testing.assert_close(actual.float().cpu(), expected, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dim", [32, 64, 128])
def test_smoke_sweep(dtype, dim):
    from systems_for_llms_amd.decode import prepare

    for groups in (1, 2, 4, 8):
        for length in (1, 31, 32, 33, 127, 513):
            cpu = make_inputs(4, 8, groups, length, dim, dtype, 2027)
            gpu = to_gpu(*cpu)
            for splits in (1, 3, 8, None):
                out = prepare(*gpu, splits=splits)()
                check(out, *cpu, dtype)


def test_maximum_splits_custom_scale():
    from systems_for_llms_amd.decode import prepare

    cpu = make_inputs(4, 8, 2, 33, 128, torch.float16, 93)
    out = prepare(*to_gpu(*cpu), splits=128, scale=0.37)()
    check(out, *cpu, torch.float16, scale=0.37)


def test_non_default_stream_and_graph_replay_with_changed_lengths():
    from systems_for_llms_amd.decode import prepare

    cpu = make_inputs(4, 8, 4, 513, 64, torch.bfloat16, 91)
    gpu = to_gpu(*cpu)
    op = prepare(*gpu, splits=8)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        result = op().clone()
    torch.cuda.current_stream().wait_stream(stream)
    check(result, *cpu, torch.bfloat16)
    with torch.cuda.stream(stream):
        op()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op()
    for sizes in ([513, 256, 0, 3], [1, 2, 3, 4], [513, 513, 513, 513]):
        new = torch.tensor(sizes, dtype=torch.int32)
        gpu[3].copy_(new)
        graph.replay()
        torch.cuda.synchronize()
        check(op.output, cpu[0], cpu[1], cpu[2], new, torch.bfloat16)


def test_config4_shape_sampled_rows():
    """B=64, H=16, D=64, bf16, ragged lengths U[1024, 16384]."""
    from systems_for_llms_amd.decode import prepare

    g = torch.Generator(device="cuda").manual_seed(4)
    b, h, n, d = 64, 16, 16384, 64
    q = torch.randn((b, h, d), device="cuda", generator=g, dtype=torch.bfloat16)
    k = torch.randn((b, h, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
    v = torch.randn((b, h, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
    lengths = torch.randint(1024, n + 1, (b,), generator=torch.Generator().manual_seed(4),
                            dtype=torch.int32).cuda()
    out = prepare(q, k, v, lengths)()
    torch.cuda.synchronize()
    for row in (0, 17, 40, 63):
        sl = slice(row, row + 1)
        check(out[sl], q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), lengths[sl].cpu(), torch.bfloat16)



@pytest.mark.parametrize("groups", [1, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stale_cache_rows_past_the_length_are_ignored(groups, dtype):
    """Cache rows at positions >= length were never written: NaN keys and inf values there must not leak."""
    from systems_for_llms_amd.decode import prepare

    q, k, v, lengths = make_inputs(4, 8, groups, 200, 128, dtype, 4242)
    k_stale, v_stale = k.clone(), v.clone()
    for b, n in enumerate(lengths.tolist()):
        k_stale[b, :, n:] = float("nan")
        v_stale[b, :, n:] = float("inf")
    gpu = to_gpu(q, k_stale, v_stale, lengths)
    for splits in (1, 3, None):
        check(prepare(*gpu, splits=splits)(), q, k, v, lengths, dtype)


@pytest.mark.parametrize("dim", [64, 128])
def test_grouped_long_ragged_caches(dim):
    """Grouped heads over caches of many 32-key tiles per wave, lengths off every tile boundary."""
    from systems_for_llms_amd.decode import prepare

    g = torch.Generator().manual_seed(dim)
    q = torch.randn((4, 32, dim), generator=g).bfloat16()
    k = torch.randn((4, 4, 3001, dim), generator=g).bfloat16()
    v = torch.randn((4, 4, 3001, dim), generator=g).bfloat16()
    lengths = torch.tensor([3001, 1499, 97, 2048], dtype=torch.int32)
    gpu = to_gpu(q, k, v, lengths)
    for splits in (1, 5, 128, None):
        check(prepare(*gpu, splits=splits)(), q, k, v, lengths, torch.bfloat16)


@pytest.mark.parametrize("groups", [4, 8])
def test_grouped_outputs_in_every_output_dtype(groups):
    """bf16 q/k/v through the C ABI into bf16, fp32 and the split-bf16 activation layout, one and several splits."""
    from systems_for_llms_amd import _lib

    batch, heads, dim, cap = 3, 16, 64, 300
    g = torch.Generator().manual_seed(groups)
    q = torch.randn(batch, heads, dim, generator=g).bfloat16()
    k = torch.randn(batch, heads // groups, cap, dim, generator=g).bfloat16()
    v = torch.randn(batch, heads // groups, cap, dim, generator=g).bfloat16()
    lengths = torch.tensor([300, 0, 129], dtype=torch.int32)
    expected = decode_reference(q, k, v, lengths)
    qd, kd, vd, ld = to_gpu(q, k, v, lengths)
    k_dim = heads * dim
    for splits in (1, 4):
        pmax = torch.empty(batch * heads * splits, device="cuda")
        psum = torch.empty_like(pmax)
        pout = torch.empty(batch * heads * splits * dim, device="cuda")
        outs = {_lib.DTYPE_CODES[torch.bfloat16]: torch.empty(batch, k_dim, device="cuda", dtype=torch.bfloat16),
                _lib.DTYPE_CODES[torch.float32]: torch.empty(batch, k_dim, device="cuda"),
                _lib.DTYPE_BF16X2: torch.zeros(16 * k_dim, device="cuda")}
        for code, out in outs.items():
            _lib.call("sfl_decode_attention", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ld.data_ptr(),
                      pmax.data_ptr(), psum.data_ptr(), pout.data_ptr(), out.data_ptr(), batch, heads,
                      heads // groups, cap, dim, splits, dim ** -0.5, 1, 1, code, _lib.stream_handle())
        torch.cuda.synchronize()
        flat = expected.reshape(batch, k_dim)
        torch.testing.assert_close(outs[1].float().cpu(), flat, atol=0.02, rtol=0.02)
        torch.testing.assert_close(outs[0].cpu(), flat, atol=0.01, rtol=0.01)
        # Split-bf16 layout: [k_dim / 32 chunks][hi, lo][4 groups][16 rows][8 values] per 16-row block.
        halves = outs[_lib.DTYPE_BF16X2].cpu().view(torch.bfloat16).view(k_dim // 32, 2, 4, 16, 8).float()
        laid = (halves[:, 0] + halves[:, 1]).permute(2, 0, 1, 3).reshape(16, k_dim)[:batch]
        assert ((laid - outs[0].cpu()).abs() <= outs[0].cpu().abs() * 2.0 ** -14).all()


def test_rejections_before_launch():
    from systems_for_llms_amd.decode import prepare

    q = torch.zeros(1, 8, 64, dtype=torch.float16, device="cuda")
    k = torch.zeros(1, 2, 17, 64, dtype=torch.float16, device="cuda")
    for splits in (0, 129, True, 2.5):
        with pytest.raises(ValueError, match="splits"):
            prepare(q, k, k, splits=splits)
    with pytest.raises(ValueError, match="variant"):
        prepare(q, k, k, variant="approximate")
    with pytest.raises(ValueError, match="divisible"):
        prepare(q[:, :7].contiguous(), k, k)
    with pytest.raises(ValueError, match="length"):
        prepare(q, k, k, torch.tensor([18], dtype=torch.int32, device="cuda"))
