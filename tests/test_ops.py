"""The ``torch.library`` registration of the operators (``torch.ops.sfl``).

CPU: the schemas (which arguments the ops write) and shape-only dispatch on
meta and fake tensors, which is what tracing (``torch.compile``, export) runs.
GPU: the ops called directly, and through a ``torch.compile`` graph, match the
CPU oracle.
"""

import pytest
import torch

import systems_for_llms_amd.attention  # noqa: F401  (registers the ops)
import systems_for_llms_amd.decode  # noqa: F401


def test_schemas_declare_the_written_arguments():
    decode = str(torch.ops.sfl.decode_attention.default._schema)
    masked = str(torch.ops.sfl.masked_attention.default._schema)
    for name in ("partial_max", "partial_sum", "partial_output", "out"):
        assert f"!) {name}" in decode
    assert "Tensor q," in decode and "Tensor k," in decode and "Tensor lengths" in decode
    assert "!) out" in masked and "!)? lse" in masked
    assert "Tensor? row_ptr" in masked and "Tensor? document_ids" in masked


def _decode_args(device):
    q = torch.empty(2, 8, 64, device=device, dtype=torch.bfloat16)
    k = torch.empty(2, 2, 128, 64, device=device, dtype=torch.bfloat16)
    lengths = torch.empty(2, device=device, dtype=torch.int32)
    pm = torch.empty(2, 8, 3, device=device)
    po = torch.empty(2, 8, 3, 64, device=device)
    return q, k, k, lengths, pm, pm.clone(), po, torch.empty_like(q), 3, 0.125


def test_meta_and_fake_dispatch_launch_nothing():
    torch.ops.sfl.decode_attention(*_decode_args("meta"))
    q = torch.empty(1, 2, 128, 64, device="meta", dtype=torch.bfloat16)
    torch.ops.sfl.masked_attention(q, q, q, torch.empty_like(q), None, 0.125, True, -1, -1, 0, None, None,
                                   None, None, True)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        torch.ops.sfl.decode_attention(*_decode_args("cpu"))


@pytest.mark.gpu
def test_decode_op_and_compiled_graph_match_oracle():
    from oracle.attention import decode_reference

    g = torch.Generator().manual_seed(3)
    q = torch.randn(3, 8, 64, generator=g).bfloat16()
    k = torch.randn(3, 2, 100, 64, generator=g).bfloat16()
    v = torch.randn(3, 2, 100, 64, generator=g).bfloat16()
    lengths = torch.tensor([100, 0, 37], dtype=torch.int32)
    expected = decode_reference(q, k, v, lengths)
    qd, kd, vd, ld = q.cuda(), k.cuda(), v.cuda(), lengths.cuda()
    pm = torch.empty(3, 8, 4, device="cuda")
    ps = torch.empty_like(pm)
    po = torch.empty(3, 8, 4, 64, device="cuda")
    out = torch.empty_like(qd)
    torch.ops.sfl.decode_attention(qd, kd, vd, ld, pm, ps, po, out, 4, 0.125)
    torch.testing.assert_close(out.float().cpu(), expected, atol=0.02, rtol=0.02)

    def step(q_, k_, v_, l_):
        o = torch.empty_like(q_)
        torch.ops.sfl.decode_attention(q_, k_, v_, l_, torch.empty(3, 8, 4, device=q_.device),
                                       torch.empty(3, 8, 4, device=q_.device),
                                       torch.empty(3, 8, 4, 64, device=q_.device), o, 4, 0.125)
        return o * 2

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    torch.testing.assert_close(compiled(qd, kd, vd, ld).float().cpu(), 2 * expected, atol=0.04, rtol=0.02)


@pytest.mark.gpu
def test_masked_op_matches_oracle_with_lse():
    from oracle.attention import dense_mask, masked_attention

    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 2, 130, 64, generator=g).bfloat16() for _ in range(3))
    out, lse = masked_attention(q, k, v, dense_mask(130, causal=True, window_left=40))
    out, lse = out.float(), lse.float()
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    o = torch.empty_like(qd)
    lse_d = torch.empty(1, 2, 130, device="cuda")
    torch.ops.sfl.masked_attention(qd, kd, vd, o, lse_d, 0.125, True, 40, -1, 0, None, None, None, None, True)
    torch.testing.assert_close(o.float().cpu(), out, atol=0.02, rtol=0.02)
    # The row sums come from the bf16-rounded probabilities: the masked-attention tests' bf16 tolerance.
    torch.testing.assert_close(lse_d.cpu(), lse, atol=1e-2, rtol=1e-2)
