"""GPU edge cases the reference's semantics fix: argmax ties, empty attention rows, untouched inputs.

* Greedy ties: ``torch.argmax`` (the reference's greedy choice, applied to
  ``forward(ids)[:, -1]``) returns the first maximal index. Planted exact ties
  within one 16-row lm_head tile, across tiles and across the next-token
  kernel's scan rounds (1024 tiles per round) must resolve to the lowest index,
  eagerly and under graph replay, through the C ABI and through ``generate``.
* Empty rows of the masked attention: zero output and LSE ``-inf``
  (``attention_lab/triton_attention.py:191-197``), for a CSR row with no tiles
  and for a row whose only tile the token mask excludes entirely.
* Inputs unchanged (``attention_lab/benchmark.py:321,335``): the attention
  operators leave q/k/v as they were, and a decode step writes the KV cache at
  the append position only.
"""

import pytest
import torch

from oracle.attention import scheduled_attention
from systems_for_llms_amd import _lib
from systems_for_llms_amd.config import ModelConfig
from systems_for_llms_amd.engine import DecodeSession
from systems_for_llms_amd.masks import MaskSpec, compile_mask
from systems_for_llms_amd.model import TransformerLM
from systems_for_llms_amd.weights import seeded_prompt, seeded_state_dict

pytestmark = pytest.mark.gpu

VOCAB, D = 20000, 128  # 1250 lm_head tiles: two scan rounds of the next-token kernel
# (rows that tie, expected winner): same tile, same lane group; same tile, other lane groups;
# different tiles in one scan round; different scan rounds (tile 1062 is in round 1); three rows.
TIES = (((5003, 5000), 5000), ((5013, 5001), 5001), ((9000, 100), 100), ((17000, 300), 300),
        ((19999, 16384, 700), 700))


def planted_head(dtype, column_for_case):
    """lm_head [VOCAB, D]: small noise, and for case c the rows of TIES[c] hold 1.0 in column c."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn((VOCAB, D), generator=g) * 0.01
    for c, (rows, _) in enumerate(TIES):
        w[list(rows), column_for_case(c)] = 1.0
    return w.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lm_head_argmax_ties_lowest_index_c_abi(dtype):
    """Batch row c has x = e_c, so its logits are sqrt(D) * w[:, c] (exact): case c's rows tie."""
    batch = len(TIES)
    code = _lib.dtype_code(dtype)
    w = planted_head(dtype, lambda c: c).cuda()
    packed = _lib.pack_gemv(w)
    x = torch.zeros((batch, D), device="cuda")
    x[torch.arange(batch), torch.arange(batch)] = 1.0
    gain = torch.ones(D, device="cuda", dtype=dtype)
    tiles = _lib.lib().sfl_lm_head_tiles(VOCAB)
    best_val = torch.empty((tiles, batch), device="cuda")
    best_idx = torch.empty((tiles, batch), device="cuda", dtype=torch.int32)
    logits = torch.zeros((batch, VOCAB), device="cuda")
    cap = 4
    tokens = torch.zeros((batch, cap), device="cuda", dtype=torch.int64)
    predicted = torch.full((batch, cap), -1, device="cuda", dtype=torch.int64)
    pos = torch.zeros(batch, device="cuda", dtype=torch.int32)
    lengths = torch.ones(batch, device="cuda", dtype=torch.int32)
    prompt_len = torch.ones(batch, device="cuda", dtype=torch.int32)
    emb = torch.zeros((VOCAB, D), device="cuda", dtype=dtype)
    x_next = torch.empty_like(x)

    def step():
        st = _lib.stream_handle()
        _lib.call("sfl_rmsnorm_lm_head", x.data_ptr(), gain.data_ptr(), packed.data_ptr(), logits.data_ptr(),
                  VOCAB, None, 0, best_val.data_ptr(), best_idx.data_ptr(), batch, batch, D, VOCAB, code, st)
        _lib.call("sfl_next_token", best_val.data_ptr(), best_idx.data_ptr(), tiles, batch, tokens.data_ptr(),
                  predicted.data_ptr(), cap, prompt_len.data_ptr(), pos.data_ptr(), lengths.data_ptr(),
                  emb.data_ptr(), x_next.data_ptr(), batch, D, cap, code, st)

    expected = torch.tensor([winner for _, winner in TIES])
    step()
    torch.cuda.synchronize()
    for c, (rows, _) in enumerate(TIES):
        vals = logits[c, list(rows)].cpu()
        assert torch.equal(vals, vals[:1].expand_as(vals)), f"case {c}: planted rows do not tie exactly"
    assert torch.equal(logits.argmax(-1).cpu(), expected)  # torch.argmax agrees: first index
    assert torch.equal(predicted[:, 1].cpu(), expected)
    assert torch.equal(tokens[:, 1].cpu(), expected)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for replay in range(3):
        pos.zero_()
        predicted.fill_(-1)
        tokens.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(predicted[:, 1].cpu(), expected), f"graph replay {replay}"
        assert torch.equal(tokens[:, 1].cpu(), expected), f"graph replay {replay}"


@pytest.mark.parametrize("use_graph", [False, True])
def test_generate_resolves_planted_ties_to_lowest_index(use_graph):
    """Through the model: layer weights zero and every embedding row ones, so x stays ones and
    the logits are the row sums of lm_head; rows planted with 0.02 everywhere (sum 2.56, the
    N(0, 0.02) rows sum to about N(0, 0.23)) tie at the top."""
    cfg = ModelConfig(vocab_size=VOCAB, context_length=16, d_model=D, num_layers=2, num_heads=2, d_ff=256,
                      rope_theta=10000.0)
    sd = seeded_state_dict(cfg, 5)
    for name in sd:
        if name.startswith("layers.") and not name.endswith("norm.weight"):
            sd[name].zero_()
    sd["token_embeddings.weight"].fill_(1.0)
    model = TransformerLM.from_config(cfg, device="cuda", dtype=torch.float32)
    model.load_state_dict(sd)
    model.eval()
    prompt = torch.zeros((1, 3), dtype=torch.int64, device="cuda")
    for rows, winner in TIES:
        head = sd["lm_head.weight"].clone()
        head[list(rows)] = 0.02
        with torch.no_grad():
            model.lm_head.weight.copy_(head)  # in place: the cached decode weights must follow
        ids = model.generate(prompt, 6, use_graph=use_graph).cpu()
        assert torch.equal(ids[0, 3:], torch.full((6,), winner)), (rows, ids.tolist())


def _edited_schedule(n, spec):
    """A compiled causal schedule edited so that query row 2 has no tiles and row 1's only
    tile is the (entirely future, hence fully masked) key tile 2."""
    sched = compile_mask(n, spec, 64, 64)
    rows = [sched.col_idx[sched.row_ptr[r]:sched.row_ptr[r + 1]] for r in range(len(sched.row_ptr) - 1)]
    full = [sched.full_blocks[sched.row_ptr[r]:sched.row_ptr[r + 1]] for r in range(len(sched.row_ptr) - 1)]
    rows[1], full[1] = [2], [False]
    rows[2], full[2] = [], []
    sched.col_idx = [c for r in rows for c in r]
    sched.full_blocks = [f for r in full for f in r]
    sched.row_ptr = [0]
    for r in rows:
        sched.row_ptr.append(sched.row_ptr[-1] + len(r))
    return sched


@pytest.mark.parametrize("d", [32, 64, 128])
def test_masked_attention_empty_rows_give_zero_and_negative_infinite_lse(d):
    from systems_for_llms_amd.attention import attention

    n = 260
    spec = MaskSpec(causal=True)
    sched = _edited_schedule(n, spec)
    g = torch.Generator().manual_seed(d)
    q, k, v = (torch.randn((2, 3, n, d), generator=g).to(torch.bfloat16) for _ in range(3))
    for use_full in (True, False):
        out, lse = attention(q.cuda(), k.cuda(), v.cuda(), sched, spec, implementation="csr",
                             use_full_blocks=use_full, return_lse=True)
        torch.cuda.synchronize()
        out, lse = out.float().cpu(), lse.cpu()
        empty = slice(64, 192)  # query rows 1 and 2
        assert torch.equal(out[:, :, empty], torch.zeros_like(out[:, :, empty]))
        assert torch.isneginf(lse[:, :, empty]).all()
        assert torch.isfinite(out).all() and torch.isfinite(lse[:, :, :64]).all()
        ref = scheduled_attention(q, k, v, sched, spec, use_full_blocks=use_full)
        torch.testing.assert_close(out, ref.float(), atol=2e-2, rtol=2e-2)


def test_attention_operators_leave_inputs_unchanged():
    from systems_for_llms_amd.attention import attention
    from systems_for_llms_amd.decode import prepare

    g = torch.Generator(device="cuda").manual_seed(17)
    for heads, kv_heads, dim in ((16, 16, 64), (32, 4, 128), (8, 4, 32)):
        q = torch.randn((3, heads, dim), device="cuda", generator=g, dtype=torch.bfloat16)
        k = torch.randn((3, kv_heads, 700, dim), device="cuda", generator=g, dtype=torch.bfloat16)
        v = torch.randn_like(k)
        lengths = torch.tensor([700, 1, 333], dtype=torch.int32, device="cuda")
        before = [t.clone() for t in (q, k, v, lengths)]
        for splits in (1, 4, None):
            prepare(q, k, v, lengths, splits=splits)()
        torch.cuda.synchronize()
        for t, b in zip((q, k, v, lengths), before):
            assert torch.equal(t, b)
    spec = MaskSpec(causal=True, window_left=100, global_prefix=64)
    q, k, v = (torch.randn((2, 4, 300, 64), device="cuda", generator=g, dtype=torch.bfloat16) for _ in range(3))
    before = [t.clone() for t in (q, k, v)]
    for impl in ("csr", "interval"):
        attention(q, k, v, compile_mask(300, spec), spec, implementation=impl, return_lse=True)
    torch.cuda.synchronize()
    for t, b in zip((q, k, v), before):
        assert torch.equal(t, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_step_writes_the_cache_only_at_the_append_position(dtype):
    cfg = ModelConfig(vocab_size=300, context_length=40, d_model=128, num_layers=2, num_heads=4, d_ff=256,
                      rope_theta=10000.0)
    model = TransformerLM.from_config(cfg, device="cuda", dtype=dtype)
    model.load_state_dict(seeded_state_dict(cfg, 9))
    model.eval()
    session = DecodeSession(model, batch=3, capacity=40, record_logits=True)
    session.start(seeded_prompt(cfg.vocab_size, 3, 10, 10).cuda())
    session.run(7, use_graph=True)  # positions 0..6 written
    torch.cuda.synchronize()
    session.k_cache[:, :, :, 8:].fill_(float("nan"))  # stale rows past the length
    session.v_cache[:, :, :, 8:].fill_(float("nan"))
    k0, v0 = session.k_cache.clone(), session.v_cache.clone()
    weights = {name: p.detach().clone() for name, p in model.named_parameters()}
    session.step()  # position 7
    torch.cuda.synchronize()

    def moved(a, b):
        return ~((a == b) | (a.isnan() & b.isnan()))

    changed = moved(session.k_cache, k0) | moved(session.v_cache, v0)
    positions = changed.any(dim=4).any(dim=2).any(dim=1).any(dim=0).nonzero().flatten().tolist()
    assert positions == [7], positions
    assert changed[:, :, :, 7].all() or dtype == torch.bfloat16  # fp32: every appended value is new
    assert torch.isnan(session.k_cache[:, :, :, 8:]).all()  # untouched, and never read:
    assert torch.isfinite(session.logits[:, 7]).all()
    for name, p in model.named_parameters():
        assert torch.equal(p.detach(), weights[name]), name
