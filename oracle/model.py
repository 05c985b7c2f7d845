"""CPU restatement of the reference ``TransformerLM`` forward and a greedy token loop.

Follows ``src/llmlab/model/layers.py``, ``attention.py`` and ``transformer.py``:
the numerics that decide rounding are kept as the reference has them --
RMSNorm computes in fp32 and divides by ``sqrt(mean(x^2)+eps)``
(``layers.py:133-141``); the RoPE table is built in fp32 and cast to the
activation dtype before the multiply (``attention.py:31-42,49-50``); attention
scales after ``QK^T`` and runs softmax in fp32 for 16-bit inputs
(``attention.py:68-98``); SwiGLU is ``w2(silu(w1 x) * w3 x)`` (``layers.py:114-115``).
Weights are a plain ``state_dict`` with the reference's keys.
"""

from __future__ import annotations

import contextlib
import math

import torch

EPS = 1e-5
_ACC = None  # accumulation dtype of the matrix products (None: the operands' own)


@contextlib.contextmanager
def accumulate_in(dtype):
    """Run the oracle's matrix products with ``dtype`` accumulation, results cast back.

    Not reference behaviour: with ``torch.float64`` it gives a second, equally
    valid restatement whose fp32 results differ from the default only in
    rounding, the yardstick for how far two exact computations drift apart
    under the same storage formats.
    """
    global _ACC
    previous, _ACC = _ACC, dtype
    try:
        yield
    finally:
        _ACC = previous


def _mm(a, b):
    if _ACC is None:
        return torch.matmul(a, b)
    return torch.matmul(a.to(_ACC), b.to(_ACC)).to(a.dtype)


def rope_tables(theta: float, d_k: int, max_seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin ``[max_seq_len, d_k/2]`` as ``attention.py:31-42`` builds them."""
    positions = torch.arange(max_seq_len)
    pairs = torch.arange(0, d_k, 2)
    inverse = 1.0 / (theta ** (pairs / d_k))
    angles = positions.to(torch.float32)[:, None] * inverse[None, :]
    return torch.cos(angles), torch.sin(angles)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``layers.py:133-141``."""
    dtype = x.dtype
    x = x.to(torch.float32)
    rms = torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + EPS)
    return ((x / rms) * weight).to(dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation, ``attention.py:44-58``; x is ``[..., T, d_k]``."""
    c = cos[positions].to(x.dtype)
    s = sin[positions].to(x.dtype)
    even, odd = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = even * c - odd * s
    out[..., 1::2] = even * s + odd * c
    return out


def attention_core(q, k, v, mask, p_dtype=None):
    """Eager masked attention, ``attention.py:61-98``; mask True = allowed.

    ``p_dtype`` (not in the reference; a storage-format floor) stores the
    softmax probabilities in that format as a batched prefill kernel does:
    see ``_attention_stored_probabilities``.
    """
    if p_dtype is not None:
        return _attention_stored_probabilities(q, k, v, mask, p_dtype)
    scores = _mm(q, k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    scores = scores.masked_fill(~mask, float("-inf"))
    work = scores.float() if scores.dtype in (torch.bfloat16, torch.float16) else scores
    peak = torch.max(work, dim=-1, keepdim=True).values
    e = torch.exp(work - peak)
    weights = (e / torch.sum(e, dim=-1, keepdim=True)).to(scores.dtype)
    return _mm(weights, v)


BLOCK_K = 64      # key tile of the batched (prefill) attention
LAZY_LOG2 = 8.0   # slack of its running maximum, in log2 units
LOG2E = 1.4426950408889634


def _attention_stored_probabilities(q, k, v, mask, p_dtype):
    """Online-softmax attention over 64-key tiles with the probabilities stored in ``p_dtype``.

    The format floor of a flash-style prefill kernel that feeds its P.V
    products with narrow probabilities: per query, key tiles in ascending
    order; a running maximum m (log2 units) that moves to a tile's maximum
    only when that exceeds it by more than ``LAZY_LOG2`` (rescaling the
    accumulators by 2^(m_old - m_new)); probabilities p = 2^(s*c - m), with
    c = scale * log2(e) in fp32, rounded to ``p_dtype``; row sum l and output
    accumulated from the rounded p in fp32; out = o * (1/l), zero for a row
    with no admissible key. The result equals softmax attention up to those
    roundings; the same scores with exact probabilities give ``attention_core``.
    """
    f32 = torch.float32
    c = torch.tensor(q.shape[-1] ** -0.5, dtype=f32) * torch.tensor(LOG2E, dtype=f32)
    scores = _mm(q.to(f32), k.to(f32).transpose(-1, -2)).masked_fill(~mask, float("-inf"))
    lead, n_keys = scores.shape[:-1], scores.shape[-1]
    m = torch.full(lead, float("-inf"), dtype=f32)
    l = torch.zeros(lead, dtype=f32)
    o = torch.zeros((*lead, v.shape[-1]), dtype=f32)
    for k0 in range(0, n_keys, BLOCK_K):
        tile = scores[..., k0:k0 + BLOCK_K]
        top = tile.amax(dim=-1) * c
        grow = top > m + LAZY_LOG2  # never for a tile with no admissible key (top = -inf)
        m_new = torch.where(grow, top, m)
        alpha = torch.where(grow, torch.exp2(m - m_new), torch.ones_like(m))
        m = m_new
        shift = torch.where(torch.isinf(m), torch.zeros_like(m), m)
        # fma(s, c, -shift) rounds once: form it in float64, round to fp32.
        p = torch.exp2((tile.double() * c.double() - shift.double()[..., None]).to(f32))
        p = p.to(p_dtype).to(f32)
        l = l * alpha + p.sum(dim=-1)
        o = o * alpha[..., None] + _mm(p, v[..., k0:k0 + BLOCK_K, :].to(f32))
    inv = torch.where(l > 0, 1.0 / torch.where(l > 0, l, torch.ones_like(l)), torch.zeros_like(l))
    return (o * inv[..., None]).to(q.dtype)


def _linear(x, w):
    return _mm(x, w.t())


def _split_heads(x, heads):
    *lead, t, d = x.shape
    return x.reshape(*lead, t, heads, d // heads).transpose(-3, -2)


def _merge_heads(x):
    *lead, h, t, dk = x.shape
    return x.transpose(-3, -2).reshape(*lead, t, h * dk)


def _round(t: torch.Tensor, dtype) -> torch.Tensor:
    """``t`` rounded through a narrower storage format (no-op for ``None``)."""
    return t if dtype is None else t.to(dtype).to(t.dtype)


def _norm_input(x, weight, act_dtype, fold):
    """The GEMM input made from ``rmsnorm(x, weight)`` and the per-token factor for its products.

    ``fold`` (not in the reference; the storage-format floor of a prefill that
    folds the norm into its GEMMs): the stored input is ``x * weight`` and the
    products are scaled by ``r = 1 / sqrt(mean(x^2) + eps)`` afterwards -- the
    same value in exact arithmetic, rounded at another point. Otherwise the
    norm's output itself is stored and the factor is ``None`` (one).
    """
    if not fold:
        return _round(rmsnorm(x, weight), act_dtype), None
    r = 1.0 / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + EPS)
    return _round(x * weight, act_dtype), r


def _scaled(y, r):
    return y if r is None else y * r


def _layer(sd, prefix, x, heads, cos, sin, positions, mask, kv_dtype=None, act_dtype=None):
    h = _round(rmsnorm(x, sd[prefix + "attn_norm.weight"]), act_dtype)
    q = _split_heads(_linear(h, sd[prefix + "attn.q_proj.weight"]), heads)
    k = _split_heads(_linear(h, sd[prefix + "attn.k_proj.weight"]), heads)
    v = _split_heads(_linear(h, sd[prefix + "attn.v_proj.weight"]), heads)
    q = _round(rope(q, cos, sin, positions), act_dtype)
    k = rope(k, cos, sin, positions)
    if kv_dtype is not None:  # keys/values stored in a narrower cache format
        k = k.to(kv_dtype).to(x.dtype)
        v = v.to(kv_dtype).to(x.dtype)
    a = _round(_merge_heads(attention_core(q, k, v, mask, act_dtype)), act_dtype)
    x = x + _linear(a, sd[prefix + "attn.output_proj.weight"])
    h = _round(rmsnorm(x, sd[prefix + "ffn_norm.weight"]), act_dtype)
    a = _linear(h, sd[prefix + "ffn.w1.weight"])
    g = _round(a * torch.sigmoid(a) * _linear(h, sd[prefix + "ffn.w3.weight"]), act_dtype)
    x = x + _linear(g, sd[prefix + "ffn.w2.weight"])
    return x


@torch.no_grad()
def forward(sd: dict, config, input_ids: torch.Tensor, dtype=torch.float32, kv_dtype=None,
            act_dtype=None) -> torch.Tensor:
    """``TransformerLM.forward`` (``transformer.py:121-139``): logits ``[..., T, V]``.

    Not in the reference, for bounding what storage formats alone change:
    ``kv_dtype`` rounds keys and values through a cache format; ``act_dtype``
    rounds what a batched prefill stores in a narrow format -- the GEMM inputs
    (the RMSNorm outputs, the final one included, q after RoPE, the merged
    attention output and the SwiGLU hidden state) and the attention's softmax
    probabilities (``attention_core``'s ``p_dtype``); the residual stream stays
    in ``dtype``.
    """
    if not 0 < input_ids.shape[-1] <= config.context_length:
        raise ValueError("sequence length must be between 1 and context_length")
    sd = {name: t.to(dtype) for name, t in sd.items()}
    cos, sin = rope_tables(config.rope_theta, config.d_model // config.num_heads, config.context_length)
    t = input_ids.shape[-1]
    positions = torch.arange(t)
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))
    x = sd["token_embeddings.weight"][input_ids]
    for layer in range(config.num_layers):
        x = _layer(sd, f"layers.{layer}.", x, config.num_heads, cos, sin, positions, mask, kv_dtype, act_dtype)
    x = _round(rmsnorm(x, sd["ln_final.weight"]), act_dtype)
    return _linear(x, sd["lm_head.weight"])


def round_weights(sd: dict, dtype=torch.bfloat16) -> dict:
    """The same state_dict with every tensor rounded through ``dtype`` and back to fp32.

    ``forward(round_weights(sd), ...)`` is the bf16-weight model with exact
    fp32 arithmetic: the accuracy floor of any kernel that stores bf16 weights.
    """
    return {name: t.to(dtype).to(torch.float32) for name, t in sd.items()}


def greedy_argmax(logits: torch.Tensor) -> torch.Tensor:
    """First maximal index along the last dim (``torch.argmax`` documents first-index ties)."""
    return torch.argmax(logits, dim=-1)


class KVCacheOracle:
    """KV-cached restatement of the same forward, one chunk of positions at a time.

    Equal to ``forward`` up to float reassociation; used as the teacher-forced
    checker for long decodes and as the CPU baseline. ``kv_dtype`` stores the
    cache in a narrower format; ``step(..., act_dtype=...)`` rounds that
    chunk's GEMM inputs as ``forward`` does, so a prompt chunk can model a
    batched prefill and the following chunk a decode that keeps fp32 inputs.
    """

    def __init__(self, sd, config, batch: int, capacity: int | None = None, dtype=torch.float32,
                 kv_dtype=None):
        self.config = config
        self.dtype = dtype
        self.kv_dtype = kv_dtype
        self.sd = {n: t.to(dtype) for n, t in sd.items()}
        self.heads = config.num_heads
        self.dk = config.d_model // config.num_heads
        cap = capacity or config.context_length
        shape = (config.num_layers, batch, self.heads, cap, self.dk)
        self.k = torch.zeros(shape, dtype=dtype)
        self.v = torch.zeros(shape, dtype=dtype)
        self.cos, self.sin = rope_tables(config.rope_theta, self.dk, config.context_length)
        self.length = 0

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, act_dtype=None, norm_fold: bool = False) -> torch.Tensor:
        """Append ``tokens [B, T]`` at the current length; return logits ``[B, T, V]``.

        ``norm_fold`` stores the layers' RMSNorm inputs as ``_norm_input`` with
        ``fold`` does (the final norm stays as it is).
        """
        sd, cfg = self.sd, self.config
        t = tokens.shape[1]
        start = self.length
        positions = torch.arange(start, start + t)
        total = start + t
        mask = torch.arange(total)[None, :] <= positions[:, None]
        x = sd["token_embeddings.weight"][tokens]
        for layer in range(cfg.num_layers):
            p = f"layers.{layer}."
            h, r = _norm_input(x, sd[p + "attn_norm.weight"], act_dtype, norm_fold)
            q = rope(_split_heads(_scaled(_linear(h, sd[p + "attn.q_proj.weight"]), r), self.heads), self.cos,
                     self.sin, positions)
            k = rope(_split_heads(_scaled(_linear(h, sd[p + "attn.k_proj.weight"]), r), self.heads), self.cos,
                     self.sin, positions)
            v = _split_heads(_scaled(_linear(h, sd[p + "attn.v_proj.weight"]), r), self.heads)
            self.k[layer, :, :, start:total] = _round(k, self.kv_dtype)
            self.v[layer, :, :, start:total] = _round(v, self.kv_dtype)
            a = attention_core(_round(q, act_dtype), self.k[layer, :, :, :total], self.v[layer, :, :, :total], mask,
                               act_dtype)
            x = x + _linear(_round(_merge_heads(a), act_dtype), sd[p + "attn.output_proj.weight"])
            h, r = _norm_input(x, sd[p + "ffn_norm.weight"], act_dtype, norm_fold)
            a1 = _scaled(_linear(h, sd[p + "ffn.w1.weight"]), r)
            g = _round(a1 * torch.sigmoid(a1) * _scaled(_linear(h, sd[p + "ffn.w3.weight"]), r), act_dtype)
            x = x + _linear(g, sd[p + "ffn.w2.weight"])
        self.length = total
        return _linear(_round(rmsnorm(x, sd["ln_final.weight"]), act_dtype), sd["lm_head.weight"])


@torch.no_grad()
def greedy_cached(sd, config, prompt: torch.Tensor, steps: int, dtype=torch.float32):
    """Greedy decode through ``KVCacheOracle``; returns ``(ids, last-position logits per step)``."""
    cache = KVCacheOracle(sd, config, prompt.shape[0], prompt.shape[1] + steps, dtype)
    logits = cache.step(prompt)[:, -1, :]
    ids = [prompt]
    history = []
    for _ in range(steps):
        history.append(logits.float())
        nxt = greedy_argmax(logits.float())[:, None]
        ids.append(nxt)
        logits = cache.step(nxt)[:, -1, :]
    return torch.cat(ids, dim=1), torch.stack(history, dim=1)
