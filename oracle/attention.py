"""CPU oracles for decode attention and masked prefill attention.

* ``decode_reference`` restates ``attention_lab/cuda_decode/study.py:23-36``:
  fp32 single-query grouped attention over a ``[B, Hkv, N, D]`` cache, keys at
  positions ``>= lengths[b]`` masked, empty rows returning zeros.
* ``dense_mask`` is the token-level truth of a ``MaskSpec`` built from signed
  distances (``attention_lab/test_masks.py:13-21``, ``validate.py:15-28``), plus
  the global-prefix rule of this build's extension.
* ``masked_attention`` is softmax attention under a dense mask with the
  reference's empty-row convention (output 0, LSE ``-inf``,
  ``attention_lab/triton_attention.py:191-197``); LSE is the natural log.
* ``scheduled_attention`` interprets a block schedule as the kernels must
  (``attention_lab/validate.py:31-55``): a query tile attends only the key
  tiles its CSR row lists; a tile flagged full is taken whole, any other tile
  through the token mask. For a schedule the compiler made from the same spec
  it equals ``masked_attention`` under ``spec_mask``; for a hand-edited one it
  is the reference of what the kernels compute.
"""

from __future__ import annotations

import torch


def decode_reference(q, k, v, lengths, *, scale=None):
    """``study.reference``: q ``[B,Hq,D]``, k/v ``[B,Hkv,N,D]``, lengths int ``[B]``."""
    batch, heads, dim = q.shape
    kv_heads, capacity = k.shape[1:3]
    groups = heads // kv_heads
    queries = q.float().reshape(batch, kv_heads, groups, dim)
    scale = dim ** -0.5 if scale is None else scale
    scores = torch.einsum("bhgd,bhnd->bhgn", queries, k.float()) * scale
    allowed = torch.arange(capacity)[None, :] < lengths.to(torch.int64)[:, None]
    scores = scores.masked_fill(~allowed[:, None, None, :], -torch.inf)
    probabilities = torch.softmax(scores, dim=-1).nan_to_num(0.0)
    return torch.einsum("bhgn,bhnd->bhgd", probabilities, v.float()).reshape(batch, heads, dim)


def dense_mask(n: int, causal=False, window_left=None, window_right=None,
               documents=None, global_prefix=None) -> torch.Tensor:
    """Boolean ``[n, n]``, True where query row may attend key column."""
    distance = torch.arange(n)[:, None] - torch.arange(n)[None, :]  # q - k
    key = torch.arange(n)[None, :].expand(n, n)
    window = torch.ones((n, n), dtype=torch.bool)
    if window_left is not None:
        window &= distance <= window_left
    if window_right is not None:
        window &= -distance <= window_right
    if global_prefix:
        window |= key < global_prefix
    allowed = window
    if causal:
        allowed &= distance >= 0
    if documents is not None:
        ids = torch.as_tensor(documents)
        allowed &= ids[:, None] == ids[None, :]
    return allowed


def spec_mask(n: int, spec, documents=None) -> torch.Tensor:
    """``dense_mask`` for any object with MaskSpec's attributes."""
    return dense_mask(n, spec.causal, spec.window_left, spec.window_right,
                      documents if spec.same_document else None,
                      getattr(spec, "global_prefix", None))


def masked_attention(q, k, v, mask, *, scale=None, dtype=torch.float64):
    """Returns ``(output [..., N, D], lse [..., N])`` computed in ``dtype``."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    scores = torch.matmul(q.to(dtype), k.to(dtype).transpose(-1, -2)) * scale
    scores = scores.masked_fill(~mask, -torch.inf)
    lse = torch.logsumexp(scores, dim=-1)
    weights = torch.softmax(scores, dim=-1).nan_to_num(0.0)
    out = torch.matmul(weights, v.to(dtype))
    return out, lse


def scheduled_attention(q, k, v, schedule, spec, documents=None, *, use_full_blocks=True,
                        dtype=torch.float64):
    """Output ``[..., N, D]`` of ``schedule`` over q/k/v ``[..., N, D]`` (``validate.py:31-55``)."""
    n = schedule.length
    allowed = spec_mask(n, spec, documents)
    mask = torch.zeros((n, n), dtype=torch.bool)
    for r in range(len(schedule.row_ptr) - 1):
        q0, q1 = r * schedule.block_q, min((r + 1) * schedule.block_q, n)
        for j in range(schedule.row_ptr[r], schedule.row_ptr[r + 1]):
            k0 = schedule.col_idx[j] * schedule.block_k
            k1 = min(k0 + schedule.block_k, n)
            whole = use_full_blocks and schedule.full_blocks[j]
            mask[q0:q1, k0:k1] = True if whole else allowed[q0:q1, k0:k1]
    return masked_attention(q, k, v, mask, dtype=dtype)[0]
