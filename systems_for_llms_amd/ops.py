"""The library's operators as ``torch.library`` custom ops (namespace ``sfl``).

The drop-in operator APIs (``decode.prepare/decode``, ``attention.attention``)
validate their arguments with the reference's messages and then launch
through these ops, so the launches are visible to PyTorch (dispatcher,
``torch.compile`` graphs, fake-tensor tracing) as ops that write into
caller-owned outputs, like the reference's JIT extension
(``attention_lab/cuda_decode/decode.cu:213-256``). Each op is a thin ctypes
call into ``libsfl.so`` on the caller's current stream; there is no CPU
implementation, and a missing library raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def _strides(t: torch.Tensor):
    return (ctypes.c_long * 3)(t.stride(0), t.stride(1), t.stride(2))


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


@torch.library.custom_op("sfl::decode_attention",
                         mutates_args=("partial_max", "partial_sum", "partial_output", "out"))
def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lengths: torch.Tensor,
                     partial_max: torch.Tensor, partial_sum: torch.Tensor, partial_output: torch.Tensor,
                     out: torch.Tensor, splits: int, scale: float) -> None:
    """Split-KV decode attention into ``out`` [B, Hq, D] (``sfl_decode_attention``).

    ``partial_*`` are the fp32 split scratch ([B, Hq, splits] and
    [B, Hq, splits, D]); ``out`` has q's dtype.
    """
    batch, heads, dim = q.shape
    kv_heads, capacity = k.shape[1], k.shape[2]
    code = _lib.dtype_code(q.dtype)
    _lib.call("sfl_decode_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), lengths.data_ptr(),
              partial_max.data_ptr(), partial_sum.data_ptr(), partial_output.data_ptr(), out.data_ptr(),
              batch, heads, kv_heads, capacity, dim, splits, scale, code, code, code,
              _lib.stream_handle(q.device))


@decode_attention.register_fake
def _decode_attention_fake(q, k, v, lengths, partial_max, partial_sum, partial_output, out, splits, scale):
    return None


@torch.library.custom_op("sfl::masked_attention", mutates_args=("out", "lse"))
def masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                     lse: torch.Tensor | None, scale: float, causal: bool, window_left: int,
                     window_right: int, global_prefix: int, document_ids: torch.Tensor | None,
                     row_ptr: torch.Tensor | None, col_idx: torch.Tensor | None,
                     full_blocks: torch.Tensor | None, use_full_blocks: bool) -> None:
    """Masked attention of [B, H, N, D] q/k/v into ``out`` (and natural-log ``lse``).

    Windows are ``-1`` when unbounded. With ``row_ptr`` the kernel walks that
    64 x 64 CSR schedule; without it, the interval schedule of the mask.
    """
    batch, heads, length, dim = q.shape
    mode = 1 if row_ptr is not None else 0
    _lib.call("sfl_masked_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _ptr(lse),
              batch, heads, length, dim, _strides(q), _strides(k), _strides(v), _strides(out), scale,
              int(causal), window_left, window_right, global_prefix, _ptr(document_ids), mode,
              _ptr(row_ptr), _ptr(col_idx), _ptr(full_blocks), int(use_full_blocks),
              _lib.dtype_code(q.dtype), _lib.stream_handle(q.device))


@masked_attention.register_fake
def _masked_attention_fake(q, k, v, out, lse, scale, causal, window_left, window_right, global_prefix,
                           document_ids, row_ptr, col_idx, full_blocks, use_full_blocks):
    return None
