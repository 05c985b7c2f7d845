"""Single-query attention over a contiguous KV cache (the ``cuda_decode`` operator API).

Drop-in for ``attention_lab/cuda_decode/kernel.py``: the same ``prepare`` /
``decode`` / ``PreparedDecode`` surface, argument meaning and errors, backed by
the gfx950 split-KV kernels of ``libsfl.so`` instead of a JIT-built CUDA
extension. The prepared operation owns its fp32 scratch and output and holds
its inputs by reference; the output is overwritten by every call; ``lengths``
may be changed in place between calls and graph replays; concurrent calls on
one prepared operation race on its scratch (``kernel.py:1-6``).

Differences, all widenings of the reference contract:

* head dimensions 16 and 32 are accepted besides 64 and 128, and fp32 besides fp16/bf16
  (the 22.7M parity model has 16 heads of 32 and runs in fp32);
* ``splits`` defaults to 1 as in the reference (``kernel.py:85``); an integer
  in [1, 128] is honoured exactly, and ``splits=None`` picks the split count
  from the shape (``auto_splits``);
* ``variant`` accepts ``"token"`` and ``"tile"`` and both run the same kernel:
  the gfx950 kernel always updates its softmax state once per tile of keys.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from . import ops  # noqa: F401  (registers torch.ops.sfl)

SUPPORTED_DIMS = (16, 32, 64, 128)
SUPPORTED_GROUPS = (1, 2, 4, 8)
MAX_SPLITS = 128


def _validate(q, k, v, lengths, splits):
    """Mirrors ``kernel.py:27-53`` (messages kept so callers' regexes still match)."""
    if splits is not None and (type(splits) is not int or not 1 <= splits <= MAX_SPLITS):
        raise ValueError("splits must be an integer in [1, 128]")
    if q.ndim != 3 or k.ndim != 4 or v.shape != k.shape:
        raise ValueError("expected q[B,Hq,D], k/v[B,Hkv,N,D]")
    batch, query_heads, dim = q.shape
    if min(q.shape) <= 0 or k.shape[0] != batch or k.shape[3] != dim:
        raise ValueError("Q/K/V batch and head dimensions must match and be nonempty")
    kv_heads, capacity = k.shape[1:3]
    if kv_heads <= 0 or capacity <= 0 or query_heads % kv_heads:
        raise ValueError("query heads must be divisible by positive KV heads")
    if dim not in SUPPORTED_DIMS or query_heads // kv_heads not in SUPPORTED_GROUPS:
        raise ValueError("supported head dimensions are 16/32/64/128 and GQA ratios 1/2/4/8")
    if q.dtype not in _lib.DTYPE_CODES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("Q/K/V must have the same FP16, BF16 or FP32 dtype")
    if not q.is_cuda or any(x.device != q.device for x in (k, v, lengths)):
        raise ValueError("all tensors must be on the same CUDA device")
    if any(not x.is_contiguous() for x in (q, k, v, lengths)):
        raise ValueError("all tensors must be contiguous")
    if lengths.dtype != torch.int32 or lengths.shape != (batch,):
        raise ValueError("lengths must be an int32 tensor of shape [B]")
    low, high = torch.aminmax(lengths)
    if low.item() < 0 or high.item() > capacity:
        raise ValueError("each length must be in [0, cache capacity]")
    return batch, query_heads, dim


def auto_splits(batch: int, kv_heads: int, capacity: int, groups: int = 1, matrix_cores: bool = False) -> int:
    """Split count for ``batch`` x ``kv_heads`` caches of ``capacity`` keys, ``groups``
    query heads per KV head.

    One workgroup owns one (batch, kv head, split) chunk and merges its waves
    through LDS; with a single split it writes the output directly and no
    merge kernel runs. Without grouping a few hundred workgroups (up to 16
    waves each) of >= 1024 keys cover the 256 CUs. A grouped workgroup on the
    VALU kernel does ``groups`` dot products per key, so it is given fewer keys
    and more workgroups: about 512 of >= 512 / groups keys. ``matrix_cores``
    (groups >= 4, head dim 64 or 128, 16-bit q and cache) selects the MFMA
    kernel's choice: about 256 workgroups of 4 waves (one or two per CU by
    LDS) of >= 128 keys, one 32-key tile per wave. Measured on MI355X over the
    reference's GQA shapes, e.g. B=1, Hq=32, Hkv=4, D=128: N=4096 11.1 us at
    32 splits (13.8 at 64), N=65536 32.1 us at 64 (40.3 at 128); B=8, N=16384
    46.4 us at 8 (48.7 at 16).
    """
    if matrix_cores:
        target, min_keys = 256, 128
    elif groups == 1:
        target, min_keys = 256, 1024
    else:
        target, min_keys = 512, max(64, 512 // groups)
    splits = math.ceil(target / (batch * kv_heads))
    return max(1, min(MAX_SPLITS, splits, math.ceil(capacity / min_keys)))


def uses_matrix_cores(q: torch.Tensor, k: torch.Tensor) -> bool:
    """Whether ``sfl_decode_attention`` runs these shapes on its MFMA kernel."""
    groups = q.shape[1] // k.shape[1]
    return (groups >= 4 and q.shape[-1] in (64, 128) and q.dtype == k.dtype
            and k.dtype in (torch.bfloat16, torch.float16))


@dataclass
class PreparedDecode:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    lengths: torch.Tensor
    partial_max: torch.Tensor
    partial_sum: torch.Tensor
    partial_output: torch.Tensor
    output: torch.Tensor
    splits: int
    scale: float
    variant: str

    def __call__(self) -> torch.Tensor:
        torch.ops.sfl.decode_attention(self.q, self.k, self.v, self.lengths, self.partial_max,
                                       self.partial_sum, self.partial_output, self.output, self.splits,
                                       self.scale)
        return self.output

    @property
    def scratch_bytes(self) -> int:
        return sum(x.numel() * x.element_size() for x in
                   (self.partial_max, self.partial_sum, self.partial_output))


def prepare(q, k, v, lengths=None, *, splits=1, scale=None, variant="token") -> PreparedDecode:
    """Validate and allocate outside capture, then return a reusable operation (``kernel.py:85-113``)."""
    if variant not in ("token", "tile"):
        raise ValueError("variant must be 'token' or 'tile'")
    if lengths is None:
        if q.ndim != 3 or k.ndim != 4:
            raise ValueError("expected q[B,Hq,D], k/v[B,Hkv,N,D]")
        lengths = torch.full((q.shape[0],), k.shape[2], device=q.device, dtype=torch.int32)
    batch, heads, dim = _validate(q, k, v, lengths, splits)
    if scale is None:
        scale = dim ** -0.5
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("scale must be finite and positive")
    _lib.lib()  # fail here, before allocation, if the library is not built
    if splits is None:
        splits = auto_splits(batch, k.shape[1], k.shape[2], heads // k.shape[1], uses_matrix_cores(q, k))
    maximum = torch.empty((batch, heads, splits), device=q.device, dtype=torch.float32)
    normalizer = torch.empty_like(maximum)
    numerator = torch.empty((batch, heads, splits, dim), device=q.device, dtype=torch.float32)
    output = torch.empty_like(q)
    return PreparedDecode(q, k, v, lengths, maximum, normalizer, numerator, output, splits,
                          float(scale), variant)


def decode(q, k, v, lengths=None, *, splits=1, scale=None, variant="token") -> torch.Tensor:
    """Allocate scratch and compute one decode step on the current stream (``kernel.py:116-118``)."""
    return prepare(q, k, v, lengths, splits=splits, scale=scale, variant=variant)()
