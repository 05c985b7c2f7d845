"""Masked prefill attention over a block schedule (the ``triton_attention.attention`` API).

Drop-in for ``attention_lab/triton_attention.py:326-438``: the same
``attention(q, k, v, schedule, spec, ...)`` signature, argument checks and error
messages, and the same output (plus natural-log LSE with ``return_lse``),
computed by the gfx950 MFMA kernel of ``libsfl.so`` instead of Triton.

Differences, all documented widenings:

* the kernel tiles queries and keys 64 x 64; a CSR schedule compiled for other
  tile sizes is recompiled for 64 x 64 from the same ``spec`` (the schedule is
  trusted compiler output of that spec, ``triton_attention.py:339-343``);
* ``spec.global_prefix`` (this build's mask extension, see ``masks.py``) is
  supported by both implementations;
* head dimension 32 is accepted besides 64 and 128;
* ``num_warps`` and ``num_stages`` are validated as in the reference but do
  not change the kernel (the launch shape is fixed per head dimension);
* ``q``, ``k`` and ``v`` may be strided views whose last dimension is
  contiguous (the model passes K/V straight out of its KV cache).
"""

from __future__ import annotations

from functools import lru_cache

import torch

from . import _lib
from . import ops  # noqa: F401  (registers torch.ops.sfl)
from .masks import BlockSchedule, MaskSpec, compile_mask, interval_regions  # noqa: F401

TILE = 64
INT32_MAX = (1 << 31) - 1


def _validated_schedule(schedule):
    """Structural validation of a schedule (``triton_attention.py:60-97``).

    Returns ``(row_ptr, col_idx, full_blocks)`` as tuples. The check walks every
    entry in Python (~0.2 ms for a 4096-token schedule), so its result is cached
    on the schedule's contents together with the types of its entries (``True
    == 1`` and both hash alike, so a cache on the values alone would let a bool
    entry through); a schedule mutated in place is therefore checked again.
    """
    scalars = (schedule.length, schedule.block_q, schedule.block_k)
    row_ptr, col_idx, full = tuple(schedule.row_ptr), tuple(schedule.col_idx), tuple(schedule.full_blocks)
    key = (scalars, row_ptr, col_idx, full, tuple(map(type, scalars)), frozenset(map(type, row_ptr)),
           frozenset(map(type, col_idx)), frozenset(map(type, full)))
    try:
        hash(key)
    except TypeError:  # an unhashable entry: let the full check name it
        return _check_schedule(*key)
    return _checked_schedule(*key)


def _check_schedule(scalars, row_ptr, col_idx, full, *_types):
    length, block_q, block_k = scalars

    def integer(name, value, minimum=0):
        if isinstance(value, bool) or not isinstance(value, int):
            raise TypeError(f"{name} must be an integer (bool is not accepted)")
        if value < minimum or value > INT32_MAX:
            raise ValueError(f"{name} must be in [{minimum}, {INT32_MAX}]")

    integer("schedule.length", length, 1)
    integer("schedule.block_q", block_q, 1)
    integer("schedule.block_k", block_k, 1)
    if block_q not in (16, 32, 64, 128) or block_k not in (16, 32, 64, 128):
        raise ValueError("block_q and block_k must each be one of 16, 32, 64, 128")
    for value in row_ptr:
        integer("row_ptr entry", value)
    for value in col_idx:
        integer("col_idx entry", value)
    if any(not isinstance(flag, bool) for flag in full):
        raise TypeError("full_blocks entries must be bool values")
    query_blocks = -(-length // block_q)
    key_blocks = -(-length // block_k)
    if (len(row_ptr) != query_blocks + 1 or not row_ptr or row_ptr[0] != 0
            or row_ptr[-1] != len(col_idx) or len(full) != len(col_idx)
            or any(x > y for x, y in zip(row_ptr, row_ptr[1:]))
            or any(c >= key_blocks for c in col_idx)):
        raise ValueError("invalid CSR block schedule")
    for start, end in zip(row_ptr, row_ptr[1:]):
        columns = col_idx[start:end]
        if tuple(sorted(set(columns))) != columns:
            raise ValueError("CSR columns must be sorted and unique in each row")
    return row_ptr, col_idx, full


_checked_schedule = lru_cache(maxsize=32)(_check_schedule)


@lru_cache(maxsize=32)
def _upload_schedule(device, row_ptr, col_idx, full):
    return (torch.tensor(row_ptr, dtype=torch.int32, device=device),
            torch.tensor(col_idx if col_idx else (0,), dtype=torch.int32, device=device),
            torch.tensor(full if full else (False,), dtype=torch.uint8, device=device))


@lru_cache(maxsize=32)
def _upload_documents(device, document_ids):
    return torch.tensor(document_ids, dtype=torch.int64, device=device)


def _kernel_schedule(schedule, spec, document_ids, length):
    """The 64 x 64 CSR the kernel walks: the given one, or the same spec recompiled."""
    if schedule.block_q == TILE and schedule.block_k == TILE:
        return schedule
    docs = None if document_ids is None else [int(x) for x in document_ids]
    return compile_mask(length, spec, TILE, TILE, docs)


def attention(q, k, v, schedule, spec, document_ids=None, num_warps=4, num_stages=2,
              implementation="csr", use_full_blocks=True, launch_metadata=None, return_lse=False,
              out=None):
    """Masked self-attention for ``[B, H, N, D]`` bf16/fp16 tensors on one device.

    Returns ``out`` or ``(out, lse)`` with ``lse`` fp32 ``[B, H, N]`` (natural
    log; ``-inf`` for rows without an admissible key, whose output is zero).
    ``out`` may be passed as a preallocated (possibly strided) ``[B, H, N, D]``
    destination -- an addition to the reference signature.
    """
    if not isinstance(spec, MaskSpec):
        raise TypeError("spec must be a MaskSpec")
    if implementation not in ("csr", "interval"):
        raise ValueError("implementation must be 'csr' or 'interval'")
    if type(use_full_blocks) is not bool:
        raise TypeError("use_full_blocks must be a bool")
    if type(return_lse) is not bool:
        raise TypeError("return_lse must be a bool")
    if launch_metadata is not None and not isinstance(launch_metadata, dict):
        raise TypeError("launch_metadata must be a dict or None")
    if implementation == "interval" and spec.same_document:
        raise ValueError("interval implementation does not support document constraints")
    row_ptr, col_idx, full = _validated_schedule(schedule)

    if any(t.requires_grad for t in (q, k, v)):
        raise RuntimeError("attention is forward-only; requires_grad inputs are unsupported")
    if q.device.type != "cuda" or any(t.device != q.device for t in (k, v)):
        raise ValueError("q, k, and v must be on the same CUDA device")
    if q.ndim != 4 or any(t.shape != q.shape for t in (k, v)):
        raise ValueError("q, k, and v must have identical [B,H,N,D] shapes")
    if q.dtype not in (torch.float16, torch.bfloat16) or any(t.dtype != q.dtype for t in (k, v)):
        raise ValueError("q, k, and v must have the same FP16 or BF16 dtype")
    if any(t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]) for t in (q, k, v)):
        raise ValueError("q, k, and v must be contiguous")
    batch, heads, length, dimension = q.shape
    if min(batch, heads, length) < 1 or dimension not in (32, 64, 128):
        raise ValueError("positive B/H/N and head dimension 32, 64 or 128 are required")
    if schedule.length != length:
        raise ValueError("schedule length must match the attention sequence length")
    if (isinstance(num_warps, bool) or not isinstance(num_warps, int)
            or isinstance(num_stages, bool) or not isinstance(num_stages, int)
            or num_warps not in (1, 2, 4, 8) or num_stages not in (1, 2, 3, 4)):
        raise ValueError("num_warps must be 1/2/4/8 and num_stages must be 1/2/3/4")

    docs_gpu = None
    if spec.same_document:
        if document_ids is None:
            raise ValueError("same_document attention requires document_ids")
        if isinstance(document_ids, torch.Tensor):
            if document_ids.ndim != 1 or document_ids.numel() != length:
                raise ValueError("document_ids must be a one-dimensional sequence of length N")
            if document_ids.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8):
                raise ValueError("document_ids must contain integers")
            docs_gpu = document_ids.to(device=q.device, dtype=torch.int64).contiguous()
            doc_list = document_ids.tolist()
        else:
            doc_list = tuple(document_ids)
            if len(doc_list) != length or any(not isinstance(d, int) or isinstance(d, bool) for d in doc_list):
                raise ValueError("document_ids must contain N integers")
            docs_gpu = _upload_documents(str(q.device), doc_list)
    else:
        doc_list = None

    _lib.lib()  # fail here, before allocating, if the library is not built
    if out is None:
        out = torch.empty_like(q)
    elif (out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(-1) != 1
          or out.data_ptr() % 8 or any(s % 4 for s in out.stride()[:3])):
        raise ValueError("out must be a [B,H,N,D] tensor like q with a contiguous last dimension")
    lse = torch.empty((batch, heads, length), dtype=torch.float32, device=q.device) if return_lse else None

    if implementation == "csr":
        sched = _kernel_schedule(schedule, spec, doc_list, length)
        csr = (row_ptr, col_idx, full) if sched is schedule else \
            (tuple(sched.row_ptr), tuple(sched.col_idx), tuple(sched.full_blocks))
        rows, cols, fulls = _upload_schedule(str(q.device), *csr)
    else:
        rows = cols = fulls = None
    torch.ops.sfl.masked_attention(
        q, k, v, out, lse, float(dimension ** -0.5), bool(spec.causal),
        -1 if spec.window_left is None else spec.window_left,
        -1 if spec.window_right is None else spec.window_right, spec.global_prefix or 0, docs_gpu,
        rows, cols, fulls, use_full_blocks)
    if launch_metadata is not None:
        _record_launch_metadata(q, k, v, spec, implementation, launch_metadata)
    return (out, lse) if return_lse else out


def _record_launch_metadata(q, k, v, spec, implementation, destination):
    """Compiler resource data of the kernel this call launched (``triton_attention.py:39-57``
    records the same fields from Triton's CompiledKernel), never a profiler measurement."""
    info = _lib.masked_kernel_info(
        q.shape[-1], q.dtype, q.shape[2], k.stride(2), v.stride(2), bool(spec.causal),
        -1 if spec.window_left is None else spec.window_left,
        -1 if spec.window_right is None else spec.window_right, spec.global_prefix or 0)
    destination.update({
        "kernel_name": info.name.decode(),
        "n_regs": info.registers,
        # hipFuncGetAttributes reports the whole private segment (spills, stack and
        # private arrays), not a spill count: n_spills is exact only when it is 0.
        "n_spills": 0 if info.private_bytes == 0 else None,
        "private_segment_bytes": info.private_bytes,
        "shared_memory_bytes": info.shared_bytes,
        "threads": info.threads,
        "block_q": TILE, "block_k": TILE, "queries_per_workgroup": info.queries_per_workgroup,
        "implementation": implementation,
        "source": "hipFuncGetAttributes of the gfx950 kernel; not rocprof profiling",
        # No assembly text is kept: the compiled kernels are identified by the library.
        "asm_sha256": {},
        "library_sha256": _lib.library_sha256(),
    })


def causal_prefill(q, k, v, out):
    """Causal attention of a prompt for the model's prefill (no LSE).

    ``q``, ``k``, ``v`` and ``out`` are ``[B, H, T, D]`` views with a
    contiguous last dimension (``k``/``v`` straight out of the KV cache) in the
    model dtype: 16-bit ones run the masked MFMA kernel on the interval
    schedule, float32 ones the fp32 kernel; launches on the current stream
    without any host synchronisation.
    """
    if q.dtype == torch.float32:
        import ctypes

        strides = [(ctypes.c_long * 3)(*t.stride()[:3]) for t in (q, k, v, out)]
        _lib.call("sfl_causal_attention_f32", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), q.shape[0],
                  q.shape[1], q.shape[2], q.shape[3], *strides, float(q.shape[-1] ** -0.5),
                  _lib.stream_handle(q.device))
        return out
    torch.ops.sfl.masked_attention(q, k, v, out, None, float(q.shape[-1] ** -0.5), True, -1, -1, 0, None,
                                   None, None, None, True)
    return out
