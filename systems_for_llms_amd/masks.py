"""Structured attention masks and their block-sparse schedules (host side).

Mirrors the reference's mask language and schedule format
(``attention_lab/masks.py:22-191``): a ``MaskSpec`` is a conjunction of
``causal`` (k <= q), ``window_left`` (k >= q - left), ``window_right``
(k <= q + right) and ``same_document`` (equal labels); ``compile_mask`` turns it
into a CSR list of key tiles per query tile, each flagged full (no elementwise
mask needed) or partial, without building a dense mask.

One extension, which the reference's ``MaskSpec`` cannot express: a global key
prefix. ``global_prefix=g`` additionally admits every key ``k < g`` regardless
of the two windows; causality and document labels still apply:

    allows(q, k) = causal_ok and document_ok and (window_ok or k < g)

"Sliding window 1024 plus the first 4 global 64-key blocks" is therefore
``MaskSpec(causal=True, window_left=1023, global_prefix=256)``; window sizes
follow the reference's convention that a "window W" workload is
``window_left=W-1`` (``attention_lab/study.py:52,110-111``). With
``global_prefix=None`` (the default) every function here behaves as the
reference's does.
"""

from __future__ import annotations

from bisect import bisect_left
from collections.abc import Sequence
from dataclasses import dataclass


def _check_int(name: str, value: object, minimum: int) -> None:
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} must be an integer")
    if value < minimum:
        raise ValueError(f"{name} must be at least {minimum}")


@dataclass(frozen=True)
class MaskSpec:
    """Conjunctive constraints (``attention_lab/masks.py:22-42``) plus a global key prefix."""

    causal: bool = False
    window_left: int | None = None
    window_right: int | None = None
    same_document: bool = False
    global_prefix: int | None = None

    def __post_init__(self) -> None:
        for name in ("causal", "same_document"):
            if not isinstance(getattr(self, name), bool):
                raise TypeError(f"{name} must be a bool")
        for name in ("window_left", "window_right", "global_prefix"):
            value = getattr(self, name)
            if value is not None:
                _check_int(name, value, 0)

    @property
    def right_bound(self) -> int | None:
        """Largest admissible ``k - q`` from causality and window_right (None = unbounded)."""
        if self.causal:
            return 0 if self.window_right is None else min(0, self.window_right)
        return self.window_right

    @property
    def globals(self) -> int:
        return self.global_prefix or 0


@dataclass
class BlockSchedule:
    """CSR over query tiles (``attention_lab/masks.py:45-59``); ``full_blocks[i]`` describes ``col_idx[i]``."""

    length: int
    block_q: int
    block_k: int
    row_ptr: list[int]
    col_idx: list[int]
    full_blocks: list[bool]


def _labels(document_ids, *, length: int | None, required: bool):
    if document_ids is None:
        if required:
            raise ValueError("same_document requires document_ids")
        return None
    if not isinstance(document_ids, Sequence) or isinstance(document_ids, (str, bytes)):
        raise TypeError("document_ids must be a sequence of integer labels")
    labels = tuple(document_ids)
    if length is not None and len(labels) != length:
        raise ValueError("document_ids must have exactly length elements")
    for label in labels:
        if isinstance(label, bool) or not isinstance(label, int):
            raise TypeError("document_ids must contain integer labels")
    return labels


def _require_spec(spec) -> None:
    if not isinstance(spec, MaskSpec):
        raise TypeError("spec must be a MaskSpec")


def allows(q: int, k: int, spec: MaskSpec, document_ids: Sequence[int] | None = None) -> bool:
    """Scalar mask semantics (``attention_lab/masks.py:84-106``) with the global-prefix rule."""
    _require_spec(spec)
    _check_int("q", q, 0)
    _check_int("k", k, 0)
    labels = _labels(document_ids, length=None, required=spec.same_document)
    if labels is not None and (q >= len(labels) or k >= len(labels)):
        raise ValueError("q and k must be within document_ids")
    if spec.causal and k > q:
        return False
    if spec.same_document and labels[q] != labels[k]:
        return False
    if k < spec.globals:
        return True
    if spec.window_left is not None and q - k > spec.window_left:
        return False
    if spec.window_right is not None and k - q > spec.window_right:
        return False
    return True


def _tile_geometry(spec: MaskSpec, length: int, q_first: int, q_last: int):
    """Key ranges for one query tile ``[q_first, q_last]``.

    Returns ``(window_lo, window_hi, global_hi, full_lo, full_hi, global_full_hi)``:
    the window union over the tile is ``[window_lo, window_hi]``; the global keys
    reachable by some row are ``[0, global_hi]``; keys in ``[full_lo, full_hi]``
    pass the window test for every row; keys in ``[0, global_full_hi]`` pass the
    global test for every row. Empty ranges have hi < lo.
    """
    right = spec.right_bound
    window_lo = 0 if spec.window_left is None else max(0, q_first - spec.window_left)
    window_hi = length - 1 if right is None else min(length - 1, q_last + right)
    full_lo = 0 if spec.window_left is None else max(0, q_last - spec.window_left)
    full_hi = length - 1 if right is None else min(length - 1, q_first + right)
    g = min(spec.globals, length)
    global_hi = g - 1 if not spec.causal else min(g - 1, q_last)
    global_full_hi = g - 1 if not spec.causal else min(g - 1, q_first)
    return window_lo, window_hi, global_hi, full_lo, full_hi, global_full_hi


def _covered(lo: int, hi: int, ranges: list[tuple[int, int]]) -> bool:
    """Whether ``[lo, hi]`` lies inside the union of the given closed ranges."""
    position = lo
    for start, stop in sorted(ranges):
        if start > position:
            break
        position = max(position, stop + 1)
        if position > hi:
            return True
    return position > hi


def compile_mask(
    length: int,
    spec: MaskSpec,
    block_q: int = 64,
    block_k: int = 64,
    document_ids: Sequence[int] | None = None,
) -> BlockSchedule:
    """Exact empty/full/partial tile classification without a dense mask.

    Interval masks cost O(query_tiles + stored_blocks). Document masks test each
    geometrically admissible block with per-label sorted positions and
    ``bisect``; a block is full only if it is geometrically full and both tiles
    carry one identical label (``attention_lab/masks.py:109-191``).
    """
    _require_spec(spec)
    for name, value in (("length", length), ("block_q", block_q), ("block_k", block_k)):
        _check_int(name, value, 1)
    labels = _labels(document_ids, length=length, required=spec.same_document)
    right = spec.right_bound

    positions: dict[int, list[int]] = {}
    if spec.same_document:
        for index, label in enumerate(labels):
            positions.setdefault(label, []).append(index)

    def single_label(start: int, stop: int):
        first = labels[start]
        return first if all(labels[i] == first for i in range(start, stop)) else None

    def row_has_key(q: int, lo: int, hi: int) -> bool:
        if lo > hi:
            return False
        candidates = positions[labels[q]]
        index = bisect_left(candidates, lo)
        return index < len(candidates) and candidates[index] <= hi

    row_ptr = [0]
    col_idx: list[int] = []
    full_blocks: list[bool] = []
    for q_first in range(0, length, block_q):
        q_last = min(q_first + block_q, length) - 1
        w_lo, w_hi, g_hi, f_lo, f_hi, gf_hi = _tile_geometry(spec, length, q_first, q_last)
        columns = set(range(w_lo // block_k, w_hi // block_k + 1)) if w_lo <= w_hi else set()
        if g_hi >= 0:
            columns.update(range(0, g_hi // block_k + 1))
        q_label = single_label(q_first, q_last + 1) if spec.same_document else None
        for col in sorted(columns):
            k_first = col * block_k
            k_last = min(k_first + block_k, length) - 1
            geometric_full = _covered(k_first, k_last, [(f_lo, f_hi), (0, gf_hi)])
            if spec.same_document:
                k_label = single_label(k_first, k_last + 1)
                nonempty = False
                for q in range(q_first, q_last + 1):
                    upper = k_last if not spec.causal else min(k_last, q)
                    g_top = min(upper, spec.globals - 1)
                    if row_has_key(q, k_first, g_top):
                        nonempty = True
                        break
                    lo = k_first if spec.window_left is None else max(k_first, q - spec.window_left)
                    hi = k_last if right is None else min(k_last, q + right)
                    if row_has_key(q, lo, hi):
                        nonempty = True
                        break
                if not nonempty:
                    continue
                full = geometric_full and q_label is not None and q_label == k_label
            else:
                full = geometric_full
            col_idx.append(col)
            full_blocks.append(full)
        row_ptr.append(len(col_idx))
    return BlockSchedule(length, block_q, block_k, row_ptr, col_idx, full_blocks)


def interval_regions(length: int, spec: MaskSpec, block_q: int, block_k: int, query_block: int):
    """Key-block ranges ``(begin, full_begin, full_end, end)`` for one query tile.

    Host mirror of the bounds the interval kernel derives in registers
    (``attention_lab/triton_attention.py:11-36``): blocks ``[begin, end)`` hold at
    least one admissible key and ``[full_begin, full_end)`` need no elementwise
    mask. Masks with document labels or a global prefix are not intervals; see
    ``interval_blocks`` for the latter.
    """
    if not isinstance(spec, MaskSpec) or spec.same_document:
        raise ValueError("interval schedules require a MaskSpec without document constraints")
    if spec.globals:
        raise ValueError("interval_regions does not describe a global_prefix; use interval_blocks")
    for name, value in (("length", length), ("block_q", block_q), ("block_k", block_k)):
        if type(value) is not int or value < 1:
            raise ValueError(f"{name} must be a positive integer")
    if type(query_block) is not int or not 0 <= query_block < -(-length // block_q):
        raise ValueError("query_block is out of bounds")
    q_first = query_block * block_q
    q_last = min(q_first + block_q, length) - 1
    w_lo, w_hi, _, f_lo, f_hi, _ = _tile_geometry(spec, length, q_first, q_last)
    begin, end = w_lo // block_k, w_hi // block_k + 1
    # A block is full when it lies inside [f_lo, f_hi]; the last block may be short.
    full_begin = min(end, max(begin, -(-f_lo // block_k)))
    if f_hi >= length - 1:
        full_end = end
    else:
        full_end = (f_hi + 1) // block_k
    full_end = max(full_begin, min(end, full_end))
    return begin, full_begin, full_end, end


def interval_blocks(length: int, spec: MaskSpec, block_q: int, block_k: int, query_block: int):
    """Ordered ``(column, full)`` pairs the interval kernel visits for one query tile.

    Equals the row of ``compile_mask`` for masks without document labels: the
    global blocks ``[0, global_end)`` below the window come first, then the
    window blocks. The kernel computes the same numbers in ``tile_bounds``.
    """
    if not isinstance(spec, MaskSpec) or spec.same_document:
        raise ValueError("interval schedules require a MaskSpec without document constraints")
    q_first = query_block * block_q
    q_last = min(q_first + block_q, length) - 1
    w_lo, w_hi, g_hi, f_lo, f_hi, gf_hi = _tile_geometry(spec, length, q_first, q_last)
    begin, end = (w_lo // block_k, w_hi // block_k + 1) if w_lo <= w_hi else (0, 0)
    global_end = g_hi // block_k + 1 if g_hi >= 0 else 0
    out = []
    for col in list(range(0, min(global_end, begin))) + list(range(begin, max(end, global_end))):
        k_first = col * block_k
        k_last = min(k_first + block_k, length) - 1
        out.append((col, _covered(k_first, k_last, [(f_lo, f_hi), (0, gf_hi)])))
    return out


def schedule_density(schedule: BlockSchedule) -> float:
    """Stored blocks over all query-tile x key-tile pairs."""
    rows = len(schedule.row_ptr) - 1
    cols = -(-schedule.length // schedule.block_k)
    return len(schedule.col_idx) / float(rows * cols)
