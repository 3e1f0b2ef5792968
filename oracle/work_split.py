"""Split-K work partition of decode attention (test infrastructure only; see oracle/__init__.py).

Integer restatement of qwen3-1.7b/kernels.py:20-70 (`compute_piece`, `assign_work`) and of the
sizing in kernels.py:294-314 (grid `target + B`, `MAX_SPLITS = next_pow2(target)`), with one
change of the build: the piece grows (in min_piece steps) until the work list fits `target`
items whenever that is possible (compute_piece below).
"""

import numpy as np


def cdiv(a, b):
    return -(-a // b)


def next_pow2(x: int) -> int:
    return 1 if x <= 1 else 1 << (int(x) - 1).bit_length()


def reference_piece(cached_lens, num_decoding: int, target: int, min_piece: int) -> int:
    """kernels.py:20-37: piece = roundup(max(min_piece, cdiv(sum(n_end), target)), min_piece)."""
    n_end = np.asarray(cached_lens[:num_decoding], np.int64) + 1
    total = int(n_end.sum())
    piece = max(min_piece, cdiv(total, target))
    return cdiv(piece, min_piece) * min_piece


def compute_piece(cached_lens, num_decoding: int, target: int, min_piece: int) -> int:
    """The build's piece rule: the reference's piece p0 (above) when num_decoding > target;
    otherwise the smallest multiple of min_piece, at least p0, whose pieces
    sum_b cdiv(n_end_b, piece) number at most target (the reference's rounding lets them reach
    target + num_decoding, more than one resident wave of workgroups)."""
    p0 = reference_piece(cached_lens, num_decoding, target, min_piece)
    if num_decoding > target or num_decoding == 0:
        return p0
    n_end = np.asarray(cached_lens[:num_decoding], np.int64) + 1
    piece = p0
    while int(cdiv(n_end, piece).sum()) > target:
        piece += min_piece
    return piece


def decode_work_plan(cached_lens, num_decoding: int, batch: int, target: int, min_piece: int):
    """kernels.py:40-70 for every work index of the grid `target + batch`.

    Returns (piece, rows) with rows[w] = (b, split, needed) and needed = 0 for idle programs.
    """
    piece = compute_piece(cached_lens, num_decoding, target, min_piece)
    n_end = np.asarray(cached_lens[:num_decoding], np.int64) + 1
    splits = cdiv(n_end, piece)
    ends = np.cumsum(splits)
    rows = []
    for w in range(target + batch):
        b = int(np.sum(ends <= w))
        if b < num_decoding:
            first = int(ends[b] - splits[b])
            rows.append((b, w - first, int(splits[b])))
        else:
            rows.append((min(max(b, 0), max(num_decoding - 1, 0)), 0, 0))
    return piece, rows
