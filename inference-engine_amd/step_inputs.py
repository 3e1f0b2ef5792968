"""Host-side packing of one engine step's attention metadata (qwen3-1.7b/engine.py:244-350).

The engine fills these int32 fields on the host and copies them to the device in one transfer;
the attention ops only ever read them on the device. This module reproduces that wire format so
the ops see exactly the tensors the reference engine hands them:

  decoding entries first (one token each, row b = entry b), then prefilling entries, then one
  padding entry on the scratch slot that tops the tokens up to the bucket size, then unused
  entries with no tokens (engine.py:305-313); every prefilling entry starts a fresh tile of
  `block_m` rows (engine.py:318-325); tile_start is padded with -1 to a shape-only length
  (engine.py:326-327); decoders have empty cached prefixes (engine.py:328-331).
"""

import itertools
import math
from dataclasses import dataclass

import torch


def make_token_buckets(M: int) -> list:
    """engine.py:244-249."""
    if M <= 0:
        return []
    return sorted({b for b in (16, 32, 64) if b < M} | set(range(128, M, 128)) | {M})


def pick_bucket(buckets: list, N: int) -> int:
    """engine.py:251-252."""
    return next((b for b in buckets if b >= N), N)


def input_layout(n_tokens: int, num_entries: int, block_m: int) -> list:
    """engine.py:254-261: field lengths of one step's packed inputs."""
    S = num_entries
    max_tiles = math.ceil(n_tokens / block_m) + S
    return [n_tokens, n_tokens, n_tokens, S + 1, S, S, S + 1, max_tiles, 1]


@dataclass
class StepInputs:
    ids: list
    positions: list
    seq_ids: list
    cu_seqlens: list
    cached_lens: list
    slot_ids: list
    cu_cached: list
    tile_start: list
    num_decoding: int

    def fields(self) -> list:
        return [self.ids, self.positions, self.seq_ids, self.cu_seqlens, self.cached_lens,
                self.slot_ids, self.cu_cached, self.tile_start, [self.num_decoding]]

    def to_device(self, device) -> dict:
        """One int32 buffer, one copy, then views (engine.py:263-295, 345-349)."""
        flat = list(itertools.chain.from_iterable(self.fields()))
        buf = torch.tensor(flat, dtype=torch.int32).to(device)
        views = buf.split([len(f) for f in self.fields()])
        names = ["ids", "positions", "seq_ids", "cu_seqlens", "cached_lens", "slot_ids",
                 "cu_cached", "tile_start", "num_decoding"]
        return dict(zip(names, views))


def fill_inputs(plan: list, num_seqs_decoding: int, n_pad: int, num_entries: int, block_m: int,
                scratch_slot: int) -> StepInputs:
    """engine.py:297-350 for a plan of (cached_len, slot, token_ids) per entry.

    Returns the packed fields; `cu_cached[-1]` is the number of prefix tokens the step reads.
    """
    S, B = num_entries, len(plan)
    assert B < S, "needs one spare entry for padding"
    N = sum(len(toks) for _, _, toks in plan)
    assert n_pad >= N
    chunk_lens = [len(toks) for _, _, toks in plan] + [n_pad - N] + [0] * (S - B - 1)
    cached_lens = [c for c, _, _ in plan] + [0] * (S - B)
    slot_ids = [s for _, s, _ in plan] + [scratch_slot] * (S - B)
    ids = [t for _, _, toks in plan for t in toks] + [0] * (n_pad - N)
    cu_seqlens = [0, *itertools.accumulate(chunk_lens)]
    positions, seq_ids, tile_start = [], [], []
    for b, (start, L) in enumerate(zip(cu_seqlens, chunk_lens)):
        positions += range(cached_lens[b], cached_lens[b] + L)
        seq_ids += [b] * L
        if b >= num_seqs_decoding:
            tile_start += range(start, start + L, block_m)
    tile_start += [-1] * (math.ceil(n_pad / block_m) + S - len(tile_start))
    prefix_lens = [0] * num_seqs_decoding + cached_lens[num_seqs_decoding:]
    cu_cached = [0, *itertools.accumulate(prefix_lens)]
    out = StepInputs(ids, positions, seq_ids, cu_seqlens, cached_lens, slot_ids, cu_cached,
                     tile_start, num_seqs_decoding)
    assert [len(f) for f in out.fields()] == input_layout(n_pad, S, block_m)
    return out
