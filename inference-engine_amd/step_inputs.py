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

import numpy as np
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

    Built per entry as arrays: S = num_entries entries of which the first len(plan) are the
    plan's, then a padding entry of n_pad - N tokens, then empty entries (both on the scratch
    slot with nothing cached). Per token: its entry and its position (the entry's cached length
    plus the token's offset inside the chunk). Tiles: every prefilling entry (index >=
    num_seqs_decoding, the padding entry included) contributes tiles at offsets 0, block_m,
    ... of its own rows, then -1 up to ceil(n_pad / block_m) + S. Prefix lengths: the cached
    lengths of the prefilling entries, 0 for decoders. `cu_cached[-1]` is the number of prefix
    tokens the step reads.
    """
    S, B = num_entries, len(plan)
    assert B < S, "needs one spare entry for padding"
    lens = np.zeros(S, np.int64)
    lens[:B] = [len(toks) for _, _, toks in plan]
    N = int(lens.sum())
    assert n_pad >= N
    lens[B] = n_pad - N
    cached = np.zeros(S, np.int64)
    cached[:B] = [c for c, _, _ in plan]
    slots = np.full(S, scratch_slot, np.int64)
    slots[:B] = [sl for _, sl, _ in plan]
    ids = np.zeros(n_pad, np.int64)
    ids[:N] = [t for _, _, toks in plan for t in toks]

    cu = np.zeros(S + 1, np.int64)
    np.cumsum(lens, out=cu[1:])
    seq_ids = np.repeat(np.arange(S), lens)
    offset = np.arange(n_pad) - cu[:-1][seq_ids]  # token's index inside its chunk
    positions = cached[seq_ids] + offset
    first_of_tile = (offset % block_m == 0) & (seq_ids >= num_seqs_decoding)
    starts = np.flatnonzero(first_of_tile)
    tile_start = np.full(-(-n_pad // block_m) + S, -1, np.int64)
    tile_start[:len(starts)] = starts
    prefix = np.where(np.arange(S) >= num_seqs_decoding, cached, 0)
    cu_cached = np.zeros(S + 1, np.int64)
    np.cumsum(prefix, out=cu_cached[1:])

    as_list = lambda a: [int(x) for x in a]
    out = StepInputs(as_list(ids), as_list(positions), as_list(seq_ids), as_list(cu),
                     as_list(cached), as_list(slots), as_list(cu_cached), as_list(tile_start),
                     num_seqs_decoding)
    assert [len(f) for f in out.fields()] == input_layout(n_pad, S, block_m)
    return out
