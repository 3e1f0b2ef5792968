"""The engine's step wire format (qwen3-1.7b/engine.py:244-350), as step_inputs builds it:
the reference's own worked example (engine.py:304-305) field by field, and the invariants the
attention ops rely on, on random plans (CPU only)."""

import math

import numpy as np
import pytest


def test_worked_example_of_the_reference(step_inputs):
    """engine.py:304-305: "A and B decoding, C prefilling 5 tokens, bucket 16, 5 entries:
    chunk_lens [1, 1, 5, 9, 0]  slot_ids [A, B, C, scratch, scratch]"."""
    A, B, C, scratch = 3, 7, 1, 9
    plan = [(10, A, [11]), (20, B, [12]), (4, C, [21, 22, 23, 24, 25])]
    st = step_inputs.fill_inputs(plan, 2, 16, 5, 128, scratch)
    chunk_lens = np.diff(st.cu_seqlens).tolist()
    assert chunk_lens == [1, 1, 5, 9, 0]
    assert st.slot_ids == [A, B, C, scratch, scratch]
    assert st.cu_seqlens == [0, 1, 2, 7, 16, 16]
    assert st.cached_lens == [10, 20, 4, 0, 0]
    assert st.ids == [11, 12, 21, 22, 23, 24, 25] + [0] * 9
    # a chunk continues after what is cached; the padding sequence starts at 0
    assert st.positions == [10, 20, 4, 5, 6, 7, 8] + list(range(9))
    assert st.seq_ids == [0, 1] + [2] * 5 + [3] * 9
    # decoding entries get no tile; C and the padding sequence start fresh tiles; -1 pads to
    # ceil(16 / 128) + 5 = 6
    assert st.tile_start == [2, 7, -1, -1, -1, -1]
    # decoders read the int8 cache directly: empty prefixes; C's 4 cached tokens
    assert st.cu_cached == [0, 0, 0, 4, 4, 4]
    assert st.num_decoding == 2
    lay = step_inputs.input_layout(16, 5, 128)
    assert lay == [16, 16, 16, 6, 5, 5, 6, 6, 1]
    assert [len(f) for f in st.fields()] == lay


def test_worked_example_small_tiles(step_inputs):
    """The same step with 4-row tiles: C's 5 rows span two tiles, the padding sequence's 9 rows
    three, none crossing an entry boundary."""
    plan = [(10, 3, [11]), (20, 7, [12]), (4, 1, [21, 22, 23, 24, 25])]
    st = step_inputs.fill_inputs(plan, 2, 16, 5, 4, 9)
    assert st.tile_start == [2, 6, 7, 11, 15] + [-1] * (4 + 5 - 5)


def test_token_buckets(step_inputs):
    """engine.py:244-252: powers of two below 128, then multiples of 128, then the cap."""
    assert step_inputs.make_token_buckets(1024) == [16, 32, 64, 128, 256, 384, 512, 640, 768,
                                                     896, 1024]
    assert step_inputs.make_token_buckets(100) == [16, 32, 64, 100]
    assert step_inputs.make_token_buckets(16) == [16]
    assert step_inputs.make_token_buckets(0) == []
    b = step_inputs.make_token_buckets(1024)
    assert step_inputs.pick_bucket(b, 1) == 16
    assert step_inputs.pick_bucket(b, 129) == 256
    assert step_inputs.pick_bucket(b, 1024) == 1024
    assert step_inputs.pick_bucket(b, 2000) == 2000


@pytest.mark.parametrize("seed", range(12))
def test_invariants_random_plans(step_inputs, seed):
    rng = np.random.default_rng(seed)
    block_m = int(rng.choice([16, 32, 64, 128, 192]))
    nd = int(rng.integers(0, 20))
    npf = int(rng.integers(0, 6))
    S = nd + npf + 1 + int(rng.integers(0, 30))
    scratch = 10_000
    plan = [(int(rng.integers(0, 4000)), b, [int(rng.integers(1, 1000))]) for b in range(nd)]
    plan += [(int(rng.integers(0, 3000)) * int(rng.integers(0, 2)), nd + j,
              [int(x) for x in rng.integers(1, 1000, int(rng.integers(0, 700)))])
             for j in range(npf)]
    N = sum(len(t) for _, _, t in plan)
    n_pad = N + int(rng.integers(0, 200))
    st = step_inputs.fill_inputs(plan, nd, n_pad, S, block_m, scratch)
    cu = np.array(st.cu_seqlens)
    seq = np.array(st.seq_ids)
    ts = np.array(st.tile_start)
    assert cu[0] == 0 and cu[-1] == n_pad and np.all(np.diff(cu) >= 0)
    # seq_ids agree with cu_seqlens, and decoding entry b is row b
    for e in range(S):
        assert np.all(seq[cu[e]:cu[e + 1]] == e)
    assert np.array_equal(seq[:nd], np.arange(nd))
    # positions continue each entry's cached prefix
    pos = np.array(st.positions)
    for e in range(S):
        L = cu[e + 1] - cu[e]
        assert np.array_equal(pos[cu[e]:cu[e + 1]], st.cached_lens[e] + np.arange(L))
    # tiles: padded to a shape-only length with -1, real ones first, each inside one entry,
    # starting at its entry's start or block_m rows after the previous tile of that entry
    assert len(ts) == math.ceil(n_pad / block_m) + S
    real = ts[ts >= 0]
    assert np.all(ts[len(real):] == -1)
    covered = np.zeros(n_pad, int)
    for r0 in real:
        e = seq[r0]
        assert e >= nd, "a decoding entry got a prefill tile"
        assert (r0 - cu[e]) % block_m == 0
        covered[r0:min(r0 + block_m, cu[e + 1])] += 1
    # every row of a prefilling entry is in exactly one tile, no decode row in any
    assert np.all(covered[:nd] == 0)
    assert np.all(covered[cu[nd]:] == 1)
    # prefixes: decoders and unused entries read none; prefilling entries their cached length
    pref = np.diff(st.cu_cached)
    assert np.all(pref[:nd] == 0)
    assert np.array_equal(pref[nd:len(plan)], [c for c, _, _ in plan[nd:]])
    assert np.all(pref[len(plan):] == 0)
    # padding and unused entries sit on the scratch slot with nothing cached
    assert st.slot_ids[len(plan):] == [scratch] * (S - len(plan))
    assert st.cached_lens[len(plan):] == [0] * (S - len(plan))


def test_needs_a_padding_entry(step_inputs):
    with pytest.raises(AssertionError):
        step_inputs.fill_inputs([(0, 0, [1])], 1, 1, 1, 128, 5)
