"""ie_hbm_read_probe (the read-rate helper bench.py reports beside the decode kernel): each
thread XORs the words it read and stores its value only when it equals the caller's `never`.
One nonzero word planted at a position shows that the position was read."""

import ctypes

import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu


def _probe(lib, buf, never, out):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.ie_hbm_read_probe(ctypes.c_void_p(buf.data_ptr()), ctypes.c_size_t(buf.numel() * 4),
                                 ctypes.c_uint32(never), ctypes.c_void_p(out.data_ptr()), stream)


@pytest.mark.parametrize("words", [4, 4 * 1000 + 4, 1 << 22])
def test_read_probe_reads_every_position(native, dev, words):
    say(f"hbm_read_probe words={words}")
    lib = native.cabi()
    V = 0x5A5A1234
    buf = torch.zeros(words, dtype=torch.int32, device=dev)
    out = torch.full((1,), 7, dtype=torch.int32, device=dev)
    for pos in sorted({0, words // 2 + 1, words - 1}):
        buf.zero_()
        buf[pos] = V
        out.fill_(7)
        assert _probe(lib, buf, V + 1, out) == 0
        torch.cuda.synchronize()
        assert out.item() == 7, pos  # no thread's XOR equals `never`: nothing written
        assert _probe(lib, buf, V, out) == 0
        torch.cuda.synchronize()
        assert out.item() == V, pos  # the thread that read `pos` saw the planted word


def test_read_probe_rejects_unaligned(native, dev):
    lib = native.cabi()
    buf = torch.zeros(8, dtype=torch.int32, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ie_hbm_read_probe(ctypes.c_void_p(buf.data_ptr()), ctypes.c_size_t(12),
                               ctypes.c_uint32(0), ctypes.c_void_p(out.data_ptr()), stream)
    assert rc != 0
