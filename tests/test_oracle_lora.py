"""Pins the LoRA pack/unpack oracle (oracle/lora.py)."""

import numpy as np

from oracle import lora as O

F32 = np.float32


def make(n=3 * 37 * 64, seed=0, p_keep=0.7):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(F32)
    keep = rng.random(n) < p_keep
    g = rng.standard_normal(n).astype(np.float16)
    return x, keep, g


def test_known_answer_closed_forms():
    """tests_local/test_lora.py:24-33 on fp16 x, scale 1.25."""
    x, keep, g = make()
    x16 = x.astype(np.float16)
    xd, bits = O.pack(x16, keep, 1.25)
    assert np.array_equal(xd, np.where(keep, (x16.astype(F32) * F32(1.25)).astype(np.float16),
                                       np.float16(0)))
    xd2, dx = O.unpack(x16, bits, g, 1.25)
    assert np.array_equal(xd2.view(np.int16), xd.view(np.int16))
    assert np.array_equal(dx, np.where(keep, g.astype(F32) * F32(1.25), F32(0)))


def test_bits_match_numpy_packbits_little():
    x, keep, _ = make(seed=2)
    _, bits = O.pack(x, keep, 1.0 / 0.95)
    assert np.array_equal(bits, np.packbits(keep, bitorder="little"))


def test_elementwise_restatement():
    x, keep, _ = make(n=256, seed=4)
    a = O.pack(x, keep, 1.0 / 0.95)
    b = O.pack_bruteforce(x, keep, 1.0 / 0.95)
    assert np.array_equal(a[0].view(np.int16), b[0].view(np.int16))
    assert np.array_equal(a[1], b[1])


def test_lsb_is_the_first_element():
    keep = np.zeros(16, bool)
    keep[0] = keep[9] = True
    _, bits = O.pack(np.ones(16, F32), keep, 1.0)
    assert bits.tolist() == [1, 2]
