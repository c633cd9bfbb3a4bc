"""LoRA dropout-mask pack/unpack oracle (numpy, bit-exact) -- test infrastructure only.

Restates solution/lora.py:30-42 (lora_dropout_pack_kernel) and 45-57
(lora_dropout_unpack_kernel): bit j of byte i is element 8i + j (least significant bit first,
lora.py:38-42 `keep << lane` summed over the 8 lanes); lora_A's input is
fp16(keep ? fp32(x) * scale : 0) (lora.py:37-39, 52-55); the input gradient is
cvt(keep ? fp32(g16) * scale : 0) (lora.py:56-57).

What pins it (tests/test_oracle_lora.py): the closed forms of the reference's own known-answer
test (tests_local/test_lora.py:24-33: xd == where(mask, fp16(x * 1.25), 0), dx == where(mask,
g * 1.25, 0), unpack(pack(...)) == pack(...)); numpy.packbits with little bit order as an
independent packing; a per-element pure-Python loop on tiny inputs.
"""

import numpy as np

F32 = np.float32


def pack(x, keep, scale):
    """(xd fp16 [n], bits uint8 [n/8]) of x (any float array) and a bool/0-1 mask."""
    x = np.asarray(x).reshape(-1).astype(F32)
    k = np.asarray(keep).reshape(-1) != 0
    if x.size % 8:
        raise ValueError("n must be a multiple of 8")
    xd = np.where(k, (x * F32(scale)).astype(F32), F32(0)).astype(np.float16)
    weights = (1 << np.arange(8, dtype=np.uint32))
    bits = (k.reshape(-1, 8).astype(np.uint32) * weights).sum(axis=1).astype(np.uint8)
    return xd, bits


def unpack(x16, bits, g16, scale, dx_dtype=np.float32):
    """(xd fp16, dx in dx_dtype) rebuilt from the fp16 copy of x, the bits and the fp16 grad."""
    x = np.asarray(x16, dtype=np.float16).reshape(-1).astype(F32)
    g = np.asarray(g16, dtype=np.float16).reshape(-1).astype(F32)
    b = np.asarray(bits, dtype=np.uint8).reshape(-1)
    keep = ((b[:, None] >> np.arange(8, dtype=np.uint8)) & 1).reshape(-1) != 0
    xd = np.where(keep, (x * F32(scale)).astype(F32), F32(0)).astype(np.float16)
    dx = np.where(keep, (g * F32(scale)).astype(F32), F32(0)).astype(dx_dtype)
    return xd, dx


def pack_bruteforce(x, keep, scale):
    """The same, element by element (tiny inputs)."""
    x = np.asarray(x).reshape(-1)
    k = np.asarray(keep).reshape(-1)
    xd, bits = [], []
    for i in range(0, x.size, 8):
        byte = 0
        for j in range(8):
            kept = bool(k[i + j])
            byte |= int(kept) << j
            xd.append(np.float16(F32(F32(x[i + j]) * F32(scale))) if kept else np.float16(0))
        bits.append(byte)
    return np.array(xd, dtype=np.float16), np.array(bits, dtype=np.uint8)
