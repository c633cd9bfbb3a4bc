"""NF4 dequantization oracle (numpy, bit-exact) -- test infrastructure only.

Restates solution/nf4.py:26-46 (nf4_dequant_kernel) and the host glue 64-82 (dequantize_nf4):
byte i of the packed weight holds element 2i in its high nibble and 2i+1 in its low nibble
(nf4.py:43); element j belongs to absmax block j // blocksize (nf4.py:34); with double
quantization the block scale is code2[absmax8[b]] * absmax2[b // blocksize2] + offset, an fp32
multiply then an fp32 add, never fused (nf4.py:37-38, 81); each output is fp32
code[nibble] * scale rounded to nearest even in the output dtype (nf4.py:41-45).

What pins it (tests/test_oracle_nf4.py): a pure-Python per-element restatement on tiny inputs
(independent code path, float32 arithmetic step by step); all 256 byte values x all 256 q8
codes; the NF4 table against its construction from normal quantiles (QLoRA, arXiv:2305.14314,
App. E); round-trip invariants of the quantizer (each block's max-|w| element comes back
exactly as +-absmax in the non-nested layout; zeros stay zero); nibble order and block
indexing on planted single-element weights. Exact parity with bitsandbytes' own bytes is not
pinned: bitsandbytes is absent here and its tests (test_nf4.py) cannot run.
"""

import numpy as np

F32 = np.float32

# QLoRA, arXiv:2305.14314, Appendix E: the 16 NF4 values (as fp32), code order 0..15.
NF4_TABLE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=F32)


def nf4_table_from_quantiles(offset=0.9677083):
    """The NF4 values from their definition: 8 positive quantiles of N(0,1) at
    linspace(offset, 0.5, 9)[:-1], 7 negative ones at linspace(offset, 0.5, 8)[:-1], and 0,
    normalised by the largest (QLoRA App. E; bitsandbytes create_normal_map)."""
    from scipy.stats import norm

    pos = norm.ppf(np.linspace(offset, 0.5, 9, dtype=np.float32)[:-1].astype(np.float64))
    neg = -norm.ppf(np.linspace(offset, 0.5, 8, dtype=np.float32)[:-1].astype(np.float64))
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    return v / v.max()


def to_bf16_bits(x):
    """fp32 -> bf16 bit pattern with round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def _cast(v32, out_dtype):
    if out_dtype == "f16":
        return v32.astype(np.float16)
    if out_dtype == "f32":
        return v32
    if out_dtype == "bf16":
        return to_bf16_bits(v32)
    raise ValueError(out_dtype)


def block_scales(absmax, nested, code2=None, absmax2=None, offset=None, blocksize2=256):
    """Per-block fp32 scale: absmax itself, or code2[q8] * absmax2[b // bs2] + offset."""
    if not nested:
        return np.asarray(absmax, dtype=F32)
    q8 = np.asarray(absmax, dtype=np.uint8)
    b = np.arange(q8.size)
    prod = np.asarray(code2, F32)[q8] * np.asarray(absmax2, F32)[b // blocksize2]
    return (prod.astype(F32) + F32(offset)).astype(F32)


def dequant(packed, absmax, code=NF4_TABLE, nested=False, code2=None, absmax2=None, offset=None,
            blocksize=64, blocksize2=256, out_dtype="f16"):
    """Flat dequantized weight (2 * packed.size elements) in `out_dtype` ('f16', 'f32', or
    'bf16' as uint16 bit patterns)."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    scale = block_scales(absmax, nested, code2, absmax2, offset, blocksize2)
    code = np.asarray(code, dtype=F32)
    blk = (np.arange(p.size, dtype=np.int64) * 2) // blocksize
    s = scale[blk]
    hi = (code[p >> 4] * s).astype(F32)
    lo = (code[p & 0xF] * s).astype(F32)
    v = np.empty(2 * p.size, dtype=F32)
    v[0::2] = hi
    v[1::2] = lo
    return _cast(v, out_dtype)


def dequant_bruteforce(packed, absmax, code=NF4_TABLE, nested=False, code2=None, absmax2=None,
                       offset=None, blocksize=64, blocksize2=256):
    """The same, one element at a time in plain Python with float32 scalars (tiny inputs)."""
    out = []
    for i, byte in enumerate(np.asarray(packed, dtype=np.uint8).reshape(-1).tolist()):
        for j, nib in enumerate((byte >> 4, byte & 0xF)):
            b = (2 * i + j) // blocksize
            if nested:
                s = F32(F32(code2[int(absmax[b])]) * F32(absmax2[b // blocksize2]))
                s = F32(s + F32(offset))
            else:
                s = F32(absmax[b])
            out.append(np.float16(F32(F32(code[nib]) * s)))
    return np.array(out, dtype=np.float16)


def dynamic_map():
    """bitsandbytes' signed 8-bit dynamic quantization map (create_dynamic_map(signed=True,
    max_exponent_bits=7, total_bits=8)), 256 sorted fp32 values."""
    data = []
    for i in range(7):
        items = 2 ** i + 1
        bounds = np.linspace(0.1, 1, items, dtype=F32)
        means = (bounds[:-1] + bounds[1:]) / F32(2.0)
        scale = 10.0 ** (-6 + i)
        data += (scale * means).astype(F32).tolist()
        data += (-scale * means).astype(F32).tolist()
    data += [0.0, 1.0]
    data += [0.0] * (256 - len(data))
    return np.array(sorted(data), dtype=F32)


def _nearest(x, code):
    mid = ((code[1:] + code[:-1]) / F32(2)).astype(F32)
    return np.searchsorted(mid, x, side="left")


def quantize(w, blocksize=64, compress_statistics=True, blocksize2=256):
    """numpy restatement of the NF4 quantizer layout (bitsandbytes quantize_4bit, nf4):
    returns dict(packed, absmax, nested, code2, absmax2, offset, blocksize, blocksize2)."""
    flat = np.asarray(w, dtype=F32).reshape(-1, blocksize)
    absmax = np.abs(flat).max(axis=1).astype(F32)
    safe = np.where(absmax > 0, absmax, F32(1))
    idx = _nearest((flat / safe[:, None]).astype(F32).reshape(-1), NF4_TABLE).astype(np.uint8)
    idx = idx.reshape(-1, 2)
    packed = ((idx[:, 0] << 4) | idx[:, 1]).astype(np.uint8)
    if not compress_statistics:
        return dict(packed=packed, absmax=absmax, nested=False, blocksize=blocksize)
    offset = F32(absmax.astype(np.float64).mean())
    centred = (absmax - offset).astype(F32)
    pad = (-centred.size) % blocksize2
    padded = np.concatenate([centred, np.zeros(pad, F32)]).reshape(-1, blocksize2)
    absmax2 = np.abs(padded).max(axis=1).astype(F32)
    safe2 = np.where(absmax2 > 0, absmax2, F32(1))
    code2 = dynamic_map()
    q8 = _nearest((padded / safe2[:, None]).astype(F32).reshape(-1), code2)[:centred.size]
    return dict(packed=packed, absmax=q8.astype(np.uint8), nested=True, code2=code2,
                absmax2=absmax2, offset=offset, blocksize=blocksize, blocksize2=blocksize2)
