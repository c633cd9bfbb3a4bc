"""The C-ABI library: loads, exports every symbol include/claudemaxing_amd.h declares, and
rejects bad arguments on the host before touching the GPU (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import pytest

from claudemaxing_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "claudemaxing_amd.h"
INVALID = 1  # hipErrorInvalidValue


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_symbols()
    assert "cm_nf4_dequant" in names and "cm_lmhead_ce" in names and len(names) >= 14


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_signatures_match_the_header_arity():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))


def test_abi_version_and_error_strings(lib):
    assert lib.cm_abi_version() == _lib.ABI_VERSION
    assert lib.cm_error_string(0) == b"success"
    assert lib.cm_error_string(INVALID) == b"invalid argument"
    assert lib.cm_error_string(12345)  # never NULL


def test_argument_checks_run_on_the_host(lib):
    # Every call below fails its argument checks before any HIP call is made.
    assert lib.cm_lora_pack(None, 0, None, None, None, 7, 1.0, None) == INVALID  # n % 8
    assert lib.cm_lora_unpack(None, None, None, None, None, 0, -8, 1.0, None) == INVALID
    assert lib.cm_nf4_dequant(None, None, 1, None, None, None, None, None, 1, 10, 48, 256,
                              None, 0, None) == INVALID  # blocksize not a power of two
    assert lib.cm_nf4_dequant(None, None, 1, None, None, None, None, None, 1, 10, 16, 256,
                              None, 0, None) == INVALID  # blocksize below 32
    # transposed expansion: rows a multiple of 64, columns of 128, blocksize a power of two >= 32
    assert lib.cm_nf4_dequant_t(None, None, 0, None, None, None, None, None, 100, 128, 64, 1,
                                None) == INVALID
    assert lib.cm_nf4_dequant_t(None, None, 0, None, None, None, None, None, 64, 64, 64, 1,
                                None) == INVALID
    assert lib.cm_nf4_dequant_t(0x1000, 0x2000, 0, 0x3000, None, None, None, 0x4000, 64, 128, 48,
                                1, None) == INVALID
    assert lib.cm_nf4_dequant_t(0x1000, 0x2000, 0, 0x3000, None, None, None, 0x4008, 64, 128, 64,
                                1, None) == INVALID  # misaligned output
    assert lib.cm_nf4_dequant_t(None, None, 0, None, None, None, None, None, 0, 128, 64, 1,
                                None) == 0  # empty
    assert lib.cm_rope(None, 1, 0, 0, 0, 1, None, 1, None, 1, 0, 0, 0, 0, None, 1, None, None,
                       1, 0, 0, 1, 1, 7, 0, None) == INVALID  # odd head_dim
    assert lib.cm_swiglu_fwd(None, 1, None, 1, None, 1, -1, 1, None) == INVALID
    # row-strided SwiGLU: row widths and strides in whole 8-element vectors, ld >= cols
    ptrs = (0x1000, 1, 0x2000, 1)
    assert lib.cm_swiglu_fwd_rows(*ptrs, 20, 0x3000, 1, 10, 4, 10, 1, None) == INVALID
    assert lib.cm_swiglu_fwd_rows(*ptrs, 12, 0x3000, 1, 16, 4, 16, 1, None) == INVALID
    assert lib.cm_swiglu_fwd_rows(0x1008, 1, 0x2000, 1, 32, 0x3000, 1, 16, 4, 16, 1,
                                  None) == INVALID  # misaligned gate
    assert lib.cm_swiglu_bwd_rows(0x1000, 1, 8, 0x2000, 1, 0x3000, 1, 32, 0x2000, 0x3000, 4, 16,
                                  1, 1, 1, None) == INVALID  # dy rows narrower than cols
    assert lib.cm_swiglu_fwd_rows(None, 1, None, 1, 32, None, 1, 16, 0, 16, 1, None) == 0
    # several LoRA adapters per launch: 1 to 4 of them
    assert lib.cm_lora_fused_fwd_multi(None, 4, 1536, 16, 1.05, 2.0, 5, None, None, None, None,
                                       None, None, None, None, None) == INVALID
    assert lib.cm_lora_fused_bwd1_multi(4, 16, 2.0, 0, None, None, None, None, None, None,
                                        None) == INVALID
    # grouped NF4 expansion: at most 8 weights; none is a no-op
    assert lib.cm_nf4_dequant_group(None, 9, None, 1, None) == INVALID
    assert lib.cm_nf4_dequant_group(None, 0, None, 1, None) == 0
    assert lib.cm_rmsnorm_fwd(None, 1, 4, None, 0, None, 1, None, None, None, None, 1, 2, 8,
                              1e-6, None) == INVALID  # row stride < n_cols
    assert lib.cm_xent_rows(None, 1, 4, None, None, None, None, 1, 8, 0, 1.0, None) == INVALID
    # residual norm: the residual and h are required; the residual gradient needs an fp32 x
    assert lib.cm_rmsnorm_add_fwd(None, 0x1000, 0, 8, 0x2000, 0, None, 0x3000, 0x4000, None,
                                  None, None, 1, 2, 8, 1e-6, None) == INVALID
    assert lib.cm_rmsnorm_bwd_res(0x1000, 1, 0x2000, 1, 0x3000, 1, 0x4000, 0x5000, 0x6000, None,
                                  None, None, None, 1, 0, 2, 8, None) == INVALID
    # fused LoRA adapter: rank must be 16, K and N multiples of 8 and <= 2048
    assert lib.cm_lora_fused_fwd(None, None, None, None, None, None, None, None, 4, 1536, 1536,
                                 8, 1.05, 2.0, None) == INVALID
    assert lib.cm_lora_fused_fwd(None, None, None, None, None, None, None, None, 4, 1532, 1536,
                                 16, 1.05, 2.0, None) == INVALID
    assert lib.cm_lora_fused_bwd1(None, None, None, None, None, 4, 4096, 16, 2.0,
                                  None) == INVALID
    # N a multiple of 8 (each lane's vector accesses are all in range or all out)
    assert lib.cm_lora_fused_fwd(None, None, None, None, None, None, None, None, 4, 1536, 1500,
                                 16, 1.05, 2.0, None) == INVALID
    assert lib.cm_lora_fused_bwd1(None, None, None, None, None, 4, 1500, 16, 2.0,
                                  None) == INVALID
    assert lib.cm_lora_fused_bwd2(None, None, None, None, None, None, None, 4, 4096, 16, 1.05,
                                  None) == INVALID


def test_empty_inputs_are_no_ops(lib):
    assert lib.cm_nf4_dequant(None, None, 0, None, None, None, None, None, 1, 0, 64, 256,
                              None) == 0
    assert lib.cm_lora_pack(None, 0, None, None, None, 0, 1.0, None) == 0
    assert lib.cm_swiglu_fwd(None, 1, None, 1, None, 1, 0, 1, None) == 0
    assert lib.cm_rmsnorm_bwd_partials(0) == 0
    assert lib.cm_rmsnorm_add_fwd(None, None, 0, 8, None, 0, None, None, None, None, None, None,
                                  1, 0, 8, 1e-6, None) == 0
    assert lib.cm_rmsnorm_bwd_res(None, 0, None, 0, None, 0, None, None, None, None, None, None,
                                  None, 1, 0, 0, 8, None) == 0
    assert lib.cm_rmsnorm_bwd_partials(10) == 12
    assert lib.cm_lora_fused_fwd(None, None, None, None, None, None, None, None, 0, 1536, 256,
                                 16, 1.05, 2.0, None) == 0
    assert lib.cm_lora_fused_bwd2(None, None, None, None, None, None, None, 0, 1536, 16, 1.05,
                                  None) == 0


def test_call_raises_with_the_library_message():
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("cm_lora_pack", None, 0, None, None, None, 7, 1.0, None)


def test_missing_library_raises_import_error(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libnothing.so")
    with pytest.raises(ImportError, match="missing"):
        _lib.load()


def test_dtype_codes():
    import torch

    assert _lib.dtype_code(torch.float16) == 1 and _lib.dtype_code(torch.bool) == 3
    with pytest.raises(TypeError):
        _lib.dtype_code(torch.complex64)
    assert ctypes.sizeof(ctypes.c_void_p) == 8


def _nf4_weight(rows, cols, blocksize=64, nested=1, scale_map=None):
    # host-side descriptor with fake, 16-byte aligned addresses: only the argument checks read it
    return _lib.NF4Weight(0x1000, 0x2000, nested, 0x3000, 0x4000, 0x5000, 0x6000, blocksize, 256,
                          rows, cols, scale_map)


def test_nf4_linear_argument_checks(lib):
    Arr = _lib.NF4Weight * 3
    ptrs = (ctypes.c_void_p * 3)(0x10000, 0x20000, 0x30000)
    lds = (ctypes.c_int64 * 3)(1536, 1536, 1536)
    fwd, bwd = lib.cm_nf4_linear_fwd, lib.cm_nf4_linear_bwd
    ok = Arr(_nf4_weight(1536, 1536), _nf4_weight(256, 1536), _nf4_weight(256, 1536))
    # empty token batch with valid weights: nothing to do
    assert fwd(0x40000, 1536, 0, ok, 3, None, ptrs, lds, 1, None, 0, None) == 0
    assert bwd(ptrs, lds, 0, ok, 3, 0x40000, 1536, 0, None, 0, None) == 0
    # no weights, too many weights, NULL descriptors
    assert fwd(0x40000, 1536, 4, ok, 0, None, ptrs, lds, 1, None, 0, None) == INVALID
    assert fwd(0x40000, 1536, 4, ok, 4, None, ptrs, lds, 1, None, 0, None) == INVALID
    assert fwd(0x40000, 1536, 4, None, 1, None, ptrs, lds, 1, None, 0, None) == INVALID
    # columns or rows not a multiple of 64, mixed column counts
    assert fwd(0x40000, 1536, 4, Arr(_nf4_weight(1536, 1500)), 1, None, ptrs, lds, 1,
               None, 0, None) == INVALID
    assert fwd(0x40000, 1536, 4, Arr(_nf4_weight(100, 1536)), 1, None, ptrs, lds, 1,
               None, 0, None) == INVALID
    assert fwd(0x40000, 1536, 4, Arr(_nf4_weight(256, 1536), _nf4_weight(256, 1472)), 2, None,
               ptrs, lds, 1, None, 0, None) == INVALID
    # blocksize below 32 or not a power of two
    assert fwd(0x40000, 1536, 4, Arr(_nf4_weight(256, 1536, 16)), 1, None, ptrs, lds, 1,
               None, 0, None) == INVALID
    assert fwd(0x40000, 1536, 4, Arr(_nf4_weight(256, 1536, 96)), 1, None, ptrs, lds, 1,
               None, 0, None) == INVALID
    # output dtype other than fp16/fp32, input row stride not a multiple of 8 or below K
    assert fwd(0x40000, 1536, 4, ok, 1, None, ptrs, lds, 2, None, 0, None) == INVALID
    assert fwd(0x40000, 1532, 4, ok, 1, None, ptrs, lds, 1, None, 0, None) == INVALID
    assert fwd(0x40000, 1540, 4, ok, 1, None, ptrs, lds, 1, None, 0, None) == INVALID
    # misaligned input, output stride below the weight's rows
    assert fwd(0x40008, 1536, 4, ok, 1, None, ptrs, lds, 1, None, 0, None) == INVALID
    small = (ctypes.c_int64 * 3)(1024, 1536, 1536)
    assert fwd(0x40000, 1536, 4, ok, 1, None, ptrs, small, 1, None, 0, None) == INVALID
    # backward: gradient row stride below the weight's rows, dx stride below K
    assert bwd(ptrs, small, 4, ok, 1, 0x40000, 1536, 1, None, 0, None) == INVALID
    assert bwd(ptrs, lds, 4, ok, 1, 0x40000, 1024, 1, None, 0, None) == INVALID
    assert bwd(ptrs, lds, 4, ok, 1, 0x40000, 1536, 3, None, 0, None) == INVALID
    # workspace sizes: split contractions need fp32 partials, the gate+up launch does not
    ws = lib.cm_nf4_linear_workspace_bytes
    assert ws(1276, Arr(_nf4_weight(8960, 1536, scale_map=0x7000),
                        _nf4_weight(8960, 1536, scale_map=0x7000)), 2, 0) == 0
    down = Arr(_nf4_weight(1536, 8960, scale_map=0x7000))
    assert ws(1276, down, 1, 0) == 4 * 4 * 1276 * 1536  # 4 slices of [1276, 1536] fp32
    assert ws(1276, Arr(_nf4_weight(1536, 8960)), 1, 0) == 0  # no scale map: the general kernel
    assert ws(0, down, 1, 0) == 0 and ws(4, Arr(_nf4_weight(100, 64)), 1, 0) == -1
    # split-K fp32 GEMM: K multiples of 8, strides >= K and multiples of 8, aligned operands,
    # a workspace of the stated size
    gf, gws = lib.cm_gemm_f32, lib.cm_gemm_f32_workspace_bytes
    assert gws(1276, 1536, 8960, 0) == 6 * 1276 * 1536 * 4 and gws(0, 1536, 64, 0) == 0
    assert gws(4, 8, 12, 0) == -1 and gws(4, 8, 0, 0) == -1
    a, b, o, w = 0x10000, 0x20000, 0x30000, 0x40000
    big = gws(64, 64, 64, 0)
    assert gf(a, 60, b, 64, 64, None, 0, None, 0, 0, 64, 64, o, w, big, None) == INVALID
    assert gf(a + 8, 64, b, 64, 64, None, 0, None, 0, 0, 64, 64, o, w, big, None) == INVALID
    assert gf(a, 64, b, 64, 64, None, 0, None, 0, 0, 64, 64, o, w, big - 4, None) == INVALID
    assert gf(a, 64, b, 64, 64, None, 0, None, 0, 8, 64, 64, o, w, big, None) == INVALID
    assert gf(a, 64, b, 64, 64, None, 0, None, 0, 0, 0, 64, o, w, 0, None) == 0
    ga = lib.cm_gemm_f32_add  # the residual is required and 16-byte aligned
    assert ga(a, 64, b, 64, 64, None, 0, None, 0, 0, 64, 64, None, o, w, big, None) == INVALID
    assert ga(a, 64, b, 64, 64, None, 0, None, 0, 0, 64, 64, w + 8, o, w, big, None) == INVALID
    gk = lib.cm_gemm_f32_kb  # B [K, N]: its row stride is at least N, N a multiple of 8
    assert gk(a, 64, b, 56, 64, None, 0, None, 0, 0, 64, 64, o, w, big, None) == INVALID
    bigk = gws(64, 60, 64, 0)
    assert gk(a, 64, b, 64, 64, None, 0, None, 0, 0, 64, 60, o, w, bigk, None) == INVALID
    assert gk(a, 64, b, 64, 64, None, 0, None, 0, 0, 0, 64, o, w, 0, None) == 0
    # batched adapter weight gradients: 1..4 jobs, rank 16, widths multiples of 8, even strides,
    # aligned outputs; one launch without a workspace
    P, L, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    wg, wgws = lib.cm_lora_weight_grads, lib.cm_lora_weight_grads_workspace_bytes
    assert wgws(1276, 1536, 4) == 0 and wgws(1276, 1536, 5) == -1 and wgws(-1, 1536, 1) == -1
    jobs = lambda d, ldw, out=0x30000, major=0: ((P * 1)(0x10000), (L * 1)(ldw), (I * 1)(d),
                                                 (P * 1)(0x20000), (P * 1)(out), (I * 1)(major))
    assert wg(*jobs(1536, 1536), 0, 64, 16, None, 0, None) == INVALID  # no jobs
    assert wg(*jobs(1536, 1536), 1, 64, 8, None, 0, None) == INVALID  # rank 8
    assert wg(*jobs(1532, 1536), 1, 64, 16, None, 0, None) == INVALID  # width % 8
    assert wg(*jobs(1536, 1535), 1, 64, 16, None, 0, None) == INVALID  # stride < width
    assert wg(*jobs(1536, 1536, 0x30008, 1), 1, 64, 16, None, 0, None) == INVALID  # [d, 16] out
    # scale map: blocksize must divide the columns; NULL output
    assert lib.cm_nf4_scale_map(Arr(_nf4_weight(256, 1536, 4096)), 0x50000, None) == INVALID
    assert lib.cm_nf4_scale_map(Arr(_nf4_weight(256, 1536)), None, None) == INVALID
    # the C layout of cm_nf4_weight on x86-64: 4 pointers, int + padding, 3 pointers, 2 ints,
    # 2 int64, 1 pointer
    assert _lib.NF4Weight.rows.offset == 64 and _lib.NF4Weight.scale_map.offset == 80
    assert ctypes.sizeof(_lib.NF4Weight) == 88



def test_lmhead_default_chunk(lib):
    """The LM head's default vocabulary chunk keeps E (fp16, tokens padded to 256 x chunk) within
    128 MiB and needs the fewest waves of K1's 256 x 256 workgroups over the whole vocabulary
    (594 vocabulary tiles), then the fewest chunks: at 2048 tokens (8 token tiles) 4 chunks of
    32768 columns and the remainder, 19 waves; at 1792 (7 token tiles) 4 of 146 tiles (1022
    workgroups) and the remainder, 17 waves; at 1193 (5 token tiles) 204-tile chunks, 12 waves
    in 3 chunks. The workspace grows with the chunk, so the default is the chunk whose workspace
    matches chunk_cols = 0."""
    ws = lib.cm_lmhead_ce_workspace_bytes
    V, H = 151936, 1536

    def default_chunk(n):
        target = ws(n, V, H, 0)
        hits = [c for c in range(256, V + 256, 256) if ws(n, V, H, c) == target]
        assert len(hits) == 1, (n, hits)
        return hits[0]

    assert default_chunk(2048) == 32768
    assert default_chunk(4096) == 16384
    assert default_chunk(1792) == 146 * 256
    assert default_chunk(1193) == 204 * 256
    assert default_chunk(16) == V // 256 * 256 + 256  # the whole vocabulary in one chunk
    for n in (64, 1193, 1792, 2048, 4096, 16384):
        assert (n + 255) // 256 * 256 * default_chunk(n) * 2 <= 128 << 20, n


def test_peak_probes_refuse_bad_arguments(lib):
    # checked before any launch: no GPU needed
    assert lib.cm_probe_hbm(1 << 40, None, 4096, 3, 1, 1 << 40, None) != 0  # 3 words per lane
    assert lib.cm_probe_hbm(1 << 40, None, 4100, 1, 1, 1 << 40, None) != 0  # not 16-byte words
    assert lib.cm_probe_mfma_f16(1 << 40, 10, 3, 1 << 40, None) != 0  # 3 accumulator chains
    assert lib.cm_probe_mfma_f16_flops(10, 3) == 0


def test_lmhead_plans(lib):
    """The chunk and gradient K-slices each LM-head entry point runs (queries, no GPU): at config
    4 four slices fill the 256 CUs (64 output tiles x 4); at its stated 8192-column chunk the
    no-allocation entry fits three slices beside the chunk's buffers in its 64 MiB scratch; no
    plan leaves a slice of a full chunk without columns."""
    from claudemaxing_amd import lm_head_loss as LH

    V, H = 151936, 1536
    assert LH.fused_head_plan(2048, V, H) == (32768, 4)
    assert LH.fused_head_plan(2048, V, H, 8192) == (8192, 4)
    assert LH.fused_head_plan(2048, V, H, 8192, noalloc=True) == (8192, 3)
    chunk, split = LH.fused_head_plan(2048, V, H, noalloc=True)
    assert 1 <= split <= 4 and chunk % 256 == 0 and chunk >= 2048
    with pytest.raises(RuntimeError, match="scratch"):
        LH.fused_head_plan(2048, V, H, V, noalloc=True)
    for n, c in ((128, 4096), (256, 0), (300, 2048), (1100, 4096), (2048, 0), (5000, 0)):
        for noalloc in (False, True):
            chunk, split = LH.fused_head_plan(n, V, H, c, noalloc=noalloc)
            groups = chunk // 128
            width = -(-groups // split)
            assert -(-groups // width) == split, (n, c, noalloc, chunk, split)
