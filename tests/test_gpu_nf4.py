"""NF4 dequant on the GPU against the oracle: bit-exact (fp16, fp32, bf16 outputs)."""

import numpy as np
import pytest
import torch

from claudemaxing_amd import _lib
from claudemaxing_amd.nf4 import QuantState, dequantize_nf4, quantize_nf4
from oracle import inputs, nf4 as O
from tests.conftest import banner
from tests.helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

NP_OUT = {torch.float16: "f16", torch.float32: "f32", torch.bfloat16: "bf16"}


def oracle_of(packed, state, dtype):
    nested = state.nested
    kw = dict(nested=nested, blocksize=state.blocksize, out_dtype=NP_OUT[dtype])
    if nested:
        kw.update(code2=state.state2.code.cpu().numpy(), absmax2=state.state2.absmax.cpu().numpy(),
                  offset=np.float32(state.offset.cpu().item()), blocksize2=state.state2.blocksize)
    ref = O.dequant(packed.cpu().numpy(), state.absmax.cpu().numpy(), **kw)
    t = torch.from_numpy(ref.view(np.int16) if dtype == torch.bfloat16 else ref)
    if dtype == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t.reshape(tuple(state.shape))


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape", [(8960, 1536), (1536, 1536), (256, 1536), (1536, 8960), (3, 64)])
def test_matches_oracle_bitwise(nested, shape, dev):
    banner(f"nf4 shape={shape} nested={nested}")
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(0)) * 0.05
    w[0, :5] = torch.tensor([0.0, -0.0, 1e-7, 3.0, -2.5])  # tests_local/test_nf4.py:21
    packed, state = quantize_nf4(w, 64, nested)
    packed_d, state_d = packed.to(dev), state.to(dev)
    for dtype in (torch.float16, torch.float32, torch.bfloat16):
        out = dequantize_nf4(packed_d, state_d, dtype)
        torch.cuda.synchronize()
        assert_bits_equal(out, oracle_of(packed, state, dtype), f"{shape} {dtype}")


def test_config1_gate_proj(dev):
    banner("nf4 config 1")
    w = inputs.nf4_weight(0)
    packed, state = quantize_nf4(w, 64, True)
    out = dequantize_nf4(packed.to(dev), state.to(dev), torch.float16)
    assert_bits_equal(out, oracle_of(packed, state, torch.float16), "config 1")
    # reconstruction error of NF4 itself stays small (sanity of the whole chain)
    err = (out.float().cpu() - w).abs().max().item()
    assert err < 0.02, err


@pytest.mark.parametrize("blocksize", [32, 64, 4096])
def test_streaming_launch_matches_oracle(blocksize, dev):
    """A weight large enough that the launch holds more workgroups than the chip keeps resident
    (one layer's NF4 weights, 46.6M elements: 5688 workgroups of 1024 packed words): that launch
    issues its packed words before the block loads, the resident-sized ones the other way round,
    and both must give the oracle's bits."""
    banner(f"nf4 streaming launch, one layer's weights, blocksize {blocksize}")
    w = torch.randn(30336, 1536, generator=torch.Generator().manual_seed(3)) * 0.02
    packed, state = quantize_nf4(w, blocksize, True)
    out = dequantize_nf4(packed.to(dev), state.to(dev), torch.float16)
    torch.cuda.synchronize()
    assert_bits_equal(out, oracle_of(packed, state, torch.float16), f"streaming bs {blocksize}")


def test_every_byte_with_every_q8_code(dev):
    banner("nf4 exhaustive bytes x q8")
    code2 = torch.from_numpy(O.dynamic_map())
    packed = torch.arange(256, dtype=torch.uint8).repeat(256)
    q8 = torch.arange(256, dtype=torch.uint8)
    absmax2 = torch.tensor([0.37, 1.5])
    state2 = QuantState(absmax=absmax2, code=code2, blocksize=128, dtype=torch.float32)
    state = QuantState(absmax=q8, shape=torch.Size([256, 512]), code=torch.tensor(O.NF4_TABLE),
                       blocksize=512, offset=torch.tensor(0.0123), state2=state2)
    out = dequantize_nf4(packed.to(dev), state.to(dev), torch.float16)
    assert_bits_equal(out, oracle_of(packed, state, torch.float16), "exhaustive")


@pytest.mark.parametrize("blocksize,blocksize2", [(32, 256), (128, 256), (4096, 256), (64, 100),
                                                  (64, 1)])
@pytest.mark.parametrize("n_bytes", [1, 3, 5, 1029, 65536 + 7])
def test_random_bytes_blocksizes_and_tails(blocksize, blocksize2, n_bytes, dev):
    banner(f"nf4 random bs={blocksize} bs2={blocksize2} n_bytes={n_bytes}")
    g = torch.Generator().manual_seed(n_bytes)
    n_blk = (2 * n_bytes + blocksize - 1) // blocksize
    packed = torch.randint(0, 256, (n_bytes,), dtype=torch.uint8, generator=g)
    q8 = torch.randint(0, 256, (n_blk,), dtype=torch.uint8, generator=g)
    absmax2 = torch.rand((n_blk + blocksize2 - 1) // blocksize2, generator=g) + 0.1
    code2 = torch.from_numpy(O.dynamic_map())
    code = torch.tensor(O.NF4_TABLE)
    offset = torch.tensor([0.03125], dtype=torch.float32)
    out = torch.empty(2 * n_bytes, dtype=torch.float16, device=dev)
    d = {k: v.to(dev) for k, v in dict(p=packed, q8=q8, a2=absmax2, c2=code2, c=code,
                                        off=offset).items()}
    _lib.call("cm_nf4_dequant", d["p"].data_ptr(), d["q8"].data_ptr(), 1, d["c"].data_ptr(),
              d["c2"].data_ptr(), d["a2"].data_ptr(), d["off"].data_ptr(), out.data_ptr(),
              _lib.F16, n_bytes, blocksize, blocksize2, _lib.stream(dev))
    ref = O.dequant(packed.numpy(), q8.numpy(), nested=True, code2=code2.numpy(),
                    absmax2=absmax2.numpy(), offset=np.float32(0.03125), blocksize=blocksize,
                    blocksize2=blocksize2)
    assert_bits_equal(out, torch.from_numpy(ref), "random")


def test_misaligned_output_takes_the_byte_path(dev):
    banner("nf4 misaligned output")
    w = torch.randn(16, 64, generator=torch.Generator().manual_seed(2)) * 0.05
    packed, state = quantize_nf4(w, 64, True)
    sd = state.to(dev)
    buf = torch.empty(16 * 64 + 1, dtype=torch.float16, device=dev)
    out = buf[1:]  # 2-byte aligned view
    code = sd.code
    _lib.call("cm_nf4_dequant", packed.to(dev).data_ptr(), sd.absmax.data_ptr(), 1,
              code.data_ptr(), sd.state2.code.data_ptr(), sd.state2.absmax.data_ptr(),
              sd.offset.reshape(1).data_ptr(), out.data_ptr(), _lib.F16, 16 * 32, 64, 256,
              _lib.stream(dev))
    assert_bits_equal(out.reshape(16, 64), oracle_of(packed, state, torch.float16), "misaligned")


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape", [(8960, 1536), (1536, 8960), (64, 128), (192, 384)])
def test_transposed_expansion_matches_oracle_bitwise(nested, shape, dev):
    """cm_nf4_dequant_t (the MLP backward's [in, out] copy of a weight) against the oracle's
    expansion transposed, bit for bit."""
    from claudemaxing_amd.nf4 import dequantize_nf4_t

    banner(f"nf4 transposed shape={shape} nested={nested}")
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(3)) * 0.05
    w[0, :5] = torch.tensor([0.0, -0.0, 1e-7, 3.0, -2.5])
    packed, state = quantize_nf4(w, 64, nested)
    out = dequantize_nf4_t(packed.to(dev), state.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (shape[1], shape[0])
    assert_bits_equal(out, oracle_of(packed, state, torch.float16).t().contiguous(),
                      f"transposed {shape}")


@pytest.mark.parametrize("blocksize,blocksize2", [(32, 256), (128, 100), (4096, 1)])
def test_transposed_expansion_random_bytes(blocksize, blocksize2, dev):
    """Every packed byte value and q8 code through the transposed kernel, with power-of-two and
    other second-level blocksizes."""
    banner(f"nf4 transposed random bs={blocksize} bs2={blocksize2}")
    rows, cols = 128, 4096
    g = torch.Generator().manual_seed(blocksize + blocksize2)
    n_bytes = rows * cols // 2
    n_blk = rows * cols // blocksize
    packed = torch.randint(0, 256, (n_bytes,), dtype=torch.uint8, generator=g)
    q8 = torch.randint(0, 256, (n_blk,), dtype=torch.uint8, generator=g)
    absmax2 = torch.rand((n_blk + blocksize2 - 1) // blocksize2, generator=g) + 0.1
    code2 = torch.from_numpy(O.dynamic_map())
    code = torch.tensor(O.NF4_TABLE)
    offset = torch.tensor([0.03125], dtype=torch.float32)
    out = torch.empty(cols, rows, dtype=torch.float16, device=dev)
    d = {k: v.to(dev) for k, v in dict(p=packed, q8=q8, a2=absmax2, c2=code2, c=code,
                                        off=offset).items()}
    _lib.call("cm_nf4_dequant_t", d["p"].data_ptr(), d["q8"].data_ptr(), 1, d["c"].data_ptr(),
              d["c2"].data_ptr(), d["a2"].data_ptr(), d["off"].data_ptr(), out.data_ptr(),
              rows, cols, blocksize, blocksize2, _lib.stream(dev))
    ref = O.dequant(packed.numpy(), q8.numpy(), nested=True, code2=code2.numpy(),
                    absmax2=absmax2.numpy(), offset=np.float32(0.03125), blocksize=blocksize,
                    blocksize2=blocksize2)
    assert_bits_equal(out, torch.from_numpy(ref).reshape(rows, cols).t().contiguous(), "random")


@pytest.mark.parametrize("nested", [True, False])
def test_state_dict_checkpoint_dequantizes_bit_exact(nested, dev, tmp_path):
    """A 4-bit layer's checkpoint in bitsandbytes Linear4bit's key layout ("<prefix>weight"
    packed [numel/2, 1] uint8 and "<prefix>weight.<serialized QuantState>"), written to a
    safetensors file, read back with NF4Linear.from_state_dict onto the GPU and dequantized
    there: bit for bit the oracle's expansion of the raw tensors stored in the file (the oracle
    reads the file's own absmax / quant_map / nested_* / JSON fields, not the loaded module)."""
    import json

    from safetensors.torch import load_file, save_file

    from claudemaxing_amd.nf4_linear import NF4Linear

    banner(f"nf4 checkpoint nested={nested}")
    w = inputs.nf4_weight(3, rows=1536, cols=1536)
    packed, state = quantize_nf4(w, 64, nested)
    sd = {"model.layers.0.self_attn.q_proj.weight": packed.reshape(-1, 1).clone()}
    for k, v in state.as_dict(packed=True).items():
        sd["model.layers.0.self_attn.q_proj.weight." + k] = v.contiguous()
    path = tmp_path / "layer.safetensors"
    save_file(sd, str(path))
    disk = load_file(str(path))
    prefix = "model.layers.0.self_attn.q_proj."
    lin = NF4Linear.from_state_dict(disk, prefix=prefix, device=dev)
    out = dequantize_nf4(lin.packed, lin.quant_state, torch.float16)
    torch.cuda.synchronize()
    key = prefix + "weight"
    fields = json.loads(bytes(disk[key + ".quant_state.bitsandbytes__nf4"].tolist()).decode())
    kw = dict(nested=nested, blocksize=fields["blocksize"], out_dtype="f16")
    if nested:
        kw.update(code2=disk[key + ".nested_quant_map"].numpy(),
                  absmax2=disk[key + ".nested_absmax"].numpy(),
                  offset=np.float32(fields["nested_offset"]),
                  blocksize2=fields["nested_blocksize"])
    ref = O.dequant(disk[key].numpy(), disk[key + ".absmax"].numpy(),
                    code=disk[key + ".quant_map"].numpy(), **kw)
    assert tuple(fields["shape"]) == (1536, 1536)
    assert_bits_equal(out, torch.from_numpy(ref).reshape(1536, 1536), f"checkpoint {nested}")
    # and the loaded layer's product uses the same weight
    x = torch.randn(7, 1536, generator=torch.Generator().manual_seed(2)).half()
    y = lin(x.to(dev)).float().cpu()
    r = x.float() @ torch.from_numpy(ref).reshape(1536, 1536).float().t()
    assert (y - r).abs().max().item() <= 2e-3 * max(1.0, r.abs().max().item())


def test_group_expansion_equals_single_expansions(dev):
    """cm_nf4_dequant_group: several weights (nested and plain, blocksizes 64 / 128 / 256,
    one empty) in one launch, into separate tensors and into the two halves of one buffer:
    bit-identical to dequantize_nf4 per weight, in every output dtype."""
    from claudemaxing_amd.nf4_linear import dequantize_group

    banner("nf4 group expansion")
    gen = torch.Generator().manual_seed(11)
    specs = [((1536, 1536), 64, True), ((896, 512), 128, True), ((640, 256), 256, True),
             ((0, 64), 64, True)]
    pairs = []
    for shape, bs, nested in specs:
        w = torch.randn(*shape, generator=gen) * 0.05
        p, st = quantize_nf4(w, bs, nested)
        pairs.append((p.to(dev), st.to(dev)))
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        outs = [torch.full(tuple(st.shape), 7.0, dtype=dtype, device=dev) for _, st in pairs]
        dequantize_group(pairs, outs)
        for (p, st), o in zip(pairs, outs):
            assert_bits_equal(o, dequantize_nf4(p, st, dtype), f"group {tuple(st.shape)} {dtype}")
    # two weights of one shape into the halves of one [2F, K] buffer (the MLP's merged weight)
    two = [quantize_nf4(torch.randn(512, 384, generator=gen) * 0.05, 64, True) for _ in range(2)]
    two = [(p.to(dev), st.to(dev)) for p, st in two]
    buf = torch.empty(1024, 384, dtype=torch.float16, device=dev)
    dequantize_group(two, [buf[:512], buf[512:]])
    assert_bits_equal(buf, torch.cat([dequantize_nf4(p, st, torch.float16) for p, st in two]),
                      "merged halves")
    # plain (not double-quantized) weights group too; a mixed group falls back to one launch per
    # weight with the same values
    plain = [quantize_nf4(torch.randn(256, 256, generator=gen) * 0.05, 64, False)
             for _ in range(2)]
    plain = [(p.to(dev), st.to(dev)) for p, st in plain]
    for group in (plain, [plain[0], pairs[0]]):
        outs = [torch.empty(tuple(st.shape), dtype=torch.float16, device=dev) for _, st in group]
        dequantize_group(group, outs)
        for (p, st), o in zip(group, outs):
            assert_bits_equal(o, dequantize_nf4(p, st, torch.float16), "plain / mixed group")
    torch.cuda.synchronize()


def test_group_expansion_misaligned_output_falls_back(dev):
    """An output that is not 16-byte aligned takes one launch per weight (the single-weight
    byte path for that one): the same values."""
    from claudemaxing_amd.nf4_linear import dequantize_group

    banner("nf4 group expansion, misaligned output")
    gen = torch.Generator().manual_seed(12)
    pairs = [quantize_nf4(torch.randn(128, 256, generator=gen) * 0.05, 64, True)
             for _ in range(2)]
    pairs = [(p.to(dev), st.to(dev)) for p, st in pairs]
    big = torch.empty(128 * 256 + 1, dtype=torch.float16, device=dev)
    outs = [big[1:].view(128, 256), torch.empty(128, 256, dtype=torch.float16, device=dev)]
    dequantize_group(pairs, outs)
    for (p, st), o in zip(pairs, outs):
        assert_bits_equal(o, dequantize_nf4(p, st, torch.float16), "misaligned group")
