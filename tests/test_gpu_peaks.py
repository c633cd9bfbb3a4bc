"""The on-box peak probes bench.py reports beside the published peaks: the HBM stream copies
exactly, the read-only stream and every matrix-core variant run, and the probe's FLOP count is
the MFMAs it issues."""

import pytest
import torch

from claudemaxing_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_lane", [1, 4, 16])
@pytest.mark.parametrize("nt", [0, 1])
def test_hbm_probe_copies_exactly(per_lane, nt, dev):
    # 64 MiB and a ragged tail (not a whole workgroup span)
    n = (64 << 20) // 4 + 4 * 37
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), dtype=torch.int32, device=dev)
    dst = torch.zeros_like(src)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    s = _lib.stream(dev)
    _lib.call("cm_probe_hbm", src.data_ptr(), dst.data_ptr(), n * 4, per_lane, nt,
              sink.data_ptr(), s)
    _lib.call("cm_probe_hbm", src.data_ptr(), None, n * 4, per_lane, nt, sink.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


@pytest.mark.parametrize("chains", [2, 4, 8])
def test_mfma_probe_runs(chains, dev):
    lib = _lib.load()
    ops = torch.randn(512 * 8, device=dev).half()
    sink = torch.zeros(4, dtype=torch.float32, device=dev)
    _lib.call("cm_probe_mfma_f16", ops.data_ptr(), 10, chains, sink.data_ptr(), _lib.stream(dev))
    torch.cuda.synchronize()
    # 2048 workgroups x 4 wavefronts x iterations x 2 x chains MFMAs of 2 * 32 * 32 * 16 FLOPs
    assert lib.cm_probe_mfma_f16_flops(10, chains) == 2048 * 4 * 10 * 2 * chains * 32768
