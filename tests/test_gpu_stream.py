"""The stream handle every entry point is given: _lib.stream() must name torch's current stream
on the device, whatever form the device comes in and inside a side-stream context (where graph
warm-up and capture run)."""

import pytest
import torch

from claudemaxing_amd import _lib

pytestmark = pytest.mark.gpu


def test_stream_handle_is_torchs_current_stream(dev):
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    forms = (dev, idx, f"cuda:{idx}", None)
    expect = torch.cuda.current_stream(dev).cuda_stream
    assert all(_lib.stream(d) == expect for d in forms)
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        assert side.cuda_stream != expect
        assert all(_lib.stream(d) == side.cuda_stream for d in forms)
    assert _lib.stream(dev) == expect
