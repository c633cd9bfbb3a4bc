"""Benchmark of the QLoRA step kernel set on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME[,NAME...]]

Every kernel runs on inputs already resident in HBM, at the shapes of BASELINE.json's configs:
  1  NF4 dequant of the [8960,1536] gate_proj weight (blocksize 64, double-quantized) to fp16
  2  RMSNorm fwd/bwd and RoPE fwd/bwd on 4 packed rows of U[128,512] tokens (hidden 1536)
  3  SwiGLU forward and in-place recompute-backward on [2048,8960] fp16
  4  fused LM head + cross-entropy, hidden [2048,1536], tied weight [151936,1536] fp16
plus the LoRA mask pack/unpack at the q/v input shape of config 5, every streaming kernel at a
bandwidth-scale shape (32768 tokens; NF4 over one decoder layer's weights), the launch floor of
the box (an empty kernel, a one-wavefront kernel, a 1 MiB copy), torch's device copy as the
practical HBM ceiling, and config 5's QLoRA training step (eager over distinct batches, and
replayed from a HIP graph).

Cold-cache protocol: each timed launch works on its own copy of the inputs, rotating through
enough copies to exceed 512 MiB (twice the 256 MiB Infinity Cache), so no launch finds its
inputs in the cache. A kernel's time is the HIP-event time of K back-to-back launches on the
launch stream divided by K. Achieved bandwidth / FLOP rate uses the ALGORITHMIC bytes / FLOPs of
one launch (inputs read once, outputs written once).

Every launch closure is built eagerly from its own tensors (sizes read from those tensors), so
no closure can pick up another kernel's sizes.

One JSON line is printed: the headline metric with its roofline and the CPU oracle timed on the
host cores (a baseline, not the target), plus every kernel's numbers under "kernels", and the
board's socket power and graphics clock (amd-smi) sampled while the headline call runs back to
back after its timed region (the matrix-core kernels run at the board's power limit), and the
two roofline denominators as the board attains them ("measured_peaks": a 2 GiB HBM stream and
the fp16 MFMA issue rate on register operands), each kernel's fraction of them beside its
fraction of the published peaks.
"""

import argparse
import gc
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
COLD_BYTES = 512 * 2 ** 20
METRIC = "kernel HBM GB/s & LM-head-CE TFLOP/s (% of roofline); QLoRA step ms"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", default="")
    p.add_argument("--step-steps", type=int, default=10, help="timed QLoRA steps (config 5)")
    p.add_argument("--no-step", action="store_true", help="skip the QLoRA step (config 5)")
    p.add_argument("--step-graphed-only", action="store_true",
                   help="time only the repeated batch replayed from its graph (for a kernel "
                        "trace of that step alone)")
    p.add_argument("--step-json-only", action="store_true",
                   help="run the QLoRA step bench alone in this process and print its record as "
                        "one JSON line (what the default run starts as a child process)")
    p.add_argument("--no-peaks", action="store_true",
                   help="skip the on-box HBM and matrix-core peak probes")
    p.add_argument("--no-power", action="store_true",
                   help="skip the board power sample of the headline (profiler runs)")
    return p.parse_args()


def copies_for(nbytes, cap=64):
    """Input copies needed so that a rotation touches more than COLD_BYTES."""
    return max(2, min(cap, -(-COLD_BYTES // max(nbytes, 1)) + 1))


class Kernel:
    """A benchmarked entry point: `launches` are (closure, tensors it uses) pairs, one per input
    copy, used round-robin; `work` is the algorithmic bytes (hbm) or FLOPs (mfma) of one."""

    def __init__(self, name, config, bound, work, launches, step=True, plan=None):
        self.name, self.config, self.bound, self.work = name, config, bound, work
        self.launches, self.step, self.plan = launches, step, plan


def bound(name, *args):
    """A launch closure of C-ABI entry point `name` with all arguments fixed now."""
    from claudemaxing_amd import _lib

    fn = getattr(_lib.load(), name)
    fixed = tuple(args)

    def launch():
        rc = fn(*fixed)
        if rc:
            raise RuntimeError(f"{name} failed with code {rc}")

    return launch


def _stream(dev):
    from claudemaxing_amd import _lib

    return _lib.stream(dev)


def k_nf4(dev):
    import torch

    from claudemaxing_amd import _lib, nf4
    from oracle import inputs

    w = inputs.nf4_weight(0)
    packed, state = nf4.quantize_nf4(w, 64, True)
    n_el = w.numel()
    n_bytes = n_el // 2
    work = n_bytes + state.absmax.numel() + state.state2.absmax.numel() * 4 + 256 * 4 + \
        16 * 4 + 4 + n_el * 2
    launches = []
    for _ in range(copies_for(work)):
        p, st = packed.to(dev), state.to(dev)
        out = torch.empty(w.shape, dtype=torch.float16, device=dev)
        assert p.numel() == n_bytes and out.numel() == 2 * n_bytes
        launches.append((bound("cm_nf4_dequant", p.data_ptr(), st.absmax.data_ptr(), 1,
                               st.code.data_ptr(), st.state2.code.data_ptr(),
                               st.state2.absmax.data_ptr(), st.offset.data_ptr(), out.data_ptr(),
                               _lib.F16, n_bytes, 64, 256, _stream(dev)), (p, st, out)))
    return [Kernel("nf4_dequant", "[8960,1536] nf4->fp16", "hbm", work, launches)]


def k_rmsnorm(dev, c2, names):
    import torch

    from claudemaxing_amd import _lib

    n_rows, hid = c2["n"], 1536
    x = c2["x"]
    w16 = c2["w"].to(torch.float16)
    fwd_work = 2 * n_rows * hid + 2 * n_rows * hid + 4 * n_rows + 2 * hid
    bwd_work = 2 * n_rows * hid * 3 + 4 * n_rows + 2 * hid
    fwd, bwd = [], []
    for _ in range(copies_for(fwd_work + bwd_work)):
        xd, wd = x.to(dev), w16.to(dev)
        out = torch.empty(n_rows, hid, dtype=torch.float16, device=dev)
        rstd = torch.empty(n_rows, dtype=torch.float32, device=dev)
        dy = c2["dy"].to(torch.float16).to(dev)
        dx = torch.empty(n_rows, hid, dtype=torch.float16, device=dev)
        assert xd.shape == out.shape == dy.shape == dx.shape == (n_rows, hid)
        keep = (xd, wd, out, rstd, dy, dx)
        f = bound("cm_rmsnorm_fwd", xd.data_ptr(), _lib.F16, hid, wd.data_ptr(), _lib.F16,
                  out.data_ptr(), _lib.F16, rstd.data_ptr(), None, None, None, 1, n_rows, hid,
                  1e-6, _stream(dev))
        b = bound("cm_rmsnorm_bwd", dy.data_ptr(), _lib.F16, xd.data_ptr(), _lib.F16,
                  wd.data_ptr(), _lib.F16, rstd.data_ptr(), dx.data_ptr(), _lib.F16, None, None,
                  None, 1, 0, n_rows, hid, _stream(dev))
        f()  # rstd of every copy holds real values before backward is timed
        fwd.append((f, keep))
        bwd.append((b, keep))
    out = []
    if "rmsnorm_fwd" in names:
        out.append(Kernel("rmsnorm_fwd", f"N={n_rows} H=1536 fp16", "hbm", fwd_work, fwd))
    if "rmsnorm_bwd" in names:
        out.append(Kernel("rmsnorm_bwd", f"N={n_rows} H=1536 fp16", "hbm", bwd_work, bwd))
    if names & {"rmsnorm_fwd_w32", "rmsnorm_bwd_w32"}:
        out += k_rmsnorm_w32(dev, c2, names)
    if names & {"rmsnorm_fwd_qlora", "rmsnorm_bwd_qlora"}:
        out += k_rmsnorm_qlora(dev, c2, names)
    return out


def k_rmsnorm_w32(dev, c2, names):
    """Config 2's fp32-weight variant: fp16 x, the fp32 weight with its 77 tiny channels (more than
    the save-low path's 64, so the exact path), fp32 out; backward fp32 dy -> fp16 dx."""
    import torch

    from claudemaxing_amd import _lib

    n_rows, hid = c2["n"], 1536
    fwd_work = 2 * n_rows * hid + 4 * n_rows * hid + 4 * n_rows + 4 * hid
    bwd_work = (4 + 2 + 2) * n_rows * hid + 4 * n_rows + 4 * hid
    fwd, bwd = [], []
    for _ in range(copies_for(fwd_work + bwd_work)):
        xd, wd = c2["x"].to(dev), c2["w"].to(torch.float32).to(dev)
        out = torch.empty(n_rows, hid, dtype=torch.float32, device=dev)
        rstd = torch.empty(n_rows, dtype=torch.float32, device=dev)
        dy = c2["dy"].to(torch.float32).to(dev)
        dx = torch.empty(n_rows, hid, dtype=torch.float16, device=dev)
        assert xd.dtype == torch.float16 and xd.shape == out.shape == dy.shape == dx.shape
        keep = (xd, wd, out, rstd, dy, dx)
        f = bound("cm_rmsnorm_fwd", xd.data_ptr(), _lib.F16, hid, wd.data_ptr(), _lib.F32,
                  out.data_ptr(), _lib.F32, rstd.data_ptr(), None, None, None, 1, n_rows, hid,
                  1e-6, _stream(dev))
        b = bound("cm_rmsnorm_bwd", dy.data_ptr(), _lib.F32, xd.data_ptr(), _lib.F16,
                  wd.data_ptr(), _lib.F32, rstd.data_ptr(), dx.data_ptr(), _lib.F16, None, None,
                  None, 1, 0, n_rows, hid, _stream(dev))
        f()
        fwd.append((f, keep))
        bwd.append((b, keep))
    out = []
    if "rmsnorm_fwd_w32" in names:
        out.append(Kernel("rmsnorm_fwd_w32", f"N={n_rows} H=1536 fp16 x, fp32 w -> fp32", "hbm",
                          fwd_work, fwd, step=False))
    if "rmsnorm_bwd_w32" in names:
        out.append(Kernel("rmsnorm_bwd_w32", f"N={n_rows} H=1536 fp32 dy -> fp16 dx", "hbm",
                          bwd_work, bwd, step=False))
    return out


def k_rmsnorm_qlora(dev, c2, names):
    """The training step's norms: fp32 residual x, frozen fp32 weight with no tiny channel
    (n_small = 0), fp32 out plus the fp16 copy of the output that the NF4 linears read (the
    save-low path); backward from that copy: fp32 dy -> fp32 dx."""
    import torch

    from claudemaxing_amd import _lib

    n_rows, hid = c2["n"], 1536
    fwd_work = (4 + 4 + 2) * n_rows * hid + 4 * n_rows + 4 * hid
    bwd_work = (4 + 2 + 4) * n_rows * hid + 4 * n_rows + 4 * hid
    w1 = torch.rand(hid, generator=torch.Generator().manual_seed(2)) + 0.5  # no |w| < 2^-10
    fwd, bwd = [], []
    for _ in range(copies_for(fwd_work + bwd_work)):
        xd, wd = c2["x"].to(torch.float32).to(dev), w1.to(dev)
        out = torch.empty(n_rows, hid, dtype=torch.float32, device=dev)
        low = torch.empty(n_rows, hid, dtype=torch.float16, device=dev)
        side = torch.empty(n_rows, 1, dtype=torch.float16, device=dev)
        slot = torch.full((hid,), -1, dtype=torch.int32, device=dev)  # no tiny column
        rstd = torch.empty(n_rows, dtype=torch.float32, device=dev)
        dy = c2["dy"].to(torch.float32).to(dev)
        dx = torch.empty(n_rows, hid, dtype=torch.float32, device=dev)
        assert xd.shape == out.shape == low.shape == dy.shape == dx.shape == (n_rows, hid)
        keep = (xd, wd, out, low, side, slot, rstd, dy, dx)
        f = bound("cm_rmsnorm_fwd", xd.data_ptr(), _lib.F32, hid, wd.data_ptr(), _lib.F32,
                  out.data_ptr(), _lib.F32, rstd.data_ptr(), low.data_ptr(), slot.data_ptr(),
                  side.data_ptr(), 0, n_rows, hid, 1e-6, _stream(dev))
        b = bound("cm_rmsnorm_bwd", dy.data_ptr(), _lib.F32, low.data_ptr(), _lib.F16,
                  wd.data_ptr(), _lib.F32, rstd.data_ptr(), dx.data_ptr(), _lib.F32, None,
                  slot.data_ptr(), side.data_ptr(), 0, 1, n_rows, hid, _stream(dev))
        f()  # the fp16 copy and rstd hold real values before backward is timed
        fwd.append((f, keep))
        bwd.append((b, keep))
    out = []
    if "rmsnorm_fwd_qlora" in names:
        out.append(Kernel("rmsnorm_fwd_qlora", f"N={n_rows} H=1536 fp32 x and w -> fp32 + fp16 "
                          "copy (the training step's save-low path)", "hbm", fwd_work, fwd))
    if "rmsnorm_bwd_qlora" in names:
        out.append(Kernel("rmsnorm_bwd_qlora", f"N={n_rows} H=1536 from the fp16 copy, fp32 dy "
                          "-> fp32 dx", "hbm", bwd_work, bwd))
    return out


def _rope_launch(dev, q, k, cos, sin, backward):
    """Launch closure of cm_rope on q [1,Hq,T,D] / k [1,Hk,T,D] strided views (cos/sin of one
    row of positions, broadcast over the batch)."""
    import torch

    from claudemaxing_amd import _lib

    b, hq, t, d = q.shape
    hk = k.shape[1]
    assert k.shape[0] == b and k.shape[2] == t and k.shape[3] == d
    assert cos.shape == sin.shape == (1, t, d) and cos.is_contiguous() and sin.is_contiguous()
    oq = torch.empty((b, hq, t, d), dtype=torch.float16, device=dev)
    ok = torch.empty((b, hk, t, d), dtype=torch.float16, device=dev)
    f = bound("cm_rope", q.data_ptr(), _lib.F16, q.stride(0), q.stride(1), q.stride(2), hq,
              oq.data_ptr(), _lib.F16, k.data_ptr(), _lib.F16, k.stride(0), k.stride(1),
              k.stride(2), hk, ok.data_ptr(), _lib.F16, cos.data_ptr(), sin.data_ptr(), _lib.F16,
              0, cos.stride(1), b, t, d, int(backward), _stream(dev))
    return f, (q, k, cos, sin, oq, ok)


def k_rope(dev, c2, names):
    import torch

    from oracle import rope as orope

    n_rows = c2["n"]
    cos, sin = orope.cos_sin(c2["pos"], 128, c2["theta"], torch.float16)
    work = 2 * 2 * n_rows * 14 * 128 + 2 * 2 * n_rows * 128  # q,k in+out fp16; cos+sin
    fwd, bwd = [], []
    for _ in range(copies_for(work)):
        q = c2["q"].transpose(1, 2).contiguous().to(dev).transpose(1, 2)
        k = c2["k"].transpose(1, 2).contiguous().to(dev).transpose(1, 2)
        cd, sd = cos.to(dev), sin.to(dev)
        fwd.append(_rope_launch(dev, q, k, cd, sd, False))
        bwd.append(_rope_launch(dev, q, k, cd, sd, True))
    out = []
    if "rope_fwd" in names:
        out.append(Kernel("rope_fwd", f"N={n_rows} 12+2 heads x 128", "hbm", work, fwd))
    if "rope_bwd" in names:
        out.append(Kernel("rope_bwd", f"N={n_rows} 12+2 heads x 128", "hbm", work, bwd))
    return out


def k_swiglu(dev, names):
    import torch

    from claudemaxing_amd import _lib
    from oracle import inputs

    gate, up, dy = inputs.swiglu(0)
    n_el = gate.numel()
    fwd, bwd = [], []
    for _ in range(copies_for(10 * n_el)):
        g, u, d = gate.to(dev), up.to(dev), dy.to(dev)
        o = torch.empty_like(g)
        assert g.numel() == u.numel() == d.numel() == o.numel() == n_el
        fwd.append((bound("cm_swiglu_fwd", g.data_ptr(), _lib.F16, u.data_ptr(), _lib.F16,
                          o.data_ptr(), _lib.F16, n_el, 1, _stream(dev)), (g, u, d, o)))
        bwd.append((bound("cm_swiglu_bwd", d.data_ptr(), _lib.F16, g.data_ptr(), _lib.F16,
                          u.data_ptr(), _lib.F16, g.data_ptr(), u.data_ptr(), n_el, 1, 1, 1,
                          _stream(dev)), (g, u, d, o)))
    out = []
    if "swiglu_fwd" in names:
        out.append(Kernel("swiglu_fwd", "[2048,8960] fp16", "hbm", 6 * n_el, fwd))
    if "swiglu_bwd" in names:
        out.append(Kernel("swiglu_bwd", "[2048,8960] fp16 in place", "hbm", 10 * n_el, bwd))
    return out


def k_lora(dev, names):
    import torch

    from claudemaxing_amd import _lib

    n_el = 1152 * 1536
    g = torch.Generator().manual_seed(0)
    x = torch.randn(n_el, generator=g)
    keep = torch.rand(n_el, generator=g) > 0.05
    scale = 1 / 0.95
    pack, unpack = [], []
    for _ in range(copies_for(18 * n_el)):
        xx, kk = x.to(dev), keep.to(dev)
        xd = torch.empty(n_el, dtype=torch.float16, device=dev)
        bits = torch.empty(n_el // 8, dtype=torch.uint8, device=dev)
        g16 = torch.randn(n_el, device=dev).half()
        dx = torch.empty(n_el, device=dev)
        xd2 = torch.empty(n_el, dtype=torch.float16, device=dev)
        tensors = (xx, kk, xd, bits, g16, dx, xd2)
        assert all(t.numel() == n_el for t in (xx, kk, xd, g16, dx, xd2))
        assert bits.numel() * 8 == n_el
        p = bound("cm_lora_pack", xx.data_ptr(), _lib.F32, kk.data_ptr(), xd.data_ptr(),
                  bits.data_ptr(), n_el, scale, _stream(dev))
        p()  # bits of every copy are real before unpack is timed
        pack.append((p, tensors))
        unpack.append((bound("cm_lora_unpack", xd.data_ptr(), bits.data_ptr(), g16.data_ptr(),
                             xd2.data_ptr(), dx.data_ptr(), _lib.F32, n_el, scale, _stream(dev)),
                       tensors))
    out = []
    if "lora_pack" in names:
        out.append(Kernel("lora_pack", "[1152,1536] fp32 x", "hbm", 7 * n_el + n_el // 8, pack))
    if "lora_unpack" in names:
        out.append(Kernel("lora_unpack", "[1152,1536] -> fp32 dx", "hbm", 10 * n_el + n_el // 8,
                          unpack))
    return out


def k_copy_ref(dev):
    import torch

    n_el = 2048 * 8960
    launches = []
    for _ in range(copies_for(4 * n_el)):
        a = torch.randn(n_el, device=dev).half()
        b = torch.empty(n_el, dtype=torch.float16, device=dev)
        launches.append(((lambda a=a, b=b: b.copy_(a)), (a, b)))
    return [Kernel("hbm_copy_ref", "fp16 [2048,8960] device copy (torch)", "hbm", 4 * n_el,
                   launches, step=False)]


def k_floor(dev, names):
    """What a launch costs on this box whatever it does: the library's empty kernel
    (cm_probe_launch, through the same ctypes path as every kernel here) with one wavefront and
    with the grid of the config-2 RoPE launch (1193 workgroups of 256 lanes), a one-wavefront
    torch kernel (a 64-element fill) and a 1 MiB torch device copy. The HIP-event figures here
    are the rate at which the host issues them back to back; the rocprofv3 kernel trace of the
    same command gives the device time of each (the floor under the small config-2 / config-5
    launches)."""
    import torch

    out = []
    st = _stream(dev)
    if "floor_empty" in names:
        out.append(Kernel("floor_empty", "cm_probe_launch: one empty wavefront", "hbm", 0,
                          [(bound("cm_probe_launch", 1, 64, st), ())], step=False))
    if "floor_empty_grid" in names:
        out.append(Kernel("floor_empty_grid", "cm_probe_launch: 1193 empty workgroups of 256 "
                          "lanes (the config-2 RoPE grid)", "hbm", 0,
                          [(bound("cm_probe_launch", 1193, 256, st), ())], step=False))
    if "floor_one_wave" in names:
        launches = []
        for _ in range(64):
            x = torch.empty(64, device=dev)
            launches.append(((lambda x=x: x.fill_(1.0)), (x,)))
        out.append(Kernel("floor_one_wave", "64-element fp32 fill (one wavefront)", "hbm", 256,
                          launches, step=False))
    if "floor_copy_1mib" in names:
        n_el = 2 ** 18
        launches = []
        for _ in range(copies_for(8 * n_el, cap=600)):
            a = torch.randn(n_el, device=dev)
            b = torch.empty_like(a)
            launches.append(((lambda a=a, b=b: b.copy_(a)), (a, b)))
        out.append(Kernel("floor_copy_1mib", "1 MiB fp32 device copy (torch)", "hbm", 8 * n_el,
                          launches, step=False))
    return out


def k_bandwidth_scale(dev, names):
    """Every streaming kernel at a size where launch latency no longer dominates: the row
    kernels at 32768 tokens, NF4 over all of one decoder layer's NF4 elements."""
    import torch

    from claudemaxing_amd import _lib, nf4
    from oracle import rope as orope

    nb, hid = 32768, 1536
    out = []
    if "nf4_dequant_bw" in names:
        # q, k, v, o, gate, up, down of one Qwen2.5-1.5B layer: 46.6M elements, one tensor
        rows = 1536 + 256 + 256 + 1536 + 8960 + 8960 + 8960
        w = torch.randn(rows, hid, generator=torch.Generator().manual_seed(1)) * 0.02
        packed, state = nf4.quantize_nf4(w, 64, True)
        n_el, n_bytes = w.numel(), w.numel() // 2
        work = n_bytes + state.absmax.numel() + state.state2.absmax.numel() * 4 + 256 * 4 + \
            16 * 4 + 4 + n_el * 2
        launches = []
        for _ in range(copies_for(work)):
            p, st = packed.to(dev), state.to(dev)
            o = torch.empty(w.shape, dtype=torch.float16, device=dev)
            assert p.numel() == n_bytes and o.numel() == n_el
            launches.append((bound("cm_nf4_dequant", p.data_ptr(), st.absmax.data_ptr(), 1,
                                   st.code.data_ptr(), st.state2.code.data_ptr(),
                                   st.state2.absmax.data_ptr(), st.offset.data_ptr(),
                                   o.data_ptr(), _lib.F16, n_bytes, 64, 256, _stream(dev)),
                             (p, st, o)))
        out.append(Kernel("nf4_dequant_bw", f"[{rows},1536] nf4->fp16 (one layer's NF4 "
                          "elements)", "hbm", work, launches, step=False))
    if "rmsnorm_bwd_bw" in names:
        xb = torch.randn(nb, hid, device=dev).half()
        wb = torch.rand(hid, device=dev).half() + 0.5
        rstd = torch.empty(nb, dtype=torch.float32, device=dev)
        o = torch.empty(nb, hid, dtype=torch.float16, device=dev)
        bound("cm_rmsnorm_fwd", xb.data_ptr(), _lib.F16, hid, wb.data_ptr(), _lib.F16,
              o.data_ptr(), _lib.F16, rstd.data_ptr(), None, None, None, 0, nb, hid, 1e-6,
              _stream(dev))()  # real rstd before the backward is timed
        launches = []
        for _ in range(2):
            dy = torch.randn(nb, hid, device=dev).half()
            dx = torch.empty(nb, hid, dtype=torch.float16, device=dev)
            launches.append((bound("cm_rmsnorm_bwd", dy.data_ptr(), _lib.F16, xb.data_ptr(),
                                   _lib.F16, wb.data_ptr(), _lib.F16, rstd.data_ptr(),
                                   dx.data_ptr(), _lib.F16, None, None, None, 0, 0, nb, hid,
                                   _stream(dev)), (xb, wb, rstd, dy, dx)))
        out.append(Kernel("rmsnorm_bwd_bw", f"N={nb} H=1536 fp16", "hbm",
                          6 * nb * hid + 4 * nb + 2 * hid, launches, step=False))
    if "lora_pack_bw" in names or "lora_unpack_bw" in names:
        n_el = nb * hid
        x = torch.randn(n_el, device=dev)
        keep = torch.rand(n_el, device=dev) > 0.05
        xd = torch.empty(n_el, dtype=torch.float16, device=dev)
        bits = torch.empty(n_el // 8, dtype=torch.uint8, device=dev)
        g16 = torch.randn(n_el, device=dev).half()
        dx = torch.empty(n_el, device=dev)
        xd2 = torch.empty(n_el, dtype=torch.float16, device=dev)
        t = (x, keep, xd, bits, g16, dx, xd2)
        p = bound("cm_lora_pack", x.data_ptr(), _lib.F32, keep.data_ptr(), xd.data_ptr(),
                  bits.data_ptr(), n_el, 1 / 0.95, _stream(dev))
        p()
        if "lora_pack_bw" in names:
            out.append(Kernel("lora_pack_bw", f"[{nb},1536] fp32 x", "hbm", 7 * n_el + n_el // 8,
                              [(p, t)], step=False))
        if "lora_unpack_bw" in names:
            u = bound("cm_lora_unpack", xd.data_ptr(), bits.data_ptr(), g16.data_ptr(),
                      xd2.data_ptr(), dx.data_ptr(), _lib.F32, n_el, 1 / 0.95, _stream(dev))
            out.append(Kernel("lora_unpack_bw", f"[{nb},1536] -> fp32 dx", "hbm",
                              10 * n_el + n_el // 8, [(u, t)], step=False))
    if "rmsnorm_fwd_bw" in names:
        xb = torch.randn(nb, hid, device=dev).half()
        wb = torch.rand(hid, device=dev).half() + 0.5
        rstd = torch.empty(nb, dtype=torch.float32, device=dev)
        launches = []
        for _ in range(2):
            o = torch.empty(nb, hid, dtype=torch.float16, device=dev)
            launches.append((bound("cm_rmsnorm_fwd", xb.data_ptr(), _lib.F16, hid, wb.data_ptr(),
                                   _lib.F16, o.data_ptr(), _lib.F16, rstd.data_ptr(), None, None,
                                   None, 1, nb, hid, 1e-6, _stream(dev)), (xb, wb, rstd, o)))
        out.append(Kernel("rmsnorm_fwd_bw", f"N={nb} H=1536 fp16", "hbm",
                          4 * nb * hid + 4 * nb + 2 * hid, launches, step=False))
    if "rope_fwd_bw" in names:
        q = torch.randn(1, nb, 12 * 128, device=dev).half().view(1, nb, 12, 128).transpose(1, 2)
        k = torch.randn(1, nb, 2 * 128, device=dev).half().view(1, nb, 2, 128).transpose(1, 2)
        cos, sin = orope.cos_sin(torch.arange(nb) % 512, 128, 1e6, torch.float16)
        cos, sin = cos.to(dev), sin.to(dev)
        launches = [_rope_launch(dev, q, k, cos, sin, False)]
        out.append(Kernel("rope_fwd_bw", f"N={nb} 12+2 heads x 128", "hbm",
                          2 * 2 * nb * 14 * 128 + 2 * 2 * nb * 128, launches, step=False))
    if "rope_bwd_bw" in names:
        q = torch.randn(1, nb, 12 * 128, device=dev).half().view(1, nb, 12, 128).transpose(1, 2)
        k = torch.randn(1, nb, 2 * 128, device=dev).half().view(1, nb, 2, 128).transpose(1, 2)
        cos, sin = orope.cos_sin(torch.arange(nb) % 512, 128, 1e6, torch.float16)
        cos, sin = cos.to(dev), sin.to(dev)
        launches = [_rope_launch(dev, q, k, cos, sin, True)]
        out.append(Kernel("rope_bwd_bw", f"N={nb} 12+2 heads x 128", "hbm",
                          2 * 2 * nb * 14 * 128 + 2 * 2 * nb * 128, launches, step=False))
    return out


def k_nf4_linear(dev, names):
    """The NF4-fused GEMM at the training step's MLP shapes (1276 packed tokens, Qwen2.5-1.5B
    gate/up [8960,1536]): the gate+up forward (also the backward's recompute) and the input
    gradient dgate Wg + dup Wu, each beside the unfused path it replaces (the dequant kernel +
    torch's fp16 GEMM)."""
    import ctypes

    import torch

    from claudemaxing_amd import _lib, gemm, nf4
    from claudemaxing_amd.nf4_linear import _weights

    m, f, h = 1276, 8960, 1536
    gen = torch.Generator().manual_seed(0)
    qs = [nf4.quantize_nf4(torch.randn(f, h, generator=gen) * 0.02, 64, True) for _ in range(2)]
    x = torch.randn(m, h, generator=gen).half()
    g = torch.randn(m, f, generator=gen).half()
    flops = 2 * 2 * m * f * h
    in_bytes = sum(p.numel() for p, _ in qs) + x.numel() * 2
    out = []
    fwd, fwd_ref, fwd_merged, bwd, bwd_ref, bwd_split = [], [], [], [], [], []
    for _ in range(copies_for(in_bytes + 2 * g.numel() * 2)):
        pairs = [(p.to(dev), st.to(dev)) for p, st in qs]
        xd, gd = x.to(dev), g.to(dev)
        ys = [torch.empty(m, f, dtype=torch.float16, device=dev) for _ in range(2)]
        dx = torch.empty(m, h, dtype=torch.float16, device=dev)
        w_arr, keep = _weights(pairs)[:2]
        out_arr = (ctypes.c_void_p * 2)(*[y.data_ptr() for y in ys])
        ldo = (ctypes.c_int64 * 2)(f, f)
        g_arr = (ctypes.c_void_p * 2)(gd.data_ptr(), gd.data_ptr())
        ldg = (ctypes.c_int64 * 2)(f, f)
        w2 = torch.empty(2 * f, h, dtype=torch.float16, device=dev)  # [Wg; Wu]
        gcat = torch.cat([gd, gd], 1)  # [dgate | dup], the merged product's gradient
        assert xd.shape == (m, h) and all(y.shape == (m, f) for y in ys) and dx.shape == (m, h)
        hold = (pairs, xd, gd, ys, dx, w_arr, keep, out_arr, ldo, g_arr, ldg, w2, gcat)
        fwd.append((bound("cm_nf4_linear_fwd", xd.data_ptr(), h, m, w_arr, 2, None, out_arr, ldo,
                          _lib.F16, None, 0, _stream(dev)), hold))
        ws_bytes = _lib.load().cm_nf4_linear_workspace_bytes(m, w_arr, 2, 1)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        bwd.append((bound("cm_nf4_linear_bwd", g_arr, ldg, m, w_arr, 2, dx.data_ptr(), h,
                          _lib.F16, ws.data_ptr(), ws_bytes, _stream(dev)), hold + (ws,)))

        def ref_f(pairs=pairs, xd=xd):
            for p, st in pairs:
                torch.nn.functional.linear(xd, nf4.dequantize_nf4(p, st, torch.float16))

        def ref_b(pairs=pairs, gd=gd):
            wg, wu = (nf4.dequantize_nf4(p, st, torch.float16) for p, st in pairs)
            torch.addmm(torch.mm(gd, wg), gd, wu)

        def expand_pair(pairs=pairs, w2=w2):
            for (p, st), half in zip(pairs, (w2[:f], w2[f:])):
                nf4.dequantize_nf4(p, st, torch.float16, out=half)

        def merged_f(xd=xd, w2=w2, expand_pair=expand_pair):
            # the training step's path: both weights expanded into one [2F, K] weight, one GEMM
            expand_pair()
            torch.nn.functional.linear(xd, w2)

        def split_b(gcat=gcat, w2=w2, expand_pair=expand_pair):
            # the training step's path: the same [2F, K] weight, then one split-K launch over the
            # concatenated contraction with an fp32 result, reading the weight k-major
            expand_pair()
            gemm.gemm_f32((gcat, w2), b_kmajor=True)

        fwd_ref.append((ref_f, hold))
        fwd_merged.append((merged_f, hold))
        bwd_ref.append((ref_b, hold))
        bwd_split.append((split_b, hold))
    if "nf4_linear_fwd" in names:
        out.append(Kernel("nf4_linear_fwd", f"gate+up {m} tokens x 2 x [{f},{h}] nf4", "mfma",
                          flops, fwd))
        out.append(Kernel("nf4_linear_fwd_unfused", "the same: dequant + torch fp16 GEMM x 2",
                          "mfma", flops, fwd_ref, step=False))
        out.append(Kernel("nf4_linear_fwd_merged", "the same: dequant x 2 into one [2F,K] weight "
                          "+ one torch fp16 GEMM (the training step's path)", "mfma", flops,
                          fwd_merged, step=False))
    if "nf4_linear_bwd" in names:
        out.append(Kernel("nf4_linear_bwd", f"dgate Wg + dup Wu, {m} tokens", "mfma", flops, bwd))
        out.append(Kernel("nf4_linear_bwd_unfused", "the same: dequant x 2 + mm + addmm", "mfma",
                          flops, bwd_ref, step=False))
        out.append(Kernel("nf4_linear_bwd_split", "the same: dequant x 2 into one [2F,K] weight "
                          "+ split-K cm_gemm_f32_kb over the 2F contraction (fp32 dx, the weight "
                          "read k-major; the training step's path)", "mfma", flops, bwd_split,
                          step=False))
    return out


def _chunk_plan(n, vocab, hidden, chunk, noalloc=False):
    """The vocabulary chunks and gradient K-slices of one LM-head call, e.g. {"chunks":
    "4x32768+20864", "k_slices": 4}."""
    from claudemaxing_amd import lm_head_loss

    c, split = lm_head_loss.fused_head_plan(n, vocab, hidden, chunk, noalloc=noalloc)
    full, rest = divmod(vocab, c)
    chunks = f"{full}x{c}" + (f"+{rest}" if rest else "")
    return {"chunks": chunks, "k_slices": split}


def k_lmhead(dev):
    import ctypes

    import torch

    from claudemaxing_amd import _lib, lm_head_loss
    from oracle import inputs

    h, w, t = inputs.lm_head(0)
    hd, wd, td = h.to(dev), w.to(dev), t.to(dev)
    n, vocab, hidden = h.shape[0], w.shape[0], h.shape[1]
    flops = 4 * n * vocab * hidden
    w16 = lm_head_loss.fp16_head_weight(wd)  # the host's cached fp16 weight, as in training
    keep = (hd, wd, td, w16)

    def launch(hd=hd, w16=w16, td=td):
        return lm_head_loss._fused_rows(hd, w16, td, True, None)

    def launch_8192(hd=hd, w16=w16, td=td):
        return lm_head_loss._fused_rows(hd, w16, td, True, 8192)

    # the entry point that allocates nothing, at its own chunk (its outputs preallocated once)
    outs = [torch.empty(n, device=dev), torch.empty(n, device=dev),
            torch.empty(n, dtype=torch.int32, device=dev), torch.empty(n, hidden, device=dev)]
    lib = _lib.load()
    noalloc_args = (hd.data_ptr(), hd.stride(0), w16.data_ptr(), w16.stride(0), td.data_ptr(), n,
                    vocab, hidden, 0, outs[0].data_ptr(), outs[1].data_ptr(),
                    outs[2].data_ptr(), outs[3].data_ptr(), ctypes.c_float(1.0),
                    _lib.stream(dev))

    def launch_noalloc():
        rc = lib.cm_lmhead_ce_noalloc(*noalloc_args)
        if rc:
            raise RuntimeError(f"cm_lmhead_ce_noalloc: {lib.cm_error_string(rc).decode()}")

    launch()
    launch_8192()
    launch_noalloc()
    torch.cuda.synchronize()
    shape = f"N={n} V={vocab} H={hidden} fp16"
    return [Kernel("lmhead_ce", shape, "mfma", flops, [(launch, keep)],
                   plan=_chunk_plan(n, vocab, hidden, None)),
            Kernel("lmhead_ce_chunk8192", shape + " in 8192-column vocabulary chunks (config 4's "
                   "stated chunk: a 32 MiB E buffer)", "mfma", flops, [(launch_8192, keep)],
                   step=False, plan=_chunk_plan(n, vocab, hidden, 8192)),
            Kernel("lmhead_ce_noalloc", shape + " through cm_lmhead_ce_noalloc (no workspace "
                   "argument: its own 64 MiB scratch array, its own chunk)", "mfma", flops,
                   [(launch_noalloc, keep + tuple(outs))], step=False,
                   plan=_chunk_plan(n, vocab, hidden, 0, noalloc=True))]


ALL = ["nf4_dequant", "rmsnorm_fwd", "rmsnorm_bwd", "rmsnorm_fwd_w32", "rmsnorm_bwd_w32",
       "rmsnorm_fwd_qlora", "rmsnorm_bwd_qlora", "rope_fwd", "rope_bwd", "swiglu_fwd",
       "swiglu_bwd", "lora_pack", "lora_unpack", "hbm_copy_ref", "floor_empty", "floor_empty_grid",
       "floor_one_wave", "floor_copy_1mib", "nf4_dequant_bw", "rmsnorm_fwd_bw", "rmsnorm_bwd_bw", "rope_fwd_bw",
       "rope_bwd_bw", "lora_pack_bw", "lora_unpack_bw", "nf4_linear_fwd", "nf4_linear_bwd",
       "lmhead_ce"]
BW_ROWS = {"nf4_dequant_bw", "rmsnorm_fwd_bw", "rmsnorm_bwd_bw", "rope_fwd_bw", "rope_bwd_bw",
           "lora_pack_bw", "lora_unpack_bw"}
FLOORS = {"floor_empty", "floor_empty_grid", "floor_one_wave", "floor_copy_1mib"}


def build_kernels(dev, only):
    from oracle import inputs

    names = set(only) if only else set(ALL)
    kernels = []
    if "nf4_dequant" in names:
        kernels += k_nf4(dev)
    c2 = inputs.rmsnorm_rope(0)
    if names & {"rmsnorm_fwd", "rmsnorm_bwd", "rmsnorm_fwd_w32", "rmsnorm_bwd_w32",
                 "rmsnorm_fwd_qlora", "rmsnorm_bwd_qlora"}:
        kernels += k_rmsnorm(dev, c2, names)
    if names & {"rope_fwd", "rope_bwd"}:
        kernels += k_rope(dev, c2, names)
    if names & {"swiglu_fwd", "swiglu_bwd"}:
        kernels += k_swiglu(dev, names)
    if names & {"lora_pack", "lora_unpack"}:
        kernels += k_lora(dev, names)
    if "hbm_copy_ref" in names:
        kernels += k_copy_ref(dev)
    if names & FLOORS:
        kernels += k_floor(dev, names)
    if names & BW_ROWS:
        kernels += k_bandwidth_scale(dev, names)
    if names & {"nf4_linear_fwd", "nf4_linear_bwd"}:
        kernels += k_nf4_linear(dev, names)
    if "lmhead_ce" in names:
        kernels += k_lmhead(dev)
    return kernels


def time_kernel(kern, steps, warmup):
    """Milliseconds per launch: `steps` launches (rotating over the input copies) issued back
    to back between two HIP events recorded on the launch stream (torch's current stream,
    which every entry point is given). The closures hold pre-converted arguments, so for the
    microsecond kernels the host issue rate stays close to the device rate; the rocprofv3
    kernel trace of the same command gives the device-only durations."""
    import torch

    fns = [f for f, _ in kern.launches]
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fns[i % len(fns)]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


TRAFFIC_PROFILES = {"lmhead_ce": ROOT / "profiles" / "lmhead_ce_N2048_V151936_H1536.md"}


def traffic_from_profile(name):
    """HBM-side bytes per launch of kernel `name` from its committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter's reading for a device copy
    of known size), or None when there is no summary. Counters cannot be read inside a timed
    run, so the figure is that of the profiled build of the same command."""
    path = TRAFFIC_PROFILES.get(name)
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_call:"):
            return int(line.split(":", 1)[1])
    return None


def _smi_sample(smi):
    """(socket power W, mean graphics clock MHz) from one `amd-smi metric -p -c --json`, or
    None when the tool's output cannot be read."""
    import subprocess

    try:
        r = subprocess.run([smi, "metric", "-p", "-c", "--json"], capture_output=True, text=True,
                           timeout=10)
        data = json.loads(r.stdout)
    except (OSError, ValueError, subprocess.SubprocessError):
        return None
    if isinstance(data, dict):
        data = data.get("gpu_data", [data])
    if not data:
        return None
    gpu = data[0]
    try:
        watts = float(gpu["power"]["socket_power"]["value"])
        clocks = [float(v["clk"]["value"]) for k, v in gpu["clock"].items()
                  if k.startswith("gfx_") and isinstance(v, dict) and "clk" in v]
    except (KeyError, TypeError, ValueError):
        return None
    return watts, (sum(clocks) / len(clocks) if clocks else None)


def measured_peaks(dev, power=True):
    """The two roofline denominators as this board attains them (cm_probe_hbm,
    cm_probe_mfma_f16): a 16-byte stream over 2 GiB, read only and copied (GB/s of bytes read +
    written; the best of 1, 4, 16 words per lane with plain or nontemporal loads), and
    v_mfma_f32_32x32x16_f16 on register operands of N(0,1) fp16 data (TFLOP/s; the best of 2, 4,
    8 accumulator chains per wavefront); median of 5 launches after 2 warm-ups, HIP events around
    each launch on the launch stream. With power, the board's power and clock while the MFMA
    probe runs back to back."""
    import torch

    from claudemaxing_amd import _lib

    lib = _lib.load()
    stream = _lib.stream(dev)
    cur = torch.cuda.current_stream(dev)

    def median_s(fn, n=5, warm=2):
        for _ in range(warm):
            fn()
        times = []
        for _ in range(n):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(cur)
            fn()
            b.record(cur)
            b.synchronize()
            times.append(a.elapsed_time(b) * 1e-3)
        return sorted(times)[n // 2]

    nbytes = 2 << 30
    src = torch.randint(0, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    read, copy = {}, {}
    for per_lane in (1, 4, 16):
        for nt in (0, 1):
            key = f"{per_lane}{'nt' if nt else ''}"
            read[key] = nbytes / median_s(
                lambda q=per_lane, t=nt: _lib.call("cm_probe_hbm", src.data_ptr(), None, nbytes,
                                                   q, t, sink.data_ptr(), stream)) / 1e9
            copy[key] = 2 * nbytes / median_s(
                lambda q=per_lane, t=nt: _lib.call("cm_probe_hbm", src.data_ptr(), dst.data_ptr(),
                                                   nbytes, q, t, sink.data_ptr(), stream)) / 1e9
    del src, dst
    gen = torch.Generator().manual_seed(0)
    ops = torch.randn(512 * 8, generator=gen).half().to(dev)
    iters = 2000
    rates = {}
    for chains in (2, 4, 8):
        flops = int(lib.cm_probe_mfma_f16_flops(iters, chains))
        sec = median_s(lambda c=chains: _lib.call("cm_probe_mfma_f16", ops.data_ptr(), iters, c,
                                                  sink.data_ptr(), stream))
        rates[chains] = flops / sec / 1e12
    best = max(rates, key=rates.get)

    def mfma():
        _lib.call("cm_probe_mfma_f16", ops.data_ptr(), iters, best, sink.data_ptr(), stream)

    out = dict(hbm_read_GBs=round(max(read.values()), 1),
               hbm_copy_GBs=round(max(copy.values()), 1),
               hbm_GBs_by_variant={q: dict(read=round(read[q], 1), copy=round(copy[q], 1))
                                   for q in read},
               mfma_f16_TFLOPs=round(rates[best], 1),
               mfma_f16_TFLOPs_by_chains={c: round(r, 1) for c, r in rates.items()},
               spec=dict(hbm_GBs=HBM_PEAK_GBS, mfma_f16_TFLOPs=MFMA_FP16_PEAK_TFLOPS),
               note="cm_probe_hbm over 2 GiB (read only; copied, bytes read + written; 1, 4 or "
                    "16 16-byte words per lane, plain or nontemporal (nt) loads: the best) and "
                    "cm_probe_mfma_f16 (2048 x 4 wavefronts x 2000 x 2 x chains MFMAs 32x32x16 "
                    "on N(0,1) fp16 register operands, chains 2, 4, 8 accumulators per "
                    "wavefront: the best), median of 5")
    if power:
        out["mfma_power"] = board_power(mfma)
    return out


def board_power(fn, seconds=2.0):
    """The board's socket power and graphics clock (amd-smi, about 5 samples a second) while
    `fn` runs back to back for `seconds`, or None without a readable amd-smi. The matrix-core
    kernels run into the board's power limit, which sets the clock they run at."""
    import shutil
    import threading

    import torch

    smi = shutil.which("amd-smi")
    if smi is None or _smi_sample(smi) is None:
        return None
    samples, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            v = _smi_sample(smi)
            if v is not None:
                samples.append(v)
            stop.wait(0.2)

    fn()
    torch.cuda.synchronize()
    th = threading.Thread(target=poll, daemon=True)
    t0 = time.perf_counter()
    th.start()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    steady = samples[1:] or samples  # the first sample may precede the ramp
    if not steady:
        return None
    watts = sorted(w for w, _ in steady)
    mhz = sorted(c for _, c in steady if c is not None)
    return dict(socket_w=watts[len(watts) // 2],
                gfx_mhz=round(mhz[len(mhz) // 2]) if mhz else None, samples=len(steady),
                window_s=seconds,
                note="amd-smi metric -p -c (median over the window) while the headline call runs "
                     "back to back, after the timed region; 2.5 PFLOP/s is the 2.4 GHz peak")


def cpu_baseline(headline):
    """The oracle of the headline kernel on the host cores, on a bounded sample."""
    import numpy as np
    import torch

    from oracle import inputs
    from oracle import nf4 as onf4

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    if headline == "lmhead_ce":
        from oracle import lm_head as olm

        h, w, t = inputs.lm_head(0)
        rows = h.shape[0]  # the whole workload: all 2048 rows, full vocabulary, with grad
        times = []
        t_all = time.perf_counter()
        while len(times) < 3 and (not times or time.perf_counter() - t_all < 10.0):
            t0 = time.perf_counter()
            olm.head(h, w, t, want_grad=True, rows_per_block=256)
            times.append(time.perf_counter() - t0)
        dt = float(np.median(times))
        flops = 4 * rows * w.shape[0] * w.shape[1]
        return dict(value=round(flops / dt / 1e12, 4), unit="TFLOP/s", cores=cores, kind="port",
                    sample=f"oracle.lm_head.head (torch CPU, fp32 GEMMs) on the whole workload "
                           f"(2048 rows, full vocabulary, with grad), median of {len(times)} "
                           f"runs of {dt:.1f} s")
    w = inputs.nf4_weight(0)
    q = onf4.quantize(w.numpy(), 64, True)
    nbytes = w.numel() // 2 + q["absmax"].size + q["absmax2"].size * 4 + 256 * 4 + 64 + 4 + \
        w.numel() * 2
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        onf4.dequant(q["packed"], q["absmax"], nested=True, code2=q["code2"],
                     absmax2=q["absmax2"], offset=q["offset"], blocksize=64, blocksize2=256)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    return dict(value=round(nbytes / dt / 1e9, 4), unit="GB/s", cores=1, kind="port",
                sample=f"oracle.nf4.dequant (numpy, 1 thread) of the full config-1 weight, "
                       f"median of 3 ({dt * 1e3:.0f} ms)")


def qlora_step_graphed_bench(dev, steps, warmup=2):
    """Config 5's repeated batch replayed from its HIP graph, nothing else (one eager step before
    the capture warms up the model), for a kernel trace of that step alone."""
    import torch

    from claudemaxing_amd import qlora_step

    model = qlora_step.build_model(dev, seed=0)
    batch, lengths = qlora_step.make_batch(dev, seed=0)
    opt = qlora_step.make_optimizer(model)
    scaler = torch.amp.GradScaler("cuda")
    qlora_step.train_step(model, opt, scaler, batch)
    rg = qlora_step.time_steps(model, opt, scaler, batch, steps, warmup, graphed=True)
    tokens = int(lengths.sum())
    return dict(fixed_batch=f"{tokens} real tokens (lengths {lengths.tolist()}), repeated",
                graphed=dict(median_ms=round(rg["median_ms"], 2),
                             step_ms=[round(x, 2) for x in rg["step_ms"]],
                             tokens_per_s=round(tokens / (rg["median_ms"] * 1e-3), 1)))


def qlora_step_bench(dev, steps, warmup=2):
    """Config 5: one QLoRA training step of the 28-layer Qwen2.5-1.5B-shaped model (random
    init, NF4 base weights, LoRA r16/a32/p0.05 on q/v, fp16 autocast, AdamW + GradScaler, batch
    of 4 rows of U[64,512] tokens packed out). Each step is timed between two device syncs, as
    the reference's harness times its trainer steps; the median is reported with the peak HBM
    of the timed steps, for the eager step and for the step replayed from a HIP graph (the same
    model and optimizer continue, so the graphed steps start from the eager steps' weights)."""
    import torch

    from claudemaxing_amd import qlora_step

    torch.cuda.reset_peak_memory_stats()  # the kernel lines above are not the step's
    t0 = time.perf_counter()
    whole = qlora_step.VramPoller(dev).__enter__()  # the build and every step below
    model = qlora_step.build_model(dev, seed=0)
    batch, lengths = qlora_step.make_batch(dev, seed=0)
    opt = qlora_step.make_optimizer(model)
    scaler = torch.amp.GradScaler("cuda")
    build_s = time.perf_counter() - t0
    build_peak_allocated = torch.cuda.max_memory_allocated() / 2 ** 30
    # the headline step figure: a fresh batch (new lengths) every step, eager, TRL's metrics
    # computed every step; then one repeated batch eager; then the fresh batches with a new HIP
    # graph captured for every batch (capture inside the timed step), and the repeated batch
    # replayed from a graph. The eager runs come first: the capture stream keeps torch's BLAS
    # workspaces, which would otherwise count in the eager peaks.
    with qlora_step.VramPoller(dev) as vram:
        rd = qlora_step.time_distinct_batches(model, opt, scaler, steps, warmup)
    r = qlora_step.time_steps(model, opt, scaler, batch, steps, warmup)
    rdg = qlora_step.time_distinct_batches(model, opt, scaler, max(3, steps // 3), 1,
                                           mode="capture_each")
    rg = qlora_step.time_steps(model, opt, scaler, batch, steps, warmup, graphed=True)
    # the SFT figure: fresh batches every step, each replayed from its 256-token bucket's graph
    # (the first batch of a bucket captures it inside its timed step), TRL's metrics every step
    torch.cuda.empty_cache()
    with qlora_step.VramPoller(dev) as vram_b:
        rb = qlora_step.time_distinct_batches(model, opt, scaler, 3 * steps, 2, seed0=5000,
                                              mode="bucketed", bucket=256)
    tokens = int(lengths.sum())
    out = dict(config="Qwen2.5-1.5B shape, 28 layers, NF4 + LoRA r16 q/v, batch 4 of U[64,512] "
                      "tokens packed out, fp16 autocast, AdamW + GradScaler",
               distinct_batches=dict(
                   median_ms=round(rd["median_ms"], 2), step_ms=[round(x, 2) for x in rd["step_ms"]],
                   tokens=rd["tokens"], tokens_per_s=round(rd["tokens_per_s"], 1),
                   peak_allocated_gb=round(rd["peak_allocated_gb"], 3),
                   peak_reserved_gb=round(rd["peak_reserved_gb"], 3),
                   peak_allocated_mib=round(rd["peak_allocated_gb"] * 1024),
                   peak_reserved_mib=round(rd["peak_reserved_gb"] * 1024),
                   device_used_peak_mib=round(vram.peak),
                   device_used_at_start_mib=round(whole.start),
                   device_used_peak_over_start_mib=round(vram.peak - whole.start),
                   memory_note="torch's peak allocated / reserved bytes over the timed steps, and "
                               "device memory in use (total - free, every 100 ms, as the "
                               "reference's harness polls nvidia-smi) at its peak over them and "
                               "before this process allocated anything; the reference publishes "
                               "2447 / 2696 MiB allocated / reserved and a 2839 MiB nvidia-smi "
                               "peak (T4, EXPERIMENTS.md run 5)",
                   note="eager, a new batch every step",
                   bucketed_graphs=dict(
                       median_ms=round(rb["median_ms"], 2), mean_ms=round(rb["mean_ms"], 2),
                       step_ms=[round(x, 2) for x in rb["step_ms"]], tokens=rb["tokens"],
                       tokens_per_s=round(rb["tokens_per_s"], 1),
                       captures_timed=rb["captures_timed"],
                       capture_ms=[round(x, 1) for x in rb["capture_ms"]],
                       buckets=rb["buckets"], graph_pool_gb=round(rb["graph_pool_gb"], 3),
                       peak_allocated_gb=round(rb["peak_allocated_gb"], 3),
                       peak_reserved_gb=round(rb["peak_reserved_gb"], 3),
                       device_used_peak_mib=round(vram_b.peak),
                       device_used_peak_over_start_mib=round(vram_b.peak - whole.start),
                       note="the step an SFT run sees: a new batch every step, packed to the "
                            "next multiple of 256 tokens (a filler row with ignored labels) and "
                            "replayed from that bucket's HIP graph; a bucket's first batch "
                            "captures its graph inside the timed step (captures_timed of them, "
                            "capture_ms each); graphs share one memory pool; TRL's three "
                            "metrics every step"),
                   graphed_with_capture=dict(
                       median_ms=round(rdg["median_ms"], 2),
                       step_ms=[round(x, 2) for x in rdg["step_ms"]],
                       note="a new HIP graph captured (one warm-up pass + capture) and replayed "
                            "for every batch, all inside the timed step")),
               fixed_batch=f"{tokens} real tokens (lengths {lengths.tolist()}), repeated",
               median_ms=round(r["median_ms"], 2), step_ms=[round(x, 2) for x in r["step_ms"]],
               tokens_per_s=round(tokens / (r["median_ms"] * 1e-3), 1),
               peak_allocated_gb=round(r["peak_allocated_gb"], 3),
               peak_reserved_gb=round(r["peak_reserved_gb"], 3),
               losses=[round(x, 4) for x in r["losses"]], build_s=round(build_s, 1),
               warmup=warmup, steps=steps,
               graphed=dict(median_ms=round(rg["median_ms"], 2),
                            step_ms=[round(x, 2) for x in rg["step_ms"]],
                            tokens_per_s=round(tokens / (rg["median_ms"] * 1e-3), 1),
                            peak_allocated_gb=round(rg["peak_allocated_gb"], 3),
                            graph_pool_gb=round(rg["graph_pool_gb"], 3),
                            peak_hbm_gb=round(rg["peak_allocated_gb"] + rg["graph_pool_gb"], 3),
                            losses=[round(x, 4) for x in rg["losses"]],
                            note="forward + backward replayed from one HIP graph per packed "
                                 "shape; packing and the GradScaler/AdamW step eager; "
                                 "peak_hbm_gb = the replay's peak allocated bytes + the "
                                 "graph's private pool (activations of the captured pass)"))
    whole.__exit__(None, None, None)
    out["build_peak_allocated_gb"] = round(build_peak_allocated, 3)
    out["device_used_peak_whole_run_mib"] = round(whole.peak)
    del model, opt
    torch.cuda.empty_cache()
    return out


def step_in_child(steps):
    """qlora_step_bench in a child process (this file with --step-json-only): its progress lines
    pass through to stderr, its record is the last line of its stdout. A failed step fails the
    run."""
    import subprocess

    print("[bench] qlora_step (child process) ...", file=sys.stderr, flush=True)
    res = subprocess.run([sys.executable, "-u", str(Path(__file__).resolve()), "--step-json-only",
                          "--only", "qlora_step", "--step-steps", str(steps), "--no-cpu",
                          "--no-peaks", "--no-power"],
                         stdout=subprocess.PIPE, text=True, timeout=900)
    if res.returncode != 0:
        sys.exit(f"bench.py: the QLoRA step's child process failed (exit {res.returncode})")
    return json.loads(res.stdout.strip().splitlines()[-1])


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this kernel set has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    only = [x for x in args.only.split(",") if x]
    step = None
    want_step = not args.no_step and (not only or "qlora_step" in only)
    if want_step and not args.step_graphed_only and not args.step_json_only:
        # the training step runs first, in a child process of its own started before this one
        # touches the GPU: its device-level memory figures (polled total - free) then start from
        # a fresh process, and the kernel lines below run in a process the step never shaped
        # (after the step in one process, NF4 config 1 measured 9.8 against 6.9 us, RMSNorm 8.2
        # against 4.4 us)
        step = step_in_child(args.step_steps)
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if want_step and (args.step_graphed_only or args.step_json_only):
        print("[bench] qlora_step ...", file=sys.stderr, flush=True)
        if args.step_graphed_only:
            step = qlora_step_graphed_bench(dev, args.step_steps)
            print(f"[bench] qlora_step: {step['graphed']['median_ms']} ms graphed", file=sys.stderr,
                  flush=True)
        else:
            step = qlora_step_bench(dev, args.step_steps)
            print(json.dumps(step), flush=True)
            return
    if step is not None and not args.step_graphed_only:
        b = step["distinct_batches"]["bucketed_graphs"]
        print(f"[bench] qlora_step: {step['distinct_batches']['median_ms']} ms per step eager over "
              f"distinct batches, {b['median_ms']} ms median ({b['mean_ms']} mean, "
              f"{b['captures_timed']} captures) replayed from bucketed graphs "
              f"({step['distinct_batches']['graphed_with_capture']['median_ms']} ms capturing a "
              f"graph per batch); fixed batch {step['median_ms']} ms eager, "
              f"{step['graphed']['median_ms']} ms graphed; eager peak allocated / reserved "
              f"{step['distinct_batches']['peak_allocated_mib']} / "
              f"{step['distinct_batches']['peak_reserved_mib']} MiB, device in use "
              f"{step['distinct_batches']['device_used_peak_over_start_mib']} MiB over the "
              f"process start", file=sys.stderr, flush=True)
    if step is not None:
        gc.collect()
        torch.cuda.empty_cache()
    kernels = build_kernels(dev, only)
    torch.cuda.synchronize()
    results = {}
    power = None
    for kern in kernels:
        print(f"[bench] {kern.name} ...", file=sys.stderr, flush=True)
        ms = time_kernel(kern, args.steps, args.warmup)
        if kern.name == "lmhead_ce" and not args.no_power:
            power = board_power(kern.launches[0][0])
            if power:
                print(f"[bench] lmhead_ce board power: {power['socket_w']} W, graphics clock "
                      f"{power['gfx_mhz']} MHz", file=sys.stderr, flush=True)
        if kern.bound == "hbm":
            achieved, peak, unit = kern.work / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
            if kern.name in FLOORS:
                unit = "GB/s (launch floor)"
        else:
            achieved, peak, unit = kern.work / (ms * 1e-3) / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s"
        results[kern.name] = dict(config=kern.config, us=round(ms * 1e3, 2),
                                  achieved=round(achieved, 1), unit=unit, bound=kern.bound,
                                  frac=round(achieved / peak, 4), work=kern.work,
                                  in_step=kern.step)
        if kern.plan is not None:
            results[kern.name]["plan"] = kern.plan
        print(f"[bench] {kern.name}: {ms * 1e3:.2f} us, {achieved:.1f} {unit} "
              f"({100 * achieved / peak:.1f}% of peak)", file=sys.stderr, flush=True)
    if not results:
        sys.exit("bench.py: --only must name at least one kernel")
    # the kernel benches' inputs (rotated copies beyond 512 MiB) must not count in the step's
    # peak memory
    del kernels, kern
    gc.collect()
    torch.cuda.empty_cache()
    headline = "lmhead_ce" if "lmhead_ce" in results else next(iter(results))
    hr = results[headline]
    peaks = None
    if not args.no_peaks:
        print("[bench] measured peaks ...", file=sys.stderr, flush=True)
        peaks = measured_peaks(dev, power=not args.no_power)
        print(f"[bench] measured peaks: HBM {peaks['hbm_read_GBs']} GB/s read, "
              f"{peaks['hbm_copy_GBs']} GB/s copy; fp16 MFMA {peaks['mfma_f16_TFLOPs']} TFLOP/s",
              file=sys.stderr, flush=True)
        # the matrix-core probe bounds every MFMA kernel; the single-stream HBM probe does not
        # bound the elementwise kernels that stream several arrays at once (LoRA pack/unpack
        # and RMSNorm forward at bandwidth scale exceed its copy rate), so HBM fractions stay
        # against the published 8 TB/s
        for r in results.values():
            if r["bound"] == "mfma":
                r["frac_of_measured"] = round(r["achieved"] / peaks["mfma_f16_TFLOPs"], 4)
    line = {
        "metric": METRIC,
        "value": hr["achieved"],
        "unit": hr["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(hr["us"] / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if headline == "lmhead_ce" else "u8->fp16",
        "data": "synthetic (seeded CPU draws of BASELINE.json configs, copied to HBM)",
        "config": {"workload": headline, "shape": hr["config"], "parallelism": "none (1 GPU)",
                   "cold_cache": "input copies rotated beyond 512 MiB", **hr.get("plan", {})},
        "roofline": {"bound": hr["bound"], "achieved": hr["achieved"],
                     "peak": HBM_PEAK_GBS if hr["bound"] == "hbm" else MFMA_FP16_PEAK_TFLOPS,
                     "unit": hr["unit"], "frac": hr["frac"],
                     "traffic": traffic_from_profile(headline),
                     "frac_of_measured_peak": hr.get("frac_of_measured")},
        "kernels": results,
        "power": power,
        "measured_peaks": peaks,
        "ms_per_step_note": "one headline call (the fused LM head at config 4) per step",
        "in_step_kernel_sum_ms": round(sum(r["us"] for r in results.values()
                                           if r["in_step"]) / 1e3, 4),
    }
    if step is not None:
        line["qlora_step"] = step
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(headline)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
