"""Benchmark of the QLoRA step kernel set on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME[,NAME...]]

Every kernel runs on inputs already resident in HBM, at the shapes of BASELINE.json's configs:
  1  NF4 dequant of the [8960,1536] gate_proj weight (blocksize 64, double-quantized) to fp16
  2  RMSNorm fwd/bwd and RoPE fwd/bwd on 4 packed rows of U[128,512] tokens (hidden 1536)
  3  SwiGLU forward and in-place recompute-backward on [2048,8960] fp16
  4  fused LM head + cross-entropy, hidden [2048,1536], tied weight [151936,1536] fp16
Cold-cache protocol: each timed launch works on its own copy of the inputs, rotating through
enough copies to exceed 512 MiB (twice the 256 MiB Infinity Cache), so no launch finds its
inputs in the cache. A kernel's time is the HIP-event time of K back-to-back launches on the
launch stream divided by K. Achieved bandwidth / FLOP rate uses the ALGORITHMIC bytes / FLOPs of
one launch (inputs read once, outputs written once).

One JSON line is printed: the headline metric with its roofline and the CPU oracle timed on the
host cores (a baseline, not the target), plus every kernel's numbers under "kernels".
"""

import argparse
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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", default="")
    return p.parse_args()


def copies_for(nbytes, cap=64):
    return max(2, min(cap, -(-COLD_BYTES // max(nbytes, 1)) + 1))


class Kernel:
    """A benchmarked launch: `make(i)` returns the i-th independent launch closure."""

    def __init__(self, name, config, bound, work, make, n_copies, step=True):
        self.name, self.config, self.bound, self.work = name, config, bound, work
        self.make, self.n_copies, self.step = make, n_copies, step


def bound(name, *args):
    """A launch closure of entry point `name` with its arguments converted once."""
    from claudemaxing_amd import _lib

    fn = getattr(_lib.load(), name)
    conv = tuple(a for a in args)

    def launch():
        rc = fn(*conv)
        if rc:
            raise RuntimeError(f"{name} failed with code {rc}")

    return launch


def build_kernels(dev, only):
    import torch

    from claudemaxing_amd import lora, nf4, rmsnorm, rope, swiglu_recompute
    from claudemaxing_amd import _lib
    from oracle import inputs

    kernels = []
    s = lambda: _lib.stream(dev)  # noqa: E731

    def want(name):
        return not only or name in only

    # ---- config 1: NF4 dequant ---------------------------------------------------------
    if want("nf4_dequant"):
        w = inputs.nf4_weight(0)
        packed, state = nf4.quantize_nf4(w, 64, True)
        n = w.numel()
        nbytes = n // 2 + state.absmax.numel() + state.state2.absmax.numel() * 4 + 256 * 4 + \
            16 * 4 + 4 + n * 2
        k = copies_for(nbytes)
        sets = [(packed.to(dev), state.to(dev), torch.empty(w.shape, dtype=torch.float16,
                                                             device=dev)) for _ in range(k)]

        def make(i, sets=sets):
            p, st, out = sets[i % len(sets)]
            s2 = st.state2
            return bound("cm_nf4_dequant", p.data_ptr(), st.absmax.data_ptr(), 1,
                         st.code.data_ptr(), s2.code.data_ptr(), s2.absmax.data_ptr(),
                         st.offset.data_ptr(), out.data_ptr(), _lib.F16, n // 2, 64, 256, s())

        kernels.append(Kernel("nf4_dequant", "[8960,1536] nf4->fp16", "hbm", nbytes, make, k))

    # ---- config 2: RMSNorm / RoPE ------------------------------------------------------
    c2 = inputs.rmsnorm_rope(0)
    N, H = c2["n"], 1536
    if want("rmsnorm_fwd") or want("rmsnorm_bwd"):
        x = c2["x"]
        w16 = c2["w"].to(torch.float16)
        fwd_bytes = 2 * N * H + 2 * N * H + 4 * N + 2 * H  # x in, out fp16, rstd, w
        bwd_bytes = 2 * N * H * 3 + 4 * N + 2 * H  # dy, x in, dx out, rstd, w
        k = copies_for(fwd_bytes + bwd_bytes)
        sets = []
        for _ in range(k):
            xd = x.to(dev)
            out = torch.empty(N, H, dtype=torch.float16, device=dev)
            rstd = torch.empty(N, dtype=torch.float32, device=dev)
            dy = c2["dy"].to(torch.float16).to(dev)
            dx = torch.empty(N, H, dtype=torch.float16, device=dev)
            sets.append((xd, w16.to(dev), out, rstd, dy, dx))

        def make_f(i, sets=sets):
            xd, wd, out, rstd, _, _ = sets[i % len(sets)]
            return bound("cm_rmsnorm_fwd", xd.data_ptr(), _lib.F16, H, wd.data_ptr(), _lib.F16,
                         out.data_ptr(), _lib.F16, rstd.data_ptr(), None, None, None, 1, N, H,
                         1e-6, s())

        def make_b(i, sets=sets):
            xd, wd, _, rstd, dy, dx = sets[i % len(sets)]
            return bound("cm_rmsnorm_bwd", dy.data_ptr(), _lib.F16, xd.data_ptr(), _lib.F16,
                         wd.data_ptr(), _lib.F16, rstd.data_ptr(), dx.data_ptr(), _lib.F16, None,
                         None, None, 1, 0, N, H, s())

        # prime rstd of every copy so backward reads real values
        for i in range(k):
            make_f(i)()
        if want("rmsnorm_fwd"):
            kernels.append(Kernel("rmsnorm_fwd", f"N={N} H=1536 fp16", "hbm", fwd_bytes, make_f, k))
        if want("rmsnorm_bwd"):
            kernels.append(Kernel("rmsnorm_bwd", f"N={N} H=1536 fp16", "hbm", bwd_bytes, make_b, k))
    if want("rope_fwd") or want("rope_bwd"):
        from oracle import rope as orope

        cos, sin = orope.cos_sin(c2["pos"], 128, c2["theta"], torch.float16)
        rope_bytes = 2 * 2 * N * 14 * 128 + 2 * 2 * N * 128  # q,k in+out fp16; cos+sin
        k = copies_for(rope_bytes)
        sets = []
        for _ in range(k):
            qp = c2["q"].transpose(1, 2).contiguous().to(dev).transpose(1, 2)
            kp = c2["k"].transpose(1, 2).contiguous().to(dev).transpose(1, 2)
            sets.append((qp, kp, cos.to(dev), sin.to(dev)))

        def make_r(i, backward, sets=sets):
            q, kk, c, sn = sets[i % len(sets)]
            dt = torch.float16
            return lambda: rope._rotate_pair(q, kk, c, sn, dt, dt, backward)

        if want("rope_fwd"):
            kernels.append(Kernel("rope_fwd", f"N={N} 12+2 heads x 128", "hbm", rope_bytes,
                                  lambda i: make_r(i, False), k))
        if want("rope_bwd"):
            kernels.append(Kernel("rope_bwd", f"N={N} 12+2 heads x 128", "hbm", rope_bytes,
                                  lambda i: make_r(i, True), k))

    # ---- config 3: SwiGLU --------------------------------------------------------------
    if want("swiglu_fwd") or want("swiglu_bwd"):
        gate, up, dy = inputs.swiglu(0)
        n = gate.numel()
        k = copies_for(10 * n)
        sets = [(gate.to(dev), up.to(dev), dy.to(dev), torch.empty_like(gate, device=dev))
                for _ in range(k)]

        def make_sf(i, sets=sets):
            g, u, _, out = sets[i % len(sets)]
            return bound("cm_swiglu_fwd", g.data_ptr(), _lib.F16, u.data_ptr(), _lib.F16,
                         out.data_ptr(), _lib.F16, n, 1, s())

        def make_sb(i, sets=sets):
            g, u, d, _ = sets[i % len(sets)]
            return bound("cm_swiglu_bwd", d.data_ptr(), _lib.F16, g.data_ptr(), _lib.F16,
                         u.data_ptr(), _lib.F16, g.data_ptr(), u.data_ptr(), n, 1, 1, 1, s())

        if want("swiglu_fwd"):
            kernels.append(Kernel("swiglu_fwd", "[2048,8960] fp16", "hbm", 6 * n, make_sf, k))
        if want("swiglu_bwd"):
            kernels.append(Kernel("swiglu_bwd", "[2048,8960] fp16 in place", "hbm", 10 * n,
                                  make_sb, k))

    # ---- config 5 component: LoRA mask pack/unpack at the q/v input shape -----------------
    if want("lora_pack") or want("lora_unpack"):
        n = 1152 * 1536
        g = torch.Generator().manual_seed(0)
        x = torch.randn(n, generator=g)
        keep = torch.rand(n, generator=g) > 0.05
        k = copies_for(18 * n)
        sets = []
        for _ in range(k):
            sets.append((x.to(dev), keep.to(dev), torch.empty(n, dtype=torch.float16, device=dev),
                         torch.empty(n // 8, dtype=torch.uint8, device=dev),
                         torch.randn(n, device=dev).half(), torch.empty(n, device=dev),
                         torch.empty(n, dtype=torch.float16, device=dev)))
        scale = 1 / 0.95

        def make_p(i, sets=sets):
            xx, kk, xd, bits, _, _, _ = sets[i % len(sets)]
            return bound("cm_lora_pack", xx.data_ptr(), _lib.F32, kk.data_ptr(), xd.data_ptr(),
                         bits.data_ptr(), n, scale, s())

        def make_u(i, sets=sets):
            xx, kk, xd, bits, g16, dx, xd2 = sets[i % len(sets)]
            return bound("cm_lora_unpack", xd.data_ptr(), bits.data_ptr(), g16.data_ptr(),
                         xd2.data_ptr(), dx.data_ptr(), _lib.F32, n, scale, s())

        for i in range(k):
            make_p(i)()
        if want("lora_pack"):
            kernels.append(Kernel("lora_pack", "[1152,1536] fp32 x", "hbm", 7 * n + n // 8,
                                  make_p, k))
        if want("lora_unpack"):
            kernels.append(Kernel("lora_unpack", "[1152,1536] -> fp32 dx", "hbm",
                                  10 * n + n // 8, make_u, k))

    # ---- practical HBM ceiling: torch's device copy of the config-3 gate tensor -----------
    if want("hbm_copy_ref"):
        n = 2048 * 8960
        k = copies_for(4 * n)
        sets = [(torch.randn(n, device=dev).half(), torch.empty(n, dtype=torch.float16,
                                                                 device=dev)) for _ in range(k)]

        def make_c(i, sets=sets):
            a, b = sets[i % len(sets)]
            return lambda: b.copy_(a)

        kernels.append(Kernel("hbm_copy_ref", "fp16 [2048,8960] device copy (torch)", "hbm",
                              4 * n, make_c, k, step=False))

    # ---- bandwidth-scale shapes of the row kernels (32768 tokens) -------------------------
    if want("rmsnorm_fwd_bw") or want("rope_fwd_bw"):
        nb = 32768
        xb = torch.randn(nb, H, device=dev).half()
        wb = torch.rand(H, device=dev).half() + 0.5
        outs = [torch.empty(nb, H, dtype=torch.float16, device=dev) for _ in range(2)]
        rstd_b = torch.empty(nb, dtype=torch.float32, device=dev)
        fb = 4 * nb * H + 4 * nb + 2 * H
        kernels.append(Kernel(
            "rmsnorm_fwd_bw", f"N={nb} H=1536 fp16", "hbm", fb,
            lambda i: (lambda o=outs[i % 2]: _lib.call(
                "cm_rmsnorm_fwd", xb.data_ptr(), _lib.F16, H, wb.data_ptr(), _lib.F16,
                o.data_ptr(), _lib.F16, rstd_b.data_ptr(), None, None, None, 1, nb, H, 1e-6,
                s())), 2, step=False))
        from oracle import rope as orope

        qb = torch.randn(1, nb, 12 * 128, device=dev).half().view(1, nb, 12, 128).transpose(1, 2)
        kb = torch.randn(1, nb, 2 * 128, device=dev).half().view(1, nb, 2, 128).transpose(1, 2)
        cb, sb = orope.cos_sin(torch.arange(nb) % 512, 128, 1e6, torch.float16)
        cb, sb = cb.to(dev), sb.to(dev)
        rb = 2 * 2 * nb * 14 * 128 + 2 * 2 * nb * 128
        kernels.append(Kernel(
            "rope_fwd_bw", f"N={nb} 12+2 heads x 128", "hbm", rb,
            lambda i: (lambda: rope._rotate_pair(qb, kb, cb, sb, torch.float16, torch.float16,
                                                 False)), 1, step=False))

    # ---- config 4: fused LM head ----------------------------------------------------------
    if want("lmhead_ce") and os.environ.get("CM_BENCH_LMHEAD", "1") != "0":
        from claudemaxing_amd import lm_head_loss

        h, w, t = inputs.lm_head(0)
        hd, wd, td = h.to(dev), w.to(dev), t.to(dev)
        flops = 4 * h.shape[0] * w.shape[0] * h.shape[1]

        w16, wt16 = lm_head_loss._fp16_weights(wd, True)  # the host's cached W^T, as in training

        def make_l(i):
            return lambda: lm_head_loss._fused_rows(hd, w16, td, True, None, wt16)

        try:
            make_l(0)()
            torch.cuda.synchronize()
            kernels.append(Kernel("lmhead_ce", "N=2048 V=151936 H=1536 fp16", "mfma", flops,
                                  make_l, 1))
        except RuntimeError as e:
            print(f"[bench] lmhead_ce unavailable: {e}", file=sys.stderr, flush=True)
    return kernels


def time_kernel(kern, steps, warmup):
    """Milliseconds per launch: `steps` launches (each on its own input copy, rotating) issued
    back to back between two HIP events recorded on the launch stream (torch's current stream,
    which every entry point is given). The launch closures hold pre-bound arguments, so for the
    microsecond kernels the host issue rate stays close to the device rate; the rocprofv3
    kernel trace of the same command gives the device-only durations."""
    import torch

    launches = [kern.make(i) for i in range(steps)]
    for i in range(warmup):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for f in launches:
        f()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


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
        rows = 64  # 64 of the 2048 rows, full vocabulary
        t0 = time.perf_counter()
        olm.head(h[:rows], w, t[:rows], want_grad=True, rows_per_block=64)
        dt = time.perf_counter() - t0
        flops = 4 * rows * w.shape[0] * w.shape[1]
        return dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                    sample=f"oracle.lm_head.head on {rows} of 2048 rows, full vocab, torch CPU "
                           f"fp32 ({dt:.1f} s)")
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
    return dict(value=nbytes / dt / 1e9, unit="GB/s", cores=1, kind="port",
                sample=f"oracle.nf4.dequant (numpy, 1 thread) of the full config-1 weight, "
                       f"median of 3 ({dt * 1e3:.0f} ms)")


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this kernel set has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    only = set(filter(None, args.only.split(",")))
    kernels = build_kernels(dev, only)
    results = {}
    for kern in kernels:
        print(f"[bench] {kern.name} ...", file=sys.stderr, flush=True)
        ms = time_kernel(kern, args.steps, args.warmup)
        if kern.bound == "hbm":
            achieved, peak, unit = kern.work / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            achieved, peak, unit = kern.work / (ms * 1e-3) / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s"
        results[kern.name] = dict(config=kern.config, us=round(ms * 1e3, 2),
                                  achieved=round(achieved, 1), unit=unit, bound=kern.bound,
                                  frac=round(achieved / peak, 4), work=kern.work,
                                  in_step=kern.step)
        print(f"[bench] {kern.name}: {ms * 1e3:.2f} us, {achieved:.1f} {unit} "
              f"({100 * achieved / peak:.1f}% of peak)", file=sys.stderr, flush=True)
    headline = "lmhead_ce" if "lmhead_ce" in results else "nf4_dequant"
    if headline not in results:
        headline = next(iter(results))
    hr = results[headline]
    line = {
        "metric": "kernel HBM GB/s & LM-head-CE TFLOP/s (% of roofline); QLoRA step ms",
        "value": hr["achieved"],
        "unit": hr["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sum(r["us"] for r in results.values() if r["in_step"]) / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if headline == "lmhead_ce" else "u8->fp16",
        "data": "synthetic (seeded CPU draws of BASELINE.json configs, copied to HBM)",
        "config": {"workload": headline, "shape": hr["config"], "parallelism": "none (1 GPU)",
                   "cold_cache": "input copies rotated beyond 512 MiB"},
        "roofline": {"bound": hr["bound"], "achieved": hr["achieved"],
                     "peak": HBM_PEAK_GBS if hr["bound"] == "hbm" else MFMA_FP16_PEAK_TFLOPS,
                     "unit": hr["unit"], "frac": hr["frac"], "traffic": None},
        "kernels": results,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(headline)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
