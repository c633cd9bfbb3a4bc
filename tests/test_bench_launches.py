"""Every launch bench.py issues stays inside the tensors it was built from.

bench.py binds C-ABI calls (raw pointers and element counts) ahead of time. This test builds
the same launch closures with CPU tensors, intercepts the bound arguments instead of calling the
library, and checks, entry point by entry point, that every byte range the kernel would touch
(from the counts, strides and block sizes passed) lies inside one of the tensors kept alive
with that launch. No GPU is used.
"""

import math

import pytest
import torch

import bench

NBYTES = {0: 4, 1: 2, 2: 2, 3: 1, 4: 4, 5: 8}  # cm_dtype -> element size


def ranges(args_by_name):
    """[(ptr, nbytes, what)] the entry point reads or writes, from its bound arguments."""
    name, a = args_by_name
    out = []
    if name == "cm_nf4_dequant":
        packed, absmax, nested, code, code2, absmax2, offset, dst, odt, nb, bs, bs2, _ = a
        n_blk = math.ceil(2 * nb / bs)
        out += [(packed, nb, "packed"), (absmax, n_blk * (1 if nested else 4), "absmax"),
                (code, 64, "code"), (dst, 2 * nb * NBYTES[odt], "out")]
        if nested:
            out += [(code2, 1024, "code2"), (absmax2, 4 * math.ceil(n_blk / bs2), "absmax2"),
                    (offset, 4, "offset")]
    elif name == "cm_rmsnorm_fwd":
        x, xdt, stride, w, wdt, o, odt, rstd, low, slot, small, n_small, rows, cols, _, _ = a
        out += [(x, ((rows - 1) * stride + cols) * NBYTES[xdt], "x"), (w, cols * NBYTES[wdt], "w"),
                (o, rows * cols * NBYTES[odt], "out"), (rstd, 4 * rows, "rstd")]
        if low:
            out += [(low, rows * cols * 2, "low16")]
            if n_small:
                out += [(small, rows * n_small * 2, "small16"), (slot, 4 * cols, "slot")]
    elif name == "cm_rmsnorm_bwd":
        dy, dydt, xs, xsdt, w, wdt, rstd, dx, dxdt, dwp, slot, small, n_small, saved, rows, cols, \
            _ = a
        out += [(dy, rows * cols * NBYTES[dydt], "dy"), (xs, rows * cols * NBYTES[xsdt], "xs"),
                (w, cols * NBYTES[wdt], "w"), (rstd, 4 * rows, "rstd"),
                (dx, rows * cols * NBYTES[dxdt], "dx")]
        if saved and n_small:
            out += [(small, rows * n_small * 2, "small16"), (slot, 4 * cols, "slot")]
    elif name == "cm_rope":
        (x0, d0, sb0, sh0, st0, h0, o0, od0, x1, d1, sb1, sh1, st1, h1, o1, od1, cos, sin, cdt,
         csb, cst, b, t, d, _, _) = a
        for x, dt, sb, sh, st, h, o, od, nm in ((x0, d0, sb0, sh0, st0, h0, o0, od0, "q"),
                                                (x1, d1, sb1, sh1, st1, h1, o1, od1, "k")):
            if h:
                last = (b - 1) * sb + (h - 1) * sh + (t - 1) * st + d
                out += [(x, last * NBYTES[dt], nm), (o, b * h * t * d * NBYTES[od], nm + " out")]
        last_cs = (b - 1) * csb + (t - 1) * cst + d
        out += [(cos, last_cs * NBYTES[cdt], "cos"), (sin, last_cs * NBYTES[cdt], "sin")]
    elif name == "cm_swiglu_fwd":
        g, gdt, u, udt, o, odt, n, _, _ = a
        out += [(g, n * NBYTES[gdt], "gate"), (u, n * NBYTES[udt], "up"),
                (o, n * NBYTES[odt], "out")]
    elif name == "cm_swiglu_bwd":
        dy, dydt, g, gdt, u, udt, dg, du, n, _, _, _, _ = a
        out += [(dy, n * NBYTES[dydt], "dy"), (g, n * NBYTES[gdt], "gate"),
                (u, n * NBYTES[udt], "up"), (dg, n * NBYTES[gdt], "dgate"),
                (du, n * NBYTES[udt], "dup")]
    elif name == "cm_lora_pack":
        x, xdt, keep, xd, bits, n, _, _ = a
        out += [(x, n * NBYTES[xdt], "x"), (keep, n, "keep"), (xd, 2 * n, "xd"),
                (bits, n // 8, "bits")]
    elif name == "cm_lora_unpack":
        x16, bits, g16, xd, dx, dxdt, n, _, _ = a
        out += [(x16, 2 * n, "x16"), (bits, n // 8, "bits"), (g16, 2 * n, "g16"),
                (xd, 2 * n, "xd"), (dx, n * NBYTES[dxdt], "dx")]
    elif name in ("cm_nf4_linear_fwd", "cm_nf4_linear_bwd"):
        if name == "cm_nf4_linear_fwd":
            x, ldx, m, w, n_w, bias, outs, ldo, odt, ws, ws_bytes, _ = a
        else:
            gs, ldg, m, w, n_w, dx, lddx, odt, ws, ws_bytes, _ = a
        for i in range(n_w):
            wi = w[i]
            n_el = wi.rows * wi.cols
            n_blk = n_el // wi.blocksize
            out += [(wi.packed, n_el // 2, "packed"), (wi.absmax, n_blk, "absmax"),
                    (wi.code, 64, "code"), (wi.code2, 1024, "code2"),
                    (wi.absmax2, 4 * math.ceil(n_blk / wi.blocksize2), "absmax2"),
                    (wi.offset, 4, "offset")]
            if name == "cm_nf4_linear_fwd":
                out.append((outs[i], ((m - 1) * ldo[i] + wi.rows) * NBYTES[odt], "out"))
            else:
                out.append((gs[i], ((m - 1) * ldg[i] + wi.rows) * 2, "g"))
        if name == "cm_nf4_linear_fwd":
            out.append((x, ((m - 1) * ldx + w[0].cols) * 2, "x"))
        else:
            out.append((dx, ((m - 1) * lddx + w[0].cols) * NBYTES[odt], "dx"))
        if ws:
            out.append((ws, ws_bytes, "workspace"))
    else:
        raise AssertionError(f"no range rule for {name}")
    return out


def storages(obj, acc):
    if isinstance(obj, torch.Tensor):
        acc.append((obj.untyped_storage().data_ptr(), obj.untyped_storage().nbytes()))
    elif isinstance(obj, (tuple, list)):
        for o in obj:
            storages(o, acc)
    elif hasattr(obj, "__dict__"):  # QuantState
        storages(list(vars(obj).values()), acc)
    return acc


@pytest.fixture
def recorded(monkeypatch):
    calls = []

    def fake_bound(name, *args):
        record = (name, args)

        def launch():
            calls.append(record)

        launch.record = record
        return launch

    monkeypatch.setattr(bench, "bound", fake_bound)
    monkeypatch.setattr(bench, "_stream", lambda dev: None)
    return calls


def test_every_bench_launch_stays_inside_its_tensors(recorded):
    dev = torch.device("cpu")
    # the device copy and the launch floors pass no tensors to check
    names = set(bench.ALL) - {"lmhead_ce", "hbm_copy_ref"} - bench.FLOORS
    kernels = bench.build_kernels(dev, sorted(names))
    # "_unfused", "_split" and "_merged" lines time torch-level paths beside a C-ABI entry
    side = ("_unfused", "_split", "_merged")
    assert {k.name for k in kernels if not k.name.endswith(side)} == names
    checked = 0
    for kern in kernels:
        for fn, keep in kern.launches:
            if not hasattr(fn, "record"):  # a torch reference path, not a C-ABI launch
                assert kern.name.endswith(side), kern.name
                continue
            owned = storages(keep, [])
            for ptr, nbytes, what in ranges(fn.record):
                if ptr is None or nbytes <= 0:
                    continue
                assert any(s <= ptr and ptr + nbytes <= s + n for s, n in owned), \
                    f"{kern.name}: {what} [{ptr:#x}, +{nbytes}) is outside its tensors"
                checked += 1
    assert checked > 100
