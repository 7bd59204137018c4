#!/usr/bin/env python3
"""Benchmark of the dynamic short-convolution hot path on one MI355X.

Metric: fwd+bwd ms & HBM GB/s (% peak), B4 T4096 D2048 W4
bf16, headwise + lowrank.

A step is one forward+backward, through the public autograd API, of each of
the three B4 T4096 D2048 W4 bf16 configurations of BASELINE.json:
    hw_hs1   headwise, head_size 1 (H 2048), static_w, residual   (configs[1])
    hw_hs32  headwise, head_size 32 (H 64), static_w, residual    (configs[2])
    lr_r16   lowrank, R 16, no static_w, residual                  (configs[3])
The three forwards run first, then the three backwards in one autograd call,
as a training step's loss.backward() would run them.
`value` = algorithmic bytes of one step (each input read once, each output
written once, at bf16) x steps / timed seconds, in GB/s.  Inputs are
synthetic (BASELINE.json distributions, CPU generator seed 0) and resident in
HBM before timing.

Also reported:
  breakdown    per configuration and direction, the average C-ABI launch
               sequence: back-to-back launches rotating over enough
               independent input sets that each launch's data is out of the
               256 MB MALL, between one pair of HIP events (every set
               launched once before; the median of three such averages); plus configs[4]
               (lowrank QKV) at its own shape, as 3 calls and as one grouped
               call reading x out of the fused [B, T, 3D] projection, the fp32
               tier, the reference bench.py's own shapes (ref_*: head
               sizes 1, 4, 16 and rank 16, no static_w, no residual), lowrank
               W 16, W 20 and W 12 at rank 40, kernel ranks 64 and 128 (passes of
               ranks) and headwise W 12 and W 24 on their wide kernels;
  qkv          configs[4] end to end through autograd (forward + backward):
               the README's pattern (split the fused projection, .contiguous()
               each slice, three calls; autograd concatenates dq, dk, dv)
               against the grouped operator;
  roofline     the dominant kernel (headwise hs1 backward, hw_bwd_fast, and
               its reduce_partials launch) against 8 TB/s.  Live: HIP events
               that the backward node's autograd pre- and post-hooks record
               around the launch, on the stream it runs on, in as many steps
               again right after the timed ones (an event record holds the GPU
               for ~5 us, so the timed steps carry no per-step events).  From
               profiles/roofline_trace.json (rocprofv3 kernel trace of this
               command): the kernel alone and kernel start to reduce end,
               reported beside the live figure (trace_* fields); `achieved`
               and `frac` always come from this run's live events;
  cpu_baseline the CPU oracle (fp32 restatement of reference.py) on configs[0]
               on this host's cores.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
    python bench.py --calibrate-copy   # a plain 256 MiB device copy, for scaling HBM counters
    python bench.py --calibrate-read   # a read-only pass over 256 MiB (a sum), the same for reads alone
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dynamic-conv1d_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd+bwd ms & HBM GB/s (% peak), B4 T4096 D2048 W4 bf16, headwise+lowrank"
PEAK_GBS = 8000.0  # MI355X HBM3E
BF16 = 2
# element size and C-ABI dtype code of a config's "dtype" (bf16 unless stated)
DTYPES = {"bf16": (2, 0), "fp16": (2, 1), "fp32": (4, 2)}


def esize(c):
    return DTYPES[c.get("dtype", "bf16")][0]


def dcode(c):
    return DTYPES[c.get("dtype", "bf16")][1]

CONFIGS = {
    "hw_hs1": dict(kind="hw", B=4, T=4096, D=2048, H=2048, W=4, static=True, residual=True),
    "hw_hs32": dict(kind="hw", B=4, T=4096, D=2048, H=64, W=4, static=True, residual=True),
    "lr_r16": dict(kind="lr", B=4, T=4096, D=2048, R=16, W=4, static=False, residual=True),
}
EXTRA = {
    # BASELINE configs[0], the CPU baseline's own workload, on the GPU (fp32, loss y.sum() in the baseline)
    "cfg0_hw_fp32": dict(kind="hw", B=2, T=1024, D=512, H=512, W=4, static=False, residual=False, dtype="fp32"),
    "lr_qkv": dict(kind="lr", B=2, T=8192, D=4096, R=31, W=4, static=True, residual=True, calls=3),
    "lr_qkv_grouped": dict(kind="lrg", B=2, T=8192, D=4096, R=31, W=4, static=True, residual=True, G=3,
                           head_dim=128),
    # the same grouped q|k|v op on one sequence of 32768 tokens (x spans 768 MiB): per-run buffer
    # resources keep it on the matrix-core kernels; per-token time against lr_qkv_grouped's 16384 tokens
    "lr_qkv_grouped_T32k": dict(kind="lrg", B=1, T=32768, D=4096, R=31, W=4, static=True, residual=True, G=3),
    # configs[4]'s shape at W 8 (two rank chunks): the backward runs as two passes of 4 taps
    "lr_qkv_W8": dict(kind="lr", B=2, T=8192, D=4096, R=31, W=8, static=True, residual=True),
    # the fp32 tier (reference test.py's 1e-5 cases) at the B4 shapes
    "hw_hs32_fp32": dict(kind="hw", B=4, T=4096, D=2048, H=64, W=4, static=True, residual=True, dtype="fp32"),
    "lr_r16_fp32": dict(kind="lr", B=4, T=4096, D=2048, R=16, W=4, static=False, residual=True, dtype="fp32"),
    # W 16 at rank 16: the forward in one pass over the taps, the backward as two passes of 8 taps
    "lr_W16": dict(kind="lr", B=4, T=4096, D=2048, R=16, W=16, static=False, residual=True),
    # headwise above W 8: the wide row-ring kernels (head sizes 1 and 32, static filter, residual)
    "hw_W12_hs1": dict(kind="hw", B=4, T=4096, D=2048, H=2048, W=12, static=True, residual=True),
    "hw_W12_hs32": dict(kind="hw", B=4, T=4096, D=2048, H=64, W=12, static=True, residual=True),
    # above W 16 the wide kernels keep one channel per lane
    "hw_W24_hs32": dict(kind="hw", B=4, T=4096, D=2048, H=64, W=24, static=True, residual=True),
    # head size 8 at W 24 on the head matrix-core kernels (two heads per 16-channel block)
    "hw_W24_hs8": dict(kind="hw", B=4, T=4096, D=2048, H=256, W=24, static=True, residual=True),
    # W 20: the forward in one pass over the taps, the backward as three passes (7 + 7 + 6)
    "lr_W20": dict(kind="lr", B=4, T=4096, D=2048, R=16, W=20, static=False, residual=True),
    # W 12 at kernel rank 40 (three rank chunks): the forward as passes of 4 + 8 taps, the backward as
    # two passes of 32 + 8 ranks x three of 4 taps
    "lr_W12_r40": dict(kind="lr", B=4, T=4096, D=2048, R=40, W=12, static=False, residual=True),
    # kernel rank 128 (R 127 + static): the forward in one pass of 128 ranks, the backward as four
    # passes of 32 for dz / dU and one launch for dx (the generic kernels took 1.9 + 15.0 ms here), and
    # kernel rank 32 at the same shape for its bytes per microsecond
    "lr_r128": dict(kind="lr", B=4, T=4096, D=2048, R=127, W=4, static=True, residual=True),
    "lr_r32_b4": dict(kind="lr", B=4, T=4096, D=2048, R=31, W=4, static=True, residual=True),
    # kernel rank 64 (R 63 + static): the forward in one pass of four rank chunks, the backward as
    # two passes of 32 ranks (four passes of one tap each before: 327 us)
    "lr_r64_b4": dict(kind="lr", B=4, T=4096, D=2048, R=63, W=4, static=True, residual=True),
    # the reference bench.py's own shapes (bench.py:7-12): head sizes 1, 4, 16 and rank 16, no static_w, no residual
    "ref_hw_hs1": dict(kind="hw", B=4, T=4096, D=2048, H=2048, W=4, static=False, residual=False),
    "ref_hw_hs4": dict(kind="hw", B=4, T=4096, D=2048, H=512, W=4, static=False, residual=False),
    "ref_hw_hs16": dict(kind="hw", B=4, T=4096, D=2048, H=128, W=4, static=False, residual=False),
    "ref_lr_r16": dict(kind="lr", B=4, T=4096, D=2048, R=16, W=4, static=False, residual=False),
}
STEP = ["hw_hs1", "hw_hs32", "lr_r16"]


def alg_bytes(c):
    """Algorithmic bytes (fwd, bwd) of one call: inputs read once, outputs written once."""
    if c["kind"] == "lrg":
        f, b = alg_bytes(dict(c, kind="lr"))
        return c["G"] * f, c["G"] * b
    e = esize(c)
    x = c["B"] * c["T"] * c["D"] * e
    sw = c["W"] * c["D"] * e if c["static"] else 0
    if c["kind"] == "hw":
        w = c["B"] * c["T"] * c["H"] * c["W"] * e
        return 2 * x + w + sw, 3 * x + 2 * w + 2 * sw
    z = c["B"] * c["T"] * c["R"] * e
    U = c["R"] * c["W"] * c["D"] * e
    return 2 * x + z + U + sw, 3 * x + 2 * z + 2 * U + 2 * sw


def make_inputs(c, torch, dev, seed=0):
    """BASELINE.json inputs: CPU generator, fp32 draw, cast to bf16, copy to the GPU."""
    g = torch.Generator().manual_seed(seed)
    B, T, D, W = c["B"], c["T"], c["D"], c["W"]
    x = torch.randn(B, T, D, generator=g)
    if c["kind"] == "hw":
        mid = [torch.randn(B, T, c["H"], W, generator=g) / math.sqrt(W)]
    else:
        R = c["R"]
        rk = R + (1 if c["static"] else 0)
        mid = [torch.randn(B, T, R, generator=g), torch.randn(R, W * D, generator=g) / math.sqrt(rk * W)]
    sw = (torch.rand(W, D, generator=g) * 2 - 1) / math.sqrt(W) if c["static"] else None
    dy = torch.randn(B, T, D, generator=g)
    bf = torch.bfloat16
    args = [t.to(bf).to(dev).requires_grad_() for t in [x] + mid]
    args.append(sw.to(bf).to(dev).requires_grad_() if sw is not None else None)
    return args, dy.to(bf).to(dev)


def cpu_baseline(torch):
    """reference.py's CPU path (the oracle's fp32 restatement) on configs[0]."""
    from oracle.reference_cpu import headwise_dynamic_convolution_ref as hw_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, T, D, H, W = 2, 1024, 512, 512, 4
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, T, D, generator=g)
    w = torch.randn(B, T, H, W, generator=g) / math.sqrt(W)

    def once():
        xs, ws = x.clone().requires_grad_(), w.clone().requires_grad_()
        hw_ref(xs, ws).sum().backward()

    for _ in range(2):
        once()
    times = []
    t_end = time.perf_counter() + 10.0
    while len(times) < 10 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    nbytes = 4 * (2 * B * T * D + B * T * H * W) + 4 * (3 * B * T * D + 2 * B * T * H * W)  # fp32 fwd + bwd
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"configs[0]: headwise fp32 B2 T1024 D512 H512 W4, no static, no residual, fwd+bwd of y.sum(); "
                   f"median of {len(times)} runs = {med * 1e3:.2f} ms on {cores} threads; {nbytes / 1e6:.1f} MB algorithmic"),
    }


MALL_BYTES = 256 << 20


def measured_traffic(kernel_key):
    """HBM bytes per dispatch of a kernel from the committed rocprofv3 counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            kernels = json.load(f)["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    for name, t in kernels.items():
        if kernel_key in name:
            return round(t["read_bytes"] + t["write_bytes"])
    return None


def n_sets(c):
    """Independent input/output sets to rotate so each launch finds its data out of the 256 MB MALL."""
    fb, _ = alg_bytes(c)
    return max(2, math.ceil(4 * MALL_BYTES / fb))


def abi_sets(c, torch, dev):
    """`n_sets(c)` sets of inputs (device-generated, BASELINE scales, the config's dtype) with outputs."""
    from dynconv import _capi

    lib = _capi.load()
    B, T, D, W = c["B"], c["T"], c["D"], c["W"]
    bf = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[c.get("dtype", "bf16")]
    dt = dcode(c)
    sets = []
    if c["kind"] == "lrg":
        G, R = c["G"], c["R"]
        rk = R + (1 if c["static"] else 0)
        for _ in range(n_sets(c)):
            d = {"x": torch.randn(B, T, G * D, device=dev).to(bf)}
            d["zs"] = [torch.randn(B, T, R, device=dev).to(bf) for _ in range(G)]
            d["Us"] = [(torch.randn(R, W * D, device=dev) / math.sqrt(rk * W)).to(bf) for _ in range(G)]
            d["sws"] = ([((torch.rand(W, D, device=dev) * 2 - 1) / math.sqrt(W)).to(bf) for _ in range(G)]
                        if c["static"] else None)
            d["ys"] = [torch.empty(B, T, D, device=dev, dtype=bf) for _ in range(G)]
            d["dys"] = [torch.randn(B, T, D, device=dev).to(bf) for _ in range(G)]
            d["dx"] = torch.empty_like(d["x"])
            d["dzs"] = [torch.empty_like(z) for z in d["zs"]]
            d["dUs"] = [torch.empty_like(u) for u in d["Us"]]
            d["dsws"] = [torch.empty_like(s) for s in d["sws"]] if c["static"] else None
            d["nws"] = lib.dc_lowrank_bwd_grouped_ws_bytes(G, B, T, D, R, W, dt, int(c["static"]))
            # the forward's padded z copy for the backward, as the autograd Function keeps it
            nz = lib.dc_lowrank_zeff_bytes(B, T, D, R, W, dt, int(c["static"]))
            d["zeffs"] = [torch.empty(nz, dtype=torch.uint8, device=dev) for _ in range(G)] if nz > 0 else None
            d["nzeff"] = max(nz, 0)
            d["ws"] = torch.empty(max(d["nws"], 1), dtype=torch.uint8, device=dev)
            sets.append(d)
        return sets
    for _ in range(n_sets(c)):
        d = {"x": torch.randn(B, T, D, device=dev).to(bf), "dy": torch.randn(B, T, D, device=dev).to(bf)}
        d["sw"] = ((torch.rand(W, D, device=dev) * 2 - 1) / math.sqrt(W)).to(bf) if c["static"] else None
        if c["kind"] == "hw":
            d["w"] = (torch.randn(B, T, c["H"], W, device=dev) / math.sqrt(W)).to(bf)
            d["dw"] = torch.empty_like(d["w"])
            nws = lib.dc_headwise_bwd_ws_bytes(B, T, D, c["H"], W, dt, int(c["static"]))
        else:
            rk = c["R"] + (1 if c["static"] else 0)
            d["z"] = torch.randn(B, T, c["R"], device=dev).to(bf)
            d["U"] = (torch.randn(c["R"], W * D, device=dev) / math.sqrt(rk * W)).to(bf)
            d["dz"], d["dU"] = torch.empty_like(d["z"]), torch.empty_like(d["U"])
            nws = lib.dc_lowrank_bwd_ws_bytes(B, T, D, c["R"], W, dt, int(c["static"]))
            nz = lib.dc_lowrank_zeff_bytes(B, T, D, c["R"], W, dt, int(c["static"]))
            d["zeff"] = torch.empty(nz, dtype=torch.uint8, device=dev) if nz > 0 else None
            d["nzeff"] = max(nz, 0)
        d["y"], d["dx"] = torch.empty_like(d["x"]), torch.empty_like(d["x"])
        d["dsw"] = torch.empty_like(d["sw"]) if c["static"] else None
        d["nws"] = nws
        d["ws"] = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
        sets.append(d)
    return sets


def abi_launchers(c, sets, torch):
    """Direct C-ABI forward / backward launches on set i (no autograd, no allocation)."""
    from dynconv import _capi

    lib = _capi.load()
    st = torch.cuda.current_stream().cuda_stream
    B, T, D, W = c["B"], c["T"], c["D"], c["W"]
    p = _capi.ptr
    res = int(c["residual"])
    dt = dcode(c)
    if c["kind"] == "lrg":
        G, R = c["G"], c["R"]
        pa = _capi.ptr_array

        def fwd(i):
            d = sets[i]
            _capi.check(lib.dc_lowrank_fwd_grouped(G, p(d["x"]), G * D, pa(d["zs"]), pa(d["Us"]), pa(d["sws"]),
                                                   pa(d["ys"]), pa(d["zeffs"]), d["nzeff"], 0, B, T, D, R, W, dt,
                                                   res, st),
                        "grouped fwd")

        def bwd(i):
            d = sets[i]
            _capi.check(lib.dc_lowrank_bwd_grouped(G, p(d["x"]), G * D, pa(d["zs"]), pa(d["Us"]), pa(d["sws"]),
                                                   pa(d["zeffs"]), d["nzeff"], pa(d["dys"]), 0, p(d["dx"]), G * D,
                                                   pa(d["dzs"]),
                                                   pa(d["dUs"]),
                                                   pa(d["dsws"]), p(d["ws"]), d["nws"], B, T, D, R, W, dt, res, st),
                        "grouped bwd")
        return fwd, bwd
    if c["kind"] == "hw":
        H = c["H"]

        def fwd(i):
            d = sets[i]
            _capi.check(lib.dc_headwise_fwd(p(d["x"]), p(d["w"]), p(d["sw"]), p(d["y"]), B, T, D, H, W, dt, res, st),
                        "fwd")

        def bwd(i):
            d = sets[i]
            _capi.check(lib.dc_headwise_bwd(p(d["x"]), p(d["w"]), p(d["sw"]), p(d["dy"]), p(d["dx"]), p(d["dw"]),
                                            p(d["dsw"]), p(d["ws"]), d["nws"], B, T, D, H, W, dt, res, st), "bwd")
    else:
        R = c["R"]

        def fwd(i):
            d = sets[i]
            _capi.check(lib.dc_lowrank_fwd(p(d["x"]), p(d["z"]), p(d["U"]), p(d["sw"]), p(d["y"]), p(d["zeff"]),
                                           d["nzeff"], B, T, D, R, W, dt, res, st), "fwd")

        def bwd(i):
            d = sets[i]
            _capi.check(lib.dc_lowrank_bwd(p(d["x"]), p(d["z"]), p(d["U"]), p(d["sw"]), p(d["zeff"]), d["nzeff"],
                                           p(d["dy"]), p(d["dx"]),
                                           p(d["dz"]), p(d["dU"]), p(d["dsw"]), p(d["ws"]), d["nws"],
                                           B, T, D, R, W, dt, res, st), "bwd")
    return fwd, bwd


def time_launches(torch, launch, nsets, reps, rounds=3):
    """Duration of one launch sequence: the median over `rounds` of the average of `reps`
    back-to-back launches rotating over `nsets` input sets, between one pair of HIP events on
    torch's current stream (the launch stream).  Every set is launched once first, so that no
    timed launch is the first to touch its freshly allocated outputs and workspace (a configs[4]
    backward call read 139 us that way against 130-132 us once warm)."""
    for i in range(nsets):
        launch(i)
    torch.cuda.synchronize()
    avg = []
    for _ in range(rounds):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(reps):
            launch(i % nsets)
        e.record()
        e.synchronize()
        avg.append(s.elapsed_time(e) * 1e3 / reps)  # us
    return statistics.median(avg)


def calibrate_copy(torch, dev, mib=256, reps=3):
    """Plain device copies of exactly `mib` MiB: what FETCH_SIZE / WRITE_SIZE read for known traffic."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "copies": reps}), flush=True)


def calibrate_read(torch, dev, mib=256, reps=3):
    """A read-only streaming pass over exactly `mib` MiB (a float32 sum: 4 bytes written): a second
    reference, besides the copy, for what FETCH_SIZE reads per byte fetched."""
    n = mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for _ in range(reps):
        out = src.sum()
    torch.cuda.synchronize()
    assert out.item() == n // 4
    print(json.dumps({"calibrate_read_bytes": n, "reads": reps}), flush=True)


def roofline_trace(kernel_key):
    """The committed rocprofv3 kernel-trace figures of the roofline launch, or None."""
    path = os.path.join(ROOT, "profiles", "roofline_trace.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t if kernel_key in t.get("kernel", "") else None


def qkv_end_to_end(torch, dev, reps=10):
    """configs[4] through autograd: the README's split / .contiguous() / three calls vs the grouped operator."""
    from lowrank import lowrank_dynamic_convolution as lr, lowrank_dynamic_convolution_grouped as lrg

    c = EXTRA["lr_qkv_grouped"]
    B, T, D, R, W, G = c["B"], c["T"], c["D"], c["R"], c["W"], c["G"]
    bf = torch.bfloat16
    qkv = torch.randn(B, T, G * D, device=dev).to(bf).requires_grad_()
    zs = [torch.randn(B, T, R, device=dev).to(bf).requires_grad_() for _ in range(G)]
    Us = [(torch.randn(R, W * D, device=dev) / math.sqrt((R + 1) * W)).to(bf).requires_grad_() for _ in range(G)]
    sws = [((torch.rand(W, D, device=dev) * 2 - 1) / math.sqrt(W)).to(bf).requires_grad_() for _ in range(G)]
    dys = [torch.randn(B, T, D, device=dev).to(bf) for _ in range(G)]

    def readme():
        outs = [lr(part.contiguous(), zs[g], Us[g], sws[g], residual=True)
                for g, part in enumerate(qkv.split(D, dim=-1))]
        torch.autograd.backward(outs, dys)

    def grouped():
        torch.autograd.backward(lrg(qkv, zs, Us, sws, residual=True), dys)

    # README.md:106-110 then reshapes q, k, v into heads for attention; contiguous
    # head-major copies against the grouped operator writing that layout itself.
    hd = c["head_dim"]
    H = D // hd
    dys_h = [d.view(B, T, H, hd).transpose(1, 2).contiguous() for d in dys]

    def readme_heads():
        outs = [lr(part.contiguous(), zs[g], Us[g], sws[g], residual=True).view(B, T, H, hd).transpose(1, 2)
                .contiguous() for g, part in enumerate(qkv.split(D, dim=-1))]
        torch.autograd.backward(outs, dys_h)

    def grouped_heads():
        torch.autograd.backward(lrg(qkv, zs, Us, sws, residual=True, head_dim=hd), dys_h)

    out = {}
    for name, fn in (("readme_split_contiguous_3_calls", readme), ("grouped", grouped),
                     ("readme_heads_contiguous", readme_heads), ("grouped_head_major", grouped_heads)):
        for t in [qkv] + zs + Us + sws:
            t.grad = None
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            for t in [qkv] + zs + Us + sws:
                t.grad = None
            fn()
        e.record()
        e.synchronize()
        out[name + "_us"] = round(s.elapsed_time(e) * 1e3 / reps, 1)
    fb, bb = alg_bytes(c)
    out["alg_MB"] = round((fb + bb) / 1e6, 1)
    out["speedup"] = round(out["readme_split_contiguous_3_calls_us"] / out["grouped_us"], 3)
    out["head_dim"] = hd
    out["speedup_heads"] = round(out["readme_heads_contiguous_us"] / out["grouped_head_major_us"], 3)
    print(f"[bench] qkv end to end (fwd+bwd, autograd): README pattern {out['readme_split_contiguous_3_calls_us']} us, "
          f"grouped {out['grouped_us']} us ({out['speedup']}x); with [B,H,T,{hd}] outputs: README + contiguous "
          f"{out['readme_heads_contiguous_us']} us, grouped head-major {out['grouped_head_major_us']} us "
          f"({out['speedup_heads']}x)", file=sys.stderr, flush=True)
    return out


def proj_in_gemm(torch, dev, reps=20):
    """The upstream proj_in GEMM of the grouped QKV module at configs[4] (README.md:67, 75): z = pre_z @ W_in^T
    for all three groups at once ([B*T, D] x [D, 3R]), and its backward (dW_in = dz^T pre_z, d pre_z = dz W_in):
    torch's GEMM (hipBLASLt, F.linear) against libdynconv.so's kernels (dc_proj_in_fwd / dc_proj_in_bwd), time per
    launch rotating over input sets that do not fit the MALL, and the bandwidth each reaches on its algorithmic
    bytes (the GEMMs are far below the bf16 ridge: 2*3R flop/byte)."""
    from dynconv.modules import _ProjInFn

    c = EXTRA["lr_qkv_grouped"]
    B, T, D, R, G = c["B"], c["T"], c["D"], c["R"], c["G"]
    bf = torch.bfloat16
    n = max(2, math.ceil(4 * MALL_BYTES / (B * T * D * 2)))
    pre = [torch.randn(B, T, D, device=dev).to(bf).requires_grad_() for _ in range(n)]
    win = (torch.randn(G * R, D, device=dev) / math.sqrt(D)).to(bf).requires_grad_()
    dz = [torch.randn(B, T, G * R, device=dev).to(bf) for _ in range(n)]
    dzs = [[d[..., g * R:(g + 1) * R].contiguous() for g in range(G)] for d in dz]
    F = torch.nn.functional
    e = 2
    f_bytes = (B * T * D + G * R * D + B * T * G * R) * e
    b_bytes = (B * T * G * R + B * T * D + G * R * D) * e + (G * R * D + B * T * D) * e  # reads dz, pre_z, W_in
    out = {"shape": f"[{B * T}, {D}] x [{D}, {G * R}] bf16", "alg_MB": round((f_bytes + b_bytes) / 1e6, 1)}
    for name in ("torch_F.linear", "dynconv"):
        if name == "dynconv":
            zs = [_ProjInFn.apply(p, win, G, R) for p in pre]
            grads = dzs

            def fwd(i):
                _ProjInFn.apply(pre[i], win, G, R)
        else:
            zs = [F.linear(p, win) for p in pre]
            grads = dz

            def fwd(i):
                F.linear(pre[i], win)

        def bwd(i):
            pre[i].grad = win.grad = None  # fresh gradients: no accumulation kernels in the timing
            torch.autograd.backward(zs[i], grads[i], retain_graph=True)

        f_us = time_launches(torch, fwd, n, reps)
        b_us = time_launches(torch, bwd, n, reps)
        out[name] = {"fwd_us": round(f_us, 2), "fwd_GBs": round(f_bytes / (f_us * 1e-6) / 1e9, 1),
                     "bwd_us": round(b_us, 2), "bwd_GBs": round(b_bytes / (b_us * 1e-6) / 1e9, 1)}
        print(f"[bench] proj_in GEMM (configs[4], 3 groups) {name}: fwd {f_us:.1f} us ({out[name]['fwd_GBs']} GB/s), "
              f"bwd {b_us:.1f} us ({out[name]['bwd_GBs']} GB/s)", file=sys.stderr, flush=True)
        del zs
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=40, help="launches per breakdown measurement")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip configs[4] (lowrank QKV) in the breakdown")
    ap.add_argument("--calibrate-copy", action="store_true", help="only run a plain 256 MiB device copy and exit")
    ap.add_argument("--calibrate-read", action="store_true", help="only run a read-only pass over 256 MiB and exit")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures the hot path on one GPU only (every box has one MI355X); "
              "multi-GPU runs are not part of it. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    import dynconv
    from headwise import headwise_dynamic_convolution as hw
    from lowrank import lowrank_dynamic_convolution as lr

    dynconv.load_library()
    dev = torch.device("cuda", 0)
    print(f"[bench] device {torch.cuda.get_device_name(0)}", file=sys.stderr, flush=True)
    if args.calibrate_copy:
        calibrate_copy(torch, dev)
        return
    if args.calibrate_read:
        calibrate_read(torch, dev)
        return

    data = {}
    for name in STEP + ([] if args.no_extra else list(EXTRA)):
        c = CONFIGS.get(name) or EXTRA[name]
        data[name] = make_inputs(c, torch, dev)
    torch.cuda.synchronize()
    print("[bench] inputs resident", file=sys.stderr, flush=True)

    ROOF = "hw_hs1"  # the dominant launch: its backward is bracketed by events in the timed loop
    ROOF_KERNEL = "hw_bwd_fastIDF16bLi4ELi1ELb1ELb1ELi1E"  # its main kernel's symbol (bf16, W4, HSV1, static, TDW)
    ROOF_LAUNCH = "headwise backward, head_size 1: hw_bwd_fast<bf16,W4,HSV1,static> (+ reduce_partials)"
    roof_ev = []

    def step(roof_events=False):
        """Forward of every config, then every backward in one autograd call, as a training step's
        loss.backward() would run them (the roofline config's launch between events when timed)."""
        ys, dys = {}, {}
        for name in STEP:
            c = CONFIGS[name]
            a, dys[name] = data[name]
            for t in a:
                if t is not None:
                    t.grad = None
            fn = hw if c["kind"] == "hw" else lr
            ys[name] = fn(*a, residual=c["residual"])
        if roof_events:
            # Events around the roofline launch itself: recorded by the backward node's pre- and
            # post-hooks, which autograd runs right before and after the node's backward (its
            # C-ABI launch: hw_bwd_fast + reduce_partials), on the stream that launch uses.
            b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            node = ys[ROOF].grad_fn
            node.register_prehook(lambda grad_outputs: b0.record())
            node.register_hook(lambda grad_inputs, grad_outputs: b1.record())
            roof_ev.append((b0, b1))
        # one backward call, as loss.backward() of a training step
        torch.autograd.backward([ys[n] for n in STEP], [dys[n] for n in STEP])

    step_bytes = sum(sum(alg_bytes(CONFIGS[n])) for n in STEP)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(args.steps):
        step()
    e_ev.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = s_ev.elapsed_time(e_ev)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    # The roofline launch is timed in as many further steps: an event record on the stream holds
    # the GPU for ~5 us, so per-step events stay out of the step timing above.
    for _ in range(args.steps):
        step(roof_events=True)
    torch.cuda.synchronize()
    roof_us = statistics.mean(b0.elapsed_time(b1) for b0, b1 in roof_ev) * 1e3
    print(f"[bench] {args.steps} steps: {ms_per_step:.4f} ms/step (events), wall {wall * 1e3 / args.steps:.4f} ms/step",
          file=sys.stderr, flush=True)

    # per-config, per-direction launch timings (C ABI, rotating cold input sets, HIP events)
    del data
    torch.cuda.empty_cache()
    breakdown = {}
    roofline = None
    names = STEP + ([] if args.no_extra else list(EXTRA))
    for name in names:
        c = CONFIGS.get(name) or EXTRA[name]
        sets = abi_sets(c, torch, dev)
        fwd, bwd = abi_launchers(c, sets, torch)
        calls = c.get("calls", 1)
        f_us = time_launches(torch, fwd, len(sets), args.reps)
        b_us = time_launches(torch, bwd, len(sets), args.reps)
        fb, bb = alg_bytes(c)
        fb_us = f_us + b_us
        gbs = (fb + bb) / (fb_us * 1e-6) / 1e9
        breakdown[name] = {
            "shape": {k: v for k, v in c.items() if k not in ("kind",)},
            "fwd_us": round(f_us * calls, 2), "bwd_us": round(b_us * calls, 2), "fwdbwd_us": round(fb_us * calls, 2),
            "fwd_GBs": round(fb / (f_us * 1e-6) / 1e9, 1), "bwd_GBs": round(bb / (b_us * 1e-6) / 1e9, 1),
            "fwdbwd_GBs": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "alg_MB": round((fb + bb) * calls / 1e6, 2),
            "ns_per_token": round(fb_us * calls * 1e3 / (c["B"] * c["T"]), 3),
        }
        print(f"[bench] {name}: fwd {f_us:.1f} us ({breakdown[name]['fwd_GBs']} GB/s)  bwd {b_us:.1f} us "
              f"({breakdown[name]['bwd_GBs']} GB/s)  fwd+bwd {fb_us:.1f} us = {gbs:.0f} GB/s ({gbs / PEAK_GBS:.1%})",
              file=sys.stderr, flush=True)
        if name == ROOF:
            gbs_of = lambda us: bb / (us * 1e-6) / 1e9
            # achieved / frac: this run's own measurement, the live HIP events around the launch.
            # The committed rocprofv3 trace of this command is reported beside it for comparison
            # (the kernel alone, without the events' own cost), never in its place.
            tr = roofline_trace(ROOF_KERNEL)
            roofline = {
                "kernel": ROOF_LAUNCH,
                "bound": "hbm", "achieved": round(gbs_of(roof_us), 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs_of(roof_us) / PEAK_GBS, 4), "traffic": measured_traffic(ROOF_KERNEL),
                "traffic_source": "profiles/bench_hbm_traffic.md (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
                "alg_bytes_per_launch": bb,
                "duration_us": round(roof_us, 2),
                "duration_source": "live HIP events around the launch in this run",
                "avg_launch_us": round(roof_us, 2),
                "trace_kernel_us": tr["kernel_us"] if tr else None,
                "trace_sequence_us": tr["sequence_us"] if tr else None,
                "frac_trace_kernel": round(gbs_of(tr["kernel_us"]) / PEAK_GBS, 4) if tr else None,
                "frac_trace_sequence": round(gbs_of(tr["sequence_us"]) / PEAK_GBS, 4) if tr else None,
                "trace_source": "profiles/roofline_trace.json (rocprofv3 kernel trace of this command)",
                "timing": f"avg_launch_us: HIP events from the pre- and post-hooks of the {ROOF} backward node "
                          f"(around its C-ABI launch, on its stream) in each of {args.steps} further steps "
                          f"after the timed ones",
                "breakdown_launch_us": round(b_us, 2),
            }
        del sets, fwd, bwd
        torch.cuda.empty_cache()

    qkv = None if args.no_extra else qkv_end_to_end(torch, dev)
    torch.cuda.empty_cache()
    if qkv is not None:
        qkv["proj_in_gemm"] = proj_in_gemm(torch, dev)
        torch.cuda.empty_cache()
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch)
    if cpu is not None and "cfg0_hw_fp32" in breakdown:
        g0 = breakdown["cfg0_hw_fp32"]
        cpu["gpu_same_config"] = {"fwdbwd_us": g0["fwdbwd_us"], "GBs": g0["fwdbwd_GBs"],
                                  "gpu_over_cpu": round(g0["fwdbwd_GBs"] / cpu["value"], 1)}

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (BASELINE.json distributions, CPU generator seed 0, bf16, resident in HBM)",
        "config": {
            "workload": "fwd+bwd of headwise hs1 (H2048) + headwise hs32 (H64) + lowrank R16, "
                        "each B4 T4096 D2048 W4 bf16 residual (headwise with static_w)",
            "B": 4, "T": 4096, "D": 2048, "W": 4, "step_alg_MB": round(step_bytes / 1e6, 2),
            "frac_of_peak": round(value / PEAK_GBS, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown": breakdown,
        "qkv": qkv,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
