"""Benchmark of the MI355X form of stable-diffusion.assembly's hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

A step is one pass of the hot path over one batch of synthetic input: the
configuration BASELINE.json's metric is quoted on, configs[1] -- the SD1.5
ResNet 3x3 convolution [2, 320, 64, 64] -> 320 by Winograd F(4x4, 3x3) with
its bias and residual add fused -- with inputs resident in HBM.  `value` is
TFLOP/s counted in direct-convolution FLOPs (2 * N * OC * OH * OW * IC * 9),
as the metric asks.  The other configurations are timed the same way and
reported under "configs"; the roofline object is that of the workload's
dominant kernel, timed with HIP events on its own stream; cpu_baseline is the
oracle's single-precision restatement of the same F(4x4) algorithm on this
host's cores (oracle/port.c).

Prints one JSON line on stdout; progress goes to stderr.
"""

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stable-diffusion.assembly_amd"))

METRIC = "TFLOP/s per op (direct-conv-equiv) + SD1.5 UNet step ms, 1 MI355X"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, dense
PEAK_FP16_MFMA = 2500.0
PEAK_HBM = 8000.0  # GB/s


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only-main", action="store_true")
    p.add_argument("--workload", default="", help="run one workload alone (cfg1 cfg2 cfg2_kept cfg3a cfg3a_kept "
                                                  "cfg3b cfg4_self cfg4_cross cfg5 unet unet_kept copy "
                                                  "vendor_products vendor_4096), for a profiler")
    p.add_argument("--no-unet", action="store_true", help="leave out the UNet step")
    p.add_argument("--no-vae", action="store_true", help="leave out the VAE decoder's operations")
    return p.parse_args()


def timed(fn, steps, warmup):
    """ms per call of fn over `steps` calls after `warmup`, bracketed by
    synchronisations, with HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def kernel_times(fn, steps):
    """{kernel: (ms per launch, launches per call)} over `steps` calls."""
    import torch

    import sdhip

    torch.cuda.synchronize()
    sdhip.profile_reset()
    sdhip.profile_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    sdhip.profile_enable(False)
    out = {}
    for name, (ms, n) in sdhip.profile_collect().items():
        out[name] = (ms / n, n / steps)
    return out


def profiled_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` in `workload`, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs summarised in profiles/hbm_traffic.md, or
    None where that table has no such row."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == workload and cells[1] == kernel:
            return int(cells[4])
    return None


_ARENA = None


def fresh_store(dev, gib=6):
    """The device store's arena, emptied: the derived forms of the weights
    kept from one call to the next -- the bits mode's quantized weights, as the
    reference keeps them by default (store.cc:64-99, 8 GiB), and Winograd's
    transformed weights, as it keeps them when SDASM_STORE_MB gives its store
    a budget (winograd.cc:2147-2149; store.h:26-34: none by default) -- the
    first, untimed call fills it.  Emptied per workload, so that no entry
    outlives the tensors it was made from."""
    import torch

    import sdhip

    global _ARENA
    if _ARENA is None:
        _ARENA = torch.empty(gib << 30, dtype=torch.uint8, device=dev)
    sdhip.store_arena(_ARENA)
    return _ARENA


def no_store():
    """No store: every call derives its weights' forms, the reference's
    default for single-precision layouts."""
    import sdhip

    sdhip.store_arena(None)


def conv_workload(dev, n, ic, h, w, oc, k, pad, bias=True, residual=True, groupnorm=False, seed=0, keep=False):
    """The convolution of a configuration with its chain, ready to run."""
    import torch

    import sdhip

    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((n, ic, h, w), generator=g, device=dev, dtype=torch.float32)
    kern = (0.02 * torch.randn((oc, ic, k, k), generator=g, device=dev)).to(torch.float16)
    oh, ow = h + 2 * pad - k + 1, w + 2 * pad - k + 1
    y = torch.empty((n, oc, oh, ow), device=dev, dtype=torch.float32)
    steps = []
    if bias:
        b = 0.01 * torch.randn((1, oc, 1, 1), generator=g, device=dev)
        steps.append(("add", b))
    if residual:
        r = torch.randn((n, oc, oh, ow), generator=g, device=dev)
        steps.append(("add", r))
    chain = sdhip.epilogue(steps)
    params = sdhip.conv_params(1, 1, pad, pad, 1, 1)
    lib = sdhip.load()
    dk, dx, dy = sdhip.desc(kern), sdhip.desc(x), sdhip.desc(y)
    size = lib.sdhip_conv2d_work_size(dk, dx, dy, params)
    work = torch.empty(max(size, 1), dtype=torch.uint8, device=dev)
    path = lib.sdhip_conv2d_path(dk, dx, dy, params)
    gn = None
    if groupnorm:
        gamma = 1.0 + 0.1 * torch.randn((1, oc, 1, 1), generator=g, device=dev)
        beta = 0.1 * torch.randn((1, oc, 1, 1), generator=g, device=dev)
        out = torch.empty_like(y)
        gn_size = lib.sdhip_group_norm_work_size(sdhip.desc(y), sdhip.desc(out), 32)
        gn_work = torch.empty(max(gn_size, 8), dtype=torch.uint8, device=dev)
        gn = (out, sdhip.epilogue([("mul", gamma), ("add", beta), ("silu", None)]), sdhip.desc(out), gn_work, gn_size)
    stream = sdhip.stream_handle()
    arena = fresh_store(dev) if keep else no_store()
    keep = (x, kern, y, steps, work, arena)

    def run():
        sdhip.check(lib.sdhip_conv2d(dk, dx, dy, params, ctypes.byref(chain), ctypes.c_void_p(work.data_ptr()),
                                     size, stream), "conv2d")
        if gn is not None:
            sdhip.check(lib.sdhip_group_norm(dy, gn[2], 32, 1e-5, ctypes.byref(gn[1]), ctypes.c_void_p(gn[3].data_ptr()),
                                             gn[4], stream), "group_norm")

    flops = 2.0 * n * oc * oh * ow * ic * k * k
    run.keep = keep
    return run, flops, path


def linear_workload(dev, k, nout, m, batch, seed=0):
    import torch

    import sdhip

    g = torch.Generator(device=dev).manual_seed(seed)
    w = (0.02 * torch.randn((nout, k), generator=g, device=dev)).to(torch.float16)
    x = torch.randn((batch, m, k), generator=g, device=dev)
    b = 0.01 * torch.randn((nout,), generator=g, device=dev)
    y = torch.empty((batch, m, nout), device=dev)
    chain = sdhip.epilogue([("add", b)])
    lib = sdhip.load()
    dw, dx, dy = sdhip.desc(w), sdhip.desc(x), sdhip.desc(y)
    size = lib.sdhip_mul_mat_work_size(dw, dx, dy)
    work = torch.empty(max(size, 1), dtype=torch.uint8, device=dev)
    stream = sdhip.stream_handle()

    def run():
        sdhip.check(lib.sdhip_mul_mat(dw, dx, dy, ctypes.byref(chain), ctypes.c_void_p(work.data_ptr()), size,
                                      stream), "mul_mat")

    run.keep = (w, x, b, y, work)
    return run, 2.0 * k * nout * m * batch


def attention_workload(dev, b, h, lq, lk, d, seed=0):
    """cfg4: Q [b, h, lq, d], K/V [b, h, lk, d] ~N(0,1), ggml's head layout."""
    import torch

    import sdhip

    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn((b, lq, h, d), generator=g, device=dev)
    k = torch.randn((b, lk, h, d), generator=g, device=dev)
    v = torch.randn((b, lk, h, d), generator=g, device=dev)
    y = torch.empty((b, lq, h, d), device=dev)
    lib = sdhip.load()
    dq, dk, dv, dy = (sdhip.desc(q.permute(0, 2, 1, 3)), sdhip.desc(k.permute(0, 2, 1, 3)),
                      sdhip.desc(v.permute(0, 2, 1, 3)), sdhip.desc(y))
    scale = 1.0 / d ** 0.5
    stream = sdhip.stream_handle()
    size = lib.sdhip_attention_work_size(dq, dk, dv, dy)  # the keys' and values' split tiles
    work = torch.empty(max(size, 1), dtype=torch.uint8, device=dev)
    ptr = work.data_ptr()

    def run():
        sdhip.check(lib.sdhip_attention(dq, dk, dv, dy, scale, 0.0, 0.0, ptr, size, stream), "attention")

    run.keep = (q, k, v, y, work)
    return run, 4.0 * b * h * lq * lk * d


def copy_workload(dev, mib=256):
    """A plain device copy of known size: the scale for the HBM byte counters
    (FETCH_SIZE, WRITE_SIZE) a profiler reads for the other kernels."""
    import torch

    src = torch.ones(mib << 18, device=dev)
    dst = torch.empty_like(src)

    def run():
        dst.copy_(src)

    run.keep = (src, dst)
    return run, 0.0


def vendor_workload(dev, batch, m, n, k, seed):
    """torch.bmm (the vendor's hipBLASLt / rocBLAS) in FP16 on contiguous
    operands, for comparison only, never a path of the library: the vendor's
    time for the same MFMA work as one of this library's kernels
    (vendor_products: configs[1]'s products, 36 points x 3 split products of
    320 x 512 x 320, as one batch of 108), or for a large square product that
    shows the MFMA rate the vendor reaches where K is long (vendor_4096)."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn(batch, m, k, device=dev, dtype=torch.float16, generator=gen)
    b = torch.randn(batch, k, n, device=dev, dtype=torch.float16, generator=gen)
    out = torch.empty(batch, m, n, device=dev, dtype=torch.float16)

    def run():
        torch.bmm(a, b, out=out)

    run.keep = (a, b, out)
    return run, 2.0 * batch * m * n * k


def unet_workload(dev, seed=7, keep=False):
    """The synthetic SD1.5 UNet step (unet_step.py) at 512x512, batch 2,
    captured in a HIP graph; with `keep`, Winograd's transformed weights kept
    in the store."""
    import unet_step

    model = unet_step.Model(unet_step.Config(), dev, seed=seed)
    arena = fresh_store(dev) if keep else no_store()
    step = unet_step.Step(model, unet_step.HipOps(dev), model.inputs(seed=seed + 1))
    step.keep = (model, arena)
    return step


def sdxl_block_workload(dev, tuning="bits=8,weight_group=0", seed=9):
    """the SDXL transformer block at 988 tokens (26x38), batch 2,
    1280 channels, 20 heads of 64, in the bits mode (weights int8 per output
    row), captured in a HIP graph with the tuning in effect."""
    import torch

    import sdhip
    import unet_step

    block = unet_step.SdxlBlock(dev, seed=seed)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    x = torch.randn((2, 988, 1280), generator=g, device=dev)
    ops = unet_step.HipOps(dev)
    # The quantized weights kept from one step to the next, as the reference
    # keeps its quantized layouts by default (store.cc:64-99).
    arena = fresh_store(dev)

    def fn():
        sdhip.set_tuning(tuning)
        try:
            return block.forward(ops, x)
        finally:
            sdhip.set_tuning("")

    graph = unet_step.Graph(fn, ops)
    graph.keep = (block, x, arena)
    return graph


def make_workload(dev, name):
    """(run, FLOPs) of a named workload: the BASELINE.json configurations."""
    if name == "cfg1":
        return linear_workload(dev, 320, 320, 4096, 2, seed=1)
    if name in ("cfg2", "cfg2_kept"):
        run, flops, _ = conv_workload(dev, 2, 320, 64, 64, 320, 3, 1, seed=2, keep=name.endswith("kept"))
        return run, flops
    if name in ("cfg3a", "cfg3a_kept"):
        run, flops, _ = conv_workload(dev, 2, 1280, 8, 8, 1280, 3, 1, bias=True, residual=False, groupnorm=True, seed=3,
                                      keep=name.endswith("kept"))
        return run, flops
    if name == "cfg3b":
        run, flops, _ = conv_workload(dev, 2, 640, 32, 32, 1280, 1, 0, bias=True, residual=False, groupnorm=True,
                                      seed=4)
        return run, flops
    if name == "cfg4_self":
        return attention_workload(dev, 2, 8, 4096, 4096, 40, seed=5)
    if name == "cfg4_cross":
        return attention_workload(dev, 2, 8, 4096, 77, 40, seed=5)
    if name == "copy":
        return copy_workload(dev)
    if name == "vendor_products":
        return vendor_workload(dev, 108, 320, 512, 320, seed=11)
    if name == "vendor_4096":
        return vendor_workload(dev, 1, 4096, 4096, 4096, seed=12)
    if name == "cfg5":
        graph = sdxl_block_workload(dev)
        return graph.run, graph.flops
    if name in ("unet", "unet_kept"):
        step = unet_workload(dev, keep=name.endswith("kept"))
        return step.run, step.flops
    raise SystemExit(f"unknown workload {name}")


def cpu_baseline(seconds):
    """The oracle's F(4x4) restatement on this host's cores, on the full
    configs[1] convolution, repeated for about `seconds`; the best rate."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc

    lib = orc.lib()
    f = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
    L, I = ctypes.c_int64, ctypes.c_int
    lib.oracle_port_winograd4.argtypes = [f, L, L, L, L, f, L, I, I, f, f, f, I]
    n, ic, h, w, oc = 2, 320, 64, 64, 320
    r = np.random.default_rng(1)
    x = r.standard_normal((n, ic, h, w)).astype(np.float32)
    k = (0.02 * r.standard_normal((oc, ic, 3, 3))).astype(np.float16).astype(np.float32)
    bias = (0.01 * r.standard_normal(oc)).astype(np.float32)
    res = r.standard_normal((n, oc, h, w)).astype(np.float32)
    y = np.empty((n, oc, h, w), np.float32)
    cores = min(16, os.cpu_count() or 1)
    flops = 2.0 * n * oc * h * w * ic * 9
    best, runs, t_end = None, 0, time.time() + seconds
    while time.time() < t_end or runs < 2:
        t = time.perf_counter()
        lib.oracle_port_winograd4(x, n, ic, h, w, k, oc, 1, 1, bias, res, y, cores)
        dt = time.perf_counter() - t
        runs += 1
        if runs > 1:  # the first run is not counted (tools/bench.cc:427-451)
            best = dt if best is None else min(best, dt)
    return {"value": round(flops / best / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"the whole configs[1] convolution (F(4x4), bias + residual) in single precision, "
                      f"best of {runs - 1} runs after one uncounted, {cores} OpenMP threads"}


# The VAE decoder's operations of the reference's bench (tools/bench.cc:146-153):
# 3x3 convolutions (w, h, ic, oc) at batch 1 with their bias, and the
# attention of its middle block (one head of 512 over 4096 positions).
VAE_CONVS = [(64, 64, 512, 512), (128, 128, 512, 512), (256, 256, 256, 256), (256, 256, 512, 512),
             (512, 512, 128, 128), (512, 512, 256, 256)]


def vae_decoder_line(dev, args):
    """Each of the VAE decoder's operations timed alone (synthetic inputs of
    their shapes, weights ~N(0,0.02))."""
    out = {}
    steps, warmup = max(3, args.steps // 10), max(1, args.warmup // 5)
    for (w, h, ic, oc) in VAE_CONVS:
        run, flops, path = conv_workload(dev, 1, ic, h, w, oc, 3, 1, bias=True, residual=False, seed=w + ic)
        ms = timed(run, steps, warmup)
        out[f"conv {w}x{h} {ic}->{oc}"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2), "path": path}
        log(f"vae conv {w}x{h} {ic}->{oc}: {ms:.3f} ms, {flops / ms / 1e9:.1f} TFLOP/s (path {path})")
        del run
    run, flops = attention_workload(dev, 1, 1, 4096, 4096, 512, seed=3)
    ms = timed(run, steps, warmup)
    out["attention 1x4096x4096x512"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2)}
    log(f"vae attention d=512: {ms:.3f} ms, {flops / ms / 1e9:.1f} TFLOP/s")
    return out


def unet_step_line(dev, args):
    """The SD1.5 UNet step in ms: the graph replayed `steps` times after
    `warmup`; the eager step (the same launches from Python) beside it, and
    where the kernels' time goes, by the library's kernel profile of one
    eager step."""
    import torch

    log("unet step: building the model and capturing the graph ...")
    step = unet_workload(dev)
    ms = timed(step.run, max(5, args.steps // 5), max(2, args.warmup // 5))
    eager_ms = timed(step.eager, 3, 1)
    kt = kernel_times(step.eager, 1)
    lib_ms = sum(v[0] * v[1] for v in kt.values())
    torch.cuda.synchronize()
    log(f"unet step: {ms:.2f} ms (graph), {eager_ms:.2f} ms eager, library kernels {lib_ms:.2f} ms")
    flops, nodes, by_class = step.flops, step.nodes, step.by_class
    del step
    # Beside it, Winograd's transformed weights kept from step to step, as the
    # reference's store keeps them when given a budget.
    kept = unet_workload(dev, keep=True)
    kept_ms = timed(kept.run, max(5, args.steps // 5), max(2, args.warmup // 5))
    del kept
    no_store()
    log(f"unet step, weights kept: {kept_ms:.2f} ms")
    return {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 2),
            "weights_kept": {"ms": round(kept_ms, 3), "tflops": round(flops / kept_ms / 1e9, 2)},
            "gflop": round(flops / 1e9, 2), "nodes": nodes,
            "gflop_by_class": {k: round(v / 1e9, 2) for k, v in by_class.items()},
            "eager_ms": round(eager_ms, 3), "library_kernels_ms": round(lib_ms, 3),
            "kernels_ms": {k: round(v[0] * v[1], 3) for k, v in sorted(kt.items(), key=lambda kv: -kv[1][0] * kv[1][1])},
            "workload": "SD1.5 UNet at 512x512 (latent 64x64), batch 2 (CFG), context 77x768, random weights "
                        "(FP16 ~N(0,0.02)); the nodes ggml keeps (concat, upsample, permutes, timestep embedding, "
                        "two-row linears) by torch on the same stream; one HIP graph",
            "reference_published_ms": {"i7-1360P 12 threads": 3540, "note": "README.md:29-34: 70.8 s for 20 steps; "
                                       "other hardware, context only"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported in this build "
              f"(each operation of the path shards by images, rows or heads without exchange)", file=sys.stderr)
        sys.exit(2)
    import torch

    import sdhip

    dev = torch.device("cuda", 0)
    sdhip.check(sdhip.load().sdhip_init(0), "init")
    log(f"device: {torch.cuda.get_device_name(0)}")

    if args.workload:
        # One workload alone, for a profiler: warmup + steps calls, one line.
        run, flops = make_workload(dev, args.workload)
        ms = timed(run, args.steps, args.warmup)
        print(json.dumps({"workload": args.workload, "ms": round(ms, 5),
                          "tflops": round(flops / ms / 1e9, 3) if flops else None}), flush=True)
        return

    # The headline: configs[1], F(4x4) with bias and residual fused.
    run, flops, path = conv_workload(dev, 2, 320, 64, 64, 320, 3, 1, seed=2)
    assert path == 4, f"configs[1] takes path {path}, not F(4x4)"
    ms = timed(run, args.steps, args.warmup)
    value = flops / ms / 1e9
    log(f"cfg2 F(4x4) 64x64x320: {ms * 1e3:.1f} us, {value:.1f} TFLOP/s direct-eq")
    kt = kernel_times(run, args.steps)
    dominant = max(kt, key=lambda n: kt[n][0] * kt[n][1])
    dom_ms = kt[dominant][0]
    # The products: 36 GEMMs of OC x IC x tiles, 2 FLOP per multiply-add,
    # each product taken as three FP16 MFMA products of its split parts, so
    # the instruction's peak is the FP16 one and a third of it the ceiling.
    tiles = 2 * 16 * 16
    alg = 2.0 * 36 * 320 * 320 * tiles
    fp32 = sdhip.get_tuning("winograd_fp32") == 1
    peak = PEAK_FP32_MFMA if fp32 else PEAK_FP16_MFMA
    roof = {"kernel": dominant, "bound": "mfma", "achieved": round(alg / dom_ms / 1e9, 2), "peak": peak,
            "unit": "TFLOP/s", "frac": round(alg / dom_ms / 1e9 / peak, 4),
            "traffic": profiled_traffic("cfg2", dominant),
            "mfma": "v_mfma_f32_16x16x4_f32" if fp32 else "v_mfma_f32_32x32x16_f16, 3 per product (split FP16)",
            "effective_peak": peak if fp32 else round(PEAK_FP16_MFMA / 3, 1),
            "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in kt.items()}}
    log(f"kernels: {roof['kernels_us']}")

    configs = {"cfg2_winograd4": {"ms": round(ms, 5), "tflops": round(value, 2)}}
    # Beside it, the transformed weights kept from call to call, as the
    # reference's store keeps them when given a budget (none by default).
    run_k, _, _ = conv_workload(dev, 2, 320, 64, 64, 320, 3, 1, seed=2, keep=True)
    ms_k = timed(run_k, args.steps, args.warmup)
    configs["cfg2_winograd4"]["weights_kept"] = {"ms": round(ms_k, 5), "tflops": round(flops / ms_k / 1e9, 2)}
    log(f"cfg2 weights kept: {ms_k * 1e3:.1f} us")
    no_store()
    if not args.only_main:
        run1, f1 = linear_workload(dev, 320, 320, 4096, 2, seed=1)
        m1 = timed(run1, args.steps, args.warmup)
        configs["cfg1_linear"] = {"ms": round(m1, 5), "tflops": round(f1 / m1 / 1e9, 2),
                                  "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in kernel_times(run1, 10).items()}}
        log(f"cfg1 linear: {m1 * 1e3:.1f} us")
        run3a, f3a, p3a = conv_workload(dev, 2, 1280, 8, 8, 1280, 3, 1, bias=True, residual=False, groupnorm=True,
                                        seed=3)
        m3a = timed(run3a, args.steps, args.warmup)
        configs["cfg3a_winograd2_gn_silu"] = {"ms": round(m3a, 5), "tflops": round(f3a / m3a / 1e9, 2), "path": p3a,
                                              "kernels_us": {k: round(v[0] * 1e3, 2)
                                                             for k, v in kernel_times(run3a, 10).items()}}
        log(f"cfg3a F(2x2)+GN+SiLU: {m3a * 1e3:.1f} us")
        run3k, _, _ = conv_workload(dev, 2, 1280, 8, 8, 1280, 3, 1, bias=True, residual=False, groupnorm=True, seed=3,
                                    keep=True)
        m3k = timed(run3k, args.steps, args.warmup)
        configs["cfg3a_winograd2_gn_silu"]["weights_kept"] = {"ms": round(m3k, 5), "tflops": round(f3a / m3k / 1e9, 2)}
        log(f"cfg3a weights kept: {m3k * 1e3:.1f} us")
        no_store()
        run3b, f3b, p3b = conv_workload(dev, 2, 640, 32, 32, 1280, 1, 0, bias=True, residual=False, groupnorm=True,
                                        seed=4)
        m3b = timed(run3b, args.steps, args.warmup)
        configs["cfg3b_pointwise_gn_silu"] = {"ms": round(m3b, 5), "tflops": round(f3b / m3b / 1e9, 2),
                                              "path": p3b,
                                              "kernels_us": {k: round(v[0] * 1e3, 2)
                                                             for k, v in kernel_times(run3b, 10).items()}}
        log(f"cfg3b 1x1+GN+SiLU: {m3b * 1e3:.1f} us")
        g5 = sdxl_block_workload(dev)
        m5 = timed(g5.run, args.steps, args.warmup)
        configs["cfg5_sdxl_block_bits8"] = {
            "ms": round(m5, 5), "tops": round(g5.flops / m5 / 1e9, 2), "gop": round(g5.flops / 1e9, 2),
            "tuning": "bits=8,weight_group=0", "store": "quantized weights kept (the reference's default)",
            "kernels_us": {k: round(v[0] * v[1] * 1e3, 2) for k, v in kernel_times(g5.eager, 5).items()}}
        log(f"cfg5 SDXL block bits=8: {m5 * 1e3:.1f} us, {g5.flops / m5 / 1e9:.1f} TOPS")
        for name, lk in (("cfg4_self_attention", 4096), ("cfg4_cross_attention", 77)):
            run4, f4 = attention_workload(dev, 2, 8, 4096, lk, 40, seed=5)
            m4 = timed(run4, args.steps, args.warmup)
            configs[name] = {"ms": round(m4, 5), "tflops": round(f4 / m4 / 1e9, 2),
                             "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in kernel_times(run4, 5).items()}}
            log(f"{name}: {m4 * 1e3:.1f} us, {f4 / m4 / 1e9:.1f} TFLOP/s")

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "configs[1]: SD1.5 ResNet 3x3 conv [2,320,64,64]->320, pad 1, Winograd F(4x4,3x3), "
                               "FP16 weights ~N(0,0.02), fused bias + residual add",
                   "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "configs": configs,
    }
    if not args.no_unet:
        line["unet_step"] = unet_step_line(dev, args)
    if not args.no_vae:
        line["vae_decoder"] = vae_decoder_line(dev, args)
    if not args.no_cpu:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
