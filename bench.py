"""Benchmark of the MI355X form of stable-diffusion.assembly's hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

A step is one pass of the hot path over one batch of synthetic input: the
configuration BASELINE.json's metric is quoted on, configs[1] -- the SD1.5
ResNet 3x3 convolution [2, 320, 64, 64] -> 320 by Winograd F(4x4, 3x3) with
its bias and residual add fused -- with inputs resident in HBM.  `value` is
TFLOP/s counted in direct-convolution FLOPs (2 * N * OC * OH * OW * IC * 9),
as the metric asks.

Every configuration of BASELINE.json is timed the same way and reported under
"configs": warm (the mean over `steps` calls after `warmup`) and cold (caches
flushed before each call), its kernels' times, and the roofline of its
dominant kernel(s) -- the algorithmic FLOPs or bytes one call gives them over
their time, measured by the library's kernel profile (HIP events stamped by
the kernels' own dispatch packets on their stream), against MI355X's peak.
The top-level roofline is configs[1]'s.  The SD1.5 UNet step follows (a HIP
graph), then the VAE decoder's operations, then cpu_baseline: every
configuration and the UNet step on the host's cores by oracle/port.c (this
repository's AVX-512 restatement of the reference's CPU algorithms), on all
the cores the run may use and on one thread, with the host named and its
measured FMA peak.

Prints one JSON line on stdout; progress goes to stderr.
"""

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stable-diffusion.assembly_amd"))

METRIC = "TFLOP/s per op (direct-conv-equiv) + SD1.5 UNet step ms, 1 MI355X"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, dense
PEAK_FP16_MFMA = 2500.0
PEAK_INT8_MFMA = 5000.0  # TOPS, dense
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

        def run():
            graph.run()

        run.eager, run.keep = graph.eager, graph
        return run, graph.flops
    if name in ("unet", "unet_kept"):
        step = unet_workload(dev, keep=name.endswith("kept"))
        return step.run, step.flops
    raise SystemExit(f"unknown workload {name}")


# ---------------------------------------------------------------- the host CPU baseline


def host_threads():
    """The host cores this run may use: its affinity, at most 16 (a GPU box
    gives one GPU's job 16 cores, whatever os.cpu_count() reports)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_info():
    """The host CPU as lscpu names it (model, sockets, cores), /proc/cpuinfo
    where lscpu is missing."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "CPU(s)": "cpus", "CPU max MHz": "max_mhz",
            "Flags": "flags"}
    for line in out.splitlines():
        key, _, val = line.partition(":")
        if key.strip() in keys:
            info[keys[key.strip()]] = val.strip()
    if "model" not in info and os.path.exists("/proc/cpuinfo"):
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["model"] = line.partition(":")[2].strip()
                break
    flags = info.pop("flags", "").split()
    info["isa"] = [f for f in ("avx2", "fma", "avx512f", "avx512_vnni", "avx512_bf16", "amx_int8") if f in flags]
    return info


def best_seconds(fn, budget, least=2):
    """The fastest of repeated runs of fn after one uncounted run, repeated
    for about `budget` seconds and at least `least` times
    (tools/bench.cc:427-451)."""
    fn()
    best, runs, end = None, 0, time.perf_counter() + budget
    while runs < least or time.perf_counter() < end:
        t = time.perf_counter()
        fn()
        dt = time.perf_counter() - t
        best = dt if best is None else min(best, dt)
        runs += 1
    return best, runs


def _orc():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib

    return oracle_lib


def cpu_ops(threads, bits=0, weight_groups=1):
    """The UNet's and the SDXL block's nodes on the host's cores by
    oracle/port.c's restatements (the cpu_baseline leg): convolutions by the
    path the library would take (F(4x4), F(2x2) or direct, by
    sdhip_conv2d_path's host-side rule), MUL_MAT, the GEGLU product,
    attention, GROUP_NORM and NORM; the nodes the reference leaves to ggml by
    torch on the CPU, as HipOps leaves them to torch.  With bits=8, the linear
    layers quantized (weights quantized and packed once, kept, as the
    reference keeps its quantized layouts; inputs per call)."""
    import unet_step

    class CpuOps(unet_step.Ops):
        def __init__(self, threads, bits=0, weight_groups=1):
            import sdhip

            self.orc = _orc()
            self.threads = threads
            self.bits = bits
            self.weight_groups = weight_groups
            self.lib = sdhip.load()  # sdhip_conv2d_path only: host code, no device call
            self.widened = {}
            self.quantized = {}
            self.reset()

        def _w32(self, w):
            key = (w.data_ptr(), tuple(w.shape))
            got = self.widened.get(key)
            if got is None:
                got = self.widened[key] = w.float().contiguous().numpy()
            return got

        @staticmethod
        def _np(t):
            return t.detach().contiguous().numpy()

        def conv(self, x, w, bias, stride=1, pad=None, add=()):
            import torch

            import sdhip

            oc, ic, kh, kw = w.shape
            pad = kh // 2 if pad is None else pad
            n, _, h, wd = x.shape
            oh, ow = (h + 2 * pad - kh) // stride + 1, (wd + 2 * pad - kw) // stride + 1
            y = torch.empty((n, oc, oh, ow))
            x = x.contiguous()
            params = sdhip.conv_params(stride, stride, pad, pad, 1, 1)
            path = self.lib.sdhip_conv2d_path(sdhip.desc(w), sdhip.desc(x), sdhip.desc(y), params)
            full = [a for a in add if tuple(a.shape) == (n, oc, oh, ow)]
            res = self._np(full[0]) if full else None
            rest = [a for a in add if not (full and a is full[0])]
            b = self._np(bias)
            if path in (2, 4):
                self.orc.port_winograd(self._np(x), self._w32(w), pad, b, res, four=path == 4, threads=self.threads,
                                       out=y.numpy())
            else:
                self.orc.port_conv2d(self._np(x), self._w32(w), stride, pad, b, res, threads=self.threads, out=y.numpy())
            for a in rest:
                y += a
            self.count_conv(x, w, y)
            return y

        def group_norm(self, x, groups, eps, gamma, beta, silu):
            import torch

            return torch.from_numpy(self.orc.port_group_norm(self._np(x), groups, eps, self._np(gamma), self._np(beta),
                                                             silu, self.threads))

        def layer_norm(self, x, eps, gamma, beta):
            import torch

            return torch.from_numpy(self.orc.port_norm(self._np(x), eps, self._np(gamma), self._np(beta), self.threads))

        def _product(self, x2, w, bias, gated=False):
            n, k = w.shape
            if self.bits:
                key = (w.data_ptr(), tuple(w.shape))
                packed = self.quantized.get(key)
                if packed is None:
                    wq, ws, wo, _ = self.orc.quantize_weights(self._w32(w), 64, 127, self.weight_groups)
                    packed = self.quantized[key] = self.orc.port_pack_qweights(wq, ws, wo, 64)
                return self.orc.port_quantized_linear(x2, packed, n, 64, 255, bias, gated=gated, threads=self.threads)
            y = self.orc.port_mul_mat(self._w32(w), x2, bias, threads=self.threads)
            return (y, self.orc.port_gated(y, self.threads)) if gated else y

        def linear(self, x, w, bias=None, add=()):
            import torch

            n, k = w.shape
            m = x.numel() // k
            self.count_linear(x, w)
            if m < 16:  # ggml's node, as HipOps leaves it to torch
                y = x.reshape(-1, k) @ torch.from_numpy(self._w32(w)).t()
                if bias is not None:
                    y = y + bias
            else:
                y = torch.from_numpy(self._product(self._np(x.reshape(-1, k)), w,
                                                   None if bias is None else self._np(bias)))
            for a in add:
                y = y + a.reshape(y.shape)
            return y.reshape(*x.shape[:-1], n)

        def geglu(self, x, w, bias):
            import torch

            n, k = w.shape
            self.count_linear(x, w)
            _, out = self._product(self._np(x.reshape(-1, k)), w, self._np(bias), gated=True)
            return torch.from_numpy(np.ascontiguousarray(out)).reshape(*x.shape[:-1], n // 2)

        def attention(self, q, k, v, heads):
            import torch

            b, lq, c = q.shape
            d = c // heads
            self.count_attention(q, k, heads)
            qn, kn, vn = (self._np(t).reshape(b, -1, heads, d) for t in (q, k, v))
            if self.bits and kn.shape[1] >= 256:
                # The bits mode's attention where the reference quantizes it
                # (attention.cc:622-624): group 64, stretches of 256 keys.
                y = self.orc.port_quantized_attention(qn, kn, vn, 1.0 / d ** 0.5, 64, 255, 127, 256,
                                                      threads=self.threads)
            else:
                y = self.orc.port_attention(qn, kn, vn, 1.0 / d ** 0.5, threads=self.threads)
            return torch.from_numpy(y).reshape(b, lq, c)

    return CpuOps(threads, bits, weight_groups)


def sdxl_block_ops(tokens=988, batch=2, c=1280):
    """configs[4]'s operations: its products (2 M N K: Q, K, V and the output
    projection C x C, the GEGLU C -> 8C, the FF out 4C -> C) and its attention
    (4 L^2 C a batch)."""
    m = tokens * batch
    return 2.0 * m * c * (4 * c + 8 * c + 4 * c) + 4.0 * batch * tokens * tokens * c


def cpu_configs():
    """Per configuration: (make(threads) -> fn, work, unit, fp32): the
    configuration's operation on the host, on synthetic inputs of its shapes
    (weights FP16 ~N(0,0.02) widened once; the bits mode's quantized once)."""
    orc = _orc()
    r = np.random.default_rng(1)

    def randn(*shape, std=1.0, mean=0.0):
        return (mean + std * r.standard_normal(shape)).astype(np.float32)

    def weights(*shape):
        return randn(*shape, std=0.02).astype(np.float16).astype(np.float32)

    out = {}
    x1, w1, b1 = randn(8192, 320), weights(320, 320), randn(320, std=0.01)
    out["cfg1_linear"] = (lambda t: (lambda: orc.port_mul_mat(w1, x1, b1, t)), 2.0 * 8192 * 320 * 320, "TFLOP/s", True)
    x2, w2, b2, r2 = randn(2, 320, 64, 64), weights(320, 320, 3, 3), randn(320, std=0.01), randn(2, 320, 64, 64)
    y2 = np.empty_like(x2)
    out["cfg2_winograd4"] = (lambda t: (lambda: orc.port_winograd(x2, w2, 1, b2, r2, True, t, out=y2)),
                             2.0 * 2 * 320 * 64 * 64 * 320 * 9, "TFLOP/s", True)
    x3, w3, b3 = randn(2, 1280, 8, 8), weights(1280, 1280, 3, 3), randn(1280, std=0.01)
    g3, be3 = randn(1280, std=0.1, mean=1.0), randn(1280, std=0.1)

    def cfg3a(t):
        def run():
            y = orc.port_winograd(x3, w3, 1, b3, None, False, t)
            orc.port_group_norm(y, 32, 1e-5, g3, be3, True, t)
        return run

    out["cfg3a_winograd2_gn_silu"] = (cfg3a, 2.0 * 2 * 1280 * 64 * 1280 * 9, "TFLOP/s", True)
    x4, w4 = randn(2, 640, 32, 32), weights(1280, 640, 1, 1)

    def cfg3b(t):
        def run():
            y = orc.port_conv2d(x4, w4, 1, 0, b3, None, t)
            orc.port_group_norm(y, 32, 1e-5, g3, be3, True, t)
        return run

    out["cfg3b_pointwise_gn_silu"] = (cfg3b, 2.0 * 2 * 1280 * 1024 * 640, "TFLOP/s", True)
    q5 = randn(2, 4096, 8, 40)
    k5, v5 = randn(2, 4096, 8, 40), randn(2, 4096, 8, 40)
    kc, vc = randn(2, 77, 8, 40), randn(2, 77, 8, 40)
    s5 = 1.0 / 40 ** 0.5
    out["cfg4_self_attention"] = (lambda t: (lambda: orc.port_attention(q5, k5, v5, s5, t)),
                                  4.0 * 2 * 8 * 4096 * 4096 * 40, "TFLOP/s", True)
    out["cfg4_cross_attention"] = (lambda t: (lambda: orc.port_attention(q5, kc, vc, s5, t)),
                                   4.0 * 2 * 8 * 4096 * 77 * 40, "TFLOP/s", True)

    def cfg5(t):
        import torch

        import unet_step

        block = unet_step.SdxlBlock(torch.device("cpu"), seed=9)
        x = torch.from_numpy(randn(2, 988, 1280))
        ops = cpu_ops(t, bits=8, weight_groups=0)
        torch.set_num_threads(t)
        return lambda: block.forward(ops, x)

    out["cfg5_sdxl_block_bits8"] = (cfg5, None, "TOPS", False)
    return out


def cpu_unet_step(threads, seconds):
    """The SD1.5 UNet step (the GPU's synthetic model and inputs, random
    weights from the CPU's generator) on the host through CpuOps: ms of the
    fastest of the timed steps after one uncounted."""
    import torch

    import unet_step

    torch.set_num_threads(threads)
    model = unet_step.Model(unet_step.Config(), torch.device("cpu"), seed=7)
    x, t, ctx = model.inputs(seed=8, device="cpu")
    ops = cpu_ops(threads)

    def step():
        ops.reset()
        return model.forward(ops, x, t, ctx)

    best, runs = best_seconds(step, seconds, least=1)
    return {"ms": round(best * 1e3, 1), "tflops": round(ops.flops / best / 1e12, 3), "threads": threads,
            "runs": runs, "gflop": round(ops.flops / 1e9, 1)}


def cpu_baseline(seconds):
    """The host CPU beside the GPU: each configuration's operation by
    oracle/port.c on all the cores this run may use and on one thread, as a
    rate and as a fraction of the host's measured FMA peak at that thread
    count; the UNet step on all cores; the host named (lscpu).  `value` is
    configs[1] on all cores."""
    import torch

    orc = _orc()
    if not orc.port_available():
        return {"value": None, "unit": "TFLOP/s", "cores": 0, "kind": "port",
                "sample": "not run: the host lacks AVX-512 with VNNI, which oracle/port.c is built for"}
    threads = host_threads()
    torch_threads = torch.get_num_threads()
    peaks = {1: orc.port_fma_peak(1, 0.3), threads: orc.port_fma_peak(threads, 0.3)}
    per = max(0.3, seconds / 16)
    table = {}
    for name, (make, work, unit, fp32) in cpu_configs().items():
        row = {}
        for t in (threads, 1):
            fn = make(t)
            best, runs = best_seconds(fn, per)
            amount = work if work is not None else sdxl_block_ops()
            entry = {"ms": round(best * 1e3, 3), unit.split("/")[0].lower(): round(amount / best / 1e12, 4),
                     "runs": runs}
            if fp32:
                entry["fma_peak_frac"] = round(amount / best / 1e9 / peaks[t], 3)
            row[f"threads_{t}"] = entry
            log(f"cpu {name} {t} threads: {best * 1e3:.2f} ms ({runs} runs)")
        table[name] = row
    unet = cpu_unet_step(threads, max(1.0, seconds / 4))
    log(f"cpu unet step {threads} threads: {unet['ms']} ms")
    torch.set_num_threads(torch_threads)
    head = table["cfg2_winograd4"][f"threads_{threads}"]
    return {"value": head["tflop"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"the whole configs[1] convolution (F(4x4), bias + residual) in single precision, the fastest "
                      f"of {head['runs']} runs after one uncounted, {threads} OpenMP threads (AVX-512); every "
                      f"configuration likewise on {threads} threads and on one under 'configs', the UNet step "
                      f"under 'unet_step'",
            "host": host_info(), "threads": threads,
            "fma_peak_gflops": {f"threads_{t}": round(v, 1) for t, v in peaks.items()},
            "configs": table, "unet_step": unet,
            "note": "oracle/port.c: this repository's AVX-512 restatement of the reference's CPU algorithms "
                    "(packed GEMM, Winograd with transforms per block, blocked attention, VNNI W8A8); the "
                    "reference's own x86 kernels need ggml and C++26 and are not built here.  cfg5 on the CPU: "
                    "the block in the bits mode, as on the GPU -- its linear layers quantized (weights per row, "
                    "kept) and its self-attention quantized (VNNI, attention.cc:612-824)"}


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


# Per configuration: its workload, its work (direct-convolution FLOPs for the
# convolutions; int8 operations for configs[4]) and the roofline of its
# dominant kernel -- the kernel(s) named, the algorithmic amount one call of
# the configuration gives them (FLOPs, or the ideal HBM bytes where HBM
# bounds them), the bound and MI355X's published peak.  The amounts are
# those of the configurations' work units, restated:
#   cfg1  Y = X W^T + b, X 2x4096x320 f32, W 320x320 f16: X 10.49 MB + W 0.20 +
#         b + Y 10.49 = 21.18 MB (AI 79: HBM-bound at the split-FP16 rate)
#   cfg2  the 36 products of 320x320 by 512 tiles: 2 x 36 x 320 x 320 x 512
#         = 3.775 GFLOP a call on the FP16 MFMA, three MFMAs a product, against
#         the raw 2.5 PF (and the split's 833 TF effective); the op's
#         direct-equivalent 15.10 GFLOP against the target of 1.5 x 2.5 PF.
#         Beside it, the products' bytes (U and V read once as two FP16
#         planes, 36 x 2 x 2 x (320 + 512) x 320 = 38.34 MB; M written once,
#         36 x 4 x 320 x 512 = 23.59 MB) against 8 TB/s, and the whole op's
#         counter bytes against its own algorithmic 33.3 MB (input 10.49 MB,
#         FP16 weights 1.84, bias, residual 10.49, output 10.49)
#   cfg3a F(2x2) of 8x8 maps: the products kernel reads the FP16 weights,
#         1280x1280x9x2 = 29.49 MB (it makes U in registers)
#   cfg3b 1x1 conv 2x640x1024 -> 1280: 3.355 GFLOP
#   cfg4  self: 4 b h L^2 d = 42.95 GFLOP; cross (77 keys): Q 10.49 MB + K, V
#         0.39 MB + Y 10.49 MB = 21.37 MB (HBM)
#   cfg5  the quantized products of the block: 103.6 G int8 operations
CONFIGS = {
    "cfg1_linear": dict(workload="cfg1", unit="TFLOP/s", kernels=("mul_mat",), bound="hbm", amount=21.18e6,
                        peak=PEAK_HBM),
    "cfg2_winograd4": dict(workload="cfg2", unit="TFLOP/s", kernels=("winograd4.products",), bound="mfma",
                           amount=2.0 * 36 * 320 * 320 * 512, peak=PEAK_FP16_MFMA, split=3,
                           hbm_bytes=36 * 2 * 2 * (320 + 512) * 320 + 36 * 4 * 320 * 512.0,
                           op_bytes=(3 * 2 * 320 * 64 * 64 + 320) * 4 + 320 * 320 * 9 * 2.0, op_target=1.5),
    "cfg3a_winograd2_gn_silu": dict(workload="cfg3a", unit="TFLOP/s", kernels=("winograd2.products",), bound="hbm",
                                    amount=1280 * 1280 * 9 * 2.0, peak=PEAK_HBM),
    "cfg3b_pointwise_gn_silu": dict(workload="cfg3b", unit="TFLOP/s", kernels=("conv_direct_pointwise",),
                                    bound="mfma", amount=2.0 * 2 * 1280 * 1024 * 640, peak=PEAK_FP16_MFMA, split=2),
    "cfg4_self_attention": dict(workload="cfg4_self", unit="TFLOP/s", kernels=("attention",), bound="mfma",
                                amount=4.0 * 2 * 8 * 4096 * 4096 * 40, peak=PEAK_FP16_MFMA, split=3),
    "cfg4_cross_attention": dict(workload="cfg4_cross", unit="TFLOP/s", kernels=("attention",), bound="hbm",
                                 amount=21.37e6, peak=PEAK_HBM),
    "cfg5_sdxl_block_bits8": dict(workload="cfg5", unit="TOPS", kernels=("qgemm", "qgemm_gated"), bound="mfma",
                                  amount=2.0 * 1976 * 1280 * 16 * 1280, peak=PEAK_INT8_MFMA),
}


def roofline(spec, kt, op_ms, work):
    """The roofline object of a configuration's dominant kernel(s): achieved
    = the algorithmic amount / their time per call (the library's kernel
    profile: HIP events stamped by the kernels' own dispatch packets, on their
    stream), against MI355X's published peak; the op's own rate beside it."""
    ms = sum(kt[k][0] * kt[k][1] for k in spec["kernels"] if k in kt)
    if ms <= 0:
        return None
    hbm = spec["bound"] == "hbm"
    achieved = spec["amount"] / ms / (1e6 if hbm else 1e9)  # GB/s or TFLOP/s
    out = {"kernel": "+".join(spec["kernels"]), "bound": spec["bound"], "achieved": round(achieved, 2),
           "peak": spec["peak"], "unit": "GB/s" if hbm else ("TOPS" if spec["unit"] == "TOPS" else "TFLOP/s"),
           "frac": round(achieved / spec["peak"], 4), "kernel_us": round(ms * 1e3, 2),
           "amount": spec["amount"], "traffic": profiled_traffic(spec["workload"], spec["kernels"][0])}
    if spec.get("split"):
        # Split-FP16: each product takes `split` FP16 MFMA products.
        out["effective_peak"] = round(spec["peak"] / spec["split"], 1)
        out["frac_of_effective"] = round(achieved * spec["split"] / spec["peak"], 4)
    if spec.get("hbm_bytes"):
        # The same kernel's algorithmic bytes against HBM's peak.
        gbs = spec["hbm_bytes"] / ms / 1e6
        out["hbm_view"] = {"achieved": round(gbs, 1), "peak": PEAK_HBM, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM, 4), "amount": spec["hbm_bytes"]}
    rate = work / op_ms / 1e9
    peak = PEAK_INT8_MFMA if spec["unit"] == "TOPS" else PEAK_FP16_MFMA
    out["op_rate"] = round(rate, 2)
    out["op_rate_vs_mfma_peak"] = round(rate / peak, 4)
    if spec.get("op_target"):
        # The north star's target for Winograd: op_target x the FP16 peak in
        # direct-convolution FLOPs.
        out["op_target"] = {"rate": spec["op_target"] * peak, "frac": round(rate / (spec["op_target"] * peak), 4)}
    if spec.get("op_bytes"):
        # Every kernel of the op, counter bytes per call, against the op's
        # algorithmic bytes (inputs and outputs once each).
        op_traffic = profiled_traffic(spec["workload"], "op")
        out["op_bytes"] = {"algorithmic": spec["op_bytes"], "traffic": op_traffic,
                           "ratio": round(op_traffic / spec["op_bytes"], 2) if op_traffic else None}
    return out


def cold_ms(fn, calls=10):
    """ms of one call with the caches cold: before each call 1 GiB is written
    (past the 4 MB L2 of each XCD and the 256 MB MALL); the median over
    `calls`, HIP events around the call alone."""
    import torch

    flush = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
    times = []
    for i in range(calls):
        flush.fill_(float(i))
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        stop.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop))
    del flush
    times.sort()
    return times[len(times) // 2]


def measure_config(dev, name, args):
    """A configuration timed warm (the mean of `steps` calls after `warmup`),
    cold (cold_ms), its kernels and its roofline."""
    spec = CONFIGS[name]
    run, work = make_workload(dev, spec["workload"])
    ms = timed(run, args.steps, args.warmup)
    kt = kernel_times(getattr(run, "eager", run), min(args.steps, 20))
    entry = {"ms": round(ms, 5), spec["unit"].split("/")[0].lower(): round(work / ms / 1e9, 2),
             "cold_ms": round(cold_ms(run), 5),
             "kernels_us": {k: round(v[0] * v[1] * 1e3, 2) for k, v in sorted(kt.items(), key=lambda kv: -kv[1][0] * kv[1][1])},
             "roofline": roofline(spec, kt, ms, work)}
    log(f"{name}: {ms * 1e3:.1f} us warm, {entry['cold_ms'] * 1e3:.1f} us cold, "
        f"{work / ms / 1e9:.1f} {spec['unit']}; roofline {entry['roofline']}")
    return entry, ms, work, kt


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
    _, _, path = conv_workload(dev, 2, 320, 64, 64, 320, 3, 1, seed=2)
    assert path == 4, f"configs[1] takes path {path}, not F(4x4)"
    head, ms, work, kt = measure_config(dev, "cfg2_winograd4", args)
    value = work / ms / 1e9
    fp32 = sdhip.get_tuning("winograd_fp32") == 1
    roof = dict(head["roofline"])
    roof["mfma"] = "v_mfma_f32_16x16x4_f32" if fp32 else "v_mfma_f32_32x32x16_f16, 3 per product (split FP16)"
    roof["kernels_us"] = {k: round(v[0] * 1e3, 2) for k, v in kt.items()}
    roof["direct_eq_vs_fp16_peak"] = round(value / PEAK_FP16_MFMA, 4)
    configs = {"cfg2_winograd4": head}
    # Beside it, the transformed weights kept from call to call, as the
    # reference's store keeps them when given a budget (none by default).
    run_k, _, _ = conv_workload(dev, 2, 320, 64, 64, 320, 3, 1, seed=2, keep=True)
    ms_k = timed(run_k, args.steps, args.warmup)
    head["weights_kept"] = {"ms": round(ms_k, 5), "tflop": round(work / ms_k / 1e9, 2)}
    log(f"cfg2 weights kept: {ms_k * 1e3:.1f} us")
    del run_k
    no_store()
    if not args.only_main:
        for name in CONFIGS:
            if name == "cfg2_winograd4":
                continue
            configs[name] = measure_config(dev, name, args)[0]
            if name == "cfg3a_winograd2_gn_silu":
                run3k, f3a, _ = conv_workload(dev, 2, 1280, 8, 8, 1280, 3, 1, bias=True, residual=False,
                                              groupnorm=True, seed=3, keep=True)
                m3k = timed(run3k, args.steps, args.warmup)
                configs[name]["weights_kept"] = {"ms": round(m3k, 5), "tflop": round(f3a / m3k / 1e9, 2)}
                del run3k
                no_store()
        configs["cfg5_sdxl_block_bits8"].update(
            {"gop": round(sdxl_block_ops() / 1e9, 2), "tuning": "bits=8,weight_group=0",
             "store": "quantized weights kept (the reference's default)"})

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
        if not args.no_unet:
            host = line["cpu_baseline"].get("unet_step")
            if host:
                line["unet_step"]["host_cpu"] = host
                line["unet_step"]["vs_host_cpu"] = round(host["ms"] / line["unet_step"]["ms"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
