"""A synthetic SD1.5 UNet denoising step over the library's operations.

This measures the "UNet step ms" half of the metric: one forward pass of
SD1.5's UNet at 512x512 (latent 64x64, batch 2 for classifier-free guidance,
a 77-token context of 768), random-initialised weights of that architecture
(FP16 conv and linear weights ~N(0, 0.02), as the reference's tests fill
them), with every node the reference takes over from ggml -- CONV_2D,
MUL_MAT, the gated GEGLU product, FLASH_ATTN_EXT, GROUP_NORM, NORM and the
chains after them -- run by libsdhip.  The nodes the reference does not take
(ggml computes them: nearest upsampling, concatenation, the permutes between
the image and token layouts, the sinusoidal timestep embedding and the
linear layers of two rows, under mul_mat_supported's 16, mul_mat.cc:181-194)
are computed by torch on the same stream, as ggml computes them for the
reference.

The graph is stable-diffusion.cpp's UNet for SD1.5 (the model the
reference's tools/bench.cc:128-145 samples its shapes from): 320 channels,
multipliers 1, 2, 4, 4, two ResBlocks a level, SpatialTransformers with 1x1
proj_in/proj_out at levels 0-2 and in the middle, 8 heads, GEGLU FF of 4x.

`Model` holds the weights and runs the step through an `Ops` backend:
`HipOps` calls the C ABI (fails if the library is missing); `TorchOps` is the
plain float64 (or float32) torch restatement of every node, used by the
tests as the checker of a whole step at reduced sizes.
"""

import ctypes
import math

import torch
import torch.nn.functional as F

import sdhip

GELU_K = 1.5957691216057308  # 2 sqrt(2 / pi), the reference's gelu (scalar_math.h:55-63)


class Config:
    """The architecture; the defaults are SD1.5 at 512x512 with CFG."""

    def __init__(self, channels=320, mult=(1, 2, 4, 4), res_blocks=2, heads=8, attn_levels=(0, 1, 2),
                 context_dim=768, context_len=77, in_channels=4, latent=64, batch=2, groups=32):
        self.channels = channels
        self.mult = tuple(mult)
        self.res_blocks = res_blocks
        self.heads = heads
        self.attn_levels = tuple(attn_levels)
        self.context_dim = context_dim
        self.context_len = context_len
        self.in_channels = in_channels
        self.latent = latent
        self.batch = batch
        self.groups = groups
        self.time_dim = 4 * channels


# ---------------------------------------------------------------- backends


class Ops:
    """The nodes of the step.  Image tensors are NCHW, token tensors [b, L, C];
    weights are FP16 ([out, in, kh, kw] or [out, in]), biases and affine
    parameters single precision."""

    def reset(self):
        """Zero the FLOP counts: direct-convolution-equivalent FLOPs of the
        nodes run, in all and by class (conv3x3, conv1x1, linear, attention)."""
        self.flops = 0.0
        self.by_class = {}
        self.nodes = {}

    def count(self, kind, f):
        self.flops += f
        self.by_class[kind] = self.by_class.get(kind, 0.0) + f
        self.nodes[kind] = self.nodes.get(kind, 0) + 1

    def count_conv(self, x, w, y):
        n, oc, oh, ow = y.shape
        ic, kh, kw = w.shape[1:]
        self.count(f"conv{kh}x{kw}", 2.0 * n * oc * oh * ow * ic * kh * kw)

    def count_linear(self, x, w):
        n, k = w.shape
        self.count("linear", 2.0 * (x.numel() // k) * n * k)

    def count_attention(self, q, k, heads):
        b, lq, c = q.shape
        self.count("attention", 4.0 * b * lq * k.shape[1] * c)


class HipOps(Ops):
    """Every node the reference takes, by libsdhip on torch's current stream."""

    def __init__(self, device):
        self.lib = sdhip.load()
        sdhip.check(self.lib.sdhip_init(device.index or 0), "init")
        self.device = device
        self.work = torch.empty(1 << 20, dtype=torch.uint8, device=device)
        self.frozen = False  # under graph capture the work buffer may not grow
        self.widened = {}  # the single-precision copies of ggml's two-row linear layers' weights
        self.reset()

    def _work(self, size):
        if size > self.work.numel():
            if self.frozen:
                raise RuntimeError(f"work buffer of {self.work.numel()} bytes, {size} needed, during capture")
            self.work = torch.empty(size, dtype=torch.uint8, device=self.device)
        return ctypes.c_void_p(self.work.data_ptr()), ctypes.c_size_t(size)

    @staticmethod
    def _chain(steps, redirect=None):
        return sdhip.epilogue(steps, redirect=redirect)

    def conv(self, x, w, bias, stride=1, pad=None, add=()):
        """Convolution, + bias, + each tensor of `add` (broadcast by extent 1)."""
        oc, ic, kh, kw = w.shape
        pad = kh // 2 if pad is None else pad
        n, _, h, wd = x.shape
        oh = (h + 2 * pad - kh) // stride + 1
        ow = (wd + 2 * pad - kw) // stride + 1
        y = torch.empty((n, oc, oh, ow), device=x.device)
        params = sdhip.conv_params(stride, stride, pad, pad, 1, 1)
        steps = [("add", bias.view(1, oc, 1, 1))] + [("add", a) for a in add]
        chain = self._chain(steps)
        dk, dx, dy = sdhip.desc(w), sdhip.desc(x), sdhip.desc(y)
        size = self.lib.sdhip_conv2d_work_size(dk, dx, dy, params)
        ptr, sz = self._work(size)
        sdhip.check(self.lib.sdhip_conv2d(dk, dx, dy, params, ctypes.byref(chain), ptr, sz, sdhip.stream_handle()),
                    f"conv2d {tuple(x.shape)} -> {oc} k{kh} s{stride}")
        self.count_conv(x, w, y)
        return y

    def group_norm(self, x, groups, eps, gamma, beta, silu):
        c = x.shape[1]
        y = torch.empty_like(x)
        steps = [("mul", gamma.view(1, c, 1, 1)), ("add", beta.view(1, c, 1, 1))] + ([("silu", None)] if silu else [])
        chain = self._chain(steps)
        dx, dy = sdhip.desc(x), sdhip.desc(y)
        size = self.lib.sdhip_group_norm_work_size(dx, dy, groups)
        ptr, sz = self._work(size)
        sdhip.check(self.lib.sdhip_group_norm(dx, dy, groups, eps, ctypes.byref(chain), ptr, sz,
                                              sdhip.stream_handle()), "group_norm")
        return y

    def layer_norm(self, x, eps, gamma, beta):
        y = torch.empty_like(x)
        chain = self._chain([("mul", gamma), ("add", beta)])
        sdhip.check(self.lib.sdhip_norm(sdhip.desc(x), sdhip.desc(y), eps, ctypes.byref(chain),
                                        sdhip.stream_handle()), "norm")
        return y

    def linear(self, x, w, bias=None, add=()):
        n, k = w.shape
        m = x.numel() // k
        self.count_linear(x, w)
        if m < 16:
            # Not taken by the reference (mul_mat.cc:181-194): ggml's node,
            # with the weights widened once and kept, as ggml's CPU backend
            # reads them without converting the tensor each time.
            wide = self.widened.get(w.data_ptr())
            if wide is None:
                wide = self.widened[w.data_ptr()] = w.float().t().contiguous()
            y = x.reshape(-1, k) @ wide
            if bias is not None:
                y = y + bias
            for a in add:
                y = y + a.reshape(y.shape)
            return y.reshape(*x.shape[:-1], n)
        y = torch.empty((*x.shape[:-1], n), device=x.device)
        steps = ([("add", bias)] if bias is not None else []) + [("add", a) for a in add]
        chain = self._chain(steps)
        dw, dx, dy = sdhip.desc(w), sdhip.desc(x), sdhip.desc(y)
        size = self.lib.sdhip_mul_mat_work_size(dw, dx, dy)
        ptr, sz = self._work(size)
        sdhip.check(self.lib.sdhip_mul_mat(dw, dx, dy, ctypes.byref(chain) if steps else None, ptr, sz,
                                           sdhip.stream_handle()), f"mul_mat {m}x{n}x{k}")
        return y

    def geglu(self, x, w, bias):
        n, k = w.shape
        m = x.numel() // k
        self.count_linear(x, w)
        y = torch.empty((*x.shape[:-1], n), device=x.device)  # described, never written
        out = torch.empty((*x.shape[:-1], n // 2), device=x.device)
        chain = self._chain([("add", bias)])
        dw, dx, dy, do = sdhip.desc(w), sdhip.desc(x), sdhip.desc(y), sdhip.desc(out)
        size = self.lib.sdhip_mul_mat_work_size(dw, dx, dy)
        ptr, sz = self._work(size)
        sdhip.check(self.lib.sdhip_mul_mat_gated(dw, dx, dy, ctypes.byref(chain), do, ptr, sz,
                                                 sdhip.stream_handle()), f"mul_mat_gated {m}x{n}x{k}")
        return out

    def attention(self, q, k, v, heads):
        """q [b, Lq, C], k/v [b, Lk, C] -> [b, Lq, C]; ggml's permuted views."""
        b, lq, c = q.shape
        lk = k.shape[1]
        d = c // heads
        y = torch.empty((b, lq, heads, d), device=q.device)
        views = [t.view(b, t.shape[1], heads, d).permute(0, 2, 1, 3) for t in (q, k, v)]
        dq, dk, dv = (sdhip.desc(t) for t in views)
        dy = sdhip.desc(y)
        size = self.lib.sdhip_attention_work_size(dq, dk, dv, dy)
        ptr, sz = self._work(size)
        sdhip.check(self.lib.sdhip_attention(dq, dk, dv, dy, 1.0 / math.sqrt(d), 0.0, 0.0, ptr, sz,
                                             sdhip.stream_handle()), f"attention {b}x{heads}x{lq}x{lk}x{d}")
        self.count_attention(q, k, heads)
        return y.view(b, lq, c)


class TorchOps(Ops):
    """The same nodes in plain torch at `dtype` (float64 for the checker):
    the textbook forms the reference's tests compute exactly
    (tests/ops_test.cc: conv 402-424, mul_mat 450-462, attention 517-553,
    GEGLU 745-767) and ggml's GROUP_NORM / NORM (norm.cc:44-175)."""

    def __init__(self, dtype=torch.float64):
        self.dtype = dtype
        self.reset()

    def conv(self, x, w, bias, stride=1, pad=None, add=()):
        kh = w.shape[2]
        pad = kh // 2 if pad is None else pad
        y = F.conv2d(x, w.to(self.dtype), bias.to(self.dtype), stride=stride, padding=pad)
        self.count_conv(x, w, y)
        for a in add:
            y = y + a
        return y

    def group_norm(self, x, groups, eps, gamma, beta, silu):
        y = F.group_norm(x, groups, gamma.to(self.dtype), beta.to(self.dtype), eps)
        return y * torch.sigmoid(y) if silu else y

    def layer_norm(self, x, eps, gamma, beta):
        return F.layer_norm(x, (x.shape[-1],), gamma.to(self.dtype), beta.to(self.dtype), eps)

    def linear(self, x, w, bias=None, add=()):
        self.count_linear(x, w)
        y = x @ w.to(self.dtype).t()
        if bias is not None:
            y = y + bias.to(self.dtype)
        for a in add:
            y = y + a
        return y

    def geglu(self, x, w, bias):
        p = self.linear(x, w, bias)
        half = p.shape[-1] // 2
        a, g = p[..., :half], p[..., half:]
        return a * (g / (1.0 + torch.exp(-GELU_K * g * (1.0 + 0.044715 * g * g))))

    def attention(self, q, k, v, heads):
        self.count_attention(q, k, heads)
        b, lq, c = q.shape
        d = c // heads
        qh, kh, vh = (t.reshape(b, t.shape[1], heads, d).transpose(1, 2) for t in (q, k, v))
        s = (qh @ kh.transpose(-1, -2).contiguous()) / math.sqrt(d)
        p = torch.softmax(s, dim=-1)
        return (p @ vh).transpose(1, 2).reshape(b, lq, c)


# ---------------------------------------------------------------- the model


def timestep_embedding(t, dim, dtype):
    """The sinusoidal embedding of SD's UNet (cos half first)."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64, device=t.device) / half)
    args = t.to(torch.float64)[:, None] * freqs[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1).to(dtype)


class Model:
    """SD1.5's UNet with random weights: FP16 weight tensors ~N(0, 0.02),
    biases ~N(0, 0.01), norm scales ~N(1, 0.1) and shifts ~N(0, 0.1)."""

    def __init__(self, cfg, device, seed=0):
        self.cfg = cfg
        self.device = device
        gdev = device if torch.device(device).type == "cuda" else "cpu"
        self.gen = torch.Generator(device=gdev).manual_seed(seed)
        self.gdev = gdev
        c = cfg.channels
        td = cfg.time_dim
        self.time = (self._lin(td, c), self._lin(td, td))
        self.conv_in = self._conv(c, cfg.in_channels, 3)
        self.down = []  # per level: [(resblock, transformer or None)], downsample conv or None
        chans = [c]
        ch = c
        for lvl, m in enumerate(cfg.mult):
            blocks = []
            for _ in range(cfg.res_blocks):
                out = c * m
                blocks.append((self._res(ch, out), self._st(out) if lvl in cfg.attn_levels else None))
                ch = out
                chans.append(ch)
            down = None
            if lvl != len(cfg.mult) - 1:
                down = self._conv(ch, ch, 3)
                chans.append(ch)
            self.down.append((blocks, down))
        self.mid = (self._res(ch, ch), self._st(ch), self._res(ch, ch))
        self.up = []
        for lvl in reversed(range(len(cfg.mult))):
            m = cfg.mult[lvl]
            blocks = []
            for _ in range(cfg.res_blocks + 1):
                skip = chans.pop()
                out = c * m
                blocks.append((self._res(ch + skip, out), self._st(out) if lvl in cfg.attn_levels else None))
                ch = out
            up = self._conv(ch, ch, 3) if lvl != 0 else None
            self.up.append((blocks, up))
        self.out_norm = self._norm(ch)
        self.conv_out = self._conv(cfg.in_channels, ch, 3)
        self._join_embeddings()

    # -- parameters

    def _randn(self, *shape, std=1.0, mean=0.0):
        if str(self.device) == "meta":  # shapes only, for counting
            return torch.empty(shape, device="meta")
        return (mean + std * torch.randn(shape, generator=self.gen, device=self.gdev)).to(self.device)

    def _w(self, *shape):
        return self._randn(*shape, std=0.02).to(torch.float16)

    def _lin(self, n, k, bias=True):
        return (self._w(n, k), self._randn(n, std=0.01) if bias else None)

    def _conv(self, oc, ic, k):
        return (self._w(oc, ic, k, k), self._randn(oc, std=0.01))

    def _norm(self, c):
        return (self._randn(c, std=0.1, mean=1.0), self._randn(c, std=0.1))

    def _res(self, ic, oc):
        return {"norm1": self._norm(ic), "conv1": self._conv(oc, ic, 3), "emb": self._lin(oc, self.cfg.time_dim),
                "norm2": self._norm(oc), "conv2": self._conv(oc, oc, 3),
                "skip": self._conv(oc, ic, 1) if ic != oc else None}

    def _st(self, c):
        cd = self.cfg.context_dim
        return {"norm": self._norm(c), "proj_in": self._conv(c, c, 1), "proj_out": self._conv(c, c, 1),
                "ln1": self._norm(c), "q1": self._lin(c, c, False), "k1": self._lin(c, c, False),
                "v1": self._lin(c, c, False), "o1": self._lin(c, c),
                "ln2": self._norm(c), "q2": self._lin(c, c, False), "k2": self._lin(c, cd, False),
                "v2": self._lin(c, cd, False), "o2": self._lin(c, c),
                "ln3": self._norm(c), "ff1": self._lin(8 * c, c), "ff2": self._lin(c, 4 * c)}

    def _resblocks(self):
        for blocks, _ in self.down:
            for res, _ in blocks:
                yield res
        yield self.mid[0]
        yield self.mid[2]
        for blocks, _ in self.up:
            for res, _ in blocks:
                yield res

    def _join_embeddings(self):
        """The ResBlocks' embedding projections side by side, [sum oc, time
        dim] and [sum oc]; each block keeps the slice of its columns."""
        ws, bs, at = [], [], 0
        for res in self._resblocks():
            w, b = res["emb"]
            res["emb_at"] = (slice(None), slice(at, at + w.shape[0]))
            at += w.shape[0]
            ws.append(w)
            bs.append(b)
        self.emb_all = (torch.cat(ws), torch.cat(bs))

    # -- blocks

    def resblock(self, ops, p, x, projections):
        g = self.cfg.groups
        h = ops.group_norm(x, g, 1e-5, *p["norm1"], silu=True)
        e = projections[p["emb_at"]]  # [b, oc]: this block's part of the embedding's projections
        oc = e.shape[1]
        h = ops.conv(h, *p["conv1"], add=(e.reshape(-1, oc, 1, 1),))
        h = ops.group_norm(h, g, 1e-5, *p["norm2"], silu=True)
        skip = x if p["skip"] is None else ops.conv(x, *p["skip"], pad=0)
        return ops.conv(h, *p["conv2"], add=(skip,))

    def transformer(self, ops, p, x, context):
        b, c, hh, ww = x.shape
        heads = self.cfg.heads
        h = ops.group_norm(x, self.cfg.groups, 1e-6, *p["norm"], silu=False)
        h = ops.conv(h, *p["proj_in"], pad=0)
        t = h.permute(0, 2, 3, 1).reshape(b, hh * ww, c).contiguous()  # ggml_cont(ggml_permute)
        n = ops.layer_norm(t, 1e-5, *p["ln1"])
        q, k, v = (ops.linear(n, p[name][0]) for name in ("q1", "k1", "v1"))
        t = ops.linear(ops.attention(q, k, v, heads), *p["o1"], add=(t,))
        n = ops.layer_norm(t, 1e-5, *p["ln2"])
        q = ops.linear(n, p["q2"][0])
        k, v = (ops.linear(context, p[name][0]) for name in ("k2", "v2"))
        t = ops.linear(ops.attention(q, k, v, heads), *p["o2"], add=(t,))
        n = ops.layer_norm(t, 1e-5, *p["ln3"])
        t = ops.linear(ops.geglu(n, *p["ff1"]), *p["ff2"], add=(t,))
        h = t.reshape(b, hh, ww, c).permute(0, 3, 1, 2).contiguous()
        return ops.conv(h, *p["proj_out"], pad=0, add=(x,))

    def forward(self, ops, x, t, context):
        """The UNet's output for latents x [b, 4, H, W], timesteps t [b] and
        context [b, L, 768], computed by `ops`."""
        dtype = x.dtype
        emb = timestep_embedding(t, self.cfg.channels, dtype)
        emb = ops.linear(emb, *self.time[0])
        emb = ops.linear(emb * torch.sigmoid(emb), *self.time[1])
        emb_silu = emb * torch.sigmoid(emb)  # each ResBlock's emb_layers begin with SiLU
        # Every ResBlock's projection of the embedding (two rows each: ggml's
        # nodes) as one product over the blocks' weights side by side.
        projections = ops.linear(emb_silu, *self.emb_all)
        h = ops.conv(x, *self.conv_in)
        hs = [h]
        for blocks, down in self.down:
            for res, st in blocks:
                h = self.resblock(ops, res, h, projections)
                if st is not None:
                    h = self.transformer(ops, st, h, context)
                hs.append(h)
            if down is not None:
                h = ops.conv(h, *down, stride=2, pad=1)
                hs.append(h)
        res1, st, res2 = self.mid
        h = self.resblock(ops, res1, h, projections)
        h = self.transformer(ops, st, h, context)
        h = self.resblock(ops, res2, h, projections)
        for blocks, up in self.up:
            for res, st in blocks:
                h = torch.cat([h, hs.pop()], dim=1)  # ggml_concat
                h = self.resblock(ops, res, h, projections)
                if st is not None:
                    h = self.transformer(ops, st, h, context)
            if up is not None:
                h = F.interpolate(h, scale_factor=2.0, mode="nearest")  # ggml_upscale
                h = ops.conv(h, *up)
        h = ops.group_norm(h, self.cfg.groups, 1e-5, *self.out_norm, silu=True)
        return ops.conv(h, *self.conv_out)

    def inputs(self, seed=1, dtype=torch.float32, device=None):
        """Synthetic latents ~N(0,1), timesteps, and a context ~N(0,1)."""
        cfg = self.cfg
        g = torch.Generator(device="cpu").manual_seed(seed)
        dev = device or self.device
        x = torch.randn((cfg.batch, cfg.in_channels, cfg.latent, cfg.latent), generator=g).to(dev, dtype)
        t = torch.full((cfg.batch,), 981.0).to(dev)
        ctx = torch.randn((cfg.batch, cfg.context_len, cfg.context_dim), generator=g).to(dev, dtype)
        return x, t, ctx

    def to_reference(self, device="cpu"):
        """A copy of the weights on `device` (FP16 kept, for TorchOps)."""
        ref = object.__new__(Model)
        ref.cfg = self.cfg
        ref.device = device

        def move(o):
            if isinstance(o, torch.Tensor):
                return o.to(device)
            if isinstance(o, dict):
                return {k: move(v) for k, v in o.items()}
            if isinstance(o, (list, tuple)):
                return type(o)(move(v) for v in o)
            return o

        for name in ("time", "conv_in", "down", "mid", "up", "out_norm", "conv_out", "emb_all"):
            setattr(ref, name, move(getattr(self, name)))
        return ref


class Graph:
    """`fn()` on the GPU, captured once in a HIP graph (torch.cuda.graph)
    after an eager call that sizes the work buffer of `ops`; `run()` replays
    it, `eager()` calls `fn` again."""

    def __init__(self, fn, ops):
        self.fn, self.ops = fn, ops
        ops.reset()
        self.out = fn()  # eager: sizes the work buffer
        self.flops, self.by_class, self.nodes = ops.flops, dict(ops.by_class), dict(ops.nodes)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        ops.frozen = True
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(self.graph, stream=stream):
                self.out = fn()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        ops.frozen = False

    def run(self):
        self.graph.replay()
        return self.out

    def eager(self):
        return self.fn()


class Step(Graph):
    """The UNet step of `model` on `inputs` (x, t, context), as a Graph."""

    def __init__(self, model, ops, inputs):
        self.model = model
        self.x, self.t, self.ctx = inputs
        super().__init__(lambda: model.forward(ops, self.x, self.t, self.ctx), ops)


class SdxlBlock:
    """The transformer block of the SDXL configuration: LayerNorm, Q/K/V
    projections (no bias), self-attention over `heads` heads, the output
    projection with its bias and the residual, LayerNorm, the GEGLU FF
    (C -> 2 x 4C with bias, gated) and its projection back with bias and the
    residual; FP16 weights ~N(0, 0.02), biases ~N(0, 0.01), norms ~N(1, 0.1) /
    ~N(0, 0.1).  `forward(ops, x)` for tokens x [b, L, C]."""

    def __init__(self, device, channels=1280, heads=20, seed=0):
        m = object.__new__(Model)
        m.device = device
        gdev = device if torch.device(device).type == "cuda" else "cpu"
        m.gen = torch.Generator(device=gdev).manual_seed(seed)
        m.gdev = gdev
        c = channels
        self.heads = heads
        self.ln1, self.ln2 = m._norm(c), m._norm(c)
        self.wq, self.wk, self.wv = (m._w(c, c) for _ in range(3))
        self.wo = m._lin(c, c)
        self.ff1 = m._lin(8 * c, c)
        self.ff2 = m._lin(c, 4 * c)

    def forward(self, ops, x):
        n = ops.layer_norm(x, 1e-5, *self.ln1)
        q, k, v = (ops.linear(n, w) for w in (self.wq, self.wk, self.wv))
        x = ops.linear(ops.attention(q, k, v, self.heads), *self.wo, add=(x,))
        n = ops.layer_norm(x, 1e-5, *self.ln2)
        return ops.linear(ops.geglu(n, *self.ff1), *self.ff2, add=(x,))
