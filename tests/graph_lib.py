"""Graphs of sdhip_node (include/sdhip.h) built as ggml builds its graphs, for
the planner's tests (sdhip_plan_nodes, sdhip_compute_nodes).

A `Graph` makes nodes the way ggml's constructors do -- an in-place ADD or MUL
is a node whose tensor is its first operand's memory, a RESHAPE or VIEW a node
over another's memory, a DUP or CONT a node of memory of its own -- and orders
them as ggml_build_forward_expand does (operands first, depth first, each node
once; tensors without an operation are leaves, not nodes).  Each node's data is
a torch tensor (on the device for the GPU tests, on the host for the planner's
CPU tests, whose predicates never read the memory).

`run(graph, ...)` computes a graph as ggml's loop over its nodes does with the
reference's hook: each node offered to sdhip_compute_nodes first, which
computes it with the nodes it fuses and says how many; the nodes it does not
take computed here with torch in single precision (ggml's own kernels stand-in:
ADD, MUL, SILU, GELU by the reference's tanh form, CONT, DUP)."""

import ctypes
import math

import numpy as np
import torch

import sdhip

OP = dict(NONE=0, VIEW=1, RESHAPE=2, PERMUTE=3, TRANSPOSE=4, ADD=5, MUL=6, CONT=7, UNARY=8, MUL_MAT=9, CONV_2D=10,
          FLASH_ATTN_EXT=11, GROUP_NORM=12, NORM=13, OTHER=14)
UNARY_SILU, UNARY_GELU = 1, 2
FLAG_COMPUTE, FLAG_OUTPUT = 1, 2


Node = sdhip.Node
Plan = sdhip.NodePlan


def bind(lib):
    """The library, its graph entry points bound (sdhip.py binds them all)."""
    return lib


def f32_bits(v):
    return int(np.float32(v).view(np.int32))


class T:
    """A tensor of the graph: its torch data (a view where ggml's is one),
    the operation that makes it (None for a leaf) and its operands."""

    def __init__(self, data, op=None, src=(), unary=0, params=(), view_src=None):
        self.data = data
        self.op = op
        self.src = list(src)
        self.unary = unary
        self.params = list(params)
        self.view_src = view_src
        self.output = False
        self.node = None  # the ctypes Node, made by Graph.build


def desc_of(t):
    """The ggml descriptor of a torch tensor of up to 4 dimensions, the
    strides as they are (views included)."""
    return sdhip.desc(t)


class Graph:
    def __init__(self, device):
        self.device = device

    # -- leaves and operations, as ggml's constructors make them

    def leaf(self, a):
        return T(torch.as_tensor(a, device=self.device).contiguous())

    def conv2d(self, w, x, s0=1, s1=1, p0=0, p1=0, d0=1, d1=1):
        n, ic, ih, iw = x.data.shape
        oc, _, kh, kw = w.data.shape
        oh = (ih + 2 * p1 - d1 * (kh - 1) - 1) // s1 + 1
        ow = (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1
        out = torch.full((n, oc, oh, ow), float("nan"), device=self.device)
        return T(out, "CONV_2D", [w, x], params=[s0, s1, p0, p1, d0, d1])

    def mul_mat(self, w, x):
        out = torch.full(tuple(x.data.shape[:-1]) + (w.data.shape[0],), float("nan"), device=self.device)
        return T(out, "MUL_MAT", [w, x])

    def group_norm(self, x, groups, eps):
        return T(torch.full_like(x.data, float("nan")), "GROUP_NORM", [x], params=[groups, f32_bits(eps)])

    def norm(self, x, eps):
        return T(torch.full_like(x.data, float("nan")), "NORM", [x], params=[f32_bits(eps)])

    def add(self, a, b):
        return T(torch.full_like(a.data, float("nan")), "ADD", [a, b])

    def add_inplace(self, a, b):
        return T(a.data, "ADD", [a, b], view_src=a)

    def mul_inplace(self, a, b):
        return T(a.data, "MUL", [a, b], view_src=a)

    def mul(self, a, b):
        return T(torch.full_like(a.data, float("nan")), "MUL", [a, b])

    def silu_inplace(self, a):
        return T(a.data, "UNARY", [a], unary=UNARY_SILU, view_src=a)

    def gelu_inplace(self, a):
        return T(a.data, "UNARY", [a], unary=UNARY_GELU, view_src=a)

    def reshape(self, a, shape):
        return T(a.data.reshape(shape), "RESHAPE", [a], view_src=a)

    def view_columns(self, a, begin, width):
        """ggml_view of columns [begin, begin + width) of a (dimension 0)."""
        return T(a.data[..., begin:begin + width], "VIEW", [a], view_src=a)

    def cont(self, a):
        return T(torch.full(tuple(a.data.shape), float("nan"), device=self.device), "CONT", [a])

    def dup(self, a):
        return T(torch.full_like(a.data, float("nan")), "OTHER", [a])

    # -- the graph

    def build(self, out, outputs=()):
        """The nodes in ggml_build_forward_expand's order, as ctypes nodes."""
        order, seen = [], set()

        def visit(t):
            if id(t) in seen:
                return
            seen.add(id(t))
            for s in t.src:
                visit(s)
            if t.view_src is not None:
                visit(t.view_src)
            if t.op is not None:
                order.append(t)

        visit(out)
        out.output = True
        for t in outputs:
            t.output = True
        # Every tensor reachable gets a ctypes node (leaves too: they are
        # sources), made before any pointer to it is taken.
        every = []

        def collect(t):
            if t.node is not None:
                return
            t.node = Node()
            every.append(t)
            for s in t.src:
                collect(s)
            if t.view_src is not None:
                collect(t.view_src)

        collect(out)
        for t in every:
            n = t.node
            n.op = OP[t.op] if t.op is not None else OP["NONE"]
            n.unary = t.unary
            n.flags = (FLAG_COMPUTE if t.op is not None else 0) | (FLAG_OUTPUT if t.output else 0)
            for i, p in enumerate(t.params):
                n.op_params[i] = p
            n.tensor = desc_of(t.data)
            for i, s in enumerate(t.src):
                n.src[i] = ctypes.pointer(s.node)
            if t.view_src is not None:
                n.view_src = ctypes.pointer(t.view_src.node)
        arr = (ctypes.POINTER(Node) * len(order))(*[ctypes.pointer(t.node) for t in order])
        return order, arr


def plan(lib, arr, n, index):
    p = Plan()
    status = lib.sdhip_plan_nodes(arr, n, index, ctypes.byref(p))
    return status, p


def gelu_ref(x):
    """The reference's GELU (scalar_math.h:58-63) in torch single precision,
    for the nodes the library does not take."""
    y = x * torch.addcmul(torch.ones_like(x), 0.044715 * x, x)
    return x / (1.0 + torch.exp(-1.5957691216057308 * y))


def compute_node(t):
    """One node the library did not take, as ggml's CPU kernels compute it."""
    if t.op in ("RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "NONE"):
        return
    s = [x.data for x in t.src]
    if t.op == "ADD":
        t.data.copy_(s[0] + s[1])
    elif t.op == "MUL":
        t.data.copy_(s[0] * s[1])
    elif t.op == "UNARY":
        v = s[0]
        t.data.copy_(v * torch.sigmoid(v) if t.unary == UNARY_SILU else gelu_ref(v))
    elif t.op in ("CONT", "OTHER"):
        t.data.copy_(s[0])
    else:
        raise AssertionError(f"node {t.op} not taken by the library")


def run(lib, order, arr, stream=None):
    """ggml's loop over the nodes with the hook in front: returns the number
    of nodes the library computed (taken and fused)."""
    n = len(order)
    size = 0
    for t in order:
        s = ctypes.c_size_t(0)
        if lib.sdhip_node_work_size(ctypes.pointer(t.node), ctypes.byref(s)):
            size = max(size, s.value)
    work = torch.empty(max(size, 1), dtype=torch.uint8, device=order[0].data.device)
    handle = stream if stream is not None else sdhip.stream_handle()
    i, by_library = 0, 0
    while i < n:
        consumed = lib.sdhip_compute_nodes(arr, n, i, ctypes.c_void_p(work.data_ptr()), size, handle)
        assert consumed >= 0, lib.sdhip_last_error().decode()
        if consumed == 0:
            compute_node(order[i])
            i += 1
        else:
            by_library += consumed
            i += consumed
    return by_library
