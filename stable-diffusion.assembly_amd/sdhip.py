"""ctypes binding of libsdhip.so (include/sdhip.h) for tests and the bench.

Tensors are described as ggml describes them: ne[] extents with ne[0] the
innermost, nb[] byte strides, and a device pointer.  `desc(t)` makes that
descriptor from a torch tensor (ne reversed from torch's shape, strides in
bytes).  Every call goes to the HIP library; nothing here computes.
"""

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsdhip.so")

TYPE_F32 = 0
TYPE_F16 = 1
OK, UNSUPPORTED, ERROR = 0, 1, 2
STEP_ADD, STEP_MUL, STEP_SILU = 0, 1, 2
MAX_STEPS = 6


class Tensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_int64 * 4),
        ("data", ctypes.c_void_p),
    ]


class Step(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("operand", Tensor)]


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("count", ctypes.c_int32),
        ("steps", Step * MAX_STEPS),
        ("redirect", ctypes.POINTER(Tensor)),
        ("from_redirect", ctypes.c_int32),
    ]


MAX_SRC = 10
MAX_OP_PARAMS = 16


class Node(ctypes.Structure):
    """sdhip_node: a node of a ggml graph as the planner reads it."""


Node._fields_ = [
    ("op", ctypes.c_int32),
    ("unary", ctypes.c_int32),
    ("flags", ctypes.c_int32),
    ("op_params", ctypes.c_int32 * MAX_OP_PARAMS),
    ("tensor", Tensor),
    ("src", ctypes.POINTER(Node) * MAX_SRC),
    ("view_src", ctypes.POINTER(Node)),
]


class NodePlan(ctypes.Structure):
    _fields_ = [
        ("taken", ctypes.c_int32),
        ("count", ctypes.c_int32),
        ("chain", Epilogue),
        ("gated_out", ctypes.POINTER(Node)),
    ]


_T = ctypes.POINTER(Tensor)
_E = ctypes.POINTER(Epilogue)
_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I6 = ctypes.c_int32 * 6

# (name, restype, argtypes) of every symbol sdhip.h declares.
SIGNATURES = [
    ("sdhip_init", ctypes.c_int, [ctypes.c_int]),
    ("sdhip_last_error", ctypes.c_char_p, []),
    ("sdhip_set_tuning", ctypes.c_int, [ctypes.c_char_p]),
    ("sdhip_get_tuning", ctypes.c_int, [ctypes.c_char_p]),
    ("sdhip_forget", None, [_P, _SZ]),
    ("sdhip_store_arena", None, [_P, _SZ]),
    ("sdhip_store_used", _SZ, [ctypes.POINTER(_SZ)]),
    ("sdhip_profile_enable", None, [ctypes.c_int]),
    ("sdhip_profile_reset", None, []),
    ("sdhip_profile_collect", ctypes.c_int, []),
    ("sdhip_profile_entry", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
    ("sdhip_mul_mat_supported", ctypes.c_int, [_T, _T, _T]),
    ("sdhip_mul_mat_work_size", _SZ, [_T, _T, _T]),
    ("sdhip_mul_mat", ctypes.c_int, [_T, _T, _T, _E, _P, _SZ, _P]),
    ("sdhip_mul_mat_gated_supported", ctypes.c_int, [_T, _T, _T, _T]),
    ("sdhip_mul_mat_gated", ctypes.c_int, [_T, _T, _T, _E, _T, _P, _SZ, _P]),
    ("sdhip_conv2d_supported", ctypes.c_int, [_T, _T, _T, _I6]),
    ("sdhip_conv2d_path", ctypes.c_int, [_T, _T, _T, _I6]),
    ("sdhip_conv2d_work_size", _SZ, [_T, _T, _T, _I6]),
    ("sdhip_conv2d", ctypes.c_int, [_T, _T, _T, _I6, _E, _P, _SZ, _P]),
    ("sdhip_attention_supported", ctypes.c_int, [_T, _T, _T, _T, ctypes.c_float, ctypes.c_float]),
    ("sdhip_attention_work_size", _SZ, [_T, _T, _T, _T]),
    ("sdhip_attention", ctypes.c_int,
     [_T, _T, _T, _T, ctypes.c_float, ctypes.c_float, ctypes.c_float, _P, _SZ, _P]),
    ("sdhip_group_norm_supported", ctypes.c_int, [_T, _T, ctypes.c_int]),
    ("sdhip_group_norm_work_size", _SZ, [_T, _T, ctypes.c_int]),
    ("sdhip_group_norm", ctypes.c_int, [_T, _T, ctypes.c_int, ctypes.c_float, _E, _P, _SZ, _P]),
    ("sdhip_group_norm_static", ctypes.c_int, [_T, _T, ctypes.c_int, ctypes.c_float, _E, _P]),
    ("sdhip_norm_supported", ctypes.c_int, [_T, _T]),
    ("sdhip_norm", ctypes.c_int, [_T, _T, ctypes.c_float, _E, _P]),
    ("sdhip_plan_nodes", ctypes.c_int,
     [ctypes.POINTER(ctypes.POINTER(Node)), ctypes.c_int, ctypes.c_int, ctypes.POINTER(NodePlan)]),
    ("sdhip_compute_nodes", ctypes.c_int,
     [ctypes.POINTER(ctypes.POINTER(Node)), ctypes.c_int, ctypes.c_int, _P, _SZ, _P]),
    ("sdhip_node_work_size", ctypes.c_int, [ctypes.POINTER(Node), ctypes.POINTER(_SZ)]),
    ("sdhip_token_downsampling", ctypes.c_int, [ctypes.c_int64, ctypes.c_int64]),
]

_lib = None


def load():
    """The library, loaded once; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it (make -C stable-diffusion.assembly_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class SdhipError(RuntimeError):
    def __init__(self, status, what):
        super().__init__(f"{what}: status {status}: {load().sdhip_last_error().decode()}")
        self.status = status


def check(status, what):
    if status != OK:
        raise SdhipError(status, what)


def desc(t):
    """The ggml descriptor of a torch tensor of at most 4 dimensions."""
    if t.dim() > 4:
        raise ValueError("at most 4 dimensions")
    d = Tensor()
    if t.dtype == torch.float32:
        d.type, size = TYPE_F32, 4
    elif t.dtype == torch.float16:
        d.type, size = TYPE_F16, 2
    else:
        raise ValueError(f"type {t.dtype}")
    shape = list(t.shape)[::-1]
    strides = [s * size for s in list(t.stride())[::-1]]
    for k in range(4):
        if k < len(shape):
            d.ne[k] = shape[k]
            d.nb[k] = strides[k]
        else:
            d.ne[k] = 1
            d.nb[k] = d.nb[k - 1] * d.ne[k - 1] if k > 0 else size
    d.data = t.data_ptr()
    return d


def view_desc(data_ptr, dtype_code, ne, nb):
    d = Tensor()
    d.type = dtype_code
    for k in range(4):
        d.ne[k] = ne[k]
        d.nb[k] = nb[k]
    d.data = data_ptr
    return d


def epilogue(steps=(), redirect=None, from_redirect=False):
    """steps: ('add'|'mul', tensor) or ('silu', None); redirect: a torch tensor."""
    e = Epilogue()
    e.count = len(steps)
    kinds = {"add": STEP_ADD, "mul": STEP_MUL, "silu": STEP_SILU}
    for i, (kind, operand) in enumerate(steps):
        e.steps[i].kind = kinds[kind]
        if operand is not None:
            e.steps[i].operand = desc(operand)
    if redirect is not None:
        e._redirect_desc = desc(redirect)  # kept alive with the epilogue
        e.redirect = ctypes.pointer(e._redirect_desc)
    e.from_redirect = 1 if from_redirect else 0
    return e


def stream_handle():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def set_tuning(text=""):
    check(load().sdhip_set_tuning(text.encode()), "set_tuning")


def get_tuning(name):
    return load().sdhip_get_tuning(name.encode())


def _work(nbytes, device):
    if nbytes == 0:
        return None, 0
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return buf, nbytes


def mul_mat(w, x, y, chain=None, work=None):
    """y (ne = [N, M...]) = x W^T with the chain; w: [N, K] f16, x: [..., K] f32."""
    lib = load()
    dw, dx, dy = desc(w), desc(x), desc(y)
    size = lib.sdhip_mul_mat_work_size(dw, dx, dy)
    buf = work
    if buf is None:
        buf, _ = _work(size, x.device)
    ptr = buf.data_ptr() if buf is not None else None
    check(lib.sdhip_mul_mat(dw, dx, dy, ctypes.byref(chain) if chain else None, ptr, size, stream_handle()),
          "mul_mat")
    return buf


def mul_mat_gated(w, x, y, out, chain=None, work=None):
    lib = load()
    dw, dx, dy, do = desc(w), desc(x), desc(y), desc(out)
    size = lib.sdhip_mul_mat_work_size(dw, dx, dy)
    buf = work
    if buf is None:
        buf, _ = _work(size, x.device)
    ptr = buf.data_ptr() if buf is not None else None
    check(lib.sdhip_mul_mat_gated(dw, dx, dy, ctypes.byref(chain) if chain else None, do, ptr, size,
                                  stream_handle()), "mul_mat_gated")
    return buf


def conv_params(s0=1, s1=1, p0=0, p1=0, d0=1, d1=1):
    return _I6(s0, s1, p0, p1, d0, d1)


def conv2d_path(kernel, x, y, params):
    return load().sdhip_conv2d_path(desc(kernel), desc(x), desc(y), params)


def conv2d(kernel, x, y, params, chain=None, work=None):
    lib = load()
    dk, dx, dy = desc(kernel), desc(x), desc(y)
    size = lib.sdhip_conv2d_work_size(dk, dx, dy, params)
    buf = work
    if buf is None:
        buf, _ = _work(size, x.device)
    ptr = buf.data_ptr() if buf is not None else None
    check(lib.sdhip_conv2d(dk, dx, dy, params, ctypes.byref(chain) if chain else None, ptr, size,
                           stream_handle()), "conv2d")
    return buf


def attention(q, k, v, y, scale, work=None):
    lib = load()
    dq, dk, dv, dy = desc(q), desc(k), desc(v), desc(y)
    size = lib.sdhip_attention_work_size(dq, dk, dv, dy)
    buf = work
    if buf is None:
        buf, _ = _work(size, q.device)
    ptr = buf.data_ptr() if buf is not None else None
    check(lib.sdhip_attention(dq, dk, dv, dy, scale, 0.0, 0.0, ptr, size, stream_handle()), "attention")
    return buf


def group_norm(x, y, groups, eps, chain=None, work=None):
    lib = load()
    dx, dy = desc(x), desc(y)
    size = lib.sdhip_group_norm_work_size(dx, dy, groups)
    buf = work
    if buf is None:
        buf, _ = _work(size, x.device)
    ptr = buf.data_ptr() if buf is not None else None
    check(lib.sdhip_group_norm(dx, dy, groups, eps, ctypes.byref(chain) if chain else None, ptr, size,
                               stream_handle()), "group_norm")
    return buf


def group_norm_static(x, y, groups, eps, chain=None):
    """sdhip_group_norm_static: no work buffer, the library's static scratch."""
    check(load().sdhip_group_norm_static(desc(x), desc(y), groups, eps, ctypes.byref(chain) if chain else None,
                                         stream_handle()), "group_norm_static")


def norm(x, y, eps, chain=None):
    check(load().sdhip_norm(desc(x), desc(y), eps, ctypes.byref(chain) if chain else None, stream_handle()),
          "norm")


def profile_enable(on=True):
    load().sdhip_profile_enable(1 if on else 0)


def profile_reset():
    load().sdhip_profile_reset()


def profile_collect():
    """{kernel name: (total ms, launches)} of the launches since the reset."""
    lib = load()
    count = lib.sdhip_profile_collect()
    out = {}
    for i in range(count):
        name = ctypes.c_char_p()
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        if lib.sdhip_profile_entry(i, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(n)):
            out[name.value.decode()] = (ms.value, n.value)
    return out


def store_arena(buf):
    """Give the library `buf` (a uint8 device tensor, or None) as its store."""
    if buf is None:
        load().sdhip_store_arena(None, 0)
    else:
        load().sdhip_store_arena(ctypes.c_void_p(buf.data_ptr()), buf.numel())


def store_used():
    n = ctypes.c_size_t()
    used = load().sdhip_store_used(ctypes.byref(n))
    return used, n.value


def forget(t):
    """sdhip_forget over the memory of tensor t."""
    load().sdhip_forget(ctypes.c_void_p(t.data_ptr()), t.numel() * t.element_size())
