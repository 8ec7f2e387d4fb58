"""numpy front end of the C oracle (oracle/oracle.h) for the tests.

The oracle is the checker: these functions compute the float64 references and
the single-precision restatements the tests compare the HIP library with.
"""

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")

_f = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_d = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64 = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32 = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8 = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_s8 = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_L = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} is missing: make -C oracle")
        L = ctypes.CDLL(ORACLE_SO)
        L.oracle_exponential.restype = _F
        L.oracle_exponential.argtypes = [_F]
        L.oracle_silu.restype = _F
        L.oracle_silu.argtypes = [_F]
        L.oracle_gelu.restype = _F
        L.oracle_gelu.argtypes = [_F]
        L.oracle_silu_array.argtypes = [_f, _L]
        L.oracle_exponential_array.argtypes = [_f, _f, _L]
        L.oracle_gelu_array.argtypes = [_f, _f, _L]
        L.oracle_port_mul_mat.argtypes = [_f, _f, ctypes.c_void_p, _L, _L, _L, _f, _I]
        L.oracle_port_available.restype = _I
        _v = ctypes.c_void_p
        for name in ("oracle_port_winograd4", "oracle_port_winograd2"):
            getattr(L, name).argtypes = [_f, _L, _L, _L, _L, _f, _L, _I, _I, _v, _v, _f, _I]
        L.oracle_port_conv2d.argtypes = [_f, _L, _L, _L, _L, _f, _L, _L, _L, _I, _I, _I, _I, _v, _v, _f, _I]
        L.oracle_port_group_norm.argtypes = [_f, _f, _L, _L, _L, _I, _F, _v, _v, _I, _I]
        L.oracle_port_norm.argtypes = [_f, _f, _L, _L, _F, _v, _v, _I]
        L.oracle_port_attention.argtypes = [_f, _f, _f, _L, _L, _L, _L, _L, _L, _F, _f, _I]
        L.oracle_port_quantized_attention.argtypes = [_f, _f, _f, _L, _L, _L, _L, _L, _L, _L, _F, _L, _I, _I, _L,
                                                      _f, _I]
        L.oracle_port_qweights_bytes.restype = ctypes.c_size_t
        L.oracle_port_qweights_bytes.argtypes = [_L, _L, _L]
        L.oracle_port_pack_qweights.argtypes = [_s8, _f, _f, _L, _L, _L, _u8]
        L.oracle_port_quantized_linear.argtypes = [_f, _L, _L, _u8, _L, _L, _I, _v, _f, _I, _v, _I]
        L.oracle_port_gated.argtypes = [_f, _L, _L, _f, _I]
        L.oracle_port_fma_peak.restype = ctypes.c_double
        L.oracle_port_fma_peak.argtypes = [_I, ctypes.c_double]
        L.oracle_gated_gelu_array.argtypes = [_f, _f, _f, _L]
        L.oracle_exact_mul_mat.argtypes = [_f, _L, _f, _L, _L, _L, _L, _d, _d]
        L.oracle_exact_conv2d.argtypes = [_f, _L, _L, _L, _L, _f, _L, _L, _L, _I, _I, _I, _I, _I, _I, _L, _L, _d, _d]
        L.oracle_exact_conv2d_at.argtypes = [_f, _L, _L, _L, _L, _f, _L, _L, _L, _I, _I, _I, _I, _I, _I, _L, _L,
                                             _i64, _L, _d, _d]
        L.oracle_exact_attention.argtypes = [_f, _f, _f, _L, _L, _L, _L, _L, _L, _L, _F, _d, _d]
        L.oracle_exact_attention_at.argtypes = [_f, _f, _f, _L, _L, _L, _L, _L, _L, _L, _F, _i64, _L, _d, _d]
        L.oracle_exact_gated.argtypes = [_f, _f, ctypes.c_void_p, _L, _L, _L, _d, _d]
        L.oracle_group_norm.argtypes = [_f, _f, _L, _L, _L, _L, _I, _F]
        L.oracle_norm.argtypes = [_f, _f, _L, _L, _F]
        L.oracle_quantize_input_row.argtypes = [_f, _L, _L, _I, _u8, ctypes.POINTER(_F), ctypes.POINTER(_F)]
        L.oracle_quantize_weights.argtypes = [_f, _L, _L, _L, _L, _I, _I, _s8, _f, _f, _i32]
        L.oracle_quantized_mul_mat.argtypes = [_f, _f, _L, _L, _L, _L, _I, _I, _I, ctypes.c_void_p, _f,
                                               _u8, _f, _f, _s8, _f, _f, _i32]
        L.oracle_quantized_conv2d.argtypes = [_f, _L, _L, _L, _L, _f, _L, _L, _L, _I, _I, _I, _I, _I, _I, _L, _L, _L,
                                              _I, _I, _I, ctypes.c_void_p, _f]
        L.oracle_quantized_winograd2.argtypes = [_f, _L, _L, _L, _L, _f, _L, _I, _I, _L, _L, _L, _I, _I, _I, _L, _I, _f]
        L.oracle_set_plant.argtypes = [_I]
        L.oracle_quantized_attention.argtypes = [_f, _f, _f, _L, _L, _L, _L, _L, _L, _L, _F, _L, _I, _I, _L, _f]
        _lib = L
    return _lib


REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref_scalar_math.so")
_ref = None


def ref_lib():
    """The reference's own sources/scalar_math.h, compiled unmodified by
    oracle/ref.mk into oracle/_ref; None where it was not built (the
    reference checkout is absent)."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        L = ctypes.CDLL(REF_SO)
        for name in ("ref_exponential", "ref_silu", "ref_gelu"):
            getattr(L, name).restype = _F
            getattr(L, name).argtypes = [_F]
        for name in ("ref_exponential_array", "ref_silu_array", "ref_gelu_array"):
            getattr(L, name).argtypes = [_f, _f, _L]
        _ref = L
    return _ref


def ref_array(name, x):
    """The reference's exponential / silu / gelu of each number of x."""
    x = c32(x)
    out = np.empty_like(x)
    getattr(ref_lib(), f"ref_{name}_array")(x, out, x.size)
    return out


def exponential(x):
    x = c32(x)
    out = np.empty_like(x)
    lib().oracle_exponential_array(x, out, x.size)
    return out


def gelu(x):
    x = c32(x)
    out = np.empty_like(x)
    lib().oracle_gelu_array(x, out, x.size)
    return out


def port_mul_mat(w, x, bias=None, threads=1):
    """port.c's packed single-precision GEMM (the CPU baseline of MUL_MAT):
    w [N, K], x [M, K] -> y [M, N] = x w^T (+ bias)."""
    w, x = c32(w), c32(x)
    N, K = w.shape
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    bp = None
    if bias is not None:
        bias = c32(bias)
        bp = bias.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_port_mul_mat(w, x, bp, M, N, K, y, threads)
    return y


def c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _opt(a):
    """A float32 array's pointer, or NULL for None (kept alive by the caller)."""
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def port_available():
    """Whether this host runs port.c (AVX-512 with VNNI)."""
    return bool(lib().oracle_port_available())


def port_winograd(x, w, pad, bias=None, residual=None, four=True, threads=1, out=None):
    """port.c's Winograd F(4x4, 3x3) (four) or F(2x2, 3x3): x [n, ic, h, w],
    w [oc, ic, 3, 3] -> y [n, oc, oh, ow] (+ bias [oc], + residual)."""
    x, w = c32(x), c32(w)
    n, ic, h, wd = x.shape
    oc = w.shape[0]
    bias = None if bias is None else c32(bias)
    residual = None if residual is None else c32(residual)
    y = out if out is not None else np.empty((n, oc, h + 2 * pad - 2, wd + 2 * pad - 2), np.float32)
    fn = lib().oracle_port_winograd4 if four else lib().oracle_port_winograd2
    fn(x, n, ic, h, wd, w, oc, pad, pad, _opt(bias), _opt(residual), y, threads)
    return y


def port_conv2d(x, w, stride=1, pad=0, bias=None, residual=None, threads=1, out=None):
    """port.c's direct convolution: x [n, ic, h, w], w [oc, ic, kh, kw]."""
    x, w = c32(x), c32(w)
    n, ic, h, wd = x.shape
    oc, _, kh, kw = w.shape
    oh, ow = (h + 2 * pad - kh) // stride + 1, (wd + 2 * pad - kw) // stride + 1
    bias = None if bias is None else c32(bias)
    residual = None if residual is None else c32(residual)
    y = out if out is not None else np.empty((n, oc, oh, ow), np.float32)
    lib().oracle_port_conv2d(x, n, ic, h, wd, w, oc, kh, kw, stride, stride, pad, pad, _opt(bias), _opt(residual), y,
                             threads)
    return y


def port_group_norm(x, groups, eps, gamma=None, beta=None, silu=False, threads=1):
    x = c32(x)
    gamma = None if gamma is None else c32(gamma)
    beta = None if beta is None else c32(beta)
    y = np.empty_like(x)
    n, c = x.shape[:2]
    lib().oracle_port_group_norm(x, y, n, c, x[0, 0].size, groups, eps, _opt(gamma), _opt(beta), int(silu), threads)
    return y


def port_norm(x, eps, gamma=None, beta=None, threads=1):
    x = c32(x)
    gamma = None if gamma is None else c32(gamma)
    beta = None if beta is None else c32(beta)
    y = np.empty_like(x)
    lib().oracle_port_norm(x, y, x.size // x.shape[-1], x.shape[-1], eps, _opt(gamma), _opt(beta), threads)
    return y


def port_attention(q, k, v, scale, threads=1):
    """port.c's attention: q [b, lq, h, d], k [b, lk, h, d], v [b, lk, h, dv]
    -> y [b, lq, h, dv]."""
    q, k, v = c32(q), c32(k), c32(v)
    b, lq, h, d = q.shape
    lk, dv = k.shape[1], v.shape[3]
    y = np.empty((b, lq, h, dv), np.float32)
    lib().oracle_port_attention(q, k, v, b, lq, lk, h, d, dv, scale, y, threads)
    return y


def port_quantized_attention(q, k, v, scale, group=64, levels=255, wmax=127, key_block=256, threads=1):
    """port.c's bits-mode self-attention (attention.cc:612-824): q [b, lq, h,
    d], k [b, lk, hk, d], v [b, lk, hk, dv] -> y [b, lq, h, dv]; key_block the
    exponentials' stretch, a multiple of the group."""
    q, k, v = c32(q), c32(k), c32(v)
    b, lq, h, d = q.shape
    lk, hk, dv = k.shape[1], k.shape[2], v.shape[3]
    y = np.empty((b, lq, h, dv), np.float32)
    lib().oracle_port_quantized_attention(q, k, v, b, lq, lk, h, hk, d, dv, scale, group, levels, wmax, key_block, y,
                                          threads)
    return y


def port_pack_qweights(wq, ws, wo, group):
    """The quantized weights (quantize_weights' q, scale, offset) packed for
    port_quantized_linear."""
    n, kp = wq.shape
    groups = kp // group
    packed = np.zeros(lib().oracle_port_qweights_bytes(n, groups, group), np.uint8)
    lib().oracle_port_pack_qweights(np.ascontiguousarray(wq), c32(ws), c32(wo), n, groups, group, packed)
    return packed


def port_quantized_linear(x, packed, n, group=64, levels=255, bias=None, gated=False, threads=1):
    """port.c's bits-mode MUL_MAT: x [M, K] -> y [M, n] (+ bias); with gated,
    (y, y[:, :n/2] GELU(y[:, n/2:]))."""
    x = c32(x)
    m, k = x.shape
    bias = None if bias is None else c32(bias)
    y = np.empty((m, n), np.float32)
    out = np.empty((m, n // 2), np.float32) if gated else None
    lib().oracle_port_quantized_linear(x, m, k, packed, n, group, levels, _opt(bias), y, int(gated), _opt(out),
                                       threads)
    return (y, out) if gated else y


def port_gated(y, threads=1):
    """port.c's GEGLU of a product y [M, N]: y[:, :N/2] GELU(y[:, N/2:])."""
    y = c32(y)
    m, n = y.shape
    out = np.empty((m, n // 2), np.float32)
    lib().oracle_port_gated(y, m, n, out, threads)
    return out


def port_fma_peak(threads, seconds=0.3):
    """The host's single-precision FMA rate on `threads` threads, GFLOP/s."""
    return lib().oracle_port_fma_peak(threads, seconds)


def metric(y, exact, mag):
    """The reference's measure (tests/ops_test.cc:173-211): the largest
    |y - exact| / (sum of product magnitudes, or 1 where that is 0)."""
    y = np.asarray(y, dtype=np.float64).reshape(-1)
    exact = np.asarray(exact, dtype=np.float64).reshape(-1)
    mag = np.asarray(mag, dtype=np.float64).reshape(-1)
    scale = np.where(mag > 0, mag, 1.0)
    e = np.abs(y - exact) / scale
    if not np.all(np.isfinite(e)):
        return float("inf")
    return float(e.max()) if e.size else 0.0


def exact_mul_mat(w, x):
    """w [N, K] (float, FP16 widened), x [M, K] -> (y, mag) [M, N] float64."""
    w, x = c32(w), c32(x)
    N, K = w.shape
    M = x.shape[0]
    y = np.empty((M, N), np.float64)
    mag = np.empty((M, N), np.float64)
    lib().oracle_exact_mul_mat(w, K, x, K, M, N, K, y, mag)
    return y, mag


def exact_conv2d(x, w, s0, s1, p0, p1, d0, d1, index=None):
    """x [n, ic, ih, iw], w [oc, ic, kh, kw] -> (y, mag) [n, oc, oh, ow], or at
    the flat indices `index` of that layout."""
    x, w = c32(x), c32(w)
    n, ic, ih, iw = x.shape
    oc, _, kh, kw = w.shape
    oh = (ih + 2 * p1 - d1 * (kh - 1) - 1) // s1 + 1
    ow = (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1
    if index is None:
        y = np.empty((n, oc, oh, ow), np.float64)
        mag = np.empty_like(y)
        lib().oracle_exact_conv2d(x, n, ic, ih, iw, w, oc, kh, kw, s0, s1, p0, p1, d0, d1, oh, ow, y, mag)
        return y, mag
    index = np.ascontiguousarray(index, dtype=np.int64)
    y = np.empty(index.size, np.float64)
    mag = np.empty(index.size, np.float64)
    lib().oracle_exact_conv2d_at(x, n, ic, ih, iw, w, oc, kh, kw, s0, s1, p0, p1, d0, d1, oh, ow, index, index.size,
                                 y, mag)
    return y, mag


def exact_attention(q, k, v, scale, queries=None):
    """q [b, lq, h, d], k [b, lk, hk, d], v [b, lk, hk, dv] -> (y, mag)
    [b, lq, h, dv], or [count, dv] for the flat queries (bi * h + hi) * lq + i."""
    q, k, v = c32(q), c32(k), c32(v)
    b, lq, h, d = q.shape
    _, lk, hk, dv = v.shape
    if queries is None:
        y = np.empty((b, lq, h, dv), np.float64)
        mag = np.empty_like(y)
        lib().oracle_exact_attention(q, k, v, d, dv, lq, lk, h, hk, b, scale, y, mag)
        return y, mag
    queries = np.ascontiguousarray(queries, dtype=np.int64)
    y = np.empty((queries.size, dv), np.float64)
    mag = np.empty_like(y)
    lib().oracle_exact_attention_at(q, k, v, d, dv, lq, lk, h, hk, b, scale, queries, queries.size, y, mag)
    return y, mag


def exact_gated(w, x, bias):
    """w [2 half, K], x [M, K], bias [2 half] or None -> (y, mag) [M, half]."""
    w, x = c32(w), c32(x)
    M, K = x.shape
    half = w.shape[0] // 2
    y = np.empty((M, half), np.float64)
    mag = np.empty_like(y)
    bp = None
    if bias is not None:
        bias = c32(bias)
        bp = bias.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_exact_gated(w, x, bp, M, half, K, y, mag)
    return y, mag


def group_norm(x, groups, eps):
    """x [ne3, ne2, ne1, ne0] -> the reference's single-precision GROUP_NORM."""
    x = c32(x)
    y = np.empty_like(x)
    ne3, ne2, ne1, ne0 = x.shape
    lib().oracle_group_norm(x, y, ne0, ne1, ne2, ne3, groups, eps)
    return y


def norm(x, eps):
    x = c32(x)
    y = np.empty_like(x)
    ne0 = x.shape[-1]
    lib().oracle_norm(x, y, ne0, x.size // ne0, eps)
    return y


def silu(v):
    """SiLU with the reference's exponential (scalar_math.h:54-56)."""
    out = np.array(v, dtype=np.float32, copy=True, order="C")
    lib().oracle_silu_array(out, out.size)
    return out


def gated_gelu(x, gate):
    """x * GELU(gate) with the reference's GELU (fusion.cc:290-310)."""
    x, gate = c32(x), c32(gate)
    out = np.empty_like(x)
    lib().oracle_gated_gelu_array(x, gate, out, out.size)
    return out


def quantize_input_row(x, group, levels):
    x = c32(x)
    dst = np.zeros(group, np.uint8)
    s, o = _F(), _F()
    lib().oracle_quantize_input_row(x, x.size, group, levels, dst, ctypes.byref(s), ctypes.byref(o))
    return dst, np.float32(s.value), np.float32(o.value)


def quantize_weights(w, group, weight_max, weight_groups):
    w = c32(w)
    rows, k = w.shape
    groups = (k + group - 1) // group
    q = np.zeros((rows, groups * group), np.int8)
    sc = np.zeros((rows, groups), np.float32)
    of = np.zeros((rows, groups), np.float32)
    su = np.zeros((rows, groups), np.int32)
    lib().oracle_quantize_weights(w, k, rows, k, group, weight_max, weight_groups, q, sc, of, su)
    return q, sc, of, su


def quantized_mul_mat(w, x, group=64, input_levels=255, weight_max=127, weight_groups=1, init=None):
    """The reference's bits-mode MUL_MAT, bit for bit: (y, xq, xs, xo, wq, ws, wo, wsum)."""
    w, x = c32(w), c32(x)
    N, K = w.shape
    M = x.shape[0]
    groups = (K + group - 1) // group
    kp = groups * group
    y = np.zeros((M, N), np.float32)
    xq = np.zeros((M, kp), np.uint8)
    xs = np.zeros((M, groups), np.float32)
    xo = np.zeros((M, groups), np.float32)
    wq = np.zeros((N, kp), np.int8)
    ws = np.zeros((N, groups), np.float32)
    wo = np.zeros((N, groups), np.float32)
    wsum = np.zeros((N, groups), np.int32)
    ip = None
    if init is not None:
        init = c32(init)
        ip = init.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_quantized_mul_mat(w, x, M, N, K, group, input_levels, weight_max, weight_groups, ip, y, xq, xs, xo,
                                   wq, ws, wo, wsum)
    return y, xq, xs, xo, wq, ws, wo, wsum


def quantized_attention(q, k, v, scale, group=64, input_levels=255, weight_max=127, key_block=256):
    """The reference's bits-mode self-attention (attention.cc:612-824):
    q [b, lq, h, d], k [b, lk, hk, d], v [b, lk, hk, dv] -> y [b, lq, h, dv].
    key_block: the reference's stretch of keys, max(group, attention_keys
    rounded down to 8 then to the group)."""
    q, k, v = c32(q), c32(k), c32(v)
    b, lq, h, d = q.shape
    _, lk, hk, dv = v.shape
    y = np.zeros((b, lq, h, dv), np.float32)
    lib().oracle_quantized_attention(q, k, v, d, dv, lq, lk, h, hk, b, scale, group, input_levels, weight_max,
                                     key_block, y)
    return y


def quantized_conv2d(x, w, s0, s1, p0, p1, d0, d1, group=64, levels=255, wmax=127, weight_groups=1, init=None):
    """The reference's bits-mode direct convolution (conv2d.cc:338-483), bit
    for bit: x [n, ic, ih, iw], w [oc, ic, kh, kw] -> y [n, oc, oh, ow],
    begun from init (the residual) if given."""
    x, w = c32(x), c32(w)
    n, ic, ih, iw = x.shape
    oc, _, kh, kw = w.shape
    oh = (ih + 2 * p1 - d1 * (kh - 1) - 1) // s1 + 1
    ow = (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1
    y = np.zeros((n, oc, oh, ow), np.float32)
    ip = None
    if init is not None:
        init = c32(init)
        ip = init.ctypes.data_as(ctypes.c_void_p)
    lib().oracle_quantized_conv2d(x, n, ic, ih, iw, w, oc, kh, kw, s0, s1, p0, p1, d0, d1, oh, ow, group, levels, wmax,
                                  weight_groups, ip, y)
    return y


class planted:
    """A mistake planted in the oracle's quantized convolutions for the length
    of a `with` block (oracle_set_plant: 1 tap-major columns, 2 Winograd's
    weights over every input channel, 3 over stretches of one group), so that
    a test can show its check sees it."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        lib().oracle_set_plant(self.mode)

    def __exit__(self, *exc):
        lib().oracle_set_plant(0)


def quantized_winograd2(x, w, p0, p1, group=64, levels=255, wmax=127, weight_groups=1, stretch=64, init=None):
    """The reference's bits-mode Winograd F(2x2) (winograd.cc:1826-2103), bit
    for bit: x [n, ic, ih, iw], w [oc, ic, 3, 3] -> y [n, oc, oh, ow], added to
    init (the residual, from_redirect) if given."""
    x, w = c32(x), c32(w)
    n, ic, ih, iw = x.shape
    oc = w.shape[0]
    oh, ow = ih + 2 * p1 - 2, iw + 2 * p0 - 2
    y = np.zeros((n, oc, oh, ow), np.float32) if init is None else np.array(c32(init), copy=True)
    lib().oracle_quantized_winograd2(x, n, ic, ih, iw, w, oc, p0, p1, oh, ow, group, levels, wmax, weight_groups,
                                     stretch, 0 if init is None else 1, y)
    return y
