"""The library's host side, on the CPU: it loads, exports every entry point
include/sdhip.h declares, parses the tuning as the reference's SDASM_TUNE
does, and takes or leaves operations by the reference's predicates
(hooks.cc:29-55 and the *_supported functions) -- none of which touches a
device.  No compute call is made here."""

import ctypes
import os
import re
import subprocess
import sys

import pytest

import sdhip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "sdhip.h")).read()
    return sorted(set(re.findall(r"\b(sdhip_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = sdhip.load()
    names = declared()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), f"{name} declared in sdhip.h but not exported"
    bound = {n for n, _, _ in sdhip.SIGNATURES}
    assert set(names) == bound, "the Python binding and the header list the same entry points"


def test_tuning_parses_like_sdasm_tune():
    try:
        sdhip.set_tuning("bits=8,group=128,weight_group=0,winograd=1")
        assert sdhip.get_tuning("bits") == 8
        assert sdhip.get_tuning("group") == 128
        assert sdhip.get_tuning("weight_group") == 0
        assert sdhip.get_tuning("winograd") == 1
        assert sdhip.get_tuning("no_such") == -1
        with pytest.raises(sdhip.SdhipError):
            sdhip.set_tuning("no_such=1")
        with pytest.raises(sdhip.SdhipError):
            sdhip.set_tuning("bits=eight")
    finally:
        sdhip.set_tuning("")
    # The reference's defaults (sources/kernels.h:91-135).
    for name, value in (("bits", 0), ("input_bits", 8), ("group", 64), ("weight_group", 1), ("quantize", 7),
                        ("winograd", 2), ("winograd_positions", 1024), ("winograd4_positions", 256),
                        ("winograd_small_tiles", 256), ("fuse", 1), ("attention_keys", 256),
                        ("attention_fp32", 0), ("attention_generic", 0), ("winograd_splits", 0)):
        assert sdhip.get_tuning(name) == value


def test_tuning_takes_every_reference_name_and_checks_its_own():
    """Every name of the reference's Tuning (kernels.h:91-135) is taken with
    its default, so that SDASM_TUNE strings carry over; this library's own
    names take only their documented values."""
    ref = {"conv_kc": 256, "conv_mc": 480, "conv_nc": 128, "conv_rows_outer": 0, "conv_shared_columns": 1024,
           "conv_columns_bytes": 4 << 20, "mul_mat_kc": 256, "mul_mat_mc": 96, "mul_mat_shared_rows": 1024,
           "amx_kc": 256, "amx_mc": 128, "amx_attention": 0, "amx_queries": 64, "amx_fp16": 1,
           "attention_queries": 32, "attention_keys": 256, "attention_sum_keys": 32, "attention_sum_dims": 40,
           "winograd": 2, "winograd_positions": 1024, "winograd4_positions": 256, "winograd_kc": 256,
           "winograd_mc": 512, "winograd_tiles": 64, "winograd_small_tiles": 256, "winograd_small_mc": 48,
           "winograd_small_kc": 128, "prefetch": 1, "wide": 1, "bf16": 0, "fuse": 1, "fuse_residual": 1,
           "guided": 1, "store_forget": 1, "bits": 0, "input_bits": 8, "group": 64, "weight_group": 1,
           "quantize": 7, "half_format": 0, "todo": 0, "todo_tokens": 2048}
    sdhip.set_tuning("")
    for name, value in ref.items():
        assert sdhip.get_tuning(name) == value, name
    try:
        sdhip.set_tuning("conv_kc=128,amx_fp16=0,fuse_residual=0,todo=2,todo_tokens=100,group=1000,bits=3")
        assert sdhip.get_tuning("conv_kc") == 128 and sdhip.get_tuning("todo_tokens") == 100
        for bad in ("gemm_stages=3", "gemm_tiles=13", "winograd_fp32=2", "attention_fp32=-1", "attention_generic=5",
                    "winograd_splits=-2", "fuse=99999999999", "gemm_core=4", "gemm_core=2",
                    "mul_mat_panels=3", "conv_panels=2"):
            with pytest.raises(sdhip.SdhipError):
                sdhip.set_tuning(bad)
        for good in ("gemm_stages=4", "gemm_tiles=21", "gemm_tiles=12", "gemm_core=1", "gemm_core=0", "gemm_core=3", "winograd_fp32=1", "winograd_splits=3", "bits=8",
                     "bits=16", "mul_mat_panels=2", "conv_panels=0"):
            sdhip.set_tuning(good)
    finally:
        sdhip.set_tuning("")


FAKE = 1 << 20  # a data pointer the predicates never dereference


def tensor(dtype, shape, data=FAKE):
    """A contiguous descriptor of a torch-ordered shape."""
    size = 4 if dtype == sdhip.TYPE_F32 else 2
    ne = list(reversed(shape)) + [1] * (4 - len(shape))
    nb = [size]
    for k in range(1, 4):
        nb.append(nb[k - 1] * ne[k - 1])
    return sdhip.view_desc(data, dtype, ne, nb)


F32, F16 = sdhip.TYPE_F32, sdhip.TYPE_F16


def test_mul_mat_predicate():
    lib = sdhip.load()
    w, x, y = tensor(F16, (320, 320)), tensor(F32, (2, 4096, 320)), tensor(F32, (2, 4096, 320))
    assert lib.sdhip_mul_mat_supported(w, x, y)
    assert lib.sdhip_mul_mat_work_size(w, x, y) == 0
    # Fewer than 16 rows, or K under 16, are left to the caller (mul_mat.cc:192-193).
    assert not lib.sdhip_mul_mat_supported(w, tensor(F32, (15, 320)), tensor(F32, (15, 320)))
    assert not lib.sdhip_mul_mat_supported(tensor(F16, (8, 8)), tensor(F32, (40, 8)), tensor(F32, (40, 8)))
    # Single-precision weights are taken, as the reference takes them (mul_mat.cc:190).
    assert lib.sdhip_mul_mat_supported(tensor(F32, (320, 320)), x, y)
    try:
        sdhip.set_tuning("bits=8")
        assert lib.sdhip_mul_mat_work_size(w, x, y) > 0
        small = tensor(F32, (255, 320))
        assert lib.sdhip_mul_mat_work_size(w, small, small) == 0  # under 256 rows: not quantized
    finally:
        sdhip.set_tuning("")


def conv_path(w_, h_, ic, oc, k, s, p, n, tuning=""):
    lib = sdhip.load()
    oh, ow = (h_ + 2 * p - k) // s + 1, (w_ + 2 * p - k) // s + 1
    kern = tensor(F16, (oc, ic, k, k))
    x = tensor(F32, (n, ic, h_, w_))
    y = tensor(F32, (n, oc, oh, ow))
    sdhip.set_tuning(tuning)
    try:
        return lib.sdhip_conv2d_path(kern, x, y, sdhip.conv_params(s, s, p, p, 1, 1))
    finally:
        sdhip.set_tuning("")


def test_conv2d_path_selection():
    """winograd_supported, four, small (winograd.cc:194-196, 1204-1206,
    2107-2123) and the direct fallback (hooks.cc:36-41)."""
    assert conv_path(64, 64, 320, 320, 3, 1, 1, 2) == 4    # configs[1]: F(4x4)
    assert conv_path(8, 8, 1280, 1280, 3, 1, 1, 2) == 2    # configs[2]: F(2x2), small images
    assert conv_path(32, 32, 640, 1280, 1, 1, 0, 2) == 0   # 1x1: direct
    assert conv_path(33, 33, 24, 30, 3, 2, 1, 1) == 0      # stride 2: direct
    assert conv_path(40, 20, 8, 8, 3, 1, 1, 1) == 4        # 800 outputs, 200 tiles: small, >= 256 outputs: F(4x4)
    assert conv_path(15, 9, 8, 8, 3, 1, 1, 2) == 2         # 135 outputs, 80 tiles: small, F(2x2)
    assert conv_path(80, 40, 8, 8, 3, 1, 1, 1) == 4        # 3200 outputs: F(4x4), not small
    assert conv_path(64, 64, 320, 320, 3, 1, 1, 2, "winograd=1") == 2
    assert conv_path(64, 64, 320, 320, 3, 1, 1, 2, "winograd=0") == 0
    assert conv_path(64, 64, 320, 320, 3, 1, 3, 2) == 0    # padding 3: not Winograd


def test_attention_and_norm_predicates():
    lib = sdhip.load()
    q = tensor(F32, (2, 8, 4096, 40))
    y = tensor(F32, (2, 4096, 8, 40))
    assert lib.sdhip_attention_supported(q, q, q, y, 0.0, 0.0)
    assert not lib.sdhip_attention_supported(q, q, q, y, 0.0, 30.0)   # a soft cap
    assert not lib.sdhip_attention_supported(q, q, q, y, 8.0, 0.0)    # ALiBi
    # Heads of any size are taken, as attention_supported takes them
    # (attention.cc:828-845): 512 (the VAE's) by chunks of the dimensions,
    # wider ones with their values in slices; in the bits mode, where the
    # quantized form applies (256 keys or more), up to 512.
    vae = tensor(F32, (1, 1, 4096, 512))
    assert lib.sdhip_attention_supported(vae, vae, vae, tensor(F32, (1, 4096, 1, 512)), 0.0, 0.0)
    big = tensor(F32, (1, 1, 4096, 640))
    assert lib.sdhip_attention_supported(big, big, big, tensor(F32, (1, 4096, 1, 640)), 0.0, 0.0)
    few = tensor(F32, (1, 1, 200, 640))
    try:
        sdhip.set_tuning("bits=8")
        assert not lib.sdhip_attention_supported(big, big, big, tensor(F32, (1, 4096, 1, 640)), 0.0, 0.0)
        assert lib.sdhip_attention_supported(big, few, few, tensor(F32, (1, 4096, 1, 640)), 0.0, 0.0)
        assert lib.sdhip_attention_supported(vae, vae, vae, tensor(F32, (1, 4096, 1, 512)), 0.0, 0.0)
    finally:
        sdhip.set_tuning("")
    x = tensor(F32, (2, 1280, 8, 8))
    assert lib.sdhip_group_norm_supported(x, x, 32)
    assert not lib.sdhip_group_norm_supported(x, x, 0)
    assert lib.sdhip_norm_supported(tensor(F32, (2, 988, 1280)), tensor(F32, (2, 988, 1280)))


def test_quantized_attention_takes_wide_heads_and_any_group():
    """In the bits mode the quantized form takes what attention_supported
    takes (attention.cc:828-845): heads of up to 512 dimensions and every
    group quant() gives, a multiple of 4 up to 1024 (quant.cc:59-67)."""
    lib = sdhip.load()
    vae = tensor(F32, (1, 1, 4096, 512))
    y = tensor(F32, (1, 4096, 1, 512))
    for tuning in ("bits=8", "bits=8,group=20", "bits=8,group=4", "bits=8,group=1024", "bits=8,group=3000"):
        sdhip.set_tuning(tuning)
        try:
            assert lib.sdhip_attention_supported(vae, vae, vae, y, 0.0, 0.0), tuning
            assert lib.sdhip_attention_work_size(vae, vae, vae, y) > 0, tuning
        finally:
            sdhip.set_tuning("")


def test_attention_work_size():
    """The split form takes the keys and values split into tiles of 32 keys in
    the work buffer: per (image, head) and tile at head size 40, the keys'
    high FP16 parts in 32 rows of 48 + 8 halves, their low parts in 32 rows
    of 32 + 8 (the last 8 dimensions keep theirs in the high rows' padding),
    the values' high parts in 64 rows of 32 + 8 halves and their low parts in
    32 (the last tile's are rows of the high parts) -- 13824 bytes, 14336 in
    whole KB; the other forms take none."""
    lib = sdhip.load()
    halves = 32 * (48 + 8) + 32 * (32 + 8) + 64 * (32 + 8) + 32 * (32 + 8)
    record = (2 * halves + 1023) // 1024 * 1024
    assert record == 14336
    q = tensor(F32, (2, 8, 4096, 40))
    k = tensor(F32, (2, 8, 4096, 40))
    y = tensor(F32, (2, 4096, 8, 40))
    assert lib.sdhip_attention_work_size(q, k, k, y) == 2 * 8 * 128 * record
    k77 = tensor(F32, (2, 8, 77, 40))
    assert lib.sdhip_attention_work_size(q, k77, k77, y) == 2 * 8 * 3 * record
    try:
        sdhip.set_tuning("attention_fp32=1")
        assert lib.sdhip_attention_work_size(q, k, k, y) == 0
        sdhip.set_tuning("attention_generic=1")
        assert lib.sdhip_attention_work_size(q, k, k, y) == 0
    finally:
        sdhip.set_tuning("")
    k16 = tensor(F16, (2, 8, 4096, 40))
    assert lib.sdhip_attention_work_size(q, k16, k16, y) == 0  # FP16 keys: the generic form


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_single_precision_weights_taken():
    """MUL_MAT and CONV_2D take single-precision weights as the reference
    does (mul_mat.cc:190; conv2d.cc:325-326); a 3x3 kernel of single
    precision takes F(2x2) where an FP16 one takes F(4x4)
    (winograd.cc:1204-1206).  Descriptors only: nothing is computed."""
    lib = sdhip.load()
    w = tensor(sdhip.TYPE_F32, (17, 32))
    x = tensor(sdhip.TYPE_F32, (40, 32))
    y = tensor(sdhip.TYPE_F32, (40, 17))
    assert lib.sdhip_mul_mat_supported(w, x, y) == 1
    assert lib.sdhip_mul_mat_work_size(w, x, y) > 0  # the split weights
    k32 = tensor(sdhip.TYPE_F32, (320, 320, 3, 3))
    k16 = tensor(sdhip.TYPE_F16, (320, 320, 3, 3))
    img = tensor(sdhip.TYPE_F32, (2, 320, 64, 64))
    out = tensor(sdhip.TYPE_F32, (2, 320, 64, 64))
    params = sdhip.conv_params(1, 1, 1, 1, 1, 1)
    assert lib.sdhip_conv2d_supported(k32, img, out, params) == 1
    assert lib.sdhip_conv2d_path(k16, img, out, params) == 4
    assert lib.sdhip_conv2d_path(k32, img, out, params) == 2


def test_quantized_convolutions_taken():
    """In the bits mode (quantize & 2) convolutions are taken: those Winograd
    takes as F(2x2) with quantized products, even where single precision
    takes F(4x4) (winograd.cc:2230-2244); the others directly
    (conv2d.cc:338-483); each with a work buffer for its quantized operands."""
    lib = sdhip.load()
    k16 = tensor(F16, (320, 320, 3, 3))
    img = tensor(F32, (2, 320, 64, 64))
    out = tensor(F32, (2, 320, 64, 64))
    params = sdhip.conv_params(1, 1, 1, 1, 1, 1)
    assert lib.sdhip_conv2d_path(k16, img, out, params) == 4
    try:
        sdhip.set_tuning("bits=8")
        assert lib.sdhip_conv2d_supported(k16, img, out, params) == 1
        assert lib.sdhip_conv2d_path(k16, img, out, params) == 2
        assert lib.sdhip_conv2d_work_size(k16, img, out, params) > 0
        sdhip.set_tuning("bits=8,quantize=5")  # not the convolutions: single precision again
        assert lib.sdhip_conv2d_path(k16, img, out, params) == 4
    finally:
        sdhip.set_tuning("")


def test_misaligned_work_buffer_refused():
    """Every entry point that takes a work buffer refuses one that is not
    16-byte aligned (its kernels move 16-byte vectors and doubles through it),
    before anything is launched: SDHIP_ERROR and a message that says so."""
    lib = sdhip.load()
    big = 1 << 40
    odd = FAKE + 8  # 8-byte aligned, not 16
    calls = []
    q = tensor(F32, (2, 8, 4096, 40))
    calls.append(lambda: lib.sdhip_attention(q, q, q, tensor(F32, (2, 4096, 8, 40)), 0.158, 0.0, 0.0,
                                             odd, big, None))
    kern, x, y = tensor(F16, (320, 320, 3, 3)), tensor(F32, (2, 320, 64, 64)), tensor(F32, (2, 320, 64, 64))
    calls.append(lambda: lib.sdhip_conv2d(kern, x, y, sdhip.conv_params(1, 1, 1, 1, 1, 1), None, odd, big, None))
    g = tensor(F32, (2, 1280, 32, 32))
    calls.append(lambda: lib.sdhip_group_norm(g, g, 32, 1e-5, None, odd, big, None))
    w, xm = tensor(F16, (320, 320)), tensor(F32, (2, 4096, 320))
    for call, tuning in zip(calls + [lambda: lib.sdhip_mul_mat(w, xm, xm, None, odd, big, None)],
                            ["", "", "", "bits=8"]):
        sdhip.set_tuning(tuning)
        try:
            assert call() == sdhip.ERROR
            assert b"16-byte aligned" in lib.sdhip_last_error()
        finally:
            sdhip.set_tuning("")
