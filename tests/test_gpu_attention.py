"""FLASH_ATTN_EXT on the device against the float64 oracle (the textbook
softmax in double, ops_test.cc:517-553) by the reference's metric, at the
reference's own cases (ops_test.cc:925-938) and the SD1.5 attention of the
bench configuration (at full size, a sample of the queries)."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten

BOUND = 1e-6  # attention, |error| / sum |products| against float64

# d, lq, lk, h, hk, b, FP16 keys and values
CASES = [
    (40, 300, 4096, 2, 2, 2, False),   # SD1.5 self-attention at 64x64, fewer queries and heads
    (40, 200, 77, 2, 2, 2, False),     # its cross-attention: 77 tokens
    (80, 100, 1024, 2, 2, 1, False),
    (160, 64, 256, 2, 2, 2, False),
    (13, 37, 29, 4, 2, 3, False),      # edges: no multiple of a tile, heads sharing keys
    (64, 50, 100, 2, 1, 1, True),      # FP16 keys and values
    (64, 988, 988, 2, 2, 1, False),    # SDXL's heads of 64
    (32, 130, 200, 3, 3, 1, False),    # the fast form's other head sizes, ragged queries and keys
    (96, 129, 65, 2, 1, 2, False),
    (128, 70, 300, 2, 2, 1, False),
    (64, 257, 1000, 4, 2, 1, False),   # heads sharing keys in the fast form
    (40, 1, 1, 1, 1, 1, False),        # one query, one key
    (512, 100, 70, 1, 1, 1, False),    # the VAE's heads of 512, by chunks of the dimensions
    (384, 65, 130, 2, 1, 2, True),     # wide heads sharing keys, FP16 keys and values
    (300, 33, 47, 2, 2, 1, False),     # wide heads of no multiple of the chunk or of 16
    (320, 64, 1000, 1, 1, 1, False),   # wide heads, the keys in three splits (the last ragged) merged
    (288, 40, 700, 2, 1, 1, True),     # two splits, heads sharing FP16 keys and values
    (640, 70, 300, 2, 1, 1, False),    # past 512: the values in two slices
    (1100, 33, 1000, 1, 1, 1, True),   # three slices, the last ragged, keys in splits, FP16 keys and values
]


def attention_case(gpu, d, lq, lk, h, hk, b, half, seed, dist="uniform"):
    r = rng(seed)
    if dist == "uniform":
        q = uniform(r, (b, lq, h, d), 1.0)
        k = uniform(r, (b, lk, hk, d), 1.0)
        v = uniform(r, (b, lk, hk, d), 1.0)
    else:
        q = r.standard_normal((b, lq, h, d)).astype(np.float32)
        k = r.standard_normal((b, lk, hk, d)).astype(np.float32)
        v = r.standard_normal((b, lk, hk, d)).astype(np.float32)
    if half:
        k = k.astype(np.float16)
        v = v.astype(np.float16)
    q_d, k_d, v_d = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    y = unwritten((b, lq, h, d), gpu)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    # ggml's views: ne = [d, lq, h, b] with the heads interleaved in memory.
    sdhip.attention(q_d.permute(0, 2, 1, 3), k_d.permute(0, 2, 1, 3), v_d.permute(0, 2, 1, 3), y, scale)
    torch.cuda.synchronize()
    return q, k.astype(np.float32), v.astype(np.float32), y.cpu().numpy(), scale


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=lambda c: "x".join(map(str, c)))
def test_attention(gpu, c):
    d, lq, lk, h, hk, b, half = c
    q, k, v, y, scale = attention_case(gpu, *c, seed=d + lq + lk)
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    print(f"attention {c}: {err:.3g}")
    assert np.isfinite(y).all()
    assert err <= BOUND


@pytest.mark.gpu
def test_attention_vae_decoder(gpu):
    """The VAE decoder's attention (tools/bench.cc:153): one head of 512
    dimensions over 4096 positions, ~N(0,1); a sample of 200 queries checked
    against float64."""
    b, h, lq, d = 1, 1, 4096, 512
    q, k, v, y, scale = attention_case(gpu, d, lq, lq, h, h, b, False, seed=512, dist="normal")
    queries = rng(9).choice(b * h * lq, size=200, replace=False)
    exact, mag = orc.exact_attention(q, k, v, scale, queries=queries)
    got = y[0, queries % lq, 0, :]
    err = orc.metric(got, exact, mag)
    print(f"VAE attention: sampled error {err:.3g}")
    assert np.isfinite(y).all()
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [(512, 100, 70, 1, 1, 1), (512, 300, 1000, 2, 1, 1), (500, 65, 33, 2, 2, 1),
                               (512, 64, 4096, 1, 1, 1)], ids=lambda c: "x".join(map(str, c)))
def test_wide_heads_in_registers_agree(gpu, c):
    """Heads of 512 dimensions (500 rounded up to them) with single-precision
    keys and values: the form that holds each wave's queries in registers
    gives the wide form's bits (attention_generic=1 takes the latter) -- the
    same products, softmax and sums in the same order -- one split or
    several, heads sharing keys, ragged queries and keys."""
    d, lq, lk, h, hk, b = c
    _, _, _, y1, _ = attention_case(gpu, d, lq, lk, h, hk, b, False, seed=d + lq)
    sdhip.set_tuning("attention_generic=1")
    try:
        _, _, _, y2, _ = attention_case(gpu, d, lq, lk, h, hk, b, False, seed=d + lq)
    finally:
        sdhip.set_tuning("")
    assert np.isfinite(y1).all()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name,lk", [("cfg4 self", 4096), ("cfg4 cross", 77)])
def test_attention_bench_shapes(gpu, name, lk):
    """cfg4: Q [2, 8, 4096, 40] ~N(0,1) against 4096 or 77 keys; a sample of
    400 queries checked against float64."""
    b, h, lq, d = 2, 8, 4096, 40
    q, k, v, y, scale = attention_case(gpu, d, lq, lk, h, h, b, False, seed=lk, dist="normal")
    r = rng(7)
    queries = r.choice(b * h * lq, size=400, replace=False)
    exact, mag = orc.exact_attention(q, k, v, scale, queries=queries)
    bi, hi, i = queries // (h * lq), (queries // lq) % h, queries % lq
    got = y[bi, i, hi, :]
    err = orc.metric(got, exact, mag)
    print(f"{name}: sampled error {err:.3g}")
    assert np.isfinite(y).all()
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("d", [32, 40, 64, 80, 96, 128, 160])
def test_attention_peaked_scores(gpu, d):
    """The split form's head sizes with queries and keys ~N(0, 9): scores of
    tens, so that the running maximum moves by large steps and most
    exponentials underflow; 1000 keys (the last tile ragged, the keys split
    across workgroups), heads sharing keys.  Against float64, within the
    bound or, where single precision itself is further off at such scores,
    twice the error of the same attention in single precision (the scores'
    rounding grows with their size: the bound's 1e-6 is taken at unit
    inputs)."""
    b, lq, lk, h, hk = 1, 150, 1000, 4, 2
    r = rng(d)
    q = (3.0 * r.standard_normal((b, lq, h, d))).astype(np.float32)
    k = (3.0 * r.standard_normal((b, lk, hk, d))).astype(np.float32)
    v = r.standard_normal((b, lk, hk, d)).astype(np.float32)
    q_d, k_d, v_d = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    y = unwritten((b, lq, h, d), gpu)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    sdhip.attention(q_d.permute(0, 2, 1, 3), k_d.permute(0, 2, 1, 3), v_d.permute(0, 2, 1, 3), y, scale)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    # The same in single precision: scores, softmax and sums in float32.
    qh = q.transpose(0, 2, 1, 3)
    kh = np.repeat(k.transpose(0, 2, 1, 3), h // hk, axis=1)
    vh = np.repeat(v.transpose(0, 2, 1, 3), h // hk, axis=1)
    sc = np.matmul(qh, kh.transpose(0, 1, 3, 2)) * np.float32(scale)
    pr = np.exp(sc - sc.max(axis=-1, keepdims=True))
    single = (np.matmul(pr, vh) / pr.sum(axis=-1, keepdims=True)).transpose(0, 2, 1, 3)
    err32 = orc.metric(single.astype(np.float32), exact, mag)
    print(f"peaked scores d={d}: {err:.3g} (single precision {err32:.3g})")
    assert np.isfinite(y).all()
    assert err <= max(BOUND, 2.0 * err32)


@pytest.mark.gpu
def test_attention_not_taken(gpu):
    """Heads of more than 512 dimensions that the bits mode would quantize
    (256 keys or more) are left to the caller; so is a soft cap."""
    q = torch.zeros((1, 300, 1, 640), device=gpu)
    y = torch.zeros((1, 300, 1, 640), device=gpu)
    qv = q.permute(0, 2, 1, 3)
    sdhip.set_tuning("bits=8")
    try:
        with pytest.raises(sdhip.SdhipError) as e:
            sdhip.attention(qv, qv, qv, y, 0.05)
    finally:
        sdhip.set_tuning("")
    assert e.value.status == sdhip.UNSUPPORTED
    q40 = torch.zeros((1, 40, 1, 40), device=gpu)
    y40 = torch.zeros((1, 40, 1, 40), device=gpu)
    assert not sdhip.load().sdhip_attention_supported(sdhip.desc(q40.permute(0, 2, 1, 3)),
                                                      sdhip.desc(q40.permute(0, 2, 1, 3)),
                                                      sdhip.desc(q40.permute(0, 2, 1, 3)), sdhip.desc(y40), 0.0, 30.0)


@pytest.mark.gpu
@pytest.mark.parametrize("c", [c for c in CASES if not c[6] and c[0] in (40, 64, 80)], ids=lambda c: "x".join(map(str, c)))
def test_attention_generic_form(gpu, c):
    """The generic kernel (attention_generic=1) on the cases the fast one
    takes, so that both stay checked."""
    sdhip.set_tuning("attention_generic=1")
    try:
        q, k, v, y, scale = attention_case(gpu, *c, seed=c[0] + 11)
    finally:
        sdhip.set_tuning("")
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    print(f"attention generic {c}: {err:.3g}")
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [c for c in CASES if not c[6] and c[0] in (32, 40, 64, 80, 96, 128, 160)],
                         ids=lambda c: "x".join(map(str, c)))
def test_attention_single_precision_form(gpu, c):
    """The fast form's products on the single-precision MFMA
    (attention_fp32=1): within the bound of float64, and of the default split
    form on the same operands -- two device routes to the same attention."""
    sdhip.set_tuning("attention_fp32=1")
    try:
        q, k, v, y, scale = attention_case(gpu, *c, seed=c[0] + 13)
    finally:
        sdhip.set_tuning("")
    _, _, _, y_split, _ = attention_case(gpu, *c, seed=c[0] + 13)
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    apart = orc.metric(y, y_split.astype(np.float64), mag)
    print(f"attention single precision {c}: {err:.3g} of exact, {apart:.3g} from the split form")
    assert err <= BOUND and apart <= 2 * BOUND


@pytest.mark.gpu
def test_attention_work_buffer_checked(gpu):
    """The split form's tiles of keys and values go to the work buffer: a
    buffer short of sdhip_attention_work_size is an error, not a launch."""
    lib = sdhip.load()
    q = torch.zeros((1, 64, 2, 40), device=gpu)
    y = torch.zeros((1, 64, 2, 40), device=gpu)
    dq, dy = sdhip.desc(q.permute(0, 2, 1, 3)), sdhip.desc(y)
    size = lib.sdhip_attention_work_size(dq, dq, dq, dy)
    assert size > 0
    work = torch.zeros(size, dtype=torch.uint8, device=gpu)
    status = lib.sdhip_attention(dq, dq, dq, dy, 0.1, 0.0, 0.0, work.data_ptr(), size - 1, sdhip.stream_handle())
    assert status == sdhip.ERROR
    assert b"work buffer" in lib.sdhip_last_error()
    sdhip.check(lib.sdhip_attention(dq, dq, dq, dy, 0.1, 0.0, 0.0, work.data_ptr(), size, sdhip.stream_handle()),
                "attention")
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("d,lq,lk,h,hk,b", [(40, 300, 77, 2, 2, 2), (40, 129, 1, 1, 1, 1), (40, 130, 31, 2, 1, 1),
                                            (40, 64, 32, 1, 1, 2), (40, 200, 33, 2, 2, 1), (64, 257, 96, 2, 1, 1),
                                            (64, 100, 97, 2, 2, 1), (96, 70, 64, 2, 2, 1), (96, 70, 65, 2, 2, 1),
                                            (160, 40, 77, 2, 1, 2), (32, 33, 90, 3, 3, 1), (128, 128, 64, 1, 1, 1)],
                         ids=lambda c: str(c))
def test_short_keys_in_the_workgroup(gpu, d, lq, lk, h, hk, b):
    """Keys and values that fit the split form's ring with a buffer to spare
    (up to three tiles of 32 keys for heads of 64 or fewer, two above): every
    workgroup splits them itself, with no tiles launch before it; at the edges
    of that (one key, 31, 32, 33, 96 and 97 of 64, 64 and 65 of 96, 77 of
    160), ragged queries, heads sharing keys."""
    q, k, v, y, scale = attention_case(gpu, d, lq, lk, h, hk, b, False, seed=d + lq + lk)
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    print(f"attention d={d} lq={lq} lk={lk}: {err:.3g}")
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [(80, 1024, 1024, 8, 8, 2), (160, 256, 256, 8, 8, 2), (80, 1000, 999, 8, 4, 1),
                               (160, 130, 96, 2, 2, 1)], ids=lambda c: "x".join(map(str, c)))
def test_attention_key_splits(gpu, c):
    """Workgroups too few to fill the chip (the UNet's 32 x 32 and 16 x 16
    self-attention, a ragged case with heads sharing keys, three tiles of
    keys): the keys split across workgroups, each writing its running
    maximum, sum and output, merged by split_combine_kernel -- held to the
    bound against float64."""
    d, lq, lk, h, hk, b = c
    q, k, v, y, scale = attention_case(gpu, d, lq, lk, h, hk, b, False, seed=d + lq + lk)
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    print(f"attention key splits {c}: {err:.3g}")
    assert np.isfinite(y).all()
    assert err <= BOUND
