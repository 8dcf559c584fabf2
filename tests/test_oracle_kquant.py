"""Pins of the oracle's K-quant restatement (ggml quantize_row_q8_K_ref,
dequantize_row_q{4,5,6}_K, ggml_vec_dot_q{4,5,6}_K_q8_K; the Q6_K, Q5_K_M and
Q4_K_M profiles' matrices, src/levo-quantization.h:47-55, 96-118).

The reference's tests hold no K-quant vectors (tests/test-quantization.cpp
checks profile parsing and type routing only) and ggml is an un-vendored
submodule, so the oracle is pinned by construction: blocks are packed here
from the published block layout (an independent packer, the inverse of the
format's unpacking) with chosen integer codes and exactly representable
scales, so every dequantized value and every dot product has an exact
expected value; Q8_K by its invariants and exact recovery of representable
rows; the floating-point dot products against float64 within the
sequential-sum error bound.
"""
from __future__ import annotations

import numpy as np
import pytest

Q4_K, Q5_K, Q6_K, Q8_K = 12, 13, 14, 15


def f16_bytes(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def pack_scales_k4(sc, mn):
    """12 bytes holding eight 6-bit scales and mins (j < 4 in the low 6 bits of
    bytes j and j + 4; j >= 4 as nibbles of byte j + 4 plus the top 2 bits of
    bytes j - 4 and j)."""
    b = np.zeros(12, np.uint8)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return b


def pack_q4_K(d, dmin, sc, mn, codes):
    qs = np.zeros(128, np.uint8)
    for g in range(4):
        qs[32 * g:32 * g + 32] = codes[64 * g:64 * g + 32] | (codes[64 * g + 32:64 * g + 64] << 4)
    return np.concatenate([f16_bytes(d), f16_bytes(dmin), pack_scales_k4(sc, mn), qs])


def pack_q5_K(d, dmin, sc, mn, codes):
    lo = codes & 15
    qs = np.zeros(128, np.uint8)
    qh = np.zeros(32, np.uint8)
    for g in range(4):
        qs[32 * g:32 * g + 32] = lo[64 * g:64 * g + 32] | (lo[64 * g + 32:64 * g + 64] << 4)
        qh |= ((codes[64 * g:64 * g + 32] >> 4) << (2 * g)).astype(np.uint8)
        qh |= ((codes[64 * g + 32:64 * g + 64] >> 4) << (2 * g + 1)).astype(np.uint8)
    return np.concatenate([f16_bytes(d), f16_bytes(dmin), pack_scales_k4(sc, mn), qh, qs])


def pack_q6_K(d, sc, codes):
    """codes in [-32, 31], 16 int8 scales."""
    c = (codes + 32).astype(np.uint8)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(2):
        b = c[128 * n:128 * n + 128]
        ql[64 * n:64 * n + 32] = (b[0:32] & 15) | ((b[64:96] & 15) << 4)
        ql[64 * n + 32:64 * n + 64] = (b[32:64] & 15) | ((b[96:128] & 15) << 4)
        qh[32 * n:32 * n + 32] = (b[0:32] >> 4) | ((b[32:64] >> 4) << 2) | ((b[64:96] >> 4) << 4) | ((b[96:128] >> 4) << 6)
    return np.concatenate([ql, qh, np.asarray(sc, np.int8).view(np.uint8), f16_bytes(d)])


def random_block(qtype, rng, d=0.5, dmin=0.25):
    """A block with exact-valued fields and its expected dequantized values (float64)."""
    if qtype == Q6_K:
        sc = rng.integers(-128, 128, 16)
        codes = rng.integers(-32, 32, 256)
        want = d * np.repeat(sc, 16) * codes
        return pack_q6_K(d, sc, codes), want
    top = 16 if qtype == Q4_K else 32
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    codes = rng.integers(0, top, 256).astype(np.uint8)
    want = d * np.repeat(sc, 32) * codes - dmin * np.repeat(mn, 32)
    pack = pack_q4_K if qtype == Q4_K else pack_q5_K
    return pack(d, dmin, sc, mn, codes), want


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_dequantize_known_blocks(oracle, qtype):
    """Every value of blocks packed from chosen codes, 6-bit (or int8) scales
    and mins, d = 0.5, dmin = 0.25: exact."""
    rng = np.random.default_rng(qtype)
    blocks, want = zip(*(random_block(qtype, rng) for _ in range(12)))
    got = oracle.dequantize_kquant(qtype, np.concatenate(blocks), 256 * 12)
    assert np.array_equal(got.astype(np.float64), np.concatenate(want))


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K])
def test_scale_packing_extremes(oracle, qtype):
    """All-63 and alternating 6-bit fields exercise every packed bit."""
    codes = np.full(256, 1, np.uint8)
    for sc, mn in ((np.full(8, 63), np.full(8, 63)), (np.arange(8) * 9, 63 - np.arange(8) * 9),
                   (np.array([0, 63, 16, 47, 32, 31, 48, 15]), np.array([63, 0, 47, 16, 31, 32, 15, 48]))):
        pack = pack_q4_K if qtype == Q4_K else pack_q5_K
        got = oracle.dequantize_kquant(qtype, pack(1.0, 1.0, sc, mn, codes), 256)
        assert np.array_equal(got, (np.repeat(sc, 32) - np.repeat(mn, 32)).astype(np.float32))


def test_q8_K_invariants_and_exact_rows(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(256 * 8) * 3).astype(np.float32)
    b = oracle.quantize_q8_K(x).reshape(8, 292)
    for i in range(8):
        d = b[i, :4].view(np.float32)[0]
        qs = b[i, 4:260].view(np.int8).astype(np.int64)
        bs = b[i, 260:292].view(np.int16)
        xi = x[256 * i:256 * i + 256]
        assert qs.min() >= -127 and qs.max() <= 127
        assert np.array_equal(bs, qs.reshape(16, 16).sum(1))
        j = np.argmax(np.abs(xi))
        assert qs[j] == -127  # iscale = -127 / max maps the extreme value to -127
        assert np.all(np.abs(xi.astype(np.float64) - d * qs) <= abs(d) * (0.5 + 1e-5))
    # exactly representable rows come back exactly: x = s * n with a single
    # extreme n = -127 (the signed max), so iscale = 1 / s, d = s, codes = n;
    # with the extreme at +127 instead, d = -s and the codes are -n
    n = rng.integers(-126, 127, 256)
    for sign in (-1, 1):
        n[17] = 127 * sign
        for s in (0.125, 2.0 ** -10, 64.0):
            blk = oracle.quantize_q8_K((n * s).astype(np.float32))
            assert blk[:4].view(np.float32)[0] == -sign * s
            assert np.array_equal(blk[4:260].view(np.int8), -sign * n)
    zero = oracle.quantize_q8_K(np.zeros(256, np.float32))
    assert not zero.any()


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_vec_dot_integer_blocks_exact(oracle, qtype):
    """d_w = 1 (and dmin = 1), d_x = 1: the dot product is an exact integer,
    equal to the float64 sum over the dequantized values."""
    rng = np.random.default_rng(20 + qtype)
    nb = 6
    blocks, wvals = [], []
    for _ in range(nb):
        blk, want = random_block(qtype, rng, d=1.0, dmin=1.0)
        blocks.append(blk)
        wvals.append(want)
    w = np.concatenate(blocks)
    xq = rng.integers(-127, 128, 256 * nb)
    xb = np.zeros((nb, 292), np.uint8)
    for i in range(nb):
        xb[i, :4] = np.array([1.0], np.float32).view(np.uint8)
        xb[i, 4:260] = xq[256 * i:256 * i + 256].astype(np.int8).view(np.uint8)
        xb[i, 260:292] = xq[256 * i:256 * i + 256].reshape(16, 16).sum(1).astype(np.int16).view(np.uint8)
    want = float(np.dot(np.concatenate(wvals), xq.astype(np.float64)))
    assert abs(want) < 2 ** 24
    assert oracle.vec_dot_kquant(qtype, w, xb.ravel(), 256 * nb) == want


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_vec_dot_against_float64(oracle, qtype):
    """Random f16 scales and real activations: within the sequential-sum bound
    of the float64 dot product of the dequantized operands."""
    rng = np.random.default_rng(40 + qtype)
    nb = 8
    blocks = []
    for _ in range(nb):
        blk, _ = random_block(qtype, rng)
        blk[-2:] = f16_bytes(rng.uniform(1e-3, 2e-2)) if qtype == Q6_K else blk[-2:]
        if qtype != Q6_K:
            blk[0:2] = f16_bytes(rng.uniform(1e-3, 2e-2))
            blk[2:4] = f16_bytes(rng.uniform(1e-3, 2e-2))
        blocks.append(blk)
    w = np.concatenate(blocks)
    x = rng.standard_normal(256 * nb).astype(np.float32)
    xb = oracle.quantize_q8_K(x)
    wd = oracle.dequantize_kquant(qtype, w, 256 * nb).astype(np.float64)
    xd = np.concatenate([xb.reshape(nb, 292)[i, :4].view(np.float32)[0] *
                         xb.reshape(nb, 292)[i, 4:260].view(np.int8).astype(np.float64) for i in range(nb)])
    want = float(np.dot(wd, xd))
    got = oracle.vec_dot_kquant(qtype, w, xb, 256 * nb)
    bound = 64 * np.finfo(np.float32).eps * float(np.abs(wd * xd).sum())
    assert abs(got - want) <= bound, (got, want, bound)


def test_mul_mat_kquant_is_vec_dot_per_row(oracle):
    rng = np.random.default_rng(77)
    rows, k = 5, 512
    for qtype in (Q4_K, Q5_K, Q6_K):
        w = np.concatenate([random_block(qtype, rng)[0] for _ in range(rows * k // 256)])
        x = rng.standard_normal((2, k)).astype(np.float32)
        y = oracle.mul_mat_kquant(qtype, w, x, rows, k)
        nbytes = {Q4_K: 144, Q5_K: 176, Q6_K: 210}[qtype] * (k // 256)
        for v in range(2):
            xb = oracle.quantize_q8_K(x[v])
            for r in range(rows):
                assert y[v, r] == np.float32(oracle.vec_dot_kquant(qtype, w[r * nbytes:(r + 1) * nbytes], xb, k))


# --- the reference quantizers (quantize_row_q{4,5,6}_K_ref) -------------------
# Unpacked here from the published layout (the inverse of the packers above),
# so the checks do not lean on the oracle's own packing.

def unpack_q45_K(qtype, blk):
    d = blk[0:2].view(np.float16)[0].astype(np.float64)
    dmin = blk[2:4].view(np.float16)[0].astype(np.float64)
    s = blk[4:16].astype(np.int64)
    sc = np.zeros(8, np.int64)
    mn = np.zeros(8, np.int64)
    for j in range(8):
        if j < 4:
            sc[j], mn[j] = s[j] & 63, s[j + 4] & 63
        else:
            sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
            mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    codes = np.zeros(256, np.int64)
    if qtype == Q4_K:
        qs = blk[16:144].astype(np.int64)
        for p in range(4):
            codes[64 * p:64 * p + 32] = qs[32 * p:32 * p + 32] & 15
            codes[64 * p + 32:64 * p + 64] = qs[32 * p:32 * p + 32] >> 4
    else:
        qh = blk[16:48].astype(np.int64)
        qs = blk[48:176].astype(np.int64)
        for p in range(4):
            codes[64 * p:64 * p + 32] = (qs[32 * p:32 * p + 32] & 15) | (((qh >> (2 * p)) & 1) << 4)
            codes[64 * p + 32:64 * p + 64] = (qs[32 * p:32 * p + 32] >> 4) | (((qh >> (2 * p + 1)) & 1) << 4)
    return d, dmin, sc, mn, codes


def unpack_q6_K(blk):
    ql = blk[0:128].astype(np.int64)
    qh = blk[128:192].astype(np.int64)
    sc = blk[192:208].view(np.int8).astype(np.int64)
    d = blk[208:210].view(np.float16)[0].astype(np.float64)
    codes = np.zeros(256, np.int64)
    for n in range(2):
        l, h = ql[64 * n:64 * n + 64], qh[32 * n:32 * n + 32]
        codes[128 * n + 0:128 * n + 32] = (l[0:32] & 15) | ((h & 3) << 4)
        codes[128 * n + 32:128 * n + 64] = (l[32:64] & 15) | (((h >> 2) & 3) << 4)
        codes[128 * n + 64:128 * n + 96] = (l[0:32] >> 4) | (((h >> 4) & 3) << 4)
        codes[128 * n + 96:128 * n + 128] = (l[32:64] >> 4) | (((h >> 6) & 3) << 4)
    return d, sc, codes - 32


BSZ = {Q4_K: 144, Q5_K: 176, Q6_K: 210}


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_quantize_zero_rows(oracle, qtype):
    """All-zero super-blocks (and -0.0) quantize to all-zero bytes."""
    x = np.zeros((2, 512), np.float32)
    x[1] = -0.0
    assert not oracle.quantize(qtype, x).any()


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K])
def test_quantize_q45_K_integer_grid(oracle, qtype):
    """Sub-blocks of integers 0..nmax holding both ends: the search keeps
    scale 1 and min 0 (the first trial fits exactly), so every sub-block scale
    is 63, d = F16(1 / 63), dmin = 0 and every code is the value itself."""
    nmax = 15 if qtype == Q4_K else 31
    rng = np.random.default_rng(40 + qtype)
    x = rng.integers(0, nmax + 1, (3, 512)).astype(np.float32)
    x[:, ::32] = 0
    x[:, 1::32] = nmax
    q = oracle.quantize(qtype, x).reshape(-1, BSZ[qtype])
    for b, blk in enumerate(q):
        d, dmin, sc, mn, codes = unpack_q45_K(qtype, blk)
        assert d == np.float64(np.float16(np.float32(1) / np.float32(63)))
        assert dmin == 0 and np.all(sc == 63) and np.all(mn == 0)
        assert np.array_equal(codes, x.reshape(-1, 256)[b].astype(np.int64))


def test_quantize_q6_K_integer_grid(oracle):
    """Sub-blocks of integers in [-32, 31] each holding -32: scale 1 in every
    sub-block, d = -1/128 and sub-block scales -128, so the codes are the
    values and dequantization is exact."""
    rng = np.random.default_rng(46)
    x = rng.integers(-32, 32, (3, 512)).astype(np.float32)
    x[:, ::16] = -32
    q = oracle.quantize(Q6_K, x)
    for b, blk in enumerate(q.reshape(-1, 210)):
        d, sc, codes = unpack_q6_K(blk)
        assert d == -1 / 128 and np.all(sc == -128)
        assert np.array_equal(codes, x.reshape(-1, 256)[b].astype(np.int64))
    assert np.array_equal(oracle.dequantize_kquant(Q6_K, q, x.size), x.ravel())


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_quantize_round_trip(oracle, qtype):
    """Gaussian rows (and all-positive rows, outliers, sub-blocks of very
    different size): each code is the nearest integer to the value measured
    in its sub-block's quantized step (t = (x + dmin*m) / (d*sc), Q6_K
    t = x / (d*sc)), or clamped at an end of the code range with t beyond
    it; the largest sub-block scale quantizes to 63 (Q6_K: the
    largest-magnitude scale to -128); the rms error stays under half a code
    step of the block's range."""
    rng = np.random.default_rng(50 + qtype)
    x = (rng.standard_normal((6, 1024)) * 0.05).astype(np.float32)
    x[1] += 0.3                                  # all-positive sub-blocks (min clamped to 0)
    x[2, ::97] = 2.0                             # outliers
    x[3, :256] *= np.repeat(np.geomspace(1e-4, 1.0, 8), 32).astype(np.float32)  # tiny vs large sub-blocks
    q = oracle.quantize(qtype, x).reshape(-1, BSZ[qtype])
    deq = oracle.dequantize_kquant(qtype, q.ravel(), x.size).reshape(-1, 256).astype(np.float64)
    xs = x.reshape(-1, 256).astype(np.float64)
    nmax = 63 if qtype == Q6_K else (15 if qtype == Q4_K else 31)
    for b, blk in enumerate(q):
        if qtype == Q6_K:
            d, sc, codes = unpack_q6_K(blk)
            assert sc[np.argmax(np.abs(sc))] == -128
            step = d * np.repeat(sc, 16)
            off = np.zeros(256)
            lo, hi = -32, 31
        else:
            d, dmin, sc, mn, codes = unpack_q45_K(qtype, blk)
            assert sc.max() == 63
            step = d * np.repeat(sc, 32)
            off = dmin * np.repeat(mn, 32)
            lo, hi = 0, nmax
        ok = step != 0
        t = (xs[b][ok] + off[ok]) / step[ok]
        c = codes[ok]
        tol = 1e-4 * np.maximum(1.0, np.abs(t))
        inside = (c > lo) & (c < hi)
        assert np.all(np.abs(t[inside] - c[inside]) <= 0.5 + tol[inside]), b
        assert np.all(t[c == lo] <= lo + 0.5 + tol[c == lo]), b
        assert np.all(t[c == hi] >= hi - 0.5 - tol[c == hi]), b
        err = np.abs(xs[b] - deq[b])
        rng_b = xs[b].max() - min(xs[b].min(), 0.0)
        assert np.sqrt(np.mean(err ** 2)) <= 0.5 * rng_b / nmax + 1e-6, b


def test_quantize_search_beats_plain_rounding(oracle):
    """The scale searches are what the K-quants add over plain rounding: on
    Gaussian data the least-squares refined (scale, min) of make_qkx2_quants
    and make_qx_quants must beat the plain affine (min..max over nmax steps)
    and symmetric (max |x| over 31.5 steps) quantizers in rms error, 6-bit /
    8-bit scale quantization included (measured: 0.91, 0.96, 0.85 of plain;
    a search that loses its least-squares step lands at or above 1.0)."""
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, 1024)) * 0.05).astype(np.float32)
    for qtype, nmax, bound in ((Q4_K, 15, 0.93), (Q5_K, 31, 0.975)):
        deq = oracle.dequantize_kquant(qtype, oracle.quantize(qtype, x), x.size).reshape(-1, 32).astype(np.float64)
        xs = x.reshape(-1, 32).astype(np.float64)
        mn = np.minimum(xs.min(1), 0)[:, None]
        step = (xs.max(1)[:, None] - mn) / nmax
        plain = np.round((xs - mn) / step) * step + mn
        assert np.sqrt(np.mean((deq - xs) ** 2)) <= bound * np.sqrt(np.mean((plain - xs) ** 2)), qtype
    deq = oracle.dequantize_kquant(Q6_K, oracle.quantize(Q6_K, x), x.size).reshape(-1, 16).astype(np.float64)
    xs = x.reshape(-1, 16).astype(np.float64)
    step = np.abs(xs).max(1)[:, None] / 31.5
    plain = np.clip(np.round(xs / step), -32, 31) * step
    assert np.sqrt(np.mean((deq - xs) ** 2)) <= 0.9 * np.sqrt(np.mean((plain - xs) ** 2))


def _finite_f16():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return h[np.isfinite(h)].astype(np.float32)


def test_dequantize_products_exact_for_every_scale():
    """Why the dequantizers cannot depend on floating-point contraction.
    Q4_K / Q5_K compute d1 * q - m1 with d1 = d * sc, m1 = dmin * m, d and
    dmin F16, sc and m in [0, 63], q in [0, 31]; Q6_K computes d * sc * q
    with sc an int8 and q in [-32, 31]. Over every finite F16 d, every scale
    and every code, each F32 product equals the exact (float64) product, so
    an FMA for the last step rounds exactly as a multiply then a subtract,
    and an F32 product never rounds. Exhaustive: 63,488 x 64 x 32 (Q4_K/Q5_K)
    and 63,488 x 256 x 64 (Q6_K) products."""
    d = _finite_f16()
    for scales, codes in ((np.arange(64), range(32)), (np.arange(-128, 128), range(-32, 32))):
        sc = scales.astype(np.float32)
        for lo in range(0, d.size, 2048):  # chunks of 2048 F16 values keep each array at a few MB
            dd = d[lo:lo + 2048, None]
            d1 = dd * sc[None, :]
            assert np.array_equal(d1.astype(np.float64), dd.astype(np.float64) * sc[None, :])
            d1_64 = d1.astype(np.float64)
            for q in codes:
                assert np.array_equal((d1 * np.float32(q)).astype(np.float64), d1_64 * q), (lo, q)


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K])
def test_dequantize_non_representable_scales(oracle, qtype):
    """Blocks with F16 d, dmin whose products with the scales and codes fill
    all 22 product bits (no power-of-two scales): every value equals the
    float32 multiply-then-subtract, which by the exactness above is also the
    correctly rounded d1 * q - m1 computed in float64."""
    rng = np.random.default_rng(100 + qtype)
    pack = pack_q4_K if qtype == Q4_K else pack_q5_K
    top = 16 if qtype == Q4_K else 32
    blocks, want = [], []
    for _ in range(16):
        d = np.float16(rng.uniform(1e-4, 2.0))
        dmin = np.float16(rng.uniform(1e-4, 2.0))
        sc = rng.integers(33, 64, 8)
        mn = rng.integers(33, 64, 8)
        codes = rng.integers(0, top, 256).astype(np.uint8)
        d1 = np.float32(d) * np.repeat(sc, 32).astype(np.float32)
        m1 = np.float32(dmin) * np.repeat(mn, 32).astype(np.float32)
        w32 = d1 * codes.astype(np.float32) - m1
        exact = (d1.astype(np.float64) * codes - m1.astype(np.float64)).astype(np.float32)
        assert np.array_equal(w32, exact)
        blocks.append(pack(float(d), float(dmin), sc, mn, codes))
        want.append(w32)
    got = oracle.dequantize_kquant(qtype, np.concatenate(blocks), 256 * len(blocks))
    assert np.array_equal(got.view(np.uint32), np.concatenate(want).view(np.uint32))
