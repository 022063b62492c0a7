"""Pins on the oracle that do not depend on the reference's vectors: closed
forms (IEEE fp16 conversion, exact rounding, the two quantizers written out in
numpy), brute-force integer sums from a second, independent numpy decoder of
the block formats, the fp64 value of whole dot products, and planted mistakes
(the oracle compiled with ORC_MUTANT) that the golden vectors must catch."""
import os
import subprocess

import numpy as np
import pytest

from oracle_lib import (BF16, F16, F32, OP_AFFINE, OP_EULER, OP_PATCH, OP_RESIDUAL, OP_UNPATCH, OP_UPSAMPLE, ORACLE_DIR, Q5_K,
                        Q6_K, Q8_0, add, attention, bias, channel_op, decode_f32, dot, gather, gelu, groupnorm, l2norm, layout,
                        load_oracle, modulate_rows, norm_rows, oracle, ptr, quant_matmul, quantize, qwen_modulate, rope, scatter,
                        shortcut, silu_gate, conv2d)
from pixelina_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---- fp16 and rounding ----

def test_half_to_float_exhaustive():
    lib = oracle()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_half_to_float(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_round_to_nearest_even():
    lib = oracle()
    rng = np.random.default_rng(5)
    x = np.concatenate([
        (rng.standard_normal(4000) * np.exp2(rng.integers(-30, 20, 4000))).astype(np.float32),
        np.array([65504.0, 65519.99, 65520.0, 1e6, -1e6, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0, np.inf, -np.inf],
                 dtype=np.float32),
        # exact ties between two fp16 neighbours (even and odd mantissas)
        (np.float32(1.0) + np.float32(2.0 ** -11) * np.arange(1, 40, 2)).astype(np.float32),
    ])
    got = np.array([lib.orc_float_to_half(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert np.isnan(np.uint16(lib.orc_float_to_half(float("nan"))).view(np.float16))


def test_fused_nearest_int_is_exact_round_half_even():
    lib = oracle()
    rng = np.random.default_rng(6)
    s = (rng.standard_normal(3000) * 50).astype(np.float32)
    x = (rng.standard_normal(3000) * 3).astype(np.float32)
    want = np.rint(s.astype(np.float64) * x.astype(np.float64)).astype(np.int64)
    got = np.array([lib.orc_nearest_int_fused(float(a), float(b)) for a, b in zip(s, x)], dtype=np.int64)
    assert np.array_equal(got, want)
    # exact halves round to even
    for a, b, r in [(1.0, 2.5, 2), (1.0, 3.5, 4), (-1.0, 2.5, -2), (0.5, 5.0, 2)]:
        assert lib.orc_nearest_int_fused(a, b) == r


# ---- the quantizers, written out ----

def q8_K_closed_form(x):
    """quantize_row_q8_K_ref (src/kernels_quant.cpp:80-118) in numpy, rows of 256."""
    out = []
    for blk in x.reshape(-1, 256):
        ax = np.abs(blk)
        j = int(np.argmax(ax))  # first index of the largest |x|
        b = np.zeros(292, np.uint8)
        if ax[j] == 0:
            out.append(b)
            continue
        iscale = np.float32(-127.0) / blk[j]
        q = np.minimum(127, np.rint(np.float64(iscale) * blk.astype(np.float64))).astype(np.int64)
        b[0:4] = np.array([np.float32(1.0) / iscale], np.float32).view(np.uint8)
        b[4:260] = q.astype(np.int8).view(np.uint8)
        b[260:292] = q.reshape(16, 16).sum(1).astype(np.int16).view(np.uint8)
        out.append(b)
    return np.concatenate(out)


def q8_0_closed_form(x):
    """quantize_row_q8_0_ref (src/kernels_quant.cpp:120-144) in numpy, rows of 32."""
    out = []
    for blk in x.reshape(-1, 32):
        amax = np.float32(np.max(np.abs(blk)))
        d = amax / np.float32(127.0)
        idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        v = (blk * idv).astype(np.float32).astype(np.float64)
        q = np.trunc(v + np.copysign(0.5, v)).astype(np.int64)  # roundf: half away from zero
        b = np.zeros(34, np.uint8)
        b[0:2] = np.array([d], np.float32).astype(np.float16).view(np.uint8)
        b[2:] = (q & 0xFF).astype(np.uint8)
        out.append(b)
    return np.concatenate(out)


@pytest.mark.parametrize("scale", [1e-4, 1.0, 300.0])
def test_quantizers_equal_closed_forms(scale):
    rng = np.random.default_rng(int(scale * 10) + 1)
    x = (rng.standard_normal((8, 512)) * scale).astype(np.float32)
    x[1, 7] = -x[1, 7] * 9  # a dominant negative entry
    x[2, :] = 0.0
    x[3, 20], x[3, 300] = 4 * scale, -4 * scale  # |max| ties across blocks and signs
    lib = oracle()
    for r in range(len(x)):
        assert np.array_equal(quantize(lib, "orc", x[r:r + 1], "q8_K")[0], q8_K_closed_form(x[r])), r
        assert np.array_equal(quantize(lib, "orc", x[r:r + 1], "q8_0")[0], q8_0_closed_form(x[r])), r


# ---- a second decoder of the block formats (numpy) ----

def f16(b, off):
    return b[..., off:off + 2].copy().view(np.float16)[..., 0].astype(np.float64)


def q5_K_ints(blocks):
    """-> d, dmin [nb], scale, min [nb, 8], q [nb, 256] for 176-byte blocks."""
    b = blocks.reshape(-1, 176)
    sc = b[:, 4:16].astype(np.int64)
    scale = np.zeros((len(b), 8), np.int64)
    mn = np.zeros((len(b), 8), np.int64)
    for s in range(8):
        if s < 4:
            scale[:, s] = sc[:, s] & 63
            mn[:, s] = sc[:, s + 4] & 63
        else:
            scale[:, s] = (sc[:, s + 4] & 15) | ((sc[:, s - 4] >> 6) << 4)
            mn[:, s] = (sc[:, s + 4] >> 4) | ((sc[:, s] >> 6) << 4)
    qh = b[:, 16:48].astype(np.int64)
    qs = b[:, 48:176].astype(np.int64)
    q = np.zeros((len(b), 256), np.int64)
    for s in range(8):
        low = (qs[:, (s // 2) * 32:(s // 2) * 32 + 32] >> (4 * (s % 2))) & 15
        q[:, 32 * s:32 * s + 32] = low | (((qh >> s) & 1) << 4)
    return f16(b, 0), f16(b, 2), scale, mn, q


def q6_K_ints(blocks):
    """-> d [nb], scale [nb, 16] (int8), q - 32 [nb, 256] for 210-byte blocks."""
    b = blocks.reshape(-1, 210)
    ql = b[:, 0:128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    q = np.zeros((len(b), 256), np.int64)
    for e in range(256):
        h, r = divmod(e, 128)
        g, i = divmod(r, 32)
        low = ql[:, 64 * h + i + 32 * (g % 2)]
        low = (low & 15) if g < 2 else (low >> 4)
        q[:, e] = low | (((qh[:, 32 * h + i] >> (2 * g)) & 3) << 4)
    return f16(b, 208), sc, q - 32


def q8_K_ints(blocks):
    b = blocks.reshape(-1, 292)
    return (b[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64), b[:, 4:260].view(np.int8).astype(np.int64),
            b[:, 260:292].copy().view(np.int16).astype(np.int64))


def weights(rng, rows, k):
    return (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)


def test_second_decoder_agrees_with_oracle_decode():
    rng = np.random.default_rng(21)
    w = weights(rng, 3, 512)
    lib = oracle()
    for wtype, blocks in ((Q5_K, synth.pack_q5_K(w)), (Q6_K, synth.pack_q6_K(w))):
        out = np.zeros(3 * 512)
        lib.orc_decode(ptr(np.ascontiguousarray(blocks)), wtype, out.size, ptr(out))
        if wtype == Q5_K:
            d, dm, sc, mn, q = q5_K_ints(blocks)
            ours = d[:, None] * np.repeat(sc, 32, 1) * q - dm[:, None] * np.repeat(mn, 32, 1)
        else:
            d, sc, q = q6_K_ints(blocks)
            ours = d[:, None] * np.repeat(sc, 16, 1) * q
        assert np.allclose(out, ours.reshape(-1), rtol=0, atol=1e-12)
        # and the packers keep the weights within their quantization step
        assert np.max(np.abs(out - w.reshape(-1))) < 0.1 * np.max(np.abs(w))


def test_integer_sums_brute_force():
    rng = np.random.default_rng(22)
    lib = oracle()
    x = (rng.standard_normal((2, 768)) * 3).astype(np.float32)
    w = weights(rng, 2, 768)
    a8k = quantize(lib, "orc", x, "q8_K")
    ad, aq, abs_ = q8_K_ints(a8k)
    assert np.array_equal(aq.reshape(-1, 16, 16).sum(2), abs_)
    for blocks, kind in ((synth.pack_q5_K(w), Q5_K), (synth.pack_q6_K(w), Q6_K)):
        size = 176 if kind == Q5_K else 210
        ints = q5_K_ints(blocks) if kind == Q5_K else q6_K_ints(blocks)
        for sb in range(blocks.size // size):
            wb = np.ascontiguousarray(blocks.reshape(-1)[sb * size:(sb + 1) * size])
            ab = np.ascontiguousarray(a8k.reshape(-1)[sb * 292:(sb + 1) * 292])
            if kind == Q5_K:
                _, _, sc, mn, q = ints
                want_s = int(sum(sc[sb, s] * np.dot(q[sb, 32 * s:32 * s + 32], aq[sb, 32 * s:32 * s + 32]) for s in range(8)))
                want_m = int(sum(mn[sb, s] * (abs_[sb, 2 * s] + abs_[sb, 2 * s + 1]) for s in range(8)))
                got_s, got_m = np.zeros(1, np.int32), np.zeros(1, np.int32)
                lib.orc_superblock_sums_q5_K(ptr(wb), ptr(ab), ptr(got_s), ptr(got_m))
                assert (int(got_s[0]), int(got_m[0])) == (want_s, want_m)
            else:
                _, sc, q = ints
                want = int(np.dot(np.repeat(sc[sb], 16) * q[sb], aq[sb]))
                assert lib.orc_superblock_sum_q6_K(ptr(wb), ptr(ab)) == want
    a80 = quantize(lib, "orc", x, "q8_0").reshape(-1, 34)
    w80 = quantize(lib, "orc", w, "q8_0").reshape(-1, 34)
    for b in range(len(a80)):
        want = int(np.dot(w80[b, 2:].view(np.int8).astype(np.int64), a80[b, 2:].view(np.int8).astype(np.int64)))
        assert lib.orc_block_sums_q8_0(ptr(np.ascontiguousarray(w80[b])), ptr(np.ascontiguousarray(a80[b]))) == want


@pytest.mark.parametrize("wtype", [Q8_0, Q5_K, Q6_K])
def test_dot_equals_fp64_dequantized_sum(wtype):
    rng = np.random.default_rng(23 + wtype)
    k = 1024
    lib = oracle()
    x = (rng.standard_normal((4, k))).astype(np.float32)
    w = weights(rng, 4, k)
    if wtype == Q8_0:
        wb, ab = quantize(lib, "orc", w, "q8_0"), quantize(lib, "orc", x, "q8_0")
    else:
        wb = synth.pack_q5_K(w) if wtype == Q5_K else synth.pack_q6_K(w)
        ab = quantize(lib, "orc", x, "q8_K")
    for r in range(4):
        wv = np.zeros(k)
        lib.orc_decode(ptr(np.ascontiguousarray(wb[r])), wtype, k, ptr(wv))
        if wtype == Q8_0:
            blk = ab[r].reshape(-1, 34)
            av = (f16(blk, 0)[:, None] * blk[:, 2:].view(np.int8)).reshape(-1)
            # the reference multiplies the two fp16 scales first, in fp32
            terms = wv * av
        else:
            d, q, _ = q8_K_ints(ab[r])
            av = (d[:, None] * q).reshape(-1)
            terms = wv * av
        got = dot(lib, "orc", wtype, wb[r], ab[r], k)
        assert abs(got - terms.sum()) <= 2e-6 * np.abs(terms).sum() + 1e-30


# ---- neighbours of the linear layer: norm and SiLU-gate ----

def test_norm_properties():
    """What the mathematics fixes about tensor_norm's output, independent of
    the oracle's formula: unit mean square (up to epsilon), zero mean when
    centered, exact scale invariance by powers of two at epsilon 0, the
    weight applied last (y_w == fl(y * w)), and the degenerate rows."""
    o = oracle()
    rng = np.random.default_rng(41)
    k = 768
    x = (rng.standard_normal((16, k)) * rng.choice([1e-2, 1.0, 30.0], (16, 1)) + rng.choice([0.0, 5.0], (16, 1))).astype(np.float32)
    w = (1.0 + 0.3 * rng.standard_normal(k)).astype(np.float32)
    for centered in (0, 1):
        y = norm_rows(o, "orc", x, None, 0.0, centered).astype(np.float64)
        assert np.allclose((y * y).mean(axis=1), 1.0, rtol=0, atol=2e-6)
        if centered:
            assert np.abs(y.mean(axis=1)).max() < 1e-6
        y1 = norm_rows(o, "orc", x, None, 0.0, centered)
        y4 = norm_rows(o, "orc", x * np.float32(4.0), None, 0.0, centered)
        assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))
        yn = norm_rows(o, "orc", x, None, 1e-5, centered)
        yw = norm_rows(o, "orc", x, w, 1e-5, centered)
        assert np.array_equal(yw.view(np.uint32), (yn * w).astype(np.float32).view(np.uint32))
    z = np.zeros((2, 256), np.float32)
    z[1] = 2.5
    assert not norm_rows(o, "orc", z[:1], None, 1e-5, 0).any()
    assert not norm_rows(o, "orc", z, None, 1e-5, 1).any()      # constant rows center to zero
    y = norm_rows(o, "orc", z[1:], None, 0.0, 0)
    assert np.all(y == 1.0)                                      # 2.5 * (1/2.5)


def test_silu_gate_properties():
    """silu(v)*u against the closed form in float64 (within two fp32 ulps: the
    rounded exponential, sum and quotient), the
    identity silu(v) - silu(-v) = v, the exact limits, and the gate applied
    last: y(g, u) == fl(y(g, 1) * u)."""
    o = oracle()
    rng = np.random.default_rng(43)
    g = (rng.standard_normal(1 << 16) * 8.0).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    one = np.ones_like(g)
    s = silu_gate(o, "orc", g, one)
    exact = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert (np.abs(s - exact) <= 2.0 * ulp + 1e-45).all()
    sn = silu_gate(o, "orc", -g, one)
    assert (np.abs((s.astype(np.float64) - sn) - g) <= 4 * np.spacing(np.abs(g))).all()
    y = silu_gate(o, "orc", g, u)
    assert np.array_equal(y.view(np.uint32), (s * u).astype(np.float32).view(np.uint32))
    lim = np.array([0.0, 104.0, 200.0, -104.0], np.float32)
    out = silu_gate(o, "orc", lim, np.ones(4, np.float32))
    assert out[0] == 0 and out[1] == 104.0 and out[2] == 200.0 and out[3] == 0.0


def test_elementwise_ops_properties():
    """GELU against the float64 closed forms (the fp32 factor 1 + erf (or tanh)
    carries an absolute error of about an ulp of 1, which for negative v cancels
    towards zero: bound |0.5 v| * 3e-7 plus 3 ulps of the result), gelu(0) = 0 and
    the exact large-|v| limits; RoPE with cos 1 / sin 0 is the identity, a
    rotation by a quarter turn maps (a, b) to (-b, a) exactly, and it keeps
    every pair's length to fp32 rounding; bias and add equal their fp32 sums."""
    o = oracle()
    rng = np.random.default_rng(47)
    x = (rng.standard_normal((8, 256)) * 4.0).astype(np.float32)
    xd = x.astype(np.float64)
    from math import erf as _erf
    exact = 0.5 * xd * (1.0 + np.vectorize(_erf)(xd / np.sqrt(2.0)))
    approx = 0.5 * xd * (1.0 + np.tanh(0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    for form, want in ((0, exact), (1, approx)):
        got = gelu(o, "orc", x, form).astype(np.float64)
        tol = 0.5 * np.abs(xd) * 3e-7 + 3 * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) + 1e-30
        assert (np.abs(got - want) <= tol).all(), form
        lim = gelu(o, "orc", np.array([[0.0, 20.0, -20.0]], np.float32), form)
        assert lim[0, 0] == 0.0 and lim[0, 1] == 20.0 and lim[0, 2] == 0.0
    heads, dim = 4, 64
    ones, zeros = np.ones((8, dim // 2), np.float32), np.zeros((8, dim // 2), np.float32)
    for il in (0, 1):
        assert np.array_equal(rope(o, "orc", x, heads, ones, zeros, il), x)
        q = rope(o, "orc", x, heads, zeros, ones, il).reshape(8, heads, -1)
        xr = x.reshape(8, heads, -1)
        first = np.arange(0, dim, 2) if il else np.arange(dim // 2)
        second = first + 1 if il else first + dim // 2
        assert np.array_equal(q[..., first], -xr[..., second]) and np.array_equal(q[..., second], xr[..., first])
        th = rng.uniform(0, 6.3, (8, dim // 2))
        r = rope(o, "orc", x, heads, np.cos(th).astype(np.float32), np.sin(th).astype(np.float32), il).reshape(8, heads, -1)
        n0 = np.hypot(xr[..., first].astype(np.float64), xr[..., second])
        n1 = np.hypot(r[..., first].astype(np.float64), r[..., second])
        assert np.allclose(n0, n1, rtol=1e-6, atol=1e-6)
    b = rng.standard_normal(256).astype(np.float32)
    y = rng.standard_normal((8, 256)).astype(np.float32)
    assert np.array_equal(bias(o, "orc", x, b), x + b) and np.array_equal(add(o, "orc", x, y), x + y)


# ---- planted mistakes ----

MUTANTS = {
    1: "nearest_int without the fused multiply-add",
    2: "hsum8 summed left to right",
    3: "Q5_K min term without the fused multiply-add",
    4: "Q8_0 quantizer dividing by the fp16 scale",
    5: "Q5_K six-bit unpack, wrong high bits for sub-blocks 4..7",
    6: "Q8_K quantizer keeping the last largest |x|",
    7: "norm adding epsilon after the square root",
    8: "norm multiplying by the weight before the inverse",
    9: "centered norm subtracting the mean in fp32",
    10: "SiLU as a reciprocal times v",
    11: "RoPE with the sine's sign flipped",
    12: "tanh GELU with v*v instead of v*v*v",
    13: "modulation as x + x*scale",
    14: "modulation by scale instead of 1 + scale",
    15: "attention's grouped heads as head % kv_heads",
    16: "causal attention without the query's own key",
    17: "l2norm without the sqrt(channels) factor",
    18: "l2norm adding epsilon instead of taking the larger",
    19: "groupnorm variance over n - 1",
    20: "groupnorm weight and bias indexed by group",
    21: "BF16 decoded as F16",
    22: "F16 decode keeping the NaN payload",
    23: "scatter keeping the first of a repeated row",
    24: "patch layout with dx and dy swapped",
    25: "upsample reading rows of the doubled width",
    26: "shortcut (down) without the division by the group",
    27: "shortcut (up) from the first time step",
    28: "qwen modulation with the two parameter rows swapped",
    29: "residual gate without tanh",
    30: "affine adding the bias before the scale",
    31: "convolution patches with the kernel's x and y swapped",
    32: "convolution padding taken from the right instead of the left",
}


def golden_mismatches(lib):
    """How many golden comparisons an oracle build fails."""
    bad = 0
    g1 = np.load(os.path.join(GOLDEN, "g1_quantize_q8_0.npz"))
    bad += int(not np.array_equal(quantize(lib, "orc", g1["x"], "q8_0"), g1["blocks"]))
    g2 = np.load(os.path.join(GOLDEN, "g2_quantize_q8_K.npz"))
    bad += int(not np.array_equal(quantize(lib, "orc", g2["x"], "q8_K"), g2["blocks"]))
    g3 = np.load(os.path.join(GOLDEN, "g3_dots.npz"))
    for wname, wtype in (("q8_0", Q8_0), ("q5_K", Q5_K), ("q6_K", Q6_K)):
        for k in (256, 512, 3840):
            w, a, y = g3[f"{wname}_{k}_w"], g3[f"{wname}_{k}_a"], g3[f"{wname}_{k}_y"]
            got = np.array([dot(lib, "orc", wtype, w[i], a[i], k) for i in range(len(y))], np.float32)
            bad += int(not np.array_equal(got.view(np.uint32), y.view(np.uint32)))
    g4 = np.load(os.path.join(GOLDEN, "g4_matmul.npz"))
    for c in range(int(g4["count"])):
        wtype, m, n, k = (int(v) for v in g4[f"c{c}_shape"])
        y = quant_matmul(lib, "orc", g4[f"c{c}_w"], wtype, g4[f"c{c}_x"], n, threads=2)
        bad += int(not np.array_equal(y.view(np.uint32), g4[f"c{c}_y"].view(np.uint32)))
    g5 = np.load(os.path.join(GOLDEN, "g5_norm.npz"))
    for centered in (0, 1):
        for wi in ("none", "w"):
            y = norm_rows(lib, "orc", g5["x"], None if wi == "none" else g5["w"], float(g5["eps"][centered]), centered)
            bad += int(not np.array_equal(y.view(np.uint32), g5[f"c{centered}_{wi}_y"].view(np.uint32)))
    g6 = np.load(os.path.join(GOLDEN, "g6_silu_gate.npz"))
    y = silu_gate(lib, "orc", g6["gate"], g6["up"])
    bad += int(not np.array_equal(y.view(np.uint32), g6["y"].view(np.uint32)))
    g7 = np.load(os.path.join(GOLDEN, "g7_ops.npz"))
    h = int(g7["heads"])
    for got, want in ((gelu(lib, "orc", g7["x"], 0), g7["gelu_exact"]), (gelu(lib, "orc", g7["x"], 1), g7["gelu_tanh"]),
                      (bias(lib, "orc", g7["x"], g7["b"]), g7["bias"]), (add(lib, "orc", g7["x"], g7["y"]), g7["add"]),
                      (rope(lib, "orc", g7["x"], h, g7["cos"], g7["sin"], 0), g7["rope_split"]),
                      (rope(lib, "orc", g7["x"], h, g7["cos"], g7["sin"], 1), g7["rope_interleaved"])):
        bad += int(not np.array_equal(got.view(np.uint32), want.view(np.uint32)))
    g9 = np.load(os.path.join(GOLDEN, "g9_attention.npz"))
    for c in range(int(g9["count"])):
        rows, keys, heads, kvh, dim, causal, offset = (int(v) for v in g9[f"c{c}_shape"])
        ranges = [tuple(int(x) for x in r) for r in g9[f"c{c}_ranges"]] or None
        got = attention(lib, "orc", g9[f"c{c}_q"], g9[f"c{c}_k"], g9[f"c{c}_v"], heads, kvh, ranges, offset, causal=bool(causal))
        bad += int(got is None or not np.array_equal(got.view(np.uint32), g9[f"c{c}_y"].view(np.uint32)))
    bad += tensor_ops_mismatches(lib)
    bad += conv_mismatches(lib)
    return bad


def g11_weight(g, c):
    """The fp32 values of case c's weight [cout][cin*ky*kx] (F32, F16 or BF16 bytes)."""
    wd, ht, cin, cout, kx, ky, wtype, _ = (int(v) for v in g[f"c{c}_shape"])
    raw = g[f"c{c}_w"]
    if wtype == 1:
        w = raw.view(np.float16).astype(np.float32)
    elif wtype == 30:
        w = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        w = raw.view(np.float32)
    return w.reshape(cout, cin * ky * kx)


def conv_mismatches(lib, tol=1e-5):
    """How many g11 cases (the reference's tensor_conv) the oracle's
    orc_conv2d misses by more than `tol` of an output row's largest value
    (the oracle sums in double, the reference in fp32 FMA tiles)."""
    g = np.load(os.path.join(GOLDEN, "g11_conv.npz"))
    bad = 0
    for c in range(int(g["count"])):
        wd, ht, cin, cout, kx, ky, wtype, has_bias = (int(v) for v in g[f"c{c}_shape"])
        geom = tuple(int(v) for v in g[f"c{c}_geometry"]) or None
        y = conv2d(lib, g[f"c{c}_x"], wd, ht, g11_weight(g, c), kx, ky, g[f"c{c}_b"] if has_bias else None, geom)
        want = g[f"c{c}_y"]
        if y is None or y.shape != want.shape:
            bad += 1
            continue
        err = np.abs(y.astype(np.float64) - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-30)
        bad += int(err.max() > tol)
    return bad


def tensor_ops_mismatches(lib):
    """How many of the g10 comparisons (the reference's tensor_l2norm,
    tensor_groupnorm, cpu_decode, tensor_gather / _scatter, tensor_upsample and
    tensor_resample_shortcut outputs) an oracle build fails."""
    g = np.load(os.path.join(GOLDEN, "g10_tensor_ops.npz"))

    def differs(got, want):
        return int(got is None or not np.array_equal(np.asarray(got, np.float32).view(np.uint32), want.view(np.uint32)))
    bad = differs(l2norm(lib, "orc", g["l2_x"], None, 1e-12), g["l2_y0"])
    bad += differs(l2norm(lib, "orc", g["l2_x"], g["l2_w"], 1e-12), g["l2_y1"])
    bad += differs(l2norm(lib, "orc", g["l2_x"], g["l2_w"], 0.5), g["l2_y2"])
    for n in ("gn", "gn2", "gn3"):
        bad += differs(groupnorm(lib, "orc", g[f"{n}_x"], g[f"{n}_w"], g[f"{n}_b"]), g[f"{n}_y"])
    for key, wtype in (("f16", F16), ("bf16", BF16), ("f32", F32), ("q8_0", Q8_0), ("q5_K", Q5_K), ("q6_K", Q6_K)):
        want = g[f"dec_{key}_y"]
        bad += differs(decode_f32(lib, "orc", g[f"dec_{key}"], wtype, want.size), want)
    bad += differs(gather(lib, "orc", g["rows_src"], g["gather_rows"]), g["gather_y"])
    bad += differs(scatter(lib, "orc", g["scatter_dst"], g["rows_src"], g["scatter_rows"]), g["scatter_y"])
    bad += differs(layout(lib, OP_UPSAMPLE, g["up_x"], 6, 4, 8), g["up_y"])
    for i, (wd, ht, cin, ch, t, up, sp) in enumerate(g["sc_cases"]):
        bad += differs(shortcut(lib, "orc", g[f"sc_x{i}"], int(wd), int(ht), int(ch), int(t), int(up), int(sp)), g[f"sc_y{i}"])
    return bad


def surface_mismatches(lib):
    """The ops the reference keeps static or inline, which cannot be linked
    here (z_residual, src/inference.cpp:279-291; the VAE and sampler affine
    steps as vulkan_pointwise runs them, :474-476, :612-631; qwen_image_euler
    and qwen_image_modulate, src/qwen_image.cpp:149-169, :347-361; the DiT patch
    loops, src/inference.cpp:374-390, :438-455), against what fixes them:
      residual: gate 0 leaves x; gate 20 (tanhf(20) = 1 in fp32) gives fl(x + o);
        no gate gives fl(x + o);
      affine, scale 2 and bias 1: fl(2x + 1) (2x is exact);
      euler, scale 0.5: fl(x + o/2) (o/2 is exact);
      qwen modulation, parameter row 0 = 0 and row 1 = s: target rows unchanged,
        rows before them x * fl(1 + s) rounded once; with a residual and row 0
        = 20, row 1 = 0: fl(x + r) on target rows, x before them;
      patch: the reshape of pixels [H, W, C] into [H/p, p, W/p, p, C], axes
        (0, 2, 1, 3, 4), then tokens; unpatch inverts it.
    Sums of two fp32 values are formed in float64 (exact here: operands of
    similar magnitude) and rounded once."""
    bad = 0
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((5, 48)) + 0.5).astype(np.float32)
    o = rng.standard_normal((5, 48)).astype(np.float32)
    xd, od = x.astype(np.float64), o.astype(np.float64)

    def same(a, b):
        return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))
    bad += int(not same(channel_op(lib, OP_RESIDUAL, x, o, np.zeros(48, np.float32)), x))
    bad += int(not same(channel_op(lib, OP_RESIDUAL, x, o, np.full(48, 20.0, np.float32)), (xd + od).astype(np.float32)))
    bad += int(not same(channel_op(lib, OP_RESIDUAL, x, o, None), (xd + od).astype(np.float32)))
    bad += int(not same(channel_op(lib, OP_AFFINE, x, scale=2.0, bias=1.0), (2.0 * xd + 1.0).astype(np.float32)))
    bad += int(not same(channel_op(lib, OP_EULER, x, o, scale=0.5), (xd + 0.5 * od).astype(np.float32)))
    s = (rng.standard_normal(48) * 0.3).astype(np.float32)
    params = np.zeros((2, 96), np.float32)
    params[1, 48:] = s
    got = qwen_modulate(lib, x, params, 3, 1)
    one_plus = (1.0 + s.astype(np.float64)).astype(np.float32).astype(np.float64)
    want = np.concatenate([(xd[:3] * one_plus).astype(np.float32), x[3:]])
    bad += int(got is None or not same(got, want))
    params[0, :48], params[1, :48] = 20.0, 0.0
    got = qwen_modulate(lib, x, params, 2, 0, residual=o)
    want = np.concatenate([x[:2], (xd[2:] + od[2:]).astype(np.float32)])
    bad += int(got is None or not same(got, want))
    bad += int(qwen_modulate(lib, x, params, 2, 2) is not None)  # (part + 1) * channels > parameter channels
    h, w, c, p = 6, 8, 4, 2
    img = rng.standard_normal((h * w, c)).astype(np.float32)
    tokens = img.reshape(h // p, p, w // p, p, c).transpose(0, 2, 1, 3, 4).reshape(h * w // (p * p), p * p * c)
    got = layout(lib, OP_PATCH, img, w, h, c, p)
    bad += int(not same(got, tokens))
    bad += int(not same(layout(lib, OP_UNPATCH, tokens, w, h, c, p), img))
    return bad


def modulation_mismatches(lib):
    """orc_modulate_rows (z_modulate, src/inference.cpp:263-277:
    x * (1.0f + scale[c]) in fp32) against what fixes it without the reference,
    which cannot be linked here (z_modulate is static in inference.cpp):
      scale 0 is the identity, bit for bit;  scale -1 gives x * 0 (signed zeros);
      scale 1 doubles exactly;  scale 2^-24 rounds 1 + scale to 1, so 1.5 stays
      1.5 (x + x*scale would give 1.5 + 2^-23);  and on random values the single
      rounding of the product of x and the rounded 1 + scale, computed in float64
      and rounded once (exact: both factors have 24-bit significands)."""
    bad = 0
    rng = np.random.default_rng(23)
    x = (rng.standard_normal((6, 64)) * 10.0 ** rng.integers(-3, 4, (6, 1))).astype(np.float32)
    x[0, :4] = [1.5, -1.5, 3.0, -0.0]
    for s_val, want in ((0.0, x), (-1.0, x * np.float32(0.0)), (1.0, x * np.float32(2.0))):
        got = modulate_rows(lib, x, np.full(64, s_val, np.float32))
        bad += int(not np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32)))
    s = np.zeros(64, np.float32)
    s[:4] = 2.0 ** -24
    got = modulate_rows(lib, x[:1], s)
    bad += int(not np.array_equal(got[0, :4].view(np.uint32), x[0, :4].view(np.uint32)))
    s = (rng.standard_normal(64) * 0.3).astype(np.float32)
    one_plus = (1.0 + s.astype(np.float64)).astype(np.float32)  # the fp32 sum: one rounding of an exact double sum
    want = (x.astype(np.float64) * one_plus.astype(np.float64)).astype(np.float32)
    bad += int(not np.array_equal(modulate_rows(lib, x, s).view(np.uint32), want.view(np.uint32)))
    return bad


def test_unmutated_oracle_passes_every_golden_comparison():
    assert golden_mismatches(oracle()) == 0


def test_modulation_closed_forms():
    assert modulation_mismatches(oracle()) == 0


def test_surface_closed_forms():
    assert surface_mismatches(oracle()) == 0


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_golden_vectors_catch_planted_mistake(mutant, tmp_path):
    so = tmp_path / f"liboracle_m{mutant}.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-pthread",
                    f"-DORC_MUTANT={mutant}", os.path.join(ORACLE_DIR, "pix_oracle.c"), "-o", str(so), "-lm"],
                   check=True, capture_output=True)
    lib = load_oracle(str(so))
    assert golden_mismatches(lib) + modulation_mismatches(lib) + surface_mismatches(lib) > 0, MUTANTS[mutant]
