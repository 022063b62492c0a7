"""Writes the golden fixtures under tests/golden/ from the reference's own CPU
path, compiled in place from the reference sources (oracle/Makefile ->
oracle/_ref/libpixref.so).  Run in the build container only:

    make -C oracle ref && python tests/golden/make_golden.py

Fixtures (numpy .npz, data only):
  g1_quantize_q8_0.npz  quantize_row_q8_0_ref on crafted and random rows
  g2_quantize_q8_K.npz  quantize_row_q8_K_ref, incl. rows whose rounding
                        depends on the fused multiply-add of nearest_int
  g3_dots.npz           pix_dot_q8_0 / q5_K / q6_K on random rows
  g4_matmul.npz         cpu_quant_matmul on small shapes and a decode slice
  g5_norm.npz           tensor_norm (RMS and centered, with and without a
                        weight) on crafted and random rows, and the Q8_K /
                        Q8_0 blocks of its outputs
  g6_silu_gate.npz      tensor_silu then tensor_gate on special and random
                        values, and the Q8_K / Q8_0 blocks of the product
  g7_ops.npz            tensor_gelu (both forms), tensor_bias, tensor_add and
                        tensor_rope (split and interleaved halves)
  g9_attention.npz      tensor_attention, causal form and ranges form: MHA and
                        grouped heads, head sizes 64 / 72 / 128, causal and
                        not, ranges with a query offset; wide heads 200 / 384 /
                        512
  g10_tensor_ops.npz    tensor_l2norm, tensor_groupnorm (group widths 4, 2, 3),
                        cpu_decode of every type (fp16 specials, random
                        blocks), tensor_gather / tensor_scatter (repeated rows),
                        tensor_slice, tensor_upsample, tensor_resample_shortcut
                        (up and down, spatial or not, one or two time steps)
  g11_conv.npz          tensor_conv, both forms: 3x3 and 1x1 kernels, stride 2
                        with one-sided padding, a 3x1 kernel, 3 input channels,
                        F32 / F16 / BF16 weights, with and without a bias

    python tests/golden/make_golden.py g5 g6 g7   # only the named fixtures
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle_lib import (BF16, F16, F32, Q5_K, Q6_K, Q8_0, add, attention, bias, decode_f32, dot, gather,  # noqa: E402
                        gelu, groupnorm, l2norm, norm_rows, quant_matmul, quantize, reference, rope, scatter, shortcut,
                        silu_gate, upsample_ref, conv2d_ref)
from pixelina_amd import synth  # noqa: E402


def crafted_q8_0():
    rows = []
    z = np.zeros(32, np.float32)
    rows.append(z.copy())                                   # all zero -> d = 0, id = 0
    r = z.copy(); r[7] = 1.0; rows.append(r)                 # single spike
    r = z.copy(); r[0] = 127.0                              # d = 1, id = 1: exact .5 ties
    r[1:12] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 63.5, -63.5, 3.5]; rows.append(r)
    r = np.linspace(-1e-3, 1e-3, 32).astype(np.float32); rows.append(r)   # fp16-subnormal d
    r = np.linspace(-1e-6, 2e-6, 32).astype(np.float32); rows.append(r)   # deeper subnormal d
    r = np.linspace(-1e7, 9e6, 32).astype(np.float32); rows.append(r)     # d overflows fp16 -> inf
    r = np.linspace(-3.0, 1.0, 32).astype(np.float32); rows.append(r)     # negative max
    r = z.copy(); r[5] = np.nan; r[6] = 2.0; rows.append(r)              # NaN ignored by amax, quantizes to 0
    r = z.copy(); r[3] = np.inf; r[4] = -5.0; rows.append(r)             # infinite amax
    r = np.full(32, -7.25, np.float32); rows.append(r)                   # constant negative
    return np.stack(rows)


def crafted_q8_K():
    rows = []
    z = np.zeros(256, np.float32)
    rows.append(z.copy())
    r = z.copy(); r[100] = -3.0; rows.append(r)              # single negative spike
    r = z.copy(); r[3] = -5.0; r[10] = 5.0; rows.append(r)   # |max| tie: first (negative) wins
    r = z.copy(); r[3] = 5.0; r[10] = -5.0; rows.append(r)   # |max| tie: first (positive) wins
    r = np.linspace(-127, 127, 256).astype(np.float32); rows.append(r)
    r = np.linspace(-1e-30, 1e-30, 256).astype(np.float32); rows.append(r)  # tiny scale
    r = z.copy(); r[0] = np.nan; r[1] = 1.0; rows.append(r)  # NaN never wins the arg-max
    r = np.full(256, 2.5, np.float32); rows.append(r)        # constant positive
    return np.stack(rows)


def fused_tie_rows(count, seed=7):
    """Random N(0,1) rows where nearest_int(iscale*x) differs between a fused
    multiply-add and a rounded product (found by exact float64 arithmetic)."""
    rng = np.random.default_rng(seed)
    found = []
    while len(found) < count:
        x = rng.standard_normal((4096, 256)).astype(np.float32)
        ax = np.abs(x)
        mx = x[np.arange(x.shape[0]), np.argmax(ax, axis=1)]
        iscale = (np.float32(-127.0) / mx).astype(np.float32)
        p = iscale.astype(np.float64)[:, None] * x.astype(np.float64)   # exact product
        fused = np.rint(p)
        unfused = np.rint(p.astype(np.float32).astype(np.float64))
        hit = np.nonzero((fused != unfused).any(axis=1))[0]
        found.extend(x[h] for h in hit[: count - len(found)])
    return np.stack(found)


def norm_rows_crafted(k):
    rng = np.random.default_rng(55)
    rows = [np.zeros(k, np.float32),                                    # square 0: inverse = 1/sqrt(eps)
            np.full(k, 3.75, np.float32),                               # constant: centered -> 0
            np.linspace(-1e-20, 1e-20, k).astype(np.float32),           # eps dominates
            (rng.standard_normal(k) * 1e18).astype(np.float32),         # squares past fp32 range
            np.where(np.arange(k) == 17, 1000.0, 0.0).astype(np.float32),  # one spike
            (rng.standard_normal(k) + 40.0).astype(np.float32)]         # large mean
    return np.stack(rows)


def write_g5(ref):
    rng = np.random.default_rng(505)
    k = 512
    x = np.concatenate([norm_rows_crafted(k), (rng.standard_normal((10, k)) * rng.choice([1e-3, 1.0, 50.0], (10, 1))).astype(np.float32)])
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    g = {"x": x, "w": w, "eps": np.array([1e-5, 1e-6], np.float32)}
    for centered in (0, 1):
        for wi, wv in (("none", None), ("w", w)):
            eps = float(g["eps"][centered])
            y = norm_rows(ref, "ref", x, wv, eps, centered)
            key = f"c{centered}_{wi}"
            g[f"{key}_y"] = y
            g[f"{key}_q8_K"] = quantize(ref, "ref", y, "q8_K")
            g[f"{key}_q8_0"] = quantize(ref, "ref", y, "q8_0")
    np.savez_compressed(os.path.join(HERE, "g5_norm.npz"), **g)


def write_g6(ref):
    rng = np.random.default_rng(606)
    rows, k = 6, 512
    gate = (rng.standard_normal((rows, k)) * 6.0).astype(np.float32)
    up = rng.standard_normal((rows, k)).astype(np.float32)
    special = np.array([0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 89.0, -89.0, 104.0, -104.0, 200.0, -200.0,
                        20.0, -20.0, 0.5, -0.5], np.float32)
    gate[0, :special.size] = special
    up[0, :special.size] = 1.0
    y = silu_gate(ref, "ref", gate, up)
    np.savez_compressed(os.path.join(HERE, "g6_silu_gate.npz"), gate=gate, up=up, y=y,
                        q8_K=quantize(ref, "ref", y, "q8_K"), q8_0=quantize(ref, "ref", y, "q8_0"))


def write_g7(ref):
    rng = np.random.default_rng(707)
    rows, heads, dim = 5, 4, 64
    x = (rng.standard_normal((rows, heads * dim)) * 3.0).astype(np.float32)
    x[0, :12] = [0.0, -0.0, 1e-30, -1e-30, 10.0, -10.0, 6.0, -6.0, 40.0, -40.0, 0.5, -0.5]
    b = rng.standard_normal(heads * dim).astype(np.float32)
    y = rng.standard_normal((rows, heads * dim)).astype(np.float32)
    theta = rng.uniform(0, 2 * np.pi, (rows, dim // 2))
    cos, sin = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "g7_ops.npz"), x=x, b=b, y=y, cos=cos, sin=sin, heads=np.array(heads),
                        gelu_exact=gelu(ref, "ref", x, 0), gelu_tanh=gelu(ref, "ref", x, 1), bias=bias(ref, "ref", x, b),
                        add=add(ref, "ref", x, y), rope_split=rope(ref, "ref", x, heads, cos, sin, 0),
                        rope_interleaved=rope(ref, "ref", x, heads, cos, sin, 1))


# (rows, keys, heads, kv_heads, dim, causal, ranges or None, query_offset)
G9_CASES = [
    (33, 33, 4, 4, 64, 0, None, 0),
    (40, 40, 6, 2, 64, 1, None, 0),
    (24, 57, 2, 1, 72, 0, None, 0),
    (64, 64, 2, 2, 128, 1, None, 0),
    (30, 48, 4, 2, 64, 0, [(0, 7, 9, 1), (7, 30, 48, 0)], 5),
    (20, 20, 3, 1, 128, 0, [(0, 12, 12, 0), (12, 20, 20, 1)], 0),
    (24, 40, 1, 1, 512, 0, None, 0),          # the VAE's single wide head
    (25, 25, 2, 1, 384, 1, None, 0),
    (16, 24, 2, 2, 200, 0, [(0, 6, 11, 1), (6, 16, 24, 0)], 4),
]


def write_g9(ref):
    rng = np.random.default_rng(909)
    g = {"count": np.array(len(G9_CASES))}
    for c, (rows, keys, heads, kvh, dim, causal, ranges, offset) in enumerate(G9_CASES):
        q = (rng.standard_normal((rows, heads * dim)) * 1.5).astype(np.float32)
        k = (rng.standard_normal((keys, kvh * dim)) * 1.5).astype(np.float32)
        v = rng.standard_normal((keys, kvh * dim)).astype(np.float32)
        y = attention(ref, "ref", q, k, v, heads, kvh, ranges, offset, causal=bool(causal))
        assert y is not None
        g[f"c{c}_shape"] = np.array([rows, keys, heads, kvh, dim, causal, offset])
        g[f"c{c}_ranges"] = np.array(ranges if ranges else [], np.uint64).reshape(-1, 4)
        g[f"c{c}_q"], g[f"c{c}_k"], g[f"c{c}_v"], g[f"c{c}_y"] = q, k, v, y
    np.savez_compressed(os.path.join(HERE, "g9_attention.npz"), **g)


# (width, height, in_channels, channels, temporal, up, spatial)
G10_SHORTCUTS = [
    (3, 2, 16, 8, 2, 1, 1),
    (4, 6, 8, 16, 2, 0, 1),
    (3, 3, 12, 24, 2, 1, 0),
    (3, 3, 24, 12, 2, 0, 0),
    (2, 2, 32, 8, 1, 1, 1),
    (4, 4, 8, 32, 1, 0, 1),
]


def random_blocks(rng, wtype, nblocks):
    """Random block bytes with finite fp16 scales (exponent field below 31)."""
    size, scales = {Q8_0: (34, (0,)), Q5_K: (176, (0, 2)), Q6_K: (210, (208,))}[wtype]
    b = rng.integers(0, 256, (nblocks, size), dtype=np.uint8)
    for off in scales:
        b[:, off + 1] = (b[:, off + 1] & 0x83) | (rng.integers(0, 30, nblocks, dtype=np.uint8) << 2 & 0x7c)
    return b.reshape(-1)


def write_g10(ref):
    rng = np.random.default_rng(1010)
    g = {}
    # l2norm: crafted rows (zero, tiny where epsilon wins, large) and random ones
    x = (rng.standard_normal((24, 96)) * rng.choice([1e-3, 1.0, 50.0], (24, 1))).astype(np.float32)
    x[0] = 0.0
    x[1] = 1e-7
    x[2, ::2] = -3e4
    w = (1.0 + 0.2 * rng.standard_normal(96)).astype(np.float32)
    g["l2_x"], g["l2_w"] = x, w
    g["l2_eps"] = np.array([1e-12, 0.5], np.float32)
    g["l2_y0"] = l2norm(ref, "ref", x, None, 1e-12)
    g["l2_y1"] = l2norm(ref, "ref", x, w, 1e-12)
    g["l2_y2"] = l2norm(ref, "ref", x, w, 0.5)
    # groupnorm: group widths 4 (128 channels), 2 (64) and 3 (96)
    for name, rows, ch in (("gn", 37, 128), ("gn2", 5, 64), ("gn3", 70, 96)):
        xg = (rng.standard_normal((rows, ch)) * rng.uniform(0.1, 4.0, ch) + rng.uniform(-3, 3, ch)).astype(np.float32)
        wg = (1.0 + 0.3 * rng.standard_normal(ch)).astype(np.float32)
        bg = (0.2 * rng.standard_normal(ch)).astype(np.float32)
        g[f"{name}_x"], g[f"{name}_w"], g[f"{name}_b"] = xg, wg, bg
        g[f"{name}_y"] = groupnorm(ref, "ref", xg, wg, bg)
    # decode: every type
    halves = np.concatenate([np.arange(0, 64, dtype=np.uint16), np.arange(0x7bf0, 0x7c10, dtype=np.uint16),
                             np.arange(0xfbf8, 0xfc08, dtype=np.uint16), np.array([0x7e00, 0xfe00, 0x7d01, 0x8000, 0x3c00], np.uint16),
                             rng.integers(0, 65536, 1024, dtype=np.uint64).astype(np.uint16)])
    g["dec_f16"] = halves.view(np.uint8)
    g["dec_bf16"] = rng.integers(0, 65536, 1024, dtype=np.uint64).astype(np.uint16).view(np.uint8)
    g["dec_f32"] = rng.standard_normal(256).astype(np.float32).view(np.uint8)
    g["dec_q8_0"] = random_blocks(rng, Q8_0, 16)
    g["dec_q5_K"] = random_blocks(rng, Q5_K, 8)
    g["dec_q6_K"] = random_blocks(rng, Q6_K, 8)
    for key, wtype, count in (("f16", F16, halves.size), ("bf16", BF16, 1024), ("f32", F32, 256), ("q8_0", Q8_0, 16 * 32),
                              ("q5_K", Q5_K, 8 * 256), ("q6_K", Q6_K, 8 * 256)):
        g[f"dec_{key}_y"] = decode_f32(ref, "ref", g[f"dec_{key}"], wtype, count)
    # rows: gather with repeats, scatter with a repeated destination row
    src = rng.standard_normal((9, 12)).astype(np.float32)
    g["rows_src"] = src
    g["gather_rows"] = np.array([3, 0, 8, 3, 5], np.uint64)
    g["gather_y"] = gather(ref, "ref", src, g["gather_rows"])
    dst = rng.standard_normal((7, 12)).astype(np.float32)
    g["scatter_dst"] = dst
    g["scatter_rows"] = np.array([6, 1, 6, 0, 2, 4, 3, 1, 5], np.uint64)
    g["scatter_y"] = scatter(ref, "ref", dst, src, g["scatter_rows"])
    # slices (row, rows, feature, channels) of a 10 x 20 tensor
    xs = rng.standard_normal((10, 20)).astype(np.float32)
    g["slice_x"] = xs
    g["slice_cases"] = np.array([[0, 10, 0, 20], [3, 4, 5, 7], [9, 1, 19, 1], [2, 8, 0, 20]], np.int64)
    for i, (r0, nr, f0, nc) in enumerate(g["slice_cases"]):
        out = np.full((nr, nc), np.nan, np.float32)
        assert ref.ref_slice(xs.ctypes.data, 10, 20, int(r0), int(nr), int(f0), int(nc), out.ctypes.data)
        g[f"slice_y{i}"] = out
    # upsample 6 x 4 pixels of 8 channels
    xu = rng.standard_normal((24, 8)).astype(np.float32)
    g["up_x"], g["up_y"] = xu, upsample_ref(ref, xu, 6, 4)
    # shortcuts
    g["sc_cases"] = np.array(G10_SHORTCUTS, np.int64)
    for i, (wd, ht, cin, ch, t, up, sp) in enumerate(G10_SHORTCUTS):
        xi = rng.standard_normal((wd * ht, cin)).astype(np.float32)
        y = shortcut(ref, "ref", xi, wd, ht, ch, t, up, sp)
        assert y is not None, G10_SHORTCUTS[i]
        g[f"sc_x{i}"], g[f"sc_y{i}"] = xi, y
    np.savez_compressed(os.path.join(HERE, "g10_tensor_ops.npz"), **g)


# (width, height, cin, cout, kx, ky, weight type, bias, geometry or None)
G11_CASES = [
    (12, 10, 32, 40, 3, 3, F32, True, None),
    (9, 7, 16, 48, 1, 1, F16, True, None),
    (11, 9, 8, 16, 3, 3, BF16, False, (2, 2, 0, 1, 0, 1)),
    (8, 6, 12, 20, 3, 1, F32, True, (1, 1, 1, 1, 0, 0)),
    (10, 10, 3, 24, 3, 3, F16, True, None),
]


def write_g11(ref):
    rng = np.random.default_rng(1111)
    g = {"count": np.array(len(G11_CASES))}
    for c, (wd, ht, cin, cout, kx, ky, wtype, has_bias, geom) in enumerate(G11_CASES):
        x = rng.standard_normal((wd * ht, cin)).astype(np.float32)
        w = (rng.standard_normal((cout, cin * ky * kx)) / np.sqrt(cin * kx * ky)).astype(np.float32)
        if wtype == F16:
            wb = w.astype(np.float16).view(np.uint8)
        elif wtype == BF16:
            wb = (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        else:
            wb = w.view(np.uint8)
        b = rng.standard_normal(cout).astype(np.float32) if has_bias else None
        y = conv2d_ref(ref, x, wd, ht, wb, wtype, kx, ky, cin, cout, b, geom)
        assert y is not None, G11_CASES[c]
        g[f"c{c}_shape"] = np.array([wd, ht, cin, cout, kx, ky, wtype, int(has_bias)])
        g[f"c{c}_geometry"] = np.array(geom if geom else [], np.int64)
        g[f"c{c}_x"], g[f"c{c}_w"], g[f"c{c}_y"] = x, np.ascontiguousarray(wb).reshape(-1), y
        if has_bias:
            g[f"c{c}_b"] = b
    np.savez_compressed(os.path.join(HERE, "g11_conv.npz"), **g)


def main():
    ref = reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libpixref.so missing: run `make -C oracle ref` first")
    only = set(sys.argv[1:])
    if only:
        if "g5" in only:
            write_g5(ref)
        if "g6" in only:
            write_g6(ref)
        if "g7" in only:
            write_g7(ref)
        if "g9" in only:
            write_g9(ref)
        if "g10" in only:
            write_g10(ref)
        if "g11" in only:
            write_g11(ref)
        return
    rng = np.random.default_rng(20260101)

    # G1
    x1 = np.concatenate([crafted_q8_0(), (rng.standard_normal((24, 32)) * rng.choice([1e-2, 1, 30], (24, 1))).astype(np.float32)])
    b1 = quantize(ref, "ref", x1, "q8_0")
    np.savez_compressed(os.path.join(HERE, "g1_quantize_q8_0.npz"), x=x1, blocks=b1)

    # G2
    ties = fused_tie_rows(12)
    x2 = np.concatenate([crafted_q8_K(), ties, rng.standard_normal((12, 256)).astype(np.float32) * 3])
    b2 = quantize(ref, "ref", x2, "q8_K")
    np.savez_compressed(os.path.join(HERE, "g2_quantize_q8_K.npz"), x=x2, blocks=b2, fused_rows=np.arange(8, 8 + len(ties)))

    # G3: dots on random rows
    g3 = {}
    for wtype, name in ((Q8_0, "q8_0"), (Q5_K, "q5_K"), (Q6_K, "q6_K")):
        for k in (256, 512, 3840):
            n = 12
            wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            if wtype == Q8_0:
                wb = quantize(ref, "ref", wf, "q8_0")
            elif wtype == Q5_K:
                wb = synth.pack_q5_K(wf)
            else:
                wb = synth.pack_q6_K(wf)
            xf = rng.standard_normal((n, k)).astype(np.float32)
            xf[:, rng.integers(0, k, 3)] *= 20.0
            ab = quantize(ref, "ref", xf, "q8_0" if wtype == Q8_0 else "q8_K")
            y = np.array([dot(ref, "ref", wtype, wb[i], ab[i], k) for i in range(n)], dtype=np.float32)
            g3[f"{name}_{k}_w"] = wb
            g3[f"{name}_{k}_x"] = xf
            g3[f"{name}_{k}_a"] = ab
            g3[f"{name}_{k}_y"] = y
    np.savez_compressed(os.path.join(HERE, "g3_dots.npz"), **g3)

    # G4: cpu_quant_matmul, small shapes + a decode-row slice of the 18944x3584 matvec
    g4 = {}
    cases = []
    for wtype, name in ((Q8_0, "q8_0"), (Q5_K, "q5_K"), (Q6_K, "q6_K")):
        for m in (1, 3):
            for n in (5, 17):
                for k in (256, 3840):
                    cases.append((wtype, name, m, n, k))
        cases.append((wtype, name, 1, 64, 3584))
    for i, (wtype, name, m, n, k) in enumerate(cases):
        wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        if wtype == Q8_0:
            wb = quantize(ref, "ref", wf, "q8_0")
        elif wtype == Q5_K:
            wb = synth.pack_q5_K(wf)
        else:
            wb = synth.pack_q6_K(wf)
        xf = rng.standard_normal((m, k)).astype(np.float32)
        y = quant_matmul(ref, "ref", wb, wtype, xf, n)
        g4[f"c{i}_w"] = wb
        g4[f"c{i}_x"] = xf
        g4[f"c{i}_y"] = y
        g4[f"c{i}_shape"] = np.array([wtype, m, n, k], dtype=np.int64)
    g4["count"] = np.array(len(cases))
    np.savez_compressed(os.path.join(HERE, "g4_matmul.npz"), **g4)
    write_g5(ref)
    write_g6(ref)
    write_g7(ref)
    write_g9(ref)
    write_g10(ref)
    write_g11(ref)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
