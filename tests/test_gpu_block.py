"""One Z-Image DiT block, z_block (src/inference.cpp:293-345), end to end
through the C ABI (pixelina_amd/zimage.py: norm + modulation fused with the
Q8_K quantizer, the qkv GEMM, the q / k / v slices, head norms, interleaved
RoPE, 30-head attention, the out GEMM, norm + gated residual, the FFN with
its fused SiLU-gate quantizer, and the last norm + residual), at the DiT's
shape -- 4608 tokens (512 caption rows, then a 64 x 64 patch grid), hidden
3840, Q5_K linears with a Q8_0 FFN-down as in the bench's block workload --
and in the refiner's form (no timestep: no modulation, ungated residuals).

The block runs op by op with every op's outputs copied back, and each op is
held to its own bar against the oracle op (oracle/pix_oracle.c) applied to
the GPU's inputs of that op: bit-exact for the norms, slices and RoPE, 1e-4
per row (TOL) for the linears (norm, modulation and quantizer included) and
the attention, an ulp for the tanh-gated residuals.  On the DiT shape the
oracle's attention and linears run on 32 sampled token rows (K and V come
from every row); the refiner's 128 rows are all checked.

The whole chain is also compared with the oracle chain from the same block
input, within CHAIN_TOL: a quantized linear turns an input difference at its
last bits into whole quantization steps wherever a value sits at a rounding
boundary, so the oracle chain itself moves by ~5e-3 of a row's magnitude
when its attention output is perturbed by 1e-5 (relative) -- less than the
attention kernel's own error bound.  CHAIN_TOL catches a wrong op, operand or
modulation slice (errors of order 1), not those steps.
"""
import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import Q5_K, Q8_0, attention, bias, channel_op, modulate_rows, norm_rows, oracle, quant_matmul, quantize, rope, \
    silu_gate
from pixelina_amd import synth, zimage
from pixelina_amd.zimage import HEAD_DIM, HEADS, HIDDEN, INTERMEDIATE, NORM_EPSILON, OP_RESIDUAL, ZBlock, ZBlockWeights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def make_block(seed, modulated):
    """Seeded block tensors: linears ~N(0, 0.02) (Q5_K, FFN-down Q8_0 via the
    oracle's quantize_row_q8_0, the modulation linear Q8_0), norm weights
    1 + N(0, 0.1), modulation bias N(0, 0.1)."""
    o = oracle()
    rng = np.random.default_rng(seed)
    lin = {}
    for key, (inner, rows) in ZBlockWeights.SHAPES.items():
        if key == "modulation" and not modulated:
            continue
        w = (rng.standard_normal((rows, inner), np.float32) * 0.02).astype(np.float32)
        if key in ("w2", "modulation"):
            lin[key] = (quantize(o, "orc", w, "q8_0"), Q8_0)
        else:
            lin[key] = (synth.pack_q5_K(w), Q5_K)
    vec = {k: (1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)
           for k in ("attention_norm1", "attention_norm2", "ffn_norm1", "ffn_norm2")}
    for k in ("q_norm", "k_norm"):
        vec[k] = (1.0 + 0.1 * rng.standard_normal(HEAD_DIM)).astype(np.float32)
    if modulated:
        vec["modulation_bias"] = (0.1 * rng.standard_normal(4 * HIDDEN)).astype(np.float32)
    return lin, vec


def oracle_block(lin, vec, x, cos, sin, pick, t=None):
    """z_block on the oracle: K and V for every row, the rest on rows `pick`.
    Returns (block output rows, attention output rows)."""
    o = oracle()
    mod = None
    if t is not None:
        w, ty = lin["modulation"]
        mod = bias(o, "orc", quant_matmul(o, "orc", w, ty, t, 4 * HIDDEN), vec["modulation_bias"])[0]

    def part(p):
        return mod[p * HIDDEN:(p + 1) * HIDDEN]

    def head_norm(a, key):
        return norm_rows(o, "orc", a.reshape(-1, HEAD_DIM), vec[key], NORM_EPSILON, False).reshape(a.shape)

    xn = norm_rows(o, "orc", x, vec["attention_norm1"], NORM_EPSILON, False)
    if mod is not None:
        xn = modulate_rows(o, xn, part(0))
    wqkv, ty = lin["qkv"]
    kv = quant_matmul(o, "orc", wqkv[HIDDEN:], ty, xn, 2 * HIDDEN)
    q = quant_matmul(o, "orc", wqkv[:HIDDEN], ty, xn[pick], HIDDEN)
    k, v = kv[:, :HIDDEN], np.ascontiguousarray(kv[:, HIDDEN:])
    q = rope(o, "orc", head_norm(q, "q_norm"), HEADS, cos[pick], sin[pick], 1)
    k = rope(o, "orc", head_norm(np.ascontiguousarray(k), "k_norm"), HEADS, cos, sin, 1)
    att = attention(o, "orc", q, k, v, HEADS, HEADS)

    def linear(key, a):
        w, ty = lin[key]
        return quant_matmul(o, "orc", w, ty, a, ZBlockWeights.SHAPES[key][1])

    y = x[pick].copy()
    res = norm_rows(o, "orc", linear("out", att), vec["attention_norm2"], NORM_EPSILON, False)
    y = channel_op(o, OP_RESIDUAL, y, res, None if mod is None else part(1))
    yn = norm_rows(o, "orc", y, vec["ffn_norm1"], NORM_EPSILON, False)
    if mod is not None:
        yn = modulate_rows(o, yn, part(2))
    h = silu_gate(o, "orc", linear("w1", yn), linear("w3", yn))
    res = norm_rows(o, "orc", linear("w2", h), vec["ffn_norm2"], NORM_EPSILON, False)
    y = channel_op(o, OP_RESIDUAL, y, res, None if mod is None else part(3))
    return y, att


CHAIN_TOL = 2e-2
ULP_TOL = 1e-6  # tanhf here correctly rounded, glibc's within about an ulp


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def check_block(sess, name, lin, vec, x, cos, sin, pick, t=None):
    """Runs the block op by op with snapshots; per-op and whole-chain checks."""
    o = oracle()
    rows = x.shape[0]
    wts = ZBlockWeights(sess, name, lin, vec)
    blk = ZBlock(sess, wts, rows, keep_gated=True)
    xb, cb, sb = sess.to_device(x), sess.to_device(cos), sess.to_device(sin)
    tb = None if t is None else sess.to_device(t)

    def dl(buf, cols):
        return buf.download(np.float32, rows * cols).reshape(rows, cols)

    writes = {"modulation": [("mod", blk.mod, None)], "qkv": [("qkv", blk.qkv, 3 * HIDDEN)],
              "split": [("q", blk.q, HIDDEN), ("k", blk.k, HIDDEN), ("v", blk.v, HIDDEN)],
              "head_norm": [("qn", blk.qn, HIDDEN), ("kn", blk.kn, HIDDEN)],
              "rope": [("qr", blk.qn, HIDDEN), ("kr", blk.kn, HIDDEN)], "attention": [("att", blk.att, HIDDEN)],
              "out": [("p1", blk.proj, HIDDEN)], "attention_norm2": [("r1", blk.res, HIDDEN)],
              "residual1": [("x1", xb, HIDDEN)], "w1": [("g", blk.gate, INTERMEDIATE)], "w3": [("u", blk.up, INTERMEDIATE)],
              "silu_gate": [("h", blk.gated, INTERMEDIATE)], "w2": [("p2", blk.proj, HIDDEN)],
              "ffn_norm2": [("r2", blk.res, HIDDEN)], "residual2": [("x2", xb, HIDDEN)]}
    g = {}
    for op, fn in blk.ops(xb.ptr, cb.ptr, sb.ptr, None if tb is None else tb.ptr):
        fn()
        sess.synchronize()
        for label, buf, cols in writes.get(op, []):
            g[label] = buf.download(np.float32, 4 * HIDDEN) if cols is None else dl(buf, cols)
    for b in (xb, cb, sb, tb):
        if b is not None:
            b.free()
    blk.free()
    wts.free()
    assert np.isfinite(g["x2"]).all()

    errs = {}

    def linear(key, a):
        w, ty = lin[key]
        return quant_matmul(o, "orc", w, ty, a, ZBlockWeights.SHAPES[key][1])

    def rel(label, got, want, tol):
        errs[label] = float(row_rel_error(got, want).max())
        assert errs[label] <= tol, (label, errs[label])

    def part(p):
        return None if t is None else g["mod"][p * HIDDEN:(p + 1) * HIDDEN]

    def norm(a, key, p=None):
        y = norm_rows(o, "orc", a, vec[key], NORM_EPSILON, False)
        return y if p is None else modulate_rows(o, y, p)

    if t is not None:
        w, ty = lin["modulation"]
        rel("modulation", g["mod"][None, :], bias(o, "orc", quant_matmul(o, "orc", w, ty, t, 4 * HIDDEN), vec["modulation_bias"]),
            TOL)
    rel("qkv", g["qkv"][pick], linear("qkv", norm(x[pick], "attention_norm1", part(0))), TOL)
    for i, label in enumerate(("q", "k", "v")):
        assert bits_equal(g[label], g["qkv"][:, i * HIDDEN:(i + 1) * HIDDEN]), label
    for src, dst, key in (("q", "qn", "q_norm"), ("k", "kn", "k_norm")):
        want = norm_rows(o, "orc", g[src][pick].reshape(-1, HEAD_DIM), vec[key], NORM_EPSILON, False).reshape(-1, HIDDEN)
        assert bits_equal(g[dst][pick], want), dst
    for src, dst in (("qn", "qr"), ("kn", "kr")):
        assert bits_equal(g[dst][pick], rope(o, "orc", g[src][pick], HEADS, cos[pick], sin[pick], 1)), dst
    rel("attention", g["att"][pick], attention(o, "orc", g["qr"][pick], g["kr"], g["v"], HEADS, HEADS), TOL)
    rel("out", g["p1"][pick], linear("out", g["att"][pick]), TOL)
    assert bits_equal(g["r1"][pick], norm(g["p1"][pick], "attention_norm2")), "attention_norm2"
    rel("residual1", g["x1"][pick], channel_op(o, OP_RESIDUAL, x[pick], g["r1"][pick], part(1)), ULP_TOL)
    a = norm(g["x1"][pick], "ffn_norm1", part(2))
    rel("w1", g["g"][pick], linear("w1", a), TOL)
    rel("w3", g["u"][pick], linear("w3", a), TOL)
    rel("silu_gate", g["h"][pick], silu_gate(o, "orc", g["g"][pick], g["u"][pick]), ULP_TOL)
    rel("w2", g["p2"][pick], linear("w2", g["h"][pick]), TOL)
    assert bits_equal(g["r2"][pick], norm(g["p2"][pick], "ffn_norm2")), "ffn_norm2"
    rel("residual2", g["x2"][pick], channel_op(o, OP_RESIDUAL, g["x1"][pick], g["r2"][pick], part(3)), ULP_TOL)

    ry, ratt = oracle_block(lin, vec, x, cos, sin, pick, t)
    errs["chain_attention"] = float(row_rel_error(g["att"][pick], ratt).max())
    errs["chain"] = float(row_rel_error(g["x2"][pick], ry).max())
    print("  " + ", ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    assert errs["chain"] <= CHAIN_TOL


def test_dit_block(sess):
    """The main DiT block (src/inference.cpp:422) at 512 caption + 4096 image
    tokens, with its timestep modulation; 32 sampled rows."""
    caption, image, pw = 512, 4096, 64
    rows = caption + image
    lin, vec = make_block(293, True)
    rng = np.random.default_rng(345)
    x = rng.standard_normal((rows, HIDDEN), np.float32)
    t = rng.standard_normal((1, zimage.TIME_DIM), np.float32)
    cc, cs = zimage.rotary(caption, 0, 0, False)
    ic, iS = zimage.rotary(image, caption, pw, True)
    cos, sin = np.concatenate([cc, ic]), np.concatenate([cs, iS])
    print(f"DiT block: {rows} tokens, hidden {HIDDEN}, {HEADS} heads of {HEAD_DIM}", flush=True)
    check_block(sess, "test:zblock", lin, vec, x, cos, sin, np.linspace(0, rows - 1, 32).astype(int), t)


def test_refiner_block(sess):
    """The context refiner's form (src/inference.cpp:399): no timestep, so no
    modulation and ungated residuals; 128 caption tokens, every row."""
    rows = 128
    lin, vec = make_block(399, False)
    x = np.random.default_rng(400).standard_normal((rows, HIDDEN), np.float32)
    cos, sin = zimage.rotary(rows, 0, 0, False)
    print(f"refiner block: {rows} tokens", flush=True)
    check_block(sess, "test:zrefiner", lin, vec, x, cos, sin, np.arange(rows))
