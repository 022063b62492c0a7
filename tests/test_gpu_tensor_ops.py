"""The rest of the backend op surface through the C ABI (pixhip_pointwise_ex,
pixhip_qwen_modulate, pixhip_l2norm, pixhip_groupnorm, pixhip_embedding,
pixhip_rows, pixhip_copy_rows, pixhip_copy_features, pixhip_layout,
pixhip_shortcut), against the reference's own outputs (tests/golden/
g10_tensor_ops, written by the compiled src/tensor.cpp and src/backend_cpu.cpp)
and the oracle (oracle/pix_oracle.c) at the models' shapes.

Bit-exact throughout, except the ops with a tanh (z_residual's gate and
qwen_image_modulate's residual form): the reference's glibc tanhf is not
correctly rounded, the kernel's tanh is, so those are held to 4 ulps of the
result plus 4 ulps of tanh scaled by the residual term.  The norms' double sums
are formed in another order than the reference's; their fp32 outputs are
still required to be bit-identical (a different double moves an fp32 result
only when it lands within its last bits of a rounding boundary).
"""
import os

import numpy as np
import pytest

from oracle_lib import (BF16, F16, F32, OP_AFFINE, OP_EULER, OP_PATCH, OP_RESIDUAL, OP_UNPATCH, OP_UPSAMPLE, Q5_K, Q6_K, Q8_0,
                        channel_op, decode_f32, gather, groupnorm, l2norm, layout, oracle, qwen_modulate, scatter, shortcut)
from pixelina_amd import _lib

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
OP_MODULATE = 8
ROW_BYTES = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q5_K: (256, 176), Q6_K: (256, 210)}


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


@pytest.fixture(scope="module")
def g10():
    return np.load(os.path.join(GOLDEN, "g10_tensor_ops.npz"))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same(a, b):
    return a.shape == b.shape and np.array_equal(bits(a), bits(b))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Dev:
    """Device copies of numpy arrays for one call, freed together."""

    def __init__(self, sess):
        self.sess, self.bufs = sess, []

    def up(self, a):
        b = self.sess.to_device(np.ascontiguousarray(a))
        self.bufs.append(b)
        return b.ptr

    def out(self, shape):
        b = self.sess.alloc(int(np.prod(shape)) * 4)
        self.bufs.append((b, shape))
        return b.ptr

    def get(self, ptr):
        for b in self.bufs:
            if isinstance(b, tuple) and b[0].ptr == ptr:
                return b[0].download(np.float32, int(np.prod(b[1]))).reshape(b[1])
        raise KeyError(ptr)

    def free(self):
        for b in self.bufs:
            (b[0] if isinstance(b, tuple) else b).free()


def inplace(sess, x, fn):
    """Run fn(dev, x_ptr) on a device copy of x and return it."""
    d = Dev(sess)
    xb = sess.to_device(f32(x))
    try:
        fn(d, xb.ptr)
        return xb.download(np.float32, x.size).reshape(x.shape)
    finally:
        xb.free()
        d.free()


def call_out(sess, shape, fn):
    """Run fn(dev, out_ptr) and return the output array."""
    d = Dev(sess)
    try:
        op = d.out(shape)
        fn(d, op)
        return d.get(op)
    finally:
        d.free()


def tanh_close(got, want, term):
    """Within 4 ulps of the result plus 4 ulps of tanh scaled by |term|."""
    got, want, term = (np.asarray(a, np.float64) for a in (got, want, term))
    tol = 4 * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) + 4 * np.abs(term) * 2.0 ** -24
    off = np.abs(got - want)
    print(f"tanh ops: {np.mean(off == 0):.4f} bit-exact, max {off.max():.3g}", flush=True)
    return bool((off <= tol).all())


# ---- golden vectors ----

def test_l2norm_golden(sess, g10):
    x = g10["l2_x"]
    for key, w, eps in (("l2_y0", None, 1e-12), ("l2_y1", g10["l2_w"], 1e-12), ("l2_y2", g10["l2_w"], 0.5)):
        y = call_out(sess, x.shape, lambda d, o: _lib.check(
            sess.l2norm(d.up(x), x.shape[0], x.shape[1], d.up(w) if w is not None else None, eps, o), "l2norm"))
        assert same(y, g10[key]), key


def test_groupnorm_golden(sess, g10):
    for n in ("gn", "gn2", "gn3"):
        x = g10[f"{n}_x"]
        print(f"groupnorm golden {n}: {x.shape}", flush=True)
        y = call_out(sess, x.shape, lambda d, o: _lib.check(
            sess.groupnorm(d.up(x), x.shape[0], x.shape[1], d.up(g10[f"{n}_w"]), d.up(g10[f"{n}_b"]), o), "groupnorm"))
        assert same(y, g10[f"{n}_y"]), n


@pytest.mark.parametrize("on_device", [False, True])
def test_embedding_decodes_golden(sess, g10, on_device):
    """Each decode fixture as a table of rows (one block per row for the block
    types), gathered in a shuffled order with repeats."""
    for key, wtype in (("f16", F16), ("bf16", BF16), ("f32", F32), ("q8_0", Q8_0), ("q5_K", Q5_K), ("q6_K", Q6_K)):
        raw, want = g10[f"dec_{key}"], g10[f"dec_{key}_y"]
        block, nbytes = ROW_BYTES[wtype]
        inner = block if block > 1 else want.size
        table = raw.reshape(-1, inner // block * nbytes)
        rows = table.shape[0]
        ids = [rows - 1, 0, rows // 2, 0] if rows > 1 else [0, 0]
        print(f"embedding {key}: {rows} rows of {inner}, device table {on_device}", flush=True)
        d = Dev(sess)
        try:
            tp = d.up(table) if on_device else table.ctypes.data
            out = d.out((len(ids), inner))
            _lib.check(sess.embedding(tp, wtype, inner, rows, ids, out), "embedding")
            y = d.get(out)
        finally:
            d.free()
        assert same(y, want.reshape(rows, inner)[ids]), key


def test_rows_golden(sess, g10):
    src = g10["rows_src"]
    rows = [int(r) for r in g10["gather_rows"]]
    y = call_out(sess, (len(rows), src.shape[1]), lambda d, o: _lib.check(
        sess.rows(d.up(src), src.shape[0], o, len(rows), src.shape[1], rows, 0), "gather"))
    assert same(y, g10["gather_y"])
    dst = g10["scatter_dst"]
    rows = [int(r) for r in g10["scatter_rows"]]
    y = inplace(sess, dst, lambda d, xp: _lib.check(sess.rows(d.up(src), src.shape[0], xp, dst.shape[0], dst.shape[1], rows, 1),
                                                    "scatter"))
    assert same(y, g10["scatter_y"])


def test_slices_and_upsample_golden(sess, g10):
    x = g10["slice_x"]
    for i, (r0, nr, f0, nc) in enumerate(g10["slice_cases"]):
        r0, nr, f0, nc = int(r0), int(nr), int(f0), int(nc)
        y = call_out(sess, (nr, nc), lambda d, o: _lib.check(sess.copy_rows(d.up(x), 10, 20, o, nr, nc, nr, r0, f0, 0), "copy rows"))
        assert same(y, g10[f"slice_y{i}"]), i
    xu = g10["up_x"]
    y = call_out(sess, (96, 8), lambda d, o: _lib.check(sess.layout(OP_UPSAMPLE, d.up(xu), 24, 8, o, 96, 8, 6), "upsample"))
    assert same(y, g10["up_y"])


def test_shortcut_golden(sess, g10):
    for i, (wd, ht, cin, ch, t, up, sp) in enumerate(g10["sc_cases"]):
        x, want = g10[f"sc_x{i}"], g10[f"sc_y{i}"]
        y = call_out(sess, want.shape, lambda d, o: _lib.check(
            sess.shortcut(d.up(x), int(wd), int(ht), int(cin), o, int(ch), int(t), int(up), int(sp)), "shortcut"))
        assert same(y, want), i


# ---- the oracle at the models' shapes ----

@pytest.mark.parametrize("rows,channels", [(4608, 3840), (77, 30), (1, 3072)])
def test_channel_ops_vs_oracle(sess, rows, channels):
    """z_modulate / z_residual / the affine and Euler steps: DiT activations
    (4608 tokens x 3840), a ragged shape (scalar path) and one row."""
    rng = np.random.default_rng(rows + channels)
    o = oracle()
    x = (rng.standard_normal((rows, channels)) * 3).astype(np.float32)
    other = rng.standard_normal((rows, channels)).astype(np.float32)
    mod = (rng.standard_normal(4 * channels) * 0.5).astype(np.float32)
    print(f"channel ops {rows}x{channels}", flush=True)
    part = 2
    p = mod[part * channels:(part + 1) * channels]
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.pointwise_ex(OP_MODULATE, xp, d.up(mod), None, rows, channels, part), "modulate"))
    assert same(y, channel_op(o, OP_MODULATE, x, p=p))
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.pointwise_ex(OP_RESIDUAL, xp, d.up(other), None, rows, channels), "residual"))
    assert same(y, channel_op(o, OP_RESIDUAL, x, other, None))
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.pointwise_ex(OP_RESIDUAL, xp, d.up(other), d.up(mod), rows, channels, part),
                                                  "gated residual"))
    assert tanh_close(y, channel_op(o, OP_RESIDUAL, x, other, p), other)
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.pointwise_ex(OP_AFFINE, xp, None, None, rows, channels, 0, 1.0 / 0.3611, 0.1159),
                                                  "affine"))
    assert same(y, channel_op(o, OP_AFFINE, x, scale=np.float32(1.0 / 0.3611), bias=np.float32(0.1159)))
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.pointwise_ex(OP_EULER, xp, d.up(other), None, rows, channels, 0, -0.0417),
                                                  "euler"))
    assert same(y, channel_op(o, OP_EULER, x, other, scale=np.float32(-0.0417)))


@pytest.mark.parametrize("rows,channels,target_begin", [(4096 + 300, 3072, 300), (50, 30, 0), (9, 64, 9)])
def test_qwen_modulate_vs_oracle(sess, rows, channels, target_begin):
    """qwen_image_modulate on the Qwen-Image joint stream (text prefix rows
    modulated by the second parameter row), both forms."""
    rng = np.random.default_rng(rows * 3 + channels)
    o = oracle()
    x = (rng.standard_normal((rows, channels)) * 2).astype(np.float32)
    res = rng.standard_normal((rows, channels)).astype(np.float32)
    params = (rng.standard_normal((2, 6 * channels)) * 0.4).astype(np.float32)
    print(f"qwen modulate {rows}x{channels} target_begin={target_begin}", flush=True)
    for part in (0, 4):
        y = inplace(sess, x, lambda d, xp: _lib.check(
            sess.qwen_modulate(xp, rows, channels, d.up(params), 6 * channels, target_begin, part), "qwen scale"))
        assert same(y, qwen_modulate(o, x, params, target_begin, part))
        y = inplace(sess, x, lambda d, xp: _lib.check(
            sess.qwen_modulate(xp, rows, channels, d.up(params), 6 * channels, target_begin, part, d.up(res)), "qwen residual"))
        assert tanh_close(y, qwen_modulate(o, x, params, target_begin, part, res), res)


@pytest.mark.parametrize("rows,channels,weighted,eps", [(128 * 128, 96, True, 1e-12), (4096, 384, False, 1e-12), (77, 30, True, 0.5),
                                                       (3, 1000, True, 1e-12), (300, 3072, True, 1e-12)])
def test_l2norm_vs_oracle(sess, rows, channels, weighted, eps):
    """The Qwen VAE's RMS norm (QWEN_VAE_L2_EPSILON 1e-12) over pixels; rows of
    up to 8 units per lane stay in registers, 3072 channels take the re-read."""
    rng = np.random.default_rng(rows + channels)
    x = (rng.standard_normal((rows, channels)) * rng.choice([1e-3, 1.0, 30.0], (rows, 1))).astype(np.float32)
    x[0] = 0.0
    w = (1.0 + 0.2 * rng.standard_normal(channels)).astype(np.float32) if weighted else None
    print(f"l2norm {rows}x{channels}", flush=True)
    y = call_out(sess, x.shape, lambda d, o: _lib.check(sess.l2norm(d.up(x), rows, channels, d.up(w) if w is not None else None, eps, o),
                                                        "l2norm"))
    assert same(y, l2norm(oracle(), "orc", x, w, eps))


@pytest.mark.parametrize("rows,channels", [(256 * 256, 512), (128 * 128, 128), (64 * 64, 256), (1000, 96), (50000, 32), (7, 8192), (3000, 384)])
def test_groupnorm_vs_oracle(sess, rows, channels):
    """The VAE's GroupNorm(32) over pixels, up to a 256x256 image of 512
    channels; group widths 1 and 3 take the scalar path."""
    rng = np.random.default_rng(rows + channels)
    x = (rng.standard_normal((rows, channels)) * rng.uniform(0.2, 3.0, channels) + rng.uniform(-4, 4, channels)).astype(np.float32)
    w = (1.0 + 0.3 * rng.standard_normal(channels)).astype(np.float32)
    b = (0.2 * rng.standard_normal(channels)).astype(np.float32)
    print(f"groupnorm {rows}x{channels}", flush=True)
    y = call_out(sess, x.shape, lambda d, o: _lib.check(sess.groupnorm(d.up(x), rows, channels, d.up(w), d.up(b), o), "groupnorm"))
    want = groupnorm(oracle(), "orc", x, w, b)
    diff = np.count_nonzero(bits(y) != bits(want))
    print(f"  {diff} of {y.size} values differ", flush=True)
    assert diff == 0


def test_groupnorm_in_place(sess):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 128)).astype(np.float32)
    w, b = np.ones(128, np.float32), np.zeros(128, np.float32)
    y = inplace(sess, x, lambda d, xp: _lib.check(sess.groupnorm(xp, 300, 128, d.up(w), d.up(b), xp), "groupnorm in place"))
    assert same(y, groupnorm(oracle(), "orc", x, w, b))


@pytest.mark.parametrize("wtype,inner,table_rows", [(Q8_0, 3584, 1000), (Q5_K, 2560, 300), (Q6_K, 3584, 200), (F16, 3584, 500),
                                                    (BF16, 1024, 100), (F32, 300, 50)])
@pytest.mark.parametrize("on_device", [False, True])
def test_embedding_vs_oracle(sess, wtype, inner, table_rows, on_device):
    """Token embedding rows of random tables (finite fp16 scales), 300 ids with
    repeats, from the host mapping and from a device-resident table."""
    rng = np.random.default_rng(wtype * 100 + inner)
    block, nbytes = ROW_BYTES[wtype]
    stride = inner // block * nbytes
    table = rng.integers(0, 256, (table_rows, stride), dtype=np.uint8)
    if wtype in (Q8_0, Q5_K, Q6_K):
        offs = {Q8_0: (0,), Q5_K: (0, 2), Q6_K: (208,)}[wtype]
        t = table.reshape(table_rows, -1, nbytes)
        for off in offs:
            t[..., off + 1] = (t[..., off + 1] & 0x83) | ((rng.integers(0, 30, t.shape[:2]).astype(np.uint8) << 2) & 0x7c)
    ids = rng.integers(0, table_rows, 300).tolist()
    print(f"embedding type {wtype} inner {inner}, device table {on_device}", flush=True)
    d = Dev(sess)
    try:
        tp = d.up(table) if on_device else table.ctypes.data
        out = d.out((len(ids), inner))
        _lib.check(sess.embedding(tp, wtype, inner, table_rows, ids, out), "embedding")
        y = d.get(out)
    finally:
        d.free()
    o = oracle()
    want = np.stack([decode_f32(o, "orc", table[i], wtype, inner) for i in ids])
    assert same(y, want)


def test_rows_at_model_shape(sess):
    """Qwen-Image's layout moves: gather text rows of the condition, scatter
    them and the image rows into the joint stream (4096 x 3072)."""
    rng = np.random.default_rng(77)
    o = oracle()
    src = rng.standard_normal((1500, 3072)).astype(np.float32)
    rows = rng.integers(0, 1500, 700).tolist()
    y = call_out(sess, (700, 3072), lambda d, op: _lib.check(sess.rows(d.up(src), 1500, op, 700, 3072, rows, 0), "gather"))
    assert same(y, gather(o, "orc", src, np.array(rows, np.uint64)))
    dst = rng.standard_normal((4096, 3072)).astype(np.float32)
    rows = rng.integers(0, 4096, 1500).tolist()  # with repeats: the last copy wins
    y = inplace(sess, dst, lambda d, xp: _lib.check(sess.rows(d.up(src), 1500, xp, 4096, 3072, rows, 1), "scatter"))
    assert same(y, scatter(o, "orc", dst, src, np.array(rows, np.uint64)))


def test_copies_at_model_shape(sess):
    """The DiT's q / k / v split of the fused projection (src/inference.cpp:
    304-306), the caption / image join (:406-407) and copy_features."""
    rng = np.random.default_rng(78)
    qkv = rng.standard_normal((4608, 3 * 3840)).astype(np.float32)
    for part in range(3):
        y = call_out(sess, (4608, 3840), lambda d, op: _lib.check(
            sess.copy_rows(d.up(qkv), 4608, 3 * 3840, op, 4608, 3840, 4608, 0, part * 3840, 0), "copy rows"))
        assert same(y, qkv[:, part * 3840:(part + 1) * 3840])
    cap = rng.standard_normal((512, 3840)).astype(np.float32)
    joint = np.zeros((4608, 3840), np.float32)
    y = inplace(sess, joint, lambda d, xp: _lib.check(sess.copy_rows(d.up(cap), 512, 3840, xp, 4608, 3840, 512, 0, 0, 4096),
                                                      "copy rows to an offset"))
    want = joint.copy()
    want[4096:] = cap
    assert same(y, want)
    odd = rng.standard_normal((1, 37)).astype(np.float32)
    row = np.zeros((1, 100), np.float32)
    y = inplace(sess, row, lambda d, xp: _lib.check(sess.copy_features(d.up(odd), 37, xp, 100, 61), "copy features"))
    want = row.copy()
    want[0, 61:98] = odd[0]
    assert same(y, want)


def test_outputs_past_the_cache(sess):
    """The non-temporal store forms, taken when an output exceeds 256 MB: l2norm
    [1M, 96] (Qwen VAE), groupnorm [1M, 128] and the 2x upsample of 512 x 512 x
    128, each against the oracle, bit-exact."""
    rng = np.random.default_rng(97)
    o = oracle()
    rows = 1 << 20
    x = rng.standard_normal((rows, 96), dtype=np.float32)
    w = (1.0 + 0.2 * rng.standard_normal(96)).astype(np.float32)
    print("l2norm [1M, 96]", flush=True)
    y = call_out(sess, x.shape, lambda d, op: _lib.check(sess.l2norm(d.up(x), rows, 96, d.up(w), 1e-12, op), "l2norm"))
    assert same(y, l2norm(o, "orc", x, w, 1e-12))
    del x, y
    x = (rng.standard_normal((rows, 128), dtype=np.float32) * 1.5 + 0.25).astype(np.float32)
    w = (1.0 + 0.3 * rng.standard_normal(128)).astype(np.float32)
    b = (0.2 * rng.standard_normal(128)).astype(np.float32)
    print("groupnorm [1M, 128]", flush=True)
    y = call_out(sess, x.shape, lambda d, op: _lib.check(sess.groupnorm(d.up(x), rows, 128, d.up(w), d.up(b), op), "groupnorm"))
    assert same(y, groupnorm(o, "orc", x, w, b))
    del x, y
    img = rng.standard_normal((512 * 512, 128), dtype=np.float32)
    print("upsample [512x512, 128]", flush=True)
    y = call_out(sess, (4 * 512 * 512, 128), lambda d, op: _lib.check(sess.layout(OP_UPSAMPLE, d.up(img), 512 * 512, 128, op, 4 * 512 * 512,
                                                                                  128, 512), "upsample"))
    assert same(y, layout(o, OP_UPSAMPLE, img, 512, 512, 128))


def test_layouts_at_model_shape(sess):
    """Z-Image DiT patchify of 128 x 128 latents of 16 channels (patch 2: 4096
    tokens of 64), unpatchify back, and the VAE's 2x upsample of 256 x 256 x 128."""
    rng = np.random.default_rng(79)
    o = oracle()
    lat = rng.standard_normal((128 * 128, 16)).astype(np.float32)
    tok = call_out(sess, (4096, 64), lambda d, op: _lib.check(sess.layout(OP_PATCH, d.up(lat), 16384, 16, op, 4096, 64, 128, 2), "patch"))
    assert same(tok, layout(o, OP_PATCH, lat, 128, 128, 16, 2))
    back = call_out(sess, (16384, 16), lambda d, op: _lib.check(sess.layout(OP_UNPATCH, d.up(tok), 4096, 64, op, 16384, 16, 128, 2),
                                                                "unpatch"))
    assert same(back, lat)
    img = rng.standard_normal((256 * 256, 128)).astype(np.float32)
    y = call_out(sess, (4 * 65536, 128), lambda d, op: _lib.check(sess.layout(OP_UPSAMPLE, d.up(img), 65536, 128, op, 4 * 65536, 128, 256),
                                                                  "upsample"))
    assert same(y, layout(o, OP_UPSAMPLE, img, 256, 256, 128))
    odd = rng.standard_normal((6 * 4, 3)).astype(np.float32)  # 3 channels: scalar path, patch 2
    tok = call_out(sess, (6, 12), lambda d, op: _lib.check(sess.layout(OP_PATCH, d.up(odd), 24, 3, op, 6, 12, 6, 2), "patch (scalar)"))
    assert same(tok, layout(o, OP_PATCH, odd, 6, 4, 3, 2))


@pytest.mark.parametrize("wd,ht,cin,ch,t,up,sp", [(64, 64, 96, 192, 2, 0, 1), (32, 32, 384, 384, 2, 1, 1), (48, 40, 192, 96, 1, 0, 1),
                                                  (24, 24, 384, 192, 2, 1, 1), (16, 16, 96, 96, 2, 1, 0)])
def test_shortcut_vs_oracle(sess, wd, ht, cin, ch, t, up, sp):
    """The Qwen VAE's resampling shortcuts (src/qwen_vae.cpp:117, :159)."""
    rng = np.random.default_rng(wd * ht + cin)
    x = rng.standard_normal((wd * ht, cin)).astype(np.float32)
    want = shortcut(oracle(), "orc", x, wd, ht, ch, t, up, sp)
    assert want is not None
    print(f"shortcut {wd}x{ht} {cin}->{ch} t={t} up={up} spatial={sp}", flush=True)
    y = call_out(sess, want.shape, lambda d, op: _lib.check(sess.shortcut(d.up(x), wd, ht, cin, op, ch, t, up, sp), "shortcut"))
    assert same(y, want)


def test_errors(sess):
    arg, uns = _lib.ERR_ARGUMENT, _lib.ERR_UNSUPPORTED
    d = Dev(sess)
    try:
        x = d.up(np.zeros((8, 64), np.float32))
        o = d.out((32, 64))
        assert sess.pointwise_ex(OP_MODULATE, x, None, None, 8, 64) == arg                       # no modulation
        assert sess.pointwise_ex(99, x, None, None, 8, 64) == uns
        assert sess.qwen_modulate(x, 8, 64, x, 64, 0, 1) == arg                                  # (part+1)*channels > 64
        assert sess.l2norm(x, 8, 64, None, 0.0, o) == arg                                        # epsilon <= 0
        assert sess.groupnorm(x, 8, 48, x, x, o) == arg                                          # 48 not of 32 groups
        assert sess.groupnorm(x, 1, 32 * 300, x, x, o) == uns                                    # groups wider than 256
        table = np.zeros((4, 34), np.uint8)
        assert sess.embedding(table.ctypes.data, Q8_0, 32, 4, [4], o) == arg                     # id out of range
        assert sess.embedding(table.ctypes.data, Q8_0, 33, 4, [0], o) == arg                     # ragged block
        assert sess.embedding(table.ctypes.data, 2, 32, 4, [0], o) == uns                        # Q4_0 not decoded
        assert sess.rows(x, 8, o, 3, 64, [1, 8, 2], 0) == arg                                    # row 8 of 8
        assert sess.rows(x, 8, o, 2, 64, [1, 2, 3], 0) == arg                                    # destination rows != count
        assert sess.rows(x, 8, o, 32, 64, [], 1) == arg                                          # empty list
        assert sess.copy_rows(x, 8, 64, o, 32, 64, 9, 0, 0, 0) == arg                            # past the source
        assert sess.copy_rows(x, 8, 64, o, 32, 32, 8, 0, 40, 0) == arg                           # features past the row
        assert sess.copy_features(x, 64, o, 64, 1) == arg
        assert sess.layout(OP_PATCH, x, 8, 64, o, 2, 256, 3, 2) == arg                           # width 3 not of patch 2
        assert sess.layout(OP_UPSAMPLE, x, 8, 64, o, 31, 64, 4) == arg                           # 4 * 8 rows expected
        assert sess.layout(7, x, 8, 64, o, 32, 64, 4) == uns
        assert sess.shortcut(x, 3, 2, 64, o, 64, 1, 0, 1) == arg                                 # odd width going down
        assert sess.shortcut(x, 4, 2, 64, o, 24, 1, 1, 1) == arg                                 # 24 * 4 not of 64
    finally:
        d.free()
