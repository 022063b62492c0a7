"""pixhip_conv2d (tensor_conv, src/convolution.cpp:34-100) through the C ABI:
the reference's own outputs (tests/golden/g11_conv, written by the compiled
src/convolution.cpp: both forms, 3x3 / 1x1 / 3x1 kernels, stride 2 with
one-sided padding, 3 to 32 input channels, F32 / F16 / BF16 weights), the
oracle (oracle/pix_oracle.c orc_conv2d, within 1e-5 of the reference) at VAE
layer shapes, and at the full 256 x 256 x 512 -> 512 shape a sampled band of
rows plus translation equivariance (an image shifted by one pixel gives the
shifted output, bit for bit, away from the border).

The kernel multiplies split-bf16 operands on MFMA with fp32 accumulation, so
outputs are held to TOL = 1e-4 of each output row's largest magnitude."""
import ctypes
import os

import numpy as np
import pytest

import model_files as mf
from gpu_helpers import TOL, Pinned, new_session, row_rel_error
from oracle_lib import conv2d, conv_out_size, oracle, same_geometry
from pixelina_amd import _lib

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32, F16, BF16 = 0, 1, 30


@pytest.fixture(scope="module")
def sess():
    s = new_session()
    yield s
    s.close()


def weight_bytes(w, wtype):
    """fp32 [cout][inner] -> (file bytes of `wtype`, the fp32 values they hold)."""
    if wtype == F16:
        h = w.astype(np.float16)
        return h.view(np.uint8), h.astype(np.float32)
    if wtype == BF16:
        b = (w.view(np.uint32) >> 16).astype(np.uint16)
        return b.view(np.uint8), (b.astype(np.uint32) << 16).view(np.float32)
    return w.view(np.uint8), w


def gpu_conv(sess, key, x, width, height, raw, wtype, kx, ky, cin, cout, bias=None, geometry=None):
    h = sess.conv_weight(key, raw, wtype, kx, ky, cin, cout)
    ow, oh = conv_out_size(width, height, kx, ky, geometry or same_geometry(kx, ky))
    xb = sess.to_device(np.ascontiguousarray(x, np.float32))
    bb = sess.to_device(np.ascontiguousarray(bias, np.float32)) if bias is not None else None
    yb = sess.alloc(ow * oh * cout * 4)
    try:
        _lib.check(sess.conv2d(h, xb.ptr, width, height, yb.ptr, geometry, bb.ptr if bb else None), "pixhip_conv2d")
        return yb.download(np.float32, ow * oh * cout).reshape(ow * oh, cout)
    finally:
        for b in (xb, bb, yb):
            if b is not None:
                b.free()


def test_reference_vectors(sess):
    g = np.load(os.path.join(GOLDEN, "g11_conv.npz"))
    for c in range(int(g["count"])):
        wd, ht, cin, cout, kx, ky, wtype, has_bias = (int(v) for v in g[f"c{c}_shape"])
        geom = tuple(int(v) for v in g[f"c{c}_geometry"]) or None
        print(f"case {c}: {wd}x{ht} {cin}->{cout} {kx}x{ky} type {wtype} geometry {geom}", flush=True)
        y = gpu_conv(sess, f"g11:{c}", g[f"c{c}_x"], wd, ht, g[f"c{c}_w"], wtype, kx, ky, cin, cout,
                     g[f"c{c}_b"] if has_bias else None, geom)
        err = row_rel_error(y, g[f"c{c}_y"]).max()
        print(f"  rel={err:.2e}", flush=True)
        assert err <= TOL, c


@pytest.mark.parametrize("wd,ht,cin,cout,k,wtype,geom,bias", [
    (64, 48, 256, 128, 3, F16, None, True),             # a VAE 3x3, 32-channel stages
    (33, 17, 128, 64, 1, BF16, None, False),            # 1x1 shortcut, ragged pixel and channel tiles
    (40, 30, 512, 256, 3, F32, (2, 2, 0, 1, 0, 1), True),  # the encoder's stride-2 downsample
    (64, 64, 16, 512, 3, F16, None, True),              # conv_in from 16 latent channels (gathered)
    (20, 15, 3, 128, 3, F32, None, True),               # RGB input
    (19, 13, 32, 160, 1, F16, None, True),              # one 32-value stage (the pipelined kernel's tail alone)
    (17, 11, 64, 96, 1, BF16, None, False),             # two stages
    (23, 9, 96, 128, 1, F32, None, True),               # three stages
])
def test_against_oracle(sess, wd, ht, cin, cout, k, wtype, geom, bias):
    rng = np.random.default_rng(wd * cin + cout)
    x = rng.standard_normal((wd * ht, cin)).astype(np.float32)
    w = (rng.standard_normal((cout, cin * k * k)) / np.sqrt(cin * k * k)).astype(np.float32)
    raw, wv = weight_bytes(w, wtype)
    b = rng.standard_normal(cout).astype(np.float32) if bias else None
    print(f"{wd}x{ht} {cin}->{cout} {k}x{k} type {wtype} geometry {geom}", flush=True)
    y = gpu_conv(sess, f"conv:{wd}:{cin}:{cout}:{wtype}", x, wd, ht, raw, wtype, k, k, cin, cout, b, geom)
    ref = conv2d(oracle(), x, wd, ht, wv, k, k, b, geom)
    err = row_rel_error(y, ref).max()
    print(f"  rel={err:.2e}", flush=True)
    assert err <= TOL


def test_vae_shape_band_and_translation(sess):
    """256 x 256 pixels, 512 -> 512 channels, 3x3 (a VAE decoder block's
    conv): output rows 0-1 and 127-128 against the oracle run on the input
    rows they read; then the image shifted right by one pixel."""
    rng = np.random.default_rng(256)
    wd = ht = 256
    cin = cout = 512
    x = rng.standard_normal((ht * wd, cin)).astype(np.float32)
    w = (rng.standard_normal((cout, cin * 9)) / np.sqrt(cin * 9)).astype(np.float32)
    raw, wv = weight_bytes(w, F16)
    b = rng.standard_normal(cout).astype(np.float32)
    y = gpu_conv(sess, "vae:256", x, wd, ht, raw, F16, 3, 3, cin, cout, b)
    img = x.reshape(ht, wd, cin)
    o = oracle()
    for y0, rows, top in ((0, slice(0, 3), 1), (127, slice(126, 130), 0)):
        band = np.ascontiguousarray(img[rows]).reshape(-1, cin)
        want = conv2d(o, band, wd, rows.stop - rows.start, wv, 3, 3, b, (1, 1, 1, 1, top, 0))
        got = y.reshape(ht, wd, cout)[y0:y0 + 2].reshape(-1, cout)
        err = row_rel_error(got, want).max()
        print(f"rows {y0}-{y0 + 1}: rel={err:.2e}", flush=True)
        assert err <= TOL
    shifted = np.zeros_like(img)
    shifted[:, 1:] = img[:, :-1]
    y2 = gpu_conv(sess, "vae:256", shifted.reshape(-1, cin), wd, ht, raw, F16, 3, 3, cin, cout, b).reshape(ht, wd, cout)
    y1 = y.reshape(ht, wd, cout)
    # columns whose taps lie inside both images: shifted column c + 1 is column c
    assert np.array_equal(y2[:, 2:-1].view(np.uint32), y1[:, 1:-2].view(np.uint32)), "not translation-equivariant"


def test_wide_image(sess):
    """An input of exactly 2 GiB (2048 rows x 1024 pixels x 256 channels),
    which takes the 64-bit-address image kernel: a random pattern whose period
    (1,000,003 values) is not a multiple of a row, uploaded once and repeated
    by device copies; output rows 0-1 and the last two against the oracle run
    on the input rows they read (the last ones lie past 2^31 bytes)."""
    wd, ht, cin, cout = 1024, 2048, 256, 64
    n = wd * ht * cin
    assert n * 4 == 1 << 31
    rng = np.random.default_rng(2048)
    period = 1_000_003
    base = rng.standard_normal(period).astype(np.float32)
    pattern = lambda lo, hi: base[np.arange(lo, hi, dtype=np.int64) % period]
    w = (rng.standard_normal((cout, cin * 9)) / np.sqrt(cin * 9)).astype(np.float32)
    raw, wv = weight_bytes(w, F16)
    b = rng.standard_normal(cout).astype(np.float32)
    h = sess.conv_weight("wide", raw, F16, 3, 3, cin, cout)
    xb = sess.alloc(n * 4)
    yb = sess.alloc(wd * ht * cout * 4)
    bb = sess.to_device(b)
    try:
        xb.upload(base)
        for lo in range(period, n, period):
            sess.copy_device(xb.ptr + lo * 4, xb.ptr, min(period, n - lo) * 4)
        print("2 GiB input in place", flush=True)
        _lib.check(sess.conv2d(h, xb.ptr, wd, ht, yb.ptr, None, bb.ptr), "pixhip_conv2d")
        o = oracle()
        row = wd * cin
        for y0, r0, r1, geom in ((0, 0, 3, (1, 1, 1, 1, 1, 0)), (ht - 2, ht - 3, ht, (1, 1, 1, 1, 0, 1))):
            band = pattern(r0 * row, r1 * row).reshape(-1, cin)
            want = conv2d(o, band, wd, r1 - r0, wv, 3, 3, b, geom)
            got = yb.download(np.float32, 2 * wd * cout, y0 * wd * cout * 4).reshape(-1, cout)
            err = row_rel_error(got, want).max()
            print(f"rows {y0}-{y0 + 1}: rel={err:.2e}", flush=True)
            assert err <= TOL
    finally:
        sess.synchronize()
        for buf in (xb, yb, bb):
            buf.free()


def test_weight_from_model_file(sess, tmp_path):
    """A rank-5 [3, 3, 1, cin, cout] F16 tensor (the Qwen VAE's causal 3-D
    conv with one time step) through pixhip_model_conv_weight."""
    rng = np.random.default_rng(5)
    cin, cout, wd, ht = 96, 96, 24, 20
    w = (rng.standard_normal((cout, cin * 9)) / np.sqrt(cin * 9)).astype(np.float32)
    raw, wv = weight_bytes(w, F16)
    path = tmp_path / "vae.gguf"
    path.write_bytes(mf.gguf([], [("decoder.conv_in.weight", F16, [3, 3, 1, cin, cout], raw.tobytes())]))
    model, h = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.check(sess.lib.pixhip_model_open(str(path).encode(), 0, ctypes.byref(model)), "open")
    try:
        _lib.check(sess.lib.pixhip_model_conv_weight(sess.handle, model, b"decoder.conv_in.weight", ctypes.byref(h)), "conv weight")
        x = rng.standard_normal((wd * ht, cin)).astype(np.float32)
        xb, yb = sess.to_device(x), sess.alloc(wd * ht * cout * 4)
        _lib.check(sess.conv2d(h.value, xb.ptr, wd, ht, yb.ptr), "conv2d")
        y = yb.download(np.float32, wd * ht * cout).reshape(-1, cout)
        xb.free()
        yb.free()
        err = row_rel_error(y, conv2d(oracle(), x, wd, ht, wv, 3, 3)).max()
        print(f"rel={err:.2e}", flush=True)
        assert err <= TOL
    finally:
        sess.synchronize()
        sess.lib.pixhip_model_close(model)


def test_weights_beyond_bf16_range(sess):
    """F32 weights of +-3.4e38 (finite, past the largest bf16: a rounded split
    would give hi = Inf, lo = NaN) against image values small enough for
    finite products: the weight split keeps hi finite, no NaN, within TOL."""
    rng = np.random.default_rng(5)
    wd, ht, cin, cout, k = 16, 12, 64, 64, 3
    x = (rng.standard_normal((wd * ht, cin)) * 1e-30).astype(np.float32)
    w = (rng.standard_normal((cout, cin * k * k)) / np.sqrt(cin * k * k)).astype(np.float32)
    w[3, 10] = np.float32(3.4e38)
    w[40, 500] = np.float32(-3.4e38)
    y = gpu_conv(sess, "conv:huge", x, wd, ht, w.view(np.uint8), F32, k, k, cin, cout)
    ref = conv2d(oracle(), x, wd, ht, w, k, k, None, None)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    err = row_rel_error(y, ref).max()
    print(f"rel={err:.2e}", flush=True)
    assert err <= TOL


def test_output_past_its_allocation():
    """An output (or input) that runs past the end of its device allocation is
    rejected before any launch (a fresh session, so every block is exactly its
    request rounded to 256 bytes)."""
    s = new_session()
    try:
        raw = np.zeros(4 * 8 * 9 * 2, np.uint8)
        w = s.conv_weight("span", raw, F16, 3, 3, 8, 4)
        x, y = s.alloc(16 * 8 * 4), s.alloc(16 * 4 * 4)      # 512 and 256 bytes
        assert s.conv2d(w, x.ptr, 4, 4, y.ptr) == _lib.OK
        s.synchronize()
        assert s.conv2d(w, x.ptr, 4, 4, y.ptr + 4) == _lib.ERR_ARGUMENT      # output one float past the end
        assert s.conv2d(w, x.ptr + 16, 4, 4, y.ptr) == _lib.ERR_ARGUMENT     # input four floats past the end
        x.free()
        y.free()
    finally:
        s.close()


def test_pinned_host_operands(sess):
    """Input, bias and output in pinned host memory: the input is copied to the
    device once (the kernel reads each pixel once per tap) and the output is
    written in place; the result is bit-identical to the device-resident call."""
    rng = np.random.default_rng(31)
    wd, ht, cin, cout = 40, 24, 64, 96
    w = (rng.standard_normal((cout, cin * 9)) / 24).astype(np.float32)
    raw, _ = weight_bytes(w, F16)
    x = rng.standard_normal((wd * ht, cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    ref = gpu_conv(sess, "test:pinned", x, wd, ht, raw, F16, 3, 3, cin, cout, bias=b)
    h = sess.conv_weight("test:pinned", raw, F16, 3, 3, cin, cout)
    hx, hb, hy = Pinned(sess, x), Pinned(sess, b), Pinned(sess, np.zeros((wd * ht, cout), np.float32))
    try:
        _lib.check(sess.conv2d(h, hx.p.value, wd, ht, hy.p.value, None, hb.p.value), "pixhip_conv2d (pinned)")
        sess.synchronize()
        y = hy.read(np.float32, (wd * ht, cout))
    finally:
        for p in (hx, hb, hy):
            p.free()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_errors(sess):
    arg, uns = _lib.ERR_ARGUMENT, _lib.ERR_UNSUPPORTED
    raw = np.zeros(4 * 8 * 9 * 2, np.uint8)
    h = ctypes.c_void_p()
    assert sess.lib.pixhip_conv_weight_get(sess.handle, b"q", raw.ctypes.data, raw.nbytes, 8, 3, 3, 8, 4, ctypes.byref(h)) == uns
    assert sess.lib.pixhip_conv_weight_get(sess.handle, b"s", raw.ctypes.data, 10, F16, 3, 3, 8, 4, ctypes.byref(h)) == arg
    w = sess.conv_weight("err", raw, F16, 3, 3, 8, 4)
    x, y = sess.alloc(16 * 8 * 4), sess.alloc(64 * 4 * 4)
    assert sess.conv2d(w, x.ptr, 4, 4, y.ptr, (0, 1, 1, 1, 1, 1)) == arg         # stride 0
    assert sess.conv2d(w, x.ptr, 1, 1, y.ptr, (1, 1, 0, 0, 0, 0)) == arg         # padded image smaller than the kernel
    assert sess.conv2d(w, x.ptr, 1 << 16, 1 << 16, y.ptr) == arg                  # 2^32 pixels (indices are 32-bit)
    assert sess.matmul(w, x.ptr, 2, y.ptr) == uns                                # not a linear weight
    x.free()
    y.free()
