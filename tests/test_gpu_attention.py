"""pixhip_attention / pixhip_attention_ranges (tensor_attention,
src/tensor.cpp:347-427) through the C ABI, against the reference's own outputs
(tests/golden/g9_attention, written by the compiled src/tensor.cpp) and the
oracle (oracle/pix_oracle.c orc_attention, bit-exact with the reference).

The kernel computes the two products with three bf16 MFMA terms per fp32
product and an online fp32 softmax, so results are held to TOL = 1e-4 of each
output row's largest magnitude (max |y - r| / max |r| per row).  At the DiT
shape (30 heads of 128, 4608 tokens) the oracle runs on a sample of query rows
(non-causal rows are independent of each other), and so at the VAE mid-block
shapes (one head of 512 over 16384 tokens, one of 384 over 4096: the wide-head
kernel, head sizes 129..512).  Size-independent properties
at full size: V of ones gives ones, a key permutation leaves non-causal
outputs unchanged, and repeats are bit-identical.
"""
import os

import numpy as np
import pytest

from gpu_helpers import TOL, Pinned, row_rel_error
from oracle_lib import attention, oracle
from pixelina_amd import _lib

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def gpu_attention(sess, q, k, v, heads, kv_heads, causal=False, ranges=None, query_offset=0):
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    rows, channels = q.shape
    keys = k.shape[0]
    qb, kb, vb = sess.to_device(q), sess.to_device(k), sess.to_device(v)
    ob = sess.alloc(rows * channels * 4)
    rc = sess.attention(qb.ptr, rows, kb.ptr, vb.ptr, keys, heads, kv_heads, channels, ob.ptr, causal, ranges, query_offset)
    _lib.check(rc, "attention")
    y = ob.download(np.float32, rows * channels).reshape(rows, channels)
    for b in (qb, kb, vb, ob):
        b.free()
    return y


def qkv(rng, rows, keys, heads, kv_heads, dim, qscale=1.5):
    q = (rng.standard_normal((rows, heads * dim)) * qscale).astype(np.float32)
    k = (rng.standard_normal((keys, kv_heads * dim)) * qscale).astype(np.float32)
    v = rng.standard_normal((keys, kv_heads * dim)).astype(np.float32)
    return q, k, v


def test_reference_vectors(sess):
    g = np.load(os.path.join(GOLDEN, "g9_attention.npz"))
    for c in range(int(g["count"])):
        rows, keys, heads, kvh, dim, causal, offset = (int(v) for v in g[f"c{c}_shape"])
        ranges = [tuple(int(x) for x in r) for r in g[f"c{c}_ranges"]] or None
        print(f"case {c}: rows={rows} keys={keys} heads={heads}/{kvh} dim={dim} causal={causal} ranges={ranges}", flush=True)
        y = gpu_attention(sess, g[f"c{c}_q"], g[f"c{c}_k"], g[f"c{c}_v"], heads, kvh, bool(causal), ranges, offset)
        err = row_rel_error(y, g[f"c{c}_y"]).max()
        print(f"  rel={err:.2e}", flush=True)
        assert err <= TOL, (c, err)


@pytest.mark.parametrize("rows,keys,heads,kvh,dim,causal", [
    (300, 300, 32, 8, 128, True),     # Qwen LM block: grouped heads, causal
    (700, 700, 16, 16, 72, False),    # Qwen vision: head size 72
    (257, 513, 4, 2, 64, False),      # ragged tiles, head size 64
    (1, 77, 8, 8, 128, False),        # one query row
    (65, 65, 2, 1, 40, True),         # head size 40 (zero-padded to 64)
    (90, 90, 3, 3, 30, False),        # head size 30: rows not 16-byte aligned, scalar stores
])
def test_against_oracle(sess, rows, keys, heads, kvh, dim, causal):
    rng = np.random.default_rng(rows * 7 + dim)
    q, k, v = qkv(rng, rows, keys, heads, kvh, dim)
    print(f"rows={rows} keys={keys} heads={heads}/{kvh} dim={dim} causal={causal}", flush=True)
    y = gpu_attention(sess, q, k, v, heads, kvh, causal)
    ref = attention(oracle(), "orc", q, k, v, heads, kvh, causal=causal)
    err = row_rel_error(y, ref).max()
    print(f"  rel={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("rows,keys,heads,kvh,dim,causal", [
    (300, 300, 2, 1, 512, True),      # head size 512, grouped, causal
    (130, 257, 3, 3, 384, False),     # head size 384, ragged key tile
    (97, 97, 4, 2, 256, True),        # head size 256
    (64, 200, 2, 2, 129, False),      # head size 129: padded to 256, scalar stores
    (33, 40, 1, 1, 508, False),       # head size 508: rows not of 8 values
    (1, 65, 1, 1, 320, False),        # one query row
])
def test_wide_heads_against_oracle(sess, rows, keys, heads, kvh, dim, causal):
    rng = np.random.default_rng(rows * 13 + dim)
    q, k, v = qkv(rng, rows, keys, heads, kvh, dim, qscale=0.6)
    print(f"rows={rows} keys={keys} heads={heads}/{kvh} dim={dim} causal={causal}", flush=True)
    y = gpu_attention(sess, q, k, v, heads, kvh, causal)
    ref = attention(oracle(), "orc", q, k, v, heads, kvh, causal=causal)
    err = row_rel_error(y, ref).max()
    print(f"  rel={err:.2e}", flush=True)
    assert err <= TOL


def test_wide_head_ranges(sess):
    """Head size 384 under the ranges form: a causal prefix, full rows and a
    key-limited block, with a query offset."""
    rng = np.random.default_rng(384)
    rows, keys, heads, dim, offset = 200, 260, 2, 384, 40
    q, k, v = qkv(rng, rows, keys, heads, heads, dim, qscale=0.6)
    ranges = [(0, 50, 260, 1), (50, 150, 260, 0), (150, 200, 77, 0)]
    y = gpu_attention(sess, q, k, v, heads, heads, ranges=ranges, query_offset=offset)
    ref = attention(oracle(), "orc", q, k, v, heads, heads, ranges, offset)
    err = row_rel_error(y, ref).max()
    print(f"rel={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("tokens,dim", [(16384, 512), (4096, 384)])
def test_vae_mid_block_sampled(sess, tokens, dim):
    """The VAE mid-block attention: one head of 512 channels over the 128 x 128
    latent (Z-Image, src/inference.cpp:485) and one of 384 (Qwen-Image,
    src/qwen_vae.cpp:97, here at 64 x 64); inputs of a GroupNorm'd scale.  The
    oracle on 32 query rows spread over the image; V of ones gives ones and a
    repeat is bit-identical at full size."""
    rng = np.random.default_rng(tokens + dim)
    q, k, v = qkv(rng, tokens, tokens, 1, 1, dim, qscale=0.6)
    print(f"tokens={tokens} dim={dim}", flush=True)
    y = gpu_attention(sess, q, k, v, 1, 1)
    pick = np.linspace(0, tokens - 1, 32).astype(int)
    ref = attention(oracle(), "orc", q[pick], k, v, 1, 1)
    err = row_rel_error(y[pick], ref).max()
    print(f"  sampled rel={err:.2e}", flush=True)
    assert err <= TOL
    y2 = gpu_attention(sess, q, k, v, 1, 1)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "repeats differ"
    ones = gpu_attention(sess, q, k, np.ones_like(v), 1, 1)
    assert np.abs(ones - 1.0).max() <= 1e-5


def test_ranges_with_query_offset(sess):
    """The Qwen-Image layout: a causal text prefix, then image rows seeing every
    key, then rows limited to a key prefix, with a query offset (KV cache)."""
    rng = np.random.default_rng(41)
    rows, keys, heads, dim, offset = 600, 700, 4, 128, 100
    q, k, v = qkv(rng, rows, keys, heads, heads, dim)
    ranges = [(0, 90, 700, 1), (90, 400, 700, 0), (400, 600, 333, 0)]
    y = gpu_attention(sess, q, k, v, heads, heads, ranges=ranges, query_offset=offset)
    ref = attention(oracle(), "orc", q, k, v, heads, heads, ranges, offset)
    err = row_rel_error(y, ref).max()
    print(f"rel={err:.2e}", flush=True)
    assert err <= TOL


def test_dit_shape_sampled(sess):
    """Z-Image DiT self-attention: 30 heads of 128, 4608 tokens, not causal;
    the oracle on 48 query rows spread over the sequence."""
    rng = np.random.default_rng(4608)
    rows, heads, dim = 4608, 30, 128
    q, k, v = qkv(rng, rows, rows, heads, heads, dim)
    y = gpu_attention(sess, q, k, v, heads, heads)
    pick = np.linspace(0, rows - 1, 48).astype(int)
    ref = attention(oracle(), "orc", q[pick], k, v, heads, heads)
    err = row_rel_error(y[pick], ref).max()
    print(f"sampled rel={err:.2e}", flush=True)
    assert err <= TOL


def test_properties_at_full_size(sess):
    rng = np.random.default_rng(9)
    rows, heads, dim = 4608, 30, 128
    q, k, _ = qkv(rng, rows, rows, heads, heads, dim)
    ones = np.ones((rows, heads * dim), np.float32)
    y = gpu_attention(sess, q, k, ones, heads, heads)
    assert np.abs(y - 1.0).max() <= 1e-5
    v = rng.standard_normal((rows, heads * dim)).astype(np.float32)
    y1 = gpu_attention(sess, q, k, v, heads, heads)
    perm = rng.permutation(rows)
    y2 = gpu_attention(sess, q, k[perm], v[perm], heads, heads)
    assert row_rel_error(y2, y1).max() <= TOL
    y3 = gpu_attention(sess, q, k, v, heads, heads)
    assert np.array_equal(y1.view(np.uint32), y3.view(np.uint32)), "repeats differ"


def test_large_magnitudes(sess):
    """V entries of +-1e30 among values of order 1 (within the kernel's range:
    the unnormalised output sums up to 2^8 * keys * max|v|, which must stay
    finite), against the oracle, with no NaN or Inf."""
    rng = np.random.default_rng(77)
    rows, keys, heads, dim = 64, 96, 2, 64
    q, k, v = qkv(rng, rows, keys, heads, heads, dim)
    v[5, 3] = np.float32(1e30)
    v[40, dim + 7] = np.float32(-1e30)
    y = gpu_attention(sess, q, k, v, heads, heads)
    ref = attention(oracle(), "orc", q, k, v, heads, heads)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    err = row_rel_error(y, ref).max()
    print(f"rel={err:.2e}", flush=True)
    assert err <= TOL


def test_pinned_host_operands(sess):
    """q, k, v and the output in pinned host memory (read and written in place
    over the bus): bit-identical to the device-resident call."""
    rng = np.random.default_rng(17)
    rows, keys, heads, kvh, dim = 130, 150, 4, 2, 64
    q, k, v = qkv(rng, rows, keys, heads, kvh, dim)
    ref = gpu_attention(sess, q, k, v, heads, kvh)
    hq, hk, hv, ho = Pinned(sess, q), Pinned(sess, k), Pinned(sess, v), Pinned(sess, np.zeros_like(q))
    try:
        _lib.check(sess.attention(hq.p.value, rows, hk.p.value, hv.p.value, keys, heads, kvh, heads * dim, ho.p.value),
                   "attention (pinned)")
        sess.synchronize()
        y = ho.read(np.float32, q.shape)
    finally:
        for p in (hq, hk, hv, ho):
            p.free()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_errors(sess):
    rng = np.random.default_rng(1)
    q, k, v = qkv(rng, 8, 8, 2, 2, 64)
    qb, kb, vb, ob = sess.to_device(q), sess.to_device(k), sess.to_device(v), sess.alloc(q.nbytes)
    arg = _lib.ERR_ARGUMENT
    assert sess.attention(qb.ptr, 8, kb.ptr, vb.ptr, 8, 3, 1, 128, ob.ptr) == arg          # channels not of heads
    assert sess.attention(qb.ptr, 8, kb.ptr, vb.ptr, 8, 2, 3, 128, ob.ptr) == arg          # heads not of kv_heads
    assert sess.attention(qb.ptr, 8, kb.ptr, vb.ptr, 7, 2, 2, 128, ob.ptr, True) == arg    # causal, rows > keys
    assert sess.attention(qb.ptr, 8, kb.ptr, vb.ptr, 8, 1, 1, 128 * 5, ob.ptr) == _lib.ERR_UNSUPPORTED  # head size 640
    for bad in ([(0, 3, 8, 0)], [(1, 8, 8, 0)], [(0, 8, 0, 0)], [(0, 8, 9, 0)], [(0, 4, 8, 0), (5, 8, 8, 0)]):
        assert sess.attention(qb.ptr, 8, kb.ptr, vb.ptr, 8, 2, 2, 128, ob.ptr, ranges=bad) == arg, bad
    for b in (qb, kb, vb, ob):
        b.free()
