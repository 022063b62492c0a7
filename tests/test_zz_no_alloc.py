"""pixhip_matmul_ex_noalloc, the allocation-free variant of pixhip_matmul_ex
(its quantized activations live in a fixed per-device array), against
pixhip_matmul_ex through the C ABI:

- two calls in a row per weight type, the second with fewer tokens, so the
  second reads an array that still holds the first call's larger activations:
  bit-identical where pixhip_matmul_ex runs its GEMM unsplit, within the fp32
  rounding of the split-K sums (max |y - r| / max |r| <= 1e-6 per token row)
  where it splits, and both within the parity tolerance of the oracle;
- the matvec (one token) bit-identical, with a bias and a strided output;
- the errors: a layout that is not resident (PIXHIP_ERR_STATE), activations
  beyond the array (PIXHIP_ERR_MEMORY), host memory (PIXHIP_ERR_ARGUMENT).
"""
import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import Q5_K, Q6_K, Q8_0, oracle, quant_matmul, quantize
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu

SPLIT_TOL = 1e-6


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def pack(wtype, wf):
    if wtype == Q5_K:
        return synth.pack_q5_K(wf)
    if wtype == Q6_K:
        return synth.pack_q6_K(wf)
    return quantize(oracle(), "orc", wf, "q8_0")


def both(sess, h, xb, m, n, bias=None, ldy=0, y_offset=0):
    span = (y_offset + (m - 1) * (ldy or n) + n)
    outs = []
    for call in (sess.matmul_ex, sess.matmul_noalloc):
        yb = sess.to_device(np.full(span, 7.0, np.float32))
        _lib.check(call(h, xb.ptr, m, yb.ptr, bias, ldy, y_offset), call.__name__)
        outs.append(yb.download(np.float32, span))
        yb.free()
    return outs


@pytest.mark.parametrize("wtype", [Q5_K, Q6_K, Q8_0])
def test_two_calls_second_smaller(sess, wtype):
    K, N = 1024, 4096
    rng = np.random.default_rng(100 + wtype)
    wb = pack(wtype, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    h = sess.weight(f"noalloc:{wtype}", wb, wtype, K, N)
    # 1100 tokens: 5 x 32 tiles of 256 x 128, more than half a round of CUs,
    # so pixhip_matmul_ex runs unsplit; 300 tokens: 64 tiles, split K.
    for m in (1100, 300):
        print(f"noalloc type {wtype}: {m} x {K} x {N}", flush=True)
        x = (rng.standard_normal((m, K)) * rng.choice([0.1, 1.0, 10.0], (m, 1))).astype(np.float32)
        xb = sess.to_device(x)
        y_ref, y = (o.reshape(m, N) for o in both(sess, h, xb, m, N))
        xb.free()
        err = row_rel_error(y, y_ref).max()
        exact = np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        print(f"  bit-identical={exact} rel={err:.2e}", flush=True)
        if m == 1100:
            assert exact
        assert err <= SPLIT_TOL
        if m == 300:  # and against the oracle
            assert row_rel_error(y, quant_matmul(oracle(), "orc", wb, wtype, x, N)).max() <= TOL


@pytest.mark.parametrize("wtype", [Q5_K, Q6_K, Q8_0])
def test_matvec_with_bias_and_stride(sess, wtype):
    K, N = 2048, 768
    rng = np.random.default_rng(200 + wtype)
    wb = pack(wtype, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    h = sess.weight(f"noalloc-mv:{wtype}", wb, wtype, K, N)
    bvec = sess.to_device(rng.standard_normal(N).astype(np.float32))
    for step in range(2):
        print(f"noalloc matvec type {wtype}, call {step}", flush=True)
        xb = sess.to_device(rng.standard_normal((1, K)).astype(np.float32))
        y_ref, y = both(sess, h, xb, 1, N, bvec.ptr, N + 5, 3)
        xb.free()
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        assert (y[:3] == 7.0).all() and (y[3 + N:] == 7.0).all()
    bvec.free()


def test_errors(sess):
    K, N = 4096, 128
    rng = np.random.default_rng(300)
    wb = synth.pack_q5_K((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    h = sess.weight("noalloc-err", wb, Q5_K, K, N)
    small = sess.to_device(rng.standard_normal((8, K)).astype(np.float32))
    yb = sess.alloc(8 * N * 4)
    print("noalloc: layout not resident", flush=True)
    assert sess.matmul_noalloc(h, small.ptr, 8, yb.ptr) == _lib.ERR_STATE
    _lib.check(sess.matmul_ex(h, small.ptr, 8, yb.ptr), "pixhip_matmul_ex")
    print("noalloc: host memory", flush=True)
    xh = np.zeros((8, K), np.float32)
    assert sess.matmul_noalloc(h, xh.ctypes.data, 8, yb.ptr) == _lib.ERR_ARGUMENT
    print("noalloc: beyond the array", flush=True)
    big_m = 8192  # 8192 x 4096 int8 activations alone are 32 MiB
    xbig = sess.alloc(big_m * K * 4)
    ybig = sess.alloc(big_m * N * 4)
    assert sess.matmul_noalloc(h, xbig.ptr, big_m, ybig.ptr) == _lib.ERR_MEMORY
    for b in (small, yb, xbig, ybig):
        b.free()
