"""The elementwise ops around the linears (pixhip_pointwise, pixhip_rope)
through the C ABI, against the reference's vectors (tests/golden/g7_ops,
written by the compiled src/tensor.cpp) and the oracle.

Bit-exact: gate, add, bias and RoPE (plain fp32 arithmetic in the reference's
order).  SiLU and GELU: the reference's expf / erff / tanhf are glibc's, not
correctly rounded; here they are the fp32 rounding of the double function. The
results are checked to 4 ulps (plus, for GELU, the cancellation in 1 + erf or
1 + tanh for negative v: |0.5 v| * 3e-7).  SiLU is also held to at most 1% of
values inexact (glibc's expf is off correct rounding for ~0.07% of arguments);
GELU is not, since glibc's erff and tanhf are for ~2% and ~8% of these inputs
(measured on the G7 values by emulating the kernel's arithmetic on the host).
"""
import os

import numpy as np
import pytest

from oracle_lib import add, bias, gelu, oracle, rope, silu_gate
from pixelina_amd import _lib

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
OP = {"silu": 2, "gate": 3, "add": 4, "bias": 14, "gelu_exact": 18, "gelu_tanh": 19}


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_op(sess, op, x, second=None):
    xb = sess.to_device(np.ascontiguousarray(x, np.float32))
    sb = sess.to_device(np.ascontiguousarray(second, np.float32)) if second is not None else None
    _lib.check(sess.pointwise(OP[op], xb.ptr, sb.ptr if sb else None, x.shape[0], x.shape[1]), op)
    return xb.download(np.float32, x.size).reshape(x.shape)


def run_rope(sess, x, heads, cos, sin, interleaved):
    xb, cb, nb = sess.to_device(x), sess.to_device(cos), sess.to_device(sin)
    _lib.check(sess.rope(xb.ptr, x.shape[0], x.shape[1], heads, cb.ptr, nb.ptr, interleaved), "rope")
    return xb.download(np.float32, x.size).reshape(x.shape)


def close(got, want, x=None):
    """Within 4 ulps (+ the GELU cancellation term when x is given); without x
    (SiLU) also at most 1% of the values inexact."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    tol = 4 * np.spacing(np.maximum(np.abs(got), np.abs(want)).astype(np.float32)).astype(np.float64)
    if x is not None:
        tol = tol + 0.5 * np.abs(np.asarray(x, np.float64)) * 3e-7
    off = np.abs(got - want)
    print(f"inexact {np.count_nonzero(off) / off.size:.4f}, max {off.max():.3g}", flush=True)
    return (off <= tol).all() and (x is not None or np.count_nonzero(off) <= 0.01 * off.size + 3)


def test_ops_golden(sess):
    g = np.load(os.path.join(GOLDEN, "g7_ops.npz"))
    x, h = g["x"], int(g["heads"])
    assert np.array_equal(bits(run_op(sess, "bias", x, g["b"])), bits(g["bias"]))
    assert np.array_equal(bits(run_op(sess, "add", x, g["y"])), bits(g["add"]))
    assert np.array_equal(bits(run_rope(sess, x, h, g["cos"], g["sin"], 0)), bits(g["rope_split"]))
    assert np.array_equal(bits(run_rope(sess, x, h, g["cos"], g["sin"], 1)), bits(g["rope_interleaved"]))
    assert close(run_op(sess, "gelu_exact", x), g["gelu_exact"], x)
    assert close(run_op(sess, "gelu_tanh", x), g["gelu_tanh"], x)


@pytest.mark.parametrize("rows,channels", [(1, 4), (37, 3840), (4608, 3840)])
def test_pointwise_vs_oracle(sess, rows, channels):
    rng = np.random.default_rng(rows + channels)
    x = (rng.standard_normal((rows, channels)) * 4.0).astype(np.float32)
    y = rng.standard_normal((rows, channels)).astype(np.float32)
    b = rng.standard_normal(channels).astype(np.float32)
    o = oracle()
    assert np.array_equal(bits(run_op(sess, "gate", x, y)), bits(x * y))
    assert np.array_equal(bits(run_op(sess, "add", x, y)), bits(add(o, "orc", x, y)))
    assert np.array_equal(bits(run_op(sess, "bias", x, b)), bits(bias(o, "orc", x, b)))
    assert close(run_op(sess, "silu", x), silu_gate(o, "orc", x, np.ones_like(x)))
    for form, name in ((0, "gelu_exact"), (1, "gelu_tanh")):
        assert close(run_op(sess, name, x), gelu(o, "orc", x, form), x), name


@pytest.mark.parametrize("rows,heads,dim,interleaved", [
    (3, 2, 8, 0), (4608, 30, 128, 0), (257, 16, 64, 1),
    (4608, 30, 128, 1),   # the DiT block's q / k (interleaved pairs, a float4 per thread)
    (5, 3, 12, 1),        # interleaved, head size a multiple of 4 only
    (5, 3, 12, 0),        # split halves of 6: the scalar pair kernel
    (7, 2, 6, 1),         # head size not a multiple of 4: the scalar pair kernel
    (70001, 1, 8, 1),     # more rows than one grid dimension holds
])
def test_rope_vs_oracle(sess, rows, heads, dim, interleaved):
    rng = np.random.default_rng(rows * heads + dim)
    x = rng.standard_normal((rows, heads * dim)).astype(np.float32)
    th = rng.uniform(0, 2 * np.pi, (rows, dim // 2))
    cos, sin = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
    got = run_rope(sess, x, heads, cos, sin, interleaved)
    assert np.array_equal(bits(got), bits(rope(oracle(), "orc", x, heads, cos, sin, interleaved)))


def test_ops_reject_bad_arguments(sess):
    xb = sess.alloc(64)
    assert sess.pointwise(5, xb.ptr, None, 1, 4) == _lib.ERR_UNSUPPORTED      # an op outside this set
    assert sess.pointwise(OP["add"], xb.ptr, None, 1, 4) == _lib.ERR_ARGUMENT  # missing operand
    assert sess.rope(xb.ptr, 1, 12, 4, xb.ptr, xb.ptr, 0) == _lib.ERR_ARGUMENT  # odd head size
