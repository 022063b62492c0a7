"""The fused producers of a linear layer's input (pixhip_norm_quantize,
pixhip_silu_gate_quantize) through the C ABI, against the reference's vectors
(tests/golden/g5_norm, g6_silu_gate) and the oracle.

- Norm (tensor_norm, src/tensor.cpp:174-197, then z_modulate,
  src/inference.cpp:263-277): the fp32 output and the quantized blocks are
  bit-exact.  The kernel takes its double sums in another order than the
  reference's running sum; that moves their last bits only, far below the fp32
  rounding of the inverse.
- SiLU * gate (src/tensor.cpp:199-209, :334-345): the reference's expf is
  glibc's, which is not correctly rounded: for about 0.07% of N(0, 16) inputs it
  rounds e^-v, lying within ~0.0004 ulp of an fp32 midpoint, the other way
  (e.g. e^6.26477 = 525.7206726, 0.4997 ulp above 525.72064: glibc returns the
  next float up).  Here e^-v is the fp32 rounding of a double exponential, i.e.
  correctly rounded.  One ulp in e^-v moves the quotient by up to ~1.5 ulp and
  the product by up to 3, so the fp32 product is checked to 4 ulps and to at
  most 0.1% inexact values.  The blocks are bit-exact against the oracle's
  quantizer applied to the same product.
- The GEMM that consumes the fused activations (PIXHIP_STAGE_MULTIPLY) is within
  max|y - r| / max|r| <= 1e-4 per token row of the oracle's matmul.
"""
import os

import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import Q5_K, Q6_K, Q8_0, modulate_rows, norm_rows, oracle, quant_matmul, quantize, silu_gate
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
STAGE_MULTIPLY = 2
BLOCK_BYTES = {"q8_K": (256, 292), "q8_0": (32, 34)}
MAX_ULP = 4  # SiLU * gate fp32 product vs the reference's (glibc expf)


def few_inexact(d):
    """At most 0.1% of the values (plus 3, for small samples) differ at all."""
    return np.count_nonzero(d) <= 0.001 * d.size + 3


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def kind_of(wtype):
    return "q8_0" if wtype == Q8_0 else "q8_K"


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_norm(sess, wtype, x, w=None, eps=1e-5, centered=0, mod=None):
    """-> (fp32 output, reference-layout blocks or None)"""
    rows, k = x.shape
    xb = sess.to_device(np.ascontiguousarray(x, np.float32))
    wb = sess.to_device(w) if w is not None else None
    mb = sess.to_device(mod) if mod is not None else None
    yb = sess.alloc(x.nbytes)
    bb = None
    if wtype:
        per, nbytes = BLOCK_BYTES[kind_of(wtype)]
        bb = sess.alloc(rows * k // per * nbytes)
    _lib.check(sess.norm_quantize(wtype, xb.ptr, rows, k, wb.ptr if wb else None, eps, centered, mb.ptr if mb else None,
                                  yb.ptr, bb.ptr if bb else None), "pixhip_norm_quantize")
    y = yb.download(np.float32, x.size).reshape(x.shape)
    blocks = None
    if bb is not None:
        per, nbytes = BLOCK_BYTES[kind_of(wtype)]
        blocks = bb.download(np.uint8, rows * k // per * nbytes).reshape(rows, -1)
    return y, blocks


def multiply(sess, wtype, wbytes, rows, k, columns, tag):
    w = sess.weight(f"fused:{tag}:{wtype}:{rows}:{k}", wbytes, wtype, k, rows)
    yb = sess.alloc(columns * rows * 4)
    _lib.check(sess.matmul_stage(w, None, columns, yb.ptr, STAGE_MULTIPLY), "pixhip_matmul_stage(MULTIPLY)")
    return yb.download(np.float32, columns * rows).reshape(columns, rows)


def pack(wtype, wf):
    if wtype == Q8_0:
        return quantize(oracle(), "orc", wf, "q8_0")
    return synth.pack_q5_K(wf) if wtype == Q5_K else synth.pack_q6_K(wf)


# ---------------------------------------------------------------- norm

@pytest.mark.parametrize("wtype", [Q5_K, Q8_0])
@pytest.mark.parametrize("centered", [0, 1])
@pytest.mark.parametrize("wi", ["none", "w"])
def test_norm_golden(sess, wtype, centered, wi):
    g = np.load(os.path.join(GOLDEN, "g5_norm.npz"))
    key = f"c{centered}_{wi}"
    y, blocks = run_norm(sess, wtype, g["x"], None if wi == "none" else g["w"], float(g["eps"][centered]), centered)
    assert np.array_equal(bits(y), bits(g[f"{key}_y"])), np.nonzero((bits(y) != bits(g[f"{key}_y"])).any(axis=1))[0]
    assert np.array_equal(blocks, g[f"{key}_{kind_of(wtype)}"])


@pytest.mark.parametrize("wtype,rows,k,centered,weighted,modulated", [
    (Q5_K, 37, 3840, 0, True, True),      # DiT block: RMS norm, weight, modulation
    (Q5_K, 9, 3072, 1, True, False),      # centered, Qwen-Image hidden size
    (Q5_K, 5, 8192, 1, True, True),       # two waves per row
    (Q6_K, 7, 12288, 0, True, False),     # four waves per row
    (Q8_0, 6, 8224, 1, False, False),     # Q8_0 padding block, four waves per row
    (Q6_K, 5, 16640, 0, False, False),    # rows past the register-resident length (re-read path)
    (Q8_0, 19, 3872, 0, True, True),      # Q8_0 with a padding block (inner % 64 == 32)
    (Q8_0, 3, 96, 1, False, True),
])
def test_norm_quantize_multiply_vs_oracle(sess, wtype, rows, k, centered, weighted, modulated):
    rng = np.random.default_rng(rows * k)
    x = (rng.standard_normal((rows, k)) * rng.choice([1e-3, 1.0, 40.0], (rows, 1)) + 2.0 * centered).astype(np.float32)
    x[:, rng.integers(0, k, 4)] *= 15.0
    w = (1.0 + 0.2 * rng.standard_normal(k)).astype(np.float32) if weighted else None
    mod = (0.3 * rng.standard_normal(k)).astype(np.float32) if modulated else None
    o = oracle()
    ref = norm_rows(o, "orc", x, w, 1e-5, centered)
    if mod is not None:
        ref = modulate_rows(o, ref, mod)
    y, blocks = run_norm(sess, wtype, x, w, 1e-5, centered, mod)
    assert np.array_equal(bits(y), bits(ref))
    assert np.array_equal(blocks, quantize(o, "orc", ref, kind_of(wtype)))
    n = 300
    wb = pack(wtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    out = multiply(sess, wtype, wb, n, k, rows, f"norm{rows}")
    want = quant_matmul(o, "orc", wb, wtype, ref, n)
    err = row_rel_error(out, want).max()
    print(f"norm type={wtype} rows={rows} K={k} rel={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("k,centered", [(512, 0), (100, 1), (4100, 0)])
def test_norm_type0_normalizes_only(sess, k, centered):
    """tensor_norm alone (vulkan_norm), any width that is a multiple of 4."""
    rng = np.random.default_rng(3 + k)
    x = (rng.standard_normal((5, k)) + centered).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    y, blocks = run_norm(sess, 0, x, w, 1e-6, centered)
    assert blocks is None
    assert np.array_equal(bits(y), bits(norm_rows(oracle(), "orc", x, w, 1e-6, centered)))
    xb = sess.to_device(x)
    assert sess.norm_quantize(0, xb.ptr, 5, k) == _lib.ERR_ARGUMENT  # nothing to write


@pytest.mark.parametrize("rows,k,centered,weighted,modulated", [
    (37 * 30, 128, 0, True, False),   # DiT per-head q / k norm: rows x heads rows of 128
    (33, 128, 1, True, True),
    (17, 124, 0, False, True),        # past-the-end lanes of the second half
    (5, 20, 1, True, False),          # one float4 per lane or none
    (3, 4, 0, True, True),
])
def test_norm_short_rows(sess, rows, k, centered, weighted, modulated):
    """Rows of up to 128 values (16 lanes per row) against the oracle, bit for bit."""
    rng = np.random.default_rng(rows + k)
    x = (rng.standard_normal((rows, k)) * rng.choice([1e-3, 1.0, 40.0], (rows, 1)) + 1.5 * centered).astype(np.float32)
    w = (1.0 + 0.2 * rng.standard_normal(k)).astype(np.float32) if weighted else None
    mod = (0.3 * rng.standard_normal(k)).astype(np.float32) if modulated else None
    o = oracle()
    ref = norm_rows(o, "orc", x, w, 1e-6, centered)
    if mod is not None:
        ref = modulate_rows(o, ref, mod)
    y, blocks = run_norm(sess, 0, x, w, 1e-6, centered, mod)
    assert blocks is None
    assert np.array_equal(bits(y), bits(ref)), np.nonzero((bits(y) != bits(ref)).any(axis=1))[0][:8]


def test_multiply_after_norm_checks_the_activation_kind(sess):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 512)).astype(np.float32)
    run_norm(sess, Q5_K, x)
    wb = pack(Q8_0, (rng.standard_normal((64, 512)) * 0.02).astype(np.float32))
    w = sess.weight("fused:kind", wb, Q8_0, 512, 64)
    yb = sess.alloc(8 * 64 * 4)
    assert sess.matmul_stage(w, None, 8, yb.ptr, STAGE_MULTIPLY) == _lib.ERR_STATE


# ---------------------------------------------------------------- SiLU * gate

def run_silu_gate(sess, wtype, gate, up, in_place=False):
    rows, k = gate.shape
    gb = sess.to_device(np.ascontiguousarray(gate, np.float32))
    ub = sess.to_device(np.ascontiguousarray(up, np.float32))
    yb = gb if in_place else sess.alloc(gate.nbytes)
    per, nbytes = BLOCK_BYTES[kind_of(wtype)]
    bb = sess.alloc(rows * k // per * nbytes)
    _lib.check(sess.silu_gate_quantize(wtype, gb.ptr, ub.ptr, rows, k, yb.ptr, bb.ptr), "pixhip_silu_gate_quantize")
    y = yb.download(np.float32, gate.size).reshape(gate.shape)
    return y, bb.download(np.uint8, rows * k // per * nbytes).reshape(rows, -1)


def ulps_apart(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    scale = np.spacing(np.maximum(np.abs(a), np.abs(b)))
    return np.where(a == b, 0.0, np.abs(a.astype(np.float64) - b) / scale)


@pytest.mark.parametrize("wtype", [Q5_K, Q8_0])
def test_silu_gate_golden(sess, wtype):
    g = np.load(os.path.join(GOLDEN, "g6_silu_gate.npz"))
    y, blocks = run_silu_gate(sess, wtype, g["gate"], g["up"])
    d = ulps_apart(y, g["y"])
    print(f"silu*gate golden: {np.mean(d == 0):.6f} bit-exact, max {d.max():.0f} ulp", flush=True)
    assert d.max() <= MAX_ULP and few_inexact(d)
    assert np.array_equal(blocks, quantize(oracle(), "orc", y, kind_of(wtype)))
    if d.max() == 0:
        assert np.array_equal(blocks, g[kind_of(wtype)])


@pytest.mark.parametrize("wtype,rows,k,in_place", [
    (Q8_0, 64, 10240, False),   # DiT block FFN down input (Q8_0 weights)
    (Q5_K, 33, 3840, True),     # in place, as tensor_silu / tensor_gate update `gate`
    (Q8_0, 7, 96, False),       # a padding block
])
def test_silu_gate_quantize_multiply_vs_oracle(sess, wtype, rows, k, in_place):
    rng = np.random.default_rng(rows + k)
    gate = (rng.standard_normal((rows, k)) * 4.0).astype(np.float32)
    up = (rng.standard_normal((rows, k)) * 2.0).astype(np.float32)
    o = oracle()
    ref = silu_gate(o, "orc", gate, up)
    y, blocks = run_silu_gate(sess, wtype, gate, up, in_place)
    d = ulps_apart(y, ref)
    print(f"silu*gate rows={rows} K={k}: {np.mean(d == 0):.6f} bit-exact, max {d.max():.0f} ulp", flush=True)
    assert d.max() <= MAX_ULP and few_inexact(d)
    assert np.array_equal(blocks, quantize(o, "orc", y, kind_of(wtype)))
    n = 257
    wb = pack(wtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    out = multiply(sess, wtype, wb, n, k, rows, f"gate{rows}")
    want = quant_matmul(o, "orc", wb, wtype, ref, n)
    err = row_rel_error(out, want).max()
    print(f"silu*gate type={wtype} rows={rows} K={k} rel={err:.2e}", flush=True)
    assert err <= TOL
