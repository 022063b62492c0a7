"""HIP path vs the oracle and the reference's golden vectors, through the C ABI.

Integer gate (bit-exact): quantized activation blocks (Q8_0, Q8_K) and the
per-block integer sums the GEMM's fp32 epilogue consumes.
Float gate: outputs within max|y - r| / max|r| <= 1e-4 per token row of the
reference CPU kernel's outputs on the same inputs.
"""
import numpy as np
import pytest

from gpu_helpers import TOL, gpu_matmul, row_rel_error
from oracle_lib import Q5_K, Q6_K, Q8_0, oracle, q8_K_blocks, quant_matmul, quantize
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    print("device:", s.device_name(), flush=True)
    yield s
    s.close()


def load(name):
    return np.load(f"{GOLDEN}/{name}.npz")


def pack(wtype, wf):
    if wtype == Q8_0:
        return quantize(oracle(), "orc", wf, "q8_0")
    return synth.pack_q5_K(wf) if wtype == Q5_K else synth.pack_q6_K(wf)


# ---------------------------------------------------------------- quantizers

def test_quantize_q8_0_golden(sess):
    g = load("g1_quantize_q8_0")
    x = g["x"]
    rows, k = x.shape
    xb = sess.to_device(x)
    bb = sess.alloc(g["blocks"].nbytes)
    _lib.check(sess.quantize_q8_0(xb.ptr, bb.ptr, rows, k), "quantize_q8_0")
    out = bb.download(np.uint8, g["blocks"].size).reshape(g["blocks"].shape)
    assert np.array_equal(out, g["blocks"]), np.nonzero((out != g["blocks"]).any(axis=1))[0]


def test_quantize_q8_K_golden(sess):
    g = load("g2_quantize_q8_K")
    x = g["x"]
    rows, k = x.shape
    xb = sess.to_device(x)
    bb = sess.alloc(g["blocks"].nbytes)
    _lib.check(sess.quantize_q8_K(xb.ptr, bb.ptr, rows, k), "quantize_q8_K")
    out = bb.download(np.uint8, g["blocks"].size).reshape(g["blocks"].shape)
    bad = np.nonzero((out != g["blocks"]).any(axis=1))[0]
    assert bad.size == 0, f"rows differ: {bad}"


@pytest.mark.parametrize("kind,k", [("q8_0", 96), ("q8_0", 3840), ("q8_K", 3840), ("q8_K", 12288)])
def test_quantize_random_vs_oracle(sess, kind, k):
    rng = np.random.default_rng(k)
    x = (rng.standard_normal((37, k)) * rng.choice([1e-3, 1.0, 50.0], (37, 1))).astype(np.float32)
    x[:, rng.integers(0, k, 5)] *= 20.0
    ref = quantize(oracle(), "orc", x, kind)
    xb = sess.to_device(x)
    bb = sess.alloc(ref.nbytes)
    fn = sess.quantize_q8_0 if kind == "q8_0" else sess.quantize_q8_K
    _lib.check(fn(xb.ptr, bb.ptr, x.shape[0], k), kind)
    out = bb.download(np.uint8, ref.size).reshape(ref.shape)
    assert np.array_equal(out, ref)


# ---------------------------------------------------------------- golden matmuls

def test_matmul_golden_cases(sess):
    g = load("g4_matmul")
    for i in range(int(g["count"])):
        wtype, m, n, k = (int(v) for v in g[f"c{i}_shape"])
        y = gpu_matmul(sess, g[f"c{i}_w"], wtype, g[f"c{i}_x"], n)
        err = row_rel_error(y, g[f"c{i}_y"]).max()
        print(f"case {i} type={wtype} M={m} N={n} K={k} rel={err:.2e}", flush=True)
        assert err <= TOL, (i, wtype, m, n, k, err)


# ---------------------------------------------------------------- integer gate

@pytest.mark.parametrize("wtype", [Q8_0, Q5_K, Q6_K])
def test_block_sums_exact(sess, wtype):
    rng = np.random.default_rng(wtype)
    m, n, k = 5, 33, 512
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = pack(wtype, wf)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.integers(0, k, 4)] *= 20.0
    w = sess.weight(f"sums:{wtype}", wb, wtype, k, n)
    blocks = k // 256 if wtype != Q8_0 else (k + 63) // 64 * 2
    xb = sess.to_device(x)
    sb = sess.alloc(m * n * blocks * 4)
    mb = sess.alloc(m * n * blocks * 4)
    _lib.check(sess.block_sums(w, xb.ptr, m, sb.ptr, mb.ptr), "block_sums")
    sums = sb.download(np.int32, m * n * blocks).reshape(m, n, blocks)
    mins = mb.download(np.int32, m * n * blocks).reshape(m, n, blocks)
    o = oracle()
    import ctypes
    if wtype == Q8_0:
        a = quantize(o, "orc", x, "q8_0")
        wb3 = wb.reshape(n, k // 32, 34)
        a3 = a.reshape(m, k // 32, 34)
        for c in range(m):
            for r in range(n):
                for b in range(k // 32):
                    want = o.orc_block_sums_q8_0(wb3[r, b].ctypes.data, a3[c, b].ctypes.data)
                    assert sums[c, r, b] == want, (c, r, b)
    else:
        a = quantize(o, "orc", x, "q8_K")
        wbytes = 176 if wtype == Q5_K else 210
        wb3 = np.ascontiguousarray(wb.reshape(n, k // 256, wbytes))
        a3 = np.ascontiguousarray(a.reshape(m, k // 256, 292))
        s_out, m_out = ctypes.c_int32(), ctypes.c_int32()
        for c in range(m):
            for r in range(n):
                for b in range(k // 256):
                    if wtype == Q5_K:
                        o.orc_superblock_sums_q5_K(wb3[r, b].ctypes.data, a3[c, b].ctypes.data, ctypes.addressof(s_out),
                                                   ctypes.addressof(m_out))
                        assert (sums[c, r, b], mins[c, r, b]) == (s_out.value, m_out.value), (c, r, b)
                    else:
                        want = o.orc_superblock_sum_q6_K(wb3[r, b].ctypes.data, a3[c, b].ctypes.data)
                        assert sums[c, r, b] == want, (c, r, b)


# ---------------------------------------------------------------- ragged shapes vs oracle

@pytest.mark.parametrize("wtype,m,n,k", [
    (Q5_K, 2, 1, 256), (Q5_K, 129, 130, 768), (Q5_K, 37, 300, 3840),
    (Q6_K, 3, 257, 512), (Q6_K, 200, 64, 1024),
    (Q8_0, 2, 7, 32), (Q8_0, 131, 129, 96), (Q8_0, 64, 256, 3840), (Q8_0, 200, 300, 4000),
    # enough 256 x 128 tiles (9 x 16) for the Q8_0 GEMM's whole-tile form; the shapes above run its K-grouped form
    (Q8_0, 2100, 2000, 512),
])
def test_gemm_ragged_vs_oracle(sess, wtype, m, n, k):
    rng = np.random.default_rng(m * 1000 + n)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = pack(wtype, wf)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = quant_matmul(oracle(), "orc", wb, wtype, x, n)
    y = gpu_matmul(sess, wb, wtype, x, n)
    err = row_rel_error(y, ref).max()
    print(f"type={wtype} M={m} N={n} K={k} rel={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("wtype,n,k", [(Q5_K, 1000, 256), (Q5_K, 77, 12288), (Q8_0, 999, 32), (Q8_0, 300, 3616),
                                       (Q6_K, 513, 4096), (Q6_K, 64, 12288),
                                       (Q5_K, 150001, 256), (Q8_0, 150001, 64), (Q6_K, 150001, 256),
                                       (Q5_K, 513, 18944), (Q8_0, 700, 18944), (Q6_K, 300, 18944),
                                       (Q5_K, 65, 24576), (Q8_0, 66, 24576), (Q6_K, 67, 24576), (Q5_K, 64, 24832)])
def test_matvec_vs_oracle(sess, wtype, n, k):
    """Every output row against the oracle.  The 150001-row cases give each wave
    more than 32 row pairs on a 256-CU device, so a wave's parked row totals are
    written out while its loop still runs (as well as at its end).  K = 18944
    (a decode FFN down projection) and 24576 are the long rows (5 and 6 units of
    64 values per lane); K = 24832 is past the matvec's limit and runs on the
    GEMM path."""
    rng = np.random.default_rng(n + k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = pack(wtype, wf)
    x = rng.standard_normal((1, k)).astype(np.float32)
    ref = quant_matmul(oracle(), "orc", wb, wtype, x, n)
    y = gpu_matmul(sess, wb, wtype, x, n)
    err = row_rel_error(y, ref).max()
    print(f"matvec type={wtype} N={n} K={k} rel={err:.2e}", flush=True)
    assert err <= TOL


def test_copy_device_is_exact(sess):
    rng = np.random.default_rng(31)
    for nbytes in (16, 4096 + 16, 3 * (1 << 20) + 5):
        data = rng.integers(0, 256, nbytes, dtype=np.uint8)
        src = sess.to_device(data)
        dst = sess.alloc(nbytes)
        sess.copy_device(dst.ptr, src.ptr, nbytes)
        sess.synchronize()
        assert np.array_equal(dst.download(np.uint8, nbytes), data)
        src.free()
        dst.free()
