"""The HIP path on the workloads the path is specified on, at their full sizes,
against the oracle (the restatement of src/kernels_quant.cpp's CPU path):

- a single Q8_0 linear, activations [256, 3840], weights [3840, 3840];
- the decode matvec, x [1, 3584], W [18944, 3584], Q8_0 / Q5_K / Q6_K, 100 repeats;
- the DiT FFN GEMM, X [4096, 3840] with 1% outlier channels x20, W Q5_K [10240, 3840];
- every linear of a DiT block (M = 4096 + 512 tokens, Q5_K except FFN-down Q8_0);
- every linear of a Qwen-Image edit block (M = 8448, K/N 3072/9216/12288, Q5_K),
  activations with per-token scales log-uniform in [0.1, 10].

The single linear, the matvecs and the FFN GEMM are compared on every output.
The block linears are compared on sampled token rows: each token row of
cpu_quant_matmul depends only on that row's activations (src/kernels_quant.cpp:
383-405), so the oracle runs on the sampled rows alone.  Every row at full size
is covered by a size-independent property instead: the GEMM of the rows rolled by
an offset that is not a multiple of the tile gives the same outputs per token
row.  Rows that fall in a tile of the last, split-K round in one placement and
a whole tile in the other sum the same integer block results in another fp32
order, so the roll property is checked to 1e-6 of each row's largest output
(an indexing mistake shows as an O(1) error).
Float gate: max|y - r| / max|r| <= 1e-4 per token row.
"""
import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import Q5_K, Q6_K, Q8_0, oracle, quant_matmul, quantize
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def weights(seed, n, k, wtype):
    wf = np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    if wtype == Q8_0:
        return quantize(oracle(), "orc", wf, "q8_0")
    return synth.pack_q5_K(wf) if wtype == Q5_K else synth.pack_q6_K(wf)


def activations(seed, m, k):
    return np.random.default_rng(seed).standard_normal((m, k), dtype=np.float32)


def run_gpu(sess, key, wb, wtype, x, n):
    m, k = x.shape
    w = sess.weight(key, wb, wtype, k, n)
    xb = sess.to_device(x)
    yb = sess.alloc(m * n * 4)
    _lib.check(sess.matmul(w, xb.ptr, m, yb.ptr), key)
    y = yb.download(np.float32, m * n).reshape(m, n)
    xb.free()
    yb.free()
    return y


def sample_rows(m, count, seed):
    """First and last rows, both sides of every 256-token tile edge, and random rows."""
    edges = [r for t in range(256, m, 256) for r in (t - 1, t)]
    rng = np.random.default_rng(seed)
    picks = set([0, m - 1] + edges[:: max(1, len(edges) // 16)]) | set(rng.integers(0, m, count).tolist())
    return np.array(sorted(picks))


def check_rows(name, y, x, rows_idx, wb, wtype, n):
    ref = quant_matmul(oracle(), "orc", wb, wtype, x[rows_idx], n)
    err = row_rel_error(y[rows_idx], ref)
    print(f"{name}: rows={len(rows_idx)} max rel={err.max():.2e}", flush=True)
    assert np.isfinite(y).all()
    assert err.max() <= TOL, (name, int(rows_idx[int(err.argmax())]))


ROLL_TOL = 1e-6


def check_roll(sess, key, wb, wtype, x, n, y, shift=37):
    """Rolling the token rows by a non-multiple of the tile moves every row to
    another tile position; each row's outputs must stay the same (to fp32
    summation order, see the module docstring)."""
    y2 = run_gpu(sess, key, wb, wtype, np.roll(x, shift, axis=0), n)
    err = row_rel_error(y2, np.roll(y, shift, axis=0))
    assert err.max() <= ROLL_TOL, (key, int(err.argmax()), float(err.max()))


def test_single_q8_0_linear(sess):
    m, k, n = 256, 3840, 3840
    x = synth.normal(synth.SEED_ACTIVATIONS, (m, k))
    wb = quantize(oracle(), "orc", synth.normal(synth.SEED_WEIGHTS, (n, k), std=0.02), "q8_0")
    y = run_gpu(sess, "wl:q8_0_linear", wb, Q8_0, x, n)
    check_rows("q8_0 linear [256,3840]x[3840,3840]", y, x, np.arange(m), wb, Q8_0, n)


@pytest.mark.parametrize("wtype", [Q8_0, Q5_K, Q6_K])
def test_decode_matvec(sess, wtype):
    n, k = 18944, 3584
    x = synth.normal(synth.SEED_ACTIVATIONS, (1, k))
    wb = weights(100 + wtype, n, k, wtype)
    w = sess.weight(f"wl:decode:{wtype}", wb, wtype, k, n)
    xb = sess.to_device(x)
    yb = sess.alloc(n * 4)
    outs = []
    for rep in range(100):
        _lib.check(sess.matmul(w, xb.ptr, 1, yb.ptr), "decode matvec")
        if rep in (0, 99):
            outs.append(yb.download(np.float32, n))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "repeats differ"
    check_rows(f"decode matvec type={wtype}", outs[0][None, :], x, np.arange(1), wb, wtype, n)


@pytest.mark.parametrize("wtype", [Q5_K, Q6_K])
def test_dit_ffn_gemm_full(sess, wtype):
    """The DiT FFN shape with the outlier channels; every output against the oracle
    (Q5_K is the specified format, Q6_K the next one at the same shape)."""
    m, k, n = 4096, 3840, 10240
    x = activations(1337, m, k)
    x[:, synth.outlier_channels(k)] *= 20.0
    wb = weights(200 + wtype, n, k, wtype)
    y = run_gpu(sess, f"wl:ffn:{wtype}", wb, wtype, x, n)
    rows = np.arange(m) if wtype == Q5_K else sample_rows(m, 64, 5)
    check_rows(f"DiT FFN type={wtype}", y, x, rows, wb, wtype, n)
    check_roll(sess, f"wl:ffn:{wtype}", wb, wtype, x, n, y)


DIT_BLOCK = [("qkv", Q5_K, 3840, 11520), ("out", Q5_K, 3840, 3840), ("w1", Q5_K, 3840, 10240),
             ("w3", Q5_K, 3840, 10240), ("w2", Q8_0, 10240, 3840)]


@pytest.mark.parametrize("name,wtype,k,n", DIT_BLOCK, ids=[d[0] for d in DIT_BLOCK])
def test_dit_block_linears(sess, name, wtype, k, n):
    m = 4096 + 512
    x = activations(300 + k, m, k)
    wb = weights(310 + n + wtype, n, k, wtype)
    y = run_gpu(sess, f"wl:dit:{name}", wb, wtype, x, n)
    check_rows(f"DiT block {name} [{m},{k}]x[{n}]", y, x, sample_rows(m, 48, n), wb, wtype, n)
    check_roll(sess, f"wl:dit:{name}", wb, wtype, x, n, y)


QWEN_BLOCK = [("qkv", 3072, 9216), ("out", 3072, 3072), ("ff_up", 3072, 12288), ("ff_down", 12288, 3072)]


@pytest.mark.parametrize("name,k,n", QWEN_BLOCK, ids=[q[0] for q in QWEN_BLOCK])
def test_qwen_image_block_linears(sess, name, k, n):
    m = 4096 + 4096 + 256
    x = activations(400 + k, m, k)
    x *= synth.log_uniform(401 + k, m, 0.1, 10.0)[:, None]
    wb = weights(410 + n, n, k, Q5_K)
    y = run_gpu(sess, f"wl:qwen:{name}", wb, Q5_K, x, n)
    check_rows(f"Qwen-Image {name} [{m},{k}]x[{n}]", y, x, sample_rows(m, 48, n), wb, Q5_K, n)
    check_roll(sess, f"wl:qwen:{name}", wb, Q5_K, x, n, y)


# ---------------------------------------------------------------- interface semantics

@pytest.mark.parametrize("m", [1, 70])
@pytest.mark.parametrize("wtype", [Q8_0, Q5_K])
def test_matmul_ex_bias_stride_offset(sess, wtype, m):
    """The conv path's push words (src/backend_vulkan.cpp:1085-1091): Y[y_offset +
    c*ldy + r] = dot + bias[r]; elements outside the written rows keep their values."""
    k, n, ldy, off = 512, 96, 130, 7
    x = activations(500 + m, m, k)
    wb = weights(510, n, k, wtype)
    bias = np.random.default_rng(520).standard_normal(n, dtype=np.float32)
    w = sess.weight(f"wl:ex:{wtype}", wb, wtype, k, n)
    xb = sess.to_device(x)
    total = off + (m - 1) * ldy + n + 5
    fill = np.full(total, -7.25, np.float32)
    yb = sess.to_device(fill)
    bb = sess.to_device(bias)
    _lib.check(sess.matmul_ex(w, xb.ptr, m, yb.ptr, bb.ptr, ldy, off), "matmul_ex")
    got = yb.download(np.float32, total)
    ref = quant_matmul(oracle(), "orc", wb, wtype, x, n)
    mask = np.zeros(total, bool)
    for c in range(m):
        row = got[off + c * ldy: off + c * ldy + n]
        mask[off + c * ldy: off + c * ldy + n] = True
        assert row_rel_error(row, ref[c] + bias) <= TOL
    assert np.all(got[~mask] == np.float32(-7.25))


@pytest.mark.parametrize("m", [1, 33])
def test_quant_matmul_host_pointers(sess, m):
    """pixhip_quant_matmul with host activations and outputs (cpu_quant_matmul's
    argument order) gives the same bits as the device-resident path."""
    k, n = 768, 200
    x = activations(600 + m, m, k)
    wb = weights(610, n, k, Q5_K)
    y = np.full((m, n), np.nan, np.float32)
    _lib.check(sess.quant_matmul(wb.ctypes.data, Q5_K, x.ctypes.data, y.ctypes.data, n, m, k), "quant_matmul")
    y_dev = run_gpu(sess, "wl:host", wb, Q5_K, x, n)
    assert np.array_equal(y.view(np.uint32), y_dev.view(np.uint32))
    assert row_rel_error(y, quant_matmul(oracle(), "orc", wb, Q5_K, x, n)).max() <= TOL


@pytest.mark.parametrize("wtype", [Q5_K, Q6_K, Q8_0])
def test_host_operands_in_chunks(sess, wtype):
    """pixhip_matmul with pinned host input and output at a shape that runs in
    row chunks on three streams (copy in, quantize + GEMM, copy out): the same
    bits as the device-resident call, the quantized activations of every row
    left in the session (a MULTIPLY-only call afterwards matches too), and
    sampled rows against the oracle."""
    from gpu_helpers import Pinned
    m, k, n = 4000, 256, 10240  # chunks of 512 rows (the last 416): no split-K either way
    x = activations(620, m, k)
    wb = weights(621, n, k, wtype)
    key = f"wl:chunks:{wtype}"
    y_dev = run_gpu(sess, key, wb, wtype, x, n)
    w = sess.weight(key, wb, wtype, k, n)
    xp, yp = Pinned(sess, x), Pinned(sess, np.full((m, n), np.nan, np.float32))
    try:
        _lib.check(sess.matmul(w, xp.p.value, m, yp.p.value), "pixhip_matmul (pinned host operands)")
        y_host = yp.read(np.float32, (m, n))
    finally:
        xp.free()
        yp.free()
    assert np.array_equal(y_host.view(np.uint32), y_dev.view(np.uint32))
    yb = sess.alloc(m * n * 4)
    _lib.check(sess.matmul_stage(w, None, m, yb.ptr, _lib.STAGE_MULTIPLY), "MULTIPLY after the chunked call")
    y_again = yb.download(np.float32, m * n).reshape(m, n)
    yb.free()
    assert np.array_equal(y_again.view(np.uint32), y_dev.view(np.uint32))
    rows = np.array([0, 1, 511, 512, 1535, 2047, 3583, 3584, 3999])
    assert row_rel_error(y_host[rows], quant_matmul(oracle(), "orc", wb, wtype, x[rows], n)).max() <= TOL


def test_rejects_what_the_reference_rejects(sess):
    """cpu_quant_matmul returns false for zero sizes, a ragged inner dimension and
    other weight types (src/kernels_quant.cpp:373-375); so does the HIP path, with
    an argument error and nothing launched."""
    wb = weights(700, 4, 256, Q5_K)
    x = activations(701, 2, 256)
    y = np.zeros((2, 4), np.float32)
    q = lambda w_type, rows, cols, inner: sess.quant_matmul(wb.ctypes.data, w_type, x.ctypes.data, y.ctypes.data, rows,
                                                           cols, inner)
    assert q(Q5_K, 0, 2, 256) == _lib.ERR_ARGUMENT
    assert q(Q5_K, 4, 0, 256) == _lib.ERR_ARGUMENT
    assert q(Q5_K, 4, 2, 0) == _lib.ERR_ARGUMENT
    assert q(Q5_K, 4, 2, 128) == _lib.ERR_ARGUMENT
    assert q(Q8_0, 4, 2, 48) == _lib.ERR_ARGUMENT
    assert q(1, 4, 2, 256) == _lib.ERR_UNSUPPORTED  # MODEL_F16 stays on the reference's float path
    assert np.all(y == 0)
    assert q(Q5_K, 4, 2, 256) == _lib.OK


def test_operands_past_their_allocation():
    """pixhip_matmul_ex with an output region (y_offset + (M-1)*ldy + N floats),
    an input (M*K floats) or a bias (N floats) that runs past the end of its
    device allocation is rejected, and nothing is launched (a fresh session:
    every block is exactly its request rounded to 256 bytes)."""
    from gpu_helpers import new_session
    s = new_session()
    try:
        m, k, n = 4, 256, 64
        w = s.weight("span:q5", weights(910, n, k, Q5_K), Q5_K, k, n)
        xb, yb, bb = s.alloc(m * k * 4), s.alloc(m * n * 4), s.alloc(n * 4)
        xb.upload(activations(911, m, k))
        bb.upload(np.zeros(n, np.float32))
        mx = lambda x, y, bias, ldy=0, off=0: s.lib.pixhip_matmul_ex(s.handle, w, x, m, y, bias, ldy, off)
        assert mx(xb.ptr, yb.ptr, bb.ptr) == _lib.OK
        s.synchronize()
        assert mx(xb.ptr, yb.ptr, bb.ptr, 0, 1) == _lib.ERR_ARGUMENT        # y offset by one float
        assert mx(xb.ptr, yb.ptr, bb.ptr, n + 1) == _lib.ERR_ARGUMENT       # a wider row stride
        assert mx(xb.ptr + 4, yb.ptr, bb.ptr) == _lib.ERR_ARGUMENT          # input one float past the end
        assert mx(xb.ptr, yb.ptr, bb.ptr + 4) == _lib.ERR_ARGUMENT          # bias one float past the end
        for b in (xb, yb, bb):
            b.free()
    finally:
        s.close()
