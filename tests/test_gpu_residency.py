"""The device weight cache under pressure (VulkanState::weight / evict and
VulkanSession::prepare_stage, src/backend_vulkan.cpp:671-681, :742-758,
:1047-1057), through the C ABI:

- LRU eviction under a budget that holds one GEMM layout at a time: every call
  still matches the oracle, the cache stays within the budget, and a weight
  used again after its eviction gives bit-identical outputs;
- handles stay valid across eviction: a norm -> quantize followed by the GEMMs
  of two cold weights (the DiT FFN gate / up pattern) where building the second
  layout evicts the first;
- pixhip_prepare_stage flushes the cache without invalidating handles;
- residency: the Q5_K GEMM layout holds ~3.05x its GGUF bytes (the device GGUF
  copy is released once the layout is built);
- pixhip_quant_matmul is stateless: the same host buffer with new contents
  gives the new results, and nothing is left in the cache.
"""
import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import Q5_K, Q8_0, modulate_rows, norm_rows, oracle, quant_matmul, quantize
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu

K, N, M = 1024, 512, 40


@pytest.fixture()
def sess():
    from gpu_helpers import new_session
    s = new_session()
    yield s
    s.close()


def weights(seed, count, wtype=Q5_K):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        out.append(synth.pack_q5_K(wf) if wtype == Q5_K else quantize(oracle(), "orc", wf, "q8_0"))
    return out


def run(sess, w, xb, m=M):
    yb = sess.alloc(m * N * 4)
    _lib.check(sess.matmul(w, xb.ptr, m, yb.ptr), "pixhip_matmul")
    y = yb.download(np.float32, m * N).reshape(m, N)
    yb.free()
    return y


def gemm_layout_bytes():
    # hi + lo planes (K bytes each per row), d and dmin fp32 and eight fp16
    # minima per super-block, rows padded to the 128-feature tile
    npad = -(-N // 128) * 128
    return npad * K * 2 + (K // 256) * npad * (4 + 4 + 16)


def test_lru_eviction_under_budget(sess):
    print("eviction under a one-layout budget", flush=True)
    x = np.random.default_rng(1).standard_normal((M, K)).astype(np.float32)
    xb = sess.to_device(x)
    wb = weights(11, 3)
    budget = gemm_layout_bytes() + 2 * wb[0].nbytes + (1 << 16)
    sess.set_weight_budget(budget)
    hs = [sess.weight(f"evict:{i}", wb[i], Q5_K, K, N) for i in range(3)]
    first = {}
    for rnd in range(3):
        for i in (0, 1, 2, 1, 0):
            y = run(sess, hs[i], xb)
            entries, held = sess.cache_info()
            assert held <= budget, (held, budget)
            if i not in first:
                ref = quant_matmul(oracle(), "orc", wb[i], Q5_K, x, N)
                assert row_rel_error(y, ref).max() <= TOL
                first[i] = y
            else:  # rebuilt after eviction: the same bits
                assert np.array_equal(y.view(np.uint32), first[i].view(np.uint32)), (rnd, i)
    entries, held = sess.cache_info()
    assert entries < 3, "the budget holds one layout: older weights must have been evicted"
    xb.free()


def test_fused_pair_survives_eviction(sess):
    print("norm -> two cold GEMMs with eviction between them", flush=True)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((M, K)) * 3.0).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    mod = (0.2 * rng.standard_normal(K)).astype(np.float32)
    wg, wu = weights(21, 2)
    sess.set_weight_budget(gemm_layout_bytes() + 2 * wg.nbytes + (1 << 16))
    hg = sess.weight("fused:gate", wg, Q5_K, K, N)
    hu = sess.weight("fused:up", wu, Q5_K, K, N)
    xb, nb, mb = sess.to_device(x), sess.to_device(nw), sess.to_device(mod)
    ref_x = modulate_rows(oracle(), norm_rows(oracle(), "orc", x, nw, 1e-5, 0), mod)
    for rnd in range(2):
        _lib.check(sess.norm_quantize(Q5_K, xb.ptr, M, K, nb.ptr, 1e-5, 0, mb.ptr), "norm_quantize")
        outs = []
        for h in (hg, hu):
            yb = sess.alloc(M * N * 4)
            _lib.check(sess.matmul_stage(h, None, M, yb.ptr, _lib.STAGE_MULTIPLY), "multiply")
            outs.append(yb.download(np.float32, M * N).reshape(M, N))
            yb.free()
        for wbytes, y in zip((wg, wu), outs):
            assert row_rel_error(y, quant_matmul(oracle(), "orc", wbytes, Q5_K, ref_x, N)).max() <= TOL, rnd
    for b in (xb, nb, mb):
        b.free()


def test_prepare_stage_keeps_handles(sess):
    print("prepare_stage flush", flush=True)
    x = np.random.default_rng(2).standard_normal((M, K)).astype(np.float32)
    xb = sess.to_device(x)
    (wb,) = weights(31, 1)
    h = sess.weight("stage:w", wb, Q5_K, K, N)
    y0 = run(sess, h, xb)
    assert sess.prepare_stage(1 << 20, 1 << 20) == _lib.OK
    assert sess.cache_info() == (0, 0), "prepare_stage releases every weight's device memory"
    y1 = run(sess, h, xb)  # the same handle, rebuilt from its host bytes
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    xv = sess.to_device(x[:1])
    yv = run(sess, h, xv, 1)  # the matvec layout, from the same handle
    assert row_rel_error(yv, quant_matmul(oracle(), "orc", wb, Q5_K, x[:1], N)).max() <= TOL
    xb.free()
    xv.free()


def test_residency_of_the_q5_K_layout(sess):
    print("residency", flush=True)
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    xb = sess.to_device(x)
    (wb,) = weights(41, 1)
    h = sess.weight("res:w", wb, Q5_K, K, N)
    gguf, resident = sess.residency()
    assert (gguf, resident) == (wb.nbytes, -(-wb.nbytes // 256) * 256), "only the GGUF upload before first use"
    run(sess, h, xb)
    gguf, resident = sess.residency()
    ratio = resident / gguf
    print(f"Q5_K GEMM layout: {resident} device bytes for {gguf} GGUF bytes = {ratio:.3f}x", flush=True)
    assert resident == gemm_layout_bytes() and ratio <= 3.1
    xb.free()


def test_quant_matmul_is_stateless(sess):
    print("quant_matmul with a reused host buffer", flush=True)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((M, K)).astype(np.float32)
    buf = np.empty_like(weights(51, 1, Q8_0)[0])
    for seed in (61, 62):
        (wb,) = weights(seed, 1, Q8_0)
        buf[...] = wb  # same address, new contents
        y = np.empty((M, N), np.float32)
        _lib.check(sess.lib.pixhip_quant_matmul(sess.handle, buf.ctypes.data, Q8_0, x.ctypes.data, y.ctypes.data, N, M, K),
                   "pixhip_quant_matmul")
        assert row_rel_error(y, quant_matmul(oracle(), "orc", wb, Q8_0, x, N)).max() <= TOL, seed
        assert sess.cache_info() == (0, 0)
