"""Weights reached through the model file reader, as the reference's model code
reaches them (PixModelFile + VulkanState::weight, src/model.cpp:138-243,
src/backend_vulkan.cpp:742-758): a GGUF file written here is opened with
pixhip_model_open, each 2-D quantized tensor becomes a cache entry with
pixhip_model_weight (key file:name:offset:bytes over the mapping's bytes), and
the GEMM (M = 33) and the matvec (M = 1) through those handles match the
oracle's cpu_quant_matmul on the tensors' bytes (max |y - r| / max |r| per row
<= 1e-4).  A second lookup returns the same handle; 1-D and absent tensors are
rejected."""
import ctypes

import numpy as np
import pytest

import model_files as mf
from gpu_helpers import TOL, new_session, row_rel_error
from oracle_lib import Q5_K, Q6_K, Q8_0, oracle, quant_matmul, quantize
from pixelina_amd import _lib, synth

pytestmark = pytest.mark.gpu


def test_weights_from_a_model_file(tmp_path):
    rng = np.random.default_rng(91)
    o = oracle()
    w = {
        "blk.0.attn_q.weight": (Q5_K, 512, 300, synth.pack_q5_K((rng.standard_normal((300, 512)) * 0.02).astype(np.float32))),
        "blk.0.ffn_down.weight": (Q8_0, 768, 64, quantize(o, "orc", (rng.standard_normal((64, 768)) * 0.02).astype(np.float32), "q8_0")),
        "output.weight": (Q6_K, 256, 130, synth.pack_q6_K((rng.standard_normal((130, 256)) * 0.02).astype(np.float32))),
    }
    tensors = [(name, t, [k, n], np.ascontiguousarray(b).tobytes()) for name, (t, k, n, b) in w.items()]
    tensors.append(("output_norm.weight", 0, [512], np.ones(512, np.float32).tobytes()))
    path = tmp_path / "model.gguf"
    path.write_bytes(mf.gguf([("general.architecture", mf.STRING, "test")], tensors))
    sess = new_session()
    lib = mf.bind(sess.lib)
    lib.pixhip_model_weight.restype = ctypes.c_int
    lib.pixhip_model_weight.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
    model = ctypes.c_void_p()
    assert lib.pixhip_model_open(str(path).encode(), 0, ctypes.byref(model)) == 0
    try:
        for name, (t, k, n, blocks) in w.items():
            h, h2 = ctypes.c_void_p(), ctypes.c_void_p()
            _lib.check(lib.pixhip_model_weight(sess.handle, model, name.encode(), ctypes.byref(h)), "pixhip_model_weight")
            _lib.check(lib.pixhip_model_weight(sess.handle, model, name.encode(), ctypes.byref(h2)), "pixhip_model_weight")
            assert h.value == h2.value, name
            for m in (33, 1):
                x = rng.standard_normal((m, k)).astype(np.float32)
                xb, yb = sess.to_device(x), sess.alloc(m * n * 4)
                _lib.check(sess.matmul(h.value, xb.ptr, m, yb.ptr), "matmul")
                y = yb.download(np.float32, m * n).reshape(m, n)
                xb.free()
                yb.free()
                err = row_rel_error(y, quant_matmul(o, "orc", blocks, t, x, n)).max()
                print(f"{name} M={m}: rel={err:.2e}", flush=True)
                assert err <= TOL, (name, m)
        h = ctypes.c_void_p()
        assert lib.pixhip_model_weight(sess.handle, model, b"output_norm.weight", ctypes.byref(h)) == _lib.ERR_ARGUMENT
        assert lib.pixhip_model_weight(sess.handle, model, b"absent", ctypes.byref(h)) == _lib.ERR_ARGUMENT
        entries = ctypes.c_uint64()
        _lib.check(sess.lib.pixhip_weight_cache_info(sess.handle, ctypes.byref(entries), None), "cache info")
        assert entries.value == 3
    finally:
        sess.synchronize()
        sess.close()
        lib.pixhip_model_close(model)
