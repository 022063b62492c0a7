"""The C++ shim (pixelina_amd/host/backend_hip.h) driven the way the
reference's model code drives its Vulkan backend, by pixelina_amd/shim_check
(built with the library): a HipSession made current on the thread, activations
in HipAllocator vectors (pinned host memory), weights reached through a
model-file / weight pair shaped like PixModelFile / PixWeight, and the calls of
tensor_linear (hip_matmul), of the DiT block's FFN (hip_norm_multiply for
the gate and up linears, hip_silu_gate_multiply for the down linear), and of
tensor_rope / tensor_bias (hip_rope, hip_pointwise) with their tables in
pageable std::vector memory, which the library stages to the device, and of
tensor_attention, tensor_l2norm, tensor_groupnorm and tensor_gather.

Against the oracle: the normalized input bit-exact; the SiLU product within 4
ulps (the reference's glibc expf is not correctly rounded; this one is); every
linear within max|y - r| / max|r| <= 1e-4 per token row.
"""
import os
import subprocess

import numpy as np
import pytest

from gpu_helpers import TOL, row_rel_error
from oracle_lib import (Q5_K, Q8_0, attention, bias, groupnorm, l2norm, modulate_rows, norm_rows, oracle, quant_matmul, quantize, rope,
                        silu_gate)
from pixelina_amd import synth

pytestmark = pytest.mark.gpu

SHIM_CHECK = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "pixelina_amd", "shim_check")


def test_shim_matmul_norm_and_gate(tmp_path):
    assert os.path.exists(SHIM_CHECK), "pixelina_amd/shim_check is not built (run __graft_entry__.build())"
    rng = np.random.default_rng(77)
    m, k, n, f = 37, 512, 300, 768
    o = oracle()
    w1 = synth.pack_q5_K((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w2 = synth.pack_q5_K((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wd = quantize(o, "orc", (rng.standard_normal((k, f)) * 0.02).astype(np.float32), "q8_0")
    x = (rng.standard_normal((m, k)) * rng.choice([0.1, 1.0, 10.0], (m, 1))).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    mod = (0.2 * rng.standard_normal(k)).astype(np.float32)
    g = (rng.standard_normal((m, f)) * 3.0).astype(np.float32)
    u = rng.standard_normal((m, f)).astype(np.float32)
    th = rng.standard_normal((m, 32)) * 3.0
    cos, sin = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
    bvec = rng.standard_normal(n).astype(np.float32)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(src, "wb") as fh:
        fh.write(np.array([Q5_K, Q8_0], np.uint32).tobytes())
        fh.write(np.array([m, k, n, f], np.uint64).tobytes())
        for wb in (w1, w2, wd):
            fh.write(np.array([wb.nbytes], np.uint64).tobytes())
            fh.write(np.ascontiguousarray(wb).tobytes())
        for a in (x, nw, mod, g, u, cos, sin, bvec):
            fh.write(np.ascontiguousarray(a, np.float32).tobytes())
    print("running shim_check", flush=True)
    proc = subprocess.run([SHIM_CHECK, str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    out = np.fromfile(dst, np.float32)
    sizes = [m * n, m * n, m * n, m * k, m * k, m * f, m * k, m * n, m * k, m * k, m * k, m * k, m * k]
    assert out.size == sum(sizes)
    y, y1, y2, normalized, d, gated, roped, biased, att, att2, l2, gn, gathered = np.split(out, np.cumsum(sizes)[:-1])

    # hip_l2norm / hip_groupnorm / hip_rows with pageable vectors: bit-exact
    assert np.array_equal(l2.reshape(m, k).view(np.uint32), l2norm(o, "orc", x, nw, 1e-12).view(np.uint32))
    assert np.array_equal(gn.reshape(m, k).view(np.uint32), groupnorm(o, "orc", x, nw, mod).view(np.uint32))
    assert np.array_equal(gathered.reshape(m, k), x[::-1])

    # hip_attention, both forms, against the oracle's tensor_attention
    h = k // 64
    for what, got, ranges in (("hip_attention (causal)", att, [(0, m, m, 1)]),
                              ("hip_attention (ranges)", att2, [(0, m // 2, m, 0), (m // 2, m, m, 1)])):
        want = attention(o, "orc", x, x, x, h, h, ranges)
        err = row_rel_error(got.reshape(m, k), want).max()
        print(f"{what}: rel={err:.2e}", flush=True)
        assert err <= TOL, what

    # hip_rope / hip_pointwise(BIAS) were handed pageable std::vector tables:
    # bit-exact against the oracle's tensor_rope / tensor_bias
    assert np.array_equal(roped.reshape(m, k).view(np.uint32), rope(o, "orc", x, k // 64, cos, sin, 0).view(np.uint32))
    assert np.array_equal(biased.reshape(m, n).view(np.uint32), bias(o, "orc", y.reshape(m, n), bvec).view(np.uint32))

    ref_norm = modulate_rows(o, norm_rows(o, "orc", x, nw, 1e-5, 0), mod)
    assert np.array_equal(normalized.view(np.uint32), ref_norm.reshape(-1).view(np.uint32))
    ref_gated = silu_gate(o, "orc", g, u)
    a, b = gated.reshape(m, f), ref_gated
    assert (np.abs(a.astype(np.float64) - b) <= 4 * np.spacing(np.maximum(np.abs(a), np.abs(b)))).all()
    checks = [("hip_matmul", y, quant_matmul(o, "orc", w1, Q5_K, x, n)),
              ("norm -> gate linear", y1, quant_matmul(o, "orc", w1, Q5_K, ref_norm, n)),
              ("norm -> up linear", y2, quant_matmul(o, "orc", w2, Q5_K, ref_norm, n)),
              ("silu*gate -> down linear", d, quant_matmul(o, "orc", wd, Q8_0, ref_gated, k))]
    for what, got, want in checks:
        err = row_rel_error(got.reshape(want.shape), want).max()
        print(f"{what}: rel={err:.2e}", flush=True)
        assert err <= TOL, what
