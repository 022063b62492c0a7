"""Host-side checks that need no GPU: the C-ABI library loads and exports every
entry point that include/pixhip.h declares (and the ctypes table matches the
header), argument errors come back as status codes without touching a device,
the C++ shim is linked in, and the seeded input generators are what they say."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from pixelina_amd import _lib, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pixhip.h")


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(pixhip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIBRARY):
        from pixelina_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("pixhip_session_create", "pixhip_matmul", "pixhip_matmul_ex", "pixhip_quant_matmul",
                     "pixhip_quantize_q8_0", "pixhip_quantize_q8_K", "pixhip_weight_get", "pixhip_allocate",
                     "pixhip_free", "pixhip_synchronize", "pixhip_prepare_stage", "pixhip_block_sums"):
        assert required in names


def test_library_exports_every_declared_function(lib):
    raw = ctypes.CDLL(_lib.LIBRARY)
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIBRARY], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pixhip_\w+)", out))
    assert set(declared_functions()) <= exported


def test_ctypes_table_matches_header():
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_cpp_shim_is_linked(lib):
    shim_check = os.path.join(os.path.dirname(_lib.LIBRARY), "shim_check")
    assert os.path.exists(shim_check), "the shim driver is built with the library"
    out = subprocess.run(["nm", "-DC", "--defined-only", _lib.LIBRARY], capture_output=True, text=True, check=True).stdout
    for sym in ("HipSession::initialize(int)", "hip_active_state()", "hip_synchronize()", "hip_matmul_weight(",
                "hip_allocate(", "hip_free(", "hip_norm_multiply(", "hip_silu_gate_multiply(", "hip_pointwise(", "hip_rope("):
        assert sym in out, sym


def test_version_and_error_text(lib):
    assert lib.pixhip_version() == 100
    assert isinstance(lib.pixhip_last_error(), bytes)


def test_session_create_rejects_bad_arguments(lib):
    assert lib.pixhip_session_create(0, None) == _lib.ERR_ARGUMENT
    h = ctypes.c_void_p(1234)
    rc = lib.pixhip_session_create(9999, ctypes.byref(h))
    # no device at all (this container) or no such device index (a GPU box)
    assert rc in (_lib.ERR_DEVICE, _lib.ERR_ARGUMENT)
    assert not h.value
    assert lib.pixhip_last_error()


def test_entry_points_without_a_session(lib):
    state = _lib.ERR_STATE
    assert lib.pixhip_matmul(None, None, None, 1, None) == state
    assert lib.pixhip_matmul_ex(None, None, None, 1, None, None, 0, 0) == state
    assert lib.pixhip_quantize_q8_0(None, None, None, 1, 32) == state
    assert lib.pixhip_quantize_q8_K(None, None, None, 1, 256) == state
    assert lib.pixhip_norm_quantize(None, 13, None, 1, 256, None, 1e-5, 0, None, None, None) == state
    assert lib.pixhip_silu_gate_quantize(None, 8, None, None, 1, 32, None, None) == state
    assert lib.pixhip_pointwise(None, 2, None, None, 1, 4) == state
    assert lib.pixhip_rope(None, None, 1, 8, 1, None, None, 0) == state
    assert lib.pixhip_synchronize(None) == state
    assert lib.pixhip_allocate(None, 16) is None
    lib.pixhip_free(None, None)  # no-op
    lib.pixhip_session_destroy(None)  # no-op
    assert b"session" in lib.pixhip_last_error()
    t, k, n = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
    assert lib.pixhip_weight_shape(None, ctypes.byref(t), ctypes.byref(k), ctypes.byref(n)) == _lib.ERR_ARGUMENT


# ---- seeded inputs ----

def test_splitmix_matches_the_published_sequence():
    # SplitMix64 seeded with 0: first output 0xe220a8397b1dcdaf, second 0x6e789e6aa1b965f4
    u = synth.splitmix_uniform(0, 2)
    want = [((v >> 11) + 0.5) * 2.0 ** -53 for v in (0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4)]
    assert u.tolist() == want


def test_normal_generator_statistics_and_determinism():
    a = synth.normal(synth.SEED_ACTIVATIONS, (64, 1024))
    b = synth.normal(synth.SEED_ACTIVATIONS, (64, 1024))
    assert a.dtype == np.float32 and np.array_equal(a, b)
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    w = synth.normal(synth.SEED_WEIGHTS, (1000,), std=0.02)
    assert abs(float(w.std()) - 0.02) < 0.002


def test_outlier_channels_are_one_percent():
    ch = synth.outlier_channels(3840)
    assert len(ch) == 38 and len(set(ch.tolist())) == 38 and ch.max() < 3840


@pytest.mark.parametrize("wtype,inner", [(_lib.Q8_0, 3584), (_lib.Q5_K, 3840), (_lib.Q6_K, 4096)])
def test_row_bytes(wtype, inner):
    from oracle_lib import oracle
    assert synth.row_bytes(inner, wtype) == oracle().orc_row_bytes(inner, wtype)
