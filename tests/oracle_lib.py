"""ctypes handles on the checkers: the oracle's C restatement
(oracle/liboracle.so) and, where it was built, the reference's own CPU path
(oracle/_ref/libpixref.so).  Test infrastructure only."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libpixref.so")

Q8_0, Q5_K, Q6_K = 8, 13, 14
Q8_0_BYTES, Q8_K_BYTES = 34, 292

_vp, _i64, _int, _sz, _u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint32

_oracle = None
_ref = None


def load_oracle(path):
    """ctypes handle on an oracle build at `path` (the default build, or a
    copy compiled with ORC_MUTANT by the tests that plant mistakes)."""
    lib = ctypes.CDLL(path)
    sig = {
        "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_nearest_int_fused": (_int, [ctypes.c_float, ctypes.c_float]),
        "orc_quantize_q8_0": (None, [_vp, _vp, _i64]),
        "orc_quantize_q8_K": (None, [_vp, _vp, _i64]),
        "orc_dot_q8_0": (ctypes.c_float, [_int, _vp, _vp]),
        "orc_dot_q5_K": (ctypes.c_float, [_int, _vp, _vp]),
        "orc_dot_q6_K": (ctypes.c_float, [_int, _vp, _vp]),
        "orc_block_sums_q8_0": (ctypes.c_int32, [_vp, _vp]),
        "orc_superblock_sums_q5_K": (None, [_vp, _vp, _vp, _vp]),
        "orc_superblock_sum_q6_K": (ctypes.c_int32, [_vp, _vp]),
        "orc_quant_matmul": (_int, [_vp, _u32, _vp, _vp, _sz, _sz, _sz, _int]),
        "orc_decode": (None, [_vp, _u32, _sz, _vp]),
        "orc_row_bytes": (ctypes.c_uint64, [ctypes.c_uint64, _u32]),
        "orc_norm_rows": (None, [_vp, _sz, _sz, _vp, ctypes.c_float, _int, _vp]),
        "orc_modulate_rows": (None, [_vp, _sz, _sz, _vp]),
        "orc_silu_gate": (None, [_vp, _vp, _sz, _vp]),
        "orc_gelu": (None, [_vp, _sz, _int]),
        "orc_bias": (None, [_vp, _sz, _sz, _vp]),
        "orc_add": (None, [_vp, _vp, _sz]),
        "orc_rope": (None, [_vp, _sz, _sz, _sz, _vp, _vp, _int]),
        "orc_attention": (_int, [_vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _vp]),
        "orc_channel_op": (None, [_int, _vp, _vp, _vp, _sz, _sz, ctypes.c_float, ctypes.c_float]),
        "orc_qwen_modulate": (_int, [_vp, _sz, _sz, _vp, _sz, _sz, _sz, _vp]),
        "orc_l2norm": (_int, [_vp, _sz, _sz, _vp, ctypes.c_float, _vp]),
        "orc_groupnorm": (None, [_vp, _sz, _sz, _vp, _vp, _vp]),
        "orc_decode_f32": (None, [_vp, _u32, _sz, _vp]),
        "orc_rows": (_int, [_vp, _sz, _vp, _sz, _sz, _vp, _sz, _int]),
        "orc_layout": (None, [_int, _vp, _vp, _sz, _sz, _sz, _sz]),
        "orc_shortcut": (_int, [_vp, _sz, _sz, _sz, _sz, _sz, _int, _int, _vp]),
        "orc_conv2d": (_int, [_vp, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-C", ORACLE_DIR, "oracle"], check=True, capture_output=True)
        _oracle = load_oracle(ORACLE_SO)
    return _oracle


def reference():
    """The compiled reference (None when oracle/_ref was not built here)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            return None
        lib = ctypes.CDLL(REF_SO)
        sig = {
            "ref_quantize_q8_0": (None, [_vp, _vp, _i64]),
            "ref_quantize_q8_K": (None, [_vp, _vp, _i64]),
            "ref_dot_q8_0": (ctypes.c_float, [_int, _vp, _vp]),
            "ref_dot_q5_K": (ctypes.c_float, [_int, _vp, _vp]),
            "ref_dot_q6_K": (ctypes.c_float, [_int, _vp, _vp]),
            "ref_nearest_int": (_int, [ctypes.c_float]),
            "ref_quant_matmul": (_int, [_vp, _u32, _vp, _vp, _sz, _sz, _sz]),
            "ref_set_threads": (None, [_sz]),
            "ref_thread_count": (_sz, []),
            "ref_decode": (None, [_vp, _u32, _sz, _vp]),
            "ref_half_float": (ctypes.c_float, [ctypes.c_uint16]),
            "ref_row_bytes": (ctypes.c_uint64, [ctypes.c_uint64, _u32]),
            "ref_norm_rows": (_int, [_vp, _sz, _sz, _vp, ctypes.c_float, _int, _vp]),
            "ref_silu_gate": (None, [_vp, _vp, _sz, _vp]),
            "ref_gelu": (None, [_vp, _sz, _int]),
            "ref_bias": (None, [_vp, _sz, _sz, _vp]),
            "ref_add": (None, [_vp, _vp, _sz]),
            "ref_rope": (None, [_vp, _sz, _sz, _sz, _vp, _vp, _int]),
            "ref_attention": (_int, [_vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _int, _vp]),
            "ref_attention_ranges": (_int, [_vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _vp]),
            "ref_l2norm": (_int, [_vp, _sz, _sz, _vp, ctypes.c_float, _vp]),
            "ref_groupnorm": (_int, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "ref_slice": (_int, [_vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
            "ref_gather": (_int, [_vp, _sz, _sz, _vp, _sz, _vp]),
            "ref_scatter": (_int, [_vp, _sz, _sz, _vp, _vp, _sz]),
            "ref_upsample": (_int, [_vp, _sz, _sz, _sz, _vp]),
            "ref_shortcut": (_sz, [_vp, _sz, _sz, _sz, _sz, _sz, _int, _int, _vp, _sz]),
            "ref_model_probe": (_sz, [ctypes.c_char_p, _int, ctypes.c_char_p, _sz]),
            "ref_conv": (_sz, [_vp, _sz, _sz, _sz, _vp, _u32, _sz, _sz, _sz, _vp, _int, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _ref = lib
    return _ref


def default_threads():
    """Host threads for the oracle and the compiled reference: every core in
    this process's affinity mask (the reference's default, src/tensor.cpp:97-101)."""
    return max(1, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1))


def ptr(a):
    return a.ctypes.data


# ---- numpy conveniences over either library (prefix "orc" or "ref") ----

def quantize(lib, prefix, x, kind):
    """Rows of x (float32 [R, K]) -> reference block bytes uint8 [R, K/QK*B]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    if kind == "q8_0":
        out = np.zeros((rows, k // 32 * Q8_0_BYTES), dtype=np.uint8)
        fn = getattr(lib, f"{prefix}_quantize_q8_0")
    else:
        out = np.zeros((rows, k // 256 * Q8_K_BYTES), dtype=np.uint8)
        fn = getattr(lib, f"{prefix}_quantize_q8_K")
    for r in range(rows):
        fn(ptr(x[r]), ptr(out[r]), k)
    return out


def dot(lib, prefix, wtype, wrow, arow, k):
    name = {Q8_0: "dot_q8_0", Q5_K: "dot_q5_K", Q6_K: "dot_q6_K"}[wtype]
    wrow = np.ascontiguousarray(wrow)
    arow = np.ascontiguousarray(arow)
    return getattr(lib, f"{prefix}_{name}")(k, ptr(wrow), ptr(arow))


def quant_matmul(lib, prefix, w, wtype, x, rows, threads=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    cols, k = x.shape
    y = np.full((cols, rows), np.nan, dtype=np.float32)
    if prefix == "orc":
        ok = lib.orc_quant_matmul(ptr(w), wtype, ptr(x), ptr(y), rows, cols, k, threads or default_threads())
    else:
        ok = lib.ref_quant_matmul(ptr(w), wtype, ptr(x), ptr(y), rows, cols, k)
    if not ok:
        raise ValueError("quant_matmul rejected its arguments")
    return y


def norm_rows(lib, prefix, x, weight, eps, centered):
    """tensor_norm over the rows of x (float32 [R, C]); weight None = empty."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, ch = x.shape
    out = np.full_like(x, np.nan)
    wp = None if weight is None else ptr(np.ascontiguousarray(weight, dtype=np.float32))
    r = getattr(lib, f"{prefix}_norm_rows")(ptr(x), rows, ch, wp, eps, int(centered), ptr(out))
    if prefix == "ref" and not r:
        raise ValueError("tensor_norm returned an empty tensor")
    return out


def modulate_rows(lib, x, scale):
    """z_modulate: x * (1 + scale[c]), through the oracle."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    lib.orc_modulate_rows(ptr(x), x.shape[0], x.shape[1], ptr(np.ascontiguousarray(scale, dtype=np.float32)))
    return x


def silu_gate(lib, prefix, gate, up):
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.full_like(g, np.nan)
    getattr(lib, f"{prefix}_silu_gate")(ptr(g), ptr(u), g.size, ptr(out))
    return out


def gelu(lib, prefix, x, approximate):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    getattr(lib, f"{prefix}_gelu")(ptr(y), y.size, int(approximate))
    return y


def bias(lib, prefix, x, b):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    getattr(lib, f"{prefix}_bias")(ptr(y), y.shape[0], y.shape[1], ptr(np.ascontiguousarray(b, dtype=np.float32)))
    return y


def add(lib, prefix, x, other):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    getattr(lib, f"{prefix}_add")(ptr(y), ptr(np.ascontiguousarray(other, dtype=np.float32)), y.size)
    return y


def rope(lib, prefix, x, heads, cosine, sine, interleaved):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    getattr(lib, f"{prefix}_rope")(ptr(y), y.shape[0], y.shape[1], heads, ptr(np.ascontiguousarray(cosine, dtype=np.float32)),
                                   ptr(np.ascontiguousarray(sine, dtype=np.float32)), int(interleaved))
    return y


def attention(lib, prefix, q, k, v, heads, kv_heads, ranges=None, query_offset=0, causal=False):
    """tensor_attention through either library: `ranges` [(query_begin,
    query_end, key_end, causal)] selects the ranges form; without it the causal
    form (the reference's own entry for prefix "ref", the one range {0, rows,
    keys, causal} for the oracle).  None when the library rejects the call."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    rows, channels = q.shape
    keys = k.shape[0]
    out = np.zeros((rows, channels), np.float32)
    if ranges is None and prefix == "ref":
        ok = lib.ref_attention(ptr(q), rows, ptr(k), ptr(v), keys, heads, kv_heads, channels, int(causal), ptr(out))
        return out if ok else None
    if ranges is None:
        ranges = [(0, rows, keys, int(causal))]
    rg = np.ascontiguousarray(np.array(ranges, dtype=np.uint64).reshape(-1, 4))
    fn = lib.ref_attention_ranges if prefix == "ref" else lib.orc_attention
    ok = fn(ptr(q), rows, ptr(k), ptr(v), keys, heads, kv_heads, channels, ptr(rg), len(rg), query_offset, ptr(out))
    return out if ok else None


def decode(lib, w, wtype, count):
    out = np.zeros(count, dtype=np.float64)
    lib.orc_decode(ptr(np.ascontiguousarray(w)), wtype, count, ptr(out))
    return out


def q8_0_blocks(blocks):
    """Split Q8_0 block bytes [..., nb*34] -> (d fp16 bits [..., nb], qs int8 [..., nb, 32])."""
    b = blocks.reshape(*blocks.shape[:-1], -1, Q8_0_BYTES)
    d = b[..., 0:2].copy().view(np.uint16)[..., 0]
    qs = b[..., 2:].view(np.int8)
    return d, qs


def q8_K_blocks(blocks):
    """Split Q8_K block bytes -> (d float32 [..., nb], qs int8 [..., nb, 256], bsums int16 [..., nb, 16])."""
    b = blocks.reshape(*blocks.shape[:-1], -1, Q8_K_BYTES)
    d = b[..., 0:4].copy().view(np.float32)[..., 0]
    qs = b[..., 4:260].view(np.int8)
    bs = b[..., 260:292].copy().view(np.int16)
    return d, qs, bs


# ---- the rest of the backend op surface ----

F32, F16, BF16 = 0, 1, 30
OP_MODULATE, OP_RESIDUAL, OP_AFFINE, OP_EULER = 8, 9, 10, 26
OP_PATCH, OP_UNPATCH, OP_UPSAMPLE = 15, 16, 17


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def channel_op(lib, op, x, other=None, p=None, scale=0.0, bias=0.0):
    """orc_channel_op on a copy of x; `p` is the modulation slice [channels]."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    o = None if other is None else _f32(other)
    pp = None if p is None else _f32(p)
    lib.orc_channel_op(op, ptr(y), None if o is None else ptr(o), None if pp is None else ptr(pp), y.shape[0], y.shape[1], scale, bias)
    return y


def qwen_modulate(lib, x, parameters, target_begin, part, residual=None):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    pm = _f32(parameters)
    r = None if residual is None else _f32(residual)
    ok = lib.orc_qwen_modulate(ptr(y), y.shape[0], y.shape[1], ptr(pm), pm.shape[1], target_begin, part, None if r is None else ptr(r))
    return y if ok else None


def l2norm(lib, prefix, x, weight, eps):
    x = _f32(x)
    out = np.full_like(x, np.nan)
    w = None if weight is None else _f32(weight)
    ok = getattr(lib, f"{prefix}_l2norm")(ptr(x), x.shape[0], x.shape[1], None if w is None else ptr(w), eps, ptr(out))
    return out if ok else None


def groupnorm(lib, prefix, x, weight, b):
    x, w, b = _f32(x), _f32(weight), _f32(b)
    out = np.full_like(x, np.nan)
    ok = getattr(lib, f"{prefix}_groupnorm")(ptr(x), x.shape[0], x.shape[1], ptr(w), ptr(b), ptr(out))
    return out if (ok is None or ok) else None


def decode_f32(lib, prefix, data, wtype, count):
    """cpu_decode (prefix "ref") or its restatement ("orc") of `count` values."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.full(count, np.nan, np.float32)
    getattr(lib, "orc_decode_f32" if prefix == "orc" else "ref_decode")(ptr(data), wtype, count, ptr(out))
    return out


def gather(lib, prefix, x, rows):
    x = _f32(x)
    r = np.ascontiguousarray(rows, dtype=np.uint64)
    out = np.full((len(r), x.shape[1]), np.nan, np.float32)
    if prefix == "ref":
        ok = lib.ref_gather(ptr(x), x.shape[0], x.shape[1], ptr(r), len(r), ptr(out))
    else:
        ok = lib.orc_rows(ptr(x), x.shape[0], ptr(out), len(r), x.shape[1], ptr(r), len(r), 0)
    return out if ok else None


def scatter(lib, prefix, destination, source, rows):
    d = np.array(destination, dtype=np.float32, copy=True, order="C")
    src = _f32(source)
    r = np.ascontiguousarray(rows, dtype=np.uint64)
    if prefix == "ref":
        ok = lib.ref_scatter(ptr(d), d.shape[0], d.shape[1], ptr(src), ptr(r), len(r))
    else:
        ok = lib.orc_rows(ptr(src), src.shape[0], ptr(d), d.shape[0], d.shape[1], ptr(r), len(r), 1)
    return d if ok else None


def layout(lib, op, x, width, height, channels, patch=1):
    """orc_layout: op 15 pixels -> tokens, 16 tokens -> pixels, 17 upsample;
    width, height and channels are the pixel image's."""
    x = _f32(x)
    if op == OP_UPSAMPLE:
        out = np.full((4 * width * height, channels), np.nan, np.float32)
    elif op == OP_PATCH:
        out = np.full((width * height // (patch * patch), patch * patch * channels), np.nan, np.float32)
    else:
        out = np.full((width * height, channels), np.nan, np.float32)
    lib.orc_layout(op, ptr(x), ptr(out), width, height, channels, patch)
    return out


def upsample_ref(lib, x, width, height):
    x = _f32(x)
    out = np.full((4 * width * height, x.shape[1]), np.nan, np.float32)
    return out if lib.ref_upsample(ptr(x), width, height, x.shape[1], ptr(out)) else None


def shortcut_out_pixels(width, height, up, spatial):
    side = 2 if spatial else 1
    return (width * side) * (height * side) if up else (width // side) * (height // side)


def shortcut(lib, prefix, x, width, height, channels, temporal, up, spatial):
    x = _f32(x)
    out = np.full((shortcut_out_pixels(width, height, up, spatial), channels), np.nan, np.float32)
    if prefix == "ref":
        n = lib.ref_shortcut(ptr(x), width, height, x.shape[1], channels, temporal, int(up), int(spatial), ptr(out), out.size)
        return out if n == out.size else None
    ok = lib.orc_shortcut(ptr(x), width, height, x.shape[1], channels, temporal, int(up), int(spatial), ptr(out))
    return out if ok else None


def conv_out_size(width, height, kx, ky, geometry):
    sx, sy, left, right, top, bottom = geometry
    return (width + left + right - kx) // sx + 1, (height + top + bottom - ky) // sy + 1


def same_geometry(kx, ky):
    """tensor_conv's first form as a geometry: stride 1, the kernel centred."""
    return (1, 1, kx // 2, kx - 1 - kx // 2, ky // 2, ky - 1 - ky // 2)


def conv2d(lib, x, width, height, weight, kx, ky, bias=None, geometry=None):
    """orc_conv2d: x [width*height][cin], weight fp32 [cout][cin*ky*kx] (the
    GGUF [kx, ky, cin, cout] order), geometry (sx, sy, left, right, top,
    bottom) or None for the first form."""
    x = _f32(x)
    w = _f32(weight)
    cout = w.shape[0]
    g = geometry or same_geometry(kx, ky)
    ow, oh = conv_out_size(width, height, kx, ky, g)
    out = np.full((ow * oh, cout), np.nan, np.float32)
    b = None if bias is None else _f32(bias)
    ok = lib.orc_conv2d(ptr(x), width, height, x.shape[1], ptr(w), kx, ky, cout, None if b is None else ptr(b), *g, ptr(out))
    return out if ok else None


def conv2d_ref(ref, x, width, height, wbytes, wtype, kx, ky, cin, cout, bias=None, geometry=None):
    """The reference's tensor_conv (first form when geometry is None, then
    with the bias it requires), through oracle/_ref."""
    x = _f32(x)
    wb = np.ascontiguousarray(wbytes, dtype=np.uint8)
    g = geometry or same_geometry(kx, ky)
    ow, oh = conv_out_size(width, height, kx, ky, g)
    out = np.full((ow * oh, cout), np.nan, np.float32)
    b = None if bias is None else _f32(bias)
    n = ref.ref_conv(ptr(x), width, height, cin, ptr(wb), wtype, kx, ky, cout, None if b is None else ptr(b), 0 if geometry is None else 1,
                     *g, ptr(out), out.size)
    return out if n == out.size else None
