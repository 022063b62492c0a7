"""Writers of GGUF (version 3) and safetensors files for the model reader's
tests, from the formats' published layouts (GGUF: magic, version, tensor and
metadata counts, typed key/value pairs, tensor infos, data aligned to
general.alignment; safetensors: an 8-byte header length, a JSON header of
dtype / shape / data_offsets, the data), and the reader's description in the
text form the reference harness prints (oracle/ref_harness.cpp
ref_model_probe)."""
import ctypes
import json
import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32T, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32T: "<f", BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 13: (256, 176), 14: (256, 210)}


def tensor_bytes(wtype, shape):
    block, size = BLOCK[wtype]
    count = shape[0] // block
    for d in shape[1:]:
        count *= d
    return count * size


def _string(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_PACK[vtype], v)


def gguf(metadata, tensors, alignment=None, version=3, pad_to=None, layout=False):
    """metadata: [(key, type, value)] (arrays as (element type, [values]));
    tensors: [(name, ggml type, shape (GGML order), data bytes or None)];
    returns the file's bytes (with layout=True also the data base offset and
    each tensor's offset from it).  Data are placed in order, each at the next
    multiple of the alignment."""
    # data laid out at the declared alignment when it is a power of two (32 otherwise)
    align = alignment if alignment and alignment & (alignment - 1) == 0 else 32
    kv = list(metadata)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vtype, v in kv:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offset, blobs = 0, []
    for name, wtype, shape, data in tensors:
        nbytes = tensor_bytes(wtype, shape) if wtype in BLOCK else 64
        head += _string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", wtype, offset)
        blob = data if data is not None else bytes((i * 7 + len(name)) & 255 for i in range(nbytes))
        blobs.append((offset, blob))
        offset += (len(blob) + align - 1) // align * align
    base = (len(head) + align - 1) // align * align
    out = bytearray(head + b"\0" * (base - len(head)))
    for off, blob in blobs:
        if len(out) < base + off:
            out += b"\0" * (base + off - len(out))
        out += blob
    if pad_to and len(out) < pad_to:
        out += b"\0" * (pad_to - len(out))
    return (bytes(out), base, [off for off, _ in blobs]) if layout else bytes(out)


def safetensors(tensors, metadata=None, header_pad=0):
    """tensors: [(name, dtype "F32" / "F16" / "BF16", shape (row-major, as the
    format stores it), data bytes)]."""
    header, offset, blobs = {}, 0, []
    for name, dtype, shape, data in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(data)]}
        blobs.append(data)
        offset += len(data)
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header).encode() + b" " * header_pad
    return struct.pack("<Q", len(text)) + text + b"".join(blobs)


# ---- the reader's description, as ref_model_probe prints it ----

CODES = {0: 0, -6: 1, -7: 2}  # pixhip_model_open's status -> MODEL_ERROR_*


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_length", ctypes.c_uint64), ("type", ctypes.c_uint32), ("rank", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 5), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


def bind(lib):
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    sig = {
        "pixhip_model_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(vp)]),
        "pixhip_model_close": (None, [vp]),
        "pixhip_model_data": (vp, [vp, ctypes.POINTER(ctypes.c_uint64)]),
        "pixhip_model_tensor_count": (ctypes.c_uint64, [vp]),
        "pixhip_model_tensor_at": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.POINTER(TensorInfo)]),
        "pixhip_model_tensor": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.POINTER(TensorInfo)]),
        "pixhip_model_metadata_count": (ctypes.c_uint64, [vp]),
        "pixhip_model_metadata_key": (ctypes.c_int64, [vp, ctypes.c_uint64, ctypes.c_char_p, sz]),
        "pixhip_model_metadata_value": (ctypes.c_int64, [vp, ctypes.c_uint64, ctypes.c_char_p, sz]),
        "pixhip_model_metadata": (ctypes.c_int64, [vp, ctypes.c_char_p, ctypes.c_char_p, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def describe(lib, path, safetensors_format=False):
    """Our reader's description of `path` in ref_model_probe's text form."""
    h = ctypes.c_void_p()
    rc = lib.pixhip_model_open(str(path).encode(), int(safetensors_format), ctypes.byref(h))
    text = f"open {CODES.get(rc, rc)}\n"
    if rc:
        return text
    try:
        info = TensorInfo()
        for i in range(lib.pixhip_model_tensor_count(h)):
            assert lib.pixhip_model_tensor_at(h, i, ctypes.byref(info)) == 0
            shape = ",".join(str(info.shape[d]) for d in range(info.rank))
            name = ctypes.string_at(info.name, info.name_length).decode("utf-8", "surrogateescape")
            text += f"T {name} {info.type} {shape} {info.offset} {info.bytes}\n"
        for i in range(lib.pixhip_model_metadata_count(h)):
            parts = []
            for fn in (lib.pixhip_model_metadata_key, lib.pixhip_model_metadata_value):
                n = fn(h, i, None, 0)
                buf = ctypes.create_string_buffer(n + 1)
                assert fn(h, i, buf, len(buf)) == n
                parts.append(buf.raw[:n].decode("utf-8", "surrogateescape"))
            text += f"M {parts[0]} {parts[1]}\n"
    finally:
        lib.pixhip_model_close(h)
    return text


def reference_describe(ref, path, safetensors_format=False):
    n = ref.ref_model_probe(str(path).encode(), int(safetensors_format), None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    ref.ref_model_probe(str(path).encode(), int(safetensors_format), buf, len(buf))
    return buf.raw[:n].decode("utf-8", "surrogateescape")


def random_q8_0(rng, rows, inner):
    """Q8_0 rows of random quantized values with finite fp16 scales."""
    b = rng.integers(0, 256, (rows, inner // 32, 34), dtype=np.uint8)
    b[..., 0:2] = np.frombuffer(np.float16(rng.uniform(0.001, 0.05, rows * inner // 32)).tobytes(), np.uint8).reshape(rows, -1, 2)
    return b.reshape(rows, -1)
