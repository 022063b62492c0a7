"""The model file reader (pixhip_model_*, pixelina_amd/csrc/model_file.cpp), the
counterpart of PixModelFile::open / read (src/model.cpp:138-243).

Against what the files were written with (tests/model_files.py): the tensor
directory (names, types, GGML shapes, absolute offsets, sizes) and every
metadata type's textual value.  Against the reference's own reader, compiled in
place (oracle/_ref ref_model_probe), where it was built: the same files, the
reader's documented rejections (version, counts, alignment, ranks, types,
offsets, overlaps, duplicate keys, safetensors header faults), every
truncation of a file's header and a few hundred random header byte flips, on
which the two readers must print the same description -- accept with the same
directory and metadata, or reject with the same code.  CPU only: the reader
touches no device."""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import model_files as mf
from oracle_lib import reference

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    from pixelina_amd import build
    if not os.path.exists(build.LIBRARY):
        pytest.skip("libpixhip.so not built")
    return mf.bind(ctypes.CDLL(build.LIBRARY))


needs_ref = pytest.mark.skipif(reference() is None, reason="oracle/_ref not built here")

METADATA = [
    ("general.architecture", mf.STRING, "qwen2vl"),
    ("general.name", mf.STRING, 'tab\there "quoted" back\\slash \x01 unicode é中'),
    ("u8", mf.U8, 200), ("i8", mf.I8, -100), ("u16", mf.U16, 65000), ("i16", mf.I16, -30000),
    ("u32", mf.U32, 4000000000), ("i32", mf.I32, -2000000000), ("u64", mf.U64, 18446744073709551615),
    ("i64", mf.I64, -9223372036854775808), ("f32", mf.F32T, 0.1), ("f32big", mf.F32T, 3.0e12), ("f64", mf.F64, -2.5e-7),
    ("yes", mf.BOOL, 1), ("no", mf.BOOL, 0),
    ("tokens", mf.ARRAY, (mf.STRING, ["<s>", "a b", "\n"])), ("ids", mf.ARRAY, (mf.I32, [1, -2, 3])),
    ("scales", mf.ARRAY, (mf.F32T, [0.5, -1.25])), ("empty", mf.ARRAY, (mf.U8, [])),
]
TENSORS = [
    ("token_embd.weight", 8, [64, 5], None),
    ("blk.0.attn_q.weight", 13, [256, 3], None),
    ("blk.0.ffn_down.weight", 14, [512, 2], None),
    ("output_norm.weight", 0, [7], None),
    ("v.patch_embd.weight", 1, [14, 14, 3, 4], None),
    ("conv3d.weight", 30, [3, 3, 1, 2, 2], None),
]


def expected_value(vtype, v):
    """The reference's textual value (PixJson scalar / JSON text)."""
    if vtype == mf.STRING:
        out = '"'
        for ch in v.encode():
            if ch in (0x22, 0x5C):
                out += "\\" + chr(ch)
            elif ch < 0x20:
                out += "\\u%04x" % ch
            else:
                out += chr(ch) if ch < 0x80 else bytes([ch]).decode("latin-1")
        return out + '"'
    if vtype == mf.ARRAY:
        et, items = v
        return "[" + ",".join(expected_value(et, x) for x in items) + "]"
    if vtype == mf.BOOL:
        return "true" if v else "false"
    if vtype == mf.F32T:
        return "%f" % float(np.float32(v))
    if vtype == mf.F64:
        return "%f" % v
    return str(v)


def normalise(text):
    """A description's bytes as latin-1 characters, the form expected_value builds."""
    return text.encode("utf-8", "surrogateescape").decode("latin-1")


def expected_gguf(metadata, tensors, base, offsets, alignment=None):
    lines = ["open 0"]
    for (name, wtype, shape, _), off in sorted(zip(tensors, offsets), key=lambda t: t[0][0]):
        lines.append(f"T {name} {wtype} {','.join(map(str, shape))} {base + off} {mf.tensor_bytes(wtype, shape)}")
    kv = list(metadata) + ([("general.alignment", mf.U32, alignment)] if alignment is not None else [])
    for key, vtype, v in sorted(kv, key=lambda t: t[0].encode()):
        lines.append(f"M {key} {expected_value(vtype, v)}")
    return "\n".join(lines) + "\n"


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return p


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_gguf_directory_and_metadata(lib, tmp_path, alignment):
    data, base, offsets = mf.gguf(METADATA, TENSORS, alignment=alignment, layout=True)
    p = write(tmp_path, "m.gguf", data)
    got = mf.describe(lib, p)
    assert normalise(got) == expected_gguf(METADATA, TENSORS, base, offsets, alignment)
    ref = reference()
    if ref is not None:
        assert got == mf.reference_describe(ref, p)


def test_tensor_lookup_and_mapping(lib, tmp_path):
    data, base, offsets = mf.gguf(METADATA, TENSORS, layout=True)
    p = write(tmp_path, "m.gguf", data)
    h = ctypes.c_void_p()
    assert lib.pixhip_model_open(str(p).encode(), 0, ctypes.byref(h)) == 0
    try:
        size = ctypes.c_uint64()
        mapping = lib.pixhip_model_data(h, ctypes.byref(size))
        assert size.value == len(data)
        info = mf.TensorInfo()
        assert lib.pixhip_model_tensor(h, b"blk.0.attn_q.weight", ctypes.byref(info)) == 0
        assert info.type == 13 and info.rank == 2 and list(info.shape)[:2] == [256, 3]
        assert ctypes.string_at(mapping + info.offset, info.bytes) == data[info.offset:info.offset + info.bytes]
        assert lib.pixhip_model_tensor(h, b"missing", ctypes.byref(info)) == -1
        buf = ctypes.create_string_buffer(64)
        n = lib.pixhip_model_metadata(h, b"general.architecture", buf, len(buf))
        assert n == len('"qwen2vl"') and buf.value == b'"qwen2vl"'
        assert lib.pixhip_model_metadata(h, b"absent", buf, len(buf)) == -1
        small = ctypes.create_string_buffer(4)  # truncated copy, full length returned
        assert lib.pixhip_model_metadata(h, b"general.architecture", small, 4) == 9 and small.value == b'"qw'
    finally:
        lib.pixhip_model_close(h)


def test_safetensors_directory_and_metadata(lib, tmp_path):
    rng = np.random.default_rng(3)
    tensors = [("model.a", "F32", [3, 5], rng.standard_normal(15).astype(np.float32).tobytes()),
               ("model.b", "F16", [2, 2, 4], np.zeros(16, np.float16).tobytes()),
               ("model.c", "BF16", [7], bytes(14))]
    meta = {"format": "pt", "note": "é \"q\" \\ \n"}
    data = mf.safetensors(tensors, meta)
    p = write(tmp_path, "m.safetensors", data)
    got = mf.describe(lib, p, True)
    hlen = struct.unpack("<Q", data[:8])[0]
    lines = ["open 0"]
    off = 0
    for name, dtype, shape, blob in tensors:
        t = {"F32": 0, "F16": 1, "BF16": 30}[dtype]
        lines.append(f"T {name} {t} {','.join(map(str, reversed(shape)))} {8 + hlen + off} {len(blob)}")
        off += len(blob)
    for k in sorted(meta):
        lines.append(f"M {k} " + json.dumps(meta[k], ensure_ascii=False).replace("\\n", "\\u000a"))
    assert got == "\n".join(lines) + "\n"
    ref = reference()
    if ref is not None:
        assert got == mf.reference_describe(ref, p, True)


def test_open_errors(lib, tmp_path):
    h = ctypes.c_void_p()
    assert lib.pixhip_model_open(str(tmp_path / "absent.gguf").encode(), 0, ctypes.byref(h)) == -6
    assert lib.pixhip_model_open(str(tmp_path).encode(), 0, ctypes.byref(h)) == -7      # a directory
    p = write(tmp_path, "short.gguf", b"GGUF\x03\x00\x00")
    assert lib.pixhip_model_open(str(p).encode(), 0, ctypes.byref(h)) == -7
    p = write(tmp_path, "zero.gguf", mf.gguf([], TENSORS, version=2))
    assert lib.pixhip_model_open(str(p).encode(), 0, ctypes.byref(h)) == -7


def faulty_gguf():
    """(label, bytes) of files the reader must reject or handle as the reference does."""
    T = TENSORS[:2]
    cases = [
        ("version 2", mf.gguf([], T, version=2)),
        ("no tensors", mf.gguf([], [])),
        ("alignment 3", mf.gguf([], T, alignment=3)),
        ("alignment 0", mf.gguf([], T, alignment=0)),
        ("alignment as f32", mf.gguf([("general.alignment", mf.F32T, 32.0)], T)),
        ("alignment as string", mf.gguf([("general.alignment", mf.STRING, "32")], T)),
        ("alignment u64", mf.gguf([("general.alignment", mf.U64, 64)], T)),
        ("duplicate key", mf.gguf([("k", mf.U8, 1), ("k", mf.U8, 2)], T)),
        ("bool 2", mf.gguf([("b", mf.BOOL, 2)], T)),
        ("nested array", mf.gguf([("a", mf.ARRAY, (mf.ARRAY, []))], T)),
        ("duplicate tensor", mf.gguf([], [T[0], T[0]])),
        ("type 2 (Q4_0)", mf.gguf([], [("w", 2, [64, 2], None)])),
        ("rank 6", mf.gguf([], [("w", 0, [2, 1, 1, 1, 1, 1], None)])),
        ("zero dimension", mf.gguf([], [("w", 0, [4, 0], None)])),
        ("ragged Q8_0", mf.gguf([], [("w", 8, [48, 2], None)])),
        ("ragged Q5_K", mf.gguf([], [("w", 13, [128, 2], None)])),
    ]
    # hand-edited fields of a valid file
    good, base, offsets = mf.gguf([], T, layout=True)
    b = bytearray(good)
    rank_pos = good.index(b"token_embd.weight") + len("token_embd.weight")
    for label, pos, val in (("rank 0", rank_pos, struct.pack("<I", 0)),
                            ("offset misaligned", rank_pos + 4 + 16 + 4, struct.pack("<Q", 8)),
                            ("offset beyond the file", rank_pos + 4 + 16 + 4, struct.pack("<Q", 1 << 40)),
                            ("overlapping tensors", rank_pos + 4 + 16 + 4, struct.pack("<Q", offsets[1])),
                            ("tensor count huge", 8, struct.pack("<Q", 2000000)),
                            ("metadata count huge", 16, struct.pack("<Q", 2000000))):
        e = bytearray(b)
        e[pos:pos + len(val)] = val
        cases.append((label, bytes(e)))
    cases.append(("truncated data", good[:-1]))
    cases.append(("header cut after the counts", good[:24]))
    t = mf.gguf([("x", mf.U8, 1)], T)
    i = t.index(struct.pack("<Q", 1) + b"x") + 9  # the key's value type
    cases.append(("metadata type 13", t[:i] + struct.pack("<I", 13) + t[i + 4:]))
    return cases


def faulty_safetensors():
    good = mf.safetensors([("a", "F32", [2, 2], bytes(16)), ("b", "F16", [4], bytes(8))], {"k": "v"})

    def with_header(text):
        text = text.encode() if isinstance(text, str) else text
        return struct.pack("<Q", len(text)) + text + bytes(24)
    return [
        ("good", good),
        ("dtype I8", with_header('{"a":{"dtype":"I8","shape":[4],"data_offsets":[0,4]}}')),
        ("shape of strings", with_header('{"a":{"dtype":"F32","shape":["2"],"data_offsets":[0,8]}}')),
        ("shape float", with_header('{"a":{"dtype":"F32","shape":[2.0],"data_offsets":[0,8]}}')),
        ("empty shape", with_header('{"a":{"dtype":"F32","shape":[],"data_offsets":[0,4]}}')),
        ("span mismatch", with_header('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,12]}}')),
        ("end before start", with_header('{"a":{"dtype":"F32","shape":[2],"data_offsets":[8,0]}}')),
        ("past the end", with_header('{"a":{"dtype":"F32","shape":[8],"data_offsets":[0,32]}}')),
        ("overlap", with_header('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},"b":{"dtype":"F32","shape":[2],"data_offsets":[4,12]}}')),
        ("only metadata", with_header('{"__metadata__":{"x":"y"}}')),
        ("metadata not an object", with_header('{"__metadata__":"x","a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("duplicate key", with_header('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"a":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}')),
        ("trailing comma", with_header('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},}')),
        ("lone surrogate", with_header('{"\\udc00":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("surrogate pair", with_header('{"\\ud83d\\ude00":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("bad escape", with_header('{"\\q":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("control char", with_header('{"a\x01":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("deep nesting", with_header('{"__metadata__":' + "[" * 70 + "]" * 70 + ',"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("number forms", with_header('{"__metadata__":{"x":-0.5e+3,"y":0,"z":true,"n":null},"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')),
        ("leading zero", with_header('{"a":{"dtype":"F32","shape":[01],"data_offsets":[0,4]}}')),
        ("header length 0", struct.pack("<Q", 0) + bytes(16)),
        ("header past the end", struct.pack("<Q", 1000) + b"{}"),
        ("not an object", with_header("[1,2]")),
    ]


@needs_ref
def test_documented_rejections_agree_with_reference(lib, tmp_path):
    ref = reference()
    for i, (label, data) in enumerate(faulty_gguf()):
        p = write(tmp_path, f"g{i}.gguf", data)
        assert mf.describe(lib, p) == mf.reference_describe(ref, p), label
    for i, (label, data) in enumerate(faulty_safetensors()):
        p = write(tmp_path, f"s{i}.safetensors", data)
        assert mf.describe(lib, p, True) == mf.reference_describe(ref, p, True), label


@needs_ref
@pytest.mark.parametrize("kind", ["gguf", "safetensors"])
def test_truncations_and_byte_flips_agree_with_reference(lib, tmp_path, kind):
    ref = reference()
    st = kind == "safetensors"
    if st:
        good = mf.safetensors([("w.a", "F32", [3, 4], bytes(48)), ("w.b", "BF16", [8], bytes(16))], {"a": "b", "c": "é"})
        head = 8 + struct.unpack("<Q", good[:8])[0]
    else:
        good, base, _ = mf.gguf(METADATA[:8], TENSORS[:3], layout=True)
        head = base
    rng = np.random.default_rng(11 if st else 12)
    variants = [good[:n] for n in range(0, head + 8)]
    for _ in range(300):
        b = bytearray(good)
        for _ in range(int(rng.integers(1, 3))):
            b[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        variants.append(bytes(b))
    accepted = 0
    p = tmp_path / ("f.safetensors" if st else "f.gguf")
    for i, data in enumerate(variants):
        p.write_bytes(data)
        ours, theirs = mf.describe(lib, p, st), mf.reference_describe(ref, p, st)
        assert ours == theirs, (i, len(data))
        accepted += ours.startswith("open 0")
    print(f"{kind}: {len(variants)} variants, {accepted} accepted by both", flush=True)
    assert 0 < accepted < len(variants)
