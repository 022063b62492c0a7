"""Seeded synthetic inputs and K-quant weight packers.

Generator: SplitMix64 (the published constants of Steele, Lea & Flood 2014)
drives Box-Muller normals; sample i of a stream uses counter i+1, so any
slice of a stream can be regenerated alone.  Pixelina seeds its noise the same
way (inference_noise, src/inference.cpp:540-562); the fill order here is
plain row-major.

Packers: the reference only decodes Q5_K / Q6_K (src/backend_cpu.cpp:56-96);
these encoders produce valid blocks of those layouts for synthetic weights.
Q8_0 weights use the reference's own quantizer semantics instead (the HIP
quantizer, bit-exact with quantize_row_q8_0_ref).
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

SEED_ACTIVATIONS = 1337  # PIXELINA_DEFAULT_SEED, src/storage.h:37
SEED_WEIGHTS = 1338
SEED_OUTLIERS = 1339

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_MIX1 = np.uint64(0xBF58476D1CE4E5B9)
_MIX2 = np.uint64(0x94D049BB133111EB)


def splitmix_uniform(seed, n, start=0):
    """n doubles in (0,1): ((mix(seed + (start+i+1)*gamma) >> 11) + 0.5) * 2^-53."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _MIX1
        z = (z ^ (z >> np.uint64(27))) * _MIX2
    z ^= z >> np.uint64(31)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def _threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _parallel(fn, items):
    """fn over items on a thread pool (numpy releases the GIL in its loops)."""
    items = list(items)
    if len(items) <= 1:
        return [fn(i) for i in items]
    with ThreadPoolExecutor(min(_threads(), len(items))) as ex:
        return list(ex.map(fn, items))


def normal(seed, shape, std=1.0, chunk=1 << 20, start=0):
    """float32 N(0, std^2) of the given shape, Box-Muller pairs in row-major order.

    `start` (even) skips that many values of the stream, so consecutive
    tensors drawn with start = the running count continue one stream."""
    if start % 2:
        raise ValueError("start must be even (values come in Box-Muller pairs)")
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2

    def fill(p0):
        p1 = min(pairs, p0 + chunk)
        u = splitmix_uniform(seed, 2 * (p1 - p0), start=start + 2 * p0)
        r = np.sqrt(-2.0 * np.log(u[0::2]))
        a = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * (p1 - p0), dtype=np.float64)
        z[0::2] = r * np.cos(a)
        z[1::2] = r * np.sin(a)
        lo, hi = 2 * p0, min(n, 2 * p1)
        out[lo:hi] = (z[: hi - lo] * std).astype(np.float32)

    _parallel(fill, range(0, pairs, chunk))
    return out.reshape(shape)


def outlier_channels(k, fraction=0.01, seed=SEED_OUTLIERS):
    """Indices of round(fraction*k) inner channels, chosen by sorting SplitMix uniforms."""
    count = int(round(fraction * k))
    return np.sort(np.argsort(splitmix_uniform(seed, k), kind="stable")[:count])


def log_uniform(seed, n, lo, hi, start=0):
    u = splitmix_uniform(seed, n, start=start)
    return np.exp(np.log(lo) + u * (np.log(hi) - np.log(lo))).astype(np.float32)


def _f16_bits(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def _by_rows(pack, w, rows=256):
    """pack() over row slices (each row's blocks depend on that row alone), on a
    thread pool; slices small enough for the temporaries to stay in cache."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.shape[0] <= rows:
        return pack(w)
    return np.concatenate(_parallel(lambda r: pack(w[r:r + rows]), range(0, w.shape[0], rows)))


def pack_q5_K(w):
    """float32 [rows, K] (K % 256 == 0) -> uint8 [rows, K/256*176] Q5_K blocks.

    Per 32-value sub-block: offset m = -min(min x, 0), step = (max x + m)/31;
    super-block d = max step/63, dmin = max m/63 (stored fp16); six-bit
    scale/min indices rounded to nearest; q = round((x + dmin*min)/(d*scale))
    clipped to [0,31].  Layout per src/kernels_quant.cpp:18-23, decode
    src/backend_cpu.cpp:56-79.
    """
    return _by_rows(_pack_q5_K, w)


def _pack_q5_K(w):
    rows, k = w.shape
    assert k % 256 == 0
    x = w.reshape(rows, k // 256, 8, 32).astype(np.float64)
    mins = np.maximum(-x.min(axis=-1), 0.0)
    steps = (x.max(axis=-1) + mins) / 31.0
    d = (steps.max(axis=-1) / 63.0).astype(np.float32).astype(np.float16)
    dmin = (mins.max(axis=-1) / 63.0).astype(np.float32).astype(np.float16)
    d64, dm64 = d.astype(np.float64)[..., None], dmin.astype(np.float64)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d64 > 0, np.rint(steps / d64), 0).clip(0, 63).astype(np.int64)
        mn = np.where(dm64 > 0, np.rint(mins / dm64), 0).clip(0, 63).astype(np.int64)
        step = (d64 * sc)[..., None]
        q = np.where(step > 0, np.rint((x + (dm64 * mn)[..., None]) / step), 0).clip(0, 31).astype(np.int64)
    blk = np.zeros((rows, k // 256, 176), dtype=np.uint8)
    blk[..., 0:2] = _f16_bits(d)[..., None].view(np.uint8).reshape(rows, k // 256, 2)
    blk[..., 2:4] = _f16_bits(dmin)[..., None].view(np.uint8).reshape(rows, k // 256, 2)
    for s in range(4):
        blk[..., 4 + s] = (sc[..., s] & 63) | ((sc[..., s + 4] >> 4) << 6)
        blk[..., 8 + s] = (mn[..., s] & 63) | ((mn[..., s + 4] >> 4) << 6)
        blk[..., 12 + s] = (sc[..., s + 4] & 15) | ((mn[..., s + 4] & 15) << 4)
    qh = np.zeros((rows, k // 256, 32), dtype=np.int64)
    for s in range(8):
        qh |= ((q[:, :, s, :] >> 4) & 1) << s
    blk[..., 16:48] = qh
    for p in range(4):
        blk[..., 48 + 32 * p: 80 + 32 * p] = (q[:, :, 2 * p, :] & 15) | ((q[:, :, 2 * p + 1, :] & 15) << 4)
    return blk.reshape(rows, -1)


def pack_q6_K(w):
    """float32 [rows, K] -> uint8 [rows, K/256*210] Q6_K blocks.

    Per 16 values: step = max|x|/31; d = max step/127 (fp16); int8 scale =
    round(step/d); q = round(x/(d*scale)) + 32 clipped to [0,63].  Layout per
    src/kernels_quant.cpp:24-29, decode src/backend_cpu.cpp:80-96.
    """
    return _by_rows(_pack_q6_K, w)


def _pack_q6_K(w):
    rows, k = w.shape
    assert k % 256 == 0
    x = w.reshape(rows, k // 256, 16, 16).astype(np.float64)
    steps = np.abs(x).max(axis=-1) / 31.0
    d = (steps.max(axis=-1) / 127.0).astype(np.float32).astype(np.float16)
    d64 = d.astype(np.float64)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d64 > 0, np.rint(steps / d64), 0).clip(-128, 127).astype(np.int64)
        step = (d64 * sc)[..., None]
        q = (np.where(step != 0, np.rint(x / step), 0).clip(-32, 31) + 32).astype(np.int64)
    q = q.reshape(rows, k // 256, 256)
    blk = np.zeros((rows, k // 256, 210), dtype=np.uint8)
    for h in range(2):
        for g in range(4):
            e = q[:, :, 128 * h + 32 * g: 128 * h + 32 * g + 32]
            lo = 64 * h + (g % 2) * 32
            if g < 2:
                blk[..., lo:lo + 32] |= (e & 15).astype(np.uint8)
            else:
                blk[..., lo:lo + 32] |= ((e & 15) << 4).astype(np.uint8)
            blk[..., 128 + 32 * h: 160 + 32 * h] |= (((e >> 4) & 3) << (2 * g)).astype(np.uint8)
    blk[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    blk[..., 208:210] = _f16_bits(d)[..., None].view(np.uint8).reshape(rows, k // 256, 2)
    return blk.reshape(rows, -1)


ROW_BYTES = {8: (32, 34), 13: (256, 176), 14: (256, 210)}


def row_bytes(inner, wtype):
    """weight_bytes({inner}, type) of src/model.cpp:87-121."""
    values, nbytes = ROW_BYTES[wtype]
    return inner // values * nbytes
