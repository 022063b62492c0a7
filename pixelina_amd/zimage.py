"""One Z-Image DiT block, z_block (src/inference.cpp:293-345), composed from the
library's C ABI on device-resident tensors: the op sequence the reference's
Vulkan build runs for the block (its tensor_* calls each take the vulkan_*
branch), here as pixhip_* calls on one session's stream.

    z_block step (src/inference.cpp)             pixhip entry point
    modulation = adaLN linear + bias  :295       pixhip_matmul_ex (bias)
    norm1, z_modulate part 0          :297-298   pixhip_norm_quantize (Q8_K for qkv)
    qkv                               :299       pixhip_matmul_stage (MULTIPLY)
    q / k / v column slices           :301-312   pixhip_copy_rows x 3
    head_norm q, k                    :315-316   pixhip_norm_quantize (type 0, rows x heads rows of 128)
    rope q, k (interleaved)           :317-318   pixhip_rope x 2
    attention, 30 heads               :319       pixhip_attention
    out                               :320       pixhip_matmul
    norm2, z_residual part 1          :321-327   pixhip_norm_quantize (type 0), pixhip_pointwise_ex RESIDUAL
    ffn_norm1, z_modulate part 2      :329-330   pixhip_norm_quantize (Q8_K for w1, w3)
    w1, w3                            :331-332   pixhip_matmul_stage (MULTIPLY) x 2
    silu(w1) * w3                     :333-334   pixhip_silu_gate_quantize (Q8_0 for w2)
    w2                                :337       pixhip_matmul_stage (MULTIPLY)
    ffn_norm2, z_residual part 3      :338-339   pixhip_norm_quantize (type 0), pixhip_pointwise_ex RESIDUAL

Without a timestep (the context refiner, :399) there is no modulation: no
z_modulate and the residuals are ungated, as in the reference.  The block
updates `x` in place; the reference's finite check (:340-343, CPU builds only)
is left to the caller.
"""
import numpy as np

from . import _lib

HIDDEN, INTERMEDIATE, HEADS, HEAD_DIM, TIME_DIM = 3840, 10240, 30, 128, 256
NORM_EPSILON = 1e-5  # COMPUTE_Z_NORM_EPSILON, src/tensor.h:33
OP_MODULATE, OP_RESIDUAL = 8, 9


class ZBlockWeights:
    """The tensors of one block (the names validate_z_block checks,
    src/inference.cpp:41-57): quantized linears as session weights, the norm
    vectors and the modulation bias in device memory.  `linears` maps qkv,
    out, w1, w3, w2 and (optionally) modulation to (GGUF bytes, type);
    `vectors` maps attention_norm1, attention_norm2, ffn_norm1, ffn_norm2,
    q_norm, k_norm and (optionally) modulation_bias to float32 arrays."""

    SHAPES = {"qkv": (HIDDEN, 3 * HIDDEN), "out": (HIDDEN, HIDDEN), "w1": (HIDDEN, INTERMEDIATE),
              "w3": (HIDDEN, INTERMEDIATE), "w2": (INTERMEDIATE, HIDDEN), "modulation": (TIME_DIM, 4 * HIDDEN)}

    def __init__(self, sess, name, linears, vectors):
        self.sess = sess
        self.types = {}
        self.w = {}
        for key, (gguf, wtype) in linears.items():
            inner, rows = self.SHAPES[key]
            self.w[key] = sess.weight(f"{name}:{key}", gguf, wtype, inner, rows)
            self.types[key] = wtype
        if self.types["w1"] != self.types["w3"]:
            raise ValueError("w1 and w3 share one quantized input: they must have one type")
        self.v = {key: sess.to_device(np.ascontiguousarray(a, np.float32)) for key, a in vectors.items()}
        self.modulated = "modulation" in self.w

    def free(self):
        for b in self.v.values():
            b.free()
        self.v = {}


class ZBlock:
    """Activation buffers for `rows` tokens and the block's op list.  ops()
    returns [(name, fn)] in the reference's order; run() calls them all.  Each
    fn enqueues its work on the session's stream and raises on an error code."""

    def __init__(self, sess, weights, rows, keep_gated=False):
        self.sess, self.wt, self.rows = sess, weights, rows
        f4 = 4
        self.mod = sess.alloc(4 * HIDDEN * f4)
        self.qkv = sess.alloc(rows * 3 * HIDDEN * f4)
        self.q, self.k, self.v = (sess.alloc(rows * HIDDEN * f4) for _ in range(3))
        self.qn, self.kn = sess.alloc(rows * HIDDEN * f4), sess.alloc(rows * HIDDEN * f4)
        self.att = sess.alloc(rows * HIDDEN * f4)
        self.proj = sess.alloc(rows * HIDDEN * f4)
        self.res = sess.alloc(rows * HIDDEN * f4)
        self.gate = sess.alloc(rows * INTERMEDIATE * f4)
        self.up = sess.alloc(rows * INTERMEDIATE * f4)
        # the fp32 SwiGLU product as well as its Q8 blocks (for a caller that
        # inspects it; the block itself needs only the blocks)
        self.gated = sess.alloc(rows * INTERMEDIATE * f4) if keep_gated else None

    def free(self):
        for b in (self.mod, self.qkv, self.q, self.k, self.v, self.qn, self.kn, self.att, self.proj, self.res, self.gate,
                  self.up, self.gated):
            if b is not None:
                b.free()

    def ops(self, x_ptr, cos_ptr, sin_ptr, timestep_ptr=None):
        s, w, v, m = self.sess, self.wt.w, self.wt.v, self.rows
        ty = self.wt.types
        ck = _lib.check
        mult = _lib.STAGE_MULTIPLY
        gated = self.wt.modulated and timestep_ptr is not None
        mod = self.mod.ptr if gated else None

        def part(p):
            return self.mod.ptr + p * HIDDEN * 4 if gated else None

        def norm_into(src, n, key, dst):
            ck(s.norm_quantize(0, src, n, HIDDEN, v[key].ptr, NORM_EPSILON, False, None, dst), key)

        ops = []
        if gated:
            ops.append(("modulation", lambda: ck(s.matmul_ex(w["modulation"], timestep_ptr, 1, self.mod.ptr,
                                                              bias_ptr=v["modulation_bias"].ptr), "modulation")))
        ops += [
            ("attention_norm1", lambda: ck(s.norm_quantize(ty["qkv"], x_ptr, m, HIDDEN, v["attention_norm1"].ptr, NORM_EPSILON,
                                                           False, part(0)), "attention_norm1")),
            ("qkv", lambda: ck(s.matmul_stage(w["qkv"], None, m, self.qkv.ptr, mult), "qkv")),
            ("split", lambda: [ck(s.copy_rows(self.qkv.ptr, m, 3 * HIDDEN, b.ptr, m, HIDDEN, m, 0, i * HIDDEN, 0), "split")
                               for i, b in enumerate((self.q, self.k, self.v))]),
            ("head_norm", lambda: [ck(s.norm_quantize(0, src.ptr, m * HEADS, HEAD_DIM, v[key].ptr, NORM_EPSILON, False, None,
                                                      dst.ptr), key)
                                   for src, dst, key in ((self.q, self.qn, "q_norm"), (self.k, self.kn, "k_norm"))]),
            ("rope", lambda: [ck(s.rope(b.ptr, m, HIDDEN, HEADS, cos_ptr, sin_ptr, True), "rope") for b in (self.qn, self.kn)]),
            ("attention", lambda: ck(s.attention(self.qn.ptr, m, self.kn.ptr, self.v.ptr, m, HEADS, HEADS, HIDDEN, self.att.ptr),
                                     "attention")),
            ("out", lambda: ck(s.matmul(w["out"], self.att.ptr, m, self.proj.ptr), "out")),
            ("attention_norm2", lambda: norm_into(self.proj.ptr, m, "attention_norm2", self.res.ptr)),
            ("residual1", lambda: ck(s.pointwise_ex(OP_RESIDUAL, x_ptr, self.res.ptr, mod, m, HIDDEN, 1), "residual")),
            ("ffn_norm1", lambda: ck(s.norm_quantize(ty["w1"], x_ptr, m, HIDDEN, v["ffn_norm1"].ptr, NORM_EPSILON, False,
                                                     part(2)), "ffn_norm1")),
            ("w1", lambda: ck(s.matmul_stage(w["w1"], None, m, self.gate.ptr, mult), "w1")),
            ("w3", lambda: ck(s.matmul_stage(w["w3"], None, m, self.up.ptr, mult), "w3")),
            ("silu_gate", lambda: ck(s.silu_gate_quantize(ty["w2"], self.gate.ptr, self.up.ptr, m, INTERMEDIATE,
                                                          None if self.gated is None else self.gated.ptr), "silu_gate")),
            ("w2", lambda: ck(s.matmul_stage(w["w2"], None, m, self.proj.ptr, mult), "w2")),
            ("ffn_norm2", lambda: norm_into(self.proj.ptr, m, "ffn_norm2", self.res.ptr)),
            ("residual2", lambda: ck(s.pointwise_ex(OP_RESIDUAL, x_ptr, self.res.ptr, mod, m, HIDDEN, 3), "residual")),
        ]
        return ops

    def run(self, x_ptr, cos_ptr, sin_ptr, timestep_ptr=None):
        for _, fn in self.ops(x_ptr, cos_ptr, sin_ptr, timestep_ptr):
            fn()


def rotary(tokens, caption, patch_width, image):
    """z_rotary (src/inference.cpp:229-259): cosine and sine tables [tokens][64]
    for the three axes (32, 48, 48 dims) -- caption rows at positions (row + 1,
    0, 0), image rows at (caption + 1, row / patch_width, row % patch_width);
    angle = float(position / 256^(2d / axis_dims)) in double, then its fp32
    cosine and sine."""
    dims = (32, 48, 48)
    pos = np.zeros((tokens, 3), np.float64)
    r = np.arange(tokens)
    if image:
        pos[:, 0] = caption + 1
        pos[:, 1] = r // patch_width
        pos[:, 2] = r % patch_width
    else:
        pos[:, 0] = r + 1
    cols = []
    for axis, d in enumerate(dims):
        freq = np.power(256.0, np.arange(d // 2) * 2.0 / d)
        cols.append((pos[:, axis:axis + 1] / freq[None, :]).astype(np.float32))
    angle = np.concatenate(cols, axis=1)
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
