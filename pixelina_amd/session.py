"""Thin Python handle over the C ABI (tests and bench drive the kernels
through exactly the entry points a C/C++ caller would use)."""
import ctypes

import numpy as np

from . import _lib
from ._lib import check


class DeviceBuffer:
    """A pixhip_allocate'd device block owned by a Session."""

    def __init__(self, session, nbytes):
        self.session = session
        self.nbytes = int(nbytes)
        self.ptr = session.lib.pixhip_allocate(session.handle, self.nbytes)
        if not self.ptr:
            raise _lib.PixhipError(_lib.ERR_MEMORY, f"pixhip_allocate({self.nbytes})")

    def upload(self, array, offset=0):
        a = np.ascontiguousarray(array)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(self.session.lib.pixhip_copy_to_device(self.session.handle, self.ptr + offset, a.ctypes.data, a.nbytes),
              "pixhip_copy_to_device")
        return self

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download larger than the buffer")
        check(self.session.lib.pixhip_copy_to_host(self.session.handle, out.ctypes.data, self.ptr + offset, out.nbytes),
              "pixhip_copy_to_host")
        return out

    def free(self):
        if self.ptr:
            self.session.lib.pixhip_free(self.session.handle, self.ptr)
            self.ptr = None


class Session:
    def __init__(self, device=0):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        check(self.lib.pixhip_session_create(device, ctypes.byref(h)), "pixhip_session_create")
        self.handle = h.value
        # The library re-reads a weight's host bytes when it rebuilds a form
        # (after eviction, or for the other kernel family): keep them alive for
        # the session, as a model file's mapping is.
        self._host_weights = {}

    def close(self):
        if self.handle:
            self.lib.pixhip_session_destroy(self.handle)
            self.handle = None
            self._host_weights = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # memory
    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, array):
        a = np.ascontiguousarray(array)
        return DeviceBuffer(self, max(a.nbytes, 4)).upload(a)

    def copy_device(self, dst_ptr, src_ptr, nbytes):
        check(self.lib.pixhip_copy_device(self.handle, dst_ptr, src_ptr, nbytes), "pixhip_copy_device")

    def synchronize(self):
        check(self.lib.pixhip_synchronize(self.handle), "pixhip_synchronize")

    def device_name(self):
        buf = ctypes.create_string_buffer(256)
        check(self.lib.pixhip_device_name(self.handle, buf, 256), "pixhip_device_name")
        return buf.value.decode()

    # weights
    def weight(self, key, gguf_bytes, wtype, inner, rows):
        b = np.ascontiguousarray(gguf_bytes, dtype=np.uint8)
        h = ctypes.c_void_p()
        check(self.lib.pixhip_weight_get(self.handle, key.encode(), b.ctypes.data, b.nbytes, wtype, inner, rows,
                                         ctypes.byref(h)), "pixhip_weight_get")
        self._host_weights[key] = b
        return h.value

    def weight_shape(self, weight):
        t, k, n = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        check(self.lib.pixhip_weight_shape(weight, ctypes.byref(t), ctypes.byref(k), ctypes.byref(n)), "pixhip_weight_shape")
        return t.value, k.value, n.value

    def cache_info(self):
        n, b = ctypes.c_uint64(), ctypes.c_uint64()
        check(self.lib.pixhip_weight_cache_info(self.handle, ctypes.byref(n), ctypes.byref(b)), "pixhip_weight_cache_info")
        return n.value, b.value

    def residency(self):
        """(GGUF bytes, resident device bytes) of the weights with device forms."""
        g, r = ctypes.c_uint64(), ctypes.c_uint64()
        check(self.lib.pixhip_weight_residency(self.handle, ctypes.byref(g), ctypes.byref(r)), "pixhip_weight_residency")
        return g.value, r.value

    def set_weight_budget(self, nbytes):
        check(self.lib.pixhip_set_weight_budget(self.handle, nbytes), "pixhip_set_weight_budget")

    def prepare_stage(self, activation_bytes, scratch_bytes):
        return self.lib.pixhip_prepare_stage(self.handle, activation_bytes, scratch_bytes)

    # the op
    def matmul(self, weight, x_ptr, columns, y_ptr):
        return self.lib.pixhip_matmul(self.handle, weight, x_ptr, columns, y_ptr)

    def matmul_ex(self, weight, x_ptr, columns, y_ptr, bias_ptr=None, ldy=0, y_offset=0):
        return self.lib.pixhip_matmul_ex(self.handle, weight, x_ptr, columns, y_ptr, bias_ptr, ldy, y_offset)

    def matmul_noalloc(self, weight, x_ptr, columns, y_ptr, bias_ptr=None, ldy=0, y_offset=0):
        return self.lib.pixhip_matmul_ex_noalloc(self.handle, weight, x_ptr, columns, y_ptr, bias_ptr, ldy, y_offset)

    def matmul_stage(self, weight, x_ptr, columns, y_ptr, stages, bias_ptr=None, ldy=0, y_offset=0):
        return self.lib.pixhip_matmul_stage(self.handle, weight, x_ptr, columns, y_ptr, bias_ptr, ldy, y_offset, stages)

    def quant_matmul(self, w_host_ptr, wtype, x_ptr, y_ptr, rows, columns, inner):
        return self.lib.pixhip_quant_matmul(self.handle, w_host_ptr, wtype, x_ptr, y_ptr, rows, columns, inner)

    def quantize_q8_0(self, x_ptr, blocks_ptr, rows, inner):
        return self.lib.pixhip_quantize_q8_0(self.handle, x_ptr, blocks_ptr, rows, inner)

    def quantize_q8_K(self, x_ptr, blocks_ptr, rows, inner):
        return self.lib.pixhip_quantize_q8_K(self.handle, x_ptr, blocks_ptr, rows, inner)

    def norm_quantize(self, wtype, x_ptr, rows, inner, norm_weight_ptr=None, eps=1e-5, centered=False,
                      modulation_ptr=None, normalized_ptr=None, blocks_ptr=None):
        return self.lib.pixhip_norm_quantize(self.handle, wtype, x_ptr, rows, inner, norm_weight_ptr, eps, int(centered),
                                             modulation_ptr, normalized_ptr, blocks_ptr)

    def silu_gate_quantize(self, wtype, gate_ptr, up_ptr, rows, inner, gated_ptr=None, blocks_ptr=None):
        return self.lib.pixhip_silu_gate_quantize(self.handle, wtype, gate_ptr, up_ptr, rows, inner, gated_ptr, blocks_ptr)

    def pointwise(self, op, dst_ptr, second_ptr, rows, channels):
        return self.lib.pixhip_pointwise(self.handle, op, dst_ptr, second_ptr, rows, channels)

    def rope(self, x_ptr, rows, channels, heads, cos_ptr, sin_ptr, interleaved):
        return self.lib.pixhip_rope(self.handle, x_ptr, rows, channels, heads, cos_ptr, sin_ptr, int(interleaved))

    def attention(self, q_ptr, rows, k_ptr, v_ptr, keys, heads, kv_heads, channels, out_ptr, causal=False, ranges=None,
                  query_offset=0):
        """tensor_attention (src/tensor.cpp:347-427): the causal form, or the
        ranges form when `ranges` [(query_begin, query_end, key_end, causal)]."""
        if ranges is None:
            return self.lib.pixhip_attention(self.handle, q_ptr, rows, k_ptr, v_ptr, keys, heads, kv_heads, channels,
                                             int(causal), out_ptr)
        arr = (_lib.AttentionRange * max(1, len(ranges)))(*[_lib.AttentionRange(*r) for r in ranges])
        return self.lib.pixhip_attention_ranges(self.handle, q_ptr, rows, k_ptr, v_ptr, keys, heads, kv_heads, channels,
                                                arr, len(ranges), query_offset, out_ptr)

    # ---- the rest of the backend op surface (src/backend_vulkan.h:141-156) ----

    def pointwise_ex(self, op, dst_ptr, second_ptr, third_ptr, rows, channels, part=0, scale=0.0, bias=0.0):
        """vulkan_pointwise with all its arguments (src/backend_vulkan.cpp:1112-1127)."""
        return self.lib.pixhip_pointwise_ex(self.handle, op, dst_ptr, second_ptr, third_ptr, rows, channels, part, scale, bias)

    def qwen_modulate(self, dst_ptr, rows, channels, params_ptr, param_channels, target_begin, part, residual_ptr=None):
        """qwen_image_modulate (src/qwen_image.cpp:149-169)."""
        return self.lib.pixhip_qwen_modulate(self.handle, dst_ptr, rows, channels, params_ptr, param_channels, target_begin, part,
                                             residual_ptr)

    def l2norm(self, x_ptr, rows, channels, weight_ptr, eps, out_ptr):
        """tensor_l2norm (src/tensor.cpp:242-258)."""
        return self.lib.pixhip_l2norm(self.handle, x_ptr, rows, channels, weight_ptr, eps, out_ptr)

    def groupnorm(self, x_ptr, rows, channels, weight_ptr, bias_ptr, out_ptr):
        """tensor_groupnorm (src/tensor.cpp:454-485)."""
        return self.lib.pixhip_groupnorm(self.handle, x_ptr, rows, channels, weight_ptr, bias_ptr, out_ptr)

    def embedding(self, table_ptr, wtype, inner, table_rows, ids, out_ptr):
        """vulkan_embedding (src/backend_vulkan.cpp:1239-1255); `ids` a sequence of ints."""
        arr = (ctypes.c_int32 * max(1, len(ids)))(*[int(i) for i in ids])
        return self.lib.pixhip_embedding(self.handle, table_ptr, wtype, inner, table_rows, arr, len(ids), out_ptr)

    def rows(self, src_ptr, src_rows, dst_ptr, dst_rows, channels, rows, scatter):
        """tensor_gather / tensor_scatter (src/tensor.cpp:274-302); `rows` a sequence of ints."""
        arr = (ctypes.c_size_t * max(1, len(rows)))(*[int(r) for r in rows])
        return self.lib.pixhip_rows(self.handle, src_ptr, src_rows, dst_ptr, dst_rows, channels, arr, len(rows), int(scatter))

    def copy_rows(self, src_ptr, src_rows, src_channels, dst_ptr, dst_rows, dst_channels, rows, src_row=0, src_feature=0, dst_row=0):
        """vulkan_copy_rows (src/backend_vulkan.cpp:1257-1269)."""
        return self.lib.pixhip_copy_rows(self.handle, src_ptr, src_rows, src_channels, dst_ptr, dst_rows, dst_channels, rows, src_row,
                                         src_feature, dst_row)

    def copy_features(self, src_ptr, src_channels, dst_ptr, dst_channels, dst_feature):
        """vulkan_copy_features (src/backend_vulkan.cpp:1271-1281)."""
        return self.lib.pixhip_copy_features(self.handle, src_ptr, src_channels, dst_ptr, dst_channels, dst_feature)

    def layout(self, op, src_ptr, src_rows, src_channels, dst_ptr, dst_rows, dst_channels, width, patch=0):
        """vulkan_layout (src/backend_vulkan.cpp:1283-1295)."""
        return self.lib.pixhip_layout(self.handle, op, src_ptr, src_rows, src_channels, dst_ptr, dst_rows, dst_channels, width, patch)

    def shortcut(self, src_ptr, width, height, src_channels, dst_ptr, channels, temporal, up, spatial):
        """tensor_resample_shortcut (src/tensor.cpp:487-527)."""
        return self.lib.pixhip_shortcut(self.handle, src_ptr, width, height, src_channels, dst_ptr, channels, temporal, int(up),
                                        int(spatial))

    def conv_weight(self, key, raw_bytes, wtype, kx, ky, cin, cout):
        """pixhip_conv_weight_get over a float tensor's bytes [kx, ky, cin, cout] (GGML order)."""
        b = np.ascontiguousarray(raw_bytes, dtype=np.uint8)
        h = ctypes.c_void_p()
        check(self.lib.pixhip_conv_weight_get(self.handle, key.encode(), b.ctypes.data, b.nbytes, wtype, kx, ky, cin, cout,
                                              ctypes.byref(h)), "pixhip_conv_weight_get")
        self._host_weights[key] = b
        return h.value

    def conv2d(self, weight, x_ptr, width, height, out_ptr, geometry=None, bias_ptr=None):
        """tensor_conv (src/convolution.cpp:34-100); geometry (sx, sy, left, right, top, bottom) or None."""
        g = None if geometry is None else ctypes.byref(_lib.ConvGeometry(*geometry))
        return self.lib.pixhip_conv2d(self.handle, weight, x_ptr, width, height, g, bias_ptr, out_ptr)

    def block_sums(self, weight, x_ptr, columns, sums_ptr, mins_ptr=None):
        return self.lib.pixhip_block_sums(self.handle, weight, x_ptr, columns, sums_ptr, mins_ptr)

    # timing
    def timer_start(self):
        check(self.lib.pixhip_timer_start(self.handle), "pixhip_timer_start")

    def bench_matmul(self, weights, x_ptr, columns, y_ptr, stages, reps):
        arr = (ctypes.c_void_p * len(weights))(*weights)
        ms = ctypes.c_float()
        check(self.lib.pixhip_bench_matmul(self.handle, arr, len(weights), x_ptr, columns, y_ptr, stages, reps,
                                           ctypes.byref(ms)), "pixhip_bench_matmul")
        return ms.value

    def timer_stop(self):
        ms = ctypes.c_float()
        check(self.lib.pixhip_timer_stop(self.handle, ctypes.byref(ms)), "pixhip_timer_stop")
        return ms.value
