/* Oracle: a plain-C restatement of Pixelina's CPU quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline) -- never as the thing measured or shipped.  The
 * product path lives in pixelina_amd/ and fails loudly without its HIP build.
 *
 * Every function follows the file:line of the reference it restates (paths are
 * relative to the reference tree).  Parity status of each function is pinned by
 * tests/test_oracle.py against golden vectors written by the compiled
 * reference (tests/golden/) plus closed-form / brute-force checks.
 *
 * Besides the linear path it restates the reference's other backend ops
 * (norms, row moves, layouts, decode, modulation), each at its file:line.
 *
 * Block layouts are the reference's (src/kernels_quant.cpp:14-38,
 * src/model_types.h:10-21):
 *   Q8_0   34 B : fp16 d, int8 qs[32]
 *   Q8_K  292 B : fp32 d, int8 qs[256], int16 bsums[16]
 *   Q5_K  176 B : fp16 d, fp16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
 *   Q6_K  210 B : u8 ql[128], u8 qh[64], int8 scales[16], fp16 d
 */
#ifndef PIX_ORACLE_H
#define PIX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORC_Q8_0 8
#define ORC_Q5_K 13
#define ORC_Q6_K 14

#ifdef __cplusplus
extern "C" {
#endif

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
int orc_nearest_int_fused(float scale, float x);
void orc_quantize_q8_0(const float* x, void* blocks, int64_t k);
void orc_quantize_q8_K(const float* x, void* blocks, int64_t k);
float orc_dot_q8_0(int n, const void* w, const void* a);
float orc_dot_q5_K(int n, const void* w, const void* a);
float orc_dot_q6_K(int n, const void* w, const void* a);
int32_t orc_block_sums_q8_0(const void* w, const void* a);
void orc_superblock_sums_q5_K(const void* w, const void* a, int32_t* scaled, int32_t* mins);
int32_t orc_superblock_sum_q6_K(const void* w, const void* a);
int orc_quant_matmul(const void* w, uint32_t type, const float* x, float* y,
                     size_t rows, size_t columns, size_t inner, int threads);
void orc_decode(const void* data, uint32_t type, size_t count, double* out);
uint64_t orc_row_bytes(uint64_t inner, uint32_t type);
void orc_norm_rows(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, int centered, float* out);
void orc_modulate_rows(float* x, size_t rows, size_t channels, const float* scale);
void orc_silu_gate(const float* gate, const float* up, size_t count, float* out);
void orc_gelu(float* x, size_t count, int approximate);
void orc_bias(float* x, size_t rows, size_t channels, const float* bias);
void orc_add(float* x, const float* y, size_t count);
void orc_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, int interleaved);
int orc_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                  size_t channels, const uint64_t* ranges, size_t nranges, size_t query_offset, float* out);

void orc_channel_op(int op, float* x, const float* other, const float* p, size_t rows, size_t channels, float scale, float bias);
int orc_qwen_modulate(float* x, size_t rows, size_t channels, const float* parameters, size_t parameter_channels, size_t target_begin,
                      size_t part, const float* residual);
int orc_l2norm(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, float* out);
void orc_groupnorm(const float* x, size_t rows, size_t channels, const float* weight, const float* bias, float* out);
void orc_decode_f32(const void* data, uint32_t type, size_t count, float* out);
int orc_rows(const float* source, size_t source_rows, float* destination, size_t destination_rows, size_t channels,
             const uint64_t* rows, size_t count, int scatter);
void orc_layout(int op, const float* source, float* destination, size_t width, size_t height, size_t channels, size_t patch);
int orc_conv2d(const float* x, size_t width, size_t height, size_t cin, const float* weight, size_t kx_n, size_t ky_n, size_t cout,
               const float* bias, size_t sx, size_t sy, size_t left, size_t right, size_t top, size_t bottom, float* out);
int orc_shortcut(const float* input, size_t width, size_t height, size_t input_channels, size_t channels, size_t temporal, int up,
                 int spatial, float* out);

#ifdef __cplusplus
}
#endif

#endif
