/* pixhip: MI355X (gfx950) backend for Pixelina's quantized linear layer.
 *
 * A C ABI (plain pointers and sizes) over hand-written HIP kernels:
 *   - activation block quantizers (Q8_0, Q8_K),
 *   - the Q5_K / Q6_K / Q8_0 integer GEMM on int8 MFMA (M > 1),
 *   - the bandwidth-bound M = 1 matvec (decode).
 * Each entry point names the reference interface it replaces (paths relative
 * to the reference tree).  Every function returns PIXHIP_OK (0) or a negative
 * PIXHIP_ERR_* code and never throws; pixhip_last_error() describes the last
 * failure on the calling thread.  Work is enqueued in order on the session's
 * stream; results are visible to the host after pixhip_synchronize(), as in
 * the Vulkan backend (src/backend_vulkan.cpp:984-987).
 *
 * Type ids are GGML's, as in src/model_types.h:10-21: Q8_0 = 8, Q5_K = 13,
 * Q6_K = 14.  Weights are row-major [rows][inner] GGUF blocks (row stride
 * weight_bytes({inner}, type), src/model.cpp:87-121); activations fp32
 * [columns][inner]; outputs fp32 [columns][rows] (src/kernels_quant.cpp:396).
 */
#ifndef PIXHIP_H
#define PIXHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PIXHIP_OK 0
#define PIXHIP_ERR_ARGUMENT (-1)    /* bad pointer, size or shape (cpu_quant_matmul's `return false`, src/kernels_quant.cpp:373-377) */
#define PIXHIP_ERR_UNSUPPORTED (-2) /* weight type other than Q8_0 / Q5_K / Q6_K; attention head size above 512 */
#define PIXHIP_ERR_MEMORY (-3)      /* device allocation failed or exceeds the budget (src/backend_vulkan.cpp:689, :718-720) */
#define PIXHIP_ERR_DEVICE (-4)      /* HIP runtime failure: no device, launch or synchronisation error */
#define PIXHIP_ERR_STATE (-5)       /* missing session, MULTIPLY without matching activations, or an evicted weight without host bytes */
#define PIXHIP_ERR_OPEN (-6)        /* the model file cannot be opened or mapped (MODEL_ERROR_OPEN, src/model.h:16) */
#define PIXHIP_ERR_FORMAT (-7)      /* not a GGUF v3 / safetensors file the reader accepts (MODEL_ERROR_FORMAT, src/model.h:17) */

#define PIXHIP_TYPE_Q8_0 8
#define PIXHIP_TYPE_Q5_K 13
#define PIXHIP_TYPE_Q6_K 14

#define PIXHIP_STAGE_QUANTIZE 1u    /* pixhip_matmul_stage: quantize the activations into session scratch */
#define PIXHIP_STAGE_MULTIPLY 2u    /* pixhip_matmul_stage: multiply the last quantized activations */

typedef struct pixhip_session pixhip_session;
typedef struct pixhip_weight pixhip_weight;

/* ---- session: VulkanSession / VulkanState (src/backend_vulkan.h:124-137) ---- */

/* VulkanSession::initialize (src/backend_vulkan.cpp:1004-1011): selects HIP
 * device `device`, creates a default-priority stream, the allocator and the
 * weight cache. */
int pixhip_session_create(int device, pixhip_session** out);

/* VulkanSession::~VulkanSession (src/backend_vulkan.cpp:1013-1016):
 * synchronises, then releases every allocation, cached weight and stream. */
void pixhip_session_destroy(pixhip_session* session);

/* No Vulkan counterpart (the Vulkan backend owns its queue): run the session
 * on a caller-owned hipStream_t instead of its own (NULL restores its own). */
int pixhip_session_set_stream(pixhip_session* session, void* stream);
void* pixhip_session_stream(pixhip_session* session);

/* VulkanSession::device_name (src/backend_vulkan.cpp:1018-1021). */
int pixhip_device_name(pixhip_session* session, char* buffer, size_t length);

/* VulkanSession::memory_limits (src/backend_vulkan.cpp:1029-1045): usable
 * device bytes and the largest single allocation. */
int pixhip_memory_limits(pixhip_session* session, uint64_t* bytes, uint64_t* range);

/* VulkanSession::prepare_stage (src/backend_vulkan.cpp:1047-1057): flush the
 * weight cache and size its budget so `activation_bytes + scratch_bytes`
 * stay available.  The budget is also capped by pixhip_set_weight_budget. */
int pixhip_prepare_stage(pixhip_session* session, uint64_t activation_bytes, uint64_t scratch_bytes);

/* VulkanSession::packed_weight_budget (src/backend_vulkan.h:136). */
int pixhip_set_weight_budget(pixhip_session* session, uint64_t bytes);

/* ---- memory: vulkan_allocate / vulkan_free / vulkan_synchronize (src/backend_vulkan.h:83-85) ---- */

/* vulkan_allocate (src/backend_vulkan.cpp:994-997 -> VulkanState::allocate
 * :683-733): device memory with reuse of freed blocks up to twice the request;
 * NULL on failure. */
void* pixhip_allocate(pixhip_session* session, size_t bytes);

/* vulkan_free (src/backend_vulkan.cpp:999-1002 -> VulkanState::release
 * :525-531): returns the block to the session pool after queued work. */
void pixhip_free(pixhip_session* session, void* pointer);

/* vulkan_synchronize (src/backend_vulkan.cpp:984-987). */
int pixhip_synchronize(pixhip_session* session);

/* Host <-> device copies on the session stream (the Vulkan backend's
 * host-coherent mappings make these implicit, src/backend_vulkan.h:87-122). */
int pixhip_copy_to_device(pixhip_session* session, void* device_dst, const void* host_src, size_t bytes);
int pixhip_copy_to_host(pixhip_session* session, void* host_dst, const void* device_src, size_t bytes);
/* Device-to-device copy, asynchronous on the session stream (activations stay
 * device-resident between ops, as tensors do in the Vulkan backend's buffers;
 * vulkan_copy_rows, src/backend_vulkan.h:151). */
int pixhip_copy_device(pixhip_session* session, void* device_dst, const void* device_src, size_t bytes);

/* ---- weights: VulkanState::weight (src/backend_vulkan.cpp:742-758) ---- */

/* Looks `key` up in the session's LRU weight cache (the reference keys it
 * "file:name:offset:bytes"); on a miss copies `bytes` host bytes of GGUF
 * blocks [rows][inner] of `type` to the device.  On first use by the GEMM
 * (columns > 1) or the matvec (columns == 1) the kernel's resident layout is
 * built from them and the device copy of the GGUF bytes is released.  The
 * handle stays valid until the session ends: eviction (budget pressure,
 * pixhip_prepare_stage) frees only the device memory, and the next call that
 * needs a layout rebuilds it from `host_bytes`.  So `host_bytes` must stay
 * readable while the handle is used, as the model file's mapping stays for
 * the reference's cache (src/backend_vulkan.cpp:742-758); a later call with
 * the same key may pass a new address of the same bytes. */
int pixhip_weight_get(pixhip_session* session, const char* key, const void* host_bytes, uint64_t bytes, uint32_t type,
                      uint64_t inner, uint64_t rows, pixhip_weight** out);

/* Number of cached weights with device memory and their resident bytes. */
int pixhip_weight_cache_info(pixhip_session* session, uint64_t* entries, uint64_t* bytes);

/* No Vulkan counterpart (residency report): the GGUF bytes of the weights
 * that hold device memory and the device bytes they hold (the Q5_K GEMM
 * layout is about 3.05x its GGUF bytes, the matvec layout 1.09x). */
int pixhip_weight_residency(pixhip_session* session, uint64_t* gguf_bytes, uint64_t* resident_bytes);

/* The type and shape a handle was created with (PixWeight::type and shape
 * {inner, rows}, src/model.h:33-39). */
int pixhip_weight_shape(const pixhip_weight* weight, uint32_t* type, uint64_t* inner, uint64_t* rows);

/* ---- model files: PixModelFile (src/model.h:41-56, src/model.cpp:87-250) ---- */

typedef struct pixhip_model pixhip_model;

/* One PixWeight (src/model.h:33-39). */
typedef struct pixhip_tensor_info {
    const char* name;   /* valid while the model is open; NUL-terminated */
    uint64_t name_length; /* bytes of the name (GGUF names may hold NUL bytes) */
    uint32_t type;      /* GGML type: F32 0, F16 1, Q8_0 8, Q5_K 13, Q6_K 14, BF16 30 */
    uint32_t rank;      /* 1..5 */
    uint64_t shape[5];  /* GGML order, first dimension contiguous; unused dimensions 0 */
    uint64_t offset;    /* absolute byte offset in the mapping */
    uint64_t bytes;     /* weight_bytes(shape, type) */
} pixhip_tensor_info;

/* PixModelFile::open (src/model.cpp:138-160) and read (:162-243): maps `path`
 * read-only and parses it as GGUF version 3 (safetensors = 0) or safetensors,
 * with the reference's acceptance rules (header within the first 64 MiB, at most
 * 1e6 tensors / metadata pairs / array items, rank 1..5, types F32 / F16 / BF16 /
 * Q8_0 / Q5_K / Q6_K with whole blocks, offsets aligned to general.alignment
 * (default 32) and inside the file, no duplicate names or keys, no overlapping
 * tensors).  PIXHIP_ERR_OPEN when the file cannot be opened or mapped,
 * PIXHIP_ERR_FORMAT when it is not accepted (MODEL_ERROR_OPEN / _FORMAT). */
int pixhip_model_open(const char* path, int safetensors, pixhip_model** out);
/* PixModelFile::close (src/model.cpp:128-136): unmaps the file. */
void pixhip_model_close(pixhip_model* model);
/* PixModelFile::data and size: the mapping. */
const unsigned char* pixhip_model_data(const pixhip_model* model, uint64_t* size);
/* PixModelFile::weights, in name order (std::map). */
uint64_t pixhip_model_tensor_count(const pixhip_model* model);
int pixhip_model_tensor_at(const pixhip_model* model, uint64_t index, pixhip_tensor_info* info);
/* PixModelFile::tensor (src/model.cpp:245-249); PIXHIP_ERR_ARGUMENT when absent. */
int pixhip_model_tensor(const pixhip_model* model, const char* name, pixhip_tensor_info* info);
/* PixModelFile::metadata, in key order: entry `index`'s key, and its value as
 * JSON text (numbers in the reference's textual form, e.g. float32 as
 * std::to_string prints it).  Each copies at most length - 1 bytes and a NUL
 * and returns the full length (call with length 0 to size a buffer), or
 * PIXHIP_ERR_ARGUMENT. */
uint64_t pixhip_model_metadata_count(const pixhip_model* model);
int64_t pixhip_model_metadata_key(const pixhip_model* model, uint64_t index, char* key, size_t length);
int64_t pixhip_model_metadata_value(const pixhip_model* model, uint64_t index, char* value, size_t length);
/* The metadata value of `key` as JSON text, as above; PIXHIP_ERR_ARGUMENT when absent. */
int64_t pixhip_model_metadata(const pixhip_model* model, const char* key, char* value, size_t length);
/* VulkanState::weight (src/backend_vulkan.cpp:742-758) for tensor `name` of an
 * open model: pixhip_weight_get with the key "file:name:offset:bytes" and the
 * mapping's bytes (a 2-D Q8_0 / Q5_K / Q6_K tensor; the model must stay open
 * while the handle is used). */
int pixhip_model_weight(pixhip_session* session, const pixhip_model* model, const char* name, pixhip_weight** out);
/* The same for a convolution weight (pixhip_conv_weight_get): tensor `name`
 * of rank 4 [kx, ky, cin, cout] or rank 5 [kx, ky, 1, cin, cout] (the checks
 * of src/convolution.cpp:60-62), type F32 / F16 / BF16. */
int pixhip_model_conv_weight(pixhip_session* session, const pixhip_model* model, const char* name, pixhip_weight** out);

/* ---- the op: vulkan_matmul / VulkanState::multiply ---- */

/* vulkan_matmul (src/backend_vulkan.h:139, src/backend_vulkan.cpp:1083-1094):
 * output[c][r] = sum_k W[r][k] * input[c][k] for c < columns, r < rows, with
 * the numerics of cpu_quant_matmul (src/kernels_quant.cpp:369-412): the
 * activations are quantized (Q8_0 for Q8_0 weights, Q8_K for K-quants) and
 * every block dot is exact in integers.  columns == 1 runs the matvec (rows
 * of up to 24576 values; longer rows and columns > 1 run the MFMA GEMM,
 * src/backend_vulkan.cpp:963-981).  `input` and
 * `output` may be device pointers (from pixhip_allocate or any HIP
 * allocation) or host pointers; host buffers are staged through the device
 * and the call then completes before returning.  Every output element is
 * written. */
int pixhip_matmul(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t columns, float* output);

/* VulkanState::multiply with the push words the convolution path uses
 * (src/backend_vulkan.cpp:1085-1091, :1186-1191): bias[rows] added when not
 * NULL (push[8]), output row stride `ldy` (push[6], 0 means rows) and element
 * offset `y_offset` (push[7]).  Device pointers only. */
int pixhip_matmul_ex(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t columns, float* output,
                     const float* bias, size_t ldy, size_t y_offset);

/* The two passes of pixhip_matmul_ex run separately (PIXHIP_STAGE_* flags),
 * for callers that reuse one quantized activation with several weights of the
 * same type and inner size, and to time the GEMM alone.  MULTIPLY without a
 * preceding QUANTIZE of a compatible shape returns PIXHIP_ERR_STATE. */
int pixhip_matmul_stage(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t columns, float* output,
                        const float* bias, size_t ldy, size_t y_offset, unsigned stages);

/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  pixhip_matmul_ex without any allocation: the quantized
 * activations go to a fixed 32 MiB device array per GPU (held until the
 * process ends) instead of session scratch, the GEMM runs without its split-K
 * workspace, and nothing is staged, so `input` and `output` must be device
 * memory.  The weight's layout must already be resident (run it once through
 * pixhip_matmul_ex with the same kind of call: columns == 1 for the matvec,
 * columns > 1 for the GEMM); otherwise PIXHIP_ERR_STATE.  Activations beyond
 * the array (Mpad*K bytes plus scales: e.g. 4096 x 3840 Q8_K takes 17.9 MB)
 * give PIXHIP_ERR_MEMORY.  Every call on one GPU shares the array: a call on
 * another stream than the previous call on that GPU first waits (on the
 * device, hipStreamWaitEvent) for that call's work, so calls from several
 * sessions or streams run one after the other there.  Results equal
 * pixhip_matmul_ex's, bit for bit where that call runs unsplit, else within
 * the fp32 rounding of the split sums.  Leaves no activations for
 * PIXHIP_STAGE_MULTIPLY. */
int pixhip_matmul_ex_noalloc(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t columns,
                             float* output, const float* bias, size_t ldy, size_t y_offset);

/* cpu_quant_matmul (src/kernels_quant.cpp:369-412) with the same argument
 * meaning: host GGUF weight bytes, input [columns][inner], output
 * [columns][rows].  Stateless like the reference: the weight is uploaded and
 * converted for this call only (nothing is cached) and the call completes
 * before returning.  Same failures: unsupported type, a zero size,
 * inner % block != 0 or inner > INT32_MAX give an error and touch nothing. */
int pixhip_quant_matmul(pixhip_session* session, const unsigned char* weights, uint32_t type, const float* input, float* output,
                        size_t rows, size_t columns, size_t inner);

/* ---- activation quantizers ---- */

/* quantize_row_q8_0_ref (src/kernels_quant.cpp:120-144) applied to `rows`
 * rows of `inner` fp32 values: writes rows*inner/32 block_q8_0 (34 B) to
 * `blocks`.  Device pointers. */
int pixhip_quantize_q8_0(pixhip_session* session, const float* input, void* blocks, size_t rows, size_t inner);

/* quantize_row_q8_K_ref (src/kernels_quant.cpp:80-118): rows*inner/256
 * block_q8_K (292 B: fp32 d, int8 qs[256], int16 bsums[16]).  Device pointers. */
int pixhip_quantize_q8_K(pixhip_session* session, const float* input, void* blocks, size_t rows, size_t inner);

/* ---- producers of a linear layer's input, fused with its quantizer ---- */

/* tensor_norm (src/tensor.cpp:174-197; vulkan_norm, src/backend_vulkan.cpp:1096-1110)
 * over `rows` rows of `inner` values: y = (float)(x - mean) * inverse * weight[c]
 * with the mean (centered != 0 only) and the mean square taken in double and
 * inverse = (float)(1 / sqrt(mean square + epsilon)); norm_weight NULL is the
 * reference's empty weight.  When `modulation` is not NULL, y is then scaled as
 * z_modulate does (src/inference.cpp:263-277): y * (1.0f + modulation[c]).
 * `type` names the weight type of the linear layers that consume y (8, 13, 14)
 * and quantizes y for them as pixhip_matmul would (Q8_0 for 8, Q8_K else) into
 * the session's activations: follow with pixhip_matmul_stage(...,
 * PIXHIP_STAGE_MULTIPLY) for each consumer of that type and inner size.
 * type 0 only normalizes (then `inner` need only be a multiple of 4; else of
 * the block size, 256 or 32).  Optional outputs (NULL to skip): `normalized` fp32
 * [rows][inner] (the tensor the reference returns), `blocks` the reference's
 * block layout (block_q8_0 / block_q8_K, as pixhip_quantize_q8_0 / _q8_K).
 * Device pointers; input, norm_weight, modulation and normalized 16-byte
 * aligned. */
int pixhip_norm_quantize(pixhip_session* session, uint32_t type, const float* input, size_t rows, size_t inner,
                         const float* norm_weight, float epsilon, int centered, const float* modulation, float* normalized,
                         void* blocks);

/* tensor_silu (src/tensor.cpp:199-209) then tensor_gate (:334-345), i.e. the
 * SwiGLU product gate = gate / (1.0f + expf(-gate)) * up in fp32 (src/
 * inference.cpp:331-335), quantized for the consumers of weight type `type`
 * as pixhip_norm_quantize does.  `gated` (NULL to skip; may equal `gate`)
 * receives the fp32 product, `blocks` the reference's block layout.  Device
 * pointers; gate, up and gated 16-byte aligned. */
int pixhip_silu_gate_quantize(pixhip_session* session, uint32_t type, const float* gate, const float* up, size_t rows,
                              size_t inner, float* gated, void* blocks);

/* ---- elementwise ops of the layer around the linears ---- */

/* Operation ids of vulkan_pointwise (src/vulkan_ops.h:24-49). */
#define PIXHIP_OP_SILU 2u        /* tensor_silu, src/tensor.cpp:199-209: v / (1.0f + expf(-v)) */
#define PIXHIP_OP_GATE 3u        /* tensor_gate, :334-345: v * second[i] */
#define PIXHIP_OP_ADD 4u         /* tensor_add, :321-332: v + second[i] */
#define PIXHIP_OP_BIAS 14u       /* tensor_bias, :226-240 (vulkan_bias): v + second[i % channels] */
#define PIXHIP_OP_GELU_EXACT 18u /* tensor_gelu(exact), :211-224: 0.5f*v*(1 + erff(v/sqrt 2)) */
#define PIXHIP_OP_GELU_TANH 19u  /* tensor_gelu(approximate): 0.5f*v*(1 + tanhf(0.7978845608f*(v + 0.044715f*v^3))) */

/* vulkan_pointwise(operation, destination, second, nullptr) (src/backend_vulkan.cpp:1112-1127)
 * and vulkan_bias: `destination` [rows][channels] updated in place with the
 * fp32 arithmetic of the CPU op named above, in its order.  `second` is
 * [rows][channels] for GATE and ADD, [channels] for BIAS, unused (NULL) for
 * SILU and GELU.  expf / erff / tanhf are correctly rounded here (glibc's are
 * within about an ulp).  `destination` is device memory or pinned host
 * memory (HipAllocator, PixTensorVals); `second` may also be pageable host
 * memory (a std::vector, as tensor_bias passes), which is staged to the device
 * first.  4-byte aligned. */
int pixhip_pointwise(pixhip_session* session, unsigned operation, float* destination, const float* second, size_t rows,
                     size_t channels);

/* tensor_rope (src/tensor.cpp:429-452; vulkan_rope, src/backend_vulkan.h:145):
 * in place on `tensor` [rows][heads * dim]; for each head and pair i < dim/2,
 * (first, second) = (2i, 2i+1) when `interleaved`, else (i, i + dim/2), and
 * (a, b) -> (a*c - b*s, a*s + b*c) with c, s = cosine, sine [rows][dim/2][i],
 * in fp32 without contraction (bit-exact).  `tensor` is device memory or
 * pinned host memory; `cosine` and `sine` may also be pageable host memory
 * (tensor_rope's std::vector tables), staged to the device first. */
int pixhip_rope(pixhip_session* session, float* tensor, size_t rows, size_t channels, size_t heads, const float* cosine,
                const float* sine, int interleaved);

/* ---- attention ---- */

/* One PixAttentionRange (src/tensor.h:58-63): query rows [query_begin,
 * query_end) see keys [0, key_end), and, when `causal`, only keys up to their
 * absolute row query_offset + row. */
typedef struct pixhip_attention_range {
    size_t query_begin, query_end, key_end;
    int causal;
} pixhip_attention_range;

/* tensor_attention(q, k, v, heads, kv_heads, causal) (src/tensor.cpp:347-382;
 * vulkan_attention, src/backend_vulkan.h:143): `output` [rows][channels] for
 * q [rows][channels] and k, v [keys][channels / heads * kv_heads], head h
 * reading kv head h / (heads / kv_heads), scale 1/sqrt(channels / heads);
 * causal rows see keys 0..row.  Head sizes 1..512 (PIXHIP_ERR_UNSUPPORTED
 * beyond; the reference's Vulkan path takes up to 1280).  Rejects
 * (PIXHIP_ERR_ARGUMENT) heads not a multiple of kv_heads, channels not a
 * multiple of heads, and causal with rows > keys (where the reference reads
 * past k).  Within 1e-4 of the fp32
 * reference per row (bf16 three-term products, fp32 softmax).  Tensors are
 * device memory or pinned host memory (q, k, v may be pageable, staged to the
 * device first), 16-byte aligned. */
int pixhip_attention(pixhip_session* session, const float* q, size_t rows, const float* k, const float* v, size_t keys,
                     size_t heads, size_t kv_heads, size_t channels, int causal, float* output);

/* tensor_attention(q, k, v, heads, kv_heads, ranges, query_offset)
 * (src/tensor.cpp:384-427; vulkan_attention, src/backend_vulkan.h:144,
 * :1318-1340): as above with per-range key limits; `ranges` must tile the
 * query rows in order with 0 < key_end <= keys (the reference's checks,
 * src/tensor.cpp:386-394, PIXHIP_ERR_ARGUMENT otherwise). */
int pixhip_attention_ranges(pixhip_session* session, const float* q, size_t rows, const float* k, const float* v, size_t keys,
                            size_t heads, size_t kv_heads, size_t channels, const pixhip_attention_range* ranges, size_t count,
                            size_t query_offset, float* output);

/* ---- the rest of the backend op surface (src/backend_vulkan.h:141-156) ----
 *
 * Tensors are row-major fp32 [rows][channels] (PixTensor, src/tensor.h:50-56).
 * Outputs and in-place tensors are device memory or pinned host memory; other
 * tensor operands may also be pageable host memory, staged to the device
 * first.  4-byte aligned (16-byte alignment and channel counts that are
 * multiples of 4 take the wider loads).  Every result is bit-identical to the
 * reference's CPU op on the same inputs, except where a comment says
 * otherwise. */

/* More operation ids of vulkan_pointwise (src/vulkan_ops.h:31-49), for
 * pixhip_pointwise_ex, and of vulkan_layout, for pixhip_layout. */
#define PIXHIP_OP_MODULATE 8u   /* z_modulate, src/inference.cpp:263-277: v * (1.0f + second[part*channels + c]) */
#define PIXHIP_OP_RESIDUAL 9u   /* z_residual, :279-291: v + second[i] * tanhf(third[part*channels + c]) (third NULL: * 1.0f) */
#define PIXHIP_OP_AFFINE 10u    /* the VAE input and sampler steps, :474-478, :612-631: v * scale + bias */
#define PIXHIP_OP_EULER 26u     /* qwen_image_euler, src/qwen_image.cpp:347-361: v + second[i] * scale */
#define PIXHIP_OP_PATCH 15u     /* inference_diffuse's patchify loop, src/inference.cpp:374-390 */
#define PIXHIP_OP_UNPATCH 16u   /* its inverse, :438-455 */
#define PIXHIP_OP_UPSAMPLE 17u  /* tensor_upsample, src/tensor.cpp:304-319 */

/* vulkan_pointwise(operation, destination, second, third, part, scale, bias)
 * (src/backend_vulkan.cpp:1112-1127) in full: the ids of pixhip_pointwise
 * (which this forwards to) plus MODULATE, RESIDUAL, AFFINE and EULER above,
 * `destination` [rows][channels] updated in place.  MODULATE reads `second`
 * values [part*channels, (part+1)*channels); RESIDUAL and EULER read `second`
 * [rows][channels], RESIDUAL also `third` (NULL: no gate) at the same slice
 * as MODULATE.  AFFINE takes only scale and bias.  tanhf is correctly rounded
 * here (glibc's is within about an ulp). */
int pixhip_pointwise_ex(pixhip_session* session, unsigned operation, float* destination, const float* second, const float* third,
                        size_t rows, size_t channels, unsigned part, float scale, float bias);

/* qwen_image_modulate (src/qwen_image.cpp:149-169; vulkan_qwen_modulate,
 * src/backend_vulkan.cpp:1418-1430): `parameters` is two rows of
 * `parameter_channels` (row 0 for the target rows >= target_begin, row 1 for
 * the rows before), p = that row's values from part * channels; without
 * `residual`, destination[r][c] *= 1 + p[c]; with it (same shape as
 * destination), destination[r][c] += residual[r][c] * tanhf(p[c]).  Rejects
 * (part + 1) * channels > parameter_channels, as the reference does. */
int pixhip_qwen_modulate(pixhip_session* session, float* destination, size_t rows, size_t channels, const float* parameters,
                         size_t parameter_channels, size_t target_begin, size_t part, const float* residual);

/* tensor_l2norm (src/tensor.cpp:242-258; vulkan_l2norm, src/backend_vulkan.cpp:
 * 1304-1316): per row, square = sum of x^2 in double, inverse =
 * (float)(sqrt(channels) / max(sqrt(square), epsilon)), y = x * inverse *
 * weight[c] (weight NULL: the empty weight).  epsilon must be > 0.  `output`
 * may equal `input`.  The double sum is formed in another order than the
 * reference's; an output differs (by an ulp) only when the two doubles fall on
 * either side of an fp32 rounding boundary. */
int pixhip_l2norm(pixhip_session* session, const float* input, size_t rows, size_t channels, const float* weight, float epsilon,
                  float* output);

/* tensor_groupnorm (src/tensor.cpp:454-485; vulkan_groupnorm, src/backend_vulkan.
 * cpp:1211-1237) with the weight and bias vectors the reference decodes from
 * the model (`name`.weight / `name`.bias): 32 groups of channels / 32
 * consecutive channels, each over all rows; mean and variance in double,
 * inverse = (float)(1 / sqrt(variance + 1e-6)), y = (float)(x - mean) *
 * inverse * weight[c] + bias[c].  channels must be a multiple of 32 (the
 * reference leaves the channels past the last whole group unwritten) and at
 * most 8192 (PIXHIP_ERR_UNSUPPORTED).  `output` may equal `input`.  The double
 * statistics are formed in another order than the reference's (chunked, then
 * merged); as for pixhip_l2norm, outputs differ only at fp32 rounding
 * boundaries. */
int pixhip_groupnorm(pixhip_session* session, const float* input, size_t rows, size_t channels, const float* weight, const float* bias,
                     float* output);

/* vulkan_embedding (src/backend_vulkan.cpp:1239-1255; the CPU path decodes
 * row by row, src/inference.cpp:184, src/qwen_vl.cpp:337): output [count][inner]
 * = rows ids[i] of `table` (table_rows GGUF rows of `inner` values of `type`:
 * F32 0, F16 1, BF16 30, Q8_0 8, Q5_K 13, Q6_K 14) decoded as cpu_decode does
 * (src/backend_cpu.cpp:24-101).  `ids` is host memory (the reference's
 * std::vector<int>); ids outside [0, table_rows) are rejected.  `table` is the
 * model file's mapping (host memory: only the selected rows are moved, as the
 * reference packs them) or device memory (gathered on the device). */
int pixhip_embedding(pixhip_session* session, const void* table, uint32_t type, uint64_t inner, uint64_t table_rows, const int32_t* ids,
                     size_t count, float* output);

/* tensor_gather / tensor_scatter (src/tensor.cpp:274-302; vulkan_rows,
 * src/backend_vulkan.cpp:1343-1357): gather (scatter = 0) writes destination
 * row i = source row rows[i] (destination_rows == count); scatter writes
 * destination row rows[i] = source row i (source_rows == count), a row listed
 * twice keeping the last, as the reference's loop does.  `rows` is host memory
 * (the reference's std::vector<size_t>); indices out of range and an empty
 * list are rejected. */
int pixhip_rows(pixhip_session* session, const float* source, size_t source_rows, float* destination, size_t destination_rows,
                size_t channels, const size_t* rows, size_t count, int scatter);

/* vulkan_copy_rows (src/backend_vulkan.cpp:1257-1269; tensor_slice,
 * src/tensor.cpp:260-272): destination rows destination_row .. + rows, all
 * destination_channels of them, = source rows source_row .. + rows from
 * feature source_feature.  The two tensors' shapes are given so that the
 * ranges are checked; they must not overlap. */
int pixhip_copy_rows(pixhip_session* session, const float* source, size_t source_rows, size_t source_channels, float* destination,
                     size_t destination_rows, size_t destination_channels, size_t rows, size_t source_row, size_t source_feature,
                     size_t destination_row);

/* vulkan_copy_features (src/backend_vulkan.cpp:1271-1281): one row of
 * source_channels values into a one-row destination from destination_feature,
 * with the reference's range checks. */
int pixhip_copy_features(pixhip_session* session, const float* source, size_t source_channels, float* destination,
                         size_t destination_channels, size_t destination_feature);

/* vulkan_layout (src/backend_vulkan.cpp:1283-1295): PATCH turns pixels
 * [width*height][C] into tokens [(width/patch)*(height/patch)][patch*patch*C]
 * (token (x, y), feature (dy*patch + dx)*C + c = pixel (x*patch + dx,
 * y*patch + dy), channel c); UNPATCH is its inverse (`width` the pixel width,
 * destination [width*height][C]); UPSAMPLE doubles a [width*height][C] image
 * by repeating each pixel 2x2 (`patch` unused).  The shapes must agree
 * (PIXHIP_ERR_ARGUMENT otherwise). */
int pixhip_layout(pixhip_session* session, unsigned operation, const float* source, size_t source_rows, size_t source_channels,
                  float* destination, size_t destination_rows, size_t destination_channels, size_t width, size_t patch);

/* tensor_resample_shortcut (src/tensor.cpp:487-527; vulkan_shortcut,
 * src/backend_vulkan.cpp:1404-1416): the Qwen VAE's parameter-free resampling
 * shortcut of a [width*height][source_channels] image into `destination`
 * [out_width*out_height][channels] (out = width*2 up, width/2 down when
 * spatial, else unchanged): up repeats channels from the last time step; down
 * averages the last time step's items of each group (fp32 sum in order, then
 * / group).  The reference's shape checks apply. */
int pixhip_shortcut(pixhip_session* session, const float* source, size_t width, size_t height, size_t source_channels,
                    float* destination, size_t channels, size_t temporal, int up, int spatial);

/* ---- convolution: vulkan_conv (src/backend_vulkan.h:146-147) ---- */

/* PixConv2D (src/tensor.h:65-68). */
typedef struct pixhip_conv_geometry {
    size_t stride_x, stride_y;
    size_t left, right, top, bottom;  /* zero padding */
} pixhip_conv_geometry;

/* The cache entry of a convolution weight (VulkanState::weight of the
 * flattened tensor, src/backend_vulkan.cpp:1195, :1388): `bytes` of a float
 * tensor (F32 0, F16 1, BF16 30) of GGML shape [kernel_x, kernel_y,
 * in_channels, out_channels] (a rank-5 [kx, ky, 1, cin, cout] tensor is the
 * same bytes), keyed like pixhip_weight_get.  On first use it is made resident
 * as two bf16 planes (hi, lo = w - hi) with the inner index reordered to
 * (ky, kx, c); F16 and BF16 weights are exact in them.  Quantized convolution
 * weights are PIXHIP_ERR_UNSUPPORTED. */
int pixhip_conv_weight_get(pixhip_session* session, const char* key, const void* host_bytes, uint64_t bytes, uint32_t type,
                           uint64_t kernel_x, uint64_t kernel_y, uint64_t in_channels, uint64_t out_channels, pixhip_weight** out);

/* tensor_conv (src/convolution.cpp:34-100; vulkan_conv, src/backend_vulkan.cpp:
 * 1177-1209, :1359-1402): `output` [out_width * out_height][out_channels] =
 * the convolution of `input` [width * height][in_channels] (pixels row-major,
 * channels innermost) with the weight, plus bias[o] when `bias` is not NULL.
 * `geometry` NULL is tensor_conv's first form (stride 1, the kernel centred at
 * offset kernel / 2, out = in); otherwise out_width = (width + left + right -
 * kernel_x) / stride_x + 1 (and likewise in y), with the reference's checks.
 * Within 1e-4 of the fp32 reference per output row (split-bf16 MFMA products,
 * fp32 accumulation).  Tensors are device or pinned host memory (input and
 * bias may be pageable), 4-byte aligned.  Images of more than 2^32 - 1 pixels
 * are PIXHIP_ERR_ARGUMENT. */
int pixhip_conv2d(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t width, size_t height,
                  const pixhip_conv_geometry* geometry, const float* bias, float* output);

/* ---- integer parity gate ---- */

/* Runs the GEMM kernel's integer path and writes, for every (column c, row r,
 * block b), the exact integer block sums the fp32 epilogue consumes:
 *   Q5_K  sums = sum_s scale_s * dot_s,  mins = sum_s min_s * (bsum_2s + bsum_2s+1)
 *         (pix_dot_q5_K's sumi and its min term, src/kernels_quant.cpp:198-245)
 *   Q6_K  sums = sum_e scale * (q - 32) * q8 (src/kernels_quant.cpp:283-331)
 *   Q8_0  sums = sum over the block of q * q8 (src/kernels_quant.cpp:353-360)
 * Layout [columns][rows][blocks] with blocks = inner/256 (K-quants) or
 * ceil(inner/64)*2 (Q8_0, the last block of an odd count is padding).
 * `mins` is only written for Q5_K.  Device pointers. */
int pixhip_block_sums(pixhip_session* session, const pixhip_weight* weight, const float* input, size_t columns, int32_t* sums,
                      int32_t* mins);

/* ---- timing (HIP events on the session stream) ---- */
int pixhip_timer_start(pixhip_session* session);
int pixhip_timer_stop(pixhip_session* session, float* milliseconds);

/* No reference counterpart (measurement support): enqueues `reps` calls of
 * pixhip_matmul_stage(weights[i % count], ...) back to back from a C loop and
 * reports the elapsed stream time between HIP events recorded before the first
 * and after the last call.  Device pointers only. */
int pixhip_bench_matmul(pixhip_session* session, const pixhip_weight* const* weights, size_t count, const float* input,
                        size_t columns, float* output, unsigned stages, size_t reps, float* milliseconds);

/* ---- diagnostics ---- */
const char* pixhip_last_error(void);
int pixhip_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PIXHIP_H */
