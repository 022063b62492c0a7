/* C++17 counterpart of src/backend_vulkan.h for the quantized linear path.
 *
 * Mirrors the reference's backend interface so that the branch in cpu_matmul
 * (src/backend_cpu.cpp:108-112) can route to HIP exactly as it routes to
 * Vulkan:
 *
 *   if (hip_active_state()) return hip_matmul(file,weight,input,columns,output);
 *
 *   HipSession          <- VulkanSession     (src/backend_vulkan.h:124-137)
 *   hip_active_state()  <- vulkan_active_state (thread_local, :82, .cpp:86)
 *   hip_allocate/free   <- vulkan_allocate/free (:83-84)
 *   hip_synchronize()   <- vulkan_synchronize (:85)
 *   HipAllocator<T>     <- VulkanAllocator<T> (:88-122)
 *   hip_matmul(...)     <- vulkan_matmul (:139)
 *
 * hip_matmul is a template over the model-file and weight types so this
 * header compiles against the reference's own PixModelFile / PixWeight
 * (src/model.h:33-56) without including them: it reads file.filename,
 * file.data, weight.name, weight.shape ({inner, rows}, GGML order),
 * weight.type, weight.offset and weight.bytes, and builds the same cache key
 * as VulkanState::weight (src/backend_vulkan.cpp:744).  No exceptions are
 * thrown (the reference builds with -fno-exceptions); failures return false.
 */
#ifndef PIXELINA_BACKEND_HIP_H
#define PIXELINA_BACKEND_HIP_H

#include <cstddef>
#include <cstdint>
#include <memory>
#include <new>
#include <string>
#include <type_traits>
#include <utility>

#include "pixhip.h"

struct HipState;  // owns one pixhip_session
std::shared_ptr<HipState> hip_active_state();
pixhip_session* hip_state_session(const std::shared_ptr<HipState> &state);
void* hip_allocate(const std::shared_ptr<HipState> &state, size_t bytes);
void hip_free(const std::shared_ptr<HipState> &state, void* pointer);
bool hip_synchronize();

// Activation buffers shared by host and device: the model code reads
// activations on the host after hip_synchronize(), as it does with the Vulkan
// backend's host-coherent mappings.  Allocates pinned host memory; the kernels
// stage it through HBM once per call (pixhip_matmul).
template <typename T> struct HipAllocator {
    using value_type = T;
    using propagate_on_container_move_assignment = std::true_type;
    std::shared_ptr<HipState> state;  // owning device lifetime, or CPU allocation mode
    HipAllocator() : state(hip_active_state()) {}
    template <typename U> HipAllocator(const HipAllocator<U> &other) : state(other.state) {}
    T* allocate(size_t count)
    {
        if (state) return static_cast<T*>(hip_allocate(state,count * sizeof(T)));
        return static_cast<T*>(::operator new(count * sizeof(T)));
    }
    void deallocate(T* pointer, size_t)
    {
        if (state) hip_free(state,pointer);
        else ::operator delete(pointer);
    }
    void construct(T* pointer)
    {
        // Output kernels overwrite every element; skip host clearing on the device path.
        if (state) ::new (static_cast<void*>(pointer)) T;
        else ::new (static_cast<void*>(pointer)) T();
    }
    template <typename... Args> void construct(T* pointer, Args&&... args)
    {
        ::new (static_cast<void*>(pointer)) T(std::forward<Args>(args)...);
    }
    template <typename U> bool operator==(const HipAllocator<U> &other) const { return state == other.state; }
    template <typename U> bool operator!=(const HipAllocator<U> &other) const { return state != other.state; }
};

class HipSession {
    std::shared_ptr<HipState> state;  // independent HIP context
public:
    HipSession() = default;
    ~HipSession();
    HipSession(const HipSession &) = delete;
    HipSession &operator=(const HipSession &) = delete;

    bool initialize(int device = 0);  // fails if a session is already active on this thread
    std::string device_name() const;
    bool memory_limits(uint64_t &bytes, uint64_t &range) const;
    bool prepare_stage(uint64_t activation_bytes, uint64_t scratch_bytes);

    uint64_t packed_weight_budget = UINT64_MAX;  // per-job cache admission after device planning
};

// The active session's cached weight for (filename, name, offset, bytes);
// nullptr when no session is active or the upload fails.
pixhip_weight* hip_weight(const std::string &key, const void* host_bytes, uint64_t bytes, uint32_t type, uint64_t inner,
                          uint64_t rows);
bool hip_matmul_weight(pixhip_weight* weight, const float* input, size_t columns, float* output);

// The cached device form of one weight of a model file, keyed as
// VulkanState::weight keys it (src/backend_vulkan.cpp:744).
template <class File, class Weight>
pixhip_weight* hip_weight_of(const File &file, const Weight &weight)
{
    if (weight.shape.size() != 2) return nullptr;
    const std::string key = file.filename + ":" + weight.name + ":" + std::to_string(weight.offset) + ":" + std::to_string(weight.bytes);
    return hip_weight(key,file.data + weight.offset,weight.bytes,weight.type,weight.shape[0],weight.shape[1]);
}

template <class File, class Weight>
bool hip_matmul(const File &file, const Weight &weight, const float* input, size_t columns, float* output)
{
    pixhip_weight* w = hip_weight_of(file,weight);
    return w && hip_matmul_weight(w,input,columns,output);
}

// Producers of a linear layer's input fused with its quantizer (no Vulkan
// counterpart: there tensor_norm / tensor_silu + tensor_gate run as their own
// ops and each tensor_linear quantizes its input again).
//
// hip_norm_multiply: tensor_norm (src/tensor.cpp:174-197), then z_modulate
// (src/inference.cpp:263-277) when `modulation` is not null, feeding `count`
// linear layers that share the weight-type class of `type` and `channels`
// inputs (e.g. the DiT block's FFN gate and up, src/inference.cpp:331-332):
// the normalized rows are quantized once and every weight's GEMM reads them.
// outputs[i] receives [rows][rows of weight i]; `normalized` (may be null) the
// fp32 tensor the reference returns.  norm_weight / modulation are host
// vectors of `channels` floats (as tensor_vector returns them), or null.
bool hip_norm_multiply(uint32_t type, pixhip_weight* const* weights, float* const* outputs, size_t count, const float* input,
                       size_t rows, size_t channels, const float* norm_weight, float epsilon, bool centered,
                       const float* modulation, float* normalized);

// hip_silu_gate_multiply: tensor_silu(gate) then tensor_gate(gate, up)
// (src/tensor.cpp:199-209, :334-345) feeding the linear `down`
// (src/inference.cpp:333-336): output [rows][rows of down]; `gated` (may be
// null, may equal gate) receives the fp32 product.
bool hip_silu_gate_multiply(uint32_t type, pixhip_weight* down, const float* gate, const float* up, size_t rows, size_t channels,
                            float* output, float* gated);

// vulkan_pointwise(operation, destination, second, nullptr) and vulkan_bias
// (src/backend_vulkan.h:142, :150) for PIXHIP_OP_SILU / GATE / ADD / BIAS /
// GELU_EXACT / GELU_TANH, and vulkan_rope (:145), on the active session's
// stream: in place on `destination` [rows][channels].
bool hip_pointwise(unsigned operation, float* destination, const float* second, size_t rows, size_t channels);
bool hip_rope(float* tensor, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, bool interleaved);

// vulkan_attention (src/backend_vulkan.h:143-144) for tensor_attention
// (src/tensor.cpp:347-427): output [rows][channels] from q [rows][channels] and
// k, v [keys][channels / heads * kv_heads], on the active session's stream.
// The ranges form takes the reference's PixAttentionRange fields as
// pixhip_attention_range.  False (with pixhip_last_error) on what the backend
// does not take (head sizes above 512) or rejects, as vulkan_attention returns
// an empty tensor.
bool hip_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                   size_t channels, bool causal, float* output);
bool hip_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                   size_t channels, const pixhip_attention_range* ranges, size_t count, size_t query_offset, float* output);

// The rest of vulkan_*'s op surface (src/backend_vulkan.h:141-156) on the
// active session, each the pixhip_ entry point of the same name over the
// tensors' value pointers (PixTensorVals under a session; pageable vectors are
// staged).  False (with pixhip_last_error) on what the backend rejects, so the
// caller falls back to its CPU code.
bool hip_pointwise_ex(unsigned operation, float* destination, const float* second, const float* third, size_t rows, size_t channels,
                      unsigned part, float scale, float bias);
bool hip_qwen_modulate(float* destination, size_t rows, size_t channels, const float* parameters, size_t parameter_channels,
                       size_t target_begin, size_t part, const float* residual);
bool hip_l2norm(const float* input, size_t rows, size_t channels, const float* weight, float epsilon, float* output);
bool hip_groupnorm(const float* input, size_t rows, size_t channels, const float* weight, const float* bias, float* output);
bool hip_embedding(const void* table, uint32_t type, uint64_t inner, uint64_t table_rows, const int32_t* ids, size_t count,
                   float* output);
bool hip_rows(const float* source, size_t source_rows, float* destination, size_t destination_rows, size_t channels, const size_t* rows,
              size_t count, bool scatter);
bool hip_copy_rows(const float* source, size_t source_rows, size_t source_channels, float* destination, size_t destination_rows,
                   size_t destination_channels, size_t rows, size_t source_row, size_t source_feature, size_t destination_row);
bool hip_copy_features(const float* source, size_t source_channels, float* destination, size_t destination_channels,
                       size_t destination_feature);
bool hip_layout(unsigned operation, const float* source, size_t source_rows, size_t source_channels, float* destination,
                size_t destination_rows, size_t destination_channels, size_t width, size_t patch);
bool hip_shortcut(const float* source, size_t width, size_t height, size_t source_channels, float* destination, size_t channels,
                  size_t temporal, bool up, bool spatial);

// vulkan_conv (src/backend_vulkan.h:146-147): the cached convolution weight of
// a model file's float tensor [kx, ky, cin, cout] (rank 5 with a unit third
// dimension accepted), keyed as hip_weight_of keys linear weights, and the
// convolution itself (geometry NULL: tensor_conv's first form).
pixhip_weight* hip_conv_weight(const std::string &key, const void* host_bytes, uint64_t bytes, uint32_t type, uint64_t kernel_x,
                               uint64_t kernel_y, uint64_t in_channels, uint64_t out_channels);
bool hip_conv2d(pixhip_weight* weight, const float* input, size_t width, size_t height, const pixhip_conv_geometry* geometry,
                const float* bias, float* output);

template <class File, class Weight>
pixhip_weight* hip_conv_weight_of(const File &file, const Weight &weight)
{
    const size_t rank = weight.shape.size();
    if ((rank != 4 && rank != 5) || (rank == 5 && weight.shape[2] != 1)) return nullptr;
    const std::string key = file.filename + ":" + weight.name + ":" + std::to_string(weight.offset) + ":" + std::to_string(weight.bytes);
    return hip_conv_weight(key,file.data + weight.offset,weight.bytes,weight.type,weight.shape[0],weight.shape[1],weight.shape[rank - 2],
                           weight.shape[rank - 1]);
}

bool hip_available(std::string &description);

#endif /* PIXELINA_BACKEND_HIP_H */
