// Implementation of the C++ shim declared in backend_hip.h, over the C ABI.
#include "backend_hip.h"

#include <hip/hip_runtime.h>

#include <map>
#include <utility>
#include <vector>

// Pinned host blocks handed to HipAllocator vectors.  A freed block may still
// be read or written by queued work, so hip_free does not wait: it records an
// event on the session stream and parks the block; once the event has
// completed the block returns to a pool that later allocations reuse (as the
// reference defers a release to the last submission that used the buffer,
// src/backend_vulkan.cpp:525-531).  The pool is trimmed past kPoolLimit.
struct HipState {
    static constexpr size_t kPoolLimit = size_t(1) << 30;
    pixhip_session* session = nullptr;
    std::vector<std::pair<hipEvent_t,std::pair<void*,size_t>>> pending;  // freed, maybe still in use
    std::multimap<size_t,void*> pool;                                     // free and idle
    std::map<void*,size_t> sizes;                                         // every live or pooled block
    size_t pooled = 0;

    // Moves the blocks whose last use has completed into the pool.
    void reap()
    {
        size_t keep = 0;
        for (size_t i = 0; i < pending.size(); i++) {
            hipError_t e = hipEventQuery(pending[i].first);
            if (e == hipErrorNotReady) {
                pending[keep++] = pending[i];
                continue;
            }
            (void)hipGetLastError();
            (void)hipEventDestroy(pending[i].first);
            pool.emplace(pending[i].second.second,pending[i].second.first);
            pooled += pending[i].second.second;
        }
        pending.resize(keep);
        while (pooled > kPoolLimit && !pool.empty()) {
            auto largest = std::prev(pool.end());
            pooled -= largest->first;
            sizes.erase(largest->second);
            (void)hipHostFree(largest->second);
            pool.erase(largest);
        }
    }

    ~HipState()
    {
        if (session) (void)pixhip_synchronize(session);
        for (auto& p : pending) {
            (void)hipEventDestroy(p.first);
            (void)hipHostFree(p.second.first);
        }
        for (auto& p : pool) (void)hipHostFree(p.second);
        if (session) pixhip_session_destroy(session);
    }
};

// One session per inference thread, as the reference's thread_local
// active_state (src/backend_vulkan.cpp:86).
static thread_local std::shared_ptr<HipState> active_state;

std::shared_ptr<HipState> hip_active_state()
{
    return active_state;
}

pixhip_session* hip_state_session(const std::shared_ptr<HipState> &state)
{
    return state? state->session : nullptr;
}

void* hip_allocate(const std::shared_ptr<HipState> &state, size_t bytes)
{
    if (!state) return nullptr;
    if (!bytes) bytes = 4;
    state->reap();
    auto hit = state->pool.lower_bound(bytes);
    if (hit != state->pool.end() && hit->first <= 2 * bytes) {  // reuse up to twice the request
        void* p = hit->second;
        state->pooled -= hit->first;
        state->pool.erase(hit);
        return p;
    }
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p,bytes,hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    state->sizes[p] = bytes;
    return p;
}

void hip_free(const std::shared_ptr<HipState> &state, void* pointer)
{
    if (!state || !pointer) return;
    auto it = state->sizes.find(pointer);
    if (it == state->sizes.end()) return;  // not ours
    hipEvent_t done = nullptr;
    if (hipEventCreateWithFlags(&done,hipEventDisableTiming) != hipSuccess ||
        hipEventRecord(done,static_cast<hipStream_t>(pixhip_session_stream(state->session))) != hipSuccess) {
        // No event: wait for the queued work instead.
        (void)hipGetLastError();
        if (done) (void)hipEventDestroy(done);
        (void)pixhip_synchronize(state->session);
        state->pool.emplace(it->second,pointer);
        state->pooled += it->second;
    } else {
        state->pending.push_back({done,{pointer,it->second}});
    }
    state->reap();
}

bool hip_synchronize()
{
    if (!active_state) return true;
    const bool ok = pixhip_synchronize(active_state->session) == PIXHIP_OK;
    active_state->reap();
    return ok;
}

bool HipSession::initialize(int device)
{
    if (active_state) return false;
    auto fresh = std::make_shared<HipState>();
    if (pixhip_session_create(device,&fresh->session) != PIXHIP_OK) return false;
    state = fresh;
    active_state = state;
    return true;
}

HipSession::~HipSession()
{
    if (active_state == state) active_state.reset();
}

std::string HipSession::device_name() const
{
    char name[256] = {0};
    if (!state || pixhip_device_name(state->session,name,sizeof(name)) != PIXHIP_OK) return std::string();
    return name;
}

bool HipSession::memory_limits(uint64_t &bytes, uint64_t &range) const
{
    return state && pixhip_memory_limits(state->session,&bytes,&range) == PIXHIP_OK && bytes != 0;
}

bool HipSession::prepare_stage(uint64_t activation_bytes, uint64_t scratch_bytes)
{
    if (!state) return false;
    if (pixhip_set_weight_budget(state->session,packed_weight_budget) != PIXHIP_OK) return false;
    return pixhip_prepare_stage(state->session,activation_bytes,scratch_bytes) == PIXHIP_OK;
}

pixhip_weight* hip_weight(const std::string &key, const void* host_bytes, uint64_t bytes, uint32_t type, uint64_t inner,
                          uint64_t rows)
{
    if (!active_state) return nullptr;
    pixhip_weight* w = nullptr;
    if (pixhip_weight_get(active_state->session,key.c_str(),host_bytes,bytes,type,inner,rows,&w) != PIXHIP_OK) return nullptr;
    return w;
}

bool hip_matmul_weight(pixhip_weight* weight, const float* input, size_t columns, float* output)
{
    return active_state && pixhip_matmul(active_state->session,weight,input,columns,output) == PIXHIP_OK;
}

namespace {

// A device copy of a host vector for the duration of one call (null stays null).
struct DeviceVector {
    pixhip_session* s;
    void* p = nullptr;
    bool ok = true;
    DeviceVector(pixhip_session* session, const float* host, size_t count) : s(session)
    {
        if (!host) return;
        p = pixhip_allocate(s,count * sizeof(float));
        ok = p && pixhip_copy_to_device(s,p,host,count * sizeof(float)) == PIXHIP_OK;
    }
    ~DeviceVector()
    {
        if (p) pixhip_free(s,p);
    }
    const float* get() const { return static_cast<const float*>(p); }
};

// The GEMM of the session's last quantized activations with `w` into a host
// (or device) output of rows x `rows of w` floats.
bool multiply_into(pixhip_session* s, pixhip_weight* w, size_t rows, size_t out_rows, float* output)
{
    const size_t bytes = rows * out_rows * sizeof(float);
    void* dev = pixhip_allocate(s,bytes);
    if (!dev) return false;
    bool ok = pixhip_matmul_stage(s,w,nullptr,rows,static_cast<float*>(dev),nullptr,0,0,PIXHIP_STAGE_MULTIPLY) == PIXHIP_OK &&
              pixhip_copy_to_host(s,output,dev,bytes) == PIXHIP_OK;
    pixhip_free(s,dev);
    return ok;
}

uint64_t weight_rows(const pixhip_weight* w)
{
    uint32_t type = 0;
    uint64_t inner = 0, rows = 0;
    return pixhip_weight_shape(w,&type,&inner,&rows) == PIXHIP_OK? rows : 0;
}

}  // namespace

bool hip_norm_multiply(uint32_t type, pixhip_weight* const* weights, float* const* outputs, size_t count, const float* input,
                       size_t rows, size_t channels, const float* norm_weight, float epsilon, bool centered,
                       const float* modulation, float* normalized)
{
    pixhip_session* s = hip_state_session(active_state);
    if (!s || !weights || !outputs) return false;
    DeviceVector w(s,norm_weight,channels), m(s,modulation,channels);
    if (!w.ok || !m.ok) return false;
    if (pixhip_norm_quantize(s,type,input,rows,channels,w.get(),epsilon,centered? 1 : 0,m.get(),normalized,nullptr) != PIXHIP_OK)
        return false;
    for (size_t i = 0; i < count; i++) {
        const uint64_t n = weights[i]? weight_rows(weights[i]) : 0;
        if (!n || !multiply_into(s,weights[i],rows,n,outputs[i])) return false;
    }
    return true;
}

bool hip_silu_gate_multiply(uint32_t type, pixhip_weight* down, const float* gate, const float* up, size_t rows, size_t channels,
                            float* output, float* gated)
{
    pixhip_session* s = hip_state_session(active_state);
    if (!s || !down) return false;
    const uint64_t n = weight_rows(down);
    if (!n || pixhip_silu_gate_quantize(s,type,gate,up,rows,channels,gated,nullptr) != PIXHIP_OK) return false;
    return multiply_into(s,down,rows,n,output);
}

bool hip_pointwise(unsigned operation, float* destination, const float* second, size_t rows, size_t channels)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_pointwise(s,operation,destination,second,rows,channels) == PIXHIP_OK;
}

bool hip_rope(float* tensor, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, bool interleaved)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_rope(s,tensor,rows,channels,heads,cosine,sine,interleaved? 1 : 0) == PIXHIP_OK;
}

bool hip_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                   size_t channels, bool causal, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_attention(s,q,rows,k,v,keys,heads,kv_heads,channels,causal? 1 : 0,output) == PIXHIP_OK;
}

bool hip_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                   size_t channels, const pixhip_attention_range* ranges, size_t count, size_t query_offset, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_attention_ranges(s,q,rows,k,v,keys,heads,kv_heads,channels,ranges,count,query_offset,output) == PIXHIP_OK;
}

bool hip_pointwise_ex(unsigned operation, float* destination, const float* second, const float* third, size_t rows, size_t channels,
                      unsigned part, float scale, float bias)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_pointwise_ex(s,operation,destination,second,third,rows,channels,part,scale,bias) == PIXHIP_OK;
}

bool hip_qwen_modulate(float* destination, size_t rows, size_t channels, const float* parameters, size_t parameter_channels,
                       size_t target_begin, size_t part, const float* residual)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_qwen_modulate(s,destination,rows,channels,parameters,parameter_channels,target_begin,part,residual) == PIXHIP_OK;
}

bool hip_l2norm(const float* input, size_t rows, size_t channels, const float* weight, float epsilon, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_l2norm(s,input,rows,channels,weight,epsilon,output) == PIXHIP_OK;
}

bool hip_groupnorm(const float* input, size_t rows, size_t channels, const float* weight, const float* bias, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_groupnorm(s,input,rows,channels,weight,bias,output) == PIXHIP_OK;
}

bool hip_embedding(const void* table, uint32_t type, uint64_t inner, uint64_t table_rows, const int32_t* ids, size_t count, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_embedding(s,table,type,inner,table_rows,ids,count,output) == PIXHIP_OK;
}

bool hip_rows(const float* source, size_t source_rows, float* destination, size_t destination_rows, size_t channels, const size_t* rows,
              size_t count, bool scatter)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_rows(s,source,source_rows,destination,destination_rows,channels,rows,count,scatter? 1 : 0) == PIXHIP_OK;
}

bool hip_copy_rows(const float* source, size_t source_rows, size_t source_channels, float* destination, size_t destination_rows,
                   size_t destination_channels, size_t rows, size_t source_row, size_t source_feature, size_t destination_row)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_copy_rows(s,source,source_rows,source_channels,destination,destination_rows,destination_channels,rows,source_row,
                                 source_feature,destination_row) == PIXHIP_OK;
}

bool hip_copy_features(const float* source, size_t source_channels, float* destination, size_t destination_channels,
                       size_t destination_feature)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_copy_features(s,source,source_channels,destination,destination_channels,destination_feature) == PIXHIP_OK;
}

bool hip_layout(unsigned operation, const float* source, size_t source_rows, size_t source_channels, float* destination,
                size_t destination_rows, size_t destination_channels, size_t width, size_t patch)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_layout(s,operation,source,source_rows,source_channels,destination,destination_rows,destination_channels,width,
                              patch) == PIXHIP_OK;
}

bool hip_shortcut(const float* source, size_t width, size_t height, size_t source_channels, float* destination, size_t channels,
                  size_t temporal, bool up, bool spatial)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && pixhip_shortcut(s,source,width,height,source_channels,destination,channels,temporal,up? 1 : 0,spatial? 1 : 0) == PIXHIP_OK;
}

pixhip_weight* hip_conv_weight(const std::string &key, const void* host_bytes, uint64_t bytes, uint32_t type, uint64_t kernel_x,
                               uint64_t kernel_y, uint64_t in_channels, uint64_t out_channels)
{
    pixhip_session* s = hip_state_session(active_state);
    pixhip_weight* w = nullptr;
    if (!s || pixhip_conv_weight_get(s,key.c_str(),host_bytes,bytes,type,kernel_x,kernel_y,in_channels,out_channels,&w) != PIXHIP_OK)
        return nullptr;
    return w;
}

bool hip_conv2d(pixhip_weight* weight, const float* input, size_t width, size_t height, const pixhip_conv_geometry* geometry,
                const float* bias, float* output)
{
    pixhip_session* s = hip_state_session(active_state);
    return s && weight && pixhip_conv2d(s,weight,input,width,height,geometry,bias,output) == PIXHIP_OK;
}

bool hip_available(std::string &description)
{
    HipSession session;
    if (!session.initialize()) {
        description = "HIP initialization failed.";
        return false;
    }
    description = session.device_name();
    return true;
}
