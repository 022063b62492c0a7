// C ABI of the HIP backend (include/pixhip.h): session, pooled device
// allocator, LRU weight cache with upload-time conversion, and the dispatch of
// VulkanState::multiply (src/backend_vulkan.cpp:963-981): M == 1 -> matvec,
// M > 1 -> activation quantize + MFMA GEMM.  Nothing here throws; every HIP
// status is checked and turned into a PIXHIP_ERR_* code.
#include "pixhip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>

#include "pixhip_internal.h"

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& message)
{
    g_error = message;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(PIXHIP_ERR_DEVICE,std::string(what) + ": " + hipGetErrorString(e));
}

#define PIX_HIP(expr, what)                               \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return hip_fail(e_,what);   \
    } while (0)

size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

constexpr size_t kTileN = PIX_GEMM_NTILE;  // GEMM feature-tile rows (weight padding)
constexpr size_t kTileM = PIX_GEMM_MTILE;  // GEMM token-tile rows (activation padding)
constexpr size_t kAlign = 256;       // sub-allocation alignment
constexpr double kHeapFraction = 0.85;  // VULKAN_HEAP_FRACTION, src/backend_vulkan.h:26
constexpr size_t kPipeChunks = 8;          // row chunks of a matmul on host operands
constexpr size_t kPipeMinColumns = 2 * kTileM;  // (fewer rows: one staged pass)
constexpr size_t kMatvecMaxInner = 24576;  // matvec keeps x in LDS and a row in registers (64 units per lane x 6)

bool supported_type(uint32_t t) { return t == PIX_Q8_0 || t == PIX_Q5_K || t == PIX_Q6_K; }
size_t block_values(uint32_t t) { return t == PIX_Q8_0? PIX_QK8 : PIX_QK; }
size_t block_bytes(uint32_t t) { return t == PIX_Q8_0? PIX_Q8_0_BYTES : (t == PIX_Q5_K? PIX_Q5_K_BYTES : PIX_Q6_K_BYTES); }

// Carves one device allocation into aligned sub-buffers.
struct Carver {
    size_t offset = 0;
    size_t take(size_t bytes)
    {
        size_t at = offset;
        offset = round_up(offset + bytes,kAlign);
        return at;
    }
};

// The allocation-free GEMM entry point (pixhip_matmul_ex_noalloc) keeps the
// quantized activations in this fixed device array instead of session
// scratch.  Each device holds its own copy until the process ends; host code
// reaches it only through the per-device address from hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
// Calls from different streams share a device's array: each call records
// g_scratch_event on its stream, and a call on another stream than the last
// one waits for that event first, so the calls run one after the other.
hipEvent_t g_scratch_event[kMaxDevices] = {};
hipStream_t g_scratch_stream[kMaxDevices] = {};
bool g_scratch_used[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// Resolves, once per device (the device current), the address of that
// device's copy of `scratch`.
int scratch_setup(int device)
{
    if (device < 0 || device >= kMaxDevices) return fail(PIXHIP_ERR_ARGUMENT,"device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device]) return PIXHIP_OK;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p,HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(PIXHIP_ERR_DEVICE,std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev,hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(PIXHIP_ERR_DEVICE,std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e));
    }
    g_scratch_event[device] = ev;
    g_scratch_ptr[device] = p;
    return PIXHIP_OK;
}

}  // namespace

// One cached weight.  The record lives until the session ends, so a handle
// never dangles: eviction frees only its device memory, and the next use
// rebuilds what it needs from the host bytes (as VulkanState::weight re-reads
// the model file's mapping, src/backend_vulkan.cpp:742-758).
struct pixhip_weight {
    std::string key;
    uint32_t type = 0;
    uint64_t inner = 0, rows = 0, gguf_bytes = 0;
    const void* host = nullptr; // the caller's GGUF bytes (re-read to rebuild a form)
    void* raw = nullptr;        // device copy of the GGUF bytes, only while a form is built from it
    void* planes = nullptr;     // GEMM form (built on first GEMM use)
    void* planar = nullptr;     // matvec form (built on first matvec use)
    pixhip::PlanesQ5K q5{};
    pixhip::PlanesQ6K q6{};
    pixhip::PlanarQ80 q80{};
    pixhip::PlanarQ5K q5p{};
    pixhip::PlanarQ6K q6p{};
    size_t resident = 0;
    uint64_t used = 0;
    // convolution weights (F32 / F16 / BF16, [cout][cin * ky * kx]): the
    // split-bf16 planes the implicit GEMM reads, built on first use
    bool conv = false;
    uint32_t kernel_x = 0, kernel_y = 0, cin = 0;
    void* conv_planes = nullptr;
    size_t conv_kp = 0, conv_npad = 0;
};

struct pixhip_session {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    std::string name;
    size_t total_memory = 0;
    size_t heap_limit = 0;
    // allocator (VulkanState::allocate / release / trim)
    std::map<uintptr_t,size_t> live;
    std::multimap<size_t,void*> pool;
    size_t pooled_bytes = 0;
    // weight cache (VulkanState::weight / evict)
    std::unordered_map<std::string,pixhip_weight*> weights;
    size_t cache_bytes = 0, cache_limit = 0, budget = SIZE_MAX;
    uint64_t uses = 0;
    // quantized-activation scratch
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // split-K partial outputs of small GEMM grids
    void* partial = nullptr;
    size_t partial_bytes = 0;
    // staging for host or misaligned pointers
    void* stage = nullptr;
    size_t stage_bytes = 0;
    // attention's bf16 split planes
    void* attn = nullptr;
    size_t attn_bytes = 0;
    // groupnorm's chunk statistics
    void* gn = nullptr;
    size_t gn_bytes = 0;
    // matmul on host operands: copy streams (input, output) and the chunks' events
    hipStream_t pipe_in = nullptr, pipe_out = nullptr;
    hipEvent_t pipe_ev[2 * kPipeChunks + 1] = {};
    // activations left by the last QUANTIZE stage
    int act_kind = 0;  // 0 none, 1 Q8_K, 2 Q8_0
    size_t act_columns = 0, act_inner = 0;
    pixhip::Act8K a8k{};
    pixhip::Act80 a80{};
};

namespace {

int use_device(pixhip_session* s)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    PIX_HIP(hipSetDevice(s->device),"hipSetDevice");
    return PIXHIP_OK;
}

// Frees a weight's device memory (the record and its handle stay valid).
// Callers synchronise the stream first when queued work may still read it.
void release_forms(pixhip_session* s, pixhip_weight* w)
{
    if (w->raw) (void)hipFree(w->raw);
    if (w->planes) (void)hipFree(w->planes);
    if (w->planar) (void)hipFree(w->planar);
    if (w->conv_planes) (void)hipFree(w->conv_planes);
    w->raw = w->planes = w->planar = w->conv_planes = nullptr;
    w->q5 = {};
    w->q6 = {};
    w->q80 = {};
    w->q5p = {};
    w->q6p = {};
    s->cache_bytes -= w->resident;
    w->resident = 0;
}

// VulkanState::evict (src/backend_vulkan.cpp:671-681): least recently used first.
bool evict_one(pixhip_session* s, const pixhip_weight* keep)
{
    pixhip_weight* victim = nullptr;
    for (auto& e : s->weights) {
        pixhip_weight* w = e.second;
        if (w == keep || !w->resident) continue;
        if (!victim || w->used < victim->used) victim = w;
    }
    if (!victim) return false;
    (void)hipStreamSynchronize(s->stream);
    release_forms(s,victim);
    return true;
}

void trim_pool(pixhip_session* s)
{
    for (auto& e : s->pool) (void)hipFree(e.second);
    s->pool.clear();
    s->pooled_bytes = 0;
}

// Device allocation for cache forms: evicts older weights, then trims the
// pool, when the budget or the device refuses.
int weight_alloc(pixhip_session* s, pixhip_weight* w, size_t bytes, void** out)
{
    while (s->cache_bytes + bytes > s->cache_limit && evict_one(s,w)) {}
    if (s->cache_bytes + bytes > s->cache_limit)
        return fail(PIXHIP_ERR_MEMORY,"weight exceeds the cache budget (" + std::to_string(s->cache_limit) + " bytes)");
    hipError_t e = hipMalloc(out,bytes);
    while (e != hipSuccess && (evict_one(s,w) || s->pooled_bytes)) {
        (void)hipGetLastError();
        if (s->pooled_bytes) trim_pool(s);
        e = hipMalloc(out,bytes);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *out = nullptr;
        return fail(PIXHIP_ERR_MEMORY,"hipMalloc of " + std::to_string(bytes) + " weight bytes failed");
    }
    w->resident += bytes;
    s->cache_bytes += bytes;
    return PIXHIP_OK;
}

int grow(pixhip_session* s, void** buffer, size_t* have, size_t need)
{
    if (*have >= need) return PIXHIP_OK;
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    if (*buffer) (void)hipFree(*buffer);
    *buffer = nullptr;
    *have = 0;
    hipError_t e = hipMalloc(buffer,need);
    if (e != hipSuccess && s->pooled_bytes) {
        (void)hipGetLastError();
        trim_pool(s);
        e = hipMalloc(buffer,need);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *buffer = nullptr;
        return fail(PIXHIP_ERR_MEMORY,"hipMalloc of " + std::to_string(need) + " scratch bytes failed");
    }
    *have = need;
    return PIXHIP_OK;
}

// A device copy of the GGUF bytes, for building a form.
int ensure_raw(pixhip_session* s, pixhip_weight* w)
{
    if (w->raw) return PIXHIP_OK;
    if (!w->host) return fail(PIXHIP_ERR_STATE,"weight " + w->key + " was evicted and has no host bytes to rebuild from");
    int rc = weight_alloc(s,w,round_up(w->gguf_bytes,kAlign),&w->raw);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(w->raw,w->host,w->gguf_bytes,hipMemcpyHostToDevice,s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e,"weight upload");
    return PIXHIP_OK;
}

// The device GGUF copy is released once a form has been built from it (the
// forms are all the kernels read); another form needed later re-reads the host
// bytes.
int release_raw(pixhip_session* s, pixhip_weight* w)
{
    if (!w->raw) return PIXHIP_OK;
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");  // the repack kernels read it
    (void)hipFree(w->raw);
    w->raw = nullptr;
    const size_t bytes = round_up(w->gguf_bytes,kAlign);
    w->resident -= bytes;
    s->cache_bytes -= bytes;
    return PIXHIP_OK;
}

// GEMM forms, built on first use from the GGUF bytes.
int ensure_gemm_form(pixhip_session* s, pixhip_weight* w)
{
    if (w->planes) return PIXHIP_OK;
    int rc0 = ensure_raw(s,w);
    if (rc0) return rc0;
    const size_t N = w->rows, K = w->inner, npad = round_up(N,kTileN), nb = K / PIX_QK;
    if (w->type == PIX_Q5_K && !w->planes) {
        Carver c;
        size_t hi = c.take(npad * K), lo = c.take(npad * K), d = c.take(nb * npad * 4), dm = c.take(nb * npad * 4),
               mn = c.take(nb * npad * 8 * 2);
        int rc = weight_alloc(s,w,c.offset,&w->planes);
        if (rc) return rc;
        uint8_t* base = static_cast<uint8_t*>(w->planes);
        PIX_HIP(hipMemsetAsync(base,0,c.offset,s->stream),"hipMemsetAsync");
        w->q5 = {reinterpret_cast<int8_t*>(base + hi),reinterpret_cast<int8_t*>(base + lo),reinterpret_cast<float*>(base + d),
                 reinterpret_cast<float*>(base + dm),reinterpret_cast<_Float16*>(base + mn),npad};
        PIX_HIP(pixhip::launch_repack_q5_K(static_cast<const uint8_t*>(w->raw),N,K,npad,const_cast<int8_t*>(w->q5.hi),
                                           const_cast<int8_t*>(w->q5.lo),const_cast<float*>(w->q5.d),const_cast<float*>(w->q5.dm),
                                           const_cast<_Float16*>(w->q5.mn),s->stream),
                "repack Q5_K");
    }
    if (w->type == PIX_Q8_0 && !w->planes) {
        const size_t kp = round_up(K,64);
        Carver c;
        size_t qs = c.take(npad * kp), dT = c.take((kp / PIX_QK8) * npad * 4);
        int rc = weight_alloc(s,w,c.offset,&w->planes);
        if (rc) return rc;
        uint8_t* base = static_cast<uint8_t*>(w->planes);
        PIX_HIP(hipMemsetAsync(base,0,c.offset,s->stream),"hipMemsetAsync");
        w->q80.qs = reinterpret_cast<int8_t*>(base + qs);
        w->q80.dT = reinterpret_cast<float*>(base + dT);
        PIX_HIP(pixhip::launch_repack_q8_0(static_cast<const uint8_t*>(w->raw),N,K,kp,npad,const_cast<int8_t*>(w->q80.qs),
                                           const_cast<float*>(w->q80.dT),nullptr,nullptr,s->stream),
                "repack Q8_0 (GEMM)");
    }
    if (w->type == PIX_Q6_K && !w->planes) {
        Carver c;
        size_t hi = c.take(npad * K), lo = c.take(npad * K), d = c.take(nb * npad * 4);
        int rc = weight_alloc(s,w,c.offset,&w->planes);
        if (rc) return rc;
        uint8_t* base = static_cast<uint8_t*>(w->planes);
        PIX_HIP(hipMemsetAsync(base,0,c.offset,s->stream),"hipMemsetAsync");
        w->q6 = {reinterpret_cast<int8_t*>(base + hi),reinterpret_cast<int8_t*>(base + lo),reinterpret_cast<float*>(base + d),npad};
        PIX_HIP(pixhip::launch_repack_q6_K_planes(static_cast<const uint8_t*>(w->raw),N,K,npad,const_cast<int8_t*>(w->q6.hi),
                                                  const_cast<int8_t*>(w->q6.lo),const_cast<float*>(w->q6.d),s->stream),
                "repack Q6_K planes");
    }
    return release_raw(s,w);
}

int build_matvec_form(pixhip_session* s, pixhip_weight* w);

int ensure_matvec_form(pixhip_session* s, pixhip_weight* w)
{
    if (w->planar) return PIXHIP_OK;
    int rc = ensure_raw(s,w);
    if (!rc) rc = build_matvec_form(s,w);
    if (!rc) rc = release_raw(s,w);
    return rc;
}

int build_matvec_form(pixhip_session* s, pixhip_weight* w)
{
    const size_t N = w->rows, K = w->inner, nb = K / PIX_QK;
    if (w->type == PIX_Q8_0) {
        const size_t kp = round_up(K,64);
        Carver c;
        size_t qs = c.take(N * kp), d = c.take(N * (kp / PIX_QK8) * 2);
        int rc = weight_alloc(s,w,c.offset,&w->planar);
        if (rc) return rc;
        uint8_t* base = static_cast<uint8_t*>(w->planar);
        PIX_HIP(hipMemsetAsync(base,0,c.offset,s->stream),"hipMemsetAsync");  // the padding unit's half
        w->q80.qs_mv = reinterpret_cast<int8_t*>(base + qs);
        w->q80.d = reinterpret_cast<_Float16*>(base + d);
        PIX_HIP(pixhip::launch_repack_q8_0(static_cast<const uint8_t*>(w->raw),N,K,kp,0,nullptr,nullptr,const_cast<int8_t*>(w->q80.qs_mv),
                                           const_cast<_Float16*>(w->q80.d),s->stream),
                "repack Q8_0 (matvec)");
        return PIXHIP_OK;
    }
    if (w->type == PIX_Q5_K) {
        Carver c;
        size_t qs = c.take(N * K / 2), rec = c.take(N * (K / 64) * 12);
        int rc = weight_alloc(s,w,c.offset,&w->planar);
        if (rc) return rc;
        uint8_t* base = static_cast<uint8_t*>(w->planar);
        w->q5p = {base + qs,reinterpret_cast<const uint32_t*>(base + rec)};
        PIX_HIP(pixhip::launch_repack_q5_K_planar(static_cast<const uint8_t*>(w->raw),N,K,const_cast<uint8_t*>(w->q5p.qs),
                                                  const_cast<uint32_t*>(w->q5p.rec),s->stream),
                "repack Q5_K planar");
        return PIXHIP_OK;
    }
    Carver c;
    size_t ql = c.take(N * K / 2), qh = c.take(N * K / 4), sc = c.take(N * K / 16), d = c.take(N * nb * 2);
    int rc = weight_alloc(s,w,c.offset,&w->planar);
    if (rc) return rc;
    uint8_t* base = static_cast<uint8_t*>(w->planar);
    w->q6p = {base + ql,base + qh,reinterpret_cast<int8_t*>(base + sc),reinterpret_cast<_Float16*>(base + d)};
    PIX_HIP(pixhip::launch_repack_q6_K_planar(static_cast<const uint8_t*>(w->raw),N,K,const_cast<uint8_t*>(w->q6p.ql),
                                              const_cast<uint8_t*>(w->q6p.qh),const_cast<int8_t*>(w->q6p.sc),
                                              const_cast<_Float16*>(w->q6p.d),s->stream),
            "repack Q6_K planar");
    return PIXHIP_OK;
}


int check_shape(uint32_t type, uint64_t inner, uint64_t rows)
{
    if (!supported_type(type)) return fail(PIXHIP_ERR_UNSUPPORTED,"unsupported weight type " + std::to_string(type));
    if (!inner || !rows || inner % block_values(type) || inner > INT32_MAX || rows > INT32_MAX)
        return fail(PIXHIP_ERR_ARGUMENT,"bad weight shape inner=" + std::to_string(inner) + " rows=" + std::to_string(rows));
    return PIXHIP_OK;
}

// Resolve a caller pointer to one the kernels may dereference: our own
// allocations and HIP device / managed memory pass through; host memory
// (pageable or pinned) is staged through HBM once instead of being re-read
// over PCIe by every tile.
bool device_visible(pixhip_session* s, const void* p, const void** dev)
{
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = s->live.upper_bound(a);
    if (it != s->live.begin()) {
        --it;
        if (a < it->first + it->second) {
            *dev = p;
            return true;
        }
    }
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr,p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) {
        *dev = attr.devicePointer? attr.devicePointer : p;
        return true;
    }
    return false;
}

// A sized operand must lie within one allocation: the session's own block
// when p is inside one, else the allocation HIP reports for p.  Pointers HIP
// does not know (pageable host memory) pass here and are staged or rejected
// by the caller.
int check_span(pixhip_session* s, const void* p, size_t bytes)
{
    if (!p || !bytes) return PIXHIP_OK;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = s->live.upper_bound(a);
    if (it != s->live.begin()) {
        --it;
        if (a < it->first + it->second) {
            if (bytes > it->first + it->second - a)
                return fail(PIXHIP_ERR_ARGUMENT,"an operand of " + std::to_string(bytes) + " bytes runs past the end of its allocation");
            return PIXHIP_OK;
        }
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base,&size,const_cast<void*>(p)) == hipSuccess && base) {
        const uintptr_t b = reinterpret_cast<uintptr_t>(base);
        if (a >= b && a - b <= size && bytes > size - (a - b))
            return fail(PIXHIP_ERR_ARGUMENT,"an operand of " + std::to_string(bytes) + " bytes runs past the end of its allocation");
        return PIXHIP_OK;
    }
    (void)hipGetLastError();
    return PIXHIP_OK;
}

// A read-only operand of an elementwise op: device memory (ours, HIP device or
// managed) and mapped pinned host memory are passed to the kernel as they
// are; pageable host memory, which a kernel must not dereference, is copied to
// a device block first (returned in *staged, freed by the caller after the
// launch: the pool reuses it only for work queued after this op).  With
// `stage_pinned`, pinned host memory is copied too (for kernels that read
// their input more than once).
int read_operand(pixhip_session* s, const void* p, size_t bytes, const void** dev, void** staged, bool stage_pinned = false)
{
    *staged = nullptr;
    if (int rc = check_span(s,p,bytes)) return rc;
    if (device_visible(s,p,dev)) return PIXHIP_OK;
    hipPointerAttribute_t attr;
    const bool pinned = hipPointerGetAttributes(&attr,p) == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer;
    if (!pinned) (void)hipGetLastError();
    if (pinned && !stage_pinned) {
        *dev = attr.devicePointer;
        return PIXHIP_OK;
    }
    void* block = pixhip_allocate(s,bytes);
    if (!block) return fail(PIXHIP_ERR_MEMORY,"staging of a host operand failed");
    hipError_t e = hipMemcpyAsync(block,p,bytes,hipMemcpyHostToDevice,s->stream);
    // Pageable memory may change after return, so its copy completes first;
    // pinned memory is the caller's until the next synchronisation, as when
    // the kernels read it in place.
    if (e == hipSuccess && !pinned) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        pixhip_free(s,block);
        return hip_fail(e,"staging of a host operand");
    }
    *dev = block;
    *staged = block;
    return PIXHIP_OK;
}

// The in-place tensor (or output) of an op, `bytes` long: device or mapped
// pinned memory only.
int write_operand(pixhip_session* s, void* p, size_t bytes, void** dev)
{
    if (int rc = check_span(s,p,bytes)) return rc;
    const void* d = nullptr;
    if (device_visible(s,p,&d)) {
        *dev = const_cast<void*>(d);
        return PIXHIP_OK;
    }
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr,p) == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer) {
        *dev = attr.devicePointer;
        return PIXHIP_OK;
    }
    (void)hipGetLastError();
    return fail(PIXHIP_ERR_ARGUMENT,"the tensor is pageable host memory: pass device memory (pixhip_allocate) or pinned host memory");
}

// Sizes the session's activation scratch for `columns` rows of K values of
// activation kind 1 (Q8_K) or 2 (Q8_0) and points s->a8k / s->a80 into it.
// The activations then belong to the next MULTIPLY stages (set_act_shape).
int act_buffers(pixhip_session* s, int kind, size_t columns, size_t K, pixhip::ActOut* out)
{
    const size_t mpad = round_up(columns,kTileM);
    Carver c;
    uint8_t* base;
    if (kind == 2) {
        const size_t kp = round_up(K,64);
        size_t qs = c.take(mpad * kp), d = c.take((kp / PIX_QK8) * mpad * 4);
        int rc = grow(s,&s->scratch,&s->scratch_bytes,c.offset);
        if (rc) return rc;
        base = static_cast<uint8_t*>(s->scratch);
        s->a80 = {reinterpret_cast<int8_t*>(base + qs),reinterpret_cast<float*>(base + d),mpad};
        if (out) *out = {s->a80.qs,s->a80.d,nullptr,mpad,nullptr,nullptr};
    } else {
        size_t qs = c.take(mpad * K), d = c.take((K / PIX_QK) * mpad * 4), bs = c.take(mpad * (K / 16) * 2);
        int rc = grow(s,&s->scratch,&s->scratch_bytes,c.offset);
        if (rc) return rc;
        base = static_cast<uint8_t*>(s->scratch);
        s->a8k = {reinterpret_cast<int8_t*>(base + qs),reinterpret_cast<float*>(base + d),reinterpret_cast<_Float16*>(base + bs),mpad};
        if (out) *out = {s->a8k.qs,s->a8k.d,s->a8k.bs,mpad,nullptr,nullptr};
    }
    s->act_kind = 0;  // until the producer is enqueued
    return PIXHIP_OK;
}

void set_act_shape(pixhip_session* s, int kind, size_t columns, size_t K)
{
    s->act_kind = kind;
    s->act_columns = columns;
    s->act_inner = K;
}

int quantize_stage(pixhip_session* s, const pixhip_weight* w, const float* x, size_t columns)
{
    const size_t K = w->inner;
    const int kind = w->type == PIX_Q8_0? 2 : 1;
    int rc = act_buffers(s,kind,columns,K,nullptr);
    if (rc) return rc;
    if (kind == 2) PIX_HIP(pixhip::launch_quantize_q8_0(x,columns,K,round_up(K,64),s->a80,nullptr,s->stream),"quantize Q8_0");
    else PIX_HIP(pixhip::launch_quantize_q8_K(x,columns,K,s->a8k,nullptr,s->stream),"quantize Q8_K");
    set_act_shape(s,kind,columns,K);
    return PIXHIP_OK;
}

int multiply_stage(pixhip_session* s, pixhip_weight* w, size_t columns, const pixhip::Output& out)
{
    const int kind = w->type == PIX_Q8_0? 2 : 1;
    if (s->act_kind != kind || s->act_columns != columns || s->act_inner != w->inner)
        return fail(PIXHIP_ERR_STATE,"no quantized activations of this shape: run the QUANTIZE stage first");
    int rc = ensure_gemm_form(s,w);
    if (rc) return rc;
    const size_t part_bytes = kind == 2 && pixhip::gemm_q8_0_grouped(columns,w->rows)
                                  ? 0
                                  : pixhip::gemm_split_bytes(columns,w->rows,round_up(w->inner,64));
    if (part_bytes) {
        rc = grow(s,&s->partial,&s->partial_bytes,part_bytes);
        if (rc) return rc;
    }
    float* part = part_bytes? static_cast<float*>(s->partial) : nullptr;
    hipError_t e;
    if (w->type == PIX_Q5_K) e = pixhip::launch_gemm_q5_K(s->a8k,w->q5,columns,w->rows,w->inner,out,part,s->stream);
    else if (w->type == PIX_Q6_K) e = pixhip::launch_gemm_q6_K(s->a8k,w->q6,columns,w->rows,w->inner,out,part,s->stream);
    else e = pixhip::launch_gemm_q8_0(s->a80,w->q80,columns,w->rows,w->inner,out,part,s->stream);
    PIX_HIP(e,"GEMM launch");
    return PIXHIP_OK;
}

bool matvec_ok(const pixhip_weight* w)
{
    return w->inner <= kMatvecMaxInner;
}

int matvec(pixhip_session* s, pixhip_weight* w, const float* x, const pixhip::Output& out)
{
    hipError_t e;
    if (w->type == PIX_Q5_K) {
        int rc = ensure_matvec_form(s,w);
        if (rc) return rc;
        e = pixhip::launch_matvec_q5_K(w->q5p,x,w->rows,w->inner,out,s->stream);
    } else if (w->type == PIX_Q8_0) {
        int rc = ensure_matvec_form(s,w);
        if (rc) return rc;
        e = pixhip::launch_matvec_q8_0(w->q80,x,w->rows,w->inner,out,s->stream);
    } else {
        int rc = ensure_matvec_form(s,w);
        if (rc) return rc;
        e = pixhip::launch_matvec_q6_K(w->q6p,x,w->rows,w->inner,out,s->stream);
    }
    PIX_HIP(e,"matvec launch");
    return PIXHIP_OK;
}

// Quantize + GEMM of a matmul whose input and output are host memory, in row
// chunks on three streams: chunk c's input is copied to HBM on pipe_in, then
// quantized and multiplied on the session stream (after that copy's event),
// then its output copied back on pipe_out (after the GEMM's event).  PCIe
// carries input chunks in one direction and output chunks in the other at the
// same time, and each chunk's GEMM runs under the copies of its neighbours.
// Every chunk starts at a multiple of the GEMM token tile, so its quantized
// activations are a view of the session's buffers for all rows (which they
// hold afterwards, as after an unchunked call) and its GEMM reads that view.
// Taken only when the chunks' GEMMs and the whole one run the same kernel
// form with no split-K, so every output is the same bits either way.
size_t pipe_chunk(size_t columns) { return round_up((columns + kPipeChunks - 1) / kPipeChunks,kTileM); }

bool pipeline_ok(const pixhip_weight* w, size_t columns)
{
    if (columns < kPipeMinColumns) return false;
    const size_t N = w->rows, Kr = round_up(w->inner,64), chunk = pipe_chunk(columns);
    const size_t last = columns - (columns - 1) / chunk * chunk;
    for (size_t m : {columns,chunk,last})
        if (pixhip::gemm_split_bytes(m,N,Kr)) return false;
    if (w->type == PIX_Q8_0) {
        const bool g = pixhip::gemm_q8_0_grouped(columns,N);
        if (pixhip::gemm_q8_0_grouped(chunk,N) != g || pixhip::gemm_q8_0_grouped(last,N) != g) return false;
    }
    return true;
}

int run_pipelined(pixhip_session* s, pixhip_weight* w, const float* input, size_t columns, float* output, const float* bias)
{
    const size_t K = w->inner, N = w->rows;
    const int kind = w->type == PIX_Q8_0? 2 : 1;
    const size_t chunk = pipe_chunk(columns);
    const size_t chunks = (columns + chunk - 1) / chunk;
    if (!s->pipe_in) PIX_HIP(hipStreamCreate(&s->pipe_in),"hipStreamCreate");
    if (!s->pipe_out) PIX_HIP(hipStreamCreate(&s->pipe_out),"hipStreamCreate");
    for (hipEvent_t& e : s->pipe_ev)
        if (!e) PIX_HIP(hipEventCreateWithFlags(&e,hipEventDisableTiming),"hipEventCreate");
    int rc = ensure_gemm_form(s,w);
    if (rc) return rc;
    const size_t in_region = round_up(columns * K * sizeof(float),kAlign);
    if ((rc = grow(s,&s->stage,&s->stage_bytes,in_region + columns * N * sizeof(float)))) return rc;
    if ((rc = act_buffers(s,kind,columns,K,nullptr))) return rc;
    float* xs = static_cast<float*>(s->stage);
    float* ys = reinterpret_cast<float*>(static_cast<uint8_t*>(s->stage) + in_region);
    // the staging buffers are free once the work already on the session stream is done
    hipEvent_t start = s->pipe_ev[2 * kPipeChunks];
    PIX_HIP(hipEventRecord(start,s->stream),"hipEventRecord");
    PIX_HIP(hipStreamWaitEvent(s->pipe_in,start,0),"hipStreamWaitEvent");
    for (size_t c = 0; c < chunks; c++) {
        const size_t r0 = c * chunk, rows = std::min(chunk,columns - r0);
        hipEvent_t in_done = s->pipe_ev[2 * c], out_ready = s->pipe_ev[2 * c + 1];
        PIX_HIP(hipMemcpyAsync(xs + r0 * K,input + r0 * K,rows * K * sizeof(float),hipMemcpyHostToDevice,s->pipe_in),"stage input");
        PIX_HIP(hipEventRecord(in_done,s->pipe_in),"hipEventRecord");
        PIX_HIP(hipStreamWaitEvent(s->stream,in_done,0),"hipStreamWaitEvent");
        const pixhip::Output out = {ys + r0 * N,bias,N,0};
        float* const part = nullptr;  // (no split-K: pipeline_ok)
        hipError_t e;
        if (kind == 2) {
            const size_t kp = round_up(K,64);
            const pixhip::Act80 a = {s->a80.qs + r0 * kp,s->a80.d + r0,s->a80.mpad};
            PIX_HIP(pixhip::launch_quantize_q8_0(xs + r0 * K,rows,K,kp,a,nullptr,s->stream),"quantize Q8_0");
            e = pixhip::launch_gemm_q8_0(a,w->q80,rows,N,K,out,part,s->stream);
        } else {
            // tiled planes: rows r0.. (r0 a multiple of 32) start r0*K bytes in, the
            // 16-value sums r0*K/16 elements in; the scales r0 columns in
            const pixhip::Act8K a = {s->a8k.qs + r0 * K,s->a8k.d + r0,s->a8k.bs + r0 * (K / 16),s->a8k.mpad};
            PIX_HIP(pixhip::launch_quantize_q8_K(xs + r0 * K,rows,K,a,nullptr,s->stream),"quantize Q8_K");
            e = w->type == PIX_Q5_K? pixhip::launch_gemm_q5_K(a,w->q5,rows,N,K,out,part,s->stream)
                                   : pixhip::launch_gemm_q6_K(a,w->q6,rows,N,K,out,part,s->stream);
        }
        PIX_HIP(e,"GEMM launch");
        PIX_HIP(hipEventRecord(out_ready,s->stream),"hipEventRecord");
        PIX_HIP(hipStreamWaitEvent(s->pipe_out,out_ready,0),"hipStreamWaitEvent");
        PIX_HIP(hipMemcpyAsync(output + r0 * N,ys + r0 * N,rows * N * sizeof(float),hipMemcpyDeviceToHost,s->pipe_out),"copy output");
    }
    set_act_shape(s,kind,columns,K);
    // pipe_out waited for the last GEMM, which waited for the last input copy
    PIX_HIP(hipStreamSynchronize(s->pipe_out),"hipStreamSynchronize");
    return PIXHIP_OK;
}

int run(pixhip_session* s, const pixhip_weight* wc, const float* input, size_t columns, float* output, const float* bias,
        size_t ldy, size_t y_offset, unsigned stages, bool allow_host)
{
    int rc = use_device(s);
    if (rc) return rc;
    pixhip_weight* w = const_cast<pixhip_weight*>(wc);
    if (!w) return fail(PIXHIP_ERR_ARGUMENT,"null weight handle");
    if (w->conv) return fail(PIXHIP_ERR_UNSUPPORTED,"a convolution weight: use pixhip_conv2d");
    if (!columns || (stages & PIXHIP_STAGE_MULTIPLY && !output) || (stages & PIXHIP_STAGE_QUANTIZE && !input))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or zero columns");
    if (!stages || stages > (PIXHIP_STAGE_QUANTIZE | PIXHIP_STAGE_MULTIPLY)) return fail(PIXHIP_ERR_ARGUMENT,"bad stage flags");
    if (!ldy) ldy = w->rows;
    if (ldy < w->rows) return fail(PIXHIP_ERR_ARGUMENT,"output stride smaller than rows");
    w->used = ++s->uses;
    const size_t K = w->inner;
    const size_t in_bytes = columns * K * sizeof(float);
    const size_t out_elems = y_offset + (columns - 1) * ldy + w->rows;
    if ((stages & PIXHIP_STAGE_QUANTIZE && (rc = check_span(s,input,in_bytes))) ||
        (stages & PIXHIP_STAGE_MULTIPLY && (rc = check_span(s,output,out_elems * sizeof(float)))) ||
        (bias && (rc = check_span(s,bias,w->rows * sizeof(float)))))
        return rc;

    // Resolve pointers; stage host or misaligned inputs and host outputs.
    const void* xin = nullptr;
    void* yout = nullptr;
    bool stage_in = false, stage_out = false;
    if (stages & PIXHIP_STAGE_QUANTIZE) {
        if (!device_visible(s,input,&xin)) {
            if (!allow_host) return fail(PIXHIP_ERR_ARGUMENT,"input is not device memory");
            stage_in = true;
        } else if (reinterpret_cast<uintptr_t>(xin) % 16) {
            stage_in = true;
        }
    }
    if (stages & PIXHIP_STAGE_MULTIPLY) {
        const void* yv = nullptr;
        if (!device_visible(s,output,&yv)) {
            if (!allow_host) return fail(PIXHIP_ERR_ARGUMENT,"output is not device memory");
            stage_out = true;
        } else {
            yout = const_cast<void*>(yv);
        }
    }
    if (stage_in && !xin && stage_out && stages == (PIXHIP_STAGE_QUANTIZE | PIXHIP_STAGE_MULTIPLY) && ldy == w->rows && !y_offset &&
        pipeline_ok(w,columns))
        return run_pipelined(s,w,input,columns,output,bias);
    const size_t in_region = stage_in? round_up(in_bytes,kAlign) : 0;
    if (stage_in || stage_out) {
        rc = grow(s,&s->stage,&s->stage_bytes,in_region + (stage_out? out_elems * sizeof(float) : 0));
        if (rc) return rc;
    }
    if (stage_in) {
        uint8_t* dst = static_cast<uint8_t*>(s->stage);
        if (xin) PIX_HIP(hipMemcpyAsync(dst,xin,in_bytes,hipMemcpyDeviceToDevice,s->stream),"stage input");
        else PIX_HIP(hipMemcpyAsync(dst,input,in_bytes,hipMemcpyHostToDevice,s->stream),"stage input");
        xin = dst;
    }
    if (stage_out) {
        yout = static_cast<uint8_t*>(s->stage) + in_region;
        if (ldy != w->rows || y_offset)  // preserve the untouched gaps of a strided host output
            PIX_HIP(hipMemcpyAsync(yout,output,out_elems * sizeof(float),hipMemcpyHostToDevice,s->stream),"stage output");
    }
    const pixhip::Output out = {static_cast<float*>(yout),bias,ldy,y_offset};
    const float* x = static_cast<const float*>(xin);

    if (columns == 1 && stages == (PIXHIP_STAGE_QUANTIZE | PIXHIP_STAGE_MULTIPLY) && matvec_ok(w)) {
        rc = matvec(s,w,x,out);
    } else {
        rc = PIXHIP_OK;
        if (stages & PIXHIP_STAGE_QUANTIZE) rc = quantize_stage(s,w,x,columns);
        if (!rc && (stages & PIXHIP_STAGE_MULTIPLY)) rc = multiply_stage(s,w,columns,out);
    }
    if (rc) return rc;
    if (stage_out) {
        PIX_HIP(hipMemcpyAsync(output,yout,out_elems * sizeof(float),hipMemcpyDeviceToHost,s->stream),"copy output");
    }
    if (stage_in || stage_out) PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    return PIXHIP_OK;
}

}  // namespace

extern "C" {

int pixhip_version(void) { return 100; }

const char* pixhip_last_error(void) { return g_error.c_str(); }

int pixhip_session_create(int device, pixhip_session** out)
{
    if (!out) return fail(PIXHIP_ERR_ARGUMENT,"null output");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return fail(PIXHIP_ERR_DEVICE,"no HIP device available");
    }
    if (device < 0 || device >= count) return fail(PIXHIP_ERR_ARGUMENT,"device index out of range");
    PIX_HIP(hipSetDevice(device),"hipSetDevice");
    pixhip_session* s = new (std::nothrow) pixhip_session();
    if (!s) return fail(PIXHIP_ERR_MEMORY,"host allocation failed");
    s->device = device;
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop,device)) != hipSuccess || (e = hipStreamCreate(&s->own_stream)) != hipSuccess ||
        (e = hipEventCreate(&s->t0)) != hipSuccess || (e = hipEventCreate(&s->t1)) != hipSuccess) {
        int rc = hip_fail(e,"session setup");
        pixhip_session_destroy(s);
        return rc;
    }
    s->stream = s->own_stream;
    if (int rc = scratch_setup(device)) {
        pixhip_session_destroy(s);
        return rc;
    }
    // hipDeviceProp_t::name can be empty (no marketing name in the driver's
    // table); fall back to the architecture name alone.
    s->name = prop.name[0]? std::string(prop.name) + " (" + prop.gcnArchName + ")" : std::string(prop.gcnArchName);
    s->total_memory = prop.totalGlobalMem;
    s->heap_limit = (size_t)(kHeapFraction * (double)prop.totalGlobalMem);
    s->cache_limit = s->heap_limit;
    *out = s;
    return PIXHIP_OK;
}

void pixhip_session_destroy(pixhip_session* s)
{
    if (!s) return;
    (void)hipSetDevice(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    for (auto& e : s->weights) {
        release_forms(s,e.second);
        delete e.second;
    }
    s->weights.clear();
    trim_pool(s);
    for (auto& e : s->live) (void)hipFree(reinterpret_cast<void*>(e.first));
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->partial) (void)hipFree(s->partial);
    if (s->stage) (void)hipFree(s->stage);
    if (s->attn) (void)hipFree(s->attn);
    if (s->gn) (void)hipFree(s->gn);
    if (s->t0) (void)hipEventDestroy(s->t0);
    if (s->t1) (void)hipEventDestroy(s->t1);
    for (hipEvent_t e : s->pipe_ev)
        if (e) (void)hipEventDestroy(e);
    if (s->pipe_in) (void)hipStreamDestroy(s->pipe_in);
    if (s->pipe_out) (void)hipStreamDestroy(s->pipe_out);
    if (s->own_stream) (void)hipStreamDestroy(s->own_stream);
    delete s;
}

int pixhip_session_set_stream(pixhip_session* s, void* stream)
{
    int rc = use_device(s);
    if (rc) return rc;
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    s->stream = stream? static_cast<hipStream_t>(stream) : s->own_stream;
    return PIXHIP_OK;
}

void* pixhip_session_stream(pixhip_session* s) { return s? static_cast<void*>(s->stream) : nullptr; }

int pixhip_device_name(pixhip_session* s, char* buffer, size_t length)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    if (!buffer || !length) return fail(PIXHIP_ERR_ARGUMENT,"empty buffer");
    std::strncpy(buffer,s->name.c_str(),length - 1);
    buffer[length - 1] = 0;
    return PIXHIP_OK;
}

int pixhip_memory_limits(pixhip_session* s, uint64_t* bytes, uint64_t* range)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t free_b = 0, total_b = 0;
    PIX_HIP(hipMemGetInfo(&free_b,&total_b),"hipMemGetInfo");
    if (bytes) *bytes = std::min<uint64_t>(s->heap_limit,free_b);
    if (range) *range = total_b;
    return PIXHIP_OK;
}

int pixhip_prepare_stage(pixhip_session* s, uint64_t activation_bytes, uint64_t scratch_bytes)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (activation_bytes > s->heap_limit || scratch_bytes > s->heap_limit - activation_bytes)
        return fail(PIXHIP_ERR_MEMORY,"stage does not fit the device heap");
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    for (auto& e : s->weights) release_forms(s,e.second);  // handles stay valid; their forms are rebuilt on use
    trim_pool(s);
    size_t held = s->scratch_bytes + s->stage_bytes;
    for (auto& e : s->live) held += e.second;
    const uint64_t reserve = std::max<uint64_t>(held,activation_bytes + scratch_bytes);
    if (reserve >= s->heap_limit) return fail(PIXHIP_ERR_MEMORY,"no room left for weights");
    s->cache_limit = (size_t)std::min<uint64_t>(s->budget,s->heap_limit - reserve);
    return s->cache_limit? PIXHIP_OK : fail(PIXHIP_ERR_MEMORY,"empty weight budget");
}

int pixhip_set_weight_budget(pixhip_session* s, uint64_t bytes)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    s->budget = (size_t)std::min<uint64_t>(bytes,SIZE_MAX);
    s->cache_limit = std::min(s->cache_limit,s->budget);
    return PIXHIP_OK;
}

void* pixhip_allocate(pixhip_session* s, size_t bytes)
{
    if (use_device(s)) return nullptr;
    bytes = round_up(bytes? bytes : 4,kAlign);
    auto hit = s->pool.lower_bound(bytes);
    if (hit != s->pool.end() && hit->first <= 2 * bytes) {
        void* p = hit->second;
        s->live.emplace(reinterpret_cast<uintptr_t>(p),hit->first);
        s->pooled_bytes -= hit->first;
        s->pool.erase(hit);
        return p;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p,bytes);
    if (e != hipSuccess && s->pooled_bytes) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(s->stream);
        trim_pool(s);
        e = hipMalloc(&p,bytes);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(PIXHIP_ERR_MEMORY,"hipMalloc of " + std::to_string(bytes) + " bytes failed");
        return nullptr;
    }
    s->live.emplace(reinterpret_cast<uintptr_t>(p),bytes);
    return p;
}

void pixhip_free(pixhip_session* s, void* p)
{
    if (!s || !p) return;
    auto it = s->live.find(reinterpret_cast<uintptr_t>(p));
    if (it == s->live.end()) return;
    // Work already queued on the session stream finishes before anything that
    // reuses the block is queued behind it.
    s->pool.emplace(it->second,p);
    s->pooled_bytes += it->second;
    s->live.erase(it);
}

int pixhip_synchronize(pixhip_session* s)
{
    int rc = use_device(s);
    if (rc) return rc;
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    return PIXHIP_OK;
}

int pixhip_copy_to_device(pixhip_session* s, void* dst, const void* src, size_t bytes)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!bytes) return PIXHIP_OK;
    if (!dst || !src) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    PIX_HIP(hipMemcpyAsync(dst,src,bytes,hipMemcpyHostToDevice,s->stream),"hipMemcpyAsync");
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    return PIXHIP_OK;
}

int pixhip_copy_device(pixhip_session* s, void* dst, const void* src, size_t bytes)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!bytes) return PIXHIP_OK;
    if (!dst || !src) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    PIX_HIP(pixhip::launch_copy_device(dst,src,bytes,s->stream),"device copy");
    return PIXHIP_OK;
}

int pixhip_copy_to_host(pixhip_session* s, void* dst, const void* src, size_t bytes)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!bytes) return PIXHIP_OK;
    if (!dst || !src) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    PIX_HIP(hipMemcpyAsync(dst,src,bytes,hipMemcpyDeviceToHost,s->stream),"hipMemcpyAsync");
    PIX_HIP(hipStreamSynchronize(s->stream),"hipStreamSynchronize");
    return PIXHIP_OK;
}

int pixhip_weight_get(pixhip_session* s, const char* key, const void* host_bytes, uint64_t bytes, uint32_t type, uint64_t inner,
                      uint64_t rows, pixhip_weight** out)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!key || !out) return fail(PIXHIP_ERR_ARGUMENT,"null key or output");
    *out = nullptr;
    if ((rc = check_shape(type,inner,rows))) return rc;
    const uint64_t expect = rows * (inner / block_values(type)) * block_bytes(type);
    auto it = s->weights.find(key);
    if (it != s->weights.end()) {
        pixhip_weight* w = it->second;
        if (w->conv || w->type != type || w->inner != inner || w->rows != rows)
            return fail(PIXHIP_ERR_ARGUMENT,"cached key with another shape");
        if (host_bytes) {
            if (bytes < expect) return fail(PIXHIP_ERR_ARGUMENT,"weight bytes shorter than rows*row_bytes");
            w->host = host_bytes;  // the caller's current mapping of the same bytes
        }
        w->used = ++s->uses;
        *out = w;
        return PIXHIP_OK;
    }
    if (!host_bytes || bytes < expect) return fail(PIXHIP_ERR_ARGUMENT,"weight bytes missing or shorter than rows*row_bytes");
    pixhip_weight* w = new (std::nothrow) pixhip_weight();
    if (!w) return fail(PIXHIP_ERR_MEMORY,"host allocation failed");
    w->key = key;
    w->type = type;
    w->inner = inner;
    w->rows = rows;
    w->gguf_bytes = expect;
    w->host = host_bytes;
    w->used = ++s->uses;
    // Upload now (the reference uploads on first use too): the forms are built
    // from this copy on their first use, then it is released.
    if ((rc = ensure_raw(s,w))) {
        release_forms(s,w);
        delete w;
        return rc;
    }
    s->weights.emplace(w->key,w);
    *out = w;
    return PIXHIP_OK;
}

int pixhip_weight_cache_info(pixhip_session* s, uint64_t* entries, uint64_t* bytes)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    uint64_t n = 0;
    for (auto& e : s->weights) n += e.second->resident? 1 : 0;
    if (entries) *entries = n;
    if (bytes) *bytes = s->cache_bytes;
    return PIXHIP_OK;
}

int pixhip_weight_residency(pixhip_session* s, uint64_t* gguf_bytes, uint64_t* resident_bytes)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    uint64_t g = 0, r = 0;
    for (auto& e : s->weights) {
        if (!e.second->resident) continue;
        g += e.second->gguf_bytes;
        r += e.second->resident;
    }
    if (gguf_bytes) *gguf_bytes = g;
    if (resident_bytes) *resident_bytes = r;
    return PIXHIP_OK;
}

int pixhip_weight_shape(const pixhip_weight* w, uint32_t* type, uint64_t* inner, uint64_t* rows)
{
    if (!w || !type || !inner || !rows) return fail(PIXHIP_ERR_ARGUMENT,"null weight handle or output pointer");
    *type = w->type;
    *inner = w->inner;
    *rows = w->rows;
    return PIXHIP_OK;
}

int pixhip_matmul(pixhip_session* s, const pixhip_weight* w, const float* input, size_t columns, float* output)
{
    return run(s,w,input,columns,output,nullptr,0,0,PIXHIP_STAGE_QUANTIZE | PIXHIP_STAGE_MULTIPLY,true);
}

int pixhip_matmul_ex(pixhip_session* s, const pixhip_weight* w, const float* input, size_t columns, float* output, const float* bias,
                     size_t ldy, size_t y_offset)
{
    return run(s,w,input,columns,output,bias,ldy,y_offset,PIXHIP_STAGE_QUANTIZE | PIXHIP_STAGE_MULTIPLY,false);
}

int pixhip_matmul_stage(pixhip_session* s, const pixhip_weight* w, const float* input, size_t columns, float* output,
                        const float* bias, size_t ldy, size_t y_offset, unsigned stages)
{
    return run(s,w,input,columns,output,bias,ldy,y_offset,stages,false);
}

int pixhip_matmul_ex_noalloc(pixhip_session* s, const pixhip_weight* wc, const float* input, size_t columns, float* output,
                             const float* bias, size_t ldy, size_t y_offset)
{
    int rc = use_device(s);
    if (rc) return rc;
    pixhip_weight* w = const_cast<pixhip_weight*>(wc);
    if (!w) return fail(PIXHIP_ERR_ARGUMENT,"null weight handle");
    if (w->conv) return fail(PIXHIP_ERR_UNSUPPORTED,"a convolution weight: use pixhip_conv2d");
    if (!columns || !input || !output) return fail(PIXHIP_ERR_ARGUMENT,"null pointer or zero columns");
    if (!ldy) ldy = w->rows;
    if (ldy < w->rows) return fail(PIXHIP_ERR_ARGUMENT,"output stride smaller than rows");
    const void* xin = nullptr;
    const void* yv = nullptr;
    if ((rc = check_span(s,input,columns * w->inner * sizeof(float))) ||
        (rc = check_span(s,output,(y_offset + (columns - 1) * ldy + w->rows) * sizeof(float))) ||
        (bias && (rc = check_span(s,bias,w->rows * sizeof(float)))))
        return rc;
    if (!device_visible(s,input,&xin) || !device_visible(s,output,&yv))
        return fail(PIXHIP_ERR_ARGUMENT,"input and output must be device memory (nothing is staged here)");
    if (reinterpret_cast<uintptr_t>(xin) % 16) return fail(PIXHIP_ERR_ARGUMENT,"input must be 16-byte aligned");
    void* dev_scratch = g_scratch_ptr[s->device];
    if (!dev_scratch) return fail(PIXHIP_ERR_STATE,"scratch not set up on this device");
    const pixhip::Output out = {static_cast<float*>(const_cast<void*>(yv)),bias,ldy,y_offset};
    const float* x = static_cast<const float*>(xin);
    const size_t K = w->inner;
    w->used = ++s->uses;
    hipError_t e;
    if (columns == 1 && matvec_ok(w)) {
        // The matvec quantizes x in LDS: no scratch, but its layout must be resident.
        if (!w->planar) return fail(PIXHIP_ERR_STATE,"matvec layout not resident: run the weight once through pixhip_matmul_ex");
        if (w->type == PIX_Q5_K) e = pixhip::launch_matvec_q5_K(w->q5p,x,w->rows,K,out,s->stream);
        else if (w->type == PIX_Q8_0) e = pixhip::launch_matvec_q8_0(w->q80,x,w->rows,K,out,s->stream);
        else e = pixhip::launch_matvec_q6_K(w->q6p,x,w->rows,K,out,s->stream);
        PIX_HIP(e,"matvec launch");
        return PIXHIP_OK;
    }
    if (!w->planes) return fail(PIXHIP_ERR_STATE,"GEMM layout not resident: run the weight once through pixhip_matmul_ex");
    // The quantized activations in `scratch`, carved as act_buffers carves the
    // session scratch; the GEMM then runs unsplit (no split-K workspace).
    // Ordered after the last call on this device that used the array.
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    const int dev = s->device;
    if (g_scratch_used[dev] && g_scratch_stream[dev] != s->stream)
        PIX_HIP(hipStreamWaitEvent(s->stream,g_scratch_event[dev],0),"hipStreamWaitEvent (scratch order)");
    const size_t mpad = round_up(columns,kTileM);
    Carver c;
    uint8_t* base = static_cast<uint8_t*>(dev_scratch);
    if (w->type == PIX_Q8_0) {
        const size_t kp = round_up(K,64);
        const size_t qs = c.take(mpad * kp), d = c.take((kp / PIX_QK8) * mpad * 4);
        if (c.offset > kNoAllocScratchBytes)
            return fail(PIXHIP_ERR_MEMORY,"activations of " + std::to_string(columns) + " x " + std::to_string(K) + " need " +
                                              std::to_string(c.offset) + " bytes, beyond the 32 MiB allocation-free scratch");
        const pixhip::Act80 a = {reinterpret_cast<int8_t*>(base + qs),reinterpret_cast<float*>(base + d),mpad};
        PIX_HIP(pixhip::launch_quantize_q8_0(x,columns,K,kp,a,nullptr,s->stream),"quantize Q8_0");
        e = pixhip::launch_gemm_q8_0(a,w->q80,columns,w->rows,K,out,nullptr,s->stream);
    } else {
        const size_t qs = c.take(mpad * K), d = c.take((K / PIX_QK) * mpad * 4), bs = c.take(mpad * (K / 16) * 2);
        if (c.offset > kNoAllocScratchBytes)
            return fail(PIXHIP_ERR_MEMORY,"activations of " + std::to_string(columns) + " x " + std::to_string(K) + " need " +
                                              std::to_string(c.offset) + " bytes, beyond the 32 MiB allocation-free scratch");
        const pixhip::Act8K a = {reinterpret_cast<int8_t*>(base + qs),reinterpret_cast<float*>(base + d),
                                 reinterpret_cast<_Float16*>(base + bs),mpad};
        PIX_HIP(pixhip::launch_quantize_q8_K(x,columns,K,a,nullptr,s->stream),"quantize Q8_K");
        e = w->type == PIX_Q5_K? pixhip::launch_gemm_q5_K(a,w->q5,columns,w->rows,K,out,nullptr,s->stream)
                               : pixhip::launch_gemm_q6_K(a,w->q6,columns,w->rows,K,out,nullptr,s->stream);
    }
    PIX_HIP(e,"GEMM launch");
    PIX_HIP(hipEventRecord(g_scratch_event[dev],s->stream),"hipEventRecord (scratch order)");
    g_scratch_stream[dev] = s->stream;
    g_scratch_used[dev] = true;
    return PIXHIP_OK;
}

int pixhip_quant_matmul(pixhip_session* s, const unsigned char* weights, uint32_t type, const float* input, float* output,
                        size_t rows, size_t columns, size_t inner)
{
    if (!s) return fail(PIXHIP_ERR_STATE,"no session");
    int rc = check_shape(type,inner,rows);
    if (rc) return rc;
    if (!columns || !weights || !input || !output) return fail(PIXHIP_ERR_ARGUMENT,"null pointer or zero columns");
    if ((rc = use_device(s))) return rc;
    // Stateless, as cpu_quant_matmul is: a temporary weight outside the cache,
    // released (after the work completes) before returning.
    pixhip_weight w;
    w.key = "quant_matmul";
    w.type = type;
    w.inner = inner;
    w.rows = rows;
    w.gguf_bytes = rows * (inner / block_values(type)) * block_bytes(type);
    w.host = weights;
    w.used = ++s->uses;
    rc = pixhip_matmul(s,&w,input,columns,output);
    hipError_t e = hipStreamSynchronize(s->stream);
    release_forms(s,&w);
    if (!rc && e != hipSuccess) rc = hip_fail(e,"hipStreamSynchronize");
    return rc;
}

int pixhip_quantize_q8_0(pixhip_session* s, const float* input, void* blocks, size_t rows, size_t inner)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!rows || !inner || inner % PIX_QK8) return fail(PIXHIP_ERR_ARGUMENT,"inner must be a positive multiple of 32");
    if (!input || !blocks || reinterpret_cast<uintptr_t>(input) % 16 || reinterpret_cast<uintptr_t>(blocks) % 2)
        return fail(PIXHIP_ERR_ARGUMENT,"input must be 16-byte aligned, blocks 2-byte aligned");
    PIX_HIP(pixhip::launch_quantize_q8_0(input,rows,inner,round_up(inner,64),pixhip::Act80{nullptr,nullptr,0},blocks,s->stream),
            "quantize Q8_0");
    return PIXHIP_OK;
}

int pixhip_quantize_q8_K(pixhip_session* s, const float* input, void* blocks, size_t rows, size_t inner)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!rows || !inner || inner % PIX_QK) return fail(PIXHIP_ERR_ARGUMENT,"inner must be a positive multiple of 256");
    if (!input || !blocks || reinterpret_cast<uintptr_t>(input) % 16 || reinterpret_cast<uintptr_t>(blocks) % 4)
        return fail(PIXHIP_ERR_ARGUMENT,"input must be 16-byte aligned, blocks 4-byte aligned");
    PIX_HIP(pixhip::launch_quantize_q8_K(input,rows,inner,pixhip::Act8K{nullptr,nullptr,nullptr,0},blocks,s->stream),
            "quantize Q8_K");
    return PIXHIP_OK;
}

}  // extern "C"

namespace {

// Shared checks and set-up of the fused producers: the activation kind of
// `type` (0: none), the scratch activations for the MULTIPLY stages, and the
// optional outputs.
int fused_setup(pixhip_session* s, uint32_t type, size_t rows, size_t inner, float* result, void* blocks, int* kind,
                pixhip::ActOut* out)
{
    if (type && !supported_type(type)) return fail(PIXHIP_ERR_UNSUPPORTED,"unsupported weight type " + std::to_string(type));
    *kind = !type? 0 : (type == PIX_Q8_0? 2 : 1);
    // quantized: whole blocks; fp32 only: whole float4 loads
    const size_t block = *kind == 1? PIX_QK : (*kind == 2? PIX_QK8 : 4);
    if (!rows || !inner || inner % block || inner > INT32_MAX || rows > INT32_MAX)
        return fail(PIXHIP_ERR_ARGUMENT,"rows must be positive and inner a positive multiple of " + std::to_string(block));
    if (!*kind && !result) return fail(PIXHIP_ERR_ARGUMENT,"nothing to write: no type and no fp32 output");
    if (!*kind && blocks) return fail(PIXHIP_ERR_ARGUMENT,"blocks need a weight type");
    if (reinterpret_cast<uintptr_t>(result) % 16 || reinterpret_cast<uintptr_t>(blocks) % (*kind == 1? 4 : 2))
        return fail(PIXHIP_ERR_ARGUMENT,"fp32 output must be 16-byte aligned, blocks 4-byte (Q8_K) or 2-byte (Q8_0) aligned");
    *out = {nullptr,nullptr,nullptr,0,nullptr,nullptr};
    if (*kind) {
        int rc = act_buffers(s,*kind,rows,inner,out);
        if (rc) return rc;
    }
    out->blocks = blocks;
    out->y = result;
    return PIXHIP_OK;
}

}  // namespace

extern "C" {

int pixhip_norm_quantize(pixhip_session* s, uint32_t type, const float* input, size_t rows, size_t inner, const float* norm_weight,
                         float epsilon, int centered, const float* modulation, float* normalized, void* blocks)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!input || reinterpret_cast<uintptr_t>(input) % 16) return fail(PIXHIP_ERR_ARGUMENT,"input must be a 16-byte aligned device pointer");
    if ((reinterpret_cast<uintptr_t>(norm_weight) | reinterpret_cast<uintptr_t>(modulation)) % 16)
        return fail(PIXHIP_ERR_ARGUMENT,"norm weight and modulation must be 16-byte aligned");
    int kind;
    pixhip::ActOut out;
    if ((rc = fused_setup(s,type,rows,inner,normalized,blocks,&kind,&out))) return rc;
    const size_t kpad = kind == 2? round_up(inner,64) : inner;
    PIX_HIP(pixhip::launch_norm_quantize(input,rows,inner,norm_weight,epsilon,centered != 0,modulation,kind,kpad,out,s->stream),
            "norm + quantize");
    if (kind) set_act_shape(s,kind,rows,inner);
    return PIXHIP_OK;
}

int pixhip_silu_gate_quantize(pixhip_session* s, uint32_t type, const float* gate, const float* up, size_t rows, size_t inner,
                              float* gated, void* blocks)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!gate || !up || (reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up)) % 16)
        return fail(PIXHIP_ERR_ARGUMENT,"gate and up must be 16-byte aligned device pointers");
    int kind;
    pixhip::ActOut out;
    if ((rc = fused_setup(s,type,rows,inner,gated,blocks,&kind,&out))) return rc;
    const size_t kpad = kind == 2? round_up(inner,64) : inner;
    PIX_HIP(pixhip::launch_silu_gate_quantize(gate,up,rows,inner,kind,kpad,out,s->stream),"silu * gate + quantize");
    if (kind) set_act_shape(s,kind,rows,inner);
    return PIXHIP_OK;
}

int pixhip_pointwise(pixhip_session* s, unsigned operation, float* destination, const float* second, size_t rows, size_t channels)
{
    int rc = use_device(s);
    if (rc) return rc;
    const bool needs_second = operation == PIXHIP_OP_GATE || operation == PIXHIP_OP_ADD || operation == PIXHIP_OP_BIAS;
    if (operation != PIXHIP_OP_SILU && operation != PIXHIP_OP_GELU_EXACT && operation != PIXHIP_OP_GELU_TANH && !needs_second)
        return fail(PIXHIP_ERR_UNSUPPORTED,"unsupported pointwise operation " + std::to_string(operation));
    if (!rows || !channels || !destination || (needs_second && !second))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    if ((reinterpret_cast<uintptr_t>(destination) | reinterpret_cast<uintptr_t>(second)) % 4)
        return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,rows * channels * sizeof(float),&dst))) return rc;
    const void* other = nullptr;
    void* staged = nullptr;
    if (needs_second) {
        const size_t count = operation == PIXHIP_OP_BIAS? channels : rows * channels;
        if ((rc = read_operand(s,second,count * sizeof(float),&other,&staged))) return rc;
    }
    hipError_t e = pixhip::launch_pointwise((int)operation,static_cast<float*>(dst),static_cast<const float*>(other),rows,channels,s->stream);
    if (staged) pixhip_free(s,staged);
    PIX_HIP(e,"pointwise");
    return PIXHIP_OK;
}

int pixhip_rope(pixhip_session* s, float* tensor, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine,
                int interleaved)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!tensor || !cosine || !sine || !rows || !heads || channels % heads || (channels / heads) % 2)
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer, or channels not heads x an even head size");
    if ((reinterpret_cast<uintptr_t>(tensor) | reinterpret_cast<uintptr_t>(cosine) | reinterpret_cast<uintptr_t>(sine)) % 4)
        return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,tensor,rows * channels * sizeof(float),&dst))) return rc;
    const size_t table = rows * (channels / heads / 2) * sizeof(float);
    const void *cd = nullptr, *sd = nullptr;
    void *cs = nullptr, *ss = nullptr;
    if ((rc = read_operand(s,cosine,table,&cd,&cs))) return rc;
    if ((rc = read_operand(s,sine,table,&sd,&ss))) {
        if (cs) pixhip_free(s,cs);
        return rc;
    }
    hipError_t e = pixhip::launch_rope(static_cast<float*>(dst),rows,channels,heads,static_cast<const float*>(cd),static_cast<const float*>(sd),
                                       interleaved != 0,s->stream);
    if (cs) pixhip_free(s,cs);
    if (ss) pixhip_free(s,ss);
    PIX_HIP(e,"rope");
    return PIXHIP_OK;
}

namespace {

// The attention ranges' common path: operands resolved to device memory, one
// kernel launch per range after the split pass.
int attention_run(pixhip_session* s, const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads,
                  size_t kv_heads, size_t channels, const pixhip::AttnRange* ranges, size_t count, size_t query_offset, float* output)
{
    const size_t dim = channels / heads, kv_channels = dim * kv_heads;
    if (!pixhip::attention_dim_pad(dim))
        return fail(PIXHIP_ERR_UNSUPPORTED,"attention head size " + std::to_string(dim) + " is not supported (1..512)");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
         reinterpret_cast<uintptr_t>(output)) % 16)
        return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 16-byte aligned");
    int rc;
    void* out = nullptr;
    if ((rc = write_operand(s,output,rows * channels * sizeof(float),&out))) return rc;
    const void *qd = nullptr, *kd = nullptr, *vd = nullptr;
    void *qs = nullptr, *ks = nullptr, *vs = nullptr;
    auto release = [&]() {
        if (qs) pixhip_free(s,qs);
        if (ks) pixhip_free(s,ks);
        if (vs) pixhip_free(s,vs);
    };
    if ((rc = read_operand(s,q,rows * channels * sizeof(float),&qd,&qs)) ||
        (rc = read_operand(s,k,keys * kv_channels * sizeof(float),&kd,&ks)) ||
        (rc = read_operand(s,v,keys * kv_channels * sizeof(float),&vd,&vs))) {
        release();
        return rc;
    }
    if ((rc = grow(s,&s->attn,&s->attn_bytes,pixhip::attention_workspace_bytes(rows,keys,heads,kv_heads,dim)))) {
        release();
        return rc;
    }
    hipError_t e = pixhip::launch_attention(static_cast<const float*>(qd),static_cast<const float*>(kd),static_cast<const float*>(vd),
                                            static_cast<float*>(out),rows,keys,heads,kv_heads,dim,ranges,count,query_offset,s->attn,
                                            s->stream);
    release();
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"attention shape beyond the kernel's 32-bit index range");
    PIX_HIP(e,"attention");
    return PIXHIP_OK;
}

}  // namespace

int pixhip_attention(pixhip_session* s, const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads,
                     size_t kv_heads, size_t channels, int causal, float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!q || !k || !v || !output) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    if (!rows || !keys || !heads || !kv_heads || heads % kv_heads || channels % heads)
        return fail(PIXHIP_ERR_ARGUMENT,"empty tensors, or heads not a multiple of kv_heads, or channels not of heads");
    if (causal && rows > keys) return fail(PIXHIP_ERR_ARGUMENT,"causal attention needs a key for every query row (rows <= keys)");
    const pixhip::AttnRange all = {0,rows,keys,causal != 0};
    return attention_run(s,q,rows,k,v,keys,heads,kv_heads,channels,&all,1,0,output);
}

int pixhip_attention_ranges(pixhip_session* s, const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads,
                            size_t kv_heads, size_t channels, const pixhip_attention_range* ranges, size_t count,
                            size_t query_offset, float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!q || !k || !v || !output || (count && !ranges)) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    // the reference's checks (src/tensor.cpp:386-394)
    if (!rows || !keys || !heads || !kv_heads || heads % kv_heads || channels % heads || query_offset > SIZE_MAX - rows)
        return fail(PIXHIP_ERR_ARGUMENT,"empty tensors, or heads not a multiple of kv_heads, or channels not of heads");
    std::vector<pixhip::AttnRange> rs(count);
    size_t covered = 0;
    for (size_t i = 0; i < count; i++) {
        const pixhip_attention_range& r = ranges[i];
        if (r.query_begin != covered || r.query_end <= r.query_begin || r.query_end > rows || !r.key_end || r.key_end > keys)
            return fail(PIXHIP_ERR_ARGUMENT,"ranges must tile the query rows in order with 0 < key_end <= keys");
        covered = r.query_end;
        rs[i] = {r.query_begin,r.query_end,r.key_end,r.causal != 0};
    }
    if (covered != rows) return fail(PIXHIP_ERR_ARGUMENT,"ranges must cover every query row");
    return attention_run(s,q,rows,k,v,keys,heads,kv_heads,channels,rs.data(),count,query_offset,output);
}

int pixhip_block_sums(pixhip_session* s, const pixhip_weight* wc, const float* input, size_t columns, int32_t* sums, int32_t* mins)
{
    int rc = use_device(s);
    if (rc) return rc;
    pixhip_weight* w = const_cast<pixhip_weight*>(wc);
    if (!w || !input || !sums || !columns || (w->type == PIX_Q5_K && !mins)) return fail(PIXHIP_ERR_ARGUMENT,"null pointer");
    if (w->conv) return fail(PIXHIP_ERR_UNSUPPORTED,"a convolution weight");
    if (reinterpret_cast<uintptr_t>(input) % 16) return fail(PIXHIP_ERR_ARGUMENT,"input must be 16-byte aligned");
    if ((rc = quantize_stage(s,w,input,columns))) return rc;
    if ((rc = ensure_gemm_form(s,w))) return rc;
    hipError_t e;
    if (w->type == PIX_Q5_K) e = pixhip::launch_sums_q5_K(s->a8k,w->q5,columns,w->rows,w->inner,sums,mins,s->stream);
    else if (w->type == PIX_Q6_K) e = pixhip::launch_sums_q6_K(s->a8k,w->q6,columns,w->rows,w->inner,sums,s->stream);
    else e = pixhip::launch_sums_q8_0(s->a80,w->q80,columns,w->rows,w->inner,sums,s->stream);
    PIX_HIP(e,"block sums launch");
    return PIXHIP_OK;
}

int pixhip_timer_start(pixhip_session* s)
{
    int rc = use_device(s);
    if (rc) return rc;
    PIX_HIP(hipEventRecord(s->t0,s->stream),"hipEventRecord");
    return PIXHIP_OK;
}

int pixhip_timer_stop(pixhip_session* s, float* ms)
{
    int rc = use_device(s);
    if (rc) return rc;
    PIX_HIP(hipEventRecord(s->t1,s->stream),"hipEventRecord");
    PIX_HIP(hipEventSynchronize(s->t1),"hipEventSynchronize");
    float v = 0;
    PIX_HIP(hipEventElapsedTime(&v,s->t0,s->t1),"hipEventElapsedTime");
    if (ms) *ms = v;
    return PIXHIP_OK;
}

int pixhip_bench_matmul(pixhip_session* s, const pixhip_weight* const* weights, size_t count, const float* input, size_t columns,
                        float* output, unsigned stages, size_t reps, float* ms)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!weights || !count || !reps) return fail(PIXHIP_ERR_ARGUMENT,"empty benchmark");
    PIX_HIP(hipEventRecord(s->t0,s->stream),"hipEventRecord");
    for (size_t i = 0; i < reps; i++) {
        rc = run(s,weights[i % count],input,columns,output,nullptr,0,0,stages,false);
        if (rc) return rc;
    }
    PIX_HIP(hipEventRecord(s->t1,s->stream),"hipEventRecord");
    PIX_HIP(hipEventSynchronize(s->t1),"hipEventSynchronize");
    float v = 0;
    PIX_HIP(hipEventElapsedTime(&v,s->t0,s->t1),"hipEventElapsedTime");
    if (ms) *ms = v;
    return PIXHIP_OK;
}

}  // extern "C"

/* ---- the rest of the backend op surface ---- */

namespace {

// Operands staged by read_operand, released together after the launch (the
// pool reuses a block only for work queued after it).
struct Staged {
    pixhip_session* s;
    std::vector<void*> blocks;
    explicit Staged(pixhip_session* session) : s(session) {}
    ~Staged()
    {
        for (void* b : blocks) pixhip_free(s,b);
    }
    int read(const void* p, size_t bytes, const void** dev, bool stage_pinned = false)
    {
        void* staged = nullptr;
        const int rc = read_operand(s,p,bytes,dev,&staged,stage_pinned);
        if (staged) blocks.push_back(staged);
        return rc;
    }
};

bool aligned4(const void* p)
{
    return reinterpret_cast<uintptr_t>(p) % 4 == 0;
}

// a * b * 4 bytes without overflow
bool float_bytes(size_t a, size_t b, size_t* bytes)
{
    if (b && a > SIZE_MAX / b / sizeof(float)) return false;
    *bytes = a * b * sizeof(float);
    return true;
}

// Bytes of one GGUF row of `inner` values (weight_bytes, src/model.cpp:87-121);
// 0 for a type cpu_decode does not know or a ragged block.
size_t gguf_row_bytes(uint32_t type, uint64_t inner)
{
    switch (type) {
    case PIX_F32: return inner * 4;
    case PIX_F16:
    case PIX_BF16: return inner * 2;
    case PIX_Q8_0: return inner % PIX_QK8? 0 : inner / PIX_QK8 * PIX_Q8_0_BYTES;
    case PIX_Q5_K: return inner % PIX_QK? 0 : inner / PIX_QK * PIX_Q5_K_BYTES;
    case PIX_Q6_K: return inner % PIX_QK? 0 : inner / PIX_QK * PIX_Q6_K_BYTES;
    default: return 0;
    }
}

}  // namespace

extern "C" {

int pixhip_pointwise_ex(pixhip_session* s, unsigned operation, float* destination, const float* second, const float* third, size_t rows,
                        size_t channels, unsigned part, float scale, float bias)
{
    if (operation != PIXHIP_OP_MODULATE && operation != PIXHIP_OP_RESIDUAL && operation != PIXHIP_OP_AFFINE &&
        operation != PIXHIP_OP_EULER)
        return pixhip_pointwise(s,operation,destination,second,rows,channels);
    int rc = use_device(s);
    if (rc) return rc;
    size_t bytes = 0;
    const bool needs_second = operation != PIXHIP_OP_AFFINE;
    if (!rows || !channels || !destination || (needs_second && !second) || !float_bytes(rows,channels,&bytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    if (!aligned4(destination) || !aligned4(second) || !aligned4(third)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    if ((size_t)part > SIZE_MAX / channels - 1) return fail(PIXHIP_ERR_ARGUMENT,"part out of range");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,bytes,&dst))) return rc;
    Staged st(s);
    const void *other = nullptr, *param = nullptr;
    const size_t slice = (size_t)part * channels;
    if (operation == PIXHIP_OP_MODULATE) {
        if ((rc = st.read(second + slice,channels * sizeof(float),&param))) return rc;
    } else if (operation == PIXHIP_OP_RESIDUAL || operation == PIXHIP_OP_EULER) {
        if ((rc = st.read(second,bytes,&other))) return rc;
        if (operation == PIXHIP_OP_RESIDUAL && third && (rc = st.read(third + slice,channels * sizeof(float),&param))) return rc;
    }
    const int op = operation == PIXHIP_OP_MODULATE? pixhip::kOpModulate
                 : operation == PIXHIP_OP_RESIDUAL? pixhip::kOpResidual
                 : operation == PIXHIP_OP_AFFINE? pixhip::kOpAffine
                                                 : pixhip::kOpEuler;
    hipError_t e = pixhip::launch_channel_op(op,static_cast<float*>(dst),static_cast<const float*>(other),static_cast<const float*>(param),
                                             nullptr,rows,channels,0,scale,bias,s->stream);
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"too many rows for one launch");
    PIX_HIP(e,"pointwise");
    return PIXHIP_OK;
}

int pixhip_qwen_modulate(pixhip_session* s, float* destination, size_t rows, size_t channels, const float* parameters,
                         size_t parameter_channels, size_t target_begin, size_t part, const float* residual)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t bytes = 0, pbytes = 0;
    if (!destination || !parameters || !rows || !channels || !float_bytes(rows,channels,&bytes) || !float_bytes(2,parameter_channels,&pbytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    // the reference's check (src/qwen_image.cpp:152)
    if (part >= SIZE_MAX / channels || (part + 1) * channels > parameter_channels)
        return fail(PIXHIP_ERR_ARGUMENT,"parameters hold fewer than (part + 1) * channels values per row");
    if (!aligned4(destination) || !aligned4(parameters) || !aligned4(residual)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,bytes,&dst))) return rc;
    Staged st(s);
    const void *param = nullptr, *other = nullptr;
    if ((rc = st.read(parameters,pbytes,&param))) return rc;
    if (residual && (rc = st.read(residual,bytes,&other))) return rc;
    const float* p0 = static_cast<const float*>(param) + part * channels;
    hipError_t e = pixhip::launch_channel_op(residual? pixhip::kOpQwenResidual : pixhip::kOpQwenScale,static_cast<float*>(dst),
                                             static_cast<const float*>(other),p0,p0 + parameter_channels,rows,channels,target_begin,0.0f,
                                             0.0f,s->stream);
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"too many rows for one launch");
    PIX_HIP(e,"qwen modulate");
    return PIXHIP_OK;
}

int pixhip_l2norm(pixhip_session* s, const float* input, size_t rows, size_t channels, const float* weight, float epsilon, float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t bytes = 0;
    // the reference's checks (src/tensor.cpp:244)
    if (!input || !output || !rows || !channels || !float_bytes(rows,channels,&bytes) || !(epsilon > 0.0f))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer, empty tensor or epsilon <= 0");
    if (!aligned4(input) || !aligned4(output) || !aligned4(weight)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* out = nullptr;
    if ((rc = write_operand(s,output,bytes,&out))) return rc;
    Staged st(s);
    const void *in = nullptr, *w = nullptr;
    if ((rc = st.read(input,bytes,&in))) return rc;
    if (weight && (rc = st.read(weight,channels * sizeof(float),&w))) return rc;
    hipError_t e = pixhip::launch_l2norm(static_cast<const float*>(in),static_cast<const float*>(w),static_cast<float*>(out),rows,channels,
                                         epsilon,s->stream);
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"too many rows for one launch");
    PIX_HIP(e,"l2norm");
    return PIXHIP_OK;
}

int pixhip_groupnorm(pixhip_session* s, const float* input, size_t rows, size_t channels, const float* weight, const float* bias,
                     float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t bytes = 0;
    if (!input || !output || !weight || !bias || !rows || !channels || !float_bytes(rows,channels,&bytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    if (channels % 32) return fail(PIXHIP_ERR_ARGUMENT,"channels must be a multiple of the 32 groups");
    const size_t work = pixhip::groupnorm_workspace_bytes(rows,channels);
    if (!work) return fail(PIXHIP_ERR_UNSUPPORTED,"groupnorm supports groups of up to 256 channels");
    if (!aligned4(input) || !aligned4(output) || !aligned4(weight) || !aligned4(bias))
        return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* out = nullptr;
    if ((rc = write_operand(s,output,bytes,&out))) return rc;
    Staged st(s);
    const void *in = nullptr, *w = nullptr, *b = nullptr;
    if ((rc = st.read(input,bytes,&in)) || (rc = st.read(weight,channels * sizeof(float),&w)) ||
        (rc = st.read(bias,channels * sizeof(float),&b)))
        return rc;
    if ((rc = grow(s,&s->gn,&s->gn_bytes,work))) return rc;
    hipError_t e = pixhip::launch_groupnorm(static_cast<const float*>(in),static_cast<const float*>(w),static_cast<const float*>(b),
                                            static_cast<float*>(out),rows,channels,1e-6f,s->gn,s->stream);
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"too many rows for one launch");
    PIX_HIP(e,"groupnorm");
    return PIXHIP_OK;
}

int pixhip_embedding(pixhip_session* s, const void* table, uint32_t type, uint64_t inner, uint64_t table_rows, const int32_t* ids,
                     size_t count, float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!table || !ids || !output || !count || !inner || !table_rows) return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    const size_t stride = gguf_row_bytes(type,inner);
    if (type != PIX_F32 && type != PIX_F16 && type != PIX_BF16 && type != PIX_Q8_0 && type != PIX_Q5_K && type != PIX_Q6_K)
        return fail(PIXHIP_ERR_UNSUPPORTED,"unsupported embedding type " + std::to_string(type));
    size_t bytes = 0;
    if (!stride || inner > SIZE_MAX / 4 || table_rows > SIZE_MAX / stride || !float_bytes(count,inner,&bytes))
        return fail(PIXHIP_ERR_ARGUMENT,"inner is not a whole number of blocks, or the table is too large");
    if (!aligned4(output)) return fail(PIXHIP_ERR_ARGUMENT,"output must be 4-byte aligned");
    for (size_t i = 0; i < count; i++)
        if (ids[i] < 0 || (uint64_t)ids[i] >= table_rows) return fail(PIXHIP_ERR_ARGUMENT,"token id " + std::to_string(ids[i]) + " out of range");
    void* out = nullptr;
    if ((rc = write_operand(s,output,bytes,&out))) return rc;
    Staged st(s);
    const void* dev_table = nullptr;
    hipError_t e;
    if (device_visible(s,table,&dev_table)) {
        // a device-resident table: gather on the device
        std::vector<int64_t> rows(ids,ids + count);
        const void* dev_ids = nullptr;
        if ((rc = st.read(rows.data(),count * sizeof(int64_t),&dev_ids))) return rc;
        e = pixhip::launch_decode_rows(dev_table,type,stride,static_cast<const int64_t*>(dev_ids),count,inner,static_cast<float*>(out),s->stream);
    } else {
        // the model file's mapping: pack the selected rows (vulkan_embedding,
        // src/backend_vulkan.cpp:1241-1243) and move only those
        std::vector<unsigned char> packed(count * stride);
        const unsigned char* base = static_cast<const unsigned char*>(table);
        for (size_t i = 0; i < count; i++) memcpy(packed.data() + i * stride,base + (size_t)ids[i] * stride,stride);
        const void* dev_rows = nullptr;
        if ((rc = st.read(packed.data(),packed.size(),&dev_rows))) return rc;
        e = pixhip::launch_decode_rows(dev_rows,type,stride,nullptr,count,inner,static_cast<float*>(out),s->stream);
    }
    PIX_HIP(e,"embedding");
    return PIXHIP_OK;
}

int pixhip_rows(pixhip_session* s, const float* source, size_t source_rows, float* destination, size_t destination_rows, size_t channels,
                const size_t* rows, size_t count, int scatter)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t sbytes = 0, dbytes = 0;
    if (!source || !destination || !rows || !count || !channels || !source_rows || !destination_rows ||
        !float_bytes(source_rows,channels,&sbytes) || !float_bytes(destination_rows,channels,&dbytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    if (!aligned4(source) || !aligned4(destination)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    // the reference's checks (src/tensor.cpp:277-279, :293-296)
    if ((scatter? source_rows : destination_rows) != count) return fail(PIXHIP_ERR_ARGUMENT,"row count does not match the row list");
    const size_t bound = scatter? destination_rows : source_rows;
    for (size_t i = 0; i < count; i++)
        if (rows[i] >= bound) return fail(PIXHIP_ERR_ARGUMENT,"row " + std::to_string(rows[i]) + " out of range");
    std::vector<uint64_t> src_rows, dst_rows;
    if (scatter) {
        // a row listed twice keeps the last copy, as the reference's in-order loop does
        std::unordered_map<size_t,size_t> last;
        for (size_t i = 0; i < count; i++) last[rows[i]] = i;
        for (size_t i = 0; i < count; i++)
            if (last[rows[i]] == i) {
                src_rows.push_back(i);
                dst_rows.push_back(rows[i]);
            }
    } else {
        src_rows.assign(rows,rows + count);
    }
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,dbytes,&dst))) return rc;
    Staged st(s);
    const void *src = nullptr, *sr = nullptr, *dr = nullptr;
    if ((rc = st.read(source,sbytes,&src)) || (rc = st.read(src_rows.data(),src_rows.size() * sizeof(uint64_t),&sr))) return rc;
    if (scatter && (rc = st.read(dst_rows.data(),dst_rows.size() * sizeof(uint64_t),&dr))) return rc;
    hipError_t e = pixhip::launch_rows(static_cast<const float*>(src),static_cast<float*>(dst),static_cast<const uint64_t*>(sr),
                                       static_cast<const uint64_t*>(dr),src_rows.size(),channels,s->stream);
    PIX_HIP(e,"rows");
    return PIXHIP_OK;
}

int pixhip_copy_rows(pixhip_session* s, const float* source, size_t source_rows, size_t source_channels, float* destination,
                     size_t destination_rows, size_t destination_channels, size_t rows, size_t source_row, size_t source_feature,
                     size_t destination_row)
{
    int rc = use_device(s);
    if (rc) return rc;
    size_t sbytes = 0, dbytes = 0;
    if (!source || !destination || !rows || !destination_channels || !float_bytes(source_rows,source_channels,&sbytes) ||
        !float_bytes(destination_rows,destination_channels,&dbytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    if (source_row > source_rows || rows > source_rows - source_row || destination_row > destination_rows ||
        rows > destination_rows - destination_row || source_feature > source_channels ||
        destination_channels > source_channels - source_feature)
        return fail(PIXHIP_ERR_ARGUMENT,"the copied rows do not lie within both tensors");
    if (!aligned4(source) || !aligned4(destination)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,dbytes,&dst))) return rc;
    Staged st(s);
    const void* src = nullptr;
    if ((rc = st.read(source,sbytes,&src))) return rc;
    hipError_t e = pixhip::launch_copy2d(static_cast<const float*>(src) + source_row * source_channels + source_feature,source_channels,
                                         static_cast<float*>(dst) + destination_row * destination_channels,destination_channels,rows,
                                         destination_channels,s->stream);
    PIX_HIP(e,"copy rows");
    return PIXHIP_OK;
}

int pixhip_copy_features(pixhip_session* s, const float* source, size_t source_channels, float* destination, size_t destination_channels,
                         size_t destination_feature)
{
    int rc = use_device(s);
    if (rc) return rc;
    // the reference's checks (src/backend_vulkan.cpp:1273)
    if (!source || !destination || !source_channels || !destination_channels || destination_feature > destination_channels ||
        source_channels > destination_channels - destination_feature)
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer, empty tensor, or the source does not fit at the destination feature");
    if (!aligned4(source) || !aligned4(destination)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,destination_channels * sizeof(float),&dst))) return rc;
    Staged st(s);
    const void* src = nullptr;
    if ((rc = st.read(source,source_channels * sizeof(float),&src))) return rc;
    hipError_t e = pixhip::launch_copy2d(static_cast<const float*>(src),source_channels,static_cast<float*>(dst) + destination_feature,
                                         destination_channels,1,source_channels,s->stream);
    PIX_HIP(e,"copy features");
    return PIXHIP_OK;
}

int pixhip_layout(pixhip_session* s, unsigned operation, const float* source, size_t source_rows, size_t source_channels, float* destination,
                  size_t destination_rows, size_t destination_channels, size_t width, size_t patch)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (operation != PIXHIP_OP_PATCH && operation != PIXHIP_OP_UNPATCH && operation != PIXHIP_OP_UPSAMPLE)
        return fail(PIXHIP_ERR_UNSUPPORTED,"unsupported layout operation " + std::to_string(operation));
    size_t sbytes = 0, dbytes = 0;
    if (!source || !destination || !source_rows || !source_channels || !destination_rows || !destination_channels || !width ||
        !float_bytes(source_rows,source_channels,&sbytes) || !float_bytes(destination_rows,destination_channels,&dbytes))
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    bool ok;
    if (operation == PIXHIP_OP_UPSAMPLE) {
        // tensor_upsample's checks (src/tensor.cpp:306)
        ok = source_rows % width == 0 && source_rows <= SIZE_MAX / 4 && destination_rows == source_rows * 4 &&
             destination_channels == source_channels;
    } else {
        // the DiT layout (src/inference.cpp:364, :374-376): width and height multiples of the patch
        const bool to_tokens = operation == PIXHIP_OP_PATCH;
        const size_t pixels = to_tokens? source_rows : destination_rows, tokens = to_tokens? destination_rows : source_rows;
        const size_t narrow = to_tokens? source_channels : destination_channels, wide = to_tokens? destination_channels : source_channels;
        ok = patch && width % patch == 0 && pixels % width == 0 && (pixels / width) % patch == 0 && patch <= SIZE_MAX / patch &&
             narrow <= SIZE_MAX / (patch * patch) && wide == narrow * patch * patch &&
             tokens == (width / patch) * (pixels / width / patch);
    }
    if (!ok) return fail(PIXHIP_ERR_ARGUMENT,"tensor shapes do not match the layout");
    if (!aligned4(source) || !aligned4(destination)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,dbytes,&dst))) return rc;
    Staged st(s);
    const void* src = nullptr;
    if ((rc = st.read(source,sbytes,&src))) return rc;
    const int op = operation == PIXHIP_OP_PATCH? pixhip::kLayoutPatch : operation == PIXHIP_OP_UNPATCH? pixhip::kLayoutUnpatch : pixhip::kLayoutUpsample;
    hipError_t e = pixhip::launch_layout(op,static_cast<const float*>(src),static_cast<float*>(dst),destination_rows,destination_channels,width,
                                         source_channels,patch,s->stream);
    PIX_HIP(e,"layout");
    return PIXHIP_OK;
}

int pixhip_shortcut(pixhip_session* s, const float* source, size_t width, size_t height, size_t source_channels, float* destination,
                    size_t channels, size_t temporal, int up, int spatial)
{
    int rc = use_device(s);
    if (rc) return rc;
    // tensor_resample_shortcut's checks (src/tensor.cpp:489-500)
    if (!source || !destination || !width || !height || !channels || !temporal || !source_channels || width > SIZE_MAX / height)
        return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty tensor");
    const size_t side = spatial? 2 : 1;
    if (temporal > SIZE_MAX / (side * side) || width > SIZE_MAX / side || height > SIZE_MAX / side)
        return fail(PIXHIP_ERR_ARGUMENT,"shape too large");
    const size_t factor = temporal * side * side;
    if (channels > SIZE_MAX / factor || source_channels > SIZE_MAX / factor) return fail(PIXHIP_ERR_ARGUMENT,"shape too large");
    if ((up && channels * factor % source_channels) || (!up && source_channels * factor % channels))
        return fail(PIXHIP_ERR_ARGUMENT,"channels do not divide into the resampled groups");
    if (!up && (width % side || height % side)) return fail(PIXHIP_ERR_ARGUMENT,"width and height must be even to go down");
    const size_t out_width = up? width * side : width / side, out_height = up? height * side : height / side;
    size_t sbytes = 0, dbytes = 0;
    if (out_width > SIZE_MAX / out_height || !float_bytes(width * height,source_channels,&sbytes) ||
        !float_bytes(out_width * out_height,channels,&dbytes))
        return fail(PIXHIP_ERR_ARGUMENT,"shape too large");
    if (!aligned4(source) || !aligned4(destination)) return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    void* dst = nullptr;
    if ((rc = write_operand(s,destination,dbytes,&dst))) return rc;
    Staged st(s);
    const void* src = nullptr;
    if ((rc = st.read(source,sbytes,&src))) return rc;
    hipError_t e = pixhip::launch_shortcut(static_cast<const float*>(src),static_cast<float*>(dst),out_width * out_height,channels,
                                           source_channels,width,side,temporal,up != 0,s->stream);
    PIX_HIP(e,"shortcut");
    return PIXHIP_OK;
}

}  // extern "C"

/* ---- convolution ---- */

namespace {

// The split-bf16 planes of a convolution weight, built from its file bytes.
int ensure_conv_form(pixhip_session* s, pixhip_weight* w)
{
    if (w->conv_planes) return PIXHIP_OK;
    int rc = ensure_raw(s,w);
    if (rc) return rc;
    const size_t plane = w->conv_npad * w->conv_kp * sizeof(uint16_t);
    if ((rc = weight_alloc(s,w,2 * plane,&w->conv_planes))) return rc;
    uint16_t* hi = static_cast<uint16_t*>(w->conv_planes);
    PIX_HIP(pixhip::launch_conv_form(w->raw,w->type,(int)w->kernel_x,(int)w->kernel_y,(int)w->cin,(int)w->rows,(int)w->conv_kp,
                                     (int)w->conv_npad,hi,hi + plane / sizeof(uint16_t),s->stream),
            "convolution weight form");
    return release_raw(s,w);
}

size_t float_type_bytes(uint32_t type)
{
    return type == PIX_F32? 4 : (type == PIX_F16 || type == PIX_BF16)? 2 : 0;
}

}  // namespace

extern "C" {

int pixhip_conv_weight_get(pixhip_session* s, const char* key, const void* host_bytes, uint64_t bytes, uint32_t type,
                           uint64_t kernel_x, uint64_t kernel_y, uint64_t in_channels, uint64_t out_channels, pixhip_weight** out)
{
    int rc = use_device(s);
    if (rc) return rc;
    if (!key || !out) return fail(PIXHIP_ERR_ARGUMENT,"null key or output");
    *out = nullptr;
    const size_t elem = float_type_bytes(type);
    if (!elem) return fail(PIXHIP_ERR_UNSUPPORTED,"convolution weights are F32, F16 or BF16 (type " + std::to_string(type) + ")");
    if (!kernel_x || !kernel_y || !in_channels || !out_channels || kernel_x > 64 || kernel_y > 64 || in_channels > (1u << 20) ||
        out_channels > (1u << 20) || in_channels * kernel_x * kernel_y > INT32_MAX / 2)
        return fail(PIXHIP_ERR_ARGUMENT,"bad convolution weight shape");
    const uint64_t inner = in_channels * kernel_x * kernel_y, expect = out_channels * inner * elem;
    auto it = s->weights.find(key);
    if (it != s->weights.end()) {
        pixhip_weight* w = it->second;
        if (!w->conv || w->type != type || w->kernel_x != kernel_x || w->kernel_y != kernel_y || w->cin != in_channels ||
            w->rows != out_channels)
            return fail(PIXHIP_ERR_ARGUMENT,"cached key with another shape");
        if (host_bytes) {
            if (bytes < expect) return fail(PIXHIP_ERR_ARGUMENT,"weight bytes shorter than the tensor");
            w->host = host_bytes;
        }
        w->used = ++s->uses;
        *out = w;
        return PIXHIP_OK;
    }
    if (!host_bytes || bytes < expect) return fail(PIXHIP_ERR_ARGUMENT,"weight bytes missing or shorter than the tensor");
    pixhip_weight* w = new (std::nothrow) pixhip_weight();
    if (!w) return fail(PIXHIP_ERR_MEMORY,"host allocation failed");
    w->key = key;
    w->type = type;
    w->inner = inner;
    w->rows = out_channels;
    w->gguf_bytes = expect;
    w->host = host_bytes;
    w->used = ++s->uses;
    w->conv = true;
    w->kernel_x = (uint32_t)kernel_x;
    w->kernel_y = (uint32_t)kernel_y;
    w->cin = (uint32_t)in_channels;
    w->conv_kp = round_up(inner,pixhip::kConvTileK);
    w->conv_npad = round_up(out_channels,pixhip::kConvTileN);
    if ((rc = ensure_raw(s,w))) {
        release_forms(s,w);
        delete w;
        return rc;
    }
    s->weights.emplace(w->key,w);
    *out = w;
    return PIXHIP_OK;
}

int pixhip_conv2d(pixhip_session* s, const pixhip_weight* wc, const float* input, size_t width, size_t height,
                  const pixhip_conv_geometry* geometry, const float* bias, float* output)
{
    int rc = use_device(s);
    if (rc) return rc;
    pixhip_weight* w = const_cast<pixhip_weight*>(wc);
    if (!w || !w->conv) return fail(PIXHIP_ERR_ARGUMENT,"not a convolution weight (pixhip_conv_weight_get)");
    if (!input || !output || !width || !height || width > SIZE_MAX / height) return fail(PIXHIP_ERR_ARGUMENT,"null pointer or empty image");
    // tensor_conv's "same" form (src/convolution.cpp:34-54): stride 1, the
    // kernel centred (offset kernel / 2), as many output pixels as input ones
    pixhip_conv_geometry g{1,1,w->kernel_x / 2,w->kernel_x - 1 - w->kernel_x / 2,w->kernel_y / 2,w->kernel_y - 1 - w->kernel_y / 2};
    if (geometry) g = *geometry;
    // the geometry form's checks (src/convolution.cpp:58-69)
    if (!g.stride_x || !g.stride_y || g.left > SIZE_MAX - width || g.right > SIZE_MAX - width - g.left || g.top > SIZE_MAX - height ||
        g.bottom > SIZE_MAX - height - g.top)
        return fail(PIXHIP_ERR_ARGUMENT,"bad convolution geometry");
    const size_t pw = width + g.left + g.right, ph = height + g.top + g.bottom;
    if (pw < w->kernel_x || ph < w->kernel_y) return fail(PIXHIP_ERR_ARGUMENT,"the padded image is smaller than the kernel");
    const size_t ow = (pw - w->kernel_x) / g.stride_x + 1, oh = (ph - w->kernel_y) / g.stride_y + 1;
    if (width > INT32_MAX / 2 || height > INT32_MAX / 2 || pw > INT32_MAX / 2 || ph > INT32_MAX / 2 || g.stride_x > INT32_MAX ||
        g.stride_y > INT32_MAX || ow > SIZE_MAX / oh || width * height > UINT32_MAX)
        return fail(PIXHIP_ERR_ARGUMENT,"image too large");  // pixel indices are 32-bit in the kernel
    size_t in_bytes = 0, out_bytes = 0;
    if (width * height > SIZE_MAX / w->cin / 4 || ow * oh > SIZE_MAX / w->rows / 4) return fail(PIXHIP_ERR_ARGUMENT,"image too large");
    in_bytes = width * height * w->cin * 4;
    out_bytes = ow * oh * w->rows * 4;
    if (reinterpret_cast<uintptr_t>(input) % 4 || reinterpret_cast<uintptr_t>(output) % 4 || reinterpret_cast<uintptr_t>(bias) % 4)
        return fail(PIXHIP_ERR_ARGUMENT,"tensors must be 4-byte aligned");
    w->used = ++s->uses;
    if ((rc = ensure_conv_form(s,w))) return rc;
    void* out = nullptr;
    if ((rc = write_operand(s,output,out_bytes,&out))) return rc;
    Staged st(s);
    const void *in = nullptr, *b = nullptr;
    // The kernel reads each input pixel once per kernel tap: pinned host input
    // is copied to HBM once rather than re-read over PCIe.
    if ((rc = st.read(input,in_bytes,&in,true))) return rc;
    if (bias && (rc = st.read(bias,w->rows * sizeof(float),&b))) return rc;
    pixhip::ConvArgs a{};
    a.x = static_cast<const float*>(in);
    a.wh = static_cast<const uint16_t*>(w->conv_planes);
    a.wl = a.wh + w->conv_npad * w->conv_kp;
    a.bias = static_cast<const float*>(b);
    a.y = static_cast<float*>(out);
    a.W = (int)width;
    a.H = (int)height;
    a.C = (int)w->cin;
    a.KX = (int)w->kernel_x;
    a.KY = (int)w->kernel_y;
    a.SX = (int)g.stride_x;
    a.SY = (int)g.stride_y;
    a.PL = (int)g.left;
    a.PT = (int)g.top;
    a.OW = (int)ow;
    a.OH = (int)oh;
    a.K = (int)w->inner;
    a.Kp = (int)w->conv_kp;
    a.N = (int)w->rows;
    a.Npad = (int)w->conv_npad;
    a.M = (long long)(ow * oh);
    hipError_t e = pixhip::launch_conv(a,s->stream);
    if (e == hipErrorInvalidValue) return fail(PIXHIP_ERR_ARGUMENT,"convolution grid too large");
    PIX_HIP(e,"convolution");
    return PIXHIP_OK;
}

}  // extern "C"
