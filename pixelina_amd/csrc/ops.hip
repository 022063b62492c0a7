// The reference's elementwise tensor ops on device rows, in place (the
// counterparts of vulkan_pointwise / vulkan_bias / vulkan_rope,
// src/backend_vulkan.h:142-150, and of the CPU ops in src/tensor.cpp they
// replace):
//   SiLU      v / (1.0f + expf(-v))                              :199-209
//   gate      v * other                                          :334-345
//   add       v + other                                          :321-332
//   bias      v + bias[c]                                        :226-240
//   GELU      0.5f * v * (1 + erff(v / sqrt 2))                  :211-224
//   GELU tanh 0.5f * v * (1 + tanhf(0.79788456f * (v + 0.044715f * v^3)))
//   RoPE      (a, b) -> (a*c - b*s, a*s + b*c) per pair          :429-452
// in fp32, operation by operation in the reference's order (the build has no
// contraction).  The transcendentals are the fp32 rounding of the double
// function (correctly rounded); the reference's glibc expf / erff / tanhf are
// within about an ulp of that.
// HBM-bound: one value per thread, grid-stride; RoPE four values per thread
// (a scalar pair per thread where alignment or the head size does not allow).
#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

__device__ __forceinline__ float silu_value(float v)
{
    return __fdiv_rn(v,__fadd_rn(1.0f,(float)exp(-(double)v)));
}

__device__ __forceinline__ float gelu_value(float v, bool tanh_form)
{
    float argument;
    if (tanh_form) {
        const float cubic = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f,v),v),v);
        argument = (float)tanh((double)__fmul_rn(0.7978845608028654f,__fadd_rn(v,cubic)));
    } else {
        argument = (float)erf((double)__fdiv_rn(v,1.4142135623730951f));
    }
    return __fmul_rn(__fmul_rn(0.5f,v),__fadd_rn(1.0f,argument));
}

template <int OP>
__global__ __launch_bounds__(256) void pointwise_kernel(float* __restrict__ x, const float* __restrict__ other, size_t count,
                                                        size_t channels)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float v = x[i];
        float r;
        if constexpr (OP == kOpSilu) r = silu_value(v);
        else if constexpr (OP == kOpGate) r = __fmul_rn(v,other[i]);
        else if constexpr (OP == kOpAdd) r = __fadd_rn(v,other[i]);
        else if constexpr (OP == kOpBias) r = __fadd_rn(v,other[i % channels]);
        else if constexpr (OP == kOpGeluExact) r = gelu_value(v,false);
        else r = gelu_value(v,true);
        x[i] = r;
    }
}

static unsigned grid_for(size_t work)
{
    return (unsigned)std::min<size_t>((work + 255) / 256,(size_t)1 << 20);
}

hipError_t launch_pointwise(int op, float* x, const float* other, size_t rows, size_t channels, hipStream_t s)
{
    const size_t count = rows * channels;
    if (!count) return hipSuccess;
    const dim3 g(grid_for(count)), b(256);
    switch (op) {
    case kOpSilu: pointwise_kernel<kOpSilu><<<g,b,0,s>>>(x,other,count,channels); break;
    case kOpGate: pointwise_kernel<kOpGate><<<g,b,0,s>>>(x,other,count,channels); break;
    case kOpAdd: pointwise_kernel<kOpAdd><<<g,b,0,s>>>(x,other,count,channels); break;
    case kOpBias: pointwise_kernel<kOpBias><<<g,b,0,s>>>(x,other,count,channels); break;
    case kOpGeluExact: pointwise_kernel<kOpGeluExact><<<g,b,0,s>>>(x,other,count,channels); break;
    case kOpGeluTanh: pointwise_kernel<kOpGeluTanh><<<g,b,0,s>>>(x,other,count,channels); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// One pair per thread: pair p of the rows x heads x dim/2 pairs.
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x, const float* __restrict__ cosine,
                                                   const float* __restrict__ sine, size_t rows, size_t heads, size_t dim,
                                                   bool interleaved)
{
    const size_t half = dim / 2, pairs = rows * heads * half;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += stride) {
        const size_t i = p % half, rh = p / half, row = rh / heads;
        float* data = x + rh * dim;  // row * channels + head * dim
        const size_t first = interleaved? 2 * i : i, second = interleaved? 2 * i + 1 : i + half;
        const float a = data[first], b = data[second];
        const float c = cosine[row * half + i], s = sine[row * half + i];
        data[first] = __fsub_rn(__fmul_rn(a,c),__fmul_rn(b,s));
        data[second] = __fadd_rn(__fmul_rn(a,s),__fmul_rn(b,c));
    }
}

// Four values per thread, same arithmetic: interleaved pairs (2i, 2i+1) two
// per float4 (head size a multiple of 4), or split halves (i, i + dim/2) a
// float4 of each half (head size a multiple of 8).  Grid: x over a row's
// float4 units (blocks of 256), y over rows (striding past 65535).  32-bit
// index math; no divisions by the head size in the inner step beyond one
// per thread.
template <bool INTERLEAVED>
__global__ __launch_bounds__(256) void rope4_kernel(float* __restrict__ x, const float* __restrict__ cosine,
                                                    const float* __restrict__ sine, uint32_t rows, uint32_t heads, uint32_t dim)
{
    const uint32_t half = dim / 2;
    const uint32_t per_head = INTERLEAVED? dim / 4 : half / 4;  // float4 units per head
    const uint32_t u = blockIdx.x * 256 + threadIdx.x;
    if (u >= heads * per_head) return;
    const uint32_t h = u / per_head, q = u - h * per_head;
    for (uint32_t row = blockIdx.y; row < rows; row += gridDim.y) {
        float* data = x + ((size_t)row * heads + h) * dim + 4 * q;
        if constexpr (INTERLEAVED) {
            const float4 v = *reinterpret_cast<const float4*>(data);
            const float2 c = *reinterpret_cast<const float2*>(cosine + (size_t)row * half + 2 * q);
            const float2 sn = *reinterpret_cast<const float2*>(sine + (size_t)row * half + 2 * q);
            float4 o;
            o.x = __fsub_rn(__fmul_rn(v.x,c.x),__fmul_rn(v.y,sn.x));
            o.y = __fadd_rn(__fmul_rn(v.x,sn.x),__fmul_rn(v.y,c.x));
            o.z = __fsub_rn(__fmul_rn(v.z,c.y),__fmul_rn(v.w,sn.y));
            o.w = __fadd_rn(__fmul_rn(v.z,sn.y),__fmul_rn(v.w,c.y));
            *reinterpret_cast<float4*>(data) = o;
        } else {
            const float4 a = *reinterpret_cast<const float4*>(data);
            const float4 b = *reinterpret_cast<const float4*>(data + half);
            const float4 c = *reinterpret_cast<const float4*>(cosine + (size_t)row * half + 4 * q);
            const float4 sn = *reinterpret_cast<const float4*>(sine + (size_t)row * half + 4 * q);
            const float as[4] = {a.x,a.y,a.z,a.w}, bs[4] = {b.x,b.y,b.z,b.w}, cs[4] = {c.x,c.y,c.z,c.w}, ss[4] = {sn.x,sn.y,sn.z,sn.w};
            float oa[4], ob[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                oa[e] = __fsub_rn(__fmul_rn(as[e],cs[e]),__fmul_rn(bs[e],ss[e]));
                ob[e] = __fadd_rn(__fmul_rn(as[e],ss[e]),__fmul_rn(bs[e],cs[e]));
            }
            *reinterpret_cast<float4*>(data) = make_float4(oa[0],oa[1],oa[2],oa[3]);
            *reinterpret_cast<float4*>(data + half) = make_float4(ob[0],ob[1],ob[2],ob[3]);
        }
    }
}

hipError_t launch_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, bool interleaved,
                       hipStream_t s)
{
    const size_t dim = channels / heads, pairs = rows * heads * (dim / 2);
    if (!pairs) return hipSuccess;
    auto at = [](const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
    const size_t units = interleaved? channels / 4 : channels / 8;
    const bool vec = at(x,16) && rows <= 0xffffffffu && channels <= 0xffffffffu &&
                     (interleaved? dim % 4 == 0 && at(cosine,8) && at(sine,8) : dim % 8 == 0 && at(cosine,16) && at(sine,16));
    if (vec) {
        const dim3 g((unsigned)((units + 255) / 256),(unsigned)std::min<size_t>(rows,65535)), b(256);
        if (interleaved) rope4_kernel<true><<<g,b,0,s>>>(x,cosine,sine,(uint32_t)rows,(uint32_t)heads,(uint32_t)dim);
        else rope4_kernel<false><<<g,b,0,s>>>(x,cosine,sine,(uint32_t)rows,(uint32_t)heads,(uint32_t)dim);
        return hipGetLastError();
    }
    rope_kernel<<<dim3(grid_for(pairs)),dim3(256),0,s>>>(x,cosine,sine,rows,heads,dim,interleaved);
    return hipGetLastError();
}

}  // namespace pixhip
