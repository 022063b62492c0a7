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
// HBM-bound: one value (RoPE: one pair) per thread, grid-stride.
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

hipError_t launch_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, bool interleaved,
                       hipStream_t s)
{
    const size_t dim = channels / heads, pairs = rows * heads * (dim / 2);
    if (!pairs) return hipSuccess;
    rope_kernel<<<dim3(grid_for(pairs)),dim3(256),0,s>>>(x,cosine,sine,rows,heads,dim,interleaved);
    return hipGetLastError();
}

}  // namespace pixhip
