// Device-side helpers shared by the kernels: the exact activation quantizers
// (one wave per block) and small wave utilities.  Built with
// -ffp-contract=off: every fused multiply-add below is written explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pixhip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float half_bits_to_float(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16,h);
}

// Round-to-nearest-even fp32 -> fp16 bits, subnormals kept (v_cvt_f16_f32 in
// the default round-to-nearest mode with fp16 denormals enabled).
__device__ __forceinline__ uint16_t float_to_half_bits(float f)
{
    return __builtin_bit_cast(uint16_t,(_Float16)f);
}

// nearest_int(iscale*x) of quantize_row_q8_K_ref as the reference compiles it
// (src/kernels_quant.cpp:41-48, :105): one fused multiply-add into the
// 1.5*2^23 rounding bias, then the low mantissa bits.
__device__ __forceinline__ int nearest_int_fused(float scale, float x)
{
    float v = __builtin_fmaf(scale,x,12582912.0f);
    return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d)
{
    return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)(d & 255) << 24);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v,o,64);
    return v;
}

// One Q8_K block (256 values) quantized by one full wave, 4 consecutive values
// per lane (lane l holds x[4l..4l+3]).  Semantics of quantize_row_q8_K_ref
// (src/kernels_quant.cpp:80-118):
//   max = the first x with the largest |x| (strict '>' scan, :89-95), so the
//   wave arg-max breaks ties toward the lowest index;  amax == 0 zeroes the
//   block (:96-102);  iscale = -127/max;  q = min(127, nearest_int(iscale*x));
//   bsums = sums of 16;  d = 1/iscale.
// Outputs: packed 4 quantized bytes of this lane, the block scale d, and the
// sum of the 16-value group this lane belongs to (group = lane/4).
__device__ __forceinline__ void quantize_q8_K_wave(float4 v, int lane, uint32_t& packed, float& d, int& group_sum)
{
    float xs[4] = {v.x,v.y,v.z,v.w};
    float amax = 0.0f, mval = 0.0f;
    int idx = 1 << 30;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float ax = fabsf(xs[i]);
        if (ax > amax) {
            amax = ax;
            mval = xs[i];
            idx = 4 * lane + i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float oa = __shfl_xor(amax,o,64);
        float ov = __shfl_xor(mval,o,64);
        int oi = __shfl_xor(idx,o,64);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            mval = ov;
            idx = oi;
        }
    }
    if (amax == 0.0f) {
        packed = 0;
        d = 0.0f;
        group_sum = 0;
        return;
    }
    float iscale = __fdiv_rn(-127.0f,mval);
    int q[4];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int t = nearest_int_fused(iscale,xs[i]);
        t = t < 127? t : 127;
        q[i] = (int)(int8_t)(uint8_t)(t & 255);
        s += q[i];
    }
    packed = pack_bytes(q[0],q[1],q[2],q[3]);
    s += __shfl_xor(s,1,64);
    s += __shfl_xor(s,2,64);
    group_sum = s;
    d = __fdiv_rn(1.0f,iscale);
}

// One Q8_0 block (32 values) quantized by 8 lanes holding 4 consecutive values
// each (the 8-lane group is aligned: lanes 8g..8g+7).  Semantics of
// quantize_row_q8_0_ref (src/kernels_quant.cpp:120-144): amax = max|x| with
// NaNs ignored (std::max(amax,|x|)), d = amax/127, id = d ? 1/d : 0,
// stored scale fp16_rne(d), q = (int8)roundf(x*id) (round half away from zero).
__device__ __forceinline__ void quantize_q8_0_group(float4 v, uint32_t& packed, float& d32, uint16_t& dh)
{
    float xs[4] = {v.x,v.y,v.z,v.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float ax = fabsf(xs[i]);
        amax = (amax < ax)? ax : amax;
    }
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) {
        float oa = __shfl_xor(amax,o,64);
        amax = (amax < oa)? oa : amax;
    }
    d32 = __fdiv_rn(amax,127.0f);
    float id = (d32 != 0.0f)? __fdiv_rn(1.0f,d32) : 0.0f;
    dh = float_to_half_bits(d32);
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = (int)roundf(__fmul_rn(xs[i],id));
    packed = pack_bytes(q[0],q[1],q[2],q[3]);
}

// Unpack the six-bit scale and minimum of sub-block s (0..7) of a Q5_K block
// from its 12 packed bytes, given as three little-endian words
// (src/backend_cpu.cpp:64-70; src/kernels_quant.cpp:189-194).
__device__ __forceinline__ void q5_scale_min(uint32_t w0, uint32_t w1, uint32_t w2, int s, int& scale, int& min)
{
    auto byte = [&](int i) -> int {
        uint32_t w = i < 4? w0 : (i < 8? w1 : w2);
        return (int)((w >> (8 * (i & 3))) & 255u);
    };
    if (s < 4) {
        scale = byte(s) & 63;
        min = byte(s + 4) & 63;
    } else {
        scale = (byte(s + 4) & 15) | ((byte(s - 4) >> 6) << 4);
        min = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
}

}  // namespace pixhip
