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
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
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

// Cross-lane moves within rows of 16 lanes (DPP, no LDS traffic); every lane of
// the wave must be active.  XOR1 / XOR2 swap neighbours within quads; after
// those, HALF_MIRROR (lane i <-> 7-i of each 8) and MIRROR (i <-> 15-i of each
// 16) complete a reduction over 8 and 16 lanes.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v)
{
    return __builtin_bit_cast(float,__builtin_amdgcn_update_dpp(0,__builtin_bit_cast(int,v),CTRL,0xf,0xf,false));
}
template <int CTRL> __device__ __forceinline__ int dpp_i32(int v)
{
    return __builtin_amdgcn_update_dpp(0,v,CTRL,0xf,0xf,false);
}
__device__ __forceinline__ float lane_f32(float v, int lane)
{
    return __builtin_bit_cast(float,__builtin_amdgcn_readlane(__builtin_bit_cast(int,v),lane));
}

// Sum over the 64 lanes (every lane active), returned to every lane: rows of
// 16 by DPP, then the four row sums in order.
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    v += dpp_f32<kDppMirror>(v);
    return (lane_f32(v,0) + lane_f32(v,16)) + (lane_f32(v,32) + lane_f32(v,48));
}

template <int CTRL> __device__ __forceinline__ double dpp_f64(double v)
{
    const int2 h = __builtin_bit_cast(int2,v);
    return __builtin_bit_cast(double,make_int2(dpp_i32<CTRL>(h.x),dpp_i32<CTRL>(h.y)));
}
__device__ __forceinline__ double lane_f64(double v, int lane)
{
    const int2 h = __builtin_bit_cast(int2,v);
    return __builtin_bit_cast(double,make_int2(__builtin_amdgcn_readlane(h.x,lane),__builtin_amdgcn_readlane(h.y,lane)));
}

// Sum over the 64 lanes in double (every lane active), the same value in every
// lane: rows of 16 by DPP, then the four row sums in order.
__device__ __forceinline__ double wave_sum_f64(double v)
{
    v += dpp_f64<kDppXor1>(v);
    v += dpp_f64<kDppXor2>(v);
    v += dpp_f64<kDppHalfMirror>(v);
    v += dpp_f64<kDppMirror>(v);
    return (lane_f64(v,0) + lane_f64(v,16)) + (lane_f64(v,32) + lane_f64(v,48));
}

// One Q8_K block (256 values) quantized by one full wave, 4 consecutive values
// per lane (lane l holds x[4l..4l+3]).  Semantics of quantize_row_q8_K_ref
// (src/kernels_quant.cpp:80-118):
//   max = the first x with the largest |x| (strict '>' scan, :89-95), so ties
//   go to the lowest index;  amax == 0 zeroes the block (:96-102);
//   iscale = -127/max;  q = min(127, nearest_int(iscale*x));  bsums = sums of
//   16;  d = 1/iscale.
// Outputs: packed 4 quantized bytes of this lane, the block scale d, and the
// sum of the 16-value group this lane belongs to (group = lane/4).
// The largest |x| is reduced over the wave; the sign of its first occurrence
// comes from ballots of |x| == amax and x < 0 per element position (wave-
// uniform bit work on the scalar unit).  The quantized values are the low
// bytes of the fused multiply-add's bit patterns, packed by v_perm, and a
// lane's 4-value sum is one signed dot product of its packed bytes with ones.
__device__ __forceinline__ void quantize_q8_K_wave(float4 v, int lane, uint32_t& packed, float& d, int& group_sum)
{
    (void)lane;
    float xs[4] = {v.x,v.y,v.z,v.w};
    // largest |x| (NaN never compares greater, as in the reference's scan).
    // The lane's maximum is a non-negative float, never NaN, so the wave
    // maximum is the unsigned maximum of the bit patterns.
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) m = fabsf(xs[i]) > m? fabsf(xs[i]) : m;
    uint32_t mb = __float_as_uint(m);
    mb = max(mb,(uint32_t)dpp_i32<kDppXor1>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppXor2>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppHalfMirror>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppMirror>((int)mb));
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)mb,0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)mb,16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)mb,32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)mb,48);
    const float amax = __uint_as_float(max(max(r0,r1),max(r2,r3)));
    if (amax == 0.0f) {
        packed = 0;
        d = 0.0f;
        group_sum = 0;
        return;
    }
    // the first x (lowest index 4*lane + i) whose |x| is that maximum: the
    // lowest lane holding one, then its lowest position; only its sign is
    // needed (its magnitude is amax)
    uint64_t eq[4], ng[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        eq[i] = __builtin_amdgcn_ballot_w64(fabsf(xs[i]) == amax);
        ng[i] = __builtin_amdgcn_ballot_w64(xs[i] < 0.0f);
    }
    const uint64_t bit = 1ull << __builtin_ctzll(eq[0] | eq[1] | eq[2] | eq[3]);
    const uint64_t neg = (eq[0] & bit)? ng[0] : (eq[1] & bit)? ng[1] : (eq[2] & bit)? ng[2] : ng[3];
    const float mval = __builtin_bit_cast(float,__builtin_bit_cast(uint32_t,amax) | ((neg & bit)? 0x80000000u : 0u));
    const float iscale = __fdiv_rn(-127.0f,mval);
    uint32_t t[4];
#pragma unroll
    for (int i = 0; i < 4; i++) t[i] = (uint32_t)min(nearest_int_fused(iscale,xs[i]),127);
    // low bytes of t[0..3] -> bytes 0..3 (0x0c selects a zero byte)
    packed = __builtin_amdgcn_perm(t[1],t[0],0x0c0c0400u) | __builtin_amdgcn_perm(t[3],t[2],0x04000c0cu);
    int s = __builtin_amdgcn_sdot4((int)packed,0x01010101,0,false);
    s += dpp_i32<kDppXor1>(s);
    s += dpp_i32<kDppXor2>(s);
    group_sum = s;
    d = __fdiv_rn(1.0f,iscale);
}

// Four Q8_K blocks quantized by one wave, 16 lanes per block, with the
// semantics of quantize_q8_K_wave.  Lane l works on block l/16 and holds its
// values 64j + 4(l%16) .. +3 in v[j] (j = 0..3): for each j the block's 16
// lanes read 256 contiguous bytes.  Outputs: packed[j], the four quantized
// bytes of v[j]; d, the block scale (the same in the block's 16 lanes);
// gsum[j], the sum of the block's 16-value group 4j + (l%16)/4 (the same in
// a lane quad).  Per-block work (the maximum, the sign of its first
// occurrence, the two divisions) is shared by four blocks per instruction.
//   The first largest |x| of the block: each lane scans its values in
//   position order (j, then the four of v[j]) with a strict '>' (NaN never
//   wins); the block maximum is the unsigned maximum of the lanes' bit
//   patterns over the 16 lanes; among the lanes whose own maximum equals it,
//   the earliest (smallest j, then lane) holds the first occurrence, whose
//   sign it broadcasts.
__device__ __forceinline__ void quantize_q8_K_x4(const float4 (&v)[4], int lane, uint32_t (&packed)[4], float& d, int (&gsum)[4])
{
    const uint32_t lp = (uint32_t)(lane & 15);
    float M = 0.0f, S = 0.0f;
    uint32_t J = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float xs[4] = {v[j].x,v[j].y,v[j].z,v[j].w};
        float m = 0.0f, s = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float ax = fabsf(xs[e]);
            const bool gt = ax > m;
            m = gt? ax : m;
            s = gt? xs[e] : s;
        }
        const bool gt = m > M;
        M = gt? m : M;
        S = gt? s : S;
        J = gt? (uint32_t)j : J;
    }
    uint32_t mb = __float_as_uint(M);
    mb = max(mb,(uint32_t)dpp_i32<kDppXor1>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppXor2>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppHalfMirror>((int)mb));
    mb = max(mb,(uint32_t)dpp_i32<kDppMirror>((int)mb));
    const float amax = __uint_as_float(mb);
    const uint32_t own = J * 16 + lp;
    uint32_t key = M == amax? own : 0xffu;
    key = min(key,(uint32_t)dpp_i32<kDppXor1>((int)key));
    key = min(key,(uint32_t)dpp_i32<kDppXor2>((int)key));
    key = min(key,(uint32_t)dpp_i32<kDppHalfMirror>((int)key));
    key = min(key,(uint32_t)dpp_i32<kDppMirror>((int)key));
    uint32_t neg = (own == key && S < 0.0f)? 1u : 0u;
    neg = max(neg,(uint32_t)dpp_i32<kDppXor1>((int)neg));
    neg = max(neg,(uint32_t)dpp_i32<kDppXor2>((int)neg));
    neg = max(neg,(uint32_t)dpp_i32<kDppHalfMirror>((int)neg));
    neg = max(neg,(uint32_t)dpp_i32<kDppMirror>((int)neg));
    const bool zero = amax == 0.0f;
    const float mval = __uint_as_float(mb | (neg << 31));
    const float iscale = __fdiv_rn(-127.0f,mval);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float xs[4] = {v[j].x,v[j].y,v[j].z,v[j].w};
        uint32_t t[4];
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = (uint32_t)min(nearest_int_fused(iscale,xs[e]),127);
        const uint32_t p = __builtin_amdgcn_perm(t[1],t[0],0x0c0c0400u) | __builtin_amdgcn_perm(t[3],t[2],0x04000c0cu);
        packed[j] = zero? 0u : p;
        int s = __builtin_amdgcn_sdot4((int)packed[j],0x01010101,0,false);
        s += dpp_i32<kDppXor1>(s);
        s += dpp_i32<kDppXor2>(s);
        gsum[j] = s;
    }
    d = zero? 0.0f : __fdiv_rn(1.0f,iscale);
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
    amax = fmaxf(amax,dpp_f32<kDppXor1>(amax));
    amax = fmaxf(amax,dpp_f32<kDppXor2>(amax));
    amax = fmaxf(amax,dpp_f32<kDppHalfMirror>(amax));
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
