// M=1 quantized matrix-vector product (decode step): y[n] = W[n][:] . x.
// The counterpart of shaders/matvec.comp:18-50 (chosen by VulkanState::multiply
// when M == 1, src/backend_vulkan.cpp:979) with the numerics of
// cpu_quant_matmul at columns == 1 (src/kernels_quant.cpp:369-412): x is first
// quantized exactly as quantize_row_q8_K_ref / quantize_row_q8_0_ref, then each
// row takes integer block dots and an fp32 epilogue.
//
// HBM-bound: every weight byte is read once with 128-bit loads; no MFMA.
// Each workgroup re-quantizes x into LDS (K <= 16384 values: 16 KB), then every
// wave streams whole rows: lane u owns one "unit" of 64 values of a row
// (Q5_K: a quarter super-block = two 32-value sub-blocks; Q8_0: two blocks;
// Q6_K: 16 positions x 4 groups of a half super-block) and the row total is a
// wave reduction.  Rows are dealt to waves in contiguous pairs so the whole
// matrix streams front to back.
#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

constexpr int kMvWaves = 4;
constexpr int kMvRows = 2;  // rows in flight per wave iteration

// Quantize x (K values) into LDS as Q8_K: qs, d per block, and the 16-value
// group sums.  All waves of the workgroup take part.
__device__ __forceinline__ void stage_x_q8_K(const float* __restrict__ x, int K, int8_t* sQ, float* sD, int* sB)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = K / PIX_QK;
    for (int b = wave; b < nb; b += kMvWaves) {
        float4 v = reinterpret_cast<const float4*>(x + b * PIX_QK)[lane];
        uint32_t packed;
        float d;
        int gsum;
        quantize_q8_K_wave(v,lane,packed,d,gsum);
        reinterpret_cast<uint32_t*>(sQ + b * PIX_QK)[lane] = packed;
        if (lane == 0) sD[b] = d;
        if ((lane & 3) == 0) sB[b * 16 + (lane >> 2)] = gsum;
    }
}

// Q8_0 staging over Kp = K rounded up to 64: the padding block is zero.
__device__ __forceinline__ void stage_x_q8_0(const float* __restrict__ x, int K, int Kp, int8_t* sQ, float* sD)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = K / PIX_QK8;
    if (Kp > K) {
        for (int i = threadIdx.x; i < Kp - K; i += blockDim.x) sQ[K + i] = 0;
        if (threadIdx.x == 0) sD[nb] = 0.0f;
    }
    for (int b0 = wave * 8; b0 < nb; b0 += kMvWaves * 8) {
        const int b = b0 + (lane >> 3);
        const int bl = b < nb? b : nb - 1;
        float4 v = reinterpret_cast<const float4*>(x + bl * PIX_QK8)[lane & 7];
        uint32_t packed;
        float d32;
        uint16_t dh;
        quantize_q8_0_group(v,packed,d32,dh);
        if (b < nb) {
            reinterpret_cast<uint32_t*>(sQ + b * PIX_QK8)[lane & 7] = packed;
            if ((lane & 7) == 0) sD[b] = half_bits_to_float(dh);
        }
    }
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a,(int)b,c,false);
}

__device__ __forceinline__ void store_row(const Output& out, size_t n, float v)
{
    out.y[out.offset + n] = v + (out.bias? out.bias[n] : 0.0f);
}

// ---------------------------------------------------------------- Q5_K (GGUF bytes)
template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q5_K_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                                    int N, int K, Output out, int rows_per_wave)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / PIX_QK;
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + K);
    int* sB = reinterpret_cast<int*>(smem + K + 4 * nb);
    stage_x_q8_K(x,K,sQ,sD,sB);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t row_bytes = (size_t)nb * PIX_Q5_K_BYTES;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * rows_per_wave;
    const int last = min(first + rows_per_wave,N);
    const int units = nb * 4;
    for (int r0 = first; r0 < last; r0 += kMvRows) {
        float part[kMvRows];
        uint4 head[kMvRows][UPL], qh0[kMvRows][UPL], qh1[kMvRows][UPL], qs0[kMvRows][UPL], qs1[kMvRows][UPL];
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            part[rr] = 0.0f;
            const int row = min(r0 + rr,last - 1);
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const int u = lane + 64 * k;
                if (u < units) {
                    const uint8_t* blk = w + (size_t)row * row_bytes + (size_t)(u >> 2) * PIX_Q5_K_BYTES;
                    const uint4* p = reinterpret_cast<const uint4*>(blk);
                    head[rr][k] = p[0];
                    qh0[rr][k] = p[1];
                    qh1[rr][k] = p[2];
                    qs0[rr][k] = p[3 + 2 * (u & 3)];
                    qs1[rr][k] = p[4 + 2 * (u & 3)];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = lane + 64 * k;
            if (u >= units) continue;
            const int b = u >> 2, j = u & 3;
            const uint4* xq = reinterpret_cast<const uint4*>(sQ + b * PIX_QK + 64 * j);
            const uint4 x0 = xq[0], x1 = xq[1], x2 = xq[2], x3 = xq[3];
            const uint32_t xa[8] = {x0.x,x0.y,x0.z,x0.w,x1.x,x1.y,x1.z,x1.w};
            const uint32_t xb[8] = {x2.x,x2.y,x2.z,x2.w,x3.x,x3.y,x3.z,x3.w};
            const float yd = sD[b];
            const int bs0 = sB[b * 16 + 4 * j] + sB[b * 16 + 4 * j + 1];
            const int bs1 = sB[b * 16 + 4 * j + 2] + sB[b * 16 + 4 * j + 3];
#pragma unroll
            for (int rr = 0; rr < kMvRows; rr++) {
                const uint4 h = head[rr][k];
                int sc0, mn0, sc1, mn1;
                q5_scale_min(h.y,h.z,h.w,2 * j,sc0,mn0);
                q5_scale_min(h.y,h.z,h.w,2 * j + 1,sc1,mn1);
                const uint32_t qhw[8] = {qh0[rr][k].x,qh0[rr][k].y,qh0[rr][k].z,qh0[rr][k].w,
                                         qh1[rr][k].x,qh1[rr][k].y,qh1[rr][k].z,qh1[rr][k].w};
                const uint32_t qsw[8] = {qs0[rr][k].x,qs0[rr][k].y,qs0[rr][k].z,qs0[rr][k].w,
                                         qs1[rr][k].x,qs1[rr][k].y,qs1[rr][k].z,qs1[rr][k].w};
                int dot0 = 0, dot1 = 0;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const uint32_t lo = qsw[q] & 0x0f0f0f0fu;
                    const uint32_t hi = (qsw[q] >> 4) & 0x0f0f0f0fu;
                    const uint32_t b0 = ((qhw[q] >> (2 * j)) & 0x01010101u) << 4;
                    const uint32_t b1 = ((qhw[q] >> (2 * j + 1)) & 0x01010101u) << 4;
                    dot0 = sdot4(lo | b0,xa[q],dot0);
                    dot1 = sdot4(hi | b1,xb[q],dot1);
                }
                const int S = sc0 * dot0 + sc1 * dot1;
                const int Mn = mn0 * bs0 + mn1 * bs1;
                const float wd = half_bits_to_float((uint16_t)(h.x & 0xffffu));
                const float wm = half_bits_to_float((uint16_t)(h.x >> 16));
                part[rr] = __builtin_fmaf(yd,__builtin_fmaf(-wm,(float)Mn,wd * (float)S),part[rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            const float v = wave_sum(part[rr]);
            if (lane == 0 && r0 + rr < last) store_row(out,(size_t)(r0 + rr),v);
        }
    }
}

// ---------------------------------------------------------------- Q8_0 (planar)
template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q8_0_kernel(PlanarQ80 w, const float* __restrict__ x, int N, int K,
                                                                    int Kp, Output out, int rows_per_wave)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nbp = Kp / PIX_QK8;
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + Kp);
    stage_x_q8_0(x,K,Kp,sQ,sD);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * rows_per_wave;
    const int last = min(first + rows_per_wave,N);
    const int units = Kp / 64;
    for (int r0 = first; r0 < last; r0 += kMvRows) {
        float part[kMvRows];
        uint4 q[kMvRows][UPL][4];
        uint32_t dd[kMvRows][UPL];
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            part[rr] = 0.0f;
            const int row = min(r0 + rr,last - 1);
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const int u = lane + 64 * k;
                if (u < units) {
                    const uint4* p = reinterpret_cast<const uint4*>(w.qs + (size_t)row * Kp + 64 * u);
#pragma unroll
                    for (int t = 0; t < 4; t++) q[rr][k][t] = p[t];
                    dd[rr][k] = *reinterpret_cast<const uint32_t*>(w.d + (size_t)row * nbp + 2 * u);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = lane + 64 * k;
            if (u >= units) continue;
            const uint4* xq = reinterpret_cast<const uint4*>(sQ + 64 * u);
            const uint4 x0 = xq[0], x1 = xq[1], x2 = xq[2], x3 = xq[3];
            const uint32_t xa[8] = {x0.x,x0.y,x0.z,x0.w,x1.x,x1.y,x1.z,x1.w};
            const uint32_t xb[8] = {x2.x,x2.y,x2.z,x2.w,x3.x,x3.y,x3.z,x3.w};
            const float xd0 = sD[2 * u], xd1 = sD[2 * u + 1];
#pragma unroll
            for (int rr = 0; rr < kMvRows; rr++) {
                const uint32_t wa[8] = {q[rr][k][0].x,q[rr][k][0].y,q[rr][k][0].z,q[rr][k][0].w,
                                        q[rr][k][1].x,q[rr][k][1].y,q[rr][k][1].z,q[rr][k][1].w};
                const uint32_t wb[8] = {q[rr][k][2].x,q[rr][k][2].y,q[rr][k][2].z,q[rr][k][2].w,
                                        q[rr][k][3].x,q[rr][k][3].y,q[rr][k][3].z,q[rr][k][3].w};
                int p0 = 0, p1 = 0;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    p0 = sdot4(wa[t],xa[t],p0);
                    p1 = sdot4(wb[t],xb[t],p1);
                }
                const float wd0 = half_bits_to_float((uint16_t)(dd[rr][k] & 0xffffu));
                const float wd1 = half_bits_to_float((uint16_t)(dd[rr][k] >> 16));
                part[rr] = __builtin_fmaf(wd0 * xd0,(float)p0,part[rr]);
                part[rr] = __builtin_fmaf(wd1 * xd1,(float)p1,part[rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            const float v = wave_sum(part[rr]);
            if (lane == 0 && r0 + rr < last) store_row(out,(size_t)(r0 + rr),v);
        }
    }
}

// ---------------------------------------------------------------- Q6_K (planar)
// Unit u of a row: super-block b = u/4, half h = (u/2)%2, position half ih = u%2;
// it covers elements 128h + 32g + 16ih + i for g = 0..3, i = 0..15.
template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q6_K_kernel(PlanarQ6K w, const float* __restrict__ x, int N, int K,
                                                                    Output out, int rows_per_wave)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / PIX_QK;
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + K);
    int* sB = reinterpret_cast<int*>(smem + K + 4 * nb);
    stage_x_q8_K(x,K,sQ,sD,sB);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * rows_per_wave;
    const int last = min(first + rows_per_wave,N);
    const int units = nb * 4;
    for (int r0 = first; r0 < last; r0 += kMvRows) {
        float part[kMvRows];
        uint4 la[kMvRows][UPL], lb[kMvRows][UPL], hh[kMvRows][UPL];
        uint2 scw[kMvRows][UPL];
        uint16_t dh[kMvRows][UPL];
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            part[rr] = 0.0f;
            const int row = min(r0 + rr,last - 1);
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const int u = lane + 64 * k;
                if (u < units) {
                    const int b = u >> 2, h = (u >> 1) & 1, ih = u & 1;
                    const uint8_t* ql = w.ql + (size_t)row * (K / 2) + b * 128 + 64 * h + 16 * ih;
                    la[rr][k] = *reinterpret_cast<const uint4*>(ql);
                    lb[rr][k] = *reinterpret_cast<const uint4*>(ql + 32);
                    hh[rr][k] = *reinterpret_cast<const uint4*>(w.qh + (size_t)row * (K / 4) + b * 64 + 32 * h + 16 * ih);
                    scw[rr][k] = *reinterpret_cast<const uint2*>(w.sc + (size_t)row * (K / 16) + b * 16 + 8 * h);
                    dh[rr][k] = __builtin_bit_cast(uint16_t,w.d[(size_t)row * nb + b]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = lane + 64 * k;
            if (u >= units) continue;
            const int b = u >> 2, h = (u >> 1) & 1, ih = u & 1;
            uint32_t xw[4][4];
            int bsg[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint4 t = *reinterpret_cast<const uint4*>(sQ + b * PIX_QK + 128 * h + 32 * g + 16 * ih);
                xw[g][0] = t.x; xw[g][1] = t.y; xw[g][2] = t.z; xw[g][3] = t.w;
                bsg[g] = sB[b * 16 + 8 * h + 2 * g + ih];
            }
            const float yd = sD[b];
#pragma unroll
            for (int rr = 0; rr < kMvRows; rr++) {
                const uint32_t lw[8] = {la[rr][k].x,la[rr][k].y,la[rr][k].z,la[rr][k].w,lb[rr][k].x,lb[rr][k].y,lb[rr][k].z,lb[rr][k].w};
                const uint32_t hw[4] = {hh[rr][k].x,hh[rr][k].y,hh[rr][k].z,hh[rr][k].w};
                const uint32_t s0 = scw[rr][k].x, s1 = scw[rr][k].y;
                int total = 0;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    int dot = 0;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t low = (g & 1)? lw[4 + q] : lw[q];
                        const uint32_t nib = (g < 2)? (low & 0x0f0f0f0fu) : ((low >> 4) & 0x0f0f0f0fu);
                        const uint32_t top = ((hw[q] >> (2 * g)) & 0x03030303u) << 4;
                        dot = sdot4(nib | top,xw[g][q],dot);
                    }
                    // scale of elements 128h + 32g + 16ih.. : byte 2g + ih of this half's 8 scales
                    const int sidx = 2 * g + ih;
                    const uint32_t sw = sidx < 4? s0 : s1;
                    const int sc = (int)(int8_t)(uint8_t)((sw >> (8 * (sidx & 3))) & 255u);
                    total += sc * (dot - 32 * bsg[g]);
                }
                const float wd = half_bits_to_float(dh[rr][k]);
                part[rr] = __builtin_fmaf(yd * wd,(float)total,part[rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < kMvRows; rr++) {
            const float v = wave_sum(part[rr]);
            if (lane == 0 && r0 + rr < last) store_row(out,(size_t)(r0 + rr),v);
        }
    }
}

// Rows per wave: enough waves to cover every CU several times over.
static int pick_rows_per_wave(size_t N)
{
    int rpw = 8;
    while (rpw > kMvRows && (N + (size_t)kMvWaves * rpw - 1) / ((size_t)kMvWaves * rpw) < 1024) rpw -= kMvRows;
    return rpw;
}

template <typename F>
static hipError_t dispatch_upl(int units, F&& f)
{
    if (units <= 64) return f(std::integral_constant<int,1>{});
    if (units <= 128) return f(std::integral_constant<int,2>{});
    if (units <= 192) return f(std::integral_constant<int,3>{});
    if (units <= 256) return f(std::integral_constant<int,4>{});
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_q5_K(const uint8_t* raw, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const int rpw = pick_rows_per_wave(N);
    const unsigned grid = (unsigned)((N + (size_t)kMvWaves * rpw - 1) / ((size_t)kMvWaves * rpw));
    const size_t nb = K / PIX_QK;
    const size_t lds = K + 4 * nb + 4 * 16 * nb;
    return dispatch_upl((int)(nb * 4),[&](auto upl) {
        matvec_q5_K_kernel<decltype(upl)::value><<<grid,64 * kMvWaves,lds,s>>>(raw,x,(int)N,(int)K,out,rpw);
        return hipGetLastError();
    });
}

hipError_t launch_matvec_q8_0(const PlanarQ80& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const int rpw = pick_rows_per_wave(N);
    const unsigned grid = (unsigned)((N + (size_t)kMvWaves * rpw - 1) / ((size_t)kMvWaves * rpw));
    const size_t Kp = (K + 63) / 64 * 64;
    const size_t lds = Kp + 4 * (Kp / PIX_QK8);
    return dispatch_upl((int)(Kp / 64),[&](auto upl) {
        matvec_q8_0_kernel<decltype(upl)::value><<<grid,64 * kMvWaves,lds,s>>>(w,x,(int)N,(int)K,(int)Kp,out,rpw);
        return hipGetLastError();
    });
}

hipError_t launch_matvec_q6_K(const PlanarQ6K& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const int rpw = pick_rows_per_wave(N);
    const unsigned grid = (unsigned)((N + (size_t)kMvWaves * rpw - 1) / ((size_t)kMvWaves * rpw));
    const size_t nb = K / PIX_QK;
    const size_t lds = K + 4 * nb + 4 * 16 * nb;
    return dispatch_upl((int)(nb * 4),[&](auto upl) {
        matvec_q6_K_kernel<decltype(upl)::value><<<grid,64 * kMvWaves,lds,s>>>(w,x,(int)N,(int)K,out,rpw);
        return hipGetLastError();
    });
}

}  // namespace pixhip
