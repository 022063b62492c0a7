// Upload-time weight conversion for the resident cache (the counterpart of
// VulkanState::weight, src/backend_vulkan.cpp:742-758, which keeps GGUF bytes).
// Runs once per cached tensor; the GEMM and matvec kernels then read
// layouts that suit MFMA operands and aligned 128-bit loads.
//
// Q5_K planes: the super-block value is d*scale_s*q - dmin*min_s with q in
// [0,31] and scale_s in [0,63] (src/backend_cpu.cpp:56-79).  The product
// p = scale_s*q <= 1953 is split exactly into two int8 planes p = 64*hi + lo,
// hi in [0,30], lo in [0,63], so one int8 MFMA per plane yields the exact
// integer sum_s scale_s*dot_s of pix_dot_q5_K (src/kernels_quant.cpp:214-245)
// with the sub-block scales already applied.
#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

__device__ __forceinline__ uint32_t load_u32_aligned(const uint8_t* p)
{
    return *reinterpret_cast<const uint32_t*>(p);
}

__device__ __forceinline__ uint32_t load_u32_bytes(const uint8_t* p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// One wave per Q5_K super-block; lane l converts values 4l..4l+3 (sub-block l/8).
__global__ __launch_bounds__(256) void repack_q5_K_kernel(const uint8_t* __restrict__ raw, size_t rows, size_t inner,
                                                          size_t npad, int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                          float* __restrict__ d, float* __restrict__ dm,
                                                          _Float16* __restrict__ mn)
{
    const size_t nb = inner / PIX_QK;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= rows * nb) return;
    const int lane = threadIdx.x & 63;
    const size_t row = blk / nb, b = blk % nb;
    const uint8_t* src = raw + blk * PIX_Q5_K_BYTES;
    const uint32_t head = load_u32_aligned(src);
    const uint32_t w0 = load_u32_aligned(src + 4), w1 = load_u32_aligned(src + 8), w2 = load_u32_aligned(src + 12);
    const int s = lane >> 3, i0 = 4 * (lane & 7);
    int scale, min;
    q5_scale_min(w0,w1,w2,s,scale,min);
    const uint32_t qh = load_u32_aligned(src + 16 + i0);
    const uint32_t ql = load_u32_aligned(src + 48 + (s >> 1) * 32 + i0);
    int h[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int q = (int)((ql >> (8 * k + 4 * (s & 1))) & 15u) | (int)(((qh >> (8 * k + s)) & 1u) << 4);
        int p = scale * q;
        h[k] = p >> 6;
        l[k] = p & 63;
    }
    const size_t off = tiled_offset(row,b * PIX_QK + 4 * lane,inner);
    *reinterpret_cast<uint32_t*>(hi + off) = pack_bytes(h[0],h[1],h[2],h[3]);
    *reinterpret_cast<uint32_t*>(lo + off) = pack_bytes(l[0],l[1],l[2],l[3]);
    if (lane == 0) {
        d[b * npad + row] = half_bits_to_float((uint16_t)(head & 0xffffu));
        dm[b * npad + row] = half_bits_to_float((uint16_t)(head >> 16));
    }
    if ((lane & 7) == 0) mn[(b * npad + row) * 8 + s] = (_Float16)(float)min;
}

// Q6_K value d*scale_{e/16}*(q-32) (src/backend_cpu.cpp:80-96): p = scale*(q-32)
// lies in [-4064, 4096] and is split p = 64*hi + lo, hi in [-64,64], lo in [0,63].
__device__ __forceinline__ int q6_raw_value(const uint8_t* src, int e)
{
    int h = e >> 7, g = (e & 127) >> 5, i = e & 31;
    int low = src[64 * h + i + (g & 1) * 32];
    low = g < 2? (low & 15) : (low >> 4);
    return low | (((src[128 + 32 * h + i] >> (2 * g)) & 3) << 4);
}

__global__ __launch_bounds__(256) void repack_q6_K_planes_kernel(const uint8_t* __restrict__ raw, size_t rows, size_t inner,
                                                                 size_t npad, int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                                 float* __restrict__ d)
{
    const size_t nb = inner / PIX_QK;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= rows * nb) return;
    const int lane = threadIdx.x & 63;
    const size_t row = blk / nb, b = blk % nb;
    const uint8_t* src = raw + blk * PIX_Q6_K_BYTES;
    int h[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int e = 4 * lane + k;
        int sc = (int)(int8_t)src[192 + (e >> 4)];
        int p = sc * (q6_raw_value(src,e) - 32);
        h[k] = p >> 6;
        l[k] = p & 63;
    }
    const size_t off = tiled_offset(row,b * PIX_QK + 4 * lane,inner);
    *reinterpret_cast<uint32_t*>(hi + off) = pack_bytes(h[0],h[1],h[2],h[3]);
    *reinterpret_cast<uint32_t*>(lo + off) = pack_bytes(l[0],l[1],l[2],l[3]);
    if (lane == 0) d[b * npad + row] = half_bits_to_float((uint16_t)(src[208] | (src[209] << 8)));
}

// Q6_K re-sliced into aligned planes of identical total size (matvec input).
__global__ __launch_bounds__(256) void repack_q6_K_planar_kernel(const uint8_t* __restrict__ raw, size_t rows, size_t inner,
                                                                 uint8_t* __restrict__ ql, uint8_t* __restrict__ qh,
                                                                 int8_t* __restrict__ sc, _Float16* __restrict__ d)
{
    const size_t nb = inner / PIX_QK;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= rows * nb) return;
    const int lane = threadIdx.x & 63;
    const size_t row = blk / nb, b = blk % nb;
    const uint8_t* src = raw + blk * PIX_Q6_K_BYTES;
    // 210 bytes: ql 0..127, qh 128..191, scales 192..207, d 208..209.
    // ql byte j of the block (half h = j/64, r = j%64) belongs to 64-value unit
    // u = 4b + 2h + (r%32)/16, as its first 16-byte piece when r < 32 and its
    // second when r >= 32.  The row's ql is stored as two planes of pieces,
    // unit-major (first pieces at u*16, second at (units + u)*16), so that a
    // load of either piece by 64 lanes reading consecutive units is one
    // contiguous 1 KB run.
    const size_t units = inner / 64;
    uint8_t* qrow = ql + row * (inner / 2);
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int r = lane;  // byte 64*hh + lane
        const size_t u = 4 * b + 2 * hh + ((r & 31) >> 4);
        qrow[((r < 32? 0 : units) + u) * 16 + (r & 15)] = src[64 * hh + lane];
    }
    qh[row * (inner / 4) + b * 64 + lane] = src[128 + lane];
    if (lane < 16) sc[row * (inner / 16) + b * 16 + lane] = (int8_t)src[192 + lane];
    if (lane == 0) d[row * nb + b] = __builtin_bit_cast(_Float16,(uint16_t)(src[208] | (src[209] << 8)));
}

// Q8_0: 34-byte blocks (2-byte aligned) -> the GEMM form (int8 plane, fp32
// transposed scales) and/or the matvec form (piece-major int8 rows, fp16
// scales), both with row stride kpad (the caller zero-fills the padding once
// at allocation).  One 8-lane group per block, 4 values per lane.
// Block b of a row holds values 32b..32b+31: unit b/2, 16-byte pieces
// 2(b%2) and 2(b%2)+1 of it.  The matvec form stores piece p of unit u at
// (p*units + u)*16 in the row, so that a load of piece p by 64 lanes reading
// consecutive units is one contiguous 1 KB run.
__global__ __launch_bounds__(256) void repack_q8_0_kernel(const uint8_t* __restrict__ raw, size_t rows, size_t inner,
                                                          size_t kpad, size_t rows_pad, int8_t* __restrict__ qs,
                                                          float* __restrict__ dT, int8_t* __restrict__ qs_mv,
                                                          _Float16* __restrict__ d)
{
    const size_t nb = inner / PIX_QK8, units = kpad / 64;
    const size_t blk = ((size_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    if (blk >= rows * nb) return;
    const int part = threadIdx.x & 7;
    const size_t row = blk / nb, b = blk % nb;
    const uint8_t* src = raw + blk * PIX_Q8_0_BYTES;
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src + 2 + 4 * part);
    uint32_t v = (uint32_t)s16[0] | ((uint32_t)s16[1] << 16);
    const uint16_t h = *reinterpret_cast<const uint16_t*>(src);
    if (qs) {
        *reinterpret_cast<uint32_t*>(qs + row * kpad + b * PIX_QK8 + 4 * part) = v;
        if (part == 0) dT[b * rows_pad + row] = half_bits_to_float(h);
    }
    if (qs_mv) {
        const size_t piece = 2 * (b & 1) + (part >> 2), u = b >> 1;
        *reinterpret_cast<uint32_t*>(qs_mv + row * kpad + (piece * units + u) * 16 + 4 * (part & 3)) = v;
        if (part == 0) d[row * (kpad / PIX_QK8) + b] = __builtin_bit_cast(_Float16,h);
    }
}

static unsigned waves_grid(size_t blocks) { return (unsigned)((blocks + 3) / 4); }

hipError_t launch_repack_q5_K(const uint8_t* raw, size_t rows, size_t inner, size_t npad, int8_t* hi, int8_t* lo, float* d,
                              float* dm, _Float16* mn, hipStream_t s)
{
    size_t blocks = rows * (inner / PIX_QK);
    if (!blocks) return hipSuccess;
    repack_q5_K_kernel<<<waves_grid(blocks),256,0,s>>>(raw,rows,inner,npad,hi,lo,d,dm,mn);
    return hipGetLastError();
}

hipError_t launch_repack_q6_K_planes(const uint8_t* raw, size_t rows, size_t inner, size_t npad, int8_t* hi, int8_t* lo, float* d,
                                     hipStream_t s)
{
    size_t blocks = rows * (inner / PIX_QK);
    if (!blocks) return hipSuccess;
    repack_q6_K_planes_kernel<<<waves_grid(blocks),256,0,s>>>(raw,rows,inner,npad,hi,lo,d);
    return hipGetLastError();
}

// Q5_K matvec form: one thread per 64-value unit (the nibbles are copied, the
// rest re-sliced into the unit's 12-byte record).
__global__ __launch_bounds__(256) void repack_q5_K_planar_kernel(const uint8_t* __restrict__ raw, size_t rows, size_t inner,
                                                                 uint8_t* __restrict__ qs, uint32_t* __restrict__ rec)
{
    const size_t units = inner / 64;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * units) return;
    const size_t row = t / units, u = t % units, b = u / 4;
    const int j = (int)(u % 4);
    const uint8_t* src = raw + (row * (inner / PIX_QK) + b) * PIX_Q5_K_BYTES;
    // 176 bytes: d, dmin 0..3, scales 4..15, qh 16..47, qs 48..175
    // The unit's 32 nibble bytes go to two half planes of the row (bytes 0..15
    // at 16u, bytes 16..31 at 16 * (units + u)): each of the matvec's two
    // 16-B loads is then contiguous across the lanes of a wave.
    const uint4* q4 = reinterpret_cast<const uint4*>(src + 48 + 32 * j);
    uint4* dq = reinterpret_cast<uint4*>(qs + row * (inner / 2));
    dq[u] = q4[0];
    dq[units + u] = q4[1];
    uint32_t h[2] = {0,0};
    for (int q = 0; q < 8; q++) {
        const uint32_t w = load_u32_aligned(src + 16 + 4 * q);
        h[q >> 2] |= ((w >> (2 * j)) & 0x03030303u) << (2 * (q & 3));
    }
    const uint32_t w0 = load_u32_aligned(src + 4), w1 = load_u32_aligned(src + 8), w2 = load_u32_aligned(src + 12);
    int sc0, mn0, sc1, mn1;
    q5_scale_min(w0,w1,w2,2 * j,sc0,mn0);
    q5_scale_min(w0,w1,w2,2 * j + 1,sc1,mn1);
    uint32_t* r = rec + (row * units + u) * 3;
    r[0] = h[0];
    r[1] = h[1];
    r[2] = (uint32_t)sc0 | ((uint32_t)sc1 << 6) | ((uint32_t)mn0 << 12) | ((uint32_t)mn1 << 18) |
           (((load_u32_aligned(src) >> (8 * j)) & 255u) << 24);
}

hipError_t launch_repack_q5_K_planar(const uint8_t* raw, size_t rows, size_t inner, uint8_t* qs, uint32_t* rec, hipStream_t s)
{
    const size_t n = rows * (inner / 64);
    if (!n) return hipSuccess;
    repack_q5_K_planar_kernel<<<dim3((unsigned)((n + 255) / 256)),256,0,s>>>(raw,rows,inner,qs,rec);
    return hipGetLastError();
}

hipError_t launch_repack_q6_K_planar(const uint8_t* raw, size_t rows, size_t inner, uint8_t* ql, uint8_t* qh, int8_t* sc,
                                     _Float16* d, hipStream_t s)
{
    size_t blocks = rows * (inner / PIX_QK);
    if (!blocks) return hipSuccess;
    repack_q6_K_planar_kernel<<<waves_grid(blocks),256,0,s>>>(raw,rows,inner,ql,qh,sc,d);
    return hipGetLastError();
}

hipError_t launch_repack_q8_0(const uint8_t* raw, size_t rows, size_t inner, size_t kpad, size_t rows_pad, int8_t* qs, float* dT,
                              int8_t* qs_mv, _Float16* d, hipStream_t s)
{
    size_t blocks = rows * (inner / PIX_QK8);
    if (!blocks) return hipSuccess;
    repack_q8_0_kernel<<<(unsigned)((blocks * 8 + 255) / 256),256,0,s>>>(raw,rows,inner,kpad,rows_pad,qs,dT,qs_mv,d);
    return hipGetLastError();
}

}  // namespace pixhip
