// Activation block quantizers (the counterpart of quantize_row_q8_0_ref /
// quantize_row_q8_K_ref, src/kernels_quant.cpp:80-144, and of the GPU pass
// shaders/quantize.comp:13-41 that precedes MMQ).  Each launch writes the
// planar layout the GEMM reads and, when asked, the reference's own block
// layout (block_q8_0 / block_q8_K) for callers and for the integer parity gate.
//
// HBM-bound byte work: 16 lanes per Q8_K block (four blocks per wave, a
// float4 per lane and block quarter), one 8-lane group per Q8_0 block; reads
// 4 B/value, writes ~1.1 B/value.
// A workgroup covers one chunk of a group of consecutive rows (kQuantRows,
// kQ8KRows).
#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

constexpr int kQuantWaves = 8;  // waves per workgroup: 8 measured ~12% faster than 4 or 16 (Q8_K, 4096x3840)
// Rows per workgroup.  A Q8_0 workgroup quantizes one 256-value chunk of
// kQuantRows consecutive rows (wave w: rows w, w + kQuantWaves, ...), so each
// block's transposed scales dT[b * mpad + row] leave it as 64-byte runs rather
// than as 4-byte pieces from workgroups spread over the XCDs.  On [4608, 10240]:
// 38.4 us with 16 rows, 40.5 with 8, 39.5 with 32, 38.5 with 64, 45.7 with one
// row's 8 consecutive chunks per workgroup.
constexpr int kQuantRows = 16;
constexpr int kQuantPer = kQuantRows / kQuantWaves;  // rows per wave
// Q8_K: a wave quantizes one block of four consecutive rows, 16 lanes per
// row (quantize_q8_K_x4), and a workgroup one block of 4 * kQuantWaves rows:
// its scales leave as one 128-byte run of dT, its 16-value sums as 32 rows of
// the tiled bs plane (one 1 KB block), its bytes as whole 64-byte row pieces.
constexpr int kQ8KRows = 4 * kQuantWaves;

// The workgroup is (row group, block), block fastest.
__global__ __launch_bounds__(64 * kQuantWaves) void quantize_q8_K_kernel(const float* __restrict__ x, size_t rows, size_t inner,
                                                                         size_t mpad, int8_t* __restrict__ qs, float* __restrict__ dT,
                                                                         _Float16* __restrict__ bs, uint8_t* __restrict__ blocks)
{
    const uint32_t nb = (uint32_t)(inner / PIX_QK);
    const uint32_t group = blockIdx.x / nb, b = blockIdx.x % nb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lp = lane & 15;
    const size_t row = (size_t)group * kQ8KRows + 4 * wave + (lane >> 4);
    const size_t r = row < rows? row : rows - 1;  // loads from a clamped row
    const size_t k0 = (size_t)b * PIX_QK + 4 * lp;
    const float* src = x + r * inner + k0;
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = *reinterpret_cast<const float4*>(src + 64 * j);
    uint32_t packed[4];
    float d;
    int gsum[4];
    quantize_q8_K_x4(v,lane,packed,d,gsum);
    if (row >= rows) return;
    if (qs) {
        // values k0 + 64j are in consecutive 1 KB pieces of the row group
        int8_t* q = qs + tiled_offset(row,k0,inner);
#pragma unroll
        for (int j = 0; j < 4; j++) *reinterpret_cast<uint32_t*>(q + 1024 * j) = packed[j];
        if (lp == 0) dT[(size_t)b * mpad + row] = d;
        // group g = 4j + lp/4 stored at (g&1)*8 + g/2: even groups first, then odd
        if ((lp & 3) == 0) {
            _Float16* o = bs + tiled_bs_index(row,b,0,inner);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = 4 * j + (lp >> 2);
                o[(g & 1) * 8 + (g >> 1)] = (_Float16)(float)gsum[j];
            }
        }
    }
    if (blocks) {
        uint8_t* blk = blocks + (row * nb + b) * PIX_Q8_K_BYTES;
#pragma unroll
        for (int j = 0; j < 4; j++) *reinterpret_cast<uint32_t*>(blk + 4 + 64 * j + 4 * lp) = packed[j];
        if (lp == 0) *reinterpret_cast<float*>(blk) = d;
        if ((lp & 3) == 0) {
#pragma unroll
            for (int j = 0; j < 4; j++) reinterpret_cast<int16_t*>(blk + 4 + PIX_QK)[4 * j + (lp >> 2)] = (int16_t)gsum[j];
        }
    }
}

// Planar rows have stride kpad = inner rounded up to 64; the padding block
// (when inner % 64 == 32) is written as zeros with a zero scale so it adds
// exactly nothing to a dot product.  A wave quantizes 8 blocks (one 256-value
// chunk) of a row, one 8-lane group per block; the workgroup is (row group,
// chunk), chunk fastest.
__global__ __launch_bounds__(64 * kQuantWaves) void quantize_q8_0_kernel(const float* __restrict__ x, size_t rows, size_t inner,
                                                                         size_t kpad, size_t mpad, int8_t* __restrict__ qs,
                                                                         float* __restrict__ dT, uint8_t* __restrict__ blocks)
{
    const uint32_t nb = (uint32_t)(inner / PIX_QK8), nbp = (uint32_t)(kpad / PIX_QK8), nch = (nbp + 7) / 8;
    const uint32_t group = blockIdx.x / nch, c = blockIdx.x % nch;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t b = c * 8 + (lane >> 3);
    // Groups past the row's real blocks read the last real block (every lane
    // joins the 8-lane shuffles) and quantize zeros.
    const bool real = b < nb;
    const size_t col = (size_t)(real? b : nb - 1) * PIX_QK8 + 4 * (lane & 7);
    const size_t first = (size_t)group * kQuantRows + wave;
    float4 v[kQuantPer];
    for (int i = 0; i < kQuantPer; i++) {  // all loads first, from clamped rows
        const size_t row = first + (size_t)kQuantWaves * i, r = row < rows? row : rows - 1;
        const float4 t = *reinterpret_cast<const float4*>(x + r * inner + col);
        v[i] = make_float4(real? t.x : 0.f,real? t.y : 0.f,real? t.z : 0.f,real? t.w : 0.f);
    }
    for (int i = 0; i < kQuantPer; i++) {
        const size_t row = first + (size_t)kQuantWaves * i;
        if (row >= rows) break;  // whole wave
        uint32_t packed;
        float d32;
        uint16_t dh;
        quantize_q8_0_group(v[i],packed,d32,dh);
        if (qs && b < nbp) {
            reinterpret_cast<uint32_t*>(qs + row * kpad + (size_t)b * PIX_QK8)[lane & 7] = packed;
            if ((lane & 7) == 0) dT[(size_t)b * mpad + row] = half_bits_to_float(dh);
        }
        if (blocks && real) {
            uint8_t* out = blocks + (row * nb + b) * PIX_Q8_0_BYTES;
            uint16_t* q16 = reinterpret_cast<uint16_t*>(out + 2 + 4 * (lane & 7));
            q16[0] = (uint16_t)(packed & 0xffffu);
            q16[1] = (uint16_t)(packed >> 16);
            if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(out) = dh;
        }
    }
}

hipError_t launch_quantize_q8_K(const float* x, size_t rows, size_t inner, Act8K planar, void* blocks, hipStream_t s)
{
    const size_t nb = inner / PIX_QK;
    if (!rows || !nb) return hipSuccess;
    const size_t grid = (rows + kQ8KRows - 1) / kQ8KRows * nb;
    if (grid >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    quantize_q8_K_kernel<<<dim3((unsigned)grid),dim3(64 * kQuantWaves),0,s>>>(x,rows,inner,planar.mpad,planar.qs,planar.d,planar.bs,
                                                                               static_cast<uint8_t*>(blocks));
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* x, size_t rows, size_t inner, size_t kpad, Act80 planar, void* blocks,
                                hipStream_t s)
{
    const size_t nch = (kpad / PIX_QK8 + 7) / 8;
    if (!rows || !nch || inner < PIX_QK8) return hipSuccess;
    const size_t grid = (rows + kQuantRows - 1) / kQuantRows * nch;
    if (grid >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    quantize_q8_0_kernel<<<dim3((unsigned)grid),dim3(64 * kQuantWaves),0,s>>>(x,rows,inner,kpad,planar.mpad,planar.qs,planar.d,
                                                                               static_cast<uint8_t*>(blocks));
    return hipGetLastError();
}

// Device-to-device copy in 16-byte words (grid-stride, one load and one store
// per word): the plain copy whose HBM byte counters calibrate the others.
__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t words)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) dst[i] = src[i];
}

hipError_t launch_copy_device(void* dst, const void* src, size_t bytes, hipStream_t s)
{
    if (!bytes) return hipSuccess;
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes) & 15)
        return hipMemcpyAsync(dst,src,bytes,hipMemcpyDeviceToDevice,s);
    const size_t words = bytes / 16;
    const size_t grid = std::min<size_t>((words + 255) / 256,(size_t)1 << 16);
    copy16_kernel<<<dim3((unsigned)grid),dim3(256),0,s>>>(static_cast<const uint4*>(src),static_cast<uint4*>(dst),words);
    return hipGetLastError();
}

}  // namespace pixhip
