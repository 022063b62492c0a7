// Convolution: tensor_conv (src/convolution.cpp:34-100) and vulkan_conv
// (src/backend_vulkan.cpp:1177-1209, :1359-1402) as an implicit GEMM on bf16
// MFMA (gfx950).
//
// The reference forms the im2col patches of every output pixel (inner index
// (c * kernel_y + ky) * kernel_x + kx, zero outside the image), multiplies them
// by the float weight [out][inner] in fp32 (cpu_gemm's FMA tiles, or the
// Vulkan matmul shader) and adds the bias.  Here the patches are never written
// out: a workgroup gathers its 128 pixels x 32 inner values straight from the
// image into LDS, with the inner dimension ordered (ky, kx, c) so that a stage
// of 32 is one kernel tap over 32 consecutive channels (one 128-byte run per
// pixel) whenever channels % 32 == 0 -- the weight is stored in that order
// when it is made resident.  Products run as attention's do: every fp32
// operand split into bf16 halves (hi = bf16(x), lo = bf16(x - hi)) and
// a*b = hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation, about 2^-16 relative per product (the weight halves are made
// once, at upload; F16 and BF16 weights are exact in them).
//
// Tile: 128 pixels x 128 output channels x 32 inner per stage, 4 waves of
// 64 x 64 (2 x 2 MFMA tiles).  The image kernel (images below 2 GiB) keeps one
// LDS stage of the split image (hi / lo planes, 80-byte rows) and a two-slot
// ring of the weight planes filled by L2 -> LDS transfers, with the image
// loads two stages ahead in registers; it is built for three waves per SIMD
// (at most 168 registers), so three workgroups share a CU.  Larger images and
// channel counts that are not a multiple of 32 take a simpler single-stage
// form (conv_body).

#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"


namespace pixhip {

namespace {

typedef __bf16 cbf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t cu32x4 __attribute__((ext_vector_type(4)));

constexpr int kCN = 128, kCK = 32;   // workgroup output channels, inner values per stage
constexpr int kCRow = 40;            // LDS row: 32 bf16 + 8 padding (80 B)

__device__ __forceinline__ uint32_t rne16(float x)
{
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// x -> (hi, lo) bf16 with x ~ hi + lo for every fp32 value (the weight form
// and the value-by-value gather): a finite x that rounds past the largest
// bf16 keeps hi truncated; Inf and NaN travel in hi alone (lo = 0).  The image
// kernel's hardware split (halves2) assumes finite values that round to a
// finite bf16, |x| < (2 - 2^-8) * 2^127 ~ 3.396e38: beyond that, and for Inf
// and NaN, its halves give NaN.
__device__ __forceinline__ void halves(float x, uint32_t& hi, uint32_t& lo)
{
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        hi = (u & 0x007FFFFFu)? 0x7FC0u | ((u >> 16) & 0x8000u) : u >> 16;
        lo = 0;
        return;
    }
    uint32_t h = rne16(x);
    if ((h & 0x7F80u) == 0x7F80u) h = u >> 16;
    hi = h;
    lo = rne16(x - __uint_as_float(h << 16));
}

typedef __bf16 cbf16x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t CRsrc;

// One 1 KB L2 -> LDS transfer (lane l's 16 bytes to lds_dst + 16 l), written
// as asm: issued through the builtin, the compiler makes every later LDS
// access wait for all transfers in flight (it cannot tell them apart), which
// would undo the ring.  The waits for these transfers are the explicit ones
// before the barriers; the compiler's own counts for the image loads only
// grow stronger from operations it does not see (the counter is in order).
// s_nop 0: one wait state between writing M0 and the transfer that reads it.
__device__ __forceinline__ void conv_dma(CRsrc r, const uint16_t* lds_dst, uint32_t voff, uint32_t soff)
{
    const uint32_t m = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds_dst;
    __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :: "s"(__builtin_amdgcn_readfirstlane(m)), "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff))
                     : "memory", "m0");
}

// s_waitcnt vmcnt(N) lgkmcnt(0), then s_barrier: the wave's own LDS reads
// and writes are done and all but its N newest vector-memory operations
// (loads and L2 -> LDS transfers, counted in issue order) have completed.
// (__syncthreads' workgroup fence must complete the wave's LDS writes, and
// with the compiler's L2 -> LDS transfers in flight that means every
// outstanding vector-memory operation.)
template <int N> __device__ __forceinline__ void conv_barrier()
{
    static_assert(N >= 0 && N < 16, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
}

// Raw buffer of `bytes` bytes (stride 0): loads at or past the end read zeros.
__device__ __forceinline__ CRsrc conv_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base),(short)0,(int)bytes,0x00020000);
}

// Two values rounded to bf16 (nearest even) by v_cvt_pk_bf16_f32; a in the
// low half.  For finite values the same bits as rne16.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b)
{
    const cbf16x2 h = {(__bf16)a,(__bf16)b};
    return __builtin_bit_cast(uint32_t,h);
}

// The split of a pair: hi = both values rounded to bf16, lo = the remainders
// rounded to bf16 (six vector instructions for two values).
__device__ __forceinline__ void halves2(float a, float b, uint32_t& hi, uint32_t& lo)
{
    hi = pack_bf16(a,b);
    lo = pack_bf16(a - __uint_as_float(hi << 16),b - __uint_as_float(hi & 0xFFFF0000u));
}

__device__ __forceinline__ float weight_value(const uint8_t* raw, uint32_t type, size_t index)
{
    if (type == PIX_F32) {
        const uint8_t* p = raw + 4 * index;
        return __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
    }
    const uint8_t* p = raw + 2 * index;
    const uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    return type == PIX_F16? half_bits_to_float(h) : __uint_as_float((uint32_t)h << 16);
}

}  // namespace

// Weight form: planes [npad][kp] of bf16 (hi, lo); row n, column k' = (ky *
// kernel_x + kx) * cin + c holds weight[n][(c * kernel_y + ky) * kernel_x + kx]
// of the GGUF / safetensors tensor; zero past cout and inner.
__global__ __launch_bounds__(256) void conv_form_kernel(const uint8_t* __restrict__ raw, uint32_t type, int kx_n, int ky_n, int cin,
                                                        int cout, int kp, int npad, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo)
{
    const size_t inner = (size_t)cin * kx_n * ky_n, total = (size_t)npad * kp, step = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const int n = (int)(e / kp), k = (int)(e % kp);
        float w = 0.0f;
        if (n < cout && (size_t)k < inner) {
            const int c = k % cin, tap = k / cin, kx = tap % kx_n, ky = tap / kx_n;
            w = weight_value(raw,type,(size_t)n * inner + ((size_t)c * ky_n + ky) * kx_n + kx);
        }
        uint32_t h, l;
        halves(w,h,l);
        hi[e] = (uint16_t)h;
        lo[e] = (uint16_t)l;
    }
}

hipError_t launch_conv_form(const void* raw, uint32_t type, int kernel_x, int kernel_y, int cin, int cout, int kp, int npad,
                            uint16_t* hi, uint16_t* lo, hipStream_t s)
{
    const size_t total = (size_t)npad * kp;
    const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256,(size_t)1 << 20);
    conv_form_kernel<<<dim3(grid),dim3(256),0,s>>>(static_cast<const uint8_t*>(raw),type,kernel_x,kernel_y,cin,cout,kp,npad,hi,lo);
    return hipGetLastError();
}

// MODE 1: cin % 32 == 0 and the image 16-byte aligned (a stage is one tap of
// 32 consecutive channels, read as float4) at 64-bit addresses, for images of
// 2 GiB and more; MODE 0: each inner value is gathered on its own (the first
// layer's 3 or 16 channels).  The next stage's loads are held in registers
// while the current one is multiplied.  Each wave owns MT = 2 tiles of 32
// pixels by 2 of 32 channels (a 256-pixel workgroup tile with 128 x 64 per
// wave ran 27% slower).
template <int MODE>
__device__ __forceinline__ void conv_body(const ConvArgs& a)
{
    constexpr bool FAST = MODE != 0;
    constexpr int MT = 2;
    constexpr int BM = 64 * MT;                        // workgroup pixels
    constexpr int PA = BM * kCRow, PB = kCN * kCRow;   // bf16 per A / B plane
    constexpr int STAGE = 2 * PA + 2 * PB;
    constexpr int AV = FAST? BM * 8 / 256 : BM * 32 / 256;  // A values (float4 or scalar) per thread
    __shared__ __attribute__((aligned(16))) uint16_t lds[STAGE];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, lr = lane & 31, hh = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const long long m0 = (long long)blockIdx.x * BM;
    const int n0 = blockIdx.y * kCN;

    // the pixels this thread loads: rows t/8 + 32i (FAST), rows t/32 + 8i (gather)
    int iy0[AV], ix0[AV];
#pragma unroll
    for (int i = 0; i < AV; i++) {
        const long long m = m0 + (FAST? t / 8 + 32 * i : t / 32 + 8 * i);
        if (m < a.M) {
            const int oy = (int)(m / a.OW), ox = (int)(m % a.OW);
            iy0[i] = oy * a.SY - a.PT;
            ix0[i] = ox * a.SX - a.PL;
        } else {
            iy0[i] = -(1 << 30);  // never inside the image
            ix0[i] = 0;
        }
    }

    float4 ra[FAST? AV : 1];
    bool ain[FAST? AV : 1];
    float rs[FAST? 1 : AV];
    cu32x4 rb[4];
    auto fetch = [&](int stage) {
        const int k0 = stage * kCK;
        if constexpr (FAST) {
            const int tap = k0 / a.C, c = k0 % a.C + (t % 8) * 4;
            const int ky = tap / a.KX, kx = tap % a.KX;
            // every lane loads: a tap outside the image reads pixel 0 and
            // store() puts zeros in its place, so no load sits behind a branch
#pragma unroll
            for (int i = 0; i < AV; i++) {
                const int iy = iy0[i] + ky, ix = ix0[i] + kx;
                ain[i] = iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const unsigned pix = ain[i]? (unsigned)iy * (unsigned)a.W + (unsigned)ix : 0u;  // < 2^32 pixels
                ra[i] = *reinterpret_cast<const float4*>(a.x + (size_t)pix * a.C + c);
            }
        } else {
            const int k = k0 + t % 32;
            const int c = k % a.C, tap = k / a.C, ky = tap / a.KX, kx = tap % a.KX;
#pragma unroll
            for (int i = 0; i < AV; i++) {
                const int iy = iy0[i] + ky, ix = ix0[i] + kx;
                rs[i] = (k < a.K && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W) ? a.x[((size_t)iy * a.W + ix) * a.C + c] : 0.0f;
            }
        }
        // B: 128 rows x 64 bytes per plane, two 16-byte pieces per thread per plane
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int q = t + 256 * (j & 1), row = q / 4, part = q % 4;
            const uint16_t* plane = (j < 2)? a.wh : a.wl;
            rb[j] = *reinterpret_cast<const cu32x4*>(plane + (size_t)(n0 + row) * a.Kp + k0 + part * 8);
        }
    };
    auto store = [&]() {
        uint16_t* st = lds;
        if constexpr (FAST) {
#pragma unroll
            for (int i = 0; i < AV; i++) {
                const int row = t / 8 + 32 * i, col = (t % 8) * 4;
                const float4 v = ain[i]? ra[i] : make_float4(0.0f,0.0f,0.0f,0.0f);
                uint32_t h01, l01, h23, l23;
                halves2(v.x,v.y,h01,l01);
                halves2(v.z,v.w,h23,l23);
                *reinterpret_cast<uint2*>(st + row * kCRow + col) = make_uint2(h01,h23);
                *reinterpret_cast<uint2*>(st + PA + row * kCRow + col) = make_uint2(l01,l23);
            }
        } else {
#pragma unroll
            for (int i = 0; i < AV; i++) {
                const int row = t / 32 + 8 * i, col = t % 32;
                uint32_t h, l;
                halves(rs[i],h,l);
                st[row * kCRow + col] = (uint16_t)h;
                st[PA + row * kCRow + col] = (uint16_t)l;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int q = t + 256 * (j & 1), row = q / 4, part = q % 4;
            *reinterpret_cast<cu32x4*>(st + 2 * PA + (j >> 1) * PB + row * kCRow + part * 8) = rb[j];
        }
    };

    v16f acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v16f{};

    const int stages = a.Kp / kCK;
    fetch(0);
    store();
    __syncthreads();
    for (int s = 0; s < stages; s++) {
        if (s + 1 < stages) fetch(s + 1);
        const uint16_t* st = lds;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int col = ks * 16 + 8 * hh;
            cbf16x8 ah[MT], al[MT], bh[2], bl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int row = wn * 64 + j * 32 + lr;
                bh[j] = *reinterpret_cast<const cbf16x8*>(st + 2 * PA + row * kCRow + col);
                bl[j] = *reinterpret_cast<const cbf16x8*>(st + 2 * PA + PB + row * kCRow + col);
            }
#pragma unroll
            for (int i = 0; i < MT; i++) {
                const int row = wm * (BM / 2) + i * 32 + lr;
                ah[i] = *reinterpret_cast<const cbf16x8*>(st + row * kCRow + col);
                al[i] = *reinterpret_cast<const cbf16x8*>(st + PA + row * kCRow + col);
            }
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i],bh[j],acc[i][j],0,0,0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i],bl[j],acc[i][j],0,0,0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i],bh[j],acc[i][j],0,0,0);
                }
        }
        if (s + 1 < stages) {
            __syncthreads();  // every wave is done reading the stage
            store();
            __syncthreads();
        }
    }

    // acc[i][j] lane: output channel n0 + wn*64 + 32j + lr, pixels
    // m0 + wm*BM/2 + 32i + 8(r/4) + 4hh + r%4
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + wn * 64 + 32 * j + lr;
        if (n >= a.N) continue;
        const float b = a.bias? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const long long m = m0 + wm * (BM / 2) + 32 * i + 8 * (r / 4) + 4 * hh + r % 4;
                if (m < a.M) a.y[(size_t)m * a.N + n] = a.bias? __fadd_rn(acc[i][j][r],b) : acc[i][j][r];
            }
    }
}


// The image kernel for images below 2 GiB, pipelined deeper than conv_body:
// the weight planes go L2 -> LDS by buffer_load ... lds into a two-slot ring
// (64-byte rows, piece c of row r at c ^ ((r >> 2) & 3), no registers), and
// the image loads run two stages ahead in two register sets, so a stage's
// stores to LDS wait on loads issued a whole stage earlier.  LDS: one A stage
// (hi, lo: 20 KB) + two B slots (hi, lo: 16 KB each) = 52 KB, three
// workgroups per CU.
__device__ __forceinline__ void conv_body_ring(const ConvArgs& a)
{
    constexpr int BM = 128, AV = 4;
    constexpr int PA = BM * kCRow;   // bf16 per A plane (80-byte rows)
    constexpr int PB = kCN * 32;     // bf16 per B plane (64-byte rows)
    // (separate arrays: the compiler can then tell the image stores from the
    // transfers in flight into the ring)
    __shared__ __attribute__((aligned(1024))) uint16_t lds[2 * PA];
    __shared__ __attribute__((aligned(1024))) uint16_t bslot0[2 * PB];  // ring slots: planes hi, lo
    __shared__ __attribute__((aligned(1024))) uint16_t bslot1[2 * PB];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), lr = lane & 31, hh = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const long long m0 = (long long)blockIdx.x * BM;
    const int n0 = blockIdx.y * kCN;

    int iy0[AV], ix0[AV];
#pragma unroll
    for (int i = 0; i < AV; i++) {
        const long long m = m0 + t / 8 + 32 * i;
        if (m < a.M) {
            const int oy = (int)(m / a.OW), ox = (int)(m % a.OW);
            iy0[i] = oy * a.SY - a.PT;
            ix0[i] = ox * a.SX - a.PL;
        } else {
            iy0[i] = -(1 << 30);
            ix0[i] = 0;
        }
    }
    const uint32_t wbytes = (uint32_t)((size_t)a.Npad * a.Kp * 2);
    const CRsrc rx = conv_rsrc(a.x,(uint32_t)((size_t)a.W * a.H * a.C * 4));
    const CRsrc rwh = conv_rsrc(a.wh,wbytes), rwl = conv_rsrc(a.wl,wbytes);
    // B DMA: the stage's 16 chunks of 1 KB (plane c / 8, rows 16 (c % 8) ..
    // +15), chunk c = wave + 4i; lane l lands at row l / 4, physical piece l % 4
    uint32_t bvo[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = wave + 4 * i, row = 16 * (c % 8) + lane / 4, logical = (lane % 4) ^ ((row >> 2) & 3);
        bvo[i] = ((uint32_t)(n0 + row) * (uint32_t)a.Kp + 8u * (uint32_t)logical) * 2u;
    }
    auto issue_b = [&](int stage, int slot) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = wave + 4 * i;
            uint16_t* dst = (slot? bslot1 : bslot0) + (c / 8) * PB + (c % 8) * 512;
            conv_dma(c < 8? rwh : rwl,dst,bvo[i],(uint32_t)(stage * kCK * 2));
        }
    };
    constexpr uint32_t kOut = 0x80000000u;
    uint32_t aoff[AV];
    int cur_tap = -1;
    auto fetch_a = [&](int stage, float4 (&ra)[AV]) {
        const int k0 = stage * kCK, tap = k0 / a.C;
        if (tap != cur_tap) {
            cur_tap = tap;
            const int ky = tap / a.KX, kx = tap % a.KX;
#pragma unroll
            for (int i = 0; i < AV; i++) {
                const int iy = iy0[i] + ky, ix = ix0[i] + kx;
                const bool in = iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                const uint32_t pix = (uint32_t)iy * (uint32_t)a.W + (uint32_t)ix;
                aoff[i] = in? (pix * (uint32_t)a.C + (uint32_t)(t % 8) * 4u) * 4u : kOut;
            }
        }
        const uint32_t cb = (uint32_t)(k0 % a.C) * 4u;
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const cu32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx,aoff[i] + cb,0,0);
            ra[i] = make_float4(__uint_as_float(v.x),__uint_as_float(v.y),__uint_as_float(v.z),__uint_as_float(v.w));
        }
    };
    auto store_a = [&](const float4 (&ra)[AV]) {
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const int row = t / 8 + 32 * i, col = (t % 8) * 4;
            uint32_t h01, l01, h23, l23;
            halves2(ra[i].x,ra[i].y,h01,l01);
            halves2(ra[i].z,ra[i].w,h23,l23);
            *reinterpret_cast<uint2*>(lds + row * kCRow + col) = make_uint2(h01,h23);
            *reinterpret_cast<uint2*>(lds + PA + row * kCRow + col) = make_uint2(l01,l23);
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v16f{};
    auto multiply = [&](int slot) {
        const uint16_t* bs = slot? bslot1 : bslot0;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int col = ks * 16 + 8 * hh;
            cbf16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int row = wn * 64 + j * 32 + lr;
                const int at = row * 32 + (((2 * ks + hh) ^ ((row >> 2) & 3)) << 3);
                bh[j] = *reinterpret_cast<const cbf16x8*>(bs + at);
                bl[j] = *reinterpret_cast<const cbf16x8*>(bs + PB + at);
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int row = wm * 64 + i * 32 + lr;
                ah[i] = *reinterpret_cast<const cbf16x8*>(lds + row * kCRow + col);
                al[i] = *reinterpret_cast<const cbf16x8*>(lds + PA + row * kCRow + col);
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i],bh[j],acc[i][j],0,0,0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i],bl[j],acc[i][j],0,0,0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i],bh[j],acc[i][j],0,0,0);
                }
        }
    };

    // Before stage s: A of s in LDS, B of s in slot s % 2, the loads of A of
    // s + 1 in flight in register set (s + 1) % 2.  Stage s issues B of s + 1
    // (the other slot, read last in stage s - 1) and A of s + 2 (set s % 2,
    // stored in stage s - 1), multiplies, and after a barrier waits for all
    // but the four newest loads (A of s + 2), so B of s + 1 and A of s + 1
    // have landed, and stores A of s + 1.
    const int stages = a.Kp / kCK;
    float4 ra0[AV], ra1[AV];
    fetch_a(0,ra0);
    issue_b(0,0);
    // The image loads are issued unconditionally (past the last stage they
    // read offsets of a further tap, in range or read as zeros, and are never
    // stored), so every stage has the same four loads newest in the counter.
    fetch_a(1,ra1);
    store_a(ra0);
    conv_barrier<4>();  // B of 0 landed (A of 1 may be in flight)
    auto step = [&](int s, float4 (&mine)[AV], float4 (&next)[AV], int slot, bool more) {
        if (more) issue_b(s + 1,slot ^ 1);
        fetch_a(s + 2,mine);
        multiply(slot);
        if (more) {
            conv_barrier<15>();  // every wave is done reading A of s and B slot s % 2
            store_a(next);       // (the compiler waits for the loads of `next`)
            conv_barrier<4>();   // B of s + 1 landed; A of s + 2 may be in flight
        }
    };
    // Whole pairs in the loop (every step has a next stage, so the loop body
    // has no path that leaves a register set's loads unwaited), then the
    // last one or two stages.
    int s = 0;
    for (; s + 2 < stages; s += 2) {
        step(s,ra0,ra1,0,true);
        step(s + 1,ra1,ra0,1,true);
    }
    step(s,ra0,ra1,0,s + 1 < stages);
    if (s + 1 < stages) step(s + 1,ra1,ra0,1,false);

#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + wn * 64 + 32 * j + lr;
        if (n >= a.N) continue;
        const float b = a.bias? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const long long m = m0 + wm * 64 + 32 * i + 8 * (r / 4) + 4 * hh + r % 4;
                if (m < a.M) a.y[(size_t)m * a.N + n] = a.bias? __fadd_rn(acc[i][j][r],b) : acc[i][j][r];
            }
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3,3))) void conv_image_kernel(ConvArgs a)
{
    conv_body_ring(a);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3,3))) void conv_image_wide_kernel(ConvArgs a)
{
    conv_body<1>(a);
}

__global__ __launch_bounds__(256) void conv_gather_kernel(ConvArgs a)
{
    conv_body<0>(a);
}

hipError_t launch_conv(const ConvArgs& a, hipStream_t s)
{
    if (!a.M || !a.N) return hipSuccess;
    const long long mt = (a.M + 127) / 128;
    if (mt > 0x7fffffffLL || a.Npad / kCN > 65535) return hipErrorInvalidValue;
    const dim3 grid((unsigned)mt,(unsigned)(a.Npad / kCN));
    const bool narrow = (size_t)a.W * a.H * a.C * 4 < ((size_t)1 << 31) && (size_t)a.Npad * a.Kp * 2 < ((size_t)1 << 31);
    if (a.C % kCK == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0) {
        if (narrow) conv_image_kernel<<<grid,dim3(256),0,s>>>(a);
        else conv_image_wide_kernel<<<grid,dim3(256),0,s>>>(a);
    } else
        conv_gather_kernel<<<grid,dim3(256),0,s>>>(a);
    return hipGetLastError();
}

}  // namespace pixhip
