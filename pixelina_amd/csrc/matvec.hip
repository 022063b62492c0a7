// M=1 quantized matrix-vector product (decode step): y[n] = W[n][:] . x.
// The counterpart of shaders/matvec.comp:18-50 (chosen by VulkanState::multiply
// when M == 1, src/backend_vulkan.cpp:979) with the numerics of
// cpu_quant_matmul at columns == 1 (src/kernels_quant.cpp:369-412): x is first
// quantized exactly as quantize_row_q8_K_ref / quantize_row_q8_0_ref, then each
// row takes integer block dots and an fp32 epilogue.
//
// HBM-bound: every weight byte is read once with 128-bit loads; no MFMA.
// Each workgroup re-quantizes x into LDS (K <= 24576 values: 24 KB), then every
// wave streams whole rows: lane u owns one "unit" of 64 values of a row
// (Q5_K: a quarter super-block = two 32-value sub-blocks; Q8_0: two blocks;
// Q6_K: 16 positions x 4 groups of a half super-block) and the row total is a
// wave reduction.  Row pairs are dealt round-robin over every wave of the
// grid (wave g takes pairs g, g + W, g + 2W, ...), so at any moment the waves
// of the whole device read one contiguous band of the matrix: DRAM sees a
// front-to-back stream, as a plain copy does.
//
// The loads are kept free of branches (row and unit indices are clamped into
// the matrix; the surplus lanes' values are ignored) and no store is issued
// while weight loads are in flight: loads and stores share the vector memory
// counter, and a wait for the current rows would otherwise have to drain the
// next rows' loads as well.  Each wave keeps two register sets of rows and
// alternates between them, so one set is computed while the other streams in.
#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

// A 16-byte load marked non-temporal: each weight byte is read once, so its
// lines need not stay in the caches.  Only for loads whose 64 lanes cover
// consecutive 16-byte pieces (the Q5_K planes: measured 10.17 -> 9.6 us at
// 18944 x 3584); where lanes read 64-byte runs in four loads (the Q8_0 rows)
// the later loads re-use the lines the first one fetched, and marking them
// non-temporal made that kernel 1.7x slower.
typedef unsigned int u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint4* p)
{
    const u4v t = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(p));
    return make_uint4(t.x,t.y,t.z,t.w);
}
// The same for the 12-byte unit records of the Q5_K form (lanes read
// consecutive 12-byte pieces: 10.0 -> 9.65 us at 18944 x 3584).
typedef unsigned int u3v __attribute__((ext_vector_type(3)));
__device__ __forceinline__ uint3 load_stream(const uint3* p)
{
    const u3v t = __builtin_nontemporal_load(reinterpret_cast<const u3v*>(p));
    return make_uint3(t.x,t.y,t.z);
}


constexpr int kMvWaves = 8;
constexpr int kMvRows = 2;  // rows per register set (the longest Q8_0 and Q6_K rows use 1)
// x staging passes per wave per 64 units of a row: a row of 64*UPL units has
// at most 16*UPL Q8_K blocks (or 16*UPL passes of 8 Q8_0 blocks).
constexpr int kXPasses = 16 / kMvWaves;
// Workgroups per CU.  One (8 waves, each with two sets of two rows in flight)
// streams fastest: measured against 2 or 3 smaller workgroups, 16 waves per
// CU, and one set per wave.
constexpr int kMvMaxWgPerCu = 1;
// s_waitcnt vmcnt(n) with the export and LDS/scalar counters left alone
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
constexpr int wait_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0f70; }
constexpr int kWaitVmcnt0 = wait_vmcnt(0);

// The wave's index in the workgroup, as a wave-uniform (scalar) value: the row
// loops then branch on scalars and never run with part of the wave masked off.
__device__ __forceinline__ int wave_id()
{
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// x staging is split in two so that its global loads go out first (before
// the first weight rows are requested) and its quantization runs while the
// weight loads are in flight.  Each wave takes blocks wave, wave+8, ...; P
// bounds the blocks per wave (Q8_K) or 8-block passes per wave (Q8_0).  The
// loads past the last block re-read the last block (no branch around them).

// Q8_K: one wave per 256-value block, a float4 per lane.
template <int P>
__device__ __forceinline__ void load_x_q8_K(const float* __restrict__ x, int K, float4 (&v)[P])
{
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nb = K / PIX_QK;
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int b = min(wave + kMvWaves * i,nb - 1);
        v[i] = reinterpret_cast<const float4*>(x + b * PIX_QK)[lane];
    }
}

template <int P>
__device__ __forceinline__ void quantize_x_q8_K(const float4 (&v)[P], int K, int8_t* sQ, float* sD, int* sB)
{
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nb = K / PIX_QK;
    // Every pass runs (a pass past the last block quantizes the re-read last
    // block and stores nothing), so that x's loads are used on every path and
    // stay ahead of the weight loads.
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int b = wave + kMvWaves * i;
        uint32_t packed;
        float d;
        int gsum;
        quantize_q8_K_wave(v[i],lane,packed,d,gsum);
        if (b < nb) {
            reinterpret_cast<uint32_t*>(sQ + b * PIX_QK)[lane] = packed;
            if (lane == 0) sD[b] = d;
            if ((lane & 3) == 0) sB[b * 16 + (lane >> 2)] = gsum;
        }
    }
}

// Q8_0 over Kp = K rounded up to 64 (the padding block is zero): an 8-lane
// group per 32-value block, 8 blocks per wave per pass.
template <int P>
__device__ __forceinline__ void load_x_q8_0(const float* __restrict__ x, int K, float4 (&v)[P])
{
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nb = K / PIX_QK8;
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int b = min((wave + kMvWaves * i) * 8 + (lane >> 3),nb - 1);
        v[i] = reinterpret_cast<const float4*>(x + b * PIX_QK8)[lane & 7];
    }
}

template <int P>
__device__ __forceinline__ void quantize_x_q8_0(const float4 (&v)[P], int K, int Kp, int8_t* sQ, float* sD)
{
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nb = K / PIX_QK8;
    if (Kp > K) {
        for (int i = threadIdx.x; i < Kp - K; i += blockDim.x) sQ[K + i] = 0;
        if (threadIdx.x == 0) sD[nb] = 0.0f;
    }
    // Every pass runs, as in quantize_x_q8_K.
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int b = (wave + kMvWaves * i) * 8 + (lane >> 3);
        uint32_t packed;
        float d32;
        uint16_t dh;
        quantize_q8_0_group(b < nb? v[i] : make_float4(0.0f,0.0f,0.0f,0.0f),packed,d32,dh);
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

// Row totals of one wave, parked one per lane: lane j holds row
// base + (j / R) * stride + j % R (R rows per set).  They are written when no
// lanes are left for another row group (a wave with more than 64 / R of them)
// and at the end.
struct RowResults {
    float v;
    int slot, base;
};

template <int R>
__device__ __forceinline__ void results_flush(RowResults& r, int lane, int stride, int last, const Output& out)
{
    if (lane < r.slot) {
        const int row = r.base + (lane / R) * stride + lane % R;
        if (row < last) store_row(out,(size_t)row,r.v);
    }
    r.base += (64 / R) * stride;
    r.slot = 0;
}

template <int R>
__device__ __forceinline__ void results_put(RowResults& r, const float (&part)[R], int lane, int stride, int last,
                                            const Output& out)
{
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const float t = wave_sum(part[rr]);
        r.v = lane == r.slot + rr? t : r.v;
    }
    r.slot += R;
    if (r.slot > 64 - R) {
        results_flush<R>(r,lane,stride,last,out);
        // Drain the stores here, so that no store is outstanding when the
        // caller next waits for row loads.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    }
}

// The row loop of every matvec kernel.  `load(rows, r0)` requests the rows
// r0 .. r0 + Rows::R - 1 (clamped to the matrix) into one register set,
// `dot(rows, part)` computes their partial sums; set a holds the rows of
// `first` on entry.  With TWO_SETS the next rows stream into set b while set
// a is computed; without (long rows, whose two sets would not fit in the
// registers) a wave computes a set before requesting the next.
template <bool TWO_SETS, class Rows, class Load, class Dot>
__device__ __forceinline__ void stream_rows(Rows& a, Rows& b, int first, int stride, int last, int lane, const Output& out,
                                            Load load, Dot dot)
{
    // The loops have no exit in their middle: the compiler's wait analysis
    // would otherwise see the exit path's loads still pending at the loop head.
    constexpr int R = Rows::R;
    RowResults res{0.0f,0,first};
    float part[R];
    int r0 = first;
    if constexpr (TWO_SETS) {
        for (; r0 + stride < last; r0 += 2 * stride) {
            load(b,r0 + stride);
            dot(a,part);
            results_put<R>(res,part,lane,stride,last,out);
            load(a,r0 + 2 * stride);
            dot(b,part);
            results_put<R>(res,part,lane,stride,last,out);
        }
    } else {
        (void)b;
        for (; r0 + stride < last; r0 += stride) {
            dot(a,part);
            results_put<R>(res,part,lane,stride,last,out);
            load(a,r0 + stride);
        }
    }
    if (r0 < last) {  // set a holds rows r0.. (requested by the last pass)
        dot(a,part);
        results_put<R>(res,part,lane,stride,last,out);
    }
    results_flush<R>(res,lane,stride,last,out);
}

// Rows per register set: two up to 16384 values per row, one beyond.  Long
// rows are few at decode shapes (an FFN down projection has K = 18944 and
// N = 3584), and one row per set spreads them over twice as many waves:
// measured 9% faster for Q5_K and 2% for Q8_0 than two rows per set, and
// faster than two sets of one row.
template <int UPL> constexpr int mv_rows() { return UPL <= 4? kMvRows : 1; }

// ---------------------------------------------------------------- Q5_K (planar)
// Weight registers of R rows: unit u = lane + 64k of a row covers two
// 32-value sub-blocks (2j, 2j+1 of super-block u/4): its 32 nibble bytes (from
// the row's two half planes) and its 12-byte record (high bits, six-bit scales
// and minima, and one byte of the super-block's d and dmin; the four units of
// a super-block sit in one lane quad, which gathers the four bytes with DPP).
// A row streams its GGUF byte count.
template <int UPL, int ROWS> struct Q5Rows {
    static constexpr int R = ROWS;
    uint4 qs0[R][UPL], qs1[R][UPL];
    uint3 rec[R][UPL];
};

// The 32-bit word made of byte 3 of v in lanes 0..3 of the caller's quad.
__device__ __forceinline__ uint32_t quad_gather_top_bytes(uint32_t v)
{
    const uint32_t b0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v,0x00,0xf,0xf,false);
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v,0x55,0xf,0xf,false);
    const uint32_t b2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v,0xaa,0xf,0xf,false);
    const uint32_t b3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v,0xff,0xf,0xf,false);
    return (b0 >> 24) | ((b1 >> 16) & 0xff00u) | ((b2 >> 8) & 0xff0000u) | (b3 & 0xff000000u);
}

template <int UPL, int R>
__device__ __forceinline__ void q5_load(Q5Rows<UPL,R>& f, const PlanarQ5K& w, int K, int r0, int last, int lane, int units)
{
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int row = min(r0 + rr,last - 1);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = min(lane + 64 * k,units - 1);
            const uint4* q = reinterpret_cast<const uint4*>(w.qs + (size_t)row * (K / 2));
            f.qs0[rr][k] = load_stream(q + u);
            f.qs1[rr][k] = load_stream(q + units + u);
            f.rec[rr][k] = load_stream(reinterpret_cast<const uint3*>(w.rec + ((size_t)row * units + u) * 3));
        }
    }
}

template <int UPL, int R>
__device__ __forceinline__ void q5_compute(const Q5Rows<UPL,R>& f, float part[R], const int8_t* sQ, const float* sD,
                                           const int* sB, int lane, int units)
{
#pragma unroll
    for (int rr = 0; rr < R; rr++) part[rr] = 0.0f;
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
        for (int rr = 0; rr < R; rr++) {
            const uint3 m = f.rec[rr][k];
            const uint32_t dd = quad_gather_top_bytes(m.z);
            const uint32_t qsw[8] = {f.qs0[rr][k].x,f.qs0[rr][k].y,f.qs0[rr][k].z,f.qs0[rr][k].w,
                                     f.qs1[rr][k].x,f.qs1[rr][k].y,f.qs1[rr][k].z,f.qs1[rr][k].w};
            int dot0 = 0, dot1 = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t t = (q < 4? m.x : m.y) >> (2 * (q & 3));
                const uint32_t lo = (qsw[q] & 0x0f0f0f0fu) | ((t & 0x01010101u) << 4);
                const uint32_t hi = ((qsw[q] >> 4) & 0x0f0f0f0fu) | (((t >> 1) & 0x01010101u) << 4);
                dot0 = sdot4(lo,xa[q],dot0);
                dot1 = sdot4(hi,xb[q],dot1);
            }
            const int sc0 = (int)(m.z & 63u), sc1 = (int)((m.z >> 6) & 63u);
            const int mn0 = (int)((m.z >> 12) & 63u), mn1 = (int)((m.z >> 18) & 63u);
            const int S = sc0 * dot0 + sc1 * dot1;
            const int Mn = mn0 * bs0 + mn1 * bs1;
            const float wd = half_bits_to_float((uint16_t)(dd & 0xffffu));
            const float wm = half_bits_to_float((uint16_t)(dd >> 16));
            part[rr] = __builtin_fmaf(yd,__builtin_fmaf(-wm,(float)Mn,wd * (float)S),part[rr]);
        }
    }
}

template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q5_K_kernel(PlanarQ5K w, const float* __restrict__ x,
                                                                    int N, int K, Output out)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / PIX_QK;
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + K);
    int* sB = reinterpret_cast<int*>(smem + K + 4 * nb);
    const int lane = threadIdx.x & 63, wave = wave_id();
    constexpr int R = mv_rows<UPL>();
    const int stride = (int)gridDim.x * kMvWaves * R;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * R;
    const int last = N;
    const int units = nb * 4;
    // The first rows' weights are requested before x is staged, so their
    // latency overlaps the quantization of x.
    float4 xv[kXPasses * UPL];
    load_x_q8_K(x,K,xv);
    __builtin_amdgcn_sched_barrier(0);
    // Long rows (one register set): x is quantized before the first rows are
    // requested, so that its staging registers are free again.
    constexpr bool two_sets = UPL <= 4;
    Q5Rows<UPL,R> a, b;
    if (two_sets) q5_load(a,w,K,first,last,lane,units);
    __builtin_amdgcn_sched_barrier(0);
    quantize_x_q8_K(xv,K,sQ,sD,sB);
    // x's loads were issued before the rows' 3 * R * UPL: this wait marks
    // them complete on every path.
    __builtin_amdgcn_s_waitcnt(wait_vmcnt(two_sets? 3 * R * UPL : 0));
    if (!two_sets) q5_load(a,w,K,first,last,lane,units);
    __syncthreads();
    stream_rows<two_sets>(a,b,first,stride,last,lane,out,
                [&](Q5Rows<UPL,R>& f, int r0) { q5_load(f,w,K,r0,last,lane,units); },
                [&](const Q5Rows<UPL,R>& f, float (&part)[R]) { q5_compute(f,part,sQ,sD,sB,lane,units); });
}

// ---------------------------------------------------------------- Q8_0 (planar)
// Unit u of a row: 64 values (two blocks) of the planar quants and their two
// fp16 scales.
template <int UPL, int ROWS> struct Q80Rows {
    static constexpr int R = ROWS;
    uint4 q[R][UPL][4];
    uint32_t dd[R][UPL];
};

template <int UPL, int R>
__device__ __forceinline__ void q80_load(Q80Rows<UPL,R>& f, const PlanarQ80& w, int Kp, int r0, int last, int lane, int units)
{
    const int nbp = Kp / PIX_QK8;
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int row = min(r0 + rr,last - 1);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = min(lane + 64 * k,units - 1);
            // piece t of unit u at (t*units + u)*16: each load is lane-contiguous
            const uint4* p = reinterpret_cast<const uint4*>(w.qs_mv + (size_t)row * Kp);
#pragma unroll
            for (int t = 0; t < 4; t++) f.q[rr][k][t] = load_stream(p + t * units + u);
            f.dd[rr][k] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(w.d + (size_t)row * nbp + 2 * u));
        }
    }
}

template <int UPL, int R>
__device__ __forceinline__ void q80_compute(const Q80Rows<UPL,R>& f, float part[R], const int8_t* sQ, const float* sD, int lane,
                                            int units)
{
#pragma unroll
    for (int rr = 0; rr < R; rr++) part[rr] = 0.0f;
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
        for (int rr = 0; rr < R; rr++) {
            const uint32_t wa[8] = {f.q[rr][k][0].x,f.q[rr][k][0].y,f.q[rr][k][0].z,f.q[rr][k][0].w,
                                    f.q[rr][k][1].x,f.q[rr][k][1].y,f.q[rr][k][1].z,f.q[rr][k][1].w};
            const uint32_t wb[8] = {f.q[rr][k][2].x,f.q[rr][k][2].y,f.q[rr][k][2].z,f.q[rr][k][2].w,
                                    f.q[rr][k][3].x,f.q[rr][k][3].y,f.q[rr][k][3].z,f.q[rr][k][3].w};
            int p0 = 0, p1 = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                p0 = sdot4(wa[t],xa[t],p0);
                p1 = sdot4(wb[t],xb[t],p1);
            }
            const float wd0 = half_bits_to_float((uint16_t)(f.dd[rr][k] & 0xffffu));
            const float wd1 = half_bits_to_float((uint16_t)(f.dd[rr][k] >> 16));
            part[rr] = __builtin_fmaf(wd0 * xd0,(float)p0,part[rr]);
            part[rr] = __builtin_fmaf(wd1 * xd1,(float)p1,part[rr]);
        }
    }
}

template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q8_0_kernel(PlanarQ80 w, const float* __restrict__ x, int N, int K,
                                                                    int Kp, Output out)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + Kp);
    const int lane = threadIdx.x & 63, wave = wave_id();
    constexpr int R = mv_rows<UPL>();
    const int stride = (int)gridDim.x * kMvWaves * R;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * R;
    const int last = N;
    const int units = Kp / 64;
    float4 xv[kXPasses * UPL];
    load_x_q8_0(x,K,xv);
    __builtin_amdgcn_sched_barrier(0);
    // Set a is requested before x is quantized unless the rows are long (see
    // the Q5_K kernel); two sets up to 3 units per lane.
    constexpr bool two_sets = UPL <= 3, rows_first = UPL <= 4;
    Q80Rows<UPL,R> a, b;
    if (rows_first) q80_load(a,w,Kp,first,last,lane,units);
    __builtin_amdgcn_sched_barrier(0);
    quantize_x_q8_0(xv,K,Kp,sQ,sD);
    // x's loads precede the rows' 5 * R * UPL (see the Q5_K kernel).
    __builtin_amdgcn_s_waitcnt(wait_vmcnt(rows_first? 5 * R * UPL : 0));
    if (!rows_first) q80_load(a,w,Kp,first,last,lane,units);
    __syncthreads();
    stream_rows<two_sets>(a,b,first,stride,last,lane,out,
                [&](Q80Rows<UPL,R>& f, int r0) { q80_load(f,w,Kp,r0,last,lane,units); },
                [&](const Q80Rows<UPL,R>& f, float (&part)[R]) { q80_compute(f,part,sQ,sD,lane,units); });
}

// ---------------------------------------------------------------- Q6_K (planar)
// Unit u of a row: super-block b = u/4, half h = (u/2)%2, position half ih = u%2;
// it covers elements 128h + 32g + 16ih + i for g = 0..3, i = 0..15.
template <int UPL, int ROWS> struct Q6Rows {
    static constexpr int R = ROWS;
    uint4 la[R][UPL], lb[R][UPL], hh[R][UPL];
    uint2 scw[R][UPL];
    uint16_t dh[R][UPL];
};

template <int UPL, int R>
__device__ __forceinline__ void q6_load(Q6Rows<UPL,R>& f, const PlanarQ6K& w, int K, int r0, int last, int lane, int units)
{
    const int nb = K / PIX_QK;
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int row = min(r0 + rr,last - 1);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = min(lane + 64 * k,units - 1);
            const int b = u >> 2, h = (u >> 1) & 1, ih = u & 1;
            // ql as two unit-major planes of 16-byte pieces; qh is unit-major as
            // stored (b*64 + 32h + 16ih = 16u): every load is lane-contiguous
            const uint4* ql = reinterpret_cast<const uint4*>(w.ql + (size_t)row * (K / 2));
            f.la[rr][k] = load_stream(ql + u);
            f.lb[rr][k] = load_stream(ql + units + u);
            f.hh[rr][k] = load_stream(reinterpret_cast<const uint4*>(w.qh + (size_t)row * (K / 4)) + u);
            f.scw[rr][k] = *reinterpret_cast<const uint2*>(w.sc + (size_t)row * (K / 16) + b * 16 + 8 * h);
            f.dh[rr][k] = __builtin_bit_cast(uint16_t,w.d[(size_t)row * nb + b]);
            (void)ih;
        }
    }
}

template <int UPL, int R>
__device__ __forceinline__ void q6_compute(const Q6Rows<UPL,R>& f, float part[R], const int8_t* sQ, const float* sD,
                                           const int* sB, int lane, int units)
{
#pragma unroll
    for (int rr = 0; rr < R; rr++) part[rr] = 0.0f;
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
        for (int rr = 0; rr < R; rr++) {
            const uint32_t lw[8] = {f.la[rr][k].x,f.la[rr][k].y,f.la[rr][k].z,f.la[rr][k].w,
                                    f.lb[rr][k].x,f.lb[rr][k].y,f.lb[rr][k].z,f.lb[rr][k].w};
            const uint32_t hw[4] = {f.hh[rr][k].x,f.hh[rr][k].y,f.hh[rr][k].z,f.hh[rr][k].w};
            const uint32_t s0 = f.scw[rr][k].x, s1 = f.scw[rr][k].y;
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
            const float wd = half_bits_to_float(f.dh[rr][k]);
            part[rr] = __builtin_fmaf(yd * wd,(float)total,part[rr]);
        }
    }
}

template <int UPL>
__global__ __launch_bounds__(64 * kMvWaves) void matvec_q6_K_kernel(PlanarQ6K w, const float* __restrict__ x, int N, int K,
                                                                    Output out)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / PIX_QK;
    int8_t* sQ = reinterpret_cast<int8_t*>(smem);
    float* sD = reinterpret_cast<float*>(smem + K);
    int* sB = reinterpret_cast<int*>(smem + K + 4 * nb);
    const int lane = threadIdx.x & 63, wave = wave_id();
    constexpr int R = mv_rows<UPL>();
    const int stride = (int)gridDim.x * kMvWaves * R;
    const int first = ((int)blockIdx.x * kMvWaves + wave) * R;
    const int last = N;
    const int units = nb * 4;
    float4 xv[kXPasses * UPL];
    load_x_q8_K(x,K,xv);
    constexpr bool two_sets = UPL <= 2;
    Q6Rows<UPL,R> a, b;
    // Long rows: x is quantized before the first rows are requested, so that
    // its staging registers are free again.
    __builtin_amdgcn_sched_barrier(0);
    if (two_sets) q6_load(a,w,K,first,last,lane,units);
    __builtin_amdgcn_sched_barrier(0);
    quantize_x_q8_K(xv,K,sQ,sD,sB);
    // x's loads precede the rows' 5 * R * UPL (see the Q5_K kernel).
    __builtin_amdgcn_s_waitcnt(wait_vmcnt(two_sets? 5 * R * UPL : 0));
    if (!two_sets) q6_load(a,w,K,first,last,lane,units);
    __syncthreads();
    stream_rows<two_sets>(a,b,first,stride,last,lane,out,
                [&](Q6Rows<UPL,R>& f, int r0) { q6_load(f,w,K,r0,last,lane,units); },
                [&](const Q6Rows<UPL,R>& f, float (&part)[R]) { q6_compute(f,part,sQ,sD,sB,lane,units); });
}

// Launch shape: one round of workgroups, kMvMaxWgPerCu per CU (fewer when the
// kernel's occupancy allows fewer, or when there are fewer row pairs than
// waves); the kernels stride over the rest.
template <typename Kernel>
static void launch_shape(Kernel kernel, size_t lds, size_t N, int rows_per_set, unsigned& grid)
{
    static int cus = 0;
    if (!cus) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v,hipDeviceAttributeMultiprocessorCount,dev) == hipSuccess && v > 0)
            cus = v;
        else
            cus = 256;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu,kernel,64 * kMvWaves,lds) != hipSuccess || per_cu < 1) per_cu = 1;
    per_cu = std::min(per_cu,kMvMaxWgPerCu);
    const size_t waves_needed = (N + rows_per_set - 1) / rows_per_set;
    const size_t slots = (size_t)cus * per_cu * kMvWaves;
    const size_t waves = std::min(waves_needed,slots);
    grid = (unsigned)((waves + kMvWaves - 1) / kMvWaves);
}

// Units of 64 values per lane: rows of up to 6 * 64 * 64 = 24576 values.
template <typename F>
static hipError_t dispatch_upl(int units, F&& f)
{
    if (units <= 64) return f(std::integral_constant<int,1>{});
    if (units <= 128) return f(std::integral_constant<int,2>{});
    if (units <= 192) return f(std::integral_constant<int,3>{});
    if (units <= 256) return f(std::integral_constant<int,4>{});
    if (units <= 320) return f(std::integral_constant<int,5>{});
    if (units <= 384) return f(std::integral_constant<int,6>{});
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_q5_K(const PlanarQ5K& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const size_t nb = K / PIX_QK;
    const size_t lds = K + 4 * nb + 4 * 16 * nb;
    return dispatch_upl((int)(nb * 4),[&](auto upl) {
        auto kernel = matvec_q5_K_kernel<decltype(upl)::value>;
        unsigned grid;
        launch_shape(kernel,lds,N,mv_rows<decltype(upl)::value>(),grid);
        kernel<<<grid,64 * kMvWaves,lds,s>>>(w,x,(int)N,(int)K,out);
        return hipGetLastError();
    });
}

hipError_t launch_matvec_q8_0(const PlanarQ80& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const size_t Kp = (K + 63) / 64 * 64;
    const size_t lds = Kp + 4 * (Kp / PIX_QK8);
    return dispatch_upl((int)(Kp / 64),[&](auto upl) {
        auto kernel = matvec_q8_0_kernel<decltype(upl)::value>;
        unsigned grid;
        launch_shape(kernel,lds,N,mv_rows<decltype(upl)::value>(),grid);
        kernel<<<grid,64 * kMvWaves,lds,s>>>(w,x,(int)N,(int)K,(int)Kp,out);
        return hipGetLastError();
    });
}

hipError_t launch_matvec_q6_K(const PlanarQ6K& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s)
{
    const size_t nb = K / PIX_QK;
    const size_t lds = K + 4 * nb + 4 * 16 * nb;
    return dispatch_upl((int)(nb * 4),[&](auto upl) {
        auto kernel = matvec_q6_K_kernel<decltype(upl)::value>;
        unsigned grid;
        launch_shape(kernel,lds,N,mv_rows<decltype(upl)::value>(),grid);
        kernel<<<grid,64 * kMvWaves,lds,s>>>(w,x,(int)N,(int)K,out);
        return hipGetLastError();
    });
}

}  // namespace pixhip
