// Quantized GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for
// Q5_K / Q6_K / Q8_0 weights and Q8_K / Q8_0 activations.  The counterpart of
// pix_dot_q5_K / pix_dot_q6_K / pix_dot_q8_0 driven by cpu_quant_matmul
// (src/kernels_quant.cpp:163-365, :369-412) and of shaders/matmul_mmq.comp.
//
// Tiling: a workgroup of 8 waves (4 along tokens x 2 along features) owns a
// 256x128 output tile; each wave owns 64x64 = 2x2 tiles of
// v_mfma_i32_32x32x32_i8 (A = activations, rows = tokens; B = weights, columns =
// output features: each lane holds one feature column and 16 token rows of
// every 32x32 accumulator).  One workgroup fills a CU at two waves per SIMD, so
// one wave's fp32 epilogue overlaps the other's MFMAs.
//
// Data movement: K advances in 64-byte stages (two 32-value sub-blocks) through
// a 3-deep LDS ring filled by global_load_lds_dwordx4 (HBM -> LDS without
// registers), so two stages are in flight while one is consumed.  Lane l of a
// DMA instruction lands at LDS base + 16*l; each lane picks its source piece so
// that the ring holds rows of four 16-byte pieces with piece c of row r at slot
// 4r + (c ^ g(r)), g(r) = ((r>>1) ^ (r>>3)) & 3, which keeps the MFMA operand
// reads (ds_read_b128, 32 rows per half-wave) free of bank conflicts.  Per
// 256-value super-block the scale data (activation d and 16-value sums, weight
// d, dmin and sub-block minima) rides in a double-buffered LDS region loaded the
// same way with the super-block's first stage.  Synchronisation is explicit:
// s_waitcnt vmcnt for this wave's DMAs, then s_barrier (no fence, which would
// drain every in-flight stage).  The loop body takes its LDS buffers as
// __restrict__ pointers: the buffer being filled and the one being read are
// distinct in every iteration, and the alias scopes this gives the compiler
// keep it from draining the DMA queue before each LDS read.
//
// Exactness: the MFMAs produce, per (token, feature, super-block), the exact
// integers the reference forms before its fp32 epilogue:
//   Q5_K  S = sum_s scale_s*dot_s   from the hi/lo planes (64*hi + lo)
//         Mn = sum_s min_s*(bsum_2s + bsum_2s+1)  by one fp16 MFMA (inputs exact
//              in fp16: min <= 63, |bsum16| <= 2032; |Mn| < 2^24 so fp32 is exact)
//   Q6_K  S = sum_e scale*(q-32)*q8 from the hi/lo planes
//   Q8_0  P = sum over the 32-value block of q*q8
// then y += yd*(wd*S - wdmin*Mn) per super-block (Q5_K), y += yd*(wd*S)
// (Q6_K), y += xd*(wd*P) per block (Q8_0), in fp32.
#include <type_traits>

#include "pixhip_device.h"
#include "pixhip_internal.h"

#define PIX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace pixhip {

constexpr int kBM = PIX_GEMM_MTILE, kBN = PIX_GEMM_NTILE, kKC = 64;
constexpr int kWavesM = 4, kWavesN = 2, kWaves = kWavesM * kWavesN, kThreads = 64 * kWaves;
constexpr int kStages = 3;
constexpr int kATile = kBM * kKC;  // 16 KB: activation tile of one stage
constexpr int kWTile = kBN * kKC;  // 8 KB: one weight plane of one stage
constexpr int kChunk = 1024;       // bytes written by one DMA instruction (64 lanes x 16 B)
constexpr int kStageBytes = 32768;
constexpr int kStageChunks = kStageBytes / kChunk;  // 32: 4 per wave
constexpr int kSBC = PIX_QK / kKC;                  // stages per super-block (4)
static_assert(kWavesM * 64 == kBM && kWavesN * 64 == kBN, "wave grid covers the tile");

enum Kind { KIND_Q5K = 0, KIND_Q6K = 1, KIND_Q80 = 2 };

// Stage slots (16 B):  K-quants  A 0..1023 | W.hi 1024..1535 | W.lo 1536..2047
//                      Q8_0      A 0..1023 | W 1024..1535 | xd[2][256] 1536..1663 |
//                                wd[2][128] 1664..1727 | pad
// Super-block scale region (K-quants, 16 KB, double buffered):
//   yd[256] 0..63 | bs[256][2] 64..575 | mn[128] 576..703 | wd[128] 704..735 |
//   wdm[128] 736..767 | pad
constexpr int kSlotW = 1024, kSlotW2 = 1536, kSlotXd80 = 1536, kSlotWd80 = 1664, kSlotPad80 = 1728;
constexpr int kScaleBytes = 16384, kScaleChunks = kScaleBytes / kChunk;  // 16: 2 per wave
constexpr int kSlotYd = 0, kSlotBs = 64, kSlotMn = 576, kSlotWd = 704, kSlotWdm = 736, kSlotScalePad = 768;

struct GemmArgs {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/QK][Mpad]  (QK = 256, or 32 for Q8_0)
    const _Float16* xbs;  // [Mpad][K/16]  (Q5_K only)
    const int8_t* whi;    // [Npad][K] (Q8_0: the quantized plane)
    const int8_t* wlo;    // [Npad][K]
    const float* wdT;     // [K/QK][Npad]
    const float* wdmT;    // [K/256][Npad] (Q5_K)
    const _Float16* wmn;  // [K/256][Npad][8] (Q5_K)
    float* y;
    const float* bias;
    int32_t* sums;        // debug: exact integer sums [M][N][blocks]
    int32_t* mins;
    int M, N, K, Mpad, Npad;
    size_t ldy, yoff;
    int tiles_m, tiles_n;
};

struct Ctx {
    int m0, n0, wave, lane, wm, wn, lr, lg, sw, K, nchunks;
};

struct Acc {
    v16i hi[2][2], lo[2][2];
    v16f y[2][2];
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt_hi[15:14]).
template <int N> __device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_uniform)
{
    __builtin_amdgcn_global_load_lds(src,PIX_LDS(lds_uniform),16,0,0);
}

__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// Bijective XCD-aware remap: hardware places workgroup b on XCD b % 8; give
// each XCD a contiguous range of logical tiles so its L2 sees neighbours.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd < r? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// Per-lane byte offset of a 64-slot DMA chunk covering 16 rows of 64 bytes
// (rows row0..row0+15 of a tile with row stride `stride`), in the swizzled
// order the MFMA operand reads expect.
__device__ __forceinline__ uint32_t tile_lane_offset(int row0, int lane, int stride)
{
    const int row = row0 + (lane >> 2);
    return (uint32_t)((lane >> 2) * stride + 16 * ((lane & 3) ^ swz(row)));
}

// Opaque copy of a per-lane 32-bit offset: stops the compiler from folding it
// into a loop-invariant 64-bit pointer (which costs two VGPRs per DMA and
// spills), so the DMA keeps the scalar-base + 32-bit-offset form.
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    __asm__ volatile("" : "+v"(v));
    return v;
}

// DMA of stage c into `st` (kStageChunks / kWaves instructions per wave).  Every
// 64-slot chunk lies in one region, so its source is a wave-uniform base plus a
// 32-bit per-lane offset.
template <int KIND>
__device__ __forceinline__ void issue_stage(const GemmArgs& g, const Ctx& x, int c, uint8_t* st)
{
    const int k0 = c * kKC;
#pragma unroll
    for (int q = 0; q < kStageChunks / kWaves; q++) {
        const int chunk = x.wave + kWaves * q;  // wave-uniform
        const int slot0 = chunk * 64;
        const uint8_t* src;
        if (slot0 < kSlotW) {
            const int row0 = slot0 >> 2;
            src = reinterpret_cast<const uint8_t*>(g.xq) + (size_t)(x.m0 + row0) * x.K + k0 + opaque(tile_lane_offset(row0,x.lane,x.K));
        } else if (KIND != KIND_Q80 || slot0 < kSlotW2) {
            const int row0 = (slot0 - (slot0 < kSlotW2? kSlotW : kSlotW2)) >> 2;
            const int8_t* plane = slot0 < kSlotW2? g.whi : g.wlo;
            src = reinterpret_cast<const uint8_t*>(plane) + (size_t)(x.n0 + row0) * x.K + k0 + opaque(tile_lane_offset(row0,x.lane,x.K));
        } else if (slot0 < kSlotWd80) {
            const int blk = (slot0 - kSlotXd80) >> 6;
            src = reinterpret_cast<const uint8_t*>(g.xdT + (size_t)(2 * c + blk) * g.Mpad + x.m0) + opaque(16 * x.lane);
        } else if (slot0 < kSlotPad80) {
            src = reinterpret_cast<const uint8_t*>(g.wdT + (size_t)(2 * c) * g.Npad + x.n0) +
                  opaque(4 * ((x.lane >> 5) * g.Npad + 4 * (x.lane & 31)));
        } else {
            src = reinterpret_cast<const uint8_t*>(g.xdT);  // padding chunk: any valid address
        }
        dma16(src,st + chunk * kChunk);
    }
}

// DMA of super-block b's scale data into `sc` (K-quants).
template <int KIND>
__device__ __forceinline__ void issue_scales(const GemmArgs& g, const Ctx& x, int b, uint8_t* sc)
{
#pragma unroll
    for (int q = 0; q < kScaleChunks / kWaves; q++) {
        const int chunk = x.wave + kWaves * q;  // wave-uniform
        const int slot0 = chunk * 64;
        const uint8_t* src = reinterpret_cast<const uint8_t*>(g.xdT);  // padding and unused chunks
        if (slot0 < kSlotBs) {
            src = reinterpret_cast<const uint8_t*>(g.xdT + (size_t)b * g.Mpad + x.m0) + opaque(16 * x.lane);
        } else if (slot0 < kSlotMn) {
            // bs: row (slot-64)/2, half (slot-64)%2
            const int row0 = (slot0 - kSlotBs) >> 1;
            if (KIND == KIND_Q5K)
                src = reinterpret_cast<const uint8_t*>(g.xbs + (size_t)(x.m0 + row0) * (x.K / 16) + b * 16) +
                      opaque((x.lane >> 1) * (x.K / 8) + 16 * (x.lane & 1));
        } else if (slot0 < kSlotWd) {
            if (KIND == KIND_Q5K)
                src = reinterpret_cast<const uint8_t*>(g.wmn + ((size_t)b * g.Npad + x.n0 + (slot0 - kSlotMn)) * 8) + opaque(16 * x.lane);
        } else if (slot0 < kSlotScalePad) {
            // wd in lanes 0..31, wdm in lanes 32..63 (Q6_K has no wdm: reread wd)
            // (a per-lane choice of plane: both sit at the same offset)
            const uint32_t off = opaque(16 * (x.lane & 31));
            const float* plane = (KIND == KIND_Q5K && x.lane >= 32)? g.wdmT : g.wdT;
            src = reinterpret_cast<const uint8_t*>(plane + (size_t)b * g.Npad + x.n0) + off;
        }
        dma16(src,sc + chunk * kChunk);
    }
}

// One iteration: start stage c+2's DMA (into dma_stage / dma_scale), consume
// stage c (cur / cur_scale).  In every call the buffers written and the
// buffers read are distinct objects.  PHASE = c % 4 is a compile-time
// constant for K-quants (the caller unrolls one super-block per loop trip), so
// the integer accumulators are visibly dead between a super-block's epilogue
// and the next super-block's first MFMA.
template <int KIND, bool SUMS, int PHASE>
__device__ __forceinline__ void gemm_step(const GemmArgs& g, const Ctx& x, int c, Acc& acc, uint8_t* __restrict__ dma_stage,
                                          uint8_t* __restrict__ dma_scale, const uint8_t* __restrict__ cur,
                                          const uint8_t* __restrict__ cur_scale)
{
    constexpr int PLANES = KIND == KIND_Q80? 1 : 2;
    if (c + 2 < x.nchunks) {
        issue_stage<KIND>(g,x,c + 2,dma_stage);
        if constexpr (KIND != KIND_Q80 && (PHASE + 2) % kSBC == 0) issue_scales<KIND>(g,x,(c + 2) / kSBC,dma_scale);
    }
    const v16i izero = {};
    const v16f fzero = {};
    constexpr bool fresh = KIND != KIND_Q80 && PHASE == 0;  // first stage of a super-block: start from zero
    if constexpr (KIND == KIND_Q5K && !SUMS) {
        // Minimum term of the super-block, applied while its integer
        // accumulators are still empty: y -= yd * wdmin * Mn.
        if constexpr (fresh) {
            const float* syd = reinterpret_cast<const float*>(cur_scale + 16 * kSlotYd);
            const float* swm = reinterpret_cast<const float*>(cur_scale + 16 * kSlotWdm);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = x.wn * 64 + j * 32 + x.lr;
                const float nwm = -swm[col];
                const v8h mnB = *reinterpret_cast<const v8h*>(cur_scale + 16 * (kSlotMn + col));
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const v8h bsA = *reinterpret_cast<const v8h*>(cur_scale + 16 * (kSlotBs + 2 * (x.wm * 64 + i * 32 + x.lr) + x.lg));
                    const v16f mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA,mnB,fzero,0,0,0);
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const float4 t = *reinterpret_cast<const float4*>(syd + x.wm * 64 + i * 32 + 8 * q4 + 4 * x.lg);
                        const float yq[4] = {t.x,t.y,t.z,t.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc.y[i][j][4 * q4 + e] = __builtin_fmaf(yq[e],mt[4 * q4 + e] * nwm,acc.y[i][j][4 * q4 + e]);
                    }
                }
            }
            // Keep the super-block's first MFMAs (which start the integer
            // accumulators) after this block, so both never hold registers at once.
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int cp = ((2 * s + x.lg) ^ x.sw) * 16;
        v4i a[2], wh[2], wl[2];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const v4i*>(cur + (x.wm * 64 + i * 32 + x.lr) * 64 + cp);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            wh[j] = *reinterpret_cast<const v4i*>(cur + 16 * kSlotW + (x.wn * 64 + j * 32 + x.lr) * 64 + cp);
            if constexpr (PLANES == 2) wl[j] = *reinterpret_cast<const v4i*>(cur + 16 * kSlotW2 + (x.wn * 64 + j * 32 + x.lr) * 64 + cp);
        }
        if constexpr (KIND == KIND_Q80) {
            // One 32-value block per sub-block: fresh accumulator, fp32 epilogue.
            const float* sxd = reinterpret_cast<const float*>(cur + 16 * kSlotXd80) + s * kBM;
            const float* swd = reinterpret_cast<const float*>(cur + 16 * kSlotWd80) + s * kBN;
            float wdv[2];
#pragma unroll
            for (int j = 0; j < 2; j++) wdv[j] = swd[x.wn * 64 + j * 32 + x.lr];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float xdv[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const float4 t = *reinterpret_cast<const float4*>(sxd + x.wm * 64 + i * 32 + 8 * q4 + 4 * x.lg);
                    xdv[4 * q4 + 0] = t.x;
                    xdv[4 * q4 + 1] = t.y;
                    xdv[4 * q4 + 2] = t.z;
                    xdv[4 * q4 + 3] = t.w;
                }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],izero,0,0,0);
                    if constexpr (SUMS) {
                        const int kb = c * 2 + s;
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = x.m0 + x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * x.lg + (r & 3);
                            const int n = x.n0 + x.wn * 64 + j * 32 + x.lr;
                            if (m < g.M && n < g.N) g.sums[((size_t)m * g.N + n) * (x.K / PIX_QK8) + kb] = p[r];
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; r++) acc.y[i][j][r] = __builtin_fmaf(xdv[r],(float)p[r] * wdv[j],acc.y[i][j][r]);
                    }
                }
            }
        } else {
            if (s == 0 && fresh) {  // fresh is a compile-time constant
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        acc.hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],izero,0,0,0);
                        acc.lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wl[j],izero,0,0,0);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        acc.hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],acc.hi[i][j],0,0,0);
                        acc.lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wl[j],acc.lo[i][j],0,0,0);
                    }
            }
        }
    }
    if constexpr (KIND != KIND_Q80) {
        if constexpr (PHASE != kSBC - 1) return;
        // Super-block epilogue: exact integer sum -> fp32, y += yd * wd * S.
        const int b = c / kSBC;
        const float* syd = reinterpret_cast<const float*>(cur_scale + 16 * kSlotYd);
        const float* swd = reinterpret_cast<const float*>(cur_scale + 16 * kSlotWd);
        float wdv[2];
#pragma unroll
        for (int j = 0; j < 2; j++) wdv[j] = swd[x.wn * 64 + j * 32 + x.lr];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float ydv[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const float4 t = *reinterpret_cast<const float4*>(syd + x.wm * 64 + i * 32 + 8 * q4 + 4 * x.lg);
                ydv[4 * q4 + 0] = t.x;
                ydv[4 * q4 + 1] = t.y;
                ydv[4 * q4 + 2] = t.z;
                ydv[4 * q4 + 3] = t.w;
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if constexpr (SUMS) {
                    v16f mt = fzero;
                    if constexpr (KIND == KIND_Q5K) {
                        const int col = x.wn * 64 + j * 32 + x.lr;
                        const v8h mnB = *reinterpret_cast<const v8h*>(cur_scale + 16 * (kSlotMn + col));
                        const v8h bsA = *reinterpret_cast<const v8h*>(cur_scale + 16 * (kSlotBs + 2 * (x.wm * 64 + i * 32 + x.lr) + x.lg));
                        mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA,mnB,fzero,0,0,0);
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = x.m0 + x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * x.lg + (r & 3);
                        const int n = x.n0 + x.wn * 64 + j * 32 + x.lr;
                        if (m < g.M && n < g.N) {
                            const size_t o = ((size_t)m * g.N + n) * (x.K / PIX_QK) + b;
                            g.sums[o] = acc.hi[i][j][r] * 64 + acc.lo[i][j][r];
                            if constexpr (KIND == KIND_Q5K) g.mins[o] = (int32_t)mt[r];
                        }
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float t = (float)(acc.hi[i][j][r] * 64 + acc.lo[i][j][r]) * wdv[j];
                        acc.y[i][j][r] = __builtin_fmaf(ydv[r],t,acc.y[i][j][r]);
                    }
                }
            }
        }
    }
}

template <int KIND, bool SUMS>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g)
{
    constexpr bool SCALES = KIND != KIND_Q80;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes + (SCALES? 2 * kScaleBytes : 0)];
    uint8_t* const scale_base = lds + kStages * kStageBytes;

    const int nblocks = g.tiles_m * g.tiles_n;
    const int lid = xcd_remap((int)blockIdx.x,nblocks);
    constexpr int GROUP = 8;  // token tiles sharing one feature tile, in launch order
    const int group = lid / (GROUP * g.tiles_n);
    const int first_m = group * GROUP;
    const int gsize = min(g.tiles_m - first_m,GROUP);
    const int within = lid % (GROUP * g.tiles_n);
    const int tm = first_m + within % gsize, tn = within / gsize;

    Ctx x;
    x.m0 = tm * kBM;
    x.n0 = tn * kBN;
    x.wave = threadIdx.x >> 6;
    x.lane = threadIdx.x & 63;
    x.wm = x.wave % kWavesM;
    x.wn = x.wave / kWavesM;
    x.lr = x.lane & 31;
    x.lg = x.lane >> 5;
    x.sw = swz(x.lr);  // rows read by this lane are lr + 32k: same swizzle
    x.K = g.K;
    x.nchunks = g.K / kKC;

    Acc acc;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc.hi[i][j] = v16i{};
            acc.lo[i][j] = v16i{};
            acc.y[i][j] = v16f{};
        }

    issue_stage<KIND>(g,x,0,lds);
    if constexpr (SCALES) issue_scales<KIND>(g,x,0,scale_base);
    if (x.nchunks > 1) issue_stage<KIND>(g,x,1,lds + kStageBytes);

    // Stage c has landed once only the DMAs of stage c+1 may still be in flight.
    // (The integer-sum debug variant also stores inside the loop; stores share
    // vmcnt and may retire early, so it drains everything.)
    auto step = [&](auto phase, int c) {
        constexpr int P = decltype(phase)::value;
        if (c + 1 < x.nchunks && !SUMS) {
            if constexpr (KIND != KIND_Q80 && P == kSBC - 1) wait_vmcnt<kStageChunks / kWaves + kScaleChunks / kWaves>();
            else wait_vmcnt<kStageChunks / kWaves>();
        } else {
            wait_vmcnt<0>();
        }
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        const int b_dma = (c + 2) / kSBC, b_cur = c / kSBC;
        gemm_step<KIND,SUMS,P>(g,x,c,acc,lds + ((c + 2) % kStages) * kStageBytes,scale_base + (b_dma & 1) * kScaleBytes,
                               lds + (c % kStages) * kStageBytes,scale_base + (b_cur & 1) * kScaleBytes);
    };
    if constexpr (KIND == KIND_Q80) {
        for (int c = 0; c < x.nchunks; c++) step(std::integral_constant<int,0>{},c);
    } else {
        for (int c = 0; c < x.nchunks; c += kSBC) {
            step(std::integral_constant<int,0>{},c);
            step(std::integral_constant<int,1>{},c + 1);
            step(std::integral_constant<int,2>{},c + 2);
            step(std::integral_constant<int,3>{},c + 3);
        }
    }

    if constexpr (!SUMS) {
        // Bias for this lane's two columns, loaded once (clamped index) and
        // drained before the stores: a load left pending here would make every
        // store below wait for all earlier stores.
        float bv[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = min(x.n0 + x.wn * 64 + j * 32 + x.lr,g.N - 1);
            bv[j] = g.bias? g.bias[n] : 0.0f;
        }
        wait_vmcnt<0>();
        const int mrow0 = x.m0 + x.wm * 64, ncol0 = x.n0 + x.wn * 64;
        const bool full = mrow0 + 64 <= g.M && ncol0 + 64 <= g.N;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = ncol0 + j * 32 + x.lr;
                float* col = g.y + g.yoff + n;
                if (full) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = mrow0 + i * 32 + 8 * (r >> 2) + 4 * x.lg + (r & 3);
                        col[(size_t)m * g.ldy] = acc.y[i][j][r] + bv[j];
                    }
                } else if (n < g.N) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = mrow0 + i * 32 + 8 * (r >> 2) + 4 * x.lg + (r & 3);
                        if (m < g.M) col[(size_t)m * g.ldy] = acc.y[i][j][r] + bv[j];
                    }
                }
            }
    }
}

static size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

template <int KIND, bool SUMS>
static hipError_t launch(GemmArgs g, size_t mpad, size_t npad, hipStream_t s)
{
    g.tiles_m = (int)((g.M + kBM - 1) / kBM);
    g.tiles_n = (int)((g.N + kBN - 1) / kBN);
    if (mpad < round_up((size_t)g.M,kBM) || npad < round_up((size_t)g.N,kBN) || g.K % kKC) return hipErrorInvalidValue;
    g.Mpad = (int)mpad;
    g.Npad = (int)npad;
    const int nblocks = g.tiles_m * g.tiles_n;
    if (!nblocks) return hipSuccess;
    gemm_kernel<KIND,SUMS><<<dim3(nblocks),dim3(kThreads),0,s>>>(g);
    return hipGetLastError();
}

static GemmArgs base_args(size_t M, size_t N, size_t K)
{
    GemmArgs g = {};
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    return g;
}

hipError_t launch_gemm_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d; g.xbs = a.bs;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdmT = w.dm; g.wmn = w.mn;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q5K,false>(g,a.mpad,w.npad,s);
}

hipError_t launch_gemm_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q6K,false>(g,a.mpad,w.npad,s);
}

hipError_t launch_gemm_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.qs; g.wdT = w.dT;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q80,false>(g,a.mpad,round_up(N,kBN),s);
}

hipError_t launch_sums_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, int32_t* scaled, int32_t* mins,
                            hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d; g.xbs = a.bs;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdmT = w.dm; g.wmn = w.mn;
    g.sums = scaled; g.mins = mins;
    return launch<KIND_Q5K,true>(g,a.mpad,w.npad,s);
}

hipError_t launch_sums_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.sums = sums;
    return launch<KIND_Q6K,true>(g,a.mpad,w.npad,s);
}

hipError_t launch_sums_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.qs; g.wdT = w.dT;
    g.sums = sums;
    return launch<KIND_Q80,true>(g,a.mpad,round_up(N,kBN),s);
}

}  // namespace pixhip
