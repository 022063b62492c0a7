// Quantized GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for
// Q5_K / Q6_K / Q8_0 weights and Q8_K / Q8_0 activations.  The counterpart of
// pix_dot_q5_K / pix_dot_q6_K / pix_dot_q8_0 driven by cpu_quant_matmul
// (src/kernels_quant.cpp:163-365, :369-412) and of shaders/matmul_mmq.comp.
//
// Tiling: a workgroup of 8 waves (4 along tokens x 2 along features) owns a
// 256x128 output tile; each wave owns 64x64 = 2x2 tiles of
// v_mfma_i32_32x32x32_i8 (A = activations, rows = tokens; B = weights, columns =
// output features: each lane holds one feature column and 16 token rows of
// every 32x32 accumulator).  One workgroup fills a CU at two waves per SIMD.
//
// Staggered epilogues: the waves of feature half 0 apply a super-block's fp32
// epilogue at the end of its last stage, those of half 1 at the start of the
// next super-block's first stage.  Waves w and w+4 (one of each half) share a
// SIMD, so each epilogue's vector ALU work overlaps the other wave's MFMAs.
//
// Data movement: K advances in 64-byte stages (two 32-value sub-blocks),
// loaded with buffer_load_dwordx4 ... lds (HBM -> LDS, no registers).  Lane l
// of a DMA lands at LDS base + 16*l; the source is a buffer resource (SGPRs) +
// a per-lane offset fixed for the whole kernel (VGPR) + a wave-uniform offset
// (SGPR), so DMA issue costs no vector ALU work.  Four consecutive lanes fetch
// one 64-byte row (coalesced), and each lane picks its piece so that the ring
// holds rows of four 16-byte pieces with piece c of row r at slot
// 4r + (c ^ ((r>>2) & 3)).  With that swizzle the MFMA operand reads
// (ds_read_b128: lane l reads row l%32, piece 2s + l/32) measured free of LDS
// bank conflicts on gfx950; swizzles on the low row bits did not.
// Per 256-value super-block the scale data (activation d and 16-value sums,
// weight d, dmin and sub-block minima) rides in a double-buffered LDS region
// loaded the same way.  Synchronisation is explicit: s_waitcnt vmcnt for this
// wave's DMAs, then s_barrier (no fence, which would drain every in-flight
// stage).  The loop body takes its LDS buffers as __restrict__ pointers: the
// buffers being filled and those being read are distinct in every iteration,
// and the alias scopes this gives the compiler keep it from draining the DMA
// queue before each LDS read.
//
// Exactness: the MFMAs produce, per (token, feature, super-block), the exact
// integers the reference forms before its fp32 epilogue:
//   Q5_K  S = sum_s scale_s*dot_s   from the hi/lo planes (64*hi + lo)
//         Mn = sum_s min_s*(bsum_2s + bsum_2s+1)  by one fp16 MFMA (inputs exact
//              in fp16: min <= 63, |bsum16| <= 2048; |Mn| < 2^24 so fp32 is exact)
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
constexpr int kStages = 4;         // ring depth: one stage read, kDist in flight
constexpr int kDist = kStages - 1; // prefetch distance in stages
constexpr int kChunk = 1024;       // bytes written by one DMA instruction (64 lanes x 16 B)
constexpr int kStageBytes = 32768;
constexpr int kStageChunks = kStageBytes / kChunk;  // 32: 4 per wave
constexpr int kPerWave = kStageChunks / kWaves;
constexpr int kSBC = PIX_QK / kKC;                  // stages per super-block (4)
static_assert(kWavesM * 64 == kBM && kWavesN * 64 == kBN, "wave grid covers the tile");
static_assert(kWavesN == 2, "the staggered epilogue pairs the two feature halves");

enum Kind { KIND_Q5K = 0, KIND_Q6K = 1, KIND_Q80 = 2 };

// Stage slots (16 B):  K-quants  A 0..1023 | W.hi 1024..1535 | W.lo 1536..2047
//                      Q8_0      A 0..1023 | W 1024..1535 | xd[2][256] 1536..1663 |
//                                wd[2][128] 1664..1727 | unused
// Super-block scale region (K-quants, 16 KB, double buffered):
//   yd[256] 0..63 | bs[256][2] 64..575 | mn[128] 576..703 | wd[128] 704..735 |
//   wdm[128] 736..767 | unused
constexpr int kSlotW = 1024, kSlotW2 = 1536, kSlotXd80 = 1536, kSlotWd80 = 1664;
constexpr int kScaleBytes = 16384, kScaleChunks = kScaleBytes / kChunk;  // 16: 2 per wave
constexpr int kScalePerWave = kScaleChunks / kWaves;
constexpr int kSlotYd = 0, kSlotBs = 64, kSlotMn = 576, kSlotWd = 704, kSlotWdm = 736;

typedef __amdgpu_buffer_rsrc_t Rsrc;

struct GemmArgs {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/QK][Mpad]  (QK = 256, or 32 for Q8_0)
    const _Float16* xbs;  // [Mpad][K/16]  (Q5_K only)
    const int8_t* whi;    // [Npad][K] (Q8_0: the quantized plane)
    const int8_t* wlo;    // [Npad][K]
    const float* wdT;     // [K/QK][Npad]; Q5_K: followed (at wdm_off bytes) by dmin [K/256][Npad]
    uint32_t wdm_off;
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
    uint32_t vo_rows, vo_lin, vo_bs, vo_wd;  // per-lane DMA offsets (bytes)
    Rsrc rx, rxd, rxbs, rwh, rwl, rwd, rwmn;
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

__device__ __forceinline__ Rsrc make_rsrc(const void* base, size_t bytes)
{
    // Raw buffer, stride 0: offsets at or beyond `bytes` read as zero.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base),(short)0,(int)bytes,0x00020000);
}

__device__ __forceinline__ void dma(Rsrc r, uint8_t* lds_uniform, uint32_t voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,PIX_LDS(lds_uniform),16,(int)voff,(int)soff,0,0);
}

// A DMA into an unused chunk, so that every wave issues the same number of
// DMAs per stage (the vmcnt waits count them): re-reads the first 1 KB of the
// activation scales.
__device__ __forceinline__ void pad_dma(const Ctx& x, uint8_t* dst) { dma(x.rxd,dst,x.vo_lin,0); }

// The lane index, recomputed where it is used (volatile, so the compiler
// cannot keep derived per-lane offsets live across the loop: the scale DMAs
// run once per super-block and their offsets would otherwise occupy VGPRs
// the MFMA loop needs).
__device__ __forceinline__ uint32_t lane_now()
{
    uint32_t l;
    __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Bijective XCD-aware remap: hardware places workgroup b on XCD b % 8; give
// each XCD a contiguous range of logical tiles so its L2 sees neighbours.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd < r? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// DMA of stage c into `st`.  Chunk q*8 + wave of the 32 is this wave's q-th;
// q = 0, 1 are activation rows, q = 2 the first weight plane, q = 3 the second
// (Q8_0: the block scales).  A 64-slot chunk covers 16 rows of 64 bytes; lane
// l fetches chunk row l/4, piece (l%4) ^ ((l/16) & 3) (vo_rows).
template <int KIND>
__device__ __forceinline__ void issue_stage(const GemmArgs& g, const Ctx& x, int c, uint8_t* st)
{
    const uint32_t k0 = (uint32_t)c * kKC;
    const uint32_t lane = lane_now();
    // lane l fetches chunk row l/4, piece (l%4) ^ ((l/16) & 3)
    const uint32_t vo_rows = (lane >> 2) * (uint32_t)x.K + 16u * ((lane & 3) ^ ((lane >> 4) & 3));
    const uint32_t vo_lin = 16u * lane;
    const uint32_t vo_wd = 16u * (lane & 31) + (lane >> 5) * 4u * (uint32_t)g.Npad;
#pragma unroll
    for (int q = 0; q < kPerWave; q++) {
        const int chunk = x.wave + kWaves * q;
        uint8_t* dst = st + chunk * kChunk;
        if (q < 2) {
            dma(x.rx,dst,vo_rows,(uint32_t)(x.m0 + chunk * 16) * x.K + k0);
        } else if (q == 2 || KIND != KIND_Q80) {
            const int row0 = (chunk - (q == 2? 16 : 24)) * 16;
            dma(q == 2? x.rwh : x.rwl,dst,vo_rows,(uint32_t)(x.n0 + row0) * x.K + k0);
        } else {
            // chunks 24, 25: activation scales of blocks 2c, 2c+1; 26: weight
            // scales of both blocks; 27..31 unused.
            if (x.wave < 2)
                dma(x.rxd,dst,vo_lin,(uint32_t)((2 * c + x.wave) * g.Mpad + x.m0) * 4u);
            else if (x.wave == 2)
                dma(x.rwd,dst,vo_wd,(uint32_t)(2 * c * g.Npad + x.n0) * 4u);
            else
                dma(x.rxd,dst,vo_lin,0);
        }
    }
}

// DMA of super-block b's scale data into `sc` (K-quants): chunk 0 yd, 1..8 bs,
// 9..10 mn, 11 wd (lanes 0..31) + wdm (lanes 32..63), 12..15 unused.
template <int KIND>
__device__ __forceinline__ void issue_scales(const GemmArgs& g, const Ctx& x, int b, uint8_t* sc)
{
    const uint32_t lane = lane_now();
    const uint32_t vo_lin = 16u * lane;
    const uint32_t vo_bs = (lane >> 1) * (uint32_t)(x.K / 8) + 16u * (lane & 1);
    const uint32_t vo_wd = 16u * (lane & 31) + (lane >> 5) * g.wdm_off;
#pragma unroll
    for (int q = 0; q < kScalePerWave; q++) {
        const int chunk = x.wave + kWaves * q;
        uint8_t* dst = sc + chunk * kChunk;
        if (chunk == 0) {
            dma(x.rxd,dst,vo_lin,(uint32_t)(b * g.Mpad + x.m0) * 4u);
        } else if (chunk <= 8) {
            if (KIND == KIND_Q5K)
                dma(x.rxbs,dst,vo_bs,((uint32_t)(x.m0 + (chunk - 1) * 32) * (x.K / 16) + b * 16) * 2u);
            else
                dma(x.rxd,dst,vo_lin,0);
        } else if (chunk <= 10) {
            if (KIND == KIND_Q5K)
                dma(x.rwmn,dst,vo_lin,(uint32_t)(b * g.Npad + x.n0 + (chunk - 9) * 64) * 16u);
            else
                dma(x.rxd,dst,vo_lin,0);
        } else if (chunk == 11) {
            dma(x.rwd,dst,vo_wd,(uint32_t)(b * g.Npad + x.n0) * 4u);
        } else {
            dma(x.rxd,dst,vo_lin,0);
        }
    }
}

// Mn of tile (I, column col) for the super-block whose scales are in `sc`:
// sum_s min_s*(bsum_2s + bsum_2s+1) as one fp16 MFMA (exact, see above).
template <int I>
__device__ __forceinline__ v16f min_term(const Ctx& x, int col, const uint8_t* __restrict__ sc)
{
    const v16f fzero = {};
    const v8h mnB = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotMn + col));
    const v8h bsA = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotBs + 2 * (x.wm * 64 + I * 32 + x.lr) + x.lg));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA,mnB,fzero,0,0,0);
}

// fp32 epilogue of one tile row (I) for super-block b: y += yd*(wd*S - wdm*Mn)
// (the integer-sum debug variant stores S, and Mn for Q5_K).  The empty asm
// statements keep the compiler from hoisting the LDS reads of later tiles
// (their scale values) above earlier ones, which would hold more registers
// than the kernel has.
template <int KIND, bool SUMS, int I>
__device__ __forceinline__ void sb_epilogue(const GemmArgs& g, const Ctx& x, int b, Acc& acc, const uint8_t* __restrict__ sc)
{
    const float* syd = reinterpret_cast<const float*>(sc + 16 * kSlotYd);
    const float* swd = reinterpret_cast<const float*>(sc + 16 * kSlotWd);
    const v16f fzero = {};
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = x.wn * 64 + j * 32 + x.lr;
        if constexpr (SUMS) {
            const v16f mt = KIND == KIND_Q5K? min_term<I>(x,col,sc) : fzero;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = x.m0 + x.wm * 64 + I * 32 + 8 * (r >> 2) + 4 * x.lg + (r & 3);
                const int n = x.n0 + col;
                if (m < g.M && n < g.N) {
                    const size_t o = ((size_t)m * g.N + n) * (x.K / PIX_QK) + b;
                    g.sums[o] = acc.hi[I][j][r] * 64 + acc.lo[I][j][r];
                    if constexpr (KIND == KIND_Q5K) g.mins[o] = (int32_t)mt[r];
                }
            }
        } else {
            __asm__ volatile("" ::: "memory");
            const float wd = swd[col];
            const float nwm = KIND == KIND_Q5K? -reinterpret_cast<const float*>(sc + 16 * kSlotWdm)[col] : 0.0f;
            const v16f mt = KIND == KIND_Q5K? min_term<I>(x,col,sc) : fzero;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const float4 t4 = *reinterpret_cast<const float4*>(syd + x.wm * 64 + I * 32 + 8 * q4 + 4 * x.lg);
                const float yq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q4 + e;
                    float t = (float)(acc.hi[I][j][r] * 64 + acc.lo[I][j][r]) * wd;
                    if constexpr (KIND == KIND_Q5K) t = __builtin_fmaf(mt[r],nwm,t);
                    acc.y[I][j][r] = __builtin_fmaf(yq[e],t,acc.y[I][j][r]);
                }
            }
        }
    }
}

// DMA instructions a wave may still have in flight when the stage of phase P
// must have landed: those of the kDist-1 iterations before it, plus the
// scales issued with the stage kDist ahead of a super-block start.
template <bool SCALES> constexpr int outstanding(int P)
{
    int n = (kDist - 1) * kPerWave;
    if (SCALES)
        for (int i = 1; i < kDist; i++)
            if ((((P - i) % kSBC + kSBC) % kSBC + kDist) % kSBC == 0) n += kScalePerWave;
    return n;
}

// One iteration on stage c (PHASE = c % 4 for K-quants): start the DMA of stage
// c+kDist into dma_st (and, when that stage starts a super-block, its scales
// into other_sc), then compute on `cur` / `cur_scale`.  other_sc is the scale
// buffer of the previous super-block, which half 1 still reads in the first
// stage of the next one (its deferred epilogue) before the buffer is refilled
// in a later iteration.  In every call the buffers written and the buffers read
// are distinct.
template <int KIND, bool SUMS, int PHASE>
__device__ __forceinline__ void step(const GemmArgs& g, const Ctx& x, int c, bool h1, Acc& acc, uint8_t* __restrict__ dma_st,
                                     uint8_t* __restrict__ other_sc, const uint8_t* __restrict__ cur,
                                     const uint8_t* __restrict__ cur_scale)
{
    constexpr int PLANES = KIND == KIND_Q80? 1 : 2;
    if (c + kDist < x.nchunks) {
        issue_stage<KIND>(g,x,c + kDist,dma_st);
        if constexpr (KIND != KIND_Q80 && (PHASE + kDist) % kSBC == 0) issue_scales<KIND>(g,x,(c + kDist) / kSBC,other_sc);
    }
    if constexpr (KIND != KIND_Q80 && PHASE == 0) {
        if (h1 && c > 0) {
            sb_epilogue<KIND,SUMS,0>(g,x,c / kSBC - 1,acc,other_sc);
            sb_epilogue<KIND,SUMS,1>(g,x,c / kSBC - 1,acc,other_sc);
        }
        // The deferred epilogue stays ahead of the MFMAs that restart the
        // integer accumulators.
        __builtin_amdgcn_sched_barrier(0);
    }
    const v16i izero = {};
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int cp = x.lr * 64 + 16 * ((2 * s + x.lg) ^ x.sw);
        v4i a[2], wh[2], wl[2];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const v4i*>(cur + (x.wm * 64 + i * 32) * 64 + cp);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            wh[j] = *reinterpret_cast<const v4i*>(cur + 16 * kSlotW + (x.wn * 64 + j * 32) * 64 + cp);
            if constexpr (PLANES == 2) wl[j] = *reinterpret_cast<const v4i*>(cur + 16 * kSlotW2 + (x.wn * 64 + j * 32) * 64 + cp);
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
                        for (int q4 = 0; q4 < 4; q4++) {
                            const float4 t4 = *reinterpret_cast<const float4*>(sxd + x.wm * 64 + i * 32 + 8 * q4 + 4 * x.lg);
                            const float xq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
                            for (int e = 0; e < 4; e++)
                                acc.y[i][j][4 * q4 + e] = __builtin_fmaf(xq[e],(float)p[4 * q4 + e] * wdv[j],acc.y[i][j][4 * q4 + e]);
                        }
                    }
                }
            }
        } else {
            constexpr bool fresh = PHASE == 0;  // first stage of a super-block: start from zero
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const bool z = fresh && s == 0;
                    acc.hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],z? izero : acc.hi[i][j],0,0,0);
                    acc.lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wl[j],z? izero : acc.lo[i][j],0,0,0);
                }
        }
    }
    if constexpr (KIND != KIND_Q80 && PHASE == kSBC - 1) {
        __builtin_amdgcn_sched_barrier(0);
        if (!h1) {
            sb_epilogue<KIND,SUMS,0>(g,x,c / kSBC,acc,cur_scale);
            sb_epilogue<KIND,SUMS,1>(g,x,c / kSBC,acc,cur_scale);
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
    x.wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    x.lane = threadIdx.x & 63;
    x.wm = x.wave % kWavesM;
    x.wn = x.wave / kWavesM;
    x.lr = x.lane & 31;
    x.lg = x.lane >> 5;
    x.sw = (x.lr >> 2) & 3;  // rows read by this lane are lr + 32k: same swizzle
    x.K = g.K;
    x.nchunks = g.K / kKC;
    {
        // chunk rows start at multiples of 16, so the swizzle of chunk row l/4 is (l/16) & 3
        x.vo_rows = (uint32_t)((x.lane >> 2) * g.K + 16 * ((x.lane & 3) ^ ((x.lane >> 4) & 3)));
        x.vo_lin = 16u * x.lane;
        x.vo_bs = (uint32_t)((x.lane >> 1) * (g.K / 8) + 16 * (x.lane & 1));
        x.vo_wd = KIND == KIND_Q80? 16u * (x.lane & 31) + (x.lane >> 5) * 4u * g.Npad
                                  : 16u * (x.lane & 31) + (x.lane >> 5) * g.wdm_off;
    }
    {
        const size_t mp = (size_t)g.Mpad, np = (size_t)g.Npad, K = (size_t)g.K;
        const size_t nblk = K / (KIND == KIND_Q80? PIX_QK8 : PIX_QK);
        x.rx = make_rsrc(g.xq,mp * K);
        x.rxd = make_rsrc(g.xdT,nblk * mp * 4);
        x.rwh = make_rsrc(g.whi,np * K);
        x.rwl = make_rsrc(KIND == KIND_Q80? g.whi : g.wlo,np * K);
        x.rwd = make_rsrc(g.wdT,KIND == KIND_Q5K? g.wdm_off + nblk * np * 4 : nblk * np * 4);
        x.rxbs = make_rsrc(KIND == KIND_Q5K? (const void*)g.xbs : (const void*)g.xq,KIND == KIND_Q5K? mp * (K / 16) * 2 : 0);
        x.rwmn = make_rsrc(KIND == KIND_Q5K? (const void*)g.wmn : (const void*)g.xq,KIND == KIND_Q5K? nblk * np * 16 : 0);
    }

    Acc acc;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc.hi[i][j] = v16i{};
            acc.lo[i][j] = v16i{};
            acc.y[i][j] = v16f{};
        }

    const int C = x.nchunks;
    const bool h1 = x.wn == 1;
    issue_stage<KIND>(g,x,0,lds);
    if constexpr (SCALES) issue_scales<KIND>(g,x,0,scale_base);
    for (int c = 1; c < kDist; c++)
        if (c < C) issue_stage<KIND>(g,x,c,lds + c * kStageBytes);

    // Stage c has landed once only the DMAs issued in the kDist-1 iterations
    // before c may still be in flight (the prologue counts as iterations
    // -kDist..-1).  The last kDist-1 iterations issue fewer, so they drain.
    // (The integer-sum debug variant also stores inside the loop; stores share
    // vmcnt and may retire early, so it drains everything.)
    auto iter = [&](auto phase, int c) {
        constexpr int P = decltype(phase)::value;
        if (c + kDist - 1 < C && !SUMS) wait_vmcnt<outstanding<SCALES>(P)>();
        else wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        const int b = c / kSBC;
        step<KIND,SUMS,P>(g,x,c,h1,acc,lds + ((c + kDist) % kStages) * kStageBytes,scale_base + ((b + 1) & 1) * kScaleBytes,
                          lds + (c % kStages) * kStageBytes,scale_base + (b & 1) * kScaleBytes);
    };
    if constexpr (KIND == KIND_Q80) {
        for (int c = 0; c < C; c++) iter(std::integral_constant<int,0>{},c);
    } else {
        for (int c = 0; c < C; c += kSBC) {
            iter(std::integral_constant<int,0>{},c);
            iter(std::integral_constant<int,1>{},c + 1);
            iter(std::integral_constant<int,2>{},c + 2);
            iter(std::integral_constant<int,3>{},c + 3);
        }
        if (h1) {  // half 1's deferred epilogue of the last super-block
            const int b = C / kSBC - 1;
            sb_epilogue<KIND,SUMS,0>(g,x,b,acc,scale_base + (b & 1) * kScaleBytes);
            sb_epilogue<KIND,SUMS,1>(g,x,b,acc,scale_base + (b & 1) * kScaleBytes);
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
    if (KIND != KIND_Q80 && g.K % PIX_QK) return hipErrorInvalidValue;
    // Buffer offsets are 32-bit: every operand plane must stay below 2 GiB.
    const size_t lim = (size_t)1 << 31;
    const size_t scales = (KIND == KIND_Q5K? 2 : 1) * ((size_t)g.K / (KIND == KIND_Q80? PIX_QK8 : PIX_QK)) * (npad > mpad? npad : mpad) * 4;
    if (mpad * g.K >= lim || npad * g.K >= lim || scales >= lim || mpad * (g.K / 16) * 2 >= lim) return hipErrorInvalidValue;
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

// The Q5_K dmin plane must follow d in the same allocation (one buffer
// resource covers both).
static bool q5_dm_offset(const PlanesQ5K& w, size_t K, uint32_t* off)
{
    const ptrdiff_t d = reinterpret_cast<const char*>(w.dm) - reinterpret_cast<const char*>(w.d);
    if (d < (ptrdiff_t)((K / PIX_QK) * w.npad * 4) || d >= ((ptrdiff_t)1 << 30)) return false;
    *off = (uint32_t)d;
    return true;
}

hipError_t launch_gemm_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    if (!q5_dm_offset(w,K,&g.wdm_off)) return hipErrorInvalidValue;
    g.xq = a.qs; g.xdT = a.d; g.xbs = a.bs;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wmn = w.mn;
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
    if (!q5_dm_offset(w,K,&g.wdm_off)) return hipErrorInvalidValue;
    g.xq = a.qs; g.xdT = a.d; g.xbs = a.bs;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wmn = w.mn;
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
