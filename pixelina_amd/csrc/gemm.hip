// Quantized GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for
// Q5_K / Q6_K / Q8_0 weights and Q8_K / Q8_0 activations.  The counterpart of
// pix_dot_q5_K / pix_dot_q6_K / pix_dot_q8_0 driven by cpu_quant_matmul
// (src/kernels_quant.cpp:163-365, :369-412) and of shaders/matmul_mmq.comp.
//
// Tiling: a workgroup of 16 waves (4 along tokens x 4 along features) owns a
// 256x128 output tile; each wave owns 64x32 = two v_mfma_i32_32x32x32_i8 tiles
// stacked along tokens (A = activations, rows = tokens; B = weights, columns =
// output features: each lane holds one feature column and 16 token rows of a
// 32x32 accumulator).  One workgroup fills a CU at four waves per SIMD, so
// while some waves wait on LDS or a barrier, or run their fp32 epilogue on the
// vector ALU, others keep the matrix cores busy.
//
// Staggered epilogues: waves with an even feature index apply a super-block's
// fp32 epilogue at the end of its last stage, odd ones at the start of the next
// super-block's first stage.  The four waves of a SIMD (w, w+4, w+8, w+12) are
// two of each kind, so each epilogue's vector ALU work overlaps MFMAs.
//
// Data movement: K advances in 64-byte stages (two 32-value sub-blocks),
// loaded with buffer_load_dwordx4 ... lds (HBM -> LDS, no registers).  Lane l
// of a DMA lands at LDS base + 16*l; the source is a buffer resource (SGPRs) +
// a per-lane offset (VGPR) + a wave-uniform offset (SGPR).  Four consecutive
// lanes fetch one 64-byte row (coalesced), and each lane picks its piece so
// that the ring holds rows of four 16-byte pieces with piece c of row r at slot
// 4r + (c ^ ((r>>2) & 3)): the MFMA operand reads (ds_read_b128, lane l reads
// row l%32, piece 2s + l/32) are then free of LDS bank conflicts on gfx950.
// Per 256-value super-block the scale data rides in small LDS regions loaded
// the same way.  Synchronisation is explicit: s_waitcnt vmcnt for this wave's
// DMAs, then s_barrier (no fence, which would drain every in-flight stage).
// Every wave issues the same number of DMAs per stage (the vmcnt waits count
// them); waves with nothing to load issue a DMA through an empty buffer
// resource, which reads nothing and writes zeros into a discard chunk.
//
// Exactness: the MFMAs produce, per (token, feature, super-block), the exact
// integers the reference forms before its fp32 epilogue:
//   Q5_K  S = sum_s scale_s*dot_s   from the hi/lo planes (64*hi + lo)
//   Q6_K  S = sum_e scale*(q-32)*q8 from the hi/lo planes
//   Q8_0  P = sum over the 32-value block of q*q8
// then y += yd*(wd*S) per super-block (Q5_K, Q6_K), y += xd*(wd*P) per block
// (Q8_0), in fp32.  The Q5_K minimum term Mn = sum_s min_s*(bsum_2s + bsum_2s+1)
// is one fp16 MFMA per tile and super-block on the 16-value activation sums and
// the six-bit minima (inputs exact in fp16: min <= 63, |bsum16| <= 2032;
// |Mn| < 2^24, so the fp32 result is exact), and the epilogue becomes
// y += yd*(wd*S - wdmin*Mn).
#include <algorithm>
#include <type_traits>

#include "pixhip_device.h"
#include "pixhip_internal.h"

#define PIX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace pixhip {

constexpr int kBM = PIX_GEMM_MTILE, kBN = PIX_GEMM_NTILE, kKC = 64;
constexpr int kWavesM = 4, kWavesN = 4, kWaves = kWavesM * kWavesN, kThreads = 64 * kWaves;
constexpr int kWN = kBN / kWavesN;  // features per wave: one 32-column MFMA tile
constexpr int kStages = 4;         // ring depth: one stage read, kDist in flight
constexpr int kDist = kStages - 1; // prefetch distance in stages
constexpr int kChunk = 1024;       // bytes written by one DMA instruction (64 lanes x 16 B)
constexpr int kStageBytes = 32768;
constexpr int kStageChunks = kStageBytes / kChunk;  // 32: 2 per wave
constexpr int kPerWave = kStageChunks / kWaves;
constexpr int kSBC = PIX_QK / kKC;                  // stages per super-block (4)
static_assert(kWavesM * 64 == kBM && kWavesN * kWN == kBN && kWN == 32, "wave grid covers the tile");
static_assert(kPerWave * kWaves == kStageChunks, "stage DMAs split evenly over the waves");

enum Kind { KIND_Q5K = 0, KIND_Q6K = 1, KIND_Q80 = 2 };

// Ring layout: the activation halves of the four stages are contiguous
// (A ring, 4 x 16 KB from LDS 0), then the weight halves (W ring, 4 x 16 KB from
// 64 KB), so that every operand read is a per-lane base register plus an
// immediate offset below 64 KB.  Within a W slot (16-B slots):
//   K-quants  W.hi 0..511 | W.lo 512..1023
//   Q8_0      W 0..511 | xd[2][256] 512..639 | wd[2][128] 640..703 | unused
constexpr int kHalfBytes = kStageBytes / 2, kWRing = kStages * kHalfBytes;
constexpr int kSlotW2 = 512, kSlotXd80 = 512, kSlotWd80 = 640;

// Per-super-block scale region, double buffered (slots of 16 B; DMA chunk c
// fills slots 64c..64c+63):
//   yd[256] 0..63 | wd[128] 64..95                                  (Q6_K, 2 KB)
//   Q5_K adds the minimum-term inputs: bs[256][2] 128..639 (16-value sums) |
//   mn[128] 640..767 (minima) | wdm[128] 768..799 (dmin)            (13 KB)
constexpr int kSlotYd = 0, kSlotWd = 64, kSlotBs = 128, kSlotMn = 640, kSlotWdm = 768;
template <int KIND> constexpr int scale_chunks() { return KIND == KIND_Q80? 0 : (KIND == KIND_Q5K? 13 : 2); }
constexpr int kScalePerWave = 1;  // every wave issues one scale DMA per super-block (real or discard)

typedef __amdgpu_buffer_rsrc_t Rsrc;

struct GemmArgs {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/QK][Mpad]  (QK = 256, or 32 for Q8_0)
    const _Float16* xbs;  // [Mpad][K/16]  (Q5_K)
    const int8_t* whi;    // [Npad][K] (Q8_0: the quantized plane)
    const int8_t* wlo;    // [Npad][K]
    const float* wdT;     // [K/QK][Npad]
    const float* wdm;     // [K/256][Npad] dmin (Q5_K)
    const _Float16* wmn;  // [K/256][Npad][8] minima (Q5_K)
    float* y;
    const float* bias;
    int32_t* sums;        // debug: exact integer sums [M][N][blocks]
    int32_t* mins;
    int M, N, K, Mpad, Npad;
    size_t ldy, yoff;
    int tiles_m, tiles_n;
    // Split-K of the last tiles: tiles full_tiles.. (in tile order) run as
    // `splits` K ranges of split_chunks stages each, writing fp32 partials
    // part[split][tile - full_tiles][kBM][kBN] that splitk_reduce_kernel sums.
    int full_tiles, splits, split_chunks;
    float* part;
};

// Tile order: GROUP token tiles share one feature tile, in launch order
// (steady-state A/B at 4096 x 3840 x 10240, quantize + GEMM: GROUP 4 ~390 us,
// 8 ~394, 2 ~396, 16 ~399, 1 ~403).
__device__ __forceinline__ void tile_of(int lid, int tiles_m, int tiles_n, int& tm, int& tn)
{
    constexpr int GROUP = 4;
    const int group = lid / (GROUP * tiles_n);
    const int first_m = group * GROUP;
    const int gsize = min(tiles_m - first_m,GROUP);
    const int within = lid % (GROUP * tiles_n);
    tm = first_m + within % gsize;
    tn = within / gsize;
}

struct Ctx {
    int m0, n0, wave, wm, wn, K;
    int c_begin, nchunks;  // this workgroup's stages: c_begin .. nchunks-1
    uint32_t oa, ow;  // per-lane LDS byte offsets of this wave's operand rows in a stage (k-step 0)
    uint32_t vo_rows; // per-lane DMA source offset of a 64-B row piece
    int ocol, oyd;    // this lane's feature column in the tile; first of its token rows in the wave
    Rsrc rx, rxd, rxbs, rwh, rwl, rwd, rwdm, rwmn, rnull;
};

struct Acc {
    v16i hi[2], lo[2];
    v16f y[2];
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
    // Raw buffer, stride 0: offsets at or beyond `bytes` read as zero.  A null
    // base gets an empty range, so a missing plane reads zeros, never address 0.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base),(short)0,base? (int)bytes : 0,0x00020000);
}

__device__ __forceinline__ void dma(Rsrc r, uint8_t* lds_uniform, uint32_t voff, uint32_t soff)
{
    __builtin_assume(lds_uniform != nullptr);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,PIX_LDS(lds_uniform),16,(int)voff,(int)soff,0,0);
}

// The lane index, recomputed where it is used (volatile, so the compiler
// cannot keep derived per-lane offsets live across the loop: the DMAs need
// them once per stage, the MFMA loop needs the registers).
__device__ __forceinline__ uint32_t lane_now()
{
    uint32_t l;
    __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// A DMA that loads nothing (empty resource) into the discard chunk, so that
// every wave issues the same number of DMAs.
__device__ __forceinline__ void null_dma(const Ctx& x, uint8_t* discard) { dma(x.rnull,discard,0,0); }

// Bijective XCD-aware remap: hardware places workgroup b on XCD b % 8; give
// each XCD a contiguous range of logical tiles so its L2 sees neighbours.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd < r? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// DMA of stage c into `st`: chunk wave + 16*q of the 32 is this wave's q-th.
// Chunks 0..15 are activation rows (16 rows of 64 B each), 16..23 the first
// weight plane, 24..31 the second (Q8_0: 24, 25 activation scales of blocks
// 2c, 2c+1; 26 weight scales of both blocks; 27..31 nothing).  Lane l fetches
// chunk row l/4, piece (l%4) ^ ((l/16) & 3).
template <int KIND>
__device__ __forceinline__ void issue_stage(const GemmArgs& g, const Ctx& x, int c, uint8_t* sa, uint8_t* sw, uint8_t* discard)
{
    const uint32_t k0 = (uint32_t)c * kKC;
    uint32_t vo_rows = x.vo_rows;
    if constexpr (KIND == KIND_Q5K) {
        // recomputed (Q5_K has no register to keep it in)
        const uint32_t lane = lane_now();
        vo_rows = (lane >> 2) * (uint32_t)x.K + 16u * ((lane & 3) ^ ((lane >> 4) & 3));
    }
#pragma unroll
    for (int q = 0; q < kPerWave; q++) {
        const int chunk = x.wave + kWaves * q;  // wave-uniform
        uint8_t* dst = chunk < 16? sa + chunk * kChunk : sw + (chunk - 16) * kChunk;
        if (chunk < 16) {
            dma(x.rx,dst,vo_rows,(uint32_t)(x.m0 + chunk * 16) * x.K + k0);
        } else if (chunk < 24 || KIND != KIND_Q80) {
            const int row0 = (chunk - (chunk < 24? 16 : 24)) * 16;
            dma(chunk < 24? x.rwh : x.rwl,dst,vo_rows,(uint32_t)(x.n0 + row0) * x.K + k0);
        } else if (chunk < 26) {
            const uint32_t lane = lane_now();
            dma(x.rxd,dst,16u * lane,(uint32_t)((2 * c + chunk - 24) * g.Mpad + x.m0) * 4u);
        } else if (chunk == 26) {
            // lanes 0..31: block 2c, lanes 32..63: block 2c+1 (128 features each)
            const uint32_t lane = lane_now();
            dma(x.rwd,dst,16u * (lane & 31) + (lane >> 5) * 4u * (uint32_t)g.Npad,(uint32_t)(2 * c * g.Npad + x.n0) * 4u);
        } else {
            null_dma(x,discard);
        }
    }
}

// DMA of super-block b's scale data into `sc` (one DMA per wave): chunk 0 yd,
// chunk 1 wd (lanes 0..31); the Q5_K integer-sum variant also loads chunks
// 2..9 bs and 10..11 mn.
template <int KIND>
__device__ __forceinline__ void issue_scales(const GemmArgs& g, const Ctx& x, int b, uint8_t* sc, uint8_t* discard)
{
    const uint32_t lane = lane_now();
    const int chunk = x.wave;
    uint8_t* dst = sc + chunk * kChunk;
    if (chunk == 0) {
        dma(x.rxd,dst,16u * lane,(uint32_t)(b * g.Mpad + x.m0) * 4u);
    } else if (chunk == 1) {
        dma(x.rwd,dst,16u * (lane & 31),(uint32_t)(b * g.Npad + x.n0) * 4u);  // lanes 32..63 repeat 0..31
    } else if (KIND == KIND_Q5K && chunk == 12) {
        dma(x.rwdm,dst,16u * (lane & 31),(uint32_t)(b * g.Npad + x.n0) * 4u);
    } else if (KIND == KIND_Q5K && chunk < 10) {
        // 32 rows of 16 fp16 sums: two lanes per row
        dma(x.rxbs,dst,(lane >> 1) * (uint32_t)(x.K / 8) + 16u * (lane & 1),
            ((uint32_t)(x.m0 + (chunk - 2) * 32) * (x.K / 16) + b * 16) * 2u);
    } else if (KIND == KIND_Q5K && chunk < 12) {
        dma(x.rwmn,dst,16u * lane,(uint32_t)(b * g.Npad + x.n0 + (chunk - 10) * 64) * 16u);
    } else {
        null_dma(x,discard);
    }
}

// Mn of row tile I for the super-block whose scales are in `sc`:
// sum_s min_s*(bsum_2s + bsum_2s+1) as one fp16 MFMA (exact, see above).
template <int I>
__device__ __forceinline__ v16f min_term_exact(const Ctx& x, int col, const uint8_t* __restrict__ sc)
{
    const uint32_t ln = lane_now();
    const v16f fzero = {};
    const v8h mnB = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotMn + col));
    const v8h bsA = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotBs + 2 * (x.wm * 64 + I * 32 + (int)(ln & 31)) + (int)(ln >> 5)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA,mnB,fzero,0,0,0);
}

// fp32 epilogue of row tile I for super-block b: y += yd*(wd*S - wdm*Mn) (the
// integer-sum debug variant stores S, and Mn for Q5_K, instead).  Q5_K keeps
// no per-lane offsets in registers (it has none to spare): it recomputes them.
template <int KIND, bool SUMS, int I>
__device__ __forceinline__ void sb_epilogue(const GemmArgs& g, const Ctx& x, int b, Acc& acc, const uint8_t* __restrict__ sc)
{
    const uint32_t ln = SUMS || KIND == KIND_Q5K? lane_now() : 0u;
    const int lg = (int)(ln >> 5);
    const int col = KIND == KIND_Q5K? x.wn * kWN + (int)(ln & 31) : x.ocol;
    const int oyd = KIND == KIND_Q5K? x.wm * 64 + 4 * lg : x.oyd;
    if constexpr (SUMS) {
        const v16f mt = KIND == KIND_Q5K? min_term_exact<I>(x,col,sc) : v16f{};
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = x.m0 + x.wm * 64 + I * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            const int n = x.n0 + col;
            if (m < g.M && n < g.N) {
                const size_t o = ((size_t)m * g.N + n) * (x.K / PIX_QK) + b;
                g.sums[o] = acc.hi[I][r] * 64 + acc.lo[I][r];
                if constexpr (KIND == KIND_Q5K) g.mins[o] = (int32_t)mt[r];
            }
        }
    } else {
        __asm__ volatile("" ::: "memory");
        const float* syd = reinterpret_cast<const float*>(sc + 16 * kSlotYd);
        const float wd = reinterpret_cast<const float*>(sc + 16 * kSlotWd)[col];
        if constexpr (KIND == KIND_Q5K) {
            // S*wd first, so the integer accumulators of this tile are dead
            // before the minimum-term MFMA result needs registers.
            v16f t;
#pragma unroll
            for (int r = 0; r < 16; r++) t[r] = (float)(acc.hi[I][r] * 64 + acc.lo[I][r]) * wd;
            __asm__ volatile("" ::: "memory");
            const float nwm = -reinterpret_cast<const float*>(sc + 16 * kSlotWdm)[col];
            const v16f mt = min_term_exact<I>(x,col,sc);
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const float4 t4 = *reinterpret_cast<const float4*>(syd + oyd + I * 32 + 8 * q4);
                const float yq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q4 + e;
                    acc.y[I][r] = __builtin_fmaf(yq[e],__builtin_fmaf(mt[r],nwm,t[r]),acc.y[I][r]);
                }
            }
            return;
        }
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const float4 t4 = *reinterpret_cast<const float4*>(syd + oyd + I * 32 + 8 * q4);
            const float yq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * q4 + e;
                acc.y[I][r] = __builtin_fmaf(yq[e],(float)(acc.hi[I][r] * 64 + acc.lo[I][r]) * wd,acc.y[I][r]);
            }
        }
    }
}

// DMA instructions a wave may still have in flight when the stage of phase P
// must have landed: those of the kDist-1 iterations before it.  Iteration p
// issues kPerWave stage DMAs, plus the scales of the next super-block when p
// is kSBC - kDist (mod kSBC).
template <int KIND> constexpr int issued(int p)
{
    p = ((p % kSBC) + kSBC) % kSBC;
    return kPerWave + (KIND != KIND_Q80 && (p + kDist) % kSBC == 0? kScalePerWave : 0);
}
template <int KIND> constexpr int outstanding(int P)
{
    if (KIND == KIND_Q80) return (kDist - 1) * kPerWave;
    int n = 0;
    for (int i = 1; i < kDist; i++) n += issued<KIND>(P - i);
    return n;
}

// One iteration on stage c (PHASE = c % 4 for K-quants): compute on the A slot
// `cur` (the W slot is at a fixed distance, folded into the lane's W offset)
// and `cur_scale`, and, after the first of its two k-steps, start the DMA of
// stage c+kDist into its A and W slots (and, when that stage starts a
// super-block, its scales into other_sc).
// other_sc is the scale buffer of the previous super-block, which odd waves
// still read in the first stage of the next one (their deferred epilogue)
// before it is refilled in a later iteration.  In every call the buffers
// written and the buffers read are distinct.
template <int KIND, bool SUMS, int PHASE, bool DEFERRED = true>
__device__ __forceinline__ void step(const GemmArgs& g, const Ctx& x, int c, bool h1, Acc& acc, uint8_t* __restrict__ dma_a,
                                     uint8_t* __restrict__ dma_w, uint8_t* __restrict__ other_sc, uint8_t* __restrict__ discard,
                                     const uint8_t* __restrict__ cur, const uint8_t* __restrict__ cur_scale)
{
    constexpr int PLANES = KIND == KIND_Q80? 1 : 2;
    if constexpr (KIND != KIND_Q80 && PHASE == 0) {
        // (DEFERRED is false in a workgroup's first super-block: nothing before it.)
        if (DEFERRED && h1) {
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
        const uint32_t oa = x.oa ^ (32u * s), ow = x.ow ^ (32u * s);
        v4i a[2], wh, wl;
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const v4i*>(cur + oa + i * 2048);
        wh = *reinterpret_cast<const v4i*>(cur + ow);
        if constexpr (PLANES == 2) wl = *reinterpret_cast<const v4i*>(cur + 16 * kSlotW2 + ow);
        if constexpr (KIND == KIND_Q80) {
            // One 32-value block per sub-block: fresh accumulator, fp32 epilogue.
            const uint8_t* cur_w = cur + kWRing;
            const float* sxd = reinterpret_cast<const float*>(cur_w + 16 * kSlotXd80) + s * kBM;
            const float wdv = (reinterpret_cast<const float*>(cur_w + 16 * kSlotWd80) + s * kBN)[x.ocol];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh,izero,0,0,0);
                if constexpr (SUMS) {
                    const uint32_t ln = lane_now();
                    const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
                    const int kb = c * 2 + s;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = x.m0 + x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                        const int n = x.n0 + x.wn * kWN + lr;
                        if (m < g.M && n < g.N) g.sums[((size_t)m * g.N + n) * (x.K / PIX_QK8) + kb] = p[r];
                    }
                } else {
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const float4 t4 = *reinterpret_cast<const float4*>(sxd + x.oyd + i * 32 + 8 * q4);
                        const float xq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc.y[i][4 * q4 + e] = __builtin_fmaf(xq[e],(float)p[4 * q4 + e] * wdv,acc.y[i][4 * q4 + e]);
                    }
                }
            }
        } else {
            constexpr bool fresh = PHASE == 0;  // first stage of a super-block: start from zero
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const bool z = fresh && s == 0;
                acc.hi[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh,z? izero : acc.hi[i],0,0,0);
                acc.lo[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wl,z? izero : acc.lo[i],0,0,0);
            }
        }
        if (s == 0) {
            // The DMAs go out after the first k-step's MFMAs rather than right
            // after the barrier: issued there by all 16 waves at once they fill
            // the address unit's queue, and each wave's issue stalls until its
            // DMAs are accepted (measured ~480 cycles per stage); issued here,
            // each wave already has MFMAs in flight while it waits.
            __builtin_amdgcn_sched_barrier(0);
            if (c + kDist < x.nchunks) {
                issue_stage<KIND>(g,x,c + kDist,dma_a,dma_w,discard);
                if constexpr (KIND != KIND_Q80 && (PHASE + kDist) % kSBC == 0)
                    issue_scales<KIND>(g,x,(c + kDist) / kSBC,other_sc,discard);
            }
            __builtin_amdgcn_sched_barrier(0);
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
    constexpr int kScaleBytes = scale_chunks<KIND>() * kChunk;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes + 2 * kScaleBytes + kChunk];
    uint8_t* const scale_base = lds + kStages * kStageBytes;  // after the A and W rings
    uint8_t* const discard = scale_base + 2 * kScaleBytes;

    // Whole tiles first (XCD-remapped), then the split tiles' pieces in launch
    // order (consecutive pieces land on different XCDs, so the last round
    // spreads over the whole device).
    const int ntiles = g.tiles_m * g.tiles_n;
    const int bid = (int)blockIdx.x;
    const bool piece = bid >= g.full_tiles;
    const int split_tiles = ntiles - g.full_tiles;
    const int pidx = bid - g.full_tiles;
    const int split = piece? pidx / split_tiles : 0;
    const int lid = piece? g.full_tiles + pidx % split_tiles : xcd_remap(bid,g.full_tiles);
    int tm, tn;
    tile_of(lid,g.tiles_m,g.tiles_n,tm,tn);

    Ctx x;
    x.m0 = tm * kBM;
    x.n0 = tn * kBN;
    x.wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    x.wm = x.wave % kWavesM;
    x.wn = x.wave / kWavesM;
    {
        // lane l reads row l%32, piece (l/32) ^ ((l%32 >> 2) & 3) of k-step 0; k-step 1 is that ^ 2
        const int lr = (int)(threadIdx.x & 31), lg = (int)((threadIdx.x >> 5) & 1);
        const uint32_t cp0 = (uint32_t)(lr * 64 + 16 * (lg ^ ((lr >> 2) & 3)));
        x.oa = (uint32_t)(x.wm * 64 * 64) + cp0;
        x.ow = (uint32_t)(kWRing + x.wn * kWN * 64) + cp0;  // relative to the A slot of the same stage
        const uint32_t lane = threadIdx.x & 63;
        x.vo_rows = (lane >> 2) * (uint32_t)g.K + 16u * ((lane & 3) ^ ((lane >> 4) & 3));
        x.ocol = x.wn * kWN + lr;
        x.oyd = x.wm * 64 + 4 * lg;
    }
    x.K = g.K;
    x.c_begin = piece? split * g.split_chunks : 0;
    x.nchunks = piece? min(x.c_begin + g.split_chunks,g.K / kKC) : g.K / kKC;
    {
        const size_t mp = (size_t)g.Mpad, np = (size_t)g.Npad, K = (size_t)g.K;
        const size_t nblk = K / (KIND == KIND_Q80? PIX_QK8 : PIX_QK);
        constexpr bool Q5 = KIND == KIND_Q5K;
        x.rx = make_rsrc(g.xq,mp * K);
        x.rxd = make_rsrc(g.xdT,nblk * mp * 4);
        x.rwh = make_rsrc(g.whi,np * K);
        x.rwl = make_rsrc(KIND == KIND_Q80? g.whi : g.wlo,np * K);
        x.rwd = make_rsrc(g.wdT,nblk * np * 4);
        x.rxbs = make_rsrc(Q5? (const void*)g.xbs : (const void*)g.xq,Q5? mp * (K / 16) * 2 : 0);
        x.rwmn = make_rsrc(Q5? (const void*)g.wmn : (const void*)g.xq,Q5? nblk * np * 16 : 0);
        x.rwdm = make_rsrc(Q5? (const void*)g.wdm : (const void*)g.xq,Q5? nblk * np * 4 : 0);
        x.rnull = make_rsrc(g.xq,0);
    }

    Acc acc;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        acc.hi[i] = v16i{};
        acc.lo[i] = v16i{};
        acc.y[i] = v16f{};
    }

    const int C0 = x.c_begin, C = x.nchunks;  // C0 starts a super-block (a multiple of kSBC)
    const bool h1 = (x.wn & 1) != 0;
    issue_stage<KIND>(g,x,C0,lds + (C0 % kStages) * kHalfBytes,lds + kWRing + (C0 % kStages) * kHalfBytes,discard);
    if constexpr (SCALES) issue_scales<KIND>(g,x,C0 / kSBC,scale_base + ((C0 / kSBC) & 1) * kScaleBytes,discard);
    for (int c = C0 + 1; c < C0 + kDist; c++)
        if (c < C) issue_stage<KIND>(g,x,c,lds + (c % kStages) * kHalfBytes,lds + kWRing + (c % kStages) * kHalfBytes,discard);

    // Stage c has landed once only the DMAs issued in the kDist-1 iterations
    // before c may still be in flight (the prologue counts as iterations
    // -kDist..-1).  The last kDist-1 iterations issue fewer, so they drain.
    // (The integer-sum debug variant also stores inside the loop; stores share
    // vmcnt and may retire early, so it drains everything.)
    auto iter = [&](auto phase, int c, auto deferred) {
        constexpr int P = decltype(phase)::value;
        constexpr bool DEFERRED = decltype(deferred)::value;
        if (c + kDist - 1 < C && !SUMS) wait_vmcnt<outstanding<KIND>(P)>();
        else wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        const int b = c / kSBC;
        const int sd = (c + kDist) % kStages, sc = c % kStages;
        step<KIND,SUMS,P,DEFERRED>(g,x,c,h1,acc,lds + sd * kHalfBytes,lds + kWRing + sd * kHalfBytes,scale_base + ((b + 1) & 1) * kScaleBytes,
                          discard,lds + sc * kHalfBytes,scale_base + (b & 1) * kScaleBytes);
    };
    if constexpr (KIND == KIND_Q80) {
        for (int c = C0; c < C; c++) iter(std::integral_constant<int,0>{},c,std::true_type{});
    } else {
        // The first super-block is peeled (no deferred epilogue before it); the
        // rest are counted in super-blocks, so that c % kStages is known in
        // every iteration.
        auto super_block = [&](int c, auto deferred) {
            iter(std::integral_constant<int,0>{},c,deferred);
            iter(std::integral_constant<int,1>{},c + 1,deferred);
            iter(std::integral_constant<int,2>{},c + 2,deferred);
            iter(std::integral_constant<int,3>{},c + 3,deferred);
        };
        super_block(C0,std::false_type{});
        for (int sb = C0 / kSBC + 1; sb < C / kSBC; sb++) super_block(sb * kSBC,std::true_type{});
        if (h1) {  // deferred epilogue of the last super-block
            const int b = C / kSBC - 1;
            sb_epilogue<KIND,SUMS,0>(g,x,b,acc,scale_base + (b & 1) * kScaleBytes);
            sb_epilogue<KIND,SUMS,1>(g,x,b,acc,scale_base + (b & 1) * kScaleBytes);
        }
    }

    if (!SUMS && (int)blockIdx.x >= g.full_tiles) {
        // Split-K: this K range's fp32 partial tile; splitk_reduce_kernel adds
        // the ranges in order and applies bias, ldy and offset.  (The piece
        // index is recomputed here rather than kept live through the loop.)
        const int p = (int)blockIdx.x - g.full_tiles, nsplit = g.tiles_m * g.tiles_n - g.full_tiles;
        const uint32_t ln = lane_now();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
        float* col = g.part + ((size_t)(p / nsplit) * nsplit + p % nsplit) * (kBM * kBN) + x.wn * kWN + lr;
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int lm = x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                col[(size_t)lm * kBN] = acc.y[i][r];
            }
        }
    } else if constexpr (!SUMS) {
        // Bias for this lane's column, loaded once (clamped index) and drained
        // before the stores: a load left pending here would make every store
        // below wait for all earlier stores.  The output is stored
        // non-temporally: written once and not read here, it would otherwise
        // push the weights and activations out of the last-level cache
        // (measured: quantize + GEMM 403 -> 392 us at the DiT FFN shape).
        const uint32_t ln = lane_now();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
        const int mrow0 = x.m0 + x.wm * 64, ncol0 = x.n0 + x.wn * kWN;
        const float bv = g.bias? g.bias[min(ncol0 + lr,g.N - 1)] : 0.0f;
        wait_vmcnt<0>();
        const bool full = mrow0 + 64 <= g.M && ncol0 + kWN <= g.N;
        const int n = ncol0 + lr;
        float* col = g.y + g.yoff + n;
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = mrow0 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                if (full || (m < g.M && n < g.N)) __builtin_nontemporal_store(acc.y[i][r] + bv,col + (size_t)m * g.ldy);
            }
        }
    }
}

static size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// For the split tiles: y[yoff + m*ldy + n] = sum over the splits, in order, of
// the partial tiles, + bias[n].  Workgroup (tile t, slice q) of 256 threads
// covers kReduceSlice elements of the tile, 4 consecutive features per thread.
constexpr int kReduceSlice = 1024, kReduceSlices = kBM * kBN / kReduceSlice;
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g)
{
    const int split_tiles = g.tiles_m * g.tiles_n - g.full_tiles;
    const int t = (int)blockIdx.x / kReduceSlices, q = (int)blockIdx.x % kReduceSlices;
    int tm, tn;
    tile_of(g.full_tiles + t,g.tiles_m,g.tiles_n,tm,tn);
    const size_t stride = (size_t)split_tiles * (kBM * kBN);
    const int e = q * kReduceSlice + 4 * (int)threadIdx.x;
    const float4* src = reinterpret_cast<const float4*>(g.part + (size_t)t * (kBM * kBN) + e);
    float4 v = src[0];
    for (int s = 1; s < g.splits; s++) {
        const float4 w = src[(size_t)s * stride / 4];
        v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
    }
    const int m = tm * kBM + e / kBN, n0 = tn * kBN + e % kBN;
    if (m >= g.M) return;
    const float vv[4] = {v.x,v.y,v.z,v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + j;
        if (n < g.N) g.y[g.yoff + (size_t)m * g.ldy + n] = vv[j] + (g.bias? g.bias[n] : 0.0f);
    }
}

static int device_cus()
{
    static int cus = 0;
    if (!cus) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v,hipDeviceAttributeMultiprocessorCount,dev) == hipSuccess && v > 0)
            cus = v;
        else
            cus = 256;
    }
    return cus;
}

// One workgroup fills a CU, so the tiles run in rounds of `CUs` workgroups.
// When the last round would fill less than half of the device, its tiles are
// split-K: each tile's K range is cut (at super-block boundaries) into up to
// CUs/tiles-in-the-round pieces, run by separate workgroups.  Returns the
// number of pieces (1: no split) and sets the whole tiles and the piece
// length in stages.
int gemm_split_plan(size_t M, size_t N, size_t K, int& full_tiles, int& split_chunks)
{
    const size_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    const int chunks = (int)(K / kKC), groups = chunks / kSBC;
    const size_t cus = (size_t)device_cus();
    full_tiles = (int)tiles;
    split_chunks = chunks;
    if (!tiles || groups < 2) return 1;
    const size_t tail = tiles - (tiles - 1) / cus * cus;  // tiles of the last round
    if (tail * 2 > cus) return 1;
    const int want = std::min<int>((int)(cus / tail),groups);
    if (want < 2) return 1;
    full_tiles = (int)(tiles - tail);
    split_chunks = (groups + want - 1) / want * kSBC;
    return (chunks + split_chunks - 1) / split_chunks;
}

size_t gemm_split_bytes(size_t M, size_t N, size_t K_stages)
{
    int full, chunks;
    const int splits = gemm_split_plan(M,N,K_stages,full,chunks);
    const size_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    return splits > 1? (size_t)splits * (tiles - full) * (kBM * kBN) * sizeof(float) : 0;
}

template <int KIND, bool SUMS>
static hipError_t launch(GemmArgs g, size_t mpad, size_t npad, hipStream_t s)
{
    g.tiles_m = (int)((g.M + kBM - 1) / kBM);
    g.tiles_n = (int)((g.N + kBN - 1) / kBN);
    if (mpad < round_up((size_t)g.M,kBM) || npad < round_up((size_t)g.N,kBN) || g.K % kKC) return hipErrorInvalidValue;
    if (KIND != KIND_Q80 && g.K % PIX_QK) return hipErrorInvalidValue;
    // Buffer offsets are 32-bit: every operand plane must stay below 2 GiB.
    const size_t lim = (size_t)1 << 31;
    const size_t scales = ((size_t)g.K / (KIND == KIND_Q80? PIX_QK8 : PIX_QK)) * (npad > mpad? npad : mpad) * 16;
    if (mpad * g.K >= lim || npad * g.K >= lim || scales >= lim || mpad * (g.K / 16) * 2 >= lim) return hipErrorInvalidValue;
    g.Mpad = (int)mpad;
    g.Npad = (int)npad;
    const int ntiles = g.tiles_m * g.tiles_n;
    if (!ntiles) return hipSuccess;
    g.splits = SUMS? 1 : gemm_split_plan((size_t)g.M,(size_t)g.N,(size_t)g.K,g.full_tiles,g.split_chunks);
    if (g.splits == 1 || !g.part) {  // unsplit (or no workspace)
        g.splits = 1;
        g.full_tiles = ntiles;
        g.split_chunks = g.K / kKC;
    }
    const int split_tiles = ntiles - g.full_tiles;
    gemm_kernel<KIND,SUMS><<<dim3(g.full_tiles + split_tiles * g.splits),dim3(kThreads),0,s>>>(g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !split_tiles) return e;
    static_assert(kReduceSlice == 4 * 256, "reduce slice: 256 threads x 4 features");
    splitk_reduce_kernel<<<dim3(split_tiles * kReduceSlices),dim3(256),0,s>>>(g);
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

hipError_t launch_gemm_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.part = part;
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.qs; g.wdT = w.dT;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q80,false>(g,a.mpad,round_up(N,kBN),s);
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
