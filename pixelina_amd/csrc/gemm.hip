// Q8_0 GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for Q8_0
// weights with Q8_0 activations -- the counterpart of pix_dot_q8_0 driven by
// cpu_quant_matmul (src/kernels_quant.cpp:339-365, :369-412) and of
// shaders/matmul_mmq.comp's Q8_0 path.  (The K-quant GEMM is gemm_kq.hip;
// this file also holds the split-K plan both use.)
//
// Numerics: per 32-value block, one v_mfma_i32_32x32x32_i8 gives the exact
// integer P = sum q * q8 of the reference; then y += (xd * wd) * P in fp32.
// The scale products xd[row] * wd[col] of a 32 x 32 tile come from one fp16
// MFMA outer product (v_mfma_f32_32x32x8_f16 with xd and wd in K slot 0, the
// other slots zero): both scales are fp16 values, so every product is exact in
// fp32, and the vector ALU is left with one convert and one FMA per element
// and block.  That epilogue, not the matrix core, bounds this kernel: per
// block a wave runs 2 i8 and 2 fp16 MFMAs (96 cycles) and 64 vector
// instructions (256 cycles).
//
// Tiling: a workgroup of 16 waves (4 per SIMD) owns a 256 (tokens) x 128
// (features) tile; wave w owns the 64 x 32 block at tokens 64*(w%4), features
// 32*(w/4): two token tiles of 32 x 32.
//
// Data movement: K advances in 64-value stages (two blocks), loaded with
// buffer_load_dwordx4 ... lds (HBM -> LDS, no registers) into a 4-stage ring.
// Lane l of a DMA lands at LDS base + 16*l; four consecutive lanes fetch one
// 64-byte row (coalesced), each lane picking its piece so that the ring holds
// rows of four 16-byte pieces with piece c of row r at slot 4r + (c ^ ((r>>2)
// & 3)): the MFMA operand reads (ds_read_b128, lane l reads row l%32, piece
// 2s + l/32) are then free of LDS bank conflicts.  Each stage's block scales
// ride in the weight half of its slot.  Synchronisation is explicit: s_waitcnt
// vmcnt for this wave's DMAs, then s_barrier.  Every wave issues the same
// number of DMAs per stage (the vmcnt waits count them); waves with nothing to
// load issue a DMA through an empty buffer resource, which reads nothing and
// writes zeros into a discard chunk.
#include <algorithm>
#include <type_traits>

#include "pixhip_device.h"
#include "pixhip_internal.h"

#define PIX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace pixhip {

constexpr int kBM = PIX_GEMM_MTILE, kBN = PIX_GEMM_NTILE, kKC = 64;
constexpr int kWavesM = 4, kWavesN = 4, kWaves = kWavesM * kWavesN, kThreads = 64 * kWaves;
constexpr int kWN = kBN / kWavesN;  // features per wave
constexpr int kNJ = kWN / 32;       // 32-column MFMA tiles per wave
constexpr int kStages = 4;          // ring depth: one stage read, kDist in flight
constexpr int kDist = kStages - 1;  // prefetch distance in stages
constexpr int kChunk = 1024;        // bytes written by one DMA instruction (64 lanes x 16 B)
constexpr int kStageBytes = 32768;
constexpr int kStageChunks = kStageBytes / kChunk;  // 32: 4 per wave
constexpr int kPerWave = kStageChunks / kWaves;
constexpr int kSBC = PIX_QK / kKC;                  // stages per 256-value super-block (the split-K granule)
static_assert(kWavesM * 64 == kBM && kWavesN * kWN == kBN && kNJ * 32 == kWN, "wave grid covers the tile");
static_assert(kPerWave * kWaves == kStageChunks, "stage DMAs split evenly over the waves");

// Ring layout: the activation halves of the four stages are contiguous
// (A ring, 4 x 16 KB from LDS 0), then the weight halves (W ring, 4 x 16 KB from
// 64 KB), so that every operand read is a per-lane base register plus an
// immediate offset below 64 KB.  Within a W slot (16-B slots):
//   W 0..511 | xd[2][256] 512..639 | wd[2][128] 640..703 | unused
constexpr int kHalfBytes = kStageBytes / 2, kWRing = kStages * kHalfBytes;
constexpr int kSlotXd80 = 512, kSlotWd80 = 640;

typedef __amdgpu_buffer_rsrc_t Rsrc;

struct GemmArgs {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/32][Mpad]
    const int8_t* wq;     // [Npad][K]
    const float* wdT;     // [K/32][Npad]
    float* y;
    const float* bias;
    int32_t* sums;        // debug: exact integer sums [M][N][blocks]
    int M, N, K, Mpad, Npad;
    size_t ldy, yoff;
    int tiles_m, tiles_n;
    // Split-K of the last tiles: tiles full_tiles.. (in tile order) run as
    // `splits` K ranges of split_chunks stages each, writing fp32 partials
    // part[split][tile - full_tiles][kBM][kBN] that splitk_reduce_kernel sums.
    int full_tiles, splits, split_chunks;
    float* part;
};

// Tile order: GROUP token tiles share one feature tile, in launch order.
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
    Rsrc rx, rxd, rwq, rwd, rnull;
};

struct Acc {
    v16f y[2][kNJ];  // [token tile][feature tile]
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

// Pins a value at this point of the instruction stream: the empty volatile asm
// "reads and writes" it, so the code computing it cannot sink below (nor its
// later uses rise above) this point.
template <class T> __device__ __forceinline__ void pin(T& v) { __asm__ volatile("" : "+v"(v)); }

// One dword per lane: lane l lands at LDS base + 4*l.
__device__ __forceinline__ void dma4(Rsrc r, uint8_t* lds_uniform, uint32_t voff, uint32_t soff)
{
    __builtin_assume(lds_uniform != nullptr);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,PIX_LDS(lds_uniform),4,(int)voff,(int)soff,0,0);
}

// The lane index, recomputed where it is used (volatile, so the compiler
// cannot keep derived per-lane offsets live across the loop).
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

// DMA of stage c into `sa` / `sw`: chunk wave + 16*q of the 32 is this wave's
// q-th.  Chunks 0..15 are activation rows (16 rows of 64 B each), 16..23 the
// weight rows, 24 and 25 the activation scales of blocks 2c and 2c+1, 26 the
// weight scales of both blocks; 27..31 load nothing.  Lane l fetches chunk row
// l/4, piece (l%4) ^ ((l/16) & 3).
__device__ __forceinline__ void issue_stage(const GemmArgs& g, const Ctx& x, int c, uint8_t* sa, uint8_t* sw, uint8_t* discard)
{
    const uint32_t k0 = (uint32_t)c * kKC;
    uint32_t vo_rows = 0;  // per-lane source offset of a 64-B row piece (for the row chunks)
#pragma unroll
    for (int q = 0; q < kPerWave; q++) {
        const int chunk = x.wave + kWaves * q;  // wave-uniform
        uint8_t* dst = chunk < 16? sa + chunk * kChunk : sw + (chunk - 16) * kChunk;
        if (chunk < 24) {
            const uint32_t lane = lane_now();
            vo_rows = (lane >> 2) * (uint32_t)x.K + 16u * ((lane & 3) ^ ((lane >> 4) & 3));
        }
        if (chunk < 16) {
            dma(x.rx,dst,vo_rows,(uint32_t)(x.m0 + chunk * 16) * x.K + k0);
        } else if (chunk < 24) {
            dma(x.rwq,dst,vo_rows,(uint32_t)(x.n0 + (chunk - 16) * 16) * x.K + k0);
        } else if (chunk < 26) {
            const uint32_t lane = lane_now();
            dma(x.rxd,dst,16u * lane,(uint32_t)((2 * c + chunk - 24) * g.Mpad + x.m0) * 4u);
        } else if (chunk == 26) {
            // lanes 0..31: block 2c, lanes 32..63: block 2c+1 (128 features each)
            const uint32_t lane = lane_now();
            dma(x.rwd,dst,16u * (lane & 31) + (lane >> 5) * 4u * (uint32_t)g.Npad,(uint32_t)(2 * c * g.Npad + x.n0) * 4u);
        } else {
            dma(x.rnull,discard,0,0);
        }
    }
}

// One stage c: two 32-value blocks (k-steps) = eight (block, token tile,
// feature tile) products t = 4*s + 2*i + j, each an i8 MFMA (the integer
// block sums) and an fp16 MFMA (the scale outer product) followed by the fp32
// update of its 32 x 32 accumulator.  The order is fixed (scheduling
// barriers): the MFMAs of product t+1 go out before the update of product t,
// so two products' results are live at a time; the DMA of stage c + kDist
// (into slots other than the one read, `cur`) goes out after the third
// product's MFMAs, when each wave has matrix work in flight while the address
// unit accepts its requests.
template <bool SUMS>
__device__ __forceinline__ void step(const GemmArgs& g, const Ctx& x, int c, Acc& acc, uint8_t* __restrict__ dma_a,
                                     uint8_t* __restrict__ dma_w, uint8_t* __restrict__ discard, const uint8_t* __restrict__ cur)
{
    const v16i izero = {};
    const v16f fzero = {};
    const uint8_t* cur_w = cur + kWRing;
    v4i a[2][2], w[2][kNJ];
    v4h xa[2][2], wb[2][kNJ];
    auto load = [&](int s) {
        // Lane l reads row l%32, piece (2s + l/32) ^ ((l%32 >> 2) & 3) (per-lane
        // offsets are recomputed here rather than kept live across the loop).
        const uint32_t ln = lane_now(), lr = ln & 31;
        const uint32_t cp = lr * 64 + 16 * ((2 * s + (ln >> 5)) ^ ((lr >> 2) & 3));
        const uint32_t oa = (uint32_t)(x.wm * 64 * 64) + cp;
        const uint32_t ow = (uint32_t)(kWRing + x.wn * kWN * 64) + cp;  // relative to the A slot of the same stage
#pragma unroll
        for (int i = 0; i < 2; i++) a[s][i] = *reinterpret_cast<const v4i*>(cur + oa + i * 2048);
#pragma unroll
        for (int j = 0; j < kNJ; j++) w[s][j] = *reinterpret_cast<const v4i*>(cur + ow + j * 2048);
        if constexpr (!SUMS) {
            // K slot 0 (lanes 0..31) carries the scales, the other slots zero;
            // xd and wd are fp16-rounded values, so the conversions are exact.
            const float* sxd = reinterpret_cast<const float*>(cur_w + 16 * kSlotXd80) + s * kBM + x.wm * 64;
            const float* swd = reinterpret_cast<const float*>(cur_w + 16 * kSlotWd80) + s * kBN + x.wn * kWN;
            const bool k0 = ln < 32;
            const _Float16 z = (_Float16)0.0f;
            // (read by every lane, then selected: no branch around the LDS reads)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float v = sxd[i * 32 + lr];
                xa[s][i] = v4h{(_Float16)(k0? v : 0.0f),z,z,z};
            }
#pragma unroll
            for (int j = 0; j < kNJ; j++) {
                const float v = swd[j * 32 + lr];
                wb[s][j] = v4h{(_Float16)(k0? v : 0.0f),z,z,z};
            }
        }
    };
    if constexpr (SUMS) {
        const uint32_t ln = lane_now();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            load(s);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < kNJ; j++) {
                    const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][i],w[s][j],izero,0,0,0);
                    const int kb = c * 2 + s;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = x.m0 + x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                        const int n = x.n0 + x.wn * kWN + j * 32 + lr;
                        if (m < g.M && n < g.N) g.sums[((size_t)m * g.N + n) * (x.K / PIX_QK8) + kb] = p[r];
                    }
                }
        }
        if (c + kDist < x.nchunks) issue_stage(g,x,c + kDist,dma_a,dma_w,discard);
        return;
    }
    constexpr int T = 2 * 2 * kNJ;  // products per stage
    v16i p[2];
    v16f cs[2];
    auto epi = [&](int t, int r0, int r1) {
        const int i = (t / kNJ) & 1, j = t % kNJ;
#pragma unroll
        for (int r = r0; r < r1; r++) acc.y[i][j][r] = __builtin_fmaf(cs[t & 1][r],(float)p[t & 1][r],acc.y[i][j][r]);
        pin(acc.y[i][j]);
    };
    load(0);
    p[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][0],w[0][0],izero,0,0,0);
    cs[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(xa[0][0],wb[0][0],fzero,0,0,0);
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int u = t + 1, s = u / (2 * kNJ), i = (u / kNJ) & 1, j = u % kNJ;
        __builtin_amdgcn_sched_barrier(0);
        if (u < T) {
            p[u & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][i],w[s][j],izero,0,0,0);
            pin(p[u & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (t == 1 && c + kDist < x.nchunks) issue_stage(g,x,c + kDist,dma_a,dma_w,discard);
        __builtin_amdgcn_sched_barrier(0);
        epi(t,0,16);
        __builtin_amdgcn_sched_barrier(0);
        if (u < T) {
            cs[u & 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(xa[s][i],wb[s][j],fzero,0,0,0);
            pin(cs[u & 1]);
        }
        if (t == 0) {
            __builtin_amdgcn_sched_barrier(0);
            load(1);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// The main loop's per-lane constants, computed once: every per-stage LDS
// address is one of these plus an immediate (the loop is unrolled over the
// ring slots), and every DMA source offset is one of these plus a
// wave-uniform scalar offset, so the loop spends no vector instructions on
// addresses.
constexpr int kZero = 16 * 704;  // a zeroed word range in every W slot (past the scales)
struct Lanes {
    uint32_t ra[2], rw[2];  // operand reads of k-step s: this lane's A row piece (ring 0) and W row piece (from kWRing)
    uint32_t sx, sw;        // block scales: xd of this lane's token row / wd of its feature (lanes 32..63: a zero word)
    uint32_t d0, d1;        // source offsets of this wave's two DMAs of a stage
};

__device__ __forceinline__ Lanes lanes_of(const GemmArgs& g, const Ctx& x)
{
    Lanes L;
    const uint32_t ln = lane_now(), lr = ln & 31, hi = ln >> 5;
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t cp = lr * 64 + 16 * ((2 * s + hi) ^ ((lr >> 2) & 3));
        L.ra[s] = (uint32_t)(x.wm * 64 * 64) + cp;
        L.rw[s] = (uint32_t)(kWRing + x.wn * kWN * 64) + cp;
    }
    L.sx = kWRing + (hi? kZero : 16 * kSlotXd80 + (x.wm * 64 + lr) * 4);
    L.sw = kWRing + (hi? kZero : 16 * kSlotWd80 + (x.wn * kWN + lr) * 4);
    const uint32_t rows = (ln >> 2) * (uint32_t)x.K + 16u * ((ln & 3) ^ ((ln >> 4) & 3));
    L.d0 = rows;  // chunk x.wave < 16: activation rows
    const int c1 = x.wave + kWaves;
    L.d1 = c1 < 24? rows : c1 < 26? 16u * ln : c1 == 26? 16u * lr + hi * 4u * (uint32_t)g.Npad : 0u;
    return L;
}

// DMA of stage c into ring slot SLOT (the chunk map of issue_stage).
template <int SLOT>
__device__ __forceinline__ void issue_slot(const GemmArgs& g, const Ctx& x, const Lanes& L, int c, uint8_t* lds)
{
    const uint32_t k0 = (uint32_t)c * kKC;
    uint8_t* sa = lds + SLOT * kHalfBytes;
    uint8_t* sw = lds + kWRing + SLOT * kHalfBytes;
    const int c0 = x.wave, c1 = x.wave + kWaves;
    dma(x.rx,sa + c0 * kChunk,L.d0,(uint32_t)(x.m0 + c0 * 16) * x.K + k0);
    if (c1 < 24) dma(x.rwq,sw + (c1 - 16) * kChunk,L.d1,(uint32_t)(x.n0 + (c1 - 16) * 16) * x.K + k0);
    else if (c1 < 26) dma(x.rxd,sw + (c1 - 16) * kChunk,L.d1,(uint32_t)((2 * c + c1 - 24) * g.Mpad + x.m0) * 4u);
    else if (c1 == 26) dma(x.rwd,sw + (c1 - 16) * kChunk,L.d1,(uint32_t)(2 * c * g.Npad + x.n0) * 4u);
    else dma(x.rnull,lds + kStages * kStageBytes,0,0);
}

// {fp16(v), 0, 0, 0}: the scale in K slot 0 of an fp16 MFMA operand (v is an
// fp16 value, so the round-toward-zero conversion is exact; lanes 32..63 read
// the zero word).
__device__ __forceinline__ v4h scale_operand(float v)
{
    const auto h = __builtin_amdgcn_cvt_pkrtz(v,0.0f);
    return v4h{(_Float16)h[0],(_Float16)h[1],(_Float16)0.0f,(_Float16)0.0f};
}

// One stage from ring slot SLOT: the product order of step() (the MFMAs of
// product t+1 before the update of product t), the DMA of stage c + kDist into
// slot (SLOT + kDist) % kStages after the second product.
template <int SLOT>
__device__ __forceinline__ void stage_slot(const GemmArgs& g, const Ctx& x, const Lanes& L, int c, Acc& acc, uint8_t* lds)
{
    const v16i izero = {};
    const v16f fzero = {};
    v4i a[2][2], w[2][kNJ];
    v4h xa[2][2], wb[2][kNJ];
    auto load = [&](int s) {
#pragma unroll
        for (int i = 0; i < 2; i++) a[s][i] = *reinterpret_cast<const v4i*>(lds + L.ra[s] + SLOT * kHalfBytes + i * 2048);
#pragma unroll
        for (int j = 0; j < kNJ; j++) w[s][j] = *reinterpret_cast<const v4i*>(lds + L.rw[s] + SLOT * kHalfBytes + j * 2048);
#pragma unroll
        for (int i = 0; i < 2; i++)
            xa[s][i] = scale_operand(*reinterpret_cast<const float*>(lds + L.sx + SLOT * kHalfBytes + (s * kBM + i * 32) * 4));
#pragma unroll
        for (int j = 0; j < kNJ; j++)
            wb[s][j] = scale_operand(*reinterpret_cast<const float*>(lds + L.sw + SLOT * kHalfBytes + (s * kBN + j * 32) * 4));
    };
    constexpr int T = 2 * 2 * kNJ;
    v16i p[2];
    v16f cs[2];
    auto epi = [&](int t) {
        const int i = (t / kNJ) & 1, j = t % kNJ;
#pragma unroll
        for (int r = 0; r < 16; r++) acc.y[i][j][r] = __builtin_fmaf(cs[t & 1][r],(float)p[t & 1][r],acc.y[i][j][r]);
        pin(acc.y[i][j]);
    };
    load(0);
    p[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][0],w[0][0],izero,0,0,0);
    cs[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(xa[0][0],wb[0][0],fzero,0,0,0);
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int u = t + 1, s = u / (2 * kNJ), i = (u / kNJ) & 1, j = u % kNJ;
        __builtin_amdgcn_sched_barrier(0);
        if (u < T) {
            p[u & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][i],w[s][j],izero,0,0,0);
            pin(p[u & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (t == 1 && c + kDist < x.nchunks) issue_slot<(SLOT + kDist) % kStages>(g,x,L,c + kDist,lds);
        __builtin_amdgcn_sched_barrier(0);
        epi(t);
        __builtin_amdgcn_sched_barrier(0);
        if (u < T) {
            cs[u & 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(xa[s][i],wb[s][j],fzero,0,0,0);
            pin(cs[u & 1]);
        }
        if (t == 0) {
            __builtin_amdgcn_sched_barrier(0);
            load(1);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Stage c (slot SLOT) of the main loop: wait for its DMAs, barrier, compute.
template <int SLOT>
__device__ __forceinline__ void loop_stage(const GemmArgs& g, const Ctx& x, const Lanes& L, int c, Acc& acc, uint8_t* lds)
{
    if (c + kDist - 1 < x.nchunks) wait_vmcnt<(kDist - 1) * kPerWave>();
    else wait_vmcnt<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    stage_slot<SLOT>(g,x,L,c,acc,lds);
}

template <bool SUMS>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g)
{
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes + kChunk];
    uint8_t* const discard = lds + kStages * kStageBytes;

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
    x.K = g.K;
    x.c_begin = piece? split * g.split_chunks : 0;
    x.nchunks = piece? min(x.c_begin + g.split_chunks,g.K / kKC) : g.K / kKC;
    {
        const size_t mp = (size_t)g.Mpad, np = (size_t)g.Npad, K = (size_t)g.K;
        const size_t nblk = K / PIX_QK8;
        x.rx = make_rsrc(g.xq,mp * K);
        x.rxd = make_rsrc(g.xdT,nblk * mp * 4);
        x.rwq = make_rsrc(g.wq,np * K);
        x.rwd = make_rsrc(g.wdT,nblk * np * 4);
        x.rnull = make_rsrc(g.xq,0);
    }

    Acc acc;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < kNJ; j++) acc.y[i][j] = v16f{};

    const int C0 = x.c_begin, C = x.nchunks;
    if constexpr (SUMS) {
        for (int c = C0; c < C0 + kDist; c++)
            if (c < C) issue_stage(g,x,c,lds + (c % kStages) * kHalfBytes,lds + kWRing + (c % kStages) * kHalfBytes,discard);
        // (The integer-sum debug variant also stores inside the loop; stores
        // share vmcnt and may retire early, so it drains everything.)
        for (int c = C0; c < C; c++) {
            wait_vmcnt<0>();
            wait_lgkm0();
            __builtin_amdgcn_s_barrier();
            const int sd = (c + kDist) % kStages, sc = c % kStages;
            step<SUMS>(g,x,c,acc,lds + sd * kHalfBytes,lds + kWRing + sd * kHalfBytes,discard,lds + sc * kHalfBytes);
        }
    } else {
        // Stage c sits in ring slot (c - C0) % kStages.  The scale operands of
        // lanes 32..63 read the zero word range of each W slot, which no DMA
        // writes: clear it once (ordered before the first reads by the first
        // barrier).
        const Lanes L = lanes_of(g,x);
        for (int i = (int)threadIdx.x; i < kStages * 320; i += kThreads)
            *reinterpret_cast<uint32_t*>(lds + kWRing + (i / 320) * kHalfBytes + kZero + (i % 320) * 4) = 0u;
        if (C0 < C) issue_slot<0>(g,x,L,C0,lds);
        if (C0 + 1 < C) issue_slot<1>(g,x,L,C0 + 1,lds);
        if (C0 + 2 < C) issue_slot<2>(g,x,L,C0 + 2,lds);
        static_assert(kStages == 4 && kDist == 3, "the prologue and the unrolled loop assume a 4-slot ring");
        // Stage c has landed once only the DMAs issued in the kDist-1 stages
        // before c may still be in flight; the last kDist-1 stages issue
        // fewer, so they drain.
        for (int c = C0; c < C; c += kStages) {
            loop_stage<0>(g,x,L,c,acc,lds);
            if (c + 1 < C) loop_stage<1>(g,x,L,c + 1,acc,lds);
            if (c + 2 < C) loop_stage<2>(g,x,L,c + 2,acc,lds);
            if (c + 3 < C) loop_stage<3>(g,x,L,c + 3,acc,lds);
        }
    }

    if (!SUMS && (int)blockIdx.x >= g.full_tiles) {
        // Split-K: this K range's fp32 partial tile; splitk_reduce_kernel adds
        // the ranges in order and applies bias, ldy and offset.
        const int p = (int)blockIdx.x - g.full_tiles, nsplit = g.tiles_m * g.tiles_n - g.full_tiles;
        const uint32_t ln = lane_now();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
        float* part = g.part + ((size_t)(p / nsplit) * nsplit + p % nsplit) * (kBM * kBN) + x.wn * kWN + lr;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < kNJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int lm = x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                    part[(size_t)lm * kBN + j * 32] = acc.y[i][j][r];
                }
    } else if constexpr (!SUMS) {
        // Bias for this lane's columns, loaded once (clamped index) and drained
        // before the stores; the output is stored non-temporally (written once,
        // it would otherwise push the operands out of the last-level cache).
        const uint32_t ln = lane_now();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
        const int mrow0 = x.m0 + x.wm * 64, ncol0 = x.n0 + x.wn * kWN;
        float bv[kNJ];
#pragma unroll
        for (int j = 0; j < kNJ; j++) bv[j] = g.bias? g.bias[min(ncol0 + j * 32 + lr,g.N - 1)] : 0.0f;
        wait_vmcnt<0>();
        const bool full = mrow0 + 64 <= g.M && ncol0 + kWN <= g.N;
#pragma unroll
        for (int j = 0; j < kNJ; j++) {
            const int n = ncol0 + j * 32 + lr;
            float* col = g.y + g.yoff + n;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = mrow0 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                    if (full || (m < g.M && n < g.N)) __builtin_nontemporal_store(acc.y[i][j][r] + bv[j],col + (size_t)m * g.ldy);
                }
        }
    }
}


// ---------------------------------------------------------------------------
// K-grouped form for grids far too small to fill the device (the 256-token
// linear has thirty 256 x 128 tiles for 256 CUs).  A workgroup owns a 64 x 64
// tile and splits its K range over four K-groups of four waves: group g runs
// stages [g*Cg, (g+1)*Cg) with its own 3-slot ring, each of its waves owns a
// 32 x 32 quarter of the tile, and at the end groups 1..3 hand their
// accumulators to group 0 through LDS, which adds them in group order and
// stores.  No fp32 partial tiles go through memory and the sum order is fixed.
// A stage slot (9 KB) holds the 64 activation rows (4 KB, four 16-row
// DMAs), the 64 weight rows (4 KB) and the activation and weight scales of the
// stage's two blocks (4 x 256 B, one dword DMA each).  Per stage each wave of a
// group issues three of the twelve DMAs.
constexpr int kSBM = 64, kSBN = 64, kSGroups = 4, kSWaves = 16, kSThreads = 64 * kSWaves;
constexpr int kSSlots = 4, kSDist = kSSlots - 1;
// kSZero: 512 zeroed bytes after the scales, read by lanes 32..63 as their
// (zero) scale operand slots.
constexpr int kSXd = 8 * kChunk, kSWd = kSXd + 2 * 256, kSZero = kSWd + 2 * 256, kSSlotBytes = kSZero + 512;
constexpr int kSChunks = 12, kSGroupBytes = kSSlots * kSSlotBytes;
constexpr int kSPerWave = 3;
constexpr int kSRedBytes = (kSGroups - 1) * 4 * 32 * 32 * 4;  // groups 1..3: four 32 x 32 fp32 blocks each
static_assert(kSGroups * 4 == kSWaves && kSPerWave * 4 == kSChunks, "K-grouped shape");
static_assert(kSRedBytes <= kSGroups * kSGroupBytes, "the reduction reuses the rings");

struct SmallCtx {
    int m0, n0, q, wm, wn, K, Mpad, Npad;
    int begin, end;  // this group's stages
    Rsrc rx, rxd, rwq, rwd;
};

// Per-lane constants of the K-grouped loop (as Lanes for the 256 x 128 form):
// operand and scale reads relative to the group's ring, DMA source offsets.
struct SmallLanes {
    uint32_t ra[2], rw[2], sx, sw;
    uint32_t d_rows, d_scale;
};

__device__ __forceinline__ SmallLanes small_lanes(const SmallCtx& x, uint32_t ring)
{
    SmallLanes L;
    const uint32_t ln = lane_now(), lr = ln & 31, hi = ln >> 5;
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t piece = 16 * ((2 * s + hi) ^ ((lr >> 2) & 3));
        L.ra[s] = ring + (x.wm * 32 + lr) * 64 + piece;
        L.rw[s] = ring + 4 * kChunk + (x.wn * 32 + lr) * 64 + piece;
    }
    L.sx = ring + (hi? kSZero : kSXd + (x.wm * 32 + lr) * 4);
    L.sw = ring + (hi? kSZero : kSWd + (x.wn * 32 + lr) * 4);
    L.d_rows = (ln >> 2) * (uint32_t)x.K + 16u * ((ln & 3) ^ ((ln >> 4) & 3));
    L.d_scale = 4u * ln;
    return L;
}

// DMA of stage c into ring slot SLOT: wave q of a group issues chunks q (an
// activation row block), q + 4 (a weight row block) and q + 8 (the scales of
// block 2c + q for q < 2, else the weight scales of block 2c + q - 2).
template <int SLOT>
__device__ __forceinline__ void small_issue(const SmallCtx& x, const SmallLanes& L, int c, uint8_t* ring)
{
    const uint32_t k0 = (uint32_t)c * kKC;
    uint8_t* slot = ring + SLOT * kSSlotBytes;
    dma(x.rx,slot + x.q * kChunk,L.d_rows,(uint32_t)(x.m0 + x.q * 16) * x.K + k0);
    dma(x.rwq,slot + (x.q + 4) * kChunk,L.d_rows,(uint32_t)(x.n0 + x.q * 16) * x.K + k0);
    if (x.q < 2) dma4(x.rxd,slot + kSXd + 256 * x.q,L.d_scale,(uint32_t)((2 * c + x.q) * x.Mpad + x.m0) * 4u);
    else dma4(x.rwd,slot + kSWd + 256 * (x.q - 2),L.d_scale,(uint32_t)((2 * c + x.q - 2) * x.Npad + x.n0) * 4u);
}

// One stage from ring slot SLOT: two blocks, each an i8 MFMA and the fp16 scale
// outer product, then y += cs * P; the DMA of stage c + kSDist goes out after
// the MFMAs.
template <int SLOT>
__device__ __forceinline__ void small_stage(const SmallCtx& x, const SmallLanes& L, int c, v16f& acc, uint8_t* lds, uint8_t* ring)
{
    const v16i izero = {};
    const v16f fzero = {};
    v4i a[2], w[2];
    v4h xa[2], wb[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        a[s] = *reinterpret_cast<const v4i*>(lds + L.ra[s] + SLOT * kSSlotBytes);
        w[s] = *reinterpret_cast<const v4i*>(lds + L.rw[s] + SLOT * kSSlotBytes);
        xa[s] = scale_operand(*reinterpret_cast<const float*>(lds + L.sx + SLOT * kSSlotBytes + s * kSBM * 4));
        wb[s] = scale_operand(*reinterpret_cast<const float*>(lds + L.sw + SLOT * kSSlotBytes + s * kSBN * 4));
    }
    v16i p[2];
    v16f cs[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        p[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s],w[s],izero,0,0,0);
        cs[s] = __builtin_amdgcn_mfma_f32_32x32x8f16(xa[s],wb[s],fzero,0,0,0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c + kSDist < x.end) small_issue<(SLOT + kSDist) % kSSlots>(x,L,c + kSDist,ring);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(cs[s][r],(float)p[s][r],acc[r]);
    pin(acc);
}

template <int SLOT>
__device__ __forceinline__ void small_loop_stage(const SmallCtx& x, const SmallLanes& L, int c, v16f& acc, uint8_t* lds,
                                                 uint8_t* ring)
{
    if (c + kSDist - 1 < x.end) wait_vmcnt<(kSDist - 1) * kSPerWave>();
    else wait_vmcnt<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    if (c < x.end) small_stage<SLOT>(x,L,c,acc,lds,ring);
}

__global__ __launch_bounds__(kSThreads, 1) void gemm_small_kernel(GemmArgs g)
{
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kSGroups * kSGroupBytes];
    const int ntiles = g.tiles_m * g.tiles_n;
    const int lid = xcd_remap((int)blockIdx.x,ntiles);
    SmallCtx x;
    x.m0 = (lid % g.tiles_m) * kSBM;  // consecutive tiles share a weight tile
    x.n0 = (lid / g.tiles_m) * kSBN;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int grp = wave / 4;
    x.q = wave % 4;
    x.wm = x.q % 2;
    x.wn = x.q / 2;
    x.K = g.K;
    x.Mpad = g.Mpad;
    x.Npad = g.Npad;
    const int C = g.K / kKC, Cg = (C + kSGroups - 1) / kSGroups;
    x.begin = min(grp * Cg,C);
    x.end = min(x.begin + Cg,C);
    {
        const size_t mp = (size_t)g.Mpad, np = (size_t)g.Npad, K = (size_t)g.K;
        const size_t nblk = K / PIX_QK8;
        x.rx = make_rsrc(g.xq,mp * K);
        x.rxd = make_rsrc(g.xdT,nblk * mp * 4);
        x.rwq = make_rsrc(g.wq,np * K);
        x.rwd = make_rsrc(g.wdT,nblk * np * 4);
    }
    uint8_t* const ring = lds + grp * kSGroupBytes;
    const SmallLanes L = small_lanes(x,(uint32_t)(grp * kSGroupBytes));
    // The zero bytes after each slot's scales (lanes 32..63's scale reads),
    // which no DMA writes; the first barrier orders this before the reads.
    for (int i = (int)threadIdx.x; i < kSGroups * kSSlots * 128; i += kSThreads)
        *reinterpret_cast<uint32_t*>(lds + (i / 128) * kSSlotBytes + kSZero + (i % 128) * 4) = 0u;

    v16f acc = {};
    static_assert(kSSlots == 4 && kSDist == 3, "the prologue and the unrolled loop assume a 4-slot ring");
    if (x.begin < x.end) small_issue<0>(x,L,x.begin,ring);
    if (x.begin + 1 < x.end) small_issue<1>(x,L,x.begin + 1,ring);
    if (x.begin + 2 < x.end) small_issue<2>(x,L,x.begin + 2,ring);
    // Every wave runs Cg iterations (one barrier each); a group past its
    // range idles through them.  Stage c (slot (c - begin) % 4) has landed
    // once at most the DMAs of stage c+1 are in flight.
    for (int i = 0; i < Cg; i += kSSlots) {
        const int c = x.begin + i;
        small_loop_stage<0>(x,L,c,acc,lds,ring);
        if (i + 1 < Cg) small_loop_stage<1>(x,L,c + 1,acc,lds,ring);
        if (i + 2 < Cg) small_loop_stage<2>(x,L,c + 2,acc,lds,ring);
        if (i + 3 < Cg) small_loop_stage<3>(x,L,c + 3,acc,lds,ring);
    }
    wait_vmcnt<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    // Groups 1..3 hand over their 32 x 32 blocks ([group-1][quarter][r][lane]
    // fp32, conflict-free), group 0 adds them in group order.
    const uint32_t ln = lane_now();
    float* red = reinterpret_cast<float*>(lds);
    if (grp > 0) {
        float* dst = red + ((grp - 1) * 4 + x.q) * 1024 + ln;
#pragma unroll
        for (int r = 0; r < 16; r++) dst[r * 64] = acc[r];
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    if (grp != 0) return;
#pragma unroll
    for (int g2 = 1; g2 < kSGroups; g2++) {
        const float* src = red + ((g2 - 1) * 4 + x.q) * 1024 + ln;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] += src[r * 64];
    }
    const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
    const int n = x.n0 + x.wn * 32 + lr;
    const float bv = g.bias? g.bias[min(n,g.N - 1)] : 0.0f;
    float* col = g.y + g.yoff + n;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = x.m0 + x.wm * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (m < g.M && n < g.N) __builtin_nontemporal_store(acc[r] + bv,col + (size_t)m * g.ldy);
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

// The Q8_0 GEMM runs the K-grouped 64 x 64 form when its 256 x 128 tiles
// would fill at most a quarter of the device (measured at N = K = 3840: 256
// and 512 tokens faster in this form, 1024 tokens -- 120 tiles, split-K --
// faster in the other).
bool gemm_q8_0_grouped(size_t M, size_t N)
{
    const size_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    return tiles * 4 <= (size_t)device_cus();
}

size_t gemm_split_bytes(size_t M, size_t N, size_t K_stages)
{
    int full, chunks;
    const int splits = gemm_split_plan(M,N,K_stages,full,chunks);
    const size_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    return splits > 1? (size_t)splits * (tiles - full) * (kBM * kBN) * sizeof(float) : 0;
}

template <bool SUMS>
static hipError_t launch(GemmArgs g, size_t mpad, size_t npad, hipStream_t s)
{
    g.tiles_m = (int)((g.M + kBM - 1) / kBM);
    g.tiles_n = (int)((g.N + kBN - 1) / kBN);
    if (mpad < round_up((size_t)g.M,kBM) || npad < round_up((size_t)g.N,kBN) || g.K % kKC) return hipErrorInvalidValue;
    // Buffer offsets are 32-bit: every operand plane must stay below 2 GiB.
    const size_t lim = (size_t)1 << 31;
    const size_t scales = ((size_t)g.K / PIX_QK8) * (npad > mpad? npad : mpad) * 4;
    if (mpad * g.K >= lim || npad * g.K >= lim || scales >= lim) return hipErrorInvalidValue;
    g.Mpad = (int)mpad;
    g.Npad = (int)npad;
    const int ntiles = g.tiles_m * g.tiles_n;
    if (!ntiles) return hipSuccess;
    if (!SUMS && gemm_q8_0_grouped((size_t)g.M,(size_t)g.N)) {
        g.tiles_m = (int)((g.M + kSBM - 1) / kSBM);
        g.tiles_n = (int)((g.N + kSBN - 1) / kSBN);
        gemm_small_kernel<<<dim3(g.tiles_m * g.tiles_n),dim3(kSThreads),0,s>>>(g);
        return hipGetLastError();
    }
    g.splits = SUMS? 1 : gemm_split_plan((size_t)g.M,(size_t)g.N,(size_t)g.K,g.full_tiles,g.split_chunks);
    if (g.splits == 1 || !g.part) {  // unsplit (or no workspace)
        g.splits = 1;
        g.full_tiles = ntiles;
        g.split_chunks = g.K / kKC;
    }
    const int split_tiles = ntiles - g.full_tiles;
    gemm_kernel<SUMS><<<dim3(g.full_tiles + split_tiles * g.splits),dim3(kThreads),0,s>>>(g);
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
    g.wq = w.qs; g.wdT = w.dT;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<false>(g,a.mpad,round_up(N,kBN),s);
}

hipError_t launch_sums_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.xq = a.qs; g.xdT = a.d;
    g.wq = w.qs; g.wdT = w.dT;
    g.sums = sums;
    return launch<true>(g,a.mpad,round_up(N,kBN),s);
}

}  // namespace pixhip
