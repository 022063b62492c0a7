// K-quant GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for Q5_K
// and Q6_K weights with Q8_K activations -- the counterpart of pix_dot_q5_K /
// pix_dot_q6_K driven by cpu_quant_matmul (src/kernels_quant.cpp:163-337,
// :369-412) and of shaders/matmul_mmq.comp's K-quant path.
//
// Exactness: every weight is held as two int8 planes with scale_s * q = 64*hi
// + lo (Q5_K) or scale * (q - 32) = 64*hi + lo (Q6_K), so two
// v_mfma_i32_32x32x32_i8 per tile and 32-value sub-block produce the exact
// integer S = sum_s scale_s * dot_s of a 256-value super-block.  The Q5_K
// minimum term Mn = sum_s min_s * (bsum_2s + bsum_2s+1) is one fp16 MFMA on the
// 16-value activation sums and the six-bit minima (integers of at most 11 bits,
// so the fp32 result is exact).  Per super-block the fp32 epilogue is
// y += yd * (wd * S - wdmin * Mn).
//
// Tiling: a workgroup of 8 waves (2 per SIMD: waves w and w+4 share one)
// owns a 256 (tokens) x 128 (features) tile; wave w owns the 64 x 64 block at
// tokens 64*(w%4), features 64*(w/4): two token tiles x two feature tiles of
// 32 x 32, each with hi, lo and fp32 accumulators (192 registers).  A wave
// keeps the operands of one 32-value sub-block in registers (two activation
// fragments, double-buffered, and four weight fragments) and reads the next
// sub-block's fragments as registers free up, each at least four MFMAs before
// its use.
//
// Data movement: K advances in 64-value stages (16 KB of activations, 16 KB of
// weight planes per stage) through LDS rings filled by buffer_load_dwordx4 ...
// lds (L2 -> LDS without registers): five activation slots, four weight slots.
// The operand planes are tiled in HBM so that one DMA instruction reads one
// contiguous 1 KB block (16 rows x 64 values): whole 128-byte lines, which the
// memory path delivers at twice the rate of the 16 half lines a row-major
// plane gives.  In LDS, rows are four 16-byte pieces, piece c of row r at
// position 4r + (c ^ ((r>>2)&3)), which makes the ds_read_b128 operand reads
// (lane l: row l%32, piece 2s + l/32) free of bank conflicts.  The epilogue
// inputs of one super-block (yd, wd, 16-value sums, minima, wdmin) sit in a
// region after the rings.
//
// Synchronisation: one s_barrier per interval of two stages; the two wave
// groups run one stage apart so that their super-block epilogues fall at
// different points of an interval (the schedule is described at wait_all).
// A wave drains its own DMAs and LDS reads before each barrier.
//
// What bounds it (Q5_K, 4096 x 3840 x 10240, ~320 us; variants that drop one
// component each): the MFMAs with their LDS operand reads alone take ~210 us
// (the int8 matrix-core time at the ~2.1 GHz this load runs at is ~145 us;
// the tile prologues and output stores of five tiles per CU are part of the
// difference), the super-block epilogue adds ~55 us and the L2 -> LDS
// traffic (2.5 GB per launch, 78% L2 hits) ~45 us.  Hardware counters put the
// matrix core at 49% busy.
#include <type_traits>

#include "pixhip_device.h"
#include "pixhip_internal.h"

#define PIX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace pixhip {
namespace {

constexpr int kBM = PIX_GEMM_MTILE, kBN = PIX_GEMM_NTILE, kKC = 64;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kASlots = 5;                  // activation ring slots
constexpr int kWSlots = 4;                  // weight ring slots
constexpr int kChunk = 1024;                // bytes written by one DMA instruction (64 lanes x 16 B)
constexpr int kHalf = 16384;                // activation (or weight) bytes of one stage
constexpr int kWRing = kASlots * kHalf;     // weight ring after the activation ring
constexpr int kScaleAt = kWRing + kWSlots * kHalf;  // one super-block's epilogue inputs after the rings
constexpr int kPlane = 8192;                // lo plane after hi within a weight slot
constexpr int kSBC = PIX_QK / kKC;          // stages per super-block
static_assert(kWaves * 64 == kThreads && kBM == 4 * 64 && kBN == 2 * 64, "wave grid covers the tile");

// Scale region of one super-block (16-B slots; DMA chunk c fills slots 64c..64c+63):
//   yd[256] 0..63 | wd[128] 64..95 | bs[256][2] 128..639 (16-value sums) |
//   mn[128] 640..767 (minima) | wdm[128] 768..799
constexpr int kSlotYd = 0, kSlotWd = 64, kSlotBs = 128, kSlotMn = 640, kSlotWdm = 768;
template <bool Q5> constexpr int scale_chunks() { return Q5? 13 : 2; }
template <bool Q5> constexpr int scale_bytes() { return scale_chunks<Q5>() * kChunk; }

typedef __amdgpu_buffer_rsrc_t Rsrc;

struct Args {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/256][Mpad]
    const _Float16* xbs;  // [Mpad][K/16] (Q5_K)
    const int8_t* whi;    // [Npad][K]
    const int8_t* wlo;    // [Npad][K]
    const float* wdT;     // [K/256][Npad]
    const float* wdm;     // [K/256][Npad] (Q5_K)
    const _Float16* wmn;  // [K/256][Npad][8] (Q5_K)
    float* y;
    const float* bias;
    int32_t* sums;        // integer-sum variant: [M][N][K/256]
    int32_t* mins;
    int M, N, K, Mpad, Npad;
    size_t ldy, yoff;
    int tiles_m, tiles_n;
    // Split-K of the last tiles: tiles full_tiles.. (tile order) run as
    // `splits` K ranges of split_chunks stages, writing fp32 partial tiles
    // part[split][tile - full_tiles][kBM][kBN] that the reduce kernel adds.
    int full_tiles, splits, split_chunks;
    float* part;
};

__device__ __forceinline__ void tile_of(int lid, int tiles_m, int tiles_n, int& tm, int& tn)
{
    constexpr int GROUP = 4;  // token tiles per feature tile, in launch order
    const int group = lid / (GROUP * tiles_n);
    const int first_m = group * GROUP;
    const int gsize = min(tiles_m - first_m,GROUP);
    const int within = lid % (GROUP * tiles_n);
    tm = first_m + within % gsize;
    tn = within / gsize;
}

// Hardware places workgroup b on XCD b % 8; give each XCD a contiguous range
// of logical tiles so its L2 sees neighbours.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd < r? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

template <int N> __device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

__device__ __forceinline__ Rsrc make_rsrc(const void* base, size_t bytes)
{
    // Raw buffer, stride 0: offsets at or beyond `bytes` read as zero; a null
    // base gets an empty range, so a missing plane reads zeros.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base),(short)0,base? (int)bytes : 0,0x00020000);
}

__device__ __forceinline__ void dma(Rsrc r, uint8_t* lds_uniform, uint32_t voff, uint32_t soff)
{
    __builtin_assume(lds_uniform != nullptr);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,PIX_LDS(lds_uniform),16,(int)voff,(int)soff,0,0);
}

__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u,__builtin_amdgcn_mbcnt_lo(~0u,0u)); }

struct Ctx {
    int m0, n0, wave, wm, wn, K;
    int c_begin, nchunks;   // this workgroup's stages c_begin .. nchunks-1 (c_begin starts a super-block)
    bool lag;               // group 1 (waves 4-7): one stage behind group 0
    uint32_t oa0;           // per-lane LDS offset of the wave's activation fragments (sub-block 0 of a stage;
                            // sub-block 1 is oa0 ^ 32)
    uint32_t ow0;           // same for the weight fragments (absolute, includes the weight ring base)
    uint32_t vo_tile;       // per-lane DMA source offset within a 1 KB tile (16 rows x 64 B)
    Rsrc rx, rxd, rxbs, rwh, rwl, rwd, rwdm, rwmn;
};

struct Opnd {
    v4i a[2][2];     // [sub-block parity][token tile]: the next sub-block's activations load into the other half
    v4i h[2], l[2];  // [feature tile] of the hi and lo planes
};

struct Acc {
    v16i hi[2][2], lo[2][2];  // [token tile][feature tile]
    v16f y[2][2];
};

// Byte offset of stage s's slot in the activation ring (runtime: five slots).
__device__ __forceinline__ uint32_t a_off(const Ctx& x, int s) { return (uint32_t)((s - x.c_begin) % kASlots) * (uint32_t)kHalf; }

// Fragments of sub-block S of a stage: activations at ring offset aoff, weights
// in ring slot PW (the stage index mod 4).
template <int S> __device__ __forceinline__ v4i frag_a(const uint8_t* lds, const Ctx& x, uint32_t aoff, int i)
{
    return *reinterpret_cast<const v4i*>(lds + (S? x.oa0 ^ 32u : x.oa0) + aoff + i * 2048);
}
template <int PW, int S> __device__ __forceinline__ v4i frag_w(const uint8_t* lds, const Ctx& x, int j, int plane)
{
    return *reinterpret_cast<const v4i*>(lds + (S? x.ow0 ^ 32u : x.ow0) + PW * kHalf + j * 2048 + plane * kPlane);
}

// Byte offset of the 1 KB tile of rows r0..r0+15 (r0 a multiple of 16) and
// stage c in a tiled plane (pixhip_internal.h, tiled_offset).
__device__ __forceinline__ uint32_t tile_at(const Ctx& x, int r0, int c)
{
    return ((uint32_t)(r0 >> 4) * (uint32_t)(x.K >> 6) + (uint32_t)c) * 1024u;
}

// DMAs of stage c: the wave's activation chunks are wave and wave+8 (16 token
// rows each), into the activation ring; its weight chunks are the 16 rows of
// features 16*wave .. of the hi and the lo plane, into weight slot c % 4 (the
// waves of group 0 load its features 0-63, those of group 1 features 64-127).
__device__ __forceinline__ void issue_act(const Ctx& x, uint8_t* lds, int c)
{
    const int w = x.wave;
    uint8_t* slot = lds + a_off(x,c);
    dma(x.rx,slot + w * kChunk,x.vo_tile,tile_at(x,x.m0 + w * 16,c));
    dma(x.rx,slot + (w + 8) * kChunk,x.vo_tile,tile_at(x,x.m0 + (w + 8) * 16,c));
}
template <int PW> __device__ __forceinline__ void issue_w(const Ctx& x, uint8_t* lds, int c)
{
    const int w = x.wave;
    dma(x.rwh,lds + kWRing + PW * kHalf + w * kChunk,x.vo_tile,tile_at(x,x.n0 + w * 16,c));
    dma(x.rwl,lds + kWRing + PW * kHalf + kPlane + w * kChunk,x.vo_tile,tile_at(x,x.n0 + w * 16,c));
}

// DMA of super-block b's epilogue inputs into `sc`: chunk q of the 13 (2 for
// Q6_K) is issued by wave q % 8.
template <bool Q5> __device__ __forceinline__ void issue_scale_chunk(const Args& g, const Ctx& x, int b, int chunk, uint8_t* sc)
{
    const uint32_t lane = lane_id();
    if (chunk == 0) {
        dma(x.rxd,sc,16u * lane,(uint32_t)(b * g.Mpad + x.m0) * 4u);
    } else if (chunk == 1) {
        dma(x.rwd,sc + kChunk,16u * (lane & 31),(uint32_t)(b * g.Npad + x.n0) * 4u);  // lanes 32..63 repeat 0..31
    } else if (Q5 && chunk < 10) {
        // 32 token rows of 16 fp16 sums, one 1 KB block of the tiled bs plane
        dma(x.rxbs,sc + chunk * kChunk,16u * lane,((uint32_t)((x.m0 >> 5) + chunk - 2) * (uint32_t)(x.K >> 8) + b) * 1024u);
    } else if (Q5 && chunk < 12) {
        dma(x.rwmn,sc + chunk * kChunk,16u * lane,(uint32_t)(b * g.Npad + x.n0 + (chunk - 10) * 64) * 16u);
    } else if (Q5 && chunk == 12) {
        dma(x.rwdm,sc + chunk * kChunk,16u * (lane & 31),(uint32_t)(b * g.Npad + x.n0) * 4u);
    }
}
template <bool Q5> __device__ __forceinline__ void issue_scales(const Args& g, const Ctx& x, int b, uint8_t* sc)
{
    if (x.wave < scale_chunks<Q5>()) issue_scale_chunk<Q5>(g,x,b,x.wave,sc);
    if (x.wave + 8 < scale_chunks<Q5>()) issue_scale_chunk<Q5>(g,x,b,x.wave + 8,sc);
}

// MFMAs of sub-block S (0 or 1 within its stage) from R, in the order hi00,
// hi10, lo00, lo10, hi01, hi11, lo01, lo11 (plane, token tile, feature tile):
// each weight fragment is free after two MFMAs.  When READ, the fragments of
// the next sub-block (sub-block 1-S of the stage at activation offset naoff and
// weight slot NPW) load as registers free up: its activations into the other
// half of R.a (at the start when EARLY, else after f0), each weight fragment
// after its last use here, so every load has at least four MFMAs to land.
// f0, f1 and f2 run after the fourth, sixth and eighth MFMA (a barrier and the
// DMAs of an interval go there, with MFMAs queued while the wave waits; the
// loads of a next stage follow f0).
struct Nop {
    __device__ __forceinline__ void operator()() const {}
};
template <bool FRESH, int S, bool READ, bool EARLY, int NPW, class F0 = Nop, class F1 = Nop, class F2 = Nop>
__device__ __forceinline__ void sub_block(Acc& acc, Opnd& R, const uint8_t* lds, const Ctx& x, uint32_t naoff, F0 f0 = {}, F1 f1 = {},
                                          F2 f2 = {})
{
    constexpr int NS = 1 - S;
    const v16i z = {};
    if constexpr (READ && EARLY) {
        R.a[NS][0] = frag_a<NS>(lds,x,naoff,0);
        R.a[NS][1] = frag_a<NS>(lds,x,naoff,1);
    }
    __builtin_amdgcn_sched_barrier(0);
    acc.hi[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][0],R.h[0],FRESH? z : acc.hi[0][0],0,0,0);
    acc.hi[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][1],R.h[0],FRESH? z : acc.hi[1][0],0,0,0);
    acc.lo[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][0],R.l[0],FRESH? z : acc.lo[0][0],0,0,0);
    acc.lo[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][1],R.l[0],FRESH? z : acc.lo[1][0],0,0,0);
    __builtin_amdgcn_sched_barrier(0);
    f0();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (READ) {
        if constexpr (!EARLY) {
            R.a[NS][0] = frag_a<NS>(lds,x,naoff,0);
            R.a[NS][1] = frag_a<NS>(lds,x,naoff,1);
        }
        R.h[0] = frag_w<NPW,NS>(lds,x,0,0);
        R.l[0] = frag_w<NPW,NS>(lds,x,0,1);
    }
    __builtin_amdgcn_sched_barrier(0);
    acc.hi[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][0],R.h[1],FRESH? z : acc.hi[0][1],0,0,0);
    acc.hi[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][1],R.h[1],FRESH? z : acc.hi[1][1],0,0,0);
    __builtin_amdgcn_sched_barrier(0);
    f1();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (READ) R.h[1] = frag_w<NPW,NS>(lds,x,1,0);
    __builtin_amdgcn_sched_barrier(0);
    acc.lo[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][0],R.l[1],FRESH? z : acc.lo[0][1],0,0,0);
    acc.lo[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(R.a[S][1],R.l[1],FRESH? z : acc.lo[1][1],0,0,0);
    __builtin_amdgcn_sched_barrier(0);
    f2();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (READ) R.l[1] = frag_w<NPW,NS>(lds,x,1,1);
    __builtin_amdgcn_sched_barrier(0);
}

template <int NPW> __device__ __forceinline__ void read_all(Opnd& R, const uint8_t* lds, const Ctx& x, uint32_t naoff)
{
    __asm__ volatile("" ::: "memory");  // not hoisted into a preceding epilogue
#pragma unroll
    for (int i = 0; i < 2; i++) {
        R.a[0][i] = frag_a<0>(lds,x,naoff,i);
        R.h[i] = frag_w<NPW,0>(lds,x,i,0);
        R.l[i] = frag_w<NPW,0>(lds,x,i,1);
    }
}

// The fp32 epilogue of super-block b for tile (I, J): y += yd * (wd*S - wdm*Mn)
// (the integer-sum variant stores S, and Mn for Q5_K, instead).
template <bool Q5, bool SUMS, int I, int J>
__device__ __forceinline__ void sb_epilogue(const Args& g, const Ctx& x, int b, Acc& acc, const uint8_t* __restrict__ sc)
{
    // The memory clobber keeps this tile's LDS reads (and the MFMA that
    // consumes them) from being hoisted above the previous tile's epilogue.
    __asm__ volatile("" ::: "memory");
    const uint32_t ln = lane_id();
    const int lg = (int)(ln >> 5), lr = (int)(ln & 31);
    const int col = x.wn * 64 + J * 32 + lr;           // feature within the tile
    const int row0 = x.wm * 64 + I * 32 + 4 * lg;      // first token row of this lane (rows row0 + 8q + e)
    v16f mt = {};
    if constexpr (Q5) {
        const v16f fzero = {};
        const v8h mnB = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotMn + col));
        const v8h bsA = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotBs + 2 * (x.wm * 64 + I * 32 + lr) + lg));
        mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA,mnB,fzero,0,0,0);
    }
    if constexpr (SUMS) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = x.m0 + row0 + 8 * (r >> 2) + (r & 3);
            const int n = x.n0 + col;
            if (m < g.M && n < g.N) {
                const size_t o = ((size_t)m * g.N + n) * (x.K / PIX_QK) + b;
                g.sums[o] = acc.hi[I][J][r] * 64 + acc.lo[I][J][r];
                if constexpr (Q5) g.mins[o] = (int32_t)mt[r];
            }
        }
    } else {
        const float* syd = reinterpret_cast<const float*>(sc + 16 * kSlotYd);
        const float wd = reinterpret_cast<const float*>(sc + 16 * kSlotWd)[col];
        const float nwm = Q5? -reinterpret_cast<const float*>(sc + 16 * kSlotWdm)[col] : 0.0f;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            __asm__ volatile("" ::: "memory");  // one float4 of yd at a time
            const float4 t4 = *reinterpret_cast<const float4*>(syd + row0 + 8 * q4);
            const float yq[4] = {t4.x,t4.y,t4.z,t4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * q4 + e;
                const float t = (float)(acc.hi[I][J][r] * 64 + acc.lo[I][J][r]) * wd;
                acc.y[I][J][r] = __builtin_fmaf(yq[e],Q5? __builtin_fmaf(mt[r],nwm,t) : t,acc.y[I][J][r]);
            }
        }
        // Pins the update here: sunk towards the next use of y (a super-block
        // later) it would keep this super-block's integer sums live next to
        // the next one's.
        __asm__ volatile("" : "+v"(acc.y[I][J]));
    }
}

// The fp32 epilogue of super-block b for the wave's four tiles, arranged for
// latency: every LDS read it needs is issued first; the integer sums of all
// four tiles become t = S * wd (the hi/lo registers are free afterwards,
// until the next super-block's first MFMAs); the four minimum-term MFMAs are
// issued back to back; then y += yd * (t - wdm * Mn).
template <bool Q5>
__device__ __forceinline__ void epilogue_y(const Ctx& x, Acc& acc, const uint8_t* __restrict__ sc)
{
    __asm__ volatile("" ::: "memory");
    const uint32_t ln = lane_id();
    const int lg = (int)(ln >> 5), lr = (int)(ln & 31);
    const float* syd = reinterpret_cast<const float*>(sc + 16 * kSlotYd);
    float wd[2], nwm[2] = {0.0f,0.0f};
    v8h mnB[2], bsA[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = x.wn * 64 + j * 32 + lr;
        wd[j] = reinterpret_cast<const float*>(sc + 16 * kSlotWd)[col];
        if constexpr (Q5) {
            nwm[j] = -reinterpret_cast<const float*>(sc + 16 * kSlotWdm)[col];
            mnB[j] = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotMn + col));
        }
    }
    if constexpr (Q5) {
#pragma unroll
        for (int i = 0; i < 2; i++) bsA[i] = *reinterpret_cast<const v8h*>(sc + 16 * (kSlotBs + 2 * (x.wm * 64 + i * 32 + lr) + lg));
    }
    float4 yd[4];  // token rows row0 + 8q .. +3 of the first token tile
    const int row0 = x.wm * 64 + 4 * lg;
#pragma unroll
    for (int q = 0; q < 4; q++) yd[q] = *reinterpret_cast<const float4*>(syd + row0 + 8 * q);
    v16f t[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) t[i][j][r] = (float)(acc.hi[i][j][r] * 64 + acc.lo[i][j][r]) * wd[j];
    const v16f fzero = {};
    v16f mt[2];
    if constexpr (Q5) {
#pragma unroll
        for (int j = 0; j < 2; j++) mt[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA[0],mnB[j],fzero,0,0,0);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        if (i == 1) {
            if constexpr (Q5) {
#pragma unroll
                for (int j = 0; j < 2; j++) mt[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA[1],mnB[j],fzero,0,0,0);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) yd[q] = *reinterpret_cast<const float4*>(syd + row0 + 32 + 8 * q);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float yq[4] = {yd[q].x,yd[q].y,yd[q].z,yd[q].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q + e;
                    acc.y[i][j][r] = __builtin_fmaf(yq[e],Q5? __builtin_fmaf(mt[j][r],nwm[j],t[i][j][r]) : t[i][j][r],acc.y[i][j][r]);
                }
            }
            __asm__ volatile("" : "+v"(acc.y[i][j]));
        }
    }
}

template <bool Q5, bool SUMS>
__device__ __forceinline__ void epilogue(const Args& g, const Ctx& x, int b, Acc& acc, const uint8_t* sc)
{
    if constexpr (!SUMS) {
        epilogue_y<Q5>(x,acc,sc);
    } else {
        // One tile at a time (the integer-sum variant is a test path).
        sb_epilogue<Q5,SUMS,0,0>(g,x,b,acc,sc);
        __builtin_amdgcn_sched_barrier(0);
        sb_epilogue<Q5,SUMS,0,1>(g,x,b,acc,sc);
        __builtin_amdgcn_sched_barrier(0);
        sb_epilogue<Q5,SUMS,1,0>(g,x,b,acc,sc);
        __builtin_amdgcn_sched_barrier(0);
        sb_epilogue<Q5,SUMS,1,1>(g,x,b,acc,sc);
    }
}

// The schedule.  K advances in 64-value stages; the waves synchronise once per
// interval of two stages.  Group 0 (waves 0-3, features 0-63 of the tile)
// works on stages C0+2k and C0+2k+1 in interval k; group 1 (waves 4-7,
// features 64-127) runs one stage behind, on C0+2k-1 and C0+2k.  So the two
// waves of a SIMD (one of each group) finish a super-block at different points
// of an interval: group 0's super-block epilogue (vector ALU) runs at the start
// of the interval while group 1 issues MFMAs, group 1's in its middle while
// group 0 does.
//
// Between barriers k-1 and k the activation ring holds stages C0+2k-1 ..
// C0+2k+1 (read in interval k) and C0+2k+2, C0+2k+3 (landed by barrier k-1);
// each group's weight slots hold its two stages of interval k and two of
// interval k+1.  After barrier k every wave issues its share of interval k+2:
// activations C0+2k+4, C0+2k+5 into the slots of C0+2k-1 and C0+2k (read for
// the last time in interval k) and its weight rows of the same stages (group
// 0) or C0+2k+3, C0+2k+4 (group 1), into the slots of the group's stages of
// interval k.  Everything a wave issues in an interval has landed before the
// barrier that ends it.  The epilogue inputs of super-block b are read in
// interval 2b+2 (relative to C0) and those of b+1 loaded in interval 2b+3.
//
// Group 0's barriers sit in its stages C0+2k+1, group 1's in C0+2k; in a
// wave's barrier stage s the interval's DMAs are activations s+3, s+4 (group
// 0) or s+4, s+5 (group 1) and weights s+3, s+4.
template <bool SUMS> __device__ __forceinline__ void wait_all()
{
    wait_vmcnt<0>();
    wait_lgkm0();
}

// Part PART (0..2) of the DMAs after the barrier in stage s (weight slot PW =
// s % 4): 0 the activations of the interval's first stage, 1 those of the
// second and the weights of the first, 2 the weights of the second and, in
// the interval that loads them, the next super-block's epilogue inputs.
template <bool Q5, int PW, int PART>
__device__ __forceinline__ void window_dma(const Args& g, const Ctx& x, uint8_t* lds, int s, uint8_t* sc)
{
    const int a0 = s + 3 + (x.lag? 1 : 0), w0 = s + 3;
    if constexpr (PART == 0) {
        if (a0 < x.nchunks) issue_act(x,lds,a0);
    } else if constexpr (PART == 1) {
        if (a0 + 1 < x.nchunks) issue_act(x,lds,a0 + 1);
        if (w0 < x.nchunks) issue_w<(PW + 3) % 4>(x,lds,w0);
    } else {
        if (w0 + 1 < x.nchunks) issue_w<PW>(x,lds,w0 + 1);
        // Super-block s / 4 (the one stage s belongs to) is loaded in the
        // interval after barrier 2b+2 relative to C0: group 0's barrier stage
        // C0+4b+5, group 1's C0+4b+4; the first super-block comes with the
        // prologue.
        if (PW == (x.lag? 0 : 1) && s - PW > x.c_begin) issue_scales<Q5>(g,x,s / kSBC,sc);
    }
}

// One stage s of a wave: sub-block 0 from registers (reading sub-block 1),
// then sub-block 1 (reading sub-block 0 of stage s+1 when READ_NEXT) with the
// hooks f0, f1, f2.
template <bool FRESH, bool READ_NEXT, bool BARRIER, int PW, class F0 = Nop, class F1 = Nop, class F2 = Nop>
__device__ __forceinline__ void stage(Acc& acc, Opnd& R, const uint8_t* lds, const Ctx& x, int s, F0 f0 = {}, F1 f1 = {}, F2 f2 = {})
{
    sub_block<FRESH,0,true,true,PW>(acc,R,lds,x,a_off(x,s));
    sub_block<false,1,READ_NEXT,!BARRIER,(PW + 1) % 4>(acc,R,lds,x,READ_NEXT? a_off(x,s + 1) : 0u,f0,f1,f2);
}

// Stage s of a super-block (PW = s % 4); group 0 has its barrier in stages 1
// and 3 of a super-block, group 1 in stages 0 and 2.  The barrier comes after
// the first four MFMAs of sub-block 1 (issued from registers, so the matrix
// core has work queued while the wave waits), the interval's DMAs spread over
// the rest of the sub-block.
template <bool Q5, bool SUMS, bool FRESH, bool READ_NEXT, int PW>
__device__ __forceinline__ void sb_stage(const Args& g, Acc& acc, Opnd& R, uint8_t* lds, const Ctx& x, int s, uint8_t* sc)
{
    const bool here = x.lag == ((PW & 1) == 0);  // (wave-uniform)
    auto f0 = [&]() {
        if (here) {
            wait_all<SUMS>();
            __builtin_amdgcn_s_barrier();
            window_dma<Q5,PW,0>(g,x,lds,s,sc);
        }
    };
    auto f1 = [&]() {
        if (here) window_dma<Q5,PW,1>(g,x,lds,s,sc);
    };
    auto f2 = [&]() {
        if (here) window_dma<Q5,PW,2>(g,x,lds,s,sc);
    };
    // (whether this wave's barrier is in this stage is only known at run time:
    // the next stage's activations load after f0 in either case)
    stage<FRESH,READ_NEXT,true,PW>(acc,R,lds,x,s,f0,f1,f2);
}

// One super-block at stage s0 (R holds sub-block 0 of s0): stages s0 .. s0+3,
// the epilogue (group 0: at the start of the interval its barrier in s0+3
// opens; group 1: in the middle of the interval its barrier in s0+2 opened),
// then the first fragments of the next super-block (both groups: in the same
// interval as the epilogue).
template <bool Q5, bool SUMS>
__device__ __forceinline__ void super_block(const Args& g, Acc& acc, Opnd& R, uint8_t* lds, const Ctx& x, int s0, uint8_t* sc)
{
    sb_stage<Q5,SUMS,true,true,0>(g,acc,R,lds,x,s0,sc);
    sb_stage<Q5,SUMS,false,true,1>(g,acc,R,lds,x,s0 + 1,sc);
    sb_stage<Q5,SUMS,false,true,2>(g,acc,R,lds,x,s0 + 2,sc);
    sb_stage<Q5,SUMS,false,false,3>(g,acc,R,lds,x,s0 + 3,sc);
    // The epilogue runs at a raised wave priority: it is the wave's critical
    // path, while the other wave of its SIMD has MFMAs to issue meanwhile
    // (1-1.5% at the DiT FFN shape).
    __builtin_amdgcn_s_setprio(2);
    epilogue<Q5,SUMS>(g,x,s0 / kSBC,acc,sc);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    // Unconditional (after the last super-block it reads a stale slot,
    // unused): a conditional read would keep the consumed fragments live
    // through the epilogue.
    read_all<0>(R,lds,x,a_off(x,s0 + 4));
}

template <bool Q5, bool SUMS>
__global__ __launch_bounds__(kThreads,1) void gemm_kq_kernel(Args g)
{
    constexpr int kScale = scale_bytes<Q5>();
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kScaleAt + kScale];
    uint8_t* const sc = lds + kScaleAt;

    // Whole tiles first (XCD-remapped), then the split tiles' pieces in launch
    // order (consecutive pieces land on different XCDs).
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
    x.wm = x.wave % 4;
    x.wn = x.wave / 4;
    x.lag = x.wn != 0;
    x.K = g.K;
    {
        // lane l reads row l%32, piece (l/32) ^ ((l%32 >> 2) & 3) of sub-block 0; sub-block 1 is that ^ 2
        const uint32_t lane = threadIdx.x & 63;
        const uint32_t lr = lane & 31, lg = lane >> 5;
        const uint32_t cp0 = lr * 64 + 16 * (lg ^ ((lr >> 2) & 3));
        x.oa0 = (uint32_t)(x.wm * 64 * 64) + cp0;
        x.ow0 = (uint32_t)(kWRing + x.wn * 64 * 64) + cp0;
        // DMA lane l lands at LDS position l of a 1 KB chunk: row l/4, piece
        // position l%4, which holds logical piece (l%4) ^ ((l/16)&3) of the row
        x.vo_tile = 16u * ((lane & ~3u) | ((lane & 3) ^ ((lane >> 4) & 3)));
    }
    x.c_begin = piece? split * g.split_chunks : 0;
    x.nchunks = piece? min(x.c_begin + g.split_chunks,g.K / kKC) : g.K / kKC;
    {
        const size_t mp = (size_t)g.Mpad, np = (size_t)g.Npad, K = (size_t)g.K, nblk = K / PIX_QK;
        x.rx = make_rsrc(g.xq,mp * K);
        x.rxd = make_rsrc(g.xdT,nblk * mp * 4);
        x.rwh = make_rsrc(g.whi,np * K);
        x.rwl = make_rsrc(g.wlo,np * K);
        x.rwd = make_rsrc(g.wdT,nblk * np * 4);
        x.rxbs = make_rsrc(Q5? (const void*)g.xbs : (const void*)g.xq,Q5? mp * (K / 16) * 2 : 0);
        x.rwmn = make_rsrc(Q5? (const void*)g.wmn : (const void*)g.xq,Q5? nblk * np * 16 : 0);
        x.rwdm = make_rsrc(Q5? (const void*)g.wdm : (const void*)g.xq,Q5? nblk * np * 4 : 0);
    }

    // (hi and lo are written fresh by the first MFMAs of every super-block.)
    Acc acc;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc.y[i][j] = v16f{};

    const int C0 = x.c_begin, C = x.nchunks;  // C0 is a multiple of kSBC; C - C0 >= kSBC
    // Prologue: intervals 0 and 1 (activations C0 .. C0+3; weights C0 ..
    // C0+3 for group 0, C0 .. C0+2 for group 1) and the first super-block's
    // epilogue inputs.  Interval 0's chunks are issued first: before the
    // prologue barrier they have landed (at most the 8 DMAs of interval 1
    // pending), interval 1's land before barrier 0.
    const bool lag = x.lag;
    issue_act(x,lds,C0);
    issue_act(x,lds,C0 + 1);
    issue_w<0>(x,lds,C0);
    if (!lag) issue_w<1>(x,lds,C0 + 1);
    issue_scales<Q5>(g,x,C0 / kSBC,sc);
    issue_act(x,lds,C0 + 2);
    issue_act(x,lds,C0 + 3);
    if (lag) issue_w<1>(x,lds,C0 + 1);
    issue_w<2>(x,lds,C0 + 2);
    if (!lag) issue_w<3>(x,lds,C0 + 3);
    if constexpr (SUMS) wait_vmcnt<0>();  // (spill traffic would join the count)
    else wait_vmcnt<8>();
    __builtin_amdgcn_s_barrier();
    Opnd R;
    read_all<0>(R,lds,x,a_off(x,C0));
    for (int s0 = C0; s0 < C; s0 += kSBC) super_block<Q5,SUMS>(g,acc,R,lds,x,s0,sc);

    if constexpr (!SUMS) {
        const uint32_t ln = lane_id();
        const int lr = (int)(ln & 31), lg = (int)(ln >> 5);
        if (piece) {
            // Split-K: this K range's fp32 partial tile; the reduce kernel adds
            // the ranges in order and applies bias, ldy and offset.
            float* part = g.part + ((size_t)split * split_tiles + pidx % split_tiles) * (kBM * kBN);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    float* col = part + x.wn * 64 + j * 32 + lr;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int lm = x.wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                        col[(size_t)lm * kBN] = acc.y[i][j][r];
                    }
                }
        } else {
            // Bias loaded once per feature column (clamped index) and drained
            // before the stores; the output is written once and stored
            // non-temporally, so it does not push the operands out of the
            // last-level cache.
            const int mrow0 = x.m0 + x.wm * 64, ncol0 = x.n0 + x.wn * 64;
            float bv[2];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = g.bias? g.bias[min(ncol0 + j * 32 + lr,g.N - 1)] : 0.0f;
            wait_vmcnt<0>();
            const bool full = mrow0 + 64 <= g.M && ncol0 + 64 <= g.N;
#pragma unroll
            for (int j = 0; j < 2; j++) {
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
}

// For the split tiles: y[yoff + m*ldy + n] = sum over the splits, in order, of
// the partial tiles, + bias[n].  Workgroup (tile t, slice q) of 256 threads
// covers kReduceSlice elements of the tile, 4 consecutive features per thread.
constexpr int kReduceSlice = 1024, kReduceSlices = kBM * kBN / kReduceSlice;
__global__ __launch_bounds__(256) void kq_reduce_kernel(Args g)
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

size_t round_up_kq(size_t v, size_t m) { return (v + m - 1) / m * m; }

template <bool Q5, bool SUMS> hipError_t launch_kq(Args g, size_t mpad, size_t npad, hipStream_t s)
{
    g.tiles_m = (int)((g.M + kBM - 1) / kBM);
    g.tiles_n = (int)((g.N + kBN - 1) / kBN);
    if (mpad < round_up_kq((size_t)g.M,kBM) || npad < round_up_kq((size_t)g.N,kBN) || g.K % PIX_QK) return hipErrorInvalidValue;
    // Buffer offsets are 32-bit: every operand plane must stay below 2 GiB.
    const size_t lim = (size_t)1 << 31;
    const size_t scales = ((size_t)g.K / PIX_QK) * (npad > mpad? npad : mpad) * 16;
    if (mpad * g.K >= lim || npad * g.K >= lim || scales >= lim || mpad * (g.K / 16) * 2 >= lim) return hipErrorInvalidValue;
    g.Mpad = (int)mpad;
    g.Npad = (int)npad;
    const int ntiles = g.tiles_m * g.tiles_n;
    if (!ntiles) return hipSuccess;
    g.splits = SUMS? 1 : gemm_split_plan((size_t)g.M,(size_t)g.N,(size_t)g.K,g.full_tiles,g.split_chunks);
    if (g.splits == 1 || !g.part) {
        g.splits = 1;
        g.full_tiles = ntiles;
        g.split_chunks = g.K / kKC;
    }
    const int split_tiles = ntiles - g.full_tiles;
    gemm_kq_kernel<Q5,SUMS><<<dim3(g.full_tiles + split_tiles * g.splits),dim3(kThreads),0,s>>>(g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !split_tiles) return e;
    static_assert(kReduceSlice == 4 * 256, "reduce slice: 256 threads x 4 features");
    kq_reduce_kernel<<<dim3(split_tiles * kReduceSlices),dim3(256),0,s>>>(g);
    return hipGetLastError();
}

Args kq_args(const Act8K& a, size_t M, size_t N, size_t K)
{
    Args g = {};
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.xq = a.qs;
    g.xdT = a.d;
    g.xbs = a.bs;
    return g;
}

}  // namespace

hipError_t launch_gemm_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s)
{
    Args g = kq_args(a,M,N,K);
    g.part = part;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdm = w.dm; g.wmn = w.mn;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch_kq<true,false>(g,a.mpad,w.npad,s);
}

hipError_t launch_gemm_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s)
{
    Args g = kq_args(a,M,N,K);
    g.part = part;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch_kq<false,false>(g,a.mpad,w.npad,s);
}

hipError_t launch_sums_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, int32_t* scaled, int32_t* mins,
                            hipStream_t s)
{
    Args g = kq_args(a,M,N,K);
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdm = w.dm; g.wmn = w.mn;
    g.sums = scaled; g.mins = mins;
    return launch_kq<true,true>(g,a.mpad,w.npad,s);
}

hipError_t launch_sums_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    Args g = kq_args(a,M,N,K);
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.sums = sums;
    return launch_kq<false,true>(g,a.mpad,w.npad,s);
}

}  // namespace pixhip
