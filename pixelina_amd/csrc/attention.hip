// Attention: tensor_attention (src/tensor.cpp:347-427) and vulkan_attention
// (src/backend_vulkan.cpp:1318-1340) on bf16 MFMA (gfx950), head sizes up to
// 512 (up to 128 in the kernel below, 129..512 in attn_wide_kernel).
//
// Numerics: the reference works in fp32 (scores = dot * 1/sqrt(dim), exp(score
// - max), probabilities p / sum, out += p * v).  Here every fp32 operand x of
// the two products is split into bf16 halves hi = bf16(x), lo = bf16(x - hi),
// and each product a*b is taken as hi_a*hi_b + hi_a*lo_b + lo_a*hi_b on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation (the dropped lo*lo term and
// the rounding of lo leave about 2^-16 relative per product), so the result
// stays within the fp32 reference's tolerance at three times the bf16 MFMA
// work, and far above what fp32 MFMAs would give.  Softmax is the online form
// (running maximum and sum per query, output rescaled per key tile), in fp32.
//
// Layout: a split pass writes K as bf16 planes [head][key][D] and V transposed,
// [head][D][key], with the keys of each 16-key group permuted (bits 2 and 3
// swapped) so that the operand a lane needs for P*V is 16 contiguous bytes (D
// = 64, 128, 256, 384 or 512: the head size rounded up, zero-padded).  Q, read
// by one workgroup per row, is split in the kernel.
//
// Kernel: a workgroup of 8 waves owns 256 queries of one head (32 per wave)
// and streams 64-key tiles of K and V^T (both planes) through a 2-stage LDS
// ring with buffer_load ... lds.  Per 32-key half tile each wave computes S^T
// = K * Q^T (keys as MFMA rows, its 32 queries as columns, so each lane owns
// one query: the softmax statistics and the output rescale stay in the lane),
// then O^T += V^T * P^T, where the P^T operand is the lane's own S^T results
// converted to bf16 -- the key order the S^T output layout gives is matched by
// the V^T permutation above.  Q stays in registers for the whole key loop.
#include <math.h>

#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"

#define PIX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace pixhip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t ARsrc;

constexpr int kAQ = 256;  // queries per workgroup
constexpr int kAK = 64;   // keys per tile
constexpr int kAWaves = 8, kAThreads = 64 * kAWaves;
constexpr float kLog2e = 1.44269504088896340736f;

__device__ __forceinline__ uint32_t bf16_rne(float x)
{
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// x -> (hi, lo) bf16 bit patterns with x ~ hi + lo, for every fp32 value: a
// finite x that rounds past the largest bf16 keeps hi truncated (finite) and
// the rest in lo; Inf and NaN travel in hi alone (lo = 0), so a product with
// them gives what the fp32 product gives instead of NaN from Inf - Inf.
__device__ __forceinline__ void split2(float x, uint32_t& hi, uint32_t& lo)
{
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        hi = (u & 0x007FFFFFu)? 0x7FC0u | ((u >> 16) & 0x8000u) : u >> 16;
        lo = 0;
        return;
    }
    uint32_t h = bf16_rne(x);
    if ((h & 0x7F80u) == 0x7F80u) h = u >> 16;
    hi = h;
    lo = bf16_rne(x - __uint_as_float(h << 16));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two values rounded to bf16 (nearest even) by v_cvt_pk_bf16_f32, a in the
// low half.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b)
{
    const bf16x2 h = {(__bf16)a,(__bf16)b};
    return __builtin_bit_cast(uint32_t,h);
}

// ---------------------------------------------------------------- split pass

// src [n][stride] fp32, head h's values at h*dim; planes [heads][npad][D] bf16
// (hi, lo), zero beyond n and dim.  One thread per (head, row, 8 values).
__global__ __launch_bounds__(256) void attn_split_rows(const float* __restrict__ src, size_t n, size_t stride, int heads, int dim,
                                                        int D, size_t npad, bool vec, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo)
{
    const size_t groups = (size_t)D / 8;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)heads * npad * groups) return;
    const int g = (int)(idx % groups);
    const size_t row = (idx / groups) % npad;
    const int h = (int)(idx / (groups * npad));
    float x[8];
    const float* p = src + row * stride + (size_t)h * dim + 8 * g;
    if (vec && row < n && 8 * g < dim) {  // 16-byte aligned rows, dim a multiple of 8
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = row < n && 8 * g + i < dim? p[i] : 0.0f;
    }
    u32x4 vh, vl;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t h0, l0, h1, l1;
        split2(x[2 * i],h0,l0);
        split2(x[2 * i + 1],h1,l1);
        vh[i] = h0 | (h1 << 16);
        vl[i] = l0 | (l1 << 16);
    }
    const size_t o = ((size_t)h * npad + row) * D + 8 * g;
    *reinterpret_cast<u32x4*>(hi + o) = vh;
    *reinterpret_cast<u32x4*>(lo + o) = vl;
}

// Position of key j (0..15) of a 16-key group in a V^T row: j = 8a + 4b + c is
// stored at 8b + 4a + c.
__device__ __forceinline__ int vt_pos(int j)
{
    return (((j >> 2) & 1) << 3) | (((j >> 3) & 1) << 2) | (j & 3);
}

// src [n][stride] -> planes [heads][D][npad] bf16 (hi, lo), keys permuted
// within 16-key groups, zero beyond n and dim (npad a multiple of 64).  One
// thread per (head, 64-key group, d), d fastest (coalesced reads along a
// source row); its 64 keys are one whole 128-byte line of each plane's row
// (16 keys per thread wrote quarter lines: 69 us per DiT call, ~15 us more).
__global__ __launch_bounds__(256) void attn_split_vt(const float* __restrict__ src, size_t n, size_t stride, int heads, int dim,
                                                      int D, size_t npad, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo)
{
    const size_t kg = npad / 64;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)heads * kg * D) return;
    const int d = (int)(idx % D);
    const size_t g64 = (idx / D) % kg;
    const int h = (int)(idx / ((size_t)D * kg));
    float x[64];
#pragma unroll
    for (int j = 0; j < 64; j++) {
        const size_t key = g64 * 64 + j;
        x[j] = key < n && d < dim? src[key * stride + (size_t)h * dim + d] : 0.0f;
    }
    const size_t o = ((size_t)h * D + d) * npad + g64 * 64;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t bh[16], bl[16];
#pragma unroll
        for (int j = 0; j < 16; j++) split2(x[16 * g + j],bh[vt_pos(j)],bl[vt_pos(j)]);
        u32x4 w[4];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i / 4][i % 4] = bh[2 * i] | (bh[2 * i + 1] << 16);
#pragma unroll
        for (int i = 0; i < 8; i++) w[2 + i / 4][i % 4] = bl[2 * i] | (bl[2 * i + 1] << 16);
        *reinterpret_cast<u32x4*>(hi + o + 16 * g) = w[0];
        *reinterpret_cast<u32x4*>(hi + o + 16 * g + 8) = w[1];
        *reinterpret_cast<u32x4*>(lo + o + 16 * g) = w[2];
        *reinterpret_cast<u32x4*>(lo + o + 16 * g + 8) = w[3];
    }
}

// ---------------------------------------------------------------- main kernel

struct AttnArgs {
    const float* q;                      // [rows][channels]
    const uint16_t *kh, *kl, *vh, *vl;  // split planes of K and V^T
    float* out;                          // [rows][channels]
    int rows, keys_pad;
    int heads, kv_group, dim, channels;
    int qb, qe, key_end, causal, qoff;  // this range (query rows [qb, qe))
    int tiles_q;
    float scale;
    // Key-split tail: units (head, query tile) full.. run as `splits` pieces of
    // their key tiles each, writing unnormalised outputs and the running
    // maximum and sum to `part` ([piece][unit - full][256 queries][D + 4]:
    // the D outputs, the maximum, the sum, two unused), which attn_combine
    // merges.
    int full, tail, splits;
    float* part;
};

template <typename T> __device__ __forceinline__ T lds_read(const uint8_t* p)
{
    return *reinterpret_cast<const T*>(p);
}

__device__ __forceinline__ void adma(ARsrc r, uint8_t* lds_uniform, uint32_t voff, uint32_t soff)
{
    __builtin_assume(lds_uniform != nullptr);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,PIX_LDS(lds_uniform),16,(int)voff,(int)soff,0,0);
}

template <int N> __device__ __forceinline__ void attn_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 16-byte piece swizzles (conflict-free ds_read_b128 of 32 rows at one logical
// piece): K rows of 2*D bytes, V^T rows of 128 bytes.
template <int D> __device__ __forceinline__ int swz_k(int r)
{
    return D == 128? (r & 15) : ((r >> 1) & 7);
}
__device__ __forceinline__ int swz_v(int r)
{
    return (r >> 1) & 7;
}

template <int D>
__global__ __launch_bounds__(kAThreads, 1) void attn_kernel(AttnArgs a)
{
    constexpr int PK = D / 8;            // 16-byte pieces per K row
    constexpr int PLANE = kAK * D * 2;   // bytes of one plane's tile (K: 64 rows x 2D; V^T: D rows x 128)
    constexpr int STAGE = 4 * PLANE;     // K hi, K lo, V hi, V lo
    constexpr int CHUNKS = STAGE / 1024;
    constexpr int PER_WAVE = CHUNKS / kAWaves;
    constexpr int KS = D / 16;           // k-steps of S^T
    constexpr int TD = D / 32;           // output dim tiles
    static_assert(PER_WAVE * kAWaves == CHUNKS, "stage DMAs split evenly");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

    const int bid = (int)blockIdx.x;
    const bool piece = bid >= a.full;
    const int pidx = bid - a.full;
    const int unit = piece? a.full + pidx % a.tail : bid;
    const int split = piece? pidx / a.tail : 0;
    const int head = unit / a.tiles_q, qt = unit % a.tiles_q;
    const int kvh = head / a.kv_group;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63), lr = lane & 31, hh = lane >> 5;
    const int q = a.qb + qt * kAQ + wave * 32 + lr;  // this lane's query row
    const bool live = q < a.qe;
    const int limit = !live? 1 : a.causal? min(a.key_end,a.qoff + q + 1) : a.key_end;
    const int q_last = min(a.qe,a.qb + (qt + 1) * kAQ) - 1;
    const int wg_limit = a.causal? min(a.key_end,a.qoff + q_last + 1) : a.key_end;
    const int all_tiles = (wg_limit + kAK - 1) / kAK;
    const int t0 = piece? split * all_tiles / a.splits : 0;
    const int t1 = piece? (split + 1) * all_tiles / a.splits : all_tiles;

    // Q fragments (B operand of S^T: lane = query, dims 16k + 8hh .. +7), split
    // here from fp32 (each query row is read by one workgroup only); rows
    // past the tensor read its last row (their outputs are not stored).
    bf16x8 qfh[KS], qfl[KS];
    {
        const float* qrow = a.q + (size_t)min(q,a.rows - 1) * a.channels + (size_t)head * a.dim;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            u32x4 vh, vl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = 16 * k + 8 * hh + 2 * i;
                uint32_t h0, l0, h1, l1;
                split2(d < a.dim? qrow[d] : 0.0f,h0,l0);
                split2(d + 1 < a.dim? qrow[d + 1] : 0.0f,h1,l1);
                vh[i] = h0 | (h1 << 16);
                vl[i] = l0 | (l1 << 16);
            }
            qfh[k] = __builtin_bit_cast(bf16x8,vh);
            qfl[k] = __builtin_bit_cast(bf16x8,vl);
        }
    }
    // the smallest key limit of the wave: tiles below it need no masking
    int wave_limit = limit;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) wave_limit = min(wave_limit,__shfl_xor(wave_limit,m));

    const size_t kplane = (size_t)a.keys_pad * D * 2;
    const ARsrc rk[2] = {__builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kh) + (size_t)kvh * a.keys_pad * D,(short)0,(int)kplane,
                                                           0x00020000),
                         __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kl) + (size_t)kvh * a.keys_pad * D,(short)0,(int)kplane,
                                                           0x00020000)};
    const ARsrc rv[2] = {__builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vh) + (size_t)kvh * a.keys_pad * D,(short)0,(int)kplane,
                                                           0x00020000),
                         __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vl) + (size_t)kvh * a.keys_pad * D,(short)0,(int)kplane,
                                                           0x00020000)};

    // DMA of key tile kt into stage `st`: chunk c = wave + 8i of the stage's
    // 4 planes; lane j of a chunk lands at chunk + 16j, which holds row r,
    // physical piece p of the plane, i.e. logical piece p ^ swizzle(r).
    auto issue = [&](int kt, int st) {
        uint8_t* base = lds + st * STAGE;
#pragma unroll
        for (int i = 0; i < PER_WAVE; i++) {
            const int c = wave + kAWaves * i;
            const int plane = c / (PLANE / 1024), ci = c % (PLANE / 1024);
            uint8_t* dst = base + plane * PLANE + ci * 1024;
            if (plane < 2) {
                const int r = ci * (1024 / (2 * D)) + lane / PK, p = lane % PK;
                const uint32_t off = (uint32_t)((kt * kAK + r) * D * 2 + 16 * (p ^ swz_k<D>(r)));
                adma(rk[plane],dst,off,0);
            } else {
                const int r = ci * 8 + lane / 8, p = lane % 8;
                const uint32_t off = (uint32_t)(((size_t)r * a.keys_pad + kt * kAK) * 2 + 16 * (p ^ swz_v(r)));
                adma(rv[plane - 2],dst,off,0);
            }
        }
    };

    v16f o[TD];
#pragma unroll
    for (int t = 0; t < TD; t++) o[t] = v16f{};
    // Running maximum (log2 units) and this lane's part of the sum (its 16 of
    // each 32 keys; the two lanes of a query combine at the end).  The
    // maximum is raised only when a half tile exceeds it by more than 8 (a
    // factor 256), so probabilities stay below 256 and the output rescale is
    // rare; output and sum share the maximum, so the final division is exact.
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;

    // S^T = K * Q^T for both 32-key halves of the tile in `st`: the two
    // halves' MFMA chains interleaved, each k-step's K fragments read while
    // the previous k-step's MFMAs run.
    auto score = [&](const uint8_t* st, v16f& s0, v16f& s1) {
        s0 = v16f{};
        s1 = v16f{};
        const int r0 = lr, r1 = 32 + lr;
        const uint8_t *h0 = st + r0 * (2 * D), *l0 = st + PLANE + r0 * (2 * D);
        const uint8_t *h1 = st + r1 * (2 * D), *l1 = st + PLANE + r1 * (2 * D);
        auto frag = [&](const uint8_t* row, int r, int k) { return lds_read<bf16x8>(row + 16 * ((2 * k + hh) ^ swz_k<D>(r))); };
        bf16x8 a0h = frag(h0,r0,0), a0l = frag(l0,r0,0), a1h = frag(h1,r1,0), a1l = frag(l1,r1,0);
#pragma unroll
        for (int k = 0; k < KS; k++) {
            bf16x8 n0h, n0l, n1h, n1l;
            if (k + 1 < KS) {
                n0h = frag(h0,r0,k + 1);
                n0l = frag(l0,r0,k + 1);
                n1h = frag(h1,r1,k + 1);
                n1l = frag(l1,r1,k + 1);
            }
            __builtin_amdgcn_sched_barrier(0);  // (the reads stay ahead of this k-step's MFMAs)
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0h,qfh[k],s0,0,0,0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1h,qfh[k],s1,0,0,0);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0h,qfl[k],s0,0,0,0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1h,qfl[k],s1,0,0,0);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0l,qfh[k],s0,0,0,0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1l,qfh[k],s1,0,0,0);
            __builtin_amdgcn_sched_barrier(0);
            if (k + 1 < KS) {
                a0h = n0h;
                a0l = n0l;
                a1h = n1h;
                a1l = n1l;
            }
        }
    };
    // Online softmax of one half (keys key0 + 8(r/4) + 4hh + r%4) -> P^T as
    // bf16 pairs for its two k-steps: hi = p rounded to nearest even, lo =
    // p - hi rounded likewise (six vector instructions per pair).
    auto softmax = [&](v16f& sv, int key0, uint32_t (&ph)[2][4], uint32_t (&pl)[2][4]) {
        const bool edge = key0 + 32 > wave_limit;
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float x = sv[r] * c2;
            if (edge && key0 + 8 * (r >> 2) + 4 * hh + (r & 3) >= limit) x = -INFINITY;
            sv[r] = x;
            mx = fmaxf(mx,x);
        }
        mx = fmaxf(mx,__shfl_xor(mx,32));
        const bool need = mx > m_run + 8.0f;
        const float m_use = need? mx : m_run;
        if (__any(need)) {
            const float alpha = need? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;  // exp2(-inf) = 0 at the start
#pragma unroll
            for (int t = 0; t < TD; t++) o[t] *= alpha;
            l_run *= alpha;
        }
        m_run = m_use;
        // no key of this query seen yet (a key piece past a causal row's
        // limit): p = exp2(-inf) = 0 rather than exp2(-inf - -inf)
        const float m_ref = m_use == -INFINITY? 0.0f : m_use;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const float p0 = __builtin_amdgcn_exp2f(sv[r] - m_ref);
            const float p1 = __builtin_amdgcn_exp2f(sv[r + 1] - m_ref);
            l_run += p0;
            l_run += p1;
            const uint32_t h = pack_bf16(p0,p1);
            const int t = r / 8, w = (r % 8) / 2;
            ph[t][w] = h;
            pl[t][w] = pack_bf16(p0 - __uint_as_float(h << 16),p1 - __uint_as_float(h & 0xFFFF0000u));
        }
    };
    // O^T += V^T * P^T over the half's two 16-key k-steps; the V^T fragments
    // of the next (k-step, output tile) are read while the current MFMAs run.
    auto pv = [&](const uint8_t* st, int u, const uint32_t (&ph)[2][4], const uint32_t (&pl)[2][4]) {
        auto frag = [&](int plane, int j, int td) {
            const int r = 32 * td + lr;
            return lds_read<bf16x8>(st + plane * PLANE + r * 128 + 16 * ((2 * (2 * u + j) + hh) ^ swz_v(r)));
        };
        bf16x8 ah = frag(2,0,0), al = frag(3,0,0);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bf16x8 bh = __builtin_bit_cast(bf16x8,u32x4{ph[j][0],ph[j][1],ph[j][2],ph[j][3]});
            const bf16x8 bl = __builtin_bit_cast(bf16x8,u32x4{pl[j][0],pl[j][1],pl[j][2],pl[j][3]});
#pragma unroll
            for (int td = 0; td < TD; td++) {
                const int nj = td + 1 < TD? j : j + 1, ntd = td + 1 < TD? td + 1 : 0;
                bf16x8 nh, nl;
                if (nj < 2) {
                    nh = frag(2,nj,ntd);
                    nl = frag(3,nj,ntd);
                }
                __builtin_amdgcn_sched_barrier(0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,bh,o[td],0,0,0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,bl,o[td],0,0,0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al,bh,o[td],0,0,0);
                __builtin_amdgcn_sched_barrier(0);
                if (nj < 2) {
                    ah = nh;
                    al = nl;
                }
            }
        }
    };

    // Per tile: both halves' S^T MFMAs go out first, so the second half's run
    // while the first half's softmax (vector ALU) does; then each half's P*V.
    if (t0 < t1) issue(t0,t0 & 1);
    for (int kt = t0; kt < t1; kt++) {
        attn_wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < t1) issue(kt + 1,(kt + 1) & 1);
        const uint8_t* st = lds + (kt & 1) * STAGE;
        v16f s0, s1;
        uint32_t ph[2][4], pl[2][4];
        score(st,s0,s1);
        __builtin_amdgcn_sched_barrier(0);
        softmax(s0,kt * kAK,ph,pl);
        __builtin_amdgcn_sched_barrier(0);
        pv(st,0,ph,pl);
        __builtin_amdgcn_sched_barrier(0);
        softmax(s1,kt * kAK + 32,ph,pl);
        __builtin_amdgcn_sched_barrier(0);
        pv(st,1,ph,pl);
        __builtin_amdgcn_sched_barrier(0);
    }
    l_run += __shfl_xor(l_run,32);
    attn_wait_vmcnt<0>();

    if (piece) {
        // unnormalised O^T (as [query][D]) and the running max / sum
        float* rec = a.part + ((size_t)(split * a.tail + pidx % a.tail) * kAQ + wave * 32 + lr) * (D + 4);
#pragma unroll
        for (int td = 0; td < TD; td++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4*>(rec + 32 * td + 8 * g + 4 * hh) =
                    make_float4(o[td][4 * g],o[td][4 * g + 1],o[td][4 * g + 2],o[td][4 * g + 3]);
        if (hh == 0) {
            rec[D] = m_run;
            rec[D + 1] = l_run;
        }
        return;
    }

    // out[q][head*dim + d] = O^T[d][q] / l: lane holds 4 consecutive dims per
    // (tile, row group)
    if (!live) return;
    float* row = a.out + (size_t)q * a.channels + (size_t)head * a.dim;
    const bool vec = (a.dim & 3) == 0;
#pragma unroll
    for (int td = 0; td < TD; td++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 32 * td + 8 * g + 4 * hh;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = o[td][4 * g + i] / l_run;
            if (vec && d0 + 4 <= a.dim) {
                *reinterpret_cast<float4*>(row + d0) = make_float4(v[0],v[1],v[2],v[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (d0 + i < a.dim) row[d0 + i] = v[i];
            }
        }
}

// Merges the key pieces of the tail units: m = max_s m_s, w_s = exp(m_s - m),
// out = sum_s w_s O_s / sum_s w_s l_s, pieces in order.  One thread per (tail
// unit, query, 4 dims).
template <int D>
__global__ __launch_bounds__(256) void attn_combine(AttnArgs a)
{
    const int per_unit = kAQ * (D / 4);
    const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (idx >= a.tail * per_unit) return;
    const int u = idx / per_unit, qi = (idx % per_unit) / (D / 4), d0 = 4 * (idx % (D / 4));
    const int unit = a.full + u, head = unit / a.tiles_q, qt = unit % a.tiles_q;
    const int q = a.qb + qt * kAQ + qi;
    if (q >= a.qe || d0 >= a.dim) return;
    const size_t stride = (size_t)a.tail * kAQ * (D + 4);
    const float* rec = a.part + ((size_t)u * kAQ + qi) * (D + 4);
    float m = -INFINITY;
    for (int s = 0; s < a.splits; s++) m = fmaxf(m,rec[s * stride + D]);
    float l = 0.0f, v[4] = {0.0f,0.0f,0.0f,0.0f};
    for (int s = 0; s < a.splits; s++) {
        const float* r = rec + s * stride;
        const float w = __builtin_amdgcn_exp2f(r[D] - m);  // maxima in log2 units; an empty piece has -inf: w = 0
        l += w * r[D + 1];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] += w * r[d0 + i];
    }
    float* row = a.out + (size_t)q * a.channels + (size_t)head * a.dim;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (d0 + i < a.dim) row[d0 + i] = v[i] / l;
}

// ---------------------------------------------------------------- wide heads

// Head sizes 129..512 (the VAEs' single head of 384 or 512 channels), padded
// to D = 4 DQ with DQ = 64, 96 or 128.  Q and O^T of a 32-query wave no longer
// fit in registers whole, so the head is cut in quarters: a workgroup of 8
// waves is 2 groups of 32 queries x 4 quarters of DQ dims.  Per 32-key tile
// each wave computes the S^T partial over its quarter (its Q quarter stays in
// registers), the four partials of a group meet in LDS and are summed in
// quarter order -- every wave of the group then holds the same scores and
// runs the same online softmax, so the four waves' running maximum and sum
// agree bit for bit -- and each wave adds V^T[quarter] * P^T into its quarter
// of O^T.  One K tile and one V^T tile are resident (K: 32 keys x D, V^T: D x
// 32 keys, both planes; 160 KB of LDS with the exchange at D = 512); V^T of
// tile t is fetched while the scores of t are formed, K of tile t + 1 while
// the softmax and P*V of t run.
constexpr int kWQ = 64;  // queries per workgroup
constexpr int kWK = 32;  // keys per tile

__device__ __forceinline__ void attn_sync_lds()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int DQ>
__global__ __launch_bounds__(kAThreads, 1) void attn_wide_kernel(AttnArgs a)
{
    constexpr int D = 4 * DQ;
    constexpr int PK = D / 8;                  // 16-byte pieces per K row
    constexpr int KPLANE = kWK * D * 2;        // one plane of a K tile: 32 rows of 2D bytes
    constexpr int VPLANE = D * kWK * 2;        // one plane of a V^T tile: D rows of 64 bytes
    constexpr int CPP = KPLANE / 1024;         // 1 KB DMA chunks per plane
    constexpr int PER_WAVE = 2 * CPP / kAWaves;  // chunks per wave per tile (K or V^T)
    constexpr int KS = DQ / 16, TD = DQ / 32;
    constexpr int EX = 2 * KPLANE + 2 * VPLANE;  // exchange: [group][quarter][4][64 lanes] float4
    static_assert(PER_WAVE * kAWaves == 2 * CPP && PK % 16 == 0, "tile DMAs split evenly, K swizzle within the row");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[EX + 2 * 4 * 4 * 1024];

    // consecutive units on one XCD (they share K and V when they share a head)
    int bid = (int)blockIdx.x;
    if ((gridDim.x & 7) == 0) bid = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);
    const int head = bid / a.tiles_q, qt = bid % a.tiles_q;
    const int kvh = head / a.kv_group;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int grp = wave >> 2, qtr = wave & 3;
    const int lane = (int)(threadIdx.x & 63), lr = lane & 31, hh = lane >> 5;
    const int q = a.qb + qt * kWQ + grp * 32 + lr;
    const bool live = q < a.qe;
    const int limit = !live? 1 : a.causal? min(a.key_end,a.qoff + q + 1) : a.key_end;
    const int q_last = min(a.qe,a.qb + (qt + 1) * kWQ) - 1;
    const int wg_limit = a.causal? min(a.key_end,a.qoff + q_last + 1) : a.key_end;
    const int tiles = (wg_limit + kWK - 1) / kWK;

    // Q quarter fragments: lane = query, dims qtr*DQ + 16k + 8hh .. +7
    bf16x8 qfh[KS], qfl[KS];
    {
        const float* qrow = a.q + (size_t)min(q,a.rows - 1) * a.channels + (size_t)head * a.dim;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            u32x4 vh, vl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = qtr * DQ + 16 * k + 8 * hh + 2 * i;
                uint32_t h0, l0, h1, l1;
                split2(d < a.dim? qrow[d] : 0.0f,h0,l0);
                split2(d + 1 < a.dim? qrow[d + 1] : 0.0f,h1,l1);
                vh[i] = h0 | (h1 << 16);
                vl[i] = l0 | (l1 << 16);
            }
            qfh[k] = __builtin_bit_cast(bf16x8,vh);
            qfl[k] = __builtin_bit_cast(bf16x8,vl);
        }
    }
    int wave_limit = limit;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) wave_limit = min(wave_limit,__shfl_xor(wave_limit,m));

    const size_t plane = (size_t)a.keys_pad * D * 2;
    const size_t hoff = (size_t)kvh * a.keys_pad * D;
    const ARsrc rk[2] = {__builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kh) + hoff,(short)0,(int)plane,0x00020000),
                         __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kl) + hoff,(short)0,(int)plane,0x00020000)};
    const ARsrc rv[2] = {__builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vh) + hoff,(short)0,(int)plane,0x00020000),
                         __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vl) + hoff,(short)0,(int)plane,0x00020000)};

    // K tile kt: chunk c = wave + 8i of the two planes; lane j of a chunk lands
    // on piece 64 ci + j of the plane = row r, physical piece p, which holds
    // logical piece p ^ (r & 15).
    auto issue_k = [&](int kt) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; i++) {
            const int c = wave + kAWaves * i, pl = c / CPP, ci = c % CPP;
            const int f = ci * 64 + lane, r = f / PK, p = f % PK;
            const uint32_t off = (uint32_t)((kt * kWK + r) * D * 2 + 16 * (p ^ (r & 15)));
            adma(rk[pl],lds + pl * KPLANE + ci * 1024,off,0);
        }
    };
    // V^T tile kt: rows of 4 pieces (32 keys); row r, physical piece p holds
    // logical piece p ^ ((r >> 2) & 3).
    auto issue_v = [&](int kt) {
#pragma unroll
        for (int i = 0; i < PER_WAVE; i++) {
            const int c = wave + kAWaves * i, pl = c / CPP, ci = c % CPP;
            const int f = ci * 64 + lane, r = f >> 2, p = f & 3;
            const uint32_t off = (uint32_t)(((size_t)r * a.keys_pad + kt * kWK) * 2 + 16 * (p ^ ((r >> 2) & 3)));
            adma(rv[pl],lds + 2 * KPLANE + pl * VPLANE + ci * 1024,off,0);
        }
    };

    v16f o[TD];
#pragma unroll
    for (int t = 0; t < TD; t++) o[t] = v16f{};
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * kLog2e;

    // partial S^T over this wave's quarter (keys = MFMA rows, lane's query =
    // column)
    auto score = [&]() {
        v16f s = v16f{};
        const uint8_t *h = lds + lr * (2 * D), *l = lds + KPLANE + lr * (2 * D);
        auto frag = [&](const uint8_t* row, int k) {
            return lds_read<bf16x8>(row + 16 * ((qtr * (DQ / 8) + 2 * k + hh) ^ (lr & 15)));
        };
        bf16x8 ah = frag(h,0), al = frag(l,0);
#pragma unroll
        for (int k = 0; k < KS; k++) {
            bf16x8 nh, nl;
            if (k + 1 < KS) {
                nh = frag(h,k + 1);
                nl = frag(l,k + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,qfh[k],s,0,0,0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,qfl[k],s,0,0,0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al,qfh[k],s,0,0,0);
            __builtin_amdgcn_sched_barrier(0);
            if (k + 1 < KS) {
                ah = nh;
                al = nl;
            }
        }
        return s;
    };
    // the online softmax of the existing kernel over one 32-key tile
    auto softmax = [&](v16f& sv, int key0, uint32_t (&ph)[2][4], uint32_t (&pl)[2][4]) {
        const bool edge = key0 + 32 > wave_limit;
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float x = sv[r] * c2;
            if (edge && key0 + 8 * (r >> 2) + 4 * hh + (r & 3) >= limit) x = -INFINITY;
            sv[r] = x;
            mx = fmaxf(mx,x);
        }
        mx = fmaxf(mx,__shfl_xor(mx,32));
        const bool need = mx > m_run + 8.0f;
        const float m_use = need? mx : m_run;
        if (__any(need)) {
            const float alpha = need? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
#pragma unroll
            for (int t = 0; t < TD; t++) o[t] *= alpha;
            l_run *= alpha;
        }
        m_run = m_use;
        const float m_ref = m_use == -INFINITY? 0.0f : m_use;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const float p0 = __builtin_amdgcn_exp2f(sv[r] - m_ref);
            const float p1 = __builtin_amdgcn_exp2f(sv[r + 1] - m_ref);
            l_run += p0;
            l_run += p1;
            const uint32_t h = pack_bf16(p0,p1);
            const int t = r / 8, w = (r % 8) / 2;
            ph[t][w] = h;
            pl[t][w] = pack_bf16(p0 - __uint_as_float(h << 16),p1 - __uint_as_float(h & 0xFFFF0000u));
        }
    };
    // O^T[quarter] += V^T[quarter] * P^T over the tile's two 16-key k-steps
    auto pv = [&](const uint32_t (&ph)[2][4], const uint32_t (&pl)[2][4]) {
        auto frag = [&](int pln, int j, int td) {
            const int r = qtr * DQ + 32 * td + lr;
            return lds_read<bf16x8>(lds + 2 * KPLANE + pln * VPLANE + r * 64 + 16 * ((2 * j + hh) ^ ((lr >> 2) & 3)));
        };
        bf16x8 ah = frag(0,0,0), al = frag(1,0,0);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bf16x8 bh = __builtin_bit_cast(bf16x8,u32x4{ph[j][0],ph[j][1],ph[j][2],ph[j][3]});
            const bf16x8 bl = __builtin_bit_cast(bf16x8,u32x4{pl[j][0],pl[j][1],pl[j][2],pl[j][3]});
#pragma unroll
            for (int td = 0; td < TD; td++) {
                const int nj = td + 1 < TD? j : j + 1, ntd = td + 1 < TD? td + 1 : 0;
                bf16x8 nh, nl;
                if (nj < 2) {
                    nh = frag(0,nj,ntd);
                    nl = frag(1,nj,ntd);
                }
                __builtin_amdgcn_sched_barrier(0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,bh,o[td],0,0,0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah,bl,o[td],0,0,0);
                o[td] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al,bh,o[td],0,0,0);
                __builtin_amdgcn_sched_barrier(0);
                if (nj < 2) {
                    ah = nh;
                    al = nl;
                }
            }
        }
    };

    uint8_t* const ex = lds + EX;
    issue_k(0);
    for (int kt = 0; kt < tiles; kt++) {
        attn_wait_vmcnt<0>();
        attn_sync_lds();  // K of kt visible; every wave is past P*V of kt - 1
        issue_v(kt);
        const v16f s = score();
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<float4*>(ex + ((grp * 4 + qtr) * 4 + i) * 1024 + lane * 16) =
                make_float4(s[4 * i],s[4 * i + 1],s[4 * i + 2],s[4 * i + 3]);
        attn_sync_lds();  // partials visible; every wave is past its K reads
        if (kt + 1 < tiles) issue_k(kt + 1);
        v16f t;
#pragma unroll
        for (int w = 0; w < 4; w++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 p = lds_read<float4>(ex + ((grp * 4 + w) * 4 + i) * 1024 + lane * 16);
                if (w == 0) {
                    t[4 * i] = p.x; t[4 * i + 1] = p.y; t[4 * i + 2] = p.z; t[4 * i + 3] = p.w;
                } else {
                    t[4 * i] += p.x; t[4 * i + 1] += p.y; t[4 * i + 2] += p.z; t[4 * i + 3] += p.w;
                }
            }
        uint32_t ph[2][4], pl[2][4];
        softmax(t,kt * kWK,ph,pl);
        if (kt + 1 < tiles) attn_wait_vmcnt<PER_WAVE>();  // this wave's V^T DMAs of kt (K of kt + 1 may still run)
        else attn_wait_vmcnt<0>();
        attn_sync_lds();  // V^T of kt visible
        pv(ph,pl);
    }
    l_run += __shfl_xor(l_run,32);
    attn_wait_vmcnt<0>();

    if (!live) return;
    float* row = a.out + (size_t)q * a.channels + (size_t)head * a.dim;
    const bool vec = (a.dim & 3) == 0;
#pragma unroll
    for (int td = 0; td < TD; td++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = qtr * DQ + 32 * td + 8 * g + 4 * hh;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = o[td][4 * g + i] / l_run;
            if (vec && d0 + 4 <= a.dim) {
                *reinterpret_cast<float4*>(row + d0) = make_float4(v[0],v[1],v[2],v[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (d0 + i < a.dim) row[d0 + i] = v[i];
            }
        }
}

// ---------------------------------------------------------------- host side

static int attn_cus()
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

static size_t aru(size_t v, size_t m) { return (v + m - 1) / m * m; }

int attention_dim_pad(size_t dim)
{
    return dim == 0? 0 : dim <= 64? 64 : dim <= 128? 128 : dim <= 256? 256 : dim <= 384? 384 : dim <= 512? 512 : 0;
}

size_t attention_workspace_bytes(size_t rows, size_t keys, size_t heads, size_t kv_heads, size_t dim)
{
    const int D = attention_dim_pad(dim);
    if (!D) return 0;
    (void)rows;
    (void)heads;
    const size_t kv = kv_heads * aru(keys,kAK) * D;
    // K and V^T planes + the key-split pieces of the narrow kernel (at most
    // one per CU)
    return 4 * kv * sizeof(uint16_t) + (D <= 128? (size_t)attn_cus() * kAQ * (D + 4) * sizeof(float) : 0);
}

hipError_t launch_attention(const float* q, const float* k, const float* v, float* out, size_t rows, size_t keys, size_t heads,
                            size_t kv_heads, size_t dim, const AttnRange* ranges, size_t count, size_t query_offset, void* workspace,
                            hipStream_t s)
{
    const int D = attention_dim_pad(dim);
    if (!D || !heads || !kv_heads || heads % kv_heads || !rows || !keys) return hipErrorInvalidValue;
    const size_t rows_pad = aru(rows,kAQ), keys_pad = aru(keys,kAK);
    const size_t channels = heads * dim, kv_channels = kv_heads * dim;
    // 32-bit bounds: the per-head K / V^T planes are addressed with 32-bit
    // buffer offsets, and the kernel's row indexes are ints.
    if (keys_pad * D * 2 >= ((size_t)1 << 31) || rows_pad + query_offset >= ((size_t)1 << 31) || keys >= ((size_t)1 << 30))
        return hipErrorInvalidValue;
    uint16_t* w = static_cast<uint16_t*>(workspace);
    const size_t kn = kv_heads * keys_pad * D;
    uint16_t *kh = w, *kl = kh + kn, *vh = kl + kn, *vl = vh + kn;
    float* part = reinterpret_cast<float*>(vl + kn);
    {
        const size_t nk = kv_heads * keys_pad * (D / 8), nv = kv_heads * (keys_pad / 64) * D;
        const bool vec = dim % 8 == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0;
        attn_split_rows<<<dim3((unsigned)((nk + 255) / 256)),dim3(256),0,s>>>(k,keys,kv_channels,(int)kv_heads,(int)dim,D,keys_pad,vec,kh,
                                                                             kl);
        attn_split_vt<<<dim3((unsigned)((nv + 255) / 256)),dim3(256),0,s>>>(v,keys,kv_channels,(int)kv_heads,(int)dim,D,keys_pad,vh,vl);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    AttnArgs a = {};
    a.q = q;
    a.kh = kh; a.kl = kl; a.vh = vh; a.vl = vl;
    a.out = out;
    a.rows = (int)rows;
    a.keys_pad = (int)keys_pad;
    a.heads = (int)heads;
    a.kv_group = (int)(heads / kv_heads);
    a.dim = (int)dim;
    a.channels = (int)channels;
    a.qoff = (int)query_offset;
    a.scale = 1.0f / sqrtf((float)dim);
    for (size_t i = 0; i < count; i++) {
        const AttnRange& r = ranges[i];
        if (r.query_end <= r.query_begin || r.query_end > rows || !r.key_end || r.key_end > keys) return hipErrorInvalidValue;
        a.qb = (int)r.query_begin;
        a.qe = (int)r.query_end;
        a.key_end = (int)r.key_end;
        a.causal = r.causal? 1 : 0;
        if (D > 128) {
            a.tiles_q = (int)((r.query_end - r.query_begin + kWQ - 1) / kWQ);
            a.full = (int)heads * a.tiles_q;
            const dim3 grid((unsigned)a.full);
            if (D == 512) attn_wide_kernel<128><<<grid,dim3(kAThreads),0,s>>>(a);
            else if (D == 384) attn_wide_kernel<96><<<grid,dim3(kAThreads),0,s>>>(a);
            else attn_wide_kernel<64><<<grid,dim3(kAThreads),0,s>>>(a);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            continue;
        }
        a.tiles_q = (int)((r.query_end - r.query_begin + kAQ - 1) / kAQ);
        // One workgroup per CU at a time: when the last round of (head, query
        // tile) units would leave at least half of the CUs idle, its units
        // are cut into key pieces that spread over every CU.
        const int cus = attn_cus(), units = (int)heads * a.tiles_q;
        const int tail = units % cus;
        a.full = units;
        a.tail = 1;
        a.splits = 1;
        a.part = part;
        if (tail && tail * 2 <= cus) {
            a.tail = tail;
            a.full = units - tail;
            a.splits = std::min(cus / tail,16);
        }
        const int pieces = a.splits > 1? a.tail * a.splits : 0;
        const dim3 grid((unsigned)(a.full + pieces));
        if (D == 128) attn_kernel<128><<<grid,dim3(kAThreads),0,s>>>(a);
        else attn_kernel<64><<<grid,dim3(kAThreads),0,s>>>(a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (pieces) {
            const int threads = a.tail * kAQ * (D / 4);
            if (D == 128) attn_combine<128><<<dim3((unsigned)((threads + 255) / 256)),dim3(256),0,s>>>(a);
            else attn_combine<64><<<dim3((unsigned)((threads + 255) / 256)),dim3(256),0,s>>>(a);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace pixhip
