// Quantized GEMM on int8 MFMA (gfx950): Y[M][N] = X[M][K] * W[N][K]^T for
// Q5_K / Q6_K / Q8_0 weights and Q8_K / Q8_0 activations.  The counterpart of
// pix_dot_q5_K / pix_dot_q6_K / pix_dot_q8_0 driven by cpu_quant_matmul
// (src/kernels_quant.cpp:163-365, :369-412) and of shaders/matmul_mmq.comp.
//
// Tiling: a workgroup (4 waves, 2x2) owns a 128x128 output tile; each wave owns
// 64x64 = 2x2 tiles of v_mfma_i32_32x32x32_i8 (A = activations, rows = tokens;
// B = weights, columns = output features, so each lane holds one feature
// column and 16 token rows of every 32x32 accumulator).  K is staged through
// LDS in 64-byte chunks (two 32-value sub-blocks), double buffered, with
// 128-bit global loads and 80-byte padded LDS rows (conflict-free ds_read_b128).
//
// Exactness: the MFMAs produce, per (token, feature, 256-value super-block),
// the exact integers the reference forms before its fp32 epilogue:
//   Q5_K  S = sum_s scale_s*dot_s   from the hi/lo planes (64*hi + lo)
//         Mn = sum_t min_{t/2}*bsum16_t  by one fp16 MFMA (all inputs exact in
//              fp16: min <= 63, |bsum16| <= 2032; |Mn| < 2^24 so fp32 is exact)
//   Q6_K  S = sum_e scale*(q-32)*q8 from the hi/lo planes
//   Q8_0  P = sum over the 32-value block of q*q8
// then y += yd*(wd*S - wdmin*Mn) per super-block (Q5_K), y += yd*wd*S (Q6_K),
// y += xd*(wd*P) per block (Q8_0), in fp32.
#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

constexpr int kBM = 128, kBN = 128, kKC = 64, kLDA = 80;  // rows x chunk bytes, padded row stride
constexpr int kThreads = 256;

enum Kind { KIND_Q5K = 0, KIND_Q6K = 1, KIND_Q80 = 2 };

struct GemmArgs {
    const int8_t* xq;     // [Mpad][K]
    const float* xdT;     // [K/QK][Mpad]  (QK = 256, or 32 for Q8_0)
    const _Float16* xbs;  // [Mpad][K/16]  (Q5_K only)
    const int8_t* whi;    // [Npad][K] (Q8_0: the quantized plane)
    const int8_t* wlo;    // [Npad][K]
    const float* wdT;     // Q5_K/Q6_K: [N][K/256]  Q8_0: [K/32][Npad]
    const float* wdm;     // [N][K/256] (Q5_K)
    const _Float16* wmn;  // [Npad][K/16] (Q5_K)
    float* y;
    const float* bias;
    int32_t* sums;        // debug: exact integer sums [M][N][blocks]
    int32_t* mins;
    int M, N, K, Mpad, Npad;
    size_t ldy, yoff;
    int tiles_m, tiles_n;
};

// Bijective XCD-aware remap: hardware places workgroup b on XCD b % 8; give
// each XCD a contiguous range of logical tiles so its L2 sees neighbours.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd < r? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

template <int KIND, bool SUMS>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g)
{
    constexpr int PLANES = KIND == KIND_Q80? 1 : 2;
    __shared__ __attribute__((aligned(16))) int8_t sA[2][kBM * kLDA];
    __shared__ __attribute__((aligned(16))) int8_t sW[2][PLANES][kBN * kLDA];
    __shared__ __attribute__((aligned(16))) float sXD[2][2][kBM];  // per chunk: 2 scales (Q8_0 blocks) or 1 (K-quants)
    __shared__ __attribute__((aligned(16))) float sWD[2][2][kBN];  // Q8_0: two block scales; K-quants: d, dmin

    const int nblocks = g.tiles_m * g.tiles_n;
    const int lid = xcd_remap((int)blockIdx.x,nblocks);
    // Grouped order: 8 token tiles share each feature tile.
    constexpr int GROUP = 8;
    const int group = lid / (GROUP * g.tiles_n);
    const int first_m = group * GROUP;
    const int gsize = min(g.tiles_m - first_m,GROUP);
    const int within = lid % (GROUP * g.tiles_n);
    const int tm = first_m + within % gsize, tn = within / gsize;
    const int m0 = tm * kBM, n0 = tn * kBN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1, lr = lane & 31, lg = lane >> 5;
    const int K = g.K;
    const int nchunks = K / kKC;
    const int nsb = K / PIX_QK;  // super-blocks (K-quants)

    // Global -> register staging of one chunk: A and W planes, 2 pieces of 16 B each per thread.
    v4i ra[2], rw[PLANES][2];
    float rxd = 0.0f, rwd = 0.0f;
    auto load_chunk = [&](int c) {
        const int k0 = c * kKC;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int p = tid + q * kThreads, row = p >> 2, c16 = p & 3;
            ra[q] = *reinterpret_cast<const v4i*>(g.xq + (size_t)(m0 + row) * K + k0 + c16 * 16);
            rw[0][q] = *reinterpret_cast<const v4i*>(g.whi + (size_t)(n0 + row) * K + k0 + c16 * 16);
            if constexpr (PLANES == 2) rw[1][q] = *reinterpret_cast<const v4i*>(g.wlo + (size_t)(n0 + row) * K + k0 + c16 * 16);
        }
        const int idx = tid & 127, half = tid >> 7;
        if constexpr (KIND == KIND_Q80) {
            const int kb = c * 2 + half;
            rxd = g.xdT[(size_t)kb * g.Mpad + m0 + idx];
            rwd = g.wdT[(size_t)kb * g.Npad + n0 + idx];
        } else {
            const int b = c / (PIX_QK / kKC);
            rxd = half == 0? g.xdT[(size_t)b * g.Mpad + m0 + idx] : 0.0f;
            const int n = min(n0 + idx,g.N - 1);
            if constexpr (KIND == KIND_Q5K) rwd = half == 0? g.wdT[(size_t)n * nsb + b] : g.wdm[(size_t)n * nsb + b];
            else rwd = half == 0? g.wdT[(size_t)n * nsb + b] : 0.0f;
        }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int p = tid + q * kThreads, row = p >> 2, c16 = p & 3;
            *reinterpret_cast<v4i*>(&sA[buf][row * kLDA + c16 * 16]) = ra[q];
#pragma unroll
            for (int pl = 0; pl < PLANES; pl++) *reinterpret_cast<v4i*>(&sW[buf][pl][row * kLDA + c16 * 16]) = rw[pl][q];
        }
        const int idx = tid & 127, half = tid >> 7;
        sXD[buf][half][idx] = rxd;
        sWD[buf][half][idx] = rwd;
    };

    v16i acc_hi[2][2], acc_lo[2][2];
    v16f yacc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc_hi[i][j] = v16i{};
            acc_lo[i][j] = v16i{};
            yacc[i][j] = v16f{};
        }
    const v16i izero = {};
    const v16f fzero = {};

    load_chunk(0);
    store_chunk(0);
    __syncthreads();

    for (int c = 0; c < nchunks; c++) {
        const int buf = c & 1;
        if (c + 1 < nchunks) load_chunk(c + 1);
        const bool sb_end = KIND != KIND_Q80 && (c % (PIX_QK / kKC)) == (PIX_QK / kKC) - 1;
        const int b = c / (PIX_QK / kKC);
        v8h bsA[2], mnB[2];
        if constexpr (KIND == KIND_Q5K) {
            if (sb_end) {
#pragma unroll
                for (int i = 0; i < 2; i++)
                    bsA[i] = *reinterpret_cast<const v8h*>(g.xbs + (size_t)(m0 + wm * 64 + i * 32 + lr) * (K / 16) + b * 16 + lg * 8);
#pragma unroll
                for (int j = 0; j < 2; j++)
                    mnB[j] = *reinterpret_cast<const v8h*>(g.wmn + (size_t)(n0 + wn * 64 + j * 32 + lr) * (K / 16) + b * 16 + lg * 8);
            }
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            v4i a[2], wh[2], wl[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const v4i*>(&sA[buf][(wm * 64 + i * 32 + lr) * kLDA + s * 32 + lg * 16]);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                wh[j] = *reinterpret_cast<const v4i*>(&sW[buf][0][(wn * 64 + j * 32 + lr) * kLDA + s * 32 + lg * 16]);
                if constexpr (PLANES == 2) wl[j] = *reinterpret_cast<const v4i*>(&sW[buf][1][(wn * 64 + j * 32 + lr) * kLDA + s * 32 + lg * 16]);
            }
            if constexpr (KIND == KIND_Q80) {
                // One 32-value block per sub-block: fresh accumulator, fp32 epilogue.
                float wdv[2];
#pragma unroll
                for (int j = 0; j < 2; j++) wdv[j] = sWD[buf][s][wn * 64 + j * 32 + lr];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    float xdv[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        float4 t = *reinterpret_cast<const float4*>(&sXD[buf][s][wm * 64 + i * 32 + 8 * q4 + 4 * lg]);
                        xdv[4 * q4 + 0] = t.x;
                        xdv[4 * q4 + 1] = t.y;
                        xdv[4 * q4 + 2] = t.z;
                        xdv[4 * q4 + 3] = t.w;
                    }
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],izero,0,0,0);
                        if constexpr (SUMS) {
                            const int kb = c * 2 + s;
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                                const int n = n0 + wn * 64 + j * 32 + lr;
                                if (m < g.M && n < g.N) g.sums[((size_t)m * g.N + n) * (K / PIX_QK8) + kb] = p[r];
                            }
                        } else {
#pragma unroll
                            for (int r = 0; r < 16; r++)
                                yacc[i][j][r] = __builtin_fmaf(xdv[r],(float)p[r] * wdv[j],yacc[i][j][r]);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        acc_hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wh[j],acc_hi[i][j],0,0,0);
                        acc_lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i],wl[j],acc_lo[i][j],0,0,0);
                    }
            }
        }
        if constexpr (KIND != KIND_Q80) {
            if (sb_end) {
                float wdv[2], wmv[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    wdv[j] = sWD[buf][0][wn * 64 + j * 32 + lr];
                    wmv[j] = sWD[buf][1][wn * 64 + j * 32 + lr];
                }
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    float ydv[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        float4 t = *reinterpret_cast<const float4*>(&sXD[buf][0][wm * 64 + i * 32 + 8 * q4 + 4 * lg]);
                        ydv[4 * q4 + 0] = t.x;
                        ydv[4 * q4 + 1] = t.y;
                        ydv[4 * q4 + 2] = t.z;
                        ydv[4 * q4 + 3] = t.w;
                    }
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        v16f mt = fzero;
                        if constexpr (KIND == KIND_Q5K) mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsA[i],mnB[j],fzero,0,0,0);
                        if constexpr (SUMS) {
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                                const int n = n0 + wn * 64 + j * 32 + lr;
                                if (m < g.M && n < g.N) {
                                    const size_t o = ((size_t)m * g.N + n) * nsb + b;
                                    g.sums[o] = acc_hi[i][j][r] * 64 + acc_lo[i][j][r];
                                    if constexpr (KIND == KIND_Q5K) g.mins[o] = (int32_t)mt[r];
                                }
                            }
                        } else {
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const int S = acc_hi[i][j][r] * 64 + acc_lo[i][j][r];
                                float t = (float)S * wdv[j];
                                if constexpr (KIND == KIND_Q5K) t = __builtin_fmaf(mt[r],-wmv[j],t);
                                yacc[i][j][r] = __builtin_fmaf(ydv[r],t,yacc[i][j][r]);
                            }
                        }
                        acc_hi[i][j] = izero;
                        acc_lo[i][j] = izero;
                    }
                }
            }
        }
        if (c + 1 < nchunks) store_chunk(buf ^ 1);
        __syncthreads();
    }

    if constexpr (!SUMS) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = n0 + wn * 64 + j * 32 + lr;
                if (n >= g.N) continue;
                const float bv = g.bias? g.bias[n] : 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
                    if (m < g.M) g.y[g.yoff + (size_t)m * g.ldy + n] = yacc[i][j][r] + bv;
                }
            }
    }
}

static size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

template <int KIND, bool SUMS>
static hipError_t launch(GemmArgs g, size_t mpad, hipStream_t s)
{
    g.tiles_m = (int)((g.M + kBM - 1) / kBM);
    g.tiles_n = (int)((g.N + kBN - 1) / kBN);
    g.Mpad = (int)round_up((size_t)g.M,kBM);
    g.Npad = (int)round_up((size_t)g.N,kBN);
    if (mpad < (size_t)g.Mpad || g.K % kKC) return hipErrorInvalidValue;
    g.Mpad = (int)mpad;
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
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdm = w.dm; g.wmn = w.mn;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q5K,false>(g,a.mpad,s);
}

hipError_t launch_gemm_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q6K,false>(g,a.mpad,s);
}

hipError_t launch_gemm_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, const Output& out, hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.qs; g.wdT = w.dT;
    g.y = out.y; g.bias = out.bias; g.ldy = out.ldy; g.yoff = out.offset;
    return launch<KIND_Q80,false>(g,a.mpad,s);
}

hipError_t launch_sums_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, int32_t* scaled, int32_t* mins,
                            hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d; g.xbs = a.bs;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d; g.wdm = w.dm; g.wmn = w.mn;
    g.sums = scaled; g.mins = mins;
    return launch<KIND_Q5K,true>(g,a.mpad,s);
}

hipError_t launch_sums_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    GemmArgs g = base_args(M,N,K);
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.hi; g.wlo = w.lo; g.wdT = w.d;
    g.sums = sums;
    return launch<KIND_Q6K,true>(g,a.mpad,s);
}

hipError_t launch_sums_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s)
{
    GemmArgs g = base_args(M,N,round_up(K,kKC));
    g.xq = a.qs; g.xdT = a.d;
    g.whi = w.qs; g.wdT = w.dT;
    g.sums = sums;
    return launch<KIND_Q80,true>(g,a.mpad,s);
}

}  // namespace pixhip
