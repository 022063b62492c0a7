// Producers of a linear layer's input fused with its activation quantizer, so
// the fp32 tensor between them need not make a round trip through HBM:
//   - tensor_norm (src/tensor.cpp:174-197), optionally followed by z_modulate
//     (src/inference.cpp:263-277): the RMS / layer norm in front of the DiT
//     block's QKV and FFN-in linears;
//   - tensor_silu (src/tensor.cpp:199-209) then tensor_gate (:334-345): the
//     SwiGLU product in front of the FFN-down linear.
// Each writes the planar activations the GEMM reads (Q8_K for K-quant weights,
// Q8_0 for Q8_0 weights), and when asked the fp32 result (what the reference's
// op returns) and the reference's block layout.
//
// Byte work, bound by HBM and by the quantizer's vector-ALU work.  A norm reads
// a row once: one to four waves per token row (two for rows of 2049-4096
// values: measured 18% faster than one wave of 16 chunks at 3 waves per SIMD,
// and as fast as four), holding the row in registers (a 256-value chunk per
// float4 per lane) from the sum of squares to the quantizer; into Q8_K, four
// chunks at a time are transposed across lanes to the 16-lanes-per-block
// quantizer.  The gate product is one wave per 256-value chunk.
#include <type_traits>

#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

constexpr int kNormWaves = 4;
constexpr size_t kStageMaxK = 4096;  // norm vectors staged in LDS up to this row length (32 KB)
constexpr int kGateWaves = 8;
// Rows per workgroup in the SiLU * gate producer.  On [4608, 10240] -> Q8_0:
// 92 us with 16 or 32 rows, 99 with 8 rows or with one row's 8 chunks per
// workgroup, 186 with 64 (two waves per SIMD for the 16 loads per lane).
constexpr int kGateRows = 16;

struct FuseArgs {
    const float* x;      // norm input [rows][K] or gate [rows][K]
    const float* u;      // up [rows][K] (gate product)
    const float* w;      // norm weight [K] or null
    const float* mod;    // modulation scale [K] or null
    size_t rows, K;
    float eps;
    int centered;
    int kind;            // 0 none, 1 Q8_K, 2 Q8_0
    int stage_vectors;   // norm: weight and modulation staged in dynamic LDS
    size_t kpad, mpad;   // Q8_0 planar row stride; planar rows allocated
    int8_t* qs;          // planar activations (null: none)
    float* d;
    _Float16* bs;
    uint8_t* blocks;     // reference block layout (null: none)
    float* y;            // fp32 result (null: none)
};

// Values k0..k0+3 of a row (k0 = 256c + 4*lane), zeros past the row's end.
// The load itself is unconditional (clamped to the row's last four values) and
// the zeros are selected afterwards: a load under a per-lane branch makes the
// compiler wait for it at the branch's end, which would serialise the loads.
__device__ __forceinline__ float4 load4(const float* row, size_t K, size_t k0)
{
    const float4 t = *reinterpret_cast<const float4*>(row + (k0 < K? k0 : K - 4));
    const bool in = k0 < K;
    return make_float4(in? t.x : 0.f,in? t.y : 0.f,in? t.z : 0.f,in? t.w : 0.f);
}

// Writes chunk c (values 256c..256c+255) of `row`: lane l holds values
// 256c+4l..+3 in v (zeros past the end).  Every lane of the wave must call it.
// Q8_K: the chunk is one block.  Q8_0: lanes 8g..8g+7 form block 8c+g; blocks
// between K/32 and kpad/32 are the planar padding (zeros, zero scale).
template <int KIND>
__device__ __forceinline__ void store_chunk(const FuseArgs& a, size_t row, int c, int lane, float4 v)
{
    const size_t K = a.K, k0 = (size_t)c * 256 + 4 * lane;
    if (a.y && k0 < K) *reinterpret_cast<float4*>(a.y + row * K + k0) = v;
    if constexpr (KIND == 1) {
        uint32_t packed;
        float d;
        int gsum;
        quantize_q8_K_wave(v,lane,packed,d,gsum);
        const size_t nb = K / PIX_QK;
        if (a.qs) {
            *reinterpret_cast<uint32_t*>(a.qs + tiled_offset(row,(size_t)c * PIX_QK + 4 * lane,K)) = packed;
            if (lane == 0) a.d[(size_t)c * a.mpad + row] = d;
            const int t = lane >> 2;  // 16-value group, stored even groups first
            if ((lane & 3) == 0) a.bs[tiled_bs_index(row,(size_t)c,(t & 1) * 8 + (t >> 1),K)] = (_Float16)(float)gsum;
        }
        if (a.blocks) {
            uint8_t* blk = a.blocks + (row * nb + c) * PIX_Q8_K_BYTES;
            reinterpret_cast<uint32_t*>(blk + 4)[lane] = packed;
            if (lane == 0) *reinterpret_cast<float*>(blk) = d;
            if ((lane & 3) == 0) reinterpret_cast<int16_t*>(blk + 4 + PIX_QK)[lane >> 2] = (int16_t)gsum;
        }
    } else if constexpr (KIND == 2) {
        uint32_t packed;
        float d32;
        uint16_t dh;
        quantize_q8_0_group(v,packed,d32,dh);
        const size_t b = (size_t)c * 8 + (lane >> 3), nb = K / PIX_QK8, nbp = a.kpad / PIX_QK8;
        if (a.qs && b < nbp) {
            reinterpret_cast<uint32_t*>(a.qs + row * a.kpad + b * PIX_QK8)[lane & 7] = packed;
            if ((lane & 7) == 0) a.d[b * a.mpad + row] = half_bits_to_float(dh);
        }
        if (a.blocks && b < nb) {
            uint8_t* out = a.blocks + (row * nb + b) * PIX_Q8_0_BYTES;
            uint16_t* q16 = reinterpret_cast<uint16_t*>(out + 2 + 4 * (lane & 7));
            q16[0] = (uint16_t)(packed & 0xffffu);
            q16[1] = (uint16_t)(packed >> 16);
            if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(out) = dh;
        }
    }
}

// Four chunks of a row in the wave layout (v[q], lane l: values 4l..4l+3 of
// chunk q) moved into the layout of quantize_q8_K_x4 (t[j], lane l: values
// 64j + 4(l%16) .. +3 of chunk l/16): a transpose of 16-lane rows, two lane
// swaps per word (permlane32 swaps the upper half of its first operand with
// the lower half of its second, permlane16 the odd rows of the first with the
// even rows of the second).
__device__ __forceinline__ void chunks_to_blocks(const float4 (&v)[4], float4 (&t)[4])
{
    auto sw = [](float a0, float a1, float a2, float a3, float& t0, float& t1, float& t2, float& t3) {
        const auto p02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0),__float_as_uint(a2),false,false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a1),__float_as_uint(a3),false,false);
        const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0],p13[0],false,false);
        const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1],p13[1],false,false);
        t0 = __uint_as_float(q01[0]);
        t1 = __uint_as_float(q01[1]);
        t2 = __uint_as_float(q23[0]);
        t3 = __uint_as_float(q23[1]);
    };
    sw(v[0].x,v[1].x,v[2].x,v[3].x,t[0].x,t[1].x,t[2].x,t[3].x);
    sw(v[0].y,v[1].y,v[2].y,v[3].y,t[0].y,t[1].y,t[2].y,t[3].y);
    sw(v[0].z,v[1].z,v[2].z,v[3].z,t[0].z,t[1].z,t[2].z,t[3].z);
    sw(v[0].w,v[1].w,v[2].w,v[3].w,t[0].w,t[1].w,t[2].w,t[3].w);
}

// Writes block c of `row` from the lanes of one 16-lane row after
// quantize_q8_K_x4 (lane l%16 = lp holds the block's values 64j + 4lp .. +3).
__device__ __forceinline__ void store_q8_K_x4(const FuseArgs& a, size_t row, int c, int lane, const uint32_t (&packed)[4], float d,
                                              const int (&gsum)[4])
{
    const int lp = lane & 15;
    const size_t K = a.K, k0 = (size_t)c * PIX_QK + 4 * lp, nb = K / PIX_QK;
    if (a.qs) {
        // values k0 + 64j are in consecutive 1 KB pieces of the row group
        int8_t* q = a.qs + tiled_offset(row,k0,K);
#pragma unroll
        for (int j = 0; j < 4; j++) *reinterpret_cast<uint32_t*>(q + 1024 * j) = packed[j];
        if (lp == 0) a.d[(size_t)c * a.mpad + row] = d;
        if ((lp & 3) == 0) {
            // group g = 4j + lp/4 at (g&1)*8 + g/2: even groups first, then odd
            _Float16* o = a.bs + tiled_bs_index(row,(size_t)c,0,K);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int g = 4 * j + (lp >> 2);
                o[(g & 1) * 8 + (g >> 1)] = (_Float16)(float)gsum[j];
            }
        }
    }
    if (a.blocks) {
        uint8_t* blk = a.blocks + (row * nb + c) * PIX_Q8_K_BYTES;
#pragma unroll
        for (int j = 0; j < 4; j++) *reinterpret_cast<uint32_t*>(blk + 4 + 64 * j + 4 * lp) = packed[j];
        if (lp == 0) *reinterpret_cast<float*>(blk) = d;
        if ((lp & 3) == 0) {
#pragma unroll
            for (int j = 0; j < 4; j++) reinterpret_cast<int16_t*>(blk + 4 + PIX_QK)[4 * j + (lp >> 2)] = (int16_t)gsum[j];
        }
    }
}

// Chunks a row is written in: K values, plus the Q8_0 padding block.
__device__ __forceinline__ int row_chunks(const FuseArgs& a)
{
    return (int)(((a.kind == 2? a.kpad : a.K) + 255) / 256);
}

// Sum over the WPR waves of one row (consecutive waves of the workgroup).
// Every wave of the workgroup must call it when WPR > 1 (it synchronises).
template <int WPR>
__device__ __forceinline__ double row_sum(double v, double* red, int wave)
{
    v = wave_sum_f64(v);
    if constexpr (WPR == 1) {
        return v;
    } else {
        if ((threadIdx.x & 63) == 0) red[wave] = v;
        __syncthreads();
        const int first = wave / WPR * WPR;
        double t = red[first];
#pragma unroll
        for (int i = 1; i < WPR; i++) t += red[first + i];
        __syncthreads();  // red is reused by the next sum
        return t;
    }
}

// WPR waves (1, 2 or 4) per token row, four waves per workgroup.  Wave `part`
// of a row owns chunks part, part + WPR, ...; with CACHE > 0 it keeps them (at
// most CACHE) in registers from the sums to the quantizer, with CACHE == 0
// (rows of more than 64 chunks) each pass re-reads the row.  CENTERED: layer
// norm (subtract the mean) rather than RMS norm.
//   mean   = (sum of x, in double) / K                      (centered only)
//   square = sum of (x - mean)^2 in double
//   inv    = (float)(1 / sqrt(square / K + eps))            (double)
//   y      = (float)(x - mean) * inv * w[k]  [* (1 + mod[k])]  (fp32)
// The double sums are formed in another order than the reference's running
// sum; `inv` is the fp32 rounding of a double that differs from the
// reference's in its last bits only.
template <int KIND, int WPR, int CACHE, bool CENTERED>
__global__ __launch_bounds__(64 * kNormWaves) void norm_quantize_kernel(FuseArgs a)
{
    constexpr int kRows = kNormWaves / WPR;  // rows per workgroup
    __shared__ double red[kNormWaves];
    // The norm weight and 1 + modulation, staged once per workgroup when the
    // launch gives dynamic LDS for them (2 * K floats), else read from memory.
    extern __shared__ float4 vec_lds[];
    const int lane = (int)(threadIdx.x & 63);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const size_t row = (size_t)blockIdx.x * kRows + wave / WPR;
    const int part = wave % WPR;
    const bool live = row < a.rows;  // wave-uniform
    const size_t K = a.K;
    const bool staged = a.stage_vectors != 0;
    if (WPR == 1 && !staged && !live) return;  // no barrier to reach
    const float* src = a.x + (live? row : 0) * K;
    const int nch = row_chunks(a);
    const int mine = live && nch > part? (nch - part + WPR - 1) / WPR : 0;  // chunks of this wave
    constexpr int kSlots = CACHE > 0? CACHE : 1;
    float4 v[kSlots];
    if constexpr (CACHE > 0) {
        // all of this wave's chunks at once (past `mine` they are zeros)
#pragma unroll
        for (int j = 0; j < CACHE; j++) {
            const size_t k0 = j < mine? (size_t)(part + WPR * j) * 256 + 4 * lane : K - 4;
            // Q8_K rows are whole chunks and slots past `mine` are never read
            if constexpr (KIND == 1) v[j] = *reinterpret_cast<const float4*>(src + k0);
            else v[j] = load4(src,K,j < mine? k0 : K);
        }
    }
    if (staged) {
        // The workgroup's copy of the vectors, every thread (also of a dead
        // row: it reaches the barrier below).  Unconditional loads (clamped
        // index; a missing vector reads the row instead and is replaced by
        // its neutral value), issued behind the row loads.
        constexpr int kIters = (int)(kStageMaxK / 4 / (64 * kNormWaves));
        const float4* wsrc = reinterpret_cast<const float4*>(a.w? a.w : src);
        const float4* msrc = reinterpret_cast<const float4*>(a.mod? a.mod : src);
        float4 wv[kIters], mv[kIters];
#pragma unroll
        for (int it = 0; it < kIters; it++) {
            const size_t i = threadIdx.x + (size_t)it * 64 * kNormWaves, ic = i < K / 4? i : K / 4 - 1;
            wv[it] = wsrc[ic];
            mv[it] = msrc[ic];
        }
#pragma unroll
        for (int it = 0; it < kIters; it++) {
            const size_t i = threadIdx.x + (size_t)it * 64 * kNormWaves;
            if (i < K / 4) {
                vec_lds[i] = a.w? wv[it] : make_float4(1.f,1.f,1.f,1.f);
                const float4 m = a.mod? mv[it] : make_float4(0.f,0.f,0.f,0.f);
                vec_lds[K / 4 + i] = make_float4(__fadd_rn(1.0f,m.x),__fadd_rn(1.0f,m.y),__fadd_rn(1.0f,m.z),__fadd_rn(1.0f,m.w));
            }
        }
        __syncthreads();
    }
    if (WPR == 1 && !live) return;
    auto chunk = [&](int j) -> float4 {
        if constexpr (CACHE > 0) return v[j < CACHE? j : CACHE - 1];  // (slots past CACHE are never live)
        else return load4(src,K,(size_t)(part + WPR * j) * 256 + 4 * lane);
    };
    const int J = CACHE > 0? CACHE : mine;

    double mean = 0.0;
    if constexpr (CENTERED) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            if (j < mine) {
                const float4 t = chunk(j);
                s += ((double)t.x + (double)t.y) + ((double)t.z + (double)t.w);
            }
        }
        mean = row_sum<WPR>(s,red,wave) / (double)K;
    }
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const size_t k0 = (size_t)(part + WPR * j) * 256 + 4 * lane;
        if (j < mine && (KIND == 1 || k0 < K)) {
            const float4 t = chunk(j);
            const double e0 = (double)t.x - mean, e1 = (double)t.y - mean, e2 = (double)t.z - mean, e3 = (double)t.w - mean;
            sq += (e0 * e0 + e1 * e1) + (e2 * e2 + e3 * e3);
        }
    }
    sq = row_sum<WPR>(sq,red,wave);
    if (!live) return;  // after the last barrier
    const float inv = (float)(1.0 / sqrt(sq / (double)K + (double)a.eps));

    // y of the wave's chunk j (zeros past the row's end)
    auto norm_y = [&](int j) -> float4 {
        const int c = part + WPR * j;
        const size_t k0 = (size_t)c * 256 + 4 * lane;
        float4 y = make_float4(0.f,0.f,0.f,0.f);
        if (KIND == 1 || k0 < K) {
            const float4 t = chunk(j);
            // weight and 1 + modulation: 1.0 where absent (multiplying by
            // 1.0 is exact, as the reference's empty weight is)
            float4 w4, m4;
            if (staged) {
                w4 = vec_lds[k0 / 4];
                m4 = vec_lds[K / 4 + k0 / 4];
            } else {
                w4 = a.w? *reinterpret_cast<const float4*>(a.w + k0) : make_float4(1.f,1.f,1.f,1.f);
                m4 = a.mod? *reinterpret_cast<const float4*>(a.mod + k0) : make_float4(0.f,0.f,0.f,0.f);
                m4 = make_float4(__fadd_rn(1.0f,m4.x),__fadd_rn(1.0f,m4.y),__fadd_rn(1.0f,m4.z),__fadd_rn(1.0f,m4.w));
            }
            const float xs[4] = {t.x,t.y,t.z,t.w}, ws[4] = {w4.x,w4.y,w4.z,w4.w}, ms[4] = {m4.x,m4.y,m4.z,m4.w};
            float ys[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // (float)(x - 0.0) is x: no double arithmetic without a mean
                const float c = CENTERED? (float)((double)xs[e] - mean) : xs[e];
                ys[e] = __fmul_rn(__fmul_rn(__fmul_rn(c,inv),ws[e]),ms[e]);
            }
            y = make_float4(ys[0],ys[1],ys[2],ys[3]);
        }
        return y;
    };
    if constexpr (KIND == 1) {
        // Q8_K: four chunks at a time through quantize_q8_K_x4 (16-lane row
        // q of the transposed set holds chunk slot j0 + q)
#pragma unroll
        for (int j0 = 0; j0 < J; j0 += 4) {
            float4 yv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int j = j0 + q;
                yv[q] = make_float4(0.f,0.f,0.f,0.f);
                if (j < mine) {  // wave-uniform
                    yv[q] = norm_y(j);
                    const size_t k0 = (size_t)(part + WPR * j) * 256 + 4 * lane;
                    if (a.y) *reinterpret_cast<float4*>(a.y + row * K + k0) = yv[q];
                }
            }
            float4 t[4];
            chunks_to_blocks(yv,t);
            uint32_t packed[4];
            float d;
            int gsum[4];
            quantize_q8_K_x4(t,lane,packed,d,gsum);
            const int jb = j0 + (lane >> 4);
            if (jb < mine) store_q8_K_x4(a,row,part + WPR * jb,lane,packed,d,gsum);
        }
    } else {
#pragma unroll
        for (int j = 0; j < J; j++) {
            if (j < mine) store_chunk<KIND>(a,row,part + WPR * j,lane,norm_y(j));  // wave-uniform
        }
    }
}

// Rows of up to 128 values written in fp32 only (the per-head q / k norm of
// a DiT block: rows x heads rows of 128): 16 lanes per row, four rows per wave.
// Lane l holds values 4(l%16) .. +3 and 64 + 4(l%16) .. +3 of row l/16, so
// each load's 16 lanes read 256 contiguous bytes; the double sums are 16-lane
// DPP reductions.  Same arithmetic as norm_quantize_kernel.
template <bool CENTERED>
__global__ __launch_bounds__(64 * kNormWaves) void norm_small_kernel(FuseArgs a)
{
    const int lane = (int)(threadIdx.x & 63), lp = lane & 15;
    const size_t row = ((size_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6)) * 4 + (size_t)(lane >> 4);
    const bool live = row < a.rows;
    const size_t K = a.K;
    const float* src = a.x + (live? row : a.rows - 1) * K;  // loads from a clamped row
    float4 v[2];
#pragma unroll
    for (int h = 0; h < 2; h++) v[h] = load4(src,K,(size_t)(64 * h + 4 * lp));
    auto row_sum16 = [](double t) {
        t += dpp_f64<kDppXor1>(t);
        t += dpp_f64<kDppXor2>(t);
        t += dpp_f64<kDppHalfMirror>(t);
        t += dpp_f64<kDppMirror>(t);
        return t;
    };
    double mean = 0.0;
    if constexpr (CENTERED) {
        double s = 0.0;
#pragma unroll
        for (int h = 0; h < 2; h++) s += ((double)v[h].x + (double)v[h].y) + ((double)v[h].z + (double)v[h].w);
        mean = row_sum16(s) / (double)K;
    }
    double sq = 0.0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        if ((size_t)(64 * h + 4 * lp) < K) {
            const double e0 = (double)v[h].x - mean, e1 = (double)v[h].y - mean, e2 = (double)v[h].z - mean, e3 = (double)v[h].w - mean;
            sq += (e0 * e0 + e1 * e1) + (e2 * e2 + e3 * e3);
        }
    }
    sq = row_sum16(sq);
    const float inv = (float)(1.0 / sqrt(sq / (double)K + (double)a.eps));
    if (!live) return;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const size_t k0 = (size_t)(64 * h + 4 * lp);
        if (k0 >= K) continue;
        const float4 w4 = a.w? *reinterpret_cast<const float4*>(a.w + k0) : make_float4(1.f,1.f,1.f,1.f);
        float4 m4 = a.mod? *reinterpret_cast<const float4*>(a.mod + k0) : make_float4(0.f,0.f,0.f,0.f);
        m4 = make_float4(__fadd_rn(1.0f,m4.x),__fadd_rn(1.0f,m4.y),__fadd_rn(1.0f,m4.z),__fadd_rn(1.0f,m4.w));
        const float xs[4] = {v[h].x,v[h].y,v[h].z,v[h].w}, ws[4] = {w4.x,w4.y,w4.z,w4.w}, ms[4] = {m4.x,m4.y,m4.z,m4.w};
        float ys[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float c = CENTERED? (float)((double)xs[e] - mean) : xs[e];
            ys[e] = __fmul_rn(__fmul_rn(__fmul_rn(c,inv),ws[e]),ms[e]);
        }
        *reinterpret_cast<float4*>(a.y + row * K + k0) = make_float4(ys[0],ys[1],ys[2],ys[3]);
    }
}

// SiLU of one value as the reference's tensor_silu computes it in fp32:
// v / (1.0f + expf(-v)).  expf is taken as the fp32 rounding of a double
// exponential (within 1e-16 relative of e^-v): the correctly rounded value.
// The reference's glibc expf rounds the other way for ~0.07% of arguments
// (those within ~0.0004 ulp of an fp32 midpoint).
__device__ __forceinline__ float silu_ref(float v)
{
    const float e = (float)exp(-(double)v);
    return __fdiv_rn(v,__fadd_rn(1.0f,e));
}

// One wave per 256-value chunk of one row: y = silu(gate) * up.
template <int KIND, bool FULL>
__global__ __launch_bounds__(64 * kGateWaves) void silu_gate_quantize_kernel(FuseArgs a)
{
    // Workgroup = (group of kGateRows rows, chunk), chunk fastest; wave w takes
    // rows w, w + kGateWaves, ...  A row group's scales for a block are written
    // by one workgroup: the transposed d planes get 64-byte runs instead of
    // 4-byte pieces from workgroups on different XCDs.
    constexpr int kPer = kGateRows / kGateWaves;
    const uint32_t nch = (uint32_t)row_chunks(a);
    const uint32_t group = blockIdx.x / nch;
    const int c = (int)(blockIdx.x % nch);
    const int lane = (int)(threadIdx.x & 63), wave = (int)(threadIdx.x >> 6);
    const size_t k0 = (size_t)c * 256 + 4 * lane, first = (size_t)group * kGateRows + wave;
    float4 g[kPer], u[kPer];
    // all loads first, from clamped rows and columns (zeros past K)
    for (int i = 0; i < kPer; i++) {
        const size_t row = first + (size_t)kGateWaves * i, r = row < a.rows? row : a.rows - 1;
        if constexpr (FULL) {  // whole 256-value chunks: no bounds on the loads
            g[i] = *reinterpret_cast<const float4*>(a.x + r * a.K + k0);
            u[i] = *reinterpret_cast<const float4*>(a.u + r * a.K + k0);
        } else {
            g[i] = load4(a.x + r * a.K,a.K,k0);
            u[i] = load4(a.u + r * a.K,a.K,k0);
        }
    }
    for (int i = 0; i < kPer; i++) {
        const size_t row = first + (size_t)kGateWaves * i;
        if (row >= a.rows) break;  // whole wave
        const float4 y = make_float4(__fmul_rn(silu_ref(g[i].x),u[i].x),__fmul_rn(silu_ref(g[i].y),u[i].y),
                                     __fmul_rn(silu_ref(g[i].z),u[i].z),__fmul_rn(silu_ref(g[i].w),u[i].w));
        store_chunk<KIND>(a,row,c,lane,y);
    }
}

template <int KIND>
static hipError_t launch_norm_kind(const FuseArgs& a, hipStream_t s)
{
    const size_t nch = ((a.kind == 2? a.kpad : a.K) + 255) / 256;
    const dim3 block(64 * kNormWaves);
    auto grid = [&](int wpr) { return dim3((unsigned)((a.rows + kNormWaves / wpr - 1) / (kNormWaves / wpr))); };
    // weight and 1 + modulation in LDS (2 * K floats) for rows of up to 4096 values
    FuseArgs b = a;
    b.stage_vectors = a.K <= kStageMaxK? 1 : 0;
    const size_t lds = b.stage_vectors? 2 * a.K * sizeof(float) : 0;
    auto go = [&](auto centered) {
        constexpr bool C = decltype(centered)::value;
        if (nch <= 1) norm_quantize_kernel<KIND,1,1,C><<<grid(1),block,lds,s>>>(b);
        else if (nch <= 2) norm_quantize_kernel<KIND,1,2,C><<<grid(1),block,lds,s>>>(b);
        else if (nch <= 4) norm_quantize_kernel<KIND,1,4,C><<<grid(1),block,lds,s>>>(b);
        else if (nch <= 8) norm_quantize_kernel<KIND,1,8,C><<<grid(1),block,lds,s>>>(b);
        else if (nch <= 16) norm_quantize_kernel<KIND,2,8,C><<<grid(2),block,lds,s>>>(b);
        else if (nch <= 32) norm_quantize_kernel<KIND,4,8,C><<<grid(4),block,lds,s>>>(b);
        else if (nch <= 64) norm_quantize_kernel<KIND,4,16,C><<<grid(4),block,lds,s>>>(b);
        else norm_quantize_kernel<KIND,4,0,C><<<grid(4),block,lds,s>>>(b);
    };
    if (a.centered) go(std::true_type{});
    else go(std::false_type{});
    return hipGetLastError();
}

static FuseArgs fuse_args(size_t rows, size_t K, int kind, size_t kpad, const ActOut& out)
{
    FuseArgs a = {};
    a.rows = rows;
    a.K = K;
    a.kind = kind;
    a.kpad = kind == 2? kpad : K;
    a.mpad = out.mpad;
    a.qs = out.qs;
    a.d = out.d;
    a.bs = out.bs;
    a.blocks = static_cast<uint8_t*>(out.blocks);
    a.y = out.y;
    return a;
}

hipError_t launch_norm_quantize(const float* x, size_t rows, size_t K, const float* weight, float eps, bool centered,
                                const float* modulation, int kind, size_t kpad, const ActOut& out, hipStream_t s)
{
    if (!rows) return hipSuccess;
    if (rows > 0x7fffffffu) return hipErrorInvalidValue;
    FuseArgs a = fuse_args(rows,K,kind,kpad,out);
    a.x = x;
    a.w = weight;
    a.mod = modulation;
    a.eps = eps;
    a.centered = centered? 1 : 0;
    if (kind == 0 && K <= 128 && !a.blocks) {
        // 16 lanes per row (a one-wave-per-row launch leaves half the lanes idle at 128 values)
        const size_t grid = (rows + 4 * kNormWaves - 1) / (4 * kNormWaves);
        if (centered) norm_small_kernel<true><<<dim3((unsigned)grid),dim3(64 * kNormWaves),0,s>>>(a);
        else norm_small_kernel<false><<<dim3((unsigned)grid),dim3(64 * kNormWaves),0,s>>>(a);
        return hipGetLastError();
    }
    if (kind == 1) return launch_norm_kind<1>(a,s);
    if (kind == 2) return launch_norm_kind<2>(a,s);
    return launch_norm_kind<0>(a,s);
}

hipError_t launch_silu_gate_quantize(const float* gate, const float* up, size_t rows, size_t K, int kind, size_t kpad,
                                     const ActOut& out, hipStream_t s)
{
    FuseArgs a = fuse_args(rows,K,kind,kpad,out);
    a.x = gate;
    a.u = up;
    const size_t nch = ((kind == 2? a.kpad : K) + 255) / 256;
    if (!rows || !nch) return hipSuccess;
    const size_t grid = (rows + kGateRows - 1) / kGateRows * nch;
    if (grid >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid), b(64 * kGateWaves);
    // whole chunks (and, for Q8_0, no planar padding chunk past K)
    const bool full = K % 256 == 0 && (kind != 2 || a.kpad == K);
    if (kind == 1) silu_gate_quantize_kernel<1,true><<<g,b,0,s>>>(a);
    else if (kind == 2 && full) silu_gate_quantize_kernel<2,true><<<g,b,0,s>>>(a);
    else if (kind == 2) silu_gate_quantize_kernel<2,false><<<g,b,0,s>>>(a);
    else if (full) silu_gate_quantize_kernel<0,true><<<g,b,0,s>>>(a);
    else silu_gate_quantize_kernel<0,false><<<g,b,0,s>>>(a);
    return hipGetLastError();
}

}  // namespace pixhip
