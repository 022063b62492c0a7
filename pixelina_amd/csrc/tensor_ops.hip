// The rest of the reference's backend op surface on device tensors (the
// counterparts of src/backend_vulkan.h:141-156 and of the CPU ops they stand
// in for).  All of it is HBM-bound data movement or one pass of arithmetic per
// value; each kernel moves contiguous runs of a row per wave (float4 where the
// shapes and pointers allow) and keeps the reference's fp32 operation order,
// so that results are bit-identical to the CPU path:
//   channel ops   z_modulate / z_residual (src/inference.cpp:263-291), the VAE
//                 and sampler affine steps (:474-478, :612-631),
//                 qwen_image_euler (src/qwen_image.cpp:347-361),
//                 qwen_image_modulate (:149-169)
//   l2norm        tensor_l2norm (src/tensor.cpp:242-258)
//   groupnorm     tensor_groupnorm (src/tensor.cpp:454-485)
//   decode        cpu_decode (src/backend_cpu.cpp:24-101) for vulkan_embedding
//   rows, copies  tensor_gather / tensor_scatter (src/tensor.cpp:274-302),
//                 vulkan_copy_rows / vulkan_copy_features
//                 (src/backend_vulkan.cpp:1257-1281)
//   layout        the DiT patch / unpatch loops (src/inference.cpp:374-390,
//                 :438-455) and tensor_upsample (src/tensor.cpp:304-319)
//   shortcut      tensor_resample_shortcut (src/tensor.cpp:487-527)
// tanh and the norms' sums are the exceptions: tanh is the fp32 rounding of the
// double function (the reference's glibc tanhf is within about an ulp of it),
// and the norms' double sums are formed in another order than the reference's
// running sums, which moves the fp32 results only when a double lands within
// its last bits of an fp32 rounding boundary.
#include <algorithm>

#include "pixhip_device.h"
#include "pixhip_internal.h"

namespace pixhip {

namespace {

unsigned grid_for(size_t work, size_t per_block = 256)
{
    return (unsigned)std::min<size_t>((work + per_block - 1) / per_block,(size_t)1 << 20);
}

// Copy-like kernels move kUnroll values per thread per pass, their loads
// issued together: a block's pass covers kUnroll * 256 consecutive values
// (value base + u * 256 + thread), so each wave keeps several KB in flight
// while the block still walks memory in order.
constexpr int kUnroll = 4;

unsigned grid_unrolled(size_t work)
{
    return grid_for((work + kUnroll - 1) / kUnroll);
}

bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <int VEC> struct Vec;
template <> struct Vec<1> {
    typedef float T;
    static __device__ __forceinline__ float get(const T& v, int) { return v; }
    static __device__ __forceinline__ void set(T& v, int, float x) { v = x; }
};
template <> struct Vec<4> {
    typedef float4 T;
    static __device__ __forceinline__ float get(const T& v, int i) { return i == 0? v.x : i == 1? v.y : i == 2? v.z : v.w; }
    static __device__ __forceinline__ void set(T& v, int i, float x)
    {
        if (i == 0) v.x = x;
        else if (i == 1) v.y = x;
        else if (i == 2) v.z = x;
        else v.w = x;
    }
};

// Non-temporal loads and stores of one Vec value. A stream's last read is
// non-temporal (groupnorm's statistics pass over [1M, 128]: 124 -> 91 us); an
// output is written non-temporally only when it exceeds kStreamBytes, the
// 256 MB Infinity Cache: a smaller one is better left there for its consumer
// (l2norm [256K, 96] then a reader of its output: 73 us with plain stores, 77
// with non-temporal ones; at [1M, 96] 280 and 265 us).
constexpr size_t kStreamBytes = (size_t)256 << 20;
template <typename T> __device__ __forceinline__ T nt_load(const T* p)
{
    if constexpr (sizeof(T) == 16) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v u = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
        return make_float4(u.x,u.y,u.z,u.w);
    } else {
        return __builtin_nontemporal_load(p);
    }
}

template <typename T> __device__ __forceinline__ void nt_store(const T& v, T* p)
{
    if constexpr (sizeof(T) == 16) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v u = {v.x,v.y,v.z,v.w};
        __builtin_nontemporal_store(u,reinterpret_cast<f4v*>(p));
    } else {
        __builtin_nontemporal_store(v,p);
    }
}

__device__ __forceinline__ float tanh_value(float v)
{
    return (float)tanh((double)v);
}

}  // namespace

// ---- channel ops ---------------------------------------------------------
//
// Thread (block x, lane) owns VEC consecutive channels and walks kChanRows
// rows of them, so the per-channel factor (1 + p, tanh p) is formed once:
//   MODULATE       x *= (1.0f + p0[c])
//   RESIDUAL       x += other[i] * tanh(p0[c])      (p0 NULL: x += other[i] * 1.0f)
//   AFFINE         x = x * scale + bias
//   EULER          x += other[i] * scale
//   QWEN_SCALE     x *= (1 + p[c]),         p = row >= split? p0 : p1
//   QWEN_RESIDUAL  x += other[i] * tanh(p[c]), p as above
constexpr int kChanRows = 8;

struct ChanArgs {
    float* x;
    const float* other;
    const float *p0, *p1;
    size_t rows, channels, split;
    float scale, bias;
};

template <int OP, int VEC>
__global__ __launch_bounds__(256) void channel_kernel(ChanArgs a)
{
    typedef typename Vec<VEC>::T T;
    const size_t c0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * VEC;
    if (c0 >= a.channels) return;
    float f0[VEC], f1[VEC];
#pragma unroll
    for (int j = 0; j < VEC; j++) {
        f0[j] = f1[j] = 1.0f;
        if constexpr (OP == kOpModulate || OP == kOpQwenScale) f0[j] = __fadd_rn(1.0f,a.p0[c0 + j]);
        if constexpr (OP == kOpQwenScale) f1[j] = __fadd_rn(1.0f,a.p1[c0 + j]);
        if constexpr (OP == kOpResidual) f0[j] = a.p0? tanh_value(a.p0[c0 + j]) : 1.0f;
        if constexpr (OP == kOpQwenResidual) {
            f0[j] = tanh_value(a.p0[c0 + j]);
            f1[j] = tanh_value(a.p1[c0 + j]);
        }
    }
    constexpr bool kOther = OP == kOpResidual || OP == kOpEuler || OP == kOpQwenResidual;
    const size_t r0 = (size_t)blockIdx.y * kChanRows;
    // every row's loads first (rows past the end re-read the last row), then
    // the arithmetic and the stores of the rows that exist
    T v[kChanRows], o[kChanRows];
#pragma unroll
    for (int k = 0; k < kChanRows; k++) {
        const size_t i = std::min(r0 + k,a.rows - 1) * a.channels + c0;
        v[k] = *reinterpret_cast<const T*>(a.x + i);
        if constexpr (kOther) o[k] = *reinterpret_cast<const T*>(a.other + i);
    }
#pragma unroll
    for (int k = 0; k < kChanRows; k++) {
        const size_t r = r0 + k;
        if (r >= a.rows) break;
        const bool first = r >= a.split;
#pragma unroll
        for (int j = 0; j < VEC; j++) {
            const float x = Vec<VEC>::get(v[k],j), f = first? f0[j] : f1[j];
            float y;
            if constexpr (OP == kOpModulate || OP == kOpQwenScale) y = __fmul_rn(x,f);
            else if constexpr (OP == kOpResidual || OP == kOpQwenResidual) y = __fadd_rn(x,__fmul_rn(Vec<VEC>::get(o[k],j),f));
            else if constexpr (OP == kOpAffine) y = __fadd_rn(__fmul_rn(x,a.scale),a.bias);
            else y = __fadd_rn(x,__fmul_rn(Vec<VEC>::get(o[k],j),a.scale));
            Vec<VEC>::set(v[k],j,y);
        }
        *reinterpret_cast<T*>(a.x + r * a.channels + c0) = v[k];
    }
}

template <int OP>
static hipError_t channel_launch(const ChanArgs& a, bool vec, hipStream_t s)
{
    const size_t vecw = vec? 4 : 1;
    const dim3 grid((unsigned)((a.channels / vecw + 255) / 256),(unsigned)((a.rows + kChanRows - 1) / kChanRows));
    if (vec) channel_kernel<OP,4><<<grid,dim3(256),0,s>>>(a);
    else channel_kernel<OP,1><<<grid,dim3(256),0,s>>>(a);
    return hipGetLastError();
}

hipError_t launch_channel_op(int op, float* x, const float* other, const float* p0, const float* p1, size_t rows, size_t channels,
                             size_t split, float scale, float bias, hipStream_t s)
{
    if (!rows || !channels) return hipSuccess;
    if ((rows + kChanRows - 1) / kChanRows > 65535) return hipErrorInvalidValue;
    const ChanArgs a{x,other,p0,p1,rows,channels,split,scale,bias};
    const bool vec = channels % 4 == 0 && aligned16(x) && (!other || aligned16(other)) && (!p0 || aligned16(p0)) &&
                     (!p1 || aligned16(p1));
    switch (op) {
    case kOpModulate: return channel_launch<kOpModulate>(a,vec,s);
    case kOpResidual: return channel_launch<kOpResidual>(a,vec,s);
    case kOpAffine: return channel_launch<kOpAffine>(a,vec,s);
    case kOpEuler: return channel_launch<kOpEuler>(a,vec,s);
    case kOpQwenScale: return channel_launch<kOpQwenScale>(a,vec,s);
    case kOpQwenResidual: return channel_launch<kOpQwenResidual>(a,vec,s);
    default: return hipErrorInvalidValue;
    }
}

// ---- l2norm ---------------------------------------------------------------
//
// A row per segment of L lanes (L a power of two, 64 / L rows per wave, four
// waves per block), so that short rows (the VAE's 96 channels: L = 8) keep
// every lane loading:
//   square  = sum of (double)x * x
//   inverse = (float)(sqrt((double)channels) / max(sqrt(square), (double)eps))
//   y       = x * inverse * w[c]      (fp32, left to right; w NULL: * 1)
// Rows of up to kL2Cache units per lane stay in registers between the two
// passes; longer rows are re-read (from L2, which the first pass filled).
constexpr int kL2Cache = 8;

// The weights of unit u (VEC of them, one load; 1.0 without a weight vector).
template <int VEC> __device__ __forceinline__ typename Vec<VEC>::T weights(const float* __restrict__ w, size_t u)
{
    typename Vec<VEC>::T t;
    if (w) return *reinterpret_cast<const typename Vec<VEC>::T*>(w + u * VEC);
#pragma unroll
    for (int j = 0; j < VEC; j++) Vec<VEC>::set(t,j,1.0f);
    return t;
}

template <int VEC, int L, bool NT>
__global__ __launch_bounds__(256) void l2norm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y,
                                                     size_t rows, size_t channels, float eps)
{
    typedef typename Vec<VEC>::T T;
    const int lane = threadIdx.x & 63, sl = lane % L;
    const size_t row = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    const bool valid = row < rows;
    const size_t units = channels / VEC;
    // rows past the end read the last row (in bounds) and write nothing: every
    // lane stays in the segment sums
    const float* in = x + (valid? row : rows - 1) * channels;
    float* out = y + row * channels;
    const double floor = (double)eps;
    double sq = 0.0;
    if (units <= (size_t)L * kL2Cache) {
        // the row's units held in registers: loads issued together, one read
        T v[kL2Cache];
#pragma unroll
        for (int k = 0; k < kL2Cache; k++) {
            const size_t u = sl + (size_t)k * L;
            if (u < units) {
                v[k] = nt_load(reinterpret_cast<const T*>(in + u * VEC));
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const double d = Vec<VEC>::get(v[k],j);
                    sq += d * d;
                }
            }
        }
#pragma unroll
        for (int m = 1; m < L; m <<= 1) sq += __shfl_xor(sq,m,64);
        if (!valid) return;
        const double root = sqrt(sq);
        const float inverse = (float)(sqrt((double)channels) / (root < floor? floor : root));
#pragma unroll
        for (int k = 0; k < kL2Cache; k++) {
            const size_t u = sl + (size_t)k * L;
            if (u < units) {
                const T wv = weights<VEC>(w,u);
#pragma unroll
                for (int j = 0; j < VEC; j++)
                    Vec<VEC>::set(v[k],j,__fmul_rn(__fmul_rn(Vec<VEC>::get(v[k],j),inverse),Vec<VEC>::get(wv,j)));
                if constexpr (NT) nt_store(v[k],reinterpret_cast<T*>(out + u * VEC));
                else *reinterpret_cast<T*>(out + u * VEC) = v[k];
            }
        }
        return;
    }
#pragma unroll 4
    for (size_t u = sl; u < units; u += L) {
        const T v = *reinterpret_cast<const T*>(in + u * VEC);
#pragma unroll
        for (int j = 0; j < VEC; j++) {
            const double d = Vec<VEC>::get(v,j);
            sq += d * d;
        }
    }
#pragma unroll
    for (int m = 1; m < L; m <<= 1) sq += __shfl_xor(sq,m,64);
    if (!valid) return;
    const double root = sqrt(sq);
    const float inverse = (float)(sqrt((double)channels) / (root < floor? floor : root));
#pragma unroll 4
    for (size_t u = sl; u < units; u += L) {
        T v = *reinterpret_cast<const T*>(in + u * VEC);
        const T wv = weights<VEC>(w,u);
#pragma unroll
        for (int j = 0; j < VEC; j++) Vec<VEC>::set(v,j,__fmul_rn(__fmul_rn(Vec<VEC>::get(v,j),inverse),Vec<VEC>::get(wv,j)));
        *reinterpret_cast<T*>(out + u * VEC) = v;
    }
}

template <int VEC, bool NT>
static void l2norm_lanes(int lanes, dim3 g, const float* x, const float* w, float* y, size_t rows, size_t channels, float eps,
                         hipStream_t s)
{
    const dim3 b(256);
    switch (lanes) {
    case 1: l2norm_kernel<VEC,1,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    case 2: l2norm_kernel<VEC,2,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    case 4: l2norm_kernel<VEC,4,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    case 8: l2norm_kernel<VEC,8,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    case 16: l2norm_kernel<VEC,16,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    case 32: l2norm_kernel<VEC,32,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    default: l2norm_kernel<VEC,64,NT><<<g,b,0,s>>>(x,w,y,rows,channels,eps); break;
    }
}

template <int VEC>
static hipError_t l2norm_launch(const float* x, const float* w, float* y, size_t rows, size_t channels, float eps, hipStream_t s)
{
    // lanes per row: all 64 for long rows, else about three units per lane
    // (96 channels: 8 lanes, each load's 8 lanes of a row reading one whole
    // 128-byte line; with 4 lanes a load read half lines of 16 rows:
    // 185 -> 145 us at [1M, 96])
    const size_t units = channels / VEC;
    int lanes = 64;
    if (units < 256)
        for (lanes = 1; lanes * 2 <= 64 && (size_t)lanes * 2 * 3 <= units;) lanes *= 2;
    const size_t per_block = 4 * (64 / lanes), blocks = (rows + per_block - 1) / per_block;
    if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
    const dim3 g((unsigned)blocks);
    if (rows * channels * sizeof(float) > kStreamBytes) l2norm_lanes<VEC,true>(lanes,g,x,w,y,rows,channels,eps,s);
    else l2norm_lanes<VEC,false>(lanes,g,x,w,y,rows,channels,eps,s);
    return hipGetLastError();
}

hipError_t launch_l2norm(const float* x, const float* w, float* y, size_t rows, size_t channels, float eps, hipStream_t s)
{
    if (!rows || !channels) return hipSuccess;
    if (channels % 4 == 0 && aligned16(x) && aligned16(y) && (!w || aligned16(w))) return l2norm_launch<4>(x,w,y,rows,channels,eps,s);
    return l2norm_launch<1>(x,w,y,rows,channels,eps,s);
}

// ---- groupnorm ------------------------------------------------------------
//
// 32 groups of gs = channels / 32 consecutive channels, each normalised over
// all rows (the VAE's GroupNorm over pixels):
//   mean    = sum of x / n                       (double, n = rows * gs)
//   square  = sum of (x - mean)^2                (double)
//   inverse = (float)(1 / sqrt(square / n + eps))
//   y       = (float)(x - mean) * inverse * w[c] + b[c]     (fp32)
// Three passes:
//   partial  a block holds kGnRows passes of a [rp rows x L columns] tile in
//            registers (columns of VEC channels, L a multiple of gs / VEC, so
//            no group straddles two tiles) and writes each group's chunk mean
//            and sum of squared deviations from it (two passes over the
//            registers, double);
//   merge    up to 64 blocks per group, then one, combine the chunks in a
//            fixed order with the pairwise update (Chan, Golub and LeVeque):
//            n = na + nb, d = mb - ma, mean = ma + d * nb / n,
//            M2 = M2a + M2b + d^2 na nb / n;
//   apply    one pass over x and the output.
// HBM traffic is two reads and one write of the tensor.
constexpr int kGroups = 32;
constexpr int kGnRows = 16;

// rows x channels in columns of VEC channels (cvec of them); a partial block
// covers a tile of `lanes` columns and rp * kGnRows rows (one chunk).
struct GnShape {
    size_t rows, channels, gs, cvec, chunks;
    int lanes, rp, tiles;
};

struct GnStat {
    double mean;
    float inverse;
    float pad;
};

// One non-temporal load of VEC floats at byte offset `off` of a raw buffer
// (zeros past its end).
template <int VEC> __device__ __forceinline__ typename Vec<VEC>::T nt_buffer_load(__amdgpu_buffer_rsrc_t r, int off)
{
    if constexpr (VEC == 4) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r,off,0,2);
        return make_float4(__uint_as_float(u.x),__uint_as_float(u.y),__uint_as_float(u.z),__uint_as_float(u.w));
    } else {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r,off,0,2));
    }
}

template <int VEC>
__global__ __launch_bounds__(256) void gn_partial_kernel(const float* __restrict__ x, GnShape sh, double* __restrict__ part)
{
    typedef typename Vec<VEC>::T T;
    __shared__ double red[256];
    __shared__ double colsum[256];
    __shared__ double gmean[256];
    const int t = threadIdx.x, col = t % sh.lanes, ro = t / sh.lanes;
    const size_t tile = blockIdx.y, chunk = blockIdx.x;
    const int cv = (int)(tile * sh.lanes) + col;
    const int q = (int)(sh.gs / VEC);  // columns per group
    const int tile_cols = (int)std::min<size_t>(sh.lanes,sh.cvec - tile * sh.lanes);
    const bool active = ro < sh.rp && col < tile_cols;
    const size_t row0 = chunk * sh.rp * kGnRows;
    const int valid = (int)std::min<size_t>(sh.rows - row0,(size_t)sh.rp * kGnRows);
    // The chunk's rows as one buffer (at most 4096 rows of 32768 channels):
    // 32-bit offsets, and the loads of rows past the end read zeros.
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x + row0 * sh.channels),(short)0,(int)((size_t)valid * sh.channels * 4),0x00020000);
    const int pitch = (int)sh.channels * 4 * sh.rp, first = (ro * (int)sh.channels + cv * VEC) * 4;
    T v[kGnRows];
    double sum[4] = {0.0,0.0,0.0,0.0};
    if (active) {
        // all loads first, then the sums (rows past the end add zero)
#pragma unroll
        for (int k = 0; k < kGnRows; k++) v[k] = nt_buffer_load<VEC>(rx,first + k * pitch);
#pragma unroll
        for (int k = 0; k < kGnRows; k++)
#pragma unroll
            for (int j = 0; j < VEC; j++) sum[k & 3] += (double)Vec<VEC>::get(v[k],j);
    }
    const int groups = tile_cols / q;
    const double n = (double)valid * (double)sh.gs;
    // pass 1: chunk means; pass 2: squared deviations from them
    for (int pass = 0; pass < 2; pass++) {
        double local = (sum[0] + sum[1]) + (sum[2] + sum[3]);
        if (pass == 1) {
            double dev[4] = {0.0,0.0,0.0,0.0};
            if (active) {
                const double m = gmean[col / q];
#pragma unroll
                for (int k = 0; k < kGnRows; k++) {
                    // hide the values from the compiler: it would otherwise keep
                    // the first pass's double conversions live (twice the registers)
#pragma unroll
                    for (int j = 0; j < VEC; j++) {
                        float f = Vec<VEC>::get(v[k],j);
                        asm volatile("" : "+v"(f));
                        Vec<VEC>::set(v[k],j,f);
                    }
                    if (ro + k * sh.rp < valid) {
#pragma unroll
                        for (int j = 0; j < VEC; j++) {
                            const double d = (double)Vec<VEC>::get(v[k],j) - m;
                            dev[k & 3] += d * d;
                        }
                    }
                }
            }
            local = (dev[0] + dev[1]) + (dev[2] + dev[3]);
        }
        red[t] = active? local : 0.0;
        __syncthreads();
        if (t < tile_cols) {
            double s = 0.0;
            for (int i = 0; i < sh.rp; i++) s += red[i * sh.lanes + t];
            colsum[t] = s;
        }
        __syncthreads();
        if (t < groups) {
            double s = 0.0;
            for (int i = 0; i < q; i++) s += colsum[t * q + i];
            const size_t g = (tile * sh.lanes) / q + t;
            if (pass == 0) {
                gmean[t] = s / n;
                part[(chunk * kGroups + g) * 2] = s / n;
            } else {
                part[(chunk * kGroups + g) * 2 + 1] = s;
            }
        }
        __syncthreads();
    }
}

// The pairwise update of (n, mean, M2) by another part (nb, mb, qb).
__device__ __forceinline__ void chan_merge(double& n, double& mean, double& m2, double nb, double mb, double qb)
{
    if (nb == 0.0) return;
    if (n == 0.0) {
        n = nb;
        mean = mb;
        m2 = qb;
        return;
    }
    const double total = n + nb, d = mb - mean;
    mean += d * (nb / total);
    m2 += qb + d * d * (n * nb / total);
    n = total;
}

// Block (g, s) merges entries [s * per, (s + 1) * per) of group g in a fixed
// order (each thread a strided run, then a tree over the block): with
// FROM_CHUNKS the partial kernel's (mean, M2) pairs, n of chunk c being its
// row count * gs; else (n, mean, M2) triples [32][count] of a first level.
// With several blocks per group (gridDim.y > 1) the result is a triple in
// `level`, else the group's statistics.
constexpr int kGnSplit = 64;  // most first-level merge blocks per group

template <bool FROM_CHUNKS>
__global__ __launch_bounds__(256) void gn_merge_kernel(const double* __restrict__ in, size_t count, GnShape sh, float eps,
                                                       double* __restrict__ level, GnStat* __restrict__ stat)
{
    __shared__ double sn[256], sm[256], s2[256];
    const int g = blockIdx.x, t = threadIdx.x;
    const size_t per = (count + gridDim.y - 1) / gridDim.y, begin = blockIdx.y * per, end = std::min(begin + per,count);
    const size_t per_chunk = (size_t)sh.rp * kGnRows;
    double n = 0.0, mean = 0.0, m2 = 0.0;
    for (size_t e = begin + t; e < end; e += 256) {
        if constexpr (FROM_CHUNKS) {
            const double nb = (double)std::min<size_t>(sh.rows - e * per_chunk,per_chunk) * (double)sh.gs;
            chan_merge(n,mean,m2,nb,in[(e * kGroups + g) * 2],in[(e * kGroups + g) * 2 + 1]);
        } else {
            const double* r = in + ((size_t)g * count + e) * 3;
            chan_merge(n,mean,m2,r[0],r[1],r[2]);
        }
    }
    sn[t] = n;
    sm[t] = mean;
    s2[t] = m2;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (t < stride) {
            double a = sn[t], b = sm[t], c = s2[t];
            chan_merge(a,b,c,sn[t + stride],sm[t + stride],s2[t + stride]);
            sn[t] = a;
            sm[t] = b;
            s2[t] = c;
        }
        __syncthreads();
    }
    if (t == 0) {
        if (gridDim.y > 1) {
            double* r = level + ((size_t)g * gridDim.y + blockIdx.y) * 3;
            r[0] = sn[0];
            r[1] = sm[0];
            r[2] = s2[0];
        } else {
            const double total = (double)sh.rows * (double)sh.gs;
            stat[g].mean = sm[0];
            stat[g].inverse = (float)(1.0 / sqrt(s2[0] / total + (double)eps));
            stat[g].pad = 0.0f;
        }
    }
}

// With FIXED (256 a multiple of cvec) every value of a thread lies in one
// column, whose weight, bias and group statistics are read once.
template <int VEC, bool FIXED, bool NT>
__global__ __launch_bounds__(256) void gn_apply_kernel(const float* __restrict__ x, GnShape sh, const GnStat* __restrict__ stat,
                                                       const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ y)
{
    typedef typename Vec<VEC>::T T;
    __shared__ GnStat st[kGroups];
    if (threadIdx.x < kGroups) st[threadIdx.x] = stat[threadIdx.x];
    __syncthreads();
    const size_t total = sh.rows * sh.cvec, span = (size_t)blockDim.x * kUnroll;
    const size_t spans = (total + span - 1) / span;
    float wf[VEC], bf[VEC];
    GnStat gf{};
    if constexpr (FIXED) {
        const size_t c = (threadIdx.x % sh.cvec) * VEC;
        gf = st[c / sh.gs];
#pragma unroll
        for (int j = 0; j < VEC; j++) {
            wf[j] = w[c + j];
            bf[j] = b[c + j];
        }
    }
    for (size_t p = blockIdx.x; p < spans; p += gridDim.x) {
        const size_t base = p * span + threadIdx.x;
        T v[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; k++)
            if (base + k * (size_t)blockDim.x < total) v[k] = nt_load(reinterpret_cast<const T*>(x + (base + k * (size_t)blockDim.x) * VEC));
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const size_t e = base + k * (size_t)blockDim.x;
            if (e >= total) break;
            if constexpr (FIXED) {
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const float d = (float)((double)Vec<VEC>::get(v[k],j) - gf.mean);
                    Vec<VEC>::set(v[k],j,__fadd_rn(__fmul_rn(__fmul_rn(d,gf.inverse),wf[j]),bf[j]));
                }
            } else {
                const size_t c = (e % sh.cvec) * VEC;
                const GnStat gs = st[c / sh.gs];
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const float d = (float)((double)Vec<VEC>::get(v[k],j) - gs.mean);
                    Vec<VEC>::set(v[k],j,__fadd_rn(__fmul_rn(__fmul_rn(d,gs.inverse),w[c + j]),b[c + j]));
                }
            }
            if constexpr (NT) nt_store(v[k],reinterpret_cast<T*>(y + e * VEC));
            else *reinterpret_cast<T*>(y + e * VEC) = v[k];
        }
    }
}

bool groupnorm_shape(size_t rows, size_t channels, bool vec, GnShape* sh)
{
    if (!rows || !channels || channels % kGroups) return false;
    const int w = vec? 4 : 1;
    sh->rows = rows;
    sh->channels = channels;
    sh->gs = channels / kGroups;
    if (sh->gs % w) return false;
    sh->cvec = channels / w;
    const size_t q = sh->gs / w;
    if (q > 256) return false;
    sh->lanes = (int)(sh->cvec <= 256? sh->cvec : 256 / q * q);
    sh->rp = 256 / sh->lanes;
    sh->tiles = (sh->cvec + sh->lanes - 1) / sh->lanes;
    sh->chunks = (rows + (size_t)sh->rp * kGnRows - 1) / ((size_t)sh->rp * kGnRows);
    return sh->chunks <= 0x7fffffffu && sh->tiles <= 65535;
}

// Workspace: the 32 group statistics, the first merge level's [32][64]
// triples, then [chunks][32] (mean, M2) pairs for the larger chunk count of
// the two column widths.
size_t groupnorm_workspace_bytes(size_t rows, size_t channels)
{
    GnShape scalar{}, vec{};
    if (!groupnorm_shape(rows,channels,false,&scalar)) return 0;
    size_t chunks = scalar.chunks;
    if (groupnorm_shape(rows,channels,true,&vec)) chunks = std::max(chunks,vec.chunks);
    return kGroups * sizeof(GnStat) + (kGroups * kGnSplit * 3 + chunks * kGroups * 2) * sizeof(double);
}

hipError_t launch_groupnorm(const float* x, const float* w, const float* b, float* y, size_t rows, size_t channels, float eps,
                            void* workspace, hipStream_t s)
{
    const bool vec = channels % (4 * kGroups) == 0 && aligned16(x) && aligned16(y);
    GnShape sh{};
    if (!groupnorm_shape(rows,channels,vec,&sh)) return hipErrorInvalidValue;
    GnStat* stat = static_cast<GnStat*>(workspace);
    double* level = reinterpret_cast<double*>(stat + kGroups);
    double* part = level + kGroups * kGnSplit * 3;
    const dim3 pgrid((unsigned)sh.chunks,(unsigned)sh.tiles), block(256);
    if (vec) gn_partial_kernel<4><<<pgrid,block,0,s>>>(x,sh,part);
    else gn_partial_kernel<1><<<pgrid,block,0,s>>>(x,sh,part);
    // at least 1024 chunks per first-level block
    const unsigned split = (unsigned)std::min<size_t>(kGnSplit,std::max<size_t>(1,(sh.chunks + 1023) / 1024));
    gn_merge_kernel<true><<<dim3(kGroups,split),block,0,s>>>(part,sh.chunks,sh,eps,level,stat);
    if (split > 1) gn_merge_kernel<false><<<dim3(kGroups,1),block,0,s>>>(level,split,sh,eps,nullptr,stat);
    const unsigned agrid = grid_unrolled(rows * sh.cvec);
    const bool fixed = 256 % sh.cvec == 0;
    auto apply = [&](auto nt) {
        constexpr bool NT = decltype(nt)::value;
        if (vec && fixed) gn_apply_kernel<4,true,NT><<<dim3(agrid),block,0,s>>>(x,sh,stat,w,b,y);
        else if (vec) gn_apply_kernel<4,false,NT><<<dim3(agrid),block,0,s>>>(x,sh,stat,w,b,y);
        else if (fixed) gn_apply_kernel<1,true,NT><<<dim3(agrid),block,0,s>>>(x,sh,stat,w,b,y);
        else gn_apply_kernel<1,false,NT><<<dim3(agrid),block,0,s>>>(x,sh,stat,w,b,y);
    };
    if (rows * channels * sizeof(float) > kStreamBytes) apply(std::true_type());
    else apply(std::false_type());
    return hipGetLastError();
}

// ---- decode (embedding rows) ----------------------------------------------
//
// Row r of the output is row ids[r] (ids NULL: row r) of a table of GGUF rows
// `stride` bytes apart, decoded as cpu_decode does, in its fp32 order:
//   F32 the bits; BF16 the bits << 16; F16 exact (NaN as the reference's
//   half_float: a quiet NaN with the sign, whatever the payload);
//   Q8_0  (float)q * d
//   Q5_K  d * scale * q - dmin * min
//   Q6_K  d * scale * (q - 32)
// One thread per output value; the block bytes it reads are shared with its
// neighbours through the cache.
__device__ __forceinline__ float half_float_ref(uint16_t h)
{
    if ((h & 0x7c00u) == 0x7c00u && (h & 0x03ffu)) return __uint_as_float((h & 0x8000u)? 0xffc00000u : 0x7fc00000u);
    return half_bits_to_float(h);
}

__device__ __forceinline__ uint16_t load16(const uint8_t* p)
{
    return (uint16_t)(p[0] | (p[1] << 8));
}

template <uint32_t TYPE>
__device__ __forceinline__ float decode_value(const uint8_t* row, size_t j)
{
    if constexpr (TYPE == PIX_F32) {
        return __uint_as_float((uint32_t)row[4 * j] | ((uint32_t)row[4 * j + 1] << 8) | ((uint32_t)row[4 * j + 2] << 16) |
                               ((uint32_t)row[4 * j + 3] << 24));
    } else if constexpr (TYPE == PIX_F16) {
        return half_float_ref(load16(row + 2 * j));
    } else if constexpr (TYPE == PIX_BF16) {
        return __uint_as_float((uint32_t)load16(row + 2 * j) << 16);
    } else if constexpr (TYPE == PIX_Q8_0) {
        const uint8_t* blk = row + (j / PIX_QK8) * PIX_Q8_0_BYTES;
        return __fmul_rn((float)(int8_t)blk[2 + j % PIX_QK8],half_float_ref(load16(blk)));
    } else if constexpr (TYPE == PIX_Q5_K) {
        const uint8_t* blk = row + (j / PIX_QK) * PIX_Q5_K_BYTES;
        const unsigned within = (unsigned)(j % PIX_QK), group = within / 32, i = within % 32;
        const uint8_t* sc = blk + 4;
        unsigned scale, min;
        if (group < 4) {
            scale = sc[group] & 63u;
            min = sc[group + 4] & 63u;
        } else {
            scale = (sc[group + 4] & 15u) | ((unsigned)(sc[group - 4] >> 6) << 4);
            min = (unsigned)(sc[group + 4] >> 4) | ((unsigned)(sc[group] >> 6) << 4);
        }
        unsigned q = blk[48 + (group / 2) * 32 + i];
        q = group % 2? q >> 4 : q & 15u;
        if (blk[16 + i] & (1u << group)) q += 16;
        const float d = half_float_ref(load16(blk)), dmin = half_float_ref(load16(blk + 2));
        return __fsub_rn(__fmul_rn(__fmul_rn(d,(float)scale),(float)q),__fmul_rn(dmin,(float)min));
    } else {
        const uint8_t* blk = row + (j / PIX_QK) * PIX_Q6_K_BYTES;
        const unsigned within = (unsigned)(j % PIX_QK), half = within / 128, group = (within % 128) / 32, i = within % 32;
        unsigned q = blk[half * 64 + i + (group % 2) * 32];
        q = group < 2? q & 15u : q >> 4;
        q |= ((unsigned)(blk[128 + half * 32 + i] >> (group * 2)) & 3u) << 4;
        const int scale = (int8_t)blk[192 + half * 8 + i / 16 + group * 2];
        return __fmul_rn(__fmul_rn(half_float_ref(load16(blk + 208)),(float)scale),(float)((int)q - 32));
    }
}

template <uint32_t TYPE>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t* __restrict__ table, const int64_t* __restrict__ ids, size_t stride,
                                                     size_t count, size_t inner, float* __restrict__ out)
{
    const size_t total = count * inner, step = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const size_t r = e / inner, j = e % inner;
        const uint8_t* row = table + (size_t)(ids? ids[r] : (int64_t)r) * stride;
        out[e] = decode_value<TYPE>(row,j);
    }
}

hipError_t launch_decode_rows(const void* table, uint32_t type, size_t stride, const int64_t* ids, size_t count, size_t inner, float* out,
                              hipStream_t s)
{
    if (!count || !inner) return hipSuccess;
    const dim3 g(grid_for(count * inner)), b(256);
    const uint8_t* t = static_cast<const uint8_t*>(table);
    switch (type) {
    case PIX_F32: decode_kernel<PIX_F32><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    case PIX_F16: decode_kernel<PIX_F16><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    case PIX_BF16: decode_kernel<PIX_BF16><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    case PIX_Q8_0: decode_kernel<PIX_Q8_0><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    case PIX_Q5_K: decode_kernel<PIX_Q5_K><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    case PIX_Q6_K: decode_kernel<PIX_Q6_K><<<g,b,0,s>>>(t,ids,stride,count,inner,out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- row moves ------------------------------------------------------------
//
// Destination row dst_rows[k] (NULL: k) = source row src_rows[k] (NULL: k),
// k < n, `cvec` columns of VEC floats, rows `src_stride` / `dst_stride` floats
// apart.  A block moves kMoveRows rows of 256 columns (column blockIdx.x * 256
// + thread), all its loads (non-temporal: the DiT's three-way split of the
// fused qkv, 92 -> 76 us) issued before the stores, and strides over the rows
// in y.
constexpr int kMoveRows = 4;

template <int VEC>
__global__ __launch_bounds__(256) void move_rows_kernel(const float* __restrict__ src, size_t src_stride, float* __restrict__ dst,
                                                        size_t dst_stride, const uint64_t* __restrict__ src_rows,
                                                        const uint64_t* __restrict__ dst_rows, size_t n, size_t cvec)
{
    typedef typename Vec<VEC>::T T;
    const size_t j = ((size_t)blockIdx.x * 256 + threadIdx.x) * VEC;
    if (j >= cvec * VEC) return;
    for (size_t r0 = (size_t)blockIdx.y * kMoveRows; r0 < n; r0 += (size_t)gridDim.y * kMoveRows) {
        T v[kMoveRows];
#pragma unroll
        for (int u = 0; u < kMoveRows; u++) {
            const size_t k = std::min(r0 + u,n - 1);
            v[u] = nt_load(reinterpret_cast<const T*>(src + (src_rows? src_rows[k] : k) * src_stride + j));
        }
#pragma unroll
        for (int u = 0; u < kMoveRows; u++) {
            const size_t k = r0 + u;
            if (k >= n) break;
            *reinterpret_cast<T*>(dst + (dst_rows? dst_rows[k] : k) * dst_stride + j) = v[u];
        }
    }
}

static hipError_t move_rows(const float* src, size_t src_stride, float* dst, size_t dst_stride, const uint64_t* src_rows,
                            const uint64_t* dst_rows, size_t n, size_t columns, hipStream_t s)
{
    if (!n || !columns) return hipSuccess;
    const bool vec = columns % 4 == 0 && src_stride % 4 == 0 && dst_stride % 4 == 0 && aligned16(src) && aligned16(dst);
    const size_t cvec = vec? columns / 4 : columns;
    if ((cvec + 255) / 256 > 0x7fffffffu) return hipErrorInvalidValue;
    const dim3 g((unsigned)((cvec + 255) / 256),(unsigned)std::min<size_t>((n + kMoveRows - 1) / kMoveRows,65535)), b(256);
    if (vec) move_rows_kernel<4><<<g,b,0,s>>>(src,src_stride,dst,dst_stride,src_rows,dst_rows,n,cvec);
    else move_rows_kernel<1><<<g,b,0,s>>>(src,src_stride,dst,dst_stride,src_rows,dst_rows,n,cvec);
    return hipGetLastError();
}

hipError_t launch_rows(const float* src, float* dst, const uint64_t* src_rows, const uint64_t* dst_rows, size_t n, size_t channels,
                       hipStream_t s)
{
    return move_rows(src,channels,dst,channels,src_rows,dst_rows,n,channels,s);
}

hipError_t launch_copy2d(const float* src, size_t src_stride, float* dst, size_t dst_stride, size_t rows, size_t columns, hipStream_t s)
{
    return move_rows(src,src_stride,dst,dst_stride,nullptr,nullptr,rows,columns,s);
}

// ---- layout ---------------------------------------------------------------
//
// Each destination value (VEC of them at a time; VEC = 4 needs the run of
// `inner` channels that moves together to be a multiple of 4) reads one source
// value:
//   PATCH    dst [ (W/p)(H/p) ][ p*p*C ]: token t, feature f -> pixel
//            (x, y) = ((t % (W/p))*p + (f/C) % p, (t / (W/p))*p + (f/C) / p),
//            channel f % C
//   UNPATCH  dst [ W*H ][ C ]: pixel (x, y), channel c -> token
//            (y/p)*(W/p) + x/p, feature ((y % p)*p + x % p)*C + c
//   UPSAMPLE dst [ 4*W*H ][ C ]: pixel (x, y) of width 2W -> (x/2, y/2)
// (W the source width for PATCH and UPSAMPLE, the destination width for UNPATCH.)
// A destination larger than kStreamBytes is written non-temporally (UPSAMPLE
// [512x512, 128] -> [1024x1024, 128]: 128 -> 93 us).
template <int OP, int VEC, typename I, bool NT>
__global__ __launch_bounds__(256) void layout_kernel(const float* __restrict__ src, float* __restrict__ dst, I rows, I channels, I width,
                                                     I src_channels, I patch)
{
    typedef typename Vec<VEC>::T T;
    const I cvec = channels / VEC, total = rows * cvec, step = (I)gridDim.x * blockDim.x;
    for (I e = (I)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const I row = e / cvec, f = (e % cvec) * VEC;
        I from;
        if constexpr (OP == kLayoutPatch) {
            const I pw = width / patch, pixel = f / src_channels;
            const I x = (row % pw) * patch + pixel % patch, y = (row / pw) * patch + pixel / patch;
            from = (y * width + x) * src_channels + f % src_channels;
        } else if constexpr (OP == kLayoutUnpatch) {
            const I x = row % width, y = row / width;
            const I token = (y / patch) * (width / patch) + x / patch;
            from = token * src_channels + ((y % patch) * patch + x % patch) * channels + f;
        } else {
            const I x = row % (width * 2), y = row / (width * 2);
            from = ((y / 2) * width + x / 2) * channels + f;
        }
        const T v = *reinterpret_cast<const T*>(src + from);
        if constexpr (NT) nt_store(v,reinterpret_cast<T*>(dst + (size_t)e * VEC));
        else *reinterpret_cast<T*>(dst + (size_t)e * VEC) = v;
    }
}

template <int OP, bool NT>
static void layout_launch(const float* src, float* dst, size_t rows, size_t channels, size_t width, size_t src_channels, size_t patch,
                          bool vec, hipStream_t s)
{
    const dim3 g(grid_for(rows * (vec? channels / 4 : channels))), b(256);
    // 32-bit index arithmetic when every index fits, the loop's last step
    // included (the grid is at most 2^28 threads): the destination holds the
    // most values (the source as many, or a quarter for UPSAMPLE)
    const bool narrow = rows * channels < (1ull << 31);
    if (vec && narrow)
        layout_kernel<OP,4,uint32_t,NT><<<g,b,0,s>>>(src,dst,(uint32_t)rows,(uint32_t)channels,(uint32_t)width,(uint32_t)src_channels,
                                                     (uint32_t)patch);
    else if (vec)
        layout_kernel<OP,4,size_t,NT><<<g,b,0,s>>>(src,dst,rows,channels,width,src_channels,patch);
    else if (narrow)
        layout_kernel<OP,1,uint32_t,NT><<<g,b,0,s>>>(src,dst,(uint32_t)rows,(uint32_t)channels,(uint32_t)width,(uint32_t)src_channels,
                                                     (uint32_t)patch);
    else
        layout_kernel<OP,1,size_t,NT><<<g,b,0,s>>>(src,dst,rows,channels,width,src_channels,patch);
}

template <int OP>
static hipError_t layout_launch(const float* src, float* dst, size_t rows, size_t channels, size_t width, size_t src_channels, size_t patch,
                                bool vec, hipStream_t s)
{
    if (rows * channels * sizeof(float) > kStreamBytes) layout_launch<OP,true>(src,dst,rows,channels,width,src_channels,patch,vec,s);
    else layout_launch<OP,false>(src,dst,rows,channels,width,src_channels,patch,vec,s);
    return hipGetLastError();
}

hipError_t launch_layout(int op, const float* src, float* dst, size_t rows, size_t channels, size_t width, size_t src_channels, size_t patch,
                         hipStream_t s)
{
    if (!rows || !channels) return hipSuccess;
    // the run of channels that stays contiguous through the move
    const size_t run = op == kLayoutPatch? src_channels : channels;
    const bool vec = run % 4 == 0 && channels % 4 == 0 && src_channels % 4 == 0 && aligned16(src) && aligned16(dst);
    switch (op) {
    case kLayoutPatch: return layout_launch<kLayoutPatch>(src,dst,rows,channels,width,src_channels,patch,vec,s);
    case kLayoutUnpatch: return layout_launch<kLayoutUnpatch>(src,dst,rows,channels,width,src_channels,patch,vec,s);
    case kLayoutUpsample: return layout_launch<kLayoutUpsample>(src,dst,rows,channels,width,src_channels,patch,vec,s);
    default: return hipErrorInvalidValue;
    }
}

// ---- resample shortcut ----------------------------------------------------
//
// Output pixel (x, y) of the resampled width, channel c, with side = 2 when
// spatial (else 1) and factor = temporal * side * side:
//   up    source pixel (x/side, y/side), channel (c*factor + (temporal-1)*side*side
//         + (y % side)*side + x % side) / (channels*factor / src_channels)
//   down  over the group = src_channels*factor / channels items i = c*group + k,
//         those whose time index i / (side*side) % temporal is the last add
//         source pixel (x*side + i % side, y*side + i/side % side), channel
//         i / factor, to an fp32 running sum in k order; then / group.
__global__ __launch_bounds__(256) void shortcut_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t out_rows, size_t channels,
                                                       size_t src_channels, size_t width, size_t side, size_t temporal, bool up)
{
    const size_t factor = temporal * side * side, out_width = up? width * side : width / side;
    const size_t total = out_rows * channels, step = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const size_t c = e % channels, pixel = e / channels, x = pixel % out_width, y = pixel / out_width;
        float value = 0.0f;
        if (up) {
            const size_t repeats = channels * factor / src_channels;
            const size_t source = (c * factor + (temporal - 1) * side * side + (y % side) * side + x % side) / repeats;
            value = src[((y / side) * width + x / side) * src_channels + source];
        } else {
            const size_t group = src_channels * factor / channels;
            for (size_t k = 0; k < group; k++) {
                const size_t item = c * group + k, source = item / factor;
                const size_t time = item / (side * side) % temporal, dy = item / side % side, dx = item % side;
                if (time == temporal - 1) value = __fadd_rn(value,src[((y * side + dy) * width + x * side + dx) * src_channels + source]);
            }
            value = __fdiv_rn(value,(float)group);
        }
        dst[e] = value;
    }
}

hipError_t launch_shortcut(const float* src, float* dst, size_t out_rows, size_t channels, size_t src_channels, size_t width, size_t side,
                           size_t temporal, bool up, hipStream_t s)
{
    if (!out_rows || !channels) return hipSuccess;
    shortcut_kernel<<<dim3(grid_for(out_rows * channels)),dim3(256),0,s>>>(src,dst,out_rows,channels,src_channels,width,side,temporal,up);
    return hipGetLastError();
}

}  // namespace pixhip
