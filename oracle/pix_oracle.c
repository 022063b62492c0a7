/* Oracle: plain-C restatement of Pixelina's CPU quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see pix_oracle.h).  Nothing in pixelina_amd/ links
 * or loads this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg do, as the checker.
 *
 * The reference computes with AVX2 intrinsics; this file restates the same
 * arithmetic one scalar lane at a time, in the same order, so that results are
 * bit-identical to the compiled reference (checked against golden vectors it
 * wrote, tests/golden/).  Two facts of the compiled reference are part of the
 * specification, established from the reference built with its own Makefile
 * flags (g++ -O3 -std=c++17):
 *   - nearest_int(iscale*x) in quantize_row_q8_K_ref is contracted into one
 *     fused multiply-add, fma(iscale, x, 12582912.f)
 *     (src/kernels_quant.cpp:41-48, :105);
 *   - `summs += dmin * isum` in pix_dot_q5_K is contracted into
 *     fma(dmin, (float)isum, summs) (src/kernels_quant.cpp:202).
 * Everything else is evaluated exactly as written (no other contraction).
 *
 * Build: gcc -std=c11 -O2 -ffp-contract=off (oracle/Makefile).
 *
 * ORC_MUTANT (default 0) plants one plausible mistake per value, for the
 * tests that show the golden vectors catch it (tests/test_oracle_pins.py
 * compiles such copies into a temporary directory; nothing else sets it):
 *   1 nearest_int rounded after a separate multiply (no fused multiply-add)
 *   2 hsum8 summed left to right
 *   3 Q5_K min term accumulated without the fused multiply-add
 *   4 Q8_0 quantizer dividing by the fp16-rounded scale
 *   5 Q5_K six-bit unpack of sub-blocks 4..7 taking the wrong high bits
 *   6 Q8_K quantizer keeping the last (not the first) largest |x|
 *   7 norm adding epsilon after the square root
 *   8 norm multiplying by the weight before the inverse
 *   9 centered norm subtracting the mean in fp32
 *  10 SiLU as v * (1 / (1 + e)) instead of a division
 *  11 RoPE with the sine's sign flipped
 *  12 tanh GELU with v*v instead of v*v*v
 *  13 modulation as x + x*scale instead of x*(1 + scale)
 *  14 modulation by scale instead of 1 + scale
 *  15 attention's grouped heads as head % kv_heads
 *  16 causal attention without the query's own key
 *  17 l2norm without the sqrt(channels) factor
 *  18 l2norm adding epsilon instead of taking the larger
 *  19 groupnorm variance over n - 1
 *  20 groupnorm weight and bias indexed by group
 *  21 BF16 decoded as F16
 *  22 F16 decode keeping the NaN payload
 *  23 scatter keeping the first of a repeated row
 *  24 patch layout with dx and dy swapped
 *  25 upsample reading rows of the doubled width
 *  26 shortcut (down) without the division by the group
 *  27 shortcut (up) from the first time step
 *  28 qwen modulation with the two parameter rows swapped
 *  29 residual gate without tanh
 *  30 affine adding the bias before the scale
 *  31 convolution patches with the kernel's x and y swapped
 *  32 convolution padding taken from the right instead of the left
 */
#ifndef ORC_MUTANT
#define ORC_MUTANT 0
#endif
#include "pix_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
#define QK8_0 32
#define Q8_0_BYTES 34
#define Q8_K_BYTES 292
#define Q5_K_BYTES 176
#define Q6_K_BYTES 210

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static float rdf32(const uint8_t* p) { float f; memcpy(&f,p,4); return f; }
static void wrf32(uint8_t* p, float f) { memcpy(p,&f,4); }

/* half_float, src/backend_cpu.cpp:12-22 (also what _cvtsh_ss computes). */
float orc_half_to_float(uint16_t h)
{
    uint32_t sign = h & 0x8000u, exponent = (h >> 10) & 31u, mantissa = h & 1023u;
    float r;
    if (!exponent) r = ldexpf((float)mantissa,-24);
    else if (exponent == 31u) r = mantissa? NAN : INFINITY;
    else r = ldexpf((float)(mantissa + 1024u),(int)exponent - 25);
    return sign? -r : r;
}

/* _cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT), src/kernels_quant.cpp:136:
 * round-to-nearest-even, subnormals kept, overflow to infinity, NaN quieted. */
uint16_t orc_float_to_half(float f)
{
    uint32_t x;
    memcpy(&x,&f,4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exponent = (x >> 23) & 0xffu, mantissa = x & 0x7fffffu;
    if (exponent == 0xffu) return (uint16_t)(sign | 0x7c00u | (mantissa? 0x200u | (mantissa >> 13) : 0u));
    int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t h = ((uint32_t)e << 10) | (mantissa >> 13), rem = mantissa & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | (h >= 0x7c00u? 0x7c00u : h));
    }
    int shift = 126 - (int)exponent;
    if (exponent == 0 || shift > 24) return sign;
    uint32_t m = mantissa | 0x800000u, h = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* nearest_int as compiled into quantize_row_q8_K_ref (src/kernels_quant.cpp:41-48):
 * bits(fma(scale, x, 1.5*2^23)) & 0x7fffff - 0x400000. */
int orc_nearest_int_fused(float scale, float x)
{
#if ORC_MUTANT == 1
    float p = scale * x;
    float v = p + 12582912.0f;
#else
    float v = fmaf(scale,x,12582912.0f);
#endif
    int32_t i;
    memcpy(&i,&v,4);
    return (i & 0x007fffff) - 0x00400000;
}

/* vcvttss2si: truncation, 0x80000000 for NaN and out-of-range. */
static int32_t cvtt_i32(float f)
{
    if (f != f || f >= 2147483648.0f || f < -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* quantize_row_q8_0_ref, src/kernels_quant.cpp:120-144 */
void orc_quantize_q8_0(const float* x, void* blocks, int64_t k)
{
    uint8_t* y = (uint8_t*)blocks;
    int nb = (int)(k / QK8_0);
    for (int i = 0; i < nb; i++, x += QK8_0, y += Q8_0_BYTES) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) {
            float ax = fabsf(x[j]);
            amax = (amax < ax)? ax : amax; /* std::max(amax, |v|), :130 */
        }
        float d = amax / 127.0f;
        float id = (d != 0.0f)? 1.0f / d : 0.0f;
#if ORC_MUTANT == 4
        id = (d != 0.0f)? 1.0f / orc_half_to_float(orc_float_to_half(d)) : 0.0f;
#endif
        wr16(y,orc_float_to_half(d));
        for (int j = 0; j < QK8_0; j++) {
            float x0 = x[j] * id;
            y[2 + j] = (uint8_t)(cvtt_i32(roundf(x0)) & 0xff);
        }
    }
}

/* quantize_row_q8_K_ref, src/kernels_quant.cpp:80-118 */
void orc_quantize_q8_K(const float* x, void* blocks, int64_t k)
{
    uint8_t* y = (uint8_t*)blocks;
    int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++, x += QK_K, y += Q8_K_BYTES) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; j++) {
            float ax = fabsf(x[j]);
#if ORC_MUTANT == 6
            if (ax >= amax && ax > 0.0f) {
#else
            if (ax > amax) {
#endif
                amax = ax;
                max = x[j];
            }
        }
        if (amax == 0.0f) {
            memset(y,0,Q8_K_BYTES);
            continue;
        }
        float iscale = -127.0f / max;
        int8_t q[QK_K];
        for (int j = 0; j < QK_K; j++) {
            int v = orc_nearest_int_fused(iscale,x[j]);
            q[j] = (int8_t)(uint8_t)((v < 127? v : 127) & 0xff);
        }
        memcpy(y + 4,q,QK_K);
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int ii = 0; ii < 16; ii++) sum += q[j * 16 + ii];
            wr16(y + 4 + QK_K + 2 * j,(uint16_t)(int16_t)sum);
        }
        wrf32(y,1.0f / iscale);
    }
}

/* pix_quant_hsum, src/kernels_quant.cpp:146-153:
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static float hsum8(const float a[8])
{
#if ORC_MUTANT == 2
    return ((((((a[0] + a[1]) + a[2]) + a[3]) + a[4]) + a[5]) + a[6]) + a[7];
#endif
    float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
    float s0 = r0 + r2, s1 = r1 + r3;
    return s0 + s1;
}

static int32_t sat16(int32_t v) { return v > 32767? 32767 : (v < -32768? -32768 : v); }
static int8_t wrap8(int v) { return (int8_t)(uint8_t)(v & 0xff); }

/* pix_quant_mul_pairs, src/kernels_quant.cpp:155-161, one int32 lane:
 * maddubs(sign(x,x), sign(y,x)) then madd with ones, over 4 adjacent bytes. */
static int32_t mul_pairs_lane(const int8_t* x, const int8_t* y)
{
    int32_t pair[2];
    for (int p = 0; p < 2; p++) {
        int32_t s = 0;
        for (int i = 0; i < 2; i++) {
            int8_t xv = x[2 * p + i], yv = y[2 * p + i];
            uint8_t ax = (uint8_t)(xv < 0? wrap8(-xv) : xv);
            int8_t sy = xv < 0? wrap8(-yv) : (xv == 0? 0 : yv);
            s += (int32_t)ax * (int32_t)sy;
        }
        pair[p] = sat16(s);
    }
    return pair[0] + pair[1];
}

/* pix_dot_q8_0, src/kernels_quant.cpp:339-365 */
float orc_dot_q8_0(int n, const void* wv, const void* av)
{
    const uint8_t* w = (const uint8_t*)wv;
    const uint8_t* a = (const uint8_t*)av;
    float acc[8] = {0};
    for (int b = 0; b < n / QK8_0; b++, w += Q8_0_BYTES, a += Q8_0_BYTES) {
        float d = orc_half_to_float(rd16(w)) * orc_half_to_float(rd16(a));
        for (int t = 0; t < 8; t++) {
            int32_t p = mul_pairs_lane((const int8_t*)w + 2 + 4 * t,(const int8_t*)a + 2 + 4 * t);
            acc[t] = fmaf(d,(float)p,acc[t]);
        }
    }
    return hsum8(acc);
}

/* Six-bit scale/min unpack; same values as the utmp word shuffle of
 * src/kernels_quant.cpp:189-194 and the decoder of src/backend_cpu.cpp:64-70. */
static void q5_scales(const uint8_t* sc, int scale[8], int min[8])
{
    for (int s = 0; s < 8; s++) {
        if (s < 4) {
            scale[s] = sc[s] & 63;
            min[s] = sc[s + 4] & 63;
        } else {
#if ORC_MUTANT == 5
            scale[s] = (sc[s + 4] & 15) | ((sc[s - 4] >> 4 & 3) << 4);
#else
            scale[s] = (sc[s + 4] & 15) | ((sc[s - 4] >> 6) << 4);
#endif
            min[s] = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
        }
    }
}

static int q5_value(const uint8_t* blk, int s, int i)
{
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    int low = (qs[(s / 2) * 32 + i] >> (4 * (s % 2))) & 15;
    return low | (((qh[i] >> s) & 1) << 4);
}

/* pix_dot_q5_K, src/kernels_quant.cpp:163-254 */
float orc_dot_q5_K(int n, const void* wv, const void* av)
{
    const uint8_t* w = (const uint8_t*)wv;
    const uint8_t* a = (const uint8_t*)av;
    float acc[8] = {0};
    float summs = 0.0f;
    for (int b = 0; b < n / QK_K; b++, w += Q5_K_BYTES, a += Q8_K_BYTES) {
        float yd = rdf32(a);
        const int8_t* q8 = (const int8_t*)(a + 4);
        const uint8_t* bs = a + 4 + QK_K;
        float d = yd * orc_half_to_float(rd16(w));
        float dmin = -yd * orc_half_to_float(rd16(w + 2));
        int scale[8], min[8];
        q5_scales(w + 4,scale,min);
        int32_t isum = 0;
        for (int s = 0; s < 8; s++) {
            int16_t pair = (int16_t)(int16_t)((int16_t)rd16(bs + 4 * s) + (int16_t)rd16(bs + 4 * s + 2));
            isum += min[s] * pair;
        }
#if ORC_MUTANT == 3
        summs = summs + dmin * (float)isum;
#else
        summs = fmaf(dmin,(float)isum,summs);
#endif
        int32_t sumi[8] = {0};
        for (int j = 0; j < 4; j++) {
            for (int half = 0; half < 2; half++) {
                int s = 2 * j + half;
                for (int t = 0; t < 8; t++) {
                    int32_t pairs[2];
                    for (int p = 0; p < 2; p++) {
                        int i0 = 4 * t + 2 * p;
                        pairs[p] = sat16(q5_value(w,s,i0) * q8[64 * j + 32 * half + i0] +
                                         q5_value(w,s,i0 + 1) * q8[64 * j + 32 * half + i0 + 1]);
                    }
                    sumi[t] += scale[s] * pairs[0] + scale[s] * pairs[1];
                }
            }
        }
        for (int t = 0; t < 8; t++) acc[t] = fmaf(d,(float)sumi[t],acc[t]);
    }
    return hsum8(acc) + summs;
}

static int q6_value(const uint8_t* blk, int e)
{
    int h = e / 128, g = (e % 128) / 32, i = e % 32;
    int low = blk[64 * h + i + (g % 2) * 32];
    low = g < 2? (low & 15) : (low >> 4);
    return low | (((blk[128 + 32 * h + i] >> (2 * g)) & 3) << 4);
}

/* pix_dot_q6_K, src/kernels_quant.cpp:256-337 */
float orc_dot_q6_K(int n, const void* wv, const void* av)
{
    const uint8_t* w = (const uint8_t*)wv;
    const uint8_t* a = (const uint8_t*)av;
    float acc[8] = {0};
    for (int b = 0; b < n / QK_K; b++, w += Q6_K_BYTES, a += Q8_K_BYTES) {
        float d = rdf32(a) * orc_half_to_float(rd16(w + 208));
        const int8_t* q8 = (const int8_t*)(a + 4);
        const uint8_t* bs = a + 4 + QK_K;
        const int8_t* sc = (const int8_t*)(w + 192);
        int32_t sumi[8] = {0};
        for (int c = 0; c < 8; c++) {
            for (int t = 0; t < 8; t++) {
                int scale = sc[2 * c + (t >= 4)];
                int32_t pairs[2];
                for (int p = 0; p < 2; p++) {
                    int e = 32 * c + 4 * t + 2 * p;
                    pairs[p] = sat16(q6_value(w,e) * q8[e] + q6_value(w,e + 1) * q8[e + 1]);
                }
                sumi[t] += scale * pairs[0] + scale * pairs[1];
            }
        }
        for (int t = 0; t < 8; t++) {
            int32_t m = (int16_t)rd16(bs + 4 * t) * sc[2 * t] + (int16_t)rd16(bs + 4 * t + 2) * sc[2 * t + 1];
            sumi[t] -= (int32_t)((uint32_t)m << 5);
            acc[t] = fmaf(d,(float)sumi[t],acc[t]);
        }
    }
    return hsum8(acc);
}

/* Integer gates: exact block sums a correct kernel must reproduce.
 * Q8_0: sum of 32 products per block (pix_dot_q8_0's per-block P, :357). */
int32_t orc_block_sums_q8_0(const void* wv, const void* av)
{
    const int8_t* w = (const int8_t*)wv + 2;
    const int8_t* a = (const int8_t*)av + 2;
    int32_t s = 0;
    for (int i = 0; i < QK8_0; i++) s += w[i] * a[i];
    return s;
}

/* Q5_K: per super-block sum_s scale_s*dot_s (the sum over lanes of pix_dot_q5_K's
 * sumi, :214-245) and sum_s min_s*(bsum_2s+bsum_2s+1) (:198-202). */
void orc_superblock_sums_q5_K(const void* wv, const void* av, int32_t* scaled, int32_t* mins)
{
    const uint8_t* w = (const uint8_t*)wv;
    const uint8_t* a = (const uint8_t*)av;
    const int8_t* q8 = (const int8_t*)(a + 4);
    const uint8_t* bs = a + 4 + QK_K;
    int scale[8], min[8];
    q5_scales(w + 4,scale,min);
    int32_t total = 0, m = 0;
    for (int s = 0; s < 8; s++) {
        int32_t dot = 0;
        for (int i = 0; i < 32; i++) dot += q5_value(w,s,i) * q8[32 * s + i];
        total += scale[s] * dot;
        m += min[s] * ((int16_t)rd16(bs + 4 * s) + (int16_t)rd16(bs + 4 * s + 2));
    }
    *scaled = total;
    *mins = m;
}

/* Q6_K: per super-block sum of scale*(q-32)*q8 (pix_dot_q6_K's lane sum, :283-331). */
int32_t orc_superblock_sum_q6_K(const void* wv, const void* av)
{
    const uint8_t* w = (const uint8_t*)wv;
    const int8_t* q8 = (const int8_t*)((const uint8_t*)av + 4);
    const int8_t* sc = (const int8_t*)(w + 192);
    int32_t total = 0;
    for (int e = 0; e < QK_K; e++) total += sc[e / 16] * (q6_value(w,e) - 32) * q8[e];
    return total;
}

/* weight_bytes for one row, src/model.cpp:87-121 */
uint64_t orc_row_bytes(uint64_t inner, uint32_t type)
{
    uint64_t block = type == ORC_Q8_0? QK8_0 : QK_K;
    uint64_t bytes = type == ORC_Q8_0? Q8_0_BYTES : (type == ORC_Q5_K? Q5_K_BYTES : (type == ORC_Q6_K? Q6_K_BYTES : 0));
    if (!bytes || !inner || inner % block) return 0;
    return inner / block * bytes;
}

struct mm_job {
    const uint8_t* w;
    uint32_t type;
    const uint8_t* xq;
    float* y;
    size_t rows, columns, inner, wstride, xstride, begin, end;
};

static void* mm_worker(void* arg)
{
    struct mm_job* j = (struct mm_job*)arg;
    for (size_t r = j->begin; r < j->end; r++) {
        for (size_t c = 0; c < j->columns; c++) {
            const uint8_t* wr = j->w + r * j->wstride;
            const uint8_t* xr = j->xq + c * j->xstride;
            float v;
            if (j->type == ORC_Q8_0) v = orc_dot_q8_0((int)j->inner,wr,xr);
            else if (j->type == ORC_Q5_K) v = orc_dot_q5_K((int)j->inner,wr,xr);
            else v = orc_dot_q6_K((int)j->inner,wr,xr);
            j->y[c * j->rows + r] = v;
        }
    }
    return NULL;
}

/* cpu_quant_matmul, src/kernels_quant.cpp:369-412: quantize every column
 * (token) of x, then y[c*rows + r] = dot(W_r, Xq_c).  Rows are split into
 * contiguous ranges as cpu_parallel does (src/tensor.cpp:67, :103-115); each
 * output is one sequential dot, so results do not depend on `threads`. */
int orc_quant_matmul(const void* wv, uint32_t type, const float* x, float* y,
                     size_t rows, size_t columns, size_t inner, int threads)
{
    if (type != ORC_Q8_0 && type != ORC_Q5_K && type != ORC_Q6_K) return 0;
    size_t block = type == ORC_Q8_0? QK8_0 : QK_K;
    if (!rows || !columns || !inner || inner % block || inner > 0x7fffffffu) return 0;
    size_t xstride = (inner / block) * (type == ORC_Q8_0? Q8_0_BYTES : Q8_K_BYTES);
    uint8_t* xq = (uint8_t*)malloc(xstride * columns);
    if (!xq) return 0;
    for (size_t c = 0; c < columns; c++) {
        if (type == ORC_Q8_0) orc_quantize_q8_0(x + c * inner,xq + c * xstride,(int64_t)inner);
        else orc_quantize_q8_K(x + c * inner,xq + c * xstride,(int64_t)inner);
    }
    if (threads < 1) threads = 1;
    size_t count = rows / 16 < (size_t)threads? rows / 16 : (size_t)threads;
    if (count < 1) count = 1;
    struct mm_job* jobs = (struct mm_job*)calloc(count,sizeof(struct mm_job));
    pthread_t* tids = (pthread_t*)calloc(count,sizeof(pthread_t));
    for (size_t i = 0; i < count; i++) {
        struct mm_job j = {(const uint8_t*)wv,type,xq,y,rows,columns,inner,orc_row_bytes(inner,type),xstride,
                           rows * i / count,rows * (i + 1) / count};
        jobs[i] = j;
    }
    for (size_t i = 1; i < count; i++) pthread_create(&tids[i],NULL,mm_worker,&jobs[i]);
    mm_worker(&jobs[0]);
    for (size_t i = 1; i < count; i++) pthread_join(tids[i],NULL);
    free(tids);
    free(jobs);
    free(xq);
    return 1;
}

/* Exact dequantization in double (the values cpu_decode computes in float,
 * src/backend_cpu.cpp:46-96), used by the tests' independent fp64 check. */
void orc_decode(const void* data, uint32_t type, size_t count, double* out)
{
    const uint8_t* p = (const uint8_t*)data;
    size_t block = type == ORC_Q8_0? QK8_0 : QK_K;
    for (size_t base = 0; base < count; base += block) {
        double* o = out + base;
        if (type == ORC_Q8_0) {
            double d = orc_half_to_float(rd16(p));
            for (int i = 0; i < QK8_0; i++) o[i] = d * (int8_t)p[2 + i];
            p += Q8_0_BYTES;
        } else if (type == ORC_Q5_K) {
            double d = orc_half_to_float(rd16(p)), dmin = orc_half_to_float(rd16(p + 2));
            int scale[8], min[8];
            q5_scales(p + 4,scale,min);
            for (int s = 0; s < 8; s++)
                for (int i = 0; i < 32; i++) o[32 * s + i] = d * scale[s] * q5_value(p,s,i) - dmin * min[s];
            p += Q5_K_BYTES;
        } else {
            double d = orc_half_to_float(rd16(p + 208));
            const int8_t* sc = (const int8_t*)(p + 192);
            for (int e = 0; e < QK_K; e++) o[e] = d * sc[e / 16] * (q6_value(p,e) - 32);
            p += Q6_K_BYTES;
        }
    }
}

/* ---- neighbours of the linear layer (producers of its input) ---- */

/* tensor_norm, src/tensor.cpp:174-197, one row at a time: the mean (centered
 * only) and the sum of squared deviations are accumulated in double in index
 * order; inverse = (float)(1/sqrt(square/channels + epsilon)) in double;
 * out = (float)(x - mean) * inverse * weight[c] in fp32, left to right
 * (weight NULL: the reference's empty weight multiplies by 1). */
void orc_norm_rows(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, int centered, float* out)
{
    for (size_t r = 0; r < rows; r++) {
        const float* from = x + r * channels;
        float* to = out + r * channels;
        double mean = 0, square = 0;
        if (centered) {
            for (size_t c = 0; c < channels; c++) mean += from[c];
            mean /= (double)channels;
        }
        for (size_t c = 0; c < channels; c++) {
            double t = (double)from[c] - mean;
            square += t * t;
        }
#if ORC_MUTANT == 7
        float inverse = (float)(1.0 / (sqrt(square / (double)channels) + (double)epsilon));
#else
        float inverse = (float)(1.0 / sqrt(square / (double)channels + (double)epsilon));
#endif
        for (size_t c = 0; c < channels; c++) {
#if ORC_MUTANT == 8
            to[c] = (float)((double)from[c] - mean) * (weight? weight[c] : 1.0f) * inverse;
#elif ORC_MUTANT == 9
            float v = (from[c] - (float)mean) * inverse;
            to[c] = v * (weight? weight[c] : 1.0f);
#else
            float v = (float)((double)from[c] - mean) * inverse;
            to[c] = v * (weight? weight[c] : 1.0f);
#endif
        }
    }
}

/* z_modulate, src/inference.cpp:263-277: x[r][c] *= (1.0f + scale[c]) in fp32. */
void orc_modulate_rows(float* x, size_t rows, size_t channels, const float* scale)
{
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < channels; c++) {
            const float v = x[r * channels + c];
#if ORC_MUTANT == 13
            x[r * channels + c] = v + v * scale[c];
#elif ORC_MUTANT == 14
            x[r * channels + c] = v * scale[c];
#else
            x[r * channels + c] = v * (1.0f + scale[c]);
#endif
        }
}

/* tensor_silu, src/tensor.cpp:199-209 (value /= 1.0f + expf(-value)), then
 * tensor_gate, :334-345 (value *= up), elementwise in fp32; `out` may be `gate`. */
void orc_silu_gate(const float* gate, const float* up, size_t count, float* out)
{
    for (size_t i = 0; i < count; i++) {
        float v = gate[i];
#if ORC_MUTANT == 10
        v = v * (1.0f / (1.0f + expf(-v)));
#else
        v = v / (1.0f + expf(-v));
#endif
        out[i] = v * up[i];
    }
}

/* tensor_gelu, src/tensor.cpp:211-224, in place: approximate (tanh) form
 * 0.5f*v*(1 + tanhf(0.7978845608f*(v + 0.044715f*v*v*v))), exact form
 * 0.5f*v*(1 + erff(v/1.4142135623730951f)), fp32 left to right. */
void orc_gelu(float* x, size_t count, int approximate)
{
    for (size_t i = 0; i < count; i++) {
        float v = x[i];
#if ORC_MUTANT == 12
        float argument = approximate? tanhf(0.7978845608028654f * (v + 0.044715f * v * v)) : erff(v / 1.4142135623730951f);
#else
        float argument = approximate? tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)) : erff(v / 1.4142135623730951f);
#endif
        x[i] = 0.5f * v * (1 + argument);
    }
}

/* tensor_bias, src/tensor.cpp:226-240: x[r][c] += bias[c]. */
void orc_bias(float* x, size_t rows, size_t channels, const float* bias)
{
    for (size_t i = 0; i < rows * channels; i++) x[i] += bias[i % channels];
}

/* tensor_add, src/tensor.cpp:321-332: x[i] += y[i]. */
void orc_add(float* x, const float* y, size_t count)
{
    for (size_t i = 0; i < count; i++) x[i] += y[i];
}

/* tensor_rope, src/tensor.cpp:429-452, in place on rows x (heads * dim):
 * for each pair i < dim/2 of each head, (first, second) = (2i, 2i+1) when
 * interleaved, else (i, i + dim/2); a, b = the pair, c, s = cosine and sine
 * [row][i]; first = a*c - b*s, second = a*s + b*c (fp32, no contraction). */
void orc_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, int interleaved)
{
    size_t dim = channels / heads;
    for (size_t row = 0; row < rows; row++)
        for (size_t head = 0; head < heads; head++) {
            float* data = x + row * channels + head * dim;
            for (size_t i = 0; i < dim / 2; i++) {
                size_t first = interleaved? i * 2 : i, second = interleaved? i * 2 + 1 : i + dim / 2;
                float a = data[first], b = data[second];
                float c = cosine[row * dim / 2 + i], s = sine[row * dim / 2 + i];
#if ORC_MUTANT == 11
                s = -s;
#endif
                data[first] = a * c - b * s;
                data[second] = a * s + b * c;
            }
        }
}

/* dot_avx, src/tensor.cpp:117-132 (cpu_dot's path on an AVX2+FMA host, :135-143):
 * two 8-lane fused multiply-add accumulators over 16-value steps, added lane
 * by lane, the 8 partials summed in order, then the tail as a product and a
 * sum (no contraction). */
static float dot_avx_lanes(const float* a, const float* b, size_t count)
{
    float s0[8] = {0}, s1[8] = {0};
    size_t i = 0;
    for (; i + 16 <= count; i += 16)
        for (int l = 0; l < 8; l++) {
            s0[l] = fmaf(a[i + l],b[i + l],s0[l]);
            s1[l] = fmaf(a[i + 8 + l],b[i + 8 + l],s1[l]);
        }
    float result = 0;
    for (int l = 0; l < 8; l++) result += s0[l] + s1[l];
    for (; i < count; i++) result += a[i] * b[i];
    return result;
}

/* tensor_attention with ranges, src/tensor.cpp:384-427 (the causal form,
 * :347-382, is the one range {0, rows, keys, causal} at query_offset 0 where
 * token + 1 <= keys).  q [rows][channels], k and v [keys][channels / heads *
 * kv_heads], out [rows][channels]; ranges [n][4] = query_begin, query_end,
 * key_end, causal (PixAttentionRange, src/tensor.h:58-63), contiguous from row
 * 0.  Per (token, head): scores = dot(q, k_j) * (1/sqrt(dim)) in fp32, the
 * maximum, exp(score - max) in fp32 summed in double, then out += float(p /
 * sum) * v_j in fp32, key by key.  Returns 0 on the arguments the reference
 * rejects (:386-394), 1 otherwise. */
int orc_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                  size_t channels, const uint64_t* ranges, size_t nranges, size_t query_offset, float* out)
{
    if (!heads || !kv_heads || heads % kv_heads || channels % heads || !rows || !keys) return 0;
    const size_t dim = channels / heads, kv_channels = dim * kv_heads;
    size_t covered = 0;
    for (size_t r = 0; r < nranges; r++) {
        const uint64_t* g = ranges + 4 * r;
        if (g[0] != covered || g[1] <= g[0] || g[1] > rows || !g[2] || g[2] > keys) return 0;
        covered = (size_t)g[1];
    }
    if (covered != rows) return 0;
    const float scale = 1.0f / sqrtf((float)dim);
    float* scores = (float*)malloc(keys * sizeof(float));
    if (!scores) return 0;
    memset(out,0,rows * channels * sizeof(float));
    size_t range = 0;
    for (size_t token = 0; token < rows; token++) {
        while (token >= ranges[4 * range + 1]) range++;
        const uint64_t* g = ranges + 4 * range;
        size_t tokens = (size_t)g[2];
#if ORC_MUTANT == 16
        if (g[3] && query_offset + token < tokens) tokens = query_offset + token;
#else
        if (g[3] && query_offset + token + 1 < tokens) tokens = query_offset + token + 1;
#endif
        for (size_t head = 0; head < heads; head++) {
#if ORC_MUTANT == 15
            const size_t kv_head = head % kv_heads;
#else
            const size_t kv_head = head / (heads / kv_heads);
#endif
            const float* query = q + token * channels + head * dim;
            float maximum = -INFINITY;
            for (size_t j = 0; j < tokens; j++) {
                scores[j] = dot_avx_lanes(query,k + j * kv_channels + kv_head * dim,dim) * scale;
                maximum = fmaxf(maximum,scores[j]);
            }
            double sum = 0;
            for (size_t j = 0; j < tokens; j++) {
                scores[j] = expf(scores[j] - maximum);
                sum += scores[j];
            }
            float* to = out + token * channels + head * dim;
            for (size_t j = 0; j < tokens; j++) {
                const float probability = (float)(scores[j] / sum);
                const float* value = v + j * kv_channels + kv_head * dim;
                for (size_t c = 0; c < dim; c++) to[c] += probability * value[c];
            }
        }
    }
    free(scores);
    return 1;
}

/* ---- the rest of the backend op surface ---- */

/* Channel ops in place on x [rows][channels] (op ids of src/vulkan_ops.h:31-49):
 *   8  z_modulate, src/inference.cpp:263-277: x * (1.0f + p[c])
 *   9  z_residual, :279-291: x + other[i] * (p? tanhf(p[c]) : 1.0f)
 *  10  the VAE input step as vulkan_pointwise runs it (:474-476): x * scale + bias
 *  26  qwen_image_euler, src/qwen_image.cpp:347-361: x + delta * other[i]
 * `p` is the modulation already offset to its part (part * channels). */
void orc_channel_op(int op, float* x, const float* other, const float* p, size_t rows, size_t channels, float scale, float bias)
{
    for (size_t i = 0; i < rows * channels; i++) {
        const size_t c = i % channels;
        if (op == 8) {
            x[i] = x[i] * (1.0f + p[c]);
        } else if (op == 9) {
#if ORC_MUTANT == 29
            x[i] += other[i] * (p? p[c] : 1.0f);
#else
            x[i] += other[i] * (p? tanhf(p[c]) : 1.0f);
#endif
        } else if (op == 10) {
#if ORC_MUTANT == 30
            x[i] = (x[i] + bias) * scale;
#else
            x[i] = x[i] * scale + bias;
#endif
        } else {
            x[i] += scale * other[i];
        }
    }
}

/* qwen_image_modulate, src/qwen_image.cpp:149-169: parameters [2][parameter_channels];
 * row r uses parameter row (r >= target_begin? 0 : 1) from part * channels;
 * x *= 1 + p, or with a residual x += residual * tanhf(p).  Returns 0 on the
 * reference's rejection (:152). */
int orc_qwen_modulate(float* x, size_t rows, size_t channels, const float* parameters, size_t parameter_channels, size_t target_begin,
                      size_t part, const float* residual)
{
    if (!rows || !channels || (part + 1) * channels > parameter_channels) return 0;
    for (size_t row = 0; row < rows; row++) {
#if ORC_MUTANT == 28
        const size_t parameter = (row >= target_begin? 1 : 0) * parameter_channels + part * channels;
#else
        const size_t parameter = (row >= target_begin? 0 : 1) * parameter_channels + part * channels;
#endif
        for (size_t c = 0; c < channels; c++) {
            const size_t index = row * channels + c;
            if (residual) x[index] += residual[index] * tanhf(parameters[parameter + c]);
            else x[index] *= 1 + parameters[parameter + c];
        }
    }
    return 1;
}

/* tensor_l2norm, src/tensor.cpp:242-258: square = running double sum of
 * double(x) * x; inverse = (float)(sqrt(double(channels)) / max(sqrt(square),
 * double(epsilon))); y = x * inverse * w[c] in fp32 (w NULL: * 1).  Returns 0
 * on the reference's rejection (epsilon <= 0). */
int orc_l2norm(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, float* out)
{
    if (!rows || !channels || !(epsilon > 0)) return 0;
    for (size_t row = 0; row < rows; row++) {
        const float* from = x + row * channels;
        double square = 0;
        for (size_t c = 0; c < channels; c++) square += (double)from[c] * from[c];
        const double root = sqrt(square);
#if ORC_MUTANT == 17
        const float inverse = (float)(1.0 / (root < (double)epsilon? (double)epsilon : root));
#elif ORC_MUTANT == 18
        const float inverse = (float)(sqrt((double)channels) / (root + (double)epsilon));
#else
        const float inverse = (float)(sqrt((double)channels) / (root < (double)epsilon? (double)epsilon : root));
#endif
        for (size_t c = 0; c < channels; c++) out[row * channels + c] = from[c] * inverse * (weight? weight[c] : 1.0f);
    }
    return 1;
}

/* tensor_groupnorm, src/tensor.cpp:454-485 (COMPUTE_VAE_GROUPS 32,
 * COMPUTE_NORM_EPSILON 1e-6f, src/tensor.h:32-34): group g = channels
 * [g*gs, (g+1)*gs), gs = channels / 32, over all rows; running double sums in
 * row-then-channel order: mean = sum / n, square = sum of (x - mean)^2,
 * inverse = (float)(1 / sqrt(square / n + 1e-6)); y = (float)(x - mean) *
 * inverse * w[c] + b[c] in fp32. */
void orc_groupnorm(const float* x, size_t rows, size_t channels, const float* weight, const float* bias, float* out)
{
    const size_t gs = channels / 32, count = rows * gs;
    for (size_t g = 0; g < 32; g++) {
        double sum = 0, square = 0;
        for (size_t r = 0; r < rows; r++)
            for (size_t c = g * gs; c < (g + 1) * gs; c++) sum += x[r * channels + c];
        const double mean = sum / count;
        for (size_t r = 0; r < rows; r++)
            for (size_t c = g * gs; c < (g + 1) * gs; c++) {
                const double delta = x[r * channels + c] - mean;
                square += delta * delta;
            }
#if ORC_MUTANT == 19
        const float inverse = (float)(1.0 / sqrt(square / (double)(count - 1) + 1e-6f));
#else
        const float inverse = (float)(1.0 / sqrt(square / count + 1e-6f));
#endif
        for (size_t r = 0; r < rows; r++)
            for (size_t c = g * gs; c < (g + 1) * gs; c++) {
#if ORC_MUTANT == 20
                out[r * channels + c] = (float)(x[r * channels + c] - mean) * inverse * weight[g] + bias[g];
#else
                out[r * channels + c] = (float)(x[r * channels + c] - mean) * inverse * weight[c] + bias[c];
#endif
            }
    }
}

/* half_float, src/backend_cpu.cpp:12-22: exact, NaN without its payload. */
static float half_float_ref(uint16_t h)
{
#if ORC_MUTANT == 22
    if ((h & 0x7c00) == 0x7c00 && (h & 0x3ff)) {
        uint32_t bits = ((uint32_t)(h & 0x8000) << 16) | 0x7f800000u | ((uint32_t)(h & 0x3ff) << 13) | 0x00400000u;
        float f;
        memcpy(&f,&bits,4);
        return f;
    }
#endif
    if ((h & 0x7c00) == 0x7c00 && (h & 0x3ff)) return (h & 0x8000)? -NAN : NAN;
    return orc_half_to_float(h);
}

/* cpu_decode, src/backend_cpu.cpp:24-101: `count` values of `type` (F32 0,
 * F16 1, BF16 30, Q8_0, Q5_K, Q6_K) to fp32 in its order of operations:
 * Q8_0 (float)q * d; Q5_K d * scale * q - dmin * min; Q6_K d * scale * (q - 32). */
void orc_decode_f32(const void* data, uint32_t type, size_t count, float* out)
{
    const uint8_t* p = (const uint8_t*)data;
    if (type == 0) {
        memcpy(out,p,count * 4);
        return;
    }
    if (type == 1 || type == 30) {
        for (size_t i = 0; i < count; i++) {
            const uint16_t raw = rd16(p + 2 * i);
#if ORC_MUTANT == 21
            if (1) {
#else
            if (type == 1) {
#endif
                out[i] = half_float_ref(raw);
            } else {
                const uint32_t bits = (uint32_t)raw << 16;
                memcpy(out + i,&bits,4);
            }
        }
        return;
    }
    const size_t block = type == ORC_Q8_0? QK8_0 : QK_K;
    for (size_t base = 0; base < count; base += block) {
        float* o = out + base;
        if (type == ORC_Q8_0) {
            const float d = half_float_ref(rd16(p));
            for (int i = 0; i < QK8_0; i++) o[i] = (int8_t)p[2 + i] * d;
            p += Q8_0_BYTES;
        } else if (type == ORC_Q5_K) {
            const float d = half_float_ref(rd16(p)), dmin = half_float_ref(rd16(p + 2));
            int scale[8], min[8];
            q5_scales(p + 4,scale,min);
            for (int s = 0; s < 8; s++)
                for (int i = 0; i < 32; i++) o[32 * s + i] = d * (float)scale[s] * (float)q5_value(p,s,i) - dmin * (float)min[s];
            p += Q5_K_BYTES;
        } else {
            const float d = half_float_ref(rd16(p + 208));
            const int8_t* sc = (const int8_t*)(p + 192);
            for (int e = 0; e < QK_K; e++) {
                o[e] = d * (float)sc[e / 16] * (float)(q6_value(p,e) - 32);
            }
            p += Q6_K_BYTES;
        }
    }
}

/* tensor_gather (scatter 0) and tensor_scatter, src/tensor.cpp:274-302: row
 * copies in list order (a scattered row listed twice keeps the last).  The
 * reference's checks: every index within its tensor; returns 0 otherwise. */
int orc_rows(const float* source, size_t source_rows, float* destination, size_t destination_rows, size_t channels,
             const uint64_t* rows, size_t count, int scatter)
{
    for (size_t i = 0; i < count; i++)
        if (rows[i] >= (scatter? destination_rows : source_rows)) return 0;
    if (scatter) {
#if ORC_MUTANT == 23
        for (size_t i = count; i-- > 0;) memcpy(destination + rows[i] * channels,source + i * channels,channels * 4);
#else
        for (size_t i = 0; i < count; i++) memcpy(destination + rows[i] * channels,source + i * channels,channels * 4);
#endif
    } else {
        for (size_t i = 0; i < count; i++) memcpy(destination + i * channels,source + rows[i] * channels,channels * 4);
    }
    return 1;
}

/* The DiT patch / unpatch loops (src/inference.cpp:374-390, :438-455) and
 * tensor_upsample (src/tensor.cpp:304-319).  op 15: pixels [width*height][C]
 * -> tokens [(width/p)(height/p)][p*p*C]; 16: the inverse (width, height the
 * pixel image's); 17: [width*height][C] -> [2width*2height][C]. */
void orc_layout(int op, const float* source, float* destination, size_t width, size_t height, size_t channels, size_t patch)
{
    if (op == 17) {
        for (size_t y = 0; y < height * 2; y++)
            for (size_t x = 0; x < width * 2; x++) {
#if ORC_MUTANT == 25
                const size_t from = ((y / 2) * width * 2 + x / 2) % (width * height);
#else
                const size_t from = (y / 2) * width + x / 2;
#endif
                memcpy(destination + (y * width * 2 + x) * channels,source + from * channels,channels * 4);
            }
        return;
    }
    const size_t pw = width / patch, ph = height / patch;
    for (size_t y = 0; y < ph; y++)
        for (size_t x = 0; x < pw; x++)
            for (size_t dy = 0; dy < patch; dy++)
                for (size_t dx = 0; dx < patch; dx++) {
                    const size_t pixel = (y * patch + dy) * width + x * patch + dx;
#if ORC_MUTANT == 24
                    const size_t token = (y * pw + x) * patch * patch + dx * patch + dy;
#else
                    const size_t token = (y * pw + x) * patch * patch + dy * patch + dx;
#endif
                    if (op == 15) memcpy(destination + token * channels,source + pixel * channels,channels * 4);
                    else memcpy(destination + pixel * channels,source + token * channels,channels * 4);
                }
}

/* tensor_resample_shortcut, src/tensor.cpp:487-527, with its checks (returns
 * 0 where the reference returns an empty tensor).  `out` [out_width *
 * out_height][channels]. */
int orc_shortcut(const float* input, size_t width, size_t height, size_t input_channels, size_t channels, size_t temporal, int up,
                 int spatial, float* out)
{
    if (!width || !height || !channels || !temporal || !input_channels) return 0;
    const size_t side = spatial? 2 : 1, factor = temporal * side * side;
    if ((up && channels * factor % input_channels) || (!up && input_channels * factor % channels)) return 0;
    if (!up && (width % side || height % side)) return 0;
    const size_t ow = up? width * side : width / side, oh = up? height * side : height / side;
    const size_t group = up? channels * factor / input_channels : input_channels * factor / channels;
    for (size_t y = 0; y < oh; y++)
        for (size_t x = 0; x < ow; x++)
            for (size_t c = 0; c < channels; c++) {
                float value = 0;
                if (up) {
#if ORC_MUTANT == 27
                    const size_t sc = (c * factor + (y % side) * side + x % side) / group;
#else
                    const size_t sc = (c * factor + (temporal - 1) * side * side + (y % side) * side + x % side) / group;
#endif
                    value = input[((y / side) * width + x / side) * input_channels + sc];
                } else {
                    for (size_t i = 0; i < group; i++) {
                        const size_t item = c * group + i, sc = item / factor;
                        const size_t time = item / (side * side) % temporal, dy = item / side % side, dx = item % side;
                        if (time == temporal - 1) value += input[((y * side + dy) * width + x * side + dx) * input_channels + sc];
                    }
#if ORC_MUTANT != 26
                    value /= group;
#endif
                }
                out[(y * ow + x) * channels + c] = value;
            }
    return 1;
}

/* tensor_conv's geometry form, src/convolution.cpp:56-100 (the first form,
 * :34-54, is the geometry {1, 1, k/2, k-1-k/2, k/2, k-1-k/2}): each output
 * pixel (ox, oy) reads input (ox*sx - left + kx, oy*sy - top + ky), zero
 * outside the image, patch index (c * kernel_y + ky) * kernel_x + kx, times
 * weight [cout][patch], plus bias[o] (NULL: none).  The sums are taken in
 * double (the reference's fp32 FMA tiles round differently; comparisons are
 * held to a tolerance).  `out` [out_w * out_h][cout]; returns 0 on the
 * reference's rejections. */
int orc_conv2d(const float* x, size_t width, size_t height, size_t cin, const float* weight, size_t kx_n, size_t ky_n, size_t cout,
               const float* bias, size_t sx, size_t sy, size_t left, size_t right, size_t top, size_t bottom, float* out)
{
    if (!width || !height || !sx || !sy || width + left + right < kx_n || height + top + bottom < ky_n) return 0;
    const size_t ow = (width + left + right - kx_n) / sx + 1, oh = (height + top + bottom - ky_n) / sy + 1;
    const size_t inner = cin * kx_n * ky_n;
    double* patch = (double*)malloc(inner * sizeof(double));
    if (!patch) return 0;
    for (size_t oy = 0; oy < oh; oy++)
        for (size_t ox = 0; ox < ow; ox++) {
#if ORC_MUTANT == 32
            const int64_t x0 = (int64_t)(ox * sx) - (int64_t)right, y0 = (int64_t)(oy * sy) - (int64_t)bottom;
#else
            const int64_t x0 = (int64_t)(ox * sx) - (int64_t)left, y0 = (int64_t)(oy * sy) - (int64_t)top;
#endif
            for (size_t c = 0; c < cin; c++)
                for (size_t ky = 0; ky < ky_n; ky++)
                    for (size_t kx = 0; kx < kx_n; kx++) {
                        const int64_t ix = x0 + (int64_t)kx, iy = y0 + (int64_t)ky;
#if ORC_MUTANT == 31
                        const size_t to = (c * kx_n + kx) * ky_n + ky;
#else
                        const size_t to = (c * ky_n + ky) * kx_n + kx;
#endif
                        patch[to] = (ix < 0 || iy < 0 || ix >= (int64_t)width || iy >= (int64_t)height)? 0.0
                                    : (double)x[((size_t)iy * width + (size_t)ix) * cin + c];
                    }
            for (size_t o = 0; o < cout; o++) {
                double acc = 0.0;
                for (size_t k = 0; k < inner; k++) acc += patch[k] * (double)weight[o * inner + k];
                out[(oy * ow + ox) * cout + o] = (float)acc + (bias? bias[o] : 0.0f);
            }
        }
    free(patch);
    return 1;
}
