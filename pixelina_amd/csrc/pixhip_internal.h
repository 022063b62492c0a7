// Internal declarations shared by the HIP kernel files and the C-ABI layer.
//
// Resident (HBM) data layouts used by the kernels.  The boundary accepts the
// reference's GGUF block bytes (src/kernels_quant.cpp:14-38); the weight cache
// converts them once, at upload, into the layouts below, which is legal because
// the cache is internal to the backend (src/backend_vulkan.cpp:742-758).
//
//   activations, Q8_K ("act8k"), M rows of K values:
//     qs   int8   tiled [Mpad/16][K/64][16][64]: value (m, k) at tiled_offset(m, k, K),
//                 so the 16 rows x 64 values of one GEMM stage are one contiguous 1 KB
//     d    fp32   [K/256][Mpad]   block scale, super-block-major
//     bs   fp16   tiled [Mpad/32][K/256][32][16]: the sums of 16 quantized values
//                 (exact, |s| <= 2032) of 32 rows and one super-block are one 1 KB
//                 block; within a row the order is 0,2,..,14,1,3,..,15 (even groups,
//                 then odd: the min-term MFMA operand order)
//   activations, Q8_0 ("act80"), rows of Kp = K rounded up to 64 (a zero pad block):
//     qs   int8   [M][Kp]
//     d    fp32   [Kp/32][Mpad]   fp16-rounded block scale widened to fp32
//   Activations are allocated with Mpad rows (multiple of PIX_GEMM_MTILE) and
//   GEMM weight forms with Npad rows (multiple of PIX_GEMM_NTILE).
//   weights Q5_K for the GEMM ("planes"), N rows padded to Npad:
//     hi   int8   tiled [Npad/16][K/64][16][64]   (scale_s * q) >> 6
//     lo   int8   tiled, as hi                    (scale_s * q) & 63
//     d    fp32   [K/256][Npad]     super-block scale d
//     dm   fp32   [K/256][Npad]     super-block dmin
//     mn   fp16   [K/256][Npad][8]  the eight six-bit sub-block minima
//   weights Q6_K for the GEMM: hi/lo of scale*(q-32) = 64*hi + lo (tiled as Q5_K), d fp32 [K/256][Npad]
//   weights Q8_0 for the GEMM, rows of Kp with a zero pad block: qs int8
//     [Npad][Kp], and the scales widened and transposed, dT fp32 [Kp/32][Npad]
//   weights Q8_0 for the matvec: qs_mv int8 [N][4][Kp/64][16] (each row
//     piece-major: 16-byte piece p of 64-value unit u at (p*Kp/64 + u)*16),
//     d fp16 [N][Kp/32]
//   weights Q5_K for the matvec ("q5 planar"): per row, the GGUF nibble bytes of
//     unit u (64 values, u = 4b + j covers sub-blocks 2j, 2j+1 of super-block b)
//     split into two half planes, qs u8 [N][2][K/64][16] (half 0: the unit's
//     bytes 0..15, half 1: bytes 16..31), and one 12-B record per unit,
//     rec u32 [N][K/64][3] -- 44 bytes per 64 values, as the GGUF blocks:
//       words 0, 1  the unit's 64 high bits: word w holds, for qh words
//                   4w..4w+3, ((qh >> 2j) & 0x03030303) << 2*(qword & 3)
//       word 2      bits 0..23: scale_2j, scale_2j+1, min_2j, min_2j+1 (six
//                   bits each); bits 24..31: byte j of the super-block's
//                   d | dmin << 16 (fp16 bits), which the four units of a
//                   super-block carry between them
//   weights Q6_K for the matvec ("q6 planar"): ql u8 [N][2][K/64][16] (each
//     64-value unit's first and second 16-byte piece of GGUF ql bytes, in two
//     unit-major planes), qh u8 [N][K/4], sc int8 [N][K/16], d fp16 [N][K/256]
//     -- the GGUF bytes re-sliced so every plane is 16-B aligned (210-B blocks
//     are only 2-B aligned) and every matvec load is lane-contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define PIX_F32 0
#define PIX_F16 1
#define PIX_BF16 30
#define PIX_Q8_0 8
#define PIX_Q5_K 13
#define PIX_Q6_K 14
#define PIX_QK 256
#define PIX_QK8 32
#define PIX_Q8_0_BYTES 34
#define PIX_Q8_K_BYTES 292
#define PIX_Q5_K_BYTES 176
#define PIX_Q6_K_BYTES 210
#define PIX_GEMM_MTILE 256  // GEMM workgroup tile: tokens
#define PIX_GEMM_NTILE 128  // GEMM workgroup tile: output features

namespace pixhip {

// Byte offset of value (row, k) in a tiled plane of K values per row: rows in
// groups of 16, each group's K bytes cut into 64-byte pieces, and the piece of
// a group for values 64s..64s+63 is one contiguous 1 KB block (16 rows x 64).
// The GEMM fetches one such block per DMA instruction: whole 128-byte lines,
// where a row-major plane would give it 16 half lines.
__host__ __device__ inline size_t tiled_offset(size_t row, size_t k, size_t K)
{
    return ((row >> 4) * (K >> 6) + (k >> 6)) * 1024 + (row & 15) * 64 + (k & 63);
}
// Element index of the 16-value sum j (0..15, even groups first) of super-block
// b of row `row` in the tiled bs plane.
__host__ __device__ inline size_t tiled_bs_index(size_t row, size_t b, int j, size_t K)
{
    return (((row >> 5) * (K >> 8) + b) * 32 + (row & 31)) * 16 + (size_t)j;
}

struct Act8K {
    int8_t* qs;       // tiled [mpad/16][K/64][16][64]
    float* d;         // [K/256][mpad]
    _Float16* bs;     // tiled [mpad/32][K/256][32][16]
    size_t mpad;      // rows allocated (multiple of the GEMM tile)
};

struct Act80 {
    int8_t* qs;       // [mpad][Kp]
    float* d;         // [Kp/32][mpad]
    size_t mpad;
};

struct PlanesQ5K {
    const int8_t* hi;
    const int8_t* lo;
    const float* d;
    const float* dm;
    const _Float16* mn;
    size_t npad;
};

struct PlanesQ6K {
    const int8_t* hi;
    const int8_t* lo;
    const float* d;
    size_t npad;
};

struct PlanarQ80 {
    const int8_t* qs;     // [Npad][Kp] (GEMM)
    const float* dT;      // [Kp/32][Npad] (GEMM)
    const int8_t* qs_mv;  // [N][4][Kp/64][16]: each row piece-major (matvec)
    const _Float16* d;    // [N][Kp/32] (matvec)
};

struct PlanarQ5K {
    const uint8_t* qs;    // [N][K/2]
    const uint32_t* rec;  // [N][K/64][3]
};

struct PlanarQ6K {
    const uint8_t* ql;
    const uint8_t* qh;
    const int8_t* sc;
    const _Float16* d;
};

struct Output {
    float* y;
    const float* bias;
    size_t ldy;
    size_t offset;
};

// quantize.hip
hipError_t launch_quantize_q8_K(const float* x, size_t rows, size_t inner, Act8K planar, void* blocks, hipStream_t s);
hipError_t launch_quantize_q8_0(const float* x, size_t rows, size_t inner, size_t kpad, Act80 planar, void* blocks,
                                hipStream_t s);
hipError_t launch_copy_device(void* dst, const void* src, size_t bytes, hipStream_t s);

// fuse.hip: producers of a linear layer's input with its quantizer.  kind 0
// (fp32 result only), 1 (Q8_K planar), 2 (Q8_0 planar, row stride kpad).
struct ActOut {
    int8_t* qs;       // planar activations (null: none)
    float* d;
    _Float16* bs;     // Q8_K 16-value sums
    size_t mpad;
    void* blocks;     // reference block layout (null: none)
    float* y;         // fp32 result (null: none)
};
hipError_t launch_norm_quantize(const float* x, size_t rows, size_t K, const float* weight, float eps, bool centered,
                                const float* modulation, int kind, size_t kpad, const ActOut& out, hipStream_t s);
hipError_t launch_silu_gate_quantize(const float* gate, const float* up, size_t rows, size_t K, int kind, size_t kpad,
                                     const ActOut& out, hipStream_t s);

// ops.hip: elementwise ops in place (operation ids of src/vulkan_ops.h:24-49)
constexpr int kOpSilu = 2, kOpGate = 3, kOpAdd = 4, kOpBias = 14, kOpGeluExact = 18, kOpGeluTanh = 19;
hipError_t launch_pointwise(int op, float* x, const float* other, size_t rows, size_t channels, hipStream_t s);
hipError_t launch_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, bool interleaved,
                       hipStream_t s);

// tensor_ops.hip: the rest of the backend op surface (ids of src/vulkan_ops.h:24-49)
constexpr int kOpModulate = 8, kOpResidual = 9, kOpAffine = 10, kOpQwenScale = 24, kOpQwenResidual = 25, kOpEuler = 26;
constexpr int kLayoutPatch = 15, kLayoutUnpatch = 16, kLayoutUpsample = 17;
// x [rows][channels] in place; p0 / p1 per-channel parameters (p1 for rows
// below `split`, QWEN ops only), `other` [rows][channels].
hipError_t launch_channel_op(int op, float* x, const float* other, const float* p0, const float* p1, size_t rows, size_t channels,
                             size_t split, float scale, float bias, hipStream_t s);
hipError_t launch_l2norm(const float* x, const float* w, float* y, size_t rows, size_t channels, float eps, hipStream_t s);
// Workspace of launch_groupnorm; 0 when the shape is not supported (channels
// not a multiple of 32, or groups wider than 1024 channels).
size_t groupnorm_workspace_bytes(size_t rows, size_t channels);
hipError_t launch_groupnorm(const float* x, const float* w, const float* b, float* y, size_t rows, size_t channels, float eps,
                            void* workspace, hipStream_t s);
// Rows ids[r] (ids null: r) of a table of GGUF rows `stride` bytes apart, decoded to fp32 [count][inner].
hipError_t launch_decode_rows(const void* table, uint32_t type, size_t stride, const int64_t* ids, size_t count, size_t inner, float* out,
                              hipStream_t s);
hipError_t launch_rows(const float* src, float* dst, const uint64_t* src_rows, const uint64_t* dst_rows, size_t n, size_t channels,
                       hipStream_t s);
hipError_t launch_copy2d(const float* src, size_t src_stride, float* dst, size_t dst_stride, size_t rows, size_t columns, hipStream_t s);
hipError_t launch_layout(int op, const float* src, float* dst, size_t rows, size_t channels, size_t width, size_t src_channels, size_t patch,
                         hipStream_t s);
hipError_t launch_shortcut(const float* src, float* dst, size_t out_rows, size_t channels, size_t src_channels, size_t width, size_t side,
                           size_t temporal, bool up, hipStream_t s);

// conv.hip: implicit-GEMM convolution on split-bf16 MFMA.  The weight form is
// two bf16 planes [Npad][Kp] (hi, lo) with the inner index in (ky, kx, c)
// order; x [H*W][C], y [OH*OW][N] (+ bias[n] when bias is not null).
struct ConvArgs {
    const float* x;
    const uint16_t *wh, *wl;
    const float* bias;
    float* y;
    int W, H, C, KX, KY, SX, SY, PL, PT, OW, OH, K, Kp, N, Npad;
    long long M;
};
constexpr int kConvTileN = 128, kConvTileK = 32;
hipError_t launch_conv_form(const void* raw, uint32_t type, int kernel_x, int kernel_y, int cin, int cout, int kp, int npad,
                            uint16_t* hi, uint16_t* lo, hipStream_t s);
hipError_t launch_conv(const ConvArgs& a, hipStream_t s);

// repack.hip
hipError_t launch_repack_q5_K(const uint8_t* raw, size_t rows, size_t inner, size_t npad, int8_t* hi, int8_t* lo, float* d,
                              float* dm, _Float16* mn, hipStream_t s);
hipError_t launch_repack_q6_K_planes(const uint8_t* raw, size_t rows, size_t inner, size_t npad, int8_t* hi, int8_t* lo, float* d,
                                     hipStream_t s);
hipError_t launch_repack_q5_K_planar(const uint8_t* raw, size_t rows, size_t inner, uint8_t* qs, uint32_t* rec, hipStream_t s);
hipError_t launch_repack_q6_K_planar(const uint8_t* raw, size_t rows, size_t inner, uint8_t* ql, uint8_t* qh, int8_t* sc,
                                     _Float16* d, hipStream_t s);
// Q8_0 forms: the GEMM's (qs, dT: pass null to skip) and the matvec's
// (qs_mv, d: pass null to skip), from the GGUF blocks.
hipError_t launch_repack_q8_0(const uint8_t* raw, size_t rows, size_t inner, size_t kpad, size_t rows_pad, int8_t* qs, float* dT,
                              int8_t* qs_mv, _Float16* d, hipStream_t s);

// gemm.hip
// Split-K workspace (fp32 partial outputs) a GEMM of M x N over K (rounded up
// to 64: the stage length) uses; 0 when it runs unsplit.  The launchers take
// a workspace of at least that size, or null to run unsplit.
size_t gemm_split_bytes(size_t M, size_t N, size_t K_stages);
// The split of a GEMM grid: number of K pieces of the last round's tiles (1:
// none), the whole tiles before them and the piece length in 64-value stages.
int gemm_split_plan(size_t M, size_t N, size_t K, int& full_tiles, int& split_chunks);
// True when the Q8_0 GEMM of M x N runs its K-grouped small-tile form, which
// needs no split-K workspace.
bool gemm_q8_0_grouped(size_t M, size_t N);
hipError_t launch_gemm_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s);
hipError_t launch_gemm_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s);
hipError_t launch_gemm_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, const Output& out, float* part,
                            hipStream_t s);
hipError_t launch_sums_q5_K(const Act8K& a, const PlanesQ5K& w, size_t M, size_t N, size_t K, int32_t* scaled, int32_t* mins,
                            hipStream_t s);
hipError_t launch_sums_q6_K(const Act8K& a, const PlanesQ6K& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s);
hipError_t launch_sums_q8_0(const Act80& a, const PlanarQ80& w, size_t M, size_t N, size_t K, int32_t* sums, hipStream_t s);

// attention.hip
// One PixAttentionRange (src/tensor.h:58-63).
struct AttnRange {
    size_t query_begin, query_end, key_end;
    bool causal;
};
// Head size rounded up to the kernel's (64 or 128); 0 when not supported.
int attention_dim_pad(size_t dim);
// Workspace of launch_attention (bf16 split planes of Q, K and V^T).
size_t attention_workspace_bytes(size_t rows, size_t keys, size_t heads, size_t kv_heads, size_t dim);
// out [rows][heads*dim] for q [rows][heads*dim], k and v [keys][kv_heads*dim]
// (device pointers), one kernel launch per range (a range's rows only).
hipError_t launch_attention(const float* q, const float* k, const float* v, float* out, size_t rows, size_t keys, size_t heads,
                            size_t kv_heads, size_t dim, const AttnRange* ranges, size_t count, size_t query_offset, void* workspace,
                            hipStream_t s);

// matvec.hip
hipError_t launch_matvec_q5_K(const PlanarQ5K& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s);
hipError_t launch_matvec_q8_0(const PlanarQ80& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s);
hipError_t launch_matvec_q6_K(const PlanarQ6K& w, const float* x, size_t N, size_t K, const Output& out, hipStream_t s);

}  // namespace pixhip
