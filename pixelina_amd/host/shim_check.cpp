// Drives the C++ shim (backend_hip.h) the way the reference's model code
// drives its Vulkan backend, for the GPU tests: a session made current on the
// thread (VulkanSession::initialize, src/backend_vulkan.cpp:1004-1011),
// activations in HipAllocator vectors (PixTensorVals, src/tensor.h:19-24),
// weights reached through a model-file / weight pair shaped like PixModelFile
// and PixWeight (src/model.h:33-56), and the calls tensor_linear and the DiT
// block's FFN make (src/tensor.cpp:156-172, src/inference.cpp:328-336).
//
//   shim_check <in> <out>
//
// <in> (little-endian): uint32 type, down_type; uint64 M, K, N, F (FFN width);
// then W1 [N][K] (type), W2 [N][K] (type), Wdown [K][F] (down_type) as GGUF
// block bytes, each preceded by its uint64 byte count; X [M][K], norm weight
// [K], modulation [K], G [M][F], U [M][F], cos, sin [M][32] and bias [N] as
// float32 (the vectors in pageable std::vector memory, as tensor_norm,
// tensor_rope and tensor_bias hold them).
// <out>: float32 Y = X W1^T [M][N] (hip_matmul); Y1, Y2 = norm(X) W1^T,
// norm(X) W2^T (hip_norm_multiply, with the weight and the modulation); the
// normalized X [M][K]; D = (silu(G) * U) Wdown^T [M][K] (hip_silu_gate_multiply);
// the gated product [M][F]; RoPE of X with K/64 heads of 64 (hip_rope, split
// halves) [M][K]; Y + bias (hip_pointwise BIAS) [M][N]; self-attention of X
// with K/64 heads of 64 (hip_attention), causal [M][K], then in the ranges form
// with rows [0, M/2) seeing every key and [M/2, M) causal [M][K]; tensor_l2norm
// of X with the norm weight (hip_l2norm, epsilon 1e-12) [M][K];
// tensor_groupnorm of X with the norm weight and the modulation as bias
// (hip_groupnorm) [M][K]; the rows of X in reverse order gathered from the
// std::vector<size_t> (hip_rows) [M][K].
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "backend_hip.h"

namespace {

struct ModelFile {  // the members of PixModelFile that hip_matmul reads
    std::string filename;
    const unsigned char* data = nullptr;
};

struct Weight {  // the members of PixWeight that hip_matmul reads
    std::string name;
    std::vector<uint64_t> shape;  // {inner, rows}
    uint32_t type = 0;
    uint64_t offset = 0, bytes = 0;
};

template <class T> using Vals = std::vector<T,HipAllocator<T>>;

bool read_all(FILE* f, void* p, size_t n) { return std::fread(p,1,n,f) == n; }

template <class V> bool read_floats(FILE* f, V& v, size_t n)
{
    v.resize(n);
    return read_all(f,v.data(),n * sizeof(float));
}

template <class V> bool write_floats(FILE* f, const V& v)
{
    return std::fwrite(v.data(),sizeof(float),v.size(),f) == v.size();
}

int fail(const char* what)
{
    std::fprintf(stderr,"shim_check: %s (%s)\n",what,pixhip_last_error());
    return 1;
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc != 3) {
        std::fprintf(stderr,"usage: shim_check <in> <out>\n");
        return 2;
    }
    FILE* in = std::fopen(argv[1],"rb");
    if (!in) return fail("cannot open input");
    uint32_t types[2];
    uint64_t dims[4];
    if (!read_all(in,types,sizeof(types)) || !read_all(in,dims,sizeof(dims))) return fail("short header");
    const uint64_t M = dims[0], K = dims[1], N = dims[2], F = dims[3];

    // The "model file": the three weights back to back in one buffer.
    std::vector<unsigned char> blob;
    uint64_t sizes[3];
    for (int i = 0; i < 3; i++) {
        if (!read_all(in,&sizes[i],8)) return fail("short weight size");
        const size_t at = blob.size();
        blob.resize(at + sizes[i]);
        if (!read_all(in,blob.data() + at,sizes[i])) return fail("short weight bytes");
    }
    ModelFile file{"shim_check.gguf",blob.data()};
    Weight w1{"blk.0.ffn_gate.weight",{K,N},types[0],0,sizes[0]};
    Weight w2{"blk.0.ffn_up.weight",{K,N},types[0],sizes[0],sizes[1]};
    Weight wd{"blk.0.ffn_down.weight",{F,K},types[1],sizes[0] + sizes[1],sizes[2]};

    HipSession session;
    if (!session.initialize()) return fail("HipSession::initialize");
    {
        // HipAllocator vectors allocate through the active session (pinned host memory).
        Vals<float> x, gate, up;
        std::vector<float> norm_weight, modulation, cosine, sine, bias;
        if (!read_floats(in,x,M * K) || !read_floats(in,norm_weight,K) || !read_floats(in,modulation,K) ||
            !read_floats(in,gate,M * F) || !read_floats(in,up,M * F) || !read_floats(in,cosine,M * 32) ||
            !read_floats(in,sine,M * 32) || !read_floats(in,bias,N))
            return fail("short activations");
        std::fclose(in);

        Vals<float> y(M * N), y1(M * N), y2(M * N), normalized(M * K), d(M * K), gated(M * F);
        // tensor_linear -> cpu_matmul -> (backend) matmul
        if (!hip_matmul(file,w1,x.data(),M,y.data())) return fail("hip_matmul");
        // the FFN input: norm + modulation, quantized once for both linears
        pixhip_weight* ws[2] = {hip_weight_of(file,w1),hip_weight_of(file,w2)};
        float* outs[2] = {y1.data(),y2.data()};
        if (!ws[0] || !ws[1]) return fail("hip_weight_of");
        if (!hip_norm_multiply(w1.type,ws,outs,2,x.data(),M,K,norm_weight.data(),1e-5f,false,modulation.data(),normalized.data()))
            return fail("hip_norm_multiply");
        // the FFN down input: silu(gate) * up, then the down linear
        pixhip_weight* down = hip_weight_of(file,wd);
        if (!down || !hip_silu_gate_multiply(wd.type,down,gate.data(),up.data(),M,F,d.data(),gated.data()))
            return fail("hip_silu_gate_multiply");
        // tensor_rope / tensor_bias hand their std::vector tables straight in
        Vals<float> roped(x.begin(),x.end()), biased(M * N);
        if (!hip_synchronize()) return fail("hip_synchronize");
        for (size_t i = 0; i < biased.size(); i++) biased[i] = y[i];
        if (!hip_rope(roped.data(),M,K,K / 64,cosine.data(),sine.data(),false)) return fail("hip_rope");
        if (!hip_pointwise(PIXHIP_OP_BIAS,biased.data(),bias.data(),M,N)) return fail("hip_pointwise(BIAS)");
        // tensor_attention, both forms
        Vals<float> att(M * K), att2(M * K);
        if (!hip_attention(x.data(),M,x.data(),x.data(),M,K / 64,K / 64,K,true,att.data())) return fail("hip_attention");
        const pixhip_attention_range ranges[2] = {{0,M / 2,M,0},{M / 2,M,M,1}};
        if (!hip_attention(x.data(),M,x.data(),x.data(),M,K / 64,K / 64,K,ranges,2,0,att2.data())) return fail("hip_attention(ranges)");
        // tensor_l2norm / tensor_groupnorm / tensor_gather with the reference's vectors
        Vals<float> l2(M * K), gn(M * K), gathered(M * K);
        if (!hip_l2norm(x.data(),M,K,norm_weight.data(),1e-12f,l2.data())) return fail("hip_l2norm");
        if (!hip_groupnorm(x.data(),M,K,norm_weight.data(),modulation.data(),gn.data())) return fail("hip_groupnorm");
        std::vector<size_t> reversed(M);
        for (size_t i = 0; i < M; i++) reversed[i] = M - 1 - i;
        if (!hip_rows(x.data(),M,gathered.data(),M,K,reversed.data(),M,false)) return fail("hip_rows");
        if (!hip_synchronize()) return fail("hip_synchronize");

        FILE* out = std::fopen(argv[2],"wb");
        if (!out) return fail("cannot open output");
        const bool ok = write_floats(out,y) && write_floats(out,y1) && write_floats(out,y2) && write_floats(out,normalized) &&
                        write_floats(out,d) && write_floats(out,gated) && write_floats(out,roped) && write_floats(out,biased) &&
                        write_floats(out,att) && write_floats(out,att2) && write_floats(out,l2) && write_floats(out,gn) &&
                        write_floats(out,gathered);
        std::fclose(out);
        if (!ok) return fail("short write");
    }
    std::printf("shim_check ok\n");
    return 0;
}
