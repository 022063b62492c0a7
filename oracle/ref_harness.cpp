/* Test infrastructure only: C-ABI harness around the reference's own CPU
 * quantized kernels, compiled in place from the reference sources by
 * oracle/Makefile into oracle/_ref/libpixref.so.
 *
 * The reference keeps its quantizers and dot products `static` inside
 * src/kernels_quant.cpp, so this translation unit includes that file (from the
 * reference tree, never a copy) to reach them.  Nothing here re-implements the
 * reference: every function forwards to the reference symbol named beside it.
 * Used by tests/golden/make_golden.py (to write fixtures), by the tests (as a
 * second checker when the library is present) and by bench.py's CPU-baseline
 * leg (cpu_baseline.kind = "reference").
 */
#include "kernels_quant.cpp"
#include "model.h"
#include "tensor.h"
#include "tensor_names.h"

#include <cstring>

extern "C" {

/* quantize_row_q8_0_ref, src/kernels_quant.cpp:120-144 */
void ref_quantize_q8_0(const float* x, void* blocks, int64_t k)
{
    quantize_row_q8_0_ref(x,static_cast<block_q8_0*>(blocks),k);
}

/* quantize_row_q8_K_ref, src/kernels_quant.cpp:80-118 */
void ref_quantize_q8_K(const float* x, void* blocks, int64_t k)
{
    quantize_row_q8_K_ref(x,static_cast<block_q8_K*>(blocks),k);
}

/* pix_dot_q8_0, src/kernels_quant.cpp:339-365 */
float ref_dot_q8_0(int n, const void* w, const void* a)
{
    return pix_dot_q8_0(n,static_cast<const block_q8_0*>(w),static_cast<const block_q8_0*>(a));
}

/* pix_dot_q5_K, src/kernels_quant.cpp:163-254 */
float ref_dot_q5_K(int n, const void* w, const void* a)
{
    return pix_dot_q5_K(n,static_cast<const block_q5_K*>(w),static_cast<const block_q8_K*>(a));
}

/* pix_dot_q6_K, src/kernels_quant.cpp:256-337 */
float ref_dot_q6_K(int n, const void* w, const void* a)
{
    return pix_dot_q6_K(n,static_cast<const block_q6_K*>(w),static_cast<const block_q8_K*>(a));
}

/* nearest_int, src/kernels_quant.cpp:41-48 */
int ref_nearest_int(float f)
{
    return nearest_int(f);
}

/* cpu_quant_matmul, src/kernels_quant.cpp:369-412 (1 = true) */
int ref_quant_matmul(const unsigned char* w, uint32_t type, const float* x, float* y,
                     size_t rows, size_t columns, size_t inner)
{
    return cpu_quant_matmul(w,type,x,y,rows,columns,inner)? 1 : 0;
}

/* cpu_set_threads / cpu_thread_count, src/tensor.cpp:92-101 */
void ref_set_threads(size_t n)
{
    cpu_set_threads(n);
}

size_t ref_thread_count(void)
{
    return cpu_thread_count();
}

/* cpu_decode, src/backend_cpu.cpp:24-101 */
void ref_decode(const unsigned char* data, uint32_t type, size_t count, float* out)
{
    cpu_decode(data,type,count,out);
}

/* half_float, src/backend_cpu.cpp:12-22 */
float ref_half_float(uint16_t h)
{
    return half_float(h);
}

/* weight_bytes, src/model.cpp:87-121, for a one-row shape {inner} */
uint64_t ref_row_bytes(uint64_t inner, uint32_t type)
{
    return weight_bytes({inner},type);
}

/* tensor_norm, src/tensor.cpp:174-197, on `rows` x `channels` (weight NULL:
 * the empty weight vector).  Returns 1 when the reference produced output. */
int ref_norm_rows(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, int centered, float* out)
{
    PixTensor in(rows,channels);
    std::copy(x,x + rows * channels,in.values.begin());
    std::vector<float> w;
    if (weight) w.assign(weight,weight + channels);
    PixTensor o = tensor_norm(in,w,epsilon,centered != 0);
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_silu, src/tensor.cpp:199-209, then tensor_gate, :334-345 */
void ref_silu_gate(const float* gate, const float* up, size_t count, float* out)
{
    PixTensor g(1,count),u(1,count);
    std::copy(gate,gate + count,g.values.begin());
    std::copy(up,up + count,u.values.begin());
    tensor_silu(g);
    tensor_gate(g,u);
    std::copy(g.values.begin(),g.values.end(),out);
}

/* tensor_gelu, src/tensor.cpp:211-224 */
void ref_gelu(float* x, size_t count, int approximate)
{
    PixTensor t(1,count);
    std::copy(x,x + count,t.values.begin());
    tensor_gelu(t,approximate != 0);
    std::copy(t.values.begin(),t.values.end(),x);
}

/* tensor_bias, src/tensor.cpp:226-240 */
void ref_bias(float* x, size_t rows, size_t channels, const float* bias)
{
    PixTensor t(rows,channels);
    std::copy(x,x + rows * channels,t.values.begin());
    tensor_bias(t,std::vector<float>(bias,bias + channels));
    std::copy(t.values.begin(),t.values.end(),x);
}

/* tensor_add, src/tensor.cpp:321-332 */
void ref_add(float* x, const float* y, size_t count)
{
    PixTensor a(1,count),b(1,count);
    std::copy(x,x + count,a.values.begin());
    std::copy(y,y + count,b.values.begin());
    tensor_add(a,b);
    std::copy(a.values.begin(),a.values.end(),x);
}

/* tensor_attention(q, k, v, heads, kv_heads, causal), src/tensor.cpp:347-382:
 * q [rows][channels], k and v [keys][channels / heads * kv_heads].  Returns 1
 * when the reference produced output. */
int ref_attention(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                  size_t channels, int causal, float* out)
{
    const size_t kv_channels = channels / heads * kv_heads;
    PixTensor tq(rows,channels),tk(keys,kv_channels),tv(keys,kv_channels);
    std::copy(q,q + rows * channels,tq.values.begin());
    std::copy(k,k + keys * kv_channels,tk.values.begin());
    std::copy(v,v + keys * kv_channels,tv.values.begin());
    PixTensor o = tensor_attention(tq,tk,tv,heads,kv_heads,causal != 0);
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_attention(q, k, v, heads, kv_heads, ranges, query_offset),
 * src/tensor.cpp:384-427; ranges [n][4] = query_begin, query_end, key_end,
 * causal (PixAttentionRange, src/tensor.h:58-63).  Returns 1 when the reference
 * produced output (0: it rejected the arguments). */
int ref_attention_ranges(const float* q, size_t rows, const float* k, const float* v, size_t keys, size_t heads, size_t kv_heads,
                         size_t channels, const uint64_t* ranges, size_t nranges, size_t query_offset, float* out)
{
    const size_t kv_channels = channels / heads * kv_heads;
    PixTensor tq(rows,channels),tk(keys,kv_channels),tv(keys,kv_channels);
    std::copy(q,q + rows * channels,tq.values.begin());
    std::copy(k,k + keys * kv_channels,tk.values.begin());
    std::copy(v,v + keys * kv_channels,tv.values.begin());
    std::vector<PixAttentionRange> rs(nranges);
    for (size_t i = 0; i < nranges; i++)
        rs[i] = PixAttentionRange{size_t(ranges[4 * i]),size_t(ranges[4 * i + 1]),size_t(ranges[4 * i + 2]),ranges[4 * i + 3] != 0};
    PixTensor o = tensor_attention(tq,tk,tv,heads,kv_heads,rs,query_offset);
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_rope, src/tensor.cpp:429-452 */
void ref_rope(float* x, size_t rows, size_t channels, size_t heads, const float* cosine, const float* sine, int interleaved)
{
    PixTensor t(rows,channels);
    std::copy(x,x + rows * channels,t.values.begin());
    const size_t half = rows * (channels / heads) / 2;
    tensor_rope(t,heads,std::vector<float>(cosine,cosine + half),std::vector<float>(sine,sine + half),interleaved != 0);
    std::copy(t.values.begin(),t.values.end(),x);
}

/* tensor_l2norm, src/tensor.cpp:242-258 (weight NULL: the empty vector).
 * Returns 1 when the reference produced output. */
int ref_l2norm(const float* x, size_t rows, size_t channels, const float* weight, float epsilon, float* out)
{
    PixTensor in(rows,channels);
    std::copy(x,x + rows * channels,in.values.begin());
    std::vector<float> w;
    if (weight) w.assign(weight,weight + channels);
    PixTensor o = tensor_l2norm(in,w,epsilon);
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_groupnorm, src/tensor.cpp:454-485, which reads `name`.weight and
 * `name`.bias from a model file: here a PixModelFile whose mapping is a
 * buffer holding the two F32 vectors (detached again before it is destroyed,
 * so that close() unmaps nothing). */
int ref_groupnorm(const float* x, size_t rows, size_t channels, const float* weight, const float* bias, float* out)
{
    std::vector<float> blob(weight,weight + channels);
    blob.insert(blob.end(),bias,bias + channels);
    PixModelFile model;
    model.data = reinterpret_cast<const unsigned char*>(blob.data());
    model.size = blob.size() * sizeof(float);
    model.weights["g" WEIGHT_SUFFIX] = PixWeight{"g" WEIGHT_SUFFIX,{uint64_t(channels)},MODEL_F32,0,uint64_t(channels) * 4};
    model.weights["g" BIAS_SUFFIX] = PixWeight{"g" BIAS_SUFFIX,{uint64_t(channels)},MODEL_F32,uint64_t(channels) * 4,uint64_t(channels) * 4};
    PixTensor in(rows,channels);
    std::copy(x,x + rows * channels,in.values.begin());
    PixTensor o = tensor_groupnorm(model,"g",in);
    model.data = nullptr;
    model.size = 0;
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_slice, src/tensor.cpp:260-272: out [rows][channels] */
int ref_slice(const float* x, size_t in_rows, size_t in_channels, size_t row, size_t rows, size_t feature, size_t channels, float* out)
{
    PixTensor in(in_rows,in_channels);
    std::copy(x,x + in_rows * in_channels,in.values.begin());
    PixTensor o = tensor_slice(in,row,rows,feature,channels);
    if (o.values.size() != rows * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_gather, src/tensor.cpp:274-289: out [count][channels] */
int ref_gather(const float* x, size_t in_rows, size_t channels, const uint64_t* rows, size_t count, float* out)
{
    PixTensor in(in_rows,channels);
    std::copy(x,x + in_rows * channels,in.values.begin());
    PixTensor o = tensor_gather(in,std::vector<size_t>(rows,rows + count));
    if (o.values.size() != count * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_scatter, src/tensor.cpp:291-302: destination [dst_rows][channels] in place */
int ref_scatter(float* destination, size_t dst_rows, size_t channels, const float* source, const uint64_t* rows, size_t count)
{
    PixTensor d(dst_rows,channels),src(count,channels);
    std::copy(destination,destination + dst_rows * channels,d.values.begin());
    std::copy(source,source + count * channels,src.values.begin());
    if (!tensor_scatter(d,src,std::vector<size_t>(rows,rows + count))) return 0;
    std::copy(d.values.begin(),d.values.end(),destination);
    return 1;
}

/* tensor_upsample, src/tensor.cpp:304-319: out [4*width*height][channels] */
int ref_upsample(const float* x, size_t width, size_t height, size_t channels, float* out)
{
    PixTensor in(width * height,channels);
    std::copy(x,x + width * height * channels,in.values.begin());
    PixTensor o = tensor_upsample(in,width,height);
    if (o.values.size() != 4 * width * height * channels) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return 1;
}

/* tensor_resample_shortcut, src/tensor.cpp:487-527: out [out_pixels][channels];
 * returns the number of output values (0: the reference rejected the shape). */
size_t ref_shortcut(const float* x, size_t width, size_t height, size_t in_channels, size_t channels, size_t temporal, int up, int spatial,
                    float* out, size_t capacity)
{
    PixTensor in(width * height,in_channels);
    std::copy(x,x + width * height * in_channels,in.values.begin());
    PixTensor o = tensor_resample_shortcut(in,width,height,channels,temporal,up != 0,spatial != 0);
    if (o.values.empty() || o.values.size() > capacity) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return o.values.size();
}

/* PixModelFile::open (src/model.cpp:138-243) on `path`, rendered as text for
 * comparison with another reader: "open <code>\n", then per tensor in name
 * order "T <name> <type> <d0,d1,...> <offset> <bytes>\n", then per metadata key
 * "M <key> <value as JSON>\n" (strings with '"', '\\' and control characters
 * escaped, numbers and booleans in PixJson's text).  Writes at most
 * `capacity` bytes; returns the full length. */
static void ref_json(const PixJson &v, std::string &out)
{
    static const char hex[] = "0123456789abcdef";
    auto quote = [&](const std::string &s) {
        out += '"';
        for (unsigned char c : s) {
            if (c == '"' || c == '\\') {
                out += '\\';
                out += char(c);
            } else if (c < 0x20) {
                out += "\\u00";
                out += hex[c >> 4];
                out += hex[c & 15];
            } else out += char(c);
        }
        out += '"';
    };
    switch (v.type) {
    case PixJson::Null: out += "null"; break;
    case PixJson::Boolean:
    case PixJson::Number: out += v.scalar; break;
    case PixJson::String: quote(v.scalar); break;
    case PixJson::Array:
        out += '[';
        for (size_t i = 0; i < v.array.size(); i++) {
            if (i) out += ',';
            ref_json(v.array[i],out);
        }
        out += ']';
        break;
    case PixJson::Object: {
        out += '{';
        bool first = true;
        for (const auto &m : v.object) {
            if (!first) out += ',';
            first = false;
            quote(m.first);
            out += ':';
            ref_json(m.second,out);
        }
        out += '}';
        break;
    }
    default: out += "?"; break;
    }
}

size_t ref_model_probe(const char* path, int safetensors, char* out, size_t capacity)
{
    PixModelFile model;
    const int code = model.open(path,safetensors != 0);
    std::string text = "open " + std::to_string(code) + "\n";
    if (!code) {
        for (const auto &e : model.weights) {
            const PixWeight &w = e.second;
            text += "T " + w.name + " " + std::to_string(w.type) + " ";
            for (size_t i = 0; i < w.shape.size(); i++) text += (i? "," : "") + std::to_string(w.shape[i]);
            text += " " + std::to_string(w.offset) + " " + std::to_string(w.bytes) + "\n";
        }
        for (const auto &m : model.metadata) {
            text += "M " + m.first + " ";
            ref_json(m.second,text);
            text += "\n";
        }
    }
    if (capacity) {
        const size_t n = std::min(text.size(),capacity - 1);
        std::memcpy(out,text.data(),n);
        out[n] = 0;
    }
    return text.size();
}

/* tensor_conv (src/convolution.cpp:34-100) with the weight `c.weight` (raw
 * bytes of `type`, GGML shape [kx, ky, cin, cout]) and bias `c.bias` (F32
 * [cout], NULL: none) in a PixModelFile whose mapping is a buffer.  form 0:
 * the first form (square kernel, bias required); form 1: the geometry form.
 * Returns the number of output values written (0: rejected). */
size_t ref_conv(const float* x, size_t width, size_t height, size_t cin, const void* weight, uint32_t type, size_t kx, size_t ky,
                size_t cout, const float* bias, int form, size_t sx, size_t sy, size_t left, size_t right, size_t top, size_t bottom,
                float* out, size_t capacity)
{
    const uint64_t wbytes = weight_bytes({uint64_t(kx),uint64_t(ky),uint64_t(cin),uint64_t(cout)},type);
    std::vector<unsigned char> blob(size_t(wbytes) + cout * 4);
    std::memcpy(blob.data(),weight,size_t(wbytes));
    if (bias) std::memcpy(blob.data() + wbytes,bias,cout * 4);
    PixModelFile model;
    model.data = blob.data();
    model.size = blob.size();
    model.filename = "conv";
    model.weights["c" WEIGHT_SUFFIX] = PixWeight{"c" WEIGHT_SUFFIX,{uint64_t(kx),uint64_t(ky),uint64_t(cin),uint64_t(cout)},type,0,wbytes};
    if (bias) model.weights["c" BIAS_SUFFIX] = PixWeight{"c" BIAS_SUFFIX,{uint64_t(cout)},MODEL_F32,wbytes,uint64_t(cout) * 4};
    PixTensor in(width * height,cin);
    std::copy(x,x + width * height * cin,in.values.begin());
    PixTensor o;
    if (form == 0) {
        o = tensor_conv(model,"c",in,width,height);
    } else {
        PixConv2D g;
        g.stride_x = sx;
        g.stride_y = sy;
        g.left = left;
        g.right = right;
        g.top = top;
        g.bottom = bottom;
        o = tensor_conv(model,"c",in,width,height,g,bias != nullptr);
    }
    model.data = nullptr;
    model.size = 0;
    if (o.values.empty() || o.values.size() > capacity) return 0;
    std::copy(o.values.begin(),o.values.end(),out);
    return o.values.size();
}

}
