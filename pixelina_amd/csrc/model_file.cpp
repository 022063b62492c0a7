// The model file reader behind pixhip_model_* (include/pixhip.h): the
// counterpart of PixModelFile::open / read (src/model.cpp:138-243), which maps a
// GGUF (version 3) or safetensors file read-only and builds its tensor
// directory and metadata with the reference's acceptance rules:
//   - the header is parsed within its first 64 MiB (MODEL_MAX_HEADER); at most
//     1e6 tensors, metadata pairs or array items; rank 1..5;
//   - a tensor's type is one of F32, F16, BF16, Q8_0, Q5_K, Q6_K and its
//     first dimension a whole number of blocks (weight_bytes,
//     src/model.cpp:87-121); GGUF offsets are multiples of general.alignment
//     (default 32, a power of two, an unsigned integer value), relative to
//     the aligned end of the header, and inside the file;
//   - safetensors entries carry dtype F32 / F16 / BF16, a shape (reversed into
//     GGML order) and data_offsets whose span is the tensor's size;
//   - duplicate tensor names or metadata keys, and overlapping tensor regions,
//     reject the file.
// Metadata values keep the reference's textual form (numbers as
// std::to_string prints them, booleans as true / false) and are handed out as
// JSON text.  The mapping stays valid until pixhip_model_close; its bytes are
// what pixhip_model_weight uploads, keyed as the weight cache keys any
// weight (file:name:offset:bytes).
#include "pixhip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace {

constexpr uint64_t kMaxHeader = 64ull * 1024 * 1024;
constexpr uint64_t kMaxItems = 1000000;
constexpr unsigned kMaxRank = 5;
constexpr unsigned kMaxDepth = 64;
constexpr uint64_t kGgufVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
enum : uint32_t { kGgufString = 8, kGgufArray = 9, kGgufFloat64 = 12 };

// A metadata or JSON value: kind, the reference's text for scalars, members.
struct Value {
    enum Kind { Invalid, Null, Boolean, Number, String, Array, Object } kind = Null;
    std::string text;
    std::vector<Value> items;
    std::map<std::string,Value> members;

    // PixJson::integer (src/json.cpp:168-177): the decimal digits of a
    // number, UINT64_MAX for anything else or on overflow.
    uint64_t integer() const
    {
        if (kind != Number || text.empty()) return UINT64_MAX;
        uint64_t r = 0;
        for (char c : text) {
            if (c < '0' || c > '9' || r > (UINT64_MAX - (uint64_t)(c - '0')) / 10) return UINT64_MAX;
            r = r * 10 + (uint64_t)(c - '0');
        }
        return r;
    }

    const Value* member(const char* key) const
    {
        if (kind != Object) return nullptr;
        auto it = members.find(key);
        return it == members.end()? nullptr : &it->second;
    }
};

Value invalid()
{
    Value v;
    v.kind = Value::Invalid;
    return v;
}

void json_escape(const std::string& s, std::string& out)
{
    static const char hex[] = "0123456789abcdef";
    out += '"';
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            out += '\\';
            out += (char)c;
        } else if (c < 0x20) {
            out += "\\u00";
            out += hex[c >> 4];
            out += hex[c & 15];
        } else {
            out += (char)c;
        }
    }
    out += '"';
}

void to_json(const Value& v, std::string& out)
{
    switch (v.kind) {
    case Value::Null: out += "null"; break;
    case Value::Boolean:
    case Value::Number: out += v.text; break;
    case Value::String: json_escape(v.text,out); break;
    case Value::Array:
        out += '[';
        for (size_t i = 0; i < v.items.size(); i++) {
            if (i) out += ',';
            to_json(v.items[i],out);
        }
        out += ']';
        break;
    case Value::Object: {
        out += '{';
        bool first = true;
        for (const auto& m : v.members) {
            if (!first) out += ',';
            first = false;
            json_escape(m.first,out);
            out += ':';
            to_json(m.second,out);
        }
        out += '}';
        break;
    }
    default: break;
    }
}

// ---- JSON (the safetensors header), RFC 8259 with the reference's limits:
// depth 64, 1e6 members, no duplicate keys (src/json.cpp) ----
class Json {
    const std::string& s;
    size_t p = 0;

    void skip()
    {
        while (p < s.size() && (s[p] == ' ' || s[p] == '\n' || s[p] == '\r' || s[p] == '\t')) p++;
    }

    int hex4()
    {
        if (s.size() - p < 4) return -1;
        int v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = s[p++];
            const int d = c >= '0' && c <= '9'? c - '0' : c >= 'a' && c <= 'f'? c - 'a' + 10 : c >= 'A' && c <= 'F'? c - 'A' + 10 : -1;
            if (d < 0) return -1;
            v = v * 16 + d;
        }
        return v;
    }

    static void utf8(unsigned cp, std::string& out)
    {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xc0 | (cp >> 6));
            out += (char)(0x80 | (cp & 63));
        } else if (cp < 0x10000) {
            out += (char)(0xe0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        } else {
            out += (char)(0xf0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 63));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        }
    }

    bool str(std::string& out)
    {
        if (p >= s.size() || s[p] != '"') return false;
        p++;
        while (p < s.size()) {
            const unsigned char c = (unsigned char)s[p++];
            if (c == '"') return true;
            if (c < 0x20) return false;
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p >= s.size()) return false;
            const char e = s[p++];
            switch (e) {
            case '"': case '\\': case '/': out += e; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                int cp = hex4();
                if (cp < 0) return false;
                if (cp >= 0xd800 && cp <= 0xdbff) {  // a high surrogate needs its low half
                    if (s.size() - p < 2 || s[p] != '\\' || s[p + 1] != 'u') return false;
                    p += 2;
                    const int lo = hex4();
                    if (lo < 0xdc00 || lo > 0xdfff) return false;
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                } else if (cp >= 0xdc00 && cp <= 0xdfff) {
                    return false;
                }
                utf8((unsigned)cp,out);
                break;
            }
            default: return false;
            }
        }
        return false;
    }

    static bool digit(char c) { return c >= '0' && c <= '9'; }

    Value val(unsigned depth)
    {
        if (depth > kMaxDepth) return invalid();
        skip();
        if (p >= s.size()) return invalid();
        Value v;
        const char c = s[p];
        if (c == '"') {
            v.kind = Value::String;
            if (!str(v.text)) return invalid();
        } else if (c == '{' || c == '[') {
            const bool obj = c == '{';
            const char close = obj? '}' : ']';
            v.kind = obj? Value::Object : Value::Array;
            p++;
            skip();
            if (p < s.size() && s[p] == close) {
                p++;
                return v;
            }
            for (;;) {
                std::string key;
                if (obj) {
                    skip();
                    if (!str(key)) return invalid();
                    skip();
                    if (p >= s.size() || s[p] != ':') return invalid();
                    p++;
                }
                Value m = val(depth + 1);
                if (m.kind == Value::Invalid) return m;
                if (obj) {
                    if (!v.members.emplace(std::move(key),std::move(m)).second) return invalid();
                } else {
                    v.items.push_back(std::move(m));
                }
                if (v.members.size() + v.items.size() > kMaxItems) return invalid();
                skip();
                if (p >= s.size()) return invalid();
                const char sep = s[p++];
                if (sep == close) break;
                if (sep != ',') return invalid();
            }
        } else if (c == 't' || c == 'f' || c == 'n') {
            const char* word = c == 't'? "true" : c == 'f'? "false" : "null";
            const size_t n = strlen(word);
            if (s.compare(p,n,word) != 0) return invalid();
            p += n;
            v.kind = c == 'n'? Value::Null : Value::Boolean;
            v.text = word;
        } else {
            const size_t start = p;
            if (s[p] == '-') p++;
            if (p >= s.size() || !digit(s[p])) return invalid();
            if (s[p] == '0') p++;
            else while (p < s.size() && digit(s[p])) p++;
            if (p < s.size() && s[p] == '.') {
                const size_t d = ++p;
                while (p < s.size() && digit(s[p])) p++;
                if (p == d) return invalid();
            }
            if (p < s.size() && (s[p] == 'e' || s[p] == 'E')) {
                p++;
                if (p < s.size() && (s[p] == '+' || s[p] == '-')) p++;
                const size_t d = p;
                while (p < s.size() && digit(s[p])) p++;
                if (p == d) return invalid();
            }
            v.kind = Value::Number;
            v.text = s.substr(start,p - start);
        }
        return v;
    }

public:
    explicit Json(const std::string& text) : s(text) {}
    Value parse()
    {
        Value v = val(0);
        skip();
        return p == s.size()? v : invalid();
    }
};

// ---- GGUF header fields, little-endian, bounded by the header limit ----
class Cursor {
    const unsigned char* d;
    uint64_t end;

public:
    uint64_t pos = 0;
    Cursor(const unsigned char* data, uint64_t size) : d(data), end(std::min(size,kMaxHeader)) {}

    bool uint(unsigned bytes, uint64_t& v)
    {
        if (pos > end || bytes > end - pos) return false;
        v = 0;
        for (unsigned i = 0; i < bytes; i++) v |= (uint64_t)d[pos + i] << (8 * i);
        pos += bytes;
        return true;
    }

    bool str(std::string& out)
    {
        uint64_t n;
        if (!uint(8,n) || n > end - pos) return false;
        out.assign(reinterpret_cast<const char*>(d + pos),(size_t)n);
        pos += n;
        return true;
    }

    // One metadata value of GGUF type `type` (gguf value types 0..12).
    Value value(uint64_t type, unsigned depth)
    {
        if (depth > kMaxDepth) return invalid();
        Value v;
        if (type == kGgufString) {
            v.kind = Value::String;
            if (!str(v.text)) return invalid();
            return v;
        }
        // u8 i8 u16 i16 u32 i32 f32 bool - - u64 i64 f64
        static const unsigned width[13] = {1,1,2,2,4,4,4,1,0,0,8,8,8};
        if (type == kGgufArray) {
            uint64_t element, count;
            if (!uint(4,element) || !uint(8,count) || count > kMaxItems || element == kGgufArray) return invalid();
            // Every item takes at least this many header bytes (a string its
            // 8-byte length): a count the rest of the header cannot hold is
            // rejected before anything is reserved for it.
            const uint64_t least = element == kGgufString? 8 : element <= kGgufFloat64 && width[element]? width[element] : 1;
            if (count > (end - pos) / least) return invalid();
            v.kind = Value::Array;
            v.items.reserve((size_t)count);
            for (uint64_t i = 0; i < count; i++) {
                Value m = value(element,depth + 1);
                if (m.kind == Value::Invalid) return m;
                v.items.push_back(std::move(m));
            }
            return v;
        }
        uint64_t raw;
        if (type > kGgufFloat64 || !uint(width[type],raw)) return invalid();
        v.kind = type == 7? Value::Boolean : Value::Number;
        switch (type) {
        case 7:
            if (raw > 1) return invalid();
            v.text = raw? "true" : "false";
            break;
        case 6: {
            float f;
            const uint32_t bits = (uint32_t)raw;
            memcpy(&f,&bits,4);
            v.text = std::to_string(f);
            break;
        }
        case kGgufFloat64: {
            double f;
            memcpy(&f,&raw,8);
            v.text = std::to_string(f);
            break;
        }
        case 1: v.text = std::to_string((int8_t)raw); break;
        case 3: v.text = std::to_string((int16_t)raw); break;
        case 5: v.text = std::to_string((int32_t)raw); break;
        case 11: v.text = std::to_string((int64_t)raw); break;
        default: v.text = std::to_string(raw); break;
        }
        return v;
    }
};

// weight_bytes (src/model.cpp:87-121): storage of a tensor, 0 when the type
// is not one the backend decodes or the shape is not whole blocks.
uint64_t tensor_bytes(const std::vector<uint64_t>& shape, uint64_t type)
{
    if (shape.empty() || shape.size() > kMaxRank) return 0;
    uint64_t block = 1, bytes;
    switch (type) {
    case 0: bytes = 4; break;
    case 1:
    case 30: bytes = 2; break;
    case 8: block = 32; bytes = 34; break;
    case 13: block = 256; bytes = 176; break;
    case 14: block = 256; bytes = 210; break;
    default: return 0;
    }
    if (!shape[0] || shape[0] % block) return 0;
    uint64_t count = shape[0] / block;
    for (size_t i = 1; i < shape.size(); i++) {
        if (!shape[i] || count > UINT64_MAX / shape[i]) return 0;
        count *= shape[i];
    }
    return count > UINT64_MAX / bytes? 0 : count * bytes;
}

struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> shape;
    uint64_t offset = 0, bytes = 0;
};

}  // namespace

struct pixhip_model {
    std::string filename;
    const unsigned char* data = nullptr;
    uint64_t size = 0;
    std::map<std::string,Value> metadata;
    std::map<std::string,Tensor> tensors;
    std::vector<const Tensor*> order;                  // tensors in name order
    std::vector<std::pair<const std::string*,std::string>> meta_json;  // key, JSON text, in key order

    ~pixhip_model()
    {
        if (data) munmap(const_cast<unsigned char*>(data),(size_t)size);
    }

    bool read_gguf()
    {
        if (memcmp(data,"GGUF",4) != 0) return false;
        Cursor c(data,size);
        c.pos = 4;
        uint64_t version, count, pairs;
        if (!c.uint(4,version) || version != kGgufVersion || !c.uint(8,count) || !c.uint(8,pairs)) return false;
        if (!count || count > kMaxItems || pairs > kMaxItems) return false;
        for (uint64_t i = 0; i < pairs; i++) {
            std::string key;
            uint64_t type;
            if (!c.str(key) || !c.uint(4,type)) return false;
            Value v = c.value(type,0);
            if (v.kind == Value::Invalid || !metadata.emplace(std::move(key),std::move(v)).second) return false;
        }
        uint64_t alignment = kDefaultAlignment;
        auto a = metadata.find("general.alignment");
        if (a != metadata.end()) alignment = a->second.integer();
        if (!alignment || (alignment & (alignment - 1)) || alignment > kMaxHeader) return false;
        for (uint64_t i = 0; i < count; i++) {
            Tensor t;
            uint64_t rank, type;
            if (!c.str(t.name) || !c.uint(4,rank) || !rank || rank > kMaxRank) return false;
            for (uint64_t d = 0; d < rank; d++) {
                uint64_t dim;
                if (!c.uint(8,dim)) return false;
                t.shape.push_back(dim);
            }
            if (!c.uint(4,type) || !c.uint(8,t.offset)) return false;
            t.type = (uint32_t)type;
            t.bytes = tensor_bytes(t.shape,type);
            if (!t.bytes || t.offset % alignment) return false;
            std::string name = t.name;
            if (!tensors.emplace(std::move(name),std::move(t)).second) return false;
        }
        const uint64_t base = (c.pos + alignment - 1) & ~(alignment - 1);
        if (base > size) return false;
        for (auto& e : tensors) {
            Tensor& t = e.second;
            if (t.offset > size - base || t.bytes > size - base - t.offset) return false;
            t.offset += base;
        }
        return true;
    }

    bool read_safetensors()
    {
        Cursor c(data,size);
        uint64_t length;
        // the length is checked against the header window (the first 64 MiB)
        if (!c.uint(8,length) || !length || length > kMaxHeader || length > std::min(size,kMaxHeader) - 8) return false;
        const std::string text(reinterpret_cast<const char*>(data + 8),(size_t)length);
        const Value root = Json(text).parse();
        if (root.kind != Value::Object) return false;
        const uint64_t base = 8 + length;
        for (const auto& e : root.members) {
            if (e.first == "__metadata__") {
                metadata = e.second.members;  // an object's members (a non-object leaves none)
                continue;
            }
            Tensor t;
            t.name = e.first;
            const Value* dtype = e.second.member("dtype");
            if (!dtype || dtype->kind != Value::String) return false;
            if (dtype->text == "F32") t.type = 0;
            else if (dtype->text == "F16") t.type = 1;
            else if (dtype->text == "BF16") t.type = 30;
            else return false;
            const Value* shape = e.second.member("shape");
            if (!shape || shape->kind != Value::Array) return false;
            for (auto it = shape->items.rbegin(); it != shape->items.rend(); ++it) t.shape.push_back(it->integer());
            const Value* offsets = e.second.member("data_offsets");
            if (!offsets || offsets->kind != Value::Array || offsets->items.size() != 2) return false;
            const uint64_t start = offsets->items[0].integer(), stop = offsets->items[1].integer();
            t.bytes = tensor_bytes(t.shape,t.type);
            if (!t.bytes || start == UINT64_MAX || stop == UINT64_MAX || stop < start || stop > size - base || stop - start != t.bytes)
                return false;
            t.offset = base + start;
            tensors.emplace(e.first,std::move(t));
        }
        return true;
    }

    bool read(bool safetensors)
    {
        if (!(safetensors? read_safetensors() : read_gguf())) return false;
        // no two tensors may share bytes
        std::vector<const Tensor*> by_offset;
        for (const auto& e : tensors) by_offset.push_back(&e.second);
        std::sort(by_offset.begin(),by_offset.end(),[](const Tensor* a, const Tensor* b) { return a->offset < b->offset; });
        uint64_t end = 0;
        for (const Tensor* t : by_offset) {
            if (t->offset < end) return false;
            end = t->offset + t->bytes;
        }
        if (tensors.empty()) return false;
        for (const auto& e : tensors) order.push_back(&e.second);
        for (const auto& m : metadata) {
            std::string j;
            to_json(m.second,j);
            meta_json.emplace_back(&m.first,std::move(j));
        }
        return true;
    }
};

namespace {

void fill(const Tensor& t, pixhip_tensor_info* info)
{
    info->name = t.name.c_str();
    info->name_length = t.name.size();
    info->type = t.type;
    info->rank = (uint32_t)t.shape.size();
    for (unsigned i = 0; i < kMaxRank; i++) info->shape[i] = i < t.shape.size()? t.shape[i] : 0;
    info->offset = t.offset;
    info->bytes = t.bytes;
}

int64_t copy_text(const std::string& s, char* out, size_t length)
{
    if (out && length) {
        const size_t n = std::min(s.size(),length - 1);
        memcpy(out,s.data(),n);
        out[n] = 0;
    }
    return (int64_t)s.size();
}

}  // namespace

extern "C" {

int pixhip_model_open(const char* path, int safetensors, pixhip_model** out)
{
    if (!path || !out) return PIXHIP_ERR_ARGUMENT;
    *out = nullptr;
    const int fd = ::open(path,O_RDONLY);
    if (fd < 0) return PIXHIP_ERR_OPEN;
    struct stat st;
    if (fstat(fd,&st) || !S_ISREG(st.st_mode) || st.st_size < 8) {
        ::close(fd);
        return PIXHIP_ERR_FORMAT;
    }
    std::unique_ptr<pixhip_model> m(new (std::nothrow) pixhip_model);
    if (!m) {
        ::close(fd);
        return PIXHIP_ERR_MEMORY;
    }
    void* mapped = mmap(nullptr,(size_t)st.st_size,PROT_READ,MAP_PRIVATE,fd,0);
    ::close(fd);
    if (mapped == MAP_FAILED) return PIXHIP_ERR_OPEN;
    m->data = static_cast<const unsigned char*>(mapped);
    m->size = (uint64_t)st.st_size;
    m->filename = path;
    if (!m->read(safetensors != 0)) return PIXHIP_ERR_FORMAT;
    *out = m.release();
    return PIXHIP_OK;
}

void pixhip_model_close(pixhip_model* model)
{
    delete model;
}

const unsigned char* pixhip_model_data(const pixhip_model* model, uint64_t* size)
{
    if (!model) return nullptr;
    if (size) *size = model->size;
    return model->data;
}

uint64_t pixhip_model_tensor_count(const pixhip_model* model)
{
    return model? model->order.size() : 0;
}

int pixhip_model_tensor_at(const pixhip_model* model, uint64_t index, pixhip_tensor_info* info)
{
    if (!model || !info || index >= model->order.size()) return PIXHIP_ERR_ARGUMENT;
    fill(*model->order[(size_t)index],info);
    return PIXHIP_OK;
}

int pixhip_model_tensor(const pixhip_model* model, const char* name, pixhip_tensor_info* info)
{
    if (!model || !name || !info) return PIXHIP_ERR_ARGUMENT;
    auto it = model->tensors.find(name);
    if (it == model->tensors.end()) return PIXHIP_ERR_ARGUMENT;
    fill(it->second,info);
    return PIXHIP_OK;
}

uint64_t pixhip_model_metadata_count(const pixhip_model* model)
{
    return model? model->meta_json.size() : 0;
}

int64_t pixhip_model_metadata_key(const pixhip_model* model, uint64_t index, char* key, size_t length)
{
    if (!model || index >= model->meta_json.size()) return PIXHIP_ERR_ARGUMENT;
    return copy_text(*model->meta_json[(size_t)index].first,key,length);
}

int64_t pixhip_model_metadata_value(const pixhip_model* model, uint64_t index, char* value, size_t length)
{
    if (!model || index >= model->meta_json.size()) return PIXHIP_ERR_ARGUMENT;
    return copy_text(model->meta_json[(size_t)index].second,value,length);
}

int64_t pixhip_model_metadata(const pixhip_model* model, const char* key, char* value, size_t length)
{
    if (!model || !key) return PIXHIP_ERR_ARGUMENT;
    for (const auto& e : model->meta_json)
        if (*e.first == key) return copy_text(e.second,value,length);
    return PIXHIP_ERR_ARGUMENT;
}

int pixhip_model_weight(pixhip_session* session, const pixhip_model* model, const char* name, pixhip_weight** out)
{
    if (!session || !model || !name || !out) return PIXHIP_ERR_ARGUMENT;
    auto it = model->tensors.find(name);
    if (it == model->tensors.end()) return PIXHIP_ERR_ARGUMENT;
    const Tensor& t = it->second;
    if (t.shape.size() != 2) return PIXHIP_ERR_ARGUMENT;
    // VulkanState::weight's key (src/backend_vulkan.cpp:744)
    const std::string key = model->filename + ":" + t.name + ":" + std::to_string(t.offset) + ":" + std::to_string(t.bytes);
    return pixhip_weight_get(session,key.c_str(),model->data + t.offset,t.bytes,t.type,t.shape[0],t.shape[1],out);
}

int pixhip_model_conv_weight(pixhip_session* session, const pixhip_model* model, const char* name, pixhip_weight** out)
{
    if (!session || !model || !name || !out) return PIXHIP_ERR_ARGUMENT;
    auto it = model->tensors.find(name);
    if (it == model->tensors.end()) return PIXHIP_ERR_ARGUMENT;
    const Tensor& t = it->second;
    const size_t rank = t.shape.size();
    if ((rank != 4 && rank != 5) || (rank == 5 && t.shape[2] != 1)) return PIXHIP_ERR_ARGUMENT;
    const std::string key = model->filename + ":" + t.name + ":" + std::to_string(t.offset) + ":" + std::to_string(t.bytes);
    return pixhip_conv_weight_get(session,key.c_str(),model->data + t.offset,t.bytes,t.type,t.shape[0],t.shape[1],t.shape[rank - 2],
                                  t.shape[rank - 1],out);
}

}  // extern "C"
