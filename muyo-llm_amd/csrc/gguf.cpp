// GGUF model files: the reader behind muyo_gguf_* and muyo_decoder_load_gguf.
//
// Reads what the reference's GgufReader reads (src/Gguf.h:40-103, src/Gguf.cpp:155-373): the
// header, the metadata table, the tensor table and the aligned data section, with the same
// conversions for its typed lookups. The file is memory-mapped and parsed through a
// bounds-checked cursor; values are located, not copied, and tensor bytes go to the device
// straight from the mapping. The decoder mapping follows src/FullModel.cpp:85-108 (the config)
// and :582-600 (tensor names), with q, k and v fused into the decoder's one QKV tensor.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace
{
constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF", little-endian
constexpr uint64_t kDefaultAlignment = 32;

// gguf_type (src/Gguf.h:11-26).
enum : uint32_t
{
    kU8 = 0,
    kI8 = 1,
    kU16 = 2,
    kI16 = 3,
    kU32 = 4,
    kI32 = 5,
    kF32 = 6,
    kBool = 7,
    kString = 8,
    kArray = 9,
    kU64 = 10,
    kI64 = 11,
    kF64 = 12,
};

// ggml_type of the two element types the decoder takes.
constexpr uint32_t kGgmlF32 = 0;
constexpr uint32_t kGgmlF16 = 1;

uint64_t ScalarBytes(uint32_t type)
{
    switch (type)
    {
        case kU8:
        case kI8:
        case kBool:
            return 1;
        case kU16:
        case kI16:
            return 2;
        case kU32:
        case kI32:
        case kF32:
            return 4;
        case kU64:
        case kI64:
        case kF64:
            return 8;
        default:
            return 0;
    }
}

/// Reads little-endian values from [data, data + size), failing (not throwing) past the end.
struct Cursor
{
    const uint8_t* data;
    uint64_t size;
    uint64_t at = 0;
    bool ok = true;

    bool Need(uint64_t n)
    {
        ok = ok && n <= size - at && at <= size;
        return ok;
    }

    template <typename T>
    T Pod()
    {
        T value{};
        if (Need(sizeof(T)))
        {
            std::memcpy(&value, data + at, sizeof(T));
            at += sizeof(T);
        }
        return value;
    }

    std::string String()
    {
        const uint64_t length = Pod<uint64_t>();
        if (!Need(length))
        {
            return {};
        }
        std::string s(reinterpret_cast<const char*>(data + at), static_cast<size_t>(length));
        at += length;
        return s;
    }

    void SkipString()
    {
        const uint64_t length = Pod<uint64_t>();
        if (Need(length))
        {
            at += length;
        }
    }
};

/// Where a metadata value sits in the file: its type, and for arrays the element type and count.
struct ValueRef
{
    uint32_t type = 0;
    uint32_t elementType = 0;
    uint64_t count = 0;
    uint64_t at = 0;  // the payload (after the array header for arrays)
};

struct TensorRef
{
    std::string name;
    uint32_t type = 0;
    uint32_t dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
};
}  // namespace

struct MuyoGguf
{
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t dataOffset = 0;
    std::vector<std::pair<std::string, ValueRef>> keys;
    std::vector<TensorRef> tensors;
    std::string scratch;  // backs the string a lookup returns

    const ValueRef* Find(const char* key) const
    {
        for (const auto& entry : keys)
        {
            if (entry.first == key)
            {
                return &entry.second;
            }
        }
        return nullptr;
    }

    const TensorRef* Tensor(const std::string& name) const
    {
        for (const TensorRef& t : tensors)
        {
            if (t.name == name)
            {
                return &t;
            }
        }
        return nullptr;
    }

    /// A scalar read as T0 then converted as a static_cast to R, as GgufReader's UintOr and
    /// FloatOr convert through std::visit (src/Gguf.cpp:251-279).
    template <typename R>
    bool Scalar(const ValueRef& v, R& out) const
    {
        Cursor c{map, size, v.at};
        switch (v.type)
        {
            case kU8:
                out = static_cast<R>(c.Pod<uint8_t>());
                break;
            case kI8:
                out = static_cast<R>(c.Pod<int8_t>());
                break;
            case kU16:
                out = static_cast<R>(c.Pod<uint16_t>());
                break;
            case kI16:
                out = static_cast<R>(c.Pod<int16_t>());
                break;
            case kU32:
                out = static_cast<R>(c.Pod<uint32_t>());
                break;
            case kI32:
                out = static_cast<R>(c.Pod<int32_t>());
                break;
            case kF32:
                out = static_cast<R>(c.Pod<float>());
                break;
            case kBool:
                out = static_cast<R>(c.Pod<uint8_t>() != 0);
                break;
            case kU64:
                out = static_cast<R>(c.Pod<uint64_t>());
                break;
            case kI64:
                out = static_cast<R>(c.Pod<int64_t>());
                break;
            case kF64:
                out = static_cast<R>(c.Pod<double>());
                break;
            default:
                return false;
        }
        return c.ok;
    }
};

namespace
{
using muyo::Fail;

/// Steps over one value of `type`, recording where it lies.
bool SkipValue(Cursor& c, uint32_t type, ValueRef& ref)
{
    ref.type = type;
    if (type == kString)
    {
        ref.at = c.at;
        c.SkipString();
        return c.ok;
    }
    if (type == kArray)
    {
        ref.elementType = c.Pod<uint32_t>();
        ref.count = c.Pod<uint64_t>();
        ref.at = c.at;
        if (ref.elementType == kString)
        {
            for (uint64_t i = 0; i < ref.count && c.ok; ++i)
            {
                c.SkipString();
            }
            return c.ok;
        }
        const uint64_t bytes = ScalarBytes(ref.elementType);
        if (bytes == 0 || ref.count > (c.size - c.at) / bytes)
        {
            return false;  // arrays of arrays are not GGUF, and the elements must fit the file
        }
        c.at += ref.count * bytes;
        return c.ok;
    }
    const uint64_t bytes = ScalarBytes(type);
    ref.at = c.at;
    return bytes != 0 && c.Need(bytes) && ((c.at += bytes), true);
}

int Parse(MuyoGguf& g, const char* path)
{
    Cursor c{g.map, g.size};
    if (c.Pod<uint32_t>() != kGgufMagic || !c.ok)
    {
        return Fail(MUYO_E_CONTRACT, "gguf_open: %s is not a GGUF file (bad magic)", path);
    }
    g.version = c.Pod<uint32_t>();
    const uint64_t tensorCount = c.Pod<uint64_t>();
    const uint64_t keyCount = c.Pod<uint64_t>();
    if (!c.ok || tensorCount > g.size || keyCount > g.size)
    {
        return Fail(MUYO_E_CONTRACT, "gguf_open: %s: truncated header", path);
    }
    for (uint64_t i = 0; i < keyCount; ++i)
    {
        std::string key = c.String();
        const uint32_t type = c.Pod<uint32_t>();
        ValueRef ref;
        if (!c.ok || !SkipValue(c, type, ref))
        {
            return Fail(MUYO_E_CONTRACT, "gguf_open: %s: metadata entry %llu is truncated or of unknown type %u", path,
                        static_cast<unsigned long long>(i), type);
        }
        g.keys.emplace_back(std::move(key), ref);
    }
    for (uint64_t i = 0; i < tensorCount; ++i)
    {
        TensorRef t;
        t.name = c.String();
        t.dims = c.Pod<uint32_t>();
        if (!c.ok || t.dims > 4)
        {
            return Fail(MUYO_E_CONTRACT, "gguf_open: %s: tensor %llu is truncated or has over 4 dimensions", path,
                        static_cast<unsigned long long>(i));
        }
        for (uint32_t d = 0; d < t.dims; ++d)
        {
            t.ne[d] = c.Pod<uint64_t>();
        }
        t.type = c.Pod<uint32_t>();
        t.offset = c.Pod<uint64_t>();
        if (!c.ok)
        {
            return Fail(MUYO_E_CONTRACT, "gguf_open: %s: tensor %llu is truncated", path,
                        static_cast<unsigned long long>(i));
        }
        g.tensors.push_back(std::move(t));
    }
    // src/Gguf.cpp:203-218: general.alignment when it is a scalar, else 32.
    uint64_t alignment = kDefaultAlignment;
    if (const ValueRef* a = g.Find("general.alignment"))
    {
        uint64_t value = 0;
        if (a->type != kString && a->type != kArray && g.Scalar(*a, value))
        {
            alignment = value;
        }
    }
    if (alignment == 0)
    {
        return Fail(MUYO_E_CONTRACT, "gguf_open: %s: general.alignment is 0", path);
    }
    g.dataOffset = (c.at + alignment - 1) / alignment * alignment;
    return MUYO_OK;
}

uint64_t Elements(const TensorRef& t)
{
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.dims; ++d)
    {
        n *= t.ne[d];
    }
    return n;
}
}  // namespace

extern "C" int muyo_gguf_open(const char* path, MuyoGguf** out)
{
    if (path == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "gguf_open: path and out are required");
    }
    *out = nullptr;
    auto* g = new MuyoGguf();
    g->fd = ::open(path, O_RDONLY);
    struct stat st
    {
    };
    if (g->fd < 0 || ::fstat(g->fd, &st) != 0)
    {
        delete g;
        return Fail(MUYO_E_RANGE, "gguf_open: cannot open %s", path);
    }
    g->size = static_cast<uint64_t>(st.st_size);
    if (g->size > 0)
    {
        void* m = ::mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (m == MAP_FAILED)
        {
            ::close(g->fd);
            delete g;
            return Fail(MUYO_E_NOMEM, "gguf_open: cannot map %s", path);
        }
        g->map = static_cast<const uint8_t*>(m);
    }
    const int status = Parse(*g, path);
    if (status != MUYO_OK)
    {
        muyo_gguf_close(g);
        return status;
    }
    *out = g;
    return MUYO_OK;
}

extern "C" void muyo_gguf_close(MuyoGguf* g)
{
    if (g == nullptr)
    {
        return;
    }
    if (g->map != nullptr)
    {
        ::munmap(const_cast<uint8_t*>(g->map), g->size);
    }
    if (g->fd >= 0)
    {
        ::close(g->fd);
    }
    delete g;
}

extern "C" uint32_t muyo_gguf_version(const MuyoGguf* g) { return g != nullptr ? g->version : 0; }

extern "C" uint64_t muyo_gguf_data_offset(const MuyoGguf* g) { return g != nullptr ? g->dataOffset : 0; }

extern "C" uint64_t muyo_gguf_tensor_count(const MuyoGguf* g) { return g != nullptr ? g->tensors.size() : 0; }

extern "C" uint64_t muyo_gguf_metadata_count(const MuyoGguf* g) { return g != nullptr ? g->keys.size() : 0; }

extern "C" int muyo_gguf_tensor_info(const MuyoGguf* g, uint64_t index, const char** name, uint32_t* type,
                                     uint32_t* n_dims, uint64_t* dims, uint64_t* offset)
{
    if (g == nullptr || index >= g->tensors.size())
    {
        return Fail(MUYO_E_RANGE, "gguf_tensor_info: no tensor %llu", static_cast<unsigned long long>(index));
    }
    const TensorRef& t = g->tensors[index];
    if (name != nullptr)
    {
        *name = t.name.c_str();
    }
    if (type != nullptr)
    {
        *type = t.type;
    }
    if (n_dims != nullptr)
    {
        *n_dims = t.dims;
    }
    if (dims != nullptr)
    {
        for (uint32_t d = 0; d < 4; ++d)
        {
            dims[d] = t.ne[d];
        }
    }
    if (offset != nullptr)
    {
        *offset = t.offset;
    }
    return MUYO_OK;
}

extern "C" int muyo_gguf_has(const MuyoGguf* g, const char* key)
{
    return g != nullptr && key != nullptr && g->Find(key) != nullptr ? 1 : 0;
}

extern "C" uint64_t muyo_gguf_uint_or(const MuyoGguf* g, const char* key, uint64_t fallback)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    uint64_t out = 0;
    return v != nullptr && g->Scalar(*v, out) ? out : fallback;
}

extern "C" double muyo_gguf_float_or(const MuyoGguf* g, const char* key, double fallback)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    double out = 0.0;
    return v != nullptr && g->Scalar(*v, out) ? out : fallback;
}

extern "C" const char* muyo_gguf_string_or(MuyoGguf* g, const char* key, const char* fallback)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    if (v == nullptr || v->type != kString)
    {
        return fallback;
    }
    Cursor c{g->map, g->size, v->at};
    g->scratch = c.String();
    return g->scratch.c_str();
}

extern "C" uint64_t muyo_gguf_string_array_size(const MuyoGguf* g, const char* key)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    return v != nullptr && v->type == kArray && v->elementType == kString ? v->count : 0;
}

extern "C" const char* muyo_gguf_string_array_at(MuyoGguf* g, const char* key, uint64_t index)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    if (v == nullptr || v->type != kArray || v->elementType != kString || index >= v->count)
    {
        return nullptr;
    }
    Cursor c{g->map, g->size, v->at};
    for (uint64_t i = 0; i < index; ++i)
    {
        c.SkipString();
    }
    g->scratch = c.String();
    return c.ok ? g->scratch.c_str() : nullptr;
}

namespace muyo
{
bool GgufStringArray(const MuyoGguf* g, const char* key, std::vector<std::string>& out)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    out.clear();
    if (v == nullptr || v->type != kArray || v->elementType != kString)
    {
        return false;
    }
    // One walk over the elements (the parse already checked that they fit the file).
    Cursor c{g->map, g->size, v->at};
    out.reserve(static_cast<size_t>(v->count));
    for (uint64_t i = 0; i < v->count && c.ok; ++i)
    {
        out.push_back(c.String());
    }
    return c.ok;
}

bool GgufInt32Array(const MuyoGguf* g, const char* key, std::vector<int32_t>& out)
{
    const ValueRef* v = g != nullptr && key != nullptr ? g->Find(key) : nullptr;
    out.clear();
    if (v == nullptr || v->type != kArray || v->elementType != kI32)
    {
        return false;
    }
    out.resize(static_cast<size_t>(v->count));
    if (!out.empty())
    {
        std::memcpy(out.data(), g->map + v->at, out.size() * sizeof(int32_t));
    }
    return true;
}
}  // namespace muyo

extern "C" int muyo_gguf_tensor_data(const MuyoGguf* g, const char* name, const void** data, uint64_t* bytes)
{
    if (g == nullptr || name == nullptr || data == nullptr || bytes == nullptr)
    {
        return Fail(MUYO_E_NULL, "gguf_tensor_data: gguf, name, data and bytes are required");
    }
    const TensorRef* t = g->Tensor(name);
    if (t == nullptr)
    {
        return Fail(MUYO_E_RANGE, "gguf_tensor_data: no tensor '%s'", name);
    }
    // src/Gguf.cpp:327-340: F32 and F16 only.
    if (t->type != kGgmlF32 && t->type != kGgmlF16)
    {
        return Fail(MUYO_E_UNSUPPORTED, "gguf_tensor_data: tensor '%s' has type %u, which is not F32 or F16", name,
                    t->type);
    }
    const uint64_t n = Elements(*t) * (t->type == kGgmlF16 ? 2 : 4);
    const uint64_t begin = g->dataOffset + t->offset;
    if (begin < g->dataOffset || begin > g->size || n > g->size - begin)
    {
        return Fail(MUYO_E_RANGE, "gguf_tensor_data: tensor '%s' runs past the end of the file", name);
    }
    *data = g->map + begin;
    *bytes = n;
    return MUYO_OK;
}

extern "C" int muyo_gguf_qwen2_config(const MuyoGguf* g, uint32_t max_seq, MuyoQwen2Config* out)
{
    if (g == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "gguf_qwen2_config: gguf and out are required");
    }
    // src/FullModel.cpp:85-108.
    MuyoQwen2Config c{};
    c.layers = static_cast<uint32_t>(muyo_gguf_uint_or(g, "qwen2.block_count", 0));
    c.hidden = static_cast<uint32_t>(muyo_gguf_uint_or(g, "qwen2.embedding_length", 0));
    c.feedForward = static_cast<uint32_t>(muyo_gguf_uint_or(g, "qwen2.feed_forward_length", 0));
    c.heads = static_cast<uint32_t>(muyo_gguf_uint_or(g, "qwen2.attention.head_count", 0));
    c.kvHeads = static_cast<uint32_t>(muyo_gguf_uint_or(g, "qwen2.attention.head_count_kv", 0));
    c.rmsEps = static_cast<float>(muyo_gguf_float_or(g, "qwen2.attention.layer_norm_rms_epsilon", 0.0));
    c.ropeBase = static_cast<float>(muyo_gguf_float_or(g, "qwen2.rope.freq_base", 10000.0));
    c.vocab = static_cast<uint32_t>(muyo_gguf_string_array_size(g, "tokenizer.ggml.tokens"));
    if (c.hidden == 0 || c.heads == 0 || c.kvHeads == 0 || c.vocab == 0)
    {
        return Fail(MUYO_E_CONTRACT, "gguf_qwen2_config: the model is missing the qwen2 dimensions or the token list");
    }
    c.headDim = c.hidden / c.heads;
    c.maxSeq = max_seq;
    // The reference always loads output.weight (src/FullModel.cpp:583); tied models omit it.
    c.untiedOutput = g->Tensor("output.weight") != nullptr ? 1u : 0u;
    *out = c;
    return MUYO_OK;
}

namespace
{
/// Copies a GGUF tensor of the expected ggml type and dimensions to `device + byteOffset`.
int Upload(MuyoDecoder* d, const MuyoGguf* g, const std::string& name, uint32_t type, uint64_t ne0, uint64_t ne1,
           uint32_t kind, uint32_t layer, uint64_t byteOffset)
{
    const TensorRef* t = g->Tensor(name);
    if (t == nullptr)
    {
        return Fail(MUYO_E_RANGE, "decoder_load_gguf: the model is missing tensor %s", name.c_str());
    }
    const uint64_t ne1Got = t->dims >= 2 ? t->ne[1] : 1;
    if (t->type != type || t->ne[0] != ne0 || ne1Got != ne1 || Elements(*t) != ne0 * ne1)
    {
        // Quantised tensors are a format the decoder does not take; F16/F32 mix-ups and wrong
        // dimensions break the model's contract.
        const bool quantised = t->type != kGgmlF16 && t->type != kGgmlF32;
        return Fail(quantised ? MUYO_E_UNSUPPORTED : MUYO_E_CONTRACT,
                    "decoder_load_gguf: tensor %s is type %u [%llu, %llu]; the decoder needs type %u [%llu, %llu]",
                    name.c_str(), t->type, static_cast<unsigned long long>(t->ne[0]),
                    static_cast<unsigned long long>(ne1Got), type, static_cast<unsigned long long>(ne0),
                    static_cast<unsigned long long>(ne1));
    }
    const void* src = nullptr;
    uint64_t bytes = 0;
    int status = muyo_gguf_tensor_data(g, name.c_str(), &src, &bytes);
    if (status != MUYO_OK)
    {
        return status;
    }
    void* base = nullptr;
    uint64_t capacity = 0;
    status = muyo_decoder_tensor(d, kind, layer, &base, &capacity);
    if (status != MUYO_OK)
    {
        return status;
    }
    if (byteOffset + bytes > capacity)
    {
        return Fail(MUYO_E_CONTRACT, "decoder_load_gguf: tensor %s does not fit the decoder's tensor", name.c_str());
    }
    MUYO_HIP_CHECK(hipMemcpy(static_cast<char*>(base) + byteOffset, src, bytes, hipMemcpyHostToDevice));
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_decoder_load_gguf(MuyoDecoder* d, const MuyoGguf* g)
{
    if (d == nullptr || g == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder_load_gguf: decoder and gguf are required");
    }
    MuyoQwen2Config want{};
    int status = muyo_gguf_qwen2_config(g, 1, &want);
    MuyoQwen2Config have{};
    if (status == MUYO_OK)
    {
        status = muyo_decoder_config(d, &have);
    }
    if (status != MUYO_OK)
    {
        return status;
    }
    if (want.layers != have.layers || want.hidden != have.hidden || want.feedForward != have.feedForward ||
        want.heads != have.heads || want.kvHeads != have.kvHeads || want.vocab != have.vocab ||
        want.untiedOutput != have.untiedOutput)
    {
        return Fail(MUYO_E_CONTRACT, "decoder_load_gguf: the file's dimensions differ from the decoder's");
    }
    const uint64_t hd = have.headDim;
    const uint64_t qdim = static_cast<uint64_t>(have.heads) * hd;
    const uint64_t kvdim = static_cast<uint64_t>(have.kvHeads) * hd;
    const uint64_t h = have.hidden;
    const uint64_t f = have.feedForward;
    // src/FullModel.cpp:582-600, tensor by tensor; q, k and v rows stack into ATTN_QKV, their
    // biases into ATTN_QKV_B.
    struct Item
    {
        const char* suffix;
        uint32_t type;
        uint64_t ne0, ne1;
        uint32_t kind;
        uint64_t offset;
    };
    const Item global[] = {
        {"token_embd.weight", kGgmlF16, h, have.vocab, MUYO_TENSOR_TOKEN_EMBD, 0},
        {"output_norm.weight", kGgmlF32, h, 1, MUYO_TENSOR_OUTPUT_NORM, 0},
        {"output.weight", kGgmlF16, h, have.vocab, MUYO_TENSOR_OUTPUT, 0},
    };
    for (const Item& it : global)
    {
        if (it.kind == MUYO_TENSOR_OUTPUT && have.untiedOutput == 0)
        {
            continue;
        }
        if ((status = Upload(d, g, it.suffix, it.type, it.ne0, it.ne1, it.kind, 0, it.offset)) != MUYO_OK)
        {
            return status;
        }
    }
    const Item layerItems[] = {
        {"attn_norm.weight", kGgmlF32, h, 1, MUYO_TENSOR_ATTN_NORM, 0},
        {"attn_q.weight", kGgmlF16, h, qdim, MUYO_TENSOR_ATTN_QKV, 0},
        {"attn_k.weight", kGgmlF16, h, kvdim, MUYO_TENSOR_ATTN_QKV, qdim * h * 2},
        {"attn_v.weight", kGgmlF16, h, kvdim, MUYO_TENSOR_ATTN_QKV, (qdim + kvdim) * h * 2},
        {"attn_q.bias", kGgmlF32, qdim, 1, MUYO_TENSOR_ATTN_QKV_B, 0},
        {"attn_k.bias", kGgmlF32, kvdim, 1, MUYO_TENSOR_ATTN_QKV_B, qdim * 4},
        {"attn_v.bias", kGgmlF32, kvdim, 1, MUYO_TENSOR_ATTN_QKV_B, (qdim + kvdim) * 4},
        {"attn_output.weight", kGgmlF16, qdim, h, MUYO_TENSOR_ATTN_OUTPUT, 0},
        {"ffn_norm.weight", kGgmlF32, h, 1, MUYO_TENSOR_FFN_NORM, 0},
        {"ffn_gate.weight", kGgmlF16, h, f, MUYO_TENSOR_FFN_GATE, 0},
        {"ffn_up.weight", kGgmlF16, h, f, MUYO_TENSOR_FFN_UP, 0},
        {"ffn_down.weight", kGgmlF16, f, h, MUYO_TENSOR_FFN_DOWN, 0},
    };
    for (uint32_t l = 0; l < have.layers; ++l)
    {
        const std::string prefix = "blk." + std::to_string(l) + ".";
        for (const Item& it : layerItems)
        {
            if ((status = Upload(d, g, prefix + it.suffix, it.type, it.ne0, it.ne1, it.kind, l, it.offset)) != MUYO_OK)
            {
                return status;
            }
        }
    }
    return MUYO_OK;
}
