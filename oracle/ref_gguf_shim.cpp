// C entry points over the reference's own muyo_llm::GgufReader (src/Gguf.h, src/Gguf.cpp),
// compiled from the reference tree into oracle/_ref/ by this directory's Makefile — TEST
// INFRASTRUCTURE ONLY. Used to pin the product's GGUF reader; nothing here is built into it.
// Exceptions the reader throws come back as a null handle, a -1 or a null string.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "Gguf.h"

namespace
{
thread_local std::string g_text;

const muyo_llm::GgufReader& R(void* h) { return *static_cast<muyo_llm::GgufReader*>(h); }
}  // namespace

extern "C"
{
void* ref_gguf_open(const char* path)
{
    try
    {
        return new muyo_llm::GgufReader(path);
    }
    catch (const std::exception& e)
    {
        g_text = e.what();
        return nullptr;
    }
}

const char* ref_gguf_last_error() { return g_text.c_str(); }

void ref_gguf_close(void* h) { delete static_cast<muyo_llm::GgufReader*>(h); }

uint32_t ref_gguf_version(void* h) { return R(h).Version(); }

uint64_t ref_gguf_data_offset(void* h) { return R(h).DataOffset(); }

uint64_t ref_gguf_tensor_count(void* h) { return R(h).Tensors().size(); }

const char* ref_gguf_tensor_name(void* h, uint64_t i) { return R(h).Tensors().at(i).name.c_str(); }

uint32_t ref_gguf_tensor_type(void* h, uint64_t i) { return R(h).Tensors().at(i).type; }

uint32_t ref_gguf_tensor_ndims(void* h, uint64_t i)
{
    return static_cast<uint32_t>(R(h).Tensors().at(i).dimensions.size());
}

uint64_t ref_gguf_tensor_dim(void* h, uint64_t i, uint32_t d) { return R(h).Tensors().at(i).dimensions.at(d); }

uint64_t ref_gguf_tensor_offset(void* h, uint64_t i) { return R(h).Tensors().at(i).offset; }

int ref_gguf_has(void* h, const char* key) { return R(h).Has(key) ? 1 : 0; }

uint64_t ref_gguf_uint_or(void* h, const char* key, uint64_t fallback) { return R(h).UintOr(key, fallback); }

double ref_gguf_float_or(void* h, const char* key, double fallback) { return R(h).FloatOr(key, fallback); }

const char* ref_gguf_string_or(void* h, const char* key, const char* fallback)
{
    g_text = R(h).StringOr(key, fallback);
    return g_text.c_str();
}

uint64_t ref_gguf_string_array_size(void* h, const char* key) { return R(h).StringArraySize(key); }

const char* ref_gguf_string_array_at(void* h, const char* key, uint64_t index)
{
    try
    {
        g_text = R(h).StringArrayAt(key, static_cast<size_t>(index));
        return g_text.c_str();
    }
    catch (const std::exception&)
    {
        return nullptr;
    }
}

/// The tensor's bytes into out[0..capacity); their count, or -1 when the reader throws.
int64_t ref_gguf_read_tensor(void* h, const char* name, uint8_t* out, uint64_t capacity)
{
    try
    {
        const std::vector<uint8_t> bytes = R(h).ReadTensorData(name);
        if (bytes.size() <= capacity)
        {
            std::memcpy(out, bytes.data(), bytes.size());
        }
        return static_cast<int64_t>(bytes.size());
    }
    catch (const std::exception& e)
    {
        g_text = e.what();
        return -1;
    }
}
}
