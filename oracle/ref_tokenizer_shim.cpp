// C entry points over the reference's own muyo_llm::Tokenizer (src/Tokenizer.h, src/Tokenizer.cpp,
// with its GgufReader and the llama.cpp Unicode helpers it vendors under src/llama/), compiled from
// the reference tree into oracle/_ref/ by this directory's Makefile — TEST INFRASTRUCTURE ONLY.
// Used to pin the oracle's tokenizer restatement and the product's tokenizer; nothing here is built
// into the product. Exceptions come back as -1 with the message in ref_tok_last_error().
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

#include "Gguf.h"
#include "Tokenizer.h"
#include "llama/unicode.h"

namespace
{
thread_local std::string g_error;

struct Handle
{
    std::unique_ptr<muyo_llm::GgufReader> reader;
    std::unique_ptr<muyo_llm::Tokenizer> tokenizer;
};

const muyo_llm::Tokenizer& T(void* h) { return *static_cast<Handle*>(h)->tokenizer; }

int64_t CopyOut(const std::string& s, char* out, uint64_t capacity)
{
    if (s.size() <= capacity && !s.empty())
    {
        std::memcpy(out, s.data(), s.size());
    }
    return static_cast<int64_t>(s.size());
}
}  // namespace

extern "C"
{
const char* ref_tok_last_error() { return g_error.c_str(); }

void* ref_tok_open(const char* path)
{
    try
    {
        auto h = std::make_unique<Handle>();
        h->reader = std::make_unique<muyo_llm::GgufReader>(path);
        h->tokenizer = std::make_unique<muyo_llm::Tokenizer>(*h->reader);
        return h.release();
    }
    catch (const std::exception& e)
    {
        g_error = e.what();
        return nullptr;
    }
}

void ref_tok_close(void* h) { delete static_cast<Handle*>(h); }

uint64_t ref_tok_vocab_size(void* h) { return T(h).VocabSize(); }

/// Token ids of text[0..length) into ids[0..capacity); returns the count (which may exceed
/// capacity, in which case nothing is written) or -1 when Encode throws.
int64_t ref_tok_encode(void* h, const char* text, uint64_t length, int parse_special, int32_t* ids, uint64_t capacity)
{
    try
    {
        const std::vector<int32_t> v = T(h).Encode(std::string(text, length), parse_special != 0);
        if (v.size() <= capacity && !v.empty())
        {
            std::memcpy(ids, v.data(), v.size() * sizeof(int32_t));
        }
        return static_cast<int64_t>(v.size());
    }
    catch (const std::exception& e)
    {
        g_error = e.what();
        return -1;
    }
}

int64_t ref_tok_decode(void* h, const int32_t* ids, uint64_t n, char* out, uint64_t capacity)
{
    return CopyOut(T(h).Decode(std::vector<int32_t>(ids, ids + n)), out, capacity);
}

int64_t ref_tok_token_bytes(void* h, int32_t id, char* out, uint64_t capacity)
{
    return CopyOut(T(h).TokenBytes(id), out, capacity);
}

int64_t ref_tok_token_text(void* h, uint64_t id, char* out, uint64_t capacity)
{
    return CopyOut(T(h).TokenFor(id), out, capacity);
}

int ref_tok_is_special(void* h, int32_t id) { return T(h).IsSpecial(id) ? 1 : 0; }

/// The vendored llama.cpp category flags of one code point (unicode.h's unicode_cpt_flags).
uint32_t ref_unicode_flags(uint32_t cpt) { return unicode_cpt_flags_from_cpt(cpt).as_uint(); }
}
