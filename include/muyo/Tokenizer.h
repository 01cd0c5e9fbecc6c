#pragma once

// The reference's tokenizer class (src/Tokenizer.h:22-88) with the same methods and meanings, over
// muyo_tokenizer_* (include/muyo_hip.h). Host code; no device is needed.

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../muyo_hip.h"

namespace muyo_llm
{
namespace hip
{
class Tokenizer
{
public:
    /// Build the tables from a GGUF file's tokenizer.ggml.* metadata.
    /// @throws std::runtime_error when the file has no tokens array.
    explicit Tokenizer(const MuyoGguf* gguf)
    {
        if (muyo_tokenizer_create(gguf, &m_tokenizer) != MUYO_OK)
        {
            throw std::runtime_error(std::string("Tokenizer: ") + muyo_last_error());
        }
    }

    Tokenizer(const Tokenizer&) = delete;
    Tokenizer& operator=(const Tokenizer&) = delete;
    ~Tokenizer() { muyo_tokenizer_destroy(m_tokenizer); }

    size_t VocabSize() const { return static_cast<size_t>(muyo_tokenizer_vocab_size(m_tokenizer)); }

    /// The vocabulary string of `id`, or an empty string out of range.
    std::string TokenFor(size_t id) const { return muyo_tokenizer_token_text(m_tokenizer, id); }

    /// The raw bytes token `id` stands for (empty out of range).
    std::string TokenBytes(int32_t id) const
    {
        return Text([&](char* out, uint64_t cap, uint64_t* n)
                    { return muyo_tokenizer_token_bytes(m_tokenizer, id, out, cap, n); });
    }

    /// True for a CONTROL or USER_DEFINED token.
    bool IsSpecial(int32_t id) const { return muyo_tokenizer_is_special(m_tokenizer, id) != 0; }

    /// @throws std::invalid_argument for a code point above U+10FFFF, as the reference throws.
    std::vector<int32_t> Encode(const std::string& text, bool parseSpecial = true) const
    {
        std::vector<int32_t> ids(3 * text.size() + 1);
        uint64_t n = 0;
        if (muyo_tokenizer_encode(m_tokenizer, text.data(), text.size(), parseSpecial ? 1 : 0, ids.data(), ids.size(),
                                  &n) != MUYO_OK)
        {
            throw std::invalid_argument(std::string("Tokenizer::Encode: ") + muyo_last_error());
        }
        ids.resize(static_cast<size_t>(n));
        return ids;
    }

    std::string Decode(const std::vector<int32_t>& ids) const
    {
        return Text([&](char* out, uint64_t cap, uint64_t* n)
                    { return muyo_tokenizer_decode(m_tokenizer, ids.data(), ids.size(), out, cap, n); });
    }

private:
    template <typename Call>
    static std::string Text(Call call)
    {
        std::string out(64, '\0');
        uint64_t n = 0;
        if (call(&out[0], out.size(), &n) != MUYO_OK)
        {
            out.assign(static_cast<size_t>(n), '\0');
            if (n != 0 && call(&out[0], out.size(), &n) != MUYO_OK)
            {
                throw std::runtime_error(std::string("Tokenizer: ") + muyo_last_error());
            }
        }
        out.resize(static_cast<size_t>(n));
        return out;
    }

    MuyoTokenizer* m_tokenizer = nullptr;
};
}  // namespace hip
}  // namespace muyo_llm
