// Byte-level BPE tokenizer built from a GGUF file's tokenizer.ggml.* metadata: the code behind
// muyo_tokenizer_*.
//
// Follows the reference's muyo_llm::Tokenizer (src/Tokenizer.h:22-88, src/Tokenizer.cpp:89-345):
// special tokens (types CONTROL and USER_DEFINED) are cut out of the text first, longest match
// first; the text between them is split into pieces by the pre-tokenizer pattern that
// tokenizer.ggml.pre selects (Qwen2's, or GPT-2's); each piece's bytes become GPT-2 byte symbols
// and the ranked merges join neighbouring symbols, lowest rank first and leftmost among equals,
// until none applies; each symbol is then looked up in the vocabulary. The reference splits with
// the llama.cpp helpers it vendors (src/llama/unicode.cpp:474-606 for Qwen2, :215-330 for GPT-2,
// :30-72 and :1130-1145 for the UTF-8 decoding); the pattern matchers here are written from the
// patterns themselves.
//
// Design: every string a merge mentions is interned once, so a merge is a hash lookup of two
// integer symbol ids, and a piece is merged through a binary heap over its neighbouring pairs
// (O(n log n) in the piece length) instead of rescanning all pairs after every merge.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstring>
#include <queue>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.hpp"

namespace muyo
{
bool GgufStringArray(const MuyoGguf* g, const char* key, std::vector<std::string>& out);
bool GgufInt32Array(const MuyoGguf* g, const char* key, std::vector<int32_t>& out);
}  // namespace muyo

namespace
{
using muyo::Fail;

#include "unicode_classes.inc"

// ------------------------------------------------------------------------------------------------
// Code-point classes of the pre-tokenizer patterns: \p{L}, \p{N} and \s (White_Space).

enum : uint8_t
{
    kOther = 0,
    kLetter = 1,
    kNumber = 2,
    kSpace = 4,
};

template <size_t N>
bool InRanges(const uint32_t (&ranges)[N][2], uint32_t cp)
{
    size_t lo = 0;
    size_t hi = N;
    while (lo < hi)
    {
        const size_t mid = (lo + hi) / 2;
        if (cp < ranges[mid][0])
        {
            hi = mid;
        }
        else if (cp > ranges[mid][1])
        {
            lo = mid + 1;
        }
        else
        {
            return true;
        }
    }
    return false;
}

struct ClassTable
{
    uint8_t ascii[128];

    ClassTable()
    {
        for (uint32_t cp = 0; cp < 128; ++cp)
        {
            ascii[cp] = Slow(cp);
        }
    }

    static uint8_t Slow(uint32_t cp)
    {
        if (InRanges(kLetterRanges, cp))
        {
            return kLetter;
        }
        if (InRanges(kNumberRanges, cp))
        {
            return kNumber;
        }
        return InRanges(kWhiteSpaceRanges, cp) ? kSpace : kOther;
    }

    uint8_t operator()(uint32_t cp) const { return cp < 128 ? ascii[cp] : Slow(cp); }
};

const ClassTable& Classes()
{
    static const ClassTable table;
    return table;
}

// ------------------------------------------------------------------------------------------------
// UTF-8.

void AppendUtf8(std::string& out, uint32_t cp)
{
    if (cp < 0x80)
    {
        out.push_back(static_cast<char>(cp));
    }
    else if (cp < 0x800)
    {
        out.push_back(static_cast<char>(0xC0 | (cp >> 6)));
        out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
    else if (cp < 0x10000)
    {
        out.push_back(static_cast<char>(0xE0 | (cp >> 12)));
        out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
    else
    {
        out.push_back(static_cast<char>(0xF0 | (cp >> 18)));
        out.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
        out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
}

constexpr uint32_t kReplacement = 0xFFFD;

/// The text as code points, decoded the way the pre-split sees it (src/llama/unicode.cpp:30-72,
/// 1130-1145): a lead byte with its continuation bytes present gives their code point (overlong
/// forms and surrogates included, as written); any other byte gives U+FFFD and the decode moves
/// on by that one byte. A 4-byte form above U+10FFFF cannot be re-encoded, and the reference's
/// split then throws: that returns false here.
bool DecodeForSplit(const char* text, size_t length, std::vector<uint32_t>& cps)
{
    cps.clear();
    const auto* b = reinterpret_cast<const uint8_t*>(text);
    size_t i = 0;
    while (i < length)
    {
        const uint8_t lead = b[i];
        size_t need = 0;
        uint32_t cp = 0;
        if (lead < 0x80)
        {
            cps.push_back(lead);
            ++i;
            continue;
        }
        if ((lead & 0xE0) == 0xC0)
        {
            need = 1;
            cp = lead & 0x1F;
        }
        else if ((lead & 0xF0) == 0xE0)
        {
            need = 2;
            cp = lead & 0x0F;
        }
        else if ((lead & 0xF8) == 0xF0)
        {
            need = 3;
            cp = lead & 0x07;
        }
        // A known lead byte whose continuation bytes all lie inside the text.
        bool whole = need != 0 && i + need < length;
        if (whole)
        {
            for (size_t k = 1; k <= need; ++k)
            {
                if ((b[i + k] & 0xC0) != 0x80)
                {
                    whole = false;
                    break;
                }
                cp = (cp << 6) | (b[i + k] & 0x3F);
            }
        }
        if (!whole)
        {
            cps.push_back(kReplacement);
            ++i;
            continue;
        }
        if (cp > 0x10FFFF)
        {
            return false;
        }
        cps.push_back(cp);
        i += need + 1;
    }
    return true;
}

/// One code point of a vocabulary string, read leniently as the reference's decoder reads them
/// (src/Tokenizer.cpp:44-68): the lead byte alone fixes the length, continuation bits are taken
/// without checking, and a sequence cut short by the end keeps what it has.
uint32_t NextCodePointLenient(const std::string& s, size_t& i)
{
    const auto lead = static_cast<uint8_t>(s[i]);
    uint32_t cp = lead;
    size_t length = 1;
    if (lead >= 0xF0)
    {
        cp = lead & 0x07;
        length = 4;
    }
    else if (lead >= 0xE0)
    {
        cp = lead & 0x0F;
        length = 3;
    }
    else if (lead >= 0xC0)
    {
        cp = lead & 0x1F;
        length = 2;
    }
    for (size_t k = 1; k < length && i + k < s.size(); ++k)
    {
        cp = (cp << 6) | (static_cast<uint8_t>(s[i + k]) & 0x3F);
    }
    i += length;
    return cp;
}

// ------------------------------------------------------------------------------------------------
// Pre-tokenizer patterns. Each matcher returns the end (exclusive) of the piece that starts at
// code point i of c[0..n); k[] holds the classes of c[].

bool IsCrLf(uint32_t cp) { return cp == '\r' || cp == '\n'; }

uint32_t AsciiLower(uint32_t cp) { return cp >= 'A' && cp <= 'Z' ? cp + 32 : cp; }

/// 's 't 're 've 'm 'll 'd, compared after `fold` (identity for GPT-2, ASCII lower-casing for
/// Qwen2's case-insensitive group). Returns the end, or i when none matches.
template <typename Fold>
size_t Contraction(const uint32_t* c, size_t i, size_t n, Fold fold)
{
    if (c[i] != '\'' || i + 1 >= n)
    {
        return i;
    }
    const uint32_t a = fold(c[i + 1]);
    if (a == 's' || a == 't' || a == 'm' || a == 'd')
    {
        return i + 2;
    }
    if (i + 2 < n)
    {
        const uint32_t b = fold(c[i + 2]);
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l'))
        {
            return i + 3;
        }
    }
    return i;
}

size_t RunOf(const uint8_t* k, size_t i, size_t n, uint8_t cls)
{
    while (i < n && k[i] == cls)
    {
        ++i;
    }
    return i;
}

/// The tail shared by both patterns: a run of white space [i, e). "\s*[\r\n]+" (Qwen2 only) ends
/// after the run's last CR or LF; "\s+(?!\S)" leaves the run's last character to the next piece
/// when a non-space follows; "\s+" takes the run.
size_t WhiteSpace(const uint32_t* c, const uint8_t* k, size_t i, size_t n, bool newlineRule)
{
    size_t e = i;
    size_t afterNewline = 0;
    while (e < n && k[e] == kSpace)
    {
        if (IsCrLf(c[e]))
        {
            afterNewline = e + 1;
        }
        ++e;
    }
    if (newlineRule && afterNewline != 0)
    {
        return afterNewline;
    }
    if (e - i > 1 && e < n)
    {
        return e - 1;
    }
    return e > i ? e : i + 1;
}

/// (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|
/// \s*[\r\n]+|\s+(?!\S)|\s+
size_t MatchQwen2(const uint32_t* c, const uint8_t* k, size_t i, size_t n)
{
    const size_t contraction = Contraction(c, i, n, AsciiLower);
    if (contraction != i)
    {
        return contraction;
    }
    if (k[i] == kLetter)
    {
        return RunOf(k, i, n, kLetter);
    }
    if (!IsCrLf(c[i]) && k[i] != kNumber && i + 1 < n && k[i + 1] == kLetter)
    {
        return RunOf(k, i + 1, n, kLetter);
    }
    if (k[i] == kNumber)
    {
        return i + 1;
    }
    const size_t j = c[i] == ' ' ? i + 1 : i;
    if (j < n && k[j] == kOther)
    {
        size_t e = RunOf(k, j, n, kOther);
        while (e < n && IsCrLf(c[e]))
        {
            ++e;
        }
        return e;
    }
    return WhiteSpace(c, k, i, n, true);
}

/// 's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
size_t MatchGpt2(const uint32_t* c, const uint8_t* k, size_t i, size_t n)
{
    const size_t contraction = Contraction(c, i, n, [](uint32_t cp) { return cp; });
    if (contraction != i)
    {
        return contraction;
    }
    const size_t j = c[i] == ' ' ? i + 1 : i;
    if (j < n && (k[j] == kLetter || k[j] == kNumber || k[j] == kOther))
    {
        return RunOf(k, j, n, k[j]);
    }
    return WhiteSpace(c, k, i, n, false);
}

// ------------------------------------------------------------------------------------------------
// GPT-2's byte <-> code point map: the printable bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF stand
// for themselves; the other 68 bytes take 256, 257, ... in byte order.

struct ByteMap
{
    uint32_t toCodePoint[256];
    int16_t toByte[256 + 68];

    ByteMap()
    {
        std::fill(std::begin(toByte), std::end(toByte), static_cast<int16_t>(-1));
        uint32_t next = 256;
        for (uint32_t b = 0; b < 256; ++b)
        {
            const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || b >= 0xAE;
            toCodePoint[b] = printable ? b : next++;
            toByte[toCodePoint[b]] = static_cast<int16_t>(b);
        }
    }
};

const ByteMap& Bytes()
{
    static const ByteMap map;
    return map;
}

/// The bytes a vocabulary string stands for; code points outside the map are dropped, as the
/// reference's ByteDecode drops them (src/Tokenizer.cpp:193-207).
void AppendTokenBytes(const std::string& token, std::string& out)
{
    const ByteMap& map = Bytes();
    size_t i = 0;
    while (i < token.size())
    {
        const uint32_t cp = NextCodePointLenient(token, i);
        if (cp < 256 + 68 && map.toByte[cp] >= 0)
        {
            out.push_back(static_cast<char>(map.toByte[cp]));
        }
    }
}

struct Special
{
    std::string text;
    int32_t id;
};

struct Candidate
{
    int32_t rank;
    uint32_t left;  // node index of the pair's left symbol; nodes are in text order
    int32_t leftSymbol;
    int32_t rightSymbol;

    bool operator>(const Candidate& o) const { return rank != o.rank ? rank > o.rank : left > o.left; }
};
}  // namespace

struct MuyoTokenizer
{
    std::vector<std::string> tokens;  // id -> vocabulary string
    uint32_t vocab = 0;
    /// Symbol ids: a vocabulary string's first id, then ids >= vocab for strings only merges name.
    std::unordered_map<std::string, int32_t> symbols;
    std::vector<std::string> extra;  // the strings of ids vocab, vocab + 1, ...
    /// (left symbol << 32 | right symbol) -> rank and the joined symbol.
    std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> merges;
    int32_t byteSymbol[256];
    bool qwen2Pattern = false;
    std::vector<uint8_t> special;       // per id: CONTROL or USER_DEFINED
    std::vector<Special> specialsByLead[256];  // by first byte; longest first, then lowest id

    int32_t Intern(const std::string& s)
    {
        const auto it = symbols.find(s);
        if (it != symbols.end())
        {
            return it->second;
        }
        const int32_t id = static_cast<int32_t>(vocab + extra.size());
        extra.push_back(s);
        symbols.emplace(s, id);
        return id;
    }

    /// Ids of one pre-split piece (UTF-8 bytes), appended to `out`.
    void MergePiece(const std::string& piece, std::vector<int32_t>& out) const
    {
        const size_t n = piece.size();
        std::vector<int32_t> sym(n);
        std::vector<int32_t> next(n);
        std::vector<int32_t> prev(n);
        for (size_t i = 0; i < n; ++i)
        {
            sym[i] = byteSymbol[static_cast<uint8_t>(piece[i])];
            next[i] = i + 1 < n ? static_cast<int32_t>(i + 1) : -1;
            prev[i] = static_cast<int32_t>(i) - 1;
        }
        std::priority_queue<Candidate, std::vector<Candidate>, std::greater<Candidate>> heap;
        const auto offer = [&](int32_t left)
        {
            const int32_t right = left >= 0 ? next[left] : -1;
            if (right < 0 || sym[left] < 0 || sym[right] < 0)
            {
                return;
            }
            const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(sym[left])) << 32) |
                                 static_cast<uint32_t>(sym[right]);
            const auto it = merges.find(key);
            if (it != merges.end())
            {
                heap.push(Candidate{it->second.first, static_cast<uint32_t>(left), sym[left], sym[right]});
            }
        };
        for (size_t i = 0; i + 1 < n; ++i)
        {
            offer(static_cast<int32_t>(i));
        }
        while (!heap.empty())
        {
            const Candidate top = heap.top();
            heap.pop();
            const int32_t left = static_cast<int32_t>(top.left);
            const int32_t right = next[left];
            // Stale when either side has merged since (a symbol only ever grows, so its id changes)
            // or the left node was absorbed.
            if (sym[left] != top.leftSymbol || right < 0 || sym[right] != top.rightSymbol)
            {
                continue;
            }
            const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(sym[left])) << 32) |
                                 static_cast<uint32_t>(sym[right]);
            sym[left] = merges.at(key).second;
            sym[right] = INT32_MIN;  // absorbed
            next[left] = next[right];
            if (next[right] >= 0)
            {
                prev[next[right]] = left;
            }
            offer(prev[left]);
            offer(left);
        }
        for (int32_t i = n > 0 ? 0 : -1; i >= 0; i = next[i])
        {
            const int32_t s = sym[i];
            if (s >= 0 && static_cast<uint32_t>(s) < vocab)
            {
                out.push_back(s);
                continue;
            }
            if (s < 0)
            {
                continue;  // a byte whose symbol no vocabulary entry or merge names
            }
            // A merged string outside the vocabulary: its code points one by one, those the
            // vocabulary holds (src/Tokenizer.cpp:256-268).
            const std::string& text = extra[static_cast<size_t>(s) - vocab];
            size_t at = 0;
            while (at < text.size())
            {
                const size_t start = at;
                NextCodePointLenient(text, at);
                const auto it = symbols.find(text.substr(start, at - start));
                if (it != symbols.end() && static_cast<uint32_t>(it->second) < vocab)
                {
                    out.push_back(it->second);
                }
            }
        }
    }

    /// Pre-split one run of text (no special tokens in it) and merge each piece.
    bool EncodeRun(const char* text, size_t length, std::vector<int32_t>& out) const
    {
        std::vector<uint32_t> cps;
        if (!DecodeForSplit(text, length, cps))
        {
            return false;
        }
        const ClassTable& classes = Classes();
        std::vector<uint8_t> k(cps.size());
        for (size_t i = 0; i < cps.size(); ++i)
        {
            k[i] = classes(cps[i]);
        }
        std::string piece;
        size_t i = 0;
        while (i < cps.size())
        {
            const size_t end = qwen2Pattern ? MatchQwen2(cps.data(), k.data(), i, cps.size())
                                            : MatchGpt2(cps.data(), k.data(), i, cps.size());
            piece.clear();
            for (size_t j = i; j < end; ++j)
            {
                AppendUtf8(piece, cps[j]);
            }
            MergePiece(piece, out);
            i = end;
        }
        return true;
    }
};

// ------------------------------------------------------------------------------------------------
// C entry points.

extern "C" int muyo_tokenizer_create(const MuyoGguf* gguf, MuyoTokenizer** out)
{
    if (gguf == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "tokenizer_create: null argument");
    }
    *out = nullptr;
    auto* t = new MuyoTokenizer();
    if (!muyo::GgufStringArray(gguf, "tokenizer.ggml.tokens", t->tokens) || t->tokens.empty())
    {
        delete t;
        return Fail(MUYO_E_CONTRACT, "tokenizer_create: the file has no tokenizer.ggml.tokens");
    }
    if (t->tokens.size() > static_cast<size_t>(INT32_MAX) / 2)
    {
        delete t;
        return Fail(MUYO_E_RANGE, "tokenizer_create: %zu tokens", t->tokens.size());
    }
    t->vocab = static_cast<uint32_t>(t->tokens.size());
    t->symbols.reserve(t->tokens.size() * 2);
    for (uint32_t id = 0; id < t->vocab; ++id)
    {
        t->symbols.emplace(t->tokens[id], static_cast<int32_t>(id));  // the first of duplicates wins
    }

    // Merges "left right", split at the first space (no byte symbol is a raw space); ranks are the
    // array order, and a repeated pair keeps its first rank (src/Tokenizer.cpp:104-116).
    std::vector<std::string> mergeLines;
    muyo::GgufStringArray(gguf, "tokenizer.ggml.merges", mergeLines);
    t->merges.reserve(mergeLines.size());
    for (size_t rank = 0; rank < mergeLines.size(); ++rank)
    {
        const std::string& line = mergeLines[rank];
        const size_t space = line.find(' ');
        if (space == std::string::npos)
        {
            continue;
        }
        const std::string left = line.substr(0, space);
        const std::string right = line.substr(space + 1);
        const int32_t l = t->Intern(left);
        const int32_t r = t->Intern(right);
        const int32_t joined = t->Intern(left + right);
        const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(l)) << 32) | static_cast<uint32_t>(r);
        t->merges.emplace(key, std::make_pair(static_cast<int32_t>(rank), joined));
    }

    const ByteMap& map = Bytes();
    for (uint32_t b = 0; b < 256; ++b)
    {
        std::string s;
        AppendUtf8(s, map.toCodePoint[b]);
        const auto it = t->symbols.find(s);
        t->byteSymbol[b] = it != t->symbols.end() ? it->second : -1;
    }

    // src/Tokenizer.cpp:118-130: Qwen2's pattern for these pre-types, GPT-2's otherwise.
    std::string pre = "gpt2";
    if (const char* value = muyo_gguf_string_or(const_cast<MuyoGguf*>(gguf), "tokenizer.ggml.pre", nullptr))
    {
        pre = value;
    }
    t->qwen2Pattern = pre == "qwen2" || pre == "stablelm2" || pre == "hunyuan" || pre == "solar-open";

    // src/Tokenizer.cpp:132-151: types 3 (CONTROL) and 4 (USER_DEFINED), from an INT32 array.
    std::vector<int32_t> types;
    if (muyo::GgufInt32Array(gguf, "tokenizer.ggml.token_type", types))
    {
        t->special.assign(t->vocab, 0);
        for (size_t id = 0; id < types.size() && id < t->vocab; ++id)
        {
            if (types[id] != 3 && types[id] != 4)
            {
                continue;
            }
            t->special[id] = 1;
            // An empty special string would match everywhere without consuming text (the
            // reference's scan never ends on one); it is never matched here.
            const std::string& text = t->tokens[id];
            if (!text.empty())
            {
                t->specialsByLead[static_cast<uint8_t>(text[0])].push_back(Special{text, static_cast<int32_t>(id)});
            }
        }
        for (auto& list : t->specialsByLead)
        {
            std::stable_sort(list.begin(), list.end(),
                             [](const Special& a, const Special& b) { return a.text.size() > b.text.size(); });
        }
    }
    *out = t;
    return MUYO_OK;
}

extern "C" void muyo_tokenizer_destroy(MuyoTokenizer* t) { delete t; }

extern "C" uint64_t muyo_tokenizer_vocab_size(const MuyoTokenizer* t) { return t != nullptr ? t->vocab : 0; }

extern "C" const char* muyo_tokenizer_token_text(const MuyoTokenizer* t, uint64_t id)
{
    return t != nullptr && id < t->vocab ? t->tokens[static_cast<size_t>(id)].c_str() : "";
}

extern "C" int muyo_tokenizer_is_special(const MuyoTokenizer* t, int32_t id)
{
    return t != nullptr && id >= 0 && static_cast<size_t>(id) < t->special.size() && t->special[id] != 0 ? 1 : 0;
}

extern "C" int muyo_tokenizer_encode(const MuyoTokenizer* t, const char* text, uint64_t length, int parse_special,
                                     int32_t* ids, uint64_t capacity, uint64_t* count)
{
    if (t == nullptr || count == nullptr || (text == nullptr && length != 0) || (ids == nullptr && capacity != 0))
    {
        return Fail(MUYO_E_NULL, "tokenizer_encode: null argument");
    }
    std::vector<int32_t> out;
    out.reserve(static_cast<size_t>(length / 3 + 8));
    // Special tokens are cut out first at every byte position, the longest that matches there
    // (the lowest id among equal lengths); the runs between them are split and merged
    // (src/Tokenizer.cpp:272-320).
    size_t runStart = 0;
    size_t i = 0;
    const auto flush = [&](size_t end)
    {
        return end == runStart || t->EncodeRun(text + runStart, end - runStart, out);
    };
    while (i < length)
    {
        const Special* match = nullptr;
        if (parse_special != 0)
        {
            for (const Special& s : t->specialsByLead[static_cast<uint8_t>(text[i])])
            {
                if (s.text.size() <= length - i && std::memcmp(text + i, s.text.data(), s.text.size()) == 0)
                {
                    match = &s;
                    break;
                }
            }
        }
        if (match == nullptr)
        {
            ++i;
            continue;
        }
        if (!flush(i))
        {
            *count = 0;
            return Fail(MUYO_E_RANGE, "tokenizer_encode: the text holds a code point above U+10FFFF");
        }
        out.push_back(match->id);
        i += match->text.size();
        runStart = i;
    }
    if (!flush(length))
    {
        *count = 0;
        return Fail(MUYO_E_RANGE, "tokenizer_encode: the text holds a code point above U+10FFFF");
    }
    *count = out.size();
    if (out.size() > capacity)
    {
        return Fail(MUYO_E_RANGE, "tokenizer_encode: %zu ids, room for %llu", out.size(),
                    static_cast<unsigned long long>(capacity));
    }
    if (!out.empty())
    {
        std::memcpy(ids, out.data(), out.size() * sizeof(int32_t));
    }
    return MUYO_OK;
}

namespace
{
int CopyText(const std::string& s, char* out, uint64_t capacity, uint64_t* length, const char* what)
{
    *length = s.size();
    if (s.size() > capacity)
    {
        return Fail(MUYO_E_RANGE, "%s: %zu bytes, room for %llu", what, s.size(),
                    static_cast<unsigned long long>(capacity));
    }
    if (!s.empty())
    {
        std::memcpy(out, s.data(), s.size());
    }
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_tokenizer_decode(const MuyoTokenizer* t, const int32_t* ids, uint64_t n, char* text,
                                     uint64_t capacity, uint64_t* length)
{
    if (t == nullptr || length == nullptr || (ids == nullptr && n != 0) || (text == nullptr && capacity != 0))
    {
        return Fail(MUYO_E_NULL, "tokenizer_decode: null argument");
    }
    std::string out;
    for (uint64_t i = 0; i < n; ++i)
    {
        if (ids[i] >= 0 && static_cast<uint32_t>(ids[i]) < t->vocab)
        {
            AppendTokenBytes(t->tokens[static_cast<size_t>(ids[i])], out);
        }
    }
    return CopyText(out, text, capacity, length, "tokenizer_decode");
}

extern "C" int muyo_tokenizer_token_bytes(const MuyoTokenizer* t, int32_t id, char* bytes, uint64_t capacity,
                                          uint64_t* length)
{
    if (t == nullptr || length == nullptr || (bytes == nullptr && capacity != 0))
    {
        return Fail(MUYO_E_NULL, "tokenizer_token_bytes: null argument");
    }
    std::string out;
    if (id >= 0 && static_cast<uint32_t>(id) < t->vocab)
    {
        AppendTokenBytes(t->tokens[static_cast<size_t>(id)], out);
    }
    return CopyText(out, bytes, capacity, length, "tokenizer_token_bytes");
}
