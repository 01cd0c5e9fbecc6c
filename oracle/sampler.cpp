// CPU restatement of the reference's host sampler — TEST INFRASTRUCTURE ONLY.
//
// Restates muyo_llm::Sampler::Sample (src/Sampler.cpp:10-100) with the parameters of
// SamplerParams (src/Sampler.h:16-23) and the engine of Sampler (src/Sampler.h:40-41:
// std::mt19937_64 seeded with params.seed, drawn through std::uniform_real_distribution<double>).
// The engine and distribution are the C++ library's own, so a draw here is the draw the reference
// makes when built by the same standard library (libstdc++ of g++ 11 in this image).
//
// One choice is this restatement's: among exactly equal logits the top-k order puts the lower
// index first. The reference leaves that order to std::partial_sort, which does not specify it.
//
// Pinned by tests/test_sampler.py against the reference's Sampler.cpp itself (compiled from
// the reference tree into oracle/_ref by this directory's Makefile), against the C++ standard's
// mt19937_64 known answer, and against closed forms (greedy, top-k 1, top-p cuts).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <random>
#include <vector>

namespace
{
struct OracleSampler
{
    float temperature;
    int32_t topK;
    float topP;
    float repeatPenalty;
    int32_t repeatLastN;
    std::mt19937_64 rng;
};

// src/Sampler.cpp:12-29: every entry of the last-N window applies the penalty once, so a token
// seen d times is divided (or multiplied) d times in a row.
void ApplyPenalty(const OracleSampler& s, float* logits, int32_t vocab, const int32_t* history, size_t count)
{
    if (s.repeatPenalty == 1.0F || count == 0)
    {
        return;
    }
    size_t first = 0;
    if (s.repeatLastN >= 0 && static_cast<size_t>(s.repeatLastN) < count)
    {
        first = count - static_cast<size_t>(s.repeatLastN);
    }
    for (size_t i = first; i < count; ++i)
    {
        const int32_t token = history[i];
        if (token < 0 || token >= vocab)
        {
            continue;
        }
        const float v = logits[token];
        logits[token] = v > 0.0F ? v / s.repeatPenalty : v * s.repeatPenalty;
    }
}

int32_t Sample(OracleSampler& s, float* logits, int32_t vocab, const int32_t* history, size_t count)
{
    ApplyPenalty(s, logits, vocab, history, count);
    if (s.temperature <= 0.0F)
    {
        // src/Sampler.cpp:31-42: strict '>', so the lowest index wins a tie.
        int32_t best = 0;
        for (int32_t i = 1; i < vocab; ++i)
        {
            best = logits[i] > logits[best] ? i : best;
        }
        return best;
    }
    for (int32_t i = 0; i < vocab; ++i)
    {
        logits[i] /= s.temperature;  // src/Sampler.cpp:44-47
    }
    const int32_t k = s.topK <= 0 ? vocab : std::min(s.topK, vocab);
    std::vector<int32_t> order(static_cast<size_t>(vocab));
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](int32_t a, int32_t b) {
        return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
    });
    // src/Sampler.cpp:58-67: the difference is a float, its exponential a double.
    const float top = logits[order[0]];
    std::vector<double> weight(static_cast<size_t>(k));
    double total = 0.0;
    for (int32_t i = 0; i < k; ++i)
    {
        weight[i] = std::exp(static_cast<double>(logits[order[i]] - top));
        total += weight[i];
    }
    // src/Sampler.cpp:69-84: the shortest prefix whose normalised mass reaches top-p.
    int32_t kept = k;
    double running = 0.0;
    for (int32_t i = 0; i < k; ++i)
    {
        running += weight[i] / total;
        if (running >= static_cast<double>(s.topP))
        {
            kept = i + 1;
            break;
        }
    }
    double keptMass = 0.0;
    for (int32_t i = 0; i < kept; ++i)
    {
        keptMass += weight[i];
    }
    // src/Sampler.cpp:86-98: one uniform double in [0, 1) scaled by the kept mass, then the first
    // index whose running weight reaches it.
    std::uniform_real_distribution<double> uniform(0.0, 1.0);
    const double target = uniform(s.rng) * keptMass;
    double reached = 0.0;
    for (int32_t i = 0; i < kept; ++i)
    {
        reached += weight[i];
        if (reached >= target)
        {
            return order[i];
        }
    }
    return order[kept - 1];
}
}  // namespace

extern "C"
{
void* oracle_sampler_new(float temperature, int32_t top_k, float top_p, float repeat_penalty, int32_t repeat_last_n,
                         uint64_t seed)
{
    return new OracleSampler{temperature, top_k, top_p, repeat_penalty, repeat_last_n, std::mt19937_64(seed)};
}

void oracle_sampler_free(void* sampler) { delete static_cast<OracleSampler*>(sampler); }

/// Samples from logits[0..vocab) (modified in place, as the reference does) with the history
/// history[0..count), oldest first.
int32_t oracle_sampler_sample(void* sampler, float* logits, int32_t vocab, const int32_t* history, uint64_t count)
{
    return Sample(*static_cast<OracleSampler*>(sampler), logits, vocab, history, static_cast<size_t>(count));
}

/// The first n outputs of std::mt19937_64(seed).
void oracle_mt64_outputs(uint64_t seed, uint64_t n, uint64_t* out)
{
    std::mt19937_64 engine(seed);
    for (uint64_t i = 0; i < n; ++i)
    {
        out[i] = engine();
    }
}

/// The first n draws of std::uniform_real_distribution<double>(0, 1) over std::mt19937_64(seed).
void oracle_mt64_uniform(uint64_t seed, uint64_t n, double* out)
{
    std::mt19937_64 engine(seed);
    std::uniform_real_distribution<double> uniform(0.0, 1.0);
    for (uint64_t i = 0; i < n; ++i)
    {
        out[i] = uniform(engine);
    }
}
}
