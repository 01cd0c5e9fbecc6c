// C entry points over the reference's own muyo_llm::Sampler (src/Sampler.h, src/Sampler.cpp),
// compiled from the reference tree into oracle/_ref/ by this directory's Makefile — TEST
// INFRASTRUCTURE ONLY. Used to pin oracle/sampler.cpp; nothing here is built into the product.
#include <cstdint>
#include <vector>

#include "Sampler.h"

extern "C"
{
void* ref_sampler_new(float temperature, int32_t top_k, float top_p, float repeat_penalty, int32_t repeat_last_n,
                      uint64_t seed)
{
    muyo_llm::SamplerParams params;
    params.temperature = temperature;
    params.topK = top_k;
    params.topP = top_p;
    params.repeatPenalty = repeat_penalty;
    params.repeatLastN = repeat_last_n;
    params.seed = seed;
    return new muyo_llm::Sampler(params);
}

void ref_sampler_free(void* sampler) { delete static_cast<muyo_llm::Sampler*>(sampler); }

int32_t ref_sampler_sample(void* sampler, float* logits, int32_t vocab, const int32_t* history, uint64_t count)
{
    const std::vector<int32_t> fed(history, history + count);
    return static_cast<muyo_llm::Sampler*>(sampler)->Sample(logits, vocab, fed);
}
}
