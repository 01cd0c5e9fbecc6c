#pragma once

// The reference's host sampler (src/Sampler.h:11-42, src/Sampler.cpp:10-100) with the same
// parameters and calling shape, sampling on the device: the logits stay in device memory and
// only the token comes back. Built on muyo_sample_f32 (include/muyo_hip.h).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../muyo_hip.h"

namespace muyo_llm
{
namespace hip
{
/// SamplerParams (src/Sampler.h:16-23), field for field.
struct SamplerParams
{
    float temperature = 0.0F;
    int32_t topK = 40;
    float topP = 0.95F;
    float repeatPenalty = 1.0F;
    int32_t repeatLastN = 64;  ///< How many of the latest tokens are penalised (< 0: every token so far).
    uint64_t seed = 0;
};

/// Samples the next token from a row of device logits (src/Sampler.h:25-42). The engine,
/// std::mt19937_64(params.seed) as in the reference, lives on the device; one object draws one
/// reproducible stream, token after token. Owns its device state and workspace.
class Sampler
{
public:
    /// @param vocab  The logits' length, fixed for the object's life.
    /// @param stream The HIP stream the samples are enqueued on (0: the null stream).
    Sampler(const SamplerParams& params, int32_t vocab, hipStream_t stream = nullptr)
        : m_vocab(vocab), m_stream(stream)
    {
        m_params.temperature = params.temperature;
        m_params.top_k = params.topK;
        m_params.top_p = params.topP;
        m_params.repeat_penalty = params.repeatPenalty;
        m_params.repeat_last_n = params.repeatLastN;
        m_params.reserved = 0;
        m_params.seed = params.seed;
        const size_t workspace = muyo_sample_workspace_bytes(static_cast<uint32_t>(vocab), &m_params);
        Check(hipMalloc(&m_state, muyo_sampler_state_bytes()) == hipSuccess ? MUYO_OK : MUYO_E_NOMEM);
        Check(hipMalloc(&m_workspace, workspace) == hipSuccess ? MUYO_OK : MUYO_E_NOMEM);
        Check(hipMalloc(reinterpret_cast<void**>(&m_token), sizeof(int32_t)) == hipSuccess ? MUYO_OK : MUYO_E_NOMEM);
        Check(hipMemsetAsync(m_workspace, 0, workspace, m_stream) == hipSuccess ? MUYO_OK : MUYO_E_STATE);
        Check(muyo_sampler_seed(m_state, params.seed, m_stream));
    }

    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;

    ~Sampler()
    {
        (void)hipFree(m_token);
        (void)hipFree(m_workspace);
        (void)hipFree(m_state);
        (void)hipFree(m_history);
    }

    /// @param logits  Device pointer to this position's logits; the penalty and the division by
    ///                the temperature are applied to them in place.
    /// @param vocab   Number of logits (the constructor's).
    /// @param history Every token so far (prompt and output), oldest first; the penalty window reads its tail.
    /// @return The sampled token id. Waits for the stream.
    int32_t Sample(float* logits, int32_t vocab, const std::vector<int32_t>& history)
    {
        if (vocab != m_vocab)
        {
            throw std::invalid_argument("Sampler::Sample: vocab differs from the constructor's");
        }
        const size_t bytes = history.size() * sizeof(int32_t);
        if (bytes > m_historyBytes)
        {
            (void)hipFree(m_history);
            m_history = nullptr;
            Check(hipMalloc(reinterpret_cast<void**>(&m_history), bytes) == hipSuccess ? MUYO_OK : MUYO_E_NOMEM);
            m_historyBytes = bytes;
        }
        if (bytes > 0)
        {
            Check(hipMemcpyAsync(m_history, history.data(), bytes, hipMemcpyHostToDevice, m_stream) == hipSuccess
                      ? MUYO_OK
                      : MUYO_E_STATE);
        }
        Check(muyo_sample_f32(logits, static_cast<uint32_t>(vocab), m_history, static_cast<uint32_t>(history.size()),
                              &m_params, m_state, m_workspace, m_token, m_stream));
        int32_t token = 0;
        Check(hipMemcpyAsync(&token, m_token, sizeof(token), hipMemcpyDeviceToHost, m_stream) == hipSuccess
                  ? MUYO_OK
                  : MUYO_E_STATE);
        Check(hipStreamSynchronize(m_stream) == hipSuccess ? MUYO_OK : MUYO_E_STATE);
        return token;
    }

private:
    static void Check(int status)
    {
        if (status != MUYO_OK)
        {
            const char* message = muyo_last_error();
            throw std::runtime_error(std::string("muyo sampler: ") + (message != nullptr ? message : "HIP call failed"));
        }
    }

    MuyoSamplerParams m_params{};
    int32_t m_vocab = 0;
    hipStream_t m_stream = nullptr;
    void* m_state = nullptr;
    void* m_workspace = nullptr;
    int32_t* m_token = nullptr;
    int32_t* m_history = nullptr;
    size_t m_historyBytes = 0;
};
}  // namespace hip
}  // namespace muyo_llm
