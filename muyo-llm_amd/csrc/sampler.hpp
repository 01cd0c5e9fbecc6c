// Device sampler: the reference's host Sampler::Sample (src/Sampler.cpp:10-100) as a short
// chain of gfx950 kernels, for the per-op C ABI and the decoder's captured step.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace muyo
{
constexpr uint32_t kSampleMaxTopK = 1024;  // largest k the device top-k keeps
constexpr uint32_t kSampleSliceKeys = 2048;  // keys one selection workgroup sorts
constexpr uint32_t kSampleFinalKeys = 4096;  // candidates the last workgroup sorts
constexpr uint32_t kMt64Words = 312;

/// std::mt19937_64's state: the 312 words and the index of the next one to temper (312: twist
/// first). 2504 bytes.
struct Mt64State
{
    uint64_t x[kMt64Words];
    uint64_t next;
};

/// The sampling parameters of one launch (SamplerParams, src/Sampler.h:16-23, less the seed,
/// which lives in the engine state).
struct SampleConfig
{
    float temperature;
    int32_t topK;
    float topP;
    float repeatPenalty;
    int32_t repeatLastN;
};

/// Device scratch of one sampler: penalty counts (one word per vocabulary entry; zero between
/// calls), two candidate buffers of 64-bit (value, index) keys for the selection rounds, the slice
/// maxima, and the collection with its count.
struct SampleWorkspace
{
    uint32_t* counts;
    uint64_t* candA;
    uint64_t* candB;
    uint64_t* blockMax;
    uint64_t* gathered;
    uint32_t* collected;
};

/// k of the top-k: topK <= 0 means the whole vocabulary (src/Sampler.cpp:49).
inline uint32_t SampleTopK(const SampleConfig& c, uint32_t vocab)
{
    return c.topK <= 0 ? vocab : (static_cast<uint32_t>(c.topK) < vocab ? static_cast<uint32_t>(c.topK) : vocab);
}

/// Whether the launch sequence for these parameters exists on the device: a temperature above
/// zero needs k <= kSampleMaxTopK.
inline bool SampleSupported(const SampleConfig& c, uint32_t vocab)
{
    return vocab >= 1 && (c.temperature <= 0.0f || SampleTopK(c, vocab) <= kSampleMaxTopK);
}

/// Candidate keys one buffer holds at most for this vocabulary and k.
size_t SampleCandidateKeys(uint32_t vocab, uint32_t k);

/// Bytes of SampleWorkspace for the vocabulary and parameters, 256-byte aligned parts. The
/// counts must be zero before the first call; every call leaves them zero.
size_t SampleWorkspaceBytes(uint32_t vocab, const SampleConfig& c);

/// Carves the parts out of `base` (SampleWorkspaceBytes long).
SampleWorkspace SampleWorkspaceAt(void* base, uint32_t vocab, const SampleConfig& c);

/// Kernels LaunchSample enqueues for these parameters (separate: src != dst).
uint32_t SampleLaunches(uint32_t vocab, const SampleConfig& c, bool separate);

/// Seeds the engine state as std::mt19937_64(seed) does.
hipError_t LaunchMt64Seed(hipStream_t s, Mt64State* state, uint64_t seed);

/// Samples one token from src[0..vocab), leaving the penalised, temperature-divided logits in
/// dst (dst == src: in place, as the reference modifies its mapped logits). The history is
/// history[0..n), with n = *position + 1 when `position` is set (the decoder: every position up to
/// the current one), at most historyCount. Writes the token to *token.
hipError_t LaunchSample(hipStream_t s, const float* src, float* dst, uint32_t vocab, const int32_t* history,
                        const int32_t* position, uint32_t historyCount, const SampleConfig& c, Mt64State* state,
                        const SampleWorkspace& ws, int32_t* token);
}  // namespace muyo
