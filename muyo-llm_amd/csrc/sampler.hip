// Token sampling on gfx950: the reference's host Sampler::Sample (src/Sampler.cpp:10-100) with
// the engine of src/Sampler.h:40-41 (std::mt19937_64, one uniform double per sampled token), so a
// decoder can pick its next token without reading the logits back.
//
//   Penalty : one workgroup; each token of the last-N window counts its occurrences with global
//             atomics, and one thread per distinct token applies the penalty that many times in a
//             row (src/Sampler.cpp:12-29 penalises once per occurrence)
//   Scale   : logits[i] /= temperature over the vocabulary (src/Sampler.cpp:44-47)
//   Select  : rounds of workgroups that each sort 2048 (value, index) keys in LDS (bitonic) and
//             keep their k best, until at most 4096 candidates remain
//   Final   : one workgroup sorts the candidates, forms the double weights exp(v_i - v_0), cuts
//             at top-p, draws u from the engine and walks the kept weights to the target
//             (src/Sampler.cpp:49-98), each sum in the reference's order by a single thread
//
// The top-k order is (value descending, index ascending): equal values go to the lower index,
// an order the reference leaves to std::partial_sort. Greedy (temperature <= 0) with a penalty is
// the same chain with k = 1 and no draw; without a penalty the decoder keeps its argmax path.
#include <algorithm>

#include "common.hpp"
#include "sampler.hpp"

namespace muyo
{
namespace
{
constexpr int kSelectThreads = 256;
constexpr int kFinalThreads = 1024;
constexpr int kPenaltyThreads = 1024;
constexpr int kScaleThreads = 256;

// std::mt19937_64's parameters ([rand.predef]: mersenne_twister_engine<uint_fast64_t, 64, 312,
// 156, 31, 0xb5026f5aa96619e9, 29, 0x5555555555555555, 17, 0x71d67fffeda60000, 37,
// 0xfff7eee000000000, 43, 6364136223846793005>).
constexpr uint32_t kMtShift = 156;
constexpr uint64_t kMtMatrix = 0xb5026f5aa96619e9ull;
constexpr uint64_t kMtUpper = 0xffffffff80000000ull;  // the high w - r = 33 bits
constexpr uint64_t kMtLower = 0x000000007fffffffull;
constexpr uint64_t kMtInit = 6364136223846793005ull;

__device__ __forceinline__ uint64_t MtTwistWord(uint64_t self, uint64_t following, uint64_t far)
{
    const uint64_t y = (self & kMtUpper) | (following & kMtLower);
    return far ^ (y >> 1) ^ ((y & 1u) ? kMtMatrix : 0u);
}

__device__ __forceinline__ uint64_t MtTemper(uint64_t z)
{
    z ^= (z >> 29) & 0x5555555555555555ull;
    z ^= (z << 17) & 0x71d67fffeda60000ull;
    z ^= (z << 37) & 0xfff7eee000000000ull;
    z ^= z >> 43;
    return z;
}

/// A 64-bit key whose descending order is (value descending, index ascending). -0 counts as +0,
/// as the reference's float comparison does.
__device__ __forceinline__ uint64_t SampleKey(float v, uint32_t index)
{
    const uint32_t u = __float_as_uint(v + 0.0f);
    const uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(ordered) << 32) | static_cast<uint64_t>(~index);
}

__device__ __forceinline__ float KeyValue(uint64_t key)
{
    const uint32_t o = static_cast<uint32_t>(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ int32_t KeyIndex(uint64_t key) { return static_cast<int32_t>(~static_cast<uint32_t>(key)); }

/// Sorts kN keys in LDS into descending order (bitonic network; kN a power of two). Ends
/// synchronised.
template <uint32_t kN, int kThreads>
__device__ void SortDescending(uint64_t* keys)
{
    for (uint32_t size = 2; size <= kN; size <<= 1)
    {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1)
        {
            for (uint32_t t = threadIdx.x; t < kN / 2; t += kThreads)
            {
                const uint32_t lo = 2 * t - (t & (stride - 1));
                const uint32_t hi = lo + stride;
                const uint64_t a = keys[lo];
                const uint64_t b = keys[hi];
                const bool descending = (lo & size) == 0;
                if (descending ? a < b : a > b)
                {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(64) void Mt64SeedKernel(Mt64State* state, uint64_t seed)
{
    if (threadIdx.x == 0)
    {
        uint64_t x = seed;
        state->x[0] = x;
        for (uint32_t i = 1; i < kMt64Words; ++i)
        {
            x = kMtInit * (x ^ (x >> 62)) + i;
            state->x[i] = x;
        }
        state->next = kMt64Words;
    }
}

/// history[0..n) with n = *position + 1 (position set) or historyCount, at most historyCount.
/// dst[t] = penalty^d(src[t]) for each token t seen d times in the window, divided by the
/// temperature when `temperature` > 0 (src and dst may be the same buffer).
__global__ __launch_bounds__(kPenaltyThreads) void SamplePenaltyKernel(const float* src, float* dst, uint32_t vocab,
                                                                       const int32_t* __restrict__ history,
                                                                       const int32_t* position, uint32_t historyCount,
                                                                       int32_t lastN, float penalty, float temperature,
                                                                       uint32_t* counts)
{
    const uint32_t n = position != nullptr ? min(static_cast<uint32_t>(max(*position, -1) + 1), historyCount)
                                           : historyCount;
    const uint32_t first = (lastN >= 0 && static_cast<uint32_t>(lastN) < n) ? n - static_cast<uint32_t>(lastN) : 0;
    // Counts start at zero for every token of the window, end at zero, and are never read for
    // any other token.
    for (uint32_t i = first + threadIdx.x; i < n; i += kPenaltyThreads)
    {
        const int32_t t = history[i];
        if (t >= 0 && static_cast<uint32_t>(t) < vocab)
        {
            counts[t] = 0;
        }
    }
    __syncthreads();
    for (uint32_t i = first + threadIdx.x; i < n; i += kPenaltyThreads)
    {
        const int32_t t = history[i];
        if (t >= 0 && static_cast<uint32_t>(t) < vocab)
        {
            atomicAdd(&counts[t], 1u);
        }
    }
    __syncthreads();
    for (uint32_t i = first + threadIdx.x; i < n; i += kPenaltyThreads)
    {
        const int32_t t = history[i];
        if (t >= 0 && static_cast<uint32_t>(t) < vocab)
        {
            const uint32_t times = atomicExch(&counts[t], 0u);  // nonzero for one entry per token
            if (times != 0)
            {
                float v = src[t];
                for (uint32_t j = 0; j < times; ++j)
                {
                    v = v > 0.0f ? v / penalty : v * penalty;
                }
                dst[t] = temperature > 0.0f ? v / temperature : v;
            }
        }
    }
}

/// dst[i] = src[i] / temperature, or a copy when temperature <= 0.
__global__ __launch_bounds__(kScaleThreads) void SampleScaleKernel(const float* src, float* dst, uint32_t vocab,
                                                                   float temperature)
{
    for (uint32_t i = blockIdx.x * kScaleThreads + threadIdx.x; i < vocab; i += gridDim.x * kScaleThreads)
    {
        dst[i] = temperature > 0.0f ? src[i] / temperature : src[i];
    }
}

/// One slice of 2048 keys (from values[] with their indices, or from earlier candidates) sorted
/// in LDS; its k best go to out[slice * k ...]. Positions past `count` are padded with key 0,
/// below every real key.
__global__ __launch_bounds__(kSelectThreads) void SampleSelectKernel(const float* __restrict__ values,
                                                                     const uint64_t* __restrict__ in, uint32_t count,
                                                                     uint32_t k, uint64_t* __restrict__ out)
{
    __shared__ uint64_t keys[kSampleSliceKeys];
    const uint32_t base = blockIdx.x * kSampleSliceKeys;
    for (uint32_t j = threadIdx.x; j < kSampleSliceKeys; j += kSelectThreads)
    {
        const uint32_t i = base + j;
        uint64_t key = 0;
        if (i < count)
        {
            key = values != nullptr ? SampleKey(values[i], i) : in[i];
        }
        keys[j] = key;
    }
    __syncthreads();
    SortDescending<kSampleSliceKeys, kSelectThreads>(keys);
    for (uint32_t j = threadIdx.x; j < k; j += kSelectThreads)
    {
        out[static_cast<uint64_t>(blockIdx.x) * k + j] = keys[j];
    }
}

__global__ __launch_bounds__(kFinalThreads) void SampleFinalKernel(const float* __restrict__ values,
                                                                   const uint64_t* __restrict__ in, uint32_t count,
                                                                   uint32_t k, float temperature, float topP,
                                                                   Mt64State* state, int32_t* token)
{
    __shared__ uint64_t keys[kSampleFinalKeys];
    __shared__ double weight[kSampleMaxTopK];
    __shared__ uint64_t old[kMt64Words];
    __shared__ uint64_t fresh[kMt64Words];
    for (uint32_t j = threadIdx.x; j < kSampleFinalKeys; j += kFinalThreads)
    {
        uint64_t key = 0;
        if (j < count)
        {
            key = values != nullptr ? SampleKey(values[j], j) : in[j];
        }
        keys[j] = key;
    }
    __syncthreads();
    SortDescending<kSampleFinalKeys, kFinalThreads>(keys);
    if (temperature <= 0.0f)
    {
        if (threadIdx.x == 0)
        {
            *token = KeyIndex(keys[0]);  // greedy: the largest value, the lowest index among equals
        }
        return;
    }
    // src/Sampler.cpp:58-67: the difference is a float, its exponential a double.
    const float top = KeyValue(keys[0]);
    for (uint32_t j = threadIdx.x; j < k; j += kFinalThreads)
    {
        weight[j] = exp(static_cast<double>(KeyValue(keys[j]) - top));
    }
    // The engine's 312 words are used up: the next generation, computed in three dependent
    // phases (words 0..155 from the old state, 156..310 from the new 0..154, 311 from the new 0
    // and 155), as the sequential twist of the standard engine produces it. The word drawn comes
    // from LDS after a twist, so the kernel never reads back state it wrote.
    const uint64_t index = state->next;  // the same for every thread: written only below
    const bool twist = index >= kMt64Words;
    if (twist)
    {
        for (uint32_t i = threadIdx.x; i < kMt64Words; i += kFinalThreads)
        {
            old[i] = state->x[i];
        }
        __syncthreads();
        if (threadIdx.x < kMtShift)
        {
            const uint32_t i = threadIdx.x;
            fresh[i] = MtTwistWord(old[i], old[i + 1], old[i + kMtShift]);
        }
        __syncthreads();
        if (threadIdx.x >= kMtShift && threadIdx.x < kMt64Words - 1)
        {
            const uint32_t i = threadIdx.x;
            fresh[i] = MtTwistWord(old[i], old[i + 1], fresh[i - kMtShift]);
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
            fresh[kMt64Words - 1] = MtTwistWord(old[kMt64Words - 1], fresh[0], fresh[kMtShift - 1]);
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < kMt64Words; i += kFinalThreads)
        {
            state->x[i] = fresh[i];
        }
    }
    else
    {
        __syncthreads();
    }
    if (threadIdx.x != 0)
    {
        return;
    }
    // src/Sampler.cpp:64-84: the total, the shortest prefix whose normalised mass reaches top-p,
    // and that prefix's mass, each summed in order.
    double total = 0.0;
    for (uint32_t j = 0; j < k; ++j)
    {
        total += weight[j];
    }
    uint32_t kept = k;
    double running = 0.0;
    for (uint32_t j = 0; j < k; ++j)
    {
        running += weight[j] / total;
        if (running >= static_cast<double>(topP))
        {
            kept = j + 1;
            break;
        }
    }
    double keptMass = 0.0;
    for (uint32_t j = 0; j < kept; ++j)
    {
        keptMass += weight[j];
    }
    // src/Sampler.cpp:86-98: uniform_real_distribution<double>(0, 1) over the 64-bit engine is
    // one tempered word over 2^64 (the word rounded to double first; a result of 1 becomes the
    // largest double below 1), scaled by the kept mass.
    const uint64_t word = MtTemper(twist ? fresh[0] : state->x[index]);
    state->next = twist ? 1 : index + 1;
    double u = static_cast<double>(word) * 0x1p-64;
    if (u >= 1.0)
    {
        u = 0x1.fffffffffffffp-1;
    }
    const double target = u * keptMass;
    double reached = 0.0;
    uint32_t chosen = kept - 1;
    for (uint32_t j = 0; j < kept; ++j)
    {
        reached += weight[j];
        if (reached >= target)
        {
            chosen = j;
            break;
        }
    }
    *token = KeyIndex(keys[chosen]);
}

size_t Align256(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }
}  // namespace

size_t SampleCandidateKeys(uint32_t vocab, uint32_t k)
{
    return vocab > kSampleFinalKeys ? static_cast<size_t>(CeilDiv(vocab, kSampleSliceKeys)) * k : 1;
}

size_t SampleWorkspaceBytes(uint32_t vocab, const SampleConfig& c)
{
    const uint32_t k = c.temperature <= 0.0f ? 1 : SampleTopK(c, vocab);
    const size_t cand = SampleCandidateKeys(vocab, k) * sizeof(uint64_t);
    return Align256(static_cast<size_t>(vocab) * sizeof(uint32_t)) + 2 * Align256(cand);
}

SampleWorkspace SampleWorkspaceAt(void* base, uint32_t vocab, const SampleConfig& c)
{
    const uint32_t k = c.temperature <= 0.0f ? 1 : SampleTopK(c, vocab);
    const size_t cand = Align256(SampleCandidateKeys(vocab, k) * sizeof(uint64_t));
    char* p = static_cast<char*>(base);
    SampleWorkspace ws;
    ws.counts = reinterpret_cast<uint32_t*>(p);
    p += Align256(static_cast<size_t>(vocab) * sizeof(uint32_t));
    ws.candA = reinterpret_cast<uint64_t*>(p);
    ws.candB = reinterpret_cast<uint64_t*>(p + cand);
    return ws;
}

uint32_t SampleLaunches(uint32_t vocab, const SampleConfig& c, bool separate)
{
    const bool greedy = c.temperature <= 0.0f;
    const uint32_t k = greedy ? 1 : SampleTopK(c, vocab);
    uint32_t launches = (c.repeatPenalty != 1.0f ? 1 : 0) + ((separate || !greedy) ? 1 : 0) + 1;
    for (uint32_t count = vocab; count > kSampleFinalKeys; count = CeilDiv(count, kSampleSliceKeys) * k)
    {
        ++launches;
    }
    return launches;
}

hipError_t LaunchMt64Seed(hipStream_t s, Mt64State* state, uint64_t seed)
{
    hipLaunchKernelGGL(Mt64SeedKernel, dim3(1), dim3(64), 0, s, state, seed);
    return hipGetLastError();
}

hipError_t LaunchSample(hipStream_t s, const float* src, float* dst, uint32_t vocab, const int32_t* history,
                        const int32_t* position, uint32_t historyCount, const SampleConfig& c, Mt64State* state,
                        const SampleWorkspace& ws, int32_t* token)
{
    if (vocab == 0 || !SampleSupported(c, vocab))
    {
        return hipErrorInvalidValue;
    }
    const bool greedy = c.temperature <= 0.0f;
    const uint32_t k = greedy ? 1 : SampleTopK(c, vocab);
    const bool penalise = c.repeatPenalty != 1.0f && (position != nullptr || historyCount > 0);
    const uint32_t scaleBlocks = std::min<uint32_t>(CeilDiv(vocab, kScaleThreads), 1024);
    // In place, the penalty reads the raw logits before the division; into a separate buffer,
    // the division (or copy) goes first and the penalty then rewrites the penalised tokens from
    // the raw logits, divided. Both leave penalty^d(x) / T, as the reference computes it.
    if (src == dst)
    {
        if (penalise)
        {
            hipLaunchKernelGGL(SamplePenaltyKernel, dim3(1), dim3(kPenaltyThreads), 0, s, src, dst, vocab, history,
                               position, historyCount, c.repeatLastN, c.repeatPenalty, 0.0f, ws.counts);
        }
        if (!greedy)
        {
            hipLaunchKernelGGL(SampleScaleKernel, dim3(scaleBlocks), dim3(kScaleThreads), 0, s, src, dst, vocab,
                               c.temperature);
        }
    }
    else
    {
        hipLaunchKernelGGL(SampleScaleKernel, dim3(scaleBlocks), dim3(kScaleThreads), 0, s, src, dst, vocab,
                           c.temperature);
        if (penalise)
        {
            hipLaunchKernelGGL(SamplePenaltyKernel, dim3(1), dim3(kPenaltyThreads), 0, s, src, dst, vocab, history,
                               position, historyCount, c.repeatLastN, c.repeatPenalty, c.temperature, ws.counts);
        }
    }
    // Rounds of slice sorts until the final workgroup can hold every candidate; each round keeps
    // k of 2048 keys per slice (k <= 1024), so the count at least halves.
    const float* values = dst;
    const uint64_t* in = nullptr;
    uint32_t count = vocab;
    uint64_t* out = ws.candA;
    while (count > kSampleFinalKeys)
    {
        const uint32_t slices = CeilDiv(count, kSampleSliceKeys);
        hipLaunchKernelGGL(SampleSelectKernel, dim3(slices), dim3(kSelectThreads), 0, s, values, in, count, k, out);
        count = slices * k;
        values = nullptr;
        in = out;
        out = out == ws.candA ? ws.candB : ws.candA;
    }
    hipLaunchKernelGGL(SampleFinalKernel, dim3(1), dim3(kFinalThreads), 0, s, values, in, count, k, c.temperature,
                       c.topP, state, token);
    return hipGetLastError();
}
}  // namespace muyo

using namespace muyo;

extern "C" size_t muyo_sampler_state_bytes(void) { return sizeof(Mt64State); }

extern "C" size_t muyo_sample_workspace_bytes(uint32_t vocab, const MuyoSamplerParams* params)
{
    if (params == nullptr || vocab == 0)
    {
        return 0;
    }
    const SampleConfig c{params->temperature, params->top_k, params->top_p, params->repeat_penalty,
                         params->repeat_last_n};
    return SampleWorkspaceBytes(vocab, c);
}

extern "C" int muyo_sampler_seed(void* state, uint64_t seed, void* stream)
{
    if (state == nullptr)
    {
        return Fail(MUYO_E_NULL, "sampler_seed: the state pointer is required");
    }
    const hipError_t launched = LaunchMt64Seed(AsStream(stream), static_cast<Mt64State*>(state), seed);
    return launched == hipSuccess ? MUYO_OK : HipStatus(launched, "sampler_seed");
}

extern "C" int muyo_sample_f32(float* logits, uint32_t vocab, const int32_t* history, uint32_t history_count,
                               const MuyoSamplerParams* params, void* state, void* workspace, int32_t* token,
                               void* stream)
{
    const char* name = "sample_f32";
    if (logits == nullptr || params == nullptr || state == nullptr || workspace == nullptr || token == nullptr ||
        (history == nullptr && history_count > 0))
    {
        return Fail(MUYO_E_NULL, "%s: logits, params, state, workspace and token are required (history when "
                                 "history_count > 0)", name);
    }
    if (vocab == 0)
    {
        return Fail(MUYO_E_RANGE, "%s: vocab must be at least 1", name);
    }
    const SampleConfig c{params->temperature, params->top_k, params->top_p, params->repeat_penalty,
                         params->repeat_last_n};
    if (!SampleSupported(c, vocab))
    {
        return Fail(MUYO_E_UNSUPPORTED, "%s: a temperature above 0 needs top_k in 1..%u (or a vocabulary of at "
                                        "most %u with top_k <= 0); got top_k %d, vocab %u",
                    name, kSampleMaxTopK, kSampleMaxTopK, params->top_k, vocab);
    }
    const hipError_t launched = LaunchSample(AsStream(stream), logits, logits, vocab, history, nullptr, history_count, c,
                                             static_cast<Mt64State*>(state), SampleWorkspaceAt(workspace, vocab, c),
                                             token);
    return launched == hipSuccess ? MUYO_OK : HipStatus(launched, name);
}
