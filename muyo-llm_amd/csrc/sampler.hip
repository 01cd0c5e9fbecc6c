// Token sampling on gfx950: the reference's host Sampler::Sample (src/Sampler.cpp:10-100) with
// the engine of src/Sampler.h:40-41 (std::mt19937_64, one uniform double per sampled token), so a
// decoder can pick its next token without reading the logits back.
//
//   Scale   : each of 256 workgroups owns a slice of the vocabulary. It counts in LDS how often
//             each of its tokens occurs in the last-N window, applies the repetition penalty that
//             many times in a row (src/Sampler.cpp:12-29 penalises once per occurrence), divides
//             by the temperature (src/Sampler.cpp:44-47) and records its slice's largest key.
//             (Slices too long for LDS counts take a separate one-workgroup Penalty kernel with
//             global counts first.)
//   Collect : the k-th largest of those 256 maxima is a threshold at least k keys reach, so the
//             top k lies among the keys at or above it: those (typically a few times k) are
//             gathered (k <= 256, vocabulary over 4096)
//   Select  : without a collection (k > 256): rounds of workgroups that each sort 2048 keys in
//             LDS (bitonic) and keep their k best, until 4096 remain
//   Final   : one workgroup orders the candidates (by rank when there are at most 512, else a
//             bitonic sort; when over 4096 keys tie at the top and overflow the collection, it
//             selects from the whole vocabulary itself, 4096 keys at a time), forms the double
//             weights exp(v_i - v_0), cuts at top-p, draws u from the engine and walks the kept
//             weights to the target (src/Sampler.cpp:49-98). Each sum runs in the reference's
//             order in a single thread; the divisions run in parallel.
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
constexpr int kFinalThreads = 256;
constexpr int kPenaltyThreads = 1024;
constexpr int kScaleThreads = 256;
constexpr uint32_t kThresholdBlocks = 256;  // slices whose maxima set the collection threshold
constexpr uint32_t kMarked = 0xFFFFFFFFu;   // a count word of a token the penalty finished
constexpr uint32_t kScaleSliceMax = 2048;   // slice length whose penalty counts fit LDS

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

/// LDS slot of key i: one pad word per 16 keys, so the runs of 8 or 16 keys that threads read in
/// the register stages start in different banks (unpadded, every lane of a wave hit one bank).
__device__ __forceinline__ uint32_t Slot(uint32_t i) { return i + (i >> 4); }

constexpr uint32_t PaddedKeys(uint32_t n) { return n + n / 16; }

/// Sorts kN keys in LDS (at Slot(i)) into descending order with a bitonic network (kN a power of
/// two, kN / kThreads keys per thread). Thread t owns the run [t * kPer, t * kPer + kPer): the stages whose
/// partners lie inside a run (stride < kPer) run in registers, the others through LDS, each pair
/// as an unconditional max/min write. Ends synchronised.
template <uint32_t kN, int kThreads>
__device__ void SortDescending(uint64_t* keys)
{
    constexpr uint32_t kPer = kN / kThreads;
    static_assert(kPer >= 2 && (kPer & (kPer - 1)) == 0, "a power-of-two run per thread");
    auto inRegisters = [&](uint32_t size, uint32_t topStride) {
        const uint32_t base = threadIdx.x * kPer;
        uint64_t v[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            v[j] = keys[Slot(base + j)];
        }
#pragma unroll
        for (uint32_t stride = kPer / 2; stride > 0; stride >>= 1)
        {
            if (stride <= topStride)
            {
#pragma unroll
                for (uint32_t j = 0; j < kPer; ++j)
                {
                    if ((j & stride) == 0)
                    {
                        // Blocks of `size` alternate direction; a run can hold several.
                        const bool descending = ((base + j) & size) == 0;
                        const uint64_t a = v[j];
                        const uint64_t b = v[j + stride];
                        const uint64_t hi = a > b ? a : b;
                        const uint64_t lo = a > b ? b : a;
                        v[j] = descending ? hi : lo;
                        v[j + stride] = descending ? lo : hi;
                    }
                }
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            keys[Slot(base + j)] = v[j];
        }
        __syncthreads();
    };
    for (uint32_t size = 2; size <= kN; size <<= 1)
    {
        uint32_t stride = size >> 1;
        for (; stride >= kPer; stride >>= 1)
        {
            uint64_t a[kPer / 2];
            uint64_t b[kPer / 2];
            uint32_t lo[kPer / 2];
#pragma unroll
            for (uint32_t j = 0; j < kPer / 2; ++j)
            {
                const uint32_t t = threadIdx.x + j * kThreads;
                lo[j] = 2 * t - (t & (stride - 1));
                a[j] = keys[Slot(lo[j])];
                b[j] = keys[Slot(lo[j] + stride)];
            }
#pragma unroll
            for (uint32_t j = 0; j < kPer / 2; ++j)
            {
                const bool descending = (lo[j] & size) == 0;
                const uint64_t hi = a[j] > b[j] ? a[j] : b[j];
                const uint64_t low = a[j] > b[j] ? b[j] : a[j];
                keys[Slot(lo[j])] = descending ? hi : low;
                keys[Slot(lo[j] + stride)] = descending ? low : hi;
            }
            __syncthreads();
        }
        inRegisters(size, stride);
    }
}

/// Fills LDS with keys base..base+kN-1: values[i] with index i, or earlier candidates in[i]; past
/// `count`, key 0 (below every real key). Every load is issued before any is used (clamped
/// indices, no branches). Ends synchronised.
template <uint32_t kN, int kThreads>
__device__ void LoadKeys(uint64_t* keys, const float* __restrict__ values, const uint64_t* __restrict__ in,
                         uint32_t base, uint32_t count)
{
    constexpr uint32_t kPer = kN / kThreads;
    uint64_t v[kPer];
    if (values != nullptr)
    {
        float f[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            f[j] = values[min(base + threadIdx.x + j * kThreads, count - 1)];
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            const uint32_t i = base + threadIdx.x + j * kThreads;
            v[j] = i < count ? SampleKey(f[j], i) : 0;
        }
    }
    else
    {
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            v[j] = in[min(base + threadIdx.x + j * kThreads, count - 1)];
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j)
        {
            v[j] = base + threadIdx.x + j * kThreads < count ? v[j] : 0;
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j)
    {
        keys[Slot(threadIdx.x + j * kThreads)] = v[j];
    }
    __syncthreads();
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

/// The last-N window of the history for the penalty (src/Sampler.cpp:12-16).
struct PenaltyWindow
{
    const int32_t* history;
    const int32_t* position;  // n = *position + 1 when set, at most historyCount
    uint32_t historyCount;
    int32_t lastN;
    float penalty;
};

/// penalty applied `times` times in a row (src/Sampler.cpp:18-27).
__device__ __forceinline__ float Penalise(float v, uint32_t times, float penalty)
{
    for (uint32_t j = 0; j < times; ++j)
    {
        v = v > 0.0f ? v / penalty : v * penalty;
    }
    return v;
}

/// history[0..n) with n = *position + 1 (position set) or historyCount, at most historyCount.
/// dst[t] = penalty^d(src[t]) for each token t seen d times in the window, divided by the
/// temperature when `temperature` > 0 (src and dst may be the same buffer), and counts[t] set to
/// kMarked so the scale kernel leaves it (and clears the mark).
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
            const uint32_t times = atomicExch(&counts[t], kMarked);  // a count for one entry per token
            if (times != 0 && times != kMarked)
            {
                const float v = Penalise(src[t], times, penalty);
                dst[t] = temperature > 0.0f ? v / temperature : v;
            }
        }
    }
}

/// The largest of a workgroup's 64-bit keys, in thread 0 (256 threads).
__device__ __forceinline__ uint64_t BlockMaxKey(uint64_t key, uint64_t* scratch)
{
    scratch[threadIdx.x] = key;
    __syncthreads();
    for (uint32_t half = kScaleThreads / 2; half > 0; half >>= 1)
    {
        if (threadIdx.x < half)
        {
            const uint64_t other = scratch[threadIdx.x + half];
            scratch[threadIdx.x] = other > scratch[threadIdx.x] ? other : scratch[threadIdx.x];
        }
        __syncthreads();
    }
    return scratch[0];
}

/// Workgroup b of kThresholdBlocks owns logits [b * slice, (b + 1) * slice). dst[i] =
/// penalty^d(src[i]) / temperature, d being the occurrences of token i in the window (counted in
/// LDS when `penalise`), without the division when temperature <= 0. Tokens
/// the separate Penalty kernel marked (`counts` set) already hold their final dst; the mark is
/// cleared here. With blockMax set, records the slice's largest key and (workgroup 0) zeroes the
/// collection count.
__global__ __launch_bounds__(kScaleThreads) void SampleScaleKernel(const float* src, float* dst, uint32_t vocab,
                                                                   float temperature, uint32_t* counts, bool penalise,
                                                                   PenaltyWindow pw, uint64_t* blockMax,
                                                                   uint32_t* collected)
{
    __shared__ uint64_t scratch[kScaleThreads];
    __shared__ uint32_t hits[kScaleSliceMax];
    const uint32_t slice = (vocab + gridDim.x - 1) / gridDim.x;
    const uint32_t begin = blockIdx.x * slice;
    const uint32_t end = min(begin + slice, vocab);
    if (penalise)
    {
        for (uint32_t i = threadIdx.x; i < end - min(begin, end); i += kScaleThreads)
        {
            hits[i] = 0;
        }
        __syncthreads();
        const uint32_t n = pw.position != nullptr
                               ? min(static_cast<uint32_t>(max(*pw.position, -1) + 1), pw.historyCount)
                               : pw.historyCount;
        const uint32_t first =
            (pw.lastN >= 0 && static_cast<uint32_t>(pw.lastN) < n) ? n - static_cast<uint32_t>(pw.lastN) : 0;
        for (uint32_t i = first + threadIdx.x; i < n; i += kScaleThreads)
        {
            const int32_t t = pw.history[i];
            if (t >= 0 && static_cast<uint32_t>(t) >= begin && static_cast<uint32_t>(t) < end)
            {
                atomicAdd(&hits[t - begin], 1u);
            }
        }
        __syncthreads();
    }
    uint64_t best = 0;
    for (uint32_t i = begin + threadIdx.x; i < end; i += kScaleThreads)
    {
        float v;
        if (counts != nullptr && counts[i] == kMarked)
        {
            counts[i] = 0;
            v = dst[i];
        }
        else
        {
            v = src[i];
            if (penalise)
            {
                v = Penalise(v, hits[i - begin], pw.penalty);
            }
            v = temperature > 0.0f ? v / temperature : v;
            dst[i] = v;
        }
        const uint64_t key = SampleKey(v, i);
        best = key > best ? key : best;
    }
    if (blockMax != nullptr)
    {
        best = BlockMaxKey(best, scratch);
        if (threadIdx.x == 0)
        {
            blockMax[blockIdx.x] = best;
            if (blockIdx.x == 0)
            {
                *collected = 0;
            }
        }
    }
}

/// The collection threshold from the kThresholdBlocks slice maxima: the k-th largest (distinct
/// keys when the slice holds any, so exactly one thread finds itself at rank k - 1), or 0 (every
/// key) when rank k - 1 falls among empty slices (maximum 0) or nowhere. kScaleThreads threads,
/// maxima[] already in LDS; ends synchronised.
__device__ uint64_t CollectionThreshold(const uint64_t* maxima, uint32_t k, uint64_t* threshold)
{
    static_assert(kScaleThreads == kThresholdBlocks, "one thread per slice maximum");
    if (threadIdx.x == 0)
    {
        *threshold = 0;
    }
    __syncthreads();
    const uint64_t mine = maxima[threadIdx.x];
    uint32_t rank = 0;
    for (uint32_t j = 0; j < kThresholdBlocks; ++j)
    {
        rank += maxima[j] > mine ? 1u : 0u;
    }
    if (rank == k - 1 && mine != 0)
    {
        *threshold = mine;
    }
    __syncthreads();
    return *threshold;
}

/// Gathers every key of its slice at or above the threshold: the k-th largest of the
/// kThresholdBlocks slice maxima (distinct keys when the slice holds any, so one thread finds
/// itself at rank k - 1). At least k keys reach it: the maxima of rank 0..k-1.
/// Appends up to kSampleFinalKeys keys to `out`; *collected counts them all, past that too.
__global__ __launch_bounds__(kScaleThreads) void SampleCollectKernel(const float* __restrict__ values,
                                                                     uint32_t vocab, uint32_t k,
                                                                     const uint64_t* __restrict__ blockMax,
                                                                     uint64_t* __restrict__ out, uint32_t* collected)
{
    __shared__ uint64_t maxima[kThresholdBlocks];
    __shared__ uint64_t threshold;
    maxima[threadIdx.x] = blockMax[threadIdx.x];
    const uint64_t floor = CollectionThreshold(maxima, k, &threshold);
    const uint32_t slice = (vocab + gridDim.x - 1) / gridDim.x;
    const uint32_t begin = blockIdx.x * slice;
    const uint32_t end = min(begin + slice, vocab);
    const uint32_t lane = threadIdx.x & (kWave - 1);
    for (uint32_t first = begin; first < end; first += kScaleThreads)
    {
        const uint32_t i = first + threadIdx.x;
        const uint64_t key = i < end ? SampleKey(values[i], i) : 0;
        const bool take = i < end && key >= floor;
        // One atomic per wave: the wave's takers get consecutive slots.
        const uint64_t mask = __ballot(take);
        if (mask != 0)
        {
            const uint32_t leader = static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(mask)) - 1);
            uint32_t base = 0;
            if (lane == leader)
            {
                base = atomicAdd(collected, static_cast<uint32_t>(__popcll(mask)));
            }
            base = __shfl(base, leader);
            if (take)
            {
                const uint32_t slot = base + static_cast<uint32_t>(__popcll(mask & ((1ull << lane) - 1)));
                if (slot < kSampleFinalKeys)
                {
                    out[slot] = key;
                }
            }
        }
    }
}

/// One slice of 2048 keys (from values[] with their indices, or from earlier candidates) sorted
/// in LDS; its k best go to out[slice * k ...]. Positions past `count` are padded with key 0,
/// below every real key.
__global__ __launch_bounds__(kSelectThreads) void SampleSelectKernel(const float* __restrict__ values,
                                                                     const uint64_t* __restrict__ in, uint32_t count,
                                                                     uint32_t k, uint64_t* __restrict__ out)
{
    __shared__ uint64_t keys[PaddedKeys(kSampleSliceKeys)];
    LoadKeys<kSampleSliceKeys, kSelectThreads>(keys, values, in, blockIdx.x * kSampleSliceKeys, count);
    SortDescending<kSampleSliceKeys, kSelectThreads>(keys);
    for (uint32_t j = threadIdx.x; j < k; j += kSelectThreads)
    {
        out[static_cast<uint64_t>(blockIdx.x) * k + j] = keys[Slot(j)];
    }
}

/// Orders keys[Slot(0..count)) (count <= 512, distinct keys) descending in place: each key's rank
/// is the number of keys above it, so one pass over LDS and two barriers replace a sort network
/// (for the few-times-k candidates a collection leaves). `ranked` holds 512 keys. Ends
/// synchronised.
__device__ void RankDescending(uint64_t* keys, uint64_t* ranked, uint32_t count)
{
    for (uint32_t i = threadIdx.x; i < count; i += kFinalThreads)
    {
        const uint64_t key = keys[Slot(i)];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < count; ++j)
        {
            rank += keys[Slot(j)] > key ? 1u : 0u;
        }
        ranked[rank] = key;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < count; i += kFinalThreads)
    {
        keys[Slot(i)] = ranked[i];
    }
    __syncthreads();
}

/// The k best keys of values[0..count) into keys[Slot(0..k)), descending: rounds that refill
/// every slot past the best k so far with the next values and sort the 4096 (the collection's
/// overflow, when over 4096 keys tie at the top; k <= 256). Ends synchronised.
__device__ void SelectFromValues(uint64_t* keys, const float* __restrict__ values, uint32_t count, uint32_t k)
{
    uint32_t have = 0;
    for (uint32_t base = 0; base < count;)
    {
        const uint32_t take = min(kSampleFinalKeys - have, count - base);
        for (uint32_t j = have + threadIdx.x; j < kSampleFinalKeys; j += kFinalThreads)
        {
            const uint32_t i = base + (j - have);
            keys[Slot(j)] = j - have < take ? SampleKey(values[i], i) : 0;
        }
        __syncthreads();
        SortDescending<kSampleFinalKeys, kFinalThreads>(keys);
        base += take;
        have = k;
    }
}

/// Candidates: the collection (`collected` set; when it overflowed, the whole of values[0..count)
/// is selected from here), else values[] or the last selection round's keys in[0..count).
__global__ __launch_bounds__(kFinalThreads) void SampleFinalKernel(const float* __restrict__ values,
                                                                   const uint64_t* __restrict__ in, uint32_t count,
                                                                   const uint64_t* __restrict__ gathered,
                                                                   const uint32_t* collected, uint32_t k,
                                                                   float temperature, float topP, Mt64State* state,
                                                                   int32_t* token)
{
    __shared__ uint64_t keys[PaddedKeys(kSampleFinalKeys)];
    __shared__ uint64_t ranked[512];
    __shared__ double weight[kSampleMaxTopK];
    __shared__ double share[kSampleMaxTopK];
    __shared__ double totalWeight;
    __shared__ uint64_t old[kMt64Words];
    __shared__ uint64_t fresh[kMt64Words];
    // The engine's index and its next word, requested now so their latency hides under the sort.
    const uint64_t index = state->next;  // the same for every thread: written only at the end
    const bool twist = index >= kMt64Words;
    const uint64_t stored = state->x[twist ? 0 : index];
    bool overflow = false;
    if (collected != nullptr)
    {
        const uint32_t n = *collected;
        if (n <= kSampleFinalKeys)
        {
            values = nullptr;
            in = gathered;
            count = n;
        }
        else
        {
            overflow = true;
        }
    }
    if (overflow)
    {
        SelectFromValues(keys, values, count, k);
    }
    else if (count <= 512)
    {
        LoadKeys<512, kFinalThreads>(keys, values, in, 0, count);
        RankDescending(keys, ranked, count);
    }
    else
    {
        LoadKeys<kSampleFinalKeys, kFinalThreads>(keys, values, in, 0, count);
        SortDescending<kSampleFinalKeys, kFinalThreads>(keys);
    }
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
        weight[j] = exp(static_cast<double>(KeyValue(keys[Slot(j)]) - top));
    }
    // The engine's 312 words are used up: the next generation, computed in three dependent
    // phases (words 0..155 from the old state, 156..310 from the new 0..154, 311 from the new 0
    // and 155), as the sequential twist of the standard engine produces it. The word drawn comes
    // from LDS after a twist, so the kernel never reads back state it wrote.
    if (twist)
    {
        for (uint32_t i = threadIdx.x; i < kMt64Words; i += kFinalThreads)
        {
            old[i] = state->x[i];
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < kMtShift; i += kFinalThreads)
        {
            fresh[i] = MtTwistWord(old[i], old[i + 1], old[i + kMtShift]);
        }
        __syncthreads();
        for (uint32_t i = kMtShift + threadIdx.x; i < kMt64Words - 1; i += kFinalThreads)
        {
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
    // src/Sampler.cpp:64-67: the total, summed in order by one thread; the normalised weights
    // weight[j] / total, each one division, computed side by side.
    if (threadIdx.x == 0)
    {
        double total = 0.0;
        for (uint32_t j = 0; j < k; ++j)
        {
            total += weight[j];
        }
        totalWeight = total;
    }
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < k; j += kFinalThreads)
    {
        share[j] = weight[j] / totalWeight;
    }
    __syncthreads();
    if (threadIdx.x != 0)
    {
        return;
    }
    // src/Sampler.cpp:68-84: the shortest prefix whose normalised mass reaches top-p, and that
    // prefix's mass, each summed in order.
    uint32_t kept = k;
    double running = 0.0;
    for (uint32_t j = 0; j < k; ++j)
    {
        running += share[j];
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
    const uint64_t word = MtTemper(twist ? fresh[0] : stored);
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
    *token = KeyIndex(keys[Slot(chosen)]);
}

size_t Align256(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }
}  // namespace

size_t SampleCandidateKeys(uint32_t vocab, uint32_t k)
{
    return vocab > kSampleFinalKeys ? static_cast<size_t>(CeilDiv(vocab, kSampleSliceKeys)) * k : 1;
}

namespace
{
uint32_t RunK(const SampleConfig& c, uint32_t vocab) { return c.temperature <= 0.0f ? 1 : SampleTopK(c, vocab); }

/// Collection applies above kSampleFinalKeys logits for k up to the number of slice maxima.
bool Collects(uint32_t vocab, uint32_t k) { return vocab > kSampleFinalKeys && k <= kThresholdBlocks; }

struct WorkspaceLayout
{
    size_t counts, candA, candB, blockMax, gathered, collected, total;
};

WorkspaceLayout Layout(uint32_t vocab, uint32_t k)
{
    WorkspaceLayout l{};
    const size_t cand = Align256(SampleCandidateKeys(vocab, k) * sizeof(uint64_t));
    l.counts = 0;
    l.candA = Align256(static_cast<size_t>(vocab) * sizeof(uint32_t));
    l.candB = l.candA + cand;
    l.blockMax = l.candB + cand;
    l.gathered = l.blockMax + Align256(kThresholdBlocks * sizeof(uint64_t));
    l.collected = l.gathered + Align256(kSampleFinalKeys * sizeof(uint64_t));
    l.total = l.collected + 256;
    return l;
}
}  // namespace

size_t SampleWorkspaceBytes(uint32_t vocab, const SampleConfig& c) { return Layout(vocab, RunK(c, vocab)).total; }

SampleWorkspace SampleWorkspaceAt(void* base, uint32_t vocab, const SampleConfig& c)
{
    const WorkspaceLayout l = Layout(vocab, RunK(c, vocab));
    char* p = static_cast<char*>(base);
    SampleWorkspace ws;
    ws.counts = reinterpret_cast<uint32_t*>(p + l.counts);
    ws.candA = reinterpret_cast<uint64_t*>(p + l.candA);
    ws.candB = reinterpret_cast<uint64_t*>(p + l.candB);
    ws.blockMax = reinterpret_cast<uint64_t*>(p + l.blockMax);
    ws.gathered = reinterpret_cast<uint64_t*>(p + l.gathered);
    ws.collected = reinterpret_cast<uint32_t*>(p + l.collected);
    return ws;
}

/// Whether the scale kernel counts the penalty's occurrences itself (its slice fits LDS).
bool PenaltyInScale(uint32_t vocab) { return CeilDiv(vocab, kThresholdBlocks) <= kScaleSliceMax; }

uint32_t SampleLaunches(uint32_t vocab, const SampleConfig& c, bool)
{
    const uint32_t k = RunK(c, vocab);
    const bool collect = Collects(vocab, k);
    uint32_t launches = (c.repeatPenalty != 1.0f && !PenaltyInScale(vocab) ? 1 : 0) + 1 + (collect ? 1 : 0) + 1;
    for (uint32_t count = vocab; !collect && count > kSampleFinalKeys; count = CeilDiv(count, kSampleSliceKeys) * k)
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
    const uint32_t k = RunK(c, vocab);
    const bool penalise = c.repeatPenalty != 1.0f && (position != nullptr || historyCount > 0);
    const bool collect = Collects(vocab, k);
    const bool penaltyInScale = penalise && PenaltyInScale(vocab);
    // The penalty is applied with the division, penalty^d(x) / T, in place or into a separate
    // buffer alike, as the reference leaves its logits: by the scale kernel from counts in LDS,
    // or (long slices) by a Penalty kernel first that finishes and marks its tokens.
    if (penalise && !penaltyInScale)
    {
        hipLaunchKernelGGL(SamplePenaltyKernel, dim3(1), dim3(kPenaltyThreads), 0, s, src, dst, vocab, history,
                           position, historyCount, c.repeatLastN, c.repeatPenalty, c.temperature, ws.counts);
    }
    const PenaltyWindow window{history, position, historyCount, c.repeatLastN, c.repeatPenalty};
    hipLaunchKernelGGL(SampleScaleKernel, dim3(kThresholdBlocks), dim3(kScaleThreads), 0, s, src, dst, vocab,
                       c.temperature, penalise && !penaltyInScale ? ws.counts : nullptr, penaltyInScale, window,
                       collect ? ws.blockMax : nullptr, ws.collected);
    if (collect)
    {
        hipLaunchKernelGGL(SampleCollectKernel, dim3(kThresholdBlocks), dim3(kScaleThreads), 0, s, dst, vocab, k,
                           ws.blockMax, ws.gathered, ws.collected);
    }
    // Without a collection: rounds of slice sorts until the final workgroup can hold every
    // candidate; each round keeps k of 2048 keys per slice (k <= 1024), so the count at least
    // halves. A collection that overflows is finished by the final workgroup from dst itself.
    const float* values = dst;
    const uint64_t* in = nullptr;
    uint32_t count = vocab;
    uint64_t* out = ws.candA;
    while (!collect && count > kSampleFinalKeys)
    {
        const uint32_t slices = CeilDiv(count, kSampleSliceKeys);
        hipLaunchKernelGGL(SampleSelectKernel, dim3(slices), dim3(kSelectThreads), 0, s, values, in, count, k, out);
        count = slices * k;
        values = nullptr;
        in = out;
        out = out == ws.candA ? ws.candB : ws.candA;
    }
    hipLaunchKernelGGL(SampleFinalKernel, dim3(1), dim3(kFinalThreads), 0, s, values, in, count,
                       collect ? ws.gathered : nullptr, collect ? ws.collected : nullptr, k, c.temperature, c.topP,
                       state, token);
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
