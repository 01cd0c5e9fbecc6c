// The persistent decode step: one cooperative launch per token that runs every layer, the LM head
// and the greedy bookkeeping, its workgroups handing activations to each other through device
// memory instead of kernel boundaries.
//
// Hand-offs use self-validating 8-byte packets (f32 value in the low word, a per-write epoch in
// the high word), stored and loaded with agent-scope relaxed atomics: a consumer keeps loading a
// packet until it carries the epoch it expects, so no fence or flag is needed. Each workgroup's
// first wave does all the waiting (the "poller") and hands what arrived to the other seven waves
// through LDS at the one barrier between phases; those waves only compute, and request the next
// phase's weights before that barrier, so the weights stream while the hand-off is in flight.
// Every wait is bounded: on giving up, a workgroup records which wait failed and raises an abort
// word that makes every other wait return at once, so the grid always drains.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode_kernels.hpp"

namespace muyo
{
/// One layer's tensors as the persistent step reads them.
struct StepLayer
{
    const float* attnNorm;  // [hidden]
    const uint16_t* qkv;    // [(heads + 2 kvHeads) * headDim][hidden]
    const float* qkvBias;   // [(heads + 2 kvHeads) * headDim]
    const uint16_t* wo;     // [hidden][heads * headDim]
    const float* ffnNorm;   // [hidden]
    const uint16_t* gate;   // [ffn][hidden]
    const uint16_t* up;     // [ffn][hidden]
    const uint16_t* downT;  // [ffn + 3][hidden]: FFN_DOWN transposed (a column of it is a row), 3 rows of slack
    uint16_t* kcache;       // [kvHeads][maxSeq][headDim]
    uint16_t* vcache;       // [kvHeads][maxSeq][headDim]
};

/// Words of the step's control block (device memory, zeroed at creation).
enum StepControl : uint32_t
{
    kStepError = 0,  // 0, or 1 + the index of the first wait that gave up
    kStepAbort = 1,  // nonzero: every wait returns at once
    kStepEpoch = 2,  // epoch of this step's first hand-off (advanced by each step)
    kStepControlWords = 4,
};

/// Everything one persistent step reads; the decoder fills it once.
struct StepPlan
{
    uint32_t layers, hidden, ffn, heads, kvHeads, headDim, vocab, maxSeq;
    float eps, attnScale;
    const float* ropePow;       // [headDim / 2]: thetaScale^j
    const StepLayer* layer;     // device array [layers]
    const uint16_t* embedding;  // [vocab][hidden]
    const uint16_t* head;       // LM head table [vocab][hidden] (the embedding when tied)
    const float* outputNorm;    // [hidden]
    float* logits;              // [vocab]
    DecodeState* state;
    float* argValue;            // [grid] per-workgroup LM-head maxima
    int32_t* argIndex;          // [grid] and their lowest indices
    const int32_t* sampled;     // the sampler's token, or null for greedy
    int32_t* history;
    uint32_t historyCap;
    int32_t* ids;
    uint32_t idsCap;
    uint64_t* packets;          // hand-off arena: two parities of the regions below
    uint32_t* control;          // StepControl words
    uint32_t spinLimit;         // polls per wait before giving up

    // Layout, filled by StepPlanLayout.
    uint32_t grid;              // workgroups, one per CU, all resident (cooperative launch)
    uint32_t chunks;            // attention chunks per kv head
    uint32_t qkvBlocks, attnUnits, rowBlocks, ffnPerGroup;
    uint32_t roleQ, roleA, roleO, roleR;  // first workgroup of each role
    uint32_t offX, offQkv, offPart, offMid, offDown, parity;  // packet offsets; parity = region size
};

/// Most layers the step takes (its layer table lives in LDS).
constexpr uint32_t kStepMaxLayers = 64;

/// Rows of slack the step may read past the end of a layer's value cache (an attention block).
constexpr uint32_t kStepCacheSlackRows = 64;

/// Why the persistent step cannot run this shape (null when it can).
const char* StepUnsupported(uint32_t hidden, uint32_t ffn, uint32_t heads, uint32_t kvHeads, uint32_t headDim,
                            uint32_t grid);

/// Fills the layout fields of `plan` for `grid` workgroups; returns the packets the arena needs.
size_t StepPlanLayout(StepPlan& plan, uint32_t grid);

/// Workgroups of the step kernel one CU holds at once (1 when it fits).
uint32_t StepResidentPerCu();

/// One step on `s` (a cooperative launch of plan.grid workgroups).
hipError_t LaunchStep(hipStream_t s, const StepPlan& plan);

/// dst[c][r] = src[r][c] for a rows x cols fp16 matrix.
hipError_t LaunchTranspose16(hipStream_t s, const uint16_t* src, uint16_t* dst, uint32_t rows, uint32_t cols);
}  // namespace muyo
