// Fused decode-step kernels (one Qwen2 layer = five launches) and their host-side launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace muyo
{
/// Shapes and scalars every fused kernel of one model needs.
struct DecodeDims
{
    uint32_t hidden;
    uint32_t ffn;
    uint32_t heads;
    uint32_t kvHeads;
    uint32_t headDim;
    uint32_t vocab;
    uint32_t maxSeq;
    float eps;
    float thetaScale;  // ropeBase^(-2/headDim), computed in f32 on the host
    float attnScale;   // 1/sqrt(headDim)
};

/// Device-resident per-step state (token and position of the step being decoded).
struct DecodeState
{
    int32_t token;
    int32_t position;
    uint32_t step;   // index into the generated-ids ring
    uint32_t pad;
};

/// Scratch the split attention and the argmax need (owned by the caller, zeroed once).
struct DecodeScratch
{
    float* attnMax;        // [kvHeads][chunks][group]
    float* attnSum;        // [kvHeads][chunks][group]
    float* attnAcc;        // [kvHeads][chunks][group][headDim]
    uint32_t* attnCount;   // [kvHeads]   arrival counters, reset by the last block
    float* argValue;       // [argBlocks]
    int32_t* argIndex;     // [argBlocks]
    uint32_t* argCount;    // [1]
};

constexpr uint32_t kAttnChunk = 64;     // keys per attention block
constexpr uint32_t kArgMaxBlocks = 1024;  // LM-head grid cap (partials for the argmax)

inline uint32_t AttnChunks(uint32_t maxSeq) { return (maxSeq + kAttnChunk - 1) / kAttnChunk; }

// Launchers. All return hipGetLastError() after the launch.
hipError_t LaunchEmbed(hipStream_t s, const uint16_t* table, const DecodeState* state, float* x, uint32_t hidden,
                       uint32_t vocab);

hipError_t LaunchQkvRopeAppend(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                               const uint16_t* wqkv, const float* bias, const DecodeState* state, float* qOut,
                               uint16_t* kcache, uint16_t* vcache);

hipError_t LaunchAttention(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                           const uint16_t* vcache, const int32_t* position, float* out, const DecodeScratch& scratch);

hipError_t LaunchMatVecResidual(hipStream_t s, const uint16_t* w, const float* x, const float* residual, float* out,
                                uint32_t rows, uint32_t cols);

hipError_t LaunchGateUpSwiGlu(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* wgate, const uint16_t* wup, float* act);

hipError_t LaunchLmHeadArgMax(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* table, float* logits, DecodeState* state, int32_t* ids, uint32_t idsCap,
                              const DecodeScratch& scratch);

/// Rope q/k and append k/v (fp16) at the position's cache row, from separate q/k/v vectors.
hipError_t LaunchRopeAppend(hipStream_t s, const float* q, const float* k, const float* v, float* qOut,
                            uint16_t* kcache, uint16_t* vcache, const int32_t* position, uint32_t heads,
                            uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, float thetaScale);
}  // namespace muyo
