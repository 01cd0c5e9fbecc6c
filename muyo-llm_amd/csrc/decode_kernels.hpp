// Fused decode-step kernels and their host-side launchers.
//
// No kernel communicates across its own workgroups (on gfx950 an agent-scope release fence
// serialises device-wide, ~60 ns per workgroup): every cross-workgroup reduction is split at a
// kernel boundary. The LM head leaves per-workgroup (max, index) partials that the next step's
// first kernel (or a finalize kernel) reduces; attention leaves per-chunk softmax partials that
// the o_proj kernel's prologue combines (all of them, or per kv group, leaving one partial sum per
// group that gate/up's prologue adds up; otherwise a small merge kernel).
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
    const float* ropePow;  // device table of thetaScale^j, j < headDim / 2 (powf on the host)
    float attnScale;   // 1/sqrt(headDim)
    uint32_t attnChunks;  // most attention chunks per kv head (kMaxAttnChunks or kMergeAttnChunks)
};

/// Device-resident state of a generation run. `token` and `position` are those of the step
/// being decoded; BeginStep derives them at the start of every step.
struct DecodeState
{
    int32_t token;
    int32_t position;
    int32_t start;  // cache row of the run's first step
    uint32_t step;  // steps begun in this run
};

/// Scratch shared by the kernels of one decoder (sized for its model).
struct DecodeScratch
{
    float* attnMax;     // [kvHeads][gridChunks][group]        chunk-local softmax max (log2 units)
    float* attnSum;     // [kvHeads][gridChunks][group]        chunk-local softmax sum
    float* attnAcc;     // [kvHeads][gridChunks][group][hd]    chunk-local P.V (relative to the max)
    float* argValue;    // [kArgMaxBlocks]                 per-workgroup LM-head max
    int32_t* argIndex;  // [kArgMaxBlocks]                 and its (lowest) index
    int32_t* sampled;   // the sampler's token; null: the next token is the argmax of the partials
    int32_t* history;   // [historyCap]                    the token embedded at each position
    uint32_t historyCap;
};

constexpr uint32_t kArgMaxBlocks = 2048;
/// Partial vectors the fused feed-forward kernel adds its down projection into (atomically); the
/// layer's output is their sum. Fewer vectors mean more atomic adds to each address, which
/// serialise: at the 0.5B shape the kernel takes 7.7 us with 8, 8.3 with 4, 12.7 with 1.
constexpr uint32_t kResidualParts = 8;
constexpr uint32_t kMaxAttnChunks = 16;    // attention chunks per kv head, at most
constexpr uint32_t kMergeAttnChunks = 8;   // the same when o_proj's prologue merges the partials
constexpr uint32_t kShortAttnChunks = 4;   // the same while every chunk's keys fit its first round
constexpr uint32_t kMaxSeq = 32768;

/// Keys one attention workgroup processes side by side: its 256 lanes hold one 16-byte slice of
/// a cache row each (headDim 64 -> 32 keys, 128 -> 16 keys).
__host__ __device__ inline uint32_t AttnSlices(uint32_t headDim) { return 2048u / headDim; }

/// Chunks per kv head (the attention grid's x): min(maxChunks, ceil(maxSeq / slices)). Blocks of
/// `slices` consecutive keys are dealt to the chunks round-robin.
inline uint32_t AttnGridChunks(uint32_t maxSeq, uint32_t headDim, uint32_t maxChunks)
{
    const uint32_t bySlices = (maxSeq + AttnSlices(headDim) - 1) / AttnSlices(headDim);
    return bySlices < maxChunks ? bySlices : maxChunks;
}

/// Key blocks an attention chunk requests at entry, before the position is known.
constexpr uint32_t kAttnBlocksPerRound = 8;

/// Keys kShortAttnChunks chunks cover in their first round: a step at a position below this
/// needs no second round with the short grid.
inline uint32_t ShortAttnKeys(uint32_t headDim) { return kShortAttnChunks * kAttnBlocksPerRound * AttnSlices(headDim); }

/// Grid of a fused GEMV launch: `blocks` workgroups; when blocks * unitsPerBlock covers the
/// units, workgroup i owns units [i * unitsPerBlock, (i + 1) * unitsPerBlock).
struct GemvShape
{
    uint32_t blocks;
    uint32_t unitsPerBlock;
};

/// Workgroups of the LM-head kernel (each leaves one argmax partial).
uint32_t LmHeadBlocks(const DecodeDims& dims);

/// True when o_proj can merge the attention partials in its prologue (small models); such a
/// decoder runs attention with at most kMergeAttnChunks chunks per kv head.
bool MergeInOProj(const DecodeDims& dims);

// Launchers. All return hipGetLastError() after the launch.

/// The state of a run whose next step embeds `token` at `position`; `step` 1 marks that step as
/// already run (a prefill's last position), so Finalize files its successor as id 0.
hipError_t LaunchSetState(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, int32_t token,
                          int32_t position, uint32_t argBlocks, uint32_t step = 0);

/// `zero` (optional): a [hidden] vector cleared at the same time (the first layer's grouped
/// o_proj target).
hipError_t LaunchBeginStep(hipStream_t s, const uint16_t* table, DecodeState* state, const DecodeScratch& scratch,
                           uint32_t argBlocks, float* x, int32_t* ids, uint32_t idsCap, uint32_t hidden,
                           uint32_t vocab, float* zero = nullptr);

hipError_t LaunchFinalize(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, uint32_t argBlocks,
                          int32_t* ids, uint32_t idsCap);

/// `xParts` 1: x is the hidden state; kResidualParts: x holds that many partial vectors (the
/// fused feed-forward kernel's output) whose sum is the hidden state.
hipError_t LaunchQkvRopeAppend(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                               const uint16_t* wqkv, const float* bias, const DecodeState* state, float* qOut,
                               uint16_t* kcache, uint16_t* vcache, uint32_t xParts = 1);

hipError_t LaunchAttention(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                           const uint16_t* vcache, const int32_t* position, const DecodeScratch& scratch);

hipError_t LaunchAttentionMerge(hipStream_t s, const DecodeDims& dims, const DecodeScratch& scratch, float* out);

/// out = residual + W_o . merged attention. `residualParts` 1 or kResidualParts (as
/// LaunchQkvRopeAppend's xParts); `parts`, when set, also receives out as the partial vectors
/// the fused feed-forward kernel adds into: parts[0] = out, parts[1..] = 0.
hipError_t LaunchOProjMerged(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const DecodeScratch& scratch,
                             const float* residual, float* out, uint32_t residualParts = 1, float* parts = nullptr);

/// The same with the attention output already merged (`attn`, heads * headDim floats).
hipError_t LaunchOProjPlain(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const float* attn,
                            const float* residual, float* out, uint32_t residualParts, float* parts);

/// True when the decoder runs gate/up, swiglu and down as one launch (FfnFused): a hidden size
/// of at most 1024 and o_proj not split by kv group.
bool FfnFusable(const DecodeDims& dims);

/// The feed-forward block in one launch: rms_norm(x) . gate/up,
/// swiglu, and the down projection from its transposed weights downT [ffn][hidden], added with
/// atomics into `parts` ([kResidualParts][hidden], holding the residual as o_proj left it). The
/// order of the atomic adds varies from run to run, so the sum does in its last bits.
hipError_t LaunchFfnFused(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                          const uint16_t* wgate, const uint16_t* wup, const uint16_t* downT, float* parts);

/// dst[c][r] = src[r][c] for an fp16 matrix of `rows` x `cols`.
hipError_t LaunchTransposeF16(hipStream_t s, const uint16_t* src, uint16_t* dst, uint32_t rows, uint32_t cols);

/// True when o_proj runs split by kv group with the attention merge in its prologue (models
/// whose q dim is too wide for MergeInOProj but whose group is at most 1024 channels wide).
bool OProjInGroups(const DecodeDims& dims);

/// o_proj per kv group: out[row] += (g == 0 ? residual[row] : 0) + W_o[row, group g's columns]
/// . merged attention of group g, one atomic add per group and row into `out`, which must hold
/// zeros. The order of the kvHeads adds varies from run to run, so the sum does in its last bits.
hipError_t LaunchOProjGroups(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const DecodeScratch& scratch,
                             const float* residual, float* out);

hipError_t LaunchMatVecResidual(hipStream_t s, const uint16_t* w, const float* x, const float* residual, float* out,
                                uint32_t rows, uint32_t cols);

/// LaunchMatVecResidual that also stores zeros to zero[0..rows) (the next layer's grouped o_proj
/// target).
hipError_t LaunchMatVecResidualZero(hipStream_t s, const uint16_t* w, const float* x, const float* residual,
                                    float* out, float* zero, uint32_t rows, uint32_t cols);

/// out[row] = (W[row] . x + bias0[row]) + bias1[row] (null biases skipped) on the fused GEMV's
/// launch shapes: W fp16 [rows][cols] with 16-byte aligned rows, x 16-byte aligned, cols % 8 == 0.
hipError_t LaunchMatVecBias(hipStream_t s, const uint16_t* w, const float* x, const float* bias0, const float* bias1,
                            float* out, uint32_t rows, uint32_t cols);

hipError_t LaunchGateUpSwiGlu(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* wgate, const uint16_t* wup, float* act);

hipError_t LaunchLmHeadArgMax(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* table, float* logits, const DecodeScratch& scratch);

/// Rope q/k and append k/v (fp16) at the position's cache row, from separate q/k/v vectors.
hipError_t LaunchRopeAppend(hipStream_t s, const float* q, const float* k, const float* v, float* qOut,
                            uint16_t* kcache, uint16_t* vcache, const int32_t* position, uint32_t heads,
                            uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, float thetaScale);
}  // namespace muyo
