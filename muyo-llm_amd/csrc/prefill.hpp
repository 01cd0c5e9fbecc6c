// Batched prefill: a prompt of many tokens through every layer at once, as GEMMs on the matrix
// cores and a causal flash attention, instead of one decode step per prompt token.
//
// Activations enter the matrix cores as two f16 planes: hi = x with its 13 low mantissa bits
// cleared (exact in f16) and lo = f16(x - hi). The weights are exact in f16, so W.hi + W.lo with
// f32 accumulation carries ~21 bits of each activation, close to the f32 path that feeds the
// prompt one token at a time.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace muyo
{
/// Rows (prompt tokens) of one prefill pass; longer prompts run in passes of at most this many.
constexpr uint32_t kPrefillRows = 2048;

/// x[m] = f32(table[tokens[m]]) for m < rows; history[pos0 + m] = tokens[m] where it fits.
hipError_t LaunchEmbedRows(hipStream_t s, const uint16_t* table, const int32_t* tokens, uint32_t rows,
                           uint32_t hidden, float* x, int32_t* history, int32_t pos0, uint32_t historyCap);

/// y = (x * rsqrt(mean(x^2) + eps)) * w per row of `cols`, written as f16 hi/lo planes [rows][cols].
hipError_t LaunchRmsNormSplit(hipStream_t s, const float* x, const float* w, uint32_t rows, uint32_t cols, float eps,
                              uint16_t* hi, uint16_t* lo);

/// hi/lo planes of a plain f32 matrix (no norm): count values, count % 4 == 0.
hipError_t LaunchSplitF32(hipStream_t s, const float* x, uint64_t count, uint16_t* hi, uint16_t* lo);

/// Most K splits of a prefill GEMM.
constexpr uint32_t kMaxGemmSplits = 4;
constexpr uint32_t kAttnMaxChunks = 8;    // key chunks a split prefill-attention query tile takes at most
constexpr uint32_t kAttnMaxItems = 512;   // work items of one split attention launch (64 tiles x 8)

/// Floats of the workspace the split prefill attention needs for `rows` queries.
inline size_t PrefillAttentionWorkspaceFloats(uint32_t rows, uint32_t heads, uint32_t headDim)
{
    return static_cast<size_t>(kAttnMaxChunks) * rows * heads * (headDim + 2);
}

/// K splits for a GEMM of this shape: more than one when its output tiles alone leave most SIMDs
/// without a wave (the 0.5B shape's q|k|v, o_proj and down at 2048 rows).
uint32_t GemmSplits(uint32_t rows, uint32_t n, uint32_t k);

/// out[m][n] = sum_k (ahi + alo)[m][k] * w[n][k] + bias[n] (bias may be null) + residual[m][n]
/// (residual may be null). A is [rows][k] (two planes), W is [n][k] f16, out is [rows][n] f32.
/// With splits > 1 the K range is split and each split's raw sums go to plane z of `partial`
/// ([splits][rows][n]); out, bias and residual are then left to the consumer
/// (LaunchReduceRmsNormSplit, LaunchRopeSplitAppend).
hipError_t LaunchGemmSplit(hipStream_t s, const uint16_t* ahi, const uint16_t* alo, const uint16_t* w,
                           const float* bias, const float* residual, float* out, uint32_t rows, uint32_t n,
                           uint32_t k, float* partial = nullptr, uint32_t splits = 1);

/// x = residual + the sum of a split GEMM's planes (split order), stored; then, with w, its rows'
/// rms_norm as f16 hi/lo planes as LaunchRmsNormSplit.
hipError_t LaunchReduceRmsNormSplit(hipStream_t s, const float* residual, const float* partial, uint32_t splits,
                                    float* x, const float* w, uint32_t rows, uint32_t cols, float eps, uint16_t* hi,
                                    uint16_t* lo);

/// h[m][f] = silu(g) * u with g = A.gate[f], u = A.up[f] (same split product), written as f16
/// hi/lo planes [rows][ffn].
hipError_t LaunchGemmSwiGlu(hipStream_t s, const uint16_t* ahi, const uint16_t* alo, const uint16_t* wgate,
                            const uint16_t* wup, uint16_t* hhi, uint16_t* hlo, uint32_t rows, uint32_t ffn,
                            uint32_t k);

/// From the QKV projection rows [rows][(heads + 2 kvHeads) * headDim] (bias included): rope_neox
/// on q and k at positions pos0 + m, q as hi/lo planes [rows][heads * headDim], k and v appended
/// to the fp16 caches [kvHeads][maxSeq][headDim] at rows pos0 + m.
/// With splits > 1, qkv is a split GEMM's partial planes and bias its bias.
hipError_t LaunchRopeSplitAppend(hipStream_t s, const float* qkv, uint32_t rows, int32_t pos0, uint32_t heads,
                                 uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, const float* ropePow,
                                 uint16_t* qhi, uint16_t* qlo, uint16_t* kcache, uint16_t* vcache,
                                 uint32_t splits = 1, const float* bias = nullptr);

/// Causal attention of the queries at positions pos0 + m (m < rows) over cache rows 0..pos0 + m:
/// out[m][h * headDim + c] as hi/lo planes [rows][heads * headDim]. With a workspace of at least
/// PrefillAttentionWorkspaceFloats floats, query tiles with long key ranges are split into key
/// chunks run by separate workgroups and merged by a second kernel.
hipError_t LaunchPrefillAttention(hipStream_t s, const uint16_t* qhi, const uint16_t* qlo, const uint16_t* kcache,
                                  const uint16_t* vcache, uint16_t* ohi, uint16_t* olo, uint32_t rows, int32_t pos0,
                                  uint32_t heads, uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, float scale,
                                  float* workspace = nullptr, size_t workspaceFloats = 0);
}  // namespace muyo
