// Fused decode-step kernels for gfx950.
//
// One step (the reference records 18 nodes per layer, src/FullModel.cpp:227-498):
//   BeginStep      : greedy id of the previous step from the LM head's per-workgroup partials,
//                    step bookkeeping (position, generated-id ring), embedding row -> f32 x
//   per layer:
//   QkvRopeAppend  : rms_norm prologue -> fused q|k|v GEMV + bias -> NeoX rope of q and k ->
//                    q to a buffer, k and v appended as fp16 at the position's cache row
//   Attention      : one workgroup per (256-key chunk, kv head); 64-key tiles of the fp16 cache
//                    staged in LDS (next tile prefetched), online softmax, P.V for the whole GQA
//                    group; chunk partials (max, sum, P.V) to scratch
//   [AttentionMerge: combine the chunk partials, when o_proj does not do it itself]
//   OProj          : [merge prologue] o_proj GEMV + residual add
//   GateUpSwiGlu   : rms_norm prologue -> gate and up GEMV rows -> silu(g)*u
//   Down           : down GEMV + residual add
//   LmHeadArgMax   : final rms_norm prologue -> tied LM head -> logits + per-workgroup argmax
//
// GEMV core (gemv_core.hpp): the activation is staged once per workgroup in LDS; a wave64
// splits into segments of LPR lanes, each segment streaming one fp16 weight row in 16-byte
// chunks with all of a lane's loads in flight at once; the first batch is requested before the
// activation is staged and the next row's batch before the current row's reduction.
#include <algorithm>

#include "common.hpp"
#include "decode_kernels.hpp"
#include "gemv_core.hpp"

namespace muyo
{
namespace
{
constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr uint32_t kMaxLds = 160 * 1024;
constexpr int kStageVec = 8;           // float4 per thread per staging round (rows <= 8192 floats)
constexpr int kMaxGroup = 8;           // query heads per kv head
constexpr uint32_t kBlocksPerCu = 4;   // GEMV grid cap: enough waves in flight, no second round
constexpr uint32_t kMergeChunks = 8;   // chunks the o_proj prologue merges (max_seq <= 2048)
constexpr uint32_t kMergeItems = 4;    // q channels per thread in that prologue (q dim <= 1024)

uint32_t GemvBlockCap()
{
    static uint32_t cap = 0;
    if (cap == 0)
    {
        int device = 0;
        int cus = 0;
        if (hipGetDevice(&device) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
        {
            cus = 256;
        }
        cap = static_cast<uint32_t>(cus) * kBlocksPerCu;
    }
    return cap;
}

// ------------------------------------------------------------------------------------------------
// Activation staging policies (each fills the LDS split layout and ends synchronised).

struct PlainStage
{
    const float* x;
    __device__ void Run(float4* xs, uint32_t n) const { StageSplit<kBlock, kStageVec, false>(x, nullptr, n, 0.0f, xs); }
};

struct NormStage
{
    const float* x;
    const float* w;
    float eps;
    __device__ void Run(float4* xs, uint32_t n) const { StageSplit<kBlock, kStageVec, true>(x, w, n, eps, xs); }
};

/// The attention output, merged from the chunk partials: out[h][d] = sum_c e^(m_c - M) acc_c /
/// sum_c e^(m_c - M) l_c (flash-decoding's combine).
struct MergeStage
{
    const int32_t* position;
    const float* attnMax;
    const float* attnSum;
    const float* attnAcc;
    uint32_t heads, group, headDim, maxChunks;

    __device__ void Run(float4* xs, uint32_t n) const
    {
        __shared__ float chunkMax[kBlock];
        __shared__ float chunkSum[kBlock];
        __shared__ float weight[kBlock];
        // Positions outside the cache are rejected on the host; clamping keeps every read in bounds.
        const uint32_t pos = static_cast<uint32_t>(max(*position, 0));
        const uint32_t chunks = min((pos + kAttnChunk) / kAttnChunk, maxChunks);
        const uint32_t nchunks = n / 8;
        // Per-(head, chunk) max and sum, and this thread's accumulators, all requested at once.
        if (threadIdx.x < heads * chunks)
        {
            const uint32_t h = threadIdx.x / chunks;
            const uint32_t c = threadIdx.x % chunks;
            const uint64_t slot = (static_cast<uint64_t>(h / group) * maxChunks + c) * group + h % group;
            chunkMax[threadIdx.x] = attnMax[slot];
            chunkSum[threadIdx.x] = attnSum[slot];
        }
        float acc[kMergeItems][kMergeChunks];
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k)
        {
            const uint32_t item = min(threadIdx.x + k * kBlock, n - 1);
            const uint32_t h = item / headDim;
            const uint32_t d = item % headDim;
#pragma unroll
            for (uint32_t c = 0; c < kMergeChunks; ++c)
            {
                const uint32_t cc = min(c, chunks - 1);
                const uint64_t slot = (static_cast<uint64_t>(h / group) * maxChunks + cc) * group + h % group;
                acc[k][c] = attnAcc[slot * headDim + d];
            }
        }
        __syncthreads();
        if (threadIdx.x < heads)
        {
            const uint32_t h = threadIdx.x;
            float m = -INFINITY;
            for (uint32_t c = 0; c < chunks; ++c)
            {
                m = fmaxf(m, chunkMax[h * chunks + c]);
            }
            float den = 0.0f;
            for (uint32_t c = 0; c < chunks; ++c)
            {
                const float e = expf(chunkMax[h * chunks + c] - m);
                weight[h * chunks + c] = e;
                den = fmaf(e, chunkSum[h * chunks + c], den);
            }
            const float inv = 1.0f / den;
            for (uint32_t c = 0; c < chunks; ++c)
            {
                weight[h * chunks + c] *= inv;
            }
        }
        __syncthreads();
        float* flat = reinterpret_cast<float*>(xs);
#pragma unroll
        for (uint32_t k = 0; k < kMergeItems; ++k)
        {
            const uint32_t item = threadIdx.x + k * kBlock;
            if (item < n)
            {
                const uint32_t h = item / headDim;
                float out = 0.0f;
#pragma unroll
                for (uint32_t c = 0; c < kMergeChunks; ++c)
                {
                    if (c < chunks)
                    {
                        out = fmaf(weight[h * chunks + c], acc[k][c], out);
                    }
                }
                flat[SplitSlot(item, nchunks)] = out;
            }
        }
        __syncthreads();
    }
};

// ------------------------------------------------------------------------------------------------
// Fused GEMV: units of kNr rows, a staging policy, an epilogue per unit, an optional block tail.

template <int kLpr, int kCpl, int kNr, class Stage, class Epi>
__global__ __launch_bounds__(kBlock) void FusedMatVec(uint32_t cols, Stage stage, Epi epi)
{
    extern __shared__ float4 xs[];
    const uint32_t nchunks = cols / 8;
    constexpr int kSegs = kWave / kLpr;
    constexpr int kUnits = kSegs / kNr;
    static_assert(kUnits >= 1, "a wave must hold at least one unit");
    const int lane = threadIdx.x & (kWave - 1);
    const int segment = lane / kLpr;
    const uint32_t lir = lane % kLpr;
    const int unitInWave = segment / kNr;
    const int part = segment % kNr;
    const uint32_t wave = blockIdx.x * kWaves + threadIdx.x / kWave;
    const uint32_t stride = gridDim.x * kWaves * kUnits;
    const uint32_t units = epi.Units();

    // Weights do not depend on the activation: start streaming them before it is staged.
    uint32_t first = wave * kUnits;
    half8 w[kCpl];
    if (first + unitInWave < units)
    {
        LoadBatch<kLpr, kCpl>(epi.Row(first + unitInWave, part), 0, nchunks, lir, w);
    }
    stage.Run(xs, cols);
    const float4* lo = xs;
    const float4* hi = xs + nchunks;

    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    for (; first < units; first += stride)
    {
        const uint32_t unit = first + unitInWave;
        const bool valid = unit < units;
        float dot = 0.0f;
        if (valid)
        {
            dot = RowDot<kLpr, kCpl>(epi.Row(unit, part), nchunks, lir, w, lo, hi);
        }
        // The next unit's first batch goes out before this unit's reduction and epilogue.
        const uint32_t next = first + stride + unitInWave;
        if (next < units)
        {
            LoadBatch<kLpr, kCpl>(epi.Row(next, part), 0, nchunks, lir, w);
        }
        dot = GroupSum<kLpr>(dot);
        float sums[kNr];
#pragma unroll
        for (int k = 0; k < kNr; ++k)
        {
            sums[k] = __shfl(dot, (unitInWave * kNr + k) * kLpr, kWave);
        }
        if (valid && part == 0 && lir == 0)
        {
            epi.Finish(unit, sums, bestValue, bestIndex);
        }
    }
    epi.Tail(bestValue, bestIndex);
}

// ------------------------------------------------------------------------------------------------
// Epilogues.

struct QkvEpi
{
    const uint16_t* w;
    const float* bias;
    const DecodeState* state;
    float* qOut;
    uint16_t* kcache;
    uint16_t* vcache;
    uint32_t cols, heads, kvHeads, headDim, maxSeq;
    float thetaScale;

    __device__ uint32_t Units() const { return (heads + 2 * kvHeads) * headDim / 2; }

    /// Rope units pair rows (j, j + hd/2) of one q or k head; value units pair adjacent rows.
    __device__ uint32_t RowOf(uint32_t unit, int part) const
    {
        const uint32_t half = headDim / 2;
        const uint32_t ropeUnits = (heads + kvHeads) * half;
        if (unit < ropeUnits)
        {
            return (unit / half) * headDim + unit % half + part * half;
        }
        return (heads + kvHeads) * headDim + 2 * (unit - ropeUnits) + part;
    }

    __device__ const uint16_t* Row(uint32_t unit, int part) const
    {
        return w + static_cast<uint64_t>(RowOf(unit, part)) * cols;
    }

    __device__ void Finish(uint32_t unit, const float* s, float&, int32_t&) const
    {
        const uint32_t half = headDim / 2;
        const uint32_t ropeUnits = (heads + kvHeads) * half;
        const int32_t pos = state->position;
        const float s0 = s[0] + bias[RowOf(unit, 0)];
        const float s1 = s[1] + bias[RowOf(unit, 1)];
        if (unit < ropeUnits)
        {
            // rope_neox (rope_funcs.glsl:76-114): theta = pos * theta_scale^j, pair (j, j + hd/2).
            const uint32_t head = unit / half;
            const uint32_t j = unit % half;
            const float theta = static_cast<float>(pos) * powf(thetaScale, static_cast<float>(j));
            const float c = cosf(theta);
            const float sn = sinf(theta);
            const float o0 = s0 * c - s1 * sn;
            const float o1 = s0 * sn + s1 * c;
            if (head < heads)
            {
                qOut[head * headDim + j] = o0;
                qOut[head * headDim + j + half] = o1;
            }
            else if (pos >= 0 && static_cast<uint32_t>(pos) < maxSeq)
            {
                const uint64_t base = (static_cast<uint64_t>(head - heads) * maxSeq + pos) * headDim;
                kcache[base + j] = FloatToHalfBits(o0);
                kcache[base + j + half] = FloatToHalfBits(o1);
            }
        }
        else if (pos >= 0 && static_cast<uint32_t>(pos) < maxSeq)
        {
            const uint32_t channel = 2 * (unit - ropeUnits);  // within kvHeads * headDim
            const uint32_t g = channel / headDim;
            const uint64_t base = (static_cast<uint64_t>(g) * maxSeq + pos) * headDim + channel % headDim;
            vcache[base] = FloatToHalfBits(s0);
            vcache[base + 1] = FloatToHalfBits(s1);
        }
    }

    __device__ void Tail(float, int32_t) const {}
};

struct ResidualEpi
{
    const uint16_t* w;
    const float* residual;
    float* out;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return w + static_cast<uint64_t>(unit) * cols; }
    __device__ void Finish(uint32_t unit, const float* s, float&, int32_t&) const { out[unit] = residual[unit] + s[0]; }
    __device__ void Tail(float, int32_t) const {}
};

struct GateUpEpi
{
    const uint16_t* gate;
    const uint16_t* up;
    float* act;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int part) const
    {
        return (part == 0 ? gate : up) + static_cast<uint64_t>(unit) * cols;
    }
    __device__ void Finish(uint32_t unit, const float* s, float&, int32_t&) const
    {
        act[unit] = s[0] / (1.0f + expf(-s[0])) * s[1];  // swiglu.comp's op
    }
    __device__ void Tail(float, int32_t) const {}
};

/// Better (value, index) under "larger value, then lower index" (the host greedy scan's rule).
__device__ __forceinline__ bool Better(float v, int32_t i, float bestV, int32_t bestI)
{
    return v > bestV || (v == bestV && i < bestI);
}

/// Reduce (value, index) over a 256-thread block; the result lands in thread 0.
__device__ __forceinline__ void BlockArgMax(float& value, int32_t& index)
{
    __shared__ float waveValue[kWaves];
    __shared__ int32_t waveIndex[kWaves];
    GroupArgMax<kWave>(value, index);
    if ((threadIdx.x & (kWave - 1)) == 0)
    {
        waveValue[threadIdx.x / kWave] = value;
        waveIndex[threadIdx.x / kWave] = index;
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        for (int k = 1; k < kWaves; ++k)
        {
            if (Better(waveValue[k], waveIndex[k], value, index))
            {
                value = waveValue[k];
                index = waveIndex[k];
            }
        }
    }
}

struct LmHeadEpi
{
    const uint16_t* table;
    float* logits;
    float* argValue;
    int32_t* argIndex;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return table + static_cast<uint64_t>(unit) * cols; }
    __device__ void Finish(uint32_t unit, const float* s, float& bestValue, int32_t& bestIndex) const
    {
        logits[unit] = s[0];
        // Units reach a lane in increasing order, so '>' keeps the lowest index on ties.
        if (s[0] > bestValue)
        {
            bestValue = s[0];
            bestIndex = static_cast<int32_t>(unit);
        }
    }
    __device__ void Tail(float value, int32_t index) const
    {
        BlockArgMax(value, index);
        if (threadIdx.x == 0)
        {
            argValue[blockIdx.x] = value;
            argIndex[blockIdx.x] = index;
        }
    }
};

// ------------------------------------------------------------------------------------------------
// Launch helpers for the fused GEMV.

template <int kLpr, int kCpl, int kNr, class Stage, class Epi>
hipError_t LaunchFusedT(hipStream_t s, uint32_t units, uint32_t blockCap, size_t lds, uint32_t cols,
                        const Stage& stage, const Epi& epi, uint32_t* blocksOut)
{
    const uint32_t unitsPerBlock = kWaves * ((kWave / kLpr) / kNr);
    const uint32_t blocks = std::max(1u, std::min(CeilDiv(units, unitsPerBlock), blockCap));
    if (blocksOut != nullptr)
    {
        *blocksOut = blocks;
        return hipSuccess;
    }
    // Opt in to more than the default 64 KB of dynamic LDS only when a launch needs it.
    static size_t configured = 64 * 1024;
    if (lds > configured)
    {
        const hipError_t status =
            hipFuncSetAttribute(reinterpret_cast<const void*>(&FusedMatVec<kLpr, kCpl, kNr, Stage, Epi>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (status != hipSuccess)
        {
            return status;
        }
        configured = lds;
    }
    hipLaunchKernelGGL((FusedMatVec<kLpr, kCpl, kNr, Stage, Epi>), dim3(blocks), dim3(kBlock), lds, s, cols, stage,
                       epi);
    return hipGetLastError();
}

/// Launches (or, with blocksOut, only sizes) the fused GEMV for a row of `cols` fp16 weights.
template <int kNr, class Stage, class Epi>
hipError_t LaunchFused(hipStream_t s, uint32_t units, uint32_t blockCap, uint32_t cols, const Stage& stage,
                       const Epi& epi, uint32_t* blocksOut = nullptr)
{
    if (cols % 8 != 0 || static_cast<size_t>(cols) * sizeof(float) > kMaxLds)
    {
        return hipErrorInvalidValue;
    }
    const RowShape shape = PickRowShape(cols / 8, kNr);
    const size_t lds = static_cast<size_t>(cols) * sizeof(float);
#define MUYO_FUSED_CASE(L, C)                                                                                \
    if (shape.lpr == L && shape.cpl == C)                                                                    \
    {                                                                                                        \
        return LaunchFusedT<L, C, kNr, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, blocksOut);    \
    }
    MUYO_FUSED_CASE(8, 8)
    MUYO_FUSED_CASE(16, 8)
    MUYO_FUSED_CASE(32, 8)
    MUYO_FUSED_CASE(32, 16)
    if constexpr (kNr == 1)
    {
        MUYO_FUSED_CASE(64, 8)
        MUYO_FUSED_CASE(64, 12)
        MUYO_FUSED_CASE(64, 16)
    }
#undef MUYO_FUSED_CASE
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------------------------------------
// Step bookkeeping.

/// Greedy id of the previous step: the best of the LM head's per-workgroup partials.
__device__ __forceinline__ int32_t ReduceArgMaxPartials(const float* __restrict__ argValue,
                                                        const int32_t* __restrict__ argIndex, uint32_t argBlocks)
{
    __shared__ int32_t token;
    float v = -INFINITY;
    int32_t i = 0x7FFFFFFF;
    constexpr int kPerThread = kArgMaxBlocks / kBlock;
    float values[kPerThread];
    int32_t indices[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
    {
        const uint32_t b = min(threadIdx.x + k * kBlock, argBlocks - 1);
        values[k] = argValue[b];
        indices[k] = argIndex[b];
    }
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
    {
        if (threadIdx.x + k * kBlock < argBlocks && Better(values[k], indices[k], v, i))
        {
            v = values[k];
            i = indices[k];
        }
    }
    BlockArgMax(v, i);
    if (threadIdx.x == 0)
    {
        token = i == 0x7FFFFFFF ? 0 : i;  // no finite logit at all: the host scan returns 0
    }
    __syncthreads();
    return token;
}

__global__ __launch_bounds__(kBlock) void SetStateKernel(DecodeState* state, float* argValue, int32_t* argIndex,
                                                         int32_t token, int32_t position, uint32_t argBlocks)
{
    for (uint32_t b = threadIdx.x; b < argBlocks; b += kBlock)
    {
        argValue[b] = b == 0 ? 0.0f : -INFINITY;
        argIndex[b] = b == 0 ? token : 0x7FFFFFFF;
    }
    if (threadIdx.x == 0)
    {
        state->token = token;
        state->position = position;
        state->start = position;
        state->step = 0;
    }
}

__global__ __launch_bounds__(kBlock) void BeginStepKernel(const uint16_t* __restrict__ table, DecodeState* state,
                                                          const float* __restrict__ argValue,
                                                          const int32_t* __restrict__ argIndex, uint32_t argBlocks,
                                                          float* __restrict__ x, int32_t* __restrict__ ids,
                                                          uint32_t idsCap, uint32_t hidden, uint32_t vocab)
{
    const int32_t token = ReduceArgMaxPartials(argValue, argIndex, argBlocks);
    if (blockIdx.x == 0 && threadIdx.x == 0)
    {
        const uint32_t step = state->step;
        if (step > 0)
        {
            ids[(step - 1) % idsCap] = token;
        }
        state->token = token;
        state->position = state->start + static_cast<int32_t>(step);
        state->step = step + 1;
    }
    const bool ok = token >= 0 && static_cast<uint32_t>(token) < vocab;
    const uint16_t* row = table + static_cast<uint64_t>(ok ? token : 0) * hidden;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < hidden; i += gridDim.x * kBlock)
    {
        x[i] = ok ? HalfBitsToFloat(row[i]) : 0.0f;
    }
}

__global__ __launch_bounds__(kBlock) void FinalizeKernel(DecodeState* state, const float* __restrict__ argValue,
                                                         const int32_t* __restrict__ argIndex, uint32_t argBlocks,
                                                         int32_t* __restrict__ ids, uint32_t idsCap)
{
    const int32_t token = ReduceArgMaxPartials(argValue, argIndex, argBlocks);
    if (threadIdx.x == 0)
    {
        const uint32_t step = state->step;
        if (step > 0)
        {
            ids[(step - 1) % idsCap] = token;
        }
        state->token = token;
    }
}

// ------------------------------------------------------------------------------------------------
// Attention over the fp16 cache: one workgroup per (256-key chunk, kv head).

template <int kHd>
__global__ __launch_bounds__(kBlock) void AttentionChunk(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         const int32_t* __restrict__ position, uint32_t group,
                                                         uint32_t maxSeq, float scale, DecodeScratch sc)
{
    constexpr int kRowChunks = kHd / 8;                  // 16-byte pieces per cache row
    constexpr int kPieces = kAttnTile * kRowChunks;      // per K (or V) tile
    constexpr int kPiecesPerThread = kPieces / kBlock;   // 2 (hd 64) or 4 (hd 128)
    constexpr int kLpk = kRowChunks;                     // lanes per key in the score pass
    constexpr int kKeysPerWave = kWave / kLpk;
    constexpr int kItems = kMaxGroup * kHd / kBlock;     // (head, channel) items per thread
    static_assert(kPieces % kBlock == 0 && (kMaxGroup * kHd) % kBlock == 0, "tile must split over the block");
    __shared__ half8 kS[kPieces];
    __shared__ half8 vS[kPieces];
    __shared__ __align__(16) float qs[kMaxGroup * kHd];
    __shared__ float probs[kMaxGroup][kAttnTile];
    __shared__ float runMax[kMaxGroup];
    __shared__ float runSum[kMaxGroup];
    __shared__ float rescale[kMaxGroup];

    const int32_t pos = *position;
    if (pos < 0 || static_cast<uint32_t>(pos) >= maxSeq)
    {
        return;
    }
    const uint32_t keys = static_cast<uint32_t>(pos) + 1;
    const uint32_t chunks = (keys + kAttnChunk - 1) / kAttnChunk;
    const uint32_t chunk = blockIdx.x;
    if (chunk >= chunks)
    {
        return;
    }
    const uint32_t g = blockIdx.y;
    const uint32_t c0 = chunk * kAttnChunk;
    const uint32_t cn = min(kAttnChunk, keys - c0);
    const uint32_t tiles = (cn + kAttnTile - 1) / kAttnTile;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const half8* kBase = reinterpret_cast<const half8*>(kc + static_cast<uint64_t>(g) * maxSeq * kHd);
    const half8* vBase = reinterpret_cast<const half8*>(vc + static_cast<uint64_t>(g) * maxSeq * kHd);

    // Tile loads: rows past the last key read the last key instead (always in bounds); their
    // probabilities are zero, so they add nothing.
    half8 kr[kPiecesPerThread];
    half8 vr[kPiecesPerThread];
    auto loadTile = [&](uint32_t t) {
#pragma unroll
        for (int i = 0; i < kPiecesPerThread; ++i)
        {
            const uint32_t piece = threadIdx.x + i * kBlock;
            const uint32_t key = min(c0 + t * kAttnTile + piece / kRowChunks, keys - 1);
            const uint64_t offset = static_cast<uint64_t>(key) * kRowChunks + piece % kRowChunks;
            kr[i] = kBase[offset];
            vr[i] = vBase[offset];
        }
    };
    loadTile(0);
    for (uint32_t i = threadIdx.x; i < group * kHd; i += kBlock)
    {
        qs[i] = q[static_cast<uint64_t>(g) * group * kHd + i];
    }
    if (threadIdx.x < kMaxGroup)
    {
        runMax[threadIdx.x] = -INFINITY;
        runSum[threadIdx.x] = 0.0f;
    }
    float acc[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k)
    {
        acc[k] = 0.0f;
    }
    const uint16_t* vFlat = reinterpret_cast<const uint16_t*>(vS);
    const int slice = lane % kLpk;

    for (uint32_t t = 0; t < tiles; ++t)
    {
        const uint32_t tn = min(kAttnTile, cn - t * kAttnTile);
        __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
        for (int i = 0; i < kPiecesPerThread; ++i)
        {
            kS[threadIdx.x + i * kBlock] = kr[i];
            vS[threadIdx.x + i * kBlock] = vr[i];
        }
        __syncthreads();
        if (t + 1 < tiles)
        {
            loadTile(t + 1);  // in flight while this tile is computed
        }

        // Scores: kLpk lanes per key, each lane one 16-byte slice against every head of the group.
        for (uint32_t jb = wave * kKeysPerWave; jb < kAttnTile; jb += kWaves * kKeysPerWave)
        {
            const uint32_t j = jb + lane / kLpk;
            const half8 k8 = kS[j * kRowChunks + slice];
#pragma unroll
            for (int h = 0; h < kMaxGroup; ++h)
            {
                float part = 0.0f;
                if (h < static_cast<int>(group))
                {
                    const float4 q0 = *reinterpret_cast<const float4*>(qs + h * kHd + slice * 8);
                    const float4 q1 = *reinterpret_cast<const float4*>(qs + h * kHd + slice * 8 + 4);
                    part = DotChunk(k8, q0, q1, 0.0f);
                }
                part = GroupSum<kLpk>(part);
                if (slice == 0 && h < static_cast<int>(group))
                {
                    probs[h][j] = j < tn ? part * scale : -INFINITY;
                }
            }
        }
        __syncthreads();

        // Online softmax, one wave per head (a tile is 64 keys: one per lane).
        for (uint32_t h = wave; h < group; h += kWaves)
        {
            const float v = probs[h][lane];
            const float tileMax = GroupMax<kWave>(v);
            const float oldMax = runMax[h];
            const float newMax = fmaxf(oldMax, tileMax);
            const float p = lane < static_cast<int>(tn) ? expf(v - newMax) : 0.0f;
            const float tileSum = GroupSum<kWave>(p);
            probs[h][lane] = p;
            if (lane == 0)
            {
                const float factor = expf(oldMax - newMax);  // 0 for the first tile
                rescale[h] = factor;
                runSum[h] = runSum[h] * factor + tileSum;
                runMax[h] = newMax;
            }
        }
        __syncthreads();

        // P.V: thread item (head, channel), accumulators rescaled to the running max.
#pragma unroll
        for (int k = 0; k < kItems; ++k)
        {
            const uint32_t item = threadIdx.x + k * kBlock;
            if (item < group * kHd)
            {
                const uint32_t h = item / kHd;
                const uint32_t d = item % kHd;
                float a0 = acc[k] * rescale[h];
                float a1 = 0.0f;
                uint32_t j = 0;
                for (; j + 1 < tn; j += 2)
                {
                    a0 = fmaf(probs[h][j], HalfBitsToFloat(vFlat[j * kHd + d]), a0);
                    a1 = fmaf(probs[h][j + 1], HalfBitsToFloat(vFlat[(j + 1) * kHd + d]), a1);
                }
                if (j < tn)
                {
                    a0 = fmaf(probs[h][j], HalfBitsToFloat(vFlat[j * kHd + d]), a0);
                }
                acc[k] = a0 + a1;
            }
        }
    }

    // Publish this chunk's partials (read after the kernel boundary).
    const uint64_t slot = static_cast<uint64_t>(g) * gridDim.x + chunk;
#pragma unroll
    for (int k = 0; k < kItems; ++k)
    {
        const uint32_t item = threadIdx.x + k * kBlock;
        if (item < group * kHd)
        {
            sc.attnAcc[(slot * group + item / kHd) * kHd + item % kHd] = acc[k];
        }
    }
    if (threadIdx.x < group)
    {
        sc.attnMax[slot * group + threadIdx.x] = runMax[threadIdx.x];
        sc.attnSum[slot * group + threadIdx.x] = runSum[threadIdx.x];
    }
}

/// Combine the chunk partials of every query head: one workgroup per head, a thread per channel.
__global__ __launch_bounds__(128) void AttentionMergeKernel(const int32_t* __restrict__ position, DecodeScratch sc,
                                                            float* __restrict__ out, uint32_t group, uint32_t headDim,
                                                            uint32_t maxChunks)
{
    const uint32_t h = blockIdx.x;
    const uint32_t g = h / group;
    const uint32_t hh = h % group;
    const uint32_t pos = static_cast<uint32_t>(max(*position, 0));
    const uint32_t chunks = min((pos + kAttnChunk) / kAttnChunk, maxChunks);
    float m[kMaxAttnChunks];
    float l[kMaxAttnChunks];
    float a[kMaxAttnChunks];
    for (uint32_t d = threadIdx.x; d < headDim; d += blockDim.x)
    {
#pragma unroll
        for (uint32_t c = 0; c < kMaxAttnChunks; ++c)
        {
            const uint32_t cc = min(c, chunks - 1);
            const uint64_t slot = (static_cast<uint64_t>(g) * maxChunks + cc) * group + hh;
            m[c] = sc.attnMax[slot];
            l[c] = sc.attnSum[slot];
            a[c] = sc.attnAcc[slot * headDim + d];
        }
        float mx = -INFINITY;
#pragma unroll
        for (uint32_t c = 0; c < kMaxAttnChunks; ++c)
        {
            mx = c < chunks ? fmaxf(mx, m[c]) : mx;
        }
        float num = 0.0f;
        float den = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < kMaxAttnChunks; ++c)
        {
            if (c < chunks)
            {
                const float e = expf(m[c] - mx);
                num = fmaf(e, a[c], num);
                den = fmaf(e, l[c], den);
            }
        }
        out[static_cast<uint64_t>(h) * headDim + d] = num / den;
    }
}

// ------------------------------------------------------------------------------------------------
// Rope + append from separate q/k/v vectors (the per-op form of the QKV epilogue).

__global__ __launch_bounds__(kBlock) void RopeAppendKernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, float* __restrict__ qOut,
                                                           uint16_t* __restrict__ kcache, uint16_t* __restrict__ vcache,
                                                           const int32_t* __restrict__ position, uint32_t heads,
                                                           uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq,
                                                           float thetaScale)
{
    const uint32_t half = headDim / 2;
    const uint32_t ropeItems = (heads + kvHeads) * half;
    const uint32_t total = ropeItems + kvHeads * headDim;
    const uint32_t item = blockIdx.x * kBlock + threadIdx.x;
    if (item >= total)
    {
        return;
    }
    const int32_t pos = *position;
    const bool inCache = pos >= 0 && static_cast<uint32_t>(pos) < maxSeq;
    if (item < ropeItems)
    {
        const uint32_t head = item / half;
        const uint32_t j = item % half;
        const float* src = head < heads ? q + head * headDim : k + (head - heads) * headDim;
        const float theta = static_cast<float>(pos) * powf(thetaScale, static_cast<float>(j));
        const float c = cosf(theta);
        const float s = sinf(theta);
        const float x0 = src[j];
        const float x1 = src[j + half];
        const float o0 = x0 * c - x1 * s;
        const float o1 = x0 * s + x1 * c;
        if (head < heads)
        {
            qOut[head * headDim + j] = o0;
            qOut[head * headDim + j + half] = o1;
        }
        else if (inCache)
        {
            const uint64_t base = (static_cast<uint64_t>(head - heads) * maxSeq + pos) * headDim;
            kcache[base + j] = FloatToHalfBits(o0);
            kcache[base + j + half] = FloatToHalfBits(o1);
        }
    }
    else if (inCache)
    {
        const uint32_t channel = item - ropeItems;
        const uint32_t g = channel / headDim;
        vcache[(static_cast<uint64_t>(g) * maxSeq + pos) * headDim + channel % headDim] = FloatToHalfBits(v[channel]);
    }
}
}  // namespace

uint32_t LmHeadBlocks(const DecodeDims& dims)
{
    uint32_t blocks = 0;
    LmHeadEpi epi{};
    epi.rows = dims.vocab;
    (void)LaunchFused<1>(nullptr, dims.vocab, std::min(kArgMaxBlocks, GemvBlockCap()), dims.hidden,
                         NormStage{nullptr, nullptr, 0.0f}, epi, &blocks);
    return blocks;
}

bool MergeInOProj(const DecodeDims& dims)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    return AttnChunks(dims.maxSeq) <= kMergeChunks && qdim <= kMergeItems * kBlock &&
           dims.heads * AttnChunks(dims.maxSeq) <= static_cast<uint32_t>(kBlock);
}

hipError_t LaunchSetState(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, int32_t token,
                          int32_t position, uint32_t argBlocks)
{
    hipLaunchKernelGGL(SetStateKernel, dim3(1), dim3(kBlock), 0, s, state, scratch.argValue, scratch.argIndex, token,
                       position, argBlocks);
    return hipGetLastError();
}

hipError_t LaunchBeginStep(hipStream_t s, const uint16_t* table, DecodeState* state, const DecodeScratch& scratch,
                           uint32_t argBlocks, float* x, int32_t* ids, uint32_t idsCap, uint32_t hidden,
                           uint32_t vocab)
{
    hipLaunchKernelGGL(BeginStepKernel, dim3(CeilDiv(hidden, kBlock)), dim3(kBlock), 0, s, table, state,
                       scratch.argValue, scratch.argIndex, argBlocks, x, ids, idsCap, hidden, vocab);
    return hipGetLastError();
}

hipError_t LaunchFinalize(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, uint32_t argBlocks,
                          int32_t* ids, uint32_t idsCap)
{
    hipLaunchKernelGGL(FinalizeKernel, dim3(1), dim3(kBlock), 0, s, state, scratch.argValue, scratch.argIndex,
                       argBlocks, ids, idsCap);
    return hipGetLastError();
}

hipError_t LaunchQkvRopeAppend(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                               const uint16_t* wqkv, const float* bias, const DecodeState* state, float* qOut,
                               uint16_t* kcache, uint16_t* vcache)
{
    QkvEpi epi{wqkv,        bias,       state,         qOut,         kcache, vcache, dims.hidden, dims.heads,
               dims.kvHeads, dims.headDim, dims.maxSeq, dims.thetaScale};
    const uint32_t units = (dims.heads + 2 * dims.kvHeads) * dims.headDim / 2;
    return LaunchFused<2>(s, units, GemvBlockCap(), dims.hidden, NormStage{x, normW, dims.eps}, epi);
}

hipError_t LaunchAttention(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                           const uint16_t* vcache, const int32_t* position, const DecodeScratch& scratch)
{
    const uint32_t group = dims.heads / dims.kvHeads;
    if (group == 0 || group > static_cast<uint32_t>(kMaxGroup) || dims.heads % dims.kvHeads != 0 ||
        AttnChunks(dims.maxSeq) > kMaxAttnChunks)
    {
        return hipErrorInvalidValue;
    }
    const dim3 grid(AttnChunks(dims.maxSeq), dims.kvHeads, 1);
    switch (dims.headDim)
    {
        case 64:
            hipLaunchKernelGGL(AttentionChunk<64>, grid, dim3(kBlock), 0, s, q, kcache, vcache, position, group,
                               dims.maxSeq, dims.attnScale, scratch);
            break;
        case 128:
            hipLaunchKernelGGL(AttentionChunk<128>, grid, dim3(kBlock), 0, s, q, kcache, vcache, position, group,
                               dims.maxSeq, dims.attnScale, scratch);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t LaunchAttentionMerge(hipStream_t s, const DecodeDims& dims, const int32_t* position,
                                const DecodeScratch& scratch, float* out)
{
    hipLaunchKernelGGL(AttentionMergeKernel, dim3(dims.heads), dim3(std::min<uint32_t>(dims.headDim, 128)), 0, s,
                       position, scratch, out, dims.heads / dims.kvHeads, dims.headDim, AttnChunks(dims.maxSeq));
    return hipGetLastError();
}

hipError_t LaunchOProjMerged(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const int32_t* position,
                             const DecodeScratch& scratch, const float* residual, float* out)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    MergeStage stage{position,   scratch.attnMax,           scratch.attnSum, scratch.attnAcc,
                     dims.heads, dims.heads / dims.kvHeads, dims.headDim,    AttnChunks(dims.maxSeq)};
    ResidualEpi epi{wo, residual, out, dims.hidden, qdim};
    return LaunchFused<1>(s, dims.hidden, GemvBlockCap(), qdim, stage, epi);
}

hipError_t LaunchMatVecResidual(hipStream_t s, const uint16_t* w, const float* x, const float* residual, float* out,
                                uint32_t rows, uint32_t cols)
{
    ResidualEpi epi{w, residual, out, rows, cols};
    return LaunchFused<1>(s, rows, GemvBlockCap(), cols, PlainStage{x}, epi);
}

hipError_t LaunchGateUpSwiGlu(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* wgate, const uint16_t* wup, float* act)
{
    GateUpEpi epi{wgate, wup, act, dims.ffn, dims.hidden};
    return LaunchFused<2>(s, dims.ffn, GemvBlockCap(), dims.hidden, NormStage{x, normW, dims.eps}, epi);
}

hipError_t LaunchLmHeadArgMax(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* table, float* logits, const DecodeScratch& scratch)
{
    LmHeadEpi epi{table, logits, scratch.argValue, scratch.argIndex, dims.vocab, dims.hidden};
    return LaunchFused<1>(s, dims.vocab, std::min(kArgMaxBlocks, GemvBlockCap()), dims.hidden,
                          NormStage{x, normW, dims.eps}, epi);
}

hipError_t LaunchRopeAppend(hipStream_t s, const float* q, const float* k, const float* v, float* qOut,
                            uint16_t* kcache, uint16_t* vcache, const int32_t* position, uint32_t heads,
                            uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, float thetaScale)
{
    const uint32_t total = (heads + kvHeads) * (headDim / 2) + kvHeads * headDim;
    hipLaunchKernelGGL(RopeAppendKernel, dim3(CeilDiv(total, kBlock)), dim3(kBlock), 0, s, q, k, v, qOut, kcache,
                       vcache, position, heads, kvHeads, headDim, maxSeq, thetaScale);
    return hipGetLastError();
}
}  // namespace muyo

// ------------------------------------------------------------------------------------------------
// C ABI for the two attention-side ops.

using namespace muyo;

namespace
{
struct AttentionScratchOwner
{
    DecodeScratch scratch{};
    size_t floats = 0;
    int device = -1;
};

thread_local AttentionScratchOwner g_attentionScratch;

int EnsureAttentionScratch(uint32_t kvHeads, uint32_t chunks, uint32_t group, uint32_t headDim)
{
    int device = 0;
    MUYO_HIP_CHECK(hipGetDevice(&device));
    AttentionScratchOwner& o = g_attentionScratch;
    const size_t small = static_cast<size_t>(kvHeads) * chunks * group;
    const size_t floats = 2 * small + small * headDim;
    if (o.device == device && o.floats >= floats)
    {
        return MUYO_OK;
    }
    if (o.scratch.attnMax != nullptr)
    {
        (void)hipFree(o.scratch.attnMax);
        o.scratch = DecodeScratch{};
        o.floats = 0;
    }
    float* base = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&base), floats * sizeof(float)) != hipSuccess)
    {
        return Fail(MUYO_E_NOMEM, "attention scratch: hipMalloc(%zu) failed", floats * sizeof(float));
    }
    o.scratch.attnMax = base;
    o.scratch.attnSum = base + small;
    o.scratch.attnAcc = base + 2 * small;
    o.floats = floats;
    o.device = device;
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_attention_decode_f16kv(const float* q, const void* kcache, const void* vcache, float* out,
                                           const int32_t* position, uint32_t heads, uint32_t kv_heads,
                                           uint32_t head_dim, uint32_t max_seq, float scale, void* stream)
{
    const char* name = "attention_decode_f16kv";
    if (q == nullptr || kcache == nullptr || vcache == nullptr || out == nullptr || position == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: q, caches, out and position are required", name);
    }
    if (kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > 8 || (head_dim != 64 && head_dim != 128) ||
        max_seq == 0 || max_seq > kMaxAttnChunks * kAttnChunk)
    {
        return Fail(MUYO_E_UNSUPPORTED,
                    "%s: needs heads %% kv_heads == 0, group <= 8, head_dim 64 or 128, max_seq <= %u", name,
                    kMaxAttnChunks * kAttnChunk);
    }
    const int status = EnsureAttentionScratch(kv_heads, AttnChunks(max_seq), heads / kv_heads, head_dim);
    if (status != MUYO_OK)
    {
        return status;
    }
    DecodeDims dims{};
    dims.heads = heads;
    dims.kvHeads = kv_heads;
    dims.headDim = head_dim;
    dims.maxSeq = max_seq;
    dims.attnScale = scale;
    hipError_t launched = LaunchAttention(AsStream(stream), dims, q, static_cast<const uint16_t*>(kcache),
                                          static_cast<const uint16_t*>(vcache), position, g_attentionScratch.scratch);
    if (launched == hipSuccess)
    {
        launched = LaunchAttentionMerge(AsStream(stream), dims, position, g_attentionScratch.scratch, out);
    }
    return launched == hipSuccess ? MUYO_OK : HipStatus(launched, name);
}

extern "C" int muyo_rope_append_f16kv(const float* q, const float* k, const float* v, float* q_out, void* kcache,
                                      void* vcache, const int32_t* position, uint32_t heads, uint32_t kv_heads,
                                      uint32_t head_dim, uint32_t max_seq, float theta_scale, void* stream)
{
    const char* name = "rope_append_f16kv";
    if (q == nullptr || k == nullptr || v == nullptr || q_out == nullptr || kcache == nullptr || vcache == nullptr ||
        position == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: every pointer is required", name);
    }
    if (head_dim == 0 || head_dim % 2 != 0 || max_seq == 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: head_dim must be even and max_seq >= 1", name);
    }
    const hipError_t launched = LaunchRopeAppend(AsStream(stream), q, k, v, q_out, static_cast<uint16_t*>(kcache),
                                                 static_cast<uint16_t*>(vcache), position, heads, kv_heads, head_dim,
                                                 max_seq, theta_scale);
    return launched == hipSuccess ? MUYO_OK : HipStatus(launched, name);
}
