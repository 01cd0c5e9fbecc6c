// Fused decode-step kernels for gfx950.
//
// One Qwen2 layer is five launches (the reference records 18 nodes per layer,
// src/FullModel.cpp:227-453):
//   1. QkvRopeAppend : rms_norm prologue -> fused q|k|v GEMV + bias -> NeoX rope of q and k ->
//                      q to a buffer, k and v appended as fp16 at the position's cache row
//   2. Attention     : split over 64-key chunks of the fp16 cache; each block computes scores,
//                      a chunk-local softmax and P.V for the whole GQA group of its KV head;
//                      the last block to finish merges the chunks (flash-decoding)
//   3. MatVecResidual: o_proj GEMV + residual add
//   4. GateUpSwiGlu  : rms_norm prologue -> gate and up GEMV rows -> silu(g)*u
//   5. MatVecResidual: down GEMV + residual add
// and the step ends with LmHeadArgMax: final rms_norm -> tied LM head -> logits + greedy
// argmax (ties to the lowest index) -> next token, position and step advanced on the device.
//
// GEMV core: the activation is staged once per workgroup in LDS (normalised in place when the
// op has an rms_norm prologue); a wave64 splits into segments of LPR lanes, each segment
// streaming one fp16 weight row in 16-byte chunks; segment sums reduce across lanes; the
// segments of one "unit" (1 or 2 rows) meet in the unit's leader lane for the epilogue.
#include <algorithm>

#include "common.hpp"
#include "decode_kernels.hpp"

namespace muyo
{
namespace
{
constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr uint32_t kMaxLds = 160 * 1024;

__device__ __forceinline__ uint32_t SplitSlot(uint32_t i, uint32_t nchunks)
{
    const uint32_t c = i >> 3;
    const uint32_t r = i & 7u;
    return r < 4 ? c * 4 + r : (nchunks + c) * 4 + (r - 4);
}

/// Stage n floats (n % 8 == 0) into LDS in the split chunk layout; with kNorm, scale them by
/// rsqrt(mean(x^2) + eps) and the norm weight (order: (scale * x) * w, as rms_norm.comp:122).
template <bool kNorm>
__device__ __forceinline__ void StageActivation(const float* __restrict__ x, const float* __restrict__ w, uint32_t n,
                                                float eps, float4* xs)
{
    __shared__ float partial[kWaves];
    float* flat = reinterpret_cast<float*>(xs);
    const uint32_t nchunks = n / 8;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += kBlock)
    {
        const float v = x[i];
        flat[SplitSlot(i, nchunks)] = v;
        if (kNorm)
        {
            ss = fmaf(v, v, ss);
        }
    }
    if (kNorm)
    {
        ss = GroupSum<kWave>(ss);
        if ((threadIdx.x & (kWave - 1)) == 0)
        {
            partial[threadIdx.x / kWave] = ss;
        }
        __syncthreads();
        const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
        const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
        for (uint32_t i = threadIdx.x; i < n; i += kBlock)
        {
            const uint32_t slot = SplitSlot(i, nchunks);
            flat[slot] = (scale * flat[slot]) * w[i];
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float Dot8(const uint16_t* __restrict__ row, uint32_t chunk, const float4* __restrict__ lo,
                                      const float4* __restrict__ hi, float acc)
{
    float w[8];
    LoadHalf8(row + static_cast<uint64_t>(chunk) * 8, w);
    const float4 x0 = lo[chunk];
    const float4 x1 = hi[chunk];
    acc = fmaf(w[0], x0.x, acc);
    acc = fmaf(w[1], x0.y, acc);
    acc = fmaf(w[2], x0.z, acc);
    acc = fmaf(w[3], x0.w, acc);
    acc = fmaf(w[4], x1.x, acc);
    acc = fmaf(w[5], x1.y, acc);
    acc = fmaf(w[6], x1.z, acc);
    acc = fmaf(w[7], x1.w, acc);
    return acc;
}

/// This lane's share of one row's dot product (not yet reduced across the segment).
template <int kLpr>
__device__ __forceinline__ float SegmentPartial(const uint16_t* __restrict__ row, uint32_t nchunks, uint32_t lir,
                                                const float4* __restrict__ lo, const float4* __restrict__ hi)
{
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    uint32_t c = lir;
    for (; c + 3 * kLpr < nchunks; c += 4 * kLpr)
    {
        a0 = Dot8(row, c, lo, hi, a0);
        a1 = Dot8(row, c + kLpr, lo, hi, a1);
        a2 = Dot8(row, c + 2 * kLpr, lo, hi, a2);
        a3 = Dot8(row, c + 3 * kLpr, lo, hi, a3);
    }
    for (; c < nchunks; c += kLpr)
    {
        a0 = Dot8(row, c, lo, hi, a0);
    }
    return (a0 + a1) + (a2 + a3);
}

struct NoTail
{
};

/// Generic fused GEMV: units of kNr rows, an epilogue per unit, an optional block tail.
template <int kLpr, int kNr, bool kNorm, class Epi>
__global__ __launch_bounds__(kBlock) void FusedMatVec(const float* __restrict__ x, const float* __restrict__ normW,
                                                      uint32_t cols, float eps, Epi epi)
{
    extern __shared__ float4 xs[];
    const uint32_t nchunks = cols / 8;
    StageActivation<kNorm>(x, normW, cols, eps, xs);
    const float4* lo = xs;
    const float4* hi = xs + nchunks;

    constexpr int kSegs = kWave / kLpr;
    constexpr int kUnits = kSegs / kNr;
    static_assert(kUnits >= 1, "a wave must hold at least one unit");
    const int lane = threadIdx.x & (kWave - 1);
    const int segment = lane / kLpr;
    const int lir = lane % kLpr;
    const int unitInWave = segment / kNr;
    const int part = segment % kNr;
    const uint32_t wave = blockIdx.x * kWaves + threadIdx.x / kWave;
    const uint32_t waves = gridDim.x * kWaves;
    const uint32_t units = epi.Units();

    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    for (uint32_t first = wave * kUnits; first < units; first += waves * kUnits)
    {
        const uint32_t unit = first + unitInWave;
        const bool valid = unit < units && segment < kUnits * kNr;
        float dot = 0.0f;
        if (valid)
        {
            dot = SegmentPartial<kLpr>(epi.Row(unit, part), nchunks, lir, lo, hi);
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
            const uint32_t channel = 2 * (unit - ropeUnits);  // within kvHeads*headDim
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
        act[unit] = s[0] / (1.0f + expf(-s[0])) * s[1];
    }
    __device__ void Tail(float, int32_t) const {}
};

struct LmHeadEpi
{
    const uint16_t* table;
    float* logits;
    DecodeState* state;
    int32_t* ids;
    uint32_t idsCap;
    uint32_t rows, cols;
    float* argValue;
    int32_t* argIndex;
    uint32_t* argCount;

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
        __shared__ float waveValue[kWaves];
        __shared__ int32_t waveIndex[kWaves];
        __shared__ int isLast;
        GroupArgMax<kWave>(value, index);
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        if (lane == 0)
        {
            waveValue[wave] = value;
            waveIndex[wave] = index;
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
            float v = waveValue[0];
            int32_t i = waveIndex[0];
            for (int k = 1; k < kWaves; ++k)
            {
                if (waveValue[k] > v || (waveValue[k] == v && waveIndex[k] < i))
                {
                    v = waveValue[k];
                    i = waveIndex[k];
                }
            }
            argValue[blockIdx.x] = v;
            argIndex[blockIdx.x] = i;
            __threadfence();
            isLast = atomicAdd(argCount, 1u) == gridDim.x - 1;
        }
        __syncthreads();
        if (!isLast)
        {
            return;
        }
        __threadfence();
        float v = -INFINITY;
        int32_t i = 0x7FFFFFFF;
        for (uint32_t b = threadIdx.x; b < gridDim.x; b += kBlock)
        {
            const float bv = __builtin_nontemporal_load(argValue + b);
            const int32_t bi = __builtin_nontemporal_load(argIndex + b);
            if (bv > v || (bv == v && bi < i))
            {
                v = bv;
                i = bi;
            }
        }
        GroupArgMax<kWave>(v, i);
        __syncthreads();
        if (lane == 0)
        {
            waveValue[wave] = v;
            waveIndex[wave] = i;
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
            v = waveValue[0];
            i = waveIndex[0];
            for (int k = 1; k < kWaves; ++k)
            {
                if (waveValue[k] > v || (waveValue[k] == v && waveIndex[k] < i))
                {
                    v = waveValue[k];
                    i = waveIndex[k];
                }
            }
            const int32_t next = i == 0x7FFFFFFF ? 0 : i;
            const uint32_t step = state->step;
            ids[step % idsCap] = next;
            state->token = next;
            state->position = state->position + 1;
            state->step = step + 1;
            *argCount = 0;
        }
    }
};

// ------------------------------------------------------------------------------------------------
// Launch helpers for the fused GEMV.

int PickLpr(uint32_t nchunks, int nr)
{
    int lpr = nchunks <= 64 ? 8 : (nchunks <= 128 ? 16 : (nchunks <= 256 ? 32 : 64));
    if (nr == 2 && lpr > 32)
    {
        lpr = 32;
    }
    return lpr;
}

template <int kLpr, int kNr, bool kNorm, class Epi>
hipError_t LaunchFusedT(hipStream_t s, uint32_t blocks, size_t lds, const float* x, const float* normW,
                        uint32_t cols, float eps, const Epi& epi)
{
    // Opt in to more than the default 64 KB of dynamic LDS only when a launch needs it.
    static size_t configured = 64 * 1024;
    if (lds > configured)
    {
        const hipError_t status =
            hipFuncSetAttribute(reinterpret_cast<const void*>(&FusedMatVec<kLpr, kNr, kNorm, Epi>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (status != hipSuccess)
        {
            return status;
        }
        configured = lds;
    }
    hipLaunchKernelGGL((FusedMatVec<kLpr, kNr, kNorm, Epi>), dim3(blocks), dim3(kBlock), lds, s, x, normW, cols, eps,
                       epi);
    return hipGetLastError();
}

template <int kNr, bool kNorm, class Epi>
hipError_t LaunchFused(hipStream_t s, uint32_t units, uint32_t blockCap, const float* x, const float* normW,
                       uint32_t cols, float eps, const Epi& epi)
{
    if (cols % 8 != 0 || static_cast<size_t>(cols) * sizeof(float) > kMaxLds)
    {
        return hipErrorInvalidValue;
    }
    const uint32_t nchunks = cols / 8;
    const int lpr = PickLpr(nchunks, kNr);
    const uint32_t unitsPerBlock = kWaves * ((kWave / lpr) / kNr);
    const uint32_t blocks = std::max(1u, std::min(CeilDiv(units, unitsPerBlock), blockCap));
    const size_t lds = static_cast<size_t>(cols) * sizeof(float);
    switch (lpr)
    {
        case 8:
            return LaunchFusedT<8, kNr, kNorm>(s, blocks, lds, x, normW, cols, eps, epi);
        case 16:
            return LaunchFusedT<16, kNr, kNorm>(s, blocks, lds, x, normW, cols, eps, epi);
        case 32:
            return LaunchFusedT<32, kNr, kNorm>(s, blocks, lds, x, normW, cols, eps, epi);
        default:
            if constexpr (kNr == 1)
            {
                return LaunchFusedT<64, kNr, kNorm>(s, blocks, lds, x, normW, cols, eps, epi);
            }
            return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------------------------------------
// Embedding gather.

__global__ __launch_bounds__(kBlock) void EmbedKernel(const uint16_t* __restrict__ table,
                                                      const DecodeState* __restrict__ state, float* __restrict__ x,
                                                      uint32_t hidden, uint32_t vocab)
{
    const int32_t token = state->token;
    const bool ok = token >= 0 && static_cast<uint32_t>(token) < vocab;
    const uint16_t* row = table + static_cast<uint64_t>(ok ? token : 0) * hidden;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < hidden; i += gridDim.x * kBlock)
    {
        x[i] = ok ? HalfBitsToFloat(row[i]) : 0.0f;
    }
}

// ------------------------------------------------------------------------------------------------
// Attention over the fp16 cache, one block per (64-key chunk, kv head).

constexpr int kMaxGroup = 8;

template <int kHd>
__global__ __launch_bounds__(kBlock) void AttentionChunk(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         const int32_t* __restrict__ position, float* __restrict__ out,
                                                         uint32_t group, uint32_t maxSeq, float scale,
                                                         DecodeScratch sc)
{
    constexpr int kLpk = kHd / 8;             // lanes per key row (16 bytes each)
    constexpr int kKeysPerWave = kWave / kLpk;
    constexpr int kKeysPerPass = kKeysPerWave * kWaves;
    constexpr int kKeyGroups = kBlock / kHd;  // P.V: threads per column
    __shared__ float qs[kMaxGroup * kHd];
    __shared__ float scores[kMaxGroup][kAttnChunk];
    __shared__ float chunkMax[kMaxGroup];
    __shared__ float chunkSum[kMaxGroup];
    __shared__ float reduce[kKeyGroups > 1 ? (kKeyGroups - 1) * kMaxGroup * kHd : 1];
    __shared__ int isLast;

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
    const uint32_t maxChunks = gridDim.x;
    const uint32_t j0 = chunk * kAttnChunk;
    const uint32_t jn = min(kAttnChunk, keys - j0);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;

    for (uint32_t i = threadIdx.x; i < group * kHd; i += kBlock)
    {
        qs[i] = q[static_cast<uint64_t>(g) * group * kHd + i];
    }
    __syncthreads();

    // Scores: kLpk lanes per key, every lane dots its 8 channels with all heads of the group.
    const uint16_t* kBase = kc + (static_cast<uint64_t>(g) * maxSeq + j0) * kHd;
    const int l8 = lane % kLpk;
    for (uint32_t jb = 0; jb < jn; jb += kKeysPerPass)
    {
        const uint32_t j = jb + wave * kKeysPerWave + lane / kLpk;
        float part[kMaxGroup];
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
        {
            part[h] = 0.0f;
        }
        if (j < jn)
        {
            float k8[8];
            LoadHalf8(kBase + static_cast<uint64_t>(j) * kHd + l8 * 8, k8);
#pragma unroll
            for (int h = 0; h < kMaxGroup; ++h)
            {
                if (h < static_cast<int>(group))
                {
                    const float* qh = qs + h * kHd + l8 * 8;
                    float acc = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                    {
                        acc = fmaf(qh[e], k8[e], acc);
                    }
                    part[h] = acc;
                }
            }
        }
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
        {
            part[h] = GroupSum<kLpk>(part[h]);
        }
        if (j < jn && l8 == 0)
        {
            for (uint32_t h = 0; h < group; ++h)
            {
                scores[h][j] = part[h] * scale;
            }
        }
    }
    __syncthreads();

    // Chunk-local softmax numerators, one wave per head.
    for (uint32_t h = wave; h < group; h += kWaves)
    {
        float m = -INFINITY;
        for (uint32_t j = lane; j < jn; j += kWave)
        {
            m = fmaxf(m, scores[h][j]);
        }
        m = GroupMax<kWave>(m);
        float l = 0.0f;
        for (uint32_t j = lane; j < jn; j += kWave)
        {
            const float p = expf(scores[h][j] - m);
            scores[h][j] = p;
            l += p;
        }
        l = GroupSum<kWave>(l);
        if (lane == 0)
        {
            chunkMax[h] = m;
            chunkSum[h] = l;
        }
    }
    __syncthreads();

    // P.V: thread (keyGroup, column) sums keys keyGroup, keyGroup + kKeyGroups, ...
    const uint32_t column = threadIdx.x % kHd;
    const uint32_t keyGroup = threadIdx.x / kHd;
    const uint16_t* vBase = vc + (static_cast<uint64_t>(g) * maxSeq + j0) * kHd;
    float acc[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
    {
        acc[h] = 0.0f;
    }
    for (uint32_t j = keyGroup; j < jn; j += kKeyGroups)
    {
        const float v = HalfBitsToFloat(vBase[static_cast<uint64_t>(j) * kHd + column]);
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h)
        {
            if (h < static_cast<int>(group))
            {
                acc[h] = fmaf(scores[h][j], v, acc[h]);
            }
        }
    }
    if (kKeyGroups > 1)
    {
        if (keyGroup > 0)
        {
            for (uint32_t h = 0; h < group; ++h)
            {
                reduce[((keyGroup - 1) * kMaxGroup + h) * kHd + column] = acc[h];
            }
        }
        __syncthreads();
        if (keyGroup == 0)
        {
            for (int kg = 1; kg < kKeyGroups; ++kg)
            {
                for (uint32_t h = 0; h < group; ++h)
                {
                    acc[h] += reduce[((kg - 1) * kMaxGroup + h) * kHd + column];
                }
            }
        }
    }

    // Publish this chunk's partials.
    const uint64_t slot = static_cast<uint64_t>(g) * maxChunks + chunk;
    if (keyGroup == 0)
    {
        for (uint32_t h = 0; h < group; ++h)
        {
            sc.attnAcc[(slot * group + h) * kHd + column] = acc[h];
        }
    }
    if (threadIdx.x < group)
    {
        sc.attnMax[slot * group + threadIdx.x] = chunkMax[threadIdx.x];
        sc.attnSum[slot * group + threadIdx.x] = chunkSum[threadIdx.x];
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
    {
        isLast = atomicAdd(sc.attnCount + g, 1u) == chunks - 1;
    }
    __syncthreads();
    if (!isLast)
    {
        return;
    }
    __threadfence();

    // Merge the chunks of this kv head: out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.
    for (uint32_t item = threadIdx.x; item < group * kHd; item += kBlock)
    {
        const uint32_t h = item / kHd;
        const uint32_t d = item % kHd;
        const uint64_t base = static_cast<uint64_t>(g) * maxChunks;
        float m = -INFINITY;
        for (uint32_t c = 0; c < chunks; ++c)
        {
            m = fmaxf(m, __builtin_nontemporal_load(sc.attnMax + (base + c) * group + h));
        }
        float num = 0.0f;
        float den = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c)
        {
            const float e = expf(__builtin_nontemporal_load(sc.attnMax + (base + c) * group + h) - m);
            num = fmaf(e, __builtin_nontemporal_load(sc.attnAcc + ((base + c) * group + h) * kHd + d), num);
            den = fmaf(e, __builtin_nontemporal_load(sc.attnSum + (base + c) * group + h), den);
        }
        out[(static_cast<uint64_t>(g) * group + h) * kHd + d] = num / den;
    }
    if (threadIdx.x == 0)
    {
        sc.attnCount[g] = 0;
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

hipError_t LaunchEmbed(hipStream_t s, const uint16_t* table, const DecodeState* state, float* x, uint32_t hidden,
                       uint32_t vocab)
{
    hipLaunchKernelGGL(EmbedKernel, dim3(CeilDiv(hidden, kBlock)), dim3(kBlock), 0, s, table, state, x, hidden, vocab);
    return hipGetLastError();
}

hipError_t LaunchQkvRopeAppend(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                               const uint16_t* wqkv, const float* bias, const DecodeState* state, float* qOut,
                               uint16_t* kcache, uint16_t* vcache)
{
    QkvEpi epi{wqkv,        bias,       state,         qOut,         kcache, vcache, dims.hidden, dims.heads,
               dims.kvHeads, dims.headDim, dims.maxSeq, dims.thetaScale};
    const uint32_t units = (dims.heads + 2 * dims.kvHeads) * dims.headDim / 2;
    return LaunchFused<2, true>(s, units, 4096, x, normW, dims.hidden, dims.eps, epi);
}

hipError_t LaunchAttention(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                           const uint16_t* vcache, const int32_t* position, float* out, const DecodeScratch& scratch)
{
    const uint32_t group = dims.heads / dims.kvHeads;
    if (group == 0 || group > static_cast<uint32_t>(kMaxGroup) || dims.heads % dims.kvHeads != 0)
    {
        return hipErrorInvalidValue;
    }
    const dim3 grid(AttnChunks(dims.maxSeq), dims.kvHeads, 1);
    switch (dims.headDim)
    {
        case 64:
            hipLaunchKernelGGL(AttentionChunk<64>, grid, dim3(kBlock), 0, s, q, kcache, vcache, position, out, group,
                               dims.maxSeq, dims.attnScale, scratch);
            break;
        case 128:
            hipLaunchKernelGGL(AttentionChunk<128>, grid, dim3(kBlock), 0, s, q, kcache, vcache, position, out, group,
                               dims.maxSeq, dims.attnScale, scratch);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t LaunchMatVecResidual(hipStream_t s, const uint16_t* w, const float* x, const float* residual, float* out,
                                uint32_t rows, uint32_t cols)
{
    ResidualEpi epi{w, residual, out, rows, cols};
    return LaunchFused<1, false>(s, rows, 4096, x, nullptr, cols, 0.0f, epi);
}

hipError_t LaunchGateUpSwiGlu(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* wgate, const uint16_t* wup, float* act)
{
    GateUpEpi epi{wgate, wup, act, dims.ffn, dims.hidden};
    return LaunchFused<2, true>(s, dims.ffn, 4096, x, normW, dims.hidden, dims.eps, epi);
}

hipError_t LaunchLmHeadArgMax(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* table, float* logits, DecodeState* state, int32_t* ids, uint32_t idsCap,
                              const DecodeScratch& scratch)
{
    LmHeadEpi epi{table,        logits,         state,           ids, idsCap, dims.vocab, dims.hidden,
                  scratch.argValue, scratch.argIndex, scratch.argCount};
    return LaunchFused<1, true>(s, dims.vocab, kArgMaxBlocks, x, normW, dims.hidden, dims.eps, epi);
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
    uint32_t kvHeads = 0;
    uint32_t chunks = 0;
    uint32_t group = 0;
    uint32_t headDim = 0;
    int device = -1;
};

thread_local AttentionScratchOwner g_attentionScratch;

int EnsureAttentionScratch(uint32_t kvHeads, uint32_t chunks, uint32_t group, uint32_t headDim)
{
    int device = 0;
    MUYO_HIP_CHECK(hipGetDevice(&device));
    AttentionScratchOwner& o = g_attentionScratch;
    if (o.device == device && o.kvHeads >= kvHeads && o.chunks == chunks && o.group >= group && o.headDim >= headDim)
    {
        return MUYO_OK;
    }
    if (o.scratch.attnMax != nullptr)
    {
        (void)hipFree(o.scratch.attnMax);
        o.scratch = DecodeScratch{};
    }
    const size_t small = static_cast<size_t>(kvHeads) * chunks * group;
    const size_t bytes = (2 * small + small * headDim) * sizeof(float) + kvHeads * sizeof(uint32_t) + 256;
    char* base = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&base), bytes) != hipSuccess)
    {
        return Fail(MUYO_E_NOMEM, "attention scratch: hipMalloc(%zu) failed", bytes);
    }
    MUYO_HIP_CHECK(hipMemset(base, 0, bytes));
    o.scratch.attnMax = reinterpret_cast<float*>(base);
    o.scratch.attnSum = o.scratch.attnMax + small;
    o.scratch.attnAcc = o.scratch.attnSum + small;
    o.scratch.attnCount = reinterpret_cast<uint32_t*>(o.scratch.attnAcc + small * headDim);
    o.kvHeads = kvHeads;
    o.chunks = chunks;
    o.group = group;
    o.headDim = headDim;
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
        max_seq == 0)
    {
        return Fail(MUYO_E_UNSUPPORTED, "%s: needs heads %% kv_heads == 0, group <= 8, head_dim 64 or 128", name);
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
    const hipError_t launched = LaunchAttention(AsStream(stream), dims, q, static_cast<const uint16_t*>(kcache),
                                                static_cast<const uint16_t*>(vcache), position, out,
                                                g_attentionScratch.scratch);
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
