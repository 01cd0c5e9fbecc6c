// Row reductions: rms_norm_f32, soft_max_f32, argmax_f32.
//
// Each row is owned by one wave64 (rms_norm, soft_max) or one workgroup (argmax over a long
// row). Sums and maxima are reduced with cross-lane shuffles; rows that fit are kept in
// registers between passes, longer rows are re-read (the re-read hits L2, so HBM traffic stays
// one read and one write per element).
#include <algorithm>
#include <cfloat>

#include "common.hpp"

namespace muyo
{
namespace
{
constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

// ------------------------------------------------------------------------------------------------
// rms_norm (shaders/llama/rms_norm.comp:53-151, do_multiply spec id 1).

struct RmsArgs
{
    uint32_t ncols;
    uint32_t nrows;      // dispatch x
    uint32_t nchannels;  // dispatch y
    uint32_t total;      // x * y * z
    uint32_t nb01, nb02, nb03;
    uint32_t ne10, ne11, ne12, ne13;
    uint32_t nb11, nb12, nb13;
    uint32_t aoff, boff, doff;
    float eps;
    uint32_t multiply;
    uint32_t aligned;   // A and D 16-byte aligned
    uint32_t wAligned;  // the weight row 16-byte aligned
};

constexpr int kRmsCachedFloat4 = 8;  // rows of up to 2048 floats stay in registers

template <typename WT>
__device__ __forceinline__ float WeightAt(const WT* w, uint64_t i);

template <>
__device__ __forceinline__ float WeightAt<float>(const float* w, uint64_t i)
{
    return w[i];
}

template <>
__device__ __forceinline__ float WeightAt<uint16_t>(const uint16_t* w, uint64_t i)
{
    return HalfBitsToFloat(w[i]);
}

/// Four consecutive weights from element i (i % 4 == 0, the row 16-byte aligned).
template <typename WT>
__device__ __forceinline__ float4 LoadWeight4(const WT* w, uint64_t i);

template <>
__device__ __forceinline__ float4 LoadWeight4<float>(const float* w, uint64_t i)
{
    return *reinterpret_cast<const float4*>(w + i);
}

template <>
__device__ __forceinline__ float4 LoadWeight4<uint16_t>(const uint16_t* w, uint64_t i)
{
    const uint2 h = *reinterpret_cast<const uint2*>(w + i);
    return make_float4(HalfBitsToFloat(static_cast<uint16_t>(h.x & 0xFFFFu)), HalfBitsToFloat(static_cast<uint16_t>(h.x >> 16)),
                       HalfBitsToFloat(static_cast<uint16_t>(h.y & 0xFFFFu)), HalfBitsToFloat(static_cast<uint16_t>(h.y >> 16)));
}

__device__ __forceinline__ uint32_t ModIfNeeded(uint32_t a, uint32_t b) { return b == 0 ? 0 : a % b; }

template <typename WT>
__global__ __launch_bounds__(kBlock) void RmsNormRows(const float* __restrict__ a, const WT* __restrict__ w,
                                                      float* __restrict__ d, RmsArgs p)
{
    const uint32_t flat = blockIdx.x * kWaves + threadIdx.x / kWave;
    if (flat >= p.total)
    {
        return;  // whole wave exits together
    }
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t row = flat % p.nrows;
    const uint32_t channel = (flat / p.nrows) % p.nchannels;
    const uint32_t sample = flat / (p.nrows * p.nchannels);
    const uint64_t aOff = static_cast<uint64_t>(sample) * p.nb03 + static_cast<uint64_t>(channel) * p.nb02 +
                          static_cast<uint64_t>(row) * p.nb01 + p.aoff;
    const uint64_t bOff = static_cast<uint64_t>(ModIfNeeded(row, p.ne11)) * p.nb11 +
                          static_cast<uint64_t>(ModIfNeeded(channel, p.ne12)) * p.nb12 +
                          static_cast<uint64_t>(ModIfNeeded(sample, p.ne13)) * p.nb13 + p.boff;
    const uint64_t dOff = static_cast<uint64_t>(flat) * p.ncols + p.doff;
    const float* x = a + aOff;
    float* y = d + dOff;

    const bool vec = p.aligned && ((aOff | dOff | p.ncols) & 3u) == 0;
    const bool wrap = p.ncols > p.ne10;
    if (vec && p.ncols <= kRmsCachedFloat4 * 4 * kWave)
    {
        // The whole row in registers: one batch of loads, the sum, then the scaled row. The row is
        // read once and written once, so both stream past L2 (non-temporal); chunks past the row
        // are not requested.
        const uint32_t n4 = p.ncols / 4;
        const float4v* x4 = reinterpret_cast<const float4v*>(x);
        const bool weights4 = p.multiply && p.wAligned && !wrap && (bOff & 3u) == 0;
        float4v v[kRmsCachedFloat4];
#pragma unroll
        for (int k = 0; k < kRmsCachedFloat4; ++k)
        {
            const uint32_t i = lane + k * kWave;
            v[k] = i < n4 ? __builtin_nontemporal_load(x4 + i) : float4v{};
        }
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < kRmsCachedFloat4; ++k)
        {
            if (lane + k * kWave < n4)
            {
                sum = fmaf(v[k].x, v[k].x, sum);
                sum = fmaf(v[k].y, v[k].y, sum);
                sum = fmaf(v[k].z, v[k].z, sum);
                sum = fmaf(v[k].w, v[k].w, sum);
            }
        }
        sum = GroupSum<kWave>(sum);
        const float scale = 1.0f / sqrtf(sum / static_cast<float>(p.ncols) + p.eps);
#pragma unroll
        for (int k = 0; k < kRmsCachedFloat4; ++k)
        {
            const uint32_t i = lane + k * kWave;
            if (i < n4)
            {
                float4v o = {scale * v[k].x, scale * v[k].y, scale * v[k].z, scale * v[k].w};
                if (weights4)
                {
                    const float4 g = LoadWeight4<WT>(w, bOff + 4ull * i);
                    o = float4v{o.x * g.x, o.y * g.y, o.z * g.z, o.w * g.w};
                }
                else if (p.multiply)
                {
                    o.x *= WeightAt<WT>(w, bOff + (4 * i + 0) % p.ne10);
                    o.y *= WeightAt<WT>(w, bOff + (4 * i + 1) % p.ne10);
                    o.z *= WeightAt<WT>(w, bOff + (4 * i + 2) % p.ne10);
                    o.w *= WeightAt<WT>(w, bOff + (4 * i + 3) % p.ne10);
                }
                __builtin_nontemporal_store(o, reinterpret_cast<float4v*>(y) + i);
            }
        }
        return;
    }
    float sum = 0.0f;
    if (vec)
    {
        const uint32_t n4 = p.ncols / 4;
        for (uint32_t i = lane; i < n4; i += kWave)
        {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            sum = fmaf(v.x, v.x, sum);
            sum = fmaf(v.y, v.y, sum);
            sum = fmaf(v.z, v.z, sum);
            sum = fmaf(v.w, v.w, sum);
        }
    }
    else
    {
        for (uint32_t i = lane; i < p.ncols; i += kWave)
        {
            sum = fmaf(x[i], x[i], sum);
        }
    }
    sum = GroupSum<kWave>(sum);
    const float scale = 1.0f / sqrtf(sum / static_cast<float>(p.ncols) + p.eps);

    if (vec && !wrap && p.multiply && p.wAligned && (bOff & 3u) == 0 && sizeof(WT) == 4)
    {
        const uint32_t n4 = p.ncols / 4;
        const float4* w4 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + bOff);
        for (uint32_t i = lane; i < n4; i += kWave)
        {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            const float4 g = w4[i];
            float4 o;
            o.x = scale * v.x * g.x;
            o.y = scale * v.y * g.y;
            o.z = scale * v.z * g.z;
            o.w = scale * v.w * g.w;
            reinterpret_cast<float4*>(y)[i] = o;
        }
        return;
    }
    for (uint32_t i = lane; i < p.ncols; i += kWave)
    {
        float value = scale * x[i];
        if (p.multiply)
        {
            value *= WeightAt<WT>(w, bOff + (wrap ? i % p.ne10 : i));
        }
        y[i] = value;
    }
}

/// The common case, dense rows: flat row f at a + aoff + f * ncols and d + doff + f * ncols, one
/// weight row (or none), everything 16-byte aligned, ncols % 4 == 0 and ncols <= 4 * 64 * kChunks.
/// One wave per row, the row held in kChunks 16-byte chunks per lane: the same sums in the same
/// order as RmsNormRows's cached path, without its per-row index arithmetic and fallbacks.
template <typename WT, int kChunks, bool kMultiply>
__global__ __launch_bounds__(kBlock) void RmsNormDense(const float* __restrict__ a, const WT* __restrict__ w,
                                                       float* __restrict__ d, uint32_t rows, uint32_t ncols,
                                                       float eps)
{
    const uint32_t flat = blockIdx.x * kWaves + threadIdx.x / kWave;
    if (flat >= rows)
    {
        return;  // whole wave exits together
    }
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t n4 = ncols / 4;
    const float4v* x4 = reinterpret_cast<const float4v*>(a + static_cast<uint64_t>(flat) * ncols);
    float4v* y4 = reinterpret_cast<float4v*>(d + static_cast<uint64_t>(flat) * ncols);
    float4v v[kChunks];
#pragma unroll
    for (int k = 0; k < kChunks; ++k)
    {
        const uint32_t i = lane + k * kWave;
        v[k] = i < n4 ? __builtin_nontemporal_load(x4 + i) : float4v{};
    }
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kChunks; ++k)
    {
        sum = fmaf(v[k].x, v[k].x, sum);
        sum = fmaf(v[k].y, v[k].y, sum);
        sum = fmaf(v[k].z, v[k].z, sum);
        sum = fmaf(v[k].w, v[k].w, sum);
    }
    sum = GroupSum<kWave>(sum);
    const float scale = 1.0f / sqrtf(sum / static_cast<float>(ncols) + eps);
#pragma unroll
    for (int k = 0; k < kChunks; ++k)
    {
        const uint32_t i = lane + k * kWave;
        if (i < n4)
        {
            float4v o = {scale * v[k].x, scale * v[k].y, scale * v[k].z, scale * v[k].w};
            if constexpr (kMultiply)
            {
                const float4 g = LoadWeight4<WT>(w, 4ull * i);
                o = float4v{o.x * g.x, o.y * g.y, o.z * g.z, o.w * g.w};
            }
            __builtin_nontemporal_store(o, y4 + i);
        }
    }
}

template <typename WT, int kChunks>
void LaunchRmsNormDense(bool multiply, const float* a, const WT* w, float* d, uint32_t rows, uint32_t ncols, float eps,
                        hipStream_t s)
{
    if (multiply)
    {
        hipLaunchKernelGGL((RmsNormDense<WT, kChunks, true>), dim3(CeilDiv(rows, kWaves)), dim3(kBlock), 0, s, a, w,
                           d, rows, ncols, eps);
    }
    else
    {
        hipLaunchKernelGGL((RmsNormDense<WT, kChunks, false>), dim3(CeilDiv(rows, kWaves)), dim3(kBlock), 0, s, a, w,
                           d, rows, ncols, eps);
    }
}

template <typename WT>
int LaunchRmsNorm(const char* name, const LlamaAddPushConstants* pc, uint32_t doMultiply, const float* a,
                  const WT* b, float* d, uint32_t gx, uint32_t gy, uint32_t gz, void* stream)
{
    if (pc == nullptr || a == nullptr || d == nullptr || (doMultiply && b == nullptr))
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A, D (and B when multiplying) are required", name);
    }
    if (gx == 0 || gy == 0 || gz == 0 || pc->ne00 == 0)
    {
        return MUYO_OK;
    }
    if (doMultiply && pc->ne10 == 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: ne10 (weight length) must be >= 1", name);
    }
    // The dispatch is the tensor's (rows, channels, samples), as in ggml's {ne01, ne02, ne03}: a
    // larger one would index past A.
    if (gx > pc->ne01 || gy > pc->ne02 || gz > pc->ne03)
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch (%u, %u, %u) exceeds the tensor's (ne01, ne02, ne03) = (%u, %u, %u)",
                    name, gx, gy, gz, pc->ne01, pc->ne02, pc->ne03);
    }
    const uint64_t total = static_cast<uint64_t>(gx) * gy * gz;
    if (total > 0xFFFFFFFFull / kWave)
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch too large", name);
    }
    RmsArgs p{};
    p.ncols = pc->ne00;
    p.nrows = gx;
    p.nchannels = gy;
    p.total = static_cast<uint32_t>(total);
    p.nb01 = pc->nb01;
    p.nb02 = pc->nb02;
    p.nb03 = pc->nb03;
    p.ne10 = pc->ne10;
    p.ne11 = pc->ne11;
    p.ne12 = pc->ne12;
    p.ne13 = pc->ne13;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb13 = pc->nb13;
    p.aoff = pc->misalignOffsets >> 16;
    p.boff = (pc->misalignOffsets >> 8) & 0xFFu;
    p.doff = pc->misalignOffsets & 0xFFu;
    p.eps = pc->param1;
    p.multiply = doMultiply ? 1u : 0u;
    p.aligned = Aligned16(a) && Aligned16(d) ? 1u : 0u;
    p.wAligned = b != nullptr && Aligned16(b) ? 1u : 0u;
    // Dense rows (the flat row index is the memory row), one weight row: the streaming kernel.
    const uint32_t ncols = p.ncols;
    const bool denseA = (gx == 1 || p.nb01 == ncols) && (gy == 1 || p.nb02 == static_cast<uint64_t>(ncols) * gx) &&
                        (gz == 1 || p.nb03 == static_cast<uint64_t>(ncols) * gx * gy);
    const bool oneWeightRow = !doMultiply || (pc->ne11 <= 1 && pc->ne12 <= 1 && pc->ne13 <= 1 && p.ne10 == ncols &&
                                              p.wAligned && p.boff == 0);
    if (denseA && oneWeightRow && p.aligned && (ncols & 3u) == 0 && ((p.aoff | p.doff) & 3u) == 0 &&
        ncols <= 4 * kWave * kRmsCachedFloat4)
    {
        const float* aa = a + p.aoff;
        float* dd = d + p.doff;
        const hipStream_t s = AsStream(stream);
        if (ncols <= 4 * kWave * 4)
        {
            LaunchRmsNormDense<WT, 4>(doMultiply != 0, aa, b, dd, p.total, ncols, p.eps, s);
        }
        else
        {
            LaunchRmsNormDense<WT, kRmsCachedFloat4>(doMultiply != 0, aa, b, dd, p.total, ncols, p.eps, s);
        }
        return LaunchStatus(name);
    }
    hipLaunchKernelGGL((RmsNormRows<WT>), dim3(CeilDiv(total, kWaves)), dim3(kBlock), 0, AsStream(stream), a, b, d,
                       p);
    return LaunchStatus(name);
}

// ------------------------------------------------------------------------------------------------
// soft_max (shaders/llama/soft_max.comp:41-172).

struct SoftMaxArgs
{
    uint32_t kx, ky;
    uint32_t ne01, ne02, ne12, ne13;
    uint32_t nb11, nb12, nb13;
    float scale, maxBias, m0, m1;
    uint32_t nHeadLog2;
    uint32_t nrowsX;
    uint32_t hasSinks;
    uint32_t gx, gy, gz;  // dispatch
};

/// Row index of dispatch slot `slot` (z*262144 + y*512 + x for the workgroup it stands for).
__device__ __forceinline__ bool SlotRow(uint32_t slot, uint32_t gx, uint32_t gy, uint32_t& row)
{
    const uint32_t x = slot % gx;
    const uint32_t y = (slot / gx) % gy;
    const uint32_t z = slot / (gx * gy);
    row = z * 262144u + y * 512u + x;
    return true;
}

constexpr int kSoftMaxCache = 16;  // float4 per lane kept in registers (rows up to 4096)

__global__ __launch_bounds__(kBlock) void SoftMaxRows(const float* __restrict__ xIn, const float* __restrict__ mask,
                                                      const float* __restrict__ sinks, float* __restrict__ d,
                                                      SoftMaxArgs p)
{
    const uint32_t slot = blockIdx.x * kWaves + threadIdx.x / kWave;
    if (slot >= p.gx * p.gy * p.gz)
    {
        return;
    }
    uint32_t rowx;
    SlotRow(slot, p.gx, p.gy, rowx);
    if (rowx >= p.nrowsX)
    {
        return;
    }
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t i03 = rowx / (p.ne01 * p.ne02);
    const uint32_t i02 = (rowx - i03 * p.ne01 * p.ne02) / p.ne01;
    const uint32_t i01 = rowx % p.ne01;
    uint64_t rowyStart = 0;
    if (p.ky > 0)
    {
        rowyStart = static_cast<uint64_t>(i01) * p.nb11 + static_cast<uint64_t>(i02 % p.ne12) * p.nb12 +
                    static_cast<uint64_t>(i03 % p.ne13) * p.nb13;
    }
    float slope = 1.0f;
    if (p.maxBias > 0.0f)
    {
        const uint32_t h = (rowx / p.ne01) % p.ne02;
        const float base = h < p.nHeadLog2 ? p.m0 : p.m1;
        const uint32_t e = h < p.nHeadLog2 ? h + 1 : 2 * (h - p.nHeadLog2) + 1;
        slope = powf(base, static_cast<float>(e));
    }
    const float* x = xIn + static_cast<uint64_t>(rowx) * p.kx;
    float* y = d + static_cast<uint64_t>(rowx) * p.kx;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0 &&
                     (p.kx & 3u) == 0 && p.ky == 0;
    const uint32_t n4 = p.kx / 4;

    float maxValue = p.hasSinks ? sinks[i02] : -INFINITY;
    if (vec && n4 <= static_cast<uint32_t>(kSoftMaxCache * kWave))
    {
        float4 cache[kSoftMaxCache];
#pragma unroll
        for (int k = 0; k < kSoftMaxCache; ++k)
        {
            const uint32_t i = lane + k * kWave;
            if (i < n4)
            {
                // The row is read and written once: non-temporal both ways (4096 x 14 x 2048:
                // 5.1 -> 5.7 TB/s).
                const float4v t = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(x) + i);
                float4 v{t.x, t.y, t.z, t.w};
                v.x *= p.scale;
                v.y *= p.scale;
                v.z *= p.scale;
                v.w *= p.scale;
                cache[k] = v;
                maxValue = fmaxf(maxValue, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
            }
        }
        maxValue = GroupMax<kWave>(maxValue);
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < kSoftMaxCache; ++k)
        {
            const uint32_t i = lane + k * kWave;
            if (i < n4)
            {
                float4 v = cache[k];
                v.x = expf(v.x - maxValue);
                v.y = expf(v.y - maxValue);
                v.z = expf(v.z - maxValue);
                v.w = expf(v.w - maxValue);
                sum += (v.x + v.y) + (v.z + v.w);
                cache[k] = v;
            }
        }
        sum = GroupSum<kWave>(sum);
        if (p.hasSinks)
        {
            sum += expf(sinks[i02] - maxValue);
        }
        const float rcp = 1.0f / sum;
#pragma unroll
        for (int k = 0; k < kSoftMaxCache; ++k)
        {
            const uint32_t i = lane + k * kWave;
            if (i < n4)
            {
                float4 v = cache[k];
                v.x *= rcp;
                v.y *= rcp;
                v.z *= rcp;
                v.w *= rcp;
                __builtin_nontemporal_store(float4v{v.x, v.y, v.z, v.w}, reinterpret_cast<float4v*>(y) + i);
            }
        }
        return;
    }

    // General path: three passes over the row (re-reads hit cache).
    for (uint32_t c = lane; c < p.kx; c += kWave)
    {
        const float b = p.ky > 0 ? mask[rowyStart + c] : 0.0f;
        maxValue = fmaxf(maxValue, x[c] * p.scale + slope * b);
    }
    maxValue = GroupMax<kWave>(maxValue);
    float sum = 0.0f;
    for (uint32_t c = lane; c < p.kx; c += kWave)
    {
        const float b = p.ky > 0 ? mask[rowyStart + c] : 0.0f;
        sum += expf(x[c] * p.scale + slope * b - maxValue);
    }
    sum = GroupSum<kWave>(sum);
    if (p.hasSinks)
    {
        sum += expf(sinks[i02] - maxValue);
    }
    const float rcp = 1.0f / sum;
    for (uint32_t c = lane; c < p.kx; c += kWave)
    {
        const float b = p.ky > 0 ? mask[rowyStart + c] : 0.0f;
        y[c] = expf(x[c] * p.scale + slope * b - maxValue) * rcp;
    }
}

/// Checks a (x, y, z) row dispatch of the `z*262144 + y*512 + x` form: with y or z in use, x and
/// y must stay within 512 so distinct workgroups name distinct rows.
int CheckRowDispatch(const char* name, uint32_t gx, uint32_t gy, uint32_t gz)
{
    if ((gy > 1 || gz > 1) && (gx > 512 || gy > 512))
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch (%u, %u, %u) overlaps rows (x and y must be <= 512 when y or z > 1)",
                    name, gx, gy, gz);
    }
    return MUYO_OK;
}

// ------------------------------------------------------------------------------------------------
// argmax (shaders/llama/argmax.comp:20-60), ties to the lowest index.

struct ArgMaxArgs
{
    uint32_t kx, ky;
    uint32_t gx, gy, gz;
};

__global__ __launch_bounds__(kBlock) void ArgMaxRows(const float* __restrict__ a, int32_t* __restrict__ d,
                                                     ArgMaxArgs p)
{
    __shared__ float bestValue[kWaves];
    __shared__ int32_t bestIndex[kWaves];
    uint32_t row;
    SlotRow(blockIdx.x, p.gx, p.gy, row);
    if (row >= p.ky)
    {
        return;
    }
    const float* x = a + static_cast<uint64_t>(row) * p.kx;
    float value = -INFINITY;
    int32_t index = 0x7FFFFFFF;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    uint32_t start = 0;
    if (vec)
    {
        const uint32_t n4 = p.kx / 4;
        const float4v* x4 = reinterpret_cast<const float4v*>(x);
        uint32_t i = threadIdx.x;
        // Four non-temporal loads in flight per thread, taken in index order (4096 x 151936:
        // 6.1 -> 6.9 TB/s against one load at a time).
        for (; i + 3 * kBlock < n4; i += 4 * kBlock)
        {
            float4v v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                v[k] = __builtin_nontemporal_load(x4 + i + k * kBlock);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                // Within one thread indices only grow, so strict '>' keeps the lowest on ties.
                const int32_t base = static_cast<int32_t>((i + k * kBlock) * 4);
                if (v[k].x > value) { value = v[k].x; index = base; }
                if (v[k].y > value) { value = v[k].y; index = base + 1; }
                if (v[k].z > value) { value = v[k].z; index = base + 2; }
                if (v[k].w > value) { value = v[k].w; index = base + 3; }
            }
        }
        for (; i < n4; i += kBlock)
        {
            const float4v v = __builtin_nontemporal_load(x4 + i);
            const int32_t base = static_cast<int32_t>(i * 4);
            if (v.x > value) { value = v.x; index = base; }
            if (v.y > value) { value = v.y; index = base + 1; }
            if (v.z > value) { value = v.z; index = base + 2; }
            if (v.w > value) { value = v.w; index = base + 3; }
        }
        start = n4 * 4;
    }
    for (uint32_t i = start + threadIdx.x; i < p.kx; i += kBlock)
    {
        if (x[i] > value)
        {
            value = x[i];
            index = static_cast<int32_t>(i);
        }
    }
    GroupArgMax<kWave>(value, index);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0)
    {
        bestValue[wave] = value;
        bestIndex[wave] = index;
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        float v = bestValue[0];
        int32_t idx = bestIndex[0];
        for (int w = 1; w < kWaves; ++w)
        {
            if (bestValue[w] > v || (bestValue[w] == v && bestIndex[w] < idx))
            {
                v = bestValue[w];
                idx = bestIndex[w];
            }
        }
        // An all -inf (or empty) row has no strict maximum: the host scan returns index 0.
        d[row] = idx == 0x7FFFFFFF ? 0 : idx;
    }
}
}  // namespace
}  // namespace muyo

using namespace muyo;

extern "C" int muyo_rms_norm_f32(const LlamaAddPushConstants* pc, uint32_t do_multiply, const float* a,
                                 const float* b, float* d, float* /*partial_sums*/, uint32_t dispatch_x,
                                 uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    return LaunchRmsNorm<float>("rms_norm_f32", pc, do_multiply, a, b, d, dispatch_x, dispatch_y, dispatch_z, stream);
}

extern "C" int muyo_rms_norm_f32_f16w(const LlamaAddPushConstants* pc, uint32_t do_multiply, const float* a,
                                      const void* b, float* d, float* /*partial_sums*/, uint32_t dispatch_x,
                                      uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    return LaunchRmsNorm<uint16_t>("rms_norm_f32_f16w", pc, do_multiply, a, static_cast<const uint16_t*>(b), d,
                                   dispatch_x, dispatch_y, dispatch_z, stream);
}

extern "C" int muyo_soft_max_f32(const LlamaSoftMaxPushConstants* pc, const float* x, const float* mask,
                                 const float* sinks, float* d, uint32_t dispatch_x, uint32_t dispatch_y,
                                 uint32_t dispatch_z, void* stream)
{
    const char* name = "soft_max_f32";
    if (pc == nullptr || x == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, X and D are required", name);
    }
    if ((pc->KY > 0 && mask == nullptr) || (pc->hasSinks && sinks == nullptr))
    {
        return Fail(MUYO_E_NULL, "%s: the mask (KY > 0) or sinks (hasSinks) binding is NULL", name);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0 || pc->KX == 0)
    {
        return MUYO_OK;
    }
    if (pc->ne01 == 0 || pc->ne02 == 0 || (pc->KY > 0 && (pc->ne12 == 0 || pc->ne13 == 0)))
    {
        return Fail(MUYO_E_CONTRACT, "%s: ne01, ne02 (and ne12, ne13 with a mask) must be >= 1", name);
    }
    const int check = CheckRowDispatch(name, dispatch_x, dispatch_y, dispatch_z);
    if (check != MUYO_OK)
    {
        return check;
    }
    SoftMaxArgs p{};
    p.kx = pc->KX;
    p.ky = pc->KY;
    p.ne01 = pc->ne01;
    p.ne02 = pc->ne02;
    p.ne12 = pc->ne12;
    p.ne13 = pc->ne13;
    p.nb11 = pc->nb11;
    p.nb12 = pc->nb12;
    p.nb13 = pc->nb13;
    p.scale = pc->scale;
    p.maxBias = pc->maxBias;
    p.m0 = pc->m0;
    p.m1 = pc->m1;
    p.nHeadLog2 = pc->nHeadLog2;
    p.nrowsX = pc->nrowsX;
    p.hasSinks = pc->hasSinks;
    p.gx = dispatch_x;
    p.gy = dispatch_y;
    p.gz = dispatch_z;
    const uint64_t slots = static_cast<uint64_t>(dispatch_x) * dispatch_y * dispatch_z;
    hipLaunchKernelGGL(SoftMaxRows, dim3(CeilDiv(slots, kWaves)), dim3(kBlock), 0, AsStream(stream), x, mask, sinks, d,
                       p);
    return LaunchStatus(name);
}

extern "C" int muyo_argmax_f32(const LlamaGenericHeadPushConstants* pc, const float* a, int32_t* d,
                               uint32_t dispatch_x, uint32_t dispatch_y, uint32_t dispatch_z, void* stream)
{
    const char* name = "argmax_f32";
    if (pc == nullptr || a == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants, A and D are required", name);
    }
    if (dispatch_x == 0 || dispatch_y == 0 || dispatch_z == 0)
    {
        return MUYO_OK;
    }
    const int check = CheckRowDispatch(name, dispatch_x, dispatch_y, dispatch_z);
    if (check != MUYO_OK)
    {
        return check;
    }
    const uint64_t slots = static_cast<uint64_t>(dispatch_x) * dispatch_y * dispatch_z;
    if (slots > 0x7FFFFFFFull)
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch too large", name);
    }
    ArgMaxArgs p{pc->KX, pc->KY, dispatch_x, dispatch_y, dispatch_z};
    hipLaunchKernelGGL(ArgMaxRows, dim3(static_cast<uint32_t>(slots)), dim3(kBlock), 0, AsStream(stream), a, d, p);
    return LaunchStatus(name);
}
