// Device building blocks shared by the per-op GEMV (gemv.hip) and the fused decode GEMVs
// (decode_kernels.hip).
//
// A row of fp16 weights is streamed in 16-byte chunks (8 halves); lane `lir` of a kLpr-lane
// segment owns chunks lir, lir + kLpr, lir + 2*kLpr, ... . A "batch" is kCpl such chunks per
// lane, all issued as independent loads before any of them is used, so one batch costs one
// memory latency however long the row is. The activation sits in LDS in the split layout
// (low and high float4 of chunk c at lo[c] and hi[c]) so the per-lane float4 reads of
// consecutive chunks are consecutive and bank-conflict free.
#pragma once

#include "common.hpp"

namespace muyo
{
/// LDS slot of element i of an activation whose chunks are split into lo/hi float4 arrays.
__device__ __forceinline__ uint32_t SplitSlot(uint32_t i, uint32_t nchunks)
{
    const uint32_t c = i >> 3;
    const uint32_t r = i & 7u;
    return r < 4 ? c * 4 + r : (nchunks + c) * 4 + (r - 4);
}

/// Issue the loads of one batch: chunks base + lir + i*kLpr (i < kCpl) of `row`. Out-of-range
/// chunks load the row's last chunk instead (a cache hit) and are dropped in DotBatch, so the
/// batch is straight-line code: every load issues back to back and each FMA group waits only
/// for its own load.
template <int kLpr, int kCpl>
__device__ __forceinline__ void LoadBatch(const uint16_t* __restrict__ row, uint32_t base, uint32_t nchunks,
                                          uint32_t lir, half8 (&w)[kCpl])
{
    const half8* chunks = reinterpret_cast<const half8*>(row);
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
    {
        const uint32_t c = min(base + lir + i * kLpr, nchunks - 1);
        // Weights are streamed once per step: non-temporal, so they do not evict activations.
        w[i] = __builtin_nontemporal_load(chunks + c);
    }
}

/// Dot one loaded chunk (8 halves, widened exactly inside the FMA) with its 8 activations.
__device__ __forceinline__ float DotChunk(const half8& w, const float4& x0, const float4& x1, float acc)
{
    acc = fmaf(static_cast<float>(w[0]), x0.x, acc);
    acc = fmaf(static_cast<float>(w[1]), x0.y, acc);
    acc = fmaf(static_cast<float>(w[2]), x0.z, acc);
    acc = fmaf(static_cast<float>(w[3]), x0.w, acc);
    acc = fmaf(static_cast<float>(w[4]), x1.x, acc);
    acc = fmaf(static_cast<float>(w[5]), x1.y, acc);
    acc = fmaf(static_cast<float>(w[6]), x1.z, acc);
    acc = fmaf(static_cast<float>(w[7]), x1.w, acc);
    return acc;
}

/// Consume one loaded batch against the activation in LDS (chunks past the row add nothing).
template <int kLpr, int kCpl>
__device__ __forceinline__ float DotBatch(const half8 (&w)[kCpl], uint32_t base, uint32_t nchunks, uint32_t lir,
                                          const float4* __restrict__ lo, const float4* __restrict__ hi, float acc)
{
    float a[4] = {acc, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
    {
        const uint32_t c = base + lir + i * kLpr;
        const uint32_t cc = min(c, nchunks - 1);
        const float part = DotChunk(w[i], lo[cc], hi[cc], 0.0f);
        a[i & 3] += c < nchunks ? part : 0.0f;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

/// Sum of the squares of one chunk's 8 values, in element order.
__device__ __forceinline__ float SquaresOf(const float4& lo, const float4& hi)
{
    float part = 0.0f;
    part = fmaf(lo.x, lo.x, part);
    part = fmaf(lo.y, lo.y, part);
    part = fmaf(lo.z, lo.z, part);
    part = fmaf(lo.w, lo.w, part);
    part = fmaf(hi.x, hi.x, part);
    part = fmaf(hi.y, hi.y, part);
    part = fmaf(hi.z, hi.z, part);
    part = fmaf(hi.w, hi.w, part);
    return part;
}

__device__ __forceinline__ float4 MulF4(const float4& a, const float4& b)
{
    return float4{a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w};
}

/// The rms_norm factor of a row of n values whose squares sum to ss: rsqrt(mean(x^2) + eps), as
/// shaders/llama/rms_norm.comp:100 computes it. The fused GEMVs with a staged or direct norm multiply their row
/// sums by it after the dot: W . ((x * w) * scale) computed as (W . (x * w)) * scale.
__device__ __forceinline__ float NormScale(float ss, uint32_t n, float eps)
{
    return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

/// This lane's activation chunks (chunk lir + i*kLpr, clamped), read from LDS once and kept in
/// registers: a lane meets the same columns in every row it processes.
template <int kLpr, int kCpl>
__device__ __forceinline__ void LoadActivation(const float4* __restrict__ lo, const float4* __restrict__ hi,
                                               uint32_t nchunks, uint32_t lir, float4 (&xlo)[kCpl],
                                               float4 (&xhi)[kCpl])
{
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
    {
        const uint32_t c = min(lir + i * kLpr, nchunks - 1);
        xlo[i] = lo[c];
        xhi[i] = hi[c];
    }
}

struct NoOp
{
    __device__ void operator()() const {}
};

/// This lane's activation chunks (chunk lir + i*kLpr, clamped) read straight from global memory
/// into registers, for rows that one kLpr-lane segment covers (kLpr * kCpl >= n/8): no LDS and
/// no workgroup barrier. With kNorm the chunks become x * w (the rms_norm weight) and the return
/// value is this lane's part of sum(x^2): the caller reduces it over the segment together with
/// its dot products and multiplies the row sums by rsqrt(mean(x^2) + eps) at the end, so the
/// norm's reduction runs beside the dot instead of before it. Without kNorm it returns 0.
/// `between` runs once the loads are issued and before the norm waits for them: work that
/// overlaps their latency, or a kernel's weight loads, which then arrive after the activation
/// (loads complete in order). Scheduling barriers keep either side from moving across.
template <int kLpr, int kCpl, bool kNorm, class Between = NoOp>
__device__ __forceinline__ float LoadActivationDirect(const float* __restrict__ x, const float* __restrict__ w,
                                                      uint32_t n, uint32_t lir, float4 (&xlo)[kCpl],
                                                      float4 (&xhi)[kCpl], Between between = Between{})
{
    const uint32_t nchunks = n / 8;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 glo[kCpl];
    float4 ghi[kCpl];
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
    {
        const uint32_t c = min(lir + i * kLpr, nchunks - 1);
        xlo[i] = x4[2 * c];
        xhi[i] = x4[2 * c + 1];
        if constexpr (kNorm)
        {
            glo[i] = w4[2 * c];
            ghi[i] = w4[2 * c + 1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    between();
    __builtin_amdgcn_sched_barrier(0);
    float ss = 0.0f;
    if constexpr (kNorm)
    {
#pragma unroll
        for (int i = 0; i < kCpl; ++i)
        {
            ss += lir + i * kLpr < nchunks ? SquaresOf(xlo[i], xhi[i]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kCpl; ++i)
        {
            xlo[i] = MulF4(xlo[i], glo[i]);
            xhi[i] = MulF4(xhi[i], ghi[i]);
        }
    }
    return ss;
}

/// One loaded single-batch row against the activation in registers (chunks past the row add
/// nothing). The summation order is DotBatch's.
template <int kLpr, int kCpl>
__device__ __forceinline__ float DotRegisters(const half8 (&w)[kCpl], const float4 (&xlo)[kCpl],
                                              const float4 (&xhi)[kCpl], uint32_t nchunks, uint32_t lir)
{
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
    {
        const float part = DotChunk(w[i], xlo[i], xhi[i], 0.0f);
        a[i & 3] += lir + i * kLpr < nchunks ? part : 0.0f;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

/// The whole row's dot product for this lane, given its first batch already loaded in `w`.
/// Rows longer than one batch are double-buffered: batch k+1 is requested before batch k is
/// consumed, so a long row costs about one memory latency plus its streaming time.
template <int kLpr, int kCpl>
__device__ __forceinline__ float RowDot(const uint16_t* __restrict__ row, uint32_t nchunks, uint32_t lir,
                                        half8 (&w)[kCpl], const float4* __restrict__ lo,
                                        const float4* __restrict__ hi)
{
    constexpr uint32_t kBatch = kLpr * kCpl;
    if (nchunks <= kBatch)
    {
        return DotBatch<kLpr, kCpl>(w, 0, nchunks, lir, lo, hi, 0.0f);
    }
    // Ping-pong between `w` and `other` (no register copies): each half-iteration requests the
    // following batch into one buffer and consumes the other.
    float acc = 0.0f;
    half8 other[kCpl];
    uint32_t base = 0;
    for (;;)
    {
        uint32_t following = base + kBatch;
        if (following >= nchunks)
        {
            return DotBatch<kLpr, kCpl>(w, base, nchunks, lir, lo, hi, acc);
        }
        LoadBatch<kLpr, kCpl>(row, following, nchunks, lir, other);
        acc = DotBatch<kLpr, kCpl>(w, base, nchunks, lir, lo, hi, acc);
        base = following;
        following = base + kBatch;
        if (following >= nchunks)
        {
            return DotBatch<kLpr, kCpl>(other, base, nchunks, lir, lo, hi, acc);
        }
        LoadBatch<kLpr, kCpl>(row, following, nchunks, lir, w);
        acc = DotBatch<kLpr, kCpl>(other, base, nchunks, lir, lo, hi, acc);
        base = following;
    }
}

/// Stage an n-float activation (n % 8 == 0) into LDS in the split chunk layout with unrolled,
/// independent float4 loads (kVec per thread per round), so staging costs one memory latency.
/// With kNorm the staged values are x * w (the rms_norm weight) and the return value is the
/// row's rms_norm factor NormScale(sum(x^2)), which the caller applies to its row sums after the
/// dot; that path holds x and w in registers and needs n/4 <= kVec * threads. The sum of
/// squares meets across the waves through the same barrier that publishes the staged row.
/// Without kNorm it returns 1.
/// With kNorm, x may also be `parts` (at most kMaxParts) consecutive vectors of n floats
/// whose sum (added in order) is the activation; `sumOut`, when set, receives that sum. Ends
/// with the block synchronised.
/// `between` runs once the staging loads are issued and before any of them is used (with kNorm;
/// without, before the loads): a kernel issues its weight rows there, so that the activation,
/// requested first, arrives first (loads complete in order) and is staged while the weights are
/// in flight. Scheduling barriers keep the compiler from moving either group of loads across.
constexpr uint32_t kMaxStageParts = 4;

template <int kBlockThreads, int kVec, bool kNorm, class Between = NoOp, uint32_t kMaxParts = kMaxStageParts>
__device__ __forceinline__ float StageSplit(const float* __restrict__ x, const float* __restrict__ w, uint32_t n,
                                            float eps, float4* xs, uint32_t parts = 1, float* sumOut = nullptr,
                                            Between between = Between{})
{
    constexpr int kWaveCount = kBlockThreads / kWave;
    const uint32_t n4 = n / 4;
    const uint32_t nchunks = n / 8;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    if constexpr (!kNorm)
    {
        between();
        for (uint32_t first = 0; first < n4; first += kVec * kBlockThreads)
        {
            float4 v[kVec];
#pragma unroll
            for (int k = 0; k < kVec; ++k)
            {
                v[k] = x4[min(first + threadIdx.x + k * kBlockThreads, n4 - 1)];
            }
#pragma unroll
            for (int k = 0; k < kVec; ++k)
            {
                const uint32_t i = first + threadIdx.x + k * kBlockThreads;
                if (i < n4)
                {
                    // float4 i holds elements 4i..4i+3: chunk i/2, the low half when i is even.
                    xs[(i & 1u) ? nchunks + (i >> 1) : (i >> 1)] = v[k];
                }
            }
        }
    }
    else
    {
        __shared__ float partial[kWaveCount];
        const float4* w4 = reinterpret_cast<const float4*>(w);
        float4 v[kVec];
        float4 g[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k)
        {
            const uint32_t i = min(threadIdx.x + k * kBlockThreads, n4 - 1);
            v[k] = x4[i];
            g[k] = w4[i];
        }
        // Every part's loads go out before any is added: one latency for all of them.
        float4 more[kMaxParts - 1][kVec];
        if (parts > 1)
        {
#pragma unroll
            for (uint32_t p = 1; p < kMaxParts; ++p)
            {
#pragma unroll
                for (int k = 0; k < kVec; ++k)
                {
                    more[p - 1][k] = x4[min(p, parts - 1) * n4 + min(threadIdx.x + k * kBlockThreads, n4 - 1)];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        between();
        __builtin_amdgcn_sched_barrier(0);
        if (parts > 1)
        {
#pragma unroll
            for (uint32_t p = 1; p < kMaxParts; ++p)
            {
#pragma unroll
                for (int k = 0; k < kVec; ++k)
                {
                    if (p < parts)
                    {
                        v[k].x += more[p - 1][k].x;
                        v[k].y += more[p - 1][k].y;
                        v[k].z += more[p - 1][k].z;
                        v[k].w += more[p - 1][k].w;
                    }
                }
            }
        }
        if (sumOut != nullptr)
        {
            float4* s4 = reinterpret_cast<float4*>(sumOut);
#pragma unroll
            for (int k = 0; k < kVec; ++k)
            {
                if (threadIdx.x + k * kBlockThreads < n4)
                {
                    s4[threadIdx.x + k * kBlockThreads] = v[k];
                }
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < kVec; ++k)
        {
            if (threadIdx.x + k * kBlockThreads < n4)
            {
                ss = fmaf(v[k].x, v[k].x, ss);
                ss = fmaf(v[k].y, v[k].y, ss);
                ss = fmaf(v[k].z, v[k].z, ss);
                ss = fmaf(v[k].w, v[k].w, ss);
            }
        }
        // The products go to LDS while the sum of squares is reduced; one barrier publishes both.
#pragma unroll
        for (int k = 0; k < kVec; ++k)
        {
            const uint32_t i = threadIdx.x + k * kBlockThreads;
            if (i < n4)
            {
                xs[(i & 1u) ? nchunks + (i >> 1) : (i >> 1)] = MulF4(v[k], g[k]);
            }
        }
        ss = GroupSum<kWave>(ss);
        if constexpr (kWaveCount == 1)
        {
            __syncthreads();
            return NormScale(ss, n, eps);
        }
        else
        {
            if ((threadIdx.x & (kWave - 1)) == 0)
            {
                partial[threadIdx.x / kWave] = ss;
            }
            __syncthreads();
            float total = 0.0f;
#pragma unroll
            for (int k = 0; k < kWaveCount; ++k)
            {
                total += partial[k];
            }
            return NormScale(total, n, eps);
        }
    }
    __syncthreads();
    return 1.0f;
}

/// (lanes per row, chunks per lane per batch) for a row of `nchunks` 16-byte chunks, with at
/// least kNr rows per wave. One batch covers the row whenever it has at most 1024 chunks.
struct RowShape
{
    int lpr;
    int cpl;
};

inline RowShape PickRowShape(uint32_t nchunks, int nr)
{
    if (nchunks <= 64)
    {
        return {8, 8};
    }
    if (nchunks <= 128)
    {
        return {16, 8};
    }
    if (nchunks <= 256)
    {
        return {32, 8};
    }
    if (nr == 2)
    {
        return {32, 16};  // two rows per wave: at most 32 lanes each
    }
    if (nchunks <= 512)
    {
        return {64, 8};
    }
    if (nchunks <= 768)
    {
        return {64, 12};
    }
    return {64, 16};
}

/// The fused decode GEMVs' single-batch shape: one segment of `lpr` lanes streams every row of a
/// unit, each lane `cpl` chunks per row with the fewest chunks that cover the row (e.g. 896
/// columns = 112 chunks -> 16 lanes x 7; 3584 columns = 448 chunks -> 64 x 7; 4864 columns =
/// 608 chunks -> 64 x 10). cpl 0 means the row does not fit one batch within the register budget
/// of `nr` rows per unit.
inline RowShape PickFusedShape(uint32_t nchunks, int nr)
{
    static constexpr int kCpls[] = {7, 8, 10, 12, 14, 16};
    RowShape shape = PickRowShape(nchunks, 1);
    const int maxCpl = nr == 1 ? 16 : 10;
    for (int cpl : kCpls)
    {
        if (cpl <= maxCpl && static_cast<uint32_t>(shape.lpr * cpl) >= nchunks)
        {
            shape.cpl = cpl;
            return shape;
        }
    }
    shape.cpl = 0;
    return shape;
}
}  // namespace muyo
