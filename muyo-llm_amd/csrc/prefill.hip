// Batched-prefill kernels for gfx950: split-f16 GEMMs on v_mfma_f32_32x32x16_f16 with fused
// epilogues, a causal flash attention over the fp16 cache, and the row-wise glue (embedding,
// rms_norm into split planes, rope + cache append).
//
// Matrix-core lane layout of v_mfma_f32_32x32x16_f16 (D = A.B, A 32x16, B 16x32), as used below:
// lane l supplies A[l % 32][8 * (l / 32) .. +8] and B[8 * (l / 32) .. +8][l % 32], and receives
// D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32] in accumulator r (0..15).
#include <algorithm>
#include <cmath>
#include <initializer_list>
#include <type_traits>

#include "common.hpp"
#include "prefill.hpp"

namespace muyo
{
namespace
{
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef uint16_t ushort4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx16 Mfma(half8 a, half8 b, floatx16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

/// v = hi + lo to ~21 bits. hi is v with its 13 low mantissa bits cleared: 11 significant bits,
/// exact in f16. Rounding hi to f16 instead is not safe here: with contraction the compiler feeds
/// a product straight into v_fma_mix*_f16 (one rounding to f16) for one use and rounds it to f32
/// first (two roundings) for another, so the stored hi and the hi subtracted for lo can differ by
/// an f16 ulp near a tie. The bit mask works on the f32 value, and lo = v - hi is exact in f32
/// before its one rounding into f16. |v| must stay below 65536 (f16's range).
__device__ __forceinline__ float HiPart(float v) { return __uint_as_float(__float_as_uint(v) & 0xFFFFE000u); }

__device__ __forceinline__ _Float16 HiHalf(float v) { return static_cast<_Float16>(HiPart(v)); }

__device__ __forceinline__ _Float16 LoHalf(float v) { return static_cast<_Float16>(v - HiPart(v)); }

__device__ __forceinline__ void StoreSplit4(uint16_t* hi, uint16_t* lo, uint64_t at, float a, float b, float c,
                                            float d)
{
    const half4 h = {HiHalf(a), HiHalf(b), HiHalf(c), HiHalf(d)};
    const half4 l = {LoHalf(a), LoHalf(b), LoHalf(c), LoHalf(d)};
    *reinterpret_cast<half4*>(hi + at) = h;
    *reinterpret_cast<half4*>(lo + at) = l;
}

// ------------------------------------------------------------------------------------------------
// Row-wise glue.

__global__ __launch_bounds__(256) void EmbedRowsKernel(const uint16_t* __restrict__ table,
                                                       const int32_t* __restrict__ tokens, uint32_t hidden,
                                                       float* __restrict__ x, int32_t* history, int32_t pos0,
                                                       uint32_t historyCap)
{
    const uint32_t m = blockIdx.x;
    const int32_t token = tokens[m];
    const uint16_t* row = table + static_cast<uint64_t>(token) * hidden;
    float* out = x + static_cast<uint64_t>(m) * hidden;
    for (uint32_t i = threadIdx.x; i < hidden; i += 256)
    {
        out[i] = HalfBitsToFloat(row[i]);
    }
    const int64_t position = static_cast<int64_t>(pos0) + m;
    if (threadIdx.x == 0 && history != nullptr && position >= 0 && position < historyCap)
    {
        history[position] = token;
    }
}

/// The K splits of a split GEMM folded into its consumer: x = residual + (P_0 + P_1 + ...) in
/// split order, the unsplit epilogue's residual + sum.
struct SplitSum
{
    const float* residual;  // may be null
    const float* partial;   // [splits][rows][cols]
    uint32_t splits;
    uint64_t stride;        // rows * cols

    __device__ float4 At(uint64_t i) const
    {
        float4 a = *reinterpret_cast<const float4*>(partial + i);
        for (uint32_t z = 1; z < splits; ++z)
        {
            const float4 b = *reinterpret_cast<const float4*>(partial + z * stride + i);
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        if (residual != nullptr)
        {
            const float4 r = *reinterpret_cast<const float4*>(residual + i);
            a = make_float4(r.x + a.x, r.y + a.y, r.z + a.z, r.w + a.w);
        }
        return a;
    }
};

/// One wave per row: sum of squares across the wave, then (scale * x) * w split into planes. With
/// a split sum (splits > 0) the row is first reduced from its parts and stored to x; without w
/// only that.
__global__ __launch_bounds__(256) void RmsNormSplitKernel(float* __restrict__ x, const float* __restrict__ w,
                                                          uint32_t rows, uint32_t cols, float eps,
                                                          uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                          SplitSum sum)
{
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
    if (row >= rows)
    {
        return;
    }
    const uint32_t lane = threadIdx.x % kWave;
    float* xr = x + static_cast<uint64_t>(row) * cols;
    float ss = 0.0f;
    for (uint32_t i = lane * 4; i < cols; i += 4 * kWave)
    {
        float4 v;
        if (sum.splits > 0)
        {
            v = sum.At(static_cast<uint64_t>(row) * cols + i);
            *reinterpret_cast<float4*>(xr + i) = v;  // read back below by this lane only
        }
        else
        {
            v = *reinterpret_cast<const float4*>(xr + i);
        }
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (w == nullptr)
    {
        return;
    }
    ss = GroupSum<kWave>(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    for (uint32_t i = lane * 4; i < cols; i += 4 * kWave)
    {
        const float4 v = *reinterpret_cast<const float4*>(xr + i);
        const float4 g = *reinterpret_cast<const float4*>(w + i);
        StoreSplit4(hi, lo, static_cast<uint64_t>(row) * cols + i, (scale * v.x) * g.x, (scale * v.y) * g.y,
                    (scale * v.z) * g.z, (scale * v.w) * g.w);
    }
}

/// RmsNormSplitKernel with kT threads per row (one wave, or the whole 256-thread workgroup) and
/// at most kChunks 16-byte chunks of the row per thread, all requested before the first is used:
/// every K split's part, the residual and the weight in one round of loads instead of one round
/// per chunk. The sums run in SplitSum::At's order; the sum of squares meets across the row's
/// waves in LDS.
template <int kT>
__global__ __launch_bounds__(256) void RmsNormSplitRowsKernel(float* __restrict__ x, const float* __restrict__ w,
                                                              uint32_t rows, uint32_t cols, float eps,
                                                              uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                              SplitSum sum)
{
    constexpr int kChunks = 4;
    constexpr int kRowsPerBlock = 256 / kT;
    constexpr int kWavesPerRow = kT / kWave;
    __shared__ float squares[kRowsPerBlock * kWavesPerRow];
    const uint32_t row = blockIdx.x * kRowsPerBlock + threadIdx.x / kT;
    const uint32_t t = threadIdx.x % kT;
    const bool live = row < rows;
    const uint64_t base = static_cast<uint64_t>(live ? row : 0) * cols;
    float4 v[kChunks];
    float4 part[kMaxGemmSplits - 1][kChunks];
    float4 res[kChunks];
    float4 g[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
    {
        const uint32_t i = (t + c * kT) * 4;
        const bool in = i < cols;
        const uint64_t at = base + (in ? i : 0);
        v[c] = *reinterpret_cast<const float4*>((sum.splits > 0 ? sum.partial : x) + at);
#pragma unroll
        for (uint32_t z = 1; z < kMaxGemmSplits; ++z)
        {
            if (z < sum.splits)
            {
                part[z - 1][c] = *reinterpret_cast<const float4*>(sum.partial + z * sum.stride + at);
            }
        }
        if (sum.splits > 0 && sum.residual != nullptr)
        {
            res[c] = *reinterpret_cast<const float4*>(sum.residual + at);
        }
        if (w != nullptr)
        {
            g[c] = *reinterpret_cast<const float4*>(w + (in ? i : 0));
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
    {
        const uint32_t i = (t + c * kT) * 4;
        if (sum.splits > 0)
        {
#pragma unroll
            for (uint32_t z = 1; z < kMaxGemmSplits; ++z)
            {
                if (z < sum.splits)
                {
                    v[c].x += part[z - 1][c].x;
                    v[c].y += part[z - 1][c].y;
                    v[c].z += part[z - 1][c].z;
                    v[c].w += part[z - 1][c].w;
                }
            }
            if (sum.residual != nullptr)
            {
                v[c] = make_float4(res[c].x + v[c].x, res[c].y + v[c].y, res[c].z + v[c].z, res[c].w + v[c].w);
            }
            if (live && i < cols)
            {
                *reinterpret_cast<float4*>(x + base + i) = v[c];
            }
        }
        if (i < cols)
        {
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
        }
    }
    if (w == nullptr)
    {
        return;
    }
    ss = GroupSum<kWave>(ss);
    if constexpr (kWavesPerRow > 1)
    {
        const uint32_t wave = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0)
        {
            squares[wave] = ss;
        }
        __syncthreads();
        const uint32_t first = (threadIdx.x / kT) * kWavesPerRow;
        ss = 0.0f;
#pragma unroll
        for (int k = 0; k < kWavesPerRow; ++k)
        {
            ss += squares[first + k];
        }
    }
    if (!live)
    {
        return;
    }
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
    {
        const uint32_t i = (t + c * kT) * 4;
        if (i < cols)
        {
            StoreSplit4(hi, lo, base + i, (scale * v[c].x) * g[c].x, (scale * v[c].y) * g[c].y,
                        (scale * v[c].z) * g[c].z, (scale * v[c].w) * g[c].w);
        }
    }
}

/// The row kernel for `cols`: a wave per row up to 1024 columns, the workgroup per row up to 4096,
/// else the loop kernel.
hipError_t LaunchRmsNormSplitRows(hipStream_t s, float* x, const float* w, uint32_t rows, uint32_t cols, float eps,
                                  uint16_t* hi, uint16_t* lo, const SplitSum& sum)
{
    if (cols <= 4 * 4 * kWave)
    {
        hipLaunchKernelGGL(RmsNormSplitRowsKernel<kWave>, dim3(CeilDiv(rows, 4)), dim3(256), 0, s, x, w, rows, cols,
                           eps, hi, lo, sum);
    }
    else if (cols <= 4 * 4 * 256)
    {
        hipLaunchKernelGGL(RmsNormSplitRowsKernel<256>, dim3(rows), dim3(256), 0, s, x, w, rows, cols, eps, hi, lo,
                           sum);
    }
    else
    {
        hipLaunchKernelGGL(RmsNormSplitKernel, dim3(CeilDiv(rows, 4)), dim3(256), 0, s, x, w, rows, cols, eps, hi, lo,
                           sum);
    }
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void SplitF32Kernel(const float* __restrict__ x, uint64_t quads,
                                                      uint16_t* __restrict__ hi, uint16_t* __restrict__ lo)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < quads; i += static_cast<uint64_t>(gridDim.x) * 256)
    {
        const float4 v = *reinterpret_cast<const float4*>(x + 4 * i);
        StoreSplit4(hi, lo, 4 * i, v.x, v.y, v.z, v.w);
    }
}

/// The decode step's rope and cache append (rope_funcs.glsl:76-114; the fp16 cache rows of
/// src/FullModel.cpp:771-784) for many positions: one thread per (row, unit), units as in the
/// decode QKV epilogue: rope pairs (j, j + hd/2) of each q and k head, then pairs of v channels.
/// With splits > 1, qkv holds the K splits' raw sums ([splits][rows][width]) and each value is
/// their sum plus bias, the unsplit epilogue's acc + bias.
__global__ __launch_bounds__(256) void RopeSplitAppendKernel(const float* __restrict__ qkv, uint32_t rows,
                                                             int32_t pos0, uint32_t heads, uint32_t kvHeads,
                                                             uint32_t headDim, uint32_t maxSeq,
                                                             const float* __restrict__ ropePow,
                                                             uint16_t* __restrict__ qhi, uint16_t* __restrict__ qlo,
                                                             uint16_t* __restrict__ kcache,
                                                             uint16_t* __restrict__ vcache, uint32_t splits,
                                                             const float* __restrict__ bias)
{
    const uint32_t half = headDim / 2;
    const uint32_t ropeUnits = (heads + kvHeads) * half;
    const uint32_t units = (heads + 2 * kvHeads) * half;
    const uint64_t index = blockIdx.x * 256ull + threadIdx.x;
    if (index >= static_cast<uint64_t>(rows) * units)
    {
        return;
    }
    const uint32_t m = static_cast<uint32_t>(index / units);
    const uint32_t unit = static_cast<uint32_t>(index % units);
    const int32_t pos = pos0 + static_cast<int32_t>(m);
    const uint32_t width = (heads + 2 * kvHeads) * headDim;
    const float* row = qkv + static_cast<uint64_t>(m) * width;
    const uint64_t stride = static_cast<uint64_t>(rows) * width;
    auto value = [&](uint32_t col) {
        if (splits <= 1)
        {
            return row[col];
        }
        float a = row[col];
        for (uint32_t z = 1; z < splits; ++z)
        {
            a += row[z * stride + col];
        }
        return a + bias[col];
    };
    if (unit < ropeUnits)
    {
        const uint32_t head = unit / half;
        const uint32_t j = unit % half;
        const float s0 = value(head * headDim + j);
        const float s1 = value(head * headDim + j + half);
        const float theta = static_cast<float>(pos) * ropePow[j];
        float c;
        float sn;
        sincosf(theta, &sn, &c);
        const float o0 = s0 * c - s1 * sn;
        const float o1 = s0 * sn + s1 * c;
        if (head < heads)
        {
            const uint64_t at = static_cast<uint64_t>(m) * heads * headDim + head * headDim + j;
            const _Float16 h0 = HiHalf(o0);
            const _Float16 h1 = HiHalf(o1);
            qhi[at] = __builtin_bit_cast(uint16_t, h0);
            qlo[at] = __builtin_bit_cast(uint16_t, LoHalf(o0));
            qhi[at + half] = __builtin_bit_cast(uint16_t, h1);
            qlo[at + half] = __builtin_bit_cast(uint16_t, LoHalf(o1));
        }
        else
        {
            const uint64_t base = (static_cast<uint64_t>(head - heads) * maxSeq + pos) * headDim;
            kcache[base + j] = FloatToHalfBits(o0);
            kcache[base + j + half] = FloatToHalfBits(o1);
        }
    }
    else
    {
        const uint32_t channel = 2 * (unit - ropeUnits);  // within kvHeads * headDim
        const uint32_t g = channel / headDim;
        const uint64_t base = (static_cast<uint64_t>(g) * maxSeq + pos) * headDim + channel % headDim;
        const uint32_t v = (heads + kvHeads) * headDim + channel;
        vcache[base] = FloatToHalfBits(value(v));
        vcache[base + 1] = FloatToHalfBits(value(v + 1));
    }
}

/// RopeSplitAppendKernel with four pairs (or four v channels) per thread: 16-byte loads, 8-byte
/// stores and the same arithmetic per element (head_dim % 8 == 0, buffers aligned). The table of
/// powers is requested before the partial sums, so the angles are computed while the sums are
/// in flight (loads complete in order).
__global__ __launch_bounds__(256) void RopeSplitAppendQuadKernel(const float* __restrict__ qkv, uint32_t rows,
                                                                 int32_t pos0, uint32_t heads, uint32_t kvHeads,
                                                                 uint32_t headDim, uint32_t maxSeq,
                                                                 const float* __restrict__ ropePow,
                                                                 uint16_t* __restrict__ qhi, uint16_t* __restrict__ qlo,
                                                                 uint16_t* __restrict__ kcache,
                                                                 uint16_t* __restrict__ vcache, uint32_t splits,
                                                                 const float* __restrict__ bias)
{
    const uint32_t half = headDim / 2;
    const uint32_t quads = half / 4;
    const uint32_t ropeUnits = (heads + kvHeads) * quads;
    const uint32_t units = ropeUnits + kvHeads * headDim / 4;
    const uint64_t index = blockIdx.x * 256ull + threadIdx.x;
    if (index >= static_cast<uint64_t>(rows) * units)
    {
        return;
    }
    const uint32_t m = static_cast<uint32_t>(index / units);
    const uint32_t unit = static_cast<uint32_t>(index % units);
    const int32_t pos = pos0 + static_cast<int32_t>(m);
    const uint32_t width = (heads + 2 * kvHeads) * headDim;
    const float* row = qkv + static_cast<uint64_t>(m) * width;
    const uint64_t stride = static_cast<uint64_t>(rows) * width;
    auto value4 = [&](uint32_t col) {
        float4v a = *reinterpret_cast<const float4v*>(row + col);
        if (splits > 1)
        {
            for (uint32_t z = 1; z < splits; ++z)
            {
                a += *reinterpret_cast<const float4v*>(row + z * stride + col);
            }
            a += *reinterpret_cast<const float4v*>(bias + col);
        }
        return a;
    };
    if (unit < ropeUnits)
    {
        const uint32_t head = unit / quads;
        const uint32_t j = (unit % quads) * 4;
        const float4v power = *reinterpret_cast<const float4v*>(ropePow + j);
        const float4v s0 = value4(head * headDim + j);
        const float4v s1 = value4(head * headDim + j + half);
        float c[4];
        float sn[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            const float theta = static_cast<float>(pos) * power[e];
            sincosf(theta, &sn[e], &c[e]);
        }
        float o0[4];
        float o1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            o0[e] = s0[e] * c[e] - s1[e] * sn[e];
            o1[e] = s0[e] * sn[e] + s1[e] * c[e];
        }
        if (head < heads)
        {
            const uint64_t at = static_cast<uint64_t>(m) * heads * headDim + head * headDim + j;
            StoreSplit4(qhi, qlo, at, o0[0], o0[1], o0[2], o0[3]);
            StoreSplit4(qhi, qlo, at + half, o1[0], o1[1], o1[2], o1[3]);
        }
        else
        {
            const uint64_t base = (static_cast<uint64_t>(head - heads) * maxSeq + pos) * headDim + j;
            const ushort4v k0 = {FloatToHalfBits(o0[0]), FloatToHalfBits(o0[1]), FloatToHalfBits(o0[2]),
                                 FloatToHalfBits(o0[3])};
            const ushort4v k1 = {FloatToHalfBits(o1[0]), FloatToHalfBits(o1[1]), FloatToHalfBits(o1[2]),
                                 FloatToHalfBits(o1[3])};
            *reinterpret_cast<ushort4v*>(kcache + base) = k0;
            *reinterpret_cast<ushort4v*>(kcache + base + half) = k1;
        }
    }
    else
    {
        const uint32_t channel = 4 * (unit - ropeUnits);  // within kvHeads * headDim
        const uint32_t g = channel / headDim;
        const uint64_t base = (static_cast<uint64_t>(g) * maxSeq + pos) * headDim + channel % headDim;
        const float4v v = value4((heads + kvHeads) * headDim + channel);
        const ushort4v out = {FloatToHalfBits(v[0]), FloatToHalfBits(v[1]), FloatToHalfBits(v[2]),
                              FloatToHalfBits(v[3])};
        *reinterpret_cast<ushort4v*>(vcache + base) = out;
    }
}

// ------------------------------------------------------------------------------------------------
// Split GEMM: out[m][n] = sum_k (ahi + alo)[m][k] * W[n][k]. Each wave owns a 64 (n) x 64 (m)
// tile as 2 x 2 blocks of 32 x 32 accumulators; the weights are the matrix core's A operand
// (rows n), the activation planes its B operand (columns m), so a lane ends with four
// consecutive n of one m per accumulator group: 16-byte stores into row-major [m][n].
// K advances 64 halves at a time through one LDS tile per operand (rows padded to 144 bytes, so
// the 16-byte fragment reads of 8 consecutive rows touch distinct banks); the next tile's global
// loads are in flight while the current one is multiplied.

constexpr int kGemmBK = 64;
constexpr int kGemmStride = kGemmBK + 8;

/// out = acc + bias[n] + residual[m][n] (either may be null); virtual rows are the weight rows.
/// With `partial` the grid splits K (blockIdx.z) and each split stores its raw sums to plane z of
/// `partial` ([splits][rows][n]); bias and residual are then the consumer's to add.
struct PlainEpi
{
    const uint16_t* w;
    const float* bias;
    const float* residual;
    float* out;
    uint32_t n, k;
    float* partial = nullptr;

    /// Weight rows u + r (r < 16 or 32, u a multiple of that): row u's index and address, uniform
    /// across the workgroup (clamped to the last row); row u + r is r * k elements on.
    __device__ uint32_t WFirst(uint32_t u) const { return u; }
    __device__ uint32_t WCount() const { return n; }
    __device__ const uint16_t* WRows(uint32_t u) const { return w + static_cast<uint64_t>(min(u, n - 1)) * k; }

    template <int kNb>
    __device__ void Finish(const floatx16 (&acc)[kNb][2], uint32_t n0, uint32_t m0, uint32_t rows) const
    {
        const uint32_t lane = threadIdx.x % kWave;
        const uint32_t h = lane / 32;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
        {
            const uint32_t m = m0 + mb * 32 + lane % 32;
            if (m >= rows)
            {
                continue;
            }
#pragma unroll
            for (int nb = 0; nb < kNb; ++nb)
            {
#pragma unroll
                for (int g = 0; g < 4; ++g)
                {
                    const uint32_t nn = n0 + nb * 32 + 8 * g + 4 * h;
                    if (nn >= n)
                    {
                        continue;
                    }
                    float4 v = make_float4(acc[nb][mb][4 * g], acc[nb][mb][4 * g + 1], acc[nb][mb][4 * g + 2],
                                           acc[nb][mb][4 * g + 3]);
                    const uint64_t at = static_cast<uint64_t>(m) * n + nn;
                    if (partial != nullptr)
                    {
                        *reinterpret_cast<float4*>(partial + static_cast<uint64_t>(blockIdx.z) * rows * n + at) = v;
                        continue;
                    }
                    if (bias != nullptr)
                    {
                        const float4 b = *reinterpret_cast<const float4*>(bias + nn);
                        v.x += b.x;
                        v.y += b.y;
                        v.z += b.z;
                        v.w += b.w;
                    }
                    if (residual != nullptr)
                    {
                        const float4 r = *reinterpret_cast<const float4*>(residual + at);
                        v.x = r.x + v.x;
                        v.y = r.y + v.y;
                        v.z = r.z + v.z;
                        v.w = r.w + v.w;
                    }
                    *reinterpret_cast<float4*>(out + at) = v;
                }
            }
        }
    }
};

/// Gate and up interleaved per wave tile: virtual rows [64 t, 64 t + 32) are gate rows
/// [32 t, 32 t + 32) and the next 32 the same up rows, so a lane holds g and u of the same
/// (m, f) and writes silu(g) * u (swiglu.comp's op) as split planes.
struct SwiGluEpi
{
    const uint16_t* gate;
    const uint16_t* up;
    uint16_t* hhi;
    uint16_t* hlo;
    uint32_t ffn, k;

    /// Virtual rows u + r (r < 16 or 32, u a multiple of that) are gate or up rows f + r of one
    /// matrix, f = (u / 64) * 32 + u % 32: uniform across the workgroup (the address clamped to
    /// the last row).
    __device__ uint32_t WFirst(uint32_t u) const { return (u / 64) * 32 + u % 32; }
    __device__ uint32_t WCount() const { return ffn; }
    __device__ const uint16_t* WRows(uint32_t u) const
    {
        return (u % 64 < 32 ? gate : up) + static_cast<uint64_t>(min(WFirst(u), ffn - 1)) * k;
    }

    /// Blocks 2p and 2p + 1 of a wave's kNb are the gate and up rows of the same 32 f.
    template <int kNb>
    __device__ void Finish(const floatx16 (&acc)[kNb][2], uint32_t n0, uint32_t m0, uint32_t rows) const
    {
        const uint32_t lane = threadIdx.x % kWave;
        const uint32_t h = lane / 32;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
        {
            const uint32_t m = m0 + mb * 32 + lane % 32;
            if (m >= rows)
            {
                continue;
            }
#pragma unroll
            for (int p = 0; p < kNb / 2; ++p)
            {
#pragma unroll
                for (int g = 0; g < 4; ++g)
                {
                    const uint32_t f = (n0 + 64 * p) / 2 + 8 * g + 4 * h;
                    if (f >= ffn)
                    {
                        continue;
                    }
                    float a[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                    {
                        const float gv = acc[2 * p][mb][4 * g + t];
                        a[t] = gv / (1.0f + expf(-gv)) * acc[2 * p + 1][mb][4 * g + t];
                    }
                    StoreSplit4(hhi, hlo, static_cast<uint64_t>(m) * ffn + f, a[0], a[1], a[2], a[3]);
                }
            }
        }
    }
};

/// The grid's z splits K into runs of kPerSplit (a multiple of kGemmBK) columns. A wave owns 64
/// tokens and kNb blocks of 32 weight rows.
///
/// Workgroups are dispatched in linear order (x fastest), and those resident at once share what
/// they read through L2 and the Infinity Cache. By default the grid's x walks the weight tiles,
/// so consecutive workgroups share an activation tile. With `mFast` it walks the token tiles:
/// consecutive workgroups share a weight slice, so a weight larger than the cache (the 7B
/// gate+up's 272 MB) is read from HBM about once instead of once per round of resident token
/// tiles, while the activation planes, the smaller operand, stay cached.
template <int kWm, int kWn, typename Epi, int kNb = 2, int kStages = 1>
__global__ __launch_bounds__(kWave * kWm * kWn, kNb == 4 || kStages == 2 ? 2 : 1) void GemmSplitKernel(const uint16_t* __restrict__ ahi,
                                                                     const uint16_t* __restrict__ alo, Epi epi,
                                                                     uint32_t rows, uint32_t k, uint32_t kPerSplit,
                                                                     uint32_t mFast)
{
    constexpr int kThreads = kWave * kWm * kWn;
    constexpr int kBM = 64 * kWm;
    constexpr int kBN = 32 * kNb * kWn;
    constexpr int kChunks = kGemmBK / 8;  // 16-byte chunks per tile row
    constexpr int kALoads = 2 * kBM * kChunks / kThreads;
    constexpr int kWLoads = kBN * kChunks / kThreads;
    static_assert((2 * kBM * kChunks) % kThreads == 0 && (kBN * kChunks) % kThreads == 0, "tile loads");
    __shared__ __attribute__((aligned(16))) uint16_t lds[(2 * kBM + kBN) * kGemmStride];

    const uint32_t tid = threadIdx.x;
    const uint32_t linear = blockIdx.x + gridDim.x * blockIdx.y;
    const uint32_t m0 = (mFast != 0 ? linear % gridDim.y : blockIdx.y) * kBM;
    const uint32_t n0 = (mFast != 0 ? linear / gridDim.y : blockIdx.x) * kBN;

    // Each thread loads one 16-byte chunk (column `col`) of rows r0, r0 + kRowsPerPass, ... of the
    // A planes and of the weight. A row group's address is uniform across the workgroup and the
    // lane adds r0 * k + col, so the addresses cost one register (scalar base + vector offset)
    // rather than a 64-bit pointer per load. A lane whose row is past the matrix reads its group's
    // first row instead (in bounds; its products land in outputs that are not stored), so the
    // loads need no branches.
    constexpr uint32_t kRowsPerPass = kThreads / kChunks;
    static_assert(kBM % kRowsPerPass == 0 && 32 % kRowsPerPass == 0, "row groups");
    const uint32_t r0 = tid / kChunks;
    const uint32_t col = (tid % kChunks) * 8;
    const uint32_t laneOffset = r0 * k + col;
    const uint32_t dst = r0 * kGemmStride + col;

    const uint32_t kBegin = blockIdx.z * kPerSplit;
    const uint32_t kEnd = min(k, kBegin + kPerSplit);
    // kStages register buffers: the loads of tile t + kStages are issued as tile t's registers
    // reach LDS, so each load has kStages tiles of matrix-core work to arrive in.
    half8 aReg[kStages][kALoads];
    half8 wReg[kStages][kWLoads];
    auto load = [&](auto buf, uint32_t k0)
    {
        constexpr int b = decltype(buf)::value;
        // A chunk past kEnd (only in a K tile that runs past it) reads the tile's first chunk of
        // its row instead, and is zeroed below.
        const bool past = k0 + kGemmBK > kEnd && k0 + col >= kEnd;
        const uint32_t c = past ? 0u : col;
        const uint32_t offset = past ? r0 * k : laneOffset;
#pragma unroll
        for (int i = 0; i < kALoads; ++i)
        {
            const uint32_t plane = i * kRowsPerPass / kBM;
            const uint32_t row = m0 + i * kRowsPerPass % kBM;
            const uint16_t* base = (plane == 0 ? ahi : alo) + static_cast<uint64_t>(min(row, rows - 1)) * k + k0;
            aReg[b][i] = *reinterpret_cast<const half8*>(base + (row + r0 < rows ? offset : c));
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i)
        {
            const uint32_t u = n0 + i * kRowsPerPass;
            const uint16_t* base = epi.WRows(u) + k0;
            wReg[b][i] = *reinterpret_cast<const half8*>(base + (epi.WFirst(u) + r0 < epi.WCount() ? offset : c));
        }
        if (past)
        {
#pragma unroll
            for (int i = 0; i < kALoads; ++i)
            {
                aReg[b][i] = half8{};
            }
#pragma unroll
            for (int i = 0; i < kWLoads; ++i)
            {
                wReg[b][i] = half8{};
            }
        }
    };

    const uint32_t wave = tid / kWave;
    const uint32_t lane = tid % kWave;
    const uint32_t wm = wave / kWn;
    const uint32_t wn = wave % kWn;
    const uint32_t lrow = lane % 32;
    const uint32_t lk = (lane / 32) * 8;
    const uint16_t* wFrag = lds + (2 * kBM + wn * 32 * kNb + lrow) * kGemmStride + lk;
    const uint16_t* hiFrag = lds + (wm * 64 + lrow) * kGemmStride + lk;
    const uint16_t* loFrag = lds + (kBM + wm * 64 + lrow) * kGemmStride + lk;

    floatx16 acc[kNb][2];
#pragma unroll
    for (int a = 0; a < kNb; ++a)
    {
#pragma unroll
        for (int b = 0; b < 2; ++b)
        {
            acc[a][b] = floatx16{};
        }
    }

    // One tile: its registers to LDS, the refill of the same registers kStages tiles ahead, then
    // the tile's products.
    auto tile = [&](auto buf, uint32_t k0)
    {
        constexpr int b = decltype(buf)::value;
        __syncthreads();  // every wave is done with the previous tile
#pragma unroll
        for (int i = 0; i < kALoads; ++i)
        {
            // Plane p's row r sits at LDS row p * kBM + r, i.e. row i * kRowsPerPass + r0.
            *reinterpret_cast<half8*>(lds + dst + i * kRowsPerPass * kGemmStride) = aReg[b][i];
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i)
        {
            *reinterpret_cast<half8*>(lds + dst + (2 * kBM + i * kRowsPerPass) * kGemmStride) = wReg[b][i];
        }
        __syncthreads();
        if (k0 + kStages * kGemmBK < kEnd)
        {
            load(buf, k0 + kStages * kGemmBK);
        }
#pragma unroll
        for (int s = 0; s < kGemmBK / 16; ++s)
        {
            half8 wf[kNb], xh[2], xl[2];
#pragma unroll
            for (int b = 0; b < kNb; ++b)
            {
                wf[b] = *reinterpret_cast<const half8*>(wFrag + b * 32 * kGemmStride + s * 16);
            }
#pragma unroll
            for (int b = 0; b < 2; ++b)
            {
                xh[b] = *reinterpret_cast<const half8*>(hiFrag + b * 32 * kGemmStride + s * 16);
                xl[b] = *reinterpret_cast<const half8*>(loFrag + b * 32 * kGemmStride + s * 16);
            }
            // The hi products of every block, then the lo products, so that independent
            // matrix-core operations separate two that accumulate into the same block.
#pragma unroll
            for (int nb = 0; nb < kNb; ++nb)
            {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                {
                    acc[nb][mb] = Mfma(wf[nb], xh[mb], acc[nb][mb]);
                }
            }
#pragma unroll
            for (int nb = 0; nb < kNb; ++nb)
            {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                {
                    acc[nb][mb] = Mfma(wf[nb], xl[mb], acc[nb][mb]);
                }
            }
        }
    };

    using First = std::integral_constant<int, 0>;
    using Second = std::integral_constant<int, kStages - 1>;
    load(First{}, kBegin);
    if (kStages == 2 && kBegin + kGemmBK < kEnd)
    {
        load(Second{}, kBegin + kGemmBK);
    }
    for (uint32_t k0 = kBegin; k0 < kEnd; k0 += kStages * kGemmBK)
    {
        tile(First{}, k0);
        if (kStages == 2 && k0 + kGemmBK < kEnd)
        {
            tile(Second{}, k0 + kGemmBK);
        }
    }
    epi.Finish(acc, n0 + wn * 32 * kNb, m0 + wm * 64, rows);
}

/// 128 x 128 tiles when they, with the K splits, give two workgroups per CU, or unsplit fill at
/// least seven eighths of that (448 of 512 on 256 CUs); 64-token tiles otherwise.
bool BigTiles(uint32_t rows, uint32_t virtualRows, uint32_t splits = 1)
{
    const uint64_t tiles = static_cast<uint64_t>(CeilDiv(rows, 128)) * CeilDiv(virtualRows, 128);
    return tiles * splits >= 512 || (splits == 1 && tiles * 8 >= 512 * 7);
}

/// 128-token x 256-row tiles (a wave 64 tokens x 128 rows, two workgroups per CU) when they give
/// four workgroups per CU or more: an activation fragment read from LDS feeds twice the
/// matrix-core work. With fewer tiles the last round's imbalance costs more than that gains,
/// unless K splits make them one nearly full round (LaunchGemm).
bool WideTiles(uint32_t rows, uint32_t virtualRows)
{
    return static_cast<uint64_t>(CeilDiv(rows, 128)) * CeilDiv(virtualRows, 256) >= 1024;
}

template <typename Epi>
hipError_t LaunchGemm(hipStream_t s, const uint16_t* ahi, const uint16_t* alo, const Epi& epi, uint32_t rows,
                      uint32_t virtualRows, uint32_t k, uint32_t splits = 1)
{
    if (rows == 0 || virtualRows == 0 || k == 0 || splits == 0)
    {
        return hipErrorInvalidValue;
    }
    const uint32_t kPerSplit = CeilDiv(CeilDiv(k, kGemmBK), splits) * kGemmBK;
    // Token tiles fastest where the weight outweighs the activation planes and K is whole (the
    // gate+up GEMMs: 7B 1200 -> 1087 us; the K-split q|k|v and o_proj measured slower so).
    const uint32_t mFast = splits == 1 && static_cast<uint64_t>(virtualRows) * 2 > static_cast<uint64_t>(rows) * 4;
    const uint64_t wideSplits = static_cast<uint64_t>(CeilDiv(rows, 128)) * CeilDiv(virtualRows, 256) * splits;
    if (WideTiles(rows, virtualRows) || (splits > 1 && wideSplits * 8 >= 512 * 7 && wideSplits <= 512))
    {
        hipLaunchKernelGGL((GemmSplitKernel<2, 2, Epi, 4, 1>), dim3(CeilDiv(virtualRows, 256), CeilDiv(rows, 128), splits),
                           dim3(256), 0, s, ahi, alo, epi, rows, k, kPerSplit, mFast);
    }
    else if (BigTiles(rows, virtualRows, splits))
    {
        hipLaunchKernelGGL((GemmSplitKernel<2, 2, Epi, 2, 2>), dim3(CeilDiv(virtualRows, 128), CeilDiv(rows, 128), splits),
                           dim3(256), 0, s, ahi, alo, epi, rows, k, kPerSplit, mFast);
    }
    else
    {
        hipLaunchKernelGGL((GemmSplitKernel<1, 2, Epi, 2, 2>), dim3(CeilDiv(virtualRows, 128), CeilDiv(rows, 64), splits),
                           dim3(128), 0, s, ahi, alo, epi, rows, k, kPerSplit, mFast);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Causal flash attention. A workgroup owns one kv head, 32 consecutive queries and up to
// kHeadsPerBlock of the group's query heads, one per wave (a group of 7 takes two workgroups when
// one per tile would leave CUs idle); the waves share each 32-key tile of K and V through LDS (V
// stored transposed, channel-major). The next tile's rows are loaded into registers while the
// current one is multiplied, so a workgroup waits on memory once, not once per tile. Per wave
// and tile:
//   S^T (keys x queries) = K . Q^T on the matrix cores (K the A operand from LDS, Q the B operand
//   held in registers as split planes), so a lane holds 16 keys of one query and the online
//   softmax needs only one exchange with the lane 32 away;
//   O^T (channels x queries) += V^T . P^T with P^T split into planes straight from the S^T
//   accumulators: the B operand's k slot (h, v) of lane j + 32h is key 16 s + 8 (v / 4) + 4 h +
//   v % 4 of the tile, and the V^T fragment reads the same keys (two 8-byte LDS reads).

constexpr int kAttnKeys = 32;
constexpr uint32_t kAttnChunkTiles = 16;  // key tiles per chunk of a split query tile, at least

/// Key tiles (of kAttnKeys) a query tile attends to: cache rows 0 .. its last query's position.
__host__ __device__ inline uint32_t AttnKeyTiles(uint32_t qtile, uint32_t rows, int32_t pos0)
{
    const uint32_t last = qtile * 32 + 31 < rows ? qtile * 32 + 31 : rows - 1;
    return (static_cast<uint32_t>(pos0) + last) / kAttnKeys + 1;
}

/// Work items of the split prefill attention, passed by value in the kernel arguments.
struct AttnWork
{
    uint32_t count;       // items; 0: one item per query tile over all of its keys
    uint32_t chunkTiles;  // key tiles per chunk
    uint16_t tile[kAttnMaxItems];
    uint8_t chunk[kAttnMaxItems];
};

/// Softmax partials of the chunks of split tiles: [kAttnMaxChunks][rows][heads] (running max in
/// log2 units, sum) and [kAttnMaxChunks][rows][heads][headDim] (unnormalised P.V).
struct AttnPartials
{
    float* max;
    float* sum;
    float* acc;
};

/// Combines the chunk partials of the split tiles' queries into their output planes: out = sum_c
/// 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c, M the largest m_c (a chunk with no key of the query
/// weighs 0). A thread per (query, head, 4 channels); queries of unsplit tiles are left alone.
__global__ __launch_bounds__(256) void PrefillAttnMergeKernel(AttnPartials part, uint16_t* __restrict__ ohi,
                                                              uint16_t* __restrict__ olo, uint32_t rows, int32_t pos0,
                                                              uint32_t heads, uint32_t headDim, uint32_t chunkTiles)
{
    const uint32_t quads = headDim / 4;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rows) * heads * quads)
    {
        return;
    }
    const uint32_t channel = static_cast<uint32_t>(i % quads) * 4;
    const uint32_t head = static_cast<uint32_t>(i / quads % heads);
    const uint32_t m = static_cast<uint32_t>(i / quads / heads);
    const uint32_t keyTiles = AttnKeyTiles(m / 32, rows, pos0);
    if (keyTiles <= chunkTiles)
    {
        return;
    }
    const uint32_t chunks = (keyTiles + chunkTiles - 1) / chunkTiles;
    // Every slot's operands requested at once (slots past `chunks` reread slot 0 and weigh 0).
    float mc[kAttnMaxChunks];
    float lc[kAttnMaxChunks];
    float4 ac[kAttnMaxChunks];
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxChunks; ++c)
    {
        const uint64_t at = (static_cast<uint64_t>(c < chunks ? c : 0) * rows + m) * heads + head;
        mc[c] = part.max[at];
        lc[c] = part.sum[at];
        ac[c] = *reinterpret_cast<const float4*>(part.acc + at * headDim + channel);
    }
    float top = -INFINITY;
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxChunks; ++c)
    {
        top = c < chunks ? fmaxf(top, mc[c]) : top;
    }
    float den = 0.0f;
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxChunks; ++c)
    {
        if (c < chunks)
        {
            const float w = mc[c] == -INFINITY ? 0.0f : exp2f(mc[c] - top);
            den = fmaf(w, lc[c], den);
            num.x = fmaf(w, ac[c].x, num.x);
            num.y = fmaf(w, ac[c].y, num.y);
            num.z = fmaf(w, ac[c].z, num.z);
            num.w = fmaf(w, ac[c].w, num.w);
        }
    }
    const float inv = 1.0f / den;
    StoreSplit4(ohi, olo, static_cast<uint64_t>(m) * heads * headDim + head * headDim + channel, num.x * inv,
                num.y * inv, num.z * inv, num.w * inv);
}
// Halves per transposed V row. The even lane of each key pair stores both keys of a channel as one
// 4-byte word, so the 16 storing lanes of a channel chunk write 64 contiguous bytes; 36 halves
// (18 words) put the two chunks a wave stores at once 16 banks apart, and the MFMA fragment reads
// of 32 consecutive rows (8 bytes each, 18 words apart) cover every bank once.
constexpr int kVStride = kAttnKeys + 4;

/// Grid (head splits, work items, kv heads): the splits of one item are dispatched together.
/// Without work items (work.count 0) item y is query tile tiles - 1 - y over all of its keys (the
/// longest tiles first) and writes the output planes. With them, item y is query tile
/// work.tile[y] over key tiles [c * C, (c + 1) * C) of its range (c = work.chunk[y],
/// C = work.chunkTiles); a tile split over several chunks leaves each chunk's unnormalised
/// softmax partial (running max, sum, P.V) in slot c of `part` for PrefillAttnMergeKernel, a tile
/// of one chunk writes its planes directly. A causal tile's key range grows with its position, so
/// the split evens the workgroups' work: a 2048-token prompt is 64 tiles of 1..64 key tiles.
template <int kHd, int kHeadsPerBlock>
__global__ __launch_bounds__(kWave * kHeadsPerBlock) void PrefillAttentionKernel(
    const uint16_t* __restrict__ qhi, const uint16_t* __restrict__ qlo, const uint16_t* __restrict__ kcache,
    const uint16_t* __restrict__ vcache, uint16_t* __restrict__ ohi, uint16_t* __restrict__ olo, uint32_t rows,
    int32_t pos0, uint32_t heads, uint32_t kvHeads, uint32_t maxSeq, float scale, AttnWork work, AttnPartials part)
{
    constexpr int kKStride = kHd + 8;
    constexpr int kChunks = kHd / 8;
    constexpr int kThreads = kWave * kHeadsPerBlock;
    constexpr int kLoads = (kAttnKeys * kChunks + kThreads - 1) / kThreads;  // K (and V) chunks per thread per tile
    __shared__ __attribute__((aligned(16))) uint16_t kTile[kAttnKeys * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t vTile[kHd * kVStride];

    const uint32_t group = heads / kvHeads;
    const bool itemized = work.count > 0;
    const uint32_t qtile = itemized ? work.tile[blockIdx.y] : gridDim.y - 1 - blockIdx.y;  // longest first
    const uint32_t g = blockIdx.z;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t h = lane / 32;
    const uint32_t inGroup = blockIdx.x * kHeadsPerBlock + wave;
    const bool active = inGroup < group;  // a wave past the group only loads tiles
    const uint32_t head = g * group + (active ? inGroup : group - 1);
    const uint32_t qdim = heads * kHd;
    const uint32_t m0 = qtile * 32;
    const uint32_t mq = m0 + lane % 32 < rows ? m0 + lane % 32 : rows - 1;
    const int32_t qpos = pos0 + static_cast<int32_t>(mq);
    const int32_t lastPos = pos0 + static_cast<int32_t>(m0 + 31 < rows ? m0 + 31 : rows - 1);
    const uint32_t keyTiles = AttnKeyTiles(qtile, rows, pos0);
    const uint32_t chunk = itemized ? work.chunk[blockIdx.y] : 0;
    const uint32_t ktBegin = itemized ? chunk * work.chunkTiles : 0;
    const uint32_t ktEnd = itemized ? min(keyTiles, ktBegin + work.chunkTiles) : keyTiles;
    const bool partial = itemized && keyTiles > work.chunkTiles;  // the tile spans several chunks

    half8 qh[kHd / 16], ql[kHd / 16];
    {
        const uint64_t at = static_cast<uint64_t>(mq) * qdim + head * kHd + 8 * h;
#pragma unroll
        for (int s = 0; s < kHd / 16; ++s)
        {
            qh[s] = *reinterpret_cast<const half8*>(qhi + at + 16 * s);
            ql[s] = *reinterpret_cast<const half8*>(qlo + at + 16 * s);
        }
    }
    floatx16 o[kHd / 32];
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c)
    {
        o[c] = floatx16{};
    }
    float runMax = -INFINITY;  // log2 units: scores scaled by log2(e), weights 2^(s - max)
    float runSum = 0.0f;
    const float scaleLog2 = scale * 1.44269504088896340736f;
    const uint16_t* kBase = kcache + static_cast<uint64_t>(g) * maxSeq * kHd;
    const uint16_t* vBase = vcache + static_cast<uint64_t>(g) * maxSeq * kHd;

    half8 kReg[kLoads], vReg[kLoads];
    auto loadTile = [&](uint32_t kt) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
        {
            const uint32_t c = threadIdx.x + i * kThreads;
            const uint32_t r = c % kAttnKeys;               // key within the tile
            const uint32_t cc = (c / kAttnKeys) % kChunks;  // 8-channel chunk
            const uint32_t key = kt * kAttnKeys + r < maxSeq ? kt * kAttnKeys + r : maxSeq - 1;
            kReg[i] = *reinterpret_cast<const half8*>(kBase + static_cast<uint64_t>(key) * kHd + cc * 8);
            vReg[i] = *reinterpret_cast<const half8*>(vBase + static_cast<uint64_t>(key) * kHd + cc * 8);
        }
    };
    loadTile(ktBegin);
    for (uint32_t kt = ktBegin; kt < ktEnd; ++kt)
    {
        __syncthreads();  // every wave is done with the previous tile
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
        {
            const uint32_t c = threadIdx.x + i * kThreads;
            if (c < kAttnKeys * kChunks)
            {
                const uint32_t r = c % kAttnKeys;
                const uint32_t cc = c / kAttnKeys;
                *reinterpret_cast<half8*>(kTile + r * kKStride + cc * 8) = kReg[i];
            }
            // Rows past the tile's last query position may hold anything (NaN, inf): their weight
            // is 0, and 0 * NaN would poison every query of the tile, so they enter the V tile as
            // zeros. Their scores are masked to -inf by position. Lanes hold consecutive keys of a
            // chunk (c % 32), so the odd lane's row reaches its even partner by a quad permute
            // (lanes swapped in pairs) and the even lane stores both keys of each channel.
            const uint32_t r = c % kAttnKeys;
            const uint32_t cc = (c / kAttnKeys) % kChunks;
            const bool live = static_cast<int32_t>(kt * kAttnKeys + r) <= lastPos;
            const half8 v = live ? vReg[i] : half8{};
            uint32_t mine[4];
            __builtin_memcpy(mine, &v, sizeof(mine));
            uint32_t other[4];
#pragma unroll
            for (int d = 0; d < 4; ++d)
            {
                other[d] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                    static_cast<int>(mine[d]), static_cast<int>(mine[d]), 0xB1, 0xF, 0xF, false));
            }
            if (c < kAttnKeys * kChunks && (r & 1u) == 0)
            {
                uint32_t* row = reinterpret_cast<uint32_t*>(vTile) + ((cc * 8) * kVStride + r) / 2;
#pragma unroll
                for (int d = 0; d < 4; ++d)
                {
                    // Channel 2d: the low halves of this key and the next; channel 2d + 1: the high.
                    row[(2 * d) * (kVStride / 2)] = (mine[d] & 0xFFFFu) | (other[d] << 16);
                    row[(2 * d + 1) * (kVStride / 2)] = (mine[d] >> 16) | (other[d] & 0xFFFF0000u);
                }
            }
        }
        __syncthreads();
        if (kt + 1 < ktEnd)
        {
            loadTile(kt + 1);  // in flight while this tile is multiplied
        }
        if (!active)
        {
            continue;
        }

        floatx16 st = floatx16{};
        const uint16_t* kFrag = kTile + (lane % 32) * kKStride + 8 * h;
#pragma unroll
        for (int s = 0; s < kHd / 16; ++s)
        {
            const half8 kf = *reinterpret_cast<const half8*>(kFrag + 16 * s);
            st = Mfma(kf, qh[s], st);
            st = Mfma(kf, ql[s], st);
        }
        float p[16];
        float tileMax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int32_t key = static_cast<int32_t>(kt * kAttnKeys + 8 * (r / 4) + 4 * h + r % 4);
            p[r] = key <= qpos ? st[r] * scaleLog2 : -INFINITY;
            tileMax = fmaxf(tileMax, p[r]);
        }
        tileMax = fmaxf(tileMax, __shfl_xor(tileMax, 32));
        // Finite over a query's whole range (key 0 is in it), but a chunk of a split tile may hold
        // no key of a query yet: then nothing accumulates (factor 1, weights 0).
        const float newMax = fmaxf(runMax, tileMax);
        const bool none = newMax == -INFINITY;
        const float factor = none ? 1.0f : exp2f(runMax - newMax);
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            p[r] = none ? 0.0f : exp2f(p[r] - newMax);
            sum += p[r];
        }
        runSum = runSum * factor + sum;
        runMax = newMax;
#pragma unroll
        for (int c = 0; c < kHd / 32; ++c)
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                o[c][r] *= factor;
            }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
        {
            half8 ph, pl;
#pragma unroll
            for (int v = 0; v < 8; ++v)
            {
                ph[v] = HiHalf(p[8 * s + v]);
                pl[v] = LoHalf(p[8 * s + v]);
            }
#pragma unroll
            for (int c = 0; c < kHd / 32; ++c)
            {
                const _Float16* row =
                    reinterpret_cast<const _Float16*>(vTile) + (c * 32 + lane % 32) * kVStride + 16 * s + 4 * h;
                const half4 v0 = *reinterpret_cast<const half4*>(row);
                const half4 v1 = *reinterpret_cast<const half4*>(row + 8);
                const half8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[c] = Mfma(vf, ph, o[c]);
                o[c] = Mfma(vf, pl, o[c]);
            }
        }
    }

    const float total = runSum + __shfl_xor(runSum, 32);
    const uint32_t m = m0 + lane % 32;
    if (active && m < rows && partial)
    {
        // Slot `chunk`: the running max and sum of the query (both halves of the wave agree on
        // the max; their sums are added), and its unnormalised P.V.
        const uint64_t at = (static_cast<uint64_t>(chunk) * rows + m) * heads + head;
        if (h == 0)
        {
            part.max[at] = runMax;
            part.sum[at] = total;
        }
#pragma unroll
        for (int c = 0; c < kHd / 32; ++c)
        {
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const uint32_t channel = c * 32 + 8 * q + 4 * h;
                *reinterpret_cast<float4*>(part.acc + at * kHd + channel) =
                    make_float4(o[c][4 * q], o[c][4 * q + 1], o[c][4 * q + 2], o[c][4 * q + 3]);
            }
        }
    }
    else if (active && m < rows)
    {
        const float inv = 1.0f / total;
        const uint64_t base = static_cast<uint64_t>(m) * qdim + head * kHd;
#pragma unroll
        for (int c = 0; c < kHd / 32; ++c)
        {
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const uint32_t channel = c * 32 + 8 * q + 4 * h;
                StoreSplit4(ohi, olo, base + channel, o[c][4 * q] * inv, o[c][4 * q + 1] * inv,
                            o[c][4 * q + 2] * inv, o[c][4 * q + 3] * inv);
            }
        }
    }
}
}  // namespace

hipError_t LaunchEmbedRows(hipStream_t s, const uint16_t* table, const int32_t* tokens, uint32_t rows,
                           uint32_t hidden, float* x, int32_t* history, int32_t pos0, uint32_t historyCap)
{
    hipLaunchKernelGGL(EmbedRowsKernel, dim3(rows), dim3(256), 0, s, table, tokens, hidden, x, history, pos0,
                       historyCap);
    return hipGetLastError();
}

hipError_t LaunchRmsNormSplit(hipStream_t s, const float* x, const float* w, uint32_t rows, uint32_t cols, float eps,
                              uint16_t* hi, uint16_t* lo)
{
    if (rows == 0 || cols == 0 || cols % 4 != 0 || w == nullptr)
    {
        return hipErrorInvalidValue;
    }
    return LaunchRmsNormSplitRows(s, const_cast<float*>(x), w, rows, cols, eps, hi, lo, SplitSum{});
}

hipError_t LaunchReduceRmsNormSplit(hipStream_t s, const float* residual, const float* partial, uint32_t splits,
                                    float* x, const float* w, uint32_t rows, uint32_t cols, float eps, uint16_t* hi,
                                    uint16_t* lo)
{
    if (rows == 0 || cols == 0 || cols % 4 != 0 || splits == 0 || splits > kMaxGemmSplits || partial == nullptr)
    {
        return hipErrorInvalidValue;
    }
    const SplitSum sum{residual, partial, splits, static_cast<uint64_t>(rows) * cols};
    return LaunchRmsNormSplitRows(s, x, w, rows, cols, eps, hi, lo, sum);
}

hipError_t LaunchSplitF32(hipStream_t s, const float* x, uint64_t count, uint16_t* hi, uint16_t* lo)
{
    if (count == 0 || count % 4 != 0)
    {
        return hipErrorInvalidValue;
    }
    const uint64_t quads = count / 4;
    const uint32_t blocks = static_cast<uint32_t>(quads / 256 + 1 < 4096 ? quads / 256 + 1 : 4096);
    hipLaunchKernelGGL(SplitF32Kernel, dim3(blocks), dim3(256), 0, s, x, quads, hi, lo);
    return hipGetLastError();
}

uint32_t GemmSplits(uint32_t rows, uint32_t n, uint32_t k)
{
    if (rows == 0 || n == 0)
    {
        return 1;
    }
    const uint64_t bigTiles = static_cast<uint64_t>(CeilDiv(rows, 128)) * CeilDiv(n, 128);
    const bool halves = CeilDiv(k, kGemmBK) >= 8;
    // 128 x 128 tiles alone fill two workgroups per CU: K halves when under four per CU.
    if (bigTiles >= 512)
    {
        return bigTiles < 1024 && halves ? 2 : 1;
    }
    // 128 x 256 tiles over two K halves that fill seven eighths to all of one round (7B o_proj
    // and down, 448 workgroups): the wide tiles' matrix-core work per LDS read outweighs the
    // partial planes the next norm sums (o_proj + down 727 -> 614 us, the norms 18 -> 37 us).
    const uint64_t wideHalves = static_cast<uint64_t>(CeilDiv(rows, 128)) * CeilDiv(n, 256) * 2;
    if (halves && wideHalves * 8 >= 512 * 7 && wideHalves <= 512)
    {
        return 2;
    }
    // Otherwise at least seven eighths of one round of 128 x 128 tiles: unsplit, with no partial
    // planes for the next norm to sum.
    if (bigTiles * 8 >= 512 * 7)
    {
        return 1;
    }
    // 128 x 128 tiles over two K halves, where that grid fills two workgroups per CU.
    if (bigTiles * 2 >= 512 && halves)
    {
        return 2;
    }
    // 64-token tiles: waves of the unsplit grid (64 x 64 outputs each); short of ~1024 (a wave
    // per SIMD), K is split so the grid reaches it, keeping at least two K tiles per split.
    const uint64_t waves = static_cast<uint64_t>(CeilDiv(rows, 64)) * CeilDiv(n, 128) * 2;
    const uint32_t tiles = CeilDiv(k, kGemmBK);
    uint32_t splits = static_cast<uint32_t>(std::min<uint64_t>(kMaxGemmSplits, CeilDiv(1024, waves)));
    while (splits > 1 && tiles / splits < 2)
    {
        --splits;
    }
    return std::max(splits, 1u);
}

hipError_t LaunchGemmSplit(hipStream_t s, const uint16_t* ahi, const uint16_t* alo, const uint16_t* w,
                           const float* bias, const float* residual, float* out, uint32_t rows, uint32_t n,
                           uint32_t k, float* partial, uint32_t splits)
{
    if (n % 4 != 0 || k % 8 != 0 || splits == 0 || splits > kMaxGemmSplits || (splits > 1 && partial == nullptr))
    {
        return hipErrorInvalidValue;
    }
    PlainEpi epi{w, bias, residual, out, n, k};
    epi.partial = splits > 1 ? partial : nullptr;
    return LaunchGemm(s, ahi, alo, epi, rows, n, k, splits);
}

hipError_t LaunchGemmSwiGlu(hipStream_t s, const uint16_t* ahi, const uint16_t* alo, const uint16_t* wgate,
                            const uint16_t* wup, uint16_t* hhi, uint16_t* hlo, uint32_t rows, uint32_t ffn,
                            uint32_t k)
{
    if (ffn % 4 != 0 || k % 8 != 0)
    {
        return hipErrorInvalidValue;
    }
    // Two virtual rows (gate, up) per output, in whole 32-row blocks.
    const uint32_t virtualRows = 2 * CeilDiv(ffn, 32) * 32;
    return LaunchGemm(s, ahi, alo, SwiGluEpi{wgate, wup, hhi, hlo, ffn, k}, rows, virtualRows, k);
}

hipError_t LaunchRopeSplitAppend(hipStream_t s, const float* qkv, uint32_t rows, int32_t pos0, uint32_t heads,
                                 uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, const float* ropePow,
                                 uint16_t* qhi, uint16_t* qlo, uint16_t* kcache, uint16_t* vcache, uint32_t splits,
                                 const float* bias)
{
    const uint64_t total = static_cast<uint64_t>(rows) * (heads + 2 * kvHeads) * (headDim / 2);
    if (total == 0 || pos0 < 0 || static_cast<uint64_t>(pos0) + rows > maxSeq || splits == 0 ||
        splits > kMaxGemmSplits || (splits > 1 && bias == nullptr))
    {
        return hipErrorInvalidValue;
    }
    const auto aligned = [](const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; };
    if (headDim % 8 == 0 && aligned(qkv, 16) && aligned(ropePow, 16) && (bias == nullptr || aligned(bias, 16)) &&
        aligned(qhi, 8) && aligned(qlo, 8) && aligned(kcache, 8) && aligned(vcache, 8))
    {
        // Threads: four pairs of a rotated head each, or four v channels.
        const uint64_t quads = static_cast<uint64_t>(rows) * ((heads + kvHeads) * (headDim / 8) + kvHeads * headDim / 4);
        hipLaunchKernelGGL(RopeSplitAppendQuadKernel, dim3(CeilDiv(quads, 256)), dim3(256), 0, s, qkv, rows, pos0,
                           heads, kvHeads, headDim, maxSeq, ropePow, qhi, qlo, kcache, vcache, splits, bias);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(RopeSplitAppendKernel, dim3(CeilDiv(total, 256)), dim3(256), 0, s, qkv, rows, pos0, heads,
                       kvHeads, headDim, maxSeq, ropePow, qhi, qlo, kcache, vcache, splits, bias);
    return hipGetLastError();
}

hipError_t LaunchPrefillAttention(hipStream_t s, const uint16_t* qhi, const uint16_t* qlo, const uint16_t* kcache,
                                  const uint16_t* vcache, uint16_t* ohi, uint16_t* olo, uint32_t rows, int32_t pos0,
                                  uint32_t heads, uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq, float scale,
                                  float* workspace, size_t workspaceFloats)
{
    if (rows == 0 || kvHeads == 0 || heads % kvHeads != 0 || heads / kvHeads > 8 || pos0 < 0 ||
        static_cast<uint64_t>(pos0) + rows > maxSeq)
    {
        return hipErrorInvalidValue;
    }
    // A workgroup per (kv head, query tile) holding the whole group when that alone fills the chip
    // (7B shape: 256 workgroups, one K/V staging per tile for all 7 heads); otherwise groups past
    // four heads take two workgroups (0.5B shape: 128 -> 256).
    const uint32_t group = heads / kvHeads;
    int device = 0;
    int cus = 256;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    {
        cus = 256;
    }
    const uint32_t tiles = CeilDiv(rows, 32);
    const bool fills = static_cast<uint64_t>(tiles) * kvHeads >= static_cast<uint64_t>(cus);
    const uint32_t perBlock = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 || !fills ? 4 : 8;
    // Split the long tiles' key ranges into chunks of at least kAttnChunkTiles key tiles (and at
    // most kAttnMaxChunks per tile), items ordered longest first. Prompts whose chunks would not
    // fit kAttnMaxItems (past 2048 queries) run unsplit.
    AttnWork work{};
    AttnPartials part{};
    const uint32_t longest = AttnKeyTiles(tiles - 1, rows, pos0);
    const uint32_t chunkTiles = std::max(kAttnChunkTiles, CeilDiv(longest, kAttnMaxChunks));
    uint64_t items = 0;
    for (uint32_t t = 0; t < tiles; ++t)
    {
        items += CeilDiv(AttnKeyTiles(t, rows, pos0), chunkTiles);
    }
    if (workspace != nullptr && workspaceFloats >= PrefillAttentionWorkspaceFloats(rows, heads, headDim) &&
        longest > chunkTiles && items <= kAttnMaxItems)
    {
        work.chunkTiles = chunkTiles;
        for (uint32_t len = chunkTiles; len > 0 && work.count < kAttnMaxItems; --len)
        {
            for (uint32_t t = tiles; t-- > 0;)
            {
                const uint32_t keyTiles = AttnKeyTiles(t, rows, pos0);
                for (uint32_t c = 0; c * chunkTiles < keyTiles; ++c)
                {
                    if (std::min(chunkTiles, keyTiles - c * chunkTiles) == len && work.count < kAttnMaxItems)
                    {
                        work.tile[work.count] = static_cast<uint16_t>(t);
                        work.chunk[work.count] = static_cast<uint8_t>(c);
                        ++work.count;
                    }
                }
            }
        }
        const size_t stats = static_cast<size_t>(kAttnMaxChunks) * rows * heads;
        part = AttnPartials{workspace, workspace + stats, workspace + 2 * stats};
    }
    const dim3 grid(CeilDiv(group, perBlock), work.count > 0 ? work.count : tiles, kvHeads);
    const dim3 block(kWave * perBlock);
#define MUYO_PREFILL_ATTENTION(HD, P)                                                                         \
    if (headDim == HD && perBlock == P)                                                                       \
    {                                                                                                         \
        hipLaunchKernelGGL((PrefillAttentionKernel<HD, P>), grid, block, 0, s, qhi, qlo, kcache, vcache, ohi,  \
                           olo, rows, pos0, heads, kvHeads, maxSeq, scale, work, part);                       \
        if (work.count == 0)                                                                                  \
        {                                                                                                     \
            return hipGetLastError();                                                                         \
        }                                                                                                     \
        const uint64_t threads = static_cast<uint64_t>(rows) * heads * (headDim / 4);                         \
        hipLaunchKernelGGL(PrefillAttnMergeKernel, dim3(static_cast<uint32_t>(CeilDiv(threads, 256))),        \
                           dim3(256), 0, s, part, ohi, olo, rows, pos0, heads, headDim, work.chunkTiles);      \
        return hipGetLastError();                                                                             \
    }
    MUYO_PREFILL_ATTENTION(64, 1)
    MUYO_PREFILL_ATTENTION(64, 2)
    MUYO_PREFILL_ATTENTION(64, 4)
    MUYO_PREFILL_ATTENTION(64, 8)
    MUYO_PREFILL_ATTENTION(128, 1)
    MUYO_PREFILL_ATTENTION(128, 2)
    MUYO_PREFILL_ATTENTION(128, 4)
    MUYO_PREFILL_ATTENTION(128, 8)
#undef MUYO_PREFILL_ATTENTION
    return hipErrorInvalidValue;
}
}  // namespace muyo

// ------------------------------------------------------------------------------------------------
// C ABI (include/muyo_hip.h).

using namespace muyo;

namespace
{
bool AllAligned16(std::initializer_list<const void*> pointers)
{
    for (const void* p : pointers)
    {
        if (p != nullptr && !Aligned16(p))
        {
            return false;
        }
    }
    return true;
}

int Launched(hipError_t status, const char* name)
{
    return status == hipSuccess ? MUYO_OK : HipStatus(status, name);
}
}  // namespace

extern "C" int muyo_split_f32_f16x2(const float* x, uint64_t count, void* hi, void* lo, void* stream)
{
    const char* name = "split_f32_f16x2";
    if (x == nullptr || hi == nullptr || lo == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: x, hi and lo are required", name);
    }
    if (count == 0 || count % 4 != 0 || !AllAligned16({x, hi, lo}))
    {
        return Fail(MUYO_E_CONTRACT, "%s: count must be a positive multiple of 4 and the buffers 16-byte aligned",
                    name);
    }
    return Launched(LaunchSplitF32(AsStream(stream), x, count, static_cast<uint16_t*>(hi), static_cast<uint16_t*>(lo)),
                    name);
}

extern "C" int muyo_rms_norm_split_f16x2(const float* x, const float* w, uint32_t rows, uint32_t cols, float eps,
                                         void* hi, void* lo, void* stream)
{
    const char* name = "rms_norm_split_f16x2";
    if (x == nullptr || w == nullptr || hi == nullptr || lo == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: x, w, hi and lo are required", name);
    }
    if (rows == 0 || cols == 0 || cols % 4 != 0 || !AllAligned16({x, w, hi, lo}))
    {
        return Fail(MUYO_E_CONTRACT, "%s: rows >= 1, cols a positive multiple of 4, buffers 16-byte aligned", name);
    }
    return Launched(LaunchRmsNormSplit(AsStream(stream), x, w, rows, cols, eps, static_cast<uint16_t*>(hi),
                                       static_cast<uint16_t*>(lo)),
                    name);
}

extern "C" int muyo_gemm_split_f16(const void* a_hi, const void* a_lo, const void* w, const float* bias,
                                   const float* residual, float* out, uint32_t rows, uint32_t n, uint32_t k,
                                   void* stream)
{
    const char* name = "gemm_split_f16";
    if (a_hi == nullptr || a_lo == nullptr || w == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: a_hi, a_lo, w and out are required", name);
    }
    if (rows == 0 || n == 0 || k == 0 || n % 4 != 0 || k % 8 != 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: rows >= 1, n a positive multiple of 4, k of 8 (got %u x %u x %u)", name,
                    rows, n, k);
    }
    if (!AllAligned16({a_hi, a_lo, w, bias, residual, out}))
    {
        return Fail(MUYO_E_CONTRACT, "%s: every buffer must be 16-byte aligned", name);
    }
    return Launched(LaunchGemmSplit(AsStream(stream), static_cast<const uint16_t*>(a_hi),
                                    static_cast<const uint16_t*>(a_lo), static_cast<const uint16_t*>(w), bias,
                                    residual, out, rows, n, k),
                    name);
}

extern "C" int muyo_gemm_swiglu_split_f16(const void* a_hi, const void* a_lo, const void* w_gate, const void* w_up,
                                          void* h_hi, void* h_lo, uint32_t rows, uint32_t ffn, uint32_t k,
                                          void* stream)
{
    const char* name = "gemm_swiglu_split_f16";
    if (a_hi == nullptr || a_lo == nullptr || w_gate == nullptr || w_up == nullptr || h_hi == nullptr ||
        h_lo == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: every buffer is required", name);
    }
    if (rows == 0 || ffn == 0 || k == 0 || ffn % 4 != 0 || k % 8 != 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: rows >= 1, ffn a positive multiple of 4, k of 8 (got %u x %u x %u)", name,
                    rows, ffn, k);
    }
    if (!AllAligned16({a_hi, a_lo, w_gate, w_up, h_hi, h_lo}))
    {
        return Fail(MUYO_E_CONTRACT, "%s: every buffer must be 16-byte aligned", name);
    }
    return Launched(LaunchGemmSwiGlu(AsStream(stream), static_cast<const uint16_t*>(a_hi),
                                     static_cast<const uint16_t*>(a_lo), static_cast<const uint16_t*>(w_gate),
                                     static_cast<const uint16_t*>(w_up), static_cast<uint16_t*>(h_hi),
                                     static_cast<uint16_t*>(h_lo), rows, ffn, k),
                    name);
}

extern "C" int muyo_rope_split_append_f16kv(const float* qkv, uint32_t rows, int32_t pos0, uint32_t heads,
                                            uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq,
                                            const float* rope_pow, void* q_hi, void* q_lo, void* kcache,
                                            void* vcache, void* stream)
{
    const char* name = "rope_split_append_f16kv";
    if (qkv == nullptr || rope_pow == nullptr || q_hi == nullptr || q_lo == nullptr || kcache == nullptr ||
        vcache == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: every buffer is required", name);
    }
    if (rows == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || head_dim % 2 != 0)
    {
        return Fail(MUYO_E_CONTRACT, "%s: rows, heads, kv_heads >= 1 and an even head_dim are required", name);
    }
    if (pos0 < 0 || static_cast<uint64_t>(pos0) + rows > max_seq)
    {
        return Fail(MUYO_E_RANGE, "%s: positions %d..%lld exceed the cache (%u rows)", name, pos0,
                    static_cast<long long>(pos0) + rows - 1, max_seq);
    }
    return Launched(LaunchRopeSplitAppend(AsStream(stream), qkv, rows, pos0, heads, kv_heads, head_dim, max_seq,
                                          rope_pow, static_cast<uint16_t*>(q_hi), static_cast<uint16_t*>(q_lo),
                                          static_cast<uint16_t*>(kcache), static_cast<uint16_t*>(vcache)),
                    name);
}

namespace
{
int CheckPrefillAttentionArgs(const char* name, const void* q_hi, const void* q_lo, const void* kcache,
                              const void* vcache, const void* out_hi, const void* out_lo, uint32_t rows, int32_t pos0,
                              uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t max_seq)
{
    if (q_hi == nullptr || q_lo == nullptr || kcache == nullptr || vcache == nullptr || out_hi == nullptr ||
        out_lo == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: every buffer is required", name);
    }
    if (rows == 0 || kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > 8 ||
        (head_dim != 64 && head_dim != 128))
    {
        return Fail(MUYO_E_UNSUPPORTED, "%s: needs rows >= 1, heads %% kv_heads == 0, group <= 8, head_dim 64 or 128",
                    name);
    }
    if (pos0 < 0 || static_cast<uint64_t>(pos0) + rows > max_seq)
    {
        return Fail(MUYO_E_RANGE, "%s: positions %d..%lld exceed the cache (%u rows)", name, pos0,
                    static_cast<long long>(pos0) + rows - 1, max_seq);
    }
    if (!AllAligned16({q_hi, q_lo, kcache, vcache, out_hi, out_lo}))
    {
        return Fail(MUYO_E_CONTRACT, "%s: every buffer must be 16-byte aligned", name);
    }
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_prefill_attention_f16kv(const void* q_hi, const void* q_lo, const void* kcache,
                                            const void* vcache, void* out_hi, void* out_lo, uint32_t rows,
                                            int32_t pos0, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                            uint32_t max_seq, float scale, void* stream)
{
    const char* name = "prefill_attention_f16kv";
    const int args = CheckPrefillAttentionArgs(name, q_hi, q_lo, kcache, vcache, out_hi, out_lo, rows, pos0, heads,
                                               kv_heads, head_dim, max_seq);
    if (args != MUYO_OK)
    {
        return args;
    }
    return Launched(LaunchPrefillAttention(AsStream(stream), static_cast<const uint16_t*>(q_hi),
                                           static_cast<const uint16_t*>(q_lo), static_cast<const uint16_t*>(kcache),
                                           static_cast<const uint16_t*>(vcache), static_cast<uint16_t*>(out_hi),
                                           static_cast<uint16_t*>(out_lo), rows, pos0, heads, kv_heads, head_dim,
                                           max_seq, scale),
                    name);
}

extern "C" size_t muyo_prefill_attention_workspace_bytes(uint32_t rows, uint32_t heads, uint32_t head_dim)
{
    if (rows == 0 || heads == 0 || (head_dim != 64 && head_dim != 128))
    {
        return 0;
    }
    return PrefillAttentionWorkspaceFloats(rows, heads, head_dim) * sizeof(float);
}

extern "C" int muyo_prefill_attention_f16kv_ws(const void* q_hi, const void* q_lo, const void* kcache,
                                               const void* vcache, void* out_hi, void* out_lo, uint32_t rows,
                                               int32_t pos0, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                               uint32_t max_seq, float scale, void* workspace,
                                               uint64_t workspace_bytes, void* stream)
{
    const char* name = "prefill_attention_f16kv_ws";
    const int args = CheckPrefillAttentionArgs(name, q_hi, q_lo, kcache, vcache, out_hi, out_lo, rows, pos0, heads,
                                               kv_heads, head_dim, max_seq);
    if (args != MUYO_OK)
    {
        return args;
    }
    const size_t floats = PrefillAttentionWorkspaceFloats(rows, heads, head_dim);
    if (workspace == nullptr || !Aligned16(workspace) || workspace_bytes < floats * sizeof(float))
    {
        return Fail(MUYO_E_CONTRACT, "%s: needs a 16-byte aligned workspace of %zu bytes (got %llu)", name,
                    floats * sizeof(float), static_cast<unsigned long long>(workspace_bytes));
    }
    return Launched(LaunchPrefillAttention(AsStream(stream), static_cast<const uint16_t*>(q_hi),
                                           static_cast<const uint16_t*>(q_lo), static_cast<const uint16_t*>(kcache),
                                           static_cast<const uint16_t*>(vcache), static_cast<uint16_t*>(out_hi),
                                           static_cast<uint16_t*>(out_lo), rows, pos0, heads, kv_heads, head_dim,
                                           max_seq, scale, static_cast<float*>(workspace), floats),
                    name);
}
