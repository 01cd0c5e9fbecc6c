// mul_mat_vec_{f16,f32}_f32_f32: the per-op GEMV launchers.
//
// Contract (shaders/llama/mul_mat_vec.comp:141-264, mul_mat_vec_base.glsl:47-87,130-229):
//   d[dOff + row] = sum_k f32(A[aOff + row*ncols + k]) * B[bOff + k]  (+ FUSE0/FUSE1[dOff + row])
// with the batch offsets of get_offsets() and the A row stride fixed to ncols.
//
// gfx950 design: a wave64 splits into 64/LPR segments of LPR lanes; each segment owns one row
// per iteration and streams it in 16-byte chunks (8 halves or 4 floats per lane per load,
// coalesced across the segment). B is staged once per workgroup in LDS in a split layout
// (low and high float4 of each chunk in separate arrays) so the per-lane float4 reads are
// consecutive and bank-conflict free. Rows are grid-strided over the waves so the staging is
// amortised; segment sums are reduced with cross-lane shuffles.
#include <algorithm>

#include "common.hpp"
#include "decode_kernels.hpp"
#include "gemv_core.hpp"

namespace muyo
{
namespace
{
struct MatVecGeometry
{
    uint32_t ncols;
    uint32_t rows;
    uint32_t batchStrideA;
    uint32_t batchStrideB;
    uint32_t batchStrideD;
    uint32_t baseWorkGroupY;
    uint32_t ne02;
    uint32_t ne12;
    uint32_t broadcast2;
    uint32_t broadcast3;
    uint32_t fusion;
};

/// get_offsets() of mul_mat_vec_base.glsl:47-87 for the non-expert path.
__device__ __forceinline__ void BatchOffsets(const MatVecGeometry& g, uint32_t batch, uint64_t& a, uint64_t& b,
                                             uint64_t& d)
{
    const uint32_t index = batch + g.baseWorkGroupY;
    uint32_t indexA = 0;
    if (index != 0)
    {
        const uint32_t i13 = index / g.ne12;
        const uint32_t i12 = index % g.ne12;
        indexA = (i13 / g.broadcast3) * g.ne02 + i12 / g.broadcast2;
    }
    a = static_cast<uint64_t>(indexA) * g.batchStrideA;
    b = static_cast<uint64_t>(index) * g.batchStrideB;
    d = static_cast<uint64_t>(index) * g.batchStrideD;
}

template <typename AT>
struct Chunk;

template <>
struct Chunk<uint16_t>
{
    static constexpr int kElems = 8;
};

template <>
struct Chunk<float>
{
    static constexpr int kElems = 4;
};

/// One 16-byte chunk of A dotted with the matching x values from LDS.
template <typename AT>
__device__ __forceinline__ float ChunkDot(const AT* __restrict__ row, uint32_t chunk, const float4* __restrict__ lo,
                                          const float4* __restrict__ hi, float acc);

template <>
__device__ __forceinline__ float ChunkDot<uint16_t>(const uint16_t* __restrict__ row, uint32_t chunk,
                                                    const float4* __restrict__ lo, const float4* __restrict__ hi,
                                                    float acc)
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

template <>
__device__ __forceinline__ float ChunkDot<float>(const float* __restrict__ row, uint32_t chunk,
                                                 const float4* __restrict__ lo, const float4* __restrict__ /*hi*/,
                                                 float acc)
{
    const float4 w = *reinterpret_cast<const float4*>(row + static_cast<uint64_t>(chunk) * 4);
    const float4 x = lo[chunk];
    acc = fmaf(w.x, x.x, acc);
    acc = fmaf(w.y, x.y, acc);
    acc = fmaf(w.z, x.z, acc);
    acc = fmaf(w.w, x.w, acc);
    return acc;
}

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

template <int kLpr, typename AT>
__global__ __launch_bounds__(kBlock) void MatVecFast(const AT* __restrict__ a, const float* __restrict__ b,
                                                     float* __restrict__ d, const float* __restrict__ fuse0,
                                                     const float* __restrict__ fuse1, MatVecGeometry g)
{
    extern __shared__ float4 xs[];
    constexpr int kCe = Chunk<AT>::kElems;
    const uint32_t nchunks = g.ncols / kCe;
    float4* lo = xs;
    float4* hi = xs + nchunks;  // used by the 8-element chunks only

    uint64_t aOff, bOff, dOff;
    BatchOffsets(g, blockIdx.y, aOff, bOff, dOff);

    // Stage B: element i of chunk c goes to lo[c] (i < 4) or hi[c] (i >= 4).
    const float* x = b + bOff;
    float* xsFlat = reinterpret_cast<float*>(xs);
    for (uint32_t i = threadIdx.x; i < g.ncols; i += kBlock)
    {
        const uint32_t c = i / kCe;
        const uint32_t r = i % kCe;
        const uint32_t slot = r < 4 ? c * 4 + r : (nchunks + c) * 4 + (r - 4);
        xsFlat[slot] = x[i];
    }
    __syncthreads();

    constexpr int kRowsPerWave = kWave / kLpr;
    const int lane = threadIdx.x & (kWave - 1);
    const int segment = lane / kLpr;
    const int laneInRow = lane % kLpr;
    const uint32_t waveId = blockIdx.x * kWavesPerBlock + (threadIdx.x / kWave);
    const uint32_t waveCount = gridDim.x * kWavesPerBlock;
    const AT* aBase = a + aOff;

    for (uint32_t first = waveId * kRowsPerWave; first < g.rows; first += waveCount * kRowsPerWave)
    {
        const uint32_t row = first + segment;
        float acc = 0.0f;
        if (row < g.rows)
        {
            const AT* rowPtr = aBase + static_cast<uint64_t>(row) * g.ncols;
            uint32_t c = laneInRow;
            constexpr int kUnroll = 4;
            for (; c + (kUnroll - 1) * kLpr < nchunks; c += kUnroll * kLpr)
            {
                float part[kUnroll];
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                {
                    part[u] = ChunkDot<AT>(rowPtr, c + u * kLpr, lo, hi, 0.0f);
                }
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                {
                    acc += part[u];
                }
            }
            for (; c < nchunks; c += kLpr)
            {
                acc = ChunkDot<AT>(rowPtr, c, lo, hi, acc);
            }
        }
        acc = GroupSum<kLpr>(acc);
        if (laneInRow == 0 && row < g.rows)
        {
            float value = acc;
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS0)
            {
                value += fuse0[dOff + row];
            }
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS1)
            {
                value += fuse1[dOff + row];
            }
            d[dOff + row] = value;
        }
    }
}

/// fp16 A: every lane's chunks of a row issued as one batch (gemv_core.hpp); the first batch is
/// requested before B is staged, and the next row's batch before this row's reduction.
template <int kLpr, int kCpl>
__global__ __launch_bounds__(kBlock) void MatVecFastF16(const uint16_t* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ d, const float* __restrict__ fuse0,
                                                        const float* __restrict__ fuse1, MatVecGeometry g)
{
    extern __shared__ float4 xs[];
    const uint32_t nchunks = g.ncols / 8;
    constexpr int kRowsPerWave = kWave / kLpr;
    constexpr uint32_t kBatch = kLpr * kCpl;
    uint64_t aOff, bOff, dOff;
    BatchOffsets(g, blockIdx.y, aOff, bOff, dOff);
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t segment = lane / kLpr;
    const uint32_t lir = lane % kLpr;
    const uint32_t stride = gridDim.x * kWavesPerBlock * kRowsPerWave;
    const uint16_t* aBase = a + aOff;

    uint32_t first = (blockIdx.x * kWavesPerBlock + threadIdx.x / kWave) * kRowsPerWave;
    half8 w[kCpl];
    if (first + segment < g.rows)
    {
        LoadBatch<kLpr, kCpl>(aBase + static_cast<uint64_t>(first + segment) * g.ncols, 0, nchunks, lir, w);
    }
    StageSplit<kBlock, 8, false>(b + bOff, nullptr, g.ncols, 0.0f, xs);
    const float4* lo = xs;
    const float4* hi = xs + nchunks;

    for (; first < g.rows; first += stride)
    {
        const uint32_t row = first + segment;
        float acc = 0.0f;
        if (row < g.rows)
        {
            acc = DotBatch<kLpr, kCpl>(w, 0, nchunks, lir, lo, hi, 0.0f);
            for (uint32_t base = kBatch; base < nchunks; base += kBatch)
            {
                LoadBatch<kLpr, kCpl>(aBase + static_cast<uint64_t>(row) * g.ncols, base, nchunks, lir, w);
                acc = DotBatch<kLpr, kCpl>(w, base, nchunks, lir, lo, hi, acc);
            }
        }
        if (first + stride + segment < g.rows)
        {
            LoadBatch<kLpr, kCpl>(aBase + static_cast<uint64_t>(first + stride + segment) * g.ncols, 0, nchunks, lir,
                                  w);
        }
        acc = GroupSum<kLpr>(acc);
        if (lir == 0 && row < g.rows)
        {
            float value = acc;
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS0)
            {
                value += fuse0[dOff + row];
            }
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS1)
            {
                value += fuse1[dOff + row];
            }
            d[dOff + row] = value;
        }
    }
}

/// Any alignment, any ncols: one wave per row, scalar loads, B read from global memory.
template <typename AT>
__device__ __forceinline__ float LoadAsFloat(const AT* p);

template <>
__device__ __forceinline__ float LoadAsFloat<uint16_t>(const uint16_t* p)
{
    return HalfBitsToFloat(*p);
}

template <>
__device__ __forceinline__ float LoadAsFloat<float>(const float* p)
{
    return *p;
}

template <typename AT>
__global__ __launch_bounds__(kBlock) void MatVecGeneric(const AT* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ d, const float* __restrict__ fuse0,
                                                        const float* __restrict__ fuse1, MatVecGeometry g)
{
    uint64_t aOff, bOff, dOff;
    BatchOffsets(g, blockIdx.y, aOff, bOff, dOff);
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t waveId = blockIdx.x * kWavesPerBlock + (threadIdx.x / kWave);
    const uint32_t waveCount = gridDim.x * kWavesPerBlock;
    for (uint32_t row = waveId; row < g.rows; row += waveCount)
    {
        const AT* rowPtr = a + aOff + static_cast<uint64_t>(row) * g.ncols;
        float acc = 0.0f;
        for (uint32_t k = lane; k < g.ncols; k += kWave)
        {
            acc = fmaf(LoadAsFloat<AT>(rowPtr + k), b[bOff + k], acc);
        }
        acc = GroupSum<kWave>(acc);
        if (lane == 0)
        {
            float value = acc;
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS0)
            {
                value += fuse0[dOff + row];
            }
            if (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS1)
            {
                value += fuse1[dOff + row];
            }
            d[dOff + row] = value;
        }
    }
}

/// Lanes per row: enough that each lane streams at most ~8 chunks per row, within [8, 64].
int PickLanesPerRow(uint32_t nchunks)
{
    if (nchunks <= 64)
    {
        return 8;
    }
    if (nchunks <= 128)
    {
        return 16;
    }
    if (nchunks <= 256)
    {
        return 32;
    }
    return 64;
}

constexpr uint32_t kMaxLdsBytes = 160 * 1024;

template <typename Kernel>
hipError_t PrepareLds(Kernel kernel, size_t lds)
{
    if (lds > 64 * 1024)
    {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(lds));
    }
    return hipSuccess;
}

template <int kLpr, typename AT>
hipError_t LaunchFast(dim3 grid, size_t lds, hipStream_t stream, const AT* a, const float* b, float* d,
                      const float* fuse0, const float* fuse1, const MatVecGeometry& g)
{
    const hipError_t status = PrepareLds(&MatVecFast<kLpr, AT>, lds);
    if (status != hipSuccess)
    {
        return status;
    }
    hipLaunchKernelGGL((MatVecFast<kLpr, AT>), grid, dim3(kBlock), lds, stream, a, b, d, fuse0, fuse1, g);
    return hipGetLastError();
}

template <int kLpr, int kCpl>
hipError_t LaunchFastF16(uint32_t gy, size_t lds, hipStream_t stream, const uint16_t* a, const float* b, float* d,
                         const float* fuse0, const float* fuse1, const MatVecGeometry& g)
{
    const hipError_t status = PrepareLds(&MatVecFastF16<kLpr, kCpl>, lds);
    if (status != hipSuccess)
    {
        return status;
    }
    const uint32_t rowsPerBlock = kWavesPerBlock * (kWave / kLpr);
    const uint32_t blocks = std::max(1u, std::min(CeilDiv(g.rows, rowsPerBlock), 2048u));
    hipLaunchKernelGGL((MatVecFastF16<kLpr, kCpl>), dim3(blocks, gy, 1), dim3(kBlock), lds, stream, a, b, d, fuse0,
                       fuse1, g);
    return hipGetLastError();
}

hipError_t DispatchFastF16(uint32_t gy, size_t lds, hipStream_t stream, const uint16_t* a, const float* b, float* d,
                           const float* fuse0, const float* fuse1, const MatVecGeometry& g)
{
    const RowShape shape = PickRowShape(g.ncols / 8, 1);
#define MUYO_GEMV_CASE(L, C)                                                          \
    if (shape.lpr == L && shape.cpl == C)                                             \
    {                                                                                 \
        return LaunchFastF16<L, C>(gy, lds, stream, a, b, d, fuse0, fuse1, g);         \
    }
    MUYO_GEMV_CASE(8, 8)
    MUYO_GEMV_CASE(16, 8)
    MUYO_GEMV_CASE(32, 8)
    MUYO_GEMV_CASE(64, 8)
    MUYO_GEMV_CASE(64, 12)
    MUYO_GEMV_CASE(64, 16)
#undef MUYO_GEMV_CASE
    return hipErrorInvalidValue;
}

template <typename AT>
int LaunchMatVec(const char* name, const LlamaMatVecPushConstants* pc, const MuyoMatVecSpec* spec, const AT* a,
                 const float* b, float* d, const float* fuse0, const float* fuse1, uint32_t gx, uint32_t gy,
                 uint32_t gz, void* stream)
{
    if (pc == nullptr || a == nullptr || b == nullptr || d == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: push constants and bindings A, B, D are required", name);
    }
    if ((pc->fusionFlags & LLAMA_MAT_VEC_FUSION_BIAS0) && fuse0 == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: BIAS0 is set but FUSE0 is NULL", name);
    }
    if ((pc->fusionFlags & LLAMA_MAT_VEC_FUSION_BIAS1) && fuse1 == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: BIAS1 is set but FUSE1 is NULL", name);
    }
    const uint32_t numRows = spec != nullptr ? spec->numRows : 1u;
    const uint32_t numCols = spec != nullptr ? spec->numCols : 1u;
    if (numRows == 0 || numCols != 1)
    {
        return Fail(MUYO_E_UNSUPPORTED, "%s: NUM_ROWS must be >= 1 and NUM_COLS must be 1 (got %u, %u)", name, numRows,
                    numCols);
    }
    if (gx == 0 || gy == 0 || gz == 0)
    {
        return MUYO_OK;  // an empty dispatch does nothing
    }
    const uint64_t dispatched = static_cast<uint64_t>(numRows) * gx * gz;
    const uint32_t rows = static_cast<uint32_t>(std::min<uint64_t>(dispatched, pc->strideD));
    if (rows == 0)
    {
        return MUYO_OK;
    }
    if ((gy > 1 || pc->baseWorkGroupY != 0) && (pc->ne12 == 0 || pc->broadcast2 == 0 || pc->broadcast3 == 0))
    {
        return Fail(MUYO_E_CONTRACT, "%s: batched dispatch needs ne12, broadcast2 and broadcast3 >= 1", name);
    }
    if (gy > 65535)
    {
        return Fail(MUYO_E_DISPATCH, "%s: dispatch y %u exceeds 65535", name, gy);
    }

    MatVecGeometry g{};
    g.ncols = pc->ncols;
    g.rows = rows;
    g.batchStrideA = pc->batchStrideA;
    g.batchStrideB = pc->batchStrideB;
    g.batchStrideD = pc->batchStrideD;
    g.baseWorkGroupY = pc->baseWorkGroupY;
    g.ne02 = pc->ne02;
    g.ne12 = pc->ne12;
    g.broadcast2 = pc->broadcast2;
    g.broadcast3 = pc->broadcast3;
    g.fusion = pc->fusionFlags & (LLAMA_MAT_VEC_FUSION_BIAS0 | LLAMA_MAT_VEC_FUSION_BIAS1);

    constexpr uint32_t ce = Chunk<AT>::kElems;
    const bool offsetsAligned = (pc->batchStrideA % ce) == 0 || (gy == 1 && pc->baseWorkGroupY == 0);
    const size_t lds = static_cast<size_t>(g.ncols) * sizeof(float);
    // The fp16 kernel stages B with float4 loads: B's batch rows must start 16-byte aligned.
    const bool bAligned = Aligned16(b) && ((pc->batchStrideB % 4) == 0 || (gy == 1 && pc->baseWorkGroupY == 0));
    const bool fast = (g.ncols % ce) == 0 && Aligned16(a) && offsetsAligned && lds <= kMaxLdsBytes &&
                      (sizeof(AT) == 4 || bAligned);
    hipStream_t s = AsStream(stream);

    hipError_t status;
    if (fast && sizeof(AT) == 2 && gy == 1 && pc->baseWorkGroupY == 0)
    {
        // One batch: the decode step's fused GEMV with its launch-shape choice (register-direct
        // 64-thread workgroups for grids within the CUs, single-wave or whole-wave rows beyond).
        status = LaunchMatVecBias(s, reinterpret_cast<const uint16_t*>(a), b,
                                  (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS0) ? fuse0 : nullptr,
                                  (g.fusion & LLAMA_MAT_VEC_FUSION_BIAS1) ? fuse1 : nullptr, d, rows, g.ncols);
    }
    else if (fast && sizeof(AT) == 2)
    {
        status = DispatchFastF16(gy, lds, s, reinterpret_cast<const uint16_t*>(a), b, d, fuse0, fuse1, g);
    }
    else if (fast)
    {
        const uint32_t nchunks = g.ncols / ce;
        const int lpr = PickLanesPerRow(nchunks);
        const uint32_t rowsPerBlock = kWavesPerBlock * (kWave / lpr);
        const uint32_t blocks = std::max(1u, std::min(CeilDiv(rows, rowsPerBlock), 2048u));
        const dim3 grid(blocks, gy, 1);
        switch (lpr)
        {
            case 8:
                status = LaunchFast<8, AT>(grid, lds, s, a, b, d, fuse0, fuse1, g);
                break;
            case 16:
                status = LaunchFast<16, AT>(grid, lds, s, a, b, d, fuse0, fuse1, g);
                break;
            case 32:
                status = LaunchFast<32, AT>(grid, lds, s, a, b, d, fuse0, fuse1, g);
                break;
            default:
                status = LaunchFast<64, AT>(grid, lds, s, a, b, d, fuse0, fuse1, g);
                break;
        }
    }
    else
    {
        const uint32_t blocks = std::max(1u, std::min(CeilDiv(rows, kWavesPerBlock), 2048u));
        hipLaunchKernelGGL((MatVecGeneric<AT>), dim3(blocks, gy, 1), dim3(kBlock), 0, s, a, b, d, fuse0, fuse1, g);
        status = hipGetLastError();
    }
    return status == hipSuccess ? MUYO_OK : HipStatus(status, name);
}
}  // namespace
}  // namespace muyo

extern "C" int muyo_mul_mat_vec_f16_f32_f32(const LlamaMatVecPushConstants* pc, const MuyoMatVecSpec* spec,
                                            const void* a, const float* b, float* d, const float* fuse0,
                                            const float* fuse1, uint32_t dispatch_x, uint32_t dispatch_y,
                                            uint32_t dispatch_z, void* stream)
{
    return muyo::LaunchMatVec<uint16_t>("mul_mat_vec_f16_f32_f32", pc, spec, static_cast<const uint16_t*>(a), b, d,
                                        fuse0, fuse1, dispatch_x, dispatch_y, dispatch_z, stream);
}

extern "C" int muyo_mul_mat_vec_f32_f32_f32(const LlamaMatVecPushConstants* pc, const MuyoMatVecSpec* spec,
                                            const float* a, const float* b, float* d, const float* fuse0,
                                            const float* fuse1, uint32_t dispatch_x, uint32_t dispatch_y,
                                            uint32_t dispatch_z, void* stream)
{
    return muyo::LaunchMatVec<float>("mul_mat_vec_f32_f32_f32", pc, spec, a, b, d, fuse0, fuse1, dispatch_x,
                                     dispatch_y, dispatch_z, stream);
}
