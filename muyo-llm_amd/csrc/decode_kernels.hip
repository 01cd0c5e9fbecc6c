// Fused decode-step kernels for gfx950.
//
// One step (the reference records 18 nodes per layer, src/FullModel.cpp:726-993):
//   BeginStep      : greedy id of the previous step from the LM head's per-workgroup partials,
//                    step bookkeeping (position, generated-id ring), embedding row -> f32 x
//   per layer:
//   QkvRopeAppend  : rms_norm prologue -> fused q|k|v GEMV + bias -> NeoX rope of q and k ->
//                    q to a buffer, k and v appended as fp16 at the position's cache row
//   Attention      : one workgroup per (chunk, kv head, query head); blocks of keys dealt to the
//                    chunks round-robin, so the first K/V rows are requested before the position
//                    arrives; online softmax in log2 units; chunk partials (max, sum, P.V) to
//                    scratch (neutral for a chunk without keys)
//   [AttentionMerge: combine the chunk partials, when o_proj does not do it itself]
//   OProj          : [merge prologue] o_proj GEMV + residual add; or, split by kv group, each
//                    workgroup merging its group's partials, one partial hidden state per group
//   GateUpSwiGlu   : rms_norm prologue (summing the o_proj group parts) -> gate and up GEMV
//                    rows -> silu(g)*u
//   Down           : down GEMV + residual add
//   (FfnFused      : gate/up, swiglu and down in one launch on decoders with a hidden size of at
//                    most 1024: each workgroup's slice of the down product is added with atomics
//                    into partial vectors of the hidden state, which the next layer sums)
//   LmHeadArgMax   : final rms_norm prologue -> tied LM head -> logits + per-workgroup argmax
//
// GEMV core (gemv_core.hpp): a wave64 splits into segments of LPR lanes, each segment streaming
// one fp16 weight row in 16-byte chunks with all of a lane's loads in flight at once; the first
// batch is requested before the activation is staged (in LDS, or per lane straight from memory)
// and the next row's batch before the current row's reduction. Work that does not depend on the
// dot products (the rope angle's cosine and sine) runs while the loads are in flight.
#include <algorithm>
#include <atomic>
#include <mutex>

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
constexpr int kStageVec = 8;           // float4 per thread per staging round at most (rows <= 8192 floats)
constexpr int kMaxGroup = 8;           // query heads per kv head
constexpr int kDirectThreads = 64;  // workgroup size of the register-direct GEMVs
constexpr uint32_t kNoLimit = 0xFFFFFFFFu;
constexpr uint32_t kWideUnits = 2048;  // most units of a short-row GEMV launched a wave per unit
constexpr uint32_t kMergeItems = 4;    // q channels per thread in the o_proj merge prologue (q dim <= 1024)

// Host-side launch caches are kept per device (the current device of the calling thread) and
// are safe to use from several host threads: device attributes are read once per device, and
// each GEMV kernel's occupancy and LDS opt-in are tracked per device under that kernel's lock.
constexpr int kMaxDevices = 64;

int CurrentDevice()
{
    int device = 0;
    return hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices ? device : 0;
}

/// CUs of the current device, read once per device (threads racing on the first read store the
/// same value).
uint32_t CuCount()
{
    static std::atomic<uint32_t> cus[kMaxDevices];
    const int device = CurrentDevice();
    uint32_t count = cus[device].load(std::memory_order_relaxed);
    if (count == 0)
    {
        int value = 0;
        if (hipDeviceGetAttribute(&value, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || value <= 0)
        {
            value = 256;
        }
        count = static_cast<uint32_t>(value);
        cus[device].store(count, std::memory_order_relaxed);
    }
    return count;
}

// ------------------------------------------------------------------------------------------------
// Activation staging policies (each fills the LDS split layout and ends synchronised).
//
// A norm stage (kNorm) stages x * w, the rms_norm weight applied but not the row's factor
// rsqrt(mean(x^2) + eps): the kernels multiply their row sums by that factor after the dot, so
// the norm's reduction overlaps the weight stream instead of standing between the activation's
// arrival and the first product. Run returns the factor (1 without a norm); Direct returns this
// lane's part of sum(x^2) (0 without a norm), which the kernel reduces with its dot products.
// The column-quarter kernel (FusedMatVecColumns) keeps a prologue of its own that scales x.

struct PlainStage
{
    const float* x;
    static constexpr bool kCanDirect = true;  // see DirectStage
    static constexpr bool kDirect = false;
    static constexpr bool kElementwise = true;  // any column range stages on its own
    static constexpr bool kNorm = false;
    template <int kLpr, int kCpl, class Between>
    __device__ float Direct(uint32_t n, uint32_t lir, float4 (&xlo)[kCpl], float4 (&xhi)[kCpl], Between between) const
    {
        return LoadActivationDirect<kLpr, kCpl, false>(x, nullptr, n, lir, xlo, xhi, between);
    }
    template <int kThreads, int kVec, class Between = NoOp>
    __device__ float Run(float4* xs, uint32_t n, Between between = Between{}) const
    {
        return StageSplit<kThreads, kVec, false>(x, nullptr, n, 0.0f, xs, 1, nullptr, between);
    }
};

struct NormStage
{
    const float* x;
    const float* w;
    float eps;
    static constexpr bool kCanDirect = true;
    static constexpr bool kDirect = false;
    static constexpr bool kElementwise = false;  // the norm needs the whole row
    static constexpr bool kNorm = true;
    template <int kLpr, int kCpl, class Between>
    __device__ float Direct(uint32_t n, uint32_t lir, float4 (&xlo)[kCpl], float4 (&xhi)[kCpl], Between between) const
    {
        return LoadActivationDirect<kLpr, kCpl, true>(x, w, n, lir, xlo, xhi, between);
    }
    template <int kThreads, int kVec, class Between = NoOp>
    __device__ float Run(float4* xs, uint32_t n, Between between = Between{}) const
    {
        return StageSplit<kThreads, kVec, true>(x, w, n, eps, xs, 1, nullptr, between);
    }
};

/// NormStage over a hidden state held as kResidualParts partial vectors laid end to end (the fused
/// feed-forward kernel's output): x = ((p0 + p1) + p2) + ..., rms_norm applied as NormStage does.
/// Always staged through LDS: every lane summing its own chunks of all the parts (the direct
/// path) reads them once per wave, and at the 0.5B QKV shape those reads made the step 12 us
/// slower than one workgroup of four waves sharing one staged copy (two waves per copy: 13 us
/// slower than that; eight: 21 us).
struct SumNormStage
{
    const float* parts;  // [kResidualParts][n]
    const float* w;
    float eps;
    static constexpr bool kCanDirect = false;
    static constexpr bool kDirect = false;
    static constexpr bool kElementwise = false;
    static constexpr bool kNorm = true;
    template <int kThreads, int kVec, class Between = NoOp>
    __device__ float Run(float4* xs, uint32_t n, Between between = Between{}) const
    {
        return StageSplit<kThreads, kVec, true, Between, kResidualParts>(parts, w, n, eps, xs, kResidualParts,
                                                                         nullptr, between);
    }
};

/// A staging policy applied by every lane to its own activation chunks, straight from global
/// memory into registers (single-batch rows, where one segment covers the row): no LDS and no
/// barrier, so the activation costs one latency that overlaps the weights'. Every segment reads
/// the whole activation, which costs L1 bandwidth; launches with more workgroups than CUs stage
/// through LDS instead.
template <class Base>
struct DirectStage : Base
{
    static constexpr bool kDirect = true;
};

/// out[k] = v of lane k of this lane's group of lanes, for k < kCount: ds_swizzle bit mode
/// within each 32 lanes, source (L & kAnd) | k (kAnd 0x10: 16-lane groups, 0: 32-lane groups).
template <int kAnd, int kK>
__device__ __forceinline__ float FromGroupLane(float v)
{
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kAnd | (kK << 5)));
}

template <int kAnd, uint32_t kCount, int kK = 0>
__device__ __forceinline__ void HeadLaneBroadcast(float v, float (&out)[kCount])
{
    if constexpr (kK < static_cast<int>(kCount))
    {
        out[kK] = FromGroupLane<kAnd, kK>(v);
        HeadLaneBroadcast<kAnd, kCount, kK + 1>(v, out);
    }
}

/// The attention output, merged from the chunk partials: out[h][d] = sum_c 2^(m_c - M) acc_c /
/// sum_c 2^(m_c - M) l_c (flash-decoding's combine, maxima in log2 units). Every slot of the
/// grid (at most kChunks) takes part; chunks without keys hold the neutral partial, so no
/// position is needed and every partial is requested at entry.
template <uint32_t kChunks>
struct MergeStage
{
    const float* attnMax;
    const float* attnSum;
    const float* attnAcc;
    uint32_t heads, group, headDim, gridChunks;
    static constexpr bool kCanDirect = false;  // the merged row is shared through LDS
    static constexpr bool kDirect = false;
    static constexpr bool kElementwise = false;
    static constexpr bool kNorm = false;

    __device__ uint64_t Slot(uint32_t h, uint32_t c) const
    {
        return (static_cast<uint64_t>(h / group) * gridChunks + min(c, gridChunks - 1)) * group + h % group;
    }

    /// Thread t owns channels 4t..4t+3 of the q dim, so a head is headDim / 4 consecutive lanes
    /// (16 or 32). Lane c < kChunks of a head's lanes turns chunk c's (max, sum) into its weight
    /// 2^(m_c - M) / sum_c' 2^(m_c' - M) l_c' and every lane adds its channels of the chunks' P.V
    /// rows with those weights, read from lane c by ds_swizzle: the exponentials and the division
    /// run once per chunk, not once per channel. One barrier publishes the merged row.
    /// `between` (a kernel's weight loads) runs once the partials are requested, so the merge
    /// runs while the weights stream.
    template <int kThreads, int kVec, class Between = NoOp>
    __device__ float Run(float4* xs, uint32_t n, Between between = Between{}) const
    {
        static_assert(kThreads == kBlock, "the merge spreads the q dim over kBlock threads");
        static_assert(kChunks <= 16, "a head's first 16 lanes weigh the chunks");
        const uint32_t nchunks = n / 8;
        const uint32_t t = min(threadIdx.x, n / 4 - 1);
        const uint32_t h = 4 * t / headDim;
        const uint32_t d = 4 * t % headDim;
        const uint32_t c = t % (headDim / 4);  // this lane's chunk, when below gridChunks
        float4 a[kChunks];
#pragma unroll
        for (uint32_t k = 0; k < kChunks; ++k)
        {
            a[k] = *reinterpret_cast<const float4*>(attnAcc + Slot(h, k) * headDim + d);
        }
        const float mcLoaded = attnMax[Slot(h, min(c, kChunks - 1))];
        const float lc = attnSum[Slot(h, min(c, kChunks - 1))];
        __builtin_amdgcn_sched_barrier(0);
        between();
        __builtin_amdgcn_sched_barrier(0);
        const float mc = c < gridChunks && c < kChunks ? mcLoaded : -INFINITY;
        // Lanes 0..15 of each head hold its chunks (the rest -inf), so 16-lane groups suffice.
        const float top = GroupMax<16>(mc);
        const float e = top == -INFINITY || mc == -INFINITY ? 0.0f : exp2f(mc - top);
        const float den = GroupSum<16>(e * lc);
        const float weight = den > 0.0f ? e / den : 0.0f;
        float wk[kChunks];
        if (headDim == 64)
        {
            HeadLaneBroadcast<0x10, kChunks>(weight, wk);
        }
        else
        {
            HeadLaneBroadcast<0x00, kChunks>(weight, wk);
        }
        float4 out = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t k = 0; k < kChunks; ++k)
        {
            out.x = fmaf(wk[k], a[k].x, out.x);
            out.y = fmaf(wk[k], a[k].y, out.y);
            out.z = fmaf(wk[k], a[k].z, out.z);
            out.w = fmaf(wk[k], a[k].w, out.w);
        }
        if (4 * threadIdx.x < n)
        {
            // Channels 4t..4t+3 are half of chunk t/2: its low float4 when t is even.
            xs[(threadIdx.x & 1u) ? nchunks + threadIdx.x / 2 : threadIdx.x / 2] = out;
        }
        __syncthreads();
        return 1.0f;
    }
};

// ------------------------------------------------------------------------------------------------
// Fused GEMV: units of kNr rows, a staging policy, an epilogue per unit, an optional block tail.
//
// kSingle (a row fits one batch): one segment of kLpr lanes streams all kNr rows of a unit. Each
// lane keeps its activation chunks in registers (read from LDS once) and requests the next
// unit's rows as soon as the current ones are consumed. One buffer per wave keeps the register
// count low enough for two or three resident waves per SIMD, which hide each other's latency
// (measured faster than double-buffering at one or two). Otherwise the kNr rows of a unit sit in
// kNr adjacent segments and each row streams through RowDot's ping-pong of batches.

/// float4 loads per thread that stage a row of at most kLpr * kCpl chunks in one round (the
/// norm prologue needs one round): fewer registers for short rows.
template <int kLpr, int kCpl, int kThreads>
constexpr int StageVecFor()
{
    constexpr int n = (kLpr * kCpl * 2 + kThreads - 1) / kThreads;
    return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : kStageVec;
}

template <int kLpr, int kNr, bool kSingle>
constexpr uint32_t UnitsPerWave()
{
    return kSingle ? kWave / kLpr : (kWave / kLpr) / kNr;
}

template <int kLpr, int kCpl, int kNr, bool kSingle, class Stage, class Epi, int kThreads = kBlock>
__global__ __launch_bounds__(kThreads) void FusedMatVec(uint32_t cols, Stage stage, Epi epi)
{
    static_assert(kThreads == kBlock || kSingle, "multi-batch rows stage with kBlock threads");
    constexpr int kWavesPerBlock = kThreads / kWave;
    extern __shared__ float4 xs[];
    const uint32_t nchunks = cols / 8;
    constexpr int kUnits = UnitsPerWave<kLpr, kNr, kSingle>();
    static_assert(kUnits >= 1 && (kNr == 1 || kNr == 2), "a wave holds whole units of one or two rows");
    const int lane = threadIdx.x & (kWave - 1);
    const int segment = lane / kLpr;
    const uint32_t lir = lane % kLpr;
    const int unitInWave = kSingle ? segment : segment / kNr;
    const int part = kSingle ? 0 : segment % kNr;
    const uint32_t wave = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    const uint32_t stride = gridDim.x * kWavesPerBlock * kUnits;
    const uint32_t units = epi.Units();
    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    uint32_t first = wave * kUnits;

    if constexpr (kSingle)
    {
        // Weights do not depend on the activation: they stream while it is staged.
        half8 w[kNr][kCpl];
        typename Epi::Pre pre{};
        auto load = [&](uint32_t unit) {
#pragma unroll
            for (int r = 0; r < kNr; ++r)
            {
                LoadBatch<kLpr, kCpl>(epi.Row(unit, r), 0, nchunks, lir, w[r]);
            }
        };
        // Branch-free (a wave without a unit loads the last unit's rows and drops them), so the
        // waits for loads issued before these can count them.
        auto loadFirst = [&] {
            const uint32_t unit = min(first + unitInWave, units - 1);
            pre = epi.Prefetch(unit);
            load(unit);
        };
        float4 xlo[kCpl];
        float4 xhi[kCpl];
        // A directly staged norm leaves each lane its part of sum(x^2), reduced over the segment
        // with every unit's row sums (one more value in the same lane permutes).
        constexpr bool kLaneNorm = Stage::kDirect && Stage::kNorm;
        float scale = 1.0f;
        float squares = 0.0f;
        // The epilogue's own work (Ready) runs while the weights and the activation are in flight.
        if constexpr (Stage::kDirect)
        {
            // The activation (an L2 hit for all but the first workgroups of an XCD) is requested
            // first and the weights right after it, so the norm's products run while the weights
            // stream rather than after the activation has queued behind them.
            squares = stage.template Direct<kLpr, kCpl>(cols, lir, xlo, xhi, [&] {
                loadFirst();
                epi.Ready(pre);
            });
        }
        else
        {
            // The staging policy issues the activation's loads first and the weights' right after
            // (Run's `between`), so the activation, which loads complete in order, is staged while
            // the weights stream.
            scale = stage.template Run<kThreads, StageVecFor<kLpr, kCpl, kThreads>()>(xs, cols, [&] {
                loadFirst();
                epi.Ready(pre);
            });
            LoadActivation<kLpr, kCpl>(xs, xs + nchunks, nchunks, lir, xlo, xhi);
        }
        for (; first < units; first += stride)
        {
            const uint32_t unit = first + unitInWave;
            float sums[kNr + (kLaneNorm ? 1 : 0)];
#pragma unroll
            for (int r = 0; r < kNr; ++r)
            {
                sums[r] = unit < units ? DotRegisters<kLpr, kCpl>(w[r], xlo, xhi, nchunks, lir) : 0.0f;
            }
            if constexpr (kLaneNorm)
            {
                sums[kNr] = squares;
            }
            // The next unit's rows go out before this unit's reduction and epilogue; with a single
            // buffer per wave the other resident waves keep the memory busy meanwhile.
            typename Epi::Pre next{};
            if (unit + stride < units)
            {
                next = epi.Prefetch(unit + stride);
                load(unit + stride);
                epi.Ready(next);
            }
            // Every lane of the segment ends with the unit's row sums.
            GroupSumN<kLpr>(sums);
            if constexpr (kLaneNorm)
            {
                scale = NormScale(sums[kNr], cols, stage.eps);
            }
            float rowSums[kNr];
#pragma unroll
            for (int r = 0; r < kNr; ++r)
            {
                rowSums[r] = Stage::kNorm ? sums[r] * scale : sums[r];
            }
            if (unit < units && lir == 0)
            {
                epi.Finish(unit, rowSums, pre, bestValue, bestIndex);
            }
            pre = next;
        }
    }
    else
    {
        half8 w[kCpl];
        typename Epi::Pre pre{};
        if (first + unitInWave < units)
        {
            pre = epi.Prefetch(first + unitInWave);
            LoadBatch<kLpr, kCpl>(epi.Row(first + unitInWave, part), 0, nchunks, lir, w);
            epi.Ready(pre);
        }
        const float scale = stage.template Run<kBlock, kStageVec>(xs, cols);
        const float4* lo = xs;
        const float4* hi = xs + nchunks;
        for (; first < units; first += stride)
        {
            const uint32_t unit = first + unitInWave;
            float dot = 0.0f;
            if (unit < units)
            {
                dot = RowDot<kLpr, kCpl>(epi.Row(unit, part), nchunks, lir, w, lo, hi);
            }
            // The next unit's first batch goes out before this unit's reduction and epilogue.
            const uint32_t next = first + stride + unitInWave;
            typename Epi::Pre nextPre{};
            if (next < units)
            {
                nextPre = epi.Prefetch(next);
                LoadBatch<kLpr, kCpl>(epi.Row(next, part), 0, nchunks, lir, w);
                epi.Ready(nextPre);
            }
            // Every lane of a segment holds its row's sum; the unit's second row sits in the
            // partner segment.
            dot = GroupSum<kLpr>(dot);
            if constexpr (Stage::kNorm)
            {
                dot *= scale;
            }
            float sums[kNr];
            sums[0] = dot;
            if constexpr (kNr == 2)
            {
                sums[1] = PartnerLane<kLpr>(dot);
            }
            if (unit < units && part == 0 && lir == 0)
            {
                epi.Finish(unit, sums, pre, bestValue, bestIndex);
            }
            pre = nextPre;
        }
    }
    epi.template Tail<kThreads>(bestValue, bestIndex);
}

/// Long rows (more than 1024 16-byte chunks): the whole workgroup streams one row as a single
/// batch of kCpl chunks per lane, rows double-buffered, the four wave sums combined in LDS.
template <int kCpl, class Stage, class Epi>
__global__ __launch_bounds__(kBlock) void FusedMatVecBlockRow(uint32_t cols, Stage stage, Epi epi)
{
    extern __shared__ float4 xs[];
    __shared__ float partial[2][kWaves];
    const uint32_t nchunks = cols / 8;
    const uint32_t lir = threadIdx.x;
    const uint32_t units = epi.Units();
    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    uint32_t parity = 0;
    float scale = 1.0f;  // the rms_norm factor of a norm stage
    auto finish = [&](uint32_t unit, float dot, const typename Epi::Pre& pre) {
        dot = GroupSum<kWave>(dot);
        if ((threadIdx.x & (kWave - 1)) == 0)
        {
            partial[parity][threadIdx.x / kWave] = dot;
        }
        __syncthreads();
        if (threadIdx.x == 0)
        {
            float sums[1] = {(partial[parity][0] + partial[parity][1]) + (partial[parity][2] + partial[parity][3])};
            if constexpr (Stage::kNorm)
            {
                sums[0] *= scale;
            }
            epi.Finish(unit, sums, pre, bestValue, bestIndex);
        }
        parity ^= 1u;
    };

    uint32_t unit = blockIdx.x;
    half8 wa[kCpl];
    half8 wb[kCpl];
    typename Epi::Pre pa{};
    typename Epi::Pre pb{};
    if (unit < units)
    {
        pa = epi.Prefetch(unit);
        LoadBatch<kBlock, kCpl>(epi.Row(unit, 0), 0, nchunks, lir, wa);
        epi.Ready(pa);
    }
    scale = stage.template Run<kBlock, kStageVec>(xs, cols);
    const float4* lo = xs;
    const float4* hi = xs + nchunks;
    for (; unit < units; unit += 2 * gridDim.x)
    {
        const uint32_t ub = unit + gridDim.x;
        if (ub < units)
        {
            pb = epi.Prefetch(ub);
            LoadBatch<kBlock, kCpl>(epi.Row(ub, 0), 0, nchunks, lir, wb);
            epi.Ready(pb);
        }
        finish(unit, DotBatch<kBlock, kCpl>(wa, 0, nchunks, lir, lo, hi, 0.0f), pa);
        if (ub >= units)
        {
            break;
        }
        const uint32_t uc = ub + gridDim.x;
        if (uc < units)
        {
            pa = epi.Prefetch(uc);
            LoadBatch<kBlock, kCpl>(epi.Row(uc, 0), 0, nchunks, lir, wa);
            epi.Ready(pa);
        }
        finish(ub, DotBatch<kBlock, kCpl>(wb, 0, nchunks, lir, lo, hi, 0.0f), pb);
    }
    epi.template Tail<kBlock>(bestValue, bestIndex);
}

/// Mid-size matrices whose units outnumber the waves resident at once: workgroup b owns kUnits
/// consecutive units and wave w the w-th quarter of every row's chunks. Each wave requests its
/// quarter of all kUnits units at once, so the whole matrix is in flight in one round instead of
/// some waves waiting a second latency for a second unit. The activation quarter is read
/// straight into registers (the norm's sum of squares meets in LDS); the quarter sums meet in
/// LDS once, after the dots.
template <int kCpl, int kNr, int kUnits, class Stage, class Epi>
__global__ __launch_bounds__(kBlock) void FusedMatVecColumns(uint32_t cols, Stage stage, Epi epi)
{
    static_assert(Stage::kCanDirect, "each wave stages its own activation quarter");
    __shared__ float partial[kUnits][kNr][kWaves];
    __shared__ float squares[kWaves];
    const uint32_t nchunks = cols / 8;
    const uint32_t quarter = (nchunks + kWaves - 1) / kWaves;
    const uint32_t waveId = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t begin = min(waveId * quarter, nchunks - 1);
    const uint32_t span = min(begin + quarter, nchunks) - begin;  // this wave's chunks, >= 1
    const uint32_t units = epi.Units();
    const uint32_t u0 = blockIdx.x * kUnits;
    const uint32_t count = u0 < units ? min(static_cast<uint32_t>(kUnits), units - u0) : 0;
    typename Epi::Pre pre{};
    if (threadIdx.x < count)
    {
        pre = epi.Prefetch(u0 + threadIdx.x);
    }
    float4 xlo[kCpl];
    float4 xhi[kCpl];
    LoadActivationDirect<kWave, kCpl, false>(stage.x + 8 * begin, nullptr, 8 * span, lane, xlo, xhi);
    float4 glo[kCpl];
    float4 ghi[kCpl];
    if constexpr (Stage::kNorm)
    {
        LoadActivationDirect<kWave, kCpl, false>(stage.w + 8 * begin, nullptr, 8 * span, lane, glo, ghi);
    }
    // Every unit at once; past the last unit (the grid's last workgroup only) a slot reloads it.
    half8 w[kUnits][kNr][kCpl];
#pragma unroll
    for (int k = 0; k < kUnits; ++k)
    {
        const uint32_t unit = min(u0 + k, units - 1);
#pragma unroll
        for (int r = 0; r < kNr; ++r)
        {
            LoadBatch<kWave, kCpl>(epi.Row(unit, r) + 8 * begin, 0, span, lane, w[k][r]);
        }
    }
    // The activation quarter and the norm weights are requested before the weights: loads
    // complete in order, so the norm's sum and barrier run while the weights stream (7B QKV
    // 8.3 -> 8.0 us). The scheduling barrier keeps the compiler from moving the norm above the
    // weight loads. Here the row's factor is applied to x before the dot, in that shadow: taken
    // to the row sums instead, its square root and division land after the weights (7B-shape
    // QKV 7.77 -> 7.97 us).
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (Stage::kNorm)
    {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kCpl; ++i)
        {
            ss += lane + i * kWave < span ? SquaresOf(xlo[i], xhi[i]) : 0.0f;
        }
        ss = GroupSum<kWave>(ss);
        if (lane == 0)
        {
            squares[waveId] = ss;
        }
        __syncthreads();
        const float scale = NormScale((squares[0] + squares[1]) + (squares[2] + squares[3]), cols, stage.eps);
#pragma unroll
        for (int i = 0; i < kCpl; ++i)
        {
            xlo[i].x = (scale * xlo[i].x) * glo[i].x;
            xlo[i].y = (scale * xlo[i].y) * glo[i].y;
            xlo[i].z = (scale * xlo[i].z) * glo[i].z;
            xlo[i].w = (scale * xlo[i].w) * glo[i].w;
            xhi[i].x = (scale * xhi[i].x) * ghi[i].x;
            xhi[i].y = (scale * xhi[i].y) * ghi[i].y;
            xhi[i].z = (scale * xhi[i].z) * ghi[i].z;
            xhi[i].w = (scale * xhi[i].w) * ghi[i].w;
        }
    }
    float d[kUnits * kNr];
#pragma unroll
    for (int k = 0; k < kUnits; ++k)
    {
#pragma unroll
        for (int r = 0; r < kNr; ++r)
        {
            d[k * kNr + r] = DotRegisters<kWave, kCpl>(w[k][r], xlo, xhi, span, lane);
        }
    }
    if constexpr (kUnits * kNr <= 8)
    {
        // Lane L < kUnits * kNr ends with the wave's sum of value L.
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            v[i] = i < kUnits * kNr ? d[i < kUnits * kNr ? i : 0] : 0.0f;
        }
        const float total = ScatterSum8(v);
        if (lane < static_cast<uint32_t>(kUnits * kNr))
        {
            (&partial[0][0][0])[lane * kWaves + waveId] = total;
        }
    }
    else
    {
        GroupSumN<kWave>(d);
        if (lane == 0)
        {
#pragma unroll
            for (int k = 0; k < kUnits; ++k)
            {
#pragma unroll
                for (int r = 0; r < kNr; ++r)
                {
                    partial[k][r][waveId] = d[k * kNr + r];
                }
            }
        }
    }
    __syncthreads();
    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    if (threadIdx.x < count)
    {
        const uint32_t k = threadIdx.x;
        float sums[kNr];
#pragma unroll
        for (int r = 0; r < kNr; ++r)
        {
            sums[r] = (partial[k][r][0] + partial[k][r][1]) + (partial[k][r][2] + partial[k][r][3]);
        }
        // Here the epilogue's own work (Ready) is left to the end: wave 0 reaching the norm's
        // barrier late held all four waves back (7B-shape QKV 8.3 -> 8.9 us).
        epi.Ready(pre);
        epi.Finish(u0 + k, sums, pre, bestValue, bestIndex);
    }
    epi.template Tail<kBlock>(bestValue, bestIndex);
}

/// Long rows, split by columns: workgroup b owns rows b, b + grid, b + 2 grid, ... (at most
/// kMaxSplitRows) and wave w the w-th quarter of every row's chunks, its activation quarter read
/// from LDS into registers once. Each wave streams its quarter of the block's rows double-buffered
/// with no barrier between rows; the quarter sums meet in LDS once, after the last row. Dealing
/// rows round-robin keeps the rows in flight across the grid one contiguous window of the matrix:
/// runs of consecutive rows per workgroup put the concurrent reads a run apart, which spreads
/// them over the HBM channels less evenly (7B down read-only: 22.7 -> 20.5 us).
constexpr uint32_t kMaxSplitRows = 32;

template <int kCpl, class Stage, class Epi>
__global__ __launch_bounds__(kBlock) void FusedMatVecSplitRows(uint32_t cols, Stage stage, Epi epi)
{
    extern __shared__ float4 xs[];
    __shared__ float partial[kMaxSplitRows][kWaves];
    const uint32_t nchunks = cols / 8;
    const uint32_t quarter = (nchunks + kWaves - 1) / kWaves;
    const uint32_t waveId = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t begin = min(waveId * quarter, nchunks - 1);
    const uint32_t span = min(begin + quarter, nchunks) - begin;  // this wave's chunks, >= 1
    const uint32_t units = epi.Units();
    const uint32_t grid = gridDim.x;
    // Rows blockIdx.x + k * grid for k < count (<= kMaxSplitRows: host check).
    const uint32_t count = blockIdx.x < units ? (units - blockIdx.x + grid - 1) / grid : 0;
    auto rowOf = [&](uint32_t k) { return blockIdx.x + k * grid; };
    typename Epi::Pre pre{};
    if (threadIdx.x < count)
    {
        pre = epi.Prefetch(rowOf(threadIdx.x));
    }
    half8 wa[kCpl];
    half8 wb[kCpl];
    auto load = [&](uint32_t k, half8(&w)[kCpl]) {
        LoadBatch<kWave, kCpl>(epi.Row(min(rowOf(k), units - 1), 0) + 8 * begin, 0, span, lane, w);
    };
    auto dot = [&](uint32_t k, const half8(&w)[kCpl], const float4(&xlo)[kCpl], const float4(&xhi)[kCpl]) {
        const float d = GroupSum<kWave>(DotRegisters<kWave, kCpl>(w, xlo, xhi, span, lane));
        if (lane == 0)
        {
            partial[k][waveId] = d;
        }
    };
    // The activation quarter first, then two rows, each buffer refilled as soon as its row is
    // consumed. Loads complete in order, so a row's dot then waits only for that row. No load sits
    // under a branch: the steady loop runs only while both refill rows exist and the tail's loads
    // are straight-line, so the compiler's waits count every load (loads under a branch had it
    // wait for the next row before using the current one). Rows are clamped into the matrix, so
    // a workgroup with a single row reloads it (an L2 hit).
    float4 xlo[kCpl];
    float4 xhi[kCpl];
    float scale = 1.0f;  // the rms_norm factor of a norm stage
    if constexpr (Stage::kElementwise)
    {
        // Each wave reads its own quarter of x straight into registers: one latency, no LDS.
        LoadActivationDirect<kWave, kCpl, false>(stage.x + 8 * begin, nullptr, 8 * span, lane, xlo, xhi);
        __builtin_amdgcn_sched_barrier(0);
    }
    load(0, wa);
    load(min(1u, count - 1), wb);
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < count)
    {
        epi.Ready(pre);
    }
    if constexpr (!Stage::kElementwise)
    {
        scale = stage.template Run<kBlock, kStageVec>(xs, cols);
        LoadActivation<kWave, kCpl>(xs + begin, xs + nchunks + begin, span, lane, xlo, xhi);
    }
    uint32_t k = 0;
    for (; k + 3 < count; k += 2)
    {
        dot(k, wa, xlo, xhi);
        load(k + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        dot(k + 1, wb, xlo, xhi);
        load(k + 3, wb);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t left = count - k;  // 1, 2 or 3 rows (0 only for a workgroup without rows)
    if (left == 3)
    {
        dot(k, wa, xlo, xhi);
        load(k + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        dot(k + 1, wb, xlo, xhi);
        dot(k + 2, wa, xlo, xhi);
    }
    else if (left == 2)
    {
        dot(k, wa, xlo, xhi);
        dot(k + 1, wb, xlo, xhi);
    }
    else if (left == 1)
    {
        dot(k, wa, xlo, xhi);
    }
    __syncthreads();
    float bestValue = -INFINITY;
    int32_t bestIndex = 0x7FFFFFFF;
    if (threadIdx.x < count)
    {
        const uint32_t k = threadIdx.x;
        float sums[1] = {(partial[k][0] + partial[k][1]) + (partial[k][2] + partial[k][3])};
        if constexpr (Stage::kNorm)
        {
            sums[0] *= scale;
        }
        epi.Finish(rowOf(k), sums, pre, bestValue, bestIndex);
    }
    epi.template Tail<kBlock>(bestValue, bestIndex);
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
    const float* ropePow;  // thetaScale^j for j < headDim / 2, powf on the host as the CPU path does
    uint32_t cols, heads, kvHeads, headDim, maxSeq;

    __device__ uint32_t Units() const { return (heads + 2 * kvHeads) * headDim / 2; }

    /// Rope units pair rows (j, j + hd/2) of one q or k head; value units pair adjacent rows.
    /// Branch-free, so the epilogue's operand loads issue with the weights.
    __device__ uint32_t RowOf(uint32_t unit, int part) const
    {
        const uint32_t half = headDim / 2;
        const uint32_t ropeUnits = (heads + kvHeads) * half;
        const uint32_t rope = (unit / half) * headDim + unit % half + part * half;
        const uint32_t value = (heads + kvHeads) * headDim + 2 * (unit - ropeUnits) + part;
        return unit < ropeUnits ? rope : value;
    }

    __device__ const uint16_t* Row(uint32_t unit, int part) const
    {
        return w + static_cast<uint64_t>(RowOf(unit, part)) * cols;
    }

    /// The epilogue's operands, requested with the unit's weights so their latency overlaps them.
    struct Pre
    {
        float bias0, bias1, pow;
        int32_t pos;
        float cos, sin;
    };

    __device__ Pre Prefetch(uint32_t unit) const
    {
        return Pre{bias[RowOf(unit, 0)], bias[RowOf(unit, 1)], ropePow[unit % (headDim / 2)], state->position,
                   0.0f, 0.0f};
    }

    /// Called once the unit's weights are requested: the rope angle's cosine and sine are worked
    /// out while those loads are in flight instead of after the dot products. The empty asm keeps
    /// the compiler from sinking them into the epilogue.
    __device__ void Ready(Pre& pre) const
    {
        // rope_neox (rope_funcs.glsl:76-114): theta = pos * theta_scale^j, pair (j, j + hd/2).
        const float theta = static_cast<float>(pre.pos) * pre.pow;
        sincosf(theta, &pre.sin, &pre.cos);  // one range reduction for both
        asm volatile("" : "+v"(pre.cos), "+v"(pre.sin));
    }

    __device__ void Finish(uint32_t unit, const float* s, const Pre& pre, float&, int32_t&) const
    {
        const uint32_t half = headDim / 2;
        const uint32_t ropeUnits = (heads + kvHeads) * half;
        const int32_t pos = pre.pos;
        const float s0 = s[0] + pre.bias0;
        const float s1 = s[1] + pre.bias1;
        if (unit < ropeUnits)
        {
            const uint32_t head = unit / half;
            const uint32_t j = unit % half;
            const float c = pre.cos;
            const float sn = pre.sin;
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

    template <int kThreads>
    __device__ void Tail(float, int32_t) const
    {
    }
};

struct ResidualEpi
{
    const uint16_t* w;
    const float* residual;
    float* out;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return w + static_cast<uint64_t>(unit) * cols; }
    struct Pre
    {
        float residual;
    };
    __device__ Pre Prefetch(uint32_t unit) const { return Pre{residual[unit]}; }
    __device__ void Ready(Pre&) const {}
    __device__ void Finish(uint32_t unit, const float* s, const Pre& pre, float&, int32_t&) const
    {
        out[unit] = pre.residual + s[0];
    }
    template <int kThreads>
    __device__ void Tail(float, int32_t) const
    {
    }
};

/// ResidualEpi that also zeroes row `unit` of `zero` (the next layer's o_proj target, which its kv
/// groups add into).
struct ResidualZeroEpi : ResidualEpi
{
    float* zero;
    __device__ void Finish(uint32_t unit, const float* s, const Pre& pre, float& v, int32_t& i) const
    {
        ResidualEpi::Finish(unit, s, pre, v, i);
        zero[unit] = 0.0f;
    }
};

/// ResidualEpi for the decoders whose feed-forward block is one launch. The residual is either a
/// single vector (inParts 1) or kResidualParts partial vectors laid end to end, added in order
/// (p0 + p1) + ... before the dot; with `parts` set the output also seeds the feed-forward
/// kernel's partial vectors: parts[0][row] = out[row], the other parts' rows zero. The residual
/// may be `parts` itself: each row is read and written only by the lanes that own it.
struct ResidualPartsEpi
{
    const uint16_t* w;
    const float* residual;
    float* out;
    float* parts;
    uint32_t rows, cols, inParts;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return w + static_cast<uint64_t>(unit) * cols; }
    struct Pre
    {
        float v[kResidualParts];
    };
    /// Branch-free: with a single residual vector every load reads it (cache hits).
    __device__ Pre Prefetch(uint32_t unit) const
    {
        Pre p;
#pragma unroll
        for (uint32_t k = 0; k < kResidualParts; ++k)
        {
            p.v[k] = residual[min(k, inParts - 1) * static_cast<uint64_t>(rows) + unit];
        }
        return p;
    }
    __device__ void Ready(Pre&) const {}
    __device__ void Finish(uint32_t unit, const float* s, const Pre& pre, float&, int32_t&) const
    {
        float res = pre.v[0];
#pragma unroll
        for (uint32_t k = 1; k < kResidualParts; ++k)
        {
            res += k < inParts ? pre.v[k] : 0.0f;
        }
        const float value = res + s[0];
        out[unit] = value;
        if (parts != nullptr)
        {
            parts[unit] = value;
#pragma unroll
            for (uint32_t k = 1; k < kResidualParts; ++k)
            {
                parts[k * static_cast<uint64_t>(rows) + unit] = 0.0f;
            }
        }
    }
    template <int kThreads>
    __device__ void Tail(float, int32_t) const
    {
    }
};

/// out[row] = (W[row] . x + bias0[row]) + bias1[row], each bias only when given: the per-op
/// GEMV's FUSE0/FUSE1 in mul_mat_vec_base.glsl's order.
struct BiasEpi
{
    static constexpr uint32_t kResidentRounds = 2;  // as the LM heads: long launches balance better
    const uint16_t* w;
    const float* bias0;
    const float* bias1;
    float* out;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return w + static_cast<uint64_t>(unit) * cols; }
    struct Pre
    {
        float b0, b1;
    };
    __device__ Pre Prefetch(uint32_t unit) const
    {
        return Pre{bias0 != nullptr ? bias0[unit] : 0.0f, bias1 != nullptr ? bias1[unit] : 0.0f};
    }
    __device__ void Ready(Pre&) const {}
    __device__ void Finish(uint32_t unit, const float* s, const Pre& pre, float&, int32_t&) const
    {
        float value = s[0];
        if (bias0 != nullptr)
        {
            value += pre.b0;
        }
        if (bias1 != nullptr)
        {
            value += pre.b1;
        }
        out[unit] = value;
    }
    template <int kThreads>
    __device__ void Tail(float, int32_t) const
    {
    }
};

struct GateUpEpi
{
    // Two rounds of resident workgroups (7B gate/up 44.1 -> 43.0 us; the 0.5B one covers its
    // units in one round of single-wave workgroups either way).
    static constexpr uint32_t kResidentRounds = 2;
    const uint16_t* gate;
    const uint16_t* up;
    float* act;
    uint32_t rows, cols;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int part) const
    {
        return (part == 0 ? gate : up) + static_cast<uint64_t>(unit) * cols;
    }
    struct Pre
    {
    };
    __device__ Pre Prefetch(uint32_t) const { return Pre{}; }
    __device__ void Ready(Pre&) const {}
    __device__ void Finish(uint32_t unit, const float* s, const Pre&, float&, int32_t&) const
    {
        act[unit] = s[0] / (1.0f + expf(-s[0])) * s[1];  // swiglu.comp's op
    }
    template <int kThreads>
    __device__ void Tail(float, int32_t) const
    {
    }
};

/// Better (value, index) under "larger value, then lower index" (the host greedy scan's rule).
__device__ __forceinline__ bool Better(float v, int32_t i, float bestV, int32_t bestI)
{
    return v > bestV || (v == bestV && i < bestI);
}

/// Reduce (value, index) over a block of kThreads; the result lands in thread 0.
template <int kThreads = kBlock>
__device__ __forceinline__ void BlockArgMax(float& value, int32_t& index)
{
    constexpr int kWaveCount = kThreads / kWave;
    GroupArgMax<kWave>(value, index);
    if constexpr (kWaveCount == 1)
    {
        return;
    }
    __shared__ float waveValue[kWaveCount];
    __shared__ int32_t waveIndex[kWaveCount];
    if ((threadIdx.x & (kWave - 1)) == 0)
    {
        waveValue[threadIdx.x / kWave] = value;
        waveIndex[threadIdx.x / kWave] = index;
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        for (int k = 1; k < kWaveCount; ++k)
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
    // Two rounds of resident workgroups, each with half the rows: 0.5B LM head 42.6 -> 41.0 us,
    // 7B 168.4 -> 164.1 us (three rounds: no better, or slower).
    static constexpr uint32_t kResidentRounds = 2;

    __device__ uint32_t Units() const { return rows; }
    __device__ const uint16_t* Row(uint32_t unit, int) const { return table + static_cast<uint64_t>(unit) * cols; }
    struct Pre
    {
    };
    __device__ Pre Prefetch(uint32_t) const { return Pre{}; }
    __device__ void Ready(Pre&) const {}
    __device__ void Finish(uint32_t unit, const float* s, const Pre&, float& bestValue, int32_t& bestIndex) const
    {
        logits[unit] = s[0];
        // Units reach a lane in increasing order, so '>' keeps the lowest index on ties.
        if (s[0] > bestValue)
        {
            bestValue = s[0];
            bestIndex = static_cast<int32_t>(unit);
        }
    }
    template <int kThreads>
    __device__ void Tail(float value, int32_t index) const
    {
        BlockArgMax<kThreads>(value, index);
        if (threadIdx.x == 0)
        {
            argValue[blockIdx.x] = value;
            argIndex[blockIdx.x] = index;
        }
    }
};

// ------------------------------------------------------------------------------------------------
// Launch helpers for the fused GEMV.

/// Rounds of resident workgroups a GEMV's grid may span: Epi::kResidentRounds, else 1.
template <class E, class = void>
struct ResidentRounds
{
    static constexpr uint32_t value = 1;
};

template <class E>
struct ResidentRounds<E, std::void_t<decltype(E::kResidentRounds)>>
{
    static constexpr uint32_t value = E::kResidentRounds;
};

/// Workgroups of `kernel` the chip holds at once with `lds` bytes of dynamic LDS each.
template <typename Kernel>
uint32_t ResidentBlocks(Kernel kernel, int threads, size_t lds)
{
    int perCu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, kernel, threads, lds) != hipSuccess || perCu < 1)
    {
        perCu = 1;
    }
    return CuCount() * static_cast<uint32_t>(perCu);
}

/// Launches `kernel` over `units`, or with shapeOut only reports its grid. The grid
/// holds at most the workgroups resident at once (each stages the activation once and then
/// strides over the units), so no workgroup waits for a second round; an epilogue may allow
/// more rounds (ResidentRounds).
template <auto kKernel, class Stage, class Epi, int kThreads = kBlock>
hipError_t LaunchGemvKernel(hipStream_t s, uint32_t units, uint32_t unitsPerBlock, uint32_t blockCap, size_t lds,
                            uint32_t cols, const Stage& stage, const Epi& epi, GemvShape* shapeOut)
{
    const auto kernel = kKernel;
    // Per device, for this kernel instantiation: the resident workgroups at the last LDS size
    // asked for, and the dynamic LDS the kernel has been opted in to (64 KB by default).
    struct Cache
    {
        std::mutex mutex;
        uint32_t resident[kMaxDevices] = {};
        size_t residentLds[kMaxDevices] = {};
        size_t configured[kMaxDevices] = {};
    };
    static Cache cache;
    std::lock_guard<std::mutex> lock(cache.mutex);
    const int device = CurrentDevice();
    if (cache.resident[device] == 0 || cache.residentLds[device] != lds)
    {
        cache.resident[device] = ResidentBlocks(kernel, kThreads, lds);
        cache.residentLds[device] = lds;
    }
    const uint32_t blocks = std::max(
        1u, std::min({CeilDiv(units, unitsPerBlock), blockCap, ResidentRounds<Epi>::value * cache.resident[device]}));
    if (shapeOut != nullptr)
    {
        *shapeOut = GemvShape{blocks, unitsPerBlock};
        return hipSuccess;
    }
    // Opt in to more than the default 64 KB of dynamic LDS only when a launch needs it.
    if (lds > std::max<size_t>(64 * 1024, cache.configured[device]))
    {
        const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                                      static_cast<int>(lds));
        if (status != hipSuccess)
        {
            return status;
        }
        cache.configured[device] = lds;
    }
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), lds, s, cols, stage, epi);
    return hipGetLastError();
}

/// The column-quarter kernel with the fewest units per workgroup whose grid is resident in one
/// round; hipErrorNotSupported (nothing launched) when none is.
template <int kNr, int kUnits, class Stage, class Epi>
hipError_t LaunchColumnsT(hipStream_t s, uint32_t units, uint32_t blockCap, uint32_t cols, const Stage& stage,
                          const Epi& epi, GemvShape* shapeOut)
{
    constexpr auto kKernel = &FusedMatVecColumns<2, kNr, kUnits, Stage, Epi>;
    GemvShape probe{};
    (void)LaunchGemvKernel<kKernel, Stage, Epi>(s, units, kUnits, blockCap, 0, cols, stage, epi, &probe);
    const uint32_t blocks = probe.blocks;
    if (static_cast<uint64_t>(blocks) * kUnits < units)
    {
        if constexpr (kUnits < 6)
        {
            return LaunchColumnsT<kNr, kUnits + 1, Stage, Epi>(s, units, blockCap, cols, stage, epi, shapeOut);
        }
        return hipErrorNotSupported;
    }
    return LaunchGemvKernel<kKernel, Stage, Epi>(s, units, kUnits, blockCap, 0, cols, stage, epi, shapeOut);
}

template <int kLpr, int kCpl, int kNr, bool kSingle, class Stage, class Epi>
hipError_t LaunchFusedT(hipStream_t s, uint32_t units, uint32_t blockCap, size_t lds, uint32_t cols,
                        const Stage& stage, const Epi& epi, GemvShape* shapeOut)
{
    constexpr uint32_t kUnitsPerBlock = kWaves * UnitsPerWave<kLpr, kNr, kSingle>();
    if constexpr (kSingle && Stage::kCanDirect)
    {
        // At most one workgroup per CU: latency-bound, so each lane stages its own chunks.
        GemvShape probe{};
        (void)LaunchGemvKernel<&FusedMatVec<kLpr, kCpl, kNr, kSingle, Stage, Epi>, Stage, Epi>(
            s, units, kUnitsPerBlock, blockCap, lds, cols, stage, epi, &probe);
        const uint32_t blocks = probe.blocks;
        if (blocks <= CuCount())
        {
            // No LDS, so the workgroups can be small and spread over more CUs.
            const DirectStage<Stage> direct{stage};
            constexpr uint32_t kDirectUnits = (kDirectThreads / kWave) * UnitsPerWave<kLpr, kNr, kSingle>();
            return LaunchGemvKernel<&FusedMatVec<kLpr, kCpl, kNr, kSingle, DirectStage<Stage>, Epi, kDirectThreads>,
                                    DirectStage<Stage>, Epi, kDirectThreads>(s, units, kDirectUnits, blockCap, 0, cols,
                                                                             direct, epi, shapeOut);
        }
        // More workgroups than CUs but few enough single-wave ones that every unit gets its own
        // segment in one round: single-wave workgroups balance the CUs (a 256-thread grid of
        // 1.2 CUs' worth leaves most CUs with one workgroup and some with two). A norm prologue
        // stages its row in one round, kStageVec float4 per thread: one wave holds rows of up to
        // 2048 floats, so wider normed rows keep 256-thread workgroups.
        constexpr bool kSmallFits = Stage::kElementwise || (kLpr * kCpl * 2 + kWave - 1) / kWave <= kStageVec;
        GemvShape smallProbe{};
        constexpr uint32_t kSmallUnits = UnitsPerWave<kLpr, kNr, kSingle>();
        (void)LaunchGemvKernel<&FusedMatVec<kLpr, kCpl, kNr, kSingle, Stage, Epi, kWave>, Stage, Epi, kWave>(
            s, units, kSmallUnits, blockCap, lds, cols, stage, epi, &smallProbe);
        const uint32_t small = smallProbe.blocks;
        if (kSmallFits && static_cast<uint64_t>(small) * kSmallUnits >= units)
        {
            return LaunchGemvKernel<&FusedMatVec<kLpr, kCpl, kNr, kSingle, Stage, Epi, kWave>, Stage, Epi, kWave>(
                s, units, kSmallUnits, blockCap, lds, cols, stage, epi, shapeOut);
        }
        // Units past one round of resident waves: column quarters with several units per
        // workgroup put the whole matrix in flight at once (rows of 257..512 chunks, where a
        // quarter is two chunks per lane).
        if (blocks * kUnitsPerBlock < units && cols / 8 > 256 && cols / 8 <= 512)
        {
            const hipError_t status = LaunchColumnsT<kNr, 3, Stage, Epi>(s, units, blockCap, cols, stage, epi,
                                                                        shapeOut);
            if (status != hipErrorNotSupported)
            {
                return status;
            }
        }
    }
    return LaunchGemvKernel<&FusedMatVec<kLpr, kCpl, kNr, kSingle, Stage, Epi>, Stage, Epi>(
        s, units, kUnitsPerBlock, blockCap, lds, cols, stage, epi, shapeOut);
}

/// hipErrorNotSupported (nothing launched) when a workgroup's share of the rows would overflow
/// its partial-sum table.
template <int kCpl, class Stage, class Epi>
hipError_t LaunchSplitRowsT(hipStream_t s, uint32_t units, uint32_t blockCap, size_t lds, uint32_t cols,
                            const Stage& stage, const Epi& epi, GemvShape* shapeOut)
{
    constexpr auto kKernel = &FusedMatVecSplitRows<kCpl, Stage, Epi>;
    const size_t used = Stage::kElementwise ? 0 : lds;
    GemvShape probe{};
    (void)LaunchGemvKernel<kKernel, Stage, Epi>(s, units, 1, blockCap, used, cols, stage, epi, &probe);
    const uint32_t blocks = probe.blocks;
    if (CeilDiv(units, blocks) > kMaxSplitRows)
    {
        return hipErrorNotSupported;
    }
    if (shapeOut != nullptr)
    {
        *shapeOut = GemvShape{blocks, CeilDiv(units, blocks)};  // rows per workgroup, dealt round-robin
        return hipSuccess;
    }
    return LaunchGemvKernel<kKernel, Stage, Epi>(s, units, 1, blockCap, used, cols, stage, epi, shapeOut);
}

template <int kCpl, class Stage, class Epi>
hipError_t LaunchBlockRowT(hipStream_t s, uint32_t units, uint32_t blockCap, size_t lds, uint32_t cols,
                           const Stage& stage, const Epi& epi, GemvShape* shapeOut)
{
    return LaunchGemvKernel<&FusedMatVecBlockRow<kCpl, Stage, Epi>, Stage, Epi>(s, units, 1, blockCap, lds, cols,
                                                                                 stage, epi, shapeOut);
}

/// Launches (or, with shapeOut, only sizes) the fused GEMV for a row of `cols` fp16 weights.
/// Rows of up to 1024 chunks (512 for two-row units) fit one batch of a wave segment; longer
/// rows use two-row units in RowDot's batch ping-pong, or one workgroup per row.
template <int kNr, class Stage, class Epi>
hipError_t LaunchFused(hipStream_t s, uint32_t units, uint32_t blockCap, uint32_t cols, const Stage& stage,
                       const Epi& epi, GemvShape* shapeOut = nullptr)
{
    if (cols % 8 != 0 || static_cast<size_t>(cols) * sizeof(float) > kMaxLds)
    {
        return hipErrorInvalidValue;
    }
    const uint32_t nchunks = cols / 8;
    const size_t lds = static_cast<size_t>(cols) * sizeof(float);
    // Short rows in a latency-bound launch (a few thousand units at most): a whole wave per unit,
    // two chunks per lane, so each lane's serial work (norm, dot, reduction) is a quarter of the
    // exact-fit 16 x 7 shape's. 0.5B-shape QKV: 3.62 -> 3.37 us.
    if (nchunks > 64 && nchunks <= 128 && units <= kWideUnits)
    {
        return LaunchFusedT<64, 2, kNr, true, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
    }
    const RowShape shape = PickFusedShape(nchunks, kNr);
#define MUYO_FUSED_CASE(L, C)                                                                                    \
    if (shape.lpr == L && shape.cpl == C)                                                                        \
    {                                                                                                            \
        return LaunchFusedT<L, C, kNr, true, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut); \
    }
    MUYO_FUSED_CASE(8, 7)
    MUYO_FUSED_CASE(8, 8)
    MUYO_FUSED_CASE(16, 7)
    MUYO_FUSED_CASE(16, 8)
    MUYO_FUSED_CASE(32, 7)
    MUYO_FUSED_CASE(32, 8)
    MUYO_FUSED_CASE(64, 7)
    MUYO_FUSED_CASE(64, 8)
    MUYO_FUSED_CASE(64, 10)
    if constexpr (kNr == 2)
    {
        // Rows past 640 chunks: the two rows of a unit in adjacent 32-lane segments.
        return LaunchFusedT<32, 16, kNr, false, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
    }
    else
    {
        MUYO_FUSED_CASE(64, 12)
        MUYO_FUSED_CASE(64, 14)
        MUYO_FUSED_CASE(64, 16)
#undef MUYO_FUSED_CASE
        // Column quarters (a wave's quarter of a row in one batch), else one workgroup per row.
        const uint32_t qcpl = CeilDiv(CeilDiv(nchunks, static_cast<uint32_t>(kWaves)), static_cast<uint32_t>(kWave));
        hipError_t split = hipErrorNotSupported;
        if (qcpl <= 8)
        {
            split = LaunchSplitRowsT<8, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
        }
        else if (qcpl <= 10)
        {
            split = LaunchSplitRowsT<10, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
        }
        else if (qcpl <= 12)
        {
            split = LaunchSplitRowsT<12, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
        }
        else if (qcpl <= 16)
        {
            split = LaunchSplitRowsT<16, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut);
        }
        if (split != hipErrorNotSupported)
        {
            return split;
        }
        const uint32_t cpl = CeilDiv(nchunks, static_cast<uint32_t>(kBlock));
#define MUYO_BLOCK_ROW_CASE(C)                                                                       \
    if (cpl <= C)                                                                                    \
    {                                                                                                \
        return LaunchBlockRowT<C, Stage, Epi>(s, units, blockCap, lds, cols, stage, epi, shapeOut); \
    }
        MUYO_BLOCK_ROW_CASE(8)
        MUYO_BLOCK_ROW_CASE(10)
        MUYO_BLOCK_ROW_CASE(12)
        MUYO_BLOCK_ROW_CASE(16)
        MUYO_BLOCK_ROW_CASE(20)
#undef MUYO_BLOCK_ROW_CASE
    }
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------------------------------------
// Feed-forward block in one launch (hidden <= 1024).
//
// Workgroup b owns the kFfnUnits intermediate units from kFfnUnits * b: wave w the units w,
// w + 4, ... . Every wave reads the activation (x * rms_norm weight) straight into registers,
// 64 lanes x 2 chunks covering a row of up to 1024 floats, and its units' gate and up rows; at the
// same time the workgroup requests its units' rows of the transposed down matrix (downT, one
// contiguous row of `hidden` weights per unit), so one launch streams all three matrices and the
// down rows arrive while the gate/up dots run. The units' swiglu values meet in LDS. Threads
// t < 2 * hidden/8 then own chunk t mod (hidden/8) of every other unit's down row, the two halves
// meet in LDS, and the workgroup adds its partial down product into partial vector
// b mod kResidualParts with one atomic add per element. Every workgroup adds to every element, so
// the adds to one address serialise at the memory: spreading them over kResidualParts vectors
// keeps that cost under the kernel's streaming time.
constexpr uint32_t kFfnUnits = 19;      // 4864 / 19 = 256 workgroups at the 0.5B shape, one per CU
constexpr uint32_t kFfnMaxChunks = 128;  // hidden <= 1024

__global__ __launch_bounds__(kBlock) void FfnFusedKernel(const float* __restrict__ x, const float* __restrict__ normW,
                                                         const uint16_t* __restrict__ wgate,
                                                         const uint16_t* __restrict__ wup,
                                                         const uint16_t* __restrict__ downT, float* parts,
                                                         uint32_t hidden, uint32_t ffn, float eps)
{
    constexpr uint32_t kPerWave = (kFfnUnits + kWaves - 1) / kWaves;
    constexpr uint32_t kPerHalf = (kFfnUnits + 1) / 2;
    __shared__ float act[kFfnUnits];
    __shared__ float4 upper[kFfnMaxChunks][2];
    __shared__ float total[8 * kFfnMaxChunks];
    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & (kWave - 1);
    // Wave-uniform, so the gate/up row addresses are scalar.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const uint32_t nchunks = hidden / 8;
    const uint32_t base = blockIdx.x * kFfnUnits;
    // Down rows: half h (0 or 1) takes units h, h + 2, ...; threads past 2 * nchunks load a copy
    // of half 1's rows (cache hits) and drop it, which keeps every load branch-free.
    const uint32_t chunk = t % nchunks;
    const uint32_t half = min(t / nchunks, 1u);
    const bool owner = t < 2 * nchunks;
    auto unitRow = [&](uint32_t j) { return min(base + min(j, kFfnUnits - 1), ffn - 1); };
    half8 g[kPerWave][2];
    half8 u[kPerWave][2];
    half8 d[kPerHalf];
    float4 xlo[2];
    float4 xhi[2];
    // The activation first, then the gate/up rows, then the down rows: loads complete in order,
    // so the norm and the gate/up dots wait only for what they use.
    const float squares = LoadActivationDirect<kWave, 2, true>(x, normW, hidden, lane, xlo, xhi, [&] {
#pragma unroll
        for (uint32_t k = 0; k < kPerWave; ++k)
        {
            const uint64_t row = unitRow(wave + kWaves * k);
            LoadBatch<kWave, 2>(wgate + row * hidden, 0, nchunks, lane, g[k]);
            LoadBatch<kWave, 2>(wup + row * hidden, 0, nchunks, lane, u[k]);
        }
#pragma unroll
        for (uint32_t k = 0; k < kPerHalf; ++k)
        {
            const uint64_t row = unitRow(half + 2 * k);
            d[k] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(downT + row * hidden) + chunk);
        }
    });
    float sums[2 * kPerWave + 1];
#pragma unroll
    for (uint32_t k = 0; k < kPerWave; ++k)
    {
        sums[2 * k] = DotRegisters<kWave, 2>(g[k], xlo, xhi, nchunks, lane);
        sums[2 * k + 1] = DotRegisters<kWave, 2>(u[k], xlo, xhi, nchunks, lane);
    }
    sums[2 * kPerWave] = squares;
    GroupSumN<kWave>(sums);
    const float scale = NormScale(sums[2 * kPerWave], hidden, eps);
#pragma unroll
    for (uint32_t k = 0; k < kPerWave; ++k)
    {
        const uint32_t j = wave + kWaves * k;
        if (j < kFfnUnits && lane == 0)
        {
            const float gv = sums[2 * k] * scale;
            const float uv = sums[2 * k + 1] * scale;
            // A unit past the matrix (the last workgroup's) weighs nothing: its clamped row is a
            // copy of the last one.
            act[j] = base + j < ffn ? gv / (1.0f + expf(-gv)) * uv : 0.0f;  // as GateUpEpi
        }
    }
    __syncthreads();
    float acc[8] = {};
#pragma unroll
    for (uint32_t k = 0; k < kPerHalf; ++k)
    {
        const uint32_t j = half + 2 * k;
        const float a = j < kFfnUnits ? act[min(j, kFfnUnits - 1)] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
            acc[e] = fmaf(a, static_cast<float>(d[k][e]), acc[e]);
        }
    }
    if (owner && half == 1)
    {
        upper[chunk][0] = float4{acc[0], acc[1], acc[2], acc[3]};
        upper[chunk][1] = float4{acc[4], acc[5], acc[6], acc[7]};
    }
    __syncthreads();
    if (owner && half == 0)
    {
        const float4 lo = upper[chunk][0];
        const float4 hi = upper[chunk][1];
        const float other[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
            total[8 * chunk + e] = acc[e] + other[e];
        }
    }
    __syncthreads();
    // Consecutive lanes add consecutive elements: each wave's atomics cover whole cache lines.
    float* dst = parts + (blockIdx.x % kResidualParts) * static_cast<uint64_t>(hidden);
    for (uint32_t i = t; i < hidden; i += kBlock)
    {
        __hip_atomic_fetch_add(dst + i, total[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/// dst[c][r] = src[r][c], through 64 x 64 tiles in LDS.
__global__ __launch_bounds__(kBlock) void TransposeF16Kernel(const uint16_t* __restrict__ src,
                                                             uint16_t* __restrict__ dst, uint32_t rows,
                                                             uint32_t cols)
{
    __shared__ uint16_t tile[64][66];
    const uint32_t r0 = blockIdx.y * 64;
    const uint32_t c0 = blockIdx.x * 64;
    for (uint32_t i = threadIdx.x; i < 64 * 64; i += kBlock)
    {
        const uint32_t r = i / 64;
        const uint32_t c = i % 64;
        if (r0 + r < rows && c0 + c < cols)
        {
            tile[r][c] = src[static_cast<uint64_t>(r0 + r) * cols + c0 + c];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < 64 * 64; i += kBlock)
    {
        const uint32_t c = i / 64;
        const uint32_t r = i % 64;
        if (r0 + r < rows && c0 + c < cols)
        {
            dst[static_cast<uint64_t>(c0 + c) * rows + r0 + r] = tile[r][c];
        }
    }
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
                                                         int32_t* sampled, int32_t token, int32_t position,
                                                         uint32_t argBlocks, uint32_t step)
{
    for (uint32_t b = threadIdx.x; b < argBlocks; b += kBlock)
    {
        argValue[b] = b == 0 ? 0.0f : -INFINITY;
        argIndex[b] = b == 0 ? token : 0x7FFFFFFF;
    }
    if (threadIdx.x == 0)
    {
        if (sampled != nullptr)
        {
            *sampled = token;
        }
        state->token = token;
        state->position = position;
        state->start = position;
        state->step = step;
    }
}

/// The next token is the sampler's when one ran (`sampled`), else the argmax of the LM head's
/// partials. It is also recorded at its position in the token history the sampler's penalty reads.
__global__ __launch_bounds__(kBlock) void BeginStepKernel(const uint16_t* __restrict__ table, DecodeState* state,
                                                          const float* __restrict__ argValue,
                                                          const int32_t* __restrict__ argIndex, uint32_t argBlocks,
                                                          const int32_t* sampled, int32_t* history,
                                                          uint32_t historyCap, float* __restrict__ x,
                                                          float* __restrict__ zero, int32_t* __restrict__ ids,
                                                          uint32_t idsCap, uint32_t hidden, uint32_t vocab)
{
    const int32_t token = sampled != nullptr ? *sampled : ReduceArgMaxPartials(argValue, argIndex, argBlocks);
    if (blockIdx.x == 0 && threadIdx.x == 0)
    {
        const uint32_t step = state->step;
        if (step > 0)
        {
            ids[(step - 1) % idsCap] = token;
        }
        const int32_t position = state->start + static_cast<int32_t>(step);
        state->token = token;
        state->position = position;
        state->step = step + 1;
        if (position >= 0 && static_cast<uint32_t>(position) < historyCap)
        {
            history[position] = token;
        }
    }
    const bool ok = token >= 0 && static_cast<uint32_t>(token) < vocab;
    const uint16_t* row = table + static_cast<uint64_t>(ok ? token : 0) * hidden;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < hidden; i += gridDim.x * kBlock)
    {
        x[i] = ok ? HalfBitsToFloat(row[i]) : 0.0f;
        if (zero != nullptr)
        {
            zero[i] = 0.0f;
        }
    }
}

__global__ __launch_bounds__(kBlock) void FinalizeKernel(DecodeState* state, const float* __restrict__ argValue,
                                                         const int32_t* __restrict__ argIndex, uint32_t argBlocks,
                                                         const int32_t* sampled, int32_t* __restrict__ ids,
                                                         uint32_t idsCap)
{
    const int32_t token = sampled != nullptr ? *sampled : ReduceArgMaxPartials(argValue, argIndex, argBlocks);
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
// Attention over the fp16 cache: one workgroup per (chunk, kv head, query head of its GQA group).
//
// Keys are dealt to the chunks in blocks of kSlices consecutive keys, block b to chunk b % G (G
// is the grid's chunk count). A chunk's first blocks are therefore known before the position is:
// the first round of K/V rows is requested at entry, together with q, and the position, which
// arrives meanwhile, only masks it. Dealt this way the keys also spread evenly over the chunks at
// every position. The 256 lanes form kSlices groups of kRC = headDim/8 lanes; a group owns one
// key of each block and each of its lanes one 16-byte slice of that key's K and V rows. Scores
// are kept in log2 units (q.k * scale * log2 e), so each softmax weight is a single exp2. At the
// end the slices are combined inside each wave by lane permutes and across the four waves through
// LDS, and the chunk's partial (max, sum, P.V) goes to the merge; a chunk without keys writes the
// neutral partial (-inf, 0, 0), so the merge needs no position either.

constexpr float kLog2e = 1.4426950408889634f;

template <int kLane>
__device__ __forceinline__ float FromOctetLane(float v)
{
    // ds_swizzle bit mode: source lane (L & 0x18) | kLane within each 32 lanes.
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (kLane << 5)));
}

/// out[k] = v of lane k of this lane's octet, for k < 8.
__device__ __forceinline__ void OctetBroadcast8(float v, float (&out)[8])
{
    out[0] = FromOctetLane<0>(v);
    out[1] = FromOctetLane<1>(v);
    out[2] = FromOctetLane<2>(v);
    out[3] = FromOctetLane<3>(v);
    out[4] = FromOctetLane<4>(v);
    out[5] = FromOctetLane<5>(v);
    out[6] = FromOctetLane<6>(v);
    out[7] = FromOctetLane<7>(v);
}
// kAttnBlocksPerRound (decode_kernels.hpp) key blocks per lane per round: 2048 keys of a 2048-row
// cache in one round with the long grids.

/// Sum (kMax false) or maximum over the slices of one wave: the lanes equal modulo kRC. Every
/// lane ends with the same bit pattern as the others of its class (each step combines the same
/// two values).
template <int kRC, bool kMax>
__device__ __forceinline__ float SliceReduce(float v)
{
    static_assert(kRC == 8 || kRC == 16, "slice width");
    auto op = [](float a, float b) { return kMax ? fmaxf(a, b) : a + b; };
    if constexpr (kRC == 8)
    {
        // row_ror:8 pairs lane i with lane i ^ 8 inside each 16-lane row.
        v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x128, 0xF, 0xF,
                                                             false)));
    }
    // Rows 2r and 2r+1, then the two halves of the wave.
    const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(rows[0]), __uint_as_float(rows[1]));
    const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(halves[0]), __uint_as_float(halves[1]));
}

template <int kHd>
__global__ __launch_bounds__(kBlock) void AttentionChunk(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         const int32_t* __restrict__ position, uint32_t group,
                                                         uint32_t maxSeq, float scale, DecodeScratch sc)
{
    constexpr int kRC = kHd / 8;           // lanes per key
    constexpr int kSlices = kBlock / kRC;  // keys of a block, side by side
    constexpr int kR = static_cast<int>(kAttnBlocksPerRound);
    static_assert(kSlices == 2048 / kHd, "slice count must match AttnSlices");
    static_assert(kHd <= kBlock, "one thread per channel in the final sums");
    __shared__ float waveMax[kWaves];
    __shared__ float waveSum[kWaves];
    __shared__ float combine[kWaves][kHd];

    const uint32_t chunk = blockIdx.x;
    const uint32_t chunks = gridDim.x;
    const uint32_t g = blockIdx.y;
    const uint32_t h = blockIdx.z;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t slice = threadIdx.x / kRC;
    const uint32_t part = threadIdx.x % kRC;
    const half8* kBase = reinterpret_cast<const half8*>(kc + static_cast<uint64_t>(g) * maxSeq * kHd) + part;
    const half8* vBase = reinterpret_cast<const half8*>(vc + static_cast<uint64_t>(g) * maxSeq * kHd) + part;
    auto keyOf = [&](uint32_t block) { return (block * chunks + chunk) * kSlices + slice; };

    // Round 0 before the position: q, then this chunk's first kR blocks of K, then of V, clamped
    // into the cache. Loads complete in order, so the scores wait only for q and K while the V
    // rows are still arriving.
    const float4* qh = reinterpret_cast<const float4*>(q + (static_cast<uint64_t>(g) * group + h) * kHd) + part * 2;
    const float4 q0 = qh[0];
    const float4 q1 = qh[1];
    half8 kk[kR], vv[kR];
#pragma unroll
    for (int k = 0; k < kR; ++k)
    {
        kk[k] = kBase[static_cast<uint64_t>(min(keyOf(k), maxSeq - 1)) * kRC];
    }
#pragma unroll
    for (int k = 0; k < kR; ++k)
    {
        vv[k] = vBase[static_cast<uint64_t>(min(keyOf(k), maxSeq - 1)) * kRC];
    }
    __builtin_amdgcn_sched_barrier(0);
    const int32_t pos = *position;
    // Positions outside the cache are refused on the host; here they leave every chunk neutral.
    const uint32_t keys = pos >= 0 && static_cast<uint32_t>(pos) < maxSeq ? static_cast<uint32_t>(pos) + 1 : 0;
    const uint32_t blocks = (keys + kSlices - 1) / kSlices;
    const uint32_t mine = chunk < blocks ? (blocks - chunk + chunks - 1) / chunks : 0;  // this chunk's blocks
    const uint64_t slot = (static_cast<uint64_t>(g) * chunks + chunk) * group + h;
    if (mine == 0)
    {
        for (uint32_t d = threadIdx.x; d < kHd; d += kBlock)
        {
            sc.attnAcc[slot * kHd + d] = 0.0f;
        }
        if (threadIdx.x == 0)
        {
            sc.attnMax[slot] = -INFINITY;
            sc.attnSum[slot] = 0.0f;
        }
        return;
    }
    const float sl = scale * kLog2e;
    float m = -INFINITY;
    float l = 0.0f;
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
    {
        acc[c] = 0.0f;
    }
    // Online softmax over one round of blocks b0 .. b0 + kR - 1. Keys past the position and
    // blocks past this chunk's are masked; their rows may hold anything, so their V is zeroed as
    // well as weighted by 0.
    static_assert(kR == 8, "the scores' reduce-scatter gives each lane of an octet one of eight blocks");
    auto consume = [&](uint32_t b0) {
        float s[kR];
        bool valid[kR];
#pragma unroll
        for (int k = 0; k < kR; ++k)
        {
            // Blocks past this chunk's hold keys past the last (block * chunks + chunk >= blocks).
            valid[k] = keyOf(b0 + k) < keys;
            s[k] = DotChunk(kk[k], q0, q1, 0.0f);
        }
        // Reduce-scatter the slice's partial dot products: lane L ends with the score of block
        // L % 8 (both octets of a 16-lane slice hold all eight), so the max, the exponential
        // and the sum run once per block instead of once per lane and block.
        float sj = OctetScatter8(s);
        if constexpr (kRC == 16)
        {
            sj += DppMove<0x128>(sj);  // the slice's other octet (row_ror:8)
        }
        const uint32_t j = threadIdx.x & 7u;
        sj = keyOf(b0 + j) < keys ? sj * sl : -INFINITY;
        const float top = fmaxf(m, GroupMax<8>(sj));
        if (top == -INFINITY)
        {
            return;  // no valid key for this slice yet
        }
#pragma unroll
        for (int k = 0; k < kR; ++k)
        {
            if (!valid[k])
            {
                vv[k] = half8{};  // 0 * NaN would be NaN
            }
        }
        const float factor = exp2f(m - top);  // 0 while m is still -inf
        m = top;
        const float pj = exp2f(sj - top);  // masked keys: exp2(-inf) = 0
        l = fmaf(l, factor, GroupSum<8>(pj));
        // Every lane takes block k's weight from lane k of its octet.
        float p[kR];
        OctetBroadcast8(pj, p);
#pragma unroll
        for (int c = 0; c < 8; ++c)
        {
            float a = acc[c] * factor;
#pragma unroll
            for (int k = 0; k < kR; ++k)
            {
                a = fmaf(p[k], static_cast<float>(vv[k][c]), a);
            }
            acc[c] = a;
        }
    };
    consume(0);
    // Caches longer than one round's reach (kR * chunks * kSlices keys): further rounds, their
    // rows clamped to the last key.
    for (uint32_t b0 = kR; b0 < mine; b0 += kR)
    {
#pragma unroll
        for (int k = 0; k < kR; ++k)
        {
            const uint32_t key = min(keyOf(b0 + k), keys - 1);
            kk[k] = kBase[static_cast<uint64_t>(key) * kRC];
            vv[k] = vBase[static_cast<uint64_t>(key) * kRC];
        }
        consume(b0);
    }

    // Combine the slices: the chunk's max (slices of a wave by permutes, then the waves), then
    // the rescaled sums the same way.
    const float mw = SliceReduce<kRC, true>(m);
    if ((threadIdx.x & (kWave - 1)) == 0)
    {
        waveMax[wave] = mw;
    }
    __syncthreads();
    float top = waveMax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
    {
        top = fmaxf(top, waveMax[w]);
    }
    const float f = m == -INFINITY ? 0.0f : exp2f(m - top);
    const float lw = SliceReduce<kRC, false>(l * f);
#pragma unroll
    for (int c = 0; c < 8; ++c)
    {
        acc[c] = SliceReduce<kRC, false>(acc[c] * f);
    }
    if ((threadIdx.x & (kWave - 1)) < kRC)
    {
#pragma unroll
        for (int c = 0; c < 8; ++c)
        {
            combine[wave][part * 8 + c] = acc[c];
        }
        if (part == 0)
        {
            waveSum[wave] = lw;
        }
    }
    __syncthreads();
    // Thread d < kHd sums channel d; thread 0 also the chunk's max and sum.
    if (threadIdx.x < kHd)
    {
        const uint32_t d = threadIdx.x;
        float sum = combine[0][d];
#pragma unroll
        for (int w = 1; w < kWaves; ++w)
        {
            sum += combine[w][d];
        }
        sc.attnAcc[slot * kHd + d] = sum;
        if (d == 0)
        {
            float total = waveSum[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w)
            {
                total += waveSum[w];
            }
            sc.attnMax[slot] = top;
            sc.attnSum[slot] = total;
        }
    }
}

/// Combine the chunk partials of one query head (max in log2 units): every slot of the grid, the
/// neutral ones weighing 0. No valid chunk at all (a refused position) gives 0.
__device__ __forceinline__ float MergeChunks(const float* m, const float* l, const float* a, uint32_t n, float* den)
{
    float top = -INFINITY;
    for (uint32_t c = 0; c < n; ++c)
    {
        top = fmaxf(top, m[c]);
    }
    float num = 0.0f;
    float sum = 0.0f;
    if (top != -INFINITY)
    {
        for (uint32_t c = 0; c < n; ++c)
        {
            const float e = exp2f(m[c] - top);
            num = fmaf(e, a[c], num);
            sum = fmaf(e, l[c], sum);
        }
    }
    *den = sum;
    return num;
}

/// Combine the chunk partials of every query head: one workgroup per head, a thread per channel.
__global__ __launch_bounds__(128) void AttentionMergeKernel(DecodeScratch sc, float* __restrict__ out, uint32_t group,
                                                            uint32_t headDim, uint32_t gridChunks)
{
    const uint32_t h = blockIdx.x;
    const uint32_t g = h / group;
    const uint32_t hh = h % group;
    for (uint32_t d = threadIdx.x; d < headDim; d += blockDim.x)
    {
        float m[kMaxAttnChunks];
        float l[kMaxAttnChunks];
        float a[kMaxAttnChunks];
#pragma unroll
        for (uint32_t c = 0; c < kMaxAttnChunks; ++c)
        {
            const uint32_t cc = min(c, gridChunks - 1);
            const uint64_t slot = (static_cast<uint64_t>(g) * gridChunks + cc) * group + hh;
            m[c] = c < gridChunks ? sc.attnMax[slot] : -INFINITY;
            l[c] = sc.attnSum[slot];
            a[c] = sc.attnAcc[slot * headDim + d];
        }
        float den = 0.0f;
        const float num = MergeChunks(m, l, a, kMaxAttnChunks, &den);
        out[static_cast<uint64_t>(h) * headDim + d] = den > 0.0f ? num / den : 0.0f;
    }
}

constexpr int kOProjThreads = 512;
constexpr uint32_t kOProjWaves = kOProjThreads / kWave;

/// v plus the value of the same lane in the paired 16-lane row (rows 0 and 1, 2 and 3).
__device__ __forceinline__ float RowPairSum(float v)
{
    const auto pair = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(pair[0]) + __uint_as_float(pair[1]);
}

/// v plus the value of the same lane in the other half of the wave.
__device__ __forceinline__ float HalfPairSum(float v)
{
    const auto pair = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(pair[0]) + __uint_as_float(pair[1]);
}

/// o_proj split by kv group, with the attention merge in its prologue. Workgroup (b, g) of 512
/// threads owns group g's query heads, the W_o columns [g * gw, (g + 1) * gw) with gw = group *
/// headDim (at most 1024), and rows b * 8 + w + k * 8 * gridDim.x (k < kRows <= 8) for its wave w.
/// Wave h merges query head h (group <= 8, kCh = headDim / 64): lane c turns chunk c's (max, sum)
/// into its weight 2^(m_c - M) / sum_c' 2^(m_c' - M) l_c', so the exponentials and the division
/// run once per chunk rather than once per channel. The head's chunk rows arrive as 16-byte
/// loads that each cover 4 / kCh chunks side by side (headDim 128: 8 loads instead of 16 of 8
/// bytes); every lane weighs its chunks with the weights read from their lanes, and the lane
/// groups' sums meet by lane swaps. The merge
/// operands are requested before the weight rows (loads complete in order) and merged into LDS
/// while the rows are in flight. The rows' dots, reduced by ScatterSum8, go to parts[g][row],
/// group 0 adding the residual; the next kernel's prologue sums the groups. A workgroup reads one
/// group's partials instead of every head's: gridChunks * gw floats.
template <int kRows, int kCh>
__global__ __launch_bounds__(kOProjThreads) void OProjGroupKernel(const uint16_t* __restrict__ wo, DecodeScratch sc,
                                                                  const float* __restrict__ residual, float* out,
                                                                  uint32_t hidden,
                                                                  uint32_t qdim, uint32_t group, uint32_t headDim,
                                                                  uint32_t gridChunks)
{
    static_assert(kRows >= 1 && kRows <= 8, "ScatterSum8 reduces eight rows");
    constexpr int kCpl = 2;
    __shared__ float4 xs[2 * kWave * kCpl];
    const uint32_t g = blockIdx.y;
    const uint32_t gw = group * headDim;
    const uint32_t nchunks = gw / 8;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t stride = kOProjWaves * gridDim.x;
    const uint32_t first = blockIdx.x * kOProjWaves + wave;
    // Merge operands first. Waves past the group's heads repeat the last head's (unused) loads,
    // which keeps the loads out of branches.
    const uint32_t hh = min(wave, group - 1);
    const uint64_t headBase = static_cast<uint64_t>(g) * gridChunks * group + hh;  // slot of chunk 0
    const uint32_t lc = min(lane, gridChunks - 1);
    float m = sc.attnMax[headBase + static_cast<uint64_t>(lc) * group];
    const float l = sc.attnSum[headBase + static_cast<uint64_t>(lc) * group];
    // A head's P.V row is kQuads float4s: each 16-byte load covers kPerLoad chunks side by side
    // (lane group `sub` takes chunks sub, sub + kPerLoad, ...), so a wave requests its head's 16
    // chunks in kLoads loads.
    constexpr uint32_t kQuads = 16 * kCh;
    constexpr uint32_t kPerLoad = kWave / kQuads;
    constexpr uint32_t kLoads = kMaxAttnChunks / kPerLoad;
    static_assert(kPerLoad * kLoads == kMaxAttnChunks, "chunks per load");
    const uint32_t sub = lane / kQuads;
    const uint32_t quad = lane % kQuads;
    float4 a[kLoads];
#pragma unroll
    for (uint32_t i = 0; i < kLoads; ++i)
    {
        const uint64_t slot = headBase + static_cast<uint64_t>(min(i * kPerLoad + sub, gridChunks - 1)) * group;
        a[i] = *reinterpret_cast<const float4*>(sc.attnAcc + slot * headDim + 4 * quad);
    }
    half8 w[kRows][kCpl];
#pragma unroll
    for (int k = 0; k < kRows; ++k)
    {
        const uint32_t row = min(first + k * stride, hidden - 1);
        LoadBatch<kWave, kCpl>(wo + static_cast<uint64_t>(row) * qdim + g * gw, 0, nchunks, lane, w[k]);
    }
    // Lane k < kRows stores row first + k * stride. Every group loads the residual (group 0 adds
    // it): a load under a branch would leave the merge's waits unable to count it.
    const uint32_t myRow = first + (lane & 7u) * stride;
    const float resLoaded = residual[min(myRow, hidden - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const float res = g == 0 ? resLoaded : 0.0f;
    {
        m = lane < gridChunks ? m : -INFINITY;
        const float top = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(GroupMax<16>(m))));
        const float e = top == -INFINITY || m == -INFINITY ? 0.0f : exp2f(m - top);
        const float den = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(GroupSum<16>(e * l))));
        const float weight = den > 0.0f ? e / den : 0.0f;
        float4 merged = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t i = 0; i < kLoads; ++i)
        {
            // Chunk i * kPerLoad + sub's weight, read from that chunk's lane.
            float wc = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < kPerLoad; ++j)
            {
                const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(weight), i * kPerLoad + j));
                wc = sub == j ? wj : wc;
            }
            merged.x = fmaf(wc, a[i].x, merged.x);
            merged.y = fmaf(wc, a[i].y, merged.y);
            merged.z = fmaf(wc, a[i].z, merged.z);
            merged.w = fmaf(wc, a[i].w, merged.w);
        }
        // The lane groups' sums: rows 2r and 2r + 1 (16-lane groups), then the wave's halves.
        if constexpr (kPerLoad == 4)
        {
            merged = float4{RowPairSum(merged.x), RowPairSum(merged.y), RowPairSum(merged.z), RowPairSum(merged.w)};
        }
        if constexpr (kPerLoad >= 2)
        {
            merged = float4{HalfPairSum(merged.x), HalfPairSum(merged.y), HalfPairSum(merged.z),
                            HalfPairSum(merged.w)};
        }
        if (wave < group && sub == 0)
        {
            // Channels ch .. ch + 3 of the group sit in chunk ch / 8: its low float4 for
            // ch % 8 == 0, its high one for ch % 8 == 4.
            const uint32_t ch = hh * headDim + 4 * quad;
            const uint32_t at = ch % 8 == 0 ? 4 * (ch / 8) : 4 * nchunks + 4 * (ch / 8);
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(xs) + at) = merged;
        }
    }
    __syncthreads();
    float4 xlo[kCpl];
    float4 xhi[kCpl];
    LoadActivation<kWave, kCpl>(xs, xs + nchunks, nchunks, lane, xlo, xhi);
    float sums[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
    {
        sums[k] = k < kRows ? DotRegisters<kWave, kCpl>(w[k < kRows ? k : 0], xlo, xhi, nchunks, lane) : 0.0f;
    }
    const float total = ScatterSum8(sums);
    // The kvHeads groups' sums meet in `out` (zeroed by the previous kernel): one atomic add per
    // group and row, so the adds to an element never queue more than kvHeads deep.
    if (lane < static_cast<uint32_t>(kRows) && myRow < hidden)
    {
        __hip_atomic_fetch_add(out + myRow, res + total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        float c;
        float s;
        sincosf(theta, &s, &c);
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
    GemvShape shape{};
    LmHeadEpi epi{};
    epi.rows = dims.vocab;
    (void)LaunchFused<1>(nullptr, dims.vocab, kArgMaxBlocks, dims.hidden,
                         NormStage{nullptr, nullptr, 0.0f}, epi, &shape);
    return shape.blocks;
}

bool MergeInOProj(const DecodeDims& dims)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    return qdim <= kMergeItems * kBlock && dims.headDim % 4 == 0;
}

hipError_t LaunchSetState(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, int32_t token,
                          int32_t position, uint32_t argBlocks, uint32_t step)
{
    hipLaunchKernelGGL(SetStateKernel, dim3(1), dim3(kBlock), 0, s, state, scratch.argValue, scratch.argIndex,
                       scratch.sampled, token, position, argBlocks, step);
    return hipGetLastError();
}

hipError_t LaunchBeginStep(hipStream_t s, const uint16_t* table, DecodeState* state, const DecodeScratch& scratch,
                           uint32_t argBlocks, float* x, int32_t* ids, uint32_t idsCap, uint32_t hidden,
                           uint32_t vocab, float* zero)
{
    hipLaunchKernelGGL(BeginStepKernel, dim3(CeilDiv(hidden, kBlock)), dim3(kBlock), 0, s, table, state,
                       scratch.argValue, scratch.argIndex, argBlocks, scratch.sampled, scratch.history,
                       scratch.historyCap, x, zero, ids, idsCap, hidden, vocab);
    return hipGetLastError();
}

hipError_t LaunchFinalize(hipStream_t s, DecodeState* state, const DecodeScratch& scratch, uint32_t argBlocks,
                          int32_t* ids, uint32_t idsCap)
{
    hipLaunchKernelGGL(FinalizeKernel, dim3(1), dim3(kBlock), 0, s, state, scratch.argValue, scratch.argIndex,
                       argBlocks, scratch.sampled, ids, idsCap);
    return hipGetLastError();
}

hipError_t LaunchQkvRopeAppend(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                               const uint16_t* wqkv, const float* bias, const DecodeState* state, float* qOut,
                               uint16_t* kcache, uint16_t* vcache, uint32_t xParts)
{
    QkvEpi epi{wqkv,       bias,         state,        qOut,         kcache,
               vcache,     dims.ropePow, dims.hidden,  dims.heads,   dims.kvHeads,
               dims.headDim, dims.maxSeq};
    const uint32_t units = (dims.heads + 2 * dims.kvHeads) * dims.headDim / 2;
    if (xParts == kResidualParts)
    {
        return LaunchFused<2>(s, units, kNoLimit, dims.hidden, SumNormStage{x, normW, dims.eps}, epi);
    }
    if (xParts != 1)
    {
        return hipErrorInvalidValue;
    }
    return LaunchFused<2>(s, units, kNoLimit, dims.hidden, NormStage{x, normW, dims.eps}, epi);
}

template <int kHd>
hipError_t LaunchAttentionT(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                            const uint16_t* vcache, const int32_t* position, const DecodeScratch& scratch)
{
    const uint32_t group = dims.heads / dims.kvHeads;
    const dim3 grid(AttnGridChunks(dims.maxSeq, kHd, dims.attnChunks), dims.kvHeads, group);
    hipLaunchKernelGGL(AttentionChunk<kHd>, grid, dim3(kBlock), 0, s, q, kcache, vcache, position, group, dims.maxSeq,
                       dims.attnScale, scratch);
    return hipGetLastError();
}

hipError_t LaunchAttention(hipStream_t s, const DecodeDims& dims, const float* q, const uint16_t* kcache,
                           const uint16_t* vcache, const int32_t* position, const DecodeScratch& scratch)
{
    if (dims.kvHeads == 0 || dims.heads % dims.kvHeads != 0 || dims.heads / dims.kvHeads > kMaxGroup ||
        dims.maxSeq == 0 || dims.maxSeq > kMaxSeq || dims.attnChunks == 0 || dims.attnChunks > kMaxAttnChunks)
    {
        return hipErrorInvalidValue;
    }
    switch (dims.headDim)
    {
        case 64:
            return LaunchAttentionT<64>(s, dims, q, kcache, vcache, position, scratch);
        case 128:
            return LaunchAttentionT<128>(s, dims, q, kcache, vcache, position, scratch);
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t LaunchAttentionMerge(hipStream_t s, const DecodeDims& dims, const DecodeScratch& scratch, float* out)
{
    hipLaunchKernelGGL(AttentionMergeKernel, dim3(dims.heads), dim3(std::min<uint32_t>(dims.headDim, 128)), 0, s,
                       scratch, out, dims.heads / dims.kvHeads, dims.headDim,
                       AttnGridChunks(dims.maxSeq, dims.headDim, dims.attnChunks));
    return hipGetLastError();
}

template <class Epi>
hipError_t LaunchOProjMergedT(hipStream_t s, const DecodeDims& dims, const DecodeScratch& scratch, const Epi& epi)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    const uint32_t chunks = AttnGridChunks(dims.maxSeq, dims.headDim, dims.attnChunks);
    if (chunks <= kShortAttnChunks)
    {
        MergeStage<kShortAttnChunks> stage{scratch.attnMax, scratch.attnSum, scratch.attnAcc, dims.heads,
                                           dims.heads / dims.kvHeads, dims.headDim, chunks};
        return LaunchFused<1>(s, dims.hidden, kNoLimit, qdim, stage, epi);
    }
    MergeStage<kMergeAttnChunks> stage{scratch.attnMax, scratch.attnSum, scratch.attnAcc, dims.heads,
                                       dims.heads / dims.kvHeads, dims.headDim, chunks};
    return LaunchFused<1>(s, dims.hidden, kNoLimit, qdim, stage, epi);
}

hipError_t LaunchOProjMerged(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const DecodeScratch& scratch,
                             const float* residual, float* out, uint32_t residualParts, float* parts)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    if (residualParts == 1 && parts == nullptr)
    {
        return LaunchOProjMergedT(s, dims, scratch, ResidualEpi{wo, residual, out, dims.hidden, qdim});
    }
    if (residualParts != 1 && residualParts != kResidualParts)
    {
        return hipErrorInvalidValue;
    }
    return LaunchOProjMergedT(s, dims, scratch,
                              ResidualPartsEpi{wo, residual, out, parts, dims.hidden, qdim, residualParts});
}

hipError_t LaunchOProjPlain(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const float* attn,
                            const float* residual, float* out, uint32_t residualParts, float* parts)
{
    const uint32_t qdim = dims.heads * dims.headDim;
    if (residualParts == 1 && parts == nullptr)
    {
        return LaunchMatVecResidual(s, wo, attn, residual, out, dims.hidden, qdim);
    }
    if (residualParts != 1 && residualParts != kResidualParts)
    {
        return hipErrorInvalidValue;
    }
    return LaunchFused<1>(s, dims.hidden, kNoLimit, qdim, PlainStage{attn},
                          ResidualPartsEpi{wo, residual, out, parts, dims.hidden, qdim, residualParts});
}

/// Groups whose o_proj sums meet in one element by atomic adds: more would queue the adds to an
/// element deeper (they serialise at the memory).
constexpr uint32_t kMaxOProjGroups = 4;

bool OProjInGroups(const DecodeDims& dims)
{
    const uint32_t gw = dims.heads / dims.kvHeads * dims.headDim;
    // A wave merges one head (at most eight a workgroup) with 1, 2 or 4 channels per lane.
    const uint32_t group = dims.heads / dims.kvHeads;
    const uint32_t channels = dims.headDim / kWave;
    return !MergeInOProj(dims) && gw <= 2 * kWave * 8 && group <= kOProjWaves && dims.headDim % kWave == 0 &&
           (channels == 1 || channels == 2 || channels == 4) && dims.kvHeads <= kMaxOProjGroups;
}

template <int kRows, int kCh>
hipError_t LaunchOProjGroupsT(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const DecodeScratch& scratch,
                              const float* residual, float* out)
{
    const dim3 grid(CeilDiv(dims.hidden, kOProjWaves * kRows), dims.kvHeads);
    const auto kernel = &OProjGroupKernel<kRows, kCh>;
    hipLaunchKernelGGL(kernel, grid, dim3(kOProjThreads), 0, s, wo, scratch, residual, out, dims.hidden,
                       dims.heads * dims.headDim, dims.heads / dims.kvHeads, dims.headDim,
                       AttnGridChunks(dims.maxSeq, dims.headDim, dims.attnChunks));
    return hipGetLastError();
}

template <int kRows>
hipError_t LaunchOProjGroupsRows(hipStream_t s, const DecodeDims& dims, const uint16_t* wo,
                                 const DecodeScratch& scratch, const float* residual, float* out)
{
    switch (dims.headDim / kWave)
    {
        case 1:
            return LaunchOProjGroupsT<kRows, 1>(s, dims, wo, scratch, residual, out);
        case 2:
            return LaunchOProjGroupsT<kRows, 2>(s, dims, wo, scratch, residual, out);
        default:
            return LaunchOProjGroupsT<kRows, 4>(s, dims, wo, scratch, residual, out);
    }
}

hipError_t LaunchOProjGroups(hipStream_t s, const DecodeDims& dims, const uint16_t* wo, const DecodeScratch& scratch,
                             const float* residual, float* out)
{
    if (!OProjInGroups(dims))
    {
        return hipErrorInvalidValue;
    }
    // About one workgroup (eight waves) per CU: the rows of each group spread over CUs / groups
    // workgroups.
    const uint32_t waves = std::max(1u, CuCount() * kOProjWaves / dims.kvHeads);
    const uint32_t perWave = CeilDiv(dims.hidden, waves);
    if (perWave <= 1)
    {
        return LaunchOProjGroupsRows<1>(s, dims, wo, scratch, residual, out);
    }
    if (perWave <= 2)
    {
        return LaunchOProjGroupsRows<2>(s, dims, wo, scratch, residual, out);
    }
    if (perWave <= 4)
    {
        return LaunchOProjGroupsRows<4>(s, dims, wo, scratch, residual, out);
    }
    if (perWave <= 7)
    {
        return LaunchOProjGroupsRows<7>(s, dims, wo, scratch, residual, out);
    }
    return LaunchOProjGroupsRows<8>(s, dims, wo, scratch, residual, out);
}

hipError_t LaunchMatVecResidualZero(hipStream_t s, const uint16_t* w, const float* x, const float* residual,
                                    float* out, float* zero, uint32_t rows, uint32_t cols)
{
    ResidualZeroEpi epi{};
    epi.w = w;
    epi.residual = residual;
    epi.out = out;
    epi.rows = rows;
    epi.cols = cols;
    epi.zero = zero;
    return LaunchFused<1>(s, rows, kNoLimit, cols, PlainStage{x}, epi);
}

hipError_t LaunchMatVecResidual(hipStream_t s, const uint16_t* w, const float* x, const float* residual, float* out,
                                uint32_t rows, uint32_t cols)
{
    ResidualEpi epi{w, residual, out, rows, cols};
    return LaunchFused<1>(s, rows, kNoLimit, cols, PlainStage{x}, epi);
}

hipError_t LaunchMatVecBias(hipStream_t s, const uint16_t* w, const float* x, const float* bias0, const float* bias1,
                            float* out, uint32_t rows, uint32_t cols)
{
    BiasEpi epi{w, bias0, bias1, out, rows, cols};
    return LaunchFused<1>(s, rows, kNoLimit, cols, PlainStage{x}, epi);
}

hipError_t LaunchGateUpSwiGlu(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* wgate, const uint16_t* wup, float* act)
{
    GateUpEpi epi{wgate, wup, act, dims.ffn, dims.hidden};
    return LaunchFused<2>(s, dims.ffn, kNoLimit, dims.hidden, NormStage{x, normW, dims.eps}, epi);
}

bool FfnFusable(const DecodeDims& dims)
{
    return dims.hidden >= 8 && dims.hidden <= 8 * kFfnMaxChunks && dims.hidden % 8 == 0 && dims.ffn >= 1 &&
           !OProjInGroups(dims);
}

hipError_t LaunchFfnFused(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                          const uint16_t* wgate, const uint16_t* wup, const uint16_t* downT, float* parts)
{
    if (!FfnFusable(dims))
    {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(FfnFusedKernel, dim3(CeilDiv(dims.ffn, kFfnUnits)), dim3(kBlock), 0, s, x, normW, wgate, wup,
                       downT, parts, dims.hidden, dims.ffn, dims.eps);
    return hipGetLastError();
}

hipError_t LaunchTransposeF16(hipStream_t s, const uint16_t* src, uint16_t* dst, uint32_t rows, uint32_t cols)
{
    if (rows == 0 || cols == 0)
    {
        return hipSuccess;
    }
    hipLaunchKernelGGL(TransposeF16Kernel, dim3(CeilDiv(cols, 64u), CeilDiv(rows, 64u)), dim3(kBlock), 0, s, src,
                       dst, rows, cols);
    return hipGetLastError();
}

hipError_t LaunchLmHeadArgMax(hipStream_t s, const DecodeDims& dims, const float* x, const float* normW,
                              const uint16_t* table, float* logits, const DecodeScratch& scratch)
{
    LmHeadEpi epi{table, logits, scratch.argValue, scratch.argIndex, dims.vocab, dims.hidden};
    return LaunchFused<1>(s, dims.vocab, kArgMaxBlocks, dims.hidden,
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
/// Floats of chunk partials one attention call needs: (max, sum) and head_dim accumulators per
/// (kv head, chunk, query head of the group).
size_t AttentionScratchFloats(uint32_t heads, uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq)
{
    const size_t slots = static_cast<size_t>(kvHeads) * AttnGridChunks(maxSeq, headDim, kMaxAttnChunks) *
                         (heads / kvHeads);
    return slots * (2 + headDim);
}

int CheckAttentionArgs(const char* name, const float* q, const void* kcache, const void* vcache, const float* out,
                       const int32_t* position, uint32_t heads, uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq)
{
    if (q == nullptr || kcache == nullptr || vcache == nullptr || out == nullptr || position == nullptr)
    {
        return Fail(MUYO_E_NULL, "%s: q, caches, out and position are required", name);
    }
    if (kvHeads == 0 || heads % kvHeads != 0 || heads / kvHeads > kMaxGroup || (headDim != 64 && headDim != 128) ||
        maxSeq == 0 || maxSeq > kMaxSeq)
    {
        return Fail(MUYO_E_UNSUPPORTED,
                    "%s: needs heads %% kv_heads == 0, group <= 8, head_dim 64 or 128, max_seq <= %u", name,
                    kMaxSeq);
    }
    if (!Aligned16(q) || !Aligned16(kcache) || !Aligned16(vcache))
    {
        return Fail(MUYO_E_CONTRACT, "%s: q and the caches must be 16-byte aligned", name);
    }
    return MUYO_OK;
}

/// Attention chunks + merge with the partials in `base` (AttentionScratchFloats floats). Every
/// slot is written before it is read (a chunk without keys writes the neutral partial), so the
/// buffer needs no clearing between calls.
int RunAttentionDecode(const char* name, const float* q, const void* kcache, const void* vcache, float* out,
                       const int32_t* position, uint32_t heads, uint32_t kvHeads, uint32_t headDim, uint32_t maxSeq,
                       float scale, float* base, void* stream)
{
    const size_t slots = AttentionScratchFloats(heads, kvHeads, headDim, maxSeq) / (2 + headDim);
    DecodeScratch scratch{};
    scratch.attnMax = base;
    scratch.attnSum = base + slots;
    scratch.attnAcc = base + 2 * slots;
    DecodeDims dims{};
    dims.heads = heads;
    dims.kvHeads = kvHeads;
    dims.headDim = headDim;
    dims.maxSeq = maxSeq;
    dims.attnScale = scale;
    dims.attnChunks = kMaxAttnChunks;
    hipError_t launched = LaunchAttention(AsStream(stream), dims, q, static_cast<const uint16_t*>(kcache),
                                          static_cast<const uint16_t*>(vcache), position, scratch);
    if (launched == hipSuccess)
    {
        launched = LaunchAttentionMerge(AsStream(stream), dims, scratch, out);
    }
    return launched == hipSuccess ? MUYO_OK : HipStatus(launched, name);
}
}  // namespace

extern "C" size_t muyo_attention_decode_f16kv_workspace_bytes(uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                                                              uint32_t max_seq)
{
    if (kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > kMaxGroup || (head_dim != 64 && head_dim != 128) ||
        max_seq == 0 || max_seq > kMaxSeq)
    {
        return 0;
    }
    return AttentionScratchFloats(heads, kv_heads, head_dim, max_seq) * sizeof(float);
}

extern "C" int muyo_attention_decode_f16kv(const float* q, const void* kcache, const void* vcache, float* out,
                                           const int32_t* position, uint32_t heads, uint32_t kv_heads,
                                           uint32_t head_dim, uint32_t max_seq, float scale, void* workspace,
                                           uint64_t workspace_bytes, void* stream)
{
    const char* name = "attention_decode_f16kv";
    const int args = CheckAttentionArgs(name, q, kcache, vcache, out, position, heads, kv_heads, head_dim, max_seq);
    if (args != MUYO_OK)
    {
        return args;
    }
    const size_t need = AttentionScratchFloats(heads, kv_heads, head_dim, max_seq) * sizeof(float);
    if (workspace == nullptr || !Aligned16(workspace) || workspace_bytes < need)
    {
        return Fail(MUYO_E_CONTRACT, "%s: needs a 16-byte aligned workspace of %zu bytes (got %llu)", name, need,
                    static_cast<unsigned long long>(workspace_bytes));
    }
    return RunAttentionDecode(name, q, kcache, vcache, out, position, heads, kv_heads, head_dim, max_seq, scale,
                              static_cast<float*>(workspace), stream);
}

// ------------------------------------------------------------------------------------------------
// The same attention with no allocation and no workspace argument, for callers that cannot
// allocate (code under graph capture, serving loops that forbid hipMalloc): the chunk partials
// live in a fixed device array. The array's name is a host-side stand-in; its device address is
// looked up once per device with hipGetSymbolAddress and only that address reaches the kernels.

constexpr size_t kStaticScratchFloats = 131072;  // 512 KiB per device, held until the process ends
static __device__ __align__(256) float scratch[kStaticScratchFloats];

namespace
{
std::mutex g_scratchMutex;
float* g_scratchAddress[kMaxDevices] = {};

/// This device's copy of `scratch` (looked up on the first call on the device, with it current).
int StaticScratch(const char* name, float** out)
{
    int device = 0;
    const hipError_t got = hipGetDevice(&device);
    if (got != hipSuccess)
    {
        return HipStatus(got, name);
    }
    if (device < 0 || device >= kMaxDevices)
    {
        return Fail(MUYO_E_UNSUPPORTED, "%s: device %d is past the %d devices this entry point serves", name, device,
                    kMaxDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratchMutex);
    if (g_scratchAddress[device] == nullptr)
    {
        void* address = nullptr;
        const hipError_t status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (status != hipSuccess || address == nullptr)
        {
            return Fail(status != hipSuccess ? static_cast<int>(status) : MUYO_E_NOMEM,
                        "%s: hipGetSymbolAddress(scratch) failed: %s", name, hipGetErrorString(status));
        }
        g_scratchAddress[device] = static_cast<float*>(address);
    }
    *out = g_scratchAddress[device];
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_attention_decode_f16kv_static(const float* q, const void* kcache, const void* vcache, float* out,
                                                  const int32_t* position, uint32_t heads, uint32_t kv_heads,
                                                  uint32_t head_dim, uint32_t max_seq, float scale, void* stream)
{
    const char* name = "attention_decode_f16kv_static";
    const int args = CheckAttentionArgs(name, q, kcache, vcache, out, position, heads, kv_heads, head_dim, max_seq);
    if (args != MUYO_OK)
    {
        return args;
    }
    const size_t need = AttentionScratchFloats(heads, kv_heads, head_dim, max_seq);
    if (need > kStaticScratchFloats)
    {
        return Fail(MUYO_E_UNSUPPORTED,
                    "%s: this shape needs %zu bytes of partials, past the fixed %zu-byte device array "
                    "(use muyo_attention_decode_f16kv with a workspace)",
                    name, need * sizeof(float), kStaticScratchFloats * sizeof(float));
    }
    float* base = nullptr;
    const int status = StaticScratch(name, &base);
    if (status != MUYO_OK)
    {
        return status;
    }
    return RunAttentionDecode(name, q, kcache, vcache, out, position, heads, kv_heads, head_dim, max_seq, scale, base,
                              stream);
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
