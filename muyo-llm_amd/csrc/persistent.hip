// The persistent decode step (see persistent.hpp for the hand-off protocol).
//
// One workgroup per CU, 8 waves: wave 0 polls, waves 1..7 compute. Per layer the workgroups take
// roles (disjoint ranges spread over the XCDs), and every workgroup takes a share of the FFN:
//   Q  (qkvBlocks): 16 rope (or value) row pairs each: rms_norm'd x . W_qkv + bias, NeoX rope,
//                   q and the fp16-rounded k/v handed on, k/v written to the cache row
//   A  (attnUnits): one query head over one chunk of the cache (blocks of keys dealt round-robin
//                   to the chunks), the row at the position taken from the hand-off; online
//                   softmax; partial (P.V, max, sum) handed on
//   O  (rowBlocks): 16 rows of o_proj; its prologue merges every attention partial
//   all           : gate/up rows (a contiguous share of the FFN), swiglu, then that share's
//                   columns of down (from the transposed copy) as a partial of the whole output
//   R  (rowBlocks): the poller sums every workgroup's down partial for 16 rows, adds the residual
//                   and hands the layer output on
// then the LM head (each workgroup a contiguous share of the vocabulary, one argmax partial each).
// Five hand-offs per layer (q|k|v, attention partials, o_proj output, down partials, layer
// output). Each wait is one barrier for the compute waves, which meanwhile request the weights of
// their next phase.
#include <algorithm>

#include "common.hpp"
#include "gemv_core.hpp"
#include "persistent.hpp"

namespace muyo
{
namespace
{
constexpr int kStepWaves = 8;  // two waves per SIMD: up to 256 VGPRs each
constexpr int kStepThreads = kStepWaves * kWave;
constexpr int kComputeWaves = kStepWaves - 1;
constexpr uint32_t kMaxRow = 1024;    // longest GEMV row (hidden, heads * headDim)
constexpr uint32_t kMaxHidden = 896;  // the down partial's chunks: at most 16 per compute wave
constexpr int kRowCpl = 2;            // 16-byte chunks per lane of a 64-lane row of <= 1024 columns
constexpr uint32_t kMaxGrid = 256;     // workgroups (the down reduction gathers 16 packets from each)
constexpr uint32_t kAttBlock = 1280;   // an attention unit's q|k|v block: (group + 2) * headDim, at most
constexpr uint32_t kSlack = 4096;      // packets past the arena's regions (a gather's whole slice)
constexpr uint32_t kMaxLayers = kStepMaxLayers;
constexpr uint32_t kMaxPart = 4096;   // attention partials merged in o_proj's prologue
constexpr uint32_t kMaxChunks = 4;    // attention chunks per kv head
constexpr int kAttnPre = 9;           // attention key rounds held in registers
constexpr int kQkvPerWave = 3;        // QKV units (o_proj rows) of a 16-unit block per compute wave
constexpr int kGuPerWave = 3;         // gate/up units per compute wave
constexpr int kDownPerLane = 6;       // transposed down rows per lane
constexpr uint32_t kMaxFfnShare = 4 * kDownPerLane - 3;  // FFN rows per workgroup (21)
static_assert(kMaxFfnShare <= static_cast<uint32_t>(kGuPerWave * kComputeWaves), "gate/up units per wave");
constexpr int kPre = 2 * kGuPerWave * kRowCpl + kDownPerLane;  // 16-byte weight slots requested ahead (18)
constexpr int kLmLpr = 16;            // LM head: lanes per row
constexpr int kLmCpl = 8;             // LM head: chunks per lane (rows of <= 1024 columns)
constexpr float kLog2e = 1.4426950408889634f;
static_assert(kPre >= 2 * kAttnPre && kPre >= 12, "the weight slots hold every role's prefetch");

// Indices of the waits, for the error word.
enum Wait : uint32_t
{
    kWaitQkv = 0,
    kWaitPart = 1,
    kWaitMid = 2,
    kWaitDown = 3,
    kWaitX = 4,
};

struct StepShared
{
    float x[kMaxHidden];  // layer input: o_proj's residual
    float xn[kMaxRow];    // layer input after attn_norm (or output_norm before the LM head)
    float mid[kMaxHidden];  // after attention: the layer output's residual
    float midn[kMaxRow];  // after ffn_norm: the gate/up activation
    float att[kAttBlock]; // attention: q of the kv head's query heads, then its k and v
    float part[kMaxPart]; // every attention partial of the layer (o_proj prologue)
    float mergeW[16 * kMaxChunks];      // per (head, chunk): the chunk's weight in the merge
    float waveAttn[kComputeWaves][130]; // per compute wave: P.V, max, sum
    float act[kMaxFfnShare];
    float downOut[kComputeWaves][128];
    float bestValue[kComputeWaves];
    int32_t bestIndex[kComputeWaves];
    int32_t token;
    StepLayer layers[kMaxLayers];  // the per-layer pointers, copied once per step
};

__device__ __forceinline__ void Put(uint64_t* slot, float value, uint32_t epoch)
{
    __hip_atomic_store(slot, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(value), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool Abandoned(const uint32_t* control)
{
    return __hip_atomic_load(control + kStepAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

__device__ __noinline__ void GiveUp(uint32_t* control, uint32_t which)
{
    uint32_t none = 0;
    __hip_atomic_compare_exchange_strong(control + kStepError, &none, which + 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(control + kStepAbort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/// Poller: waits until packets src[i], i < n (n <= 64 * kPer), all carry `epoch`. Each pass
/// requests kPer packets per lane at once (one memory round trip; packets past n come from the
/// regions after, or the arena's slack, and are ignored), calls restart() and then take(i, value,
/// valid) for every slot i < 64 * kPer; a pass that found a packet not yet written is repeated.
/// No per-packet branches: validity is a per-lane select, so the pass needs no exec masks. `live`
/// turns false when this wait gives up or another one did; later waits then return at once.
template <int kPer, class Restart, class Take>
__device__ __forceinline__ void Gather(const uint64_t* __restrict__ src, uint32_t n, uint32_t epoch, Restart restart,
                                       Take take, uint32_t* control, uint32_t limit, uint32_t which, bool& live)
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint64_t* from = src + lane;  // packet k is 512 bytes further (an instruction offset)
    uint32_t spins = 0;
    while (live)
    {
        restart();
        // The base is made opaque on every pass, so the compiler forms each packet's address next
        // to its load (an instruction offset from a few bases) instead of hoisting one 64-bit
        // address per packet out of the retry loop and keeping them all live.
        using Global = const __attribute__((address_space(1))) uint64_t;
        Global* at = (Global*)from;  // a C cast: the only cast C++ allows into an address space
        asm volatile("" : "+v"(at));
        uint64_t d[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
        {
            d[k] = __hip_atomic_load(at + k * kWave, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        bool ready = true;
#pragma unroll
        for (int k = 0; k < kPer; ++k)
        {
            const uint32_t i = lane + k * kWave;
            const bool valid = i < n;
            ready = ready && (!valid || static_cast<uint32_t>(d[k] >> 32) == epoch);
            take(i, __uint_as_float(static_cast<uint32_t>(d[k])), valid);
        }
        if (__all(ready))
        {
            return;
        }
        ++spins;
        if (spins >= limit)
        {
            GiveUp(control, which);
            live = false;
            return;
        }
        if ((spins & 15) == 0 && Abandoned(control))
        {
            live = false;
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

/// Sum over the lanes that share lane % kFrom (lanes kFrom, 2 kFrom, ... apart; kFrom 8, 16 or 32).
template <int kFrom>
__device__ __forceinline__ float XorSum(float v)
{
    static_assert(kFrom == 8 || kFrom == 16 || kFrom == 32, "width");
    if constexpr (kFrom == 8)
    {
        // row_ror:8 pairs lane i with lane i ^ 8 inside each 16-lane row.
        v += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x128, 0xF, 0xF, false));
    }
    if constexpr (kFrom <= 16)
    {
        const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(rows[0]) + __uint_as_float(rows[1]);
    }
    const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(halves[0]) + __uint_as_float(halves[1]);
}

template <int kFrom>
__device__ __forceinline__ float XorMax(float v)
{
    static_assert(kFrom == 8 || kFrom == 16 || kFrom == 32, "width");
    if constexpr (kFrom == 8)
    {
        v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x128, 0xF, 0xF,
                                                                 false)));
    }
    if constexpr (kFrom <= 16)
    {
        const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(rows[0]), __uint_as_float(rows[1]));
    }
    const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(halves[0]), __uint_as_float(halves[1]));
}

/// Poller: rms_norm of the row held in `x` (n <= 1024, this lane's elements lane + 64k) into
/// `out`, in rms_norm.comp:122's order (scale * x) * w; `w` is this lane's weights, requested
/// before the wait.
__device__ __forceinline__ void PollerNorm(const float* x, const float (&w)[kMaxRow / kWave], uint32_t n, float eps,
                                           float* out)
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    float v[kMaxRow / kWave];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < static_cast<int>(kMaxRow / kWave); ++k)
    {
        const uint32_t i = lane + k * kWave;
        v[k] = i < n ? x[i] : 0.0f;
        ss = fmaf(v[k], v[k], ss);
    }
    ss = GroupSum<kWave>(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
    for (int k = 0; k < static_cast<int>(kMaxRow / kWave); ++k)
    {
        const uint32_t i = lane + k * kWave;
        if (i < n)
        {
            out[i] = (scale * v[k]) * w[k];
        }
    }
}

__device__ __forceinline__ void LoadNormWeights(const float* w, uint32_t n, float (&out)[kMaxRow / kWave])
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int k = 0; k < static_cast<int>(kMaxRow / kWave); ++k)
    {
        out[k] = w[min(lane + k * kWave, n - 1)];
    }
}

/// This lane's activation chunks (lane and lane + 64) of an LDS row of `n` floats.
__device__ __forceinline__ void RowActivation(const float* x, uint32_t n, float4 (&lo)[kRowCpl], float4 (&hi)[kRowCpl])
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t nchunks = n / 8;
#pragma unroll
    for (int i = 0; i < kRowCpl; ++i)
    {
        const uint32_t c = min(lane + i * kWave, nchunks - 1);
        lo[i] = *reinterpret_cast<const float4*>(x + 8 * c);
        hi[i] = *reinterpret_cast<const float4*>(x + 8 * c + 4);
    }
}

/// Requests this lane's chunks of a row of `cols` fp16 weights into slots [first, first + kRowCpl).
__device__ __forceinline__ half8 RowChunk(const uint16_t* row, uint32_t cols, int i)
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t c = min(lane + i * kWave, cols / 8 - 1);
    return __builtin_nontemporal_load(reinterpret_cast<const half8*>(row) + c);
}

/// Dot of this lane's chunks of a row with its activation chunks (chunks past the row add 0).
__device__ __forceinline__ float RowDot(const half8* w, const float4 (&lo)[kRowCpl], const float4 (&hi)[kRowCpl],
                                        uint32_t cols)
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kRowCpl; ++i)
    {
        const float part = DotChunk(w[i], lo[i], hi[i], 0.0f);
        acc += lane + i * kWave < cols / 8 ? part : 0.0f;
    }
    return acc;
}

struct Roles
{
    bool q, a, o, r;
    uint32_t qb;           // QKV block
    uint32_t g, c, h;      // attention: kv head, chunk, query head within the group
    uint32_t ob;           // o_proj / reduction row block
    uint32_t rb;
};

__device__ __forceinline__ Roles RolesOf(const StepPlan& p, uint32_t b)
{
    Roles r{};
    r.q = b >= p.roleQ && b < p.roleQ + p.qkvBlocks;
    r.qb = b - p.roleQ;
    const uint32_t group = p.heads / p.kvHeads;
    if (b >= p.roleA)
    {
        const uint32_t rel = b - p.roleA;
        const uint32_t pair = rel % 8 + 8 * ((rel / 8) / group);
        r.h = (rel / 8) % group;
        r.a = pair < p.kvHeads * p.chunks;
        r.g = pair / p.chunks;
        r.c = pair % p.chunks;
    }
    r.o = b >= p.roleO && b < p.roleO + p.rowBlocks;
    r.ob = b - p.roleO;
    r.r = b >= p.roleR && b < p.roleR + p.rowBlocks;
    r.rb = b - p.roleR;
    return r;
}

/// Rows (r0, r1) of QKV unit u of block qb, and the rope index j (or -1 for a value pair).
__device__ __forceinline__ void QkvUnitRows(const StepPlan& p, uint32_t qb, uint32_t u, uint32_t& r0, uint32_t& r1,
                                            int32_t& j)
{
    const uint32_t hd = p.headDim;
    const uint32_t perHead = hd / 32;
    const uint32_t ropeBlocks = (p.heads + p.kvHeads) * perHead;
    if (qb < ropeBlocks)
    {
        const uint32_t head = qb / perHead;
        j = static_cast<int32_t>((qb % perHead) * 16 + u);
        r0 = head * hd + static_cast<uint32_t>(j);
        r1 = r0 + hd / 2;
    }
    else
    {
        r0 = (p.heads + p.kvHeads) * hd + (qb - ropeBlocks) * 32 + 2 * u;
        r1 = r0 + 1;
        j = -1;
    }
}

/// Hand-off slot of q|k|v row r: per kv head g, the q rows of its query heads, then its k rows,
/// then its v rows, so an attention unit waits on one contiguous block.
__device__ __forceinline__ uint32_t QkvPacket(const StepPlan& p, uint32_t r, uint32_t group, uint32_t hd)
{
    const uint32_t qdim = p.heads * hd;
    const uint32_t kvdim = p.kvHeads * hd;
    const uint32_t block = (group + 2) * hd;
    if (r < qdim)
    {
        const uint32_t h = r / hd;
        return (h / group) * block + (h % group) * hd + r % hd;
    }
    if (r < qdim + kvdim)
    {
        return ((r - qdim) / hd) * block + group * hd + r % hd;
    }
    return ((r - qdim - kvdim) / hd) * block + (group + 1) * hd + r % hd;
}

template <int kHd>
struct AttnShape
{
    static constexpr int kLpk = kHd / 8;                              // lanes per key (16 bytes each)
    static constexpr uint32_t kKeysPerRound = (kComputeWaves * kWave) / kLpk;  // keys per round (= block)
};

/// The cache rows of round r of this attention unit (slot = compute thread / lanes per key).
template <int kHd>
__device__ __forceinline__ uint32_t AttnKey(const StepPlan& p, const Roles& ro, uint32_t r, uint32_t slot)
{
    return (ro.c + r * p.chunks) * AttnShape<kHd>::kKeysPerRound + slot;
}

/// Per-lane byte offsets of the chunks a compute lane requests, fixed for the whole step: its two
/// chunks of a hidden-wide row and of a q-dim-wide row (clamped into the row), its transposed-down
/// chunk, and its 16-byte slice of an attention key's row.
struct LaneOffsets
{
    uint32_t rowH[kRowCpl];
    uint32_t rowQ[kRowCpl];
    uint32_t down;
    uint32_t attn;
};

template <int kHd>
__device__ __forceinline__ LaneOffsets MakeLaneOffsets(const StepPlan& p, uint32_t cw, uint32_t ct)
{
    const uint32_t lane = threadIdx.x & (kWave - 1);
    LaneOffsets o;
#pragma unroll
    for (int i = 0; i < kRowCpl; ++i)
    {
        o.rowH[i] = 16 * min(lane + i * kWave, p.hidden / 8 - 1);
        o.rowQ[i] = 16 * min(lane + i * kWave, p.heads * kHd / 8 - 1);
    }
    // Down: output chunk c = cw * perWave + lane % 16 of row k = lane / 16 (+ 4i, in the base).
    const uint32_t perWave = (p.hidden / 8 + kComputeWaves - 1) / kComputeWaves;
    const uint32_t c = min(cw * perWave + min(lane % 16, perWave - 1), p.hidden / 8 - 1);
    o.down = (lane / 16) * p.hidden * 2 + 16 * c;
    // Attention: key slot ct / (lanes per key) of a round, 16-byte part ct % (lanes per key).
    using S = AttnShape<kHd>;
    o.attn = (ct / S::kLpk) * kHd * 2 + 16 * (ct % S::kLpk);
    return o;
}

/// The 16-byte weight chunks a compute lane requests ahead: slot k is base[k] + off[k], with
/// base[k] the same for the whole wave. Every slot always holds a valid address (unused slots
/// repeat slot 0, a cache hit), and the loads are issued from one place whatever the role:
/// different code paths filling the same registers with loads of their own cost the compiler a
/// second set of registers.
struct Slots
{
    const char* base[kPre];
    uint32_t off[kPre];
};

/// This workgroup's role weights for a layer (QKV units, the attention unit's K/V rows, o_proj
/// rows); false when it has no role.
template <int kHd>
__device__ __forceinline__ bool RoleSlots(const StepPlan& p, const Roles& ro, const StepLayer& ly,
                                          const LaneOffsets& lo, uint32_t cw, Slots& s)
{
    if (ro.q)
    {
        // Units cw, cw + 7 and cw + 14 of the block's 16 (slots 4t .. 4t + 3: r0's chunks, r1's).
#pragma unroll
        for (int t = 0; t < kQkvPerWave; ++t)
        {
            const uint32_t u = min(cw + kComputeWaves * t, 15u);
            uint32_t r0, r1;
            int32_t j;
            QkvUnitRows(p, ro.qb, u, r0, r1, j);
#pragma unroll
            for (int i = 0; i < kRowCpl; ++i)
            {
                s.base[4 * t + i] = reinterpret_cast<const char*>(ly.qkv + static_cast<uint64_t>(r0) * p.hidden);
                s.base[4 * t + 2 + i] = reinterpret_cast<const char*>(ly.qkv + static_cast<uint64_t>(r1) * p.hidden);
                s.off[4 * t + i] = lo.rowH[i];
                s.off[4 * t + 2 + i] = lo.rowH[i];
            }
        }
#pragma unroll
        for (int k = 4 * kQkvPerWave; k < kPre; ++k)
        {
            s.base[k] = s.base[0];
            s.off[k] = s.off[0];
        }
        return true;
    }
    if (ro.a)
    {
        // Rounds r < kAttnPre: K at slot 2r, V at 2r + 1. A round's block of keys starts at
        // (c + r * chunks) * keysPerRound; rows past the position are read (the cache and the
        // arena run on past maxSeq by a block) and masked.
        using S = AttnShape<kHd>;
        const uint64_t head = static_cast<uint64_t>(ro.g) * p.maxSeq * kHd * 2;
#pragma unroll
        for (int r = 0; r < kAttnPre; ++r)
        {
            const uint32_t first = min((ro.c + r * p.chunks) * S::kKeysPerRound, p.maxSeq - 1);
            const uint64_t at = head + static_cast<uint64_t>(first) * kHd * 2;
            s.base[2 * r] = reinterpret_cast<const char*>(ly.kcache) + at;
            s.base[2 * r + 1] = reinterpret_cast<const char*>(ly.vcache) + at;
            s.off[2 * r] = lo.attn;
            s.off[2 * r + 1] = lo.attn;
        }
#pragma unroll
        for (int k = 2 * kAttnPre; k < kPre; ++k)
        {
            s.base[k] = s.base[0];
            s.off[k] = s.off[0];
        }
        return true;
    }
    if (ro.o)
    {
        // Rows cw, cw + 7 and cw + 14 of the block's 16 (slots 2t, 2t + 1).
        const uint32_t qdim = p.heads * kHd;
#pragma unroll
        for (int t = 0; t < kQkvPerWave; ++t)
        {
            const uint32_t row = ro.ob * 16 + min(cw + kComputeWaves * t, 15u);
#pragma unroll
            for (int i = 0; i < kRowCpl; ++i)
            {
                s.base[2 * t + i] = reinterpret_cast<const char*>(ly.wo + static_cast<uint64_t>(row) * qdim);
                s.off[2 * t + i] = lo.rowQ[i];
            }
        }
#pragma unroll
        for (int k = 2 * kQkvPerWave; k < kPre; ++k)
        {
            s.base[k] = s.base[0];
            s.off[k] = s.off[0];
        }
        return true;
    }
    return false;
}

/// This workgroup's FFN share: gate/up units cw + 7t (slots 4t .. 4t + 3: gate's chunks, up's)
/// and the lane's transposed-down rows lane / 16 + 4i (slots 12 + i).
__device__ __forceinline__ void FfnSlots(const StepPlan& p, const StepLayer& ly, const LaneOffsets& lo, uint32_t b,
                                         uint32_t cw, Slots& s)
{
    const uint32_t share = p.ffnPerGroup;
    const uint32_t first = b * share;
#pragma unroll
    for (int t = 0; t < kGuPerWave; ++t)
    {
        const uint32_t k = cw + kComputeWaves * t;
        const uint64_t row = min(first + min(k, share - 1), p.ffn - 1);
#pragma unroll
        for (int i = 0; i < kRowCpl; ++i)
        {
            s.base[4 * t + i] = reinterpret_cast<const char*>(ly.gate + row * p.hidden);
            s.base[4 * t + 2 + i] = reinterpret_cast<const char*>(ly.up + row * p.hidden);
            s.off[4 * t + i] = lo.rowH[i];
            s.off[4 * t + 2 + i] = lo.rowH[i];
        }
    }
    // The lane offset adds up to three rows to a base row; the transposed tensor carries three
    // rows of slack, and rows past the share are read but never used.
#pragma unroll
    for (int i = 0; i < kDownPerLane; ++i)
    {
        const uint32_t row = min(first + 4 * i, p.ffn - 1);
        s.base[2 * kGuPerWave * kRowCpl + i] = reinterpret_cast<const char*>(ly.downT + static_cast<uint64_t>(row) * p.hidden);
        s.off[2 * kGuPerWave * kRowCpl + i] = lo.down;
    }
}

__device__ __forceinline__ void Issue(const Slots& s, half8 (&pre)[kPre])
{
#pragma unroll
    for (int k = 0; k < kPre; ++k)
    {
        pre[k] = *reinterpret_cast<const half8*>(s.base[k] + s.off[k]);
    }
}

/// Values every wave of a step workgroup derives the same way.
struct StepContext
{
    uint32_t b;       // workgroup
    uint32_t lane;
    Roles ro;
    uint32_t group;   // query heads per kv head
    uint32_t qdim;
    uint32_t step;    // steps begun in this run
    int32_t pos;      // cache row of this step
    uint32_t epoch0;  // epoch of this step's first hand-off
};

/// Wave 0: every wait of the step, each ending at the barrier that hands its data to the compute
/// waves. The barrier sequence (1 + 6 per layer + 1) is the compute program's; the two programs
/// are separate loops so that neither's registers are live across the other's code.
template <int kHd>
__device__ __forceinline__ void PollerProgram(const StepPlan& p, StepShared& sh, const StepContext& cx)
{
    const uint32_t lane = cx.lane;
    const Roles& ro = cx.ro;
    const uint32_t group = cx.group;
    const uint32_t epoch0 = cx.epoch0;
    bool live = !Abandoned(p.control);
    float normW[kMaxRow / kWave];

    // ---- start: the token (the sampler's, or the argmax of the last step's LM-head partials),
    // its embedding row as the layer-0 input, attn_norm[0].
    {
        LoadNormWeights(sh.layers[0].attnNorm, p.hidden, normW);
        int32_t token;
        if (p.sampled != nullptr)
        {
            token = *p.sampled;
        }
        else
        {
            float v = -INFINITY;
            int32_t idx = 0x7FFFFFFF;
            for (uint32_t k = lane; k < p.grid; k += kWave)
            {
                const float cv = p.argValue[k];
                const int32_t ci = p.argIndex[k];
                if (cv > v || (cv == v && ci < idx))
                {
                    v = cv;
                    idx = ci;
                }
            }
            GroupArgMax<kWave>(v, idx);
            token = idx == 0x7FFFFFFF ? 0 : idx;  // no finite logit at all: the host scan returns 0
        }
        const bool ok = token >= 0 && static_cast<uint32_t>(token) < p.vocab;
        const uint16_t* row = p.embedding + static_cast<uint64_t>(ok ? token : 0) * p.hidden;
        for (uint32_t i = lane; i < p.hidden; i += kWave)
        {
            sh.x[i] = ok ? HalfBitsToFloat(row[i]) : 0.0f;
        }
        if (lane == 0)
        {
            sh.token = token;
        }
        PollerNorm(sh.x, normW, p.hidden, p.eps, sh.xn);
    }
    __syncthreads();

    for (uint32_t l = 0; l < p.layers; ++l)
    {
        const StepLayer& ly = sh.layers[l];
        uint64_t* region = p.packets + static_cast<uint64_t>(l & 1) * p.parity;
        const uint32_t eQkv = epoch0 + 5 * l;
        const uint32_t ePart = eQkv + 1;
        const uint32_t eMid = eQkv + 2;
        const uint32_t eDown = eQkv + 3;
        const uint32_t eX = eQkv + 4;

        // ---- Q: an attention workgroup waits for its kv head's block of the hand-off: the q of
        // every query head of the group, then k and v (QkvPacket's layout).
        if (ro.a)
        {
            const uint32_t block = (group + 2) * kHd;
            Gather<kAttBlock / kWave>(
                region + p.offQkv + ro.g * block, block, eQkv, [] {}, [&](uint32_t i, float v, bool) { sh.att[i] = v; },
                p.control, p.spinLimit, kWaitQkv, live);
        }
        __syncthreads();
        // ---- A1 (the compute waves' attention)
        __syncthreads();
        // ---- A2: an o_proj workgroup gathers every partial of the layer and each chunk's weight
        // in the merge.
        if (ro.o)
        {
            const uint32_t nPart = p.kvHeads * p.chunks * group * (kHd + 2);
            Gather<kMaxPart / kWave>(
                region + p.offPart, nPart, ePart, [] {}, [&](uint32_t i, float v, bool) { sh.part[i] = v; },
                p.control, p.spinLimit, kWaitPart, live);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            if (lane < p.heads)
            {
                const uint32_t h = lane;
                const uint32_t g = h / group;
                const uint32_t hh = h % group;
                float mc[kMaxChunks];
                float lc[kMaxChunks];
                float top = -INFINITY;
#pragma unroll
                for (uint32_t c = 0; c < kMaxChunks; ++c)
                {
                    const uint32_t slotBase = ((g * p.chunks + min(c, p.chunks - 1)) * group + hh) * (kHd + 2);
                    mc[c] = c < p.chunks ? sh.part[slotBase + kHd] : -INFINITY;
                    lc[c] = sh.part[slotBase + kHd + 1];
                    top = fmaxf(top, mc[c]);
                }
                float den = 0.0f;
#pragma unroll
                for (uint32_t c = 0; c < kMaxChunks; ++c)
                {
                    mc[c] = mc[c] == -INFINITY ? 0.0f : exp2f(mc[c] - top);
                    den = fmaf(mc[c], lc[c], den);
                }
                const float inv = den > 0.0f ? 1.0f / den : 0.0f;
                for (uint32_t c = 0; c < p.chunks; ++c)
                {
                    sh.mergeW[h * kMaxChunks + c] = mc[c] * inv;
                }
            }
        }
        __syncthreads();
        // ---- O: the o_proj output, normalised for gate/up.
        {
            LoadNormWeights(ly.ffnNorm, p.hidden, normW);
            Gather<kMaxHidden / kWave>(
                region + p.offMid, p.hidden, eMid, [] {}, [&](uint32_t i, float v, bool) { sh.mid[i] = v; },
                p.control, p.spinLimit, kWaitMid, live);
            PollerNorm(sh.mid, normW, p.hidden, p.eps, sh.midn);
        }
        __syncthreads();
        // ---- G1 (the compute waves' gate/up)
        __syncthreads();
        // ---- G2: the reduction rows sum every down partial and hand the layer output on; every
        // poller then waits for the whole of it.
        {
            if (ro.r)
            {
                // Row block rb of every workgroup's partial: [rb][workgroup][16] is contiguous, and
                // a lane's packets all belong to row lane % 16.
                float total = 0.0f;
                Gather<kMaxGrid * 16 / kWave>(
                    region + p.offDown + static_cast<uint64_t>(ro.rb) * p.grid * 16, p.grid * 16, eDown,
                    [&] { total = 0.0f; }, [&](uint32_t, float v, bool valid) { total += valid ? v : 0.0f; },
                    p.control, p.spinLimit, kWaitDown, live);
                total = XorSum<16>(total);  // lanes sharing lane % 16 hold the same row
                if (lane < 16)
                {
                    const uint32_t row = ro.rb * 16 + lane;
                    Put(region + p.offX + row, sh.mid[row] + total, eX);
                }
            }
            // The layer output feeds the next layer's QKV blocks (normalised) and o_proj rows
            // (the residual), and after the last layer every workgroup's LM-head share.
            const bool last = l + 1 == p.layers;
            if (last || ro.q || ro.o)
            {
                LoadNormWeights(last ? p.outputNorm : sh.layers[l + 1].attnNorm, p.hidden, normW);
                Gather<kMaxHidden / kWave>(
                    region + p.offX, p.hidden, eX, [] {}, [&](uint32_t i, float v, bool) { sh.x[i] = v; },
                    p.control, p.spinLimit, kWaitX, live);
                PollerNorm(sh.x, normW, p.hidden, p.eps, sh.xn);
            }
        }
        __syncthreads();
    }
    // ---- LM head (the compute waves')
    __syncthreads();
}

/// Waves 1..7: the step's arithmetic. Each phase's weights were requested before the barrier
/// that delivers its input.
template <int kHd>
__device__ __forceinline__ void ComputeProgram(const StepPlan& p, StepShared& sh, const StepContext& cx)
{
    const uint32_t b = cx.b;
    const uint32_t lane = cx.lane;
    const Roles& ro = cx.ro;
    const uint32_t group = cx.group;
    const uint32_t qdim = cx.qdim;
    const int32_t pos = cx.pos;
    const uint32_t epoch0 = cx.epoch0;
    const uint32_t cw = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) - 1;
    const uint32_t ct = threadIdx.x - kWave;
    half8 pre[kPre];
    const bool hasRole = ro.q || ro.a || ro.o;
    const LaneOffsets lanes = MakeLaneOffsets<kHd>(p, cw, ct);
    // A QKV block's epilogue operands, requested with its weights: lane t < 3 finishes unit
    // cw + 7t and holds that unit's two biases and rope power.
    const bool qLane = ro.q && lane < kQkvPerWave && cw + kComputeWaves * lane < 16;
    float qBias0 = 0.0f, qBias1 = 0.0f, qPow = 0.0f;
    auto prefetchQkvOperands = [&](const StepLayer& next) {
        if (qLane)
        {
            uint32_t r0, r1;
            int32_t j;
            QkvUnitRows(p, ro.qb, cw + kComputeWaves * lane, r0, r1, j);
            qBias0 = next.qkvBias[r0];
            qBias1 = next.qkvBias[r1];
            qPow = j >= 0 ? p.ropePow[j] : 0.0f;
        }
    };

    {
        Slots slots;
        if (!RoleSlots<kHd>(p, ro, sh.layers[0], lanes, cw, slots))
        {
            FfnSlots(p, sh.layers[0], lanes, b, cw, slots);
        }
        Issue(slots, pre);
        prefetchQkvOperands(sh.layers[0]);
    }
    __syncthreads();

    for (uint32_t l = 0; l < p.layers; ++l)
    {
        const StepLayer& ly = sh.layers[l];
        uint64_t* region = p.packets + static_cast<uint64_t>(l & 1) * p.parity;
        const uint32_t eQkv = epoch0 + 5 * l;
        const uint32_t ePart = eQkv + 1;
        const uint32_t eMid = eQkv + 2;
        const uint32_t eDown = eQkv + 3;

        // ---- Q: the QKV blocks.
        if (ro.q)
        {
            float4 lo[kRowCpl], hi[kRowCpl];
            RowActivation(sh.xn, p.hidden, lo, hi);
            float s[2 * kQkvPerWave];
#pragma unroll
            for (int t = 0; t < kQkvPerWave; ++t)
            {
                s[2 * t] = RowDot(&pre[4 * t], lo, hi, p.hidden);
                s[2 * t + 1] = RowDot(&pre[4 * t + 2], lo, hi, p.hidden);
            }
            GroupSumN<kWave>(s);
            if (qLane)
            {
                // Lane t finishes unit cw + 7t: bias, rope, hand-off, cache row.
                const uint32_t t = lane;
                uint32_t r0, r1;
                int32_t j;
                QkvUnitRows(p, ro.qb, cw + kComputeWaves * t, r0, r1, j);
                const float s0 = (t == 0 ? s[0] : t == 1 ? s[2] : s[4]) + qBias0;
                const float s1 = (t == 0 ? s[1] : t == 1 ? s[3] : s[5]) + qBias1;
                uint64_t* out = region + p.offQkv;
                const bool inCache = pos >= 0 && static_cast<uint32_t>(pos) < p.maxSeq;
                if (j >= 0)
                {
                    // rope_neox (rope_funcs.glsl:76-114): theta = pos * theta_scale^j, pair (j, j + hd/2).
                    const float theta = static_cast<float>(pos) * qPow;
                    const float cs = cosf(theta);
                    const float sn = sinf(theta);
                    float o0 = s0 * cs - s1 * sn;
                    float o1 = s0 * sn + s1 * cs;
                    if (r0 >= qdim)
                    {
                        // A k row: the cache holds it as fp16, and attention uses those values.
                        const uint32_t g = (r0 - qdim) / kHd;
                        const uint16_t h0 = FloatToHalfBits(o0);
                        const uint16_t h1 = FloatToHalfBits(o1);
                        if (inCache)
                        {
                            uint16_t* krow = ly.kcache + (static_cast<uint64_t>(g) * p.maxSeq + pos) * kHd;
                            krow[j] = h0;
                            krow[j + kHd / 2] = h1;
                        }
                        o0 = HalfBitsToFloat(h0);
                        o1 = HalfBitsToFloat(h1);
                    }
                    Put(out + QkvPacket(p, r0, group, kHd), o0, eQkv);
                    Put(out + QkvPacket(p, r1, group, kHd), o1, eQkv);
                }
                else
                {
                    const uint32_t channel = r0 - qdim - p.kvHeads * kHd;
                    const uint32_t g = channel / kHd;
                    const uint16_t h0 = FloatToHalfBits(s0);
                    const uint16_t h1 = FloatToHalfBits(s1);
                    if (inCache)
                    {
                        uint16_t* vrow = ly.vcache + (static_cast<uint64_t>(g) * p.maxSeq + pos) * kHd + channel % kHd;
                        vrow[0] = h0;
                        vrow[1] = h1;
                    }
                    Put(out + QkvPacket(p, r0, group, kHd), HalfBitsToFloat(h0), eQkv);
                    Put(out + QkvPacket(p, r1, group, kHd), HalfBitsToFloat(h1), eQkv);
                }
            }
        }
        __syncthreads();

        // ---- A1: attention over this unit's keys, one key of each round per lane group.
        if (ro.a)
        {
            using S = AttnShape<kHd>;
            const uint32_t slot = ct / S::kLpk;
            const uint32_t part = ct % S::kLpk;
            const float* qh = sh.att + ro.h * kHd + 8 * part;  // this head's q slice
            const float4 q0 = *reinterpret_cast<const float4*>(qh);
            const float4 q1 = *reinterpret_cast<const float4*>(qh + 4);
            const float sl = p.attnScale * kLog2e;
            const uint32_t keys = static_cast<uint32_t>(pos) + 1;
            const uint32_t blocks = (keys + S::kKeysPerRound - 1) / S::kKeysPerRound;
            const uint32_t rounds = blocks > ro.c ? (blocks - 1 - ro.c) / p.chunks + 1 : 0;
            // The row at the position was written this step: its fp16 values come from the
            // hand-off, patched into the registers of the round and lane group that hold it.
            const uint32_t posBlock = static_cast<uint32_t>(pos) / S::kKeysPerRound;
            const bool ownsPos = posBlock % p.chunks == ro.c && slot == static_cast<uint32_t>(pos) % S::kKeysPerRound;
            const uint32_t posRound = posBlock / p.chunks;
            half8 kNew, vNew;
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                kNew[e] = static_cast<_Float16>(sh.att[group * kHd + 8 * part + e]);
                vNew[e] = static_cast<_Float16>(sh.att[(group + 1) * kHd + 8 * part + e]);
            }
#pragma unroll
            for (int r = 0; r < kAttnPre; ++r)
            {
                if (ownsPos && posRound == static_cast<uint32_t>(r))
                {
                    pre[2 * r] = kNew;
                    pre[2 * r + 1] = vNew;
                }
            }
            float m = -INFINITY;
            float lsum = 0.0f;
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            auto consume = [&](uint32_t key, const half8& kh, const half8& vh) {
                float sc = static_cast<float>(kh[0]) * q0.x;
                sc = fmaf(static_cast<float>(kh[1]), q0.y, sc);
                sc = fmaf(static_cast<float>(kh[2]), q0.z, sc);
                sc = fmaf(static_cast<float>(kh[3]), q0.w, sc);
                sc = fmaf(static_cast<float>(kh[4]), q1.x, sc);
                sc = fmaf(static_cast<float>(kh[5]), q1.y, sc);
                sc = fmaf(static_cast<float>(kh[6]), q1.z, sc);
                sc = fmaf(static_cast<float>(kh[7]), q1.w, sc);
                sc = GroupSum<S::kLpk>(sc);
                if (key < keys)
                {
                    sc *= sl;
                    const float top = fmaxf(m, sc);
                    const float f = exp2f(m - top);  // 0 while m is -inf
                    const float e = exp2f(sc - top);
                    lsum = fmaf(lsum, f, e);
#pragma unroll
                    for (int d = 0; d < 8; ++d)
                    {
                        acc[d] = fmaf(e, static_cast<float>(vh[d]), acc[d] * f);
                    }
                    m = top;
                }
            };
#pragma unroll
            for (int r = 0; r < kAttnPre; ++r)
            {
                if (static_cast<uint32_t>(r) < rounds)
                {
                    consume(AttnKey<kHd>(p, ro, r, slot), pre[2 * r], pre[2 * r + 1]);
                }
            }
            // Caches longer than the rounds held in registers.
            const uint64_t base = static_cast<uint64_t>(ro.g) * p.maxSeq * kHd + 8 * part;
            for (uint32_t r = kAttnPre; r < rounds; ++r)
            {
                const uint32_t key = AttnKey<kHd>(p, ro, r, slot);
                const uint32_t row = min(key, min(static_cast<uint32_t>(pos), p.maxSeq - 1));
                const bool fresh = key == static_cast<uint32_t>(pos);
                const half8 kh = fresh ? kNew : *reinterpret_cast<const half8*>(ly.kcache + base + static_cast<uint64_t>(row) * kHd);
                const half8 vh = fresh ? vNew : *reinterpret_cast<const half8*>(ly.vcache + base + static_cast<uint64_t>(row) * kHd);
                consume(key, kh, vh);
            }
            // Combine the key slots of this wave (lanes with the same `part`).
            constexpr int kFrom = S::kLpk;
            const float top = XorMax<kFrom>(m);
            const float f = m == -INFINITY ? 0.0f : exp2f(m - top);
            const float lw = XorSum<kFrom>(lsum * f);
#pragma unroll
            for (int d = 0; d < 8; ++d)
            {
                acc[d] = XorSum<kFrom>(acc[d] * f);
            }
            if (lane < static_cast<uint32_t>(S::kLpk))
            {
#pragma unroll
                for (int d = 0; d < 8; ++d)
                {
                    sh.waveAttn[cw][8 * part + d] = acc[d];
                }
                if (lane == 0)
                {
                    sh.waveAttn[cw][kHd] = top;
                    sh.waveAttn[cw][kHd + 1] = lw;
                }
            }
        }
        __syncthreads();

        // ---- A2: an attention unit combines its waves and hands the partial on.
        if (ro.a)
        {
            const uint32_t slotBase = ((ro.g * p.chunks + ro.c) * group + ro.h) * (kHd + 2);
            float top = -INFINITY;
#pragma unroll
            for (int w = 0; w < kComputeWaves; ++w)
            {
                top = fmaxf(top, sh.waveAttn[w][kHd]);
            }
            if (ct <= static_cast<uint32_t>(kHd) + 1)
            {
                float value;
                if (ct == static_cast<uint32_t>(kHd))
                {
                    value = top;
                }
                else
                {
                    const uint32_t col = ct < static_cast<uint32_t>(kHd) ? ct : kHd + 1;
                    value = 0.0f;
#pragma unroll
                    for (int w = 0; w < kComputeWaves; ++w)
                    {
                        const float mw = sh.waveAttn[w][kHd];
                        const float f = mw == -INFINITY ? 0.0f : exp2f(mw - top);
                        value = fmaf(f, sh.waveAttn[w][col], value);
                    }
                }
                Put(region + p.offPart + slotBase + ct, value, ePart);
            }
        }
        __syncthreads();

        // ---- O: o_proj rows with the merge in the prologue, plus the residual.
        if (ro.o)
        {
            // This lane's attention outputs (its two chunks of the q dim), merged.
            float4 lo[kRowCpl], hi[kRowCpl];
#pragma unroll
            for (int i = 0; i < kRowCpl; ++i)
            {
                const uint32_t chunk = min(lane + i * kWave, qdim / 8 - 1);
                const uint32_t h = 8 * chunk / kHd;
                const uint32_t g = h / group;
                const uint32_t hh = h % group;
                const uint32_t d0 = 8 * chunk % kHd;
                float out[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                for (uint32_t c = 0; c < p.chunks; ++c)
                {
                    const float w = sh.mergeW[h * kMaxChunks + c];
                    const float* acc = sh.part + ((g * p.chunks + c) * group + hh) * (kHd + 2) + d0;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                    {
                        out[e] = fmaf(w, acc[e], out[e]);
                    }
                }
                lo[i] = make_float4(out[0], out[1], out[2], out[3]);
                hi[i] = make_float4(out[4], out[5], out[6], out[7]);
            }
            float s[kQkvPerWave];
#pragma unroll
            for (int t = 0; t < kQkvPerWave; ++t)
            {
                s[t] = RowDot(&pre[2 * t], lo, hi, qdim);
            }
            GroupSumN<kWave>(s);
            if (lane < kQkvPerWave && cw + kComputeWaves * lane < 16)
            {
                const uint32_t row = ro.ob * 16 + cw + kComputeWaves * lane;
                Put(region + p.offMid + row, sh.x[row] + (lane == 0 ? s[0] : lane == 1 ? s[1] : s[2]), eMid);
            }
        }
        if (hasRole)
        {
            // A role's weights are spent by now: request the FFN share.
            Slots slots;
            FfnSlots(p, ly, lanes, b, cw, slots);
            Issue(slots, pre);
        }
        __syncthreads();

        // ---- G1: this workgroup's gate/up rows and swiglu.
        {
            float4 lo[kRowCpl], hi[kRowCpl];
            RowActivation(sh.midn, p.hidden, lo, hi);
            float s[2 * kGuPerWave];
#pragma unroll
            for (int t = 0; t < kGuPerWave; ++t)
            {
                s[2 * t] = RowDot(&pre[4 * t], lo, hi, p.hidden);
                s[2 * t + 1] = RowDot(&pre[4 * t + 2], lo, hi, p.hidden);
            }
            GroupSumN<kWave>(s);
            if (lane == 0)
            {
#pragma unroll
                for (int t = 0; t < kGuPerWave; ++t)
                {
                    const uint32_t k = cw + kComputeWaves * t;
                    if (k < p.ffnPerGroup && b * p.ffnPerGroup + k < p.ffn)
                    {
                        const float g = s[2 * t];
                        sh.act[k] = g / (1.0f + expf(-g)) * s[2 * t + 1];  // swiglu.comp's op
                    }
                }
            }
        }
        __syncthreads();

        // ---- G2: the share's down columns as a partial of the whole output.
        {
            const uint32_t share = p.ffnPerGroup;
            const uint32_t perWave = (p.hidden / 8 + kComputeWaves - 1) / kComputeWaves;
            const uint32_t c16 = lane % 16;
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < kDownPerLane; ++i)
            {
                const uint32_t k = lane / 16 + 4 * i;
                if (4 * i < static_cast<int>(share) && k < share && b * share + k < p.ffn)
                {
                    const float a = sh.act[k];
                    const half8 w = pre[2 * kGuPerWave * kRowCpl + i];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                    {
                        acc[e] = fmaf(a, static_cast<float>(w[e]), acc[e]);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                acc[e] = XorSum<16>(acc[e]);
            }
            // Lanes 0..15 hold this wave's chunks; lay them out row-contiguous so each store
            // instruction writes whole lines.
            if (lane < 16 && c16 < perWave)
            {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                {
                    sh.downOut[cw][8 * c16 + e] = acc[e];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            // Row r of this workgroup's partial goes to [r / 16][b][r % 16]: each 16-row line has
            // this workgroup as its only writer, and a reduction reads one contiguous run.
            const uint32_t first = cw * perWave * 8;
            uint64_t* out = region + p.offDown + static_cast<uint64_t>(b) * 16;
#pragma unroll
            for (int t = 0; t < 2; ++t)
            {
                const uint32_t e = lane + kWave * t;
                const uint32_t row = first + e;
                if (e < perWave * 8 && row < p.hidden)
                {
                    Put(out + static_cast<uint64_t>(row / 16) * p.grid * 16 + row % 16, sh.downOut[cw][e], eDown);
                }
            }
            if (l + 1 < p.layers)
            {
                Slots slots;
                if (!RoleSlots<kHd>(p, ro, sh.layers[l + 1], lanes, cw, slots))
                {
                    FfnSlots(p, sh.layers[l + 1], lanes, b, cw, slots);
                }
                Issue(slots, pre);
                prefetchQkvOperands(sh.layers[l + 1]);
            }
        }
        __syncthreads();
    }

    // ---- LM head: a contiguous share of the vocabulary per workgroup, 16 lanes per row.
    {
        const uint32_t share = (p.vocab + p.grid - 1) / p.grid;
        const uint32_t first = b * share;
        const uint32_t end = min(first + share, p.vocab);
        const uint32_t nchunks = p.hidden / 8;
        const uint32_t lir = lane % kLmLpr;
        const uint32_t seg = lane / kLmLpr;
        float4 xlo[kLmCpl], xhi[kLmCpl];
#pragma unroll
        for (int i = 0; i < kLmCpl; ++i)
        {
            const uint32_t c = min(lir + i * kLmLpr, nchunks - 1);
            xlo[i] = *reinterpret_cast<const float4*>(sh.xn + 8 * c);
            xhi[i] = *reinterpret_cast<const float4*>(sh.xn + 8 * c + 4);
        }
        constexpr uint32_t kRowsPerRound = kComputeWaves * (kWave / kLmLpr);
        float bestValue = -INFINITY;
        int32_t bestIndex = 0x7FFFFFFF;
        half8 wa[kLmCpl], wb[kLmCpl];
        auto load = [&](uint32_t row, half8(&w)[kLmCpl]) {
            const half8* chunks = reinterpret_cast<const half8*>(p.head + static_cast<uint64_t>(min(row, p.vocab - 1)) * p.hidden);
#pragma unroll
            for (int i = 0; i < kLmCpl; ++i)
            {
                w[i] = __builtin_nontemporal_load(chunks + min(lir + i * kLmLpr, nchunks - 1));
            }
        };
        auto finish = [&](uint32_t row, const half8(&w)[kLmCpl]) {
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < kLmCpl; ++i)
            {
                const float part = DotChunk(w[i], xlo[i], xhi[i], 0.0f);
                a[i & 3] += lir + i * kLmLpr < nchunks ? part : 0.0f;
            }
            const float sum = GroupSum<kLmLpr>((a[0] + a[1]) + (a[2] + a[3]));
            if (row < end && lir == 0)
            {
                p.logits[row] = sum;
                // Rows reach a lane in increasing order, so '>' keeps the lowest index on ties.
                if (sum > bestValue)
                {
                    bestValue = sum;
                    bestIndex = static_cast<int32_t>(row);
                }
            }
        };
        uint32_t row = first + cw * (kWave / kLmLpr) + seg;
        if (row < end)
        {
            load(row, wa);
        }
        for (; row < end; row += 2 * kRowsPerRound)
        {
            const uint32_t next = row + kRowsPerRound;
            if (next < end)
            {
                load(next, wb);
            }
            finish(row, wa);
            if (next >= end)
            {
                break;
            }
            if (next + kRowsPerRound < end)
            {
                load(next + kRowsPerRound, wa);
            }
            finish(next, wb);
        }
        GroupArgMax<kWave>(bestValue, bestIndex);
        if (lane == 0)
        {
            sh.bestValue[cw] = bestValue;
            sh.bestIndex[cw] = bestIndex;
        }
    }
    __syncthreads();
}

template <int kHd>
__global__ __launch_bounds__(kStepThreads) void StepKernel(const StepPlan p)
{
    __shared__ StepShared sh;
    StepContext cx;
    cx.b = blockIdx.x;
    cx.lane = threadIdx.x % kWave;
    cx.ro = RolesOf(p, cx.b);
    cx.group = p.heads / p.kvHeads;
    cx.qdim = p.heads * kHd;
    cx.step = p.state->step;
    cx.pos = p.state->start + static_cast<int32_t>(cx.step);
    cx.epoch0 = p.control[kStepEpoch];
    const uint32_t b = cx.b;
    const uint32_t step = cx.step;
    const int32_t pos = cx.pos;
    const uint32_t epoch0 = cx.epoch0;
    // The layer table to LDS once (pointer words), so no layer's first use waits on memory.
    {
        constexpr uint32_t kWords = sizeof(StepLayer) / sizeof(uint32_t);
        const uint32_t* from = reinterpret_cast<const uint32_t*>(p.layer);
        uint32_t* to = reinterpret_cast<uint32_t*>(sh.layers);
        for (uint32_t i = threadIdx.x; i < p.layers * kWords; i += kStepThreads)
        {
            to[i] = from[i];
        }
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) == 0)
    {
        PollerProgram<kHd>(p, sh, cx);
    }
    else
    {
        ComputeProgram<kHd>(p, sh, cx);
    }
    if (threadIdx.x == 0)
    {
        float v = sh.bestValue[0];
        int32_t idx = sh.bestIndex[0];
        for (int w = 1; w < kComputeWaves; ++w)
        {
            if (sh.bestValue[w] > v || (sh.bestValue[w] == v && sh.bestIndex[w] < idx))
            {
                v = sh.bestValue[w];
                idx = sh.bestIndex[w];
            }
        }
        p.argValue[b] = v;
        p.argIndex[b] = idx;
        if (b == 0)
        {
            // Every workgroup read the state, the partials and the epoch before any could reach
            // the LM head (that needs every workgroup's last down partial), so they are replaced now.
            const int32_t token = sh.token;
            if (step > 0)
            {
                p.ids[(step - 1) % p.idsCap] = token;
            }
            p.state->token = token;
            p.state->position = pos;
            p.state->step = step + 1;
            if (pos >= 0 && static_cast<uint32_t>(pos) < p.historyCap)
            {
                p.history[pos] = token;
            }
            const uint32_t span = 5 * p.layers;
            const uint32_t next = epoch0 > 0xFFFFFFFFu - 2 * span ? 1u : epoch0 + span;
            p.control[kStepEpoch] = next;
        }
    }
}


__global__ __launch_bounds__(256) void Transpose16Kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                        uint32_t rows, uint32_t cols)
{
    __shared__ uint16_t tile[32][33];
    const uint32_t c0 = blockIdx.x * 32;
    const uint32_t r0 = blockIdx.y * 32;
    const uint32_t tx = threadIdx.x % 32;
    const uint32_t ty = threadIdx.x / 32;
    for (uint32_t y = ty; y < 32; y += 8)
    {
        const uint32_t r = r0 + y;
        const uint32_t c = c0 + tx;
        if (r < rows && c < cols)
        {
            tile[y][tx] = src[static_cast<uint64_t>(r) * cols + c];
        }
    }
    __syncthreads();
    for (uint32_t y = ty; y < 32; y += 8)
    {
        const uint32_t c = c0 + y;
        const uint32_t r = r0 + tx;
        if (r < rows && c < cols)
        {
            dst[static_cast<uint64_t>(c) * rows + r] = tile[tx][y];
        }
    }
}

uint32_t Round8(uint32_t v) { return (v + 7) / 8 * 8; }
uint32_t Round16(uint32_t v) { return (v + 15) / 16 * 16; }

uint32_t ChunksFor(uint32_t heads, uint32_t headDim)
{
    const uint32_t fit = kMaxPart / (heads * (headDim + 2));
    return std::min(kMaxChunks, fit);
}
}  // namespace

const char* StepUnsupported(uint32_t hidden, uint32_t ffn, uint32_t heads, uint32_t kvHeads, uint32_t headDim,
                            uint32_t grid)
{
    const uint32_t qdim = heads * headDim;
    if (headDim != 64 && headDim != 128)
    {
        return "head_dim must be 64 or 128";
    }
    if (kvHeads == 0 || heads % kvHeads != 0 || heads / kvHeads > 8)
    {
        return "heads must be a multiple of kv_heads with a group of at most 8";
    }
    if (hidden % 16 != 0 || hidden > kMaxHidden || qdim > kMaxRow || qdim % 16 != 0)
    {
        return "hidden must be a multiple of 16 up to 896, heads * head_dim one up to 1024";
    }
    if (heads > 16 || ChunksFor(heads, headDim) == 0)
    {
        return "too many heads for the merge in o_proj's prologue";
    }
    if (grid == 0 || grid > kMaxGrid || (ffn + grid - 1) / grid > kMaxFfnShare || ffn % 8 != 0)
    {
        return "the FFN share per workgroup exceeds 21 rows";
    }
    StepPlan probe{};
    probe.hidden = hidden;
    probe.ffn = ffn;
    probe.heads = heads;
    probe.kvHeads = kvHeads;
    probe.headDim = headDim;
    (void)StepPlanLayout(probe, grid);
    if (probe.roleR + probe.rowBlocks > grid)
    {
        return "the roles need more workgroups than CUs";
    }
    return nullptr;
}

size_t StepPlanLayout(StepPlan& p, uint32_t grid)
{
    p.grid = grid;
    p.chunks = ChunksFor(p.heads, p.headDim);
    const uint32_t group = p.heads / p.kvHeads;
    const uint32_t qkvRows = (p.heads + 2 * p.kvHeads) * p.headDim;
    p.qkvBlocks = qkvRows / 32;
    const uint32_t pairs = p.kvHeads * p.chunks;
    p.attnUnits = pairs * group;
    p.rowBlocks = p.hidden / 16;
    p.ffnPerGroup = (p.ffn + grid - 1) / grid;
    p.roleQ = 0;
    p.roleA = Round8(p.qkvBlocks);
    p.roleO = p.roleA + (pairs + 7) / 8 * group * 8;
    p.roleR = p.roleO + Round8(p.rowBlocks);
    uint32_t at = 0;
    p.offX = at;
    at += Round16(p.hidden);
    p.offQkv = at;
    at += Round16(qkvRows);
    p.offPart = at;
    at += Round16(p.attnUnits * (p.headDim + 2));
    p.offMid = at;
    at += Round16(p.hidden);
    p.offDown = at;
    at += p.rowBlocks * grid * 16;
    p.parity = at;
    return 2 * static_cast<size_t>(at) + kSlack;
}

uint32_t StepResidentPerCu()
{
    int perCu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, StepKernel<64>, kStepThreads, 0) != hipSuccess)
    {
        return 0;
    }
    int perCu128 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu128, StepKernel<128>, kStepThreads, 0) != hipSuccess)
    {
        return 0;
    }
    return static_cast<uint32_t>(std::min(perCu, perCu128));
}

hipError_t LaunchStep(hipStream_t s, const StepPlan& plan)
{
    void* args[] = {const_cast<StepPlan*>(&plan)};
    const void* kernel = plan.headDim == 64 ? reinterpret_cast<const void*>(&StepKernel<64>)
                                            : reinterpret_cast<const void*>(&StepKernel<128>);
    return hipLaunchCooperativeKernel(kernel, dim3(plan.grid), dim3(kStepThreads), args, 0, s);
}

hipError_t LaunchTranspose16(hipStream_t s, const uint16_t* src, uint16_t* dst, uint32_t rows, uint32_t cols)
{
    hipLaunchKernelGGL(Transpose16Kernel, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, s, src, dst, rows,
                       cols);
    return hipGetLastError();
}
}  // namespace muyo
