// The decode-step executor behind the muyo_decoder_* C ABI.
//
// It plays the role of RunFullModel's render graph (src/FullModel.cpp:685-998) plus its
// feedToken/sampleNext loop (:1096-1117): one arena of device memory holds every weight, the
// fp16 KV cache and the activations; one step is 2 + 5 * layers launches on one stream
// (6 per layer for the shapes whose attention partials need their own merge kernel: q dim over
// 1024 with a kv group over 1024 channels or more than four kv heads; decode_kernels.hip).
// The first step runs eagerly; later steps replay a hipGraph captured once, because everything
// that changes per token (token id, position, step counter) lives in device memory: the first
// kernel of a step reduces the previous step's argmax partials into its token and advances the
// position. Greedy generation therefore needs no host round trip between tokens.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <utility>
#include <vector>

#include "common.hpp"
#include "decode_kernels.hpp"
#include "prefill.hpp"
#include "sampler.hpp"

using namespace muyo;

namespace
{
constexpr uint32_t kIdsCapacity = 4096;
constexpr size_t kAlign = 256;

size_t AlignUp(size_t value) { return (value + kAlign - 1) / kAlign * kAlign; }

struct TensorSlot
{
    size_t offset = 0;
    size_t bytes = 0;
};

enum LayerTensor
{
    kAttnNorm,
    kQkv,
    kQkvBias,
    kOut,
    kFfnNorm,
    kGate,
    kUp,
    kDown,
    kKCache,
    kVCache,
    kLayerTensorCount
};

LayerTensor ToLayerTensor(uint32_t kind)
{
    switch (kind)
    {
        case MUYO_TENSOR_ATTN_NORM:
            return kAttnNorm;
        case MUYO_TENSOR_ATTN_QKV:
            return kQkv;
        case MUYO_TENSOR_ATTN_QKV_B:
            return kQkvBias;
        case MUYO_TENSOR_ATTN_OUTPUT:
            return kOut;
        case MUYO_TENSOR_FFN_NORM:
            return kFfnNorm;
        case MUYO_TENSOR_FFN_GATE:
            return kGate;
        case MUYO_TENSOR_FFN_UP:
            return kUp;
        case MUYO_TENSOR_FFN_DOWN:
            return kDown;
        case MUYO_TENSOR_KCACHE:
            return kKCache;
        case MUYO_TENSOR_VCACHE:
            return kVCache;
        default:
            return kLayerTensorCount;
    }
}

}  // namespace

struct MuyoDecoder
{
    MuyoQwen2Config config{};
    DecodeDims dims{};
    int device = 0;
    hipStream_t stream = nullptr;

    char* arena = nullptr;
    size_t arenaBytes = 0;
    TensorSlot tokenEmbd, outputNorm, logits;
    TensorSlot output;  // the untied LM head (config.untiedOutput); empty when tied to tokenEmbd
    std::vector<TensorSlot> layers;  // layer * kLayerTensorCount + tensor

    float* xA = nullptr;
    float* xB = nullptr;
    float* xMid = nullptr;
    float* q = nullptr;
    float* attnOut = nullptr;
    float* xMid2 = nullptr;   // with o_proj split by kv group: odd layers' hidden state after attention
    float* act = nullptr;
    DecodeState* state = nullptr;
    int32_t* ids = nullptr;
    DecodeScratch scratch{};
    uint32_t argBlocks = 0;     // LM-head workgroups = argmax partials per step
    bool mergeInOProj = false;  // o_proj's prologue merges the attention partials
    bool oProjGroups = false;   // o_proj runs per kv group, merging that group's partials
    // Feed-forward block in one launch (FfnFused) for every layer but the last: its down product
    // lands in kResidualParts partial vectors of the hidden state (resParts), which the next
    // layer's QKV and o_proj sum. It reads the down weights transposed (downT, one copy per fused
    // layer), rebuilt before the next step whenever the down weights may have changed.
    bool ffnFused = false;
    float* resParts = nullptr;       // [kResidualParts][hidden]
    std::vector<TensorSlot> downT;   // per fused layer: [ffn][hidden] fp16
    bool downTStale = true;

    // Sampling (muyo_decoder_set_sampler): off = greedy from the LM head's argmax partials.
    bool sampling = false;
    SampleConfig sample{};
    float* sampleLogits = nullptr;  // the sampler's penalised, temperature-divided copy
    int32_t* sampledToken = nullptr;
    Mt64State* rng = nullptr;
    void* sampleWorkspace = nullptr;

    bool warm = false;
    // One graph per attention grid: [0] the long grid, [1] the short one (kShortAttnChunks chunks,
    // used while the position is below ShortAttnKeys and o_proj merges the partials).
    hipGraph_t graph[2] = {nullptr, nullptr};
    hipGraphExec_t exec[2] = {nullptr, nullptr};

    // Batched prefill (muyo_decoder_prefill): row-major activations of up to prefillRows prompt
    // tokens, allocated on first use. Split planes (hi, lo) feed the matrix cores.
    char* prefillArena = nullptr;
    uint32_t prefillRows = 0;
    int32_t* pTokens = nullptr;
    float* pxA = nullptr;   // [rows][hidden] residual stream, ping
    float* pxB = nullptr;   // pong
    float* pxMid = nullptr; // after attention
    float* pQkv = nullptr;  // [rows][qkvRows] projection with bias
    uint16_t* pNormHi = nullptr;  // [rows][hidden] normalised input of QKV and gate/up
    uint16_t* pNormLo = nullptr;
    uint16_t* pQHi = nullptr;  // [rows][qdim] roped queries
    uint16_t* pQLo = nullptr;
    uint16_t* pAttnHi = nullptr;  // [rows][qdim] attention output
    uint16_t* pAttnLo = nullptr;
    uint16_t* pActHi = nullptr;  // [rows][ffn] swiglu output
    uint16_t* pActLo = nullptr;
    float* pPartial = nullptr;   // [kMaxGemmSplits][rows][max(qkv rows, hidden)] K-split partial sums
    size_t pPartialFloats = 0;  // (or the split attention's partials, when larger)

    template <typename T>
    T* At(const TensorSlot& slot) const
    {
        return reinterpret_cast<T*>(arena + slot.offset);
    }

    const TensorSlot& Layer(uint32_t layer, LayerTensor tensor) const
    {
        return layers[static_cast<size_t>(layer) * kLayerTensorCount + tensor];
    }
};

namespace
{
int Validate(const MuyoQwen2Config& c)
{
    if (c.layers == 0 || c.hidden == 0 || c.feedForward == 0 || c.heads == 0 || c.kvHeads == 0 || c.headDim == 0 ||
        c.vocab == 0 || c.maxSeq == 0)
    {
        return Fail(MUYO_E_RANGE, "decoder: every dimension must be >= 1");
    }
    if (c.untiedOutput > 1)
    {
        return Fail(MUYO_E_RANGE, "decoder: untiedOutput must be 0 or 1");
    }
    if (c.heads % c.kvHeads != 0 || c.heads / c.kvHeads > 8)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: heads must be a multiple of kvHeads with a group of at most 8");
    }
    if (c.headDim != 64 && c.headDim != 128)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: headDim must be 64 or 128 (got %u)", c.headDim);
    }
    const uint64_t qdim = static_cast<uint64_t>(c.heads) * c.headDim;
    if (c.hidden % 8 != 0 || c.feedForward % 8 != 0 || qdim % 8 != 0)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: hidden, feedForward and heads*headDim must be multiples of 8");
    }
    if (static_cast<uint64_t>(std::max<uint64_t>({c.hidden, c.feedForward, qdim})) * 4 > 160 * 1024)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: a GEMV input longer than 40960 floats does not fit LDS");
    }
    if (c.hidden > 8192)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: hidden %u exceeds 8192 (the fused rms_norm prologue's one round)",
                    c.hidden);
    }
    if (c.maxSeq > kMaxSeq)
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder: maxSeq %u exceeds %u", c.maxSeq, kMaxSeq);
    }
    return MUYO_OK;
}

size_t LayerTensorBytes(const MuyoQwen2Config& c, LayerTensor t)
{
    const size_t hd = c.headDim;
    const size_t qkvRows = (static_cast<size_t>(c.heads) + 2 * c.kvHeads) * hd;
    const size_t qdim = static_cast<size_t>(c.heads) * hd;
    switch (t)
    {
        case kAttnNorm:
        case kFfnNorm:
            return static_cast<size_t>(c.hidden) * sizeof(float);
        case kQkv:
            return qkvRows * c.hidden * 2;
        case kQkvBias:
            return qkvRows * sizeof(float);
        case kOut:
            return static_cast<size_t>(c.hidden) * qdim * 2;
        case kGate:
        case kUp:
        case kDown:
            return static_cast<size_t>(c.feedForward) * c.hidden * 2;
        case kKCache:
        case kVCache:
            return static_cast<size_t>(c.kvHeads) * c.maxSeq * hd * 2;
        default:
            return 0;
    }
}

int LaunchFailed(hipError_t status, const char* kernel, uint32_t layer)
{
    return Fail(static_cast<int>(status), "decoder step: launching %s (layer %u) failed: %s (%d)", kernel, layer,
                hipGetErrorString(status), static_cast<int>(status));
}

/// The hidden state after layer l's attention. With o_proj split by kv group the groups add into
/// it atomically, so it alternates between two buffers by layer: the kernel before o_proj (the
/// step's BeginStep for layer 0, the previous layer's down projection otherwise) zeroes it while
/// the other one is still being read.
float* LayerMid(const MuyoDecoder* d, uint32_t l) { return d->oProjGroups && l % 2 == 1 ? d->xMid2 : d->xMid; }

hipError_t EnqueueEmbed(MuyoDecoder* d, hipStream_t s)
{
    return LaunchBeginStep(s, d->At<uint16_t>(d->tokenEmbd), d->state, d->scratch, d->argBlocks, d->xA, d->ids,
                           kIdsCapacity, d->config.hidden, d->config.vocab, d->oProjGroups ? LayerMid(d, 0) : nullptr);
}

/// The hidden state entering layer l: a single vector for layer 0 (the embedding) and on
/// decoders without the fused feed-forward block; otherwise the previous layer's partial vectors.
uint32_t LayerInputParts(const MuyoDecoder* d, uint32_t l) { return d->ffnFused && l > 0 ? kResidualParts : 1; }

/// True when layer l's feed-forward block is the one-launch FfnFused (all layers but the last,
/// whose output the LM head reads as one vector).
bool LayerFfnFused(const MuyoDecoder* d, uint32_t l) { return d->ffnFused && l + 1 < d->config.layers; }

hipError_t EnqueueQkv(MuyoDecoder* d, hipStream_t s, uint32_t l, const float* x)
{
    const uint32_t parts = LayerInputParts(d, l);
    return LaunchQkvRopeAppend(s, d->dims, parts > 1 ? d->resParts : x, d->At<float>(d->Layer(l, kAttnNorm)),
                               d->At<uint16_t>(d->Layer(l, kQkv)), d->At<float>(d->Layer(l, kQkvBias)), d->state,
                               d->q, d->At<uint16_t>(d->Layer(l, kKCache)), d->At<uint16_t>(d->Layer(l, kVCache)),
                               parts);
}

hipError_t EnqueueAttention(MuyoDecoder* d, hipStream_t s, uint32_t l)
{
    hipError_t status = LaunchAttention(s, d->dims, d->q, d->At<uint16_t>(d->Layer(l, kKCache)),
                                        d->At<uint16_t>(d->Layer(l, kVCache)), &d->state->position, d->scratch);
    if (status == hipSuccess && !d->mergeInOProj && !d->oProjGroups)
    {
        status = LaunchAttentionMerge(s, d->dims, d->scratch, d->attnOut);
    }
    return status;
}

hipError_t EnqueueOProj(MuyoDecoder* d, hipStream_t s, uint32_t l, const float* residual, float* out)
{
    const uint16_t* wo = d->At<uint16_t>(d->Layer(l, kOut));
    if (d->ffnFused)
    {
        // The residual is the layer's input; the output also seeds the fused block's parts.
        const uint32_t parts = LayerInputParts(d, l);
        const float* res = parts > 1 ? d->resParts : residual;
        float* seed = LayerFfnFused(d, l) ? d->resParts : nullptr;
        if (d->mergeInOProj)
        {
            return LaunchOProjMerged(s, d->dims, wo, d->scratch, res, out, parts, seed);
        }
        return LaunchOProjPlain(s, d->dims, wo, d->attnOut, res, out, parts, seed);
    }
    if (d->mergeInOProj)
    {
        return LaunchOProjMerged(s, d->dims, wo, d->scratch, residual, out);
    }
    if (d->oProjGroups)
    {
        return LaunchOProjGroups(s, d->dims, wo, d->scratch, residual, out);
    }
    return LaunchMatVecResidual(s, wo, d->attnOut, residual, out, d->config.hidden, d->config.heads * d->config.headDim);
}

/// `x` is the hidden state after attention.
hipError_t EnqueueGateUp(MuyoDecoder* d, hipStream_t s, uint32_t l, float* x)
{
    return LaunchGateUpSwiGlu(s, d->dims, x, d->At<float>(d->Layer(l, kFfnNorm)), d->At<uint16_t>(d->Layer(l, kGate)),
                              d->At<uint16_t>(d->Layer(l, kUp)), d->act);
}

/// Layer l's gate/up, swiglu and down in one launch, into the partial vectors o_proj seeded.
hipError_t EnqueueFfn(MuyoDecoder* d, hipStream_t s, uint32_t l)
{
    return LaunchFfnFused(s, d->dims, d->xMid, d->At<float>(d->Layer(l, kFfnNorm)),
                          d->At<uint16_t>(d->Layer(l, kGate)), d->At<uint16_t>(d->Layer(l, kUp)),
                          d->At<uint16_t>(d->downT[l]), d->resParts);
}

/// Rebuilds the transposed down weights of the fused layers when the down weights may have
/// changed since the last build (queued on `s`, before any step that reads them).
hipError_t PrepareDerived(MuyoDecoder* d, hipStream_t s)
{
    if (!d->ffnFused || !d->downTStale)
    {
        return hipSuccess;
    }
    for (uint32_t l = 0; l + 1 < d->config.layers; ++l)
    {
        const hipError_t status = LaunchTransposeF16(s, d->At<uint16_t>(d->Layer(l, kDown)), d->At<uint16_t>(d->downT[l]),
                                                     d->config.hidden, d->config.feedForward);
        if (status != hipSuccess)
        {
            return status;
        }
    }
    d->downTStale = false;
    return hipSuccess;
}

hipError_t EnqueueDown(MuyoDecoder* d, hipStream_t s, uint32_t l, const float* residual, float* out)
{
    if (d->oProjGroups && l + 1 < d->config.layers)
    {
        // Also zeroes the next layer's o_proj target.
        return LaunchMatVecResidualZero(s, d->At<uint16_t>(d->Layer(l, kDown)), d->act, residual, out,
                                        LayerMid(d, l + 1), d->config.hidden, d->config.feedForward);
    }
    return LaunchMatVecResidual(s, d->At<uint16_t>(d->Layer(l, kDown)), d->act, residual, out, d->config.hidden,
                                d->config.feedForward);
}

hipError_t EnqueueLmHead(MuyoDecoder* d, hipStream_t s, const float* x)
{
    const TensorSlot& head = d->config.untiedOutput != 0 ? d->output : d->tokenEmbd;
    return LaunchLmHeadArgMax(s, d->dims, x, d->At<float>(d->outputNorm), d->At<uint16_t>(head),
                              d->At<float>(d->logits), d->scratch);
}

int Enqueue(MuyoDecoder* d, hipStream_t s)
{
    const MuyoQwen2Config& c = d->config;
    hipError_t status = EnqueueEmbed(d, s);
    if (status != hipSuccess)
    {
        return LaunchFailed(status, "embed", 0);
    }
    float* x = d->xA;
    float* other = d->xB;
    for (uint32_t l = 0; l < d->config.layers; ++l)
    {
        if ((status = EnqueueQkv(d, s, l, x)) != hipSuccess)
        {
            return LaunchFailed(status, "qkv", l);
        }
        if ((status = EnqueueAttention(d, s, l)) != hipSuccess)
        {
            return LaunchFailed(status, "attention", l);
        }
        if ((status = EnqueueOProj(d, s, l, x, LayerMid(d, l))) != hipSuccess)
        {
            return LaunchFailed(status, "o_proj", l);
        }
        if (LayerFfnFused(d, l))
        {
            if ((status = EnqueueFfn(d, s, l)) != hipSuccess)
            {
                return LaunchFailed(status, "ffn", l);
            }
            continue;
        }
        if ((status = EnqueueGateUp(d, s, l, LayerMid(d, l))) != hipSuccess)
        {
            return LaunchFailed(status, "gate_up", l);
        }
        if ((status = EnqueueDown(d, s, l, LayerMid(d, l), other)) != hipSuccess)
        {
            return LaunchFailed(status, "down", l);
        }
        std::swap(x, other);
    }
    if ((status = EnqueueLmHead(d, s, x)) != hipSuccess)
    {
        return LaunchFailed(status, "lm_head", 0);
    }
    if (d->sampling)
    {
        // The logits stay as the LM head wrote them; the sampler works on its own copy, with the
        // history up to the current position.
        status = LaunchSample(s, d->At<float>(d->logits), d->sampleLogits, c.vocab, d->scratch.history,
                              &d->state->position, c.maxSeq, d->sample, d->rng,
                              SampleWorkspaceAt(d->sampleWorkspace, c.vocab, d->sample), d->sampledToken);
        if (status != hipSuccess)
        {
            return LaunchFailed(status, "sample", 0);
        }
    }
    return MUYO_OK;
}

/// The next step re-records its launches (eagerly, then a fresh capture).
void DropGraph(MuyoDecoder* d)
{
    for (int v = 0; v < 2; ++v)
    {
        if (d->exec[v] != nullptr)
        {
            (void)hipGraphExecDestroy(d->exec[v]);
            d->exec[v] = nullptr;
        }
        if (d->graph[v] != nullptr)
        {
            (void)hipGraphDestroy(d->graph[v]);
            d->graph[v] = nullptr;
        }
    }
    d->warm = false;
}

/// Captures the step with attention on `chunks` chunks per kv head into graph[variant] and
/// instantiates it. Runs nothing.
int CaptureStep(MuyoDecoder* d, int variant, uint32_t chunks)
{
    const uint32_t longChunks = d->dims.attnChunks;
    const hipError_t begin = hipStreamBeginCapture(d->stream, hipStreamCaptureModeRelaxed);
    if (begin != hipSuccess)
    {
        return HipStatus(begin, "graph capture");
    }
    d->dims.attnChunks = chunks;
    const int status = Enqueue(d, d->stream);
    d->dims.attnChunks = longChunks;
    hipGraph_t graph = nullptr;
    const hipError_t end = hipStreamEndCapture(d->stream, &graph);
    if (status != MUYO_OK)
    {
        if (graph != nullptr)
        {
            (void)hipGraphDestroy(graph);
        }
        return status;
    }
    if (end != hipSuccess)
    {
        return HipStatus(end, "hipStreamEndCapture");
    }
    d->graph[variant] = graph;
    MUYO_HIP_CHECK(hipGraphInstantiate(&d->exec[variant], d->graph[variant], nullptr, nullptr, 0));
    return MUYO_OK;
}

/// The step at `position` on `s`: eager the first time, graph replay afterwards. While o_proj
/// merges the attention partials and the position is below ShortAttnKeys, attention runs on
/// kShortAttnChunks chunks, whose first round of key blocks then covers every key: half the
/// partials for the merge to read (0.5B step at cache rows 960..1087: 0.561 -> 0.546 ms), where
/// past that point the second round costs more than the merge saves. Both graphs are captured
/// together, at the first replayed step, so crossing ShortAttnKeys later only switches between
/// two hipGraphLaunch calls (no synchronisation, no capture).
int RunStep(MuyoDecoder* d, hipStream_t s, int32_t position)
{
    MUYO_HIP_CHECK(PrepareDerived(d, s));
    const uint32_t longChunks = d->dims.attnChunks;
    const int variant =
        d->mergeInOProj && static_cast<uint32_t>(position) < ShortAttnKeys(d->config.headDim) ? 1 : 0;
    if (!d->warm)
    {
        d->dims.attnChunks = variant == 1 ? kShortAttnChunks : longChunks;
        const int status = Enqueue(d, s);
        d->dims.attnChunks = longChunks;
        d->warm = status == MUYO_OK;
        return status;
    }
    if (d->exec[0] == nullptr)
    {
        // Captured on the decoder's own stream once everything queued on `s` has run (the
        // capture itself runs nothing).
        MUYO_HIP_CHECK(hipStreamSynchronize(s));
        int status = CaptureStep(d, 0, longChunks);
        if (status == MUYO_OK && d->mergeInOProj)
        {
            status = CaptureStep(d, 1, kShortAttnChunks);
        }
        if (status != MUYO_OK)
        {
            DropGraph(d);
            return status;
        }
    }
    MUYO_HIP_CHECK(hipGraphLaunch(d->exec[variant], s));
    return MUYO_OK;
}

int FillTensor(MuyoDecoder* d, const TensorSlot& slot, bool half, uint64_t seed, double mean, double stddev)
{
    if (half)
    {
        return muyo_fill_normal_f16(d->arena + slot.offset, slot.bytes / 2, seed, mean, stddev, d->stream);
    }
    return muyo_fill_normal_f32(reinterpret_cast<float*>(d->arena + slot.offset), slot.bytes / 4, seed, mean, stddev,
                                d->stream);
}
}  // namespace

extern "C" int muyo_decoder_create(const MuyoQwen2Config* config, MuyoDecoder** out)
{
    if (config == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder_create: config and out are required");
    }
    *out = nullptr;
    const int valid = Validate(*config);
    if (valid != MUYO_OK)
    {
        return valid;
    }
    auto* d = new MuyoDecoder();
    d->config = *config;
    const MuyoQwen2Config& c = d->config;
    d->dims.hidden = c.hidden;
    d->dims.ffn = c.feedForward;
    d->dims.heads = c.heads;
    d->dims.kvHeads = c.kvHeads;
    d->dims.headDim = c.headDim;
    d->dims.vocab = c.vocab;
    d->dims.maxSeq = c.maxSeq;
    d->dims.eps = c.rmsEps;
    // The same f32 host computations as src/FullModel.cpp:184 and :201.
    d->dims.thetaScale = std::pow(c.ropeBase, -2.0F / static_cast<float>(c.headDim));
    d->dims.attnScale = 1.0F / std::sqrt(static_cast<float>(c.headDim));
    d->mergeInOProj = MergeInOProj(d->dims);
    d->dims.attnChunks = d->mergeInOProj ? kMergeAttnChunks : kMaxAttnChunks;
    d->oProjGroups = OProjInGroups(d->dims);
    d->ffnFused = FfnFusable(d->dims) && c.layers >= 2;

    // Arena layout: embedding, output norm, logits, then each layer's tensors, then activations
    // and scratch. Every tensor starts on a 256-byte boundary.
    size_t cursor = 0;
    auto place = [&cursor](size_t bytes)
    {
        TensorSlot slot{cursor, bytes};
        cursor = AlignUp(cursor + bytes);
        return slot;
    };
    d->tokenEmbd = place(static_cast<size_t>(c.vocab) * c.hidden * 2);
    d->outputNorm = place(static_cast<size_t>(c.hidden) * 4);
    d->logits = place(static_cast<size_t>(c.vocab) * 4);
    if (c.untiedOutput != 0)
    {
        d->output = place(static_cast<size_t>(c.vocab) * c.hidden * 2);
    }
    d->layers.resize(static_cast<size_t>(c.layers) * kLayerTensorCount);
    for (uint32_t l = 0; l < c.layers; ++l)
    {
        for (int t = 0; t < kLayerTensorCount; ++t)
        {
            d->layers[static_cast<size_t>(l) * kLayerTensorCount + t] =
                place(LayerTensorBytes(c, static_cast<LayerTensor>(t)));
        }
    }
    const size_t qdim = static_cast<size_t>(c.heads) * c.headDim;
    const size_t group = c.heads / c.kvHeads;
    const size_t chunks = AttnGridChunks(c.maxSeq, c.headDim, d->dims.attnChunks);
    const TensorSlot xA = place(c.hidden * 4);
    const TensorSlot xB = place(c.hidden * 4);
    const TensorSlot xMid = place(c.hidden * 4);
    const TensorSlot q = place(qdim * 4);
    const TensorSlot attnOut = place(qdim * 4);
    const TensorSlot xMid2 = place(c.hidden * 4);
    const TensorSlot act = place(static_cast<size_t>(c.feedForward) * 4);
    const TensorSlot resParts = place(d->ffnFused ? static_cast<size_t>(kResidualParts) * c.hidden * 4 : 0);
    if (d->ffnFused)
    {
        d->downT.resize(c.layers - 1);
        for (TensorSlot& slot : d->downT)
        {
            slot = place(static_cast<size_t>(c.feedForward) * c.hidden * 2);
        }
    }
    const TensorSlot state = place(sizeof(DecodeState));
    const TensorSlot ids = place(kIdsCapacity * 4);
    const size_t small = c.kvHeads * chunks * group;
    const TensorSlot attnMax = place(small * 4);
    const TensorSlot attnSum = place(small * 4);
    const TensorSlot attnAcc = place(small * c.headDim * 4);
    const TensorSlot argValue = place(kArgMaxBlocks * 4);
    const TensorSlot argIndex = place(kArgMaxBlocks * 4);
    const TensorSlot ropePow = place(static_cast<size_t>(c.headDim / 2) * 4);
    const TensorSlot history = place(static_cast<size_t>(c.maxSeq) * 4);
    const TensorSlot sampleLogits = place(static_cast<size_t>(c.vocab) * 4);
    const TensorSlot sampledToken = place(4);
    const TensorSlot rng = place(sizeof(Mt64State));
    // Room for the largest top-k the sampler takes; smaller ones use a prefix of each part.
    const SampleConfig widest{1.0F, static_cast<int32_t>(kSampleMaxTopK), 1.0F, 1.0F, 0};
    const TensorSlot sampleWorkspace = place(SampleWorkspaceBytes(c.vocab, widest));
    d->arenaBytes = cursor;

    hipError_t status = hipGetDevice(&d->device);
    if (status == hipSuccess)
    {
        status = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    }
    if (status == hipSuccess)
    {
        status = hipMalloc(reinterpret_cast<void**>(&d->arena), d->arenaBytes);
        if (status != hipSuccess)
        {
            d->arena = nullptr;
            const int code = Fail(MUYO_E_NOMEM, "decoder_create: hipMalloc of %zu bytes failed", d->arenaBytes);
            muyo_decoder_destroy(d);
            return code;
        }
    }
    if (status == hipSuccess)
    {
        status = hipMemsetAsync(d->arena, 0, d->arenaBytes, d->stream);
    }
    // The rope angles' powers, as the CPU path computes them (std::pow in f32, src/Rope.cpp:48-51).
    std::vector<float> powers(c.headDim / 2);
    for (uint32_t j = 0; j < c.headDim / 2; ++j)
    {
        powers[j] = std::pow(d->dims.thetaScale, static_cast<float>(j));
    }
    if (status == hipSuccess)
    {
        status = hipMemcpyAsync(d->arena + ropePow.offset, powers.data(), powers.size() * sizeof(float),
                                hipMemcpyHostToDevice, d->stream);
    }
    if (status == hipSuccess)
    {
        status = hipStreamSynchronize(d->stream);
    }
    if (status != hipSuccess)
    {
        const int code = HipStatus(status, "decoder_create");
        muyo_decoder_destroy(d);
        return code;
    }
    d->xA = d->At<float>(xA);
    d->xB = d->At<float>(xB);
    d->xMid = d->At<float>(xMid);
    d->q = d->At<float>(q);
    d->attnOut = d->At<float>(attnOut);
    d->xMid2 = d->At<float>(xMid2);
    d->act = d->At<float>(act);
    d->resParts = d->ffnFused ? d->At<float>(resParts) : nullptr;
    d->state = d->At<DecodeState>(state);
    d->ids = d->At<int32_t>(ids);
    d->scratch.attnMax = d->At<float>(attnMax);
    d->scratch.attnSum = d->At<float>(attnSum);
    d->scratch.attnAcc = d->At<float>(attnAcc);
    d->dims.ropePow = d->At<float>(ropePow);
    d->scratch.argValue = d->At<float>(argValue);
    d->scratch.argIndex = d->At<int32_t>(argIndex);
    d->scratch.history = d->At<int32_t>(history);
    d->scratch.historyCap = c.maxSeq;
    d->sampleLogits = d->At<float>(sampleLogits);
    d->sampledToken = d->At<int32_t>(sampledToken);
    d->rng = d->At<Mt64State>(rng);
    d->sampleWorkspace = d->arena + sampleWorkspace.offset;
    d->argBlocks = LmHeadBlocks(d->dims);
    *out = d;
    return MUYO_OK;
}

extern "C" int muyo_decoder_config(const MuyoDecoder* d, MuyoQwen2Config* out)
{
    if (d == nullptr || out == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder_config: decoder and out are required");
    }
    *out = d->config;
    return MUYO_OK;
}

extern "C" void muyo_decoder_destroy(MuyoDecoder* d)
{
    if (d == nullptr)
    {
        return;
    }
    for (int v = 0; v < 2; ++v)
    {
        if (d->exec[v] != nullptr)
        {
            (void)hipGraphExecDestroy(d->exec[v]);
        }
        if (d->graph[v] != nullptr)
        {
            (void)hipGraphDestroy(d->graph[v]);
        }
    }
    if (d->stream != nullptr)
    {
        (void)hipStreamSynchronize(d->stream);
    }
    if (d->arena != nullptr || d->prefillArena != nullptr)
    {
        (void)hipDeviceSynchronize();
        (void)hipFree(d->arena);
        (void)hipFree(d->prefillArena);
    }
    if (d->stream != nullptr)
    {
        (void)hipStreamDestroy(d->stream);
    }
    delete d;
}

namespace
{
int Lookup(MuyoDecoder* d, uint32_t kind, uint32_t layer, TensorSlot& slot)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    switch (kind)
    {
        case MUYO_TENSOR_TOKEN_EMBD:
            slot = d->tokenEmbd;
            return MUYO_OK;
        case MUYO_TENSOR_OUTPUT_NORM:
            slot = d->outputNorm;
            return MUYO_OK;
        case MUYO_TENSOR_LOGITS:
            slot = d->logits;
            return MUYO_OK;
        case MUYO_TENSOR_OUTPUT:
            if (d->config.untiedOutput == 0)
            {
                return Fail(MUYO_E_RANGE, "decoder: the LM head is tied to TOKEN_EMBD (config.untiedOutput is 0)");
            }
            slot = d->output;
            return MUYO_OK;
        default:
            break;
    }
    const LayerTensor t = ToLayerTensor(kind);
    if (t == kLayerTensorCount)
    {
        return Fail(MUYO_E_RANGE, "decoder: unknown tensor kind %u", kind);
    }
    if (layer >= d->config.layers)
    {
        return Fail(MUYO_E_RANGE, "decoder: layer %u out of range (%u layers)", layer, d->config.layers);
    }
    slot = d->Layer(layer, t);
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_decoder_tensor(MuyoDecoder* d, uint32_t kind, uint32_t layer, void** device_ptr, uint64_t* bytes)
{
    TensorSlot slot;
    const int status = Lookup(d, kind, layer, slot);
    if (status != MUYO_OK)
    {
        return status;
    }
    if (kind == MUYO_TENSOR_FFN_DOWN && device_ptr != nullptr)
    {
        d->downTStale = true;  // the caller may write through the pointer
    }
    if (device_ptr != nullptr)
    {
        *device_ptr = d->arena + slot.offset;
    }
    if (bytes != nullptr)
    {
        *bytes = slot.bytes;
    }
    return MUYO_OK;
}

extern "C" int muyo_decoder_upload(MuyoDecoder* d, uint32_t kind, uint32_t layer, const void* host, uint64_t bytes)
{
    TensorSlot slot;
    const int status = Lookup(d, kind, layer, slot);
    if (status != MUYO_OK)
    {
        return status;
    }
    if (host == nullptr || bytes != slot.bytes)
    {
        return Fail(MUYO_E_RANGE, "decoder_upload: %llu bytes given, tensor holds %zu",
                    static_cast<unsigned long long>(bytes), slot.bytes);
    }
    if (kind == MUYO_TENSOR_FFN_DOWN)
    {
        d->downTStale = true;
    }
    MUYO_HIP_CHECK(hipMemcpyAsync(d->arena + slot.offset, host, bytes, hipMemcpyHostToDevice, d->stream));
    MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    return MUYO_OK;
}

extern "C" int muyo_decoder_download(MuyoDecoder* d, uint32_t kind, uint32_t layer, void* host, uint64_t bytes)
{
    TensorSlot slot;
    const int status = Lookup(d, kind, layer, slot);
    if (status != MUYO_OK)
    {
        return status;
    }
    if (host == nullptr || bytes != slot.bytes)
    {
        return Fail(MUYO_E_RANGE, "decoder_download: %llu bytes given, tensor holds %zu",
                    static_cast<unsigned long long>(bytes), slot.bytes);
    }
    MUYO_HIP_CHECK(hipDeviceSynchronize());
    MUYO_HIP_CHECK(hipMemcpy(host, d->arena + slot.offset, bytes, hipMemcpyDeviceToHost));
    return MUYO_OK;
}

extern "C" int muyo_decoder_fill_random(MuyoDecoder* d, uint64_t seed)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    int status = FillTensor(d, d->tokenEmbd, true, muyo_tensor_seed(seed, MUYO_TENSOR_TOKEN_EMBD, 0), 0.0, 0.02);
    if (status == MUYO_OK)
    {
        status = FillTensor(d, d->outputNorm, false, muyo_tensor_seed(seed, MUYO_TENSOR_OUTPUT_NORM, 0), 1.0, 0.1);
    }
    if (status == MUYO_OK && d->config.untiedOutput != 0)
    {
        status = FillTensor(d, d->output, true, muyo_tensor_seed(seed, MUYO_TENSOR_OUTPUT, 0), 0.0, 0.02);
    }
    static const struct
    {
        uint32_t kind;
        LayerTensor tensor;
        bool half;
        double mean;
        double stddev;
    } kPlan[] = {
        {MUYO_TENSOR_ATTN_NORM, kAttnNorm, false, 1.0, 0.1}, {MUYO_TENSOR_ATTN_QKV, kQkv, true, 0.0, 0.02},
        {MUYO_TENSOR_ATTN_QKV_B, kQkvBias, false, 0.0, 0.02}, {MUYO_TENSOR_ATTN_OUTPUT, kOut, true, 0.0, 0.02},
        {MUYO_TENSOR_FFN_NORM, kFfnNorm, false, 1.0, 0.1},   {MUYO_TENSOR_FFN_GATE, kGate, true, 0.0, 0.02},
        {MUYO_TENSOR_FFN_UP, kUp, true, 0.0, 0.02},           {MUYO_TENSOR_FFN_DOWN, kDown, true, 0.0, 0.02},
    };
    for (uint32_t l = 0; l < d->config.layers && status == MUYO_OK; ++l)
    {
        for (const auto& p : kPlan)
        {
            status = FillTensor(d, d->Layer(l, p.tensor), p.half, muyo_tensor_seed(seed, p.kind, l), p.mean, p.stddev);
            if (status != MUYO_OK)
            {
                break;
            }
        }
        if (status == MUYO_OK)
        {
            const TensorSlot& kc = d->Layer(l, kKCache);
            const TensorSlot& vc = d->Layer(l, kVCache);
            if (hipMemsetAsync(d->arena + kc.offset, 0, kc.bytes, d->stream) != hipSuccess ||
                hipMemsetAsync(d->arena + vc.offset, 0, vc.bytes, d->stream) != hipSuccess)
            {
                status = HipStatus(hipGetLastError(), "decoder_fill_random: clearing the caches");
            }
        }
    }
    d->downTStale = true;
    if (status == MUYO_OK)
    {
        MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    }
    return status;
}

extern "C" int muyo_decoder_fill_kv_random(MuyoDecoder* d, uint32_t positions, uint64_t seed)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    const MuyoQwen2Config& c = d->config;
    if (positions > c.maxSeq)
    {
        return Fail(MUYO_E_RANGE, "decoder_fill_kv_random: %u positions exceed maxSeq %u", positions, c.maxSeq);
    }
    const size_t rowBytes = static_cast<size_t>(c.headDim) * 2;
    const size_t headBytes = rowBytes * c.maxSeq;
    for (uint32_t l = 0; l < c.layers; ++l)
    {
        for (uint32_t kind : {static_cast<uint32_t>(MUYO_TENSOR_KCACHE), static_cast<uint32_t>(MUYO_TENSOR_VCACHE)})
        {
            const TensorSlot& slot = d->Layer(l, ToLayerTensor(kind));
            // Whole tensor from the generator, then rows at or past `positions` cleared.
            int status = FillTensor(d, slot, true, muyo_tensor_seed(seed, kind, l), 0.0, 1.0);
            if (status != MUYO_OK)
            {
                return status;
            }
            const size_t tail = headBytes - rowBytes * positions;
            if (tail > 0)
            {
                for (uint32_t g = 0; g < c.kvHeads; ++g)
                {
                    MUYO_HIP_CHECK(hipMemsetAsync(d->arena + slot.offset + g * headBytes + rowBytes * positions, 0,
                                                  tail, d->stream));
                }
            }
        }
    }
    MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    return MUYO_OK;
}

extern "C" int muyo_decoder_generate_async(MuyoDecoder* d, int32_t token, int32_t position, uint32_t count,
                                           void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    const MuyoQwen2Config& c = d->config;
    if (token < 0 || static_cast<uint32_t>(token) >= c.vocab)
    {
        return Fail(MUYO_E_RANGE, "decoder: token %d outside [0, %u)", token, c.vocab);
    }
    if (position < 0 || static_cast<uint64_t>(position) + count > c.maxSeq)
    {
        return Fail(MUYO_E_RANGE, "decoder: positions %d..%d exceed the cache (%u rows)", position,
                    position + static_cast<int32_t>(count) - 1, c.maxSeq);
    }
    if (count > kIdsCapacity)
    {
        return Fail(MUYO_E_RANGE, "decoder: at most %u steps per call", kIdsCapacity);
    }
    hipStream_t s = AsStream(stream);
    MUYO_HIP_CHECK(LaunchSetState(s, d->state, d->scratch, token, position, d->argBlocks));
    for (uint32_t i = 0; i < count; ++i)
    {
        const int status = RunStep(d, s, position + static_cast<int32_t>(i));
        if (status != MUYO_OK)
        {
            return status;
        }
    }
    // The last step's id: its argmax partials reduced by a one-workgroup kernel.
    MUYO_HIP_CHECK(LaunchFinalize(s, d->state, d->scratch, d->argBlocks, d->ids, kIdsCapacity));
    return MUYO_OK;
}

extern "C" int muyo_decoder_generated_ids(MuyoDecoder* d, int32_t* ids, uint32_t count)
{
    if (d == nullptr || ids == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder_generated_ids: decoder and ids are required");
    }
    if (count > kIdsCapacity)
    {
        return Fail(MUYO_E_RANGE, "decoder_generated_ids: at most %u ids", kIdsCapacity);
    }
    MUYO_HIP_CHECK(hipDeviceSynchronize());
    MUYO_HIP_CHECK(hipMemcpy(ids, d->ids, static_cast<size_t>(count) * 4, hipMemcpyDeviceToHost));
    return MUYO_OK;
}

extern "C" int muyo_decoder_generate(MuyoDecoder* d, int32_t token, int32_t position, uint32_t count, int32_t* ids,
                                     void* stream)
{
    const int status = muyo_decoder_generate_async(d, token, position, count, stream);
    if (status != MUYO_OK)
    {
        return status;
    }
    MUYO_HIP_CHECK(hipStreamSynchronize(AsStream(stream)));
    return ids != nullptr ? muyo_decoder_generated_ids(d, ids, count) : MUYO_OK;
}

extern "C" int muyo_decoder_step(MuyoDecoder* d, int32_t token, int32_t position, int32_t* next_token)
{
    int32_t next = 0;
    const int status = muyo_decoder_generate(d, token, position, 1, &next, nullptr);
    if (status == MUYO_OK && next_token != nullptr)
    {
        *next_token = next;
    }
    return status;
}

extern "C" uint32_t muyo_decoder_launches_per_step(const MuyoDecoder* d)
{
    if (d == nullptr)
    {
        return 0;
    }
    uint32_t greedy = 2u + (d->mergeInOProj || d->oProjGroups ? 5u : 6u) * d->config.layers;
    if (d->ffnFused)
    {
        greedy -= d->config.layers - 1;  // one launch for gate/up and down in every layer but the last
    }
    return greedy + (d->sampling ? SampleLaunches(d->config.vocab, d->sample, true) : 0u);
}


extern "C" int muyo_decoder_set_sampler(MuyoDecoder* d, const MuyoSamplerParams* params)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    SampleConfig c{0.0F, 40, 0.95F, 1.0F, 64};
    uint64_t seed = 0;
    if (params != nullptr)
    {
        c = SampleConfig{params->temperature, params->top_k, params->top_p, params->repeat_penalty,
                         params->repeat_last_n};
        seed = params->seed;
    }
    if (!SampleSupported(c, d->config.vocab))
    {
        return Fail(MUYO_E_UNSUPPORTED, "decoder_set_sampler: a temperature above 0 needs top_k in 1..%u; got %d",
                    kSampleMaxTopK, c.topK);
    }
    MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    DropGraph(d);
    // Greedy without a penalty is the LM head's argmax; anything else runs the sampler.
    d->sampling = !(c.temperature <= 0.0F && c.repeatPenalty == 1.0F);
    d->sample = c;
    d->scratch.sampled = d->sampling ? d->sampledToken : nullptr;
    MUYO_HIP_CHECK(LaunchMt64Seed(d->stream, d->rng, seed));
    MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    return MUYO_OK;
}

extern "C" int muyo_decoder_set_history(MuyoDecoder* d, const int32_t* tokens, uint32_t count)
{
    if (d == nullptr || (tokens == nullptr && count > 0))
    {
        return Fail(MUYO_E_NULL, "decoder_set_history: decoder (and tokens when count > 0) required");
    }
    if (count > d->config.maxSeq)
    {
        return Fail(MUYO_E_RANGE, "decoder_set_history: %u tokens exceed the cache (%u rows)", count,
                    d->config.maxSeq);
    }
    MUYO_HIP_CHECK(hipStreamSynchronize(d->stream));
    MUYO_HIP_CHECK(hipMemcpy(d->scratch.history, tokens, static_cast<size_t>(count) * 4, hipMemcpyHostToDevice));
    return MUYO_OK;
}

extern "C" int muyo_decoder_set_state(MuyoDecoder* d, int32_t token, int32_t position, void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    if (token < 0 || static_cast<uint32_t>(token) >= d->config.vocab || position < 0 ||
        static_cast<uint32_t>(position) >= d->config.maxSeq)
    {
        return Fail(MUYO_E_RANGE, "decoder_set_state: token %d / position %d out of range", token, position);
    }
    const hipError_t status = LaunchSetState(AsStream(stream), d->state, d->scratch, token, position, d->argBlocks);
    return status == hipSuccess ? MUYO_OK : HipStatus(status, "decoder_set_state");
}

extern "C" int muyo_decoder_enqueue_kernel(MuyoDecoder* d, uint32_t kernel, uint32_t layer, void* stream)
{
    if (d == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder is NULL");
    }
    const MuyoQwen2Config& c = d->config;
    if (layer >= c.layers)
    {
        return Fail(MUYO_E_RANGE, "decoder_enqueue_kernel: layer %u out of range", layer);
    }
    hipStream_t s = AsStream(stream);
    hipError_t status = PrepareDerived(d, s);
    if (status != hipSuccess)
    {
        return HipStatus(status, "decoder_enqueue_kernel");
    }
    switch (kernel)
    {
        case MUYO_KERNEL_EMBED:
            status = EnqueueEmbed(d, s);
            break;
        case MUYO_KERNEL_QKV:
            status = EnqueueQkv(d, s, layer, d->xA);
            break;
        case MUYO_KERNEL_ATTENTION:
            status = EnqueueAttention(d, s, layer);
            break;
        case MUYO_KERNEL_O_PROJ:
            status = EnqueueOProj(d, s, layer, d->xA, LayerMid(d, layer));
            break;
        case MUYO_KERNEL_GATE_UP:
            status = EnqueueGateUp(d, s, layer, LayerMid(d, layer));
            break;
        case MUYO_KERNEL_DOWN:
            status = EnqueueDown(d, s, layer, LayerMid(d, layer), d->xB);
            break;
        case MUYO_KERNEL_FFN:
            if (!LayerFfnFused(d, layer))
            {
                return Fail(MUYO_E_UNSUPPORTED, "decoder_enqueue_kernel: layer %u runs gate/up and down apart", layer);
            }
            status = EnqueueFfn(d, s, layer);
            break;
        case MUYO_KERNEL_LM_HEAD:
            status = EnqueueLmHead(d, s, d->xA);
            break;
        default:
            return Fail(MUYO_E_RANGE, "decoder_enqueue_kernel: unknown kernel %u", kernel);
    }
    return status == hipSuccess ? MUYO_OK : HipStatus(status, "decoder_enqueue_kernel");
}

namespace
{
int EnsurePrefill(MuyoDecoder* d)
{
    if (d->prefillArena != nullptr)
    {
        return MUYO_OK;
    }
    const MuyoQwen2Config& c = d->config;
    const size_t rows = std::min<uint32_t>(kPrefillRows, c.maxSeq);
    const size_t qdim = static_cast<size_t>(c.heads) * c.headDim;
    const size_t qkvRows = (static_cast<size_t>(c.heads) + 2 * c.kvHeads) * c.headDim;
    size_t cursor = 0;
    auto place = [&cursor](size_t bytes)
    {
        const size_t at = cursor;
        cursor = AlignUp(cursor + bytes);
        return at;
    };
    const size_t tokens = place(rows * 4);
    const size_t xA = place(rows * c.hidden * 4);
    const size_t xB = place(rows * c.hidden * 4);
    const size_t xMid = place(rows * c.hidden * 4);
    const size_t qkv = place(rows * qkvRows * 4);
    const size_t normHi = place(rows * c.hidden * 2);
    const size_t normLo = place(rows * c.hidden * 2);
    const size_t qHi = place(rows * qdim * 2);
    const size_t qLo = place(rows * qdim * 2);
    const size_t attnHi = place(rows * qdim * 2);
    const size_t attnLo = place(rows * qdim * 2);
    const size_t actHi = place(rows * c.feedForward * 2);
    const size_t actLo = place(rows * c.feedForward * 2);
    // K-split partial sums of the GEMMs whose tiles alone leave the chip idle (GemmSplits), and,
    // between the q|k|v and o_proj GEMMs, the split attention's key-chunk partials.
    const size_t partialFloats = std::max(kMaxGemmSplits * rows * std::max<size_t>(qkvRows, c.hidden),
                                          PrefillAttentionWorkspaceFloats(static_cast<uint32_t>(rows), c.heads,
                                                                          c.headDim));
    const size_t partial = place(partialFloats * 4);
    char* arena = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&arena), cursor) != hipSuccess)
    {
        return Fail(MUYO_E_NOMEM, "decoder_prefill: hipMalloc of %zu bytes failed", cursor);
    }
    d->prefillArena = arena;
    d->prefillRows = static_cast<uint32_t>(rows);
    d->pTokens = reinterpret_cast<int32_t*>(arena + tokens);
    d->pxA = reinterpret_cast<float*>(arena + xA);
    d->pxB = reinterpret_cast<float*>(arena + xB);
    d->pxMid = reinterpret_cast<float*>(arena + xMid);
    d->pQkv = reinterpret_cast<float*>(arena + qkv);
    d->pNormHi = reinterpret_cast<uint16_t*>(arena + normHi);
    d->pNormLo = reinterpret_cast<uint16_t*>(arena + normLo);
    d->pQHi = reinterpret_cast<uint16_t*>(arena + qHi);
    d->pQLo = reinterpret_cast<uint16_t*>(arena + qLo);
    d->pAttnHi = reinterpret_cast<uint16_t*>(arena + attnHi);
    d->pAttnLo = reinterpret_cast<uint16_t*>(arena + attnLo);
    d->pActHi = reinterpret_cast<uint16_t*>(arena + actHi);
    d->pActLo = reinterpret_cast<uint16_t*>(arena + actLo);
    d->pPartial = reinterpret_cast<float*>(arena + partial);
    d->pPartialFloats = partialFloats;
    return MUYO_OK;
}

/// One pass of `rows` prompt tokens (already in pTokens) at positions pos0..: every layer as
/// GEMMs and a causal attention. Returns the residual stream holding the last layer's output.
int EnqueuePrefillPass(MuyoDecoder* d, hipStream_t s, uint32_t rows, int32_t pos0, float** result)
{
    const MuyoQwen2Config& c = d->config;
    const uint32_t qdim = c.heads * c.headDim;
    const uint32_t qkvRows = (c.heads + 2 * c.kvHeads) * c.headDim;
    hipError_t status = LaunchEmbedRows(s, d->At<uint16_t>(d->tokenEmbd), d->pTokens, rows, c.hidden, d->pxA,
                                        d->scratch.history, pos0, d->scratch.historyCap);
    if (status != hipSuccess)
    {
        return LaunchFailed(status, "prefill embed", 0);
    }
    float* x = d->pxA;
    float* other = d->pxB;
    uint32_t pending = 0;  // K splits of the previous layer's down GEMM not yet summed into x
    for (uint32_t l = 0; l < c.layers; ++l)
    {
        uint16_t* kcache = d->At<uint16_t>(d->Layer(l, kKCache));
        uint16_t* vcache = d->At<uint16_t>(d->Layer(l, kVCache));
        const float* attnNorm = d->At<float>(d->Layer(l, kAttnNorm));
        status = pending > 0 ? LaunchReduceRmsNormSplit(s, d->pxMid, d->pPartial, pending, x, attnNorm, rows,
                                                        c.hidden, c.rmsEps, d->pNormHi, d->pNormLo)
                             : LaunchRmsNormSplit(s, x, attnNorm, rows, c.hidden, c.rmsEps, d->pNormHi, d->pNormLo);
        if (status != hipSuccess)
        {
            return LaunchFailed(status, "prefill attn_norm", l);
        }
        const float* qkvBias = d->At<float>(d->Layer(l, kQkvBias));
        const uint32_t qkvSplits = GemmSplits(rows, qkvRows, c.hidden);
        if ((status = LaunchGemmSplit(s, d->pNormHi, d->pNormLo, d->At<uint16_t>(d->Layer(l, kQkv)), qkvBias, nullptr,
                                      d->pQkv, rows, qkvRows, c.hidden, d->pPartial, qkvSplits)) != hipSuccess)
        {
            return LaunchFailed(status, "prefill qkv", l);
        }
        if ((status = LaunchRopeSplitAppend(s, qkvSplits > 1 ? d->pPartial : d->pQkv, rows, pos0, c.heads, c.kvHeads,
                                            c.headDim, c.maxSeq, d->dims.ropePow, d->pQHi, d->pQLo, kcache, vcache,
                                            qkvSplits, qkvBias)) != hipSuccess)
        {
            return LaunchFailed(status, "prefill rope", l);
        }
        // The q|k|v partials are consumed (rope) and o_proj's are not yet written: the split
        // attention keeps its key-chunk partials in the same buffer meanwhile.
        if ((status = LaunchPrefillAttention(s, d->pQHi, d->pQLo, kcache, vcache, d->pAttnHi, d->pAttnLo, rows, pos0,
                                             c.heads, c.kvHeads, c.headDim, c.maxSeq, d->dims.attnScale,
                                             d->pPartial, d->pPartialFloats)) != hipSuccess)
        {
            return LaunchFailed(status, "prefill attention", l);
        }
        const uint32_t oSplits = GemmSplits(rows, c.hidden, qdim);
        if ((status = LaunchGemmSplit(s, d->pAttnHi, d->pAttnLo, d->At<uint16_t>(d->Layer(l, kOut)), nullptr, x,
                                      d->pxMid, rows, c.hidden, qdim, d->pPartial, oSplits)) != hipSuccess)
        {
            return LaunchFailed(status, "prefill o_proj", l);
        }
        const float* ffnNorm = d->At<float>(d->Layer(l, kFfnNorm));
        status = oSplits > 1 ? LaunchReduceRmsNormSplit(s, x, d->pPartial, oSplits, d->pxMid, ffnNorm, rows, c.hidden,
                                                        c.rmsEps, d->pNormHi, d->pNormLo)
                             : LaunchRmsNormSplit(s, d->pxMid, ffnNorm, rows, c.hidden, c.rmsEps, d->pNormHi,
                                                  d->pNormLo);
        if (status != hipSuccess)
        {
            return LaunchFailed(status, "prefill ffn_norm", l);
        }
        if ((status = LaunchGemmSwiGlu(s, d->pNormHi, d->pNormLo, d->At<uint16_t>(d->Layer(l, kGate)),
                                       d->At<uint16_t>(d->Layer(l, kUp)), d->pActHi, d->pActLo, rows, c.feedForward,
                                       c.hidden)) != hipSuccess)
        {
            return LaunchFailed(status, "prefill gate_up", l);
        }
        const uint32_t downSplits = GemmSplits(rows, c.hidden, c.feedForward);
        if ((status = LaunchGemmSplit(s, d->pActHi, d->pActLo, d->At<uint16_t>(d->Layer(l, kDown)), nullptr,
                                      d->pxMid, other, rows, c.hidden, c.feedForward, d->pPartial, downSplits)) !=
            hipSuccess)
        {
            return LaunchFailed(status, "prefill down", l);
        }
        pending = downSplits > 1 ? downSplits : 0;
        std::swap(x, other);
    }
    if (pending > 0)
    {
        status = LaunchReduceRmsNormSplit(s, d->pxMid, d->pPartial, pending, x, nullptr, rows, c.hidden, c.rmsEps,
                                          nullptr, nullptr);
        if (status != hipSuccess)
        {
            return LaunchFailed(status, "prefill down", c.layers - 1);
        }
    }
    *result = x;
    return MUYO_OK;
}
}  // namespace

extern "C" int muyo_decoder_prefill(MuyoDecoder* d, const int32_t* tokens, uint32_t count, int32_t position,
                                    int32_t* next_token)
{
    if (d == nullptr || tokens == nullptr)
    {
        return Fail(MUYO_E_NULL, "decoder_prefill: decoder and tokens are required");
    }
    const MuyoQwen2Config& c = d->config;
    if (count == 0)
    {
        return Fail(MUYO_E_RANGE, "decoder_prefill: at least one token is required");
    }
    if (position < 0 || static_cast<uint64_t>(position) + count > c.maxSeq)
    {
        return Fail(MUYO_E_RANGE, "decoder_prefill: positions %d..%lld exceed the cache (%u rows)", position,
                    static_cast<long long>(position) + count - 1, c.maxSeq);
    }
    for (uint32_t i = 0; i < count; ++i)
    {
        if (tokens[i] < 0 || static_cast<uint32_t>(tokens[i]) >= c.vocab)
        {
            return Fail(MUYO_E_RANGE, "decoder_prefill: token %d (index %u) outside [0, %u)", tokens[i], i, c.vocab);
        }
    }
    int status = EnsurePrefill(d);
    if (status != MUYO_OK)
    {
        return status;
    }
    // Work queued earlier on other streams (an asynchronous generation) writes the same caches.
    MUYO_HIP_CHECK(hipDeviceSynchronize());
    hipStream_t s = d->stream;
    float* x = nullptr;
    uint32_t rows = 0;
    for (uint32_t done = 0; done < count; done += rows)
    {
        rows = std::min(d->prefillRows, count - done);
        MUYO_HIP_CHECK(hipMemcpyAsync(d->pTokens, tokens + done, static_cast<size_t>(rows) * 4,
                                      hipMemcpyHostToDevice, s));
        status = EnqueuePrefillPass(d, s, rows, position + static_cast<int32_t>(done), &x);
        if (status != MUYO_OK)
        {
            return status;
        }
    }
    // The last prompt position is the step just run: its logits give the next token, greedy or
    // sampled, exactly as after a decode step there.
    const int32_t last = position + static_cast<int32_t>(count) - 1;
    MUYO_HIP_CHECK(LaunchSetState(s, d->state, d->scratch, tokens[count - 1], last, d->argBlocks, 1));
    const hipError_t head = EnqueueLmHead(d, s, x + static_cast<size_t>(rows - 1) * c.hidden);
    if (head != hipSuccess)
    {
        return LaunchFailed(head, "prefill lm_head", 0);
    }
    if (d->sampling)
    {
        const hipError_t sampled =
            LaunchSample(s, d->At<float>(d->logits), d->sampleLogits, c.vocab, d->scratch.history,
                         &d->state->position, c.maxSeq, d->sample, d->rng,
                         SampleWorkspaceAt(d->sampleWorkspace, c.vocab, d->sample), d->sampledToken);
        if (sampled != hipSuccess)
        {
            return LaunchFailed(sampled, "prefill sample", 0);
        }
    }
    MUYO_HIP_CHECK(LaunchFinalize(s, d->state, d->scratch, d->argBlocks, d->ids, kIdsCapacity));
    int32_t next = 0;
    MUYO_HIP_CHECK(hipMemcpyAsync(&next, d->ids, sizeof(next), hipMemcpyDeviceToHost, s));
    MUYO_HIP_CHECK(hipStreamSynchronize(s));
    if (next_token != nullptr)
    {
        *next_token = next;
    }
    return MUYO_OK;
}
