// The reference's node self-tests (`int RunX()`, src/{MatVec,RmsNorm,Rope,SoftMax,Argmax,
// ElementwiseAdd,Swiglu,GetRows,KvCache,Attention}.cpp) on the gfx950 launchers.
//
// Each test keeps its reference's inputs, its push-constant fill (include/muyo/Nodes.h), its CPU
// check and its tolerance, and prints the same "[op] OK: ..." line. Only the execution differs:
// a node's Execute(stream) replaces the render graph's record and submit.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "muyo/Argmax.h"
#include "muyo/Attention.h"
#include "muyo/ElementwiseAdd.h"
#include "muyo/GetRows.h"
#include "muyo/KvCache.h"
#include "muyo/MatVec.h"
#include "muyo/Nodes.h"
#include "muyo/RmsNorm.h"
#include "muyo/Rope.h"
#include "muyo/SoftMax.h"
#include "muyo/Swiglu.h"

namespace muyo_llm
{
namespace
{
using namespace hip;

/// Device copy of a host vector, freed with the object.
template <typename T>
class DeviceBuffer
{
public:
    explicit DeviceBuffer(size_t count) : m_count(count)
    {
        if (hipMalloc(reinterpret_cast<void**>(&m_ptr), std::max<size_t>(count, 1) * sizeof(T)) != hipSuccess)
        {
            m_ptr = nullptr;
        }
        else
        {
            (void)hipMemset(m_ptr, 0, std::max<size_t>(count, 1) * sizeof(T));
        }
    }
    explicit DeviceBuffer(const std::vector<T>& host) : DeviceBuffer(host.size())
    {
        if (m_ptr != nullptr)
        {
            (void)hipMemcpy(m_ptr, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice);
        }
    }
    ~DeviceBuffer()
    {
        if (m_ptr != nullptr)
        {
            (void)hipFree(m_ptr);
        }
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    T* get() const { return m_ptr; }
    bool ok() const { return m_ptr != nullptr; }
    void Upload(const std::vector<T>& host) { (void)hipMemcpy(m_ptr, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice); }
    std::vector<T> Download() const
    {
        std::vector<T> host(m_count);
        if (hipDeviceSynchronize() != hipSuccess ||
            hipMemcpy(host.data(), m_ptr, m_count * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        {
            std::fill(host.begin(), host.end(), T{});
        }
        return host;
    }

private:
    T* m_ptr = nullptr;
    size_t m_count = 0;
};

uint16_t ToHalf(float value) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(value)); }
float FromHalf(uint16_t bits) { return static_cast<float>(__builtin_bit_cast(_Float16, bits)); }

bool Launched(int status, const char* op)
{
    if (status != MUYO_OK)
    {
        std::fprintf(stderr, "[fail] %s launch: %s (%d)\n", op, muyo_last_error(), status);
        return false;
    }
    return true;
}

bool Near(float actual, float expected, float tolerance)
{
    return std::fabs(actual - expected) <= tolerance * (1.0F + std::fabs(expected));
}

/// Counts the elements outside the tolerance and prints the first few.
uint32_t CountWrong(const std::vector<float>& actual, const std::vector<float>& expected, float tolerance,
                    const char* label)
{
    uint32_t wrong = 0;
    for (size_t i = 0; i < expected.size(); ++i)
    {
        if (!(tolerance == 0.0F ? actual[i] == expected[i] : Near(actual[i], expected[i], tolerance)))
        {
            if (wrong < 4)
            {
                std::fprintf(stderr, "[fail] %s[%zu] = %g, expected %g\n", label, i, actual[i], expected[i]);
            }
            ++wrong;
        }
    }
    return wrong;
}

/// Single-head attention over `keys` cached rows, in the reference's order (src/Attention.cpp:253-294).
std::vector<float> HostAttention(const std::vector<float>& query, const std::vector<std::vector<float>>& keys,
                                 const std::vector<std::vector<float>>& values)
{
    const size_t dim = query.size();
    std::vector<float> scores(keys.size());
    for (size_t j = 0; j < keys.size(); ++j)
    {
        float dot = 0.0F;
        for (size_t d = 0; d < dim; ++d)
        {
            dot += keys[j][d] * query[d];
        }
        scores[j] = dot / std::sqrt(static_cast<float>(dim));
    }
    const float top = *std::max_element(scores.begin(), scores.end());
    double sum = 0.0;
    std::vector<double> weights(keys.size());
    for (size_t j = 0; j < keys.size(); ++j)
    {
        weights[j] = std::exp(scores[j] - top);
        sum += weights[j];
    }
    std::vector<float> out(dim, 0.0F);
    for (size_t j = 0; j < keys.size(); ++j)
    {
        for (size_t d = 0; d < dim; ++d)
        {
            out[d] += static_cast<float>(weights[j] / sum) * values[j][d];
        }
    }
    return out;
}

/// NeoX rotation of one row at `position` (src/KvCache.cpp:78-91).
std::vector<float> HostRope(const std::vector<float>& x, int32_t position, float freqBase)
{
    const uint32_t n = static_cast<uint32_t>(x.size());
    const float thetaScale = std::pow(freqBase, -2.0F / static_cast<float>(n));
    std::vector<float> out(n);
    for (uint32_t j = 0; j < n / 2; ++j)
    {
        const float theta = static_cast<float>(position) * std::pow(thetaScale, static_cast<float>(j));
        out[j] = x[j] * std::cos(theta) - x[j + n / 2] * std::sin(theta);
        out[j + n / 2] = x[j] * std::sin(theta) + x[j + n / 2] * std::cos(theta);
    }
    return out;
}
}  // namespace

int RunMatVec()
{
    constexpr uint32_t kRows = 128;
    constexpr uint32_t kCols = 256;
    std::vector<uint16_t> hostA(kRows * kCols);
    std::vector<float> hostB(kCols);
    for (uint32_t row = 0; row < kRows; ++row)
    {
        for (uint32_t column = 0; column < kCols; ++column)
        {
            hostA[row * kCols + column] = ToHalf(static_cast<float>(static_cast<int>(column % 7) - 3));
        }
    }
    for (uint32_t column = 0; column < kCols; ++column)
    {
        hostB[column] = static_cast<float>(static_cast<int>(column % 5) - 2);
    }
    DeviceBuffer<uint16_t> a(hostA);
    DeviceBuffer<float> b(hostB);
    DeviceBuffer<float> d(kRows);
    MatVecF16Node node;
    node.pc = MakeMatVec(kCols, kRows);
    node.a = a.get();
    node.b = b.get();
    node.d = d.get();
    node.dispatch = {kRows, 1, 1};
    if (!Launched(node.Execute(nullptr), "matvec"))
    {
        return 1;
    }
    std::vector<float> expected(kRows);
    for (uint32_t row = 0; row < kRows; ++row)
    {
        float sum = 0.0F;
        for (uint32_t column = 0; column < kCols; ++column)
        {
            sum += FromHalf(hostA[row * kCols + column]) * hostB[column];
        }
        expected[row] = sum;
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 0.0F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u rows wrong\n", wrong, kRows);
        return 1;
    }
    std::printf("[matvec] OK: mul_mat_vec (F16 weights) over %ux%u matches the CPU reference\n", kRows, kCols);
    return 0;
}

int RunRmsNorm()
{
    constexpr uint32_t kRows = 8;
    constexpr uint32_t kCols = 512;
    constexpr float kEpsilon = 1e-6F;
    std::vector<float> hostA(kRows * kCols);
    std::vector<float> hostWeight(kCols);
    for (uint32_t i = 0; i < kRows * kCols; ++i)
    {
        hostA[i] = static_cast<float>(static_cast<int>(i % 13) - 6);
    }
    for (uint32_t column = 0; column < kCols; ++column)
    {
        hostWeight[column] = 0.5F + 0.001F * static_cast<float>(column % 11);
    }
    DeviceBuffer<float> a(hostA);
    DeviceBuffer<float> w(hostWeight);
    DeviceBuffer<float> d(kRows * kCols);
    RmsNormNode node;
    node.pc = MakeRows(kCols, kRows, kEpsilon);
    node.a = a.get();
    node.b = w.get();
    node.d = d.get();
    node.dispatch = {kRows, 1, 1};
    if (!Launched(node.Execute(nullptr), "rms_norm"))
    {
        return 1;
    }
    std::vector<float> expected(kRows * kCols);
    for (uint32_t row = 0; row < kRows; ++row)
    {
        double sumSquares = 0.0;
        for (uint32_t column = 0; column < kCols; ++column)
        {
            const double value = hostA[row * kCols + column];
            sumSquares += value * value;
        }
        const float scale = static_cast<float>(1.0 / std::sqrt(sumSquares / kCols + kEpsilon));
        for (uint32_t column = 0; column < kCols; ++column)
        {
            expected[row * kCols + column] = hostA[row * kCols + column] * scale * hostWeight[column];
        }
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 1e-4F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u elements wrong\n", wrong, kRows * kCols);
        return 1;
    }
    std::printf("[rmsnorm] OK: rms_norm over %ux%u matches the CPU reference\n", kRows, kCols);
    return 0;
}

int RunRope()
{
    constexpr uint32_t kDims = 8;
    constexpr float kFreqBase = 10000.0F;
    constexpr int32_t kPosition = 3;
    std::vector<float> hostX(kDims);
    for (uint32_t c = 0; c < kDims; ++c)
    {
        hostX[c] = static_cast<float>(static_cast<int>(c) - 3);
    }
    DeviceBuffer<float> x(hostX);
    DeviceBuffer<int32_t> position(std::vector<int32_t>{kPosition});
    DeviceBuffer<float> d(kDims);
    RopeNode node;
    node.pc = MakeRopeNeox(1, kDims, kFreqBase);
    node.x = x.get();
    node.positions = position.get();
    node.d = d.get();
    node.dispatch = {1, 1, 1};
    if (!Launched(node.Execute(nullptr), "rope"))
    {
        return 1;
    }
    const uint32_t wrong = CountWrong(d.Download(), HostRope(hostX, kPosition, kFreqBase), 1e-5F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u channels wrong\n", wrong, kDims);
        return 1;
    }
    std::printf("[rope] OK: rope_neox over %u channels matches the CPU reference\n", kDims);
    return 0;
}

int RunSoftMax()
{
    constexpr uint32_t kColumns = 64;
    constexpr float kScale = 1.0F / 8.0F;
    std::vector<float> hostX(kColumns);
    for (uint32_t c = 0; c < kColumns; ++c)
    {
        hostX[c] = static_cast<float>(static_cast<int>(c % 9) - 4);
    }
    DeviceBuffer<float> x(hostX);
    DeviceBuffer<float> d(kColumns);
    SoftMaxNode node;
    node.pc = MakeSoftMax(1, kColumns, kScale);
    node.x = x.get();
    node.d = d.get();
    node.dispatch = {1, 1, 1};
    if (!Launched(node.Execute(nullptr), "soft_max"))
    {
        return 1;
    }
    float top = -INFINITY;
    for (float v : hostX)
    {
        top = std::max(top, v * kScale);
    }
    double sum = 0.0;
    std::vector<float> expected(kColumns);
    for (uint32_t c = 0; c < kColumns; ++c)
    {
        expected[c] = std::exp(hostX[c] * kScale - top);
        sum += expected[c];
    }
    for (float& e : expected)
    {
        e = static_cast<float>(e / sum);
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 1e-5F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u columns wrong\n", wrong, kColumns);
        return 1;
    }
    std::printf("[softmax] OK: soft_max over %u columns matches the CPU reference\n", kColumns);
    return 0;
}

int RunArgmax()
{
    constexpr uint32_t kLogits = 32;
    constexpr int32_t kExpected = 21;
    std::vector<float> hostLogits(kLogits);
    for (uint32_t i = 0; i < kLogits; ++i)
    {
        hostLogits[i] = -1.0F + 0.001F * static_cast<float>(i);
    }
    hostLogits[kExpected] = 5.0F;
    DeviceBuffer<float> a(hostLogits);
    DeviceBuffer<int32_t> d(1);
    ArgmaxNode node;
    node.pc = MakeArgmax(kLogits);
    node.a = a.get();
    node.d = d.get();
    if (!Launched(node.Execute(nullptr), "argmax"))
    {
        return 1;
    }
    const int32_t result = d.Download()[0];
    if (result != kExpected)
    {
        std::fprintf(stderr, "[fail] argmax picked %d, expected %d\n", result, kExpected);
        return 1;
    }
    std::printf("[argmax] OK: argmax picked token %d from %u logits\n", result, kLogits);
    return 0;
}

int RunElementwiseAdd()
{
    constexpr uint32_t kCount = 1000;
    std::vector<float> hostA(kCount);
    std::vector<float> hostB(kCount);
    for (uint32_t i = 0; i < kCount; ++i)
    {
        hostA[i] = 0.5F * static_cast<float>(i);
        hostB[i] = 1.0F + 0.25F * static_cast<float>(i);
    }
    DeviceBuffer<float> a(hostA);
    DeviceBuffer<float> b(hostB);
    DeviceBuffer<float> d(kCount);
    AddNode node;
    node.pc = MakeAdd(kCount);
    node.a = a.get();
    node.b = b.get();
    node.d = d.get();
    node.dispatch = ElementDispatch(kCount);
    if (!Launched(node.Execute(nullptr), "add"))
    {
        return 1;
    }
    std::vector<float> expected(kCount);
    for (uint32_t i = 0; i < kCount; ++i)
    {
        expected[i] = hostA[i] + hostB[i];
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 0.0F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u elements wrong\n", wrong, kCount);
        return 1;
    }
    std::printf("[add] OK: add_f32 over %u elements matches the CPU reference\n", kCount);
    return 0;
}

int RunSwiglu()
{
    constexpr uint32_t kCount = 600;
    std::vector<float> hostGate(kCount);
    std::vector<float> hostUp(kCount);
    for (uint32_t i = 0; i < kCount; ++i)
    {
        hostGate[i] = 0.01F * static_cast<float>(static_cast<int>(i % 17) - 8);
        hostUp[i] = 0.5F + 0.01F * static_cast<float>(i % 7);
    }
    DeviceBuffer<float> gate(hostGate);
    DeviceBuffer<float> up(hostUp);
    DeviceBuffer<float> d(kCount);
    SwigluNode node;
    node.pc = MakeSwiglu(kCount);
    node.a = gate.get();
    node.b = up.get();
    node.d = d.get();
    node.dispatch = ElementDispatch(kCount);
    if (!Launched(node.Execute(nullptr), "swiglu"))
    {
        return 1;
    }
    std::vector<float> expected(kCount);
    for (uint32_t i = 0; i < kCount; ++i)
    {
        expected[i] = hostGate[i] / (1.0F + std::exp(-hostGate[i])) * hostUp[i];
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 1e-5F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u elements wrong\n", wrong, kCount);
        return 1;
    }
    std::printf("[swiglu] OK: swiglu over %u elements matches the CPU reference\n", kCount);
    return 0;
}

int RunGetRows()
{
    constexpr uint32_t kDim = 512;
    constexpr uint32_t kVocab = 1024;
    constexpr int32_t kToken = 7;
    std::vector<uint16_t> hostTable(kVocab * kDim);
    for (uint32_t t = 0; t < kVocab; ++t)
    {
        for (uint32_t c = 0; c < kDim; ++c)
        {
            hostTable[t * kDim + c] =
                ToHalf(static_cast<float>(static_cast<int>(t % 5) - 2) + 0.001F * static_cast<float>(c));
        }
    }
    DeviceBuffer<uint16_t> table(hostTable);
    DeviceBuffer<int32_t> index(std::vector<int32_t>{kToken});
    DeviceBuffer<float> d(kDim);
    GetRowsF16Node node;
    node.pc = MakeGetRows(kDim, kVocab);
    node.a = table.get();
    node.b = index.get();
    node.d = d.get();
    node.dispatch = {1, 1, 1};
    if (!Launched(node.Execute(nullptr), "get_rows"))
    {
        return 1;
    }
    std::vector<float> expected(kDim);
    for (uint32_t c = 0; c < kDim; ++c)
    {
        expected[c] = FromHalf(hostTable[kToken * kDim + c]);
    }
    const uint32_t wrong = CountWrong(d.Download(), expected, 0.0F, "D");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u channels wrong\n", wrong, kDim);
        return 1;
    }
    std::printf("[getrows] OK: get_rows gathered token %d's %u-channel embedding\n", kToken, kDim);
    return 0;
}

int RunAttention()
{
    constexpr uint32_t kDim = 8;
    constexpr uint32_t kKeys = 16;
    std::vector<float> hostQuery(kDim);
    std::vector<std::vector<float>> keys(kKeys, std::vector<float>(kDim));
    std::vector<std::vector<float>> values(kKeys, std::vector<float>(kDim));
    std::vector<float> keysFlat(kKeys * kDim);
    std::vector<float> valuesTransposed(kDim * kKeys);
    for (uint32_t d = 0; d < kDim; ++d)
    {
        hostQuery[d] = static_cast<float>(static_cast<int>(d % 5) - 2);
    }
    for (uint32_t key = 0; key < kKeys; ++key)
    {
        for (uint32_t d = 0; d < kDim; ++d)
        {
            keys[key][d] = static_cast<float>(static_cast<int>((key + d) % 3) - 1);
            values[key][d] = static_cast<float>(static_cast<int>((key * 2 + d) % 7) - 3);
            keysFlat[key * kDim + d] = keys[key][d];
            valuesTransposed[d * kKeys + key] = values[key][d];
        }
    }
    DeviceBuffer<float> q(hostQuery);
    DeviceBuffer<float> k(keysFlat);
    DeviceBuffer<float> vt(valuesTransposed);
    DeviceBuffer<float> scores(kKeys);
    DeviceBuffer<float> probs(kKeys);
    DeviceBuffer<float> out(kDim);
    MatVecF32Node score;
    score.pc = MakeMatVec(kDim, kKeys);
    score.a = k.get();
    score.b = q.get();
    score.d = scores.get();
    score.dispatch = {kKeys, 1, 1};
    SoftMaxNode softmax;
    softmax.pc = MakeSoftMax(1, kKeys, 1.0F / std::sqrt(static_cast<float>(kDim)));
    softmax.x = scores.get();
    softmax.d = probs.get();
    MatVecF32Node value;
    value.pc = MakeMatVec(kKeys, kDim);
    value.a = vt.get();
    value.b = probs.get();
    value.d = out.get();
    value.dispatch = {kDim, 1, 1};
    if (!Launched(score.Execute(nullptr), "scores") || !Launched(softmax.Execute(nullptr), "softmax") ||
        !Launched(value.Execute(nullptr), "values"))
    {
        return 1;
    }
    const uint32_t wrong = CountWrong(out.Download(), HostAttention(hostQuery, keys, values), 1e-4F, "out");
    if (wrong != 0)
    {
        std::fprintf(stderr, "[fail] %u of %u attention outputs wrong\n", wrong, kDim);
        return 1;
    }
    std::printf("[attention] OK: scores -> softmax -> values over %u keys matches the CPU reference\n", kKeys);
    return 0;
}

int RunKvCache()
{
    constexpr uint32_t kKvDim = 16;
    constexpr uint32_t kMaxSeq = 4;
    constexpr uint32_t kTokens = 2;
    constexpr float kFreqBase = 10000.0F;
    std::vector<float> query(kKvDim);
    for (uint32_t d = 0; d < kKvDim; ++d)
    {
        query[d] = static_cast<float>(static_cast<int>(d % 5) - 2);
    }
    DeviceBuffer<float> keyCache(kMaxSeq * kKvDim);
    DeviceBuffer<float> valueCacheT(kKvDim * kMaxSeq);
    DeviceBuffer<float> keyVector(kKvDim);
    DeviceBuffer<float> valueVector(kKvDim);
    DeviceBuffer<float> q(query);
    DeviceBuffer<float> scores(kMaxSeq);
    DeviceBuffer<float> probs(kMaxSeq);
    DeviceBuffer<float> out(kKvDim);
    DeviceBuffer<int32_t> ropePosition(1);
    std::vector<std::vector<float>> roped;
    std::vector<std::vector<float>> cachedValues;
    uint32_t wrongTotal = 0;
    for (uint32_t token = 0; token < kTokens; ++token)
    {
        std::vector<float> key(kKvDim);
        std::vector<float> value(kKvDim);
        for (uint32_t d = 0; d < kKvDim; ++d)
        {
            key[d] = static_cast<float>(static_cast<int>((token * 3 + d) % 5) - 2);
            value[d] = static_cast<float>(static_cast<int>((token + d) % 5) - 2);
        }
        keyVector.Upload(key);
        valueVector.Upload(value);
        ropePosition.Upload(std::vector<int32_t>{static_cast<int32_t>(token)});
        roped.push_back(HostRope(key, static_cast<int32_t>(token), kFreqBase));
        cachedValues.push_back(value);

        // Append: k roped into cache row `token`, v into column `token` of the transposed cache.
        RopeNode appendKey;
        appendKey.pc = MakeRopeNeox(1, kKvDim, kFreqBase, kKvDim * kMaxSeq, token * kKvDim);
        appendKey.x = keyVector.get();
        appendKey.positions = ropePosition.get();
        appendKey.d = keyCache.get();
        CopyNode appendValue;
        appendValue.pc = MakeCacheValueColumn(kKvDim, kMaxSeq, token);
        appendValue.a = valueVector.get();
        appendValue.d = valueCacheT.get();
        appendValue.dispatch = {1, 1, 1};
        // Attention over the token + 1 cached keys.
        const uint32_t keys = token + 1;
        MatVecF32Node score;
        score.pc = MakeMatVec(kKvDim, keys);
        score.a = keyCache.get();
        score.b = q.get();
        score.d = scores.get();
        score.dispatch = {keys, 1, 1};
        SoftMaxNode softmax;
        softmax.pc = MakeSoftMax(1, keys, 1.0F / std::sqrt(static_cast<float>(kKvDim)));
        softmax.x = scores.get();
        softmax.d = probs.get();
        // The GEMV's A row stride is ncols, so the value GEMV spans whole cache rows; columns past
        // the last key are still zero and add nothing (src/KvCache.cpp:296-303).
        MatVecF32Node weighted;
        weighted.pc = MakeMatVec(kMaxSeq, kKvDim);
        weighted.a = valueCacheT.get();
        weighted.b = probs.get();
        weighted.d = out.get();
        weighted.dispatch = {kKvDim, 1, 1};
        if (!Launched(appendKey.Execute(nullptr), "k append") || !Launched(appendValue.Execute(nullptr), "v append") ||
            !Launched(score.Execute(nullptr), "scores") || !Launched(softmax.Execute(nullptr), "softmax") ||
            !Launched(weighted.Execute(nullptr), "values"))
        {
            return 1;
        }
        const uint32_t wrong = CountWrong(out.Download(), HostAttention(query, roped, cachedValues), 1e-4F, "out");
        if (wrong != 0)
        {
            std::fprintf(stderr, "[fail] token %u: %u of %u outputs wrong\n", token, wrong, kKvDim);
            wrongTotal += wrong;
        }
    }
    if (wrongTotal != 0)
    {
        return 1;
    }
    std::printf("[kvcache] OK: %u appended tokens, attention over the growing cache matches the CPU reference\n",
                kTokens);
    return 0;
}
}  // namespace muyo_llm

/// The self-tests by the reference CLI's mode names (src/main.cpp:246-248).
extern "C" int muyo_self_test(const char* mode)
{
    using Test = int (*)();
    static const struct
    {
        const char* mode;
        Test run;
    } kTests[] = {{"--add", muyo_llm::RunElementwiseAdd}, {"--matvec", muyo_llm::RunMatVec},
                  {"--rmsnorm", muyo_llm::RunRmsNorm},     {"--rope", muyo_llm::RunRope},
                  {"--swiglu", muyo_llm::RunSwiglu},       {"--getrows", muyo_llm::RunGetRows},
                  {"--argmax", muyo_llm::RunArgmax},       {"--softmax", muyo_llm::RunSoftMax},
                  {"--attention", muyo_llm::RunAttention}, {"--kvcache", muyo_llm::RunKvCache}};
    if (mode == nullptr)
    {
        return MUYO_E_NULL;
    }
    const bool all = std::strcmp(mode, "--smoke") == 0;
    int failures = 0;
    bool known = false;
    for (const auto& test : kTests)
    {
        if (all || std::strcmp(mode, test.mode) == 0)
        {
            known = true;
            failures += test.run() != 0 ? 1 : 0;
        }
    }
    if (!known)
    {
        return MUYO_E_RANGE;
    }
    return failures == 0 ? 0 : 1;
}
