// The streaming floor of a decode step: a chain of kernels that only read bytes.
//
// Measurement infrastructure for bench.py (libmuyo_floor.so, not part of the decode library):
// each launch of a chain streams its own region of one buffer with 16-byte non-temporal loads,
// grid-stride, four loads in flight per thread, and depends on no other launch's data. Replayed
// from one hipGraph, such a chain with a decode step's launch count and per-launch algorithmic
// bytes is what the step would cost if every kernel did nothing but read its operands: the
// bound that kernel boundaries and HBM set together, below which no kernel-per-phase decoder
// can go.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

namespace
{
constexpr int kThreads = 512;
constexpr int kInFlight = 4;
constexpr uint32_t kSinkWords = 1u << 16;

typedef unsigned int uint4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void StreamKernel(const uint4v* __restrict__ src, uint64_t n16,
                                                         uint32_t* __restrict__ sink)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    uint32_t acc = 0;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16; i += kInFlight * stride)
    {
        uint4v v[kInFlight];
#pragma unroll
        for (int k = 0; k < kInFlight; ++k)
        {
            const uint64_t j = i + k * stride;
            v[k] = j < n16 ? __builtin_nontemporal_load(src + j) : uint4v{0, 0, 0, 0};
        }
#pragma unroll
        for (int k = 0; k < kInFlight; ++k)
        {
            acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    // Practically never taken; keeps the loads.
    if (acc == 0x9E3779B9u)
    {
        sink[blockIdx.x] = acc;
    }
}

int Fail(hipError_t status) { return status == hipSuccess ? 0 : static_cast<int>(status); }
}  // namespace

/* Times a hipGraph chain of `launches` streaming kernels: launch i reads bytes[i] (rounded up to
 * 16) from its own 256-byte-aligned region of one buffer, on min(CUs * blocks_per_cu,
 * ceil(bytes / 8 KiB)) workgroups of 512 threads. Returns 0 and the median milliseconds per chain
 * over `reps` replays (after two warm-up replays), or a hipError_t. */
extern "C" int muyo_floor_chain(const uint64_t* bytes, uint32_t launches, uint32_t blocks_per_cu, uint32_t reps,
                                double* ms_out)
{
    if (bytes == nullptr || ms_out == nullptr || launches == 0 || blocks_per_cu == 0 || blocks_per_cu > 8 ||
        reps == 0)
    {
        return static_cast<int>(hipErrorInvalidValue);
    }
    int device = 0;
    int cus = 0;
    hipError_t st = hipGetDevice(&device);
    if (st == hipSuccess)
    {
        st = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    }
    if (st != hipSuccess || cus <= 0)
    {
        return Fail(st != hipSuccess ? st : hipErrorInvalidDevice);
    }
    std::vector<uint64_t> offset(launches);
    uint64_t total = 0;
    for (uint32_t i = 0; i < launches; ++i)
    {
        offset[i] = total;
        total += (bytes[i] + 255) / 256 * 256;
    }
    char* buffer = nullptr;
    uint32_t* sink = nullptr;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<hipEvent_t> events(2 * (reps + 2), nullptr);
    std::vector<float> times;
    st = hipMalloc(reinterpret_cast<void**>(&buffer), std::max<uint64_t>(total, 256));
    if (st == hipSuccess)
    {
        st = hipMalloc(reinterpret_cast<void**>(&sink), kSinkWords * sizeof(uint32_t));
    }
    if (st == hipSuccess)
    {
        st = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    }
    if (st == hipSuccess)
    {
        st = hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed);
    }
    if (st == hipSuccess)
    {
        for (uint32_t i = 0; i < launches; ++i)
        {
            const uint64_t n16 = (bytes[i] + 15) / 16;
            const uint64_t wanted = std::max<uint64_t>(1, (n16 + kThreads - 1) / kThreads);
            const uint32_t blocks = static_cast<uint32_t>(
                std::min<uint64_t>({wanted, static_cast<uint64_t>(cus) * blocks_per_cu, kSinkWords}));
            hipLaunchKernelGGL(StreamKernel, dim3(blocks), dim3(kThreads), 0, stream,
                               reinterpret_cast<const uint4v*>(buffer + offset[i]), n16, sink);
        }
        const hipError_t launched = hipGetLastError();
        st = hipStreamEndCapture(stream, &graph);
        if (st == hipSuccess)
        {
            st = launched;
        }
    }
    if (st == hipSuccess)
    {
        st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    }
    for (size_t e = 0; e < events.size() && st == hipSuccess; ++e)
    {
        st = hipEventCreate(&events[e]);
    }
    for (uint32_t r = 0; r < reps + 2 && st == hipSuccess; ++r)
    {
        st = hipEventRecord(events[2 * r], stream);
        if (st == hipSuccess)
        {
            st = hipGraphLaunch(exec, stream);
        }
        if (st == hipSuccess)
        {
            st = hipEventRecord(events[2 * r + 1], stream);
        }
    }
    if (st == hipSuccess)
    {
        st = hipStreamSynchronize(stream);
    }
    for (uint32_t r = 2; r < reps + 2 && st == hipSuccess; ++r)
    {
        float ms = 0.0F;
        st = hipEventElapsedTime(&ms, events[2 * r], events[2 * r + 1]);
        times.push_back(ms);
    }
    if (st == hipSuccess)
    {
        std::sort(times.begin(), times.end());
        *ms_out = times[times.size() / 2];
    }
    for (hipEvent_t e : events)
    {
        if (e != nullptr)
        {
            (void)hipEventDestroy(e);
        }
    }
    if (exec != nullptr)
    {
        (void)hipGraphExecDestroy(exec);
    }
    if (graph != nullptr)
    {
        (void)hipGraphDestroy(graph);
    }
    if (stream != nullptr)
    {
        (void)hipStreamSynchronize(stream);
        (void)hipStreamDestroy(stream);
    }
    (void)hipFree(buffer);
    (void)hipFree(sink);
    return Fail(st);
}
