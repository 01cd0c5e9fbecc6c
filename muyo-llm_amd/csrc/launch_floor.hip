// What a kernel boundary costs on this GPU, measured four ways (bench.py --launch-floor).
//
// Measurement infrastructure, not part of the decode library. Built twice by the Makefile: as the
// executable ../launch_floor (host code plus the kernels for HIP launches) and, device code only,
// as the raw code object ../launch_floor_kernels.co, which the executable loads through the HSA
// runtime to dispatch the same kernels from its own AQL queue with chosen fence scopes.
//
//   graph_empty   chains of empty kernels replayed from one hipGraph: graphs of 122 and of 1952
//                 kernels, microseconds per kernel (the difference is what a graph launch adds);
//   aql_empty     2000 empty kernels written straight into an AQL queue, each packet's acquire
//                 and release fences at system, agent or no scope (and without the barrier bit):
//                 the command processor's cost per dispatch, and what the cache fences add;
//   aql_stream    a launch sequence read by pure-stream kernels (each launch reads its bytes from
//                 its own region), packets with agent-scope fences (what hipGraph replay uses) and
//                 with none;
//   aql_handoff   the same sequence where every launch also reads an 896-float activation that
//                 the previous launch wrote (every workgroup reads all of it) and writes the next
//                 one, in five coherence schemes: plain loads and stores with agent fences; plain
//                 with no fences (stale lines: counted wrong elements); device-scope loads and
//                 stores with no fences; device-scope loads, no acquire fence, agent release;
//                 device-scope stores, agent acquire, no release fence.
//
// Input (stdin): the launch sequence's byte counts, one per line. Output (stdout): one JSON object.
// Every wait is bounded (10 s); the process exits non-zero on a timeout or any runtime error.
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

typedef unsigned int Lfu4 __attribute__((ext_vector_type(4)));

constexpr int kStreamThreads = 512;

extern "C" __global__ void lf_empty(int* p)
{
    (void)p;
}

/// Reads n16 16-byte chunks grid-stride, four non-temporal loads in flight per thread (stride is
/// the grid's thread count, passed in so the kernel needs no implicit arguments).
__device__ __forceinline__ uint32_t LfStream(const Lfu4* __restrict__ src, uint64_t n16, uint64_t stride)
{
    uint32_t acc = 0;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kStreamThreads + threadIdx.x; i < n16; i += 4 * stride)
    {
        Lfu4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const uint64_t j = i + k * stride;
            v[k] = j < n16 ? __builtin_nontemporal_load(src + j) : Lfu4{0, 0, 0, 0};
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    return acc;
}

extern "C" __global__ __launch_bounds__(kStreamThreads) void lf_stream(const Lfu4* __restrict__ src, uint64_t n16,
                                                                      uint64_t stride, uint32_t* __restrict__ sink)
{
    const uint32_t acc = LfStream(src, n16, stride);
    if (acc == 0x9E3779B9u)  // practically never: keeps the loads
    {
        sink[blockIdx.x] = acc;
    }
}

/// One link of a hand-off chain: the stream, then every element of `in` (as a GEMV stages its
/// activation), then out[i] = in[(i + 1) % n] + 1 with the outputs spread over the workgroups.
/// kDeviceLoads / kDeviceStores: agent-scope (device-coherent) accesses instead of plain ones.
template <bool kDeviceLoads, bool kDeviceStores>
__device__ __forceinline__ void LfHandoff(const Lfu4* __restrict__ src, uint64_t n16, uint64_t stride,
                                          const float* in, float* out, uint32_t n, uint32_t* __restrict__ sink)
{
    auto load = [&](uint32_t i) {
        return kDeviceLoads ? __hip_atomic_load(in + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : in[i];
    };
    const uint32_t acc = LfStream(src, n16, stride);
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += kStreamThreads)
    {
        s += load(i);
    }
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kStreamThreads + threadIdx.x; i < n; i += stride)
    {
        const float v = load(static_cast<uint32_t>((i + 1) % n)) + 1.0f;
        if constexpr (kDeviceStores)
        {
            __hip_atomic_store(out + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        else
        {
            out[i] = v;
        }
    }
    if (acc == 0x9E3779B9u || s == -1.5f)
    {
        sink[blockIdx.x] = acc;
    }
}

#define MUYO_LF_HANDOFF(name, loads, stores)                                                            \
    extern "C" __global__ __launch_bounds__(kStreamThreads) void name(                                 \
        const Lfu4* __restrict__ src, uint64_t n16, uint64_t stride, const float* in, float* out,       \
        uint32_t n, uint32_t* __restrict__ sink)                                                        \
    {                                                                                                   \
        LfHandoff<loads, stores>(src, n16, stride, in, out, n, sink);                                   \
    }
MUYO_LF_HANDOFF(lf_handoff_plain, false, false)
MUYO_LF_HANDOFF(lf_handoff_device, true, true)
MUYO_LF_HANDOFF(lf_handoff_device_loads, true, false)
MUYO_LF_HANDOFF(lf_handoff_device_stores, false, true)
#undef MUYO_LF_HANDOFF

#ifndef __HIP_DEVICE_COMPILE__

namespace
{
constexpr uint32_t kActivation = 896;  // floats handed from launch to launch

[[noreturn]] void Die(const char* what, int code)
{
    std::fprintf(stderr, "launch_floor: %s (%d)\n", what, code);
    std::exit(2);
}

void Hip(hipError_t status, const char* what)
{
    if (status != hipSuccess)
    {
        std::fprintf(stderr, "launch_floor: %s: %s\n", what, hipGetErrorString(status));
        std::exit(2);
    }
}

void Hsa(hsa_status_t status, const char* what)
{
    if (status != HSA_STATUS_SUCCESS && status != HSA_STATUS_INFO_BREAK)
    {
        const char* msg = nullptr;
        hsa_status_string(status, &msg);
        std::fprintf(stderr, "launch_floor: %s: %s\n", what, msg != nullptr ? msg : "?");
        std::exit(2);
    }
}

double Median(std::vector<double> v)
{
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

/// Microseconds per kernel of hipGraph chains of `perGraph` empty kernels (256 workgroups of 64),
/// `total` kernels in all per timing, median of 5.
double GraphEmpty(int perGraph, int total)
{
    hipStream_t s = nullptr;
    Hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    Hip(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "capture");
    for (int i = 0; i < perGraph; ++i)
    {
        hipLaunchKernelGGL(lf_empty, dim3(256), dim3(64), 0, s, nullptr);
    }
    Hip(hipStreamEndCapture(s, &graph), "end capture");
    Hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
    hipEvent_t b = nullptr;
    hipEvent_t e = nullptr;
    Hip(hipEventCreate(&b), "event");
    Hip(hipEventCreate(&e), "event");
    for (int w = 0; w < 3; ++w)
    {
        Hip(hipGraphLaunch(exec, s), "graph launch");
    }
    std::vector<double> us;
    for (int t = 0; t < 5; ++t)
    {
        Hip(hipEventRecord(b, s), "record");
        for (int r = 0; r < total / perGraph; ++r)
        {
            Hip(hipGraphLaunch(exec, s), "graph launch");
        }
        Hip(hipEventRecord(e, s), "record");
        Hip(hipStreamSynchronize(s), "sync");
        float ms = 0.0F;
        Hip(hipEventElapsedTime(&ms, b, e), "elapsed");
        us.push_back(1000.0 * ms / (total / perGraph * perGraph));
    }
    Hip(hipEventDestroy(b), "event");
    Hip(hipEventDestroy(e), "event");
    Hip(hipGraphExecDestroy(exec), "graph");
    Hip(hipGraphDestroy(graph), "graph");
    Hip(hipStreamDestroy(s), "stream");
    return Median(us);
}

struct Kernel
{
    uint64_t object = 0;
    uint32_t group = 0;
    uint32_t priv = 0;
};

struct Launch
{
    const Kernel* kernel;
    void* kernarg;
    uint32_t workgroups;
    uint32_t threads;
};

/// The HSA side: the first GPU agent (the one HIP's device 0 is, on a one-GPU box), its
/// coarse-grained device pool, the kernarg region for host-written staging, a queue and the code
/// object's kernels.
struct Aql
{
    hsa_agent_t gpu{};
    bool haveGpu = false;
    hsa_region_t kernarg{};
    bool haveKernarg = false;
    hsa_amd_memory_pool_t pool{};
    bool havePool = false;
    hsa_queue_t* queue = nullptr;
    hsa_signal_t done{};
    hsa_executable_t exec{};
    hsa_code_object_reader_t reader{};
    uint32_t cus = 0;

    Kernel Get(const char* name)
    {
        hsa_executable_symbol_t sym;
        Hsa(hsa_executable_get_symbol_by_name(exec, name, &gpu, &sym), name);
        Kernel k;
        Hsa(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &k.object), name);
        Hsa(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, &k.group), name);
        Hsa(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, &k.priv), name);
        return k;
    }

    void* Device(size_t bytes)
    {
        void* p = nullptr;
        Hsa(hsa_amd_memory_pool_allocate(pool, bytes, 0, &p), "device allocation");
        return p;
    }

    void* Staging(size_t bytes)
    {
        void* p = nullptr;
        Hsa(hsa_memory_allocate(kernarg, bytes, &p), "staging allocation");
        return p;
    }

    /// Writes the launches as one run of dispatch packets: the first acquires at system scope
    /// (after whatever ran before), the last releases at system scope and signals completion,
    /// the others carry (barrier, acq, rel). Returns host microseconds from the first packet
    /// write to the completion signal.
    double Run(const std::vector<Launch>& launches, bool barrier, int acq, int rel)
    {
        const uint32_t size = queue->size;
        const uint32_t count = static_cast<uint32_t>(launches.size());
        if (count == 0 || count > size - 1)
        {
            Die("launch count does not fit the queue", static_cast<int>(count));
        }
        hsa_signal_store_relaxed(done, 1);
        const auto t0 = std::chrono::steady_clock::now();
        const auto deadline = t0 + std::chrono::seconds(10);
        const uint64_t first = hsa_queue_add_write_index_scacq_screl(queue, count);
        while (first + count - hsa_queue_load_read_index_scacquire(queue) > size)
        {
            if (std::chrono::steady_clock::now() > deadline)
            {
                Die("timeout waiting for queue space", 0);
            }
        }
        auto* packets = static_cast<hsa_kernel_dispatch_packet_t*>(queue->base_address);
        for (uint32_t i = 0; i < count; ++i)
        {
            const Launch& l = launches[i];
            hsa_kernel_dispatch_packet_t* p = &packets[(first + i) & (size - 1)];
            std::memset(reinterpret_cast<uint8_t*>(p) + 4, 0, sizeof(*p) - 4);
            p->workgroup_size_x = static_cast<uint16_t>(l.threads);
            p->workgroup_size_y = 1;
            p->workgroup_size_z = 1;
            p->grid_size_x = l.workgroups * l.threads;
            p->grid_size_y = 1;
            p->grid_size_z = 1;
            p->private_segment_size = l.kernel->priv;
            p->group_segment_size = l.kernel->group;
            p->kernel_object = l.kernel->object;
            p->kernarg_address = l.kernarg;
            const bool last = i + 1 == count;
            p->completion_signal = last ? done : hsa_signal_t{0};
            const int a = i == 0 ? HSA_FENCE_SCOPE_SYSTEM : acq;
            const int r = last ? HSA_FENCE_SCOPE_SYSTEM : rel;
            const uint32_t header = (HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                                    ((barrier || last ? 1u : 0u) << HSA_PACKET_HEADER_BARRIER) |
                                    (static_cast<uint32_t>(a) << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                                    (static_cast<uint32_t>(r) << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE);
            const uint32_t setup = 1u << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
            __atomic_store_n(reinterpret_cast<uint32_t*>(p), header | (setup << 16), __ATOMIC_RELEASE);
        }
        hsa_signal_store_screlease(queue->doorbell_signal, first + count - 1);
        while (hsa_signal_load_scacquire(done) != 0)
        {
            if (std::chrono::steady_clock::now() > deadline)
            {
                Die("timeout waiting for a chain", 0);
            }
        }
        return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    }
};

hsa_status_t FindGpu(hsa_agent_t agent, void* data)
{
    auto* q = static_cast<Aql*>(data);
    hsa_device_type_t type;
    Hsa(hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type), "agent info");
    if (type == HSA_DEVICE_TYPE_GPU && !q->haveGpu)
    {
        q->gpu = agent;
        q->haveGpu = true;
        return HSA_STATUS_INFO_BREAK;
    }
    return HSA_STATUS_SUCCESS;
}

hsa_status_t FindKernarg(hsa_region_t region, void* data)
{
    auto* q = static_cast<Aql*>(data);
    hsa_region_segment_t seg;
    Hsa(hsa_region_get_info(region, HSA_REGION_INFO_SEGMENT, &seg), "region info");
    uint32_t flags = 0;
    if (seg == HSA_REGION_SEGMENT_GLOBAL)
    {
        Hsa(hsa_region_get_info(region, HSA_REGION_INFO_GLOBAL_FLAGS, &flags), "region flags");
    }
    if ((flags & HSA_REGION_GLOBAL_FLAG_KERNARG) != 0 && !q->haveKernarg)
    {
        q->kernarg = region;
        q->haveKernarg = true;
        return HSA_STATUS_INFO_BREAK;
    }
    return HSA_STATUS_SUCCESS;
}

hsa_status_t FindPool(hsa_amd_memory_pool_t pool, void* data)
{
    auto* q = static_cast<Aql*>(data);
    hsa_amd_segment_t seg;
    Hsa(hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg), "pool info");
    uint32_t flags = 0;
    if (seg == HSA_AMD_SEGMENT_GLOBAL)
    {
        Hsa(hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags), "pool flags");
    }
    if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_COARSE_GRAINED) != 0 && !q->havePool)
    {
        q->pool = pool;
        q->havePool = true;
        return HSA_STATUS_INFO_BREAK;
    }
    return HSA_STATUS_SUCCESS;
}

void OpenAql(Aql& q, const std::string& codeObject)
{
    Hsa(hsa_init(), "hsa_init");
    Hsa(hsa_iterate_agents(FindGpu, &q), "agents");
    if (!q.haveGpu)
    {
        Die("no GPU agent", 0);
    }
    Hsa(hsa_agent_iterate_regions(q.gpu, FindKernarg, &q), "regions");
    Hsa(hsa_amd_agent_iterate_memory_pools(q.gpu, FindPool, &q), "pools");
    if (!q.haveKernarg || !q.havePool)
    {
        Die("no kernarg region or device pool", 0);
    }
    Hsa(hsa_agent_get_info(q.gpu, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_COMPUTE_UNIT_COUNT), &q.cus),
        "compute units");
    std::ifstream f(codeObject, std::ios::binary);
    if (!f)
    {
        Die("cannot open the kernels' code object", 0);
    }
    const std::string blob((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    Hsa(hsa_code_object_reader_create_from_memory(blob.data(), blob.size(), &q.reader), "code object");
    Hsa(hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr, &q.exec),
        "executable");
    Hsa(hsa_executable_load_agent_code_object(q.exec, q.gpu, q.reader, nullptr, nullptr), "load code object");
    Hsa(hsa_executable_freeze(q.exec, nullptr), "freeze");
    Hsa(hsa_queue_create(q.gpu, 4096, HSA_QUEUE_TYPE_SINGLE, nullptr, nullptr, UINT32_MAX, UINT32_MAX, &q.queue),
        "queue");
    Hsa(hsa_signal_create(1, 0, nullptr, &q.done), "signal");
}

void CloseAql(Aql& q)
{
    Hsa(hsa_queue_destroy(q.queue), "queue");
    Hsa(hsa_signal_destroy(q.done), "signal");
    Hsa(hsa_executable_destroy(q.exec), "executable");
    Hsa(hsa_code_object_reader_destroy(q.reader), "code object");
    Hsa(hsa_shut_down(), "hsa_shut_down");
}

const char* kScope[3] = {"none", "agent", "system"};

/// Per-kernel microseconds of 2000 empty kernels (256 workgroups of 64 threads), the fixed cost
/// of one packet taken out by a one-packet run; median of 5.
double AqlEmpty(Aql& q, const Kernel& k, void* args, bool barrier, int scope)
{
    const uint32_t chain = 2000;
    std::vector<Launch> one{Launch{&k, args, 256, 64}};
    std::vector<Launch> many(chain, Launch{&k, args, 256, 64});
    std::vector<double> us;
    for (int rep = 0; rep < 5; ++rep)
    {
        const double t1 = q.Run(one, barrier, scope, scope);
        const double tn = q.Run(many, barrier, scope, scope);
        us.push_back((tn - t1) / (chain - 1));
    }
    return Median(us);
}

struct Chain
{
    char* buffer = nullptr;
    uint32_t* sink = nullptr;
    float* act[2] = {nullptr, nullptr};
    char* args = nullptr;
    char* staging = nullptr;
    size_t argBytes = 0;
    std::vector<Launch> launches;
};

/// Kernargs of launch i: (src, n16, stride, act[i & 1], act[(i + 1) & 1], n, sink); the stream
/// kernel reads the first three and sink through the same layout's prefix and last field.
Chain MakeChain(Aql& q, const std::vector<uint64_t>& bytes, const Kernel& k, bool handoff)
{
    Chain c;
    std::vector<uint64_t> offset(bytes.size());
    uint64_t total = 0;
    for (size_t i = 0; i < bytes.size(); ++i)
    {
        offset[i] = total;
        total += (bytes[i] + 255) / 256 * 256;
    }
    c.buffer = static_cast<char*>(q.Device(total));
    c.sink = static_cast<uint32_t*>(q.Device(4 * 65536));
    c.act[0] = static_cast<float*>(q.Device(4096));
    c.act[1] = static_cast<float*>(q.Device(4096));
    constexpr size_t kArgStride = 64;
    c.argBytes = bytes.size() * kArgStride;
    c.args = static_cast<char*>(q.Device(c.argBytes));
    c.staging = static_cast<char*>(q.Staging(std::max<size_t>(c.argBytes, 4096)));
    std::memset(c.staging, 0, c.argBytes);
    for (size_t i = 0; i < bytes.size(); ++i)
    {
        const uint64_t n16 = (bytes[i] + 15) / 16;
        const uint64_t wanted = std::max<uint64_t>(2, (n16 + kStreamThreads - 1) / kStreamThreads);
        const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>(wanted, 3ull * q.cus));  // 3 per CU
        const uint64_t stride = static_cast<uint64_t>(blocks) * kStreamThreads;
        char* a = c.staging + i * kArgStride;
        const void* src = c.buffer + offset[i];
        std::memcpy(a + 0, &src, 8);
        std::memcpy(a + 8, &n16, 8);
        std::memcpy(a + 16, &stride, 8);
        if (handoff)
        {
            const float* in = c.act[i & 1];
            float* out = c.act[(i + 1) & 1];
            const uint32_t n = kActivation;
            std::memcpy(a + 24, &in, 8);
            std::memcpy(a + 32, &out, 8);
            std::memcpy(a + 40, &n, 4);
            std::memcpy(a + 48, &c.sink, 8);
        }
        else
        {
            std::memcpy(a + 24, &c.sink, 8);
        }
        c.launches.push_back(Launch{&k, c.args + i * kArgStride, blocks, kStreamThreads});
    }
    Hsa(hsa_memory_copy(c.args, c.staging, c.argBytes), "kernarg upload");
    return c;
}

void FreeChain(Chain& c)
{
    Hsa(hsa_amd_memory_pool_free(c.buffer), "free");
    Hsa(hsa_amd_memory_pool_free(c.sink), "free");
    Hsa(hsa_amd_memory_pool_free(c.act[0]), "free");
    Hsa(hsa_amd_memory_pool_free(c.act[1]), "free");
    Hsa(hsa_amd_memory_pool_free(c.args), "free");
    Hsa(hsa_memory_free(c.staging), "free");
}

/// Median microseconds of 12 runs of a chain, and (hand-off chains) the elements that did not end
/// at the launch count.
double RunChain(Aql& q, Chain& c, bool handoff, int acq, int rel, long* wrong)
{
    std::vector<double> us;
    long bad = 0;
    auto* host = reinterpret_cast<float*>(c.staging);  // the kernargs are uploaded: free to reuse
    for (int rep = 0; rep < 12; ++rep)
    {
        if (handoff)
        {
            std::memset(host, 0, 4096);
            Hsa(hsa_memory_copy(c.act[0], host, 4096), "reset");
            Hsa(hsa_memory_copy(c.act[1], host, 4096), "reset");
        }
        us.push_back(q.Run(c.launches, true, acq, rel));
        if (handoff)
        {
            Hsa(hsa_memory_copy(host, c.act[c.launches.size() & 1], 4096), "read back");
            for (uint32_t e = 0; e < kActivation; ++e)
            {
                bad += host[e] != static_cast<float>(c.launches.size());
            }
        }
    }
    if (wrong != nullptr)
    {
        *wrong = bad;
    }
    return Median(us);
}
}  // namespace

int main(int argc, char** argv)
{
    const std::string codeObject = argc > 1 ? argv[1] : "launch_floor_kernels.co";
    std::vector<uint64_t> bytes;
    unsigned long long v = 0;
    while (std::scanf("%llu", &v) == 1)
    {
        bytes.push_back(v);
    }
    if (bytes.empty() || bytes.size() > 4000)
    {
        Die("expected 1..4000 byte counts on stdin", static_cast<int>(bytes.size()));
    }
    Hip(hipSetDevice(0), "device");
    std::printf("{\"graph_empty_us_per_kernel\": {\"122\": %.3f, \"1952\": %.3f}", GraphEmpty(122, 122 * 256),
                GraphEmpty(1952, 1952 * 16));
    std::fflush(stdout);

    Aql q;
    OpenAql(q, codeObject);
    const Kernel empty = q.Get("lf_empty.kd");
    void* emptyArgs = q.Device(256);
    std::printf(", \"aql_empty_us_per_kernel\": {");
    for (int scope : {2, 1, 0})
    {
        std::printf("\"%s\": %.3f, ", kScope[scope], AqlEmpty(q, empty, emptyArgs, true, scope));
    }
    std::printf("\"none_no_barrier\": %.3f}", AqlEmpty(q, empty, emptyArgs, false, 0));
    std::fflush(stdout);

    const Kernel stream = q.Get("lf_stream.kd");
    Chain sc = MakeChain(q, bytes, stream, false);
    std::printf(", \"launches\": %zu, \"aql_stream_us\": {\"agent\": %.1f, \"none\": %.1f, \"agent_again\": %.1f, "
                "\"none_again\": %.1f}",
                bytes.size(), RunChain(q, sc, false, 1, 1, nullptr), RunChain(q, sc, false, 0, 0, nullptr),
                RunChain(q, sc, false, 1, 1, nullptr), RunChain(q, sc, false, 0, 0, nullptr));
    FreeChain(sc);
    std::fflush(stdout);

    struct Mode
    {
        const char* name;
        const char* kernel;
        int acq;
        int rel;
    };
    const Mode modes[] = {
        {"plain_agent_fences", "lf_handoff_plain.kd", 1, 1},
        {"plain_no_fences", "lf_handoff_plain.kd", 0, 0},
        {"device_scope_no_fences", "lf_handoff_device.kd", 0, 0},
        {"device_loads_release_only", "lf_handoff_device_loads.kd", 0, 1},
        {"device_stores_acquire_only", "lf_handoff_device_stores.kd", 1, 0},
    };
    std::printf(", \"aql_handoff\": {");
    for (size_t m = 0; m < sizeof(modes) / sizeof(modes[0]); ++m)
    {
        const Kernel k = q.Get(modes[m].kernel);
        Chain hc = MakeChain(q, bytes, k, true);
        long wrong = 0;
        const double us = RunChain(q, hc, true, modes[m].acq, modes[m].rel, &wrong);
        std::printf("%s\"%s\": {\"us\": %.1f, \"wrong_elements_of_%u_x_12\": %ld}", m == 0 ? "" : ", ",
                    modes[m].name, us, kActivation, wrong);
        std::fflush(stdout);
        FreeChain(hc);
    }
    std::printf("}}\n");
    Hsa(hsa_amd_memory_pool_free(emptyArgs), "free");
    CloseAql(q);
    return 0;
}

#endif  // __HIP_DEVICE_COMPILE__
