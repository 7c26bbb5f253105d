// evk core over HIP: buffers, stream-ordered commands, submissions, timestamps.
//
// Replaces the Vulkan runtime behind /root/reference/evk.h for the AI path
// (evk_vulkan.cpp: buffer creation :1715-1732 with deferred deletion
// :237-243, command buffers and submission :1990-2060, timestamps :1011).
// One HIP stream carries every command in issue order; a submission is an
// event on that stream.
#include <evk.h>
#include <evkhip.h>

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <deque>
#include <string>
#include <vector>

namespace evk {
namespace {

[[noreturn]] void die(const char* what, hipError_t e) {
    std::fprintf(stderr, "evk: %s failed: %s\n", what, hipGetErrorString(e));
    std::abort();
}
#define EVK_CHECK(call)                          \
    do {                                         \
        hipError_t e_ = (call);                  \
        if (e_ != hipSuccess) die(#call, e_);    \
    } while (0)

[[noreturn]] void misuse(const char* msg) {
    std::fprintf(stderr, "evk: %s\n", msg);
    std::abort();
}

struct BufferRes final : Resource {
    void* dev = nullptr;   // device address (device memory, or the mapping of pinned host memory)
    void* host = nullptr;  // pinned host address, nullptr for device memory
    uint64_t size = 0;
    MemoryType type = MemoryType::GPU;
    std::string name;
    ~BufferRes() override;
};

struct PendingFree {
    hipEvent_t after;  // the stream point after which the memory is unused
    void* dev;
    void* host;
};

struct Staging {
    void* ptr;
    uint64_t size;
    hipEvent_t done;  // last copy out of this chunk
    bool used;
};

struct TimestampPair {
    const char* name;
    hipEvent_t begin, end;
};

struct Submission {
    uint64_t index;
    hipEvent_t done;
    std::vector<TimestampPair> stamps;
};

struct Runtime {
    bool up = false;
    EvkDesc desc;
    Features features;
    hipStream_t stream = nullptr;
    Cmd cmd;
    bool open = false;
    uint64_t submitted = 0;  // index of the latest submission
    uint64_t completed = 0;  // every submission <= completed has finished
    std::deque<Submission> inflight;
    std::vector<TimestampPair> stamps;  // of the open command
    std::vector<TimestampEntry> last_stamps;
    std::vector<PendingFree> frees;
    std::vector<Staging> staging;
    uint64_t live_allocs = 0, live_bytes = 0;
};

Runtime& rt() {
    static Runtime r;
    return r;
}

hipEvent_t new_event(bool timing) {
    hipEvent_t e;
    EVK_CHECK(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming));
    return e;
}

void release_memory(void* dev, void* host) {
    if (host) {
        EVK_CHECK(hipHostFree(host));
    } else if (dev) {
        EVK_CHECK(hipFree(dev));
    }
}

// Frees every deferred allocation whose stream point has been reached.
void reclaim() {
    Runtime& r = rt();
    size_t keep = 0;
    for (size_t i = 0; i < r.frees.size(); ++i) {
        PendingFree& f = r.frees[i];
        hipError_t q = hipEventQuery(f.after);
        if (q == hipSuccess) {
            release_memory(f.dev, f.host);
            EVK_CHECK(hipEventDestroy(f.after));
        } else if (q == hipErrorNotReady) {
            r.frees[keep++] = f;
        } else {
            die("hipEventQuery", q);
        }
    }
    r.frees.resize(keep);
}

BufferRes::~BufferRes() {
    Runtime& r = rt();
    if (r.up) {
        // the stream may still read or write this memory: free it once the
        // stream has passed everything enqueued so far
        hipEvent_t e = new_event(false);
        EVK_CHECK(hipEventRecord(e, r.stream));
        r.frees.push_back({e, dev, host});
        r.live_allocs -= 1;
        r.live_bytes -= size;
    } else {
        release_memory(dev, host);
    }
}

void require_up() {
    if (!rt().up) misuse("the runtime is not initialized (call evk::InitializeEVK or evk::ai::initialize first)");
}

// A pinned staging chunk of at least `size` bytes whose previous copy has completed.
Staging& staging_for(uint64_t size) {
    Runtime& r = rt();
    Staging* best = nullptr;
    for (Staging& s : r.staging) {
        if (s.size < size) continue;
        if (s.used) {
            hipError_t q = hipEventQuery(s.done);
            if (q == hipErrorNotReady) continue;
            if (q != hipSuccess) die("hipEventQuery", q);
            s.used = false;
        }
        if (!best || s.size < best->size) best = &s;
    }
    if (best) return *best;
    uint64_t cap = 1ull << 20;
    while (cap < size) cap <<= 1;
    Staging s{nullptr, cap, new_event(false), false};
    EVK_CHECK(hipHostMalloc(&s.ptr, cap, hipHostMallocDefault));
    r.staging.push_back(s);
    return r.staging.back();
}

BufferRes* res_of(Buffer& b) {
    if (!b.res) misuse("null buffer");
    return static_cast<BufferRes*>(b.res);
}

void finish_submission(Submission& s) {
    Runtime& r = rt();
    if (!s.stamps.empty()) {
        // every entry is measured from the first begin event: destroy the
        // events only after all of them have been read
        r.last_stamps.clear();
        const hipEvent_t origin = s.stamps.front().begin;
        for (const TimestampPair& p : s.stamps) {
            float t0 = 0.0f, t1 = 0.0f;
            EVK_CHECK(hipEventElapsedTime(&t0, origin, p.begin));
            EVK_CHECK(hipEventElapsedTime(&t1, origin, p.end));
            r.last_stamps.push_back({double(t0), double(t1), p.name});
        }
        for (const TimestampPair& p : s.stamps) {
            EVK_CHECK(hipEventDestroy(p.begin));
            EVK_CHECK(hipEventDestroy(p.end));
        }
    }
    EVK_CHECK(hipEventDestroy(s.done));
}

}  // namespace

void Resource::decRef() {
    if (--refCount == 0) delete this;
}

void* Buffer::GetPtr() {
    return res ? static_cast<BufferRes*>(res)->host : nullptr;
}
uint64_t Buffer::GetReference() {
    return res ? reinterpret_cast<uint64_t>(static_cast<BufferRes*>(res)->dev) : 0;
}
uint64_t Buffer::GetSize() {
    return res ? static_cast<BufferRes*>(res)->size : 0;
}

Buffer CreateBuffer(const BufferDesc& desc) {
    require_up();
    reclaim();
    Runtime& r = rt();
    auto* b = new BufferRes();
    b->size = desc.size;
    b->type = desc.memoryType;
    b->name = desc.name;
    const uint64_t bytes = desc.size ? desc.size : 1;  // zero-sized tensors still get an address
    if (desc.memoryType == MemoryType::GPU) {
        EVK_CHECK(hipMalloc(&b->dev, bytes));
    } else {
        EVK_CHECK(hipHostMalloc(&b->host, bytes, hipHostMallocMapped));
        EVK_CHECK(hipHostGetDevicePointer(&b->dev, b->host, 0));
    }
    r.live_allocs += 1;
    r.live_bytes += desc.size;
    return Buffer(b);
}

void WriteBuffer(Buffer& buffer, void* src, uint64_t size, uint64_t offset) {
    require_up();
    BufferRes* b = res_of(buffer);
    if (offset + size > b->size) misuse("WriteBuffer out of range");
    if (b->host) {
        EVK_CHECK(hipStreamSynchronize(rt().stream));
        std::memcpy(static_cast<char*>(b->host) + offset, src, size);
        return;
    }
    EVK_CHECK(hipMemcpyAsync(static_cast<char*>(b->dev) + offset, src, size, hipMemcpyHostToDevice, rt().stream));
    EVK_CHECK(hipStreamSynchronize(rt().stream));
}

void ReadBuffer(Buffer& buffer, void* dst, uint64_t size, uint64_t offset) {
    require_up();
    BufferRes* b = res_of(buffer);
    if (offset + size > b->size) misuse("ReadBuffer out of range");
    if (b->host) {
        EVK_CHECK(hipStreamSynchronize(rt().stream));
        std::memcpy(dst, static_cast<char*>(b->host) + offset, size);
        return;
    }
    EVK_CHECK(hipMemcpyAsync(dst, static_cast<char*>(b->dev) + offset, size, hipMemcpyDeviceToHost, rt().stream));
    EVK_CHECK(hipStreamSynchronize(rt().stream));
}

bool InitializeEVK(const EvkDesc& info) {
    Runtime& r = rt();
    if (r.up) return true;
    if (info.enableSwapchain) {
        std::fprintf(stderr, "evk: this library has no presentation engine (enableSwapchain)\n");
        return false;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || info.device < 0 || info.device >= n) {
        std::fprintf(stderr, "evk: HIP device %d not available (%d devices)\n", info.device, n);
        return false;
    }
    EVK_CHECK(hipSetDevice(info.device));
    hipDeviceProp_t prop;
    EVK_CHECK(hipGetDeviceProperties(&prop, info.device));
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
        std::fprintf(stderr, "evk: device %d is %s; this library is built for gfx950 (MI355X)\n", info.device,
                     prop.gcnArchName);
        return false;
    }
    // default priority: every stream of this library runs at the same priority
    EVK_CHECK(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
    r.desc = info;
    r.features = Features{};
    r.features.coopmat = true;
    r.features.timestamps = info.enableTimestamps;
    r.cmd._internal = &r;
    r.up = true;
    return true;
}

bool IsInitialized() {
    return rt().up;
}

void Shutdown() {
    Runtime& r = rt();
    if (!r.up) return;
    EVK_CHECK(hipStreamSynchronize(r.stream));
    for (Submission& s : r.inflight) finish_submission(s);
    r.inflight.clear();
    for (TimestampPair& p : r.stamps) {
        EVK_CHECK(hipEventDestroy(p.begin));
        EVK_CHECK(hipEventDestroy(p.end));
    }
    r.stamps.clear();
    reclaim();
    for (Staging& s : r.staging) {
        EVK_CHECK(hipHostFree(s.ptr));
        EVK_CHECK(hipEventDestroy(s.done));
    }
    r.staging.clear();
    EVK_CHECK(hipStreamDestroy(r.stream));
    r.stream = nullptr;
    r.open = false;
    r.up = false;  // buffers still alive are freed directly when they die
}

const Features& GetFeatures() {
    return rt().features;
}

MemoryBudget GetMemoryBudget() {
    require_up();
    MemoryBudget m{};
    size_t free_b = 0, total_b = 0;
    EVK_CHECK(hipMemGetInfo(&free_b, &total_b));
    m.heaps[0].allocationCount = uint32_t(rt().live_allocs);
    m.heaps[0].allocationBytes = rt().live_bytes;
    m.heaps[0].blockCount = uint32_t(rt().live_allocs);
    m.heaps[0].blockBytes = rt().live_bytes;
    m.heaps[0].usage = total_b - free_b;
    m.heaps[0].budget = total_b;
    return m;
}

const std::vector<TimestampEntry>& CmdTimestamps() {
    return rt().last_stamps;
}

void Cmd::barrier() {}

void Cmd::fill(Buffer dst, uint32_t data, uint64_t size, uint64_t offset) {
    BufferRes* b = res_of(dst);
    if (offset + size > b->size || (size & 3) || (offset & 3)) misuse("Cmd::fill: range must be 4-byte aligned and inside the buffer");
    // a fill kernel, not a memset: a captured graph then holds no memset node
    if (evkhip_fill(static_cast<char*>(b->dev) + offset, size, data, rt().stream) != 0)
        misuse(evkhip_last_error());
}

void Cmd::copy(Buffer& src, Buffer& dst, uint64_t size, uint64_t srcOffset, uint64_t dstOffset) {
    BufferRes* s = res_of(src);
    BufferRes* d = res_of(dst);
    if (srcOffset + size > s->size || dstOffset + size > d->size) misuse("Cmd::copy out of range");
    EVK_CHECK(hipMemcpyAsync(static_cast<char*>(d->dev) + dstOffset, static_cast<char*>(s->dev) + srcOffset, size,
                             hipMemcpyDefault, rt().stream));
}

void Cmd::copy(void* src, Buffer& dst, uint64_t size, uint64_t dstOffset) {
    BufferRes* d = res_of(dst);
    if (dstOffset + size > d->size) misuse("Cmd::copy out of range");
    if (size == 0) return;
    Staging& st = staging_for(size);
    std::memcpy(st.ptr, src, size);
    EVK_CHECK(hipMemcpyAsync(static_cast<char*>(d->dev) + dstOffset, st.ptr, size, hipMemcpyHostToDevice, rt().stream));
    EVK_CHECK(hipEventRecord(st.done, rt().stream));
    st.used = true;
}

void Cmd::update(Buffer& dst, uint64_t dstOffset, uint64_t size, void* src) {
    copy(src, dst, size, dstOffset);
}

int Cmd::beginTimestamp(const char* name) {
    Runtime& r = rt();
    if (!r.desc.enableTimestamps) return -1;
    TimestampPair p{name, new_event(true), new_event(true)};
    EVK_CHECK(hipEventRecord(p.begin, r.stream));
    r.stamps.push_back(p);
    return int(r.stamps.size()) - 1;
}

void Cmd::endTimestamp(int id) {
    Runtime& r = rt();
    if (id < 0 || id >= int(r.stamps.size())) return;
    EVK_CHECK(hipEventRecord(r.stamps[size_t(id)].end, r.stream));
}

uint64_t Cmd::submit() {
    Runtime& r = rt();
    require_up();
    Submission s{++r.submitted, new_event(false), std::move(r.stamps)};
    r.stamps.clear();
    EVK_CHECK(hipEventRecord(s.done, r.stream));
    r.inflight.push_back(std::move(s));
    r.open = false;
    if (r.desc.enableValidation) {
        EVK_CHECK(hipStreamSynchronize(r.stream));
        EVK_CHECK(hipGetLastError());
    }
    return r.submitted;
}

void* Cmd::stream() const {
    return rt().stream;
}

Cmd& CmdBegin(Queue) {
    require_up();
    Runtime& r = rt();
    reclaim();
    // retire finished submissions
    while (!r.inflight.empty()) {
        hipError_t q = hipEventQuery(r.inflight.front().done);
        if (q == hipErrorNotReady) break;
        if (q != hipSuccess) die("hipEventQuery", q);
        r.completed = r.inflight.front().index;
        finish_submission(r.inflight.front());
        r.inflight.pop_front();
    }
    r.open = true;
    return r.cmd;
}

bool CmdDone(uint64_t submissionIndex) {
    Runtime& r = rt();
    if (submissionIndex <= r.completed) return true;
    for (Submission& s : r.inflight) {
        if (s.index == submissionIndex) {
            hipError_t q = hipEventQuery(s.done);
            if (q == hipErrorNotReady) return false;
            if (q != hipSuccess) die("hipEventQuery", q);
            return true;
        }
    }
    return submissionIndex <= r.submitted;
}

void CmdWait(uint64_t submissionIndex) {
    Runtime& r = rt();
    require_up();
    if (submissionIndex > r.submitted) misuse("CmdWait on a submission that was never made");
    while (!r.inflight.empty() && r.inflight.front().index <= submissionIndex) {
        EVK_CHECK(hipEventSynchronize(r.inflight.front().done));
        r.completed = r.inflight.front().index;
        finish_submission(r.inflight.front());
        r.inflight.pop_front();
    }
    reclaim();
}

}  // namespace evk
