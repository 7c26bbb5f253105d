// evk core, HIP edition: the part of the evk runtime API that the evk::ai hot
// path uses (buffers, command recording/submission, timestamps), implemented
// over one HIP stream on one MI355X.
//
// Mirrors /root/reference/evk.h (Buffer :245-262, ResourceRef :126-170,
// EvkDesc/InitializeEVK :332-354, TimestampEntry :93-96, Cmd :373-476,
// CmdBegin/CmdDone/CmdWait :484-490) with these semantics:
//   * a Cmd is not a recorded command buffer: every command is enqueued on the
//     library's HIP stream as it is issued, in order.  Stream order gives the
//     same guarantee as the reference's per-op full barrier, so barrier() is
//     a no-op.  submit() marks a point in the stream (an event) and returns
//     its index; CmdWait(index) blocks the host until that point has run.
//   * Buffer memory: MemoryType::GPU is device memory (hipMalloc); the other
//     memory types are pinned, device-mapped host memory (hipHostMalloc), so
//     GetPtr() is the host address for those and nullptr for GPU buffers.
//     GetReference() is the device address of any buffer (the analogue of a
//     Vulkan buffer device address); kernels and the C ABI take it directly.
//   * A buffer whose last reference drops is freed only after the stream
//     has passed everything submitted so far (deferred free, no mid-stream
//     synchronous hipFree).
//   * Single-threaded, one device, like the reference's global state.
// Graphics, images, pipelines, ray tracing and the swapchain are not part of
// this library.
#pragma once

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace evk {

enum class BufferUsage {
    TransferSrc = 1,
    TransferDst = 2,
    Vertex = 4,
    Index = 8,
    Indirect = 16,
    Storage = 32,
    AccelerationStructure = 64,
    AccelerationStructureInput = 128,
};
inline BufferUsage operator|(BufferUsage a, BufferUsage b) {
    return BufferUsage(int(a) | int(b));
}

enum class MemoryType {
    CPU,         // pinned host memory, visible to the device
    GPU,         // HBM
    CPU_TO_GPU,  // pinned host memory (upload staging)
    GPU_TO_CPU,  // pinned host memory (read back)
};

struct TimestampEntry {
    double start, end;  // milliseconds, relative to the first timestamp of the submission
    const char* name;
};

struct MemoryBudget {
    static constexpr uint32_t MAX_HEAPS = 16u;
    struct Heap {
        uint32_t blockCount;
        uint32_t allocationCount;
        uint64_t blockBytes;
        uint64_t allocationBytes;
        uint64_t usage;
        uint64_t budget;
    } heaps[MAX_HEAPS];
};

// Intrusively reference-counted resource.
struct Resource {
    int refCount = 0;
    virtual ~Resource() = default;
    void incRef() { ++refCount; }
    void decRef();  // destroys (deferred) at zero
};

struct ResourceRef {
    Resource* res = nullptr;
    ResourceRef() = default;
    ResourceRef(Resource* r) : res(r) {
        if (res) res->incRef();
    }
    ResourceRef(const ResourceRef& o) : res(o.res) {
        if (res) res->incRef();
    }
    ResourceRef(ResourceRef&& o) noexcept : res(o.res) { o.res = nullptr; }
    ResourceRef& operator=(const ResourceRef& o) {
        if (o.res) o.res->incRef();
        if (res) res->decRef();
        res = o.res;
        return *this;
    }
    ResourceRef& operator=(ResourceRef&& o) noexcept {
        if (this != &o) {
            if (res) res->decRef();
            res = o.res;
            o.res = nullptr;
        }
        return *this;
    }
    ~ResourceRef() {
        if (res) res->decRef();
    }
    explicit operator bool() const { return res != nullptr; }
    void release() {
        if (res) res->decRef();
        res = nullptr;
    }
};

struct BufferDesc {
    std::string name = "";
    uint64_t size = 0;
    BufferUsage usage = BufferUsage::Storage;
    MemoryType memoryType = MemoryType::GPU;
};

struct Buffer : ResourceRef {
    Buffer(Resource* res = nullptr) : ResourceRef(res) {}
    void* GetPtr();            // host address (pinned memory types), nullptr for GPU memory
    uint64_t GetReference();   // device address
    uint64_t GetSize();
};
Buffer CreateBuffer(const BufferDesc& desc);
// Synchronous host<->buffer copies (complete on return).
void WriteBuffer(Buffer& buffer, void* src, uint64_t size, uint64_t offset = 0u);
void ReadBuffer(Buffer& buffer, void* dst, uint64_t size, uint64_t offset = 0u);

struct EvkDesc {
    std::string applicationName = "";
    std::uint32_t applicationVersion = 0;
    std::string engineName = "";
    std::uint32_t engineVersion = 0;
    std::vector<std::string> instanceLayers = {};
    std::vector<std::string> instanceExtensions = {};
    uint32_t frameBufferingCount = 3;
    bool enableSwapchain = false;   // no presentation in this library: must stay false
    bool enableValidation = false;  // checks every HIP call's status eagerly (hipStreamSynchronize after each submit)
    bool enableTimestamps = false;  // Cmd::beginTimestamp/endTimestamp record HIP events
    int device = 0;                 // HIP device ordinal (this library's addition)
};

struct Features {
    bool raytracing = false;
    bool coopmat = false;     // true: the matrix-core (MFMA) kernels are available
    bool timestamps = false;
};

bool InitializeEVK(const EvkDesc& info);
void Shutdown();
bool IsInitialized();
const Features& GetFeatures();
MemoryBudget GetMemoryBudget();
// Timestamps of the last submission that CmdWait() saw complete.
const std::vector<TimestampEntry>& CmdTimestamps();

enum class Queue {
    Graphics,
};

struct Cmd {
    void* _internal = nullptr;

    // Stream order already serialises every command: kept for API parity.
    void barrier();

    // Buffer commands (all stream-ordered; the host source of copy(void*) and
    // update() is staged, so it may be reused as soon as the call returns).
    void fill(Buffer dst, uint32_t data, uint64_t size, uint64_t offset = 0);
    void update(Buffer& dst, uint64_t dstOffset, uint64_t size, void* src);
    void copy(Buffer& src, Buffer& dst, uint64_t size, uint64_t srcOffset = 0, uint64_t dstOffset = 0);
    void copy(void* src, Buffer& dst, uint64_t size, uint64_t dstOffset = 0);

    // GPU timestamps (HIP events; only when EvkDesc::enableTimestamps).
    int beginTimestamp(const char* name);
    void endTimestamp(int id);
    template <typename T>
    void timestamp(const char* name, T callback) {
        int id = beginTimestamp(name);
        callback();
        endTimestamp(id);
    }

    // Marks the end of this submission on the stream; returns its index.
    uint64_t submit();

    // The HIP stream (hipStream_t) commands are enqueued on.
    void* stream() const;
};

Cmd& CmdBegin(Queue queue = Queue::Graphics);
bool CmdDone(uint64_t submissionIndex);
void CmdWait(uint64_t submissionIndex);

}  // namespace evk
