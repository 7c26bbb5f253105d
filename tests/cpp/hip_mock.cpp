// A host-memory stand-in for the HIP runtime calls made by the evk core
// (evk_amd/csrc/evk_runtime.cpp) and evk::ai (evk_amd/csrc/evk_ai.cpp), so
// their host logic runs on a machine without a GPU, under the address and
// undefined-behaviour sanitizers.  Test infrastructure only.
//
// Model: one device ("gfx950"), memory is host heap memory, every copy and
// fill takes effect immediately, but completion is reported the way a real
// stream would: an event recorded at stream position p reads as complete only
// after a synchronisation has covered p (hipStreamSynchronize,
// hipEventSynchronize) -- or, to model a GPU that advances on its own, after
// mock_advance().  Freeing memory that is still "in flight" (allocated and
// enqueued-on after the last completed position) is reported as an error, as
// are unknown or double frees.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>

struct ihipStream_t {
    int id;
};
struct ihipEvent_t {
    bool timing;
    bool recorded = false;
    unsigned long long pos = 0;  // stream position at record time
    double ms = 0.0;
};

namespace {

struct Alloc {
    size_t size;
    bool host;
    unsigned long long last_use;  // stream position of the last enqueued access
};

struct MockState {
    std::map<const char*, Alloc> allocs;
    std::set<ihipEvent_t*> events;
    std::set<ihipStream_t*> streams;
    unsigned long long enqueued = 0;   // stream position of the latest enqueued op
    unsigned long long completed = 0;  // every op <= completed has "run"
    int errors = 0;
    int device = 0;
};

MockState& M() {
    static MockState s;
    return s;
}

void fail(const char* what) {
    std::fprintf(stderr, "hip_mock: %s\n", what);
    M().errors++;
}

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// The allocation containing [p, p+n), or nullptr.
Alloc* find(const void* p, size_t n) {
    auto& a = M().allocs;
    auto it = a.upper_bound(static_cast<const char*>(p));
    if (it == a.begin()) return nullptr;
    --it;
    const char* base = it->first;
    if (static_cast<const char*>(p) < base || static_cast<const char*>(p) + n > base + it->second.size) return nullptr;
    return &it->second;
}

bool touch(const void* p, size_t n, const char* what) {
    if (n == 0) return true;
    Alloc* a = find(p, n);
    if (!a) {
        fail(what);
        return false;
    }
    a->last_use = ++M().enqueued;
    return true;
}

}  // namespace

extern "C" int mock_errors() {
    return M().errors;
}
extern "C" size_t mock_live_allocations() {
    return M().allocs.size();
}
extern "C" size_t mock_live_events() {
    return M().events.size();
}
// Lets the "GPU" finish everything enqueued so far (without a host sync).
extern "C" void mock_advance() {
    M().completed = M().enqueued;
}

hipError_t hipGetDeviceCount(int* count) {
    *count = 1;
    return hipSuccess;
}
hipError_t hipSetDevice(int id) {
    if (id != 0) return hipErrorInvalidDevice;
    M().device = id;
    return hipSuccess;
}
hipError_t hipGetDevice(int* id) {
    *id = M().device;
    return hipSuccess;
}
hipError_t hipGetDeviceProperties(hipDeviceProp_t* prop, int id) {
    if (id != 0) return hipErrorInvalidDevice;
    std::memset(prop, 0, sizeof(*prop));
    std::strcpy(prop->gcnArchName, "gfx950:sramecc+:xnack-");
    prop->multiProcessorCount = 256;
    return hipSuccess;
}
hipError_t hipGetLastError(void) {
    return hipSuccess;
}
const char* hipGetErrorString(hipError_t e) {
    return e == hipSuccess ? "hipSuccess" : "mock HIP error";
}

hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned int) {
    *s = new ihipStream_t{int(M().streams.size())};
    M().streams.insert(*s);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
    if (!M().streams.erase(s)) {
        fail("hipStreamDestroy of an unknown stream");
        return hipErrorInvalidHandle;
    }
    delete s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) {
    M().completed = M().enqueued;
    return hipSuccess;
}

hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned flags) {
    *e = new ihipEvent_t{(flags & hipEventDisableTiming) == 0};
    M().events.insert(*e);
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    if (!M().events.erase(e)) {
        fail("hipEventDestroy of an unknown event");
        return hipErrorInvalidHandle;
    }
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
    if (!M().events.count(e)) {
        fail("hipEventRecord of an unknown event");
        return hipErrorInvalidHandle;
    }
    e->recorded = true;
    e->pos = ++M().enqueued;
    e->ms = now_ms();
    return hipSuccess;
}
hipError_t hipEventQuery(hipEvent_t e) {
    if (!M().events.count(e)) {
        fail("hipEventQuery of an unknown event");
        return hipErrorInvalidHandle;
    }
    return (!e->recorded || e->pos <= M().completed) ? hipSuccess : hipErrorNotReady;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
    if (!M().events.count(e)) {
        fail("hipEventSynchronize of an unknown event");
        return hipErrorInvalidHandle;
    }
    if (e->pos > M().completed) M().completed = e->pos;
    return hipSuccess;
}
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    if (!M().events.count(a) || !M().events.count(b) || !a->timing || !b->timing) {
        fail("hipEventElapsedTime on unknown or non-timing events");
        return hipErrorInvalidHandle;
    }
    if (a->pos > M().completed || b->pos > M().completed) {
        fail("hipEventElapsedTime before the events completed");
        return hipErrorNotReady;
    }
    *ms = float(b->ms - a->ms);
    return hipSuccess;
}

static hipError_t mock_alloc(void** p, size_t size, bool host) {
    char* m = static_cast<char*>(std::malloc(size ? size : 1));
    std::memset(m, 0xA5, size ? size : 1);
    M().allocs[m] = Alloc{size ? size : 1, host, M().enqueued};
    *p = m;
    return hipSuccess;
}
static hipError_t mock_free(void* p, bool host) {
    if (!p) return hipSuccess;
    auto it = M().allocs.find(static_cast<const char*>(p));
    if (it == M().allocs.end()) {
        fail("free of an unknown pointer (double free?)");
        return hipErrorInvalidValue;
    }
    if (it->second.host != host) fail("hipFree/hipHostFree mismatch");
    if (it->second.last_use > M().completed) fail("memory freed while the stream may still use it");
    M().allocs.erase(it);
    std::free(p);
    return hipSuccess;
}
hipError_t hipMalloc(void** p, size_t size) {
    return mock_alloc(p, size, false);
}
hipError_t hipFree(void* p) {
    return mock_free(p, false);
}
hipError_t hipHostMalloc(void** p, size_t size, unsigned int) {
    return mock_alloc(p, size, true);
}
hipError_t hipHostFree(void* p) {
    return mock_free(p, true);
}
hipError_t hipHostGetDevicePointer(void** dev, void* host, unsigned int) {
    Alloc* a = find(host, 1);
    if (!a || !a->host) {
        fail("hipHostGetDevicePointer of non-pinned memory");
        return hipErrorInvalidValue;
    }
    *dev = host;
    return hipSuccess;
}
hipError_t hipMemGetInfo(size_t* free_b, size_t* total_b) {
    *total_b = size_t(288) << 30;
    *free_b = *total_b - (size_t(1) << 30);
    return hipSuccess;
}

hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind kind, hipStream_t) {
    // host sources of HostToDevice copies may be pageable: only device/pinned ends are checked
    const bool src_known = kind != hipMemcpyHostToDevice;
    const bool dst_known = kind != hipMemcpyDeviceToHost;
    if (src_known && !touch(src, n, "hipMemcpyAsync source outside any allocation")) return hipErrorInvalidValue;
    if (dst_known && !touch(dst, n, "hipMemcpyAsync destination outside any allocation")) return hipErrorInvalidValue;
    ++M().enqueued;
    std::memmove(dst, src, n);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int value, size_t n, hipStream_t) {
    if (!touch(dst, n, "hipMemsetAsync outside any allocation")) return hipErrorInvalidValue;
    std::memset(dst, value, n);
    return hipSuccess;
}
hipError_t hipMemsetD32Async(hipDeviceptr_t dst, int value, size_t count, hipStream_t) {
    if (!touch(dst, count * 4, "hipMemsetD32Async outside any allocation")) return hipErrorInvalidValue;
    uint32_t* p = static_cast<uint32_t*>(dst);
    for (size_t i = 0; i < count; ++i) p[i] = uint32_t(value);
    return hipSuccess;
}

// Kernel "launch" bookkeeping used by the evkhip stub: marks [p, p+n) as
// accessed by the stream.
extern "C" bool mock_stream_access(const void* p, size_t n) {
    return touch(p, n, "kernel access outside any allocation");
}
