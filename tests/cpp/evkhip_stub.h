// Recording stand-in for the evkhip C ABI (include/evkhip.h), used with
// hip_mock.cpp to test the evk::ai host layer without a GPU.  Each entry
// point records its arguments and marks every tensor it was given as read or
// written by the stream.  Test infrastructure only.
#pragma once

#include <evkhip.h>

#include <string>
#include <vector>

struct StubCall {
    std::string name;
    std::vector<evkhip_tensor> tensors;
    std::vector<long long> ints;
    std::vector<double> floats;
    const void* ptr = nullptr;  // lse
    void* stream = nullptr;
};

const StubCall& stub_last_call();
int stub_call_count();
// Names of the entry points called since the last stub_clear_log(), in order.
const std::vector<std::string>& stub_call_log();
void stub_clear_log();
// The next entry point call returns `status` (once) with message `msg`.
void stub_fail_next(int status, const char* msg);

extern "C" int mock_errors();
extern "C" size_t mock_live_allocations();
extern "C" size_t mock_live_events();
extern "C" void mock_advance();
extern "C" bool mock_stream_access(const void* p, size_t n);
