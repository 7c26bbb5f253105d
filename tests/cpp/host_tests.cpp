// Host-logic tests of the evk core and evk::ai (evk_amd/csrc/evk_runtime.cpp,
// evk_amd/csrc/evk_ai.cpp) on a machine without a GPU: HIP is the host mock
// of hip_mock.cpp and the kernel library is the recording stub of
// evkhip_stub.cpp.  Built with g++ and the address/undefined-behaviour
// sanitizers by tests/test_cpp_host.py.
//
// Covered: buffer kinds and addresses, stream-ordered fill/copy/update with
// staged host sources, deferred frees (never before the stream has passed
// the last use), submission indices, CmdDone/CmdWait, timestamps, Tensor
// upload/download/identity/fill/item/stats/print, the descriptors and flags
// every evk::ai op hands to the C ABI, abort-on-error paths, and that
// shutdown leaves no allocation or event behind.
#include <evk_ai.h>

#include <sys/wait.h>
#include <unistd.h>

#include <csignal>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "evkhip_stub.h"

#define TEST(expr)                                                                \
    do {                                                                          \
        if (expr) {                                                               \
            std::printf(" TEST(" #expr ") [PASS]\n");                            \
        } else {                                                                  \
            std::printf(" TEST(" #expr ") [FAIL] [%s:%d]\n", __FILE__, __LINE__); \
            std::fflush(stdout);                                                  \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)

// Runs fn in a child process; true when the child died of SIGABRT.
template <typename F>
static bool aborts(F fn) {
    std::fflush(stdout);
    std::fflush(stderr);
    const pid_t pid = fork();
    if (pid == 0) {
        std::freopen("/dev/null", "w", stderr);
        fn();
        std::_Exit(0);
    }
    int status = 0;
    waitpid(pid, &status, 0);
    return WIFSIGNALED(status) && WTERMSIG(status) == SIGABRT;
}

static bool same_dims(const evkhip_tensor& d, Tensor& t) {
    if (d.rank != t.shape.rank() || d.data != t.device_ptr()) return false;
    for (uint32_t i = 0; i < d.rank; ++i)
        if (d.dims[i] != t.shape.values[i]) return false;
    return true;
}

static void test_uninitialized_use_aborts() {
    std::printf("test_uninitialized_use_aborts()\n");
    TEST(!evk::IsInitialized());
    TEST(aborts([] { Tensor t({4}); }));
    TEST(aborts([] { evk::CmdBegin(); }));
}

static void test_buffers_and_commands() {
    std::printf("test_buffers_and_commands()\n");
    evk::Buffer gpu = evk::CreateBuffer({.size = 4096});
    evk::Buffer pinned = evk::CreateBuffer({.size = 4096, .memoryType = evk::MemoryType::CPU});
    TEST(gpu.GetPtr() == nullptr && gpu.GetReference() != 0 && gpu.GetSize() == 4096);
    TEST(pinned.GetPtr() != nullptr && pinned.GetReference() == reinterpret_cast<uint64_t>(pinned.GetPtr()));
    std::vector<uint32_t> src(512);
    for (uint32_t i = 0; i < 512; ++i) src[i] = i * 7u + 1u;
    evk::Cmd& cmd = evk::CmdBegin();
    cmd.fill(gpu, 0x01020304u, 4096);
    cmd.copy(src.data(), gpu, 2048, 1024);
    std::fill(src.begin(), src.end(), 0u);  // staged: the copy already owns the bytes
    cmd.update(gpu, 0, 4, src.data());
    cmd.copy(gpu, pinned, 4096);
    const uint64_t idx = cmd.submit();
    TEST(!evk::CmdDone(idx));  // the mock stream has not run yet
    evk::CmdWait(idx);
    TEST(evk::CmdDone(idx));
    const uint32_t* h = static_cast<const uint32_t*>(pinned.GetPtr());
    bool ok = h[0] == 0u;
    for (uint32_t i = 1; i < 1024; ++i) ok &= h[i] == ((i >= 256 && i < 768) ? (i - 256) * 7u + 1u : 0x01020304u);
    TEST(ok);
    std::vector<uint32_t> back(1024);
    evk::ReadBuffer(gpu, back.data(), 4096);
    TEST(std::memcmp(back.data(), h, 4096) == 0);
    uint32_t w = 99;
    evk::WriteBuffer(gpu, &w, 4, 8);
    evk::ReadBuffer(gpu, back.data(), 12);
    TEST(back[2] == 99u);
    TEST(aborts([&] { evk::CmdBegin().copy(gpu, pinned, 4097); }));
    TEST(aborts([&] { evk::CmdBegin().fill(gpu, 0, 6); }));
    TEST(mock_errors() == 0);
}

static void test_deferred_free() {
    std::printf("test_deferred_free()\n");
    evk::ai::SubmitCmd(true);  // retire frees left by earlier tests
    const size_t before = mock_live_allocations();
    {
        Tensor t({256, 256});
        evk::ai::zero(t);  // the stream now uses t
    }
    // t is gone on the host but its memory is still owned by queued work
    TEST(mock_live_allocations() == before + 1);
    evk::ai::SubmitCmd(true);
    TEST(mock_live_allocations() == before);
    {
        Tensor t({64});
        evk::ai::zero(t);
    }
    mock_advance();               // the stream ran on its own ...
    evk::ai::SubmitCmd(false);
    evk::ai::GetCmd();            // ... and the next CmdBegin reclaims
    TEST(mock_live_allocations() == before);
    TEST(mock_errors() == 0);
}

static void test_staging_reuse() {
    std::printf("test_staging_reuse()\n");
    Tensor t({1 << 16});
    evk::ai::SubmitCmd(true);
    const size_t base = mock_live_allocations();
    std::vector<uint8_t> data(1 << 17, 3);
    for (int round = 0; round < 20; ++round) {
        evk::ai::GetCmd().copy(data.data(), t.buffer, 1000 + round * 50);
        evk::ai::SubmitCmd(true);
    }
    TEST(mock_live_allocations() <= base + 1);  // one reused staging chunk
    // several copies in flight need distinct chunks
    for (int i = 0; i < 3; ++i) evk::ai::GetCmd().copy(data.data(), t.buffer, 4096);
    evk::ai::SubmitCmd(true);
    TEST(mock_live_allocations() <= base + 3);
    TEST(mock_errors() == 0);
}

static void test_submissions_and_timestamps() {
    std::printf("test_submissions_and_timestamps()\n");
    Tensor a({8});
    evk::Cmd& cmd = evk::ai::GetCmd();
    const int id0 = cmd.beginTimestamp("first");
    evk::ai::zero(a);
    cmd.endTimestamp(id0);
    cmd.timestamp("second", [&] { evk::ai::zero(a); });
    const uint64_t s1 = evk::ai::SubmitCmd(false);
    const uint64_t s2 = evk::ai::SubmitCmd(false);
    TEST(s2 == s1 + 1);
    evk::CmdWait(s2);
    TEST(evk::CmdDone(s1) && evk::CmdDone(s2));
    const auto& ts = evk::CmdTimestamps();
    TEST(ts.size() == 2);
    TEST(std::strcmp(ts[0].name, "first") == 0 && std::strcmp(ts[1].name, "second") == 0);
    TEST(ts[0].start == 0.0 && ts[0].end >= ts[0].start && ts[1].start >= ts[0].start);
    TEST(aborts([&] { evk::CmdWait(s2 + 5); }));
    TEST(mock_errors() == 0);
}

static void test_tensor_host_paths() {
    std::printf("test_tensor_host_paths()\n");
    Tensor a({3, 3}), b({3, 3}), c({3, 3});
    a.identity(float16_t(2.0f));
    b.fill(float16_t(0.25f));
    evk::ai::add(a, b, c);  // the stub computes this one
    c.cpu_download();
    bool ok = true;
    for (uint32_t i = 0; i < 9; ++i) ok &= float(c.cpu()[i]) == ((i % 4 == 0) ? 2.25f : 0.25f);
    TEST(ok);
    Tensor one({1}), two({1}), sum({1});
    one.fill(float16_t(1.5f));
    two.fill(float16_t(2.25f));
    evk::ai::add(one, two, sum);
    TEST(float(sum.item()) == 3.75f);
    Tensor s({6});
    float16_t* h = s.cpu();
    const float vals[6] = {1.0f, -3.0f, 0.0f, NAN, INFINITY, 2.0f};
    for (int i = 0; i < 6; ++i) h[i] = float16_t(vals[i]);
    s.cpu_upload();
    std::memset(h, 0, 12);
    GradStats st = s.stats();
    TEST(st.nan_count == 1 && st.inf_count == 1 && st.zero_count == 1);
    TEST(st.min_val == -3.0f && st.max_val == 2.0f && st.mean == 0.0f);
    Tensor big({2, 10, 12});
    big.fill(float16_t(1.0f));
    big.print();
    Tensor g({4});
    TEST(&g.grad() == &g.grad() && g.grad().shape.count() == 4);
    Tensor al = Tensor::alias(Shape({2, 2}), g.buffer);
    TEST(al.device_ptr() == g.device_ptr());
    TEST(mock_errors() == 0);
}

static void test_op_marshalling() {
    std::printf("test_op_marshalling()\n");
    void* stream = evk::ai::GetCmd().stream();
    Tensor a({2, 64, 32}), b({32, 48}), c({2, 64, 48});
    evk::ai::matmul(a, b, c, true, false, true, 16, 32);
    const StubCall& m = stub_last_call();
    TEST(m.name == "matmul" && m.tensors.size() == 3);
    TEST(same_dims(m.tensors[0], a) && same_dims(m.tensors[1], b) && same_dims(m.tensors[2], c));
    TEST(m.ints == std::vector<long long>({1, 0, 1, 16, 32}) && m.stream == stream);
    evk::ai::matmul(a, b, c);
    TEST(stub_last_call().ints == std::vector<long long>({0, 0, 0, 80, 80}));

    const uint32_t B = 2, N = 32, H = 4, Dh = 16;
    Tensor q({B, N, H * Dh}), k({B, N, Dh}), v({B, N, Dh}), o({B, N, H * Dh}), lse({B, H, N, 2});
    evk::ai::flash_attention(q, k, v, o);
    TEST(stub_last_call().name == "flash_attention" && stub_last_call().ints[0] == 0 && !stub_last_call().ptr);
    evk::ai::flash_attention(q, k, v, o, true, &lse);
    TEST(stub_last_call().ints[0] == 1 && stub_last_call().ptr == lse.device_ptr());
    TEST(same_dims(stub_last_call().tensors[3], o));
    Tensor dO({B, N, H * Dh}), dQ({B, N, H * Dh}), dK({B, N, Dh}), dV({B, N, Dh});
    evk::ai::flash_attention_bwd(q, k, v, o, dO, dQ, dK, dV);
    TEST(stub_last_call().name == "flash_attention_bwd" && stub_last_call().tensors.size() == 8);
    TEST(stub_last_call().ints == std::vector<long long>({0, 0}) && !stub_last_call().ptr);
    evk::ai::flash_attention_bwd(q, k, v, o, dO, dQ, dK, dV, H, true, &lse);
    TEST(stub_last_call().ints == std::vector<long long>({H, 1}) && stub_last_call().ptr == lse.device_ptr());
    TEST(same_dims(stub_last_call().tensors[7], dV) && same_dims(stub_last_call().tensors[5], dQ));
    Tensor bad_lse({B, H, N});
    TEST(aborts([&] { evk::ai::flash_attention(q, k, v, o, true, &bad_lse); }));

    Tensor sq({768}), kc({100, 768}), vc({100, 768}), so({768});
    evk::ai::single_query_attention(sq, kc, vc, so, 57, 12);
    TEST(stub_last_call().ints == std::vector<long long>({57, 12}) && same_dims(stub_last_call().tensors[2], vc));
    evk::ai::single_query_attention(sq, kc, vc, so, 3);
    TEST(stub_last_call().ints == std::vector<long long>({3, 1}));

    Tensor x({1, 5, 24}), y({1, 5, 24});
    evk::ai::rope(x, y, 1, 5, 24);
    TEST(stub_last_call().ints == std::vector<long long>({1, 5, 24, 0, 0}) && stub_last_call().floats[0] == 10000.0);
    evk::ai::rope(x, y, 1, 5, 24, 500000.0f, 1031, 8);
    TEST(stub_last_call().ints == std::vector<long long>({1, 5, 24, 1031, 8}) && stub_last_call().floats[0] == 500000.0);
    evk::ai::rms_norm(x, y);
    TEST(stub_last_call().name == "rms_norm" && stub_last_call().floats[0] == double(1e-4f));
    evk::ai::rms_norm(x, y, 1e-5f);
    TEST(stub_last_call().floats[0] == double(1e-5f));
    evk::ai::gelu(x, y);
    TEST(stub_last_call().name == "gelu" && same_dims(stub_last_call().tensors[1], y));
    Tensor table({10, 24}), ids({5}), emb({5, 24});
    evk::ai::embed(table, ids, emb);
    TEST(stub_last_call().name == "embed" && same_dims(stub_last_call().tensors[1], ids));
    Tensor logits({2, 3, 50}), tok({2});
    evk::ai::greedy_sample(logits, tok, 2, 7, 40);
    TEST(stub_last_call().ints == std::vector<long long>({2, 7, 40}));

    stub_fail_next(EVKHIP_ERR_SHAPE, "matmul: injected shape error");
    TEST(aborts([&] { evk::ai::matmul(a, b, c); }));
    stub_fail_next(0, "");
    evk::ai::SubmitCmd(true);
    TEST(mock_errors() == 0);
}

// AdamState bookkeeping and the Graph's call order, against the recording
// stub: bias corrections from the step count, the forward functions in
// order and the backward ones in reverse, causal_attention on the fused
// flash entry points (the unfused chain only for a non-default scale).
// The entry points of the stub's log other than the fills (Graph::eval
// zeroes gradients with evkhip_fill before the backward pass), and the
// number of fills.
static std::vector<std::string> ops_of_log(int* fills = nullptr) {
    std::vector<std::string> ops;
    int n = 0;
    for (const std::string& s : stub_call_log()) {
        if (s == "fill") ++n;
        else ops.push_back(s);
    }
    if (fills) *fills = n;
    return ops;
}

static void test_training_host() {
    std::printf("test_training_host()\n");
    Tensor p({40}), g({40});
    evk::ai::AdamState st;
    evk::ai::adam(p, g, st, 0.01f, 0.9f, 0.999f, 1e-4f);
    evk::ai::adam(p, g, st, 0.01f, 0.9f, 0.999f, 1e-4f);
    const StubCall& a = stub_last_call();
    TEST(a.name == "adam" && st.t == 2 && bool(st.m_buffer) && bool(st.v_buffer));
    TEST(a.tensors.size() == 4 && a.tensors[2].dims[0] == 40 && a.tensors[3].dims[0] == 40);
    const double c1 = 1.0 / (1.0 - 0.9 * 0.9), c2 = 1.0 / (1.0 - 0.999 * 0.999);
    TEST(std::fabs(a.floats[3] - c1) < 1e-4 * c1 && std::fabs(a.floats[4] - c2) < 1e-3 * c2);
    st.reset();
    TEST(!st.m_buffer && st.t == 0);

    Graph gr;
    Tensor& x = gr.tensor({8, 8});
    Tensor& w = gr.tensor({8, 8}, true);
    Tensor& tgt = gr.tensor({8, 8});
    Tensor& loss = gr.mse_loss(gr.relu(gr.matmul(w, x)), tgt);
    (void)loss;
    stub_clear_log();
    gr.eval(true);
    gr.step(0.1f);
    const std::vector<std::string> want = {"matmul", "relu", "mse_loss", "relu_backward", "matmul", "matmul", "sgd"};
    int fills = 0;
    TEST(ops_of_log(&fills) == want);
    TEST(fills > 0);  // gradients zeroed by a kernel, never a memset

    Graph ga;
    Tensor& q = ga.tensor({2, 16, 32}, true);
    Tensor& k = ga.tensor({2, 16, 32}, true);
    Tensor& v = ga.tensor({2, 16, 32}, true);
    ga.causal_attention(q, k, v);
    stub_clear_log();
    ga.eval(true);
    const std::vector<std::string> fused = {"flash_attention", "flash_attention_bwd", "add", "add", "add"};
    TEST(ops_of_log() == fused);
    Graph gu;
    Tensor& q2 = gu.tensor({2, 16, 32}, true);
    gu.causal_attention(q2, q2, q2, 0.5f);
    stub_clear_log();
    gu.eval(false);
    const std::vector<std::string> unfused = {"matmul", "apply_causal_mask", "softmax", "matmul"};
    TEST(ops_of_log() == unfused);
    // a head size without MFMA flash kernels keeps the unfused chain; the
    // reference's own head of 256 takes the fused one
    Graph gd;
    Tensor& q3 = gd.tensor({2, 16, 40}, true);
    gd.causal_attention(q3, q3, q3);
    stub_clear_log();
    gd.eval(false);
    TEST(!evkhip_flash_has_mfma(40) && ops_of_log() == unfused);
    Graph gw;
    Tensor& q4 = gw.tensor({2, 16, 256}, true);
    gw.causal_attention(q4, q4, q4);
    stub_clear_log();
    gw.eval(false);
    TEST(evkhip_flash_has_mfma(256) && ops_of_log() == std::vector<std::string>{"flash_attention"});
    evk::ai::SubmitCmd(true);
    TEST(mock_errors() == 0);
}

int main() {
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    test_uninitialized_use_aborts();
    evk::EvkDesc desc;
    desc.enableTimestamps = true;
    TEST(evk::InitializeEVK(desc));
    evk::ai::initialize();
    TEST(evk::IsInitialized() && evk::GetFeatures().coopmat && evk::GetFeatures().timestamps);
    test_buffers_and_commands();
    test_deferred_free();
    test_staging_reuse();
    test_submissions_and_timestamps();
    test_tensor_host_paths();
    test_op_marshalling();
    test_training_host();
    evk::ai::shutdown();
    TEST(!evk::IsInitialized());
    TEST(mock_live_allocations() == 0);
    TEST(mock_live_events() == 0);
    TEST(mock_errors() == 0);
    // the runtime comes back up after a shutdown
    evk::ai::initialize();
    {
        Tensor t({1});
        t.fill(float16_t(1.0f));
        TEST(float(t.item()) == 1.0f);
    }
    evk::ai::shutdown();
    TEST(mock_live_allocations() == 0 && mock_live_events() == 0 && mock_errors() == 0);
    std::printf("ALL PASSED\n");
    return 0;
}
