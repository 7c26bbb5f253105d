// The reference caller's decode through evk::ai::KVCacheDecoder, at the shape
// example/main_llm.cpp trains and samples (:694-702: B=16 sequences, model
// dim 256 as one head, hidden 512, 8 layers, vocab 144, 160 positions; the
// sampling loop :622-654 picks ids from the coordinate range [3, 131)).
//
//   kv_decoder_tool dump <dir> [steps]
//       Builds the model with the reference's initialisation (srand(42),
//       N(0, 0.02), residual projections 0.02/sqrt(2L), main_llm.cpp:599-611),
//       prefills an 18-token prompt per sequence (BOS + condition tokens),
//       then runs `steps` greedy steps (default 32) feeding each sequence its
//       own sampled id.  Writes, as raw little-endian files:
//         weights.bin  the model in the CPU oracle's blob layout (fp16 bits):
//                      E (V,D); per layer Wqkv (D,3D) = [Wq|Wk|Wv], Wo (D,D),
//                      W1 (D,HID), W2 (HID,D); then Wout (D,V)
//         prompt.bin   (B, 19) uint16: positions 0..18 (18 is the first fed)
//         logits.bin   (steps, B, V) fp16 bits: logits of positions 18..
//         ids.bin      (steps, B) uint16: the greedy id after each step
//       The oracle parity test (tests/test_gpu_kv_decoder.py) replays every
//       sequence through the oracle model with these ids.
//
//   kv_decoder_tool bench [reps]
//       Times the caller's whole sampling loop, positions 18..107 (90 ids per
//       sequence), three ways, and prints one JSON line:
//         full_recompute  the reference's loop: per position upload the
//                         tokens, Graph::eval over all 160 positions,
//                         greedy_sample at pos, download the ids (SubmitCmd(true))
//         kv_host_ids     KVCacheDecoder prefill + one step per position, the
//                         ids downloaded every step as the reference's loop does
//         kv_device_ids   the same, each step fed the previous step's ids on
//                         the device; one synchronisation at the end
//         kv_op_by_op     kv_device_ids with the op-by-op step (16 launches a
//                         layer) instead of the fused one-launch step
//       Both paths compute the same logits up to rounding (the oracle test
//       checks the decoder); a near-tie can send a sequence down another
//       path, which changes none of the timed work.
#include <evk_ai.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>



namespace {

constexpr uint32_t B = 16, S = 160, V = 144, D = 256, HID = 512, L = 8;
constexpr uint32_t PROMPT = 18;         // positions prefilled: BOS + 17 condition tokens
constexpr uint32_t FIRST = PROMPT;      // first fed position (kConditionCoordTokens)
constexpr uint32_t LAST = 108;          // main_llm's loop ends before kCoordTokenCount
constexpr uint16_t BASE = 3, BINS = 128;

struct Lcg {
    uint64_t s;
    explicit Lcg(uint64_t seed) : s(seed * 2862933555777941757ull + 3037000493ull) {}
    float uniform() {  // [-1, 1)
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return float(int64_t(s >> 40) - (1ll << 23)) / float(1 << 23);
    }
};

struct Model {
    Graph g;
    Tensor* in = nullptr;
    Tensor* emb = nullptr;
    Tensor* w_out = nullptr;
    Tensor* logits = nullptr;
    std::vector<evk::ai::DecoderLayer> layers;

    Model() {
        in = &g.tensor({B, S});
        emb = &g.tensor({V, D}, true);
        Tensor* x = &g.embed(*emb, *in);
        layers.resize(L);
        for (uint32_t l = 0; l < L; ++l) {
            evk::ai::DecoderLayer& w = layers[l];
            w.w_q = &g.tensor({D, D}, true);
            w.w_k = &g.tensor({D, D}, true);
            w.w_v = &g.tensor({D, D}, true);
            w.w_o = &g.tensor({D, D}, true);
            w.w1 = &g.tensor({D, HID}, true);
            w.w2 = &g.tensor({HID, D}, true);
            // CausalAttentionBlock::forward (main_llm.cpp:528-546)
            Tensor& nin = g.rms_norm(*x);
            Tensor& q = g.rope(g.matmul(nin, *w.w_q), 10000.0f);
            Tensor& k = g.rope(g.matmul(nin, *w.w_k), 10000.0f);
            Tensor& v = g.matmul(nin, *w.w_v);
            Tensor& res1 = g.residual(*x, g.matmul(g.causal_attention(q, k, v), *w.w_o));
            Tensor& hid = g.gelu(g.matmul(g.rms_norm(res1), *w.w1));
            x = &g.residual(res1, g.matmul(hid, *w.w2));
        }
        w_out = &g.tensor({D, V}, true);
        logits = &g.matmul(g.rms_norm(*x), *w_out, 16, 16);
        // MeshTokenModel::init_weights (main_llm.cpp:599-611)
        srand(42);
        const float sd = 0.02f, rsd = 0.02f / std::sqrt(2.0f * float(L));
        emb->random_init(sd);
        w_out->random_init(sd);
        for (auto& w : layers) {
            w.w_q->random_init(sd);
            w.w_k->random_init(sd);
            w.w_v->random_init(sd);
            w.w_o->random_init(rsd);
            w.w1->random_init(sd);
            w.w2->random_init(rsd);
        }
    }
};

std::vector<uint16_t> bits(Tensor& t) {
    t.cpu_download();
    std::vector<uint16_t> v(t.shape.count());
    for (size_t i = 0; i < v.size(); ++i) v[i] = t.cpu()[i].value;
    return v;
}

void put_ids(Tensor& t, const uint16_t* src, bool submit = true) {
    float16_t* h = t.cpu();
    for (uint32_t i = 0; i < t.shape.count(); ++i) h[i].value = src[i];
    t.cpu_upload(submit);
}

// (B, S) tokens: BOS, 18 condition tokens in [BASE, BASE + BINS), pads after
std::vector<uint16_t> make_tokens() {
    std::vector<uint16_t> toks(B * S, 0);
    Lcg rng(77);
    for (uint32_t b = 0; b < B; ++b) {
        toks[b * S] = 1;
        for (uint32_t i = 1; i <= FIRST; ++i)
            toks[b * S + i] = uint16_t(BASE + uint32_t((rng.uniform() + 1.0f) * 0.5f * BINS) % BINS);
    }
    return toks;
}

void write_file(const std::string& path, const void* p, size_t bytes) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, bytes, f) != bytes) {
        std::fprintf(stderr, "kv_decoder_tool: cannot write %s\n", path.c_str());
        std::exit(1);
    }
    std::fclose(f);
}

int dump(const std::string& dir, uint32_t steps) {
    if (steps == 0 || FIRST + steps > S) {
        std::fprintf(stderr, "kv_decoder_tool: steps must be in [1, %u]\n", S - FIRST);
        return 2;
    }
    Model m;
    // the oracle's weight blob
    std::vector<uint16_t> blob = bits(*m.emb);
    for (auto& w : m.layers) {
        const std::vector<uint16_t> q = bits(*w.w_q), k = bits(*w.w_k), v = bits(*w.w_v);
        for (uint32_t i = 0; i < D; ++i) {
            blob.insert(blob.end(), q.begin() + i * D, q.begin() + (i + 1) * D);
            blob.insert(blob.end(), k.begin() + i * D, k.begin() + (i + 1) * D);
            blob.insert(blob.end(), v.begin() + i * D, v.begin() + (i + 1) * D);
        }
        for (Tensor* t : {w.w_o, w.w1, w.w2}) {
            const std::vector<uint16_t> x = bits(*t);
            blob.insert(blob.end(), x.begin(), x.end());
        }
    }
    const std::vector<uint16_t> wo = bits(*m.w_out);
    blob.insert(blob.end(), wo.begin(), wo.end());
    write_file(dir + "/weights.bin", blob.data(), blob.size() * 2);

    const std::vector<uint16_t> toks = make_tokens();
    std::vector<uint16_t> prompt(B * (FIRST + 1));
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t i = 0; i <= FIRST; ++i) prompt[b * (FIRST + 1) + i] = toks[b * S + i];
    write_file(dir + "/prompt.bin", prompt.data(), prompt.size() * 2);

    evk::ai::KVCacheDecoder dec(*m.emb, *m.w_out, m.layers, B, S);
    Tensor pre({B, PROMPT});
    {
        std::vector<uint16_t> p(B * PROMPT);
        for (uint32_t b = 0; b < B; ++b)
            for (uint32_t i = 0; i < PROMPT; ++i) p[b * PROMPT + i] = toks[b * S + i];
        put_ids(pre, p.data());
    }
    dec.prefill(pre);
    Tensor ids_a({B}), ids_b({B});
    {
        std::vector<uint16_t> first(B);
        for (uint32_t b = 0; b < B; ++b) first[b] = toks[b * S + FIRST];
        put_ids(ids_a, first.data());
    }
    std::vector<uint16_t> all_logits, all_ids;
    Tensor* cur = &ids_a;
    Tensor* nxt = &ids_b;
    for (uint32_t s = 0; s < steps; ++s) {
        Tensor& lg = dec.step(*cur);
        evk::ai::greedy_sample(lg, *nxt, 0, BASE, BINS);
        const std::vector<uint16_t> l = bits(lg), id = bits(*nxt);
        all_logits.insert(all_logits.end(), l.begin(), l.end());
        all_ids.insert(all_ids.end(), id.begin(), id.end());
        std::swap(cur, nxt);
    }
    write_file(dir + "/logits.bin", all_logits.data(), all_logits.size() * 2);
    write_file(dir + "/ids.bin", all_ids.data(), all_ids.size() * 2);
    std::printf("kv_decoder_tool: dumped %u steps x %u sequences to %s\n", steps, B, dir.c_str());
    return 0;
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// The reference's sample_autoregressive loop (main_llm.cpp:622-654) on the
// Graph: full recompute per position.  Returns ms; toks receives the ids.
double run_full(Model& m, std::vector<uint16_t>& toks) {
    Tensor sampled({B});
    evk::ai::SubmitCmd(true);
    const double t0 = now_ms();
    for (uint32_t pos = FIRST; pos < LAST; ++pos) {
        put_ids(*m.in, toks.data(), false);
        m.g.eval(false, false, false);
        evk::ai::greedy_sample(*m.logits, sampled, pos, BASE, BINS);
        sampled.cpu_download(false);
        evk::ai::SubmitCmd(true);
        for (uint32_t b = 0; b < B; ++b) toks[b * S + pos + 1] = sampled.cpu()[b].value;
    }
    return now_ms() - t0;
}

// KVCacheDecoder over the same positions; host_ids: download the ids every
// step (the reference loop's pattern), else feed them on the device.
double run_kv(Model& m, evk::ai::KVCacheDecoder& dec, std::vector<uint16_t>& toks, bool host_ids, bool fused = true) {
    dec.set_fused(fused);
    Tensor pre({B, PROMPT}), ids_a({B}), ids_b({B});
    std::vector<uint16_t> p(B * PROMPT), first(B);
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t i = 0; i < PROMPT; ++i) p[b * PROMPT + i] = toks[b * S + i];
        first[b] = toks[b * S + FIRST];
    }
    put_ids(pre, p.data());
    put_ids(ids_a, first.data());
    evk::ai::SubmitCmd(true);
    const double t0 = now_ms();
    dec.reset();
    dec.prefill(pre);
    Tensor* cur = &ids_a;
    Tensor* nxt = &ids_b;
    for (uint32_t pos = FIRST; pos < LAST; ++pos) {
        Tensor& lg = dec.step(*cur);
        evk::ai::greedy_sample(lg, *nxt, 0, BASE, BINS);
        if (host_ids) {
            nxt->cpu_download(false);
            evk::ai::SubmitCmd(true);
            for (uint32_t b = 0; b < B; ++b) toks[b * S + pos + 1] = nxt->cpu()[b].value;
        }
        std::swap(cur, nxt);
    }
    evk::ai::SubmitCmd(true);
    return now_ms() - t0;
}

int bench(int reps) {
    Model m;
    evk::ai::KVCacheDecoder dec(*m.emb, *m.w_out, m.layers, B, S);
    const std::vector<uint16_t> base_toks = make_tokens();
    auto best = [&](auto fn) {
        double b = 1e30;
        for (int r = 0; r < reps + 1; ++r) {  // the first run warms up
            std::vector<uint16_t> t = base_toks;
            const double ms = fn(t);
            if (r > 0) b = std::fmin(b, ms);
        }
        return b;
    };
    const double full = best([&](std::vector<uint16_t>& t) { return run_full(m, t); });
    const double kvh = best([&](std::vector<uint16_t>& t) { return run_kv(m, dec, t, true); });
    const double kvd = best([&](std::vector<uint16_t>& t) { return run_kv(m, dec, t, false); });
    const double kvo = best([&](std::vector<uint16_t>& t) { return run_kv(m, dec, t, false, false); });
    const double n_tok = double(B) * (LAST - FIRST);
    std::printf("{\"workload\": \"example/main_llm.cpp sample_autoregressive: B=%u, D=%u (1 head), hidden %u, "
                "%u layers, vocab %u, positions %u..%u\", \"ids_per_sequence\": %u, "
                "\"full_recompute_ms\": %.3f, \"full_recompute_tokens_per_s\": %.1f, "
                "\"kv_host_ids_ms\": %.3f, \"kv_host_ids_tokens_per_s\": %.1f, "
                "\"kv_device_ids_ms\": %.3f, \"kv_device_ids_tokens_per_s\": %.1f, "
                "\"kv_op_by_op_ms\": %.3f, \"kv_op_by_op_tokens_per_s\": %.1f, "
                "\"speedup_kv_host_ids\": %.2f, \"speedup_kv_device_ids\": %.2f, \"step\": \"fused: one launch "
                "per position (evkhip_kv_decode_step); op_by_op: 16 launches a layer\", \"timing\": \"best of %d "
                "runs after one warm-up, host wall clock around the whole loop\"}\n",
                B, D, HID, L, V, FIRST, LAST - 1, LAST - FIRST, full, n_tok / (full * 1e-3), kvh,
                n_tok / (kvh * 1e-3), kvd, n_tok / (kvd * 1e-3), kvo, n_tok / (kvo * 1e-3), full / kvh, full / kvd,
                reps);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: kv_decoder_tool dump <dir> [steps] | bench [reps]\n");
        return 2;
    }
    const std::string mode = argv[1];
    evk::ai::initialize();
    int rc = 2;
    if (mode == "dump" && argc >= 3) rc = dump(argv[2], argc >= 4 ? uint32_t(std::atoi(argv[3])) : 32u);
    else if (mode == "bench") rc = bench(argc >= 3 ? std::max(1, std::atoi(argv[2])) : 3);
    else std::fprintf(stderr, "usage: kv_decoder_tool dump <dir> [steps] | bench [reps]\n");
    evk::ai::shutdown();
    return rc;
}
