// Tests of the C++ host API (cpp_inference_train_engine_amd/host/mla_host.hpp), written
// the way the reference tests its backends: an execution's prefill / decode logits
// against the CPU decoder (tests/test_mps.cpp:126-166, here the oracle's restatement of
// CpuDecoder, oracle/mla_oracle.h), the sampler's known answers
// (tests/test_training.cpp:77-110), tokenizer round trips (tests/test_files.cpp:68-107),
// and the engine / server on a model export.
//
//   test_host --cpu <golden dir>                 host-only tests (no GPU)
//   test_host --gpu <golden dir> <export dir>    everything
#include "mla_host.hpp"
#include "mla_oracle.h"

#include <algorithm>
#include <cmath>
#include <span>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

using namespace mla_host;

namespace {

int failures = 0;
std::string golden, export_dir;

#define CHECK(cond)                                                                  \
    do {                                                                             \
        if (!(cond)) {                                                               \
            std::printf("  CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                              \
        }                                                                            \
    } while (0)
#define REQUIRE(cond)                                                                  \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            std::printf("  REQUIRE failed at %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                                \
            return;                                                                    \
        }                                                                              \
    } while (0)

struct Test {
    const char* name;
    bool gpu;
    std::function<void()> fn;
};
std::vector<Test>& registry() {
    static std::vector<Test> r;
    return r;
}
struct Register {
    Register(const char* n, bool gpu, std::function<void()> f) { registry().push_back({n, gpu, std::move(f)}); }
};
#define HOST_TEST(name, gpu)                              \
    void name();                                          \
    const Register reg_##name(#name, gpu, name);          \
    void name()

// tiny-test (config/tiny-test.json of the reference).
ModelConfig tiny() {
    ModelConfig c{};
    c.vocab_size = 264;
    c.max_sequence_length = 64;
    c.n_layers = 2;
    c.d_model = 32;
    c.n_heads = 2;
    c.head_dim_nope = 12;
    c.head_dim_rope = 4;
    c.head_dim_value = 16;
    c.q_lora_rank = 16;
    c.kv_lora_rank = 8;
    c.d_ff = 64;
    c.norm_epsilon = 1e-5F;
    c.rope_theta = 10000.0F;
    return c;
}
orc_config as_orc(const ModelConfig& m) {
    orc_config c{};
    std::memcpy(&c, &m, sizeof(c));
    return c;
}

// Model::create(seed) weights rounded through fp16, the values the device holds.
std::vector<float> tiny_params(const ModelConfig& m, uint64_t seed) {
    const orc_config c = as_orc(m);
    std::vector<float> p(orc_parameter_count(&c));
    orc_model_init(&c, seed, p.data());
    for (float& x : p)
        x = orc_f16_to_f32(orc_f32_to_f16(x));
    return p;
}

// CpuDecoder over the oracle (inference.cpp:47-174): prefill runs the full forward and
// keeps its cache rows (rounded to fp16, as the device cache holds them); decode appends.
struct CpuDecoder {
    orc_config c;
    const std::vector<float>& params;
    std::vector<float> proj, latent, rope, logits;
    int position = 0;
    CpuDecoder(const ModelConfig& m, const std::vector<float>& p)
        : c(as_orc(m)), params(p),
          proj((size_t)m.n_layers * m.n_heads * m.kv_lora_rank * m.d_model),
          latent((size_t)m.n_layers * m.max_sequence_length * m.kv_lora_rank),
          rope((size_t)m.n_layers * m.max_sequence_length * m.head_dim_rope),
          logits((size_t)m.vocab_size) {
        orc_output_projection(&c, params.data(), proj.data());
    }
    const std::vector<float>& decode(uint16_t t) {
        orc_decode(&c, params.data(), proj.data(), latent.data(), rope.data(), position++, t, 1, 1,
                   logits.data());
        return logits;
    }
    const std::vector<float>& prefill(const std::vector<uint16_t>& ids) {
        const int T = (int)ids.size(), L = c.n_layers, kv = c.kv_lora_rank, rp = c.head_dim_rope;
        const size_t S = (size_t)c.max_sequence_length;
        std::vector<float> all((size_t)T * c.vocab_size), ckv((size_t)L * T * kv),
            kr((size_t)L * T * rp);
        orc_forward(&c, params.data(), ids.data(), T, all.data(), ckv.data(), kr.data());
        auto h = [](float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); };
        for (int l = 0; l < L; ++l)
            for (int t = 0; t < T; ++t) {
                for (int j = 0; j < kv; ++j)
                    latent[((size_t)l * S + t) * kv + j] = h(ckv[((size_t)l * T + t) * kv + j]);
                for (int j = 0; j < rp; ++j)
                    rope[((size_t)l * S + t) * rp + j] = h(kr[((size_t)l * T + t) * rp + j]);
            }
        std::copy(all.end() - c.vocab_size, all.end(), logits.begin());
        position = T;
        return logits;
    }
};

float max_abs_diff(std::span<const float> a, const std::vector<float>& b) {
    float m = 0;
    for (size_t i = 0; i < b.size(); ++i)
        m = std::max(m, std::fabs(a[i] - b[i]));
    return m;
}

std::vector<uint16_t> prompt_ids(int n, int vocab, uint64_t seed) {
    std::vector<uint16_t> ids;
    for (int i = 0; i < n; ++i)
        ids.push_back((uint16_t)orc_rng_bounded(&seed, (uint64_t)vocab));
    return ids;
}

// ------------------------------------------------------------------ host ----
HOST_TEST(sampling_is_seeded_and_respects_filters, false) {  // test_training.cpp:77-110
    const float scores[] = {2, -1, 1, 0};
    GenerationConfig c;
    c.temperature = 0;
    uint64_t rng = 1;
    auto greedy = sample_token(scores, {}, c, rng);
    REQUIRE(greedy);
    CHECK(greedy.value() == 0);
    c.repetition_penalty = 3;
    const uint16_t history[] = {0, 0};
    auto penalized = sample_token(scores, history, c, rng);
    REQUIRE(penalized);
    CHECK(penalized.value() == 2);
    c.temperature = 0.7F;
    c.top_k = 1;
    c.repetition_penalty = 1;
    for (int i = 0; i < 30; ++i) {
        auto id = sample_token(scores, {}, c, rng);
        REQUIRE(id);
        CHECK(id.value() == 0);
    }
    c.top_k = 0;
    c.top_p = 1;
    uint64_t a = 99, b = 99;
    for (int i = 0; i < 50; ++i) {
        auto x = sample_token(scores, {}, c, a), y = sample_token(scores, {}, c, b);
        REQUIRE(x && y);
        CHECK(x.value() == y.value());
    }
    const uint16_t banned[] = {0, 1, 2, 3};
    auto none = sample_token(scores, {}, c, rng, banned);
    CHECK(!none && none.error().code == ErrorCode::invalid_argument);
    c.top_p = 0;
    CHECK(!sample_token(scores, {}, c, rng));
    CHECK(!c.validate());
}

HOST_TEST(tokenizer_round_trips_and_specials, false) {  // test_files.cpp:68-86
    auto t = Tokenizer::load(golden + "/tokenizer_tiny.json");
    REQUIRE(t);
    const Tokenizer& tok = *t.value();
    CHECK(tok.vocab_size() == 264 && tok.hash().size() == 64);
    const std::string text = "Hello, caf\xc3\xa9 <|eos|>";
    auto ids = tok.encode(text);
    REQUIRE(ids && ids.value().size() == text.size());
    auto back = tok.decode(ids.value());
    CHECK(back && back.value() == text);
    auto sp = tok.encode("<|eos|>", true);
    CHECK(sp && sp.value().size() == 1 && sp.value()[0] == tok.special("<|eos|>"));
    CHECK(tok.special("<|bos|>") == 257);
    const uint16_t unknown[] = {300};
    auto bad = tok.decode(unknown);
    CHECK(!bad && bad.error().code == ErrorCode::invalid_argument);
    auto missing = Tokenizer::load(golden + "/no-such-tokenizer.json");
    CHECK(!missing && missing.error().code == ErrorCode::io_error);
}

HOST_TEST(config_errors_use_reference_codes, false) {
    ModelConfig c = tiny();
    c.head_dim_rope = 3;  // RoPE needs an even dimension
    auto e = HipEngine::create(c, std::vector<float>(10), {});
    CHECK(!e && e.error().code == ErrorCode::invalid_argument);
}

// ------------------------------------------------------------------- GPU ----
HOST_TEST(hip_execution_matches_cpu_decoder, true) {  // test_mps.cpp:126-166
    const ModelConfig m = tiny();
    const std::vector<float> params = tiny_params(m, 0);
    auto engine = HipEngine::create(m, params, {4, 64, 32, 16});
    REQUIRE(engine);
    auto exec = make_hip_execution(engine.value());
    REQUIRE(exec);
    Execution& x = *exec.value();
    CHECK(x.attention_name() == "paged-mla");
    CpuDecoder cpu(m, params);
    const std::vector<uint16_t> prompt = prompt_ids(32, m.vocab_size, 0);
    auto out = x.prefill(prompt);
    REQUIRE(out);
    float worst = max_abs_diff(out.value(), cpu.prefill(prompt));
    for (int i = 0; i < 16; ++i) {
        const auto& want = cpu.logits;
        const uint16_t t = (uint16_t)(std::max_element(want.begin(), want.end()) - want.begin());
        out = x.decode(t);
        REQUIRE(out);
        worst = std::max(worst, max_abs_diff(out.value(), cpu.decode(t)));
    }
    std::printf("  max |hip - cpu| over prefill + 16 decodes: %.3g\n", worst);
    CHECK(worst < 5e-3F);
}

HOST_TEST(weight_changes_invalidate_decode_cache, true) {  // test_training.cpp:111-122
    const ModelConfig m = tiny();
    std::vector<float> params = tiny_params(m, 9);
    auto engine = HipEngine::create(m, params, {4, 64, 32, 16});
    REQUIRE(engine);
    auto exec = make_execution(engine.value(), "hip");  // the reference's default, "fp32"
    REQUIRE(exec);
    Execution& x = *exec.value();
    const std::vector<uint16_t> ids = {1, 2, 3};
    REQUIRE(x.prefill(ids));
    params[0] += 0.01F;
    REQUIRE(engine.value()->update_weights(params));
    auto stale = x.decode(4);
    CHECK(!stale && stale.error().code == ErrorCode::invalid_argument);
    REQUIRE(x.prefill(ids));
    auto fresh = x.decode(4);
    REQUIRE(fresh);
    CpuDecoder cpu(m, params);
    cpu.prefill(ids);
    CHECK(max_abs_diff(fresh.value(), cpu.decode(4)) < 5e-3F);
    auto bad = make_execution(engine.value(), "hip", "bf16");
    CHECK(!bad && bad.error().code == ErrorCode::unsupported);
    auto other = make_execution(engine.value(), "mps");
    CHECK(!other && other.error().code == ErrorCode::unsupported);
}

HOST_TEST(forward_and_stats, true) {  // execution.hpp:25-39, bench_main.cpp:358-396
    const ModelConfig m = tiny();
    const std::vector<float> params = tiny_params(m, 4);
    auto engine = HipEngine::create(m, params, {4, 64, 32, 16});
    REQUIRE(engine);
    auto exec = make_execution(engine.value(), "hip", "fp16");
    REQUIRE(exec);
    Execution& x = *exec.value();
    std::vector<uint16_t> ids = prompt_ids(24, m.vocab_size, 11);
    const ExecutionStats before = x.stats();
    auto full = x.forward(ids, 2, 12);
    REQUIRE(full);
    const Matrix& f = *full.value();
    CHECK(f.rows == 24 && f.cols == m.vocab_size);
    // sequence 1 on its own: its prefill gives row 23 (the last of the second sequence)
    auto out = x.prefill(std::span<const uint16_t>(ids).subspan(12, 11));
    REQUIRE(out);
    auto step = x.decode(ids[23]);
    REQUIRE(step);
    float worst = 0;
    for (int j = 0; j < m.vocab_size; ++j)
        worst = std::max(worst, std::abs(step.value()[(std::size_t)j] - f(23, j)));
    std::printf("  decode vs forward row: %.3g\n", worst);
    CHECK(worst < 5e-3F);
    const ExecutionStats after = x.stats();
    CHECK(after.graph_submissions - before.graph_submissions == 3);  // forward, prefill, decode
    CHECK(after.host_waits - before.host_waits == 3);
    CHECK(after.metal_kernel_submissions > before.metal_kernel_submissions);
}

HOST_TEST(forks_share_weights_and_reject_bad_input, true) {
    const ModelConfig m = tiny();
    const std::vector<float> params = tiny_params(m, 1);
    auto engine = HipEngine::create(m, params, {4, 64, 32, 16});
    REQUIRE(engine);
    auto a = engine.value()->session();
    REQUIRE(a);
    auto b = a.value()->fork_inference();
    REQUIRE(b);
    const std::vector<uint16_t> prompt = prompt_ids(20, m.vocab_size, 7);
    auto la = a.value()->prefill(prompt);
    REQUIRE(la);
    const std::vector<float> first(la.value().begin(), la.value().end());
    auto lb = b.value()->prefill(prompt);
    REQUIRE(lb);
    CHECK(max_abs_diff(lb.value(), first) == 0.0F);
    auto too_big = a.value()->decode((uint16_t)m.vocab_size);
    CHECK(!too_big && too_big.error().code == ErrorCode::invalid_argument);
    auto c = engine.value()->session();
    REQUIRE(c);
    auto empty = c.value()->decode(1);  // nothing cached yet (inference.cpp:71-75)
    CHECK(!empty && empty.error().code == ErrorCode::invalid_argument);
    auto none = c.value()->prefill({});
    CHECK(!none && none.error().code == ErrorCode::invalid_argument);
}

HOST_TEST(batched_step_equals_single_sessions, true) {
    const ModelConfig m = tiny();
    const std::vector<float> params = tiny_params(m, 2);
    auto engine = HipEngine::create(m, params, {8, 64, 48, 16});
    REQUIRE(engine);
    HipEngine& e = *engine.value();
    std::vector<std::vector<uint16_t>> prompts;
    for (int k = 0; k < 4; ++k)
        prompts.push_back(prompt_ids(1 + 9 * k, m.vocab_size, 30 + (uint64_t)k));
    std::vector<std::unique_ptr<Execution>> solo, batch;
    std::vector<std::vector<float>> want;
    for (const auto& p : prompts) {
        auto a = e.session(), b = e.session();
        REQUIRE(a && b);
        auto l = a.value()->prefill(p);
        REQUIRE(l);
        want.emplace_back(l.value().begin(), l.value().end());
        solo.push_back(std::move(a).value());
        batch.push_back(std::move(b).value());
    }
    // sessions 0 and 1 prefilled alone, then one step: their decodes beside 2 and 3's prompts
    REQUIRE(batch[0]->prefill(prompts[0]) && batch[1]->prefill(prompts[1]));
    const std::vector<std::vector<uint16_t>> chunks = {{7}, {9}, prompts[2], prompts[3]};
    for (int k = 0; k < 2; ++k) {
        auto l = solo[(size_t)k]->decode(chunks[(size_t)k][0]);
        REQUIRE(l);
        want[(size_t)k].assign(l.value().begin(), l.value().end());
    }
    std::vector<Execution*> raw;
    for (auto& b : batch)
        raw.push_back(b.get());
    std::vector<float> logits;
    std::vector<int32_t> next;
    REQUIRE(e.step(raw, chunks, &logits, &next));
    float worst = 0;
    for (size_t k = 0; k < 4; ++k)
        worst = std::max(worst, max_abs_diff(std::span<const float>(logits).subspan(
                                                 k * (size_t)m.vocab_size, (size_t)m.vocab_size),
                                             want[k]));
    CHECK(worst <= 1e-5F);
    CHECK(next.size() == 4);
    std::vector<Execution*> wrong = {raw[0], raw[0]};  // a session twice
    CHECK(!e.step(wrong, std::vector<std::vector<uint16_t>>{{1}, {2}}, nullptr, nullptr));
}

HOST_TEST(inference_engine_and_server_on_an_export, true) {
    auto loaded = InferenceEngine::load(export_dir, {8, 64, 64, 16});
    REQUIRE(loaded);
    InferenceEngine& eng = *loaded.value();
    // generate = <|bos|> + encode(prompt), then generate_tokens; greedy with the banned ids
    GenerationConfig greedy;
    greedy.max_new_tokens = 12;
    greedy.temperature = 0;
    // (streamed chunks are cleaned one by one, so they are compared with another run's
    // chunks, not with the text cleaned as a whole)
    std::string streamed, streamed_again;
    auto g = eng.generate("Say hi.", greedy, [&](std::string_view s) {
        streamed += s;
        return true;
    });
    REQUIRE(g);
    CHECK(g.value().prompt_tokens == 8);
    // the same loop by hand on a fork: prefill, greedy over host logits, decode
    auto fork = eng.fork();
    REQUIRE(fork);
    auto ids = eng.tokenizer().encode("Say hi.");
    REQUIRE(ids);
    ids.value().insert(ids.value().begin(), eng.tokenizer().special("<|bos|>"));
    auto again = fork.value()->generate_tokens(ids.value(), greedy, [&](std::string_view s) {
        streamed_again += s;
        return true;
    });
    REQUIRE(again);
    CHECK(again.value().tokens == g.value().tokens);
    CHECK(again.value().text == g.value().text);
    CHECK(streamed_again == streamed);
    CHECK(again.value().finish_reason == g.value().finish_reason);
    // the server: batched requests give what each gets alone
    auto tok = Tokenizer::load(export_dir + "/tokenizer.json");
    REQUIRE(tok);
    auto server = Server::create(eng.engine(), tok.value(), {64, 16, 8, 30});
    REQUIRE(server);
    std::vector<GenerationConfig> cfgs(4);
    std::vector<std::vector<uint16_t>> prompts;
    std::vector<uint64_t> ids_out;
    for (int k = 0; k < 4; ++k) {
        cfgs[k].max_new_tokens = 6 + 2 * k;
        cfgs[k].temperature = k % 2 ? 0.9F : 0.0F;
        cfgs[k].seed = 11 + (uint64_t)k;
        std::vector<uint16_t> p = prompt_ids(3 + 5 * k, 256, 100 + (uint64_t)k);
        p.insert(p.begin(), eng.tokenizer().special("<|bos|>"));
        prompts.push_back(p);
        auto id = server.value()->submit(p, cfgs[k], k % 2 == 0, cfgs[k].max_new_tokens);
        REQUIRE(id);
        ids_out.push_back(id.value());
    }
    auto over = server.value()->submit(prompts[0], cfgs[0], false, 17);  // > max_new_tokens 16
    CHECK(!over && over.error().code == ErrorCode::invalid_argument);
    for (int k = 0; k < 4; ++k) {
        std::string text;
        RequestStatus st;
        for (int tries = 0; tries < 600 && !st.done; ++tries) {
            auto r = server.value()->poll(ids_out[k], 100);
            REQUIRE(r);
            text += r.value().first;
            st = std::move(r.value().second);
        }
        REQUIRE(st.done && !st.error);
        auto solo = eng.fork();
        REQUIRE(solo);
        std::string chunks;
        auto want = solo.value()->generate_tokens(prompts[k], cfgs[k], [&](std::string_view s) {
            chunks += s;
            return true;
        });
        REQUIRE(want);
        CHECK(st.tokens == want.value().tokens);
        CHECK(text == (k % 2 == 0 ? chunks : want.value().text));  // streamed: the chunks
        CHECK(st.finish_reason == want.value().finish_reason);
    }
    auto metrics = server.value()->metrics_text();
    REQUIRE(metrics);
    CHECK(metrics.value().find("mini_mla_completed_total 4\n") != std::string::npos);
    CHECK(metrics.value().find("mini_mla_errors_total 1\n") != std::string::npos);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3 || (std::strcmp(argv[1], "--cpu") && std::strcmp(argv[1], "--gpu")) ||
        (!std::strcmp(argv[1], "--gpu") && argc < 4)) {
        std::fprintf(stderr, "usage: %s --cpu GOLDEN | --gpu GOLDEN EXPORT_DIR\n", argv[0]);
        return 2;
    }
    const bool gpu = !std::strcmp(argv[1], "--gpu");
    golden = argv[2];
    if (gpu)
        export_dir = argv[3];
    int run = 0;
    for (const Test& t : registry()) {
        if (t.gpu && !gpu)
            continue;
        const int before = failures;
        std::printf("%s\n", t.name);
        std::fflush(stdout);
        t.fn();
        std::printf("%s %s\n", failures == before ? "PASS" : "FAIL", t.name);
        std::fflush(stdout);
        ++run;
    }
    std::printf("%d tests, %d failed checks\n", run, failures);
    return failures ? 1 : 0;
}
