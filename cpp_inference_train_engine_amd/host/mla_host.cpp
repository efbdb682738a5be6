// C++ host API over the C ABI: see mla_host.hpp.
#include "mla_host.hpp"

#include <chrono>
#include <cstring>

namespace mla_host {

Status check(int status) {
    if (status == MLA_OK)
        return ok();
    return Status::failure(static_cast<ErrorCode>(status - 1), mla_last_error());
}

namespace {

template <typename T>
Result<T> fail_as(const Status& s) {
    return Result<T>::failure(s.error());
}

double ms_since(std::chrono::steady_clock::time_point t) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

// A GenerationConfig as the C struct, with the arrays it points into.
struct CConfig {
    mla_generation_config c{};
    std::vector<const char*> stop;
    std::vector<size_t> stop_len;
    std::vector<int> seq_len;
    std::vector<uint16_t> seq;
    explicit CConfig(const GenerationConfig& g) {
        c.max_new_tokens = g.max_new_tokens;
        c.top_k = g.top_k;
        c.temperature = g.temperature;
        c.top_p = g.top_p;
        c.repetition_penalty = g.repetition_penalty;
        c.seed = g.seed;
        for (const std::string& s : g.stop) {
            stop.push_back(s.data());
            stop_len.push_back(s.size());
        }
        for (const auto& q : g.stop_tokens) {
            seq_len.push_back((int)q.size());
            seq.insert(seq.end(), q.begin(), q.end());
        }
        c.n_stop = (int)stop.size();
        c.stop = stop.data();
        c.stop_len = stop_len.data();
        c.n_stop_tokens = (int)seq_len.size();
        c.stop_tokens_len = seq_len.data();
        c.stop_tokens = seq.data();
    }
};

class HipExecution final : public Execution {
  public:
    HipExecution(std::shared_ptr<HipEngine> engine, int session)
        : engine_(std::move(engine)), session_(session),
          logits_((size_t)engine_->config().vocab_size) {}
    ~HipExecution() override { (void)mla_session_release(engine_->handle(), session_); }
    std::string device_name() const override { return "HIP / MI355X (gfx950)"; }
    std::string attention_name() const override { return "paged-mla"; }
    ExecutionStats stats() const override { return engine_->stats(); }
    Result<std::unique_ptr<Execution>> fork_inference() override { return engine_->session(); }
    Result<const Matrix*> forward(std::span<const std::uint16_t> ids, int batch,
                                  int sequence) override {
        const Status s = engine_->forward(ids, batch, sequence, output_);
        if (!s)
            return fail_as<const Matrix*>(s);
        return Result<const Matrix*>::success(&output_);
    }
    Result<std::span<const float>> prefill(std::span<const std::uint16_t> ids) override {
        const Status s = check(mla_session_prefill(engine_->handle(), session_, ids.data(),
                                                   (int)std::min<size_t>(ids.size(), 1u << 30),
                                                   logits_.data()));
        if (!s)
            return fail_as<std::span<const float>>(s);
        return Result<std::span<const float>>::success(logits_);
    }
    [[nodiscard]] int session() const { return session_; }
    [[nodiscard]] const HipEngine* engine() const { return engine_.get(); }
    Result<std::span<const float>> decode(std::uint16_t token) override {
        const Status s = check(mla_session_decode(engine_->handle(), session_, token, logits_.data()));
        if (!s)
            return fail_as<std::span<const float>>(s);
        return Result<std::span<const float>>::success(logits_);
    }

  private:
    std::shared_ptr<HipEngine> engine_;
    int session_;
    std::vector<float> logits_;
    Matrix output_;  // forward's logits, valid until the next forward
};

int text_callback(void* user, const char* text, size_t len) {
    auto* f = static_cast<std::function<bool(std::string_view)>*>(user);
    try {
        return (*f)(std::string_view(text, len)) ? 1 : 0;
    } catch (...) {
        return 0;  // an exception in the callback cancels
    }
}

}  // namespace

// ------------------------------------------------------------------ engine ----
Result<std::shared_ptr<HipEngine>> HipEngine::create(const ModelConfig& config,
                                                     std::span<const float> params,
                                                     const EngineLimits& lim) {
    using R = Result<std::shared_ptr<HipEngine>>;
    if (const Status s = check(mla_config_validate(&config)); !s)
        return fail_as<std::shared_ptr<HipEngine>>(s);
    if (params.size() != mla_config_parameter_count(&config))
        return R::failure(ErrorCode::invalid_argument, "Parameter count does not match the model");
    std::shared_ptr<HipEngine> e(new HipEngine());
    e->config_ = config;
    const Status s = check(mla_engine_create(&config, params.data(), lim.max_sessions,
                                             lim.max_rows, lim.num_pages, lim.page_size, &e->h_));
    if (!s)
        return fail_as<std::shared_ptr<HipEngine>>(s);
    return R::success(std::move(e));
}

Result<std::shared_ptr<HipEngine>> HipEngine::load(const std::string& path, const EngineLimits& lim) {
    std::shared_ptr<HipEngine> e(new HipEngine());
    const Status s = check(mla_engine_load(path.c_str(), lim.max_sessions, lim.max_rows,
                                           lim.num_pages, lim.page_size, &e->config_, &e->h_));
    if (!s)
        return fail_as<std::shared_ptr<HipEngine>>(s);
    return Result<std::shared_ptr<HipEngine>>::success(std::move(e));
}

HipEngine::~HipEngine() {
    if (h_)
        (void)mla_engine_destroy(h_);
}

Result<std::unique_ptr<Execution>> HipEngine::session() {
    int id = -1;
    const Status s = check(mla_session_create(h_, &id));
    if (!s)
        return fail_as<std::unique_ptr<Execution>>(s);
    return Result<std::unique_ptr<Execution>>::success(
        std::make_unique<HipExecution>(shared_from_this(), id));
}

Status HipEngine::set_banned(std::span<const std::uint16_t> ids) {
    return check(mla_engine_set_banned(h_, ids.data(), ids.size()));
}

Status HipEngine::update_weights(std::span<const float> params) {
    if (params.size() != mla_config_parameter_count(&config_))
        return Status::failure(ErrorCode::invalid_argument, "Parameter count does not match the model");
    return check(mla_engine_update_weights(h_, params.data()));
}

ExecutionStats HipEngine::stats() const {
    std::uint64_t v[6] = {};
    if (mla_engine_stats(h_, v) != MLA_OK)
        return {};
    return ExecutionStats{v[0], v[1], v[2]};
}

Status HipEngine::forward(std::span<const std::uint16_t> ids, int batch, int sequence,
                          Matrix& out) {
    if (batch < 1 || sequence < 1 || ids.size() != (std::size_t)batch * (std::size_t)sequence)
        return Status::failure(ErrorCode::invalid_argument,
                               "Forward requires batch * sequence token ids");
    out.rows = batch * sequence;
    out.cols = config_.vocab_size;
    out.values.resize((std::size_t)out.rows * (std::size_t)out.cols);
    return check(mla_engine_forward(h_, batch, sequence, ids.data(), out.values.data()));
}

Status HipEngine::step(std::span<Execution* const> sessions,
                       std::span<const std::vector<std::uint16_t>> tokens,
                       std::vector<float>* logits, std::vector<std::int32_t>* next_tokens) {
    if (sessions.size() != tokens.size())
        return Status::failure(ErrorCode::invalid_argument, "step: one token list per session");
    std::vector<int> ids, counts;
    std::vector<std::uint16_t> flat;
    for (size_t i = 0; i < sessions.size(); ++i) {
        const auto* x = dynamic_cast<const HipExecution*>(sessions[i]);
        if (!x || x->engine() != this)
            return Status::failure(ErrorCode::invalid_argument,
                                   "step: a session of another engine or backend");
        ids.push_back(x->session());
        counts.push_back((int)tokens[i].size());
        flat.insert(flat.end(), tokens[i].begin(), tokens[i].end());
    }
    const size_t n = ids.size();
    if (logits)
        logits->assign(n * (size_t)config_.vocab_size, 0.0f);
    if (next_tokens)
        next_tokens->assign(n, 0);
    return check(mla_engine_step(h_, (int)n, ids.data(), counts.data(), flat.data(),
                                 logits ? logits->data() : nullptr,
                                 next_tokens ? next_tokens->data() : nullptr));
}

Result<std::unique_ptr<Execution>> make_hip_execution(const std::shared_ptr<HipEngine>& engine) {
    if (!engine)
        return Result<std::unique_ptr<Execution>>::failure(ErrorCode::invalid_argument,
                                                           "make_hip_execution: null engine");
    return engine->session();
}

Result<std::unique_ptr<Execution>> make_execution(const std::shared_ptr<HipEngine>& engine,
                                                  std::string_view backend,
                                                  std::string_view precision) {
    if (backend != "hip")  // an unknown backend is unsupported, as in inference.cpp:320-322
        return Result<std::unique_ptr<Execution>>::failure(ErrorCode::unsupported,
                                                           "Select hip/fp32|fp16");
    if (precision != "fp32" && precision != "fp16")
        return Result<std::unique_ptr<Execution>>::failure(ErrorCode::unsupported,
                                                           "HIP precision must be fp32 or fp16");
    return make_hip_execution(engine);
}

// --------------------------------------------------------------- tokenizer ----
Result<std::shared_ptr<const Tokenizer>> Tokenizer::load(const std::string& path) {
    std::shared_ptr<Tokenizer> t(new Tokenizer());
    Status s = check(mla_tokenizer_load(path.c_str(), &t->h_));
    char hex[65] = {};
    if (s)
        s = check(mla_tokenizer_info(t->h_, &t->vocab_, hex));
    if (!s)
        return fail_as<std::shared_ptr<const Tokenizer>>(s);
    t->hash_ = hex;
    return Result<std::shared_ptr<const Tokenizer>>::success(std::move(t));
}

Tokenizer::~Tokenizer() {
    if (h_)
        (void)mla_tokenizer_destroy(h_);
}

Result<std::vector<std::uint16_t>> Tokenizer::encode(std::string_view text, bool allow_special) const {
    size_t n = 0;
    Status s = check(mla_tokenizer_encode(h_, text.data(), text.size(), allow_special, nullptr, 0, &n));
    std::vector<std::uint16_t> ids(n);
    if (s)
        s = check(mla_tokenizer_encode(h_, text.data(), text.size(), allow_special, ids.data(),
                                       ids.size(), &n));
    if (!s)
        return fail_as<std::vector<std::uint16_t>>(s);
    return Result<std::vector<std::uint16_t>>::success(std::move(ids));
}

Result<std::string> Tokenizer::decode(std::span<const std::uint16_t> ids, bool skip_special) const {
    size_t n = 0;
    Status s = check(mla_tokenizer_decode(h_, ids.data(), ids.size(), skip_special, nullptr, 0, &n));
    std::string out(n, '\0');
    if (s)
        s = check(mla_tokenizer_decode(h_, ids.data(), ids.size(), skip_special, out.data(),
                                       out.size(), &n));
    if (!s)
        return fail_as<std::string>(s);
    return Result<std::string>::success(std::move(out));
}

std::uint16_t Tokenizer::special(std::string_view name) const {
    std::uint16_t id = 0xffff;  // unknown names: an id past every vocabulary
    (void)mla_tokenizer_special(h_, std::string(name).c_str(), &id);
    return id;
}

// -------------------------------------------------------------- generation ----
Status GenerationConfig::validate() const {
    const CConfig c(*this);
    return check(mla_generation_config_validate(&c.c));
}

Result<std::uint16_t> sample_token(std::span<const float> logits,
                                   std::span<const std::uint16_t> history,
                                   const GenerationConfig& config, std::uint64_t& rng_state,
                                   std::span<const std::uint16_t> banned) {
    const CConfig c(config);
    std::uint16_t token = 0;
    const Status s = check(mla_sample_token(logits.data(), logits.size(), history.data(),
                                            history.size(), &c.c, &rng_state, banned.data(),
                                            banned.size(), &token));
    if (!s)
        return fail_as<std::uint16_t>(s);
    return Result<std::uint16_t>::success(token);
}

Result<std::unique_ptr<InferenceEngine>> InferenceEngine::load(const std::string& path,
                                                               const EngineLimits& lim) {
    auto engine = HipEngine::load(path, lim);
    if (!engine)
        return Result<std::unique_ptr<InferenceEngine>>::failure(engine.error());
    auto tok = Tokenizer::load(path + "/tokenizer.json");
    if (!tok)
        return Result<std::unique_ptr<InferenceEngine>>::failure(tok.error());
    return create(std::move(engine).value(), std::move(tok).value());
}

Result<std::unique_ptr<InferenceEngine>> InferenceEngine::create(
    std::shared_ptr<HipEngine> engine, std::shared_ptr<const Tokenizer> tokenizer) {
    using R = Result<std::unique_ptr<InferenceEngine>>;
    if (!engine || !tokenizer)
        return R::failure(ErrorCode::invalid_argument, "InferenceEngine: null engine or tokenizer");
    if (tokenizer->vocab_size() != engine->config().vocab_size)
        return R::failure(ErrorCode::invalid_argument, "Checkpoint tokenizer mismatch");
    auto session = engine->session();
    if (!session)
        return R::failure(session.error());
    std::unique_ptr<InferenceEngine> e(new InferenceEngine());
    e->engine_ = std::move(engine);
    e->tokenizer_ = std::move(tokenizer);
    e->execution_ = std::move(session).value();
    return R::success(std::move(e));
}

Result<std::unique_ptr<InferenceEngine>> InferenceEngine::fork() {
    return create(engine_, tokenizer_);
}

Result<Generation> InferenceEngine::generate(std::string_view prompt, const GenerationConfig& c,
                                             std::function<bool(std::string_view)> callback) {
    auto ids = tokenizer_->encode(prompt);
    if (!ids)
        return Result<Generation>::failure(ids.error());
    ids.value().insert(ids.value().begin(), tokenizer_->special("<|bos|>"));
    return generate_tokens(ids.value(), c, std::move(callback));
}

Result<Generation> InferenceEngine::generate_tokens(std::span<const std::uint16_t> prompt,
                                                    const GenerationConfig& c,
                                                    std::function<bool(std::string_view)> callback) {
    using R = Result<Generation>;
    const CConfig cc(c);
    void* g = nullptr;
    Status s = check(mla_generation_create(tokenizer_->handle(), &cc.c, prompt.data(),
                                           prompt.size(), config().max_sequence_length,
                                           callback ? &text_callback : nullptr,
                                           callback ? &callback : nullptr, &g));
    if (!s)
        return fail_as<Generation>(s);
    struct Release {
        void* g;
        ~Release() { (void)mla_generation_destroy(g); }
    } release{g};
    Generation out;
    out.prompt_tokens = prompt.size();
    const auto started = std::chrono::steady_clock::now();
    auto logits = execution_->prefill(prompt);
    if (!logits)
        return R::failure(logits.error());
    out.prefill_ms = ms_since(started);
    for (bool first = true; !mla_generation_finished(g); first = false) {
        int32_t next = -1;
        s = check(mla_generation_step(g, logits.value().data(), logits.value().size(), &next));
        if (!s)
            return fail_as<Generation>(s);
        if (first)
            out.time_to_first_token_ms = ms_since(started);
        if (next < 0)
            break;
        const auto t = std::chrono::steady_clock::now();
        logits = execution_->decode((std::uint16_t)next);
        if (!logits)
            return R::failure(logits.error());
        out.decode_ms += ms_since(t);
    }
    size_t n_text = 0, n_tok = 0;
    char reason[16] = {};
    s = check(mla_generation_result(g, nullptr, 0, &n_text, nullptr, 0, &n_tok, reason));
    out.text.assign(n_text, '\0');
    out.tokens.assign(n_tok, 0);
    if (s)
        s = check(mla_generation_result(g, out.text.data(), n_text, &n_text, out.tokens.data(),
                                        n_tok, &n_tok, reason));
    if (!s)
        return fail_as<Generation>(s);
    out.finish_reason = reason;
    return R::success(std::move(out));
}

// ------------------------------------------------------------------ server ----
Result<std::unique_ptr<Server>> Server::create(std::shared_ptr<HipEngine> engine,
                                               std::shared_ptr<const Tokenizer> tokenizer,
                                               const ServerConfig& config) {
    using R = Result<std::unique_ptr<Server>>;
    if (!engine || !tokenizer)
        return R::failure(ErrorCode::invalid_argument, "Server: null engine or tokenizer");
    const mla_scheduler_config sc{config.max_context, config.max_new_tokens, config.max_queue,
                                  config.request_timeout_seconds};
    std::unique_ptr<Server> srv(new Server());
    const Status s = check(mla_scheduler_create(engine->handle(), tokenizer->handle(), &sc, &srv->h_));
    if (!s)
        return fail_as<std::unique_ptr<Server>>(s);
    srv->engine_ = std::move(engine);
    srv->tokenizer_ = std::move(tokenizer);
    srv->max_new_tokens_ = config.max_new_tokens;
    return R::success(std::move(srv));
}

Server::~Server() {
    if (h_)
        (void)mla_scheduler_destroy(h_);
}

Result<std::uint64_t> Server::submit(std::span<const std::uint16_t> prompt,
                                     const GenerationConfig& config, bool stream,
                                     std::optional<int> max_tokens) {
    CConfig cc(config);
    cc.c.max_new_tokens = max_tokens ? *max_tokens : -1;
    std::uint64_t id = 0;
    const Status s = check(mla_scheduler_submit(h_, prompt.data(), prompt.size(), &cc.c, stream, &id));
    if (!s)
        return fail_as<std::uint64_t>(s);
    return Result<std::uint64_t>::success(id);
}

Status Server::cancel(std::uint64_t request) { return check(mla_scheduler_cancel(h_, request)); }

Result<std::pair<std::string, RequestStatus>> Server::poll(std::uint64_t request, int timeout_ms) {
    using R = Result<std::pair<std::string, RequestStatus>>;
    std::string text(1 << 16, '\0');
    std::vector<std::uint16_t> tokens((size_t)std::max(max_new_tokens_, 1));
    size_t n = 0;
    mla_request_status st{};
    const Status s = check(mla_scheduler_poll(h_, request, timeout_ms, text.data(), text.size(),
                                              &n, tokens.data(), tokens.size(), &st));
    if (!s)
        return fail_as<std::pair<std::string, RequestStatus>>(s);
    text.resize(n);
    RequestStatus rs;
    rs.done = st.done != 0;
    if (st.error != MLA_OK)
        rs.error = Error{static_cast<ErrorCode>(st.error - 1), st.error_message};
    rs.finish_reason = st.finish_reason;
    rs.prompt_tokens = st.prompt_tokens;
    rs.completion_tokens = st.completion_tokens;
    rs.queue_seconds = st.queue_seconds;
    rs.prefill_seconds = st.prefill_seconds;
    rs.decode_seconds = st.decode_seconds;
    rs.first_token_seconds = st.first_token_seconds;
    if (rs.done)
        rs.tokens.assign(tokens.begin(), tokens.begin() + (long)st.completion_tokens);
    return R::success({std::move(text), std::move(rs)});
}

Result<std::string> Server::metrics_text() const {
    size_t n = 0;
    Status s = check(mla_scheduler_metrics_text(h_, nullptr, 0, &n));
    std::string out(n, '\0');
    if (s)
        s = check(mla_scheduler_metrics_text(h_, out.data(), out.size(), &n));
    if (!s)
        return fail_as<std::string>(s);
    return Result<std::string>::success(std::move(out));
}

}  // namespace mla_host
