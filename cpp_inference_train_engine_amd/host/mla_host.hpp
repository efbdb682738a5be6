// C++20 host API of the MI355X backend: the reference engine's inference interfaces
// (include/mini_mla/execution.hpp, inference.hpp, server.hpp) over the C ABI of
// libmla_hip.so (include/mla_hip.h).  A host written against the reference's
// Execution / InferenceEngine / serve() finds the same calls, argument meanings, error
// codes and messages here:
//
//   Execution           the inference part of mini_mla::Execution (execution.hpp:28-62):
//                       prefill, decode, fork_inference, device_name, attention_name;
//   HipEngine           one uploaded model and one paged latent cache shared by sessions
//                       (make_execution(..., "hip") hands out HipExecution sessions);
//   Tokenizer           mini_mla::Tokenizer (tokenizer.hpp): load, encode, decode, special;
//   InferenceEngine     load, fork, generate, generate_tokens (inference.hpp:45-66);
//   Server              the request scheduler under mini_mla_serve (server.hpp), batched.
//
// Results use Result<T> / Status with the reference's ErrorCode values; the message is
// the library's (the reference's wording where the reference has one).
#pragma once

#include "mla_hip.h"

#include <cstdint>
#include <functional>
#include <memory>
#include <optional>
#include <span>
#include <string>
#include <string_view>
#include <utility>
#include <variant>
#include <vector>

namespace mla_host {

// ErrorCode (include/mini_mla/result.hpp:12-19) plus the scheduler's "unavailable".
enum class ErrorCode : std::uint8_t {
    invalid_argument,
    io_error,
    unsupported,
    out_of_memory,
    gpu_error,
    numerical_error,
    unavailable,
};

struct Error {
    ErrorCode code;
    std::string message;
};

template <typename T>
class [[nodiscard]] Result {
  public:
    static Result success(T v) { return Result(std::move(v)); }
    static Result failure(ErrorCode code, std::string message) {
        return Result(Error{code, std::move(message)});
    }
    static Result failure(Error e) { return Result(std::move(e)); }
    explicit operator bool() const { return std::holds_alternative<T>(v_); }
    T& value() & { return std::get<T>(v_); }
    const T& value() const& { return std::get<T>(v_); }
    T&& value() && { return std::get<T>(std::move(v_)); }
    const Error& error() const { return std::get<Error>(v_); }

  private:
    explicit Result(T v) : v_(std::move(v)) {}
    explicit Result(Error e) : v_(std::move(e)) {}
    std::variant<T, Error> v_;
};
using Status = Result<std::monostate>;
inline Status ok() { return Status::success({}); }

// The status of a C-ABI call as a Status (the library's last message on failure).
Status check(int status);

using ModelConfig = mla_model_config;  // ModelConfig's architecture fields (config.hpp)

// Sizes of an engine: sessions, new tokens per batched step, cache pages and their size.
struct EngineLimits {
    int max_sessions = 16, max_rows = 1024, num_pages = 1024, page_size = 64;
};

class HipEngine;

// ExecutionStats (execution.hpp:25-27), with the reference's field names.  On HIP:
// model forwards submitted to the engine's stream, host waits on that stream, and
// kernels launched (metal_kernel_submissions counts HIP kernel launches).
struct ExecutionStats {
    std::uint64_t graph_submissions = 0, host_waits = 0, metal_kernel_submissions = 0;
};

// The logits Execution::forward returns: rows x cols, row-major, read as m(r, c) like the
// reference's Matrix.
struct Matrix {
    int rows = 0, cols = 0;
    std::vector<float> values;
    [[nodiscard]] float operator()(int r, int c) const { return values[(std::size_t)r * cols + c]; }
    float& operator()(int r, int c) { return values[(std::size_t)r * cols + c]; }
    [[nodiscard]] const float* data() const { return values.data(); }
};

// The inference part of mini_mla::Execution (execution.hpp:28-62).
class Execution {
  public:
    virtual ~Execution() = default;
    [[nodiscard]] virtual std::string device_name() const = 0;
    [[nodiscard]] virtual std::string attention_name() const { return "reference"; }
    [[nodiscard]] virtual ExecutionStats stats() const { return {}; }
    [[nodiscard]] virtual Result<std::unique_ptr<Execution>> fork_inference() {
        return Result<std::unique_ptr<Execution>>::failure(
            ErrorCode::unsupported, "Execution cannot fork inference sessions");
    }
    // Logits of every position of `batch` sequences of `sequence` ids (row-major); the
    // matrix stays valid until the execution's next forward.
    [[nodiscard]] virtual Result<const Matrix*> forward(std::span<const std::uint16_t>, int, int) {
        return Result<const Matrix*>::failure(ErrorCode::unsupported,
                                              "Execution has no forward pass");
    }
    [[nodiscard]] virtual Result<std::span<const float>> prefill(std::span<const std::uint16_t>) = 0;
    [[nodiscard]] virtual Result<std::span<const float>> decode(std::uint16_t) = 0;
};

// One uploaded model and its paged latent cache (mla_engine_*).  Sessions share it.
class HipEngine : public std::enable_shared_from_this<HipEngine> {
  public:
    static Result<std::shared_ptr<HipEngine>> create(const ModelConfig&, std::span<const float> params,
                                                     const EngineLimits& = {});
    // A mini-mla-model export or checkpoint (load_checkpoint(path, false)).
    static Result<std::shared_ptr<HipEngine>> load(const std::string& path, const EngineLimits& = {});
    ~HipEngine();
    HipEngine(const HipEngine&) = delete;
    HipEngine& operator=(const HipEngine&) = delete;
    [[nodiscard]] const ModelConfig& config() const { return config_; }
    [[nodiscard]] void* handle() const { return h_; }
    // A new empty session (Execution::fork_inference semantics).
    Result<std::unique_ptr<Execution>> session();
    // The ids the greedy token of batched steps skips (sample_token's banned list).
    Status set_banned(std::span<const std::uint16_t> ids);
    // New weights (registry order), as Model::mark_weights_changed: sessions holding
    // cached tokens must prefill again before they decode (inference.cpp:71-75).
    Status update_weights(std::span<const float> params);
    // Counters since creation, shared by every session of the engine.
    [[nodiscard]] ExecutionStats stats() const;
    // Every position's logits of `batch` sequences of `sequence` ids (mla_engine_forward).
    Status forward(std::span<const std::uint16_t> ids, int batch, int sequence, Matrix& out);
    // One batched forward (continuous batching): sessions[i], a session of this engine,
    // appends tokens[i] (one token: a decode; several: a prompt chunk).  logits (may be
    // null) receives [n x vocab] of each session's last new token, next_tokens (may be
    // null) its greedy token (mla_engine_step).
    Status step(std::span<Execution* const> sessions,
                std::span<const std::vector<std::uint16_t>> tokens, std::vector<float>* logits,
                std::vector<std::int32_t>* next_tokens);

  private:
    HipEngine() = default;
    void* h_ = nullptr;
    ModelConfig config_{};
};

// make_execution(model, nullptr, "hip") for an engine: a new session on it.
Result<std::unique_ptr<Execution>> make_hip_execution(const std::shared_ptr<HipEngine>&);
// make_execution(model, nullptr, backend, precision) (execution.hpp:63-66): backend "hip";
// precision "fp32" (the reference's default) or "fp16".  Both keep fp16 weights and cache
// with fp32 accumulation, so an "fp32" execution matches the CPU path to the fp16
// tolerance of test_mps.cpp:140 (0.015), not to fp32's 1e-4.  Anything else is
// unsupported, with the reference's message for an unknown backend.
Result<std::unique_ptr<Execution>> make_execution(const std::shared_ptr<HipEngine>&,
                                                  std::string_view backend,
                                                  std::string_view precision = "fp32");

// mini_mla::Tokenizer (src/infer/tokenizer.cpp) over mla_tokenizer_*.
class Tokenizer {
  public:
    static Result<std::shared_ptr<const Tokenizer>> load(const std::string& path);
    ~Tokenizer();
    Tokenizer(const Tokenizer&) = delete;
    Tokenizer& operator=(const Tokenizer&) = delete;
    [[nodiscard]] Result<std::vector<std::uint16_t>> encode(std::string_view text,
                                                            bool allow_special = false) const;
    [[nodiscard]] Result<std::string> decode(std::span<const std::uint16_t> ids,
                                             bool skip_special = false) const;
    [[nodiscard]] std::uint16_t special(std::string_view name) const;
    [[nodiscard]] int vocab_size() const { return vocab_; }
    [[nodiscard]] const std::string& hash() const { return hash_; }
    [[nodiscard]] void* handle() const { return h_; }

  private:
    Tokenizer() = default;
    void* h_ = nullptr;
    int vocab_ = 0;
    std::string hash_;
};

// GenerationConfig and Generation (inference.hpp:27-40).
struct GenerationConfig {
    int max_new_tokens = 128, top_k = 0;
    float temperature = 0.8F, top_p = 0.95F, repetition_penalty = 1;
    std::uint64_t seed = 42;
    std::vector<std::string> stop;
    std::vector<std::vector<std::uint16_t>> stop_tokens;
    [[nodiscard]] Status validate() const;
};
struct Generation {
    std::string text, finish_reason;
    std::vector<std::uint16_t> tokens;
    std::size_t prompt_tokens = 0;
    double prefill_ms = 0, decode_ms = 0, time_to_first_token_ms = 0;
};

// sample_token (inference.cpp:345-412); rng_state is the Rng state, advanced by a draw.
Result<std::uint16_t> sample_token(std::span<const float> logits,
                                   std::span<const std::uint16_t> history,
                                   const GenerationConfig&, std::uint64_t& rng_state,
                                   std::span<const std::uint16_t> banned = {});

// InferenceEngine (inference.hpp:45-66) on a HipEngine session.
class InferenceEngine {
  public:
    static Result<std::unique_ptr<InferenceEngine>> load(const std::string& path,
                                                         const EngineLimits& = {});
    // A session on an existing engine, with a tokenizer of the engine's vocabulary.
    static Result<std::unique_ptr<InferenceEngine>> create(std::shared_ptr<HipEngine>,
                                                           std::shared_ptr<const Tokenizer>);
    [[nodiscard]] Result<std::unique_ptr<InferenceEngine>> fork();
    [[nodiscard]] Result<Generation> generate(std::string_view prompt, const GenerationConfig&,
                                              std::function<bool(std::string_view)> callback = {});
    [[nodiscard]] Result<Generation>
    generate_tokens(std::span<const std::uint16_t> prompt, const GenerationConfig&,
                    std::function<bool(std::string_view)> callback = {});
    [[nodiscard]] const Tokenizer& tokenizer() const { return *tokenizer_; }
    [[nodiscard]] const ModelConfig& config() const { return engine_->config(); }
    [[nodiscard]] std::string device_name() const { return execution_->device_name(); }
    [[nodiscard]] const std::shared_ptr<HipEngine>& engine() const { return engine_; }

  private:
    std::shared_ptr<HipEngine> engine_;
    std::shared_ptr<const Tokenizer> tokenizer_;
    std::unique_ptr<Execution> execution_;
};

// ServerConfig's limits (server.hpp:5-10) and the batched request scheduler under the
// server (mla_scheduler_*).  The HTTP layer calls submit / poll / cancel / metrics_text.
struct ServerConfig {
    int max_context = 2048, max_new_tokens = 128, max_queue = 16;
    int request_timeout_seconds = 60;
};
struct RequestStatus {
    bool done = false;
    std::optional<Error> error;  // why the request ended early (queue deadline, failure)
    std::string finish_reason;
    std::size_t prompt_tokens = 0, completion_tokens = 0;
    double queue_seconds = 0, prefill_seconds = 0, decode_seconds = 0, first_token_seconds = 0;
    std::vector<std::uint16_t> tokens;  // once done
};
class Server {
  public:
    static Result<std::unique_ptr<Server>> create(std::shared_ptr<HipEngine>,
                                                  std::shared_ptr<const Tokenizer>,
                                                  const ServerConfig& = {});
    ~Server();
    // max_tokens empty: the server's default budget (server.cpp:300-304).
    Result<std::uint64_t> submit(std::span<const std::uint16_t> prompt, const GenerationConfig&,
                                 bool stream, std::optional<int> max_tokens);
    Status cancel(std::uint64_t request);
    // Text produced since the last poll (waits up to timeout_ms for some); status.done
    // once finished (the request is then forgotten).
    Result<std::pair<std::string, RequestStatus>> poll(std::uint64_t request, int timeout_ms);
    [[nodiscard]] Result<std::string> metrics_text() const;

  private:
    Server() = default;
    void* h_ = nullptr;
    std::shared_ptr<HipEngine> engine_;
    std::shared_ptr<const Tokenizer> tokenizer_;
    int max_new_tokens_ = 0;
};

}  // namespace mla_host
