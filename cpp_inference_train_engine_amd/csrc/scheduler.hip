// Continuous-batching request scheduler, host code (the "one stepping thread over the
// batched API" that replaces mini_mla_serve's worker pool, src/serve/server.cpp).
//
// The reference server queues accepted connections (bounded by max_queue) and gives
// each of `workers` threads a forked session that runs one request's generate_tokens at
// a time.  Here requests are queued the same way, but a single thread admits them into
// engine sessions and advances all of them together: every mla_engine_step carries one
// decode row per running request plus prompt chunks of newly admitted requests, up to
// the engine's max_rows.  Each request keeps the reference's own generation loop
// (Generation, the state machine of generate_tokens), its deadline, cancellation and
// timings, and the scheduler keeps the server's counters.
//
// Admission: a request starts when a session slot is free and the cache has pages for
// its prompt plus max_new_tokens beyond what running requests may still claim, so a
// step never runs out of pages and nothing has to be evicted.  Greedy requests
// (temperature 0, no repetition penalty) take the device's greedy token, which skips
// the tokenizer's banned ids exactly as sample_token does; the others are sampled on the
// host from the step's logits, which are copied back only for steps that need them.
#include "mla_capi_util.hpp"
#include "mla_generation.hpp"
#include "mla_hip.h"
#include "mla_tokenizer.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace mla {
namespace {

using Clock = std::chrono::steady_clock;
double seconds(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double>(b - a).count();
}

struct Request {
    uint64_t id = 0;
    std::vector<uint16_t> prompt;
    GenConfig cfg;
    bool stream = false;
    Clock::time_point accepted, deadline, started;
    std::atomic<bool> cancel{false};
    int pages = 0;  // cache pages reserved: prompt + max_new_tokens
    // Owned by the stepping thread while the request runs.
    int session = -1;
    size_t fed = 0;     // prompt tokens stepped
    int length = 0;     // tokens in the session's cache
    int32_t next = -1;  // token to decode in the next step
    Generation gen;
    std::string pending;  // text streamed during the current step
    int failed = MLA_OK;
    std::string failure;
    // This step's timings, published into prefill_s / decode_s under Scheduler::mu.
    double step_prefill_s = -1, step_decode_s = 0;
    double queue_s = 0, prefill_s = 0, decode_s = 0, first_s = 0;
    // Shared with pollers, under Scheduler::mu.
    std::string outbox;
    bool done = false;
    int error = MLA_OK;
    std::string message, reason;
    size_t n_tokens = 0;
    std::vector<uint16_t> tokens;
};
using RequestPtr = std::shared_ptr<Request>;

// A few helper threads that run the host side of a step's rows (sampling from 16 K-wide
// logits is the one costly part) in parallel with the stepping thread.
class Workers {
  public:
    explicit Workers(int helpers) {
        for (int i = 0; i < helpers; ++i)
            threads_.emplace_back([this] { loop(); });
    }
    ~Workers() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            quit_ = true;
        }
        go_.notify_all();
        for (std::thread& t : threads_)
            t.join();
    }
    // fn(i) for every i in [0, count), on the helpers and the calling thread.
    void run(int count, const std::function<void(int)>& fn) {
        if (threads_.empty() || count < 2) {
            for (int i = 0; i < count; ++i)
                fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            fn_ = &fn;
            count_ = count;
            next_ = 0;
            busy_ = (int)threads_.size();
            ++epoch_;
        }
        go_.notify_all();
        drain();
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return busy_ == 0; });
        fn_ = nullptr;
    }

  private:
    void drain() {
        for (int i; (i = next_.fetch_add(1)) < count_;)
            (*fn_)(i);
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                go_.wait(lk, [&] { return quit_ || epoch_ != seen; });
                if (quit_)
                    return;
                seen = epoch_;
            }
            drain();
            std::lock_guard<std::mutex> lk(mu_);
            if (--busy_ == 0)
                done_.notify_one();
        }
    }
    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable go_, done_;
    const std::function<void(int)>* fn_ = nullptr;
    int count_ = 0, busy_ = 0;
    std::atomic<int> next_{0};
    uint64_t epoch_ = 0;
    bool quit_ = false;
};

struct Row {
    Request* r;
    int count;
    bool prompt;  // a prompt chunk (else one decode token)
    bool last;    // its logits pick the next token
};

struct Scheduler {
    void* engine = nullptr;
    const Tokenizer* tok = nullptr;
    mla_scheduler_config cfg{};
    int vocab = 0, max_seq = 0, max_rows = 0, max_sessions = 0, page_size = 0, num_pages = 0;
    std::vector<uint16_t> banned;

    std::mutex mu;
    std::condition_variable wake, progress;
    // API calls in progress on other threads (under mu); destroy waits for none.
    int calls = 0;
    std::condition_variable idle;
    std::mutex join_mu;  // one thread joins the stepping thread
    std::deque<RequestPtr> queue;
    std::vector<RequestPtr> running;
    std::unordered_map<uint64_t, RequestPtr> live;  // submitted and not yet retired by poll
    uint64_t last_id = 0;
    bool stopping = false;
    std::atomic<bool> stop_flag{false};
    uint64_t requests = 0, completed = 0, rejected = 0, errors = 0, generated = 0, steps = 0;
    double queue_s = 0, prefill_s = 0, decode_s = 0, first_s = 0;
    std::thread thread;

    // stepping thread only
    size_t rotate = 0;
    std::vector<Row> rows;
    std::vector<int> b_sessions, b_counts;
    std::vector<uint16_t> b_tokens;
    std::vector<int32_t> b_next;
    std::vector<int> picks;
    std::vector<float> b_logits;
    std::unique_ptr<Workers> workers;

    void run();
    void admit(Clock::time_point now);
    void plan();
    void retire(const RequestPtr& r);
    void end_unstarted(const RequestPtr& r, int error, const std::string& message);
};

int held_pages(int length, int page_size) { return (length + page_size - 1) / page_size; }

void Scheduler::end_unstarted(const RequestPtr& r, int error, const std::string& message) {
    r->error = error;
    r->message = message;
    r->reason = "cancelled";
    r->done = true;
}

// Under mu.  Starts queued requests while a slot and their pages are free.
void Scheduler::admit(Clock::time_point now) {
    int64_t info[8];
    if (mla_engine_info(engine, info) != MLA_OK)
        return;
    int64_t spare = info[1];  // free pages less what running requests may still claim
    for (const RequestPtr& r : running)
        spare -= r->pages - held_pages(r->length, page_size);
    while (!queue.empty()) {
        RequestPtr r = queue.front();
        if (r->cancel.load()) {  // gone before it started (server.cpp:309-310)
            queue.pop_front();
            end_unstarted(r, MLA_OK, "");
            continue;
        }
        if (now >= r->deadline) {  // server.cpp:305-308
            queue.pop_front();
            end_unstarted(r, MLA_ERR_UNAVAILABLE, "Request queue deadline exceeded");
            continue;
        }
        if ((int)running.size() >= max_sessions || spare < r->pages)
            break;
        int s = -1;
        if (mla_session_create(engine, &s) != MLA_OK)
            break;  // every slot is held, some outside this scheduler
        queue.pop_front();
        r->session = s;
        r->started = now;
        r->queue_s = seconds(r->accepted, now);
        Request* rp = r.get();
        Generation::Callback cb = [this, rp](std::string_view text) {
            if (stop_flag.load() || rp->cancel.load() || Clock::now() >= rp->deadline)
                return false;
            if (rp->stream)
                rp->pending.append(text.data(), text.size());
            return true;
        };
        const int st = r->gen.start(*tok, r->cfg, r->prompt.data(), r->prompt.size(), max_seq,
                                    &banned, std::move(cb));
        if (st) {
            r->failed = st;
            r->failure = mla_last_error();
        }
        spare -= r->pages;
        running.push_back(r);
    }
}

// Stepping thread.  The batch: one decode row per running request that has a token to
// decode (starting at a rotating request when max_rows cannot hold them all), then
// prompt chunks in admission order with the rows that are left.
void Scheduler::plan() {
    rows.clear();
    int budget = max_rows;
    const size_t n = running.size();
    for (size_t k = 0; k < n && budget > 0; ++k) {
        Request* r = running[(rotate + k) % n].get();
        if (!r->failed && !r->gen.finished() && r->next >= 0) {
            rows.push_back({r, 1, false, true});
            --budget;
        }
    }
    rotate = n ? (rotate + 1) % n : 0;
    for (size_t k = 0; k < n && budget > 0; ++k) {
        Request* r = running[k].get();
        if (r->failed || r->gen.finished() || r->fed >= r->prompt.size())
            continue;
        const int c = (int)std::min<size_t>(r->prompt.size() - r->fed, (size_t)budget);
        rows.push_back({r, c, true, r->fed + c == r->prompt.size()});
        budget -= c;
    }
}

// Under mu.  Frees the session and publishes the outcome.
void Scheduler::retire(const RequestPtr& r) {
    (void)mla_session_release(engine, r->session);
    r->session = -1;
    const Generation& g = r->gen;
    r->n_tokens = g.tokens().size();
    r->tokens = g.tokens();
    r->reason = g.finish_reason();
    if (r->failed) {  // server.cpp:364-370
        r->error = r->failed;
        r->message = r->failure;
        ++errors;
    } else {
        generated += r->n_tokens;
        if (r->reason != "cancelled") {  // server.cpp:355-361
            ++completed;
            queue_s += r->queue_s;
            prefill_s += r->prefill_s;
            decode_s += r->decode_s;
            first_s += r->queue_s + r->first_s;
            if (!r->stream)
                r->outbox = g.text();
        }
    }
    r->done = true;
}

void Scheduler::run() {
    std::unique_lock<std::mutex> lk(mu);
    for (;;) {
        wake.wait(lk, [&] { return stopping || !running.empty() || !queue.empty(); });
        if (stopping)
            break;
        admit(Clock::now());
        // Requests that ended at admission (max_new_tokens 0, a failed start) or whose
        // deadline or cancellation came while they waited are retired before the step.
        for (size_t k = 0; k < running.size();) {
            const RequestPtr& r = running[k];
            if (r->failed || r->gen.finished()) {
                retire(r);
                running.erase(running.begin() + (long)k);
            } else {
                ++k;
            }
        }
        progress.notify_all();
        if (running.empty()) {
            if (!queue.empty())  // waiting for pages or slots held elsewhere
                wake.wait_for(lk, std::chrono::milliseconds(2));
            continue;
        }
        plan();
        lk.unlock();

        const int n = (int)rows.size();
        b_sessions.resize(n);
        b_counts.resize(n);
        b_next.assign(n, 0);
        b_tokens.clear();
        bool host_logits = false;
        for (int i = 0; i < n; ++i) {
            const Row& w = rows[i];
            b_sessions[i] = w.r->session;
            b_counts[i] = w.count;
            if (w.prompt)
                b_tokens.insert(b_tokens.end(), w.r->prompt.begin() + (long)w.r->fed,
                                w.r->prompt.begin() + (long)w.r->fed + w.count);
            else
                b_tokens.push_back((uint16_t)w.r->next);
            host_logits = host_logits || (w.last && !w.r->gen.greedy_on_device());
        }
        if (host_logits)
            b_logits.resize((size_t)n * vocab);
        const Clock::time_point t0 = Clock::now();
        const int st = mla_engine_step(engine, n, b_sessions.data(), b_counts.data(),
                                       b_tokens.data(), host_logits ? b_logits.data() : nullptr,
                                       b_next.data());
        const std::string step_error = st ? mla_last_error() : "";
        const Clock::time_point t1 = Clock::now();
        // A non-finite logit or an all-banned row is reported after the sessions
        // advanced; it matters only to the rows whose token is chosen from it.
        bool advanced = st == MLA_OK || st == MLA_ERR_NUMERICAL;
        for (int i = 0; i < n && !advanced; ++i)
            advanced = st == MLA_ERR_INVALID_ARGUMENT && b_next[i] == -2;
        picks.clear();
        for (int i = 0; i < n; ++i) {
            const Row& w = rows[i];
            Request* r = w.r;
            if (!advanced) {
                r->failed = st;
                r->failure = step_error;
                continue;
            }
            r->length += w.count;
            if (w.prompt) {
                r->fed += w.count;
                if (w.last)
                    r->step_prefill_s = seconds(r->started, t1);
            } else {
                r->step_decode_s += seconds(t0, t1);
            }
            if (w.last)
                picks.push_back(i);
        }
        // Each pick touches only its own request (and reads the shared tokenizer and
        // banned list), so the picks run in parallel.
        workers->run((int)picks.size(), [&](int k) {
            const int i = picks[(size_t)k];
            const Row& w = rows[(size_t)i];
            Request* r = w.r;
            const size_t before = r->gen.tokens().size();
            int32_t next = -1;
            int gs;
            if (r->gen.greedy_on_device()) {
                const int32_t v = b_next[i];
                gs = v == -1 ? fail(MLA_ERR_NUMERICAL, w.prompt ? "Invalid sampler logits"
                                                                : "Nonfinite decode output")
                     : v == -2 ? fail(MLA_ERR_INVALID_ARGUMENT, "All tokens are banned")
                               : r->gen.step_token((uint16_t)v, &next);
            } else {
                gs = r->gen.step(b_logits.data() + (size_t)i * vocab, (size_t)vocab, &next);
            }
            if (before == 0 && r->gen.tokens().size() == 1)
                r->first_s = seconds(r->started, Clock::now());
            if (gs) {
                r->failed = gs;
                r->failure = mla_last_error();
            }
            r->next = next;
        });

        lk.lock();
        ++steps;
        for (const Row& w : rows) {
            Request* r = w.r;
            if (!r->pending.empty()) {
                r->outbox += r->pending;
                r->pending.clear();
            }
            if (r->step_prefill_s >= 0) {
                r->prefill_s = r->step_prefill_s;
                r->step_prefill_s = -1;
            }
            r->decode_s += r->step_decode_s;
            r->step_decode_s = 0;
        }
        for (size_t k = 0; k < running.size();) {
            const RequestPtr& r = running[k];
            if (r->failed || r->gen.finished()) {
                retire(r);
                running.erase(running.begin() + (long)k);
            } else {
                ++k;
            }
        }
        progress.notify_all();
    }
    // Stopping: what is queued never starts; what runs ends as cancelled.
    for (const RequestPtr& r : queue)
        end_unstarted(r, MLA_OK, "");
    queue.clear();
    for (const RequestPtr& r : running) {
        (void)mla_session_release(engine, r->session);
        r->n_tokens = r->gen.tokens().size();
        r->tokens = r->gen.tokens();
        r->reason = "cancelled";
        r->done = true;
    }
    running.clear();
    progress.notify_all();
}

Scheduler* as_scheduler(void* p) { return static_cast<Scheduler*>(p); }

// Counts an API call in progress.  Constructed and destroyed under S.mu (declare it after
// the lock), so destroy can wait until no other thread is inside the scheduler.
struct InCall {
    Scheduler& S;
    explicit InCall(Scheduler& s) : S(s) { ++S.calls; }
    ~InCall() {
        if (--S.calls == 0 && S.stopping)
            S.idle.notify_all();
    }
    InCall(const InCall&) = delete;
    InCall& operator=(const InCall&) = delete;
};

// Ends the stepping thread: what is queued never starts, what runs ends as cancelled.
void stop(Scheduler* S) {
    {
        std::lock_guard<std::mutex> lk(S->mu);
        S->stopping = true;
        S->stop_flag = true;
    }
    S->wake.notify_all();
    S->progress.notify_all();  // pollers waiting for text wake up
    std::lock_guard<std::mutex> j(S->join_mu);
    if (S->thread.joinable())
        S->thread.join();
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

void mla_scheduler_config_init(mla_scheduler_config* c) {
    if (!c)
        return;
    c->max_context = 2048;  // ServerConfig defaults (server.hpp:7-8)
    c->max_new_tokens = 128;
    c->max_queue = 16;
    c->request_timeout_seconds = 60;
}

int mla_scheduler_create(void* engine, void* tokenizer, const mla_scheduler_config* config,
                         void** scheduler) {
    if (!engine || !tokenizer || !config || !scheduler)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_create: null argument");
    mla_model_config mc{};
    int64_t info[8];
    int st = mla_engine_config(engine, &mc);
    if (!st)
        st = mla_engine_info(engine, info);
    if (st)
        return st;
    const mla_scheduler_config& c = *config;
    if (c.max_queue < 1 || c.request_timeout_seconds < 1 || c.max_context < 1 ||
        c.max_context > mc.max_sequence_length || c.max_new_tokens < 1)  // server.cpp:172-176
        return fail(MLA_ERR_INVALID_ARGUMENT, "Invalid server limits");
    const Tokenizer* t = static_cast<const Tokenizer*>(tokenizer);
    if (t->vocab != mc.vocab_size)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Tokenizer vocabulary does not match the model");
    auto S = std::make_unique<Scheduler>();
    S->engine = engine;
    S->tok = t;
    S->cfg = c;
    S->vocab = mc.vocab_size;
    S->max_seq = mc.max_sequence_length;
    S->num_pages = (int)info[2];
    S->page_size = (int)info[3];
    S->max_rows = (int)info[4];
    S->max_sessions = (int)info[5];
    S->banned = banned_tokens(*t);
    if ((st = mla_engine_set_banned(engine, S->banned.data(), S->banned.size())))
        return st;
    Scheduler* raw = S.get();
    try {
        const unsigned hw = std::thread::hardware_concurrency();
        S->workers = std::make_unique<Workers>((int)std::min(15u, hw > 1 ? hw - 1 : 0u));
        S->thread = std::thread([raw] { raw->run(); });
    } catch (const std::exception& e) {
        return fail(MLA_ERR_OUT_OF_MEMORY, std::string("mla_scheduler_create: ") + e.what());
    }
    *scheduler = S.release();
    return MLA_OK;
}

int mla_scheduler_stop(void* scheduler) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_stop: null scheduler");
    stop(S);
    return MLA_OK;
}

int mla_scheduler_destroy(void* scheduler) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S)
        return MLA_OK;
    stop(S);
    {
        // Calls already inside the scheduler on other threads (a poll that was waiting
        // has been woken by stop) return before the memory goes.
        std::unique_lock<std::mutex> lk(S->mu);
        S->idle.wait(lk, [&] { return S->calls == 0; });
    }
    delete S;
    return MLA_OK;
}

int mla_scheduler_submit(void* scheduler, const uint16_t* prompt, size_t n,
                         const mla_generation_config* config, int stream, uint64_t* request) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S || !request || (!prompt && n))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_submit: null argument");
    GenConfig c;
    if (config)
        if (const int st = gen_config_from_c(config, c))
            return st;
    std::lock_guard<std::mutex> lk(S->mu);
    const InCall in(*S);
    if (S->stopping)
        return fail(MLA_ERR_UNAVAILABLE, "Scheduler is stopping");
    if (S->queue.size() >= (size_t)S->cfg.max_queue) {  // server.cpp:213-219
        ++S->rejected;
        return fail(MLA_ERR_UNAVAILABLE, "Request queue is full");
    }
    ++S->requests;
    if (!config || config->max_new_tokens < 0)  // no max_tokens: server.cpp:300-304
        c.max_new_tokens = std::min(S->cfg.max_new_tokens, S->cfg.max_context - (int)std::min<size_t>(n, 1u << 30));
    int st = validate(c);
    if (!st && (c.max_new_tokens > S->cfg.max_new_tokens ||
                n + (size_t)c.max_new_tokens > (size_t)S->cfg.max_context))
        st = fail(MLA_ERR_INVALID_ARGUMENT, "Request exceeds context or token limit");
    if (!st && n == 0)
        st = fail(MLA_ERR_INVALID_ARGUMENT, "Prompt plus requested tokens exceeds context");
    for (size_t k = 0; !st && k < n; ++k)
        if (prompt[k] >= S->vocab)
            st = fail(MLA_ERR_INVALID_ARGUMENT, "Prompt token exceeds vocabulary");
    for (const auto& seq : c.stop_tokens)
        for (const uint16_t id : seq)
            if (!st && id >= S->vocab)
                st = fail(MLA_ERR_INVALID_ARGUMENT, "Stop token exceeds vocabulary");
    const int pages = held_pages((int)n + c.max_new_tokens, S->page_size);
    if (!st && pages > S->num_pages)
        st = fail(MLA_ERR_OUT_OF_MEMORY, "Request needs more cache pages than the engine has");
    if (st) {
        ++S->errors;  // server.cpp:364-366
        return st;
    }
    auto r = std::make_shared<Request>();
    r->id = ++S->last_id;
    r->prompt.assign(prompt, prompt + n);
    r->cfg = std::move(c);
    r->stream = stream != 0;
    r->pages = pages;
    r->accepted = Clock::now();
    r->deadline = r->accepted + std::chrono::seconds(S->cfg.request_timeout_seconds);
    S->queue.push_back(r);
    S->live.emplace(r->id, r);
    *request = r->id;
    S->wake.notify_one();
    return MLA_OK;
}

int mla_scheduler_cancel(void* scheduler, uint64_t request) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_cancel: null scheduler");
    std::lock_guard<std::mutex> lk(S->mu);
    const InCall in(*S);
    auto it = S->live.find(request);
    if (it == S->live.end())
        return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown request");
    it->second->cancel = true;
    S->wake.notify_one();
    return MLA_OK;
}

int mla_scheduler_poll(void* scheduler, uint64_t request, int timeout_ms, char* text,
                       size_t text_capacity, size_t* text_len, uint16_t* tokens,
                       size_t tokens_capacity, mla_request_status* status) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S || !text_len || !status || (!text && text_capacity))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_poll: null argument");
    std::unique_lock<std::mutex> lk(S->mu);
    const InCall in(*S);
    auto it = S->live.find(request);
    if (it == S->live.end())
        return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown request");
    const RequestPtr r = it->second;
    if (timeout_ms > 0)
        S->progress.wait_for(lk, std::chrono::milliseconds(timeout_ms),
                             [&] { return r->done || !r->outbox.empty() || S->stopping; });
    // The request may have been retired by another poll while this one waited.
    it = S->live.find(request);
    if (it == S->live.end())
        return fail(MLA_ERR_INVALID_ARGUMENT, "Unknown request");
    const size_t take = std::min(text_capacity, r->outbox.size());
    if (take)
        std::memcpy(text, r->outbox.data(), take);
    r->outbox.erase(0, take);
    *text_len = take;
    std::memset(status, 0, sizeof(*status));
    status->error = r->error;
    std::snprintf(status->error_message, sizeof(status->error_message), "%s", r->message.c_str());
    std::snprintf(status->finish_reason, sizeof(status->finish_reason), "%s", r->reason.c_str());
    status->prompt_tokens = r->prompt.size();
    status->completion_tokens = r->n_tokens;
    status->queue_seconds = r->queue_s;
    status->prefill_seconds = r->prefill_s;
    status->decode_seconds = r->decode_s;
    status->first_token_seconds = r->done ? r->queue_s + r->first_s : 0.0;
    if (r->done && r->outbox.empty()) {
        if (tokens && tokens_capacity < r->tokens.size())
            return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_poll: needs room for " +
                                                      std::to_string(r->tokens.size()) + " tokens");
        if (tokens && !r->tokens.empty())
            std::memcpy(tokens, r->tokens.data(), r->tokens.size() * sizeof(uint16_t));
        status->done = 1;
        S->live.erase(it);
    }
    return MLA_OK;
}

int mla_scheduler_metrics_get(void* scheduler, mla_scheduler_metrics* m) {
    Scheduler* S = as_scheduler(scheduler);
    if (!S || !m)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_metrics_get: null argument");
    std::lock_guard<std::mutex> lk(S->mu);
    const InCall in(*S);
    m->requests = S->requests;
    m->completed = S->completed;
    m->rejected = S->rejected;
    m->errors = S->errors;
    m->generated_tokens = S->generated;
    m->queue_seconds = S->queue_s;
    m->prefill_seconds = S->prefill_s;
    m->decode_seconds = S->decode_s;
    m->first_token_seconds = S->first_s;
    m->queue_depth = S->queue.size();
    m->running = S->running.size();
    m->steps = S->steps;
    return MLA_OK;
}

int mla_scheduler_metrics_text(void* scheduler, char* text, size_t capacity, size_t* len) {
    mla_scheduler_metrics m;
    if (const int st = mla_scheduler_metrics_get(scheduler, &m))
        return st;
    if (!len)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_metrics_text: null argument");
    // server.cpp:272-289: integers, then the sums as std::to_string prints doubles ("%f").
    std::string out = "mini_mla_requests_total " + std::to_string(m.requests) +
                      "\nmini_mla_completed_total " + std::to_string(m.completed) +
                      "\nmini_mla_rejected_total " + std::to_string(m.rejected) +
                      "\nmini_mla_errors_total " + std::to_string(m.errors) +
                      "\nmini_mla_generated_tokens_total " + std::to_string(m.generated_tokens) +
                      "\n";
    out += "mini_mla_queue_seconds_sum " + std::to_string(m.queue_seconds) +
           "\nmini_mla_prefill_seconds_sum " + std::to_string(m.prefill_seconds) +
           "\nmini_mla_decode_seconds_sum " + std::to_string(m.decode_seconds) +
           "\nmini_mla_first_token_seconds_sum " + std::to_string(m.first_token_seconds) + "\n";
    out += "mini_mla_queue_depth " + std::to_string(m.queue_depth) + "\n";
    // The batched scheduler's own gauges.
    out += "mini_mla_running_requests " + std::to_string(m.running) +
           "\nmini_mla_batch_steps_total " + std::to_string(m.steps) + "\n";
    *len = out.size();
    if (!text)
        return MLA_OK;
    if (capacity < out.size())
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_scheduler_metrics_text: buffer too small");
    std::memcpy(text, out.data(), out.size());
    return MLA_OK;
}

}  // extern "C"
