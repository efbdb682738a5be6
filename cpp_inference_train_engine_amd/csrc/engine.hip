// Session engine: the reference's per-session inference contract (Execution::prefill,
// decode and fork_inference, include/mini_mla/execution.hpp:28-62, implemented by
// CpuDecoder, src/infer/inference.cpp:47-174, and MpsExecution,
// src/backends/mps_backend.mm:872-977) for many sessions that share one uploaded model
// and one paged latent cache, plus the batched step that serves them together
// (continuous batching with chunked prefill; the reference's only batched precedent is
// the Gemma engine's prefill_batch / decode(sessions, tokens) / release,
// src/infer/gemma.cpp:300-548).
//
// Host side of every call: validate like the reference, allocate pages (a free list
// with reference counts, so forked sessions share their prefix pages and a shared
// page is copied before a session appends into it), stage the step's inputs in pinned
// memory, then on the engine's stream: one metadata build, one model forward, the
// copies of the results back, and one synchronisation.
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_internal.hpp"
#include "mla_model.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace mla {
namespace {

constexpr int kSplitPages = 4;  // MLA_DECODE_SPLIT_PAGES
// The pinned host words a step reads back: the metadata info, the decode workspace's head
// (merge counters and status word), then the greedy token of each session.
constexpr int kHeadInts = MLA_DECODE_STATUS_OFFSET / 4 + 1;
constexpr int kHostInfo = 0, kHostHead = MLA_INFO_INTS, kHostNext = kHostHead + kHeadInts + 7;

struct Session {
    bool active = false;
    int length = 0;              // tokens cached: the reference's position_
    uint64_t revision = 0;       // weight revision its cache was computed with
    std::vector<int32_t> pages;  // physical page ids, position order
};

struct Engine {
    std::mutex mu;
    void* model = nullptr;
    mla_model_config cfg{};
    int page_size = 0, num_pages = 0, max_rows = 0, max_sessions = 0, max_pages = 0;
    int work_cap = 0;
    int n_xcd = 0;  // XCDs when the device supports XCD placement of the work list, else 0
    hipStream_t stream = nullptr;
    size_t rec_words = 0;
    uint16_t* pool = nullptr;  // [n_layers][num_pages][rec_words]
    std::vector<void*> layer_pools;
    std::vector<int> refs;       // per page
    std::vector<int32_t> free_;  // free page ids (stack)
    std::vector<Session> sessions;
    uint64_t steps = 0;
    uint64_t revision = 0;  // bumped by mla_engine_update_weights
    // stats: model forwards submitted, host waits on the stream, kernels and copies issued
    uint64_t host_waits = 0, meta_launches = 0, copies = 0;
    // device
    int32_t* d_in = nullptr;  // staged inputs, see step()
    size_t in_cap = 0;        // int32 elements
    int32_t *cu_q = nullptr, *cu_k = nullptr, *table = nullptr, *slots = nullptr,
            *nsplit = nullptr, *cu_split = nullptr, *w_sess = nullptr, *w_split = nullptr,
            *w_desc = nullptr, *w_pages = nullptr, *info = nullptr, *d_next = nullptr;
    float* d_logits = nullptr;
    float* d_logits_all = nullptr;  // [max_rows x vocab] for mla_engine_forward (first use)
    int32_t* d_next_all = nullptr;  // [max_rows]
    void* workspace = nullptr;
    size_t ws_bytes = 0;
    // pinned host
    int32_t* h_in = nullptr;
    float* h_logits = nullptr;
    float* h_logits_all = nullptr;  // [max_rows x vocab] pinned, with d_logits_all
    int32_t* h_out = nullptr;  // info, decode status, next tokens (kHostInfo .. kHostNext)
    uint64_t reruns = 0;       // steps rerun through the two-launch path (failed fused check)
    std::vector<void*> dev_allocs, host_allocs;

    ~Engine() {
        if (stream)
            (void)hipStreamSynchronize(stream);
        if (model)
            mla_model_destroy(model);
        for (void* p : dev_allocs)
            (void)hipFree(p);
        for (void* p : host_allocs)
            (void)hipHostFree(p);
        if (stream)
            (void)hipStreamDestroy(stream);
    }
    template <typename T>
    hipError_t dalloc(T*& p, size_t n) {
        void* v = nullptr;
        const hipError_t e = hipMalloc(&v, std::max<size_t>(n, 1) * sizeof(T));
        if (e == hipSuccess)
            dev_allocs.push_back(v);
        p = static_cast<T*>(v);
        return e;
    }
    template <typename T>
    hipError_t halloc(T*& p, size_t n) {
        void* v = nullptr;
        const hipError_t e = hipHostMalloc(&v, std::max<size_t>(n, 1) * sizeof(T), 0);
        if (e == hipSuccess)
            host_allocs.push_back(v);
        p = static_cast<T*>(v);
        return e;
    }
};

int ceil_div(long long a, int b) { return (int)((a + b - 1) / b); }

Engine* as_engine(void* e) { return static_cast<Engine*>(e); }

int check_session(Engine* E, int s, const char* fn) {
    if (s < 0 || s >= E->max_sessions || !E->sessions[s].active)
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": unknown session");
    return MLA_OK;
}

void release_pages(Engine* E, Session& S) {
    for (int32_t p : S.pages)
        if (--E->refs[p] == 0)
            E->free_.push_back(p);
    S.pages.clear();
    S.length = 0;
}

// Device copy of one page record in every layer (copy-on-write of a shared page).
hipError_t copy_page(Engine* E, int32_t dst, int32_t src) {
    const size_t bytes = E->rec_words * 2;
    for (int l = 0; l < E->cfg.n_layers; ++l) {
        uint16_t* base = static_cast<uint16_t*>(E->layer_pools[l]);
        const hipError_t e = hipMemcpyAsync(base + (size_t)dst * E->rec_words,
                                            base + (size_t)src * E->rec_words, bytes,
                                            hipMemcpyDeviceToDevice, E->stream);
        if (e != hipSuccess)
            return e;
        ++E->copies;
    }
    return hipSuccess;
}

// One batched step: session ids[i] appends counts[i] tokens (tokens concatenated in
// order).  Logits of each session's last new row go to `logits` [n x vocab] (host,
// may be null), greedy tokens to `next` [n] (host, may be null).  Lengths advance only
// on success.
// Whether this step's work list is built XCD-placed (each layer's decode attention then one
// launch): the device supports it, the batch has at most MLA_PLACE_MAX_SESSIONS sessions,
// and the placed list fits the work capacity.  The slot count repeats mla_build_metadata's
// deal (sessions by pages read, largest first, snake rounds over the XCDs) on the host's
// lengths, so the build never fails for want of room.
bool placed_fits(const Engine* E, int n, const int32_t* ctx, const int32_t* q) {
    if (E->n_xcd < 1 || n > MLA_PLACE_MAX_SESSIONS)
        return false;
    std::vector<int> pages(n), order(n);
    for (int b = 0; b < n; ++b) {
        pages[b] = q[b] > 0 ? ceil_div((long long)ctx[b] + q[b], E->page_size) : 0;
        order[b] = b;
    }
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return pages[a] > pages[b]; });
    std::vector<long long> items(E->n_xcd, 0);
    for (int r = 0; r < n; ++r) {
        const int x = (r / E->n_xcd) % 2 == 0 ? r % E->n_xcd : E->n_xcd - 1 - r % E->n_xcd;
        items[x] += ceil_div(pages[order[r]], kSplitPages);
    }
    return (long long)E->n_xcd * *std::max_element(items.begin(), items.end()) <= E->work_cap;
}

int step(Engine* E, int n, const int* ids, const int* counts, const uint16_t* tokens,
         float* logits, int32_t* next, const char* fn, bool all_rows = false) {
    const mla_model_config& c = E->cfg;
    if (n < 1 || n > E->max_sessions || !ids || !counts || !tokens)
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": invalid batch");
    std::vector<char> seen(E->max_sessions, 0);
    long long rows = 0;
    int max_q = 1;
    for (int i = 0; i < n; ++i) {
        if (int st = check_session(E, ids[i], fn))
            return st;
        if (seen[ids[i]])
            return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": session listed twice");
        seen[ids[i]] = 1;
        const Session& S = E->sessions[ids[i]];
        if (counts[i] < 1 || (long long)S.length + counts[i] > c.max_sequence_length)
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        std::string(fn) + ": prompt exceeds context or is empty");
        if (S.length > 0 && S.revision != E->revision)  // inference.cpp:71-75
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "Decode requires current-weight prefill, available context, and a "
                        "valid token");
        rows += counts[i];
        max_q = std::max(max_q, counts[i]);
    }
    if (rows > E->max_rows)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": more new tokens than the engine's max_rows");
    for (long long r = 0; r < rows; ++r)
        if (tokens[r] >= c.vocab_size)
            return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": token exceeds vocabulary");

    // ---- pages: copy-on-write of a shared partial last page, then new pages ----
    struct Undo {
        int session, slot;
        int32_t old_page;
    };
    std::vector<Undo> cow;
    std::vector<std::pair<int, size_t>> grown;  // (session, old page count)
    auto rollback = [&]() {
        for (auto& [s, old] : grown) {
            Session& S = E->sessions[s];
            for (size_t k = old; k < S.pages.size(); ++k)
                if (--E->refs[S.pages[k]] == 0)
                    E->free_.push_back(S.pages[k]);
            S.pages.resize(old);
        }
        for (auto it = cow.rbegin(); it != cow.rend(); ++it) {
            Session& S = E->sessions[it->session];
            const int32_t p = S.pages[it->slot];
            if (--E->refs[p] == 0)
                E->free_.push_back(p);
            S.pages[it->slot] = it->old_page;
            ++E->refs[it->old_page];
        }
    };
    for (int i = 0; i < n; ++i) {
        Session& S = E->sessions[ids[i]];
        const int partial = S.length % E->page_size ? S.length / E->page_size : -1;
        if (partial >= 0 && E->refs[S.pages[partial]] > 1) {
            if (E->free_.empty()) {
                rollback();
                return fail(MLA_ERR_OUT_OF_MEMORY, std::string(fn) + ": page pool exhausted");
            }
            const int32_t np = E->free_.back();
            E->free_.pop_back();
            E->refs[np] = 1;
            const int32_t old = S.pages[partial];
            --E->refs[old];
            S.pages[partial] = np;
            cow.push_back({ids[i], partial, old});
            if (hipError_t e = copy_page(E, np, old); e != hipSuccess) {
                rollback();
                return gpu_status(e, fn);
            }
        }
        const int need = ceil_div((long long)S.length + counts[i], E->page_size);
        grown.push_back({ids[i], S.pages.size()});
        while ((int)S.pages.size() < need) {
            if (E->free_.empty()) {
                rollback();
                return fail(MLA_ERR_OUT_OF_MEMORY, std::string(fn) + ": page pool exhausted");
            }
            S.pages.push_back(E->free_.back());
            E->free_.pop_back();
            E->refs[S.pages.back()] = 1;
        }
    }

    // ---- staged inputs: ctx[n] q[n] cu_pages[n+1] tokens[rows] positions[rows] pages[] ----
    long long total_pages = 0;
    int work = 0;
    for (int i = 0; i < n; ++i) {
        const Session& S = E->sessions[ids[i]];
        total_pages += (long long)S.pages.size();
        work += ceil_div((long long)S.pages.size(), kSplitPages);
    }
    const size_t need_in = (size_t)3 * n + 1 + 2 * (size_t)rows + (size_t)total_pages;
    if (need_in > E->in_cap || work > E->work_cap) {
        rollback();
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": batch exceeds engine capacity");
    }
    float* const d_logits = all_rows ? E->d_logits_all : E->d_logits;
    int32_t* const d_next = all_rows ? E->d_next_all : E->d_next;
    float* const h_logits = all_rows ? E->h_logits_all : E->h_logits;
    const long long out_rows = all_rows ? rows : n;
    int32_t* h = E->h_in;
    int32_t *h_ctx = h, *h_q = h + n, *h_cup = h + 2 * n, *h_tok = h + 3 * n + 1;
    int32_t *h_pos = h_tok + rows, *h_ids = h_pos + rows;
    h_cup[0] = 0;
    long long r = 0;
    for (int i = 0; i < n; ++i) {
        const Session& S = E->sessions[ids[i]];
        h_ctx[i] = S.length;
        h_q[i] = counts[i];
        std::memcpy(h_ids + h_cup[i], S.pages.data(), S.pages.size() * sizeof(int32_t));
        h_cup[i + 1] = h_cup[i] + (int32_t)S.pages.size();
        for (int k = 0; k < counts[i]; ++k, ++r) {
            h_tok[r] = tokens[r];
            h_pos[r] = S.length + k;
        }
    }
    hipError_t e = hipMemcpyAsync(E->d_in, h, need_in * sizeof(int32_t), hipMemcpyHostToDevice,
                                  E->stream);
    int32_t *d_ctx = E->d_in, *d_q = d_ctx + n, *d_cup = d_ctx + 2 * n, *d_tok = d_ctx + 3 * n + 1;
    int32_t *d_pos = d_tok + rows, *d_ids = d_pos + rows;
    int st = gpu_status(e, fn);
    // Metadata build, forward and read-back of one attempt; placed: the work list XCD-placed
    // and each layer's decode attention one launch.
    auto attempt = [&](bool placed) {
        int rc = mla_build_metadata(E->stream, n, d_ctx, d_q, d_cup, d_ids, E->page_size,
                                    E->max_pages, E->num_pages, kSplitPages, 1024, E->work_cap,
                                    E->max_rows, placed ? 1 : 0, E->cu_q, E->cu_k, E->table,
                                    E->slots, E->nsplit, E->cu_split, E->w_sess, E->w_split,
                                    E->w_desc, E->w_pages, E->info);
        if (!rc) {
            const MetaPtrs md{E->cu_q,     E->cu_k,    E->table,   E->slots,
                              E->nsplit,   E->cu_split, E->w_desc, E->w_pages,
                              E->info,     E->max_pages, E->num_pages, E->work_cap,
                              placed ? MLA_DECODE_FUSED_MERGE : 0};
            rc = model_forward(static_cast<Model*>(E->model), E->stream, (int)rows, d_tok, d_pos,
                               n, max_q, md, E->layer_pools.data(), E->workspace, E->ws_bytes,
                               d_logits, d_next, all_rows);
        }
        if (rc)
            return rc;
        hipError_t err = hipMemcpyAsync(E->h_out + kHostInfo, E->info,
                                        MLA_INFO_INTS * sizeof(int32_t), hipMemcpyDeviceToHost,
                                        E->stream);
        if (err == hipSuccess && placed)
            err = hipMemcpyAsync(E->h_out + kHostHead, E->workspace, kHeadInts * sizeof(int32_t),
                                 hipMemcpyDeviceToHost, E->stream);
        if (err == hipSuccess && !all_rows)
            err = hipMemcpyAsync(E->h_out + kHostNext, d_next, n * sizeof(int32_t),
                                 hipMemcpyDeviceToHost, E->stream);
        if (err == hipSuccess && logits)
            err = hipMemcpyAsync(h_logits, d_logits,
                                 (size_t)out_rows * c.vocab_size * sizeof(float),
                                 hipMemcpyDeviceToHost, E->stream);
        if (err == hipSuccess)
            err = hipStreamSynchronize(E->stream);
        E->meta_launches += 1;
        E->copies += 2 + placed + !all_rows + (logits != nullptr);
        E->host_waits += 1;
        return gpu_status(err, fn);
    };
    const bool placed = placed_fits(E, n, h_ctx, h_q);
    if (!st)
        st = attempt(placed);
    if (!st && placed && decode_head_status(E->h_out + kHostHead) != 0) {
        // A fused merge's premise failed (a session's items did not meet in one L2: this
        // device does not dispatch as probed).  Stop placing, clear the workspace head
        // (status and merge counters) and run the step again through the two-launch path;
        // its appends rewrite the same values into the same slots.
        E->n_xcd = 0;
        ++E->reruns;
        st = gpu_status(hipMemsetAsync(E->workspace, 0, MLA_DECODE_WORKSPACE_HEAD, E->stream),
                        fn);
        if (!st)
            st = attempt(false);
    }
    if (!st && E->h_out[kHostInfo] < 0)
        st = fail(MLA_ERR_INVALID_ARGUMENT,
                  std::string(fn) + ": ragged metadata rejected session " +
                      std::to_string(E->h_out[kHostInfo + 1]));
    if (st) {
        (void)hipStreamSynchronize(E->stream);
        rollback();
        return st;
    }
    ++E->steps;
    bool finite = true, open = true;
    for (int i = 0; i < n; ++i) {
        Session& S = E->sessions[ids[i]];
        S.length += counts[i];
        S.revision = E->revision;
        if (all_rows)
            continue;
        finite = finite && E->h_out[kHostNext + i] != -1;
        open = open && E->h_out[kHostNext + i] != -2;
        if (next)
            next[i] = E->h_out[kHostNext + i];
    }
    if (logits && logits != h_logits)
        std::memcpy(logits, h_logits, (size_t)out_rows * c.vocab_size * sizeof(float));
    if (all_rows && logits)
        for (size_t k = 0; k < (size_t)out_rows * c.vocab_size && finite; ++k)
            finite = std::isfinite(logits[k]);
    if (!finite)  // inference.cpp:170-172
        return fail(MLA_ERR_NUMERICAL, "Nonfinite decode output");
    if (!open)  // inference.cpp:375-377
        return fail(MLA_ERR_INVALID_ARGUMENT, "All tokens are banned");
    return MLA_OK;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int mla_engine_create(const mla_model_config* config, const float* params, int max_sessions,
                      int max_rows, int num_pages, int page_size, void** engine) {
    if (!engine)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_create: null output");
    *engine = nullptr;
    if (int st = mla_config_validate(config))
        return st;
    if (!params || max_sessions < 1 || max_sessions > 65535 || max_rows < 1 ||
        max_rows > 65536 || num_pages < 1 || page_size < 1 || page_size > 4096)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_create: invalid argument");
    auto* E = new (std::nothrow) Engine();
    if (!E)
        return fail(MLA_ERR_OUT_OF_MEMORY, "mla_engine_create: host allocation");
    auto bail = [&](int st) {
        delete E;
        return st;
    };
    E->cfg = *config;
    E->page_size = page_size;
    E->num_pages = num_pages;
    E->max_rows = max_rows;
    E->max_sessions = max_sessions;
    E->max_pages = ceil_div(config->max_sequence_length, page_size);
    // XCD placement (each layer's decode attention in one launch) needs room for the placed
    // work list: every XCD holds at most ceil(sessions / n) sessions' items.
    E->n_xcd = mla_xcd_placement_supported();
    const long long per_session = ceil_div(E->max_pages, kSplitPages);
    const long long placed_cap =
        E->n_xcd > 0 ? (long long)E->n_xcd * ceil_div(max_sessions, E->n_xcd) * per_session : 0;
    E->work_cap = (int)std::min<long long>(
        kMaxWork, std::max((long long)max_sessions * per_session, placed_cap));
    E->rec_words = (size_t)page_size * (config->kv_lora_rank + config->head_dim_rope);
    E->refs.assign(num_pages, 0);
    for (int p = num_pages - 1; p >= 0; --p)
        E->free_.push_back(p);
    E->sessions.resize(max_sessions);
    if (int st = mla_model_create(config, params, max_rows, page_size, &E->model))
        return bail(st);
    hipError_t e = hipStreamCreateWithFlags(&E->stream, hipStreamNonBlocking);
    const int L = config->n_layers, V = config->vocab_size, H = config->n_heads;
    const size_t S = max_sessions;
    E->in_cap = 3 * S + 1 + 2 * (size_t)max_rows + S * E->max_pages;
    E->ws_bytes = mla_decode_workspace_bytes(E->work_cap, max_sessions, H,
                                             config->kv_lora_rank);
    if (e == hipSuccess) e = E->dalloc(E->pool, (size_t)L * num_pages * E->rec_words);
    if (e == hipSuccess) e = hipMemset(E->pool, 0, (size_t)L * num_pages * E->rec_words * 2);
    if (e == hipSuccess) e = E->dalloc(E->d_in, E->in_cap);
    if (e == hipSuccess) e = E->dalloc(E->cu_q, S + 1);
    if (e == hipSuccess) e = E->dalloc(E->cu_k, S + 1);
    if (e == hipSuccess) e = E->dalloc(E->table, S * E->max_pages);
    if (e == hipSuccess) e = E->dalloc(E->slots, max_rows);
    if (e == hipSuccess) e = E->dalloc(E->nsplit, S);
    if (e == hipSuccess) e = E->dalloc(E->cu_split, S + 1);
    if (e == hipSuccess) e = E->dalloc(E->w_sess, E->work_cap);
    if (e == hipSuccess) e = E->dalloc(E->w_split, E->work_cap);
    if (e == hipSuccess) e = E->dalloc(E->w_desc, (size_t)E->work_cap * MLA_WORK_DESC_INTS);
    if (e == hipSuccess) e = E->dalloc(E->w_pages, (size_t)E->work_cap * MLA_WORK_PAGES);
    if (e == hipSuccess) e = E->dalloc(E->info, MLA_INFO_INTS);
    if (e == hipSuccess) e = E->dalloc(E->d_next, S);
    if (e == hipSuccess) e = E->dalloc(E->d_logits, S * V);
    if (e == hipSuccess) {
        uint8_t* w = nullptr;
        e = E->dalloc(w, E->ws_bytes);
        E->workspace = w;
    }
    if (e == hipSuccess)  // the fused merge's counters start at zero
        e = hipMemset(E->workspace, 0, E->ws_bytes);
    if (e == hipSuccess) e = E->halloc(E->h_in, E->in_cap);
    if (e == hipSuccess) e = E->halloc(E->h_logits, S * V);
    if (e == hipSuccess) e = E->halloc(E->h_out, kHostNext + S);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess)
        return bail(gpu_status(e, "mla_engine_create"));
    for (int l = 0; l < L; ++l)
        E->layer_pools.push_back(E->pool + (size_t)l * num_pages * E->rec_words);
    *engine = E;
    return MLA_OK;
}

int mla_engine_destroy(void* engine) {
    delete as_engine(engine);
    return MLA_OK;
}

int mla_engine_info(void* engine, int64_t* info) {
    Engine* E = as_engine(engine);
    if (!E || !info)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_info: invalid argument");
    std::lock_guard lock(E->mu);
    int active = 0;
    for (const Session& S : E->sessions)
        active += S.active;
    info[0] = active;
    info[1] = (int64_t)E->free_.size();
    info[2] = E->num_pages;
    info[3] = E->page_size;
    info[4] = E->max_rows;
    info[5] = E->max_sessions;
    info[6] = (int64_t)E->steps;
    info[7] = (int64_t)E->rec_words * 2 * E->cfg.n_layers * E->num_pages;
    return MLA_OK;
}

int mla_engine_config(void* engine, mla_model_config* config) {
    Engine* E = as_engine(engine);
    if (!E || !config)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_config: invalid argument");
    *config = E->cfg;
    return MLA_OK;
}

int mla_session_create(void* engine, int* session) {
    Engine* E = as_engine(engine);
    if (!E || !session)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_create: invalid argument");
    std::lock_guard lock(E->mu);
    for (int s = 0; s < E->max_sessions; ++s)
        if (!E->sessions[s].active) {
            E->sessions[s] = Session{};
            E->sessions[s].active = true;
            *session = s;
            return MLA_OK;
        }
    return fail(MLA_ERR_OUT_OF_MEMORY, "mla_session_create: every session slot is in use");
}

int mla_session_fork(void* engine, int source, int* session) {
    Engine* E = as_engine(engine);
    if (!E || !session)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_fork: invalid argument");
    std::lock_guard lock(E->mu);
    if (int st = check_session(E, source, "mla_session_fork"))
        return st;
    for (int s = 0; s < E->max_sessions; ++s)
        if (!E->sessions[s].active) {
            E->sessions[s] = E->sessions[source];  // same pages, same length
            for (int32_t p : E->sessions[s].pages)
                ++E->refs[p];
            *session = s;
            return MLA_OK;
        }
    return fail(MLA_ERR_OUT_OF_MEMORY, "mla_session_fork: every session slot is in use");
}

int mla_session_release(void* engine, int session) {
    Engine* E = as_engine(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_release: invalid argument");
    std::lock_guard lock(E->mu);
    if (int st = check_session(E, session, "mla_session_release"))
        return st;
    release_pages(E, E->sessions[session]);
    E->sessions[session].active = false;
    return MLA_OK;
}

int mla_session_length(void* engine, int session, int* length) {
    Engine* E = as_engine(engine);
    if (!E || !length)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_length: invalid argument");
    std::lock_guard lock(E->mu);
    if (int st = check_session(E, session, "mla_session_length"))
        return st;
    *length = E->sessions[session].length;
    return MLA_OK;
}

int mla_session_prefill(void* engine, int session, const uint16_t* ids, int n, float* logits) {
    Engine* E = as_engine(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_prefill: invalid argument");
    std::lock_guard lock(E->mu);
    if (int st = check_session(E, session, "mla_session_prefill"))
        return st;
    Session& S = E->sessions[session];
    release_pages(E, S);  // CpuDecoder::prefill restarts at position 0 (inference.cpp:48)
    if (!ids || n < 1 || n > E->cfg.max_sequence_length)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Prompt exceeds context or is empty");
    for (int i = 0; i < n; ++i)
        if (ids[i] >= E->cfg.vocab_size)
            return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_prefill: token exceeds vocabulary");
    // Chunks of at most max_rows tokens, each appended on top of the previous ones.
    for (int off = 0; off < n;) {
        const int cnt = std::min(n - off, E->max_rows);
        const bool last = off + cnt == n;
        if (int st = step(E, 1, &session, &cnt, ids + off, last ? logits : nullptr, nullptr,
                          "mla_session_prefill")) {
            release_pages(E, S);
            return st;
        }
        off += cnt;
    }
    return MLA_OK;
}

int mla_session_decode(void* engine, int session, uint16_t token, float* logits) {
    Engine* E = as_engine(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_session_decode: invalid argument");
    std::lock_guard lock(E->mu);
    if (int st = check_session(E, session, "mla_session_decode"))
        return st;
    const Session& S = E->sessions[session];
    // inference.cpp:71-75
    if (S.length < 1 || S.length >= E->cfg.max_sequence_length || token >= E->cfg.vocab_size)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "Decode requires current-weight prefill, available context, and a valid "
                    "token");
    const int one = 1;
    return step(E, 1, &session, &one, &token, logits, nullptr, "mla_session_decode");
}

int mla_engine_set_banned(void* engine, const uint16_t* ids, size_t n) {
    Engine* E = static_cast<Engine*>(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_set_banned: null engine");
    std::lock_guard<std::mutex> lock(E->mu);
    return mla_model_set_banned(E->model, ids, n);
}

int mla_engine_step(void* engine, int n, const int* sessions, const int* counts,
                    const uint16_t* tokens, float* logits, int32_t* next_tokens) {
    Engine* E = as_engine(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_step: invalid argument");
    std::lock_guard lock(E->mu);
    return step(E, n, sessions, counts, tokens, logits, next_tokens, "mla_engine_step");
}

int mla_engine_update_weights(void* engine, const float* params) {
    Engine* E = as_engine(engine);
    if (!E || !params)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_update_weights: invalid argument");
    std::lock_guard lock(E->mu);
    if (hipError_t e = hipStreamSynchronize(E->stream); e != hipSuccess)
        return gpu_status(e, "mla_engine_update_weights");
    ++E->host_waits;
    uint64_t rev = 0;
    if (int st = mla_model_update_weights(E->model, params, &rev))
        return st;
    // Every cached token was computed with the old weights: sessions must prefill again
    // (CpuDecoder::decode's revision check, inference.cpp:71-75).
    E->revision = rev;
    return MLA_OK;
}

int mla_engine_stats(void* engine, uint64_t* stats) {
    Engine* E = as_engine(engine);
    if (!E || !stats)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_stats: invalid argument");
    std::lock_guard lock(E->mu);
    stats[0] = E->steps;
    stats[1] = E->host_waits;
    stats[2] = E->meta_launches + model_launches(static_cast<Model*>(E->model));
    stats[3] = E->copies;
    stats[4] = E->revision;
    stats[5] = E->reruns;
    return MLA_OK;
}

int mla_engine_forward(void* engine, int batch, int sequence, const uint16_t* ids,
                       float* logits) {
    Engine* E = as_engine(engine);
    if (!E)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_forward: invalid argument");
    std::lock_guard lock(E->mu);
    const mla_model_config& c = E->cfg;
    if (!ids || !logits || batch < 1 || sequence < 1 || sequence > c.max_sequence_length ||
        (long long)batch * sequence > (1LL << 31) / std::max(1, c.vocab_size))
        return fail(MLA_ERR_INVALID_ARGUMENT, "Forward requires a positive batch and sequence "
                                              "within the context");
    for (long long k = 0; k < (long long)batch * sequence; ++k)
        if (ids[k] >= c.vocab_size)
            return fail(MLA_ERR_INVALID_ARGUMENT, "mla_engine_forward: token exceeds vocabulary");
    hipError_t e = hipSuccess;
    if (!E->d_logits_all) {
        e = E->dalloc(E->d_logits_all, (size_t)E->max_rows * c.vocab_size);
        if (e == hipSuccess)
            e = E->dalloc(E->d_next_all, (size_t)E->max_rows);
        if (e == hipSuccess)
            e = E->halloc(E->h_logits_all, (size_t)E->max_rows * c.vocab_size);
        if (e != hipSuccess) {
            E->d_logits_all = nullptr;
            return gpu_status(e, "mla_engine_forward");
        }
    }
    // Temporary sessions, one per sequence; a step takes whole rows of as many sequences
    // as fit in max_rows (a longer sequence goes through in chunks of its own), so each
    // chunk's rows attend to everything before them in their sequence (causality makes
    // the chunks equal to one full pass, tests/test_model.cpp:65-77).
    std::vector<int> temp;
    auto release_all = [&]() {
        for (int s : temp) {
            release_pages(E, E->sessions[s]);
            E->sessions[s].active = false;
        }
        temp.clear();
    };
    const int per_step = std::max(1, E->max_rows / sequence);
    for (int b0 = 0; b0 < batch;) {
        const int nb = std::min(per_step, batch - b0);
        for (int s = 0; s < E->max_sessions && (int)temp.size() < nb; ++s)
            if (!E->sessions[s].active) {
                E->sessions[s] = Session{};
                E->sessions[s].active = true;
                temp.push_back(s);
            }
        if ((int)temp.size() < nb) {
            release_all();
            return fail(MLA_ERR_OUT_OF_MEMORY, "mla_engine_forward: no free session slots");
        }
        for (int off = 0; off < sequence;) {
            const int cnt = std::min(sequence - off, E->max_rows);
            std::vector<int> counts(nb, cnt);
            std::vector<uint16_t> toks((size_t)nb * cnt);
            for (int i = 0; i < nb; ++i)
                std::memcpy(toks.data() + (size_t)i * cnt,
                            ids + (size_t)(b0 + i) * sequence + off, (size_t)cnt * 2);
            const int st = step(E, nb, temp.data(), counts.data(), toks.data(), E->h_logits_all,
                                nullptr, "mla_engine_forward", true);
            if (st && st != MLA_ERR_NUMERICAL) {
                release_all();
                return st;
            }
            for (int i = 0; i < nb; ++i)
                std::memcpy(logits + ((size_t)(b0 + i) * sequence + off) * c.vocab_size,
                            E->h_logits_all + (size_t)i * cnt * c.vocab_size,
                            (size_t)cnt * c.vocab_size * sizeof(float));
            if (st) {  // a non-finite logit: the rows are out, the error stands
                release_all();
                return st;
            }
            off += cnt;
        }
        release_all();
        b0 += nb;
    }
    return MLA_OK;
}

}  // extern "C"
