// rh_sched.cpp -- request scheduler over one context (the multistream
// ForwardScheduler analogue, crates/engine/src/multistream.rs:54-161).
//
// The reference runs N worker threads, each with its own compiled kernels
// and workspace, pulling single-sequence forwards from a bounded channel.
// On one GPU the same concurrency is worth more as batching: one worker
// thread owns the context and drains the queue in batches -- up to max_batch
// forward requests of equal length become one rh_forward launch (M = B * S
// rows), and generation requests with equal prompt length and step count
// become one rh_prefill + rh_decode.  The submit side keeps the reference's
// semantics: a bounded FIFO that blocks when full, results carrying the
// request id, queue wait, service and total time, and run_batch returning
// results sorted by request id.
#include "../../include/rustane_hip.h"
#include "rh_internal.h"

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

namespace {

using Clock = std::chrono::steady_clock;

struct Job {
    int kind = RH_JOB_FORWARD;
    uint64_t id = 0;
    std::vector<uint32_t> tokens, targets;  // forward: tokens/targets [len]; generate: prompt [len]
    int len = 0, nsteps = 0;
    uint32_t* out_tokens = nullptr;         // generate: caller's [nsteps]
    Clock::time_point submitted;
    int status = RH_OK;                     // set at submit for a request that cannot run
    std::string message;
};

// The first id >= vocab in ids[0..n), as an error message; empty if none.
std::string bad_id(const std::vector<uint32_t>& ids, int vocab, const char* what) {
    for (size_t i = 0; i < ids.size(); ++i)
        if (ids[i] >= (uint32_t)vocab)
            return std::string(what) + " id " + std::to_string(ids[i]) + " at index " + std::to_string(i) +
                   " >= vocab " + std::to_string(vocab);
    return std::string();
}

float ms_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<float, std::milli>(b - a).count();
}

}  // namespace

struct rh_sched {
    rh_ctx* ctx = nullptr;
    rh_sched_config cfg{};
    int ctx_max_batch = 0, ctx_max_ctx = 0, vocab = 0;
    std::mutex mu;
    std::condition_variable cv_jobs, cv_space, cv_results;
    std::deque<Job> queue;
    std::deque<rh_sched_result> results;
    int in_flight = 0;  // submitted and not yet returned by rh_sched_wait
    bool stop = false;
    std::thread worker;

    void run();
    void serve(std::vector<Job>& batch);
    void post(const Job& j, int status, float loss, int batch, Clock::time_point t0, Clock::time_point t1,
              const std::string& msg);
};

void rh_sched::post(const Job& j, int status, float loss, int batch, Clock::time_point t0, Clock::time_point t1,
                    const std::string& msg) {
    rh_sched_result r{};
    r.request_id = j.id;
    r.kind = j.kind;
    r.status = status;
    r.loss = loss;
    r.batch = batch;
    r.queue_wait_ms = ms_between(j.submitted, t0);
    r.service_ms = ms_between(t0, t1);
    r.total_ms = ms_between(j.submitted, t1);
    std::strncpy(r.message, msg.c_str(), sizeof(r.message) - 1);
    std::lock_guard<std::mutex> lk(mu);
    results.push_back(r);
    cv_results.notify_all();
}

void rh_sched::serve(std::vector<Job>& batch) {
    const int B = (int)batch.size();
    const Job& j0 = batch[0];
    const auto t0 = Clock::now();
    int rc = RH_OK;
    std::vector<float> loss(B, 0.0f);
    if (j0.status != RH_OK) {  // refused at submit; always served alone
        post(j0, j0.status, 0.0f, 1, t0, Clock::now(), j0.message);
        return;
    }
    if (j0.kind == RH_JOB_FORWARD) {
        const int S = j0.len;
        std::vector<uint32_t> tok((size_t)B * S), tgt((size_t)B * S);
        for (int b = 0; b < B; ++b) {
            std::memcpy(&tok[(size_t)b * S], batch[b].tokens.data(), (size_t)S * 4);
            std::memcpy(&tgt[(size_t)b * S], batch[b].targets.data(), (size_t)S * 4);
        }
        rc = rh_forward(ctx, tok.data(), tgt.data(), B, S, nullptr, nullptr, loss.data());
    } else {
        const int P = j0.len, n = j0.nsteps;
        std::vector<uint32_t> prompt((size_t)B * P), first(B), rest((size_t)std::max(n - 1, 0) * B);
        for (int b = 0; b < B; ++b) std::memcpy(&prompt[(size_t)b * P], batch[b].tokens.data(), (size_t)P * 4);
        rc = rh_prefill(ctx, prompt.data(), B, P, first.data(), nullptr);
        if (rc == RH_OK && n > 1) rc = rh_decode(ctx, B, first.data(), n - 1, rest.data());
        if (rc == RH_OK)
            for (int b = 0; b < B; ++b) {
                batch[b].out_tokens[0] = first[b];
                for (int s = 1; s < n; ++s) batch[b].out_tokens[s] = rest[(size_t)(s - 1) * B + b];
            }
    }
    const auto t1 = Clock::now();
    const std::string msg = rc == RH_OK ? std::string() : std::string(rh_last_error(ctx));
    for (int b = 0; b < B; ++b) post(batch[b], rc, loss[b], B, t0, t1, msg);
}

void rh_sched::run() {
    for (;;) {
        std::vector<Job> batch;
        {
            std::unique_lock<std::mutex> lk(mu);
            cv_jobs.wait(lk, [&] { return stop || !queue.empty(); });
            if (queue.empty()) return;  // stop requested and drained
            const Job& head = queue.front();
            const int cap = head.kind == RH_JOB_FORWARD ? std::min(cfg.max_batch, ctx_max_batch)
                                                        : std::min({cfg.max_batch, ctx_max_batch, 16});
            // Optionally hold the head for up to max_wait_us so a batch can fill.
            if (cfg.max_wait_us > 0 && !stop) {
                const auto deadline = head.submitted + std::chrono::microseconds(cfg.max_wait_us);
                cv_jobs.wait_until(lk, deadline, [&] {
                    if (stop) return true;
                    int same = 0;
                    for (const Job& j : queue)
                        same += j.status == RH_OK && j.kind == queue.front().kind &&
                                j.len == queue.front().len && j.nsteps == queue.front().nsteps;
                    return queue.front().status != RH_OK || same >= cap;
                });
            }
            // FIFO: the head, then every later runnable job with the same
            // shape, up to cap.  A job refused at submit is never batched: its
            // bad ids would fail the whole launch.
            const int kind = queue.front().kind, len = queue.front().len, nsteps = queue.front().nsteps;
            const int batch_cap = queue.front().status == RH_OK ? cap : 1;
            for (auto it = queue.begin(); it != queue.end() && (int)batch.size() < batch_cap;) {
                if (batch.empty() ||
                    (it->status == RH_OK && it->kind == kind && it->len == len && it->nsteps == nsteps)) {
                    batch.push_back(std::move(*it));
                    it = queue.erase(it);
                } else {
                    ++it;
                }
            }
            cv_space.notify_all();
        }
        serve(batch);
    }
}

extern "C" {

int rh_sched_create(rh_ctx* ctx, const rh_sched_config* cfg, rh_sched** out) {
    if (!ctx || !cfg || !out) return rh_internal_fail(ctx, RH_EINVAL, "null argument");
    *out = nullptr;
    if (cfg->max_batch <= 0 || cfg->queue_capacity <= 0 || cfg->max_wait_us < 0)
        return rh_internal_fail(ctx, RH_EINVAL, "scheduler needs max_batch > 0, queue_capacity > 0, max_wait_us >= 0");
    rh_sched* s = new (std::nothrow) rh_sched;
    if (!s) return rh_internal_fail(ctx, RH_ENOMEM, "out of host memory");
    s->ctx = ctx;
    s->cfg = *cfg;
    rh_config c{};
    rh_context_info(ctx, &c, &s->ctx_max_batch, &s->ctx_max_ctx);
    s->vocab = c.vocab;
    try {
        s->worker = std::thread([s] { s->run(); });
    } catch (...) {
        delete s;
        return rh_internal_fail(ctx, RH_ENOMEM, "cannot start the scheduler thread");
    }
    *out = s;
    return RH_OK;
}

void rh_sched_destroy(rh_sched* s) {
    if (!s) return;
    {
        std::lock_guard<std::mutex> lk(s->mu);
        s->stop = true;
    }
    s->cv_jobs.notify_all();
    s->worker.join();  // the worker drains the queue first
    delete s;
}

int rh_sched_submit(rh_sched* s, const rh_sched_request* rq) {
    if (!s || !rq || !rq->tokens || rq->len <= 0) return RH_EINVAL;
    Job j;
    j.kind = rq->kind;
    j.id = rq->request_id;
    j.len = rq->len;
    if (rq->kind == RH_JOB_FORWARD) {
        if (!rq->targets) return RH_EINVAL;
        j.tokens.assign(rq->tokens, rq->tokens + rq->len);
        j.targets.assign(rq->targets, rq->targets + rq->len);
    } else if (rq->kind == RH_JOB_GENERATE) {
        if (rq->nsteps <= 0 || !rq->out_tokens) return RH_EINVAL;
        if (s->ctx_max_ctx <= 0 || rq->len + rq->nsteps > s->ctx_max_ctx) return RH_ERANGE;
        j.nsteps = rq->nsteps;
        j.out_tokens = rq->out_tokens;
        j.tokens.assign(rq->tokens, rq->tokens + rq->len);
    } else {
        return RH_EINVAL;
    }
    // Out-of-range ids fail this request alone (its result carries
    // RH_ERANGE); the reference's per-request workers are independent too.
    j.message = bad_id(j.tokens, s->vocab, "token");
    if (j.message.empty() && j.kind == RH_JOB_FORWARD) j.message = bad_id(j.targets, s->vocab, "target");
    if (!j.message.empty()) j.status = RH_ERANGE;
    std::unique_lock<std::mutex> lk(s->mu);
    if (s->stop) return RH_ESTATE;
    s->cv_space.wait(lk, [&] { return (int)s->queue.size() < s->cfg.queue_capacity; });
    j.submitted = Clock::now();
    s->queue.push_back(std::move(j));
    ++s->in_flight;
    s->cv_jobs.notify_one();
    return RH_OK;
}

int rh_sched_wait(rh_sched* s, rh_sched_result* out) {
    if (!s || !out) return RH_EINVAL;
    std::unique_lock<std::mutex> lk(s->mu);
    if (s->in_flight == 0) return RH_ESTATE;  // nothing submitted: waiting would never end
    s->cv_results.wait(lk, [&] { return !s->results.empty(); });
    *out = s->results.front();
    s->results.pop_front();
    --s->in_flight;
    return RH_OK;
}

int rh_sched_run_batch(rh_sched* s, const rh_sched_request* rq, int n, rh_sched_result* results) {
    if (!s || (n > 0 && (!rq || !results)) || n < 0) return RH_EINVAL;
    {
        std::lock_guard<std::mutex> lk(s->mu);
        if (s->in_flight != 0) return RH_ESTATE;  // results of other submissions would mix in
    }
    int submitted = 0, rc = RH_OK;
    for (; submitted < n; ++submitted)
        if ((rc = rh_sched_submit(s, &rq[submitted])) != RH_OK) break;
    for (int i = 0; i < submitted; ++i) rh_sched_wait(s, &results[i]);
    std::sort(results, results + submitted,
              [](const rh_sched_result& a, const rh_sched_result& b) { return a.request_id < b.request_id; });
    return rc;
}

}  // extern "C"
