// Continuous-batching speculative scheduler and prefix cache (host code).
//
// BatchScheduler (src/paged/scheduler.rs:37-534) runs one packed forward per
// step: admit waiting requests while pages allow (:221-296), feed prefill
// chunks and one-token decodes under max_batch_tokens in request-id order
// (:299-337), sample, stream, stop on EOS / max tokens (:369-480) and reap
// (:482-517).  Here a decode is a speculative round (vx_spec_step: D draft
// tokens, one verify forward, acceptance), so a decoding request costs
// draft_k + 1 verify rows of the budget and may commit several tokens per
// step.  PrefixCache (src/paged/prefix_cache.rs) keys whole prompt pages by a
// chained hash; here an entry holds the target and the draft page of the
// same positions, and stores its tokens and parent hash so that a hash
// collision is a miss, never a wrong page.
//
// Differences from the reference, all deliberate:
//  * prompt pages enter the cache as soon as the prefill has written them
//    (the reference inserts when the request finishes, :482-505), so
//    requests running at the same time share them;
//  * a waiting request whose next uncached page is being prefilled by a
//    running request waits for it instead of computing it again;
//  * prefill is cut into chunks at the budget (the reference defers a whole
//    prompt that does not fit, :316-320);
//  * the lookup never matches the page holding prompt position len - 1:
//    that position is written by the first round's verify forward, and a
//    shared page is never written.
//
// No HIP calls: the engine is reached through vx_sched_backend only.

#include <algorithm>
#include <chrono>
#include <cstring>
#include <deque>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "velox_hip.h"

namespace vx {
int set_error(const std::string &msg);
int spec_sched_backend(vx_spec *e, void *stream, vx_sched_backend *out, void (**release)(void *));
}  // namespace vx

#define SX_REQUIRE(cond, msg)                     \
    do {                                          \
        if (!(cond)) return vx::set_error(msg);   \
    } while (0)

// An engine call failed: keep its message, or name the call when it left none.
#define SX_ENGINE(call, what)                                                         \
    do {                                                                              \
        vx::set_error("");                                                            \
        if ((call) != 0) {                                                            \
            if (!*vx_last_error()) vx::set_error("scheduler: engine " what " failed"); \
            return -1;                                                                \
        }                                                                             \
    } while (0)

namespace {

constexpr uint64_t kChainSeed = 0x243F6A8885A308D3ull;  // any fixed non-zero value

uint64_t mix64(uint64_t x) {  // splitmix64 finaliser
    x ^= x >> 30;
    x *= 0xBF58476D1CE4E5B9ull;
    x ^= x >> 27;
    x *= 0x94D049BB133111EBull;
    x ^= x >> 31;
    return x;
}

// h_n = H(h_{n-1}, tokens of page n)
uint64_t chain(uint64_t h, const uint32_t *t, int64_t n) {
    for (int64_t i = 0; i < n; i++) h = mix64(h ^ ((uint64_t)t[i] << 1 | 1ull) ^ ((uint64_t)i << 40));
    return h;
}

// ---------------------------------------------------------------------------
// prefix cache over (target page, draft page) pairs
// ---------------------------------------------------------------------------
class PrefixCache {
   public:
    PrefixCache(const vx_sched_backend &be, int64_t capacity) : be_(be), cap_(capacity) {}
    ~PrefixCache() { clear(); }

    struct Match {
        int64_t pages = 0;
        std::vector<uint32_t> tp, dp;
        uint64_t next_hash = kChainSeed;  // chain value after the matched pages
    };

    // Longest cached prefix of prompt, whole pages only, at most max_pages.
    // No side effects (PrefixCache::lookup without the incref).
    Match match(const uint32_t *prompt, int64_t max_pages) const {
        Match m;
        const int64_t ps = be_.page_size;
        uint64_t h = kChainSeed;
        for (int64_t p = 0; p < max_pages; p++) {
            const uint32_t *t = prompt + p * ps;
            const uint64_t hn = chain(h, t, ps);
            auto it = map_.find(hn);
            if (it == map_.end() || it->second.parent != h ||
                memcmp(it->second.tokens.data(), t, (size_t)ps * 4) != 0)
                break;
            m.tp.push_back(it->second.tp);
            m.dp.push_back(it->second.dp);
            h = hn;
            m.pages++;
        }
        m.next_hash = h;
        return m;
    }

    // The caller becomes a co-owner of the matched pages (lookup's incref,
    // prefix_cache.rs:150-160); the entries become most recently used.
    void acquire(const uint32_t *prompt, const Match &m) {
        if (m.pages == 0) return;
        uint64_t h = kChainSeed;
        for (int64_t p = 0; p < m.pages; p++) {
            h = chain(h, prompt + p * be_.page_size, be_.page_size);
            auto it = map_.find(h);
            lru_.splice(lru_.end(), lru_, it->second.pos);
        }
        be_.incref(be_.ctx, 0, m.tp.data(), m.pages);
        be_.incref(be_.ctx, 1, m.dp.data(), m.pages);
    }

    // Registers pages [first, first + n) of prompt (insert,
    // prefix_cache.rs:177-203); start_hash is the chain value before page
    // `first`.  Returns the chain value after the last page.
    uint64_t insert(const uint32_t *prompt, int64_t first, int64_t n, uint64_t start_hash, const uint32_t *tp,
                    const uint32_t *dp) {
        const int64_t ps = be_.page_size;
        uint64_t h = start_hash;
        for (int64_t i = 0; i < n; i++) {
            const uint32_t *t = prompt + (first + i) * ps;
            const uint64_t hn = chain(h, t, ps);
            if (cap_ > 0 && !map_.count(hn)) {  // present (or a collision): keep the existing entry
                Entry en;
                en.parent = h;
                en.tokens.assign(t, t + ps);
                en.tp = tp[i];
                en.dp = dp[i];
                be_.incref(be_.ctx, 0, &en.tp, 1);
                be_.incref(be_.ctx, 1, &en.dp, 1);
                en.pos = lru_.insert(lru_.end(), hn);
                map_.emplace(hn, std::move(en));
                evict_to_capacity();
            }
            h = hn;
        }
        return h;
    }

    void clear() {
        for (auto &kv : map_) release(kv.second);
        map_.clear();
        lru_.clear();
    }

    int64_t size() const { return (int64_t)map_.size(); }

   private:
    struct Entry {
        uint64_t parent = 0;
        std::vector<uint32_t> tokens;
        uint32_t tp = 0, dp = 0;
        std::list<uint64_t>::iterator pos;
    };

    void release(const Entry &e) {
        be_.decref(be_.ctx, 0, &e.tp, 1);
        be_.decref(be_.ctx, 1, &e.dp, 1);
    }

    void evict_to_capacity() {  // prefix_cache.rs:205-216
        while ((int64_t)map_.size() > cap_ && !lru_.empty()) {
            auto it = map_.find(lru_.front());
            lru_.pop_front();
            release(it->second);
            map_.erase(it);
        }
    }

    const vx_sched_backend &be_;
    int64_t cap_;
    std::unordered_map<uint64_t, Entry> map_;
    std::list<uint64_t> lru_;  // front = least recently used
};

enum { ST_WAITING = 0, ST_RUNNING = 1, ST_FINISHED = 2, ST_ABORTED = 3 };
enum { FIN_NONE = 0, FIN_STOP = 1, FIN_LENGTH = 2, FIN_CANCELLED = 3 };

struct Request {
    int64_t id = 0;
    std::vector<uint32_t> prompt, generated;
    int64_t max_new = 1;
    float temperature = 0.f;
    uint32_t stream = 0;
    int status = ST_WAITING, finish = FIN_NONE;
    int64_t state = -1;
    int64_t kv = 0;  // prompt positions in KV
    bool ready = false;
    int64_t registered = 0;       // prompt pages [0, registered) are in the cache or came from it
    uint64_t chain = kChainSeed;  // chain value after page `registered`
    std::vector<uint64_t> pending;  // hashes of pages this request will still register
};

}  // namespace

struct vx_sched {
    vx_sched_backend be{};
    void (*release_ctx)(void *) = nullptr;
    vx_sched_config cfg{};
    std::vector<uint32_t> eos;
    std::unique_ptr<PrefixCache> cache;
    std::mutex mu;
    int64_t next_id = 1;
    std::map<int64_t, std::unique_ptr<Request>> reqs;  // every live record, by id
    std::deque<int64_t> waiting;                       // FCFS
    std::map<int64_t, Request *> running;              // ordered by id (scheduler.rs:309-311)
    std::unordered_map<uint64_t, int> pending;         // page hashes running prefills will register
    vx_sched_stats stats{};

    ~vx_sched() {
        for (auto &kv : running)
            if (kv.second->state >= 0) be.free_state(be.ctx, kv.second->state);
        cache.reset();
        if (release_ctx) release_ctx(be.ctx);
    }

    int64_t ps() const { return be.page_size; }
    // whole pages of prompt[..len-1]: the only pages a lookup may match
    int64_t prompt_pages(const Request &r) const { return ((int64_t)r.prompt.size() - 1) / ps(); }

    void drop_pending(Request &r) {
        for (uint64_t h : r.pending) {
            auto it = pending.find(h);
            if (it != pending.end() && --it->second == 0) pending.erase(it);
        }
        r.pending.clear();
    }

    void finish(Request &r, int status, int reason) {
        if (r.state >= 0) be.free_state(be.ctx, r.state);
        r.state = -1;
        drop_pending(r);
        r.status = status;
        r.finish = reason;
        running.erase(r.id);
    }

    // Registers the prompt pages the prefill has completed.
    int register_pages(Request &r) {
        const int64_t done = std::min(r.kv / ps(), prompt_pages(r));
        if (done <= r.registered) return 0;
        const int64_t nb = be.state_pages(be.ctx, r.state, 0, nullptr, 0);
        SX_REQUIRE(nb >= done, "scheduler: state block table shorter than its prefill");
        std::vector<uint32_t> tp(nb), dp(nb);
        SX_REQUIRE(be.state_pages(be.ctx, r.state, 0, tp.data(), nb) == nb &&
                       be.state_pages(be.ctx, r.state, 1, dp.data(), nb) == nb,
                   "scheduler: block tables of the two models differ");
        if (cache)
            r.chain = cache->insert(r.prompt.data(), r.registered, done - r.registered, r.chain,
                                    tp.data() + r.registered, dp.data() + r.registered);
        // these pages are now cached: later requests stop waiting for them
        const int64_t n_done = done - r.registered;
        for (int64_t i = 0; i < n_done && !r.pending.empty(); i++) {
            auto it = pending.find(r.pending.front());
            if (it != pending.end() && --it->second == 0) pending.erase(it);
            r.pending.erase(r.pending.begin());
        }
        r.registered = done;
        return 0;
    }

    // admit_waiting (scheduler.rs:221-296)
    void admit() {
        const int64_t k = cfg.draft_k;
        for (auto it = waiting.begin(); it != waiting.end();) {
            if ((int64_t)running.size() >= cfg.max_running_requests) break;
            Request &r = *reqs.at(*it);
            const int64_t len = (int64_t)r.prompt.size();
            const int64_t max_pages = prompt_pages(r);
            PrefixCache::Match m;
            if (cache) m = cache->match(r.prompt.data(), max_pages);
            // the next uncached page is being prefilled by a running request: wait for it
            if (cache && m.pages < max_pages) {
                const uint64_t hn = chain(m.next_hash, r.prompt.data() + m.pages * ps(), ps());
                if (pending.count(hn)) {
                    ++it;
                    continue;
                }
            }
            if (cache) cache->acquire(r.prompt.data(), m);
            int64_t state = -1;
            const int64_t reserve = len + r.max_new + k;
            if (be.add_state(be.ctx, r.prompt.data(), len, m.pages * ps(), m.tp.data(), m.dp.data(), reserve,
                             r.stream, r.temperature, &state) != 0) {
                // not enough pages: give the cache references back, keep FCFS order
                if (m.pages) {
                    be.decref(be.ctx, 0, m.tp.data(), m.pages);
                    be.decref(be.ctx, 1, m.dp.data(), m.pages);
                }
                break;
            }
            if (cache) {
                if (m.pages) {
                    stats.prefix_cache_hits++;
                    stats.prefix_tokens_skipped += (uint64_t)(m.pages * ps());
                } else {
                    stats.prefix_cache_misses++;
                }
            }
            r.state = state;
            r.kv = m.pages * ps();
            r.ready = r.kv == len - 1;
            r.registered = m.pages;
            r.chain = m.next_hash;
            r.status = ST_RUNNING;
            if (cache) {
                uint64_t h = m.next_hash;
                for (int64_t p = m.pages; p < max_pages; p++) {
                    h = chain(h, r.prompt.data() + p * ps(), ps());
                    r.pending.push_back(h);
                    pending[h]++;
                }
            }
            running[r.id] = &r;
            it = waiting.erase(it);
        }
    }

    int step(int64_t *out_tokens) {
        const auto t0 = std::chrono::steady_clock::now();
        *out_tokens = 0;
        admit();
        if (running.empty()) return 0;
        const int64_t k = cfg.draft_k;
        std::vector<Request *> pre, dec;
        std::vector<int64_t> pre_states, pre_n;
        int64_t total = 0;
        for (auto &kv : running) {
            Request &r = *kv.second;
            if (!r.ready) {
                const int64_t rest = (int64_t)r.prompt.size() - 1 - r.kv;
                const int64_t take = std::min(rest, cfg.max_batch_tokens - total);
                if (take <= 0) continue;
                pre.push_back(&r);
                pre_states.push_back(r.state);
                pre_n.push_back(take);
                total += take;
            } else {
                if (total > 0 && total + k + 1 > cfg.max_batch_tokens) continue;  // defer (scheduler.rs:316-320)
                dec.push_back(&r);
                total += k + 1;
            }
        }
        if (total == 0) return 0;
        if (!pre.empty()) {
            SX_ENGINE(be.prefill_chunk(be.ctx, pre_states.data(), pre_n.data(), (int64_t)pre.size()), "prefill");
            for (size_t i = 0; i < pre.size(); i++) {
                Request &r = *pre[i];
                r.kv += pre_n[i];
                stats.prefill_tokens += (uint64_t)pre_n[i];
                if (r.kv == (int64_t)r.prompt.size() - 1) r.ready = true;
                if (register_pages(r) != 0) return -1;
            }
        }
        // one round per distinct temperature, in id order within each
        std::vector<bool> done(dec.size(), false);
        std::vector<Request *> reap;
        for (size_t g = 0; g < dec.size(); g++) {
            if (done[g]) continue;
            std::vector<Request *> grp;
            for (size_t j = g; j < dec.size(); j++)
                if (!done[j] && dec[j]->temperature == dec[g]->temperature) {
                    grp.push_back(dec[j]);
                    done[j] = true;
                }
            const int64_t n = (int64_t)grp.size();
            std::vector<int64_t> st(n);
            for (int64_t b = 0; b < n; b++) st[b] = grp[b]->state;
            std::vector<vx_round_outcome> out(n);
            std::vector<uint32_t> com((size_t)n * (k + 1));
            SX_ENGINE(be.step(be.ctx, st.data(), n, k, out.data(), com.data()), "step");
            stats.rounds++;
            for (int64_t b = 0; b < n; b++) {
                Request &r = *grp[b];
                stats.draft_tokens_proposed += (uint64_t)k;
                stats.draft_tokens_accepted += (uint64_t)std::max(out[b].accepted, 0);
                for (int32_t i = 0; i < out[b].n_committed; i++) {
                    const uint32_t t = com[(size_t)b * (k + 1) + i];
                    r.generated.push_back(t);
                    stats.tokens_generated++;
                    const bool is_eos = std::find(eos.begin(), eos.end(), t) != eos.end();
                    if (is_eos || (int64_t)r.generated.size() >= r.max_new) {
                        r.finish = is_eos ? FIN_STOP : FIN_LENGTH;  // scheduler.rs:463-479
                        break;
                    }
                }
                if (r.finish != FIN_NONE) reap.push_back(&r);
            }
        }
        for (Request *r : reap) {
            finish(*r, ST_FINISHED, r->finish);
            stats.requests_completed++;
        }
        stats.steps++;
        stats.last_batch_size = pre.size() + dec.size();
        stats.last_step_us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                                 std::chrono::steady_clock::now() - t0)
                                 .count();
        *out_tokens = total;
        return 0;
    }
};

namespace {
int make_sched(const vx_sched_backend &be, void (*release)(void *), const vx_sched_config *cfg,
               const uint32_t *eos_ids, int64_t n_eos, vx_sched **out) {
    auto s = std::make_unique<vx_sched>();
    s->be = be;
    s->release_ctx = release;
    if (!cfg || !out || (n_eos > 0 && !eos_ids) || be.page_size < 1 || !be.add_state || !be.prefill_chunk ||
        !be.step || !be.state_pages || !be.free_state || !be.incref || !be.decref) {
        s->release_ctx = nullptr;  // the caller keeps its context on argument errors
        return vx::set_error("scheduler: null or incomplete argument");
    }
    if (cfg->max_running_requests < 1 || cfg->max_batch_tokens < 1 || cfg->prefix_cache_capacity < 0 ||
        cfg->draft_k < 1 || cfg->draft_k + 1 > 64) {
        s->release_ctx = nullptr;
        return vx::set_error("scheduler: max_running_requests, max_batch_tokens >= 1, draft_k in [1, 63]");
    }
    s->cfg = *cfg;
    s->eos.assign(eos_ids, eos_ids + std::max<int64_t>(n_eos, 0));
    if (cfg->prefix_cache_capacity > 0) s->cache = std::make_unique<PrefixCache>(s->be, cfg->prefix_cache_capacity);
    *out = s.release();
    return 0;
}
}  // namespace

extern "C" int vx_sched_create(vx_spec *engine, const vx_sched_config *cfg, const uint32_t *eos_ids, int64_t n_eos,
                               void *stream, vx_sched **out) {
    SX_REQUIRE(engine, "scheduler: null engine");
    vx_sched_backend be{};
    void (*release)(void *) = nullptr;
    if (vx::spec_sched_backend(engine, stream, &be, &release) != 0) return -1;
    const int rc = make_sched(be, release, cfg, eos_ids, n_eos, out);
    if (rc != 0) release(be.ctx);
    return rc;
}

extern "C" int vx_sched_create_with_backend(const vx_sched_backend *backend, const vx_sched_config *cfg,
                                            const uint32_t *eos_ids, int64_t n_eos, vx_sched **out) {
    SX_REQUIRE(backend, "scheduler: null backend");
    return make_sched(*backend, nullptr, cfg, eos_ids, n_eos, out);
}

extern "C" void vx_sched_destroy(vx_sched *s) { delete s; }

extern "C" int vx_sched_submit(vx_sched *s, const uint32_t *prompt, int64_t len, int64_t max_new_tokens,
                               float temperature, int64_t stream, int64_t *out_id) {
    SX_REQUIRE(s && out_id && (prompt || len == 0), "submit: null argument");
    if (len <= 0) return vx::set_error("Empty prompt");
    SX_REQUIRE(len >= 2, "speculative prefill requires a prompt with at least 2 tokens");
    std::lock_guard<std::mutex> lk(s->mu);
    auto r = std::make_unique<Request>();
    r->id = s->next_id++;
    r->prompt.assign(prompt, prompt + len);
    r->max_new = std::max<int64_t>(max_new_tokens, 1);
    r->temperature = temperature <= 1e-7f ? 0.f : temperature;
    r->stream = (uint32_t)(stream < 0 ? r->id : stream);
    *out_id = r->id;
    s->waiting.push_back(r->id);
    s->reqs[r->id] = std::move(r);
    return 0;
}

extern "C" int vx_sched_step(vx_sched *s, int64_t *out_tokens) {
    SX_REQUIRE(s && out_tokens, "step: null argument");
    std::lock_guard<std::mutex> lk(s->mu);
    return s->step(out_tokens);
}

extern "C" int vx_sched_poll(vx_sched *s, int64_t id, uint32_t *tokens, int64_t cap, int64_t *n_tokens, int *status,
                             int *finish_reason) {
    SX_REQUIRE(s, "poll: null scheduler");
    std::lock_guard<std::mutex> lk(s->mu);
    auto it = s->reqs.find(id);
    SX_REQUIRE(it != s->reqs.end(), "poll: unknown request");
    const Request &r = *it->second;
    if (tokens && cap > 0)
        memcpy(tokens, r.generated.data(), (size_t)std::min<int64_t>(cap, (int64_t)r.generated.size()) * 4);
    if (n_tokens) *n_tokens = (int64_t)r.generated.size();
    if (status) *status = r.status;
    if (finish_reason) *finish_reason = r.finish;
    return 0;
}

extern "C" int vx_sched_abort(vx_sched *s, int64_t id) {
    SX_REQUIRE(s, "abort: null scheduler");
    std::lock_guard<std::mutex> lk(s->mu);
    auto it = s->reqs.find(id);
    SX_REQUIRE(it != s->reqs.end(), "abort: unknown request");
    Request &r = *it->second;
    if (r.status == ST_WAITING) {
        s->waiting.erase(std::find(s->waiting.begin(), s->waiting.end(), id));
        r.status = ST_ABORTED;
        r.finish = FIN_CANCELLED;
    } else if (r.status == ST_RUNNING) {
        s->finish(r, ST_ABORTED, FIN_CANCELLED);
    } else {
        return 0;
    }
    s->stats.requests_aborted++;
    return 0;
}

extern "C" int vx_sched_release(vx_sched *s, int64_t id) {
    SX_REQUIRE(s, "release: null scheduler");
    std::lock_guard<std::mutex> lk(s->mu);
    auto it = s->reqs.find(id);
    SX_REQUIRE(it != s->reqs.end(), "release: unknown request");
    SX_REQUIRE(it->second->status == ST_FINISHED || it->second->status == ST_ABORTED,
               "release: request still waiting or running");
    s->reqs.erase(it);
    return 0;
}

extern "C" int vx_sched_get_stats(vx_sched *s, vx_sched_stats *out) {
    SX_REQUIRE(s && out, "stats: null argument");
    std::lock_guard<std::mutex> lk(s->mu);
    *out = s->stats;
    return 0;
}

extern "C" int64_t vx_sched_num_waiting(vx_sched *s) {
    if (!s) return -1;
    std::lock_guard<std::mutex> lk(s->mu);
    return (int64_t)s->waiting.size();
}

extern "C" int64_t vx_sched_num_running(vx_sched *s) {
    if (!s) return -1;
    std::lock_guard<std::mutex> lk(s->mu);
    return (int64_t)s->running.size();
}

extern "C" int64_t vx_sched_cache_pages(vx_sched *s) {
    if (!s) return -1;
    std::lock_guard<std::mutex> lk(s->mu);
    return s->cache ? s->cache->size() : 0;
}
