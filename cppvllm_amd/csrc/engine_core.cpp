// Host-side serving core: sequences, paged KV block manager with prefix caching, and the
// continuous-batching scheduler with chunked prefill. Plain C++17 (no GPU, no libtorch), exposed
// through include/cppvllm_engine.h.
//
// Behaviour follows the reference engine so that a batch stream (which sequences run, how many
// tokens each, which blocks they own) is the one its kernels would see:
//   * sequence bookkeeping           engine/sequence.h:26-88
//   * block manager                  engine/block_manager.cpp:28-158 (LRF free list, ref counts,
//                                    prefix cache over full blocks keyed by a chained hash)
//   * scheduler                      engine/scheduler.cpp:17-154 (running first under a token
//                                    budget and a per-sequence chunk cap, preemption by recompute
//                                    of the most recently admitted, then FIFO admission)
//   * step groups                    engine/model_runner.cpp:147-196
//   * two-deep launch ring           engine/llm_engine.cpp:70-113 (a step may be scheduled while
//                                    the previous one is still running: its sampled tokens are
//                                    placeholders the runner feeds on the device, batch.feed_src)
// A caller may also run steps synchronously (schedule, then postprocess, then schedule ...).
#include "../../include/cppvllm_engine.h"

#include <algorithm>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <unordered_map>
#include <vector>

namespace cve {
namespace {

constexpr int32_t kPending = -1;       // placeholder of a token being sampled this step
constexpr uint64_t kNoHash = 0;

enum class State : uint8_t { kWaiting, kRunning, kFinished };

struct Seq {
    int64_t id = 0;
    State state = State::kWaiting;
    int32_t max_tokens = 0;
    bool ignore_eos = false;
    std::vector<int32_t> tokens;       // prompt, then generated tokens
    std::vector<int32_t> table;        // physical block of each logical block
    int64_t num_prompt = 0;
    int64_t num_cached = 0;            // tokens whose K/V are in the cache
    int64_t num_sched = 0;             // tokens scheduled in the step being built
    int32_t inflight = 0;              // scheduled steps containing this sequence, not yet post-processed
    int64_t last_row = -1;             // its row in the newest scheduled step, if that step samples it
    bool done = false;                 // finished; its blocks are released once inflight == 0

    int64_t size() const { return static_cast<int64_t>(tokens.size()); }
    int64_t completion() const { return size() - num_prompt; }
    int64_t uncached() const { return size() - num_cached; }
};

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// 64-bit finaliser (MurmurHash3 fmix64) applied after each 32-bit token is folded in, seeded
// with the parent block's hash so that a block's key names its whole prefix.
uint64_t fmix64(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdULL;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ULL;
    x ^= x >> 33;
    return x;
}
uint64_t chain_hash(const int32_t* t, int64_t n, uint64_t parent) {
    uint64_t h = fmix64(parent ^ 0x6a09e667f3bcc909ULL);
    for (int64_t i = 0; i < n; ++i) h = fmix64(h ^ (static_cast<uint64_t>(static_cast<uint32_t>(t[i])) << 1));
    return h == kNoHash ? 1 : h;
}

class BlockManager {
public:
    BlockManager(int32_t n, int32_t bs) : bs_(bs), meta_(n), content_(static_cast<size_t>(n) * bs, 0) {
        for (int32_t i = 0; i < n; ++i) push_free(i);
    }
    int32_t num_blocks() const { return static_cast<int32_t>(meta_.size()); }
    int64_t num_free() const { return nfree_; }
    int32_t ref_count(int32_t id) const { return meta_[id].ref; }
    int64_t hit_tokens() const { return hit_tokens_; }

    // Full blocks of the prompt (never the block holding the last token: its K/V is recomputed
    // so the step that contains it can sample) that the cache already holds, in order.
    int64_t cached_prefix(const Seq& s, std::vector<int32_t>* ids) const {
        const int64_t limit = (s.size() - 1) / bs_;
        uint64_t parent = kNoHash;
        int64_t k = 0;
        for (; k < limit; ++k) {
            const int32_t* t = s.tokens.data() + k * bs_;
            const uint64_t h = chain_hash(t, bs_, parent);
            const auto it = index_.find(h);
            if (it == index_.end()) break;
            const int32_t id = it->second;
            if (!std::equal(t, t + bs_, content_.data() + static_cast<size_t>(id) * bs_)) break;
            if (ids) ids->push_back(id);
            parent = h;
        }
        return k;
    }
    bool can_allocate(const Seq& s) const {
        std::vector<int32_t> hit;
        cached_prefix(s, &hit);
        int64_t need = ceil_div(s.size(), bs_);
        for (int32_t id : hit)
            if (meta_[id].ref > 0) --need;          // shared with a live sequence: no free block used
        return nfree_ >= need;
    }
    void allocate(Seq& s) {
        std::vector<int32_t> hit;
        cached_prefix(s, &hit);
        for (int32_t id : hit) {
            if (meta_[id].ref == 0) unlink_free(id);
            ++meta_[id].ref;
            s.table.push_back(id);
        }
        s.num_cached = static_cast<int64_t>(hit.size()) * bs_;
        hit_tokens_ += s.num_cached;
        while (static_cast<int64_t>(s.table.size()) < ceil_div(s.size(), bs_)) s.table.push_back(take_fresh());
    }
    bool can_append(const Seq& s) const { return nfree_ >= ceil_div(s.size(), bs_) - static_cast<int64_t>(s.table.size()); }
    void append(Seq& s) {
        while (static_cast<int64_t>(s.table.size()) < ceil_div(s.size(), bs_)) s.table.push_back(take_fresh());
    }
    // Register every full, cached block of s that has no key yet (block_manager.cpp:118-134).
    void commit(const Seq& s) {
        const int64_t full = s.num_cached / bs_;
        for (int64_t i = 0; i < full; ++i) {
            Meta& m = meta_[s.table[i]];
            if (m.hash != kNoHash) continue;
            const uint64_t parent = i == 0 ? kNoHash : meta_[s.table[i - 1]].hash;
            const int32_t* t = s.tokens.data() + i * bs_;
            m.hash = chain_hash(t, bs_, parent);
            std::copy(t, t + bs_, content_.begin() + static_cast<size_t>(s.table[i]) * bs_);
            index_.emplace(m.hash, s.table[i]);
        }
    }
    // Drop s's references, last block first, so the tail of a sequence is reused before its
    // (more shareable) head (block_manager.cpp:136-144).
    void release(Seq& s) {
        for (auto it = s.table.rbegin(); it != s.table.rend(); ++it)
            if (--meta_[*it].ref == 0) push_free(*it);
        s.table.clear();
        s.num_cached = 0;
    }

private:
    struct Meta {
        int32_t ref = 0, prev = -1, next = -1;
        uint64_t hash = kNoHash;
    };
    void push_free(int32_t id) {
        Meta& m = meta_[id];
        m.prev = tail_;
        m.next = -1;
        if (tail_ >= 0) meta_[tail_].next = id;
        else head_ = id;
        tail_ = id;
        ++nfree_;
    }
    void unlink_free(int32_t id) {
        Meta& m = meta_[id];
        if (m.prev >= 0) meta_[m.prev].next = m.next;
        else head_ = m.next;
        if (m.next >= 0) meta_[m.next].prev = m.prev;
        else tail_ = m.prev;
        m.prev = m.next = -1;
        --nfree_;
    }
    // Least recently freed block; its old prefix-cache key (if still its own) is forgotten.
    int32_t take_fresh() {
        const int32_t id = head_;
        unlink_free(id);
        Meta& m = meta_[id];
        if (m.hash != kNoHash) {
            const auto it = index_.find(m.hash);
            if (it != index_.end() && it->second == id) index_.erase(it);
            m.hash = kNoHash;
        }
        m.ref = 1;
        return id;
    }

    int32_t bs_;
    std::vector<Meta> meta_;
    std::vector<int32_t> content_;     // tokens of every keyed block, to confirm a hash hit
    std::unordered_map<uint64_t, int32_t> index_;
    int32_t head_ = -1, tail_ = -1;
    int64_t nfree_ = 0;
    int64_t hit_tokens_ = 0;
};

struct Output {
    int64_t id;
    std::vector<int32_t> tokens;
};

class Engine {
public:
    explicit Engine(const cve_config& c) : cfg_(c), bm_(c.num_blocks, c.block_size) {}

    int64_t add(const int32_t* prompt, int64_t n, int32_t max_tokens, bool ignore_eos) {
        if (n <= 0 || !prompt || max_tokens < 0) return CVE_ERR_INVALID_ARG;
        if (ceil_div(n + max_tokens, cfg_.block_size) > bm_.num_blocks()) return CVE_ERR_TOO_LONG;
        auto s = std::make_unique<Seq>();
        s->id = next_id_++;
        s->max_tokens = max_tokens;
        s->ignore_eos = ignore_eos;
        s->tokens.assign(prompt, prompt + n);
        s->tokens.reserve(static_cast<size_t>(n + max_tokens));
        s->num_prompt = n;
        waiting_.push_back(s.get());
        const int64_t id = s->id;
        live_.emplace(id, std::move(s));
        return id;
    }

    int schedule(cve_batch* out) {
        if (flights_.size() >= kMaxFlights) return CVE_ERR_STATE;
        // preemption releases blocks, which is only safe when no scheduled step can still touch them
        std::vector<Seq*> picked = pick(/*allow_preempt=*/flights_.empty());
        if (picked.empty()) {
            *out = cve_batch{};
            if (!flights_.empty()) return CVE_ERR_BUSY;
            return (waiting_.empty() && running_.empty()) ? CVE_OK : CVE_ERR_EMPTY;
        }
        build(picked, out);
        ++stats_.steps;
        return CVE_OK;
    }

    // Accept the sampled tokens of the oldest scheduled step (scheduler.cpp:121-154).
    int postprocess(const int64_t* sampled, int64_t n) {
        if (flights_.empty()) return CVE_ERR_STATE;
        Flight& f = flights_.front();
        if (n != static_cast<int64_t>(f.seqs.size()) || (n > 0 && !sampled)) return CVE_ERR_INVALID_ARG;
        for (int64_t j = 0; j < n; ++j) {
            Seq* s = f.seqs[j];
            --s->inflight;
            const int64_t at = f.at[j];
            if (s->done) continue;               // finished by an older step: a dropped extra token
            if (at < 0) {                        // a prefill chunk that does not reach the end
                bm_.commit(*s);
                continue;
            }
            const int32_t tok = static_cast<int32_t>(sampled[j]);
            s->tokens[at] = tok;
            ++stats_.tokens_sampled;
            const bool eos = !s->ignore_eos && cfg_.eos_token_id >= 0 && tok == cfg_.eos_token_id;
            const bool len = at + 1 - s->num_prompt >= s->max_tokens;
            bm_.commit(*s);
            if (eos || len) {
                s->tokens.resize(static_cast<size_t>(at) + 1);   // drops a newer step's placeholder
                s->done = true;
                s->state = State::kFinished;
                finish(s);
            }
        }
        running_.erase(std::remove_if(running_.begin(), running_.end(),
                                      [](const Seq* s) { return s->state == State::kFinished; }),
                       running_.end());
        std::vector<Seq*> seqs = std::move(f.seqs);
        flights_.pop_front();
        for (Seq* s : seqs)
            if (s->done && s->inflight == 0 && s->table.size() > 0) bm_.release(*s);
        for (Seq* s : seqs)
            if (s->done && s->inflight == 0) live_.erase(s->id);   // frees s (duplicates: find fails)
        return CVE_OK;
    }

    bool finished() const { return waiting_.empty() && running_.empty() && flights_.empty(); }
    int64_t inflight() const { return static_cast<int64_t>(flights_.size()); }
    cve_stats stats() const {
        cve_stats s = stats_;
        s.free_blocks = bm_.num_free();
        s.prefix_hit_tokens = bm_.hit_tokens();
        return s;
    }
    const std::map<int64_t, Output>& outputs() const { return done_; }
    void clear_outputs() { done_.clear(); }
    const BlockManager& blocks() const { return bm_; }
    const Seq* find(int64_t id) const {
        const auto it = live_.find(id);
        return it == live_.end() ? nullptr : it->second.get();
    }

private:
    // Which sequences run this step and how many tokens each (scheduler.cpp:37-103).
    std::vector<Seq*> pick(bool allow_preempt) {
        int64_t budget = cfg_.max_num_batched_tokens;
        const int64_t cap = cfg_.max_chunk_tokens > 0 ? cfg_.max_chunk_tokens : INT64_MAX;
        std::vector<Seq*> out;
        std::deque<Seq*> pending(running_.begin(), running_.end());
        std::vector<Seq*> kept;
        bool preempted = false;
        while (!pending.empty()) {
            Seq* s = pending.front();
            pending.pop_front();
            // a sequence whose last sample (possibly still in flight) completes max_tokens has
            // nothing more to run
            const bool complete = s->inflight > 0 && s->completion() >= s->max_tokens;
            const int64_t want = complete ? 0 : std::min({s->uncached(), budget, cap});
            if (want <= 0 || static_cast<int64_t>(out.size()) >= cfg_.max_num_seqs) {
                kept.push_back(s);
                continue;
            }
            if (!allow_preempt && !bm_.can_append(*s)) {   // wait for the ring to drain
                kept.push_back(s);
                continue;
            }
            bool gave_up = false;
            while (!bm_.can_append(*s)) {      // recompute-preempt the newest running sequence
                Seq* victim = pending.empty() ? s : pending.back();
                if (!pending.empty()) pending.pop_back();
                preempt(victim);
                preempted = true;
                if (victim == s) {
                    gave_up = true;
                    break;
                }
            }
            if (gave_up) continue;
            bm_.append(*s);
            take(s, want, &budget, &out);
            kept.push_back(s);
        }
        running_ = std::move(kept);
        // new requests are admitted whatever is in flight (admission only takes free blocks)
        while (!preempted && !waiting_.empty() && budget > 0 &&
               static_cast<int64_t>(running_.size()) < cfg_.max_num_seqs) {
            Seq* s = waiting_.front();
            if (!bm_.can_allocate(*s)) break;
            waiting_.pop_front();
            bm_.allocate(*s);
            s->state = State::kRunning;
            running_.push_back(s);
            take(s, std::min({s->uncached(), budget, cap}), &budget, &out);
        }
        return out;
    }
    void take(Seq* s, int64_t n, int64_t* budget, std::vector<Seq*>* out) {
        s->num_sched = n;
        *budget -= n;
        out->push_back(s);
    }
    void preempt(Seq* s) {
        bm_.release(*s);
        s->state = State::kWaiting;
        s->num_sched = 0;
        waiting_.push_front(s);
        ++stats_.preemptions;
    }
    int group_of(const Seq& s) const {
        if (s.num_sched == 1 && s.num_cached > 0 && ceil_div(s.num_cached + 1, cfg_.block_size) <= cfg_.graph_max_blocks)
            return CVE_GROUP_DECODE;
        if (s.num_cached == 0 && s.num_sched > 1) return CVE_GROUP_FRESH;
        return CVE_GROUP_CONT;
    }
    // Flat batch of the step, ordered by group, then the launch bookkeeping of
    // scheduler.cpp:105-119 (cached count advances, a sampling row reserves its token slot).
    void build(const std::vector<Seq*>& picked, cve_batch* out) {
        flights_.emplace_back();
        Flight& f = flights_.back();
        std::vector<Seq*>& rows = f.seqs;
        int64_t gs[CVE_NUM_GROUPS + 1] = {0, 0, 0, 0};
        for (int g = 0; g < CVE_NUM_GROUPS; ++g) {
            gs[g] = static_cast<int64_t>(rows.size());
            for (Seq* s : picked)
                if (group_of(*s) == g) rows.push_back(s);
        }
        gs[CVE_NUM_GROUPS] = static_cast<int64_t>(rows.size());
        const int64_t S = gs[CVE_NUM_GROUPS];
        int64_t T = 0, W = 1;
        for (Seq* s : rows) {
            T += s->num_sched;
            W = std::max(W, ceil_div(s->num_cached + s->num_sched, cfg_.block_size));
        }
        tokens_.assign(T, 0);
        feed_.assign(T, -1);
        positions_.assign(T, 0);
        cu_.assign(S + 1, 0);
        kv_.assign(S, 0);
        tables_.assign(S * W, -1);
        shared_.assign(S, 0);
        samples_.assign(S, 0);
        ids_.assign(S, 0);
        int64_t t = 0;
        for (int64_t j = 0; j < S; ++j) {
            Seq* s = rows[j];
            const int64_t c = s->num_cached, q = s->num_sched, kv = c + q;
            for (int64_t k = 0; k < q; ++k, ++t) {
                tokens_[t] = s->tokens[c + k];
                positions_[t] = c + k;
                // a placeholder is being sampled by the previous (still running) step: the runner
                // copies it on the device from that step's sampled row
                if (tokens_[t] == kPending) feed_[t] = s->last_row;
            }
            cu_[j + 1] = t;
            kv_[j] = kv;
            for (int64_t b = 0; b < ceil_div(kv, cfg_.block_size); ++b) tables_[j * W + b] = s->table[b];
            // leading blocks another live sequence also references (prefix-cache hits)
            int32_t sh = 0;
            while (sh < static_cast<int32_t>(s->table.size()) && bm_.ref_count(s->table[sh]) > 1) ++sh;
            shared_[j] = sh;
            ids_[j] = s->id;
            const bool samples = kv == s->size();
            samples_[j] = samples ? 1 : 0;
            s->num_cached = kv;
            s->num_sched = 0;
            ++s->inflight;
            f.at.push_back(samples ? s->size() : -1);
            s->last_row = samples ? j : -1;
            if (samples) s->tokens.push_back(kPending);
            stats_.tokens_scheduled += q;
        }
        out->num_seqs = S;
        out->num_tokens = T;
        out->table_width = W;
        std::memcpy(out->group_start, gs, sizeof(gs));
        out->tokens = tokens_.data();
        out->positions = positions_.data();
        out->cu_seqlens = cu_.data();
        out->kv_lens = kv_.data();
        out->block_tables = tables_.data();
        out->samples = samples_.data();
        out->seq_ids = ids_.data();
        out->feed_src = feed_.data();
        out->shared_blocks = shared_.data();
    }
    void finish(Seq* s) {
        Output o;
        o.id = s->id;
        o.tokens.assign(s->tokens.begin() + s->num_prompt, s->tokens.end());
        done_.emplace(o.id, std::move(o));
        ++stats_.finished;
    }

    cve_config cfg_;
    BlockManager bm_;
    std::deque<Seq*> waiting_;
    std::vector<Seq*> running_;
    std::unordered_map<int64_t, std::unique_ptr<Seq>> live_;
    std::map<int64_t, Output> done_;
    struct Flight {
        std::vector<Seq*> seqs;          // rows of the step
        std::vector<int64_t> at;         // token index each row samples, -1 = none
    };
    static constexpr size_t kMaxFlights = 2;   // llm_engine.h:51 (kDepth)
    std::deque<Flight> flights_;
    int64_t next_id_ = 0;
    cve_stats stats_{};
    std::vector<int64_t> tokens_, feed_, positions_, cu_, kv_, tables_, ids_;
    std::vector<int8_t> samples_;
    std::vector<int32_t> shared_;
};

Engine* E(void* p) { return static_cast<Engine*>(p); }

}  // namespace
}  // namespace cve

extern "C" {

void* cve_create(const cve_config* c) {
    if (!c || c->block_size <= 0 || c->num_blocks <= 0 || c->max_num_batched_tokens <= 0 || c->max_num_seqs <= 0 ||
        c->max_chunk_tokens < 0)
        return nullptr;
    return new cve::Engine(*c);
}
void cve_destroy(void* e) { delete cve::E(e); }

int64_t cve_add_request(void* e, const int32_t* prompt, int64_t n, int32_t max_tokens, int32_t ignore_eos) {
    if (!e) return CVE_ERR_INVALID_ARG;
    return cve::E(e)->add(prompt, n, max_tokens, ignore_eos != 0);
}
int cve_schedule(void* e, cve_batch* out) {
    if (!e || !out) return CVE_ERR_INVALID_ARG;
    return cve::E(e)->schedule(out);
}
int cve_postprocess(void* e, const int64_t* sampled, int64_t n) {
    if (!e) return CVE_ERR_INVALID_ARG;
    return cve::E(e)->postprocess(sampled, n);
}
int cve_is_finished(void* e) { return e && cve::E(e)->finished() ? 1 : 0; }
int64_t cve_num_outstanding(void* e) { return e ? cve::E(e)->inflight() : 0; }
int cve_get_stats(void* e, cve_stats* out) {
    if (!e || !out) return CVE_ERR_INVALID_ARG;
    *out = cve::E(e)->stats();
    return CVE_OK;
}
int64_t cve_num_finished(void* e) { return e ? static_cast<int64_t>(cve::E(e)->outputs().size()) : 0; }
int64_t cve_finished_output(void* e, int64_t i, int64_t* request_id, int32_t* tokens, int64_t cap) {
    if (!e || i < 0) return -1;
    const auto& m = cve::E(e)->outputs();
    if (i >= static_cast<int64_t>(m.size())) return -1;
    auto it = m.begin();
    std::advance(it, i);
    if (request_id) *request_id = it->first;
    const int64_t n = static_cast<int64_t>(it->second.tokens.size());
    if (tokens) std::copy(it->second.tokens.begin(), it->second.tokens.begin() + std::min(n, cap), tokens);
    return n;
}
void cve_clear_finished(void* e) {
    if (e) cve::E(e)->clear_outputs();
}
int32_t cve_block_ref_count(void* e, int32_t id) {
    if (!e || id < 0 || id >= cve::E(e)->blocks().num_blocks()) return -1;
    return cve::E(e)->blocks().ref_count(id);
}
int64_t cve_block_table(void* e, int64_t request_id, int32_t* out, int64_t cap) {
    if (!e) return -1;
    const auto* s = cve::E(e)->find(request_id);
    if (!s) return -1;
    const int64_t n = static_cast<int64_t>(s->table.size());
    if (out) std::copy(s->table.begin(), s->table.begin() + std::min(n, cap), out);
    return n;
}

}  // extern "C"
