// engine.hip — the continuous-batching engine: block pool, block tables, prefix
// cache, sequences and the Sarathi step planner, driving the device model.
//
// Reference (restated in C++, same decisions in the same order):
//   BlockPool              src/kv_cache/block_pool.rs:1-68
//   BlockTable             src/kv_cache/block_table.rs:1-63
//   PrefixCache            src/kv_cache/prefix_cache.rs:1-116
//   allocate_zeroed        src/kv_cache/mod.rs:25-35
//   Sequence               src/scheduler/sequence.rs:1-74
//   Engine::step           src/engine.rs:213-505
//   drain_finished / cancel_request   src/engine.rs:511-531
//   decode_needs_block / ensure_blocks / preempt_lowest_priority_after / preempt
//                          src/engine.rs:534-601
//
// Host code only. One step builds a compact plan (kanso_seq_plan per planned
// sequence, this step's tokens and every planned sequence's block table) and hands
// it to model_forward, which packs it on the device (kanso_pack_step) and returns
// the greedy token of every sequence's last row. Blocks allocated while planning
// are erased in one kernel before the forward, which is when allocate_zeroed's
// erase must have happened by.
#include <algorithm>
#include <cstring>
#include <unordered_map>

#include "model.hpp"

namespace kanso {
namespace {

enum SeqStatus { kWaiting = 0, kRunning = 1, kPreempted = 2, kFinished = 3 };

class BlockPool {
   public:
    explicit BlockPool(uint32_t total) : ref_(total, 0), total_(total) {
        free_.reserve(total);
        for (uint32_t b = total; b-- > 0;) free_.push_back(b);
    }
    size_t free_count() const { return free_.size(); }
    bool allocate(uint32_t* out) {
        if (free_.empty()) return false;
        *out = free_.back();
        free_.pop_back();
        ref_[*out] = 1;
        return true;
    }
    bool claim(uint32_t b) {
        if (b >= total_) return false;
        if (ref_[b] > 0) {
            ++ref_[b];
            return true;
        }
        auto it = std::find(free_.begin(), free_.end(), b);
        if (it == free_.end()) return false;
        free_.erase(it);
        ref_[b] = 1;
        return true;
    }
    void free(uint32_t b) {
        if (b < total_ && ref_[b] > 0 && --ref_[b] == 0) free_.push_back(b);
    }

   private:
    std::vector<uint32_t> free_;
    std::vector<uint32_t> ref_;
    uint32_t total_;
};

using TokenKey = std::vector<uint32_t>;
struct KeyHash {
    size_t operator()(const TokenKey& k) const {
        uint64_t h = 0xcbf29ce484222325ull;
        for (uint32_t t : k) h = (h ^ t) * 0x100000001b3ull;
        return static_cast<size_t>(h);
    }
};

class PrefixCache {
   public:
    explicit PrefixCache(uint32_t bs, size_t max_entries = 64) : bs_(bs), max_(std::max<size_t>(max_entries, 1)) {}

    void insert(const std::vector<uint32_t>& tokens, const std::vector<uint32_t>& blocks) {
        const size_t n = tokens.size() / bs_;
        for (size_t b = 1; b <= n; ++b) {
            TokenKey key(tokens.begin(), tokens.begin() + b * bs_);
            std::vector<uint32_t> bp(blocks.begin(), blocks.begin() + b);
            ++tick_;
            auto it = cached_.find(key);
            if (it != cached_.end()) {
                std::vector<uint32_t> old = it->second;
                it->second = bp;
                for (uint32_t blk : old)
                    if (std::find(bp.begin(), bp.end(), blk) == bp.end()) detach(key, blk);
            } else {
                cached_.emplace(key, bp);
            }
            for (uint32_t blk : bp) {
                auto& keys = block_to_keys_[blk];
                if (std::find(keys.begin(), keys.end(), key) == keys.end()) keys.push_back(key);
            }
            last_used_[key] = tick_;
        }
        while (cached_.size() > max_) {
            if (last_used_.empty()) break;
            auto oldest = last_used_.begin();
            for (auto it = last_used_.begin(); it != last_used_.end(); ++it)
                if (it->second < oldest->second) oldest = it;
            TokenKey k = oldest->first;
            remove_entry(k);
        }
    }

    void invalidate_block(uint32_t block) {
        auto it = block_to_keys_.find(block);
        if (it == block_to_keys_.end()) return;
        std::vector<TokenKey> keys = std::move(it->second);
        block_to_keys_.erase(it);
        for (const auto& k : keys) remove_entry(k);
    }

    size_t find_longest(const std::vector<uint32_t>& tokens, std::vector<uint32_t>* blocks) {
        const size_t n = tokens.size() / bs_;
        for (size_t b = n; b >= 1; --b) {
            TokenKey key(tokens.begin(), tokens.begin() + b * bs_);
            auto it = cached_.find(key);
            if (it != cached_.end()) {
                ++tick_;
                last_used_[key] = tick_;
                *blocks = it->second;
                return b * bs_;
            }
        }
        blocks->clear();
        return 0;
    }

   private:
    void remove_entry(const TokenKey& key) {
        auto it = cached_.find(key);
        if (it != cached_.end()) {
            std::vector<uint32_t> blocks = std::move(it->second);
            cached_.erase(it);
            for (uint32_t blk : blocks) detach(key, blk);
        }
        last_used_.erase(key);
    }
    void detach(const TokenKey& key, uint32_t block) {
        auto it = block_to_keys_.find(block);
        if (it == block_to_keys_.end()) return;
        auto& keys = it->second;
        keys.erase(std::remove(keys.begin(), keys.end(), key), keys.end());
        if (keys.empty()) block_to_keys_.erase(it);
    }

    uint32_t bs_;
    size_t max_;
    uint64_t tick_ = 0;
    std::unordered_map<TokenKey, std::vector<uint32_t>, KeyHash> cached_;
    std::unordered_map<uint32_t, std::vector<TokenKey>> block_to_keys_;
    std::unordered_map<TokenKey, uint64_t, KeyHash> last_used_;
};

struct Sequence {
    uint64_t id = 0;
    std::vector<uint32_t> prompt, generated, stop_ids;
    std::vector<uint32_t> blocks;  // BlockTable::blocks
    size_t num_tokens = 0;         // BlockTable::num_tokens
    int status = kWaiting;
    size_t prefilled = 0;
    size_t max_tokens = 0;
    bool finished() const { return status == kFinished; }
    bool done_after(uint32_t tok) const {
        return generated.size() >= max_tokens || std::find(stop_ids.begin(), stop_ids.end(), tok) != stop_ids.end();
    }
};

struct Planned {
    size_t idx;
    size_t start_pos;
    std::vector<uint32_t> tokens;
    bool is_prefill;
};

}  // namespace
}  // namespace kanso

struct kanso_engine {
    kanso_model* model = nullptr;
    uint32_t dry_vocab = 0;
    kanso::BlockPool pool;
    kanso::PrefixCache prefix;
    std::vector<kanso::Sequence> seqs;
    size_t max_running, block_size, token_budget;
    uint64_t current_step = 0, next_id = 1;
    uint64_t prefix_matched = 0, prompt_admitted = 0, prefix_hits = 0, prefix_lookups = 0;
    std::vector<uint32_t> pending_reset;  // blocks allocated while planning this step
    // The last step's flattened batch (engine.rs:376-402) for inspection.
    std::vector<uint32_t> lp_tokens, lp_positions, lp_ctx, lp_qlen, lp_table_lens, lp_tables, lp_sample_rows;
    std::vector<uint64_t> lp_slots;
    kanso_engine(uint32_t total, uint32_t bs) : pool(total), prefix(bs) {}
};

namespace kanso {
namespace {

size_t running_count(const kanso_engine* e) {
    size_t n = 0;
    for (const auto& s : e->seqs) n += s.status == kRunning;
    return n;
}

uint32_t dry_token(uint64_t id, uint32_t pos, uint32_t vocab) {
    const uint64_t h = (id * 2654435761ull + static_cast<uint64_t>(pos) * 40503ull + 12345ull) & 0xffffffffull;
    return static_cast<uint32_t>(h % vocab);
}

void preempt(kanso_engine* e, size_t idx) {
    Sequence& s = e->seqs[idx];
    for (uint32_t b : s.blocks) e->pool.free(b);
    const size_t emitted = s.generated.size();
    s.prompt.insert(s.prompt.end(), s.generated.begin(), s.generated.end());
    s.generated.clear();
    s.max_tokens = s.max_tokens > emitted ? s.max_tokens - emitted : 0;
    s.blocks.clear();
    s.num_tokens = 0;
    s.prefilled = 0;
    s.status = kWaiting;
}

bool preempt_lowest_priority_after(kanso_engine* e, size_t idx, const std::vector<bool>& planned) {
    for (size_t j = e->seqs.size(); j-- > idx + 1;) {
        const Sequence& s = e->seqs[j];
        if (!planned[j] && s.status == kRunning && !s.finished()) {
            preempt(e, j);
            return true;
        }
    }
    return false;
}

bool ensure_blocks(kanso_engine* e, size_t idx, size_t want, const std::vector<bool>& planned) {
    while (e->pool.free_count() < want)
        if (!preempt_lowest_priority_after(e, idx, planned)) return false;
    for (size_t i = 0; i < want; ++i) {
        uint32_t blk;
        if (!e->pool.allocate(&blk)) return false;
        e->pending_reset.push_back(blk);  // allocate_zeroed's erase, batched per step
        e->prefix.invalidate_block(blk);
        e->seqs[idx].blocks.push_back(blk);
    }
    return true;
}

bool decode_needs_block(const kanso_engine* e, size_t idx) {
    const Sequence& s = e->seqs[idx];
    return s.num_tokens + 1 > s.blocks.size() * e->block_size;
}

int engine_step(kanso_engine* e, std::vector<kanso_step_output>* outputs) {
    ++e->current_step;
    size_t budget = e->token_budget;
    std::vector<Planned> planned;
    std::vector<bool> flags(e->seqs.size(), false);
    e->pending_reset.clear();

    // 1. decode rows (engine.rs:228-266)
    for (size_t idx = 0; idx < e->seqs.size(); ++idx) {
        const Sequence& s = e->seqs[idx];
        if (s.status != kRunning || s.finished() || s.prefilled < s.prompt.size()) continue;
        if (budget == 0) break;
        if (decode_needs_block(e, idx) && !ensure_blocks(e, idx, 1, flags)) continue;
        const Sequence& s2 = e->seqs[idx];
        const size_t pos = s2.prompt.size() + s2.generated.size() - 1;
        planned.push_back({idx, pos, {s2.generated.back()}, false});
        flags[idx] = true;
        budget -= 1;
    }

    // 2. admission with the prefix-cache lookup (engine.rs:268-319)
    const size_t running = running_count(e);
    const size_t available = e->max_running > running ? e->max_running - running : 0;
    size_t admitted = 0;
    for (auto& s : e->seqs) {
        if (s.status == kWaiting && admitted < available && (e->pool.free_count() > 0 || s.prefilled > 0)) {
            if (s.prefilled == 0 && s.generated.empty()) {
                ++e->prefix_lookups;
                e->prompt_admitted += s.prompt.size();
                std::vector<uint32_t> matched_blocks;
                const size_t matched = e->prefix.find_longest(s.prompt, &matched_blocks);
                if (matched > 0) {
                    std::vector<uint32_t> claimed;
                    bool all = true;
                    for (uint32_t b : matched_blocks) {
                        if (e->pool.claim(b)) {
                            claimed.push_back(b);
                        } else {
                            all = false;
                            break;
                        }
                    }
                    if (all) {
                        s.blocks.insert(s.blocks.end(), matched_blocks.begin(), matched_blocks.end());
                        const size_t eff = matched == s.prompt.size() ? matched - 1 : matched;
                        s.num_tokens = eff;
                        s.prefilled = eff;
                        ++e->prefix_hits;
                        e->prefix_matched += matched;
                    } else {
                        for (uint32_t b : claimed) e->pool.free(b);
                    }
                }
            }
            s.status = kRunning;
            ++admitted;
        }
    }

    // 3. prefill chunks with the remaining budget (engine.rs:321-364)
    for (size_t idx = 0; idx < e->seqs.size(); ++idx) {
        const Sequence& s = e->seqs[idx];
        if (s.status != kRunning || s.finished() || s.prefilled >= s.prompt.size()) continue;
        if (budget == 0) continue;
        const size_t needed = s.prompt.size() - s.prefilled;
        const size_t chunk = std::min(needed, budget);
        if (chunk == 0) continue;
        const size_t start = s.prefilled, end = start + chunk;
        const size_t need_blocks = (end + (end == s.prompt.size() ? 1 : 0) + e->block_size - 1) / e->block_size;
        const size_t cur = s.blocks.size();
        if (need_blocks > cur && !ensure_blocks(e, idx, need_blocks - cur, flags)) continue;
        const Sequence& s2 = e->seqs[idx];
        planned.push_back({idx, start, std::vector<uint32_t>(s2.prompt.begin() + start, s2.prompt.begin() + end), true});
        flags[idx] = true;
        budget -= chunk;
    }

    // 4. the batched forward (engine.rs:371-412)
    e->lp_tokens.clear();
    e->lp_positions.clear();
    e->lp_slots.clear();
    e->lp_ctx.clear();
    e->lp_qlen.clear();
    e->lp_table_lens.clear();
    e->lp_tables.clear();
    e->lp_sample_rows.clear();
    std::vector<uint32_t> next;
    if (!planned.empty()) {
        HostStep hs;
        for (size_t row = 0; row < planned.size(); ++row) {
            const Planned& p = planned[row];
            const Sequence& s = e->seqs[p.idx];
            for (size_t i = 0; i < p.tokens.size(); ++i) {
                const size_t pos = p.start_pos + i;
                const size_t bi = pos / e->block_size;
                if (bi >= s.blocks.size()) {
                    set_error("Position %zu requires block index %zu but block table only has %zu blocks", pos, bi,
                              s.blocks.size());
                    return KANSO_E_OUT_OF_BOUNDS;
                }
                e->lp_tokens.push_back(p.tokens[i]);
                e->lp_positions.push_back(static_cast<uint32_t>(pos));
                e->lp_slots.push_back(static_cast<uint64_t>(s.blocks[bi]) * e->block_size + pos % e->block_size);
            }
            e->lp_ctx.push_back(static_cast<uint32_t>(p.start_pos + p.tokens.size()));
            e->lp_qlen.push_back(static_cast<uint32_t>(p.tokens.size()));
            e->lp_table_lens.push_back(static_cast<uint32_t>(s.blocks.size()));
            kanso_seq_plan sp;
            sp.start_pos = static_cast<uint32_t>(p.start_pos);
            sp.q_len = static_cast<uint32_t>(p.tokens.size());
            sp.table_offset = static_cast<uint32_t>(hs.table_arena.size());
            sp.table_len = static_cast<uint32_t>(s.blocks.size());
            // token_offset + pos indexes this step's tokens (modulo 2^32)
            sp.token_offset = static_cast<uint32_t>(hs.token_arena.size()) - sp.start_pos;
            hs.plan.push_back(sp);
            hs.token_arena.insert(hs.token_arena.end(), p.tokens.begin(), p.tokens.end());
            hs.table_arena.insert(hs.table_arena.end(), s.blocks.begin(), s.blocks.end());
            if (!p.is_prefill || p.start_pos + p.tokens.size() == s.prompt.size())
                e->lp_sample_rows.push_back(static_cast<uint32_t>(row));
        }
        e->lp_tables = hs.table_arena;
        next.resize(planned.size());
        if (e->model) {
            hipStream_t st = nullptr;
            int rc = model_reset_blocks(e->model, e->pending_reset.data(),
                                        static_cast<uint32_t>(e->pending_reset.size()), st);
            if (rc) return rc;
            if ((rc = model_forward(e->model, hs, nullptr, next.data(), st))) return rc;
        } else {
            for (size_t row = 0; row < planned.size(); ++row)
                next[row] = dry_token(e->seqs[planned[row].idx].id, e->lp_ctx[row], e->dry_vocab);
        }
    }

    // 5. commit in plan order (engine.rs:414-487)
    std::vector<size_t> finished;
    for (size_t row = 0; row < planned.size(); ++row) {
        const Planned& p = planned[row];
        Sequence& s = e->seqs[p.idx];
        if (p.is_prefill) {
            const size_t end = p.start_pos + p.tokens.size();
            s.prefilled = end;
            s.num_tokens = end;
            if (end != s.prompt.size()) continue;
        }
        const uint32_t tok = next[row];
        s.generated.push_back(tok);
        s.num_tokens += 1;
        const bool done = s.done_after(tok);
        if (done) {
            s.status = kFinished;
            finished.push_back(p.idx);
        }
        outputs->push_back({s.id, tok, done ? 1u : 0u});
    }
    for (const Planned& p : planned) {
        const Sequence& s = e->seqs[p.idx];
        if (p.is_prefill && s.prefilled == s.prompt.size()) e->prefix.insert(s.prompt, s.blocks);
    }
    // 6. retirement (engine.rs:496-502)
    for (size_t idx : finished)
        for (uint32_t b : e->seqs[idx].blocks) e->pool.free(b);
    return KANSO_OK;
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" {

uint32_t kanso_engine_dry_token(uint64_t request_id, uint32_t position, uint32_t vocab) {
    return vocab ? dry_token(request_id, position, vocab) : 0u;
}

int kanso_engine_create(kanso_model* model, uint32_t max_running, uint32_t total_blocks, uint32_t block_size,
                        uint32_t token_budget, uint32_t dry_vocab, kanso_engine** out) {
    if (!out) {
        set_error("kanso_engine_create: null out");
        return KANSO_E_INVALID_ARG;
    }
    *out = nullptr;
    if (total_blocks == 0 || block_size == 0 || token_budget == 0 || max_running == 0) {
        set_error("kanso_engine_create: total_blocks %u, block_size %u, token_budget %u, max_running %u must be "
                  "non-zero",
                  total_blocks, block_size, token_budget, max_running);
        return KANSO_E_INVALID_SHAPE;
    }
    if (!model && dry_vocab == 0) {
        set_error("kanso_engine_create: a model-less engine needs dry_vocab > 0");
        return KANSO_E_INVALID_ARG;
    }
    if (model) {
        if (!model->k_pool) {
            int rc = kanso_model_alloc_kv(model, total_blocks, block_size, token_budget, max_running + 1);
            if (rc) return rc;
        } else if (model->num_blocks != total_blocks || model->block_size != block_size) {
            set_error("kanso_engine_create: the model's KV pool (%u blocks of %u) differs from %u blocks of %u",
                      model->num_blocks, model->block_size, total_blocks, block_size);
            return KANSO_E_INVALID_SHAPE;
        }
    }
    auto* e = new kanso_engine(total_blocks, block_size);
    e->model = model;
    e->dry_vocab = dry_vocab;
    e->max_running = max_running;
    e->block_size = block_size;
    e->token_budget = token_budget;
    *out = e;
    return KANSO_OK;
}

int kanso_engine_destroy(kanso_engine* e) {
    delete e;
    return KANSO_OK;
}

int kanso_engine_add_request(kanso_engine* e, const uint32_t* prompt, uint32_t prompt_len, uint32_t max_tokens,
                             const uint32_t* stop_ids, uint32_t num_stop, uint64_t* request_id) {
    if (!e || (prompt_len && !prompt) || (num_stop && !stop_ids)) {
        set_error("kanso_engine_add_request: null argument");
        return KANSO_E_INVALID_ARG;
    }
    // An empty prompt has no row to sample from (the reference's server rejects it
    // before the engine, src/server/routes.rs:109).
    if (prompt_len == 0) {
        set_error("kanso_engine_add_request: empty prompt");
        return KANSO_E_INVALID_ARG;
    }
    // Token ids index the embedding table: ids past the vocabulary are refused here
    // rather than read as row 0 on the device.
    const uint32_t vocab = e->model ? kanso_model_vocab(e->model) : 0;
    for (uint32_t i = 0; vocab && i < prompt_len; ++i)
        if (prompt[i] >= vocab) {
            set_error("kanso_engine_add_request: token %u at %u outside the vocabulary (%u)", prompt[i], i, vocab);
            return KANSO_E_INVALID_ARG;
        }
    Sequence s;
    s.id = e->next_id++;
    s.prompt.assign(prompt, prompt + prompt_len);
    s.stop_ids.assign(stop_ids, stop_ids + num_stop);
    s.max_tokens = max_tokens;
    e->seqs.push_back(std::move(s));
    if (request_id) *request_id = e->seqs.back().id;
    return KANSO_OK;
}

int kanso_engine_step(kanso_engine* e, kanso_step_output* outputs, uint32_t capacity, uint32_t* num_outputs) {
    if (!e || !num_outputs || (capacity && !outputs)) {
        set_error("kanso_engine_step: null argument");
        return KANSO_E_INVALID_ARG;
    }
    std::vector<kanso_step_output> outs;
    int rc = engine_step(e, &outs);
    if (rc) return rc;
    *num_outputs = static_cast<uint32_t>(outs.size());
    if (outs.size() > capacity) {
        set_error("kanso_engine_step: %zu outputs exceed capacity %u", outs.size(), capacity);
        return KANSO_E_OUT_OF_BOUNDS;
    }
    std::memcpy(outputs, outs.data(), outs.size() * sizeof(kanso_step_output));
    return KANSO_OK;
}

int kanso_engine_last_plan(kanso_engine* e, uint32_t* sizes, uint32_t* tokens, uint32_t* positions, uint64_t* slots,
                           uint32_t* context_lens, uint32_t* query_lens, uint32_t* table_lens, uint32_t* tables,
                           uint32_t* sample_rows) {
    if (!e || !sizes) {
        set_error("kanso_engine_last_plan: null argument");
        return KANSO_E_INVALID_ARG;
    }
    sizes[0] = static_cast<uint32_t>(e->lp_tokens.size());
    sizes[1] = static_cast<uint32_t>(e->lp_ctx.size());
    sizes[2] = static_cast<uint32_t>(e->lp_tables.size());
    sizes[3] = static_cast<uint32_t>(e->lp_sample_rows.size());
    auto put = [](auto* dst, const auto& src) {
        if (dst) std::copy(src.begin(), src.end(), dst);
    };
    put(tokens, e->lp_tokens);
    put(positions, e->lp_positions);
    put(slots, e->lp_slots);
    put(context_lens, e->lp_ctx);
    put(query_lens, e->lp_qlen);
    put(table_lens, e->lp_table_lens);
    put(tables, e->lp_tables);
    put(sample_rows, e->lp_sample_rows);
    return KANSO_OK;
}

int kanso_engine_stats(kanso_engine* e, uint64_t* st) {
    if (!e || !st) {
        set_error("kanso_engine_stats: null argument");
        return KANSO_E_INVALID_ARG;
    }
    uint64_t waiting = 0, running = 0, unfinished = 0;
    for (const auto& s : e->seqs) {
        waiting += s.status == kWaiting;
        running += s.status == kRunning;
        unfinished += !s.finished();
    }
    st[0] = waiting;
    st[1] = running;
    st[2] = e->pool.free_count();
    st[3] = unfinished;
    st[4] = e->seqs.size();
    st[5] = e->prefix_hits;
    st[6] = e->prefix_lookups;
    st[7] = e->prefix_matched;
    st[8] = e->prompt_admitted;
    st[9] = e->current_step;
    return KANSO_OK;
}

int kanso_engine_cancel(kanso_engine* e, uint64_t request_id, uint32_t* found) {
    if (!e) {
        set_error("kanso_engine_cancel: null engine");
        return KANSO_E_INVALID_ARG;
    }
    uint32_t hit = 0;
    for (auto& s : e->seqs) {
        if (s.id == request_id) {
            for (uint32_t b : s.blocks) e->pool.free(b);
            s.status = kFinished;
            hit = 1;
            break;
        }
    }
    if (hit) e->seqs.erase(std::remove_if(e->seqs.begin(), e->seqs.end(), [](const Sequence& s) { return s.finished(); }),
                           e->seqs.end());
    if (found) *found = hit;
    return KANSO_OK;
}

int kanso_engine_drain_finished(kanso_engine* e, uint32_t* dropped) {
    if (!e) {
        set_error("kanso_engine_drain_finished: null engine");
        return KANSO_E_INVALID_ARG;
    }
    const size_t before = e->seqs.size();
    e->seqs.erase(std::remove_if(e->seqs.begin(), e->seqs.end(), [](const Sequence& s) { return s.finished(); }),
                  e->seqs.end());
    if (dropped) *dropped = static_cast<uint32_t>(before - e->seqs.size());
    return KANSO_OK;
}

}  // extern "C"
