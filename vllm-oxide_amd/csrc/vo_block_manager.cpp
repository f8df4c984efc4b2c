// vo_block_manager.cpp -- KV block manager with refcounted blocks and a
// full-block prefix cache (host side, behind the C ABI).
//
// The reference plans this component (the owner's M2 block manager and M4
// prefix cache; README.md:14, CLAUDE.md:26, docs/process.md:43-47) and fixes
// its invariant (CLAUDE.md:71): every block is either free or referenced by
// >= 1 block table, its refcount equals the number of references, and nothing
// is freed while a running sequence uses it.  The M0 driver's counter
// (generate.rs:4-7) is what it replaces.
//
// Model:
//  - The pool's blocks are 0 .. num_blocks-1.  Each is in exactly one state:
//    free (on the free list), cached-idle (refcount 0 but holding a hashed
//    full block, on an LRU list, reusable or evictable), or in use
//    (refcount >= 1).
//  - A sequence owns a block table and its token ids.  Token t lives at
//    slot table[t / bs] * bs + t % bs (paged.rs:47-52).
//  - Appending at a block boundary takes a new block (free list first, then
//    the least recently used cached-idle block).  Appending into a block that
//    a fork shares (refcount > 1) copies it first: the manager hands the
//    caller the (source, destination) pair to copy on the device.
//  - Prefix caching works on full blocks.  Block i of a sequence hashes
//    (hash of block i-1, its bs token ids) with FNV-1a 64, which only finds
//    the candidate: a hit is accepted when the cached block's token ids
//    equal the prompt's block AND the block was registered right after the
//    block the lookup accepted for position i-1 (its id, and its generation,
//    which changes whenever a block is given new contents).  By induction an
//    accepted run's whole prefix equals the prompt's, so a hash collision
//    (FNV is not collision-resistant) can only cost a miss, never reuse KV
//    computed under another prefix.  A prompt reuses its longest run of
//    cached leading blocks, but never the block holding its last token,
//    which the step must compute to produce logits.
//  - Freeing a sequence drops one reference per table entry; a block reaching
//    refcount 0 goes to the LRU list if it is a hashed full block, else to
//    the free list.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <list>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "vo_paged.hpp"

using namespace vo;

namespace {

constexpr uint32_t kNone = 0xffffffffu;
constexpr uint64_t kFnvOffset = 0xcbf29ce484222325ull;
constexpr uint64_t kFnvPrime = 0x100000001b3ull;

uint64_t fnv1a(uint64_t h, const void *data, size_t bytes) {
    const unsigned char *p = static_cast<const unsigned char *>(data);
    for (size_t i = 0; i < bytes; ++i) {
        h ^= p[i];
        h *= kFnvPrime;
    }
    return h;
}

struct Block {
    uint32_t refcount = 0;
    bool hashed = false;       // a full block registered in the prefix cache
    uint64_t hash = 0;
    uint64_t gen = 0;          // bumped whenever the block takes new contents
    uint32_t parent = kNone;   // while hashed: the block before it (kNone at position 0)
    uint64_t parent_gen = 0;   // and that block's generation then
    std::vector<uint32_t> tokens;  // its bs token ids while hashed
    std::list<uint32_t>::iterator lru_it;
    bool on_lru = false;
    bool on_free = false;
};

struct Seq {
    std::vector<uint32_t> table;
    std::vector<uint32_t> tokens;
    std::vector<uint64_t> hashes;  // chained hash of each full block
    // The verified chain: for each full block i, the cached block that
    // stands for it in the prefix cache -- the sequence's own block once
    // registered, or an equal block the cache already held for this prefix
    // -- with that block's generation then; kNone where there is none (the
    // hash is held by a block that is not this prefix's, or the chain broke
    // earlier).  A later block is registered with chain[i - 1] as its parent.
    std::vector<uint32_t> chain;
    std::vector<uint64_t> chain_gen;
};

}  // namespace

struct vo_block_manager {
    uint64_t num_blocks = 0, block_size = 0;
    bool prefix_caching = false;
    // Test hook (vo_bm_test_unchained_hash): hash a block's own tokens only,
    // so that equal blocks after different prefixes collide on purpose.
    bool unchained_hash = false;
    std::vector<Block> blocks;
    std::vector<uint32_t> free_list;       // LIFO
    std::list<uint32_t> lru;               // cached-idle blocks, least recently used first
    std::unordered_map<uint64_t, uint32_t> cache;  // hash -> block
    std::unordered_map<uint64_t, Seq> seqs;
    vo_bm_stats stats{};

    uint64_t available() const { return free_list.size() + lru.size(); }

    void unregister(uint32_t b) {
        Block &k = blocks[b];
        if (!k.hashed) return;
        auto it = cache.find(k.hash);
        if (it != cache.end() && it->second == b) cache.erase(it);
        k.hashed = false;
        k.tokens.clear();
    }

    // Takes a block for new contents: the free list first, then the least
    // recently used cached-idle block (evicted from the cache).
    uint32_t take() {
        uint32_t b;
        if (!free_list.empty()) {
            b = free_list.back();
            free_list.pop_back();
            blocks[b].on_free = false;
        } else if (!lru.empty()) {
            b = lru.front();
            lru.pop_front();
            blocks[b].on_lru = false;
            unregister(b);
            ++stats.evictions;
        } else {
            return kNone;
        }
        blocks[b].refcount = 1;
        ++blocks[b].gen;
        return b;
    }

    // One more reference to a cached block (a prefix-cache hit).
    void ref(uint32_t b) {
        Block &k = blocks[b];
        if (k.on_lru) {
            lru.erase(k.lru_it);
            k.on_lru = false;
        }
        ++k.refcount;
    }

    void unref(uint32_t b) {
        Block &k = blocks[b];
        if (--k.refcount > 0) return;
        if (k.hashed) {
            lru.push_back(b);
            k.lru_it = std::prev(lru.end());
            k.on_lru = true;
        } else {
            free_list.push_back(b);
            k.on_free = true;
        }
    }

    uint64_t block_hash(uint64_t prev, const uint32_t *toks) const {
        if (unchained_hash) prev = 0;
        return fnv1a(fnv1a(kFnvOffset, &prev, sizeof(prev)), toks, block_size * sizeof(uint32_t));
    }

    // Whether cached block b may stand at a position whose predecessor in
    // the verified chain is `parent` (kNone at position 0, taken at
    // generation parent_gen) and whose tokens are toks.
    bool accepts(uint32_t b, uint32_t parent, uint64_t parent_gen, const uint32_t *toks) const {
        const Block &k = blocks[b];
        if (!std::equal(k.tokens.begin(), k.tokens.end(), toks)) return false;
        if (parent == kNone) return k.parent == kNone;
        return k.parent == parent && k.parent_gen == parent_gen && blocks[parent].gen == parent_gen;
    }

    // Full block i of `s` (blocks 0 .. i-1 done): its chained hash, its link
    // in the verified chain, and -- when the cache holds nothing under its
    // hash and its predecessor is verified -- its registration, with that
    // predecessor as parent.  An equal block already cached for this prefix
    // stands for it instead; a hash held by a block of another prefix (a
    // collision, or the cache's first writer for another chain) leaves the
    // chain broken from here on, so no entry is made that no lookup could
    // accept.
    void register_full(Seq &s, uint64_t i) {
        const uint64_t prev = i ? s.hashes[i - 1] : 0;
        const uint32_t *toks = s.tokens.data() + i * block_size;
        const uint64_t h = block_hash(prev, toks);
        if (s.hashes.size() <= i) s.hashes.resize(i + 1);
        s.hashes[i] = h;
        if (s.chain.size() <= i) {
            s.chain.resize(i + 1, kNone);
            s.chain_gen.resize(i + 1, 0);
        }
        s.chain[i] = kNone;
        if (!prefix_caching) return;
        const uint32_t parent = i ? s.chain[i - 1] : kNone;
        const uint64_t parent_gen = i ? s.chain_gen[i - 1] : 0;
        if (i && (parent == kNone || blocks[parent].gen != parent_gen)) return;
        auto it = cache.find(h);
        if (it != cache.end()) {
            if (accepts(it->second, parent, parent_gen, toks)) {
                s.chain[i] = it->second;
                s.chain_gen[i] = blocks[it->second].gen;
            }
            return;
        }
        const uint32_t b = s.table[i];
        if (blocks[b].hashed) return;  // registered under another hash
        blocks[b].hashed = true;
        blocks[b].hash = h;
        blocks[b].parent = parent;
        blocks[b].parent_gen = parent_gen;
        blocks[b].tokens.assign(toks, toks + block_size);
        cache.emplace(h, b);
        s.chain[i] = b;
        s.chain_gen[i] = blocks[b].gen;
    }
};

namespace {

vo_status fail_seq(const char *op, uint64_t seq, const char *what) {
    return fail_argument(op, "sequence " + std::to_string(seq) + " " + what);
}

vo_status fail_exhausted(const char *op, uint64_t need, uint64_t have) {
    // The reference treats an empty pool as a scheduling policy case
    // (preemption, docs/grill-log.md:86-88); the manager reports it and
    // changes nothing.
    return fail_capacity(op, need, have);
}

}  // namespace

extern "C" int32_t vo_bm_create(uint64_t num_blocks, uint64_t block_size, int32_t prefix_caching,
                                vo_block_manager **out) {
    const char *op = "block_manager_create";
    if (!out) return fail_argument(op, "null output");
    *out = nullptr;
    if (num_blocks == 0 || block_size == 0) return fail_shape(op, "num_blocks and block_size must be non-zero");
    if (num_blocks >= kNone) return fail_capacity("blocks (u32 ids)", num_blocks, kNone - 1);
    vo_block_manager *bm = new (std::nothrow) vo_block_manager();
    if (!bm) return fail_argument(op, "out of host memory");
    bm->num_blocks = num_blocks;
    bm->block_size = block_size;
    bm->prefix_caching = prefix_caching != 0;
    bm->blocks.resize(num_blocks);
    bm->free_list.reserve(num_blocks);
    // Hand out low block ids first.
    for (uint64_t b = num_blocks; b-- > 0;) {
        bm->free_list.push_back(static_cast<uint32_t>(b));
        bm->blocks[b].on_free = true;
    }
    *out = bm;
    clear_error();
    return VO_OK;
}

extern "C" void vo_bm_destroy(vo_block_manager *bm) { delete bm; }

extern "C" int32_t vo_bm_test_unchained_hash(vo_block_manager *bm, int32_t on) {
    const char *op = "block_manager_test_unchained_hash";
    if (!bm) return fail_argument(op, "null manager");
    if (!bm->seqs.empty() || !bm->cache.empty())
        return fail_argument(op, "only before the first sequence");
    bm->unchained_hash = on != 0;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_bm_add_sequence(vo_block_manager *bm, uint64_t seq_id,
                                      const uint32_t *tokens, uint64_t num_tokens,
                                      uint64_t *cached_tokens) {
    const char *op = "add_sequence";
    if (!bm || (num_tokens && !tokens)) return fail_argument(op, "null manager or tokens");
    if (bm->seqs.count(seq_id)) return fail_seq(op, seq_id, "already exists");
    const uint64_t bs = bm->block_size;
    const uint64_t nblk = (num_tokens + bs - 1) / bs;
    // Longest run of cached leading full blocks, never the block holding the
    // last token.
    std::vector<uint32_t> hits;
    std::vector<uint64_t> hit_hashes;
    if (bm->prefix_caching) {
        uint64_t prev = 0;
        // Full blocks that do not hold the last token: (i + 1) * bs < n.
        for (uint64_t i = 0; (i + 1) * bs < num_tokens; ++i) {
            const uint64_t h = bm->block_hash(prev, tokens + i * bs);
            auto it = bm->cache.find(h);
            const uint32_t parent = hits.empty() ? kNone : hits.back();
            const uint64_t parent_gen = hits.empty() ? 0 : bm->blocks[parent].gen;
            if (it == bm->cache.end() || !bm->accepts(it->second, parent, parent_gen, tokens + i * bs))
                break;
            hits.push_back(it->second);
            hit_hashes.push_back(h);
            prev = h;
        }
    }
    const uint64_t fresh = nblk - hits.size();
    // Blocks on the LRU that are hits must not count as available for the
    // fresh ones.
    uint64_t hit_idle = 0;
    for (uint32_t b : hits) hit_idle += bm->blocks[b].on_lru ? 1 : 0;
    if (fresh > bm->available() - hit_idle) return fail_exhausted("kv blocks", fresh, bm->available() - hit_idle);
    Seq s;
    s.tokens.assign(tokens, tokens + num_tokens);
    for (uint32_t b : hits) {
        bm->ref(b);
        s.table.push_back(b);
    }
    s.hashes = hit_hashes;
    s.chain = hits;
    for (uint32_t b : hits) s.chain_gen.push_back(bm->blocks[b].gen);
    for (uint64_t i = 0; i < fresh; ++i) s.table.push_back(bm->take());
    for (uint64_t i = hits.size(); (i + 1) * bs <= num_tokens; ++i) bm->register_full(s, i);
    bm->stats.hit_blocks += hits.size();
    bm->stats.lookup_blocks += (num_tokens ? (num_tokens - 1) / bs : 0);
    if (cached_tokens) *cached_tokens = hits.size() * bs;
    bm->seqs.emplace(seq_id, std::move(s));
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_bm_append_token(vo_block_manager *bm, uint64_t seq_id, uint32_t token,
                                      uint32_t *slot, uint32_t *copy_src, uint32_t *copy_dst) {
    const char *op = "append_token";
    if (!bm) return fail_argument(op, "null manager");
    auto it = bm->seqs.find(seq_id);
    if (it == bm->seqs.end()) return fail_seq(op, seq_id, "does not exist");
    Seq &s = it->second;
    const uint64_t bs = bm->block_size;
    const uint64_t pos = s.tokens.size();
    uint32_t src = kNone, dst = kNone;
    if (pos % bs == 0) {
        // Append on a block boundary (docs/grill-log.md:86-88).
        if (bm->available() == 0) return fail_exhausted("kv blocks", 1, 0);
        s.table.push_back(bm->take());
    } else {
        const uint32_t last = s.table[pos / bs];
        if (bm->blocks[last].refcount > 1) {
            // Copy on write: the block is shared with a fork.
            if (bm->available() == 0) return fail_exhausted("kv blocks", 1, 0);
            const uint32_t b = bm->take();
            bm->unref(last);
            s.table[pos / bs] = b;
            src = last;
            dst = b;
            ++bm->stats.copies;
        }
    }
    s.tokens.push_back(token);
    if ((pos + 1) % bs == 0) bm->register_full(s, pos / bs);
    if (slot) *slot = s.table[pos / bs] * static_cast<uint32_t>(bs) + static_cast<uint32_t>(pos % bs);
    if (copy_src) *copy_src = src;
    if (copy_dst) *copy_dst = dst;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_bm_fork(vo_block_manager *bm, uint64_t parent, uint64_t child) {
    const char *op = "fork";
    if (!bm) return fail_argument(op, "null manager");
    auto it = bm->seqs.find(parent);
    if (it == bm->seqs.end()) return fail_seq(op, parent, "does not exist");
    if (bm->seqs.count(child)) return fail_seq(op, child, "already exists");
    Seq c = it->second;
    for (uint32_t b : c.table) bm->ref(b);
    bm->seqs.emplace(child, std::move(c));
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_bm_free_sequence(vo_block_manager *bm, uint64_t seq_id) {
    const char *op = "free_sequence";
    if (!bm) return fail_argument(op, "null manager");
    auto it = bm->seqs.find(seq_id);
    if (it == bm->seqs.end()) return fail_seq(op, seq_id, "does not exist");
    // Later blocks first, so a prefix's leading blocks stay cached longest.
    for (auto b = it->second.table.rbegin(); b != it->second.table.rend(); ++b) bm->unref(*b);
    bm->seqs.erase(it);
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_bm_block_table(const vo_block_manager *bm, uint64_t seq_id, uint32_t *out,
                                     uint64_t capacity, uint64_t *len, uint64_t *num_tokens) {
    const char *op = "block_table";
    if (!bm) return fail_argument(op, "null manager");
    auto it = bm->seqs.find(seq_id);
    if (it == bm->seqs.end()) return fail_seq(op, seq_id, "does not exist");
    const auto &t = it->second.table;
    if (len) *len = t.size();
    if (num_tokens) *num_tokens = it->second.tokens.size();
    if (out) {
        if (capacity < t.size()) return fail_capacity("block table entries", t.size(), capacity);
        std::copy(t.begin(), t.end(), out);
    }
    clear_error();
    return VO_OK;
}

extern "C" uint64_t vo_bm_num_available(const vo_block_manager *bm) {
    return bm ? bm->available() : 0;
}

extern "C" int32_t vo_bm_get_stats(const vo_block_manager *bm, vo_bm_stats *out) {
    if (!bm || !out) return fail_argument("bm_stats", "null manager or output");
    *out = bm->stats;
    out->free_blocks = bm->free_list.size();
    out->cached_idle_blocks = bm->lru.size();
    out->sequences = bm->seqs.size();
    clear_error();
    return VO_OK;
}

// CLAUDE.md:71 plus the manager's own bookkeeping, checked exhaustively.
extern "C" int32_t vo_bm_check_invariants(const vo_block_manager *bm) {
    const char *op = "bm_invariants";
    if (!bm) return fail_argument(op, "null manager");
    const uint64_t N = bm->num_blocks, bs = bm->block_size;
    std::vector<uint64_t> refs(N, 0);
    for (const auto &kv : bm->seqs) {
        const Seq &s = kv.second;
        const uint64_t need = (s.tokens.size() + bs - 1) / bs;
        if (s.table.size() != need)
            return fail_shape(op, "sequence " + std::to_string(kv.first) + " has " +
                                      std::to_string(s.table.size()) + " blocks for " +
                                      std::to_string(s.tokens.size()) + " tokens");
        for (uint32_t b : s.table) {
            if (b >= N) return fail_shape(op, "block id " + std::to_string(b) + " out of range");
            ++refs[b];
        }
    }
    std::vector<int> on_free(N, 0), on_lru(N, 0);
    for (uint32_t b : bm->free_list) on_free[b]++;
    for (uint32_t b : bm->lru) on_lru[b]++;
    for (uint64_t b = 0; b < N; ++b) {
        const Block &k = bm->blocks[b];
        const std::string id = "block " + std::to_string(b);
        if (k.refcount != refs[b])
            return fail_shape(op, id + ": refcount " + std::to_string(k.refcount) + " but " +
                                      std::to_string(refs[b]) + " table references");
        const int states = (refs[b] > 0) + on_free[b] + on_lru[b];
        if (states != 1) return fail_shape(op, id + " is in " + std::to_string(states) + " states");
        if (on_free[b] != k.on_free || on_lru[b] != k.on_lru) return fail_shape(op, id + ": stale list flags");
        if (on_free[b] && k.hashed) return fail_shape(op, id + " is free but still cached");
        if (on_lru[b] && !k.hashed) return fail_shape(op, id + " is idle but not cached");
        if (k.hashed) {
            auto it = bm->cache.find(k.hash);
            if (it == bm->cache.end() || it->second != b) return fail_shape(op, id + " hash not indexed");
            if (k.tokens.size() != bs) return fail_shape(op, id + " cached without its tokens");
        }
    }
    for (const auto &kv : bm->cache)
        if (kv.second >= N || !bm->blocks[kv.second].hashed || bm->blocks[kv.second].hash != kv.first)
            return fail_shape(op, "cache entry points at an unhashed block");
    clear_error();
    return VO_OK;
}
