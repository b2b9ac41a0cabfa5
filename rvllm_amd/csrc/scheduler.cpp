// scheduler.cpp - host-side continuous-batching scheduler over the paged KV
// pool: refcounted block pool, per-sequence block tables, a prefix cache
// of full blocks, FIFO admission queue and recompute preemption.
//
// It restates the contract rvllm's engine uses from the kv-cache-scheduler
// crate (0.2.0, not vendored; src/engine.rs:351-539):
//   waiting (FIFO) / running lists, sequences with token_ids and a block
//   table (blocks(), num_tokens(), logical_to_physical(i)), pool.available()
//   and total_allocs, prefix_cache.match_prefix(tokens) -> matched blocks,
//   prefill(seq) (allocate the prompt's blocks, reusing matched ones),
//   step() (every running sequence gets one more slot, preempting from the
//   back of running when the pool is empty), finish_sequence(seq), and the
//   prefix_hits / prefix_total metrics.
// The crate's own allocation order and eviction policy are not available,
// so the choices here are stated instead:
//   * free blocks are reused last-freed-first;
//   * a block whose every token is final is entered in the prefix cache
//     under the hash of (previous block's hash, its tokens); when its last
//     user releases it, it stays matchable on an LRU list and counts as
//     available; allocation takes a never-cached free block first, then
//     evicts the least recently released cached one;
//   * preemption evicts the most recently admitted running sequence
//     (recompute: its full blocks stay cached, it goes back to the front of
//     waiting);
//   * the block holding a sequence's last prompt token is never matched, so
//     at least that token runs through the model and nothing writes into a
//     shared block (the engine's skip is min(matched * bs, n - 1));
//   * a shared (refcount > 1) last block that is about to be written gets a
//     private copy first (copy-on-write); the (src, dst) pairs are handed to
//     the caller for rvkv_copy_blocks.
#include <cstdint>
#include <cstring>
#include <deque>
#include <list>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/rvkv.h"

namespace {

thread_local std::string g_sched_err;

int sfail(int code, const char *what) {
  g_sched_err = what;
  return code;
}

uint64_t mix(uint64_t h, uint64_t x) {  // FNV-1a over 8 bytes, then a finaliser
  for (int i = 0; i < 8; ++i) {
    h ^= (x >> (8 * i)) & 0xffu;
    h *= 0x100000001b3ull;
  }
  return h;
}

uint64_t block_hash(uint64_t parent, const int32_t *toks, uint32_t n) {
  uint64_t h = mix(0xcbf29ce484222325ull, parent);
  for (uint32_t i = 0; i < n; ++i) h = mix(h, (uint32_t)toks[i]);
  h ^= h >> 33;
  h *= 0xff51afd7ed558ccdull;
  h ^= h >> 33;
  return h;
}

struct Block {
  uint32_t ref = 0;
  bool cached = false;
  uint64_t hash = 0, parent = 0;
  std::vector<int32_t> toks;  // content, kept while cached (exact match)
  std::list<uint32_t>::iterator lru_it;
  bool in_lru = false;
};

struct Seq {
  std::vector<int32_t> tokens;
  std::vector<uint32_t> blocks;
  uint32_t num_tokens = 0;  // tokens that have a slot
  uint32_t committed = 0;   // tokens whose content and K/V are final
  uint32_t registered = 0;  // leading blocks already entered in the cache
};

}  // namespace

struct rvkv_sched {
  uint32_t nb, bs;
  std::vector<Block> blk;
  std::vector<uint32_t> free_list;  // never-cached (or evicted) free blocks
  std::list<uint32_t> lru;          // cached blocks with refcount 0
  std::unordered_map<uint64_t, uint32_t> cache;
  std::unordered_map<int64_t, Seq> seqs;
  std::deque<int64_t> waiting;
  std::vector<int64_t> running;
  int64_t next_id = 0;
  uint64_t total_allocs = 0, prefix_hits = 0, prefix_total = 0;
  uint64_t preemptions = 0;
  std::vector<std::pair<uint32_t, uint32_t>> cow;

  uint32_t available() const {
    return (uint32_t)(free_list.size() + lru.size());
  }

  bool alloc(uint32_t *out) {
    uint32_t b;
    if (!free_list.empty()) {
      b = free_list.back();
      free_list.pop_back();
    } else if (!lru.empty()) {
      b = lru.front();
      lru.pop_front();
      Block &x = blk[b];
      x.in_lru = false;
      auto it = cache.find(x.hash);
      if (it != cache.end() && it->second == b) cache.erase(it);
      x.cached = false;
      x.toks.clear();
    } else {
      return false;
    }
    blk[b].ref = 1;
    ++total_allocs;
    *out = b;
    return true;
  }

  void acquire(uint32_t b) {
    Block &x = blk[b];
    if (x.in_lru) {
      lru.erase(x.lru_it);
      x.in_lru = false;
    }
    ++x.ref;
  }

  void release(uint32_t b) {
    Block &x = blk[b];
    if (x.ref == 0) return;
    if (--x.ref > 0) return;
    if (x.cached) {
      lru.push_back(b);
      x.lru_it = std::prev(lru.end());
      x.in_lru = true;
    } else {
      free_list.push_back(b);
    }
  }

  // Enters the sequence's full, committed blocks in the prefix cache.
  void register_blocks(Seq &s) {
    while (s.registered < s.blocks.size() &&
           (uint64_t)(s.registered + 1) * bs <= s.committed) {
      const uint32_t i = s.registered;
      const uint64_t parent = i ? blk[s.blocks[i - 1]].hash : 0;
      const int32_t *t = s.tokens.data() + (size_t)i * bs;
      Block &x = blk[s.blocks[i]];
      if (!x.cached) {
        const uint64_t h = block_hash(parent, t, bs);
        x.hash = h;
        x.parent = parent;
        if (!cache.count(h)) {
          cache[h] = s.blocks[i];
          x.cached = true;
          x.toks.assign(t, t + bs);
        }
      }
      ++s.registered;
    }
  }

  // Longest run of leading full blocks of `toks` found in the cache, at
  // most `max_blocks`.
  void match(const int32_t *toks, uint32_t n, uint32_t max_blocks,
             std::vector<uint32_t> *out) const {
    uint64_t parent = 0;
    for (uint32_t i = 0; i < max_blocks && (uint64_t)(i + 1) * bs <= n; ++i) {
      const int32_t *t = toks + (size_t)i * bs;
      const uint64_t h = block_hash(parent, t, bs);
      auto it = cache.find(h);
      if (it == cache.end()) break;
      const Block &x = blk[it->second];
      if (x.parent != parent || x.toks.size() != bs ||
          memcmp(x.toks.data(), t, (size_t)bs * 4) != 0)
        break;
      out->push_back(it->second);
      parent = h;
    }
  }

  static uint32_t matchable(uint32_t n, uint32_t bs) {
    return n ? (n - 1) / bs : 0;  // never the block of the last token
  }

  void preempt(int64_t id) {
    Seq &s = seqs[id];
    register_blocks(s);
    for (uint32_t b : s.blocks) release(b);
    s.blocks.clear();
    s.num_tokens = s.committed = s.registered = 0;
    for (size_t i = 0; i < running.size(); ++i)
      if (running[i] == id) {
        running.erase(running.begin() + (long)i);
        break;
      }
    waiting.push_front(id);
    ++preemptions;
  }
};

extern "C" {

const char *rvkv_sched_last_error(void) { return g_sched_err.c_str(); }

rvkv_sched *rvkv_sched_create(uint32_t num_blocks, uint32_t block_size) {
  if (num_blocks == 0 || block_size == 0) {
    sfail(RVKV_EINVAL, "sched: num_blocks and block_size must be positive");
    return nullptr;
  }
  auto *s = new rvkv_sched();
  s->nb = num_blocks;
  s->bs = block_size;
  s->blk.resize(num_blocks);
  s->free_list.reserve(num_blocks);
  for (uint32_t i = num_blocks; i-- > 0;) s->free_list.push_back(i);
  return s;
}

void rvkv_sched_destroy(rvkv_sched *s) { delete s; }

int64_t rvkv_sched_add_request(rvkv_sched *s, const int32_t *tokens,
                               uint32_t n) {
  if (!s || (!tokens && n)) return sfail(RVKV_EINVAL, "sched: bad arguments");
  const int64_t id = s->next_id++;
  Seq &q = s->seqs[id];
  q.tokens.assign(tokens, tokens + n);
  s->waiting.push_back(id);
  return id;
}

uint32_t rvkv_sched_available(const rvkv_sched *s) { return s->available(); }
uint64_t rvkv_sched_total_allocs(const rvkv_sched *s) {
  return s->total_allocs;
}
void rvkv_sched_metrics(const rvkv_sched *s, uint64_t *prefix_hits,
                        uint64_t *prefix_total, uint64_t *preemptions) {
  if (prefix_hits) *prefix_hits = s->prefix_hits;
  if (prefix_total) *prefix_total = s->prefix_total;
  if (preemptions) *preemptions = s->preemptions;
}

uint32_t rvkv_sched_num_waiting(const rvkv_sched *s) {
  return (uint32_t)s->waiting.size();
}
uint32_t rvkv_sched_num_running(const rvkv_sched *s) {
  return (uint32_t)s->running.size();
}
uint32_t rvkv_sched_waiting(const rvkv_sched *s, int64_t *out, uint32_t cap) {
  uint32_t n = 0;
  for (int64_t id : s->waiting) {
    if (n < cap) out[n] = id;
    ++n;
  }
  return n;
}
uint32_t rvkv_sched_running(const rvkv_sched *s, int64_t *out, uint32_t cap) {
  uint32_t n = 0;
  for (int64_t id : s->running) {
    if (n < cap) out[n] = id;
    ++n;
  }
  return n;
}

int rvkv_sched_has_seq(const rvkv_sched *s, int64_t id) {
  return s->seqs.count(id) ? 1 : 0;
}

uint32_t rvkv_sched_match_prefix(const rvkv_sched *s, const int32_t *tokens,
                                 uint32_t n, uint32_t *blocks, uint32_t cap) {
  std::vector<uint32_t> m;
  s->match(tokens, n, rvkv_sched::matchable(n, s->bs), &m);
  for (uint32_t i = 0; i < m.size() && i < cap; ++i) blocks[i] = m[i];
  return (uint32_t)m.size();
}

int rvkv_sched_prefill(rvkv_sched *s, int64_t id, uint32_t *matched_blocks) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return sfail(RVKV_EINVAL, "sched: unknown sequence");
  Seq &q = it->second;
  if (!q.blocks.empty())
    return sfail(RVKV_EINVAL, "sched: sequence already has blocks");
  const uint32_t n = (uint32_t)q.tokens.size();
  if (n == 0) return sfail(RVKV_EINVAL, "sched: empty sequence");
  const uint32_t need = (n + s->bs - 1) / s->bs;
  std::vector<uint32_t> m;
  s->match(q.tokens.data(), n, rvkv_sched::matchable(n, s->bs), &m);
  // All-or-nothing: count what a fresh allocation needs before touching
  // anything (matched blocks on the LRU list leave it, so they count too).
  uint32_t from_lru = 0;
  for (uint32_t b : m) from_lru += s->blk[b].in_lru ? 1u : 0u;
  if ((uint64_t)(need - m.size()) + from_lru > s->available())
    return sfail(RVKV_ENOMEM, "sched: not enough free blocks for the prompt");
  for (uint32_t b : m) s->acquire(b);
  q.blocks = m;
  while (q.blocks.size() < need) {
    uint32_t b;
    s->alloc(&b);
    q.blocks.push_back(b);
  }
  q.num_tokens = n;
  q.committed = n;
  q.registered = (uint32_t)m.size();
  s->prefix_hits += m.size();
  s->prefix_total += rvkv_sched::matchable(n, s->bs);
  s->register_blocks(q);
  for (size_t i = 0; i < s->waiting.size(); ++i)
    if (s->waiting[i] == id) {
      s->waiting.erase(s->waiting.begin() + (long)i);
      break;
    }
  s->running.push_back(id);
  if (matched_blocks) *matched_blocks = (uint32_t)m.size();
  return RVKV_OK;
}

int rvkv_sched_step(rvkv_sched *s, uint32_t *n_preempted) {
  uint32_t pre = 0;
  for (int64_t id : s->running) {  // every earlier token is final now
    Seq &q = s->seqs[id];
    q.committed = q.num_tokens;
    s->register_blocks(q);
  }
  size_t i = 0;
  while (i < s->running.size()) {
    const int64_t id = s->running[i];
    Seq &q = s->seqs[id];
    const uint32_t pos = q.num_tokens;
    bool gone = false;
    const bool new_block = pos == (uint32_t)q.blocks.size() * s->bs;
    const bool shared =
        !new_block && !q.blocks.empty() && s->blk[q.blocks.back()].ref > 1;
    if (new_block || shared) {
      uint32_t b;
      while (!s->alloc(&b)) {
        const int64_t victim = s->running.back();
        s->preempt(victim);
        ++pre;
        if (victim == id) {
          gone = true;
          break;
        }
      }
      if (gone) continue;  // running[i] is now the next sequence
      if (shared) {
        const uint32_t old = q.blocks.back();
        s->cow.emplace_back(old, b);
        s->release(old);
        q.blocks.back() = b;
        if (q.registered == q.blocks.size()) --q.registered;
      } else {
        q.blocks.push_back(b);
      }
    }
    q.tokens.push_back(0);  // placeholder; the engine writes the real token
    ++q.num_tokens;
    ++i;
  }
  if (n_preempted) *n_preempted = pre;
  return RVKV_OK;
}

uint32_t rvkv_sched_take_cow(rvkv_sched *s, uint32_t *src, uint32_t *dst,
                             uint32_t cap) {
  const uint32_t n = (uint32_t)s->cow.size();
  if (n > cap) return n;  // caller retries with room for all
  for (uint32_t i = 0; i < n; ++i) {
    src[i] = s->cow[i].first;
    dst[i] = s->cow[i].second;
  }
  s->cow.clear();
  return n;
}

int rvkv_sched_finish(rvkv_sched *s, int64_t id) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return sfail(RVKV_EINVAL, "sched: unknown sequence");
  Seq &q = it->second;
  q.committed = q.num_tokens;
  s->register_blocks(q);
  for (uint32_t b : q.blocks) s->release(b);
  q.blocks.clear();
  q.num_tokens = q.committed = q.registered = 0;
  for (size_t i = 0; i < s->running.size(); ++i)
    if (s->running[i] == id) {
      s->running.erase(s->running.begin() + (long)i);
      break;
    }
  for (size_t i = 0; i < s->waiting.size(); ++i)
    if (s->waiting[i] == id) {
      s->waiting.erase(s->waiting.begin() + (long)i);
      break;
    }
  return RVKV_OK;
}

int rvkv_sched_remove(rvkv_sched *s, int64_t id) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return RVKV_OK;
  rvkv_sched_finish(s, id);  // releases blocks, leaves waiting/running
  s->seqs.erase(id);
  return RVKV_OK;
}

int64_t rvkv_sched_fork(rvkv_sched *s, int64_t parent) {
  auto it = s->seqs.find(parent);
  if (it == s->seqs.end()) return sfail(RVKV_EINVAL, "sched: unknown sequence");
  const Seq src = it->second;
  const int64_t id = s->next_id++;
  Seq &q = s->seqs[id];
  q = src;
  for (uint32_t b : q.blocks) s->acquire(b);
  bool was_running = false;
  for (int64_t r : s->running) was_running |= r == parent;
  if (was_running)
    s->running.push_back(id);
  else
    s->waiting.push_back(id);
  return id;
}

uint32_t rvkv_sched_num_tokens(const rvkv_sched *s, int64_t id) {
  auto it = s->seqs.find(id);
  return it == s->seqs.end() ? 0u : it->second.num_tokens;
}

uint32_t rvkv_sched_num_blocks(const rvkv_sched *s, int64_t id) {
  auto it = s->seqs.find(id);
  return it == s->seqs.end() ? 0u : (uint32_t)it->second.blocks.size();
}

uint32_t rvkv_sched_table(const rvkv_sched *s, int64_t id, uint32_t *out,
                          uint32_t cap) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return 0;
  const auto &b = it->second.blocks;
  for (uint32_t i = 0; i < b.size() && i < cap; ++i) out[i] = b[i];
  return (uint32_t)b.size();
}

int rvkv_sched_slot(const rvkv_sched *s, int64_t id, uint32_t pos,
                    uint32_t *block, uint32_t *offset) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return sfail(RVKV_EINVAL, "sched: unknown sequence");
  const Seq &q = it->second;
  if (pos >= q.blocks.size() * (uint64_t)s->bs)
    return sfail(RVKV_EINVAL, "sched: position past the block table");
  *block = q.blocks[pos / s->bs];
  *offset = pos % s->bs;
  return RVKV_OK;
}

uint32_t rvkv_sched_tokens(const rvkv_sched *s, int64_t id, int32_t *out,
                           uint32_t cap) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return 0;
  const auto &t = it->second.tokens;
  for (uint32_t i = 0; i < t.size() && i < cap; ++i) out[i] = t[i];
  return (uint32_t)t.size();
}

int rvkv_sched_set_tokens(rvkv_sched *s, int64_t id, const int32_t *tokens,
                          uint32_t n) {
  auto it = s->seqs.find(id);
  if (it == s->seqs.end()) return sfail(RVKV_EINVAL, "sched: unknown sequence");
  Seq &q = it->second;
  if (n < q.committed)
    return sfail(RVKV_EINVAL, "sched: cannot drop tokens that hold K/V");
  for (uint32_t i = 0; i < q.committed; ++i)
    if (q.tokens[i] != tokens[i])
      return sfail(RVKV_EINVAL, "sched: cannot rewrite tokens that hold K/V");
  q.tokens.assign(tokens, tokens + n);
  return RVKV_OK;
}

uint32_t rvkv_sched_refcount(const rvkv_sched *s, uint32_t block) {
  return block < s->nb ? s->blk[block].ref : 0u;
}

}  // extern "C"
