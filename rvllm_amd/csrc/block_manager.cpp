// block_manager.cpp - host-side block pool, block tables, slot mapping and
// refcounted prefix sharing with copy-on-write, behind rvkv_bm_* in
// include/rvkv.h.
//
// It stands in for the external kv-cache-scheduler 0.2.0 crate as rvllm's
// engine uses it (src/engine.rs:351-539): BlockPool::available(),
// BlockTable::{blocks, num_tokens, logical_to_physical}, blocks shared by
// the prefix cache. The crate's source is not available, so only the
// behaviour the engine relies on is restated:
//   * slot of position i = (table[i / block_size], i % block_size)
//     (logical_to_physical, src/engine.rs:375-377, 446-451);
//   * a sequence holding n tokens owns ceil(n / block_size) blocks;
//   * freeing a sequence returns every block it alone held, so
//     available() returns to its starting value after a drain
//     (src/engine.rs:834, 851, 903);
//   * a shared block is never written in place (src/conv_cache.rs:11-14):
//     appending into one first moves the sequence onto a private copy.
// Single-threaded, like the engine thread that drives it.
#include <cstdint>
#include <unordered_map>
#include <vector>

#include "../../include/rvkv.h"

namespace {

struct Seq {
  std::vector<uint32_t> table;
  uint32_t num_tokens = 0;
};

uint64_t splitmix64(uint64_t &s) {
  uint64_t z = (s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

}  // namespace

struct rvkv_bm {
  uint32_t num_blocks, block_size;
  std::vector<uint32_t> free_list;  // pop_back() hands out the next block
  std::vector<uint32_t> refcount;
  std::unordered_map<int64_t, Seq> seqs;
  int64_t next_id = 0;

  bool take(uint32_t *blk) {
    if (free_list.empty()) return false;
    *blk = free_list.back();
    free_list.pop_back();
    refcount[*blk] = 1;
    return true;
  }
  void drop(uint32_t blk) {
    if (--refcount[blk] == 0) free_list.push_back(blk);
  }
  uint32_t blocks_for(uint32_t n_tokens) const {
    return (uint32_t)(((uint64_t)n_tokens + block_size - 1) / block_size);
  }
};

extern "C" {

rvkv_bm *rvkv_bm_create(uint32_t num_blocks, uint32_t block_size) {
  if (num_blocks == 0 || block_size == 0) return nullptr;
  rvkv_bm *bm = new rvkv_bm();
  bm->num_blocks = num_blocks;
  bm->block_size = block_size;
  bm->refcount.assign(num_blocks, 0);
  bm->free_list.reserve(num_blocks);
  for (uint32_t i = num_blocks; i-- > 0;) bm->free_list.push_back(i);
  return bm;
}

void rvkv_bm_destroy(rvkv_bm *bm) { delete bm; }

uint32_t rvkv_bm_available(const rvkv_bm *bm) {
  return bm ? (uint32_t)bm->free_list.size() : 0;
}

void rvkv_bm_shuffle_free(rvkv_bm *bm, uint64_t seed) {
  if (!bm) return;
  auto &f = bm->free_list;
  uint64_t s = seed;
  for (size_t i = f.size(); i > 1; --i) {
    size_t j = (size_t)(splitmix64(s) % i);
    std::swap(f[i - 1], f[j]);
  }
}

int64_t rvkv_bm_add_seq(rvkv_bm *bm, uint32_t n_tokens) {
  if (!bm) return RVKV_EINVAL;
  const uint32_t need = bm->blocks_for(n_tokens);
  if (need > bm->free_list.size()) return RVKV_ENOMEM;
  Seq s;
  s.table.resize(need);
  for (uint32_t i = 0; i < need; ++i) bm->take(&s.table[i]);
  s.num_tokens = n_tokens;
  const int64_t id = bm->next_id++;
  bm->seqs.emplace(id, std::move(s));
  return id;
}

int64_t rvkv_bm_fork_seq(rvkv_bm *bm, int64_t parent, uint32_t n_shared,
                         uint32_t n_tokens) {
  if (!bm) return RVKV_EINVAL;
  auto it = bm->seqs.find(parent);
  if (it == bm->seqs.end()) return RVKV_EINVAL;
  if (n_shared > it->second.num_tokens || n_shared > n_tokens)
    return RVKV_EINVAL;
  // Tokens past the shared prefix need private blocks; a prefix ending
  // inside a block would put them into the shared one.
  if (n_tokens > n_shared && n_shared % bm->block_size != 0)
    return RVKV_EINVAL;
  const uint32_t shared = bm->blocks_for(n_shared);
  const uint32_t total = bm->blocks_for(n_tokens);
  if (total - shared > bm->free_list.size()) return RVKV_ENOMEM;
  Seq s;
  s.table.assign(it->second.table.begin(), it->second.table.begin() + shared);
  for (uint32_t b : s.table) ++bm->refcount[b];
  for (uint32_t i = shared; i < total; ++i) {
    uint32_t blk;
    bm->take(&blk);
    s.table.push_back(blk);
  }
  s.num_tokens = n_tokens;
  const int64_t id = bm->next_id++;
  bm->seqs.emplace(id, std::move(s));
  return id;
}

int rvkv_bm_free_seq(rvkv_bm *bm, int64_t seq) {
  if (!bm) return RVKV_EINVAL;
  auto it = bm->seqs.find(seq);
  if (it == bm->seqs.end()) return RVKV_EINVAL;
  for (uint32_t b : it->second.table) bm->drop(b);
  bm->seqs.erase(it);
  return RVKV_OK;
}

int rvkv_bm_append_slot(rvkv_bm *bm, int64_t seq, uint32_t *block,
                        uint32_t *offset, uint32_t *cow_src,
                        uint32_t *cow_dst) {
  if (!bm || !block || !offset || !cow_src || !cow_dst) return RVKV_EINVAL;
  auto it = bm->seqs.find(seq);
  if (it == bm->seqs.end()) return RVKV_EINVAL;
  Seq &s = it->second;
  *cow_src = *cow_dst = UINT32_MAX;
  const uint32_t pos = s.num_tokens;
  const uint32_t bi = pos / bm->block_size;
  if (bi >= s.table.size()) {  // block boundary: a fresh block
    uint32_t blk;
    if (!bm->take(&blk)) return RVKV_ENOMEM;
    s.table.push_back(blk);
  } else if (bm->refcount[s.table[bi]] > 1) {  // shared: copy on write
    uint32_t blk;
    if (!bm->take(&blk)) return RVKV_ENOMEM;
    *cow_src = s.table[bi];
    *cow_dst = blk;
    bm->drop(s.table[bi]);
    s.table[bi] = blk;
  }
  *block = s.table[bi];
  *offset = pos % bm->block_size;
  s.num_tokens = pos + 1;
  return RVKV_OK;
}

int rvkv_bm_free_seqs(rvkv_bm *bm, const int64_t *seqs, uint32_t n) {
  if (!bm || (n && !seqs)) return RVKV_EINVAL;
  for (uint32_t i = 0; i < n; ++i) {
    const int rc = rvkv_bm_free_seq(bm, seqs[i]);
    if (rc != RVKV_OK) return rc;
  }
  return RVKV_OK;
}

int rvkv_bm_add_seqs(rvkv_bm *bm, const uint32_t *n_tokens, uint32_t n,
                     int64_t *ids) {
  if (!bm || (n && (!n_tokens || !ids))) return RVKV_EINVAL;
  uint64_t need = 0;
  for (uint32_t i = 0; i < n; ++i) need += bm->blocks_for(n_tokens[i]);
  if (need > bm->free_list.size()) return RVKV_ENOMEM;  // all or nothing
  for (uint32_t i = 0; i < n; ++i) ids[i] = rvkv_bm_add_seq(bm, n_tokens[i]);
  return RVKV_OK;
}

int rvkv_bm_append_slots(rvkv_bm *bm, const int64_t *seqs, uint32_t n,
                         uint32_t *blocks, uint32_t *offsets,
                         uint32_t *cow_src, uint32_t *cow_dst,
                         uint32_t *n_cow) {
  if (!bm || (n && (!seqs || !blocks || !offsets || !cow_src || !cow_dst)) ||
      !n_cow)
    return RVKV_EINVAL;
  uint32_t k = 0;
  for (uint32_t i = 0; i < n; ++i) {
    uint32_t cs, cd;
    const int rc =
        rvkv_bm_append_slot(bm, seqs[i], &blocks[i], &offsets[i], &cs, &cd);
    if (rc != RVKV_OK) {
      *n_cow = k;
      return rc;
    }
    if (cs != UINT32_MAX) {
      cow_src[k] = cs;
      cow_dst[k] = cd;
      ++k;
    }
  }
  *n_cow = k;
  return RVKV_OK;
}

int rvkv_bm_fill_tables(const rvkv_bm *bm, const int64_t *seqs, uint32_t n,
                        uint32_t max_blocks, uint32_t *tables,
                        uint32_t *ctx_lens) {
  if (!bm || (n && (!seqs || !tables || !ctx_lens))) return RVKV_EINVAL;
  for (uint32_t i = 0; i < n; ++i) {
    auto it = bm->seqs.find(seqs[i]);
    if (it == bm->seqs.end()) return RVKV_EINVAL;
    const auto &t = it->second.table;
    if (t.size() > max_blocks) return RVKV_EINVAL;
    uint32_t *row = tables + (size_t)i * max_blocks;
    const uint32_t pad = t.empty() ? 0 : t.back();
    for (uint32_t j = 0; j < max_blocks; ++j)
      row[j] = j < t.size() ? t[j] : pad;
    ctx_lens[i] = it->second.num_tokens;
  }
  return RVKV_OK;
}

int rvkv_bm_slot(const rvkv_bm *bm, int64_t seq, uint32_t pos, uint32_t *block,
                 uint32_t *offset) {
  if (!bm || !block || !offset) return RVKV_EINVAL;
  auto it = bm->seqs.find(seq);
  if (it == bm->seqs.end()) return RVKV_EINVAL;
  const uint32_t bi = pos / bm->block_size;
  if (bi >= it->second.table.size()) return RVKV_EINVAL;
  *block = it->second.table[bi];
  *offset = pos % bm->block_size;
  return RVKV_OK;
}

uint32_t rvkv_bm_num_tokens(const rvkv_bm *bm, int64_t seq) {
  if (!bm) return 0;
  auto it = bm->seqs.find(seq);
  return it == bm->seqs.end() ? 0 : it->second.num_tokens;
}

uint32_t rvkv_bm_num_blocks(const rvkv_bm *bm, int64_t seq) {
  if (!bm) return 0;
  auto it = bm->seqs.find(seq);
  return it == bm->seqs.end() ? 0 : (uint32_t)it->second.table.size();
}

uint32_t rvkv_bm_refcount(const rvkv_bm *bm, uint32_t block) {
  return (bm && block < bm->num_blocks) ? bm->refcount[block] : 0;
}

int rvkv_bm_table(const rvkv_bm *bm, int64_t seq, uint32_t *table,
                  uint32_t cap) {
  if (!bm) return RVKV_EINVAL;
  auto it = bm->seqs.find(seq);
  if (it == bm->seqs.end()) return RVKV_EINVAL;
  const auto &t = it->second.table;
  if (table) {
    for (uint32_t i = 0; i < cap && i < t.size(); ++i) table[i] = t[i];
  }
  return (int)t.size();
}

}  // extern "C"
