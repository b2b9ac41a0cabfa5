/*
 * rvkv_oracle.c - TEST INFRASTRUCTURE ONLY. CPU restatement of rvllm's
 * paged-KV path, used as the parity checker by tests/, by
 * __graft_entry__.smoke() and as bench.py's cpu_baseline leg. Nothing in the
 * product (rvllm_amd/) links, loads or calls this file.
 *
 * Every function names the reference file:line it restates. The reference is
 * Rust (candle tensors); it cannot be built in this image (no Rust
 * toolchain), so this C file is the oracle. Storage follows rvllm's LOGICAL
 * per-layer layout [num_blocks, block_size, n_kv_heads, head_dim]
 * (src/kv_storage.rs:7-13) with either f32 cells (the reference's own dtype,
 * src/kv_storage.rs:94-97) or f16 cells (this build's storage type; values
 * are rounded f32->f16 round-to-nearest-even on write).
 *
 * Pinning (see the tests): the reference's known-answer tests
 * (src/kv_storage.rs:193-255, src/cuda/ops.rs:1070-1259,
 * src/model.rs:879-975, src/cuda/cublas_ops.rs:263-352,
 * src/model.rs:1184-1197), numpy's float16 conversion, a float64 brute force
 * and torch's CPU scaled_dot_product_attention.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_F16 1
#define ORC_F32 2

/* ---- f32 <-> f16, IEEE-754 binary16, round to nearest, ties to even ------
 * Written from the format definition: 1 sign, 5 exponent (bias 15),
 * 10 fraction bits; subnormals below 2^-14; overflow to infinity. */
uint16_t orc_f32_to_f16(float x) {
  uint32_t f;
  memcpy(&f, &x, 4);
  uint32_t sign = (f >> 16) & 0x8000u;
  uint32_t exp = (f >> 23) & 0xffu;
  uint32_t man = f & 0x7fffffu;
  if (exp == 0xffu) { /* inf or NaN */
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    uint32_t m = man >> 13;
    if (m == 0) m = 1; /* keep it a NaN */
    return (uint16_t)(sign | 0x7c00u | m | 0x200u);
  }
  int32_t e = (int32_t)exp - 127 + 15; /* rebiased exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow */
  if (e <= 0) {
    /* subnormal (or zero) in f16: value = man_full * 2^(exp-150);
     * f16 subnormal unit is 2^-24, so shift = 126 - exp... computed below */
    if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
    uint32_t full = man | 0x800000u; /* implicit 1 */
    uint32_t shift = (uint32_t)(14 - e); /* 24-bit significand -> 10-e bits */
    uint32_t q = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q); /* q may carry into the exponent field: ok */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1; /* may -> inf */
  return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t f;
  if (exp == 0x1fu) {
    f = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    if (man == 0) {
      f = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      f = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else {
    f = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &f, 4);
  return out;
}

void orc_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

static inline float cell_get(const void *cache, int dtype, size_t i) {
  if (dtype == ORC_F16) return orc_f16_to_f32(((const uint16_t *)cache)[i]);
  return ((const float *)cache)[i];
}

static inline void cell_set(void *cache, int dtype, size_t i, float x) {
  if (dtype == ORC_F16)
    ((uint16_t *)cache)[i] = orc_f32_to_f16(x);
  else
    ((float *)cache)[i] = x;
}

/* ---- KvStorage::write_tokens (src/kv_storage.rs:116-150) -------------
 * Consecutive tokens landing in consecutive slots of one block form a run
 * copied together (the reference's slice_set); a run is exactly the
 * per-token scatter of kv_write.cu:17-35, dest = ((block*bs + offset)*n_kv +
 * head)*hd + d. Returns 0, or -1 if a slot is out of range. */
int orc_write_tokens(void *cache_k, void *cache_v, int dtype,
                     uint32_t num_blocks, uint32_t bs, uint32_t n_kv,
                     uint32_t hd, const uint32_t *blocks,
                     const uint32_t *offsets, uint32_t n_tokens,
                     const float *k, const float *v) {
  size_t row = (size_t)n_kv * hd;
  uint32_t start = 0;
  while (start < n_tokens) {
    uint32_t block = blocks[start], off = offsets[start];
    uint32_t len = 1;
    while (start + len < n_tokens && blocks[start + len] == block &&
           offsets[start + len] == off + len)
      ++len;
    if (block >= num_blocks || off + len > bs) return -1;
    size_t dst = ((size_t)block * bs + off) * row;
    size_t src = (size_t)start * row;
    for (size_t i = 0; i < (size_t)len * row; ++i) {
      cell_set(cache_k, dtype, dst + i, k[src + i]);
      cell_set(cache_v, dtype, dst + i, v[src + i]);
    }
    start += len;
  }
  return 0;
}

/* Same, with f16 source rows copied bit for bit into an f16 cache. */
int orc_write_tokens_f16src(uint16_t *cache_k, uint16_t *cache_v,
                            uint32_t num_blocks, uint32_t bs, uint32_t n_kv,
                            uint32_t hd, const uint32_t *blocks,
                            const uint32_t *offsets, uint32_t n_tokens,
                            const uint16_t *k, const uint16_t *v) {
  size_t row = (size_t)n_kv * hd;
  for (uint32_t t = 0; t < n_tokens; ++t) {
    if (blocks[t] >= num_blocks || offsets[t] >= bs) return -1;
    size_t dst = ((size_t)blocks[t] * bs + offsets[t]) * row;
    memcpy(cache_k + dst, k + (size_t)t * row, row * 2);
    memcpy(cache_v + dst, v + (size_t)t * row, row * 2);
  }
  return 0;
}

/* ---- GatherPlan::new (src/kv_storage.rs:50-75) ------------------------
 * tables: the sequences' block tables concatenated; table_lens[b] entries
 * each; n_tokens[b] = read_num_tokens. Pads each table to max_blocks with
 * its own last block (0 for an empty table). out_idx may be NULL to only
 * size the plan. */
void orc_gather_plan(uint32_t batch, const uint32_t *table_lens,
                     const uint32_t *tables, const uint32_t *n_tokens,
                     uint32_t *out_idx, uint32_t *out_max_blocks,
                     uint32_t *out_ctx_len) {
  uint32_t max_blocks = 0, ctx_len = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    if (table_lens[b] > max_blocks) max_blocks = table_lens[b];
    if (n_tokens[b] > ctx_len) ctx_len = n_tokens[b];
  }
  *out_max_blocks = max_blocks;
  *out_ctx_len = ctx_len;
  if (!out_idx) return;
  size_t at = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    uint32_t n = table_lens[b];
    uint32_t pad = n ? tables[at + n - 1] : 0;
    for (uint32_t i = 0; i < max_blocks; ++i)
      out_idx[(size_t)b * max_blocks + i] = i < n ? tables[at + i] : pad;
    at += n;
  }
}

/* ---- KvStorage::gather (src/kv_storage.rs:157-173) --------------------
 * index_select over the padded plan, reshape to [batch, max_blocks*bs, n_kv,
 * hd], narrow to ctx_len, transpose to [batch, n_kv, ctx_len, hd]. Element
 * formula as kv_gather.cu:53-71. Out-of-range block ids read zeros. */
void orc_gather(const void *cache, int dtype, uint32_t num_blocks, uint32_t bs,
                uint32_t n_kv, uint32_t hd, const uint32_t *block_idx,
                uint32_t batch, uint32_t max_blocks, uint32_t ctx_len,
                float *out) {
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t h = 0; h < n_kv; ++h)
      for (uint32_t p = 0; p < ctx_len; ++p) {
        uint32_t blk = block_idx[(size_t)b * max_blocks + p / bs];
        float *o = out + (((size_t)b * n_kv + h) * ctx_len + p) * hd;
        if (blk >= num_blocks) {
          memset(o, 0, (size_t)hd * 4);
          continue;
        }
        size_t src = (((size_t)blk * bs + p % bs) * n_kv + h) * hd;
        for (uint32_t d = 0; d < hd; ++d) o[d] = cell_get(cache, dtype, src + d);
      }
}

/* ---- batch_mask (src/model.rs:346-369) ---------------------------------
 * mask[b][i][j] = -inf if j >= read_num_tokens[b] or j > offset_b + i or (a
 * window w > 0 and) j + w <= offset_b + i; 0 otherwise. */
void orc_batch_mask(uint32_t batch, const uint32_t *position_offset,
                    const uint32_t *read_num_tokens, uint32_t q_len,
                    uint32_t ctx_len, int32_t window, float *mask) {
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t i = 0; i < q_len; ++i)
      for (uint32_t j = 0; j < ctx_len; ++j) {
        uint64_t pos = (uint64_t)position_offset[b] + i;
        int outside = window > 0 && (uint64_t)j + (uint64_t)window <= pos;
        mask[((size_t)b * q_len + i) * ctx_len + j] =
            (j >= read_num_tokens[b] || j > pos || outside) ? -INFINITY : 0.0f;
      }
}

/* ---- gqa_attention (src/model.rs:377-415), f32 ------------------------
 * q [batch, n_heads, q_len, hd]; k, v [batch, n_kv, ctx_len, hd];
 * mask [batch, q_len, ctx_len]; out [batch, n_heads, q_len, hd].
 * Query head h reads KV head h / (n_heads/n_kv) (the group fold of
 * src/model.rs:389-392). scores = (q.k) * (1/sqrt(hd)) + mask; row softmax
 * (max-subtracted, candle_nn::ops::softmax); out = probs . v. */
static void attend_one(const float *q, const float *k, const float *v,
                       const float *mask_row0, uint32_t q_len,
                       uint32_t ctx_len, uint32_t hd, float scale, float *out,
                       float *scores) {
  for (uint32_t i = 0; i < q_len; ++i) {
    const float *qi = q + (size_t)i * hd;
    const float *mrow = mask_row0 + (size_t)i * ctx_len;
    float mx = -INFINITY;
    for (uint32_t j = 0; j < ctx_len; ++j) {
      const float *kj = k + (size_t)j * hd;
      float dot = 0.0f;
      for (uint32_t d = 0; d < hd; ++d) dot += qi[d] * kj[d];
      float s = dot * scale + mrow[j];
      scores[j] = s;
      if (s > mx) mx = s;
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < ctx_len; ++j) {
      float e = expf(scores[j] - mx);
      scores[j] = e;
      sum += e;
    }
    float *oi = out + (size_t)i * hd;
    for (uint32_t d = 0; d < hd; ++d) oi[d] = 0.0f;
    for (uint32_t j = 0; j < ctx_len; ++j) {
      float p = scores[j] / sum;
      const float *vj = v + (size_t)j * hd;
      for (uint32_t d = 0; d < hd; ++d) oi[d] += p * vj[d];
    }
  }
}

void orc_gqa_attention(const float *q, const float *k, const float *v,
                       const float *mask, uint32_t batch, uint32_t n_heads,
                       uint32_t n_kv, uint32_t q_len, uint32_t ctx_len,
                       uint32_t hd, float *out) {
  uint32_t group = n_heads / n_kv;
  float scale = (float)(1.0 / sqrt((double)hd));
  float *scores = (float *)malloc((size_t)(ctx_len ? ctx_len : 1) * 4);
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t h = 0; h < n_heads; ++h) {
      uint32_t kvh = h / group;
      attend_one(q + (((size_t)b * n_heads + h) * q_len) * hd,
                 k + (((size_t)b * n_kv + kvh) * ctx_len) * hd,
                 v + (((size_t)b * n_kv + kvh) * ctx_len) * hd,
                 mask + (size_t)b * q_len * ctx_len, q_len, ctx_len, hd, scale,
                 out + (((size_t)b * n_heads + h) * q_len) * hd, scores);
    }
  free(scores);
}

/* ---- float64 paged reference (src/metal/ops.rs:719-745) --------------------
 * Direct attention over the paged cache through the (unpadded) block table,
 * in double precision: for decode row b, keys j in [lo_b, ctx_lens[b]) with
 * lo_b = max(0, ctx - window) when window > 0. q, out: [batch, n_heads, hd].
 * Cache in the logical layout with f32 or f16 cells. ctx_len 0 -> zeros. */
void orc_paged_decode_f64(const void *cache_k, const void *cache_v, int dtype,
                          uint32_t bs, uint32_t n_kv, uint32_t hd,
                          const float *q, const uint32_t *tables,
                          uint32_t max_blocks, const uint32_t *ctx_lens,
                          uint32_t batch, uint32_t n_heads, double scale,
                          int32_t window, float *out) {
  uint32_t group = n_heads / n_kv;
  uint32_t cap = max_blocks * bs;
  double *sc = (double *)malloc((size_t)(cap ? cap : 1) * 8);
  double *acc = (double *)malloc((size_t)hd * 8);
  for (uint32_t b = 0; b < batch; ++b) {
    uint32_t ctx = ctx_lens[b];
    uint32_t lo = (window > 0 && ctx > (uint32_t)window) ? ctx - window : 0;
    for (uint32_t h = 0; h < n_heads; ++h) {
      uint32_t kvh = h / group;
      const float *qh = q + ((size_t)b * n_heads + h) * hd;
      float *oh = out + ((size_t)b * n_heads + h) * hd;
      if (ctx == 0) {
        memset(oh, 0, (size_t)hd * 4);
        continue;
      }
      double mx = -INFINITY;
      for (uint32_t j = lo; j < ctx; ++j) {
        size_t blk = tables[(size_t)b * max_blocks + j / bs];
        size_t at = ((blk * bs + j % bs) * n_kv + kvh) * hd;
        double dot = 0.0;
        for (uint32_t d = 0; d < hd; ++d)
          dot += (double)qh[d] * (double)cell_get(cache_k, dtype, at + d);
        sc[j] = dot * scale;
        if (sc[j] > mx) mx = sc[j];
      }
      double total = 0.0;
      for (uint32_t d = 0; d < hd; ++d) acc[d] = 0.0;
      for (uint32_t j = lo; j < ctx; ++j) {
        size_t blk = tables[(size_t)b * max_blocks + j / bs];
        size_t at = ((blk * bs + j % bs) * n_kv + kvh) * hd;
        double e = exp(sc[j] - mx);
        total += e;
        for (uint32_t d = 0; d < hd; ++d)
          acc[d] += e * (double)cell_get(cache_v, dtype, at + d);
      }
      for (uint32_t d = 0; d < hd; ++d) oh[d] = (float)(acc[d] / total);
    }
  }
  free(sc);
  free(acc);
}

/* ---- paged prefill / chunked attention, q_len >= 1 ---------
 * Float64 attention straight over the paged cache for q_len query rows per
 * sequence, with batch_mask's rule (src/model.rs:346-369): row i of
 * sequence b sits at position p = pos_offset[b] + i and sees key j iff
 * j < read_num[b], j <= p and, with a window w > 0, j + w > p. This is
 * src/metal/ops.rs:719-745 (the Metal attn_decode test reference, which
 * takes q_len > 1 with that causal mask) with the mask written as
 * batch_mask's. q and out are token-major: [batch * q_len, n_heads, hd].
 * A row that sees no key gets zeros (as a decode with ctx_len 0). */
void orc_paged_prefill_f64(const void *cache_k, const void *cache_v,
                           int dtype, uint32_t bs, uint32_t n_kv, uint32_t hd,
                           const float *q, const uint32_t *tables,
                           uint32_t max_blocks, const uint32_t *pos_offset,
                           const uint32_t *read_num, uint32_t batch,
                           uint32_t q_len, uint32_t n_heads, double scale,
                           int32_t window, float *out) {
  uint32_t group = n_heads / n_kv;
  uint32_t cap = max_blocks * bs;
  double *sc = (double *)malloc((size_t)(cap ? cap : 1) * 8);
  double *acc = (double *)malloc((size_t)hd * 8);
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t i = 0; i < q_len; ++i) {
      uint64_t p = (uint64_t)pos_offset[b] + i;
      uint64_t hi = read_num[b] < p + 1 ? read_num[b] : p + 1;
      if (hi > cap) hi = cap;
      uint64_t lo = (window > 0 && p + 1 > (uint64_t)window)
                        ? p + 1 - (uint64_t)window : 0;
      size_t row = (size_t)b * q_len + i;
      for (uint32_t h = 0; h < n_heads; ++h) {
        uint32_t kvh = h / group;
        const float *qh = q + (row * n_heads + h) * hd;
        float *oh = out + (row * n_heads + h) * hd;
        if (lo >= hi) {
          memset(oh, 0, (size_t)hd * 4);
          continue;
        }
        double mx = -INFINITY;
        for (uint64_t j = lo; j < hi; ++j) {
          size_t blk = tables[(size_t)b * max_blocks + j / bs];
          size_t at = ((blk * bs + j % bs) * n_kv + kvh) * hd;
          double dot = 0.0;
          for (uint32_t d = 0; d < hd; ++d)
            dot += (double)qh[d] * (double)cell_get(cache_k, dtype, at + d);
          sc[j] = dot * scale;
          if (sc[j] > mx) mx = sc[j];
        }
        double total = 0.0;
        for (uint32_t d = 0; d < hd; ++d) acc[d] = 0.0;
        for (uint64_t j = lo; j < hi; ++j) {
          size_t blk = tables[(size_t)b * max_blocks + j / bs];
          size_t at = ((blk * bs + j % bs) * n_kv + kvh) * hd;
          double e = exp(sc[j] - mx);
          total += e;
          for (uint32_t d = 0; d < hd; ++d)
            acc[d] += e * (double)cell_get(cache_v, dtype, at + d);
        }
        for (uint32_t d = 0; d < hd; ++d) oh[d] = (float)(acc[d] / total);
      }
    }
  free(sc);
  free(acc);
}

/* ---- copy-on-write block copy (new behaviour; invariants only) -------
 * dst block := src block, every cell, for one layer's K or V tensor. */
void orc_copy_blocks(void *cache, int dtype, uint32_t bs, uint32_t n_kv,
                     uint32_t hd, const uint32_t *src, const uint32_t *dst,
                     uint32_t n) {
  size_t cell = dtype == ORC_F16 ? 2 : 4;
  size_t blk = (size_t)bs * n_kv * hd * cell;
  for (uint32_t i = 0; i < n; ++i)
    memmove((char *)cache + dst[i] * blk, (const char *)cache + src[i] * blk,
            blk);
}

/* 64-bit FNV-1a over the logical bytes of each listed block, read as 16-bit
 * words (hd counts words: two per f32 cell) - the checksum
 * rvkv_block_checksums computes on the device. */
void orc_block_checksums(const uint16_t *cache, uint32_t bs, uint32_t n_kv,
                         uint32_t hd, const uint32_t *blocks, uint32_t n,
                         uint64_t *out) {
  size_t cells = (size_t)bs * n_kv * hd;
  for (uint32_t i = 0; i < n; ++i) {
    const uint16_t *c = cache + (size_t)blocks[i] * cells;
    uint64_t hsh = 0xcbf29ce484222325ull;
    for (size_t j = 0; j < cells; ++j) {
      hsh = (hsh ^ (c[j] & 0xffu)) * 0x100000001b3ull;
      hsh = (hsh ^ (c[j] >> 8)) * 0x100000001b3ull;
    }
    out[i] = hsh;
  }
}

/* ---- the reference decode pipeline, for the CPU baseline -------------------
 * One decode step of one layer exactly as rvllm's CPU path runs it
 * (src/model.rs:628-644 with q_len 1): write_tokens of each sequence's new
 * row, then the padded gather, the batch mask and gqa_attention. Work is
 * split over (sequence, KV head) across n_threads pthreads; each does the
 * gather of its slice (a padded [ctx_len, hd] K and V in f32) and the
 * attention of its group of query heads against it, so the arithmetic is the
 * reference's, parallelised. Cache: logical layout, f16 or f32 cells. */
typedef struct {
  const void *ck, *cv;
  int dtype;
  uint32_t bs, n_kv, hd, n_heads, max_blocks, ctx_len, batch;
  const uint32_t *block_idx, *read_num_tokens;
  const float *q;
  float *out;
  uint32_t next; /* work counter */
  pthread_mutex_t mu;
} orc_job;

static void *orc_worker(void *arg) {
  orc_job *J = (orc_job *)arg;
  uint32_t group = J->n_heads / J->n_kv;
  size_t slab = (size_t)J->ctx_len * J->hd;
  float *k = (float *)malloc((slab ? slab : 1) * 4);
  float *v = (float *)malloc((slab ? slab : 1) * 4);
  float *mask = (float *)malloc((size_t)(J->ctx_len ? J->ctx_len : 1) * 4);
  float *scores = (float *)malloc((size_t)(J->ctx_len ? J->ctx_len : 1) * 4);
  float scale = (float)(1.0 / sqrt((double)J->hd));
  for (;;) {
    pthread_mutex_lock(&J->mu);
    uint32_t w = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (w >= J->batch * J->n_kv) break;
    uint32_t b = w / J->n_kv, h = w % J->n_kv;
    for (uint32_t p = 0; p < J->ctx_len; ++p) { /* the padded gather */
      size_t blk = J->block_idx[(size_t)b * J->max_blocks + p / J->bs];
      size_t src = ((blk * J->bs + p % J->bs) * J->n_kv + h) * J->hd;
      for (uint32_t d = 0; d < J->hd; ++d) {
        k[(size_t)p * J->hd + d] = cell_get(J->ck, J->dtype, src + d);
        v[(size_t)p * J->hd + d] = cell_get(J->cv, J->dtype, src + d);
      }
    }
    uint32_t pos = J->read_num_tokens[b] ? J->read_num_tokens[b] - 1 : 0;
    orc_batch_mask(1, &pos, &J->read_num_tokens[b], 1, J->ctx_len, 0, mask);
    for (uint32_t g = 0; g < group; ++g) {
      uint32_t qh = h * group + g;
      attend_one(J->q + ((size_t)b * J->n_heads + qh) * J->hd, k, v, mask, 1,
                 J->ctx_len, J->hd, scale,
                 J->out + ((size_t)b * J->n_heads + qh) * J->hd, scores);
    }
  }
  free(k);
  free(v);
  free(mask);
  free(scores);
  return NULL;
}

/* Appends one f32 row per sequence (src/kv_storage.rs:116-150), then runs
 * the padded-gather attention above. Returns 0 or -1 on a bad slot. */
int orc_decode_step(void *cache_k, void *cache_v, int dtype, uint32_t num_blocks,
                    uint32_t bs, uint32_t n_kv, uint32_t hd,
                    const uint32_t *slot_block, const uint32_t *slot_off,
                    const float *new_k, const float *new_v,
                    const uint32_t *block_idx, uint32_t max_blocks,
                    const uint32_t *read_num_tokens, uint32_t batch,
                    uint32_t n_heads, const float *q, float *out,
                    uint32_t n_threads) {
  if (orc_write_tokens(cache_k, cache_v, dtype, num_blocks, bs, n_kv, hd,
                       slot_block, slot_off, batch, new_k, new_v))
    return -1;
  uint32_t ctx_len = 0;
  for (uint32_t b = 0; b < batch; ++b)
    if (read_num_tokens[b] > ctx_len) ctx_len = read_num_tokens[b];
  orc_job J;
  J.ck = cache_k;
  J.cv = cache_v;
  J.dtype = dtype;
  J.bs = bs;
  J.n_kv = n_kv;
  J.hd = hd;
  J.n_heads = n_heads;
  J.max_blocks = max_blocks;
  J.ctx_len = ctx_len;
  J.batch = batch;
  J.block_idx = block_idx;
  J.read_num_tokens = read_num_tokens;
  J.q = q;
  J.out = out;
  J.next = 0;
  pthread_mutex_init(&J.mu, NULL);
  if (n_threads < 1) n_threads = 1;
  if (n_threads > 256) n_threads = 256;
  pthread_t th[256];
  for (uint32_t t = 1; t < n_threads; ++t)
    pthread_create(&th[t], NULL, orc_worker, &J);
  orc_worker(&J);
  for (uint32_t t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
  pthread_mutex_destroy(&J.mu);
  return 0;
}

/* ---- attention prep before the append -------------------------
 * rope_cos_sin (src/model.rs:224-250): theta_j = rope_theta^(-2j/hd) (f32),
 * divided by factors[j] when given (Llama 3); angle = pos * theta_j;
 * cos/sin [n, hd/2] in f32. */
void orc_rope_cos_sin(float rope_theta, const float *factors, uint32_t hd,
                      const uint32_t *positions, uint32_t n, float *cos_out,
                      float *sin_out) {
  uint32_t half = hd / 2;
  for (uint32_t j = 0; j < half; ++j) {
    float theta = powf(rope_theta, -2.0f * (float)j / (float)hd);
    if (factors) theta = theta / factors[j];
    for (uint32_t i = 0; i < n; ++i) {
      float a = (float)positions[i] * theta;
      cos_out[(size_t)i * half + j] = cosf(a);
      sin_out[(size_t)i * half + j] = sinf(a);
    }
  }
}

/* rms_norm over the last dim (src/model.rs:200-215): rms = sqrt(mean(x^2) +
 * eps); out = x / rms * w. rows x dim, in place allowed. */
void orc_rms_norm(const float *x, const float *w, uint32_t rows, uint32_t dim,
                  float eps, float *out) {
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * dim;
    float ss = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) ss += xr[d] * xr[d];
    float rms = sqrtf(ss / (float)dim + eps);
    for (uint32_t d = 0; d < dim; ++d)
      out[(size_t)r * dim + d] = (xr[d] / rms) * w[d];
  }
}

/* rope_apply, rotate-half (src/model.rs:252-264), rows x hd with one cos/sin
 * row per input row. */
void orc_rope_apply(const float *x, const float *cos_t, const float *sin_t,
                    uint32_t rows, uint32_t hd, float *out) {
  uint32_t half = hd / 2;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t j = 0; j < half; ++j) {
      float first = x[(size_t)r * hd + j], second = x[(size_t)r * hd + half + j];
      float c = cos_t[(size_t)r * half + j], s = sin_t[(size_t)r * half + j];
      float a = first * c, b = second * s, e = first * s, f = second * c;
      out[(size_t)r * hd + j] = a - b;
      out[(size_t)r * hd + half + j] = e + f;
    }
}

/* The prep segment of Attention::forward (src/model.rs:600-626) for `rows`
 * tokens, then write_tokens of K/V (src/model.rs:628-639): q/k/v inputs are
 * the projection outputs [rows, heads, hd] (bias not yet added); q_out gets
 * the normed + rotated q; the cache (logical layout, f16 or f32 cells)
 * gets the normed + rotated k and the biased v at each row's slot. NULL bias/norm = absent. */
int orc_attn_prep(const float *q_in, const float *k_in, const float *v_in,
                  uint32_t rows, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                  const float *q_bias, const float *k_bias, const float *v_bias,
                  const float *q_norm, const float *k_norm, float eps,
                  const float *cos_t, const float *sin_t,
                  const uint32_t *slot_block, const uint32_t *slot_off,
                  void *cache_k, void *cache_v, int dtype, uint32_t num_blocks,
                  uint32_t bs, float *q_out) {
  uint32_t half = hd / 2;
  float *buf = (float *)malloc((size_t)hd * 4 * 2);
  float *nb = buf + hd;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *cr = cos_t + (size_t)r * half, *sr = sin_t + (size_t)r * half;
    for (uint32_t h = 0; h < n_heads + 2 * n_kv; ++h) {
      int is_q = h < n_heads, is_v = h >= n_heads + n_kv;
      uint32_t hh = is_q ? h : (is_v ? h - n_heads - n_kv : h - n_heads);
      const float *src =
          (is_q ? q_in + ((size_t)r * n_heads + hh) * hd
                : (is_v ? v_in : k_in) + ((size_t)r * n_kv + hh) * hd);
      const float *bias = is_q ? q_bias : (is_v ? v_bias : k_bias);
      for (uint32_t d = 0; d < hd; ++d)
        buf[d] = bias ? src[d] + bias[(size_t)hh * hd + d] : src[d];
      if (is_v) {
        if (slot_block[r] >= num_blocks || slot_off[r] >= bs) {
          free(buf);
          return -1;
        }
        size_t dst = (((size_t)slot_block[r] * bs + slot_off[r]) * n_kv + hh) * hd;
        for (uint32_t d = 0; d < hd; ++d) cell_set(cache_v, dtype, dst + d, buf[d]);
        continue;
      }
      const float *w = is_q ? q_norm : k_norm;
      if (w) {
        orc_rms_norm(buf, w, 1, hd, eps, nb);
        memcpy(buf, nb, (size_t)hd * 4);
      }
      orc_rope_apply(buf, cr, sr, 1, hd, nb);
      if (is_q) {
        memcpy(q_out + ((size_t)r * n_heads + hh) * hd, nb, (size_t)hd * 4);
      } else {
        if (slot_block[r] >= num_blocks || slot_off[r] >= bs) {
          free(buf);
          return -1;
        }
        size_t dst = (((size_t)slot_block[r] * bs + slot_off[r]) * n_kv + hh) * hd;
        for (uint32_t d = 0; d < hd; ++d) cell_set(cache_k, dtype, dst + d, nb[d]);
      }
    }
  }
  free(buf);
  return 0;
}
