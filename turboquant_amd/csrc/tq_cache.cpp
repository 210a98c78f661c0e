// tq_cache.cpp -- device-resident compressed KV caches behind a C ABI:
// CompressedStorage (reference src/cache/storage.rs:24-203), PqoCache
// (src/cache/pqo.rs:21-236; PQO, and PQ with outlier_blocks = 0) and TqCache
// (src/cache/tq.rs: PQ codes plus the QJL sketch of the keys' residuals),
// each with the CompressedKVCache contract.
//
// Layout per layer: K/V codes [num_kv_heads][capacity][head_dim*bits/8] u8
// and scales [num_kv_heads][capacity][head_dim/32] f16, token t of head h at
// record h * capacity + t, exactly what the fused kernels read with
// kv_head_stride = capacity; a TqCache adds signs [num_kv_heads][capacity]
// [head_dim/8] u8 and residual norms [num_kv_heads][capacity] f16 at the
// same records.  Appends quantize straight into their records (one launch
// per tensor, all heads at once; a TqCache then sketches the new keys);
// growth reallocates to needed + max(needed / 4, 128) and copies the old rows
// (storage.rs:108-139, tq.rs:64-94).  Decode runs the single-launch fused
// attention over the stored records.
#include "tq_common.h"

#include <cstring>
#include <new>
#include <vector>

namespace {

struct LayerBuffers {
  uint8_t *k_idx = nullptr, *v_idx = nullptr;
  uint16_t *k_sc = nullptr, *v_sc = nullptr;
  uint8_t *signs = nullptr;     // QJL only
  uint16_t *norms = nullptr;    // QJL only
  size_t cap = 0;   // records per head
  size_t seq = 0;   // stored tokens per head
  bool active = false;
};

struct CacheMode {
  int bits = 3;
  int norm_mode = TQ_NORM_MAXNORM;
  size_t outlier_blocks = TQ_OUTLIER_ALL;
  bool qjl = false;
};

// Stream-ordered device memory from the device's default pool.
template <class T>
bool pool_alloc(T **p, size_t bytes, hipStream_t stream) {
  void *q = nullptr;
  if (hipMallocAsync(&q, bytes, stream) != hipSuccess) return false;
  *p = static_cast<T *>(q);
  return true;
}
inline void pool_free(void *p, hipStream_t stream) {
  if (p) (void)hipFreeAsync(p, stream);
}

class CompressedStorage {
 public:
  CompressedStorage(int num_kv_heads, int head_dim, int bits, int num_layers, bool qjl)
      : heads_(num_kv_heads), head_dim_(head_dim), bits_(bits), qjl_(qjl), layers_(num_layers) {}
  ~CompressedStorage() { release_all(nullptr); }

  int packed_dim() const { return head_dim_ * bits_ / 8; }
  int num_blocks() const { return head_dim_ / 32; }
  int sign_bytes() const { return head_dim_ / 8; }
  size_t seq_len(int l) const { return layers_[l].seq; }
  size_t capacity(int l) const { return layers_[l].cap; }
  bool is_active(int l) const { return layers_[l].active && layers_[l].seq > 0; }
  const LayerBuffers &layer(int l) const { return layers_[l]; }

  // storage.rs:108-139 (and ensure_qjl_capacity, tq.rs:64-94, same rule)
  int ensure_capacity(int l, size_t needed, hipStream_t stream) {
    LayerBuffers &L = layers_[l];
    if (L.cap >= needed) return TQ_OK;
    const size_t grow = needed / 4 > 128 ? needed / 4 : 128;
    const size_t cap = needed + grow;
    const size_t ib = (size_t)heads_ * cap * packed_dim(), sb = (size_t)heads_ * cap * num_blocks() * 2;
    const size_t gb = (size_t)heads_ * cap * sign_bytes(), nb = (size_t)heads_ * cap * 2;
    LayerBuffers N;
    N.cap = cap;
    N.seq = L.seq;
    N.active = L.active;
    // stream-ordered allocation and release (the device's memory pool): the
    // old buffers go back to the pool after the work queued before them, so
    // growth never waits on the host
    bool ok = pool_alloc(&N.k_idx, ib, stream) && pool_alloc(&N.v_idx, ib, stream) && pool_alloc(&N.k_sc, sb, stream) &&
              pool_alloc(&N.v_sc, sb, stream);
    if (ok && qjl_) ok = pool_alloc(&N.signs, gb, stream) && pool_alloc(&N.norms, nb, stream);
    if (!ok) {
      free_layer(N, stream);
      return tqh::fail(TQ_ERR_DEVICE, "cache allocation of %zu records per head failed", cap);
    }
    // new capacity starts zeroed, as Tensor::zeros
    ok = hipMemsetAsync(N.k_idx, 0, ib, stream) == hipSuccess && hipMemsetAsync(N.v_idx, 0, ib, stream) == hipSuccess &&
         hipMemsetAsync(N.k_sc, 0, sb, stream) == hipSuccess && hipMemsetAsync(N.v_sc, 0, sb, stream) == hipSuccess;
    if (ok && qjl_)
      ok = hipMemsetAsync(N.signs, 0, gb, stream) == hipSuccess && hipMemsetAsync(N.norms, 0, nb, stream) == hipSuccess;
    if (!ok) {
      free_layer(N, stream);
      return tqh::fail(TQ_ERR_DEVICE, "cache clear failed");
    }
    if (L.seq > 0) {
      auto copy = [&](void *dst, const void *src, size_t rec_bytes) {
        return hipMemcpy2DAsync(dst, cap * rec_bytes, src, L.cap * rec_bytes, L.seq * rec_bytes, heads_,
                                hipMemcpyDeviceToDevice, stream) == hipSuccess;
      };
      const size_t pi = packed_dim(), ps = (size_t)num_blocks() * 2;
      ok = copy(N.k_idx, L.k_idx, pi) && copy(N.v_idx, L.v_idx, pi) && copy(N.k_sc, L.k_sc, ps) &&
           copy(N.v_sc, L.v_sc, ps);
      if (ok && qjl_) ok = copy(N.signs, L.signs, sign_bytes()) && copy(N.norms, L.norms, 2);
      if (!ok) {
        free_layer(N, stream);
        return tqh::fail(TQ_ERR_DEVICE, "cache growth copy failed");
      }
    }
    // queued work may still read the old buffers: they return to the pool in
    // stream order, after it
    free_layer(L, stream);
    L = N;
    return TQ_OK;
  }

  void set_seq(int l, size_t seq) {
    layers_[l].seq = seq;
    layers_[l].active = true;
  }

  // storage.rs:175-186 (and the QJL buffers, tq.rs:303-312): the buffers go
  // back to the pool in the order of `stream`, after the work queued on it
  void reset(hipStream_t stream) { release_all(stream); }

  // storage.rs:188-202, plus the whole QJL tensors as tq.rs:314-323 counts them
  size_t memory_usage() const {
    size_t total = 0;
    for (const LayerBuffers &L : layers_) {
      if (L.seq > 0) {
        total += 2 * (size_t)heads_ * L.seq * packed_dim();
        total += 2 * (size_t)heads_ * L.seq * num_blocks() * 2;
      }
      if (qjl_ && L.signs) total += (size_t)heads_ * L.cap * (sign_bytes() + 2);
    }
    return total;
  }

 private:
  static void free_layer(LayerBuffers &L, hipStream_t stream) {
    for (void *p : {(void *)L.k_idx, (void *)L.v_idx, (void *)L.k_sc, (void *)L.v_sc, (void *)L.signs, (void *)L.norms})
      pool_free(p, stream);
    L = LayerBuffers{};
  }
  void release_all(hipStream_t stream) {
    for (LayerBuffers &L : layers_) free_layer(L, stream);
  }

  int heads_, head_dim_, bits_;
  bool qjl_;
  std::vector<LayerBuffers> layers_;
};

// A PqoCache (mode.qjl false) or TqCache (mode.qjl true).
class KvCache {
 public:
  KvCache(int num_layers, int num_kv_heads, int head_dim, const CacheMode &mode)
      : layers_(num_layers), heads_(num_kv_heads), head_dim_(head_dim), mode_(mode),
        storage_(num_kv_heads, head_dim, mode.bits, num_layers, mode.qjl) {}
  // Every buffer is released in the order of the stream of the cache's last
  // call (as the reference's tensors are freed on their device's stream): no
  // host synchronization, and queued work that reads them runs first.
  ~KvCache() {
    storage_.reset(stream_);
    for (void *p : {ws_, rmat_, rq_}) pool_free(p, stream_);
  }
  // the stream of the cache's latest call
  void use_stream(hipStream_t stream) { stream_ = stream; }
  hipStream_t last_stream() const { return stream_; }

  int layers() const { return layers_; }
  int num_kv_heads() const { return heads_; }
  int head_dim() const { return head_dim_; }
  const CacheMode &mode() const { return mode_; }
  CompressedStorage &storage() { return storage_; }

  // quantize_and_store (pqo.rs:64-100, tq.rs:97-145): k, v [num_kv_heads][tokens][head_dim].
  // A TqCache given q (num_q_rows rows) also projects it into the rq scratch
  // in the sketch's launch.
  int append(int l, const void *k, const void *v, int dtype, int tokens, size_t *old_seq, hipStream_t stream,
             const void *q = nullptr, int q_dtype = TQ_DTYPE_F32, size_t num_q_rows = 0) {
    const size_t old = storage_.seq_len(l);
    *old_seq = old;
    if (tokens == 0) return TQ_OK;
    int rc = storage_.ensure_capacity(l, old + tokens, stream);
    if (rc) return rc;
    const LayerBuffers &L = storage_.layer(l);
    rc = tq_polar_quantize_to_cache(k, dtype, heads_, tokens, L.k_idx, L.k_sc, (long long)L.cap, (long long)old,
                                    head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode, stream);
    if (rc) return rc;
    rc = tq_polar_quantize_to_cache(v, dtype, heads_, tokens, L.v_idx, L.v_sc, (long long)L.cap, (long long)old,
                                    head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode, stream);
    if (rc) return rc;
    if (mode_.qjl) {
      rc = sign_matrix(stream);
      if (rc) return rc;
      if (num_q_rows) {
        rc = rq_scratch(num_q_rows, stream);
        if (rc) return rc;
      }
      rc = tq_qjl_cache_sketch_project(k, dtype, heads_, tokens, L.k_idx, L.k_sc,
                                       static_cast<const uint32_t *>(rmat_), L.signs, L.norms, (long long)L.cap,
                                       (long long)old, head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode,
                                       q, q_dtype, static_cast<float *>(rq_), num_q_rows, stream);
      if (rc) return rc;
    }
    storage_.set_seq(l, old + tokens);
    return TQ_OK;
  }

  // dequantize_full (common.rs:16-62): [num_kv_heads][seq][head_dim]
  int dequantize_full(int l, void *k_out, void *v_out, int dtype, hipStream_t stream) {
    const LayerBuffers &L = storage_.layer(l);
    int rc = tq_polar_dequantize_from_cache(L.k_idx, L.k_sc, (long long)L.cap, heads_, (int)L.seq, k_out, dtype,
                                            head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode, stream);
    if (rc) return rc;
    return tq_polar_dequantize_from_cache(L.v_idx, L.v_sc, (long long)L.cap, heads_, (int)L.seq, v_out, dtype,
                                          head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode, stream);
  }

  int rq_scratch(size_t num_rows, hipStream_t stream) {
    const size_t need = num_rows * (size_t)head_dim_ * sizeof(float);
    if (need <= rq_bytes_) return TQ_OK;
    pool_free(rq_, stream);  // after the queued work that reads it
    rq_ = nullptr;
    rq_bytes_ = 0;
    if (!pool_alloc(&rq_, need, stream)) return tqh::fail(TQ_ERR_DEVICE, "rq allocation failed");
    rq_bytes_ = need;
    return TQ_OK;
  }

  // rq = R q for num_rows query rows, in the cache's scratch
  int project(const void *q, int q_dtype, size_t num_rows, hipStream_t stream) {
    int rc = sign_matrix(stream);
    if (rc) return rc;
    rc = rq_scratch(num_rows, stream);
    if (rc) return rc;
    return tq_qjl_project(q, q_dtype, static_cast<const uint32_t *>(rmat_), static_cast<float *>(rq_), num_rows,
                          head_dim_, stream);
  }

  // compute_logit_bias (tq.rs:185-253): q [num_q_heads][q_len][head_dim],
  // bias [num_q_heads][q_len][seq_len] in q's dtype
  int logit_bias(int l, const void *q, int q_dtype, int num_q_heads, int q_len, void *bias, hipStream_t stream) {
    int rc = project(q, q_dtype, (size_t)num_q_heads * q_len, stream);
    if (rc) return rc;
    const LayerBuffers &L = storage_.layer(l);
    return tq_qjl_logit_bias(static_cast<const float *>(rq_), num_q_heads, q_len, L.signs, L.norms, heads_,
                             (int)L.seq, (long long)L.cap, head_dim_, bias, q_dtype, stream);
  }

  // decode_cuda (pqo.rs:106-174) as one fused launch over the stored records;
  // a TqCache adds the QJL correction inline (rq_ready: the append already
  // projected q)
  int attend(int l, const void *q, int q_dtype, int num_q_heads, float scale, void *out, int out_dtype,
             hipStream_t stream, bool rq_ready = false) {
    const LayerBuffers &L = storage_.layer(l);
    int rc = TQ_OK;
    const size_t need = tq_attention_workspace_size(1, num_q_heads, heads_, head_dim_, (int)L.cap);
    if (need == 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid attention shape");
    if (need > ws_bytes_) {
      pool_free(ws_, stream);  // after the queued decodes that use it
      ws_ = nullptr;
      ws_bytes_ = 0;
      if (!pool_alloc(&ws_, need, stream)) return tqh::fail(TQ_ERR_DEVICE, "workspace allocation failed");
      ws_bytes_ = need;
      rc = tq_attention_workspace_init(ws_, ws_bytes_, 1, num_q_heads, heads_, head_dim_, (int)L.cap, stream);
      if (rc) return rc;
    }
    // a TqCache whose append did not project q (no token appended): the
    // decode launch projects it from the sign matrix
    const bool in_launch = mode_.qjl && !rq_ready;
    if (in_launch) {
      rc = sign_matrix(stream);
      if (rc) return rc;
    }
    // the length is known here: the kernel reads none from memory
    return tqh::decode_attention(q, q_dtype, L.k_idx, L.k_sc, L.v_idx, L.v_sc,
                                 mode_.qjl && !in_launch ? static_cast<const float *>(rq_) : nullptr,
                                 mode_.qjl ? L.signs : nullptr, mode_.qjl ? L.norms : nullptr, nullptr, (int)L.seq, 1,
                                 num_q_heads, heads_, head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode,
                                 (int)L.cap, (long long)L.cap, 0, scale, out, out_dtype, ws_, ws_bytes_, stream,
                                 in_launch ? static_cast<const uint32_t *>(rmat_) : nullptr);
  }

  // multi-query attention of q [num_q_heads][q_len][head_dim] over the whole
  // layer, the queries at its last q_len positions
  int attend_prefill(int l, const void *q, int q_dtype, int num_q_heads, int q_len, int causal, float scale, void *out,
                     int out_dtype, hipStream_t stream) {
    const LayerBuffers &L = storage_.layer(l);
    if (mode_.qjl) {
      int rc = project(q, q_dtype, (size_t)num_q_heads * q_len, stream);
      if (rc) return rc;
    }
    return tq_cache_prefill_attention(q, q_dtype, L.k_idx, L.k_sc, L.v_idx, L.v_sc,
                                      mode_.qjl ? static_cast<const float *>(rq_) : nullptr,
                                      mode_.qjl ? L.signs : nullptr, mode_.qjl ? L.norms : nullptr, num_q_heads, q_len,
                                      heads_, head_dim_, mode_.bits, mode_.outlier_blocks, mode_.norm_mode,
                                      (int)L.seq, (long long)L.cap, causal, scale, out, out_dtype, stream);
  }

 private:
  // build_rademacher_matrix (precomputed/mod.rs:116-125) as sign bits, once
  int sign_matrix(hipStream_t stream) {
    if (rmat_) return TQ_OK;
    const size_t bytes = (size_t)head_dim_ * head_dim_ / 8;
    if (!pool_alloc(&rmat_, bytes, stream)) {
      rmat_ = nullptr;
      return tqh::fail(TQ_ERR_DEVICE, "sign matrix allocation failed");
    }
    return tq_qjl_sign_matrix(static_cast<uint32_t *>(rmat_), head_dim_, kDefaultQjlSeed, stream);
  }

  static constexpr uint64_t kDefaultQjlSeed = 12345;  // DEFAULT_QJL_SEED (config.rs:17)

  int layers_, heads_, head_dim_;
  CacheMode mode_;
  CompressedStorage storage_;
  hipStream_t stream_ = nullptr;
  void *ws_ = nullptr;
  size_t ws_bytes_ = 0;
  void *rmat_ = nullptr;
  void *rq_ = nullptr;
  size_t rq_bytes_ = 0;
};

KvCache *as_cache(void *h) { return static_cast<KvCache *>(h); }

int check_layer(KvCache *c, int layer) {
  if (!c) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null cache");
  if (layer < 0 || layer >= c->layers())
    return tqh::fail(TQ_ERR_LAYER_OUT_OF_RANGE, "layer %d out of range (num_layers %d)", layer, c->layers());
  return TQ_OK;
}

int check_q(KvCache *c, const void *q, int q_dtype, int num_q_heads) {
  if (!q) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null query");
  if (!tqh::valid_dtype(q_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", q_dtype);
  if (num_q_heads <= 0 || num_q_heads % c->num_kv_heads() != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_q_heads (%d) must be a multiple of num_kv_heads (%d)", num_q_heads,
                     c->num_kv_heads());
  return TQ_OK;
}

}  // namespace

extern "C" int tq_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, int norm_mode,
                               size_t outlier_blocks, int qjl, void **cache) {
  if (!cache) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null handle pointer");
  *cache = nullptr;
  if (head_dim <= 0 || head_dim % 32 != 0)  // PqoCache::new / TqCache::new (pqo.rs:30-39, tq.rs:33-40)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT,
                     "head_dim (%d) must be divisible by QUANT_BLOCK_SIZE (32). Models with head_dim=%d are not "
                     "supported by TurboQuant compression.", head_dim, head_dim);
  if (num_layers <= 0 || num_kv_heads <= 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "empty cache shape");
  tqh::PolarCodec codec;
  int rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (qjl && codec.outlier)  // only outlier_blocks = 0 builds the Rademacher matrix (precomputed/mod.rs:84-88)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL Rademacher matrix not precomputed: TqCache needs outlier_blocks 0");
  if (qjl && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "TqCache takes head_dim 64, 128 or 256 (got %d)", head_dim);
  CacheMode mode;
  mode.bits = bits;
  mode.norm_mode = norm_mode;
  mode.outlier_blocks = outlier_blocks;
  mode.qjl = qjl != 0;
  KvCache *c = new (std::nothrow) KvCache(num_layers, num_kv_heads, head_dim, mode);
  if (!c) return tqh::fail(TQ_ERR_DEVICE, "out of host memory");
  *cache = c;
  return TQ_OK;
}

extern "C" void tq_cache_destroy(void *cache) {
  KvCache *c = as_cache(cache);
  if (!c) return;
  delete c;  // every buffer released in the order of the cache's last stream
}

extern "C" int tq_cache_is_tq(void *cache) {
  KvCache *c = as_cache(cache);
  return c && c->mode().qjl ? 1 : 0;
}

extern "C" int tq_cache_prefill(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                                const void *q, int q_dtype, int num_q_heads, int q_len, void *k_out, void *v_out,
                                int *returned_originals, void *logit_bias_out, hipStream_t stream) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  if (!tqh::valid_dtype(dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (tokens < 0 || !returned_originals) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  const bool tq = c->mode().qjl;
  if (tq) {
    rc = check_q(c, q, q_dtype, num_q_heads);
    if (rc) return rc;
    if (q_len < 0 || (q_len > 0 && !logit_bias_out))
      return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "TqCache prefill needs q_len >= 0 and a logit bias output");
  }
  size_t old = 0;
  c->use_stream(stream);
  rc = c->append(layer, k, v, dtype, tokens, &old, stream);
  if (rc) return rc;
  // pqo.rs:184-200, tq.rs:258-273: the first prefill returns the caller's own K/V
  *returned_originals = old == 0 ? 1 : 0;
  if (old != 0) {
    if (!k_out || !v_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null output for the dequantized cache");
    rc = c->dequantize_full(layer, k_out, v_out, dtype, stream);
    if (rc) return rc;
  }
  if (tq && q_len > 0) return c->logit_bias(layer, q, q_dtype, num_q_heads, q_len, logit_bias_out, stream);
  return TQ_OK;
}

extern "C" int tq_cache_decode(void *cache, int layer, const void *k, const void *v, int kv_dtype, int tokens,
                               const void *q, int q_dtype, int num_q_heads, float softmax_scale, void *out,
                               int out_dtype, hipStream_t stream) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  if (!tqh::valid_dtype(kv_dtype) || !tqh::valid_dtype(out_dtype))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype");
  rc = check_q(c, q, q_dtype, num_q_heads);
  if (rc) return rc;
  if (tokens < 0 || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  const CacheMode &m = c->mode();
  if (m.outlier_blocks > 0 && m.outlier_blocks < (size_t)c->head_dim() / 32)  // checked before anything is stored
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT,
                     "fused decode takes outlier_blocks 0 or all (mixed configs: tq_cache_decode_dequantized)");
  size_t old = 0;
  const bool fuse_rq = m.qjl && tokens > 0;  // the sketch launch projects q too
  c->use_stream(stream);
  rc = c->append(layer, k, v, kv_dtype, tokens, &old, stream, fuse_rq ? q : nullptr, q_dtype,
                 fuse_rq ? (size_t)num_q_heads : 0);
  if (rc) return rc;
  if (!c->storage().is_active(layer)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "decode over an empty cache");
  return c->attend(layer, q, q_dtype, num_q_heads, softmax_scale, out, out_dtype, stream, fuse_rq);
}

extern "C" int tq_cache_decode_dequantized(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                                           const void *q, int q_dtype, int num_q_heads, int q_len, void *k_out,
                                           void *v_out, void *logit_bias_out, hipStream_t stream) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  if (!tqh::valid_dtype(dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (tokens < 0 || !k_out || !v_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  const bool tq = c->mode().qjl;
  if (tq) {
    rc = check_q(c, q, q_dtype, num_q_heads);
    if (rc) return rc;
    if (q_len <= 0 || !logit_bias_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "TqCache decode needs a logit bias output");
  }
  size_t old = 0;
  c->use_stream(stream);
  rc = c->append(layer, k, v, dtype, tokens, &old, stream);
  if (rc) return rc;
  rc = c->dequantize_full(layer, k_out, v_out, dtype, stream);  // pqo.rs:219-221, tq.rs:284-289
  if (rc) return rc;
  if (tq) return c->logit_bias(layer, q, q_dtype, num_q_heads, q_len, logit_bias_out, stream);
  return TQ_OK;
}

extern "C" int tq_cache_attend_prefill(void *cache, int layer, const void *q, int q_dtype, int num_q_heads, int q_len,
                                       int causal, float softmax_scale, void *out, int out_dtype, hipStream_t stream) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  rc = check_q(c, q, q_dtype, num_q_heads);
  if (rc) return rc;
  if (!out || !tqh::valid_dtype(out_dtype) || q_len < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  c->use_stream(stream);
  return c->attend_prefill(layer, q, q_dtype, num_q_heads, q_len, causal, softmax_scale, out, out_dtype, stream);
}

extern "C" size_t tq_cache_seq_len(void *cache, int layer) {
  KvCache *c = as_cache(cache);
  return check_layer(c, layer) ? 0 : c->storage().seq_len(layer);
}

extern "C" size_t tq_cache_capacity(void *cache, int layer) {
  KvCache *c = as_cache(cache);
  return check_layer(c, layer) ? 0 : c->storage().capacity(layer);
}

extern "C" int tq_cache_reset(void *cache) {
  KvCache *c = as_cache(cache);
  if (!c) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null cache");
  // storage.rs:175-186 touches no device: the buffers return to the pool in
  // the order of the cache's last stream, after the work queued on it, and
  // the next append allocates afresh (zeroed) on its own stream
  c->storage().reset(c->last_stream());
  return TQ_OK;
}

extern "C" size_t tq_cache_memory_usage(void *cache) {
  KvCache *c = as_cache(cache);
  return c ? c->storage().memory_usage() : 0;
}

extern "C" int tq_cache_buffers(void *cache, int layer, uint8_t **k_indices, uint16_t **k_scales, uint8_t **v_indices,
                                uint16_t **v_scales, uint8_t **qjl_signs, uint16_t **qjl_norms) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  const LayerBuffers &L = c->storage().layer(layer);
  if (k_indices) *k_indices = L.k_idx;
  if (k_scales) *k_scales = L.k_sc;
  if (v_indices) *v_indices = L.v_idx;
  if (v_scales) *v_scales = L.v_sc;
  if (qjl_signs) *qjl_signs = L.signs;
  if (qjl_norms) *qjl_norms = L.norms;
  return TQ_OK;
}

extern "C" int tq_cache_read_layer(void *cache, int layer, uint8_t *k_indices, uint16_t *k_scales, uint8_t *v_indices,
                                   uint16_t *v_scales, uint8_t *qjl_signs, uint16_t *qjl_norms, hipStream_t stream) {
  KvCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  const LayerBuffers &L = c->storage().layer(layer);
  if (L.seq == 0) return TQ_OK;
  if (!k_indices || !k_scales || !v_indices || !v_scales) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t h = (size_t)c->num_kv_heads();
  c->use_stream(stream);
  auto copy = [&](void *dst, const void *src, size_t rec_bytes) {
    return hipMemcpy2DAsync(dst, L.seq * rec_bytes, src, L.cap * rec_bytes, L.seq * rec_bytes, h,
                            hipMemcpyDeviceToDevice, stream) == hipSuccess;
  };
  const size_t pi = (size_t)c->storage().packed_dim(), ps = (size_t)c->storage().num_blocks() * 2;
  bool ok = copy(k_indices, L.k_idx, pi) && copy(v_indices, L.v_idx, pi) && copy(k_scales, L.k_sc, ps) &&
            copy(v_scales, L.v_sc, ps);
  if (ok && c->mode().qjl) {
    if (qjl_signs) ok = copy(qjl_signs, L.signs, (size_t)c->storage().sign_bytes());
    if (ok && qjl_norms) ok = copy(qjl_norms, L.norms, 2);
  }
  return ok ? TQ_OK : tqh::fail(TQ_ERR_DEVICE, "layer copy failed");
}

// ---- PqoCache / TqCache entry points of the earlier interface ----

extern "C" int tq_pqo_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, void **cache) {
  return tq_cache_create(num_layers, num_kv_heads, head_dim, bits, TQ_NORM_MAXNORM, TQ_OUTLIER_ALL, 0, cache);
}

extern "C" int tq_tq_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, void **cache) {
  return tq_cache_create(num_layers, num_kv_heads, head_dim, bits, TQ_NORM_MAXNORM, 0, 1, cache);
}

extern "C" void tq_pqo_cache_destroy(void *cache) { tq_cache_destroy(cache); }

extern "C" int tq_pqo_cache_prefill(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                                    void *k_out, void *v_out, int *returned_originals, hipStream_t stream) {
  if (tq_cache_is_tq(cache)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "TqCache prefill takes q (tq_cache_prefill)");
  return tq_cache_prefill(cache, layer, k, v, dtype, tokens, nullptr, 0, 0, 0, k_out, v_out, returned_originals,
                          nullptr, stream);
}

extern "C" int tq_pqo_cache_decode(void *cache, int layer, const void *k, const void *v, int kv_dtype, int tokens,
                                   const void *q, int q_dtype, int num_q_heads, float softmax_scale, void *out,
                                   int out_dtype, hipStream_t stream) {
  return tq_cache_decode(cache, layer, k, v, kv_dtype, tokens, q, q_dtype, num_q_heads, softmax_scale, out, out_dtype,
                         stream);
}

extern "C" size_t tq_pqo_cache_seq_len(void *cache, int layer) { return tq_cache_seq_len(cache, layer); }
extern "C" size_t tq_pqo_cache_capacity(void *cache, int layer) { return tq_cache_capacity(cache, layer); }
extern "C" int tq_pqo_cache_reset(void *cache) { return tq_cache_reset(cache); }
extern "C" size_t tq_pqo_cache_memory_usage(void *cache) { return tq_cache_memory_usage(cache); }

extern "C" int tq_pqo_cache_buffers(void *cache, int layer, uint8_t **k_indices, uint16_t **k_scales,
                                    uint8_t **v_indices, uint16_t **v_scales) {
  return tq_cache_buffers(cache, layer, k_indices, k_scales, v_indices, v_scales, nullptr, nullptr);
}

extern "C" int tq_pqo_cache_read_layer(void *cache, int layer, uint8_t *k_indices, uint16_t *k_scales,
                                       uint8_t *v_indices, uint16_t *v_scales, hipStream_t stream) {
  return tq_cache_read_layer(cache, layer, k_indices, k_scales, v_indices, v_scales, nullptr, nullptr, stream);
}
