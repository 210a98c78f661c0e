// tq_cache.cpp -- device-resident PQO KV cache: CompressedStorage
// (reference src/cache/storage.rs:24-203) and PqoCache with the
// CompressedKVCache contract (src/cache/pqo.rs:21-236), behind a C ABI.
//
// Layout per layer: K/V codes [num_kv_heads][capacity][head_dim*bits/8] u8
// and scales [num_kv_heads][capacity][head_dim/32] f16, token t of head h at
// record h * capacity + t, exactly what the fused kernels read with
// kv_head_stride = capacity.  Appends quantize straight into their records
// (one launch per tensor, all heads at once); growth reallocates to
// needed + max(needed / 4, 128) and copies the old rows (storage.rs:108-139).
// Decode runs the single-launch fused attention over the stored records.
#include "tq_common.h"

#include <cstring>
#include <new>
#include <vector>

namespace {

__global__ void set_len_kernel(int *p, int v) {
  if (threadIdx.x == 0) p[0] = v;
}

struct LayerBuffers {
  uint8_t *k_idx = nullptr, *v_idx = nullptr;
  uint16_t *k_sc = nullptr, *v_sc = nullptr;
  size_t cap = 0;   // records per head
  size_t seq = 0;   // stored tokens per head
  bool active = false;
};

class CompressedStorage {
 public:
  CompressedStorage(int num_kv_heads, int head_dim, int bits, int num_layers)
      : heads_(num_kv_heads), head_dim_(head_dim), bits_(bits), layers_(num_layers) {}
  ~CompressedStorage() { release_all(); }

  int packed_dim() const { return head_dim_ * bits_ / 8; }
  int num_blocks() const { return head_dim_ / 32; }
  size_t seq_len(int l) const { return layers_[l].seq; }
  size_t capacity(int l) const { return layers_[l].cap; }
  bool is_active(int l) const { return layers_[l].active && layers_[l].seq > 0; }
  const LayerBuffers &layer(int l) const { return layers_[l]; }

  // storage.rs:108-139
  int ensure_capacity(int l, size_t needed, hipStream_t stream) {
    LayerBuffers &L = layers_[l];
    if (L.cap >= needed) return TQ_OK;
    const size_t grow = needed / 4 > 128 ? needed / 4 : 128;
    const size_t cap = needed + grow;
    const size_t ib = (size_t)heads_ * cap * packed_dim(), sb = (size_t)heads_ * cap * num_blocks() * 2;
    LayerBuffers N;
    N.cap = cap;
    N.seq = L.seq;
    N.active = L.active;
    if (hipMalloc(&N.k_idx, ib) != hipSuccess || hipMalloc(&N.v_idx, ib) != hipSuccess ||
        hipMalloc(&N.k_sc, sb) != hipSuccess || hipMalloc(&N.v_sc, sb) != hipSuccess) {
      free_layer(N);
      return tqh::fail(TQ_ERR_DEVICE, "cache allocation of %zu records per head failed", cap);
    }
    // new capacity starts zeroed, as Tensor::zeros
    if (hipMemsetAsync(N.k_idx, 0, ib, stream) != hipSuccess || hipMemsetAsync(N.v_idx, 0, ib, stream) != hipSuccess ||
        hipMemsetAsync(N.k_sc, 0, sb, stream) != hipSuccess || hipMemsetAsync(N.v_sc, 0, sb, stream) != hipSuccess) {
      free_layer(N);
      return tqh::fail(TQ_ERR_DEVICE, "cache clear failed");
    }
    if (L.seq > 0) {
      const size_t pi = packed_dim(), ps = (size_t)num_blocks() * 2;
      bool ok = hipMemcpy2DAsync(N.k_idx, cap * pi, L.k_idx, L.cap * pi, L.seq * pi, heads_, hipMemcpyDeviceToDevice,
                                 stream) == hipSuccess;
      ok = ok && hipMemcpy2DAsync(N.v_idx, cap * pi, L.v_idx, L.cap * pi, L.seq * pi, heads_,
                                  hipMemcpyDeviceToDevice, stream) == hipSuccess;
      ok = ok && hipMemcpy2DAsync(N.k_sc, cap * ps, L.k_sc, L.cap * ps, L.seq * ps, heads_, hipMemcpyDeviceToDevice,
                                  stream) == hipSuccess;
      ok = ok && hipMemcpy2DAsync(N.v_sc, cap * ps, L.v_sc, L.cap * ps, L.seq * ps, heads_, hipMemcpyDeviceToDevice,
                                  stream) == hipSuccess;
      if (!ok) {
        free_layer(N);
        return tqh::fail(TQ_ERR_DEVICE, "cache growth copy failed");
      }
    }
    // the old buffers may still be read by queued work: wait before freeing
    if (hipStreamSynchronize(stream) != hipSuccess) return tqh::fail(TQ_ERR_DEVICE, "stream synchronize failed");
    free_layer(L);
    L = N;
    return TQ_OK;
  }

  void set_seq(int l, size_t seq) {
    layers_[l].seq = seq;
    layers_[l].active = true;
  }

  // storage.rs:175-186
  void reset() { release_all(); }

  // storage.rs:188-202
  size_t memory_usage() const {
    size_t total = 0;
    for (const LayerBuffers &L : layers_) {
      if (L.seq == 0) continue;
      total += 2 * (size_t)heads_ * L.seq * packed_dim();
      total += 2 * (size_t)heads_ * L.seq * num_blocks() * 2;
    }
    return total;
  }

 private:
  static void free_layer(LayerBuffers &L) {
    if (L.k_idx) (void)hipFree(L.k_idx);
    if (L.v_idx) (void)hipFree(L.v_idx);
    if (L.k_sc) (void)hipFree(L.k_sc);
    if (L.v_sc) (void)hipFree(L.v_sc);
    L = LayerBuffers{};
  }
  void release_all() {
    for (LayerBuffers &L : layers_) free_layer(L);
  }

  int heads_, head_dim_, bits_;
  std::vector<LayerBuffers> layers_;
};

class PqoCache {
 public:
  PqoCache(int num_layers, int num_kv_heads, int head_dim, int bits)
      : layers_(num_layers), heads_(num_kv_heads), head_dim_(head_dim), bits_(bits),
        storage_(num_kv_heads, head_dim, bits, num_layers), lens_(num_layers, nullptr) {}
  ~PqoCache() {
    for (int *p : lens_)
      if (p) (void)hipFree(p);
    if (ws_) (void)hipFree(ws_);
  }

  int layers() const { return layers_; }
  int num_kv_heads() const { return heads_; }
  CompressedStorage &storage() { return storage_; }

  // quantize_and_store (pqo.rs:64-100): k, v [num_kv_heads][tokens][head_dim]
  int append(int l, const void *k, const void *v, int dtype, int tokens, size_t *old_seq, hipStream_t stream) {
    const size_t old = storage_.seq_len(l);
    *old_seq = old;
    if (tokens == 0) return TQ_OK;
    int rc = storage_.ensure_capacity(l, old + tokens, stream);
    if (rc) return rc;
    const LayerBuffers &L = storage_.layer(l);
    rc = tq_pqo_quantize_to_cache(k, dtype, heads_, tokens, L.k_idx, L.k_sc, (long long)L.cap, (long long)old,
                                  head_dim_, bits_, stream);
    if (rc) return rc;
    rc = tq_pqo_quantize_to_cache(v, dtype, heads_, tokens, L.v_idx, L.v_sc, (long long)L.cap, (long long)old,
                                  head_dim_, bits_, stream);
    if (rc) return rc;
    storage_.set_seq(l, old + tokens);
    return TQ_OK;
  }

  // dequantize_full (pqo.rs:176-180, common.rs:16-62): [num_kv_heads][seq][head_dim]
  int dequantize_full(int l, void *k_out, void *v_out, int dtype, hipStream_t stream) {
    const LayerBuffers &L = storage_.layer(l);
    int rc = tq_pqo_dequantize_from_cache(L.k_idx, L.k_sc, (long long)L.cap, heads_, (int)L.seq, k_out, dtype,
                                          head_dim_, bits_, stream);
    if (rc) return rc;
    return tq_pqo_dequantize_from_cache(L.v_idx, L.v_sc, (long long)L.cap, heads_, (int)L.seq, v_out, dtype,
                                        head_dim_, bits_, stream);
  }

  // decode_cuda (pqo.rs:106-174) as one fused launch over the stored records
  int attend(int l, const void *q, int q_dtype, int num_q_heads, float scale, void *out, int out_dtype,
             hipStream_t stream) {
    const LayerBuffers &L = storage_.layer(l);
    if (!lens_[l] && hipMalloc(&lens_[l], sizeof(int)) != hipSuccess)
      return tqh::fail(TQ_ERR_DEVICE, "length buffer allocation failed");
    hipLaunchKernelGGL(set_len_kernel, dim3(1), dim3(64), 0, stream, lens_[l], (int)L.seq);
    int rc = tqh::check_launch("set_len_kernel");
    if (rc) return rc;
    const size_t need = tq_attention_workspace_size(1, num_q_heads, heads_, head_dim_, (int)L.cap);
    if (need == 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid attention shape");
    if (need > ws_bytes_) {
      if (hipStreamSynchronize(stream) != hipSuccess) return tqh::fail(TQ_ERR_DEVICE, "stream synchronize failed");
      if (ws_) (void)hipFree(ws_);
      ws_ = nullptr;
      ws_bytes_ = 0;
      if (hipMalloc(&ws_, need) != hipSuccess) return tqh::fail(TQ_ERR_DEVICE, "workspace allocation failed");
      ws_bytes_ = need;
      rc = tq_attention_workspace_init(ws_, ws_bytes_, 1, num_q_heads, heads_, head_dim_, (int)L.cap, stream);
      if (rc) return rc;
    }
    return tq_pqo_decode_attention(q, q_dtype, L.k_idx, L.k_sc, L.v_idx, L.v_sc, lens_[l], 1, num_q_heads, heads_,
                                   head_dim_, bits_, (int)L.cap, (long long)L.cap, 0, scale, out, out_dtype, ws_,
                                   ws_bytes_, stream);
  }

 private:
  int layers_, heads_, head_dim_, bits_;
  CompressedStorage storage_;
  std::vector<int *> lens_;
  void *ws_ = nullptr;
  size_t ws_bytes_ = 0;
};

PqoCache *as_cache(void *h) { return static_cast<PqoCache *>(h); }

int check_layer(PqoCache *c, int layer) {
  if (!c) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null cache");
  if (layer < 0 || layer >= c->layers())
    return tqh::fail(TQ_ERR_LAYER_OUT_OF_RANGE, "layer %d out of range (num_layers %d)", layer, c->layers());
  return TQ_OK;
}

}  // namespace

extern "C" int tq_pqo_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, void **cache) {
  if (!cache) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null handle pointer");
  *cache = nullptr;
  if (bits != 3 && bits != 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bits=%d, expected 3 or 4", bits);
  if (head_dim <= 0 || head_dim % 32 != 0)  // PqoCache::new, pqo.rs:30-39
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT,
                     "head_dim (%d) must be divisible by QUANT_BLOCK_SIZE (32). Models with head_dim=%d are not "
                     "supported by TurboQuant compression.", head_dim, head_dim);
  if (num_layers <= 0 || num_kv_heads <= 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "empty cache shape");
  PqoCache *c = new (std::nothrow) PqoCache(num_layers, num_kv_heads, head_dim, bits);
  if (!c) return tqh::fail(TQ_ERR_DEVICE, "out of host memory");
  *cache = c;
  return TQ_OK;
}

extern "C" void tq_pqo_cache_destroy(void *cache) { delete as_cache(cache); }

extern "C" int tq_pqo_cache_prefill(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                                    void *k_out, void *v_out, int *returned_originals, hipStream_t stream) {
  PqoCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  if (!tqh::valid_dtype(dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (tokens < 0 || !returned_originals) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  size_t old = 0;
  rc = c->append(layer, k, v, dtype, tokens, &old, stream);
  if (rc) return rc;
  // pqo.rs:184-200: the first prefill returns the caller's own K/V
  *returned_originals = old == 0 ? 1 : 0;
  if (old == 0) return TQ_OK;
  if (!k_out || !v_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null output for the dequantized cache");
  return c->dequantize_full(layer, k_out, v_out, dtype, stream);
}

extern "C" int tq_pqo_cache_decode(void *cache, int layer, const void *k, const void *v, int kv_dtype, int tokens,
                                   const void *q, int q_dtype, int num_q_heads, float softmax_scale, void *out,
                                   int out_dtype, hipStream_t stream) {
  PqoCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  if (!tqh::valid_dtype(kv_dtype) || !tqh::valid_dtype(q_dtype) || !tqh::valid_dtype(out_dtype))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (tokens < 0 || !q || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid arguments");
  size_t old = 0;
  rc = c->append(layer, k, v, kv_dtype, tokens, &old, stream);
  if (rc) return rc;
  if (!c->storage().is_active(layer)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "decode over an empty cache");
  return c->attend(layer, q, q_dtype, num_q_heads, softmax_scale, out, out_dtype, stream);
}

extern "C" size_t tq_pqo_cache_seq_len(void *cache, int layer) {
  PqoCache *c = as_cache(cache);
  return check_layer(c, layer) ? 0 : c->storage().seq_len(layer);
}

extern "C" size_t tq_pqo_cache_capacity(void *cache, int layer) {
  PqoCache *c = as_cache(cache);
  return check_layer(c, layer) ? 0 : c->storage().capacity(layer);
}

extern "C" int tq_pqo_cache_reset(void *cache) {
  PqoCache *c = as_cache(cache);
  if (!c) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null cache");
  if (hipDeviceSynchronize() != hipSuccess) return tqh::fail(TQ_ERR_DEVICE, "device synchronize failed");
  c->storage().reset();
  return TQ_OK;
}

extern "C" size_t tq_pqo_cache_memory_usage(void *cache) {
  PqoCache *c = as_cache(cache);
  return c ? c->storage().memory_usage() : 0;
}

extern "C" int tq_pqo_cache_buffers(void *cache, int layer, uint8_t **k_indices, uint16_t **k_scales,
                                    uint8_t **v_indices, uint16_t **v_scales) {
  PqoCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  const LayerBuffers &L = c->storage().layer(layer);
  if (k_indices) *k_indices = L.k_idx;
  if (k_scales) *k_scales = L.k_sc;
  if (v_indices) *v_indices = L.v_idx;
  if (v_scales) *v_scales = L.v_sc;
  return TQ_OK;
}

extern "C" int tq_pqo_cache_read_layer(void *cache, int layer, uint8_t *k_indices, uint16_t *k_scales,
                                       uint8_t *v_indices, uint16_t *v_scales, hipStream_t stream) {
  PqoCache *c = as_cache(cache);
  int rc = check_layer(c, layer);
  if (rc) return rc;
  const LayerBuffers &L = c->storage().layer(layer);
  if (L.seq == 0) return TQ_OK;
  if (!k_indices || !k_scales || !v_indices || !v_scales) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t pi = (size_t)c->storage().packed_dim(), ps = (size_t)c->storage().num_blocks() * 2;
  const size_t h = (size_t)c->num_kv_heads();
  bool ok = hipMemcpy2DAsync(k_indices, L.seq * pi, L.k_idx, L.cap * pi, L.seq * pi, h, hipMemcpyDeviceToDevice,
                             stream) == hipSuccess;
  ok = ok && hipMemcpy2DAsync(v_indices, L.seq * pi, L.v_idx, L.cap * pi, L.seq * pi, h, hipMemcpyDeviceToDevice,
                              stream) == hipSuccess;
  ok = ok && hipMemcpy2DAsync(k_scales, L.seq * ps, L.k_sc, L.cap * ps, L.seq * ps, h, hipMemcpyDeviceToDevice,
                              stream) == hipSuccess;
  ok = ok && hipMemcpy2DAsync(v_scales, L.seq * ps, L.v_sc, L.cap * ps, L.seq * ps, h, hipMemcpyDeviceToDevice,
                              stream) == hipSuccess;
  return ok ? TQ_OK : tqh::fail(TQ_ERR_DEVICE, "layer copy failed");
}
