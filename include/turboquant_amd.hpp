// turboquant_amd.hpp -- C++17 host API over the C ABI (turboquant_amd.h),
// mirroring the reference crate's public Rust types and functions so that
// code written against them ports line by line:
//
//   TurboQuantConfig         packed/mod.rs:92-139
//   PackedBlock              packed/mod.rs:149-233 (LSB-first bitstream)
//   quantize_vec / dequantize_vec / dequantize_rotated   quantize.rs:142-316
//   QjlBlock, quantize_with_qjl                          qjl.rs:111-134, 355-377
//   precompute_query_projections, EstimationContext,
//   estimate_inner_product(_single)                      qjl.rs:488-627
//   QuantizedKVCache                                     attention.rs:45-700
//   CacheConfig, CompressedKVCache, PqoCache, TqCache    cache/config.rs, pqo.rs, tq.rs
//
// Errors are thrown as tq::Error carrying the TurboQuantError kind
// (error.rs:5-29).  Host-side values (slices, Vec<f32>) cross as std::vector;
// the per-vector functions stage their data through device memory and run
// the batched gfx950 kernels, so they are conveniences, not the hot path:
// batch work belongs on the device entry points of turboquant_amd.h.  The
// cache classes keep all data in device memory and take device pointers.
#ifndef TURBOQUANT_AMD_HPP
#define TURBOQUANT_AMD_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "turboquant_amd.h"

namespace tq {

// ---- errors (error.rs:5-29) ----
enum class ErrorKind : int {
  InvalidDimension = TQ_ERR_INVALID_DIMENSION,
  UnsupportedBits = TQ_ERR_UNSUPPORTED_BITS,
  DimensionMismatch = TQ_ERR_DIMENSION_MISMATCH,
  LayerOutOfRange = TQ_ERR_LAYER_OUT_OF_RANGE,
  RangeOutOfBounds = TQ_ERR_RANGE_OUT_OF_BOUNDS,
  InvalidArgument = TQ_ERR_INVALID_ARGUMENT,
  Device = TQ_ERR_DEVICE,
};

class Error : public std::runtime_error {
 public:
  Error(ErrorKind kind, const std::string &msg) : std::runtime_error(msg), kind_(kind) {}
  ErrorKind kind() const { return kind_; }

 private:
  ErrorKind kind_;
};

inline void check(int rc) {
  if (rc != TQ_OK) throw Error(static_cast<ErrorKind>(rc), tq_last_error());
}
inline void require(bool cond, ErrorKind kind, const std::string &msg) {
  if (!cond) throw Error(kind, msg);
}
inline void check_values_match(size_t actual, size_t expected) {
  require(actual == expected, ErrorKind::DimensionMismatch,
          "expected vector of length " + std::to_string(expected) + ", got " + std::to_string(actual));
}

namespace detail {
// Owned device allocation (staging for the per-vector conveniences and the
// QuantizedKVCache's growable arrays).
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t bytes) { resize(bytes); }
  ~DeviceBuffer() { release(); }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr, o.n_ = 0; }
  DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
    if (this != &o) {
      release();
      p_ = o.p_, n_ = o.n_;
      o.p_ = nullptr, o.n_ = 0;
    }
    return *this;
  }
  void resize(size_t bytes) {
    release();
    if (bytes && hipMalloc(&p_, bytes) != hipSuccess) throw Error(ErrorKind::Device, "device allocation failed");
    n_ = bytes;
  }
  // grows to at least `bytes`, keeping the first `keep` bytes
  void grow(size_t bytes, size_t keep, hipStream_t s) {
    if (bytes <= n_) return;
    DeviceBuffer nb(bytes);
    if (keep) copy_d2d(nb.p_, p_, keep, s);
    sync(s);
    *this = std::move(nb);
  }
  void *get() const { return p_; }
  template <typename T>
  T *as() const { return static_cast<T *>(p_); }
  size_t size() const { return n_; }

  static void copy_d2d(void *dst, const void *src, size_t n, hipStream_t s) {
    if (n && hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, s) != hipSuccess)
      throw Error(ErrorKind::Device, "device copy failed");
  }
  static void sync(hipStream_t s) {
    if (hipStreamSynchronize(s) != hipSuccess) throw Error(ErrorKind::Device, "stream synchronize failed");
  }

 private:
  void release() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = 0;
  }
  void *p_ = nullptr;
  size_t n_ = 0;
};

inline void to_device(void *dst, const void *src, size_t n, hipStream_t s) {
  if (n && hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s) != hipSuccess)
    throw Error(ErrorKind::Device, "host to device copy failed");
}
inline void to_host(void *dst, const void *src, size_t n, hipStream_t s) {
  if (n && hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s) != hipSuccess)
    throw Error(ErrorKind::Device, "device to host copy failed");
  DeviceBuffer::sync(s);
}
}  // namespace detail

// ---- TurboQuantConfig (packed/mod.rs:92-139) ----
struct TurboQuantConfig {
  uint8_t bits = 3;
  size_t dim = 0;
  uint64_t rotation_seed = 0;

  // TurboQuantConfig::new: bits in {2, 3, 4}, dim a non-zero power of two
  static TurboQuantConfig create(uint8_t bits, size_t dim) {
    require(bits == 2 || bits == 3 || bits == 4, ErrorKind::UnsupportedBits,
            "unsupported bit width " + std::to_string(bits) + ", expected 2, 3, or 4");
    require(dim > 0 && (dim & (dim - 1)) == 0, ErrorKind::InvalidDimension,
            "dimension " + std::to_string(dim) + " is not a power of two");
    TurboQuantConfig c;
    c.bits = bits;
    c.dim = dim;
    return c;
  }
  TurboQuantConfig with_seed(uint64_t seed) const {
    TurboQuantConfig c = *this;
    c.rotation_seed = seed;
    return c;
  }
};

// ---- PackedBlock (packed/mod.rs:149-233) ----
// Index i occupies bits [i*bits, i*bits + bits) of a little-endian
// bitstream; the byte length follows the reference packers' zero-padded
// tails (4 indices per byte for 2-bit, 8 per 3 bytes for 3-bit, 2 per byte
// for 4-bit, packed/indices.rs).
inline size_t packed_len(uint8_t bits, size_t count) {
  switch (bits) {
    case 2: return (count + 3) / 4;
    case 3: return (count + 7) / 8 * 3;
    default: return (count + 1) / 2;
  }
}

struct PackedBlock {
  uint8_t bits = 0;
  uint16_t scale = 0;  // f16 bits (the vector's L2 norm)
  std::vector<uint8_t> packed_indices;

  // PackedBlock::new: packs host indices
  static PackedBlock create(uint8_t bits, uint16_t scale, const std::vector<uint8_t> &indices) {
    require(bits >= 2 && bits <= 4, ErrorKind::UnsupportedBits, "bits validated to be 2, 3, or 4");
    PackedBlock b;
    b.bits = bits;
    b.scale = scale;
    b.packed_indices.assign(packed_len(bits, indices.size()), 0);
    const uint32_t mask = (1u << bits) - 1u;
    for (size_t i = 0; i < indices.size(); i++) {
      const size_t pos = i * bits;
      const uint32_t v = (uint32_t)(indices[i] & mask) << (pos & 7);
      b.packed_indices[pos >> 3] |= (uint8_t)(v & 0xff);
      if ((pos & 7) + bits > 8) b.packed_indices[(pos >> 3) + 1] |= (uint8_t)(v >> 8);
    }
    return b;
  }
  // PackedBlock::from_raw
  static PackedBlock from_raw(uint8_t bits, uint16_t scale, std::vector<uint8_t> packed) {
    PackedBlock b;
    b.bits = bits;
    b.scale = scale;
    b.packed_indices = std::move(packed);
    return b;
  }
  size_t size_bytes() const { return 2 + packed_indices.size(); }
  void unpack_into(size_t count, std::vector<uint8_t> &buf) const {
    buf.assign(count, 0);
    const uint32_t mask = (1u << bits) - 1u;
    for (size_t i = 0; i < count; i++) {
      const size_t pos = i * bits, byte = pos >> 3;
      uint32_t w = packed_indices[byte];
      if (byte + 1 < packed_indices.size()) w |= (uint32_t)packed_indices[byte + 1] << 8;
      buf[i] = (uint8_t)((w >> (pos & 7)) & mask);
    }
  }
  std::vector<uint8_t> unpack(size_t count) const {
    std::vector<uint8_t> out;
    unpack_into(count, out);
    return out;
  }
};

// ---- quantize_vec / dequantize_vec / dequantize_rotated (quantize.rs) ----
inline PackedBlock quantize_vec(const TurboQuantConfig &config, const std::vector<float> &data,
                                hipStream_t stream = nullptr) {
  check_values_match(data.size(), config.dim);
  const size_t pb = config.dim * config.bits / 8;
  detail::DeviceBuffer x(data.size() * 4), p(pb), s(2);
  detail::to_device(x.get(), data.data(), data.size() * 4, stream);
  check(tq_quantize_vec_batch(x.as<float>(), p.as<uint8_t>(), s.as<uint16_t>(), 1, config.bits, (int)config.dim,
                              config.rotation_seed, stream));
  PackedBlock b;
  b.bits = config.bits;
  b.packed_indices.resize(pb);
  detail::to_host(b.packed_indices.data(), p.get(), pb, stream);
  detail::to_host(&b.scale, s.get(), 2, stream);
  return b;
}

inline std::vector<float> dequantize_vec(const TurboQuantConfig &config, const PackedBlock &block,
                                         hipStream_t stream = nullptr) {
  detail::DeviceBuffer p(block.packed_indices.size()), s(2), o(config.dim * 4);
  detail::to_device(p.get(), block.packed_indices.data(), block.packed_indices.size(), stream);
  detail::to_device(s.get(), &block.scale, 2, stream);
  check(tq_dequantize_vec_batch(p.as<uint8_t>(), s.as<uint16_t>(), o.as<float>(), 1, block.bits, (int)config.dim,
                                config.rotation_seed, stream));
  std::vector<float> out(config.dim);
  detail::to_host(out.data(), o.get(), config.dim * 4, stream);
  return out;
}

inline std::vector<float> dequantize_rotated(const TurboQuantConfig &config, const PackedBlock &block,
                                             hipStream_t stream = nullptr) {
  detail::DeviceBuffer p(block.packed_indices.size()), s(2), o(config.dim * 4);
  detail::to_device(p.get(), block.packed_indices.data(), block.packed_indices.size(), stream);
  detail::to_device(s.get(), &block.scale, 2, stream);
  check(tq_dequantize_rotated_batch(p.as<uint8_t>(), s.as<uint16_t>(), o.as<float>(), 1, block.bits,
                                    (int)config.dim, stream));
  std::vector<float> out(config.dim);
  detail::to_host(out.data(), o.get(), config.dim * 4, stream);
  return out;
}

// ---- QJL (qjl.rs) ----
struct QjlBlock {
  PackedBlock polar_block;            // (bits - 1)-bit PolarQuant block
  std::vector<uint8_t> qjl_signs;     // sign(R r) packed LSB first
  uint16_t residual_norm = 0;         // f16 bits
  static QjlBlock from_parts(PackedBlock polar, std::vector<uint8_t> signs, uint16_t norm) {
    QjlBlock b;
    b.polar_block = std::move(polar);
    b.qjl_signs = std::move(signs);
    b.residual_norm = norm;
    return b;
  }
  size_t size_bytes() const { return polar_block.size_bytes() + qjl_signs.size() + 2; }  // attention.rs:78-80
};

inline void validate_qjl_config(uint8_t bits) {
  require(bits == 3 || bits == 4, ErrorKind::UnsupportedBits,
          "unsupported bit width " + std::to_string(bits) + ", expected 2, 3, or 4");
}

inline QjlBlock quantize_with_qjl(const TurboQuantConfig &config, const std::vector<float> &data, uint64_t qjl_seed,
                                  hipStream_t stream = nullptr) {
  validate_qjl_config(config.bits);
  check_values_match(data.size(), config.dim);
  const size_t pb = config.dim * (config.bits - 1) / 8, sb = config.dim / 8;
  detail::DeviceBuffer x(data.size() * 4), p(pb), s(2), g(sb), n(2);
  detail::to_device(x.get(), data.data(), data.size() * 4, stream);
  check(tq_qjl_quantize_batch(x.as<float>(), p.as<uint8_t>(), s.as<uint16_t>(), g.as<uint8_t>(), n.as<uint16_t>(), 1,
                              config.bits, (int)config.dim, config.rotation_seed, qjl_seed, stream));
  QjlBlock b;
  b.polar_block.bits = (uint8_t)(config.bits - 1);
  b.polar_block.packed_indices.resize(pb);
  b.qjl_signs.resize(sb);
  detail::to_host(b.polar_block.packed_indices.data(), p.get(), pb, stream);
  detail::to_host(&b.polar_block.scale, s.get(), 2, stream);
  detail::to_host(b.qjl_signs.data(), g.get(), sb, stream);
  detail::to_host(&b.residual_norm, n.get(), 2, stream);
  return b;
}

// precompute_query_projections (qjl.rs:488-492): R q
inline std::vector<float> precompute_query_projections(const std::vector<float> &query, size_t dim, uint64_t qjl_seed,
                                                       hipStream_t stream = nullptr) {
  check_values_match(query.size(), dim);
  detail::DeviceBuffer q(dim * 4), ctx(2 * dim * 4);
  detail::to_device(q.get(), query.data(), dim * 4, stream);
  check(tq_qjl_query_context(q.as<float>(), ctx.as<float>(), 1, (int)dim, 0, qjl_seed, stream));
  std::vector<float> out(dim);
  detail::to_host(out.data(), ctx.as<float>() + dim, dim * 4, stream);
  return out;
}

// EstimationContext (qjl.rs:561-572): what is fetched once per batch of
// keys -- here the query's device context (rotated query and R q).
struct EstimationContext {
  TurboQuantConfig polar_config;
  size_t dim = 0;
  uint64_t qjl_seed = 0;
  detail::DeviceBuffer ctx;  // [2 dim] f32: rotated query, then R q

  EstimationContext(const TurboQuantConfig &config, const std::vector<float> &query, uint64_t qjl_seed_,
                    hipStream_t stream = nullptr)
      : dim(config.dim), qjl_seed(qjl_seed_) {
    validate_qjl_config(config.bits);
    check_values_match(query.size(), config.dim);
    polar_config = TurboQuantConfig::create((uint8_t)(config.bits - 1), config.dim).with_seed(config.rotation_seed);
    detail::DeviceBuffer q(dim * 4);
    ctx.resize(2 * dim * 4);
    detail::to_device(q.get(), query.data(), dim * 4, stream);
    check(tq_qjl_query_context(q.as<float>(), ctx.as<float>(), 1, (int)dim, config.rotation_seed, qjl_seed, stream));
    detail::DeviceBuffer::sync(stream);
  }

  // estimate_inner_product_with_codebook (qjl.rs:585-606) over many keys:
  // <q, x_mse> + |r| sqrt(pi/2)/sqrt(d) sum_j rq_j sgn_j for each block
  std::vector<float> estimate(const std::vector<QjlBlock> &keys, hipStream_t stream = nullptr) const {
    const size_t n = keys.size();
    if (n == 0) return {};
    const size_t pb = dim * polar_config.bits / 8, sb = dim / 8;
    std::vector<uint8_t> hp(n * pb), hg(n * sb);
    std::vector<uint16_t> hs(n), hn(n);
    for (size_t i = 0; i < n; i++) {
      check_values_match(keys[i].polar_block.packed_indices.size(), pb);
      std::memcpy(hp.data() + i * pb, keys[i].polar_block.packed_indices.data(), pb);
      std::memcpy(hg.data() + i * sb, keys[i].qjl_signs.data(), sb);
      hs[i] = keys[i].polar_block.scale;
      hn[i] = keys[i].residual_norm;
    }
    detail::DeviceBuffer p(n * pb), g(n * sb), s(n * 2), nm(n * 2), o(n * 4);
    detail::to_device(p.get(), hp.data(), n * pb, stream);
    detail::to_device(g.get(), hg.data(), n * sb, stream);
    detail::to_device(s.get(), hs.data(), n * 2, stream);
    detail::to_device(nm.get(), hn.data(), n * 2, stream);
    check(tq_qjl_scores(ctx.as<float>(), 1, p.as<uint8_t>(), s.as<uint16_t>(), g.as<uint8_t>(), nm.as<uint16_t>(), n,
                        polar_config.bits, (int)dim, polar_config.rotation_seed, o.as<float>(), stream));
    std::vector<float> out(n);
    detail::to_host(out.data(), o.get(), n * 4, stream);
    return out;
  }
};

// estimate_inner_product_single (qjl.rs:619-627)
inline float estimate_inner_product_single(const std::vector<float> &query, const QjlBlock &block,
                                           const TurboQuantConfig &config, uint64_t qjl_seed,
                                           hipStream_t stream = nullptr) {
  EstimationContext ctx(config, query, qjl_seed, stream);
  return ctx.estimate({block}, stream)[0];
}

// ---- QuantizedKVCache (attention.rs:45-700): QJL blocks per layer, kept in
// device memory as flat arrays ----
class QuantizedKVCache {
 public:
  QuantizedKVCache(const TurboQuantConfig &config, size_t num_layers, uint64_t qjl_seed)
      : config_(config), qjl_seed_(qjl_seed), keys_(num_layers), values_(num_layers) {}

  size_t num_layers() const { return keys_.size(); }
  const TurboQuantConfig &config() const { return config_; }
  uint64_t qjl_seed() const { return qjl_seed_; }
  size_t entry_count(size_t layer) const { return keys_.at(layer).count; }

  void push(size_t layer, const std::vector<float> &key, const std::vector<float> &value,
            hipStream_t stream = nullptr) {
    push_batch(layer, {key}, {value}, stream);
  }

  // push_batch (attention.rs:274-301)
  void push_batch(size_t layer, const std::vector<std::vector<float>> &keys,
                  const std::vector<std::vector<float>> &values, hipStream_t stream = nullptr) {
    check_layer(layer);
    check_values_match(keys.size(), values.size());
    for (size_t i = 0; i < keys.size(); i++) {
      check_values_match(keys[i].size(), config_.dim);
      check_values_match(values[i].size(), config_.dim);
    }
    validate_qjl_config(config_.bits);
    append(keys_[layer], keys, stream);
    append(values_[layer], values, stream);
  }

  // attention_scores (attention.rs:319-353)
  std::vector<float> attention_scores(size_t layer, const std::vector<float> &query,
                                      hipStream_t stream = nullptr) const {
    check_layer(layer);
    const Blocks &k = keys_[layer];
    if (k.count == 0) return {};
    EstimationContext ctx(config_, query, qjl_seed_, stream);
    detail::DeviceBuffer o(k.count * 4);
    check(tq_qjl_scores(ctx.ctx.as<float>(), 1, k.polar.as<uint8_t>(), k.scales.as<uint16_t>(), k.signs.as<uint8_t>(),
                        k.norms.as<uint16_t>(), k.count, config_.bits - 1, (int)config_.dim, config_.rotation_seed,
                        o.as<float>(), stream));
    std::vector<float> out(k.count);
    detail::to_host(out.data(), o.get(), k.count * 4, stream);
    return out;
  }

  // weighted_values (attention.rs:371-408)
  std::vector<float> weighted_values(size_t layer, const std::vector<float> &weights,
                                     hipStream_t stream = nullptr) const {
    check_layer(layer);
    const Blocks &v = values_[layer];
    check_values_match(weights.size(), keys_[layer].count);
    std::vector<float> out(config_.dim, 0.0f);
    if (v.count == 0) return out;
    detail::DeviceBuffer w(v.count * 4), o(config_.dim * 4);
    detail::to_device(w.get(), weights.data(), v.count * 4, stream);
    const size_t ws = tq_qjl_weighted_values_workspace_size(1, v.count, (int)config_.dim);
    detail::DeviceBuffer scratch(ws ? ws : 4);
    check(tq_qjl_weighted_values(v.polar.as<uint8_t>(), v.scales.as<uint16_t>(), v.count, w.as<float>(), 1,
                                 config_.bits - 1, (int)config_.dim, config_.rotation_seed, o.as<float>(),
                                 scratch.get(), scratch.size(), stream));
    detail::to_host(out.data(), o.get(), config_.dim * 4, stream);
    return out;
  }

  // memory_usage / fp16_equivalent_memory (attention.rs:414-441)
  size_t memory_usage() const {
    size_t total = 0;
    const size_t per = 2 + config_.dim * (config_.bits - 1) / 8 + config_.dim / 8 + 2;
    for (size_t l = 0; l < keys_.size(); l++) total += (keys_[l].count + values_[l].count) * per;
    return total;
  }
  size_t fp16_equivalent_memory() const {
    size_t n = 0;
    for (const Blocks &b : keys_) n += b.count;
    return n * config_.dim * 2 * 2;
  }

  // key_block (attention.rs:456-458); throws RangeOutOfBounds past the end
  QjlBlock key_block(size_t layer, size_t index, hipStream_t stream = nullptr) const {
    check_layer(layer);
    return read_block(keys_[layer], index, stream);
  }

  std::vector<std::vector<float>> dequantize_all_keys(size_t layer, hipStream_t stream = nullptr) const {
    check_layer(layer);
    return dequantize_range(keys_[layer], 0, keys_[layer].count, stream);
  }
  std::vector<std::vector<float>> dequantize_all_values(size_t layer, hipStream_t stream = nullptr) const {
    check_layer(layer);
    return dequantize_range(values_[layer], 0, values_[layer].count, stream);
  }
  std::vector<std::vector<float>> dequantize_keys_range(size_t layer, size_t start, size_t end,
                                                        hipStream_t stream = nullptr) const {
    check_layer(layer);
    check_range(start, end, keys_[layer].count);
    return dequantize_range(keys_[layer], start, end, stream);
  }
  std::vector<std::vector<float>> dequantize_values_range(size_t layer, size_t start, size_t end,
                                                          hipStream_t stream = nullptr) const {
    check_layer(layer);
    check_range(start, end, values_[layer].count);
    return dequantize_range(values_[layer], start, end, stream);
  }

 private:
  struct Blocks {
    detail::DeviceBuffer polar, scales, signs, norms;
    size_t count = 0, cap = 0;
  };

  size_t polar_bytes() const { return config_.dim * (config_.bits - 1) / 8; }
  void check_layer(size_t layer) const {
    require(layer < keys_.size(), ErrorKind::LayerOutOfRange,
            "layer index " + std::to_string(layer) + " out of range (num_layers = " + std::to_string(keys_.size()) +
                ")");
  }
  static void check_range(size_t start, size_t end, size_t n) {
    require(start <= end && end <= n, ErrorKind::RangeOutOfBounds,
            "range [" + std::to_string(start) + ".." + std::to_string(end) + ") out of bounds for entry_count = " +
                std::to_string(n));
  }
  void reserve(Blocks &b, size_t need, hipStream_t stream) {
    if (need <= b.cap) return;
    size_t cap = b.cap ? b.cap : 64;
    while (cap < need) cap *= 2;
    const size_t pb = polar_bytes(), sb = config_.dim / 8;
    b.polar.grow(cap * pb, b.count * pb, stream);
    b.scales.grow(cap * 2, b.count * 2, stream);
    b.signs.grow(cap * sb, b.count * sb, stream);
    b.norms.grow(cap * 2, b.count * 2, stream);
    b.cap = cap;
  }
  void append(Blocks &b, const std::vector<std::vector<float>> &rows, hipStream_t stream) {
    const size_t n = rows.size();
    if (n == 0) return;
    reserve(b, b.count + n, stream);
    std::vector<float> flat(n * config_.dim);
    for (size_t i = 0; i < n; i++) std::memcpy(flat.data() + i * config_.dim, rows[i].data(), config_.dim * 4);
    detail::DeviceBuffer x(flat.size() * 4);
    detail::to_device(x.get(), flat.data(), flat.size() * 4, stream);
    const size_t pb = polar_bytes(), sb = config_.dim / 8;
    check(tq_qjl_quantize_batch(x.as<float>(), b.polar.as<uint8_t>() + b.count * pb, b.scales.as<uint16_t>() + b.count,
                                b.signs.as<uint8_t>() + b.count * sb, b.norms.as<uint16_t>() + b.count, n, config_.bits,
                                (int)config_.dim, config_.rotation_seed, qjl_seed_, stream));
    detail::DeviceBuffer::sync(stream);
    b.count += n;
  }
  QjlBlock read_block(const Blocks &b, size_t i, hipStream_t stream) const {
    check_range(i, i + 1, b.count);
    const size_t pb = polar_bytes(), sb = config_.dim / 8;
    QjlBlock q;
    q.polar_block.bits = (uint8_t)(config_.bits - 1);
    q.polar_block.packed_indices.resize(pb);
    q.qjl_signs.resize(sb);
    detail::to_host(q.polar_block.packed_indices.data(), b.polar.as<uint8_t>() + i * pb, pb, stream);
    detail::to_host(&q.polar_block.scale, b.scales.as<uint16_t>() + i, 2, stream);
    detail::to_host(q.qjl_signs.data(), b.signs.as<uint8_t>() + i * sb, sb, stream);
    detail::to_host(&q.residual_norm, b.norms.as<uint16_t>() + i, 2, stream);
    return q;
  }
  std::vector<std::vector<float>> dequantize_range(const Blocks &b, size_t start, size_t end,
                                                   hipStream_t stream) const {
    const size_t n = end - start;
    std::vector<std::vector<float>> out;
    if (n == 0) return out;
    detail::DeviceBuffer o(n * config_.dim * 4);
    check(tq_dequantize_vec_batch(b.polar.as<uint8_t>() + start * polar_bytes(), b.scales.as<uint16_t>() + start,
                                  o.as<float>(), n, config_.bits - 1, (int)config_.dim, config_.rotation_seed, stream));
    std::vector<float> flat(n * config_.dim);
    detail::to_host(flat.data(), o.get(), flat.size() * 4, stream);
    out.resize(n);
    for (size_t i = 0; i < n; i++) out[i].assign(flat.begin() + i * config_.dim, flat.begin() + (i + 1) * config_.dim);
    return out;
  }

  TurboQuantConfig config_;
  uint64_t qjl_seed_;
  std::vector<Blocks> keys_, values_;
};

// ---- compressed KV caches (cache/config.rs, pqo.rs, tq.rs) ----
enum class QuantNormMode : int { MaxNorm = TQ_NORM_MAXNORM, L2Norm = TQ_NORM_L2NORM };
constexpr size_t kOutlierAll = TQ_OUTLIER_ALL;  // usize::MAX

struct CacheConfig {
  uint8_t bits = 3;
  size_t head_dim = 128;
  size_t num_kv_heads = 8;
  size_t num_layers = 1;
  QuantNormMode norm_mode = QuantNormMode::MaxNorm;
  size_t outlier_blocks = kOutlierAll;
  bool qjl_enabled() const { return outlier_blocks == 0; }
  size_t num_blocks() const { return head_dim / 32; }
  size_t packed_dim() const { return head_dim * bits / 8; }
};

struct AttendConfig {  // cache_pqo_tests.rs:130-133
  float softmax_scale;
  size_t n_kv_groups;
};

// Element type of device tensors crossing these calls.
enum class DType : int { F32 = TQ_DTYPE_F32, BF16 = TQ_DTYPE_BF16, F16 = TQ_DTYPE_F16 };

// Device views standing in for candle tensors: k, v [num_kv_heads][tokens]
// [head_dim]; q [num_q_heads][q_len][head_dim].
struct KvInput {
  const void *k, *v;
  DType dtype;
  int tokens;
};
struct QueryInput {
  const void *q;
  DType dtype;
  int num_q_heads, q_len;
};
// DequantResult (common.rs:115-121) as caller-owned device outputs: k, v
// [num_kv_heads][seq_len][head_dim] (written unless the first prefill hands
// back the inputs: returned_originals), logit_bias [num_q_heads][q_len]
// [seq_len] for a TqCache.
struct DequantOutput {
  void *k = nullptr, *v = nullptr, *logit_bias = nullptr;
  bool returned_originals = false;
};

// The CompressedKVCache trait (mistralrs-kv-cache; methods as used by
// pqo.rs:183-236 and tq.rs:256-324).
class CompressedKVCache {
 public:
  virtual ~CompressedKVCache() = default;
  virtual void prefill(size_t layer, const KvInput &kv, const QueryInput &q, DequantOutput &out,
                       hipStream_t stream = nullptr) = 0;
  // DecodeOutput::Fused: out [num_q_heads][head_dim] in out_dtype
  virtual void decode(size_t layer, const KvInput &kv, const QueryInput &q, const AttendConfig &cfg, void *out,
                      DType out_dtype, hipStream_t stream = nullptr) = 0;
  virtual size_t seq_len(size_t layer) const = 0;
  virtual void reset() = 0;
  virtual size_t memory_usage() const = 0;
};

namespace detail {
class DeviceCache : public CompressedKVCache {
 public:
  DeviceCache(const CacheConfig &c, bool qjl) : config_(c) {
    check(tq_cache_create((int)c.num_layers, (int)c.num_kv_heads, (int)c.head_dim, c.bits, (int)c.norm_mode,
                          c.outlier_blocks, qjl ? 1 : 0, &h_));
  }
  ~DeviceCache() override {
    if (h_) {
      (void)hipDeviceSynchronize();
      tq_cache_destroy(h_);
    }
  }
  DeviceCache(const DeviceCache &) = delete;
  DeviceCache &operator=(const DeviceCache &) = delete;

  void prefill(size_t layer, const KvInput &kv, const QueryInput &q, DequantOutput &out,
               hipStream_t stream = nullptr) override {
    int orig = 0;
    check(tq_cache_prefill(h_, (int)layer, kv.k, kv.v, (int)kv.dtype, kv.tokens, q.q, (int)q.dtype, q.num_q_heads,
                           q.q_len, out.k, out.v, &orig, out.logit_bias, stream));
    out.returned_originals = orig != 0;
  }
  void decode(size_t layer, const KvInput &kv, const QueryInput &q, const AttendConfig &cfg, void *out,
              DType out_dtype, hipStream_t stream = nullptr) override {
    check(tq_cache_decode(h_, (int)layer, kv.k, kv.v, (int)kv.dtype, kv.tokens, q.q, (int)q.dtype, q.num_q_heads,
                          cfg.softmax_scale, out, (int)out_dtype, stream));
  }
  // DecodeOutput::Dequantized
  void decode_dequantized(size_t layer, const KvInput &kv, const QueryInput &q, DequantOutput &out,
                          hipStream_t stream = nullptr) {
    check(tq_cache_decode_dequantized(h_, (int)layer, kv.k, kv.v, (int)kv.dtype, kv.tokens, q.q, (int)q.dtype,
                                      q.num_q_heads, q.q_len, out.k, out.v, out.logit_bias, stream));
  }
  size_t seq_len(size_t layer) const override { return tq_cache_seq_len(h_, (int)layer); }
  size_t capacity(size_t layer) const { return tq_cache_capacity(h_, (int)layer); }
  void reset() override { check(tq_cache_reset(h_)); }
  size_t memory_usage() const override { return tq_cache_memory_usage(h_); }
  const CacheConfig &config() const { return config_; }
  void *handle() const { return h_; }

 private:
  CacheConfig config_;
  void *h_ = nullptr;
};
}  // namespace detail

// PqoCache::new (pqo.rs:21-51): PQO (outlier_blocks all), PQ (0) or mixed
class PqoCache : public detail::DeviceCache {
 public:
  explicit PqoCache(const CacheConfig &c) : DeviceCache(c, false) {}
};

// TqCache::new (tq.rs:20-57): needs outlier_blocks == 0
class TqCache : public detail::DeviceCache {
 public:
  explicit TqCache(const CacheConfig &c) : DeviceCache(c, true) {}
};

}  // namespace tq

#endif
