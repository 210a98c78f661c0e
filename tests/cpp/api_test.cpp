// api_test.cpp -- drives the C++ host API (include/turboquant_amd.hpp) the
// way the reference crate's own tests drive its Rust API, printing the
// results as JSON for tests/test_cpp_api.py to check against the oracle.
//
//   api_test host                     config validation and PackedBlock
//                                     packing (no device calls)
//   api_test gpu <inputs.bin>         quantize_vec / dequantize_vec /
//                                     quantize_with_qjl / estimates /
//                                     QuantizedKVCache / PqoCache / TqCache
//
// inputs.bin: uint32 n, uint32 dim, n*dim f32 vectors, dim f32 query.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "turboquant_amd.hpp"

namespace {

void print_bytes(const char *key, const std::vector<uint8_t> &b) {
  std::printf("\"%s\": [", key);
  for (size_t i = 0; i < b.size(); i++) std::printf("%s%u", i ? "," : "", b[i]);
  std::printf("]");
}
void print_floats(const char *key, const std::vector<float> &v) {
  std::printf("\"%s\": [", key);
  for (size_t i = 0; i < v.size(); i++) std::printf("%s%.9g", i ? "," : "", v[i]);
  std::printf("]");
}

int error_kind(void (*fn)()) {
  try {
    fn();
  } catch (const tq::Error &e) {
    return static_cast<int>(e.kind());
  }
  return 0;
}

int run_host() {
  // TurboQuantConfig::new validation (packed/mod.rs:121-127)
  const int e_bits = error_kind([] { tq::TurboQuantConfig::create(5, 128); });
  const int e_dim = error_kind([] { tq::TurboQuantConfig::create(3, 100); });
  const int e_zero = error_kind([] { tq::TurboQuantConfig::create(3, 0); });
  const auto ok = tq::TurboQuantConfig::create(4, 64).with_seed(42);
  std::printf("{\"config\": {\"unsupported_bits\": %d, \"invalid_dim\": %d, \"zero_dim\": %d, \"bits\": %u, "
              "\"dim\": %zu, \"seed\": %llu}}\n",
              e_bits, e_dim, e_zero, ok.bits, ok.dim, (unsigned long long)ok.rotation_seed);
  // PackedBlock::new over index ramps, full and ragged counts
  for (int bits = 2; bits <= 4; bits++) {
    for (size_t count : {128u, 13u, 1u}) {
      std::vector<uint8_t> idx(count);
      for (size_t i = 0; i < count; i++) idx[i] = (uint8_t)((i * 7 + 3) % (1u << bits));
      const tq::PackedBlock b = tq::PackedBlock::create((uint8_t)bits, 0x3c00, idx);
      const bool round_trip = b.unpack(count) == idx;
      std::printf("{\"pack\": {\"bits\": %d, \"count\": %zu, \"size_bytes\": %zu, \"round_trip\": %s, ", bits, count,
                  b.size_bytes(), round_trip ? "true" : "false");
      print_bytes("indices", idx);
      std::printf(", ");
      print_bytes("packed", b.packed_indices);
      std::printf("}}\n");
    }
  }
  return 0;
}

int run_gpu(const char *path) {
  FILE *f = std::fopen(path, "rb");
  if (!f) return 2;
  uint32_t n = 0, dim = 0;
  if (std::fread(&n, 4, 1, f) != 1 || std::fread(&dim, 4, 1, f) != 1) return 2;
  std::vector<std::vector<float>> vecs(n, std::vector<float>(dim));
  for (auto &v : vecs)
    if (std::fread(v.data(), 4, dim, f) != dim) return 2;
  std::vector<float> query(dim);
  if (std::fread(query.data(), 4, dim, f) != dim) return 2;
  std::fclose(f);

  // quantize_vec / dequantize_vec / dequantize_rotated (quantize.rs:142-316)
  const auto cfg = tq::TurboQuantConfig::create(3, dim).with_seed(42);
  for (uint32_t i = 0; i < 3 && i < n; i++) {
    const tq::PackedBlock b = tq::quantize_vec(cfg, vecs[i]);
    std::printf("{\"quantize_vec\": {\"i\": %u, \"scale\": %u, ", i, b.scale);
    print_bytes("packed", b.packed_indices);
    std::printf(", ");
    print_floats("dequant", tq::dequantize_vec(cfg, b));
    std::printf(", ");
    print_floats("rotated", tq::dequantize_rotated(cfg, b));
    std::printf("}}\n");
  }
  const int e_mismatch = error_kind([] {
    tq::quantize_vec(tq::TurboQuantConfig::create(3, 64), std::vector<float>(32, 1.0f));
  });
  std::printf("{\"dimension_mismatch\": %d}\n", e_mismatch);

  // quantize_with_qjl + estimates (qjl.rs:355-377, 488-627)
  const uint64_t qjl_seed = 12345;
  const tq::QjlBlock qb = tq::quantize_with_qjl(cfg, vecs[0], qjl_seed);
  std::printf("{\"qjl_block\": {\"polar_bits\": %u, \"scale\": %u, \"norm\": %u, \"size_bytes\": %zu, ",
              qb.polar_block.bits, qb.polar_block.scale, qb.residual_norm, qb.size_bytes());
  print_bytes("polar", qb.polar_block.packed_indices);
  std::printf(", ");
  print_bytes("signs", qb.qjl_signs);
  std::printf(", \"single\": %.9g}}\n", tq::estimate_inner_product_single(query, qb, cfg, qjl_seed));
  std::printf("{");
  print_floats("rq", tq::precompute_query_projections(query, dim, qjl_seed));
  std::printf("}\n");

  // QuantizedKVCache (attention.rs)
  tq::QuantizedKVCache cache(cfg, 2, qjl_seed);
  std::vector<std::vector<float>> keys(vecs.begin(), vecs.begin() + n / 2), values(vecs.begin() + n / 2,
                                                                                    vecs.begin() + 2 * (n / 2));
  cache.push_batch(1, keys, values);
  cache.push(1, vecs[0], vecs[1]);
  const std::vector<float> scores = cache.attention_scores(1, query);
  std::vector<float> w(scores.size());
  for (size_t i = 0; i < w.size(); i++) w[i] = 1.0f / (float)(i + 1);
  const std::vector<float> wv = cache.weighted_values(1, w);
  const int e_layer = error_kind([] {
    tq::QuantizedKVCache c(tq::TurboQuantConfig::create(3, 64), 1, 1);
    c.attention_scores(3, std::vector<float>(64));
  });
  const tq::QjlBlock kb = cache.key_block(1, 2);
  std::printf("{\"kv_cache\": {\"entries\": %zu, \"empty_layer\": %zu, \"memory\": %zu, \"fp16\": %zu, "
              "\"layer_error\": %d, \"key2_scale\": %u, ",
              cache.entry_count(1), cache.entry_count(0), cache.memory_usage(), cache.fp16_equivalent_memory(),
              e_layer, kb.polar_block.scale);
  print_floats("scores", scores);
  std::printf(", ");
  print_floats("weights", w);
  std::printf(", ");
  print_floats("weighted", wv);
  std::printf(", ");
  print_floats("key1", cache.dequantize_keys_range(1, 1, 2)[0]);
  std::printf("}}\n");

  // PqoCache / TqCache through the CompressedKVCache trait (device buffers)
  if (dim == 128) {
    const int heads = 2, t = 8;
    std::vector<float> kv(heads * t * dim), q(4 * dim);
    for (size_t i = 0; i < kv.size(); i++) kv[i] = vecs[(i / dim) % n][i % dim];
    for (size_t i = 0; i < q.size(); i++) q[i] = query[i % dim];
    tq::detail::DeviceBuffer dk(kv.size() * 4), dq(q.size() * 4), dout(4 * dim * 4), dbias(4 * (t + 1) * 4);
    tq::detail::to_device(dk.get(), kv.data(), kv.size() * 4, nullptr);
    tq::detail::to_device(dq.get(), q.data(), q.size() * 4, nullptr);
    for (int kind = 0; kind < 2; kind++) {
      tq::CacheConfig cc;
      cc.bits = 3;
      cc.head_dim = 128;
      cc.num_kv_heads = heads;
      cc.num_layers = 1;
      cc.outlier_blocks = kind ? 0 : tq::kOutlierAll;
      tq::PqoCache pqo(cc);
      tq::TqCache *tqc = nullptr;
      tq::detail::DeviceCache *c = &pqo;
      if (kind) c = tqc = new tq::TqCache(cc);
      tq::DequantOutput o;
      o.logit_bias = kind ? dbias.get() : nullptr;
      c->prefill(0, {dk.get(), dk.get(), tq::DType::F32, t}, {dq.get(), tq::DType::F32, 4, 1}, o);
      const tq::KvInput one{dk.get(), dk.get(), tq::DType::F32, 1};
      c->decode(0, one, {dq.get(), tq::DType::F32, 4, 1}, {0.0883883476f, 2}, dout.get(), tq::DType::F32);
      std::vector<float> out(4 * dim);
      tq::detail::to_host(out.data(), dout.get(), out.size() * 4, nullptr);
      std::printf("{\"cache\": {\"kind\": \"%s\", \"originals\": %s, \"seq\": %zu, \"memory\": %zu, ",
                  kind ? "tq" : "pqo", o.returned_originals ? "true" : "false", c->seq_len(0), c->memory_usage());
      print_floats("out", out);
      std::printf("}}\n");
      c->reset();
      delete tqc;
    }
  }
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  try {
    if (argc >= 2 && std::string(argv[1]) == "host") return run_host();
    if (argc >= 3 && std::string(argv[1]) == "gpu") return run_gpu(argv[2]);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  std::fprintf(stderr, "usage: api_test host | api_test gpu <inputs.bin>\n");
  return 2;
}
