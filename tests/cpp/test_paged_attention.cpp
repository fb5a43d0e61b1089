// Tests of the C++ mirror of the reference's paged/flash attention API
// (sketchpad_amd/host/paged_attention.hpp). The first group restates the reference's own unit
// tests (crates/sketchpad-core/src/paged_attention.rs:560-675, transformer.rs:524-536) against
// the mirror; the second exercises the device paths: store/gather round trips, the paged cache
// against the concatenating cache, and flash attention against a direct host computation.
//
//   test_paged_attention [--cpu-only]     (exit status 0 = all passed)
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <functional>
#include <random>
#include <vector>

#include "paged_attention.hpp"
#include "test_harness.hpp"

using namespace sketchpad;

// ---- restated reference tests (paged_attention.rs:560-675) -----------------------------------

TEST(test_block_table, false) {
  BlockTable table(4);
  CHECK(table.seq_len() == 0);
  CHECK(table.num_blocks() == 0);
  CHECK(!table.needs_new_block());
  table.add_block(0);
  table.increment_seq_len(4);
  CHECK(table.seq_len() == 4);
  CHECK(table.num_blocks() == 1);
  CHECK(table.needs_new_block());
  CHECK(table.get_block(0) == std::optional<size_t>(0));
  CHECK(table.get_block(3) == std::optional<size_t>(0));
  CHECK(table.get_slot(0) == 0);
  CHECK(table.get_slot(3) == 3);
  table.add_block(5);
  table.increment_seq_len(2);
  CHECK(table.seq_len() == 6);
  CHECK(table.get_block(4) == std::optional<size_t>(5));
  CHECK(table.get_block(5) == std::optional<size_t>(5));
  CHECK(table.get_slot(4) == 0);
  CHECK(table.get_slot(5) == 1);
  CHECK(!table.get_block(8).has_value());  // Option::None past the table
}

TEST(test_config_from_memory_budget, false) {
  const auto config = PagedKvCacheConfig::from_memory_budget(1024ull * 1024 * 1024, 8, 128, 32, 16);
  CHECK(config.num_blocks == 256);
}

TEST(test_causal_mask, false) {  // transformer.rs:524-536
  const auto m = causal_mask(4);
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) CHECK((j > i) == (m[i * 4 + j] == -INFINITY));
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j <= i; ++j) CHECK(m[i * 4 + j] == 0.f);
}

TEST(test_result_errors, false) {
  auto e = Result<Unit>::Err("Out of memory: no free blocks");
  CHECK(e.is_err());
  bool threw = false;
  try {
    e.unwrap();
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw);
}

TEST(test_paged_kv_cache_allocation, true) {
  PagedKvCache cache(PagedKvCacheConfig(4, 10, 8, 64, 2));
  CHECK(cache.num_blocks() == 10);
  CHECK(cache.num_free_blocks() == 10);
  auto b0 = cache.allocate_block();
  auto b1 = cache.allocate_block();
  CHECK(b0.has_value() && b1.has_value());
  CHECK(*b0 == 0 && *b1 == 1);  // FIFO free list over 0..num_blocks
  CHECK(cache.num_free_blocks() == 8);
  cache.free_block(*b0);
  CHECK(cache.num_free_blocks() == 9);
}

TEST(test_paged_scheduler, true) {
  PagedScheduler scheduler(PagedKvCacheConfig(4, 10, 8, 64, 2));
  const size_t seq0 = scheduler.add_sequence().unwrap();
  const size_t seq1 = scheduler.add_sequence().unwrap();
  CHECK(seq0 == 0 && seq1 == 1);
  CHECK(scheduler.num_sequences() == 2);
  CHECK(scheduler.allocate(seq0, 3).is_ok());  // 1 block
  CHECK(scheduler.allocate(seq1, 5).is_ok());  // 2 blocks
  CHECK(scheduler.cache.num_free_blocks() == 7);
  scheduler.free_sequence(seq0);
  CHECK(scheduler.cache.num_free_blocks() == 8);
  CHECK(std::string(scheduler.allocate(7, 1).error()) == "Invalid sequence ID");
  CHECK(scheduler.available_tokens() == 8 * 4);
}

TEST(test_out_of_blocks, true) {
  PagedScheduler scheduler(PagedKvCacheConfig(4, 2, 1, 8, 1));
  const size_t s = scheduler.add_sequence().unwrap();
  auto r = scheduler.allocate(s, 9);  // needs 3 blocks, the pool has 2
  CHECK(r.is_err() && std::string(r.error()) == "Out of memory: no free blocks");
}

TEST(test_gather_kv_empty, true) {
  PagedKvCache cache(PagedKvCacheConfig(4, 10, 8, 64, 2));
  BlockTable table(4);
  auto kv = cache.gather_kv(0, table);
  CHECK((kv.first.dims() == std::vector<int64_t>{8, 0, 64}));
  CHECK((kv.second.dims() == std::vector<int64_t>{8, 0, 64}));
}

// ---- device paths ---------------------------------------------------------------------------

static std::vector<float> randn(size_t n, uint32_t seed) {
  std::mt19937 g(seed);
  std::normal_distribution<float> d;
  std::vector<float> v(n);
  for (auto& x : v) x = d(g);
  return v;
}

TEST(test_store_gather_round_trip, true) {
  // two layers interleaved in every block; positions spread over a shuffled block table
  const size_t H = 2, D = 64, BS = 4;
  PagedKvCache cache(PagedKvCacheConfig(BS, 12, H, D, 2));
  BlockTable table(BS);
  for (size_t b : {7, 2, 9, 0, 5}) table.add_block(b);
  const size_t L = 18;
  table.increment_seq_len(L);
  auto kh = randn(H * L * D, 1), vh = randn(H * L * D, 2);
  auto k = DeviceTensor::from_host(kh.data(), {(int64_t)H, (int64_t)L, (int64_t)D}, SP_F32);
  auto v = DeviceTensor::from_host(vh.data(), {(int64_t)H, (int64_t)L, (int64_t)D}, SP_F32);
  cache.store_kv(1, table, k, v, 0);
  auto kv = cache.gather_kv(1, table);
  std::vector<float> kg(H * L * D), vg(H * L * D);
  kv.first.to_host(kg.data());
  kv.second.to_host(vg.data());
  CHECK(memcmp(kg.data(), kh.data(), kg.size() * 4) == 0);
  CHECK(memcmp(vg.data(), vh.data(), vg.size() * 4) == 0);
  // layer 0 and the untouched blocks stay zero
  std::vector<float> pool(12 * 2 * H * BS * D);
  cache.k_cache().to_host(pool.data());
  for (size_t b = 0; b < 12; ++b)
    for (size_t i = 0; i < H * BS * D; ++i) CHECK(pool[(b * 2 + 0) * H * BS * D + i] == 0.f);
  for (size_t b : {1, 3, 4, 6, 8, 10, 11})
    for (size_t i = 0; i < H * BS * D; ++i) CHECK(pool[(b * 2 + 1) * H * BS * D + i] == 0.f);
  // a position without a block: the reference panics "Block not allocated"
  bool threw = false;
  try {
    cache.store_kv(1, table, k, v, 5);  // positions 5..22, the table covers 0..19
  } catch (const std::runtime_error& e) {
    threw = std::string(e.what()) == "Block not allocated";
  }
  CHECK(threw);
}

TEST(test_paged_cache_equals_concat_cache, true) {
  // AttentionCache through the paged pool == the concatenating ModelKvCache, bit for bit, over
  // a prefill of 5 tokens and 6 single-token steps on 3 layers (every layer, not only layer 0).
  const size_t H = 4, D = 128, BS = 16, layers = 3;
  PagedAttentionCache paged(PagedKvCacheConfig(BS, 8, H, D, layers), SP_BF16);
  ModelKvCache concat(layers, 1024);
  uint32_t seed = 10;
  for (size_t step = 0; step < 7; ++step) {
    const size_t S = step == 0 ? 5 : 1;
    for (size_t layer = 0; layer < layers; ++layer) {
      std::vector<uint16_t> kh(H * S * D), vh(H * S * D);
      auto kf = randn(kh.size(), seed++), vf = randn(vh.size(), seed++);
      for (size_t i = 0; i < kh.size(); ++i) {
        uint32_t a, b;
        memcpy(&a, &kf[i], 4);
        memcpy(&b, &vf[i], 4);
        kh[i] = (uint16_t)(a >> 16);
        vh[i] = (uint16_t)(b >> 16);
      }
      const std::vector<int64_t> shape = {1, (int64_t)H, (int64_t)S, (int64_t)D};
      auto k = DeviceTensor::from_host(kh.data(), shape, SP_BF16);
      auto v = DeviceTensor::from_host(vh.data(), shape, SP_BF16);
      auto a = paged.update_layer(layer, k, v);
      auto b = concat.update_layer(layer, k, v);
      CHECK(a.k.dims() == b.k.dims());
      std::vector<uint16_t> ka(a.k.numel()), kb(b.k.numel()), va(a.v.numel()), vb(b.v.numel());
      a.k.to_host(ka.data());
      b.k.to_host(kb.data());
      a.v.to_host(va.data());
      b.v.to_host(vb.data());
      CHECK(ka == kb);
      CHECK(va == vb);
    }
    CHECK(paged.seq_len() == concat.seq_len());
  }
  CHECK(paged.seq_len() == 11);
  paged.clear();
  CHECK(paged.seq_len() == 0);
  CHECK(paged.cache().num_free_blocks() == 8);
}

static void host_attention(const std::vector<float>& q, const std::vector<float>& k,
                           const std::vector<float>& v, int B, int H, int Sq, int Sk, int D,
                           bool causal, std::vector<double>& out) {
  out.assign((size_t)B * H * Sq * D, 0.0);
  const double scale = 1.0 / sqrt((double)D);
  for (int bh = 0; bh < B * H; ++bh)
    for (int i = 0; i < Sq; ++i) {
      std::vector<double> s(Sk);
      double m = -INFINITY;
      for (int j = 0; j < Sk; ++j) {
        double acc = 0;
        for (int e = 0; e < D; ++e)
          acc += (double)q[((size_t)bh * Sq + i) * D + e] * k[((size_t)bh * Sk + j) * D + e];
        s[j] = (causal && j > i) ? -INFINITY : acc * scale;
        m = fmax(m, s[j]);
      }
      double l = 0;
      for (int j = 0; j < Sk; ++j) l += (s[j] = s[j] == -INFINITY ? 0.0 : exp(s[j] - m));
      for (int e = 0; e < D; ++e) {
        double acc = 0;
        for (int j = 0; j < Sk; ++j) acc += s[j] * v[((size_t)bh * Sk + j) * D + e];
        out[((size_t)bh * Sq + i) * D + e] = acc / l;
      }
    }
}

TEST(test_flash_attention_causal_bf16, true) {
  // shapes of the reference's flash tests (correctness_cpu.rs:1104-1234), bf16 inputs
  for (auto shp : {std::vector<int>{1, 4, 16, 64}, std::vector<int>{2, 8, 64, 64}}) {
    const int B = shp[0], H = shp[1], S = shp[2], D = shp[3];
    const size_t n = (size_t)B * H * S * D;
    auto qf = randn(n, 100 + S), kf = randn(n, 200 + S), vf = randn(n, 300 + S);
    std::vector<uint16_t> qh(n), kh(n), vh(n);
    for (size_t i = 0; i < n; ++i) {  // round to bf16, keep the rounded values for the check
      for (auto* pr : {&qf, &kf, &vf}) {
        uint32_t u;
        memcpy(&u, &(*pr)[i], 4);
        u += 0x7fff + ((u >> 16) & 1);
        u &= 0xffff0000u;
        memcpy(&(*pr)[i], &u, 4);
      }
      uint32_t a, b, c;
      memcpy(&a, &qf[i], 4);
      memcpy(&b, &kf[i], 4);
      memcpy(&c, &vf[i], 4);
      qh[i] = a >> 16;
      kh[i] = b >> 16;
      vh[i] = c >> 16;
    }
    const std::vector<int64_t> shape = {B, H, S, D};
    auto q = DeviceTensor::from_host(qh.data(), shape, SP_BF16);
    auto k = DeviceTensor::from_host(kh.data(), shape, SP_BF16);
    auto v = DeviceTensor::from_host(vh.data(), shape, SP_BF16);
    auto r = flash_attention(q, k, v, FlashAttentionOptions::causal_());
    CHECK(r.is_ok());
    if (!r.is_ok()) continue;
    CHECK(hipDeviceSynchronize() == hipSuccess);
    std::vector<uint16_t> oh(n);
    r.out->to_host(oh.data());
    std::vector<double> ref;
    host_attention(qf, kf, vf, B, H, S, S, D, true, ref);
    double worst = 0;
    for (size_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)oh[i] << 16;
      float f;
      memcpy(&f, &u, 4);
      worst = fmax(worst, fabs((double)f - ref[i]));
    }
    CHECK(worst <= 2e-2);
    // qkv_attention with the causal mask tensor (attention.rs:4-42) is the same computation,
    // bit for bit: masked keys get zero weight either way
    auto o2 = qkv_attention(q, k, v, causal_mask_tensor(S));
    std::vector<uint16_t> oh2(n);
    o2.to_host(oh2.data());
    CHECK(oh2 == oh);
    // and without a mask it is the bidirectional flash_attention
    auto o3 = qkv_attention(q, k, v, std::nullopt);
    auto r3 = flash_attention(q, k, v, FlashAttentionOptions());
    CHECK(r3.is_ok());
    if (r3.is_ok()) {
      std::vector<uint16_t> a3(n), b3(n);
      o3.to_host(a3.data());
      r3.out->to_host(b3.data());
      CHECK(a3 == b3);
    }
  }
}

TEST(test_flash_attention_f32, true) {
  // f32 is the element type the reference's flash tests run (correctness_cpu.rs:1104-1234);
  // checked per output row at 1e-5 relative against a double-precision host computation
  for (auto shp : {std::vector<int>{1, 4, 16, 64}, std::vector<int>{2, 8, 64, 64},
                   std::vector<int>{1, 2, 100, 128}}) {
    for (bool causal : {false, true}) {
      const int B = shp[0], H = shp[1], S = shp[2], D = shp[3];
      const size_t n = (size_t)B * H * S * D;
      auto qf = randn(n, 400 + S), kf = randn(n, 500 + S), vf = randn(n, 600 + S);
      const std::vector<int64_t> shape = {B, H, S, D};
      auto q = DeviceTensor::from_host(qf.data(), shape, SP_F32);
      auto k = DeviceTensor::from_host(kf.data(), shape, SP_F32);
      auto v = DeviceTensor::from_host(vf.data(), shape, SP_F32);
      auto r = flash_attention(q, k, v, FlashAttentionOptions().with_causal(causal));
      CHECK(r.is_ok());
      if (!r.is_ok()) continue;
      CHECK(hipDeviceSynchronize() == hipSuccess);
      std::vector<float> oh(n);
      r.out->to_host(oh.data());
      std::vector<double> ref;
      host_attention(qf, kf, vf, B, H, S, S, D, causal, ref);
      double worst = 0;
      for (size_t row = 0; row < n / D; ++row) {
        double scale = 1e-30, err = 0;
        for (int d = 0; d < D; ++d) {
          scale = fmax(scale, fabs(ref[row * D + d]));
          err = fmax(err, fabs((double)oh[row * D + d] - ref[row * D + d]));
        }
        worst = fmax(worst, err / scale);
      }
      CHECK(worst <= 1e-5);
    }
  }
}

TEST(test_flash_attention_masked_f32, true) {
  // flash_attention_masked (attention.rs:119-128): an all-zero mask reproduces flash_attention
  // bit for bit, and the reference tests' additive causal mask (-inf above the diagonal, one
  // [Sq, Sk] mask expanded over batch and heads) reproduces causal flash_attention bit for bit
  const int B = 2, H = 2, S = 70, D = 64;
  const size_t n = (size_t)B * H * S * D;
  auto qf = randn(n, 700), kf = randn(n, 701), vf = randn(n, 702);
  const std::vector<int64_t> shape = {B, H, S, D};
  auto q = DeviceTensor::from_host(qf.data(), shape, SP_F32);
  auto k = DeviceTensor::from_host(kf.data(), shape, SP_F32);
  auto v = DeviceTensor::from_host(vf.data(), shape, SP_F32);
  std::vector<float> zero((size_t)S * S, 0.f), causal((size_t)S * S, 0.f);
  for (int i = 0; i < S; ++i)
    for (int j = i + 1; j < S; ++j) causal[(size_t)i * S + j] = -INFINITY;
  auto mz = DeviceTensor::from_host(zero.data(), {S, S}, SP_F32);
  auto mc = DeviceTensor::from_host(causal.data(), {S, S}, SP_F32);
  auto plain = flash_attention(q, k, v, FlashAttentionOptions());
  auto plain_c = flash_attention(q, k, v, FlashAttentionOptions::causal_());
  auto masked0 = flash_attention_masked(q, k, v, mz, FlashAttentionOptions());
  auto maskedc = flash_attention_masked(q, k, v, mc, FlashAttentionOptions());
  CHECK(plain.is_ok() && plain_c.is_ok() && masked0.is_ok() && maskedc.is_ok());
  if (!(plain.is_ok() && plain_c.is_ok() && masked0.is_ok() && maskedc.is_ok())) return;
  CHECK(hipDeviceSynchronize() == hipSuccess);
  std::vector<float> a(n), b(n), c(n), d(n);
  plain.out->to_host(a.data());
  masked0.out->to_host(b.data());
  plain_c.out->to_host(c.data());
  maskedc.out->to_host(d.data());
  CHECK(memcmp(a.data(), b.data(), n * 4) == 0);
  CHECK(memcmp(c.data(), d.data(), n * 4) == 0);
  // malformed masks are setup errors, not launches
  auto bad = DeviceTensor::from_host(zero.data(), {S, S - 1}, SP_F32);
  CHECK(!flash_attention_masked(q, k, v, bad, FlashAttentionOptions()).is_ok());
  DeviceTensor m16({S, S}, SP_BF16);
  CHECK(!flash_attention_masked(q, k, v, m16, FlashAttentionOptions()).is_ok());
}

TEST(test_flash_attention_setup_errors, true) {
  DeviceTensor q({1, 2, 8, 64}, SP_BF16), k({1, 2, 8, 32}, SP_BF16);
  auto r = flash_attention(q, k, k, FlashAttentionOptions());
  CHECK(!r.is_ok() && r.error.has_value());
  // a head dim no kernel covers is reported by the library
  DeviceTensor q48({1, 2, 8, 48}, SP_F32);
  auto r48 = flash_attention(q48, q48, q48, FlashAttentionOptions());
  CHECK(!r48.is_ok() && r48.error->message.find("head_dim") != std::string::npos);
}

TEST(test_flash_attention_options, true) {
  // FlashAttentionOptions.out_dtype and a value head dim of its own (attention.rs:39-69,
  // :140-147): out is [B, H, Sq, Dv] of out_dtype; bf16 / f16 outputs are the f32 result rounded
  // once, bit for bit
  const int B = 1, H = 2, Sq = 40, Sk = 57, D = 80, Dv = 48;
  auto qf = randn((size_t)B * H * Sq * D, 801), kf = randn((size_t)B * H * Sk * D, 802);
  auto vf = randn((size_t)B * H * Sk * Dv, 803);
  auto q = DeviceTensor::from_host(qf.data(), {B, H, Sq, D}, SP_F32);
  auto k = DeviceTensor::from_host(kf.data(), {B, H, Sk, D}, SP_F32);
  auto v = DeviceTensor::from_host(vf.data(), {B, H, Sk, Dv}, SP_F32);
  auto r32 = flash_attention(q, k, v, FlashAttentionOptions());
  auto rbf = flash_attention(q, k, v, FlashAttentionOptions().with_dtype(SP_BF16));
  CHECK(r32.is_ok() && rbf.is_ok());
  if (!(r32.is_ok() && rbf.is_ok())) return;
  CHECK((r32.out->dims() == std::vector<int64_t>{B, H, Sq, Dv}) && rbf.out->dtype() == SP_BF16);
  std::vector<float> o32((size_t)B * H * Sq * Dv);
  std::vector<uint16_t> obf(o32.size());
  r32.out->to_host(o32.data());
  rbf.out->to_host(obf.data());
  size_t same = 0;
  for (size_t i = 0; i < o32.size(); ++i) {
    uint32_t u;
    memcpy(&u, &o32[i], 4);
    u += 0x7fff + ((u >> 16) & 1);
    same += (uint16_t)(u >> 16) == obf[i];
  }
  CHECK(same == o32.size());
  // against double precision, per row at 1e-5 relative (Dv != D: the host loop takes Dv rows)
  double worst = 0;
  for (int bh = 0; bh < B * H; ++bh)
    for (int i = 0; i < Sq; ++i) {
      std::vector<double> sc(Sk);
      double mx = -1e300;
      for (int j = 0; j < Sk; ++j) {
        double acc = 0;
        for (int e = 0; e < D; ++e)
          acc += (double)qf[((size_t)bh * Sq + i) * D + e] * kf[((size_t)bh * Sk + j) * D + e];
        sc[j] = acc / sqrt((double)D);
        mx = fmax(mx, sc[j]);
      }
      double l = 0;
      for (auto& x : sc) l += (x = exp(x - mx));
      double scale = 1e-30, err = 0;
      for (int e = 0; e < Dv; ++e) {
        double o = 0;
        for (int j = 0; j < Sk; ++j) o += sc[j] * vf[((size_t)bh * Sk + j) * Dv + e];
        o /= l;
        scale = fmax(scale, fabs(o));
        err = fmax(err, fabs(o - o32[((size_t)bh * Sq + i) * Dv + e]));
      }
      worst = fmax(worst, err / scale);
    }
  CHECK(worst <= 1e-5);
}

int main(int argc, char** argv) {
  const bool cpu_only = argc > 1 && strcmp(argv[1], "--cpu-only") == 0;
  int ran = 0;
  for (const auto& c : cases()) {
    if (c.gpu && cpu_only) continue;
    const int before = g_failures;
    printf("[test] %s\n", c.name);
    fflush(stdout);
    try {
      c.fn();
    } catch (const std::exception& e) {
      fprintf(stderr, "  exception: %s\n", e.what());
      ++g_failures;
    }
    printf("  %s\n", g_failures == before ? "ok" : "FAILED");
    ++ran;
  }
  printf("%d tests, %d failed checks\n", ran, g_failures);
  return g_failures == 0 ? 0 : 1;
}
