// test_engine.cpp — tests of the C++ engine layer.
//
//   test_engine --cpu   host-only: expected, registry, the KV-cache
//                       transaction state machine (reference preconditions of
//                       src/kvcache/*.cpp), views, graph order, RoPE table.
//   test_engine --gpu   the Qwen3 attention slice (qk-norm, RoPE, KV append,
//                       attention; src/models/Qwen3.cpp:61-88) built with the
//                       engine's OpFactory, scheduled on HIPBackend over a
//                       KVCacheManager, for a prefill and several decode
//                       steps, checked against the CPU oracle: cache bytes
//                       bit-exact, attention within 1e-4 rel / 1e-5 abs.
//
// Prints one line per check; the exit status is the number of failures.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../infer-llm_amd/engine/backend.hpp"
#include "../../infer-llm_amd/engine/graph.hpp"
#include "../../infer-llm_amd/engine/hip_backend.hpp"
#include "../../infer-llm_amd/engine/kvcache/kvcache_manager.hpp"
#include "../../infer-llm_amd/engine/kvcache/offload_storage.hpp"
#include "../../infer-llm_amd/engine/op_factory.hpp"
#include "../../infer-llm_amd/engine/scheduler.hpp"
#include "../../include/ikv.h"
#include "../../oracle/oracle.h"

static int g_fail = 0;
#define CHECK(cond, name)                                         \
  do {                                                            \
    if (cond) {                                                   \
      std::printf("PASS %s\n", name);                             \
    } else {                                                      \
      std::printf("FAIL %s (%s:%d)\n", name, __FILE__, __LINE__); \
      ++g_fail;                                                   \
    }                                                             \
    std::fflush(stdout);                                          \
  } while (0)

static bool is_err(const std::error_code &e, std::errc want) { return e == std::make_error_code(want); }

// Host backend test double: malloc pools, counts frees, computes nothing.
class HostBackend : public Backend {
 public:
  explicit HostBackend(int id = 0) : Backend(id, {"host:" + std::to_string(id), DeviceType::CPU, 0}, {}) {
    init_pools(std::make_unique<HostPhysicalAllocator>());
  }
  DeviceType device_type() const override { return DeviceType::CPU; }
  std::string device_name() const override { return "HOST"; }
  bool supports_op(OperationType, const Tensor &) const override { return false; }
  bool is_host() const override { return true; }
  infer::expected<void *, std::error_code> alloc(BufferKind k, size_t b) override {
    ++allocs;
    return Backend::alloc(k, b);
  }
  void free(BufferKind k, void *p) override {
    if (p) ++frees;
    Backend::free(k, p);
  }
  infer::expected<void, std::error_code> copy_tensor_set(Tensor *t, const void *d, size_t o, size_t s) override {
    std::memcpy(static_cast<char *>(t->data) + o, d, s);
    return {};
  }
  infer::expected<void, std::error_code> copy_tensor_get(const Tensor *t, void *d, size_t o, size_t s) override {
    std::memcpy(d, static_cast<const char *>(t->data) + o, s);
    return {};
  }
  infer::expected<bool, std::error_code> copy_tensor_high(const Tensor *, Tensor *) const override { return false; }
  infer::expected<void, std::error_code> compute(Graph &) override { return infer::fail(std::errc::not_supported); }
  int allocs = 0, frees = 0;
};

// splitmix64 -> Box-Muller, the generator of the Python tests
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  std::vector<float> normal(size_t n, double std = 1.0) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i += 2) {
      const double u1 = (double((next() >> 11)) + 1.0) * 0x1.0p-53;
      const double u2 = double(next() >> 11) * 0x1.0p-53;
      const double r = std::sqrt(-2.0 * std::log(u1));
      v[i] = float(r * std::cos(2.0 * M_PI * u2) * std);
      if (i + 1 < n) v[i + 1] = float(r * std::sin(2.0 * M_PI * u2) * std);
    }
    return v;
  }
};

// ---------------------------------------------------------------------------
// CPU checks

static void paged_cpu_tests();
static void offload_cpu_tests();
static void offload_gpu_tests(HIPBackend *hip);
static void producer_cache_gpu_tests(HIPBackend *hip);
static void host_copy_gpu_tests(HIPBackend *hip);

static void cpu_tests() {
  {
    // the decode workspace reserved up front covers every context: no
    // allocation inside a decode step (host arithmetic, no device)
    bool ok = true;
    for (auto [hq, hkv] : {std::pair{16, 8}, {32, 8}, {64, 8}, {8, 8}, {16, 2}}) {
      for (int64_t cap : {64, 130, 2560, 4352, 9000}) {
        const size_t r = HIPBackend::decode_workspace_reservation(hq, hkv, 128, cap);
        size_t most = 0;
        for (int64_t n = 1; n <= cap; ++n) {
          const size_t w = ikv_attn_decode_workspace_bytes(hq, hkv, 128, n);
          ok = ok && w <= r;
          most = std::max(most, w);
        }
        ok = ok && most == r;
      }
    }
    // the split count is not monotone in the context (Qwen3-0.6B shape: 2048
    // keys take 32 splits, 2080 keys 22), so a reservation sized from the
    // largest context alone would be too small
    const size_t at2048 = ikv_attn_decode_workspace_bytes(16, 8, 128, 2048);
    const size_t at2080 = ikv_attn_decode_workspace_bytes(16, 8, 128, 2080);
    ok = ok && at2080 < at2048 &&
         HIPBackend::decode_workspace_reservation(16, 8, 128, 2080) >= at2048;
    CHECK(ok, "decode workspace reservation covers every context up to capacity");
  }
  {
    infer::expected<int, std::error_code> a = 5;
    infer::expected<int, std::error_code> b = infer::fail(std::errc::invalid_argument);
    infer::expected<void, std::error_code> c;
    CHECK(a && *a == 5 && !b && is_err(b.error(), std::errc::invalid_argument) && c, "expected polyfill");
  }
  {
    auto &reg = BackendRegistry::instance();
    reg.register_backend(
        "host", [] { return std::vector<DeviceInfo>{{"host:0", DeviceType::CPU, 1}}; },
        [](int id, DeviceInfo, const PoolConfig &) -> std::unique_ptr<Backend> {
          return std::make_unique<HostBackend>(id);
        });
    reg.probe_all();
    auto ok = reg.create("host:0", {});
    auto missing = reg.create("host:7", {});
    CHECK(ok && (*ok)->is_host() && !missing && is_err(missing.error(), std::errc::no_such_device),
          "registry create by name");
    CHECK(BackendRegistry::extract_type("hip:3") == "hip" && BackendRegistry::extract_device_id("hip:3") == 3 &&
              BackendRegistry::extract_device_id("cpu") == 0,
          "registry name parsing");
  }

  HostBackend be;
  const size_t L = 3, cap = 16;
  std::vector<KVLayerSpec> specs(L, KVLayerSpec{8, 128, 128, GGML_TYPE_F32, GGML_TYPE_F32});
  std::vector<Backend *> place(L, &be);
  KVCacheManager kv(std::make_unique<ContiguousKVStrategy>(std::make_unique<NaiveKVStorage>()));
  CHECK(kv.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = cap}), "kv init");
  auto bad_init = KVCacheManager(std::make_unique<ContiguousKVStrategy>(std::make_unique<NaiveKVStorage>()))
                      .init(specs, place, KVCacheConfig{.layers = 2, .max_tokens_per_sequence = cap});
  CHECK(!bad_init && is_err(bad_init.error(), std::errc::invalid_argument), "kv init rejects layer mismatch");

  auto sid = kv.create_sequence();
  CHECK(sid && *sid == 1 && be.allocs == int(L), "create_sequence allocates one K+V block per layer");
  const SequenceId id = *sid;
  auto over = kv.reserve_append(id, cap + 1);
  CHECK(!over && is_err(over.error(), std::errc::not_enough_memory), "reserve beyond capacity");
  auto no_pending = kv.acquire_layer(id, 0);
  CHECK(!no_pending && is_err(no_pending.error(), std::errc::invalid_argument), "acquire without reserve");
  CHECK(kv.reserve_append(id, 4), "reserve 4");
  auto busy = kv.reserve_append(id, 1);
  CHECK(!busy && is_err(busy.error(), std::errc::device_or_resource_busy), "second reserve is busy");

  auto a0 = kv.acquire_layer(id, 0);
  CHECK(bool(a0), "acquire layer 0");
  const KVStorage *st = kv.strategy()->storage();
  const Tensor &rk = a0->readable.k.front().view, &wk = a0->writable.k.front().view;
  const Tensor &rv = a0->readable.v.front().view;
  const size_t row = 8 * 128 * 4;
  CHECK(a0->n_past == 0 && a0->n_new == 4 && rk.dims[0] == 128 && rk.dims[1] == 8 && rk.dims[2] == 4 &&
            rk.strides[2] == int64_t(row) && wk.data == rk.data &&
            static_cast<char *>(rv.data) == static_cast<char *>(rk.data) + cap * row &&
            rk.tensorRole == TensorRole::TENSOR_ROLE_KVCACHE,
          "views: [128,8,n] token-major, V after K");
  CHECK(st->state(1) && st->state(1)->active_users == 1, "storage acquired once per access");
  CHECK(kv.release_layer(*a0) && a0->released() && st->state(1)->active_users == 0, "release_layer");
  CHECK(kv.release_layer(*a0), "second release is a no-op");
  CHECK(kv.commit_append(id) && *kv.length(id) == 4, "commit -> length 4");
  auto no_commit = kv.commit_append(id);
  CHECK(!no_commit && is_err(no_commit.error(), std::errc::invalid_argument), "commit without pending");

  CHECK(kv.reserve_append(id, 1), "reserve 1 (decode)");
  auto a1 = kv.acquire_layer(id, 2);
  CHECK(a1 && a1->n_past == 4 && a1->readable.k.front().view.dims[2] == 5 &&
            static_cast<char *>(a1->writable.k.front().view.data) ==
                static_cast<char *>(a1->readable.k.front().view.data) + 4 * row,
          "decode views: readable [0,5), writable row 4");
  CHECK(kv.abort_append(id) && *kv.length(id) == 4, "abort keeps length");
  CHECK(kv.release_layer(*a1) && st->state(3)->active_users == 0, "release after abort");

  // deferred free while an access is outstanding
  CHECK(kv.reserve_append(id, 1), "reserve after abort");
  auto a2 = kv.acquire_layer(id, 1);
  const int frees_before = be.frees;
  CHECK(kv.release_sequence(id) && be.frees == frees_before + int(L) - 1, "release_sequence defers in-use layer");
  CHECK(kv.strategy()->release_layer(*a2) && be.frees == frees_before + int(L), "last release frees it");
  auto gone = kv.length(id);
  CHECK(!gone && is_err(gone.error(), std::errc::invalid_argument), "released sequence is gone");

  // capacity boundary
  auto s2 = kv.create_sequence();
  CHECK(s2 && kv.reserve_append(*s2, cap) && kv.commit_append(*s2), "fill to capacity");
  auto full = kv.reserve_append(*s2, 1);
  CHECK(!full && is_err(full.error(), std::errc::not_enough_memory), "no room after capacity");
  CHECK(kv.reserve_append(*s2, 0), "empty append at capacity");
  kv.abort_append(*s2);

  // context: busy while accesses are outstanding; theta table matches the oracle
  {
    GraphContext ctx(&be);
    auto s3 = kv.create_sequence();
    CHECK(ctx.set_kv_cache(&kv, *s3) && kv.reserve_append(*s3, 2), "context bind");
    auto acc = ctx.acquire_kv_layer(0);
    auto sw = ctx.set_kv_cache(&kv, *s2);
    CHECK(acc && !sw && is_err(sw.error(), std::errc::device_or_resource_busy), "context busy while acquired");
    CHECK(ctx.release_kv_access() && ctx.outstanding_kv_accesses() == 0 && ctx.set_kv_cache(&kv, *s2),
          "context release then rebind");
    kv.abort_append(*s3);
    auto th = ctx.get_rope_theta_table(1e6f, 128, 40960);
    std::vector<float> want(64 * 40960);
    oracle_rope_theta_table(1e6f, 128, 40960, want.data());
    CHECK(th && (*th)->dims[0] == 64 && (*th)->dims[1] == 40960 &&
              std::memcmp((*th)->data, want.data(), want.size() * 4) == 0,
          "rope angle table bit-exact with the oracle");
    auto th2 = ctx.get_rope_theta_table(1e6f, 128, 40960);
    CHECK(th2 && *th2 == *th, "rope angle table cached");
  }

  // graph order and append_kv wiring
  {
    Graph g;
    Tensor x("x", GGML_TYPE_F32, {128, 8, 1, 1}), w("w", GGML_TYPE_F32, {128, 1, 1, 1});
    float xb[1024] = {0}, wb[128] = {0};
    x.data = xb;
    w.data = wb;
    Tensor cache_w("cw", GGML_TYPE_F32, {128, 8, 1, 1}), cache_r("cr", GGML_TYPE_F32, {128, 8, 3, 1});
    std::vector<float> cache(3 * 1024);
    cache_r.data = cache.data();
    cache_w.data = cache.data() + 2 * 1024;
    Tensor *n = OpFactory::rms_norm(g, &x, &w, 1e-6f, "n");
    Tensor *view = append_kv(g, n, cache_w, cache_r);
    g.mark_output(view);
    CHECK(g.compute() && g.nodes().size() == 3 && g.nodes()[0] == n &&
              g.nodes()[1]->op == OperationType::GGML_OP_CPY && g.nodes()[2] == view &&
              view->src[0] == g.nodes()[1] && g.nodes()[1]->src[0] == n && g.nodes()[1]->pinned &&
              g.nodes()[1]->data == cache_w.data && view->data == cache_r.data && g.leafs().size() == 2,
          "graph topo order; append_kv = CPY then VIEW over the cache");
  }
  // view_rows: a VIEW of the last rows of an activation, aliased at its offset
  {
    Graph g;
    Tensor x("x", GGML_TYPE_F32, {1024, 5, 1, 1}), w("w", GGML_TYPE_F32, {1024, 1, 1, 1});
    std::vector<float> xb(5 * 1024), wb(1024);
    x.data = xb.data();
    w.data = wb.data();
    Tensor *n = OpFactory::rms_norm(g, &x, &w, 1e-6f, "n");
    Tensor *last = OpFactory::view_rows(g, n, 4, 1, "last");
    g.mark_output(last);
    CHECK(g.compute() && last->op == OperationType::GGML_OP_VIEW && last->src[0] == n &&
              last->dims == (std::array<int64_t, 4>{1024, 1, 1, 1}) && last->offset == 4 * 1024 * 4 &&
              !last->data && last->is_contiguous(),
          "view_rows: [1024, 1] VIEW of row 4 at byte offset 16384, placed with its source");
  }
  paged_cpu_tests();
  offload_cpu_tests();
}

// Paged strategy over a block pool (KVCacheConfig::block_tokens > 0): block
// lists, slices per block, the device block table, pool exhaustion with
// rollback, abort trimming, reuse of returned blocks.
static void paged_cpu_tests() {
  HostBackend be;
  const size_t L = 2, bt = 64, nb = 6, row = 8 * 128 * 4;
  std::vector<KVLayerSpec> specs(L, KVLayerSpec{8, 128, 128, GGML_TYPE_F32, GGML_TYPE_F32});
  std::vector<Backend *> place(L, &be);
  {
    auto bad = KVCacheManager(std::make_unique<PagedKVStrategy>(std::make_unique<BlockPoolKVStorage>(nb, bt)))
                   .init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = 320, .block_tokens = 32});
    CHECK(!bad && is_err(bad.error(), std::errc::invalid_argument), "paged init: block size must match the pool");
  }
  auto pool_owner = std::make_unique<BlockPoolKVStorage>(nb, bt);
  BlockPoolKVStorage *pool = pool_owner.get();
  auto strat_owner = std::make_unique<PagedKVStrategy>(std::move(pool_owner));
  PagedKVStrategy *strat = strat_owner.get();
  KVCacheManager kv(std::move(strat_owner));
  const int allocs0 = be.allocs;
  CHECK(kv.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = 320, .block_tokens = bt}) &&
            be.allocs == allocs0 + int(L) && pool->free_blocks(0) == nb && pool->k_pool(1) != nullptr,
        "paged init: one pool allocation per layer");
  auto a = kv.create_sequence();
  CHECK(a && pool->free_blocks(0) == nb, "create_sequence takes no block");
  CHECK(kv.reserve_append(*a, 100) && strat->blocks(*a, 0) == std::vector<int64_t>({0, 1}) &&
            strat->blocks(*a, 1) == std::vector<int64_t>({0, 1}) && pool->free_blocks(0) == nb - 2,
        "reserve 100 tokens: two blocks per layer");
  {
    auto acc = kv.acquire_layer(*a, 0);
    bool ok = bool(acc) && acc->readable.k.size() == 2 && acc->writable.k.size() == 2 && acc->pages;
    if (ok) {
      const auto &r = acc->readable.k;
      const char *kp = static_cast<const char *>(acc->pages.k_pool);
      ok = r[0].token_begin == 0 && r[0].token_count == 64 && r[1].token_begin == 64 &&
           r[1].token_count == 36 && r[0].view.data == kp && r[1].view.data == kp + bt * row &&
           acc->pages.block_tokens == bt && acc->pages.pool_blocks == nb &&
           static_cast<const int32_t *>(acc->pages.block_table->data)[1] == 1;
      CHECK(ok, "paged access: one segment per block, pool addresses, device table");
      (void)kv.release_layer(*acc);
    } else {
      CHECK(false, "paged access: one segment per block, pool addresses, device table");
    }
  }
  CHECK(kv.commit_append(*a) && kv.reserve_append(*a, 1) && strat->blocks(*a, 0).size() == 2, "decode step within a block");
  {
    auto acc = kv.acquire_layer(*a, 1);
    CHECK(acc && acc->writable.k.size() == 1 && acc->writable.k[0].token_begin == 100 &&
              acc->writable.k[0].view.data == static_cast<char *>(acc->pages.k_pool) + (bt + 36) * row,
          "decode write slice lands at block 1 offset 36");
    if (acc) (void)kv.release_layer(*acc);
  }
  CHECK(kv.commit_append(*a), "commit");
  auto b = kv.create_sequence();
  CHECK(b && kv.reserve_append(*b, 200) && strat->blocks(*b, 0) == std::vector<int64_t>({2, 3, 4, 5}) &&
            pool->free_blocks(0) == 0,
        "second sequence takes the remaining four blocks");
  auto exhausted = kv.reserve_append(*a, 100);
  CHECK(!exhausted && is_err(exhausted.error(), std::errc::not_enough_memory), "pool exhausted: reserve fails");
  CHECK(strat->blocks(*a, 0).size() == 2 && strat->blocks(*a, 1).size() == 2 && pool->free_blocks(1) == 0,
        "failed reserve leaves the sequence and the pool as they were");
  CHECK(kv.abort_append(*b) && pool->free_blocks(0) == 4 && strat->blocks(*b, 0).empty(),
        "abort returns the blocks that hold no committed token");
  CHECK(kv.reserve_append(*a, 100) && strat->blocks(*a, 0) == std::vector<int64_t>({0, 1, 2, 3}),
        "returned blocks are reused");
  {
    auto acc = kv.acquire_layer(*a, 0);
    const int32_t *tab = acc ? static_cast<const int32_t *>(acc->pages.block_table->data) : nullptr;
    CHECK(acc && tab && tab[0] == 0 && tab[1] == 1 && tab[2] == 2 && tab[3] == 3 && acc->writable.k.size() == 3 &&
              acc->writable.k[0].token_count == 27 && acc->writable.k[2].token_count == 9,
          "device table updated for the new blocks; tokens 101..200 span three blocks");
    if (acc) (void)kv.release_layer(*acc);
  }
  CHECK(kv.commit_append(*a) && kv.release_sequence(*a) && pool->free_blocks(0) == nb, "release returns every block");
  auto c = kv.create_sequence();
  CHECK(c && kv.reserve_append(*c, 128) && strat->blocks(*c, 0) == std::vector<int64_t>({3, 2}),
        "a new sequence gets the last returned blocks first (non-identity table)");
  auto over = kv.reserve_append(*c, 321);
  CHECK(!over && is_err(over.error(), std::errc::device_or_resource_busy), "one pending append per sequence");
  CHECK(kv.abort_append(*c) && pool->free_blocks(0) == 6, "abort at length 0 frees all");
  auto big = kv.reserve_append(*c, 321);
  CHECK(!big && is_err(big.error(), std::errc::not_enough_memory), "beyond max_tokens_per_sequence");
  CHECK(kv.clear_sequence() && pool->free_blocks(0) == nb && pool->free_blocks(1) == nb, "clear returns all blocks");
}

// Offload storage: host copies, an HBM budget, LRU eviction with write-back,
// busy objects, prefetch. The "device" is host memory that reports itself as
// not host, so every transfer is a memcpy the test can check.
class FakeDevice : public HostBackend {
 public:
  bool is_host() const override { return false; }
  DeviceType device_type() const override { return DeviceType::HIP; }
};

static void offload_cpu_tests() {
  HostBackend host;
  FakeDevice dev;
  const size_t L = 3, cap = 16, obj = cap * 8 * 128 * 4 * 2;
  std::vector<KVLayerSpec> specs(L, KVLayerSpec{8, 128, 128, GGML_TYPE_F32, GGML_TYPE_F32});
  std::vector<Backend *> place(L, &dev);
  auto make = [&](std::vector<KVDeviceBudget> budgets) {
    OffloadKVStorageConfig oc;
    oc.host_backend = &host;
    oc.device_budgets = std::move(budgets);
    return std::make_unique<OffloadKVStorage>(std::move(oc), std::make_unique<LRUKVEvictionPolicy>(),
                                              std::make_unique<NextAccessKVPrefetchPolicy>(2));
  };
  {
    KVCacheManager bad(std::make_unique<ContiguousKVStrategy>(make({})));
    auto r = bad.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = cap});
    CHECK(!r && is_err(r.error(), std::errc::invalid_argument), "offload init: a device without a budget");
  }
  auto owner = make({{.backend = &dev, .resident_bytes = 2 * obj, .prefetch_bytes = 2 * obj}});
  OffloadKVStorage *st = owner.get();
  KVCacheManager kv(std::make_unique<ContiguousKVStrategy>(std::move(owner)));
  CHECK(kv.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = cap}), "offload init");
  const int host_allocs = host.allocs, dev_allocs = dev.allocs;
  auto sid = kv.create_sequence();
  CHECK(sid && host.allocs == host_allocs + int(L) && dev.allocs == dev_allocs && st->resident_bytes(&dev) == 0,
        "sequence: one host copy per layer, nothing in HBM yet");
  CHECK(kv.reserve_append(*sid, 4), "reserve");
  const StorageId id0 = 1, id1 = 2, id2 = 3;
  const size_t row = 8 * 128 * 4 * 2;  // one token row of K and of V
  auto a0 = kv.acquire_layer(*sid, 0);
  CHECK(a0 && st->resident(id0) && st->stats().page_ins == 0 && st->stats().bytes_in == 0 &&
            st->resident_bytes(&dev) == obj,
        "acquire makes a new layer resident without a transfer (its host copy holds no rows)");
  // write a pattern through the view (the HBM copy)
  float *k0 = a0 ? static_cast<float *>(a0->readable.k.front().view.data) : nullptr;
  if (k0)
    for (int i = 0; i < 4 * 1024; ++i) k0[i] = float(i) * 0.5f;
  if (a0) (void)kv.release_layer(*a0);
  auto a1 = kv.acquire_layer(*sid, 1);
  if (a1) (void)kv.release_layer(*a1);
  auto a2 = kv.acquire_layer(*sid, 2);
  CHECK(a2 && !st->resident(id0) && st->resident(id1) && st->resident(id2) && st->stats().evictions == 1 &&
            st->stats().page_outs == 1 && st->stats().bytes_out == 4 * row,
        "budget of two: the least recently used layer is written back (its 4 written rows) and dropped");
  if (a2) (void)kv.release_layer(*a2);
  auto b0 = kv.acquire_layer(*sid, 0);
  bool same = b0.has_value();
  if (b0) {
    const float *k = static_cast<const float *>(b0->readable.k.front().view.data);
    for (int i = 0; i < 4 * 1024 && same; ++i) same = k[i] == float(i) * 0.5f;
  }
  CHECK(same && !st->resident(id1) && st->resident(id0) && st->stats().page_ins == 1 &&
            st->stats().bytes_in == 4 * row,
        "paged back in with its 4 rows; LRU victim next was layer 1");
  auto b2 = kv.acquire_layer(*sid, 2);
  auto b1 = kv.acquire_layer(*sid, 1);
  CHECK(b0 && b2 && !b1 && is_err(b1.error(), std::errc::not_enough_memory),
        "no room while both resident layers are held");
  auto busy = st->evict(id0);
  CHECK(!busy && is_err(busy.error(), std::errc::device_or_resource_busy), "evict refuses a held layer");
  if (b0) (void)kv.release_layer(*b0);
  if (b2) (void)kv.release_layer(*b2);
  CHECK(st->evict(id0) && st->evict(id2) && st->resident_bytes(&dev) == 0, "explicit evictions");
  const KVPrefetchRequest up[] = {{id1, 4}, {id2, 4}, {id0, 4}};
  auto n = st->prefetch(KVPrefetchContext{.current = id0, .upcoming = up});
  CHECK(n && *n == 2 && st->resident(id1) && st->resident(id2) && !st->resident(id0),
        "prefetch uploads the next two within the budget, evicting nothing");
  auto n2 = st->prefetch(KVPrefetchContext{.current = id1, .upcoming = std::span(up + 2, 1)});
  CHECK(n2 && *n2 == 0 && !st->resident(id0), "prefetch skips what does not fit");
  const int dev_frees = dev.frees, host_frees = host.frees;
  CHECK(kv.commit_append(*sid) && kv.release_sequence(*sid) && dev.frees == dev_frees + 2 &&
            host.frees == host_frees + int(L),
        "release frees every copy");

  // Valid rows across an aborted append and its retry: an HBM budget of one
  // layer, so every acquire of the other layer writes this one back.
  {
    auto own = make({{.backend = &dev, .resident_bytes = obj, .prefetch_bytes = 0}});
    OffloadKVStorage *s2 = own.get();
    KVCacheManager kv2(std::make_unique<ContiguousKVStrategy>(std::move(own)));
    const size_t L2 = 2, row_floats = 8 * 128;
    std::vector<KVLayerSpec> specs2(L2, specs[0]);
    std::vector<Backend *> place2(L2, &dev);
    bool ok = bool(kv2.init(specs2, place2, KVCacheConfig{.layers = L2, .max_tokens_per_sequence = cap}));
    auto q = kv2.create_sequence();
    ok = ok && bool(q);
    // one step: write rows [n_past, n_past + n) of layer 0 (K = base + i,
    // V = -(base + i) by float index i), touch layer 1, then commit or abort
    auto step = [&](size_t n, float base, bool commit) {
      if (!kv2.reserve_append(*q, n)) return false;
      auto a = kv2.acquire_layer(*q, 0);
      if (!a) return false;
      auto *k = static_cast<float *>(a->readable.k.front().view.data);
      auto *v = static_cast<float *>(a->readable.v.front().view.data);
      for (size_t i = a->n_past * row_floats; i < (a->n_past + n) * row_floats; ++i) {
        k[i] = base + float(i);
        v[i] = -(base + float(i));
      }
      (void)kv2.release_layer(*a);
      auto b = kv2.acquire_layer(*q, 1);
      if (!b) return false;
      (void)kv2.release_layer(*b);
      return commit ? bool(kv2.commit_append(*q)) : bool(kv2.abort_append(*q));
    };
    ok = ok && step(4, 100.f, true);   // rows 0..3
    const OffloadStats after_first = s2->stats();
    ok = ok && step(2, 500.f, false);  // rows 4..5, aborted
    ok = ok && step(2, 900.f, true);   // rows 4..5 again
    bool rows_ok = false;
    if (ok && kv2.reserve_append(*q, 1)) {
      auto c = kv2.acquire_layer(*q, 0);
      if (c) {
        const auto *k = static_cast<const float *>(c->readable.k.front().view.data);
        const auto *v = static_cast<const float *>(c->readable.v.front().view.data);
        rows_ok = true;
        for (size_t i = 0; i < 6 * row_floats && rows_ok; ++i) {
          const float want = (i < 4 * row_floats ? 100.f : 900.f) + float(i);
          rows_ok = k[i] == want && v[i] == -want;
        }
        (void)kv2.release_layer(*c);
      }
      (void)kv2.abort_append(*q);
    }
    CHECK(ok && after_first.page_ins == 0 && after_first.bytes_out == 4 * row,
          "first step: nothing uploaded, the 4 written rows written back");
    CHECK(rows_ok, "a retried append's rows replace the aborted ones in the host copy");
    if (q) (void)kv2.release_sequence(*q);
  }
}

// ---------------------------------------------------------------------------
// GPU: attention slice on HIPBackend vs the oracle

static bool attn_close(const float *got, const float *want, size_t n, double *worst) {
  bool ok = true;
  *worst = 0;
  for (size_t i = 0; i < n; ++i) {
    const double e = std::fabs(double(got[i]) - double(want[i]));
    const double b = 1e-5 + 1e-4 * std::fabs(double(want[i]));
    if (e > b) ok = false;
    *worst = std::max(*worst, e - b);
  }
  return ok;
}

static void gpu_tests() {
  register_hip_backend();
  auto &reg = BackendRegistry::instance();
  reg.probe_all();
  auto created = reg.create("hip:0", {});
  CHECK(bool(created), "create hip:0");
  if (!created) return;
  auto *hip = static_cast<HIPBackend *>(created->get());
  CHECK(hip->device_type() == DeviceType::HIP && !hip->is_host(), "hip backend identity");

  oracle_set_workers(4);
  const int Hq = 16, Hkv = 8, D = 128, L = 2, P = 37, N = 5;
  const size_t cap = P + N + 1;  // one spare row for the bad-position check
  AttentionSliceParams sp;  // Qwen3-0.6B attention shape
  std::vector<KVLayerSpec> specs(L, KVLayerSpec{size_t(Hkv), size_t(D), size_t(D)});
  std::vector<Backend *> place(L, hip);
  KVCacheManager kv(std::make_unique<ContiguousKVStrategy>(std::make_unique<NaiveKVStorage>()));
  CHECK(kv.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = cap}), "kv init on hip");
  auto sid = kv.create_sequence();
  CHECK(bool(sid), "sequence with HBM caches");
  CHECK(hip->reserve_decode_workspace(Hq, Hkv, D, cap), "reserve decode workspace");

  Rng rng(0x1F0000 + 7);
  auto upload = [&](const std::vector<float> &h, std::initializer_list<int64_t> shape, const char *name) {
    auto t = std::make_unique<Tensor>(name, GGML_TYPE_F32, shape);
    t->data = *hip->alloc(BufferKind::WEIGHTS, t->byte_size());
    t->backend = hip;
    t->device = DeviceType::HIP;
    t->tensorRole = TensorRole::TENSOR_ROLE_WEIGHT;
    hip->copy_tensor_set(t.get(), h.data(), 0, h.size() * 4);
    return t;
  };
  std::vector<std::vector<float>> qw(L), kw(L);
  std::vector<std::unique_ptr<Tensor>> qw_d, kw_d;
  for (int l = 0; l < L; ++l) {
    qw[l] = rng.normal(D, 0.5);
    kw[l] = rng.normal(D, 0.5);
    for (auto &x : qw[l]) x += 1.0f;
    for (auto &x : kw[l]) x += 1.0f;
    qw_d.push_back(upload(qw[l], {D, 1, 1, 1}, "q_norm_w"));
    kw_d.push_back(upload(kw[l], {D, 1, 1, 1}, "k_norm_w"));
  }

  // oracle state: host caches per layer
  std::vector<std::vector<float>> hk(L, std::vector<float>(cap * Hkv * D)), hv = hk;
  std::vector<float> theta(size_t(64) * sp.n_ctx_train);
  oracle_rope_theta_table(sp.rope_theta, D, sp.n_ctx_train, theta.data());

  Scheduler sched(hip);
  GraphContext ctx(nullptr);
  CHECK(ctx.set_kv_cache(&kv, *sid), "bind context");
  Tensor *pos_t = ctx.make_tensor("inp_pos", GGML_TYPE_I32, {1});
  pos_t->device = DeviceType::CPU;
  pos_t->tensorRole = TensorRole::TNESOR_ROLE_INPUT;
  ctx.set_input_pos(pos_t);
  std::vector<int32_t> pos;

  size_t n_past = 0;
  for (int step = 0; step <= N; ++step) {
    const int n = step == 0 ? P : 1;
    const std::string tag = step == 0 ? "prefill" : "decode step " + std::to_string(step);
    pos.resize(n);
    for (int i = 0; i < n; ++i) pos[i] = int32_t(n_past + i);
    pos_t->dims = {n, 1, 1, 1};
    pos_t->set_contiguous_strides();
    pos_t->data = pos.data();
    if (!kv.reserve_append(*sid, n)) {
      CHECK(false, "reserve");
      return;
    }
    Graph g;
    std::vector<std::unique_ptr<Tensor>> inputs;
    std::vector<std::vector<float>> hq(L), hkp(L), hvp(L);
    std::vector<Tensor *> outs;
    for (int l = 0; l < L; ++l) {
      hq[l] = rng.normal(size_t(n) * Hq * D);
      hkp[l] = rng.normal(size_t(n) * Hkv * D);
      hvp[l] = rng.normal(size_t(n) * Hkv * D);
      inputs.push_back(upload(hq[l], {Hq * D, n, 1, 1}, "q_proj"));
      inputs.push_back(upload(hkp[l], {Hkv * D, n, 1, 1}, "k_proj"));
      inputs.push_back(upload(hvp[l], {Hkv * D, n, 1, 1}, "v_proj"));
      auto out = build_attention_slice(g, ctx, inputs[3 * l].get(), inputs[3 * l + 1].get(),
                                       inputs[3 * l + 2].get(), qw_d[l].get(), kw_d[l].get(), l, sp);
      if (!out) {
        CHECK(false, ("build slice " + tag).c_str());
        return;
      }
      g.mark_output(*out);
      outs.push_back(*out);
    }
    auto ex = sched.execute(g);
    auto sy = hip->synchronize();
    CHECK(ex && sy, ("execute " + tag).c_str());
    const auto &stt = hip->last_stats();
    // prefill: qk-norm + RoPE fused per q and k; decode: qk-norm + RoPE and
    // the append folded into the decode launch
    CHECK(step == 0 ? stt.fused_norm_rope == 2 * L && stt.fused_append_decode == 0
                    : stt.fused_norm_rope == 0 && stt.fused_append_decode == L &&
                          stt.fused_rope_decode == L,
          ("fusions " + tag).c_str());

    for (int l = 0; l < L; ++l) {
      // oracle: qk-norm -> rope -> append -> attention
      std::vector<float> qn(hq[l].size()), kn(hkp[l].size()), qr(hq[l].size()), kr(hkp[l].size());
      oracle_rms_norm_f32(hq[l].data(), qw[l].data(), qn.data(), int64_t(n) * Hq, D, sp.rms_norm_eps);
      oracle_rms_norm_f32(hkp[l].data(), kw[l].data(), kn.data(), int64_t(n) * Hkv, D, sp.rms_norm_eps);
      oracle_rope_neox_f32(qn.data(), pos.data(), theta.data(), sp.n_ctx_train, qr.data(), D, Hq, n);
      oracle_rope_neox_f32(kn.data(), pos.data(), theta.data(), sp.n_ctx_train, kr.data(), D, Hkv, n);
      oracle_cpy(hk[l].data() + n_past * Hkv * D, kr.data(), kr.size() * 4);
      oracle_cpy(hv[l].data() + n_past * Hkv * D, hvp[l].data(), hvp[l].size() * 4);
      std::vector<float> want(size_t(n) * Hq * D), got(want.size());
      oracle_flash_attn_f32(qr.data(), hk[l].data(), hv[l].data(), want.data(), D, Hq, n, Hkv,
                            int64_t(n_past + n), int64_t(n_past));
      hip->copy_tensor_get(outs[l], got.data(), 0, got.size() * 4);
      double worst;
      const bool ok = attn_close(got.data(), want.data(), got.size(), &worst);
      if (!ok) std::printf("  layer %d worst excess %.3e\n", l, worst);
      CHECK(ok, ("attention within tolerance, layer " + std::to_string(l) + ", " + tag).c_str());
      // cache bytes: committed prefix + this step's rows, K and V
      const StorageState *ss = kv.strategy()->storage()->state(StorageId(l + 1));
      const size_t bytes = (n_past + n) * Hkv * D * 4;
      std::vector<float> dk(bytes / 4), dv(bytes / 4);
      (void)hipMemcpy(dk.data(), ss->object.k_base, bytes, hipMemcpyDeviceToHost);
      (void)hipMemcpy(dv.data(), ss->object.v_base, bytes, hipMemcpyDeviceToHost);
      CHECK(std::memcmp(dk.data(), hk[l].data(), bytes) == 0 && std::memcmp(dv.data(), hv[l].data(), bytes) == 0,
            ("cache bit-exact, layer " + std::to_string(l) + ", " + tag).c_str());
    }
    CHECK(ctx.release_kv_access() && kv.commit_append(*sid) && *kv.length(*sid) == n_past + n,
          ("commit " + tag).c_str());
    for (auto &t : inputs) hip->free(BufferKind::WEIGHTS, t->data);
    n_past += n;
  }

  // A position beyond the angle table is reported at synchronize (no fault).
  {
    AttentionSliceParams small = sp;
    small.n_ctx_train = 16;  // table of 16 positions; the next position is 42
    if (kv.reserve_append(*sid, 1)) {
      Graph g;
      pos.assign(1, int32_t(n_past));
      pos_t->dims = {1, 1, 1, 1};
      pos_t->set_contiguous_strides();
      pos_t->data = pos.data();
      auto q = upload(rng.normal(Hq * D), {Hq * D, 1, 1, 1}, "q");
      auto k = upload(rng.normal(Hkv * D), {Hkv * D, 1, 1, 1}, "k");
      auto v = upload(rng.normal(Hkv * D), {Hkv * D, 1, 1, 1}, "v");
      auto out = build_attention_slice(g, ctx, q.get(), k.get(), v.get(), qw_d[0].get(), kw_d[0].get(), 0, small);
      if (out) g.mark_output(*out);
      auto ex = out ? sched.execute(g) : infer::expected<void, std::error_code>(infer::fail(std::errc::io_error));
      auto sy = hip->synchronize();
      CHECK(ex && !sy && is_err(sy.error(), std::errc::invalid_argument), "bad RoPE position reported, no fault");
      CHECK(hip->synchronize(), "status cleared after report");
      ctx.release_kv_access();
      kv.abort_append(*sid);
      for (auto *t : {q.get(), k.get(), v.get()}) hip->free(BufferKind::WEIGHTS, t->data);
    } else {
      CHECK(false, "reserve for bad-position check");
    }
  }
  CHECK(kv.release_sequence(*sid), "release sequence (frees HBM caches)");
  for (auto &t : qw_d) hip->free(BufferKind::WEIGHTS, t->data);
  for (auto &t : kw_d) hip->free(BufferKind::WEIGHTS, t->data);
  host_copy_gpu_tests(hip);
  producer_cache_gpu_tests(hip);
  offload_gpu_tests(hip);
}

// copy_tensor_set: small copies (up to 256 bytes) travel in a kernel's
// arguments, larger ones through hipMemcpyAsync. At sizes either side of
// that bound and at unaligned offsets, the device bytes equal the host's,
// the bytes around the range are untouched, and the host buffer may be
// overwritten at once after the call (the copy took its bytes at launch).
static void host_copy_gpu_tests(HIPBackend *hip) {
  const size_t n = 4096;
  Tensor t("host_copy", GGML_TYPE_I32, {int64_t(n / 4)});
  t.data = *hip->alloc(BufferKind::ACTIVATION, n);
  t.backend = hip;
  t.device = DeviceType::HIP;
  std::vector<unsigned char> fill(n, 0xA5), back(n);
  bool ok = bool(hip->copy_tensor_set(&t, fill.data(), 0, n));
  std::vector<unsigned char> want = fill;
  unsigned char v = 1;
  for (const auto &[off, len] : std::vector<std::pair<size_t, size_t>>{
           {3, 1}, {17, 255}, {300, 256}, {700, 257}, {1101, 1000}, {2500, 4}}) {
    std::vector<unsigned char> src(len);
    for (auto &b : src) b = v++;
    ok = ok && bool(hip->copy_tensor_set(&t, src.data(), off, len));
    std::copy(src.begin(), src.end(), want.begin() + off);
    std::fill(src.begin(), src.end(), 0);  // the call must not read it later
  }
  ok = ok && bool(hip->synchronize()) && bool(hip->copy_tensor_get(&t, back.data(), 0, n));
  CHECK(ok && back == want, "copy_tensor_set: kernel-argument and memcpy sizes, unaligned offsets");
  CHECK(!hip->copy_tensor_set(&t, fill.data(), n - 8, 16), "copy_tensor_set past the tensor is rejected");
  hip->free(BufferKind::ACTIVATION, t.data);
}

// The prefill rows a layer's projections write straight into the cache (the
// k projection through qk-norm + RoPE, the v projection as is): with the
// fusions on, the producers write the cache rows themselves; with them off,
// each result lands in an activation and a CPY copies it. The cache bytes
// must be equal bit for bit, at prompt lengths that run the projections on
// the few-token MFMA kernel (20), the mid-size path (70) and this build's
// GEMM (2048).
static void producer_cache_gpu_tests(HIPBackend *hip) {
  const int Hq = 16, Hkv = 8, D = 128, E = 1024;
  AttentionSliceParams sp;
  Rng rng(0x1F0000 + 77);
  auto upload = [&](const std::vector<float> &h, std::initializer_list<int64_t> shape, const char *name) {
    auto t = std::make_unique<Tensor>(name, GGML_TYPE_F32, shape);
    t->data = *hip->alloc(BufferKind::WEIGHTS, t->byte_size());
    t->backend = hip;
    t->device = DeviceType::HIP;
    t->tensorRole = TensorRole::TENSOR_ROLE_WEIGHT;
    hip->copy_tensor_set(t.get(), h.data(), 0, h.size() * 4);
    return t;
  };
  auto wq = upload(rng.normal(size_t(Hq) * D * E, 0.02), {E, Hq * D, 1, 1}, "wq");
  auto wk = upload(rng.normal(size_t(Hkv) * D * E, 0.02), {E, Hkv * D, 1, 1}, "wk");
  auto wv = upload(rng.normal(size_t(Hkv) * D * E, 0.02), {E, Hkv * D, 1, 1}, "wv");
  std::vector<float> ones(D, 1.0f);
  auto qnw = upload(ones, {D, 1, 1, 1}, "q_norm_w");
  auto knw = upload(ones, {D, 1, 1, 1}, "k_norm_w");
  for (const int P : {20, 70, 2048}) {
    std::vector<std::vector<float>> k_bytes(2), v_bytes(2);
    auto xh = rng.normal(size_t(P) * E);
    auto x = upload(xh, {E, P, 1, 1}, "x");
    for (int fused = 1; fused >= 0; --fused) {
      const std::string tag = "P=" + std::to_string(P) + (fused ? " fused" : " unfused");
      hip->set_fusion(fused != 0);
      std::vector<KVLayerSpec> specs(1, KVLayerSpec{size_t(Hkv), size_t(D), size_t(D)});
      std::vector<Backend *> place(1, hip);
      KVCacheManager kv(std::make_unique<ContiguousKVStrategy>(std::make_unique<NaiveKVStorage>()));
      CHECK(kv.init(specs, place, KVCacheConfig{.layers = 1, .max_tokens_per_sequence = size_t(P)}),
            ("kv init " + tag).c_str());
      auto sid = kv.create_sequence();
      if (!sid || !kv.reserve_append(*sid, P)) {
        CHECK(false, ("sequence " + tag).c_str());
        return;
      }
      GraphContext ctx(nullptr);
      CHECK(ctx.set_kv_cache(&kv, *sid), ("bind " + tag).c_str());
      std::vector<int32_t> pos(P);
      for (int i = 0; i < P; ++i) pos[i] = i;
      Tensor *pos_t = ctx.make_tensor("inp_pos", GGML_TYPE_I32, {P});
      pos_t->device = DeviceType::CPU;
      pos_t->tensorRole = TensorRole::TNESOR_ROLE_INPUT;
      pos_t->data = pos.data();
      ctx.set_input_pos(pos_t);
      Graph g;
      Tensor *q = OpFactory::mul_mat(g, wq.get(), x.get(), "q_proj");
      Tensor *k = OpFactory::mul_mat(g, wk.get(), x.get(), "k_proj");
      Tensor *v = OpFactory::mul_mat(g, wv.get(), x.get(), "v_proj");
      auto out = build_attention_slice(g, ctx, q, k, v, qnw.get(), knw.get(), 0, sp);
      CHECK(bool(out), ("build " + tag).c_str());
      if (!out) return;
      g.mark_output(*out);
      Scheduler sched(hip);
      auto ex = sched.execute(g);
      auto sy = hip->synchronize();
      CHECK(ex && sy, ("execute " + tag).c_str());
      const StorageState *ss = kv.strategy()->storage()->state(StorageId(1));
      const size_t bytes = size_t(P) * Hkv * D * 4;
      k_bytes[fused].resize(bytes / 4);
      v_bytes[fused].resize(bytes / 4);
      (void)hipMemcpy(k_bytes[fused].data(), ss->object.k_base, bytes, hipMemcpyDeviceToHost);
      (void)hipMemcpy(v_bytes[fused].data(), ss->object.v_base, bytes, hipMemcpyDeviceToHost);
      if (fused) {
        const auto &st = hip->last_stats();
        CHECK(st.fused_append == 2, ("producers write the cache rows, " + tag).c_str());
      }
      ctx.release_kv_access();
      (void)kv.abort_append(*sid);
      (void)kv.release_sequence(*sid);
    }
    const size_t bytes = size_t(P) * Hkv * D * 4;
    CHECK(std::memcmp(k_bytes[0].data(), k_bytes[1].data(), bytes) == 0,
          ("K rows written by the RoPE producer equal the copied ones, P=" + std::to_string(P)).c_str());
    CHECK(std::memcmp(v_bytes[0].data(), v_bytes[1].data(), bytes) == 0,
          ("V rows written by the v projection equal the copied ones, P=" + std::to_string(P)).c_str());
    hip->free(BufferKind::WEIGHTS, x->data);
  }
  hip->set_fusion(true);
  for (auto *t : {wq.get(), wk.get(), wv.get(), qnw.get(), knw.get()}) hip->free(BufferKind::WEIGHTS, t->data);
}

// Two sequences on an offloaded cache whose HBM budget holds one sequence's
// layers: every switch writes the rows the other sequence's last step wrote
// back to pinned host memory and uploads this one's committed rows. Attention within tolerance of the
// oracle and cache rows bit-exact, after every switch.
static void offload_gpu_tests(HIPBackend *hip) {
  const int Hq = 16, Hkv = 8, D = 128, L = 2, P = 21, N = 3;
  const size_t cap = P + N;
  const size_t layer_bytes = cap * Hkv * D * 4 * 2;
  AttentionSliceParams sp;
  std::vector<KVLayerSpec> specs(L, KVLayerSpec{size_t(Hkv), size_t(D), size_t(D)});
  std::vector<Backend *> place(L, hip);
  PinnedHostBackend host(0);
  OffloadKVStorageConfig oc;
  oc.host_backend = &host;
  oc.device_budgets.push_back({.backend = hip, .resident_bytes = L * layer_bytes, .prefetch_bytes = 0});
  auto owner = std::make_unique<OffloadKVStorage>(std::move(oc), std::make_unique<LRUKVEvictionPolicy>(),
                                                  std::make_unique<NoKVPrefetchPolicy>());
  OffloadKVStorage *st = owner.get();
  KVCacheManager kv(std::make_unique<ContiguousKVStrategy>(std::move(owner)));
  CHECK(kv.init(specs, place, KVCacheConfig{.layers = L, .max_tokens_per_sequence = cap}), "offload kv init on hip");
  CHECK(hip->reserve_decode_workspace(Hq, Hkv, D, cap), "offload: workspace");
  Rng rng(0x1F0000 + 9);
  std::vector<std::unique_ptr<Tensor>> owned;
  auto upload = [&](const std::vector<float> &h, std::initializer_list<int64_t> shape) {
    auto t = std::make_unique<Tensor>("t", GGML_TYPE_F32, shape);
    t->data = *hip->alloc(BufferKind::WEIGHTS, t->byte_size());
    t->backend = hip;
    t->device = DeviceType::HIP;
    t->tensorRole = TensorRole::TENSOR_ROLE_WEIGHT;
    hip->copy_tensor_set(t.get(), h.data(), 0, h.size() * 4);
    return t;
  };
  std::vector<std::vector<float>> qw(L), kw(L);
  std::vector<std::unique_ptr<Tensor>> qw_d, kw_d;
  for (int l = 0; l < L; ++l) {
    qw[l] = rng.normal(D, 0.5);
    kw[l] = rng.normal(D, 0.5);
    qw_d.push_back(upload(qw[l], {D, 1, 1, 1}));
    kw_d.push_back(upload(kw[l], {D, 1, 1, 1}));
  }
  std::vector<float> theta(size_t(64) * sp.n_ctx_train);
  oracle_rope_theta_table(sp.rope_theta, D, sp.n_ctx_train, theta.data());
  struct Seq {
    SequenceId sid = kInvalidSequenceId;
    size_t n_past = 0;
    std::vector<std::vector<float>> hk, hv;
  };
  Seq seqs[2];
  for (auto &q : seqs) {
    auto sid = kv.create_sequence();
    q.sid = sid ? *sid : kInvalidSequenceId;
    q.hk.assign(L, std::vector<float>(cap * Hkv * D, 0.f));
    q.hv = q.hk;
  }
  Scheduler sched(hip);
  bool all_ok = seqs[0].sid != kInvalidSequenceId && seqs[1].sid != kInvalidSequenceId;
  // Transfers the valid-row rules imply: a step evicts the other sequence's
  // layers, each writing back the rows that sequence's last step wrote, and
  // uploads this sequence's committed rows (none on its first step).
  const size_t row = size_t(Hkv) * D * 4 * 2;
  size_t want_in = 0, want_out = 0, want_page_ins = 0, last_n[2] = {0, 0};
  bool first_step = true;
  for (int round = 0; round <= N && all_ok; ++round) {
    for (Seq &q : seqs) {
      const int n = round == 0 ? P : 1;
      const size_t qi = size_t(&q - seqs);
      if (!first_step) want_out += L * last_n[1 - qi] * row;
      if (q.n_past > 0) {
        want_in += L * q.n_past * row;
        want_page_ins += L;
      }
      first_step = false;
      last_n[qi] = size_t(n);
      GraphContext ctx(nullptr);
      Tensor *pos_t = ctx.make_tensor("inp_pos", GGML_TYPE_I32, {n});
      pos_t->device = DeviceType::CPU;
      pos_t->tensorRole = TensorRole::TNESOR_ROLE_INPUT;
      ctx.set_input_pos(pos_t);
      std::vector<int32_t> pos(n);
      for (int i = 0; i < n; ++i) pos[i] = int32_t(q.n_past + i);
      pos_t->data = pos.data();
      if (!ctx.set_kv_cache(&kv, q.sid) || !kv.reserve_append(q.sid, n)) {
        all_ok = false;
        break;
      }
      Graph g;
      std::vector<std::vector<float>> hq(L), hkp(L), hvp(L);
      std::vector<std::unique_ptr<Tensor>> in;
      std::vector<Tensor *> outs;
      for (int l = 0; l < L && all_ok; ++l) {
        hq[l] = rng.normal(size_t(n) * Hq * D);
        hkp[l] = rng.normal(size_t(n) * Hkv * D);
        hvp[l] = rng.normal(size_t(n) * Hkv * D);
        in.push_back(upload(hq[l], {Hq * D, n, 1, 1}));
        in.push_back(upload(hkp[l], {Hkv * D, n, 1, 1}));
        in.push_back(upload(hvp[l], {Hkv * D, n, 1, 1}));
        auto out = build_attention_slice(g, ctx, in[3 * l].get(), in[3 * l + 1].get(), in[3 * l + 2].get(),
                                         qw_d[l].get(), kw_d[l].get(), l, sp);
        if (!out) all_ok = false;
        else {
          g.mark_output(*out);
          outs.push_back(*out);
        }
      }
      all_ok = all_ok && sched.execute(g) && hip->synchronize();
      for (int l = 0; l < L && all_ok; ++l) {
        std::vector<float> qn(hq[l].size()), kn(hkp[l].size()), qr(hq[l].size()), kr(hkp[l].size());
        oracle_rms_norm_f32(hq[l].data(), qw[l].data(), qn.data(), int64_t(n) * Hq, D, sp.rms_norm_eps);
        oracle_rms_norm_f32(hkp[l].data(), kw[l].data(), kn.data(), int64_t(n) * Hkv, D, sp.rms_norm_eps);
        oracle_rope_neox_f32(qn.data(), pos.data(), theta.data(), sp.n_ctx_train, qr.data(), D, Hq, n);
        oracle_rope_neox_f32(kn.data(), pos.data(), theta.data(), sp.n_ctx_train, kr.data(), D, Hkv, n);
        oracle_cpy(q.hk[l].data() + q.n_past * Hkv * D, kr.data(), kr.size() * 4);
        oracle_cpy(q.hv[l].data() + q.n_past * Hkv * D, hvp[l].data(), hvp[l].size() * 4);
        std::vector<float> want(size_t(n) * Hq * D), got(want.size());
        oracle_flash_attn_f32(qr.data(), q.hk[l].data(), q.hv[l].data(), want.data(), D, Hq, n, Hkv,
                              int64_t(q.n_past + n), int64_t(q.n_past));
        hip->copy_tensor_get(outs[l], got.data(), 0, got.size() * 4);
        double worst;
        all_ok = attn_close(got.data(), want.data(), got.size(), &worst);
        if (!all_ok) std::printf("  offload round %d layer %d worst excess %.3e\n", round, l, worst);
        // the HBM copy this step used holds the committed rows, bit for bit
        const size_t bytes = (q.n_past + n) * Hkv * D * 4;
        std::vector<float> dk(bytes / 4), dv(bytes / 4);
        const StorageState *ss = st->state(StorageId(1 + (&q - seqs) * L + l));
        (void)hipMemcpy(dk.data(), ss->object.k_base, bytes, hipMemcpyDeviceToHost);
        (void)hipMemcpy(dv.data(), ss->object.v_base, bytes, hipMemcpyDeviceToHost);
        all_ok = all_ok && std::memcmp(dk.data(), q.hk[l].data(), bytes) == 0 &&
                 std::memcmp(dv.data(), q.hv[l].data(), bytes) == 0;
      }
      all_ok = all_ok && ctx.release_kv_access() && kv.commit_append(q.sid);
      q.n_past += n;
      for (auto &t : in) hip->free(BufferKind::WEIGHTS, t->data);
    }
  }
  const OffloadStats &os = st->stats();
  CHECK(all_ok, "offload: two sequences in one sequence's HBM, attention and caches exact at every switch");
  CHECK(os.evictions == size_t(2 * N + 1) * L && os.page_outs == os.evictions && os.page_ins == want_page_ins &&
            os.bytes_in == want_in && os.bytes_out == want_out,
        "offload: every switch wrote back only the rows written since the upload and uploaded only "
        "committed rows");
  for (auto &q : seqs)
    if (q.sid != kInvalidSequenceId) (void)kv.release_sequence(q.sid);
  CHECK(st->resident_bytes(hip) == 0, "offload: released sequences leave nothing in HBM");
  for (auto &t : qw_d) hip->free(BufferKind::WEIGHTS, t->data);
  for (auto &t : kw_d) hip->free(BufferKind::WEIGHTS, t->data);
}

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "--cpu";
  if (mode == "--cpu") cpu_tests();
  else if (mode == "--gpu") gpu_tests();
  else {
    std::fprintf(stderr, "usage: test_engine --cpu | --gpu\n");
    return 2;
  }
  std::printf("%s: %d failure(s)\n", mode.c_str(), g_fail);
  return g_fail;
}
