// Host model of the decode step's cross-workgroup protocol (std::atomic, one thread per
// workgroup), used by tests/test_protocol_model.py.
//
// What it models (transformer_amd/csrc/msdecode.hip, decode_step_kernel):
//   * exchange words: 64-bit (f32 value | 32-bit epoch tag), written with relaxed atomic
//     stores and polled with relaxed atomic loads; a word is valid iff its tag is the
//     step's epoch, never re-zeroed between steps;
//   * the epoch sequence of the host (Decoder.launch): 1, 2, ..., 0xFFFFFFFE, 1, ...;
//   * the end of a step: every workgroup takes an atomic max of (ordered value | ~index)
//     into a 64-bit key, then a fetch_add on a 32-bit arrival counter; the workgroup that
//     sees GR - 1 publishes the token and the status;
//   * the start of a step: workgroup 0 resets the counter and the key and writes a sentinel
//     status before it publishes anything ("reset" rule), or, as the kernel did before, the
//     counter is never reset and the publisher is the arrival with old % GR == GR - 1
//     ("modulo" rule, kept as the negative control).
// A step is one launch: all threads are joined before the next starts (kernel boundary).
//
// Usage: protocol_model <rule: reset|modulo> <GR> <steps> <counter preset> <key preset>
//                       <epoch preset> <seed>
// (the presets stand for what an earlier step or a non-zeroed workspace left behind)
// Prints one line per step: "step <i> epoch <e> publishers <n> token <t> expected <x> status <s>"
// and "ok" at the end when every step had exactly one publisher with the expected token,
// every gathered word carried the step's values and no stale word was accepted.
#include <atomic>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr uint32_t kUnfinished = 0x80000000u;
constexpr int kLayers = 3;

uint64_t argmax_key(float v, int idx) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (uint64_t(u) << 32) | uint64_t(0xffffffffu - uint32_t(idx));
}

// the device's 64-bit atomic max, as a compare-and-swap loop
void atomic_max(std::atomic<uint64_t>& a, uint64_t v) {
  uint64_t cur = a.load(std::memory_order_relaxed);
  while (cur < v && !a.compare_exchange_weak(cur, v, std::memory_order_relaxed)) {
  }
}

float as_float(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
uint32_t as_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// Output of workgroup w at layer l of step s, from the sum of the previous layer's vector.
float produce(int s, int l, int w, double prev_sum) {
  const double x = std::sin(0.37 * s + 1.3 * l + 0.11 * w) + 1e-3 * prev_sum;
  return float(x);
}

struct Shared {
  std::vector<std::atomic<uint64_t>> words;   // kLayers x GR exchange words
  std::atomic<uint32_t> status{0};
  std::atomic<uint32_t> counter{0};
  std::atomic<uint64_t> key{0};
  std::atomic<int32_t> out_token{-1};
  std::atomic<uint32_t> out_status{0};
  std::atomic<int> publishers{0};
  std::atomic<int> stale_accepted{0};
  explicit Shared(int n) : words(n) {
    for (auto& w : words) w.store(0);
  }
};

void workgroup(Shared& sh, bool reset_rule, int GR, int w, int step, uint32_t epoch, unsigned seed,
               std::vector<double>& expect_sums) {
  std::mt19937 rng(seed * 7919u + unsigned(w));
  auto jitter = [&]() {
    const int r = int(rng() % 8);
    for (int i = 0; i < r; ++i) std::this_thread::yield();
  };
  if (reset_rule && w == 0) {
    sh.counter.store(0, std::memory_order_relaxed);
    sh.key.store(0, std::memory_order_relaxed);
    sh.out_status.store(kUnfinished, std::memory_order_relaxed);
    std::atomic_thread_fence(std::memory_order_seq_cst);   // the kernel waits for completion
  }
  double prev = 0.0;
  for (int l = 0; l < kLayers; ++l) {
    jitter();
    const float y = produce(step, l, w, prev);
    sh.words[size_t(l) * GR + w].store((uint64_t(epoch) << 32) | as_bits(y), std::memory_order_relaxed);
    // gather the whole vector of layer l: poll until every tag is this step's epoch
    double sum = 0.0;
    for (int j = 0; j < GR; ++j) {
      uint64_t v;
      while (uint32_t((v = sh.words[size_t(l) * GR + j].load(std::memory_order_relaxed)) >> 32) != epoch)
        std::this_thread::yield();
      const float got = as_float(uint32_t(v));
      if (got != produce(step, l, j, l == 0 ? 0.0 : expect_sums[l - 1])) sh.stale_accepted.fetch_add(1);
      sum += got;
    }
    prev = sum;
  }
  // logits of this workgroup's vocabulary slice: one value, index w (ties resolve low)
  const float best = float(std::floor(std::cos(0.7 * step + 0.05 * w) * 4.0));
  atomic_max(sh.key, argmax_key(best, w));
  const uint32_t old = sh.counter.fetch_add(1, std::memory_order_relaxed);
  const bool last = reset_rule ? old == uint32_t(GR - 1) : (old % uint32_t(GR)) == uint32_t(GR - 1);
  if (last) {
    const uint64_t k = sh.key.load(std::memory_order_relaxed);
    sh.out_token.store(int32_t(0xffffffffu - uint32_t(k & 0xffffffffu)), std::memory_order_relaxed);
    sh.out_status.store(sh.status.load(std::memory_order_relaxed), std::memory_order_relaxed);
    sh.publishers.fetch_add(1);
    if (!reset_rule) sh.key.store(0, std::memory_order_relaxed);   // the old rule reset the key here
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 8) {
    std::fprintf(stderr, "usage: %s reset|modulo GR steps counter_preset key_preset epoch_preset seed\n", argv[0]);
    return 2;
  }
  const bool reset_rule = std::string(argv[1]) == "reset";
  const int GR = std::atoi(argv[2]);
  const int steps = std::atoi(argv[3]);
  const uint32_t counter_preset = uint32_t(std::strtoull(argv[4], nullptr, 0));
  const uint64_t key_preset = uint64_t(std::strtoull(argv[5], nullptr, 0));
  uint32_t epoch = uint32_t(std::strtoull(argv[6], nullptr, 0));
  const unsigned seed = unsigned(std::atoi(argv[7]));
  Shared sh(kLayers * GR);
  sh.counter.store(counter_preset);
  sh.key.store(key_preset);
  bool ok = true;
  for (int s = 0; s < steps; ++s) {
    epoch = (epoch % 0xFFFFFFFEu) + 1;   // Decoder.launch: 1 .. 0xFFFFFFFE, never 0
    // expected per-layer sums and argmax, computed serially
    std::vector<double> sums(kLayers);
    for (int l = 0; l < kLayers; ++l) {
      double t = 0.0;
      for (int w = 0; w < GR; ++w) t += produce(s, l, w, l == 0 ? 0.0 : sums[l - 1]);
      sums[l] = t;
    }
    int expect = -1;
    float bv = 0.f;
    for (int w = 0; w < GR; ++w) {
      const float b = float(std::floor(std::cos(0.7 * s + 0.05 * w) * 4.0));
      if (expect < 0 || b > bv) {
        bv = b;
        expect = w;
      }
    }
    sh.publishers.store(0);
    sh.out_token.store(-1);
    if (!reset_rule) sh.out_status.store(0);
    std::vector<std::thread> th;
    for (int w = 0; w < GR; ++w)
      th.emplace_back(workgroup, std::ref(sh), reset_rule, GR, w, s, epoch, seed + unsigned(s), std::ref(sums));
    for (auto& t : th) t.join();
    const int pubs = sh.publishers.load();
    const int tok = sh.out_token.load();
    const uint32_t st = sh.out_status.load();
    std::printf("step %d epoch %" PRIu32 " publishers %d token %d expected %d status %#" PRIx32 "\n", s, epoch, pubs,
                tok, expect, st);
    if (pubs != 1 || tok != expect || st != 0) ok = false;
  }
  if (sh.stale_accepted.load() != 0) {
    std::printf("stale words accepted: %d\n", sh.stale_accepted.load());
    ok = false;
  }
  std::printf("%s\n", ok ? "ok" : "FAILED");
  return ok ? 0 : 1;
}
