// HipNetwork adapter under concurrent callers and injected failures, on the
// CPU fake of the C ABI (mfh_fake.cpp) -- TEST INFRASTRUCTURE ONLY.  Built
// with -fsanitize=thread by tests/test_sanitizers.py.
//
// * Eight threads call EvaluateBatch (and EvaluateBatchPriors) on one net at
//   once, as MCTS workers do (reference src/mcts/search.cpp:433,
//   backend_adapter.cpp:244-276); every result must equal the serial one bit
//   for bit, and ThreadSanitizer must see no race on the adapter's shared
//   output buffers.
// * One failed call or one non-finite result is retried; a second one throws
//   std::runtime_error (reference cuda_network.cpp:199-231, 444-458).
// Prints "adapter concurrency ok" and exits 0 on success.
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "hip_network.h"

extern "C" {
void mfh_fake_fail_next(int n);
void mfh_fake_nan_next(int n);
int mfh_fake_eval_calls(void);
}

using namespace MetalFish::NN;

namespace {

int g_failures = 0;

void Check(bool ok, const char *what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++g_failures;
  }
}

// Seeded planes: 0/1 piece planes, a rule-50 count and an all-ones plane.
std::vector<InputPlanes> MakeSet(int n, std::uint32_t seed) {
  std::vector<InputPlanes> set(static_cast<std::size_t>(n));
  std::uint32_t s = seed * 2654435761u + 1u;
  for (auto &planes : set) {
    for (auto &plane : planes)
      plane.fill(0.0f);
    for (int p = 0; p < 104; ++p)
      for (int sq = 0; sq < 64; ++sq) {
        s = s * 1664525u + 1013904223u;
        if ((s >> 27) == 0)
          planes[p][sq] = 1.0f;
      }
    s = s * 1664525u + 1013904223u;
    planes[109].fill(static_cast<float>(s >> 26));
    planes[111].fill(1.0f);
  }
  return set;
}

bool Same(const NetworkOutput &a, const NetworkOutput &b) {
  return std::memcmp(a.policy.data(), b.policy.data(), sizeof(float) * kPolicyOutputs) == 0 &&
         std::memcmp(a.wdl, b.wdl, sizeof(a.wdl)) == 0 && a.value == b.value &&
         a.has_wdl == b.has_wdl;
}

bool SameAll(const std::vector<NetworkOutput> &a, const std::vector<NetworkOutput> &b) {
  if (a.size() != b.size())
    return false;
  for (std::size_t i = 0; i < a.size(); ++i)
    if (!Same(a[i], b[i]))
      return false;
  return true;
}

bool SamePriors(const std::vector<Hip::PriorsOutput> &a, const std::vector<Hip::PriorsOutput> &b) {
  if (a.size() != b.size())
    return false;
  for (std::size_t i = 0; i < a.size(); ++i)
    if (a[i].priors != b[i].priors || a[i].value != b[i].value ||
        std::memcmp(a[i].wdl, b[i].wdl, sizeof(a[i].wdl)) != 0)
      return false;
  return true;
}

}  // namespace

int main() {
  Hip::HipNetworkConfig config;
  config.headcount = 8;
  config.max_batch = 8;  // 13-position sets run as chunks of 8 + 5
  Hip::HipNetwork net(std::vector<Hip::WeightTensor>{}, config);
  Check(net.GetBackendCapabilities().actual_backend == "hip", "actual_backend");

  constexpr int kSets = 6, kThreads = 8, kIters = 20;
  std::vector<std::vector<InputPlanes>> sets;
  std::vector<std::vector<NetworkOutput>> serial;
  std::vector<std::vector<std::vector<std::int16_t>>> moves;
  std::vector<std::vector<Hip::PriorsOutput>> serial_priors;
  for (int i = 0; i < kSets; ++i) {
    sets.push_back(MakeSet(13, 100 + i));
    serial.push_back(net.EvaluateBatch(sets.back()));
    std::vector<std::vector<std::int16_t>> m(13);
    for (int b = 0; b < 13; ++b)
      for (int k = 0; k < 20 + b; ++k)
        m[b].push_back(static_cast<std::int16_t>((b * 97 + k * 31 + i) % 1858));
    moves.push_back(m);
    serial_priors.push_back(net.EvaluateBatchPriors(sets.back(), m, 1.4f));
  }
  // Serial repeats are deterministic.
  Check(SameAll(net.EvaluateBatch(sets[0]), serial[0]), "serial repeat");

  std::atomic<int> mismatches{0};
  std::vector<std::thread> threads;
  for (int t = 0; t < kThreads; ++t)
    threads.emplace_back([&, t]() {
      for (int it = 0; it < kIters; ++it) {
        const int s = (t + it) % kSets;
        if ((t + it) % 4 == 3) {
          if (!SamePriors(net.EvaluateBatchPriors(sets[s], moves[s], 1.4f), serial_priors[s]))
            mismatches.fetch_add(1);
        } else if (!SameAll(net.EvaluateBatch(sets[s]), serial[s])) {
          mismatches.fetch_add(1);
        }
        if (!Same(net.Evaluate(sets[s][3]), serial[s][3]))
          mismatches.fetch_add(1);
      }
    });
  for (auto &th : threads)
    th.join();
  Check(mismatches.load() == 0, "concurrent results equal serial results");

  // Retry: one injected non-finite result or failed call is retried once.
  const std::vector<InputPlanes> small(sets[1].begin(), sets[1].begin() + 5);
  const std::vector<NetworkOutput> want(serial[1].begin(), serial[1].begin() + 5);
  int calls = mfh_fake_eval_calls();
  mfh_fake_nan_next(1);
  Check(SameAll(net.EvaluateBatch(small), want), "retry after one non-finite result");
  Check(mfh_fake_eval_calls() == calls + 2, "one retry call after a non-finite result");
  calls = mfh_fake_eval_calls();
  mfh_fake_fail_next(1);
  Check(SameAll(net.EvaluateBatch(small), want), "retry after one failed call");
  Check(mfh_fake_eval_calls() == calls + 2, "one retry call after a failed call");
  // Twice in a row: the adapter gives up with std::runtime_error.
  bool threw = false;
  mfh_fake_nan_next(2);
  try {
    net.EvaluateBatch(small);
  } catch (const std::runtime_error &e) {
    threw = std::string(e.what()).find("invalid outputs") != std::string::npos;
  }
  Check(threw, "two non-finite results throw");
  threw = false;
  mfh_fake_fail_next(2);
  try {
    net.EvaluateBatch(small);
  } catch (const std::runtime_error &e) {
    threw = std::string(e.what()).find("injected device failure") != std::string::npos;
  }
  Check(threw, "two failed calls throw with the library's message");
  // The net still works afterwards.
  Check(SameAll(net.EvaluateBatch(sets[2]), serial[2]), "net usable after a throw");
  Check(net.EvaluateBatch({}).empty(), "empty batch gives an empty result");

  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("adapter concurrency ok\n");
  return 0;
}
