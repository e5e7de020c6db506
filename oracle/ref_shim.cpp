// Driver around the compiled reference sampler (verbo::Sampler, reference src/sampler.cpp).
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with the reference's own
// sources, read in place from the reference tree, into oracle/_ref/libvref.so. The library is used
// to pin the oracle (golden fixtures, direct comparisons) and as the bench's CPU baseline
// ("kind": "reference"). It calls only the reference's public C++ API
// (include/verbo/verbo.hpp:56-64,116-132): Sampler(Sampling), accept, pick.
#include <atomic>
#include <chrono>
#include <thread>
#include <vector>

#include "verbo/verbo.hpp"

#define VREF_API extern "C" __attribute__((visibility("default")))

namespace {

using clk = std::chrono::steady_clock;

void run_rows(const float* logits, int V, long long ld, const verbo::Sampling* cfgs, int per_row, const int* hist,
              const int* hist_off, int* out, int r0, int r1) {
  for (int r = r0; r < r1; ++r) {
    verbo::Sampler s(cfgs[per_row ? r : 0]);
    if (hist && hist_off) {
      for (int i = hist_off[r]; i < hist_off[r + 1]; ++i) s.accept(hist[i]);
    }
    out[r] = s.pick(logits + static_cast<std::size_t>(r) * static_cast<std::size_t>(ld), V);
  }
}

}  // namespace

// One reference Sampler: accept hist[0..H), then n_picks picks on the same logits; with
// accept_each the picked id is accepted before the next pick. Returns 0.
VREF_API int vref_sampler_run(const float* logits, int n, const verbo::Sampling* cfg, const int* hist, int H,
                              int n_picks, int accept_each, int* out) {
  verbo::Sampler s(*cfg);
  for (int i = 0; i < H; ++i) s.accept(hist[i]);
  for (int p = 0; p < n_picks; ++p) {
    out[p] = s.pick(logits, n);
    if (accept_each) s.accept(out[p]);
  }
  return 0;
}

// B independent reference Samplers, one pick each (row r: params[per_row ? r : 0], history
// hist[hist_off[r]..hist_off[r+1]) accepted first). Rows are split over `threads` threads.
VREF_API int vref_pick_rows(const float* logits, int B, int V, long long ld, const verbo::Sampling* cfgs,
                            int per_row, const int* hist, const int* hist_off, int* out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > B) threads = B;
  std::vector<std::thread> th;
  for (int t = 0; t < threads; ++t) {
    const int r0 = static_cast<int>(static_cast<long long>(B) * t / threads);
    const int r1 = static_cast<int>(static_cast<long long>(B) * (t + 1) / threads);
    th.emplace_back(run_rows, logits, V, ld, cfgs, per_row, hist, hist_off, out, r0, r1);
  }
  for (auto& x : th) x.join();
  return 0;
}

// CPU-baseline timing: each of `threads` threads owns a static share of the B rows, builds one
// Sampler per row (history accepted, outside the timer), then all threads call pick() on their
// rows round-robin until `budget_s` seconds of wall time have passed. Returns the wall seconds of
// the timed region and stores the number of picks done in *picks.
VREF_API double vref_time_rows(const float* logits, int B, int V, long long ld, const verbo::Sampling* cfgs,
                               int per_row, const int* hist, const int* hist_off, int threads, double budget_s,
                               long long* picks) {
  if (threads < 1) threads = 1;
  if (threads > B) threads = B;
  std::atomic<int> ready{0};
  std::atomic<bool> go{false};
  std::atomic<long long> done{0};
  std::vector<std::thread> th;
  clk::time_point t0;
  for (int t = 0; t < threads; ++t) {
    const int r0 = static_cast<int>(static_cast<long long>(B) * t / threads);
    const int r1 = static_cast<int>(static_cast<long long>(B) * (t + 1) / threads);
    th.emplace_back([&, r0, r1]() {
      std::vector<verbo::Sampler> smp;
      smp.reserve(static_cast<std::size_t>(r1 - r0));
      for (int r = r0; r < r1; ++r) {
        smp.emplace_back(cfgs[per_row ? r : 0]);
        if (hist && hist_off) {
          for (int i = hist_off[r]; i < hist_off[r + 1]; ++i) smp.back().accept(hist[i]);
        }
      }
      ready.fetch_add(1);
      while (!go.load()) std::this_thread::yield();
      long long n = 0;
      const auto end = t0 + std::chrono::duration_cast<clk::duration>(std::chrono::duration<double>(budget_s));
      for (;;) {
        for (int r = r0; r < r1; ++r) {
          volatile int id = smp[static_cast<std::size_t>(r - r0)].pick(
              logits + static_cast<std::size_t>(r) * static_cast<std::size_t>(ld), V);
          (void)id;
          ++n;
        }
        if (clk::now() >= end) break;
      }
      done.fetch_add(n);
    });
  }
  while (ready.load() < threads) std::this_thread::yield();
  t0 = clk::now();
  go.store(true);
  for (auto& x : th) x.join();
  const double s = std::chrono::duration<double>(clk::now() - t0).count();
  *picks = done.load();
  return s;
}

// One reference verbo::Sampler behind a handle, for recorders that interleave picks and accepts
// across several samplers (the batched decode golden).
VREF_API void* vref_sampler_new(const verbo::Sampling* cfg) { return new verbo::Sampler(*cfg); }
VREF_API void vref_sampler_free(void* s) { delete static_cast<verbo::Sampler*>(s); }
VREF_API void vref_sampler_accept(void* s, int tok) { static_cast<verbo::Sampler*>(s)->accept(tok); }
VREF_API int vref_sampler_pick(void* s, const float* logits, int n) {
  return static_cast<verbo::Sampler*>(s)->pick(logits, n);
}
