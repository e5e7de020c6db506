// Drop-in verbo::Sampler (reference src/sampler.cpp:11-109) whose pick runs on the GPU.
//
// Seeding, the xorshift128+ stream and the history window are host-side and behave exactly like
// the reference's (src/sampler.cpp:11-48): a non-greedy pick takes one draw from the stream, a
// greedy pick takes none. The draw and the history are handed to vsmp_pick_host, which runs the
// pick's arithmetic on the device. GPU state lives in a per-thread vsmp_ctx, not in the object,
// because the object layout is fixed by the public header.
#include <chrono>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "verbo/verbo.hpp"
#include "vsmp.h"
#include "vsmp_error.hpp"
#include "vsmp_internal.hpp"

namespace vsmp {

std::uint64_t splitmix(std::uint64_t& s) {
  std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void seed_stream(std::uint64_t seed, std::uint64_t out[2]) {
  // seed 0 seeds from the clock (src/sampler.cpp:27)
  const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
  std::uint64_t s = seed ? seed : static_cast<std::uint64_t>(us);
  out[0] = splitmix(s);
  out[1] = splitmix(s);
}

}  // namespace vsmp

namespace verbo {

namespace {

struct CtxDeleter {
  void operator()(vsmp_ctx* c) const { vsmp_ctx_free(c); }
};

// The calling thread's context on its current HIP device, created there on first use.
vsmp_ctx* thread_ctx() {
  thread_local std::vector<std::unique_ptr<vsmp_ctx, CtxDeleter>> ctxs;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) throw std::runtime_error("vsmp: no current HIP device");
  if (ctxs.size() <= static_cast<size_t>(dev)) ctxs.resize(static_cast<size_t>(dev) + 1);
  auto& ctx = ctxs[static_cast<size_t>(dev)];
  if (!ctx) {
    ctx.reset(vsmp_ctx_new(dev));
    if (!ctx) throw std::runtime_error(vsmp_last_error());
  }
  return ctx.get();
}

}  // namespace

Sampler::Sampler(Sampling cfg) : cfg_(cfg) { reset(); }

void Sampler::reset() {
  vsmp::seed_stream(cfg_.seed, rng_);
  hist_.clear();
}

double Sampler::unit() {
  std::uint64_t a = rng_[0];
  const std::uint64_t b = rng_[1];
  const std::uint64_t out = a + b;
  rng_[0] = b;
  a ^= a << 23;
  rng_[1] = a ^ b ^ (a >> 18) ^ (b >> 5);
  return static_cast<double>(out >> 11) * (1.0 / 9007199254740992.0);
}

void Sampler::accept(int tok) {
  hist_.push_back(tok);
  const std::size_t keep = cfg_.repeat_last > 0 ? static_cast<std::size_t>(cfg_.repeat_last) : 0;
  if (keep && hist_.size() > 4 * keep) hist_.erase(hist_.begin(), hist_.end() - static_cast<std::ptrdiff_t>(keep));
}

int Sampler::pick(const float* logits, int n) {
  if (n <= 0) throw std::invalid_argument("verbo: pick needs at least one logit");
  const double u = cfg_.temp > 0.0f ? unit() : 0.0;
  const vsmp_params p{cfg_.temp, cfg_.top_k, cfg_.top_p, cfg_.min_p, cfg_.repeat, cfg_.repeat_last, cfg_.seed};
  int id = -1;
  if (vsmp_pick_host(thread_ctx(), logits, n, &p, hist_.data(), static_cast<int>(hist_.size()), u, &id, nullptr) != 0)
    throw std::runtime_error(vsmp_last_error());
  return id;
}

}  // namespace verbo

// ---- C handle over the drop-in Sampler ----------------------------------------------------------

struct vsmp_sampler {
  verbo::Sampler s;
};

extern "C" {

vsmp_sampler* vsmp_sampler_new(const vsmp_params* cfg) {
  verbo::Sampling c;
  if (cfg) {
    c.temp = cfg->temp;
    c.top_k = cfg->top_k;
    c.top_p = cfg->top_p;
    c.min_p = cfg->min_p;
    c.repeat = cfg->repeat;
    c.repeat_last = cfg->repeat_last;
    c.seed = cfg->seed;
  }
  return new vsmp_sampler{verbo::Sampler(c)};
}

void vsmp_sampler_free(vsmp_sampler* s) { delete s; }

int vsmp_sampler_pick(vsmp_sampler* s, const float* logits, int n) {
  try {
    return s->s.pick(logits, n);
  } catch (const std::exception& e) {
    return vsmp::set_error(e.what());
  }
}

void vsmp_sampler_accept(vsmp_sampler* s, int tok) { s->s.accept(tok); }

void vsmp_sampler_reset(vsmp_sampler* s) { s->s.reset(); }

}  // extern "C"
