// The part of verbo's public C++ interface that the MI355X sampler implements or calls
// (reference include/verbo/verbo.hpp). It declares the same names, signatures and, for Sampler,
// the same data members in the same order (the reference header compiles Sampler::cfg() inline
// into its callers, so the object layout is part of the interface).
//
// libvsmp.so exports verbo::Sampler and verbo::generate built against this header, and a verbo
// build links them in place of its src/sampler.cpp, so every type they touch keeps the
// reference's exact layout: Config (generate reads cfg().vocab), Sampling, Stats, GenOpts, and the
// single pointer members of Model, Session, Tokenizer and Detok.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace verbo {

enum class DType : std::uint8_t { F32 = 0, Q8 = 1, Q4 = 2 };

// Model configuration (reference include/verbo/verbo.hpp:18-36); the sampler path reads `vocab`.
struct Config {
  std::string arch;
  int dim = 0;
  int hidden = 0;
  int layers = 0;
  int heads = 0;
  int kv_heads = 0;
  int head_dim = 0;
  int vocab = 0;
  int max_ctx = 0;
  float eps = 1e-5f;
  float theta = 10000.0f;
  bool qkv_bias = false;
  bool tied = false;
  float rope_factor = 0.0f;
  float rope_low = 1.0f;
  float rope_high = 4.0f;
  int rope_orig = 8192;
};

// The tokenizer (reference include/verbo/verbo.hpp:38-54); generate reaches it through Detok.
class Tokenizer {
 public:
  std::string piece(int id) const;
  int size() const;

  struct Impl;

 private:
  std::shared_ptr<const Impl> impl_;
};

// Sampling parameters and their defaults (reference include/verbo/verbo.hpp:56-64).
struct Sampling {
  float temp = 0.7f;
  int top_k = 40;
  float top_p = 0.9f;
  float min_p = 0.0f;
  float repeat = 1.0f;
  int repeat_last = 64;
  std::uint64_t seed = 0;
};

class Model {
 public:
  static std::shared_ptr<const Model> load(const std::string& path, DType dt = DType::Q8);

  const Config& cfg() const;
  const Tokenizer& tok() const;
  bool is_stop(int id) const;
  Sampling sampling() const;

  struct Impl;
  const Impl& impl() const { return *impl_; }

 private:
  std::shared_ptr<Impl> impl_;
};

class Session {
 public:
  explicit Session(std::shared_ptr<const Model> mdl, int ctx = 0, int threads = 0);
  ~Session();
  Session(Session&&) noexcept;
  Session& operator=(Session&&) noexcept;

  const float* eval(const int* toks, int n);
  const float* eval(const std::vector<int>& toks) { return eval(toks.data(), static_cast<int>(toks.size())); }

  int pos() const;
  int ctx() const;
  void rewind(int pos);
  const Model& model() const;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// The token sampler (reference include/verbo/verbo.hpp:116-132). pick() runs on the GPU.
class Sampler {
 public:
  explicit Sampler(Sampling cfg = {});

  int pick(const float* logits, int n);
  void accept(int tok);
  void reset();
  const Sampling& cfg() const { return cfg_; }

 private:
  Sampling cfg_;
  std::uint64_t rng_[2];
  std::vector<int> hist_;
  std::vector<std::pair<float, int>> buf_;  // unused on the GPU path; kept for the layout

  double unit();
};

class Detok {
 public:
  explicit Detok(const Tokenizer& tok) : tok_(&tok) {}

  std::string push(int id);
  std::string flush();

 private:
  const Tokenizer* tok_;
  std::string pend_;
};

struct Stats {
  int prompt = 0;
  int gen = 0;
  double prompt_ms = 0.0;
  double gen_ms = 0.0;
  bool stopped = false;
  std::vector<int> toks;
};

struct GenOpts {
  int max_tokens = 256;
  Sampling smp;
  std::vector<std::string> stop_text;
};

Stats generate(Session& ses, const std::vector<int>& prompt, const GenOpts& opt,
               const std::function<bool(std::string_view)>& on_text);

}  // namespace verbo
