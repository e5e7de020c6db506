// Test double for verbo::generate: a deterministic Model / Session / Detok behind verbo's own
// interface (reference include/verbo/verbo.hpp), and a driver that runs a fixed list of decode
// scenarios through verbo::generate and prints one JSON line per scenario.
//
// TEST INFRASTRUCTURE. Built three times from this one file: against the reference's header and its
// src/sampler.cpp (oracle/Makefile, target _ref/gen_ref: the golden outputs), against this
// repository's header and libvsmp.so (tests/generate/Makefile, gen_ours: the GPU sampler under
// the drop-in generate), and with VSMP_DEVICE_GENERATE (gen_ours_device: the device-resident
// generate_device, its logits copied to the device as an LM head on the GPU would leave them). The scenarios exercise the loop's ordering (src/sampler.cpp:111-181):
// stop ids, stop strings split across tokens (the hold-back), a callback that stops, the context
// limit, max_tokens, the detokeniser's held text and its flush, greedy and sampled picks.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "verbo/verbo.hpp"
#ifdef VSMP_DEVICE_GENERATE
#include <hip/hip_runtime.h>

#include "vsmp_generate.hpp"
#endif

namespace {

struct Scenario {
  const char* name;
  int vocab;
  std::uint64_t data_seed;
  verbo::Sampling smp;
  int max_tokens;
  std::vector<std::string> stop_text;
  int ctx;
  std::vector<int> stop_ids;
  int stop_after;  // from this position on, the first stop id gets a large bonus (0: never)
  std::vector<int> prompt;
  int cb_limit;    // the callback returns false on this call (0: never)
};

std::uint64_t mix(std::uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

const Scenario* g_sc = nullptr;

// Pieces by id % 16; '#' pieces are held by the detokeniser until the next push or the flush.
const char* const kPieces[16] = {"a", "b", "c", "d", " ", "cd", "x", "y", "z", "#q", "", "ab", "\n", "e", "f", "g"};

}  // namespace

namespace verbo {

struct Model::Impl {
  Config cfg;
  Tokenizer tok;
  std::vector<int> stops;
};

std::shared_ptr<const Model> Model::load(const std::string&, DType) {
  auto m = std::make_shared<Model>();
  m->impl_ = std::make_shared<Impl>();
  m->impl_->cfg.vocab = g_sc->vocab;
  m->impl_->stops = g_sc->stop_ids;
  return m;
}

const Config& Model::cfg() const { return impl_->cfg; }
const Tokenizer& Model::tok() const { return impl_->tok; }
bool Model::is_stop(int id) const {
  for (const int s : impl_->stops)
    if (s == id) return true;
  return false;
}

struct Session::Impl {
  std::shared_ptr<const Model> mdl;
  int ctx = 0;
  int pos = 0;
  int last = -1;
  std::vector<float> logits;
};

Session::Session(std::shared_ptr<const Model> mdl, int ctx, int) : impl_(new Impl) {
  impl_->mdl = std::move(mdl);
  impl_->ctx = ctx;
}
Session::~Session() = default;
Session::Session(Session&&) noexcept = default;
Session& Session::operator=(Session&&) noexcept = default;

// Logits of the next position: N(0, 3^2)-like values from the scenario's seed, the position and
// the last token, plus a bonus for the first stop id from stop_after on.
const float* Session::eval(const int* toks, int n) {
  Impl& s = *impl_;
  s.pos += n;
  if (n > 0) s.last = toks[n - 1];
  const int V = g_sc->vocab;
  s.logits.assign(V, 0.0f);
  for (int i = 0; i < V; ++i) {
    const std::uint64_t h = mix(g_sc->data_seed * 0x9E3779B97F4A7C15ull + static_cast<std::uint64_t>(s.pos) * 1000003u +
                                static_cast<std::uint64_t>(s.last + 1) * 7919u + static_cast<std::uint64_t>(i));
    const double u1 = (static_cast<double>(h >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = static_cast<double>(mix(h) >> 11) * (1.0 / 9007199254740992.0);
    s.logits[i] = static_cast<float>(3.0 * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
  if (g_sc->stop_after > 0 && s.pos >= g_sc->stop_after && !g_sc->stop_ids.empty()) s.logits[g_sc->stop_ids[0]] += 20.0f;
  return s.logits.data();
}

int Session::pos() const { return impl_->pos; }
int Session::ctx() const { return impl_->ctx; }
const Model& Session::model() const { return *impl_->mdl; }

std::string Detok::push(int id) {
  const std::string piece = kPieces[id % 16];
  if (!piece.empty() && piece[0] == '#') {
    pend_ += piece;
    return std::string();
  }
  std::string out;
  out.swap(pend_);
  return out + piece;
}

std::string Detok::flush() {
  std::string out;
  out.swap(pend_);
  return out;
}

}  // namespace verbo

namespace {

#ifdef VSMP_DEVICE_GENERATE
// The test double's session as a device-resident LM head would present it (the device generate
// variant, gen_ours_device): each evaluation's logits are written to a device buffer on the
// session's stream, as an LM head's output would be.
class DeviceFake : public vsmp::DeviceSession {
 public:
  explicit DeviceFake(verbo::Session& s) : s_(s) {
    (void)hipStreamCreateWithFlags(&st_, hipStreamNonBlocking);
    (void)hipMalloc(reinterpret_cast<void**>(&d_), sizeof(float) * static_cast<size_t>((g_sc->vocab + 3) & ~3));
  }
  ~DeviceFake() override {
    (void)hipStreamSynchronize(st_);
    (void)hipFree(d_);
    (void)hipStreamDestroy(st_);
  }
  const float* eval(const int* ids, int n) override {
    const float* h = s_.eval(ids, n);
    // the host row stays unchanged until the next eval, which follows the pick's wait for this stream
    (void)hipMemcpyAsync(d_, h, sizeof(float) * static_cast<size_t>(g_sc->vocab), hipMemcpyHostToDevice, st_);
    return d_;
  }
  int pos() const override { return s_.pos(); }
  int ctx() const override { return s_.ctx(); }
  const verbo::Model& model() const override { return s_.model(); }
  void* stream() const override { return st_; }

 private:
  verbo::Session& s_;
  hipStream_t st_ = nullptr;
  float* d_ = nullptr;
};
#endif

std::string json_str(const std::string& s) {
  std::string o = "\"";
  for (const char c : s) {
    if (c == '"' || c == '\\') o += '\\', o += c;
    else if (c == '\n') o += "\\n";
    else o += c;
  }
  return o + "\"";
}

verbo::Sampling smp(float temp, int top_k, float top_p, float min_p, float repeat, int repeat_last, std::uint64_t seed) {
  verbo::Sampling s;
  s.temp = temp;
  s.top_k = top_k;
  s.top_p = top_p;
  s.min_p = min_p;
  s.repeat = repeat;
  s.repeat_last = repeat_last;
  s.seed = seed;
  return s;
}

}  // namespace

int main() {
  const std::vector<Scenario> scs = {
      {"greedy", 64, 1, smp(0.0f, 40, 0.9f, 0.0f, 1.0f, 64, 0), 20, {}, 1000, {}, 0, {5, 6, 7}, 0},
      {"greedy_penalty", 64, 2, smp(0.0f, 40, 0.9f, 0.0f, 1.5f, 8, 0), 30, {}, 1000, {}, 0, {1, 2, 3}, 0},
      {"sampled", 512, 3, smp(0.8f, 40, 0.9f, 0.05f, 1.2f, 8, 7), 40, {}, 1000, {}, 0, {9, 8}, 0},
      {"sampled_wide", 300, 4, smp(1.2f, 0, 0.97f, 0.0f, 1.0f, 64, 11), 40, {}, 1000, {}, 0, {}, 0},
      {"stop_id", 128, 5, smp(0.7f, 20, 0.9f, 0.0f, 1.1f, 16, 3), 60, {}, 1000, {3}, 12, {4}, 0},
      {"stop_text", 128, 6, smp(1.0f, 16, 1.0f, 0.0f, 1.0f, 64, 5), 80, {"cd", "xyz", ""}, 1000, {}, 0, {0}, 0},
      {"stop_text_long", 64, 7, smp(1.5f, 0, 1.0f, 0.0f, 1.0f, 64, 9), 120, {"abcd", "y\nz"}, 1000, {}, 0, {}, 0},
      {"callback_stops", 64, 8, smp(0.9f, 10, 0.95f, 0.0f, 1.0f, 64, 13), 50, {}, 1000, {}, 0, {1}, 4},
      {"ctx_limit", 64, 9, smp(0.9f, 10, 0.95f, 0.0f, 1.0f, 64, 17), 50, {}, 10, {}, 0, {1, 2, 3}, 0},
      {"held_piece_flush", 32, 10, smp(0.0f, 40, 0.9f, 0.0f, 1.0f, 64, 0), 6, {}, 1000, {}, 0, {9}, 0},
      {"empty_prompt", 64, 11, smp(0.6f, 30, 0.85f, 0.0f, 1.0f, 64, 21), 15, {}, 1000, {}, 0, {}, 0},
  };
  for (const Scenario& sc : scs) {
    g_sc = &sc;
    verbo::Session ses(verbo::Model::load(sc.name), sc.ctx, 1);
    verbo::GenOpts o;
    o.max_tokens = sc.max_tokens;
    o.smp = sc.smp;
    o.stop_text = sc.stop_text;
    std::vector<std::string> chunks;
    int calls = 0;
    const auto on_text = [&](std::string_view t) {
      chunks.emplace_back(t);
      ++calls;
      return !(sc.cb_limit > 0 && calls >= sc.cb_limit);
    };
#ifdef VSMP_DEVICE_GENERATE
    DeviceFake dev(ses);
    const verbo::Stats st = vsmp::generate_device(dev, sc.prompt, o, on_text);
#else
    const verbo::Stats st = verbo::generate(ses, sc.prompt, o, on_text);
#endif
    std::string line = std::string("{\"name\": ") + json_str(sc.name) + ", \"prompt\": " + std::to_string(st.prompt) +
                       ", \"gen\": " + std::to_string(st.gen) + ", \"stopped\": " + (st.stopped ? "true" : "false") +
                       ", \"pos\": " + std::to_string(ses.pos()) + ", \"toks\": [";
    for (std::size_t i = 0; i < st.toks.size(); ++i) line += (i ? ", " : "") + std::to_string(st.toks[i]);
    line += "], \"text\": [";
    for (std::size_t i = 0; i < chunks.size(); ++i) line += (i ? ", " : "") + json_str(chunks[i]);
    line += "]}";
    std::printf("%s\n", line.c_str());
  }
  return 0;
}
