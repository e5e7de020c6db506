// Drop-in verbo::generate (reference src/sampler.cpp:111-181): the decode loop around the sampler.
//
// Per step, in the reference's order: pick the next id from the session's logits; a stop id ends
// generation without being accepted or emitted; otherwise accept it into the sampler's history,
// count it, detokenise it and emit the text that can no longer turn into a stop string; then end
// on a false callback, a full context or max_tokens, else evaluate the id. The text hold-back
// keeps the longest tail of the pending text that is a proper prefix of some stop string.
#include <algorithm>
#include <chrono>
#include <string>

#include "verbo/verbo.hpp"

namespace verbo {

namespace {

double wall_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Pending decoded text between the detokeniser and the caller's callback.
class TextGate {
 public:
  TextGate(const std::vector<std::string>& stops, const std::function<bool(std::string_view)>& sink)
      : stops_(stops), sink_(sink) {
    for (const std::string& s : stops_) longest_ = std::max(longest_, s.size());
  }

  void add(const std::string& text) { pend_ += text; }

  // Emits what is safe. A stop string found in the pending text emits the text before it and
  // ends generation (false). Otherwise everything is emitted except, before the end, a tail that
  // could still grow into a stop string; returns the callback's verdict (true when nothing was
  // emitted).
  bool release(bool at_end) {
    for (const std::string& s : stops_) {
      if (s.empty()) continue;
      const std::size_t at = pend_.find(s);
      if (at == std::string::npos) continue;
      if (at > 0) sink_(std::string_view(pend_).substr(0, at));
      pend_.clear();
      return false;
    }
    const std::size_t keep = at_end ? 0 : held_tail();
    const std::size_t n = pend_.size() - keep;
    if (n == 0) return true;
    const bool go = sink_(std::string_view(pend_).substr(0, n));
    pend_.erase(0, n);
    return go;
  }

 private:
  // Length of the longest tail of pend_ (shorter than the longest stop string) that equals the
  // beginning of a longer stop string.
  std::size_t held_tail() const {
    if (longest_ == 0) return 0;
    for (std::size_t k = std::min(pend_.size(), longest_ - 1); k > 0; --k) {
      const std::size_t from = pend_.size() - k;
      for (const std::string& s : stops_)
        if (s.size() > k && pend_.compare(from, k, s, 0, k) == 0) return k;
    }
    return 0;
  }

  const std::vector<std::string>& stops_;
  const std::function<bool(std::string_view)>& sink_;
  std::size_t longest_ = 0;
  std::string pend_;
};

}  // namespace

Stats generate(Session& ses, const std::vector<int>& prompt, const GenOpts& opt,
               const std::function<bool(std::string_view)>& on_text) {
  Stats st;
  const Model& model = ses.model();
  const int vocab = model.cfg().vocab;
  Sampler sampler(opt.smp);
  for (const int id : prompt) sampler.accept(id);  // the prompt is history for the penalty
  st.prompt = static_cast<int>(prompt.size());

  double t = wall_ms();
  const float* logits = ses.eval(prompt);
  st.prompt_ms = wall_ms() - t;

  Detok detok(model.tok());
  TextGate gate(opt.stop_text, on_text);
  t = wall_ms();
  bool go = true;
  while (go && st.gen < opt.max_tokens) {
    const int id = sampler.pick(logits, vocab);
    if (model.is_stop(id)) {  // not accepted, not emitted
      st.stopped = true;
      break;
    }
    sampler.accept(id);
    ++st.gen;
    st.toks.push_back(id);
    gate.add(detok.push(id));
    go = gate.release(false);
    if (!go) {
      st.stopped = true;
      break;
    }
    if (ses.pos() >= ses.ctx() || st.gen >= opt.max_tokens) break;
    logits = ses.eval(&id, 1);
  }
  if (go) {  // a stop id or the end of the budget: flush what the detokeniser still holds
    gate.add(detok.flush());
    gate.release(true);
  }
  st.gen_ms = wall_ms() - t;
  return st;
}

}  // namespace verbo
