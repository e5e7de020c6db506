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

#include "text_gate.hpp"
#include "verbo/verbo.hpp"

namespace verbo {

namespace {

double wall_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

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
  vsmp::TextGate gate(opt.stop_text, on_text);
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
