// verbo::generate (reference src/sampler.cpp:111-181) on a session whose logits stay on the device.
//
// The step order is the reference's, as in generate.cpp: pick; a stop id ends generation without
// being accepted or emitted; otherwise accept, count, detokenise, release the text that can no
// longer become a stop string; end on a false callback, a full context or max_tokens; else
// evaluate the id. The picks and accepts run on the session's stream against a vsmp_dsampler, so
// the logits never leave the device; the id comes back (4 bytes) for the stop check and the
// detokeniser. Plain C++ over the C ABI, compiled with the program that provides verbo's types.
#include <chrono>
#include <memory>
#include <stdexcept>
#include <string>

#include "text_gate.hpp"
#include "vsmp_generate.hpp"

namespace vsmp {

namespace {

double wall_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct DsamplerDeleter {
  void operator()(vsmp_dsampler* s) const { vsmp_dsampler_free(s); }
};

void check(int rc) {
  if (rc < 0) throw std::runtime_error(vsmp_last_error());
}

}  // namespace

verbo::Stats generate_device(DeviceSession& ses, const std::vector<int>& prompt, const verbo::GenOpts& opt,
                             const std::function<bool(std::string_view)>& on_text) {
  verbo::Stats st;
  const verbo::Model& model = ses.model();
  const int vocab = model.cfg().vocab;
  const vsmp_params p{opt.smp.temp, opt.smp.top_k, opt.smp.top_p, opt.smp.min_p, opt.smp.repeat, opt.smp.repeat_last,
                      opt.smp.seed};
  std::unique_ptr<vsmp_dsampler, DsamplerDeleter> sampler(vsmp_dsampler_new(-1, &p));
  if (!sampler) throw std::runtime_error(vsmp_last_error());
  void* stream = ses.stream();
  check(vsmp_dsampler_accept(sampler.get(), prompt.data(), static_cast<int>(prompt.size()), stream));
  st.prompt = static_cast<int>(prompt.size());

  double t = wall_ms();
  const float* logits = ses.eval(prompt.data(), static_cast<int>(prompt.size()));
  st.prompt_ms = wall_ms() - t;

  verbo::Detok detok(model.tok());
  TextGate gate(opt.stop_text, on_text);
  t = wall_ms();
  bool go = true;
  while (go && st.gen < opt.max_tokens) {
    const int id = vsmp_dsampler_pick(sampler.get(), logits, vocab, stream);
    check(id);
    if (model.is_stop(id)) {  // not accepted, not emitted
      st.stopped = true;
      break;
    }
    check(vsmp_dsampler_accept(sampler.get(), &id, 1, stream));
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

}  // namespace vsmp
