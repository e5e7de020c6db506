// verbo_generate (reference src/capi.cpp:131-151) on the reference's tiny test models, through
// whichever libverbo.so this program is linked with: the reference's own sampler, or the MI355X
// sampler swapped in by the integration notes' CMake blocks. Test infrastructure.
//
//   capi_generate <dir holding tiny-qwen2/ and tiny-llama/>
//
// Prints one JSON line per scenario: its name, verbo_generate's return value (tokens generated),
// the number of text callbacks and the emitted text as hex (the bytes need no escaping then).
#include <cstdio>
#include <string>
#include <vector>

#include "verbo/verbo.h"

namespace {

struct Sink {
  std::string text;
  int calls = 0;
  int stop_after = 0;  // > 0: the callback returns 0 on its stop_after-th call
};

int on_text(const char* t, size_t n, void* user) {
  Sink* s = static_cast<Sink*>(user);
  s->text.append(t, n);
  ++s->calls;
  return (s->stop_after > 0 && s->calls >= s->stop_after) ? 0 : 1;
}

struct Case {
  const char* name;
  const char* model;
  bool defaults;  // start from verbo_model_defaults (generation_config.json), else the fields below
  int max_tokens;
  float temp;
  int top_k;
  float top_p;
  float min_p;
  float repeat;
  unsigned long long seed;
  int stop_after;
};

std::string hex(const std::string& s) {
  static const char* d = "0123456789abcdef";
  std::string h;
  for (unsigned char c : s) {
    h += d[c >> 4];
    h += d[c & 15];
  }
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string root = argc > 1 ? argv[1] : "tests/data";
  const Case cases[] = {
      {"qwen_greedy", "tiny-qwen2", false, 16, 0.0f, 40, 0.9f, 0.0f, 1.0f, 0, 0},
      {"qwen_greedy_repeat", "tiny-qwen2", false, 24, 0.0f, 40, 0.9f, 0.0f, 1.3f, 0, 0},
      {"qwen_defaults_seed7", "tiny-qwen2", true, 24, 0.0f, 0, 0.0f, 0.0f, 0.0f, 7, 0},
      {"qwen_wide_minp_repeat", "tiny-qwen2", false, 24, 1.0f, 0, 0.95f, 0.02f, 1.3f, 11, 0},
      {"qwen_topk5", "tiny-qwen2", false, 32, 0.8f, 5, 1.0f, 0.0f, 1.1f, 12345, 0},
      {"qwen_callback_stops", "tiny-qwen2", false, 32, 0.7f, 40, 0.9f, 0.0f, 1.0f, 3, 3},
      {"llama_greedy_repeat", "tiny-llama", false, 16, 0.0f, 40, 0.9f, 0.0f, 1.2f, 0, 0},
      {"llama_defaults_seed99", "tiny-llama", true, 24, 0.0f, 0, 0.0f, 0.0f, 0.0f, 99, 0},
      {"llama_hot_topp", "tiny-llama", false, 20, 1.5f, 0, 0.9f, 0.0f, 1.0f, 5, 0},
  };
  int failed = 0;
  for (const Case& c : cases) {
    verbo_model* m = verbo_model_load((root + "/" + c.model).c_str(), "q8");
    if (!m) {
      std::fprintf(stderr, "%s: %s\n", c.name, verbo_last_error());
      return 2;
    }
    const char* roles[] = {"user"};
    const char* texts[] = {"hola"};
    const int need = verbo_chat_prompt(m, roles, texts, 1, 1, nullptr, 0);
    std::string prompt(static_cast<size_t>(need) + 1, '\0');
    verbo_chat_prompt(m, roles, texts, 1, 1, &prompt[0], need + 1);
    prompt.resize(static_cast<size_t>(need));
    const int n = verbo_tokenize(m, prompt.data(), prompt.size(), 1, nullptr, 0);
    std::vector<int> ids(static_cast<size_t>(n));
    verbo_tokenize(m, prompt.data(), prompt.size(), 1, ids.data(), n);
    verbo_gen_opts o = verbo_model_defaults(m);
    if (!c.defaults) {
      o.temp = c.temp;
      o.top_k = c.top_k;
      o.top_p = c.top_p;
      o.min_p = c.min_p;
      o.repeat = c.repeat;
    }
    o.max_tokens = c.max_tokens;
    o.seed = c.seed;
    verbo_session* s = verbo_session_new(m, 128, 2);
    Sink sink;
    sink.stop_after = c.stop_after;
    const int gen = verbo_generate(s, ids.data(), n, &o, on_text, &sink);
    if (gen < 0) {
      std::fprintf(stderr, "%s: verbo_generate: %s\n", c.name, verbo_last_error());
      ++failed;
    }
    std::printf("{\"name\": \"%s\", \"gen\": %d, \"calls\": %d, \"text_hex\": \"%s\"}\n", c.name, gen, sink.calls,
                hex(sink.text).c_str());
    std::fflush(stdout);
    verbo_session_free(s);
    verbo_model_free(m);
  }
  return failed ? 1 : 0;
}
