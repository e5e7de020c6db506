// Prints the object layout of the verbo types the drop-in sampler and generate share with verbo
// (sizes and the offsets generate and its callers read). Compiled once against this
// repository's include/verbo/verbo.hpp and once against the reference's header; the two outputs
// must be equal (tests/test_capi.py). TEST INFRASTRUCTURE.
#include <cstdio>

#include "verbo/verbo.hpp"

#define OFF(obj, field) static_cast<long>(reinterpret_cast<const char*>(&(obj).field) - reinterpret_cast<const char*>(&(obj)))

int main() {
  verbo::Config c;
  verbo::Sampling s;
  verbo::Stats st;
  verbo::GenOpts g;
  std::printf("Config %zu vocab %ld max_ctx %ld rope_orig %ld\n", sizeof c, OFF(c, vocab), OFF(c, max_ctx), OFF(c, rope_orig));
  std::printf("Sampling %zu temp %ld top_k %ld top_p %ld min_p %ld repeat %ld repeat_last %ld seed %ld\n", sizeof s,
              OFF(s, temp), OFF(s, top_k), OFF(s, top_p), OFF(s, min_p), OFF(s, repeat), OFF(s, repeat_last), OFF(s, seed));
  std::printf("Stats %zu prompt %ld gen %ld prompt_ms %ld gen_ms %ld stopped %ld toks %ld\n", sizeof st, OFF(st, prompt),
              OFF(st, gen), OFF(st, prompt_ms), OFF(st, gen_ms), OFF(st, stopped), OFF(st, toks));
  std::printf("GenOpts %zu max_tokens %ld smp %ld stop_text %ld\n", sizeof g, OFF(g, max_tokens), OFF(g, smp),
              OFF(g, stop_text));
  std::printf("Sampler %zu Detok %zu Model %zu Session %zu Tokenizer %zu\n", sizeof(verbo::Sampler),
              sizeof(verbo::Detok), sizeof(verbo::Model), sizeof(verbo::Session), sizeof(verbo::Tokenizer));
  return 0;
}
