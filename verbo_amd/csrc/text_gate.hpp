// The stop-text hold-back of verbo::generate (reference src/sampler.cpp:126-154), shared by the
// drop-in generate loops: decoded text waits here until it can no longer turn into a stop string.
#pragma once

#include <algorithm>
#include <functional>
#include <string>
#include <string_view>
#include <vector>

namespace vsmp {

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


}  // namespace vsmp
