// Device-resident decode state behind the C ABI: one sequence (vsmp_dsampler) and a batch of
// sequences (vsmp_bsampler), each verbo::Sampler (reference src/sampler.cpp:24-109) with its draw
// stream and history window in device memory.
//
// The stream is seeded on the host exactly as Sampler::reset seeds it (two SplitMix64 outputs of the
// seed) and then lives on the device: the pick kernels advance it in place (VSMP_U_XORSHIFT), once
// per sampled row and never for a greedy one, as Sampler::pick draws (src/sampler.cpp:66-70,101).
// The history window follows Sampler::accept (src/sampler.cpp:43-48): appended on the device by
// k_hist_accept, trimmed to the last repeat_last ids once it would exceed 4 * repeat_last.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

#include "vsmp.h"
#include "vsmp_common.hpp"
#include "vsmp_error.hpp"
#include "vsmp_internal.hpp"

using vsmp::hip_ok;

namespace {

// The length a history of h ids reaches after accepting m more (src/sampler.cpp:43-48): the
// window keeps only its newest ids, so the result is always the last ids of the concatenation.
int accepted_length(int h, int m, int repeat_last) {
  for (int i = 0; i < m; ++i) {
    ++h;
    if (repeat_last > 0 && h > 4 * repeat_last) h = repeat_last;
  }
  return h;
}

// Device memory for a stream and a window, released together.
template <class T>
bool dev_alloc(T*& p, size_t n, const char* what) {
  void* q = nullptr;
  if (!hip_ok(hipMalloc(&q, std::max<size_t>(n, 1) * sizeof(T)), what)) return false;
  p = static_cast<T*>(q);
  return true;
}

}  // namespace

// ---- one sequence ------------------------------------------------------------------------------

struct vsmp_dsampler {
  int device = 0;
  vsmp_ctx* ctx = nullptr;      // scratch of the pick kernels
  vsmp_params cfg{};
  int* hist = nullptr;          // the history window, cap ids
  int cap = 0;
  int* meta = nullptr;          // {0, h}: the window's CSR offsets (one row)
  unsigned long long* rng = nullptr;  // the xorshift128+ state
  int* out = nullptr;           // the last picked id
  int* host = nullptr;          // pinned: [0] the id copied back, [2..3] staging of meta
  int h = 0;                    // ids in the window (every change goes through this object)
};

namespace {

bool ds_free_bufs(vsmp_dsampler* s) {
  vsmp::DeviceScope scope(s->device);
  for (void* p : {static_cast<void*>(s->hist), static_cast<void*>(s->meta), static_cast<void*>(s->rng),
                  static_cast<void*>(s->out)})
    if (p) (void)hipFree(p);
  if (s->host) (void)hipHostFree(s->host);
  return true;
}

// Window capacity for h ids: 4 * repeat_last when the reference trims, else grown by doubling.
bool ds_reserve(vsmp_dsampler* s, int need, hipStream_t st) {
  if (need <= s->cap) return true;
  int cap = std::max(need, std::max(2 * s->cap, 256));
  int* q = nullptr;
  if (!dev_alloc(q, static_cast<size_t>(cap), "history window")) return false;
  if (s->hist) {
    if (s->h > 0 && !hip_ok(hipMemcpyAsync(q, s->hist, sizeof(int) * static_cast<size_t>(s->h), hipMemcpyDeviceToDevice, st),
                            "copy history window"))
      return false;
    if (!hip_ok(hipStreamSynchronize(st), "synchronise")) return false;
    (void)hipFree(s->hist);
  }
  s->hist = q;
  s->cap = cap;
  return true;
}

bool ds_set_length(vsmp_dsampler* s, int h, hipStream_t st) {
  // the staging ints stay untouched until the copy has read them: it completes before the call returns
  s->host[2] = 0;
  s->host[3] = h;
  if (!hip_ok(hipMemcpyAsync(s->meta, s->host + 2, 2 * sizeof(int), hipMemcpyHostToDevice, st), "copy window length") ||
      !hip_ok(hipStreamSynchronize(st), "synchronise"))
    return false;
  s->h = h;
  return true;
}

}  // namespace

extern "C" {

vsmp_dsampler* vsmp_dsampler_new(int device, const vsmp_params* cfg) {
  vsmp::clear_error();
  if (!cfg) {
    vsmp::set_error("vsmp: null parameters");
    return nullptr;
  }
  vsmp_dsampler* s = new vsmp_dsampler();
  s->ctx = vsmp_ctx_new(device);
  if (!s->ctx) {
    delete s;
    return nullptr;
  }
  s->device = vsmp::ctx_device(s->ctx);
  vsmp::DeviceScope scope(s->device);  // the sampler's buffers live on the context's device
  if (!scope.ok()) {
    vsmp_dsampler_free(s);
    return nullptr;
  }
  s->cfg = *cfg;
  void* host = nullptr;
  const int first_cap = cfg->repeat_last > 0 ? 4 * cfg->repeat_last : 256;
  bool ok = dev_alloc(s->meta, 2, "window offsets") && dev_alloc(s->rng, 2, "draw stream") && dev_alloc(s->out, 1, "id") &&
            hip_ok(hipHostMalloc(&host, 4 * sizeof(int), hipHostMallocDefault), "pinned staging");
  s->host = static_cast<int*>(host);
  ok = ok && ds_reserve(s, first_cap, nullptr) && vsmp_dsampler_reset(s) == 0;
  if (!ok) {
    vsmp_dsampler_free(s);
    return nullptr;
  }
  return s;
}

void vsmp_dsampler_free(vsmp_dsampler* s) {
  if (!s) return;
  if (s->ctx) vsmp_ctx_free(s->ctx);  // waits for the device
  ds_free_bufs(s);
  delete s;
}

int vsmp_dsampler_reset(vsmp_dsampler* s) {
  vsmp::clear_error();
  if (!s) return vsmp::set_error("vsmp: null sampler");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  // Picks and accepts still queued on the caller's streams advance the draw stream and the window in
  // place; the reset must land after them, and it has no stream of its own: wait for the device.
  if (!hip_ok(hipDeviceSynchronize(), "synchronise")) return -1;
  std::uint64_t st[2];
  vsmp::seed_stream(s->cfg.seed, st);
  if (!hip_ok(hipMemcpy(s->rng, st, sizeof st, hipMemcpyHostToDevice), "copy draw stream")) return -1;
  return ds_set_length(s, 0, nullptr) ? 0 : -1;
}

int vsmp_dsampler_accept(vsmp_dsampler* s, const int* ids, int n, void* stream) {
  vsmp::clear_error();
  if (!s || (n > 0 && !ids) || n < 0) return vsmp::set_error("vsmp: bad accept arguments");
  if (n == 0) return 0;
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rl = s->cfg.repeat_last;
  const int len = accepted_length(s->h, n, rl);
  if (len <= n) {
    // the new window is the last `len` of the given ids: one copy (a prompt, or a long batch of ids)
    if (!ds_reserve(s, len, st) ||
        !hip_ok(hipMemcpyAsync(s->hist, ids + (n - len), sizeof(int) * static_cast<size_t>(len), hipMemcpyHostToDevice, st),
                "copy history ids") ||
        !ds_set_length(s, len, st))
      return -1;
    return 0;
  }
  // otherwise the window keeps some of its ids: append one by one on the device
  for (int i = 0; i < n; ++i) {
    if (rl <= 0 && !ds_reserve(s, s->h + 1, st)) return -1;
    vsmp::launch_hist_accept(s->hist, s->meta, s->meta + 1, s->cap, nullptr, s->cfg, nullptr, ids[i], nullptr, nullptr, 1,
                             nullptr, st);
    if (!hip_ok(hipGetLastError(), "accept launch")) return -1;
    s->h = accepted_length(s->h, 1, rl);
  }
  return 0;
}

int vsmp_dsampler_pick_async(vsmp_dsampler* s, const float* logits, int n, int* out, void* stream) {
  vsmp::clear_error();
  if (!s) return vsmp::set_error("vsmp: null sampler");
  if (n <= 0) return vsmp::set_error("vsmp: pick needs at least one logit");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  const long long ld = (static_cast<long long>(n) + 3) & ~3LL;
  return vsmp::pick_batch(s->ctx, logits, 1, n, ld, &s->cfg, 0, s->hist, s->meta, VSMP_U_XORSHIFT, nullptr, s->rng, 0,
                          out ? out : s->out, nullptr, static_cast<hipStream_t>(stream));
}

int vsmp_dsampler_pick(vsmp_dsampler* s, const float* logits, int n, void* stream) {
  if (vsmp_dsampler_pick_async(s, logits, n, nullptr, stream) != 0) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!hip_ok(hipMemcpyAsync(s->host, s->out, sizeof(int), hipMemcpyDeviceToHost, st), "copy id") ||
      !hip_ok(hipStreamSynchronize(st), "synchronise"))
    return -1;
  return s->host[0];
}

}  // extern "C"

// ---- a batch of sequences ----------------------------------------------------------------------

struct vsmp_bsampler {
  int device = 0;
  vsmp_ctx* ctx = nullptr;
  int n = 0;
  int cap = 0;                       // ids per row region
  vsmp_params* params = nullptr;     // device [n]
  unsigned long long* rng = nullptr; // device [2n]
  int* hist = nullptr;               // device [n][cap]
  int* off = nullptr;                // device [n]: r * cap
  int* len = nullptr;                // device [n]
  int* full = nullptr;               // device flag
  int* host = nullptr;               // pinned staging: the flag read back
};

extern "C" {

vsmp_bsampler* vsmp_bsampler_new(int device, int n, const vsmp_params* params, int cap) {
  vsmp::clear_error();
  if (n < 1 || !params || cap < 1) {
    vsmp::set_error("vsmp: need n >= 1, parameters and cap >= 1");
    return nullptr;
  }
  for (int r = 0; r < n; ++r)
    if (params[r].repeat_last > 0 && static_cast<long long>(params[r].repeat_last) * 4 > cap) {
      vsmp::set_error("vsmp: cap must hold 4 * repeat_last ids (row " + std::to_string(r) + ")");
      return nullptr;
    }
  if (static_cast<long long>(n) * cap > INT32_MAX) {
    vsmp::set_error("vsmp: n * cap too large");
    return nullptr;
  }
  vsmp_bsampler* s = new vsmp_bsampler();
  s->ctx = vsmp_ctx_new(device);
  if (!s->ctx) {
    delete s;
    return nullptr;
  }
  s->device = vsmp::ctx_device(s->ctx);
  vsmp::DeviceScope scope(s->device);  // the sampler's buffers live on the context's device
  if (!scope.ok()) {
    vsmp_bsampler_free(s);
    return nullptr;
  }
  s->n = n;
  s->cap = cap;
  std::vector<std::uint64_t> st(2 * static_cast<size_t>(n));
  std::vector<int> off(static_cast<size_t>(n));
  for (int r = 0; r < n; ++r) {
    // seed 0 stands for the clock, as in the reference; such rows then differ by their index
    vsmp::seed_stream(params[r].seed, &st[2 * static_cast<size_t>(r)]);
    if (!params[r].seed) st[2 * static_cast<size_t>(r)] += static_cast<std::uint64_t>(r);
    off[static_cast<size_t>(r)] = r * cap;
  }
  void* host = nullptr;
  bool ok = dev_alloc(s->params, static_cast<size_t>(n), "parameters") && dev_alloc(s->rng, 2 * static_cast<size_t>(n), "draw streams") &&
            dev_alloc(s->hist, static_cast<size_t>(n) * cap, "history windows") && dev_alloc(s->off, static_cast<size_t>(n), "offsets") &&
            dev_alloc(s->len, static_cast<size_t>(n), "lengths") && dev_alloc(s->full, 1, "flag") &&
            hip_ok(hipHostMalloc(&host, sizeof(int), hipHostMallocDefault), "pinned staging");
  s->host = static_cast<int*>(host);
  ok = ok &&
       hip_ok(hipMemcpy(s->params, params, sizeof(vsmp_params) * static_cast<size_t>(n), hipMemcpyHostToDevice), "copy parameters") &&
       hip_ok(hipMemcpy(s->rng, st.data(), sizeof(std::uint64_t) * st.size(), hipMemcpyHostToDevice), "copy draw streams") &&
       hip_ok(hipMemcpy(s->off, off.data(), sizeof(int) * off.size(), hipMemcpyHostToDevice), "copy offsets") &&
       hip_ok(hipMemset(s->len, 0, sizeof(int) * static_cast<size_t>(n)), "clear lengths") &&
       hip_ok(hipMemset(s->full, 0, sizeof(int)), "clear flag") && hip_ok(hipDeviceSynchronize(), "synchronise");
  if (!ok) {
    vsmp_bsampler_free(s);
    return nullptr;
  }
  return s;
}

void vsmp_bsampler_free(vsmp_bsampler* s) {
  if (!s) return;
  if (s->ctx) vsmp_ctx_free(s->ctx);
  vsmp::DeviceScope scope(s->device);
  for (void* p : {static_cast<void*>(s->params), static_cast<void*>(s->rng), static_cast<void*>(s->hist),
                  static_cast<void*>(s->off), static_cast<void*>(s->len), static_cast<void*>(s->full)})
    if (p) (void)hipFree(p);
  if (s->host) (void)hipHostFree(s->host);
  delete s;
}

int vsmp_bsampler_accept_host(vsmp_bsampler* s, int row, const int* ids, int m) {
  vsmp::clear_error();
  if (!s || row < 0 || row >= s->n || m < 0 || (m > 0 && !ids)) return vsmp::set_error("vsmp: bad accept arguments");
  if (m == 0) return 0;
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok() || !hip_ok(hipDeviceSynchronize(), "synchronise")) return -1;
  // the row's parameters and current length, from the device (prompts are accepted before decoding)
  vsmp_params p{};
  int h = 0;
  if (!hip_ok(hipMemcpy(&p, s->params + row, sizeof p, hipMemcpyDeviceToHost), "read parameters") ||
      !hip_ok(hipMemcpy(&h, s->len + row, sizeof h, hipMemcpyDeviceToHost), "read length"))
    return -1;
  const int len = accepted_length(h, m, p.repeat_last);
  int* region = s->hist + static_cast<size_t>(row) * s->cap;
  if (len > s->cap) return vsmp::set_error("vsmp: history longer than the row's region");
  if (len <= m) {
    if (!hip_ok(hipMemcpy(region, ids + (m - len), sizeof(int) * static_cast<size_t>(len), hipMemcpyHostToDevice), "copy ids"))
      return -1;
  } else {
    // keep the last len - m ids of the window, then the new ones
    std::vector<int> w(static_cast<size_t>(len));
    if (!hip_ok(hipMemcpy(w.data(), region + (h - (len - m)), sizeof(int) * static_cast<size_t>(len - m), hipMemcpyDeviceToHost),
                "read window"))
      return -1;
    std::copy(ids, ids + m, w.begin() + (len - m));
    if (!hip_ok(hipMemcpy(region, w.data(), sizeof(int) * w.size(), hipMemcpyHostToDevice), "copy window")) return -1;
  }
  return hip_ok(hipMemcpy(s->len + row, &len, sizeof len, hipMemcpyHostToDevice), "copy length") ? 0 : -1;
}

int vsmp_bsampler_pick(vsmp_bsampler* s, const float* logits, int V, long long ld, int* out, void* stream) {
  vsmp::clear_error();
  if (!s) return vsmp::set_error("vsmp: null sampler");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  return vsmp::pick_batch(s->ctx, logits, s->n, V, ld, s->params, 1, s->hist, s->off, VSMP_U_XORSHIFT, nullptr, s->rng, 0,
                          out, nullptr, static_cast<hipStream_t>(stream), s->len);
}

int vsmp_bsampler_accept(vsmp_bsampler* s, const int* ids, const int* active, void* stream) {
  vsmp::clear_error();
  if (!s || !ids) return vsmp::set_error("vsmp: bad accept arguments");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  vsmp::launch_hist_accept(s->hist, s->off, s->len, s->cap, s->params, vsmp_params{}, ids, 0, active, nullptr, s->n,
                           s->full, static_cast<hipStream_t>(stream));
  return hip_ok(hipGetLastError(), "accept launch") ? 0 : -1;
}

int vsmp_bsampler_admit(vsmp_bsampler* s, int slot, const vsmp_params* params, const int* prompt, int m, void* stream) {
  vsmp::clear_error();
  if (!s || !params || slot < 0 || slot >= s->n || m < 0 || (m > 0 && !prompt))
    return vsmp::set_error("vsmp: bad admit arguments");
  const vsmp_params p = *params;
  if (p.repeat_last > 0 && static_cast<long long>(p.repeat_last) * 4 > s->cap)
    return vsmp::set_error("vsmp: cap must hold 4 * repeat_last ids");
  // Sampler(cfg) then accept() of each prompt id (src/sampler.cpp:24-48): the window the prompt
  // leaves is its last `len` ids
  const int len = accepted_length(0, m, p.repeat_last);
  if (len > s->cap) return vsmp::set_error("vsmp: the prompt's history window is longer than the slot's region");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  std::uint64_t rs[2];
  vsmp::seed_stream(p.seed, rs);
  if (!p.seed) rs[0] += static_cast<std::uint64_t>(slot);  // seed 0 stands for the clock; slots then differ
  // the ids are read from pageable host memory before the copy call returns; the copy is ordered
  // on `st` after the slot's earlier picks and accepts, and before the admit kernel
  if (len > 0 && !hip_ok(hipMemcpyAsync(s->hist + static_cast<size_t>(slot) * s->cap, prompt + (m - len),
                                        sizeof(int) * static_cast<size_t>(len), hipMemcpyHostToDevice, st),
                         "copy prompt ids"))
    return -1;
  vsmp::launch_slot_admit(s->params, s->rng, s->len, slot, p, rs[0], rs[1], len, st);
  return hip_ok(hipGetLastError(), "admit launch") ? 0 : -1;
}

int vsmp_bsampler_pick_rows(vsmp_bsampler* s, const float* logits, int V, long long ld, const int* rows, int n_rows,
                            int* out, void* stream) {
  vsmp::clear_error();
  if (!s) return vsmp::set_error("vsmp: null sampler");
  if (n_rows < 0 || n_rows > s->n || (n_rows > 0 && !rows))
    return vsmp::set_error("vsmp: need 0 <= n_rows <= the sampler's slots, and the slot list");
  if (n_rows == 0) return 0;
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  return vsmp::pick_batch(s->ctx, logits, n_rows, V, ld, s->params, 1, s->hist, s->off, VSMP_U_XORSHIFT, nullptr, s->rng,
                          0, out, nullptr, static_cast<hipStream_t>(stream), s->len, rows);
}

int vsmp_bsampler_accept_rows(vsmp_bsampler* s, const int* ids, const int* rows, const int* active, int n_rows,
                              void* stream) {
  vsmp::clear_error();
  if (!s || n_rows < 0 || n_rows > s->n || (n_rows > 0 && (!ids || !rows)))
    return vsmp::set_error("vsmp: bad accept arguments");
  if (n_rows == 0) return 0;
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  vsmp::launch_hist_accept(s->hist, s->off, s->len, s->cap, s->params, vsmp_params{}, ids, 0, active, rows, n_rows,
                           s->full, static_cast<hipStream_t>(stream));
  return hip_ok(hipGetLastError(), "accept launch") ? 0 : -1;
}

int vsmp_bsampler_full(vsmp_bsampler* s, void* stream) {
  vsmp::clear_error();
  if (!s) return vsmp::set_error("vsmp: null sampler");
  vsmp::DeviceScope scope(s->device);
  if (!scope.ok()) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!hip_ok(hipMemcpyAsync(s->host, s->full, sizeof(int), hipMemcpyDeviceToHost, st), "copy flag") ||
      !hip_ok(hipStreamSynchronize(st), "synchronise"))
    return -1;
  return s->host[0] ? 1 : 0;
}

}  // extern "C"
