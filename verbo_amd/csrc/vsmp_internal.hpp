// Host-side pieces shared by the library's C-ABI sources (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "vsmp.h"

namespace vsmp {

// false, with the calling thread's error set to "vsmp: <what>: <HIP message>", unless e is success.
bool hip_ok(hipError_t e, const char* what);

// The device a context was created on.
int ctx_device(const vsmp_ctx* c);
// true when `st` (null: the device's null stream) belongs to the context's device; else false, with
// the error set.
bool stream_on_device(const vsmp_ctx* c, hipStream_t st);

// An entry point's device: makes `dev` the calling thread's current HIP device for the scope, and
// gives the caller's current device back on leaving it, so that a call leaves the thread's device
// as it found it. ok() is false (error set) when the device could not be made current.
class DeviceScope {
 public:
  explicit DeviceScope(int dev) : dev_(dev) {
    if (dev < 0) {  // no device named (a null handle, which the entry point then rejects)
      ok_ = true;
      return;
    }
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    ok_ = prev_ == dev || hip_ok(hipSetDevice(dev), "hipSetDevice");
  }
  ~DeviceScope() {
    if (prev_ >= 0 && prev_ != dev_) (void)hipSetDevice(prev_);
  }
  DeviceScope(const DeviceScope&) = delete;
  DeviceScope& operator=(const DeviceScope&) = delete;
  bool ok() const { return ok_; }

 private:
  int dev_;
  int prev_ = -1;
  bool ok_ = false;
};

// One batched pick: the work of vsmp_pick_batch. hist_len (device-resident decode loops): row r's
// history is hist[hist_off[r], hist_off[r] + hist_len[r]) instead of ending at hist_off[r + 1], so
// that each row may own a region larger than its history. slot (device, B distinct entries): row r
// (logits row r, out[r]) samples for sequence slot[r], whose parameters (per row), history entries
// and draw stream it uses. Returns 0 or -1 (error set).
int pick_batch(vsmp_ctx* ctx, const float* logits, int B, int V, long long ld, const vsmp_params* params,
               int params_per_row, const int* hist, const int* hist_off, int u_mode, const double* u,
               unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
               hipStream_t st, const int* hist_len = nullptr, const int* slot = nullptr);

// verbo::Sampler's seeding (reference src/sampler.cpp:11-16,26-31): two successive SplitMix64
// outputs of the seed; seed 0 stands for the steady clock in microseconds.
std::uint64_t splitmix(std::uint64_t& s);
void seed_stream(std::uint64_t seed, std::uint64_t out[2]);

}  // namespace vsmp
