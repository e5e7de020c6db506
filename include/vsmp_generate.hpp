// verbo::generate over a session whose LM head leaves its logits on the GPU: the device-resident
// hand-off. The reference has no such session (Session::eval returns a host row,
// src/session.cpp:196-200); the decode loop is the reference's (src/sampler.cpp:111-181), with the
// sampler's draw stream and history on the device (vsmp_dsampler in vsmp.h), so that per token
// only the 4-byte id crosses to the host, for the stop check and the detokeniser.
#pragma once

#include <functional>
#include <string_view>
#include <vector>

#include "verbo/verbo.hpp"
#include "vsmp.h"

namespace vsmp {

// What a session with a device-resident LM head provides: verbo::Session's decode interface
// (reference include/verbo/verbo.hpp, Session) with eval returning device logits.
class DeviceSession {
 public:
  virtual ~DeviceSession() = default;
  // Logits of the position after ids[0..n) (vocab floats, 16-byte aligned, readable up to the next
  // multiple of 4 floats) in device memory, written on stream() and valid until the next eval.
  virtual const float* eval(const int* ids, int n) = 0;
  virtual int pos() const = 0;
  virtual int ctx() const = 0;
  virtual const verbo::Model& model() const = 0;
  virtual void* stream() const = 0;  // the hipStream_t the logits are written on
};

// verbo::generate (reference src/sampler.cpp:111-181) on a DeviceSession: the same step order,
// Stats and stop-text hold-back, with the sampler state of vsmp_dsampler on the current device.
// Throws std::runtime_error with the library's message on a HIP error.
verbo::Stats generate_device(DeviceSession& ses, const std::vector<int>& prompt, const verbo::GenOpts& opt,
                             const std::function<bool(std::string_view)>& on_text);

}  // namespace vsmp
