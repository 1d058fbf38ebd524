// Per-kernel timing of one step: an event is recorded on the launch stream
// after every kernel, tagged with the kernel's algorithmic work, so the
// profiler entry point can attribute time kernel by kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

namespace volta {

struct KernelMark {
  std::string label;
  double flops;  // algorithmic fp32 flops of the launch
  double bytes;  // algorithmic HBM bytes of the launch
  hipEvent_t ev;
};

struct Recorder {
  hipStream_t st = nullptr;
  hipEvent_t start = nullptr;
  std::vector<KernelMark> marks;

  hipError_t mark(const std::string& label, double flops, double bytes) {
    hipEvent_t e = nullptr;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) return err;
    marks.push_back({label, flops, bytes, e});
    return hipEventRecord(e, st);
  }

  ~Recorder() {
    for (auto& m : marks)
      if (m.ev) (void)hipEventDestroy(m.ev);
    if (start) (void)hipEventDestroy(start);
  }
};

// Record a mark when a recorder is attached; propagate errors.
inline hipError_t mark(Recorder* rec, const std::string& label, double flops, double bytes) {
  return rec ? rec->mark(label, flops, bytes) : hipSuccess;
}

}  // namespace volta
