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

// Two modes: every kernel (target < 0: an event after each launch), or one
// kernel bracketed (target = k: events `before` and `after` launch k only,
// so a captured graph of the step carries just two extra nodes).
struct Recorder {
  hipStream_t st = nullptr;
  hipEvent_t start = nullptr;
  std::vector<KernelMark> marks;
  int target = -1;
  bool empty = false;  // record `after` right behind `before` (the markers' own cost)
  int count = 0;
  hipEvent_t before = nullptr;  // recorded by the caller when target == 0
  hipEvent_t after = nullptr;
  std::string target_label;

  hipError_t mark(const std::string& label, double flops, double bytes) {
    if (target >= 0) {
      const int k = count++;
      hipError_t err = hipSuccess;
      if (k == target - 1) {
        err = hipEventRecord(before, st);
        if (empty && err == hipSuccess) err = hipEventRecord(after, st);
      }
      if (k == target) {
        target_label = label;
        if (!empty) err = hipEventRecord(after, st);
      }
      return err;
    }
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
    if (before) (void)hipEventDestroy(before);
    if (after) (void)hipEventDestroy(after);
  }
};

// Record a mark when a recorder is attached; propagate errors.
inline hipError_t mark(Recorder* rec, const std::string& label, double flops, double bytes) {
  return rec ? rec->mark(label, flops, bytes) : hipSuccess;
}

}  // namespace volta
