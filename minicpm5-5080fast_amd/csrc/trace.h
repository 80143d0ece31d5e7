// trace.h - roctx ranges around the library's launchers (the counterpart of
// the reference's optional NVTX ranges, native/kernels/sm120/kernels.h:78-86).
// Switched at run time instead of at build time: set MC_ROCTX in the
// environment (read once) and every mc_kv_* launcher and mc_* step pushes a
// named range that rocprofv3 --marker-trace records; unset, a range costs
// one branch on a cached flag.
#pragma once

#include <rocprofiler-sdk-roctx/roctx.h>

namespace mckv {

bool trace_enabled();

class TraceRange {
  public:
    explicit TraceRange(const char* name) : on_(trace_enabled()) {
        if (on_) roctxRangePushA(name);
    }
    ~TraceRange() {
        if (on_) roctxRangePop();
    }
    TraceRange(const TraceRange&) = delete;
    TraceRange& operator=(const TraceRange&) = delete;

  private:
    bool on_;
};

}  // namespace mckv
