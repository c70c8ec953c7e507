// Scoped profiler ranges for rocprofv3 (--marker-trace): the counterpart of the
// reference's NVTX::Range (src/utils/device/nvtx.h:23-69). The engine brackets the same
// phases under the same names (EDGEFM_PREFILL, EDGEFM_DECODE_GRAPH_REPLAY, ...,
// standard_engine.cpp:894-1047), so a trace attributes GPU time to prefill, decode
// replay, sampler and response copy. Ranges are host-side markers only; they cost a
// function call when no profiler is attached.
#pragma once

#include <rocprofiler-sdk-roctx/roctx.h>

namespace edge_fm {

class RoctxRange {
public:
    explicit RoctxRange(const char* name) : pushed_(name != nullptr && name[0] != '\0') {
        if (pushed_) roctxRangePushA(name);
    }
    ~RoctxRange() {
        if (pushed_) roctxRangePop();
    }
    RoctxRange(const RoctxRange&) = delete;
    RoctxRange& operator=(const RoctxRange&) = delete;

private:
    bool pushed_;
};

}  // namespace edge_fm
