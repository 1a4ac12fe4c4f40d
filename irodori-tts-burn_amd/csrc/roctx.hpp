// Host-side range annotations for rocprofv3 --marker-trace, under the names of the
// reference's NVTX ranges (profiling.rs:29-92; used at dit/model.rs:238-392,
// diffusion.rs:88-158, euler_sampler.rs:409-580).  The reference compiles them in with its
// `profile` feature; here they are chosen at run time: with IRODORI_ROCTX=1 in the
// environment at the first range, librocprofiler-sdk-roctx is loaded with dlopen and every
// range is one roctxRangePushA / roctxRangePop pair.  Otherwise a range costs one branch.
// The ranges mark host-side spans (enqueues and graph launches; kernels run asynchronously,
// and the per-block ranges of a captured sampler evaluation appear once, at its capture).
#pragma once

namespace irodori {

struct RoctxApi {
    int (*push)(const char*);
    int (*pop)();
};
// The loaded API, or null when ranges are off (not requested, or the library is missing).
const RoctxApi* roctx_api();

class RoctxRange {
   public:
    explicit RoctxRange(const char* name) : api_(roctx_api()) {
        if (api_) api_->push(name);
    }
    ~RoctxRange() {
        if (api_) api_->pop();
    }
    RoctxRange(const RoctxRange&) = delete;
    RoctxRange& operator=(const RoctxRange&) = delete;

   private:
    const RoctxApi* api_;
};

}  // namespace irodori
