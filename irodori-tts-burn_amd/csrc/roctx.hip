// Run-time loading of the roctx range API (see roctx.hpp).
#include <dlfcn.h>

#include <cstdlib>
#include <cstring>
#include <mutex>

#include "roctx.hpp"

namespace irodori {

const RoctxApi* roctx_api() {
    static std::once_flag once;
    static RoctxApi api{};
    static bool on = false;
    std::call_once(once, [] {
        const char* env = std::getenv("IRODORI_ROCTX");
        if (!env || std::strcmp(env, "1") != 0) return;
        void* lib = dlopen("librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_GLOBAL);
        if (!lib) lib = dlopen("/opt/rocm/lib/librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_GLOBAL);
        if (!lib) return;
        api.push = reinterpret_cast<int (*)(const char*)>(dlsym(lib, "roctxRangePushA"));
        api.pop = reinterpret_cast<int (*)()>(dlsym(lib, "roctxRangePop"));
        on = api.push && api.pop;
    });
    return on ? &api : nullptr;
}

}  // namespace irodori

extern "C" int irodori_roctx_enabled(void) { return irodori::roctx_api() ? 1 : 0; }
