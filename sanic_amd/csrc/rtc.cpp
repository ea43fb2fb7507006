// hipRTC compilation of generated kernels, with an on-disk code-object cache keyed by a hash of
// the source and the options (the reference compiles MSL at runtime, metal.rs:166-185; this is
// its counterpart). No fast-math: ±inf and NaN semantics are kept, as the reference does for
// the −∞ mask (tests/reserved_cache.rs:1-12).
#include <hip/hiprtc.h>

#include <dlfcn.h>
#include <sys/stat.h>
#include <utime.h>
#include <unistd.h>

#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <vector>

#include "common.h"

namespace sanic {

static const char* kOptions[] = {
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    // packed-f32 instruction forms are disabled: some have returned wrong results on MI355X
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
};

static uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ULL) {
    for (unsigned char c : s) { h ^= c; h *= 1099511628211ULL; }
    return h;
}

static std::string cache_dir() {
    if (const char* e = getenv("SANIC_HIP_CACHE")) return e;
    Dl_info info;
    if (dladdr((void*)&cache_dir, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        auto slash = p.rfind('/');
        if (slash != std::string::npos) return p.substr(0, slash) + "/_kcache";
    }
    return "/tmp/sanic_hip_kcache";
}

static bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return !out.empty();
}

std::string compile_source(const std::string& generated) {
    std::vector<std::string> opts(std::begin(kOptions), std::end(kOptions));
    // a generated source may open with "// sched-strategy: <name>\n" to pick the machine
    // scheduler's strategy for its kernel (set by the lowering that measured it faster)
    static const std::string kMark = "// sched-strategy: ";
    if (generated.compare(0, kMark.size(), kMark) == 0) {
        const size_t eol = generated.find('\n');
        opts.push_back("-mllvm");
        opts.push_back("-amdgpu-sched-strategy=" + generated.substr(kMark.size(), eol - kMark.size()));
    }
    std::string opts_key;
    for (auto& o : opts) opts_key += o, opts_key += ' ';
    char hex[32];
    snprintf(hex, sizeof hex, "%016llx", (unsigned long long)fnv1a(opts_key + generated));
    // debugging: SANIC_HIP_DUMP=<dir> writes every generated source as <dir>/<hash>.hip
    if (const char* dd = getenv("SANIC_HIP_DUMP")) {
        mkdir(dd, 0755);
        std::ofstream f(std::string(dd) + "/" + hex + ".hip");
        f << generated;
    }
    const std::string& source = generated;
    std::string dir = cache_dir();
    std::string path = dir + "/" + hex + ".co";
    std::string code;
    if (!getenv("SANIC_HIP_NO_CACHE") && read_file(path, code)) {
        utime(path.c_str(), nullptr);   // mark as in use (the build prunes entries it did not touch)
        return code;
    }

    static std::mutex create_mu;
    hiprtcProgram prog;
    hiprtcResult cr;
    {
        std::lock_guard<std::mutex> lk(create_mu);
        cr = hiprtcCreateProgram(&prog, source.c_str(), "sanic_kernel.hip", 0, nullptr, nullptr);
    }
    if (cr != HIPRTC_SUCCESS)
        fail(SANIC_ERR_COMPILE, std::string("hiprtcCreateProgram failed: ") + hiprtcGetErrorString(cr));
    std::vector<const char*> optp;
    for (auto& o : opts) optp.push_back(o.c_str());
    hiprtcResult r = hiprtcCompileProgram(prog, (int)optp.size(), optp.data());
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n + 1, '\0');
        hiprtcGetProgramLog(prog, log.data());
        hiprtcDestroyProgram(&prog);
        fail(SANIC_ERR_COMPILE, "hipRTC compile failed:\n" + log + "\n--- source ---\n" + source);
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    code.resize(n);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    mkdir(dir.c_str(), 0755);
    std::string tmp = path + ".tmp." + std::to_string(getpid());
    {
        std::ofstream f(tmp, std::ios::binary);
        f.write(code.data(), (std::streamsize)code.size());
    }
    rename(tmp.c_str(), path.c_str());
    return code;
}

}  // namespace sanic
