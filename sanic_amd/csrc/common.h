// Shared plumbing of the HIP backend: error text, HIP status checks, the program model used by
// the emitter and the runtime.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/sanic_hip.h"

namespace sanic {

// A failure carrying the C-ABI status it maps to (compile.rs:42-58 RunError / CompileError).
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& s);

#define SANIC_HIP(call)                                                                      \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            throw ::sanic::Error(SANIC_ERR_BACKEND, std::string(#call) + ": " +              \
                                                        hipGetErrorString(e_));              \
    } while (0)

[[noreturn]] inline void fail(int code, const std::string& m) { throw Error(code, m); }

// One kernel argument: a program buffer's device address, a byte offset into the executable's
// scratch arena, or an immediate 64-bit value.
struct Arg {
    enum Kind { BUF, SCRATCH, IMM } kind;
    int64_t v;
};

// One kernel launch of a lowered stage.
struct Launch {
    std::string kernel;        // symbol name inside the module
    std::string module_key;    // key of the compiled code object
    dim3 grid, block;
    uint32_t lds = 0;          // dynamic LDS bytes
    std::vector<Arg> args;
    hipFunction_t fn = nullptr;
    bool zero_scratch = false; // clear `zero_bytes` of scratch at zero_off before this launch
    int64_t zero_off = 0, zero_bytes = 0;
};

// A stage lowered onto one or more launches.
struct LoweredStage {
    std::string kernel_kind;   // "skeleton:<name>" or "fold:<scalar|coop|split>" or "pointwise"
    std::string source;        // generated HIP source
    int variants = 1;          // tiling variants the lowering offers (sanic_sched.variant)
    std::vector<Launch> launches;
};

struct Lowered {
    std::vector<LoweredStage> stages;
    int64_t scratch_bytes = 0;
};

// Validate a descriptor and lower every stage (emit_hip.cpp).
Lowered lower_program(const sanic_program_desc* d);

// hipRTC compile with an on-disk code-object cache (rtc.cpp).
std::string compile_source(const std::string& source);   // returns the code object bytes

}  // namespace sanic
