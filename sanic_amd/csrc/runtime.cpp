// The HIP runtime behind the C ABI: device, buffers, prepared executables, eager execution and
// hipGraph capture/replay.
//
// Counterparts in the reference: MetalDevice (/root/reference/src/metal.rs:148-838), the Metal
// Backend impl (/root/reference/src/compile.rs:694-787) and MetalReplay
// (/root/reference/src/compile.rs:800-1035). One HIP stream per device serialises the stages,
// so the reference's static barrier schedule (metal.rs:754-796) is implied by stream order; a
// replay is one hipGraph whose kernel nodes follow that order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>

#include "emit.h"

namespace sanic {

static thread_local std::string g_last_error;
void set_last_error(const std::string& s) { g_last_error = s; }

}  // namespace sanic

using namespace sanic;

struct sanic_hip_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    char* scratch_ptr = nullptr;   // this GPU's copy of `scratch` (execute_static)
};

// ── the static scratch of sanic_hip_execute_static ─────────────────────────────────────────
// Device memory that entry point uses beyond the caller's inputs and outputs: the
// executable's split-partial / arrival-counter arena and its intermediate (SCRATCH-role)
// buffers, laid out back to back at 256-byte alignment. Every GPU the library runs on holds
// its own copy until the process ends. In host code `scratch` names a host-side stand-in, not
// a device address: host code uses only the per-device address hipGetSymbolAddress returns
// (sanic_hip_device::scratch_ptr, taken in sanic_hip_open with the device current).
static const size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

// Which XCD each workgroup of a launch runs on (the hardware register XCC_ID): kernels that let
// the workgroups sharing an arrival counter exchange partials through one XCD's L2 rely on the
// dispatcher's round-robin placement (linear block b on XCD b mod 8). Checked once per GPU at
// its first open, on a grid of an odd size; any other placement switches those kernels to the
// device-coherent exchange for the rest of the process.
__global__ void sanic_xcc_probe(int* out) {
    if (threadIdx.x == 0) {
        unsigned v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = (int)(v & 0xF);
    }
}

static bool probe_xcd_round_robin(hipStream_t stream, char* dev_buf) {
    const int kBlocks = 1001;
    int* out = (int*)dev_buf;
    hipLaunchKernelGGL(sanic_xcc_probe, dim3(kBlocks), dim3(64), 0, stream, out);
    if (hipGetLastError() != hipSuccess) return false;
    std::vector<int> h(kBlocks, -1);
    if (hipMemcpyAsync(h.data(), out, kBlocks * sizeof(int), hipMemcpyDeviceToHost, stream) != hipSuccess) return false;
    if (hipStreamSynchronize(stream) != hipSuccess) return false;
    bool seen[16] = {};
    for (int b = 0; b < kBlocks; b++) {
        if (h[b] != b % 8) return false;
        seen[h[b]] = true;
    }
    for (int x = 0; x < 8; x++)
        if (!seen[x]) return false;
    return true;
}

// One event per GPU marking the end of the last sanic_hip_execute_static call's work on that
// GPU. Each call makes its stream wait on it before touching the scratch and records it after
// enqueueing, so calls from different device handles (each with its own stream) on one GPU are
// ordered instead of racing on the shared scratch. Created once per ordinal in sanic_hip_open.
static std::mutex g_static_mu;
static std::map<int, hipEvent_t> g_static_done;

struct Storage {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool owned = false;
    int ordinal = 0;
    ~Storage() {
        if (owned && ptr) {
            hipSetDevice(ordinal);
            hipFree(ptr);
        }
    }
};

struct sanic_hip_buffer {
    sanic_hip_device* dev = nullptr;
    std::shared_ptr<Storage> storage;
    size_t offset = 0;
    size_t bytes = 0;
    char* ptr() const { return (char*)storage->ptr + offset; }
};

struct Module {
    hipModule_t mod = nullptr;
};

struct sanic_hip_exe {
    sanic_hip_device* dev = nullptr;
    std::vector<sanic_buffer_desc> buffers;
    std::vector<int> stage_out;       // output buffer of each stage
    std::vector<int> stage_out_role;
    Lowered low;
    std::map<std::string, std::shared_ptr<Module>> modules;  // source -> module
    ~sanic_hip_exe() {
        for (auto& kv : modules)
            if (kv.second->mod) hipModuleUnload(kv.second->mod);
    }
};

struct sanic_hip_replay {
    sanic_hip_exe* exe = nullptr;
    std::vector<sanic_hip_buffer*> bound;     // per program buffer (borrowed or owned)
    std::vector<std::unique_ptr<sanic_hip_buffer>> owned;
    std::unique_ptr<sanic_hip_buffer> scratch;
    std::vector<std::pair<int, int>> feedback;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // kMultiStep consecutive steps in one graph (built on the first step_many that can use it):
    // back-to-back steps then pay one graph launch per kMultiStep steps instead of one each
    hipGraph_t graph_n = nullptr;
    hipGraphExec_t graph_n_exec = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    ~sanic_hip_replay() {
        if (graph_n_exec) hipGraphExecDestroy(graph_n_exec);
        if (graph_n) hipGraphDestroy(graph_n);
        if (graph_exec) hipGraphExecDestroy(graph_exec);
        if (graph) hipGraphDestroy(graph);
        if (ev0) hipEventDestroy(ev0);
        if (ev1) hipEventDestroy(ev1);
    }
};

// ── built-in kernels: scratch clearing (graph-safe, no memset nodes) and feedback conversion ──

__global__ void sanic_zero_words(uint32_t* p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0u;
}

__device__ float load_as_float(const void* p, int dt, float scale, int64_t i) {
    switch (dt) {
    case SANIC_Q8: return (float)((const int8_t*)p)[i] * scale;
    case SANIC_F32: return ((const float*)p)[i];
    case SANIC_BF16: return __uint_as_float(((uint32_t)((const uint16_t*)p)[i]) << 16);
    case SANIC_U32: return (float)((const uint32_t*)p)[i];
    case SANIC_F16: return (float)((const _Float16*)p)[i];
    default: return 0.0f;
    }
}

__device__ void store_from_float(void* p, int dt, float scale, int64_t i, float v) {
    switch (dt) {
    case SANIC_Q8: ((int8_t*)p)[i] = (int8_t)__builtin_fminf(__builtin_fmaxf(__builtin_rintf(v / scale), -127.0f), 127.0f); break;
    case SANIC_F32: ((float*)p)[i] = v; break;
    case SANIC_BF16: {
        uint32_t b = __float_as_uint(v);
        uint16_t r = (v != v) ? (uint16_t)((b >> 16) | 0x40u) : (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
        ((uint16_t*)p)[i] = r;
        break;
    }
    case SANIC_U32: ((uint32_t*)p)[i] = v >= 4294967040.0f ? 0xFFFFFFFFu : (!(v > 0.0f) ? 0u : (uint32_t)(v + 0.5f)); break;
    case SANIC_F16: ((_Float16*)p)[i] = (_Float16)v; break;
    default: break;
    }
}

__global__ void sanic_convert(const void* src, int sdt, float sscale, void* dst, int ddt, float dscale, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) store_from_float(dst, ddt, dscale, i, load_as_float(src, sdt, sscale, i));
}

// ── helpers ──────────────────────────────────────────────────────────────────────────────

template <class F>
static int guarded(F&& f) {
    try {
        f();
        return SANIC_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return SANIC_ERR_BACKEND;
    }
}

static int64_t buffer_bytes(const sanic_buffer_desc& b) {
    int64_t n = 1;
    for (int i = 0; i < b.rank; i++) n *= b.shape[i];
    return dtype_bytes(b.dtype, n);
}

// device allocations made by this library (every one goes through new_buffer)
static std::atomic<uint64_t> g_device_allocations{0};

static sanic_hip_buffer* new_buffer(sanic_hip_device* dev, size_t bytes) {
    SANIC_HIP(hipSetDevice(dev->ordinal));
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    auto st = std::make_shared<Storage>();
    st->bytes = bytes;
    st->owned = true;
    st->ordinal = dev->ordinal;
    SANIC_HIP(hipMalloc(&st->ptr, std::max<size_t>(bytes, 256)));
    auto* b = new sanic_hip_buffer;
    b->dev = dev;
    b->storage = st;
    b->bytes = bytes;
    return b;
}

static void compile_all(sanic_hip_exe* exe, bool load) {
    std::vector<std::string> sources;
    for (auto& s : exe->low.stages)
        if (!s.launches.empty() && !exe->modules.count(s.source)) {
            exe->modules[s.source] = std::make_shared<Module>();
            sources.push_back(s.source);
        }
    std::vector<std::string> codes(sources.size());
    std::vector<std::string> errors(sources.size());
    std::vector<int> err_codes(sources.size(), 0);
    std::atomic<size_t> next{0};
    int nthreads = (int)std::min<size_t>(sources.size(), std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; t++)
        pool.emplace_back([&] {
            for (size_t i = next++; i < sources.size(); i = next++) {
                try {
                    codes[i] = compile_source(sources[i]);
                } catch (const Error& e) {
                    errors[i] = e.what();
                    err_codes[i] = e.code;
                }
            }
        });
    for (auto& th : pool) th.join();
    for (size_t i = 0; i < sources.size(); i++)
        if (err_codes[i]) fail(err_codes[i], errors[i]);
    if (!load) return;
    for (size_t i = 0; i < sources.size(); i++)
        SANIC_HIP(hipModuleLoadData(&exe->modules[sources[i]]->mod, codes[i].data()));
    for (auto& s : exe->low.stages)
        for (auto& l : s.launches)
            SANIC_HIP(hipModuleGetFunction(&l.fn, exe->modules[s.source]->mod, l.kernel.c_str()));
}

// Enqueue every stage's launches on the device stream. `bound[i]` is program buffer i.
static void enqueue(sanic_hip_exe* exe, const std::vector<sanic_hip_buffer*>& bound, char* arena,
                    hipEvent_t* stage_events = nullptr) {
    hipStream_t s = exe->dev->stream;
    for (size_t si = 0; si < exe->low.stages.size(); si++) {
        if (stage_events) SANIC_HIP(hipEventRecord(stage_events[si], s));
        for (auto& l : exe->low.stages[si].launches) {
            if (l.zero_scratch && l.zero_bytes > 0) {
                int64_t words = l.zero_bytes / 4;
                unsigned blocks = (unsigned)std::min<int64_t>((words + 255) / 256, 4096);
                hipLaunchKernelGGL(sanic_zero_words, dim3(blocks), dim3(256), 0, s, (uint32_t*)(arena + l.zero_off), words);
                SANIC_HIP(hipGetLastError());
            }
            std::vector<uint64_t> kargs;
            for (auto& a : l.args) {
                switch (a.kind) {
                case Arg::BUF: {
                    sanic_hip_buffer* b = bound[a.v];
                    if (!b) fail(SANIC_ERR_MISSING_INPUT, "buffer " + std::to_string(a.v) + " is not bound");
                    kargs.push_back((uint64_t)(uintptr_t)b->ptr());
                    break;
                }
                case Arg::SCRATCH: kargs.push_back((uint64_t)(uintptr_t)(arena + a.v)); break;
                case Arg::IMM: kargs.push_back((uint64_t)a.v); break;
                }
            }
            size_t sz = kargs.size() * 8;
            void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, kargs.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                           HIP_LAUNCH_PARAM_END};
            SANIC_HIP(hipModuleLaunchKernel(l.fn, l.grid.x, l.grid.y, l.grid.z, l.block.x, l.block.y, l.block.z,
                                            l.lds, s, nullptr, cfg));
        }
    }
    if (stage_events) SANIC_HIP(hipEventRecord(stage_events[exe->low.stages.size()], s));
}

static void check_binding(sanic_hip_exe* exe, int i, sanic_hip_buffer* b) {
    const sanic_buffer_desc& bd = exe->buffers[i];
    if (!b) fail(SANIC_ERR_MISSING_INPUT, "program buffer " + std::to_string(i) + " is not bound (MissingInput)");
    if ((int64_t)b->bytes < buffer_bytes(bd))
        fail(SANIC_ERR_SHAPE, "program buffer " + std::to_string(i) + " binding holds " + std::to_string(b->bytes) +
                                  " bytes; its shape needs " + std::to_string(buffer_bytes(bd)));
    if (b->dev != exe->dev) fail(SANIC_ERR_ARG, "binding lives on another device");
}

// ── SANIC_DEBUG (the reference's debug levels, lib.rs:25-46, compile.rs:1141-1300) ─────────
// 1: the compiled schedule at prepare (one line per stage: output buffer, kernel kind, launch
//    shape, logical bytes); 2: one line per replay call with its GPU time and the fraction of
//    the HBM peak its logical bytes reach; 3: the frozen graph's launches once at capture;
//    4: the first step of each replay call runs stage by stage between GPU events and prints
//    each stage's time, share and bandwidth. Logical bytes = sizes of the buffers a launch
//    binds (an upper bound on its traffic), as the reference counts them.

static const double kHbmBytesPerS = 8.0e12;   // MI355X HBM3E peak

static int debug_level() {
    static int level = [] {
        const char* e = getenv("SANIC_DEBUG");
        return e ? atoi(e) : 0;
    }();
    return level;
}

static double launch_bytes(const std::vector<sanic_buffer_desc>& buffers, const Launch& l) {
    double b = 0;
    for (auto& a : l.args)
        if (a.kind == Arg::BUF) b += (double)buffer_bytes(buffers[a.v]);
    return b;
}

static double stage_bytes(const std::vector<sanic_buffer_desc>& buffers, const LoweredStage& s) {
    double b = 0;
    for (auto& l : s.launches) b += launch_bytes(buffers, l);
    return b;
}

static void dump_schedule(const char* what, const sanic_program_desc* d, const Lowered& low) {
    std::vector<sanic_buffer_desc> buffers(d->buffers, d->buffers + d->n_buffers);
    double total = 0;
    fprintf(stderr, "*** hip %s: %d stages\n", what, (int)low.stages.size());
    for (size_t i = 0; i < low.stages.size(); i++) {
        const LoweredStage& s = low.stages[i];
        const double mb = stage_bytes(buffers, s) / 1e6;
        total += mb;
        std::string shape;
        for (auto& l : s.launches)
            shape += " grid=(" + std::to_string(l.grid.x) + "," + std::to_string(l.grid.y) + ") block=" + std::to_string(l.block.x);
        fprintf(stderr, "***   %4zu b%-4d %-44s%s ~%.1fMB\n", i, d->stages[i].out_buffer, s.kernel_kind.c_str(),
                shape.empty() ? " (in another launch)" : shape.c_str(), mb);
    }
    fprintf(stderr, "*** hip %s: ~%.1fMB logical\n", what, total);
}

static double program_bytes(const sanic_hip_exe* exe) {
    double b = 0;
    for (auto& s : exe->low.stages) b += stage_bytes(exe->buffers, s);
    return b;
}

// ── C ABI ────────────────────────────────────────────────────────────────────────────────

extern "C" {

const char* sanic_hip_last_error(void) { return g_last_error.c_str(); }

int sanic_hip_open(int ordinal, sanic_hip_device** out) {
    return guarded([&] {
        if (!out) fail(SANIC_ERR_ARG, "null out");
        *out = nullptr;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n <= ordinal || ordinal < 0)
            fail(SANIC_ERR_BACKEND, "no HIP device " + std::to_string(ordinal));
        auto* d = new sanic_hip_device;
        d->ordinal = ordinal;
        SANIC_HIP(hipSetDevice(ordinal));
        SANIC_HIP(hipGetDeviceProperties(&d->props, ordinal));
        SANIC_HIP(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
        void* sp = nullptr;
        hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (se != hipSuccess || !sp) {
            hipStreamDestroy(d->stream);
            delete d;
            fail(SANIC_ERR_BACKEND, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se));
        }
        d->scratch_ptr = (char*)sp;
        {
            std::lock_guard<std::mutex> lk(g_static_mu);
            if (!g_static_done.count(ordinal)) {
                hipEvent_t ev = nullptr;
                hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
                if (ee != hipSuccess) {
                    hipStreamDestroy(d->stream);
                    delete d;
                    fail(SANIC_ERR_BACKEND, std::string("hipEventCreateWithFlags: ") + hipGetErrorString(ee));
                }
                g_static_done[ordinal] = ev;
                // first open of this GPU: nothing has used its static scratch yet
                if (!probe_xcd_round_robin(d->stream, d->scratch_ptr)) set_xcd_local(false);
            }
        }
        *out = d;
    });
}

void sanic_hip_close(sanic_hip_device* dev) {
    if (!dev) return;
    hipSetDevice(dev->ordinal);
    if (dev->stream) {
        hipStreamSynchronize(dev->stream);
        hipStreamDestroy(dev->stream);
    }
    delete dev;
}

int sanic_hip_specs(sanic_hip_device* dev, sanic_device_specs* out) {
    return guarded([&] {
        if (!dev || !out) fail(SANIC_ERR_ARG, "null argument");
        memset(out, 0, sizeof *out);
        snprintf(out->name, sizeof out->name, "%s", dev->props.gcnArchName);
        out->compute_units = dev->props.multiProcessorCount;
        out->wave_size = dev->props.warpSize;
        out->lds_bytes_per_cu = 160 * 1024;
        out->hbm_bytes_per_s = kHbmBytesPerS;
        out->bf16_mfma_flops = 2.5e15;             // dense bf16 MFMA
        out->f32_flops = 157.3e12;
        out->clock_hz = dev->props.clockRate * 1000.0;
        out->hbm_bytes = (int64_t)dev->props.totalGlobalMem;
        const MachineSpecs m = mi355x_specs();
        out->sram_bytes = m.sram_bytes;
        out->regfile_bytes = m.regfile_bytes;
        out->launch_overhead_s = m.launch;
        out->min_blocks = 2.0 * out->compute_units;
        out->mem_latency_s = m.latency;
    });
}

int sanic_hip_alloc(sanic_hip_device* dev, size_t bytes, sanic_hip_buffer** out) {
    return guarded([&] {
        if (!dev || !out) fail(SANIC_ERR_ARG, "null argument");
        *out = new_buffer(dev, bytes);
    });
}

void sanic_hip_free(sanic_hip_buffer* buf) { delete buf; }

int sanic_hip_upload(sanic_hip_buffer* buf, size_t offset, const void* host, size_t bytes) {
    return guarded([&] {
        if (!buf || (!host && bytes)) fail(SANIC_ERR_ARG, "null argument");
        if (offset + bytes > buf->bytes) fail(SANIC_ERR_ARG, "upload past the end of the buffer");
        SANIC_HIP(hipSetDevice(buf->dev->ordinal));
        SANIC_HIP(hipMemcpyAsync(buf->ptr() + offset, host, bytes, hipMemcpyHostToDevice, buf->dev->stream));
        SANIC_HIP(hipStreamSynchronize(buf->dev->stream));
    });
}

int sanic_hip_download(sanic_hip_buffer* buf, size_t offset, void* host, size_t bytes) {
    return guarded([&] {
        if (!buf || (!host && bytes)) fail(SANIC_ERR_ARG, "null argument");
        if (offset + bytes > buf->bytes) fail(SANIC_ERR_ARG, "download past the end of the buffer");
        SANIC_HIP(hipSetDevice(buf->dev->ordinal));
        SANIC_HIP(hipMemcpyAsync(host, buf->ptr() + offset, bytes, hipMemcpyDeviceToHost, buf->dev->stream));
        SANIC_HIP(hipStreamSynchronize(buf->dev->stream));
    });
}

int sanic_hip_slice(sanic_hip_buffer* buf, size_t offset, size_t bytes, sanic_hip_buffer** out) {
    return guarded([&] {
        if (!buf || !out) fail(SANIC_ERR_ARG, "null argument");
        if (offset % 4) fail(SANIC_ERR_ARG, "slice offsets must be 4-byte aligned (metal.rs:80-90)");
        if (offset + bytes > buf->bytes) fail(SANIC_ERR_ARG, "slice past the end of the buffer");
        auto* b = new sanic_hip_buffer(*buf);
        b->offset = buf->offset + offset;
        b->bytes = bytes;
        *out = b;
    });
}

size_t sanic_hip_buffer_bytes(const sanic_hip_buffer* buf) { return buf ? buf->bytes : 0; }
void* sanic_hip_buffer_device_ptr(const sanic_hip_buffer* buf) { return buf ? buf->ptr() : nullptr; }

int sanic_hip_wrap(sanic_hip_device* dev, void* device_ptr, size_t bytes, sanic_hip_buffer** out) {
    return guarded([&] {
        if (!dev || !out || !device_ptr) fail(SANIC_ERR_ARG, "null argument");
        auto st = std::make_shared<Storage>();
        st->ptr = device_ptr;
        st->bytes = bytes;
        st->owned = false;
        auto* b = new sanic_hip_buffer;
        b->dev = dev;
        b->storage = st;
        b->bytes = bytes;
        *out = b;
    });
}

int sanic_hip_prepare(sanic_hip_device* dev, const sanic_program_desc* desc, sanic_hip_exe** out) {
    return guarded([&] {
        if (!dev || !desc || !out) fail(SANIC_ERR_ARG, "null argument");
        *out = nullptr;
        SANIC_HIP(hipSetDevice(dev->ordinal));
        auto exe = std::make_unique<sanic_hip_exe>();
        exe->dev = dev;
        exe->low = lower_program(desc);
        exe->buffers.assign(desc->buffers, desc->buffers + desc->n_buffers);
        for (int s = 0; s < desc->n_stages; s++) {
            exe->stage_out.push_back(desc->stages[s].out_buffer);
            exe->stage_out_role.push_back(desc->buffers[desc->stages[s].out_buffer].role);
        }
        compile_all(exe.get(), true);
        if (debug_level() >= 1) dump_schedule("schedule", desc, exe->low);
        *out = exe.release();
    });
}

void sanic_hip_exe_free(sanic_hip_exe* exe) { delete exe; }

static int copy_text(const std::string& s, char* out, size_t cap) {
    if (!out || cap == 0) fail(SANIC_ERR_ARG, "null output");
    size_t n = std::min(cap - 1, s.size());
    memcpy(out, s.data(), n);
    out[n] = 0;
    if (s.size() >= cap) fail(SANIC_ERR_ARG, "output buffer too small: need " + std::to_string(s.size() + 1));
    return 0;
}

int sanic_hip_exe_stage_kernel(const sanic_hip_exe* exe, int stage, char* out, size_t cap) {
    return guarded([&] {
        if (!exe || stage < 0 || stage >= (int)exe->low.stages.size()) fail(SANIC_ERR_ARG, "stage out of range");
        copy_text(exe->low.stages[stage].kernel_kind, out, cap);
    });
}

int sanic_hip_exe_stage_source(const sanic_hip_exe* exe, int stage, char* out, size_t cap) {
    return guarded([&] {
        if (!exe || stage < 0 || stage >= (int)exe->low.stages.size()) fail(SANIC_ERR_ARG, "stage out of range");
        copy_text(exe->low.stages[stage].source, out, cap);
    });
}

// Allocate the executable-owned buffers (OUTPUT, SCRATCH roles) and the scratch arena.
static void bind_all(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n, std::vector<sanic_hip_buffer*>& bound,
                     std::vector<std::unique_ptr<sanic_hip_buffer>>& owned, std::unique_ptr<sanic_hip_buffer>& scratch) {
    int nb = (int)exe->buffers.size();
    if (n != nb) fail(SANIC_ERR_ARG, "expected " + std::to_string(nb) + " bindings, got " + std::to_string(n));
    bound.assign(nb, nullptr);
    for (int i = 0; i < nb; i++) {
        int role = exe->buffers[i].role;
        if (role == SANIC_BUF_INPUT || role == SANIC_BUF_STATE) {
            check_binding(exe, i, bindings ? bindings[i] : nullptr);
            bound[i] = bindings[i];
        } else {
            owned.emplace_back(new_buffer(exe->dev, (size_t)buffer_bytes(exe->buffers[i])));
            bound[i] = owned.back().get();
        }
    }
    scratch.reset(new_buffer(exe->dev, (size_t)std::max<int64_t>(exe->low.scratch_bytes, 256)));
    // arrival counters in the arena must start at zero; kernels re-arm them after each launch
    SANIC_HIP(hipMemsetAsync(scratch->ptr(), 0, scratch->bytes, exe->dev->stream));
    SANIC_HIP(hipStreamSynchronize(exe->dev->stream));
}

int sanic_hip_execute(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings, sanic_hip_buffer** outputs) {
    return guarded([&] {
        if (!exe || !outputs) fail(SANIC_ERR_ARG, "null argument");
        for (int r : exe->stage_out_role)
            if (r == SANIC_BUF_STATE)
                fail(SANIC_ERR_IN_PLACE, "this program writes state in place; use capture (compile.rs:745-751)");
        SANIC_HIP(hipSetDevice(exe->dev->ordinal));
        std::vector<sanic_hip_buffer*> bound;
        std::vector<std::unique_ptr<sanic_hip_buffer>> owned;
        std::unique_ptr<sanic_hip_buffer> scratch;
        bind_all(exe, bindings, n_bindings, bound, owned, scratch);
        enqueue(exe, bound, scratch->ptr());
        SANIC_HIP(hipStreamSynchronize(exe->dev->stream));
        for (int i = 0; i < (int)exe->buffers.size(); i++) outputs[i] = nullptr;
        for (auto& o : owned) {
            for (int i = 0; i < (int)exe->buffers.size(); i++)
                if (bound[i] == o.get() && exe->buffers[i].role == SANIC_BUF_OUTPUT) outputs[i] = o.release();
        }
    });
}

int sanic_hip_execute_static(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings) {
    return guarded([&] {
        if (!exe || !bindings) fail(SANIC_ERR_ARG, "null argument");
        for (int r : exe->stage_out_role)
            if (r == SANIC_BUF_STATE)
                fail(SANIC_ERR_IN_PLACE, "this program writes state in place; use sanic_hip_capture");
        const int nb = (int)exe->buffers.size();
        if (n_bindings != nb) fail(SANIC_ERR_ARG, "expected " + std::to_string(nb) + " bindings, got " + std::to_string(n_bindings));
        char* base = exe->dev->scratch_ptr;
        if (!base) fail(SANIC_ERR_BACKEND, "the device has no static scratch address");
        // layout: the arena first, then every SCRATCH-role buffer, each at 256-byte alignment
        auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
        const int64_t arena = up(std::max<int64_t>(exe->low.scratch_bytes, 0));
        int64_t need = arena;
        std::vector<int64_t> at(nb, -1);
        for (int i = 0; i < nb; i++)
            if (exe->buffers[i].role == SANIC_BUF_SCRATCH) {
                at[i] = need;
                need += up(buffer_bytes(exe->buffers[i]));
            }
        if (need > (int64_t)kStaticScratchBytes)
            fail(SANIC_ERR_ARG, "this program needs " + std::to_string(need) + " bytes of scratch; the static scratch holds " +
                                    std::to_string(kStaticScratchBytes));
        std::vector<sanic_hip_buffer> views(nb);
        std::vector<sanic_hip_buffer*> bound(nb, nullptr);
        auto whole = std::make_shared<Storage>();     // not owned: never freed
        whole->ptr = base;
        whole->bytes = kStaticScratchBytes;
        for (int i = 0; i < nb; i++) {
            if (at[i] >= 0) {
                views[i].dev = exe->dev;
                views[i].storage = whole;
                views[i].offset = (size_t)at[i];
                views[i].bytes = (size_t)buffer_bytes(exe->buffers[i]);
                bound[i] = &views[i];
            } else {
                check_binding(exe, i, bindings[i]);
                bound[i] = bindings[i];
            }
        }
        SANIC_HIP(hipSetDevice(exe->dev->ordinal));
        hipStream_t s = exe->dev->stream;
        hipEvent_t done;
        {
            std::lock_guard<std::mutex> lk(g_static_mu);
            done = g_static_done.at(exe->dev->ordinal);
        }
        // after the previous call's work on this GPU, whichever stream it ran on (a wait on a
        // never-recorded event is satisfied at once); not under graph capture, where an event
        // recorded outside the graph is no dependency the graph can hold
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        SANIC_HIP(hipStreamIsCapturing(s, &cap));
        const bool eager = cap == hipStreamCaptureStatusNone;
        if (eager) SANIC_HIP(hipStreamWaitEvent(s, done, 0));
        // arrival counters start at zero (a fill kernel, not a memset: safe under graph capture)
        if (arena > 0) {
            const int64_t words = arena / 4;
            hipLaunchKernelGGL(sanic_zero_words, dim3((unsigned)std::min<int64_t>((words + 255) / 256, 4096)), dim3(256), 0, s,
                               (uint32_t*)base, words);
            SANIC_HIP(hipGetLastError());
        }
        enqueue(exe, bound, base);
        if (eager) SANIC_HIP(hipEventRecord(done, s));
    });
}

uint64_t sanic_hip_device_allocations(void) { return g_device_allocations.load(std::memory_order_relaxed); }

static const int kMultiStep = 8;

// Capture `steps` consecutive steps (every stage, then the feedback conversions) into one graph.
static void capture_steps(sanic_hip_replay* rp, int steps, hipGraph_t* graph, hipGraphExec_t* exec) {
    sanic_hip_exe* exe = rp->exe;
    hipStream_t s = exe->dev->stream;
    SANIC_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
        for (int step = 0; step < steps; step++) {
            enqueue(exe, rp->bound, rp->scratch->ptr());
            for (auto& fb : rp->feedback) {
                const auto& ob = exe->buffers[fb.first];
                const auto& ib = exe->buffers[fb.second];
                int64_t n = 1;
                for (int k = 0; k < ob.rank; k++) n *= ob.shape[k];
                hipLaunchKernelGGL(sanic_convert, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                                   (const void*)rp->bound[fb.first]->ptr(), ob.dtype, ob.scale,
                                   (void*)rp->bound[fb.second]->ptr(), ib.dtype, ib.scale, n);
            }
        }
    } catch (...) {
        hipGraph_t g;
        hipStreamEndCapture(s, &g);
        if (g) hipGraphDestroy(g);
        throw;
    }
    SANIC_HIP(hipStreamEndCapture(s, graph));
    SANIC_HIP(hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0));
}

int sanic_hip_capture(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings, const int32_t* feedback,
                      int n_pairs, sanic_hip_replay** out) {
    return guarded([&] {
        if (!exe || !out) fail(SANIC_ERR_ARG, "null argument");
        *out = nullptr;
        SANIC_HIP(hipSetDevice(exe->dev->ordinal));
        auto rp = std::make_unique<sanic_hip_replay>();
        rp->exe = exe;
        bind_all(exe, bindings, n_bindings, rp->bound, rp->owned, rp->scratch);
        int nb = (int)exe->buffers.size();
        for (int p = 0; p < n_pairs; p++) {
            int o = feedback[2 * p], i = feedback[2 * p + 1];
            if (o < 0 || o >= nb || i < 0 || i >= nb) fail(SANIC_ERR_FEEDBACK, "feedback index out of range");
            const auto& ob = exe->buffers[o];
            const auto& ib = exe->buffers[i];
            if (ob.role != SANIC_BUF_OUTPUT && ob.role != SANIC_BUF_SCRATCH)
                fail(SANIC_ERR_FEEDBACK, "feedback source must be a program output");
            if (ib.role != SANIC_BUF_INPUT && ib.role != SANIC_BUF_STATE)
                fail(SANIC_ERR_FEEDBACK, "feedback target must be a bound input");
            int64_t no = 1, ni = 1;
            for (int k = 0; k < ob.rank; k++) no *= ob.shape[k];
            for (int k = 0; k < ib.rank; k++) ni *= ib.shape[k];
            if (no != ni) fail(SANIC_ERR_FEEDBACK, "feedback pair volumes differ (RunError::Feedback)");
            for (int dt : {exe->buffers[o].dtype, exe->buffers[i].dtype})
                if (dt != SANIC_F32 && dt != SANIC_BF16 && dt != SANIC_F16 && dt != SANIC_U32 && dt != SANIC_Q8)
                    fail(SANIC_ERR_FEEDBACK, "feedback between unconvertible storage dtypes");
            rp->feedback.push_back({o, i});
        }
        hipStream_t s = exe->dev->stream;
        capture_steps(rp.get(), 1, &rp->graph, &rp->graph_exec);
        if (debug_level() >= 3) {
            int nl = 0;
            for (auto& st : exe->low.stages) nl += (int)st.launches.size();
            fprintf(stderr, "*** hip graph: %d launches + %zu feedback conversions, ~%.1fMB logical\n", nl,
                    rp->feedback.size(), program_bytes(exe) / 1e6);
            for (size_t i = 0; i < exe->low.stages.size(); i++)
                for (auto& l : exe->low.stages[i].launches)
                    fprintf(stderr, "***   %4zu %-32s grid=(%u,%u) block=%u lds=%u ~%.1fMB\n", i, l.kernel.c_str(), l.grid.x,
                            l.grid.y, l.block.x, l.lds, launch_bytes(exe->buffers, l) / 1e6);
        }
        SANIC_HIP(hipEventCreate(&rp->ev0));
        SANIC_HIP(hipEventCreate(&rp->ev1));
        *out = rp.release();
    });
}

int sanic_hip_replay_buffer(sanic_hip_replay* rp, int index, sanic_hip_buffer** out) {
    return guarded([&] {
        if (!rp || !out || index < 0 || index >= (int)rp->bound.size()) fail(SANIC_ERR_ARG, "bad replay buffer index");
        *out = nullptr;
        int role = rp->exe->buffers[index].role;
        if (role != SANIC_BUF_OUTPUT && role != SANIC_BUF_SCRATCH) fail(SANIC_ERR_ARG, "only owned buffers are returned");
        auto* b = new sanic_hip_buffer(*rp->bound[index]);   // shares the storage
        *out = b;
    });
}

int sanic_hip_step_many(sanic_hip_replay* rp, int n, double* gpu_seconds) {
    return guarded([&] {
        if (!rp || n < 1) fail(SANIC_ERR_ARG, "bad replay");
        hipStream_t s = rp->exe->dev->stream;
        SANIC_HIP(hipSetDevice(rp->exe->dev->ordinal));
        const double peak = kHbmBytesPerS;
        int first = 0;
        double first_s = 0;
        if (debug_level() >= 4) {
            // the first step stage by stage between GPU events (the step itself, not a re-run)
            const auto& st = rp->exe->low.stages;
            std::vector<hipEvent_t> ev(st.size() + 1);
            for (auto& e : ev) SANIC_HIP(hipEventCreate(&e));
            enqueue(rp->exe, rp->bound, rp->scratch->ptr(), ev.data());
            SANIC_HIP(hipEventSynchronize(ev[st.size()]));
            float tot = 0;
            SANIC_HIP(hipEventElapsedTime(&tot, ev[0], ev[st.size()]));
            for (size_t i = 0; i < st.size(); i++) {
                if (st[i].launches.empty()) continue;
                float ms = 0;
                hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
                const double bytes = stage_bytes(rp->exe->buffers, st[i]);
                fprintf(stderr, "*** hip  %4zu b%-4d %9.1fus %5.1f%%  ~%8.1fMB bw %3.0f%%  %s\n", i, rp->exe->stage_out[i], ms * 1e3,
                        100.0 * ms / std::max(tot, 1e-9f), bytes / 1e6, 100.0 * bytes / std::max(ms * 1e-3, 1e-12) / peak,
                        st[i].kernel_kind.c_str());
            }
            fprintf(stderr, "*** hip  stage-by-stage step %.1fus (between events: includes each stage's launch)\n", tot * 1e3);
            for (auto& e : ev) hipEventDestroy(e);
            first = 1;
            first_s = tot * 1e-3;
            // feedback conversions of that step
            for (auto& fb : rp->feedback) {
                const auto& ob = rp->exe->buffers[fb.first];
                const auto& ib = rp->exe->buffers[fb.second];
                int64_t cnt = 1;
                for (int k = 0; k < ob.rank; k++) cnt *= ob.shape[k];
                hipLaunchKernelGGL(sanic_convert, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s,
                                   (const void*)rp->bound[fb.first]->ptr(), ob.dtype, ob.scale,
                                   (void*)rp->bound[fb.second]->ptr(), ib.dtype, ib.scale, cnt);
            }
            SANIC_HIP(hipStreamSynchronize(s));
        }
        const int many = (n - first) / kMultiStep;
        if (many > 0 && !rp->graph_n_exec) capture_steps(rp, kMultiStep, &rp->graph_n, &rp->graph_n_exec);
        SANIC_HIP(hipEventRecord(rp->ev0, s));
        for (int i = 0; i < many; i++) SANIC_HIP(hipGraphLaunch(rp->graph_n_exec, s));
        for (int i = first + many * kMultiStep; i < n; i++) SANIC_HIP(hipGraphLaunch(rp->graph_exec, s));
        SANIC_HIP(hipEventRecord(rp->ev1, s));
        SANIC_HIP(hipEventSynchronize(rp->ev1));
        float ms = 0;
        SANIC_HIP(hipEventElapsedTime(&ms, rp->ev0, rp->ev1));
        const double secs = ms * 1e-3 + first_s;
        if (gpu_seconds) *gpu_seconds = secs;
        if (debug_level() >= 2) {
            const double per = secs / n, bytes = program_bytes(rp->exe);
            fprintf(stderr, "*** hip batched %zu stages x%d %8.3fms GPU per step  ~%.0fMB bw %3.0f%%\n", rp->exe->low.stages.size(), n,
                    per * 1e3, bytes / 1e6, 100.0 * bytes / std::max(per, 1e-12) / peak);
        }
    });
}

int sanic_hip_step(sanic_hip_replay* rp, double* gpu_seconds) { return sanic_hip_step_many(rp, 1, gpu_seconds); }

void sanic_hip_replay_free(sanic_hip_replay* rp) { delete rp; }

int sanic_hip_profile_stages(sanic_hip_replay* rp, double* seconds, int n) {
    return guarded([&] {
        if (!rp || !seconds) fail(SANIC_ERR_ARG, "null argument");
        int ns = (int)rp->exe->low.stages.size();
        if (n < ns) fail(SANIC_ERR_ARG, "seconds[] is shorter than the stage count");
        std::vector<hipEvent_t> ev(ns + 1);
        for (auto& e : ev) SANIC_HIP(hipEventCreate(&e));
        enqueue(rp->exe, rp->bound, rp->scratch->ptr(), ev.data());
        SANIC_HIP(hipEventSynchronize(ev[ns]));
        for (int i = 0; i < ns; i++) {
            float ms = 0;
            hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
            seconds[i] = ms * 1e-3;
        }
        for (auto& e : ev) hipEventDestroy(e);
    });
}

int sanic_hip_sync(sanic_hip_device* dev) {
    return guarded([&] {
        if (!dev) fail(SANIC_ERR_ARG, "null device");
        SANIC_HIP(hipStreamSynchronize(dev->stream));
    });
}

// ── device-free entry points: emit and precompile without a GPU ────────────────────────────

int sanic_hip_emit_source(const sanic_program_desc* desc, int stage, char* kind, size_t kcap, char* src, size_t scap) {
    return guarded([&] {
        Lowered low = lower_program(desc);
        if (stage < 0 || stage >= (int)low.stages.size()) fail(SANIC_ERR_ARG, "stage out of range");
        if (kind) copy_text(low.stages[stage].kernel_kind, kind, kcap);
        if (src) copy_text(low.stages[stage].source, src, scap);
    });
}

int sanic_hip_stage_variants(const sanic_program_desc* desc, int stage, int* count) {
    return guarded([&] {
        Lowered low = lower_program(desc);
        if (!count) fail(SANIC_ERR_ARG, "null count");
        auto one = [&](int i) { return low.stages[i].launches.empty() ? 0 : low.stages[i].variants; };
        if (stage == -1) {
            for (int i = 0; i < (int)low.stages.size(); i++) count[i] = one(i);
            return;
        }
        if (stage < 0 || stage >= (int)low.stages.size()) fail(SANIC_ERR_ARG, "stage out of range");
        *count = one(stage);
    });
}

int sanic_hip_precompile(const sanic_program_desc* desc) {
    return guarded([&] {
        sanic_hip_exe exe;
        exe.low = lower_program(desc);
        if (debug_level() >= 1) dump_schedule("schedule", desc, exe.low);
        compile_all(&exe, false);
    });
}

size_t sanic_hip_abi_sizeof(const char* name) {
    std::string n = name ? name : "";
    if (n == "sanic_node") return sizeof(sanic_node);
    if (n == "sanic_expr") return sizeof(sanic_expr);
    if (n == "sanic_slot") return sizeof(sanic_slot);
    if (n == "sanic_carrier") return sizeof(sanic_carrier);
    if (n == "sanic_sched") return sizeof(sanic_sched);
    if (n == "sanic_stage") return sizeof(sanic_stage);
    if (n == "sanic_buffer_desc") return sizeof(sanic_buffer_desc);
    if (n == "sanic_program_desc") return sizeof(sanic_program_desc);
    if (n == "sanic_device_specs") return sizeof(sanic_device_specs);
    return 0;
}

}  // extern "C"
