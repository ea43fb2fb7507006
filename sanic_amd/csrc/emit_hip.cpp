// emit_hip — lowers a validated program descriptor onto HIP kernels.
//
// The counterpart of the reference's Metal emitter (/root/reference/src/emit_metal.rs) and its
// shared node→code recursion (/root/reference/src/codegen.rs:283-522), written for gfx950:
//   * every fused stage is first offered to the hand-written CDNA4 skeletons (skeletons.cpp),
//     which accept a stage from the structure of its carrier and leaves, never from a name;
//   * otherwise it becomes the generic carrier fold: scalar (one lane per output point,
//     emit_metal.rs:626-736), cooperative (a workgroup of wave64s folds one output point's
//     stream and merges partial carriers with the carrier's own combine through DPP shuffles
//     then LDS, emit_metal.rs:760-1101) or split (workgroups fold disjoint stream slices into a
//     scratch arena and a second kernel merges them with the combine: the split-K combine,
//     oracle interp.rs:555-643);
//   * pointwise stages become one lane per output element, with the in-place `where` storing
//     only where its condition holds (emit_metal.rs:1103-1178).
// All arithmetic is f32 (accumulators included); loads widen from the storage dtype and the
// single store narrows through it (emit_metal.rs:162-232).
#include "emit.h"
#include "skeletons.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <map>
#include <set>
#include <sstream>

namespace sanic {

// ───────────────────────────── validation ─────────────────────────────────────────────────

static int64_t vol(const int64_t* s, int r) {
    int64_t v = 1;
    for (int i = 0; i < r; i++) v *= s[i];
    return v;
}

static std::vector<int64_t> shp(const sanic_node& n) { return {n.shape, n.shape + n.rank}; }

// Ordering (HIP's scoped memory model): every thread's partial stores happen before the
// barrier (workgroup scope), the barrier before thread 0's agent-scope release RMW. The last
// arriver's RMW reads the release sequence of every earlier arrival, and its agent-scope
// acquire fence after the RMW synchronises with all of them; the fence happens before that
// workgroup's barrier and so before every one of its threads reads the partials. The
// waitcnt makes each wave's own stores complete before the barrier, so the release has nothing
// of theirs left in flight.
// true until a GPU's probe at its first open finds another placement (read by lowerings that
// may run on other threads)
static std::atomic<bool> g_xcd_local{true};
void set_xcd_local(bool on) { g_xcd_local.store(on, std::memory_order_relaxed); }
bool xcd_local_enabled() { return g_xcd_local.load(std::memory_order_relaxed) && !getenv("SANIC_HIP_AGENT_MERGE"); }

void emit_arrival(Code& k, const std::string& flag, const std::string& tid, const std::string& cnt,
                  const std::string& expected, bool xcd_local) {
    k.line("__shared__ int " + flag + ";");
    k.line("__builtin_amdgcn_s_waitcnt(0);");
    k.line("__syncthreads();");
    if (xcd_local) {
        // one XCD: the waitcnt above has every wave's partial stores acknowledged by the XCD's
        // L2 before the barrier, the counter RMW is performed there after them, and the last
        // arriver's loads issue after its RMW returns (the barrier below) — no L2 write-back,
        // no invalidation, no round trip past the L2
        k.line("if (" + tid + " == 0) " + flag + " = __hip_atomic_fetch_add(" + cnt + ", 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (" + expected + ") - 1u;");
        k.line("__syncthreads();");
        return;
    }
    // release on every arrival; only the last arriver, which goes on to read the others'
    // partials, takes the acquire (a fence after its RMW, which reads the release sequence of
    // every earlier arrival) — the others skip the acquire's cache invalidation
    k.line("if (" + tid + " == 0) {");
    k.line("  " + flag + " = __hip_atomic_fetch_add(" + cnt + ", 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == (" + expected + ") - 1u;");
    k.line("  if (" + flag + ") __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, \"agent\");");
    k.line("}");
    k.line("__syncthreads();");
}

MachineSpecs mi355x_specs() {
    // HBM3E peak; f32 VALU peak; LDS a workgroup may allocate; one CU's vector registers; the
    // measured dependent-launch floor; 2 workgroups per CU fill the chip; loaded HBM latency
    return {8.0e12, 157.3e12, 160.0 * 1024, 4 * 128.0 * 1024, 2.6e-6, 2.0 * 256, 2.0e-6};
}

int64_t dtype_bytes(int dt, int64_t n) {
    switch (dt) {
    case SANIC_F64: return 8 * n;
    case SANIC_F32: case SANIC_U32: return 4 * n;
    case SANIC_F16: case SANIC_BF16: return 2 * n;
    case SANIC_I8: case SANIC_Q8: return n;
    case SANIC_I4: case SANIC_U4: return (n + 1) / 2;
    }
    fail(SANIC_ERR_DTYPE, "unknown dtype " + std::to_string(dt));
}

static void check_node(const sanic_program_desc* d, int i) {
    const sanic_node& n = d->nodes[i];
    auto bad = [&](const std::string& m) {
        fail(SANIC_ERR_COMPILE, "node " + std::to_string(i) + ": " + m);
    };
    if (n.rank < 0 || n.rank > SANIC_MAX_RANK) bad("rank out of range");
    for (int k = 0; k < n.rank; k++)
        if (n.shape[k] < 1) bad("non-positive extent");
    for (int k = 0; k < n.n_in; k++)
        if (n.in[k] < 0 || n.in[k] >= i) bad("child index must precede the node");
    auto child = [&](int k) -> const sanic_node& { return d->nodes[n.in[k]]; };
    switch (n.kind) {
    case SANIC_NODE_INPUT: {
        if (n.buffer < 0 || n.buffer >= d->n_buffers) bad("input buffer out of range");
        const sanic_buffer_desc& b = d->buffers[n.buffer];
        if (b.rank != n.rank || vol(b.shape, b.rank) != vol(n.shape, n.rank)) bad("input shape differs from its buffer");
        for (int k = 0; k < n.rank; k++) if (b.shape[k] != n.shape[k]) bad("input shape differs from its buffer");
        if (b.dtype != n.dtype) bad("input dtype differs from its buffer");
        if (n.dtype == SANIC_F64) bad("f64 buffers are not a device storage format");
        break;
    }
    case SANIC_NODE_CONST: if (n.rank != 0) bad("const must be rank 0"); break;
    case SANIC_NODE_IOTA: if (n.rank != 1) bad("iota must be rank 1"); break;
    case SANIC_NODE_COORDINATE: if (n.dim < 0 || n.dim >= n.rank) bad("coordinate dim"); break;
    case SANIC_NODE_FOLD: break;
    case SANIC_NODE_MAP: {
        int ar = (n.op == SANIC_OP_WHERE) ? 3 : (n.op <= SANIC_OP_LT ? 2 : 1);
        if (n.op < 0 || n.op > SANIC_OP_ROUND_F16 || n.n_in != ar) bad("map arity");
        if (n.op == SANIC_OP_ROUND_Q8 && !(n.value > 0.0)) bad("Q8 rounding needs a positive scale");
        for (int k = 0; k < n.n_in; k++) {
            const sanic_node& c = child(k);
            if (c.rank > n.rank) bad("map input rank exceeds output rank");
            int lead = n.rank - c.rank;
            for (int j = 0; j < c.rank; j++)
                if (c.shape[j] != 1 && c.shape[j] != n.shape[lead + j]) bad("map broadcast mismatch");
        }
        break;
    }
    case SANIC_NODE_REDUCE: {
        const sanic_node& c = child(0);
        if (n.n_in != 1 || n.dim < 0 || n.dim >= c.rank || n.rank != c.rank - 1) bad("reduce shape");
        for (int j = 0, o = 0; j < c.rank; j++)
            if (j != n.dim && c.shape[j] != n.shape[o++]) bad("reduce shape");
        if (n.op < 0 || n.op > SANIC_MON_LSE) bad("reduce monoid");
        break;
    }
    case SANIC_NODE_SCAN: {
        const sanic_node& c = child(0);
        if (n.n_in != 1 || n.dim < 0 || n.dim >= c.rank || n.rank != c.rank) bad("scan shape");
        for (int j = 0; j < c.rank; j++)
            if (c.shape[j] != n.shape[j]) bad("scan shape");
        if (n.op < 0 || n.op > SANIC_MON_LSE) bad("scan monoid");
        break;
    }
    case SANIC_NODE_GATHER: {
        const sanic_node& s = child(0);
        const sanic_node& x = child(1);
        if (n.n_in != 2 || n.dim < 0 || n.dim >= s.rank || n.rank != s.rank - 1 + x.rank) bad("gather shape");
        for (int j = 0; j < n.rank; j++) {
            int64_t want = j < n.dim ? s.shape[j] : j < n.dim + x.rank ? x.shape[j - n.dim] : s.shape[j - x.rank + 1];
            if (n.shape[j] != want) bad("gather shape");
        }
        break;
    }
    case SANIC_NODE_VIEW: {
        const sanic_node& s = child(0);
        int sd = 0;
        for (int j = 0; j < n.rank; j++) {
            int g = n.group[j];
            if (g < 1 || sd + g > s.rank) bad("view groups");
            if (vol(s.shape + sd, g) != n.shape[j]) bad("view extent");
            sd += g;
        }
        if (sd != s.rank) bad("view groups must cover the source");
        break;
    }
    case SANIC_NODE_REINDEX: {
        const sanic_node& s = child(0);
        int64_t p = n.map_offset;
        if (p < 0) bad("reindex map");
        for (int j = 0; j < s.rank; j++) {
            if (p + 2 > d->n_reindex) bad("reindex table overrun");
            int64_t nt = d->reindex[p];
            p += 2;
            if (nt < 0 || p + 2 * nt > d->n_reindex) bad("reindex table overrun");
            int64_t lo = d->reindex[p - 1], hi = lo;
            for (int64_t t = 0; t < nt; t++) {
                int64_t coef = d->reindex[p + 2 * t], od = d->reindex[p + 2 * t + 1];
                if (od < 0 || od >= n.rank) bad("reindex output dim");
                int64_t span = coef * (n.shape[od] - 1);
                if (span < 0) lo += span; else hi += span;
            }
            p += 2 * nt;
            if (!n.padded && (lo < 0 || hi >= s.shape[j])) bad("unpadded reindex reads out of bounds");
        }
        break;
    }
    default: bad("unknown node kind");
    }
}

static void check_expr_tree(const sanic_program_desc* d, int root, int max_field, int allowed) {
    if (root < 0 || root >= d->n_exprs) fail(SANIC_ERR_COMPILE, "expr root out of range");
    std::vector<int> st{root};
    while (!st.empty()) {
        int i = st.back();
        st.pop_back();
        if (i < 0 || i >= d->n_exprs) fail(SANIC_ERR_COMPILE, "expr child out of range");
        const sanic_expr& e = d->exprs[i];
        if (e.op >= SANIC_EX_ITEM && e.op <= SANIC_EX_F) {
            if (e.op != allowed && !(allowed == SANIC_EX_A && e.op == SANIC_EX_B))
                fail(SANIC_ERR_COMPILE, "expr reads a field its context does not have");
            if (e.index < 0 || e.index >= max_field) fail(SANIC_ERR_COMPILE, "expr field out of range");
        } else if (e.op != SANIC_EX_CONST) {
            if (e.op < 0 || e.op > SANIC_OP_ROUND_F32) fail(SANIC_ERR_COMPILE, "expr op");
            for (int c : {e.a, e.b, e.c}) if (c >= 0) st.push_back(c);
        }
    }
}

static bool tree_has_fold(const sanic_program_desc* d, int root) {
    const sanic_node& n = d->nodes[root];
    if (n.kind == SANIC_NODE_FOLD) return true;
    for (int k = 0; k < n.n_in; k++) if (tree_has_fold(d, n.in[k])) return true;
    return false;
}

void validate(const sanic_program_desc* d) {
    if (!d || d->n_nodes < 0 || d->n_stages < 1 || d->n_buffers < 1) fail(SANIC_ERR_ARG, "empty program");
    for (int i = 0; i < d->n_nodes; i++) check_node(d, i);
    for (int b = 0; b < d->n_buffers; b++) {
        const sanic_buffer_desc& bd = d->buffers[b];
        if (bd.rank < 0 || bd.rank > SANIC_MAX_RANK) fail(SANIC_ERR_COMPILE, "buffer rank");
        if (bd.dtype == SANIC_Q8 && !(bd.scale > 0.0f)) fail(SANIC_ERR_DTYPE, "Q8 buffer without a positive scale");
        if (bd.role < SANIC_BUF_INPUT || bd.role > SANIC_BUF_SCRATCH) fail(SANIC_ERR_COMPILE, "buffer role");
        dtype_bytes(bd.dtype, 1);
    }
    for (int s = 0; s < d->n_stages; s++) {
        const sanic_stage& st = d->stages[s];
        auto bad = [&](const std::string& m) { fail(SANIC_ERR_COMPILE, "stage " + std::to_string(s) + ": " + m); };
        if (st.out_buffer < 0 || st.out_buffer >= d->n_buffers) bad("output buffer");
        const sanic_buffer_desc& ob = d->buffers[st.out_buffer];
        if (ob.role == SANIC_BUF_INPUT) bad("a stage cannot write an input buffer");
        if (ob.dtype != st.out_dtype) bad("output dtype differs from its buffer");
        if (st.out_dtype == SANIC_F64 || st.out_dtype == SANIC_I4 || st.out_dtype == SANIC_U4 || st.out_dtype == SANIC_I8)
            bad("unstorable output width (compile.rs:426-453)");
        if (st.rank < 0 || st.rank > SANIC_MAX_RANK || vol(st.grid, st.rank) != vol(ob.shape, ob.rank)) bad("grid volume differs from the output buffer");
        for (int k = 0; k < st.rank; k++) if (st.grid[k] < 1) bad("grid extent");
        if (st.kind == SANIC_STAGE_FUSED) {
            if (st.stream < 1) bad("empty stream");
            if (st.n_leaves < 0 || st.n_leaves > SANIC_MAX_LEAVES) bad("leaf count");
            for (int l = 0; l < st.n_leaves; l++) {
                if (st.leaf[l] < 0 || st.leaf[l] >= d->n_nodes) bad("leaf node");
                const sanic_node& ln = d->nodes[st.leaf[l]];
                if (tree_has_fold(d, st.leaf[l])) bad("a leaf cannot read the fold value");
                for (int j = 0; j < ln.rank; j++) {
                    int b = st.bind[l][j];
                    int64_t want = b == SANIC_BIND_STREAM ? st.stream : b == SANIC_BIND_BCAST ? 1 : (b >= 0 && b < st.rank ? st.grid[b] : -1);
                    if (want != ln.shape[j]) bad("leaf " + std::to_string(l) + " dim " + std::to_string(j) + " binding mismatch");
                }
            }
            const sanic_carrier& c = st.carrier;
            if (c.slots < 1 || c.slots > SANIC_MAX_SLOTS) bad("slot count");
            for (int k = 0; k < c.slots; k++) {
                check_expr_tree(d, c.into[k], st.n_leaves, SANIC_EX_ITEM);
                check_expr_tree(d, c.combine[k], c.slots, SANIC_EX_A);
                const sanic_slot& sk = c.kind[k];
                if ((sk.kind == SANIC_SLOT_EXP_SHIFTED || sk.kind == SANIC_SLOT_AT_EXTREMUM) &&
                    (sk.ref_slot < 0 || sk.ref_slot >= c.slots)) bad("slot reference");
            }
            check_expr_tree(d, c.project, c.slots, SANIC_EX_F);
            if (st.epilogue >= 0) {
                if (st.epilogue >= d->n_nodes) bad("epilogue node");
                const sanic_node& en = d->nodes[st.epilogue];
                if (vol(en.shape, en.rank) != vol(st.grid, st.rank) || en.rank != st.rank) bad("epilogue shape");
            }
            for (int i = 0; i < d->n_nodes; i++)
                if (d->nodes[i].kind == SANIC_NODE_FOLD && d->nodes[i].rank != st.rank && st.epilogue >= 0 && tree_has_fold(d, st.epilogue)) {}
            if (st.sched.split < 0 || st.sched.waves < 0 || st.sched.chunk < 0) bad("fold schedule");
        } else if (st.kind == SANIC_STAGE_POINTWISE) {
            if (st.value < 0 || st.value >= d->n_nodes) bad("value node");
            const sanic_node& vn = d->nodes[st.value];
            if (vn.rank > st.rank) bad("value rank");
            if (tree_has_fold(d, st.value)) bad("pointwise value reads a fold");
            if (st.where >= 0 && st.where >= d->n_nodes) bad("where node");
        } else {
            bad("unknown stage kind");
        }
    }
}

// ───────────────────────────── rendering ──────────────────────────────────────────────────

std::string flit(double v) {
    if (std::isnan(v)) return "__builtin_nanf(\"\")";
    if (std::isinf(v)) return v > 0 ? "__builtin_huge_valf()" : "(-__builtin_huge_valf())";
    float f = (float)v;
    if (std::isinf(f)) return f > 0 ? "__builtin_huge_valf()" : "(-__builtin_huge_valf())";
    char buf[64];
    snprintf(buf, sizeof buf, "%a", (double)f);
    return std::string("((float)") + buf + ")";
}

const char* kPrelude = R"PRE(
typedef long long idx_t;
typedef unsigned sanic_u32x4 __attribute__((ext_vector_type(4)));
typedef float sanic_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float sanic_bf16(unsigned short b) { return __uint_as_float(((unsigned)b) << 16); }
__device__ __forceinline__ unsigned short sanic_to_bf16(float v) {
  unsigned b = __float_as_uint(v);
  if (v != v) return (unsigned short)((b >> 16) | 0x0040u);
  return (unsigned short)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float sanic_round_bf16(float v) { return sanic_bf16(sanic_to_bf16(v)); }
// sin / cos of an f32 angle: Cody–Waite reduction by π/2 (Cody & Waite, "Software Manual for the
// Elementary Functions", 1980) with π/2 split into 8 + 11 significant bits and an f32 tail, so
// n·c1 and n·c2 are exact for |n| < 4096 (|a| < 6400), then the hardware sine / cosine of the
// remainder (|r| ≤ π/4, in revolutions as v_sin/v_cos take them) and the quadrant. Outside that
// range, and for non-finite angles, the library functions.
__device__ __forceinline__ void sanic_sincos_red(float a, float& s, float& c, int& q) {
  const float n = __builtin_rintf(a * 0.63661977236758134f);
  float r = __builtin_fmaf(-n, 0x1.92p0f, a);
  r = __builtin_fmaf(-n, 0x1.fb4p-12f, r);
  r = __builtin_fmaf(-n, 0x1.4442d2p-24f, r);
  const float t = r * 0.15915494309189535f;
  s = __builtin_amdgcn_sinf(t);
  c = __builtin_amdgcn_cosf(t);
  q = (int)n & 3;
}
__device__ __forceinline__ float sanic_sin(float a) {
  if (!(__builtin_fabsf(a) < 6400.0f)) return sinf(a);
  float s, c; int q;
  sanic_sincos_red(a, s, c, q);
  return q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
}
__device__ __forceinline__ float sanic_cos(float a) {
  if (!(__builtin_fabsf(a) < 6400.0f)) return cosf(a);
  float s, c; int q;
  sanic_sincos_red(a, s, c, q);
  return q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
}
__device__ __forceinline__ unsigned sanic_to_u32(float v) {
  if (v >= 4294967040.0f) return 0xFFFFFFFFu;
  if (!(v > 0.0f)) return 0u;
  return (unsigned)(v + 0.5f);
}
// Q8 store: v/s rounded half-to-even in f32, clamped to the signed grid ±127 (a NaN lands on
// −127, as with a NaN-ignoring clamp)
__device__ __forceinline__ signed char sanic_to_q8(float v, float s) {
  return (signed char)__builtin_fminf(__builtin_fmaxf(__builtin_rintf(v / s), -127.0f), 127.0f);
}
__device__ __forceinline__ float sanic_w4(const unsigned char* p, idx_t i) {
  return (float)(int)((p[i >> 1] >> ((i & 1) << 2)) & 0xF) - 8.0f;
}
__device__ __forceinline__ float sanic_u4(const unsigned char* p, idx_t i) {
  return (float)(int)((p[i >> 1] >> ((i & 1) << 2)) & 0xF);
}
// device-coherent (agent-scope) accesses for data exchanged between workgroups of one kernel:
// written through to the level every XCD sees, read past the local L2
// 16 bytes at base + off from the device-coherent level (the agent-scope atomics' cache
// policy), as one buffer load the compiler can keep in flight with others
__device__ __forceinline__ sanic_f32x4 sanic_ld4(const float* base, unsigned off_bytes) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, 0x7fffffff, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b128(r, off_bytes, 0, 16);
}
template <class T> __device__ __forceinline__ T sanic_ld(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T> __device__ __forceinline__ void sanic_st(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// data exchanged between workgroups of one XCD (the kernel places every workgroup that shares an
// arrival counter on one XCD): plain accesses through that XCD's L2 — stores write through the
// L1, and the merging workgroup reads each partial once per launch, so its L1 (invalidated at
// kernel start) holds no earlier copy
template <class T> __device__ __forceinline__ T sanic_ldx(const T* p) { return *p; }
template <class T> __device__ __forceinline__ void sanic_stx(T* p, T v) { *p = v; }
__device__ __forceinline__ sanic_f32x4 sanic_ldx4(const float* base, unsigned off_bytes) {
  return *(const sanic_f32x4*)((const char*)base + off_bytes);
}
// Cross-lane reductions without the LDS pipe (__shfl_xor lowers to ds_bpermute, ~100 cycles a
// step on a dependent chain): DPP within rows of 16 lanes — quad_perm [1,0,3,2] (lane ^ 1),
// [2,3,0,1] (lane ^ 2), row_ror 4 / 8 — and the gfx950 permlane swaps across rows. After
// permlane32_swap(v, v) the pair holds v[i mod 32] and v[i mod 32 + 32]; after
// permlane16_swap(v, v) lanes of rows 2j and 2j+1 hold rows 2j and 2j+1.
// (a lane whose source is disabled reads `fill`: 0 for sums, its own value for maxima)
template <int C> __device__ __forceinline__ float sanic_dpp(float v, float fill = 0.0f) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), C, 0xF, 0xF, false));
}
__device__ __forceinline__ float sanic_rows_sum(float v) {   // Σ over lanes i, i^16, i^32, i^48
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}
__device__ __forceinline__ float sanic_rows_max(float v) {
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}
__device__ __forceinline__ float sanic_quad_sum(float v) {   // Σ over the 4 lanes of a quad
  v += sanic_dpp<0xB1>(v);
  return v + sanic_dpp<0x4E>(v);
}
__device__ __forceinline__ float sanic_wave_sum(float v) {   // Σ over all 64 lanes, in every lane
  v = sanic_quad_sum(v);
  v += sanic_dpp<0x124>(v);
  v += sanic_dpp<0x128>(v);
  return sanic_rows_sum(v);
}
__device__ __forceinline__ float sanic_wave_max(float v) {
  v = __builtin_fmaxf(v, sanic_dpp<0xB1>(v, v));
  v = __builtin_fmaxf(v, sanic_dpp<0x4E>(v, v));
  v = __builtin_fmaxf(v, sanic_dpp<0x124>(v, v));
  v = __builtin_fmaxf(v, sanic_dpp<0x128>(v, v));
  return sanic_rows_max(v);
}
__device__ __forceinline__ float sanic_stride4_sum(float v) { // Σ over lanes ≡ i (mod 4)
  v += sanic_dpp<0x124>(v);
  v += sanic_dpp<0x128>(v);
  return sanic_rows_sum(v);
}
__device__ __forceinline__ float sanic_half_sum(float v) {   // Σ over lanes i, i^32
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float sanic_stride8_sum(float v) { // Σ over lanes ≡ i (mod 8)
  return sanic_rows_sum(v + sanic_dpp<0x128>(v));
}
// The partner's value at one step of an ascending butterfly (off = 1, 2, 4, ...): before the
// step with offset `off` every aligned group of `off` lanes holds one value, so any lane of the
// partner group serves — lane ^ 1 and lane ^ 2 by quad_perm, the other half of 8 by
// row_half_mirror, the other half of 16 by row_mirror, then the permlane swaps.
template <int OFF> __device__ __forceinline__ float sanic_bfly(float v) {
  if constexpr (OFF == 1) return sanic_dpp<0xB1>(v, v);
  else if constexpr (OFF == 2) return sanic_dpp<0x4E>(v, v);
  else if constexpr (OFF == 4) return sanic_dpp<0x141>(v, v);
  else if constexpr (OFF == 8) return sanic_dpp<0x140>(v, v);
  else if constexpr (OFF == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  }
}
__device__ __forceinline__ float sanic_lse(float a, float b) {
  if (a == -__builtin_huge_valf()) return b;
  if (b == -__builtin_huge_valf()) return a;
  float m = fmaxf(a, b);
  return m + logf(expf(a - m) + expf(b - m));
}
)PRE";

const char* ctype_of(int dt) {
    switch (dt) {
    case SANIC_F32: return "float";
    case SANIC_F16: return "_Float16";
    case SANIC_BF16: return "unsigned short";
    case SANIC_U32: return "unsigned";
    case SANIC_I8: case SANIC_Q8: return "signed char";
    case SANIC_I4: case SANIC_U4: return "unsigned char";
    }
    return "float";
}

std::string map_expr(int op, const std::string& a, const std::string& b, const std::string& c) {
    switch (op) {
    case SANIC_OP_ADD: return "(" + a + " + " + b + ")";
    case SANIC_OP_SUB: return "(" + a + " - " + b + ")";
    case SANIC_OP_MUL: return "(" + a + " * " + b + ")";
    case SANIC_OP_DIV: return "(" + a + " / " + b + ")";
    case SANIC_OP_MAX: return "fmaxf(" + a + ", " + b + ")";
    case SANIC_OP_MIN: return "fminf(" + a + ", " + b + ")";
    case SANIC_OP_LT: return "((" + a + " < " + b + ") ? 1.0f : 0.0f)";
    case SANIC_OP_NEG: return "(-" + a + ")";
    // relaxed math, as the reference compiles its kernels (metal.rs:164-172): the hardware
    // exp2 / log2 / reciprocal / square root (about 1 ulp) instead of the libm sequences
    case SANIC_OP_RECIP: return "__builtin_amdgcn_rcpf(" + a + ")";
    case SANIC_OP_EXP: return "__builtin_amdgcn_exp2f((" + a + ") * 1.44269504088896341f)";
    case SANIC_OP_LOG: return "(__builtin_amdgcn_logf(" + a + ") * 0.693147180559945309f)";
    case SANIC_OP_SQRT: return "__builtin_amdgcn_sqrtf(" + a + ")";
    case SANIC_OP_TANH: return "tanhf(" + a + ")";
    case SANIC_OP_SIN: return "sanic_sin(" + a + ")";
    case SANIC_OP_COS: return "sanic_cos(" + a + ")";
    case SANIC_OP_WHERE: return "((" + a + " != 0.0f) ? " + b + " : " + c + ")";
    case SANIC_OP_ROUND_BF16: return "sanic_round_bf16(" + a + ")";
    case SANIC_OP_ROUND_F32: return "(" + a + ")";
    case SANIC_OP_ROUND_F16: return "((float)(_Float16)(" + a + "))";
    }
    fail(SANIC_ERR_COMPILE, "unknown map op");
}

std::string monoid_combine(int m, const std::string& a, const std::string& b) {
    switch (m) {
    case SANIC_MON_ADD: return "(" + a + " + " + b + ")";
    case SANIC_MON_MUL: return "(" + a + " * " + b + ")";
    case SANIC_MON_MAX: return "fmaxf(" + a + ", " + b + ")";
    case SANIC_MON_MIN: return "fminf(" + a + ", " + b + ")";
    case SANIC_MON_LSE: return "sanic_lse(" + a + ", " + b + ")";
    }
    fail(SANIC_ERR_COMPILE, "unknown monoid");
}

double monoid_identity(int m) {
    switch (m) {
    case SANIC_MON_ADD: return 0.0;
    case SANIC_MON_MUL: return 1.0;
    case SANIC_MON_MAX: case SANIC_MON_LSE: return -INFINITY;
    default: return INFINITY;
    }
}

std::string Code::str() const { return s.str(); }
void Code::line(const std::string& l) {
    for (int i = 0; i < indent; i++) s << "  ";
    s << l << "\n";
}

std::string Renderer::param(int buffer) {
    auto it = buf_param.find(buffer);
    if (it != buf_param.end()) return it->second;
    // parameters are named by position, not by program buffer: stages that differ only in which
    // buffers they read (the layers of a model) render to the same source and share one code
    // object (the reference dedups isomorphic kernels, emit_metal.rs:1283-1327)
    std::string name = "a.b" + std::to_string(bufs.size());
    buf_param[buffer] = name;
    bufs.push_back(buffer);
    return name;
}

std::string Renderer::fresh(const char* p) { return std::string(p) + std::to_string(tmp++); }

std::string Renderer::args_struct(const std::vector<std::string>& extra) const {
    std::ostringstream o;
    o << "struct Args {\n";
    for (size_t i = 0; i < bufs.size(); i++) {
        int dt = d->buffers[bufs[i]].dtype;
        o << "  " << ctype_of(dt) << "* __restrict__ b" << i << ";\n";
    }
    for (auto& e : extra) o << "  " << e << ";\n";
    o << "};\n";
    return o.str();
}

std::vector<Arg> Renderer::arg_list() const {
    std::vector<Arg> v;
    for (int b : bufs) v.push_back({Arg::BUF, b});
    return v;
}

std::string Renderer::load(int node, const std::vector<std::string>& c) {
    const sanic_node& n = d->nodes[node];
    std::string lin;
    for (int j = 0; j < n.rank; j++) {
        if (j == 0) lin = "(idx_t)(" + c[0] + ")";
        else lin = "(" + lin + " * " + std::to_string(n.shape[j]) + " + (idx_t)(" + c[j] + "))";
    }
    if (lin.empty()) lin = "0";
    std::string p = param(n.buffer);
    if (coherent.count(n.buffer)) {
        std::string a = "sanic_ld(" + p + " + " + lin + ")";
        switch (n.dtype) {
        case SANIC_F32: return a;
        case SANIC_BF16: return "sanic_bf16(" + a + ")";
        case SANIC_F16: case SANIC_U32: case SANIC_I8: return "(float)" + a;
        case SANIC_Q8: return "((float)" + a + " * " + flit(d->buffers[n.buffer].scale) + ")";
        }
    }
    switch (n.dtype) {
    case SANIC_F32: return p + "[" + lin + "]";
    case SANIC_F16: return "(float)" + p + "[" + lin + "]";
    case SANIC_BF16: return "sanic_bf16(" + p + "[" + lin + "])";
    case SANIC_U32: return "(float)" + p + "[" + lin + "]";
    case SANIC_I8: return "(float)" + p + "[" + lin + "]";
    // dequantization is the load: the buffer's scale as a literal (emit_metal.rs:134-137)
    case SANIC_Q8: return "((float)" + p + "[" + lin + "] * " + flit(d->buffers[n.buffer].scale) + ")";
    case SANIC_I4: return "sanic_w4(" + p + ", " + lin + ")";
    case SANIC_U4: return "sanic_u4(" + p + ", " + lin + ")";
    }
    fail(SANIC_ERR_DTYPE, "unloadable dtype");
}

// Emit the value of `node` at coordinates `c` (integer expressions) into `code`; returns an
// expression (usually a fresh local) holding the f32 value.
std::string Renderer::value(Code& code, int node, const std::vector<std::string>& c) {
    const sanic_node& n = d->nodes[node];
    auto sb = subst.find(node);
    if (sb != subst.end()) return sb->second;
    std::string key = std::to_string(node) + "@";
    for (auto& x : c) key += x + ",";
    for (auto it = memo.rbegin(); it != memo.rend(); ++it) {
        auto f = it->find(key);
        if (f != it->end()) return f->second;
    }
    std::string out;
    switch (n.kind) {
    case SANIC_NODE_CONST: return flit(n.value);
    case SANIC_NODE_IOTA: return "((float)(" + c[0] + "))";
    case SANIC_NODE_COORDINATE: return "((float)(" + c[n.dim] + "))";
    case SANIC_NODE_FOLD: return fold_var;
    case SANIC_NODE_INPUT: {
        if (n.rank == 0 && !coherent.count(n.buffer)) {
            // a scalar input (a position, a step count) is loaded once at kernel entry
            auto sv = scalar_vars.find(n.buffer);
            if (sv != scalar_vars.end()) return sv->second;
            std::string v = "sc" + std::to_string(n.buffer);
            scalars.indent = 1;
            scalars.line("const float " + v + " = " + load(node, c) + ";");
            scalar_vars[n.buffer] = v;
            return v;
        }
        out = fresh("v");
        code.line("const float " + out + " = " + load(node, c) + ";");
        break;
    }
    case SANIC_NODE_MAP: {
        std::string a[3];
        for (int k = 0; k < n.n_in; k++) {
            const sanic_node& m = d->nodes[n.in[k]];
            int lead = n.rank - m.rank;
            std::vector<std::string> cc(m.rank);
            for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? "0" : c[lead + j];
            a[k] = value(code, n.in[k], cc);
        }
        out = fresh("m");
        if (n.op == SANIC_OP_ROUND_Q8)   // the value a Q8 store + load gives (emit_metal.rs:100-103)
            code.line("const float " + out + " = (float)sanic_to_q8(" + a[0] + ", " + flit(n.value) + ") * " + flit(n.value) + ";");
        else
            code.line("const float " + out + " = " + map_expr(n.op, a[0], a[1], a[2]) + ";");
        break;
    }
    case SANIC_NODE_SCAN: {
        // each output point folds its own prefix (codegen.rs Scan arm): parallel across points,
        // serial within one; inclusive of the point's own position
        out = fresh("r");
        std::string r = fresh("i");
        code.line("float " + out + " = " + flit(monoid_identity(n.op)) + ";");
        code.line("for (idx_t " + r + " = 0; " + r + " <= (idx_t)(" + c[n.dim] + "); ++" + r + ") {");
        code.indent++;
        memo.emplace_back();
        std::vector<std::string> cc(c);
        cc[n.dim] = r;
        std::string v = value(code, n.in[0], cc);
        code.line(out + " = " + monoid_combine(n.op, out, v) + ";");
        memo.pop_back();
        code.indent--;
        code.line("}");
        break;
    }
    case SANIC_NODE_REDUCE: {
        const sanic_node& m = d->nodes[n.in[0]];
        out = fresh("r");
        std::string r = fresh("i");
        code.line("float " + out + " = " + flit(monoid_identity(n.op)) + ";");
        code.line("for (idx_t " + r + " = 0; " + r + " < " + std::to_string(m.shape[n.dim]) + "; ++" + r + ") {");
        code.indent++;
        memo.emplace_back();
        std::vector<std::string> cc;
        for (int j = 0, o = 0; j < m.rank; j++) cc.push_back(j == n.dim ? r : c[o++]);
        std::string v = value(code, n.in[0], cc);
        code.line(out + " = " + monoid_combine(n.op, out, v) + ";");
        memo.pop_back();
        code.indent--;
        code.line("}");
        break;
    }
    case SANIC_NODE_GATHER: {
        const sanic_node& s = d->nodes[n.in[0]];
        const sanic_node& x = d->nodes[n.in[1]];
        std::vector<std::string> ic(c.begin() + n.dim, c.begin() + n.dim + x.rank);
        std::string iv = value(code, n.in[1], ic);
        std::string gi = fresh("gx");
        // round half away from zero (f64::round), clamped so a bad index cannot fault
        code.line("idx_t " + gi + " = (idx_t)roundf(" + iv + ");");
        code.line(gi + " = " + gi + " < 0 ? 0 : (" + gi + " > " + std::to_string(s.shape[n.dim] - 1) + " ? " +
                  std::to_string(s.shape[n.dim] - 1) + " : " + gi + ");");
        std::vector<std::string> sc;
        for (int j = 0; j < s.rank; j++)
            sc.push_back(j < n.dim ? c[j] : j == n.dim ? gi : c[j - 1 + x.rank]);
        return value(code, n.in[0], sc);
    }
    case SANIC_NODE_VIEW: {
        const sanic_node& s = d->nodes[n.in[0]];
        std::vector<std::string> sc(s.rank);
        int sd = 0;
        for (int j = 0; j < n.rank; j++) {
            int g = n.group[j];
            if (g == 1) { sc[sd] = c[j]; sd++; continue; }
            int64_t inner = 1;
            for (int t = g - 1; t >= 0; t--) {
                int64_t ext = s.shape[sd + t];
                std::string e = "((idx_t)(" + c[j] + ")";
                if (inner != 1) e += " / " + std::to_string(inner);
                e += ")";
                if (t > 0) e = "(" + e + " % " + std::to_string(ext) + ")";
                sc[sd + t] = e;
                inner *= ext;
            }
            sd += g;
        }
        return value(code, n.in[0], sc);
    }
    case SANIC_NODE_REINDEX: {
        const sanic_node& s = d->nodes[n.in[0]];
        std::vector<std::string> sc(s.rank);
        int64_t p = n.map_offset;
        std::string ok;
        for (int j = 0; j < s.rank; j++) {
            int64_t nt = d->reindex[p], off = d->reindex[p + 1];
            p += 2;
            std::string e = std::to_string(off);
            int64_t lo = off, hi = off;
            for (int64_t t = 0; t < nt; t++) {
                int64_t coef = d->reindex[p++], od = d->reindex[p++];
                e += " + " + std::to_string(coef) + " * (idx_t)(" + c[od] + ")";
                int64_t span = coef * (n.shape[od] - 1);
                if (span < 0) lo += span; else hi += span;
            }
            std::string v = fresh("ix");
            code.line("const idx_t " + v + " = " + e + ";");
            sc[j] = v;
            if (n.padded && (lo < 0 || hi >= s.shape[j])) {
                if (!ok.empty()) ok += " && ";
                ok += "(" + v + " >= 0 && " + v + " < " + std::to_string(s.shape[j]) + ")";
            }
        }
        if (ok.empty()) return value(code, n.in[0], sc);
        out = fresh("p");
        code.line("float " + out + " = 0.0f;");
        code.line("if (" + ok + ") {");
        code.indent++;
        memo.emplace_back();
        std::string v = value(code, n.in[0], sc);
        code.line(out + " = " + v + ";");
        memo.pop_back();
        code.indent--;
        code.line("}");
        break;
    }
    default: fail(SANIC_ERR_COMPILE, "unrenderable node");
    }
    memo.back()[key] = out;
    return out;
}

// Render a carrier Expr; fields map through `item`, `a`, `b`, `f` name prefixes.
std::string Renderer::expr(Code& code, int e, const std::string& item, const std::string& a,
                           const std::string& b, const std::string& f) {
    const sanic_expr& x = d->exprs[e];
    switch (x.op) {
    case SANIC_EX_CONST: return flit(x.value);
    case SANIC_EX_ITEM: return item + std::to_string(x.index);
    case SANIC_EX_A: return a + std::to_string(x.index);
    case SANIC_EX_B: return b + std::to_string(x.index);
    case SANIC_EX_F: return f + std::to_string(x.index);
    }
    std::string s[3];
    int kids[3] = {x.a, x.b, x.c};
    for (int k = 0; k < 3; k++) if (kids[k] >= 0) s[k] = expr(code, kids[k], item, a, b, f);
    // structurally equal subexpressions (e.g. the rescale factor every ExpShifted slot of a
    // carrier shares) are computed once per scope
    std::string text = map_expr(x.op, s[0], s[1], s[2]);
    for (auto it = memo.rbegin(); it != memo.rend(); ++it) {
        auto hit = it->find("expr:" + text);
        if (hit != it->end()) return hit->second;
    }
    std::string out = fresh("e");
    code.line("const float " + out + " = " + text + ";");
    memo.back()["expr:" + text] = out;
    return out;
}

std::string store_stmt(const std::string& ptr, const std::string& idx, int dt, const std::string& v, bool coherent, double scale) {
    if (dt == SANIC_Q8) {
        // quantize at the store, clamped to the signed grid (emit_metal.rs:182-185, 226-229)
        if (!(scale > 0.0)) fail(SANIC_ERR_DTYPE, "Q8 store without a positive scale");
        const std::string q = "sanic_to_q8(" + v + ", " + flit(scale) + ")";
        return coherent ? "sanic_st(" + ptr + " + " + idx + ", " + q + ");" : ptr + "[" + idx + "] = " + q + ";";
    }
    if (coherent) {
        switch (dt) {
        case SANIC_F32: return "sanic_st(" + ptr + " + " + idx + ", (float)(" + v + "));";
        case SANIC_F16: return "sanic_st(" + ptr + " + " + idx + ", (_Float16)(" + v + "));";
        case SANIC_BF16: return "sanic_st(" + ptr + " + " + idx + ", sanic_to_bf16(" + v + "));";
        case SANIC_U32: return "sanic_st(" + ptr + " + " + idx + ", sanic_to_u32(" + v + "));";
        }
    }
    switch (dt) {
    case SANIC_F32: return ptr + "[" + idx + "] = " + v + ";";
    case SANIC_F16: return ptr + "[" + idx + "] = (_Float16)" + v + ";";
    case SANIC_BF16: return ptr + "[" + idx + "] = sanic_to_bf16(" + v + ");";
    case SANIC_U32: return ptr + "[" + idx + "] = sanic_to_u32(" + v + ");";
    }
    fail(SANIC_ERR_DTYPE, "unstorable dtype");
}

void decode_grid(Code& code, const sanic_stage& st, const std::string& gid) {
    std::string rem = gid;
    for (int j = st.rank - 1; j >= 0; j--) {
        if (j == 0) code.line("const idx_t g0 = " + rem + ";");
        else {
            code.line("const idx_t g" + std::to_string(j) + " = " + rem + " % " + std::to_string(st.grid[j]) + ";");
            std::string nr = "q" + std::to_string(j);
            code.line("const idx_t " + nr + " = " + rem + " / " + std::to_string(st.grid[j]) + ";");
            rem = nr;
        }
    }
}

std::vector<std::string> leaf_coords(const sanic_stage& st, const sanic_program_desc* d, int l,
                                     const std::string& s) {
    const sanic_node& ln = d->nodes[st.leaf[l]];
    std::vector<std::string> c(ln.rank);
    for (int j = 0; j < ln.rank; j++) {
        int b = st.bind[l][j];
        c[j] = b == SANIC_BIND_STREAM ? s : b == SANIC_BIND_BCAST ? "0" : "g" + std::to_string(b);
    }
    return c;
}

// ───────────────────── honest window (emit_metal.rs:442-505, :555-585) ─────────────────────
// A leaf that adds a prefix mask to the value feeding a Max slot lets the stream stop early:
// masked elements contribute exactly nothing to the (m, ℓ, o) fold once one visible element
// has been folded. Recognised forms (additive terms of the leaf, K ≤ −1e29 or −∞):
//   where(E < s, K, 0)  → visible iff s ≤ E  → hi = floor(E) + 1
//   where(s < E, 0, K)  → visible iff s < E  → hi = ceil(E)
//   where(s < E, K, 0)  → visible iff s ≥ E  → lo = ceil(E)
// where s is the stream coordinate and E does not depend on it.

static bool depends_on_stream(const sanic_program_desc* d, int node, const std::vector<int>& bind_of_dims) {
    // bind_of_dims: for the node's dims, which are the stream (value -1)
    const sanic_node& n = d->nodes[node];
    switch (n.kind) {
    case SANIC_NODE_CONST: return false;
    case SANIC_NODE_IOTA: return bind_of_dims[0] == SANIC_BIND_STREAM;
    case SANIC_NODE_COORDINATE: return bind_of_dims[n.dim] == SANIC_BIND_STREAM;
    case SANIC_NODE_MAP: {
        for (int k = 0; k < n.n_in; k++) {
            const sanic_node& m = d->nodes[n.in[k]];
            int lead = n.rank - m.rank;
            std::vector<int> b(m.rank);
            for (int j = 0; j < m.rank; j++) b[j] = m.shape[j] == 1 ? SANIC_BIND_BCAST : bind_of_dims[lead + j];
            if (depends_on_stream(d, n.in[k], b)) return true;
        }
        return false;
    }
    default: {
        for (int j = 0; j < n.rank; j++) if (bind_of_dims[j] == SANIC_BIND_STREAM) return true;
        return false;
    }
    }
}

static bool is_stream_coord(const sanic_program_desc* d, int node, const std::vector<int>& b) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_IOTA) return b[0] == SANIC_BIND_STREAM;
    if (n.kind == SANIC_NODE_COORDINATE) return b[n.dim] == SANIC_BIND_STREAM;
    return false;
}

static bool is_big_negative(const sanic_program_desc* d, int node) {
    const sanic_node& n = d->nodes[node];
    return n.kind == SANIC_NODE_CONST && n.value <= -1e29;
}
static bool is_zero(const sanic_program_desc* d, int node) {
    const sanic_node& n = d->nodes[node];
    return n.kind == SANIC_NODE_CONST && n.value == 0.0;
}

static std::vector<int> child_bind(const sanic_program_desc* d, int node, int k, const std::vector<int>& b) {
    const sanic_node& n = d->nodes[node];
    const sanic_node& m = d->nodes[n.in[k]];
    int lead = n.rank - m.rank;
    std::vector<int> cb(m.rank);
    for (int j = 0; j < m.rank; j++) cb[j] = m.shape[j] == 1 ? SANIC_BIND_BCAST : b[lead + j];
    return cb;
}

// Collect window bounds from additive mask terms of `node`.
static void collect_window(const sanic_program_desc* d, int node, const std::vector<int>& b,
                           std::vector<WindowBound>& out) {
    const sanic_node& n = d->nodes[node];
    if (n.kind != SANIC_NODE_MAP) return;
    if (n.op == SANIC_OP_ADD) {
        collect_window(d, n.in[0], child_bind(d, node, 0, b), out);
        collect_window(d, n.in[1], child_bind(d, node, 1, b), out);
        return;
    }
    if (n.op != SANIC_OP_WHERE) return;
    const sanic_node& cond = d->nodes[n.in[0]];
    if (cond.kind != SANIC_NODE_MAP || cond.op != SANIC_OP_LT) return;
    std::vector<int> cb = child_bind(d, node, 0, b);
    std::vector<int> lb = child_bind(d, n.in[0], 0, cb), rb = child_bind(d, n.in[0], 1, cb);
    bool l_s = is_stream_coord(d, cond.in[0], lb), r_s = is_stream_coord(d, cond.in[1], rb);
    bool l_dep = depends_on_stream(d, cond.in[0], lb), r_dep = depends_on_stream(d, cond.in[1], rb);
    bool t_big = is_big_negative(d, n.in[1]), t_zero = is_zero(d, n.in[1]);
    bool f_big = is_big_negative(d, n.in[2]), f_zero = is_zero(d, n.in[2]);
    if (r_s && !l_dep && t_big && f_zero) out.push_back({WindowBound::HI_FLOOR_PLUS1, cond.in[0], lb, node});
    else if (l_s && !r_dep && t_zero && f_big) out.push_back({WindowBound::HI_CEIL, cond.in[1], rb, node});
    else if (l_s && !r_dep && t_big && f_zero) out.push_back({WindowBound::LO_CEIL, cond.in[1], rb, node});
}

// Window bounds for a fused stage: only when the carrier has an ExpShifted slot whose max slot's
// `into` is exactly one item, and that item's leaf carries the mask terms.
std::vector<WindowBound> honest_window(const sanic_program_desc* d, const sanic_stage& st) {
    std::vector<WindowBound> out;
    const sanic_carrier& c = st.carrier;
    int max_slot = -1;
    for (int k = 0; k < c.slots; k++)
        if (c.kind[k].kind == SANIC_SLOT_EXP_SHIFTED) {
            if (max_slot >= 0 && max_slot != c.kind[k].ref_slot) return out;
            max_slot = c.kind[k].ref_slot;
        }
    if (max_slot < 0) return out;
    if (c.kind[max_slot].kind != SANIC_SLOT_PLAIN || c.kind[max_slot].monoid != SANIC_MON_MAX) return out;
    const sanic_expr& e = d->exprs[c.into[max_slot]];
    if (e.op != SANIC_EX_ITEM) return out;
    int l = e.index;
    // the masked item may feed only the max slot's into (ExpShifted slots read it via the combine)
    for (int k = 0; k < c.slots; k++) {
        if (k == max_slot) continue;
        std::vector<int> st_{c.into[k]};
        while (!st_.empty()) {
            int i = st_.back(); st_.pop_back();
            const sanic_expr& x = d->exprs[i];
            if (x.op == SANIC_EX_ITEM && x.index == l) return out;
            for (int ch : {x.a, x.b, x.c}) if (ch >= 0 && x.op < SANIC_EX_CONST) st_.push_back(ch);
        }
    }
    const sanic_node& ln = d->nodes[st.leaf[l]];
    std::vector<int> b(st.bind[l], st.bind[l] + ln.rank);
    collect_window(d, st.leaf[l], b, out);
    return out;
}

void emit_window(Renderer& R, Code& code, const sanic_stage& st, const std::vector<WindowBound>& w,
                 const std::string& lo, const std::string& hi) {
    code.line("idx_t " + lo + " = 0, " + hi + " = " + std::to_string(st.stream) + ";");
    for (auto& b : w) {
        std::vector<std::string> c(b.bind.size());
        for (size_t j = 0; j < b.bind.size(); j++)
            c[j] = b.bind[j] == SANIC_BIND_BCAST ? "0" : b.bind[j] == SANIC_BIND_STREAM ? "0" : "g" + std::to_string(b.bind[j]);
        std::string v = R.value(code, b.node, c);
        switch (b.kind) {
        case WindowBound::HI_FLOOR_PLUS1:
            code.line("{ const float w_ = floorf(" + v + ") + 1.0f; if (w_ < (float)" + hi + ") " + hi + " = w_ < 0.0f ? 0 : (idx_t)w_; }");
            break;
        case WindowBound::HI_CEIL:
            code.line("{ const float w_ = ceilf(" + v + "); if (w_ < (float)" + hi + ") " + hi + " = w_ < 0.0f ? 0 : (idx_t)w_; }");
            break;
        case WindowBound::LO_CEIL:
            code.line("{ const float w_ = ceilf(" + v + "); if (w_ > (float)" + lo + ") " + lo + " = w_ > (float)" + std::to_string(st.stream) + " ? " + std::to_string(st.stream) + " : (idx_t)w_; }");
            break;
        }
    }
    // an empty visible range folds the whole stream, as the unmasked definition does
    code.line("if (" + hi + " <= " + lo + ") { " + lo + " = 0; " + hi + " = " + std::to_string(st.stream) + "; }");
}

// ───────────────────────────── generic fold ───────────────────────────────────────────────

static void emit_fold_body(Renderer& R, Code& code, const sanic_stage& st, const std::string& s) {
    const sanic_carrier& c = st.carrier;
    R.memo.emplace_back();
    for (int l = 0; l < st.n_leaves; l++) {
        std::string v = R.value(code, st.leaf[l], leaf_coords(st, R.d, l, s));
        code.line("const float x" + std::to_string(l) + " = " + v + ";");
    }
    for (int k = 0; k < c.slots; k++) {
        std::string v = R.expr(code, c.into[k], "x", "", "", "");
        code.line("const float el" + std::to_string(k) + " = " + v + ";");
    }
    for (int k = 0; k < c.slots; k++) {
        std::string v = R.expr(code, c.combine[k], "", "acc", "el", "");
        code.line("const float nx" + std::to_string(k) + " = " + v + ";");
    }
    for (int k = 0; k < c.slots; k++) code.line("acc" + std::to_string(k) + " = nx" + std::to_string(k) + ";");
    R.memo.pop_back();
}

// merge `acc` with `oth` (acc ⊕ oth) in place
static void emit_merge(Renderer& R, Code& code, const sanic_carrier& c, const std::string& oth) {
    code.line("{");
    code.indent++;
    R.memo.emplace_back();
    for (int k = 0; k < c.slots; k++) {
        std::string v = R.expr(code, c.combine[k], "", "acc", oth, "");
        code.line("const float nx" + std::to_string(k) + " = " + v + ";");
    }
    for (int k = 0; k < c.slots; k++) code.line("acc" + std::to_string(k) + " = nx" + std::to_string(k) + ";");
    R.memo.pop_back();
    code.indent--;
    code.line("}");
}

static void emit_finish(Renderer& R, Code& code, const sanic_stage& st, const std::string& gid) {
    std::string f = R.expr(code, st.carrier.project, "", "", "", "acc");
    code.line("const float fold_v = " + f + ";");
    std::string v = "fold_v";
    if (st.epilogue >= 0) {
        R.fold_var = "fold_v";
        std::vector<std::string> gc;
        for (int j = 0; j < st.rank; j++) gc.push_back("g" + std::to_string(j));
        R.memo.emplace_back();
        v = R.value(code, st.epilogue, gc);
        R.memo.pop_back();
    }
    code.line(store_stmt(R.param(st.out_buffer), gid, st.out_dtype, v, false, R.d->buffers[st.out_buffer].scale));
}

// ── the default schedule of a generic fold (plan.rs:604-850 re-derived for wave64) ─────────
//
// A stage that carries no FoldSched (waves = 0, not lane_stream, split = 1) is priced over the
// candidate schedules this emitter has, with the cost model of cost.rs:150-210 over the MI355X
// figures sanic_hip_specs reports: time = max(compute / (f32 peak · occupancy), bytes /
// sustainable bandwidth) + launch floor, sustainable bandwidth = peak · clamp(bytes in flight /
// (peak · latency), 1/64, 1) (Little's law: lanes × bytes each lane keeps outstanding). The
// candidates: scalar (one lane per output point); one workgroup of 64·w lanes per point (w =
// 1..16) folding a strided stream; and s = 2..64 workgroups per point whose partial carriers the
// last one merges. A split unit must not be empty (64·w·s ≤ stream). Ties go to the cooperative
// form (lanes splitting the stream read consecutive elements, one cache line serving a whole
// wave — a stated rule as in best_fold_sched, not a priced one); the winner's lanes then fold
// contiguous runs of 8, 4 or 2 elements where the stream divides (more bytes in flight per load).
static int64_t count_ops(const sanic_program_desc* d, int node, std::set<int>& seen) {
    if (node < 0 || seen.count(node)) return 0;
    seen.insert(node);
    const sanic_node& n = d->nodes[node];
    int64_t ops = n.kind == SANIC_NODE_CONST ? 0 : 1;
    if (n.kind == SANIC_NODE_REDUCE || n.kind == SANIC_NODE_SCAN) {
        // an in-body contraction re-issues its subtree once per contracted element
        std::set<int> sub;
        return ops + count_ops(d, n.in[0], sub) * std::max<int64_t>(1, d->nodes[n.in[0]].shape[n.dim]);
    }
    for (int k = 0; k < n.n_in; k++) ops += count_ops(d, n.in[k], seen);
    return ops;
}

static int64_t expr_ops(const sanic_program_desc* d, int e) {
    if (e < 0) return 0;
    const sanic_expr& x = d->exprs[e];
    if (x.op >= SANIC_EX_CONST) return 0;
    return 1 + expr_ops(d, x.a) + expr_ops(d, x.b) + expr_ops(d, x.c);
}

static void collect_input_nodes(const sanic_program_desc* d, int node, std::set<int>& out) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_INPUT) out.insert(node);
    for (int k = 0; k < n.n_in; k++) collect_input_nodes(d, n.in[k], out);
}

bool sched_is_auto(const sanic_sched& s) { return !s.lane_stream && s.waves == 0 && s.split <= 1; }

FoldChoice choose_fold_sched(const sanic_program_desc* d, const sanic_stage& st) {
    const MachineSpecs M = mi355x_specs();
    const sanic_carrier& c = st.carrier;
    const double gvol = (double)std::max<int64_t>(1, vol(st.grid, st.rank));
    const double S = (double)std::max<int64_t>(1, st.stream);
    // issue ops per (point, stream element): leaf evaluation + the slot updates
    double per_el = 0;
    std::set<int> seen;
    for (int l = 0; l < st.n_leaves; l++) per_el += (double)count_ops(d, st.leaf[l], seen);
    double slot_ops = 0;
    for (int k = 0; k < c.slots; k++) slot_ops += (double)(expr_ops(d, c.into[k]) + expr_ops(d, c.combine[k]));
    per_el += slot_ops;
    // traffic: every input a leaf reads (once), plus the output; bytes a lane loads per stream
    // step: the widths of the inputs whose leaf carries the streamed axis
    double bytes = 0, streamed = 0;
    std::set<int> bufs_seen;
    for (int l = 0; l < st.n_leaves; l++) {
        std::set<int> ins;
        collect_input_nodes(d, st.leaf[l], ins);
        bool streams = false;
        for (int j = 0; j < d->nodes[st.leaf[l]].rank; j++) streams |= st.bind[l][j] == SANIC_BIND_STREAM;
        for (int in : ins) {
            const sanic_node& n = d->nodes[in];
            const double w = (double)dtype_bytes(n.dtype, 1 << 10) / 1024.0;
            if (streams) streamed += w;
            if (bufs_seen.insert(n.buffer).second) bytes += (double)dtype_bytes(n.dtype, vol(n.shape, n.rank));
        }
    }
    bytes += gvol * 4.0;
    streamed = std::max(streamed, 1.0);
    auto price = [&](int waves, int split, int chunk) -> double {
        const bool scalar = waves == 0;
        const double lanes_per_wg = scalar ? 256.0 : 64.0 * waves;
        const double wgs = scalar ? std::ceil(gvol / 256.0) : gvol * split;
        const double lds = scalar ? c.slots * 4.0 : waves * c.slots * 4.0;
        const double regs = lanes_per_wg * c.slots * 4.0;
        if (lds > M.sram_bytes || regs > M.regfile_bytes) return INFINITY;
        double flops = gvol * S * per_el;
        if (!scalar) flops += gvol * split * std::log2(64.0 * waves) * slot_ops + gvol * split * slot_ops;
        const double resident = std::max(1.0, std::min({std::floor(M.sram_bytes / std::max(lds, 1.0)),
                                                         std::floor(M.regfile_bytes / regs), wgs}));
        const double occ = std::min(1.0, std::max(1.0 / 64.0, resident / M.min_blocks));
        const double lanes = scalar ? gvol : wgs * lanes_per_wg;
        const double in_flight = lanes * streamed * (scalar ? 1.0 : chunk);
        const double bw = M.hbm * std::min(1.0, std::max(1.0 / 64.0, in_flight / (M.hbm * M.latency)));
        return std::max(flops / (M.f32_flops * occ), bytes / bw) + M.launch * (split > 1 && gvol > 4096 ? 2 : 1);
    };
    FoldChoice best{0, 1, 1, price(0, 1, 1)};
    for (int w : {1, 2, 4, 8, 16})
        for (int sp : {1, 2, 4, 8, 16, 32, 64}) {
            if (64.0 * w * sp > S) continue;            // an empty split unit would merge identity
            if (sp > 1 && gvol * sp * c.slots * 4.0 > 16.0 * (1 << 20)) continue;   // partials stay ≤ 16 MiB (half of execute_static's scratch)
            const double t = price(w, sp, 1);
            if (t < best.time || (t == best.time && best.waves == 0)) best = {w, sp, 1, t};
        }
    if (best.waves > 0)
        for (int ch : {8, 4, 2})
            if (st.stream % ((int64_t)64 * best.waves * best.split * ch) == 0) {
                best.chunk = ch;
                break;
            }
    return best;
}

LoweredStage lower_generic_fold(const sanic_program_desc* d, int si, int64_t& scratch, const std::vector<int>& tails) {
    const sanic_stage& st = d->stages[si];
    const sanic_carrier& c = st.carrier;
    LoweredStage L;
    int64_t gvol = vol(st.grid, st.rank);
    auto win = honest_window(d, st);
    sanic_sched sch = st.sched;
    std::string auto_tag;
    if (sched_is_auto(sch)) {
        const FoldChoice fc = choose_fold_sched(d, st);
        sch.lane_stream = fc.waves > 0;
        sch.waves = fc.waves;
        sch.split = fc.split;
        sch.chunk = fc.chunk;
        auto_tag = "[auto w" + std::to_string(fc.waves) + " s" + std::to_string(fc.split) + " c" + std::to_string(fc.chunk) + "]";
    }
    int split = sch.split > 1 ? (int)std::min<int64_t>(sch.split, st.stream) : 1;
    int waves = sch.lane_stream ? std::max(1, std::min(16, sch.waves)) : 0;
    int chunk = std::max(1, sch.chunk);
    Renderer R(d);
    for (int t : tails) R.coherent.insert(d->stages[t].out_buffer);
    if (!tails.empty()) R.coherent.insert(st.out_buffer);   // tails may read the merged result
    Code body;
    body.indent = 1;
    std::ostringstream src;
    src << kPrelude;

    auto init_acc = [&](Code& code) {
        for (int k = 0; k < c.slots; k++) code.line("float acc" + std::to_string(k) + " = " + flit(c.identity[k]) + ";");
    };

    if (waves == 0 && split == 1) {
        L.kernel_kind = "fold:scalar" + auto_tag;
        body.line("const idx_t gid = (idx_t)blockIdx.x * 256 + threadIdx.x;");
        body.line("if (gid >= " + std::to_string(gvol) + ") return;");
        decode_grid(body, st, "gid");
        init_acc(body);
        emit_window(R, body, st, win, "lo", "hi");
        body.line("for (idx_t s = lo; s < hi; ++s) {");
        body.indent++;
        emit_fold_body(R, body, st, "s");
        body.indent--;
        body.line("}");
        emit_finish(R, body, st, "gid");
        src << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) sanic_fold(Args a) {\n"
            << R.entry() << body.str() << "}\n";
        Launch ln{"sanic_fold", "", dim3((unsigned)((gvol + 255) / 256)), dim3(256), 0, R.arg_list()};
        L.launches.push_back(ln);
        L.source = src.str();
        return L;
    }

    // cooperative / split: one workgroup of `nth` lanes folds one (grid point, split slice)
    int nth = 64 * std::max(1, waves);
    int nw = nth / 64;
    L.kernel_kind = (split > 1 ? "fold:split" : "fold:coop") + auto_tag;
    int64_t part_off = scratch;
    const bool fused_merge = split > 1 && gvol <= 4096;
    const int64_t part_bytes = ((gvol * split * c.slots * 4 + 255) / 256) * 256;
    if (split > 1) scratch += part_bytes + (fused_merge ? 256 : 0);
    body.line("const idx_t gid = (idx_t)blockIdx.x / " + std::to_string(split) + ";");
    body.line("const int part = (int)(blockIdx.x % " + std::to_string(split) + ");");
    body.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
    decode_grid(body, st, "gid");
    init_acc(body);
    emit_window(R, body, st, win, "lo0", "hi0");
    body.line("const idx_t span_ = hi0 - lo0;");
    body.line("const idx_t lo = lo0 + (idx_t)part * span_ / " + std::to_string(split) + ";");
    body.line("const idx_t hi = lo0 + ((idx_t)part + 1) * span_ / " + std::to_string(split) + ";");
    body.line("for (idx_t base = lo + (idx_t)t * " + std::to_string(chunk) + "; base < hi; base += " +
              std::to_string((int64_t)nth * chunk) + ") {");
    body.indent++;
    body.line("#pragma unroll");
    body.line("for (int j = 0; j < " + std::to_string(chunk) + "; ++j) {");
    body.indent++;
    body.line("const idx_t s = base + j;");
    body.line("if (s < hi) {");
    body.indent++;
    emit_fold_body(R, body, st, "s");
    body.indent--;
    body.line("}");
    body.indent--;
    body.line("}");
    body.indent--;
    body.line("}");
    // wave-level butterfly: the lower lane's partial is the left operand, so the merge order
    // follows lane order
    for (int off = 1; off < 64; off <<= 1) {
    const std::string offs = std::to_string(off);
    body.line("{");
    body.indent++;
    for (int k = 0; k < c.slots; k++)
        body.line("float o" + std::to_string(k) + " = sanic_bfly<" + offs + ">(acc" + std::to_string(k) + ");");
    body.line("if (lane & " + offs + ") {");
    body.indent++;
    for (int k = 0; k < c.slots; k++)
        body.line("const float sw" + std::to_string(k) + " = acc" + std::to_string(k) + "; acc" + std::to_string(k) + " = o" +
                  std::to_string(k) + "; o" + std::to_string(k) + " = sw" + std::to_string(k) + ";");
    body.indent--;
    body.line("}");
    emit_merge(R, body, c, "o");
    body.indent--;
    body.line("}");
    }
    if (nw > 1) {
        body.line("__shared__ float lds_acc[" + std::to_string(nw) + "][" + std::to_string(c.slots) + "];");
        body.line("if (lane == 0) {");
        for (int k = 0; k < c.slots; k++) body.line("  lds_acc[wv][" + std::to_string(k) + "] = acc" + std::to_string(k) + ";");
        body.line("}");
        body.line("__syncthreads();");
        body.line(fused_merge ? "if (t == 0) {" : "if (t != 0) return;");
        body.line("for (int w = 1; w < " + std::to_string(nw) + "; ++w) {");
        body.indent++;
        for (int k = 0; k < c.slots; k++)
            body.line("const float o" + std::to_string(k) + " = lds_acc[w][" + std::to_string(k) + "];");
        emit_merge(R, body, c, "o");
        body.indent--;
        body.line("}");
    } else {
        body.line(fused_merge ? "if (t == 0) {" : "if (t != 0) return;");
    }
    if (split == 1) {
        emit_finish(R, body, st, "gid");
        src << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(" << nth
            << ") sanic_fold(Args a) {\n" << R.entry() << body.str() << "}\n";
        Launch ln{"sanic_fold", "", dim3((unsigned)gvol), dim3(nth), 0, R.arg_list()};
        L.launches.push_back(ln);
        L.source = src.str();
        return L;
    }
    // split: write the partial carrier, then merge with the combine: in the last workgroup to
    // arrive when the grid is small (then the following small pointwise stages run there too),
    // else in a second kernel
    for (int k = 0; k < c.slots; k++) {
        std::string at = "a.scratch + ((idx_t)gid * " + std::to_string(split) + " + part) * " + std::to_string(c.slots) + " + " + std::to_string(k);
        body.line(fused_merge ? "sanic_st(" + at + ", acc" + std::to_string(k) + ");" : "*(" + at + ") = acc" + std::to_string(k) + ";");
    }
    auto merge_point = [&](Renderer& RR, Code& mb) {
        decode_grid(mb, st, "gid");
        mb.line("const float* pp = a.scratch + (idx_t)gid * " + std::to_string(split * c.slots) + ";");
        for (int k = 0; k < c.slots; k++) mb.line("float acc" + std::to_string(k) + " = sanic_ld(pp + " + std::to_string(k) + ");");
        mb.line("for (int p = 1; p < " + std::to_string(split) + "; ++p) {");
        mb.indent++;
        for (int k = 0; k < c.slots; k++)
            mb.line("const float o" + std::to_string(k) + " = sanic_ld(pp + p * " + std::to_string(c.slots) + " + " + std::to_string(k) + ");");
        emit_merge(RR, mb, c, "o");
        mb.indent--;
        mb.line("}");
        emit_finish(RR, mb, st, "gid");
    };
    if (fused_merge) {
        body.line("}");
        body.line("unsigned* cnt = (unsigned*)((char*)a.scratch + " + std::to_string(part_bytes) + ");");
        emit_arrival(body, "sanic_last", "t", "cnt", "gridDim.x");
        body.line("if (!sanic_last) return;");
        // Few output points: L = split rounded up to a power of two lanes per point load one
        // partial each (all loads in flight at once) and merge in log2(L) butterfly steps of the
        // carrier's combine, the lower partial index always on the left — the same order as the
        // serial walk, so a first-index tie rule (AtExtremum) is kept. Otherwise one thread per
        // point walks its partials.
        int LPP = 1;
        while (LPP < split) LPP <<= 1;
        const bool butterfly = LPP <= 64 && gvol <= (int64_t)(nth / LPP) * 4;
        if (butterfly) {
            const int PPP = nth / LPP;                 // points per pass
            body.line("for (idx_t base = 0; base < " + std::to_string(gvol) + "; base += " + std::to_string(PPP) + ") {");
            body.indent++;
            body.line("const idx_t gid = base + t / " + std::to_string(LPP) + ";");
            body.line("const int p = t % " + std::to_string(LPP) + ";");
            body.line("const bool live = gid < " + std::to_string(gvol) + " && p < " + std::to_string(split) + ";");
            body.line("const float* pp = a.scratch + ((gid < " + std::to_string(gvol) + " ? gid : 0) * " + std::to_string(split) + " + (p < " +
                      std::to_string(split) + " ? p : 0)) * " + std::to_string(c.slots) + ";");
            for (int k = 0; k < c.slots; k++)
                body.line("float acc" + std::to_string(k) + " = live ? sanic_ld(pp + " + std::to_string(k) + ") : " + flit(c.identity[k]) + ";");
            for (int off = 1; off < LPP; off <<= 1) {
            const std::string offs = std::to_string(off);
            body.line("{");
            body.indent++;
            body.line("const bool up = (p & " + offs + ") != 0;");
            for (int k = 0; k < c.slots; k++) {
                std::string ks = std::to_string(k);
                body.line("const float o" + ks + " = sanic_bfly<" + offs + ">(acc" + ks + ");");
                body.line("const float lo" + ks + " = up ? o" + ks + " : acc" + ks + ", hi" + ks + " = up ? acc" + ks + " : o" + ks + ";");
            }
            R.memo.emplace_back();
            for (int k = 0; k < c.slots; k++) {
                std::string v = R.expr(body, c.combine[k], "", "lo", "hi", "");
                body.line("const float nx" + std::to_string(k) + " = " + v + ";");
            }
            R.memo.pop_back();
            for (int k = 0; k < c.slots; k++) body.line("acc" + std::to_string(k) + " = nx" + std::to_string(k) + ";");
            body.indent--;
            body.line("}");
            }
            body.line("if (p == 0 && gid < " + std::to_string(gvol) + ") {");
            body.indent++;
            R.memo.emplace_back();
            decode_grid(body, st, "gid");
            emit_finish(R, body, st, "gid");
            R.memo.pop_back();
            body.indent--;
            body.line("}");
            body.indent--;
            body.line("}");
        } else {
            body.line("for (idx_t gid = t; gid < " + std::to_string(gvol) + "; gid += " + std::to_string(nth) + ") {");
            body.indent++;
            R.memo.emplace_back();
            merge_point(R, body);
            R.memo.pop_back();
            body.indent--;
            body.line("}");
        }
        for (int ts : tails) {
            body.line("__syncthreads();");
            emit_pointwise_loop(R, body, d, ts, "(idx_t)t", nth);
        }
        body.line("if (t == 0) sanic_st(cnt, 0u);");
        src << R.args_struct({"float* __restrict__ scratch"});
        src << "extern \"C\" __global__ void __launch_bounds__(" << nth << ") sanic_fold_split(Args a) {\n" << R.entry() << body.str() << "}\n";
        std::vector<Arg> args = R.arg_list();
        args.push_back({Arg::SCRATCH, part_off});
        L.launches.push_back({"sanic_fold_split", "", dim3((unsigned)(gvol * split)), dim3(nth), 0, args});
        L.kernel_kind = "fold:split+merge" + auto_tag + std::string(tails.empty() ? "" : "+tail" + std::to_string(tails.size()));
        L.source = src.str();
        return L;
    }
    Code mb;
    mb.indent = 1;
    Renderer R2(d);
    R2.bufs = R.bufs;
    R2.buf_param = R.buf_param;
    mb.line("const idx_t gid = (idx_t)blockIdx.x * 256 + threadIdx.x;");
    mb.line("if (gid >= " + std::to_string(gvol) + ") return;");
    merge_point(R2, mb);
    // both kernels share one Args layout: the union of their buffers
    for (int b : R2.bufs) R.param(b);
    src << R.args_struct({"float* __restrict__ scratch"});
    src << "extern \"C\" __global__ void __launch_bounds__(" << nth << ") sanic_fold_part(Args a) {\n" << R.entry() << body.str() << "}\n";
    src << "extern \"C\" __global__ void __launch_bounds__(256) sanic_fold_merge(Args a) {\n" << R2.entry() << mb.str() << "}\n";
    std::vector<Arg> args = R.arg_list();
    args.push_back({Arg::SCRATCH, part_off});
    L.launches.push_back({"sanic_fold_part", "", dim3((unsigned)(gvol * split)), dim3(nth), 0, args});
    L.launches.push_back({"sanic_fold_merge", "", dim3((unsigned)((gvol + 255) / 256)), dim3(256), 0, args});
    L.source = src.str();
    return L;
}

static bool stage_touches_q8(const sanic_program_desc* d, int s);

// Elementwise stage as runs of 8 along its innermost dim: each thread renders 8 consecutive
// outputs with wide loads (render_run) and stores them with one 16-byte (bf16) or two (f32)
// stores. For stages without a `where`, bf16/f32 outputs and an innermost extent that is a
// multiple of 8; the values are the scalar renderer's, element for element.
static bool lower_pointwise_runs(const sanic_program_desc* d, int si, LoweredStage& L) {
    const sanic_stage& st = d->stages[si];
    if (st.where >= 0 || st.rank < 1 || st.grid[st.rank - 1] % 8) return false;
    const int odt = st.out_dtype;
    if ((odt != SANIC_BF16 && odt != SANIC_F32) || d->buffers[st.out_buffer].dtype != odt) return false;
    const sanic_node& vn = d->nodes[st.value];
    std::vector<Sym> c(vn.rank);
    const int lead = st.rank - vn.rank;
    for (int j = 0; j < vn.rank; j++) c[j] = vn.shape[j] == 1 ? Sym() : Sym::var(lead + j);
    std::vector<std::string> vars;
    std::vector<int64_t> ext;
    for (int j = 0; j < st.rank; j++) {
        vars.push_back("g" + std::to_string(j));
        ext.push_back(st.grid[j]);
    }
    Code lc, dc;
    lc.indent = dc.indent = 1;
    std::vector<int> bufs, dts;
    bool ok = true;
    auto vals = render_run(d, st.value, c, ext, vars, st.rank - 1, lc, dc, "_r", bufs, dts, ok);
    if (!ok || vals.size() != 8) return false;
    Renderer R(d);
    Code body;
    body.indent = 1;
    const int64_t gvol = vol(st.grid, st.rank), runs = gvol / 8;
    body.line("const idx_t gr = (idx_t)blockIdx.x * 256 + threadIdx.x;");
    body.line("if (gr >= " + std::to_string(runs) + ") return;");
    body.line("const idx_t gid = gr * 8;");
    decode_grid(body, st, "gid");
    for (size_t b = 0; b < bufs.size(); b++)
        body.line("const " + std::string(ctype_of(dts[b])) + "* __restrict__ rb" + std::to_string(b) + "_r = " + R.param(bufs[b]) + ";");
    body.s << lc.str() << dc.str();
    const std::string out = R.param(st.out_buffer);
    if (odt == SANIC_BF16) {
        std::string w = "(sanic_u32x4){";
        for (int q = 0; q < 4; q++)
            w += std::string(q ? ", " : "") + "(unsigned)sanic_to_bf16(" + vals[2 * q] + ") | ((unsigned)sanic_to_bf16(" + vals[2 * q + 1] + ") << 16)";
        body.line("*(sanic_u32x4*)(" + out + " + gid) = " + w + "};");
    } else {
        body.line("*(sanic_f32x4*)(" + out + " + gid) = (sanic_f32x4){" + vals[0] + ", " + vals[1] + ", " + vals[2] + ", " + vals[3] + "};");
        body.line("*(sanic_f32x4*)(" + out + " + gid + 4) = (sanic_f32x4){" + vals[4] + ", " + vals[5] + ", " + vals[6] + ", " + vals[7] + "};");
    }
    std::ostringstream src;
    src << kPrelude << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) sanic_pointwise_x8(Args a) {\n"
        << R.entry() << body.str() << "}\n";
    L.kernel_kind = "pointwise:runs8";
    L.source = src.str();
    L.launches.push_back({"sanic_pointwise_x8", "", dim3((unsigned)((runs + 255) / 256)), dim3(256), 0, R.arg_list()});
    return true;
}

LoweredStage lower_pointwise(const sanic_program_desc* d, int si) {
    const sanic_stage& st = d->stages[si];
    LoweredStage L;
    if (!getenv("SANIC_HIP_GENERIC") && !stage_touches_q8(d, si) && lower_pointwise_runs(d, si, L)) return L;
    L.kernel_kind = st.where >= 0 ? "pointwise:in-place-where" : "pointwise";
    Renderer R(d);
    Code body;
    body.indent = 1;
    int64_t gvol = vol(st.grid, st.rank);
    body.line("const idx_t gid = (idx_t)blockIdx.x * 256 + threadIdx.x;");
    body.line("if (gid >= " + std::to_string(gvol) + ") return;");
    decode_grid(body, st, "gid");
    std::vector<std::string> gc;
    for (int j = 0; j < st.rank; j++) gc.push_back("g" + std::to_string(j));
    auto at = [&](int node) {
        const sanic_node& n = d->nodes[node];
        int lead = st.rank - n.rank;
        std::vector<std::string> c(n.rank);
        for (int j = 0; j < n.rank; j++) c[j] = n.shape[j] == 1 ? "0" : gc[lead + j];
        return R.value(body, node, c);
    };
    if (st.where >= 0) {
        std::string w = at(st.where);
        body.line("if (" + w + " == 0.0f) return;");
    }
    std::string v = at(st.value);
    body.line(store_stmt(R.param(st.out_buffer), "gid", st.out_dtype, v, false, d->buffers[st.out_buffer].scale));
    std::ostringstream src;
    src << kPrelude << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) sanic_pointwise(Args a) {\n"
        << R.entry() << body.str() << "}\n";
    L.source = src.str();
    L.launches.push_back({"sanic_pointwise", "", dim3((unsigned)((gvol + 255) / 256)), dim3(256), 0, R.arg_list()});
    return L;
}

// Does the stage read or write a Q8 buffer? The hand-written skeletons load and store only the
// float, bf16 and nibble formats; such stages take the generic renderer.
static bool stage_touches_q8(const sanic_program_desc* d, int s) {
    const sanic_stage& st = d->stages[s];
    if (d->buffers[st.out_buffer].dtype == SANIC_Q8) return true;
    std::vector<int> todo;
    if (st.kind == SANIC_STAGE_FUSED) {
        for (int l = 0; l < st.n_leaves; l++) todo.push_back(st.leaf[l]);
        if (st.epilogue >= 0) todo.push_back(st.epilogue);
    } else {
        todo.push_back(st.value);
        if (st.where >= 0) todo.push_back(st.where);
    }
    while (!todo.empty()) {
        const sanic_node& n = d->nodes[todo.back()];
        todo.pop_back();
        if (n.kind == SANIC_NODE_INPUT && n.dtype == SANIC_Q8) return true;
        if (n.kind == SANIC_NODE_MAP && n.op == SANIC_OP_ROUND_Q8) return true;
        if (n.kind != SANIC_NODE_INPUT)
            for (int k = 0; k < n.n_in; k++) todo.push_back(n.in[k]);
    }
    return false;
}

Lowered lower_program(const sanic_program_desc* d) {
    validate(d);
    Lowered out;
    for (int s = 0; s < d->n_stages;) {
        const sanic_stage& st = d->stages[s];
        // skeletons may batch or absorb the next few stages: none of them may touch Q8 either
        bool generic = getenv("SANIC_HIP_GENERIC") != nullptr;
        for (int t = s; t < std::min(d->n_stages, s + 8) && !generic; t++) generic = stage_touches_q8(d, t);
        if (st.kind == SANIC_STAGE_FUSED) {
            std::vector<LoweredStage> grp;
            if (!generic && lower_gemv_group(d, s, out.scratch_bytes, grp)) {
                for (auto& g : grp) out.stages.push_back(std::move(g));
                s += (int)grp.size();
                continue;
            }
            LoweredStage L;
            if (!generic && lower_skeleton(d, s, out.scratch_bytes, L)) {
                out.stages.push_back(std::move(L));
                s++;
                continue;
            }
            // a small split fold merges in its last workgroup and runs the small pointwise
            // stages that follow it there as well
            std::vector<int> tails;
            int64_t gv = 1;
            for (int j = 0; j < st.rank; j++) gv *= st.grid[j];
            sanic_sched es = st.sched;
            if (sched_is_auto(es)) {
                const FoldChoice fc = choose_fold_sched(d, st);
                es.lane_stream = fc.waves > 0;
                es.split = fc.split;
            }
            if (es.lane_stream && es.split > 1 && std::min<int64_t>(es.split, st.stream) > 1 && gv <= 4096)
                for (int t = s + 1; tail_candidate(d, t) && !stage_touches_q8(d, t) && tails.size() < 4; t++) tails.push_back(t);
            L = lower_generic_fold(d, s, out.scratch_bytes, tails);
            out.stages.push_back(std::move(L));
            for (size_t t = 0; t < tails.size(); t++) {
                LoweredStage B;
                B.kernel_kind = "tail-of:" + std::to_string(s);
                out.stages.push_back(std::move(B));
            }
            s += (int)tails.size();
        } else {
            LoweredStage L;
            int ab = generic ? -1 : attn_absorber(d, s);
            if (ab >= 0) {
                L.kernel_kind = "absorbed-into:" + std::to_string(ab);
                out.stages.push_back(std::move(L));
                s++;
                continue;
            }
            if (generic || !lower_pointwise_skeleton(d, s, out.scratch_bytes, L))
                L = lower_pointwise(d, s);
            out.stages.push_back(std::move(L));
        }
        s++;
    }
    return out;
}

}  // namespace sanic
