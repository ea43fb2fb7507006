/*
 * sanic_hip.h — the C ABI of the MI355X (gfx950) backend for sanic's carrier-fold hot path.
 *
 * The reference backend boundary is the sealed Rust trait
 *   `Backend { specs, prepare, execute }`            (/root/reference/src/compile.rs:87-108)
 * plus capture/replay of a compiled step
 *   `Program::capture` / `MetalReplay::step_timed`   (/root/reference/src/compile.rs:820-1035)
 * and the stateful decode machine
 *   `Graph::compile_for` / `StepProgram::instantiate` / `Machine::step`
 *                                                    (/root/reference/src/graph.rs:231-345).
 * Buffers mirror `MetalDevice::alloc_*` / `from_bytes` / `write_f64` / `read_*`
 *                                                    (/root/reference/src/metal.rs:197-412).
 *
 * What crosses this boundary is plain data: a program descriptor that serialises the schedule
 * the reference hands its backend — `Stage`s (/root/reference/src/partition.rs:44-127), each
 * fused stage's derived `Carrier` (/root/reference/src/derive.rs:261-392) with its `Expr`
 * trees (derive.rs:95-118) and `SlotKind`s (derive.rs:518-530), the carrier's leaf node trees
 * in the positional IR (/root/reference/src/ir.rs:72-123), the `FoldSched`
 * (/root/reference/src/plan.rs:434-476) and the resolved storage dtypes. No torch or HIP type
 * appears in any signature.
 *
 * Every entry point returns an int status: 0 = ok, otherwise an error whose text is readable
 * through sanic_hip_last_error() (thread-local). Status codes map onto the reference's
 * `CompileError::Backend` (prepare) and `RunError::{Shape,Dtype,Feedback,Backend,...}`
 * (execute/capture/step) (/root/reference/src/compile.rs:42-58).
 */
#ifndef SANIC_HIP_H
#define SANIC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------
 * Status codes (compile.rs:42-58 `RunError`, compile.rs `CompileError::Backend`).
 * ------------------------------------------------------------------------------------------- */
enum {
    SANIC_OK = 0,
    SANIC_ERR_COMPILE = 1,      /* CompileError::Backend: infeasible stage / unstorable width  */
    SANIC_ERR_MISSING_INPUT = 2,/* RunError::MissingInput                                      */
    SANIC_ERR_SHAPE = 3,        /* RunError::Shape                                             */
    SANIC_ERR_DTYPE = 4,        /* RunError::Dtype                                             */
    SANIC_ERR_FEEDBACK = 5,     /* RunError::Feedback                                          */
    SANIC_ERR_BACKEND = 6,      /* RunError::Backend: a HIP runtime failure                    */
    SANIC_ERR_ARG = 7,          /* invalid argument at the C boundary                          */
    SANIC_ERR_IN_PLACE = 8      /* an in-place program refuses execute; use capture            */
};

/* ---------------------------------------------------------------------------------------------
 * Storage dtypes (/root/reference/src/scalar.rs:180-326 `Dtype`). U4 is the unsigned nibble
 * form used by asymmetric group quantisation (value = u); I4 is the reference's signed nibble
 * (value = u - 8, emit_metal.rs:179-181). Both pack two values per byte, low nibble = even index.
 * Q8 is the reference's affine-quantized byte `Dtype::Q8 { scale }` (scalar.rs:190-198): one
 * signed byte q per element, value q·scale, the scale carried by the buffer
 * (`sanic_buffer_desc.scale`); stores round v/scale to the nearest integer in f32 and clamp it
 * to ±127 (emit_metal.rs:182-185, 226-229), so ±∞ land on ±127·scale.
 * ------------------------------------------------------------------------------------------- */
enum {
    SANIC_F64 = 0, SANIC_F32 = 1, SANIC_F16 = 2, SANIC_BF16 = 3, SANIC_U32 = 4,
    SANIC_I8 = 5, SANIC_I4 = 6, SANIC_U4 = 7, SANIC_Q8 = 8
};

/* MapOp (/root/reference/src/scalar.rs:45-69). ROUND_BF16/ROUND_F32/ROUND_F16 are
 * `RoundTo(dtype)`; ROUND_Q8 is `RoundTo(Q8 { scale })` with the scale in the MAP node's `value`
 * (emit_metal.rs:95-104: the value a store + load at that width would give). ROUND_Q8 and
 * ROUND_F16 are node ops only, not carrier Expr ops. */
enum {
    SANIC_OP_ADD = 0, SANIC_OP_SUB, SANIC_OP_MUL, SANIC_OP_DIV, SANIC_OP_MAX, SANIC_OP_MIN,
    SANIC_OP_LT, SANIC_OP_NEG, SANIC_OP_RECIP, SANIC_OP_EXP, SANIC_OP_LOG, SANIC_OP_SQRT,
    SANIC_OP_TANH, SANIC_OP_SIN, SANIC_OP_COS, SANIC_OP_WHERE, SANIC_OP_ROUND_BF16,
    SANIC_OP_ROUND_F32, SANIC_OP_ROUND_Q8, SANIC_OP_ROUND_F16
};

/* Monoid (/root/reference/src/scalar.rs:18-41). */
enum { SANIC_MON_ADD = 0, SANIC_MON_MUL, SANIC_MON_MAX, SANIC_MON_MIN, SANIC_MON_LSE };

/* ---------------------------------------------------------------------------------------------
 * Positional IR node (/root/reference/src/ir.rs:72-123), one record per node, children by index
 * into the same node table (children precede parents).
 *   INPUT       buffer  = program buffer index; dtype = storage dtype; shape = its shape
 *   CONST       value
 *   IOTA        shape = [n]; value at i is i
 *   COORDINATE  shape = any; value at c is c[dim]            (ir.rs `coordinate`)
 *   MAP         op, in[0..n_in)   inputs right-aligned against the output rank, extent-1
 *               dims broadcast (interp.rs `Map` arm)
 *   REDUCE      in[0] = src, dim, op = monoid; output = src shape without `dim`
 *   GATHER      in[0] = src, in[1] = index, dim; out = src[:dim] ++ index.shape ++ src[dim+1:];
 *               the index value is rounded to the nearest integer (interp.rs `Gather` arm)
 *   VIEW        in[0] = src; group[j] = how many consecutive source dims merge into output
 *               dim j (flatten; a 1 is a rename) (interp.rs `eval_view`)
 *   REINDEX     in[0] = src; affine map per source dim stored in the reindex table starting at
 *               map_offset: for each source dim: n_terms, offset, then n_terms (coef, out_dim)
 *               pairs; out of range reads 0 when padded (interp.rs `Reindex` arm)
 *   FOLD        placeholder for the enclosing fused stage's projected fold value at the
 *               stage's grid coordinate (used only inside an epilogue tree; shape = grid)
 *   SCAN        in[0] = src, dim, op = monoid; shape = src shape; the inclusive prefix fold
 *               along `dim` (interp.rs `eval_scan`, ir.rs `scan`)
 * ------------------------------------------------------------------------------------------- */
enum {
    SANIC_NODE_INPUT = 0, SANIC_NODE_CONST, SANIC_NODE_IOTA, SANIC_NODE_COORDINATE,
    SANIC_NODE_MAP, SANIC_NODE_REDUCE, SANIC_NODE_GATHER, SANIC_NODE_VIEW, SANIC_NODE_REINDEX,
    SANIC_NODE_FOLD, SANIC_NODE_SCAN
};

#define SANIC_MAX_RANK 8

typedef struct sanic_node {
    int32_t kind;
    int32_t op;          /* MapOp for MAP, Monoid for REDUCE                         */
    int32_t dtype;       /* storage dtype for INPUT                                   */
    int32_t buffer;      /* program buffer index for INPUT                            */
    int32_t n_in;
    int32_t in[3];
    int32_t rank;
    int32_t dim;         /* REDUCE / GATHER / COORDINATE                              */
    int64_t shape[SANIC_MAX_RANK];
    int32_t group[SANIC_MAX_RANK]; /* VIEW                                            */
    int32_t padded;      /* REINDEX                                                   */
    int32_t map_offset;  /* REINDEX: offset into the reindex table                   */
    double value;        /* CONST; MAP ROUND_Q8: the scale                            */
} sanic_node;

/* ---------------------------------------------------------------------------------------------
 * Carrier Expr (/root/reference/src/derive.rs:95-118), flat, children by index.
 *   ITEM(i): field i of the lifted element (into), A(i)/B(i): the two accumulators (combine),
 *   F(i): the final accumulator (project). Binary/unary ops reuse the MapOp codes.
 * ------------------------------------------------------------------------------------------- */
enum {
    SANIC_EX_CONST = 100, SANIC_EX_ITEM, SANIC_EX_A, SANIC_EX_B, SANIC_EX_F
    /* values 0..17 are the MapOp codes above (ADD..ROUND_F32); LT is `a < b` as 1/0 and
       WHERE is `c != 0 ? a : b`, exactly as derive.rs:95-118 */
};

typedef struct sanic_expr {
    int32_t op;
    int32_t index;       /* ITEM/A/B/F slot or field                                  */
    int32_t a, b, c;     /* children (expr table indices), -1 when absent             */
    double value;        /* CONST                                                     */
} sanic_expr;

/* SlotKind (/root/reference/src/derive.rs:518-530). */
enum { SANIC_SLOT_PLAIN = 0, SANIC_SLOT_EXP_SHIFTED = 1, SANIC_SLOT_AT_EXTREMUM = 2 };

#define SANIC_MAX_SLOTS 8
#define SANIC_MAX_LEAVES 8

typedef struct sanic_slot {
    int32_t kind;
    int32_t monoid;      /* PLAIN: the monoid; AT_EXTREMUM: the key monoid            */
    int32_t ref_slot;    /* EXP_SHIFTED: max_slot; AT_EXTREMUM: key_slot              */
    int32_t ties;        /* AT_EXTREMUM: the ties monoid                              */
} sanic_slot;

typedef struct sanic_carrier {
    int32_t slots;
    sanic_slot kind[SANIC_MAX_SLOTS];
    double identity[SANIC_MAX_SLOTS];
    int32_t into[SANIC_MAX_SLOTS];     /* expr roots                                    */
    int32_t combine[SANIC_MAX_SLOTS];  /* expr roots                                    */
    int32_t project;                   /* expr root (scalar-projecting carriers only)  */
} sanic_carrier;

/* FoldSched (/root/reference/src/plan.rs:434-476), re-derived for wave64:
 *   lane_stream: lanes of a wavefront fold strided/chunked slices of the stream
 *   waves:       wavefronts per workgroup that split the stream further (`sgs`)
 *   chunk:       contiguous run each lane folds before striding
 *   split:       workgroups that fold disjoint slices of the stream; their partial carriers are
 *                merged by the carrier's own combine in a second pass (the split-K /
 *                Flash-Decoding combine; oracle = interp.rs:555-643 run_carrier_split)      */
/* variant:     tiling variant of the hand-written kernel that lowers the stage (0 = the
 *              analytic choice): the measured tuner's handle, as the reference's SANIC_TUNE swaps
 *              FoldSched candidates (compile.rs:1348-1630). Generic folds ignore it.       */
typedef struct sanic_sched {
    int32_t lane_stream;
    int32_t waves;
    int32_t chunk;
    int32_t split;
    int32_t variant;
} sanic_sched;

/* Stage kinds (/root/reference/src/partition.rs:44-98). */
enum { SANIC_STAGE_FUSED = 0, SANIC_STAGE_POINTWISE = 1 };

/* Leaf axis binding: leaf dim -> a grid dim (>= 0), the streamed axis, or broadcast. */
#define SANIC_BIND_STREAM (-1)
#define SANIC_BIND_BCAST  (-2)

typedef struct sanic_stage {
    int32_t kind;
    int32_t out_buffer;          /* program buffer written by this stage                  */
    int32_t out_dtype;           /* its storage dtype (the narrowing store)               */
    int32_t rank;                /* grid (= output) rank                                  */
    int64_t grid[SANIC_MAX_RANK];
    /* FUSED */
    int64_t stream;              /* extent of the folded axis                             */
    int32_t n_leaves;
    int32_t leaf[SANIC_MAX_LEAVES];                  /* node index                        */
    int32_t bind[SANIC_MAX_LEAVES][SANIC_MAX_RANK];  /* per leaf dim                      */
    sanic_carrier carrier;
    int32_t epilogue;            /* node tree over FOLD (+ other inputs), -1 = none       */
    sanic_sched sched;
    /* POINTWISE */
    int32_t value;               /* node tree evaluated per output point                  */
    int32_t where;               /* in-place: store only where nonzero; -1 = store all    */
} sanic_stage;

/* Program buffer roles. INPUT and STATE are bound by the caller; OUTPUT and SCRATCH are owned
 * by the executable (execute) or the replay (capture). */
enum { SANIC_BUF_INPUT = 0, SANIC_BUF_STATE = 1, SANIC_BUF_OUTPUT = 2, SANIC_BUF_SCRATCH = 3 };

typedef struct sanic_buffer_desc {
    int32_t role;
    int32_t dtype;
    int32_t rank;
    float scale;                 /* Q8: the grid step (value = q·scale); ignored otherwise */
    int64_t shape[SANIC_MAX_RANK];
} sanic_buffer_desc;

typedef struct sanic_program_desc {
    int32_t n_nodes;          const sanic_node* nodes;
    int32_t n_exprs;          const sanic_expr* exprs;
    int32_t n_reindex;        const int64_t* reindex;
    int32_t n_buffers;        const sanic_buffer_desc* buffers;
    int32_t n_stages;         const sanic_stage* stages;
} sanic_program_desc;

/* DeviceSpecs (/root/reference/src/cost.rs:33-60), filled with MI355X figures. The last five
 * fields are the cost model's own (cost.rs:40-50, used by kernel_time / sustainable_bandwidth,
 * cost.rs:150-210): the Rust side's `Backend::specs` copies them into `DeviceSpecs` together
 * with hbm_bytes_per_s (hbm_bandwidth) and bf16_mfma_flops (peak_flops). */
typedef struct sanic_device_specs {
    char name[64];
    int32_t compute_units;
    int32_t wave_size;
    int32_t lds_bytes_per_cu;
    double hbm_bytes_per_s;
    double bf16_mfma_flops;
    double f32_flops;
    double clock_hz;
    int64_t hbm_bytes;
    double sram_bytes;          /* LDS one workgroup may allocate (160 KiB on gfx950)          */
    double regfile_bytes;       /* vector registers of one CU (4 SIMDs × 128 KiB)             */
    double launch_overhead_s;   /* measured floor of a dependent kernel launch in a hipGraph  */
    double min_blocks;          /* workgroups that fill the chip: 2 per CU                    */
    double mem_latency_s;       /* loaded HBM latency (Little's law: ≈16 MB in flight at 8 TB/s) */
} sanic_device_specs;

typedef struct sanic_hip_device sanic_hip_device;
typedef struct sanic_hip_buffer sanic_hip_buffer;
typedef struct sanic_hip_exe sanic_hip_exe;
typedef struct sanic_hip_replay sanic_hip_replay;

/* thread-local text of the last error */
const char* sanic_hip_last_error(void);

/* MetalDevice::open (metal.rs:148-160): returns SANIC_ERR_BACKEND when no HIP device exists. */
int sanic_hip_open(int ordinal, sanic_hip_device** out);
void sanic_hip_close(sanic_hip_device* dev);
/* Backend::specs (compile.rs:87-108) */
int sanic_hip_specs(sanic_hip_device* dev, sanic_device_specs* out);

/* Buffers: MetalDevice::alloc_elems / from_bytes / write_f64 / read_* (metal.rs:197-412). */
int sanic_hip_alloc(sanic_hip_device* dev, size_t bytes, sanic_hip_buffer** out);
void sanic_hip_free(sanic_hip_buffer* buf);
int sanic_hip_upload(sanic_hip_buffer* buf, size_t offset, const void* host, size_t bytes);
int sanic_hip_download(sanic_hip_buffer* buf, size_t offset, void* host, size_t bytes);
/* MetalBuf::slice (metal.rs:80-90): a view at a 4-byte-aligned offset sharing the storage. */
int sanic_hip_slice(sanic_hip_buffer* buf, size_t offset, size_t bytes, sanic_hip_buffer** out);
size_t sanic_hip_buffer_bytes(const sanic_hip_buffer* buf);
/* raw device address (for callers that interoperate with another HIP runtime user) */
void* sanic_hip_buffer_device_ptr(const sanic_hip_buffer* buf);
/* wrap caller-owned device memory without taking ownership (MetalDevice::from_bytes_nocopy) */
int sanic_hip_wrap(sanic_hip_device* dev, void* device_ptr, size_t bytes, sanic_hip_buffer** out);

/* Backend::prepare (compile.rs:87-108, Metal impl compile.rs:694-731): emit one kernel per
 * stage (a hand-written CDNA4 skeleton chosen from the carrier's structure, else the generic
 * carrier fold), compile through hipRTC, load the code objects. */
int sanic_hip_prepare(sanic_hip_device* dev, const sanic_program_desc* desc, sanic_hip_exe** out);
void sanic_hip_exe_free(sanic_hip_exe* exe);
/* Which kernel each stage lowered onto ("skeleton:<name>" or "fold:scalar" ...). */
int sanic_hip_exe_stage_kernel(const sanic_hip_exe* exe, int stage, char* out, size_t cap);
/* The generated HIP source of one stage (SANIC_MSL's counterpart, compile.rs:723-728). */
int sanic_hip_exe_stage_source(const sanic_hip_exe* exe, int stage, char* out, size_t cap);

/* Backend::execute (compile.rs:733-787): `bindings[i]` is the buffer for program buffer i when
 * its role is INPUT or STATE (NULL otherwise). Allocates OUTPUT and SCRATCH buffers, runs every
 * stage on the device's stream and waits. `outputs[i]` receives a new owned buffer for program
 * buffer i when its role is OUTPUT (NULL otherwise); free each with sanic_hip_free. */
int sanic_hip_execute(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings,
                      sanic_hip_buffer** outputs);

/* No counterpart in the reference. sanic_hip_execute without device allocation, for callers
 * that cannot call hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid it):
 * `bindings[i]` must hold a caller-owned buffer for every INPUT, STATE and OUTPUT program buffer
 * (NULL for SCRATCH-role ones). The executable's intermediates and its split-partial / counter
 * arena live in the library's static device scratch — 32 MiB per GPU, held until the process
 * ends; a program that needs more is refused with SANIC_ERR_ARG. The stages are enqueued on the
 * device's stream and the call returns without waiting (a download on the same buffers waits).
 * Every call on one GPU shares that scratch; the arena's counters are cleared at the start of
 * each call, its other contents are whatever the last call left. Eager calls are ordered per GPU:
 * each waits for the previous eager call's work on that GPU, whichever device handle (stream)
 * made it. A call made while the device's stream is being captured into a HIP graph is not
 * ordered that way: replays of such a graph that overlap other calls on the GPU race on the
 * scratch. In-place programs are refused as by sanic_hip_execute. */
int sanic_hip_execute_static(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings);

/* No counterpart in the reference. The number of device allocations (hipMalloc) this library
 * has made in this process; a test hook showing that sanic_hip_execute_static allocates none. */
uint64_t sanic_hip_device_allocations(void);

/* Program::capture (compile.rs:820-961): freeze the bindings into a hipGraph of every stage.
 * feedback = n_pairs (output buffer index, input buffer index) pairs: after each step the
 * output's value is converted into the input's dtype and written to the input buffer, inside
 * the same graph (the reference's feedback ping-pong, compile.rs:869-961). */
int sanic_hip_capture(sanic_hip_exe* exe, sanic_hip_buffer* const* bindings, int n_bindings,
                      const int32_t* feedback, int n_pairs, sanic_hip_replay** out);
/* the replay-owned buffer of program buffer i (OUTPUT or SCRATCH role) */
int sanic_hip_replay_buffer(sanic_hip_replay* rp, int index, sanic_hip_buffer** out);
/* MetalReplay::step_timed (compile.rs:985-1022): launch one replay, wait, report GPU seconds
 * measured with HIP events around the graph launch. */
int sanic_hip_step(sanic_hip_replay* rp, double* gpu_seconds);
/* Launch `n` replays back to back without waiting in between; report total GPU seconds. */
int sanic_hip_step_many(sanic_hip_replay* rp, int n, double* gpu_seconds);
void sanic_hip_replay_free(sanic_hip_replay* rp);

/* Per-kernel timing of one replay launched eagerly (SANIC_DEBUG=4's counterpart,
 * metal.rs:437-541): seconds[i] = GPU time of stage i, from HIP events on the stream. */
int sanic_hip_profile_stages(sanic_hip_replay* rp, double* seconds, int n);

/* Synchronise the device's stream. */
int sanic_hip_sync(sanic_hip_device* dev);

/* Device-free entry points (no GPU needed): lower a program and return one stage's kernel kind
 * and generated source; lower and compile every stage into the code-object cache; and the
 * sizeof of each record above (for binding layout checks). */
int sanic_hip_emit_source(const sanic_program_desc* desc, int stage, char* kind, size_t kind_cap,
                          char* source, size_t source_cap);
int sanic_hip_precompile(const sanic_program_desc* desc);
/* Number of tiling variants (sanic_sched.variant values) the kernel lowering `stage` offers
 * (1 when it has none; 0 for a stage folded into another stage's launch): the measured
 * tuner's candidate space (the reference prices FoldSched candidates, plan.rs:604-850, and
 * SANIC_TUNE times them in the full step, compile.rs:1348-1630). With stage = -1, `count`
 * holds n_stages entries and receives every stage's count from one lowering. */
int sanic_hip_stage_variants(const sanic_program_desc* desc, int stage, int* count);
size_t sanic_hip_abi_sizeof(const char* record_name);

#ifdef __cplusplus
}
#endif
#endif
