// Internal interface of the HIP emitter: node/Expr rendering shared by the generic carrier fold
// (emit_hip.cpp) and the hand-written skeletons (skeletons.cpp).
#pragma once
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "common.h"

namespace sanic {

struct Code {
    std::ostringstream s;
    int indent = 0;
    void line(const std::string& l);
    std::string str() const;
};

// Renders node trees (codegen.rs:283-443) and carrier Exprs (codegen.rs:457-487) into HIP.
struct Renderer {
    const sanic_program_desc* d;
    std::vector<int> bufs;                       // program buffers referenced, in Args order
    std::map<int, std::string> buf_param;
    std::vector<std::map<std::string, std::string>> memo;  // scoped common-subexpression cache
    int tmp = 0;
    std::string fold_var = "fold_v";
    std::map<int, std::string> subst;
    std::set<int> coherent;                      // buffers read with device-coherent loads
    Code scalars;                                // rank-0 input loads hoisted to kernel entry
    std::map<int, std::string> scalar_vars;
    std::string entry() const { return scalars.str(); }            // node id -> precomputed value expression
    explicit Renderer(const sanic_program_desc* dd) : d(dd) { memo.emplace_back(); }

    std::string param(int buffer);
    std::string fresh(const char* p);
    std::string args_struct(const std::vector<std::string>& extra) const;
    std::vector<Arg> arg_list() const;
    std::string load(int node, const std::vector<std::string>& c);
    std::string value(Code& code, int node, const std::vector<std::string>& c);
    std::string expr(Code& code, int e, const std::string& item, const std::string& a,
                     const std::string& b, const std::string& f);
};

struct WindowBound {
    enum Kind { HI_FLOOR_PLUS1, HI_CEIL, LO_CEIL } kind;
    int node;                 // the stream-independent edge expression
    std::vector<int> bind;    // its dims' bindings
    int where_node = -1;      // the additive mask term this bound was read from
};

extern const char* kPrelude;
std::string flit(double v);
const char* ctype_of(int dt);
std::string map_expr(int op, const std::string& a, const std::string& b, const std::string& c);
std::string monoid_combine(int m, const std::string& a, const std::string& b);
double monoid_identity(int m);
std::string store_stmt(const std::string& ptr, const std::string& idx, int dt, const std::string& v, bool coherent = false,
                       double scale = 0.0);
void decode_grid(Code& code, const sanic_stage& st, const std::string& gid);
std::vector<std::string> leaf_coords(const sanic_stage& st, const sanic_program_desc* d, int l,
                                     const std::string& s);
std::vector<WindowBound> honest_window(const sanic_program_desc* d, const sanic_stage& st);
void emit_window(Renderer& R, Code& code, const sanic_stage& st, const std::vector<WindowBound>& w,
                 const std::string& lo, const std::string& hi);
int64_t dtype_bytes(int dt, int64_t n);
// Last-arriver handshake: the workgroups sharing counter `cnt` each add 1 once their partials
// are stored; `flag` (a __shared__ int it declares) is true in the one that arrives last.
// With xcd_local every workgroup sharing `cnt` runs on one XCD and exchanges data through
// sanic_stx / sanic_ldx (that XCD's L2); otherwise through sanic_st / sanic_ld (device-coherent).
void emit_arrival(Code& k, const std::string& flag, const std::string& tid, const std::string& cnt,
                  const std::string& expected, bool xcd_local = false);
// Workgroups are dispatched round-robin over the 8 XCDs by linear block index; the runtime
// checks that once per process (set_xcd_local) and kernels whose merging workgroups share
// blockIdx mod 8 then exchange partials through the L2 of their XCD.
void set_xcd_local(bool on);
bool xcd_local_enabled();
void validate(const sanic_program_desc* d);

// The MI355X figures the cost model reads (the same numbers sanic_hip_specs reports).
struct MachineSpecs {
    double hbm, f32_flops, sram_bytes, regfile_bytes, launch, min_blocks, latency;
};
MachineSpecs mi355x_specs();
// A generic fold's schedule: waves = 0 is the scalar form; split workgroups per point; chunk.
struct FoldChoice {
    int waves, split, chunk;
    double time;
};
bool sched_is_auto(const sanic_sched& s);
FoldChoice choose_fold_sched(const sanic_program_desc* d, const sanic_stage& st);
LoweredStage lower_generic_fold(const sanic_program_desc* d, int si, int64_t& scratch, const std::vector<int>& tails);
bool tail_candidate(const sanic_program_desc* d, int si);
void emit_pointwise_loop(Renderer& R, Code& body, const sanic_program_desc* d, int si, const std::string& tid, int nth);
LoweredStage lower_pointwise(const sanic_program_desc* d, int si);
// Offer a stage to the hand-written skeletons; false when none accepts its structure.
bool lower_skeleton(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out);
bool lower_pointwise_skeleton(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out);

}  // namespace sanic
