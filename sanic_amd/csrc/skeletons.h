// Structural analysis shared by the skeletons: symbolic affine coordinates and accesses.
#pragma once
#include <set>
#include <string>
#include <vector>

#include "emit.h"

namespace sanic {

// coef · ((var / div) % mod); mod 0 = none
struct SymTerm {
    int64_t coef;
    int var;
    int64_t div;
    int64_t mod;
};

// c0 + Σ terms: an integer coordinate as a function of kernel variables
struct Sym {
    int64_t c0 = 0;
    std::vector<SymTerm> terms;
    static Sym var(int v);
    std::string render(const std::vector<std::string>& vars) const;
};

// An Input read through Reindex/View chains, as element address = Sym.
struct Access {
    int buffer = -1, dtype = -1, node = -1;
    Sym addr;
};

// The element address of `node` at symbolic coordinates `c` (ext = extent of each variable);
// false when the node is not an affine view of one input (or a padded read may go out of
// bounds).
bool sym_access(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                const std::vector<int64_t>& ext, Access& out);

bool sym_child_coords(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                      const std::vector<int64_t>& ext, std::vector<Sym>& sc);

void collect_inputs(const sanic_program_desc* d, int node, std::set<int>& bufs);
// match Lt(coordinate, X + 1) (inside a product) with X scalar: the row dim and X's node
bool match_row_cond(const sanic_program_desc* d, int node, int rank, int& dim, int& pos);
// The decode-attention stage that performs in-place row write `si` itself (the K/V cache
// update of this step feeding that attention), or -1.
int attn_absorber(const sanic_program_desc* d, int si);

// One run of 8 of an elementwise leaf (see skeletons.cpp): loads in `lc` through pointers
// rb<i><sfx> for `bufs`, arithmetic in `dc`.
std::vector<std::string> render_run(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                                    const std::vector<int64_t>& ext, const std::vector<std::string>& vars, int kv,
                                    Code& lc, Code& dc, const std::string& sfx, std::vector<int>& bufs,
                                    std::vector<int>& dtypes, bool& ok);

bool lower_gemm(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out);
bool lower_flash_prefill(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out);
bool lower_attn_decode(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out);

// Lower stage `si` (and the following stages it batches with) onto the gemv skeleton.
bool lower_gemv_group(const sanic_program_desc* d, int si, int64_t& scratch, std::vector<LoweredStage>& out);

}  // namespace sanic
