// FlashAttention prefill skeleton: the online-softmax (m, ℓ, o) carrier over the key axis on
// bf16 MFMA (v_mfma_f32_16x16x32_bf16), for stages whose query grid has a head axis and a
// query-row axis (the causal / sliding-window prefill of the reference's
// scaled_dot_product_attention, /root/reference/src/nn.rs:27-105, folded as
// /root/reference/tests/laws.rs:108-126).
//
// Structure required (read from the carrier and the leaves, never from names): the carrier of
// skel_attention.cpp (a Plain(Max) score slot, ExpShifted slots with constant or value `into`);
// the score leaf = one in-body contraction Σ_d Q·K (both affine bf16 views with d contiguous,
// the head entering K as ⌊h/rep⌋) with scalar factors and additive mask terms around it; the
// value leaf an affine bf16 view.
//
// Kernel shape (one workgroup = one head × 128 query rows, 4 waves × 32 rows):
//   S^T = K·Q^T per 64-key tile (so a lane owns one query column: the running max, the sum and
//   the O rescale are lane-local, with one 4-lane shuffle per tile for the max);
//   O^T += V^T·P^T with P packed to bf16 in registers (the MFMA k-order is chosen to match the
//   S^T accumulator layout, so P never goes through LDS);
//   K and V tiles go from global memory straight into a ring of three LDS buffers, two tiles
//   ahead; Q stays in registers; exp2 with log2(e) folded; the −∞ guard of the
//   carrier's combine on the rescale; tiles outside every row's honest window are skipped and
//   tiles entirely inside it skip the mask arithmetic;
//   blockIdx → (KV head, query head, query block) places all query heads of one KV head on one
//   XCD (blockIdx mod 8) so their K/V stay in that XCD's L2, heaviest causal blocks first.
#include <algorithm>
#include <cmath>

#include <functional>
#include <regex>

#include "emit.h"
#include "skeletons.h"

namespace sanic {

namespace {

struct FlashPlan {
    int sleaf = -1, vleaf = -1, max_slot = -1;
    std::vector<int> vec_slots, scalar_slots;
    std::vector<double> scalar_into;
    int hdim = -1, qdim = -1, edim = -1;
    int64_t NH = 1, NQ = 1, E = 1, T = 1, HD = 1;
    int rep = 1;
    int dot_reduce = -1;
    Access qacc, kacc, vacc;
    // a query side that is an elementwise expression (RoPE'd Q, say) rather than one affine
    // view: rendered per element once per workgroup, at coordinates qcoords over the vars
    // {0: head, 1: key, 2: d, 3: query row}
    bool qexpr = false;
    int qnode = -1;
    std::vector<Sym> qcoords;
};

bool has_reduce_below(const sanic_program_desc* d, int node) {
    std::vector<int> st{node};
    while (!st.empty()) {
        int i = st.back();
        st.pop_back();
        if (d->nodes[i].kind == SANIC_NODE_REDUCE || d->nodes[i].kind == SANIC_NODE_SCAN) return true;
        for (int q = 0; q < d->nodes[i].n_in; q++) st.push_back(d->nodes[i].in[q]);
    }
    return false;
}

bool sym_is_var(const Sym& s, int& var) {
    if (s.c0 != 0 || s.terms.size() != 1) return false;
    const SymTerm& t = s.terms[0];
    if (t.coef != 1 || t.div != 1 || t.mod != 0) return false;
    var = t.var;
    return true;
}

// address = c0 + Σ terms; returns per-var coefficient (div 1, no mod) and the h term's div
bool split_addr(const Sym& a, int nvars, std::vector<int64_t>& coef, int& hdiv, int64_t& hcoef) {
    coef.assign(nvars, 0);
    hdiv = 0;
    hcoef = 0;
    for (auto& t : a.terms) {
        if (t.mod) return false;
        if (t.var == 0 && t.div != 1) {
            if (hdiv) return false;
            hdiv = (int)t.div;
            hcoef = t.coef;
            continue;
        }
        if (t.div != 1) return false;
        coef[t.var] += t.coef;
    }
    return true;
}

bool find_flash_dot(const sanic_program_desc* d, int node, const std::vector<Sym>& c, const std::vector<int64_t>& ext,
                    FlashPlan& P) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_MAP) {
        int found = 0;
        for (int k = 0; k < n.n_in; k++) {
            const sanic_node& m = d->nodes[n.in[k]];
            bool has_reduce = false;
            std::vector<int> st{n.in[k]};
            while (!st.empty()) {
                int i = st.back(); st.pop_back();
                if (d->nodes[i].kind == SANIC_NODE_REDUCE || d->nodes[i].kind == SANIC_NODE_SCAN) has_reduce = true;
                for (int q = 0; q < d->nodes[i].n_in; q++) st.push_back(d->nodes[i].in[q]);
            }
            if (!has_reduce) continue;
            int lead = n.rank - m.rank;
            std::vector<Sym> cc(m.rank);
            for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? Sym() : c[lead + j];
            if (!find_flash_dot(d, n.in[k], cc, ext, P)) return false;
            found++;
        }
        return found == 1;
    }
    if (n.kind != SANIC_NODE_REDUCE || n.op != SANIC_MON_ADD) return false;
    const sanic_node& mp = d->nodes[n.in[0]];
    if (mp.kind != SANIC_NODE_MAP || mp.op != SANIC_OP_MUL) return false;
    // vars: 0 = head, 1 = key (stream), 2 = contraction d, 3 = query row
    std::vector<Sym> mc;
    for (int j = 0, o = 0; j < mp.rank; j++) mc.push_back(j == n.dim ? Sym::var(2) : c[o++]);
    std::vector<int64_t> ext4 = {ext[0], ext[1], mp.shape[n.dim], ext[3]};
    int kside = -1;
    std::vector<std::vector<Sym>> cc(2);
    for (int k = 0; k < 2; k++) {
        const sanic_node& ch = d->nodes[mp.in[k]];
        int lead = mp.rank - ch.rank;
        cc[k].resize(ch.rank);
        bool moves = false;
        for (int j = 0; j < ch.rank; j++) {
            cc[k][j] = ch.shape[j] == 1 ? Sym() : mc[lead + j];
            for (auto& t : cc[k][j].terms) moves |= t.var == 1;
        }
        if (moves) {
            if (kside >= 0) return false;
            kside = k;
        }
    }
    if (kside < 0) return false;
    if (!sym_access(d, mp.in[kside], cc[kside], ext4, P.kacc)) return false;
    if (!sym_access(d, mp.in[1 - kside], cc[1 - kside], ext4, P.qacc)) {
        if (has_reduce_below(d, mp.in[1 - kside])) return false;
        P.qexpr = true;
        P.qnode = mp.in[1 - kside];
        P.qcoords = cc[1 - kside];
    }
    P.dot_reduce = node;
    P.HD = mp.shape[n.dim];
    return true;
}

bool flash_plan(const sanic_program_desc* d, int si, FlashPlan& P) {
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_FUSED || st.n_leaves != 2) return false;
    const sanic_carrier& c = st.carrier;
    P = FlashPlan();
    for (int k = 0; k < c.slots; k++)
        if (c.kind[k].kind == SANIC_SLOT_PLAIN && c.kind[k].monoid == SANIC_MON_MAX) {
            if (P.max_slot >= 0) return false;
            P.max_slot = k;
        }
    if (P.max_slot < 0) return false;
    const sanic_expr& mi = d->exprs[c.into[P.max_slot]];
    if (mi.op != SANIC_EX_ITEM) return false;
    P.sleaf = mi.index;
    for (int k = 0; k < c.slots; k++) {
        if (k == P.max_slot) continue;
        if (c.kind[k].kind != SANIC_SLOT_EXP_SHIFTED || c.kind[k].ref_slot != P.max_slot) return false;
        const sanic_expr& e = d->exprs[c.into[k]];
        if (e.op == SANIC_EX_ITEM && e.index != P.sleaf) {
            if (P.vleaf >= 0 && P.vleaf != e.index) return false;
            P.vleaf = e.index;
            P.vec_slots.push_back(k);
        } else if (e.op == SANIC_EX_CONST) {
            P.scalar_slots.push_back(k);
            P.scalar_into.push_back(e.value);
        } else {
            return false;
        }
    }
    if (P.vleaf < 0 || P.vec_slots.size() != 1) return false;
    const sanic_node& sl = d->nodes[st.leaf[P.sleaf]];
    const sanic_node& vl = d->nodes[st.leaf[P.vleaf]];
    std::vector<bool> in_s(st.rank, false), in_v(st.rank, false);
    for (int j = 0; j < sl.rank; j++) if (st.bind[P.sleaf][j] >= 0) in_s[st.bind[P.sleaf][j]] = true;
    for (int j = 0; j < vl.rank; j++) if (st.bind[P.vleaf][j] >= 0) in_v[st.bind[P.vleaf][j]] = true;
    std::vector<int> qdims;
    for (int j = 0; j < st.rank; j++) {
        if (st.grid[j] == 1) continue;
        if (in_v[j] && !in_s[j]) {
            if (P.edim >= 0) return false;
            P.edim = j;
        } else {
            qdims.push_back(j);
        }
    }
    if (P.edim < 0 || qdims.size() != 2) return false;
    // the head dim is the one the value leaf reads; the query row is read only by the score
    for (int j : qdims) {
        if (in_v[j]) P.hdim = j;
        else P.qdim = j;
    }
    if (P.hdim < 0 || P.qdim < 0) return false;
    P.NH = st.grid[P.hdim];
    P.NQ = st.grid[P.qdim];
    P.E = st.grid[P.edim];
    P.T = st.stream;
    std::vector<Sym> scs(sl.rank);
    for (int j = 0; j < sl.rank; j++) {
        int b = st.bind[P.sleaf][j];
        scs[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.hdim ? Sym::var(0) : b == P.qdim ? Sym::var(3) : Sym();
    }
    if (!find_flash_dot(d, st.leaf[P.sleaf], scs, {P.NH, P.T, 1, P.NQ}, P)) return false;
    std::vector<Sym> vcs(vl.rank);
    for (int j = 0; j < vl.rank; j++) {
        int b = st.bind[P.vleaf][j];
        vcs[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.hdim ? Sym::var(0) : b == P.edim ? Sym::var(2) : Sym();
    }
    if (!sym_access(d, st.leaf[P.vleaf], vcs, {P.NH, P.T, P.E}, P.vacc)) return false;
    if ((!P.qexpr && P.qacc.dtype != SANIC_BF16) || P.kacc.dtype != SANIC_BF16 || P.vacc.dtype != SANIC_BF16) return false;
    if (P.HD != 64 || P.E != 64 || P.NQ % 128 != 0 || P.T % 64 != 0) return false;
    // Q: (h, d, i) with d contiguous; K: (⌊h/rep⌋, t, d) with d contiguous; V: (⌊h/rep⌋, t, e)
    std::vector<int64_t> qc, kc, vc;
    int qh, kh, vh;
    int64_t qhc, khc, vhc;
    if (!P.qexpr && (!split_addr(P.qacc.addr, 4, qc, qh, qhc) || qh != 0 || qc[2] != 1 || qc[1] != 0)) return false;
    if (!split_addr(P.kacc.addr, 4, kc, kh, khc)) return false;
    if (!split_addr(P.vacc.addr, 3, vc, vh, vhc)) return false;
    if (kc[2] != 1 || kc[3] != 0 || (vc[2] != 1 && vc[1] != 1)) return false;
    int repk = kh ? kh : (kc[0] ? 1 : (int)P.NH);
    int repv = vh ? vh : (vc[0] ? 1 : (int)P.NH);
    if (repk != repv) return false;
    P.rep = repk;
    return true;
}

// On tiles every row sees entirely, the score must be `dot · c` (the additive mask terms are
// zero there): read c off the leaf so the tile can fold the scale into the exp2 argument.
bool full_score_scale(const sanic_program_desc* d, int node, int dot, const std::vector<WindowBound>& win, double& c) {
    const sanic_node& n = d->nodes[node];
    if (node == dot) { c = 1.0; return true; }
    if (n.kind != SANIC_NODE_MAP) return false;
    if (n.op == SANIC_OP_ADD) {
        for (int k = 0; k < 2; k++)
            for (auto& w : win)
                if (n.in[k] == w.where_node) return full_score_scale(d, n.in[1 - k], dot, win, c);
        return false;
    }
    if (n.op == SANIC_OP_MUL) {
        for (int k = 0; k < 2; k++) {
            const sanic_node& o = d->nodes[n.in[1 - k]];
            if (o.kind == SANIC_NODE_CONST && o.rank == 0) {
                double inner;
                if (!full_score_scale(d, n.in[k], dot, win, inner)) return false;
                c = inner * o.value;
                return true;
            }
        }
    }
    return false;
}

}  // namespace

bool lower_flash_prefill(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    FlashPlan P;
    if (!flash_plan(d, si, P)) return false;
    const sanic_stage& st = d->stages[si];
    const sanic_carrier& c = st.carrier;
    const int64_t NH = P.NH, NQ = P.NQ, T = P.T, E = P.E, HD = P.HD;
    const int64_t NQB = NQ / 128;
    std::vector<int64_t> qc, kc, vc;
    int qh, kh, vh;
    int64_t qhc, khc, vhc;
    if (!P.qexpr) split_addr(P.qacc.addr, 4, qc, qh, qhc);
    split_addr(P.kacc.addr, 4, kc, kh, khc);
    split_addr(P.vacc.addr, 3, vc, vh, vhc);
    const bool v_rows = vc[2] == 1;                  // V[t, e] rows (else V^T with t contiguous)
    auto hterm = [&](const std::vector<int64_t>& cf, int div, int64_t hcf) {
        // address contribution of head hh
        if (div) return "(hh / " + std::to_string(div) + ") * " + std::to_string(hcf);
        return "hh * " + std::to_string(cf[0]);
    };

    Renderer R(d);
    // score functions: the leaf with its contraction replaced by `dotv`; the "full" variant also
    // drops the additive mask terms (used only on tiles every row sees entirely)
    auto win = honest_window(d, st);
    const sanic_node& sl = d->nodes[st.leaf[P.sleaf]];
    std::vector<std::string> lc(sl.rank);
    for (int j = 0; j < sl.rank; j++) {
        int b = st.bind[P.sleaf][j];
        lc[j] = b == SANIC_BIND_STREAM ? "kj" : b == P.hdim ? "hh" : b == P.qdim ? "qi" : "0";
    }
    Renderer Rs(d);
    Code sp, sf;
    sp.indent = sf.indent = 1;
    Rs.subst[P.dot_reduce] = "dotv";
    std::string vpart = Rs.value(sp, st.leaf[P.sleaf], lc);
    std::string entry_part = Rs.entry();
    Renderer Rf(d);
    Rf.subst[P.dot_reduce] = "dotv";
    for (auto& w : win) Rf.subst[w.where_node] = "0.0f";
    std::string vfull = Rf.value(sf, st.leaf[P.sleaf], lc);
    std::string entry_full = Rf.entry();
    for (int b : Rs.bufs) R.param(b);
    for (int b : Rf.bufs) R.param(b);
    double scale_c = 0.0;
    const bool scale_known = full_score_scale(d, st.leaf[P.sleaf], P.dot_reduce, win, scale_c) && scale_c > 0.0;

    // window edges per query row (for tile skipping / full-tile detection)
    Code wc;
    wc.indent = 1;
    Renderer Rw(d);
    std::vector<std::string> gcw(st.rank, "0");
    gcw[P.hdim] = "hh";
    gcw[P.qdim] = "qrow";
    {
        Code tmp;
        tmp.indent = 1;
        // emit_window names grid coords g<j>
        for (int j = 0; j < st.rank; j++) tmp.line("const idx_t g" + std::to_string(j) + " = " + gcw[j] + ";");
        emit_window(Rw, tmp, st, win, "wlo", "whi");
        wc.s << tmp.str();
    }
    for (int b : Rw.bufs) R.param(b);

    // finish: project (+ epilogue) and the narrowing store of one output point
    Renderer Ro(d);
    Code fo;
    fo.indent = 1;
    {
        for (int sl2 = 0; sl2 < c.slots; sl2++) fo.line("const float fs" + std::to_string(sl2) + " = fs[" + std::to_string(sl2) + "];");
        std::string f = Ro.expr(fo, c.project, "", "", "", "fs");
        fo.line("const float fold_v = " + f + ";");
        std::vector<std::string> gc(st.rank, "0");
        gc[P.hdim] = "hh";
        gc[P.qdim] = "qi";
        gc[P.edim] = "ee";
        std::string v = "fold_v";
        if (st.epilogue >= 0) {
            Ro.fold_var = "fold_v";
            v = Ro.value(fo, st.epilogue, gc);
        }
        std::string lin;
        for (int j = 0; j < st.rank; j++)
            lin = j == 0 ? "(idx_t)(" + gc[0] + ")" : "(" + lin + " * " + std::to_string(st.grid[j]) + " + (idx_t)(" + gc[j] + "))";
        fo.line(store_stmt(Ro.param(st.out_buffer), lin, st.out_dtype, v, false, d->buffers[st.out_buffer].scale));
    }
    for (int b : Ro.bufs) R.param(b);
    if (P.qexpr) {
        // register the expression's buffers before the argument struct is written
        Code scratch_code;
        R.memo.emplace_back();
        std::vector<std::string> cs;
        for (auto& sy : P.qcoords) cs.push_back(sy.render({"hh", "(idx_t)0", "dd", "qrow"}));
        R.value(scratch_code, P.qnode, cs);
        R.memo.pop_back();
    }
    std::string qp = P.qexpr ? std::string() : R.param(P.qacc.buffer), kp = R.param(P.kacc.buffer), vp = R.param(P.vacc.buffer);

    std::ostringstream src;
    src << kPrelude;
    src << "typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;\n";
    src << "typedef short sanic_s16x4 __attribute__((ext_vector_type(4)));\n";
    src << "typedef short sanic_s16x8 __attribute__((ext_vector_type(8)));\n";
    src << "typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;\n";
    // tiling variants for the measured tuner: {3 workgroups per CU, 2 per CU, key range split
    // in two}. The split form gives every (head, query block) two workgroups, each folding half
    // of the block's key tiles; they exchange their (m, ℓ, o) partials through scratch and the
    // second to arrive combines them (the carrier's ExpShifted combine with its −∞ guard) and
    // projects. It evens out launches whose equal-sized blocks overfill the resident slots.
    const int fvar = d->stages[si].sched.variant;
    int SPL = fvar == 2 ? 2 : 1;
    src << (SPL > 1 ? R.args_struct({"float* __restrict__ scratch"}) : R.args_struct({}));
    src << "typedef __bf16 sanic_bf16x2 __attribute__((ext_vector_type(2)));\n";
    src << "typedef float sanic_f32x2 __attribute__((ext_vector_type(2)));\n";
    src << "__device__ __forceinline__ unsigned pk_bf16(float x, float y) {\n"
           "  return __builtin_bit_cast(unsigned, __builtin_convertvector((sanic_f32x2){x, y}, sanic_bf16x2));\n}\n";
    // max across the 4 lane groups of a query column (lanes l, l^16, l^32, l^48): gfx950
    // permlane swaps, no LDS round trip
    // compiler-visible maxima: the compiler forms v_max3_f32 itself and, unlike for inline asm
    // (which it cannot see into), inserts the wait states a VALU read of a fresh MFMA result
    // needs; an asm max placed right after the MFMA read stale accumulator registers
    src << "__device__ __forceinline__ float hmax(float a, float b) {\n"
           "  return __builtin_fmaxf(a, b);\n}\n";
    src << "__device__ __forceinline__ float hmax3(float a, float b, float c) {\n"
           "  return __builtin_fmaxf(__builtin_fmaxf(a, b), c);\n}\n";
    src << "__device__ __forceinline__ float wave_max_x4(float v) {\n"
           "  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);\n"
           "  v = hmax(__uint_as_float(r32[0]), __uint_as_float(r32[1]));\n"
           "  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);\n"
           "  return hmax(__uint_as_float(r16[0]), __uint_as_float(r16[1]));\n}\n";
    src << "__device__ __forceinline__ float wave_sum_x4(float v) {\n"
           "  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);\n"
           "  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);\n"
           "  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);\n"
           "  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);\n}\n";
    src << "__device__ __forceinline__ float score_part(const Args& a, float dotv, int hh, int qi, int kj) {\n"
        << entry_part << sp.str() << "  return " << vpart << ";\n}\n";
    src << "__device__ __forceinline__ float score_full(const Args& a, float dotv, int hh, int qi, int kj) {\n"
        << entry_full << sf.str() << "  return " << vfull << ";\n}\n";
    src << "__device__ __forceinline__ void window(const Args& a, idx_t hh, idx_t qrow, idx_t& lo, idx_t& hi) {\n"
        << Rw.entry() << wc.str() << "  lo = wlo; hi = whi;\n}\n";
    // the same bounds before an empty window is widened to the whole stream; true = non-empty
    bool raw_ok = true;
    {
        static const std::regex reset(R"(\n *if \(whi <= wlo\) \{ wlo = 0; whi = \d+; \})");
        const std::string raw = std::regex_replace(wc.str(), reset, "");
        // without the reset line removed, window_raw could not tell an empty window: edge
        // tiles then take the rendered leaf
        if (raw == wc.str() && wc.str().find("whi <= wlo") != std::string::npos) raw_ok = false;
        src << "__device__ __forceinline__ bool window_raw(const Args& a, idx_t hh, idx_t qrow, idx_t& lo, idx_t& hi) {\n"
            << Rw.entry() << raw << "  lo = wlo; hi = whi;\n  return whi > wlo;\n}\n";
    }
    src << "__device__ __forceinline__ void finish(const Args& a, const float* fs, idx_t hh, idx_t qi, idx_t ee) {\n"
        << Ro.entry() << fo.str() << "}\n";

    const std::string kname = "sanic_flash_h" + std::to_string(NH) + "_s" + std::to_string(NQ) + "_t" + std::to_string(T);
    Code k;
    k.indent = 1;
    // K and V tiles in a ring of three LDS buffers, filled straight from global memory
    // (global_load_lds, no register staging) two tiles ahead of the MFMAs. Rows are 128 bytes
    // unpadded with the 16-byte chunk index XORed by (row mod 8): a padded stride would put the
    // 16 rows of one fragment read into 2-way bank conflicts on gfx950, and the direct loads
    // write each wave's 1 KB contiguously, so the swizzle is applied to the source addresses.
    k.line("__shared__ __attribute__((aligned(16))) unsigned short kv_lds[3][2][64 * 64];");
    // (the wave index through a scalar register: the LDS destinations of the direct loads and
    // the wave's row range are then scalar arithmetic)
    k.line("const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);");
    k.line("const int l16 = lane & 15, lq = lane >> 4;");
    // XCD-aware block order: blockIdx mod 8 picks the KV head group, heaviest query blocks first
    const int64_t NKV = NH / P.rep;
    const int64_t NB = NH * NQB;
    if (SPL > 1) {
        k.line("const idx_t bid = blockIdx.x % " + std::to_string(NB) + ";");   // partners share an XCD
        k.line("const int part = (int)(blockIdx.x / " + std::to_string(NB) + ");");
    } else {
        k.line("const idx_t bid = blockIdx.x;");
    }
    if (NKV % 8 == 0 || NKV == 8) {
        k.line("const idx_t kvh = bid % " + std::to_string(NKV) + ", rest = bid / " + std::to_string(NKV) + ";");
        k.line("const idx_t hh = kvh * " + std::to_string(P.rep) + " + rest % " + std::to_string(P.rep) + ";");
        k.line("const idx_t qb = " + std::to_string(NQB - 1) + " - rest / " + std::to_string(P.rep) + ";");
    } else {
        k.line("const idx_t hh = bid % " + std::to_string(NH) + ";");
        k.line("const idx_t qb = " + std::to_string(NQB - 1) + " - bid / " + std::to_string(NH) + ";");
    }
    k.line("const idx_t q0 = qb * 128 + wv * 32;");   // this wave's 32 query rows
    // block and wave key ranges from the honest window of the first and last rows
    k.line("idx_t blo_a, bhi_a, blo_b, bhi_b, wlo_a, whi_a, wlo_b, whi_b;");
    k.line("window(a, hh, qb * 128, blo_a, bhi_a);");
    k.line("window(a, hh, qb * 128 + 127, blo_b, bhi_b);");
    k.line("window(a, hh, q0, wlo_a, whi_a);");
    k.line("window(a, hh, q0 + 31, wlo_b, whi_b);");
    if (SPL > 1) {
        k.line("const idx_t klo0 = (blo_a < blo_b ? blo_a : blo_b) / 64 * 64;");
        k.line("const idx_t khi0 = bhi_a > bhi_b ? bhi_a : bhi_b;");
        k.line("const idx_t ntl = khi0 > klo0 ? (khi0 - klo0 + 63) / 64 : 0;");
        k.line("const idx_t klo = klo0 + (part * ntl / 2) * 64;");
        k.line("const idx_t khi = part == 0 ? (klo0 + (ntl / 2) * 64 < khi0 ? klo0 + (ntl / 2) * 64 : khi0) : khi0;");
    } else {
        k.line("const idx_t klo = (blo_a < blo_b ? blo_a : blo_b) / 64 * 64;");
        k.line("const idx_t khi = bhi_a > bhi_b ? bhi_a : bhi_b;");
    }
    k.line("const idx_t wlo = wlo_a < wlo_b ? wlo_a : wlo_b, whi = whi_a > whi_b ? whi_a : whi_b;");
    k.line("const idx_t flo = wlo_a > wlo_b ? wlo_a : wlo_b, fhi = whi_a < whi_b ? whi_a : whi_b;");
    // the bounds are wave-uniform (they depend on the block and wave only): held in scalar
    // registers, the key loop's control and the tile classification run on the scalar unit
    k.line("const int klo_s = __builtin_amdgcn_readfirstlane((int)klo), khi_s = __builtin_amdgcn_readfirstlane((int)khi);");
    k.line("const int wlo_s = __builtin_amdgcn_readfirstlane((int)wlo), whi_s = __builtin_amdgcn_readfirstlane((int)whi);");
    k.line("const int flo_s = __builtin_amdgcn_readfirstlane((int)flo), fhi_s = __builtin_amdgcn_readfirstlane((int)fhi);");
    // Edge tiles, per element: inside a row's honest window the score is the unmasked form
    // (the full-tile identity); outside it −1e30 instead of the rendered mask (a finite mask
    // gives that same value for any score below ~1e22; a −∞ mask differs only while a row has
    // seen no visible key). Once a row has seen a visible key either weighs exactly 0, and what
    // a row accumulated before that is scaled by α = exp(−1e30 − m) = 0 on its first visible
    // tile, so the result is the same bit for bit — provided every row of the wave has a
    // non-empty window (else the rendered leaf per element). A finite value, not −∞, keeps
    // fully masked tiles at α = 1 (no rescale pass).
    // (the row bounds are recomputed on edge tiles only: kept live across the loop they cost
    // registers the window configuration spills)
    // (variant 3 takes the rendered leaf on every edge tile: the reference form the fast path
    // is tested against bit for bit)
    const bool edge_on = raw_ok && fvar != 3;
    // Q^T as the B operand (lane = query column l16 (+16·qt), d-slots lq·8 + 0..7 (+32·ds)),
    // held in registers for the whole key loop, loaded once from global memory
    k.line("bf16x8 qf[2][2];");
    if (!P.qexpr) {
        k.line("#pragma unroll");
        k.line("for (int qt = 0; qt < 2; ++qt)");
        k.line("  #pragma unroll");
        k.line("  for (int ds = 0; ds < 2; ++ds)");
        k.line("    qf[qt][ds] = *(const bf16x8*)(" + qp + " + " + std::to_string(P.qacc.addr.c0) + " + " + hterm(qc, qh, qhc) +
               " + (q0 + qt * 16 + l16) * " + std::to_string(qc[3]) + " + (ds * 4 + lq) * 8);");
    }
    // An expression query side is rendered element by element (the lane's 2 × 16 values), once
    // per workgroup, after the first K/V transfers are requested so its loads and arithmetic
    // overlap them; each value goes to the MFMA rounded to bf16 (RNE), the operand width.
    // The vectorised form's loads go out first, where the plain Q load would (loads complete in
    // issue order, so the rotation's operands are not queued behind the first K/V tiles), and
    // its arithmetic after the transfers are requested; the per-element form runs after them.
    Code q_lc, q_dc;
    bool q_runs = false;
    std::vector<std::string> q_vals[2][2];
    if (P.qexpr) {
        q_lc.indent = q_dc.indent = k.indent + 1;
        bool ok = true;
        for (int qt = 0; qt < 2 && ok; qt++)
            for (int ds = 0; ds < 2 && ok; ds++) {
                const std::string sfx = "_q" + std::to_string(qt) + std::to_string(ds);
                const std::vector<std::string> vars = {"hh", "(idx_t)0", "((idx_t)lq * 8 + " + std::to_string(ds * 32) + ")",
                                                       "(q0 + " + std::to_string(qt * 16) + " + l16)"};
                std::vector<int> bufs, dts;
                q_vals[qt][ds] = render_run(d, P.qnode, P.qcoords, {NH, T, HD, NQ}, vars, 2, q_lc, q_dc, sfx, bufs, dts, ok);
                for (size_t b = 0; b < bufs.size() && ok; b++)
                    k.line("const " + std::string(ctype_of(dts[b])) + "* __restrict__ rb" + std::to_string(b) + sfx + " = " + R.param(bufs[b]) + ";");
            }
        q_runs = ok;
        // the loads right away, as the plain Q load would be
        if (q_runs) k.s << q_lc.str();
    }
    auto emit_qexpr = [&]() {
        if (q_runs) {
            k.s << q_dc.str();
            for (int qt = 0; qt < 2; qt++)
                for (int ds = 0; ds < 2; ds++) {
                    const auto& v = q_vals[qt][ds];
                    k.line("qf[" + std::to_string(qt) + "][" + std::to_string(ds) + "] = __builtin_bit_cast(bf16x8, (sanic_u32x4){pk_bf16(" + v[0] + ", " + v[1] +
                           "), pk_bf16(" + v[2] + ", " + v[3] + "), pk_bf16(" + v[4] + ", " + v[5] + "), pk_bf16(" + v[6] + ", " + v[7] + ")});");
                }
            return;
        }
        for (int qt = 0; qt < 2; qt++) {
            k.line("{");
            k.indent++;
            k.line("const idx_t qrow = q0 + " + std::to_string(qt * 16) + " + l16;");
            R.memo.emplace_back();
            std::string vals[2][8];
            for (int ds = 0; ds < 2; ds++)
                for (int j = 0; j < 8; j++) {
                    const std::string dd = "((idx_t)lq * 8 + " + std::to_string(ds * 32 + j) + ")";
                    std::vector<std::string> cs;
                    for (auto& sy : P.qcoords) cs.push_back(sy.render({"hh", "(idx_t)0", dd, "qrow"}));
                    vals[ds][j] = R.value(k, P.qnode, cs);
                }
            R.memo.pop_back();
            for (int ds = 0; ds < 2; ds++) {
                std::string pk = "(sanic_u32x4){";
                for (int q = 0; q < 4; q++)
                    pk += std::string(q ? ", " : "") + "pk_bf16(" + vals[ds][2 * q] + ", " + vals[ds][2 * q + 1] + ")";
                k.line("qf[" + std::to_string(qt) + "][" + std::to_string(ds) + "] = __builtin_bit_cast(bf16x8, " + pk + "});");
            }
            k.indent--;
            k.line("}");
        }
    };
    k.line("f32x4 o[4][2];");
    k.line("#pragma unroll");
    k.line("for (int dt = 0; dt < 4; ++dt) { o[dt][0] = (f32x4){0, 0, 0, 0}; o[dt][1] = (f32x4){0, 0, 0, 0}; }");
    k.line("float m_run[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};");
    // row sums ℓ accumulate on the matrix cores: a row of ones times P^T (same bf16 P as O)
    k.line("f32x4 lsum[2] = {(f32x4){0, 0, 0, 0}, (f32x4){0, 0, 0, 0}};");
    k.line("const bf16x8 ones = {0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80};");
    const double LOG2E = 1.4426950408889634;
    // Lazy reference max: the running max moves only when a tile's max exceeds it by more than
    // TAU (natural-log units, so every p stays below 2^8): the online softmax is exact for any
    // reference point, and rescaling O and ℓ becomes rare. Only when the projection does not
    // read the max slot itself.
    std::function<bool(int)> reads_f = [&](int e) -> bool {
        const sanic_expr& x = d->exprs[e];
        if (x.op == SANIC_EX_F) return x.index == P.max_slot;
        if (x.op >= SANIC_EX_CONST) return false;
        for (int ch : {x.a, x.b, x.c}) if (ch >= 0 && reads_f(ch)) return true;
        return false;
    };
    const bool lazy = !reads_f(c.project);
    const double TAU = 8.0 / LOG2E;
    // One tile (K: 64 keys × 64 d; V rows [key][e] or V^T rows [e][key] as they lie in memory)
    // into ring buffer b: wave w's transfer u fills LDS rows 8(w + 4u) .. +7, lane l landing on
    // row 8(w + 4u) + l/8, chunk l%8 — so it fetches global chunk (l%8) ^ (l/8) of that row.
    // Four transfers per lane per tile, counted by vmcnt like any global load.
    std::string kbase = std::to_string(P.kacc.addr.c0) + " + " + hterm(kc, kh, khc);
    std::string vbase = std::to_string(P.vacc.addr.c0) + " + " + hterm(vc, vh, vhc);
    k.line("auto fetch = [&](idx_t tt, int b) {");
    k.line("  #pragma unroll");
    k.line("  for (int u = 0; u < 2; ++u) {");
    k.line("    const int r = 8 * (wv + 4 * u) + (lane >> 3), c = (lane & 7) ^ (lane >> 3);");
    k.line("    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(" + kp + " + " + kbase + " + (tt + r) * " +
           std::to_string(kc[1]) + " + c * 8), (__attribute__((address_space(3))) void*)(&kv_lds[b][0][(wv + 4 * u) * 512]), 16, 0, 0);");
    const std::string vsrc = v_rows ? "(tt + r) * " + std::to_string(vc[1]) + " + c * 8"
                                    : "(idx_t)r * " + std::to_string(vc[2]) + " + tt + c * 8";
    k.line("    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(" + vp + " + " + vbase + " + " + vsrc +
           "), (__attribute__((address_space(3))) void*)(&kv_lds[b][1][(wv + 4 * u) * 512]), 16, 0, 0);");
    k.line("  }");
    k.line("};");
    k.line("if (klo_s < khi_s) {");
    k.indent++;
    k.line("fetch(klo_s, 0);");
    k.line("if (klo_s + 64 < khi_s) fetch(klo_s + 64, 1);");
    if (P.qexpr) emit_qexpr();
    k.line("int buf = 0;");
    k.line("for (int t0 = klo_s; t0 < khi_s; t0 += 64) {");
    k.indent++;
    // this tile's transfers have landed for every wave (only the next tile's four may still be
    // in flight; loads complete in issue order). The buffer the transfer below refills was read
    // in the previous iteration: this barrier orders every wave's reads of it before the refill,
    // so the refill must stay after the barrier. The asm carries the memory clobber that keeps
    // the compiler from moving LDS accesses across the barrier.
    k.line("if (t0 + 64 < khi_s) asm volatile(\"s_waitcnt vmcnt(4)\\n\\ts_barrier\" ::: \"memory\");");
    k.line("else asm volatile(\"s_waitcnt vmcnt(0)\\n\\ts_barrier\" ::: \"memory\");");
    k.line("if (t0 + 128 < khi_s) fetch(t0 + 128, buf == 0 ? 2 : buf - 1);");
    // wave-uniform tile classification (scalar branches)
    k.line("const int live = t0 < whi_s && t0 + 64 > wlo_s;");   // some row sees it
    k.line("if (live) {");
    k.indent++;
    k.line("const int full = t0 >= flo_s && t0 + 64 <= fhi_s;");  // every row sees all
    // S^T tiles: kt (16 keys) × qt (16 queries), contraction over d in 2 steps of 32
    // both query tiles' scores first: each K fragment is read from LDS once for the two tiles
    // (measured: 2% over re-reading it per tile, the kernel being bound by LDS and MFMA issue).
    // The split variant and the rendered-mask reference variant keep one query tile's scores
    // live at a time (with both live they spill 12–13 registers); the products are the same
    // MFMAs in the same order either way.
    const bool s_both = SPL == 1 && fvar != 3;
    k.line("f32x4 s[4][2];");
    k.line("sanic_u32x4 pw[2][2];");
    auto scores = [&](bool both) {
        k.line("#pragma unroll");
        k.line("for (int kt = 0; kt < 4; ++kt) {");
        k.line(both ? "  s[kt][0] = (f32x4){0, 0, 0, 0};" : "  s[kt][qt] = (f32x4){0, 0, 0, 0};");
        if (both) k.line("  s[kt][1] = (f32x4){0, 0, 0, 0};");
        k.line("  #pragma unroll");
        k.line("  for (int ds = 0; ds < 2; ++ds) {");
        k.line("    const bf16x8 ka = *(const bf16x8*)(&kv_lds[buf][0][(kt * 16 + l16) * 64 + (((ds * 4 + lq) ^ (l16 & 7)) * 8)]);");
        if (both) {
            k.line("    #pragma unroll");
            k.line("    for (int qt = 0; qt < 2; ++qt) {");
        } else {
            k.line("    {");
        }
        k.line("      s[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[qt][ds], s[kt][qt], 0, 0, 0);");
        k.line("    }");
        k.line("  }");
        k.line("}");
    };
    if (s_both) scores(true);
    // online softmax per query column (lane-local; the max reduces across the 4 lane groups)
    k.line("#pragma unroll");
    k.line("for (int qt = 0; qt < 2; ++qt) {");
    k.indent++;
    if (!s_both) scores(false);
    k.line("const int qi = (int)(q0 + qt * 16 + l16);");
    k.line("float sv[16];");
    k.line("float p[16];");
    k.line("float mn, alpha;");
    if (scale_known) {
        // full tiles: score = dot·c, so max and exp2 work on the raw dot (c > 0)
        k.line("if (full) {");
        k.indent++;
        // 16 → 1 in 8 three-input maxes
        k.line("const float ma = hmax3(s[0][qt][0], s[0][qt][1], s[0][qt][2]), mb_ = hmax3(s[0][qt][3], s[1][qt][0], s[1][qt][1]);");
        k.line("const float mc = hmax3(s[1][qt][2], s[1][qt][3], s[2][qt][0]), md = hmax3(s[2][qt][1], s[2][qt][2], s[2][qt][3]);");
        k.line("const float me = hmax3(s[3][qt][0], s[3][qt][1], s[3][qt][2]);");
        k.line("float mt = hmax3(hmax3(ma, mb_, mc), hmax3(md, me, s[3][qt][3]), ma);");
        // Common case: no lane's scores move its row's running max (every lane's own maximum
        // within the rescale threshold, the running max finite). Then mn = m_run and alpha = 1
        // exactly, as the general form below would find, without the cross-lane reduction,
        // the rescale factor's exp2 or the rescale.
        const std::string keep = lazy ? "m_run[qt] + " + flit(TAU) : std::string("m_run[qt]");
        k.line("if (__all(mt * " + flit(scale_c) + " <= " + keep + " && m_run[qt] > -1e29f)) {");
        k.line("  mn = m_run[qt];");
        k.line("  alpha = 1.0f;");
        k.line("  const float mb = mn * " + flit(LOG2E) + ";");
        k.line("  #pragma unroll");
        k.line("  for (int kt = 0; kt < 4; ++kt)");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < 4; ++r) p[kt * 4 + r] = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][r], " + flit(scale_c * LOG2E) + ", -mb));");
        k.line("} else {");
        k.indent++;
        k.line("mt = wave_max_x4(mt) * " + flit(scale_c) + ";");
        k.line(lazy ? "mn = mt > m_run[qt] + " + flit(TAU) + " ? mt : m_run[qt];" : "mn = fmaxf(m_run[qt], mt);");
        k.line("alpha = m_run[qt] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((m_run[qt] - mn) * " + flit(LOG2E) + ");");
        k.line("if (__all(mn > -1e29f)) {");
        k.line("  const float mb = mn * " + flit(LOG2E) + ";");
        k.line("  #pragma unroll");
        k.line("  for (int kt = 0; kt < 4; ++kt)");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < 4; ++r) p[kt * 4 + r] = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][r], " + flit(scale_c * LOG2E) + ", -mb));");
        k.line("} else {");
        k.line("  #pragma unroll");
        k.line("  for (int kt = 0; kt < 4; ++kt)");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < 4; ++r) p[kt * 4 + r] = mn == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((s[kt][qt][r] * " + flit(scale_c) + " - mn) * " + flit(LOG2E) + ");");
        k.line("}");
        k.indent--;
        k.line("}");
        k.indent--;
        k.line("} else {");
        k.indent++;
    } else {
        k.line("{");
        k.indent++;
    }
    // partial tiles (and scores of any other shape): the rendered leaf per element
    // (full and edge_fast are wave-uniform: one branch per tile, not a select per element)
    // (the key indices are formed here, in the branch that uses them: the compiler would
    // otherwise hoist them ahead of the full-tile branch)
    k.line("int kb = t0 + lq * 4;");
    k.line("asm volatile(\"\" : \"+v\"(kb));");
    k.line("int elo = -1, ehi = 0x7fffffff;");
    if (edge_on) {
        k.line("if (!full) {");
        k.line("  idx_t rl, rh;");
        k.line("  const bool ok = window_raw(a, hh, qi, rl, rh);");
        k.line("  if (__all(ok)) { elo = (int)rl; ehi = (int)rh; } else { elo = 0x7fffffff; }");
        k.line("}");
    } else {
        k.line("if (!full) elo = 0x7fffffff;");
    }
    k.line("if (elo != 0x7fffffff) {");
    k.line("  #pragma unroll");
    k.line("  for (int kt = 0; kt < 4; ++kt)");
    k.line("    #pragma unroll");
    k.line("    for (int r = 0; r < 4; ++r) {");
    k.line("      const int kj = kb + kt * 16 + r;");
    k.line("      const float sf = score_full(a, s[kt][qt][r], (int)hh, qi, kj);");
    k.line("      sv[kt * 4 + r] = kj >= elo && kj < ehi ? sf : -1e30f;");
    k.line("    }");
    k.line("} else {");
    k.line("  #pragma unroll");
    k.line("  for (int kt = 0; kt < 4; ++kt)");
    k.line("    #pragma unroll");
    k.line("    for (int r = 0; r < 4; ++r) sv[kt * 4 + r] = score_part(a, s[kt][qt][r], (int)hh, qi, kb + kt * 16 + r);");
    k.line("}");
    k.line("float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));");
    k.line("#pragma unroll");
    k.line("for (int i = 4; i < 16; i += 2) mt = fmaxf(mt, fmaxf(sv[i], sv[i + 1]));");
    k.line("mt = wave_max_x4(mt);");
    k.line(lazy ? "mn = mt > m_run[qt] + " + flit(TAU) + " ? mt : m_run[qt];" : "mn = fmaxf(m_run[qt], mt);");
    // the carrier's guarded rescale: a side whose max is −∞ weighs 0
    k.line("alpha = m_run[qt] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((m_run[qt] - mn) * " + flit(LOG2E) + ");");
    // Fast form exp2(s·log2e − m·log2e) (one FMA) while every row of the wave has a moderate
    // max; when some row's max is a masked score (≈ −1e30) or −∞ the fused form does not
    // cancel exactly, so (s − m)·log2e is used for that tile.
    k.line("if (__all(mn > -1e29f)) {");
    k.line("  const float mb = mn * " + flit(LOG2E) + ";");
    k.line("  #pragma unroll");
    k.line("  for (int i = 0; i < 16; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], " + flit(LOG2E) + ", -mb));");
    k.line("} else {");
    k.line("  #pragma unroll");
    k.line("  for (int i = 0; i < 16; ++i) p[i] = mn == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((sv[i] - mn) * " + flit(LOG2E) + ");");
    k.line("}");
    k.indent--;
    k.line("}");
    k.line("m_run[qt] = mn;");
    k.line("if (!__all(alpha == 1.0f)) {");   // the running max moved for some row: rescale
    k.line("  #pragma unroll");
    k.line("  for (int dt = 0; dt < 4; ++dt) { o[dt][qt][0] *= alpha; o[dt][qt][1] *= alpha; o[dt][qt][2] *= alpha; o[dt][qt][3] *= alpha; }");
    k.line("  lsum[qt] *= alpha;");
    k.line("}");
    // P^T as the B operand for key step ks: slots 0..3 = keys 32ks + lq·4 + r (tile 2ks),
    // slots 4..7 = keys 32ks + 16 + lq·4 + r (tile 2ks+1); two slots per dword, RNE in hardware
    k.line("#pragma unroll");
    k.line("for (int ks = 0; ks < 2; ++ks) {");
    k.line("  pw[qt][ks].x = pk_bf16(p[8 * ks + 0], p[8 * ks + 1]);");
    k.line("  pw[qt][ks].y = pk_bf16(p[8 * ks + 2], p[8 * ks + 3]);");
    k.line("  pw[qt][ks].z = pk_bf16(p[8 * ks + 4], p[8 * ks + 5]);");
    k.line("  pw[qt][ks].w = pk_bf16(p[8 * ks + 6], p[8 * ks + 7]);");
    k.line("}");
    k.indent--;
    k.line("}");
    k.line("bf16x8 pf[2][2];");
    k.line("#pragma unroll");
    k.line("for (int qt = 0; qt < 2; ++qt) { pf[qt][0] = __builtin_bit_cast(bf16x8, pw[qt][0]); pf[qt][1] = __builtin_bit_cast(bf16x8, pw[qt][1]); }");
    // O^T += V^T · P^T ; V^T A operand: row e = dt·16 + l16, keys in the same slot order
    k.line("#pragma unroll");
    k.line("for (int ks = 0; ks < 2; ++ks) {");
    k.line("  lsum[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[0][ks], lsum[0], 0, 0, 0);");
    k.line("  lsum[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[1][ks], lsum[1], 0, 0, 0);");
    k.line("}");
    if (v_rows) {
        // V rows in LDS, read transposed (ds_read_b64_tr_b16): in each 16-lane group, source
        // lane s reads 4 values of e at key row (base + s/4), e = dt·16 + 4·(s%4); lane i then
        // holds keys base + 0..3 of e = dt·16 + i — slots 0..3, and base + 16 gives slots 4..7
        // (row + 16 has the same swizzle as row). The reads are issued from inline asm, two
        // value tiles (8 reads) at a time, each group completed by an explicit lgkmcnt wait
        // that the fragments pass through: the compiler's own form of this read waits for
        // every outstanding direct-to-LDS transfer first (vmcnt(0), i.e. the next tile's
        // prefetch), which the loop-top barrier already orders for this buffer.
        k.line("sanic_s16x4 vt[4][2][2];");
        auto vreads = [&](int dt0) {
            for (int dt = dt0; dt < dt0 + 2; dt++)
                for (int ks = 0; ks < 2; ks++) {
                    const std::string ix = "[" + std::to_string(dt) + "][" + std::to_string(ks) + "]";
                    k.line("{");
                    k.line("  const int vrow = " + std::to_string(ks * 32) + " + lq * 4 + (l16 >> 2), vcol = " + std::to_string(dt * 16) + " + (l16 & 3) * 4;");
                    k.line("  const unsigned va_ = (unsigned)(size_t)((__attribute__((address_space(3))) const unsigned short*)&kv_lds[buf][1][vrow * 64 + (((vcol >> 3) ^ (vrow & 7)) << 3) + (vcol & 7)]);");
                    k.line("  asm volatile(\"ds_read_b64_tr_b16 %0, %1\" : \"=v\"(vt" + ix + "[0]) : \"v\"(va_));");
                    k.line("  asm volatile(\"ds_read_b64_tr_b16 %0, %1 offset:2048\" : \"=v\"(vt" + ix + "[1]) : \"v\"(va_));");
                    k.line("}");
                }
        };
        auto vwait = [&](int dt0) {
            std::string ops;
            for (int dt = dt0; dt < dt0 + 2; dt++)
                for (int ks = 0; ks < 2; ks++)
                    for (int h = 0; h < 2; h++)
                        ops += std::string(ops.empty() ? "" : ", ") + "\"+v\"(vt[" + std::to_string(dt) + "][" + std::to_string(ks) + "][" + std::to_string(h) + "])";
            k.line("asm volatile(\"s_waitcnt lgkmcnt(0)\" : " + ops + ");");
        };
        auto vmfma = [&](int dt0) {
            for (int dt = dt0; dt < dt0 + 2; dt++)
                for (int ks = 0; ks < 2; ks++) {
                    const std::string ix = "[" + std::to_string(dt) + "][" + std::to_string(ks) + "]";
                    const std::string va = "__builtin_bit_cast(bf16x8, (sanic_s16x8)__builtin_shufflevector(vt" + ix + "[0], vt" + ix + "[1], 0, 1, 2, 3, 4, 5, 6, 7))";
                    k.line("o[" + std::to_string(dt) + "][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(" + va + ", pf[0][" + std::to_string(ks) + "], o[" + std::to_string(dt) + "][0], 0, 0, 0);");
                    k.line("o[" + std::to_string(dt) + "][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(" + va + ", pf[1][" + std::to_string(ks) + "], o[" + std::to_string(dt) + "][1], 0, 0, 0);");
                }
        };
        vreads(0);
        vwait(0);
        vreads(2);
        vmfma(0);
        vwait(2);
        vmfma(2);
    }
    if (!v_rows) {
    k.line("#pragma unroll");
    k.line("for (int dt = 0; dt < 4; ++dt)");
    k.line("  #pragma unroll");
    k.line("  for (int ks = 0; ks < 2; ++ks) {");
    {
        k.line("    const int vrow = dt * 16 + l16, vcol = ks * 32 + lq * 4;");
        k.line("    const unsigned short* vr = &kv_lds[buf][1][vrow * 64 + (((vcol >> 3) ^ (vrow & 7)) << 3) + (vcol & 7)];");
        k.line("    const unsigned short* vr2 = &kv_lds[buf][1][vrow * 64 + ((((vcol + 16) >> 3) ^ (vrow & 7)) << 3) + (vcol & 7)];");
        k.line("    const uint2 lo4 = *(const uint2*)(vr), hi4 = *(const uint2*)(vr2);");
        k.line("    const bf16x8 va = __builtin_bit_cast(bf16x8, (sanic_u32x4){lo4.x, lo4.y, hi4.x, hi4.y});");
    }
    k.line("    o[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[0][ks], o[dt][0], 0, 0, 0);");
    k.line("    o[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[1][ks], o[dt][1], 0, 0, 0);");
    k.line("  }");
    }
    k.indent--;
    k.line("}");
    k.line("buf = buf == 2 ? 0 : buf + 1;");
    k.indent--;
    k.line("}");
    k.indent--;
    k.line("}");
    int64_t soff = -1;
    if (SPL > 1) {
        // partials [block][part][36][256 lanes] (o in accumulator order, m, ℓ), then one arrival
        // counter per block (zeroed at bind time, re-armed by the combining workgroup)
        soff = scratch;
        const int64_t pbytes = NB * 2 * 36 * 256 * 4;
        scratch += pbytes + ((NB * 4 + 255) / 256) * 256;
        k.line("{");
        k.indent++;
        k.line("float* pw = a.scratch + ((idx_t)bid * 2 + part) * 9216 + tid;");
        k.line("#pragma unroll");
        k.line("for (int dt = 0; dt < 4; ++dt)");
        k.line("  #pragma unroll");
        k.line("  for (int qt = 0; qt < 2; ++qt)");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < 4; ++r) sanic_st(pw + ((dt * 2 + qt) * 4 + r) * 256, o[dt][qt][r]);");
        k.line("for (int qt = 0; qt < 2; ++qt) { sanic_st(pw + (32 + qt) * 256, m_run[qt]); sanic_st(pw + (34 + qt) * 256, lsum[qt][0]); }");
        k.line("unsigned* cnt = (unsigned*)((char*)a.scratch + " + std::to_string(pbytes) + ") + bid;");
        emit_arrival(k, "sp_last", "tid", "cnt", "2u");
        k.line("if (!sp_last) return;");
        k.line("if (tid == 0) sanic_st(cnt, 0u);");
        // the combine always takes part 0's values as the left operand of one explicit fma
        // (a·wa + b·wb with the product b·wb rounded first), so the rounding does not depend on
        // which half arrived last
        k.line("const float* pr = a.scratch + ((idx_t)bid * 2 + (1 - part)) * 9216 + tid;");
        k.line("#pragma unroll");
        k.line("for (int qt = 0; qt < 2; ++qt) {");
        k.line("  const float mo = sanic_ld(pr + (32 + qt) * 256), lo = sanic_ld(pr + (34 + qt) * 256);");
        k.line("  const float M = __builtin_fmaxf(m_run[qt], mo);");
        k.line("  const float ws = m_run[qt] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((m_run[qt] - M) * " + flit(LOG2E) + ");");
        k.line("  const float wo = mo == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f((mo - M) * " + flit(LOG2E) + ");");
        k.line("  const bool p0 = part == 0;");
        k.line("  lsum[qt][0] = p0 ? __builtin_fmaf(lsum[qt][0], ws, lo * wo) : __builtin_fmaf(lo, wo, lsum[qt][0] * ws);");
        k.line("  m_run[qt] = M;");
        k.line("  #pragma unroll");
        k.line("  for (int dt = 0; dt < 4; ++dt)");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < 4; ++r) {");
        k.line("      const float ov = sanic_ld(pr + ((dt * 2 + qt) * 4 + r) * 256);");
        k.line("      o[dt][qt][r] = p0 ? __builtin_fmaf(o[dt][qt][r], ws, ov * wo) : __builtin_fmaf(ov, wo, o[dt][qt][r] * ws);");
        k.line("    }");
        k.line("}");
        k.indent--;
        k.line("}");
    }
    // finish: the row sum across the 4 lane groups, then project per output point
    k.line("#pragma unroll");
    k.line("for (int qt = 0; qt < 2; ++qt) {");
    k.indent++;
    k.line("const float lt = lsum[qt][0];");
    k.line("const idx_t qi = q0 + qt * 16 + l16;");
    k.line("#pragma unroll");
    k.line("for (int dt = 0; dt < 4; ++dt)");
    k.line("  #pragma unroll");
    k.line("  for (int r = 0; r < 4; ++r) {");
    k.line("    float fs[" + std::to_string(c.slots) + "];");
    k.line("    fs[" + std::to_string(P.max_slot) + "] = m_run[qt];");
    for (size_t s = 0; s < P.scalar_slots.size(); s++)
        k.line("    fs[" + std::to_string(P.scalar_slots[s]) + "] = " + flit(P.scalar_into[s]) + " * lt;");
    k.line("    fs[" + std::to_string(P.vec_slots[0]) + "] = o[dt][qt][r];");
    k.line("    finish(a, fs, hh, qi, dt * 16 + lq * 4 + r);");
    k.line("  }");
    k.indent--;
    k.line("}");

    // three waves per SIMD: the softmax of one wave overlaps the MFMAs of the others (the
    // register cap costs a few spilled values outside the inner loop)
    // tiling variants for the measured tuner: workgroups per CU {3, 2}
    int occ = d->stages[si].sched.variant == 1 ? 2 : 3;
    src << "extern \"C\" __global__ void __launch_bounds__(256, " << occ << ") " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
    out.kernel_kind = "skeleton:flash_prefill[rep " + std::to_string(P.rep) + "]" + (SPL > 1 ? "+split2" : "");
    out.source = src.str();
    out.variants = 4;
    std::vector<Arg> args = R.arg_list();
    if (SPL > 1) args.push_back({Arg::SCRATCH, soff});
    out.launches.push_back({kname, "", dim3((unsigned)(NB * SPL)), dim3(256), 0, args});
    return true;
}

}  // namespace sanic
