// Attention skeletons: the online-softmax (m, ℓ, o) carrier over a streamed key axis.
//
// Accepted structurally (derive.rs:518-530 slot kinds, the FlashAttention carrier of
// /root/reference/tests/laws.rs:108-126): one Plain(Max) slot whose `into` is a score item, the
// other slots ExpShifted on it with `into` either a constant (ℓ) or the value item (o); the
// score leaf contains exactly one in-body contraction Σ_d A·B where A (the query side) does not
// move with the stream and B (the key side) is an affine view of one buffer; the value leaf is
// an affine view too. GQA is read off the key/value addresses: when the head coordinate enters
// them as ⌊h / rep⌋, the `rep` query heads that share a key row are processed together so each
// K/V byte is read once.
//
//   attn_decode  (query grid = heads only) Flash-Decoding: the visible stream (honest window)
//                is cut into 64-position chunks, one workgroup per (KV head group, chunk) folds
//                its chunk into partial (m, ℓ, o) carriers in scratch; a second kernel merges the
//                partials with the carrier's own rendered combine (−∞ guard included), projects,
//                runs the epilogue and stores. Oracle: interp.rs:555-643 run_carrier_split.
#include <algorithm>
#include <regex>
#include <set>
#include <sstream>
#include <cmath>

#include "emit.h"
#include "skeletons.h"

namespace sanic {

namespace {

struct Dot {
    int reduce = -1;     // the Reduce(Add) node
    int a = -1, b = -1;  // query side (A) / key side (B) children of its Map(Mul)
    std::vector<std::string> a_coords;  // A coords in terms of "hq", "dd" (and 0)
    Access kacc;         // B address over vars {0: h, 1: t, 2: d}
    int64_t depth = 0;   // contraction length
};

struct AttnPlan {
    int stage = -1;
    int sleaf = -1, vleaf = -1;
    int max_slot = -1;
    std::vector<int> vec_slots, scalar_slots;
    std::vector<double> scalar_into;
    int hdim = -1, edim = -1;
    int64_t NH = 1, E = 1, T = 1;
    int rep = 1;
    Dot dot;
    Access vacc;         // V address over vars {0: h, 1: t, 2: e}
};

bool expr_is_item(const sanic_program_desc* d, int e, int& item) {
    const sanic_expr& x = d->exprs[e];
    if (x.op != SANIC_EX_ITEM) return false;
    item = x.index;
    return true;
}

bool expr_is_const(const sanic_program_desc* d, int e, double& v) {
    const sanic_expr& x = d->exprs[e];
    if (x.op != SANIC_EX_CONST) return false;
    v = x.value;
    return true;
}

bool contains_reduce(const sanic_program_desc* d, int node) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_REDUCE || n.kind == SANIC_NODE_SCAN) return true;
    for (int k = 0; k < n.n_in; k++) if (contains_reduce(d, n.in[k])) return true;
    return false;
}

bool sym_uses(const Sym& s, int var) {
    for (auto& t : s.terms) if (t.var == var) return true;
    return false;
}

// Find the single contraction in the score tree. `c` are the node's coords over {h, t}.
bool find_dot(const sanic_program_desc* d, int node, const std::vector<Sym>& c, const std::vector<int64_t>& ext, Dot& out) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_MAP) {
        int found = 0;
        for (int k = 0; k < n.n_in; k++) {
            if (!contains_reduce(d, n.in[k])) continue;
            const sanic_node& m = d->nodes[n.in[k]];
            int lead = n.rank - m.rank;
            std::vector<Sym> cc(m.rank);
            for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? Sym() : c[lead + j];
            if (!find_dot(d, n.in[k], cc, ext, out)) return false;
            found++;
        }
        return found == 1;
    }
    if (n.kind != SANIC_NODE_REDUCE || n.op != SANIC_MON_ADD) return false;
    const sanic_node& mp = d->nodes[n.in[0]];
    if (mp.kind != SANIC_NODE_MAP || mp.op != SANIC_OP_MUL) return false;
    std::vector<Sym> mc;
    for (int j = 0, o = 0; j < mp.rank; j++) mc.push_back(j == n.dim ? Sym::var(2) : c[o++]);
    std::vector<int64_t> ext3 = {ext[0], ext[1], mp.shape[n.dim]};
    int kside = -1;
    std::vector<std::vector<Sym>> childc(2);
    for (int k = 0; k < 2; k++) {
        const sanic_node& ch = d->nodes[mp.in[k]];
        int lead = mp.rank - ch.rank;
        childc[k].resize(ch.rank);
        bool moves = false;
        for (int j = 0; j < ch.rank; j++) {
            childc[k][j] = ch.shape[j] == 1 ? Sym() : mc[lead + j];
            moves |= sym_uses(childc[k][j], 1);
        }
        if (moves) {
            if (kside >= 0) return false;
            kside = k;
        }
    }
    if (kside < 0) return false;
    int qside = 1 - kside;
    if (!sym_access(d, mp.in[kside], childc[kside], ext3, out.kacc)) return false;
    // query-side coords as strings: h -> "hq", d -> "dd"
    const auto& qc = childc[qside];
    for (auto& s : qc) {
        if (s.terms.empty()) { out.a_coords.push_back(std::to_string(s.c0)); continue; }
        if (s.terms.size() != 1 || s.c0 != 0 || s.terms[0].coef != 1 || s.terms[0].div != 1 || s.terms[0].mod) return false;
        out.a_coords.push_back(s.terms[0].var == 0 ? "hq" : s.terms[0].var == 2 ? "dd" : "??");
        if (s.terms[0].var == 1) return false;
    }
    out.reduce = node;
    out.a = mp.in[qside];
    out.b = mp.in[kside];
    out.depth = mp.shape[n.dim];
    return true;
}

// Split an address into (h term div, stride of var v) — h may enter only as ⌊h/rep⌋.
bool addr_parts(const Sym& a, int& rep, int64_t NH, int64_t& s1, int64_t& s2, int64_t& sh) {
    rep = (int)NH;   // no h term: every head reads the same rows
    s1 = s2 = sh = 0;
    for (auto& t : a.terms) {
        if (t.mod != 0) return false;
        if (t.var == 0) {
            if (t.div < 1 || NH % t.div) return false;
            rep = (int)t.div;
            sh = t.coef;
        } else if (t.div != 1) {
            return false;
        } else if (t.var == 1) {
            s1 += t.coef;
        } else {
            s2 += t.coef;
        }
    }
    return true;
}

bool attn_plan(const sanic_program_desc* d, int si, AttnPlan& P) {
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_FUSED) return false;
    const sanic_carrier& c = st.carrier;
    P = AttnPlan();
    P.stage = si;
    for (int k = 0; k < c.slots; k++) {
        const sanic_slot& s = c.kind[k];
        if (s.kind == SANIC_SLOT_PLAIN && s.monoid == SANIC_MON_MAX) {
            if (P.max_slot >= 0) return false;
            P.max_slot = k;
        }
    }
    if (P.max_slot < 0) return false;
    if (!expr_is_item(d, c.into[P.max_slot], P.sleaf)) return false;
    for (int k = 0; k < c.slots; k++) {
        if (k == P.max_slot) continue;
        const sanic_slot& s = c.kind[k];
        if (s.kind != SANIC_SLOT_EXP_SHIFTED || s.ref_slot != P.max_slot) return false;
        int it;
        double v;
        if (expr_is_item(d, c.into[k], it)) {
            if (it == P.sleaf) return false;
            if (P.vleaf >= 0 && P.vleaf != it) return false;
            P.vleaf = it;
            P.vec_slots.push_back(k);
        } else if (expr_is_const(d, c.into[k], v)) {
            P.scalar_slots.push_back(k);
            P.scalar_into.push_back(v);
        } else {
            return false;
        }
    }
    if (P.vleaf < 0 || P.vec_slots.empty() || st.n_leaves != 2) return false;
    // grid: value dim = bound by the value leaf only; head dim = the other dim with extent > 1
    const sanic_node& sl = d->nodes[st.leaf[P.sleaf]];
    const sanic_node& vl = d->nodes[st.leaf[P.vleaf]];
    std::vector<bool> in_s(st.rank, false), in_v(st.rank, false);
    for (int j = 0; j < sl.rank; j++) if (st.bind[P.sleaf][j] >= 0) in_s[st.bind[P.sleaf][j]] = true;
    for (int j = 0; j < vl.rank; j++) if (st.bind[P.vleaf][j] >= 0) in_v[st.bind[P.vleaf][j]] = true;
    for (int j = 0; j < st.rank; j++) {
        if (st.grid[j] == 1) continue;
        if (in_v[j] && !in_s[j]) {
            if (P.edim >= 0) return false;
            P.edim = j;
        } else {
            if (P.hdim >= 0) return false;
            P.hdim = j;
        }
    }
    if (P.edim < 0) return false;
    P.E = st.grid[P.edim];
    P.NH = P.hdim >= 0 ? st.grid[P.hdim] : 1;
    P.T = st.stream;
    if (P.E > 256) return false;
    // the score leaf's contraction
    std::vector<Sym> sc(sl.rank);
    for (int j = 0; j < sl.rank; j++) {
        int b = st.bind[P.sleaf][j];
        sc[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : (b >= 0 && b == P.hdim) ? Sym::var(0) : Sym();
    }
    if (!find_dot(d, st.leaf[P.sleaf], sc, {P.NH, P.T}, P.dot)) return false;
    // value address over {h, t, e}
    std::vector<Sym> vc(vl.rank);
    for (int j = 0; j < vl.rank; j++) {
        int b = st.bind[P.vleaf][j];
        vc[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.hdim ? Sym::var(0) : b == P.edim ? Sym::var(2) : Sym();
    }
    if (!sym_access(d, st.leaf[P.vleaf], vc, {P.NH, P.T, P.E}, P.vacc)) return false;
    int repk, repv;
    int64_t kt, kd, kh, vt, ve, vh;
    if (!addr_parts(P.dot.kacc.addr, repk, P.NH, kt, kd, kh)) return false;
    if (!addr_parts(P.vacc.addr, repv, P.NH, vt, ve, vh)) return false;
    if (repk != repv || kd != 1 || P.dot.kacc.dtype != SANIC_BF16 || P.vacc.dtype != SANIC_BF16) return false;
    if (P.dot.depth % 8 || P.dot.depth > 256) return false;
    P.rep = repk;
    if (P.rep > 8) return false;
    return true;
}

// ── in-place K/V row writes performed by the attention kernel ──
// The decode step writes this position's K row and V column into the caches (a pointwise stage
// with a row `where`, emit_metal.rs:1103-1178) right before the attention reads them. The
// attention kernel does those writes itself: the workgroup whose chunk holds the row computes
// the group's row elements, stores them, and uses the stored (narrowed) values in place of the
// ones it prefetched, so no other launch or cross-workgroup ordering is needed.
struct RowWrite {
    int stage = -1, buffer = -1, rdim = -1, pos = -1;
    bool is_k = false;
    std::vector<int64_t> shape, stride;
};

int64_t eval_sym(const Sym& s, const std::vector<int64_t>& v) {
    int64_t r = s.c0;
    for (auto& t : s.terms) {
        int64_t x = v[t.var] / t.div;
        if (t.mod) x %= t.mod;
        r += t.coef * x;
    }
    return r;
}

// Does the attention's read of `acc` over (grp, t, x) (x < X) touch exactly the row t of the
// buffer, every element of it once across all groups?
bool row_mapping_ok(const Sym& addr, int REP, int64_t NG, int64_t T, int64_t X, const RowWrite& w) {
    int64_t vol = 1;
    for (auto e : w.shape) vol *= e;
    if (w.shape[w.rdim] != T || vol / T != NG * X) return false;
    for (int64_t t : {(int64_t)0, T / 2, T - 1}) {
        std::set<int64_t> seen;
        for (int64_t g = 0; g < NG; g++)
            for (int64_t x = 0; x < X; x++) {
                int64_t f = eval_sym(addr, {g * REP, t, x});
                if (f < 0 || f >= vol || (f / w.stride[w.rdim]) % w.shape[w.rdim] != t) return false;
                seen.insert(f);
            }
        if ((int64_t)seen.size() != NG * X) return false;
    }
    return true;
}

std::vector<RowWrite> absorbed_writes(const sanic_program_desc* d, int ai, const AttnPlan& P) {
    std::vector<RowWrite> out;
    if (getenv("SANIC_HIP_GENERIC")) return out;
    const int64_t NG = P.NH / P.rep;
    for (int s = ai - 1; s >= 0 && out.size() < 2; s--) {
        const sanic_stage& st = d->stages[s];
        if (st.kind != SANIC_STAGE_POINTWISE || st.where < 0) break;
        RowWrite w;
        w.stage = s;
        w.buffer = st.out_buffer;
        if (d->buffers[w.buffer].role != SANIC_BUF_STATE) break;
        if (!match_row_cond(d, st.where, st.rank, w.rdim, w.pos)) break;
        if (w.buffer == P.dot.kacc.buffer) w.is_k = true;
        else if (w.buffer != P.vacc.buffer) break;
        bool dup = false;
        for (auto& o : out) dup |= o.buffer == w.buffer;
        if (dup) break;
        std::set<int> reads;
        collect_inputs(d, st.value, reads);
        collect_inputs(d, st.where, reads);
        if (reads.count(P.dot.kacc.buffer) || reads.count(P.vacc.buffer)) break;
        for (int j = 0; j < st.rank; j++) w.shape.push_back(st.grid[j]);
        w.stride.assign(st.rank, 1);
        for (int j = st.rank - 2; j >= 0; j--) w.stride[j] = w.stride[j + 1] * w.shape[j + 1];
        bool ok = w.is_k ? row_mapping_ok(P.dot.kacc.addr, P.rep, NG, P.T, P.dot.depth, w)
                         : row_mapping_ok(P.vacc.addr, P.rep, NG, P.T, P.E, w);
        if (!ok) break;
        out.push_back(w);
    }
    return out;
}

}  // namespace

int attn_absorber(const sanic_program_desc* d, int si) {
    if (si >= d->n_stages || d->stages[si].kind != SANIC_STAGE_POINTWISE) return -1;
    int ai = si + 1;
    while (ai < d->n_stages && d->stages[ai].kind == SANIC_STAGE_POINTWISE && d->stages[ai].where >= 0) ai++;
    if (ai >= d->n_stages || ai - si > 2) return -1;
    AttnPlan P;
    if (!attn_plan(d, ai, P)) return -1;
    for (auto& w : absorbed_writes(d, ai, P))
        if (w.stage == si) return ai;
    return -1;
}

bool lower_attn_decode(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    AttnPlan P;
    if (!attn_plan(d, si, P)) return false;
    const sanic_stage& st = d->stages[si];
    const sanic_carrier& c = st.carrier;
    const int REP = P.rep;
    const int64_t HD = P.dot.depth, E = P.E, T = P.T, NH = P.NH;
    const int64_t NG = NH / REP;
    const int NS = (int)P.scalar_slots.size(), NV = (int)P.vec_slots.size();
    const int PSZ = 1 + NS + NV * (int)E;         // floats per (chunk, head) partial
    // stream positions per workgroup: 128 (measured best at ~2k positions against 64 and 256),
    // doubled until one group's partials fit the merging workgroup's LDS
    // threads per workgroup: 512 (8 waves, two per SIMD, so the dependent LDS/shuffle phases of
    // one wave hide behind the other's), over 128-position chunks: measured in the full decode
    // step against 1024 threads × 256 positions (the measured tuner's pick, 3% per step)
    // tiling variants for the measured tuner: (threads, positions per chunk; 0 = the rule below)
    static const int kVariants[][2] = {{512, 0}, {1024, 0}, {1024, 512}, {512, 256}, {256, 0}, {256, 128}, {512, 512}};   // positions a multiple of NT/4
    const int nvar = (int)(sizeof kVariants / sizeof *kVariants);
    const int var = st.sched.variant >= 0 && st.sched.variant < nvar ? st.sched.variant : 0;
    int NT = kVariants[var][0];
    // long caches: 1024 threads × 256 positions keeps the chunk count near 16 (C3 at 4096
    // positions: 8.9 µs against 9.6 µs for 512 × 128)
    if (var == 0 && T >= 3072) NT = 1024;
    const int NW = NT / 64;
    int CH = kVariants[var][1] ? kVariants[var][1] : NT / 4;
    while (CH < 1024 && ((T + CH - 1) / CH) * REP * PSZ * 4 > 40 * 1024) CH *= 2;
    const int64_t NCH = (T + CH - 1) / CH;
    const std::vector<RowWrite> writes = absorbed_writes(d, si, P);
    bool wk = false, wvv = false;
    for (auto& w : writes) (w.is_k ? wk : wvv) = true;
    if (wvv && !(P.vacc.dtype == SANIC_BF16)) return false;
    // Separate row writer: when this step's K row and V column are absorbed at the same
    // position, one extra workgroup per KV group (chunk index NCH) computes and stores them and
    // contributes that single position as its own partial carrier (m = its score, ℓ = 1, o = its
    // value row); the regular chunks leave the position out. No regular chunk then waits on the
    // row's loads and RoPE arithmetic, which otherwise put the chunk holding the row last.
    bool sep = wk && wvv;
    if (sep) {
        std::string rp[2];
        for (int i = 0; i < 2; i++) {
            Renderer R2(d);
            Code c2;
            const sanic_node& pn = d->nodes[writes[i].pos];
            rp[i] = R2.value(c2, writes[i].pos, std::vector<std::string>(pn.rank, "0"));
            rp[i] = c2.str() + "|" + rp[i];
        }
        sep = rp[0] == rp[1];
    }
    const int64_t NPART = NCH + (sep ? 1 : 0);   // partial carriers per KV group
    // scratch offsets in the source are relative to this stage's base (passed as the argument),
    // so the same stage in every layer renders to the same source
    const int64_t sbase = scratch;
    const int64_t part_off = 0;
    scratch += ((NPART * NH * PSZ * 4 + 255) / 256) * 256;
    Renderer R(d);
    Code k;
    k.indent = 1;
    k.line("__shared__ __attribute__((aligned(16))) float q_lds[" + std::to_string(REP * HD) + "];");
    if (wk) k.line("__shared__ float knew_lds[" + std::to_string(HD) + "];");
    if (wvv) k.line("__shared__ float vnew_lds[" + std::to_string(E) + "];");
    k.line("__shared__ __attribute__((aligned(16))) float p_lds[" + std::to_string(REP) + "][" + std::to_string(CH) + "];");
    k.line("__shared__ float stat_lds[" + std::to_string(REP) + "][2];");
    k.line("__shared__ float o_lds[" + std::to_string(NW) + "][" + std::to_string(REP) + "][" + std::to_string(E) + "];");
    k.line("const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;");
    k.line("const idx_t grp = blockIdx.x, chunk = blockIdx.y;");
    // honest window (per first head of the group; bounds not depending on the head)
    auto win = honest_window(d, st);
    k.line("idx_t lo0 = 0, hi0 = " + std::to_string(T) + ";");
    {
        Code wc;
        wc.indent = 1;
        R.memo.emplace_back();
        // evaluate window edges with grid coords g* = first head of the group, e = 0
        for (int j = 0; j < st.rank; j++)
            wc.line("const idx_t g" + std::to_string(j) + " = " + (j == P.hdim ? "grp * " + std::to_string(REP) : std::string("0")) + ";");
        emit_window(R, wc, st, win, "wlo", "whi");
        wc.line("lo0 = wlo; hi0 = whi;");
        R.memo.pop_back();
        k.line("{");
        k.s << wc.str();
        k.line("}");
    }
    k.line("const idx_t t0 = lo0 + chunk * " + std::to_string(CH) + ";");
    k.line("float* part = a.scratch + " + std::to_string(part_off / 4) + " + (chunk * " + std::to_string(NH) + " + grp * " + std::to_string(REP) + ") * " + std::to_string(PSZ) + ";");
    // ── prefetch: every K row and V run of this chunk is requested before any compute. When the
    // window has no lower edge (causal / decode prefix) the chunk's rows do not depend on the
    // position, so the requests go out before the position load returns; addresses are clamped
    // to the cache capacity and every use below still tests the window.
    bool lo_static = true;
    for (auto& b : win) lo_static &= b.kind != WindowBound::LO_CEIL;
    const std::string tpre = lo_static ? "((idx_t)chunk * " + std::to_string(CH) + ")" : "t0";
    constexpr int LPT = 4;                               // lanes per key position
    const int64_t DPL = HD / LPT;                        // contiguous d per lane (multiple of 8)
    const int PPP = NT / LPT;                            // key positions per score pass
    const int NP = CH / PPP;                             // score passes
    const int PG = CH / NW;                              // value phase: positions per wave group
    const int NSB = PG / 16;                             // 16-position runs per value group
    int repk; int64_t kt, kd, kh;
    addr_parts(P.dot.kacc.addr, repk, NH, kt, kd, kh);
    int repv; int64_t vt, ve, vh;
    addr_parts(P.vacc.addr, repv, NH, vt, ve, vh);
    const bool vfast = vt == 1 && E <= 64;
    k.line("const unsigned short* __restrict__ kp = " + R.param(P.dot.kacc.buffer) + " + " + std::to_string(P.dot.kacc.addr.c0) +
           " + grp * " + std::to_string(kh) + ";");
    k.line("const unsigned short* __restrict__ vp = " + R.param(P.vacc.buffer) + " + " + std::to_string(P.vacc.addr.c0) +
           " + grp * " + std::to_string(vh) + ";");
    k.line("const int sub = tid % " + std::to_string(LPT) + ";");
    auto emit_writes = [&](bool force) {
    // absorbed row writes: the workgroup whose chunk holds the row (chunk 0 when the row is
    // outside the window) computes and stores this group's row elements
    for (auto& w : writes) {
        const sanic_stage& wst = d->stages[w.stage];
        const std::string nm = w.is_k ? "k" : "v";
        const int64_t X = w.is_k ? HD : E;
        const Sym& addr = w.is_k ? P.dot.kacc.addr : P.vacc.addr;
        R.memo.emplace_back();
        const sanic_node& pn = d->nodes[w.pos];
        std::string pv = R.value(k, w.pos, std::vector<std::string>(pn.rank, "0"));
        R.memo.pop_back();
        k.line("const float " + nm + "pf = roundf(" + pv + ");");
        k.line("const idx_t " + nm + "row = (" + nm + "pf >= 0.0f && " + nm + "pf < " + std::to_string(T) + ".0f) ? (idx_t)" + nm + "pf : -1;");
        if (force) k.line("const bool " + nm + "writer = " + nm + "row >= 0;");
        else k.line("const bool " + nm + "writer = " + nm + "row >= 0 && chunk == ((" + nm + "row >= lo0 && " + nm + "row < hi0) ? (" + nm + "row - lo0) / " +
               std::to_string(CH) + " : 0);");
        k.line("if (" + nm + "writer) {");
        k.indent++;
        k.line("for (int xw = tid; xw < " + std::to_string(X) + "; xw += " + std::to_string(NT) + ") {");
        k.indent++;
        k.line("const idx_t wf = " + addr.render({"(grp * " + std::to_string(REP) + ")", nm + "row", "xw"}) + ";");
        std::vector<std::string> wc;
        for (size_t j = 0; j < w.shape.size(); j++) {
            k.line("const idx_t w" + nm + std::to_string(j) + " = (wf / " + std::to_string(w.stride[j]) + ") % " + std::to_string(w.shape[j]) + ";");
            wc.push_back("w" + nm + std::to_string(j));
        }
        R.memo.emplace_back();
        std::string cond = R.value(k, wst.where, wc);
        std::string val = R.value(k, wst.value, wc);
        R.memo.pop_back();
        k.line("float " + nm + "val = " + val + ";");
        k.line("if (" + cond + " != 0.0f) {");
        k.line("  " + store_stmt(R.param(w.buffer), "wf", d->buffers[w.buffer].dtype, nm + "val", false, d->buffers[w.buffer].scale));
        if (d->buffers[w.buffer].dtype == SANIC_BF16) k.line("  " + nm + "val = __uint_as_float((unsigned)sanic_to_bf16(" + nm + "val) << 16);");
        k.line("} else {");
        k.line("  " + nm + "val = " + (w.is_k ? std::string("sanic_bf16(kp[") + nm + "row * " + std::to_string(kt) + " + xw])"
                                                  : std::string("sanic_bf16(vp[xw * ") + std::to_string(ve) + " + " + nm + "row * " + std::to_string(vt) + "])") + ";");
        k.line("}");
        k.line(nm + "new_lds[xw] = " + nm + "val;");
        k.indent--;
        k.line("}");
        k.indent--;
        k.line("}");
    }
    };
    // query vectors (the A side, rendered) into LDS. With one element per thread the rendered
    // code is split: index arithmetic and plain buffer loads go out ahead of the K/V prefetch
    // (loads complete in issue order, so a q load issued after the prefetch would wait for all of
    // it), the arithmetic (RoPE, with its branchy sin/cos) runs after the prefetch is issued.
    std::string q_post;
    auto emit_q = [&]() {
        if (REP * HD != 256) {
            k.line("for (int i = tid; i < " + std::to_string(REP * HD) + "; i += " + std::to_string(NT) + ") {");
            k.indent++;
            k.line("const idx_t hq = grp * " + std::to_string(REP) + " + i / " + std::to_string(HD) + ";");
            k.line("const idx_t dd = i % " + std::to_string(HD) + ";");
            R.memo.emplace_back();
            std::string v = R.value(k, P.dot.a, P.dot.a_coords);
            R.memo.pop_back();
            k.line("q_lds[i] = " + v + ";");
            k.indent--;
            k.line("}");
            return;
        }
        k.line("const int qt = tid & 255;");
        k.line("const idx_t hq = grp * " + std::to_string(REP) + " + qt / " + std::to_string(HD) + ";");
        k.line("const idx_t dd = qt % " + std::to_string(HD) + ";");
        Code tmp;
        tmp.indent = 0;
        R.memo.emplace_back();
        std::string v = R.value(tmp, P.dot.a, P.dot.a_coords);
        R.memo.pop_back();
        std::set<std::string> known = {"hq", "dd", "qt", "grp", "tid", "lane", "wv", "chunk"};
        std::istringstream in(tmp.str());
        std::string ln, post;
        static const std::regex decl(R"(^\s*const (idx_t|int|float) (\w+) = (.*);\s*$)");
        static const std::regex load(R"(^a\.b\d+\[\(idx_t\)\((\w+)\)\]$)");
        static const std::regex ident(R"([A-Za-z_]\w*)");
        static const std::regex call(R"([A-Za-z_]\w*\s*\()");
        while (std::getline(in, ln)) {
            std::smatch m;
            bool hoist = false;
            if (std::regex_match(ln, m, decl)) {
                const std::string ty = m[1], name = m[2], rhs = m[3];
                bool ok = ty != "float" || std::regex_match(rhs, load);
                std::string r2 = std::regex_replace(rhs, std::regex(R"(a\.b\d+)"), " ");
                ok = ok && !std::regex_search(r2, call);
                for (auto it = std::sregex_iterator(r2.begin(), r2.end(), ident); ok && it != std::sregex_iterator(); ++it) {
                    const std::string id = it->str();
                    if (id == "idx_t" || id == "float" || id == "int") continue;
                    if (!known.count(id) && !(id.size() > 2 && id[0] == 's' && id[1] == 'c' && isdigit((unsigned char)id[2]))) ok = false;
                }
                if (ok) {
                    hoist = true;
                    known.insert(name);
                }
            }
            if (hoist) k.line(ln.substr(ln.find_first_not_of(' ')));
            else post += "  " + ln + "\n";
        }
        q_post = post + (NT > 256 ? "  if (tid < 256) q_lds[qt] = " : "  q_lds[qt] = ") + v + ";\n";
    };
    emit_q();
    k.line("sanic_u32x4 kq[" + std::to_string(NP) + "][" + std::to_string(DPL / 8) + "];");
    if (vfast) k.line("sanic_u32x4 vq[" + std::to_string(NSB) + "][2];");
    k.line("const int e_ = tid % 64, tg = tid / 64;");   // value phase: lane = value dim, 4 groups of CH/4 positions
    k.line("#pragma unroll");
    k.line("for (int ps = 0; ps < " + std::to_string(NP) + "; ++ps) {");
    k.line("  const idx_t t = " + tpre + " + ps * " + std::to_string(PPP) + " + tid / " + std::to_string(LPT) + ";");
    k.line("  const idx_t tt = t < " + std::to_string(T) + " ? t : 0;");
    k.line("  #pragma unroll");
    k.line("  for (int v8 = 0; v8 < " + std::to_string(DPL / 8) + "; ++v8)");
    k.line("    kq[ps][v8] = *(const sanic_u32x4*)(kp + tt * " + std::to_string(kt) + " + sub * " + std::to_string(DPL) + " + v8 * 8);");
    k.line("}");
    if (vfast) {
        k.line("#pragma unroll");
        k.line("for (int sb = 0; sb < " + std::to_string(NSB) + "; ++sb) {");
        k.line("  const idx_t tb = " + tpre + " + tg * " + std::to_string(PG) + " + sb * 16;");
        k.line("  const bool full = tb + 16 <= " + std::to_string(T) + " && e_ < " + std::to_string(E) + ";");
        k.line("  const unsigned short* src = vp + (full ? (idx_t)e_ * " + std::to_string(ve) + " + tb : 0);");
        k.line("  vq[sb][0] = *(const sanic_u32x4*)(src);");
        k.line("  vq[sb][1] = *(const sanic_u32x4*)(src + 8);");
        k.line("}");
    }
    if (!q_post.empty()) { k.line("{"); k.s << q_post; k.line("}"); }
    if (sep) {
        k.line("if (chunk == " + std::to_string(NCH) + ") {");
        k.indent++;
            emit_writes(true);
        k.line("__syncthreads();");
        k.line("const bool nvis = krow >= 0 && krow >= lo0 && krow < hi0;");
        for (int r = 0; r < REP; r++) {
            // score of head grp·REP + r at the new row (wave r % 4), the leaf with its contraction substituted
            k.line("if (wv == " + std::to_string(r % NW) + ") {");
            k.indent++;
            k.line("float dv = 0.0f;");
            k.line("for (int dd = lane; dd < " + std::to_string(HD) + "; dd += 64) dv = fmaf(q_lds[" + std::to_string(r * HD) + " + dd], knew_lds[dd], dv);");
            k.line("dv = sanic_wave_sum(dv);");
            k.line("if (lane == 0) {");
            k.indent++;
            k.line("const float dotv = dv;");
            k.line("const idx_t s = krow < 0 ? 0 : krow;");
            R.memo.emplace_back();
            R.subst[P.dot.reduce] = "dotv";
            const sanic_node& sl = d->nodes[st.leaf[P.sleaf]];
            std::vector<std::string> lc(sl.rank);
            for (int j = 0; j < sl.rank; j++) {
                int bd = st.bind[P.sleaf][j];
                lc[j] = bd == SANIC_BIND_STREAM ? "s" : bd == P.hdim ? "(grp * " + std::to_string(REP) + " + " + std::to_string(r) + ")" : "0";
            }
            std::string v = R.value(k, st.leaf[P.sleaf], lc);
            R.subst.clear();
            R.memo.pop_back();
            k.line("stat_lds[" + std::to_string(r) + "][0] = nvis ? " + v + " : (-__builtin_huge_valf());");
            k.indent--;
            k.line("}");
            k.indent--;
            k.line("}");
        }
        k.line("__syncthreads();");
        // the one-position partial: m = score, scalar slots into·1, vector slots the value row
        k.line("for (int i = tid; i < " + std::to_string(REP * PSZ) + "; i += " + std::to_string(NT) + ") {");
        k.indent++;
        k.line("const int r = i / " + std::to_string(PSZ) + ", f = i % " + std::to_string(PSZ) + ";");
        k.line("const float m = stat_lds[r][0];");
        k.line("const bool live = (-__builtin_huge_valf()) < m;");
        k.line("float v;");
        k.line("if (f == 0) v = m;");
        for (int sidx = 0; sidx < NS; sidx++)
            k.line("else if (f == " + std::to_string(1 + sidx) + ") v = live ? " + flit(P.scalar_into[sidx]) + " : 0.0f;");
        k.line("else v = live ? vnew_lds[(f - " + std::to_string(1 + NS) + ") % " + std::to_string(E) + "] : 0.0f;");
        k.line("sanic_st(part + r * " + std::to_string(PSZ) + " + f, v);");
        k.indent--;
        k.line("}");
        k.indent--;
        k.line("} else");
    }
    // identity partial for chunks past the visible window
    k.line("if (t0 >= hi0) {");
    k.line("  for (int i = tid; i < " + std::to_string(REP * PSZ) + "; i += " + std::to_string(NT) + ") {");
    k.line("    const int r = i / " + std::to_string(PSZ) + ", f = i % " + std::to_string(PSZ) + ";");
    k.line("    sanic_st(part + r * " + std::to_string(PSZ) + " + f, f == 0 ? " + flit(c.identity[P.max_slot]) + " : 0.0f);");
    k.line("  }");
    k.line("} else {");
    k.line("const idx_t t1 = t0 + " + std::to_string(CH) + " < hi0 ? t0 + " + std::to_string(CH) + " : hi0;");
    if (sep) {
        // the new row's position: excluded here, folded by the writer workgroup
        R.memo.emplace_back();
        const sanic_node& pn = d->nodes[writes[0].pos];
        std::string pv = R.value(k, writes[0].pos, std::vector<std::string>(pn.rank, "0"));
        R.memo.pop_back();
        k.line("const float npf = roundf(" + pv + ");");
        k.line("const idx_t nrow = (npf >= 0.0f && npf < " + std::to_string(T) + ".0f) ? (idx_t)npf : -1;");
    } else {
        emit_writes(false);
    }
    k.line("__syncthreads();");
    // scores
    k.line("#pragma unroll");
    k.line("for (int ps = 0; ps < " + std::to_string(NP) + "; ++ps) {");
    k.indent++;
    k.line("const int tl = ps * " + std::to_string(PPP) + " + tid / " + std::to_string(LPT) + ";");
    k.line("const idx_t t = t0 + tl;");
    k.line("float dot[" + std::to_string(REP) + "];");
    k.line("#pragma unroll");
    k.line("for (int r = 0; r < " + std::to_string(REP) + "; ++r) dot[r] = 0.0f;");
    k.line("#pragma unroll");
    k.line("for (int v8 = 0; v8 < " + std::to_string(DPL / 8) + "; ++v8) {");
    k.indent++;
    k.line("const int d0 = sub * " + std::to_string(DPL) + " + v8 * 8;");
    k.line("const sanic_u32x4 kv = kq[ps][v8];");
    k.line(std::string(wk ? "" : "const ") + "float kf[8] = {__uint_as_float(kv.x << 16), __uint_as_float(kv.x & 0xFFFF0000u), __uint_as_float(kv.y << 16), __uint_as_float(kv.y & 0xFFFF0000u), __uint_as_float(kv.z << 16), __uint_as_float(kv.z & 0xFFFF0000u), __uint_as_float(kv.w << 16), __uint_as_float(kv.w & 0xFFFF0000u)};");
    if (wk && !sep) {
        k.line("if (kwriter && t == krow) {");
        k.line("  #pragma unroll");
        k.line("  for (int j = 0; j < 8; ++j) kf[j] = knew_lds[d0 + j];");
        k.line("}");
    }
    // q as 16-byte LDS reads (d0 is a multiple of 8)
    k.line("#pragma unroll");
    k.line("for (int r = 0; r < " + std::to_string(REP) + "; ++r) {");
    k.line("  const sanic_f32x4 qa = *(const sanic_f32x4*)(&q_lds[r * " + std::to_string(HD) + " + d0]);");
    k.line("  const sanic_f32x4 qb = *(const sanic_f32x4*)(&q_lds[r * " + std::to_string(HD) + " + d0 + 4]);");
    k.line("  dot[r] = fmaf(qa.x, kf[0], fmaf(qa.y, kf[1], fmaf(qa.z, kf[2], fmaf(qa.w, kf[3], dot[r]))));");
    k.line("  dot[r] = fmaf(qb.x, kf[4], fmaf(qb.y, kf[5], fmaf(qb.z, kf[6], fmaf(qb.w, kf[7], dot[r]))));");
    k.line("}");
    k.indent--;
    k.line("}");
    k.line("#pragma unroll");
    k.line("for (int r = 0; r < " + std::to_string(REP) + "; ++r) {");
    static_assert(LPT == 4, "the score reduction is a quad sum");
    k.line("  dot[r] = sanic_quad_sum(dot[r]);");
    k.line("}");
    k.line("if (sub == 0) {");
    k.indent++;
    k.line("const idx_t s = t;");
    for (int r = 0; r < REP; r++) {
        // the score at (h = grp·REP + r, t): the leaf with its contraction substituted
        k.line("{");
        k.indent++;
        k.line("const float dotv = dot[" + std::to_string(r) + "];");
        R.memo.emplace_back();
        R.subst[P.dot.reduce] = "dotv";
        const sanic_node& sl = d->nodes[st.leaf[P.sleaf]];
        std::vector<std::string> lc(sl.rank);
        for (int j = 0; j < sl.rank; j++) {
            int bd = st.bind[P.sleaf][j];
            lc[j] = bd == SANIC_BIND_STREAM ? "s" : bd == P.hdim ? "(grp * " + std::to_string(REP) + " + " + std::to_string(r) + ")" : "0";
        }
        std::string v = R.value(k, st.leaf[P.sleaf], lc);
        R.subst.clear();
        R.memo.pop_back();
        k.line("p_lds[" + std::to_string(r) + "][tl] = " + std::string(sep ? "t < t1 && t != nrow" : "t < t1") + " ? " + v + " : (-__builtin_huge_valf());");
        k.indent--;
        k.line("}");
    }
    k.indent--;
    k.line("}");
    k.indent--;
    k.line("}");
    k.line("__syncthreads();");
    // per head: max, p = exp(s − m) (0 when m = −∞), Σ p
    k.line("for (int r = wv; r < " + std::to_string(REP) + "; r += " + std::to_string(NW) + ") {");
    k.indent++;
    k.line("float m = (-__builtin_huge_valf());");
    k.line("for (int i = lane; i < " + std::to_string(CH) + "; i += 64) m = fmaxf(m, p_lds[r][i]);");
    k.line("m = sanic_wave_max(m);");
    k.line("float l = 0.0f;");
    k.line("for (int i = lane; i < " + std::to_string(CH) + "; i += 64) {");
    k.line("  const float p = m == (-__builtin_huge_valf()) ? 0.0f : __builtin_amdgcn_exp2f((p_lds[r][i] - m) * 1.44269504088896341f);");
    k.line("  p_lds[r][i] = p;");
    k.line("  l += p;");
    k.line("}");
    k.line("l = sanic_wave_sum(l);");
    k.line("if (lane == 0) { stat_lds[r][0] = m; stat_lds[r][1] = l; }");
    k.indent--;
    k.line("}");
    k.line("__syncthreads();");
    // o[r][e] = Σ_t p[r][t] · V(h, t, e)
    k.line("for (int e = e_; e < " + std::to_string(E) + "; e += 64) {");
    k.indent++;
    k.line("float o[" + std::to_string(REP) + "];");
    k.line("#pragma unroll");
    k.line("for (int r = 0; r < " + std::to_string(REP) + "; ++r) o[r] = 0.0f;");
    k.line("#pragma unroll");
    k.line("for (int sb = 0; sb < " + std::to_string(NSB) + "; ++sb) {");
    k.indent++;
    k.line("const int tbase = tg * " + std::to_string(PG) + " + sb * 16;");
    if (vfast) {
        // the prefetched run covers the block whenever it lies inside the cache; positions past
        // the window contribute nothing (their value is masked to 0 and their probability is 0)
        k.line("if (t0 + tbase + 16 <= " + std::to_string(T) + ") {");
        if (sep) k.line("  const bool partial = t0 + tbase + 16 > t1 || (nrow >= t0 + tbase && nrow < t0 + tbase + 16);");
        else k.line("  const bool partial = t0 + tbase + 16 > t1;");
        k.line("  const unsigned vw[8] = {vq[sb][0].x, vq[sb][0].y, vq[sb][0].z, vq[sb][0].w, vq[sb][1].x, vq[sb][1].y, vq[sb][1].z, vq[sb][1].w};");
        // this run's probabilities as 16-byte LDS reads (tbase is a multiple of 16)
        k.line("  float pr[" + std::to_string(REP) + "][16];");
        k.line("  #pragma unroll");
        k.line("  for (int r = 0; r < " + std::to_string(REP) + "; ++r)");
        k.line("    #pragma unroll");
        k.line("    for (int q4 = 0; q4 < 4; ++q4) {");
        k.line("      const sanic_f32x4 pv4 = *(const sanic_f32x4*)(&p_lds[r][tbase + q4 * 4]);");
        k.line("      pr[r][q4 * 4] = pv4.x; pr[r][q4 * 4 + 1] = pv4.y; pr[r][q4 * 4 + 2] = pv4.z; pr[r][q4 * 4 + 3] = pv4.w;");
        k.line("    }");
        k.line("  #pragma unroll");
        k.line("  for (int j = 0; j < 16; ++j) {");
        k.line("    float vf = __uint_as_float((j & 1) ? (vw[j >> 1] & 0xFFFF0000u) : (vw[j >> 1] << 16));");
        if (wvv && !sep) k.line("    if (vwriter && t0 + tbase + j == vrow) vf = vnew_lds[e];");
        if (sep) k.line("    if (partial && (t0 + tbase + j >= t1 || t0 + tbase + j == nrow)) vf = 0.0f;");
        else k.line("    if (partial && t0 + tbase + j >= t1) vf = 0.0f;");
        k.line("    #pragma unroll");
        k.line("    for (int r = 0; r < " + std::to_string(REP) + "; ++r) o[r] = fmaf(pr[r][j], vf, o[r]);");
        k.line("  }");
        k.line("} else {");
        k.line("  for (int j = 0; j < 16; ++j) {");
        k.line("    const idx_t t = t0 + tbase + j;");
        k.line(std::string("    if (t < t1") + (sep ? " && t != nrow" : "") + ") {");
        k.line(std::string("      ") + (wvv ? "" : "const ") + "float vf = sanic_bf16(vp[e * " + std::to_string(ve) + " + t]);");
        if (wvv && !sep) k.line("      if (vwriter && t == vrow) vf = vnew_lds[e];");
        k.line("      for (int r = 0; r < " + std::to_string(REP) + "; ++r) o[r] = fmaf(p_lds[r][tbase + j], vf, o[r]);");
        k.line("    }");
        k.line("  }");
        k.line("}");
    } else {
        k.line("for (int j = 0; j < 16; ++j) {");
        k.line("  const idx_t t = t0 + tbase + j;");
        k.line(std::string("  if (t < t1") + (sep ? " && t != nrow" : "") + ") {");
        k.line(std::string("    ") + (wvv ? "" : "const ") + "float vf = sanic_bf16(vp[e * " + std::to_string(ve) + " + t * " + std::to_string(vt) + "]);");
        if (wvv && !sep) k.line("    if (vwriter && t == vrow) vf = vnew_lds[e];");
        k.line("    for (int r = 0; r < " + std::to_string(REP) + "; ++r) o[r] = fmaf(p_lds[r][tbase + j], vf, o[r]);");
        k.line("  }");
        k.line("}");
    }
    k.indent--;
    k.line("}");
    k.line("#pragma unroll");
    k.line("for (int r = 0; r < " + std::to_string(REP) + "; ++r) o_lds[tg][r][e] = o[r];");
    k.indent--;
    k.line("}");
    k.line("__syncthreads();");
    // write the partial carriers: [m, scalar slots (into·ℓ), vector slots (o)]
    k.line("for (int i = tid; i < " + std::to_string(REP * PSZ) + "; i += " + std::to_string(NT) + ") {");
    k.indent++;
    k.line("const int r = i / " + std::to_string(PSZ) + ", f = i % " + std::to_string(PSZ) + ";");
    k.line("float v;");
    k.line("if (f == 0) v = stat_lds[r][0];");
    for (int s = 0; s < NS; s++)
        k.line("else if (f == " + std::to_string(1 + s) + ") v = " + flit(P.scalar_into[s]) + " * stat_lds[r][1];");
    k.line("else { const int e = (f - " + std::to_string(1 + NS) + ") % " + std::to_string(E) + "; v = o_lds[0][r][e]; for (int g = 1; g < " + std::to_string(NW) + "; ++g) v += o_lds[g][r][e]; }");
    k.line("sanic_st(part + r * " + std::to_string(PSZ) + " + f, v);");
    k.indent--;
    k.line("}");

    k.line("}  // visible chunk");
    // Merge, fused: the last workgroup of this KV group to finish stages the group's partials in
    // LDS and merges them in one n-way step of the ExpShifted combine (derive.rs:1688-1747
    // applied to all chunks at once): M = max_c m_c, w_c = [−∞ < m_c]·exp(m_c − M), every
    // ExpShifted slot = Σ_c w_c·x_c. This is the pairwise combine of run_carrier_split
    // (interp.rs:555-643) regrouped — no chain of NCH dependent steps.
    const int64_t counter_off = scratch - sbase;
    scratch += ((NG * 4 + 255) / 256) * 256;
    const int64_t GP = NPART * REP * PSZ;       // floats of one group's partials
    if (GP * 4 > 64 * 1024) return false;
    k.line("{");
    k.indent++;
    k.line("unsigned* cnt = (unsigned*)((char*)a.scratch + " + std::to_string(counter_off) + ") + grp;");
    emit_arrival(k, "sanic_last", "tid", "cnt", std::to_string(NPART) + "u");
    k.line("if (!sanic_last) return;");
    k.line("__shared__ __attribute__((aligned(16))) float g_lds[" + std::to_string(GP) + "];");
    k.line("__shared__ float w_lds[" + std::to_string(REP) + "][" + std::to_string(NPART) + "];");
    k.line("__shared__ float mx_lds[" + std::to_string(REP) + "];");
    // every coherent load is issued before the first is consumed (one round trip, not GP/256):
    // 16-byte loads when a chunk's group partials are 16-byte aligned runs
    if ((REP * PSZ) % 4 == 0 && (NH * PSZ) % 4 == 0 && part_off % 16 == 0) {
        const int64_t Q4 = REP * PSZ / 4;                     // float4 per chunk
        const int64_t PER = (NPART * Q4 + NT - 1) / NT;
        k.line("const float* gbase = a.scratch + " + std::to_string(part_off / 4) + " + grp * " + std::to_string(REP * PSZ) + ";");
        k.line("sanic_f32x4 gv[" + std::to_string(PER) + "];");
        k.line("#pragma unroll");
        k.line("for (int j = 0; j < " + std::to_string(PER) + "; ++j) {");
        k.line("  const int i = tid + j * " + std::to_string(NT) + ";");
        k.line("  const int ch = i / " + std::to_string(Q4) + ", w = i % " + std::to_string(Q4) + ";");
        k.line("  gv[j] = sanic_ld4(gbase, (unsigned)((i < " + std::to_string(NPART * Q4) + " ? ch * " + std::to_string(NH * PSZ) + " + w * 4 : 0) * 4));");
        k.line("}");
        k.line("#pragma unroll");
        k.line("for (int j = 0; j < " + std::to_string(PER) + "; ++j)");
        k.line("  if (tid + j * " + std::to_string(NT) + " < " + std::to_string(NPART * Q4) + ") *(sanic_f32x4*)(g_lds + (tid + j * " + std::to_string(NT) + ") * 4) = gv[j];");
    } else {
        const int64_t PER = (GP + NT - 1) / NT;
        k.line("float gv[" + std::to_string(PER) + "];");
        k.line("#pragma unroll");
        k.line("for (int j = 0; j < " + std::to_string(PER) + "; ++j) {");
        k.line("  const int i = tid + j * " + std::to_string(NT) + ";");
        k.line("  const int ch = i / " + std::to_string(REP * PSZ) + ", rem = i % " + std::to_string(REP * PSZ) + ";");
        k.line("  gv[j] = i < " + std::to_string(GP) + " ? sanic_ld(a.scratch + " + std::to_string(part_off / 4) + " + (ch * " + std::to_string(NH) + " + grp * " +
               std::to_string(REP) + ") * " + std::to_string(PSZ) + " + rem) : 0.0f;");
        k.line("}");
        k.line("#pragma unroll");
        k.line("for (int j = 0; j < " + std::to_string(PER) + "; ++j)");
        k.line("  if (tid + j * " + std::to_string(NT) + " < " + std::to_string(GP) + ") g_lds[tid + j * " + std::to_string(NT) + "] = gv[j];");
    }
    k.line("__syncthreads();");
    k.line("if (tid == 0) sanic_st(cnt, 0u);");
    // per head (one wave each): M and the chunk weights
    k.line("for (int r = wv; r < " + std::to_string(REP) + "; r += " + std::to_string(NW) + ") {");
    k.indent++;
    k.line("float m = (-__builtin_huge_valf());");
    k.line("for (int ch = lane; ch < " + std::to_string(NPART) + "; ch += 64) m = fmaxf(m, g_lds[(ch * " + std::to_string(REP) + " + r) * " + std::to_string(PSZ) + "]);");
    k.line("m = sanic_wave_max(m);");
    k.line("for (int ch = lane; ch < " + std::to_string(NPART) + "; ch += 64) {");
    k.line("  const float mc = g_lds[(ch * " + std::to_string(REP) + " + r) * " + std::to_string(PSZ) + "];");
    k.line("  w_lds[r][ch] = (-__builtin_huge_valf()) < mc ? __builtin_amdgcn_exp2f((mc - m) * 1.44269504088896341f) : 0.0f;");
    k.line("}");
    k.line("if (lane == 0) mx_lds[r] = m;");
    k.indent--;
    k.line("}");
    k.line("__syncthreads();");
    k.line("for (int pt = tid; pt < " + std::to_string(REP * E) + "; pt += " + std::to_string(NT) + ") {");
    k.indent++;
    k.line("const int r = pt / " + std::to_string(E) + ", ee = pt % " + std::to_string(E) + ";");
    for (int j = 0; j < st.rank; j++) {
        std::string v = j == P.hdim ? "(grp * " + std::to_string(REP) + " + r)" : j == P.edim ? "(idx_t)ee" : "0";
        k.line("const idx_t g" + std::to_string(j) + " = " + v + ";");
    }
    std::string lin = "0";
    for (int j = 0; j < st.rank; j++)
        lin = j == 0 ? "g0" : "(" + lin + " * " + std::to_string(st.grid[j]) + " + g" + std::to_string(j) + ")";
    k.line("const idx_t gid = " + lin + ";");
    auto field = [&](int slot) -> std::string {
        for (int sidx = 0; sidx < NS; sidx++) if (P.scalar_slots[sidx] == slot) return std::to_string(1 + sidx);
        for (int v = 0; v < NV; v++) if (P.vec_slots[v] == slot) return std::to_string(1 + NS + v * E) + " + ee";
        return "0";
    };
    for (int sidx = 0; sidx < c.slots; sidx++) {
        std::string ss = std::to_string(sidx);
        if (sidx == P.max_slot) { k.line("const float acc" + ss + " = mx_lds[r];"); continue; }
        k.line("float acc" + ss + " = 0.0f;");
    }
    k.line("for (int ch = 0; ch < " + std::to_string(NPART) + "; ++ch) {");
    k.line("  const float wc = w_lds[r][ch];");
    k.line("  const float* pc = g_lds + (ch * " + std::to_string(REP) + " + r) * " + std::to_string(PSZ) + ";");
    for (int sidx = 0; sidx < c.slots; sidx++) {
        if (sidx == P.max_slot) continue;
        std::string ss = std::to_string(sidx);
        k.line("  acc" + ss + " = fmaf(wc, pc[" + field(sidx) + "], acc" + ss + ");");
    }
    k.line("}");
    R.memo.emplace_back();
    std::string f = R.expr(k, c.project, "", "", "", "acc");
    k.line("const float fold_v = " + f + ";");
    std::string v = "fold_v";
    if (st.epilogue >= 0) {
        std::vector<std::string> gc;
        for (int j = 0; j < st.rank; j++) gc.push_back("g" + std::to_string(j));
        R.fold_var = "fold_v";
        v = R.value(k, st.epilogue, gc);
    }
    R.memo.pop_back();
    k.line(store_stmt(R.param(st.out_buffer), "gid", st.out_dtype, v, false, d->buffers[st.out_buffer].scale));
    k.indent--;
    k.line("}");
    k.indent--;
    k.line("}");

    const std::string tag = "h" + std::to_string(NH) + "_t" + std::to_string(T);
    const std::string kpart = "sanic_attn_decode_" + tag;
    std::ostringstream src;
    src << kPrelude << R.args_struct({"float* __restrict__ scratch"});
    src << "extern \"C\" __global__ void __launch_bounds__(" << NT << ") " << kpart << "(Args a) {\n" << R.entry() << k.str() << "}\n";
    out.kernel_kind = "skeleton:attn_decode[rep " + std::to_string(REP) + "]" + (writes.empty() ? "" : "+writes" + std::to_string(writes.size())) + (sep ? "+rowwg" : "");
    // the ILP-maximising machine scheduler: C3 11.2 → 10.75 µs (the default strategy interleaves
    // the chunk's loads with its arithmetic to save registers)
    out.source = "// sched-strategy: iterative-ilp\n" + src.str();
    out.variants = nvar;
    std::vector<Arg> args = R.arg_list();
    args.push_back({Arg::SCRATCH, sbase});
    out.launches.push_back({kpart, "", dim3((unsigned)NG, (unsigned)NPART), dim3((unsigned)NT), 0, args});
    return true;
}

}  // namespace sanic
