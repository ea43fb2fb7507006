// Hand-written CDNA4 skeletons, chosen from the STRUCTURE of a stage's carrier and leaves —
// never from a name (the reference's rule for its emitters, /root/reference/tests/structure.rs:
// 97-200). Each skeleton is a fixed kernel shape written for gfx950 (wave64, 160 KiB LDS per CU,
// 128-bit loads) whose carrier-specific pieces — leaf values, each slot's `into`, the
// `project`, the epilogue and the narrowing store — are rendered from the descriptor and
// spliced in, then compiled through hipRTC.
//
//   gemv      Plain(Add) carriers (dot, norm-fused projection, int4 dequant matvec) with one
//             output axis: lanes stream K in 128-bit runs, row-only slots (Σx²) are folded once
//             per workgroup, per-row partials merge across the wave by shuffles. Consecutive
//             stages with the same row leaves are batched into one launch (q/k/v, gate/up).
//   rowwrite  the in-place `where(at_pos, new, cache)` stage: launched over the cache row only.
#include <algorithm>
#include <cmath>
#include <set>

#include "emit.h"
#include "skeletons.h"

namespace sanic {

// ───────────────────────── symbolic affine access analysis ────────────────────────────────

std::string Sym::render(const std::vector<std::string>& vars) const {
    std::string s = std::to_string(c0);
    for (auto& t : terms) {
        std::string v = "(idx_t)(" + vars[t.var] + ")";
        if (t.div != 1) v = "(" + v + " / " + std::to_string(t.div) + ")";
        if (t.mod != 0) v = "(" + v + " % " + std::to_string(t.mod) + ")";
        s += " + " + std::to_string(t.coef) + " * " + v;
    }
    return "(" + s + ")";
}

Sym Sym::var(int v) {
    Sym s;
    s.terms.push_back({1, v, 1, 0});
    return s;
}

static Sym sym_add(const Sym& a, const Sym& b, int64_t kb) {
    Sym r = a;
    r.c0 += kb * b.c0;
    for (auto t : b.terms) {
        t.coef *= kb;
        bool merged = false;
        for (auto& u : r.terms)
            if (u.var == t.var && u.div == t.div && u.mod == t.mod) {
                u.coef += t.coef;
                merged = true;
            }
        if (!merged) r.terms.push_back(t);
    }
    r.terms.erase(std::remove_if(r.terms.begin(), r.terms.end(), [](const SymTerm& t) { return t.coef == 0; }),
                  r.terms.end());
    return r;
}

// Interval of a symbolic coordinate given variable extents (for padded reindex proofs).
static void sym_range(const Sym& s, const std::vector<int64_t>& ext, int64_t& lo, int64_t& hi) {
    lo = hi = s.c0;
    for (auto& t : s.terms) {
        int64_t vmax = ext[t.var] - 1;
        int64_t m = vmax / t.div;
        if (t.mod) m = std::min(m, t.mod - 1);
        int64_t span = t.coef * m;
        if (span < 0) lo += span; else hi += span;
    }
}

// Coordinates of a Reindex/View node's source, as Syms; false when not affine.
bool sym_child_coords(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                      const std::vector<int64_t>& ext, std::vector<Sym>& sc) {
    const sanic_node& n = d->nodes[node];
    const sanic_node& s = d->nodes[n.in[0]];
    sc.assign(s.rank, Sym());
    if (n.kind == SANIC_NODE_REINDEX) {
        int64_t p = n.map_offset;
        for (int j = 0; j < s.rank; j++) {
            int64_t nt = d->reindex[p], off = d->reindex[p + 1];
            p += 2;
            Sym v;
            v.c0 = off;
            for (int64_t t = 0; t < nt; t++) {
                int64_t coef = d->reindex[p++], od = d->reindex[p++];
                v = sym_add(v, c[od], coef);
            }
            int64_t lo, hi;
            sym_range(v, ext, lo, hi);
            if (lo < 0 || hi >= s.shape[j]) return false;   // padding would be needed
            sc[j] = v;
        }
        return true;
    }
    if (n.kind == SANIC_NODE_VIEW) {
        int sd = 0;
        for (int j = 0; j < n.rank; j++) {
            int g = n.group[j];
            if (g == 1) {
                sc[sd++] = c[j];
                continue;
            }
            const Sym& cj = c[j];
            if (cj.c0 != 0 || cj.terms.size() != 1 || cj.terms[0].coef != 1) return false;
            SymTerm base = cj.terms[0];
            int64_t inner = 1;
            for (int t = g - 1; t >= 0; t--) {
                int64_t e = s.shape[sd + t];
                SymTerm nt{1, base.var, base.div * inner, 0};
                if (t > 0) {
                    if (base.mod && base.mod % (inner * e)) return false;
                    nt.mod = e;
                } else if (base.mod) {
                    if (base.mod % inner) return false;
                    nt.mod = base.mod / inner;
                }
                Sym v;
                v.terms.push_back(nt);
                sc[sd + t] = v;
                inner *= e;
            }
            sd += g;
        }
        return true;
    }
    return false;
}

bool sym_access(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                const std::vector<int64_t>& ext, Access& out) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_INPUT) {
        Sym addr;
        int64_t stride = 1;
        for (int j = n.rank - 1; j >= 0; j--) {
            addr = sym_add(addr, c[j], stride);
            stride *= n.shape[j];
        }
        out.buffer = n.buffer;
        out.dtype = n.dtype;
        out.addr = addr;
        out.node = node;
        return true;
    }
    if (n.kind == SANIC_NODE_REINDEX || n.kind == SANIC_NODE_VIEW) {
        std::vector<Sym> sc;
        if (!sym_child_coords(d, node, c, ext, sc)) return false;
        return sym_access(d, n.in[0], sc, ext, out);
    }
    return false;
}

// ───────────────────────── Expr structure helpers ─────────────────────────────────────────

static bool expr_reads_item(const sanic_program_desc* d, int e, int item) {
    const sanic_expr& x = d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == item;
    if (x.op >= SANIC_EX_CONST) return false;
    for (int c : {x.a, x.b, x.c})
        if (c >= 0 && expr_reads_item(d, c, item)) return true;
    return false;
}

// `into` is linear in item w through products only: W·rest.
static bool linear_in_product(const sanic_program_desc* d, int e, int w) {
    const sanic_expr& x = d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == w;
    if (x.op == SANIC_OP_MUL) {
        bool a = expr_reads_item(d, x.a, w), b = expr_reads_item(d, x.b, w);
        if (a == b) return false;
        return a ? linear_in_product(d, x.a, w) : linear_in_product(d, x.b, w);
    }
    return false;
}

// Render an Expr where item `w` reads as 1 (the factor `rest` of W·rest).
static std::string expr_without(Renderer& R, Code& code, int e, int w, const std::string& item) {
    const sanic_expr& x = R.d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == w ? "1.0f" : item + std::to_string(x.index);
    if (x.op == SANIC_EX_CONST) return flit(x.value);
    if (x.op >= SANIC_EX_CONST) return R.expr(code, e, item, "", "", "");
    std::string s[3];
    int kids[3] = {x.a, x.b, x.c};
    for (int k = 0; k < 3; k++) if (kids[k] >= 0) s[k] = expr_without(R, code, kids[k], w, item);
    std::string out = R.fresh("e");
    code.line("const float " + out + " = " + map_expr(x.op, s[0], s[1], s[2]) + ";");
    return out;
}

static int64_t vol(const int64_t* s, int r) {
    int64_t v = 1;
    for (int i = 0; i < r; i++) v *= s[i];
    return v;
}

static void collect_inputs(const sanic_program_desc* d, int node, std::set<int>& bufs) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_INPUT) bufs.insert(n.buffer);
    for (int k = 0; k < n.n_in; k++) collect_inputs(d, n.in[k], bufs);
}

// ───────────────────────── vector weight renderer ─────────────────────────────────────────
// Renders the weight leaf W(n, k0 + j), j = 0..7, as 8 f32 expressions. The leaf must be an
// elementwise tree (Map/Const) over affine accesses; each access is loaded once per run of 8:
// a contiguous 128-bit (bf16) / 32-bit (nibbles) / 256-bit (f32) load, a single scalar when
// it does not move with k inside the run (per-group scale / zero point), or 8 scalar loads.

struct VecW {
    const sanic_program_desc* d;
    std::vector<int> bufs;        // access buffers in traversal order -> local pointers wb<i>
    std::vector<int> dtypes;
    int tmp = 0;
    bool ok = true;
    bool contiguous = true;   // every access moves by 0 or 1 element along k
    std::string fresh(const char* p) { return std::string(p) + std::to_string(tmp++); }

    // c: leaf dims as Syms over vars {0: n, 1: k}; "k" is rendered as k0 (a multiple of 8)
    std::vector<std::string> render(Code& code, int node, const std::vector<Sym>& c, const std::vector<int64_t>& ext) {
        const sanic_node& n = d->nodes[node];
        if (n.kind == SANIC_NODE_CONST) return std::vector<std::string>(8, flit(n.value));
        if (n.kind == SANIC_NODE_MAP) {
            std::vector<std::string> a[3];
            for (int k = 0; k < n.n_in; k++) {
                const sanic_node& m = d->nodes[n.in[k]];
                int lead = n.rank - m.rank;
                std::vector<Sym> cc(m.rank);
                for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? Sym() : c[lead + j];
                a[k] = render(code, n.in[k], cc, ext);
                if (!ok) return {};
            }
            std::vector<std::string> out(8);
            for (int j = 0; j < 8; j++) {
                std::string v = fresh("w");
                code.line("const float " + v + " = " + map_expr(n.op, a[0][j], a[1].empty() ? "" : a[1][j], a[2].empty() ? "" : a[2][j]) + ";");
                out[j] = v;
            }
            return out;
        }
        if (n.kind == SANIC_NODE_REINDEX || n.kind == SANIC_NODE_VIEW) {
            std::vector<Sym> sc;
            if (!sym_child_coords(d, node, c, ext, sc)) { ok = false; return {}; }
            return render(code, n.in[0], sc, ext);
        }
        Access acc;
        if (!sym_access(d, node, c, ext, acc)) { ok = false; return {}; }
        int64_t jstride = 0;
        for (auto& t : acc.addr.terms) {
            if (t.var != 1) continue;
            if (t.div == 1 && (t.mod == 0 || t.mod % 8 == 0)) jstride += t.coef;
            else if (t.div % 8 != 0) { ok = false; return {}; }
        }
        if (jstride != 0 && jstride != 1) contiguous = false;
        int slot = (int)bufs.size();
        bufs.push_back(acc.buffer);
        dtypes.push_back(acc.dtype);
        std::string p = "wb" + std::to_string(slot);
        std::string addr = acc.addr.render({"nn", "k0"});
        std::vector<std::string> out(8);
        auto one = [&](const std::string& idx) -> std::string {
            switch (acc.dtype) {
            case SANIC_F32: return p + "[" + idx + "]";
            case SANIC_BF16: return "sanic_bf16(" + p + "[" + idx + "])";
            case SANIC_F16: return "(float)" + p + "[" + idx + "]";
            case SANIC_I4: return "sanic_w4(" + p + ", " + idx + ")";
            case SANIC_U4: return "sanic_u4(" + p + ", " + idx + ")";
            case SANIC_I8: case SANIC_U32: return "(float)" + p + "[" + idx + "]";
            }
            return "0.0f";
        };
        std::string base = fresh("ad");
        code.line("const idx_t " + base + " = " + addr + ";");
        if (jstride == 0) {
            std::string v = fresh("w");
            code.line("const float " + v + " = " + one(base) + ";");
            return std::vector<std::string>(8, v);
        }
        if (jstride == 1 && acc.dtype == SANIC_BF16) {
            std::string v = fresh("wq");
            code.line("const uint4 " + v + " = *(const uint4*)(" + p + " + " + base + ");");
            const char* comp[4] = {"x", "y", "z", "w"};
            for (int j = 0; j < 8; j++)
                out[j] = std::string("__uint_as_float(") + (j % 2 == 0 ? "(" + v + "." + comp[j / 2] + " << 16)"
                                                                        : "(" + v + "." + comp[j / 2] + " & 0xFFFF0000u)") + ")";
            return out;
        }
        if (jstride == 1 && acc.dtype == SANIC_F32) {
            std::string v0 = fresh("f"), v1 = fresh("f");
            code.line("const float4 " + v0 + " = *(const float4*)(" + p + " + " + base + ");");
            code.line("const float4 " + v1 + " = *(const float4*)(" + p + " + " + base + " + 4);");
            const char* comp[4] = {"x", "y", "z", "w"};
            for (int j = 0; j < 8; j++) out[j] = (j < 4 ? v0 : v1) + "." + comp[j % 4];
            return out;
        }
        if (jstride == 1 && (acc.dtype == SANIC_U4 || acc.dtype == SANIC_I4)) {
            std::string v = fresh("u");
            code.line("const unsigned " + v + " = *(const unsigned*)(" + p + " + (" + base + " >> 1));");
            for (int j = 0; j < 8; j++) {
                std::string e = "(float)((" + v + " >> " + std::to_string(4 * j) + ") & 0xFu)";
                out[j] = acc.dtype == SANIC_I4 ? "(" + e + " - 8.0f)" : e;
            }
            return out;
        }
        for (int j = 0; j < 8; j++) {
            std::string v = fresh("w");
            code.line("const float " + v + " = " + one(base + " + " + std::to_string(jstride * j)) + ";");
            out[j] = v;
        }
        return out;
    }
};

// ───────────────────────── gemv ───────────────────────────────────────────────────────────

struct GemvPlan {
    int stage = -1;
    int ndim = -1;         // the one grid dim with extent > 1
    int64_t N = 0, K = 0;
    int w = -1;            // weight leaf index
    std::vector<int> cslots, rslots;
};

static bool gemv_plan(const sanic_program_desc* d, int si, GemvPlan& P) {
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_FUSED) return false;
    const sanic_carrier& c = st.carrier;
    for (int k = 0; k < c.slots; k++)
        if (c.kind[k].kind != SANIC_SLOT_PLAIN || c.kind[k].monoid != SANIC_MON_ADD) return false;
    int ndim = -1;
    for (int j = 0; j < st.rank; j++)
        if (st.grid[j] > 1) {
            if (ndim >= 0) return false;
            ndim = j;
        }
    if (ndim < 0) return false;
    if (st.stream % 8 != 0 || st.stream < 64) return false;
    int w = -1;
    for (int l = 0; l < st.n_leaves; l++) {
        const sanic_node& ln = d->nodes[st.leaf[l]];
        bool has_n = false, has_s = false;
        for (int j = 0; j < ln.rank; j++) {
            has_n |= st.bind[l][j] == ndim;
            has_s |= st.bind[l][j] == SANIC_BIND_STREAM;
        }
        if (has_n && has_s) {
            if (w >= 0) return false;
            w = l;
        } else if (has_n) {
            return false;
        }
    }
    if (w < 0) return false;
    P = GemvPlan();
    P.stage = si;
    P.ndim = ndim;
    P.N = st.grid[ndim];
    P.K = st.stream;
    P.w = w;
    for (int k = 0; k < c.slots; k++) {
        if (!expr_reads_item(d, c.into[k], w)) P.rslots.push_back(k);
        else if (linear_in_product(d, c.into[k], w)) P.cslots.push_back(k);
        else return false;
    }
    if (P.cslots.empty() || P.cslots.size() > 2) return false;
    // the weight leaf must vectorise over runs of 8 along k with row-contiguous access
    const sanic_node& wn = d->nodes[st.leaf[w]];
    std::vector<Sym> cw(wn.rank);
    for (int j = 0; j < wn.rank; j++) {
        int b = st.bind[w][j];
        cw[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == ndim ? Sym::var(0) : Sym();
    }
    VecW vw{d};
    Code scratch;
    vw.render(scratch, st.leaf[w], cw, {P.N, P.K});
    // K-contiguous weights (the reference's [out, in] layout): every access moves by 1 or 0
    // along a run of k; other layouts go to the K-major skeleton or the generic fold
    return vw.ok && vw.contiguous;
}

// Render the pieces of one gemv stage: the row prologue (leaf values and per-k factors), the
// weight vector code, and the finish (project + epilogue + store).
struct GemvParts {
    std::string prologue;      // runs once per k (computes u<c>, adds row slots into racc<r>)
    std::string wvec;          // computes w0..w7 at (nn, k0) from wb<i>
    std::vector<int> wbufs, wdtypes;
    std::vector<std::string> wvals;
};

static GemvParts gemv_parts(Renderer& R, const sanic_program_desc* d, const GemvPlan& P) {
    const sanic_stage& st = d->stages[P.stage];
    const sanic_carrier& c = st.carrier;
    GemvParts out;
    Code pc;
    pc.indent = 2;
    R.memo.emplace_back();
    for (int l = 0; l < st.n_leaves; l++) {
        if (l == P.w) continue;
        const sanic_node& ln = d->nodes[st.leaf[l]];
        std::vector<std::string> lc(ln.rank);
        for (int j = 0; j < ln.rank; j++) lc[j] = st.bind[l][j] == SANIC_BIND_STREAM ? "k" : "0";
        std::string v = R.value(pc, st.leaf[l], lc);
        pc.line("const float x" + std::to_string(l) + " = " + v + ";");
    }
    for (size_t i = 0; i < P.cslots.size(); i++) {
        std::string v = expr_without(R, pc, c.into[P.cslots[i]], P.w, "x");
        pc.line("u_lds[" + std::to_string(i) + " * " + std::to_string(P.K) + " + k] = " + v + ";");
    }
    for (size_t i = 0; i < P.rslots.size(); i++) {
        std::string v = R.expr(pc, c.into[P.rslots[i]], "x", "", "", "");
        pc.line("racc" + std::to_string(i) + " += " + v + ";");
    }
    R.memo.pop_back();
    out.prologue = pc.str();
    const sanic_node& wn = d->nodes[st.leaf[P.w]];
    std::vector<Sym> cw(wn.rank);
    for (int j = 0; j < wn.rank; j++) {
        int b = st.bind[P.w][j];
        cw[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.ndim ? Sym::var(0) : Sym();
    }
    VecW vw{d};
    Code wc;
    wc.indent = 4;
    out.wvals = vw.render(wc, st.leaf[P.w], cw, {P.N, P.K});
    out.wvec = wc.str();
    out.wbufs = vw.bufs;
    out.wdtypes = vw.dtypes;
    return out;
}

static void gemv_finish(Renderer& R, Code& code, const sanic_program_desc* d, const GemvPlan& P) {
    const sanic_stage& st = d->stages[P.stage];
    const sanic_carrier& c = st.carrier;
    // slot values: contraction slots from the wave reduction, row slots from the block
    for (size_t i = 0; i < P.cslots.size(); i++)
        code.line("const float fs" + std::to_string(P.cslots[i]) + " = accq[" + std::to_string(i) + "];");
    for (size_t i = 0; i < P.rslots.size(); i++)
        code.line("const float fs" + std::to_string(P.rslots[i]) + " = racc" + std::to_string(i) + ";");
    std::string f = R.expr(code, c.project, "", "", "", "fs");
    code.line("const float fold_v = " + f + ";");
    std::string v = "fold_v";
    if (st.epilogue >= 0) {
        std::vector<std::string> gc(st.rank, "0");
        gc[P.ndim] = "nn";
        R.fold_var = "fold_v";
        R.memo.emplace_back();
        v = R.value(code, st.epilogue, gc);
        R.memo.pop_back();
    }
    code.line(store_stmt(R.param(st.out_buffer), "nn", st.out_dtype, v));
}

bool lower_gemv_group(const sanic_program_desc* d, int si, int64_t&, std::vector<LoweredStage>& out) {
    GemvPlan P0;
    if (!gemv_plan(d, si, P0)) return false;
    // batch the following stages that share the row prologue and weight-vector shape and do
    // not read an earlier member's output
    std::vector<GemvPlan> group{P0};
    Renderer probe0(d);
    GemvParts parts0 = gemv_parts(probe0, d, P0);
    std::set<int> written{d->stages[si].out_buffer};
    for (int s = si + 1; s < d->n_stages && group.size() < 8; s++) {
        GemvPlan P;
        if (!gemv_plan(d, s, P) || P.K != P0.K || P.cslots.size() != P0.cslots.size() || P.rslots.size() != P0.rslots.size())
            break;
        Renderer probe(d);
        GemvParts parts = gemv_parts(probe, d, P);
        if (parts.prologue != parts0.prologue || parts.wvec != parts0.wvec || parts.wdtypes != parts0.wdtypes) break;
        std::set<int> reads;
        const sanic_stage& st = d->stages[s];
        for (int l = 0; l < st.n_leaves; l++) collect_inputs(d, st.leaf[l], reads);
        if (st.epilogue >= 0) collect_inputs(d, st.epilogue, reads);
        bool dep = false;
        for (int b : reads) dep |= written.count(b) > 0;
        if (dep || written.count(st.out_buffer)) break;
        written.insert(st.out_buffer);
        group.push_back(P);
    }

    Renderer R(d);
    GemvParts parts = gemv_parts(R, d, P0);
    const int64_t K = P0.K;
    const int SC = (int)P0.cslots.size(), SR = (int)P0.rslots.size();
    int64_t NTOT = 0;
    std::vector<int64_t> seg_off;
    for (auto& P : group) { seg_off.push_back(NTOT); NTOT += P.N; }
    const int KI = (int)((K + 511) / 512);
    const int RQ = K <= 4096 ? 2 : 1;            // rows in flight per wave iteration
    // per-segment weight pointers
    std::vector<std::vector<int>> seg_wbufs;
    for (auto& P : group) {
        Renderer pr(d);
        seg_wbufs.push_back(gemv_parts(pr, d, P).wbufs);
    }
    Code k;
    k.indent = 1;
    k.line("extern __shared__ float u_lds[];");
    k.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
    for (int i = 0; i < SR; i++) k.line("float racc" + std::to_string(i) + " = 0.0f;");
    k.line("for (idx_t k = t; k < " + std::to_string(K) + "; k += 256) {");
    k.s << parts.prologue;
    k.line("}");
    if (SR > 0) {
        k.line("float* red = u_lds + " + std::to_string(SC * K) + ";");
        for (int i = 0; i < SR; i++) {
            k.line("for (int off = 32; off > 0; off >>= 1) racc" + std::to_string(i) + " += __shfl_xor(racc" + std::to_string(i) + ", off, 64);");
            k.line("if (lane == 0) red[wv * " + std::to_string(SR) + " + " + std::to_string(i) + "] = racc" + std::to_string(i) + ";");
        }
    }
    k.line("__syncthreads();");
    for (int i = 0; i < SR; i++)
        k.line("racc" + std::to_string(i) + " = ((red[" + std::to_string(i) + "] + red[" + std::to_string(SR + i) + "]) + red[" +
               std::to_string(2 * SR + i) + "]) + red[" + std::to_string(3 * SR + i) + "];");
    k.line("const idx_t nwaves = (idx_t)gridDim.x * 4;");
    k.line("for (idx_t r0 = ((idx_t)blockIdx.x * 4 + wv) * " + std::to_string(RQ) + "; r0 < " + std::to_string(NTOT) +
           "; r0 += nwaves * " + std::to_string(RQ) + ") {");
    k.indent++;
    k.line("float acc[" + std::to_string(RQ) + "][" + std::to_string(SC) + "];");
    // per row: segment, local row index, weight pointers
    for (int q = 0; q < RQ; q++) {
        std::string qs = std::to_string(q);
        k.line("const idx_t row" + qs + " = r0 + " + qs + ";");
        k.line("const bool live" + qs + " = row" + qs + " < " + std::to_string(NTOT) + ";");
        k.line("int seg" + qs + " = 0;");
        for (size_t g = 1; g < group.size(); g++)
            k.line("if (row" + qs + " >= " + std::to_string(seg_off[g]) + ") seg" + qs + " = " + std::to_string(g) + ";");
        std::string nnexpr = "row" + qs;
        for (size_t g = 1; g < group.size(); g++)
            nnexpr = "(seg" + qs + " == " + std::to_string(g) + " ? row" + qs + " - " + std::to_string(seg_off[g]) + " : " + nnexpr + ")";
        k.line("const idx_t nn" + qs + " = live" + qs + " ? " + nnexpr + " : 0;");
        for (size_t b = 0; b < parts.wbufs.size(); b++) {
            std::string sel = R.param(seg_wbufs[0][b]);
            for (size_t g = 1; g < group.size(); g++)
                sel = "(seg" + qs + " == " + std::to_string(g) + " ? " + R.param(seg_wbufs[g][b]) + " : " + sel + ")";
            k.line("const " + std::string(ctype_of(parts.wdtypes[b])) + "* __restrict__ wb" + std::to_string(b) + "_" + qs + " = " + sel + ";");
        }
        for (int c = 0; c < SC; c++) k.line("acc[" + qs + "][" + std::to_string(c) + "] = 0.0f;");
    }
    k.line("#pragma unroll");
    k.line("for (int i = 0; i < " + std::to_string(KI) + "; ++i) {");
    k.indent++;
    k.line("const idx_t k0 = (idx_t)i * 512 + lane * 8;");
    if (K % 512) k.line("if (k0 < " + std::to_string(K) + ") {");
    for (int c = 0; c < SC; c++) {
        std::string cs = std::to_string(c);
        k.line("const float4 ua" + cs + " = *(const float4*)(u_lds + " + cs + " * " + std::to_string(K) + " + k0);");
        k.line("const float4 ub" + cs + " = *(const float4*)(u_lds + " + cs + " * " + std::to_string(K) + " + k0 + 4);");
    }
    for (int q = 0; q < RQ; q++) {
        std::string qs = std::to_string(q);
        k.line("{");
        k.line("  const idx_t nn = nn" + qs + ";");
        for (size_t b = 0; b < parts.wbufs.size(); b++)
            k.line("  const " + std::string(ctype_of(parts.wdtypes[b])) + "* __restrict__ wb" + std::to_string(b) + " = wb" + std::to_string(b) + "_" + qs + ";");
        k.s << parts.wvec;
        for (int c = 0; c < SC; c++) {
            std::string cs = std::to_string(c);
            const char* comp[4] = {"x", "y", "z", "w"};
            std::string sum = "acc[" + qs + "][" + cs + "]";
            for (int j = 0; j < 8; j++)
                sum = "fmaf(" + std::string(j < 4 ? "ua" : "ub") + cs + "." + comp[j % 4] + ", " + parts.wvals[j] + ", " + sum + ")";
            k.line("  acc[" + qs + "][" + cs + "] = " + sum + ";");
        }
        k.line("}");
    }
    if (K % 512) k.line("}");
    k.indent--;
    k.line("}");
    // wave reduction and the finish
    for (int q = 0; q < RQ; q++)
        for (int c = 0; c < SC; c++) {
            std::string a = "acc[" + std::to_string(q) + "][" + std::to_string(c) + "]";
            k.line("for (int off = 32; off > 0; off >>= 1) " + a + " += __shfl_xor(" + a + ", off, 64);");
        }
    k.line("if (lane == 0) {");
    k.indent++;
    for (int q = 0; q < RQ; q++) {
        std::string qs = std::to_string(q);
        k.line("if (live" + qs + ") {");
        k.indent++;
        k.line("const idx_t nn = nn" + qs + ";");
        k.line("const float* accq = acc[" + qs + "];");
        for (size_t g = 0; g < group.size(); g++) {
            k.line(std::string(g ? "} else " : "") + "if (seg" + qs + " == " + std::to_string(g) + ") {");
            k.indent++;
            R.memo.emplace_back();
            gemv_finish(R, k, d, group[g]);
            R.memo.pop_back();
            k.indent--;
        }
        k.line("}");
        k.indent--;
        k.line("}");
    }
    k.indent--;
    k.line("}");
    k.indent--;
    k.line("}");

    // kernel names carry the shape so profiles tell the launches apart
    const std::string kname = "sanic_gemv_" + std::to_string(NTOT) + "x" + std::to_string(K);
    std::ostringstream src;
    src << kPrelude << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) " << kname << "(Args a) {\n"
        << k.str() << "}\n";
    int64_t waves = (NTOT + RQ - 1) / RQ;
    int64_t blocks = std::min<int64_t>((waves + 3) / 4, 2048);
    LoweredStage L;
    L.kernel_kind = "skeleton:gemv" + std::string(group.size() > 1 ? "[batched " + std::to_string(group.size()) + "]" : "");
    L.source = src.str();
    uint32_t lds = (uint32_t)((SC * K + 4 * std::max(SR, 1)) * 4);
    L.launches.push_back({kname, "", dim3((unsigned)blocks), dim3(256), lds, R.arg_list()});
    out.push_back(std::move(L));
    for (size_t g = 1; g < group.size(); g++) {
        LoweredStage B;
        B.kernel_kind = "batched-into:" + std::to_string(si);
        out.push_back(std::move(B));
    }
    return true;
}

// ───────────────────────── in-place row write (emit_metal.rs:1103-1178) ───────────────────
// A pointwise stage with `where = Lt(idx, P + 1) · Lt(P, idx + 1)` (update_cache, nn.rs:208-212)
// on one grid dim stores only the row idx = P: launch over the other dims with that dim pinned
// to round(P), re-checking the full condition before the store.

static bool scalar_tree(const sanic_program_desc* d, int node) {
    const sanic_node& n = d->nodes[node];
    for (int j = 0; j < n.rank; j++) if (n.shape[j] != 1) return false;
    if (n.kind == SANIC_NODE_IOTA || n.kind == SANIC_NODE_COORDINATE || n.kind == SANIC_NODE_FOLD) return false;
    for (int k = 0; k < n.n_in; k++) if (!scalar_tree(d, n.in[k])) return false;
    return true;
}

// match Lt(coord_dim, X + 1) where X is scalar: returns dim and X
static bool match_row_cond(const sanic_program_desc* d, int node, int rank, int& dim, int& pos) {
    const sanic_node& n = d->nodes[node];
    if (n.kind != SANIC_NODE_MAP) return false;
    if (n.op == SANIC_OP_MUL) {
        return match_row_cond(d, n.in[0], rank, dim, pos) || match_row_cond(d, n.in[1], rank, dim, pos);
    }
    if (n.op != SANIC_OP_LT) return false;
    const sanic_node& l = d->nodes[n.in[0]];
    const sanic_node& r = d->nodes[n.in[1]];
    if (l.kind != SANIC_NODE_COORDINATE || l.rank != n.rank) return false;
    if (r.kind != SANIC_NODE_MAP || r.op != SANIC_OP_ADD) return false;
    const sanic_node& r1 = d->nodes[r.in[1]];
    if (r1.kind != SANIC_NODE_CONST || r1.value != 1.0 || !scalar_tree(d, r.in[0])) return false;
    dim = l.dim + (rank - l.rank);
    pos = r.in[0];
    return true;
}

bool lower_pointwise_skeleton(const sanic_program_desc* d, int si, int64_t&, LoweredStage& out) {
    const sanic_stage& st = d->stages[si];
    if (st.where < 0) return false;
    int dim = -1, pos = -1;
    if (!match_row_cond(d, st.where, st.rank, dim, pos)) return false;
    Renderer R(d);
    Code body;
    body.indent = 1;
    int64_t rows = 1;
    for (int j = 0; j < st.rank; j++) if (j != dim) rows *= st.grid[j];
    body.line("const idx_t rid = (idx_t)blockIdx.x * 256 + threadIdx.x;");
    body.line("if (rid >= " + std::to_string(rows) + ") return;");
    std::string p = R.value(body, pos, std::vector<std::string>(d->nodes[pos].rank, "0"));
    body.line("const float pf = roundf(" + p + ");");
    body.line("if (!(pf >= 0.0f && pf < " + std::to_string(st.grid[dim]) + ".0f)) return;");
    std::string rem = "rid";
    for (int j = st.rank - 1; j >= 0; j--) {
        if (j == dim) continue;
        body.line("const idx_t g" + std::to_string(j) + " = " + rem + " % " + std::to_string(st.grid[j]) + ";");
        body.line("const idx_t q" + std::to_string(j) + " = " + rem + " / " + std::to_string(st.grid[j]) + ";");
        rem = "q" + std::to_string(j);
    }
    body.line("const idx_t g" + std::to_string(dim) + " = (idx_t)pf;");
    std::string lin;
    for (int j = 0; j < st.rank; j++)
        lin = j == 0 ? "g0" : "(" + lin + " * " + std::to_string(st.grid[j]) + " + g" + std::to_string(j) + ")";
    body.line("const idx_t gid = " + lin + ";");
    std::vector<std::string> gc;
    for (int j = 0; j < st.rank; j++) gc.push_back("g" + std::to_string(j));
    auto at = [&](int node) {
        const sanic_node& n = d->nodes[node];
        int lead = st.rank - n.rank;
        std::vector<std::string> c(n.rank);
        for (int j = 0; j < n.rank; j++) c[j] = n.shape[j] == 1 ? "0" : gc[lead + j];
        return R.value(body, node, c);
    };
    std::string w = at(st.where);
    body.line("if (" + w + " == 0.0f) return;");
    std::string v = at(st.value);
    body.line(store_stmt(R.param(st.out_buffer), "gid", st.out_dtype, v));
    std::ostringstream src;
    src << kPrelude << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) sanic_rowwrite(Args a) {\n"
        << body.str() << "}\n";
    out.kernel_kind = "skeleton:rowwrite";
    out.source = src.str();
    out.launches.push_back({"sanic_rowwrite", "", dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, R.arg_list()});
    return true;
}

bool lower_skeleton(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    if (lower_attn_decode(d, si, scratch, out)) return true;
    return false;
}

}  // namespace sanic
