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
#include <numeric>
#include <algorithm>
#include <regex>
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

void collect_inputs(const sanic_program_desc* d, int node, std::set<int>& bufs) {
    const sanic_node& n = d->nodes[node];
    if (n.kind == SANIC_NODE_INPUT) bufs.insert(n.buffer);
    for (int k = 0; k < n.n_in; k++) collect_inputs(d, n.in[k], bufs);
}

// ───────────────────────── vector weight renderer ─────────────────────────────────────────
// Renders the weight leaf W(n, k0 + j), j = 0..7, as 8 f32 expressions. The leaf must be an
// elementwise tree (Map/Const, through Reindex/View) over affine accesses; each access is
// loaded once per run of 8: a contiguous 128-bit (bf16) / 32-bit (nibbles) / 2×128-bit (f32)
// load, a single scalar when it does not move with k inside the run (per-group scale / zero
// point), or 8 scalar loads. Loads go to `lc` and the arithmetic to `dc`, so a kernel can issue
// every load of a row before it needs any of them.

struct VecW {
    const sanic_program_desc* d;
    std::vector<int> bufs;        // access buffers in traversal order -> pointers <ptr><i>
    std::vector<int> dtypes;
    int tmp = 0;
    bool ok = true;
    bool contiguous = true;       // every access moves by 0 or 1 element along k
    std::string nn = "nn", k0 = "k0", ptr = "wb", psfx, sfx;
    std::string last_raw;     // the 128-bit bf16 register of the last contiguous access
    bool stream = true;           // weights are read once: non-temporal loads
    bool byte_split = false;      // packed 4-bit runs through byte-to-float converts
    // run-invariant bf16 values loaded as raw 16-bit words in `lc`, widened in `dc` (so a caller
    // can hold the loaded words across a loop's back edge without waiting for the load there)
    bool raw_loads = false;
    // gcd of the k divisors of every access that does not move within a run (0: none moves
    // with k at all): such an access is constant over every aligned block of that many k
    int64_t uniform_div = 0;
    // general form: the coordinate variables' names and which of them the run of 8 moves
    // along (default: {nn, k0}, runs along var 1)
    std::vector<std::string> vars;
    int kv = 1;
    std::vector<std::string> names() const { return vars.empty() ? std::vector<std::string>{nn, k0} : vars; }
    std::string ld(const std::string& ty, const std::string& ptr) const {
        return stream ? "__builtin_nontemporal_load((const " + ty + "*)(" + ptr + "))" : "*(const " + ty + "*)(" + ptr + ")";
    }
    std::string fresh(const char* p) { return std::string(p) + std::to_string(tmp++) + sfx; }

    std::vector<std::string> render(Code& lc, Code& dc, int node, const std::vector<Sym>& c, const std::vector<int64_t>& ext) {
        const sanic_node& n = d->nodes[node];
        if (n.kind == SANIC_NODE_CONST) return std::vector<std::string>(8, flit(n.value));
        if (n.kind == SANIC_NODE_GATHER) {
            // src[.., index(..), ..]: the index (rounded half away from zero and clamped, as the
            // scalar renderer's gather) must be one value for the whole run; the gathered source
            // dim becomes a run-invariant variable of its own
            const sanic_node& src = d->nodes[n.in[0]];
            const sanic_node& ix = d->nodes[n.in[1]];
            std::vector<Sym> ic(c.begin() + n.dim, c.begin() + n.dim + ix.rank);
            std::vector<std::string> iv = render(lc, dc, n.in[1], ic, ext);
            if (!ok) return {};
            for (auto& v : iv) if (v != iv[0]) { ok = false; return {}; }
            // the index value is needed for addressing, so its arithmetic goes with the loads
            Code tmp;
            tmp.indent = lc.indent;
            tmp.s << dc.str();
            dc.s.str("");
            const std::string gi = fresh("gi");
            lc.s << tmp.str();
            lc.line("idx_t " + gi + " = (idx_t)roundf(" + iv[0] + ");");
            lc.line(gi + " = " + gi + " < 0 ? 0 : (" + gi + " > " + std::to_string(src.shape[n.dim] - 1) + " ? " +
                    std::to_string(src.shape[n.dim] - 1) + " : " + gi + ");");
            if (vars.empty()) vars = {nn, k0};
            const int gv = (int)vars.size();
            vars.push_back(gi);
            std::vector<int64_t> ext2 = ext;
            ext2.resize(gv + 1, 1);
            ext2[gv] = src.shape[n.dim];
            std::vector<Sym> sc(src.rank);
            for (int j = 0; j < src.rank; j++)
                sc[j] = j < n.dim ? c[j] : j == n.dim ? Sym::var(gv) : c[j - 1 + ix.rank];
            return render(lc, dc, n.in[0], sc, ext2);
        }
        if (n.kind == SANIC_NODE_IOTA || n.kind == SANIC_NODE_COORDINATE) {
            // the coordinate's own value: one value per run when it does not move within an
            // aligned run of 8, else base + j·coef when it moves by a constant step
            const Sym& cs = c[n.kind == SANIC_NODE_IOTA ? 0 : n.dim];
            int64_t step = 0;
            for (auto& t : cs.terms) {
                if (t.var != kv) continue;
                if (t.div == 1 && t.mod == 0) step += t.coef;
                else if (t.div % 8 != 0 || (t.div == 1 && t.mod % 8 != 0)) { ok = false; return {}; }
            }
            std::string base = fresh("ci");
            lc.line("const float " + base + " = (float)(" + cs.render(names()) + ");");
            std::vector<std::string> out(8);
            for (int j = 0; j < 8; j++) out[j] = step == 0 ? base : "(" + base + " + " + flit((double)(step * j)) + ")";
            return out;
        }
        if (n.kind == SANIC_NODE_MAP) {
            std::vector<std::string> a[3];
            for (int k = 0; k < n.n_in; k++) {
                const sanic_node& m = d->nodes[n.in[k]];
                int lead = n.rank - m.rank;
                std::vector<Sym> cc(m.rank);
                for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? Sym() : c[lead + j];
                a[k] = render(lc, dc, n.in[k], cc, ext);
                if (!ok) return {};
            }
            std::vector<std::string> out(8);
            for (int j = 0; j < 8; j++) {
                std::string v = fresh("w");
                dc.line("const float " + v + " = " + map_expr(n.op, a[0][j], a[1].empty() ? "" : a[1][j], a[2].empty() ? "" : a[2][j]) + ";");
                out[j] = v;
            }
            return out;
        }
        if (n.kind == SANIC_NODE_REINDEX || n.kind == SANIC_NODE_VIEW) {
            std::vector<Sym> sc;
            if (!sym_child_coords(d, node, c, ext, sc)) { ok = false; return {}; }
            return render(lc, dc, n.in[0], sc, ext);
        }
        Access acc;
        if (!sym_access(d, node, c, ext, acc)) { ok = false; return {}; }
        int64_t jstride = 0;
        for (auto& t : acc.addr.terms) {
            if (t.var != kv) continue;
            if (t.div == 1 && (t.mod == 0 || t.mod % 8 == 0)) jstride += t.coef;
            else if (t.div % 8 != 0) { ok = false; return {}; }
        }
        if (jstride != 0 && jstride != 1) contiguous = false;
        int slot = (int)bufs.size();
        bufs.push_back(acc.buffer);
        dtypes.push_back(acc.dtype);
        std::string p = ptr + std::to_string(slot) + psfx;
        std::string addr = acc.addr.render(names());
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
        lc.line("const idx_t " + base + " = " + addr + ";");
        const char* comp[4] = {"x", "y", "z", "w"};
        if (jstride == 0) {
            for (auto& t : acc.addr.terms)
                if (t.var == kv) uniform_div = std::gcd(uniform_div, t.div);
            std::string v = fresh("w");
            if (raw_loads && acc.dtype == SANIC_BF16) {
                const std::string h = fresh("h");
                lc.line("const unsigned short " + h + " = " + p + "[" + base + "];");
                dc.line("const float " + v + " = sanic_bf16(" + h + ");");
            } else {
                lc.line("const float " + v + " = " + one(base) + ";");
            }
            return std::vector<std::string>(8, v);
        }
        if (jstride == 1 && acc.dtype == SANIC_BF16) {
            std::string v = fresh("wq");
            lc.line("const sanic_u32x4 " + v + " = " + ld("sanic_u32x4", p + " + " + base) + ";");
            last_raw = v;
            for (int j = 0; j < 8; j++)
                out[j] = std::string("__uint_as_float(") + (j % 2 == 0 ? "(" + v + "." + comp[j / 2] + " << 16)"
                                                                        : "(" + v + "." + comp[j / 2] + " & 0xFFFF0000u)") + ")";
            return out;
        }
        if (jstride == 1 && acc.dtype == SANIC_F32) {
            std::string v0 = fresh("f"), v1 = fresh("f");
            lc.line("const sanic_f32x4 " + v0 + " = " + ld("sanic_f32x4", p + " + " + base) + ";");
            lc.line("const sanic_f32x4 " + v1 + " = " + ld("sanic_f32x4", p + " + " + base + " + 4") + ";");
            for (int j = 0; j < 8; j++) out[j] = (j < 4 ? v0 : v1) + "." + comp[j % 4];
            return out;
        }
        if (jstride == 1 && (acc.dtype == SANIC_U4 || acc.dtype == SANIC_I4)) {
            std::string v = fresh("u");
            lc.line("const unsigned " + v + " = " + ld("unsigned", p + " + (" + base + " >> 1)") + ";");
            if (!byte_split) {
                for (int j = 0; j < 8; j++) {
                    std::string e = "(float)((" + v + " >> " + std::to_string(4 * j) + ") & 0xFu)";
                    out[j] = acc.dtype == SANIC_I4 ? "(" + e + " - 8.0f)" : e;
                }
                return out;
            }
            // even nibbles to the low halves of the 4 bytes, odd ones to a second word: each value
            // is then one byte-to-float convert (v_cvt_f32_ubyteN; measured on the int4 GEMV,
            // 4.74 → 4.60 µs; the GEMM's dequantizing tile loads are slower with it, 21.8 → 25.3)
            const std::string ev = v + "e", od = v + "o";
            // (the empty asm hides the masks from the combiner, which would fold them back into
            // one bit-field extract per value)
            dc.line("unsigned " + ev + " = " + v + " & 0x0F0F0F0Fu, " + od + " = (" + v + " >> 4) & 0x0F0F0F0Fu;");
            dc.line("asm(\"\" : \"+v\"(" + ev + "), \"+v\"(" + od + "));");
            for (int j = 0; j < 8; j++) {
                std::string e = "(float)((" + (j % 2 ? od : ev) + " >> " + std::to_string(8 * (j / 2)) + ") & 0xFFu)";
                out[j] = acc.dtype == SANIC_I4 ? "(" + e + " - 8.0f)" : e;
            }
            return out;
        }
        for (int j = 0; j < 8; j++) {
            std::string v = fresh("w");
            lc.line("const float " + v + " = " + one(base + " + " + std::to_string(jstride * j)) + ";");
            out[j] = v;
        }
        return out;
    }

    // The leaf as q·A (± B) over a run of 8: q an integer-valued access (a packed 4-bit run), A
    // and B each the same value for the whole run (a group's scale and zero point), found
    // through views and reindexes. Renders in the same traversal order as render(), so the
    // buffer slots agree; on failure the caller discards this renderer and its code.
    bool render_affine(Code& lc, Code& dc, int node, const std::vector<Sym>& c, const std::vector<int64_t>& ext,
                       std::vector<std::string>& q, std::string& A, std::string& B, bool& negB) {
        const sanic_node& n = d->nodes[node];
        if (n.kind == SANIC_NODE_REINDEX || n.kind == SANIC_NODE_VIEW) {
            std::vector<Sym> sc;
            if (!sym_child_coords(d, node, c, ext, sc)) return false;
            return render_affine(lc, dc, n.in[0], sc, ext, q, A, B, negB);
        }
        if (n.kind != SANIC_NODE_MAP) return false;
        auto coords = [&](int k) {
            const sanic_node& m = d->nodes[n.in[k]];
            int lead = n.rank - m.rank;
            std::vector<Sym> cc(m.rank);
            for (int j = 0; j < m.rank; j++) cc[j] = m.shape[j] == 1 ? Sym() : c[lead + j];
            return cc;
        };
        auto uniform = [](const std::vector<std::string>& v) {
            for (auto& x : v) if (x != v[0]) return false;
            return !v.empty();
        };
        if ((n.op == SANIC_OP_SUB || n.op == SANIC_OP_ADD) && n.n_in == 2) {
            const sanic_node& m0 = d->nodes[n.in[0]];
            if (m0.kind != SANIC_NODE_MAP || m0.op != SANIC_OP_MUL) return false;
            std::string b0;
            bool nb = false;
            if (!render_affine(lc, dc, n.in[0], coords(0), ext, q, A, b0, nb) || !b0.empty()) return false;
            std::vector<std::string> bv = render(lc, dc, n.in[1], coords(1), ext);
            if (!ok || !uniform(bv)) return false;
            B = bv[0];
            negB = n.op == SANIC_OP_SUB;
            return true;
        }
        if (n.op != SANIC_OP_MUL || n.n_in != 2) return false;
        std::vector<std::string> v[2];
        int qi = -1;
        for (int k = 0; k < 2; k++) {
            const sanic_node& m = d->nodes[n.in[k]];
            const bool packed = m.kind == SANIC_NODE_INPUT && (m.dtype == SANIC_U4 || m.dtype == SANIC_I4);
            v[k] = render(lc, dc, n.in[k], coords(k), ext);
            if (!ok) return false;
            if (packed) {
                if (qi >= 0) return false;
                qi = k;
            }
        }
        if (qi < 0 || !uniform(v[1 - qi])) return false;
        q = v[qi];
        A = v[1 - qi][0];
        B.clear();
        negB = false;
        return true;
    }
};

// One run of 8 of a leaf at (nn, k0) through the vector renderer (used by the GEMM skeleton).
// `raw_bf16` names the 128-bit register when the leaf is exactly one contiguous bf16 access.
std::vector<std::string> render_weight_run(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                                           const std::vector<int64_t>& ext, Code& lc, Code& dc, const std::string& nn,
                                           const std::string& k0, const std::string& sfx, std::vector<int>& bufs,
                                           std::vector<int>& dtypes, bool& ok, bool& contiguous, std::string& raw_bf16,
                                           bool stream) {
    VecW vw{d};
    vw.stream = stream;
    vw.nn = nn;
    vw.k0 = k0;
    vw.ptr = "wb";
    vw.psfx = sfx;
    vw.sfx = sfx;
    auto vals = vw.render(lc, dc, node, c, ext);
    bufs = vw.bufs;
    dtypes = vw.dtypes;
    ok = vw.ok;
    contiguous = vw.contiguous;
    int kind = d->nodes[node].kind;
    raw_bf16 = (bufs.size() == 1 && dtypes[0] == SANIC_BF16 && kind != SANIC_NODE_MAP && kind != SANIC_NODE_CONST) ? vw.last_raw : "";
    return vals;
}

// One run of 8 of a weight leaf of the form q·A ± B (q a packed 4-bit run, A and B constant
// over the run) at (nn, k0): q's 8 values, A and B (B empty when absent; negB for q·A − B).
// `uniform_div`: A and B are constant over every aligned block of that many k (0: over all k).
bool render_weight_affine(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                          const std::vector<int64_t>& ext, Code& lc, Code& dc, const std::string& nn,
                          const std::string& k0, const std::string& sfx, std::vector<int>& bufs,
                          std::vector<int>& dtypes, std::vector<std::string>& q, std::string& A, std::string& B,
                          bool& negB, int64_t& uniform_div, bool stream, bool raw_loads) {
    VecW vw{d};
    vw.stream = stream;
    vw.raw_loads = raw_loads;
    vw.nn = nn;
    vw.k0 = k0;
    vw.ptr = "wb";
    vw.psfx = sfx;
    vw.sfx = sfx;
    negB = false;
    const bool ok = vw.render_affine(lc, dc, node, c, ext, q, A, B, negB) && vw.ok;
    bufs = vw.bufs;
    dtypes = vw.dtypes;
    uniform_div = vw.uniform_div;
    return ok;
}

// One run of 8 of an elementwise leaf at coordinates `c` over named variables `vars`, the run
// moving along variable `kv` from its value vars[kv] (a multiple of 8): 8 f32 expressions, loads
// in `lc`, arithmetic in `dc`; plain (not non-temporal) loads through pointers named
// rb<i><sfx> for the buffers `bufs` (dtypes `dtypes`), which the caller declares.
std::vector<std::string> render_run(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                                    const std::vector<int64_t>& ext, const std::vector<std::string>& vars, int kv,
                                    Code& lc, Code& dc, const std::string& sfx, std::vector<int>& bufs,
                                    std::vector<int>& dtypes, bool& ok) {
    VecW vw{d};
    vw.stream = false;
    vw.vars = vars;
    vw.kv = kv;
    vw.ptr = "rb";
    vw.psfx = sfx;
    vw.sfx = sfx;
    auto vals = vw.render(lc, dc, node, c, ext);
    ok = vw.ok;
    bufs = vw.bufs;
    dtypes = vw.dtypes;
    return vals;
}

// ───────────────────────── gemv ───────────────────────────────────────────────────────────

struct GemvPlan {
    int stage = -1;
    int ndim = -1;         // the one grid dim with extent > 1
    int64_t N = 0, K = 0;
    int w = -1;            // weight leaf index
    std::vector<int> cslots, rslots;
};

// weight leaf coordinates over {0: n, 1: k} (swapped: {0: k, 1: n}, runs of 8 along n)
static std::vector<Sym> weight_coords(const sanic_program_desc* d, const sanic_stage& st, int w, int ndim, bool swapped = false) {
    const sanic_node& wn = d->nodes[st.leaf[w]];
    std::vector<Sym> cw(wn.rank);
    for (int j = 0; j < wn.rank; j++) {
        int b = st.bind[w][j];
        cw[j] = b == SANIC_BIND_STREAM ? Sym::var(swapped ? 0 : 1) : b == ndim ? Sym::var(swapped ? 1 : 0) : Sym();
    }
    return cw;
}

static bool gemv_plan(const sanic_program_desc* d, int si, GemvPlan& P, bool kmajor = false) {
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
    if (st.stream % 8 != 0 || st.stream < 64 || st.stream > 16384) return false;
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
    VecW vw{d};
    Code lc, dc;
    if (kmajor) {
        // N-contiguous weights ([in, out]): runs of 8 along n
        vw.render(lc, dc, st.leaf[w], weight_coords(d, st, w, ndim, true), {P.K, P.N});
        return vw.ok && vw.contiguous;
    }
    vw.render(lc, dc, st.leaf[w], weight_coords(d, st, w, ndim), {P.N, P.K});
    // K-contiguous weights (the reference's [out, in] layout): every access moves by 1 or 0
    // along a run of k; other layouts go to the generic fold
    return vw.ok && vw.contiguous;
}

// The row prologue of a gemv stage: leaf values at k, each contraction slot's factor `rest`
// stored to LDS, each row slot accumulated into racc<i>.
static std::string gemv_prologue(Renderer& R, const sanic_program_desc* d, const GemvPlan& P) {
    const sanic_stage& st = d->stages[P.stage];
    const sanic_carrier& c = st.carrier;
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
    return pc.str();
}

static std::string gemv_finish(Renderer& R, Code& code, const sanic_program_desc* d, const GemvPlan& P, bool coherent) {
    const sanic_stage& st = d->stages[P.stage];
    const sanic_carrier& c = st.carrier;
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
    code.line(store_stmt(R.param(st.out_buffer), "nn", st.out_dtype, v, coherent, d->buffers[st.out_buffer].scale));
    return v;
}

// A pointwise stage right after a batched group whose value is elementwise over the group's
// outputs at its own index (e.g. silu(gate)·up): only MAP / CONST / INPUT nodes, every rank-1
// input of extent N. Computed in the group kernel itself when each wave holds row i of every
// segment, so the product never takes a launch or a re-read.
static bool paired_candidate(const sanic_program_desc* d, int si, int64_t N) {
    if (si >= d->n_stages) return false;
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_POINTWISE || st.where >= 0 || st.rank != 1 || st.grid[0] != N) return false;
    if (d->buffers[st.out_buffer].role == SANIC_BUF_STATE || d->buffers[st.out_buffer].role == SANIC_BUF_INPUT) return false;
    std::vector<int> stack{st.value};
    while (!stack.empty()) {
        const sanic_node& n = d->nodes[stack.back()];
        stack.pop_back();
        if (n.kind == SANIC_NODE_CONST) continue;
        if (n.kind == SANIC_NODE_INPUT) {
            if (n.rank > 1 || (n.rank == 1 && n.shape[0] != N)) return false;
            continue;
        }
        if (n.kind != SANIC_NODE_MAP) return false;
        for (int k = 0; k < n.n_in; k++) stack.push_back(n.in[k]);
    }
    return true;
}

// ───────────────────────── in-place row write (emit_metal.rs:1103-1178) ───────────────────
// A pointwise stage with `where = Lt(idx, P + 1) · Lt(P, idx + 1)` (update_cache, nn.rs:208-212)
// on one grid dim stores only the row idx = P: iterate the other dims with that dim pinned to
// round(P), re-checking the full condition before the store.

static bool scalar_tree(const sanic_program_desc* d, int node) {
    const sanic_node& n = d->nodes[node];
    for (int j = 0; j < n.rank; j++) if (n.shape[j] != 1) return false;
    if (n.kind == SANIC_NODE_IOTA || n.kind == SANIC_NODE_COORDINATE || n.kind == SANIC_NODE_FOLD) return false;
    for (int k = 0; k < n.n_in; k++) if (!scalar_tree(d, n.in[k])) return false;
    return true;
}

// match Lt(coord_dim, X + 1) where X is scalar: returns dim and X
bool match_row_cond(const sanic_program_desc* d, int node, int rank, int& dim, int& pos) {
    const sanic_node& n = d->nodes[node];
    if (n.kind != SANIC_NODE_MAP) return false;
    if (n.op == SANIC_OP_MUL)
        return match_row_cond(d, n.in[0], rank, dim, pos) || match_row_cond(d, n.in[1], rank, dim, pos);
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

// Iterations a pointwise stage needs (rows only, for a row write).
static int64_t pointwise_work(const sanic_program_desc* d, int si, int& dim, int& pos) {
    const sanic_stage& st = d->stages[si];
    dim = pos = -1;
    int64_t n = vol(st.grid, st.rank);
    if (st.where >= 0 && match_row_cond(d, st.where, st.rank, dim, pos)) n /= st.grid[dim];
    return n;
}

// Emit a pointwise stage as a loop `for (rid = tid; rid < work; rid += nth)`.
void emit_pointwise_loop(Renderer& R, Code& body, const sanic_program_desc* d, int si, const std::string& tid,
                                int nth) {
    const sanic_stage& st = d->stages[si];
    int dim, pos;
    int64_t work = pointwise_work(d, si, dim, pos);
    body.line("for (idx_t rid = " + tid + "; rid < " + std::to_string(work) + "; rid += " + std::to_string(nth) + ") {");
    body.indent++;
    R.memo.emplace_back();
    std::string rem = "rid";
    if (dim >= 0) {
        std::string p = R.value(body, pos, std::vector<std::string>(d->nodes[pos].rank, "0"));
        body.line("const float pf = roundf(" + p + ");");
        body.line("if (!(pf >= 0.0f && pf < " + std::to_string(st.grid[dim]) + ".0f)) continue;");
    }
    for (int j = st.rank - 1; j >= 0; j--) {
        if (j == dim) continue;
        body.line("const idx_t g" + std::to_string(j) + " = " + rem + " % " + std::to_string(st.grid[j]) + ";");
        body.line("const idx_t q" + std::to_string(j) + " = " + rem + " / " + std::to_string(st.grid[j]) + ";");
        rem = "q" + std::to_string(j);
    }
    if (dim >= 0) body.line("const idx_t g" + std::to_string(dim) + " = (idx_t)pf;");
    std::string lin = "0";
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
    if (st.where >= 0) {
        std::string w = at(st.where);
        body.line("if (" + w + " == 0.0f) continue;");
    }
    std::string v = at(st.value);
    body.line(store_stmt(R.param(st.out_buffer), "gid", st.out_dtype, v, false, d->buffers[st.out_buffer].scale));
    R.memo.pop_back();
    body.indent--;
    body.line("}");
}

// Stages that may run as the tail of the kernel before them: small pointwise stages.
bool tail_candidate(const sanic_program_desc* d, int si) {
    if (si >= d->n_stages) return false;
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_POINTWISE) return false;
    if (attn_absorber(d, si) >= 0) return false;     // the attention kernel performs it
    int dim, pos;
    return pointwise_work(d, si, dim, pos) <= 65536;
}

// Last-workgroup tail: after every workgroup's writes are released, the last one to arrive runs
// the absorbed stages (program order is kept: they start only once the whole kernel's outputs
// are visible). The arrival counter re-arms itself for the next launch.
void emit_tail(Renderer& R, Code& k, const sanic_program_desc* d, const std::vector<int>& tails, const std::string& counter,
               const std::string& expected) {
    if (tails.empty()) return;
    // data the tails write is never hoisted or cached across them
    for (int t : tails) R.coherent.insert(d->stages[t].out_buffer);
    k.line("{");
    k.indent++;
    emit_arrival(k, "sanic_last", "threadIdx.x", counter, expected);
    k.line("if (sanic_last) {");
    k.indent++;
    for (size_t i = 0; i < tails.size(); i++) {
        if (i) k.line("__syncthreads();");
        emit_pointwise_loop(R, k, d, tails[i], "(idx_t)threadIdx.x", 256);
    }
    k.line("if (threadIdx.x == 0) sanic_st(" + counter + ", 0u);");
    k.indent--;
    k.line("}");
    k.indent--;
    k.line("}");
}

// The loads an elementwise epilogue makes at the output point `gc` (a residual read, say),
// rendered ahead of time: the epilogue is rendered once with a stand-in fold value and the
// variables of its buffer loads are returned by node, to be substituted when the epilogue is
// rendered for real. The loads then go out with the weight stream instead of after the
// reduction. Empty when the tree has an in-body reduction (a node could then be read at
// several points).
static std::map<int, std::string> prefetch_epilogue(Renderer& R, Code& k, const sanic_program_desc* d, int epi,
                                                    const std::vector<std::string>& gc) {
    std::map<int, std::string> vars;
    std::vector<int> stack{epi};
    while (!stack.empty()) {
        int ni = stack.back();
        stack.pop_back();
        const sanic_node& n = d->nodes[ni];
        if (n.kind == SANIC_NODE_REDUCE || n.kind == SANIC_NODE_SCAN || n.kind == SANIC_NODE_GATHER) return vars;
        for (int j = 0; j < n.n_in; j++) stack.push_back(n.in[j]);
    }
    const std::string saved = R.fold_var;
    R.fold_var = "0.0f";
    R.memo.emplace_back();
    Code tmp;
    tmp.indent = k.indent;
    R.value(tmp, epi, gc);
    for (auto& kv : R.memo.back()) {
        int node = atoi(kv.first.c_str());
        if (d->nodes[node].kind == SANIC_NODE_INPUT) vars[node] = kv.second;
    }
    R.memo.pop_back();
    R.fold_var = saved;
    k.s << tmp.str();
    return vars;
}

bool lower_gemv_group(const sanic_program_desc* d, int si, int64_t& scratch, std::vector<LoweredStage>& out) {
    GemvPlan P0;
    if (!gemv_plan(d, si, P0)) return false;
    // batch the following stages that share the row prologue and weight-vector shape and do
    // not read an earlier member's output (q/k/v; gate/up)
    std::vector<GemvPlan> group{P0};
    Renderer probe0(d);
    std::string pro0 = gemv_prologue(probe0, d, P0);
    auto wshape = [&](const GemvPlan& P, std::vector<int>& bufs, std::vector<int>& dts) {
        VecW vw{d};
        Code lc, dc;
        vw.render(lc, dc, d->stages[P.stage].leaf[P.w], weight_coords(d, d->stages[P.stage], P.w, P.ndim), {P.N, P.K});
        bufs = vw.bufs;
        dts = vw.dtypes;
        return lc.str() + dc.str();
    };
    std::vector<int> wb0, wd0;
    std::string ws0 = wshape(P0, wb0, wd0);
    std::set<int> written{d->stages[si].out_buffer};
    std::vector<std::vector<int>> seg_wbufs{wb0};
    const bool no_batch = getenv("SANIC_HIP_NO_BATCH") != nullptr;   // measurement knob
    for (int s = si + 1; s < d->n_stages && group.size() < 8 && !no_batch; s++) {
        GemvPlan P;
        if (!gemv_plan(d, s, P) || P.K != P0.K || P.cslots.size() != P0.cslots.size() || P.rslots.size() != P0.rslots.size())
            break;
        Renderer probe(d);
        std::vector<int> wb, wd;
        if (gemv_prologue(probe, d, P) != pro0 || wshape(P, wb, wd) != ws0 || wd != wd0) break;
        std::set<int> reads;
        const sanic_stage& st = d->stages[s];
        for (int l = 0; l < st.n_leaves; l++) collect_inputs(d, st.leaf[l], reads);
        if (st.epilogue >= 0) collect_inputs(d, st.epilogue, reads);
        bool dep = false;
        for (int b : reads) dep |= written.count(b) > 0;
        if (dep || written.count(st.out_buffer)) break;
        written.insert(st.out_buffer);
        group.push_back(P);
        seg_wbufs.push_back(wb);
    }
    // an elementwise consumer of the whole group, computed per row pair in the kernel
    int paired = -1;
    {
        bool same = group.size() >= 2;
        for (auto& P : group) same = same && P.N == P0.N;
        if (same && paired_candidate(d, si + (int)group.size(), P0.N)) paired = si + (int)group.size();
        if (paired >= 0) {
            // it may read only group outputs and buffers nobody in the group writes
            std::set<int> reads;
            collect_inputs(d, d->stages[paired].value, reads);
            for (int b : reads)
                if (!written.count(b) && d->buffers[b].role != SANIC_BUF_INPUT && d->buffers[b].role != SANIC_BUF_STATE) paired = -1;
        }
    }
    // absorb the small pointwise stages that follow as the kernel's tail
    std::vector<int> tails;
    for (int s = si + (int)group.size() + (paired >= 0); tail_candidate(d, s) && tails.size() < 4; s++) tails.push_back(s);

    Renderer R(d);
    std::string prologue = gemv_prologue(R, d, P0);
    for (auto& P : group) R.coherent.insert(d->stages[P.stage].out_buffer);
    const int64_t K = P0.K;
    const int SC = (int)P0.cslots.size(), SR = (int)P0.rslots.size();
    int64_t NTOT = 0;
    std::vector<int64_t> seg_off;
    for (auto& P : group) { seg_off.push_back(NTOT); NTOT += P.N; }
    const int KI = (int)((K + 511) / 512);
    int RQ = K <= 2048 ? 2 : 1;                  // rows in flight per wave iteration
    if (paired >= 0) RQ = (int)group.size();     // row i of every segment in one wave
    int64_t waves = (NTOT + RQ - 1) / RQ;
    const int64_t max_blocks = 1024;
    int64_t blocks = std::min<int64_t>((waves + 3) / 4, max_blocks);
    int64_t counter_off = -1;
    if (!tails.empty()) {
        counter_off = scratch;
        scratch += 256;
    }

    // ── split-K form: the 4 waves of a workgroup take one quarter of K each, every lane keeps
    // its activation factors in registers (loaded once, reused by all rows of the workgroup),
    // and the per-wave partials meet in LDS once at the end: no LDS staging of the activation
    // and no barrier before the weight FMAs.
    if (K % 2048 == 0 && K <= 16384) {
        const int64_t KQ = K / 4;
        const int KIq = (int)(KQ / 512);
        const int NSEG = (int)group.size();
        // rows per workgroup: 4 for very tall matrices (lm_head: fewer, fuller workgroups
        // measured faster) and for packed 4-bit weights (a lane's run of 8 weights is 4 bytes,
        // so more rows keep more bytes in flight: int4 8192×2048 5.37 → 5.09 µs, 8 rows 5.75),
        // else 2 (the measured tuner's pick for the 2048×8192 down projection in the decode
        // step: 680 → 655 µs per step against 4)
        bool packed4 = false;
        for (int dt : wd0) packed4 |= dt == SANIC_U4 || dt == SANIC_I4;
        int RBI = NTOT >= 65536 || packed4 ? 4 : 2;
        // tiling variants for the measured tuner: rows per workgroup {rule, 1, 2, 4} ({2, 1, 4}
        // for a paired launch, whose workgroup holds row i of every segment)
        const int gvar = d->stages[si].sched.variant;
        const int nvar = paired >= 0 ? 3 : 4;
        if (gvar > 0 && gvar < nvar) RBI = paired >= 0 ? (gvar == 1 ? 1 : 4) : (1 << (gvar - 1));
        if (paired >= 0 && !(gvar > 0 && gvar < nvar)) RBI = 2;
        const int RB = paired >= 0 ? RBI * NSEG : RBI;           // rows per workgroup
        const int64_t UNITS = paired >= 0 ? P0.N : NTOT;
        const int64_t nblocks = (UNITS + RBI - 1) / RBI;
        const int RW = RB * SC + SR;                             // partials per wave
        Code k;
        k.indent = 1;
        k.line("__shared__ float red[4][" + std::to_string(RW) + "];");
        k.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
        k.line("const idx_t kb = (idx_t)wv * " + std::to_string(KQ) + ";");
        // rows of this workgroup
        for (int q = 0; q < RB; q++) {
            std::string qs = std::to_string(q);
            if (paired >= 0) {
                // row q = unit q / NSEG of this workgroup, segment q % NSEG
                const int u = q / NSEG, g = q % NSEG;
                const std::string unit = "((idx_t)blockIdx.x * " + std::to_string(RBI) + " + " + std::to_string(u) + ")";
                k.line("const idx_t row" + qs + " = " + unit + " + " + std::to_string(g * P0.N) + ";");
                k.line("const bool live" + qs + " = " + unit + " < " + std::to_string(P0.N) + ";");
                k.line("const int seg" + qs + " = " + std::to_string(g) + ";");
                k.line("const idx_t nn" + qs + " = live" + qs + " ? " + unit + " : 0;");
                for (size_t b = 0; b < wb0.size(); b++)
                    k.line("const " + std::string(ctype_of(wd0[b])) + "* __restrict__ wb" + std::to_string(b) + "_" + qs + " = " + R.param(seg_wbufs[g][b]) + ";");
                continue;
            }
            k.line("const idx_t row" + qs + " = (idx_t)blockIdx.x * " + std::to_string(RBI) + " + " + qs + ";");
            k.line("const bool live" + qs + " = row" + qs + " < " + std::to_string(NTOT) + ";");
            k.line("int seg" + qs + " = 0;");
            for (size_t g = 1; g < group.size(); g++)
                k.line("if (row" + qs + " >= " + std::to_string(seg_off[g]) + ") seg" + qs + " = " + std::to_string(g) + ";");
            std::string nnexpr = "row" + qs;
            for (size_t g = 1; g < group.size(); g++)
                nnexpr = "(seg" + qs + " == " + std::to_string(g) + " ? row" + qs + " - " + std::to_string(seg_off[g]) + " : " + nnexpr + ")";
            k.line("const idx_t nn" + qs + " = live" + qs + " ? " + nnexpr + " : 0;");
            for (size_t b = 0; b < wb0.size(); b++) {
                std::string sel = R.param(seg_wbufs[0][b]);
                for (size_t g = 1; g < group.size(); g++)
                    sel = "(seg" + qs + " == " + std::to_string(g) + " ? " + R.param(seg_wbufs[g][b]) + " : " + sel + ")";
                k.line("const " + std::string(ctype_of(wd0[b])) + "* __restrict__ wb" + std::to_string(b) + "_" + qs + " = " + sel + ";");
            }
        }
        // weight loads: every (row, run) is requested before any arithmetic
        std::vector<std::vector<std::vector<std::string>>> wvals(RB, std::vector<std::vector<std::string>>(KIq));
        // A weight of the form q·A ± B with q a packed 4-bit run and A, B constant over the run
        // (group scale and zero point) is not dequantized per element: the run's dot product
        // Σ x·w = A·Σ x·q ± B·Σ x takes one FMA per weight instead of two (plus two per run)
        const int wleaf = d->stages[P0.stage].leaf[P0.w];
        const std::vector<Sym> wcoords = weight_coords(d, d->stages[P0.stage], P0.w, P0.ndim);
        bool affine = SC == 1 && packed4;
        if (affine) {
            VecW t{d};
            Code l1, d1;
            std::vector<std::string> qq;
            std::string A_, B_;
            bool nb = false;
            affine = t.render_affine(l1, d1, wleaf, wcoords, {P0.N, P0.K}, qq, A_, B_, nb) && t.ok;
        }
        std::vector<std::vector<std::string>> aA(RB, std::vector<std::string>(KIq)), aB(RB, std::vector<std::string>(KIq));
        bool negB = false;
        Code wdc;
        wdc.indent = k.indent;
        for (int q = 0; q < RB; q++)
            for (int i = 0; i < KIq; i++) {
                VecW vw{d};
                vw.nn = "nn" + std::to_string(q);
                vw.k0 = "(kb + " + std::to_string(i * 512) + " + lane * 8)";
                vw.ptr = "wb";
                vw.psfx = "_" + std::to_string(q);
                vw.sfx = "_" + std::to_string(q) + "_" + std::to_string(i);
                Code l1;
                l1.indent = k.indent;
                if (affine) {
                    vw.byte_split = true;
                    if (!vw.render_affine(l1, wdc, wleaf, wcoords, {P0.N, P0.K}, wvals[q][i], aA[q][i], aB[q][i], negB)) return false;
                } else {
                    wvals[q][i] = vw.render(l1, wdc, wleaf, wcoords, {P0.N, P0.K});
                }
                if (!vw.ok) return false;
                k.s << l1.str();
            }
        // activation factors of this lane's k runs (loads, then arithmetic)
        const sanic_stage& st0 = d->stages[P0.stage];
        const sanic_carrier& c0 = st0.carrier;
        std::vector<std::vector<std::vector<std::string>>> lvals(st0.n_leaves, std::vector<std::vector<std::string>>(KIq));
        Code adc;
        adc.indent = k.indent;
        for (int l = 0; l < st0.n_leaves; l++) {
            if (l == P0.w) continue;
            const sanic_node& ln = d->nodes[st0.leaf[l]];
            std::vector<Sym> cl(ln.rank);
            for (int j = 0; j < ln.rank; j++) cl[j] = st0.bind[l][j] == SANIC_BIND_STREAM ? Sym::var(1) : Sym();
            for (int i = 0; i < KIq; i++) {
                VecW vw{d};
                vw.stream = false;
                vw.nn = "0";
                vw.k0 = "(kb + " + std::to_string(i * 512) + " + lane * 8)";
                vw.ptr = "xb";
                vw.psfx = "_" + std::to_string(l) + "_" + std::to_string(i);
                vw.sfx = "_x" + std::to_string(l) + "_" + std::to_string(i);
                Code l1;
                l1.indent = k.indent;
                lvals[l][i] = vw.render(l1, adc, st0.leaf[l], cl, {1, P0.K});
                if (!vw.ok) return false;
                for (size_t b = 0; b < vw.bufs.size(); b++)
                    k.line("const " + std::string(ctype_of(vw.dtypes[b])) + "* __restrict__ xb" + std::to_string(b) + vw.psfx + " = " + R.param(vw.bufs[b]) + ";");
                k.s << l1.str();
            }
        }
        // epilogue operands of each row, requested behind the weights (single-segment launches)
        std::vector<std::map<int, std::string>> epi_pre(RB);
        if (group.size() == 1 && paired < 0 && st0.epilogue >= 0)
            for (int q = 0; q < RB; q++) {
                std::vector<std::string> gc(st0.rank, "0");
                gc[P0.ndim] = "nn" + std::to_string(q);
                epi_pre[q] = prefetch_epilogue(R, k, d, st0.epilogue, gc);
            }
        k.s << adc.str() << wdc.str();
        for (int r = 0; r < SR; r++) k.line("float rpart" + std::to_string(r) + " = 0.0f;");
        for (int q = 0; q < RB; q++)
            for (int cs = 0; cs < SC; cs++) k.line("float acc" + std::to_string(q) + "_" + std::to_string(cs) + " = 0.0f;");
        for (int i = 0; i < KIq; i++) {
            const std::string is = std::to_string(i);
            if (affine) {
                for (int q = 0; q < RB; q++) k.line("float rr" + std::to_string(q) + "_" + is + " = 0.0f;");
                if (!aB[0][i].empty()) k.line("float xs_" + is + " = 0.0f;");
            }
            for (int j = 0; j < 8; j++) {
                std::string ij = std::to_string(i) + "_" + std::to_string(j);
                for (int cs = 0; cs < SC; cs++) k.line("float af" + std::to_string(cs) + "_" + ij + ";");
                k.line("{");
                k.indent++;
                R.memo.emplace_back();
                for (int l = 0; l < st0.n_leaves; l++)
                    if (l != P0.w) k.line("const float x" + std::to_string(l) + " = " + lvals[l][i][j] + ";");
                for (int cs = 0; cs < SC; cs++)
                    k.line("af" + std::to_string(cs) + "_" + ij + " = " + expr_without(R, k, c0.into[P0.cslots[cs]], P0.w, "x") + ";");
                for (int r = 0; r < SR; r++)
                    k.line("rpart" + std::to_string(r) + " += " + R.expr(k, c0.into[P0.rslots[r]], "x", "", "", "") + ";");
                R.memo.pop_back();
                k.indent--;
                k.line("}");
                if (affine) {
                    for (int q = 0; q < RB; q++) {
                        const std::string r = "rr" + std::to_string(q) + "_" + is;
                        k.line(r + " = fmaf(af0_" + ij + ", " + wvals[q][i][j] + ", " + r + ");");
                    }
                    if (!aB[0][i].empty()) k.line("xs_" + is + " += af0_" + ij + ";");
                    continue;
                }
                for (int q = 0; q < RB; q++)
                    for (int cs = 0; cs < SC; cs++) {
                        std::string a = "acc" + std::to_string(q) + "_" + std::to_string(cs);
                        k.line(a + " = fmaf(af" + std::to_string(cs) + "_" + ij + ", " + wvals[q][i][j] + ", " + a + ");");
                    }
            }
            if (affine)
                for (int q = 0; q < RB; q++) {
                    const std::string a = "acc" + std::to_string(q) + "_0";
                    k.line(a + " = fmaf(" + aA[q][i] + ", rr" + std::to_string(q) + "_" + is + ", " + a + ");");
                    if (!aB[q][i].empty())
                        k.line(a + " = fmaf(" + std::string(negB ? "-" : "") + aB[q][i] + ", xs_" + is + ", " + a + ");");
                }
        }
        // keep the prefetched epilogue operands where they were requested (not sunk into the
        // finishing thread's branch)
        for (auto& m : epi_pre)
            for (auto& kv : m) k.line("asm volatile(\"\" :: \"v\"(" + kv.second + "));");
        // wave partials -> LDS -> one thread per row finishes it
        std::vector<std::string> parts;
        for (int q = 0; q < RB; q++)
            for (int cs = 0; cs < SC; cs++) parts.push_back("acc" + std::to_string(q) + "_" + std::to_string(cs));
        for (int r = 0; r < SR; r++) parts.push_back("rpart" + std::to_string(r));
        for (size_t i = 0; i < parts.size(); i++) {
            k.line(parts[i] + " = sanic_wave_sum(" + parts[i] + ");");
        }
        k.line("if (lane == 0) {");
        for (size_t i = 0; i < parts.size(); i++) k.line("  red[wv][" + std::to_string(i) + "] = " + parts[i] + ";");
        k.line("}");
        k.line("__syncthreads();");
        auto sum4 = [&](int i) {
            std::string is = std::to_string(i);
            return "((red[0][" + is + "] + red[1][" + is + "]) + red[2][" + is + "]) + red[3][" + is + "]";
        };
        auto finish_row = [&](Code& c, int q, int g) -> std::string {
            std::string qs = std::to_string(q);
            c.line("const idx_t nn = nn" + qs + ";");
            std::string arr = "const float accq[" + std::to_string(SC) + "] = {";
            for (int cs = 0; cs < SC; cs++) arr += (cs ? ", " : "") + sum4(q * SC + cs);
            c.line(arr + "};");
            for (int r = 0; r < SR; r++) c.line("const float racc" + std::to_string(r) + " = " + sum4(RB * SC + r) + ";");
            R.memo.emplace_back();
            for (auto& kv : epi_pre[q]) R.subst[kv.first] = kv.second;
            std::string v = gemv_finish(R, c, d, group[g], !tails.empty());
            for (auto& kv : epi_pre[q]) R.subst.erase(kv.first);
            R.memo.pop_back();
            return v;
        };
        if (paired >= 0) for (int u = 0; u < RBI; u++) {
            const std::string q0s = std::to_string(u * NSEG);
            k.line("if (t == " + std::to_string(u) + " && live" + q0s + ") {");
            k.indent++;
            k.line("const idx_t wi = nn" + q0s + ";");
            const sanic_stage& pst = d->stages[paired];
            std::map<int, std::string> outv;
            for (int g = 0; g < NSEG; g++) {
                const int q = u * NSEG + g;
                std::string gs = std::to_string(g);
                k.line("float pv" + gs + ";");
                k.line("{");
                k.indent++;
                std::string v = finish_row(k, q, g);
                k.line("pv" + gs + " = " + v + ";");
                k.indent--;
                k.line("}");
                outv[d->stages[group[g].stage].out_buffer] = "pv" + gs;
            }
            std::vector<int> stack{pst.value};
            while (!stack.empty()) {
                int ni = stack.back();
                stack.pop_back();
                const sanic_node& n = d->nodes[ni];
                if (n.kind == SANIC_NODE_INPUT) {
                    auto it = outv.find(n.buffer);
                    if (it != outv.end()) R.subst[ni] = it->second;
                }
                for (int kk = 0; kk < n.n_in; kk++) stack.push_back(n.in[kk]);
            }
            R.memo.emplace_back();
            std::string pv = R.value(k, pst.value, {"wi"});
            R.memo.pop_back();
            R.subst.clear();
            k.line(store_stmt(R.param(pst.out_buffer), "wi", pst.out_dtype, pv, !tails.empty(), d->buffers[pst.out_buffer].scale));
            k.indent--;
            k.line("}");
        } else {
            for (int q = 0; q < RB; q++) {
                std::string qs = std::to_string(q);
                k.line("if (t == " + qs + " && live" + qs + ") {");
                k.indent++;
                for (size_t g = 0; g < group.size(); g++) {
                    k.line(std::string(g ? "} else " : "") + "if (seg" + qs + " == " + std::to_string(g) + ") {");
                    k.indent++;
                    finish_row(k, q, (int)g);
                    k.indent--;
                }
                k.line("}");
                k.indent--;
                k.line("}");
            }
        }
        if (!tails.empty())
            emit_tail(R, k, d, tails, "(unsigned*)a.scratch", "gridDim.x");
        const std::string kname = "sanic_gemv_" + std::to_string(NTOT) + "x" + std::to_string(K);
        std::ostringstream src;
        src << kPrelude << R.args_struct(tails.empty() ? std::vector<std::string>{} : std::vector<std::string>{"float* __restrict__ scratch"})
            << "extern \"C\" __global__ void __launch_bounds__(256) " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
        LoweredStage L;
        L.kernel_kind = "skeleton:gemv" + std::string(group.size() > 1 ? "[batched " + std::to_string(group.size()) + "]" : "") +
                        (paired >= 0 ? "+paired" : "") + (tails.empty() ? "" : "+tail" + std::to_string(tails.size()));
        // machine-scheduler strategy by shape (decode-step means of five runs each): the
        // memory-clause form keeps the weight loads of large GEMVs together (gate/up, lm_head:
        // 652.5 → 648.5 µs); long rows (K ≥ 4096, the down projection) and packed 4-bit weights,
        // whose nibble decoding adds arithmetic per load, prefer the ILP form (648.6 → 646.9 µs
        // together with the next rule; D1 5.17 → 5.0 µs); small GEMVs (≤ 8 Mi weights: q/k/v, o)
        // keep the default
        const char* strat = packed4 || K >= 4096 ? "iterative-ilp" : NTOT * K <= (int64_t(8) << 20) ? nullptr : "max-memory-clause";
        L.source = (strat ? std::string("// sched-strategy: ") + strat + "\n" : std::string()) + src.str();
        L.variants = nvar;
        std::vector<Arg> args = R.arg_list();
        if (!tails.empty()) args.push_back({Arg::SCRATCH, counter_off});   // the tail counter: relative offset 0
        L.launches.push_back({kname, "", dim3((unsigned)nblocks), dim3(256), 0, args});
        out.push_back(std::move(L));
        for (size_t g = 1; g < group.size(); g++) {
            LoweredStage B;
            B.kernel_kind = "batched-into:" + std::to_string(si);
            out.push_back(std::move(B));
        }
        if (paired >= 0) {
            LoweredStage B;
            B.kernel_kind = "paired-into:" + std::to_string(si);
            out.push_back(std::move(B));
        }
        for (size_t t = 0; t < tails.size(); t++) {
            LoweredStage B;
            B.kernel_kind = "tail-of:" + std::to_string(si);
            out.push_back(std::move(B));
        }
        return true;
    }

    Code k;
    k.indent = 1;
    k.line("extern __shared__ float u_lds[];");
    k.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
    k.line("const idx_t nwaves = (idx_t)gridDim.x * 4;");
    k.line("idx_t r0 = ((idx_t)blockIdx.x * 4 + wv) * " + std::to_string(RQ) + ";");
    for (int i = 0; i < SR; i++) k.line("float racc" + std::to_string(i) + " = 0.0f;");

    // row setup: segment, local row, weight pointers (rows past the end read row 0, unused)
    auto setup = [&](Code& c) {
        for (int q = 0; q < RQ; q++) {
            std::string qs = std::to_string(q);
            if (paired >= 0)
                c.line("const idx_t row" + qs + " = r0 / " + std::to_string(RQ) + " + " + std::to_string(q * P0.N) + ";");
            else
                c.line("const idx_t row" + qs + " = r0 + " + qs + ";");
            c.line("const bool live" + qs + " = row" + qs + " < " + std::to_string(NTOT) + ";");
            c.line("int seg" + qs + " = 0;");
            for (size_t g = 1; g < group.size(); g++)
                c.line("if (row" + qs + " >= " + std::to_string(seg_off[g]) + ") seg" + qs + " = " + std::to_string(g) + ";");
            std::string nnexpr = "row" + qs;
            for (size_t g = 1; g < group.size(); g++)
                nnexpr = "(seg" + qs + " == " + std::to_string(g) + " ? row" + qs + " - " + std::to_string(seg_off[g]) + " : " + nnexpr + ")";
            c.line("const idx_t nn" + qs + " = live" + qs + " ? " + nnexpr + " : 0;");
            for (size_t b = 0; b < wb0.size(); b++) {
                std::string sel = R.param(seg_wbufs[0][b]);
                for (size_t g = 1; g < group.size(); g++)
                    sel = "(seg" + qs + " == " + std::to_string(g) + " ? " + R.param(seg_wbufs[g][b]) + " : " + sel + ")";
                c.line("const " + std::string(ctype_of(wd0[b])) + "* __restrict__ wb" + std::to_string(b) + "_" + qs + " = " + sel + ";");
            }
        }
    };
    // weight loads for every (row, run) and their decode + FMA against the LDS factors
    std::vector<std::vector<std::vector<std::string>>> wv_(RQ, std::vector<std::vector<std::string>>(KI));
    auto loads = [&](Code& lc, Code& dc) {
        for (int q = 0; q < RQ; q++)
            for (int i = 0; i < KI; i++) {
                VecW vw{d};
                vw.nn = "nn" + std::to_string(q);
                vw.k0 = "(" + std::to_string(i * 512) + " + lane * 8)";
                vw.ptr = "wb";
                vw.psfx = "_" + std::to_string(q);          // pointer names carry the row
                vw.sfx = "_" + std::to_string(q) + "_" + std::to_string(i);
                Code l1, d1;
                auto vals = vw.render(l1, d1, d->stages[P0.stage].leaf[P0.w], weight_coords(d, d->stages[P0.stage], P0.w, P0.ndim),
                                      {P0.N, P0.K});
                std::string ls = l1.str(), ds = d1.str();
                bool guard = K % 512 != 0 && (int64_t)(i + 1) * 512 > K;
                if (guard) {
                    lc.line("const bool in_" + std::to_string(q) + "_" + std::to_string(i) + " = " + std::to_string(i * 512) + " + lane * 8 < " + std::to_string(K) + ";");
                    // clamp the run inside the row: the lane's contribution is dropped below
                    std::string k0c = "(" + std::to_string(i * 512) + " + lane * 8 < " + std::to_string(K) + " ? " + std::to_string(i * 512) + " + lane * 8 : 0)";
                    size_t pos = 0;
                    std::string from = vw.k0;
                    while ((pos = ls.find(from, pos)) != std::string::npos) { ls.replace(pos, from.size(), k0c); pos += k0c.size(); }
                }
                lc.s << ls;
                dc.s << ds;
                wv_[q][i] = vals;
            }
    };
    auto fma_all = [&](Code& c) {
        for (int i = 0; i < KI; i++) {
            bool guard = K % 512 != 0 && (int64_t)(i + 1) * 512 > K;
            std::string is = std::to_string(i);
            c.line("{");
            c.indent++;
            c.line("const int kk = " + std::to_string(i * 512) + " + lane * 8;");
            for (int cs = 0; cs < SC; cs++) {
                std::string css = std::to_string(cs);
                c.line("const float4 ua" + css + " = *(const float4*)(u_lds + " + css + " * " + std::to_string(K) + " + (kk < " + std::to_string(K) + " ? kk : 0));");
                c.line("const float4 ub" + css + " = *(const float4*)(u_lds + " + css + " * " + std::to_string(K) + " + (kk < " + std::to_string(K) + " ? kk : 0) + 4);");
            }
            for (int q = 0; q < RQ; q++) {
                const char* comp[4] = {"x", "y", "z", "w"};
                for (int cs = 0; cs < SC; cs++) {
                    std::string css = std::to_string(cs);
                    std::string acc = "acc" + std::to_string(q) + "_" + css;
                    std::string sum = acc;
                    for (int j = 0; j < 8; j++)
                        sum = "fmaf(" + std::string(j < 4 ? "ua" : "ub") + css + "." + comp[j % 4] + ", " + wv_[q][i][j] + ", " + sum + ")";
                    if (guard) c.line("if (in_" + std::to_string(q) + "_" + is + ") " + acc + " = " + sum + ";");
                    else c.line(acc + " = " + sum + ";");
                }
            }
            c.indent--;
            c.line("}");
        }
    };
    auto finish = [&](Code& c) {
        if (paired >= 0) {
            for (int q = 0; q < RQ; q++)
                for (int cs = 0; cs < SC; cs++) {
                    std::string a = "acc" + std::to_string(q) + "_" + std::to_string(cs);
                    c.line(a + " = sanic_wave_sum(" + a + ");");
                }
            c.line("if (lane == 0 && live0) {");
            c.indent++;
            c.line("const idx_t wi = nn0;");
            const sanic_stage& pst = d->stages[paired];
            std::map<int, std::string> outv;      // segment output buffer -> its value in this wave
            for (int q = 0; q < RQ; q++) {
                std::string qs = std::to_string(q);
                c.line("float pv" + qs + ";");
                c.line("{");
                c.indent++;
                c.line("const idx_t nn = nn" + qs + ";");
                std::string arr = "const float accq[" + std::to_string(SC) + "] = {";
                for (int cs = 0; cs < SC; cs++) arr += (cs ? ", acc" : "acc") + qs + "_" + std::to_string(cs);
                c.line(arr + "};");
                R.memo.emplace_back();
                std::string v = gemv_finish(R, c, d, group[q], !tails.empty());
                R.memo.pop_back();
                c.line("pv" + qs + " = " + v + ";");
                c.indent--;
                c.line("}");
                outv[d->stages[group[q].stage].out_buffer] = "pv" + qs;
            }
            // the consumer's inputs that are group outputs read this wave's values
            std::vector<int> stack{pst.value};
            while (!stack.empty()) {
                int ni = stack.back();
                stack.pop_back();
                const sanic_node& n = d->nodes[ni];
                if (n.kind == SANIC_NODE_INPUT) {
                    auto it = outv.find(n.buffer);
                    if (it != outv.end()) R.subst[ni] = it->second;
                }
                for (int kk = 0; kk < n.n_in; kk++) stack.push_back(n.in[kk]);
            }
            R.memo.emplace_back();
            std::string pv = R.value(c, pst.value, {"wi"});
            R.memo.pop_back();
            R.subst.clear();
            c.line(store_stmt(R.param(pst.out_buffer), "wi", pst.out_dtype, pv, !tails.empty(), d->buffers[pst.out_buffer].scale));
            c.indent--;
            c.line("}");
            return;
        }
        for (int q = 0; q < RQ; q++)
            for (int cs = 0; cs < SC; cs++) {
                std::string a = "acc" + std::to_string(q) + "_" + std::to_string(cs);
                c.line(a + " = sanic_wave_sum(" + a + ");");
            }
        c.line("if (lane == 0) {");
        c.indent++;
        for (int q = 0; q < RQ; q++) {
            std::string qs = std::to_string(q);
            c.line("if (live" + qs + ") {");
            c.indent++;
            c.line("const idx_t nn = nn" + qs + ";");
            std::string arr = "const float accq[" + std::to_string(SC) + "] = {";
            for (int cs = 0; cs < SC; cs++) arr += (cs ? ", acc" : "acc") + qs + "_" + std::to_string(cs);
            c.line(arr + "};");
            for (size_t g = 0; g < group.size(); g++) {
                c.line(std::string(g ? "} else " : "") + "if (seg" + qs + " == " + std::to_string(g) + ") {");
                c.indent++;
                R.memo.emplace_back();
                gemv_finish(R, c, d, group[g], !tails.empty());
                R.memo.pop_back();
                c.indent--;
            }
            c.line("}");
            c.indent--;
            c.line("}");
        }
        c.indent--;
        c.line("}");
    };
    auto iteration = [&](Code& c, bool first) {
        setup(c);
        for (int q = 0; q < RQ; q++)
            for (int cs = 0; cs < SC; cs++) c.line("float acc" + std::to_string(q) + "_" + std::to_string(cs) + " = 0.0f;");
        Code lc, dc;
        lc.indent = dc.indent = c.indent;
        loads(lc, dc);
        c.s << lc.str();
        if (first) {
            // the row prologue runs while this iteration's weight loads are in flight
            // constant trip count, fully unrolled: every prologue load is issued up front
            c.line("#pragma unroll");
            c.line("for (int it = 0; it < " + std::to_string((K + 255) / 256) + "; ++it) {");
            c.line("  const idx_t k = t + (idx_t)it * 256;");
            if (K % 256) c.line("  if (k < " + std::to_string(K) + ") {");
            c.s << prologue;
            if (K % 256) c.line("  }");
            c.line("}");
            if (SR > 0) {
                c.line("float* red = u_lds + " + std::to_string(SC * K) + ";");
                for (int i = 0; i < SR; i++) {
                    c.line("racc" + std::to_string(i) + " = sanic_wave_sum(racc" + std::to_string(i) + ");");
                    c.line("if (lane == 0) red[wv * " + std::to_string(SR) + " + " + std::to_string(i) + "] = racc" + std::to_string(i) + ";");
                }
            }
            c.line("__syncthreads();");
            for (int i = 0; i < SR; i++)
                c.line("racc" + std::to_string(i) + " = ((red[" + std::to_string(i) + "] + red[" + std::to_string(SR + i) + "]) + red[" +
                       std::to_string(2 * SR + i) + "]) + red[" + std::to_string(3 * SR + i) + "];");
        }
        c.s << dc.str();
        fma_all(c);
        finish(c);
    };
    k.line("{");
    k.indent++;
    iteration(k, true);
    k.indent--;
    k.line("}");
    k.line("for (r0 += nwaves * " + std::to_string(RQ) + "; r0 < " + std::to_string(NTOT) + "; r0 += nwaves * " + std::to_string(RQ) + ") {");
    k.indent++;
    iteration(k, false);
    k.indent--;
    k.line("}");
    if (!tails.empty())
        emit_tail(R, k, d, tails, "(unsigned*)a.scratch", "gridDim.x");

    // kernel names carry the shape so profiles tell the launches apart
    const std::string kname = "sanic_gemv_" + std::to_string(NTOT) + "x" + std::to_string(K);
    std::ostringstream src;
    src << kPrelude << R.args_struct(tails.empty() ? std::vector<std::string>{} : std::vector<std::string>{"float* __restrict__ scratch"})
        << "extern \"C\" __global__ void __launch_bounds__(256) " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
    LoweredStage L;
    L.kernel_kind = "skeleton:gemv" + std::string(group.size() > 1 ? "[batched " + std::to_string(group.size()) + "]" : "") +
                    (paired >= 0 ? "+paired" : "") +
                    (tails.empty() ? "" : "+tail" + std::to_string(tails.size()));
    L.source = src.str();
    uint32_t lds = (uint32_t)((SC * K + 4 * std::max(SR, 1)) * 4);
    std::vector<Arg> args = R.arg_list();
    if (!tails.empty()) args.push_back({Arg::SCRATCH, counter_off});   // the tail counter: relative offset 0
    L.launches.push_back({kname, "", dim3((unsigned)blocks), dim3(256), lds, args});
    out.push_back(std::move(L));
    for (size_t g = 1; g < group.size(); g++) {
        LoweredStage B;
        B.kernel_kind = "batched-into:" + std::to_string(si);
        out.push_back(std::move(B));
    }
    if (paired >= 0) {
        LoweredStage B;
        B.kernel_kind = "paired-into:" + std::to_string(si);
        out.push_back(std::move(B));
    }
    for (size_t t = 0; t < tails.size(); t++) {
        LoweredStage B;
        B.kernel_kind = "tail-of:" + std::to_string(si);
        out.push_back(std::move(B));
    }
    return true;
}

bool lower_pointwise_skeleton(const sanic_program_desc* d, int si, int64_t&, LoweredStage& out) {
    int dim, pos;
    int64_t work = pointwise_work(d, si, dim, pos);
    if (dim < 0) return false;
    Renderer R(d);
    Code body;
    body.indent = 1;
    emit_pointwise_loop(R, body, d, si, "((idx_t)blockIdx.x * 256 + threadIdx.x)", (int)std::min<int64_t>(work, 1 << 30));
    std::ostringstream src;
    src << kPrelude << R.args_struct({}) << "extern \"C\" __global__ void __launch_bounds__(256) sanic_rowwrite(Args a) {\n"
        << R.entry() << body.str() << "}\n";
    out.kernel_kind = "skeleton:rowwrite";
    out.source = src.str();
    out.launches.push_back({"sanic_rowwrite", "", dim3((unsigned)((work + 255) / 256)), dim3(256), 0, R.arg_list()});
    return true;
}

// ───────────────────────── gemv over N-contiguous weights ──────────────────────────────────
// y[n] = project(Σ_k into(x(k), W[k, n])) with W stored [K, N] (the K-major layout of the
// RMSNorm-fused projection's configuration): each lane owns 8 adjacent columns (one 16-byte
// load per k row), a workgroup covers 512 columns × a K slice whose rows its 4 waves split,
// the waves meet in LDS, and the workgroups of a column group meet through f32 partials in
// scratch: the last one to arrive adds the K slices in order, folds the row slots (Σx², …)
// over the whole of K itself, projects, runs the epilogue and stores.
bool lower_gemv_kmajor(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    GemvPlan P;
    if (getenv("SANIC_HIP_GENERIC") || !gemv_plan(d, si, P, true)) return false;
    const sanic_stage& st = d->stages[si];
    const sanic_carrier& c = st.carrier;
    const int64_t N = P.N, K = P.K;
    // Strip form: a workgroup owns SW columns over K / KSL rows. The activation factors of every k
    // (and the row slots, over the whole K) are computed once into LDS; lane l reads 8 columns
    // (16 bytes) of row (l / (SW/8)) of each row step, the 8 waves take an eighth of the slice
    // each; lanes of one column group meet by shuffles, waves in LDS.
    //   variant 0: 128-column strips (256 contiguous bytes per row) over four K slices; the slices
    //     of a strip sit on one XCD (blockIdx b, b + 8, ...) and meet through scratch: the last
    //     arrival adds them in slice order (deterministic) and finishes. B1 (2048 × 8192):
    //     11.3 µs, against 12.3 for variant 1, 12.4 for 64 × 2 and 11.9 for 256 × 8 — longer
    //     contiguous runs per row help; whole 128-byte lines alone (64 × 2) do not.
    //   variant 1: 32-column strips over the whole K (no merge); workgroups b and b + 8 own
    //     adjacent strips so the two halves of a 128-byte line are read through the same L2.
    //   variants 2, 3: 64 / 256-column strips over 2 / 8 K slices.
    static const int kStrip[][2] = {{128, 4}, {32, 1}, {64, 2}, {256, 8}};   // (columns, K slices)
    const int kvar = st.sched.variant > 0 && st.sched.variant < 4 ? st.sched.variant : 0;
    const int SW = kStrip[kvar][0];               // strip width (columns)
    const int KSL = kStrip[kvar][1];              // K slices per strip
    const int NT = 512;                           // 8 waves: 16 row loads per lane
    const int LPR = SW / 8, RPS = 64 / LPR, NWV = NT / 64;   // lanes per row, rows per step, waves
    if (N % (SW * 8) == 0 && K % (RPS * NWV * KSL) == 0 && K <= 8192) {
        const int SC = (int)P.cslots.size(), SR = (int)P.rslots.size();
        const int64_t NS = N / SW, KH = K / KSL, KQ = KH / NWV, IT = KQ / RPS;   // strips, slice rows, rows per wave, row steps
        const bool xl = KSL > 1 && xcd_local_enabled();
        int64_t part_off = 0, counter_off = 0;
        if (KSL > 1) {
            part_off = scratch;
            scratch += ((KSL * SC * N * 4 + 255) / 256) * 256;
            counter_off = scratch;
            scratch += ((NS * 4 + 255) / 256) * 256;
        }
        Renderer R(d);
        Code k;
        k.indent = 1;
        k.line("__shared__ float fl[" + std::to_string(std::max(SC, 1)) + "][" + std::to_string(K) + "];");
        k.line("__shared__ __attribute__((aligned(16))) float red[" + std::to_string(NWV) + "][" + std::to_string(SC * SW) + "];");
        if (SR) k.line("__shared__ float rred[" + std::to_string(NWV) + "][" + std::to_string(SR) + "];");
        k.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
        k.line("const idx_t strip = (blockIdx.x % 8) * " + std::to_string(NS / 8) + " + (blockIdx.x / 8) / " + std::to_string(KSL) + ";");
        k.line("const idx_t slice = (blockIdx.x / 8) % " + std::to_string(KSL) + ";");
        k.line("const idx_t n0 = strip * " + std::to_string(SW) + " + (lane & " + std::to_string(LPR - 1) + ") * 8;");
        const std::string krow0 = "(slice * " + std::to_string(KH) + " + (idx_t)wv * " + std::to_string(KQ) + ")";
        // the row leaves' values of this thread's K / NT rows are requested first, then the
        // weight loads (every row step of this lane), then the LDS prologue on those values: it
        // waits only for the earliest requests, so it runs while the weights are in flight
        const int64_t PR = (K + NT - 1) / NT;     // prologue rows per thread (the last partial)
        auto pro_row = [&](int64_t i) {
            const std::string r = "(t + " + std::to_string(i * NT) + ")";
            return (i + 1) * NT <= K ? r : "(" + r + " < " + std::to_string(K) + " ? " + r + " : 0)";
        };
        for (int64_t i = 0; i < PR; i++) {
            const std::string kr = pro_row(i);
            R.memo.emplace_back();
            for (int l = 0; l < st.n_leaves; l++) {
                if (l == P.w) continue;
                const sanic_node& ln = d->nodes[st.leaf[l]];
                std::vector<std::string> lc(ln.rank);
                for (int j = 0; j < ln.rank; j++) lc[j] = st.bind[l][j] == SANIC_BIND_STREAM ? kr : "0";
                k.line("const float x" + std::to_string(l) + "_p" + std::to_string(i) + " = " + R.value(k, st.leaf[l], lc) + ";");
            }
            R.memo.pop_back();
        }
        std::vector<std::vector<std::string>> wv_(IT);
        Code wdc;
        wdc.indent = k.indent;
        for (int64_t i = 0; i < IT; i++) {
            VecW vw{d};
            vw.nn = "(" + krow0 + " + " + std::to_string(i * RPS) + " + (lane / " + std::to_string(LPR) + "))";
            vw.k0 = "n0";
            vw.ptr = "wb";
            vw.psfx = "";
            vw.sfx = "_" + std::to_string(i);
            Code l1;
            l1.indent = k.indent;
            wv_[i] = vw.render(l1, wdc, st.leaf[P.w], weight_coords(d, st, P.w, P.ndim, true), {K, N});
            if (!vw.ok) return false;
            if (i == 0)
                for (size_t b = 0; b < vw.bufs.size(); b++)
                    k.line("const " + std::string(ctype_of(vw.dtypes[b])) + "* __restrict__ wb" + std::to_string(b) + " = " + R.param(vw.bufs[b]) + ";");
            // one bf16 weight buffer under 4 GB: 32-bit byte offsets from its uniform base (one
            // address register per load instead of two, so every row's request issues before
            // the prologue's first wait)
            std::string ls = l1.str();
            if (vw.bufs.size() == 1 && vw.dtypes[0] == SANIC_BF16 && K * N * 2 < (int64_t(1) << 32)) {
                ls = std::regex_replace(ls, std::regex("const idx_t (ad\\w+) = "), "const unsigned $1 = ");
                ls = std::regex_replace(ls, std::regex(R"(\(wb0 \+ (ad\w+)\))"), "((const unsigned short*)((const char*)wb0 + $1 * 2u))");
            }
            k.s << ls;
        }
        // activation factors of every k into LDS; this workgroup's row slots (after the weight
        // requests: the scheduler would otherwise hoist this arithmetic, and its waits, above them)
        k.line("__builtin_amdgcn_sched_barrier(0);");
        for (int r = 0; r < SR; r++) k.line("float rpart" + std::to_string(r) + " = 0.0f;");
        for (int64_t i = 0; i < PR; i++) {
            const std::string kr = "(t + " + std::to_string(i * NT) + ")", ps = "_p" + std::to_string(i);
            R.memo.emplace_back();
            auto item = [&](int it) { return "x" + std::to_string(it) + ps; };
            k.line((i + 1) * NT <= K ? "{" : "if (" + kr + " < " + std::to_string(K) + ") {");
            for (int l = 0; l < st.n_leaves; l++)
                if (l != P.w) k.line("  const float x" + std::to_string(l) + " = " + item(l) + ";");
            for (int cs = 0; cs < SC; cs++)
                k.line("  fl[" + std::to_string(cs) + "][" + kr + "] = " + expr_without(R, k, c.into[P.cslots[cs]], P.w, "x") + ";");
            for (int r = 0; r < SR; r++) k.line("  rpart" + std::to_string(r) + " += " + R.expr(k, c.into[P.rslots[r]], "x", "", "", "") + ";");
            k.line("}");
            R.memo.pop_back();
        }
        for (int r = 0; r < SR; r++) {
            std::string rs = std::to_string(r);
            k.line("rpart" + rs + " = sanic_wave_sum(rpart" + rs + ");");
            k.line("if (lane == 0) rred[wv][" + rs + "] = rpart" + rs + ";");
        }
        k.line("__syncthreads();");
        k.s << wdc.str();
        for (int cs = 0; cs < SC; cs++)
            for (int j = 0; j < 8; j++) k.line("float acc" + std::to_string(cs) + "_" + std::to_string(j) + " = 0.0f;");
        for (int64_t i = 0; i < IT; i++) {
            const std::string kr = "(int)(" + krow0 + " + " + std::to_string(i * RPS) + " + (lane / " + std::to_string(LPR) + "))";
            for (int cs = 0; cs < SC; cs++) {
                const std::string f = "f" + std::to_string(cs) + "_" + std::to_string(i);
                k.line("const float " + f + " = fl[" + std::to_string(cs) + "][" + kr + "];");
                for (int j = 0; j < 8; j++) {
                    std::string a = "acc" + std::to_string(cs) + "_" + std::to_string(j);
                    k.line(a + " = fmaf(" + f + ", " + wv_[i][j] + ", " + a + ");");
                }
            }
        }
        // the 16 row lanes of each column group, then the 4 waves
        for (int cs = 0; cs < SC; cs++)
            for (int j = 0; j < 8; j++) {
                std::string a = "acc" + std::to_string(cs) + "_" + std::to_string(j);
                k.line(a + " = " + (LPR == 4 ? "sanic_stride4_sum(" : LPR == 8 ? "sanic_stride8_sum(" : LPR == 16 ? "sanic_rows_sum(" : "sanic_half_sum(") + a + ");");
            }
        k.line("if (lane < " + std::to_string(LPR) + ") {");
        for (int cs = 0; cs < SC; cs++) {
            std::string css = std::to_string(cs), base = css + " * " + std::to_string(SW);
            k.line("  *(sanic_f32x4*)(&red[wv][" + base + " + lane * 8]) = (sanic_f32x4){acc" + css + "_0, acc" + css + "_1, acc" + css + "_2, acc" + css + "_3};");
            k.line("  *(sanic_f32x4*)(&red[wv][" + base + " + lane * 8 + 4]) = (sanic_f32x4){acc" + css + "_4, acc" + css + "_5, acc" + css + "_6, acc" + css + "_7};");
        }
        k.line("}");
        k.line("__syncthreads();");
        auto wave_sum_of = [&](int cs) {
            std::string i = std::to_string(cs) + " * " + std::to_string(SW) + " + t", sum = "red[0][" + i + "]";
            for (int w = 1; w < NWV; w++) sum = "(" + sum + " + red[" + std::to_string(w) + "][" + i + "])";
            return sum;
        };
        if (KSL > 1) {
            // this slice's column sums to scratch, then the later of the strip's workgroups
            // finishes: the slices' partials added in slice order
            k.line("if (t < " + std::to_string(SW) + ") {");
            // (the slices of a strip share blockIdx mod 8, i.e. one XCD: through its L2)
            for (int cs = 0; cs < SC; cs++)
                k.line(std::string("  ") + (xl ? "sanic_stx" : "sanic_st") + "(a.scratch + " + std::to_string(part_off / 4) + " + (slice * " + std::to_string(SC) + " + " +
                       std::to_string(cs) + ") * " + std::to_string(N) + " + strip * " + std::to_string(SW) + " + t, " + wave_sum_of(cs) + ");");
            k.line("}");
            k.line("unsigned* cnt = (unsigned*)((char*)a.scratch + " + std::to_string(counter_off) + ") + strip;");
            emit_arrival(k, "sanic_last", "t", "cnt", std::to_string(KSL) + "u", xl);
            k.line("if (!sanic_last) return;");
            k.line("if (t == 0) sanic_st(cnt, 0u);");
        }
        k.line("if (t < " + std::to_string(SW) + ") {");
        k.indent++;
        k.line("const idx_t nn = strip * " + std::to_string(SW) + " + t;");
        std::string arr = "const float accq[" + std::to_string(std::max(SC, 1)) + "] = {";
        for (int cs = 0; cs < SC; cs++) {
            std::string sum;
            if (KSL > 1) {
                for (int q = 0; q < KSL; q++) {
                    std::string pq = std::string(xl ? "sanic_ldx" : "sanic_ld") + "(a.scratch + " + std::to_string(part_off / 4) + " + (" + std::to_string(q * SC + cs) + ") * " +
                                     std::to_string(N) + " + nn)";
                    sum = q ? "(" + sum + " + " + pq + ")" : pq;
                }
            } else {
                sum = wave_sum_of(cs);
            }
            arr += std::string(cs ? ", " : "") + sum;
        }
        if (SC == 0) arr += "0.0f";
        k.line(arr + "};");
        for (int r = 0; r < SR; r++) {
            std::string rs = std::to_string(r);
            std::string sum = "rred[0][" + rs + "]";
            for (int w = 1; w < NWV; w++) sum = "(" + sum + " + rred[" + std::to_string(w) + "][" + rs + "])";
            k.line("const float racc" + rs + " = " + sum + ";");
        }
        R.memo.emplace_back();
        gemv_finish(R, k, d, P, false);
        R.memo.pop_back();
        k.indent--;
        k.line("}");
        const std::string kname = "sanic_gemvt_" + std::to_string(N) + "x" + std::to_string(K);
        std::ostringstream src;
        src << kPrelude << R.args_struct(KSL > 1 ? std::vector<std::string>{"float* __restrict__ scratch"} : std::vector<std::string>{})
            << "extern \"C\" __global__ void __launch_bounds__(" << NT << ") " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
        out.kernel_kind = "skeleton:gemv_kmajor[strips " + std::to_string(SW) + (KSL > 1 ? " x" + std::to_string(KSL) + " slices" : "") + "]" + (xl ? "+xcd" : "");
        out.source = "// sched-strategy: max-memory-clause\n" + src.str();   // B1 12.26 → 12.07 µs
        out.variants = 4;
        std::vector<Arg> args = R.arg_list();
        if (KSL > 1) args.push_back({Arg::SCRATCH, 0});
        out.launches.push_back({kname, "", dim3((unsigned)(NS * KSL)), dim3((unsigned)NT), 0, args});
        return true;
    }
    if (N % 512 || K % 64) return false;
    const int SC = (int)P.cslots.size(), SR = (int)P.rslots.size();
    const int64_t NCG = N / 512;
    int64_t KS = std::max<int64_t>(1, std::min<int64_t>(K / 128, 128 / NCG));   // K slices
    while (K % KS || (K / KS) % 4) KS--;
    const int64_t KB = K / KS, KW = KB / 4;                                    // rows per slice / wave
    int64_t part_off = scratch;
    scratch += ((KS * SC * N * 4 + 255) / 256) * 256;
    int64_t rpart_off = scratch;                 // per-slice row-slot partials [NCG][KS][SR]
    scratch += ((NCG * KS * std::max(SR, 1) * 4 + 255) / 256) * 256;
    int64_t counter_off = scratch;
    scratch += ((NCG * 4 + 255) / 256) * 256;

    Renderer R(d);
    Code k;
    k.indent = 1;
    k.line("__shared__ __attribute__((aligned(16))) float red[4][" + std::to_string(SC * 512) + "];");
    k.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
    k.line("const idx_t cg = blockIdx.x % " + std::to_string(NCG) + ", ks = blockIdx.x / " + std::to_string(NCG) + ";");
    k.line("const idx_t n0 = cg * 512 + lane * 8;");
    k.line("const idx_t kbeg = ks * " + std::to_string(KB) + " + wv * " + std::to_string(KW) + ";");
    for (size_t b = 0; b < 1; b++) {}
    // weight runs: one per k row of this wave
    std::vector<std::vector<std::string>> wv_(KW);
    Code wdc;
    wdc.indent = k.indent;
    std::vector<int> wbufs, wdts;
    for (int64_t i = 0; i < KW; i++) {
        VecW vw{d};
        vw.nn = "(kbeg + " + std::to_string(i) + ")";
        vw.k0 = "n0";
        vw.ptr = "wb";
        vw.psfx = "";
        vw.sfx = "_" + std::to_string(i);
        Code l1;
        l1.indent = k.indent;
        wv_[i] = vw.render(l1, wdc, st.leaf[P.w], weight_coords(d, st, P.w, P.ndim, true), {K, N});
        if (!vw.ok) return false;
        if (i == 0) {
            wbufs = vw.bufs;
            wdts = vw.dtypes;
            for (size_t b = 0; b < wbufs.size(); b++)
                k.line("const " + std::string(ctype_of(wdts[b])) + "* __restrict__ wb" + std::to_string(b) + " = " + R.param(wbufs[b]) + ";");
        }
        k.s << l1.str();
    }
    k.s << wdc.str();
    // activation factors per k row (the same for every lane: broadcast loads)
    for (int cs = 0; cs < SC; cs++)
        for (int j = 0; j < 8; j++) k.line("float acc" + std::to_string(cs) + "_" + std::to_string(j) + " = 0.0f;");
    for (int r = 0; r < SR; r++) k.line("float rpart" + std::to_string(r) + " = 0.0f;");
    for (int64_t i = 0; i < KW; i++) {
        k.line("{");
        k.indent++;
        k.line("const idx_t kr = kbeg + " + std::to_string(i) + ";");
        R.memo.emplace_back();
        for (int l = 0; l < st.n_leaves; l++) {
            if (l == P.w) continue;
            const sanic_node& ln = d->nodes[st.leaf[l]];
            std::vector<std::string> lc(ln.rank);
            for (int j = 0; j < ln.rank; j++) lc[j] = st.bind[l][j] == SANIC_BIND_STREAM ? "kr" : "0";
            k.line("const float x" + std::to_string(l) + " = " + R.value(k, st.leaf[l], lc) + ";");
        }
        for (int cs = 0; cs < SC; cs++) {
            std::string f = expr_without(R, k, c.into[P.cslots[cs]], P.w, "x");
            for (int j = 0; j < 8; j++) {
                std::string a = "acc" + std::to_string(cs) + "_" + std::to_string(j);
                k.line(a + " = fmaf(" + f + ", " + wv_[i][j] + ", " + a + ");");
            }
        }
        // row slots of this wave's rows (every lane holds the same value)
        for (int r = 0; r < SR; r++) k.line("rpart" + std::to_string(r) + " += " + R.expr(k, c.into[P.rslots[r]], "x", "", "", "") + ";");
        R.memo.pop_back();
        k.indent--;
        k.line("}");
    }
    // waves -> LDS -> this slice's partial for 512 columns
    for (int cs = 0; cs < SC; cs++) {
        std::string css = std::to_string(cs);
        k.line("*(sanic_f32x4*)(&red[wv][" + css + " * 512 + lane * 8]) = (sanic_f32x4){acc" + css + "_0, acc" + css + "_1, acc" + css + "_2, acc" + css + "_3};");
        k.line("*(sanic_f32x4*)(&red[wv][" + css + " * 512 + lane * 8 + 4]) = (sanic_f32x4){acc" + css + "_4, acc" + css + "_5, acc" + css + "_6, acc" + css + "_7};");
    }
    if (SR > 0) {
        k.line("__shared__ float rred[4][" + std::to_string(SR) + "];");
        for (int r = 0; r < SR; r++) k.line("if (lane == 0) rred[wv][" + std::to_string(r) + "] = rpart" + std::to_string(r) + ";");
    }
    k.line("__syncthreads();");
    for (int r = 0; r < SR; r++) {
        std::string rs = std::to_string(r);
        k.line("if (t == 0) sanic_st(a.scratch + " + std::to_string(rpart_off / 4) + " + (cg * " + std::to_string(KS) + " + ks) * " + std::to_string(SR) + " + " + rs +
               ", ((rred[0][" + rs + "] + rred[1][" + rs + "]) + rred[2][" + rs + "]) + rred[3][" + rs + "]);");
    }
    k.line("for (int i = t; i < " + std::to_string(SC * 512) + "; i += 256) {");
    k.line("  const float v = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];");
    k.line("  const int cs = i / 512, col = i % 512;");
    k.line("  sanic_st(a.scratch + " + std::to_string(part_off / 4) + " + (ks * " + std::to_string(SC) + " + cs) * " + std::to_string(N) + " + cg * 512 + col, v);");
    k.line("}");
    k.line("unsigned* cnt = (unsigned*)((char*)a.scratch + " + std::to_string(counter_off) + ") + cg;");
    emit_arrival(k, "sanic_last", "t", "cnt", std::to_string(KS) + "u");
    k.line("if (!sanic_last) return;");
    k.line("if (t == 0) sanic_st(cnt, 0u);");
    // row slots: the K slices' partials, in slice order
    for (int r = 0; r < SR; r++) {
        std::string rs = std::to_string(r);
        k.line("float racc" + rs + " = 0.0f;");
        k.line("#pragma unroll");
        k.line("for (int q = 0; q < " + std::to_string(KS) + "; ++q) racc" + rs + " += sanic_ld(a.scratch + " + std::to_string(rpart_off / 4) + " + (cg * " +
               std::to_string(KS) + " + q) * " + std::to_string(SR) + " + " + rs + ");");
    }
    // the K slices of each column, in slice order; then project / epilogue / store
    k.line("for (int col = t; col < 512; col += 256) {");
    k.indent++;
    k.line("const idx_t nn = cg * 512 + col;");
    std::string arr = "float accq[" + std::to_string(SC) + "] = {";
    for (int cs = 0; cs < SC; cs++) arr += cs ? ", 0.0f" : "0.0f";
    k.line(arr + "};");
    k.line("float pv[" + std::to_string(KS * SC) + "];");
    k.line("#pragma unroll");
    k.line("for (int q = 0; q < " + std::to_string(KS * SC) + "; ++q) pv[q] = sanic_ld(a.scratch + " + std::to_string(part_off / 4) + " + (idx_t)q * " + std::to_string(N) + " + nn);");
    k.line("#pragma unroll");
    k.line("for (int q = 0; q < " + std::to_string(KS) + "; ++q)");
    k.line("  #pragma unroll");
    k.line("  for (int cs = 0; cs < " + std::to_string(SC) + "; ++cs) accq[cs] += pv[q * " + std::to_string(SC) + " + cs];");
    R.memo.emplace_back();
    gemv_finish(R, k, d, P, false);
    R.memo.pop_back();
    k.indent--;
    k.line("}");

    const std::string kname = "sanic_gemvt_" + std::to_string(N) + "x" + std::to_string(K);
    std::ostringstream src;
    src << kPrelude << R.args_struct({"float* __restrict__ scratch"})
        << "extern \"C\" __global__ void __launch_bounds__(256) " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
    out.kernel_kind = "skeleton:gemv_kmajor[" + std::to_string(KS) + " slices]";   // the strip form's fallback
    out.source = src.str();
    std::vector<Arg> args = R.arg_list();
    args.push_back({Arg::SCRATCH, 0});
    out.launches.push_back({kname, "", dim3((unsigned)(NCG * KS)), dim3(256), 0, args});
    return true;
}

bool lower_skeleton(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    if (lower_gemv_kmajor(d, si, scratch, out)) return true;
    if (lower_gemm(d, si, scratch, out)) return true;
    if (lower_flash_prefill(d, si, scratch, out)) return true;
    if (lower_attn_decode(d, si, scratch, out)) return true;
    return false;
}

}  // namespace sanic
