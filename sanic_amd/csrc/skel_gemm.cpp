// GEMM skeleton: Plain(Add) carriers with two output axes (rows m from the row leaves, columns
// n from the weight leaf) on bf16 MFMA (v_mfma_f32_16x16x32_bf16) — the RMSNorm-fused projection
// at prefill sizes and the int4 group-quantized matmul (configs B2/D2), i.e. the gemv carriers
// of skeletons.cpp when M is large enough to be a real contraction.
//
// Structure required: every slot Plain(Add); one weight leaf binding (n, stream); row leaves
// binding (m, stream) or (stream); each slot's `into` is either W·rest(row items) (a contraction
// slot: A = rest, B = W, both rounded to bf16 for the MFMA) or free of W (a row slot: Σx² of a
// fused RMSNorm, folded per row in f32 alongside the A tile).
//
// Kernel shape: workgroup tile BM × BN (8 waves in 4 × 2 for 128-row tiles at least 64 columns
// wide, else 4 waves in 2 × 2; each wave a block of 16×16 MFMA tiles), K in 64-wide steps, A and B tiles double-buffered in LDS with k contiguous so every
// MFMA operand is one ds_read_b128 (A planes written by a first launch skip LDS: stored in MFMA
// fragment order, each wave loads its A fragments directly); the weight leaf is loaded by the vector renderer (128-bit
// runs of 8 along k, per-group scale/zero once per run, packed nibbles decoded in registers);
// project, epilogue and the narrowing store per output element.
#include <algorithm>
#include <cmath>
#include <functional>
#include <set>

#include <regex>

#include "emit.h"
#include "skeletons.h"

namespace sanic {

namespace {

struct GemmPlan {
    int mdim = -1, ndim = -1;
    int64_t M = 0, N = 0, K = 0;
    int w = -1;
    std::vector<int> rows;          // row leaves
    std::vector<int> cslots, rslots;
};

bool expr_reads(const sanic_program_desc* d, int e, int item) {
    const sanic_expr& x = d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == item;
    if (x.op >= SANIC_EX_CONST) return false;
    for (int c : {x.a, x.b, x.c}) if (c >= 0 && expr_reads(d, c, item)) return true;
    return false;
}

bool linear_mul(const sanic_program_desc* d, int e, int w) {
    const sanic_expr& x = d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == w;
    if (x.op == SANIC_OP_MUL) {
        bool a = expr_reads(d, x.a, w), b = expr_reads(d, x.b, w);
        if (a == b) return false;
        return a ? linear_mul(d, x.a, w) : linear_mul(d, x.b, w);
    }
    return false;
}

// Render an Expr with item w read as 1 and items named by `item(i)`.
std::string expr_rest(Renderer& R, Code& code, int e, int w, const std::function<std::string(int)>& item) {
    const sanic_expr& x = R.d->exprs[e];
    if (x.op == SANIC_EX_ITEM) return x.index == w ? "1.0f" : item(x.index);
    if (x.op == SANIC_EX_CONST) return flit(x.value);
    std::string s[3];
    int kids[3] = {x.a, x.b, x.c};
    for (int k = 0; k < 3; k++) if (kids[k] >= 0) s[k] = expr_rest(R, code, kids[k], w, item);
    std::string out = R.fresh("e");
    code.line("const float " + out + " = " + map_expr(x.op, s[0], s[1], s[2]) + ";");
    return out;
}

bool gemm_plan(const sanic_program_desc* d, int si, GemmPlan& P) {
    const sanic_stage& st = d->stages[si];
    if (st.kind != SANIC_STAGE_FUSED) return false;
    const sanic_carrier& c = st.carrier;
    for (int k = 0; k < c.slots; k++)
        if (c.kind[k].kind != SANIC_SLOT_PLAIN || c.kind[k].monoid != SANIC_MON_ADD) return false;
    std::vector<int> big;
    for (int j = 0; j < st.rank; j++) if (st.grid[j] > 1) big.push_back(j);
    if (big.size() != 2 || st.stream % 64) return false;
    P = GemmPlan();
    P.K = st.stream;
    // leaves bound to a big grid dim (plus the stream); the rest depend on the stream only
    std::vector<std::pair<int, int>> dimmed;   // (leaf, dim)
    std::vector<int> free_rows;
    for (int l = 0; l < st.n_leaves; l++) {
        const sanic_node& ln = d->nodes[st.leaf[l]];
        std::set<int> dims;
        bool has_s = false;
        for (int j = 0; j < ln.rank; j++) {
            int b = st.bind[l][j];
            if (b == SANIC_BIND_STREAM) has_s = true;
            else if (b >= 0 && st.grid[b] > 1) dims.insert(b);
        }
        if (dims.size() > 1 || !has_s) return false;
        if (dims.empty()) free_rows.push_back(l);
        else dimmed.push_back({l, *dims.begin()});
    }
    // the weight is the one dim-bound leaf that every row slot ignores and every other slot
    // multiplies in exactly once; all other dim-bound leaves share the other (row) dim
    // Of the valid role assignments, prefer the one that recomputes the least: a side that is not
    // a stored bf16 value (x·g, a dequantized weight) is rebuilt by every workgroup along the
    // other output dim.
    GemmPlan best;
    int64_t best_cost = -1;
    auto raw_leaf = [&](int l) {
        const sanic_node& n = d->nodes[st.leaf[l]];
        return n.kind == SANIC_NODE_INPUT && n.dtype == SANIC_BF16;
    };
    for (auto& cand : dimmed) {
        GemmPlan Q = P;
        Q.w = cand.first;
        Q.ndim = cand.second;
        bool good = true;
        for (auto& o : dimmed) {
            if (o.first == cand.first) continue;
            if (o.second == Q.ndim || (Q.mdim >= 0 && o.second != Q.mdim)) { good = false; break; }
            Q.mdim = o.second;
            Q.rows.push_back(o.first);
        }
        if (!good || Q.mdim < 0) continue;
        for (int l : free_rows) Q.rows.push_back(l);
        for (int k = 0; k < c.slots && good; k++) {
            if (!expr_reads(d, c.into[k], Q.w)) Q.rslots.push_back(k);
            else if (linear_mul(d, c.into[k], Q.w)) Q.cslots.push_back(k);
            else good = false;
        }
        if (!good || Q.cslots.size() != 1) continue;
        bool a_raw = false;
        {
            const sanic_expr& e = d->exprs[c.into[Q.cslots[0]]];
            if (e.op == SANIC_OP_MUL) {
                const sanic_expr& ea = d->exprs[e.a];
                const sanic_expr& eb = d->exprs[e.b];
                const sanic_expr* other = nullptr;
                if (ea.op == SANIC_EX_ITEM && ea.index == Q.w) other = &eb;
                if (eb.op == SANIC_EX_ITEM && eb.index == Q.w) other = &ea;
                if (other && other->op == SANIC_EX_ITEM && raw_leaf(other->index)) a_raw = true;
            }
        }
        // element rebuilds: A (M×K) once per column block, B (N×K) once per row block
        const int64_t Mq = st.grid[Q.mdim], Nq = st.grid[Q.ndim];
        const int64_t cost = (a_raw ? 0 : Mq * ((Nq + 127) / 128)) + (raw_leaf(Q.w) ? 0 : Nq * ((Mq + 127) / 128));
        // ties: keep the stored bf16 operand on the A side (its tile needs no arithmetic)
        const int64_t key = cost * 2 + (a_raw ? 0 : 1);
        if (best_cost < 0 || key < best_cost) { best = Q; best_cost = key; }
    }
    P = best;
    if (P.w < 0) return false;
    P.M = st.grid[P.mdim];
    P.N = st.grid[P.ndim];
    if (P.cslots.size() != 1) return false;
    if (P.M < 64 || P.M % 64 || P.N % 32) return false;
    return true;
}

}  // namespace

// the vector weight renderer lives in skeletons.cpp
std::vector<std::string> render_weight_run(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                                           const std::vector<int64_t>& ext, Code& lc, Code& dc, const std::string& nn,
                                           const std::string& k0, const std::string& sfx, std::vector<int>& bufs,
                                           std::vector<int>& dtypes, bool& ok, bool& contiguous, std::string& raw_bf16,
                                           bool stream);

bool render_weight_affine(const sanic_program_desc* d, int node, const std::vector<Sym>& c,
                          const std::vector<int64_t>& ext, Code& lc, Code& dc, const std::string& nn,
                          const std::string& k0, const std::string& sfx, std::vector<int>& bufs,
                          std::vector<int>& dtypes, std::vector<std::string>& q, std::string& A, std::string& B,
                          bool& negB, int64_t& uniform_div, bool stream, bool raw_loads = false);

bool lower_gemm(const sanic_program_desc* d, int si, int64_t& scratch, LoweredStage& out) {
    GemmPlan P;
    if (!gemm_plan(d, si, P)) return false;
    const sanic_stage& st = d->stages[si];
    const sanic_carrier& c = st.carrier;
    const int64_t M = P.M, N = P.N, K = P.K;
    int BM = M % 128 == 0 ? 128 : 64;
    int BN = 128;
    while (BN > 32 && (M / BM) * (N / BN) < 256) BN /= 2;
    if (N % BN) return false;
    // 8 waves (4 × 2, two per SIMD) when the tile is 128 rows and at least 64 columns, so one
    // wave's LDS operand reads and global loads proceed under the other's MFMAs; else 4 (2 × 2)
    int NTH = (BM == 128 && BN >= 64) ? 512 : 256;
    const int SR = (int)P.rslots.size();
    // k-contiguous tiles: unpadded 128-byte rows (64 bf16) with the 16-byte chunk index XORed
    // by (row mod 8) — a 72-element padded stride 2-way bank-conflicts the 16-row operand reads
    // on gfx950
    const int AS = 64, BS = 64;               // LDS row strides (bf16)
    // element offset of (row, k) in a k-contiguous tile; k a multiple of 8
    auto koff = [&](const std::string& row, const std::string& k8, int) {
        return "(" + row + ") * 64 + (((" + k8 + ") / 8) ^ ((" + row + ") & 7)) * 8";
    };
    // An operand that is not a bf16 input as stored (x·g, dequantized weights) goes to the MFMA
    // as hi + lo bf16 pair (hi = rn(v), lo = rn(v − hi): 16 significant bits, exact for the
    // product of two bf16 values), so products match an f32 evaluation; one extra MFMA each.
    auto raw_bf16_input = [&](int leaf) {
        const sanic_node& n = d->nodes[st.leaf[leaf]];
        return n.kind == SANIC_NODE_INPUT && n.dtype == SANIC_BF16;
    };
    bool splitB = !raw_bf16_input(P.w);
    bool splitA = true;
    {
        const sanic_expr& e = d->exprs[c.into[P.cslots[0]]];
        if (e.op == SANIC_OP_MUL) {
            const sanic_expr& ea = d->exprs[e.a];
            const sanic_expr& eb = d->exprs[e.b];
            const sanic_expr* other = nullptr;
            if (ea.op == SANIC_EX_ITEM && ea.index == P.w) other = &eb;
            if (eb.op == SANIC_EX_ITEM && eb.index == P.w) other = &ea;
            if (other && other->op == SANIC_EX_ITEM && raw_bf16_input(other->index)) splitA = false;
        }
    }
    // A is one stored bf16 row leaf and no row slot reads it: its 16-byte runs go to LDS as
    // loaded (no unpack to f32 and repack)
    bool rawA = !splitA && P.rslots.empty() && P.rows.size() == 1;

    Renderer R(d);
    // weight leaf vector form over vars {0: n, 1: k}
    const sanic_node& wn = d->nodes[st.leaf[P.w]];
    std::vector<Sym> cw(wn.rank);
    for (int j = 0; j < wn.rank; j++) {
        int b = st.bind[P.w][j];
        cw[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.ndim ? Sym::var(0) : Sym();
    }
    std::vector<int> wbufs, wdts;
    bool ok = true, contig = true;
    std::string raw;
    {
        Code l1, d1;
        render_weight_run(d, st.leaf[P.w], cw, {N, K}, l1, d1, "nn", "k0", "_p", wbufs, wdts, ok, contig, raw, false);
        if (!ok) return false;
    }
    // N-contiguous weights ([K, N]): runs of 8 along n, the B tile kept [k][n] in LDS and read
    // transposed into the MFMA's k-major operand (ds_read_b64_tr_b16)
    std::vector<Sym> cwt(wn.rank);
    for (int j = 0; j < wn.rank; j++) {
        int b = st.bind[P.w][j];
        cwt[j] = b == SANIC_BIND_STREAM ? Sym::var(0) : b == P.ndim ? Sym::var(1) : Sym();
    }
    bool bkn = false;
    if (!contig) {
        std::vector<int> tb, td;
        bool tok = true, tc = true;
        std::string tr;
        Code l1, d1;
        render_weight_run(d, st.leaf[P.w], cwt, {K, N}, l1, d1, "kk", "n0", "_p", tb, td, tok, tc, tr, false);
        bkn = tok && tc;
    }
    // Grouped dequantization (packed 4-bit weights): the weight leaf is q·s ± z with q a packed
    // 4-bit run and s, z constant over every 64-wide K tile (a quantization group of 64 or a
    // multiple of it). Per tile, Σ_k x·w = s·Σ_k x·q ± z·Σ_k x, so the MFMA's B operand is q
    // itself — small integers, exact in bf16: one MFMA per fragment instead of a hi + lo pair,
    // and no dequantizing arithmetic ahead of the MFMAs — into a per-tile accumulator that the
    // lanes fold into the output with their column's s and z and the rows' Σ x (the int4
    // GEMV's per-run fold at tile granularity); Σ x comes from the matrix cores as well (the A
    // fragment times a fragment of ones), not from VALU adds. Oracle: the same sum over
    // w = q·s ± z in f64.
    bool grouped = false;
    bool gneg = false;
    if (splitB && !bkn && contig && K % 64 == 0 && P.rslots.empty() && P.rows.size() == 1) {
        std::vector<int> gb, gd;
        std::vector<std::string> qv;
        std::string A_, B_;
        int64_t ud = 0;
        Code l1, d1;
        grouped = render_weight_affine(d, st.leaf[P.w], cw, {N, K}, l1, d1, "nn", "k0", "_g", gb, gd, qv, A_, B_, gneg, ud, false) &&
                  ud % 64 == 0 && qv.size() == 8;
    }
    // [k][n] B tile row stride (bf16). The transposed operand read takes, per 32 lanes, 32
    // bytes of each of rows r..r+3 and r+8..r+11: a stride of 72 words puts rows r..r+3 on
    // disjoint 8-bank runs of the 64 banks, and flipping the 64-element half of the row for
    // rows with bit 3 set moves r+8..r+11 onto the other 32 banks (B2: LDS bank-conflict
    // cycles 2.1 M → 0 per launch, LDS-busy cycles 9.5 M → 7.4 M); other widths keep BN + 8
    const bool bswz = BN == 128;
    const int BNS = BN + (bswz ? 16 : 8);
    // row leaves vector forms over vars {0: m, 1: k}
    std::vector<std::vector<Sym>> crow;
    for (int l : P.rows) {
        const sanic_node& ln = d->nodes[st.leaf[l]];
        std::vector<Sym> cr(ln.rank);
        for (int j = 0; j < ln.rank; j++) {
            int b = st.bind[l][j];
            cr[j] = b == SANIC_BIND_STREAM ? Sym::var(1) : b == P.mdim ? Sym::var(0) : Sym();
        }
        std::vector<int> rb, rd;
        bool rok = true, rc = true;
        std::string rr;
        Code l1, d1;
        render_weight_run(d, st.leaf[l], cr, {M, K}, l1, d1, "mm", "k0", "_p", rb, rd, rok, rc, rr, false);
        if (!rok || !rc) return false;
        if (rr.empty()) rawA = false;
        crow.push_back(cr);
    }
    if (!rawA) grouped = false;
    if (grouped) splitB = false;
    // grouped tiles: tiling variants {8 waves, load depth 4; 4 waves, depth 4; 8 waves, depth 2}
    const int gvar = grouped && st.sched.variant > 0 && st.sched.variant < 3 ? st.sched.variant : 0;
    if (grouped && BM == 128 && BN == 32 && gvar != 1) NTH = 512;
    // A operands that need arithmetic (x·g of the fused RMSNorm) are built once by a first
    // launch into bf16 hi/lo planes [M][K] (plus the row slots), instead of by every one of the
    // N/BN column workgroups
    const bool pre = splitA && N / BN >= 4 && K % 512 == 0;
    const int64_t NKT = K / 64;
    int DEPTH = grouped ? (gvar == 2 ? 2 : 4) : 2;
    if (!grouped && st.sched.variant == 1) DEPTH = 4;
    if (NKT % DEPTH || NKT < 2 * DEPTH) DEPTH = 2;
    const bool deep = NKT % DEPTH == 0 && NKT >= 2 * DEPTH;
    // With the x·g planes written by the first launch, each wave loads its own A fragments
    // instead of staging A through LDS: the A tile's LDS stores and fragment reads were over half
    // of a K step's LDS traffic (B2: ≈96 of ≈176 KB per CU). The planes are then stored in
    // fragment order — per 16-row × 32-k block, lane (l16 = row, lq = k run) at 16·lane bytes —
    // so every fragment load is 1 KB contiguous (in 4-wave tiles, where two waves share rows,
    // both load them; the second from L1)
    const bool adirect = pre && deep && !getenv("SANIC_HIP_GEMM_ALDS");
    // element offset of (row, k) in a plane: row-major, or fragment order (k a multiple of 8)
    auto plane_off = [&](const std::string& row, const std::string& k8) {
        if (!adirect) return "(" + row + ") * " + std::to_string(K) + " + " + k8;
        return "((" + row + ") / 16 * " + std::to_string(K / 32) + " + (" + k8 + ") / 32) * 512 + ((" + row + ") % 16 + 16 * (((" + k8 + ") % 32) / 8)) * 8";
    };
    // waves along m and n: 4 × 2 / 2 × 2; grouped 32-column tiles of 8 waves 8 × 1, so no two
    // waves form the same rows' Σ x; 8 × 1 also for fragment-loaded A (each wave its own rows,
    // so no A fragment is loaded twice: B2 45.9 → 42.9 µs against 4 × 2)
    const int WGN = ((grouped && NTH == 512 && BN == 32 && BM == 128) || (adirect && NTH == 512 && BM == 128)) ? 1 : 2;
    const int WGM = NTH / 64 / WGN;
    const int WM = BM / WGM, WN = BN / WGN;   // per-wave tile
    const int MT = WM / 16, NT = WN / 16;
    // threads that load the B tile (all of them unless the tile has fewer runs of 8)
    const int BTH = std::min(NTH, BN * 8);
    const std::string btid = BTH < NTH ? "(tid % " + std::to_string(BTH) + ")" : std::string("tid");

    int64_t hi_off = 0, lo_off = 0, rs_off = 0;
    // K slices of the first launch in fragment order (8 at K = 2048: 256 workgroups for M = 512)
    int PKS = 1;
    while (adirect && PKS < 8 && K % (PKS * 2 * 4 * 32) == 0 && K / (PKS * 2) >= 256) PKS *= 2;
    Code kp;
    kp.indent = 1;
    if (pre) {
        hi_off = scratch;
        scratch += ((M * K * 2 + 255) / 256) * 256;
        lo_off = scratch;
        scratch += ((M * K * 2 + 255) / 256) * 256;
        rs_off = scratch;
        scratch += ((PKS * M * std::max(SR, 1) * 4 + 255) / 256) * 256;
        kp.line("const int t = threadIdx.x, lane = t & 63, wv = t >> 6;");
        if (adirect) {
            // fragment order: a workgroup takes one 16-row block and one of PKS K slices, each
            // wave a quarter of it in 32-k blocks; lane (l16, lq) builds row l16's run lq of a
            // block and stores it at 16·lane bytes, so every wave store is 1 KB contiguous
            kp.line("const idx_t mp = (idx_t)(blockIdx.x / " + std::to_string(PKS) + ") * 16 + (lane & 15);");
            kp.line("const int pks = blockIdx.x % " + std::to_string(PKS) + ";");
        } else {
            kp.line("const idx_t mp = (idx_t)blockIdx.x * 4 + wv;");
        }
        kp.line("unsigned short* ahi = (unsigned short*)((char*)a.scratch + " + std::to_string(hi_off) + ");");
        kp.line("unsigned short* alo = (unsigned short*)((char*)a.scratch + " + std::to_string(lo_off) + ");");
        for (int i = 0; i < SR; i++) kp.line("float rp" + std::to_string(i) + " = 0.0f;");
        const int64_t PIT = adirect ? K / PKS / 4 / 32 : K / 512;   // runs per lane
        for (int64_t i = 0; i < PIT; i++) {
            const std::string is = std::to_string(i);
            const std::string k0 = adirect ? "(pks * " + std::to_string(K / PKS) + " + wv * " + std::to_string(K / PKS / 4) + " + " + std::to_string(i * 32) + " + (lane >> 4) * 8)"
                                           : "(" + std::to_string(i * 512) + " + lane * 8)";
            kp.line("{");
            kp.indent++;
            R.memo.emplace_back();
            std::vector<std::vector<std::string>> vals(P.rows.size());
            for (size_t li = 0; li < P.rows.size(); li++) {
                std::vector<int> rb, rd;
                bool rok = true, rc = true;
                std::string rr;
                Code l1, d1;
                l1.indent = d1.indent = kp.indent;
                vals[li] = render_weight_run(d, st.leaf[P.rows[li]], crow[li], {M, K}, l1, d1, "mp", k0, "_p" + std::to_string(li) + "_" + is, rb, rd, rok, rc, rr, false);
                for (size_t b = 0; b < rb.size(); b++)
                    kp.line("const " + std::string(ctype_of(rd[b])) + "* __restrict__ wb" + std::to_string(b) + "_p" + std::to_string(li) + "_" + is + " = " + R.param(rb[b]) + ";");
                kp.s << l1.str() << d1.str();
            }
            std::vector<std::string> av(8);
            for (int j = 0; j < 8; j++) {
                auto item = [&](int it) -> std::string {
                    for (size_t li = 0; li < P.rows.size(); li++)
                        if (P.rows[li] == it) return vals[li][j];
                    return "0.0f";
                };
                av[j] = expr_rest(R, kp, c.into[P.cslots[0]], P.w, item);
                for (int sidx = 0; sidx < SR; sidx++)
                    kp.line("rp" + std::to_string(sidx) + " += " + expr_rest(R, kp, c.into[P.rslots[sidx]], -1, item) + ";");
            }
            R.memo.pop_back();
            kp.line("unsigned h_[4], l_[4];");
            for (int q = 0; q < 4; q++)
                kp.line("split_bf16(" + av[2 * q] + ", " + av[2 * q + 1] + ", h_[" + std::to_string(q) + "], l_[" + std::to_string(q) + "]);");
            kp.line("*(sanic_u32x4*)(ahi + " + plane_off("mp", k0) + ") = (sanic_u32x4){h_[0], h_[1], h_[2], h_[3]};");
            kp.line("*(sanic_u32x4*)(alo + " + plane_off("mp", k0) + ") = (sanic_u32x4){l_[0], l_[1], l_[2], l_[3]};");
            kp.indent--;
            kp.line("}");
        }
        if (adirect && SR) {
            // row slots: the four lanes of a row, then the four waves; one partial per K slice
            kp.line("__shared__ float rps[4][16][" + std::to_string(SR) + "];");
            for (int i = 0; i < SR; i++) {
                std::string r = "rp" + std::to_string(i);
                kp.line(r + " = sanic_rows_sum(" + r + ");");
                kp.line("if (lane < 16) rps[wv][lane][" + std::to_string(i) + "] = " + r + ";");
            }
            kp.line("__syncthreads();");
            kp.line("if (t < " + std::to_string(16 * SR) + ") {");
            kp.line("  const int r = t / " + std::to_string(SR) + ", sl = t % " + std::to_string(SR) + ";");
            kp.line("  ((float*)((char*)a.scratch + " + std::to_string(rs_off) + "))[((idx_t)pks * " + std::to_string(M) + " + (blockIdx.x / " + std::to_string(PKS) +
                    ") * 16 + r) * " + std::to_string(SR) + " + sl] = ((rps[0][r][sl] + rps[1][r][sl]) + rps[2][r][sl]) + rps[3][r][sl];");
            kp.line("}");
        }
        for (int i = 0; i < SR && !adirect; i++) {
            std::string r = "rp" + std::to_string(i);
            kp.line(r + " = sanic_wave_sum(" + r + ");");
            kp.line("if (lane == 0) ((float*)((char*)a.scratch + " + std::to_string(rs_off) + "))[mp * " + std::to_string(SR) + " + " + std::to_string(i) + "] = " + r + ";");
        }
    }

    Code k;
    k.indent = 1;
    k.line("__shared__ unsigned short a_lds[2][" + std::to_string(BM * AS) + "];");
    const int BTILE = bkn ? 64 * BNS : BN * BS;
    k.line("__shared__ unsigned short b_lds[2][" + std::to_string(BTILE) + "];");
    if (splitA) k.line("__shared__ unsigned short a_lo[2][" + std::to_string(BM * AS) + "];");
    if (splitB) k.line("__shared__ unsigned short b_lo[2][" + std::to_string(BTILE) + "];");
    if (SR) k.line("__shared__ float rs_lds[" + std::to_string(BM * SR) + "];");
    if (grouped) {
        k.line("__shared__ __attribute__((aligned(8))) float sz_lds[2][" + std::to_string(BN * 2) + "];");
        // a B fragment of ones: the matrix cores also give each row's Σ x over the tile
        k.line("const bf16x8 ones8 = __builtin_bit_cast(bf16x8, (sanic_u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});");
    }
    k.line("const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;");
    k.line("const int l16 = lane & 15, lq = lane >> 4;");
    k.line("const idx_t nb = blockIdx.x % " + std::to_string(N / BN) + ", mb = blockIdx.x / " + std::to_string(N / BN) + ";");
    k.line("const idx_t m0 = mb * " + std::to_string(BM) + ", n0 = nb * " + std::to_string(BN) + ";");
    k.line("const int wm = (wv / " + std::to_string(WGN) + ") * " + std::to_string(WM) + ", wn = (wv % " + std::to_string(WGN) + ") * " + std::to_string(WN) + ";");
    k.line("f32x4 acc[" + std::to_string(MT) + "][" + std::to_string(NT) + "];");
    k.line("#pragma unroll");
    k.line("for (int i = 0; i < " + std::to_string(MT) + "; ++i)");
    k.line("  #pragma unroll");
    k.line("  for (int j = 0; j < " + std::to_string(NT) + "; ++j) acc[i][j] = (f32x4){0, 0, 0, 0};");
    for (int i = 0; i < SR; i++) k.line("float racc" + std::to_string(i) + " = 0.0f;");

    // A tile: BM rows × 64 k; NTH/BM consecutive threads per row, each a contiguous run of
    // 64·BM/NTH k in runs of 8
    const int TPR = NTH / BM;              // threads per row: 4 (BM 128 at 512 threads, BM 64 at 256)
    const int RUNS_A = 64 / TPR / 8;       // runs of 8 per thread per tile
    // B tile: BN n × 64 k = BN·8 runs; k-contiguous weights: 8 lanes per row (coalesced rows),
    // else adjacent lanes take adjacent n
    const int RUNS_B = BN * 8 / BTH;
    auto emit_loads = [&](Code& c2, const std::string& kt0, const std::string& sfx) {
        // A runs
        c2.line("const idx_t mm" + sfx + " = m0 + tid / " + std::to_string(TPR) + ";");
        for (int i = 0; i < MT && adirect; i++)
            for (int ks = 0; ks < 2; ks++) {
                // the operand fragment itself: lane (l16, lq) holds row wm + 16·i + l16, k run lq·8
                // of the tile's 32-deep half ks (16 contiguous bytes of the row)
                const std::string nm = std::to_string(i) + "_" + std::to_string(ks) + sfx;
                const std::string at = "((m0 + wm + " + std::to_string(i * 16) + ") / 16 * " + std::to_string(K / 32) + " + (" + kt0 + " + " + std::to_string(ks * 32) + ") / 32) * 512 + lane * 8";
                c2.line("const sanic_u32x4 pah" + nm + " = *(const sanic_u32x4*)((const unsigned short*)((const char*)a.scratch + " + std::to_string(hi_off) + ") + " + at + ");");
                c2.line("const sanic_u32x4 pal" + nm + " = *(const sanic_u32x4*)((const unsigned short*)((const char*)a.scratch + " + std::to_string(lo_off) + ") + " + at + ");");
            }
        for (int r = 0; r < RUNS_A && pre && !adirect; r++) {
            std::string k0 = "(" + kt0 + " + (tid % " + std::to_string(TPR) + ") * " + std::to_string(64 / TPR) + " + " + std::to_string(r * 8) + ")";
            const std::string rs = std::to_string(r);
            c2.line("const sanic_u32x4 pah" + rs + sfx + " = *(const sanic_u32x4*)((const unsigned short*)((const char*)a.scratch + " + std::to_string(hi_off) + ") + mm" + sfx +
                    " * " + std::to_string(K) + " + " + k0 + ");");
            c2.line("const sanic_u32x4 pal" + rs + sfx + " = *(const sanic_u32x4*)((const unsigned short*)((const char*)a.scratch + " + std::to_string(lo_off) + ") + mm" + sfx +
                    " * " + std::to_string(K) + " + " + k0 + ");");
        }
        for (int r = 0; r < RUNS_A && !pre; r++) {
            std::string k0 = "(" + kt0 + " + (tid % " + std::to_string(TPR) + ") * " + std::to_string(64 / TPR) + " + " + std::to_string(r * 8) + ")";
            for (size_t li = 0; li < P.rows.size(); li++) {
                std::vector<int> rb, rd;
                bool rok = true, rc = true;
                std::string rr;
                Code l1, d1;
                l1.indent = d1.indent = c2.indent;
                auto vals = render_weight_run(d, st.leaf[P.rows[li]], crow[li], {M, K}, l1, d1, "mm" + sfx, k0,
                                              "_a" + std::to_string(li) + "_" + std::to_string(r) + sfx, rb, rd, rok, rc, rr, false);
                for (size_t b = 0; b < rb.size(); b++)
                    c2.line("const " + std::string(ctype_of(rd[b])) + "* __restrict__ wb" + std::to_string(b) + "_a" + std::to_string(li) + "_" + std::to_string(r) + sfx + " = " + R.param(rb[b]) + ";");
                if (rawA && !rr.empty()) {
                    c2.s << l1.str();
                    c2.line("const sanic_u32x4 rawa" + std::to_string(r) + sfx + " = " + rr + ";");
                    continue;
                }
                c2.s << l1.str() << d1.str();
                for (int j = 0; j < 8; j++)
                    c2.line("const float ra" + std::to_string(li) + "_" + std::to_string(r) + "_" + std::to_string(j) + sfx + " = " + vals[j] + ";");
            }
        }
        // B runs
        for (int r = 0; r < RUNS_B; r++) {
            std::string rs = std::to_string(r);
            std::string nn, kk;
            if (bkn) {
                // chunk c = tid + 256·r: k row c / (BN/8), 8 columns from (c % (BN/8))·8
                const std::string cc = "(" + btid + " + " + std::to_string(r * BTH) + ")";
                kk = "(" + kt0 + " + " + cc + " / " + std::to_string(BN / 8) + ")";
                nn = "(n0 + (" + cc + " % " + std::to_string(BN / 8) + ") * 8)";
            } else if (contig) {
                nn = "(n0 + (" + btid + " / 8) + " + std::to_string(r * (BTH / 8)) + ")";
                kk = "(" + kt0 + " + (" + btid + " % 8) * 8)";
            } else {
                nn = "(n0 + (" + btid + " % " + std::to_string(BN) + "))";
                kk = "(" + kt0 + " + ((" + btid + " / " + std::to_string(BN) + ") + " + std::to_string(r * (BTH / BN)) + ") * 8)";
            }
            std::vector<int> rb, rd;
            bool rok = true, rc = true;
            std::string rr;
            Code l1, d1;
            l1.indent = d1.indent = c2.indent;
            if (grouped) {
                // the loads only (q's packed word, the group's s and z as stored): the words
                // are what a load set holds across the loop, and emit_stores widens them (so
                // the back edge never waits for a load issued in the same iteration)
                std::vector<std::string> qv;
                std::string A_, B_;
                bool nb = false;
                int64_t ud = 0;
                render_weight_affine(d, st.leaf[P.w], cw, {N, K}, l1, d1, nn, kk, "_b" + rs + sfx, rb, rd, qv, A_, B_, nb, ud, false, true);
                for (size_t b = 0; b < rb.size(); b++)
                    c2.line("const " + std::string(ctype_of(rd[b])) + "* __restrict__ wb" + std::to_string(b) + "_b" + rs + sfx + " = " + R.param(rb[b]) + ";");
                c2.s << l1.str();
                continue;
            }
            auto vals = bkn ? render_weight_run(d, st.leaf[P.w], cwt, {K, N}, l1, d1, kk, nn, "_b" + rs + sfx, rb, rd, rok, rc, rr, false)
                            : render_weight_run(d, st.leaf[P.w], cw, {N, K}, l1, d1, nn, kk, "_b" + rs + sfx, rb, rd, rok, rc, rr, false);
            for (size_t b = 0; b < rb.size(); b++)
                c2.line("const " + std::string(ctype_of(rd[b])) + "* __restrict__ wb" + std::to_string(b) + "_b" + rs + sfx + " = " + R.param(rb[b]) + ";");
            c2.s << l1.str();
            if (!rr.empty()) {
                c2.line("const sanic_u32x4 rb" + rs + sfx + " = " + rr + ";");
            } else if (splitB) {
                c2.s << d1.str();
                const std::string h = "rbh" + rs + sfx, l = "rbl" + rs + sfx;
                c2.line("unsigned " + h + "[4], " + l + "[4];");
                for (int q = 0; q < 4; q++)
                    c2.line("split_bf16(" + vals[2 * q] + ", " + vals[2 * q + 1] + ", " + h + "[" + std::to_string(q) + "], " + l + "[" + std::to_string(q) + "]);");
                c2.line("const sanic_u32x4 rb" + rs + sfx + " = (sanic_u32x4){" + h + "[0], " + h + "[1], " + h + "[2], " + h + "[3]};");
                c2.line("const sanic_u32x4 rl" + rs + sfx + " = (sanic_u32x4){" + l + "[0], " + l + "[1], " + l + "[2], " + l + "[3]};");
            } else {
                c2.s << d1.str();
                c2.line("const sanic_u32x4 rb" + rs + sfx + " = (sanic_u32x4){pk_bf16(" + vals[0] + ", " + vals[1] + "), pk_bf16(" + vals[2] + ", " +
                        vals[3] + "), pk_bf16(" + vals[4] + ", " + vals[5] + "), pk_bf16(" + vals[6] + ", " + vals[7] + ")};");
            }
        }
    };
    auto emit_stores = [&](Code& c2, const std::string& buf, const std::string& sfx) {
        c2.line("{");
        c2.indent++;
        c2.line("const int ar = tid / " + std::to_string(TPR) + ";");
        for (int r = 0; r < RUNS_A && pre && !adirect; r++) {
            const std::string rs = std::to_string(r);
            const std::string aoff = koff("ar", "(tid % " + std::to_string(TPR) + ") * " + std::to_string(64 / TPR) + " + " + std::to_string(r * 8), AS);
            c2.line("*(sanic_u32x4*)(&a_lds[" + buf + "][" + aoff + "]) = pah" + rs + sfx + ";");
            c2.line("*(sanic_u32x4*)(&a_lo[" + buf + "][" + aoff + "]) = pal" + rs + sfx + ";");
        }
        for (int r = 0; r < RUNS_A && !pre && rawA; r++) {
            const std::string aoff = koff("ar", "(tid % " + std::to_string(TPR) + ") * " + std::to_string(64 / TPR) + " + " + std::to_string(r * 8), AS);
            c2.line("*(sanic_u32x4*)(&a_lds[" + buf + "][" + aoff + "]) = rawa" + std::to_string(r) + sfx + ";");
        }

        for (int r = 0; r < RUNS_A && !pre && !rawA; r++) {
            std::string rs = std::to_string(r);
            // rest of the contraction slot (A) and the row slots, per element
            std::string pk[4];
            std::vector<std::string> av(8);
            for (int j = 0; j < 8; j++) {
                auto item = [&](int i) -> std::string {
                    for (size_t li = 0; li < P.rows.size(); li++)
                        if (P.rows[li] == i) return "ra" + std::to_string(li) + "_" + rs + "_" + std::to_string(j) + sfx;
                    return "0.0f";
                };
                std::string v = expr_rest(R, c2, c.into[P.cslots[0]], P.w, item);
                av[j] = v;
                for (int sidx = 0; sidx < SR; sidx++) {
                    std::string rv = expr_rest(R, c2, c.into[P.rslots[sidx]], -1, item);
                    c2.line("racc" + std::to_string(sidx) + " += " + rv + ";");
                }
            }
            const std::string aoff = koff("ar", "(tid % " + std::to_string(TPR) + ") * " + std::to_string(64 / TPR) + " + " + std::to_string(r * 8), AS);
            if (splitA) {
                const std::string h = R.fresh("ah"), l = R.fresh("al");
                c2.line("unsigned " + h + "[4], " + l + "[4];");
                for (int q = 0; q < 4; q++)
                    c2.line("split_bf16(" + av[2 * q] + ", " + av[2 * q + 1] + ", " + h + "[" + std::to_string(q) + "], " + l + "[" + std::to_string(q) + "]);");
                c2.line("*(sanic_u32x4*)(&a_lds[" + buf + "][" + aoff + "]) = (sanic_u32x4){" + h + "[0], " + h + "[1], " + h + "[2], " + h + "[3]};");
                c2.line("*(sanic_u32x4*)(&a_lo[" + buf + "][" + aoff + "]) = (sanic_u32x4){" + l + "[0], " + l + "[1], " + l + "[2], " + l + "[3]};");
            } else {
                c2.line("*(sanic_u32x4*)(&a_lds[" + buf + "][" + aoff + "]) = (sanic_u32x4){pk_bf16(" + av[0] + ", " + av[1] + "), pk_bf16(" + av[2] + ", " + av[3] +
                        "), pk_bf16(" + av[4] + ", " + av[5] + "), pk_bf16(" + av[6] + ", " + av[7] + ")};");
            }
        }
        if (BTH < NTH) c2.line("if (tid < " + std::to_string(BTH) + ") {");
        for (int r = 0; r < RUNS_B; r++) {
            std::string rs = std::to_string(r);
            std::string row, col;
            int stride = BS;
            if (bkn) {
                const std::string cc = "(" + btid + " + " + std::to_string(r * BTH) + ")";
                row = "(" + cc + " / " + std::to_string(BN / 8) + ")";
                col = "((" + cc + " % " + std::to_string(BN / 8) + ") * 8)";
                stride = BNS;
            } else if (contig) {
                row = "((" + btid + " / 8) + " + std::to_string(r * (BTH / 8)) + ")";
                col = "((" + btid + " % 8) * 8)";
            } else {
                row = "(" + btid + " % " + std::to_string(BN) + ")";
                col = "(((" + btid + " / " + std::to_string(BN) + ") + " + std::to_string(r * (BTH / BN)) + ") * 8)";
            }
            const std::string boff = bkn ? row + " * " + std::to_string(stride) + " + " + (bswz ? "(" + col + " ^ (((" + row + " >> 3) & 1) * 64))" : col) : koff(row, col, stride);
            if (grouped) {
                // q as exact bf16 integers; this row's group s and z for the lanes' fold (the
                // same rendering as emit_loads', whose loaded words these expressions read)
                std::vector<std::string> qv;
                std::string A_, B_;
                bool nb = false;
                int64_t ud = 0;
                std::vector<int> gb, gd;
                Code l1, d1;
                l1.indent = d1.indent = c2.indent;
                render_weight_affine(d, st.leaf[P.w], cw, {N, K}, l1, d1, "nn", "k0", "_b" + rs + sfx, gb, gd, qv, A_, B_, nb, ud, false, true);
                c2.line("{");
                c2.s << d1.str();
                c2.line("*(sanic_u32x4*)(&b_lds[" + buf + "][" + boff + "]) = (sanic_u32x4){pk_bf16(" + qv[0] + ", " + qv[1] + "), pk_bf16(" + qv[2] + ", " +
                        qv[3] + "), pk_bf16(" + qv[4] + ", " + qv[5] + "), pk_bf16(" + qv[6] + ", " + qv[7] + ")};");
                c2.line("if (tid % 8 == 0) *(sanic_f32x2*)(&sz_lds[" + buf + "][" + row + " * 2]) = (sanic_f32x2){" + A_ + ", " +
                        (B_.empty() ? std::string("0.0f") : (nb ? "-" : "") + B_) + "};");
                c2.line("}");
                continue;
            }
            c2.line("*(sanic_u32x4*)(&b_lds[" + buf + "][" + boff + "]) = rb" + rs + sfx + ";");
            if (splitB) c2.line("*(sanic_u32x4*)(&b_lo[" + buf + "][" + boff + "]) = rl" + rs + sfx + ";");
        }
        if (BTH < NTH) c2.line("}");
        c2.indent--;
        c2.line("}");
    };
    // one K tile's MFMAs over its two 32-deep halves: the first half's operand fragments are
    // read from LDS, then the second half's reads are interleaved one by one with the first
    // half's MFMAs (scheduling groups), then the second half's MFMAs — so LDS reads proceed
    // under MFMAs within each wave as well as across the two waves of a SIMD (8-wave tiles:
    // 44.5 → 41.7 µs for B2's GEMM against reading everything first)
    auto emit_mfma = [&](Code& c2, const std::string& buf, const std::string& aset = "") {
        const std::string MTs = std::to_string(MT), NTs = std::to_string(NT);
        c2.line("{");
        c2.line("bf16x8 af[2][" + MTs + "], bf[2][" + NTs + "];");
        if (splitA) c2.line("bf16x8 afl[2][" + MTs + "];");
        if (splitB) c2.line("bf16x8 bfl[2][" + NTs + "];");
        auto reads = [&](int ks) {
            const std::string kss = std::to_string(ks);
            const std::string aidx = "[" + koff("wm + i * 16 + l16", kss + " * 32 + lq * 8", AS) + "]";
            if (adirect) {
                for (int i = 0; i < MT; i++) {
                    const std::string nm = std::to_string(i) + "_" + kss + aset;
                    c2.line("af[" + kss + "][" + std::to_string(i) + "] = __builtin_bit_cast(bf16x8, pah" + nm + ");");
                    c2.line("afl[" + kss + "][" + std::to_string(i) + "] = __builtin_bit_cast(bf16x8, pal" + nm + ");");
                }
            } else {
            c2.line("#pragma unroll");
            c2.line("for (int i = 0; i < " + MTs + "; ++i) {");
            c2.line("  af[" + kss + "][i] = *(const bf16x8*)(&a_lds[" + buf + "]" + aidx + ");");
            if (splitA) c2.line("  afl[" + kss + "][i] = *(const bf16x8*)(&a_lo[" + buf + "]" + aidx + ");");
            c2.line("}");
            }
            c2.line("#pragma unroll");
            c2.line("for (int j = 0; j < " + NTs + "; ++j) {");
            if (bkn) {
                // rows ks·32 + lq·8 + (0..3 | 4..7), column wn + j·16 + l16: in each 16-lane
                // group, source lane s reads 4 columns 4·(s%4) of row base + s/4; lane i gets 4
                // rows of column i
                const std::string br = "[(" + kss + " * 32 + lq * 8 + (l16 >> 2)) * " + std::to_string(BNS) + " + " +
                                       (bswz ? std::string("((wn + j * 16 + (l16 & 3) * 4) ^ ((lq & 1) * 64))") : std::string("wn + j * 16 + (l16 & 3) * 4")) + "]";
                auto tr = [&](const std::string& arr, const std::string& dst) {
                    c2.line("  {");
                    c2.line("    const unsigned short* bp = &" + arr + "[" + buf + "]" + br + ";");
                    c2.line("    const sanic_s16x4 t0_ = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) sanic_s16x4*)(bp));");
                    c2.line("    const sanic_s16x4 t1_ = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) sanic_s16x4*)(bp + 4 * " + std::to_string(BNS) + "));");
                    c2.line("    " + dst + " = __builtin_bit_cast(bf16x8, (sanic_s16x8)__builtin_shufflevector(t0_, t1_, 0, 1, 2, 3, 4, 5, 6, 7));");
                    c2.line("  }");
                };
                tr("b_lds", "bf[" + kss + "][j]");
                if (splitB) tr("b_lo", "bfl[" + kss + "][j]");
            } else {
                const std::string bidx = "[" + koff("wn + j * 16 + l16", kss + " * 32 + lq * 8", BS) + "]";
                c2.line("  bf[" + kss + "][j] = *(const bf16x8*)(&b_lds[" + buf + "]" + bidx + ");");
                if (splitB) c2.line("  bfl[" + kss + "][j] = *(const bf16x8*)(&b_lo[" + buf + "]" + bidx + ");");
            }
            c2.line("}");
        };
        const std::string accv = grouped ? "tq" : "acc";
        if (grouped) {
            c2.line("f32x4 tq[" + MTs + "][" + NTs + "], xq[" + MTs + "];");
            c2.line("#pragma unroll");
            c2.line("for (int i = 0; i < " + MTs + "; ++i) {");
            c2.line("  xq[i] = (f32x4){0, 0, 0, 0};");
            c2.line("  #pragma unroll");
            c2.line("  for (int j = 0; j < " + NTs + "; ++j) tq[i][j] = (f32x4){0, 0, 0, 0};");
            c2.line("}");
        }
        auto mfmas = [&](int ks) {
            const std::string kss = std::to_string(ks);
            c2.line("#pragma unroll");
            c2.line("for (int i = 0; i < " + MTs + "; ++i)");
            c2.line("  #pragma unroll");
            c2.line("  for (int j = 0; j < " + NTs + "; ++j) {");
            c2.line("    " + accv + "[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[" + kss + "][i], bf[" + kss + "][j], " + accv + "[i][j], 0, 0, 0);");
            if (splitA) c2.line("    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afl[" + kss + "][i], bf[" + kss + "][j], acc[i][j], 0, 0, 0);");
            if (splitB) c2.line("    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[" + kss + "][i], bfl[" + kss + "][j], acc[i][j], 0, 0, 0);");
            c2.line("  }");
            if (grouped) {
                c2.line("#pragma unroll");
                c2.line("for (int i = 0; i < " + MTs + "; ++i) xq[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[" + kss + "][i], ones8, xq[i], 0, 0, 0);");
            }
        };
        // instruction counts of one half: LDS reads and MFMAs
        const int nds = (adirect ? 0 : MT * (splitA ? 2 : 1)) + NT * (bkn ? 2 : 1) * (splitB ? 2 : 1);
        const int nmf = MT * NT * (1 + (splitA ? 1 : 0) + (splitB ? 1 : 0)) + (grouped ? MT : 0);
        reads(0);
        c2.line("__builtin_amdgcn_sched_barrier(0);");
        reads(1);
        mfmas(0);
        const int pairs = std::min(nds, nmf);
        for (int i = 0; i < pairs; i++) {
            c2.line("__builtin_amdgcn_sched_group_barrier(0x008, 1, 0);");   // one MFMA
            c2.line("__builtin_amdgcn_sched_group_barrier(0x100, 1, 0);");   // one LDS read
        }
        if (nmf > pairs) c2.line("__builtin_amdgcn_sched_group_barrier(0x008, " + std::to_string(nmf - pairs) + ", 0);");
        if (nds > pairs) c2.line("__builtin_amdgcn_sched_group_barrier(0x100, " + std::to_string(nds - pairs) + ", 0);");
        c2.line("__builtin_amdgcn_sched_barrier(0);");
        mfmas(1);
        if (grouped) {
            // fold the tile: acc += s·Σ x·q ± z·Σ x (the sign rides z), per output element
            c2.line("#pragma unroll");
            c2.line("for (int i = 0; i < " + MTs + "; ++i) {");
            c2.line("  const f32x4 xr = xq[i];");
            c2.line("  #pragma unroll");
            c2.line("  for (int j = 0; j < " + NTs + "; ++j) {");
            c2.line("    const sanic_f32x2 sz = *(const sanic_f32x2*)(&sz_lds[" + buf + "][(wn + j * 16 + l16) * 2]);");
            c2.line("    #pragma unroll");
            c2.line("    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(sz.y, xr[r], fmaf(sz.x, tq[i][j][r], acc[i][j][r]));");
            c2.line("  }");
            c2.line("}");
        }
        c2.line("}");
    };
    // Loads run DEPTH tiles ahead of the MFMAs: one workgroup per CU leaves a single wave per
    // SIMD, so a tile's global loads (≈1–2 µs under load) must be in flight for several tiles'
    // MFMAs, not one. DEPTH register sets rotate in a loop unrolled by DEPTH; a set's loaded
    // values are plain variables declared before the loop (the loads' address temporaries stay
    // scoped). Set u holds the tiles ≡ u (mod DEPTH): at step t the set of tile t (already in
    // LDS) takes tile t + DEPTH, and the set of tile t + 1 goes to LDS behind the MFMAs.
    // Depth 2 for bf16 tiles; 4 for grouped 4-bit tiles, whose per-tile MFMA work is small
    // against the load latency. Variant 1 takes the other depth.
    if (!adirect) {
        k.line("{");
        k.indent++;
        emit_loads(k, "(idx_t)0", "_0");
        emit_stores(k, "0", "_0");
        k.indent--;
        k.line("}");
        k.line("__syncthreads();");
    }
    if (deep) {
        auto persistent = [&](const std::string& sfx, Code& decl) {
            Code tmp;
            tmp.indent = k.indent + 1;
            emit_loads(tmp, "(idx_t)0", sfx);
            static const std::regex re(R"(const (sanic_u32x4|float|unsigned short|unsigned) (\w+) = )");
            std::string t = tmp.str();
            std::set<std::string> seen;
            for (auto it = std::sregex_iterator(t.begin(), t.end(), re); it != std::sregex_iterator(); ++it) {
                const std::string name = (*it)[2];
                if (name.size() > sfx.size() && name.compare(name.size() - sfx.size(), sfx.size(), sfx) == 0 &&
                    (name.rfind("pah", 0) == 0 || name.rfind("pal", 0) == 0 || name.rfind("rb", 0) == 0 ||
                     name.rfind("rl", 0) == 0 || name.rfind("ra", 0) == 0 || name.rfind("gs", 0) == 0 ||
                     name.rfind("gz", 0) == 0 || (grouped && (name[0] == 'u' || name[0] == 'h'))) && name.rfind("rbh", 0) != 0 &&
                    name.rfind("rbl", 0) != 0 && !seen.count(name)) {
                    seen.insert(name);
                    decl.line(std::string((*it)[1]) + " " + name + ";");
                }
            }
            return seen;
        };
        // loads into a set: address temporaries in a block, the values assigned to the set
        auto load_into = [&](const std::string& kt0, const std::string& sfx, const std::set<std::string>& names) {
            Code tmp;
            tmp.indent = k.indent + 1;
            emit_loads(tmp, kt0, sfx);
            std::string t = tmp.str();
            for (auto& n : names) {
                for (const char* ty : {"const sanic_u32x4 ", "const float ", "const unsigned short ", "const unsigned "}) {
                    const std::string from = std::string(ty) + n + " = ";
                    size_t pos = t.find(from);
                    if (pos != std::string::npos) t.replace(pos, from.size(), n + " = ");
                }
            }
            k.line("{");
            k.s << t;
            k.line("}");
            // keep the requests ahead of this step's MFMAs (the scheduler would sink them)
            k.line("__builtin_amdgcn_sched_barrier(0);");
        };
        Code decl;
        decl.indent = k.indent;
        std::vector<std::set<std::string>> names(DEPTH);
        auto set_sfx = [](int u) { return "_s" + std::to_string(u); };
        for (int u = 0; u < DEPTH; u++) names[u] = persistent(set_sfx(u), decl);
        k.s << decl.str();
        if (adirect) {
            // tile 0's set: its A fragments stay in registers for the first step, its B goes to LDS
            load_into("(idx_t)0", set_sfx(0), names[0]);
            emit_stores(k, "0", set_sfx(0));
            k.line("__syncthreads();");
        }
        for (int u = 1; u < DEPTH; u++) load_into("(idx_t)" + std::to_string(64 * u), set_sfx(u), names[u]);   // tiles 1..DEPTH-1
        const std::string N2 = std::to_string(NKT), DS = std::to_string(DEPTH);
        k.line("for (idx_t kt = 0; kt < " + N2 + "; kt += " + DS + ") {");
        k.indent++;
        for (int u = 0; u < DEPTH; u++) {
            // step kt+u: tile kt+u is in LDS buffer u % 2; its set takes tile kt+u+DEPTH
            // (A fragments in the set: the MFMAs take them before the set is reloaded)
            if (!adirect) load_into("(((kt + " + std::to_string(u + DEPTH) + ") % " + N2 + ") * 64)", set_sfx(u), names[u]);
            emit_mfma(k, std::to_string(u % 2), set_sfx(u));
            if (adirect) load_into("(((kt + " + std::to_string(u + DEPTH) + ") % " + N2 + ") * 64)", set_sfx(u), names[u]);
            const int nx = (u + 1) % DEPTH;
            if (u == DEPTH - 1) {
                k.line("if (kt + " + DS + " < " + N2 + ") {");
                k.indent++;
            }
            emit_stores(k, std::to_string((u + 1) % 2), set_sfx(nx));
            if (u == DEPTH - 1) {
                k.indent--;
                k.line("}");
            }
            k.line("__syncthreads();");
        }
        k.indent--;
        k.line("}");
    } else {
    k.line("for (idx_t kt = 0; kt < " + std::to_string(NKT) + "; ++kt) {");
    k.indent++;
    k.line("const int buf = (int)(kt & 1);");
    k.line("const bool more = kt + 1 < " + std::to_string(NKT) + ";");
    // next tile's loads in flight during this tile's MFMAs (the last step re-reads tile 0)
    emit_loads(k, "(((kt + 1) % " + std::to_string(NKT) + ") * 64)", "_n");
    emit_mfma(k, "buf");
    k.line("if (more) {");
    k.indent++;
    emit_stores(k, "buf ^ 1", "_n");
    k.indent--;
    k.line("}");
    k.line("__syncthreads();");
    k.indent--;
    k.line("}");
    }
    // row slots: sum the TPR partial rows, publish per row
    if (SR && pre) {
        std::string sum;
        for (int q = 0; q < PKS; q++) {
            const std::string pq = "((const float*)((const char*)a.scratch + " + std::to_string(rs_off) + "))[" + std::to_string((int64_t)q * M * SR) + " + m0 * " + std::to_string(SR) + " + i]";
            sum = q ? "(" + sum + " + " + pq + ")" : pq;
        }
        k.line("for (int i = tid; i < " + std::to_string(BM * SR) + "; i += " + std::to_string(NTH) + ") rs_lds[i] = " + sum + ";");
        k.line("__syncthreads();");
    }
    if (SR && !pre) {
        for (int i = 0; i < SR; i++) {
            std::string r = "racc" + std::to_string(i);
            // TPR consecutive lanes (2 or 4) hold one row's partials: lane ^ 1, then lane ^ 2
            k.line(r + " += sanic_dpp<0xB1>(" + r + ");");
            if (TPR == 4) k.line(r + " += sanic_dpp<0x4E>(" + r + ");");
            k.line("if (tid % " + std::to_string(TPR) + " == 0) rs_lds[(tid / " + std::to_string(TPR) + ") * " + std::to_string(SR) + " + " + std::to_string(i) + "] = " + r + ";");
        }
        k.line("__syncthreads();");
    }
    // finish: project, epilogue, narrowing store per element
    k.line("#pragma unroll");
    k.line("for (int i = 0; i < " + std::to_string(MT) + "; ++i)");
    k.line("  #pragma unroll");
    k.line("  for (int j = 0; j < " + std::to_string(NT) + "; ++j)");
    k.line("    #pragma unroll");
    k.line("    for (int r = 0; r < 4; ++r) {");
    k.indent += 3;
    k.line("const int ml = wm + i * 16 + lq * 4 + r;");
    k.line("const idx_t gm = m0 + ml, gn = n0 + wn + j * 16 + l16;");
    k.line("const float fs" + std::to_string(P.cslots[0]) + " = acc[i][j][r];");
    for (int i = 0; i < SR; i++)
        k.line("const float fs" + std::to_string(P.rslots[i]) + " = rs_lds[ml * " + std::to_string(SR) + " + " + std::to_string(i) + "];");
    R.memo.emplace_back();
    std::string f = R.expr(k, c.project, "", "", "", "fs");
    k.line("const float fold_v = " + f + ";");
    std::vector<std::string> gc(st.rank, "0");
    gc[P.mdim] = "gm";
    gc[P.ndim] = "gn";
    std::string v = "fold_v";
    if (st.epilogue >= 0) {
        R.fold_var = "fold_v";
        v = R.value(k, st.epilogue, gc);
    }
    R.memo.pop_back();
    std::string lin;
    for (int j = 0; j < st.rank; j++)
        lin = j == 0 ? "(idx_t)(" + gc[0] + ")" : "(" + lin + " * " + std::to_string(st.grid[j]) + " + (idx_t)(" + gc[j] + "))";
    k.line(store_stmt(R.param(st.out_buffer), lin, st.out_dtype, v, false, d->buffers[st.out_buffer].scale));
    k.indent -= 3;
    k.line("    }");

    const std::string kname = "sanic_gemm_" + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K);
    std::ostringstream src;
    src << kPrelude;
    src << "typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;\n";
    src << "typedef short sanic_s16x4 __attribute__((ext_vector_type(4)));\n";
    src << "typedef short sanic_s16x8 __attribute__((ext_vector_type(8)));\n";
    src << "typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;\n";
    src << "typedef __bf16 sanic_bf16x2 __attribute__((ext_vector_type(2)));\n";
    src << "typedef float sanic_f32x2 __attribute__((ext_vector_type(2)));\n";
    src << "__device__ __forceinline__ unsigned pk_bf16(float x, float y) {\n"
           "  return __builtin_bit_cast(unsigned, __builtin_convertvector((sanic_f32x2){x, y}, sanic_bf16x2));\n}\n";
    src << "__device__ __forceinline__ void split_bf16(float x, float y, unsigned& hi, unsigned& lo) {\n"
           "  const unsigned h = pk_bf16(x, y);\n"
           "  hi = h;\n"
           "  lo = pk_bf16(x - __uint_as_float(h << 16), y - __uint_as_float(h & 0xFFFF0000u));\n}\n";
    src << R.args_struct(pre ? std::vector<std::string>{"float* __restrict__ scratch"} : std::vector<std::string>{});
    if (pre) src << "extern \"C\" __global__ void __launch_bounds__(256) " << kname << "_pre(Args a) {\n" << R.entry() << kp.str() << "}\n";
    src << "extern \"C\" __global__ void __launch_bounds__(" << NTH << ") " << kname << "(Args a) {\n" << R.entry() << k.str() << "}\n";
    out.kernel_kind = "skeleton:gemm[" + std::to_string(BM) + "x" + std::to_string(BN) + (splitA ? ",a2" : "") + (splitB ? ",b2" : "") +
                      (grouped ? ",grp" : "") + (bkn ? ",kn" : "") + (pre ? ",pre" : "") + (deep ? ",d" + std::to_string(DEPTH) : "") + ",w" + std::to_string(NTH / 64) + (adirect ? ",ad" : "") + "]";
    out.variants = grouped ? 3 : 2;
    // dequantized-weight tiles (int4): the ILP-maximising machine scheduler, D2 25.1 → 22.9 µs;
    // bf16 tiles keep the default strategy (no measurable difference)
    out.source = (splitB || grouped ? std::string("// sched-strategy: iterative-ilp\n") : std::string()) + src.str();
    std::vector<Arg> args = R.arg_list();
    if (pre) {
        args.push_back({Arg::SCRATCH, 0});
        out.launches.push_back({kname + "_pre", "", dim3((unsigned)(adirect ? M / 16 * PKS : M / 4)), dim3(256), 0, args});
    }
    out.launches.push_back({kname, "", dim3((unsigned)((M / BM) * (N / BN))), dim3(NTH), 0, args});
    return true;
}

}  // namespace sanic
