/*
 * oracle/interp.c — TEST INFRASTRUCTURE, not product code.
 *
 * A plain-C, dense-f64 restatement of sanic's interpreter oracle:
 *   eval              /root/reference/src/interp.rs:270-430  (every intermediate materialised)
 *   apply_map         /root/reference/src/interp.rs:472-498
 *   monoid_combine    /root/reference/src/interp.rs:500-518  (stable LogSumExp with −∞ guard)
 *   run_carrier_split /root/reference/src/interp.rs:555-643  (chunk b covers [b·n/B, (b+1)·n/B))
 *   Carrier eval      /root/reference/src/derive.rs:283-343  (lift / merge / project)
 *   Schedule execute  /root/reference/src/partition.rs:2117-2176 (stage by stage, each stage's
 *                     output narrowed through its storage dtype, round_to scalar.rs:120-152)
 * It reads the same flat program descriptor as the product (include/sanic_hip.h). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as the checker.
 *
 * Buffers are arrays of f64 VALUES (packed int4 etc. are decoded by the caller).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/sanic_hip.h"
#include "oracle.h"

/* ── scalar semantics ─────────────────────────────────────────────────────── */

/* Rust f64::max / f64::min ignore a NaN operand. */
static double rmax(double a, double b) { if (isnan(a)) return b; if (isnan(b)) return a; return a > b ? a : b; }
static double rmin(double a, double b) { if (isnan(a)) return b; if (isnan(b)) return a; return a < b ? a : b; }

double oracle_round_bf16(double v) {
    /* scalar.rs:128-135: RNE on the high half of the f32 pattern, NaN kept quiet */
    float f = (float)v;
    uint32_t b;
    memcpy(&b, &f, 4);
    if (isnan(f)) {
        uint32_t r = ((b >> 16) | 0x0040u) << 16;
        memcpy(&f, &r, 4);
        return (double)f;
    }
    uint32_t r = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
    r <<= 16;
    memcpy(&f, &r, 4);
    return (double)f;
}

/* scalar.rs:143-147: the Q8 grid {q·scale : −127 ≤ q ≤ 127}, q = round(v/scale) with ties
   away from zero (f64::round), clamped; grid points are fixed points */
double oracle_round_q8(double scale, double v) {
    double q = round(v / scale);
    if (q < -127.0) q = -127.0;
    if (q > 127.0) q = 127.0;
    return q * scale;
}

/* scalar.rs:154-178 semantics (f64 → f32 → IEEE half → f32, ties to even, overflow to ±∞,
   half subnormals on the 2^-24 grid), restated as "round to the half ulp of the value's binade":
   the ulp is 2^(e−10) for |x| in [2^e, 2^(e+1)), never below 2^-24 */
double oracle_round_f16(double v) {
    float f = (float)v;
    if (isnan(f) || isinf(f)) return (double)f;
    double m = fabs((double)f);
    if (m == 0.0) return (double)f;
    int e;
    frexp(m, &e);                       /* m in [2^(e−1), 2^e) */
    int ue = e - 1 - 10;
    if (ue < -24) ue = -24;
    double q = nearbyint(ldexp(m, -ue)); /* default rounding mode: ties to even */
    double r = ldexp(q, ue);
    if (r > 65504.0) r = INFINITY;
    return f < 0 ? -r : r;
}

double oracle_round_to(int dtype, double v) {
    switch (dtype) {
    case SANIC_F64: return v;
    case SANIC_F32: return (double)(float)v;
    case SANIC_BF16: return oracle_round_bf16(v);
    case SANIC_F16: return oracle_round_f16(v);
    case SANIC_U32: {
        /* the saturating u32 store (emit_metal.rs:186-190): computed in f32 */
        float f = (float)v;
        if (f >= 4294967040.0f) return 4294967295.0;
        if (!(f > 0.0f)) return 0.0;
        return (double)(uint32_t)(f + 0.5f);
    }
    default: return v;
    }
}

double oracle_apply_map(int op, const double* a) {
    switch (op) {
    case SANIC_OP_ADD: return a[0] + a[1];
    case SANIC_OP_SUB: return a[0] - a[1];
    case SANIC_OP_MUL: return a[0] * a[1];
    case SANIC_OP_DIV: return a[0] / a[1];
    case SANIC_OP_MAX: return rmax(a[0], a[1]);
    case SANIC_OP_MIN: return rmin(a[0], a[1]);
    case SANIC_OP_LT: return a[0] < a[1] ? 1.0 : 0.0;
    case SANIC_OP_NEG: return -a[0];
    case SANIC_OP_RECIP: return 1.0 / a[0];
    case SANIC_OP_EXP: return exp(a[0]);
    case SANIC_OP_LOG: return log(a[0]);
    case SANIC_OP_SQRT: return sqrt(a[0]);
    case SANIC_OP_TANH: return tanh(a[0]);
    case SANIC_OP_SIN: return sin(a[0]);
    case SANIC_OP_COS: return cos(a[0]);
    case SANIC_OP_WHERE: return a[0] != 0.0 ? a[1] : a[2];
    case SANIC_OP_ROUND_BF16: return oracle_round_bf16(a[0]);
    case SANIC_OP_ROUND_F32: return (double)(float)a[0];
    case SANIC_OP_ROUND_F16: return oracle_round_f16(a[0]);
    }
    return NAN;
}

double oracle_monoid_identity(int m) {
    switch (m) {
    case SANIC_MON_ADD: return 0.0;
    case SANIC_MON_MUL: return 1.0;
    case SANIC_MON_MAX: case SANIC_MON_LSE: return -INFINITY;
    default: return INFINITY;
    }
}

double oracle_monoid_combine(int m, double a, double b) {
    switch (m) {
    case SANIC_MON_ADD: return a + b;
    case SANIC_MON_MUL: return a * b;
    case SANIC_MON_MAX: return rmax(a, b);
    case SANIC_MON_MIN: return rmin(a, b);
    default: {
        if (a == -INFINITY) return b;
        if (b == -INFINITY) return a;
        double mm = rmax(a, b);
        return mm + log(exp(a - mm) + exp(b - mm));
    }
    }
}

/* ── Expr evaluation (derive.rs eval over Item/A/B/F environments) ────────── */

double oracle_eval_expr(const sanic_expr* ex, int i, const double* item, const double* a,
                        const double* b, const double* f) {
    const sanic_expr* e = &ex[i];
    switch (e->op) {
    case SANIC_EX_CONST: return e->value;
    case SANIC_EX_ITEM: return item[e->index];
    case SANIC_EX_A: return a[e->index];
    case SANIC_EX_B: return b[e->index];
    case SANIC_EX_F: return f[e->index];
    default: {
        double v[3] = {0, 0, 0};
        if (e->a >= 0) v[0] = oracle_eval_expr(ex, e->a, item, a, b, f);
        if (e->b >= 0) v[1] = oracle_eval_expr(ex, e->b, item, a, b, f);
        if (e->c >= 0) v[2] = oracle_eval_expr(ex, e->c, item, a, b, f);
        return oracle_apply_map(e->op, v);
    }
    }
}

/* ── dense evaluation of node trees ───────────────────────────────────────── */

typedef struct {
    const sanic_program_desc* d;
    double* const* buffers;       /* program buffer values                              */
    const double* fold;           /* FOLD placeholder values (epilogue), or NULL         */
    double** memo;                /* per node dense value, NULL until computed           */
} ctx_t;

static int64_t volume(const sanic_node* n) {
    int64_t v = 1;
    for (int i = 0; i < n->rank; i++) v *= n->shape[i];
    return v;
}

static void unflatten(int64_t flat, const int64_t* shape, int rank, int64_t* c) {
    for (int i = rank - 1; i >= 0; i--) {
        c[i] = flat % shape[i];
        flat /= shape[i];
    }
}

static int64_t flatten_at(const int64_t* c, const int64_t* shape, int rank) {
    int64_t f = 0;
    for (int i = 0; i < rank; i++) f = f * shape[i] + c[i];
    return f;
}

static const double* eval_node(ctx_t* cx, int idx);

static const double* eval_node(ctx_t* cx, int idx) {
    if (cx->memo[idx]) return cx->memo[idx];
    const sanic_node* n = &cx->d->nodes[idx];
    int64_t vol = volume(n);
    double* out = (double*)malloc(sizeof(double) * (size_t)(vol > 0 ? vol : 1));
    int64_t c[SANIC_MAX_RANK], s[SANIC_MAX_RANK];
    switch (n->kind) {
    case SANIC_NODE_INPUT:
        memcpy(out, cx->buffers[n->buffer], sizeof(double) * (size_t)vol);
        break;
    case SANIC_NODE_CONST:
        out[0] = n->value;
        break;
    case SANIC_NODE_IOTA:
        for (int64_t i = 0; i < vol; i++) out[i] = (double)i;
        break;
    case SANIC_NODE_COORDINATE:
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            out[i] = (double)c[n->dim];
        }
        break;
    case SANIC_NODE_FOLD:
        memcpy(out, cx->fold, sizeof(double) * (size_t)vol);
        break;
    case SANIC_NODE_MAP: {
        const double* ins[3];
        const sanic_node* in_n[3];
        for (int k = 0; k < n->n_in; k++) {
            ins[k] = eval_node(cx, n->in[k]);
            in_n[k] = &cx->d->nodes[n->in[k]];
        }
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            double args[3];
            for (int k = 0; k < n->n_in; k++) {
                const sanic_node* m = in_n[k];
                int lead = n->rank - m->rank;
                for (int j = 0; j < m->rank; j++) s[j] = m->shape[j] == 1 ? 0 : c[lead + j];
                args[k] = ins[k][flatten_at(s, m->shape, m->rank)];
            }
            out[i] = n->op == SANIC_OP_ROUND_Q8 ? oracle_round_q8(n->value, args[0]) : oracle_apply_map(n->op, args);
        }
        break;
    }
    case SANIC_NODE_REDUCE: {
        const sanic_node* m = &cx->d->nodes[n->in[0]];
        const double* src = eval_node(cx, n->in[0]);
        int64_t len = m->shape[n->dim];
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            for (int j = 0, o = 0; j < m->rank; j++) s[j] = j == n->dim ? 0 : c[o++];
            double acc = oracle_monoid_identity(n->op);
            for (int64_t r = 0; r < len; r++) {
                s[n->dim] = r;
                acc = oracle_monoid_combine(n->op, acc, src[flatten_at(s, m->shape, m->rank)]);
            }
            out[i] = acc;
        }
        break;
    }
    case SANIC_NODE_SCAN: {
        /* interp.rs eval_scan: the prefix fold up to and including this coordinate */
        const double* src = eval_node(cx, n->in[0]);
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            for (int j = 0; j < n->rank; j++) s[j] = c[j];
            double acc = oracle_monoid_identity(n->op);
            for (int64_t r = 0; r <= c[n->dim]; r++) {
                s[n->dim] = r;
                acc = oracle_monoid_combine(n->op, acc, src[flatten_at(s, n->shape, n->rank)]);
            }
            out[i] = acc;
        }
        break;
    }
    case SANIC_NODE_GATHER: {
        const sanic_node* m = &cx->d->nodes[n->in[0]];
        const sanic_node* ix = &cx->d->nodes[n->in[1]];
        const double* src = eval_node(cx, n->in[0]);
        const double* idx_v = eval_node(cx, n->in[1]);
        int64_t ic[SANIC_MAX_RANK];
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            for (int j = 0; j < ix->rank; j++) ic[j] = c[n->dim + j];
            double iv = idx_v[flatten_at(ic, ix->shape, ix->rank)];
            int64_t g = (int64_t)llround(iv);
            if (g < 0 || g >= m->shape[n->dim]) {
                fprintf(stderr, "oracle: gather index %lld out of bounds\n", (long long)g);
                abort();
            }
            for (int j = 0; j < m->rank; j++) {
                if (j < n->dim) s[j] = c[j];
                else if (j == n->dim) s[j] = g;
                else s[j] = c[j - 1 + ix->rank];
            }
            out[i] = src[flatten_at(s, m->shape, m->rank)];
        }
        break;
    }
    case SANIC_NODE_VIEW: {
        const sanic_node* m = &cx->d->nodes[n->in[0]];
        const double* src = eval_node(cx, n->in[0]);
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            int sd = 0;
            for (int j = 0; j < n->rank; j++) {
                int64_t flat = c[j];
                int g = n->group[j];
                for (int t = g - 1; t >= 0; t--) {
                    s[sd + t] = flat % m->shape[sd + t];
                    flat /= m->shape[sd + t];
                }
                sd += g;
            }
            out[i] = src[flatten_at(s, m->shape, m->rank)];
        }
        break;
    }
    case SANIC_NODE_REINDEX: {
        const sanic_node* m = &cx->d->nodes[n->in[0]];
        const double* src = eval_node(cx, n->in[0]);
        const int64_t* tab = cx->d->reindex;
        for (int64_t i = 0; i < vol; i++) {
            unflatten(i, n->shape, n->rank, c);
            int64_t p = n->map_offset;
            int oob = 0;
            for (int j = 0; j < m->rank; j++) {
                int64_t nt = tab[p++];
                int64_t v = tab[p++];
                for (int64_t t = 0; t < nt; t++) {
                    int64_t coef = tab[p++];
                    int64_t od = tab[p++];
                    v += coef * c[od];
                }
                if (v < 0 || v >= m->shape[j]) oob = 1;
                s[j] = v;
            }
            if (oob) {
                if (!n->padded) {
                    fprintf(stderr, "oracle: reindex out of bounds on an unpadded node\n");
                    abort();
                }
                out[i] = 0.0;
            } else {
                out[i] = src[flatten_at(s, m->shape, m->rank)];
            }
        }
        break;
    }
    default:
        fprintf(stderr, "oracle: unknown node kind %d\n", n->kind);
        abort();
    }
    cx->memo[idx] = out;
    return out;
}

static void ctx_init(ctx_t* cx, const sanic_program_desc* d, double* const* buffers, const double* fold) {
    cx->d = d;
    cx->buffers = buffers;
    cx->fold = fold;
    cx->memo = (double**)calloc((size_t)d->n_nodes, sizeof(double*));
}

static void ctx_free(ctx_t* cx) {
    for (int i = 0; i < cx->d->n_nodes; i++) free(cx->memo[i]);
    free(cx->memo);
}

int oracle_eval(const sanic_program_desc* d, int node, double* const* buffers, double* out) {
    ctx_t cx;
    ctx_init(&cx, d, buffers, NULL);
    const double* v = eval_node(&cx, node);
    memcpy(out, v, sizeof(double) * (size_t)volume(&d->nodes[node]));
    ctx_free(&cx);
    return 0;
}

/* ── run_carrier_split over one fused stage ─────────────────────────────── */

static void carrier_merge(const sanic_program_desc* d, const sanic_carrier* car, const double* a,
                          const double* b, double* out) {
    double tmp[SANIC_MAX_SLOTS];
    for (int s = 0; s < car->slots; s++) tmp[s] = oracle_eval_expr(d->exprs, car->combine[s], NULL, a, b, NULL);
    memcpy(out, tmp, sizeof(double) * (size_t)car->slots);
}

int oracle_fold_stage(const sanic_program_desc* d, int stage, double* const* buffers, int blocks,
                      double* fold_out, double* acc_out) {
    const sanic_stage* st = &d->stages[stage];
    const sanic_carrier* car = &st->carrier;
    int64_t n = st->stream;
    if (blocks < 1 || blocks > n) return 1;   /* interp.rs:588-593: every chunk non-empty */
    ctx_t cx;
    ctx_init(&cx, d, buffers, NULL);
    const double* leaf_v[SANIC_MAX_LEAVES];
    for (int l = 0; l < st->n_leaves; l++) leaf_v[l] = eval_node(&cx, st->leaf[l]);
    int64_t gvol = 1;
    for (int i = 0; i < st->rank; i++) gvol *= st->grid[i];
    int64_t g[SANIC_MAX_RANK], lc[SANIC_MAX_RANK];
    double item[SANIC_MAX_LEAVES], el[SANIC_MAX_SLOTS], acc[SANIC_MAX_SLOTS], tot[SANIC_MAX_SLOTS];
    for (int64_t gi = 0; gi < gvol; gi++) {
        unflatten(gi, st->grid, st->rank, g);
        for (int b = 0; b < blocks; b++) {
            int64_t lo = (int64_t)b * n / blocks, hi = (int64_t)(b + 1) * n / blocks;
            for (int s = 0; s < car->slots; s++) acc[s] = car->identity[s];
            for (int64_t i = lo; i < hi; i++) {
                for (int l = 0; l < st->n_leaves; l++) {
                    const sanic_node* ln = &d->nodes[st->leaf[l]];
                    for (int j = 0; j < ln->rank; j++) {
                        int bd = st->bind[l][j];
                        lc[j] = bd == SANIC_BIND_STREAM ? i : bd == SANIC_BIND_BCAST ? 0 : g[bd];
                    }
                    item[l] = leaf_v[l][flatten_at(lc, ln->shape, ln->rank)];
                }
                for (int s = 0; s < car->slots; s++) el[s] = oracle_eval_expr(d->exprs, car->into[s], item, NULL, NULL, NULL);
                carrier_merge(d, car, acc, el, acc);
            }
            if (b == 0) memcpy(tot, acc, sizeof(double) * (size_t)car->slots);
            else carrier_merge(d, car, tot, acc, tot);
        }
        if (acc_out) memcpy(acc_out + gi * car->slots, tot, sizeof(double) * (size_t)car->slots);
        fold_out[gi] = oracle_eval_expr(d->exprs, car->project, NULL, NULL, NULL, tot);
    }
    ctx_free(&cx);
    return 0;
}

/* Execute one stage into its output buffer, narrowing through the stored dtype. */
/* the stage's narrowing store: round_to of its storage dtype, Q8 with the buffer's scale */
static double store_round(const sanic_program_desc* d, const sanic_stage* st, double v) {
    if (st->out_dtype == SANIC_Q8) return oracle_round_q8((double)d->buffers[st->out_buffer].scale, v);
    return oracle_round_to(st->out_dtype, v);
}

int oracle_run_stage(const sanic_program_desc* d, int stage, double* const* buffers, int blocks) {
    const sanic_stage* st = &d->stages[stage];
    int64_t gvol = 1;
    for (int i = 0; i < st->rank; i++) gvol *= st->grid[i];
    double* out = buffers[st->out_buffer];
    double* val = (double*)malloc(sizeof(double) * (size_t)gvol);
    if (st->kind == SANIC_STAGE_FUSED) {
        int bl = blocks > 0 ? blocks : 1;
        if (bl > st->stream) bl = (int)st->stream;
        if (oracle_fold_stage(d, stage, buffers, bl, val, NULL)) { free(val); return 1; }
        if (st->epilogue >= 0) {
            ctx_t cx;
            ctx_init(&cx, d, buffers, val);
            const double* e = eval_node(&cx, st->epilogue);
            memcpy(val, e, sizeof(double) * (size_t)gvol);
            ctx_free(&cx);
        }
        for (int64_t i = 0; i < gvol; i++) out[i] = store_round(d, st, val[i]);
    } else {
        ctx_t cx;
        ctx_init(&cx, d, buffers, NULL);
        const double* v = eval_node(&cx, st->value);
        const double* w = st->where >= 0 ? eval_node(&cx, st->where) : NULL;
        const sanic_node* vn = &d->nodes[st->value];
        const sanic_node* wn = st->where >= 0 ? &d->nodes[st->where] : NULL;
        int64_t g[SANIC_MAX_RANK], s[SANIC_MAX_RANK];
        for (int64_t i = 0; i < gvol; i++) {
            /* value and condition broadcast against the grid as Map inputs do */
            unflatten(i, st->grid, st->rank, g);
            if (w) {
                int lead = st->rank - wn->rank;
                for (int j = 0; j < wn->rank; j++) s[j] = wn->shape[j] == 1 ? 0 : g[lead + j];
                if (w[flatten_at(s, wn->shape, wn->rank)] == 0.0) continue;
            }
            int lead = st->rank - vn->rank;
            for (int j = 0; j < vn->rank; j++) s[j] = vn->shape[j] == 1 ? 0 : g[lead + j];
            out[i] = store_round(d, st, v[flatten_at(s, vn->shape, vn->rank)]);
        }
        ctx_free(&cx);
    }
    free(val);
    return 0;
}

int oracle_run_program(const sanic_program_desc* d, double* const* buffers, int blocks) {
    for (int s = 0; s < d->n_stages; s++)
        if (oracle_run_stage(d, s, buffers, blocks)) return 1;
    return 0;
}
