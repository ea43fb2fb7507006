/*
 * oracle/configs.c — TEST INFRASTRUCTURE: fused f64 restatements of the hot-path graphs and the
 * synthetic-data generators. Each function evaluates the graph semantics named in its comment
 * with one f64 fold per output point (the loop shape rustgen emits,
 * /root/reference/src/rustgen.rs:151-245); tests pin each against interp.c on small shapes.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

static double bf(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

static uint16_t to_bf16_bits(double v) {
    double r = oracle_round_bf16(v);
    float f = (float)r;
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

/* ── generators ───────────────────────────────────────────────────────────── */

double oracle_lcg_next(uint64_t* state) {
    /* xorshift64* exactly as /root/reference/tests/metal.rs:86-96 */
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return ((double)((x * 0x2545F4914F6CDD1DULL) >> 11) / (double)(1ULL << 53)) * 2.0 - 1.0;
}

void oracle_lcg_fill(uint64_t seed, int64_t n, double* out) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i++) out[i] = oracle_lcg_next(&s);
}

/* splitmix64 finaliser: a counter-based stream so that any element can be drawn independently
 * (parallel on the host and on the device). */
static uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double unit_open(uint64_t h) { return ((double)(h >> 11) + 0.5) / 9007199254740992.0; }

double oracle_synth_uniform(uint64_t seed, uint64_t i) {
    return unit_open(mix64(seed * 0xD1B54A32D192ED03ULL ^ mix64(i))) * 2.0 - 1.0;
}

double oracle_synth_normal(uint64_t seed, uint64_t i) {
    uint64_t base = seed * 0xD1B54A32D192ED03ULL;
    double u1 = unit_open(mix64(base ^ mix64(2 * i)));
    double u2 = unit_open(mix64(base ^ mix64(2 * i + 1)));
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static double synth_value(uint64_t seed, int64_t i, int kind, double a, double b) {
    if (kind == 1) return a + (b - a) * (oracle_synth_uniform(seed, (uint64_t)i) + 1.0) * 0.5;
    return a + b * oracle_synth_normal(seed, (uint64_t)i);
}

void oracle_synth_fill(uint64_t seed, int64_t n, int kind, double a, double b, int dtype,
                       double* out, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = oracle_round_to(dtype, synth_value(seed, i, kind, a, b));
}

void oracle_synth_fill_bf16(uint64_t seed, int64_t n, int kind, double a, double b,
                            uint16_t* out, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = to_bf16_bits(synth_value(seed, i, kind, a, b));
}

/* ── attention: nn.rs:27-105 scaled_dot_product_attention with GQA repeat (nn.rs:107-151) ── */

void oracle_attention(const double* q, const double* k, const double* v, int Hq, int Hkv,
                      int Sq, int Sk, int D, int v_transposed, double scale, int mask,
                      int64_t q_pos0, int64_t window, double* out, int threads) {
    int rep = Hq / Hkv;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        double* p = (double*)malloc(sizeof(double) * (size_t)Sk);
#pragma omp for collapse(2) schedule(dynamic, 4)
        for (int h = 0; h < Hq; h++) {
            for (int i = 0; i < Sq; i++) {
                int kvh = h / rep;
                const double* qi = q + ((int64_t)h * Sq + i) * D;
                int64_t pos = q_pos0 + i;
                double mx = -INFINITY;
                for (int t = 0; t < Sk; t++) {
                    const double* kt = k + ((int64_t)kvh * Sk + t) * D;
                    double s = 0.0;
                    for (int d = 0; d < D; d++) s += qi[d] * kt[d];
                    s *= scale;
                    int visible = 1;
                    if (mask == 1) visible = t <= pos;
                    else if (mask == 2) visible = t <= pos && t > pos - window;
                    else if (mask == 3) visible = t <= q_pos0;
                    /* causal_mask_like adds −1e30 (ir.rs:1511-1526); the decode prefix mask
                     * adds −∞ (llama3_2.rs:175-176). Both give exp(·) = 0 in f64 here. */
                    p[t] = visible ? s : -INFINITY;
                    if (p[t] > mx) mx = p[t];
                }
                double l = 0.0;
                for (int t = 0; t < Sk; t++) {
                    p[t] = p[t] == -INFINITY ? 0.0 : exp(p[t] - mx);
                    l += p[t];
                }
                double* o = out + ((int64_t)h * Sq + i) * D;
                for (int d = 0; d < D; d++) {
                    double acc = 0.0;
                    if (v_transposed) {
                        const double* vr = v + ((int64_t)kvh * D + d) * Sk;
                        for (int t = 0; t < Sk; t++) acc += p[t] * vr[t];
                    } else {
                        for (int t = 0; t < Sk; t++) acc += p[t] * v[((int64_t)kvh * Sk + t) * D + d];
                    }
                    o[d] = acc / l;
                }
            }
        }
        free(p);
    }
}

void oracle_inv_freq(double theta, int F, int llama3, double* out) {
    for (int f = 0; f < F; f++) {
        /* nn.rs:196-199: exp(f · (−ln θ / F)) */
        double inv = exp((double)f * (-log(theta) / (double)F));
        if (llama3) {
            /* examples/llama3_2.rs:91-107 with factor 32, original context 8192, low 1, high 4 */
            double wave = 2.0 * M_PI / inv;
            double low_wave = 8192.0 / 1.0, high_wave = 8192.0 / 4.0;
            double smooth = (8192.0 / wave - 1.0) / (4.0 - 1.0);
            double scaled = inv / 32.0;
            double blended = (1.0 - smooth) * scaled + smooth * inv;
            inv = low_wave < wave ? scaled : (wave < high_wave ? inv : blended);
        }
        out[f] = inv;
    }
}

void oracle_rope(double* x, int H, int S, int D, int64_t pos0, const double* inv_freq) {
    /* nn.rs:171-194: pair = 2 halves of the head dim, out = x·cos + flip(x)·sign·sin with
     * sign = −1 on the first half, +1 on the second. */
    int F = D / 2;
    for (int h = 0; h < H; h++)
        for (int s = 0; s < S; s++) {
            double* r = x + ((int64_t)h * S + s) * D;
            for (int f = 0; f < F; f++) {
                double ang = (double)(pos0 + s) * inv_freq[f];
                double c = cos(ang), sn = sin(ang);
                double a = r[f], b = r[f + F];
                r[f] = a * c - b * sn;
                r[f + F] = b * c + a * sn;
            }
        }
}

/* tests/laws.rs:621-646 closed form: Σ x·g·w / √(Σx²/n + ε) */
void oracle_rmsnorm_proj(const double* x, const double* g, const uint16_t* w, int M, int K,
                         int N, double eps, double* y, int threads) {
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        double* acc = (double*)malloc(sizeof(double) * (size_t)N);
#pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            const double* xm = x + (int64_t)m * K;
            double ss = 0.0;
            for (int k = 0; k < K; k++) ss += xm[k] * xm[k];
            double inv = 1.0 / sqrt(ss / (double)K + eps);
            for (int n = 0; n < N; n++) acc[n] = 0.0;
            for (int k = 0; k < K; k++) {
                double u = xm[k] * g[k];
                const uint16_t* wr = w + (int64_t)k * N;
                for (int n = 0; n < N; n++) acc[n] += u * bf(wr[n]);
            }
            for (int n = 0; n < N; n++) y[(int64_t)m * N + n] = acc[n] * inv;
        }
        free(acc);
    }
}

/* The reference's W4 matvec graph (tests/metal.rs:1179-1273) with the asymmetric dequant
 * u·s − z; with z = 8·s this is exactly the reference's signed I4 load times scale. */
void oracle_int4_matmul(const double* x, const uint8_t* packed, const double* s,
                        const double* z, int M, int K, int N, int G, double* y, int threads) {
    int ng = K / G;
#pragma omp parallel for collapse(2) num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            const uint8_t* row = packed + (int64_t)n * (K / 2);
            for (int k = 0; k < K; k++) {
                int u = (row[k >> 1] >> ((k & 1) * 4)) & 0xF;
                double w = (double)u * s[(int64_t)n * ng + k / G] - z[(int64_t)n * ng + k / G];
                acc += x[(int64_t)m * K + k] * w;
            }
            y[(int64_t)m * N + n] = acc;
        }
}

/* ── Llama decode step ────────────────────────────────────────────────────── */

static double f32r(double v) { return (double)(float)v; }

/* y[n] = Σ_k u[k]·W[n, k] for a row-major (out, in) bf16 weight */
static void matvec_rows(const double* u, const uint16_t* w, int N, int K, double* y, int threads) {
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int n = 0; n < N; n++) {
        const uint16_t* r = w + (int64_t)n * K;
        double acc = 0.0;
        for (int k = 0; k < K; k++) acc += u[k] * bf(r[k]);
        y[n] = acc;
    }
}

static double rms_inv(const double* x, int n, double eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    return 1.0 / sqrt(ss / (double)n + eps);
}

int64_t oracle_llama_step(oracle_llama* m, int64_t token, int64_t pos, double* logits,
                          int threads) {
    /* the storage of a materialised intermediate: the boundary policy's width */
#define BND(v) (m->boundary_bf16 ? oracle_round_bf16(v) : f32r(v))
    const int H = m->hidden, NH = m->heads, NKV = m->kv_heads, HD = m->head_dim, FF = m->ffn;
    const int F = HD / 2;
    double* x = (double*)malloc(sizeof(double) * H);
    double* u = (double*)malloc(sizeof(double) * (FF > H ? FF : H));
    double* q = (double*)malloc(sizeof(double) * NH * HD);
    double* kk = (double*)malloc(sizeof(double) * NKV * HD);
    double* vv = (double*)malloc(sizeof(double) * NKV * HD);
    double* att = (double*)malloc(sizeof(double) * NH * HD);
    double* o = (double*)malloc(sizeof(double) * (FF > H ? FF : H));
    double* gt = (double*)malloc(sizeof(double) * FF);
    double* up = (double*)malloc(sizeof(double) * FF);
    double* sc = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
    double inv_freq[128];
    oracle_inv_freq(m->theta, F, 1, inv_freq);

    /* embedding gather (llama3_2.rs:222) */
    for (int i = 0; i < H; i++) x[i] = bf(m->embed[token * H + i]);

    for (int l = 0; l < m->layers; l++) {
        /* RMSNorm fused into the q/k/v projections; stage outputs stored f32 */
        double r = rms_inv(x, H, m->eps);
        for (int i = 0; i < H; i++) u[i] = x[i] * bf(m->attn_norm[l][i]);
        matvec_rows(u, m->wq[l], NH * HD, H, q, threads);
        matvec_rows(u, m->wk[l], NKV * HD, H, kk, threads);
        matvec_rows(u, m->wv[l], NKV * HD, H, vv, threads);
        for (int i = 0; i < NH * HD; i++) q[i] = BND(q[i] * r);
        for (int i = 0; i < NKV * HD; i++) { kk[i] = BND(kk[i] * r); vv[i] = BND(vv[i] * r); }
        /* RoPE (llama3 schedule) on q and k at `pos`; in-place cache row writes in bf16
         * (update_cache, nn.rs:208-212; V stored transposed, llama3_2.rs:160-173) */
        oracle_rope(q, NH, 1, HD, pos, inv_freq);
        oracle_rope(kk, NKV, 1, HD, pos, inv_freq);
        for (int j = 0; j < NKV; j++)
            for (int d = 0; d < HD; d++) {
                double kv = oracle_round_bf16(kk[j * HD + d]);
                double vb = oracle_round_bf16(vv[j * HD + d]);
                m->kcache[l][((int64_t)j * m->capacity + pos) * HD + d] = to_bf16_bits(kv);
                m->vcache[l][((int64_t)j * HD + d) * m->capacity + pos] = to_bf16_bits(vb);
            }
        /* attention over the visible prefix t <= pos (mask −∞ beyond, llama3_2.rs:175-176) */
        for (int h = 0; h < NH; h++) {
            int j = h / (NH / NKV);
            double mx = -INFINITY;
            for (int64_t t = 0; t <= pos; t++) {
                const uint16_t* kr = m->kcache[l] + ((int64_t)j * m->capacity + t) * HD;
                double s = 0.0;
                for (int d = 0; d < HD; d++) s += q[h * HD + d] * bf(kr[d]);
                s *= 1.0 / sqrt((double)HD);
                sc[t] = s;
                if (s > mx) mx = s;
            }
            double lsum = 0.0;
            for (int64_t t = 0; t <= pos; t++) { sc[t] = exp(sc[t] - mx); lsum += sc[t]; }
            for (int d = 0; d < HD; d++) {
                const uint16_t* vr = m->vcache[l] + ((int64_t)j * HD + d) * m->capacity;
                double acc = 0.0;
                for (int64_t t = 0; t <= pos; t++) acc += sc[t] * bf(vr[t]);
                att[h * HD + d] = BND(acc / lsum);
            }
        }
        /* o projection + residual */
        matvec_rows(att, m->wo[l], H, NH * HD, o, threads);
        for (int i = 0; i < H; i++) x[i] = BND(x[i] + o[i]);
        /* MLP: gate/up with fused RMSNorm, silu(gate)·up in the down projection's leaf (as
         * its own bf16 stage under the bf16 policy) */
        r = rms_inv(x, H, m->eps);
        for (int i = 0; i < H; i++) u[i] = x[i] * bf(m->mlp_norm[l][i]);
        matvec_rows(u, m->wg[l], FF, H, gt, threads);
        matvec_rows(u, m->wu[l], FF, H, up, threads);
        for (int i = 0; i < FF; i++) {
            double g = BND(gt[i] * r), uu = BND(up[i] * r);
            u[i] = g * (1.0 / (1.0 + exp(-g))) * uu;
            if (m->boundary_bf16) u[i] = oracle_round_bf16(u[i]);
        }
        matvec_rows(u, m->wd[l], H, FF, o, threads);
        for (int i = 0; i < H; i++) x[i] = BND(x[i] + o[i]);
    }
    /* final norm fused into the tied lm_head, logits stored f32, first argmax */
    double r = rms_inv(x, H, m->eps);
    for (int i = 0; i < H; i++) u[i] = x[i] * bf(m->final_norm[i]);
    matvec_rows(u, m->embed, m->vocab, H, logits, threads);
    int64_t best = 0;
    for (int n = 0; n < m->vocab; n++) {
        logits[n] = BND(logits[n] * r);
        if (logits[n] > logits[best]) best = n;
    }
    free(x); free(u); free(q); free(kk); free(vv); free(att); free(o); free(gt); free(up); free(sc);
    return best;
#undef BND
}
