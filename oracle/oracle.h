/*
 * oracle/oracle.h — TEST INFRASTRUCTURE (the checker), never the product path.
 *
 * Two independent CPU restatements of sanic's semantics:
 *   interp.c  — the generic dense-f64 interpreter over the flat program descriptor
 *               (/root/reference/src/interp.rs), schedule execution stage by stage;
 *   configs.c — fused f64 loops for the hot-path configurations (one f64 fold per output point,
 *               the shape of rustgen's generated code, /root/reference/src/rustgen.rs:151-245),
 *               cross-checked against interp.c on small shapes and used as the CPU baseline.
 */
#ifndef SANIC_ORACLE_H
#define SANIC_ORACLE_H
#include <stdint.h>
#include "../include/sanic_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* scalar.rs:120-152 */
double oracle_round_bf16(double v);
double oracle_round_to(int dtype, double v);
double oracle_round_q8(double scale, double v);
double oracle_round_f16(double v);
double oracle_apply_map(int op, const double* a);
double oracle_monoid_identity(int m);
double oracle_monoid_combine(int m, double a, double b);
double oracle_eval_expr(const sanic_expr* ex, int i, const double* item, const double* a,
                        const double* b, const double* f);

/* interp.rs eval of one node over its full shape */
int oracle_eval(const sanic_program_desc* d, int node, double* const* buffers, double* out);
/* interp.rs run_carrier_split of one fused stage: projected fold value per grid point and,
 * when acc_out != NULL, the raw accumulator (slots per grid point) */
int oracle_fold_stage(const sanic_program_desc* d, int stage, double* const* buffers, int blocks,
                      double* fold_out, double* acc_out);
int oracle_run_stage(const sanic_program_desc* d, int stage, double* const* buffers, int blocks);
int oracle_run_program(const sanic_program_desc* d, double* const* buffers, int blocks);

/* ── synthetic data ─────────────────────────────────────────────────────── */
/* The reference tests' xorshift64* generator (/root/reference/tests/metal.rs:86-96):
 * returns U(-1, 1) and advances *state. */
double oracle_lcg_next(uint64_t* state);
void oracle_lcg_fill(uint64_t seed, int64_t n, double* out);
/* Counter-based synthetic values (the twin of the product's device-side generator):
 * uniform(seed, i) in (-1, 1) and normal(seed, i) by Box–Muller; see configs.c. */
double oracle_synth_uniform(uint64_t seed, uint64_t i);
double oracle_synth_normal(uint64_t seed, uint64_t i);
/* fill `n` values of N(mean, std) (or U(lo, hi) when kind = 1) rounded to dtype, as f64 */
void oracle_synth_fill(uint64_t seed, int64_t n, int kind, double a, double b, int dtype,
                       double* out, int threads);
/* same, written as raw bf16 bit patterns */
void oracle_synth_fill_bf16(uint64_t seed, int64_t n, int kind, double a, double b,
                            uint16_t* out, int threads);

/* ── fused f64 loops (configs) ──────────────────────────────────────────── */
/* GQA attention softmax(Q·Kᵀ·scale + mask)·V, f64.
 * q [Hq, Sq, D], k [Hkv, Sk, D], v [Hkv, Sk, D] (or v_t [Hkv, D, Sk] when v_transposed),
 * query row i sits at absolute position q_pos0 + i. mask: 0 none, 1 causal (k <= pos),
 * 2 sliding window (pos - window < k <= pos), 3 prefix (k <= q_pos0, decode).
 * out [Hq, Sq, D]. */
void oracle_attention(const double* q, const double* k, const double* v, int Hq, int Hkv,
                      int Sq, int Sk, int D, int v_transposed, double scale, int mask,
                      int64_t q_pos0, int64_t window, double* out, int threads);
/* rotate-half RoPE in place, x [H, S, D], positions pos0 + s, inv_freq[D/2] */
void oracle_rope(double* x, int H, int S, int D, int64_t pos0, const double* inv_freq);
/* inv_freq(f) = θ^(−f/F) (nn.rs:196-199), with the llama-3 wavelength blend when llama3 */
void oracle_inv_freq(double theta, int F, int llama3, double* out);
/* y[m, n] = Σ_k x·g·W[k, n] / √(Σ_k x²/K + eps), W K-major [K, N] bf16 bits */
void oracle_rmsnorm_proj(const double* x, const double* g, const uint16_t* w, int M, int K,
                         int N, double eps, double* y, int threads);
/* y[m, n] = Σ_k x[m,k]·(u[n,k]·s[n,k/G] − z[n,k/G]); packed [N, K/2] low nibble = even k,
 * s, z [N, K/G] as f64 values */
void oracle_int4_matmul(const double* x, const uint8_t* packed, const double* s,
                        const double* z, int M, int K, int N, int G, double* y, int threads);

/* ── the Llama-3.2-1B-shape decode step (examples/llama3_2.rs:112-253) ───── */
typedef struct oracle_llama {
    int layers, hidden, heads, kv_heads, head_dim, ffn, vocab, capacity;
    double eps, theta;
    const uint16_t* embed;                    /* [vocab, hidden] bf16 (tied lm_head)     */
    const uint16_t* final_norm;               /* [hidden]                               */
    const uint16_t* attn_norm[32];            /* [hidden]                               */
    const uint16_t* mlp_norm[32];
    const uint16_t* wq[32];                   /* [heads·hd, hidden]  (out, in) rows      */
    const uint16_t* wk[32];                   /* [kv·hd, hidden]                        */
    const uint16_t* wv[32];
    const uint16_t* wo[32];                   /* [hidden, hidden]                       */
    const uint16_t* wg[32];                   /* [ffn, hidden]                          */
    const uint16_t* wu[32];
    const uint16_t* wd[32];                   /* [hidden, ffn]                          */
    uint16_t* kcache[32];                     /* [kv, capacity, hd] bf16                */
    uint16_t* vcache[32];                     /* [kv, hd, capacity] bf16 (transposed)   */
    int boundary_bf16;                        /* 1: every materialised intermediate is
                                               * stored bf16 (Policy { boundary: BF16 },
                                               * cost.rs:16-27); 0: f32                   */
} oracle_llama;

/* One decode step at `pos` for `token`; writes logits [vocab] (f32-rounded values) and
 * returns the greedy token (first index of the maximum). */
int64_t oracle_llama_step(oracle_llama* m, int64_t token, int64_t pos, double* logits,
                          int threads);

#ifdef __cplusplus
}
#endif
#endif
