/*
 * lamq_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C, single-threaded CPU restatement of the reference's per-matrix quantization
 * arithmetic (ShinMegamiBoson/lookatmyquant), used only as the checker for the HIP library:
 * by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg. Nothing in the
 * product path may link, load or call it.
 *
 * Every function names the reference lines it restates. Floating-point contraction is off
 * (the Makefile passes -ffp-contract=off); where a fused multiply-add is intended it is
 * written as fma(), so the order of operations is the one spelled out here and the HIP
 * kernels follow the same order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_EINVAL (-22)
#define ORC_ENOMEM (-12)

/* ---------------------------------------------------------------------------------------
 * Viterbi over a bitshift trellis: opgraph/codes.py:151-181.
 *   state s_t = (s_{t-1} * 2^k + b_t) mod 2^L emits C[s_t]
 *   cost_0(s) = (x_0 - C[s])^2, restricted to ((start << k) | b) & (2^L-1) when start is given
 *   best(r), arg(r) = min over h of cost[h*2^(L-k) + r], lowest h on ties     (codes.py:170)
 *   cost_t(r*2^k + b) = best(r) + (x_t - C[r*2^k + b])^2                      (codes.py:172)
 *   final state = argmin cost, lowest state on ties                            (codes.py:173)
 *   traceback s_{t-1} = (s_t >> k) + back_t[s_t >> k] * 2^(L-k)                (codes.py:176-179)
 * x and C are float32 (the reference casts both with .to(float32), codes.py:159,162).
 * ------------------------------------------------------------------------------------- */
static void viterbi_row(const float* xr, int T, const float* C, int L, int k, int64_t start,
                        float* cost, float* nc, uint8_t* back, int32_t* out)
{
    const int64_t S = (int64_t)1 << L, R = (int64_t)1 << (L - k);
    const int nb = 1 << k;
    for (int64_t s = 0; s < S; ++s) {
        float d = xr[0] - C[s];
        cost[s] = d * d;
    }
    if (start >= 0) {
        const int64_t r0 = start & (R - 1);
        for (int64_t s = 0; s < S; ++s)
            if ((s >> k) != r0) cost[s] = INFINITY;
    }
    for (int t = 1; t < T; ++t) {
        const float xt = xr[t];
        for (int64_t r = 0; r < R; ++r) {
            float best = cost[r];
            int arg = 0;
            for (int h = 1; h < nb; ++h) {
                float c = cost[(int64_t)h * R + r];
                if (c < best) { best = c; arg = h; }
            }
            back[(int64_t)t * R + r] = (uint8_t)arg;
            for (int b = 0; b < nb; ++b) {
                int64_t s = r * nb + b;
                float d = xt - C[s];
                nc[s] = best + d * d;
            }
        }
        float* tmp = cost; cost = nc; nc = tmp;
    }
    int64_t s = 0;
    for (int64_t i = 1; i < S; ++i)
        if (cost[i] < cost[s]) s = i;
    out[T - 1] = (int32_t)s;
    for (int t = T - 1; t > 0; --t) {
        int64_t r = s >> k;
        s = r + (int64_t)back[(int64_t)t * R + r] * R;
        out[t - 1] = (int32_t)s;
    }
}

/* x: B rows of T floats (row stride ldx); C: 2^L floats; start: NULL or B int64 states.
 * out: B*T int32 states, row-major. */
int orc_viterbi(const float* x, int64_t B, int T, int64_t ldx, const float* C, int L, int k,
                const int64_t* start, int32_t* out)
{
    if (!x || !C || !out || B < 0 || T < 1 || L < 1 || L > 20 || k < 1 || k > 8 || k >= L + 1 || k > L)
        return ORC_EINVAL;
    const int64_t S = (int64_t)1 << L, R = (int64_t)1 << (L - k);
    float* cost = (float*)malloc(sizeof(float) * S);
    float* nc = (float*)malloc(sizeof(float) * S);
    uint8_t* back = (uint8_t*)malloc((size_t)T * R);
    if (!cost || !nc || !back) { free(cost); free(nc); free(back); return ORC_ENOMEM; }
    for (int64_t b = 0; b < B; ++b)
        viterbi_row(x + b * ldx, T, C, L, k, start ? start[b] : -1, cost, nc, back, out + b * T);
    free(cost); free(nc); free(back);
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------------
 * The lazy block-LDLQ sweep of one row: opgraph/syntax.py:86-124.
 *   columns settled `width` at a time inside runs of `lazy` columns [b0, b1);
 *   E = T[cols] - q ;  z = E * U[cols,cols]^-1 (solve_triangular, upper, right)  (syntax.py:117-119)
 *   T[j+w : b1] -= z @ U[cols, j+w : b1]                                         (syntax.py:120)
 *   after the run: T[b1 :] -= Z @ U[b0:b1, b1:]                                   (syntax.py:123)
 * Order of floating-point operations used here (and by the HIP kernels):
 *   z[c]  = (E[c] fma-minus sum_{l<c} z[l]*U[j+l][j+c], l ascending) * (1 / U[j+c][j+c])
 *           (the diagonal through its reciprocal, as BLAS trsm kernels apply it)
 *   acc   = sum_l z[l]*U[j+l][col] as an fma chain from 0, l ascending;  T[col] = T[col] - acc
 *   trail = sum_c Z[c]*U[b0+c][col] as an fma chain from 0, c ascending; T[col] = T[col] - trail
 * ------------------------------------------------------------------------------------- */
static void solve_block(const double* E, int w, const double* U, int64_t ldU, int64_t j, double* z)
{
    for (int c = 0; c < w; ++c) {
        double acc = E[c];
        for (int l = 0; l < c; ++l) acc = fma(-z[l], U[(j + l) * ldU + j + c], acc);
        z[c] = acc * (1.0 / U[(j + c) * ldU + j + c]);
    }
}

static void inblock_update(double* Tr, const double* z, int w, const double* U, int64_t ldU, int64_t j,
                           int64_t c0, int64_t c1)
{
    for (int64_t col = c0; col < c1; ++col) {
        double acc = 0.0;
        for (int l = 0; l < w; ++l) acc = fma(z[l], U[(j + l) * ldU + col], acc);
        Tr[col] = Tr[col] - acc;
    }
}

static void trailing_update(double* Tr, int64_t n, const double* Z, int bw, const double* U, int64_t ldU,
                            int64_t b0, int64_t b1)
{
    for (int64_t col = b1; col < n; ++col) {
        double acc = 0.0;
        for (int c = 0; c < bw; ++c) acc = fma(Z[c], U[(b0 + c) * ldU + col], acc);
        Tr[col] = Tr[col] - acc;
    }
}

/* Row-trellis LDLQ: opgraph/codes.py:413-462 (ldlq_words with H) driving RowTrellisCode.step
 * (codes.py:397-404) through the project closure (codes.py:442-450), inside syntax.sweep.
 *   xs    = T[j : j+w] / S ,  ahead = T[j+w : j+w+look] / S   (fp64 divide, then float32 cast)
 *   path  = viterbi(cat(xs, ahead), start = state)[:w] ; state = path[w-1] (0 before column 0)
 *   q     = table64[path] * S  (the value returned to the sweep)
 * T: m x n (row stride ldT), modified in place. U: n x n upper (row stride ldU). S: m.
 * table64: 2^L doubles; Cf: the same table cast to float32. dead: NULL or n flags (T[:, dead] = 0,
 * syntax.py:101). states: m x n int32 output. */
int orc_ldlq_trellis(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                     const double* S, const double* table64, int L, int k, int width, int look, int lazy,
                     const uint8_t* dead, int32_t* states, double* before)
{
    if (!T || !U || !S || !table64 || !states || m < 0 || n < 1 || width < 1 || lazy < width || lazy % width
        || look < 0 || L < 1 || L > 20 || k < 1 || k > 8 || k > L)
        return ORC_EINVAL;
    const int64_t NS = (int64_t)1 << L, R = (int64_t)1 << (L - k);
    const int TV = width + look;
    float* Cf = (float*)malloc(sizeof(float) * NS);
    float* cost = (float*)malloc(sizeof(float) * NS);
    float* nc = (float*)malloc(sizeof(float) * NS);
    uint8_t* back = (uint8_t*)malloc((size_t)TV * R);
    float* xv = (float*)malloc(sizeof(float) * TV);
    int32_t* path = (int32_t*)malloc(sizeof(int32_t) * TV);
    double* Z = (double*)malloc(sizeof(double) * lazy);
    double* E = (double*)malloc(sizeof(double) * width);
    double* z = (double*)malloc(sizeof(double) * width);
    if (!Cf || !cost || !nc || !back || !xv || !path || !Z || !E || !z) {
        free(Cf); free(cost); free(nc); free(back); free(xv); free(path); free(Z); free(E); free(z);
        return ORC_ENOMEM;
    }
    for (int64_t s = 0; s < NS; ++s) Cf[s] = (float)table64[s];
    for (int64_t r = 0; r < m; ++r) {
        double* Tr = T + r * ldT;
        const double Sr = S[r];
        if (dead)
            for (int64_t c = 0; c < n; ++c)
                if (dead[c]) Tr[c] = 0.0;
        int64_t state = 0;
        for (int64_t b0 = 0; b0 < n; b0 += lazy) {
            const int64_t b1 = b0 + lazy < n ? b0 + lazy : n;
            for (int64_t j = b0; j < b1; j += width) {
                const int w = (int)((j + width <= b1) ? width : (b1 - j));
                int64_t na = n - (j + w);
                const int a = (int)(na < look ? na : look);
                if (before)
                    for (int c = 0; c < w; ++c) before[r * n + j + c] = Tr[j + c];
                for (int c = 0; c < w + a; ++c) xv[c] = (float)(Tr[j + c] / Sr);
                viterbi_row(xv, w + a, Cf, L, k, state, cost, nc, back, path);
                for (int c = 0; c < w; ++c) {
                    states[r * n + j + c] = path[c];
                    E[c] = Tr[j + c] - table64[path[c]] * Sr;
                }
                state = path[w - 1];
                solve_block(E, w, U, ldU, j, z);
                inblock_update(Tr, z, w, U, ldU, j, j + w, b1);
                for (int c = 0; c < w; ++c) Z[j - b0 + c] = z[c];
            }
            trailing_update(Tr, n, Z, (int)(b1 - b0), U, ldU, b0, b1);
        }
    }
    free(Cf); free(cost); free(nc); free(back); free(xv); free(path); free(Z); free(E); free(z);
    return ORC_OK;
}

/* Scalar LDLQ, width 1, two variants of the per-column projection:
 *  mode 0 -- opgraph/nested.py:104-147 (multirate_sweep, one rate of weight 1): the sweep runs on
 *            T = X / S already divided; index = first argmin_i (t - lv_i)^2 (nested.py:137-138);
 *            q = lv[index].
 *  mode 1 -- opgraph/codes.py:322-332 + 442-450 (ldlq_words with a ScalarCode): the sweep runs on
 *            X; index = bucketize(t / S, midpoints), halfway ties to the lower level
 *            (verbs.py:107-110); q = lv[index] * S.
 * Then E = T[j] - q; z = E / U[j][j]; T[col] = T[col] - z*U[j][col] for col in (j, b1)
 * (a K = 1 product: the product is rounded, then subtracted); trailing update as above. */
int orc_ldlq_scalar(double* T, int64_t m, int64_t n, int64_t ldT, const double* U, int64_t ldU,
                    const double* S, const double* levels, int K, int mode, int lazy,
                    const uint8_t* dead, int32_t* idx, double* before)
{
    if (!T || !U || !levels || !idx || m < 0 || n < 1 || K < 1 || K > 256 || lazy < 1 || (mode != 0 && mode != 1)
        || (mode == 1 && !S))
        return ORC_EINVAL;
    double* mids = (double*)malloc(sizeof(double) * (K > 1 ? K - 1 : 1));
    double* Z = (double*)malloc(sizeof(double) * lazy);
    if (!mids || !Z) { free(mids); free(Z); return ORC_ENOMEM; }
    for (int i = 0; i + 1 < K; ++i) mids[i] = (levels[i + 1] + levels[i]) / 2;
    for (int64_t r = 0; r < m; ++r) {
        double* Tr = T + r * ldT;
        if (dead)
            for (int64_t c = 0; c < n; ++c)
                if (dead[c]) Tr[c] = 0.0;
        for (int64_t b0 = 0; b0 < n; b0 += lazy) {
            const int64_t b1 = b0 + lazy < n ? b0 + lazy : n;
            for (int64_t j = b0; j < b1; ++j) {
                const double t = Tr[j];
                if (before) before[r * n + j] = t;
                int best = 0;
                double q;
                if (mode == 0) {
                    double dt = t - levels[0];
                    double bd = dt * dt;
                    for (int i = 1; i < K; ++i) {
                        double d = t - levels[i];
                        d = d * d;
                        if (d < bd) { bd = d; best = i; }
                    }
                    q = levels[best];
                } else {
                    const double ts = t / S[r];
                    while (best < K - 1 && ts > mids[best]) ++best;
                    q = levels[best] * S[r];
                }
                idx[r * n + j] = best;
                const double zj = (t - q) / U[j * ldU + j];
                for (int64_t col = j + 1; col < b1; ++col) {
                    double p = zj * U[j * ldU + col];
                    Tr[col] = Tr[col] - p;
                }
                Z[j - b0] = zj;
            }
            trailing_update(Tr, n, Z, (int)(b1 - b0), U, ldU, b0, b1);
        }
    }
    free(mids); free(Z);
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------------
 * KL(p_ref || p_q) per token, in float64: compiler.py:177-188 (the measure loop's kl()),
 * quantize.py:904-920, text_kl.py:57-61.
 *   lr = log_softmax(ref), lq = log_softmax(q);  kl = sum_v exp(lr_v) * (lr_v - lq_v)
 * Logits are bfloat16 (raw uint16 bit patterns). w: NULL or one weight per token; *wsum gets
 * sum_t w_t * kl_t and *wtot sum_t w_t (the measure variant divides one by the other).
 * ------------------------------------------------------------------------------------- */
static double bf16_to_double(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

int orc_kl_rows(const uint16_t* ref, const uint16_t* q, int64_t T, int64_t V, int64_t ldr, int64_t ldq,
                const float* w, double* kl_tok, double* wsum, double* wtot)
{
    if (!ref || !q || !kl_tok || T < 0 || V < 1) return ORC_EINVAL;
    double sw = 0.0, st = 0.0;
    for (int64_t t = 0; t < T; ++t) {
        const uint16_t* r = ref + t * ldr;
        const uint16_t* p = q + t * ldq;
        double mr = -INFINITY, mq = -INFINITY;
        for (int64_t v = 0; v < V; ++v) {
            double a = bf16_to_double(r[v]), b = bf16_to_double(p[v]);
            if (a > mr) mr = a;
            if (b > mq) mq = b;
        }
        double sr = 0.0, sq = 0.0;
        for (int64_t v = 0; v < V; ++v) {
            sr += exp(bf16_to_double(r[v]) - mr);
            sq += exp(bf16_to_double(p[v]) - mq);
        }
        const double lser = mr + log(sr), lseq = mq + log(sq);
        double kl = 0.0;
        for (int64_t v = 0; v < V; ++v) {
            double lr = bf16_to_double(r[v]) - lser, lq = bf16_to_double(p[v]) - lseq;
            kl += exp(lr) * (lr - lq);
        }
        kl_tok[t] = kl;
        const double wt = w ? (double)w[t] : 1.0;
        sw += wt * kl;
        st += wt;
    }
    if (wsum) *wsum = sw;
    if (wtot) *wtot = st;
    return ORC_OK;
}
