/*
 * The synaptic-current op through libglif's C ABI from plain C (no Python, no torch), as a
 * TensorFlow custom op or any other C/C++ host would call it: a small recurrent table built
 * from host arrays in the reference's layout (synapses sorted by (post, pre), column
 * pre + n_post * (delay - 1)), weights and spikes in HIP device memory, then
 *   - glif_make_pre_ind_table against a stable counting sort written out here;
 *   - glif_syn_fwd, deterministic mode: bit-exact against the reference's accumulation order
 *     (per (b, post, r) from +0, events in ascending column, each term the fp32 product
 *     w * basis[syn_id][r]);
 *   - glif_syn_fwd, event mode, and glif_syn_bwd (dz and dW): within 1e-5 of each element's
 *     sum of absolute terms + 1e-6 of float64 sums;
 *   - error codes: a NULL table, a batch of 0 and a short workspace are refused.
 * Prints "PASS" and exits 0, or names the first failed check and exits 1.
 * Build: tests/c/Makefile (gcc, -ffp-contract=off so the C sums round as written).
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glif.h"

#define N_POST 193
#define D 3
#define NB 3
#define NT 4
#define B 4
#define N_COLS (D * N_POST)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) { /* xorshift64* */
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    return (uint32_t)((rng_state * 0x2545F4914F6CDD1Dull) >> 32);
}
static float rnd_unit(void) { return (float)(rnd() >> 8) / 16777216.0f; }

static int fail(const char *what) {
    printf("FAIL %s (%s)\n", what, glif_last_error());
    return 1;
}

#define HIP_OK(x) do { if ((x) != hipSuccess) return fail(#x); } while (0)

int main(void) {
    /* ---- network: each post draws distinct pres, sorted ascending (the reference order) ---- */
    enum { MAX_S = N_POST * 24 };
    static int64_t post[MAX_S], col[MAX_S];
    static uint8_t sid[MAX_S];
    static float w[MAX_S], basis[NT * NB];
    int64_t S = 0;
    for (int p = 0; p < N_POST; ++p) {
        int fan = 1 + (int)(rnd() % 23);
        static uint8_t taken[N_POST];
        memset(taken, 0, sizeof taken);
        for (int k = 0; k < fan; ++k) taken[rnd() % N_POST] = 1;
        for (int pre = 0; pre < N_POST; ++pre) {
            if (!taken[pre]) continue;
            post[S] = p;
            col[S] = pre + (int64_t)N_POST * (int64_t)(rnd() % D);
            sid[S] = (uint8_t)(rnd() % NT);
            w[S] = rnd_unit() * 2.0f - 1.0f;
            ++S;
        }
    }
    for (int i = 0; i < NT * NB; ++i) basis[i] = rnd_unit();
    static float z[B * N_COLS], dy[B * N_POST * NB];
    for (int i = 0; i < B * N_COLS; ++i) z[i] = (rnd() % 10 == 0) ? 1.0f : 0.0f;
    for (int i = 0; i < B * N_POST * NB; ++i) dy[i] = rnd_unit() - 0.5f;

    /* ---- pre_ind_table: stable counting sort by column ---- */
    static int32_t order[MAX_S], splits[N_COLS + 1], e_order[MAX_S], e_splits[N_COLS + 1];
    int64_t bad = -1;
    if (glif_make_pre_ind_table(col, S, N_COLS, order, splits, &bad) != GLIF_OK) return fail("pre_ind_table");
    memset(e_splits, 0, sizeof e_splits);
    for (int64_t k = 0; k < S; ++k) ++e_splits[col[k] + 1];
    for (int c = 0; c < N_COLS; ++c) e_splits[c + 1] += e_splits[c];
    {
        static int32_t fillp[N_COLS];
        memcpy(fillp, e_splits, sizeof fillp);
        for (int64_t k = 0; k < S; ++k) e_order[fillp[col[k]]++] = (int32_t)k;
    }
    if (memcmp(order, e_order, S * sizeof(int32_t)) || memcmp(splits, e_splits, sizeof splits))
        return fail("pre_ind_table differs from a stable counting sort");

    /* ---- device side ---- */
    glif_table *t = NULL;
    if (glif_table_create(post, col, sid, S, N_POST, N_COLS, D, basis, NT, NB, &t) != GLIF_OK)
        return fail("glif_table_create");
    float *d_w, *d_z, *d_dy, *d_I, *d_dz, *d_dw;
    void *d_ws;
    size_t ws_bytes = glif_syn_workspace(t, B);
    HIP_OK(hipMalloc((void **)&d_w, S * sizeof(float)));
    HIP_OK(hipMalloc((void **)&d_z, sizeof z));
    HIP_OK(hipMalloc((void **)&d_dy, sizeof dy));
    HIP_OK(hipMalloc((void **)&d_I, sizeof(float) * B * N_POST * NB));
    HIP_OK(hipMalloc((void **)&d_dz, sizeof z));
    HIP_OK(hipMalloc((void **)&d_dw, S * sizeof(float)));
    HIP_OK(hipMalloc(&d_ws, ws_bytes ? ws_bytes : 1));
    HIP_OK(hipMemcpy(d_w, w, S * sizeof(float), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_z, z, sizeof z, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_dy, dy, sizeof dy, hipMemcpyHostToDevice));
    if (glif_table_set_weights(t, d_w, NULL) != GLIF_OK) return fail("glif_table_set_weights");

    /* ---- forward, deterministic: the reference's order, bit for bit ---- */
    static float I[B * N_POST * NB], e_I[B * N_POST * NB];
    static double abs_I[B * N_POST * NB], f64_I[B * N_POST * NB];
    memset(e_I, 0, sizeof e_I);
    memset(abs_I, 0, sizeof abs_I);
    memset(f64_I, 0, sizeof f64_I);
    for (int b = 0; b < B; ++b)
        for (int c = 0; c < N_COLS; ++c) {
            if (!(z[b * N_COLS + c] > 0.0f)) continue;
            for (int32_t i = e_splits[c]; i < e_splits[c + 1]; ++i) {
                const int32_t k = e_order[i];
                for (int r = 0; r < NB; ++r) {
                    const float term = w[k] * basis[sid[k] * NB + r];
                    const size_t o = ((size_t)b * N_POST + (size_t)post[k]) * NB + r;
                    e_I[o] = e_I[o] + term;
                    abs_I[o] += fabs((double)term);
                    f64_I[o] += (double)w[k] * (double)basis[sid[k] * NB + r];
                }
            }
        }
    if (glif_syn_fwd(t, d_z, B, 0, GLIF_MODE_DETERMINISTIC, d_I, d_ws, ws_bytes, NULL) != GLIF_OK)
        return fail("glif_syn_fwd deterministic");
    HIP_OK(hipMemcpy(I, d_I, sizeof I, hipMemcpyDeviceToHost));
    if (memcmp(I, e_I, sizeof I)) return fail("deterministic forward not bit-exact");

    /* ---- forward, event ---- */
    if (glif_syn_fwd(t, d_z, B, 0, GLIF_MODE_EVENT, d_I, d_ws, ws_bytes, NULL) != GLIF_OK)
        return fail("glif_syn_fwd event");
    HIP_OK(hipMemcpy(I, d_I, sizeof I, hipMemcpyDeviceToHost));
    for (size_t o = 0; o < (size_t)B * N_POST * NB; ++o)
        if (fabs((double)I[o] - f64_I[o]) > 1e-5 * abs_I[o] + 1e-6) return fail("event forward outside the bar");

    /* ---- custom gradient ---- */
    static float dz[B * N_COLS], dw[MAX_S];
    static double e_dz[B * N_COLS], a_dz[B * N_COLS], e_dw[MAX_S], a_dw[MAX_S];
    memset(e_dz, 0, sizeof e_dz);
    memset(a_dz, 0, sizeof a_dz);
    memset(e_dw, 0, sizeof e_dw);
    memset(a_dw, 0, sizeof a_dw);
    for (int b = 0; b < B; ++b)
        for (int64_t k = 0; k < S; ++k) {
            double g = 0.0, ga = 0.0;
            for (int r = 0; r < NB; ++r) {
                const double x = (double)dy[((size_t)b * N_POST + (size_t)post[k]) * NB + r] * basis[sid[k] * NB + r];
                g += x;
                ga += fabs(x);
            }
            e_dz[(size_t)b * N_COLS + col[k]] += (double)w[k] * g;   /* dz: every synapse */
            a_dz[(size_t)b * N_COLS + col[k]] += fabs((double)w[k]) * ga;
            if (z[b * N_COLS + col[k]] > 0.0f) {                    /* dW: active ones */
                e_dw[k] += g;
                a_dw[k] += ga;
            }
        }
    if (glif_syn_bwd(t, d_z, d_dy, B, 0, d_dz, d_dw, d_ws, ws_bytes, NULL) != GLIF_OK) return fail("glif_syn_bwd");
    HIP_OK(hipMemcpy(dz, d_dz, sizeof dz, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(dw, d_dw, S * sizeof(float), hipMemcpyDeviceToHost));
    for (size_t i = 0; i < (size_t)B * N_COLS; ++i)
        if (fabs((double)dz[i] - e_dz[i]) > 1e-5 * a_dz[i] + 1e-6) return fail("dz outside the bar");
    for (int64_t k = 0; k < S; ++k)
        if (fabs((double)dw[k] - e_dw[k]) > 1e-5 * a_dw[k] + 1e-6) return fail("dW outside the bar");

    /* ---- refusals ---- */
    if (glif_syn_fwd(NULL, d_z, B, 0, GLIF_MODE_EVENT, d_I, d_ws, ws_bytes, NULL) != GLIF_EINVAL)
        return fail("a NULL table was not refused");
    if (glif_syn_fwd(t, d_z, 0, 0, GLIF_MODE_EVENT, d_I, d_ws, ws_bytes, NULL) != GLIF_EINVAL)
        return fail("B = 0 was not refused");
    if (ws_bytes > 0 &&
        glif_syn_bwd(t, d_z, d_dy, B, 0, d_dz, d_dw, d_ws, ws_bytes - 1, NULL) != GLIF_ENOMEM)
        return fail("a short workspace was not refused");

    HIP_OK(hipDeviceSynchronize());
    glif_table_destroy(t);
    hipFree(d_w);
    hipFree(d_z);
    hipFree(d_dy);
    hipFree(d_I);
    hipFree(d_dz);
    hipFree(d_dw);
    hipFree(d_ws);
    printf("PASS %lld synapses, %d x %d columns\n", (long long)S, B, N_COLS);
    return 0;
}
