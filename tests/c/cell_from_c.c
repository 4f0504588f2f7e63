/*
 * The fused GLIF_3 cell through libglif's C ABI from plain C (no Python, no torch): a small
 * network built in C -- recurrent table over D delay slots, LGN and background tables, per-neuron
 * parameters -- run for T ticks by glif_cell_forward (deterministic mode) and differentiated by
 * glif_cell_backward, against the C restatement (oracle/glif_oracle.c, compiled into this
 * program) on the same inputs:
 *   - spike trains, voltages and the final state (z_buf, v, r, asc, psc_rise, psc) bit-exact;
 *   - the three weight gradients of a random dL/dz within 1e-5 of the largest |dW| + 1e-6.
 * Prints "PASS" and exits 0, or names the first failed check and exits 1.
 * Build: tests/c/Makefile.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glif.h"
#include "glif_oracle.h"

#define N 150
#define D 3
#define NB 3
#define NT 4
#define NL 40
#define NK 6
#define B 3
#define T 40

static uint64_t rng_state = 0xD1B54A32D192ED03ull;
static uint32_t rnd(void) {
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    return (uint32_t)((rng_state * 0x2545F4914F6CDD1Dull) >> 32);
}
static float unit(void) { return (float)(rnd() >> 8) / 16777216.0f; }
static float uni(float lo, float hi) { return lo + (hi - lo) * unit(); }

static int fail(const char *what) {
    printf("FAIL %s (%s)\n", what, glif_last_error());
    return 1;
}
#define HIP_OK(x) do { if ((x) != hipSuccess) return fail(#x); } while (0)

/* One population in reference order: per post, distinct sources ascending, max_fan of them at
 * most; col = source + N * (delay - 1) over n_slots delay slots. */
typedef struct {
    int64_t S, n_cols;
    int64_t *post, *col, *order, *splits;
    uint8_t *sid;
    float *w;
} pop;

static int make_pop(pop *p, int n_src, int n_slots, int max_fan, float w_lo, float w_hi) {
    const int64_t cap = (int64_t)N * max_fan;
    p->post = malloc(cap * sizeof(int64_t));
    p->col = malloc(cap * sizeof(int64_t));
    p->sid = malloc(cap);
    p->w = malloc(cap * sizeof(float));
    p->n_cols = (int64_t)n_src * n_slots;
    p->order = malloc((cap + 1) * sizeof(int64_t));
    p->splits = malloc((p->n_cols + 1) * sizeof(int64_t));
    uint8_t *taken = malloc(n_src);
    if (!p->post || !p->col || !p->sid || !p->w || !p->order || !p->splits || !taken) return 1;
    p->S = 0;
    for (int n = 0; n < N; ++n) {
        memset(taken, 0, n_src);
        const int fan = 1 + (int)(rnd() % (unsigned)max_fan);
        for (int k = 0; k < fan; ++k) taken[rnd() % (unsigned)n_src] = 1;
        for (int s = 0; s < n_src; ++s) {
            if (!taken[s]) continue;
            p->post[p->S] = n;
            p->col[p->S] = s + (int64_t)n_src * (int64_t)(rnd() % (unsigned)n_slots);
            p->sid[p->S] = (uint8_t)(rnd() % NT);
            p->w[p->S] = uni(w_lo, w_hi);
            ++p->S;
        }
    }
    free(taken);
    int64_t bad = -1;
    return orc_csr_build(p->col, p->S, p->n_cols, p->order, p->splits, &bad);
}

static orc_table orc_of(const pop *p) {
    orc_table t = {p->S, p->n_cols, p->post, p->col, p->order, p->splits, p->w, p->sid};
    return t;
}

static int to_device(const pop *p, int n_post, int n_slots, const float *basis, glif_table **t, float **d_w) {
    if (glif_table_create(p->post, p->col, p->sid, p->S, n_post, p->n_cols, n_slots, basis, NT, NB, t) != GLIF_OK)
        return 1;
    if (hipMalloc((void **)d_w, (p->S ? p->S : 1) * sizeof(float)) != hipSuccess) return 1;
    if (hipMemcpy(*d_w, p->w, p->S * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return 1;
    return glif_table_set_weights(*t, *d_w, NULL) != GLIF_OK;
}

int main(void) {
    /* ---- network and parameters ---- */
    pop rec, lgn, bkg;
    if (make_pop(&rec, N, D, 16, -1.0f, 0.5f) || make_pop(&lgn, NL, 1, 6, 0.0f, 1.0f) ||
        make_pop(&bkg, NK, 1, 3, 0.0f, 0.8f))
        return fail("network build");
    static float decay[N], cf[N], asc_decay[2 * N], asc_amps[2 * N], syn_decay[NB], psc_initial[NB], basis[NT * NB];
    static int32_t tref[N];
    for (int n = 0; n < N; ++n) {
        decay[n] = expf(-1.0f / uni(5.0f, 30.0f));
        cf[n] = uni(0.02f, 0.06f);
        tref[n] = 1 + (int32_t)(rnd() % 5);
        for (int j = 0; j < 2; ++j) {
            asc_decay[2 * n + j] = uni(0.7f, 0.99f);
            asc_amps[2 * n + j] = uni(-0.2f, 0.2f);
        }
    }
    for (int q = 0; q < NB; ++q) {
        const float tau = uni(2.0f, 20.0f);
        syn_decay[q] = expf(-1.0f / tau);
        psc_initial[q] = 2.7182817f / tau;
    }
    for (int i = 0; i < NT * NB; ++i) basis[i] = unit();
    static uint8_t x_lgn[T * B * NL], x_bkg[T * B * NK];
    for (int i = 0; i < T * B * NL; ++i) x_lgn[i] = rnd() % 8 == 0;
    for (int i = 0; i < T * B * NK; ++i) x_bkg[i] = (uint8_t)(rnd() % 4 == 0 ? 1 + rnd() % 2 : 0);

    const float dt = 1.0f, lr_scale = 1.0f, vgd = 0.5f, rd = 0.3f, gstd = 0.5f, damp = 0.5f;
    orc_cell oc = {N, D, NB, NT, decay, cf, asc_decay, asc_amps, tref, syn_decay, psc_initial, basis,
                   dt, lr_scale, vgd, rd, gstd, damp, 1, 0, orc_of(&rec), orc_of(&lgn), orc_of(&bkg)};

    /* ---- oracle ---- */
    static float o_zbuf[B * D * N], o_v[B * N], o_asc[B * 2 * N], o_R[B * N * NB], o_P[B * N * NB], o_vout[T * B * N];
    static int32_t o_r[B * N];
    static uint8_t o_z[T * B * N], o_ref[T * B * N];
    if (orc_forward(&oc, T, B, x_lgn, x_bkg, o_zbuf, o_v, o_r, o_asc, o_R, o_P, o_z, o_vout, o_ref))
        return fail("oracle forward");
    long spikes = 0;
    for (int i = 0; i < T * B * N; ++i) spikes += o_z[i];
    if (spikes < 20) return fail("network nearly silent");
#ifdef ORACLE_ONLY
    printf("oracle: %ld spikes (%.2f %% of the entries)\n", spikes, 100.0 * spikes / (T * B * N));
    return 0;
#endif

    /* ---- the cell through the C ABI ---- */
    glif_table *t_rec, *t_lgn, *t_bkg;
    float *d_wr, *d_wl, *d_wb;
    if (to_device(&rec, N, D, basis, &t_rec, &d_wr) || to_device(&lgn, N, 1, basis, &t_lgn, &d_wl) ||
        to_device(&bkg, N, 1, basis, &t_bkg, &d_wb))
        return fail("tables");
    glif_cell_config cfg = {N, D, NB, dt, lr_scale, vgd, rd, gstd, damp, 1, 0};
    glif_cell *cell = NULL;
    if (glif_cell_create(&cfg, decay, cf, asc_decay, asc_amps, tref, syn_decay, psc_initial, t_rec, t_lgn, t_bkg,
                         &cell) != GLIF_OK)
        return fail("glif_cell_create");
    uint8_t *d_lgn, *d_bkg;
    float *d_z, *d_vout, *d_gz, *d_dwr, *d_dwl, *d_dwb;
    glif_state st;
    HIP_OK(hipMalloc((void **)&d_lgn, sizeof x_lgn));
    HIP_OK(hipMalloc((void **)&d_bkg, sizeof x_bkg));
    HIP_OK(hipMemcpy(d_lgn, x_lgn, sizeof x_lgn, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_bkg, x_bkg, sizeof x_bkg, hipMemcpyHostToDevice));
    HIP_OK(hipMalloc((void **)&st.z_buf, sizeof o_zbuf));
    HIP_OK(hipMalloc((void **)&st.v, sizeof o_v));
    HIP_OK(hipMalloc((void **)&st.r, B * N * sizeof(int16_t)));
    HIP_OK(hipMalloc((void **)&st.asc, sizeof o_asc));
    HIP_OK(hipMalloc((void **)&st.psc_rise, sizeof o_R));
    HIP_OK(hipMalloc((void **)&st.psc, sizeof o_P));
    HIP_OK(hipMemset(st.z_buf, 0, sizeof o_zbuf));
    HIP_OK(hipMemset(st.v, 0, sizeof o_v));
    HIP_OK(hipMemset(st.r, 0, B * N * sizeof(int16_t)));
    HIP_OK(hipMemset(st.asc, 0, sizeof o_asc));
    HIP_OK(hipMemset(st.psc_rise, 0, sizeof o_R));
    HIP_OK(hipMemset(st.psc, 0, sizeof o_P));
    HIP_OK(hipMalloc((void **)&d_z, sizeof(float) * T * B * N));
    HIP_OK(hipMalloc((void **)&d_vout, sizeof o_vout));
    const size_t ws_bytes = glif_cell_workspace(cell, B, T);
    void *d_ws;
    HIP_OK(hipMalloc(&d_ws, ws_bytes));
    if (glif_cell_forward(cell, B, T, GLIF_MODE_DETERMINISTIC, d_lgn, d_bkg, &st, d_z, d_vout, NULL, d_ws, ws_bytes,
                          NULL) != GLIF_OK)
        return fail("glif_cell_forward");

    static float z[T * B * N], vout[T * B * N], zbuf[B * D * N], v[B * N], asc[B * 2 * N], R[B * N * NB],
        P[B * N * NB];
    static int16_t r[B * N];
    HIP_OK(hipMemcpy(z, d_z, sizeof z, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(vout, d_vout, sizeof vout, hipMemcpyDeviceToHost));
    for (int i = 0; i < T * B * N; ++i)
        if ((z[i] > 0.0f) != (o_z[i] != 0)) return fail("spike trains differ");
    if (memcmp(vout, o_vout, sizeof vout)) return fail("voltages not bit-exact");
    HIP_OK(hipMemcpy(zbuf, st.z_buf, sizeof zbuf, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(v, st.v, sizeof v, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(r, st.r, sizeof r, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(asc, st.asc, sizeof asc, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(R, st.psc_rise, sizeof R, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(P, st.psc, sizeof P, hipMemcpyDeviceToHost));
    if (memcmp(zbuf, o_zbuf, sizeof zbuf) || memcmp(v, o_v, sizeof v) || memcmp(asc, o_asc, sizeof asc) ||
        memcmp(R, o_R, sizeof R) || memcmp(P, o_P, sizeof P))
        return fail("final state not bit-exact");
    for (int i = 0; i < B * N; ++i)
        if (r[i] != o_r[i]) return fail("refractory counters differ");

    /* ---- BPTT of a random dL/dz ---- */
    static float gz[T * B * N];
    for (int i = 0; i < T * B * N; ++i) gz[i] = uni(-1.0f, 1.0f);
    HIP_OK(hipMalloc((void **)&d_gz, sizeof gz));
    HIP_OK(hipMemcpy(d_gz, gz, sizeof gz, hipMemcpyHostToDevice));
    HIP_OK(hipMalloc((void **)&d_dwr, rec.S * sizeof(float)));
    HIP_OK(hipMalloc((void **)&d_dwl, lgn.S * sizeof(float)));
    HIP_OK(hipMalloc((void **)&d_dwb, bkg.S * sizeof(float)));
    if (glif_cell_backward(cell, B, T, d_gz, NULL, NULL, d_dwr, d_dwl, d_dwb, d_ws, ws_bytes, NULL) != GLIF_OK)
        return fail("glif_cell_backward");
    float *o_dw[3], *g_dw[3];
    const pop *pops[3] = {&rec, &lgn, &bkg};
    float *d_dw[3] = {d_dwr, d_dwl, d_dwb};
    for (int k = 0; k < 3; ++k) {
        o_dw[k] = calloc(pops[k]->S + 1, sizeof(float));
        g_dw[k] = malloc((pops[k]->S + 1) * sizeof(float));
        if (!o_dw[k] || !g_dw[k]) return fail("host allocation");
        HIP_OK(hipMemcpy(g_dw[k], d_dw[k], pops[k]->S * sizeof(float), hipMemcpyDeviceToHost));
    }
    if (orc_backward(&oc, T, B, x_lgn, x_bkg, NULL, o_z, o_ref, o_vout, gz, NULL, NULL, o_dw[0], o_dw[1], o_dw[2],
                     NULL))
        return fail("oracle backward");
    static const char *names[3] = {"dW_rec", "dW_lgn", "dW_bkg"};
    for (int k = 0; k < 3; ++k) {
        double scale = 0.0, err = 0.0;
        for (int64_t i = 0; i < pops[k]->S; ++i) {
            scale = fmax(scale, fabs((double)o_dw[k][i]));
            err = fmax(err, fabs((double)g_dw[k][i] - (double)o_dw[k][i]));
        }
        if (!(scale > 0.0)) return fail(names[k]);
        if (err > 1e-5 * scale + 1e-6) {
            printf("%s max err %.3g of max |dW| %.3g\n", names[k], err, scale);
            return fail(names[k]);
        }
    }

    HIP_OK(hipDeviceSynchronize());
    glif_cell_destroy(cell);
    glif_table_destroy(t_rec);
    glif_table_destroy(t_lgn);
    glif_table_destroy(t_bkg);
    printf("PASS %ld spikes over %d ticks x %d x %d neurons; %lld / %lld / %lld synapses\n", spikes, T, B, N,
           (long long)rec.S, (long long)lgn.S, (long long)bkg.S);
    return 0;
}
