/*
 * glif_oracle.h -- types and entry points of the CPU restatement (glif_oracle.c).
 * TEST INFRASTRUCTURE ONLY: included by the oracle itself and by the C test programs under
 * tests/c; the product never includes it.
 */
#ifndef GLIF_ORACLE_H
#define GLIF_ORACLE_H

#include <stdint.h>

#define ORC_EINVAL (-22)
#define ORC_ERANGE (-34)
#define ORC_ENOMEM (-12)

/* One synapse population in reference order, with its pre_ind_table (orc_csr_build). */
typedef struct {
    int64_t S, n_cols;
    const int64_t *post, *col, *order, *row_splits;
    const float *w;
    const uint8_t *sid;
} orc_table;

/* The cell's parameters (models.py:450-611 after its derivations) and three populations. */
typedef struct {
    int64_t N, D;
    int32_t nb, n_types;
    const float *decay, *cf;            /* [N] */
    const float *asc_decay, *asc_amps;  /* [N][2] */
    const int32_t *tref;                /* [N] */
    const float *syn_decay, *psc_initial; /* [nb] */
    const float *basis;                 /* [n_types][nb] */
    float dt, lr_scale, vgd, rd, gauss_std, damp;
    int32_t pseudo_gauss, hard_reset;
    orc_table rec, lgn, bkg;
} orc_cell;

int orc_set_threads(int n);
int orc_csr_build(const int64_t *cols, int64_t S, int64_t n_cols, int64_t *order, int64_t *row_splits,
                  int64_t *bad_index);
int64_t orc_where_gt0(const float *z, int64_t rows, int64_t cols, int64_t *out);
void orc_syn_fwd(int B, int64_t n_post, int64_t n_cols, int nb, const float *act, int use_count,
                 const int64_t *post, const float *w, const uint8_t *sid, const float *basis,
                 const int64_t *order, const int64_t *row_splits, float *I);
void orc_syn_bwd(int B, int64_t n_post, int64_t n_cols, int nb, int64_t S, const float *act, int use_count,
                 const int64_t *post, const int64_t *col, const float *w, const uint8_t *sid, const float *basis,
                 const int64_t *order, const int64_t *row_splits, const float *dy, float *dz, float *dW,
                 float *scratch);
int orc_forward(const orc_cell *c, int T, int B, const uint8_t *lgn, const uint8_t *bkg, float *zbuf, float *v,
                int32_t *r, float *asc, float *R, float *P, uint8_t *z_out, float *v_out, uint8_t *ref_out);
int orc_backward(const orc_cell *c, int T, int B, const uint8_t *lgn, const uint8_t *bkg, const float *zbuf0,
                 const uint8_t *zs, const uint8_t *refs, const float *vs, const float *gz_loss,
                 const float *gz_neuron, const float *gv_loss, float *dW_rec, float *dW_lgn, float *dW_bkg,
                 float *gz_out);

#endif
