/*
 * glif.h -- C ABI of libglif, the MI355X (gfx950) implementation of the GLIF_3 V1
 * cell hot path of JavierGalvan9/V1_GLIF_model (`v1_model_utils/models.py`).
 *
 * Conventions
 *   - Every call returns GLIF_OK (0) or a negative glif_status; glif_last_error()
 *     returns a thread-local message for the last failing call.  No C++ exception
 *     crosses this boundary.
 *   - Device pointers are plain HIP device allocations (e.g. torch tensors' data).
 *     Host pointers are marked "host".  All device work is stream-ordered on the
 *     caller's stream (a hipStream_t passed as void*, NULL = default stream); no
 *     call synchronises the device except glif_table_create / glif_cell_create
 *     (one-time uploads).
 *   - Index limits: n_syn < 2^31, n_post and presynaptic ids < 2^24, <= 256
 *     synapse types, <= 256 delay slots, B <= 32, n_basis <= 8.
 *
 * The reference has no FFI: its boundary is the Python op and the Keras cell API.
 * Each entry point below names the reference function it replaces; the Python
 * mirror in v1_glif_model_amd/ keeps the reference names and argument order.
 */
#ifndef GLIF_H
#define GLIF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    GLIF_OK = 0,
    GLIF_EINVAL = -22,   /* bad argument (the reference raises ValueError)       */
    GLIF_ERANGE = -34,   /* index out of range (models.py:308-314 ValueError)     */
    GLIF_ENOMEM = -12,   /* host or device allocation failed / workspace too small */
    GLIF_EHIP = -1000    /* a HIP runtime call failed                            */
} glif_status;

typedef enum {
    GLIF_MODE_EVENT = 0,         /* event-driven push of active columns, fp32 atomics;     */
                                 /* sums order-free, within 1e-5 of the reference's (a     */
                                 /* table with columns > 2048 synapses, whose inputs each  */
                                 /* fan out to thousands of posts, is pulled instead)      */
    GLIF_MODE_DETERMINISTIC = 1  /* post-row pull in the reference's accumulation order   */
} glif_mode;

typedef struct glif_table glif_table;  /* one synapse population, device resident */
typedef struct glif_cell glif_cell;    /* GLIF_3 parameters + rec/LGN/bkg tables  */

const char *glif_last_error(void);
int glif_version(void);

/* ----------------------------------------------- CSR (pre_ind_table) --------
 * make_pre_ind_table (models.py:343-373 with _validate_inputs :299-315 and
 * _build_csr_order_numba :317-341): stable counting sort of synapse ids by
 * presynaptic column.  host in: cols [n_syn] int64 (column 1 of `indices`);
 * host out: order [n_syn] int32, row_splits [n_source + 1] int32.
 * GLIF_EINVAL if n_source <= 0, GLIF_ERANGE (bad_index set) on an id outside
 * [0, n_source). */
int glif_make_pre_ind_table(const int64_t *cols, int64_t n_syn, int64_t n_source,
                            int32_t *order, int32_t *row_splits, int64_t *bad_index);

/* -------------------------------------------------- spike compaction --------
 * tf.where(z > 0) (models.py:128, 823-826, 890): row-major list of (row, col)
 * pairs of a [rows][cols] float32 device array.  device out: pairs [<= rows*cols][2]
 * int64 and count [1] int64.  Workspace: glif_where_workspace(). */
size_t glif_where_workspace(int64_t rows, int64_t cols);
int glif_where_gt0(const float *z, int64_t rows, int64_t cols, int64_t *pairs, int64_t *count,
                   void *ws, size_t ws_bytes, void *stream);

/* ----------------------------------------------------- synapse tables -------
 * Synapse table of one population, built from the arrays V1Column.__init__ keeps
 * (models.py:625-773).  host in, reference order (sorted by (post, pre)):
 *   post [n_syn] int64, col [n_syn] int64 (pre + n_post*(delay-1) for the recurrent
 *   table, pre for LGN/background), syn_id [n_syn] uint8,
 *   basis [n_types][n_basis] float32 (synaptic_basis_weights).
 * n_delay_slots = D for the recurrent table (n_cols = D * n_post), 1 for inputs. */
int glif_table_create(const int64_t *post, const int64_t *col, const uint8_t *syn_id,
                      int64_t n_syn, int32_t n_post, int64_t n_cols, int32_t n_delay_slots,
                      const float *basis, int32_t n_types, int32_t n_basis, glif_table **out);
void glif_table_destroy(glif_table *t);
int64_t glif_table_n_syn(const glif_table *t);
/* Device pointers owned by the table: the bit-exact pre_ind_table (order int32 [n_syn],
 * row_splits int32 [n_cols + 1]). */
int glif_table_pre_ind(const glif_table *t, const int32_t **order, const int32_t **row_splits);
/* refresh_recurrent_weight_shadow (models.py:966-976): copy the trainable weight
 * vector w [n_syn] (device, reference order) into the table's column- and
 * row-grouped copies.  Must be called before use and after every weight update.  It
 * writes the table's weight copies (and stages through a buffer of the table's), so calls
 * on one table must not overlap, and no call that reads the table may run beside one.
 * A table without synapses has no weights: w may then be NULL and nothing is launched. */
int glif_table_set_weights(glif_table *t, const float *w, void *stream);

/* --------------------------------------- synaptic-current op (fwd, grad) ----
 * calculate_synaptic_currents (models.py:103-263).
 * Forward: z [B][n_cols] float32 device (event where z > 0; with counts != 0 the
 * value scales the weight as the background current does, models.py:917-931);
 * out: I [B*n_post][n_basis] float32 (overwritten).  mode: glif_mode.
 * ws: glif_syn_workspace(t, B) bytes of device memory.  The calls that pull spikes -- mode
 * GLIF_MODE_DETERMINISTIC, or a table with a column longer than 2048 synapses, with counts == 0
 * -- build batch masks in it and return GLIF_ENOMEM without it; the event push and the pull of
 * counts use none and accept ws = NULL. */
size_t glif_syn_workspace(const glif_table *t, int32_t B);
int glif_syn_fwd(const glif_table *t, const float *z, int32_t B, int32_t counts, int32_t mode,
                 float *I, void *ws, size_t ws_bytes, void *stream);
/* No counterpart in the reference.  glif_syn_fwd for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the same arguments, results and errors minus the workspace, whose place takes a static
 * device array of GLIF_NOALLOC_SCRATCH_BYTES in the library -- one per GPU the library runs
 * on, held until the process ends, its address looked up on the first call on each device.
 * The forward needs about 4 bytes of scratch per column (n_cols; the deterministic row pull's
 * batch masks and activity bits -- the event push uses none, but the limit holds for both
 * modes): 32 MiB covers tables of up to ~8M columns (the 230k-neuron, 5-delay recurrent table
 * has 1.15M); larger ones fail with GLIF_ENOMEM.  Calls on one GPU share the array: calls that overlap on one GPU (other
 * streams, other threads) race, so serialise them.  The stream must belong to the calling
 * thread's current device.  No allocation, no synchronisation. */
#define GLIF_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int glif_syn_fwd_noalloc(const glif_table *t, const float *z, int32_t B, int32_t counts, int32_t mode,
                         float *I, void *stream);

/* Custom gradient (models.py:174-261): dy [B*n_post][n_basis] float32 device;
 * out dz [B][n_cols] (the gradient w.r.t. rec_z_buf, dense over all synapses; NULL
 * to skip) and dw [n_syn] (w.r.t. weight_values, reference order; NULL to skip),
 * both overwritten. */
int glif_syn_bwd(const glif_table *t, const float *z, const float *dy, int32_t B, int32_t counts,
                 float *dz, float *dw, void *ws, size_t ws_bytes, void *stream);

/* --------------------------------------------------- GLIF_3 cell, BPTT -------
 * V1Column (models.py:450-1135) run over T steps on one stream. */
typedef struct {
    int32_t n_neurons;
    int32_t n_delay;            /* max_delay (D) */
    int32_t n_basis;            /* nb */
    float dt;
    float lr_scale;
    float voltage_gradient_dampening;  /* vgd, models.py:1010 */
    float recurrent_dampening;         /* rd,  models.py:1081 */
    float gauss_std;
    float dampening_factor;
    int32_t pseudo_gauss;       /* 1: spike_gauss surrogate, 0: triangular spike_function */
    int32_t hard_reset;
} glif_cell_config;

/* host in: decay, current_factor [N]; asc_decay, asc_amps [N][2]; t_ref_steps [N]
 * int32; syn_decay, psc_initial [n_basis].  The tables are borrowed (not owned) and
 * must outlive the cell; their n_post must equal n_neurons and rec must have
 * n_delay slots. */
int glif_cell_create(const glif_cell_config *cfg, const float *decay, const float *current_factor,
                     const float *asc_decay, const float *asc_amps, const int32_t *t_ref_steps,
                     const float *syn_decay, const float *psc_initial, glif_table *rec,
                     glif_table *lgn, glif_table *bkg, glif_cell **out);
void glif_cell_destroy(glif_cell *c);

/* The state tuple of models.py:1030-1056, device pointers, reference layouts:
 * z_buf [B][D*N] f32, v [B][N] f32, r [B][N] int16 (refractory steps left),
 * asc [B][N*2] f32, psc_rise [B][N*nb] f32, psc [B][N*nb] f32. */
typedef struct {
    float *z_buf;
    float *v;
    int16_t *r;
    float *asc;
    float *psc_rise;
    float *psc;
} glif_state;

/* Workspace of a T-step rollout at batch B: rings, spike history, saved voltages
 * and the backward's adjoint buffers.  The same workspace must be passed to the
 * glif_cell_backward that follows a glif_cell_forward. */
size_t glif_cell_workspace(const glif_cell *c, int32_t B, int32_t T);

/* Forward rollout (the Keras RNN over V1Column.call, models.py:1317-1322).
 * device in: lgn [T][B][n_lgn] uint8 (spike where > 0), bkg [T][B][n_bkg] uint8
 * (Poisson counts; TF's stateless Poisson stream is not reproducible, so counts are
 * an input).  state: in/out.  out (each may be NULL): z [T][B][N] f32, v [T][B][N]
 * f32 (the cell outputs), spike_count [B][N] int32 (accumulated over the ticks of the
 * trimming window, glif_cell_set_trim; all ticks by default). */
int glif_cell_forward(glif_cell *c, int32_t B, int32_t T, int32_t mode, const uint8_t *lgn,
                      const uint8_t *bkg, glif_state *state, float *z_out, float *v_out,
                      int32_t *spike_count, void *ws, size_t ws_bytes, void *stream);

/* BPTT through the last glif_cell_forward on `ws` (zero initial state assumed for
 * the adjoint; gradients do not flow into the initial state).  All its scratch, the
 * reordering of the weight gradients included, lives in `ws`, so backwards on one cell with
 * workspaces of their own may run on different streams at once.
 * device in (each may be NULL): gz [T][B][N] dL/dz, gz_neuron [N] dL/dz broadcast
 * over b and the ticks of the trimming window, gv [T][B][N] dL/dv.  out (each may be NULL): dw_rec, dw_lgn, dw_bkg,
 * gradients of the three weight vectors in reference order (overwritten). */
int glif_cell_backward(glif_cell *c, int32_t B, int32_t T, const float *gz,
                       const float *gz_neuron, const float *gv, float *dw_rec, float *dw_lgn,
                       float *dw_bkg, void *ws, size_t ws_bytes, void *stream);

/* ----------------------------------------------- one step's backward --------
 * The gradient of one V1Column.call (models.py:1059-1135) for callers that keep the Keras
 * RNN (models.py:1317-1322) and let a tape differentiate it step by step (the reference's
 * GradientTape over the RNN, multi_training.py:368-372, 485-493).  The step's forward is
 * glif_cell_forward with T = 1 (its state in/out and its z, v outputs).
 * Gradients of the state tuple (r and noise_step have none); every field may be NULL. */
typedef struct {
    float *z_buf;      /* [B][D*N] */
    float *v;          /* [B][N] */
    float *asc;        /* [B][N*2] */
    float *psc_rise;   /* [B][N*nb] */
    float *psc;        /* [B][N*nb] */
} glif_state_grad;

size_t glif_step_workspace(const glif_cell *c, int32_t B);
/* device in: lgn [B][n_lgn] u8 and bkg [B][n_bkg] u8 (the step's inputs; needed for dw_lgn /
 * dw_bkg), z_buf [B][D*N] the step's OLD spike buffer (needed for g_old->z_buf and dw_rec),
 * v_new [B][N] the step's output voltage, r_new [B][N] int16 its new refractory counter;
 * gz, gv [B][N] dL/dz and dL/dv of the step's outputs (nullable); g_new: dL/d(new state)
 * (nullable, as its fields).  out: g_old, dL/d(old state) for each non-NULL field
 * (overwritten); dw_rec, dw_lgn, dw_bkg [n_syn] this step's weight gradients in reference
 * order (nullable, overwritten).  With the straight-through dampening of models.py:284-296
 * (rd on the spike buffer, 1 - vgd on v), stop_gradient on the previous spikes and r, the
 * surrogate masked where r_new > 0, and hard reset cutting the voltage path there. */
int glif_step_backward(glif_cell *c, int32_t B, const uint8_t *lgn, const uint8_t *bkg, const float *z_buf,
                       const float *v_new, const int16_t *r_new, const float *gz, const float *gv,
                       const glif_state_grad *g_new, glif_state_grad *g_old, float *dw_rec, float *dw_lgn,
                       float *dw_bkg, void *ws, size_t ws_bytes, void *stream);

/* Fused voltage regularization (VoltageRegularization, loss_functions.py:1047-1119):
 * mode 0 off, 1 "range" (penalty relu(|v - 0.5| - 0.5)^2), 2 "threshold" ((v - 1)^2),
 * loss = cost * mean over (T, B, N) of the penalty of the cell's output voltages.  While
 * enabled, glif_cell_backward adds its gradient to dL/dv inside the adjoint (no dense dL/dv
 * tensor), and glif_cell_voltage_loss reduces the loss of the last forward on `ws` into
 * loss_out (device f32) in a fixed order. */
int glif_cell_set_voltage_loss(glif_cell *c, int32_t mode, float cost);
int glif_cell_voltage_loss(glif_cell *c, int32_t B, int32_t T, float *loss_out, void *ws, size_t ws_bytes,
                           void *stream);

/* The core mask of the voltage regularization (VoltageRegularization's core_mask,
 * loss_functions.py:1105-1109: the penalty's mean runs over the selected neurons only):
 * mask device uint8 [n_neurons] (nonzero = selected; the caller keeps it alive while the
 * loss is enabled) and the number it selects, or NULL for every neuron. */
int glif_cell_set_voltage_mask(glif_cell *c, const uint8_t *mask, int32_t n_selected);

/* Spike trimming of the rate losses (spike_trimming, loss_functions.py:604-611, applied
 * by SpikeRateDistributionTarget.__call__ :873-881): of a T-tick forward, only ticks
 * [pre_delay, T - post_delay) add to spike_count, and glif_cell_backward broadcasts
 * gz_neuron over those ticks only.  Default 0, 0 (every tick). */
int glif_cell_set_trim(glif_cell *c, int32_t pre_delay, int32_t post_delay);

/* Layout of the backward's per-synapse-type projection G (no counterpart in the reference,
 * whose gradient projects dy through the basis per receptor, models.py:182-241): rows per
 * post neuron (n_types, or fewer when no post receives more than three quarters of the
 * types: then *compact = 1 and each post keeps rows for its own types only). */
int glif_cell_g_layout(const glif_cell *c, int32_t *rows_per_post, int32_t *compact);
/* Choose the layout (for timing the two against each other): compact 0 = type-major rows,
 * 1 = compact rows (GLIF_EINVAL when the cell has none).  The workspace size follows the
 * layout: query glif_cell_workspace again.  What a backward reads of its forward sits at
 * offsets that do not depend on the layout, so a backward after a switch is valid on a
 * workspace large enough for the new layout (GLIF_ENOMEM otherwise). */
int glif_cell_set_g_layout(glif_cell *c, int32_t compact);

/* ----------------------------------------------------------------- losses -----
 * Rate-distribution loss (SpikeRateDistributionTarget.__call__, loss_functions.py:873-889
 * -> compute_spike_rate_target_loss :634-664 -> compute_spike_rate_distribution_loss
 * :666-681 -> huber_quantile_loss :626-632, kappa 0.002 at :680).
 * rate[n] = (sum_r count[r][n]) / n_samples (count [count_rows][n_neurons] int32,
 * device: the forward's spike_count, rows = B, n_samples = window ticks x B).
 * Populations: ids [pop_ptr[n_pop]] int32 (device) holds the selected neuron ids of
 * population k at [pop_ptr[k], pop_ptr[k+1]) (pop_ptr host, n_pop <= 64, ids distinct);
 * targets (device f32, same layout) each population's ascending sampled target rates.
 * Each population's rates are sorted ascending; ties are ordered by a Philox4x32-10 word
 * (seed, offset + position) when shuffle != 0 (the reference's tf.random.shuffle), else
 * by position in ids.  loss_out (device f32) = rate_cost * sum of the Huber-quantile
 * terms / pop_ptr[n_pop] (NaN when an id is outside [0, n_neurons) or a count exceeds
 * n_samples); gz_neuron [n_neurons] (device f32) += dL/drate / n_samples, the per-tick
 * dL/dz for glif_cell_backward's gz_neuron.  Workspace: glif_rate_loss_workspace. */
/* Mean-squared firing-rate error, the loss the benchmark's training configuration names (no
 * counterpart in the reference's loss_functions.py; the per-neuron form of its rate losses):
 * rbar[n] = (sum_r count[r][n]) / n_samples, loss_out = sum_n (rbar[n] - targets[n])^2 /
 * n_neurons (fixed order), gz_neuron[n] += (rbar[n] - targets[n]) * 2 / (n_neurons *
 * n_samples), the per-tick dL/dz.  Workspace: glif_rate_mse_workspace() bytes. */
size_t glif_rate_mse_workspace(void);
int glif_rate_mse_loss(const int32_t *count, int32_t count_rows, int32_t n_neurons, int32_t n_samples,
                       const float *targets, float *loss_out, float *gz_neuron, void *ws, size_t ws_bytes,
                       void *stream);

size_t glif_rate_loss_workspace(int64_t n_sel);
int glif_rate_dist_loss(const int32_t *count, int32_t count_rows, int32_t n_neurons, int32_t n_samples,
                        const int32_t *ids, const int32_t *pop_ptr, int32_t n_pop, const float *targets,
                        float kappa, float rate_cost, int32_t shuffle, uint64_t seed, uint64_t offset,
                        float *loss_out, float *gz_neuron, void *ws, size_t ws_bytes, void *stream);

/* ------------------------------------------------------------- optimizer ------
 * Replaces ExponentiatedAdam.update_step, dense branch (v1_model_utils/optimizers.py:
 * 354-376; alpha :273-283), followed by the variable's SignedConstraint (models.py:419-427, attached
 * at :666, :729, :764), which Keras applies after the optimizer step.  One pass:
 *   m += (g - m)(1 - beta_1);  v += (g^2 - v)(1 - beta_2);  AMSGrad: vhat = max(vhat, v)
 *   w *= exp(-alpha * m / (sqrt(vhat or v) + epsilon) * sign(w)),  sign(0) = +1
 *   positive != NULL: w = positive ? relu(w) : -relu(-w)
 * alpha = learning_rate * sqrt(1 - beta_2^t) / (1 - beta_1^t) (t = iterations + 1) is
 * the caller's fp32 scalar.  device: w, m, v [n] f32 in/out, vhat [n] (NULL: no
 * AMSGrad), g [n] f32, positive [n] u8 (NULL: no constraint). */
int glif_exp_adam(float *w, float *m, float *v, float *vhat, const float *g, const uint8_t *positive,
                  int64_t n, float alpha, float beta_1, float beta_2, float epsilon, void *stream);

/* ------------------------------------------------------------ input sampling -
 * On-device replacements for the host input streams: LGN spikes (stim_dataset.py:182-197,
 * Bernoulli with p = 1 - exp(-rate * dt / 1000)) and background counts (models.py:865-887,
 * Poisson with lambda = rate * dt / 1000; TF's stateless stream cannot be reproduced).
 * Generator: Philox4x32-10; element i of the stream (seed) is word i % 4 of the block for
 * counter i / 4; `offset` continues a stream (element offset + i).  u = (word >> 8) * 2^-24.
 * Bernoulli: out[i] = u < p[i].  Poisson: sequential inverse CDF in fp32 from
 * exp_neg_lam = expf(-lam) (the caller's, so hosts and device agree bit for bit), counts
 * capped at 255.  device: p [n] f32, out [n] u8. */
int glif_sample_bernoulli(const float *p, int64_t n, uint64_t seed, uint64_t offset, uint8_t *out, void *stream);
int glif_sample_poisson(float lam, float exp_neg_lam, int64_t n, uint64_t seed, uint64_t offset, uint8_t *out,
                        void *stream);

/* ------------------------------------------------------------ profiling ------
 * No reference counterpart (the reference times whole steps with time(),
 * callbacks.py:1442-1449).  Kernel classes: 0 push, 1 step, 2 adj, 3 bwd_rec,
 * 4 bwd_lgn, 5 bwd_bkg, 6 syn_fwd, 7 syn_bwd, 8 lgn.  In the cell's event mode "step" is
 * the one launch per tick that runs the step beside that tick's pushes and "push" only the
 * push of tick 0; in deterministic mode "push" is the row pull where it runs as a launch
 * of its own.  "lgn" is the pass that computes 64 ticks of LGN currents ahead of the loop
 * (batch sizes up to 8).  "adj" includes the
 * previous window's weight-gradient passes and the rest of its dz walk, which share its launch.
 * While bit k of `mask` is set, every launch of class k (every `every`-th, glif_prof_stride,
 * counted from glif_prof_enable; default 1) is bracketed by two HIP events on its stream.
 * glif_prof_collect waits for the recorded events and returns, per class, the
 * summed elapsed milliseconds and the number of bracketed launches since the last collect. */
int glif_prof_enable(uint32_t mask);
int glif_prof_stride(int32_t every);
int glif_prof_collect(double *total_ms, int64_t *count, int32_t n);
const char *glif_prof_name(int32_t kind);

#ifdef __cplusplus
}
#endif
#endif /* GLIF_H */
