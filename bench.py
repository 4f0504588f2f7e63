#!/usr/bin/env python
"""Benchmark of the GLIF_3 V1 cell hot path on one MI355X.

One step = one training pass of the config-2 workload: forward rollout of the
66k-neuron network over T=500 ms at batch 5 (event-driven synaptic currents + fused
GLIF_3 step), the firing-rate MSE loss, BPTT through all 500 steps giving the
recurrent and LGN weight gradients, and the ExponentiatedAdam update with the sign
constraints of both weight vectors.  Inputs (LGN spikes, background Poisson counts)
are resident in HBM before timing.  Prints one JSON line.

The dominant kernel's roofline is measured live: its launches are bracketed by
HIP events on the stream they run on (libglif's per-kernel timer), and its
algorithmic bytes per launch are computed from the table sizes and the measured
activity.  `traffic` comes from rocprofv3 FETCH_SIZE / WRITE_SIZE runs committed
under profiles/ (null when absent).  The CPU baseline times the C restatement of
the reference (oracle/) on a bounded prefix of the same workload.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0
METRIC = "neuron-timesteps/s fwd+bwd (66k neurons, B=5, T=500) + achieved HBM GB/s %"


def _args():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2,
                    help="benchmark configuration: 2 fwd+BPTT (default), 1 or 3 forward, 4 the firing-rate "
                         "sweep of the event push against the deterministic row pull (B=32)")
    ap.add_argument("--rates", default="1,5,20,50", help="config 4: target mean rates in Hz")
    ap.add_argument("--mode", default="event", choices=["event", "deterministic"])
    ap.add_argument("--loss", default="mse", choices=["mse", "reference"],
                    help="mse: the configuration's firing-rate MSE against lognormal(4 Hz) targets; "
                         "reference: the reference's rate-distribution target + voltage regularization")
    ap.add_argument("--seq-len", type=int, default=None)
    ap.add_argument("--cpu-steps", type=int, default=None,
                    help="timesteps of the CPU baseline sample, timed with one thread and with the "
                         "host's cores (0: skip; default 30, config 0 its whole 50 ms)")
    ap.add_argument("--cpu-start", type=int, default=None,
                    help="first tick of the CPU baseline sample (the state there comes from the GPU's "
                         "deterministic rollout; configs 1-3 are silent for their first ~50-70 ms: default "
                         "200, config 0 from tick 0)")
    ap.add_argument("--forward-only", action="store_true")
    ap.add_argument("--syn-types", type=int, default=None,
                    help="synapse types of the generated network (the configurations use 5; the "
                         "reference's basis table has 121)")
    ap.add_argument("--n-basis", type=int, default=None, help="receptors (basis functions) per neuron")
    ap.add_argument("--target-rate", type=float, default=None, metavar="HZ",
                    help="scale all three weight populations by one factor, found by bisection on "
                         "deterministic rollouts, so the network fires at this mean rate (e.g. 5 for "
                         "the many-type network, whose weights are not calibrated)")
    ap.add_argument("--dense-basis", action="store_true",
                    help="a dense random basis table instead of the identity (every type feeds every "
                         "receptor, as in the reference's table)")
    ap.add_argument("--expand-receptors", action="store_true",
                    help="receptor-space form of a many-type network: every synapse becomes n_basis synapses "
                         "(one per receptor r, weight w * basis[syn_id][r]) over an identity basis, so the "
                         "backward's projection G holds dy itself (n_basis rows per neuron) instead of one "
                         "row per synapse type; same currents, more synapses")
    ap.add_argument("--class-types", type=int, default=None, metavar="K",
                    help="synapse types by (presynaptic class, postsynaptic class) over K neuron classes "
                         "(K*K types, dense random basis, inputs of class 0), the structure of the "
                         "reference's 121-type table: each neuron receives at most K of the types")
    ap.add_argument("--g-layout", default="auto", choices=["auto", "type-major"],
                    help="rows of the backward's per-type projection G: auto (compact rows, one per type "
                         "reaching the neuron, when no neuron receives more than 3/4 of the types) or "
                         "type-major (a row per type and neuron)")
    ap.add_argument("--op", action="store_true",
                    help="time the op-level entry points instead (calculate_synaptic_currents forward in "
                         "both modes and its custom gradient) on a config-2 table (--op-table, default "
                         "the recurrent one with z_buf spikes at 5 Hz), B = --op-batch")
    ap.add_argument("--op-table", default="rec", choices=["rec", "lgn", "bkg"],
                    help="with --op: the config-2 table the op runs on: rec (z_buf spikes at 5 Hz), lgn "
                         "(one tick of the config's LGN spikes) or bkg (one tick of its Poisson "
                         "background counts, counts mode)")
    ap.add_argument("--op-batch", type=int, default=5, help="with --op: the batch size (1-32)")
    ap.add_argument("--step-loop", action="store_true",
                    help="time the Keras-RNN form of the config-2 training step instead: a loop of T "
                         "V1Column.call steps differentiated by autograd step by step (glif_step_backward "
                         "per step), rate MSE loss, against the fused rollout + BPTT of the default run")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (5 times): the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE for streaming kernels")
    ap.add_argument("--gather-calibration", type=int, default=0, metavar="MIB",
                    help="only run 16M random 64-byte row gathers (torch index_select, 5 times) from a "
                         "MIB MiB table: a known-size gather kernel for rocprofv3's read counters (its "
                         "requests mix 128- and 64-byte reads, unlike the copy's 128-byte ones)")
    args = ap.parse_args()
    if args.cpu_steps is None:
        args.cpu_steps = 50 if args.config == 0 else 30
    if args.cpu_start is None:
        args.cpu_start = 0 if args.config == 0 else 200
    return args


def copy_calibration(mib):
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read_per_launch": n * 4, "copy_bytes_written_per_launch": n * 4,
                      "launches": 5}))


def gather_calibration(mib, n_gathers=1 << 24):
    """index_select of n_gathers random rows of 16 float32 (64 bytes) from a [rows, 16] table of
    mib MiB: per launch it reads n_gathers * 64 bytes at random rows plus the int64 indices
    (8 bytes each, streamed) and writes n_gathers * 64 bytes (streamed)."""
    import torch
    rows = mib * (1 << 20) // 64
    src = torch.ones((rows, 16), dtype=torch.float32, device="cuda")
    idx = torch.randint(0, rows, (n_gathers,), dtype=torch.int64, device="cuda")
    out = torch.empty((n_gathers, 16), dtype=torch.float32, device="cuda")
    for _ in range(5):
        torch.index_select(src, 0, idx, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"gather_rows_per_launch": n_gathers, "row_bytes": 64, "table_bytes": rows * 64,
                      "bytes_read_per_launch": n_gathers * (64 + 8), "bytes_written_per_launch": n_gathers * 64,
                      "launches": 5}))


def event_counts(tables, lgn, bkg, spike_count_total):
    """Synaptic events of one rollout: rec spikes x fan-out, LGN / bkg active x fan-out."""
    import numpy as np
    N = tables.n_neurons
    rec_fan = np.bincount(tables.rec.col % N, minlength=N).astype(np.float64)
    lgn_fan = np.bincount(tables.lgn.col, minlength=tables.lgn.n_cols).astype(np.float64)
    bkg_fan = np.bincount(tables.bkg.col, minlength=tables.bkg.n_cols).astype(np.float64)
    e_rec = float(spike_count_total.astype(np.float64).sum(0) @ rec_fan)
    e_lgn = float((lgn > 0).sum((0, 1)).astype(np.float64) @ lgn_fan)
    e_bkg = float((bkg > 0).sum((0, 1)).astype(np.float64) @ bkg_fan)
    return e_rec, e_lgn, e_bkg


def load_traffic(name):
    path = os.path.join(HERE, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


class RateCalibrator:
    """One factor on a cell's weight populations, set by bisection in log space on deterministic
    rollouts so that the mean firing rate meets a target (the configurations fix the network's
    shape, not its rate; the factor is reported).  populations ("rec",) scales the recurrent
    weights only, the role of the reference's recurrent_weight_scale (models.py:664), the LGN
    and background weights staying as generated; ("rec", "lgn", "bkg") scales all three."""

    def __init__(self, cell, lgn, bkg, populations=("rec", "lgn", "bkg")):
        import torch
        self.cell, self.lgn, self.bkg = cell, lgn, bkg
        every = {"rec": cell.recurrent_weight_values, "lgn": cell.input_weight_values,
                 "bkg": cell.bkg_input_weights}
        self.populations = tuple(populations)
        self.ws = tuple(every[k] for k in self.populations)
        self.base = [w.detach().clone() for w in self.ws]
        B, N = lgn.shape[1], cell.tables.n_neurons
        self.sc = torch.zeros((B, N), dtype=torch.int32, device=cell.device)
        self.floor_hz = None   # recurrent-only: the rate with the recurrent weights at zero

    def set_scale(self, f):
        import torch
        with torch.no_grad():
            for w, b0 in zip(self.ws, self.base):
                w.copy_(b0 * f)
        self.cell.refresh_weights(force=True)

    def rate_hz(self, f, Tp):
        import torch
        self.set_scale(f)
        self.sc.zero_()
        self.cell.rollout(self.lgn[:Tp], self.bkg[:Tp], record_z=False, record_v=False, spike_count=self.sc,
                          mode="deterministic")
        torch.cuda.synchronize()
        return float(self.sc.sum().item()) / self.sc.numel() / Tp * 1000.0

    def find_scale(self, target, Tp):   # the whole rollout: the rate ramps up from rest
        """The factor that meets `target` Hz; with the recurrent weights alone, 0.0 when the
        inputs by themselves already drive the network at or above it (the lowest reachable
        rate is then floor_hz)."""
        import numpy as np
        if self.populations == ("rec",):
            if self.floor_hz is None:
                self.floor_hz = self.rate_hz(0.0, Tp)
            if self.floor_hz >= target:
                return 0.0
        lo, hi = None, None
        f = 1.0
        r = self.rate_hz(f, Tp)
        for _ in range(12):   # bracket
            if r < target:
                lo = (f, r)
                if hi is not None:
                    break
                f *= 2.0
            else:
                hi = (f, r)
                if lo is not None:
                    break
                f *= 0.5
            r = self.rate_hz(f, Tp)
        if lo is None or hi is None:
            return f
        for _ in range(9):   # bisect in log space
            f = float(np.sqrt(lo[0] * hi[0]))
            r = self.rate_hz(f, Tp)
            if r < target:
                lo = (f, r)
            else:
                hi = (f, r)
        return float(np.sqrt(lo[0] * hi[0]))


def sweep_rates(args):
    """Config 4: forward throughput of the event push and the deterministic row pull at
    several mean firing rates.  One factor scales the recurrent weights only (the role of
    the reference's recurrent_weight_scale, models.py:664; the LGN and background weights stay
    as generated); it is set per target rate by bisection in log space on whole rollouts (the
    achieved rate of the timed rollout is reported)."""
    import numpy as np
    import torch
    from v1_glif_model_amd import _lib
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.models import V1Column

    cfg = sy.config(4)
    T = args.seq_len or cfg.seq_len
    B = cfg.batch
    net = sy.make_network(cfg, seed=0)
    lgn_np, bkg_np = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode="event", gauss_std=0.5, dampening_factor=0.5, pseudo_gauss=True)
    tb = cell.tables
    N, S = tb.n_neurons, tb.rec.n_syn
    dev = cell.device
    lgn = torch.tensor(lgn_np, device=dev)
    bkg = torch.tensor(bkg_np, device=dev)
    cal = RateCalibrator(cell, lgn, bkg, populations=("rec",))
    sc = cal.sc
    set_scale = cal.set_scale

    def find_scale(target, Tp=T):
        return cal.find_scale(target, Tp)

    def timed(mode, reps=2):
        ws = cell.workspace(B, T)
        out = []
        for i in range(reps + 1):
            st = cell.zero_state(B)
            sc.zero_()
            _lib.prof_enable(list(_lib.PROF_KINDS) if i == reps else [])
            _lib.prof_collect()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            cell.rollout(lgn, bkg, state=st, record_z=False, record_v=False, spike_count=sc, mode=mode, ws=ws)
            torch.cuda.synchronize()
            if i > 0:
                out.append((time.perf_counter() - t0) * 1000.0 / T)
        prof = _lib.prof_collect()
        _lib.prof_enable([])
        rate = float(sc.sum().item()) / (B * N * T) * 1000.0
        return min(out), rate, {k: round(v[0] / T * 1000.0, 2) for k, v in prof.items()}

    rows = []
    for target in [float(x) for x in args.rates.split(",") if x]:
        f = find_scale(target)
        set_scale(f)
        ev_ms, ev_rate, ev_k = timed("event")
        pl_ms, pl_rate, pl_k = timed("deterministic")
        events = ev_rate / 1000.0 * B * S   # recurrent synaptic events per step
        rows.append({"target_hz": target, "recurrent_weight_factor": round(f, 5), "rate_hz": round(ev_rate, 3),
                     "reachable": f > 0.0 or (cal.floor_hz or 0.0) <= target,
                     "event_ms_per_step": round(ev_ms, 4), "pull_ms_per_step": round(pl_ms, 4),
                     "event_kernel_us_per_step": ev_k, "pull_kernel_us_per_step": pl_k,
                     "rec_events_per_step": round(events),
                     # push bytes: 8-byte entry + one 4-byte atomic per event, over the whole
                     # event forward's kernel time (the pushes run inside the step launch);
                     # pull: every post-row entry (4 bytes) + the active entries' weight and
                     # type (5), over the pull kernel's time
                     "event_push_GBps": round(events * 12 / (sum(ev_k.values()) * 1e-6) / 1e9, 1),
                     "pull_GBps": round((S * 4 + events * 5) / (pl_k.get("push", 1e9) * 1e-6) / 1e9, 1)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    best5 = min((r for r in rows), key=lambda r: abs(r["target_hz"] - 5.0)) if rows else None
    value = B * N / (min(best5["event_ms_per_step"], best5["pull_ms_per_step"]) / 1000.0) if best5 else 0.0
    print(json.dumps({
        "metric": "forward neuron-timesteps/s (66k neurons, B=32, T=500) at the ~5 Hz point; sweep over rates",
        "value": round(value, 1), "unit": "neuron-timesteps/s", "n_gpus": 1, "steps": 2, "warmup": 1,
        "ms_per_step": min(best5["event_ms_per_step"], best5["pull_ms_per_step"]) if best5 else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"config 4: {N} GLIF_3 neurons, {S} recurrent synapses, B={B}, T={T}, "
                               "modulated LGN, forward; recurrent weights scaled to each rate; event push vs "
                               "deterministic row pull",
                   "neurons": N, "recurrent_synapses": S, "batch": B, "seq_len": T,
                   "rate_with_recurrent_weights_at_zero_hz": round(cal.floor_hz, 3) if cal.floor_hz is not None
                   else None},
        "sweep": rows}))


def bench_step_loop(args):
    """The config-2 training step's forward and backward in the Keras RNN's form (models.py:1317-1322
    with the tape of multi_training.py:368-372): T calls of V1Column.call, each an autograd node
    whose backward is glif_step_backward, the rate MSE of the loop's spikes, loss.backward().
    Same network, inputs, batch and loss targets as the default run; no optimizer step."""
    import numpy as np
    import torch
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.models import V1Column
    cfg = sy.config(2)
    T = args.seq_len or cfg.seq_len
    B = cfg.batch
    net = sy.make_network(cfg, seed=0)
    lgn_np, bkg_np = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode=args.mode, gauss_std=0.5, dampening_factor=0.5, train_recurrent_per_type=False,
                    recurrent_dampening_factor=0.5, voltage_gradient_dampening=0.5, pseudo_gauss=True,
                    train_input=True)
    dev = cell.device
    lgn = torch.tensor(lgn_np, dtype=torch.float32, device=dev)
    bkg = torch.tensor(bkg_np, device=dev)
    targets = torch.tensor(sy.make_rate_targets(cfg.n_neurons, seed=2), dtype=torch.float32, device=dev)
    w_rec, w_lgn = cell.recurrent_weight_values, cell.input_weight_values
    w_rec.requires_grad_(True)
    w_lgn.requires_grad_(True)

    def step():
        w_rec.grad = None
        w_lgn.grad = None
        state = cell.zero_state(B)
        zsum = torch.zeros((B, cfg.n_neurons), dtype=torch.float32, device=dev)
        for t in range(T):
            (z, _), state = cell.call(lgn[t], state, bkg_counts=bkg[t])
            zsum = zsum + z
        loss = ((zsum.mean(0) / T - targets) ** 2).mean()
        loss.backward()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000 / args.steps
    print(json.dumps({"metric": "Keras-RNN form: T calls + per-step autograd backward, ms per training step",
                      "value": round(ms, 2), "unit": "ms per step", "steps": args.steps, "warmup": args.warmup,
                      "higher_is_better": False, "dtype": "f32", "data": "synthetic",
                      "config": {"workload": f"config 2 network, B={B}, T={T}, rate MSE, mode {args.mode}, "
                                             "no optimizer step", "neurons": cfg.n_neurons, "batch": B,
                                 "seq_len": T},
                      "neuron_timesteps_per_s": round(B * cfg.n_neurons * T / (ms / 1000), 1)}), flush=True)


def bench_op(args):
    """Op-level timing (glif_syn_fwd / glif_syn_bwd, models.py:103-263) on a config-2 table:
    the recurrent one with z_buf [B][D*N] Bernoulli(0.005) spikes, or an input table with one
    tick of the config's LGN spikes / background counts (models.py:814-940); dy [B*N][nb]
    normal."""
    import numpy as np
    import torch
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.ops import SynapseTable
    from v1_glif_model_amd.tables import build_cell_tables
    if not 1 <= args.op_batch <= 32:
        raise SystemExit("--op-batch must be in [1, 32]")
    cfg = sy.config(2)
    if args.n_basis:
        cfg = dataclasses.replace(cfg, n_basis=args.n_basis)
    net = sy.make_network(cfg, seed=0)
    if args.class_types:
        net = sy.class_types(net, n_classes=args.class_types)
    tb = build_cell_tables(net)
    N, D, B, nb = tb.n_neurons, tb.max_delay, args.op_batch, tb.n_basis
    pop = {"rec": tb.rec, "lgn": tb.lgn, "bkg": tb.bkg}[args.op_table]
    counts = args.op_table == "bkg"
    t = SynapseTable(np.stack([pop.post, pop.col], -1), pop.syn_id, (N, pop.n_cols), tb.basis,
                     n_delay_slots=D if args.op_table == "rec" else 1)
    t.set_weights(torch.tensor(pop.weight, device="cuda"))
    rng = np.random.default_rng(3)
    if args.op_table == "rec":
        zc = (rng.uniform(size=(B, D * N)) < 0.005).astype(np.float32)
        inputs = "z_buf density 0.005"
    else:
        lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=1, batch=B)
        zc = (lgn if args.op_table == "lgn" else bkg)[0].astype(np.float32)
        inputs = ("one tick of the config's LGN spikes" if args.op_table == "lgn" else
                  "one tick of the config's Poisson background counts (counts mode)")
    z = torch.tensor(zc, device="cuda")
    dy = torch.tensor(rng.normal(0, 1, (B * N, nb)).astype(np.float32), device="cuda")
    events = int(sum(np.count_nonzero(zc[b][pop.col]) for b in range(B)))
    out = {}
    for name, fn in (("fwd_event", lambda: t.forward(z, counts=counts, mode="event")),
                     ("fwd_deterministic", lambda: t.forward(z, counts=counts, mode="deterministic")),
                     ("bwd", lambda: t.backward(z, dy, counts=counts))):
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1000.0 / args.steps
    S = pop.n_syn
    what = {"rec": f"config-2 recurrent table: {N} posts, {D} delay slots",
            "lgn": f"config-2 LGN table: {N} posts, {pop.n_cols} inputs",
            "bkg": f"config-2 background table: {N} posts, {pop.n_cols} inputs"}[args.op_table]
    print(json.dumps({
        "metric": "op-level synaptic-current forward / custom gradient, us per call",
        "value": round(out["fwd_event"] + out["bwd"], 2), "unit": "us per fwd+bwd call", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "higher_is_better": False, "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{what}, {S} synapses, B={B}, {inputs} ({events} synapse events per call)",
                   "table": args.op_table, "neurons": N, "synapses": S, "batch": B,
                   "syn_types": int(tb.basis.shape[0]), "receptors": int(nb)},
        "us_per_call": {k: round(v, 2) for k, v in out.items()},
        "synaptic_events_per_s": {"fwd_event": round(events / (out["fwd_event"] * 1e-6), 1),
                                  "fwd_deterministic": round(events / (out["fwd_deterministic"] * 1e-6), 1)},
        # the gradient touches every synapse for every batch entry: dz needs all of them
        "bwd_synapse_batch_products_per_s": round(S * B / (out["bwd"] * 1e-6), 1)}))


def main():
    args = _args()
    if args.op and args.gpus == 1:
        bench_op(args)
        return
    if args.step_loop and args.gpus == 1:
        bench_step_loop(args)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gather_calibration:
        gather_calibration(args.gather_calibration)
        return
    if args.config == 4 and args.gpus == 1:
        sweep_rates(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; multi-GPU data parallelism "
                                   "is designed but not built (--gpus must be 1)"}))
        sys.exit(2)
    import numpy as np
    import torch
    from v1_glif_model_amd import _lib
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.losses import (RateMSE, SpikeRateDistributionTarget, VoltageRegularization,
                                          population_neuron_ids)
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.optim import ExponentiatedAdam, SignedConstraint

    cfg = sy.config(args.config)
    if args.syn_types or args.n_basis:
        import dataclasses
        cfg = dataclasses.replace(cfg, n_syn_types=args.syn_types or cfg.n_syn_types,
                                  n_basis=args.n_basis or cfg.n_basis)
    if args.config in (0, 1, 3):
        args.forward_only = True   # forward workloads
    T = args.seq_len or cfg.seq_len
    B = cfg.batch
    t_gen = time.time()
    net = sy.make_network(cfg, seed=0, dense_basis=args.dense_basis)
    if args.class_types:
        net = sy.class_types(net, n_classes=args.class_types)
    if args.expand_receptors:
        net = sy.expand_receptors(net)
    lgn_np, bkg_np = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode=args.mode, gauss_std=0.5, dampening_factor=0.5, train_recurrent_per_type=False,
                    recurrent_dampening_factor=0.5, voltage_gradient_dampening=0.5,
                    pseudo_gauss=True, train_input=True)
    if args.g_layout == "type-major":
        cell.set_g_layout(False)
    t_gen = time.time() - t_gen
    dev = cell.device
    tb = cell.tables
    N, S = tb.n_neurons, tb.rec.n_syn
    lgn = torch.tensor(lgn_np, device=dev)
    bkg = torch.tensor(bkg_np, device=dev)
    weight_factor = None
    if args.target_rate:
        cal = RateCalibrator(cell, lgn, bkg)
        weight_factor = cal.find_scale(args.target_rate, T)
        cal.set_scale(weight_factor)
        print(json.dumps({"calibration": {"target_hz": args.target_rate, "weight_factor": round(weight_factor, 4)}}),
              file=sys.stderr, flush=True)
    ws = cell.workspace(B, T)
    spike_count = torch.zeros((B, N), dtype=torch.int32, device=dev)
    zero = cell.zero_state(B)
    state = [s.clone() for s in zero]
    want = ("rec", "lgn")
    # the reference's optimizer and weight constraints (multi_training.py:1042, 1046;
    # models.py:666, 729): ExponentiatedAdam, lr 0.005
    opt = ExponentiatedAdam(learning_rate=0.005)
    w_rec, w_lgn = cell.recurrent_weight_values, cell.input_weight_values
    cons = {w_rec.data_ptr(): SignedConstraint(cell.recurrent_weight_positive),
            w_lgn.data_ptr(): SignedConstraint(cell.input_weight_positive)}
    if args.loss == "mse":
        # the configuration's loss: mean-squared firing-rate error against per-neuron
        # lognormal(4 Hz) targets
        targets_np = sy.make_rate_targets(cfg.n_neurons, seed=2)
        rate_loss = RateMSE(targets_np, device=dev)
        volt_loss = None
    else:
        # the reference's training losses (multi_training.py:211-229, flags :1065-1078): the
        # rate-distribution target over the cell types (rate_cost 1e4) and the voltage
        # regularization ("threshold", voltage_cost 1), both fused with the cell
        pops = population_neuron_ids(sy.make_cell_types(N, net["network"]["n_exc"]))
        rate_loss = SpikeRateDistributionTarget(populations=pops, type_rates=sy.make_type_rates(),
                                                rate_cost=10000.0, cell=cell, device=dev)
        volt_loss = VoltageRegularization(cell, voltage_cost=1.0, penalty_mode="threshold")
    gz_neuron = torch.zeros(N, dtype=torch.float32, device=dev)
    fwd_ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    timings = []

    zero_each_step = [*state, spike_count]

    def step():
        # every batch starts from the zero state (one multi-tensor fill)
        torch._foreach_zero_(zero_each_step)
        # the weight copies of the tables the last update changed (the optimizer bumps its
        # variables' versions; the background weights are not trained here)
        cell.refresh_weights()
        fwd_ev[0].record()
        cell.rollout(lgn, bkg, state=state, record_z=False, record_v=False, spike_count=spike_count,
                     ws=ws)
        fwd_ev[1].record()
        if not args.forward_only:
            gz_neuron.zero_()
            if volt_loss is None:
                rate_loss(spike_count, T, gz_neuron=gz_neuron)
            else:
                rate_loss(spike_count=spike_count, T=T, gz_neuron=gz_neuron)
                volt_loss()
            g = cell.backward(gz_neuron=gz_neuron, want=want)
            opt.apply_gradients([(g["rec"], w_rec), (g["lgn"], w_lgn)], constraints=cons)
        fwd_ev[2].record()
        timings.append(fwd_ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    sc_host = spike_count.cpu().numpy()
    # one more, untimed step with every kernel class timed: the breakdown, and the dominant
    # class (most time per step), whose launches the timed steps bracket with HIP events.
    # Event mode's forward is one fused launch per tick (the step of t - 1 beside the pushes,
    # "step"), and so is deterministic mode's (the row pull of t beside the step of t, whose R
    # takes the currents of t - 1; "step"; where the pull and the step run as two launches the
    # row pull is "push"); "lgn" computes 64 ticks of LGN currents ahead of the loop (batch
    # sizes up to 8); "adj" is the adjoint launch with the
    # previous window's weight gradients and the rest of its dz walk; "bwd_rec" the dz walk
    # over the columns the next adjoint reads.
    _lib.prof_enable(list(_lib.PROF_KINDS))
    step()
    torch.cuda.synchronize()
    breakdown = {k: {"ms_per_step": round(v[0], 3), "launches": v[1]} for k, v in _lib.prof_collect().items()}
    _lib.prof_enable([])
    dominant = max(breakdown, key=lambda k: breakdown[k]["ms_per_step"])
    # a class launched once per tick is sampled (about 50 bracketed launches per step): two
    # event records per launch would cost more host time than the launches themselves
    # the stride is coprime with the class's launches per step, so that over the timed steps
    # every phase of the step is sampled alike (a stride dividing 500 would time the same ticks
    # every step, tick 0's first-launch work among them)
    per_step = breakdown[dominant]["launches"]
    stride = max(1, per_step // 50)
    while math.gcd(stride, per_step) != 1:
        stride += 1
    _lib.prof_stride(stride)
    _lib.prof_enable([dominant])
    _lib.prof_collect()
    fwd_ms = bwd_ms = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        torch.cuda.synchronize()
        fwd_ms += fwd_ev[0].elapsed_time(fwd_ev[1])
        bwd_ms += fwd_ev[1].elapsed_time(fwd_ev[2])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    prof = _lib.prof_collect()
    _lib.prof_enable([])
    _lib.prof_stride(1)

    ms_per_step = wall * 1000.0 / args.steps
    value = B * N * T / (ms_per_step / 1000.0)
    e_rec, e_lgn, e_bkg = event_counts(tb, lgn_np, bkg_np, sc_host)
    fwd_ms /= args.steps
    bwd_ms /= args.steps

    # roofline of the dominant kernel
    D, nb, nt = tb.max_delay, tb.n_basis, tb.basis.shape[0]
    Wwin = 3 if 3 * B <= 16 else 1
    Rg = 4
    while Rg < Wwin * B:
        Rg *= 2
    words = (N + 63) // 64
    # LGN currents computed ahead of the loop (the "lgn" class ran): the tick's launch then
    # pushes or pulls the recurrent events only, and in event mode the step leaves the
    # current slot to the next LGN pass instead of clearing it
    lgn_ahead = breakdown.get("lgn", {}).get("launches", 0) > 0
    e_in = 0.0 if lgn_ahead else e_lgn
    tot_ms, launches = prof.get(dominant, (0.0, 0))
    # the grouped dz walk (16-float G rows) with the weight gradients deferred splits each
    # window's walk: the columns of delays <= 2 Wwin - 3 (what the next window's adjoint reads,
    # rounded up to whole waves of 16 four-column groups) in its own launch, the rest in the
    # next adjoint's launch (libglif's glif_cell_backward)
    n_cols = D * N
    n_groups = (n_cols + 3) // 4
    split = Rg == 16 and not args.forward_only
    if split:
        g = (max(0, 2 * Wwin - 3) * N + 3) // 4
        cols_a = min(n_cols, min(n_groups, (g + 15) // 16 * 16) * 4)
    else:
        cols_a = n_cols
    s_a = int(np.count_nonzero(tb.rec.col < cols_a))
    # the window's dW passes run in the walk's launch when one G buffer is at most 32 MiB,
    # else in the next adjoint's launch (libglif's glif_cell_backward)
    g_rows = cell.g_layout()[0]
    dw_walk = split and N * g_rows * Rg * 4 <= (32 << 20)
    windows = max(T - 2, 1) / Wwin
    if dominant == "bwd_rec":
        # per launch = one backward window of Wwin timesteps (the last window may be
        # shorter)
        steps_per_launch = (T - 2) / max(breakdown[dominant]["launches"], 1)
        if split:
            # the first part of the grouped dz walk: one 8-byte table entry per synapse of
            # its columns, their pointers, the dz rows of the window's steps, G read once
            # + the window's recurrent and LGN dW behind it (per active synapse event: 4-byte
            # entry, the dW read and written, one G element)
            act_ev = (e_rec + e_lgn) / max(T, 1) * steps_per_launch if dw_walk else 0.0
            alg_bytes = (s_a * 8 + (cols_a + 1) * 4 + steps_per_launch * B * cols_a * 4 + N * nt * Rg * 4
                         + act_ev * 16)
            unit_desc = (f"bytes per backward window of {Wwin} timesteps (recurrent dz over the {cols_a} columns "
                         f"of delays <= {max(0, 2 * Wwin - 3)}" + (", and the window's dW)" if dw_walk else ")"))
        else:
            # dz and the dW of the window's active events in one pass
            active = e_rec / max(T, 1) * steps_per_launch
            alg_bytes = (S * 8 + (nt * D * N + 1) * 4 + steps_per_launch * B * D * N * 4 + N * nt * Rg * 4
                         + (steps_per_launch + D) * B * words * 8 + active * 8)
            unit_desc = f"bytes per backward window of {Wwin} timesteps (recurrent dz + dW)"
    elif dominant == "adj":
        # per launch = one backward window: the adjoint's state stream per (b, n) and tick
        # (D dz values, saved voltage, refractory bit; gV, gP, gR read and written once per
        # launch), its G rows written, and the rest of the previous window's dz walk (8-byte
        # entries of the other columns, their pointers and dz rows)
        # (+ with a large G the previous window's dW: per active synapse event 4-byte entry, the
        # dW read and written, one G element)
        act_ev = 0.0 if dw_walk else (e_rec + e_lgn) / max(T, 1) * Wwin
        alg_bytes = (Wwin * B * N * (D * 4 + 4) + Wwin * B * words * 8 + 2 * B * N * (1 + 2 * nb) * 4
                     + N * g_rows * Rg * 4 + act_ev * 16
                     + (S - s_a) * 8 + (n_cols - cols_a + 1) * 4 + Wwin * B * (n_cols - cols_a) * 4)
        unit_desc = (f"bytes per backward window of {Wwin} timesteps (adjoint + previous window's dz rest"
                     + (")" if dw_walk else " and dW)"))
    elif dominant == "step" and args.mode == "deterministic":
        # per launch = one tick: the row pull (every recurrent entry's bitmap index, and the
        # LGN ones when their currents are not computed ahead, 4 bytes; the row pointers; each
        # active entry's batch mask, weight and type, 9 bytes; the currents written) beside the
        # GLIF_3 step's state stream per (b, n) -- reads the previous tick's pulled I and its
        # LGN currents (I2 or the LGN ring's slot), R, P (nb floats each), A (2 floats), v, r
        # (int16); writes R, P, A, v, r and the saved voltage -- the per-neuron constants
        # (7 floats) and the background rows (8 bytes per synapse)
        active = (e_rec + e_in) / max(T, 1)
        tables = 1 if lgn_ahead else 2
        per_bn = (4 * nb * 4 + 14) + (2 * nb * 4 + 18)
        alg_bytes = ((S + (0 if lgn_ahead else tb.lgn.n_syn)) * 4 + tables * (N + 1) * 4 + active * 9
                     + tables * nb * B * N * 4 + B * N * per_bn + N * 28 + tb.bkg.n_syn * 8)
        unit_desc = "bytes per forward timestep (deterministic row pull beside the GLIF_3 step)"
    elif dominant == "step":
        # per launch = one tick: the GLIF_3 step's state stream per (b, n) -- reads I, R, P
        # (nb floats each), A (2 floats), v, r (int16); writes R, P, A, v, r, the saved voltage
        # and, without the LGN ring, I (cleared) -- the per-neuron constants (7 floats), the
        # background rows (8 bytes per synapse), and the tick's pushed events (8-byte entry +
        # one 4-byte atomic each; the LGN events too when their currents are not computed ahead)
        active = (e_rec + e_in) / max(T, 1)
        per_bn = (3 * nb * 4 + 14) + ((2 if lgn_ahead else 3) * nb * 4 + 18)
        alg_bytes = B * N * per_bn + N * 28 + tb.bkg.n_syn * 8 + active * 12
        unit_desc = "bytes per forward timestep (GLIF_3 step + the tick's pushed events)"
    elif dominant == "lgn":
        # per launch = 64 ticks of LGN currents: every LGN entry (input, weight, type: 9
        # bytes), the row pointers, the segment's tick masks per (input, batch entry), 8 bytes,
        # and the 64 current slots written ([nb][B][N] floats each)
        alg_bytes = (tb.lgn.n_syn * 9 + (N + 1) * 4 + tb.lgn.n_cols * B * 8 + 64 * nb * B * N * 4)
        unit_desc = "bytes per 64-tick segment of LGN currents"
    else:
        # per launch = one timestep's row pull: every recurrent entry's bitmap index, and the
        # LGN ones when their currents are not computed ahead (4 bytes), the row pointers, each
        # active entry's batch mask, weight and type (9 bytes), and the currents written
        active = (e_rec + e_in) / max(T, 1)
        tables = 1 if lgn_ahead else 2
        alg_bytes = ((S + (0 if lgn_ahead else tb.lgn.n_syn)) * 4 + tables * (N + 1) * 4 + active * 9
                     + tables * nb * B * N * 4)
        unit_desc = "bytes per forward timestep (deterministic row pull)"
    # the per-step algorithmic bytes of the path's operations, independent of how the kernels
    # batch them (the op's backward re-reads its table every step; the forward's push reads each
    # event's entry): per step, op backward (dz, + dW) 9 B per synapse (entry + syn_id), the
    # column pointers, dz written, dy read, 8 B per recurrent event (dW read-modify-write); the
    # GLIF_3 step (3 nb * 4 + 13 B read, 2 nb * 4 + 21 B written per (b, n), + 25 B of constants
    # per neuron); the adjoint (4 + 8 nb + 13 B read, 4 + 12 nb B written per (b, n)); the push
    # per source: per active column 12 B (column and row pointers), per event 9 B (post, weight,
    # type), the currents written once; the row pull 9 B per synapse, the packed spikes, the
    # currents written.  Times the steps one launch covers, over the launch's columns.
    e_step = e_rec / max(T, 1)
    a_step = float(sc_host.sum()) / max(T, 1) * D   # active (b, column) pairs per step, all delays
    k3 = B * N * ((3 * nb * 4 + 13) + (2 * nb * 4 + 21)) + 25 * N
    k4_cols = lambda syn, cols: syn * 9 + (cols + 1) * 4 + B * cols * 4
    k_bytes = None
    if dominant == "bwd_rec":
        steps_per_launch = (T - 2) / max(breakdown[dominant]["launches"], 1)
        k_bytes = steps_per_launch * (k4_cols(s_a, cols_a) + B * N * nb * 4 + e_step * 8)
        k_desc = (f"per-step op-backward bytes over the launch's {cols_a} columns (9 B per synapse, column "
                  f"pointers, dz written, dy read, 8 B per recurrent event) x {steps_per_launch:.2f} steps")
    elif dominant == "adj":
        k5 = B * N * ((4 + 2 * nb * 4 + 13) + (4 + 3 * nb * 4))
        k_bytes = Wwin * (k5 + k4_cols(S - s_a, n_cols - cols_a))
        k_desc = (f"per-step adjoint bytes (4 + 8 nb + 13 B read, 4 + 12 nb B written per (b, n)) + op-backward "
                  f"bytes over the other {n_cols - cols_a} columns, x {Wwin} steps")
    elif dominant == "step" and args.mode == "deterministic":
        k_bytes = k3 + S * 9 + B * D * N / 8 + B * N * nb * 4
        k_desc = "per-step bytes of the GLIF_3 step + the recurrent row pull (9 B per synapse, packed spikes)"
    elif dominant == "step":
        k_bytes = k3 + a_step * 12 + e_step * 9 + B * N * nb * 4
        k_desc = "per-step bytes of the GLIF_3 step + the recurrent push (12 B per active column, 9 B per event)"
    avg_ms = tot_ms / max(launches, 1)
    own_bytes, own_desc = alg_bytes, unit_desc
    if k_bytes is not None:
        alg_bytes, unit_desc = k_bytes, k_desc
    achieved = alg_bytes / (avg_ms / 1000.0) / 1e9 if avg_ms > 0 else 0.0
    own_achieved = own_bytes / (avg_ms / 1000.0) / 1e9 if avg_ms > 0 else 0.0
    # measured traffic per kernel class (deterministic mode's fused launch has its own)
    traffic = load_traffic("pull_step" if (dominant == "step" and args.mode == "deterministic") else dominant)
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic.get("bytes_per_launch") if traffic else None,
                "algorithmic_bytes_per_launch": int(alg_bytes), "basis": unit_desc,
                # the same launch on the bytes this build's kernels cannot avoid (the table read
                # once per backward window of several steps, G read once, ...)
                "own_algorithmic_bytes_per_launch": int(own_bytes), "own_basis": own_desc,
                "own_achieved": round(own_achieved, 1), "own_frac": round(own_achieved / HBM_PEAK_GBS, 4),
                "avg_launch_us": round(avg_ms * 1000.0, 2), "launches_timed": launches,
                "launch_sampling": f"every {stride} of the kernel's launches" if stride > 1 else "every launch"}
    if traffic and avg_ms > 0:
        # the measured L2 <-> memory-fabric bytes (FETCH_SIZE + WRITE_SIZE: HBM and
        # Infinity Cache) over the same live launch time
        tg = traffic["bytes_per_launch"] / (avg_ms / 1000.0) / 1e9
        roofline["traffic_gbs"] = round(tg, 1)
        roofline["traffic_frac"] = round(tg / HBM_PEAK_GBS, 4)

    # CPU baseline: the C restatement on a bounded window of the same workload, timed with one
    # thread and with the cores this process may use (its OpenMP loops keep every sum's order,
    # so both give the same bits).  The window starts at tick --cpu-start (past the network's
    # silent onset, so the recurrent events are those of the active regime) from the state the
    # deterministic GPU rollout reaches there (bit-exact with the oracle's own trajectory).
    cpu = cpu_1t = None
    if args.cpu_steps > 0:
        from oracle import cpu as orc_cpu
        from oracle.cpu import OracleCell
        t_a = min(max(args.cpu_start, 0), T - 1)
        Tc = min(args.cpu_steps, T - t_a)
        tb_cpu = tb
        if weight_factor:
            import dataclasses
            f32 = np.float32
            tb_cpu = dataclasses.replace(tb, **{k: dataclasses.replace(getattr(tb, k), weight=(
                getattr(tb, k).weight * f32(weight_factor)).astype(f32)) for k in ("rec", "lgn", "bkg")})
        oc = OracleCell(tb_cpu, vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)
        st_dev = [z.clone() for z in zero]
        if t_a > 0:
            cell.rollout(lgn[:t_a], bkg[:t_a], state=st_dev, record_z=False, record_v=False, mode="deterministic")
            torch.cuda.synchronize()
        st0 = dict(zbuf=st_dev[0].cpu().numpy(), v=st_dev[1].cpu().numpy(),
                   r=st_dev[2].cpu().numpy().astype(np.int32), asc=st_dev[3].cpu().numpy(),
                   psc_rise=st_dev[4].cpu().numpy(), psc=st_dev[5].cpu().numpy())
        lw, bw = lgn_np[t_a:t_a + Tc], bkg_np[t_a:t_a + Tc]

        def cpu_run(threads):
            used = orc_cpu.set_threads(threads)
            c0 = time.perf_counter()
            oz, ov, oref, _ = oc.forward(lw, bw, state=st0)
            if not args.forward_only:
                from oracle.rate_loss_ref import rate_dist_loss, rate_mse
                cnt = oz.reshape(Tc, B, N).sum((0, 1))
                gv = None
                if args.loss == "mse":
                    _, gzn = rate_mse(cnt, Tc * B, targets_np)
                else:
                    ids = np.concatenate([rate_loss.populations[k] for k in rate_loss.populations])
                    tgt = np.concatenate([rate_loss.target_rates[k]["sorted_target_rates"] for k in rate_loss.populations])
                    ptrs = np.concatenate([[0], np.cumsum([rate_loss.populations[k].size for k in rate_loss.populations])])
                    _, gzn = rate_dist_loss(cnt, Tc * B, ids, ptrs, tgt, rate_cost=10000.0, shuffle=True)
                    gv = (np.float32(2.0 / (Tc * B * N)) * (ov - np.float32(1.0))).astype(np.float32)
                oc.backward(lw, bw, oz, oref, ov, gz_neuron=gzn, gv_loss=gv, want=("rec", "lgn"), zbuf0=st0["zbuf"])
            return used, time.perf_counter() - c0, int(oz.sum())

        n1, s1, spk = cpu_run(1)
        what = (f"ticks {t_a}-{t_a + Tc - 1} of {T} of the same workload (B={B}, N={N}, {spk} spikes in the window), "
                f"{'forward only' if args.forward_only else 'forward + BPTT'}")
        cpu_1t = {"value": round(B * N * Tc / s1, 1), "unit": "neuron-timesteps/s", "cores": n1, "kind": "port",
                  "sample": f"oracle/glif_oracle.c single thread, {what}, {s1:.1f} s"}
        # every core this process may use (OMP_NUM_THREADS, where set, is the host's share for it)
        cores = len(os.sched_getaffinity(0))
        if os.environ.get("OMP_NUM_THREADS", "").isdigit():
            cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
        nt, st, _ = cpu_run(cores) if cores > 1 else (n1, s1, spk)
        cpu = {"value": round(B * N * Tc / st, 1), "unit": "neuron-timesteps/s", "cores": nt, "kind": "port",
               "sample": f"oracle/glif_oracle.c, {nt} OpenMP threads (batch entries and columns in parallel, "
                         f"same sums as one thread), {what}, {st:.1f} s"}
        orc_cpu.set_threads(1)

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "neuron-timesteps/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"config {args.config}: {N} GLIF_3 neurons, {S} recurrent synapses, "
                               f"B={B}, T={T}, {'forward' if args.forward_only else ('forward + firing-rate MSE' if args.loss == 'mse' else 'forward + rate-distribution and voltage losses') + ' + BPTT (rec + LGN dW) + ExponentiatedAdam update'}",
                   "neurons": N, "recurrent_synapses": S, "lgn_synapses": tb.lgn.n_syn,
                   "bkg_synapses": tb.bkg.n_syn, "batch": B, "seq_len": T, "mode": args.mode,
                   "syn_types": int(tb.basis.shape[0]), "receptors": int(tb.n_basis),
                   "basis": ("dense" if args.dense_basis or args.class_types else "identity")
                            + (f", types by {args.class_types} neuron classes" if args.class_types else "")
                            + (", receptor-expanded" if args.expand_receptors else ""),
                   "g_rows_per_neuron": cell.g_layout()[0],
                   "weight_factor": round(weight_factor, 4) if weight_factor else None,
                   "loss": None if args.forward_only else args.loss},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_1t": cpu_1t,
        "fwd_ms": round(fwd_ms, 3), "bwd_ms": round(bwd_ms, 3),
        "synaptic_events_per_s": round((e_rec + e_lgn + e_bkg) / (fwd_ms / 1000.0), 1) if fwd_ms else None,
        "mean_rate_hz": round(float(sc_host.mean()) / T * 1000.0, 3),
        "kernel_breakdown_ms": breakdown,
        "setup_s": round(t_gen, 1),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
