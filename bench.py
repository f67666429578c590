#!/usr/bin/env python3
"""Benchmark of the uncertain-gpt layer-kernel set on one MI355X.

Workload (benchmark config 5): one GPT-2-124M Bayesian step's layer-kernel path,
fp32, L=12 H=12 C=768 V=50257 B=8 T=1024, on the reference's buffer layout:
    bayes_materialize over n = 124,439,808 parameters (tied-head count)
    -> the layer kernels of gpt2_forward (encoder, 25 LayerNorm, 24 residual,
       12 GELU) -> the layer kernels of gpt2_backward (same, backward).
The dense ops between them (GEMMs, attention) are not part of the path; their
output buffers hold synthetic data. A "step" is that sequence, queued by the
native step driver of libugk.so (ugk_gpt2_layers_forward/backward), which runs
the encoder -> LayerNorm pair and each residual -> LayerNorm and LayerNorm ->
residual pair as one pass and adds
the LayerNorm weight/bias gradients of the whole backward in one launch; the
buffers it writes are bit-identical to the op-by-op sequence (a LayerNorm ->
residual pair does not write its LayerNorm's dinp back: in gpt2_backward only
the residual_backward it fuses reads that).

Printed JSON line (the last line of stdout):
    value        the reference sequence's algorithmic bytes (18.05 GB, unfused) / step
                 time: the effective rate of the reference's work; GBps_moved divides the
                 bytes the fused sequence must move (16.22 GB) instead
    ms_per_step  mean over --steps steps (events on the kernels' stream; median, p25, p75
                 of the per-step times beside it)
    zeroed_backward  the same step with ugk_gpt2_layers_backward_zeroed (for callers that
                 zero grads_acts before the backward, as every reference arm does; it does
                 not read those zeros): ms per step, rates on the reference's and moved bytes
    exact_forms  the same step with every exact mode on (GELU, encoder backward, LayerNorm: the
                 layer kernels' outputs bit-identical to train_bnn.c's), and the LayerNorm and
                 GELU kernels alone in their exact forms, cold, at the step's shapes
    in_step      each op of the step, timed inside the step with a HIP event pair that
                 its kernel's dispatch records (the library's op timer), over --op-steps
                 further steps: launches per step, mean us, us per step, algorithmic GB/s
    roofline     the op with the most microseconds per step (GELU backward or the fused
                 LayerNorm -> residual backward pairs, within a few percent of each other),
                 achieved = its algorithmic bytes per launch / its mean
                 in-step duration; traffic = HBM bytes per launch from rocprofv3 --pmc
                 FETCH_SIZE and WRITE_SIZE runs (profiles/pmc_traffic_cfg5.json)
    kernels      each kernel at its step shape, cold (launches rotate over buffer sets
                 totalling > 1.5 GiB, so neither L2 nor the 256 MB MALL holds the operands):
                 median of 5 batches of back-to-back launches (p25, p75), GB/s from
                 algorithmic bytes, fraction of 8 TB/s, and the stream ceiling of its mix
    configs      the same kernels at the shapes of benchmark configs 2-4 (LayerNorm at
                 16,384 x 768 and 256 x 384, GELU and residual at 50.3M, the encoder at
                 B=16 T=1024 with uniform and Zipf(1.1) tokens), cold
    head         softmax + cross-entropy forward and backward over B*T rows of V = 50257
    posterior    the ops around the step over the same n parameters, cold
    cpu_baseline the reference's own train_bnn.c ops (oracle/_ref, else this repo's
                 bit-identical restatement) on one pinned host core: median of 9 runs per
                 op at the config-5 step shapes (composed by launch count) and at configs
                 2-4, with nproc, the CPU model and the glibc version
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "uncertain-gpt_amd"))

METRIC = "achieved HBM GB/s (% of peak) per layer kernel fwd+bwd; layer-kernel ms/step"
PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(B, T, C, L, n_mat):
    """Algorithmic bytes: each fp32 input read once, each output written once, += = read+write."""
    BT, N = B * T, B * T * C
    per = {
        "encoder_forward": 12 * N + 4 * BT,
        "encoder_backward": 20 * N + 4 * BT,
        "layernorm_forward": 8 * N + 8 * BT + 8 * C,
        "layernorm_backward": 16 * N + 8 * BT + 20 * C,
        "gelu_forward": 8 * 4 * N,
        "gelu_backward": 16 * 4 * N,
        "residual_forward": 12 * N,
        "residual_backward": 20 * N,
        "bayes_materialize": 16 * n_mat,
    }
    count = {"encoder_forward": 1, "encoder_backward": 1, "layernorm_forward": 2 * L + 1,
             "layernorm_backward": 2 * L + 1, "gelu_forward": L, "gelu_backward": L,
             "residual_forward": 2 * L, "residual_backward": 2 * L, "bayes_materialize": 1}
    return per, count, sum(per[k] * count[k] for k in per)


KERNEL_KEYS = [  # (substring of the rocprof kernel name, short name)
    ("k_map_vec4<ugk::(anonymous namespace)::GeluBwdFast>", "gelu_backward"),
    ("k_map_vec4<ugk::(anonymous namespace)::GeluBwdFastZero>", "gelu_backward (dinp not read)"),
    ("k_map_vec4<ugk::(anonymous namespace)::GeluBwdZero>", "gelu_backward (exact form, dinp not read)"),
    ("k_map_vec4<ugk::(anonymous namespace)::GeluFwdFast>", "gelu_forward"),
    ("k_map_vec4<ugk::(anonymous namespace)::GeluBwd>", "gelu_backward (exact form)"),
    ("k_map_vec4<ugk::(anonymous namespace)::GeluFwd>", "gelu_forward (exact form)"),
    ("k_map_vec4<ugk::(anonymous namespace)::Materialize>", "bayes_materialize"),
    ("k_map_vec4<ugk::(anonymous namespace)::ResidualBwd>", "residual_backward"),
    ("k_map_vec4<ugk::(anonymous namespace)::ResidualFwd>", "residual_forward"),
    ("k_ln_bwd_vec", "layernorm_backward (main)"),
    ("k_ln_bwd_team", "layernorm_backward (main, row teams)"),
    ("k_ln_bwd_reduce_batch", "layernorm_backward (batched column sums)"),
    ("k_ln_bwd_reduce", "layernorm_backward (reduce)"),
    ("k_ln_fwd_exact", "layernorm_forward (exact form)"),
    ("k_ln_bwd_exact", "layernorm_backward (exact form: rows and columns in one launch)"),
    ("k_ln_fwd_vec", "layernorm_forward"),
    ("k_enc_fwd_vec", "encoder_forward"),
    ("k_enc_fwd_row", "encoder_forward"),
    ("k_enc_ln_fwd_vec", "encoder_layernorm_forward"),
    ("k_enc_bwd_insert", "encoder_backward (insert + dwpe)"),
    ("k_enc_bwd_add", "encoder_backward (add)"),
    ("k_enc_bwd_large", "encoder_backward (large buckets, exact order)"),
    ("k_enc_bwd_blocked", "encoder_backward (large buckets, blocked)"),
    ("k_ids_guard", "id guard"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesSampleEps<true>", "bayes_sample (eps stored)"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesSampleEps<false>", "bayes_sample (eps stored, glibc-exact)"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesSample<true>", "bayes_sample"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesSample<false>", "bayes_sample (glibc-exact)"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesBackwardPhilox<true>", "bayes_backward_philox"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesBackwardPhilox<false>", "bayes_backward_philox (glibc-exact)"),
    ("k_map_vec4<ugk::(anonymous namespace)::BayesBackward>", "bayes_backward"),
    ("k_map_vec4<ugk::(anonymous namespace)::KlBackward>", "kl_backward"),
    ("k_map_vec4<ugk::(anonymous namespace)::AdamW>", "adamw_update"),
    ("k_map_vec4<ugk::(anonymous namespace)::BbbStepFused<true>", "bbb_step_fused"),
    ("k_map_vec4<ugk::(anonymous namespace)::BbbStepFused<false>", "bbb_step_fused (glibc-exact)"),
    ("k_softmax_xent<", "softmax_crossentropy"),
    ("k_softmax_xent_split<", "softmax_crossentropy"),
    ("k_softmax_stats", "softmax_crossentropy (row statistics)"),
    ("k_softmax_norm_rows", "softmax_crossentropy (exact form, normalise)"),
    ("k_softmax_norm", "softmax_crossentropy (normalise)"),
    ("k_softmax_rowmax", "softmax_crossentropy (exact form, row max)"),
    ("k_softmax_sum_exact", "softmax_crossentropy (exact form, serial row sums)"),
    ("k_xent_softmax_bwd_flat4<true>", "crossentropy_softmax_backward (dlogits not read)"),
    ("k_xent_softmax_bwd<true>", "crossentropy_softmax_backward (dlogits not read)"),
    ("k_xent_softmax_bwd", "crossentropy_softmax_backward"),
    ("k_kl_partial<true>", "kl_forward (partial sums)"),
    ("k_kl_partial<false>", "kl_forward (partial sums, glibc-exact)"),
    ("k_kl_final", "kl_forward (final sum)"),
    ("__amd_rocclr_copyBuffer", "calibration copy 1 GiB"),
    ("k_stream<", "stream ceiling probe"),
]
PMC_TRAFFIC = os.path.join(ROOT, "profiles", "pmc_traffic_cfg5.json")
# in-step op name -> the prefix of its kernel's short name in the PMC summary
PMC_KEY = {"layernorm_residual_backward (main)":
           "layernorm_backward (main, row teams) <3, 4, 4, true, 3, true, 1, false, false>",
           "layernorm_backward (main)": "layernorm_backward (main, row teams) <3, 4, 2, false, 1, false, 0, false, false>",
           "residual_layernorm_forward": "layernorm_forward <3, true", "layernorm_forward": "layernorm_forward <3, false",
           "layernorm column sums (batched)": "layernorm_backward (batched column sums)"}


def short_name(name):
    for key, short in KERNEL_KEYS:
        if key in name:
            if (key.startswith("k_ln_") or key == "k_stream<") and "<" in name:  # one line per instantiation
                short += " " + name[name.index("<"):name.index(">") + 1]
            return short
    return None


def summarize_pmc(fetch_csv, write_csv):
    """Per-kernel HBM bytes per dispatch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE CSVs, each
    scaled so that the 1 GiB calibration copy reads and writes exactly 1 GiB."""
    import csv
    vals = {}
    for path, counter in ((fetch_csv, "FETCH_SIZE"), (write_csv, "WRITE_SIZE")):
        for r in csv.DictReader(open(path)):
            k = short_name(r["Kernel_Name"])
            if k and r["Counter_Name"] == counter:
                vals.setdefault(k, {}).setdefault(counter, []).append(float(r["Counter_Value"]) * 1024)
    # the blit kernel also serves small copies (e.g. a result read back); only the
    # 1 GiB copies calibrate, and they read well above 64 MiB on either counter
    cal = {c: [x for x in vals["calibration copy 1 GiB"][c] if x > 2 ** 26] for c in ("FETCH_SIZE", "WRITE_SIZE")}
    f_scale = 2 ** 30 / statistics.mean(cal["FETCH_SIZE"])
    w_scale = 2 ** 30 / statistics.mean(cal["WRITE_SIZE"])
    vals["calibration copy 1 GiB"] = cal
    out = {"fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "kernels": {}}
    for k, d in vals.items():
        fb = statistics.mean(d.get("FETCH_SIZE", [0])) * f_scale
        wb = statistics.mean(d.get("WRITE_SIZE", [0])) * w_scale
        out["kernels"][k] = {"read_bytes": round(fb), "write_bytes": round(wb), "traffic_bytes": round(fb + wb),
                             "dispatches": len(d.get("FETCH_SIZE", []))}
    return out


def summarize_stats(stats_csv):
    """Mean/min/max duration per kernel from rocprofv3 --stats (kernel_stats.csv), as text."""
    import csv
    lines = [f"{'kernel':34s} {'calls':>6s} {'mean us':>9s} {'min us':>9s} {'max us':>9s}"]
    for r in csv.DictReader(open(stats_csv)):
        k = short_name(r["Name"])
        if k:
            lines.append(f"{k:34s} {r['Calls']:>6s} {float(r['AverageNs']) / 1e3:9.2f} "
                         f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f}")
    return "\n".join(lines)


def summarize_trace(trace_csv):
    """Mean/min/max duration per kernel and grid size from a rocprofv3 --kernel-trace CSV, as
    text: the per-shape split of summarize_stats (one kernel serves several configurations)."""
    import csv
    groups = {}
    for r in csv.DictReader(open(trace_csv)):
        k = short_name(r["Kernel_Name"])
        if k:
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            groups.setdefault((k, int(r["Grid_Size_X"])), []).append(d)
    lines = [f"{'kernel':34s} {'grid':>10s} {'calls':>6s} {'mean us':>9s} {'min us':>9s} {'max us':>9s}"]
    for (k, grid), ds in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{k:34s} {grid:10d} {len(ds):6d} {statistics.mean(ds):9.2f} {min(ds):9.2f} {max(ds):9.2f}")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--reps", type=int, default=40,
                    help="cold launches per timed batch of a kernel (at least one per buffer set); 5 batches")
    ap.add_argument("--op-steps", type=int, default=10, help="steps timed op by op with the library's op timer")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true", help="skip the kernels at the other benchmark configurations' shapes")
    ap.add_argument("--no-head", action="store_true",
                    help="skip softmax + cross-entropy forward/backward at the GPT-2 head shape")
    ap.add_argument("--no-exact", action="store_true",
                    help="skip the exact forms (train_bnn.c's order of every addition, or its libm)")
    ap.add_argument("--no-posterior", action="store_true",
                    help="skip the posterior-update ops (Philox sample, bayes/KL backward, AdamW, fused step)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print per-kernel HBM traffic from two rocprofv3 --pmc runs of this script, and exit")
    ap.add_argument("--summarize-stats", metavar="STATS_CSV",
                    help="print per-kernel durations from a rocprofv3 --stats run of this script, and exit")
    ap.add_argument("--summarize-trace", metavar="TRACE_CSV",
                    help="print per-kernel, per-grid durations from a rocprofv3 --kernel-trace run of this "
                         "script, and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1, sort_keys=True))
        return
    if args.summarize_stats:
        print(summarize_stats(args.summarize_stats))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the layer kernels shard by rows with no exchange, so per-GPU throughput is the one-GPU figure",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ugk

    torch.cuda.set_device(0)
    dev = "cuda"
    B, T, C, V, NH, maxT, L = 8, 1024, 768, 50257, 12, 1024, 12
    cfg = ugk.Config(B=B, T=T, C=C, V=V, NH=NH, maxT=maxT, L=L)
    P = ugk.param_count(cfg)
    n_mat = P - (C * V + V)  # GPT-2-124M with the head tied to wte: 124,439,808
    A = ugk.act_count(cfg)
    per, count, total_bytes = step_bytes(B, T, C, L, n_mat)
    # the fused pairs of the driver skip 2L + 1 LayerNorm input reads (the first LayerNorm
    # normalises the encoder's rows as it writes them), 2L residual dout reads and the 2L
    # LayerNorm dinp writes that only the fused residual_backward would read
    moved_bytes = total_bytes - (3 * (2 * L) + 1) * 4 * (B * T * C)
    log(f"bench: params {P} (materialize {n_mat}), acts {A}, algorithmic bytes/step {total_bytes / 1e9:.3f} GB")

    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    mu = torch.randn(P, generator=g, device=dev) * 0.02
    rho = torch.randn(P, generator=g, device=dev) * 0.1 - 5.0
    eps = torch.randn(P, generator=g, device=dev)
    w = torch.empty(P, device=dev)
    acts = torch.randn(A, generator=g, device=dev)
    grads = torch.zeros(P, device=dev)
    grads_acts = torch.randn(A, generator=g, device=dev)
    inputs = torch.randint(0, V, (B * T,), generator=g, device=dev, dtype=torch.int32)
    flush = torch.empty(256 * 1024 * 1024, device=dev)  # 1 GiB, beyond L2 + MALL
    torch.cuda.synchronize()
    lib = ugk.lib
    ugk.set_stream(None)  # the null stream: torch's default stream too, so its events bracket our kernels

    def chk(rc):
        if rc != 0:
            raise ugk.UgkError(rc, lib.ugk_last_error().decode())

    wp, mup, rhop, epsp = w.data_ptr(), mu.data_ptr(), rho.data_ptr(), eps.data_ptr()
    ap_, gp, gap, ip = acts.data_ptr(), grads.data_ptr(), grads_acts.data_ptr(), inputs.data_ptr()

    def step():
        chk(lib.ugk_bayes_materialize(wp, mup, rhop, epsp, n_mat))
        chk(lib.ugk_gpt2_layers_forward(ap_, wp, ip, cfg, None))
        chk(lib.ugk_gpt2_layers_backward(gp, gap, ap_, wp, ip, cfg, None))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for k in range(args.steps):
        step()
        ev[k + 1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_step = ev[0].elapsed_time(ev[-1]) / args.steps
    per_step = sorted(ev[k].elapsed_time(ev[k + 1]) for k in range(args.steps))
    q = lambda xs, f: xs[min(len(xs) - 1, int(f * (len(xs) - 1) + 0.5))]
    step_stats = {"median": round(q(per_step, 0.5), 4), "p25": round(q(per_step, 0.25), 4),
                  "p75": round(q(per_step, 0.75), 4)}
    value = total_bytes / (ms_step * 1e-3) / 1e9
    moved_gbs = moved_bytes / (ms_step * 1e-3) / 1e9
    log(f"bench: step {ms_step:.4f} ms (median {step_stats['median']}, host wall {wall:.4f} ms) -> {value:.1f} GB/s "
        f"({100 * value / PEAK_GBS:.1f}% of peak) on the reference's {total_bytes / 1e9:.2f} GB, {moved_gbs:.1f} GB/s "
        f"({100 * moved_gbs / PEAK_GBS:.1f}%) on the {moved_bytes / 1e9:.2f} GB the fused sequence moves")

    # ---- the same step with ugk_gpt2_layers_backward_zeroed, the backward for callers that zero
    # grads_acts before it (every reference arm does): it does not read those zeros (GELU
    # backward's dinp, the residual splits' dx and dy, the final LayerNorm's dinp), and on this
    # layout it reads nothing of what those buffers hold, so the steps need no zeroing between them
    def step_zeroed():
        chk(lib.ugk_bayes_materialize(wp, mup, rhop, epsp, n_mat))
        chk(lib.ugk_gpt2_layers_forward(ap_, wp, ip, cfg, None))
        chk(lib.ugk_gpt2_layers_backward_zeroed(gp, gap, ap_, wp, ip, cfg, None))

    for _ in range(args.warmup):
        step_zeroed()
    torch.cuda.synchronize()
    z0, z1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    z0.record()
    for _ in range(args.steps):
        step_zeroed()
    z1.record()
    torch.cuda.synchronize()
    ms_zeroed = z0.elapsed_time(z1) / args.steps
    moved_zeroed = moved_bytes - (32 * L + 4) * (B * T * C)
    zeroed = {"ms_per_step": round(ms_zeroed, 4), "value_GBps": round(total_bytes / (ms_zeroed * 1e-3) / 1e9, 1),
              "bytes_per_step_moved": moved_zeroed,
              "GBps_moved": round(moved_zeroed / (ms_zeroed * 1e-3) / 1e9, 1),
              "frac_moved": round(moved_zeroed / (ms_zeroed * 1e-3) / 1e9 / PEAK_GBS, 4),
              "note": "ugk_gpt2_layers_backward_zeroed: the precondition of every reference arm (grads_acts "
                      "zeroed before the backward) lets it skip reading those zeros"}
    log(f"bench: step with the zeroed-gradient backward {ms_zeroed:.4f} ms -> {zeroed['value_GBps']:.1f} GB/s on the "
        f"reference's bytes, {zeroed['GBps_moved']:.1f} GB/s moved ({moved_zeroed / 1e9:.2f} GB)")

    # ---- the same step with every exact mode on (GELU's glibc tanhf, the encoder backward's and
    # LayerNorm's train_bnn.c orders): every buffer the layer kernels write is train_bnn.c's, bit for bit
    exact_forms = {}
    exact_setters = (ugk.set_gelu_exact, ugk.set_encoder_exact, ugk.set_layernorm_exact)
    if not args.no_exact:
        for f in exact_setters:
            f(True)
        try:
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
            x0, x1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            x0.record()
            for _ in range(args.steps):
                step()
            x1.record()
            torch.cuda.synchronize()
        finally:
            for f in exact_setters:
                f(False)
        ms_exact = x0.elapsed_time(x1) / args.steps
        exact_forms["step (every exact mode)"] = {
            "ms_per_step": round(ms_exact, 4), "GBps": round(total_bytes / (ms_exact * 1e-3) / 1e9, 1),
            "note": "ugk_set_gelu_exact, ugk_set_encoder_exact, ugk_set_layernorm_exact: the layer kernels' "
                    "outputs bit-identical to train_bnn.c's"}
        log(f"bench: step with every exact mode {ms_exact:.4f} ms -> "
            f"{exact_forms['step (every exact mode)']['GBps']:.1f} GB/s on the reference's bytes")

    # ---- each op inside the step: a HIP event pair recorded by the dispatch of
    # every kernel the step driver issues (ugk_op_timer_start/_read; the three-kernel
    # encoder backward is bracketed by two event records instead), over
    # --op-steps further steps; materialize is bracketed here by two records
    N = B * T * C
    op_bytes = {  # algorithmic bytes per launch at the step shape
        "encoder_forward": per["encoder_forward"], "layernorm_forward": per["layernorm_forward"],
        "encoder_layernorm_forward": 16 * N + 12 * B * T + 8 * C,
        "residual_layernorm_forward": 16 * N + 8 * B * T + 8 * C, "gelu_forward": per["gelu_forward"],
        "layernorm_backward (main)": 16 * N + 8 * B * T + 4 * C,
        "layernorm_residual_backward (main)": 28 * N + 8 * B * T + 4 * C,  # dinp read, not written
        "gelu_backward": per["gelu_backward"], "layernorm column sums (batched)": (2 * L + 1) * 16 * C,
        "encoder_backward": per["encoder_backward"], "bayes_materialize": per["bayes_materialize"]}
    m0, m1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    agg, mat_ms = {}, []
    for _ in range(args.op_steps):
        ugk.op_timer_start(1024)
        m0.record()
        chk(lib.ugk_bayes_materialize(wp, mup, rhop, epsp, n_mat))
        m1.record()
        chk(lib.ugk_gpt2_layers_forward(ap_, wp, ip, cfg, None))
        chk(lib.ugk_gpt2_layers_backward(gp, gap, ap_, wp, ip, cfg, None))
        for name, ms in ugk.op_timer_read(1024):
            agg.setdefault(name, []).append(ms)
        mat_ms.append(m0.elapsed_time(m1))
    agg["bayes_materialize"] = mat_ms
    in_step = {}
    for name, ms_list in agg.items():
        mean_ms = statistics.mean(ms_list)
        per_launch = op_bytes[name]
        gbs = per_launch / (mean_ms * 1e-3) / 1e9
        in_step[name] = {"launches_per_step": len(ms_list) / args.op_steps, "mean_us": round(mean_ms * 1e3, 2),
                         "us_per_step": round(sum(ms_list) * 1e3 / args.op_steps, 1), "bytes": per_launch,
                         "GBps": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
    for name, r in sorted(in_step.items(), key=lambda kv: -kv[1]["us_per_step"]):
        log(f"bench: in-step {name:38s} x{r['launches_per_step']:4.0f} {r['mean_us']:8.2f} us "
            f"{r['us_per_step']:8.1f} us/step {r['GBps']:8.1f} GB/s {100 * r['frac']:5.1f}%")

    # ---- each kernel alone at its step shape, cold ----------------------------
    # Each kernel cycles through k private buffer sets whose total exceeds
    # 1.5 GiB, so every launch finds its operands outside the L2 and the 256 MB
    # MALL; a batch of R*k back-to-back launches sits between two HIP events on
    # the stream the kernels run on; the launch time is the median over 5
    # batches of (t1 - t0) / (R*k).
    rnd = lambda n: torch.randn(n, generator=g, device=dev)

    def sets_for(make, set_bytes):
        k = max(2, -(-int(1.5 * 2 ** 30) // set_bytes))
        return [make() for _ in range(k)]

    def mk_enc():
        return {"out": torch.empty(N, device=dev), "wte": rnd(V * C) * 0.02, "wpe": rnd(maxT * C) * 0.01,
                "dout": rnd(N), "inp": torch.randint(0, V, (B * T,), generator=g, device=dev, dtype=torch.int32)}

    def mk_ln():
        d = {"x": rnd(N), "out": torch.empty(N, device=dev), "mean": torch.empty(B * T, device=dev),
             "rstd": torch.empty(B * T, device=dev), "w": torch.ones(C, device=dev), "b": torch.zeros(C, device=dev),
             "dout": rnd(N), "dinp": rnd(N), "dw": torch.zeros(C, device=dev), "db": torch.zeros(C, device=dev)}
        ugk.layernorm_forward(d["out"], d["mean"], d["rstd"], d["x"], d["w"], d["b"], B, T, C)
        return d

    def mk_enc_ln():
        d = mk_enc()
        d.update({"ln": torch.empty(N, device=dev), "mean": torch.empty(B * T, device=dev),
                  "rstd": torch.empty(B * T, device=dev), "w": torch.ones(C, device=dev),
                  "b": torch.zeros(C, device=dev)})
        return d

    def mk_ln_res():
        d = mk_ln()
        d["rx"], d["ry"] = rnd(N), rnd(N)
        return d

    def mk_gelu():
        return {"x": rnd(4 * N), "out": torch.empty(4 * N, device=dev), "dout": rnd(4 * N), "dinp": rnd(4 * N)}

    def mk_res():
        return {"x": rnd(N), "y": rnd(N), "out": torch.empty(N, device=dev), "dout": rnd(N)}

    def mk_mat():
        return {"mu": rnd(n_mat) * 0.02, "rho": rnd(n_mat) * 0.1 - 5.0, "eps": rnd(n_mat),
                "w": torch.empty(n_mat, device=dev)}

    P_ = lambda t: t.data_ptr()
    plan = {
        "encoder_forward": (mk_enc, 16 * N, lambda d: chk(lib.ugk_encoder_forward(
            P_(d["out"]), P_(d["inp"]), P_(d["wte"]), P_(d["wpe"]), B, T, C))),
        "encoder_backward": (mk_enc, 16 * N, lambda d: chk(lib.ugk_encoder_backward(
            P_(d["wte"]), P_(d["wpe"]), P_(d["dout"]), P_(d["inp"]), B, T, C))),
        "layernorm_forward": (mk_ln, 20 * N, lambda d: chk(lib.ugk_layernorm_forward(
            P_(d["out"]), P_(d["mean"]), P_(d["rstd"]), P_(d["x"]), P_(d["w"]), P_(d["b"]), B, T, C))),
        "layernorm_backward": (mk_ln, 20 * N, lambda d: chk(lib.ugk_layernorm_backward(
            P_(d["dinp"]), P_(d["dw"]), P_(d["db"]), P_(d["dout"]), P_(d["x"]), P_(d["w"]), P_(d["mean"]),
            P_(d["rstd"]), B, T, C))),
        "gelu_forward": (mk_gelu, 64 * N, lambda d: chk(lib.ugk_gelu_forward(P_(d["out"]), P_(d["x"]), 4 * N))),
        "gelu_backward": (mk_gelu, 64 * N, lambda d: chk(lib.ugk_gelu_backward(
            P_(d["dinp"]), P_(d["x"]), P_(d["dout"]), 4 * N))),
        "residual_forward": (mk_res, 16 * N, lambda d: chk(lib.ugk_residual_forward(
            P_(d["out"]), P_(d["x"]), P_(d["y"]), N))),
        "residual_backward": (mk_res, 16 * N, lambda d: chk(lib.ugk_residual_backward(
            P_(d["x"]), P_(d["y"]), P_(d["dout"]), N))),
        "bayes_materialize": (mk_mat, 16 * n_mat, lambda d: chk(lib.ugk_bayes_materialize(
            P_(d["w"]), P_(d["mu"]), P_(d["rho"]), P_(d["eps"]), n_mat))),
    }
    # the fused pairs the step driver runs (not separate entries of `per`: their
    # bytes are the pair's, 16, 16 and 32 per element, see step_bytes)
    fused_plan = {
        "encoder_layernorm_forward (fused pair)": (mk_enc_ln, 20 * N, 16 * N + 12 * B * T + 8 * C, lambda d: chk(
            lib.ugk_encoder_layernorm_forward(P_(d["out"]), P_(d["ln"]), P_(d["mean"]), P_(d["rstd"]),
                                              P_(d["inp"]), P_(d["wte"]), P_(d["wpe"]), P_(d["w"]), P_(d["b"]),
                                              B, T, C))),
        "residual_layernorm_forward (fused pair)": (mk_ln, 20 * N, 16 * N + 8 * B * T + 8 * C, lambda d: chk(
            lib.ugk_residual_layernorm_forward(P_(d["dinp"]), P_(d["out"]), P_(d["mean"]), P_(d["rstd"]),
                                               P_(d["x"]), P_(d["dout"]), P_(d["w"]), P_(d["b"]), B, T, C))),
        "layernorm_residual_backward (fused pair)": (mk_ln_res, 28 * N, 32 * N + 8 * B * T + 20 * C, lambda d: chk(
            lib.ugk_layernorm_residual_backward(P_(d["dinp"]), P_(d["dw"]), P_(d["db"]), P_(d["rx"]), P_(d["ry"]),
                                                P_(d["dout"]), P_(d["x"]), P_(d["w"]), P_(d["mean"]),
                                                P_(d["rstd"]), B, T, C))),
    }
    def time_cold(make, set_bytes, fn):
        """Mean time of one call, cycling over enough buffer sets (1.5 GB) that no input is
        cache resident (MI355X's 256 MB last-level cache would otherwise hold small ones)."""
        sets = sets_for(make, set_bytes)
        for d in sets:
            fn(d)
        torch.cuda.synchronize()
        rounds = max(1, args.reps // len(sets))
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        batches = []
        for _ in range(5):
            s.record()
            for _ in range(rounds):
                for d in sets:
                    fn(d)
            e.record()
            e.synchronize()
            batches.append(s.elapsed_time(e) / (rounds * len(sets)))
        batches.sort()
        n_sets = len(sets)
        del sets
        torch.cuda.empty_cache()
        time_cold.spread = (batches[1], batches[3])
        return batches[2], 5 * rounds * n_sets, n_sets

    def record(table, name, nbytes, ms, launches, n_sets, extra=None):
        gbs = nbytes / (ms * 1e-3) / 1e9
        p25, p75 = time_cold.spread
        table[name] = {"ms": round(ms, 5), "ms_p25": round(p25, 5), "ms_p75": round(p75, 5), "GBps": round(gbs, 1),
                       "frac": round(gbs / PEAK_GBS, 4), "bytes": nbytes, "launches_timed": launches,
                       "buffer_sets": n_sets, **(extra or {})}
        log(f"bench: {name:34s} {ms * 1e3:9.2f} us  {gbs:8.1f} GB/s  {100 * gbs / PEAK_GBS:5.1f}% of peak"
            f"  (median of 5 batches, p25-p75 {p25 * 1e3:.2f}-{p75 * 1e3:.2f} us; {launches} launches over "
            f"{n_sets} buffer sets)")

    # The encoder ops are also rated on the bytes they must move: the distinct wte rows the batch
    # gathers or scatters into (a repeated token's row comes from cache), wpe's T rows, dout or the
    # output once, the ids (enc_distinct_bytes). The forward lines take that as their basis (the
    # per-element count treats every repeat of a token as a fresh row), as the config-4 lines do;
    # the backward keeps the per-element count of the metric and gives the distinct basis beside it.
    probe_tok = mk_enc()["inp"]
    enc_distinct = int(torch.unique(probe_tok).numel())
    del probe_tok

    def enc_distinct_bytes(name, rows, Tn, distinct):
        Nn = rows * C
        if "encoder_backward" in name:  # dout once, RMW of the touched wte and wpe rows, ids
            return 4 * Nn + 8 * C * distinct + 8 * C * Tn + 4 * rows
        extra = 4 * Nn + 8 * rows + 8 * C if "encoder_layernorm" in name else 0
        return 4 * C * (distinct + Tn) + 4 * Nn + 4 * rows + extra

    def enc_record(table, name, abytes, ms, launches, n_sets, rows, Tn, distinct, extra):
        dbytes = enc_distinct_bytes(name, rows, Tn, distinct)
        dfrac = round(dbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)
        afrac = round(abytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)
        info = {"distinct_tokens": distinct, "bytes_algorithmic": abytes, "frac_algorithmic": afrac,
                "bytes_distinct": dbytes, "frac_distinct": dfrac, **extra}
        if "encoder_backward" in name:
            record(table, name, abytes, ms, launches, n_sets, info)
        else:
            record(table, name, dbytes, ms, launches, n_sets,
                   {**info, "bytes_basis": "distinct wte rows + wpe rows + out + ids"})
        log(f"bench: {'':34s} {100 * dfrac:5.1f}% of peak on the {dbytes / 1e6:.1f} MB it must move "
            f"({distinct} distinct tokens), {100 * afrac:5.1f}% on the per-element count")

    kernels, mean_ms = {}, {}
    for name, (make, set_bytes, fn) in plan.items():
        ms, launches, n_sets = time_cold(make, set_bytes, fn)
        mean_ms[name] = ms
        if name.startswith("encoder"):
            enc_record(kernels, name, per[name], ms, launches, n_sets, B * T, T, enc_distinct,
                       {"per_step": count[name]})
        else:
            record(kernels, name, per[name], ms, launches, n_sets, {"per_step": count[name]})
    for name, (make, set_bytes, nbytes, fn) in fused_plan.items():
        ms, launches, n_sets = time_cold(make, set_bytes, fn)
        extra = {"per_step": 1 if name.startswith("encoder") else 2 * L}
        if name.startswith("encoder"):
            enc_record(kernels, name, nbytes, ms, launches, n_sets, B * T, T, enc_distinct, extra)
        else:
            record(kernels, name, nbytes, ms, launches, n_sets, extra)
    # materialize over the reference's own untied layout at this shape (it stores
    # the head weight and bias, gpt2_kernels.cuh:681-683): all P parameters
    ms, launches, n_sets = time_cold(lambda: {"mu": rnd(P) * 0.02, "rho": rnd(P) * 0.1 - 5.0, "eps": rnd(P),
                                              "w": torch.empty(P, device=dev)}, 16 * P,
                                     lambda d: chk(lib.ugk_bayes_materialize(P_(d["w"]), P_(d["mu"]), P_(d["rho"]),
                                                                             P_(d["eps"]), P)))
    record(kernels, f"bayes_materialize (untied layout, n={P})", 16 * P, ms, launches, n_sets, {"per_step": 0})
    # the exact forms of the kernels that have one, cold at the same shapes (into exact_forms)
    if not args.no_exact:
        for names, setter in ((("layernorm_forward", "layernorm_backward"), ugk.set_layernorm_exact),
                              (("gelu_forward", "gelu_backward"), ugk.set_gelu_exact)):
            setter(True)
            try:
                for name in names:
                    make, set_bytes, fn = plan[name]
                    ms, launches, n_sets = time_cold(make, set_bytes, fn)
                    record(exact_forms, f"{name} (exact form)", per[name], ms, launches, n_sets)
            finally:
                setter(False)

    # ---- the practical HBM ceiling of each kernel's load/store mix: a pure
    # stream (ugk_diag_stream) with the same number of input and output
    # tensors of the same size, timed cold the same way
    pattern = {  # kernel: (tensors read, tensors written, floats per tensor)
        "encoder_forward": (2, 1, N), "encoder_backward": (3, 2, N),
        "layernorm_forward": (1, 1, N), "layernorm_backward": (3, 1, N),
        "gelu_forward": (1, 1, 4 * N), "gelu_backward": (3, 1, 4 * N),
        "residual_forward": (2, 1, N), "residual_backward": (3, 2, N),
        "bayes_materialize": (3, 1, n_mat),
        "residual_layernorm_forward (fused pair)": (2, 2, N),
        "encoder_layernorm_forward (fused pair)": (2, 2, N),
        "layernorm_residual_backward (fused pair)": (5, 3, N),
    }
    ceil_cache = {}
    for name, (nr, nw, n) in pattern.items():
        if (nr, nw, n) not in ceil_cache:
            best = 0.0
            for u, bs in ((1, 256), (2, 256), (3, 256), (1, 512), (2, 512)):  # the best of a few shapes
                ms, _, _ = time_cold(lambda: torch.empty((nr + nw) * n, device=dev), 4 * (nr + nw) * n,
                                     lambda b: chk(lib.ugk_diag_stream(P_(b), n, nr, nw, u, bs)))
                best = max(best, 4 * (nr + nw) * n / (ms * 1e-3) / 1e9)
            ceil_cache[(nr, nw, n)] = best
        ceil = ceil_cache[(nr, nw, n)]
        k = kernels[name]
        k["stream_ceiling_GBps"] = round(ceil, 1)
        k["frac_of_ceiling"] = round(k["GBps"] / ceil, 4)
        log(f"bench: ceiling {name:34s} {nr}R{nw}W stream {ceil:8.1f} GB/s ({100 * ceil / PEAK_GBS:4.1f}% of peak);"
            f" kernel at {100 * k['GBps'] / ceil:5.1f}% of it")
    # the step driver's LayerNorm -> residual backward pairs read five tensors and write two
    # (their dinp store is dead); their in-step rate against the cold stream of that mix
    best = 0.0
    for u, bs in ((1, 256), (2, 256), (3, 256), (1, 512), (2, 512)):
        ms, _, _ = time_cold(lambda: torch.empty(7 * N, device=dev), 28 * N,
                             lambda b: chk(lib.ugk_diag_stream(P_(b), N, 5, 2, u, bs)))
        best = max(best, 28 * N / (ms * 1e-3) / 1e9)
    pair = in_step["layernorm_residual_backward (main)"]
    pair["stream_ceiling_GBps"] = round(best, 1)
    pair["frac_of_ceiling"] = round(pair["GBps"] / best, 4)
    log(f"bench: ceiling in-step layernorm_residual_backward (main)  5R2W stream {best:8.1f} GB/s "
        f"({100 * best / PEAK_GBS:4.1f}% of peak); in-step op at {100 * pair['GBps'] / best:5.1f}% of it")

    # ---- the same kernels at the other benchmark configurations' shapes (not part of the step)
    configs = {}
    if not args.no_configs:
        import numpy as np
        B2, T2 = 16, 1024
        R2, N3 = B2 * T2, 16 * 1024 * 3072
        for rows_, C_ in ((R2, 768), (256, 384)):
            def mk_ln2(rows_=rows_, C_=C_):
                d = {"x": rnd(rows_ * C_), "out": torch.empty(rows_ * C_, device=dev),
                     "mean": torch.empty(rows_, device=dev), "rstd": torch.empty(rows_, device=dev),
                     "w": torch.ones(C_, device=dev), "b": torch.zeros(C_, device=dev), "dout": rnd(rows_ * C_),
                     "dinp": rnd(rows_ * C_), "dw": torch.zeros(C_, device=dev), "db": torch.zeros(C_, device=dev)}
                ugk.layernorm_forward(d["out"], d["mean"], d["rstd"], d["x"], d["w"], d["b"], 1, rows_, C_)
                return d
            tag = f"cfg2 {rows_}x{C_}"
            ms, l_, k_ = time_cold(mk_ln2, 20 * rows_ * C_, lambda d, rows_=rows_, C_=C_: chk(lib.ugk_layernorm_forward(
                P_(d["out"]), P_(d["mean"]), P_(d["rstd"]), P_(d["x"]), P_(d["w"]), P_(d["b"]), 1, rows_, C_)))
            record(configs, f"{tag} layernorm_forward", 8 * rows_ * C_ + 8 * rows_ + 8 * C_, ms, l_, k_)
            ms, l_, k_ = time_cold(mk_ln2, 20 * rows_ * C_, lambda d, rows_=rows_, C_=C_: chk(lib.ugk_layernorm_backward(
                P_(d["dinp"]), P_(d["dw"]), P_(d["db"]), P_(d["dout"]), P_(d["x"]), P_(d["w"]), P_(d["mean"]),
                P_(d["rstd"]), 1, rows_, C_)))
            record(configs, f"{tag} layernorm_backward", 16 * rows_ * C_ + 8 * rows_ + 20 * C_, ms, l_, k_)

        def mk_big():
            return {"x": rnd(N3), "y": rnd(N3), "out": torch.empty(N3, device=dev), "dout": rnd(N3)}
        for nm, nb, fn in (
                ("gelu_forward", 8, lambda d: chk(lib.ugk_gelu_forward(P_(d["out"]), P_(d["x"]), N3))),
                ("gelu_backward", 16, lambda d: chk(lib.ugk_gelu_backward(P_(d["y"]), P_(d["x"]), P_(d["dout"]), N3))),
                ("residual_forward", 12, lambda d: chk(lib.ugk_residual_forward(P_(d["out"]), P_(d["x"]), P_(d["y"]), N3))),
                ("residual_backward", 20, lambda d: chk(lib.ugk_residual_backward(P_(d["x"]), P_(d["y"]), P_(d["dout"]), N3)))):
            ms, l_, k_ = time_cold(mk_big, 16 * N3, fn)
            record(configs, f"cfg3 N={N3} {nm}", nb * N3, ms, l_, k_)

        wcdf = np.cumsum(1.0 / np.arange(1, V + 1, dtype=np.float64) ** 1.1)
        wcdf /= wcdf[-1]
        zrng = np.random.Generator(np.random.Philox(key=11))
        for law in ("uniform", "zipf1.1"):
            def mk_enc4(law=law):
                if law == "uniform":
                    tok = torch.randint(0, V, (R2,), generator=g, device=dev, dtype=torch.int32)
                else:
                    tok = torch.from_numpy(np.minimum(np.searchsorted(wcdf, zrng.random(R2)), V - 1)
                                           .astype(np.int32)).to(dev)
                return {"out": torch.empty(R2 * C, device=dev), "wte": rnd(V * C) * 0.02, "wpe": rnd(maxT * C) * 0.01,
                        "dout": rnd(R2 * C), "inp": tok}
            N4 = R2 * C
            # the distinct wte rows a call gathers (the repeats of a Zipf batch come from cache), wpe's T
            # rows, the output and the ids: the bytes that must cross HBM
            probe = mk_enc4()
            distinct = int(torch.unique(probe["inp"]).numel())
            del probe
            ms, l_, k_ = time_cold(mk_enc4, 16 * N4, lambda d: chk(lib.ugk_encoder_forward(
                P_(d["out"]), P_(d["inp"]), P_(d["wte"]), P_(d["wpe"]), B2, T2, C)))
            # bytes and frac on those distinct rows (a frequent token's repeats are cache hits, so
            # the per-element count would exceed the HBM peak); the per-element count beside them
            enc_record(configs, f"cfg4 {law} encoder_forward", 12 * N4 + 4 * R2, ms, l_, k_, R2, T2, distinct, {})
            ms, l_, k_ = time_cold(mk_enc4, 16 * N4, lambda d: chk(lib.ugk_encoder_backward(
                P_(d["wte"]), P_(d["wpe"]), P_(d["dout"]), P_(d["inp"]), B2, T2, C)))
            enc_record(configs, f"cfg4 {law} encoder_backward", 20 * N4 + 4 * R2, ms, l_, k_, R2, T2, distinct, {})

    # ---- the posterior update around the layer kernels, over the same n (not part of the step)
    posterior = {}
    if not args.no_posterior:
        n = n_mat
        seed, pstep = 0x5EED, 3
        bc1, bc2 = 1.0 - 0.9 ** pstep, 1.0 - 0.999 ** pstep

        def mk_post():
            return {k: rnd(n) * 0.01 for k in ("mu", "dw", "eps", "dmu", "drho", "m_mu", "m_rho")} | \
                   {"rho": rnd(n) * 0.1 - 5.0, "v_mu": rnd(n).abs_() * 1e-4, "v_rho": rnd(n).abs_() * 1e-4,
                    "w": torch.empty(n, device=dev)}
        post_plan = (
            ("bayes_sample", 12, lambda d: chk(lib.ugk_bayes_sample(
                P_(d["w"]), None, P_(d["mu"]), P_(d["rho"]), n, seed, pstep))),
            ("bayes_sample (eps stored)", 16, lambda d: chk(lib.ugk_bayes_sample(
                P_(d["w"]), P_(d["eps"]), P_(d["mu"]), P_(d["rho"]), n, seed, pstep))),
            ("bayes_backward", 28, lambda d: chk(lib.ugk_bayes_backward(
                P_(d["dmu"]), P_(d["drho"]), P_(d["dw"]), P_(d["eps"]), P_(d["rho"]), n))),
            ("bayes_backward_philox", 24, lambda d: chk(lib.ugk_bayes_backward_philox(
                P_(d["dmu"]), P_(d["drho"]), P_(d["dw"]), P_(d["rho"]), n, seed, pstep))),
            ("kl_backward", 24, lambda d: chk(lib.ugk_kl_backward(
                P_(d["dmu"]), P_(d["drho"]), P_(d["mu"]), P_(d["rho"]), n, 0.1, 1e-6))),
            ("adamw_update", 28, lambda d: chk(lib.ugk_adamw_update(
                P_(d["mu"]), P_(d["dw"]), P_(d["m_mu"]), P_(d["v_mu"]), n, pstep, 3e-4, 0.9, 0.999, 1e-8, 0.0))),
            ("bbb_step_fused", 60, lambda d: chk(lib.ugk_bbb_step_fused(
                P_(d["mu"]), P_(d["rho"]), P_(d["m_mu"]), P_(d["v_mu"]), P_(d["m_rho"]), P_(d["v_rho"]),
                P_(d["w"]), P_(d["dw"]), n, seed, pstep, 0.1, 1e-6, bc1, bc2, 3e-4, 0.9, 0.999, 1e-8, 0.0))),
        )
        for nm, nb, fn in post_plan:
            ms, l_, k_ = time_cold(mk_post, 44 * n, fn)
            record(posterior, nm, nb * n, ms, l_, k_)
        # the Philox ops in their glibc-exact form (ugk_set_philox_exact(1): glibc-exact softplus and
        # sigmoid, the device library's logf and a correctly rounded root in the Box-Muller radius),
        # beside the default hardware-transcendental form timed above
        ugk.set_philox_exact(True)
        try:
            for nm, nb, fn in post_plan:
                if nm in ("bayes_sample", "bayes_backward_philox", "bbb_step_fused"):
                    ms, l_, k_ = time_cold(mk_post, 44 * n, fn)
                    record(posterior, f"{nm} (glibc-exact form)", nb * n, ms, l_, k_)
        finally:
            ugk.set_philox_exact(False)
        kl_out = ctypes.c_double(0.0)
        kl_fn = lambda d: chk(lib.ugk_kl_forward(ctypes.byref(kl_out), P_(d["mu"]), P_(d["rho"]), n, 0.1))
        ms, l_, k_ = time_cold(mk_post, 44 * n, kl_fn)
        record(posterior, "kl_forward (incl. the result's wait)", 8 * n, ms, l_, k_)
        # its glibc-exact form (ugk_set_kl_exact(1)), beside the default one
        ugk.set_kl_exact(True)
        try:
            ms, l_, k_ = time_cold(mk_post, 44 * n, kl_fn)
            record(posterior, "kl_forward (incl. the result's wait, glibc-exact form)", 8 * n, ms, l_, k_)
        finally:
            ugk.set_kl_exact(False)

    # ---- softmax + cross-entropy at the head shape, B*T rows of V logits (not part of the step)
    head = {}
    if not args.no_head:
        rows_h = B * T
        NV = rows_h * V

        def mk_head():
            return {"logits": rnd(NV) * 3.0, "probs": torch.empty(NV, device=dev), "dlogits": torch.zeros(NV, device=dev),
                    "losses": torch.empty(rows_h, device=dev),
                    "targets": torch.randint(0, V, (rows_h,), generator=g, device=dev, dtype=torch.int32)}
        ms, l_, k_ = time_cold(mk_head, 12 * NV, lambda d: chk(lib.ugk_softmax_crossentropy(
            P_(d["losses"]), P_(d["probs"]), P_(d["logits"]), P_(d["targets"]), B, T, V)))
        record(head, "softmax_crossentropy", 8 * NV + 8 * rows_h, ms, l_, k_)
        ms, l_, k_ = time_cold(mk_head, 12 * NV, lambda d: chk(lib.ugk_crossentropy_softmax_backward(
            P_(d["dlogits"]), P_(d["probs"]), P_(d["targets"]), B, T, V)))
        record(head, "crossentropy_softmax_backward", 12 * NV + 4 * rows_h, ms, l_, k_)
        # the zeroed variant writes dlogits without reading it: 8 B per logit moved
        ms, l_, k_ = time_cold(mk_head, 12 * NV, lambda d: chk(lib.ugk_crossentropy_softmax_backward_zeroed(
            P_(d["dlogits"]), P_(d["probs"]), P_(d["targets"]), B, T, V)))
        record(head, "crossentropy_softmax_backward_zeroed", 8 * NV + 4 * rows_h, ms, l_, k_)
        # the forward in its exact form (ugk_set_softmax_exact(1): train_bnn.c's serial row sums)
        if not args.no_exact:
            ugk.set_softmax_exact(True)
            try:
                ms, l_, k_ = time_cold(mk_head, 12 * NV, lambda d: chk(lib.ugk_softmax_crossentropy(
                    P_(d["losses"]), P_(d["probs"]), P_(d["logits"]), P_(d["targets"]), B, T, V)))
                record(head, "softmax_crossentropy (exact form)", 8 * NV + 8 * rows_h, ms, l_, k_)
            finally:
                ugk.set_softmax_exact(False)

    # ---- roofline of the op with the most microseconds per step, from its in-step
    # launches (a HIP event pair around each, on the library stream)
    dom = max(in_step, key=lambda k: in_step[k]["us_per_step"])
    d = in_step[dom]
    achieved = d["bytes"] / (d["mean_us"] * 1e-6) / 1e9
    traffic, traffic_src = None, None
    if os.path.exists(PMC_TRAFFIC):  # recorded by two rocprofv3 --pmc runs of this script
        pmc = json.load(open(PMC_TRAFFIC)).get("kernels", {})
        want = PMC_KEY.get(dom, dom)  # an exact name, else the first one it begins
        key = want if want in pmc else next((k for k in pmc if k.startswith(want)), None)
        if key:
            traffic, traffic_src = pmc[key]["traffic_bytes"], f"{os.path.relpath(PMC_TRAFFIC, ROOT)}: {key}"
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "launch_ms": round(d["mean_us"] * 1e-3, 5), "bytes_per_launch": d["bytes"],
                "launches_per_step": d["launches_per_step"], "us_per_step": d["us_per_step"],
                "measured": f"in-step: a HIP event pair recorded by each of its dispatches (ugk op timer, "
                            f"hipExtLaunchKernelGGL), {args.op_steps} steps"}

    # a plain 1 GiB device-to-device copy (torch's copy kernel): the known-size
    # reference that scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings
    calib = torch.empty_like(flush)
    for _ in range(3):
        calib.copy_(flush)
    torch.cuda.synchronize()
    del calib

    cpu = None if args.no_cpu else cpu_baseline(B, T, C, V, L, n_mat, per, count, total_bytes, moved_bytes)

    rec = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "BASELINE config 5: GPT-2-124M Bayesian step, layer-kernel path "
                               "(materialize + encoder/LN/GELU/residual fwd+bwd)",
                   "L": L, "H": NH, "C": C, "V": V, "B": B, "T": T, "materialize_n": n_mat,
                   "param_layout_n": P, "parallelism": "single GPU"},
        "ms_per_step_stats": step_stats, "value_basis": "reference sequence's algorithmic bytes (unfused) / step time",
        "frac_of_peak": round(value / PEAK_GBS, 4), "bytes_per_step": total_bytes,
        "bytes_per_step_moved": moved_bytes, "GBps_moved": round(moved_bytes / (ms_step * 1e-3) / 1e9, 1),
        "frac_moved": round(moved_bytes / (ms_step * 1e-3) / 1e9 / PEAK_GBS, 4), "zeroed_backward": zeroed, "exact_forms": exact_forms,
        "in_step": in_step,
        "kernels": kernels, "configs": configs, "posterior": posterior, "head": head, "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


def host_facts():
    """nproc, the CPU model and the C library of the host the baseline runs on."""
    import platform
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = " ".join(platform.libc_ver())
    return {"nproc": os.cpu_count(), "cpus_allowed": len(os.sched_getaffinity(0)), "cpu_model": model,
            "libc": libc}


def cpu_baseline(B, T, C, V, L, n_mat, per, count, total_bytes, moved_bytes):
    """The reference's CPU ops (train_bnn.c, single-threaded) on one pinned core: the median of
    9 runs of each op at the config-5 step shapes, composed by launch count into a step, and at
    the shapes of configs 2-4 (GELU/residual over 50.3M values on a 1/8 slice, scaled;
    materialize on a 1/8 slice, scaled). About 10 s of CPU work in all."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, REF_SO
    kind = "reference" if os.path.exists(REF_SO) else "port"
    o = Oracle(reference=(kind == "reference"))
    facts = host_facts()
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[len(allowed) // 2]
    os.sched_setaffinity(0, {core})
    try:
        rng = np.random.Generator(np.random.Philox(key=7))
        f = lambda n: rng.standard_normal(n, dtype=np.float32)
        reps = 9
        t_sample = 0.0

        def med(fn, scale=1.0):
            nonlocal t_sample
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            t_sample += sum(ts)
            ts.sort()
            return ts[reps // 2] * scale, ts[reps // 4] * scale, ts[3 * reps // 4] * scale

        # config 5, the step's shapes
        N = B * T * C
        x, y, d = f(N), f(N), f(N)
        h, hd = f(4 * N), f(4 * N)
        wv, bv = np.ones(C, np.float32), np.zeros(C, np.float32)
        mean, rstd = np.zeros(B * T, np.float32), np.zeros(B * T, np.float32)
        out, out4 = np.zeros(N, np.float32), np.zeros(4 * N, np.float32)
        inp = rng.integers(0, V, B * T, dtype=np.int32)
        wte, wpe = f(V * C) * np.float32(0.02), f(T * C) * np.float32(0.01)
        dwte, dwpe = np.zeros(V * C, np.float32), np.zeros(T * C, np.float32)
        dwl, dbl = np.zeros(C, np.float32), np.zeros(C, np.float32)
        ns = n_mat // 8
        mu, rh, ep, wm = f(ns) * np.float32(0.02), f(ns) * np.float32(0.1) - np.float32(5), f(ns), np.zeros(ns, np.float32)
        ops = {
            "encoder_forward": (lambda: o.encoder_forward(out, inp, wte, wpe, B, T, C), 1),
            "encoder_backward": (lambda: o.encoder_backward(dwte, dwpe, d, inp, B, T, C), 1),
            "layernorm_forward": (lambda: o.layernorm_forward(out, mean, rstd, x, wv, bv, B, T, C), 1),
            "layernorm_backward": (lambda: o.layernorm_backward(y, dwl, dbl, d, x, wv, mean, rstd, B, T, C), 1),
            "gelu_forward": (lambda: o.gelu_forward(out4, h, 4 * N), 1),
            "gelu_backward": (lambda: o.gelu_backward(hd, h, out4, 4 * N), 1),
            "residual_forward": (lambda: o.residual_forward(out, x, y, N), 1),
            "residual_backward": (lambda: o.residual_backward(y, out, d, N), 1),
            "bayes_materialize": (lambda: o.bayes_materialize(wm, mu, rh, ep, ns), n_mat / ns),
        }
        t_op, spread = {}, {}
        for name, (fn, scale) in ops.items():
            t_op[name], lo, hi = med(fn, scale)
            spread[name] = (lo, hi)
        del x, y, d, h, hd, out, out4, wte, dwte, mu, rh, ep, wm
        step_s = sum(t_op[k] * count[k] for k in t_op)
        gbs = total_bytes / step_s / 1e9
        # configs 2-4
        cfgs = {}
        for rows, Cc in ((256, 384), (16384, 768)):
            n2 = rows * Cc
            x2, d2, y2 = f(n2), f(n2), f(n2)
            w2, b2 = np.ones(Cc, np.float32), np.zeros(Cc, np.float32)
            m2, r2, o2 = np.zeros(rows, np.float32), np.zeros(rows, np.float32), np.zeros(n2, np.float32)
            g2, bb2 = np.zeros(Cc, np.float32), np.zeros(Cc, np.float32)
            t, _, _ = med(lambda: o.layernorm_forward(o2, m2, r2, x2, w2, b2, 1, rows, Cc))
            cfgs[f"cfg2 {rows}x{Cc} layernorm_forward"] = t
            t, _, _ = med(lambda: o.layernorm_backward(y2, g2, bb2, d2, x2, w2, m2, r2, 1, rows, Cc))
            cfgs[f"cfg2 {rows}x{Cc} layernorm_backward"] = t
        n3 = 16 * 1024 * 3072
        s3 = n3 // 8
        a3, b3, c3, e3 = f(s3), f(s3), f(s3), np.zeros(s3, np.float32)
        for nm, fn in (("gelu_forward", lambda: o.gelu_forward(e3, a3, s3)),
                       ("gelu_backward", lambda: o.gelu_backward(c3, a3, b3, s3)),
                       ("residual_forward", lambda: o.residual_forward(e3, a3, b3, s3)),
                       ("residual_backward", lambda: o.residual_backward(c3, e3, b3, s3))):
            cfgs[f"cfg3 N={n3} {nm}"] = med(fn, 8.0)[0]
        del a3, b3, c3, e3
        B4, T4 = 16, 1024
        n4 = B4 * T4 * C
        d4, o4 = f(n4), np.zeros(n4, np.float32)
        wte4, wpe4 = f(V * C) * np.float32(0.02), f(T4 * C) * np.float32(0.01)
        dwte4, dwpe4 = np.zeros(V * C, np.float32), np.zeros(T4 * C, np.float32)
        wcdf = np.cumsum(1.0 / np.arange(1, V + 1, dtype=np.float64) ** 1.1)
        wcdf /= wcdf[-1]
        for law in ("uniform", "zipf1.1"):
            tok = (rng.integers(0, V, B4 * T4, dtype=np.int32) if law == "uniform" else
                   np.minimum(np.searchsorted(wcdf, rng.random(B4 * T4)), V - 1).astype(np.int32))
            cfgs[f"cfg4 {law} encoder_forward"] = med(lambda: o.encoder_forward(o4, tok, wte4, wpe4, B4, T4, C))[0]
            cfgs[f"cfg4 {law} encoder_backward"] = med(lambda: o.encoder_backward(dwte4, dwpe4, d4, tok, B4, T4, C))[0]
    finally:
        os.sched_setaffinity(0, set(allowed))
    log(f"bench: cpu ({kind}, 1 core: cpu {core}) step {step_s * 1e3:.1f} ms -> {gbs:.2f} GB/s; "
        f"sample {t_sample:.1f} s; {facts}")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": kind, "ms_per_step": round(step_s * 1e3, 1),
            "GBps_moved_equivalent": round(moved_bytes / step_s / 1e9, 3), "pinned_cpu": core, **facts,
            "per_op_ms": {k: round(v * 1e3, 2) for k, v in t_op.items()},
            "per_op_ms_p25_p75": {k: [round(a * 1e3, 2), round(b * 1e3, 2)] for k, (a, b) in spread.items()},
            "configs_ms": {k: round(v * 1e3, 3) for k, v in cfgs.items()},
            "sample": "train_bnn.c's ops on one pinned core, median of 9 runs each: at the config-5 step "
                      "shapes (materialize on a 1/8 slice, scaled) composed by launch count per step, and at the "
                      "config 2-4 shapes (config-3 ops on a 1/8 slice, scaled); "
                      f"{t_sample:.1f} s of CPU work"}


if __name__ == "__main__":
    main()
