"""Benchmark: accepted tokens/s of MTP speculative decoding on one MI355X.

Workload (default, --config B): 1B-class decoder (24 layers, hidden 2048, 16
heads x 128, SwiGLU 5632, tied vocab 16384), all matrices Q4 (32-wide
blocks, fp16 scale, weights N(0, 0.02)), 4 Q4 MTP heads, int8 3-tier KV
(sink 4, window 8192), greedy draft = 4, batch 1, 2048-token uniform random
prompt, 512 generated.  --config S / B-mix / B-long select the other
single-sequence workloads (see CONFIGS).

A step is one decode of 512 tokens after the prompt: the engine is reset and
the first 2047 prompt tokens are prefilled before the timer starts (their KV
is resident in HBM); the timed call is generate([last prompt token], 512),
which forwards the last prompt token and runs the MTP rounds.  value =
generated tokens / decode wall time over the K timed steps.

Also reported: the one-row pass's layer launch (k_stack: every layer in one
launch) and its achieved HBM bandwidth (HIP events around every dispatch,
algorithmic bytes = every layer's packed matrices with their fp32 input and
output rows + the visible int8 K/V rows with scales), the verify pass as a
whole, and
the CPU restatement (oracle) timed on the host cores on a bounded sample of
the same call: generate([last prompt token], 64 tokens on all cores, 16 on
one) from the GPU's
prefilled state at the workload's context, imported into the oracle.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "accepted tok/s @1B Q4 MTP draft=4, bs=1; verify-step HBM GB/s vs peak"

# Single-sequence workloads: model, weight formats, KV geometry (sink,
# window, pool), prompt and generated lengths, sampling (temperature,
# top-p, top-k, greedy).  "B" is the headline configuration.
CONFIGS = {
    "B": dict(model="ONE_B", fmts="ALL_Q4", kv=(4, 8192, 64), prompt=2048, new=512, samp=(0.8, 0.95, 40, 1),
              name="1B Q4 (24L, d2048, 16x128 heads, ff5632, vocab 16384 tied), 4 Q4 MTP heads, greedy"),
    "S": dict(model="SMALL", fmts="ALL_Q4", kv=(4, 8192, 64), prompt=64, new=256, samp=(0.8, 0.95, 40, 1),
              name="150M Q4 (12L, d768, 12x64 heads, ff2048, vocab 16384 tied), 4 Q4 MTP heads, greedy"),
    "B-mix": dict(model="ONE_B", fmts="MIXED", kv=(4, 8192, 64), prompt=1024, new=512, samp=(0.8, 0.95, 40, 0),
                  name="1B mixed (attention Q4, gate/up Q2, down Q1.5), 4 Q4 MTP heads, temperature 0.8, top-p 0.95 "
                       "(top-k 40 not reached: the reference dispatch takes top-p first), Philox seed 7"),
    "B-long": dict(model="ONE_B", fmts="ALL_Q4", kv=(4, 4096, 16), prompt=32768, new=256, samp=(0.8, 0.95, 40, 1),
                   name="1B Q4, 4 Q4 MTP heads, greedy, long context"),
    # many sequences decoded together: verify passes of 64 x 5 = 320 rows on
    # the int8 MFMA GEMM; a step generates `new` tokens per sequence
    "E": dict(model="ONE_B", fmts="ALL_Q4", kv=(4, 8192, 64), prompt=8192, new=64, samp=(0.8, 0.95, 40, 1),
              seqs=64, name="1B Q4, 4 Q4 MTP heads, greedy, 64 sequences (distinct prompts) decoded together"),
}


def view_count(pos, sink, window, pool):
    """Visible entries of a query at position pos (sink + pooled + window)."""
    s = min(pos, sink)
    nw = max(0, pos - sink)
    win = min(nw, window)
    return s + (nw - win) // pool + win


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "stack_traffic_1b_q4.md")


def measured_traffic():
    """HBM bytes per k_stack dispatch of the headline workload from the
    committed hardware-counter profile (FETCH_SIZE and WRITE_SIZE, scaled by
    a copy kernel of known size), or None when the profile is absent."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch_avg:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def snapshot_planes(eng, cfg, kv):
    """Every KV plane of the engine's sequence (pf_engine_kv_export) at its
    position, with the first window position, for the oracle's import."""
    P = eng.pos
    cap = 8 + kv["window_size"] + kv["pool_block"] + P // kv["pool_block"] + 8
    planes = []
    for l in range(cfg["n_layers"]):
        for h in range(cfg["n_heads"]):
            k, ks, v, vs, counts = eng.kv_export(0, l, h, cap)
            planes.append((l, h, counts, kv["sink_size"] + counts[1] * kv["pool_block"] + counts[3], k, ks, v, vs))
    return P, planes


def cpu_baseline(cfg, w, kv, snapshot, last, n_new, samp, what, gpu_tokens, threads=0):
    """The oracle (C restatement) running a step's timed call,
    generate([last prompt token], n_new), on the host cores from the GPU's
    prefilled state at the workload's context (every KV plane exported and
    imported): all cores (threads=0) or a given number of threads (1: the
    reference's single-threaded compute).  Bounded by n_new."""
    import oracle as O
    c = dict(cfg)
    c.update(kv)
    all_threads = int(O.lib().orc_num_threads())
    O.lib().orc_set_num_threads(threads or all_threads)
    om = O.Model(c, w)
    P, planes = snapshot
    for l, h, counts, wpos0, k, ks, v, vs in planes:
        om.kv_import(l, h, counts, wpos0, k, ks, v, vs)
    om.set_state(P)
    t0 = time.perf_counter()
    toks, acc, rej = om.generate([last], n_new, O.Sampling(*samp), 7)
    wall = time.perf_counter() - t0
    om.close()
    used = int(O.lib().orc_num_threads())
    O.lib().orc_set_num_threads(all_threads)
    gen = len(toks) - 1
    # the MTP rounds of both runs agree while n + 4 <= n_new
    k = max(0, n_new - 4)
    agree = None if gpu_tokens is None else bool(np.array_equal(toks[1:1 + k], gpu_tokens[1:1 + k]))
    par = "single thread" if used == 1 else f"OpenMP row-parallel GEMVs, {used} threads"
    return {
        "value": round(gen / wall, 4),
        "unit": "tok/s",
        "cores": used,
        "kind": "port",
        "sample": (f"oracle (C restatement, {par}): generate([last prompt token], {n_new}) from the GPU's prefilled "
                   f"state at context {P} (all {len(planes)} KV planes exported and imported), the same call, "
                   f"weights and sampling as a timed step of {what}; {gen} tokens in {wall:.2f}s wall"),
        "context": P,
        "tokens_match_gpu": agree,
    }


def copy_probe(nbytes):
    """Three device-to-device copies of nbytes through the runtime's copy
    kernel: the known-size reference that scales the FETCH_SIZE and
    WRITE_SIZE counters of the decode kernels."""
    import pocketforge_amd as pf
    ctx = pf.Context(0)
    a = pf.DeviceArray(ctx, (nbytes,), np.uint8)
    b = pf.DeviceArray(ctx, (nbytes,), np.uint8)
    for _ in range(3):
        ctx.check(pf.lib().pf_memcpy(ctx.h, b.ptr, a.ptr, nbytes, 2), "pf_memcpy")
    ctx.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}), flush=True)
    a.free()
    b.free()
    ctx.close()


def gemm_probe(M):
    """The int8 MFMA GEMM alone: pf_gemv_q on M activation rows (rows
    quantized, then k_gemm) for the four products of one 1B layer (QKV,
    O, gate|up, down; Q4 weights N(0, 0.02)), 10 launches each, with the
    host time per call (synchronized) beside it.  The workload of the
    GEMM's kernel-trace and hardware-counter passes."""
    import pocketforge_amd as pf
    from pocketforge_amd import weights as W
    cfg = W.ONE_B
    D, F = cfg["n_embd"], cfg["n_ff"]
    ctx = pf.Context(0)
    rng = np.random.default_rng(5)
    out = {"gemm_probe_rows": M, "products": []}
    for name, (N, K) in (("qkv", (3 * D, D)), ("o", (D, D)), ("gate_up", (2 * F, D)), ("down", (D, F))):
        codes, scales = pf.gen_matrix(1234, 77, 0.02, N, K, pf.FMT_Q4)
        Wm = ctx.upload_matrix(pf.FMT_Q4, codes, scales)
        x = ctx.to_device(rng.normal(0.0, 1.0, (M, K)).astype(np.float32))
        ctx.gemv_q(Wm, x)
        t0 = time.perf_counter()
        for _ in range(10):
            ctx.gemv_q(Wm, x)
        us = (time.perf_counter() - t0) / 10 * 1e6
        out["products"].append({"name": name, "N": N, "K": K, "host_us_per_call": round(us, 1),
                                "ops": 2 * M * N * K})
        Wm.close()
    print(json.dumps(out), flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", default="B", choices=sorted(CONFIGS),
                    help="workload (default B, the headline configuration)")
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=0, help="prompt length (default: the configuration's)")
    ap.add_argument("--new", type=int, default=0, help="generated tokens (default: the configuration's)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--layer-skip", type=float, default=0.0,
                    help="layer-skip threshold (0: off, the default; single-sequence configurations)")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only run 3 device-to-device copies of this many bytes (hardware-counter calibration)")
    ap.add_argument("--gemm-probe", type=int, default=0,
                    help="only run the int8 GEMM on this many rows for the four 1B layer products (counter passes)")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gemm_probe:
        gemm_probe(args.gemm_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is a design note only "
                                   "(batch-1 MTP decode has no data-parallel axis)", "n_gpus": args.gpus}))
        sys.exit(2)

    import pocketforge_amd as pf
    from pocketforge_amd import weights as W

    C = CONFIGS[args.config]
    args.prompt = args.prompt or C["prompt"]
    args.new = args.new or C["new"]
    cfg = getattr(W, C["model"])
    t0 = time.perf_counter()
    w = W.make_weights(cfg, seed=1234, fmts=getattr(W, C["fmts"]))
    log(f"weights generated in {time.perf_counter() - t0:.1f}s")
    ctx = pf.Context(0)
    dev, cus = ctx.device_info()
    t0 = time.perf_counter()
    model = pf.Model(ctx, cfg, w)
    log(f"weights uploaded in {time.perf_counter() - t0:.1f}s on {dev} ({cus} CUs)")
    if "seqs" in C:
        bench_batch(args, C, cfg, w, ctx, dev, model)
        return
    max_ctx = args.prompt + args.new + 64
    sink, window, pool = C["kv"]
    kv = dict(sink_size=sink, window_size=window, pool_block=pool, max_context=max_ctx)
    eng = pf.Engine(model, **kv)
    if args.layer_skip:
        eng.set_layer_skip(args.layer_skip, 4)
    prompt = W.prompt_ids(args.prompt, cfg["n_vocab"], seed=42)
    greedy = pf.Sampling(*C["samp"])

    prefill_s = []

    def step(profile):
        eng.reset()
        t = time.perf_counter()
        for i in range(0, args.prompt - 1, 256):
            eng.prefill(prompt[i:min(i + 256, args.prompt - 1)])
        ctx.synchronize()
        prefill_s.append(time.perf_counter() - t)
        eng.profile(profile)
        t = time.perf_counter()
        toks, res = eng.generate(prompt[-1:], args.new, greedy, 7)
        ctx.synchronize()
        return time.perf_counter() - t, toks, res

    for i in range(args.warmup):
        dt, toks, res = step(False)
        log(f"warmup {i}: {len(toks) - 1} tokens in {dt * 1e3:.1f} ms")
    times, gens, accs, rejs, rounds, round_us = [], [], [], [], [], []
    for i in range(args.steps):
        dt, toks, res = step(False)
        times.append(dt)
        gens.append(len(toks) - 1)
        accs.append(res.mtp_accepted)
        rejs.append(res.mtp_rejected)
        rounds.append(res.rounds)
        log(f"step {i}: {gens[-1]} tokens in {dt * 1e3:.1f} ms ({gens[-1] / dt:.1f} tok/s), rounds {res.rounds}, "
            f"accepted {res.mtp_accepted}")
    value = sum(gens) / sum(times)
    # the device time per round from one more step of the same decode with
    # HIP events around every round (pf_engine_set_round_timing; the timed
    # steps run without them, whose recording costs wall time)
    eng.set_round_timing(True)
    step(False)
    r_us, r_n = eng.round_time()
    eng.set_round_timing(False)
    round_us.append((r_us, r_n))
    log(f"round-timed step: device time per MTP round {r_us:.1f} us over {r_n} rounds")
    # one more decode of the same workload, kernels issued one by one with
    # HIP start/stop events attached to every layer launch of the decode
    # passes (k_stack for one row)
    dt_p, toks_p, res_p = step(True)
    n_l, gemv_us, gemv_bytes = eng.gemv_stats()
    gemv_groups = eng.gemv_by_size()
    a_n, attn_us = eng.attn_stats()
    v_ev, b_ev, _, _ = eng.pass_times()
    log(f"profiled step: {dt_p * 1e3:.1f} ms, verify pass {v_ev:.1f} us, base pass {b_ev:.1f} us (with dispatch "
        f"events), layer launch {gemv_us:.2f} us avg x{n_l}")
    # and one more, issued the same way with events around each pass only:
    # the pass times without the dispatch events' own cost
    step(2)
    v_us, b_us, vn, bn = eng.pass_times()
    eng.profile(False)
    log(f"pass-timed step: verify pass {v_us:.1f} us x{vn}, base pass {b_us:.1f} us x{bn}")
    # the same workload with every round verifying all n_mtp + 1 rows in one
    # pass (pf_engine_set_verify_full): one timed step in graphs, one
    # pass-timed step
    eng.set_verify_full(True)
    dt_f, toks_f, res_f = step(False)
    step(2)
    vf_us, _, vf_n, _ = eng.pass_times()
    eng.profile(False)
    eng.set_verify_full(False)
    log(f"full-verify step: {len(toks_f) - 1} tokens in {dt_f * 1e3:.1f} ms ({(len(toks_f) - 1) / dt_f:.1f} tok/s), "
        f"verify pass ({cfg['n_mtp'] + 1} rows) {vf_us:.1f} us x{vf_n}")
    # labelled diagnostic: the same shapes with every layer and MTP-head
    # matrix zero (the hidden state is the token's embedding, so the model
    # repeats its input and every greedy draft is accepted): rounds that
    # commit all n_mtp + 1 tokens with one verify pass, the k + 1 ceiling of
    # the round; the matrices are read in full, so the passes cost what they
    # cost with the random weights
    full_accept = None
    if args.config == "B":
        mz = pf.Model(ctx, cfg, zero_weights(w))
        ez = pf.Engine(mz, **kv)

        def zstep(profile):
            ez.reset()
            for i in range(0, args.prompt - 1, 256):
                ez.prefill(prompt[i:min(i + 256, args.prompt - 1)])
            ctx.synchronize()
            ez.profile(profile)
            t = time.perf_counter()
            toks, res = ez.generate(prompt[-1:], args.new, greedy, 7)
            ctx.synchronize()
            return time.perf_counter() - t, toks, res

        zstep(False)
        dt_z, toks_z, res_z = zstep(False)
        zstep(2)
        vz_us, bz_us, vz_n, bz_n = ez.pass_times()
        ez.profile(False)
        full_accept = {
            "value": round((len(toks_z) - 1) / dt_z, 3),
            "weights": "every layer and MTP-head matrix zero (diagnostic; same shapes and bytes read)",
            "mtp_accepted": res_z.mtp_accepted, "mtp_rejected": res_z.mtp_rejected, "rounds": res_z.rounds,
            "committed_per_round": round((len(toks_z) - 1) / max(1, res_z.rounds), 3),
            "verify_pass_us": round(vz_us, 2), "verify_passes": vz_n,
            "base_passes": bz_n,
        }
        log(f"full-acceptance step: {len(toks_z) - 1} tokens in {dt_z * 1e3:.1f} ms "
            f"({(len(toks_z) - 1) / dt_z:.1f} tok/s), {res_z.rounds} rounds, accepted {res_z.mtp_accepted}, "
            f"verify pass {vz_us:.1f} us x{vz_n}")
        ez.close()
        mz.close()
    achieved = gemv_bytes / gemv_us / 1e3
    r_avg = sum(r[0] * r[1] for r in round_us) / max(1, sum(r[1] for r in round_us))
    # verify pass algorithmic bytes: every packed weight once (incl. the tied
    # unembedding) + the visible int8 KV rows with fp32 scales, at the mean
    # visible list length of the decode
    wbytes = W.packed_bytes(w) + w["emb"][1].nbytes + w["emb"][2].nbytes
    ctx_mean = sum(view_count(p, sink, window, pool) for p in range(args.prompt, args.prompt + args.new)) / args.new
    kv_bytes = cfg["n_layers"] * 2 * cfg["n_heads"] * (cfg["head_dim"] + 4) * ctx_mean
    pass_bytes = wbytes + kv_bytes
    headline = args.config == "B"
    out = {
        "metric": METRIC if headline else f"accepted tok/s, configuration {args.config}, MTP draft=4, bs=1",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * sum(times) / len(times), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init weights N(0,0.02), uniform random prompt ids)",
        "config": {
            "workload": (f"{C['name']}, draft=4, bs=1, {args.prompt}-token prompt, {args.new} generated, "
                         f"int8 3-tier KV (sink {sink}, window {window}, pool {pool})"),
            "accepted_per_round": round(sum(accs) / max(1, sum(rounds)), 4),
            "mtp_accepted": sum(accs), "mtp_rejected": sum(rejs), "rounds": sum(rounds),
            "tokens_per_step": gens[0],
            "device_us_per_round": round(r_avg, 2),
            "prefill_tok_s": round((args.prompt - 1) / min(prefill_s), 1),
            "device": dev,
            **({"layer_skip_threshold": args.layer_skip,
                "ffn_blocks_skipped_last_step": eng.layer_skip_count()} if args.layer_skip else {}),
        },
        "roofline": {
            "kernel": ("k_stack (one-row decode pass: every layer's QKV product, attention, chunk merge, O, "
                       "gate|up and down products in one launch; bytes = every layer's four matrices with their fp32 "
                       "input and output rows + the visible int8 K/V rows with scales)" if headline else
                       "the decode passes' layer launches: k_stack for one-row passes, k_o_ffn (merge, O, gate|up) "
                       "for passes of 2-8 rows; bytes = the launch's matrices with their fp32 rows (+ K/V rows for "
                       "k_stack)"),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic() if headline else None,
            "traffic_source": "profiles/stack_traffic_1b_q4.md (rocprofv3 FETCH_SIZE and WRITE_SIZE per k_stack "
                              "dispatch of this workload, scaled by a copy kernel of known size)",
            "avg_launch_us": round(gemv_us, 3),
            "avg_bytes_per_launch": round(gemv_bytes),
            "launches": n_l,
            "timing": "HIP start/stop events attached to each k_stack dispatch (hipExtLaunchKernelGGL) on the engine "
                      "stream, in one extra decode step of the same workload issued without graphs",
            "range": ({"min_bytes": round(min(b for b, _, _ in gemv_groups)),
                       "max_bytes": round(max(b for b, _, _ in gemv_groups)),
                       "min_us": round(min(u for _, _, u in gemv_groups), 3),
                       "max_us": round(max(u for _, _, u in gemv_groups), 3)} if gemv_groups else None),
        },
        "verify_pass": {
            "avg_us": round(v_us, 2),
            "bytes": round(pass_bytes),
            "achieved_GBps": round(pass_bytes / v_us / 1e3, 1),
            "frac": round(pass_bytes / v_us / 1e3 / HBM_PEAK_GBPS, 4),
            "attention_avg_us": round(attn_us, 2),
            "attention_launches": a_n,
            "timing": "HIP events around each verify pass on the engine stream, in one more decode step of the same "
                      "workload issued without graphs and without per-dispatch events",
            "with_dispatch_events_us": round(v_ev, 2),
        },
        # every round verifying all n_mtp + 1 rows in one pass (the segment
        # policy's alternative): throughput and the undisturbed pass time
        "verify_full": {
            "value": round((len(toks_f) - 1) / dt_f, 3),
            "rows": cfg["n_mtp"] + 1,
            "verify_pass_us": round(vf_us, 2),
            "achieved_GBps": round(pass_bytes / vf_us / 1e3, 1),
            "frac": round(pass_bytes / vf_us / 1e3 / HBM_PEAK_GBPS, 4),
        },
        **({"full_acceptance": dict(full_accept, achieved_GBps=round(pass_bytes / full_accept["verify_pass_us"] / 1e3, 1),
                                     frac=round(pass_bytes / full_accept["verify_pass_us"] / 1e3 / HBM_PEAK_GBPS, 4))}
           if full_accept else {}),
    }
    if not args.no_cpu:
        # the prefilled state of a step, exported once for both oracle runs
        eng.reset()
        for i in range(0, args.prompt - 1, 256):
            eng.prefill(prompt[i:min(i + 256, args.prompt - 1)])
        snap = snapshot_planes(eng, cfg, kv)
        log(f"cpu baseline from the state at context {snap[0]} ...")
        out["cpu_baseline"] = cpu_baseline(cfg, w, kv, snap, int(prompt[-1]), 64, C["samp"], args.config, toks_p)
        log("cpu baseline, one thread ...")
        out["cpu_baseline_1thread"] = cpu_baseline(cfg, w, kv, snap, int(prompt[-1]), 16, C["samp"], args.config,
                                                   toks_p, threads=1)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    eng.close()
    model.close()
    ctx.close()


GEMM_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA


def zero_weights(w):
    """The weight set with every layer and MTP-head matrix zero (every code
    the zero value, every block scale 0); the tied embedding kept."""
    import copy
    import pocketforge_amd as pf
    zero_code = {pf.FMT_Q4: 0x88, pf.FMT_Q2: 0xAA, pf.FMT_Q15: 0x55}
    w2 = copy.copy(w)
    w2["layers"] = [{n: (f, np.full_like(c, zero_code[f]), np.zeros_like(s)) for n, (f, c, s) in lw.items()}
                    for lw in w["layers"]]
    w2["mtp"] = [{n: (f, np.full_like(c, zero_code[f]), np.zeros_like(s)) for n, (f, c, s) in hw.items()}
                 for hw in w["mtp"]]
    return w2


def bench_batch(args, C, cfg, w, ctx, dev, model):
    """Many sequences decoded together.  Every sequence's prompt (its own
    seed) is prefilled once, outside the timer, up to its last token; step k
    is one batched generate of `new` tokens per sequence that forwards each
    sequence's last token and continues its decode (the contexts grow by
    about new + 1 per step).  value = generated tokens of all sequences /
    wall time of the timed steps."""
    import pocketforge_amd as pf
    from pocketforge_amd import weights as W
    N = C["seqs"]
    sink, window, pool = C["kv"]
    n_steps = args.warmup + args.steps + 1
    max_ctx = args.prompt + (args.new + 8) * n_steps + 64
    kv = dict(sink_size=sink, window_size=window, pool_block=pool, max_context=max_ctx)
    eng = pf.BatchEngine(model, N, **kv)
    samp = pf.Sampling(*C["samp"])
    seeds = np.full(N, 7, np.uint64)
    prompts = [W.prompt_ids(args.prompt, cfg["n_vocab"], seed=42 + s) for s in range(N)]
    t = time.perf_counter()
    for s in range(N):
        eng.prefill_seq(s, prompts[s][:-1])
        if s % 8 == 7:
            log(f"prefilled {s + 1} sequences ({time.perf_counter() - t:.1f}s)")
    prefill_s = time.perf_counter() - t
    last = [p[-1:] for p in prompts]

    def step(profile):
        eng.profile(profile)
        t0 = time.perf_counter()
        toks, res = eng.generate_batch(last, args.new, samp, seeds)
        ctx.synchronize()
        dt = time.perf_counter() - t0
        for s in range(N):
            last[s] = toks[s][-1:]
        return dt, toks, res

    for i in range(args.warmup):
        dt, toks, res = step(False)
        log(f"warmup {i}: {sum(len(x) - 1 for x in toks)} tokens in {dt * 1e3:.1f} ms")
    times, gens, accs, rejs, rounds, round_us = [], [], [], [], [], []
    for i in range(args.steps):
        dt, toks, res = step(False)
        r_us, r_n = eng.round_time()
        times.append(dt)
        gens.append(sum(len(x) - 1 for x in toks))
        accs.append(sum(r.mtp_accepted for r in res))
        rejs.append(sum(r.mtp_rejected for r in res))
        rounds.append(max(r.rounds for r in res))
        round_us.append((r_us, r_n))
        log(f"step {i}: {gens[-1]} tokens in {dt * 1e3:.1f} ms ({gens[-1] / dt:.1f} tok/s), rounds {rounds[-1]}, "
            f"device time per round {r_us:.1f} us")
    value = sum(gens) / sum(times)
    # one more step of the same workload with HIP start/stop events attached
    # to every GEMM dispatch of the verify passes (M = 5 x sequences)
    dt_p, toks_p, res_p = step(True)
    n_l, gemm_us, gemm_bytes = eng.gemv_stats()
    a_n, attn_us = eng.attn_stats()
    v_ev, b_ev, _, _ = eng.pass_times()
    # one more step with events around each pass only (undisturbed pass times)
    step(2)
    v_us, b_us, vn, bn = eng.pass_times()
    eng.profile(False)
    M = N * (cfg["n_mtp"] + 1)
    D, F = cfg["n_embd"], cfg["n_ff"]
    nk = [(3 * D, D), (D, D), (2 * F, D), (D, F)]    # QKV, O, gate|up, down (N x K) of every layer
    gemm_ops = 2.0 * M * sum(n * k for n, k in nk) / len(nk)
    log(f"profiled step: {dt_p * 1e3:.1f} ms, verify pass {v_ev:.1f} us (with dispatch events), "
        f"gemm {gemm_us:.2f} us avg x{n_l}; pass-timed step: verify pass {v_us:.1f} us x{vn}, "
        f"base pass {b_us:.1f} us x{bn}")
    achieved = gemm_ops / gemm_us / 1e6
    r_avg = sum(r[0] * r[1] for r in round_us) / max(1, sum(r[1] for r in round_us))
    wbytes = W.packed_bytes(w) + w["emb"][1].nbytes + w["emb"][2].nbytes
    p_mid = args.prompt + (args.warmup + args.steps // 2) * (args.new + 1)
    kv_bytes = N * cfg["n_layers"] * 2 * cfg["n_heads"] * (cfg["head_dim"] + 4) * view_count(p_mid, sink, window, pool)
    # verify-pass attention of one layer: every sequence's visible K/V rows
    # (int8 codes + fp32 row scales) once, at the profiled step's mid context
    p_prof = args.prompt + (args.warmup + args.steps) * (args.new + 1) + args.new // 2
    attn_bytes = N * 2 * cfg["n_heads"] * (cfg["head_dim"] + 4) * view_count(p_prof, sink, window, pool)
    attn_gbps = attn_bytes / attn_us / 1e3 if attn_us else 0.0
    out = {
        "metric": f"accepted tok/s (all sequences), configuration E, MTP draft=4, {N} sequences",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * sum(times) / len(times), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init weights N(0,0.02), uniform random prompt ids, one prompt seed per sequence)",
        "config": {
            "workload": (f"{C['name']}, draft=4, {args.prompt}-token prompt per sequence, {args.new} generated per "
                         f"sequence per step, int8 3-tier KV (sink {sink}, window {window}, pool {pool})"),
            "sequences": N,
            "verify_rows": M,
            "accepted_per_round": round(sum(accs) / max(1, sum(rounds) * N), 4),
            "mtp_accepted": sum(accs), "mtp_rejected": sum(rejs), "rounds": sum(rounds),
            "tokens_per_step": gens[0],
            "device_us_per_round": round(r_avg, 2),
            "prefill_tok_s": round(N * (args.prompt - 1) / prefill_s, 1),
            "device": dev,
        },
        # the step's dominant kernel: verify-pass attention (78% of the decode's
        # kernel time), bound by HBM
        "roofline": {
            "kernel": f"k_attn_seq<8> (verify-pass attention, {M} rows over {N} sequences' int8 K/V)",
            "bound": "hbm",
            "achieved": round(attn_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "avg_launch_us": round(attn_us, 2),
            "avg_bytes_per_launch": round(attn_bytes),
            "launches": a_n,
            "timing": "HIP start/stop events attached to each attention dispatch of the verify passes "
                      "(hipExtLaunchKernelGGL) on the engine stream, in one extra step of the same workload",
        },
        "gemm_roofline": {
            "kernel": f"k_gemm<Q4> (verify-pass int8 x Q4 MFMA GEMM, M={M}; average over QKV, O, gate|up, down)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": GEMM_PEAK_TOPS,
            "unit": "TOP/s",
            "frac": round(achieved / GEMM_PEAK_TOPS, 4),
            "avg_launch_us": round(gemm_us, 3),
            "avg_ops_per_launch": round(gemm_ops),
            "avg_bytes_per_launch": round(gemm_bytes),
            "launches": n_l,
        },
        "verify_pass": {
            "avg_us": round(v_us, 2),
            "bytes": round(wbytes + kv_bytes),
            "achieved_GBps": round((wbytes + kv_bytes) / v_us / 1e3, 1),
            "frac": round((wbytes + kv_bytes) / v_us / 1e3 / HBM_PEAK_GBPS, 4),
            "timing": "HIP events around each verify pass on the engine stream, in one more step of the same "
                      "workload issued without graphs and without per-dispatch events",
        },
    }
    if not args.no_cpu:
        # sequence 0's state after the steps; the next step forwards last[0]
        snap = snapshot_planes(eng, cfg, kv)
        log(f"cpu baseline from sequence 0's state at context {snap[0]} ...")
        out["cpu_baseline"] = cpu_baseline(cfg, w, kv, snap, int(last[0][0]), 16, C["samp"], "E, one sequence",
                                           None)
        out["cpu_baseline_1thread"] = cpu_baseline(cfg, w, kv, snap, int(last[0][0]), 8, C["samp"],
                                                   "E, one sequence", None, threads=1)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    eng.close()
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
