"""Decode throughput of the random-init Qwen3.5-0.8B-shape hybrid model (Q4)
on one MI355X at 32K / 64K / 128K context, with the HBM roofline fraction and
a CPU baseline from the oracle.

A step is one greedy decode token through all 24 layers and the vocab head
(one replay of the captured decode graph). Each context starts with a prompt
of uniform-random token ids consumed by the batched prefill (its time to
first token is reported as `ttft_ms`, host clock around the whole request);
the decode steps are then timed from that post-prefill state. Weights are the
seeded random-init model. `value` is decode tok/s at the 128K context; 32K
and 64K are reported alongside.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "enginesmith-qwen35-08b-long-decode-m5max-round005_amd")
sys.path.insert(0, PKG)
import esdecode as E  # noqa: E402

N_LAYERS, VOCAB = 24, 248320
HBM_PEAK = 8.0e12
GDN_STATE_BYTES = 18 * 2 * 16 * 128 * 128 * 4      # fp32 state read + write
CONV_HISTORY_BYTES = 18 * 73728                      # history read + write (reference byte model)
KV_BYTES_PER_POS = 6 * 2 * 2 * 256 * 2               # 6 layers x {K,V} x 2 heads x 256 x bf16
# k_attn_fused per attended position: K and V rows of the 2 KV heads
# (2048 B); per launch: q|gate, k and v projections read, the new K/V rows
# written, chain outputs and (max, sum) written.
FUSED_BYTES_PER_POS = 2 * 2 * 256 * 2
FUSED_FIXED_BYTES = 8 * 512 * 2 + 2 * 2 * 256 * 2 + 2 * 2 * 256 * 2 + 8 * 64 * (256 + 2) * 4
PROFILES = os.path.join(ROOT, "profiles")
GEN_STEPS = 256  # generate() wall time per context


def committed_traffic(kernel, ctx):
    """HBM bytes per launch from the committed counter summary, if any
    (lines 'fetch_bytes_per_launch: N' and 'write_bytes_per_launch: N')."""
    path = os.path.join(PROFILES, f"{kernel}_ctx{ctx}_counters.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line:
            k, v = line.split(":", 1)
            vals[k.strip()] = v.strip()
    try:
        return int(float(vals["fetch_bytes_per_launch"]) + float(vals["write_bytes_per_launch"]))
    except (KeyError, ValueError):
        return None


def weight_bytes():
    lay = E.weights_layout(N_LAYERS, VOCAB)
    return sum(b for _, _, b, _ in lay) + 576        # + the embedding row gathered per token


def bytes_per_token(ctx, w):
    return w + GDN_STATE_BYTES + CONV_HISTORY_BYTES + KV_BYTES_PER_POS * ctx


def oracle_from_gpu_state(eng, blob, position, extra):
    """The oracle with the GPU's post-prefill state handed over (KV rows, GDN
    conv rings mapped to the reference's [3,6144] history, GDN states)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    views = E.tensor_views(blob, N_LAYERS, VOCAB)
    m = O.OracleModel(views, N_LAYERS, VOCAB, capacity=position + extra)
    for l in range(N_LAYERS):
        if l % 4 == 3:
            m.kcache[l][:, :position] = eng.read_kv(l, 0, 0, position)
            m.vcache[l][:, :position] = eng.read_kv(l, 1, 0, position)
        else:
            ring, state = eng.read_gdn(l)
            m.load_ring(l, ring, position)
            m.state[l][...] = state
    m.position = position
    return m


def bf16_random(r, n, scale=1.0):
    """n bf16 values of N(0, scale) (upper halves of the float32 bits)."""
    return (r.normal(0.0, scale, n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


def median_time(fn, reps):
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_isolated(views, contexts, reps=3):
    """Oracle timings of the path's pieces on the host cores (median of reps,
    the oracle's current thread count): the Q4 matvec at the model's four
    shapes, one GDN step of all 18 layers (conv, gates and delta rule over 16
    heads), and the decode attention of the 6 GQA layers at each context over
    synthetic K/V rows (one layer timed, times 6)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    r = np.random.default_rng(7)
    qmv = {}
    for name, n, k in (("layers.0.mlp.gate_proj", 3584, 1024), ("layers.0.mlp.down_proj", 1024, 3584),
                       ("layers.0.linear_attn.in_proj_qkv", 6144, 1024), ("embed_tokens", VOCAB, 1024)):
        codes = views[name + ".weight"].reshape(n, k // 8)
        sc = views[name + ".scales"].reshape(n, k // 64)
        bi = views[name + ".biases"].reshape(n, k // 64)
        x = bf16_random(r, k)
        dt = median_time(lambda: O.q4_matvec(codes, sc, bi, x), reps)
        nbytes = codes.nbytes + sc.nbytes + bi.nbytes + 2 * (k + n)
        qmv[f"{k}->{n}"] = dict(us=round(dt * 1e6, 1), GBs=round(nbytes / dt / 1e9, 2))
    gdn_layers = [l for l in range(N_LAYERS) if l % 4 != 3]
    raw, a, b = bf16_random(r, 6144, 0.5), bf16_random(r, 16), bf16_random(r, 16)
    hist = {l: np.zeros((3, 6144), dtype=np.uint16) for l in gdn_layers}
    state = {l: np.zeros((16, 128, 128), dtype=np.float32) for l in gdn_layers}

    def gdn_step():
        for l in gdn_layers:
            g = f"layers.{l}.linear_attn"
            conv, gate, beta = O.gdn_conv_prepare(raw, hist[l], views[g + ".conv1d.weight"], a, b,
                                                  views[g + ".A_log"], views[g + ".dt_bias"])
            O.gdn_recur(conv, gate, beta, state[l])

    gdn_s = median_time(gdn_step, reps)
    cap = max(contexts) + 1
    kc = bf16_random(r, 2 * cap * 256, 0.5).reshape(2, cap, 256)
    vc = bf16_random(r, 2 * cap * 256, 0.5).reshape(2, cap, 256)
    query, q_proj = bf16_random(r, 2048, 0.1), bf16_random(r, 4096)
    gqa = {}
    for ctx in contexts:
        dt = median_time(lambda: O.attn_decode_gated(query, kc, vc, ctx, cap, q_proj), reps)
        gqa[str(ctx)] = dict(us_6_layers=round(6 * dt * 1e6, 1), GBs=round(ctx * 2048 / dt / 1e9, 2))
    return dict(q4_matvec=qmv, gdn_18_layers_us=round(gdn_s * 1e6, 1), gqa_decode=gqa)


def cpu_decode_sample(orc, first, stream, threads):
    """Oracle decode steps from the GPU's post-prefill state on `threads`
    host threads, replaying the GPU's greedy stream teacher-forced: seconds
    per step and the number of disagreeing steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.set_threads(threads)
    inp, mism = first, 0
    t0 = time.perf_counter()
    for t in stream:
        mism += orc.step(inp) != t
        inp = t
    return (time.perf_counter() - t0) / max(len(stream), 1), mism


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--contexts", default="32768,65536,131072")
    ap.add_argument("--cpu-steps", type=int, default=16,
                    help="oracle steps per context (timed, and judged for token agreement)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--attn-reps", type=int, default=20)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run the 1 GiB plain-copy kernel that calibrates the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this engine runs on one GPU; multi-GPU decode is not built (it would "
                                   "shard the KV cache by position chain, one all-gather of chain states "
                                   "per attention layer)"}))
        sys.exit(2)
    if E.device_count() < 1:
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)

    contexts = [int(c) for c in args.contexts.split(",")]
    seed = 20260101
    t0 = time.perf_counter()
    blob = E.random_weights(N_LAYERS, VOCAB, seed, threads=min(os.cpu_count() or 8, 16))
    gen_s = time.perf_counter() - t0
    cap = max(contexts) + args.steps + args.warmup + 16 + GEN_STEPS + args.cpu_steps + 1
    eng = E.Engine(blob, N_LAYERS, VOCAB, capacity=cap)
    w = weight_bytes()
    per_ctx, cpu_ctx, agreement = {}, {}, []
    host_cores = os.cpu_count() or 1
    threads = min(host_cores, 16)
    single = None
    r = np.random.default_rng(seed)
    # allocate the prefill buffers and capture the graphs outside the clocks
    eng.generate(r.integers(0, VOCAB, 600).tolist(), 1, reset=True)
    for ctx in contexts:
        # prompt: the decode steps timed below are centred on the context
        start = ctx - args.warmup - args.steps // 2
        prompt = r.integers(0, VOCAB, start).tolist()
        t0 = time.perf_counter()
        first = eng.generate(prompt, 1, reset=True)[0]
        ttft_ms = (time.perf_counter() - t0) * 1e3
        if not args.no_cpu:
            # oracle sample: the state handed over after the prompt, then a few
            # greedy GPU tokens that the oracle replays teacher-forced on the
            # host cores (the GPU is idle meanwhile); at the headline context
            # one more step on a single thread
            head = ctx == max(contexts)
            n_cpu = args.cpu_steps
            orc = oracle_from_gpu_state(eng, blob, eng.position, n_cpu + 4)
            stream = eng.generate([], n_cpu + (1 if head else 0), reset=False)
            sec, mism = cpu_decode_sample(orc, first, stream[:n_cpu], threads)
            cpu_ctx[ctx] = round(1.0 / sec, 3)
            if head:
                sec1, mism1 = cpu_decode_sample(orc, stream[n_cpu - 1], stream[n_cpu:], 1)
                single = dict(tok_s=round(1.0 / sec1, 4), steps=1, context=ctx)
                mism += mism1
            agreement.append(dict(context=ctx, steps=len(stream), mismatches=int(mism)))
            del orc
        ms = eng.time_decode(args.steps, args.warmup)
        # the serving path: generate() with its host synchronisation every 16 steps
        t0 = time.perf_counter()
        eng.generate([], GEN_STEPS, reset=False)
        gen_ms = (time.perf_counter() - t0) * 1e3
        tps = args.steps / (ms / 1e3)
        b = bytes_per_token(ctx, w)
        per_ctx[ctx] = dict(tok_s=round(tps, 1), ms_per_step=round(ms / args.steps, 4),
                            bytes_per_token=b, achieved_GBs=round(b * tps / 1e9, 1),
                            roofline_frac=round(b * tps / HBM_PEAK, 4),
                            prompt_tokens=start, ttft_ms=round(ttft_ms, 1),
                            prefill_tok_s=round((start - 1) / (ttft_ms / 1e3), 1),
                            generate_256=dict(wall_ms=round(gen_ms, 1), tok_s=round(GEN_STEPS / (gen_ms / 1e3), 1)))
        print(f"# ctx {ctx}: TTFT {ttft_ms:.0f} ms for {start} prompt tokens; {tps:.1f} tok/s, "
              f"{ms / args.steps * 1e3:.1f} us/step, "
              f"{b * tps / 1e9:.0f} GB/s ({b * tps / HBM_PEAK * 100:.1f}% of 8 TB/s)", file=sys.stderr, flush=True)
    head_ctx = max(contexts)
    # dominant kernel: the fused scores + per-chain online softmax of one
    # attention layer at the headline context (it streams the layer's K and V)
    eng.fill_synthetic(head_ctx - 1, seed=1, pending=1)
    # rotate over the six attention layers: every launch streams a cold cache
    parts = {p: eng.time_attention(-1, args.attn_reps, p) for p in ("chains", "merge", "all")}
    chain_ms = parts["chains"]
    n_att = head_ctx  # attended positions, including the new one
    chain_bytes = FUSED_BYTES_PER_POS * n_att + FUSED_FIXED_BYTES
    head_ms = eng.time_head(args.attn_reps)
    eng.close()
    copy_bytes = 1 << 30
    copy_ms = E.time_copy(copy_bytes, reps=20 if args.copy_calibration else 5)
    copy_gbs = 2 * copy_bytes / (copy_ms / 1e3) / 1e9
    read_ms = E.time_read(copy_bytes, reps=10)
    read_gbs = copy_bytes / (read_ms / 1e3) / 1e9

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        O.set_threads(threads)
        iso = cpu_isolated(E.tensor_views(blob, N_LAYERS, VOCAB), contexts)
        cpu = dict(value=cpu_ctx[head_ctx], unit="tok/s", cores=threads, kind="port",
                   sample=f"oracle decode steps of the 24-layer model from the GPU's post-prefill state "
                          f"({args.cpu_steps} at each context, replaying the GPU's greedy tokens), "
                          f"{threads} OpenMP threads; isolated pieces median of 3",
                   threads=threads, host_cores=host_cores, per_context={str(k): v for k, v in cpu_ctx.items()},
                   single_thread=single, isolated=iso)

    main_ctx = per_ctx[head_ctx]
    line = {
        "metric": "decode tok/s at 32K/64K/128K ctx on 1 MI355X; % of HBM roofline",
        "value": main_ctx["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_ctx["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4-affine weights, bf16 activations, fp32 accumulate",
        "data": "synthetic: seeded random-init weights, uniform-random prompt ids prefilled on the GPU",
        "config": {
            "workload": f"batch-1 greedy decode, Qwen3.5-0.8B-shape hybrid (18 GDN + 6 GQA layers, Q4 g64), "
                        f"{head_ctx} context",
            "n_layers": N_LAYERS, "vocab": VOCAB, "contexts": contexts,
            "per_context": {str(k): v for k, v in per_ctx.items()},
            "step_roofline_frac_8TBs": main_ctx["roofline_frac"],
            "ttft_ms": {str(k): v["ttft_ms"] for k, v in per_ctx.items()},
            "token_agreement": dict(contexts=agreement,
                                    judged="greedy GPU tokens replayed teacher-forced by the oracle "
                                           "from the GPU's post-prefill state") if agreement else None,
            "weight_gen_s": round(gen_s, 1),
            "head_kernel_us": round(head_ms * 1e3, 2),
        },
        "roofline": {
            "kernel": f"k_attn_fused (scores + per-chain online softmax over K and V, one attention "
                      f"layer, {n_att} positions)",
            "bound": "hbm",
            "achieved": round(chain_bytes / (chain_ms / 1e3) / 1e9, 1),
            "peak": 8000.0,
            "unit": "GB/s",
            "frac": round(chain_bytes / (chain_ms / 1e3) / HBM_PEAK, 4),
            "traffic": committed_traffic("k_attn_fused", head_ctx),
            "traffic_source": f"profiles/k_attn_fused_ctx{head_ctx}_counters.txt: rocprofv3 FETCH_SIZE + "
                              f"WRITE_SIZE per launch from a committed run, not measured in this one",
            "algorithmic_bytes": chain_bytes,
            "launch_us": round(chain_ms * 1e3, 2),
            "attention_layer_us": {k: round(v * 1e3, 2) for k, v in parts.items()},
            "measured_copy_GBs": round(copy_gbs, 1),
            "measured_read_GBs": round(read_gbs, 1),
            "frac_of_measured_read": round(chain_bytes / (chain_ms / 1e3) / 1e9 / read_gbs, 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
