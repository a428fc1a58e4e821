#!/usr/bin/env python3
"""Benchmark of the quantized MoE expert path on one MI355X.

Workload (decode b=1): MoE layers of 256 experts, top-8, hidden 2048,
expert FFN 512, gate/up IQ2_XXS and down IQ2_S, router logits ~ N(0,1), SwiGLU, every expert
resident. A step is one token through a chain of --layers such layers (40 by default, the layer
count of the model config 3 copies); each layer reads its own 224 MB bank, so the 256 MB
Infinity Cache cannot serve a step's 280 MB of picked expert weights from a previous step, and
every step routes with fresh logits. Weights are seeded synthetic blocks built on the device.

Prints one JSON line: the headline value is the achieved HBM throughput on the algorithmic bytes
of a decode layer (the picked experts' GGUF blocks plus activations in and out), beside µs per
layer, the roofline fraction, a prefill measurement at 1,500 tokens, the parity of layer 0
against the CPU oracle, and the oracle timed on the host as the CPU baseline.
"""
import argparse
import json
import os
import sys
import time

METRIC = "MoE layer µs + achieved HBM GB/s (decode b=1); prefill tokens/s; MFMA util"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_F16_TFLOPS = 2500.0  # dense fp16
MFMA_PEAK_F6F4_TFLOPS = 10100.0  # dense fp6 / fp4 (the block-scaled MFMA)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def time_replays(torch, g, calls, warm=3, timed=5):
    """Median µs per call over `timed` replays of graph g (`calls` calls each), after `warm`
    untimed replays: the first replays of a prefill graph run while the GPU's clocks ramp up (the
    config 4 layer measured 808, 777, 759, then ~750 µs per replay)."""
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(timed):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        stop.record()
        torch.cuda.synchronize()
        per.append(start.elapsed_time(stop) * 1e3 / calls)
    per.sort()
    return per[len(per) // 2], per


COPY_BYTES = 1 << 30
SPIN_CYCLES = 20_000_000      # torch.cuda._sleep: ~10 ms of one wave's spin at the shader clock


def host_cpu():
    """The host the CPU baseline runs on: CPU model, logical CPUs and physical cores in this process's
    affinity mask, and the x86 vector tiers candle's CPU path selects among
    (vendor/candle-core/src/quantized/repack_x86.rs: AVX512-VNNI, else AVX-VNNI, else AVX2; AMX for
    Q4_K from 32 rows). Candle's default thread count is the physical cores
    (vendor/candle-core/src/utils.rs:382-421)."""
    allowed = sorted(os.sched_getaffinity(0))
    model, flags, cores, cur = "unknown", set(), {}, {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().splitlines() + [""]:
                if not line.strip():
                    if "processor" in cur:
                        cores[int(cur["processor"])] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                cur[k] = v
                if k == "model name":
                    model = v
                elif k == "flags" and not flags:
                    flags = set(v.split())
    except OSError:
        pass
    physical = len({cores.get(c, (0, c)) for c in allowed}) or len(allowed)
    isa = [f for f in ("avx2", "fma", "avx512f", "avx512_vnni", "avx512bw", "avx_vnni", "amx_tile", "amx_int8") if f in flags]
    tier = ("avx512_vnni" if {"avx512f", "avx512_vnni"} <= flags else "avx_vnni" if "avx_vnni" in flags
            else "avx2" if "avx2" in flags else "scalar")
    return {"model": model, "logical": len(allowed), "physical": physical, "isa": isa, "tier": tier,
            "amx": {"amx_tile", "amx_int8"} <= flags}


TRAFFIC_PROFILE = "profiles/moe_c3_hbm_traffic.md"
TRAFFIC_PROFILE_C4 = "profiles/moe_c4_kernels.md"
TRAFFIC_PROFILE_C5 = "profiles/bank_c5_kernels.md"
TRAFFIC_PROFILE_DENSE = "profiles/dense_qmatmul_kernels.md"


def measured_traffic(root, profile=TRAFFIC_PROFILE):
    """HBM bytes per decode-layer launch from a committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (counters scaled by a copy kernel of known size), or None when the summary is absent."""
    try:
        with open(os.path.join(root, profile)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def copy_calibration(torch, dev):
    """A plain copy kernel of known size: 1 GiB read, 1 GiB written per launch (an elementwise add
    of zero, so it is a kernel dispatch and not a DMA copy). HBM counters read on it give the
    factor that turns the same counters read on the MoE kernels into bytes."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.add(src, 0.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "launches": 3, "bytes_read_per_launch": COPY_BYTES,
                      "bytes_written_per_launch": COPY_BYTES}), flush=True)


def time_graph(torch, layers, x_all, logits_all, warmup, steps):
    """Captures warmup and timed steps (each step a token through every layer) as two graphs;
    replays the warmup, then returns the timed graph's milliseconds."""
    L = len(layers)

    def capture(lo, hi):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for s in range(lo, hi):
                for l in range(L):
                    layers[l].forward(x_all[s], logits_all[s, l])
        return g

    for l in range(L):  # workspaces exist before capture
        layers[l].forward(x_all[0], logits_all[0, l])
    torch.cuda.synchronize()
    g_warm, g_run = capture(0, warmup), capture(warmup, warmup + steps)
    torch.cuda.synchronize()
    g_warm.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    g_run.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def bench_c5(args, torch, np, dev):
    """Config 5: MoE layers of 512 experts, top-10, hidden 2048, FFN 512, gate/up IQ3_S and down
    Q4_K, each layer's experts in a host store (pinned memory) and 56 of them in the layer's device
    bank (cw_bank). Two measurements:
      - the bank chain: 56 seeded experts per layer resident, logits N(0,1) masked to them (as the
        reference's restrict does, crates/engine/src/experts.rs:2355-2360), every pick resolved
        through the bank's table; captured in a graph and timed like config 3;
      - streaming: unmasked N(0,1) logits, and per layer route -> ids to the host -> ensure (misses
        copied over PCIe into LRU slots) -> the layer, one token at a time, as the reference's
        plain bank path does (experts.rs:1489-1641, the ids readback 2736 the sync point)."""
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth
    from coachwhip_amd.bank import Bank
    from oracle import oracle as O
    E, K, H, I, S = 512, 10, 2048, 512, 56
    dts = (F.IQ3_S, F.IQ3_S, F.Q4_K)
    shapes = [(I, H), (I, H), (H, I)]
    L = args.layers or 48
    eb = [F.matrix_bytes(d, *sh) for d, sh in zip(dts, shapes)]
    expert_bytes = sum(eb)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    log("building %d host stores of %d experts (%.1f GB pinned) and %d banks of %d slots" %
        (L, E, L * E * expert_bytes / 1e9, L, S))
    banks = []
    for l in range(L):
        host = []
        for m in range(3):
            d = synth.device_blocks(dts[m], E * shapes[m][0] * shapes[m][1], gen, dev).reshape(-1)
            h = torch.empty(d.numel(), dtype=torch.uint8, pin_memory=True)
            h.copy_(d)
            host.append(h)
            del d
        banks.append(Bank(host, dts, shapes, E, S, dev))
    torch.cuda.synchronize()
    layers = [b.moe_layer(K) for b in banks]

    # -- the bank chain: S seeded experts per layer resident, logits masked to them
    resident = [rng.choice(E, S, replace=False) for _ in range(L)]
    for l in range(L):
        assert banks[l].ensure(resident[l]) == S
    mask = torch.full((L, E), -1e30, device=dev)
    for l in range(L):
        mask[l, torch.from_numpy(resident[l]).to(dev)] = 0.0
    total = args.warmup + args.steps
    x_all = torch.randn((total, 1, H), generator=gen, device=dev)
    logits_all = torch.randn((total, L, 1, E), generator=gen, device=dev) + mask[None, :, None, :]
    torch.cuda.synchronize()
    log("parity of layer 0 against the CPU oracle")
    missing = torch.zeros(1, dtype=torch.int32, device=dev)
    out0, ids0, w0 = layers[0].forward(x_all[0], logits_all[0, 0], missing)
    host_layer = synth.MoeWeights(E, K, H, I, dts, [h.numpy() for h in banks[0].host], eb, E)
    x0, lg0 = x_all[0].cpu().numpy(), logits_all[0, 0].cpu().numpy()
    want, wids, ww, _ = O.moe_layer(host_layer, x0, lg0)
    parity = {"rel_l2": O.rel_l2(out0.cpu().numpy(), want),
              "ids_equal": bool(np.array_equal(ids0.cpu().numpy().view(np.uint32), wids)),
              "max_weight_err": float(np.max(np.abs(w0.cpu().numpy() - ww))), "missing": int(missing.cpu()[0])}
    log("parity", parity)
    log("timing the bank chain: %d steps x %d layers" % (args.steps, L))
    ms = time_graph(torch, layers, x_all, logits_all, args.warmup, args.steps)
    us_per_layer = ms * 1e3 / (args.steps * L)
    layer_bytes = K * expert_bytes + H * 4 + E * 4 + H * 4
    gbs = layer_bytes / (us_per_layer * 1e-6) / 1e9
    log("bank chain: %.2f us/layer, %.1f GB/s" % (us_per_layer, gbs))

    # -- a plain pinned host-to-device copy: what PCIe gives one DMA stream
    src = banks[0].host[2]
    dst = torch.empty(src.numel(), dtype=torch.uint8, device=dev)
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(4):
        dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    h2d_gbs = 4 * src.numel() / (time.perf_counter() - t0) / 1e9
    del dst
    log("plain pinned H2D copy: %.1f GB/s" % h2d_gbs)

    # -- streaming: unmasked routing, misses loaded per layer
    n_tok = args.stream_tokens
    xs = torch.randn((n_tok + 2, 1, H), generator=gen, device=dev)
    lgs = torch.randn((n_tok + 2, L, 1, E), generator=gen, device=dev)

    def token(t):
        for l in range(L):
            ids, _ = ops.route(lgs[t, l], K, True)
            if banks[l].ensure(ids.cpu().numpy()) is None:
                raise RuntimeError("bank refused %d picks" % K)
            layers[l].forward(xs[t], lgs[t, l], missing)

    missing.zero_()
    for t in range(2):
        token(t)
    torch.cuda.synchronize()
    before = [b.stats() for b in banks]
    t0 = time.perf_counter()
    for t in range(2, n_tok + 2):
        token(t)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    after = [b.stats() for b in banks]
    loads = sum(a["loads"] - b["loads"] for a, b in zip(after, before))
    hits = sum(a["hits"] - b["hits"] for a, b in zip(after, before))
    loaded = sum(a["bytes_loaded"] - b["bytes_loaded"] for a, b in zip(after, before))
    streaming = {"tokens": n_tok, "ms_per_token": round(wall * 1e3 / n_tok, 3),
                 "tokens_per_s": round(n_tok / wall, 2), "loads_per_token": round(loads / n_tok, 2),
                 "hit_rate": round(hits / max(hits + loads, 1), 4),
                 "loaded_gbs": round(loaded / wall / 1e9, 2), "plain_h2d_gbs": round(h2d_gbs, 2),
                 "frac_of_plain_h2d": round(loaded / wall / 1e9 / h2d_gbs, 4),
                 "missing_picks": int(missing.cpu()[0]),
                 "routing": "unmasked N(0,1) logits, fresh per token and layer (no locality: a worst case)"}
    log("streaming", streaming)

    cpu = None
    if not args.no_cpu_baseline:
        host = host_cpu()
        O.set_threads(host["physical"])
        threads = O.get_threads()
        n, t_cpu = 0, 0.0
        while t_cpu < min(args.cpu_seconds, 5.0) and n < 1000:
            lg = logits_all[n % total, 0].cpu().numpy()
            t1 = time.perf_counter()
            O.moe_layer(host_layer, x0, lg)
            t_cpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": t_cpu / n * 1e6, "unit": "us/layer", "cores": threads, "host": host, "kind": "port",
               "sample": "%d decode calls (T=1) of the C oracle MoE layer on layer 0's host store" % n}
    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded GGUF blocks generated on the device, kept in pinned host stores)",
        "config": {"workload": "config 5: bank chain, 56 of 512 experts resident per layer, b=1", "experts": E,
                   "top_k": K, "hidden": H, "expert_ffn": I, "gate_up": "iq3_s", "down": "q4_K", "layers": L,
                   "slots": S, "tokens": 1},
        "us_per_layer": round(us_per_layer, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_PROFILE_C5),
                     "traffic_source": TRAFFIC_PROFILE_C5,
                     "kernel": "MoE decode layer through the bank's slot table", "bytes_per_launch": layer_bytes},
        "streaming": streaming, "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_c4(args, torch, np, dev):
    """Config 4: gpt-oss-style MoE layers: 128 experts, top-4, hidden and expert FFN 2880, MXFP4
    gate/up/down, clamped SwiGLU (alpha 1.702, limit 7) with per-expert biases N(0, 0.02^2),
    activations N(0,1) rounded to bf16 values (passed as f32). Decode b=1 through a chain of
    --layers layers (12 by default: 20 GB of experts, so a step's 635 MB of picked experts cannot
    come from the 256 MB Infinity Cache), captured in a graph and timed like config 3; prefill:
    2,048 tokens, ten layer calls over the chain's layers captured in one graph (each call reads
    another layer's 1.69 GB of experts from HBM). The experts are generated as GGUF rows and
    repacked once, at load, into row groups of 16 (cw_repack_rows16), the library's layout for
    MXFP4 experts; --gguf-rows times the GGUF rows instead. The other layout is timed after the
    line's own (`layout_alternative`)."""
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth
    from oracle import oracle as O
    E, K, H, I, T = 128, 4, 2880, 2880, 2048
    dts = (F.MXFP4,) * 3
    shapes = [(I, H), (I, H), (H, I)]
    L = args.layers or 12
    eb = [F.matrix_bytes(d, *sh) for d, sh in zip(dts, shapes)]
    expert_bytes = sum(eb)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    log("building %d layers of %d MXFP4 experts (%.1f GB) on the device" % (L, E, L * E * expert_bytes / 1e9))
    layers, biases = [], []
    for l in range(L):
        banks = [ops.ExpertBank(synth.device_blocks(dts[m], E * shapes[m][0] * shapes[m][1], gen, dev), dts[m],
                                shapes[m][0], shapes[m][1], E, eb[m]) for m in range(3)]
        bias = [torch.randn((E, I), generator=gen, device=dev) * 0.02, torch.randn((E, I), generator=gen, device=dev) * 0.02,
                torch.randn((E, H), generator=gen, device=dev) * 0.02]
        layers.append(ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True,
                                   act=ops.ExpertAct.clamped_swiglu(1.702, 7.0, *bias)))
        biases.append(bias)
    rows16 = [ops.MoeLayer(*[b.rows16() for b in lay.banks], n_experts=E, top_k=K, norm_topk_prob=True, act=lay.act)
              for lay in layers]
    gguf = layers
    layers, alt, alt_name = (gguf, rows16, "rows16") if args.gguf_rows else (rows16, gguf, "gguf rows")
    total = args.warmup + args.steps
    x_all = torch.randn((total, 1, H), generator=gen, device=dev).to(torch.bfloat16).float()
    logits_all = torch.randn((total, L, 1, E), generator=gen, device=dev)
    torch.cuda.synchronize()

    log("parity of layer 0 against the CPU oracle")
    out0, ids0, w0 = layers[0].forward(x_all[0], logits_all[0, 0])
    host_layer = synth.MoeWeights(E, K, H, I, dts, [b.data.cpu().numpy() for b in gguf[0].banks],
                                  [b.slot_stride for b in gguf[0].banks], E, act=1,
                                  bias=[b.cpu().numpy() for b in biases[0]])
    x0, lg0 = x_all[0].cpu().numpy(), logits_all[0, 0].cpu().numpy()
    want, wids, ww, _ = O.moe_layer(host_layer, x0, lg0)
    parity = {"rel_l2": O.rel_l2(out0.cpu().numpy(), want),
              "ids_equal": bool(np.array_equal(ids0.cpu().numpy().view(np.uint32), wids)),
              "max_weight_err": float(np.max(np.abs(w0.cpu().numpy() - ww)))}
    log("parity", parity)

    log("timing the decode chain: %d steps x %d layers" % (args.steps, L))
    ms = time_graph(torch, layers, x_all, logits_all, args.warmup, args.steps)
    us_per_layer = ms * 1e3 / (args.steps * L)
    layer_bytes = K * expert_bytes + K * 3 * I * 4 + H * 4 + E * 4 + H * 4  # picked experts, their biases, x, logits, out
    gbs = layer_bytes / (us_per_layer * 1e-6) / 1e9
    log("decode: %.2f us/layer, %.1f GB/s" % (us_per_layer, gbs))

    xp = torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16).float()
    lp = torch.randn((T, E), generator=gen, device=dev)
    eager = [layers[l].forward(xp, lp)[0].clone() for l in range(min(L, 2))]
    torch.cuda.synchronize()
    reps = 10
    g_pre = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_pre):
        pre_outs = [layers[r % L].forward(xp, lp)[0] for r in range(reps)]
    torch.cuda.synchronize()
    pre_us, pre_all = time_replays(torch, g_pre, reps)
    pre_same = all(bool(torch.equal(pre_outs[r], eager[r % L])) for r in range(reps) if r % L < len(eager))
    pre_flops = 2.0 * T * K * 3 * H * I
    tflops = pre_flops / (pre_us * 1e-6) / 1e12
    # every expert is picked at 2,048 tokens: the layer reads all its experts once
    pre_bytes = E * expert_bytes + 3 * E * I * 4 + T * H * 4 + T * E * 4 + T * H * 4
    prefill = {"tokens": T, "us_per_layer": round(pre_us, 2), "tokens_per_s": round(T / (pre_us * 1e-6)),
               "tflops": round(tflops, 2), "mfma_util": round(tflops / MFMA_PEAK_F16_TFLOPS, 4),
               "mfma_peak_tflops": MFMA_PEAK_F16_TFLOPS, "hbm_gbs": round(pre_bytes / (pre_us * 1e-6) / 1e9, 1),
               "hbm_frac": round(pre_bytes / (pre_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "graph_replay_equals_eager": pre_same, "calls_timed": reps,
               "timing": "median of 5 graph replays after 3 warm-up replays",
               "us_per_layer_replays": [round(v, 1) for v in pre_all],
               # the scaled MFMA runs three FP4 x FP6 products (one per activation term) per product
               # of the layer: issued work against the dense FP6/FP4 peak
               "mfma_issued_tflops": round(3 * tflops, 2), "mfma_peak_f6f4_tflops": MFMA_PEAK_F6F4_TFLOPS,
               "mfma_util_f6f4": round(3 * tflops / MFMA_PEAK_F6F4_TFLOPS, 4),
               "path": ("grouped GEMMs on the block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4): MXFP4 weights "
                        "as stored, activations as three FP6 E2M3 terms with E8M0 scales per 32, f32 accumulate")}
    log("prefill", prefill)

    # the same experts in the other layout: prefill outputs bit-equal (the same blocks in the same
    # order); the one-token layer with gate/up in row groups sums in its own order (K-split), so its
    # distance from the oracle is given instead
    other = None
    if not args.no_alternative:
        log("the other layout (%s)" % alt_name)
        same = all(bool(torch.equal(alt[l].forward(xp, lp)[0], eager[l])) for l in range(len(eager)))
        d_alt = alt[0].forward(x_all[0], logits_all[0, 0])[0]
        g_alt = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_alt):
            for r in range(reps):
                alt[r % L].forward(xp, lp)
        torch.cuda.synchronize()
        pre_alt, pre_alt_all = time_replays(torch, g_alt, reps)
        del g_alt
        ms_alt = time_graph(torch, alt, x_all, logits_all, args.warmup, args.steps)
        dec_alt = ms_alt * 1e3 / (args.steps * L)
        other = {"layout": alt_name, "prefill_us_per_layer": round(pre_alt, 2),
                 "prefill_tokens_per_s": round(T / (pre_alt * 1e-6)),
                 "prefill_us_per_layer_replays": [round(v, 1) for v in pre_alt_all],
                 "decode_us_per_layer": round(dec_alt, 3), "decode_gbs": round(layer_bytes / (dec_alt * 1e-6) / 1e9, 2),
                 "prefill_outputs_equal": same, "decode_rel_l2": O.rel_l2(d_alt.cpu().numpy(), want)}
        log("other layout", other)
    del alt
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        host = host_cpu()
        O.set_threads(host["physical"])
        threads = O.get_threads()
        # candle's own CPU path for this layer: per picked expert, QMatMul with x quantized to Q8_0
        # (MXFP4 x Q8_0 vec-dot), clamped SwiGLU with biases, down QMatMul, weighted index-add in
        # expert order (experts.rs:2500-2537, k_quants.rs:738-759, 2551-2670)
        n, t_cpu, dev_l2 = 0, 0.0, 0.0
        while t_cpu < args.cpu_seconds and n < 1000:
            lg = logits_all[n % total, 0].cpu().numpy()
            t1 = time.perf_counter()
            got_c, _, _ = O.candle_moe_layer(host_layer, x0, lg, threads)
            t_cpu += time.perf_counter() - t1
            if n < 4:
                dev_l2 = max(dev_l2, O.rel_l2(got_c, O.moe_layer(host_layer, x0, lg)[0]))
            n += 1
        n_f64, t_f64 = 0, 0.0
        while t_f64 < min(args.cpu_seconds, 5.0) and n_f64 < 1000:
            lg = logits_all[n_f64 % total, 0].cpu().numpy()
            t1 = time.perf_counter()
            O.moe_layer(host_layer, x0, lg)
            t_f64 += time.perf_counter() - t1
            n_f64 += 1
        cpu = {"value": t_cpu / n * 1e6, "unit": "us/layer", "cores": threads, "host": host, "kind": "port",
               "sample": "%d decode calls (T=1) of candle's MXFP4 CPU MoE path on layer 0: route, then per picked "
                         "expert gate/up/down QMatMuls with x quantized to Q8_0 (MXFP4 x Q8_0 vec-dot), "
                         "clamped SwiGLU with biases and the weighted index-add in expert order" % n,
               "candle_rel_l2_vs_f64": dev_l2,
               "f64_oracle_us_per_layer": t_f64 / n_f64 * 1e6}
        log("cpu", cpu)
    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded MXFP4 blocks, biases and bf16-valued N(0,1) activations, generated on the device)",
        "config": {"workload": "config 4 decode: gpt-oss-style MoE layer chain, b=1", "experts": E, "top_k": K,
                   "hidden": H, "expert_ffn": I, "weights": "mxfp4", "act": "clamped swiglu", "layers": L, "tokens": 1,
                   "expert_layout": "gguf rows" if args.gguf_rows else "rows in groups of 16 (repacked at load)"},
        "us_per_layer": round(us_per_layer, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_PROFILE_C4),
                     "traffic_source": TRAFFIC_PROFILE_C4,
                     "kernel": "MoE decode layer (MXFP4%s, clamped SwiGLU)" % ("" if args.gguf_rows else " in row groups of 16"),
                     "bytes_per_launch": layer_bytes},
        "prefill": prefill, "layout_alternative": other, "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_dense(args, torch, np, dev):
    """Configs 1 and 2: one quantized matrix, y = x . W^T (QMatMul): Q8_0 2048 x 2048 at M = 1, and
    Q4_K 4096 x 4096 at M in {1, 16, 128, 512}. Each case captures one call per copy of the matrix
    (copies past ~600 MB, so the Infinity Cache cannot serve them) in a graph and times its replay
    behind a bounded GPU spin, so the calls run back to back on the device (us); us_host_fed is the
    same replay started on an idle device, where a call of a few µs waits for the host to submit
    the next one. Achieved rates use the algorithmic bytes (matrix + x + y) and flops (2 M n k), against HBM
    (8 TB/s) or fp16 MFMA (2.5 PFLOP/s), whichever bounds the case. Parity of each case against
    the f64 oracle; the CPU baseline is the restatement of candle's x86 QMatMul (the repacked
    AVX-512 VNNI tiles of repack_x86.rs where candle takes them, else the generic vec_dot driver)
    on the host's physical cores."""
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth
    from oracle import oracle as O
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    host = host_cpu()
    O.set_threads(host["physical"])
    threads = O.get_threads()
    cases, packs = [], {}
    for name, dt, n, k, ms in (("config 1: Q8_0 GEMV", F.Q8_0, 2048, 2048, (1,)),
                               ("config 2: Q4_K matmul", F.Q4_K, 4096, 4096, (1, 16, 128, 512))):
        wb = F.matrix_bytes(dt, n, k)
        copies = max(8, -(-600_000_000 // wb))
        mats = [ops.QMatMul(ops.QTensor(synth.device_blocks(dt, n * k, gen, dev), dt, (n, k))) for _ in range(copies)]
        host_w = mats[0].w.data.cpu().numpy()
        for m in ms:
            x = torch.randn((m, k), generator=gen, device=dev)
            y0 = mats[0].forward(x)
            torch.cuda.synchronize()
            xh = x.cpu().numpy()
            err = O.rel_l2(y0.cpu().numpy(), O.qmatmul_f64(dt, host_w, n, k, xh))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for c in range(copies):
                    mats[c].forward(x)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            g.replay()
            stop.record()
            torch.cuda.synchronize()
            us_fed = start.elapsed_time(stop) * 1e3 / copies
            # A call of a few µs finishes before the host has submitted the next node of the
            # replayed graph, so the replay above measures the host's submission rate. Timed
            # again behind a bounded GPU spin that outlasts the submission, the calls run back to
            # back and the events measure the device.
            spin0 = torch.cuda.Event(enable_timing=True)
            spin0.record()
            torch.cuda._sleep(SPIN_CYCLES)
            start.record()
            t_host = time.perf_counter()
            g.replay()
            t_host = time.perf_counter() - t_host
            stop.record()
            torch.cuda.synchronize()
            us = start.elapsed_time(stop) * 1e3 / copies
            spin_us = spin0.elapsed_time(start) * 1e3
            if t_host * 1e6 >= spin_us:
                log("warning: the graph's submission (%.0f us) outlasted the spin (%.0f us)" % (t_host * 1e6, spin_us))
            nbytes = wb + 4 * m * k + 4 * m * n
            flops = 2.0 * m * n * k
            t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_PEAK_F16_TFLOPS * 1e12)
            bound = "hbm" if t_hbm >= t_mfma else "mfma"
            case = {"case": name, "m": m, "n": n, "k": k, "us": round(us, 3),
                    "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                    "bound": bound, "roofline_frac": round(max(t_hbm, t_mfma) / (us * 1e-6), 4), "rel_l2": err,
                    "us_host_fed": round(us_fed, 3)}
            if not args.no_cpu_baseline:
                # candle's CPU QMatMul on this host: the repacked x86 tiles where it takes them
                # (weights packed once, as candle caches them), else the generic vec_dot driver
                if O.x86_select(dt, m, n, k):
                    if dt not in packs:
                        packs[dt] = O.x86_pack(dt, host_w, n, k)
                    run = lambda: O.x86_matmul(dt, packs[dt], n, k, xh)  # noqa: E731
                    case["cpu_path"] = "x86 tiles, tier %d" % O.x86_level()
                else:
                    run = lambda: O.candle_matmul(dt, host_w, n, k, xh)  # noqa: E731
                    case["cpu_path"] = "generic vec_dot"
                yc = run()
                case["cpu_rel_l2"] = O.rel_l2(yc, O.qmatmul_f64(dt, host_w, n, k, xh))
                reps, t_cpu = 0, 0.0
                while t_cpu < 2.0 and reps < 200:
                    t1 = time.perf_counter()
                    run()
                    t_cpu += time.perf_counter() - t1
                    reps += 1
                case["cpu_us"] = round(t_cpu / reps * 1e6, 1)
            log(case)
            cases.append(case)
        del mats
        torch.cuda.empty_cache()
    head = cases[0]
    line = {
        "metric": METRIC, "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": head["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded Q8_0 / Q4_K blocks generated on the device, x ~ N(0,1))",
        "config": {"workload": "configs 1 and 2: dense QMatMul (Q8_0 2048x2048 M=1; Q4_K 4096x4096 M=1,16,128,512)"},
        "roofline": {"bound": head["bound"], "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["roofline_frac"],
                     "traffic": measured_traffic(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_PROFILE_DENSE),
                     "traffic_source": TRAFFIC_PROFILE_DENSE, "kernel": "QMatMul, config 1"},
        "cases": cases,
        "cpu_baseline": None if args.no_cpu_baseline else {
            "value": head["cpu_us"], "unit": "us per call (config 1)", "cores": threads, "host": host, "kind": "port",
            "sample": "candle's CPU QMatMul restated (repack_x86.rs: weights in 16-row tiles packed once, "
                      "activations to Q8_K, AVX-512 VNNI units over the physical cores; the generic vec_dot "
                      "driver where candle does not take the tiles), ~2 s per case; cpu_us, cpu_path and "
                      "cpu_rel_l2 (against the f64 product) in each case"},
    }
    print(json.dumps(line), flush=True)


def bench_shrink(args, torch, np, dev):
    """The GPU shrink (cw_requant_q2k) on experts of config 5's shape with the reference's model-file
    formats (gate/up Q3_K 512 x 2048, down Q5_K 2048 x 512, crates/engine/tests/gpu_shrink.rs):
    one launch per matrix over 64 experts at once (throughput), and the three launches of a single
    expert (the latency a bank miss sees). HBM roofline on source + output bytes."""
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth
    from oracle import oracle as O
    H, I, n_exp = 2048, 512, 64
    mats = [(F.Q3_K, I, H), (F.Q3_K, I, H), (F.Q5_K, H, I)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    srcs, outs, nbs = [], [], []
    for dt, r, c in mats:
        nb = n_exp * r * c // 256
        srcs.append(synth.device_blocks(dt, nb * 256, gen, dev))
        outs.append(torch.empty(nb * 84, dtype=torch.uint8, device=dev))
        nbs.append(nb)
    in_bytes = sum(nb * F.type_size(dt) for nb, (dt, _, _) in zip(nbs, mats))
    out_bytes = sum(nb * 84 for nb in nbs)
    log("parity of the first 4096 blocks of each matrix against the oracle")
    parity = True
    for (dt, _, _), src, out in zip(mats, srcs, outs):
        ops.requant_q2k(dt, src, 4096, out=out)
        parity &= bool(np.array_equal(out[:4096 * 84].cpu().numpy(), O.requant_q2k(dt, src[:4096 * F.type_size(dt)].cpu().numpy(), 4096)))
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def run_all(reps):
        start.record()
        for _ in range(reps):
            for (dt, _, _), src, out, nb in zip(mats, srcs, outs, nbs):
                ops.requant_q2k(dt, src, nb, out=out)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / reps

    run_all(args.warmup)
    ms = run_all(args.steps)
    gbs = (in_bytes + out_bytes) / (ms * 1e-3) / 1e9
    one = [nb // n_exp for nb in nbs]

    def run_one(reps):
        start.record()
        for _ in range(reps):
            for (dt, _, _), src, out, nb in zip(mats, srcs, outs, one):
                ops.requant_q2k(dt, src, nb, out=out)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / reps

    run_one(args.warmup)
    one_us = run_one(args.steps) * 1e3
    log("shrink: %d experts in %.3f ms (%.1f GB/s); one expert %.1f us" % (n_exp, ms, gbs, one_us))
    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded Q3_K / Q5_K blocks generated on the device)",
        "config": {"workload": "GPU shrink to Q2_K: %d config-5 experts (gate/up Q3_K %dx%d, down Q5_K %dx%d)"
                               % (n_exp, I, H, H, I), "blocks": sum(nbs)},
        "us_per_expert_alone": round(one_us, 2), "us_per_expert_batched": round(ms * 1e3 / n_exp, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_requant_q2k",
                     "bytes_per_step": in_bytes + out_bytes},
        "parity": {"bytes_equal_oracle": parity}, "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        host = host_cpu()
        O.set_threads(host["physical"])
        threads = O.get_threads()
        src0 = srcs[2][:nbs[2] // n_exp * F.type_size(F.Q5_K)].cpu().numpy()
        n, t_cpu = 0, 0.0
        while t_cpu < min(args.cpu_seconds, 5.0) and n < 200:
            t1 = time.perf_counter()
            O.requant_q2k(F.Q5_K, src0, nbs[2] // n_exp)
            t_cpu += time.perf_counter() - t1
            n += 1
        line["cpu_baseline"] = {"value": t_cpu / n * 1e6, "unit": "us per Q5_K 2048x512 matrix", "cores": threads, "host": host,
                                "kind": "port", "sample": "%d shrinks of one down matrix by the C oracle" % n}
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=None, help="layers per step (40 for config 3, 48 for config 5)")
    ap.add_argument("--workload", choices=("c3", "c4", "c5", "shrink", "dense"), default="c3",
                    help="c3: the headline decode chain; c4: the gpt-oss-style MXFP4 chain and its 2,048-token "
                         "prefill; c5: the bank chain (56 of 512 slots) and streaming; dense: configs 1-2 QMatMul; "
                         "shrink: the GPU shrink to Q2_K of config-5-shaped experts")
    ap.add_argument("--stream-tokens", type=int, default=16, help="config 5: tokens of the streaming run")
    ap.add_argument("--prefill-tokens", type=int, default=1500)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--gguf-rows", action="store_true", help="c4: time the experts as GGUF rows (default: row groups of 16)")
    ap.add_argument("--no-alternative", action="store_true", help="c4: skip timing the other expert layout")
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (for scaling HBM counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (experts would shard across GPUs "
              "by expert id with one all-reduce per decode layer; not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    import coachwhip_amd as cw
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth

    cw.lib()  # fails loudly when the HIP library is not built
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(torch, dev)
        return
    if args.workload == "c4":
        bench_c4(args, torch, np, dev)
        return
    if args.workload == "dense":
        bench_dense(args, torch, np, dev)
        return
    if args.workload == "c5":
        bench_c5(args, torch, np, dev)
        return
    if args.workload == "shrink":
        bench_shrink(args, torch, np, dev)
        return
    E, K, H, I = 256, 8, 2048, 512
    dts = (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S)
    L = args.layers or 40
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    log("building %d layers of %d experts on the device" % (L, E))
    shapes = [(I, H), (I, H), (H, I)]
    layers = []
    for l in range(L):
        banks = []
        for m in range(3):
            n, k = shapes[m]
            raw = synth.device_blocks(dts[m], E * n * k, gen, dev)
            banks.append(ops.ExpertBank(raw, dts[m], n, k, E, F.matrix_bytes(dts[m], n, k)))
        layers.append(ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True))
    expert_bytes = sum(F.matrix_bytes(dts[m], *shapes[m]) for m in range(3))
    total_steps = args.warmup + args.steps
    x_all = torch.randn((total_steps, 1, H), generator=gen, device=dev)
    logits_all = torch.randn((total_steps, L, 1, E), generator=gen, device=dev)
    torch.cuda.synchronize()

    # parity of layer 0, step 0 against the CPU oracle (picked experts only travel to the host)
    log("parity check against the CPU oracle")
    from oracle import oracle as O
    out0, ids0, w0 = layers[0].forward(x_all[0], logits_all[0, 0])
    torch.cuda.synchronize()
    host_layer = synth.MoeWeights(E, K, H, I, dts, [b.data.cpu().numpy() for b in layers[0].banks],
                                  [b.slot_stride for b in layers[0].banks], E)
    x0 = x_all[0].cpu().numpy()
    lg0 = logits_all[0, 0].cpu().numpy()
    want, wids, ww, _ = O.moe_layer(host_layer, x0, lg0)
    parity = {"rel_l2": O.rel_l2(out0.cpu().numpy(), want),
              "ids_equal": bool(np.array_equal(ids0.cpu().numpy().view(np.uint32), wids)),
              "max_weight_err": float(np.max(np.abs(w0.cpu().numpy() - ww)))}
    log("parity", parity)

    # one graph per phase: warmup steps, then the timed steps; each step is L layer calls
    def capture(step_lo, step_hi):
        g = torch.cuda.CUDAGraph()
        outs = []
        with torch.cuda.graph(g):
            for s in range(step_lo, step_hi):
                for l in range(L):
                    outs.append(layers[l].forward(x_all[s], logits_all[s, l])[0])
        return g, outs

    for l in range(L):  # workspaces exist before capture
        layers[l].forward(x_all[0], logits_all[0, l])
    torch.cuda.synchronize()
    log("capturing graphs")
    g_warm, _ = capture(0, args.warmup)
    g_run, _ = capture(args.warmup, total_steps)
    torch.cuda.synchronize()
    g_warm.replay()
    torch.cuda.synchronize()

    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log("timing %d steps x %d layers" % (args.steps, L))
    t0 = time.perf_counter()
    torch.cuda.synchronize()
    start.record()
    g_run.replay()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop)
    us_per_layer = ms * 1e3 / (args.steps * L)

    # algorithmic bytes of one decode layer: the K distinct picked experts' blocks + x, logits, out
    layer_bytes = K * expert_bytes + H * 4 + E * 4 + H * 4
    gbs = layer_bytes / (us_per_layer * 1e-6) / 1e9
    log("decode: %.2f us/layer, %.1f GB/s (wall %.3f s)" % (us_per_layer, gbs, wall))

    # prefill: one layer, T tokens (the reference reads prompts in pieces; this is one piece).
    # reps calls are captured in one graph, so the time is the GPU's and not the host's launch
    # overhead; the replay's output is checked against an eager call.
    T = args.prefill_tokens
    xp = torch.randn((T, H), generator=gen, device=dev)
    lp = torch.randn((T, E), generator=gen, device=dev)
    # the calls rotate over ROT layers (ROT x 224 MB of experts, past the 256 MB Infinity Cache), so
    # each call reads its experts from HBM
    ROT = min(3, L)
    eager = [layers[1 + r % (L - 1) if L > 1 else 0].forward(xp, lp)[0].clone() for r in range(ROT)]
    torch.cuda.synchronize()
    reps = 12
    g_pre = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_pre):
        pre_outs = [layers[1 + (r % ROT) % (L - 1) if L > 1 else 0].forward(xp, lp)[0] for r in range(reps)]
    torch.cuda.synchronize()
    pre_us, pre_all = time_replays(torch, g_pre, reps)
    pre_same = all(bool(torch.equal(o, eager[r % ROT])) for r, o in enumerate(pre_outs))
    pre_flops = 2.0 * T * K * 3 * H * I
    tflops = pre_flops / (pre_us * 1e-6) / 1e12
    prefill = {"tokens": T, "us_per_layer": round(pre_us, 2), "tokens_per_s": round(T / (pre_us * 1e-6)),
               "tflops": round(tflops, 2), "mfma_util": round(tflops / MFMA_PEAK_F16_TFLOPS, 4),
               "mfma_peak_tflops": MFMA_PEAK_F16_TFLOPS, "graph_replay_equals_eager": pre_same, "calls_timed": reps,
               "timing": "median of 5 graph replays after 3 warm-up replays",
               "us_per_layer_replays": [round(v, 1) for v in pre_all], "layers_rotated": ROT,
               "path": "grouped MFMA GEMMs (fp16 integer weight codes, fp16 activations, f32 accumulate)"}
    log("prefill", prefill)

    cpu = None
    if not args.no_cpu_baseline:
        host = host_cpu()
        O.set_threads(host["physical"])
        threads = O.get_threads()
        log("cpu baseline: oracle MoE layer, %d threads, ~%.0f s" % (threads, args.cpu_seconds))
        rng = np.random.default_rng(args.seed)
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds and n < 1000:
            lg = rng.standard_normal((1, E)).astype(np.float32)
            t1 = time.perf_counter()
            O.moe_layer(host_layer, x0, lg)
            t_cpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": t_cpu / n * 1e6, "unit": "us/layer", "cores": threads, "host": host, "kind": "port",
               "sample": "%d decode calls (T=1) of the C oracle MoE layer (dequantize the picked experts, f64 dots) "
                         "on layer 0 of the same bank; IQ formats have no candle CPU path" % n}
        log("cpu", cpu)

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded GGUF blocks and N(0,1) activations/logits, generated on the device)",
        "config": {"workload": "config 3 decode: MoE layer chain, b=1", "experts": E, "top_k": K, "hidden": H,
                   "expert_ffn": I, "gate_up": "iq2_xxs", "down": "iq2_s", "layers": L, "tokens": 1},
        "us_per_layer": round(us_per_layer, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(root),
                     "traffic_source": TRAFFIC_PROFILE,
                     "kernel": "MoE decode layer (route + fused gate/up+SwiGLU + fused down+combine)",
                     "bytes_per_launch": layer_bytes},
        "prefill": prefill,
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
