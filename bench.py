"""Benchmark of the FP8-blockwise MoE layer on one MI355X.

Workload (the `value` line): DeepSeek-V3 MoE layer at decode, 64 tokens,
hidden 7168, moe_intermediate 2048, 256 routed experts + 1 shared, sigmoid
grouped top-8 (8 groups, 4 kept), correction bias, renorm, x2.5. Weights are
synthetic (seeded N(0, 0.02) quantized to e4m3fn with 128x128 block scales),
generated on the GPU; inputs are resident in HBM before timing starts.

Phases:
  A  K steps of the whole layer through the C-ABI entry moe_layer_forward
     (router -> top-k -> align -> act quant -> gate_up -> down -> combine);
     `value` = 64 * K / elapsed.
  B  K steps of the same kernels launched one by one, with HIP events around the
     two expert GEMMs on the launch stream, for the per-kernel roofline.
  C  the same layer at prefill (8192 tokens), reported under "prefill8k".
  D  the CPU oracle on a bounded token sample (rank 0, N = 1 only): median of 3
     timed runs after one warm-up.
  E  (unless --no-extra) the other workloads, under "extra", each the median of three
     timed loops (its "timing" field): the small layer
     (64 tokens, hidden 1024, 8 experts, top-2), Kimi-K2 over 1..16384 tokens
     (1 token also with 32 inputs cycled so the weights do not stay in the 256 MB
     MALL), GLM-4.5 with Zipf-skewed routing, and the GPT-OSS-120B layer with
     MXFP4 experts (up to 64 tokens also "graph_ms_per_step": the same call replayed
     from a HIP graph, timed on the GPU's clock without the host's launch cost, and
     "flushed_ms_per_step": each call after a 1 GiB fill that evicts the weights from
     L2 and the MALL, timed with HIP events); and under
     "cpu_extra" the oracle timed on the small layer in the reference's dense
     all-experts form and on token samples of each layer.
Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "vllm-neuron_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense OCP-fp8 MFMA
METRIC = "MoE layer tokens/s + % HBM/fp8-MFMA roofline, DSV3 shape decode64/prefill8k"


def expert_bytes(H, I, part):
    """Algorithmic weight bytes of one expert for the gate_up or down GEMM
    (fp8 codes + fp32 128x128 block scales)."""
    if part == "gate_up":
        return 2 * I * H + 4 * (2 * I // 128) * (H // 128)
    return H * I + 4 * (H // 128) * (I // 128)


TRAFFIC_FILE = os.path.join(REPO, "profiles", "expert_gemm_dsv3_hbm_traffic_pmc.md")


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed counter
    summary (rocprofv3 FETCH_SIZE and WRITE_SIZE passes, each scaled by its
    calibration factor against a plain copy kernel); None when absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if not line.startswith("traffic:"):
                    continue
                kv = dict(t.split("=", 1) for t in line.split()[1:])
                if kv.get("kernel") == kernel and kv.get("workload") == workload:
                    return int((float(kv["fetch_kib"]) * float(kv["fetch_factor"])
                                + float(kv["write_kib"]) * float(kv["write_factor"])) * 1024)
    except (OSError, ValueError, KeyError):
        return None
    return None


def layer_counts(ids, E):
    import torch
    counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
    return int((counts > 0).sum().item()), int(counts.sum().item())


def run_phase_b(x, w, cfg, steps, torch, ops):
    """Op-by-op pipeline; events around gate_up and down on the launch stream."""
    T = x.shape[0]
    E, K, B, S = cfg.n_experts, cfg.top_k, cfg.block_size, w.n_shared
    mt = ops.choose_mt(T, K, E)
    block = ops.use_block_kernels(T, K, E)
    st = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    ids = None
    for i in range(steps):
        lg = ops.router_logits(x, w.router_w, w.router_bias)
        ids, wts = ops.router_topk(lg, K, ops.ORDER_GROUPED, cfg.scoring, cfg.n_group, cfg.topk_group,
                                   w.corr_bias, cfg.renorm, 1e-20, cfg.routed_scaling)
        m = ops.blockwise_mapping(ids=ids, n_experts=E, block_size=B)
        xq, xs = ops.act_quant(x)
        NB = m["token_position_to_id"].numel()
        tpid = m["token_position_to_id"]
        if block:
            tiles, num, mx = ops.build_block_tiles(tpid, m["block_to_expert"], B, T, K, E, S)
        else:
            tiles, num, mx = ops.build_tiles(tpid, m["block_to_expert"], B, T, K, E, S, mt)
        ev[i][0].record(st)
        if block:
            hq, hs = ops.expert_gate_up_block(xq, xs, w, tpid, NB, tiles, num, mx)
        else:
            hq, hs = ops.expert_gate_up(xq, xs, w, tpid, NB, tiles, num, mx, mt)
        ev[i][1].record(st)
        ev[i][2].record(st)
        if block:
            y = ops.expert_down_block(hq, hs, w, T, NB, tiles, num, mx)
        else:
            y = ops.expert_down(hq, hs, w, T, NB, tiles, num, mx, mt)
        ev[i][3].record(st)
        ops.combine(y, m["inv_pos"], wts, T, cfg.hidden, NB, S)
    torch.cuda.synchronize()
    gu = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    dn = sum(e[2].elapsed_time(e[3]) for e in ev) / steps
    return gu, dn, ids


def time_layer(x, w, cfg, steps, warmup, torch, ops, loops=1):
    """Seconds per layer call: the mean over `steps` calls, or with loops > 1 the
    median of that many timed loops (one stall then moves one loop, not the figure)."""
    for _ in range(warmup):
        ops.layer_forward(x, w, cfg)
    runs = []
    for _ in range(loops):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            ops.layer_forward(x, w, cfg)
        torch.cuda.synchronize()
        runs.append((time.perf_counter() - t0) / steps)
    return sorted(runs)[len(runs) // 2]


def graph_ms(fn, reps, torch):
    """Device time per call of fn replayed from a HIP graph: two warm-up calls on a
    side stream, one capture, then `reps` replays queued behind a short spin kernel
    (so the host's launch cost stays off the GPU's timeline) and timed with HIP
    events on the replay stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(20_000_000)  # ~10 ms of GPU spin while the replays are queued
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del g
    torch.cuda.empty_cache()
    return round(ms, 4)


def flushed_ms(fn, steps, torch):
    """Device time per call of fn with the caches cold: before each call a read of
    1 GiB evicts the weights from L2 and the 256 MB MALL (as the other layers' weights,
    which a decode step reads in between, would; a read leaves no dirty lines whose
    write-back would overlap the call), then a short spin kernel lets the host queue
    the call, which HIP events on the launch stream bracket. Median over `steps` calls."""
    buf = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    fn()
    torch.cuda.synchronize()
    ev = []
    for i in range(steps):
        buf.amax()
        torch.cuda._sleep(400_000)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        ev.append((e0, e1))
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in ev)
    del buf
    torch.cuda.empty_cache()
    return round(ts[len(ts) // 2], 4)


def small_loop(T, steps):
    """Calls per timed loop of an extra workload. Up to 64 tokens a call takes tens of
    microseconds to about a millisecond, and the first launch after the synchronize
    exposes the queue's whole latency: 100 calls or more, so that start is spread thin
    (with 10 it added about a microsecond per one-token call)."""
    return max(steps * 5, 100) if T <= 64 else max(steps // 2, 5)


def workload_report(name, x, w, cfg, steps, torch, ops):
    """Whole-layer timing of one extra workload with its algorithmic roofline (and, up to
    64 tokens, the device time of the same call replayed from a HIP graph)."""
    T = x.shape[0]
    H, I, E = cfg.hidden, cfg.intermediate, cfg.n_experts
    loop = small_loop(T, steps)
    sec = time_layer(x, w, cfg, loop, 2, torch, ops, loops=3)
    gms = graph_ms(lambda: ops.layer_forward(x, w, cfg), max(steps, 20), torch) if T <= 64 else None
    fms = flushed_ms(lambda: ops.layer_forward(x, w, cfg), max(steps, 20), torch) if T <= 64 else None
    ids = ops.layer_forward(x, w, cfg, return_routing=True)[1]
    active, rows = layer_counts(ids, E)
    flops = 2 * (rows + T * cfg.n_shared) * 3 * H * I + 2 * T * H * E
    nbytes = ((active + cfg.n_shared) * (expert_bytes(H, I, "gate_up") + expert_bytes(H, I, "down"))
              + E * H * 2 + T * H * 2 * 2)
    rep = {"workload": name, "tokens": T, "ms_per_step": round(sec * 1e3, 4),
           "timing": f"median of 3 loops of {loop} calls after 2 warm-up calls",
           "tokens_per_s": round(T / sec, 1), "active_experts": active,
           "alg_bytes": nbytes, "alg_flops": flops,
           "hbm_frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
           "mfma_frac": round(flops / sec / 1e12 / FP8_PEAK_TFLOPS, 4),
           "roofline_frac": round(max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (FP8_PEAK_TFLOPS * 1e12)) / sec, 4)}
    if gms is not None:
        rep["graph_ms_per_step"] = gms
        rep["graph_hbm_frac"] = round(nbytes / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if fms is not None:
        rep["flushed_ms_per_step"] = fms
        rep["flushed_hbm_frac"] = round(nbytes / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    return rep


def run_prologue(calls, torch, ops, dev, H=7168):
    """Residual add + RMSNorm + 1x128 quantization, fused (moe_rms_norm_quant) and as
    separate launches (bf16 add, moe_rms_norm, moe_act_quant_1x128), for a kernel trace."""
    g = torch.Generator().manual_seed(7)
    for T in (64, 8192):
        print(f"[bench] prologue T={T}", file=sys.stderr, flush=True)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        r = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(dev)
        for _ in range(calls):
            ops.rms_norm_quant(x, gamma, 1e-6, None, r)
            ops.act_quant(ops.rms_norm(x + r, gamma, 1e-6))
        torch.cuda.synchronize()


def rotated_report(name, xs, w, cfg, torch, ops, rounds=3):
    """Whole-layer timing cycling through the inputs xs (different tokens route to
    different experts, so the weights of one step are not cache-resident in the next)."""
    T = xs[0].shape[0]
    H, I, E = cfg.hidden, cfg.intermediate, cfg.n_experts
    for x in xs[:4]:
        ops.layer_forward(x, w, cfg)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(rounds):
        for x in xs:
            ops.layer_forward(x, w, cfg)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / (rounds * len(xs))
    act = []
    for x in xs:
        ids = ops.layer_forward(x, w, cfg, return_routing=True)[1]
        act.append(layer_counts(ids, E))
    active = sum(a for a, _ in act) / len(act)
    rows = sum(r for _, r in act) / len(act)
    nbytes = ((active + cfg.n_shared) * (expert_bytes(H, I, "gate_up") + expert_bytes(H, I, "down"))
              + E * H * 2 + T * H * 2 * 2)
    flops = 2 * (rows + T * cfg.n_shared) * 3 * H * I + 2 * T * H * E
    return {"workload": name, "tokens": T, "inputs_cycled": len(xs),
            "ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(T / sec, 1),
            "active_experts": active, "alg_bytes": int(nbytes), "alg_flops": int(flops),
            "hbm_frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
            "roofline_frac": round(max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (FP8_PEAK_TFLOPS * 1e12)) / sec, 4)}


def mx_report(name, layer, x, steps, torch):
    """Whole-layer timing of the GPT-OSS MXFP4 layer (module forward, decode form)."""
    w = layer.w
    T, H = x.shape
    E, I, hr = w.n_experts, w.intermediate, layer.hidden_actual or H
    for _ in range(2):
        layer(x, None, True, None)
    loop, runs = small_loop(T, steps), []
    for _ in range(3):  # median of three timed loops
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(loop):
            layer(x, None, True, None)
        torch.cuda.synchronize()
        runs.append((time.perf_counter() - t0) / loop)
    sec = sorted(runs)[1]
    gms = graph_ms(lambda: layer(x, None, True, None), max(steps, 20), torch) if T <= 64 else None
    fms = flushed_ms(lambda: layer(x, None, True, None), max(steps, 20), torch) if T <= 64 else None
    from vllm_neuron_amd import ops
    ids = ops.layer_forward_mx(x, w, layer.top_k, layer.act, layer.limits[:2], layer.limits[2:],
                               return_routing=True, gamma=layer.norm_weight, eps=layer.rms_norm_eps,
                               hidden_actual=layer.hidden_actual)[1]
    active, rows = layer_counts(ids, E)
    # per expert: fp4 codes (half a byte per weight), one E8M0 byte per 32 weights, fp32 biases
    per_expert = 3 * H * I // 2 + 3 * H * I // 32 + 4 * (2 * I + H)
    nbytes = active * per_expert + E * H * 2 + T * H * 2 * 2
    flops = 2 * rows * 3 * hr * hr + 2 * T * H * E
    rep = {"workload": name, "tokens": T, "ms_per_step": round(sec * 1e3, 4),
           "timing": f"median of 3 loops of {loop} calls after 2 warm-up calls",
           "tokens_per_s": round(T / sec, 1), "active_experts": active,
           "alg_bytes": nbytes, "alg_flops": flops,
           "hbm_frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
           "roofline_frac": round(max(nbytes / (HBM_PEAK_GBS * 1e9),
                                      flops / (FP8_PEAK_TFLOPS * 1e12)) / sec, 4)}
    if gms is not None:
        rep["graph_ms_per_step"] = gms
        rep["graph_hbm_frac"] = round(nbytes / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if fms is not None:
        rep["flushed_ms_per_step"] = fms
        rep["flushed_hbm_frac"] = round(nbytes / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    return rep


def extra_workloads(steps, torch, ops, synthetic, PRESETS, dev, cpu_tokens):
    """The small layer, Kimi-K2 over its token sweep, GLM-4.5 with Zipf-skewed
    routing and GPT-OSS-120B with MXFP4 experts on the GPU; the oracle on token
    samples of each (and the small layer in the dense form) on the CPU."""
    out, cpu = [], []
    cfg = PRESETS["small"]
    print("[bench] extra: small T=64", file=sys.stderr, flush=True)
    w = synthetic.make_weights(cfg, 0, device=dev)
    x = synthetic.hidden_states(64, cfg.hidden, 0).to(dev)
    out.append(workload_report("small MoE layer, 64 tokens, hidden 1024, 8 experts, softmax top-2",
                               x, w, cfg, steps * 4, torch, ops))
    if cpu_tokens > 0:
        cpu.append(cpu_dense_small(x, w, cfg))
        cpu.append(oracle_sample("small MoE layer (64 tokens)", x, w, cfg, 64))
    cfg = PRESETS["kimi_k2"]
    w = synthetic.make_weights(cfg, 3, device=dev, experts_device=dev)
    for T in (1, 16, 256, 2048, 16384):
        print(f"[bench] extra: kimi_k2 T={T}", file=sys.stderr, flush=True)
        x = synthetic.hidden_states(T, cfg.hidden, 3).to(dev)
        out.append(workload_report(f"Kimi-K2 MoE layer, {T} tokens", x, w, cfg, steps, torch, ops))
        if T == 1:
            xs = [synthetic.hidden_states(1, cfg.hidden, 100 + i).to(dev) for i in range(32)]
            out.append(rotated_report("Kimi-K2 MoE layer, 1 token, 32 inputs cycled", xs, w, cfg,
                                      torch, ops))
        if T == 16 and cpu_tokens > 0:
            cpu.append(oracle_sample("Kimi-K2 MoE layer", x, w, cfg, max(1, cpu_tokens // 4)))
    del w
    torch.cuda.empty_cache()
    cfg = PRESETS["glm45"]
    print("[bench] extra: glm45 T=4096 zipf", file=sys.stderr, flush=True)
    w = synthetic.make_weights(cfg, 4, device=dev, zipf=True, experts_device=dev)
    x = synthetic.hidden_states(4096, cfg.hidden, 4).to(dev)
    out.append(workload_report("GLM-4.5 MoE layer, 4096 tokens, Zipf(1.2) routing, 10% empty experts",
                               x, w, cfg, steps, torch, ops))
    if cpu_tokens > 0:
        cpu.append(oracle_sample("GLM-4.5 MoE layer (Zipf)", x, w, cfg, max(1, cpu_tokens // 4)))
    del w
    torch.cuda.empty_cache()
    print("[bench] extra: gpt-oss-120b mxfp4", file=sys.stderr, flush=True)
    layer, inputs = gpt_oss_setup(torch, dev)
    for T in (1, 64, 2048):
        out.append(mx_report(gpt_oss_name(T), layer, inputs(T), steps, torch))
    del layer
    torch.cuda.empty_cache()
    return out, cpu


def gpt_oss_setup(torch, dev):
    """The GPT-OSS-120B MXFP4 layer (128 experts, top-4, hidden 2880 padded to 3072, the
    pre-MoE RMSNorm) with seeded synthetic weights, and its input rows for T tokens."""
    from vllm_neuron_amd import MXFP4MoE, synthetic
    E, Hp, Ip, Hr = 128, 3072, 3072, 2880
    wm = synthetic.make_mx_weights(E, Hp, Ip, 5, device=dev, h_real=Hr, i_real=Hr)
    gamma = (1 + 0.1 * torch.randn(Hp, generator=torch.Generator().manual_seed(5))).to(dev)
    gamma[Hr:] = 0
    layer = MXFP4MoE(wm, 4, norm_weight=gamma, eps=1e-5, hidden_actual=Hr)

    def inputs(T):
        x = torch.zeros(T, Hp)
        x[:, :Hr] = torch.randn(T, Hr, generator=torch.Generator().manual_seed(6))
        return x.to(torch.bfloat16).to(dev)
    return layer, inputs


def gpt_oss_name(T):
    return f"GPT-OSS-120B MoE layer, MXFP4 experts (128, top-4, Swish, clamps, biases), {T} tokens"


def cpu_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        return os.cpu_count()


def _route_cpu(cfg, lg, w):
    import numpy as np
    from oracle import router as R
    sc = R.SOFTMAX if cfg.scoring == "softmax" else R.SIGMOID
    if cfg.grouped:
        cb = None if w.corr_bias is None else w.corr_bias.float().cpu().numpy()
        return R.route_grouped(lg, cb, cfg.top_k, cfg.n_group, cfg.topk_group, sc, cfg.renorm,
                               1e-20, cfg.routed_scaling)
    return R.route_topk_act(lg, cfg.top_k, sc, cfg.renorm, 1e-20, cfg.routed_scaling)


def cpu_baseline(x, w, cfg, n_tokens, reps=3):
    """The oracle (numpy, fp32; sparse per-expert form: router, top-k, each routed
    expert's weights dequantized and applied to its tokens, weighted combine) on
    the first n_tokens tokens of the workload, the weights already in host memory.
    One warm-up run, then the median of `reps` timed runs.
    Returns (tokens/s, experts, median seconds, all timed seconds)."""
    import numpy as np
    import torch
    from oracle import router as R
    from oracle.moe import moe_sparse_fp8
    xs = x[:n_tokens].float().cpu().numpy()
    rb = None if w.router_bias is None else w.router_bias.float().cpu().numpy()
    rw = w.router_w.float().cpu().numpy()
    lg = R.router_logits(xs, rw, rb)
    ids0, _ = _route_cpu(cfg, lg, w)
    experts = sorted(set(np.unique(ids0).tolist()))
    q13 = {e: w.w13[e].view(torch.uint8).cpu().numpy() for e in experts}
    s13 = {e: w.w13_scale[e].cpu().numpy() for e in experts}
    q2 = {e: w.w2[e].view(torch.uint8).cpu().numpy() for e in experts}
    s2 = {e: w.w2_scale[e].cpu().numpy() for e in experts}
    sh = None
    if w.n_shared:
        sh = (w.shared_w13[0].view(torch.uint8).cpu().numpy(), w.shared_w13_scale[0].cpu().numpy(),
              w.shared_w2[0].view(torch.uint8).cpu().numpy(), w.shared_w2_scale[0].cpu().numpy())

    class _D(dict):
        shape = (cfg.n_experts,)

    def run():
        lg = R.router_logits(xs, rw, rb)
        ids, wts = _route_cpu(cfg, lg, w)
        moe_sparse_fp8(xs, ids, wts, _D(q13), _D(s13), _D(q2), _D(s2), shared=sh, experts=experts)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    return n_tokens / dt, len(experts), dt, times


def oracle_sample(name, x, w, cfg, n_tokens):
    print(f"[bench] cpu: {name}, {n_tokens} tokens", file=sys.stderr, flush=True)
    tps, nexp, dt, times = cpu_baseline(x, w, cfg, n_tokens)
    return {"workload": name, "form": "sparse per-expert (oracle)", "tokens": n_tokens,
            "routed_experts": nexp, "seconds": round(dt, 3), "tokens_per_s": round(tps, 3),
            "runs_s": [round(t, 3) for t in times], "timing": "median of 3 after 1 warm-up",
            "cores": cpu_threads()}


def cpu_dense_small(x, w, cfg, reps=3):
    """The small layer in the reference's dense form (_torch_moe_impl, moe_cte.py:465-612:
    every expert on every token, weighted by the dense affinities), on dequantized
    weights; median of `reps` timed runs after one warm-up."""
    import numpy as np
    import torch
    from oracle import router as R
    from oracle.fp8 import dequant_weight_128x128
    from oracle.moe import moe_dense_reference
    print("[bench] cpu: small layer, dense form", file=sys.stderr, flush=True)
    xs = x.float().cpu().numpy()
    T, E, I = xs.shape[0], cfg.n_experts, cfg.intermediate
    w13 = np.stack([dequant_weight_128x128(w.w13[e].view(torch.uint8).cpu().numpy(),
                                           w.w13_scale[e].cpu().numpy()) for e in range(E)])
    w2 = np.stack([dequant_weight_128x128(w.w2[e].view(torch.uint8).cpu().numpy(),
                                          w.w2_scale[e].cpu().numpy()) for e in range(E)])
    gate_up = np.stack([w13[:, :I].transpose(0, 2, 1), w13[:, I:].transpose(0, 2, 1)], axis=2)
    down = np.ascontiguousarray(w2.transpose(0, 2, 1))

    def run():
        lg = R.router_logits(xs, w.router_w.float().cpu().numpy(), None)
        ids, wts = _route_cpu(cfg, lg, w)
        aff = R.scatter_dense(ids, wts, E).reshape(T * E, 1)
        return moe_dense_reference(xs, aff, gate_up, down)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    return {"workload": "small MoE layer (64 tokens)", "form": "dense all-experts (_torch_moe_impl)",
            "tokens": T, "seconds": round(dt, 4), "tokens_per_s": round(T / dt, 1),
            "cores": cpu_threads()}


# --only workloads (the same weights and inputs as the full run): name, preset, tokens,
# weight seed, input seed, Zipf routing
ONLY = {
    "dsv3_prefill8k": ("DeepSeek-V3 MoE layer, 8192 tokens", "dsv3", 8192, 1, 2, False),
    "kimi_k2_1": ("Kimi-K2 MoE layer, 1 token", "kimi_k2", 1, 3, 3, False),
    "dsv3_decode64": ("DeepSeek-V3 MoE layer, decode 64 tokens", "dsv3", 64, 1, 1, False),
    "kimi_k2_2048": ("Kimi-K2 MoE layer, 2048 tokens", "kimi_k2", 2048, 3, 3, False),
    "kimi_k2_16384": ("Kimi-K2 MoE layer, 16384 tokens", "kimi_k2", 16384, 3, 3, False),
    "glm45_zipf4096": ("GLM-4.5 MoE layer, 4096 tokens, Zipf(1.2) routing, 10% empty experts",
                       "glm45", 4096, 4, 4, True),
}
# --only GPT-OSS-120B MXFP4 workloads: tokens
ONLY_MX = {"gpt_oss_1": 1, "gpt_oss_64": 64, "gpt_oss_2048": 2048}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=2)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other workloads (small, Kimi-K2 sweep, GLM-4.5 Zipf, GPT-OSS "
                         "MXFP4) and the CPU samples of them")
    ap.add_argument("--prologue-calls", type=int, default=0,
                    help="only run the decode prologue (fused, then as separate launches) this "
                         "many times at 64 and 8192 tokens, for a kernel trace; no timing")
    ap.add_argument("--only", choices=sorted(ONLY) + sorted(ONLY_MX),
                    help="time one workload alone (whole layer, --steps calls after 2 warm-up "
                         "calls) and print its report line; for kernel traces and counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the layer keeps all experts "
                          "resident on a single MI355X (no expert parallelism); run with --gpus 1"}))
        sys.exit(2)

    import torch
    from vllm_neuron_amd import PRESETS, ops, synthetic

    dev = torch.device("cuda:0")
    if args.only in ONLY_MX:
        T = ONLY_MX[args.only]
        print(f"[bench] only: {gpt_oss_name(T)}", file=sys.stderr, flush=True)
        layer, inputs = gpt_oss_setup(torch, dev)
        print(json.dumps(mx_report(gpt_oss_name(T), layer, inputs(T), args.steps, torch)))
        return
    if args.only:
        name, preset, T, wseed, xseed, zipf = ONLY[args.only]
        cfg = PRESETS[preset]
        print(f"[bench] only: {name}", file=sys.stderr, flush=True)
        w = synthetic.make_weights(cfg, wseed, device=dev, zipf=zipf, experts_device=dev)
        x = synthetic.hidden_states(T, cfg.hidden, xseed).to(dev)
        print(json.dumps(workload_report(name, x, w, cfg, args.steps, torch, ops)))
        return
    if args.prologue_calls:
        run_prologue(args.prologue_calls, torch, ops, dev)
        return
    cfg = PRESETS["dsv3"]
    H, I, E, K = cfg.hidden, cfg.intermediate, cfg.n_experts, cfg.top_k
    print(f"[bench] generating DeepSeek-V3 weights on {torch.cuda.get_device_name(0)}", file=sys.stderr, flush=True)
    w = synthetic.make_weights(cfg, 1, device=dev, experts_device=dev)
    x = synthetic.hidden_states(64, H, 1).to(dev)
    torch.cuda.synchronize()

    # ---- A: whole layer, decode 64
    print("[bench] phase A: decode layer", file=sys.stderr, flush=True)
    sec = time_layer(x, w, cfg, args.steps, args.warmup, torch, ops)
    value = 64 / sec

    # ---- B: per-kernel timing of the expert GEMMs
    print("[bench] phase B: per-kernel events", file=sys.stderr, flush=True)
    gu_ms, dn_ms, ids = run_phase_b(x, w, cfg, args.steps, torch, ops)
    active, routed_rows = layer_counts(ids, E)
    n_units = active + cfg.n_shared
    gu_bytes = n_units * expert_bytes(H, I, "gate_up") + 64 * (H + 4 * H // 128)
    dn_bytes = n_units * expert_bytes(H, I, "down") + (routed_rows + 64) * (I + 4 * I // 128)
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    layer_bytes = (n_units * (expert_bytes(H, I, "gate_up") + expert_bytes(H, I, "down"))
                   + E * H * 2 + 64 * H * 2 * 2)
    layer_flops = 2 * (routed_rows + 64 * cfg.n_shared) * 3 * H * I + 2 * 64 * H * E

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights quantized to e4m3fn 128x128 blocks; x ~ N(0,1) bf16)",
        "config": {"workload": "DeepSeek-V3 MoE layer, decode 64 tokens", "tokens": 64, "hidden": H,
                   "moe_intermediate": I, "routed_experts": E, "shared_experts": cfg.n_shared,
                   "top_k": K, "routing": "sigmoid grouped top-8 (8 groups, 4 kept), bias, renorm, x2.5",
                   "active_experts": active, "parallelism": "none (1 GPU, all experts resident)"},
        "roofline": {"bound": "hbm", "kernel": "expert_gemm_kernel gate_up (decode)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("expert_gemm_kernel<16,0,3,4>", "decode64"),
                     "alg_bytes_per_launch": gu_bytes, "avg_launch_ms": round(gu_ms, 4)},
        "layer": {"alg_bytes": layer_bytes, "alg_flops": layer_flops,
                  "hbm_GBs": round(layer_bytes / sec / 1e9, 1),
                  "hbm_frac": round(layer_bytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                  "down_avg_ms": round(dn_ms, 4),
                  "down_GBs": round(dn_bytes / (dn_ms * 1e-3) / 1e9, 1)},
    }

    # ---- C: prefill 8192 (same layer weights, prefill inputs)
    if not args.no_prefill:
        print("[bench] phase C: prefill 8192", file=sys.stderr, flush=True)
        xp = synthetic.hidden_states(8192, H, 2).to(dev)
        psteps = max(3, args.steps // 4)
        psec = time_layer(xp, w, cfg, psteps, 2, torch, ops)
        pgu, pdn, pids = run_phase_b(xp, w, cfg, psteps, torch, ops)
        pact, prows = layer_counts(pids, E)
        pflops = 2 * (prows + 8192 * cfg.n_shared) * 3 * H * I + 2 * 8192 * H * E
        pbytes = ((pact + cfg.n_shared) * (expert_bytes(H, I, "gate_up") + expert_bytes(H, I, "down"))
                  + E * H * 2 + 8192 * H * 2 * 2)
        gu_flops = 2 * (prows + 8192 * cfg.n_shared) * 2 * H * I
        result["prefill8k"] = {
            "tokens_per_s": round(8192 / psec, 1), "ms_per_step": round(psec * 1e3, 4),
            "steps": psteps, "alg_flops": pflops, "alg_bytes": pbytes,
            "TFLOPs": round(pflops / psec / 1e12, 1),
            "mfma_frac": round(pflops / psec / 1e12 / FP8_PEAK_TFLOPS, 4),
            "hbm_frac": round(pbytes / psec / 1e9 / HBM_PEAK_GBS, 4),
            "roofline_frac": round(max(pbytes / 8e12, pflops / 5e15) / psec, 4),
            "gate_up_avg_ms": round(pgu, 4), "gate_up_TFLOPs": round(gu_flops / (pgu * 1e-3) / 1e12, 1),
            "down_avg_ms": round(pdn, 4),
        }
        del xp

    # ---- D: CPU oracle on a bounded sample
    if args.cpu_tokens > 0:
        print("[bench] phase D: CPU oracle sample", file=sys.stderr, flush=True)
        tps, nexp, dt, times = cpu_baseline(x, w, cfg, args.cpu_tokens)
        cores = cpu_threads()
        result["cpu_baseline"] = {
            "value": round(tps, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first {args.cpu_tokens} of the 64 decode tokens ({nexp} routed experts + shared, "
                      f"full layer math incl. per-expert dequant), numpy fp32 BLAS; median of 3 "
                      f"timed runs after 1 warm-up: {dt:.2f} s (runs "
                      f"{', '.join(f'{t:.2f}' for t in times)} s)"}
    if not args.no_extra:
        del w
        torch.cuda.empty_cache()
        result["extra"], cpu_extra = extra_workloads(max(3, args.steps // 4), torch, ops, synthetic,
                                                     PRESETS, dev, args.cpu_tokens)
        if cpu_extra:
            result["cpu_extra"] = cpu_extra
    print(json.dumps(result))


if __name__ == "__main__":
    main()
