"""
bench.py — routed-expert MXFP4 layer, forward + backward, on one MI355X.

Workload ("config 4"): one MoE layer of 896 experts, each
w1/w3 [2048, 7168] and w2 [7168, 2048] in MXFP4 (uniform e2m1 codes, E8M0 scales
2^-10..2^-6), 1024 tokens of d_model 7168 (fp32 ~N(0,1)), router logits ~N(0,1) -> top-8 with
renormalised softmax weights, upstream gradient ~N(0,1) fp32. One step = the routed forward
(saving gate/up for the backward) + the manual backward (dX through the transposed experts,
GLU derivative, routing-weight gradient). Weights and inputs are resident in HBM before the
timed region starts; nothing is skipped inside it. Before the timed regions the layer also gets
its forward- and backward-layout copies of the expert weights (ExpertLayer.prepare_forward_layout,
prepare_backward_layout: the same bytes in the order the forward and the transposed work-groups
load them, built once, as a resident training or serving process would at load time;
`config.weight_layout` reports their sizes and build times; --no-forward-layout and
--no-backward-layout leave either out).

Prints one JSON line. `value` is MoE-layer fwd+bwd tokens/s; `roofline` is the dominant
kernel's algorithmic weight bytes per launch over its mean duration, measured with HIP events
recorded by the library on the launch stream inside the timed region; `cpu_baseline` is this
repo's C restatement of the reference CPU path timed on a bounded sample of the same layer.

    python bench.py [--steps 20] [--warmup 3] [--routing uniform|zipf] [--no-cpu] [--no-extra]

The default run also times the same step reading only the checkpoint layout (key
"checkpoint_layout_only") and with the forward layout alone (key "forward_layout_only"), the
Zipf-skewed routing of the same layer (key "zipf"), config 3's forward alone under both
routings (key "config3_forward"), config 2 at M = 1 and M = 256 tokens per expert (key
"config2"), a 12-layer sample of config 5's out-of-core sweep (key
"config5_sample", with the same sweep under Zipf routing copying only the selected experts) and
the reference-signature streamed node fed by a streamer of pageable ExpertWeightBundle-shaped
objects (key "streamed_node"), each in its own timed region after the headline's. The CPU
baseline runs on both routings (key "cpu_baseline_zipf" for the Zipf layer, where the
reference's rows > 48 branch runs).
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MXFP4 expert-GEMM HBM GB/s (% of peak); MoE-layer fwd+bwd tokens/s"
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
E, D, F, N, TOPK = 896, 7168, 2048, 1024, 8
SCALE_LO, SCALE_HI = 117, 121  # E8M0 2^-10 .. 2^-6

# algorithmic bytes of one matrix kind per expert: packed codes + E8M0 scales
GATEUP_BYTES = 2 * (F * D // 2 + F * D // 32)  # w1 + w3: 15,597,568
DOWN_BYTES = D * F // 2 + D * F // 32           # w2: 7,798,784
EXPERT_BYTES = GATEUP_BYTES + DOWN_BYTES        # 23,396,352
PHASE_BYTES = {"fwd_gateup": GATEUP_BYTES, "fwd_down": DOWN_BYTES,
               "bwd_down_t": DOWN_BYTES, "bwd_gateup_t": GATEUP_BYTES}
PHASE_KERNEL = {"fwd_gateup": "fwd_fused_kernel<kFwdGateUp>", "fwd_down": "fwd_fused_kernel<kFwdDown>",
                "bwd_down_t": "bwd_wide_kernel<kBwdDownT>", "bwd_gateup_t": "bwd_kernel<kBwdGateUpT>"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "routed_layer_config4_hbm_traffic.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` (calibrated FETCH_SIZE + WRITE_SIZE) from the committed
    rocprofv3 summary, or None when the summary does not list it."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    for line in text.splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == kernel and parts[1].startswith("read=") and parts[2].startswith("write="):
            return int(parts[1][5:]) + int(parts[2][6:])
    return None


def make_layer(seed: int):
    from lazylora_amd.experts import ExpertLayer
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def codes(*shape):
        return torch.randint(0, 256, shape, dtype=torch.uint8, device="cuda", generator=gen)

    def scales(*shape):
        return torch.randint(SCALE_LO, SCALE_HI + 1, shape, dtype=torch.uint8, device="cuda", generator=gen)

    return ExpertLayer(codes(E, F, D // 2), scales(E, F, D // 32), codes(E, F, D // 2), scales(E, F, D // 32),
                       codes(E, D, F // 2), scales(E, D, F // 32))


def forward_layout(args, layer, backward: bool = True) -> dict:
    """Builds the layer's forward-layout copy of the expert weights unless --no-forward-layout
    and, with `backward`, its backward-layout copy unless --no-backward-layout (one-time load
    steps, outside every timed region); returns what the JSON line reports of them."""
    out = {"forward_layout": not args.no_forward_layout,
           "backward_layout": backward and not args.no_backward_layout}
    for name, on, prep in (("forward", out["forward_layout"], layer.prepare_forward_layout),
                           ("backward", out["backward_layout"], layer.prepare_backward_layout)):
        if not on:
            continue
        torch.cuda.synchronize()
        t0 = time.time()
        extra = prep()
        torch.cuda.synchronize()
        ms = (time.time() - t0) * 1e3
        log(f"[bench] {name} layout: {extra / 1e9:.2f} GB more in HBM, built in {ms:.1f} ms")
        out[f"{name}_layout_bytes"] = extra
        out[f"{name}_layout_build_ms"] = round(ms, 1)
    return out


def make_inputs(seed: int, routing: str):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((N, D), dtype=np.float32)
    logits = rng.standard_normal((N, E), dtype=np.float32)
    if routing == "zipf":  # per-expert offset -1.1 * ln(rank), rank a seeded permutation
        logits += (-1.1 * np.log(rng.permutation(E) + 1)).astype(np.float32)[None, :]
    g = rng.standard_normal((N, D), dtype=np.float32)
    lt = torch.from_numpy(logits).cuda()
    val, idx = torch.topk(lt, TOPK, dim=-1, sorted=True)
    w = torch.softmax(val.double(), dim=-1).float()
    return torch.from_numpy(h).cuda(), idx.contiguous(), w.contiguous(), torch.from_numpy(g).cuda()


def _cpu_info() -> dict:
    """Host CPU model, sockets, logical CPUs and the vector extensions the C path uses, from
    /proc/cpuinfo."""
    info = {"model": "unknown", "sockets": None, "logical_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}
    sockets, flags = set(), set()
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and info["model"] == "unknown":
                info["model"] = val
            elif key == "physical id":
                sockets.add(val)
            elif key in ("cpu family", "model", "stepping") and f"cpu_{key.replace(' ', '_')}" not in info:
                info[f"cpu_{key.replace(' ', '_')}"] = val
            elif key == "flags" and not flags:
                flags = set(val.split())
    except OSError:
        pass
    info["sockets"] = len(sockets) or None
    info["vector_flags"] = sorted(f for f in flags if f in ("avx2", "fma", "avx512f", "avx512bw", "avx512_bf16"))
    return info


def cpu_host_layer(layer):
    """The layer's packed tensors on the host as the CPU leg's ExpertSet (copied once)."""
    import oracle
    return oracle.ExpertSet(*[t.cpu().numpy() for t in layer.tensors()])


def cpu_baseline(ex, H, I, W, G, budget_s: float, act: str):
    """The reference trainer's CPU path over the whole layer (every active expert, every token):
    oracle/reference_path.py composes it as lazy_trainer.py:746-880 does, the fused C products
    (oracle/mxfp4_oracle.c, the reference's schedule and flags) for buckets of at most 48 rows and
    C dequantisation + torch's CPU sgemm above. One forward sweep + one backward sweep (which
    recomputes the forward, as the reference does). The median of up to 3 runs that fit the
    budget."""
    import oracle
    from oracle import reference_path
    lib = oracle.oracle_lib()
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    h, idx, w, g = H.cpu().numpy(), I.cpu().numpy(), W.cpu().numpy(), G.cpu().numpy()
    times = []
    while len(times) < 3:
        t0 = time.perf_counter()
        reference_path.routed_forward(lib, h, idx, w, ex, act)
        reference_path.routed_backward(lib, h, idx, w, ex, g, act)
        times.append(time.perf_counter() - t0)
        log(f"[bench] CPU run {len(times)}: {times[-1]:.2f} s")
        if sum(times) + times[0] > budget_s:
            break
    t = float(np.median(times))
    counts = np.bincount(idx.ravel(), minlength=E)
    big = counts > reference_path.FUSED_MAX_ROWS
    return {"value": N / t, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"the whole layer ({int((counts > 0).sum())} active experts, {int(big.sum())} of them above 48 "
                      f"rows, every token), fwd+bwd, median of {len(times)} run(s): {[round(x, 2) for x in times]} s",
            "experts_above_48_rows": int(big.sum()), "pairs_in_experts_above_48_rows": int(counts[big].sum()),
            "cpu": _cpu_info(), "threads": {"openmp": lib.threads(), "torch": torch.get_num_threads()},
            "compile_flags": "gcc -O3 -mavx2 -mfma -fopenmp (oracle/Makefile; the reference's build.sh flags)",
            "path": "reference composition: fused C products for buckets <= 48 rows, C dequant + torch CPU "
                    "sgemm above (lazy_trainer.py:746-880)"}


def make_lora(r: int):
    """Rank-r gate/up/down adapters of the layer (lora_alpha 32, as lazy_lora/core/config.py:69),
    with nonzero A and B so every LoRA term is computed on real values."""
    import types
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)

    def adapter(n_in, n_out):
        A = 0.02 * torch.randn((r, n_in), device="cuda", generator=gen)
        B = 0.02 * torch.randn((n_out, r), device="cuda", generator=gen)
        return types.SimpleNamespace(lora_A=A, lora_B=B, scaling=32.0 / r, dropout_rate=0.0)

    return (adapter(D, F), adapter(D, F), adapter(F, D))


def expert_sweep(args, k, Ms):
    """Config 2: the single-expert MXFP4 GLU block (gate/up 2048x7168, down 7168x2048) forward at
    M tokens. One launch covers 32 distinct expert copies (749 MB, beyond the 256 MB MALL) with M
    tokens each, so every timed pass streams its weights from HBM; per-expert figures are the
    launch's divided by 32."""
    from lazylora_amd.experts import ExpertLayer
    copies = 32
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2)
    codes = lambda *sh: torch.randint(0, 256, sh, dtype=torch.uint8, device="cuda", generator=gen)
    scales = lambda *sh: torch.randint(117, 122, sh, dtype=torch.uint8, device="cuda", generator=gen)
    layer = ExpertLayer(codes(copies, F, D // 2), scales(copies, F, D // 32), codes(copies, F, D // 2),
                        scales(copies, F, D // 32), codes(copies, D, F // 2), scales(copies, D, F // 32))
    forward_layout(args, layer, backward=False)  # a forward-only workload
    sweep = []
    for M in Ms:
        n = copies * M
        rng = np.random.default_rng(M)
        H = torch.from_numpy(rng.standard_normal((n, D), dtype=np.float32)).cuda()
        I = (torch.arange(n, device="cuda") // M).to(torch.int64).reshape(n, 1)
        W = torch.ones((n, 1), device="cuda")
        ws = torch.empty(k.moe_workspace_bytes(n, 1, copies, D, F), dtype=torch.uint8, device="cuda")
        for _ in range(args.warmup):
            k.routed_forward(H, I, W, layer, act=args.act, workspace=ws)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            k.routed_forward(H, I, W, layer, act=args.act, workspace=ws)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps  # phase timer off: its event records cost time
        k.set_timing(True)
        for _ in range(args.steps):
            k.routed_forward(H, I, W, layer, act=args.act, workspace=ws)
        torch.cuda.synchronize()
        calls = k.phase_times()
        k.set_timing(False)
        ph = {}
        for call in calls:
            for name, t in call:
                ph.setdefault(name, []).append(t)
        ph = {n_: float(np.mean(v)) for n_, v in ph.items()}
        prod_ms = ph["fwd_gateup"] + ph["fwd_down"]
        wbytes = copies * EXPERT_BYTES
        row = {"M": M, "us_per_expert": ms * 1e3 / copies, "products_us_per_expert": prod_ms * 1e3 / copies,
               "weight_GBps_products": wbytes / (prod_ms * 1e-3) / 1e9,
               "frac_of_hbm_peak_products": wbytes / (prod_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
               "weight_GBps_whole_call": wbytes / (ms * 1e-3) / 1e9,
               "TFLOPs_products": copies * 6.0 * F * D * M / (prod_ms * 1e-3) / 1e12,
               "phases_ms": {n_: round(v, 4) for n_, v in ph.items()}}
        sweep.append(row)
        log(f"[bench] expert M={M:3d}: {row['us_per_expert']:7.2f} us/expert (products "
            f"{row['products_us_per_expert']:6.2f} us, {row['weight_GBps_products']:7.1f} GB/s, "
            f"{row['TFLOPs_products']:6.1f} TFLOP/s)")
    del layer
    torch.cuda.empty_cache()
    return sweep, copies


def expert_main(args, k):
    sweep, copies = expert_sweep(args, k, (1, 4, 16, 64, 256))
    line = {
        "metric": "config 2: single-expert MXFP4 GLU block forward, weight GB/s of the products (M = 1)",
        "value": sweep[0]["weight_GBps_products"],
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sweep[0]["us_per_expert"] * copies / 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4", "data": "synthetic",
        "config": {"workload": f"config 2: expert block gate/up {F}x{D}, down {D}x{F} MXFP4, M in 1..256 tokens, "
                               f"{copies} distinct expert copies per launch", "act": args.act},
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


def stream_hosts(ring):
    """`ring` distinct config-3 layers in pinned host memory (93 x 20.96 GB cannot be pinned)."""
    from lazylora_amd.streaming import host_layer_from
    hosts = []
    for r in range(ring):
        layer = make_layer(r)
        hosts.append(host_layer_from(layer, pin=True))
        del layer
        torch.cuda.empty_cache()
    return hosts


def stream_sweep(args, k, layers, ring, routing, hosts=None, active_only=False):
    """Config 5: an out-of-core sweep of `layers` routed-expert layers of the config-3 shape, each
    copied from pinned host memory (a ring of `ring` distinct layers) into one of two HBM slots on
    a copy stream while the compute stream runs the layer forward for 1024 tokens on the previous
    slot. active_only: copy only the experts the routing selects (as the reference's streamer
    loads only the active experts); with uniform routing that is every expert. Returns the
    sweep's timings."""
    from lazylora_amd.streaming import LayerStreamer
    t_setup = time.time()
    if hosts is None:
        hosts = stream_hosts(ring)
    H, I, W, _ = make_inputs(1, routing)
    active = torch.unique(I).tolist() if active_only else None
    ids = (lambda n: [active] * n) if active_only else (lambda n: None)
    ws = torch.empty(k.moe_workspace_bytes(N, TOPK, E, D, F), dtype=torch.uint8, device="cuda")
    streamer = LayerStreamer(E, D, F, slots=2, timing=True)
    log(f"[bench] stream: {ring} pinned host layers of {hosts[0].nbytes / 1e9:.2f} GB, setup "
        f"{time.time() - t_setup:.1f}s")
    # one warm sweep of a few layers (first-touch of the slots and the workspace)
    for _, layer in streamer.stream((hosts[i % ring] for i in range(min(3, layers))), ids(min(3, layers))):
        k.routed_forward(H, I, W, layer, act=args.act, workspace=ws)
    torch.cuda.synchronize()
    streamer.copy_events.clear()
    comp = []
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i, layer in streamer.stream((hosts[i % ring] for i in range(layers)), ids(layers)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        k.routed_forward(H, I, W, layer, act=args.act, workspace=ws)
        b.record(stream)
        comp.append((a, b))
        if (i + 1) % 16 == 0:
            log(f"[bench] stream: {i + 1} layers issued")
    end.record(stream)
    torch.cuda.synchronize()
    t_total = start.elapsed_time(end) / 1e3
    t_comp = sum(a.elapsed_time(b) for a, b in comp) / 1e3
    copy_ms, copy_bytes = streamer.copy_stats()
    t_copy = copy_ms / 1e3
    hidden = max(0.0, min(1.0, (t_copy + t_comp - t_total) / t_comp)) if t_comp > 0 else 0.0
    del streamer, ws
    torch.cuda.empty_cache()
    return {"total_s": t_total, "compute_s": t_comp, "copy_s": t_copy, "copy_bytes": copy_bytes,
            "hidden_compute_fraction": hidden, "experts_copied": len(active) if active_only else E}


def stream_main(args, k):
    """Config 5 as the bench line (`--workload stream`): the full sweep of args.layers layers."""
    r = stream_sweep(args, k, args.layers, args.ring, args.routing, active_only=args.active_only)
    t_total, t_comp, t_copy, copy_bytes, hidden = (r["total_s"], r["compute_s"], r["copy_s"], r["copy_bytes"],
                                                   r["hidden_compute_fraction"])
    h2d = copy_bytes / t_copy / 1e9
    line = {
        "metric": "config 5 out-of-core sweep: tokens/s through all layers (H2D-bound)",
        "value": N / t_total,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.layers,
        "warmup": 3,
        "ms_per_step": t_total * 1e3 / args.layers,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4",
        "data": "synthetic",
        "config": {"workload": f"config 5: {args.layers} routed-expert layers (config-3 shape, 20.96 GB each) "
                               f"streamed from a ring of {args.ring} pinned host layers into 2 HBM slots, layer "
                               f"forward for {N} tokens x {D}, top-{TOPK}",
                   "routing": args.routing, "act": args.act, "experts_copied_per_layer": r["experts_copied"]},
        "h2d_GBps": h2d,
        "h2d_bytes_per_layer": copy_bytes / args.layers,
        "copy_s": t_copy,
        "compute_s": t_comp,
        "total_s": t_total,
        "hidden_compute_fraction": hidden,
    }
    print(json.dumps(line), flush=True)


def streamed_node_sample(args, k, layer, H, I, W, G, reps: int = 3):
    """The reference-signature node (routed.StreamedRoutedExpertsFunction, lazy_trainer.py:45-77)
    fed by a streamer that yields ExpertWeightBundle-shaped objects of pageable host tensors, as
    the reference's DynamicExpertStreamer does (expert_streamer.py:27-50, :315-369), in a seeded
    'disk' order: the active experts of the given routing, each pass staging them through pinned
    buffers into a compact HBM layer. Reports the staging rate alone (generator to layer ready)
    and the node's forward and forward + backward (two streaming passes) per layer."""
    from types import SimpleNamespace
    from lazylora_amd.routed import StreamedRoutedExpertsFunction, _stager
    active = torch.unique(I).tolist()
    order = {e: i for i, e in enumerate(np.random.default_rng(5).permutation(active).tolist())}
    names = ("gate_packed", "gate_scale", "up_packed", "up_scale", "down_packed", "down_scale")
    bundles = {e: SimpleNamespace(expert_idx=e, packed=True,
                                  **{n: t[e].cpu() for n, t in zip(names, layer.tensors())}) for e in active}

    class Streamer:
        def stream_experts(self, layer_idx, ids):
            for e in sorted(ids, key=order.__getitem__):
                yield e, bundles[e]

    streamer = Streamer()
    trainer = SimpleNamespace(expert_streamer=streamer)
    nbytes = len(active) * EXPERT_BYTES
    stager = _stager(H.device)
    stager.stage(streamer.stream_experts(0, active), len(active))  # warm: pinned buffers, allocator
    torch.cuda.synchronize()
    stage_s = []
    for _ in range(reps):
        t0 = time.perf_counter()
        stager.stage(streamer.stream_experts(0, active), len(active))
        torch.cuda.synchronize()
        stage_s.append(time.perf_counter() - t0)
    fwd_s, step_s = [], []
    for _ in range(reps):
        h = H.detach().requires_grad_()
        w = W.detach().requires_grad_()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = StreamedRoutedExpertsFunction.apply(h, w, I, trainer, 0, None, active, None)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        out.backward(G)
        torch.cuda.synchronize()
        fwd_s.append(t1 - t0)
        step_s.append(time.perf_counter() - t0)
    t_stage = float(np.median(stage_s))
    log(f"[bench] streamed node: {len(active)} experts ({nbytes / 1e9:.2f} GB) staged in {t_stage * 1e3:.1f} ms "
        f"({nbytes / t_stage / 1e9:.1f} GB/s), forward {np.median(fwd_s) * 1e3:.1f} ms, "
        f"fwd+bwd {np.median(step_s) * 1e3:.1f} ms")
    del bundles
    return {"experts_streamed": len(active), "bytes_per_pass": nbytes,
            "staging_s": t_stage, "staging_GBps": nbytes / t_stage / 1e9,
            "forward_s": float(np.median(fwd_s)), "forward_backward_s": float(np.median(step_s)),
            "source": "pageable host tensors (ExpertWeightBundle-shaped), pinned staging, copy stream"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--routing", choices=["uniform", "zipf"], default="uniform")
    ap.add_argument("--act", choices=["swiglu", "situ"], default="swiglu")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=30.0, help="budget of the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the Zipf-routing step and the config-2 points reported beside the headline")
    ap.add_argument("--workload", choices=["layer", "stream", "expert"], default="layer",
                    help="layer: config 4 (the metric); stream: config 5, layers streamed from pinned host memory; "
                         "expert: config 2, the single-expert block swept over token counts")
    ap.add_argument("--layers", type=int, default=93, help="stream: layers per sweep (Kimi K3 has 93 MoE layers)")
    ap.add_argument("--ring", type=int, default=2, help="stream: distinct pinned host layers cycled through")
    ap.add_argument("--active-only", action="store_true",
                    help="stream: copy only the experts the routing selects (every expert under uniform routing)")
    ap.add_argument("--lora-rank", type=int, default=0,
                    help="rank of the layer's gate/up/down LoRA adapters (0: off, the BASELINE configs)")
    ap.add_argument("--no-forward-layout", action="store_true",
                    help="no forward-layout copy of the expert weights (the forward reads the checkpoint layout)")
    ap.add_argument("--no-backward-layout", action="store_true",
                    help="no backward-layout copy (the transposed products read the checkpoint layout)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (reference kernel for rocprof byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU: the routed-expert path is measured on one "
                                   "MI355X (expert-parallel sharding is a design note, not implemented)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if not torch.cuda.is_available():
        sys.exit("bench.py needs the MI355X")

    from lazylora_amd.native import kernel
    k = kernel()
    torch.cuda.set_device(0)
    if args.workload == "stream":
        stream_main(args, k)
        return
    if args.workload == "expert":
        expert_main(args, k)
        return
    t_setup = time.time()
    layer = make_layer(0)
    layout = forward_layout(args, layer)
    H, I, W, G = make_inputs(1, args.routing)
    n_active = int(torch.unique(I).numel())
    ws = torch.empty(k.moe_workspace_bytes(N, TOPK, E, D, F), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    log(f"[bench] layer {layer.nbytes / 1e9:.2f} GB in HBM, {n_active} active experts, setup {time.time() - t_setup:.1f}s")

    lora = make_lora(args.lora_rank) if args.lora_rank else None
    ms_step, phase_avg = time_layer(args, k, layer, H, I, W, G, ws, lora, n_active, calibrate=args.copy_calibration)

    dom = max((n for n in phase_avg if n in PHASE_BYTES), key=lambda n: phase_avg[n])
    dom_bytes = PHASE_BYTES[dom] * n_active
    dom_gbs = dom_bytes / (phase_avg[dom] * 1e-3) / 1e9
    step_bytes = 2 * EXPERT_BYTES * n_active  # one forward pass + one transposed pass over the weights
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9

    extra = {}
    if lora is not None:
        extra["lora_overhead"] = time_lora_ab(args, k, layer, H, I, W, G, ws, lora)
    zipf_inputs = None
    if not args.no_extra and layout.get("backward_layout") and layout.get("forward_layout"):
        # the same step with the forward layout alone, for comparison (then the copy is rebuilt)
        layer.drop_backward_layout()
        ms_fo, _ = time_layer(args, k, layer, H, I, W, G, ws, lora, n_active)
        extra["forward_layout_only"] = {"ms_per_step": ms_fo, "tokens_per_s": N / (ms_fo * 1e-3)}
        layer.prepare_backward_layout()
    if not args.no_extra and (layout.get("forward_layout") or layout.get("backward_layout")):
        # the same step reading only the checkpoint layout, for comparison (then the copies are rebuilt)
        layer.drop_forward_layout()
        layer.drop_backward_layout()
        ms_ck, _ = time_layer(args, k, layer, H, I, W, G, ws, lora, n_active)
        extra["checkpoint_layout_only"] = {"ms_per_step": ms_ck, "tokens_per_s": N / (ms_ck * 1e-3)}
        if layout.get("forward_layout"):
            layer.prepare_forward_layout()
        if layout.get("backward_layout"):
            layer.prepare_backward_layout()
    if not args.no_extra and args.routing == "uniform" and not args.lora_rank:
        # the skewed variant of configs 3/4 ([3]) on the same layer
        Hz, Iz, Wz, Gz = make_inputs(1, "zipf")
        nz = int(torch.unique(Iz).numel())
        counts = torch.bincount(Iz.flatten(), minlength=E)
        log(f"[bench] zipf routing: {nz} active experts, largest bucket {int(counts.max())}")
        ms_z, ph_z = time_layer(args, k, layer, Hz, Iz, Wz, Gz, ws, None, nz)
        extra["zipf"] = {"ms_per_step": ms_z, "tokens_per_s": N / (ms_z * 1e-3), "active_experts": nz,
                         "largest_bucket": int(counts.max()),
                         "weight_GBps": 2 * EXPERT_BYTES * nz / (ms_z * 1e-3) / 1e9,
                         "phases_ms": {n: round(v, 4) for n, v in ph_z.items()}}
        # config 3: the same layer's forward alone, both routings
        extra["config3_forward"] = {"uniform": time_forward(args, k, layer, H, I, W, ws, n_active),
                                    "zipf": time_forward(args, k, layer, Hz, Iz, Wz, ws, nz)}
        # the reference-signature streamed node on the Zipf routing's active experts
        extra["streamed_node"] = streamed_node_sample(args, k, layer, Hz, Iz, Wz, Gz)
        zipf_inputs = (Hz, Iz, Wz, Gz)
        # config 2 at its two ends, M = 1 (HBM-bound) and M = 256 (MFMA-bound)
        del ws
        torch.cuda.empty_cache()
        sweep, copies = expert_sweep(args, k, (1, 256))
        extra["config2"] = {f"M={r['M']}": {"us_per_expert": r["us_per_expert"],
                                            "products_us_per_expert": r["products_us_per_expert"],
                                            "weight_GBps_products": r["weight_GBps_products"],
                                            "TFLOPs_products": r["TFLOPs_products"]} for r in sweep}
        extra["config2"]["expert_copies_per_launch"] = copies
        # config 5 on a sample of its sweep: 12 of the 93 layers streamed
        # from pinned host memory; the full sweep is `--workload stream`
        n5 = 12
        hosts = stream_hosts(2)
        r5 = stream_sweep(args, k, n5, 2, args.routing, hosts=hosts)
        per_layer = r5["total_s"] / n5
        extra["config5_sample"] = {
            "layers_streamed": n5, "s_per_layer": per_layer,
            "tokens_per_s_93_layers": N / (93 * per_layer),
            "h2d_GBps": r5["copy_bytes"] / r5["copy_s"] / 1e9,
            "hidden_compute_fraction": r5["hidden_compute_fraction"],
            "note": "a 93-layer sweep costs 93 x s_per_layer (the sweep is H2D-bound, so the per-layer time "
                    "does not depend on the layer count)"}
        # the same sweep under the Zipf-skewed routing, copying only the experts it selects
        r5z = stream_sweep(args, k, n5, 2, "zipf", hosts=hosts, active_only=True)
        per_layer_z = r5z["total_s"] / n5
        extra["config5_sample"]["zipf_active_experts_only"] = {
            "experts_copied": r5z["experts_copied"], "s_per_layer": per_layer_z,
            "tokens_per_s_93_layers": N / (93 * per_layer_z),
            "h2d_GBps": r5z["copy_bytes"] / r5z["copy_s"] / 1e9,
            "hidden_compute_fraction": r5z["hidden_compute_fraction"]}
        del hosts
        ls = extra["config5_sample"]["zipf_active_experts_only"]["h2d_GBps"]
        extra["streamed_node"]["layer_streamer_GBps_same_experts"] = ls
        extra["streamed_node"]["staging_vs_layer_streamer"] = extra["streamed_node"]["staging_GBps"] / ls

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline (the reference composition on the C restatement + torch CPU) ...")
        ex = cpu_host_layer(layer)
        cpu = cpu_baseline(ex, H, I, W, G, args.cpu_seconds, args.act)
        log(f"[bench] CPU baseline {cpu['value']:.2f} tokens/s on {cpu['cores']} threads")
        if zipf_inputs is not None:  # the Zipf layer, where the reference's > 48-row branch runs
            cz = cpu_baseline(ex, *zipf_inputs, args.cpu_seconds, args.act)
            log(f"[bench] CPU baseline, Zipf routing: {cz['value']:.2f} tokens/s")
            extra["cpu_baseline_zipf"] = cz
            if "zipf" in extra:
                extra["zipf"]["vs_cpu_baseline_zipf"] = extra["zipf"]["tokens_per_s"] / cz["value"]
        del ex

    line = {
        "metric": METRIC,
        "value": N / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4",
        "data": "synthetic",
        "config": {
            "workload": "config 4: routed-expert MoE layer fwd+bwd, 896 experts (w1/w3 2048x7168, w2 7168x2048 "
                        "MXFP4), 1024 tokens x 7168, top-8",
            "routing": args.routing, "act": args.act, "active_experts": n_active, "lora_rank": args.lora_rank,
            "arithmetic": "MXFP4 weights x two-term e4m3 activations (fwd, fp4-native scaled MFMA) / exact bf16 "
                          "decode x two-term bf16 gradients (bwd, bf16 MFMA), fp32 accumulate",
            "weight_bytes_per_step": step_bytes,
            "weight_layout": layout,
        },
        "weight_GBps": step_gbs,
        "weight_frac_of_hbm_peak": step_gbs / PEAK_HBM_GBS,
        "phases_ms": {n: round(v, 4) for n, v in phase_avg.items()},
        "roofline": {"bound": "hbm", "achieved": dom_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": dom_gbs / PEAK_HBM_GBS, "traffic": measured_traffic(PHASE_KERNEL[dom]),
                     "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT), "kernel": PHASE_KERNEL[dom],
                     "algorithmic_bytes_per_launch": dom_bytes, "mean_launch_ms": phase_avg[dom]},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def time_forward(args, k, layer, H, I, W, ws, n_active):
    """Config 3: the routed layer's forward alone (routing, quantised x,
    gate/up + GLU, down, combine; nothing saved for a backward). A dict of ms per forward,
    tokens/s and weight GB/s over args.steps timed calls after args.warmup."""
    def fwd():
        return k.routed_forward(H, I, W, layer, act=args.act, save_for_backward=False, workspace=ws)

    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        fwd()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    log(f"[bench] forward alone: {ms:.3f} ms ({n_active} active experts)")
    return {"ms_per_forward": ms, "tokens_per_s": N / (ms * 1e-3), "active_experts": n_active,
            "weight_GBps": EXPERT_BYTES * n_active / (ms * 1e-3) / 1e9}


def time_lora_ab(args, k, layer, H, I, W, G, ws, lora, rounds=6):
    """The step with the adapters against the same step without them, timed in alternating
    rounds of args.steps steps in one process (so clock and thermal drift affect both alike):
    median ms per step of each and the median of the paired differences."""
    def run(lo):
        k.routed_forward(H, I, W, layer, act=args.act, save_for_backward=True, workspace=ws, lora=lo)
        k.routed_backward(H, I, W, layer, G, act=args.act, reuse_forward=True, workspace=ws, lora=lo)

    stream = torch.cuda.current_stream()
    on, off = [], []
    for _ in range(rounds):
        for lo, out in ((None, off), (lora, on)):
            run(lo)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(args.steps):
                run(lo)
            end.record(stream)
            torch.cuda.synchronize()
            out.append(start.elapsed_time(end) / args.steps)
    diff = [a - b for a, b in zip(on, off)]
    res = {"rank": args.lora_rank, "rounds": rounds, "steps_per_round": args.steps,
           "lora_off_ms": float(np.median(off)), "lora_on_ms": float(np.median(on)),
           "overhead_ms": float(np.median(diff)), "overhead_ms_per_round": [round(d, 4) for d in diff]}
    log(f"[bench] LoRA rank {args.lora_rank}: {res['lora_on_ms']:.3f} ms/step vs {res['lora_off_ms']:.3f} without "
        f"(+{res['overhead_ms']:.3f} ms, median of {rounds} alternating rounds)")
    return res


def time_layer(args, k, layer, H, I, W, G, ws, lora, n_active, calibrate=False):
    """(ms per fwd+bwd step, mean ms per phase) over args.steps timed steps after args.warmup."""
    def step():
        k.routed_forward(H, I, W, layer, act=args.act, save_for_backward=True, workspace=ws, lora=lora)
        return k.routed_backward(H, I, W, layer, G, act=args.act, reuse_forward=True, workspace=ws, lora=lora)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done")
    if calibrate:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # the step time with the library's phase timer off (its per-phase event records cost time on
    # the stream), then the per-phase times over a separate run of the same steps
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / args.steps
    log(f"[bench] timed {args.steps} steps: {ms_step:.3f} ms/step")
    k.set_timing(True)
    for _ in range(max(3, args.steps // 4)):
        step()
    torch.cuda.synchronize()
    calls = k.phase_times()
    k.set_timing(False)
    phase_ms = {}
    for call in calls:
        for name, ms in call:
            phase_ms.setdefault(name, []).append(ms)
    phase_avg = {n: float(np.mean(v)) for n, v in phase_ms.items()}
    for n, v in sorted(phase_avg.items(), key=lambda kv: -kv[1]):
        extra = ""
        if n in PHASE_BYTES:
            extra = f"  {PHASE_BYTES[n] * n_active / (v * 1e-3) / 1e9:8.1f} GB/s algorithmic"
        log(f"[bench]   {n:14s} {v:8.3f} ms{extra}")
    return ms_step, phase_avg


if __name__ == "__main__":
    main()
