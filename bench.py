#!/usr/bin/env python3
"""Benchmark: Qwen3-VL-8B-shape decoder layer, bf16 prefill at S=4096 (headline) + B=32 decode.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--seq 4096] [--no-cpu-baseline] [--no-decode]

One step = one CudaTextDecoderLayer forward over a (1, S, 4096) batch of
synthetic N(0,1) inputs with N(0,0.02) weights, all resident in HBM before
timing. Prints ONE JSON line on stdout; details go to stderr.

roofline: the dominant kernel (the fused gate/up/SwiGLU GEMM, 2*S*4096*12288*2
FLOP per launch) timed with HIP events on the stream it runs on, against the
MI355X dense bf16 MFMA peak. cpu_baseline: the CPU oracle (a restatement of the
reference's torch path) on this host's cores, same shapes, bf16.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

# Bytes the dominant kernel (gate/up + SwiGLU GEMM, S=4096) moves between L2
# and memory per launch, from two rocprofv3 --pmc passes over `bench.py
# --traffic-probe` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled
# by what the same counter reads for a plain 512 MiB device copy in the same
# run (FETCH_SIZE 262157.5 KiB -> x1.9999; WRITE_SIZE 524288 KiB -> x1.000).
# GEMM (2 X + 3 W ring slots, 16x16x32 loop, bf16 LDS-staged epilogue):
# FETCH_SIZE 589992.7, WRITE_SIZE 98304.0 KiB. Re-measure when the kernel changes; the command and
# per-dispatch counts are in profiles/.
GATE_UP_TRAFFIC_BYTES = int((589992.7 * (524_288 / 262157.5) + 98304.0 * 1.0) * 1024)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_gpu(fn, steps: int, warmup: int) -> float:
    """Average ms per call, HIP events on torch's current stream (where every op launches)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_launch_modes(step, first, steps: int, warmup: int, warm_s: float = 0.0):
    """Time `step` with eager launches, then replayed from a HIP graph, each
    as max(HIP events, host wall) per step. `first(out)` picks the tensor of a
    step's output that every replay must reproduce bit for bit (checked before
    and after the timed replays). Returns (ms, ms_eager, ms_graph, launch):
    the faster mode's time, both times, and which mode that was.

    `warm_s` > 0 keeps warming up past `warmup` steps until that much wall time
    of back-to-back steps has passed (each mode): a GPU coming from idle runs
    its first ~40 ms of load at a lower clock, which a short step's few
    warm-up steps do not cover (the S=1024 layer measured ~0.51 ms after 2
    warm-up steps against ~0.46 ms in steady rounds).

    On a box whose host is slow or contended, eager launches have left the GPU
    idle between kernels (3.2 ms per S=4096 layer against 1.5 with every kernel
    at its usual speed); with a fast host, eager launches run back to back and
    the graph's node-to-node dispatch costs ~2-4 us per kernel more (1.382
    against 1.435 ms in one run)."""
    import torch
    from qwen3_5_vl_cuda_custom_amd.modules import StepGraph

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ms_events = time_gpu(fn, steps, 0)
        torch.cuda.synchronize()
        return max(ms_events, (time.perf_counter() - t0) * 1e3 / steps)

    def warm(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warm_s:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()

    warm(step)
    ms_eager = timed(step)
    ref = first(step()).clone()
    graph = StepGraph(step)
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(first(graph.out), ref):
        raise RuntimeError("bench: the graph replay of the step differs from the eager step")
    warm(graph.replay)
    ms_graph = timed(graph.replay)
    if not torch.equal(first(graph.out), ref):
        raise RuntimeError("bench: a timed graph replay of the step differs from the eager step")
    del graph
    launch = "HIP graph replay" if ms_graph <= ms_eager else "eager launches"
    return min(ms_graph, ms_eager), ms_eager, ms_graph, launch


def usable_cpus() -> int:
    """CPUs this process may run on: its affinity set, capped by a cgroup CPU quota if one is set."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            n = min(n, max(1, -(-int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, seq: int, layer, budget_s: float = 20.0) -> dict:
    """The oracle's decoder layer on CPU tensors (bf16), 1 warm-up + timed runs within the budget,
    with torch's intra-op threads set to every CPU the process may use."""
    import torch

    from oracle import layers as L
    from oracle import ops as O
    prev = torch.get_num_threads()
    threads = usable_cpus()
    torch.set_num_threads(threads)
    try:
        return _cpu_baseline(torch, L, O, cfg, seq, layer, budget_s, threads)
    finally:
        torch.set_num_threads(prev)


def _cpu_baseline(torch, L, O, cfg, seq, layer, budget_s, threads) -> dict:
    p = {n: t.detach().to("cpu") for n, t in layer.state_dict().items()}
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, seq, cfg.hidden, generator=g).to(torch.bfloat16)
    pos = torch.arange(seq).view(1, 1, seq).expand(3, 1, seq)
    cos3, sin3 = O.mrope_cos_sin(pos, cfg.head_dim, cfg.theta)

    def run():
        return L.text_decoder_layer(x, p, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                                    eps=cfg.eps, cos_3d=cos3, sin_3d=sin3, mrope_section=list(cfg.mrope_section))

    t0 = time.perf_counter()
    run()
    first = time.perf_counter() - t0
    times = []
    while sum(times) + first < budget_s and len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    if not times:
        times = [first]
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(seq / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "threads": f"torch.set_num_threads({threads}): the CPUs the process may use (affinity, cgroup quota)",
            "sample": f"oracle decoder layer (torch CPU, bf16) at S={seq}, 1 warm-up + median of {len(times)} "
                      f"run(s), {med:.2f} s/layer"}


def parity_leg(cases: dict) -> dict:
    """Per configuration: the GPU output against the fp32 oracle and the reference's bf16
    path (the oracle with every op output rounded to bf16), both on CPU, on the same
    seeded inputs. Runs after every timed region; the oracle is only the checker here."""
    import torch

    from oracle import layers as L
    from oracle import ops as O
    prev = torch.get_num_threads()
    torch.set_num_threads(usable_cpus())
    ident = lambda t: t  # noqa: E731

    def metrics(out, ref):
        d = (out.float() - ref).abs()
        return float(d.max()), float(d.mean() / ref.abs().mean().clamp_min(1e-30))

    def ulp_at_worst(out, ref):
        import math
        w = float(ref.reshape(-1)[int((out.float() - ref).abs().argmax())])
        return 2.0 ** (math.frexp(abs(w))[1] - 8) if w else 0.0

    res, secs = {}, {}
    try:
        for name, (gpu_out, run) in cases.items():
            t0 = time.perf_counter()
            ref = run(L, O, ident)
            secs[name] = time.perf_counter() - t0
            emu = run(L, O, O.round_bf16)
            ma, mr = metrics(gpu_out, ref)
            ema, emr = metrics(emu, ref)
            res[name] = {"max_abs": round(ma, 5), "mean_rel": round(mr, 6), "ref_bf16_max_abs": round(ema, 5),
                         "ref_bf16_mean_rel": round(emr, 6), "bar_max_abs": 2e-2, "bar_mean_rel": 5e-3,
                         "within_2e-2": ma <= 2e-2,
                         # the test bar: no worse than the reference bf16 path, up to
                         # equal-rounding ties (2% of mean-rel, one bf16 ulp of the worst element)
                         "within_ref_bf16": (ma <= max(2e-2, ema + ulp_at_worst(gpu_out, ref))
                                             and mr <= emr * 1.02 and (mr <= 5e-3 or emr > 5e-3))}
            log(f"parity {name}: {res[name]} ({time.perf_counter() - t0:.1f} s)")
    finally:
        torch.set_num_threads(prev)
    return res, secs


# Work per run of each configuration's oracle (for the per-configuration CPU baseline).
CPU_UNITS = {"c3_decode_b32": (32, "tokens/s", "one B=32 decode step of the 8B-shape layer (per-sequence "
                                               "attention over each sequence's cache rows)"),
             "c4_moe_layer_t4096": (4096, "tokens/s", "the 30B-A3B-shape MoE layer on 4096 tokens"),
             "c5_vision_patch_embed_block": (3136, "patches/s", "C5 patch embed + vision block on 4 x 784 "
                                                                "patches")}


def cpu_baseline_other(secs: dict) -> dict:
    """The oracle's own CPU run of each non-headline configuration (its fp32 pass of the parity leg:
    torch CPU ops on the bf16-rounded inputs), as throughput: a reported baseline, not a target."""
    out = {}
    for name, (n, unit, what) in CPU_UNITS.items():
        if name in secs:
            out[name] = {"value": round(n / secs[name], 1), "unit": unit, "seconds": round(secs[name], 3),
                         "cores": usable_cpus(), "kind": "port",
                         "sample": f"oracle (torch CPU, fp32 math on bf16-rounded values): {what}, one run"}
    return out


def _params_cpu(module) -> dict:
    return {n: t.detach().float().cpu() for n, t in module.state_dict().items()}


def text_layer_case(cfg, layer, x, pos, y, router_logits=None):
    """(GPU output, oracle closure) for a prefill layer, everything on the CPU."""
    p, xc, posc = _params_cpu(layer), x.detach().float().cpu(), pos.detach().cpu()
    rl = router_logits.detach().float().cpu() if router_logits is not None else None

    def run(L, O, rd):
        cos3, sin3 = O.mrope_cos_sin(posc, cfg.head_dim, cfg.theta)
        return L.text_decoder_layer(xc, p, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                                    eps=cfg.eps, cos_3d=cos3, sin_3d=sin3, mrope_section=list(cfg.mrope_section),
                                    use_moe=cfg.use_moe, top_k=cfg.top_k, router_logits=rl, rd=rd)[0]
    return y.detach().float().cpu(), run


def decode_case(cfg, layer, x, pos, lens, k_cache, v_cache, y):
    """(GPU output, oracle closure) for one decode step: each sequence attends to its cache rows
    [0, L_b) plus the new token (the reference's past_kv form, one sequence at a time)."""
    p, xc, posc = _params_cpu(layer), x.detach().float().cpu(), pos.detach().cpu()
    kc, vc, lc = k_cache.detach().cpu(), v_cache.detach().cpu(), [int(v) for v in lens]

    def run(L, O, rd):
        import torch
        outs = []
        for b, Lb in enumerate(lc):
            cos3, sin3 = O.mrope_cos_sin(posc[:, b:b + 1], cfg.head_dim, cfg.theta)
            past = (kc[b:b + 1, :, :Lb].float(), vc[b:b + 1, :, :Lb].float())
            outs.append(L.text_decoder_layer(xc[b:b + 1], p, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads,
                                             head_dim=cfg.head_dim, eps=cfg.eps, cos_3d=cos3, sin_3d=sin3,
                                             mrope_section=list(cfg.mrope_section), past_kv=past, rd=rd)[0])
        return torch.cat(outs)
    return y.detach().float().cpu(), run


def other_configs(torch, W, dev: str, warmup: int, cases: dict) -> dict:
    """The other BASELINE configurations, one GPU each: C2 at S=1024 and 16384,
    the C4 MoE layer (4096 tokens) and the C5 patch embed + vision block. Each
    takes the faster of eager launches and a HIP graph replay (both reported,
    the replay checked bit-identical to the eager step), each mode after
    0.25 s of back-to-back warm-up steps (steady clock)."""
    out = {}
    for S in (1024, 16384):
        cfg = W.C2
        layer = W.make_text_layer(cfg, torch.bfloat16, dev, seed=0)
        x, pos = W.text_inputs(cfg, 1, S, torch.bfloat16, dev, seed=0)
        b = W.make_rope(cfg, dev).bind(pos)
        ms, me, mg, launch = time_launch_modes(lambda: layer(x, b), lambda o: o[0], 5 if S > 4096 else 20,
                                                max(2, warmup // 2), warm_s=0.25)
        fl = cfg.gemm_flops_per_token() * S + cfg.causal_attn_flops(S)
        out[f"c2_prefill_s{S}"] = {"ms": round(ms, 4), "tok_s": round(S / (ms / 1e3), 1),
                                   "tflops": round(fl / (ms / 1e3) / 1e12, 1),
                                   "mfma_frac": round(fl / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                   "launch": launch, "eager_ms": round(me, 4), "graph_ms": round(mg, 4)}
        log(f"C2 prefill S={S}: {out[f'c2_prefill_s{S}']}")
        del layer, x
    cfg = W.C4
    layer = W.make_text_layer(cfg, torch.bfloat16, dev, seed=0)
    x, pos = W.text_inputs(cfg, 1, 4096, torch.bfloat16, dev, seed=0)
    b = W.make_rope(cfg, dev).bind(pos)
    y, logits, _ = layer(x, b)
    cases["c4_moe_layer_t4096"] = text_layer_case(cfg, layer, x, pos, y, router_logits=logits)
    ms, me, mg, launch = time_launch_modes(lambda: layer(x, b), lambda o: o[0], 20, warmup, warm_s=0.25)
    fl = cfg.gemm_flops_per_token() * 4096 + cfg.causal_attn_flops(4096)
    # Both bounds: MFMA on the layer's FLOPs, HBM on the bytes it must move at
    # least once (every weight, the token activations in and out).
    wbytes = sum(t.numel() * t.element_size() for t in layer.parameters())
    abytes = 2 * 4096 * cfg.hidden * 2
    out["c4_moe_layer_t4096"] = {"ms": round(ms, 4), "tok_s": round(4096 / (ms / 1e3), 1),
                                 "tflops": round(fl / (ms / 1e3) / 1e12, 1),
                                 "mfma_frac": round(fl / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                 "min_bytes": wbytes + abytes,
                                 "hbm_gbs": round((wbytes + abytes) / (ms / 1e3) / 1e9, 1),
                                 "hbm_frac": round((wbytes + abytes) / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                                 "floor_ms": {"mfma": round(fl / PEAK_BF16_TFLOPS / 1e9, 4),
                                              "hbm": round((wbytes + abytes) / PEAK_HBM_GBS / 1e6, 4)},
                                 "launch": launch, "eager_ms": round(me, 4), "graph_ms": round(mg, 4)}
    log(f"C4 MoE layer: {out['c4_moe_layer_t4096']}")
    del layer, x
    v = W.C5
    blk = W.make_vision_block(v, torch.bfloat16, dev, seed=0)
    pe = W.make_patch_embed(v, torch.bfloat16, dev, seed=0)
    patches = W.vision_inputs(v, torch.bfloat16, dev, seed=0)
    cos, sin = W.vision_rope_cos_sin(v, dev)

    def vis():
        h = pe(patches)
        return blk(h.view(v.images, v.patches_per_image, v.hidden), cos, sin)

    yv = vis()
    pp, pb = _params_cpu(pe), _params_cpu(blk)
    pc, cc, sc = patches.detach().float().cpu(), cos.detach().float().cpu(), sin.detach().float().cpu()

    def run_vis(L, O, rd):
        h = rd(L.patch_embed(pc, pp["weight"], pp["bias"], v.channels, v.temporal, v.patch))
        return L.vision_block(h.view(v.images, v.patches_per_image, v.hidden), pb, num_heads=v.heads, cos=cc,
                              sin=sc, eps=v.eps, rd=rd)
    cases["c5_vision_patch_embed_block"] = (yv.detach().float().cpu(), run_vis)

    ms, me, mg, launch = time_launch_modes(vis, lambda o: o, 40, warmup, warm_s=0.25)
    fl = v.flops()
    n = v.images * v.patches_per_image
    out["c5_vision_patch_embed_block"] = {"ms": round(ms, 4), "patches_s": round(n / (ms / 1e3), 1),
                                          "tflops": round(fl / (ms / 1e3) / 1e12, 1),
                                          "mfma_frac": round(fl / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                          "launch": launch, "eager_ms": round(me, 4), "graph_ms": round(mg, 4)}
    log(f"C5 vision: {out['c5_vision_patch_embed_block']}")
    return out


def traffic_probe(torch, K, W, cfg, S: int, dev: str) -> int:
    """Launch the dominant kernel and a plain copy of known size, nothing else
    timed: the workload for the FETCH_SIZE / WRITE_SIZE counter passes."""
    with torch.inference_mode():
        layer = W.make_text_layer(cfg, torch.bfloat16, dev, seed=0)
        x, _ = W.text_inputs(cfg, 1, S, torch.bfloat16, dev, seed=0)
        h = layer.post_attention_layernorm(x)
        wg, wu = layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight
        for _ in range(3):
            K.matmul_swiglu(h, wg, wu)
        src = torch.empty(256 << 20, dtype=torch.bfloat16, device=dev).normal_()  # 512 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    log("traffic probe done: 3 gate/up GEMMs, 3 copies of 512 MiB")
    return 0


def counter_probe(torch, K, W, dev: str) -> int:
    """Launch every kernel of the path, nothing timed: C2 prefill layer at
    S=4096 (2x), C3 decode step (eager, 2x), C4 MoE layer, C5 patch embed +
    vision block, and the op-level elementwise / norm kernels at layer sizes
    (2x each). The workload for per-kernel MFMA and HBM counter passes."""
    with torch.inference_mode():
        cfg = W.C2
        layer = W.make_text_layer(cfg, torch.bfloat16, dev, seed=0)
        x, pos = W.text_inputs(cfg, 1, 4096, torch.bfloat16, dev, seed=0)
        b = W.make_rope(cfg, dev).bind(pos)
        for _ in range(2):
            layer(x, b)
        del x
        case = W.make_decode_case(cfg, batch=32, capacity=8193 + 4, device=dev, seed=0, layer=layer)
        dbind = case.rope.bind(case.positions.to(torch.int32))
        for _ in range(2):
            case.layer(case.x, dbind, kv_cache=case.cache)
        torch.cuda.synchronize()
        del case, layer
        c4 = W.C4
        moe = W.make_text_layer(c4, torch.bfloat16, dev, seed=0)
        x, pos = W.text_inputs(c4, 1, 4096, torch.bfloat16, dev, seed=0)
        moe(x, W.make_rope(c4, dev).bind(pos))
        del moe, x
        v = W.C5
        blk = W.make_vision_block(v, torch.bfloat16, dev, seed=0)
        pe = W.make_patch_embed(v, torch.bfloat16, dev, seed=0)
        patches = W.vision_inputs(v, torch.bfloat16, dev, seed=0)
        cos, sin = W.vision_rope_cos_sin(v, dev)
        blk(pe(patches).view(v.images, v.patches_per_image, v.hidden), cos, sin)
        g = torch.Generator(device=dev)
        g.manual_seed(0)

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)

        a, c = rnd(4096, 4096), rnd(4096, 4096)
        gate, up = rnd(4096, 12288), rnd(4096, 12288)
        hv, wv, bv = rnd(3136, 1152), rnd(1152), rnd(1152)
        act = rnd(3136, 4304)
        for _ in range(2):
            K.rmsnorm(a, c[0], 1e-6)
            K.layernorm(hv, wv, bv, 1e-6)
            K.swiglu(gate, up)
            K.residual_add(a, c)
            K.gelu_tanh(act)
        torch.cuda.synchronize()
    log("counter probe done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seq", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the C2 S=1024/16384, C4 and C5 measurements")
    ap.add_argument("--counter-probe", action="store_true",
                    help="run every kernel of the path a few times and exit, for PMC counter passes")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the gate/up GEMM (3x) and a 512 MiB device copy (3x), for PMC counter passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from qwen3_5_vl_cuda_custom_amd import kernels as K
    from qwen3_5_vl_cuda_custom_amd import workloads as W
    from qwen3_5_vl_cuda_custom_amd.modules import StepGraph

    dev = "cuda:0"
    torch.cuda.set_device(0)
    cfg = W.C2
    S = args.seq
    if args.traffic_probe:
        return traffic_probe(torch, K, W, cfg, S, dev)
    if args.counter_probe:
        return counter_probe(torch, K, W, dev)
    with torch.inference_mode():
        layer = W.make_text_layer(cfg, torch.bfloat16, dev, seed=0)
        x, pos = W.text_inputs(cfg, 1, S, torch.bfloat16, dev, seed=0)
        rope = W.make_rope(cfg, dev)
        binding = rope.bind(pos)

        def step():
            return layer(x, binding)

        cases = {}
        if not args.no_cpu_baseline:
            cases[f"c2_prefill_s{S}"] = text_layer_case(cfg, layer, x, pos, step()[0])
        # Order of the GPU measurements: the layer's other GEMMs and attention
        # (for the record, ~40 ms of load), then the headline steps, so that the
        # headline's W warm-up and K timed steps run on a GPU already at its
        # steady clocks, then the dominant GEMM. From idle, the first ~40 ms of
        # load run slower (same box: the first 20 steps after a 2 s idle with 5
        # warm-up steps averaged 1.500 ms per layer, every later round
        # 1.437-1.445 ms).
        # Other GEMMs of the layer and attention, for the record.
        a = torch.empty(S, cfg.hidden, dtype=torch.bfloat16, device=dev).normal_()
        detail = {}
        for name, w in [("q_proj", layer.self_attn.q_proj.weight), ("k_proj", layer.self_attn.k_proj.weight),
                        ("o_proj", layer.self_attn.o_proj.weight)]:
            t = time_gpu(lambda w=w: K.matmul(a, w), 40, 2)
            detail[name] = round(2 * S * w.shape[0] * w.shape[1] / (t / 1e3) / 1e12, 1)
        act = torch.empty(S, cfg.intermediate, dtype=torch.bfloat16, device=dev).normal_()
        t = time_gpu(lambda: K.matmul(act, layer.mlp.down_proj.weight), 40, 2)
        detail["down_proj"] = round(2 * S * cfg.hidden * cfg.intermediate / (t / 1e3) / 1e12, 1)
        q = torch.empty(1, cfg.heads, S, cfg.head_dim, dtype=torch.bfloat16, device=dev).normal_()
        kk = torch.empty(1, cfg.kv_heads, S, cfg.head_dim, dtype=torch.bfloat16, device=dev).normal_()
        t = time_gpu(lambda: K.flash_attention(q, kk, kk, cfg.head_dim ** -0.5, True, 4), 40, 2)
        detail["flash_attention"] = round(cfg.causal_attn_flops(S) / (t / 1e3) / 1e12, 1)
        log(f"per-kernel TFLOP/s: {detail}")
        del a, act, q, kk

        # The headline takes the faster of eager launches and a HIP graph
        # replay of the step, both reported; the replay must equal the eager step.
        ms, ms_eager, ms_graph, launch = time_launch_modes(step, lambda o: o[0], args.steps, args.warmup)
        tok_s = S / (ms / 1e3)
        layer_flop = cfg.gemm_flops_per_token() * S + cfg.causal_attn_flops(S)
        layer_tflops = layer_flop / (ms / 1e3) / 1e12
        log(f"prefill S={S}: {ms:.3f} ms/layer, {tok_s:,.0f} tok/s, {layer_tflops:.1f} TFLOP/s "
            f"({layer_tflops / PEAK_BF16_TFLOPS:.1%} of bf16 peak), {launch}; HIP graph replay {ms_graph:.3f} ms, "
            f"eager {ms_eager:.3f} ms")

        # Dominant kernel: the fused gate/up/SwiGLU GEMM on the post-attention activations.
        h = layer.post_attention_layernorm(x)
        wg, wu = layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight
        gemm_ms = time_gpu(lambda: K.matmul_swiglu(h, wg, wu), args.steps, 3)
        gemm_flop = 2 * S * cfg.hidden * cfg.intermediate * 2
        gemm_tflops = gemm_flop / (gemm_ms / 1e3) / 1e12
        log(f"dominant kernel gate/up+SwiGLU GEMM (M={S}, N=2x{cfg.intermediate}, K={cfg.hidden}): "
            f"{gemm_ms:.3f} ms, {gemm_tflops:.1f} TFLOP/s ({gemm_tflops / PEAK_BF16_TFLOPS:.1%})")

        decode = None
        if not args.no_decode:
            # A serving loop's decode step: every replay appends one token per
            # sequence (the cache lengths advance; the rotary positions stay
            # those of the first step, which does not change the work).
            n_steps = 4 * (max(args.steps, 20) + args.warmup) + 16  # every timed and untimed step appends
            case = W.make_decode_case(cfg, batch=32, capacity=8193 + n_steps, device=dev, seed=0, layer=layer)
            dbind = case.rope.bind(case.positions.to(torch.int32))

            def dstep():
                return case.layer(case.x, dbind, kv_cache=case.cache)[0]

            if not args.no_cpu_baseline:
                # one step from the initial cache, for the parity check (rows [0, L_b) stay as they are)
                cases["c3_decode_b32"] = decode_case(cfg, layer, case.x, case.positions, case.lens, case.cache.k,
                                                     case.cache.v, dstep())
            eager_ms = time_gpu(dstep, max(args.steps, 20), args.warmup)
            # One layer per HIP graph launch (the replay's own launch cost lands on the layer).
            graph = StepGraph(dstep, caches=[case.cache])
            one_ms = time_gpu(graph.replay, max(args.steps, 20), args.warmup)
            del graph
            # The step as a model's decode runs it: one HIP graph per token over a
            # stack of distinct layers (own weights, own seed-0-length caches; each
            # layer's output feeds the next), so the per-token launch is shared.
            # The layer's cost is the graph's time over the stack depth.
            depth = 4
            stack = [case] + [W.make_decode_case(cfg, batch=32, capacity=8193 + n_steps, device=dev, seed=0,
                                                 layer=W.make_text_layer(cfg, torch.bfloat16, dev, seed=10 + i))
                              for i in range(depth - 1)]
            for c in stack[1:]:
                c.cache.set_lens(case.cache.lens.cpu())

            def stack_step():
                h = case.x
                for c in stack:
                    h = c.layer(h, dbind, kv_cache=c.cache)[0]
                return h

            stack_step()
            graph = StepGraph(stack_step, caches=[c.cache for c in stack])
            for _ in range(args.warmup):
                graph.replay()
            torch.cuda.synchronize()
            lens_before = int(case.cache.lens.sum())
            dms = time_gpu(graph.replay, max(args.steps, 20), 0) / depth
            lens_after = int(case.cache.lens.sum())
            wbytes = sum(t.numel() * t.element_size() for t in layer.parameters())
            # K and V of every attended row: the cached rows plus the new token's, averaged over the steps
            mean_rows = (lens_before + lens_after) / 2 + 32 / 2
            kvbytes = int(mean_rows * cfg.kv_heads * cfg.head_dim * 2 * 2)
            gbs = (wbytes + kvbytes) / (dms / 1e3) / 1e9
            decode = {"tok_s": round(32 / (dms / 1e3), 1), "ms_per_step": round(dms, 4),
                      "method": f"HIP graph of {depth} distinct layers per token, time / {depth}",
                      "one_layer_graph_ms": round(one_ms, 4), "eager_ms_per_step": round(eager_ms, 4),
                      "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                      "bytes_per_step": wbytes + kvbytes, "batch": 32, "kv_lens_sum_initial": int(case.lens.sum()),
                      "kv_lens_sum_timed": [lens_before, lens_after]}
            log(f"decode B=32: {dms:.3f} ms/step per layer ({depth}-layer graph), {decode['tok_s']:,.0f} tok/s, "
                f"{gbs:,.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of HBM); one-layer graph {one_ms:.3f} ms, "
                f"eager {eager_ms:.3f} ms")
            del case, stack, graph

    extra = None
    if not args.no_extra:
        with torch.inference_mode():
            extra = other_configs(torch, W, dev, args.warmup, cases if not args.no_cpu_baseline else {})

    cpu = parity = cpu_other = None
    if not args.no_cpu_baseline:
        with torch.inference_mode():
            cpu = cpu_baseline(cfg, S, layer)
            log(f"cpu baseline: {cpu}")
            parity, secs = parity_leg(cases)
            cpu_other = cpu_baseline_other(secs)
            log(f"cpu baseline, other configurations: {cpu_other}")

    out = {
        "metric": "decoder-layer prefill tokens/s (8B, S=4096) + decode tok/s; % MFMA/HBM roofline",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) inputs)",
        "config": {"workload": "qwen3vl-8b-shape dense decoder layer, bf16 prefill", "batch": 1, "seq_len": S,
                   "hidden": cfg.hidden, "heads": f"{cfg.heads}q/{cfg.kv_heads}kv x {cfg.head_dim}",
                   "intermediate": cfg.intermediate, "parallelism": "single GPU"},
        "launch": f"{launch} (the faster of eager launches and a HIP graph replay of the layer step, "
                  "the replay checked bit-identical to the eager step)",
        "eager_ms_per_step": round(ms_eager, 4),
        "graph_ms_per_step": round(ms_graph, 4),
        "layer_tflops": round(layer_tflops, 1),
        "layer_mfma_frac": round(layer_tflops / PEAK_BF16_TFLOPS, 4),
        "roofline": {"bound": "mfma", "kernel": "gemm_bf16 gate/up+SwiGLU (M=S, N=2x12288, K=4096)",
                     "achieved": round(gemm_tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": GATE_UP_TRAFFIC_BYTES if S == 4096 else None},
        "kernel_tflops": detail,
        "decode": decode,
        "other_configs": extra,
        "cpu_baseline": cpu,
        "cpu_baseline_other_configs": cpu_other,
        "parity": parity,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
