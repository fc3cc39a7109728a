#!/usr/bin/env python3
"""Benchmark of the Qwen3.5 hybrid-attention hot path on one MI355X.

Headline (the JSON `value`): Gated DeltaNet chunked prefill, B = 1, T = 4096, 16 heads, d_k = d_v = 128, bf16
q/k/v, chunk 64, fp32 state -> tokens per second. The same line carries a breakdown of the other workloads (GDN
decode step, gated-attention prefill T = 4096, gated-attention decode B = 3 and 32 over an 8192 context), each as
tok/s and as a fraction of its roofline, plus the CPU oracle timed on the host cores.

Method: every step is one call of the op on fresh device-resident inputs. The calls over all input sets are captured
back to back in one HIP graph and replayed (as a model's layers run); HIP events recorded on the launch stream around
each replay, divided by the calls it holds, give the per-step GPU time.
Input sets rotate so that the bytes touched between two uses of one set exceed the 256 MB Infinity Cache: the GB/s
figures are HBM figures, not cache figures.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--only gdn_prefill,...] [--no-cpu]
"""
import argparse
import json
import math
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "duo-mech-interp_amd"))

PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
ROTATE_BYTES = 640 << 20     # distinct bytes cycled through between two uses of one input set

# Algorithmic work per unit (minimum HBM bytes / nominal FLOPs)
GDN_PREFILL_BYTES = 68_681_728      # q,k,v bf16 + g,beta fp32 + o bf16 + final S fp32 (T 4096, H 16, d 128)
GDN_PREFILL_FLOPS = 1.190e10
# HBM bytes one GDN prefill launch (prep + scan kernels) actually moves: rocprofv3 FETCH_SIZE / WRITE_SIZE per
# dispatch, each scaled by what the counter reads for a 256 MiB device copy, on the kernels of commit cc5e284
# (profiles/counters_gdn_attn_gemm_kernels.md: prep 72.0 + 67.1 MB, scan 67.3 + 17.8 MB)
GDN_PREFILL_TRAFFIC_BYTES = 224_200_000
GDN_PREFILL_TRAFFIC_COMMIT = "cc5e284"  # the kernels the traffic was counted on
GDN_DECODE_STEP_BYTES = 2_130_048   # S read + write fp32 + q,k,v,o,g,beta (B 1, H 16, d 128)
ATTN_PREFILL_FLOPS = 6.874e10       # 4 * D * Hq * T (T + 1) / 2, T 4096, Hq 8, D 256
ATTN_PREFILL_BYTES = 58_720_256
ATTN_DECODE_ROW_BYTES = 16_789_504  # K + V span 16,777,216 + q, gate, out 12,288


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="", help="comma list of workloads to run")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the headline CPU baseline sample")
    ap.add_argument("--cpu-case-seconds", type=float, default=2.0,
                    help="budget of each per-workload CPU baseline sample (all threads and one thread)")
    return ap.parse_args()


class Timer:
    """Graph-captured steps over rotating input sets, timed with events on the capture/launch stream."""

    def __init__(self, torch, make_call, n_sets, reps=1):
        """reps calls are captured per graph (one per input set, cycling), so that a replay costs one graph launch
        for `reps` steps: per-step times of microsecond kernels are then not graph-launch bound."""
        self.torch = torch
        self.graphs = []
        self.keep = []
        self.reps = reps
        stream = torch.cuda.Stream()
        calls = [make_call(i) for i in range(n_sets)]
        with torch.cuda.stream(stream):  # warm the allocator outside the graphs
            for c in calls:
                c()
        torch.cuda.synchronize()
        n_graphs = max(1, n_sets // reps) if reps > 1 else n_sets
        for gi in range(n_graphs):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                outs = [calls[(gi * reps + r) % n_sets]() for r in range(reps)]
            self.graphs.append(g)
            self.keep.append(outs)
        torch.cuda.synchronize()

    def run(self, steps, warmup):
        torch = self.torch
        n = len(self.graphs)
        for i in range(warmup):
            self.graphs[i % n].replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            ev[i][0].record(stream)
            self.graphs[i % n].replay()
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per = [a.elapsed_time(b) * 1e-3 / self.reps for a, b in ev]  # seconds per call
        return {"wall_s": wall / self.reps, "step_s": sum(per) / len(per), "min_step_s": min(per)}


def n_sets_for(bytes_per_set, cap=24):
    return max(2, min(cap, math.ceil(ROTATE_BYTES / max(bytes_per_set, 1)) + 1))


def bench_gdn_prefill(torch, q35hip, workloads, steps, warmup, dev):
    B, T, H, D = 1, 4096, 16, 128
    per_set = GDN_PREFILL_BYTES + 88 * 1024 * 1024  # inputs/outputs + the op's workspace
    n = n_sets_for(per_set, cap=8)
    sets = []
    for i in range(n):
        sets.append(workloads.to_device(workloads.gdn_inputs(B=B, T=T, H=H, D=D, seed=i, dtype=torch.bfloat16), dev))

    def make_call(i):
        d = sets[i]
        return lambda: q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                                     output_final_state=True, use_qk_l2norm_in_kernel=True)
    r = Timer(torch, make_call, n, reps=n).run(steps, warmup)
    t = r["step_s"]
    gbs = GDN_PREFILL_BYTES / t / 1e9
    return {"tok_s": T * B / t, "ms": t * 1e3, "achieved_gbs": gbs, "frac": gbs / PEAK_HBM_GBS,
            "tflops": GDN_PREFILL_FLOPS / t / 1e12, "wall_ms_per_step": r["wall_s"] / steps * 1e3, "sets": n}


def bench_gdn_prefill_f32(torch, q35hip, workloads, steps, warmup, dev):
    """The chunked rule on fp32 inputs (the fp32 path: every product in fp32) at the hybrid stack's GDN prefill
    shape, B = 3, T = 2048, 16 heads, from a carried state."""
    B, T, H, D = 3, 2048, 16, 128
    n = 4
    sets = [workloads.to_device(workloads.gdn_inputs(B=B, T=T, H=H, D=D, seed=i, dtype=torch.float32), dev)
            for i in range(n)]
    s0 = torch.zeros(B, H, D, D, device=dev)

    def make_call(i):
        d = sets[i]
        return lambda: q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=s0,
                                                     output_final_state=True, use_qk_l2norm_in_kernel=True)
    r = Timer(torch, make_call, n, reps=n).run(steps, warmup)
    t = r["step_s"]
    return {"tok_s": B * T / t, "us": t * 1e6, "shape": "B3 T2048 H16 d128 fp32"}


def bench_gdn_decode(torch, q35hip, workloads, steps, warmup, dev):
    """One decode step (T = 1). Two shapes: the latency-bound B = 1 step (state 1 MiB, as in a model where the layer's
    state stays resident between steps) and a bandwidth shape, B = 16 over 20 distinct layer states (320 MB cycled)."""
    out = {}
    for name, B, nstate in (("b1", 1, 64), ("b16", 16, 20)):
        H, D = 16, 128
        inp = workloads.to_device(workloads.gdn_inputs(B=B, T=1, H=H, D=D, seed=0, dtype=torch.float32), dev)
        states = [torch.zeros(B, H, D, D, device=dev) for _ in range(nstate)]

        def make_call(i, inp=inp, states=states):
            return lambda: q35hip.gdn_decode_step_(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], states[i])
        r = Timer(torch, make_call, nstate, reps=nstate).run(steps, warmup)
        t = r["step_s"]
        by = B * GDN_DECODE_STEP_BYTES
        out[name] = {"tok_s": B / t, "us": t * 1e6, "achieved_gbs": by / t / 1e9, "frac": by / t / 1e9 / PEAK_HBM_GBS,
                     "state_mb_cycled": nstate * B * H * D * D * 4 / 1e6}
    # The 64 sequential tokens of the decode configuration as one launch of the token-serial kernel (the state stays
    # in registers across tokens; each token still waits for the previous one): a decode loop whose inputs are all
    # known, as a prompt replayed token by token is. The per-step figures above are one launch per token.
    B, T, H, D, nstate = 1, 64, 16, 128, 16
    inp = workloads.to_device(workloads.gdn_inputs(B=B, T=T, H=H, D=D, seed=0, dtype=torch.float32), dev)
    states = [torch.zeros(B, H, D, D, device=dev) for _ in range(nstate)]

    def make_seq(i):
        return lambda: q35hip.gdn_decode_step_(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], states[i])
    r = Timer(torch, make_seq, nstate, reps=nstate).run(steps, warmup)
    t = r["step_s"]
    out["b1_t64_one_launch"] = {"tok_s": T / t, "us_per_token": t * 1e6 / T, "us_per_launch": t * 1e6}
    return out


def bench_attn_prefill(torch, q35hip, workloads, steps, warmup, dev):
    B, T = 1, 4096
    n = n_sets_for(ATTN_PREFILL_BYTES, cap=8)
    cos, sin = [x.to(dev) for x in workloads.rope_tables(T)]
    sets = [workloads.to_device(workloads.attn_prefill_inputs(B=B, T=T, seed=i), dev) for i in range(n)]

    def make_call(i):
        d = sets[i]
        return lambda: q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos, sin)
    r = Timer(torch, make_call, n, reps=n).run(steps, warmup)
    t = r["step_s"]
    tf = ATTN_PREFILL_FLOPS / t / 1e12
    return {"tok_s": T / t, "ms": t * 1e3, "achieved_tflops": tf, "frac": tf / PEAK_BF16_TFLOPS, "sets": n}


def bench_attn_decode(torch, q35hip, workloads, steps, warmup, dev):
    out = {}
    N = 8192
    cos, sin = [x.to(dev) for x in workloads.rope_tables(N)]
    for B in (3, 32):
        by = B * ATTN_DECODE_ROW_BYTES
        n = n_sets_for(by, cap=16)
        sets = [workloads.to_device(workloads.attn_decode_inputs(B=B, N=N, seed=i), dev) for i in range(n)]

        def make_call(i, sets=sets):
            d = sets[i]
            return lambda: q35hip.gated_attention_decode(d["q"], d["k_cache"], d["v_cache"], d["gate"],
                                                         d["cache_len"], cos, sin)
        r = Timer(torch, make_call, n, reps=n).run(steps, warmup)
        t = r["step_s"]
        out[f"b{B}"] = {"tok_s": B / t, "us": t * 1e6, "achieved_gbs": by / t / 1e9,
                        "frac": by / t / 1e9 / PEAK_HBM_GBS, "sets": n}
        del sets
        torch.cuda.empty_cache()
    return out


GEMM_SHAPES = (("gdn_in_proj", 8224, 1024, "store"), ("mlp_gate_up", 7168, 1024, "swiglu"),
               ("mlp_down", 1024, 3584, "add"), ("attn_in_proj", 5120, 1024, "store"),
               ("out_proj", 1024, 2048, "add"))


def bench_gemm(torch, q35hip, steps, warmup, dev, M=6144):
    """The int8 prefill GEMM on the stack's projection shapes at M = 3 rows x 2048 tokens (x fp32, W int8 with one
    scale per group of 128 inputs, the stack's format), and torch's fp32 GEMM on the dequantised weights for
    comparison. TFLOP/s count the nominal 2 M N K (the kernel executes twice that: the hi and lo parts of x).
    us_split: the same product on x handed over already split into bf16 hi + lo (the stack's norm writes the inputs
    of the mixers' input projections and of gate/up that way)."""
    out = {}
    g = torch.Generator(device=dev).manual_seed(0)
    for name, N, K, epi in GEMM_SHAPES:
        x = torch.randn(M, K, device=dev, generator=g)
        q = torch.randint(-127, 128, (N, K), device=dev, generator=g, dtype=torch.int8)
        sc = torch.rand(N, K // 128, device=dev, generator=g) * 1e-3
        y = torch.zeros(M, N // 2 if epi == "swiglu" else N, device=dev)
        pushes = q35hip.ops.pack_pushes([(0, "add", [0.0])], dev) if epi == "swiglu" else None

        def make_call(i):
            return lambda: q35hip.ops.gemm_q8(x, q, sc, out=y, epilogue=epi, pushes=pushes, T=2048)
        r = Timer(torch, make_call, 1, reps=8).run(steps, warmup)
        xs = q35hip.ops.split_activations(x)

        def make_split(i):
            return lambda: q35hip.ops.gemm_q8(xs, q, sc, out=y, epilogue=epi, pushes=pushes, T=2048)
        r3 = Timer(torch, make_split, 1, reps=8).run(steps, warmup)
        wf = (q.float().reshape(N, K // 128, 128) * sc[:, :, None]).reshape(N, K).contiguous()
        r2 = Timer(torch, lambda i: (lambda: torch.mm(x, wf.T)), 1, reps=8).run(steps, warmup)
        fl = 2.0 * M * N * K
        out[name] = {"M": M, "N": N, "K": K, "us": r["step_s"] * 1e6, "tflops": fl / r["step_s"] / 1e12,
                     "frac_bf16_peak": fl / r["step_s"] / 1e12 / PEAK_BF16_TFLOPS,
                     "us_split": r3["step_s"] * 1e6, "torch_fp32_us": r2["step_s"] * 1e6}
        del x, xs, q, wf, y
    return out


GEMV_SHAPES = (("mlp_gate_up_norm_swiglu", 7168, 1024, "swiglu", True), ("mlp_down_add", 1024, 3584, "add", False),
               ("gdn_in_proj_norm", 8224, 1024, "store", True), ("lm_head_norm", 151936, 1024, "store", True))


def bench_gemv(torch, q35hip, steps, warmup, dev):
    """The decode GEMV (int8 weights with one scale per group of 128 inputs) on the stack's decode shapes at 1, 3 and
    8 rows of x: weights rotated over enough copies to leave the Infinity Cache, so GB/s is HBM; 'add' is the split-K
    residual accumulation, the norm forms read the residual and apply the RMSNorm prologue."""
    out = {}
    g = torch.Generator(device=dev).manual_seed(0)
    for name, N, K, epi, norm in GEMV_SHAPES:
        wbytes = N * K + N * (K // 128) * 4
        n = n_sets_for(wbytes, cap=24)
        qs = [torch.randint(-127, 128, (N, K), device=dev, generator=g, dtype=torch.int8) for _ in range(n)]
        ss = [torch.rand(N, K // 128, device=dev, generator=g) * 1e-3 for _ in range(n)]
        nw = torch.rand(K, device=dev, generator=g) * 0.1
        pushes = q35hip.ops.pack_pushes([(0, "add", [0.0])], dev) if epi == "swiglu" else None
        for M in (1, 3, 8):
            if M * K * 4 > 64 * 1024:  # x is staged in 64 KiB of LDS (q35_gemv's limit)
                continue
            x = torch.randn(M, K, device=dev, generator=g)
            y = torch.zeros(M, N // 2 if epi == "swiglu" else N, device=dev)
            pn = (None, nw, 1e-6, None) if norm else None

            def make_call(i, x=x, y=y, pn=pn):
                return lambda: q35hip.ops.gemv(x, qs[i], ss[i], out=y, epilogue=epi, pushes=pushes, prenorm=pn)
            r = Timer(torch, make_call, n, reps=n).run(steps, warmup)
            t = r["step_s"]
            out[f"{name}_m{M}"] = {"M": M, "N": N, "K": K, "us": t * 1e6, "gbs": wbytes / t / 1e9,
                                   "frac_hbm": wbytes / t / 1e9 / PEAK_HBM_GBS}
        del qs, ss
    return out


def bench_copy(torch, dev, mb=256, reps=5):
    """A plain device copy of known size (mb MiB read + mb MiB written per launch): the calibration point for the
    FETCH_SIZE / WRITE_SIZE counters of a profiler run."""
    src = torch.ones(mb << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    return {"bytes_per_launch": 2 * (mb << 20), "us": t * 1e6, "gbs": 2 * (mb << 20) / t / 1e9}


def stack_quantization(mlp_group):
    """The weight format of every linear of the config-5 stack as bench_stack builds it."""
    mlp = "int8, one fp32 scale per output channel" if mlp_group == 0 else \
        f"int8, one fp32 scale per group of {mlp_group} inputs"
    eng = "int8, one fp32 scale per group of 128 inputs (the engine's q8 format)"
    return {"mlp_gate_up_down": mlp, "gdn_in_out_proj": eng, "attn_qkv_o_proj": eng, "embedding_lm_head_tied": eng}


def bench_stack(torch, q35hip, workloads, dev, steps=256, mlp_group=0, both_prefills=True):
    """The Qwen3.5-0.8B-shaped hybrid stack (24 layers, SwiGLU 3584, tied 151,936 embedding), batch 3 steered rows:
    2048-token prefill, then `steps` greedy decode steps. mlp_group 0: the MLP int8 per output channel (the stated
    config-5 workload); 128: the engine's per-group format. The prefill is timed with each Gated DeltaNet prefill
    kernel (the chunked default, fp32 products on the stack's fp32 activations, and the token-serial one); decode is
    timed host-driven (eager) and as replays of one captured decode step (HIP graph)."""
    from q35hip import model as gm
    cfg = workloads.Q35Config()
    W = workloads.init_weights(cfg, seed=0, mlp_group=mlp_group)
    g = gm.HybridModel(cfg, W, dev, max_len=2048 + steps + 8, rows=3)
    del W
    prompt = torch.randint(0, cfg.vocab, (1, 2048), generator=torch.Generator().manual_seed(0)).repeat(3, 1)
    # the workload's steering vector: randn (seed 0) scaled to 0.8 x the median residual norm after layer 12 of the
    # unsteered prompt (tokens 1..2047), +v on row 0, none on row 1, -v on row 2
    _, resid = g.forward(prompt, stop_after=12, collect_layer=12)
    med = gm.median_resid_norm(resid[0])
    v = torch.randn(cfg.hidden, generator=torch.Generator().manual_seed(0))
    v = v / v.norm() * (0.8 * med)
    g.set_vectors(torch.stack([v, -v]), [0, -1, 1])
    out = {"rows": 3, "prompt": 2048, "steps": steps, "steer_norm": round(float(v.norm()), 4),
           "quantization": stack_quantization(mlp_group)}
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    # the default ("chunk") last: its states feed the decode loops
    for mode in (("recurrent", "chunk") if both_prefills else ("chunk",)):
        g.gdn_prefill = mode
        for _ in range(2):  # warm: allocator, library handles
            g.reset()
            g.forward(prompt[:, :256])
            g.forward(torch.zeros(3, 1, dtype=torch.long))
        torch.cuda.synchronize()
        g.reset()
        e0, e1 = ev(), ev()
        e0.record()
        logits, _ = g.forward(prompt)
        e1.record()
        torch.cuda.synchronize()
        tp = e0.elapsed_time(e1) * 1e-3
        out[f"prefill_{mode}_tok_s"] = 3 * 2048 / tp
        out[f"prefill_{mode}_ms"] = tp * 1e3
    n_eager = 32
    e1, e2 = ev(), ev()
    e1.record()
    for _ in range(n_eager):
        logits = g.decode_step(q35hip.ops.argmax_rows(logits))
    e2.record()
    torch.cuda.synchronize()
    td = e1.elapsed_time(e2) * 1e-3 / n_eager
    out.update({"decode_eager_tok_s": 3 / td, "decode_eager_ms_per_step": td * 1e3})
    g.enable_decode_graph()
    logits, _ = g.forward(prompt)
    g.decode_step(q35hip.ops.argmax_rows(logits))  # first generated token; its argmax now sits in the graph's ids
    e1, e2 = ev(), ev()
    e1.record()
    for _ in range(steps):
        g.decode_greedy()
    e2.record()
    torch.cuda.synchronize()
    td = e1.elapsed_time(e2) * 1e-3 / steps
    out.update({"decode_tok_s": 3 / td, "decode_ms_per_step": td * 1e3,
                "note": "decode_tok_s: each step one HIP-graph replay of the 24-layer step, greedy argmax included "
                        "(on the device, feeding the next replay)"})
    return out


def host_cpu():
    """The host CPU model (from /proc/cpuinfo) and the logical CPUs this process may run on."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count()
    return model, n


def _time_calls(fn, budget_s, min_calls=2):
    """Median seconds per call of fn() over about budget_s (at least min_calls calls)."""
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < min_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times), sum(times)


def cpu_baseline(budget_s):
    """The headline's CPU baseline: the oracle's chunked gated delta rule (a PyTorch-CPU restatement of the reference's
    fp32 path, HF:249-327) on the full B=1 T=4096 H=16 workload, fp32, all the threads torch uses, called repeatedly
    for about budget_s seconds; the median call is reported."""
    import torch
    sys.path.insert(0, REPO)
    import oracle
    from q35hip import workloads
    inp = workloads.gdn_inputs(B=1, T=4096, H=16, D=128, seed=0, dtype=torch.bfloat16)
    threads = torch.get_num_threads()
    t, n, total = _time_calls(lambda: oracle.chunk_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"],
                                                                   inp["beta"], use_qk_l2norm_in_kernel=True),
                              budget_s, 3)
    model, ncpu = host_cpu()
    return {"value": round(4096 / t, 1), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle chunk_gated_delta_rule (fp32) on the full B=1 T=4096 H=16 d=128 workload, "
                      f"{n} calls in {total:.1f} s, median {t * 1e3:.1f} ms per call; host {model}, "
                      f"{ncpu} logical CPUs available"}


def cpu_baselines(per_case_s):
    """The oracle (PyTorch-CPU fp32 restatement of the reference path) on every workload, at all threads and at one
    thread, each a bounded sample of about per_case_s seconds: config 1 one decode step (B 1, H 16) from a state
    carried over 64 steps; config 2 the chunked rule at full size; config 3 the gated attention prefill at T 4096;
    config 4 one decode step over 8192 keys at B 3 and B 32; config 5 the 24-layer stack at B 3 (MLP int8 per output
    channel): at all threads the full workload (the 2048-token prefill and 256 greedy decode steps), at one thread a
    bounded sample of it (a 128-token prefill and 4 decode steps). Returns tok/s per case."""
    import torch
    sys.path.insert(0, REPO)
    import oracle
    from oracle import model as om
    from q35hip import workloads
    model, ncpu = host_cpu()
    all_threads = torch.get_num_threads()
    out = {"host": model, "logical_cpus": ncpu, "kind": "port", "unit": "tok/s", "threads": {}}
    g1 = workloads.gdn_inputs(B=1, T=64, H=16, D=128, seed=0)
    g2 = workloads.gdn_inputs(B=1, T=4096, H=16, D=128, seed=0, dtype=torch.bfloat16)
    a3 = workloads.attn_prefill_inputs(B=1, T=4096, seed=0)
    cos3, sin3 = workloads.rope_tables(8192)
    a4 = {B: workloads.attn_decode_inputs(B=B, N=8192, seed=0) for B in (3, 32)}
    cfg = workloads.Q35Config()
    W = workloads.init_weights(cfg, seed=0, mlp_group=0)
    prompt_full = torch.randint(0, cfg.vocab, (1, 2048), generator=torch.Generator().manual_seed(0)).repeat(3, 1)
    for threads in sorted({all_threads, 1}, reverse=True):
        torch.set_num_threads(threads)
        r = {}
        S = [torch.zeros(1, 16, 128, 128)]

        def dec1():
            t = len(S) % 64
            sl = {k: v[:, t:t + 1] for k, v in g1.items()}
            _, S[0] = oracle.recurrent_gated_delta_rule(sl["q"], sl["k"], sl["v"], sl["g"], sl["beta"],
                                                        initial_state=S[0], use_qk_l2norm_in_kernel=True)
        t, n, _ = _time_calls(dec1, per_case_s / 2, 8)
        r["cfg1_gdn_decode_b1"] = {"tok_s": 1 / t, "ms_per_step": t * 1e3, "calls": n}
        t, n, _ = _time_calls(lambda: oracle.chunk_gated_delta_rule(g2["q"], g2["k"], g2["v"], g2["g"], g2["beta"],
                                                                    use_qk_l2norm_in_kernel=True), per_case_s, 1)
        r["cfg2_gdn_prefill_t4096"] = {"tok_s": 4096 / t, "ms": t * 1e3, "calls": n}
        t, n, _ = _time_calls(lambda: oracle.gated_attention(a3["q"], a3["k"], a3["v"], a3["gate"], cos3, sin3),
                              per_case_s, 1)
        r["cfg3_attn_prefill_t4096"] = {"tok_s": 4096 / t, "ms": t * 1e3, "calls": n}
        for B, d in a4.items():
            t, n, _ = _time_calls(lambda d=d: oracle.gated_attention_decode(d["q"], d["k_cache"], d["v_cache"],
                                                                            d["gate"], d["cache_len"], cos3, sin3),
                                  per_case_s / 2, 1)
            r[f"cfg4_attn_decode_b{B}"] = {"tok_s": B / t, "ms": t * 1e3, "calls": n}
        ref = om.OracleModel(cfg, W, steer_layer=12)
        full = threads == all_threads
        T, n_dec = (2048, 256) if full else (128, 4)
        t0 = time.perf_counter()
        logits, _ = ref.forward(prompt_full[:, :T])
        tp = time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(n_dec):
            logits, _ = ref.forward(logits.argmax(-1, keepdim=True))
        td = (time.perf_counter() - t0) / n_dec
        r["cfg5_stack_b3"] = {"prefill_tok_s": 3 * T / tp, "decode_tok_s": 3 / td, "prefill_tokens": T,
                              "prefill_ms": tp * 1e3, "decode_steps": n_dec, "decode_ms_per_step": td * 1e3,
                              "sample": "full workload" if full else "bounded sample"}
        out["threads"][str(threads)] = r
    torch.set_num_threads(all_threads)
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the hot path's "
              "multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    import torch
    import q35hip
    from q35hip import workloads
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    q35hip.lib()
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only  # noqa: E731

    res = {}
    if want("gdn_prefill"):
        res["gdn_prefill"] = bench_gdn_prefill(torch, q35hip, workloads, args.steps, args.warmup, dev)
        print(f"# gdn_prefill {res['gdn_prefill']}", file=sys.stderr, flush=True)
    if want("attn_decode"):
        res["attn_decode"] = bench_attn_decode(torch, q35hip, workloads, args.steps, args.warmup, dev)
        print(f"# attn_decode {res['attn_decode']}", file=sys.stderr, flush=True)
    if want("attn_prefill"):
        res["attn_prefill"] = bench_attn_prefill(torch, q35hip, workloads, args.steps, args.warmup, dev)
        print(f"# attn_prefill {res['attn_prefill']}", file=sys.stderr, flush=True)
    if want("gdn_prefill_f32"):
        res["gdn_prefill_f32"] = bench_gdn_prefill_f32(torch, q35hip, workloads, args.steps, args.warmup, dev)
        print(f"# gdn_prefill_f32 {res['gdn_prefill_f32']}", file=sys.stderr, flush=True)
    if want("gdn_decode"):
        res["gdn_decode"] = bench_gdn_decode(torch, q35hip, workloads, args.steps, args.warmup, dev)
        print(f"# gdn_decode {res['gdn_decode']}", file=sys.stderr, flush=True)

    if want("gemm"):
        res["gemm"] = bench_gemm(torch, q35hip, args.steps, args.warmup, dev)
        print(f"# gemm {res['gemm']}", file=sys.stderr, flush=True)
    if want("gemv"):
        res["gemv"] = bench_gemv(torch, q35hip, args.steps, args.warmup, dev)
        print(f"# gemv {res['gemv']}", file=sys.stderr, flush=True)
    if only and "copy" in only:
        res["copy"] = bench_copy(torch, dev)
        print(f"# copy {res['copy']}", file=sys.stderr, flush=True)
    if want("stack"):
        res["stack"] = bench_stack(torch, q35hip, workloads, dev, mlp_group=0)
        print(f"# stack {res['stack']}", file=sys.stderr, flush=True)
    if want("stack_mlp_g128"):
        res["stack_mlp_g128"] = bench_stack(torch, q35hip, workloads, dev, mlp_group=128, both_prefills=False)
        print(f"# stack_mlp_g128 {res['stack_mlp_g128']}", file=sys.stderr, flush=True)

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    if not args.no_cpu and not only:
        res["cpu"] = cpu_baselines(args.cpu_case_seconds)
        print(f"# cpu {res['cpu']}", file=sys.stderr, flush=True)
    gp = res.get("gdn_prefill")
    line = {
        "metric": "GDN prefill tok/s + gated-attn decode tok/s @1 GPU; % of HBM/MFMA roofline",
        "value": round(gp["tok_s"], 1) if gp else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gp["ms"], 4) if gp else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "gdn_chunked_prefill", "batch": 1, "seq_len": 4096, "heads": 16, "d_k": 128,
                   "d_v": 128, "chunk": 64, "state": "fp32", "activations": "bf16", "parallelism": "none (1 GPU)"},
        "roofline": ({"bound": "hbm", "achieved": round(gp["achieved_gbs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                      "frac": round(gp["frac"], 4), "traffic": GDN_PREFILL_TRAFFIC_BYTES,
                      "traffic_profiled_at": GDN_PREFILL_TRAFFIC_COMMIT} if gp else None),
        "cpu_baseline": cpu,
        "breakdown": res,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
