"""Headline benchmark: FP8 paged decode attention, BASELINE config 3, on one MI355X.

A step is one decode step's attention over all 28 layers of Qwen3-0.6B: 256 sequences (one
query token each), contexts U{100..1024} + U{0..1024}, 16 query / 8 kv heads, head_dim 128,
FP8 e4m3 cache in 256-token blocks with per-(token, head) scales (the reference's scale mode),
seeded random block tables. Each layer has its own cache (28 distinct ~630 MB K+V pools), so
every layer's KV read is cold in the 256 MB last-level cache, as in a real decode step.

`value` is algorithmic KV-read bandwidth in GB/s: sum over layers of
  sum_t kv_len(t) * KV * (2*HD + 8)  +  2 * T * H * HD * 2   bytes
divided by the timed wall time of K steps (inputs resident in HBM before timing starts).

The same line carries `e2e`: config 5's end-to-end output tokens/s (256 requests through the
engine with a random-init Qwen3-0.6B; `--no-e2e` skips it, `--e2e` runs it alone).

Prints one JSON line (rank 0). Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "FP8 paged-decode KV-read GB/s (% of HBM peak), 256 seqs; e2e output tok/s"
HBM_PEAK_GBS = 8000.0
LAYERS = 28
TRAFFIC_FILE = ROOT / "profiles" / "paged_decode_config3_traffic.txt"


def read_traffic():
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 PMC summary."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(b, reps: int = 5):
    """The oracle (scalar C restatement, OpenMP over (token, kv head)) on one full layer of the
    same workload, timed on this host: median of `reps` after one warm-up."""
    import numpy as np

    import oracle
    from cppvllm_amd import workloads

    threads = min(16, len(os.sched_getaffinity(0)))
    oracle.set_threads(threads)

    def host(t):
        import torch
        if t.dtype == torch.bfloat16:
            return t.cpu().view(torch.int16).numpy().view(np.uint16)
        return t.cpu().numpy()

    args = [host(b[k]) for k in ("q", "k_cache", "v_cache", "k_scale", "v_scale", "block_tables", "token_seq",
                                 "token_kv_len")]
    H, KV, HD, BS = b["n_heads"], b["n_kv_heads"], b["head_dim"], b["block_size"]
    # one warm-up layer, then at least `reps` layers and about 10 s of timed CPU work
    times = []
    i = 0
    while i <= reps or sum(times) < 10.0:
        t0 = time.perf_counter()
        oracle.paged_attention_fp8(*args, H, KV, HD, BS, oracle.PER_TOKEN_HEAD, b["scale"])
        if i:
            times.append(time.perf_counter() - t0)
        i += 1
    med = statistics.median(times)
    nbytes = workloads.attention_bytes(args[7].tolist(), n_kv=KV, n_heads=H)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "omp_max_threads": oracle.max_threads(),
            "sample": f"one layer of config 3 (all 256 tokens, {nbytes / 1e6:.1f} MB algorithmic), "
                      f"median of {len(times)} ({sum(times):.1f} s timed) after 1 warm-up: {med * 1e3:.1f} ms/layer"}


def e2e_requests(seed: int = 1005, n: int = 256):
    """Config 5's workload (bench.cpp:13-45): n prompts of U{100..1024} random token ids in
    [0, 10000], output lengths U{100..1024}, greedy, EOS ignored. Seeded numpy draws."""
    import numpy as np
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, 10001, size=int(rng.integers(100, 1025))).tolist() for _ in range(n)]
    outs = [int(x) for x in rng.integers(100, 1025, size=n)]
    return prompts, outs


def run_e2e(args):
    """Config 5: end-to-end generation through the engine (continuous batching, chunked prefill,
    HIP-graph decode) with a random-init Qwen3-0.6B; output tokens/s on one GPU."""
    import torch

    from cppvllm_amd.llm_engine import EngineConfig, LLMEngine, SamplingParams

    t_init = time.perf_counter()
    cfg = EngineConfig(max_num_batched_tokens=4096, max_num_seqs=256, max_chunk_tokens=1024, max_model_len=4096,
                       block_size=args.e2e_block_size, seed=0, enforce_eager=args.eager)
    eng = LLMEngine(cfg)
    init_s = time.perf_counter() - t_init
    eng.generate([[1, 2, 3, 4, 5, 6, 7, 8]], SamplingParams(max_tokens=16, ignore_eos=True))   # warm-up
    prompts, outs = e2e_requests(n=args.e2e_requests)
    before = eng.stats()
    rep0, rows0, keys0 = eng.runner.decode_replays, eng.runner.decode_rows, eng.runner.decode_keys
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for p, n in zip(prompts, outs):
        eng.add_request(p, SamplingParams(max_tokens=n, ignore_eos=True))
    steps = 0
    while not eng.is_finished():
        eng.step()
        steps += 1
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    got = eng.take_finished()
    total = sum(len(v) for v in got.values())
    assert total == sum(outs), (total, sum(outs))
    after = eng.stats()
    run = eng.runner
    c = eng.model.cfg
    reps = max(run.decode_replays - rep0, 1)
    # algorithmic bytes of one decode-attention launch (one layer), averaged over the graph replays
    dec_bytes = ((run.decode_keys - keys0) * c.n_kv_heads * (2 * c.head_dim + 8)
                 + 2 * (run.decode_rows - rows0) * c.n_heads * c.head_dim * 2) / reps
    return {
        "metric": "e2e output tok/s (config 5)", "value": round(total / dt, 2), "unit": "tok/s",
        "n_gpus": 1, "steps": steps, "warmup": 1, "ms_per_step": round(dt * 1e3 / max(steps, 1), 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init Qwen3-0.6B weights N(0,0.02); seeded random prompt ids)",
        "config": {"workload": "BASELINE config 5: 256 requests, input U(100,1024), output U(100,1024), greedy, "
                               "ignore EOS; continuous batching, chunked prefill, HIP-graph decode",
                   "requests": len(prompts), "output_tokens": total, "prompt_tokens": sum(len(p) for p in prompts),
                   "seconds": round(dt, 3), "block_size": cfg.block_size, "kv_blocks": eng.num_blocks,
                   "preemptions": after.preemptions - before.preemptions, "init_s": round(init_s, 1),
                   "launch": "eager" if args.eager else "hip_graph",
                   "decode_replays": run.decode_replays - rep0,
                   "decode_rows_avg": round((run.decode_rows - rows0) / reps, 1),
                   "decode_attn_bytes_per_launch": round(dec_bytes)},
    }


def run_prefill(args):
    """The MFMA multi-query kernel on one prefill step of config-5-shaped prompts (4096 tokens),
    28 distinct layer caches, HIP-graph replay; MFMA-bound: reports TFLOP/s against the bf16 dense
    peak, with the stream-K decode kernel on the same rows for comparison."""
    import torch

    from cppvllm_amd import _lib, ops, workloads

    dev = torch.device("cuda", 0)
    lens = workloads.prefill_lens()
    b = workloads.prefill_batch(lens, 256, 1005, dev)
    layers = [(b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"])]
    layers += [tuple(x.clone() for x in layers[0]) for _ in range(args.layers - 1)]
    out = torch.empty_like(b["q"])
    T = b["q"].shape[0]
    ws = ops.paged_attention_workspace(T, 16, 8, 128, b["block_tables"].shape[1], 256, 0, dev)
    pws = ops.prefill_workspace(T, dev)

    def run(kernel):
        def f():
            if kernel == "prefill":     # the step's plan (longest 64-token groups first), then the layers
                ops.paged_attention_prefill_plan(b["token_seq"], b["token_kv_len"], b["block_tables"].shape[1], 256,
                                                 pws)
            for kc, vc, ks, vs in layers:
                if kernel in ("prefill", "prefill_unplanned"):
                    ops.paged_attention_fp8_prefill(out, b["q"], kc, vc, ks, vs, b["block_tables"], b["token_seq"],
                                                    b["token_kv_len"], b["scale"],
                                                    workspace=pws if kernel == "prefill" else None)
                else:
                    ops.paged_attention_fp8(out, b["q"], kc, vc, ks, vs, b["block_tables"], b["token_seq"],
                                            b["token_kv_len"], b["scale"], workspace=ws)
        f()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f()
        for _ in range(args.warmup):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (args.steps * len(layers))      # ms per launch

    ms = run("prefill")
    ms_unplanned = run("prefill_unplanned")
    ms_decode = run("decode")
    kvl = b["token_kv_len"].cpu().tolist()
    flops = workloads.attention_flops(kvl)
    uniq = sum(lens) * 8 * (2 * 128 + 8) + 2 * T * 16 * 128 * 2
    tf = flops / (ms / 1e3) / 1e12
    return {
        "metric": "FP8 paged attention, prefill rows: TFLOP/s (MFMA multi-query kernel)", "value": round(tf, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms * len(layers), 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 (MFMA), fp32 softmax",
        "data": "synthetic (seeded N(0,1) K/V quantised to e4m3 per (token, head); random block tables)",
        "config": {"workload": "one 4096-token prefill step of config-5 prompts (U{100..1024}), 28 layers",
                   "prompts": lens, "tokens": T, "flops_per_layer": flops, "unique_kv_bytes_per_layer": uniq,
                   "us_per_layer": round(ms * 1e3, 2), "plan": "once per step (included: 1/28 per layer)",
                   "unplanned_us_per_layer": round(ms_unplanned * 1e3, 2),
                   "decode_kernel_us_per_layer": round(ms_decode * 1e3, 2),
                   "speedup_vs_decode_kernel": round(ms_decode / ms, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tf / 2500.0, 4), "traffic": None,
                     "kernel": "paged_prefill_kernel<2, per_token_head, true> (planned, 8 waves)",
                     "avg_launch_us": round(ms * 1e3, 2)},
    }


def run_fused(args):
    """Config 2: the fused pre-attention ops over 4096 packed tokens (add_rms_norm, then
    QK-norm + RoPE + FP8 quantise-and-scatter through slot_mapping with -1 padding rows), each
    launch timed with HIP events over K replays of a graph; GB/s of algorithmic bytes. The
    working set (~95 MB) is resident in the 256 MB last-level cache, so this is a launch/latency
    measurement, not an HBM one. CPU baseline: the oracle (scalar C) on the same inputs."""
    import numpy as np
    import torch

    import oracle
    from cppvllm_amd import ops, workloads

    dev = torch.device("cuda", 0)
    w = workloads.fused_batch(device=dev)
    T, D, HD = w["x"].shape[0], w["x"].shape[1], w["head_dim"]
    H, KV, BS = w["n_heads"], w["n_kv_heads"], w["block_size"]
    nb = w["num_blocks"]
    kc = torch.zeros((nb, BS, KV, HD), dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((nb, KV, BS), dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    cos, sin = ops.rope_tables(w["max_position"], HD, w["theta"])
    cos, sin = cos.to(dev), sin.to(dev)
    q = torch.empty((T, H, HD), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(w["x"])
    resid = w["resid"].clone()

    def norm():
        ops.fused.add_rms_norm(resid, w["x"], w["w"], out, 1e-6)

    def qkv():
        ops.fused.qk_norm_rope_kv_write_fp8(q, w["qkv"], w["q_norm"], w["k_norm"], cos, sin, w["positions"],
                                            w["slots"], kc, vc, ks, vs, None, None, H, KV, 1e-6)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(10):
                fn()
        for _ in range(args.warmup):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (10 * args.steps)          # ms per launch

    ms_norm, ms_qkv = timed(norm), timed(qkv)
    valid = w["valid_tokens"]
    b_norm = 4 * T * D * 2 + D * 2
    b_qkv = T * ((H + 2 * KV) * HD * 2 + H * HD * 2 + HD // 2 * 4 * 2) + valid * KV * (2 * HD + 8) + 2 * HD * 2
    gbs_norm = b_norm / (ms_norm / 1e3) / 1e9
    gbs_qkv = b_qkv / (ms_qkv / 1e3) / 1e9

    def host(t):
        return t.cpu().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.cpu().numpy()

    hx = {k: host(w[k]) for k in ("resid", "x", "w", "qkv", "q_norm", "k_norm", "positions", "slots")}
    kco, vco = np.zeros((nb, BS, KV, HD), np.uint8), np.zeros((nb, BS, KV, HD), np.uint8)
    kso, vso = np.zeros((nb, KV, BS), np.float32), np.zeros((nb, KV, BS), np.float32)
    times = []
    for i in range(4):
        t0 = time.perf_counter()
        oracle.add_rms_norm(hx["resid"], hx["x"], hx["w"], 1e-6)
        oracle.qk_norm_rope_kv_write_fp8(hx["qkv"], hx["q_norm"], hx["k_norm"], cos.cpu().numpy(), sin.cpu().numpy(),
                                         hx["positions"], hx["slots"], kco, vco, kso, vso, H, KV, HD, BS)
        if i:
            times.append(time.perf_counter() - t0)
    cpu_s = statistics.median(times)
    return {
        "metric": "fused pre-attention ops GB/s (config 2)", "value": round((b_norm + b_qkv) / ((ms_norm + ms_qkv) / 1e3) / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_norm + ms_qkv, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in/out, f32 math, e4m3 cache", "data": "synthetic (seeded config 2 batch)",
        "config": {"workload": "BASELINE config 2: 4096 packed tokens, 32 segments, -1 padding rows",
                   "valid_tokens": valid, "add_rms_norm_us": round(ms_norm * 1e3, 2),
                   "qk_norm_rope_kv_write_us": round(ms_qkv * 1e3, 2), "add_rms_norm_bytes": b_norm,
                   "qk_norm_rope_kv_write_bytes": b_qkv, "add_rms_norm_GBs": round(gbs_norm, 1),
                   "qk_norm_rope_kv_write_GBs": round(gbs_qkv, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs_qkv, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_qkv / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qk_norm_rope_kv_kernel<128, per_token_head> (working set cache-resident)",
                     "avg_launch_us": round(ms_qkv * 1e3, 2)},
        "cpu_baseline": {"value": round((b_norm + b_qkv) / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1,
                         "kind": "port", "sample": f"both ops once over the full config-2 batch (scalar C), median "
                                                   f"of 3 after 1 warm-up: {cpu_s * 1e3:.1f} ms"},
    }


GEMM_SHAPES = {"qkv": (4096, 1024), "o_proj": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072),
               "lm_head": (151936, 1024)}


def run_gemm(args):
    """Decode-projection GEMMs of Qwen3-0.6B: hipBLASLt (torch.mm) vs cvh_gemm_bf16_nt's automatic
    configuration (and, with --gemm-all, every compiled configuration) per row count, plus the gate/up
    GEMM with the SwiGLU epilogue. HIP-graph replay of back-to-back calls cycling distinct weight
    copies (48, or 2 for the lm_head) so the weights come from HBM as in a 28-layer step."""
    import ctypes as C

    import torch

    from cppvllm_amd import _lib, ops
    L = _lib.lib()
    dev = "cuda"

    def codes(fn):
        n = fn(None, 0)
        b = (C.c_int * n)()
        fn(b, n)
        return list(b)

    def timed(body, reps):
        body()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                body()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / 5 / reps

    rows = [1, 8, 16, 32, 48, 64, 96, 128, 192, 256]
    every = codes(L.cvh_gemm_bf16_nt_configs)
    res = {"metric": "decode-projection GEMM us per call", "unit": "us", "rows": rows, "shapes": {}}
    for name, (N, K) in GEMM_SHAPES.items():
        ws = [(torch.randn(N, K, device=dev) * 0.02).to(torch.bfloat16) for _ in range(2 if N > 100000 else 48)]
        per = {}
        for M in rows:
            x = torch.randn(M, K, device=dev).to(torch.bfloat16)
            y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
            auto = L.cvh_gemm_bf16_nt_config(M, N, K)
            ent = {"hipblaslt": timed(lambda: [torch.mm(x, w.t(), out=y) for w in ws], len(ws)),
                   "auto_code": auto,
                   "auto": timed(lambda: [ops.linear(y, x, w) for w in ws], len(ws))}
            if args.gemm_all:
                cand = {}
                for c in every:
                    if L.cvh_gemm_bf16_nt(y.data_ptr(), x.data_ptr(), ws[0].data_ptr(), M, N, K, c,
                                          torch.cuda.current_stream().cuda_stream) != 0:
                        continue            # tile or K split does not fit this shape
                    cand[c] = timed(lambda: [ops.linear(y, x, w, c) for w in ws], len(ws))
                ent["best_code"], ent["best"] = min(cand.items(), key=lambda kv: kv[1])
            ent["weight_gbs"] = N * K * 2 / ent["auto"] / 1e3
            per[M] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in ent.items()}
            print(f"bench: {name} M={M} " + " ".join(f"{k}={v}" for k, v in per[M].items()), flush=True,
                  file=sys.stderr)
        res["shapes"][f"{name} ({N}x{K})"] = per
        del ws
    I, K = 3072, 1024
    ws = [(torch.randn(2 * I, K, device=dev) * 0.02).to(torch.bfloat16) for _ in range(48)]
    per = {}
    for M in rows:
        x = torch.randn(M, K, device=dev).to(torch.bfloat16)
        gu = torch.empty(M, 2 * I, device=dev, dtype=torch.bfloat16)
        act = torch.empty(M, I, device=dev, dtype=torch.bfloat16)

        def unfused():
            for w in ws:
                torch.mm(x, w.t(), out=gu)
                ops.fused.swiglu(act, gu)
        per[M] = {"hipblaslt_plus_swiglu": round(timed(unfused, len(ws)), 3),
                  "auto_code": L.cvh_gemm_bf16_nt_swiglu_config(M, I, K),
                  "fused": round(timed(lambda: [ops.linear_swiglu(act, x, w) for w in ws], len(ws)), 3)}
        print(f"bench: gate_up+swiglu M={M} {per[M]}", flush=True, file=sys.stderr)
    res["shapes"]["gate_up + SwiGLU epilogue (6144x1024 -> 3072)"] = per
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--partitions", type=int, default=0, help="work partitions (0 = automatic)")
    ap.add_argument("--eager", action="store_true", help="launch eagerly instead of replaying HIP graphs")
    ap.add_argument("--unplanned", action="store_true",
                    help="no per-step plan: every layer's launch derives its work layout itself")
    ap.add_argument("--config", type=int, default=3, choices=(2, 3, 4),
                    help="3: 256 seqs, ctx U(100,1024)+U(0,1024) (headline); 4: 64 seqs, ctx log-U(4k,32k); "
                         "2: the fused pre-attention ops over 4096 packed tokens")
    ap.add_argument("--seqs", type=int, default=256,
                    help="config 3 with this many sequences (a smaller decode batch; the headline is 256)")
    ap.add_argument("--shared-prefix", action="store_true", help="config 4b: even sequences share 8 blocks")
    ap.add_argument("--gqa", type=int, default=0, choices=(0, 1, 2, 4, 8),
                    help="query heads per kv head over the same K/V (0: the workload's own, 2)")
    ap.add_argument("--tp", type=int, default=1, choices=(1, 2, 4, 8),
                    help="configs 3/4 at one GPU's tensor-parallel share: kv heads 8/tp, query heads 16/tp")
    ap.add_argument("--no-shared-reuse", action="store_true",
                    help="config 4b without telling the plan which blocks are shared (every sequence reads its prefix)")
    ap.add_argument("--e2e", action="store_true", help="config 5: end-to-end generation tok/s through the engine")
    ap.add_argument("--e2e-requests", type=int, default=256)
    ap.add_argument("--prefill", action="store_true", help="time the MFMA multi-query (prefill) kernel alone")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 end-to-end leg of the default run")
    ap.add_argument("--e2e-block-size", type=int, default=256)
    ap.add_argument("--gemm", action="store_true",
                    help="decode-projection GEMMs: hipBLASLt vs cvh_gemm_bf16_nt per row count")
    ap.add_argument("--gemm-all", action="store_true", help="with --gemm: also time every compiled configuration")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 3 plain 1 GiB device-to-device copies (rocprofv3 FETCH/WRITE_SIZE scale)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode attention shards by sequence or kv head with no exchange inside the path).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from cppvllm_amd import _lib, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.e2e:
        print(json.dumps(run_e2e(args)), flush=True)
        return
    if args.prefill:
        print(json.dumps(run_prefill(args)), flush=True)
        return
    if args.gemm:
        print(json.dumps(run_gemm(args)), flush=True)
        return
    if args.config == 2:
        print(json.dumps(run_fused(args)), flush=True)
        return
    if args.calibrate_copy:
        a = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        c = torch.empty_like(a)
        for _ in range(3):
            c.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "3 x 1 GiB device copy", "bytes_per_copy": 1 << 30}))
        return
    print(f"bench: building config {args.config} on device", flush=True, file=sys.stderr)
    if args.config == 3:
        b = workloads.config3(device=dev, seqs=args.seqs)
    else:
        b = workloads.config4(device=dev, shared_prefix=args.shared_prefix)
    if args.tp > 1:
        b = workloads.tp_share(b, args.tp)
    if args.gqa:
        # the same K/V read by gqa query heads per kv head (GQA ratio args.gqa)
        g = torch.Generator(device=dev).manual_seed(77)
        b["n_heads"] = b["n_kv_heads"] * args.gqa
        b["q"] = torch.randn((b["q"].shape[0], b["n_heads"], b["head_dim"]), generator=g, device=dev).to(torch.bfloat16)
    lens = b["token_kv_len"].cpu().tolist()
    T, H, KV, HD, BS = len(lens), b["n_heads"], b["n_kv_heads"], b["head_dim"], b["block_size"]
    W = b["block_tables"].shape[1]
    layers = []
    for l in range(args.layers):
        if l == 0:
            layers.append((b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"]))
        else:
            layers.append(tuple(x.clone() for x in (b["k_cache"], b["v_cache"], b["k_scale"], b["v_scale"])))
    lib = _lib.lib()
    shared = args.shared_prefix and not args.no_shared_reuse and not args.unplanned
    ws_fn = lib.cvh_paged_attention_workspace_bytes_shared if shared else lib.cvh_paged_attention_workspace_bytes
    ws_bytes = ws_fn(T, H, KV, HD, W, BS, args.partitions)
    ws = torch.zeros(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    out = torch.empty_like(b["q"])
    layer_ptrs = [tuple(x.data_ptr() for x in lay) for lay in layers]
    # the op = decode kernel (split phase) + merge of cut rows (merge phase); by default a plan of
    # the step's layout is built once per step and read by every layer's decode launch
    planned = not args.unplanned
    split_fn = lib.cvh_paged_attention_fp8_split_phase
    if planned:
        split_fn = lib.cvh_paged_attention_fp8_planned_split_phase
    if planned and args.shared_prefix and not args.no_shared_reuse:
        split_fn = lib.cvh_paged_attention_fp8_planned_shared_split_phase
    merge_fn = lib.cvh_paged_attention_fp8_planned_shared_merge_phase if shared else \
        lib.cvh_paged_attention_fp8_merge_phase

    def launch(fn, lp):
        sp = torch.cuda.current_stream(dev).cuda_stream      # the capture stream during capture
        code = fn(out.data_ptr(), b["q"].data_ptr(), *lp, b["block_tables"].data_ptr(), W, b["token_seq"].data_ptr(),
                  b["token_kv_len"].data_ptr(), T, H, KV, HD, BS, _lib.SCALE_PER_TOKEN_HEAD, b["scale"],
                  args.partitions, ws.data_ptr(), ws_bytes, sp)
        if code:
            raise _lib.CvhError("paged_attention_fp8", code)


    def plan():
        sp = torch.cuda.current_stream(dev).cuda_stream
        if shared:        # config 4b: the shared prefix is read once per unit of up to 8 sequences
            code = lib.cvh_paged_attention_plan_shared(b["block_tables"].data_ptr(), W, b["token_seq"].data_ptr(),
                                                       b["token_kv_len"].data_ptr(), b["shared_blocks"].data_ptr(), T,
                                                       H, KV, HD, BS, args.partitions, ws.data_ptr(), ws_bytes, sp)
        else:
            code = lib.cvh_paged_attention_plan(b["block_tables"].data_ptr(), W, b["token_seq"].data_ptr(),
                                                b["token_kv_len"].data_ptr(), T, H, KV, HD, BS, args.partitions,
                                                ws.data_ptr(), ws_bytes, sp)
        if code:
            raise _lib.CvhError("paged_attention_plan", code)

    def step():                   # one decode step: (plan), then 28 layers, each decode + merge
        if planned:
            plan()
        for lp in layer_ptrs:
            launch(split_fn, lp)
            launch(merge_fn, lp)

    def decode_only():            # the dominant kernel alone, 28 launches back to back (plan left by step())
        for lp in layer_ptrs:
            launch(split_fn, lp)

    def capture(fn):
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    def timed(replay, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    if args.eager:
        run_step, run_decode = step, decode_only
    else:                         # HIP graphs, as a decode engine replays them
        g_step, g_dec = capture(step), capture(decode_only)
        run_step, run_decode = g_step.replay, g_dec.replay
    for _ in range(args.warmup):
        run_step()
    total_ms = timed(run_step, args.steps)
    # events bracket K back-to-back replays of the 28 decode-kernel launches (same stream)
    dec_ms = timed(run_decode, args.steps)
    avg_layer_ms = dec_ms / (args.steps * len(layer_ptrs))

    bytes_layer = workloads.attention_bytes(lens, n_kv=KV, n_heads=H)
    bytes_step = bytes_layer * len(layer_ptrs)
    value = bytes_step * args.steps / (total_ms / 1e3) / 1e9
    achieved = bytes_layer / (avg_layer_ms / 1e3) / 1e9
    # the PMC summary covers config 3 at all 8 kv heads
    traffic = read_traffic() if args.config == 3 and args.tp == 1 and args.seqs == 256 else None
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) K/V quantised to e4m3 per (token, head); random block tables)",
        "config": {
            "workload": ("BASELINE config 3: 256-seq FP8 paged decode step, 28 layers, distinct per-layer caches"
                         if args.config == 3 else
                         "BASELINE config 4%s: 64-seq long-context FP8 paged decode, 28 layers, distinct per-layer "
                         "caches" % ("b (shared 8-block prefix)" if args.shared_prefix else "")),
            "tp_share": ("kv heads 0..%d of 8 (the first GPU's shard at tp=%d)" % (KV - 1, args.tp)) if args.tp > 1
            else None,
            "seqs": T, "ctx_sum": int(sum(lens)), "ctx_min": int(min(lens)), "ctx_max": int(max(lens)),
            "n_heads": H, "n_kv_heads": KV, "head_dim": HD, "block_size": BS, "layers": len(layer_ptrs),
            "scale_mode": "per_token_head", "partitions": lib.cvh_paged_attention_partitions(T, H, KV, HD, W, BS)
            if args.partitions == 0 else args.partitions,
            "bytes_per_layer": bytes_layer, "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "launch": "eager" if args.eager else "hip_graph",
            "plan": ("once per step (%s), read by all layers" % ("cvh_paged_attention_plan_shared" if shared else
                                                                 "cvh_paged_attention_plan")) if planned else "none",
            "op_us_per_layer": round(total_ms * 1e3 / (args.steps * len(layer_ptrs)), 2),
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "paged_decode_kernel (%s split phase; graph of 28 back-to-back launches)"
                               % ("planned" if planned else "unplanned"),
                     "avg_launch_us": round(avg_layer_ms * 1e3, 2),
                     "timing": "achieved = bytes_per_layer / avg_launch_us; avg_launch_us = HIP events around "
                               "K replays of a graph of the 28 decode-kernel launches on the launch stream, / (28 K)"},
    }
    if not args.no_cpu:
        print("bench: CPU baseline (oracle, one layer)", flush=True, file=sys.stderr)
        res["cpu_baseline"] = cpu_baseline(b)
    if args.config == 3 and not args.no_e2e:
        # the metric's second half: config 5 end-to-end output tok/s through the engine
        del b, layers, layer_ptrs, ws, out
        if not args.eager:
            del g_step, g_dec
        torch.cuda.empty_cache()
        print("bench: config 5 end-to-end generation", flush=True, file=sys.stderr)
        e = run_e2e(args)
        res["e2e"] = {"value": e["value"], "unit": e["unit"], "seconds": e["config"]["seconds"],
                      "output_tokens": e["config"]["output_tokens"], "steps": e["steps"],
                      "workload": e["config"]["workload"], "data": e["data"],
                      "reference_published": {"value": 5156.19, "unit": "tok/s", "hardware": "1x NVIDIA A10G",
                                              "source": "README.md:25 of the reference"}}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
